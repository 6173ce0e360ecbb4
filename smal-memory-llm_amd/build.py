"""Build libslotscan.so (the gfx950 slot-scan / slot-read kernels and their C-ABI) in place.

    python smal-memory-llm_amd/build.py            # compile
    python smal-memory-llm_amd/build.py --check    # also print per-kernel VGPR / scratch / LDS use

hipcc cross-compiles for gfx950 without a GPU.  Each source is compiled to its own object in parallel
(objects under _build/), then the objects are linked into the library.  The library is linked against
libamdhip64.so.7 by SONAME, so inside a process that imported torch first it binds to torch's own HIP runtime
(one runtime, one set of streams).  Code object v5 is requested explicitly so that runtimes older than the
compiler load it.

Every compile keeps the compiler's per-kernel resource report (-Rpass-analysis=kernel-resource-usage:
registers, scratch, occupancy, LDS) in _build/<source>.resources.txt, headed by a hash of the source and the
flags it was built with; resource_report() parses it (and recompiles the device code when it is stale), so
tests can check properties such as "no scratch" on the kernels that rely on them.
"""
import hashlib
import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
SOURCES = [os.path.join(CSRC, f) for f in ("slotscan.hip", "slotread.hip", "slotmem.hip", "slotwin.hip", "slotgen.hip",
                                                 "slotproj.hip")]
OUT = os.path.join(HERE, "libslotscan.so")
BUILD_DIR = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-mcode-object-version=5",
    # no packed-fp32 instructions anywhere: some of their forms have given silent wrong results on
    # these boxes; hipcc's host pass warns that it does not know the feature, which is harmless
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]
REMARKS = "-Rpass-analysis=kernel-resource-usage"


def _stamp(src):
    """Hash of a source, the headers it can include and the flags: identifies the build a report is from."""
    h = hashlib.sha256(" ".join(FLAGS).encode())
    for p in [src] + sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")) + \
            sorted(os.path.join(ROOT, "include", f) for f in os.listdir(os.path.join(ROOT, "include"))):
        with open(p, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def _report_path(src):
    return os.path.join(BUILD_DIR, os.path.basename(src) + ".resources.txt")


def _write_report(src, stderr):
    lines = [l for l in stderr.splitlines() if "kernel-resource-usage" in l and "remark:" in l]
    with open(_report_path(src), "w") as f:
        f.write(f"# stamp {_stamp(src)}\n")
        f.write("\n".join(lines) + "\n")


def _compile(src):
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC] + FLAGS + [REMARKS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and "kernel-resource-usage" not in l
                    and not re.match(r"^\s+\d+ \| |^\s+\| \^", l))
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n" + err[-6000:])
    _write_report(src, r.stderr)
    return obj, err


def build(check=False, verbose=False):
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(s)]
    with ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 1)) as ex:
        res = list(ex.map(_compile, srcs))
    tmp = OUT + ".tmp"
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC"] + [o for o, _ in res] + ["-o", tmp],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc link failed:\n" + r.stderr[-6000:])
    os.replace(tmp, OUT)
    if verbose and not check:
        for _, err in res:
            if err.strip():
                print(err[-3000:])
    if check:
        for s in srcs:
            for name, d in resource_report(s).items():
                print(f"{name:55s} VGPR={d.get('VGPRs')} AGPR={d.get('AGPRs')} "
                      f"scratch={d.get('ScratchSize [bytes/lane]')} occ={d.get('Occupancy [waves/SIMD]')} "
                      f"lds={d.get('LDS Size [bytes/block]')}")
    return OUT


def _demangle(names):
    out = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True).stdout.splitlines()
    return [d.replace("(anonymous namespace)::", "").split("(")[0] for d in out]


def resource_report(src):
    """{demangled kernel name: {remark key: value}} for one source, from the current build's report, or from
    a device-only compile when the report is missing or was made from other sources or flags."""
    src = src if os.path.isabs(src) else os.path.join(CSRC, src)
    path = _report_path(src)
    stamp = _stamp(src)
    if not os.path.exists(path) or open(path).readline().split()[-1] != stamp:
        os.makedirs(BUILD_DIR, exist_ok=True)
        r = subprocess.run([HIPCC] + FLAGS + [REMARKS, "--cuda-device-only", "-c", src, "-o", os.devnull],
                           capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n" + r.stderr[-6000:])
        _write_report(src, r.stderr)
    cur, raw = None, {}
    for line in open(path):
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = m.group(1)
            raw[cur] = {}
            continue
        m = re.search(r"remark:\s+([\w \[\]/]+?): (\S+) \[", line)
        if cur and m:
            raw[cur][m.group(1).strip()] = m.group(2)
    names = list(raw)
    return dict(zip(_demangle(names), (raw[n] for n in names))) if names else {}


if __name__ == "__main__":
    print(build(check="--check" in sys.argv, verbose=True))
