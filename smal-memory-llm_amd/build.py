"""Build libslotscan.so (the gfx950 slot-scan / slot-read kernels and their C-ABI) in place.

    python smal-memory-llm_amd/build.py            # compile
    python smal-memory-llm_amd/build.py --check    # also print per-kernel VGPR / scratch / LDS use

hipcc cross-compiles for gfx950 without a GPU.  The library is linked against libamdhip64.so.7 by SONAME,
so inside a process that imported torch first it binds to torch's own HIP runtime (one runtime, one set of
streams).  Code object v5 is requested explicitly so that runtimes older than the compiler load it.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCES = [os.path.join(HERE, "csrc", f) for f in ("slotscan.hip", "slotread.hip", "slotmem.hip", "slotwin.hip", "slotgen.hip")]
OUT = os.path.join(HERE, "libslotscan.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-mcode-object-version=5",
    # no packed-fp32 instructions anywhere: some of their forms have given silent wrong results on
    # these boxes; hipcc's host pass warns that it does not know the feature, which is harmless
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]


def build(check=False, verbose=False):
    srcs = [s for s in SOURCES if os.path.exists(s)]
    tmp = OUT + ".tmp"
    cmd = [HIPCC] + FLAGS + (["-Rpass-analysis=kernel-resource-usage"] if check else []) + srcs + ["-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + err[-6000:])
    os.replace(tmp, OUT)
    if verbose and err.strip() and not check:
        print(err[-3000:])
    if check:
        _print_resources(r.stderr)
    return OUT


def _print_resources(log):
    import re
    cur, out = None, {}
    for line in log.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = m.group(1)
            out[cur] = {}
            continue
        m = re.search(r"remark:\s+([\w \[\]/]+?): (\S+) \[", line)
        if cur and m:
            out[cur][m.group(1).strip()] = m.group(2)
    for f, d in out.items():
        dm = subprocess.run(["c++filt", f], capture_output=True, text=True).stdout.strip()
        dm = dm.replace("(anonymous namespace)::", "").split("(")[0]
        print(f"{dm:55s} VGPR={d.get('VGPRs')} AGPR={d.get('AGPRs')} scratch={d.get('ScratchSize [bytes/lane]')} "
              f"occ={d.get('Occupancy [waves/SIMD]')} lds={d.get('LDS Size [bytes/block]')}")


if __name__ == "__main__":
    print(build(check="--check" in sys.argv, verbose=True))
