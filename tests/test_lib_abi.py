"""CPU checks of the C-ABI library: it loads, exports every function include/*.h declares, and its host-side
argument validation rejects bad calls with the documented codes before any GPU work is attempted."""
import ctypes
import glob
import os
import re

import pytest

import slotscan_lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        txt = open(h).read()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        names += re.findall(r"^[A-Za-z_][\w \*]*?\b(\w+)\s*\(", txt, flags=re.M)
    return sorted(set(n for n in names if n.startswith("slot")))


def test_every_declared_symbol_is_exported_and_bound():
    lib = L.lib()
    names = _declared()
    assert len(names) >= 5
    for n in names:
        assert hasattr(lib, n), f"{n} is declared in include/ but not exported"
        assert n in L.SIGNATURES, f"{n} has no ctypes signature in slotscan_lib"


def _declared_arity():
    """name -> number of parameters, from every prototype in include/*.h."""
    out = {}
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        txt = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(slot\w+)\s*\(([^)]*)\)\s*;", txt, flags=re.M):
            params = m.group(2).strip()
            out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_ctypes_signatures_match_the_prototypes():
    """Every binding in slotscan_lib passes exactly as many arguments as the C prototype takes: a missing or
    extra pointer would shift every later argument of the call."""
    arity = _declared_arity()
    assert set(arity) == set(_declared())
    for name, n in arity.items():
        assert len(L.SIGNATURES[name][1]) == n, f"{name}: ctypes binds {len(L.SIGNATURES[name][1])} args, C has {n}"


def test_single_hip_runtime_in_process():
    """The library binds to the HIP runtime torch already loaded (same SONAME), not a second copy."""
    L.lib()
    maps = open("/proc/self/maps").read()
    libs = set(re.findall(r"(\S*libamdhip64\.so\S*)", maps))
    assert len(libs) == 1, libs


@pytest.mark.parametrize("B,T,H,N,chunks", [
    (3, 100, 2, 40, 2),        # 7 windows of 16 steps, at least 4 per chunk
    (64, 1024, 6, 192, 2),     # config 2: 384 chains x 2 chunks of 32 windows = 768 workgroups
    (512, 128, 6, 96, 1),      # config 3, (512, 128): 3,072 chains already, one chunk each
    (1, 8, 1, 16, 1),
])
def test_workspace_size(B, T, H, N, chunks):
    """Dn (B*H, N, T) fp32, 256-byte aligned, then two fp32 partials per chain and time chunk of the address
    backward."""
    dn = B * H * N * T * 4
    assert L.lib().slotscan_bwd_workspace(B, T, H, N) == ((dn + 255) & ~255) + B * H * chunks * 2 * 4


def _fwd_call(**over):
    a = dict(k=1 << 20, q=1 << 20, v=1 << 20, dtype=0, gate=1 << 20, fr=1 << 20, frt=1, temp=1 << 20,
             B=1, T=8, H=1, N=16, D=64, G=8, eps=1e-4, occ=1, k0=None, v0=None, o0=None,
             kbuf=1 << 20, vbuf=1 << 20, am=1 << 20, kold=None, vold=None, oold=None, cslog=None,
             kfin=1 << 20, vfin=1 << 20, ofin=1 << 20)
    a.update(over)
    vp = lambda x: None if x is None else ctypes.c_void_p(x)
    return L.lib().slotscan_fwd(vp(a["k"]), vp(a["q"]), vp(a["v"]), a["dtype"], vp(a["gate"]), vp(a["fr"]),
                                a["frt"], vp(a["temp"]), a["B"], a["T"], a["H"], a["N"], a["D"], a["G"],
                                a["eps"], a["occ"], vp(a["k0"]), vp(a["v0"]), vp(a["o0"]), vp(a["kbuf"]),
                                vp(a["vbuf"]), vp(a["am"]), vp(a["kold"]), vp(a["vold"]), vp(a["oold"]),
                                vp(a["cslog"]), vp(a["kfin"]), vp(a["vfin"]), vp(a["ofin"]), None)


@pytest.mark.parametrize("over,code", [
    (dict(D=96), 1), (dict(N=193), 1), (dict(G=0), 1), (dict(T=0), 1),
    (dict(dtype=7), 2), (dict(k=None), 3), (dict(kold=1 << 20), 3), (dict(k=(1 << 20) + 4), 4),
])
def test_fwd_validation_rejects_before_launch(over, code):
    assert _fwd_call(**over) == code
    assert L.lib().slotscan_last_error()


def test_dtype_codes():
    import torch
    assert L.dtype_code(torch.float32) == L.SLOTSCAN_F32
    assert L.dtype_code(torch.bfloat16) == L.SLOTSCAN_BF16
    with pytest.raises(TypeError):
        L.dtype_code(torch.float16)


@pytest.mark.parametrize("T,H,N,D,G,mem,untracked", [
    (1024, 6, 192, 128, 8, 0, True),        # config 2
    (1024, 6, 192, 128, 8, 1, True),        # config 2, fused epilogue
    (1024, 6, 192, 64, 8, 1, False),        # the fused contract's untracked kernel is built for D = 128
    (1000, 6, 192, 128, 8, 0, False),       # T % 16 != 0
    (1024, 6, 192, 128, 7, 0, False),       # G != 8
    (58240, 6, 192, 128, 8, 0, True),       # NB * H * N * D * 4 = 4,293,918,720 B: just fits 32 bits
    (58256, 6, 192, 128, 8, 0, False),      # 4,295,098,368 B: past 2^32, the tracked kernel runs
    (58256, 6, 192, 128, 8, 1, True),       # bf16 gradients: half the bytes
    (116512, 6, 192, 128, 8, 1, False),
])
def test_bwd_plan_untracked_rows_kernel_guard(T, H, N, D, G, mem, untracked):
    """The untracked G = 8 row kernel forms a batch row's snapshot-gradient offsets in 32 bits: the library
    uses it only where they fit (slotscan_bwd_plan exposes the choice; no GPU work)."""
    plan = L.lib().slotscan_bwd_plan(T, H, N, D, G, mem)
    assert plan >= 0
    assert bool(plan & 1) == untracked
    assert L.lib().slotscan_bwd_plan(0, H, N, D, G, mem) == -1


def test_integration_doc_stubs_match_the_bindings():
    """Every `lib.<name>.argtypes = ...` line of the integration guide at the repository root binds exactly
    the argument list of the C prototype (the same types, in order, as slotscan_lib.SIGNATURES): a maintainer
    copies these stubs."""
    txt = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    found = re.findall(r"^lib\.(\w+)\.argtypes = (.+)$", txt, flags=re.M)
    assert len(found) >= 5
    env = {"vp": ctypes.c_void_p, "i64": ctypes.c_int64, "i32": ctypes.c_int, "f32": ctypes.c_float,
           "ctypes": ctypes}
    arity = _declared_arity()
    for name, expr in found:
        got = eval(expr, env)                                 # noqa: S307 -- the repository's own doc
        assert len(got) == arity[name], f"{name}: the doc binds {len(got)} args, C has {arity[name]}"
        assert got == L.SIGNATURES[name][1], f"{name}: the doc's argument types differ from the binding"


@pytest.mark.parametrize("M,N,K,code", [(0, 256, 64, 1), (8, 300, 64, 1), (8, 256, 48, 1), (8, 256, 64, 3)])
def test_proj_validation_rejects_before_launch(M, N, K, code):
    """slotproj_fwd refuses a shape its tiles do not cover (N a multiple of 256, K of 32) or a NULL operand with
    an error code and message, before any GPU call (so this runs without a GPU)."""
    assert L.lib().slotproj_fwd(None, None, None, M, N, K, None, None) == code
    assert L.lib().slotscan_last_error()


def _codes_call(**over):
    a = dict(B=1, T=8, H=1, N=16, D=64, G=8, bits=8, group=64, kcode=1 << 20, kscale=1 << 20, vcode=1 << 20,
             vscale=1 << 20, kcarry=None)
    a.update(over)
    vp = lambda x: None if x is None else ctypes.c_void_p(x)
    p = vp(1 << 20)
    return L.lib().slotscan_fwd_codes(p, p, p, 0, p, p, 1, p, a["B"], a["T"], a["H"], a["N"], a["D"], a["G"], 1e-4,
                                      1, a["bits"], a["group"], None, None, None, vp(a["kcode"]), vp(a["kscale"]),
                                      vp(a["vcode"]), vp(a["vscale"]), p, p, p, p, vp(a["kcarry"]), None)


@pytest.mark.parametrize("over,code", [
    (dict(bits=1), 1), (dict(bits=9), 1), (dict(group=3), 1), (dict(group=128), 1), (dict(group=2), 1),
    (dict(kcode=None), 3), (dict(vscale=None), 3),
    (dict(T=1024), 3),                        # a multi-chunk forward needs the key replay's carry
    (dict(kcode=(1 << 20) + 4), 4),
])
def test_codes_validation_rejects_before_launch(over, code):
    """slotscan_fwd_codes refuses bad quantiser parameters (bits 2..8, group a power of two in [4, D]), NULL
    outputs, a missing key carry where the forward runs as a pipeline, and misaligned codes, before any GPU
    call."""
    assert _codes_call(**over) == code
    assert L.lib().slotscan_last_error()


@pytest.mark.parametrize("B,T,H,N,D,G,nbytes", [
    (8, 1024, 6, 192, 128, 8, 8 * 6 * 192 * 128 * 4),   # config 5's calls: the 8-chunk pipeline
    (2, 511, 2, 64, 64, 8, 0),                          # one chunk: no carry
    (1, 512, 1, 16, 64, 8, 16 * 64 * 4),
])
def test_fwd_carry_bytes(B, T, H, N, D, G, nbytes):
    assert L.lib().slotscan_fwd_carry_bytes(B, T, H, N, D, G) == nbytes


@pytest.mark.parametrize("M,N,K,code", [(0, 256, 256, 1), (8, 300, 256, 1), (8, 256, 96, 1), (8, 256, 256, 3)])
def test_proj_bwd_validation_rejects_before_launch(M, N, K, code):
    """slotproj_bwd refuses shapes its tiles do not cover (N and K multiples of 256) and NULL operands before
    any GPU call; its workspace holds the transposed weight and the token splits' fp32 partials."""
    assert L.lib().slotproj_bwd(None, None, None, M, N, K, None, None, None, None) == code
    assert L.lib().slotscan_last_error()
    ws = L.lib().slotproj_bwd_workspace(65536, 2048, 768)
    assert ws >= 2048 * 768 * 2 + 2048 * 768 * 4 and (ws - ((2048 * 768 * 2 + 255) & ~255)) % (2048 * 768 * 4) == 0


@pytest.mark.parametrize("which", ["out", "dq", "dk", "dv"])
def test_window_refuses_8_byte_aligned_outputs(which):
    """win_fwd / win_bwd write out, dq, dk and dv as 16-byte row pieces: an 8-byte-aligned output pointer is
    refused with SLOTSCAN_ERR_ALIGN before any GPU call."""
    good, bad = ctypes.c_void_p(1 << 20), ctypes.c_void_p((1 << 20) + 8)
    if which == "out":
        rc = L.lib().slotwin_fwd(good, good, good, 1, 16, 2, 2, 64, 16, 0.125, bad, good, None)
    else:
        o = {n: (bad if n == which else good) for n in ("dq", "dk", "dv")}
        rc = L.lib().slotwin_bwd(good, good, good, good, good, good, 1, 16, 2, 2, 64, 16, 0.125, good, o["dq"], o["dk"],
                                 o["dv"], None)
    assert rc == 4
    assert b"16-byte" in L.lib().slotscan_last_error()
