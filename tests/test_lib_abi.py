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


def test_workspace_size():
    B, T, H, N = 3, 100, 2, 40
    dn = B * H * N * T * 4
    assert L.lib().slotscan_bwd_workspace(B, T, H, N) == ((dn + 255) & ~255) + B * H * 2 * 4


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
