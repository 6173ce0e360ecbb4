"""The allocation-free backward, slotscan_bwd_noalloc, through the C-ABI: the same results as slotscan_bwd with a
caller-provided workspace, bitwise (the same kernels on the same inputs), on two calls in a row -- the second
with a smaller input, so it runs on the static scratch the first call left behind -- and a shape whose
scratch would exceed the array is refused before any GPU work."""
import ctypes

import pytest
import torch

import slotscan_lib as L
from scan_inputs import scan_inputs, upstream

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import slotkern_hip as KH

DEV = "cuda"
TEMP = 16.0


def _backward(noalloc, B, T, H, N, D, G, seed, dtype):
    """Forward with the undo log (slotkern_hip's own forward), then one backward call through the C-ABI.
    Returns the six gradient tensors."""
    k, q, v, g, fr = (x.to(DEV) for x in scan_inputs(B, T, H, D, seed, dtype=dtype))
    NB = (T + G - 1) // G
    dkbuf, dvbuf = (x.to(DEV) for x in upstream((B, NB, H, N, D), seed + 1))
    dt, k_, q_, v_, g_, fr_, frt, temp_ = KH._prep(k, q, v, g, fr, torch.tensor(TEMP, device=DEV), False)
    _kb, _vb, am, kold, vold, oold, cslog, kfin, vfin, ofin = KH._fwd(k_, q_, v_, g_, fr_, frt, temp_, N, G, 1e-4,
                                                                      True, dt, logs=True)
    dk, dq, dv = torch.empty_like(k_), torch.empty_like(q_), torch.empty_like(v_)
    dg = torch.empty(B, T, H, device=DEV)
    dfr = torch.empty_like(fr_)
    dtemp = torch.empty(1, device=DEV)
    head = (L.ptr(k_), L.ptr(q_), L.ptr(v_), L.dtype_code(dt), L.ptr(g_), L.ptr(fr_), int(frt), L.ptr(temp_),
            B, T, H, N, D, G, 1e-4, 1, L.ptr(am), L.ptr(kold), L.ptr(vold), L.ptr(oold), L.ptr(cslog),
            L.ptr(kfin), L.ptr(vfin), L.ptr(ofin), L.ptr(dkbuf), L.ptr(dvbuf))
    tail = (L.ptr(dk), L.ptr(dq), L.ptr(dv), L.ptr(dg), L.ptr(dfr), L.ptr(dtemp), L.stream_of(torch.device(DEV)))
    if noalloc:
        L.check(L.lib().slotscan_bwd_noalloc(*head, *tail), "slotscan_bwd_noalloc")
    else:
        ws = torch.empty(L.lib().slotscan_bwd_workspace(B, T, H, N), device=DEV, dtype=torch.uint8)
        L.check(L.lib().slotscan_bwd(*head, L.ptr(ws), *tail), "slotscan_bwd")
    torch.cuda.synchronize()
    return dk, dq, dv, dg, dfr, dtemp


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_backward_equals_workspace_backward(dtype):
    for case in ((2, 256, 3, 192, 128, 8, 61), (1, 100, 2, 40, 64, 7, 62)):   # the second call is smaller
        print(f"noalloc case B{case[0]} T{case[1]} H{case[2]} N{case[3]} D{case[4]} G{case[5]} {dtype}", flush=True)
        ref = _backward(False, *case, dtype)
        got = _backward(True, *case, dtype)
        for name, x, y in zip(("dk", "dq", "dv", "dgate", "dfr", "dtemp"), ref, got):
            assert torch.equal(x, y), name


def test_noalloc_refuses_shapes_beyond_its_scratch():
    vp = lambda: ctypes.c_void_p(1 << 20)
    B, T, H, N = 64, 1024, 6, 192                       # config 2: 302 MB of Dn, beyond the 64 MiB array
    assert L.lib().slotscan_bwd_workspace(B, T, H, N) > 64 << 20
    rc = L.lib().slotscan_bwd_noalloc(vp(), vp(), vp(), 0, vp(), vp(), 1, vp(), B, T, H, N, 128, 8, 1e-4, 1,
                                      *[vp() for _ in range(17)])
    assert rc == 1 and b"exceeds the static scratch" in L.lib().slotscan_last_error()
