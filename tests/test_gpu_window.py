"""GPU parity of the rolling-window attention (slotwin_hip.window, libslotscan.so's slotwin_fwd / slotwin_bwd)
against the fp64 oracle (oracle/window_oracle.py) on the same bf16 inputs.

Bar: forward and every gradient within 1.5e-2 relative to the tensor's max |value|.  The kernel rounds
what the GPU reference rounds to bf16 -- the exponentials before the value contraction, the score and
probability gradients before theirs, and the bf16 outputs -- each at most 2^-9 relative."""
import numpy as np
import pytest
import torch

from oracle import window_oracle as WO

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import slotwin_hip as WH

DEV = "cuda"


def _rel(a, b):
    """Max error relative to the reference's max |value|, floored at 1e-2: the inputs are N(0, 1), so the
    outputs and gradients are O(1), except where the maths makes them exactly 0 (W = 1: one allowed key,
    p = 1, and dS = dP - <dO, O> = 0, so dq = dk = 0 up to the kernel's bf16 rounding)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-2))


def _case(B, Hq, Hk, T, D, W, seed, views=True):
    print(f"window case B{B} Hq{Hq} Hk{Hk} T{T} D{D} W{W} views={views}", flush=True)
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)
    if views:                      # the reference's operands: (B, T, H, D) tensors viewed as (B, H, T, D)
        q, k, v = r(B, T, Hq, D).transpose(1, 2), r(B, T, Hk, D).transpose(1, 2), r(B, T, Hk, D).transpose(1, 2)
    else:
        q, k, v = r(B, Hq, T, D), r(B, Hk, T, D), r(B, Hk, T, D)
    do = r(B, Hq, T, D)
    qg, kg, vg = (x.to(DEV).requires_grad_() for x in (q, k, v))
    o = WH.window(qg, kg, vg, W)
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    n = lambda x: x.detach().float().cpu().numpy()
    oo, _ = WO.window_forward(n(q), n(k), n(v), W)
    dq, dk, dv = WO.window_backward(n(q), n(k), n(v), W, n(do))
    errs = {"o": _rel(n(o), oo), "dq": _rel(n(qg.grad), dq), "dk": _rel(n(kg.grad), dk), "dv": _rel(n(vg.grad), dv)}
    print("   rel err:", {kk: f"{x:.1e}" for kk, x in errs.items()}, flush=True)
    assert o.shape == q.shape and o.dtype == torch.bfloat16
    for name, e in errs.items():
        assert e < 1.5e-2, f"{name} rel err {e:.3e}"


CASES = [  # B, Hq, Hk, T, D, W
    (2, 4, 4, 256, 128, 16),        # the training window: 4 heads x 128, W = 16 (run_sh25.sh:223)
    (2, 12, 4, 200, 128, 16),       # kv_nq 4: the 12 extra queries on the 4 shared heads, T % 64 != 0
    (1, 3, 1, 70, 64, 7),           # D = 64, W < 16
    (1, 2, 2, 9, 64, 16),           # T < W
    (1, 2, 1, 33, 128, 1),          # W = 1: o = v
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}Hq{}Hk{}T{}D{}W{}".format(*c))
def test_window_matches_oracle(case):
    _case(*case, seed=5)


def test_window_contiguous_operands():
    _case(1, 4, 2, 96, 128, 16, seed=6, views=False)


def test_window_is_deterministic():
    g = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(2, 4, 130, 128, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3))
    do = torch.randn(2, 4, 130, 128, generator=g).to(torch.bfloat16).to(DEV)
    res = []
    for _ in range(2):
        qq, kk, vv = (x.clone().requires_grad_() for x in (q, k, v))
        o = WH.window(qq, kk, vv, 16)
        o.backward(do)
        res.append((o.detach(), qq.grad, kk.grad, vv.grad))
    for x, y in zip(*res):
        assert torch.equal(x, y)


def test_window_refuses_unsupported():
    q = torch.zeros(1, 2, 8, 128, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        WH.window(q, q, q, 17)
    with pytest.raises(NotImplementedError):
        WH.window(q.float(), q.float(), q.float(), 16)
    with pytest.raises(ValueError):
        WH.window(q, q[:, :1].expand(1, 1, 8, 128).contiguous()[:, :, :4], q[:, :1], 16)
