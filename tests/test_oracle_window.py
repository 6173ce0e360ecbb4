"""The window-attention oracle (oracle/window_oracle.py) pinned against torch's scaled_dot_product_attention
with the reference's boolean band mask (memlm_sh.py:341-345, 359) and torch autograd in float64, and against
a per-query loop.  CPU only."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import window_oracle as WO


def _inputs(B, Hq, Hk, T, D, seed):
    g = np.random.default_rng(seed)
    q = g.standard_normal((B, Hq, T, D))
    k = g.standard_normal((B, Hk, T, D))
    v = g.standard_normal((B, Hk, T, D))
    do = g.standard_normal((B, Hq, T, D))
    return q, k, v, do


def _torch_ref(q, k, v, W, do):
    qt, kt, vt = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    r = q.shape[1] // k.shape[1]
    T = q.shape[2]
    i = torch.arange(T)
    m = (i[:, None] >= i[None, :]) & ((i[:, None] - i[None, :]) < W)
    o = F.scaled_dot_product_attention(qt, kt.repeat_interleave(r, dim=1), vt.repeat_interleave(r, dim=1),
                                       attn_mask=m)
    o.backward(torch.tensor(do))
    return o.detach().numpy(), qt.grad.numpy(), kt.grad.numpy(), vt.grad.numpy()


@pytest.mark.parametrize("B,Hq,Hk,T,D,W", [(2, 4, 4, 40, 16, 16), (1, 6, 2, 37, 8, 5), (1, 3, 1, 20, 32, 1),
                                           (2, 2, 2, 9, 8, 16)])
def test_window_oracle_matches_torch_sdpa(B, Hq, Hk, T, D, W):
    q, k, v, do = _inputs(B, Hq, Hk, T, D, 1)
    o, _ = WO.window_forward(q, k, v, W)
    dq, dk, dv = WO.window_backward(q, k, v, W, do)
    ro, rdq, rdk, rdv = _torch_ref(q, k, v, W, do)
    for a, b in ((o, ro), (dq, rdq), (dk, rdk), (dv, rdv)):
        np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12)


def test_window_oracle_matches_loop():
    q, k, v, _ = _inputs(1, 4, 2, 13, 8, 2)
    o, _ = WO.window_forward(q, k, v, 4)
    np.testing.assert_allclose(o, WO.window_loop(q, k, v, 4), rtol=1e-12, atol=1e-12)


def test_window_one_is_identity_on_values():
    """W = 1: every query sees only its own key, so o = v exactly."""
    q, k, v, _ = _inputs(1, 2, 2, 11, 8, 3)
    o, p = WO.window_forward(q, k, v, 1)
    np.testing.assert_allclose(o, v, rtol=0, atol=1e-15)
    assert np.array_equal(p, np.broadcast_to(np.eye(11), p.shape))


def test_window_oracle_finite_differences():
    q, k, v, do = _inputs(1, 2, 1, 7, 4, 4)
    dq, dk, dv = WO.window_backward(q, k, v, 4, do)
    f = lambda q_, k_, v_: float((WO.window_forward(q_, k_, v_, 4)[0] * do).sum())
    h = 1e-6
    for arr, grad, name in ((q, dq, "q"), (k, dk, "k"), (v, dv, "v")):
        idx = (0, 0, 3, 1)
        xp, xm = arr.copy(), arr.copy()
        xp[idx] += h
        xm[idx] -= h
        args_p = {"q": (xp, k, v), "k": (q, xp, v), "v": (q, k, xp)}[name]
        args_m = {"q": (xm, k, v), "k": (q, xm, v), "v": (q, k, xm)}[name]
        fd = (f(*args_p) - f(*args_m)) / (2 * h)
        assert abs(fd - grad[idx]) < 1e-6 * max(1.0, abs(fd)), name
