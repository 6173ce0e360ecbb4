"""CPU oracle for the 16-token rolling-window attention -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.

window_forward / window_backward restate SharedMixer._window (/root/reference/gqa25/memlm_sh.py:349-359):
scaled dot-product attention over (B, H, T, D) with the band mask
    allowed[i, j] = (i >= j) & (i - j < W)                      (memlm_sh.py:341-345, 355)
and the default scale 1/sqrt(D) (F.scaled_dot_product_attention / flex attention with no scale argument):
    s[i, j] = scale <q_i, k_j>,  p[i, :] = softmax over the allowed j,  o_i = sum_j p[i, j] v_j.
Grouped queries: query head hq reads key/value head hq // (Hq / Hk).  This is the kv_nq path
(memlm_sh.py:488-492), whose second window call attends the Hq = KVH * (kv_nq - 1) extra queries to
ck.repeat_interleave(kv_nq - 1, dim=1) -- the same mapping.  Every query has at least one allowed key (its
own position), so no row is empty.

The backward is the textbook softmax-attention adjoint:
    dv_j = sum_i p[i, j] do_i,  dp[i, j] = <do_i, v_j>,  ds[i, j] = p[i, j] (dp[i, j] - <do_i, o_i>),
    dq_i = scale sum_j ds[i, j] k_j,  dk_j = scale sum_i ds[i, j] q_i,
with dk, dv summed over the query heads that share a key/value head.

Pinning (tests/test_oracle_window.py): window_forward and window_backward against torch's
scaled_dot_product_attention with the boolean band mask and torch autograd, in float64 (a library routine
the reference's own CPU path calls, memlm_sh.py:359), and window_forward against a per-query loop over the
allowed keys on tiny inputs.
"""
import numpy as np


def band(T, W):
    i = np.arange(T)
    return (i[:, None] >= i[None, :]) & ((i[:, None] - i[None, :]) < W)


def _expand(k, Hq):
    Hk = k.shape[1]
    if Hq % Hk:
        raise ValueError(f"query heads {Hq} must be a multiple of key/value heads {Hk}")
    return np.repeat(k, Hq // Hk, axis=1)


def window_forward(q, k, v, W, scale=None):
    """q (B, Hq, T, D), k and v (B, Hk, T, D) -> (o (B, Hq, T, D), p (B, Hq, T, T)), float64."""
    q = np.asarray(q, np.float64)
    B, Hq, T, D = q.shape
    sc = 1.0 / np.sqrt(D) if scale is None else scale
    ke = _expand(np.asarray(k, np.float64), Hq)
    ve = _expand(np.asarray(v, np.float64), Hq)
    s = np.einsum("bhid,bhjd->bhij", q, ke) * sc
    m = band(T, W)
    s = np.where(m, s, -np.inf)
    s = s - s.max(-1, keepdims=True)
    e = np.exp(s)
    p = e / e.sum(-1, keepdims=True)
    return np.einsum("bhij,bhjd->bhid", p, ve), p


def window_backward(q, k, v, W, do, scale=None):
    """Gradients (dq, dk, dv) of sum(o * do)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    do = np.asarray(do, np.float64)
    B, Hq, T, D = q.shape
    Hk = k.shape[1]
    sc = 1.0 / np.sqrt(D) if scale is None else scale
    o, p = window_forward(q, k, v, W, scale)
    ke, ve = _expand(k, Hq), _expand(v, Hq)
    dve = np.einsum("bhij,bhid->bhjd", p, do)
    dp = np.einsum("bhid,bhjd->bhij", do, ve)
    ds = p * (dp - (do * o).sum(-1, keepdims=True))
    dq = sc * np.einsum("bhij,bhjd->bhid", ds, ke)
    dke = sc * np.einsum("bhij,bhid->bhjd", ds, q)
    r = Hq // Hk
    dk = dke.reshape(B, Hk, r, T, D).sum(2)
    dv = dve.reshape(B, Hk, r, T, D).sum(2)
    return dq, dk, dv


def window_loop(q, k, v, W, scale=None):
    """Per-query loop over the allowed keys (independent indexing; tiny inputs only)."""
    q = np.asarray(q, np.float64)
    B, Hq, T, D = q.shape
    Hk = k.shape[1]
    sc = 1.0 / np.sqrt(D) if scale is None else scale
    o = np.zeros_like(q)
    for b in range(B):
        for h in range(Hq):
            hk = h // (Hq // Hk)
            for i in range(T):
                js = list(range(max(0, i - W + 1), i + 1))
                s = np.array([sc * float(np.dot(q[b, h, i], k[b, hk, j])) for j in js])
                e = np.exp(s - s.max())
                w = e / e.sum()
                for wj, j in zip(w, js):
                    o[b, h, i] += wj * np.asarray(v[b, hk, j], np.float64)
    return o
