"""CPU checks that pin the scan oracle (oracle/scan_oracle.py) before it is trusted to judge the HIP path.

Forward: closed forms, fill-order and tie-break rules, stride and chunking identities, the per-token /
scalar fr identity, and an independent scalar loop.  Backward: torch autograd of an independent torch
forward (oracle/torch_scan.py) in every mode, and central finite differences in soft mode."""
import itertools
import math

import numpy as np
import pytest
import torch

from oracle import scan_oracle as SO
from oracle.torch_scan import scan_torch


def _inputs(B, T, H, DK, DV, seed, per_token_fr=False, sep_q=False, clustered=False):
    rng = np.random.default_rng(seed)
    if clustered:                               # taken rows genuinely compete with the free row (test_frtok.py:13-17)
        cen = rng.standard_normal((B, 4, H, DK))
        idx = rng.integers(0, 4, (B, T))
        k = np.take_along_axis(cen, idx[:, :, None, None].repeat(H, 2).repeat(DK, 3), 1)
        k = k + 0.3 * rng.standard_normal((B, T, H, DK))
    else:
        k = rng.standard_normal((B, T, H, DK))
    q = k + 0.2 * rng.standard_normal((B, T, H, DK)) if sep_q else None
    v = rng.standard_normal((B, T, H, DV))
    g = 1 / (1 + np.exp(-rng.standard_normal((B, T, H))))
    fr = rng.uniform(0, 2, (B, T, H)) if per_token_fr else np.array([1.5])
    return k, q, v, g, fr


# ---------------------------------------------------------------------------------------------- forward


def test_first_write_closed_form():
    """Every row empty: only row 0 competes, so step 0 writes g*k_0 into row 0 (and g into o_0)."""
    k, q, v, g, fr = _inputs(2, 2, 3, 5, 4, 0)
    kb, vb, info = SO.scan_forward(k, v, g, fr, 6, 16.0, G=1, hard=True, occ_bin=True)
    assert np.all(info["am"][:, 0] == 0)
    np.testing.assert_array_equal(kb[:, 1, :, 0], g[:, 0, :, None] * k[:, 0])
    np.testing.assert_array_equal(vb[:, 1, :, 0], g[:, 0, :, None] * v[:, 0])
    np.testing.assert_array_equal(info["obuf"][:, 1, :, 0], g[:, 0])
    assert np.all(kb[:, 1, :, 1:] == 0) and np.all(kb[:, 0] == 0)


def test_gate_one_copies_and_gate_zero_is_noop():
    k, q, v, g, fr = _inputs(1, 6, 2, 4, 4, 1)
    g[:] = 1.0
    g[:, 3] = 0.0
    kb, vb, info = SO.scan_forward(k, v, g, fr, 8, 16.0, G=1, hard=True, occ_bin=True)
    for t in range(5):
        for h in range(2):
            r = info["am"][0, t, h]
            if t == 3:
                np.testing.assert_array_equal(kb[0, t + 1, h], kb[0, t, h])      # g = 0 writes nothing
            else:
                np.testing.assert_array_equal(kb[0, t + 1, h, r], k[0, t, h])    # g = 1 copies the key
                np.testing.assert_array_equal(vb[0, t + 1, h, r], v[0, t, h])


@pytest.mark.parametrize("occ_bin", [False, True])
def test_first_free_fill_order(occ_bin):
    """fr/temp > 1: no cosine can beat a free row, so tokens fill rows 0..N-1 in order (slotkern_kv.py:46-51)."""
    N = 7
    k, q, v, g, fr = _inputs(2, N + 3, 2, 6, 6, 2)
    g = 0.5 + 0.5 * g
    kb, vb, info = SO.scan_forward(k, v, g, np.array([40.0]), N, 16.0, G=1, hard=True, occ_bin=occ_bin)
    assert np.all(info["am"][:, :N] == np.arange(N)[None, :, None])


def test_tie_goes_to_lowest_index():
    """Two occupied rows holding the same key score identically; the lower index must win."""
    B, T, H, D, N = 1, 5, 1, 4, 6
    rng = np.random.default_rng(3)
    key = rng.standard_normal(D)
    k = np.tile(key, (B, T, H, 1))
    v = rng.standard_normal((B, T, H, D))
    g = np.ones((B, T, H))
    fr = np.zeros((B, T, H))
    fr[:, :2] = 100.0                       # first two tokens take rows 0 and 1
    kb, vb, info = SO.scan_forward(k, v, g, fr, N, 16.0, G=1, hard=True, occ_bin=True)
    assert list(info["am"][0, :, 0]) == [0, 1, 0, 0, 0]


def test_soft_write_goes_only_to_first_free_row():
    k, q, v, g, fr = _inputs(1, 1, 2, 4, 4, 4)
    kb, vb, info = SO.scan_forward(k, v, g, fr, 5, 16.0, G=1, hard=False)
    K1 = SO.scan_forward(np.concatenate([k, k], 1), np.concatenate([v, v], 1), np.concatenate([g, g], 1),
                         fr, 5, 16.0, G=1, hard=False)[0][:, 1]
    np.testing.assert_array_equal(K1[:, :, 0], g[:, 0, :, None] * k[:, 0])
    assert np.all(K1[:, :, 1:] == 0)


@pytest.mark.parametrize("hard", [False, True])
def test_stride_copies_equal_per_step_state(hard):
    k, q, v, g, fr = _inputs(2, 23, 2, 5, 3, 5, per_token_fr=True, sep_q=True)
    k1, v1, _ = SO.scan_forward(k, v, g, fr, 6, 16.0, G=1, hard=hard, q=q, occ_bin=True)
    k4, v4, _ = SO.scan_forward(k, v, g, fr, 6, 16.0, G=4, hard=hard, q=q, occ_bin=True)
    assert k4.shape[1] == 6
    np.testing.assert_array_equal(k4, k1[:, ::4])
    np.testing.assert_array_equal(v4, v1[:, ::4])


@pytest.mark.parametrize("hard", [False, True])
def test_constant_token_fr_equals_scalar(hard):
    """test_frtok.py:56-70: a constant per-token fr is the scalar path; forward identical, sum dfr == dfr."""
    k, q, v, g, _ = _inputs(2, 20, 3, 6, 6, 6, sep_q=True, clustered=True)
    frs = np.array([9.0])
    frt = np.full(g.shape, 9.0)
    a = SO.scan_forward(k, v, g, frs, 8, 16.0, G=4, hard=hard, q=q, occ_bin=True)
    b = SO.scan_forward(k, v, g, frt, 8, 16.0, G=4, hard=hard, q=q, occ_bin=True)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])
    rng = np.random.default_rng(0)
    dkb, dvb = rng.standard_normal(a[0].shape), rng.standard_normal(a[1].shape)
    ga = SO.scan_backward(k, v, g, frs, 8, 16.0, a[0], a[1], a[2], dkb, dvb, G=4, hard=hard, q=q, occ_bin=True)
    gb = SO.scan_backward(k, v, g, frt, 8, 16.0, b[0], b[1], b[2], dkb, dvb, G=4, hard=hard, q=q, occ_bin=True)
    assert gb["dfr"].shape == g.shape
    assert abs(ga["dfr"][0] - gb["dfr"].sum()) <= 1e-12 * max(1.0, abs(ga["dfr"][0]))


@pytest.mark.parametrize("occ_bin", [False, True])
def test_chunked_scan_with_carried_state_is_identical(occ_bin):
    k, q, v, g, fr = _inputs(2, 24, 2, 5, 4, 7, per_token_fr=True, sep_q=True)
    kb, vb, info = SO.scan_forward(k, v, g, fr, 6, 16.0, G=4, hard=True, q=q, occ_bin=occ_bin)
    state, parts = None, []
    for c0 in (0, 8, 16):
        sl = slice(c0, c0 + 8)
        kc, vc, ic = SO.scan_forward(k[:, sl], v[:, sl], g[:, sl], fr[:, sl], 6, 16.0, G=4, hard=True, q=q[:, sl],
                                     occ_bin=occ_bin, state=state)
        state = (ic["kfin"], ic["vfin"], ic["ofin"])
        parts.append((kc, vc, ic["am"]))
    np.testing.assert_array_equal(np.concatenate([p[0] for p in parts], 1), kb)
    np.testing.assert_array_equal(np.concatenate([p[1] for p in parts], 1), vb)
    np.testing.assert_array_equal(np.concatenate([p[2] for p in parts], 1), info["am"])
    np.testing.assert_array_equal(state[0], info["kfin"])


def _scalar_scan(k, v, g, fr, N, temp, hard, eps=1e-4, occ_bin=True):
    """Pure-Python scalar loop (one chain at a time) -- independent indexing of the same rules."""
    B, T, H, D = len(k), len(k[0]), len(k[0][0]), len(k[0][0][0])
    out = []
    for b in range(B):
        for h in range(H):
            K = [[0.0] * D for _ in range(N)]
            o = [0.0] * N
            hist = []
            for t in range(T):
                hist.append([row[:] for row in K])
                qt = [k[b][t][h][d] for d in range(D)]
                qn = math.sqrt(sum(x * x for x in qt))
                z = []
                first_free_seen = False
                for n in range(N):
                    kn = math.sqrt(sum(x * x for x in K[n]))
                    s = temp * sum(K[n][d] / max(kn, 1e-6) * qt[d] / max(qn, 1e-6) for d in range(D))
                    occ = (1.0 if o[n] >= eps else 0.0) if occ_bin else o[n]
                    zn = s - fr * occ
                    if o[n] < eps:
                        if first_free_seen:
                            zn = None
                        first_free_seen = True
                    z.append(zn)
                cand = [n for n in range(N) if z[n] is not None]
                if hard:
                    best = cand[0]
                    for n in cand[1:]:
                        if z[n] > z[best]:
                            best = n
                    a = [1.0 if n == best else 0.0 for n in range(N)]
                else:
                    m = max(z[n] for n in cand)
                    e = [math.exp(z[n] - m) if z[n] is not None else 0.0 for n in range(N)]
                    ssum = sum(e)
                    a = [x / ssum for x in e]
                gg = g[b][t][h]
                for n in range(N):
                    w = gg * a[n]
                    K[n] = [(1 - w) * K[n][d] + w * k[b][t][h][d] for d in range(D)]
                    o[n] = (1 - w) * o[n] + w
            out.append(((b, h), hist))
    return out


@pytest.mark.parametrize("hard", [False, True])
def test_forward_matches_independent_scalar_loop(hard):
    k, q, v, g, fr = _inputs(2, 9, 2, 3, 3, 8, clustered=True)
    kb, vb, info = SO.scan_forward(k, v, g, np.array([1.0]), 5, 16.0, G=1, hard=hard, occ_bin=True)
    for (b, h), hist in _scalar_scan(k.tolist(), v.tolist(), g.tolist(), 1.0, 5, 16.0, hard):
        np.testing.assert_allclose(kb[b, :, h], np.array(hist), rtol=0, atol=1e-12)


# --------------------------------------------------------------------------------------------- backward

MODES = [  # hard, detach, occ_bin, per_token_fr, hard_gate, pin, sep_q, G
    (True, True, True, True, False, False, True, 4),     # the training setting (run_sh25.sh:213-224)
    (True, True, True, False, False, False, False, 5),
    (True, True, False, True, False, False, True, 3),
    (True, True, True, True, True, False, True, 4),
    (True, False, True, True, False, True, True, 4),
    (False, True, True, True, False, False, True, 4),
    (False, False, False, False, False, True, False, 1),
    (False, False, True, True, False, True, True, 6),
    (False, True, False, False, True, False, True, 3),
    (True, False, False, False, False, True, False, 2),
]


@pytest.mark.parametrize("hard,detach,occ_bin,frt,hardg,pin,sep_q,G", MODES)
def test_backward_matches_torch_autograd(hard, detach, occ_bin, frt, hardg, pin, sep_q, G):
    B, T, H, N, DK, DV = 2, 13, 2, 5, 4, 3
    k, q, v, g, fr = _inputs(B, T, H, DK, DV, 11, per_token_fr=frt, sep_q=sep_q, clustered=True)
    if frt:
        fr = fr * 4.0
    temp = 16.0
    kb, vb, info = SO.scan_forward(k, v, g, fr, N, temp, G=G, hard=hard, hard_gate=hardg, detach_addr=detach, q=q,
                                   pin=pin, occ_bin=occ_bin)
    rng = np.random.default_rng(12)
    dkb, dvb = rng.standard_normal(kb.shape), rng.standard_normal(vb.shape)
    got = SO.scan_backward(k, v, g, fr, N, temp, kb, vb, info, dkb, dvb, G=G, hard=hard, hard_gate=hardg,
                           detach_addr=detach, q=q, pin=pin, occ_bin=occ_bin)
    L = {n: torch.tensor(x, dtype=torch.float64, requires_grad=True)
         for n, x in dict(k=k, v=v, g=g, fr=fr, q=q, temp=np.array(temp)).items() if x is not None}
    kt, vt = scan_torch(L["k"], L["v"], L["g"], L["fr"], N, L["temp"], G=G, hard=hard, hard_gate=hardg, eps=1e-4,
                        detach_addr=detach, q=L.get("q"), pin=pin, occ_bin=occ_bin,
                        teacher=torch.tensor(info["am"]) if hard else None)
    np.testing.assert_allclose(kt.detach().numpy(), kb, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(vt.detach().numpy(), vb, rtol=1e-12, atol=1e-12)
    ((kt * torch.tensor(dkb)).sum() + (vt * torch.tensor(dvb)).sum()).backward()
    ref = dict(dk=L["k"].grad, dv=L["v"].grad, dgate=L["g"].grad, dfr=L["fr"].grad, dtemp=L["temp"].grad)
    mine = dict(dk=got["dk"] + (0 if sep_q else got["dq"]), dv=got["dv"], dgate=got["dgate"], dfr=got["dfr"],
                dtemp=got["dtemp"])
    if sep_q:
        ref["dq"], mine["dq"] = L["q"].grad, got["dq"]
    for name in ref:
        r = ref[name].numpy().reshape(np.shape(mine[name]))
        scale = max(np.abs(r).max(), 1e-12)
        err = np.abs(np.asarray(mine[name]) - r).max() / scale
        assert err < 1e-10, (name, err)


@pytest.mark.parametrize("occ_bin", [False, True])
def test_backward_matches_finite_differences_soft(occ_bin):
    """Soft, attached address: the scan is smooth, so central differences in float64 pin every gradient.
    (A detached address is deliberately NOT the derivative of the forward, so it is pinned by autograd only.)"""
    detach = False
    B, T, H, N, DK, DV, G = 1, 9, 2, 4, 3, 3, 3
    k, q, v, g, fr = _inputs(B, T, H, DK, DV, 21, per_token_fr=True, sep_q=True, clustered=True)
    temp = 5.0
    rng = np.random.default_rng(22)
    args = dict(G=G, hard=False, detach_addr=detach, occ_bin=occ_bin)

    def loss(kk, qq, vv, gg, ff, tt):
        kb, vb, _ = SO.scan_forward(kk, vv, gg, ff, N, tt, q=qq, **args)
        return (kb * wk).sum() + (vb * wv).sum()

    kb, vb, info = SO.scan_forward(k, v, g, fr, N, temp, q=q, **args)
    wk, wv = rng.standard_normal(kb.shape), rng.standard_normal(vb.shape)
    got = SO.scan_backward(k, v, g, fr, N, temp, kb, vb, info, wk, wv, q=q, **args)
    base = dict(kk=k, qq=q, vv=v, gg=g, ff=fr, tt=np.array(temp))
    names = dict(kk="dk", qq="dq", vv="dv", gg="dgate", ff="dfr", tt="dtemp")
    for key, gname in names.items():
        dirn = rng.standard_normal(np.shape(base[key]))
        eps = 1e-6
        plus = dict(base)
        minus = dict(base)
        plus[key] = base[key] + eps * dirn
        minus[key] = base[key] - eps * dirn
        fd = (loss(**plus) - loss(**minus)) / (2 * eps)
        an = float((np.asarray(got[gname]) * dirn).sum())
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(fd)), (gname, fd, an)


def test_hard_gradient_is_soft_gradient_at_hard_state():
    """Straight-through: in hard mode dz comes from the SOFT softmax of the hard trajectory's scores."""
    k, q, v, g, fr = _inputs(1, 10, 2, 4, 4, 31, per_token_fr=True, sep_q=True, clustered=True)
    kb, vb, info = SO.scan_forward(k, v, g, fr, 5, 16.0, G=2, hard=True, q=q, occ_bin=True, detach_addr=True)
    rng = np.random.default_rng(0)
    dkb, dvb = rng.standard_normal(kb.shape), rng.standard_normal(vb.shape)
    got = SO.scan_backward(k, v, g, fr, 5, 16.0, kb, vb, info, dkb, dvb, G=2, hard=True, q=q, occ_bin=True,
                           detach_addr=True)
    assert np.all(np.isfinite(got["dq"])) and np.abs(got["dq"]).max() > 0
    assert np.abs(got["dfr"]).max() > 0 and np.abs(got["dtemp"]) > 0


def test_teacher_forcing_follows_given_rows():
    k, q, v, g, fr = _inputs(1, 12, 1, 4, 4, 41, per_token_fr=True, clustered=True)
    kb, vb, info = SO.scan_forward(k, v, g, fr, 6, 16.0, G=1, hard=True, occ_bin=True)
    kb2, vb2, info2 = SO.scan_forward(k, v, g, fr, 6, 16.0, G=1, hard=True, occ_bin=True, teacher=info["am"])
    np.testing.assert_array_equal(kb, kb2)
    assert info2["agree"].all() and np.all(info2["margin"] == 0)
