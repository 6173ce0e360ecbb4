"""CPU checks that pin the read / quantiser oracle (oracle/read_oracle.py)."""
import numpy as np
import pytest

from oracle import read_oracle as RO
from oracle import scan_oracle as SO


def _unit(x):
    return x / np.maximum(np.linalg.norm(x, axis=-1, keepdims=True), 1e-6)


def test_strided_read_equals_naive_block_start_read():
    """gqa25/test_sh.py:77-86: the strided (block) read == a per-token read of the state at t0 = (t//G)*G,
    with T not a multiple of G (padded last block) and block 0 reading an empty memory (exactly 0)."""
    B, T, H, NQ, N, D, G = 2, 13, 2, 2, 5, 4, 4
    rng = np.random.default_rng(0)
    k = rng.standard_normal((B, T, H, D))
    v = rng.standard_normal((B, T, H, D))
    g = 1 / (1 + np.exp(-rng.standard_normal((B, T, H))))
    fr = rng.uniform(0, 2, (B, T, H))
    k1, v1, _ = SO.scan_forward(k, v, g, fr, N, 16.0, G=1, hard=True, occ_bin=True)      # every position
    kG, vG, _ = SO.scan_forward(k, v, g, fr, N, 16.0, G=G, hard=True, occ_bin=True)
    NB = kG.shape[1]
    q = _unit(rng.standard_normal((B, T, H, NQ, D)))
    sc_tok = np.exp(np.log(8.0) + 2 * np.tanh(rng.standard_normal((B, T, H, NQ)) / 2))
    # pack tokens into blocks exactly as memlm_sh.py:380-382 (pad T to NB*G, queries of a block are (G*NQ))
    Tp = NB * G
    qp = np.zeros((B, Tp, H, NQ, D)); qp[:, :T] = q
    sp = np.ones((B, Tp, H, NQ)); sp[:, :T] = sc_tok
    qh = qp.reshape(B, NB, G, H, NQ, D).transpose(0, 1, 3, 2, 4, 5).reshape(B, NB, H, G * NQ, D)
    sh = sp.reshape(B, NB, G, H, NQ).transpose(0, 1, 3, 2, 4).reshape(B, NB, H, G * NQ)
    kinv, valid = RO.writer_epilogue(kG)
    rd, _ = RO.read_forward(qh, kG, vG, kinv, valid, sh)
    rd = rd.reshape(B, NB, H, G, NQ, D).transpose(0, 1, 3, 2, 4, 5).reshape(B, Tp, H, NQ, D)[:, :T]
    slow = RO.naive_block_read(q, k1, v1, sc_tok, G)
    np.testing.assert_allclose(rd, slow, rtol=0, atol=1e-12)
    assert np.all(rd[:, :G] == 0.0)                     # block 0: nothing written yet, reads exactly 0


def test_single_valid_row_reads_that_row():
    B, NB, H, M, N, D = 1, 2, 1, 3, 4, 5
    rng = np.random.default_rng(1)
    kbuf = rng.standard_normal((B, NB, H, N, D))
    buf = rng.standard_normal((B, NB, H, N, D))
    valid = np.zeros((B, NB, H, N), bool); valid[..., 2] = True
    kinv = 1 / np.linalg.norm(kbuf, axis=-1)
    rd, _ = RO.read_forward(rng.standard_normal((B, NB, H, M, D)), kbuf, buf, kinv, valid, np.ones((B, NB, H, M)))
    np.testing.assert_allclose(rd, np.broadcast_to(buf[..., 2:3, :], rd.shape), rtol=1e-15)


def test_read_backward_matches_finite_differences():
    B, NB, H, M, N, D = 1, 2, 2, 3, 5, 4
    rng = np.random.default_rng(2)
    x = dict(qh=rng.standard_normal((B, NB, H, M, D)), kbuf=rng.standard_normal((B, NB, H, N, D)),
             buf=rng.standard_normal((B, NB, H, N, D)), kinv=rng.uniform(0.5, 2, (B, NB, H, N)),
             scale=rng.uniform(1, 3, (B, NB, H, M)))
    valid = rng.random((B, NB, H, N)) > 0.3
    valid[0, 1, 1] = False                              # one all-masked block: its gradients must be 0
    drd = rng.standard_normal((B, NB, H, M, D))
    rd, cache = RO.read_forward(x["qh"], x["kbuf"], x["buf"], x["kinv"], valid, x["scale"])
    got = RO.read_backward(x["qh"], x["kbuf"], x["buf"], x["kinv"], valid, x["scale"], cache, drd)
    names = dict(qh="dq", kbuf="dkbuf", buf="dbuf", kinv="dkinv", scale="dscale")
    for key, gname in names.items():
        dirn = rng.standard_normal(x[key].shape)
        e = 1e-6
        xp, xm = dict(x), dict(x)
        xp[key] = x[key] + e * dirn
        xm[key] = x[key] - e * dirn
        fp = (RO.read_forward(xp["qh"], xp["kbuf"], xp["buf"], xp["kinv"], valid, xp["scale"])[0] * drd).sum()
        fm = (RO.read_forward(xm["qh"], xm["kbuf"], xm["buf"], xm["kinv"], valid, xm["scale"])[0] * drd).sum()
        fd = (fp - fm) / (2 * e)
        an = float((got[gname] * dirn).sum())
        assert abs(fd - an) <= 1e-7 * max(1.0, abs(fd)), (gname, fd, an)
    assert np.all(got["dq"][0, 1, 1] == 0)


def test_bf16_round_matches_torch():
    torch = pytest.importorskip("torch")
    x = np.random.default_rng(3).standard_normal(10000).astype(np.float32) * 100
    x[:4] = [0.0, -0.0, 1e-40, 3.3895314e38]
    ref = torch.tensor(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(RO.bf16_round(x), ref)


# ------------------------------------------------------------------------------------------- quantiser


def test_fq_katas():
    """gqa25/test_sh.py:96-108: <= 2^b distinct values per group, a zero row stays zero, error falls with bits."""
    rng = np.random.default_rng(3)
    xx = rng.standard_normal((2, 5, 3, 7, 64)).astype(np.float32)
    xx[0, 0, 0, 0] = 0.0
    q3, c3, s3 = RO.fq(xx, 3, 16)
    groups = q3.reshape(-1, 16)
    assert max(len(np.unique(gg)) for gg in groups[:200]) <= 8
    assert np.all(q3[0, 0, 0, 0] == 0.0)
    e3 = np.linalg.norm(q3 - xx) / np.linalg.norm(xx)
    e4 = np.linalg.norm(RO.fq(xx, 4, 16)[0] - xx) / np.linalg.norm(xx)
    assert e3 < 0.2 and e4 < e3


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_fq_is_the_midrise_level_containing_x(bits):
    """Brute force: the midrise quantiser picks the level (i+0.5)*s of the cell [i*s, (i+1)*s) holding x,
    clamped to the outermost levels; the 8-bit code fits int8 and code*s reconstructs the value."""
    rng = np.random.default_rng(bits)
    x = rng.standard_normal((50, 32)).astype(np.float32)
    val, code, s = RO.fq(x, bits, 16)
    half = 2 ** (bits - 1)
    xg = x.reshape(50, 2, 16).astype(np.float64)
    sg = s.astype(np.float64)[..., None]
    cells = np.arange(-half, half)
    lo = cells[None, None, None, :] * sg[..., None]
    inside = (xg[..., None] >= lo) & (xg[..., None] < lo + sg[..., None])
    want = np.where(inside.any(-1), cells[np.argmax(inside, -1)], np.where(xg > 0, half - 1, -half))
    np.testing.assert_array_equal(code.reshape(50, 2, 16), want)
    np.testing.assert_allclose(val.reshape(50, 2, 16), (want + 0.5) * sg, rtol=1e-6)
    assert code.min() >= -half and code.max() <= half - 1


def test_fq_matches_torch_statement():
    """The float32 arithmetic of memlm_sh.py:221-229 in torch gives the same values bit for bit."""
    torch = pytest.importorskip("torch")
    x = np.random.default_rng(9).standard_normal((4, 3, 128)).astype(np.float32) * 3
    x[1, 2] = 0.0
    xt = torch.tensor(x)
    xg = xt.reshape(4, 3, 8, 16)
    a = xg.abs().amax(-1, keepdim=True)
    s = (a / 4).clamp_min(1e-30)
    qq = (torch.floor(xg / s).clamp(-4, 3) + 0.5) * s
    qq = torch.where(a > 0, qq, torch.zeros_like(qq)).reshape(4, 3, 128)
    np.testing.assert_array_equal(RO.fq(x, 3, 16)[0], qq.numpy())


def test_fq_ste_and_quantize_mem_match_torch_statement():
    """_fq's return value x + (q - x) (memlm_sh.py:229) and _quantize_mem (:231-234) in torch float32 give the
    oracle's values bit for bit (kinv to rsqrt's last bit)."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(11)
    k = (rng.standard_normal((3, 4, 64)) * 2).astype(np.float32)
    v = rng.standard_normal((3, 4, 64)).astype(np.float32)
    k[0, 1] = 0.0
    k[1, 2, :5] = 1e-9                                       # tiny entries: q - x inexact cases
    kt, vt = torch.tensor(k), torch.tensor(v)

    def fq(x, bits, group):
        sh = x.shape
        xg = x.float().reshape(*sh[:-1], sh[-1] // group, group)
        a = xg.abs().amax(-1, keepdim=True)
        half = 2 ** (bits - 1)
        s = (a / half).clamp_min(1e-30)
        q = ((torch.floor(xg / s).clamp(-half, half - 1) + 0.5) * s)
        q = torch.where(a > 0, q, torch.zeros_like(q)).reshape(sh)
        return x + (q.to(x.dtype) - x).detach()

    for bits, group in ((3, 16), (8, 64), (2, 4)):
        np.testing.assert_array_equal(RO.fq_ste(k, bits, group), fq(kt, bits, group).numpy())
        kq = fq(kt, bits, group)
        nsq = kq.float().pow(2).sum(-1)
        okq, ovq, oki, ova = RO.quantize_mem(k, v, bits, group)
        np.testing.assert_array_equal(okq, kq.numpy())
        np.testing.assert_array_equal(ovq, fq(vt, bits, group).numpy())
        np.testing.assert_array_equal(ova, (nsq > 1e-12).numpy())
        np.testing.assert_allclose(oki, torch.rsqrt(nsq.clamp_min(1e-12)).numpy(), rtol=1e-6)
