"""CPU oracle for the cosine slot read and the storage quantiser -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.

read_forward / read_backward restate the kernel-level core of SharedMixer._read
(/root/reference/gqa25/memlm_sh.py:362-397): per (b, block j, head h), with M = G*NQ queries that share the
block's pre-write copy (memlm_sh.py:380-382),
    raw[m, n] = <qhat_m, kbuf_n>                      (bf16 einsum, memlm_sh.py:383)
    sc[m, n]  = raw[m, n] * kinv_n * scale_m          (kinv and exp(log_rsel) at :383, exp(C tanh(s/C)) at :384-393)
    att       = nan_to_num(softmax(sc masked to -inf where ~valid_n))   (memlm_sh.py:394)
    rd[m, :]  = sum_n att[m, n] buf_n                 (bf16 einsum, memlm_sh.py:395)
`scale` is the combined per-query multiplier exp(log_rsel) * exp(C tanh(s/C)).  With bf16=True the two
roundings the reference's bf16 einsums make are reproduced: raw is rounded to bf16 before scaling and att
is rounded to bf16 before the value contraction.

naive_block_read is the reference's own per-token check of the strided read (gqa25/test_sh.py:77-86,
kvu/test_rs.py:102-112): every token t reads the copy taken at the start of its block, t // G.

fq restates the midrise storage quantiser _fq (memlm_sh.py:221-228) in float32 arithmetic, fq_ste its
straight-through return value (memlm_sh.py:229), and quantize_mem restates _quantize_mem
(memlm_sh.py:231-234).

Pinning (tests/test_oracle_read.py): read_forward against naive_block_read (a per-token loop with its
own indexing), against the textbook identity for one valid row (att = 1 there), all-invalid blocks read
exactly 0; read_backward against central finite differences in float64; fq against the quantiser KATs
of gqa25/test_sh.py:96-108 and a brute-force nearest-level search.
"""
import numpy as np


def bf16_round(x):
    """Round float32 values to the nearest bfloat16 (ties to even) and return them as float32."""
    x = np.ascontiguousarray(np.asarray(x, np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def read_forward(qh, kbuf, buf, kinv, valid, scale, bf16=False, dtype=np.float64):
    """qh (B,NB,H,M,DK), kbuf (B,NB,H,N,DK), buf (B,NB,H,N,DV), kinv/valid (B,NB,H,N), scale (B,NB,H,M).
    Returns (rd (B,NB,H,M,DV), cache)."""
    qh, kbuf, buf = (np.asarray(x, dtype) for x in (qh, kbuf, buf))
    kinv, scale = np.asarray(kinv, dtype), np.asarray(scale, dtype)
    valid = np.asarray(valid, bool)
    raw = np.einsum("bjhmd,bjhnd->bjhmn", qh, kbuf)
    if bf16:
        raw = bf16_round(raw).astype(dtype)
    sc = raw * kinv[..., None, :] * scale[..., :, None]
    vm = valid[..., None, :]
    zm = np.where(vm, sc, -np.inf)
    mx = zm.max(-1, keepdims=True)
    anyv = np.isfinite(mx)
    e = np.where(vm, np.exp(zm - np.where(anyv, mx, 0.0)), 0.0)
    den = e.sum(-1, keepdims=True)
    att = np.where(anyv, e / np.where(den > 0, den, 1.0), 0.0)      # nan_to_num: an all-masked row reads 0
    attc = bf16_round(att).astype(dtype) if bf16 else att
    rd = np.einsum("bjhmn,bjhnv->bjhmv", attc, buf)
    return rd, dict(raw=raw, sc=sc, att=att, attc=attc)


def read_backward(qh, kbuf, buf, kinv, valid, scale, cache, drd, dtype=np.float64):
    """Gradients of read_forward w.r.t. qh, kbuf, buf, kinv and scale (roundings treated as identity)."""
    qh, kbuf, buf = (np.asarray(x, dtype) for x in (qh, kbuf, buf))
    kinv, scale = np.asarray(kinv, dtype), np.asarray(scale, dtype)
    drd = np.asarray(drd, dtype)
    raw, att, attc = cache["raw"], cache["att"], cache["attc"]
    dbuf = np.einsum("bjhmn,bjhmv->bjhnv", attc, drd)
    datt = np.einsum("bjhmv,bjhnv->bjhmn", drd, buf)
    dsc = att * (datt - (att * datt).sum(-1, keepdims=True))
    dkinv = (dsc * raw * scale[..., :, None]).sum(-2)
    dscale = (dsc * raw * kinv[..., None, :]).sum(-1)
    draw = dsc * kinv[..., None, :] * scale[..., :, None]
    dqh = np.einsum("bjhmn,bjhnd->bjhmd", draw, kbuf)
    dkbuf = np.einsum("bjhmn,bjhmd->bjhnd", draw, qh)
    return dict(dq=dqh, dkbuf=dkbuf, dbuf=dbuf, dkinv=dkinv, dscale=dscale)


def naive_block_read(q_tok, Kstates, Vstates, scale_tok, G, dtype=np.float64):
    """Per-token loop: q_tok (B,T,H,NQ,DK) unit queries, Kstates/Vstates (B,T,H,N,D) the PRE-write state at
    every position, scale_tok (B,T,H,NQ).  Token t reads the state at t0 = (t // G) * G; rows with
    |K| <= 1e-6 are invalid; an all-invalid state reads exactly 0."""
    B, T, H, NQ, DK = q_tok.shape
    DV = Vstates.shape[-1]
    out = np.zeros((B, T, H, NQ, DV), dtype)
    for b in range(B):
        for t in range(T):
            t0 = (t // G) * G
            for h in range(H):
                Kt = np.asarray(Kstates[b, t0, h], dtype)
                Vt = np.asarray(Vstates[b, t0, h], dtype)
                nrm = np.sqrt((Kt * Kt).sum(-1))
                ok = nrm > 1e-6
                for r in range(NQ):
                    if not ok.any():
                        continue
                    sc = (Kt @ np.asarray(q_tok[b, t, h, r], dtype)) / np.maximum(nrm, 1e-6) * scale_tok[b, t, h, r]
                    sc = np.where(ok, sc, -np.inf)
                    e = np.exp(sc - sc.max())
                    out[b, t, h, r] = (e / e.sum()) @ Vt
    return out


def fq(x, bits, group):
    """Forward value of the midrise storage quantiser (memlm_sh.py:221-229), float32 arithmetic.
    Returns (value, code, scale): code int8 in [-2^(b-1), 2^(b-1)-1], scale (..., D/group) float32."""
    x = np.asarray(x, np.float32)
    sh = x.shape
    xg = x.reshape(*sh[:-1], sh[-1] // group, group)
    a = np.abs(xg).max(-1, keepdims=True)
    half = np.float32(2 ** (bits - 1))
    s = np.maximum(a / half, np.float32(1e-30)).astype(np.float32)
    code = np.clip(np.floor(xg / s), -half, half - 1).astype(np.float32)
    val = ((code + np.float32(0.5)) * s).astype(np.float32)
    val = np.where(a > 0, val, np.float32(0.0))
    return val.reshape(sh), code.astype(np.int8).reshape(sh), s[..., 0]


def fq_ste(x, bits, group):
    """What _fq RETURNS for a float32 x (memlm_sh.py:229): x + (q - x), each operation rounded to float32 --
    the straight-through expression's forward value, which equals q except where q - x is inexact."""
    x = np.asarray(x, np.float32)
    q, _, _ = fq(x, bits, group)
    return (x + (q - x).astype(np.float32)).astype(np.float32)


def quantize_mem(kbuf, buf, bits, group):
    """_quantize_mem (memlm_sh.py:231-234): (kq, vq, kinv, valid) from the float32 copies."""
    kq = fq_ste(kbuf, bits, group)
    vq = fq_ste(buf, bits, group)
    nsq = (kq.astype(np.float32) ** 2).sum(-1, dtype=np.float32)
    kinv = (1.0 / np.sqrt(np.maximum(nsq, np.float32(1e-12)))).astype(np.float32)
    return kq, vq, kinv, nsq > 1e-12


def writer_epilogue(kbuf):
    """Full-precision writer epilogue (memlm_sh.py:474-475): kinv = rsqrt(max(|K|^2, 1e-12)), valid = |K|^2 > 1e-12."""
    kbuf = np.asarray(kbuf, np.float64)
    nsq = (kbuf * kbuf).sum(-1)
    return 1.0 / np.sqrt(np.maximum(nsq, 1e-12)), nsq > 1e-12
