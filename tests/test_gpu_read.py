"""GPU parity of the HIP cosine slot read (slotread_hip.slot_read through libslotscan.so) against the fp64
oracle (oracle/read_oracle.py), which reproduces the reference's two bf16 roundings (memlm_sh.py:383, 395).

Bar: |rd - oracle| <= 2e-2 * max|oracle| per case (the north star's bf16-read tolerance), mean error below
2e-3 * max|oracle|, and exactly 0 for a block with no valid row (masked_fill + nan_to_num, memlm_sh.py:394).
The inputs follow the read's own conventions: keys from an fp32 copy cast to bf16 with kinv and valid taken
from the fp32 copy (the writer epilogue, memlm_sh.py:474-475); block 0 is the empty memory of t = 0."""
import numpy as np
import pytest
import torch

import slotscan_lib as L
from oracle import read_oracle as RO

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import slotread_hip as RH

DEV = "cuda"


def make_read_inputs(B, T, H, NQ, N, D, G, seed, sharp="rsharp", empty_rows=0.25, empty_block0=True):
    gen = torch.Generator().manual_seed(seed)
    NB = (T + G - 1) // G
    K = torch.randn(B, NB, H, N, D, generator=gen)
    V = torch.randn(B, NB, H, N, D, generator=gen)
    drop = torch.rand(B, NB, H, N, generator=gen) < empty_rows          # never-written rows are exactly 0
    K[drop] = 0.0
    if empty_block0:
        K[:, 0] = 0.0
        V[:, 0] = 0.0
    nsq = K.pow(2).sum(-1)
    kinv = torch.rsqrt(nsq.clamp_min(1e-12))
    valid = nsq > 1e-12
    q = torch.randn(B, T, H, NQ, D, generator=gen)
    q = q / q.norm(dim=-1, keepdim=True).clamp_min(1e-6)
    s = torch.randn(B, T, H, NQ, generator=gen)
    if sharp == "rsharp":                       # exp(log 8) * exp(2 tanh(s / 2)), memlm_sh.py:383-393
        scale = 8.0 * torch.exp(2.0 * torch.tanh(s / 2.0))
    else:                                       # BASELINE configs 1 and 4: softplus(N(0,1)) + 1
        scale = torch.nn.functional.softplus(s) + 1.0
    bf = torch.bfloat16
    return q.to(bf), K.to(bf), V.to(bf), kinv.float(), valid, scale.float()


def to_blocks(x, G, NB):
    """(B,T,H,NQ,...) token-major -> (B,NB,H,G*NQ,...) blocks, zero-padded (memlm_sh.py:380-382)."""
    B, T, H, NQ = x.shape[:4]
    rest = x.shape[4:]
    pad = np.zeros((B, NB * G, H, NQ) + rest, x.dtype)
    pad[:, :T] = x
    y = pad.reshape((B, NB, G, H, NQ) + rest)
    y = np.moveaxis(y, 3, 2)                    # (B, NB, H, G, NQ, ...)
    return y.reshape((B, NB, H, G * NQ) + rest)


def from_blocks(y, T, NQ):
    B, NB, H, M = y.shape[:4]
    G = M // NQ
    rest = y.shape[4:]
    x = y.reshape((B, NB, H, G, NQ) + rest)
    x = np.moveaxis(x, 2, 3).reshape((B, NB * G, H, NQ) + rest)
    return x[:, :T]


def oracle_read(q, K, V, kinv, valid, scale, G):
    B, T, H, NQ, D = q.shape
    NB = K.shape[1]
    f = lambda t: t.double().numpy()
    qh = to_blocks(f(q), G, NB)
    sh = to_blocks(f(scale), G, NB)
    rd, _ = RO.read_forward(qh, f(K), f(V), f(kinv), valid.numpy(), sh, bf16=True)
    return from_blocks(rd, T, NQ)


def run_case(B, T, H, NQ, N, D, G, seed, **kw):
    kw.setdefault("empty_block0", (T + G - 1) // G > 1)      # a one-block store is a written store
    q, K, V, kinv, valid, scale = make_read_inputs(B, T, H, NQ, N, D, G, seed, **kw)
    print(f"read case B{B} T{T} H{H} NQ{NQ} N{N} D{D} G{G} seed {seed}", flush=True)
    c = lambda t: t.to(DEV)
    rd = RH.slot_read(c(q), c(K), c(V), c(kinv), c(valid), c(scale), G)
    torch.cuda.synchronize()
    ref = oracle_read(q, K, V, kinv, valid, scale, G)
    got = rd.double().cpu().numpy()
    den = max(np.abs(ref).max(), 1e-30)
    err = np.abs(got - ref)
    print(f"   max rel err {err.max() / den:.2e}  mean {err.mean() / den:.2e}", flush=True)
    assert err.max() <= 2e-2 * den
    assert err.mean() <= 2e-3 * den
    return q, K, V, kinv, valid, scale, rd


READ_CASES = [  # B, T, H, NQ, N, D, G
    (2, 64, 3, 2, 192, 128, 8),      # training shape per block (sh25: G=8, NQ=2, M=16)
    (2, 61, 2, 2, 192, 128, 8),      # ragged last block
    (1, 50, 2, 1, 40, 64, 16),       # partial slot tiles, D=64
    (2, 100, 2, 2, 96, 128, 16),     # N=96 (encoder memory), M=32: two query tiles per block
    (2, 256, 2, 1, 192, 128, 256),   # frozen store (config 4 shape per head): one block, 16 query tiles
    (1, 1024, 1, 1, 192, 128, 1024), # one slab split over many workgroups
    (1, 37, 3, 3, 17, 64, 5),        # odd everything
    (2, 300, 2, 1, 40, 64, 300),     # wide-block kernel: partial slot chunk, ragged last query tile
    (1, 200, 3, 2, 96, 128, 256),    # wide-block kernel with NQ=2 and a partial block (T < G)
]


@pytest.mark.parametrize("case", READ_CASES, ids=lambda c: "B{}T{}H{}NQ{}N{}D{}G{}".format(*c))
def test_read_matches_oracle(case):
    run_case(*case, seed=3)


WIDE_FULL_CASES = [  # B, T, H, N, D, G (NQ = 1), slabs checked against the oracle
    # config 4's shape: 384 slabs x 4 chunks of 256 queries over 256 workgroups, 6 chunks each, so every
    # other workgroup starts mid-slab and every one restages the store once; slabs 1, 2, 192, 193 and 383 are
    # split between two workgroups or end a range
    ((64, 1024, 6, 192, 128, 1024), (0, 1, 2, 3, 191, 192, 193, 382, 383)),
    # ragged: 96 slabs x 4 chunks (the last of 232 queries) over 256 workgroups of 1 or 2 chunks each
    ((16, 1000, 6, 192, 128, 1000), (0, 1, 2, 47, 48, 94, 95)),
]


@pytest.mark.parametrize("case", WIDE_FULL_CASES, ids=lambda c: "B{}T{}H{}N{}D{}G{}".format(*c[0]))
def test_wide_read_full_size_sampled_slabs(case):
    """The wide kernel at sizes where a workgroup walks several chunks and crosses slab boundaries (the
    parity cases above give every workgroup one chunk at most): the whole launch at full size, then the
    sampled slabs against the fp64 oracle, at the same bar as run_case."""
    (B, T, H, N, D, G), slabs = case
    q, K, V, kinv, valid, scale = make_read_inputs(B, T, H, 1, N, D, G, seed=3, sharp="softplus",
                                                   empty_block0=False)
    print(f"wide full-size read B{B} T{T} H{H} N{N} D{D} G{G}", flush=True)
    c = lambda t: t.to(DEV)
    rd = RH.slot_read(c(q), c(K), c(V), c(kinv), c(valid), c(scale), G).cpu()
    torch.cuda.synchronize()
    for s in slabs:
        b, h = divmod(s, H)
        sl = lambda t: t[b:b + 1, :, h:h + 1].contiguous()
        ref = oracle_read(sl(q), sl(K), sl(V), sl(kinv), sl(valid), sl(scale), G)
        got = sl(rd).double().numpy()
        den = max(np.abs(ref).max(), 1e-30)
        err = np.abs(got - ref)
        assert err.max() <= 2e-2 * den, (s, err.max() / den)
        assert err.mean() <= 2e-3 * den, (s, err.mean() / den)


def test_read_softplus_sharpness_all_rows_valid():
    run_case(2, 128, 2, 1, 192, 128, 128, seed=4, sharp="softplus", empty_rows=0.0, empty_block0=False)


def test_empty_block_reads_exact_zero_and_is_deterministic():
    q, K, V, kinv, valid, scale, rd = run_case(2, 40, 2, 2, 64, 128, 8, seed=5)
    G = 8
    assert torch.all(rd[:, :G] == 0)                  # block 0 has no valid row
    c = lambda t: t.to(DEV)
    rd2 = RH.slot_read(c(q), c(K), c(V), c(kinv), c(valid), c(scale), G)
    assert torch.equal(rd, rd2)


def oracle_read_grads(q, K, V, kinv, valid, scale, G, drd):
    B, T, H, NQ, D = q.shape
    NB = K.shape[1]
    f = lambda t: t.double().numpy()
    qh = to_blocks(f(q), G, NB)
    sh = to_blocks(f(scale), G, NB)
    dh = to_blocks(f(drd), G, NB)
    _, cache = RO.read_forward(qh, f(K), f(V), f(kinv), valid.numpy(), sh, bf16=True)
    gr = RO.read_backward(qh, f(K), f(V), f(kinv), valid.numpy(), sh, cache, dh)
    return dict(dq=from_blocks(gr["dq"], T, NQ), dkbuf=gr["dkbuf"], dbuf=gr["dbuf"], dkinv=gr["dkinv"],
                dscale=from_blocks(gr["dscale"], T, NQ))


def run_grad_case(B, T, H, NQ, N, D, G, seed, **kw):
    kw.setdefault("empty_block0", (T + G - 1) // G > 1)
    q, K, V, kinv, valid, scale = make_read_inputs(B, T, H, NQ, N, D, G, seed, **kw)
    drd = torch.randn(B, T, H, NQ, D, generator=torch.Generator().manual_seed(seed + 100)).to(torch.bfloat16)
    print(f"read grad case B{B} T{T} H{H} NQ{NQ} N{N} D{D} G{G} seed {seed}", flush=True)
    c = lambda t: t.to(DEV)
    qq, kk, vv, ki, sc = (c(x).requires_grad_() for x in (q, K, V, kinv, scale))
    rd = RH.slot_read(qq, kk, vv, ki, c(valid), sc, G)
    rd.backward(c(drd))
    torch.cuda.synchronize()
    ref = oracle_read_grads(q, K, V, kinv, valid, scale, G, drd)
    got = dict(dq=qq.grad, dkbuf=kk.grad, dbuf=vv.grad, dkinv=ki.grad, dscale=sc.grad)
    for name in ref:
        g_ = got[name].double().cpu().numpy()
        r_ = ref[name]
        den = max(np.abs(r_).max(), 1e-30)
        err = np.abs(g_ - r_)
        print(f"   {name}: max rel err {err.max() / den:.2e}  mean {err.mean() / den:.2e}", flush=True)
        assert err.max() <= 2e-2 * den, name
        assert err.mean() <= 3e-3 * den, name
    return got


GRAD_CASES = [  # B, T, H, NQ, N, D, G
    (2, 64, 3, 2, 192, 128, 8),      # training shape: one 16-query tile per block
    (2, 61, 2, 2, 192, 128, 8),      # ragged last block
    (1, 50, 2, 1, 40, 64, 16),       # partial slot tiles, D=64, one tile
    (2, 100, 2, 2, 96, 128, 16),     # two query tiles per block: accumulated dK, dV
    (1, 37, 3, 3, 17, 64, 5),        # odd everything
]


@pytest.mark.parametrize("case", GRAD_CASES, ids=lambda c: "B{}T{}H{}NQ{}N{}D{}G{}".format(*c))
def test_read_gradients_match_oracle(case):
    run_grad_case(*case, seed=7)


def test_read_backward_is_deterministic():
    a = run_grad_case(2, 64, 2, 2, 192, 128, 8, seed=8)
    b = run_grad_case(2, 64, 2, 2, 192, 128, 8, seed=8)
    for name in a:
        assert torch.equal(a[name], b[name]), name


def test_shared_read_matches_the_readers_formula():
    """slotread_hip.shared_read, the replacement of SharedMixer._read from the projected queries on
    (memlm_sh.py:379-397), against the oracle read with the reader's own preparation: q / max(|q|, 1e-6) in
    q's dtype (:379), the multiplier exp(log_rsel) * exp(C tanh(s / C)) with C = 2 (:383-393, run_sh25.sh:223),
    NQ = 2 and T not a multiple of G (the padded tail, :380-382).  Gradients of q (through the
    normalisation), the copies, kinv, log_rsel and s are checked at the bf16 read bar."""
    B, T, H, NQ, N, D, G, C = 2, 61, 3, 2, 192, 128, 8, 2.0
    _, K, V, kinv, valid, _ = make_read_inputs(B, T, H, NQ, N, D, G, seed=19)
    gen = torch.Generator().manual_seed(20)
    q = (3.0 * torch.randn(B, T, H, NQ, D, generator=gen)).to(torch.bfloat16)   # projected, not unit
    s = torch.randn(B, T, H, NQ, generator=gen)
    drd = torch.randn(B, T, H, NQ, D, generator=gen).to(torch.bfloat16)
    lr = float(np.log(8.0))
    c = lambda t: t.to(DEV).requires_grad_()
    qq, kk, vv, ki, ss = c(q), c(K), c(V), c(kinv), c(s)
    lrs = torch.tensor(lr, device=DEV, requires_grad=True)
    rd = RH.shared_read(qq, kk, vv, ki, valid.to(DEV), lrs, G, s=ss, rsharp=C)
    rd.backward(drd.to(DEV))
    torch.cuda.synchronize()
    # the oracle: the reader's preparation in float64 (the normalised query rounded to bf16 as q's dtype)
    qf = q.double().numpy()
    nrm = np.maximum(np.sqrt((qf * qf).sum(-1, keepdims=True)), 1e-6)
    qhat = RO.bf16_round(qf / RO.bf16_round(nrm)).astype(np.float64)
    th = np.tanh(s.double().numpy() / C)
    scale = np.exp(lr) * np.exp(C * th)
    NB = (T + G - 1) // G
    f = lambda t: t.double().numpy()
    qh, sh, dh = to_blocks(qhat, G, NB), to_blocks(scale, G, NB), to_blocks(f(drd), G, NB)
    ref, cache = RO.read_forward(qh, f(K), f(V), f(kinv), valid.numpy(), sh, bf16=True)
    ref = from_blocks(ref, T, NQ)
    gr = RO.read_backward(qh, f(K), f(V), f(kinv), valid.numpy(), sh, cache, dh)
    dqh = from_blocks(gr["dq"], T, NQ)
    dscale = from_blocks(gr["dscale"], T, NQ)
    qn = qf / nrm
    want = dict(rd=ref, dq=(dqh - qn * (dqh * qn).sum(-1, keepdims=True)) / nrm, dkbuf=gr["dkbuf"],
                dbuf=gr["dbuf"], dkinv=gr["dkinv"], dlog_rsel=np.array((dscale * scale).sum()),
                ds=dscale * scale * (1.0 - th * th))
    got = dict(rd=rd, dq=qq.grad, dkbuf=kk.grad, dbuf=vv.grad, dkinv=ki.grad, dlog_rsel=lrs.grad, ds=ss.grad)
    l1 = dict(dlog_rsel=np.abs(dscale * scale).sum())      # a sum of mixed-sign terms: bar on their magnitude
    for name, r_ in want.items():
        g_ = got[name].detach().double().cpu().numpy().reshape(np.shape(r_))
        den = max(np.abs(r_).max(), l1.get(name, 0.0), 1e-30)
        err = np.abs(g_ - r_)
        print(f"   {name}: max rel err {err.max() / den:.2e}  mean {err.mean() / den:.2e}", flush=True)
        assert err.max() <= 2e-2 * den, name
        assert err.mean() <= 3e-3 * den, name


@pytest.mark.parametrize("with_delta", [True, False])
def test_read_out_matches_oracle(with_delta):
    """slotread_hip.shared_read_out, the reader's read followed by its output projection into the residual,
    delta + wo_tk(rd) (memlm_sh.py:499-501), against the oracle read (bf16 roundings, rd rounded to bf16 as
    the read's output) followed by an fp64 projection; backward through dRD = dDelta Wo, dWo = dDelta^T rd and
    the read's own adjoint.  Bar: the bf16 read bar, 2e-2 of each tensor's max."""
    B, T, H, NQ, N, D, G, C, DM = 2, 61, 3, 2, 192, 128, 8, 2.0, 256
    _, K, V, kinv, valid, _ = make_read_inputs(B, T, H, NQ, N, D, G, seed=23)
    gen = torch.Generator().manual_seed(24)
    q = (3.0 * torch.randn(B, T, H, NQ, D, generator=gen)).to(torch.bfloat16)
    s = torch.randn(B, T, H, NQ, generator=gen)
    wo = (torch.randn(DM, H * NQ * D, generator=gen) / (H * NQ * D) ** 0.5).to(torch.bfloat16)
    delta = torch.randn(B, T, DM, generator=gen).to(torch.bfloat16) if with_delta else None
    dout = torch.randn(B, T, DM, generator=gen).to(torch.bfloat16)
    lr = float(np.log(8.0))
    c = lambda t: t.to(DEV).requires_grad_()
    qq, kk, vv, ki, ss, ww = c(q), c(K), c(V), c(kinv), c(s), c(wo)
    dd = c(delta) if with_delta else None
    lrs = torch.tensor(lr, device=DEV, requires_grad=True)
    out = RH.shared_read_out(qq, kk, vv, ki, valid.to(DEV), lrs, G, ww, s=ss, rsharp=C, delta=dd)
    assert out.shape == (B, T, DM) and out.dtype == torch.bfloat16
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    # oracle
    qf = q.double().numpy()
    nrm = np.maximum(np.sqrt((qf * qf).sum(-1, keepdims=True)), 1e-6)
    qhat = RO.bf16_round(qf / RO.bf16_round(nrm)).astype(np.float64)
    th = np.tanh(s.double().numpy() / C)
    scale = np.exp(lr) * np.exp(C * th)
    NB = (T + G - 1) // G
    f = lambda t: t.double().numpy()
    qh, sh = to_blocks(qhat, G, NB), to_blocks(scale, G, NB)
    rdh, cache = RO.read_forward(qh, f(K), f(V), f(kinv), valid.numpy(), sh, bf16=True)
    rd = RO.bf16_round(from_blocks(rdh, T, NQ)).astype(np.float64).reshape(B, T, -1)
    W = f(wo)
    ref = rd @ W.T + (f(delta) if with_delta else 0.0)
    g = f(dout)
    drd = (g @ W).reshape(B, T, H, NQ, D)
    gr = RO.read_backward(qh, f(K), f(V), f(kinv), valid.numpy(), sh, cache, to_blocks(drd, G, NB))
    dqh = from_blocks(gr["dq"], T, NQ)
    dscale = from_blocks(gr["dscale"], T, NQ)
    qn = qf / nrm
    want = dict(out=ref, dwo=g.reshape(-1, DM).T @ rd.reshape(-1, H * NQ * D),
                dq=(dqh - qn * (dqh * qn).sum(-1, keepdims=True)) / nrm, dkbuf=gr["dkbuf"], dbuf=gr["dbuf"],
                dkinv=gr["dkinv"], dlog_rsel=np.array((dscale * scale).sum()), ds=dscale * scale * (1.0 - th * th))
    got = dict(out=out, dwo=ww.grad, dq=qq.grad, dkbuf=kk.grad, dbuf=vv.grad, dkinv=ki.grad, dlog_rsel=lrs.grad,
               ds=ss.grad)
    if with_delta:
        want["ddelta"], got["ddelta"] = g, dd.grad
    l1 = dict(dlog_rsel=np.abs(dscale * scale).sum())      # a sum of mixed-sign terms: bar on their magnitude
    for name, r_ in want.items():
        g_ = got[name].detach().double().cpu().numpy().reshape(np.shape(r_))
        den = max(np.abs(r_).max(), l1.get(name, 0.0), 1e-30)
        err = np.abs(g_ - r_)
        print(f"   {name}: max rel err {err.max() / den:.2e}  mean {err.mean() / den:.2e}", flush=True)
        assert err.max() <= 2e-2 * den, name
        assert err.mean() <= 3e-3 * den, name


def _bf16_ulp(x):
    """Spacing of bf16 numbers at |x| (8 significand bits), for x of any magnitude (min normal spacing below)."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    return 2.0 ** (e - 7)


@pytest.mark.parametrize("M,N,K,with_delta", [(1, 256, 32, True), (300, 512, 768, True), (513, 2048, 64, False),
                                              (256, 256, 800, False), (70, 512, 96, True), (200, 256, 128, True),
                                              (257, 256, 800, True), (100, 256, 32, False)])
def test_proj_gemm_matches_fp64(M, N, K, with_delta):
    """slotproj_fwd, the reader's wo_tk projection with the residual add in the GEMM epilogue, against an fp64
    GEMM of the same bf16 operands.  The kernel rounds as the reference does: the product (fp32 accumulation)
    is rounded to bf16 -- the bf16 Linear output, memlm_sh.py:500 -- then added to delta in fp32 and rounded
    again -- the bf16 residual add, :501.  So |out - exact| <= 1/2 bf16 ulp of the result, plus 1/2 bf16 ulp
    of the product when there is a delta, plus the fp32 accumulation error (2^-20 * sum |rd||wo|).  Ragged M
    (1, 300, 513) covers partial row tiles; rows past M of a larger buffer are checked untouched; K = 800 is
    25 k stages (an odd count; the loop runs stages in pairs); K = 32, 64, 96 and 128 are 1-4 stages, the
    short-loop paths of the ring's prologue and counted waits (delta is read in the epilogue only)."""
    gen = torch.Generator().manual_seed(M * 7 + K)
    a = torch.randn(M, K, generator=gen).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=gen) / K ** 0.5).to(torch.bfloat16)
    d = torch.randn(M, N, generator=gen).to(torch.bfloat16) if with_delta else None
    print(f"   proj M={M} N={N} K={K} delta={with_delta}", flush=True)
    out = torch.full((M + 3, N), 7.0, dtype=torch.bfloat16, device=DEV)   # 3 guard rows past M
    ad, wd = a.to(DEV), w.to(DEV)
    dd = d.to(DEV) if with_delta else None
    rc = L.lib().slotproj_fwd(L.ptr(ad), L.ptr(wd), None if dd is None else L.ptr(dd), M, N, K, L.ptr(out),
                              L.stream_of(ad.device))
    L.check(rc, "slotproj_fwd")
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    assert (got[M:] == 7.0).all(), "rows past M were written"
    A, W = a.double().numpy(), w.double().numpy()
    prod = A @ W.T
    ref = prod + (d.double().numpy() if with_delta else 0.0)
    bound = 0.5 * _bf16_ulp(ref) + 2.0 ** -20 * (np.abs(A) @ np.abs(W).T) + \
        (0.5 * _bf16_ulp(prod) if with_delta else 0.0)
    err = np.abs(got[:M] - ref)
    print(f"   max err / bound {np.max(err / bound):.3f}", flush=True)
    assert (err <= bound).all()


def test_read_out_projection_runs_the_library_gemm():
    """The read-out op's projection is the library's proj_gemm kernel (not a library GEMM) at the shapes it
    tiles: the library's per-kernel launch count of "proj" advances by one per forward."""
    B, T, H, NQ, N, D, G, DM = 1, 40, 2, 2, 64, 64, 4, 256
    _, K, V, kinv, valid, _ = make_read_inputs(B, T, H, NQ, N, D, G, seed=5)
    gen = torch.Generator().manual_seed(6)
    q = torch.randn(B, T, H, NQ, D, generator=gen)
    q = (q / q.norm(dim=-1, keepdim=True)).to(torch.bfloat16).to(DEV)
    scale = torch.full((B, T, H, NQ), 4.0, device=DEV)
    wo = torch.randn(DM, H * NQ * D, generator=gen).to(torch.bfloat16).to(DEV)
    args = (q, K.to(DEV), V.to(DEV), kinv.to(DEV), valid.to(DEV), scale, G, wo)
    L.profile_read()                                     # drop earlier counts
    L.profile(True)
    try:
        RH.slot_read_out(*args)
        RH.slot_read_out(*args)
        torch.cuda.synchronize()
    finally:
        L.profile(False)
    prof = L.profile_read()
    assert prof.get("proj", (0.0, 0))[1] == 2 and prof.get("read_fwd", (0.0, 0))[1] == 2


def test_proj_gemm_in_place_residual_add():
    """slotproj.h allows delta to alias out (the residual updated in place): with a ragged M the result equals the
    out-of-place call bitwise, and the rows past M are untouched."""
    M, N, K = 300, 512, 256
    gen = torch.Generator().manual_seed(5)
    a = torch.randn(M, K, generator=gen).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K, generator=gen) / K ** 0.5).to(torch.bfloat16).to(DEV)
    buf = torch.full((M + 3, N), 7.0, dtype=torch.bfloat16, device=DEV)
    buf[:M] = torch.randn(M, N, generator=gen).to(torch.bfloat16).to(DEV)
    ref = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    L.check(L.lib().slotproj_fwd(L.ptr(a), L.ptr(w), L.ptr(buf), M, N, K, L.ptr(ref), L.stream_of(a.device)), "fwd")
    L.check(L.lib().slotproj_fwd(L.ptr(a), L.ptr(w), L.ptr(buf), M, N, K, L.ptr(buf), L.stream_of(a.device)), "fwd")
    torch.cuda.synchronize()
    assert torch.equal(buf[:M], ref)
    assert (buf[M:].float() == 7.0).all()


@pytest.mark.parametrize("M,N,K", [(1, 256, 256), (122, 256, 768), (300, 512, 768), (1000, 256, 512),
                                   (8192, 2048, 768)])
def test_proj_bwd_matches_fp64(M, N, K):
    """slotproj_bwd, the backward of the read-out projection (drd = dout wo, dwo = dout^T rd), against fp64
    products of the same bf16 operands.  Each output is one fp32 accumulation rounded to bf16 (the reference's
    bf16 matmuls), so |got - exact| <= 1/2 bf16 ulp of the result + 2^-20 * sum |a||b| (fp32 accumulation; for
    dwo also the fp32 sum of the token splits).  M = 1, 122, 300, 1000 leave a partial 32-token stage (and
    splits with no full stage); 8192 x 2048 x 768 is config4_wo's weight shape (about 22 splits of 12 stages).
    Run twice: bitwise the same (fixed-order split sum, no atomics)."""
    gen = torch.Generator().manual_seed(M + N + K)
    g = torch.randn(M, N, generator=gen).to(torch.bfloat16)
    x = torch.randn(M, K, generator=gen).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=gen) / K ** 0.5).to(torch.bfloat16)
    print(f"   proj bwd M={M} N={N} K={K}", flush=True)
    gd, xd, wd = g.to(DEV), x.to(DEV), w.to(DEV)
    outs = [RH._proj_bwd(gd, xd, wd) for _ in range(2)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    G_, X, W = g.double().numpy(), x.double().numpy(), w.double().numpy()
    for name, got, ref, mag in (("drd", outs[0][0], G_ @ W, np.abs(G_) @ np.abs(W)),
                                ("dwo", outs[0][1], G_.T @ X, np.abs(G_).T @ np.abs(X))):
        bound = 0.5 * _bf16_ulp(ref) + 2.0 ** -20 * mag
        err = np.abs(got.double().cpu().numpy() - ref)
        print(f"   {name}: max err / bound {np.max(err / bound):.3f}", flush=True)
        assert (err <= bound).all(), name


def test_proj_bwd_refuses_untiled_shapes():
    """The backward tiles d_model and H*NQ*dv in multiples of 256; other shapes raise (no second GEMM backend)."""
    g = torch.zeros(4, 256, dtype=torch.bfloat16, device=DEV)
    x = torch.zeros(4, 96, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(NotImplementedError):
        RH._proj_bwd(g, x, torch.zeros(256, 96, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(NotImplementedError):
        RH._proj(x, torch.zeros(200, 96, dtype=torch.bfloat16, device=DEV), None)
