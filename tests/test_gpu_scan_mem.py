"""GPU parity of the fused scan + writer epilogue (slotkern_hip.kv_scan_mem, libslotscan.so's
slotscan_fwd_mem / slotscan_bwd_mem) -- the writer layer's kv_scan_g followed by its full-precision
epilogue (memlm_sh.py:453-456, 473-475).

Two references on the same seeded inputs:
  - the unfused GPU path, writer_epilogue(kv_scan_c(...)): the bf16 copies and validity must be bitwise equal
    (the same fp32 snapshot rounded to nearest-even once), kinv within 2e-6 relative (the row sum's order
    differs), every gradient within 5e-5 relative to its max (fp32 tokens);
  - the fp64 oracle, teacher-forced on the GPU's addresses, with the epilogue's autograd folded into the
    upstream snapshot gradients: dkbuf = dkb + 2 K dnsq, dnsq = -0.5 kinv^3 dkinv where |K|^2 >= 1e-12, dvbuf
    = dvb.  Gradients within 1e-4 relative to max for fp32 tokens and 1e-2 for bf16 tokens (the bar of the
    unfused scan's tests)."""
import numpy as np
import pytest
import torch

from oracle import read_oracle as RO
from oracle import scan_oracle as SO
from scan_inputs import assert_no_flips, np64, scan_inputs, upstream

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import slotkern_hip as KH
    import slotmem_hip as MH

DEV = "cuda"
TEMP = 16.0


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def _leaves(k, q, v, g, fr):
    d = lambda x: None if x is None else x.to(DEV).requires_grad_()
    return d(k), d(q), d(v), d(g), d(fr), torch.tensor(TEMP, device=DEV, requires_grad=True)


def _run(fused, k, q, v, g, fr, N, G, occb, hardg, wk, wv, wi):
    """Forward + backward of loss = sum(kb * wk) + sum(vb * wv) + sum(kinv * wi) (a None weight drops the
    term).  Returns ((kb, vb, kinv, valid), grads)."""
    kk, qq, vv, gg, ff, tp = _leaves(k, q, v, g, fr)
    kw = dict(G=G, hard=True, hard_gate=hardg, detach_addr=True, q=qq, occ_bin=occb)
    if fused:
        kb, vb, kinv, valid = KH.kv_scan_mem(kk, vv, gg, ff, N, tp, **kw)
    else:
        kbuf, vbuf = KH.kv_scan_c(kk, vv, gg, ff, N, tp, **kw)
        kb, vb, kinv, valid = MH.writer_epilogue(kbuf, vbuf, dtype=torch.bfloat16)
    loss = (kb.float() * wk.to(DEV)).sum()
    if wv is not None:
        loss = loss + (vb.float() * wv.to(DEV)).sum()
    if wi is not None:
        loss = loss + (kinv * wi.to(DEV)).sum()
    loss.backward()
    torch.cuda.synchronize()
    grads = dict(dk=kk.grad, dv=vv.grad, dgate=gg.grad, dfr=ff.grad, dtemp=tp.grad,
                 dq=None if qq is None else qq.grad)
    return (kb.detach(), vb.detach(), kinv.detach(), valid), grads


def _am(k, q, v, g, fr, N, G, occb, hardg):
    qq = k if q is None else q
    dt, k_, q_, v_, g_, fr_, frt, temp_ = KH._prep(k.to(DEV), qq.to(DEV), v.to(DEV), g.to(DEV), fr.to(DEV),
                                                   torch.tensor(TEMP, device=DEV), hardg)
    out = KH._fwd(k_, q_, v_, g_, fr_, frt, temp_, N, G, 1e-4, occb, dt, logs=False)
    torch.cuda.synchronize()
    return out[2].cpu().numpy().astype(np.int64)


def _oracle_grads(k, q, v, g, fr, N, G, occb, hardg, am, wk, wv, wi):
    """Oracle gradients of the same loss: the epilogue's autograd gives the snapshot upstream, then the
    oracle's scan backward."""
    kn, qn, vn, gn, frn = np64(k), np64(q), np64(v), np64(g), np64(fr)
    kb, vb, info = SO.scan_forward(kn, vn, gn, frn, N, TEMP, G=G, hard=True, hard_gate=hardg, eps=1e-4,
                                   detach_addr=True, q=qn, occ_bin=occb, teacher=am)
    kinv, _ = RO.writer_epilogue(kb)
    nsq = (kb * kb).sum(-1)
    dkb = np64(wk.to(torch.bfloat16))                     # the gradient reaching a bf16 output is bf16
    dvb = np.zeros_like(vb) if wv is None else np64(wv.to(torch.bfloat16))
    dnsq = np.zeros_like(nsq) if wi is None else np.where(nsq >= 1e-12, -0.5 * kinv ** 3 * np64(wi), 0.0)
    gr = SO.scan_backward(kn, vn, gn, frn, N, TEMP, kb, vb, info, dkb + 2.0 * kb * dnsq[..., None], dvb, G=G,
                          hard=True, hard_gate=hardg, eps=1e-4, detach_addr=True, q=qn, occ_bin=occb)
    return kb, info, gr


def _check(B, T, H, N, D, G, frt, occb, sep_q, hardg, seed, dtype=torch.float32, terms=("k", "v", "i")):
    print(f"mem case B{B} T{T} H{H} N{N} D{D} G{G} frt={frt} occb={occb} q={sep_q} hardg={hardg} {dtype} "
          f"terms={terms}", flush=True)
    k, q, v, g, fr = scan_inputs(B, T, H, D, seed, sep_q=sep_q, frt=frt, dtype=dtype)
    NB = (T + G - 1) // G
    wk, wv = upstream((B, NB, H, N, D), seed + 1000)
    wi = torch.randn(B, NB, H, N, generator=torch.Generator().manual_seed(seed + 2000))
    wv = wv if "v" in terms else None
    wi = wi if "i" in terms else None
    (kb, vb, kinv, valid), gf = _run(True, k, q, v, g, fr, N, G, occb, hardg, wk, wv, wi)
    (kb0, vb0, kinv0, valid0), gu = _run(False, k, q, v, g, fr, N, G, occb, hardg, wk, wv, wi)
    # ---- forward against the unfused path: the same snapshots, rounded once
    assert kb.dtype == torch.bfloat16 and vb.dtype == torch.bfloat16 and valid.dtype == torch.bool
    assert kb.shape == (B, NB, H, N, D) and kinv.shape == (B, NB, H, N)
    assert torch.equal(kb, kb0) and torch.equal(vb, vb0)
    assert torch.equal(valid, valid0)
    np.testing.assert_allclose(kinv.cpu().numpy(), kinv0.cpu().numpy(), rtol=2e-6)
    # ---- gradients against the unfused path
    names = ["dk", "dv", "dgate", "dfr", "dtemp"] + (["dq"] if sep_q else [])
    tol_u = 5e-5 if dtype == torch.float32 else 1e-2
    for n in names:
        a, b = gf[n].double().cpu().numpy(), gu[n].double().cpu().numpy()
        assert _rel(a, b) < tol_u, f"{n} fused vs unfused rel err {_rel(a, b):.3e}"
    # ---- against the oracle
    am = _am(k, q, v, g, fr, N, G, occb, hardg)
    okb, info, ogr = _oracle_grads(k, q, v, g, fr, N, G, occb, hardg, am, wk, wv, wi)
    assert_no_flips(info)
    _, ova = RO.writer_epilogue(okb)
    assert np.array_equal(valid.cpu().numpy(), ova)
    assert _rel(kb.float().cpu(), okb) < 2 ** -8
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    worst = {}
    for n in names:
        ref = ogr[n] if (n != "dk" or sep_q) else ogr["dk"] + ogr["dq"]
        worst[n] = _rel(gf[n].double().cpu().numpy().reshape(np.shape(ref)), ref)
    print("   rel err vs oracle:", {kk: f"{x:.1e}" for kk, x in worst.items()}, flush=True)
    for n, x in worst.items():
        assert x < tol, f"{n} rel err {x:.3e} >= {tol}"


MEM_CASES = [  # B, T, H, N, D, G, frt, occb, sep_q, hardg
    (2, 256, 2, 192, 128, 8, True, True, True, False),      # config 2 shape per chain: the G = 8 row kernel
    (2, 200, 2, 96, 128, 8, True, True, True, False),       # T % 16 != 0: the general row kernel at D = 128
    (2, 250, 3, 192, 64, 8, True, True, True, False),       # D = 64
    (1, 300, 4, 40, 64, 16, False, False, False, False),    # scalar fr, no occ_bin, q = k
    (1, 300, 3, 50, 128, 7, False, True, True, True),       # G = 7, hard gate
    (1, 600, 2, 96, 128, 8, True, True, True, False),       # chunked two-stream forward
    (1, 5, 2, 20, 64, 8, True, True, True, False),          # T < G
]


@pytest.mark.parametrize("case", MEM_CASES, ids=lambda c: "B{}T{}H{}N{}D{}G{}f{}o{}q{}h{}".format(*c))
def test_scan_mem_matches_unfused_and_oracle(case):
    _check(*case, seed=31)


def test_scan_mem_bf16_tokens():
    _check(2, 256, 2, 192, 128, 8, True, True, True, False, seed=33, dtype=torch.bfloat16)


def test_scan_mem_missing_upstream_gradients():
    """Only kb reaches the loss: the value and kinv gradients arrive as None and count as zeros."""
    _check(2, 128, 2, 64, 128, 8, True, True, True, False, seed=35, terms=("k",))


def test_scan_mem_refuses_other_copy_dtypes():
    """Only bf16 copies are emitted, in every mode (the general modes compose the scan and the epilogue:
    tests/test_gpu_scan_gen.py)."""
    k, q, v, g, fr = (x.to(DEV) for x in scan_inputs(1, 16, 1, 64, 0))
    with pytest.raises(NotImplementedError):
        KH.kv_scan_mem(k, v, g, fr, 16, TEMP, G=8, hard=True, detach_addr=True, q=q, dtype=torch.float32)
    with pytest.raises(NotImplementedError):
        KH.kv_scan_mem(k, v, g, fr, 16, TEMP, G=8, hard=False, detach_addr=True, q=q, dtype=torch.float16)


# ---------------------------------------------------------------- the quantised epilogue (sh25's QAT phase)
def _run_q(fused, k, q, v, g, fr, N, G, occb, hardg, wk, wv, wi, bits, group):
    """As _run, with the storage quantiser: fused = kv_scan_mem(bits, group) (slotscan_fwd_memq /
    slotscan_bwd_memq), unfused = kv_scan_c then quantize_mem (the two-pass path, memlm_sh.py:453-456 then
    :468-471).  Also returns the unfused path's fp32 snapshots."""
    kk, qq, vv, gg, ff, tp = _leaves(k, q, v, g, fr)
    kw = dict(G=G, hard=True, hard_gate=hardg, detach_addr=True, q=qq, occ_bin=occb)
    snaps = None
    if fused:
        kb, vb, kinv, valid = KH.kv_scan_mem(kk, vv, gg, ff, N, tp, bits=bits, group=group, **kw)
    else:
        kbuf, vbuf = KH.kv_scan_c(kk, vv, gg, ff, N, tp, **kw)
        kb, vb, kinv, valid = MH.quantize_mem(kbuf, vbuf, bits, group, dtype=torch.bfloat16)
        snaps = (kbuf.detach(), vbuf.detach())
    loss = (kb.float() * wk.to(DEV)).sum() + (vb.float() * wv.to(DEV)).sum() + (kinv * wi.to(DEV)).sum()
    loss.backward()
    torch.cuda.synchronize()
    grads = dict(dk=kk.grad, dv=vv.grad, dgate=gg.grad, dfr=ff.grad, dtemp=tp.grad,
                 dq=None if qq is None else qq.grad)
    return (kb.detach(), vb.detach(), kinv.detach(), valid), grads, snaps


def _check_q(B, T, H, N, D, G, frt, occb, sep_q, hardg, bits, group, seed, dtype=torch.float32):
    print(f"memq case B{B} T{T} H{H} N{N} D{D} G{G} bits={bits} group={group} frt={frt} occb={occb} q={sep_q} "
          f"hardg={hardg} {dtype}", flush=True)
    k, q, v, g, fr = scan_inputs(B, T, H, D, seed, sep_q=sep_q, frt=frt, dtype=dtype)
    NB = (T + G - 1) // G
    wk, wv = upstream((B, NB, H, N, D), seed + 1000)
    wi = torch.randn(B, NB, H, N, generator=torch.Generator().manual_seed(seed + 2000))
    (kb, vb, kinv, valid), gf, _ = _run_q(True, k, q, v, g, fr, N, G, occb, hardg, wk, wv, wi, bits, group)
    (kb0, vb0, kinv0, valid0), gu, (kbuf, vbuf) = _run_q(False, k, q, v, g, fr, N, G, occb, hardg, wk, wv, wi,
                                                         bits, group)
    # ---- forward against the two-pass path: the same quantiser values, bitwise
    assert kb.dtype == torch.bfloat16 and kb.shape == (B, NB, H, N, D) and kinv.shape == (B, NB, H, N)
    assert torch.equal(kb, kb0) and torch.equal(vb, vb0)
    assert torch.equal(valid, valid0)
    np.testing.assert_allclose(kinv.cpu().numpy(), kinv0.cpu().numpy(), rtol=2e-6)
    # ---- the quantiser against the oracle on the same fp32 snapshots (bitwise), the snapshots against the
    # fp64 oracle teacher-forced on the GPU's addresses
    okq, ovq, okinv, ova = RO.quantize_mem(kbuf.cpu().numpy(), vbuf.cpu().numpy(), bits, group)
    np.testing.assert_array_equal(kb.float().cpu().numpy(), RO.bf16_round(okq))
    np.testing.assert_array_equal(vb.float().cpu().numpy(), RO.bf16_round(ovq))
    assert np.array_equal(valid.cpu().numpy(), ova)
    np.testing.assert_allclose(kinv.cpu().numpy(), okinv, rtol=2e-6)
    am = _am(k, q, v, g, fr, N, G, occb, hardg)
    kn, qn, vn, gn, frn = np64(k), np64(q), np64(v), np64(g), np64(fr)
    okb, ovb, info = SO.scan_forward(kn, vn, gn, frn, N, TEMP, G=G, hard=True, hard_gate=hardg, eps=1e-4,
                                     detach_addr=True, q=qn, occ_bin=occb, teacher=am)
    assert_no_flips(info)
    assert _rel(kbuf.cpu(), okb) < 1e-5 and _rel(vbuf.cpu(), ovb) < 1e-5
    # ---- gradients: against the two-pass path, and against the oracle with the quantised epilogue's
    # autograd folded into the snapshot upstream (straight-through: dkbuf = dkb + 2 kq dnsq, kq = _fq(K))
    names = ["dk", "dv", "dgate", "dfr", "dtemp"] + (["dq"] if sep_q else [])
    tol_u = 5e-5 if dtype == torch.float32 else 1e-2
    for n in names:
        a, b = gf[n].double().cpu().numpy(), gu[n].double().cpu().numpy()
        assert _rel(a, b) < tol_u, f"{n} fused vs two-pass rel err {_rel(a, b):.3e}"
    kq = okq.astype(np.float64)
    nsq = (kq * kq).sum(-1)
    kiq = 1.0 / np.sqrt(np.maximum(nsq, 1e-12))
    dnsq = np.where(nsq >= 1e-12, -0.5 * kiq ** 3 * np64(wi), 0.0)
    dkb = np64(wk.to(torch.bfloat16)) + 2.0 * kq * dnsq[..., None]
    ogr = SO.scan_backward(kn, vn, gn, frn, N, TEMP, okb, ovb, info, dkb, np64(wv.to(torch.bfloat16)), G=G,
                           hard=True, hard_gate=hardg, eps=1e-4, detach_addr=True, q=qn, occ_bin=occb)
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    worst = {}
    for n in names:
        ref = ogr[n] if (n != "dk" or sep_q) else ogr["dk"] + ogr["dq"]
        worst[n] = _rel(gf[n].double().cpu().numpy().reshape(np.shape(ref)), ref)
    print("   rel err vs oracle:", {kk: f"{x:.1e}" for kk, x in worst.items()}, flush=True)
    for n, x in worst.items():
        assert x < tol, f"{n} rel err {x:.3e} >= {tol}"


MEMQ_CASES = [  # B, T, H, N, D, G, frt, occb, sep_q, hardg, bits, group
    (2, 256, 2, 192, 128, 8, True, True, True, False, 3, 16),      # sh25's QAT setting (run_sh25.sh:224)
    (2, 200, 2, 96, 128, 8, True, True, True, False, 3, 16),       # T % 16 != 0: the general row kernel
    (2, 250, 3, 192, 64, 8, True, True, True, False, 4, 8),        # D = 64, group 8 (two lanes)
    (1, 600, 2, 96, 128, 8, True, True, True, False, 3, 16),       # chunked forward: the key replay's carry
    (1, 300, 3, 50, 128, 7, False, True, True, True, 8, 128),      # one scale per row, G = 7, hard gate
    (1, 300, 2, 40, 64, 16, False, False, False, False, 2, 64),    # q = k, scalar fr, group = D = 64
    (1, 5, 2, 20, 128, 8, True, True, True, False, 5, 32),         # T < G, group 32
]


@pytest.mark.parametrize("case", MEMQ_CASES, ids=lambda c: "B{}T{}H{}N{}D{}G{}f{}o{}q{}h{}b{}g{}".format(*c))
def test_scan_memq_matches_two_pass_and_oracle(case):
    _check_q(*case, seed=37)


def test_scan_memq_bf16_tokens():
    _check_q(2, 256, 2, 192, 128, 8, True, True, True, False, 3, 16, seed=39, dtype=torch.bfloat16)
