"""Cosine slot read with per-token sharpness on MI355X, backed by libslotscan.so (include/slotread.h).

    slot_read(q, kbuf, buf, kinv, valid, scale, G) -> rd
        the kernel-level core of SharedMixer._read (gqa25/memlm_sh.py:383-397), token-major in and out:
        q (B,T,H,NQ,D) unit queries, kbuf / buf (B,NB,H,N,D), kinv / valid (B,NB,H,N), scale (B,T,H,NQ)
        -> rd (B,T,H,NQ,D); token t reads block t // G (memlm_sh.py:380-382).
    shared_read(q, kbuf, buf, kinv, valid, log_rsel, G, s=None, rsharp=None) -> rd
        memlm_sh.py:379-397 from the projected queries: normalises q (:379), forms the per-query multiplier
        exp(log_rsel) * exp(C tanh(s / C)) (:383-393) and calls slot_read.

Token tensors and the copies are bf16 (the reference casts the memory to the activation dtype,
memlm_sh.py:475, and the einsums run in it); other float dtypes are cast to bf16 first.  kinv and scale are
fp32, valid is bool.  The forward reproduces the reference's two bf16 roundings (the score einsum's output
and att.to(bf16)); softmax statistics are fp32.  There is no CPU path: a missing library raises.
"""
import torch

import slotscan_lib as L

_SUPPORTED_D = (64, 128)
_MAX_N = 192


def _check(q, kbuf, buf, kinv, valid, scale, G):
    if not q.is_cuda:
        raise RuntimeError("the HIP slot read runs on GPU tensors only (no CPU path in this package)")
    if q.dim() != 5 or kbuf.dim() != 5 or buf.shape != kbuf.shape:
        raise ValueError("q must be (B,T,H,NQ,D) and kbuf / buf (B,NB,H,N,D)")
    B, T, H, NQ, D = q.shape
    Bk, NB, Hk, N, Dk = kbuf.shape
    if (Bk, Hk, Dk) != (B, H, D) or NB != (T + G - 1) // G:
        raise ValueError(f"kbuf {tuple(kbuf.shape)} does not match q {tuple(q.shape)} with G={G}")
    if kinv.shape != (B, NB, H, N) or valid.shape != (B, NB, H, N) or scale.shape != (B, T, H, NQ):
        raise ValueError("kinv / valid must be (B,NB,H,N) and scale (B,T,H,NQ)")
    if D not in _SUPPORTED_D or N > _MAX_N:
        raise NotImplementedError(f"the HIP slot read needs D in {_SUPPORTED_D} and N <= {_MAX_N} (D={D}, N={N})")
    return B, T, H, NQ, D, NB, N


def _fwd(q, kbuf, buf, kinv, valid, scale, G):
    B, T, H, NQ, D, NB, N = _check(q, kbuf, buf, kinv, valid, scale, G)
    bf = torch.bfloat16
    q_, kb_, vb_ = (x.contiguous().to(bf) for x in (q, kbuf, buf))
    ki_ = kinv.contiguous().to(torch.float32)
    va_ = valid.contiguous().to(torch.bool).view(torch.uint8)
    sc_ = scale.contiguous().to(torch.float32)
    rd = torch.empty(B, T, H, NQ, D, device=q.device, dtype=bf)
    rc = L.lib().slotread_fwd(L.ptr(q_), L.ptr(kb_), L.ptr(vb_), L.ptr(ki_), L.ptr(va_), L.ptr(sc_),
                              B, T, H, NQ, N, D, int(G), L.ptr(rd), L.stream_of(q.device))
    L.check(rc, "slotread_fwd")
    return rd, (q_, kb_, vb_, ki_, va_, sc_)


class _SlotReadHip(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, kbuf, buf, kinv, valid, scale, G):
        rd, saved = _fwd(q, kbuf, buf, kinv, valid, scale, G)
        ctx.save_for_backward(*saved)
        ctx.G = int(G)
        ctx.dtypes = (q.dtype, kbuf.dtype, buf.dtype, kinv.dtype, scale.dtype)
        return rd

    @staticmethod
    def backward(ctx, drd):
        q_, kb_, vb_, ki_, va_, sc_ = ctx.saved_tensors
        B, T, H, NQ, D = q_.shape
        _, NB, _, N, _ = kb_.shape
        bf = torch.bfloat16
        do_ = drd.contiguous().to(bf)
        dq = torch.empty_like(q_)
        dkb = torch.empty_like(kb_)
        dvb = torch.empty_like(vb_)
        dki = torch.empty_like(ki_)
        dsc = torch.empty_like(sc_)
        rc = L.lib().slotread_bwd(L.ptr(q_), L.ptr(kb_), L.ptr(vb_), L.ptr(ki_), L.ptr(va_), L.ptr(sc_), L.ptr(do_),
                                  B, T, H, NQ, N, D, ctx.G, L.ptr(dq), L.ptr(dkb), L.ptr(dvb), L.ptr(dki),
                                  L.ptr(dsc), L.stream_of(q_.device))
        L.check(rc, "slotread_bwd")
        return dq, dkb, dvb, dki, None, dsc, None


def slot_read(q, kbuf, buf, kinv, valid, scale, G):
    """rd (B,T,H,NQ,D) bf16 = the cosine read of every token's NQ unit queries against its block's copy."""
    return _SlotReadHip.apply(q, kbuf, buf, kinv, valid, scale, int(G))


def shared_read(q, kbuf, buf, kinv, valid, log_rsel, G, s=None, rsharp=None):
    """memlm_sh.py:379-397 given the projected read queries q (B,T,H,NQ,D): q / max(|q|, 1e-6) in q's dtype
    (:379), multiplier exp(log_rsel) (:383) times exp(rsharp * tanh(s / rsharp)) when s (B,T,H,NQ) is given
    (:385-393)."""
    qn = q / q.float().norm(dim=-1, keepdim=True).clamp_min(1e-6).to(q.dtype)
    B, T, H, NQ, _ = q.shape
    scale = torch.exp(log_rsel.float()).expand(B, T, H, NQ)
    if s is not None:
        sf = s.float()
        if rsharp:
            sf = rsharp * torch.tanh(sf / rsharp)
        scale = scale * torch.exp(sf)
    return slot_read(qn, kbuf, buf, kinv, valid, scale, G)
