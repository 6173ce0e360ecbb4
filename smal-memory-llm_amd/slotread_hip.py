"""Cosine slot read with per-token sharpness on MI355X, backed by libslotscan.so (include/slotread.h).

    slot_read(q, kbuf, buf, kinv, valid, scale, G) -> rd
        the kernel-level core of SharedMixer._read (gqa25/memlm_sh.py:383-397), token-major in and out:
        q (B,T,H,NQ,D) unit queries, kbuf / buf (B,NB,H,N,D), kinv / valid (B,NB,H,N), scale (B,T,H,NQ)
        -> rd (B,T,H,NQ,D); token t reads block t // G (memlm_sh.py:380-382).
    shared_read(q, kbuf, buf, kinv, valid, log_rsel, G, s=None, rsharp=None) -> rd
        memlm_sh.py:379-397 from the projected queries: normalises q (:379), forms the per-query multiplier
        exp(log_rsel) * exp(C tanh(s / C)) (:383-393) and calls slot_read.
    slot_read_out(q, kbuf, buf, kinv, valid, scale, G, wo, delta=None) -> delta_out
    shared_read_out(q, kbuf, buf, kinv, valid, log_rsel, G, wo, s=None, rsharp=None, delta=None) -> delta_out
        the read followed by the reader's output projection into the residual, delta (+)= wo_tk(rd)
        (memlm_sh.py:499-501): the gfx950 read kernel, then the library's gfx950 bf16 GEMM (slotproj_fwd) whose
        epilogue is the residual add (rd is written by the read kernel in the GEMM's row-major layout, so
        nothing is copied).  A single
        kernel doing both would have to keep a token tile x d_model fp32 output on chip; at d_model = 2048
        that bounds the tile to 32-64 tokens, and the wo_tk weight would then stream from L2 once per tile
        (or the read be recomputed per output slice), which costs more than the rd round trip it saves.

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


def _proj(x, w, d2):
    """delta + x @ w^T for x (M, K), w (N, K), d2 (M, N) or None, all bf16 on one GPU: the library's gfx950 GEMM
    with the add in its epilogue (slotproj_fwd).  Its tiles need N a multiple of 256 and K of 32; other shapes
    raise NotImplementedError (there is no second GEMM backend here)."""
    M, K = x.shape
    N = w.shape[0]
    if N % 256 or K % 32:
        raise NotImplementedError(f"the HIP read-out projection tiles d_model in multiples of 256 and H*NQ*dv in "
                                  f"multiples of 32 (got d_model={N}, H*NQ*dv={K})")
    w_ = w.contiguous()
    out = torch.empty(M, N, device=x.device, dtype=x.dtype)
    rc = L.lib().slotproj_fwd(L.ptr(x), L.ptr(w_), None if d2 is None else L.ptr(d2), M, N, K, L.ptr(out),
                              L.stream_of(x.device))
    L.check(rc, "slotproj_fwd")
    return out


def _proj_bwd(g, x, w):
    """(dx, dw) = (g w, g^T x) for the projection out = x w^T: g (M, N), x (M, K), w (N, K), bf16, on the
    library's GEMMs (slotproj_bwd).  N and K multiples of 256."""
    M, N = g.shape
    K = x.shape[1]
    if N % 256 or K % 256:
        raise NotImplementedError(f"the HIP read-out projection's backward tiles d_model and H*NQ*dv in multiples "
                                  f"of 256 (got d_model={N}, H*NQ*dv={K})")
    g_, x_, w_ = g.contiguous(), x.contiguous(), w.contiguous()
    dx = torch.empty(M, K, device=g.device, dtype=torch.bfloat16)
    dw = torch.empty(N, K, device=g.device, dtype=torch.bfloat16)
    ws = torch.empty(L.lib().slotproj_bwd_workspace(M, N, K), device=g.device, dtype=torch.uint8)
    rc = L.lib().slotproj_bwd(L.ptr(g_), L.ptr(x_), L.ptr(w_), M, N, K, L.ptr(dx), L.ptr(dw), L.ptr(ws),
                              L.stream_of(g.device))
    L.check(rc, "slotproj_bwd")
    return dx, dw


class _ReadOutHip(torch.autograd.Function):
    """delta_out = delta + rd @ wo^T with rd the slot read, as one op: the read runs on the gfx950 kernel
    (slotread_fwd), the projection is the library's bf16 GEMM with the residual add in its epilogue
    (slotproj_fwd: fp32 accumulation rounded to bf16, then added to delta and rounded again, the reference's
    bf16 Linear output and bf16 residual add), and rd -- written by the read kernel already in
    the GEMM's row-major (B*T, H*NQ*D) layout -- is kept in bf16 for dwo, as the reference's autograd keeps it
    for wo_tk.  The backward's two products (dRD = dDelta Wo, dWo = dDelta^T rd) run on the library's own GEMMs
    (slotproj_bwd), each rounded to bf16 once, as the reference's bf16 matmuls round."""

    @staticmethod
    def forward(ctx, q, kbuf, buf, kinv, valid, scale, wo, delta, G):
        rd, saved = _fwd(q, kbuf, buf, kinv, valid, scale, G)
        B, T = rd.shape[:2]
        x = rd.reshape(B * T, -1)
        w = wo.to(rd.dtype)
        if w.shape[1] != x.shape[1]:
            raise ValueError(f"wo must be (d_model, H*NQ*D) = (*, {x.shape[1]}), got {tuple(wo.shape)}")
        d2 = None
        if delta is not None:
            if delta.shape != (B, T, w.shape[0]):
                raise ValueError(f"delta must be (B, T, d_model) = {(B, T, w.shape[0])}, got {tuple(delta.shape)}")
            d2 = delta.reshape(B * T, -1).to(rd.dtype).contiguous()
        out = _proj(x, w, d2)
        ctx.save_for_backward(*saved, rd, w)
        ctx.G = int(G)
        ctx.meta = (wo.dtype, delta is not None, None if delta is None else delta.dtype)
        return out.reshape(B, T, -1)

    @staticmethod
    def backward(ctx, dout):
        q_, kb_, vb_, ki_, va_, sc_, rd, w = ctx.saved_tensors
        wo_dtype, has_delta, delta_dtype = ctx.meta
        B, T, H, NQ, D = q_.shape
        _, NB, _, N, _ = kb_.shape
        g = dout.reshape(B * T, -1).to(rd.dtype)
        drd, dwo = _proj_bwd(g, rd.reshape(B * T, -1), w)        # dRD = dDelta Wo, dWo = dDelta^T rd
        drd = drd.reshape(B, T, H, NQ, D)
        dwo = dwo.to(wo_dtype)
        dq = torch.empty_like(q_)
        dkb = torch.empty_like(kb_)
        dvb = torch.empty_like(vb_)
        dki = torch.empty_like(ki_)
        dsc = torch.empty_like(sc_)
        rc = L.lib().slotread_bwd(L.ptr(q_), L.ptr(kb_), L.ptr(vb_), L.ptr(ki_), L.ptr(va_), L.ptr(sc_),
                                  L.ptr(drd.contiguous()), B, T, H, NQ, N, D, ctx.G, L.ptr(dq), L.ptr(dkb),
                                  L.ptr(dvb), L.ptr(dki), L.ptr(dsc), L.stream_of(q_.device))
        L.check(rc, "slotread_bwd")
        ddelta = dout.to(delta_dtype) if has_delta else None
        return dq, dkb, dvb, dki, None, dsc, dwo, ddelta, None


def slot_read_out(q, kbuf, buf, kinv, valid, scale, G, wo, delta=None):
    """delta (+)= wo_tk(rd): the slot read followed by the reader's output projection (memlm_sh.py:499-501),
    wo the (d_model, H*NQ*D) weight of wo_tk (bias-free, memlm_sh.py:313), delta the (B, T, d_model) window
    output it is added to (None: the layer has no window).  Returns (B, T, d_model) in the read's dtype (bf16)."""
    return _ReadOutHip.apply(q, kbuf, buf, kinv, valid, scale, wo, delta, int(G))


def shared_read_out(q, kbuf, buf, kinv, valid, log_rsel, G, wo, s=None, rsharp=None, delta=None):
    """memlm_sh.py:379-397 then :499-501: shared_read's query preparation and multiplier, the read, and the
    wo_tk projection added to the window output delta, in one op."""
    qn = q / q.float().norm(dim=-1, keepdim=True).clamp_min(1e-6).to(q.dtype)
    B, T, H, NQ, _ = q.shape
    scale = torch.exp(log_rsel.float()).expand(B, T, H, NQ)
    if s is not None:
        sf = s.float()
        if rsharp:
            sf = rsharp * torch.tanh(sf / rsharp)
        scale = scale * torch.exp(sf)
    return slot_read_out(qn, kbuf, buf, kinv, valid, scale, G, wo, delta=delta)
