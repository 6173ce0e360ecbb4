"""Rolling-window attention on MI355X (include/slotwin.h): the exact short-term window of every layer.

    window(cq, ck, cv, W, scale=None) -> (B, Hq, T, D)

Replaces SharedMixer._window (memlm_sh.py:349-359), i.e. flex attention / scaled_dot_product_attention with
the band mask (i >= j) & (i - j < W) and the default scale 1/sqrt(D).  cq is (B, Hq, T, D), ck and cv are
(B, Hk, T, D) with Hq a multiple of Hk: query head h reads key/value head h // (Hq // Hk), which is what the
kv_nq path computes with ck.repeat_interleave(kv_nq - 1, dim=1) (memlm_sh.py:488-492) -- pass the un-repeated
keys and values here.  bf16 only (the model's activation dtype), D in {64, 128}, 1 <= W <= 16.  The operands
are read in the token-major layout the reference's views are transposed from, so those views cost no copy;
the result is returned as the same kind of view.  Autograd gives dq, dk, dv (bf16).  No CPU path: a missing
library raises.
"""
import torch

import slotscan_lib as L


def _check(cq, ck, cv, W):
    if not (cq.is_cuda and ck.is_cuda and cv.is_cuda):
        raise RuntimeError("the HIP window attention runs on GPU tensors only (no CPU path in this package)")
    if not (cq.dtype == ck.dtype == cv.dtype == torch.bfloat16):
        raise NotImplementedError("the HIP window attention computes in bf16 (got %s)" % cq.dtype)
    if cq.dim() != 4 or ck.shape != cv.shape or cq.shape[0] != ck.shape[0] or cq.shape[2:] != ck.shape[2:]:
        raise ValueError(f"expected cq (B, Hq, T, D) and ck, cv (B, Hk, T, D); got {tuple(cq.shape)}, "
                         f"{tuple(ck.shape)}, {tuple(cv.shape)}")
    if cq.shape[1] % ck.shape[1]:
        raise ValueError("the query heads must be a multiple of the key/value heads")
    if cq.shape[3] not in (64, 128):
        raise NotImplementedError(f"the HIP window attention needs D in (64, 128) (got {cq.shape[3]})")
    if not 1 <= int(W) <= 16:
        raise NotImplementedError(f"the HIP window attention supports 1 <= W <= 16 (got {W})")


class _Window(torch.autograd.Function):
    @staticmethod
    def forward(ctx, cq, ck, cv, W, scale):
        q, k, v = (x.transpose(1, 2).contiguous() for x in (cq, ck, cv))      # (B, T, H, D)
        B, T, Hq, D = q.shape
        Hk = k.shape[2]
        out = torch.empty_like(q)
        lse = torch.empty(B, Hq, T, device=q.device, dtype=torch.float32)
        rc = L.lib().slotwin_fwd(L.ptr(q), L.ptr(k), L.ptr(v), B, T, Hq, Hk, D, int(W), float(scale), L.ptr(out),
                                 L.ptr(lse), L.stream_of(q.device))
        L.check(rc, "slotwin_fwd")
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.meta = (int(W), float(scale))
        return out.transpose(1, 2)

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        W, scale = ctx.meta
        B, T, Hq, D = q.shape
        Hk = k.shape[2]
        do = dout.transpose(1, 2).contiguous().to(torch.bfloat16)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        dsum = torch.empty(B, Hq, T, device=q.device, dtype=torch.float32)
        rc = L.lib().slotwin_bwd(L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(out), L.ptr(lse), L.ptr(do), B, T, Hq, Hk, D,
                                 W, scale, L.ptr(dsum), L.ptr(dq), L.ptr(dk), L.ptr(dv), L.stream_of(q.device))
        L.check(rc, "slotwin_bwd")
        return dq.transpose(1, 2), dk.transpose(1, 2), dv.transpose(1, 2), None, None


def window(cq, ck, cv, W, scale=None):
    """Band attention over the last W tokens, the maths of memlm_sh.py:349-359 (see the module docstring)."""
    _check(cq, ck, cv, W)
    sc = cq.shape[3] ** -0.5 if scale is None else float(scale)
    return _Window.apply(cq, ck, cv, int(W), sc)
