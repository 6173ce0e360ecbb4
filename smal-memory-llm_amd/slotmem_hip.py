"""Writer epilogue and storage quantiser of the shared slot memory on MI355X (include/slotmem.h).

    writer_epilogue(kbuf, vbuf, dtype=torch.bfloat16) -> (kb, vb, kinv, valid)
        memlm_sh.py:474-475: nsq = sum K^2, kinv = rsqrt(max(nsq, 1e-12)), valid = nsq > 1e-12, the copies
        cast to `dtype` (the activation dtype).
    quantize_mem(kbuf, vbuf, bits, group, dtype=torch.bfloat16) -> (kq, vq, kinv, valid)
        memlm_sh.py:231-234 with the cast of :471: the midrise quantiser _fq on both copies (straight-through
        gradient), kinv / valid from the quantised keys.
    fq_codes(x, bits, group) -> (codes int8, scales fp32)
        the quantiser's storage form (forward only): (codes + 0.5) * scales reproduces _fq's value; an all-zero
        group has scale 0.  bits = 8, group = D is BASELINE config 5's int8 + per-row fp32 scale.
    fq_decode(codes, scales, group, dtype=torch.float32) -> values

kbuf / vbuf are the scan's fp32 snapshot copies (..., D) with D in {64, 128}.  Gradients: d kbuf = d kb +
2 K dnsq (dnsq = -0.5 kinv^3 dkinv where nsq >= 1e-12), d vbuf = d vb, the quantiser the identity -- the
autograd of the reference's expressions.  No CPU path: a missing library raises.
"""
import torch

import slotscan_lib as L

_SUPPORTED_D = (64, 128)


def _rows(x):
    D = x.shape[-1]
    if D not in _SUPPORTED_D:
        raise NotImplementedError(f"the HIP writer epilogue needs D in {_SUPPORTED_D} (got {D})")
    if not x.is_cuda:
        raise RuntimeError("the HIP writer epilogue runs on GPU tensors only (no CPU path in this package)")
    return x.numel() // D, D


def _check_q(bits, group, D):
    if bits and (bits < 2 or bits > 8 or group < 4 or group > D or group & (group - 1) or D % group):
        raise ValueError(f"bits must be 0 or 2..8 and group a power of two in [4, D] dividing D (bits={bits}, "
                         f"group={group}, D={D})")


class _Epilogue(torch.autograd.Function):
    @staticmethod
    def forward(ctx, kbuf, vbuf, bits, group, dtype):
        if kbuf.shape != vbuf.shape:
            raise ValueError("kbuf and vbuf must have the same shape")
        rows, D = _rows(kbuf)
        _check_q(bits, group, D)
        k_ = kbuf.contiguous().to(torch.float32)
        v_ = vbuf.contiguous().to(torch.float32)
        kb = torch.empty(kbuf.shape, device=kbuf.device, dtype=dtype)
        vb = torch.empty_like(kb)
        kinv = torch.empty(kbuf.shape[:-1], device=kbuf.device, dtype=torch.float32)
        valid = torch.empty(kbuf.shape[:-1], device=kbuf.device, dtype=torch.bool)
        rc = L.lib().slotmem_epilogue_fwd(L.ptr(k_), L.ptr(v_), rows, D, int(bits), int(group), L.dtype_code(dtype),
                                          L.ptr(kb), L.ptr(vb), L.ptr(kinv), L.ptr(valid.view(torch.uint8)),
                                          L.stream_of(kbuf.device))
        L.check(rc, "slotmem_epilogue_fwd")
        ctx.save_for_backward(k_)
        ctx.meta = (int(bits), int(group), dtype)
        ctx.mark_non_differentiable(valid)
        return kb, vb, kinv, valid

    @staticmethod
    def backward(ctx, dkb, dvb, dkinv, _dvalid):
        (k_,) = ctx.saved_tensors
        bits, group, dtype = ctx.meta
        rows, D = _rows(k_)
        z = lambda: torch.zeros(k_.shape, device=k_.device, dtype=dtype)
        dkb = z() if dkb is None else dkb.contiguous().to(dtype)
        dvb = z() if dvb is None else dvb.contiguous().to(dtype)
        dkinv = (torch.zeros(k_.shape[:-1], device=k_.device, dtype=torch.float32) if dkinv is None
                 else dkinv.contiguous().to(torch.float32))
        dk = torch.empty_like(k_)
        dv = torch.empty_like(k_)
        rc = L.lib().slotmem_epilogue_bwd(L.ptr(k_), L.ptr(dkb), L.ptr(dvb), L.ptr(dkinv), rows, D, bits, group,
                                          L.dtype_code(dtype), L.ptr(dk), L.ptr(dv), L.stream_of(k_.device))
        L.check(rc, "slotmem_epilogue_bwd")
        return dk, dv, None, None, None


def writer_epilogue(kbuf, vbuf, dtype=torch.bfloat16):
    """(kb, vb, kinv, valid) = the full-precision writer epilogue of memlm_sh.py:474-475."""
    return _Epilogue.apply(kbuf, vbuf, 0, 0, dtype)


def quantize_mem(kbuf, vbuf, bits, group, dtype=torch.bfloat16):
    """(kq, vq, kinv, valid) = _quantize_mem(kbuf, vbuf, bits, group) with the copies cast to `dtype`
    (memlm_sh.py:231-234, 468-471)."""
    return _Epilogue.apply(kbuf, vbuf, int(bits), int(group), dtype)


@torch.no_grad()
def fq_codes(x, bits, group):
    """(codes int8 (..., D), scales fp32 (..., D // group)) of the midrise quantiser (memlm_sh.py:221-228)."""
    rows, D = _rows(x)
    _check_q(bits, group, D)
    if not bits:
        raise ValueError("fq_codes needs bits in 2..8")
    x_ = x.contiguous().to(torch.float32)
    codes = torch.empty(x.shape, device=x.device, dtype=torch.int8)
    scales = torch.empty(x.shape[:-1] + (D // group,), device=x.device, dtype=torch.float32)
    rc = L.lib().slotmem_codes(L.ptr(x_), rows, D, int(bits), int(group), L.ptr(codes), L.ptr(scales),
                               L.stream_of(x.device))
    L.check(rc, "slotmem_codes")
    return codes, scales


def fq_decode(codes, scales, group, dtype=torch.float32):
    """(codes + 0.5) * scale per group: the quantiser's value (0 for an all-zero group)."""
    sh = codes.shape
    c = codes.float().reshape(*sh[:-1], sh[-1] // group, group)
    return ((c + 0.5) * scales.unsqueeze(-1)).reshape(sh).to(dtype)
