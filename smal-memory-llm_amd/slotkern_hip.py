"""Key-matched slot scan on MI355X: the reference's slotkern_* entry points, backed by libslotscan.so.

Drop-in surface (same names, arguments, layouts and autograd contract as the reference):
    kv_scan_c(k, v, gate, fr, N, temp, G=16, hard=False, hard_gate=False, eps=1e-4, detach_addr=False,
              q=None, nw=None, nwb=None, occ_bin=False) -> (kbuf, vbuf)       gqa25/slotkern_cuda.py:536-543
    kv_scan_g(...same...)                                                     gqa25/slotkern_kvg.py:257-265
    scan_kv(k, v, gate, fr, N, temp, G=1, hard=False, hard_gate=False, eps=1e-4, detach_addr=False, q=None)
                                                                              gqa25/slotkern_kv.py:29-41
    kv_scan(k, v, gate, fr, N, temp, hard=False, hard_gate=False, eps=1e-4, detach_addr=False, q=None,
            occ_bin=False)                                                    gqa25/slotkern_kvt.py:298-302
    ref_scan_kv(k, v, gate, fr, N, temp, G=1, hard=False, hard_gate=False, eps=1e-4, return_w=False,
                detach_addr=False, q=None, pin=True, occ_bin=False)           gqa25/slotkern_kv.py:54-64
plus kv_scan_stream(...) -- forward only, with a carried (K, V, o) state in and out, for chunked streaming,
and kv_scan_mem(...) -- the scan with the writer epilogue fused in (memlm_sh.py:453-456 then :473-475),
returning the bf16 copies with kinv and valid instead of the fp32 snapshots.

Layouts: k, q (B,T,H,DK); v (B,T,H,DV); gate (B,T,H); fr one value or (B,T,H) (per-token when fr.dim()==3,
slotkern_cuda.py:491); temp a float or 0-d tensor.  Returns fp32 kbuf (B,ceil(T/G),H,N,DK) and vbuf
(B,ceil(T/G),H,N,DV): the PRE-write state at t = 0, G, 2G, ... (slotkern_kvg.py:258-259).

Autograd: gradients for k, v, gate, fr, temp and q.  When q is None, k is passed as both the stored key and
the search query and autograd adds the two paths (slotkern_cuda.py:543).  hard_gate is straight-through:
the forward uses [gate > 0.5] and dgate flows to gate unchanged (slotkern_cuda.py:490, 533).  dfr has fr's
shape; dtemp is 0-d.  A missing upstream gradient is zeros (slotkern_cuda.py:521-522).  The op computes in
fp32; bf16 token inputs are read as bf16 and their gradients written as bf16 (autograd would cast them to
the input dtype anyway); other dtypes are cast to fp32 first.

Modes: hard=True with detach_addr=True and DK == DV in {64, 128} -- the model's training setting
(run_sh25.sh:213, 222-223) and the mode the reference's CUDA kernels cover (slotkern_cuda.py:540) -- runs
the row-sparse kernels.  Every other mode (soft addresses, the attached address gradient, DK != DV, each of
DK and DV in {64, 128}) runs the general-mode kernels (slotscan_gen_fwd / slotscan_gen_bwd), as the
reference runs it on its general Triton scan (slotkern_cuda.py:539-542).  N <= 192 in both.  Anything else
raises NotImplementedError: there is no Triton or CPU fallback here.
"""
import torch

import slotmem_hip as MH
import slotscan_lib as L

_SUPPORTED_D = (64, 128)


def _unsupported(hard, detach_addr, DK, DV, N):
    """Why the row-sparse kernels (hard + detached address, DK == DV) cannot run this call, or None."""
    if not hard:
        return "the soft write address (hard=False) is not implemented by the row-sparse HIP scan"
    if not detach_addr:
        return "an attached address gradient (detach_addr=False) is not implemented by the row-sparse HIP scan"
    if DK != DV or DK not in _SUPPORTED_D:
        return f"the HIP scan needs DK == DV in {_SUPPORTED_D} (got DK={DK}, DV={DV})"
    if N > L.lib().slotscan_max_slots(DK):
        return f"the HIP scan supports at most {L.lib().slotscan_max_slots(DK)} slots (got N={N})"
    return None


def _unsupported_gen(DK, DV, N):
    """Why the general-mode kernels cannot run this call, or None."""
    if DK not in _SUPPORTED_D or DV not in _SUPPORTED_D:
        return f"the HIP scan needs DK and DV in {_SUPPORTED_D} (got DK={DK}, DV={DV})"
    if N > L.lib().slotscan_max_slots(DK):
        return f"the HIP scan supports at most {L.lib().slotscan_max_slots(DK)} slots (got N={N})"
    return None


def _prep(k, q, v, gate, fr, temp, hard_gate):
    if not (k.is_cuda and q.is_cuda and v.is_cuda):
        raise RuntimeError("the HIP slot scan runs on GPU tensors only (no CPU path in this package)")
    dt = k.dtype if (k.dtype in (torch.float32, torch.bfloat16) and q.dtype == k.dtype and v.dtype == k.dtype) \
        else torch.float32
    k_, q_, v_ = (x.contiguous().to(dt) for x in (k, q, v))
    g = (gate > 0.5).to(torch.float32).contiguous() if hard_gate else gate.contiguous().to(torch.float32)
    frt = fr.dim() == 3
    if frt:
        if fr.shape != gate.shape:
            raise ValueError(f"per-token fr must be shaped like the gate: {tuple(fr.shape)} vs {tuple(gate.shape)}")
        fr_ = fr.contiguous().to(torch.float32)
    else:
        fr_ = fr.to(torch.float32).reshape(1).contiguous()
    temp_ = torch.as_tensor(temp, dtype=torch.float32, device=k.device).reshape(1).contiguous()
    return dt, k_, q_, v_, g, fr_, frt, temp_


def _state_in(state, B, H, N, D):
    if state is None:
        return None, None, None
    k0, v0, o0 = (x.contiguous().to(torch.float32) for x in state)
    if k0.shape != (B * H, N, D) or v0.shape != (B * H, N, D) or o0.shape != (B * H, N):
        raise ValueError("state must be (K (B*H,N,D), V (B*H,N,D), o (B*H,N))")
    return k0, v0, o0


def _carry(B, T, H, N, D, G, dev):
    """The key replay's chunk carry (slotscan_fwd_carry_bytes), or None when the forward runs as one chunk."""
    nb = L.lib().slotscan_fwd_carry_bytes(B, T, H, N, D, G)
    return torch.empty(nb // 4, device=dev, dtype=torch.float32) if nb else None


def _fwd(k_, q_, v_, g, fr_, frt, temp_, N, G, eps, occ_bin, dt, logs, state=None, mem=False, bits=0, group=16):
    """One forward launch.  mem=False: returns (kbuf, vbuf, am, logs..., final state).  mem=True: the writer
    epilogue is fused in, and the first two results are replaced by the four (kb, vb, kinv, valid); with
    bits > 0 it is the quantised epilogue (slotscan_fwd_memq: the storage quantiser's values, kinv and valid
    of the quantised keys)."""
    B, T, H, D = k_.shape
    NB = (T + G - 1) // G
    dev = k_.device
    f32 = torch.float32
    e = lambda *s, dtype=f32: torch.empty(*s, device=dev, dtype=dtype)
    if mem:
        kbuf, vbuf = e(B, NB, H, N, D, dtype=torch.bfloat16), e(B, NB, H, N, D, dtype=torch.bfloat16)
        kinv, valid = e(B, NB, H, N), e(B, NB, H, N, dtype=torch.bool)
    else:
        kbuf, vbuf = e(B, NB, H, N, D), e(B, NB, H, N, D)
    am = e(B, T, H, dtype=torch.int32)
    kold = vold = oold = cslog = None
    if logs:
        kold, vold, oold, cslog = e(B, T, H, D), e(B, T, H, D), e(B, T, H), e(B * H, T, N)
    kfin, vfin, ofin = e(B * H, N, D), e(B * H, N, D), e(B * H, N)
    k0, v0, o0 = _state_in(state, B, H, N, D)
    pre = (L.ptr(k_), L.ptr(q_), L.ptr(v_), L.dtype_code(dt), L.ptr(g), L.ptr(fr_), int(frt), L.ptr(temp_),
           B, T, H, N, D, G, float(eps), int(bool(occ_bin)))
    head = pre + (L.ptr(k0), L.ptr(v0), L.ptr(o0))
    tail = (L.ptr(am), L.ptr(kold), L.ptr(vold), L.ptr(oold), L.ptr(cslog), L.ptr(kfin), L.ptr(vfin),
            L.ptr(ofin))
    if mem and bits:
        kc = _carry(B, T, H, N, D, G, dev)
        rc = L.lib().slotscan_fwd_memq(*pre, int(bits), int(group), L.ptr(k0), L.ptr(v0), L.ptr(o0), L.ptr(kbuf),
                                       L.ptr(vbuf), L.ptr(kinv), L.ptr(valid), *tail, L.ptr(kc), L.stream_of(dev))
        L.check(rc, "slotscan_fwd_memq")
        return (kbuf, vbuf, kinv, valid), am, kold, vold, oold, cslog, kfin, vfin, ofin
    tail = tail + (L.stream_of(dev),)
    if mem:
        rc = L.lib().slotscan_fwd_mem(*head, L.ptr(kbuf), L.ptr(vbuf), L.ptr(kinv), L.ptr(valid), *tail)
        L.check(rc, "slotscan_fwd_mem")
        return (kbuf, vbuf, kinv, valid), am, kold, vold, oold, cslog, kfin, vfin, ofin
    rc = L.lib().slotscan_fwd(*head, L.ptr(kbuf), L.ptr(vbuf), *tail)
    L.check(rc, "slotscan_fwd")
    return kbuf, vbuf, am, kold, vold, oold, cslog, kfin, vfin, ofin


class _KVScanHip(torch.autograd.Function):
    @staticmethod
    def forward(ctx, k, q, v, gate, fr, temp, N, G, hard_gate, eps, occ_bin):
        D = k.shape[-1]
        if v.shape[-1] != D:
            raise ValueError("the HIP scan needs DK == DV")
        dt, k_, q_, v_, g, fr_, frt, temp_ = _prep(k, q, v, gate, fr, temp, hard_gate)
        logs = any(ctx.needs_input_grad[:6])
        kbuf, vbuf, am, kold, vold, oold, cslog, kfin, vfin, ofin = _fwd(k_, q_, v_, g, fr_, frt, temp_, N, G,
                                                                         eps, occ_bin, dt, logs)
        if logs:
            ctx.save_for_backward(k_, q_, v_, g, fr_, temp_, am, kold, vold, oold, cslog, kfin, vfin, ofin)
        ctx.meta = (int(N), int(G), frt, float(eps), bool(occ_bin), dt, tuple(fr.shape), torch.is_tensor(temp))
        return kbuf, vbuf

    @staticmethod
    def backward(ctx, dkbuf, dvbuf):
        N, G = ctx.meta[:2]
        B, T, H, D = ctx.saved_tensors[0].shape
        NB = (T + G - 1) // G
        f32 = torch.float32
        z = lambda: torch.zeros(B, NB, H, N, D, device=ctx.saved_tensors[0].device, dtype=f32)
        dkbuf = z() if dkbuf is None else dkbuf.contiguous().to(f32)
        dvbuf = z() if dvbuf is None else dvbuf.contiguous().to(f32)
        return _bwd(ctx, (dkbuf, dvbuf), mem=False) + (None,) * 5


def _bwd(ctx, grads, mem, bits=0, group=16):
    """One backward launch: grads = (dkbuf, dvbuf) fp32, or (dkb, dvb bf16, dkinv fp32) with mem=True (and
    the quantised epilogue's backward with bits > 0).  Returns the gradients of (k, q, v, gate, fr, temp)."""
    k_, q_, v_, g, fr_, temp_, am, kold, vold, oold, cslog, kfin, vfin, ofin = ctx.saved_tensors
    N, G, frt, eps, occ_bin, dt, fr_shape, temp_is_tensor = ctx.meta
    B, T, H, D = k_.shape
    dev = k_.device
    f32 = torch.float32
    ws = torch.empty(L.lib().slotscan_bwd_workspace(B, T, H, N), device=dev, dtype=torch.uint8)
    dk, dq, dv = torch.empty_like(k_), torch.empty_like(q_), torch.empty_like(v_)
    dg = torch.empty(B, T, H, device=dev, dtype=f32)
    dfr = torch.empty_like(fr_)
    dtemp = torch.empty(1, device=dev, dtype=f32)
    qa = (int(bits), int(group)) if mem and bits else ()
    args = (L.ptr(k_), L.ptr(q_), L.ptr(v_), L.dtype_code(dt), L.ptr(g), L.ptr(fr_), int(frt), L.ptr(temp_),
            B, T, H, N, D, G, float(eps), int(occ_bin)) + qa + (L.ptr(am), L.ptr(kold), L.ptr(vold), L.ptr(oold),
            L.ptr(cslog), L.ptr(kfin), L.ptr(vfin), L.ptr(ofin)) + tuple(L.ptr(x) for x in grads) + \
        (L.ptr(ws), L.ptr(dk), L.ptr(dq), L.ptr(dv), L.ptr(dg), L.ptr(dfr), L.ptr(dtemp), L.stream_of(dev))
    name = ("slotscan_bwd_memq" if qa else "slotscan_bwd_mem") if mem else "slotscan_bwd"
    L.check(getattr(L.lib(), name)(*args), name)
    dfr = dfr.reshape(fr_shape) if not frt else dfr
    dtemp = dtemp.reshape(()) if temp_is_tensor else None
    return dk, dq, dv, dg, dfr, dtemp


class _KVScanGenHip(torch.autograd.Function):
    """Every mode outside hard + detached address (slotkern_kvg._KVScanG, slotkern_kvg.py:208-253): the
    general-mode kernels, whose backward replays each stride-G segment from its emitted copy."""

    @staticmethod
    def forward(ctx, k, q, v, gate, fr, temp, N, G, hard, hard_gate, eps, detach_addr, occ_bin, pin=False,
                return_w=False):
        dt, k_, q_, v_, g, fr_, frt, temp_ = _prep(k, q, v, gate, fr, temp, hard_gate)
        B, T, H, DK = k_.shape
        DV = v_.shape[-1]
        NB = (T + G - 1) // G
        dev = k_.device
        f32 = torch.float32
        kbuf = torch.empty(B, NB, H, N, DK, device=dev, dtype=f32)
        vbuf = torch.empty(B, NB, H, N, DV, device=dev, dtype=f32)
        obuf = torch.empty(B, NB, H, N, device=dev, dtype=f32)
        am = torch.empty(B, T, H, device=dev, dtype=torch.int32) if hard else None
        wb = torch.empty(B, T, H, N, device=dev, dtype=f32) if return_w else None
        # the address log the backward replays from (only when a backward can follow)
        rlog = torch.empty(L.lib().slotscan_gen_log_bytes(B, T, H, N) // 4, device=dev, dtype=f32) \
            if any(ctx.needs_input_grad[:6]) else None
        rc = L.lib().slotscan_gen_fwd(L.ptr(k_), L.ptr(q_), L.ptr(v_), L.dtype_code(dt), L.ptr(g), L.ptr(fr_),
                                      int(frt), L.ptr(temp_), B, T, H, N, DK, DV, G, float(eps), int(occ_bin),
                                      int(hard), int(pin), L.ptr(kbuf), L.ptr(vbuf), L.ptr(obuf), L.ptr(am),
                                      L.ptr(wb), L.ptr(rlog), L.stream_of(dev))
        L.check(rc, "slotscan_gen_fwd")
        ctx.save_for_backward(k_, q_, v_, g, fr_, temp_, kbuf, vbuf, obuf, am, rlog)
        ctx.meta = (int(N), int(G), bool(hard), float(eps), bool(detach_addr), bool(occ_bin), frt, dt,
                    tuple(fr.shape), torch.is_tensor(temp), bool(pin))
        if return_w:
            ctx.mark_non_differentiable(wb)
            return kbuf, vbuf, wb
        return kbuf, vbuf

    @staticmethod
    def backward(ctx, dkbuf, dvbuf, _dwb=None):
        k_, q_, v_, g, fr_, temp_, kbuf, vbuf, obuf, am, rlog = ctx.saved_tensors
        N, G, hard, eps, detach_addr, occ_bin, frt, dt, fr_shape, temp_is_tensor, pin = ctx.meta
        B, T, H, DK = k_.shape
        DV = v_.shape[-1]
        dev = k_.device
        f32 = torch.float32
        dkbuf = torch.zeros_like(kbuf) if dkbuf is None else dkbuf.contiguous().to(f32)
        dvbuf = torch.zeros_like(vbuf) if dvbuf is None else dvbuf.contiguous().to(f32)
        ws = torch.empty(L.lib().slotscan_gen_bwd_workspace(B, H, N, DK, DV, G), device=dev, dtype=torch.uint8)
        dk, dq, dv = torch.empty_like(k_), torch.empty_like(q_), torch.empty_like(v_)
        dg = torch.empty(B, T, H, device=dev, dtype=f32)
        dfr = torch.empty_like(fr_)
        dtemp = torch.empty(1, device=dev, dtype=f32)
        rc = L.lib().slotscan_gen_bwd(L.ptr(k_), L.ptr(q_), L.ptr(v_), L.dtype_code(dt), L.ptr(g), L.ptr(fr_),
                                      int(frt), L.ptr(temp_), B, T, H, N, DK, DV, G, float(eps), int(occ_bin),
                                      int(hard), int(detach_addr), int(pin), L.ptr(kbuf), L.ptr(vbuf),
                                      L.ptr(obuf), L.ptr(am), L.ptr(rlog), L.ptr(dkbuf), L.ptr(dvbuf), L.ptr(ws),
                                      L.ptr(dk), L.ptr(dq),
                                      L.ptr(dv), L.ptr(dg), L.ptr(dfr), L.ptr(dtemp), L.stream_of(dev))
        L.check(rc, "slotscan_gen_bwd")
        dfr = dfr.reshape(fr_shape) if not frt else dfr
        dtemp = dtemp.reshape(()) if temp_is_tensor else None
        return dk, dq, dv, dg, dfr, dtemp, None, None, None, None, None, None, None, None, None


class _KVScanMemHip(torch.autograd.Function):
    """The scan with the writer epilogue fused in: forward returns (kb, vb, kinv, valid) directly."""

    @staticmethod
    def forward(ctx, k, q, v, gate, fr, temp, N, G, hard_gate, eps, occ_bin, bits=0, group=16):
        D = k.shape[-1]
        if v.shape[-1] != D:
            raise ValueError("the HIP scan needs DK == DV")
        dt, k_, q_, v_, g, fr_, frt, temp_ = _prep(k, q, v, gate, fr, temp, hard_gate)
        logs = any(ctx.needs_input_grad[:6])
        (kb, vb, kinv, valid), am, kold, vold, oold, cslog, kfin, vfin, ofin = _fwd(
            k_, q_, v_, g, fr_, frt, temp_, N, G, eps, occ_bin, dt, logs, mem=True, bits=bits, group=group)
        if logs:
            ctx.save_for_backward(k_, q_, v_, g, fr_, temp_, am, kold, vold, oold, cslog, kfin, vfin, ofin)
        ctx.meta = (int(N), int(G), frt, float(eps), bool(occ_bin), dt, tuple(fr.shape), torch.is_tensor(temp))
        ctx.q = (int(bits), int(group))
        ctx.mark_non_differentiable(valid)
        return kb, vb, kinv, valid

    @staticmethod
    def backward(ctx, dkb, dvb, dkinv, _dvalid):
        N, G = ctx.meta[:2]
        B, T, H, D = ctx.saved_tensors[0].shape
        NB = (T + G - 1) // G
        dev = ctx.saved_tensors[0].device
        bf = torch.bfloat16
        dkb = torch.zeros(B, NB, H, N, D, device=dev, dtype=bf) if dkb is None else dkb.contiguous().to(bf)
        dvb = torch.zeros(B, NB, H, N, D, device=dev, dtype=bf) if dvb is None else dvb.contiguous().to(bf)
        dkinv = torch.zeros(B, NB, H, N, device=dev, dtype=torch.float32) if dkinv is None \
            else dkinv.contiguous().to(torch.float32)
        return _bwd(ctx, (dkb, dvb, dkinv), mem=True, bits=ctx.q[0], group=ctx.q[1]) + (None,) * 7


def kv_scan_c(k, v, gate, fr, N, temp, G=16, hard=False, hard_gate=False, eps=1e-4, detach_addr=False, q=None,
              nw=None, nwb=None, occ_bin=False):
    """The slot scan on gfx950 in every mode of slotkern_cuda.kv_scan_c (slotkern_cuda.py:536-543): hard +
    detached address on the row-sparse kernels, every other mode on the general-mode kernels.  nw / nwb (the reference's warp counts) are accepted and ignored: the launch
    shape here is fixed by the gfx950 design, not tuned per call."""
    if _unsupported(hard, detach_addr, k.shape[-1], v.shape[-1], N) is None:
        return _KVScanHip.apply(k, k if q is None else q, v, gate, fr, temp, N, int(G), bool(hard_gate), eps,
                                bool(occ_bin))
    why = _unsupported_gen(k.shape[-1], v.shape[-1], N)
    if why:
        raise NotImplementedError(why)
    return _KVScanGenHip.apply(k, k if q is None else q, v, gate, fr, temp, N, int(G), bool(hard), bool(hard_gate),
                               eps, bool(detach_addr), bool(occ_bin))


def kv_scan_mem(k, v, gate, fr, N, temp, G=16, hard=False, hard_gate=False, eps=1e-4, detach_addr=False, q=None,
                occ_bin=False, dtype=torch.bfloat16, bits=0, group=16):
    """kv_scan_g followed by the writer layer's epilogue, in one forward and one backward (memlm_sh.py:453-456
    then :466-475): returns (kb, vb, kinv, valid), each (B, ceil(T/G), H, N[, D]).
    bits = 0: the full-precision epilogue (:473-475) -- kb, vb the snapshots in bf16, kinv =
    rsqrt(max(|K|^2, 1e-12)) fp32, valid = |K|^2 > 1e-12 (bool).
    bits > 0: the storage quantiser (:468-471, _quantize_mem :231-234), the setting sh25 trains its last 20 %
    in (run_sh25.sh:224, bits 3, group 16): kb, vb = _fq(snapshot, bits, group) in bf16 with a
    straight-through gradient, kinv and valid from the quantised keys.
    In the row-sparse mode (hard, detached address, DK == DV) the fp32 snapshots are never materialised.
    Every other mode runs the general-mode scan and then the epilogue kernels (two passes, the same
    outputs and autograd).  Only the bf16 copies (the activation dtype of training) are emitted."""
    if dtype != torch.bfloat16:
        raise NotImplementedError("the fused scan + epilogue emits bf16 copies only; use kv_scan_g and "
                                  "writer_epilogue for another dtype")
    MH._check_q(int(bits), int(group), k.shape[-1])
    if _unsupported(hard, detach_addr, k.shape[-1], v.shape[-1], N) is not None:
        why = _unsupported_gen(k.shape[-1], v.shape[-1], N)
        if why:
            raise NotImplementedError(why)
        kbuf, vbuf = kv_scan_c(k, v, gate, fr, N, temp, G=G, hard=hard, hard_gate=hard_gate, eps=eps,
                               detach_addr=detach_addr, q=q, occ_bin=occ_bin)
        if bits:
            return MH.quantize_mem(kbuf, vbuf, int(bits), int(group), dtype=dtype)
        return MH.writer_epilogue(kbuf, vbuf, dtype=dtype)
    return _KVScanMemHip.apply(k, k if q is None else q, v, gate, fr, temp, N, int(G), bool(hard_gate), eps,
                               bool(occ_bin), int(bits), int(group))


def kv_scan_g(k, v, gate, fr, N, temp, G=16, hard=False, hard_gate=False, eps=1e-4, detach_addr=False, q=None,
              nw=None, nwb=None, occ_bin=False):
    """Same contract as the reference's stride-G scan (slotkern_kvg.py:257-265), on the gfx950 kernels."""
    return kv_scan_c(k, v, gate, fr, N, temp, G=G, hard=hard, hard_gate=hard_gate, eps=eps,
                     detach_addr=detach_addr, q=q, occ_bin=occ_bin)


def scan_kv(k, v, gate, fr, N, temp, G=1, hard=False, hard_gate=False, eps=1e-4, detach_addr=False, q=None):
    """slotkern_kv.scan_kv's signature and dispatch (slotkern_kv.py:29-41): at G = 1 the unpinned kernel
    function (the reference's Triton kv_scan), at G > 1 ref_scan_kv with its default pin=True (rows with
    |K| < 1e-6 score 0 and take no address gradient).  Errors are raised, never swallowed."""
    if int(G) == 1:
        return kv_scan_c(k, v, gate, fr, N, temp, G=1, hard=hard, hard_gate=hard_gate, eps=eps,
                         detach_addr=detach_addr, q=q)
    return ref_scan_kv(k, v, gate, fr, N, temp, G=G, hard=hard, hard_gate=hard_gate, eps=eps,
                       detach_addr=detach_addr, q=q)


def kv_scan(k, v, gate, fr, N, temp, hard=False, hard_gate=False, eps=1e-4, detach_addr=False, q=None,
            occ_bin=False):
    """slotkern_kvt.kv_scan's signature (G = 1).  Like the reference, occ_bin is refused here
    (slotkern_kvt.py:300-301)."""
    if occ_bin:
        raise NotImplementedError("occ_bin is implemented in kv_scan_g only (the G=1 entry point refuses it, "
                                  "as the reference's does)")
    return kv_scan_c(k, v, gate, fr, N, temp, G=1, hard=hard, hard_gate=hard_gate, eps=eps,
                     detach_addr=detach_addr, q=q)


def ref_scan_kv(k, v, gate, fr, N, temp, G=1, hard=False, hard_gate=False, eps=1e-4, return_w=False,
                detach_addr=False, q=None, pin=True, occ_bin=False):
    """The reference's torch scan (slotkern_kv.py:54-64, _ref_scan_kv_impl :66-123) on the gfx950 kernels:
    same signature, defaults and outputs.  pin (its default) scores a row with |K| < 1e-6 as 0 and cuts its
    address gradient (slotkern_kv.py:88-101); memlm_sh calls it with pin=False (memlm_sh.py:461), which is
    the function the other entry points compute.  return_w=True adds the write distribution of every step
    before the gate, (B, T, H, N) fp32 -- one-hot in hard mode (slotkern_kv.py:115-117); here it carries no
    gradient.  GPU tensors only: the reference also runs on the CPU, this package has no CPU path."""
    if not pin and not return_w and _unsupported(hard, detach_addr, k.shape[-1], v.shape[-1], N) is None:
        return kv_scan_c(k, v, gate, fr, N, temp, G=G, hard=hard, hard_gate=hard_gate, eps=eps,
                         detach_addr=detach_addr, q=q, occ_bin=occ_bin)
    why = _unsupported_gen(k.shape[-1], v.shape[-1], N)
    if why:
        raise NotImplementedError(why)
    return _KVScanGenHip.apply(k, k if q is None else q, v, gate, fr, temp, N, int(G), bool(hard), bool(hard_gate),
                               eps, bool(detach_addr), bool(occ_bin), bool(pin), bool(return_w))

@torch.no_grad()
def kv_scan_stream(k, v, gate, fr, N, temp, G=8, hard_gate=False, eps=1e-4, q=None, occ_bin=False, state=None):
    """Forward-only hard scan over one chunk of a long stream, with the slot state carried across calls.

    state: None (all rows free) or the (K (B*H,N,D), V (B*H,N,D), o (B*H,N)) fp32 triple returned by the
    previous chunk.  Returns (kbuf, vbuf, state_out).  Scanning a sequence chunk by chunk this way gives
    bitwise the same snapshots as one call over the whole sequence when every chunk length is a multiple
    of G (the reference has no carry: it restarts from zero per call, memlm_sh.py:676)."""
    why = _unsupported(True, True, k.shape[-1], v.shape[-1], N)
    if why:
        raise NotImplementedError(why)
    qq = k if q is None else q
    dt, k_, q_, v_, g, fr_, frt, temp_ = _prep(k, qq, v, gate, fr, temp, hard_gate)
    kbuf, vbuf, _am, _ko, _vo, _oo, _cs, kfin, vfin, ofin = _fwd(k_, q_, v_, g, fr_, frt, temp_, int(N), int(G),
                                                                 eps, occ_bin, dt, logs=False, state=state)
    return kbuf, vbuf, (kfin, vfin, ofin)


@torch.no_grad()
def kv_scan_stream_q(k, v, gate, fr, N, temp, G=8, hard_gate=False, eps=1e-4, q=None, occ_bin=False, state=None,
                     bits=8, group=None):
    """kv_scan_stream with the emitted copies in the storage quantiser's integer form (memlm_sh.py:221-228),
    in one fused forward (slotscan_fwd_codes: the chain stores no snapshots, the row replay rebuilds every key
    and value row and emits its codes): returns ((kcodes, kscales), (vcodes, vscales), state_out), codes int8
    (B, NB, H, N, D) and fp32 scales (B, NB, H, N, D // group), bitwise the codes of kv_scan_stream's fp32
    snapshots.  bits = 8 with group = D (the default) is one fp32 absmax scale per row."""
    why = _unsupported(True, True, k.shape[-1], v.shape[-1], N)
    if why:
        raise NotImplementedError(why)
    qq = k if q is None else q
    dt, k_, q_, v_, g, fr_, frt, temp_ = _prep(k, qq, v, gate, fr, temp, hard_gate)
    B, T, H, D = k_.shape
    grp = D if group is None else int(group)
    MH._check_q(int(bits), grp, D)
    if not bits:
        raise ValueError("kv_scan_stream_q needs bits in 2..8")
    NB = (T + G - 1) // G
    dev = k_.device
    e = lambda *s_, dtype=torch.float32: torch.empty(*s_, device=dev, dtype=dtype)
    kc, vc = e(B, NB, H, N, D, dtype=torch.int8), e(B, NB, H, N, D, dtype=torch.int8)
    ks, vs = e(B, NB, H, N, D // grp), e(B, NB, H, N, D // grp)
    am = e(B, T, H, dtype=torch.int32)
    kfin, vfin, ofin = e(B * H, N, D), e(B * H, N, D), e(B * H, N)
    k0, v0, o0 = _state_in(state, B, H, N, D)
    kcar = _carry(B, T, H, N, D, int(G), dev)
    rc = L.lib().slotscan_fwd_codes(L.ptr(k_), L.ptr(q_), L.ptr(v_), L.dtype_code(dt), L.ptr(g), L.ptr(fr_),
                                    int(frt), L.ptr(temp_), B, T, H, int(N), D, int(G), float(eps),
                                    int(bool(occ_bin)), int(bits), grp, L.ptr(k0), L.ptr(v0), L.ptr(o0),
                                    L.ptr(kc), L.ptr(ks), L.ptr(vc), L.ptr(vs), L.ptr(am), L.ptr(kfin),
                                    L.ptr(vfin), L.ptr(ofin), L.ptr(kcar), L.stream_of(dev))
    L.check(rc, "slotscan_fwd_codes")
    return (kc, ks), (vc, vs), (kfin, vfin, ofin)
