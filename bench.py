#!/usr/bin/env python3
"""Slot-scan fwd+bwd throughput on one MI355X (BASELINE metric, config 2).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--workload config2|config2_mem|config2_soft|config3*|config4|config4_wo|config5|read_train|window_train]

One step = one hard-address slot scan forward (kv_scan_c) plus its backward (torch.autograd.grad of the two
snapshot outputs against fixed upstream gradients) over one synthetic batch already resident in HBM:
B=64, T=1024 (65,536 tokens), H=6 heads, N=192 slots, DK=DV=128, G=8, temp=16, per-token fr, occ_bin,
hard, detached address (the reference's training setting, run_sh25.sh:213, 222-224).  k, q, v are bf16
N(0,1) with k and q L2-normalised, gate = sigmoid(N(0,1.5)) bf16, fr ~ U[0,2) bf16, upstream gradients
N(0,1) drawn in bf16 and passed as fp32 -- all drawn on the GPU from a seeded generator (seed 1).

--workload config2_mem runs the writer layer's scan with its epilogue fused in (kv_scan_mem: bf16 copies,
kinv, valid) and also times the two-pass path (kv_scan_c then writer_epilogue) on the same inputs.

--workload config2_soft runs the same shape with soft write addresses and the attached address gradient (the
reference's kv_scan_g defaults, on the general-mode kernels).

--workload config4 measures the read instead: one step = the 6 independent reader-layer reads of the frozen
store, forward only, with the read kernel's HBM and MFMA fractions.

Prints ONE JSON line.  `value` is tokens/s over the K timed steps; `roofline` is the dominant kernel's
algorithmic HBM bytes per launch over its average launch time, measured with HIP events recorded inside the
library on the launch stream during the timed region; `step_roofline` applies the same formula to the
whole step's algorithmic bytes.  Only the dominant kernel carries timing events during the timed steps (each
timed launch costs its stream a few microseconds); `kernels_ms` times every kernel on the last warm-up
step.  The forward-only read workloads (config4, config4_wo) run six identical layers per step and time the
first layer's launches of each timed step only: a launch with completion events cannot overlap the next.  The
streaming workload (config5) times no kernel during its timed passes (its kernels_ms are the last warm-up
pass's) and hands each call one contiguous chunk of the synthetic stream, as a streaming caller does.
`hbm_measured` is the write-only and read-only bandwidth this box reaches with plain streaming
kernels (torch fill_ and a column sum over 4 GiB), the practical ceilings beside the published 8 TB/s.
`cpu_baseline` is the fp32 torch restatement of the reference's torch scan (oracle/torch_scan.py) timed with
autograd on this host's cores: a B = 1 slice of the same workload, with config 1 beside it.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "smal-memory-llm_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBPS = 8000.0          # MI355X HBM3E, published
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, published

WORKLOADS = {
    "config2": dict(kind="scan", B=64, T=1024, H=6, N=192, D=128, G=8),
    # the writer layer's scan with its epilogue fused in (bf16 copies, kinv, valid), against the two-pass path
    "config2_mem": dict(kind="scan", B=64, T=1024, H=6, N=192, D=128, G=8, mem=True),
    # the same with sh25's storage quantiser in training (run_sh25.sh:224: 3 bits, one scale per 16 channels),
    # fused (kv_scan_mem(bits, group)) against the two-pass path (kv_scan_c, then quantize_mem)
    "config2_mem_q": dict(kind="scan", B=64, T=1024, H=6, N=192, D=128, G=8, mem=True, qbits=3, qgroup=16),
    "config2_soft": dict(kind="scan", B=64, T=1024, H=6, N=192, D=128, G=8, soft=True),
    "config3": dict(kind="scan", B=64, T=1024, H=6, N=96, D=128, G=8, seed=2),
    "config3_t512": dict(kind="scan", B=128, T=512, H=6, N=96, D=128, G=8, seed=2),
    "config3_t256": dict(kind="scan", B=256, T=256, H=6, N=96, D=128, G=8, seed=2),
    "config3_t128": dict(kind="scan", B=512, T=128, H=6, N=96, D=128, G=8, seed=2),
    # frozen-store read fan-out: 6 reader layers, one block (NB = 1: G = T), one query per head and token
    "config4": dict(kind="read", B=64, T=1024, H=6, N=192, D=128, G=1024, NQ=1, layers=6),
    # long-context streaming: 128 chunks of 1024 tokens, state carried, int8 + per-row fp32 scale emission
    "config5": dict(kind="stream", B=8, T=131072, H=6, N=192, D=128, G=8, chunk=1024, seed=4),
    # config 4 with each reader layer's output projection into the residual (memlm_sh.py:499-501): the read,
    # then wo_tk (d_model 2048, bias-free) added to the window output, forward only
    "config4_wo": dict(kind="read_out", B=64, T=1024, H=6, N=192, D=128, G=1024, NQ=1, layers=6, DM=2048),
    # one reader layer of training at the sh25 shape (G = 8, NQ = 2, d_model 2048): the read and wo_tk into
    # the residual, forward + backward (the projection's backward on the library's GEMMs, slotproj_bwd)
    "read_out_train": dict(kind="read_out", B=64, T=1024, H=6, N=192, D=128, G=8, NQ=2, layers=1, DM=2048,
                           backward=True),
    # one reader layer of training at the config-2 memory: G = 8 tokens per block, NQ = 2, forward + backward
    "read_train": dict(kind="read", B=64, T=1024, H=6, N=192, D=128, G=8, NQ=2, layers=1, backward=True),
    # one layer's 16-token window at the training shape (run_sh25.sh:223): 4 K/V heads x 128, kv_nq 4 (the
    # main call plus the 12 extra queries on the same K/V heads), forward + backward
    "window_train": dict(kind="window", B=64, T=1024, Hk=4, D=128, W=16, NQ=4),
}


def scan_workload_inputs(W, dev):
    """The scan workloads' synthetic batch, drawn on the GPU from a seeded generator (seed W['seed'], 1 by
    default) in a fixed order: k, q, v bf16 N(0,1) with k and q L2-normalised, gate = sigmoid(N(0,1.5)) bf16,
    fr ~ U[0,2) bf16, then the upstream snapshot gradients N(0,1) drawn in bf16 and passed as fp32.  Returns
    (k, q, v, gate, fr, temp, dkb, dvb, rn) with the six inputs requiring grad and rn the generator's
    normal draw for later tensors.  The full-size parity tests run on exactly this batch."""
    import torch
    B, T, H, N, D, G = (W[x] for x in ("B", "T", "H", "N", "D", "G"))
    gen = torch.Generator(device=dev).manual_seed(W.get("seed", 1))
    rn = lambda *s: torch.randn(*s, device=dev, generator=gen)
    unit = lambda x: x / x.norm(dim=-1, keepdim=True)
    k = unit(rn(B, T, H, D)).to(torch.bfloat16).requires_grad_()
    q = unit(rn(B, T, H, D)).to(torch.bfloat16).requires_grad_()
    v = rn(B, T, H, D).to(torch.bfloat16).requires_grad_()
    gate = torch.sigmoid(rn(B, T, H) * 1.5).to(torch.bfloat16).requires_grad_()
    fr = (torch.rand(B, T, H, device=dev, generator=gen) * 2).to(torch.bfloat16).requires_grad_()
    temp = torch.tensor(16.0, device=dev, requires_grad=True)
    NB = (T + G - 1) // G
    dkb = rn(B, NB, H, N, D).to(torch.bfloat16).float()
    dvb = rn(B, NB, H, N, D).to(torch.bfloat16).float()
    return k, q, v, gate, fr, temp, dkb, dvb, rn


def stream_workload_inputs(W, T, dev):
    """The streaming workload's synthetic tokens (config 5), T of them per batch row, drawn on the GPU from
    the workload's seeded generator (seed 4) in a fixed order: k, q, v bf16 N(0,1) with k and q L2-normalised,
    gate = sigmoid(N(0,1.5)) bf16, fr ~ U[0,2) bf16 -- config 2's distributions.  The parity test of the
    carried-state stream draws its 3,072 tokens per row the same way."""
    import torch
    B, H, D = W["B"], W["H"], W["D"]
    gen = torch.Generator(device=dev).manual_seed(W.get("seed", 4))
    rn = lambda *s: torch.randn(*s, device=dev, generator=gen)
    unit = lambda x: x / x.norm(dim=-1, keepdim=True)
    k = unit(rn(B, T, H, D)).to(torch.bfloat16)
    q = unit(rn(B, T, H, D)).to(torch.bfloat16)
    v = rn(B, T, H, D).to(torch.bfloat16)
    gate = torch.sigmoid(rn(B, T, H) * 1.5).to(torch.bfloat16)
    fr = (torch.rand(B, T, H, device=dev, generator=gen) * 2).to(torch.bfloat16)
    return k, q, v, gate, fr


def algorithmic_bytes(B, T, H, N, D, G, mem=False, soft=False, memq=False):
    """Per-kernel and per-step algorithmic HBM bytes (inputs read once, outputs written once; logs, Dn and
    staging are implementation choices and are not counted).  Token tensors bf16, snapshots fp32, gate and
    fr bf16 as the caller holds them (the kernels read the fp32 copies the wrapper makes: 4 B each).
    mem: the fused writer epilogue -- bf16 snapshot copies, plus kinv (fp32) and valid (1 B) per key row
    out and dkinv (fp32) per key row in.  soft: the general-mode kernels, whose forward also emits the
    occupancy snapshot (fp32 per row) and whose backward reads the three snapshots back (the replay
    scratch is an implementation choice and is not counted).  memq: the quantised epilogue, whose copies the
    row replay emits (it reads the key tokens too) and the chain none."""
    tok = B * T * H
    NB = (T + G - 1) // G
    rows = B * NB * H * N
    snap = rows * D * (2 if mem else 4)
    kx_f, kx_b = (rows * 5, rows * 4) if mem else (0, 0)
    row = tok * D * 2
    if soft:
        per_kernel = {
            "gen_fwd": 3 * row + 2 * tok * 4 + 2 * snap + rows * 4,
            "gen_bwd": 3 * row + 2 * tok * 4 + 2 * snap + rows * 4 + 2 * snap + 3 * row + 2 * tok * 4,
        }
        step = (3 * row + 2 * tok * 2 + 2 * snap) + (2 * snap + 3 * row + 2 * tok * 2 + 3 * row + 2 * tok * 2)
        return per_kernel, step
    per_kernel = {
        "chain_fwd": 2 * row + 2 * tok * 4 + snap + kx_f,          # q, k, gate, fr in; kbuf (kinv, valid) out
        "rows_fwd": row + tok * 4 + snap,                          # v, gate in; vbuf out
        "rows_bwd": 2 * snap + kx_b + 2 * row + tok * 4 + 2 * row,  # dkbuf, dvbuf (dkinv), k, v, gate in; dk, dv out
        "chain_bwd": row + 2 * tok * 4 + row + 2 * tok * 4,        # q, gate, fr in; dq, dgate, dfr out
    }
    if memq:
        per_kernel["chain_fwd"] = 2 * row + 2 * tok * 4              # q, k, gate, fr in
        per_kernel["rows_fwd"] = 2 * row + tok * 4 + 2 * snap + kx_f  # k, v, gate in; kb, vb, kinv, valid out
    step = (3 * row + 2 * tok * 2 + 2 * snap + kx_f) + \
        (2 * snap + kx_b + 3 * row + 2 * tok * 2 + 3 * row + 2 * tok * 2)
    return per_kernel, step


def read_algorithmic(B, T, H, N, D, NQ, layers, NB=1):
    """Per-launch (one reader layer) algorithmic bytes and MFMA flops of the forward read: q and rd bf16, the
    sharpness multiplier as the bf16 value the model holds, one pass over the bf16 copies (NB blocks) and
    their kinv / valid."""
    tok = B * T * H * NQ
    by = tok * (2 * D + 2 * D + 2) + 2 * B * NB * H * N * D * 2 + (B * NB * H * N * 5 if NB > 1 else 0)
    fl = 2 * 2 * tok * N * D
    return by, fl


def read_bwd_algorithmic(B, T, H, N, D, NQ, NB):
    """Backward read: q, drd, the two copies, kinv / valid and the multiplier in; dq, dkbuf, dvbuf bf16 and
    dkinv, dscale out."""
    tok = B * T * H * NQ
    cp = B * NB * H * N * D * 2
    return tok * (2 * D + 2 * D + 2) + 2 * cp + B * NB * H * N * 5 + tok * 2 * D + 2 * cp + B * NB * H * N * 4 + tok * 4


def copy_calibration(dev):
    """One 1 GiB device-to-device copy (reads 1 GiB, writes 1 GiB), so that HBM byte counters of the same
    run (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE) can be scaled by what they report for it."""
    import torch
    src = torch.empty(1 << 28, device=dev, dtype=torch.float32).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def hbm_ceilings(dev, nbytes=1 << 32, reps=5):
    """The HBM bandwidth this box reaches with plain streaming kernels, beside the 8 TB/s published peak: a
    write-only pass (torch fill_) and a read-only pass (a column sum, torch sum over dim 0 of a 4096-row view)
    over a 4 GiB buffer, best of `reps`, in GB/s.
    The row-parallel scan kernels are bounded by these rather than by the published figure."""
    import torch
    buf = torch.empty(nbytes // 4, device=dev, dtype=torch.float32)
    buf.fill_(1.0)
    torch.cuda.synchronize()
    out = {}
    for name, fn in (("write", lambda: buf.fill_(2.0)), ("read", lambda: buf.view(4096, -1).sum(0))):
        best = None
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            b.synchronize()
            ms = a.elapsed_time(b)
            best = ms if best is None else min(best, ms)
        out[f"{name}_GBps"] = round(nbytes / (best * 1e-3) / 1e9, 1)
    del buf
    out["method"] = "torch fill_ (write) and column sum (read) over 4 GiB, best of 5"
    return out


def measured_traffic(workload):
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE (scaled by a copy kernel of known
    size), read from the committed summary profiles/hbm_traffic_<workload>.md; {} when there is none."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{workload}.md")
    out = {}
    if os.path.exists(path):
        for line in open(path):
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) == 5 and cells[4].replace(",", "").isdigit():
                out[cells[0]] = int(cells[4].replace(",", ""))
    return out


def _host_cpu():
    """(model name, cores this process may run on) of the host, for the CPU baseline's record."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, len(os.sched_getaffinity(0))


def _timed(fn, reps=3):
    """Median wall-clock seconds of `reps` runs after one warm-up run."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def cpu_baseline(W, seed=1):
    """The scan's fp32 torch restatement (oracle/torch_scan.py, the reference's own torch loop
    slotkern_kv.py:66-123) forward plus autograd backward on this host's cores, all of them
    (torch.set_num_threads over the CPUs this process may use): BASELINE config 1 in full, and a B = 1
    slice of the workload at its full T, H, N, D (the full batch's autograd graph would need on the order of
    100 GB of saved per-step state).  Median of 3 runs after one warm-up each.  `value` is the slice's
    tokens/s; config 1's is reported beside it."""
    import torch
    from oracle.torch_scan import scan_torch
    model, cores = _host_cpu()
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    hard = not W.get("soft", False)
    mem = W.get("mem", False)

    def case(B, T, H, N, D, G, sd):
        gen = torch.Generator().manual_seed(sd)
        r = lambda *s: torch.randn(*s, generator=gen)
        unit = lambda x: x / x.norm(dim=-1, keepdim=True)
        k, q, v = unit(r(B, T, H, D)).requires_grad_(), unit(r(B, T, H, D)).requires_grad_(), r(B, T, H, D).requires_grad_()
        g = torch.sigmoid(1.5 * r(B, T, H)).requires_grad_()
        fr = (2 * torch.rand(B, T, H, generator=gen)).requires_grad_()
        temp = torch.tensor(16.0, requires_grad=True)
        NB = (T + G - 1) // G
        dkb, dvb = r(B, NB, H, N, D), r(B, NB, H, N, D)
        dki = r(B, NB, H, N)

        def step():
            kb, vb = scan_torch(k, v, g, fr, N, temp, G=G, hard=hard, detach_addr=hard, q=q, occ_bin=True)
            outs, ups = (kb, vb), (dkb, dvb)
            if mem:                          # the writer epilogue (memlm_sh.py:474-475) and its autograd
                kinv = torch.rsqrt(kb.pow(2).sum(-1).clamp_min(1e-12))
                outs, ups = (kb.to(torch.bfloat16), vb.to(torch.bfloat16), kinv), (dkb, dvb, dki)
            torch.autograd.grad(outs, (k, q, v, g, fr, temp), ups)
        return _timed(step)

    try:
        t1 = case(2, 128, 1, 64, 64, 8, 0)
        ts = case(1, W["T"], W["H"], W["N"], W["D"], W["G"], seed)      # B = 1 slice of the workload
    finally:
        torch.set_num_threads(prev)
    mode = ("hard, detached address" if hard else "soft address, attached") + (", writer epilogue" if mem else "")
    return dict(value=round(W["T"] / ts, 1), unit="tokens/s", cores=cores, kind="port",
                sample=f"B=1 slice of the workload (T={W['T']}, H={W['H']}, N={W['N']}, D={W['D']}, G={W['G']}, "
                       f"{mode}): fp32 torch restatement of the reference's torch scan (oracle/torch_scan.py), "
                       f"forward + autograd backward, median of 3 after a warm-up, {ts:.2f} s per run",
                seconds=round(ts, 3), threads=cores, cpu_model=model, os_cpu_count=os.cpu_count(),
                config1={"tokens_per_s": round(2 * 128 / t1, 1), "seconds": round(t1, 4),
                         "shape": "B=2, T=128, H=1, N=64, D=64, G=8, fwd+bwd, fp32"})


def cpu_baseline_read(W, seed=3):
    """The read's fp32 torch restatement (oracle/torch_scan.read_torch, memlm_sh.py:383-395) on this host's
    cores: the whole workload (every reader layer at the full batch), median of 3 after a warm-up."""
    import torch
    from oracle.torch_scan import read_torch
    model, cores = _host_cpu()
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    Bs, T, H, N, D, NQ, layers = W["B"], W["T"], W["H"], W["N"], W["D"], W["NQ"], W["layers"]
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen)
    unit = lambda x: x / x.norm(dim=-1, keepdim=True)
    K, V = unit(r(Bs, 1, H, N, D)), r(Bs, 1, H, N, D)
    q = unit(r(Bs, 1, H, T * NQ, D))
    sc = torch.nn.functional.softplus(r(Bs, 1, H, T * NQ)) + 1.0
    kinv, valid = torch.ones(Bs, 1, H, N), torch.ones(Bs, 1, H, N, dtype=torch.bool)
    try:
        with torch.no_grad():
            dt = _timed(lambda: [read_torch(q, K, V, kinv, valid, sc) for _ in range(layers)])
    finally:
        torch.set_num_threads(prev)
    return dict(value=round(Bs * T / dt, 1), unit="tokens/s", cores=cores, kind="port",
                sample=f"the whole workload: {layers} reader layers at B={Bs} (T={T}, H={H}, N={N}, D={D}), fp32 "
                       f"torch restatement of the read (oracle/torch_scan.read_torch), median of 3 after a "
                       f"warm-up, {dt:.3f} s per run",
                seconds=round(dt, 4), threads=cores, cpu_model=model)


def bench_stream(args, W):
    """Config 5: forward-only streaming scan, 1024-token chunks with the slot state carried, every chunk's
    snapshot copies emitted as int8 codes + one fp32 scale per row (the storage quantiser, bits 8, group D).
    Each chunk is one kv_scan_stream_q call, the fused path (slotscan_fwd_codes): the chain stores no
    snapshots and the row replay emits both copies' codes, beside the next chain chunk.  The line also times
    the two-pass path on the same stream (kv_scan_stream's fp32 snapshots, then fq_codes on a second stream)
    as `two_pass_ms_per_step`.  One step = the whole T-token stream."""
    import torch
    import slotkern_hip as KH
    import slotmem_hip as MH
    import slotscan_lib as L

    B, T, H, N, D, G, C = (W[x] for x in ("B", "T", "H", "N", "D", "G", "chunk"))
    dev = torch.device("cuda:0")
    k, q, v, gate, fr = stream_workload_inputs(W, T, dev)
    temp = torch.tensor(16.0, device=dev)                   # resident: no host copy per call
    side = torch.cuda.Stream(device=dev)                  # default priority
    main = torch.cuda.current_stream(dev)
    # the stream's chunks as they reach a streaming caller: one contiguous (B, C, ...) tensor per chunk, resident
    # before the timed region (slicing the whole (B, T, ...) synthetic input per call would time a strided
    # copy of every chunk, which is the bench's own layout, not the scan)
    chunks = [tuple(x[:, t0:t0 + C].contiguous() for x in (k, q, v, gate, fr)) for t0 in range(0, T, C)]
    del k, q, v, gate, fr

    def stream_pass():
        st = None
        out = None
        for kc, qc, vc, gc, fc in chunks:
            kq, vq, st = KH.kv_scan_stream_q(kc, vc, gc, fc, N, temp, G=G, q=qc, occ_bin=True, state=st, bits=8)
            out = (kq, vq)
        return st, out

    def stream_pass_two():
        st = None
        pending = None
        for kc, qc, vc, gc, fc in chunks:
            kb, vb, st = KH.kv_scan_stream(kc, vc, gc, fc, N, temp, G=G, q=qc, occ_bin=True, state=st)
            ev = torch.cuda.Event()
            ev.record(main)
            side.wait_event(ev)
            with torch.cuda.stream(side):
                kb.record_stream(side)
                vb.record_stream(side)
                pending = (MH.fq_codes(kb, 8, D), MH.fq_codes(vb, 8, D))
            del kb, vb
        main.wait_stream(side)
        return st, pending

    stream_pass_two()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    stream_pass_two()
    torch.cuda.synchronize()
    two_ms = (time.perf_counter() - t0) * 1e3
    # every kernel is timed on the last warm-up pass; the timed passes run without completion events
    for i in range(args.warmup):
        if i == args.warmup - 1:
            L.profile(True)
        stream_pass()
    torch.cuda.synchronize()
    L.profile(False)
    prof = L.profile_read()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        stream_pass()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    tok = B * T
    NBc = (C + G - 1) // G
    per_tok = 3 * H * D * 2 + 2 * H * 2 + 2 * H * N * (D + 4) // G      # inputs + int8 emission with row scales
    by = tok * per_tok
    out = {
        "metric": "streaming slot-scan forward tokens/s (config 5: B8 T131072 H6 S192 d128, int8 + row-scale emission)",
        "value": round(tok / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32 state, bf16 tokens, int8 emission",
        "data": "synthetic (seeded GPU generator, seed 4)",
        "config": {"workload": args.workload, "B": B, "T": T, "H": H, "N": N, "D": D, "G": G, "chunk": C,
                   "chunks": T // C, "snapshots_per_chunk": NBc, "tokens_per_step": tok},
        "step_roofline": {"algorithmic_bytes": by, "achieved": round(by / (ms * 1e-3) / 1e9, 1),
                          "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                          "frac": round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)},
        "kernels_ms": {n: round(x / c, 4) for n, (x, c) in prof.items()},
        "kernels_total_ms": {n: round(x, 3) for n, (x, c) in prof.items()},     # one stream pass
        "two_pass_ms_per_step": round(two_ms, 3),
    }
    print(json.dumps(out), flush=True)


def window_bytes(B, T, Hq, Hk, D):
    """Algorithmic HBM bytes of one window call: forward q, k, v in, out and the fp32 log-sum-exp out;
    backward q, k, v, out, dout and the log-sum-exp in, dq, dk, dv out (bf16 tokens)."""
    row = B * T * D * 2
    fwd = row * (2 * Hq + 2 * Hk) + B * T * Hq * 4
    bwd = row * (3 * Hq + 2 * Hk) + B * T * Hq * 4 + row * (Hq + 2 * Hk)
    return fwd, bwd


def bench_window(args, W):
    """One layer's rolling window (memlm_sh.py:482-492) at the training shape: window(cq, ck, cv) over the
    Hk K/V heads plus window(cq2, ck, cv) for the Hk (NQ - 1) extra queries, forward and backward."""
    import torch
    import slotwin_hip as WH
    import slotscan_lib as L

    B, T, Hk, D, Wn, NQ = (W[x] for x in ("B", "T", "Hk", "D", "W", "NQ"))
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(6)
    rn = lambda *s: torch.randn(*s, device=dev, generator=gen).to(torch.bfloat16)
    view = lambda x: x.transpose(1, 2).requires_grad_()           # (B, T, H, D) viewed as (B, H, T, D)
    cq, ck, cv = view(rn(B, T, Hk, D)), view(rn(B, T, Hk, D)), view(rn(B, T, Hk, D))
    cq2 = view(rn(B, T, Hk * (NQ - 1), D))
    # the upstream gradients arrive as the same kind of view: the caller transposes the window's output back
    # and flattens it token-major (memlm_sh.py:485-486, 493-494)
    do1, do2 = rn(B, T, Hk, D).transpose(1, 2), rn(B, T, Hk * (NQ - 1), D).transpose(1, 2)
    leaves = (cq, cq2, ck, cv)

    def step():
        o1 = WH.window(cq, ck, cv, Wn)
        o2 = WH.window(cq2, ck, cv, Wn)
        return torch.autograd.grad((o1, o2), leaves, (do1, do2))

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    L.profile(True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    L.profile(False)
    prof = L.profile_read()
    if args.copy_calibration:
        copy_calibration(dev)
    ms = (t1 - t0) * 1e3 / args.steps
    f1, b1 = window_bytes(B, T, Hk, Hk, D)
    f2, b2 = window_bytes(B, T, Hk * (NQ - 1), Hk, D)
    step_bytes = f1 + b1 + f2 + b2
    kms = {n: tot / cnt for n, (tot, cnt) in prof.items()}
    fwd_ms = prof["win_fwd"][0] / args.steps
    bwd_ms = prof["win_bwd"][0] / args.steps
    out = {
        "metric": f"window attention fwd+bwd tokens/s (W{Wn}, {Hk} K/V heads x {D}, kv_nq {NQ}, B{B} T{T})",
        "value": round(B * T / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded GPU generator, seed 6)",
        "config": {"workload": args.workload, "B": B, "T": T, "Hk": Hk, "Hq": [Hk, Hk * (NQ - 1)], "D": D, "W": Wn,
                   "tokens_per_step": B * T},
        "roofline": {"bound": "hbm", "kernel": "win_fwd + win_bwd (step)",
                     "achieved": round(step_bytes / ((fwd_ms + bwd_ms) * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(step_bytes / ((fwd_ms + bwd_ms) * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                     "traffic": None, "algorithmic_bytes_per_step": step_bytes,
                     "kernel_ms_per_step": round(fwd_ms + bwd_ms, 4)},
        "fwd_roofline": {"achieved": round((f1 + f2) / (fwd_ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBPS,
                         "frac": round((f1 + f2) / (fwd_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                         "algorithmic_bytes": f1 + f2, "ms": round(fwd_ms, 4)},
        "bwd_roofline": {"achieved": round((b1 + b2) / (bwd_ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBPS,
                         "frac": round((b1 + b2) / (bwd_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                         "algorithmic_bytes": b1 + b2, "ms": round(bwd_ms, 4)},
        "kernels_ms": {n: round(x, 4) for n, x in kms.items()},
    }
    print(json.dumps(out), flush=True)


def bench_read_out(args, W):
    """Config 4 with the output projection: per reader layer slot_read_out = the read kernel, then the library's
    bf16 GEMM delta + rd wo^T into the residual (proj_gemm).  Reports the GEMM's MFMA fraction and the read
    kernel's HBM fraction from the library's own HIP events on the launch stream, and, for comparison, the
    same GEMM as one library call (torch.addmm, hipBLASLt) timed with events on the current stream."""
    import torch
    import slotread_hip as RH
    import slotscan_lib as L

    B, T, H, N, D, G, NQ, layers, DM = (W[x] for x in ("B", "T", "H", "N", "D", "G", "NQ", "layers", "DM"))
    NB = (T + G - 1) // G
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(3)
    rn = lambda *s: torch.randn(*s, device=dev, generator=gen)
    unit = lambda x: x / x.norm(dim=-1, keepdim=True)
    bf = torch.bfloat16
    K = unit(rn(B, NB, H, N, D)).to(bf)
    V = rn(B, NB, H, N, D).to(bf)
    kinv = torch.ones(B, NB, H, N, device=dev)
    valid = torch.ones(B, NB, H, N, device=dev, dtype=torch.bool)
    qs = [unit(rn(B, T, H, NQ, D)).to(bf) for _ in range(layers)]
    scs = [torch.nn.functional.softplus(rn(B, T, H, NQ)) + 1.0 for _ in range(layers)]
    KD = H * NQ * D
    wos = [(rn(DM, KD) / KD ** 0.5).to(bf) for _ in range(layers)]
    deltas = [rn(B, T, DM).to(bf) for _ in range(layers)]

    bwd = W.get("backward", False)
    if bwd:
        for t_ in [K, V, kinv] + qs + scs + wos + deltas:
            t_.requires_grad_()
        douts = [rn(B, T, DM).to(bf) for _ in range(layers)]

    def step(probe=False):
        if bwd:
            for t_ in [K, V, kinv] + qs + scs + wos + deltas:
                t_.grad = None                                  # time the op, not a gradient accumulation
            outs = [RH.slot_read_out(qs[i], K, V, kinv, valid, scs[i], G, wos[i], delta=deltas[i])
                    for i in range(layers)]
            torch.autograd.backward(outs, douts)
            return outs
        with torch.no_grad():
            outs = []
            for i in range(layers):
                if probe and i == 0:
                    L.profile(True)
                outs.append(RH.slot_read_out(qs[i], K, V, kinv, valid, scs[i], G, wos[i], delta=deltas[i]))
                if probe and i == 0:
                    L.profile(False)
            return outs

    # As bench_read: the forward-only workload times the first layer's launches of each timed step, the
    # training workload every launch.
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    if bwd:
        L.profile(True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(probe=not bwd)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    L.profile(False)
    prof = L.profile_read()
    if args.copy_calibration:
        copy_calibration(dev)
    ms = (t1 - t0) * 1e3 / args.steps
    # the projection GEMM alone, same shapes (x (B*T, KD) bf16 @ wo^T into delta), timed with HIP events
    x = torch.empty(B * T, KD, device=dev, dtype=bf).normal_()
    d2 = deltas[0].reshape(B * T, DM)
    for _ in range(3):
        torch.addmm(d2, x, wos[0].t())
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = max(args.steps, 10)
    e0.record()
    for _ in range(reps):
        torch.addmm(d2, x, wos[0].t())
    e1.record()
    torch.cuda.synchronize()
    gemm_ms = e0.elapsed_time(e1) / reps
    bwd_lib_ms = None
    if bwd:     # the projection's backward products as library GEMMs (torch.mm, hipBLASLt), same operands
        g2 = douts[0].reshape(B * T, DM)
        w0 = wos[0].detach()
        lib = lambda: (torch.mm(g2, w0), torch.mm(g2.t(), x))
        for _ in range(3):
            lib()
        e0.record()
        for _ in range(reps):
            lib()
        e1.record()
        torch.cuda.synchronize()
        bwd_lib_ms = e0.elapsed_time(e1) / reps
    tot, cnt = prof["read_fwd"]
    rms = tot / cnt
    ptot, pcnt = prof["proj"]
    pms = ptot / pcnt
    rby, rfl = read_algorithmic(B, T, H, N, D, NQ, 1, NB)
    gfl = 2.0 * B * T * KD * DM
    gby = 2 * (B * T * KD + DM * KD + 2 * B * T * DM)          # x, wo and delta in, the sum out (bf16)
    mt = measured_traffic(args.workload)                        # committed rocprofv3 FETCH/WRITE summary
    out = {
        "metric": f"slot-read + wo_tk fan-out tokens/s ({layers} reader layers, frozen store B{B} H{H} S{N} d{D}, "
                  f"d_model {DM}, forward)",
        "value": round(B * T / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded GPU generator, seed 3)",
        "config": {"workload": args.workload, "B": B, "T": T, "H": H, "N": N, "D": D, "NQ": NQ, "G": G,
                   "layers": layers, "d_model": DM, "tokens_per_step": B * T},
        "roofline": {"bound": "mfma", "kernel": "proj_gemm (wo_tk projection + residual add)",
                     "achieved": round(gfl / (pms * 1e-3) / 1e12, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(gfl / (pms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                     "traffic": mt.get("proj_gemm"), "traffic_source": "profiles/hbm_traffic_config4_wo.md"
                     if "proj_gemm" in mt else None, "flops_per_launch": gfl, "algorithmic_bytes_per_launch": gby,
                     "avg_launch_ms": round(pms, 4), "hbm_gbps": round(gby / (pms * 1e-3) / 1e9, 1),
                     "hbm_frac": round(gby / (pms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                     "library_gemm_ms": round(gemm_ms, 4)},
        "read_roofline": {"bound": "hbm", "kernel": "read_fwd", "achieved": round(rby / (rms * 1e-3) / 1e9, 1),
                          "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(rby / (rms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                          "algorithmic_bytes_per_launch": rby, "avg_launch_ms": round(rms, 4),
                          "mfma_frac": round(rfl / (rms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)},
        "per_layer_ms": {"read_fwd": round(rms, 4), "proj_gemm": round(pms, 4), "library_gemm": round(gemm_ms, 4),
                         "layer_total": round(ms / layers, 4)},
        "kernels_ms": {n: round(x / c, 4) for n, (x, c) in prof.items()},
    }
    if bwd:
        kb_ = {n: prof[n][0] / prof[n][1] for n in ("proj_drd", "proj_dwo", "proj_reduce")}
        bms = sum(kb_.values())
        bfl = 2 * gfl                                               # drd and dwo, each the forward's flops
        out["metric"] = (f"slot-read + wo_tk training tokens/s (one reader layer, B{B} T{T} H{H} S{N} d{D} G{G} "
                         f"NQ{NQ}, d_model {DM}, forward + backward)")
        out["proj_bwd_roofline"] = {"bound": "mfma", "kernel": "slotproj_bwd (weight transpose, proj_gemm for drd, "
                                    "projt_gemm + proj_reduce for dwo)", "flops_per_launch": bfl,
                                    "achieved": round(bfl / (bms * 1e-3) / 1e12, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                                    "unit": "TFLOP/s", "frac": round(bfl / (bms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                                    "avg_launch_ms": round(bms, 4), "kernels_ms": {n: round(x, 4) for n, x in kb_.items()},
                                    "library_gemms_ms": round(bwd_lib_ms, 4)}
        out["per_layer_ms"]["proj_bwd"] = round(bms, 4)
        out["per_layer_ms"]["library_bwd_gemms"] = round(bwd_lib_ms, 4)
    print(json.dumps(out), flush=True)


def bench_read(args, W):
    import torch
    import slotread_hip as RH
    import slotscan_lib as L

    B, T, H, N, D, G, NQ, layers = (W[x] for x in ("B", "T", "H", "N", "D", "G", "NQ", "layers"))
    NB = (T + G - 1) // G
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(3)
    rn = lambda *s: torch.randn(*s, device=dev, generator=gen)
    unit = lambda x: x / x.norm(dim=-1, keepdim=True)
    K = unit(rn(B, NB, H, N, D)).to(torch.bfloat16)
    V = rn(B, NB, H, N, D).to(torch.bfloat16)
    kinv = torch.ones(B, NB, H, N, device=dev)
    valid = torch.ones(B, NB, H, N, device=dev, dtype=torch.bool)
    qs = [unit(rn(B, T, H, NQ, D)).to(torch.bfloat16) for _ in range(layers)]
    scs = [torch.nn.functional.softplus(rn(B, T, H, NQ)) + 1.0 for _ in range(layers)]
    bwd = W.get("backward", False)
    if bwd:
        K.requires_grad_()
        V.requires_grad_()
        for x in qs + scs:
            x.requires_grad_()
        drd = rn(B, T, H, NQ, D).to(torch.bfloat16)

    def step(probe=False):
        if bwd:
            rd = RH.slot_read(qs[0], K, V, kinv, valid, scs[0], G)
            return torch.autograd.grad(rd, (qs[0], K, V, scs[0]), drd)
        with torch.no_grad():
            out = []
            for i in range(layers):
                if probe and i == 0:
                    L.profile(True)
                out.append(RH.slot_read(qs[i], K, V, kinv, valid, scs[i], G))
                if probe and i == 0:
                    L.profile(False)
            return out

    # The forward-only workload times one layer's launch per timed step (a timed launch is dispatched with
    # completion events, so it cannot overlap the launch after it; the layers are identical), the training
    # workload every launch.  Every kernel is also timed on the last warm-up step.
    for i in range(args.warmup):
        if i == args.warmup - 1:
            L.profile(True)
        step()
    torch.cuda.synchronize()
    L.profile(False)
    warm = L.profile_read()
    if bwd:
        L.profile(True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(probe=not bwd)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    L.profile(False)
    prof = L.profile_read()
    if args.copy_calibration:
        copy_calibration(torch.device("cuda:0"))
    ms = (t1 - t0) * 1e3 / args.steps
    tot, cnt = prof["read_fwd"]
    kms = tot / cnt
    by, fl = read_algorithmic(B, T, H, N, D, NQ, layers, NB)
    ach = by / (kms * 1e-3) / 1e9
    out = {
        "metric": "slot-read fan-out tokens/s (6 reader layers, frozen store B64 H6 S192 d128, forward)",
        "value": round(B * T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded GPU generator, seed 3)",
        "config": {"workload": args.workload, "B": B, "T": T, "H": H, "N": N, "D": D, "NQ": NQ, "G": G,
                   "layers": layers, "tokens_per_step": B * T},
        "roofline": {"bound": "hbm", "kernel": "read_fwd", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic(args.workload).get("read_fwd"),
                     "traffic_source": f"profiles/hbm_traffic_{args.workload}.md: committed rocprofv3 FETCH_SIZE and "
                                       "WRITE_SIZE passes, not measured in this run",
                     "algorithmic_bytes_per_launch": by, "avg_launch_ms": round(kms, 4),
                     "mfma_tflops": round(fl / (kms * 1e-3) / 1e12, 1), "mfma_peak_tflops": MFMA_BF16_PEAK_TFLOPS,
                     "mfma_frac": round(fl / (kms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                     "timed_launches": cnt},
        "kernels_ms": {n: round(x / c, 4) for n, (x, c) in (warm or prof).items()},
    }
    if bwd:
        bt, bc = prof["read_bwd"]
        bby = read_bwd_algorithmic(B, T, H, N, D, NQ, NB)
        out["metric"] = "slot-read fwd+bwd tokens/s (one reader layer, training shape G8 NQ2, B64 H6 S192 d128)"
        out["read_bwd_roofline"] = {"achieved": round(bby / (bt / bc * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBPS,
                                    "unit": "GB/s", "frac": round(bby / (bt / bc * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                                    "algorithmic_bytes_per_launch": bby, "avg_launch_ms": round(bt / bc, 4)}
    if not args.no_cpu and not bwd:
        out["cpu_baseline"] = cpu_baseline_read(W)
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="config2", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one 1 GiB device-to-device copy (reads 1 GiB, writes 1 GiB) after the timed "
                         "steps, so HBM byte counters (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE) can be scaled")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the scan has no cross-GPU exchange and this build runs on "
              "single-GPU boxes (every (batch, head) chain is independent, so N GPUs would each run B/N of the "
              "batch)",
              file=sys.stderr)
        sys.exit(2)

    W = WORKLOADS[args.workload]
    if W["kind"] == "read":
        return bench_read(args, W)
    if W["kind"] == "read_out":
        return bench_read_out(args, W)
    if W["kind"] == "stream":
        return bench_stream(args, W)
    if W["kind"] == "window":
        return bench_window(args, W)

    import torch
    import slotkern_hip as KH
    import slotscan_lib as L

    B, T, H, N, D, G = (W[x] for x in ("B", "T", "H", "N", "D", "G"))
    dev = torch.device("cuda:0")
    k, q, v, gate, fr, temp, dkb, dvb, rn = scan_workload_inputs(W, dev)
    NB = (T + G - 1) // G
    inputs = (k, q, v, gate, fr, temp)
    mem = W.get("mem", False)
    soft = W.get("soft", False)
    qb, qg = W.get("qbits", 0), W.get("qgroup", 16)
    kw = dict(G=G, hard=not soft, hard_gate=False, detach_addr=not soft, q=q, occ_bin=True)

    if mem:
        import slotmem_hip as MH
        dkb, dvb = dkb.to(torch.bfloat16), dvb.to(torch.bfloat16)
        dki = rn(B, NB, H, N)

        def step():
            kb, vb, kinv, _valid = KH.kv_scan_mem(k, v, gate, fr, N, temp, bits=qb, group=qg, **kw)
            return torch.autograd.grad((kb, vb, kinv), inputs, (dkb, dvb, dki))

        def step_two_pass():                 # the same outputs through the scan, then the epilogue
            kbuf, vbuf = KH.kv_scan_c(k, v, gate, fr, N, temp, **kw)
            if qb:
                kb, vb, kinv, _valid = MH.quantize_mem(kbuf, vbuf, qb, qg, dtype=torch.bfloat16)
            else:
                kb, vb, kinv, _valid = MH.writer_epilogue(kbuf, vbuf, dtype=torch.bfloat16)
            return torch.autograd.grad((kb, vb, kinv), inputs, (dkb, dvb, dki))
    else:
        def step():
            kb, vb = KH.kv_scan_c(k, v, gate, fr, N, temp, **kw)
            return torch.autograd.grad((kb, vb), inputs, (dkb, dvb))

    # Every kernel is timed on the last warm-up step.  The timed steps time only the dominant kernel: each
    # timed launch costs the stream a few microseconds, which would otherwise inflate the step time.
    for i in range(args.warmup):
        if i == args.warmup - 1:
            L.profile(True)
        step()
    torch.cuda.synchronize()
    L.profile(False)
    warm = L.profile_read()
    per_kernel_bytes, step_bytes = algorithmic_bytes(B, T, H, N, D, G, mem=mem, soft=soft, memq=bool(qb))
    dom = max((n for n in warm if n in per_kernel_bytes), key=lambda n: warm[n][0] / warm[n][1], default=None)
    L.profile(True, kernels=None if dom is None else [dom])
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    L.profile(False)
    prof = L.profile_read()
    if not warm:                                          # no warm-up step: every kernel was timed above
        warm = {n: (tot / args.steps, cnt / args.steps) for n, (tot, cnt) in prof.items()}
        dom = max((n for n in warm if n in per_kernel_bytes), key=lambda n: warm[n][0] / warm[n][1])
    if args.copy_calibration:
        copy_calibration(dev)
    ms = (t1 - t0) * 1e3 / args.steps
    two_pass_ms = None
    if mem:
        for _ in range(args.warmup):
            step_two_pass()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        for _ in range(args.steps):
            step_two_pass()
        torch.cuda.synchronize()
        two_pass_ms = (time.perf_counter() - t2) * 1e3 / args.steps
    tokens = B * T
    kern_ms = {name: tot / cnt for name, (tot, cnt) in warm.items()}          # one step, every kernel
    # the forward runs as a chunk pipeline (several launches per step): per-launch bytes are the per-step
    # bytes over the launches per step
    per_step = {name: cnt for name, (tot, cnt) in warm.items()}
    launch_bytes = {n: int(per_kernel_bytes[n] / per_step[n]) for n in per_kernel_bytes if n in per_step}
    dom_tot, dom_cnt = prof[dom]
    dom_ms = dom_tot / dom_cnt                                                 # over the timed steps
    ach = launch_bytes[dom] / (dom_ms * 1e-3) / 1e9
    traffic = measured_traffic(args.workload).get(dom)
    out = {
        "metric": (f"slot-scan + writer epilogue{f' (storage quantiser, {qb} bits, group {qg})' if qb else ''} "
                   f"fwd+bwd tokens/s at B{B} T{T} H{H} S{N} d{D}" if mem else
                   "slot-scan fwd+bwd tokens/s at B64 T1024 H6 S192 d128; % HBM/MFMA roofline"
                   if args.workload == "config2" else f"slot-scan fwd+bwd tokens/s at B{B} T{T} H{H} S{N} d{D}"),
        "value": round(tokens / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 state, bf16 tokens" + (", bf16 copies" if mem else ""),
        "data": f"synthetic (seeded GPU generator, seed {W.get('seed', 1)})",
        "config": {"workload": args.workload, "B": B, "T": T, "H": H, "N": N, "D": D, "G": G, "temp": 16.0,
                   "mode": ("soft address, attached address gradient" if soft else "hard, detach_addr") +
                           ", occ_bin, per-token fr", "tokens_per_step": tokens},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "traffic_source": (f"profiles/hbm_traffic_{args.workload}.md: committed rocprofv3 FETCH_SIZE and "
                                        "WRITE_SIZE passes, not measured in this run") if traffic else None,
                     "algorithmic_bytes_per_launch": launch_bytes[dom],
                     "avg_launch_ms": round(dom_ms, 4), "timed_launches": dom_cnt},
        "step_roofline": {"algorithmic_bytes": step_bytes,
                          "achieved": round(step_bytes / (ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBPS,
                          "unit": "GB/s", "frac": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)},
        "kernels_ms": {n: round(x, 4) for n, x in kern_ms.items()},          # per launch, last warm-up step
        "launches_per_step": {n: round(x, 2) for n, x in per_step.items()},
    }
    if mem:
        out["two_pass_ms_per_step"] = round(two_pass_ms, 4)
        out["speedup_vs_two_pass"] = round(two_pass_ms / ms, 3)
    out["hbm_measured"] = hbm_ceilings(dev)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(W)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
