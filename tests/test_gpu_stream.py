"""GPU parity of the long-context streaming scan with the slot state carried across calls.

Config 5 is B=8, H=6, N=192, D=128, G=8, forward only, in 1024-token calls whose (K, V, o) state carries
over, each call's snapshot copies emitted as int8 codes with one fp32 absmax scale per row (the storage
quantiser at bits 8, group D, memlm_sh.py:221-228).  A 1024-token call runs the forward's 8-chunk two-stream
pipeline, so the carried state enters its chunk 0 and crosses its seven inner chunk boundaries.

Three consecutive calls at config 5's full shape (inputs drawn as bench.py's config 5, 3,072 tokens per
row), through both streaming entry points on the same state chain:
  - kv_scan_stream_q, the fused path (slotscan_fwd_codes: the chain stores no snapshots, the row replay
    rebuilds every key and value row and emits its codes);
  - kv_scan_stream, the fp32 snapshots and the address log of the same calls.
Checks, every call:
  1. both paths carry bitwise the same state out (so they took the same addresses);
  2. the fused codes and scales are bitwise the two-pass quantiser's (fq_codes) over the whole launch, and
     on the sampled rows bitwise the oracle quantiser's (oracle fq in float32) of the same fp32 snapshots;
  3. on both batch ends (b = 0 and b = 7), every head: the fp64 oracle, teacher-forced on the GPU's
     addresses, with its OWN state carried from call to call (oracle.scan_forward(state=...)) -- addresses
     bit-exact (zero flips), final occupancy masks identical, snapshots and the carried (K, V, o) within 1e-5
     relative to max.
The reference has no carry (it restarts from zero per call, memlm_sh.py:676); the carry is this build's
streaming contract."""
import numpy as np
import pytest
import torch

import bench
from oracle import read_oracle as RO
from oracle import scan_oracle as SO
from scan_inputs import assert_no_flips

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import slotkern_hip as KH
    import slotmem_hip as MH

TEMP = 16.0


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def _np(x):
    return x.detach().double().cpu().numpy()


def _fp32_call(k, q, v, g, fr, N, G, state):
    """kv_scan_stream's forward of one call with its address log: (kbuf, vbuf, am, (kfin, vfin, ofin))."""
    dt, k_, q_, v_, g_, fr_, frt, temp_ = KH._prep(k, q, v, g, fr, torch.tensor(TEMP, device=k.device), False)
    out = KH._fwd(k_, q_, v_, g_, fr_, frt, temp_, N, G, 1e-4, True, dt, logs=False, state=state)
    return out[0], out[1], out[2], (out[7], out[8], out[9])


def test_config5_stream_carried_state_matches_oracle():
    W = dict(bench.WORKLOADS["config5"])
    B, H, N, D, G, C = (W[x] for x in ("B", "H", "N", "D", "G", "chunk"))
    calls = 3
    dev = torch.device("cuda:0")
    k, q, v, gate, fr = bench.stream_workload_inputs(W, calls * C, dev)
    bs = [0, B - 1]                                   # both batch ends, every head
    ost = None                                        # the oracle's own carried state (fp64), sampled rows
    stq = st = None
    for c in range(calls):
        sl = slice(c * C, (c + 1) * C)
        print(f"config5 stream call {c}: B{B} T{C} H{H} N{N} D{D} G{G}", flush=True)
        ins = (k[:, sl], v[:, sl], gate[:, sl], fr[:, sl])
        (kc, ks), (vc, vs), stq = KH.kv_scan_stream_q(*ins, N, TEMP, G=G, q=q[:, sl], occ_bin=True, state=stq,
                                                      bits=8)
        kbuf, vbuf, am, st = _fp32_call(k[:, sl], q[:, sl], v[:, sl], gate[:, sl], fr[:, sl], N, G, st)
        torch.cuda.synchronize()
        # 1. the same state chain
        for x, y in zip(stq, st):
            assert torch.equal(x, y), f"call {c}: fused and fp32 paths carry different states"
        # 2. codes and scales: bitwise the two-pass quantiser's, whole launch
        assert kc.dtype == torch.int8 and kc.shape == (B, C // G, H, N, D) and ks.shape == (B, C // G, H, N, 1)
        for (cd, sc), x in (((kc, ks), kbuf), ((vc, vs), vbuf)):
            c2, s2 = MH.fq_codes(x, 8, D)
            assert torch.equal(cd, c2) and torch.equal(sc, s2), f"call {c}: fused codes differ from the two-pass"
        # ... and the oracle quantiser's on the sampled rows (scale 0 where a row is all zero)
        for (cd, sc), x in (((kc, ks), kbuf), ((vc, vs), vbuf)):
            xs = x[bs].cpu().numpy()
            _, ocode, oscale = RO.fq(xs, 8, D)
            oscale = np.where(np.abs(xs).max(-1, keepdims=True) > 0, oscale, 0.0).astype(np.float32)
            np.testing.assert_array_equal(cd[bs].cpu().numpy(), ocode)
            np.testing.assert_array_equal(sc[bs].cpu().numpy(), oscale)
        # 3. the fp64 oracle, teacher-forced, its own state carried
        kn, qn, vn, gn, frn = (_np(x[bs][:, sl]) for x in (k, q, v, gate, fr))
        okb, ovb, info = SO.scan_forward(kn, vn, gn, frn, N, TEMP, G=G, hard=True, eps=1e-4, detach_addr=True,
                                         q=qn, occ_bin=True, state=ost,
                                         teacher=am[bs].cpu().numpy().astype(np.int64))
        flips = assert_no_flips(info)
        ost = (info["kfin"], info["vfin"], info["ofin"])
        kf, vf, of = (x.reshape(B, H, N, -1)[bs].double().cpu().numpy() for x in st)
        of = of[..., 0]
        assert np.array_equal(of >= 1e-4, info["ofin"] >= 1e-4), f"call {c}: occupancy masks differ"
        errs = {"kbuf": _rel(kbuf[bs].cpu(), okb), "vbuf": _rel(vbuf[bs].cpu(), ovb),
                "kfin": _rel(kf, info["kfin"]), "vfin": _rel(vf, info["vfin"]), "ofin": _rel(of, info["ofin"])}
        print("   rel err vs fp64 oracle:", {n: f"{e:.1e}" for n, e in errs.items()}, "flips:", flips, flush=True)
        for n, e in errs.items():
            assert e < 1e-5, f"call {c}: {n} rel err {e:.3e}"
