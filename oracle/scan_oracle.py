"""CPU oracle for the key-matched slot scan -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as
the checker (or as the timed CPU baseline).  The product path (the HIP library and its Python wrapper)
never imports it.

This is a numpy restatement of the reference's torch scan `_ref_scan_kv_impl`
(/root/reference/gqa25/slotkern_kv.py:66-123) and of the adjoint list that its autograd produces
(documented by the reference at gqa25/slotkern_kvt.py:157-171, with the stride-G gradient entry of
gqa25/slotkern_kvg.py:165-168, the per-token free-row preference of slotkern_kvg.py:178-181 and the
occupancy-indicator rule of slotkern_kvg.py:193-196).  It runs in float64 by default (dtype=np.float32
gives the fp32 CPU baseline).

Per (b, h) chain the state is K (N, DK), V (N, DV), o (N), all zero (or a carried state).  For t = 0..T-1:
  1. if t % G == 0: emit (K, V, o) -- the PRE-write state (slotkern_kv.py:76-77)
  2. s_n = temp * <K_n / max(|K_n|, 1e-6), q_t / max(|q_t|, 1e-6)>          (slotkern_kv.py:85-87)
     pin: s_n = 0 where |K_n| < 1e-6                                          (slotkern_kv.py:100-101)
  3. z_n = s_n - fr_t * (occ_bin ? [o_n >= eps] : o_n)                        (slotkern_kv.py:104-105)
  4. only occupied rows and the FIRST free row compete (others get -1e30)     (slotkern_kv.py:46-51, 106)
  5. a = softmax(z); hard: a = onehot(argmax z), first maximum wins            (slotkern_kv.py:107-110)
  6. g = gate_t (hard_gate: [g > 0.5]); w = g * a                              (slotkern_kv.py:111-114)
  7. K <- (1-w)K + w k_t ; V <- (1-w)V + w v_t ; o <- (1-w)o + w              (slotkern_kv.py:118-120)

Pinning (how each function here is checked -- tests/test_oracle_scan.py):
  scan_forward   closed forms (T=1 write, g=1 copy, g=0 no-op), first-free fill order, tie-break to the
                 lowest index, stride-G copies == per-step state, constant per-token fr == scalar fr,
                 chunked scan with carried state == one-shot scan, soft-mode empties-as-one, and an
                 independent scalar pure-Python loop on tiny inputs.
  scan_backward  torch autograd (float64) of an independent torch statement of the forward in every mode
                 (hard/soft, detach/attached, occ_bin, per-token fr, hard_gate, pin, G not dividing T),
                 plus central finite differences in soft mode.
"""
import numpy as np

NEG = -1e30          # masked score, as the reference (slotkern_kv.py:43): not -inf, so softmax never NaNs
NORM_EPS = 1e-6      # clamp on |K| and |q| (slotkern_kv.py:85-86)


def _first_empty_mask(o, eps):
    """True on occupied rows and on the lowest-index free row (slotkern_kv.py:46-51)."""
    empty = o < eps
    first = empty & (np.cumsum(empty, axis=-1) == 1)
    return (~empty) | first


def _softmax(z):
    m = z.max(-1, keepdims=True)
    e = np.exp(z - m)
    return e / e.sum(-1, keepdims=True)


def _fr_at(fr, t):
    """fr is a scalar (shape () or (1,)) or per-token (B, T, H) (slotkern_kv.py:103)."""
    fr = np.asarray(fr)
    if fr.ndim == 3:
        return fr[:, t][..., None]
    return fr.reshape(-1)[0]


def _step_scores(K, o, qt, temp, frt, eps, occ_bin, pin):
    """Scores of one step for every chain: returns (s_raw, s, z_masked, okrow, knorm, kinv, kn, qnorm, qinv, qn, occ)."""
    knorm = np.sqrt((K * K).sum(-1))
    kinv = 1.0 / np.maximum(knorm, NORM_EPS)
    kn = K * kinv[..., None]
    qnorm = np.sqrt((qt * qt).sum(-1))
    qinv = 1.0 / np.maximum(qnorm, NORM_EPS)
    qn = qt * qinv[..., None]
    s_raw = np.einsum("bhnd,bhd->bhn", kn, qn) * temp
    s = np.where(knorm < NORM_EPS, 0.0, s_raw) if pin else s_raw
    occ = (o >= eps).astype(K.dtype) if occ_bin else o
    z = s - frt * occ
    okrow = _first_empty_mask(o, eps)
    zm = np.where(okrow, z, NEG)
    return s_raw, s, zm, okrow, knorm, kinv, kn, qnorm, qinv, qn, occ


def _top2_margin(zm, okrow):
    """z(best) - z(second best) over the competing rows; +inf when only one row competes."""
    zz = np.where(okrow, zm, -np.inf)
    part = -np.sort(-zz, axis=-1)
    return part[..., 0] - part[..., 1]


def scan_forward(k, v, gate, fr, N, temp, G=1, hard=False, hard_gate=False, eps=1e-4, detach_addr=False,
                 q=None, pin=False, occ_bin=False, state=None, teacher=None, dtype=np.float64):
    """Forward scan.  k (B,T,H,DK), v (B,T,H,DV), gate (B,T,H), fr scalar or (B,T,H), temp scalar.
    Returns (kbuf, vbuf, info): kbuf (B,NB,H,N,DK), vbuf (B,NB,H,N,DV) the PRE-write state every G steps,
    info = dict(obuf, am, margin, agree, kfin, vfin, ofin).

    detach_addr changes nothing in the forward (slotkern_kv.py:79-84).
    state = (K0, V0, o0) with shapes (B,H,N,DK), (B,H,N,DV), (B,H,N) carries a previous chunk's final state
    (the reference has no state input; this is the carry that chunked streaming needs).
    teacher (B,T,H) int: in hard mode, write to these rows instead of the argmax (teacher forcing) and record
    in info['agree'] whether the argmax agreed and in info['margin'] z(argmax) - z(teacher row)."""
    k = np.asarray(k, dtype)
    v = np.asarray(v, dtype)
    gate = np.asarray(gate, dtype)
    q = k if q is None else np.asarray(q, dtype)
    fr = np.asarray(fr, dtype)
    temp = dtype(temp) if np.ndim(temp) == 0 else np.asarray(temp, dtype).reshape(-1)[0]
    B, T, H, DK = k.shape
    DV = v.shape[-1]
    NB = (T + G - 1) // G
    if state is None:
        K = np.zeros((B, H, N, DK), dtype)
        V = np.zeros((B, H, N, DV), dtype)
        o = np.zeros((B, H, N), dtype)
    else:
        K, V, o = (np.array(x, dtype) for x in state)
    kbuf = np.empty((B, NB, H, N, DK), dtype)
    vbuf = np.empty((B, NB, H, N, DV), dtype)
    obuf = np.empty((B, NB, H, N), dtype)
    am = np.zeros((B, T, H), np.int64)
    margin = np.zeros((B, T, H), np.float64)
    agree = np.ones((B, T, H), bool)
    for t in range(T):
        if t % G == 0:
            kbuf[:, t // G] = K
            vbuf[:, t // G] = V
            obuf[:, t // G] = o
        kt = k[:, t]
        qt = q[:, t]
        _, _, zm, okrow, *_ = _step_scores(K, o, qt, temp, _fr_at(fr, t), eps, occ_bin, pin)
        if hard:
            best = zm.argmax(-1)                     # numpy argmax returns the FIRST maximum
            if teacher is None:
                idx = best
                margin[:, t] = _top2_margin(zm, okrow)
            else:
                idx = np.asarray(teacher)[:, t].astype(np.int64)
                zb = np.take_along_axis(zm, best[..., None], -1)[..., 0]
                zt = np.take_along_axis(zm, idx[..., None], -1)[..., 0]
                agree[:, t] = idx == best
                margin[:, t] = zb - zt
            am[:, t] = idx
            a = np.zeros_like(zm)
            np.put_along_axis(a, idx[..., None], 1.0, -1)
        else:
            a = _softmax(zm)
            am[:, t] = zm.argmax(-1)
        g = gate[:, t]
        if hard_gate:
            g = (g > 0.5).astype(dtype)
        w = g[..., None] * a
        K = (1 - w)[..., None] * K + w[..., None] * kt[:, :, None, :]
        V = (1 - w)[..., None] * V + w[..., None] * v[:, t][:, :, None, :]
        o = (1 - w) * o + w
    info = dict(obuf=obuf, am=am, margin=margin, agree=agree, kfin=K, vfin=V, ofin=o)
    return kbuf, vbuf, info


def scan_backward(k, v, gate, fr, N, temp, kbuf, vbuf, info, dkbuf, dvbuf, G=1, hard=False, hard_gate=False,
                  eps=1e-4, detach_addr=False, q=None, pin=False, occ_bin=False, dtype=np.float64):
    """Explicit reverse pass of scan_forward (which produced kbuf, vbuf, info).

    Each stride-G segment is replayed forward from its emitted copy (kbuf/vbuf/obuf) -- in hard mode along
    info['am'], the rows the forward actually wrote -- and then walked backward with the adjoints of
    slotkern_kvt.py:157-171:
        dw_n  = <k_t - K_n, dK'_n> + <v_t - V_n, dV'_n> + (1 - o_n) do'_n
        dk_t  = sum_n w_n dK'_n,  dv_t = sum_n w_n dV'_n,  dgate_t = sum_n a_n dw_n
        dz_n  = a_s,n (g dw_n - sum_m a_s,m g dw_m)      (a_s the soft address; masked rows 0)
        dfr_t = -sum_n occ_n dz_n,  dtemp += sum_n dz_n s_n / temp
        dq_t  = qinv (dqn - qn <qn, dqn>)  (qinv dqn where |q| < 1e-6),  dqn = temp sum_n dz_n kn_n
        attached address only: dK_n += kinv (dkn - kn <kn, dkn>) (dkn / 1e-6 where |K_n| < 1e-6)
        carry: dK = (1-w) dK' (+ dkbuf at t % G == 0), dV likewise, do = (1-w) do' - fr dz (occ_bin: no -fr dz)
    Returns dict(dk, dq, dv, dgate, dfr, dtemp); dq is the search-query gradient (autograd adds it to dk when
    the caller passed q=None, i.e. q is k)."""
    k = np.asarray(k, dtype)
    v = np.asarray(v, dtype)
    gate = np.asarray(gate, dtype)
    q = k if q is None else np.asarray(q, dtype)
    fr = np.asarray(fr, dtype)
    frt_mode = fr.ndim == 3
    temp = dtype(temp) if np.ndim(temp) == 0 else np.asarray(temp, dtype).reshape(-1)[0]
    B, T, H, DK = k.shape
    DV = v.shape[-1]
    NB = (T + G - 1) // G
    obuf = info["obuf"]
    am = info["am"]
    dkbuf = np.asarray(dkbuf, dtype)
    dvbuf = np.asarray(dvbuf, dtype)
    dk = np.zeros_like(k)
    dq = np.zeros_like(q)
    dv = np.zeros_like(v)
    dgate = np.zeros_like(gate)
    dfr = np.zeros((B, T, H), dtype) if frt_mode else np.zeros((), dtype)
    dtemp = 0.0
    dK = np.zeros((B, H, N, DK), dtype)
    dV = np.zeros((B, H, N, DV), dtype)
    do = np.zeros((B, H, N), dtype)
    for tb in range(NB - 1, -1, -1):
        t0, t1 = tb * G, min(tb * G + G, T)
        K, V, o = kbuf[:, tb].astype(dtype), vbuf[:, tb].astype(dtype), obuf[:, tb].astype(dtype)
        steps = []
        for t in range(t0, t1):                     # replay the segment, keeping each step's pre-write state
            kt, qt = k[:, t], q[:, t]
            frt = _fr_at(fr, t)
            s_raw, s, zm, okrow, knorm, kinv, kn, qnorm, qinv, qn, occ = _step_scores(K, o, qt, temp, frt, eps,
                                                                                  occ_bin, pin)
            a_s = _softmax(zm)
            if hard:
                a = np.zeros_like(zm)
                np.put_along_axis(a, am[:, t][..., None], 1.0, -1)
            else:
                a = a_s
            g = gate[:, t]
            if hard_gate:
                g = (g > 0.5).astype(dtype)
            w = g[..., None] * a
            steps.append((K, V, o, s_raw, okrow, knorm, kinv, kn, qnorm, qinv, qn, occ, a_s, a, g, w, frt))
            K = (1 - w)[..., None] * K + w[..., None] * kt[:, :, None, :]
            V = (1 - w)[..., None] * V + w[..., None] * v[:, t][:, :, None, :]
            o = (1 - w) * o + w
        for t in range(t1 - 1, t0 - 1, -1):
            (K, V, o, s_raw, okrow, knorm, kinv, kn, qnorm, qinv, qn, occ, a_s, a, g, w, frt) = steps[t - t0]
            kt, vt = k[:, t], v[:, t]
            dw = (((kt[:, :, None, :] - K) * dK).sum(-1) + ((vt[:, :, None, :] - V) * dV).sum(-1)
                  + (1 - o) * do)
            dk[:, t] = (w[..., None] * dK).sum(2)
            dv[:, t] = (w[..., None] * dV).sum(2)
            dgate[:, t] = (a * dw).sum(-1)
            da = g[..., None] * dw
            dz = a_s * (da - (a_s * da).sum(-1, keepdims=True))
            dz = np.where(okrow, dz, 0.0)
            ds = np.where(knorm < NORM_EPS, 0.0, dz) if pin else dz
            if frt_mode:
                dfr[:, t] = -(occ * dz).sum(-1)
            else:
                dfr = dfr - (occ * dz).sum()
            dtemp += float((ds * s_raw).sum() / temp)
            dkn = temp * ds[..., None] * qn[:, :, None, :]
            dqn = temp * (ds[..., None] * kn).sum(2)
            prjq = (dqn * qn).sum(-1, keepdims=True)
            dq[:, t] = np.where((qnorm < NORM_EPS)[..., None], qinv[..., None] * dqn,
                                qinv[..., None] * (dqn - qn * prjq))
            dKm = 0.0
            if not detach_addr:
                prj = (dkn * kn).sum(-1, keepdims=True)
                dKm = np.where((knorm < NORM_EPS)[..., None], kinv[..., None] * dkn,
                               kinv[..., None] * (dkn - kn * prj))
            omw = 1 - w
            dK = omw[..., None] * dK + dKm
            dV = omw[..., None] * dV
            do = omw * do if occ_bin else omw * do - frt * dz
            if t == t0:                              # the emitted copy is the pre-write state of step t0
                dK = dK + dkbuf[:, tb]
                dV = dV + dvbuf[:, tb]
    if not frt_mode:
        dfr = np.asarray(dfr).reshape(1)
    return dict(dk=dk, dq=dq, dv=dv, dgate=dgate, dfr=dfr, dtemp=np.asarray(dtemp, dtype))
