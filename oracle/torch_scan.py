"""Independent torch statement of the slot-scan forward -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module: the tests use it
(float64 on the CPU) to obtain gradients by autograd, which pins the numpy oracle's hand-written backward
(autograd derives the adjoints from this forward, scan_oracle.py writes them out by hand); bench.py times it
in float32 with autograd on the host's cores as the CPU baseline.  The product path never imports it.

Follows /root/reference/gqa25/slotkern_kv.py:66-123 (the reference's own torch loop), with teacher
forcing added so that a hard-address run can follow a given address sequence."""
import torch

NEG = -1e30


def scan_torch(k, v, gate, fr, N, temp, G=1, hard=False, hard_gate=False, eps=1e-4, detach_addr=False, q=None,
               pin=False, occ_bin=False, teacher=None):
    B, T, H, DK = k.shape
    DV = v.shape[-1]
    K = k.new_zeros(B, H, N, DK)
    V = v.new_zeros(B, H, N, DV)
    o = k.new_zeros(B, H, N)
    kb, vb = [], []
    for t in range(T):
        if t % G == 0:
            kb.append(K)
            vb.append(V)
        kt = k[:, t]
        qt = kt if q is None else q[:, t]
        Ka = K.detach() if detach_addr else K
        knorm = Ka.norm(dim=-1)
        kn = Ka / knorm.clamp_min(1e-6).unsqueeze(-1)
        qn = qt / qt.norm(dim=-1, keepdim=True).clamp_min(1e-6)
        s = (kn * qn.unsqueeze(2)).sum(-1) * temp
        if pin:
            s = torch.where(knorm < 1e-6, torch.zeros_like(s), s)
        frt = fr[:, t].unsqueeze(-1) if fr.dim() == 3 else fr
        occ = (o >= eps).to(o.dtype) if occ_bin else o
        z = s - frt * occ
        empty = o < eps
        keep = (~empty) | (empty & (empty.to(torch.int64).cumsum(-1) == 1))
        z = z.masked_fill(~keep, NEG)
        a = torch.softmax(z, -1)
        if hard:
            idx = z.argmax(-1) if teacher is None else teacher[:, t]
            oh = torch.nn.functional.one_hot(idx, N).to(a.dtype)
            a = oh + a - a.detach()
        g = gate[:, t]
        if hard_gate:
            g = (g > 0.5).to(g.dtype) + g - g.detach()
        w = (g.unsqueeze(-1) * a).unsqueeze(-1)
        K = (1 - w) * K + w * kt.unsqueeze(2)
        V = (1 - w) * V + w * v[:, t].unsqueeze(2)
        o = (1 - w[..., 0]) * o + w[..., 0]
    return torch.stack(kb, 1), torch.stack(vb, 1)


def read_torch(qh, kbuf, buf, kinv, valid, scale):
    """The kernel-level core of SharedMixer._read (/root/reference/gqa25/memlm_sh.py:383-395) in torch, in the
    inputs' dtype: per (b, block, head), qh (B,NB,H,M,DK) unit queries against that block's copy kbuf
    (B,NB,H,N,DK), scores times kinv (B,NB,H,N) and the per-query multiplier scale (B,NB,H,M), the softmax
    over the valid rows (an all-invalid block reads 0), then the value contraction with buf (B,NB,H,N,DV)."""
    sc = torch.einsum("bjhmd,bjhnd->bjhmn", qh, kbuf) * kinv.unsqueeze(-2) * scale.unsqueeze(-1)
    att = torch.nan_to_num(torch.softmax(sc.masked_fill(~valid.unsqueeze(-2), float("-inf")), -1))
    return torch.einsum("bjhmn,bjhnv->bjhmv", att, buf)
