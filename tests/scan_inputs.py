"""Seeded synthetic inputs for the slot scan, drawn on the CPU so every machine sees the same numbers.

Draw order (fixed): k, q, v, gate logits, fr, read-sharpness logits, upstream gradients.  Distributions
follow the benchmark configurations: k, q, v ~ N(0,1) (k and q optionally L2-normalised), gate =
sigmoid(N(0, gate_sd)), per-token fr ~ U[0, 2) (the reference's training-setting tests draw it so,
kvu/test_cuda.py:27), temp = 16 (memlm_sh.py:298), upstream gradients ~ N(0,1)."""
import numpy as np
import torch


def scan_inputs(B, T, H, D, seed, normalise=True, sep_q=True, frt=True, gate_sd=1.0, gate_mix=False,
                dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen, dtype=torch.float32)
    k = r(B, T, H, D)
    q = r(B, T, H, D) if sep_q else None
    v = r(B, T, H, D)
    if normalise:
        k = k / k.norm(dim=-1, keepdim=True)
        if q is not None:
            q = q / q.norm(dim=-1, keepdim=True)
    g = torch.sigmoid(r(B, T, H) * gate_sd)
    if gate_mix:                               # exact zeros (15%) and ones (8%) as in kvu/test_cuda.py:24-26
        m = torch.rand(B, T, H, generator=gen)
        g = torch.where(m < 0.15, torch.zeros_like(g), torch.where(m > 0.92, torch.ones_like(g), g))
    fr = torch.rand(B, T, H, generator=gen) * 2 if frt else torch.tensor([1.5])
    if dtype != torch.float32:
        k = k.to(dtype)
        v = v.to(dtype)
        q = None if q is None else q.to(dtype)
    return k, q, v, g, fr


def upstream(shape, seed):
    gen = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=gen), torch.randn(*shape, generator=gen)


def np64(x):
    return None if x is None else x.detach().double().cpu().numpy()


def assert_no_flips(info):
    """Slot addresses bit-exact: the GPU's row equals the fp64 oracle's own argmax at every step (the
    reference's acceptance is "rows differing == 0", kvu/test_cuda.py:62).  On failure the message gives the
    count and the worst fp64 margin z(argmax) - z(GPU row), so a genuine near-tie on a new seed (|margin|
    far below what fp32 scores resolve) can be told apart from a wrong address."""
    bad = ~info["agree"]
    n = int(bad.sum())
    if n:
        worst = float(np.abs(info["margin"][bad]).max())
        raise AssertionError(f"{n} address disagreements with the fp64 oracle, worst fp64 margin {worst:.3e}")
    return n
