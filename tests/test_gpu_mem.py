"""GPU parity of the writer epilogue and storage quantiser (slotmem_hip through libslotscan.so) against the
oracle (oracle/read_oracle.py: writer_epilogue, fq, fq_ste, quantize_mem) and against torch autograd of the
reference's own expressions (memlm_sh.py:221-234, 474-475) for the backward.

Bar: bf16 / fp32 copies, codes, scales and validity bit-exact (the same float32 operations in the same
order per element); kinv within 2e-6 relative (the row sum's order and rsqrt's last bit differ from
torch's); gradients within 1e-5 relative to max."""
import numpy as np
import pytest
import torch

from oracle import read_oracle as RO

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import slotmem_hip as MH

DEV = "cuda"


def _copies(shape, seed, zero_rows=0.2, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(*shape, generator=g) * scale
    v = torch.randn(*shape, generator=g) * scale
    z = torch.rand(shape[:-1], generator=g) < zero_rows          # never-written rows are exactly zero
    k[z] = 0.0
    v[z] = 0.0
    return k, v


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_writer_epilogue_matches_oracle(D, dtype):
    k, v = _copies((3, 5, 2, 37, D), 1)
    print(f"epilogue D{D} {dtype}", flush=True)
    kb, vb, kinv, valid = MH.writer_epilogue(k.to(DEV), v.to(DEV), dtype=dtype)
    torch.cuda.synchronize()
    assert torch.equal(kb.cpu(), k.to(dtype)) and torch.equal(vb.cpu(), v.to(dtype))
    ki, va = RO.writer_epilogue(k.numpy())
    assert np.array_equal(valid.cpu().numpy(), va)
    np.testing.assert_allclose(kinv.cpu().numpy(), ki, rtol=2e-6)


@pytest.mark.parametrize("bits,group,D", [(3, 16, 128), (2, 4, 64), (4, 32, 128), (8, 128, 128), (8, 64, 64), (3, 8, 64)])
def test_quantize_mem_matches_oracle(bits, group, D):
    k, v = _copies((2, 4, 3, 29, D), 2, scale=2.5)
    print(f"quantize bits{bits} group{group} D{D}", flush=True)
    kq, vq, kinv, valid = MH.quantize_mem(k.to(DEV), v.to(DEV), bits, group, dtype=torch.float32)
    torch.cuda.synchronize()
    okq, ovq, oki, ova = RO.quantize_mem(k.numpy(), v.numpy(), bits, group)
    np.testing.assert_array_equal(kq.cpu().numpy(), okq)
    np.testing.assert_array_equal(vq.cpu().numpy(), ovq)
    assert np.array_equal(valid.cpu().numpy(), ova)
    np.testing.assert_allclose(kinv.cpu().numpy(), oki, rtol=2e-6)
    kb, vb, _, _ = MH.quantize_mem(k.to(DEV), v.to(DEV), bits, group)           # bf16 copies: the cast of :471
    assert torch.equal(kb.cpu(), torch.from_numpy(okq).to(torch.bfloat16))
    assert torch.equal(vb.cpu(), torch.from_numpy(ovq).to(torch.bfloat16))


@pytest.mark.parametrize("bits,group,D", [(8, 128, 128), (3, 16, 128), (4, 4, 64)])
def test_codes_and_scales_match_oracle(bits, group, D):
    x, _ = _copies((3, 7, 41, D), 3, scale=4.0)
    codes, scales = MH.fq_codes(x.to(DEV), bits, group)
    torch.cuda.synchronize()
    val, code, s = RO.fq(x.numpy(), bits, group)
    np.testing.assert_array_equal(codes.cpu().numpy(), code)
    a = np.abs(x.numpy().reshape(*x.shape[:-1], D // group, group)).max(-1)
    np.testing.assert_array_equal(scales.cpu().numpy(), np.where(a > 0, s, 0.0).astype(np.float32))
    np.testing.assert_array_equal(MH.fq_decode(codes, scales, group).cpu().numpy(), val)


def _torch_epilogue_grad(k, v, bits, group, dkb, dvb, dkinv):
    """Autograd of the reference's expressions in float64 (memlm_sh.py:221-234, 474-475)."""
    kk = k.double().requires_grad_()
    vv = v.double().requires_grad_()
    if bits:
        def fq(x):
            sh = x.shape
            xg = x.reshape(*sh[:-1], sh[-1] // group, group)
            a = xg.abs().amax(-1, keepdim=True)
            half = 2 ** (bits - 1)
            s = (a / half).clamp_min(1e-30)
            q = (torch.floor(xg / s).clamp(-half, half - 1) + 0.5) * s
            q = torch.where(a > 0, q, torch.zeros_like(q)).reshape(sh)
            return x + (q - x).detach()
        kq, vq = fq(kk), fq(vv)
    else:
        kq, vq = kk, vv
    nsq = kq.pow(2).sum(-1)
    kinv = torch.rsqrt(nsq.clamp_min(1e-12))
    (kq * dkb.double()).sum().backward(retain_graph=True)
    (vq * dvb.double()).sum().backward(retain_graph=True)
    (kinv * dkinv.double()).sum().backward()
    return kk.grad, vv.grad


@pytest.mark.parametrize("bits,group", [(0, 0), (3, 16)])
def test_epilogue_backward_matches_torch_autograd(bits, group):
    D = 128
    k, v = _copies((2, 3, 2, 33, D), 4)
    g = torch.Generator().manual_seed(5)
    dkb = torch.randn(k.shape, generator=g).to(torch.bfloat16)
    dvb = torch.randn(k.shape, generator=g).to(torch.bfloat16)
    dkinv = torch.randn(k.shape[:-1], generator=g)
    kk = k.to(DEV).requires_grad_()
    vv = v.to(DEV).requires_grad_()
    kb, vb, kinv, valid = MH.quantize_mem(kk, vv, bits, group) if bits else MH.writer_epilogue(kk, vv)
    torch.autograd.backward((kb, vb, kinv), (dkb.to(DEV), dvb.to(DEV), dkinv.to(DEV)))
    torch.cuda.synchronize()
    rk, rv = _torch_epilogue_grad(k, v, bits, group, dkb, dvb, dkinv)
    for got, ref in ((kk.grad, rk), (vv.grad, rv)):
        got = got.double().cpu()
        err = (got - ref).abs().max().item() / max(ref.abs().max().item(), 1e-30)
        print(f"   grad rel err {err:.2e}", flush=True)
        assert err < 1e-5
