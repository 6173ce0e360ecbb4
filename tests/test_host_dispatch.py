"""CPU checks of the scan's mode routing (slotkern_hip): which calls run the row-sparse kernels, which the
general-mode kernels, and which are refused -- the reference's split (slotkern_cuda.py:536-543: hard +
detached address with DK == DV on its CUDA kernels, everything else on its Triton scan).  No GPU work."""
import pytest
import torch

import slotkern_hip as KH


@pytest.mark.parametrize("hard,detach,DK,DV,N,row_sparse,general", [
    (True, True, 128, 128, 192, True, True),
    (True, True, 64, 64, 40, True, True),
    (False, True, 128, 128, 192, False, True),       # soft address
    (True, False, 128, 128, 192, False, True),       # attached address gradient
    (False, False, 64, 128, 100, False, True),       # the reference's defaults with DK != DV
    (True, True, 64, 128, 100, False, True),         # DK != DV: general kernels even in the hard mode
    (True, True, 96, 96, 64, False, False),          # unsupported head size
    (False, False, 128, 128, 193, False, False),     # too many slots
])
def test_mode_routing(hard, detach, DK, DV, N, row_sparse, general):
    assert (KH._unsupported(hard, detach, DK, DV, N) is None) == row_sparse
    assert (KH._unsupported_gen(DK, DV, N) is None) == general


def test_cpu_tensors_are_refused_not_computed():
    """The product path has no CPU fallback: CPU inputs raise before any kernel work."""
    k = torch.randn(1, 4, 1, 64)
    g = torch.rand(1, 4, 1)
    with pytest.raises(RuntimeError, match="GPU tensors only"):
        KH.kv_scan_c(k, k, g, torch.tensor([1.0]), 8, 16.0, G=2, hard=False)
    with pytest.raises(RuntimeError, match="GPU tensors only"):
        KH.kv_scan_c(k, k, g, torch.tensor([1.0]), 8, 16.0, G=2, hard=True, detach_addr=True)


def test_scan_kv_dispatch_follows_the_reference(monkeypatch):
    """scan_kv: G = 1 runs the unpinned kernel function (the reference's Triton kv_scan), G > 1 the
    reference's torch scan with its default pin=True (slotkern_kv.py:39-41)."""
    calls = []
    monkeypatch.setattr(KH, "kv_scan_c", lambda *a, **kw: calls.append(("kv_scan_c", kw["G"])))
    monkeypatch.setattr(KH, "ref_scan_kv", lambda *a, **kw: calls.append(("ref_scan_kv", kw["G"], kw.get("pin", True))))
    k = torch.randn(1, 4, 1, 64)
    g = torch.rand(1, 4, 1)
    KH.scan_kv(k, k, g, torch.tensor([1.0]), 8, 16.0)
    KH.scan_kv(k, k, g, torch.tensor([1.0]), 8, 16.0, G=8, hard=True, detach_addr=True)
    assert calls == [("kv_scan_c", 1), ("ref_scan_kv", 8, True)]
