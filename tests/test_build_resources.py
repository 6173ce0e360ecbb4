"""CPU checks of properties of the compiled gfx950 kernels that the code relies on, read from the compiler's
per-kernel resource report of the current build (build.resource_report; a device-only compile when the
report is stale).  No GPU work."""
import re

import build


def test_untracked_rows_kernels_use_no_scratch():
    """rows_bwd's G = 8 variant issues its gradient, token and undo loads through inline asm that the compiler
    does not track and waits for them with hand-counted `s_waitcnt vmcnt(n)` (csrc/slotscan.hip, rows_bwd).
    On gfx9 one vector-memory counter covers loads, stores and scratch accesses, so a scratch spill or reload
    inside the counted window would break every count without any error.  The counts are only valid while
    every such instantiation has no scratch at all."""
    rep = build.resource_report("slotscan.hip")
    g8 = {n: d for n, d in rep.items() if re.fullmatch(r"void rows_bwd<\d+, [\w ]+, true, (true|false)>", n)}
    assert len(g8) == 6, sorted(g8)          # D 128: bf16 / f32 tokens x both contracts; D 64: fp32 contract
    for name, d in g8.items():
        assert d["ScratchSize [bytes/lane]"] == "0", f"{name} uses scratch: {d}"
        assert d["VGPRs Spill"] == "0", f"{name} spills: {d}"
        assert d["Dynamic Stack"] == "False", name


def test_proj_gemm_uses_no_scratch():
    """proj_gemm fills its LDS ring with direct global -> LDS loads issued through inline asm (untracked by the
    compiler) and waits for each stage with a counted `s_waitcnt vmcnt(n)` (csrc/slotproj.hip).  A scratch
    spill or reload in the k loop would be one more vector-memory operation on the same counter, so a stage
    could be published before its loads land.  The counts hold only while the kernel has no scratch."""
    rep = build.resource_report("slotproj.hip")
    kern = {n: d for n, d in rep.items() if n in ("proj_gemm", "projt_gemm")}   # projt_gemm: the same ring
    assert len(kern) == 2, sorted(rep)
    for name, d in kern.items():
        assert d["ScratchSize [bytes/lane]"] == "0", f"{name} uses scratch: {d}"
        assert d["VGPRs Spill"] == "0", f"{name} spills: {d}"
        assert d["Dynamic Stack"] == "False", name


def test_general_mode_kernels_use_no_scratch():
    """gen_fwd / gen_bwd hold a chain's rows in registers at up to 256 VGPRs (RPL = 6: 6 rows x D / 16 dims of
    K, V or their adjoints per lane).  A spill there is a scratch round trip inside the per-step loop; every
    instantiation (token dtype x DK x DV x RPL) is kept free of it."""
    rep = build.resource_report("slotgen.hip")
    kern = {n: d for n, d in rep.items() if re.fullmatch(r"void gen_(fwd|bwd)<.*>", n)}
    assert len(kern) == 48, sorted(kern)        # 2 dtypes x 2 DK x 2 DV x 3 RPL, forward and backward
    for name, d in kern.items():
        assert d["ScratchSize [bytes/lane]"] == "0", f"{name} uses scratch: {d}"
        assert d["VGPRs Spill"] == "0", f"{name} spills: {d}"


def test_read_and_window_kernels_use_no_scratch():
    """read_fwd, read_fwd_wide and win_bwd stage operands with direct global -> LDS loads the compiler does not
    track, so the wait the compiler puts before a spill reload cannot be narrowed to the reload: it waits for
    every direct load in flight (one memory round trip per reload; read_fwd_wide lost about 9 k cycles per
    unit that way before its staging offsets stopped spilling).  read_bwd runs at the register budget of three
    waves per SIMD (168 VGPRs), where a spill is a scratch round trip inside its tile loop.  Every
    instantiation of the read and window kernels is kept free of scratch."""
    for src, n_kern in (("slotread.hip", 8), ("slotwin.hip", 4)):
        rep = build.resource_report(src)
        kern = {n: d for n, d in rep.items() if re.fullmatch(r"void (read_fwd_wide|read_fwd|read_bwd|win_fwd|win_bwd)<.*>", n)}
        assert len(kern) == n_kern, (src, sorted(rep))
        for name, d in kern.items():
            assert d["ScratchSize [bytes/lane]"] == "0", f"{name} uses scratch: {d}"
            assert d["VGPRs Spill"] == "0", f"{name} spills: {d}"
            assert d["Dynamic Stack"] == "False", name
