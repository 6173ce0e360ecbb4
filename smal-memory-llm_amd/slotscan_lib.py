"""ctypes binding of libslotscan.so (declarations: include/slotscan.h, slotread.h, slotmem.h, slotwin.h,
slotproj.h).

torch is imported BEFORE the library is opened: libslotscan.so needs libamdhip64.so.7 by SONAME, and with
torch loaded first the dynamic loader binds it to torch's own HIP runtime, so the streams and device
pointers torch hands over belong to the same runtime the kernels are launched on.

There is no fallback: if the library is missing or cannot be opened this module raises, and every op that
needs it fails loudly (the reference makes the same choice for its kernels, gqa25/memlm_sh.py:45-47 and
gqa25/slotkern_kv.py:37-38)."""
import ctypes
import os

import torch  # noqa: F401  -- must precede the CDLL below (shared HIP runtime)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libslotscan.so")

SLOTSCAN_F32 = 0
SLOTSCAN_BF16 = 1

_vp, _i64, _i32, _f32, _sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t

# name -> (restype, argtypes); every symbol declared in include/*.h appears here
SIGNATURES = {
    "slotscan_last_error": (ctypes.c_char_p, []),
    "slotscan_max_slots": (_i32, [_i64]),
    "slotscan_fwd": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _vp,
                            _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i32,
                            _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "slotscan_fwd_mem": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _vp,
                                _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i32] + [_vp] * 16),
    "slotscan_fwd_carry_bytes": (_sz, [_i64] * 6),
    "slotscan_fwd_memq": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _vp,
                                 _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _i32, _i64] + [_vp] * 17),
    "slotscan_bwd_memq": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _vp,
                                 _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _i32, _i64] + [_vp] * 19),
    "slotscan_fwd_codes": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _vp,
                                  _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _i32, _i64] + [_vp] * 13),
    "slotscan_bwd_workspace": (_sz, [_i64, _i64, _i64, _i64]),
    "slotscan_bwd_plan": (_i32, [_i64, _i64, _i64, _i64, _i64, _i32]),
    "slotscan_profile": (_i32, [_i32]),
    "slotscan_profile_read": (_i32, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64), _i32]),
    "slotscan_bwd": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _vp,
                            _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i32,
                            _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                            _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "slotscan_bwd_noalloc": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _vp,
                                    _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i32] + [_vp] * 17),
    "slotscan_bwd_mem": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _vp,
                                _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i32] + [_vp] * 19),
    "slotscan_gen_fwd": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _vp,
                                _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _i32, _i32] + [_vp] * 7),
    "slotscan_gen_log_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "slotscan_gen_bwd_workspace": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "slotscan_gen_bwd": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _vp,
                                _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _i32, _i32, _i32] + [_vp] * 15),
    "slotread_fwd": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp]),
    "slotread_bwd": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                            _vp, _vp, _vp, _vp, _vp, _vp]),
    "slotmem_epilogue_fwd": (_i32, [_vp, _vp, _i64, _i64, _i32, _i64, _i32, _vp, _vp, _vp, _vp, _vp]),
    "slotmem_epilogue_bwd": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i32, _i64, _i32, _vp, _vp, _vp]),
    "slotmem_codes": (_i32, [_vp, _i64, _i64, _i32, _i64, _vp, _vp, _vp]),
    "slotproj_fwd": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "slotproj_bwd_workspace": (_sz, [_i64, _i64, _i64]),
    "slotproj_bwd": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "slotwin_fwd": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _vp, _vp, _vp]),
    "slotwin_bwd": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _f32,
                           _vp, _vp, _vp, _vp, _vp]),
}

_lib = None


def lib():
    """The opened library (cached).  Raises RuntimeError when it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `python smal-memory-llm_amd/build.py` "
                               "(or __graft_entry__.build()) first")
        h = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(h, name)
            f.restype = res
            f.argtypes = args
        _lib = h
    return _lib


def check(rc, what):
    if rc != 0:
        msg = lib().slotscan_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def ptr(t):
    """Device pointer of a tensor, or None."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def dtype_code(dt):
    if dt == torch.float32:
        return SLOTSCAN_F32
    if dt == torch.bfloat16:
        return SLOTSCAN_BF16
    raise TypeError(f"token dtype {dt} is not supported by the HIP kernels (float32 or bfloat16)")


KERNEL_NAMES = ("chain_fwd", "rows_fwd", "rows_bwd", "chain_bwd", "reduce_parts", "read_fwd", "read_bwd", "mem_fwd",
                "mem_bwd", "win_fwd", "win_bwd", "gen_fwd", "gen_bwd", "proj", "proj_drd", "proj_dwo",
                "proj_reduce")


def profile(enable, kernels=None):
    """Start (True) or stop (False) per-kernel HIP-event timing inside the library; `kernels` (names from
    KERNEL_NAMES) restricts the timing to those kernels, None times every kernel."""
    if not enable:
        mask = 0
    elif kernels is None:
        mask = -1
    else:
        mask = 0
        for k in kernels:
            mask |= 1 << KERNEL_NAMES.index(k)
    check(lib().slotscan_profile(int(mask)), "slotscan_profile")


def profile_read():
    """{kernel name: (total ms, launches)} since the last read (waits for the recorded events)."""
    nk = len(KERNEL_NAMES)
    ms = (ctypes.c_double * nk)()
    cnt = (ctypes.c_int64 * nk)()
    check(lib().slotscan_profile_read(ms, cnt, nk), "slotscan_profile_read")
    return {KERNEL_NAMES[i]: (ms[i], cnt[i]) for i in range(nk) if cnt[i]}
