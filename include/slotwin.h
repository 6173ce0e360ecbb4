/* C-ABI of the MI355X (gfx950) rolling-window attention, part of libslotscan.so.
 *
 * Replaces SharedMixer._window (/root/reference/gqa25/memlm_sh.py:349-359): the reference runs flex
 * attention with the block mask (qi >= ki) & (qi - ki < W) on GPU (memlm_sh.py:350-357), or
 * F.scaled_dot_product_attention with the same band as a boolean mask (memlm_sh.py:341-345, 359).  Scale is
 * the caller's (the reference's default 1/sqrt(D)).  Query head hq reads key/value head hq / (Hq / Hk): the
 * kv_nq path's repeat_interleave'd keys and values (memlm_sh.py:488-492) without the copies.
 *
 * Conventions: every tensor is bf16 (uint16 bit patterns) and token-major, (B, T, H, D) contiguous with
 * H = Hq for q, out, dout, dq and H = Hk for k, v, dk, dv -- the reference's (B, H, T, D) operands are
 * transposed views of this layout (memlm_sh.py:482-484).  D is 64 or 128, 1 <= W <= 16.  Pointers are device
 * pointers; q, k, v, out, dout, dq, dk, dv 16-byte aligned (the outputs are written in 16-byte row pieces).
 * Error codes as in slotscan.h. */
#ifndef SLOTWIN_H
#define SLOTWIN_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SLOTWIN_MAX_W 16

/* Forward: out (B, T, Hq, D) bf16 and lse (B, Hq, T) fp32, the log-sum-exp of every query's scaled scores
 * over its window (kept for the backward). */
int slotwin_fwd(const void* q, const void* k, const void* v, int64_t B, int64_t T, int64_t Hq, int64_t Hk,
                int64_t D, int64_t W, float scale, void* out, float* lse, void* stream);

/* Backward of slotwin_fwd for the upstream gradient dout (B, T, Hq, D): dq (B, T, Hq, D), dk and dv
 * (B, T, Hk, D), bf16, the key/value gradients summed over the query heads that share them.  dsum is
 * (B, Hq, T) fp32 workspace (rowsum(dout o out) per query). */
int slotwin_bwd(const void* q, const void* k, const void* v, const void* out, const float* lse,
                const void* dout, int64_t B, int64_t T, int64_t Hq, int64_t Hk, int64_t D, int64_t W,
                float scale, float* dsum, void* dq, void* dk, void* dv, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* SLOTWIN_H */
