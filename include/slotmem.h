/* C-ABI of the MI355X (gfx950) writer epilogue and storage quantiser, part of libslotscan.so.
 *
 * The reference post-processes the scan's fp32 snapshot copies in SharedMixer.forward
 * (/root/reference/gqa25/memlm_sh.py:466-475) with torch ops: either the full-precision epilogue
 * (nsq = sum K^2, kinv = rsqrt(max(nsq, 1e-12)), valid = nsq > 1e-12, copies cast to the activation
 * dtype, :474-475) or the storage quantiser _quantize_mem / _fq (:221-234, applied at :468-471).
 * slotmem_epilogue_fwd does either in one pass over the copies; slotmem_epilogue_bwd is the autograd of
 * the same expressions (the quantiser passes the gradient straight through, :229); slotmem_codes emits
 * the quantiser's integer codes and per-group scales (the storage form of BASELINE config 5: bits = 8,
 * group = D, one fp32 scale per row).
 *
 * Conventions as in slotscan.h (device pointers, caller-allocated, launched on `stream`, 0 or a
 * SLOTSCAN_ERR_* code).  A tensor of `rows` rows of D channels (D = 64 or 128), contiguous, 16-byte aligned.
 *   bits   0 = full precision; 2..8 = the midrise quantiser with one scale per `group` channels
 *          (group a power of two, 4 <= group <= D)
 */
#ifndef SLOTMEM_H
#define SLOTMEM_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* kout, vout: the copies the readers see (SLOTSCAN_BF16 or SLOTSCAN_F32, out_dtype), the straight-through
 * quantised values when bits > 0; kinv (rows) fp32 and valid (rows) uint8 from the (quantised) keys.
 * Replaces memlm_sh.py:468-475. */
int slotmem_epilogue_fwd(const float* kbuf, const float* vbuf, int64_t rows, int64_t D, int bits, int64_t group,
                         int out_dtype, void* kout, void* vout, float* kinv, uint8_t* valid, void* stream);

/* Gradients of slotmem_epilogue_fwd: dkbuf = dkout + 2 K dnsq, dnsq = -0.5 kinv^3 dkinv where nsq >= 1e-12
 * (K = the quantised keys when bits > 0), dvbuf = dvout.  dkout, dvout in grad_dtype (SLOTSCAN_BF16 or F32). */
int slotmem_epilogue_bwd(const float* kbuf, const void* dkout, const void* dvout, const float* dkinv,
                         int64_t rows, int64_t D, int bits, int64_t group, int grad_dtype,
                         float* dkbuf, float* dvbuf, void* stream);

/* Quantiser codes: codes (rows, D) int8 = clamp(floor(x / s), -2^(bits-1), 2^(bits-1) - 1), scales
 * (rows, D / group) fp32 = s, or 0 for an all-zero group; (code + 0.5) * scale is _fq's value
 * (memlm_sh.py:221-228). */
int slotmem_codes(const float* x, int64_t rows, int64_t D, int bits, int64_t group, int8_t* codes, float* scales,
                  void* stream);

#ifdef __cplusplus
}
#endif
#endif /* SLOTMEM_H */
