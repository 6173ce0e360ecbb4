/* C-ABI of the reader layer's output projection on MI355X (gfx950), part of libslotscan.so.
 *
 * The reference runs the read's output through the bias-free Linear wo_tk and adds it to the window output:
 *     _dr = self.wo_tk(rd.reshape(B, T, Hs * NQ * dv));  delta = _dr if delta is None else delta + _dr
 * (/root/reference/gqa25/memlm_sh.py:499-501; wo_tk declared at :313).  slotproj_fwd is that projection and add
 * as one bf16 MFMA GEMM whose epilogue is the add, reading rd in the layout slotread_fwd writes it. */
#ifndef SLOTPROJ_H
#define SLOTPROJ_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* out (M, N) = delta (M, N) + rd (M, K) wo (N, K)^T, all bf16 row-major.  Rounded as the reference rounds:
 * the product (fp32 accumulation) to bf16, then, with delta, the fp32 sum of the two to bf16 (round to nearest
 * even both times).  delta may be NULL (no window output: out = rd wo^T) and may alias out.  M = B*T tokens
 * (any), N = d_model (a multiple of 256), K = H*NQ*dv (a multiple of 32).  All four pointers 16-byte aligned.
 * Returns 0 or a SLOTSCAN_ERR_* code (slotscan_last_error). */
int slotproj_fwd(const void* rd, const void* wo, const void* delta, int64_t M, int64_t N, int64_t K, void* out,
                 void* stream);

#ifdef __cplusplus
}
#endif
#endif /* SLOTPROJ_H */
