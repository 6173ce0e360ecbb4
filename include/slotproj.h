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

/* The projection's backward, the two products autograd forms for wo_tk (memlm_sh.py:500) from the upstream
 * gradient dout (M, N) of out:
 *     drd (M, K) = dout wo            dwo (N, K) = dout^T rd
 * each a bf16 product with fp32 accumulation rounded to bf16 once, as the reference's bf16 matmuls are (the
 * gradient of delta is dout itself and needs no kernel).  drd runs on the forward's GEMM kernel with the
 * transposed weight; dwo on a GEMM that reads both token-major operands through gfx950's transposing LDS
 * read, split over the tokens, then a fixed-order sum of the splits (no atomics: bitwise reproducible).
 * N and K multiples of 256, M any.  workspace: slotproj_bwd_workspace(M, N, K) bytes, 256-byte aligned (the
 * transposed weight and the splits' fp32 partials).  Other pointers 16-byte aligned. */
size_t slotproj_bwd_workspace(int64_t M, int64_t N, int64_t K);
int slotproj_bwd(const void* dout, const void* rd, const void* wo, int64_t M, int64_t N, int64_t K, void* drd,
                 void* dwo, void* workspace, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* SLOTPROJ_H */
