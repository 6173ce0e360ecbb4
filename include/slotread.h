/* C-ABI of the MI355X (gfx950) cosine slot read, part of libslotscan.so.
 *
 * The reference computes the read inside SharedMixer._read (/root/reference/gqa25/memlm_sh.py:362-397) as
 * torch ops: a pad + permute of the queries into (B, NB, Hs, G*NQ, dk) blocks (:378-382), a bf16 einsum
 * against the block's key copy (:383), the per-row kinv and per-query sharpness multipliers (:383-393), a
 * masked softmax with nan_to_num (:394), a bf16 einsum against the value copy (:395) and the inverse
 * permute (:396-397).  slotread_fwd replaces :383-397 in one kernel that reads the queries and writes the
 * result in token-major order directly (no padded or permuted copies); slotread_bwd is its adjoint.
 *
 * Conventions (shared with slotscan.h: device pointers, caller-allocated, launched on `stream`, no
 * allocation, no synchronisation, 0 or a SLOTSCAN_ERR_* code with slotscan_last_error()):
 *   q       (B, T, H, NQ, D) bf16  unit-normalised read queries q / max(|q|, 1e-6) (memlm_sh.py:379)
 *   kbuf    (B, NB, H, N, D) bf16  the PRE-write key copy of each block of G tokens (NB = ceil(T / G))
 *   vbuf    (B, NB, H, N, D) bf16  the value copy
 *   kinv    (B, NB, H, N) fp32     1 / max(|K_n|, 1e-6) from the writer epilogue (memlm_sh.py:474-475)
 *   valid   (B, NB, H, N) uint8    row was ever written (|K_n|^2 > 1e-12); a block with no valid row reads 0
 *   scale   (B, T, H, NQ) fp32     the combined per-query multiplier exp(log_rsel) * exp(C tanh(s / C))
 *   rd      (B, T, H, NQ, D) bf16  token t reads block t / G:
 *             raw_n = bf16(<q, K_n>), sc_n = raw_n * kinv_n * scale, a = softmax over valid n (fp32),
 *             rd = bf16(sum_n bf16(a_n) V_n)
 * D (= dk = dv) must be 64 or 128 and N <= 192.
 */
#ifndef SLOTREAD_H
#define SLOTREAD_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Forward read.  Replaces memlm_sh.py:383-397 (the two einsums, the multipliers, the masked softmax and
 * the block permutes). */
int slotread_fwd(const void* q, const void* kbuf, const void* vbuf, const float* kinv, const uint8_t* valid,
                 const float* scale, int64_t B, int64_t T, int64_t H, int64_t NQ, int64_t N, int64_t D,
                 int64_t G, void* rd, void* stream);

/* Backward read: the gradients autograd computes through memlm_sh.py:383-395, with the same bf16 roundings
 * (d att_bf16 = bf16(drd V^T); softmax adjoint in fp32; d raw = bf16(dsc * kinv * scale)).
 *   drd     (B, T, H, NQ, D) bf16  upstream gradient of rd
 *   dq      (B, T, H, NQ, D) bf16  gradient of q
 *   dkbuf, dvbuf (B, NB, H, N, D) bf16  gradients of the copies (8-byte aligned)
 *   dkinv   (B, NB, H, N) fp32;  dscale (B, T, H, NQ) fp32
 * Every output element is written (no accumulation into the caller's buffers). */
int slotread_bwd(const void* q, const void* kbuf, const void* vbuf, const float* kinv, const uint8_t* valid,
                 const float* scale, const void* drd, int64_t B, int64_t T, int64_t H, int64_t NQ, int64_t N,
                 int64_t D, int64_t G, void* dq, void* dkbuf, void* dvbuf, float* dkinv, float* dscale,
                 void* stream);

#ifdef __cplusplus
}
#endif
#endif /* SLOTREAD_H */
