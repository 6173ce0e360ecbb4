/* C-ABI of the MI355X (gfx950) slot-scan library, libslotscan.so.
 *
 * The reference reaches its scan kernels through torch.cuda._compile_kernel launches made by the autograd
 * function _KVScanC (/root/reference/gqa25/slotkern_cuda.py:482-533).  This library exports one entry point
 * per direction instead of per kernel: slotscan_fwd replaces the addr_fwd + val_fwd launch pair
 * (slotkern_cuda.py:505-509), slotscan_bwd replaces rows_bwd + addr_bwd (slotkern_cuda.py:525-532) and adds a
 * fixed-order reduction for dtemp and the scalar dfr (the reference uses atomicAdd, slotkern_cuda.py:437-442).
 *
 * Conventions
 *   - Every pointer is a device pointer, allocated by the caller (torch's caching allocator in the Python
 *     binding).  The library allocates nothing, synchronises nothing, and launches on `stream`
 *     (a hipStream_t; NULL = the legacy default stream).
 *   - Token tensors k, q, v are (B, T, H, D) contiguous, all of `dtype` (SLOTSCAN_F32 or SLOTSCAN_BF16);
 *     gate is (B, T, H) fp32; fr is (B, T, H) fp32 when fr_per_token, else one fp32; temp is one fp32.
 *   - Snapshots kbuf, vbuf are (B, ceil(T/G), H, N, D) fp32: the PRE-write state at t = 0, G, 2G, ...
 *     (slotkern_kvg.py:258-259).  Final state kfin, vfin (B*H, N, D) and ofin (B*H, N) fp32.
 *   - Undo log: am (B, T, H) int32 = the written row; kold, vold (B, T, H, D) fp32 and oold (B, T, H) fp32 =
 *     that row's key, value and occupancy BEFORE the write (the reference's saved tensors,
 *     slotkern_cuda.py:502-504, 510); cslog (B*H, T, N) fp32 = the cosine of every row with q_t as the
 *     forward computed it, so the backward rebuilds the forward's soft address without recomputing scores.
 *   - Return value: 0 on success, else one of the SLOTSCAN_ERR_* codes; slotscan_last_error() then holds a
 *     message (per calling thread).
 *   - Semantics: slotscan_fwd / slotscan_bwd (and the _mem pair): hard address, detached address gradient,
 *     DK == DV (slotkern_cuda.py:536-543); slotscan_gen_fwd / slotscan_gen_bwd: every other mode.  hard_gate
 *     is applied by the caller by passing the binarised gate (slotkern_cuda.py:490).
 */
#ifndef SLOTSCAN_H
#define SLOTSCAN_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SLOTSCAN_F32 0
#define SLOTSCAN_BF16 1

#define SLOTSCAN_MAX_SLOTS 192

#define SLOTSCAN_ERR_SHAPE 1
#define SLOTSCAN_ERR_DTYPE 2
#define SLOTSCAN_ERR_NULL 3
#define SLOTSCAN_ERR_ALIGN 4
#define SLOTSCAN_ERR_HIP 5

/* Message of the last failing call on this thread. */
const char* slotscan_last_error(void);

/* Largest slot count N the kernels are built for. */
int slotscan_max_slots(int64_t D);

/* Forward scan.  Replaces _KVScanC.forward's two launches (slotkern_cuda.py:484-512).
 *   k0, v0, o0   optional carried state (B*H, N, D) / (B*H, N); NULL = the all-zero, all-free start
 *                (the reference always starts from zero, slotkern_cuda.py:83-87, 190-192)
 *   kold, vold, oold, cslog  the undo log; all NULL for a forward that will not be differentiated
 *   am, kfin, vfin, ofin  always written (am drives the value replay; the final state is the carry out). */
int slotscan_fwd(const void* k, const void* q, const void* v, int dtype,
                 const float* gate, const float* fr, int fr_per_token, const float* temp,
                 int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                 float eps, int occ_bin,
                 const float* k0, const float* v0, const float* o0,
                 float* kbuf, float* vbuf, int32_t* am,
                 float* kold, float* vold, float* oold, float* cslog,
                 float* kfin, float* vfin, float* ofin, void* stream);

/* Bytes of device workspace slotscan_bwd needs: the row adjoint Dn (B*H, N, T) fp32 plus (B*H*chunks, 2)
 * fp32 partials of the address backward, which runs each chain as concurrent chunks of its steps (chunks
 * depends on B*H and T only).  The reference allocates Dn inside _KVScanC.backward (slotkern_cuda.py:524). */
size_t slotscan_bwd_workspace(int64_t B, int64_t T, int64_t H, int64_t N);

/* Which backward kernels slotscan_bwd (mem = 0) or slotscan_bwd_mem (mem = 1) runs for a shape, as a bit
 * set; no GPU work.  SLOTSCAN_PLAN_ROWS_UNTRACKED: the row kernel's G = 8 variant with explicitly counted
 * loads, used when G == 8, T % 16 == 0 (D == 128 for mem) and a batch row's snapshot gradients span at
 * most 4 GiB (its loads use 32-bit offsets); otherwise the compiler-tracked variant runs.  Returns -1 for
 * an invalid shape.  No counterpart in the reference (whose backward has one kernel per direction): it lets
 * a caller, and the CPU tests, see the choice the library makes. */
#define SLOTSCAN_PLAN_ROWS_UNTRACKED 1
int slotscan_bwd_plan(int64_t T, int64_t H, int64_t N, int64_t D, int64_t G, int mem);

/* Backward scan.  Replaces _KVScanC.backward's launches (slotkern_cuda.py:514-533).
 *   dkbuf, dvbuf  upstream gradients of kbuf, vbuf (fp32, same layout; pass zeros for a missing one)
 *   workspace     >= slotscan_bwd_workspace(...) bytes, 256-byte aligned
 *   dk, dq, dv    (B, T, H, D) in `dtype`: the store-path key gradient, the search-query gradient and the
 *                 value gradient (when the caller's q IS k, it adds dk and dq, slotkern_cuda.py:543)
 *   dgate         (B, T, H) fp32;  dfr  (B, T, H) fp32 if fr_per_token else one fp32;  dtemp  one fp32. */
int slotscan_bwd(const void* k, const void* q, const void* v, int dtype,
                 const float* gate, const float* fr, int fr_per_token, const float* temp,
                 int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                 float eps, int occ_bin,
                 const int32_t* am, const float* kold, const float* vold, const float* oold,
                 const float* cslog, const float* kfin, const float* vfin, const float* ofin,
                 const float* dkbuf, const float* dvbuf, void* workspace,
                 void* dk, void* dq, void* dv, float* dgate, float* dfr, float* dtemp,
                 void* stream);

/* Allocation-free variant of slotscan_bwd.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, results and kernels as slotscan_bwd, without `workspace`: the backward's
 * scratch (Dn and the per-chain partials) lives in a file-scope device array of
 * SLOTSCAN_NOALLOC_SCRATCH_BYTES that each device holds for the life of the process.  Shapes whose
 * slotscan_bwd_workspace(B, T, H, N) exceeds it return SLOTSCAN_ERR_SHAPE before any GPU work
 * (B*H*N*T <= about 16.7 M: e.g. B*H = 48 chains of T = 1024 steps at N = 192).  The call allocates
 * nothing (with kernel timing, slotscan_profile, off).  Every call on a device shares that device's array:
 * calls that overlap on one device race, so a caller serialises them (one stream, or events). */
#define SLOTSCAN_NOALLOC_SCRATCH_BYTES (64ull << 20)
int slotscan_bwd_noalloc(const void* k, const void* q, const void* v, int dtype,
                         const float* gate, const float* fr, int fr_per_token, const float* temp,
                         int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                         float eps, int occ_bin,
                         const int32_t* am, const float* kold, const float* vold, const float* oold,
                         const float* cslog, const float* kfin, const float* vfin, const float* ofin,
                         const float* dkbuf, const float* dvbuf,
                         void* dk, void* dq, void* dv, float* dgate, float* dfr, float* dtemp,
                         void* stream);

/* Forward scan with the writer epilogue fused in.  Replaces kv_scan_g followed by the full-precision epilogue
 * of the writer layer (memlm_sh.py:453-456 then :473-475):
 *     nsq = kbuf.pow(2).sum(-1);  mem = (kbuf.to(bf16), vbuf.to(bf16), rsqrt(nsq.clamp_min(1e-12)), nsq > 1e-12)
 * The fp32 snapshots are never stored: the chain kernel emits each key snapshot row as bf16 together with
 * its kinv and valid, and the value replay emits each value snapshot row as bf16.
 *   kb, vb   (B, ceil(T/G), H, N, D) bf16 (uint16 bit patterns)
 *   kinv     (B, ceil(T/G), H, N) fp32;  valid  (B, ceil(T/G), H, N) uint8 (0 / 1)
 * Every other argument is as in slotscan_fwd.  Applies where the epilogue follows the scan directly: not
 * with the value renormalisation (memlm_sh.py:464-465) or the storage quantiser (memlm_sh.py:468-471). */
int slotscan_fwd_mem(const void* k, const void* q, const void* v, int dtype,
                     const float* gate, const float* fr, int fr_per_token, const float* temp,
                     int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                     float eps, int occ_bin,
                     const float* k0, const float* v0, const float* o0,
                     void* kb, void* vb, float* kinv, uint8_t* valid, int32_t* am,
                     float* kold, float* vold, float* oold, float* cslog,
                     float* kfin, float* vfin, float* ofin, void* stream);

/* Backward of slotscan_fwd_mem: the autograd of the epilogue's expressions (memlm_sh.py:473-475) folded
 * into the row adjoint.  The snapshot gradients it forms from its inputs are
 *     dkbuf = dkb + 2 K dnsq,  dnsq = -0.5 kinv^3 dkinv where nsq >= 1e-12 (else 0);  dvbuf = dvb
 * with K the snapshot the replay restores, and from there it is slotscan_bwd.
 *   dkb, dvb  gradients of kb, vb: (B, ceil(T/G), H, N, D) bf16;  dkinv  (B, ceil(T/G), H, N) fp32
 * Every other argument is as in slotscan_bwd (the same workspace size). */
int slotscan_bwd_mem(const void* k, const void* q, const void* v, int dtype,
                     const float* gate, const float* fr, int fr_per_token, const float* temp,
                     int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                     float eps, int occ_bin,
                     const int32_t* am, const float* kold, const float* vold, const float* oold,
                     const float* cslog, const float* kfin, const float* vfin, const float* ofin,
                     const void* dkb, const void* dvb, const float* dkinv, void* workspace,
                     void* dk, void* dq, void* dv, float* dgate, float* dfr, float* dtemp,
                     void* stream);

/* Forward scan with the writer epilogue and the storage quantiser fused in.  Replaces kv_scan_g followed by
 * the quantised epilogue of the writer layer (memlm_sh.py:453-456 then :468-471, _quantize_mem :231-234):
 *     kq = _fq(kbuf, bits, group);  nsq = kq.pow(2).sum(-1)
 *     mem = (kq.to(bf16), _fq(vbuf, bits, group).to(bf16), rsqrt(nsq.clamp_min(1e-12)), nsq > 1e-12)
 * with _fq the midrise quantiser (memlm_sh.py:221-229; bits 2..8, one fp32 scale per `group` channels, a
 * power of two in [4, D]); bits = 0 emits the plain values (the same outputs as slotscan_fwd_mem).  The
 * chain kernel stores no key snapshots: the row replay rebuilds every key and value row from the address
 * log (bitwise the chain's state) and emits both copies.  run_sh25.sh:224 trains the last 20 % of its steps
 * this way (--qat_bits 3 --sh_qgroup 16).
 *   kcarry  (B*H, N, D) fp32 scratch in which the key replay carries its state across the forward
 *           pipeline's inner chunk boundaries: slotscan_fwd_carry_bytes(B, T, H, N, D, G) bytes, NULL when
 *           that is 0 (one chunk)
 * Every other argument is as in slotscan_fwd_mem. */
size_t slotscan_fwd_carry_bytes(int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G);
int slotscan_fwd_memq(const void* k, const void* q, const void* v, int dtype,
                      const float* gate, const float* fr, int fr_per_token, const float* temp,
                      int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                      float eps, int occ_bin, int bits, int64_t group,
                      const float* k0, const float* v0, const float* o0,
                      void* kb, void* vb, float* kinv, uint8_t* valid, int32_t* am,
                      float* kold, float* vold, float* oold, float* cslog,
                      float* kfin, float* vfin, float* ofin, float* kcarry, void* stream);

/* Backward of slotscan_fwd_memq: as slotscan_bwd_mem, with K in dkbuf = dkb + 2 K dnsq the quantised key
 * _fq(K, bits, group) that kinv was taken from, and the quantiser's own gradient the identity
 * (straight-through, memlm_sh.py:229). */
int slotscan_bwd_memq(const void* k, const void* q, const void* v, int dtype,
                      const float* gate, const float* fr, int fr_per_token, const float* temp,
                      int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                      float eps, int occ_bin, int bits, int64_t group,
                      const int32_t* am, const float* kold, const float* vold, const float* oold,
                      const float* cslog, const float* kfin, const float* vfin, const float* ofin,
                      const void* dkb, const void* dvb, const float* dkinv, void* workspace,
                      void* dk, void* dq, void* dv, float* dgate, float* dfr, float* dtemp,
                      void* stream);

/* Forward-only scan emitting both copies in the storage quantiser's integer form: the streaming scan of
 * BASELINE config 5 (int8 values with one fp32 absmax scale per row: bits = 8, group = D).  Replaces
 * kv_scan_g followed by _fq (memlm_sh.py:221-228) kept as codes:
 *     codes = clamp(floor(x / s), -2^(bits-1), 2^(bits-1) - 1) int8,  s = max(absmax / 2^(bits-1), 1e-30)
 * per group, scale = s (0 for an all-zero group), so (code + 0.5) * scale is _fq's value.
 *   kcode, vcode    (B, ceil(T/G), H, N, D) int8, 16-byte aligned
 *   kscale, vscale  (B, ceil(T/G), H, N, D / group) fp32
 *   k0, v0, o0 / kfin, vfin, ofin  the carried state in / out, as in slotscan_fwd (the stream's chunks)
 *   kcarry          as in slotscan_fwd_memq
 * No undo log is written (no backward follows).  The chain stores no snapshots; the row replay emits them. */
int slotscan_fwd_codes(const void* k, const void* q, const void* v, int dtype,
                       const float* gate, const float* fr, int fr_per_token, const float* temp,
                       int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                       float eps, int occ_bin, int bits, int64_t group,
                       const float* k0, const float* v0, const float* o0,
                       int8_t* kcode, float* kscale, int8_t* vcode, float* vscale, int32_t* am,
                       float* kfin, float* vfin, float* ofin, float* kcarry, void* stream);

/* General-mode scan: every mode the row-sparse kernels above do not cover -- soft write addresses
 * (hard = 0), the attached address gradient (detach_addr = 0), DK != DV -- as the reference runs them on its
 * general Triton scan (gqa25/slotkern_cuda.py:539-542 -> gqa25/slotkern_kvg.py:257-265; forward
 * slotkern_kvt._kvfwd, backward slotkern_kvg._kvbwd_g).  DK and DV each 64 or 128, N <= SLOTSCAN_MAX_SLOTS.
 *
 * slotscan_gen_fwd: the forward of slotkern_kvg._KVScanG (slotkern_kvg.py:210-230).
 *   kbuf (B, ceil(T/G), H, N, DK), vbuf (.., DV), obuf (B, ceil(T/G), H, N) fp32: the PRE-write state at
 *   t = 0, G, 2G, ...;  am (B, T, H) int32, hard = 1 only: the row each step wrote (first maximum);
 *   wb (B, T, H, N) fp32 or NULL: every step's write distribution before the gate (one-hot when hard),
 *   ref_scan_kv's return_w output (slotkern_kv.py:115-117).  pin: ref_scan_kv's pin (slotkern_kv.py:88-101),
 *   a row with |K| < 1e-6 scores 0 and takes no address gradient.  rlog: the address log the backward
 *   replays from, slotscan_gen_log_bytes(B, T, H, N) bytes, 16-byte aligned, or NULL when no backward
 *   follows: per (b, h) chain and step the pre-write occupancy, soft address, scaled cosine and |K| of every
 *   row, then 1 / max(|q_t|, 1e-6) per chain and step (an implementation layout, no counterpart in the
 *   reference, which recomputes them in its backward).
 * slotscan_gen_bwd: the backward (slotkern_kvg.py:233-253) for the upstream gradients dkbuf, dvbuf (fp32,
 *   shaped like kbuf, vbuf), from the forward's kbuf, vbuf, obuf, am and rlog (required).  Writes dk, dq (B, T, H, DK),
 *   dv (B, T, H, DV) in the token dtype, dgate (B, T, H), dfr (fr's shape), dtemp (1).  workspace:
 *   slotscan_gen_bwd_workspace(B, H, N, DK, DV, G) bytes, 16-byte aligned: the replay scratch (about
 *   G * N * (1 + DK / 4) fp32 per chain) and the per-chain partials.
 * Other arguments as in slotscan_fwd / slotscan_bwd. */
int slotscan_gen_fwd(const void* k, const void* q, const void* v, int dtype, const float* gate,
                     const float* fr, int fr_per_token, const float* temp, int64_t B, int64_t T,
                     int64_t H, int64_t N, int64_t DK, int64_t DV, int64_t G, float eps, int occ_bin,
                     int hard, int pin, float* kbuf, float* vbuf, float* obuf, int32_t* am, float* wb,
                     float* rlog, void* stream);
size_t slotscan_gen_log_bytes(int64_t B, int64_t T, int64_t H, int64_t N);
size_t slotscan_gen_bwd_workspace(int64_t B, int64_t H, int64_t N, int64_t DK, int64_t DV, int64_t G);
int slotscan_gen_bwd(const void* k, const void* q, const void* v, int dtype, const float* gate,
                     const float* fr, int fr_per_token, const float* temp, int64_t B, int64_t T,
                     int64_t H, int64_t N, int64_t DK, int64_t DV, int64_t G, float eps, int occ_bin,
                     int hard, int detach_addr, int pin, const float* kbuf, const float* vbuf,
                     const float* obuf, const int32_t* am, const float* rlog, const float* dkbuf,
                     const float* dvbuf, void* workspace, void* dk, void* dq, void* dv, float* dgate,
                     float* dfr, float* dtemp, void* stream);

/* Per-kernel timing (the reference's kvu/prof_cuda.py:9-20 wraps each compiled kernel's launch in CUDA
 * events; this is the same facility inside the library).  slotscan_profile(mask): 0 disables timing;
 * otherwise every launch of a kernel whose bit (1 << SLOTSCAN_K_*) is set in mask -- -1 = every kernel --
 * gets a pair of hipEvents stamped with the kernel's own start and end (hipExtLaunchKernel).  Each timed
 * launch costs the stream a few microseconds, so a caller timing a whole step times only the kernels it
 * needs.  slotscan_profile_read waits for the recorded events, writes the summed milliseconds and launch
 * counts per kernel id into total_ms[nk] / count[nk], and clears the records.  Returns 0, or
 * SLOTSCAN_ERR_HIP if an event query failed. */
#define SLOTSCAN_K_CHAIN_FWD 0
#define SLOTSCAN_K_ROWS_FWD 1
#define SLOTSCAN_K_ROWS_BWD 2
#define SLOTSCAN_K_CHAIN_BWD 3
#define SLOTSCAN_K_REDUCE 4
#define SLOTSCAN_K_READ_FWD 5
#define SLOTSCAN_K_READ_BWD 6
#define SLOTSCAN_K_MEM 7
#define SLOTSCAN_K_MEM_BWD 8
#define SLOTSCAN_K_WIN_FWD 9
#define SLOTSCAN_K_WIN_BWD 10
#define SLOTSCAN_K_GEN_FWD 11
#define SLOTSCAN_K_GEN_BWD 12
#define SLOTSCAN_K_PROJ 13
#define SLOTSCAN_K_PROJ_DRD 14
#define SLOTSCAN_K_PROJ_DWO 15
#define SLOTSCAN_K_PROJ_RED 16
#define SLOTSCAN_NK 17
int slotscan_profile(int enable);
int slotscan_profile_read(double* total_ms, int64_t* count, int nk);

#ifdef __cplusplus
}
#endif
#endif /* SLOTSCAN_H */
