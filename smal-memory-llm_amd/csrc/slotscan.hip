// Key-matched slot scan, hard address with a detached address gradient, for MI355X (gfx950).
//
// Semantics (reference: /root/reference/gqa25/slotkern_kv.py:66-123, production contract
// gqa25/slotkern_cuda.py:482-543).  Per chain (b, h) the state is K (N x D), V (N x D), o (N), zero or a
// carried state.  For t = 0 .. T-1:
//   t % G == 0 : emit the PRE-write K and V                                 (slotkern_kv.py:76-77)
//   s_n = temp * <K_n / max(|K_n|, 1e-6), q_t / max(|q_t|, 1e-6)>            (slotkern_kv.py:85-87)
//   z_n = s_n - fr_t * (occ_bin ? [o_n >= eps] : o_n)                        (slotkern_kv.py:104-105)
//   candidates = occupied rows + the lowest-index free row                   (slotkern_kv.py:46-51, 106)
//   a = argmax z (larger z wins, equal z -> lower index)                     (slotkern_kv.py:108-109)
//   row a <- (1-g) row a + g (k_t, v_t);  o_a <- (1-g) o_a + g               (slotkern_kv.py:118-120)
// Backward: the straight-through softmax adjoint (slotkern_kvt.py:157-171) with the address detached
// from the stored keys (slotkern_kv.py:80-84) and no gradient through [o >= eps] (slotkern_kvg.py:193-196).
//
// A hard write changes exactly one row (kvu/slotkern_kvu.py:8-13), and with the address detached the
// key/value gradient recursion depends only on WHICH row was written.  The work therefore splits into
//   chain_fwd  one workgroup per chain, sequential in t: keys + occupancy, the argmax address, the undo log
//              (row, old key row, old occupancy) and the key snapshots;
//   rows_fwd   parallel over rows: replays each row's value from the address log, value snapshots;
//   rows_bwd   parallel over rows, reverse in t: undoes rows from the log, runs dK/dV, emits dk, dv and
//              Dn[t, n] = <k_t - K_n, dK_n> + <v_t - V_n, dV_n>;
//   chain_bwd  one workgroup per chain, reverse in t: undoes keys + occupancy, rebuilds the soft address
//              and runs its adjoint: dgate, dq, per-token dfr, and per-chain dtemp / scalar-dfr partials
//              that a fixed-order reduction (reduce_parts) sums -- no float atomics anywhere.
//
// gfx950 mapping of the chain kernels.  A chain workgroup is 192 lanes = 3 waves = 12 row groups of 16
// lanes (one DPP row each); a row group holds P slot rows (P = 16 at N <= 192), lane c keeping elements
// {4c..4c+3, 64+4c..} of every one of them, in the same register order in every lane (so the written
// row's register index is wave-uniform and the update never diverges).  The per-step dot products
// <K_n, q_t> are finished with a DPP REDUCE-SCATTER instead of a 16-lane all-reduce, after which each
// lane holds the complete dot product of ONE row: all per-row scalar work (score, occupancy, softmax,
// adjoint) is done once per row instead of 16 times.  Rows increase with the lane index, so the argmax
// tie rule (lowest index) is a ballot plus a find-first-set.  The 3 waves meet in one ping-pong LDS
// slot: ONE workgroup barrier per step.  A barrier every step makes the step time the per-SIMD sum of
// issued instructions, so the design minimises per-wave work: the next step's dot products are computed
// before the barrier with the current keys and only the one rewritten row is corrected afterwards; row
// norms use v_rsq; the key snapshot slab is written every G steps as 256-byte contiguous runs, and the
// cosines of every step go to a log so the backward chain never recomputes a dot product for its scores.
// Token inputs (q, k, gate, fr; in the backward also the undo log, Dn and the cosine log) are staged in
// LDS as fp32 in double-buffered chunks.
#include "slot_common.h"
#include "slot_host.h"

using namespace slot;
typedef uint64_t u64;
typedef uint32_t u32;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define SLOT_CT 16          // tokens per staged chunk
#define CHAIN_WAVES 3
#define CHAIN_THREADS (64 * CHAIN_WAVES)

#define CHAIN_ATTR __global__ __attribute__((amdgpu_flat_work_group_size(CHAIN_THREADS, CHAIN_THREADS), amdgpu_waves_per_eu(2)))
#define ROWS_ATTR __global__ __attribute__((amdgpu_flat_work_group_size(512, 512)))

namespace {

constexpr int CT = SLOT_CT;

__device__ __forceinline__ float readlanef(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

template <int EPL>
__device__ __forceinline__ void ld_slice(float* d, const float* row, int c) {
#pragma unroll
    for (int jj = 0; jj < EPL / 4; jj++) {
        float4 x = ld4(row + 4 * c + 64 * jj);
        d[4 * jj + 0] = x.x; d[4 * jj + 1] = x.y; d[4 * jj + 2] = x.z; d[4 * jj + 3] = x.w;
    }
}
template <int EPL>
__device__ __forceinline__ void ld_slice(float* d, const bf16_t* row, int c) {
#pragma unroll
    for (int jj = 0; jj < EPL / 4; jj++) {
        float4 x = ld4(row + 4 * c + 64 * jj);
        d[4 * jj + 0] = x.x; d[4 * jj + 1] = x.y; d[4 * jj + 2] = x.z; d[4 * jj + 3] = x.w;
    }
}
template <int EPL, typename TO>
__device__ __forceinline__ void st_slice(TO* row, const float* s, int c) {
#pragma unroll
    for (int jj = 0; jj < EPL / 4; jj++)
        st4(row + 4 * c + 64 * jj, make_float4(s[4 * jj], s[4 * jj + 1], s[4 * jj + 2], s[4 * jj + 3]));
}
// streaming store of a row slice: vector non-temporal stores (full 16-byte pieces)
template <int EPL>
__device__ __forceinline__ void st_slice_nt(float* row, const float* s, int c) {
#pragma unroll
    for (int jj = 0; jj < EPL / 4; jj++) {
        f32x4 v = {s[4 * jj], s[4 * jj + 1], s[4 * jj + 2], s[4 * jj + 3]};
        __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(row + 4 * c + 64 * jj));
    }
}
template <int EPL>
__device__ __forceinline__ void ld_slice_nt(float* d, const float* row, int c) {
#pragma unroll
    for (int jj = 0; jj < EPL / 4; jj++) {
        f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(row + 4 * c + 64 * jj));
        d[4 * jj + 0] = v.x; d[4 * jj + 1] = v.y; d[4 * jj + 2] = v.z; d[4 * jj + 3] = v.w;
    }
}
// 4 raw token elements (fp32 or bf16 bits in a uint4 lane word group) -> fp32 into LDS
__device__ __forceinline__ void stage_store(float* dst, uint4 raw, bool bf) {
    if (bf) {   // 8 bf16 values
        float4 lo = make_float4(__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                                __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u));
        float4 hi = make_float4(__uint_as_float(raw.z << 16), __uint_as_float(raw.z & 0xffff0000u),
                                __uint_as_float(raw.w << 16), __uint_as_float(raw.w & 0xffff0000u));
        reinterpret_cast<float4*>(dst)[0] = lo;
        reinterpret_cast<float4*>(dst)[1] = hi;
    } else {
        *reinterpret_cast<uint4*>(dst) = raw;
    }
}

// ------------------------------------------------------------------ DPP reduce-scatter over a row group
// Every lane holds partial sums x[0..P) of the same P slot rows of its row group.  Four stages pair lanes
// with row_mirror (lane^15), row_half_mirror (lane^7), lane^2 and lane^1; the first log2(P) stages SPLIT
// (a lane keeps the half of the remaining slots picked by lane bit 3, 2, 1, 0 and receives its partner's
// partial of that half), the rest add.  Afterwards lane c holds the full 16-lane sum of slot c >> (4 -
// log2 P): each lane owns one row, so all per-row scalar work runs once per row.
template <int P> struct RS {
    static constexpr int SH = P == 16 ? 0 : P == 8 ? 1 : P == 4 ? 2 : P == 2 ? 3 : 4;
};
template <int CTRL> __device__ __forceinline__ void rs_stage(float* x, int V, bool hi) {
    const int half = V / 2;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        if (j < half) {
            const float snd = hi ? x[j] : x[j + half];
            const float kp = hi ? x[j + half] : x[j];
            x[j] = kp + dppf<CTRL>(snd);
        }
    }
}
template <int P> __device__ __forceinline__ float rs_reduce(float* x, int c) {
    // stage 0: row_mirror / lane bit 3
    if constexpr (P >= 2) rs_stage<SLOT_DPP_MIR>(x, P, c & 8); else x[0] += dppf<SLOT_DPP_MIR>(x[0]);
    // stage 1: row_half_mirror / lane bit 2
    if constexpr (P >= 4) rs_stage<SLOT_DPP_HMIR>(x, P / 2, c & 4); else x[0] += dppf<SLOT_DPP_HMIR>(x[0]);
    // stage 2: lane^2 / lane bit 1
    if constexpr (P >= 8) rs_stage<SLOT_DPP_XOR2>(x, P / 4, c & 2); else x[0] += dppf<SLOT_DPP_XOR2>(x[0]);
    // stage 3: lane^1 / lane bit 0
    if constexpr (P >= 16) rs_stage<SLOT_DPP_XOR1>(x, P / 8, c & 1); else x[0] += dppf<SLOT_DPP_XOR1>(x[0]);
    return x[0];
}

// 1 / max(sqrt(x), 1e-6) as one v_rsq_f32 (sqrt(x) < 1e-6 exactly when x < 1e-12)
__device__ __forceinline__ float rsq_clamped(float x) { return __builtin_amdgcn_rsqf(fmaxf(x, 1e-12f)); }

// one hard write of a row slice: x <- (1 - g) x + g v, as ONE explicit fma so that the chain, the row
// replay and any other kernel that re-applies the log produce bitwise the same state
__device__ __forceinline__ float blend(float x, float v, float g, float omw) { return fmaf(g, v, omw * x); }

__device__ __forceinline__ float wavemax(float v) {
    v = rowmax16(v);
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// K independent wave reductions in lockstep: the same trees as wavemax / wavesum, stage by stage over the
// K values, so the DPP and permlane latencies of different values overlap.
template <int K> __device__ __forceinline__ void wavemax_k(float* v) {
#pragma unroll
    for (int k = 0; k < K; k++) v[k] = fmaxf(v[k], dppf<SLOT_DPP_XOR1>(v[k]));
#pragma unroll
    for (int k = 0; k < K; k++) v[k] = fmaxf(v[k], dppf<SLOT_DPP_XOR2>(v[k]));
#pragma unroll
    for (int k = 0; k < K; k++) v[k] = fmaxf(v[k], dppf<SLOT_DPP_HMIR>(v[k]));
#pragma unroll
    for (int k = 0; k < K; k++) v[k] = fmaxf(v[k], dppf<SLOT_DPP_MIR>(v[k]));
#pragma unroll
    for (int k = 0; k < K; k++) {
        auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[k]), __float_as_uint(v[k]), false, false);
        v[k] = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    }
#pragma unroll
    for (int k = 0; k < K; k++) {
        auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[k]), __float_as_uint(v[k]), false, false);
        v[k] = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
}
template <int K> __device__ __forceinline__ void wavesum_k(float* v) {
#pragma unroll
    for (int k = 0; k < K; k++) v[k] += dppf<SLOT_DPP_XOR1>(v[k]);
#pragma unroll
    for (int k = 0; k < K; k++) v[k] += dppf<SLOT_DPP_XOR2>(v[k]);
#pragma unroll
    for (int k = 0; k < K; k++) v[k] += dppf<SLOT_DPP_HMIR>(v[k]);
#pragma unroll
    for (int k = 0; k < K; k++) v[k] += dppf<SLOT_DPP_MIR>(v[k]);
#pragma unroll
    for (int k = 0; k < K; k++) {
        auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[k]), __float_as_uint(v[k]), false, false);
        v[k] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
#pragma unroll
    for (int k = 0; k < K; k++) {
        auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[k]), __float_as_uint(v[k]), false, false);
        v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
}

// Row layout of a chain workgroup.  Lane `lane` of wave `w`: row group r = lane >> 4, c = lane & 15;
// register slot j holds row rowbase + j (the same order in every lane); after a reduce-scatter the lane
// owns row rowbase + (c >> SH).  Rows therefore increase with the lane index, and the lowest lane of each
// row (the "primary" lane, c % 2^SH == 0) is the one a ballot's find-first-set returns.
template <int P> struct ChainRows {
    int rowbase, n_me;
    bool prim;
    __device__ __forceinline__ ChainRows(int tid) {
        const int w = tid >> 6, lane = tid & 63, r = lane >> 4, c = lane & 15;
        rowbase = (w * 4 + r) * P;
        n_me = rowbase + (c >> RS<P>::SH);
        prim = (c & ((1 << RS<P>::SH) - 1)) == 0;
    }
    __device__ __forceinline__ int row(int j) const { return rowbase + j; }
};
template <int P> __device__ __forceinline__ int row_of_lane(int wave, int lane) {
    return (wave * 4 + (lane >> 4)) * P + ((lane & 15) >> RS<P>::SH);
}

// =========================================================================================== chain_fwd
struct ChainFwdArgs {
    const void* q; const void* k; const float* gate; const float* fr; const float* temp;
    const float* k0; const float* o0;
    float* kbuf; int32_t* am; float* kold; float* oold; float* cslog; float* kfin; float* ofin;
    int T, H, N, G, NB; float eps; int frt, occb;
    int ts, te;                                          // steps [ts, te) of the T-long sequence; ts % G == 0
    // the writer-epilogue emission (all NULL: fp32 kbuf): bf16 key copies, kinv and valid per snapshot row
    bf16_t* kbm; float* kinvm; uint8_t* validm;
    // chain (b, h) of k0 and kfin is slab b * k0bs + h (kfbs): H for (B*H, N, D) carries; NB * H where a chunk
    // of the pipeline starts from (ends in) the key snapshot of its first (next) block.  skip0: that first
    // snapshot is already written (by the previous chunk), so this chunk does not store it.
    int k0bs, kfbs, skip0;
};

// Wave-local LDS ordering: lanes of one wave exchange data through LDS (DS instructions of a wave execute
// in order; the fences keep the compiler from moving the accesses across).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Row-slice stores at a scalar base plus a 32-bit lane byte offset (the saddr form: no per-row 64-bit
// address registers)
template <int EPL, bool NT>
__device__ __forceinline__ void st_slice_at(float* base, u32 boff, const float* s) {
    char* p = reinterpret_cast<char*>(base) + boff;
#pragma unroll
    for (int jj = 0; jj < EPL / 4; jj++) {
        f32x4 v = {s[4 * jj], s[4 * jj + 1], s[4 * jj + 2], s[4 * jj + 3]};
        if (NT) __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p + 256 * jj));
        else *reinterpret_cast<f32x4*>(p + 256 * jj) = v;
    }
}

// The same slice as bf16 (the writer epilogue's cast, round to nearest even): 8 bytes per 4 elements
template <int EPL>
__device__ __forceinline__ void st_slice_bf_at(bf16_t* base, u32 boff, const float* s) {
    char* p = reinterpret_cast<char*>(base) + boff;
#pragma unroll
    for (int jj = 0; jj < EPL / 4; jj++) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 r = {pack_bf16x2(s[4 * jj], s[4 * jj + 1]), pack_bf16x2(s[4 * jj + 2], s[4 * jj + 3])};
        __builtin_nontemporal_store(r, reinterpret_cast<u32x2*>(p + 128 * jj));
    }
}

// Wave max of an ordered key (fkey), at every lane: integer max needs no NaN canonicalisation, so each
// DPP stage is one v_max_u32 with a DPP source.
__device__ __forceinline__ u32 wavemax_key(u32 v) {
    v = max(v, dppu<SLOT_DPP_XOR1>(v));
    v = max(v, dppu<SLOT_DPP_XOR2>(v));
    v = max(v, dppu<SLOT_DPP_HMIR>(v));
    v = max(v, dppu<SLOT_DPP_MIR>(v));
    auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max(p[0], p[1]);
    auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return max(r[0], r[1]);
}

// The sequential key chain, windowed over the staged 16-step chunks.
//
// Three compute waves hold the keys in registers (row layout of ChainRows; the P row slots of a lane are
// P-wide vectors, one per element, so the written row -- a wave-uniform slot -- is addressed with an
// M0-relative move instead of a branch).  A fourth, producer wave stages the tokens of the next chunk in
// LDS, and with one MFMA pass per chunk computes the chunk's Gram block E[s][u] = <k_s, q_u> and the
// query norms.  The producer does every global load, so the compute waves never wait on the
// vector-memory counter, which on gfx9 also counts their snapshot and log stores.
//
// At the start of a window every compute wave computes the dot products of ALL its rows with the 16
// queries of the window, S[n][u] = <K_n, q_u>, as fp32 MFMA (v_mfma_f32_16x16x4f32): the keys go through
// a wave-private LDS tile into the B-operand layout, 16 rows at a time.  Inside the window a step writes
// one row a; its dot products with the window's later queries follow exactly from linearity,
//     <(1-g) K_a + g k_t, q_u> = (1-g) <K_a, q_u> + g E[t][u],
// which the owner lane applies to its row's scores (rounded once per term, re-derived from the keys at
// the next window).  The row norm of the written row is recomputed from its new elements.  The per-step
// work left is the score, the argmax, and the one-row update.
//
// EM selects the key emission: CF_F32 the fp32 snapshots (kbuf); CF_BF the writer epilogue's bf16 copies with
// kinv and valid; CF_NONE no key snapshots at all -- the row replay (rows_fwd with RF_CODES / RF_MEMQ) rebuilds
// every key row bitwise from the address log and emits both copies, so the latency-bound chain carries no
// snapshot bursts.
#define FWD_THREADS (CHAIN_THREADS + 64)
enum { CF_F32 = 0, CF_BF = 1, CF_NONE = 2 };
template <int D, int P, typename TI, int EM>
__global__ __attribute__((amdgpu_flat_work_group_size(FWD_THREADS, FWD_THREADS), amdgpu_waves_per_eu(2)))
void chain_fwd(ChainFwdArgs a) {
    constexpr bool MB = EM == CF_BF;
    constexpr int EPL = D / 16;
    constexpr int DP = D + 4;                           // padded LDS row: 16 rows at stride DP hit 16 bank groups
    constexpr int EPU = 16 / (int)sizeof(TI);          // token elements per uint4
    constexpr int RU = D / EPU;                         // uint4 per token row
    constexpr int NU = CT * 2 * RU;                     // uint4 per staged chunk: (q row, k row) per token
    constexpr int UPT = (NU + 63) / 64;                // per producer lane
    constexpr bool BF = sizeof(TI) == 2;
    constexpr int WR = 4 * P;                           // rows per compute wave
    constexpr int NT = WR >= 16 ? WR / 16 : 1;          // 16-row MFMA tiles per wave
    constexpr int KL = D / 4;                           // MFMA operand dims per lane group
    constexpr int SS = CT + 4;                          // padded row of the per-wave score table
    constexpr int KT = (16 * DP > WR * SS) ? 16 * DP : WR * SS;
    typedef float rowv __attribute__((ext_vector_type(P)));
    __shared__ __align__(16) float s_q[2][CT][DP];
    __shared__ __align__(16) float s_k[2][CT][DP];
    __shared__ __align__(16) float s_E[2][CT][CT];
    __shared__ float s_qi[2][CT], s_g[2][CT], s_fr[2][CT];
    __shared__ __align__(16) float s_kt[CHAIN_WAVES][KT];
    __shared__ uint4 s_red[2][CHAIN_WAVES];

    const int T = a.T, H = a.H, N = a.N, G = a.G, ts = a.ts, te = a.te;
    const int bh = blockIdx.x, b = bh / H, h = bh - b * H;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c = tid & 15;
    const int m16 = lane & 15, ag = lane >> 4;          // MFMA operand position: row / column m16, k group ag
    const TI* __restrict__ qp = (const TI*)a.q;
    const TI* __restrict__ kp = (const TI*)a.k;
    const size_t tok0 = (size_t)b * T * H + h;          // token (b, t, h) = tok0 + t * H

    if (wave == CHAIN_WAVES) {                          // the producer wave
        uint4 rq[UPT];
        float rs = 0.f;                                 // lanes < CT: the gate of step lane; CT.. 2 CT: fr
        bool rsok = false;                              // rs is live (else 0 is staged)
        // the step scalars come from one of two uniform pointers, chosen per lane; the value is masked when it
        // is staged, so nothing waits for the load here (indexing the argument block per lane had fetched the
        // pointer with a vector load and waited for every load in flight)
        const float* const gate_p = a.gate;
        const float* const fr_p = a.frt ? a.fr : a.gate;
        auto load_chunk = [&](int ch) {
#pragma unroll
            for (int m = 0; m < UPT; m++) {
                const int u = lane + 64 * m;
                rq[m] = make_uint4(0u, 0u, 0u, 0u);
                if (u < NU) {
                    const int j = u / (2 * RU), arr = (u / RU) & 1, w = u % RU;
                    const int t = ts + ch * CT + j;
                    if (t < te) rq[m] = reinterpret_cast<const uint4*>((arr ? kp : qp) + (tok0 + (size_t)t * H) * D)[w];
                }
            }
            const int t = ts + ch * CT + (lane & (CT - 1));
            const float* sp = lane < CT ? gate_p : fr_p;
            rs = sp[tok0 + (size_t)min(t, te - 1) * H];
            rsok = lane < 2 * CT && t < te && (lane < CT || a.frt);
        };
        auto store_chunk = [&](int bf) {
#pragma unroll
            for (int m = 0; m < UPT; m++) {
                const int u = lane + 64 * m;
                if (u < NU) {
                    const int j = u / (2 * RU), arr = (u / RU) & 1, w = u % RU;
                    stage_store(arr ? &s_k[bf][j][w * EPU] : &s_q[bf][j][w * EPU], rq[m], BF);
                }
            }
            const float rv = rsok ? rs : 0.f;
            if (lane < CT) s_g[bf][lane] = rv;
            else if (lane < 2 * CT) s_fr[bf][lane - CT] = rv;
        };
        // E[s][u] = <k_s, q_u> (A = key tokens, B = query tokens; lane l, reg r -> E[4 ag + r][m16]) and
        // 1 / max(|q_u|, 1e-6) (four lanes per query, dims split in quarters)
        auto gram = [&](int bf) {
            wave_lds_sync();
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i4 = 0; i4 < KL / 4; i4++) {
                const float4 ka = ld4(&s_k[bf][m16][ag * KL + 4 * i4]);
                const float4 qb = ld4(&s_q[bf][m16][ag * KL + 4 * i4]);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.x, qb.x, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.y, qb.y, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.z, qb.z, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.w, qb.w, acc, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; r++) s_E[bf][4 * ag + r][m16] = acc[r];
            const int u = lane >> 2, p4 = lane & 3;
            float qq = 0.f;
#pragma unroll
            for (int i4 = 0; i4 < D / 16; i4++) {
                const float4 x = ld4(&s_q[bf][u][p4 * (D / 4) + 4 * i4]);
                qq = fmaf(x.x, x.x, qq); qq = fmaf(x.y, x.y, qq); qq = fmaf(x.z, x.z, qq); qq = fmaf(x.w, x.w, qq);
            }
            qq += dppf<SLOT_DPP_XOR1>(qq);
            qq += dppf<SLOT_DPP_XOR2>(qq);
            if (p4 == 0) s_qi[bf][u] = rsq_clamped(qq);
        };
        load_chunk(0);
        store_chunk(0);
        gram(0);
        __syncthreads();
        load_chunk(1);
        int j = 0, buf = 0;
        for (int t = ts; t < te; t++) {
            if (j == CT - 3) store_chunk(buf ^ 1);      // chunk +1 -> the other buffer (read from the next window)
            else if (j == CT - 2) {
                gram(buf ^ 1);
                load_chunk((t - ts) / CT + 2);
            }
            __syncthreads();
            if (++j == CT) { j = 0; buf ^= 1; }
        }
        return;
    }

    const ChainRows<P> R(tid);
    const size_t sstride = (size_t)H * N * D;
    const size_t snap0 = ((size_t)b * a.NB + ts / G) * H + h;           // (b, ts / G, h): snapshot of block ts / G
    float* kb = EM == CF_F32 ? a.kbuf + snap0 * N * D + (a.skip0 ? sstride : 0) : nullptr;   // skip0: the first slab is written
    bf16_t* kbm = MB ? a.kbm + snap0 * N * D : nullptr;
    float* kinvm = MB ? a.kinvm + snap0 * N : nullptr;
    uint8_t* validm = MB ? a.validm + snap0 * N : nullptr;
    rowv Kv[EPL];                                       // Kv[e][j]: element e of this lane's slice of row j
    float o_me = 0.f, kinv_me;
    bool vld_me;                                        // |K_me|^2 > 1e-12 (the epilogue's `valid`)
    {
        // the P rows' loads go out together (from row min(n, N - 1), unconditionally) and rows past N are
        // zeroed afterwards: a load per row behind a branch, used right away, waited for each row in turn
        const float* k0r = a.k0 ? a.k0 + (size_t)(b * a.k0bs + h) * N * D : nullptr;
        if (k0r) {
#pragma unroll
            for (int j = 0; j < P; j++) {
                float row[EPL];
                ld_slice<EPL>(row, k0r + (size_t)min(R.row(j), N - 1) * D, c);
#pragma unroll
                for (int e = 0; e < EPL; e++) Kv[e][j] = row[e];
            }
        } else {
#pragma unroll
            for (int j = 0; j < P; j++)
#pragma unroll
                for (int e = 0; e < EPL; e++) Kv[e][j] = 0.f;
        }
        float x[P];
#pragma unroll
        for (int j = 0; j < P; j++) {
            const bool in = R.row(j) < N;
            float kk = 0.f;
#pragma unroll
            for (int e = 0; e < EPL; e++) {
                Kv[e][j] = in ? Kv[e][j] : 0.f;
                kk = fmaf(Kv[e][j], Kv[e][j], kk);
            }
            x[j] = kk;
        }
        // each row's norm summed over its 16 lanes in rowsum16's order, the order of the row update after a
        // write: a chunk then starts from bitwise the kinv the previous chunk ended with, and the scan's
        // results do not depend on where the pipeline cuts the sequence (at multiples of the 16-step window)
        float nsq0 = 0.f;
#pragma unroll
        for (int j = 0; j < P; j++) {
            const float sj = rowsum16(x[j]);
            nsq0 = (c >> RS<P>::SH) == j ? sj : nsq0;
        }
        kinv_me = rsq_clamped(nsq0);
        vld_me = nsq0 > 1e-12f;
        if (a.o0 && R.n_me < N) o_me = a.o0[(size_t)bh * N + R.n_me];
    }
    auto row_of = [&](int j, float* row) {
#pragma unroll
        for (int e = 0; e < EPL; e++) row[e] = Kv[e][j];
    };

    const float temp = a.temp[0];
    const float fr_s = a.frt ? 0.f : a.fr[0];
    const float eps = a.eps;
    const bool occb = a.occb != 0, frt = a.frt != 0;
    const bool valid_me = R.n_me < N;
    const u32 roff = (u32)((R.rowbase * D + 4 * c) * 4);  // byte offset of this lane's slice of row rowbase
    const int nvalid = min(max(N - R.rowbase, 0), P);    // rows of this row group below N
    const int nl_me = (lane >> 4) * P + (c >> RS<P>::SH);  // this lane's row, wave-local
    float* kt = &s_kt[wave][0];

    __syncthreads();                                    // the producer staged the first chunk
    int par = 0, gc = 0;
    for (int w0 = ts; w0 < te; w0 += CT) {
        const int buf = ((w0 - ts) / CT) & 1;
        f32x16 Sr;                                      // <K_me, q_{w0+u}>
        int amw = -1;                                   // wave 0: the window's addresses, step j in lane j
        {   // window GEMM: S^T = Q K^T, 16 rows per tile; lane l, reg r -> S[16 tau + m16][4 ag + r]
            f32x4 acc[NT];
#pragma unroll
            for (int tau = 0; tau < NT; tau++) {
                // P divides 16, so a row group's rows lie in one tile: (lane >> 4) * P / 16
                if (WR <= 16 || (lane >> 4) * P / 16 == tau) {
#pragma unroll
                    for (int jr = 0; jr < P; jr++) {
                        float row[EPL];
                        row_of(jr, row);
                        st_slice<EPL>(kt + ((lane >> 4) * P + jr - 16 * tau) * DP, row, c);
                    }
                }
                wave_lds_sync();
                acc[tau] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i4 = 0; i4 < KL / 4; i4++) {
                    const float4 qa = ld4(&s_q[buf][m16][ag * KL + 4 * i4]);
                    const float4 kb4 = ld4(kt + m16 * DP + ag * KL + 4 * i4);
                    acc[tau] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa.x, kb4.x, acc[tau], 0, 0, 0);
                    acc[tau] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa.y, kb4.y, acc[tau], 0, 0, 0);
                    acc[tau] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa.z, kb4.z, acc[tau], 0, 0, 0);
                    acc[tau] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa.w, kb4.w, acc[tau], 0, 0, 0);
                }
                wave_lds_sync();
            }
#pragma unroll
            for (int tau = 0; tau < NT; tau++)
                if (16 * tau + m16 < WR) *reinterpret_cast<f32x4*>(kt + (16 * tau + m16) * SS + 4 * ag) = acc[tau];
            wave_lds_sync();
#pragma unroll
            for (int q4 = 0; q4 < CT / 4; q4++) {
                const float4 v = ld4(kt + nl_me * SS + 4 * q4);
                Sr[4 * q4 + 0] = v.x; Sr[4 * q4 + 1] = v.y; Sr[4 * q4 + 2] = v.z; Sr[4 * q4 + 3] = v.w;
            }
            wave_lds_sync();
        }
#pragma unroll 1
        for (int j = 0; j < CT; j++) {                  // rolled: the step's score is one M0-relative move
            const int t = w0 + j;
            if (t >= te) break;
            const float g = s_g[buf][j];
            const float frv = frt ? s_fr[buf][j] : fr_s;
            const float cs = (Sr[j] * kinv_me) * s_qi[buf][j];   // cosine of this lane's row with q_t
            const float s = temp * cs;
            // the logs (cosines, kold) are read only by the backward, after the forward's snapshot traffic: streaming
            // stores (forward 2.298 -> 2.272 ms at config 2, in one process)
            if (a.cslog && R.prim && valid_me) __builtin_nontemporal_store(cs, a.cslog + ((size_t)bh * T + t) * N + R.n_me);
            const bool taken = o_me >= eps;
            const float occ = occb ? (taken ? 1.f : 0.f) : o_me;
            const float z = s - frv * occ;
            {   // this wave's candidates: best occupied (z, lowest row) and lowest free row; the ballots are
                // wave-uniform, so the readlane runs outside divergent code
                const u32 zk = (valid_me && taken) ? fkey(z) : 0u;
                const u32 wm = wavemax_key(zk);
                const u64 mo = __ballot(valid_me && taken && zk == wm);
                const u64 mf = __ballot(valid_me && !taken);
                int bo = -1, fo = -1;
                u32 fz = 0u;
                if (mo) bo = row_of_lane<P>(wave, __builtin_ctzll(mo));
                if (mf) {
                    const int lf = __builtin_ctzll(mf);
                    fo = row_of_lane<P>(wave, lf);
                    fz = (u32)__builtin_amdgcn_readlane((int)fkey(z), lf);
                }
                if (lane == 0) s_red[par][wave] = make_uint4(wm, (u32)bo, (u32)fo, fz);
            }
            float kv[EPL];                                  // the key token, for the write below
            ld_slice<EPL>(kv, &s_k[buf][j][0], c);
            __syncthreads();
            uint4 r[CHAIN_WAVES];
#pragma unroll
            for (int w = 0; w < CHAIN_WAVES; w++) r[w] = s_red[par][w];
            if (EM != CF_NONE && gc == 0 && (MB || t != ts || !a.skip0)) {   // the PRE-write key state of block t / G:
                u32 ro = roff;                              // every row group stores whole rows
                int nvv = nvalid;
                asm volatile("" : "+v"(ro), "+v"(nvv));     // per-snapshot offsets, not 16 live registers
                if constexpr (MB) {                         // the writer epilogue: bf16 copy, kinv, valid
#pragma unroll
                    for (int jr = 0; jr < P; jr++) {
                        float row[EPL];
                        row_of(jr, row);
                        if (jr < nvv) st_slice_bf_at<EPL>(kbm, (ro >> 1) + (u32)(jr * D * 2), row);
                    }
                    if (R.prim && valid_me) {
                        kinvm[R.n_me] = kinv_me;
                        validm[R.n_me] = vld_me ? 1 : 0;
                    }
                    kbm += sstride;
                    kinvm += (size_t)H * N;
                    validm += (size_t)H * N;
                } else {
#pragma unroll
                    for (int jr = 0; jr < P; jr++) {
                        float row[EPL];
                        row_of(jr, row);
                        if (jr < nvv) st_slice_at<EPL, true>(kb, ro + (u32)(jr * D * 4), row);
                    }
                    kb += sstride;
                }
            }
            if (++gc == G) gc = 0;
            // waves in order = rows in order: strict '>' keeps the lowest row on ties
            u32 bz = 0u, fz = 0u;
            int bo = -1, fo = -1;
#pragma unroll
            for (int w = 0; w < CHAIN_WAVES; w++) {
                const int o2 = (int)r[w].y, f2 = (int)r[w].z;
                const bool tk = o2 >= 0 && (bo < 0 || r[w].x > bz);
                bz = tk ? r[w].x : bz;
                bo = tk ? o2 : bo;
                const bool tf = f2 >= 0 && fo < 0;
                fo = tf ? f2 : fo;
                fz = tf ? r[w].w : fz;
            }
            par ^= 1;
            const int amv = __builtin_amdgcn_readfirstlane((fo >= 0 && (bo < 0 || fz > bz || (fz == bz && fo < bo))) ? fo : bo);
            const size_t ix = tok0 + (size_t)t * H;
            // the address log is stored once per window (below): a store every step, behind the snapshot
            // bursts in the wave's store queue, held wave 0 on the chain's critical path
            amw = lane == j ? amv : amw;
            if (amv >= R.rowbase && amv < R.rowbase + P) {  // this row group holds the written row
                const int sl = amv & (P - 1);               // its register slot: the same in every lane
                const float omw = 1.f - g;
                // the step's E row first: its LDS latency overlaps the row update
                const f32x4* er = reinterpret_cast<const f32x4*>(&s_E[buf][j][0]);
                f32x4 e4[CT / 4];
#pragma unroll
                for (int q4 = 0; q4 < CT / 4; q4++) e4[q4] = er[q4];
                float old[EPL], nv[EPL], part = 0.f;
#pragma unroll
                for (int e = 0; e < EPL; e++) old[e] = Kv[e][sl];
#pragma unroll
                for (int e = 0; e < EPL; e++) nv[e] = blend(old[e], kv[e], g, omw);
#pragma unroll
                for (int e = 0; e < EPL; e++) Kv[e][sl] = nv[e];
#pragma unroll
                for (int e = 0; e < EPL; e++) part = fmaf(nv[e], nv[e], part);
                if (a.kold) st_slice_nt<EPL>(a.kold + ix * D, old, c);
                const float kk = rowsum16(part);
                if (R.n_me == amv) {
                    if (a.oold && R.prim) a.oold[ix] = o_me;
                    o_me = omw * o_me + g;
                    kinv_me = rsq_clamped(kk);
                    vld_me = kk > 1e-12f;
                    // all 16 entries: those at or before step j are never read again in this window
#pragma unroll
                    for (int q4 = 0; q4 < CT / 4; q4++)
#pragma unroll
                        for (int x = 0; x < 4; x++) Sr[4 * q4 + x] = fmaf(omw, Sr[4 * q4 + x], g * e4[q4][x]);
                }
            }
        }
        if (wave == 0 && lane < CT && w0 + lane < te) a.am[tok0 + (size_t)(w0 + lane) * H] = amw;
    }
#pragma unroll
    for (int jr = 0; jr < P; jr++) {
        float row[EPL];
        row_of(jr, row);
        if (jr < nvalid) st_slice_at<EPL, false>(a.kfin + (size_t)(b * a.kfbs + h) * N * D, roff + (u32)(jr * D * 4), row);
    }
    if (valid_me && R.prim) a.ofin[(size_t)bh * N + R.n_me] = o_me;
}

// =========================================================================================== rows_fwd
struct RowsFwdArgs {
    const void* v; const float* gate; const int32_t* am; const float* v0;
    float* vbuf; float* vold; float* vfin;
    int T, H, N, G, NB;
    int ts, te;                                          // steps [ts, te); ts % G == 0
    bf16_t* vbm;                                         // the writer-epilogue emission (NULL: fp32 vbuf)
    int v0bs, vfbs, skip0;                               // as ChainFwdArgs' k0bs, kfbs, skip0
    // RF_CODES / RF_MEMQ: the key replay (tokens k, start state k0 (B*H, N, D) or NULL, end state kfin) and the
    // emission of both copies -- integer codes + per-group scales (RF_CODES), or the quantiser's values (bits
    // 0: the plain values) as bf16 with kinv and valid of the emitted keys (RF_MEMQ, into kbm, vbm, kinvm,
    // validm)
    const void* k; const float* k0; float* kfin;
    int bits, group;
    bf16_t* kbm; float* kinvm; uint8_t* validm;
    int8_t* kcode; float* kscale; int8_t* vcode; float* vscale;
};

// The storage quantiser _fq (memlm_sh.py:221-228) over a row slice held the row-group way: EPL / 4 pieces of
// 4 consecutive channels, piece jj at channels 64 jj + 4 c, the row's 16 lanes c one DPP row.  A group of
// `group` channels is group / 4 consecutive lanes of one piece (group <= 64), or the whole row (group 128,
// D = 128).  Per element: a = the group's absmax, s = max(a / 2^(bits-1), 1e-30), code = clamp(floor(x / s),
// -2^(bits-1), 2^(bits-1) - 1) (IEEE division), value x + (q - x) with q = (code + 0.5) s, or 0 where a == 0
// -- the expressions of the two-pass quantiser (slotmem.hip), so codes, scales and values are bitwise its own.
// scl[jj]: the scale of piece jj's group (0 for an all-zero group).
template <int EPL>
__device__ __forceinline__ void fq_slice(const float* x, int bits, int group, float* val, float* code, float* scl) {
    constexpr int NP = EPL / 4;
    const float half = (float)(1 << (bits - 1));
    float am[NP];
#pragma unroll
    for (int jj = 0; jj < NP; jj++) {
        float m = 0.f;
#pragma unroll
        for (int e = 0; e < 4; e++) m = fmaxf(m, fabsf(x[4 * jj + e]));
        am[jj] = m;
    }
    if (NP == 2 && group > 64) {                         // one group per row of 128 channels
        const float m = rowmax16(fmaxf(am[0], am[NP - 1]));
#pragma unroll
        for (int jj = 0; jj < NP; jj++) am[jj] = m;
    } else {
#pragma unroll
        for (int jj = 0; jj < NP; jj++) {
            float m = am[jj];
            if (group >= 8) m = fmaxf(m, dppf<SLOT_DPP_XOR1>(m));
            if (group >= 16) m = fmaxf(m, dppf<SLOT_DPP_XOR2>(m));
            if (group >= 32) m = fmaxf(m, dppf<SLOT_DPP_HMIR>(m));
            if (group >= 64) m = fmaxf(m, dppf<SLOT_DPP_MIR>(m));
            am[jj] = m;
        }
    }
#pragma unroll
    for (int jj = 0; jj < NP; jj++) {
        const float ag = am[jj];
        const float sc = fmaxf(ag / half, 1e-30f);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float xe = x[4 * jj + e];
            const float cd = fminf(fmaxf(floorf(xe / sc), -half), half - 1.f);
            float q = (cd + 0.5f) * sc;
            q = ag > 0.f ? q : 0.f;
            val[4 * jj + e] = xe + (q - xe);
            code[4 * jj + e] = cd;
        }
        scl[jj] = ag > 0.f ? sc : 0.f;
    }
}

// codes of one piece (4 floats holding integers in [-128, 127]) packed as 4 bytes, channel order
__device__ __forceinline__ u32 pack_codes4(const float* cd) {
    return ((u32)(int)cd[0] & 0xffu) | (((u32)(int)cd[1] & 0xffu) << 8) | (((u32)(int)cd[2] & 0xffu) << 16) |
           (((u32)(int)cd[3] & 0xffu) << 24);
}

// 512 lanes = 32 rows of one chain per workgroup; grid (B*H, ceil(N/32)).  Replays every row's value from
// the address log and emits the value snapshots with full-row non-temporal stores.  A row changes only at
// its own writes, so the replay visits events, not steps: per 16-step piece of the staged address log a
// lane forms the mask of steps that wrote its row (4 LDS reads) and, with the piece's G-aligned snapshot
// steps, walks the set bits in step order (snapshot first: it is the PRE-write state).
// EM: RF_F32 fp32 value snapshots; RF_BF bf16 value copies; RF_CODES / RF_MEMQ also replay the KEY rows (the
// chain's own blend on the same staged token values, so bitwise the chain's keys) and emit both copies in
// the storage quantiser's integer form (RF_CODES) or as the writer epilogue's bf16 values with kinv and
// valid (RF_MEMQ).  The key state crosses the forward pipeline's inner chunk boundaries through kfin (each
// chunk's replay ends by writing it and the next starts from it), apart from the chain's own carry.
enum { RF_F32 = 0, RF_BF = 1, RF_CODES = 2, RF_MEMQ = 3 };
template <int D, typename TI, int EM>
ROWS_ATTR void rows_fwd(RowsFwdArgs a) {
    constexpr int EPL = D / 16;
    constexpr int NP = EPL / 4;
    constexpr bool MB = EM == RF_BF;
    constexpr bool KR = EM >= RF_CODES;                  // the key rows are replayed too
    constexpr int TC = 256;                              // staged steps: 2 KB of LDS, so the replay blocks fit beside two chain blocks on a CU
    __shared__ __align__(16) int s_am[TC];
    __shared__ float s_g[TC];
    const int T = a.T, H = a.H, N = a.N, G = a.G;
    const int bh = blockIdx.x, b = bh / H, h = bh - b * H;
    const int tid = threadIdx.x, rg = tid >> 4, c = tid & 15;
    const int n = blockIdx.y * 32 + rg;
    const bool live = n < N;
    const TI* __restrict__ vp = (const TI*)a.v;
    const TI* __restrict__ kp = (const TI*)a.k;
    const size_t tok0 = (size_t)b * T * H + h;
    float V[EPL], K[EPL];
#pragma unroll
    for (int e = 0; e < EPL; e++) { V[e] = 0.f; K[e] = 0.f; }
    if (live && a.v0) ld_slice<EPL>(V, a.v0 + ((size_t)(b * a.v0bs + h) * N + n) * D, c);
    if (KR && live && a.k0) ld_slice<EPL>(K, a.k0 + ((size_t)bh * N + n) * D, c);
    const size_t vrow0 = (((size_t)b * a.NB + a.ts / G) * H + h) * N * D + (size_t)(live ? n : 0) * D;
    float* vb = EM == RF_F32 ? a.vbuf + vrow0 : nullptr;
    bf16_t* vbh = MB ? a.vbm + vrow0 : nullptr;
    const size_t sstride = (size_t)H * N * D;
    // RF_CODES / RF_MEMQ outputs: the row's snapshot index advances by one (b, nb, h) slab per snapshot
    size_t srow = (((size_t)b * a.NB + a.ts / G) * H + h) * N + (size_t)(live ? n : 0);
    const int gpr = KR && EM == RF_CODES ? D / a.group : 0;   // scales per row
    auto emit = [&]() {
        if constexpr (EM == RF_CODES) {
            float kv[EPL], kc[EPL], ks[NP], vv[EPL], vc[EPL], vs[NP];
            fq_slice<EPL>(K, a.bits, a.group, kv, kc, ks);
            fq_slice<EPL>(V, a.bits, a.group, vv, vc, vs);
            int8_t* kcr = a.kcode + srow * D;
            int8_t* vcr = a.vcode + srow * D;
#pragma unroll
            for (int jj = 0; jj < NP; jj++) {
                __builtin_nontemporal_store(pack_codes4(kc + 4 * jj), reinterpret_cast<u32*>(kcr + 64 * jj + 4 * c));
                __builtin_nontemporal_store(pack_codes4(vc + 4 * jj), reinterpret_cast<u32*>(vcr + 64 * jj + 4 * c));
                const int ch = 64 * jj + 4 * c;          // the group's first lane stores its scale
                if (ch % a.group == 0) {
                    a.kscale[srow * gpr + ch / a.group] = ks[jj];
                    a.vscale[srow * gpr + ch / a.group] = vs[jj];
                }
            }
        } else if constexpr (EM == RF_MEMQ) {
            float kv[EPL], vv[EPL];
            if (a.bits) {
                float cd[EPL], sc[NP];
                fq_slice<EPL>(K, a.bits, a.group, kv, cd, sc);
                fq_slice<EPL>(V, a.bits, a.group, vv, cd, sc);
            } else {
#pragma unroll
                for (int e = 0; e < EPL; e++) { kv[e] = K[e]; vv[e] = V[e]; }
            }
            float sq = 0.f;
#pragma unroll
            for (int e = 0; e < EPL; e++) sq = fmaf(kv[e], kv[e], sq);
            const float nsq = rowsum16(sq);
            st_slice_bf_at<EPL>(a.kbm + srow * D, 8u * (u32)c, kv);
            st_slice_bf_at<EPL>(a.vbm + srow * D, 8u * (u32)c, vv);
            if (c == 0) {                                // kinv and valid of the emitted (quantised) keys
                a.kinvm[srow] = rsqrtf(fmaxf(nsq, 1e-12f));
                a.validm[srow] = nsq > 1e-12f ? 1 : 0;
            }
        }
    };
    for (int t0 = a.ts; t0 < a.te; t0 += TC) {
        const int tn = min(TC, a.te - t0);
        __syncthreads();
        for (int u = tid; u < tn; u += 512) {
            const size_t ix = tok0 + (size_t)(t0 + u) * H;
            s_am[u] = a.am[ix];
            s_g[u] = a.gate[ix];
        }
        for (int u = tn + tid; u < ((tn + 15) & ~15); u += 512) s_am[u] = -1;
        __syncthreads();
        if (!live) continue;
        for (int j0 = 0; j0 < tn; j0 += 16) {
            u32 hm = 0;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int4 a4 = *reinterpret_cast<const int4*>(&s_am[j0 + 4 * u]);
                hm |= ((a4.x == n ? 1u : 0u) | (a4.y == n ? 2u : 0u) | (a4.z == n ? 4u : 0u) | (a4.w == n ? 8u : 0u)) << (4 * u);
            }
            const int len = min(16, tn - j0);
            const int ph = (t0 + j0 - a.ts) % G;          // steps since the last snapshot (ts % G == 0)
            u32 sm = 0;
            for (int i = ph == 0 ? 0 : G - ph; i < len; i += G) sm |= 1u << i;
            u32 ev = hm | sm;
            while (ev) {
                const int i = __builtin_ctz(ev);
                ev &= ev - 1;
                if ((sm >> i) & 1u) {
                    if constexpr (MB) { st_slice_bf_at<EPL>(vbh, 8u * (u32)c, V); vbh += sstride; }
                    else if constexpr (EM == RF_F32) {
                        if (t0 + j0 + i != a.ts || !a.skip0) st_slice_nt<EPL>(vb, V, c);   // skip0: already written
                        vb += sstride;
                    } else {
                        emit();
                        srow += (size_t)H * N;
                    }
                }
                if ((hm >> i) & 1u) {
                    const size_t ix = tok0 + (size_t)(t0 + j0 + i) * H;
                    const float g = s_g[j0 + i], omw = 1.f - g;
                    float vv[EPL];
                    ld_slice<EPL>(vv, vp + ix * D, c);
                    if (a.vold) st_slice_nt<EPL>(a.vold + ix * D, V, c);      // streaming, as kold
#pragma unroll
                    for (int e = 0; e < EPL; e++) V[e] = blend(V[e], vv[e], g, omw);
                    if constexpr (KR) {
                        float kk[EPL];
                        ld_slice<EPL>(kk, kp + ix * D, c);
#pragma unroll
                        for (int e = 0; e < EPL; e++) K[e] = blend(K[e], kk[e], g, omw);
                    }
                }
            }
        }
    }
    if (live) st_slice<EPL>(a.vfin + ((size_t)(b * a.vfbs + h) * N + n) * D, V, c);
    if (KR && live && a.kfin) st_slice<EPL>(a.kfin + ((size_t)bh * N + n) * D, K, c);   // the key carry (inner chunks)
}

// =========================================================================================== rows_bwd
struct RowsBwdArgs {
    const void* k; const void* v; const float* gate; const int32_t* am;
    const float* kold; const float* vold; const float* kfin; const float* vfin;
    const float* dkbuf; const float* dvbuf;
    void* dk; void* dv; float* dn;
    int T, H, N, G, NB;
    // the writer-epilogue contract upstream (rows_bwd<..., MB = true>): the bf16 copies' gradients and dkinv;
    // qbits > 0: the copies were the storage quantiser's values (qbits, qgroup), whose gradient is straight
    // through, while kinv came from the quantised keys
    const bf16_t* dkbm; const bf16_t* dvbm; const float* dkinvm;
    int qbits, qgroup;
};

// 512 lanes = 32 rows per workgroup, grid (B*H, ceil(N/32)); reverse in t, in 16-step chunks aligned to
// t % 16 == 0, one workgroup barrier per chunk.  k_t, v_t are staged through LDS (fp32) one chunk ahead.
// Per step a lane forms <k_t, dK> + <v_t, dV> - (<K, dK> + <V, dV>) over its 8 elements (the bracket is
// kept up to date at the rare events that change it: a write to this row, a block boundary) and parks it
// in an LDS tile; at the end of the chunk lane c sums the 16 lanes' partials of step 16m + c and stores
// Dn (B*H, N, T), 64 contiguous bytes per row.  The upstream snapshot gradient is prefetched two blocks
// ahead.  The step loop is not unrolled, which keeps the rare write/boundary paths from multiplying
// register copies.
// An empty asm whose output `o` (a load offset) depends on the register set's last uses: loads addressed
// with `o` cannot be scheduled before those uses, so they can reuse the set's registers.
#define RB_AFTER(o) { if constexpr (EPL == 8) asm volatile("" : "+v"(o) : "v"(cp), "v"(dK[0]), "v"(dK[1]), "v"(dK[2]), "v"(dK[3]), "v"(dK[4]), "v"(dK[5]), "v"(dK[6]), "v"(dK[7]), "v"(dV[0]), "v"(dV[1]), "v"(dV[2]), "v"(dV[3]), "v"(dV[4]), "v"(dV[5]), "v"(dV[6]), "v"(dV[7])); \
    else asm volatile("" : "+v"(o) : "v"(cp), "v"(dK[0]), "v"(dK[1]), "v"(dK[2]), "v"(dK[3]), "v"(dV[0]), "v"(dV[1]), "v"(dV[2]), "v"(dV[3])); }
// Loads the compiler does not track (it inserts no wait of its own for them).  The consumer waits with an
// explicit vmcnt whose asm operands are the destinations, so no use can be scheduled before the wait; "+v"
// keeps each destination in place, so no copy of a value that has not arrived can be made.  Used where the
// compiler's own bookkeeping would otherwise wait with vmcnt(0) on loads issued a moment earlier.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void ldg_untracked_nt(f32x4& d, const void* p) {
    asm volatile("global_load_dwordx4 %0, %1, off nt" : "+v"(d) : "v"(p));
}
__device__ __forceinline__ void ldg_untracked(u32x4& d, const void* p) {
    asm volatile("global_load_dwordx4 %0, %1, off" : "+v"(d) : "v"(p));
}
__device__ __forceinline__ void ldg_untracked(float& d, const void* p) {
    asm volatile("global_load_dword %0, %1, off" : "+v"(d) : "v"(p));
}
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void ldg_untracked_nt(u32x2& d, const void* p) {
    asm volatile("global_load_dwordx2 %0, %1, off nt" : "+v"(d) : "v"(p));
}
__device__ __forceinline__ void ldg_untracked_nt(float& d, const void* p) {
    asm volatile("global_load_dword %0, %1, off nt" : "+v"(d) : "v"(p));
}
// Waits for a gradient set.  `all`: wait for every load (the last chunk, where fewer younger operations
// than the count may have been issued, so the counted wait would not cover the set).
// the MB set of D = 128: K and V bf16 slices (2 x 8 bytes each) and dkinv; the 5 youngest may fly
__device__ __forceinline__ void vm_wait_mb(u32x2* k, u32x2* v, float& ki, bool all) {
    if (all) asm volatile("s_waitcnt vmcnt(0)" : "+v"(k[0]), "+v"(k[1]), "+v"(v[0]), "+v"(v[1]), "+v"(ki));
    else asm volatile("s_waitcnt vmcnt(5)" : "+v"(k[0]), "+v"(k[1]), "+v"(v[0]), "+v"(v[1]), "+v"(ki));
}
template <int N4> __device__ __forceinline__ void vm_wait(f32x4* a, f32x4* b, bool all);
template <> __device__ __forceinline__ void vm_wait<1>(f32x4* a, f32x4* b, bool all) {     // the 2 youngest may fly
    if (all) asm volatile("s_waitcnt vmcnt(0)" : "+v"(a[0]), "+v"(b[0]));
    else asm volatile("s_waitcnt vmcnt(2)" : "+v"(a[0]), "+v"(b[0]));
}
template <> __device__ __forceinline__ void vm_wait<2>(f32x4* a, f32x4* b, bool all) {     // the 4 youngest may fly
    if (all) asm volatile("s_waitcnt vmcnt(0)" : "+v"(a[0]), "+v"(a[1]), "+v"(b[0]), "+v"(b[1]));
    else asm volatile("s_waitcnt vmcnt(4)" : "+v"(a[0]), "+v"(a[1]), "+v"(b[0]), "+v"(b[1]));
}

template <int D, typename TI, bool G8, bool MB>
ROWS_ATTR void rows_bwd(RowsBwdArgs a) {
    static_assert(!(G8 && MB) || D == 128, "the untracked MB path is built for D = 128");
    constexpr int EPL = D / 16;
    constexpr int EPU = 16 / (int)sizeof(TI);
    constexpr int RU = D / EPU;
    constexpr int NU = 16 * 2 * RU;
    constexpr int UPT = (NU + 511) / 512;
    constexpr bool BF = sizeof(TI) == 2;
    __shared__ __align__(16) float s_tok[2][16][2][D];
    __shared__ __align__(16) int s_am[2][16];
    __shared__ float s_g[2][16];
    __shared__ __align__(16) float s_part[32][16][17];   // [row group][step][lane], padded

    const int T = a.T, H = a.H, N = a.N, G = a.G;
    const int bh = blockIdx.x, b = bh / H, h = bh - b * H;
    const int tid = threadIdx.x, rg = tid >> 4, c = tid & 15;
    const int n0 = blockIdx.y * 32 + rg;
    const bool live = n0 < N;
    const int n = live ? n0 : 0;
    const TI* __restrict__ kp = (const TI*)a.k;
    const TI* __restrict__ vp = (const TI*)a.v;
    TI* __restrict__ dkp = (TI*)a.dk;
    TI* __restrict__ dvp = (TI*)a.dv;
    const size_t tok0 = (size_t)b * T * H + h;

    u32x4 rq[UPT];
    float ram = __int_as_float(-1);                     // the address, as bits
    float rgt = 0.f;
    auto load_chunk = [&](int m) {                      // chunk m: t in [16m, 16m + 16)
#pragma unroll
        for (int u2 = 0; u2 < UPT; u2++) {
            const int u = tid + 512 * u2;
            rq[u2] = u32x4{0u, 0u, 0u, 0u};
            if (u < NU && m >= 0) {
                const int i = u / (2 * RU), arr = (u / RU) & 1, w = u % RU, t = 16 * m + i;
                if (t < T) {
                    const u32x4* src = reinterpret_cast<const u32x4*>((arr ? vp : kp) + (tok0 + (size_t)t * H) * D) + w;
                    if constexpr (G8) ldg_untracked(rq[u2], src); else rq[u2] = *src;
                }
            }
        }
        if (tid < 16) {
            const int t = 16 * m + tid;
            ram = __int_as_float(-1); rgt = 0.f;
            if (m >= 0 && t < T) {
                const size_t ix = tok0 + (size_t)t * H;
                if constexpr (G8) { ldg_untracked(ram, a.am + ix); ldg_untracked(rgt, a.gate + ix); }
                else { ram = __int_as_float(a.am[ix]); rgt = a.gate[ix]; }
            }
        }
    };
    // `fly`: the vector-memory operations that may still be in flight, all issued after the tokens (the
    // G8 path's untracked token loads; the general path's loads are tracked by the compiler)
    auto store_chunk = [&](int buf, auto fly) {
        if constexpr (G8) {
#define RB_TOKWAIT(S) { if constexpr (UPT == 1) asm volatile(S : "+v"(rq[0]), "+v"(ram), "+v"(rgt)); \
                        else asm volatile(S : "+v"(rq[0]), "+v"(rq[1]), "+v"(ram), "+v"(rgt)); }
            if constexpr (decltype(fly)::value == 0) RB_TOKWAIT("s_waitcnt vmcnt(0)")
            else if constexpr (decltype(fly)::value == 2) RB_TOKWAIT("s_waitcnt vmcnt(2)")
            else if constexpr (decltype(fly)::value == 5) RB_TOKWAIT("s_waitcnt vmcnt(5)")
            else RB_TOKWAIT("s_waitcnt vmcnt(4)")
#undef RB_TOKWAIT
        }
#pragma unroll
        for (int u2 = 0; u2 < UPT; u2++) {
            const int u = tid + 512 * u2;
            if (u < NU) {
                const int i = u / (2 * RU), arr = (u / RU) & 1, w = u % RU;
                const uint4 r4 = make_uint4(rq[u2].x, rq[u2].y, rq[u2].z, rq[u2].w);
                stage_store(&s_tok[buf][i][arr][w * EPU], r4, BF);
            }
        }
        if (tid < 16) { s_am[buf][tid] = __float_as_int(ram); s_g[buf][tid] = rgt; }
    };

    constexpr int NQ = EPL / 4;                          // 16-byte pieces of a row slice
    float K[EPL], V[EPL], dK[EPL], dV[EPL], pk1[EPL], pv1[EPL], pk2[EPL], pv2[EPL];
    f32x4 gk1[NQ], gv1[NQ], gk2[NQ], gv2[NQ];           // the G8 path's two untracked gradient sets
    u32x2 hk1[NQ], hv1[NQ], hk2[NQ], hv2[NQ];           // ... in the MB contract: bf16 slices (8 bytes each)
    float hi1 = 0.f, hi2 = 0.f, pki1 = 0.f, pki2 = 0.f;  // dkinv of a set / of the general path's blocks
    ld_slice<EPL>(K, a.kfin + ((size_t)bh * N + n) * D, c);
    ld_slice<EPL>(V, a.vfin + ((size_t)bh * N + n) * D, c);
#pragma unroll
    for (int e = 0; e < EPL; e++) { dK[e] = 0.f; dV[e] = 0.f; pk2[e] = 0.f; pv2[e] = 0.f; }
#pragma unroll
    for (int q = 0; q < NQ; q++) {
        gk1[q] = gv1[q] = gk2[q] = gv2[q] = f32x4{0.f, 0.f, 0.f, 0.f};
        hk1[q] = hv1[q] = hk2[q] = hv2[q] = u32x2{0u, 0u};
    }
    float cp = 0.f;                                      // this lane's share of <K, dK> + <V, dV>
    const size_t sbstride = (size_t)H * N * D;
    const float* dkb0 = a.dkbuf + ((size_t)b * a.NB * H + h) * N * D + (size_t)n * D;
    const float* dvb0 = a.dvbuf + ((size_t)b * a.NB * H + h) * N * D + (size_t)n * D;
    // MB: the bf16 gradients of the writer epilogue's copies and dkinv, same (b, nb, h, n) order
    const size_t kistride = (size_t)H * N;
    const bf16_t* dkh0 = MB ? a.dkbm + ((size_t)b * a.NB * H + h) * N * D + (size_t)n * D : nullptr;
    const bf16_t* dvh0 = MB ? a.dvbm + ((size_t)b * a.NB * H + h) * N * D + (size_t)n * D : nullptr;
    const float* dki0 = MB ? a.dkinvm + ((size_t)b * a.NB * H + h) * N + n : nullptr;
    // MB, the G8 path: load q of a set's 2 NQ + 1 (K slice pieces, V slice pieces, dkinv), untracked
    auto refill_mb = [&](u32x2* hk, u32x2* hv, float& hki, int blk, int q) {
        const u32 o = (u32)max(blk, 0) * (u32)(sbstride * sizeof(bf16_t)) + 8u * (u32)c;
        if (q < NQ) ldg_untracked_nt(hk[q], (const char*)dkh0 + o + 128 * q);
        else if (q < 2 * NQ) ldg_untracked_nt(hv[q - NQ], (const char*)dvh0 + o + 128 * (q - NQ));
        else ldg_untracked_nt(hki, dki0 + (size_t)max(blk, 0) * kistride);
    };
    // the G8 path's reload of a gradient set with block `blk` (clamped), untracked; the offset passes
    // through an empty asm that takes the set's last uses as inputs, so the loads issue after them
    auto reload = [&](f32x4* gk, f32x4* gv, int blk) {
        u32 o = (u32)max(blk, 0) * (u32)(sbstride * sizeof(float)) + 16u * (u32)c;
        RB_AFTER(o)
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            ldg_untracked_nt(gk[q], (const char*)dkb0 + o + 256 * q);
            ldg_untracked_nt(gv[q], (const char*)dvb0 + o + 256 * q);
        }
    };
    int nxt = (T - 1) / G;                               // next block whose gradient enters (reverse order)
    if constexpr (G8 && MB) {
#pragma unroll
        for (int q = 0; q < 2 * NQ + 1; q++) refill_mb(hk1, hv1, hi1, nxt, q);   // set 2: the first chunk
    } else if constexpr (G8) {
        reload(gk1, gv1, nxt);                           // set 2 is refilled during the first chunk
    } else if constexpr (MB) {
        ld_slice<EPL>(pk1, dkh0 + (size_t)nxt * sbstride, c);
        ld_slice<EPL>(pv1, dvh0 + (size_t)nxt * sbstride, c);
        pki1 = dki0[(size_t)nxt * kistride];
        if (nxt >= 1) {
            ld_slice<EPL>(pk2, dkh0 + (size_t)(nxt - 1) * sbstride, c);
            ld_slice<EPL>(pv2, dvh0 + (size_t)(nxt - 1) * sbstride, c);
            pki2 = dki0[(size_t)(nxt - 1) * kistride];
        }
    } else {
        ld_slice_nt<EPL>(pk1, dkb0 + (size_t)nxt * sbstride, c);
        ld_slice_nt<EPL>(pv1, dvb0 + (size_t)nxt * sbstride, c);
        if (nxt >= 1) {
            ld_slice_nt<EPL>(pk2, dkb0 + (size_t)(nxt - 1) * sbstride, c);
            ld_slice_nt<EPL>(pv2, dvb0 + (size_t)(nxt - 1) * sbstride, c);
        }
    }
    int tb = nxt * G;                                    // the step at which block `nxt` enters
    const int nblk = (T + 15) / 16;
    load_chunk(nblk - 1);
    store_chunk(0, std::integral_constant<int, 0>());
    __syncthreads();
    load_chunk(nblk - 2);
    int buf = 0;
    // one reverse step of this row: undo at a write, the Dn partial, the write's token gradients
    auto step = [&](int i, int t, u32 hm) {
        const bool hit = (hm >> i) & 1u;
        if (hit) {                                      // undo: the row before this step's write
            const size_t ix = tok0 + (size_t)t * H;
            if constexpr (G8) {                         // untracked, so no tracked load stays pending
                f32x4 k4[NQ], v4[NQ];
#pragma unroll
                for (int q = 0; q < NQ; q++) {
                    k4[q] = v4[q] = f32x4{0.f, 0.f, 0.f, 0.f};
                    ldg_untracked_nt(k4[q], a.kold + ix * D + 4 * c + 64 * q);
                    ldg_untracked_nt(v4[q], a.vold + ix * D + 4 * c + 64 * q);
                }
                if constexpr (NQ == 2) asm volatile("s_waitcnt vmcnt(0)" : "+v"(k4[0]), "+v"(k4[1]), "+v"(v4[0]), "+v"(v4[1]));
                else asm volatile("s_waitcnt vmcnt(0)" : "+v"(k4[0]), "+v"(v4[0]));
#pragma unroll
                for (int q = 0; q < NQ; q++)
#pragma unroll
                    for (int x = 0; x < 4; x++) { K[4 * q + x] = k4[q][x]; V[4 * q + x] = v4[q][x]; }
            } else {
                ld_slice<EPL>(K, a.kold + ix * D, c);
                ld_slice<EPL>(V, a.vold + ix * D, c);
            }
            cp = 0.f;
#pragma unroll
            for (int e = 0; e < EPL; e++) cp = fmaf(K[e], dK[e], fmaf(V[e], dV[e], cp));
        }
        float p = -cp;
        const float* kt = &s_tok[buf][i][0][0];
        const float* vt = &s_tok[buf][i][1][0];
#pragma unroll
        for (int jj = 0; jj < EPL / 4; jj++) {
            const float4 k4 = *reinterpret_cast<const float4*>(kt + 4 * c + 64 * jj);
            const float4 v4 = *reinterpret_cast<const float4*>(vt + 4 * c + 64 * jj);
            p = fmaf(k4.x, dK[4 * jj + 0], p); p = fmaf(k4.y, dK[4 * jj + 1], p);
            p = fmaf(k4.z, dK[4 * jj + 2], p); p = fmaf(k4.w, dK[4 * jj + 3], p);
            p = fmaf(v4.x, dV[4 * jj + 0], p); p = fmaf(v4.y, dV[4 * jj + 1], p);
            p = fmaf(v4.z, dV[4 * jj + 2], p); p = fmaf(v4.w, dV[4 * jj + 3], p);
        }
        s_part[rg][i][c] = p;
        if (hit) {
            const size_t ix = tok0 + (size_t)t * H;
            const float g = s_g[buf][i], omw = 1.f - g;
            float x[EPL], y[EPL];
#pragma unroll
            for (int e = 0; e < EPL; e++) { x[e] = g * dK[e]; y[e] = g * dV[e]; dK[e] *= omw; dV[e] *= omw; }
            cp *= omw;
            st_slice<EPL>(dkp + ix * D, x, c);
            st_slice<EPL>(dvp + ix * D, y, c);
        }
    };
    // the gradient of the snapshot emitted at a block boundary enters (it is the pre-write state)
    auto enter = [&](const float* pk, const float* pv) {
#pragma unroll
        for (int e = 0; e < EPL; e++) {
            dK[e] += pk[e];
            dV[e] += pv[e];
            cp = fmaf(K[e], pk[e], fmaf(V[e], pv[e], cp));
        }
    };
    // MB: the writer epilogue's key gradient at this snapshot, d kbuf = d kb + 2 K dnsq with
    // dnsq = -0.5 kinv^3 dkinv where |K|^2 >= 1e-12 (slotmem.hip's backward); K is the snapshot's value, or
    // with the storage quantiser its quantised value (memlm_sh.py:231-234: kinv is taken from _fq(kbuf), and
    // _fq passes the gradient straight through)
    auto combine = [&](float* pk, float dki) {
        float kq[EPL];
        if (a.qbits) {
            float cd[EPL], sc[NQ];
            fq_slice<EPL>(K, a.qbits, a.qgroup, kq, cd, sc);
        } else {
#pragma unroll
            for (int e = 0; e < EPL; e++) kq[e] = K[e];
        }
        float nsq = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) nsq = fmaf(kq[e], kq[e], nsq);
        nsq = rowsum16(nsq);
        const float ki = rsq_clamped(nsq);
        const float coef = nsq >= 1e-12f ? -(ki * ki * ki) * dki : 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) pk[e] = fmaf(coef, kq[e], pk[e]);
    };
    auto enter_mb = [&](const u32x2* hk, const u32x2* hv, float hki) {
        float pk[EPL], pv[EPL];
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            pk[4 * q + 0] = __uint_as_float(hk[q].x << 16); pk[4 * q + 1] = __uint_as_float(hk[q].x & 0xffff0000u);
            pk[4 * q + 2] = __uint_as_float(hk[q].y << 16); pk[4 * q + 3] = __uint_as_float(hk[q].y & 0xffff0000u);
            pv[4 * q + 0] = __uint_as_float(hv[q].x << 16); pv[4 * q + 1] = __uint_as_float(hv[q].x & 0xffff0000u);
            pv[4 * q + 2] = __uint_as_float(hv[q].y << 16); pv[4 * q + 3] = __uint_as_float(hv[q].y & 0xffff0000u);
        }
        combine(pk, hki);
        enter(pk, pv);
    };
    // lane c sums the row group's 16 partials of step 16m + c (same wave wrote them: wave barrier only)
    // A row's Dn slice of one chunk is 64 bytes, half a 128-byte line; the odd chunk's value is held until
    // the even chunk below it is done, and both halves of the line are stored together (written a chunk
    // apart, the halves reached HBM as separate partial-line writes).
    float dn_hold = 0.f;
    auto emit_dn = [&](int m) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float dnv = 0.f;
#pragma unroll
        for (int l = 0; l < 16; l++) dnv += s_part[rg][c][l];
        float* drow = a.dn + ((size_t)bh * N + n) * T;
        if (m & 1) {
            dn_hold = dnv;                              // chunk m - 1 always follows
        } else {
            if (live && 16 * m + c < T) __builtin_nontemporal_store(dnv, drow + 16 * m + c);
            if (live && m + 1 < nblk && 16 * (m + 1) + c < T) __builtin_nontemporal_store(dn_hold, drow + 16 * (m + 1) + c);
        }
    };
    for (int m = nblk - 1; m >= 0; m--) {
        u32 hm = 0;                                      // steps of this chunk that wrote this row
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int4 a4 = *reinterpret_cast<const int4*>(&s_am[buf][4 * u]);
            hm |= (a4.x == n ? 1u : 0u) << (4 * u) | (a4.y == n ? 2u : 0u) << (4 * u)
                | (a4.z == n ? 4u : 0u) << (4 * u) | (a4.w == n ? 8u : 0u) << (4 * u);
        }
        if (!live) hm = 0;
        if constexpr (G8 && MB) {
            // The same schedule for the writer-epilogue contract: a set is 2 NQ + 1 = 5 loads (the bf16 K
            // and V slice pieces and dkinv), refilled at steps 15..11 (set 2) and 7..3 (set 1); every wait
            // lets the latest refill's 5 loads fly.
            constexpr int NSM = 2 * NQ + 1;
            using FLY = std::integral_constant<int, NSM>;
#pragma unroll
            for (int i = 15; i >= 16 - NSM; i--) { step(i, 16 * m + i, hm); refill_mb(hk2, hv2, hi2, 2 * m, 15 - i); }
#pragma unroll 1
            for (int i = 15 - NSM; i >= 9; i--) step(i, 16 * m + i, hm);
            step(8, 16 * m + 8, hm);
            vm_wait_mb(hk1, hv1, hi1, false);
            enter_mb(hk1, hv1, hi1);
#pragma unroll
            for (int i = 7; i >= 8 - NSM; i--) { step(i, 16 * m + i, hm); if (m > 0) refill_mb(hk1, hv1, hi1, 2 * m - 1, 7 - i); }
#pragma unroll 1
            for (int i = 7 - NSM; i >= 1; i--) step(i, 16 * m + i, hm);
            if (m > 0) store_chunk(buf ^ 1, FLY());
            step(0, 16 * m, hm);
            vm_wait_mb(hk2, hv2, hi2, m == 0);
            enter_mb(hk2, hv2, hi2);
            emit_dn(m);
            if (m > 0) load_chunk(m - 2);
        } else if constexpr (G8) {
            // G == 8, T % 16 == 0: boundaries at i = 8 (block 2m + 1, set 1) and i = 0 (block 2m, set 2).
            // Each set is refilled untracked and in place, ONE load per step so the vector-memory queue
            // never fills: set 2 (block 2m) during steps 15..12 of this chunk, set 1 (block 2m - 1, used by
            // the next chunk) during steps 7..4 after its use at i = 8.  Every wait is explicit; at each one
            // the NS = 2 NQ loads of the latest refill are younger than the data it needs:
            //   set 1 at i = 8       (refilled in the previous chunk; younger: this chunk's set-2 loads),
            //   tokens before i = 0  (loaded at the previous chunk's end; younger: both refills),
            //   set 2 after i = 0    (refilled at steps 15..12; younger: the set-1 loads of steps 7..4 --
            //                         except in the last chunk, which waits for all).
            // A write adds younger operations, which only makes a wait stricter.
            using FLY = std::integral_constant<int, 2 * NQ>;
            auto refill = [&](f32x4* gk, f32x4* gv, int blk, int q) {     // load q of a set's 2 NQ
                const u32 o = (u32)max(blk, 0) * (u32)(sbstride * sizeof(float)) + 16u * (u32)c;
                if (q < NQ) ldg_untracked_nt(gk[q], (const char*)dkb0 + o + 256 * q);
                else ldg_untracked_nt(gv[q - NQ], (const char*)dvb0 + o + 256 * (q - NQ));
            };
#pragma unroll
            for (int i = 15; i >= 16 - 2 * NQ; i--) { step(i, 16 * m + i, hm); refill(gk2, gv2, 2 * m, 15 - i); }
#pragma unroll 1
            for (int i = 15 - 2 * NQ; i >= 9; i--) step(i, 16 * m + i, hm);
            step(8, 16 * m + 8, hm);
            vm_wait<NQ>(gk1, gv1, false);
            enter(reinterpret_cast<const float*>(gk1), reinterpret_cast<const float*>(gv1));
            // (no set-1 refill in the last chunk: nothing would wait for it, and a load still in flight when
            // the loop ends would land in registers the code after the loop may be given)
#pragma unroll
            for (int i = 7; i >= 8 - 2 * NQ; i--) { step(i, 16 * m + i, hm); if (m > 0) refill(gk1, gv1, 2 * m - 1, 7 - i); }
#pragma unroll 1
            for (int i = 7 - 2 * NQ; i >= 1; i--) step(i, 16 * m + i, hm);
            if (m > 0) store_chunk(buf ^ 1, FLY());
            step(0, 16 * m, hm);
            vm_wait<NQ>(gk2, gv2, m == 0);             // the last chunk issued no set-1 refill after set 2
            enter(reinterpret_cast<const float*>(gk2), reinterpret_cast<const float*>(gv2));
            emit_dn(m);
            if (m > 0) load_chunk(m - 2);
        } else {
            const int i_hi = min(15, T - 1 - 16 * m);
            for (int i = 15; i > i_hi; i--) s_part[rg][i][c] = 0.f;
            for (int i = i_hi; i >= 0; i--) {
                const int t = 16 * m + i;
                step(i, t, hm);
                if (t == tb) {
                    if constexpr (MB) combine(pk1, pki1);
                    enter(pk1, pv1);
#pragma unroll
                    for (int e = 0; e < EPL; e++) { pk1[e] = pk2[e]; pv1[e] = pv2[e]; }
                    pki1 = pki2;
                    nxt -= 1;
                    tb -= G;
                    if (nxt >= 1) {
                        if constexpr (MB) {
                            ld_slice<EPL>(pk2, dkh0 + (size_t)(nxt - 1) * sbstride, c);
                            ld_slice<EPL>(pv2, dvh0 + (size_t)(nxt - 1) * sbstride, c);
                            pki2 = dki0[(size_t)(nxt - 1) * kistride];
                        } else {
                            ld_slice_nt<EPL>(pk2, dkb0 + (size_t)(nxt - 1) * sbstride, c);
                            ld_slice_nt<EPL>(pv2, dvb0 + (size_t)(nxt - 1) * sbstride, c);
                        }
                    }
                }
            }
            emit_dn(m);
            if (m > 0) {
                store_chunk(buf ^ 1, std::integral_constant<int, 0>());
                load_chunk(m - 2);
            }
        }
        __syncthreads();
        buf ^= 1;
    }
    if constexpr (G8) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // no untracked load is left in flight; belt and braces
}

// =========================================================================================== chain_bwd
struct ChainBwdArgs {
    const void* q; const float* gate; const float* fr; const float* temp;
    const int32_t* am; const float* kold; const float* oold; const float* cslog; const float* kfin; const float* ofin;
    const float* dn;                                     // (B*H, N, T)
    void* dq; float* dg; float* dfr; float* part;        // part (B*H*chunks, 2): dtemp and scalar-dfr partials
    int T, H, N; float eps; int frt, occb;
    int wpc;                                             // chain_bwd_w: windows per chunk (grid.y = chunks)
};

// OCCB (occ_bin) is a template flag: with it the occupancy enters only through [o >= eps] and its
// adjoint dO is identically zero, so the kernel carries no dO.  The scores are not recomputed: the
// forward logged every row's cosine with q_t (cslog), so the backward rebuilds exactly the forward's
// soft address and keeps the keys only for the query gradient dq = sum_n dz_n kinv_n K_n.
template <int D, int P, typename TI, bool OCCB>
CHAIN_ATTR void chain_bwd(ChainBwdArgs a) {
    constexpr int CT = P >= 16 ? 4 : SLOT_CT;           // fewer staging registers at N > 96
    constexpr int EPL = D / 16;
    constexpr int EPU = 16 / (int)sizeof(TI);
    constexpr int RUQ = D / EPU, RUK = D / 4;
    constexpr int NUQ = CT * RUQ, NU = NUQ + CT * RUK;
    constexpr int UPT = (NU + CHAIN_THREADS - 1) / CHAIN_THREADS;
    constexpr int NMAX = 4 * CHAIN_WAVES * P;
    constexpr int DPT = (CT * NMAX + CHAIN_THREADS - 1) / CHAIN_THREADS;
    constexpr int EPW = D / 64;                          // q elements per lane in the dq finaliser
    constexpr bool BF = sizeof(TI) == 2;
    __shared__ __align__(16) float s_q[2][CT][D];
    __shared__ __align__(16) float s_ko[2][CT][D];
    __shared__ float s_dn[2][CT][NMAX];
    __shared__ float s_cs[2][CT][NMAX];
    __shared__ float s_g[2][CT], s_fr[2][CT], s_oo[2][CT];
    __shared__ int s_am[2][CT];
    __shared__ __align__(16) float s_st[2][CHAIN_WAVES][8];
    __shared__ float s_pq[2][CHAIN_WAVES][D];
    __shared__ float s_pfr[2][CHAIN_WAVES];
    __shared__ float s_fin[2][CHAIN_WAVES];
    __shared__ __align__(16) float s_cf[NMAX];

    const int T = a.T, H = a.H, N = a.N;
    const int bh = blockIdx.x, b = bh / H, h = bh - b * H;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c = tid & 15;
    const ChainRows<P> R(tid);
    const TI* __restrict__ qp = (const TI*)a.q;
    const size_t tok0 = (size_t)b * T * H + h;
    const float temp = a.temp[0];
    const float fr_s = a.frt ? 0.f : a.fr[0];
    const float eps = a.eps;
    const bool frt = a.frt != 0;
    const bool valid_me = R.n_me < N;

    float K[P][EPL];
    float o_me = 0.f, dO_me = 0.f, kinv_me;
    {
        float x[P];
#pragma unroll
        for (int j = 0; j < P; j++) {
            const int n = R.row(j);
#pragma unroll
            for (int e = 0; e < EPL; e++) K[j][e] = 0.f;
            if (n < N) ld_slice<EPL>(K[j], a.kfin + ((size_t)bh * N + n) * D, c);
            float kk = 0.f;
#pragma unroll
            for (int e = 0; e < EPL; e++) kk = fmaf(K[j][e], K[j][e], kk);
            x[j] = kk;
        }
        kinv_me = rsq_clamped(rs_reduce<P>(x, c));
        if (valid_me) o_me = a.ofin[(size_t)bh * N + R.n_me];
    }

    uint4 rq[UPT];
    float rdn[DPT], rcs[DPT];
    float rs = 0.f;
    auto load_chunk = [&](int ch) {
#pragma unroll
        for (int m = 0; m < UPT; m++) {
            const int u = tid + CHAIN_THREADS * m;
            rq[m] = make_uint4(0u, 0u, 0u, 0u);
            if (u < NUQ) {
                const int jj = u / RUQ, w = u % RUQ, t = T - 1 - (ch * CT + jj);
                if (t >= 0) rq[m] = reinterpret_cast<const uint4*>(qp + (tok0 + (size_t)t * H) * D)[w];
            } else if (u < NU) {
                const int u2 = u - NUQ, jj = u2 / RUK, w = u2 % RUK, t = T - 1 - (ch * CT + jj);
                if (t >= 0) rq[m] = reinterpret_cast<const uint4*>(a.kold + (tok0 + (size_t)t * H) * D)[w];
            }
        }
#pragma unroll
        for (int m = 0; m < DPT; m++) {
            const int u = tid + CHAIN_THREADS * m;
            rdn[m] = 0.f;
            rcs[m] = 0.f;
            if (u < CT * N) {
                int nn = u / CT, jj = u % CT, t = T - 1 - (ch * CT + jj);
                if (t >= 0) rdn[m] = a.dn[((size_t)bh * N + nn) * T + t];          // Dn is (N, T) per chain
                jj = u / N; nn = u % N; t = T - 1 - (ch * CT + jj);
                if (t >= 0) rcs[m] = a.cslog[((size_t)bh * T + t) * N + nn];       // the cosines are (T, N)
            }
        }
        if (tid < 4 * CT) {
            const int jj = tid & (CT - 1), t = T - 1 - (ch * CT + jj);
            rs = 0.f;
            if (t >= 0) {
                const size_t ix = tok0 + (size_t)t * H;
                const int kind = tid / CT;
                rs = kind == 0 ? __int_as_float(a.am[ix]) : kind == 1 ? a.gate[ix]
                   : kind == 2 ? (frt ? a.fr[ix] : 0.f) : a.oold[ix];
            }
        }
    };
    auto store_chunk = [&](int buf) {
#pragma unroll
        for (int m = 0; m < UPT; m++) {
            const int u = tid + CHAIN_THREADS * m;
            if (u < NUQ) stage_store(&s_q[buf][u / RUQ][(u % RUQ) * EPU], rq[m], BF);
            else if (u < NU) {
                const int u2 = u - NUQ;
                stage_store(&s_ko[buf][u2 / RUK][(u2 % RUK) * 4], rq[m], false);
            }
        }
#pragma unroll
        for (int m = 0; m < DPT; m++) {
            const int u = tid + CHAIN_THREADS * m;
            if (u < CT * N) {
                s_dn[buf][u % CT][u / CT] = rdn[m];
                s_cs[buf][u / N][u % N] = rcs[m];
            }
        }
        if (tid < 4 * CT) {
            const int jj = tid & (CT - 1), kind = tid / CT;
            if (kind == 0) s_am[buf][jj] = __float_as_int(rs);
            else if (kind == 1) s_g[buf][jj] = rs;
            else if (kind == 2) s_fr[buf][jj] = rs;
            else s_oo[buf][jj] = rs;
        }
    };
    // dq (and per-token dfr) of processed step sp, by one wave, from the per-wave partials of that step
    auto finalize = [&](int sp) {
        const int pp = sp & 1, bp = (sp / CT) & 1, jp = sp % CT, tp = T - 1 - sp;
        float dqn[EPW], qe[EPW];
        float pr = 0.f, qq = 0.f;
#pragma unroll
        for (int m = 0; m < EPW; m++) {
            const int e = lane + 64 * m;
            float acc = 0.f;
#pragma unroll
            for (int w = 0; w < CHAIN_WAVES; w++) acc += s_pq[pp][w][e];
            dqn[m] = temp * acc;
            qe[m] = s_q[bp][jp][e];
            pr = fmaf(dqn[m], qe[m], pr);
            qq = fmaf(qe[m], qe[m], qq);
        }
        qq = wavesum(qq);
        const float qi = rsq_clamped(qq);
        pr = wavesum(pr) * qi;                            // <qhat, dqn>
        TI* dqp = (TI*)a.dq + (tok0 + (size_t)tp * H) * D;
#pragma unroll
        for (int m = 0; m < EPW; m++) {
            const float r = qq < 1e-12f ? qi * dqn[m] : qi * (dqn[m] - (qe[m] * qi) * pr);   // |q| < 1e-6: no projection
            st1<TI>(dqp + lane + 64 * m, r);
        }
        if (frt && lane == 0) {
            float f = 0.f;
#pragma unroll
            for (int w = 0; w < CHAIN_WAVES; w++) f += s_pfr[pp][w];
            a.dfr[tok0 + (size_t)tp * H] = f;
        }
    };

    float dtemp_acc = 0.f, dfr_acc = 0.f;
    load_chunk(0);
    store_chunk(0);
    __syncthreads();
    load_chunk(1);
    int par = 0, j = 0, buf = 0, fin_wave = 0;
    for (int s = 0; s < T; s++) {
        const int t = T - 1 - s;
        const int amv = __builtin_amdgcn_readfirstlane(s_am[buf][j]);
        const float g = s_g[buf][j];
        const float frv = frt ? s_fr[buf][j] : fr_s;
        const float omw = 1.f - g;
        // undo this step's write: the written row goes back to its logged pre-write key and occupancy
        if (amv >= R.rowbase && amv < R.rowbase + P) {
            const int sl = amv & (P - 1);
            float kv[EPL];
            ld_slice<EPL>(kv, &s_ko[buf][j][0], c);
            float part = 0.f;
#pragma unroll
            for (int jr = 0; jr < P; jr++) {
                if (jr == sl) {
#pragma unroll
                    for (int e = 0; e < EPL; e++) { K[jr][e] = kv[e]; part = fmaf(kv[e], kv[e], part); }
                }
            }
            const float kk = rowsum16(part);
            if (R.n_me == amv) {
                o_me = s_oo[buf][j];
                kinv_me = rsq_clamped(kk);
            }
        }
        const float cs = valid_me ? s_cs[buf][j][R.n_me] : 0.f;   // the forward's cosine of this row
        const bool taken = valid_me && o_me >= eps;
        float z, dw;
        if constexpr (OCCB) {
            z = temp * cs - (taken ? frv : 0.f);
            dw = valid_me ? s_dn[buf][j][R.n_me] : 0.f;
        } else {
            z = temp * cs - frv * o_me;
            dw = (valid_me ? s_dn[buf][j][R.n_me] : 0.f) + (1.f - o_me) * dO_me;
        }
        {   // this wave's softmax partials over occupied rows (each row counted at its primary lane), and
            // its lowest free row with that row's z and dw
            const float zo = taken ? z : -INFINITY;
            const float wm = wavemax(zo);
            const float e = (taken && R.prim) ? __expf(z - wm) : 0.f;
            const float S = wavesum(e), SD = wavesum(e * dw);
            const u64 mf = __ballot(valid_me && !taken);
            int fo = -1;
            float fz = 0.f, fd = 0.f;
            if (mf) {
                const int lf = __builtin_ctzll(mf);
                fo = row_of_lane<P>(wave, lf);
                fz = readlanef(z, lf);
                fd = readlanef(dw, lf);
            }
            if (lane == 0) {
                *reinterpret_cast<float4*>(&s_st[par][wave][0]) = make_float4(wm, S, SD, __int_as_float(fo));
                *reinterpret_cast<float2*>(&s_st[par][wave][4]) = make_float2(fz, fd);
            }
        }
        if (j == CT - 2) {
            store_chunk(buf ^ 1);
            load_chunk(s / CT + 2);
        }
        __syncthreads();
        if (s > 0 && wave == fin_wave) finalize(s - 1);
        if (s > 0 && ++fin_wave == CHAIN_WAVES) fin_wave = 0;
        float4 st0[CHAIN_WAVES];
        float2 st1[CHAIN_WAVES];
#pragma unroll
        for (int w = 0; w < CHAIN_WAVES; w++) {
            st0[w] = *reinterpret_cast<const float4*>(&s_st[par][w][0]);
            st1[w] = *reinterpret_cast<const float2*>(&s_st[par][w][4]);
        }
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < CHAIN_WAVES; w++) M = fmaxf(M, st0[w].x);
        float FZ = 0.f, FD = 0.f;
        int FO = -1;
#pragma unroll
        for (int w = 0; w < CHAIN_WAVES; w++) {
            const int f2 = __float_as_int(st0[w].w);
            const bool tf = f2 >= 0 && FO < 0;
            FO = tf ? f2 : FO;
            FZ = tf ? st1[w].x : FZ;
            FD = tf ? st1[w].y : FD;
        }
        if (FO >= 0) M = fmaxf(M, FZ);                       // the first free row competes too
        float SS = 0.f, SSD = 0.f;
#pragma unroll
        for (int w = 0; w < CHAIN_WAVES; w++) {
            const float sc = st0[w].x == -INFINITY ? 0.f : __expf(st0[w].x - M);
            SS = fmaf(st0[w].y, sc, SS);
            SSD = fmaf(st0[w].z, sc, SSD);
        }
        if (FO >= 0) {
            const float ef = __expf(FZ - M);
            SS += ef;
            SSD = fmaf(ef, FD, SSD);
        }
        const float sa = g * SSD / SS;                       // sum_n asoft_n * g * dw_n
        const bool elig = taken || (valid_me && R.n_me == FO);
        const float as = elig ? __expf(z - M) / SS : 0.f;
        const float dz = as * (g * dw - sa);
        const size_t ix = tok0 + (size_t)t * H;
        if (R.n_me == amv && R.prim) a.dg[ix] = dw;
        float frp = 0.f;
        if (R.prim) {
            dtemp_acc = fmaf(dz, cs, dtemp_acc);
            if constexpr (OCCB) frp = taken ? -dz : 0.f;
            else frp = -o_me * dz;
        }
        if constexpr (!OCCB) dO_me = (R.n_me == amv ? omw : 1.f) * dO_me - frv * dz;
        // dqn partial: sum over this row group's rows of dz kinv K_n, then over the wave's 4 row groups.
        // Each row's coefficient goes through LDS to the 16 lanes holding that row (same wave: a wave
        // barrier orders the write and the reads).
        if (R.prim) s_cf[R.n_me] = dz * kinv_me;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float cf[P];
#pragma unroll
        for (int jr = 0; jr < P; jr++) cf[jr] = s_cf[R.rowbase + jr];
        float pq[EPL];
#pragma unroll
        for (int e = 0; e < EPL; e++) pq[e] = 0.f;
#pragma unroll
        for (int jr = 0; jr < P; jr++) {
#pragma unroll
            for (int e = 0; e < EPL; e++) pq[e] = fmaf(cf[jr], K[jr][e], pq[e]);
        }
#pragma unroll
        for (int e = 0; e < EPL; e++) pq[e] = sum4rows(pq[e]);
        frp = wavesum(frp);
        if (lane < 16) {
#pragma unroll
            for (int jj = 0; jj < EPL / 4; jj++)
                *reinterpret_cast<float4*>(&s_pq[par][wave][4 * c + 64 * jj]) =
                    make_float4(pq[4 * jj], pq[4 * jj + 1], pq[4 * jj + 2], pq[4 * jj + 3]);
        }
        if (lane == 0) { s_pfr[par][wave] = frp; dfr_acc += frp; }
        par ^= 1;
        if (++j == CT) { j = 0; buf ^= 1; }
    }
    __syncthreads();
    if (wave == fin_wave) finalize(T - 1);
    dtemp_acc = wavesum(dtemp_acc);
    if (lane == 0) { s_fin[0][wave] = dtemp_acc; s_fin[1][wave] = dfr_acc; }
    __syncthreads();
    if (tid == 0) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int w = 0; w < CHAIN_WAVES; w++) { s0 += s_fin[0][w]; s1 += s_fin[1][w]; }
        a.part[2 * (size_t)bh + 0] = s0;
        a.part[2 * (size_t)bh + 1] = s1;
    }
}

// ====================================================================================== chain_bwd_w
// Windowed address backward for the occ_bin mode.  With occupancy entering only through [o >= eps], the
// adjoint of step t needs no carry from step t + 1: given the occupancy at t, the logged cosines and Dn, every
// step's softmax adjoint is independent, and the keys enter only through dq.  The chain is cut into chunks of
// `wpc` 16-step windows, one workgroup each (grid (B*H, chunks)): the state at a chunk's end t_end is exact
// from the undo log -- row n holds kold (oold) of its first write at or after t_end, or kfin (ofin) when no
// later step writes it -- so the chunks run concurrently.  A workgroup of NW = D / 16 waves walks its windows
// in reverse, three barriers per window (B1 after S1, B2 after S4, B3 after S7):
//   S1  publish the prefetched window (Dn transposed to step-major, kold and query rows, the step scalars) and
//       derive from registers alone what the window's writes need: 1 / |kold_i| and 1 / |q_t| (lane sums over
//       each row's prefetch lanes), and from the step scalars, which every wave loads, each wave's share of the
//       occupancy masks (bit s of row n = row n occupied at step s) and per write the next write to the same
//       row inside the window and whether it is the row's first;
//   S4  the softmax adjoints of all 16 steps at once: step s is a group of NC = NT / 16 lanes (one or two DPP
//       rows), each lane RPC slot rows strided by NC, its cosines straight from its prefetch registers.  The
//       exponentials are shifted by the largest z over the eligible rows
//       (the occupied ones and the lowest free one, a step-group max); SS and sum e dw are step-group sums;
//       W[s][n] = temp dz_n goes to LDS; dgate = Dn of the written row; dfr in closed form over the occupied
//       rows; dtemp accumulates sum dz cs;
//   S6  dqn = W Kh on bf16 MFMA (v_mfma_f32_16x16x32_bf16) over operands split into two bf16 terms (hi*hi +
//       hi*lo + lo*hi, within about 2^-16 of the fp32 products), wave w owning dims [16 w, 16 w + 16).  The
//       normalised keys stay in LDS TRANSPOSED (dim-major hi and lo planes, row stride P = NR + 8): a lane's
//       8 consecutive rows of a k-block are one 16-byte read per plane, and so are its W operand's (the
//       reference's order: normalise, then contract, slotkern_kvt.py:86-90);
//   S7  the undo, every write at once: x_i = Kh(kold_i); the key after write i is Kh(kold_j) of the next write
//       j to the same row in the window, else the window-end key; delta_i = x_i - after_i.  Then each row the
//       window wrote takes x of its FIRST write: the keys at the window start;
//   S8  the rewritten rows' correction, sum_{s >= t} W[t][a_s] delta_s, as a 16 x 16 x 16 MFMA (S6 and S8 produce
//       dqn transposed, so each lane holds four consecutive dims of one step and stores them at once);
//   S9  dq = qinv (dqn - qhat <qhat, dqn>) (qinv dqn where |q| < 1e-6), one LDS exchange for the dot products.
// What S8 and S9 need from LDS that the next window's S1 and S4 overwrite is read into registers before B3, and
// the undo deltas have their own buffer, so no barrier closes a window.
// Every Kh value is an element times rsq_clamped(|row|^2), |row|^2 summed in one fixed order (sq4 of each
// lane's 4-element piece, then lanesum over the row's D / 4 lanes) wherever a key is normalised, so a chunk
// starts from bitwise the keys the reverse walk of the whole chain would hold there: the results do not depend
// on the chunking.
#define WIN 16

// Reductions over the NC lanes of one step in the softmax phase: one DPP row (NC = 16) or two (NC = 32, the
// row pair joined by a permlane16 swap); every lane of the group gets the bitwise-same result.
template <int NC> __device__ __forceinline__ float step_sum(float v) {
    v = rowsum16(v);
    if constexpr (NC == 32) {
        auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    return v;
}
template <int NC> __device__ __forceinline__ float step_max(float v) {
    v = rowmax16(v);
    if constexpr (NC == 32) {
        auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    }
    return v;
}
template <int NC> __device__ __forceinline__ int step_min(int v) {
    v = min(v, __builtin_amdgcn_update_dpp(0, v, SLOT_DPP_XOR1, 0xF, 0xF, false));
    v = min(v, __builtin_amdgcn_update_dpp(0, v, SLOT_DPP_XOR2, 0xF, 0xF, false));
    v = min(v, __builtin_amdgcn_update_dpp(0, v, SLOT_DPP_HMIR, 0xF, 0xF, false));
    v = min(v, __builtin_amdgcn_update_dpp(0, v, SLOT_DPP_MIR, 0xF, 0xF, false));
    if constexpr (NC == 32) {
        auto p = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
        v = min((int)p[0], (int)p[1]);
    }
    return v;
}

// The lowest index over a step's lanes with two payload values: at every stage a lane takes its partner's
// triple when the partner's index is smaller (indices are distinct or equal-with-equal-payload).
template <int CTRL> __device__ __forceinline__ void argmin_stage(int& i, float& x, float& y) {
    const int i2 = __builtin_amdgcn_update_dpp(0, i, CTRL, 0xF, 0xF, false);
    const float x2 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
    const float y2 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(y), CTRL, 0xF, 0xF, false));
    const bool t = i2 < i;
    i = t ? i2 : i; x = t ? x2 : x; y = t ? y2 : y;
}
template <int NC> __device__ __forceinline__ void step_argmin(int& i, float& x, float& y) {
    argmin_stage<SLOT_DPP_XOR1>(i, x, y);
    argmin_stage<SLOT_DPP_XOR2>(i, x, y);
    argmin_stage<SLOT_DPP_HMIR>(i, x, y);
    argmin_stage<SLOT_DPP_MIR>(i, x, y);
    if constexpr (NC == 32) {
        auto pi = __builtin_amdgcn_permlane16_swap((uint32_t)i, (uint32_t)i, false, false);
        auto px = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        auto py = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
        const bool lo = (int)pi[0] <= (int)pi[1];
        i = lo ? (int)pi[0] : (int)pi[1];
        x = __uint_as_float(lo ? px[0] : px[1]);
        y = __uint_as_float(lo ? py[0] : py[1]);
    }
}

// Sum over aligned groups of L consecutive lanes (L = 8, 16 or 32), the bitwise-same result at every lane of a
// group: each stage adds the same two partial sums (IEEE addition is commutative).
template <int L> __device__ __forceinline__ float lanesum(float v) {
    static_assert(L == 8 || L == 16 || L == 32, "lane group");
    v += dppf<SLOT_DPP_XOR1>(v);
    v += dppf<SLOT_DPP_XOR2>(v);
    v += dppf<SLOT_DPP_HMIR>(v);
    if constexpr (L >= 16) v += dppf<SLOT_DPP_MIR>(v);
    if constexpr (L == 32) {
        auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    return v;
}
// An empty use of values in vector registers: the loads that produce them are issued before it on every path,
// so a group of LDS reads is issued together and waited on once (the compiler otherwise sinks each read into
// the branch of the select that consumes it, one wait per read).
__device__ __forceinline__ void keep() {}
template <typename T, typename... Ts> __device__ __forceinline__ void keep(T& v, Ts&... r) {
    asm volatile("" : "+v"(v));
    keep(r...);
}
// The squares of a 4-element key piece, summed in one fixed order (the first term of every key norm).
__device__ __forceinline__ float sq4(float4 x) { return fmaf(x.w, x.w, fmaf(x.z, x.z, fmaf(x.y, x.y, x.x * x.x))); }

// Two-term bfloat16 split of fp32 operands: x = hi + lo + r with hi = bf16(x), lo = bf16(x - hi) (x - hi is exact
// in fp32), |r| <= 2^-18 |x|.  hi*hi + hi*lo + lo*hi on bf16 MFMAs then carries a product to within about
// 3 * 2^-18 of its fp32 value (the dropped lo*lo is below 2^-18), at 3 bf16 MFMAs of 16 cycles per 32-deep
// k-block where fp32 MFMAs take 8 of 32 cycles.  Pairs are packed element 0 in bits 0-15.  The inputs pass an
// empty asm first: x is then the rounded fp32 value on every path (a product feeding x - hi would otherwise be
// contracted into an fma on some paths and not on others, and the same key would split differently).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ void split_bf2(float x0, float x1, u32& hi, u32& lo) {
    asm volatile("" : "+v"(x0), "+v"(x1));
    hi = pack_bf16x2(x0, x1);
    lo = pack_bf16x2(x0 - __uint_as_float(hi << 16), x1 - __uint_as_float(hi & 0xffff0000u));
}
__device__ __forceinline__ float join_bf(bf16_t hi, bf16_t lo) { return bf2f(hi) + bf2f(lo); }
__device__ __forceinline__ f32x4 mfma_bf32(const uint4& a, const uint4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
}

template <int D, int RPL, typename TI>
__global__ __launch_bounds__(4 * D) void chain_bwd_w(ChainBwdArgs a) {
    constexpr int NW = D / 16;                          // waves: wave w owns dims [16 w, 16 w + 16) in S6, S8, S9
    constexpr int NT = 64 * NW;
    constexpr int NR = 64 * RPL;                        // slot-row capacity
    constexpr int KG = NR / 4;                          // S6: rows per MFMA lane group (k = 8 g .. 8 g + 7 of a block)
    constexpr int KB = NR / 32;                         // S6: 32-deep bf16 k-blocks over the rows
    // LDS: 4-byte accesses are served 32 lanes per pass over 32 banks, 16-byte accesses 16 lanes per pass over 64
    constexpr int P = NR + 8;                           // transposed key planes' stride (bf16), 400 B = 144 mod 256 at
    constexpr int SW = NR + 8;                          // NR 192: S6's 16 dims / steps per 16-byte pass on 16 distinct
                                                        // 16-byte bank groups; W's planes likewise
    constexpr int SD = NR + 4;                          // Dn stride (fp32; its columns swizzled, dnc below)
    constexpr int NC = NT / WIN;                        // lanes per step in the softmax phase
    constexpr int RPC = NR / NC;                        // slot rows per lane there (groups of 4, then a pair)
    constexpr int KOS = D + 8;                          // kold and undo-delta row strides, 8 mod 32: a 4-byte pass of
    constexpr int DEL = D + 8;                          // the undo (4 writes x 8 dims) hits 32 distinct banks
    constexpr int QS = D + 4;                           // query row stride: S9's four steps per wave on distinct banks
    constexpr int DPT = D / NC;                         // dims per lane in the undo (4)
    constexpr int EPU = 16 / (int)sizeof(TI);           // query elements per 16-byte piece
    constexpr int KLR = D / 4;                          // lanes per kold row in the prefetch (one float4 each)
    constexpr int QLR = D / EPU;                        // lanes per query row in the prefetch (one 16-byte piece)
    constexpr int QL0 = NT - WIN * QLR;                 // the query rows' first lane (whole waves at the end)
    constexpr int UDN = (4 * NR + NT - 1) / NT;         // Dn float4 pieces per lane in the prefetch (4 per row)
    constexpr int Q4 = RPC / 4, R2 = (RPC % 4) / 2;     // softmax lane rows: Q4 groups of 4, then R2 pairs
    // Dn column swizzle: row n of step s sits at column n ^ 8 [s & 8].  The transposing publish stores rows n .. n + 7
    // at steps i, i + 4, i + 8, i + 12 in one pass: without it steps i and i + 8 share banks (2-way); the XOR
    // moves whole 4-row groups, so the softmax phase's 16-byte reads of 4 rows stay contiguous
    auto dnc = [](int s, int n) { return n ^ (s & 8); };
    constexpr bool BF = sizeof(TI) == 2;
    static_assert(DPT == 4 && NR % 32 == 0 && WIN * KLR == NT && WIN * QLR <= NT && (WIN * QLR) % 64 == 0 &&
                  RPC == 4 * Q4 + 2 * R2 && (4 * NR) % 64 == 0 && RPL + 1 <= NW, "layout assumptions");
    __shared__ __align__(16) bf16_t sKT[2][D * P];      // normalised keys, transposed, split: [0] hi, [1] lo
    __shared__ __align__(16) bf16_t sW[2][WIN * SW];    // W = temp dz [step][row], split likewise
    __shared__ __align__(16) float sDN[WIN * SD];       // Dn [step][row]
    __shared__ __align__(16) float sDel[WIN * DEL];     // undo deltas [write][dim]
    __shared__ __align__(16) float sKO[WIN * KOS];      // kold rows of the window's writes
    __shared__ __align__(16) float sQ[WIN * QS];        // query rows
    __shared__ u32 s_tkm[NR];                           // per row: bit s = occupied at window step s
    __shared__ u32 s_sc[4 * WIN];                       // step scalars (address, oold, gate, fr; 16 each)
    __shared__ float s_kil[WIN], s_qi[WIN], s_pr[WIN];
    __shared__ float s_dgf[2][WIN];                     // per step: dgate and the per-token dfr, stored by wave 0
    __shared__ int s_nx[WIN], s_first[WIN];
    __shared__ float s_fin[2][NW];
    const int* s_am = reinterpret_cast<const int*>(s_sc);
    const float* s_g = reinterpret_cast<const float*>(s_sc + 2 * WIN);
    const float* s_fr = reinterpret_cast<const float*>(s_sc + 3 * WIN);

    const int T = a.T, H = a.H, N = a.N;
    const int bh = blockIdx.x, b = bh / H, h = bh - b * H;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const TI* __restrict__ qp = (const TI*)a.q;
    const size_t tok0 = (size_t)b * T * H + h;
    const float temp = a.temp[0];
    const float fr_s = a.frt ? 0.f : a.fr[0];
    const float eps = a.eps;
    const bool frt = a.frt != 0;
    const int d0 = 16 * wave;

    // ---- this chunk: windows [m_lo, m_hi), steps before t_end.  s_fw[n]: the first step at or after t_end
    // that writes row n (T: none), from the address log by LDS integer minima (order-independent)
    const int nwin = (T + WIN - 1) / WIN;
    const int m_lo = blockIdx.y * a.wpc, m_hi = min(nwin, m_lo + a.wpc);
    const int t_end = min(m_hi * WIN, T);
    // element (dim d, row n) of the split transposed keys, from the low 16 bits of each half
    auto st_kt = [&](int d, int n, u32 hi, u32 lo) {
        sKT[0][d * P + n] = (bf16_t)hi;
        sKT[1][d * P + n] = (bf16_t)lo;
    };
    int* s_fw = reinterpret_cast<int*>(&sW[0][0]);
    for (int n = tid; n < NR; n += NT) s_fw[n] = T;
    __syncthreads();
    for (int t = t_end + tid; t < T; t += NT) atomicMin(&s_fw[min(max(a.am[tok0 + (size_t)t * H], 0), NR - 1)], t);
    __syncthreads();
    // the keys at t_end (kold of the row's first later write, else kfin), normalised, transposed into sKT.
    // KLR lanes per row, lane l holding elements 4 l .. 4 l + 3: sq4 per lane, then lanesum<KLR>, the one order
    // of every key norm in this kernel
    {
        constexpr int NP = NR / (NT / KLR);              // row passes; every pass's piece is loaded first
        const int l = tid % KLR;
        float4 xs[NP];
#pragma unroll
        for (int p = 0; p < NP; p++) {
            const int row = (NT / KLR) * p + tid / KLR;
            xs[p] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (row < N) {
                const int fw = s_fw[row];
                const float* src = fw < T ? a.kold + (tok0 + (size_t)fw * H) * D : a.kfin + ((size_t)bh * N + row) * D;
                xs[p] = ld4(src + 4 * l);
            }
        }
#pragma unroll
        for (int p = 0; p < NP; p++) {
            const int row = (NT / KLR) * p + tid / KLR;
            const float ki = rsq_clamped(lanesum<KLR>(sq4(xs[p])));
            u32 h01, l01, h23, l23;
            split_bf2(xs[p].x * ki, xs[p].y * ki, h01, l01);
            split_bf2(xs[p].z * ki, xs[p].w * ki, h23, l23);
            st_kt(4 * l + 0, row, h01, l01);
            st_kt(4 * l + 1, row, h01 >> 16, l01 >> 16);
            st_kt(4 * l + 2, row, h23, l23);
            st_kt(4 * l + 3, row, h23 >> 16, l23 >> 16);
        }
    }
    // the occupancy at t_end, likewise, held in a register by row n's mask lane (thread n; NR < NT): the mask loop
    // below carries it from each window's end to its start
    float o_row = 0.f;
    if (tid < NR) {
        const int fw = tid < N ? s_fw[tid] : T;
        o_row = tid >= N ? 0.f : (fw < T ? a.oold[tok0 + (size_t)fw * H] : a.ofin[(size_t)bh * N + tid]);
    }
    __syncthreads();

    // ---- window prefetch into registers, 16 bytes per lane wherever the layout allows (the address unit takes
    // about as long per load instruction whatever its width): the cosines as the softmax phase's lanes hold them
    // (step tid / NC; rows 4 (r + NC k) .. + 3 for k < Q4, then 4 NC Q4 + 2 r, + 1); Dn in 4-step pieces of a row
    // (its 16 steps are 64 contiguous bytes), transposed through LDS; one float4 of a kold row and one 16-byte piece
    // of a query row per lane; the step scalars in lanes 16 k + i (k: address, oold, gate, fr) of the waves that
    // derive the occupancy masks and same-row links from them.  Rows whose pieces are not 16-byte aligned (N or T
    // not a multiple of 4) or cross the end take scalar loads.  Each value is loaded under one condition into a
    // register zeroed beforehand (address: -1), so the load is an exec-masked instruction whose result nothing
    // waits for until the consumer.
    const int s4 = tid / NC, r4 = tid % NC;
    const bool n4 = (N & 3) == 0, n2 = (N & 1) == 0, t4 = (T & 3) == 0;
    float ncs[RPC];
    float4 ndn[UDN];
    float4 nko;
    uint4 nq = make_uint4(0u, 0u, 0u, 0u);
    u32 nsc = 0u;
    // A window's loads come in NPART parts, issued between the next window's MFMA groups (all at once, the
    // loads of the eight waves queue in the address unit for longer than the matrix phase lasts).
    constexpr int NPART = 5;
    auto load_part = [&](int m, int part) {
        const int t0 = m * WIN, nt = min(WIN, T - t0);
        if (part == 3 || part == 4) {                   // the cosines: the groups of 4, then the pair
            const float* csb = a.cslog + ((size_t)bh * T + t0) * N + (u32)(s4 * N);
            const bool sok = s4 < nt;
            if (part == 3) {
#pragma unroll
                for (int k = 0; k < Q4; k++) {
                    const int n = 4 * (r4 + NC * k);
                    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (sok && n4 && n + 3 < N) x = ld4(csb + n);
                    else if (sok && !(n4 && n + 3 < N)) {
                        if (n < N) x.x = csb[n];
                        if (n + 1 < N) x.y = csb[n + 1];
                        if (n + 2 < N) x.z = csb[n + 2];
                        if (n + 3 < N) x.w = csb[n + 3];
                    }
                    ncs[4 * k] = x.x; ncs[4 * k + 1] = x.y; ncs[4 * k + 2] = x.z; ncs[4 * k + 3] = x.w;
                }
            } else if (R2) {
                const int n = 4 * NC * Q4 + 2 * r4;
                float2 x = make_float2(0.f, 0.f);
                if (sok && n2 && n + 1 < N) x = *reinterpret_cast<const float2*>(csb + n);
                else if (sok && !(n2 && n + 1 < N)) {
                    if (n < N) x.x = csb[n];
                    if (n + 1 < N) x.y = csb[n + 1];
                }
                ncs[4 * Q4] = x.x; ncs[4 * Q4 + 1] = x.y;
            }
        }
        if (part == 1 || part == 2) {                   // Dn: piece u = 4 n + q holds steps 4 q .. 4 q + 3 of row n
            const float* dnb = a.dn + (size_t)bh * N * T + t0;
#pragma unroll
            for (int u2 = part == 1 ? 0 : (UDN + 1) / 2; u2 < (part == 1 ? (UDN + 1) / 2 : UDN); u2++) {
                const int u = tid + NT * u2, n = u >> 2, i = 4 * (u & 3);
                const bool live = u < 4 * NR && n < N;
                const float* src = dnb + (size_t)n * T + i;
                float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
                if (live && t4 && i + 3 < nt) x = ld4(src);
                else if (live && !(t4 && i + 3 < nt)) {
                    if (i < nt) x.x = src[0];
                    if (i + 1 < nt) x.y = src[1];
                    if (i + 2 < nt) x.z = src[2];
                    if (i + 3 < nt) x.w = src[3];
                }
                ndn[u2] = x;
            }
        }
        if (part != 0) return;
        {
            const int i = tid / KLR;
            nko = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < nt) nko = ld4(a.kold + (tok0 + (size_t)(t0 + i) * H) * D + 4 * (tid % KLR));
        }
        if (tid >= QL0) {                               // whole waves: the last ones (the first hold the step scalars)
            const int i = (tid - QL0) / QLR;
            nq = make_uint4(0u, 0u, 0u, 0u);
            if (i < nt) nq = *reinterpret_cast<const uint4*>(qp + (tok0 + (size_t)(t0 + i) * H) * D + EPU * ((tid - QL0) % QLR));
        }
        if (tid < 64 * (RPL + 1)) {                     // the mask and link waves; one load per 16-lane kind (a
            const int kind = lane >> 4, i = lane & 15;  // per-lane choice of base pointer compiles to a load of it)
            const size_t ix = tok0 + (size_t)(t0 + i) * H;
            nsc = kind == 0 ? 0xffffffffu : 0u;
            if (i < nt) {
                if (kind == 0) nsc = (u32)a.am[ix];
                else if (kind == 1) nsc = __float_as_uint(a.oold[ix]);
                else if (kind == 2) nsc = __float_as_uint(a.gate[ix]);
                else if (frt) nsc = __float_as_uint(a.fr[ix]);
            }
        }
    };

    float dtemp_acc = 0.f, dfr_acc = 0.f;
#pragma unroll
    for (int pp = 0; pp < NPART; pp++) load_part(m_hi - 1, pp);
    for (int m = m_hi - 1; m >= m_lo; m--) {
        const int t0 = m * WIN, nt = min(WIN, T - t0);
        // lane indices re-derived from an opaque copy every window: comparisons on them are then not loop
        // invariant, so the compiler does not hoist dozens of 64-bit lane masks into (spilled) scalar registers
        u32 tidw;
        asm volatile("v_mov_b32 %0, %1" : "=v"(tidw) : "v"(tid));
        const int lanew = (int)(tidw & 63u), cw = lanew & 15, grpw = lanew >> 4;
        // S1: publish the window, with everything about its writes that needs no other wave's data
#pragma unroll
        for (int u2 = 0; u2 < UDN; u2++) {
            const u32 u = tidw + NT * u2;
            if (u < 4 * NR) {                            // whole waves
                const u32 n = u >> 2, i = 4 * (u & 3);
                sDN[(i + 0) * SD + dnc(i + 0, n)] = ndn[u2].x;
                sDN[(i + 1) * SD + dnc(i + 1, n)] = ndn[u2].y;
                sDN[(i + 2) * SD + dnc(i + 2, n)] = ndn[u2].z;
                sDN[(i + 3) * SD + dnc(i + 3, n)] = ndn[u2].w;
            }
        }
        {                                                // kold rows and 1 / |kold_i|
            const int i = (int)(tidw / KLR), l = (int)(tidw % KLR);
            *reinterpret_cast<float4*>(&sKO[i * KOS + 4 * l]) = nko;
            const float ki = rsq_clamped(lanesum<KLR>(sq4(nko)));
            if (l == 0) s_kil[i] = ki;
        }
        if (tidw >= (u32)QL0) {      // query rows and 1 / max(|q_t|, 1e-6), negative where |q_t|^2 < 1e-12 (no projection)
            const int i = (int)((tidw - QL0) / QLR), l = (int)((tidw - QL0) % QLR);
            stage_store(&sQ[i * QS + EPU * l], nq, BF);
            float qq;
            if constexpr (BF) {
                const u32 w4[4] = {nq.x, nq.y, nq.z, nq.w};
                qq = 0.f;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float lo = __uint_as_float(w4[k] << 16), hi = __uint_as_float(w4[k] & 0xffff0000u);
                    qq = fmaf(lo, lo, qq);
                    qq = fmaf(hi, hi, qq);
                }
            } else {
                qq = sq4(make_float4(__uint_as_float(nq.x), __uint_as_float(nq.y), __uint_as_float(nq.z),
                                     __uint_as_float(nq.w)));
            }
            qq = lanesum<QLR>(qq);
            if (l == 0) s_qi[i] = qq < 1e-12f ? -rsq_clamped(qq) : rsq_clamped(qq);
        }
        if (tidw < 64 * (RPL + 1)) {                     // waves 0 .. RPL (whole waves) hold the step scalars: wave 0
            const int wv = (int)(tidw >> 6);             // publishes the block's copy; each takes the addresses and
            if (wv == 0) s_sc[lanew] = nsc;              // pre-write occupancies as scalars from its own lanes
            int ai[WIN];
            float oi[WIN];
#pragma unroll
            for (int i = 0; i < WIN; i++) {
                ai[i] = __builtin_amdgcn_readlane((int)nsc, i);
                oi[i] = __int_as_float(__builtin_amdgcn_readlane((int)nsc, WIN + i));
            }
            if (wv < RPL) {                              // occupancy masks, row n = 64 wave + lane: over the window's
                const int n = (int)tidw;                 // 16 steps backwards from the window-end occupancy, o becomes
                float o = o_row;                         // the pre-write occupancy at each write to the row, and at
                u32 mk = 0u;                             // the end the window-start occupancy (the next window's end)
#pragma unroll
                for (int i = WIN - 1; i >= 0; i--) {
                    o = ai[i] == n ? oi[i] : o;
                    mk |= (n < N && o >= eps ? 1u : 0u) << i;
                }
                s_tkm[n] = mk;
                o_row = o;
            } else if (lanew < WIN) {                    // per write: the next write to the same row inside the
                const int i = lanew, me = (int)nsc;      // window, and whether it is the row's first
                int nx = -1;
                bool first = true;
#pragma unroll
                for (int j = WIN - 1; j >= 0; j--) {
                    if (j > i && ai[j] == me) nx = j;    // ends at the smallest such j
                    if (j < i && ai[j] == me) first = false;
                }
                s_nx[i] = i < nt ? nx : -1;
                s_first[i] = (i < nt && first) ? 1 : 0;
            }
        }
        __syncthreads();                                                      // B1
        // S4: the softmax adjoint of every step: step s = lanes [NC s, NC s + NC), rows as in the prefetch.  The
        // addresses S8 needs (steps 4 kc + grp) are read with S4's own operands, so that S8's W reads go out at once
        int as8[4];
        {
            const int s = (int)(tidw / NC), r = (int)(tidw % NC);
            const bool live = s < nt;
#pragma unroll
            for (int kc = 0; kc < 4; kc++) as8[kc] = s_am[4 * kc + grpw];
            const float g = s_g[s], frv = frt ? s_fr[s] : fr_s;
            auto rowof = [&](int j) { return j < 4 * Q4 ? 4 * (r + NC * (j >> 2)) + (j & 3) : 4 * NC * Q4 + 2 * r + j - 4 * Q4; };
            float dw[RPC];
            u32 tkm[RPC];
#pragma unroll
            for (int k = 0; k < Q4; k++) {
                const float4 x = ld4(&sDN[s * SD + dnc(s, rowof(4 * k))]);
                const uint4 y = *reinterpret_cast<const uint4*>(&s_tkm[rowof(4 * k)]);
                dw[4 * k] = x.x; dw[4 * k + 1] = x.y; dw[4 * k + 2] = x.z; dw[4 * k + 3] = x.w;
                tkm[4 * k] = y.x; tkm[4 * k + 1] = y.y; tkm[4 * k + 2] = y.z; tkm[4 * k + 3] = y.w;
            }
            if constexpr (R2 > 0) {
                const float2 x = *reinterpret_cast<const float2*>(&sDN[s * SD + dnc(s, rowof(4 * Q4))]);
                const uint2 y = *reinterpret_cast<const uint2*>(&s_tkm[rowof(4 * Q4)]);
                dw[4 * Q4] = x.x; dw[4 * Q4 + 1] = x.y; tkm[4 * Q4] = y.x; tkm[4 * Q4 + 1] = y.y;
            }
            keep(as8[0], as8[1], as8[2], as8[3]);
            u32 tk = 0u, rows = 0u;                      // occupied at step s; below N
#pragma unroll
            for (int j = 0; j < RPC; j++) {
                tk |= ((tkm[j] >> s) & 1u) << j;
                rows |= (rowof(j) < N ? 1u : 0u) << j;
            }
            const float* cs = ncs;
            // the lowest free row of the step with its z and Dn, and the largest z over the occupied rows
            const u32 fm = rows & ~tk;
            const int jf = fm ? (int)__builtin_ctz(fm) : 0;
            float zf = 0.f, FD = 0.f, mz = -INFINITY;
#pragma unroll
            for (int j = 0; j < RPC; j++) {
                zf = j == jf ? temp * cs[j] : zf;
                FD = j == jf ? dw[j] : FD;
                if ((tk >> j) & 1u) mz = fmaxf(mz, fmaf(temp, cs[j], -frv));
            }
            int ff = INT_MAX;                            // rows increase with j: the first free j is the lowest
#pragma unroll
            for (int j = RPC - 1; j >= 0; j--) ff = j == jf && fm ? rowof(j) : ff;
            step_argmin<NC>(ff, zf, FD);
            mz = step_max<NC>(mz);
            const bool hasf = ff < N;
            if (!hasf) { zf = -INFINITY; FD = 0.f; }
            const float M = fmaxf(mz, zf);
            float ev[RPC], s0 = 0.f, s1 = 0.f;
#pragma unroll
            for (int j = 0; j < RPC; j++) {
                const float e = ((tk >> j) & 1u) ? __expf(fmaf(temp, cs[j], -frv) - M) : 0.f;
                ev[j] = e;
                s0 += e;
                s1 = fmaf(e, dw[j], s1);
            }
            const float SSt = step_sum<NC>(s0), SSDt = step_sum<NC>(s1);
            const float ef = hasf ? __expf(zf - M) : 0.f;
            const float SS = SSt + ef, SSD = fmaf(ef, FD, SSDt);
            const float rss = live ? __builtin_amdgcn_rcpf(SS) : 0.f, sa = (g * SSD) * rss;
            float dt = 0.f, wv[RPC];
#pragma unroll
            for (int j = 0; j < RPC; j++) {
                const float as = ((tk >> j) & 1u) ? ev[j] * rss : (rowof(j) == ff ? ef * rss : 0.f);
                const float dz = as * (g * dw[j] - sa);
                dt = fmaf(dz, cs[j], dt);
                wv[j] = temp * dz;
            }
#pragma unroll
            for (int k = 0; k < Q4; k++) {
                uint2 hi, lo;
                split_bf2(wv[4 * k], wv[4 * k + 1], hi.x, lo.x);
                split_bf2(wv[4 * k + 2], wv[4 * k + 3], hi.y, lo.y);
                *reinterpret_cast<uint2*>(&sW[0][s * SW + rowof(4 * k)]) = hi;
                *reinterpret_cast<uint2*>(&sW[1][s * SW + rowof(4 * k)]) = lo;
            }
            if constexpr (R2 > 0) {
                u32 hi, lo;
                split_bf2(wv[4 * Q4], wv[4 * Q4 + 1], hi, lo);
                *reinterpret_cast<u32*>(&sW[0][s * SW + rowof(4 * Q4)]) = hi;
                *reinterpret_cast<u32*>(&sW[1][s * SW + rowof(4 * Q4)]) = lo;
            }
            dtemp_acc += dt;
            const float pstep = temp * step_sum<NC>(dt);        // <qhat_s, dqn_s> = temp sum_n dz_n cs_n
            if (r == 0) {
                const float dfl = -(g * SSDt - sa * SSt) * rss;
                s_pr[s] = pstep;
                s_dgf[0][s] = sDN[s * SD + dnc(s, max(s_am[s], 0))];   // dgate of the written row: its Dn entry
                s_dgf[1][s] = dfl;
                if (live && !frt) dfr_acc += dfl;
            }
        }
        __syncthreads();                                                      // B2
        // S8's B operand, W[c][a_s] for s = 4 kc + grp >= c, and S9's operands (the query of step c at this lane's
        // four dims), read before B3: past it the next window's publish may overwrite them
        float av8[4], qsv, prv;
        float4 qv;
        {
            qv = ld4(&sQ[cw * QS + d0 + 4 * grpw]);
            qsv = s_qi[cw];
            prv = s_pr[cw];
#pragma unroll
            for (int kc = 0; kc < 4; kc++) {
                const int o = cw * SW + min(max(as8[kc], 0), NR - 1);
                av8[kc] = join_bf(sW[0][o], sW[1][o]);
            }
            keep(av8[0], av8[1], av8[2], av8[3]);
#pragma unroll
            for (int kc = 0; kc < 4; kc++) {
                const int s = 4 * kc + grpw;
                av8[kc] = (s < nt && s >= cw) ? av8[kc] : 0.f;
            }
        }
        // S6: dqn^T = Kh^T W^T over every row for this wave's dims (keys as the A operand, so lane (c, g) ends with
        // dims 4 g .. 4 g + 3 of step c) on split bf16 operands: hi*hi, hi*lo and lo*hi in three accumulation
        // chains, k-block j of lane group g = rows KG g + 8 j .. + 7, one 16-byte read per operand plane, each
        // block's reads issued one block ahead.  S5, the prefetch of the next (earlier) window, is issued part by
        // part between the MFMA blocks
        f32x4 acc = {0.f, 0.f, 0.f, 0.f}, acc2 = {0.f, 0.f, 0.f, 0.f}, acc3 = {0.f, 0.f, 0.f, 0.f};
        const bool pf = m > m_lo;
        const bf16_t* wh = &sW[0][cw * SW + KG * grpw];
        const bf16_t* wl = &sW[1][cw * SW + KG * grpw];
        const bf16_t* kh = &sKT[0][(d0 + cw) * P + KG * grpw];
        const bf16_t* kl = &sKT[1][(d0 + cw) * P + KG * grpw];
        auto ld8 = [](const bf16_t* p) { return *reinterpret_cast<const uint4*>(p); };
        uint4 ah = ld8(kh), al = ld8(kl), bh = ld8(wh), bl = ld8(wl);
#pragma unroll
        for (int j = 0; j < KB; j++) {
            uint4 nah = ah, nal = al, nbh = bh, nbl = bl;
            if (j + 1 < KB) {
                nah = ld8(kh + 8 * j + 8);
                nal = ld8(kl + 8 * j + 8);
                nbh = ld8(wh + 8 * j + 8);
                nbl = ld8(wl + 8 * j + 8);
            }
            if (pf && j < NPART) load_part(m - 1, j);
            acc = mfma_bf32(ah, bh, acc);
            acc2 = mfma_bf32(ah, bl, acc2);
            acc3 = mfma_bf32(al, bh, acc3);
            ah = nah; al = nal; bh = nbh; bl = nbl;
        }
#pragma unroll
        for (int pp = KB; pp < NPART; pp++)
            if (pf) load_part(m - 1, pp);
        // S7: the undo of every write at once: lane 128 w4 + 8 ui + g takes write ui, dims g + 8 (w4 + (D / 32) e).
        // A pass of 32 lanes is 4 writes x 8 dims: the column accesses of the transposed key planes (stride P per
        // dim) land on 8 bank groups per write, offset by the writes' (different) rows; the kold and delta rows on
        // 32 banks (both candidates for the key after each write are read, unconditionally, and selected)
        const int ui = (int)((tidw >> 3) & 15), ud = (int)(tidw & 7) + 8 * (int)(tidw >> 7);
        auto udim = [&](int e) { return ud + 8 * (D / 32) * e; };
        const bool uev = ui < nt;
        int uam = s_am[ui], unx = s_nx[ui], ufi = s_first[ui];
        float ki = s_kil[ui];
        keep(uam, unx, ufi, ki);
        const int uai = min(max(uam, 0), NR - 1), nxc = max(unx, 0);
        const bool ufirst = uev && ufi != 0;
        float ux[DPT];
        {
            float kn = s_kil[nxc], ko[DPT], kx[DPT], kt[DPT];
#pragma unroll
            for (int e = 0; e < DPT; e++) {
                const int d = udim(e);
                ko[e] = sKO[ui * KOS + d];
                kx[e] = sKO[nxc * KOS + d];
                kt[e] = join_bf(sKT[0][d * P + uai], sKT[1][d * P + uai]);
            }
            keep(kn, ko[0], ko[1], ko[2], ko[3], kx[0], kx[1], kx[2], kx[3], kt[0], kt[1], kt[2], kt[3]);
#pragma unroll
            for (int e = 0; e < DPT; e++) {
                ux[e] = ko[e] * ki;
                const float af = unx >= 0 ? kx[e] * kn : kt[e];
                sDel[ui * DEL + udim(e)] = uev ? ux[e] - af : 0.f;
            }
        }
        __syncthreads();                                                      // B3: every read of the window-end keys done
        if (tidw >= NT - 64 && lanew < 2 * WIN) {       // the steps' dgate (and per-token dfr), one store each, by the
            const int i = lanew & 15, k = lanew >> 4;   // last wave (the one with the shortest publish): read before
            const size_t ix = tok0 + (size_t)(t0 + i) * H;   // it reaches the next B1, past which S4 rewrites them
            const float v = s_dgf[k][i];
            if (i < nt && k == 0) a.dg[ix] = v;
            if (i < nt && k == 1 && frt) a.dfr[ix] = v;
        }
        if (ufirst) {
#pragma unroll
            for (int e = 0; e < DPT; e += 2) {
                u32 hi, lo;
                split_bf2(ux[e], ux[e + 1], hi, lo);
                st_kt(udim(e), uai, hi, lo);
                st_kt(udim(e + 1), uai, hi >> 16, lo >> 16);
            }
        }
        // S8: the rewritten rows' correction, sum_{s >= t} W[t][a_s] delta_s (rows of steps past the chain end
        // are zero deltas)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[r] += acc2[r] + acc3[r];
        float bv8[4];
#pragma unroll
        for (int kc = 0; kc < 4; kc++) bv8[kc] = sDel[(4 * kc + grpw) * DEL + d0 + cw];
        keep(bv8[0], bv8[1], bv8[2], bv8[3]);
#pragma unroll
        for (int kc = 0; kc < 4; kc++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(bv8[kc], av8[kc], acc, 0, 0, 0);
        // S9: dq = qinv (dqn - qhat <qhat, dqn>), or qinv dqn where |q| < 1e-6.  <qhat, dqn> = sum_n W_n <qhat, Kh_n>
        // and <qhat_t, Kh_n(t)> is the cosine the forward logged, so the projection needs no sum over the dims.
        // Lane (c, g) stores dims 4 g .. 4 g + 3 of step c in one 8-byte (bf16) or 16-byte store
        if (cw < nt) {
            const float qi = fabsf(qsv), qd[4] = {qv.x, qv.y, qv.z, qv.w};
            float rr[4];
#pragma unroll
            for (int r = 0; r < 4; r++) rr[r] = qsv < 0.f ? qi * acc[r] : qi * (acc[r] - (qd[r] * qi) * prv);
            const size_t off = (tok0 + (size_t)(t0 + cw) * H) * D + d0 + 4 * grpw;
            if constexpr (BF) {
                const uint2 pk = make_uint2((u32)f2bf(rr[0]) | ((u32)f2bf(rr[1]) << 16),
                                            (u32)f2bf(rr[2]) | ((u32)f2bf(rr[3]) << 16));
                *reinterpret_cast<uint2*>((bf16_t*)a.dq + off) = pk;
            } else {
                *reinterpret_cast<float4*>((float*)a.dq + off) = make_float4(rr[0], rr[1], rr[2], rr[3]);
            }
        }
        // no barrier here: what the next window's S1 and S4 overwrite was read before B3, and S7's next deltas
        // are written only after the next B2
    }
    dtemp_acc = wavesum(dtemp_acc);
    dfr_acc = wavesum(dfr_acc);
    if (lane == 0) { s_fin[0][wave] = dtemp_acc; s_fin[1][wave] = dfr_acc; }
    __syncthreads();
    if (tid == 0) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) { s0 += s_fin[0][w]; s1 += s_fin[1][w]; }
        const size_t pi = (size_t)bh * gridDim.y + blockIdx.y;
        a.part[2 * pi + 0] = s0;
        a.part[2 * pi + 1] = s1;
    }
}

// fixed-order sum of the partials (one per chain, or per chain and chunk): dtemp = sum_i part[i][0]; scalar
// dfr = sum_i part[i][1]
__global__ __launch_bounds__(256) void reduce_parts(const float* __restrict__ part, int nbh, float* dtemp,
                                                    float* dfr) {
    __shared__ float s0[256], s1[256];
    const int tid = threadIdx.x;
    float a0 = 0.f, a1 = 0.f;
    for (int i = tid; i < nbh; i += 256) { a0 += part[2 * (size_t)i]; a1 += part[2 * (size_t)i + 1]; }
    s0[tid] = a0; s1[tid] = a1;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) { s0[tid] += s0[tid + w]; s1[tid] += s1[tid + w]; }
        __syncthreads();
    }
    if (tid == 0) { dtemp[0] = s0[0]; if (dfr) dfr[0] = s1[0]; }
}

// ===================================================================================== host dispatch
template <int D, typename TI>
hipError_t launch_chain_fwd(const ChainFwdArgs& a, int B, hipStream_t st) {
    dim3 grid(B * a.H), block(FWD_THREADS);
#define SLOT_CF(PP) if (a.N <= 4 * CHAIN_WAVES * PP) { \
        if (a.kbm) slothost::launch((chain_fwd<D, PP, TI, CF_BF>), grid, block, 0, st, a); \
        else if (a.kbuf) slothost::launch((chain_fwd<D, PP, TI, CF_F32>), grid, block, 0, st, a); \
        else slothost::launch((chain_fwd<D, PP, TI, CF_NONE>), grid, block, 0, st, a); \
        return hipGetLastError(); }
    SLOT_CF(1) SLOT_CF(2) SLOT_CF(4) SLOT_CF(8) SLOT_CF(16)
#undef SLOT_CF
    return hipErrorInvalidValue;
}
// chain_bwd_w's chunks: windows per chunk so that the launch has about 768 workgroups (three rounds of one
// per CU: the 157 KB of LDS holds one), and at least 4 windows each, so that a chunk's start (a scan of the
// later address log and one gather of the key rows) stays a small part of its work.  Measured at config 2:
// 0.608 ms at this target (2 chunks per chain), 0.637 at 1,536 workgroups, 0.673 at 3,072.
static int chain_bwd_wpc(int64_t BH, int64_t T) {
    const int64_t nwin = (T + WIN - 1) / WIN;
    const int64_t w = (nwin * BH + 767) / 768;
    return (int)std::min<int64_t>(nwin, std::max<int64_t>(4, w));
}
static int64_t chain_bwd_chunks(int64_t BH, int64_t T) {
    const int64_t nwin = (T + WIN - 1) / WIN, w = chain_bwd_wpc(BH, T);
    return (nwin + w - 1) / w;
}

template <int D, typename TI>
hipError_t launch_chain_bwd(const ChainBwdArgs& a, int B, hipStream_t st) {
    if (a.occb) {                                        // windowed kernel, D / 16 waves, time chunks
        dim3 grid(B * a.H, (unsigned)chain_bwd_chunks((int64_t)B * a.H, a.T)), block(4 * D);
        if (a.N <= 64) slothost::launch((chain_bwd_w<D, 1, TI>), grid, block, 0, st, a);
        else if (a.N <= 128) slothost::launch((chain_bwd_w<D, 2, TI>), grid, block, 0, st, a);
        else if (a.N <= 192) slothost::launch((chain_bwd_w<D, 3, TI>), grid, block, 0, st, a);
        else return hipErrorInvalidValue;
        return hipGetLastError();
    }
    dim3 grid(B * a.H), block(CHAIN_THREADS);
#define SLOT_CB(PP) if (a.N <= 4 * CHAIN_WAVES * PP) { \
        if (a.occb) slothost::launch((chain_bwd<D, PP, TI, true>), grid, block, 0, st, a); \
        else slothost::launch((chain_bwd<D, PP, TI, false>), grid, block, 0, st, a); \
        return hipGetLastError(); }
    SLOT_CB(1) SLOT_CB(2) SLOT_CB(4) SLOT_CB(8) SLOT_CB(16)
#undef SLOT_CB
    return hipErrorInvalidValue;
}

}  // namespace

// ======================================================================================== C-ABI
#include "slotscan.h"
#include <algorithm>
#include <mutex>
#include <vector>

// Optional per-kernel timing with HIP events recorded on the launch stream around every kernel (the
// reference times its compiled kernels the same way with CUDA events, kvu/prof_cuda.py:9-20).
namespace slotprof {
std::mutex mu;
bool on = false;
uint32_t mask = 0;                                   // kernel ids timed while on
std::vector<hipEvent_t> pool;
struct Rec { int kid; hipEvent_t a, b; };
std::vector<Rec> recs;
hipEvent_t get() {
    if (!pool.empty()) { hipEvent_t e = pool.back(); pool.pop_back(); return e; }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}
}  // namespace slotprof

namespace slothost {
Scope*& current_scope() {
    static thread_local Scope* cur = nullptr;
    return cur;
}
Scope::Scope(int k, hipStream_t s) : kid(k), st(s) {
    prev = current_scope();
    current_scope() = this;
    if (!slotprof::on || kid < 0 || kid >= 32 || !((slotprof::mask >> kid) & 1u)) return;
    std::lock_guard<std::mutex> g(slotprof::mu);
    a = slotprof::get();
    b = slotprof::get();
    if (!a || !b) {
        if (a) slotprof::pool.push_back(a);
        if (b) slotprof::pool.push_back(b);
        a = b = nullptr;
    }
}
Scope::~Scope() {
    current_scope() = prev;
    if (!a) return;
    std::lock_guard<std::mutex> g(slotprof::mu);
    if (used) {
        slotprof::recs.push_back({kid, a, b});
    } else {
        slotprof::pool.push_back(a);
        slotprof::pool.push_back(b);
    }
}

static std::mutex side_mu;
struct SideRes { hipStream_t s = nullptr; std::vector<hipEvent_t> ev; };
static SideRes side_res[64];
int side_stream(hipStream_t* side, hipEvent_t** ev, int nev) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= 64) return fail(SLOTSCAN_ERR_HIP, "device id out of range");
    std::lock_guard<std::mutex> g(side_mu);
    SideRes& r = side_res[dev];
    if (!r.s && (e = hipStreamCreateWithFlags(&r.s, hipStreamNonBlocking)) != hipSuccess) {
        r.s = nullptr;
        return hip_fail(e, "hipStreamCreateWithFlags");
    }
    while ((int)r.ev.size() < nev) {
        hipEvent_t x = nullptr;
        if ((e = hipEventCreateWithFlags(&x, hipEventDisableTiming)) != hipSuccess) return hip_fail(e, "hipEventCreate");
        r.ev.push_back(x);
    }
    *side = r.s;
    *ev = r.ev.data();
    return 0;
}

static thread_local char g_err[512];
int fail(int code, const char* msg) {
    snprintf(g_err, sizeof g_err, "%s", msg);
    return code;
}
int hip_fail(hipError_t e, const char* where) {
    snprintf(g_err, sizeof g_err, "%s: %s", where, hipGetErrorString(e));
    return SLOTSCAN_ERR_HIP;
}
}  // namespace slothost
using slothost::fail;
using slothost::hip_fail;
using slothost::al16;

extern "C" int slotscan_profile(int enable) {
    std::lock_guard<std::mutex> g(slotprof::mu);
    slotprof::on = enable != 0;
    slotprof::mask = (uint32_t)enable;
    return 0;
}

extern "C" int slotscan_profile_read(double* total_ms, int64_t* count, int nk) {
    std::lock_guard<std::mutex> g(slotprof::mu);
    for (int i = 0; i < nk; i++) { total_ms[i] = 0.0; count[i] = 0; }
    int rc = 0;
    for (auto& r : slotprof::recs) {
        float ms = 0.f;
        if (hipEventSynchronize(r.b) != hipSuccess || hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) rc = SLOTSCAN_ERR_HIP;
        if (r.kid >= 0 && r.kid < nk) { total_ms[r.kid] += ms; count[r.kid] += 1; }
        slotprof::pool.push_back(r.a);
        slotprof::pool.push_back(r.b);
    }
    slotprof::recs.clear();
    return rc;
}

extern "C" const char* slotscan_last_error(void) { return slothost::g_err; }
extern "C" int slotscan_max_slots(int64_t D) { (void)D; return SLOTSCAN_MAX_SLOTS; }

static int check_common(int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G, int dtype) {
    if (B < 1 || T < 1 || H < 1 || N < 1 || G < 1) return fail(SLOTSCAN_ERR_SHAPE, "B, T, H, N and G must be >= 1");
    if (D != 64 && D != 128) return fail(SLOTSCAN_ERR_SHAPE, "the scan supports DK == DV in {64, 128}");
    if (N > SLOTSCAN_MAX_SLOTS) return fail(SLOTSCAN_ERR_SHAPE, "N exceeds SLOTSCAN_MAX_SLOTS (192)");
    if (dtype != SLOTSCAN_F32 && dtype != SLOTSCAN_BF16) return fail(SLOTSCAN_ERR_DTYPE, "token dtype must be f32 or bf16");
    if (B * H > 0x7fffffffLL || T > 0x7fffffffLL) return fail(SLOTSCAN_ERR_SHAPE, "B*H and T must fit in int32");
    return 0;
}

// What one forward call emits.  FE_F32: fp32 snapshots (kbuf, vbuf).  FE_MEM: the writer epilogue's bf16
// copies with kinv and valid, the keys from the chain (kbm, vbm, kinvm, validm).  FE_MEMQ: the same outputs
// with the storage quantiser applied (bits > 0; bits 0 = plain values), both copies from the row replay.
// FE_CODES: the quantiser's integer codes and per-group scales of both copies, from the row replay.
enum { FE_F32 = 0, FE_MEM = 1, FE_MEMQ = 2, FE_CODES = 3 };
struct FwdOut {
    int mode;
    float* kbuf; float* vbuf;
    bf16_t* kbm; bf16_t* vbm; float* kinvm; uint8_t* validm;
    int8_t* kcode; float* kscale; int8_t* vcode; float* vscale;
    int bits, group;
    float* kcarry;                                       // FE_MEMQ / FE_CODES: the key replay's chunk carry
};

// chunk length of the forward pipeline (a multiple of G); T < 512 runs as one chunk
static int64_t fwd_chunk_len(int64_t T, int64_t G) {
    return T >= 512 ? ((std::max<int64_t>(128, T / 8) + G - 1) / G) * G : T;
}

// The forward pipeline's chunk boundaries b[0] = 0 < b[1] < ... < b[n] = T (inner ones multiples of G);
// returns n (at most FWD_MAX_CHUNKS).  Equal chunks of fwd_chunk_len, unless the value replay fits one round
// of workgroups (two per CU): it then takes well under half the chain's time per step (the chain is bound
// by its step latency), and the chunks halve towards the end (..., 128, 64, 32, 32 steps at G = 8), so that
// the tail the replay leaves exposed (the last chunk's) and the number of chunk starts are both small, while
// each replay still hides behind the next chain chunk, half as long.
#define FWD_MAX_CHUNKS 40
static int fwd_chunks(int64_t B, int64_t T, int64_t H, int64_t N, int64_t G, int64_t* b) {
    b[0] = 0;
    const int64_t len = fwd_chunk_len(T, G);
    if (len >= T) { b[1] = T; return 1; }
    int n = 0;
    if (B * H * ((N + 31) / 32) > 512) {
        for (int64_t t = 0; t < T; t += len) b[++n] = std::min<int64_t>(T, t + len);
        return n;
    }
    // on the whole blocks of T (the last chunk takes T % G too): the tail m, m, 2m, 4m, ... from the end while
    // the rest is at least twice the next size, then the rest as one chunk, or two if it is over twice the tail's
    // largest (a replay runs at well under half its chain's time per step, so each hides behind the next chunk)
    const int64_t Tg = (T / G) * G;
    const int64_t m = ((std::max<int64_t>(32, G) + G - 1) / G) * G;
    int64_t tail[FWD_MAX_CHUNKS];
    int nt = 0;
    int64_t total = 0, next = m;
    while (nt < FWD_MAX_CHUNKS - 3 && total + 2 * next <= Tg) {
        tail[nt++] = next;
        total += next;
        if (nt >= 2) next *= 2;
    }
    const int64_t R = Tg - total;
    if (nt > 0 && R > 2 * tail[nt - 1]) {
        const int64_t r1 = std::max<int64_t>(G, (R / 2 / G) * G);
        b[++n] = r1;
    }
    b[++n] = R;
    for (int i = nt - 1; i >= 0; i--, n++) b[n + 1] = b[n] + tail[i];
    b[n] = T;
    return n;
}

static int check_q(int bits, int64_t group, int64_t D, bool codes) {
    if (codes ? (bits < 2 || bits > 8) : (bits != 0 && (bits < 2 || bits > 8)))
        return fail(SLOTSCAN_ERR_SHAPE, codes ? "bits must be 2..8" : "bits must be 0 or 2..8");
    if (bits != 0 && (group < 4 || group > D || (group & (group - 1)) != 0))
        return fail(SLOTSCAN_ERR_SHAPE, "group must be a power of two in [4, D]");
    return 0;
}

// The forward of every contract.
static int scan_fwd(const void* k, const void* q, const void* v, int dtype,
                    const float* gate, const float* fr, int fr_per_token, const float* temp,
                    int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                    float eps, int occ_bin,
                    const float* k0, const float* v0, const float* o0, FwdOut o,
                    int32_t* am, float* kold, float* vold, float* oold, float* cslog,
                    float* kfin, float* vfin, float* ofin, void* stream) {
    if (int r = check_common(B, T, H, N, D, G, dtype)) return r;
    const int mode = o.mode;
    const bool kr = mode == FE_MEMQ || mode == FE_CODES;         // the row replay emits the keys
    int64_t cb[FWD_MAX_CHUNKS + 1];
    const int nch = fwd_chunks(B, T, H, N, G, cb);
    if (!k || !q || !v || !gate || !fr || !temp || !am || !kfin || !vfin || !ofin ||
        (mode == FE_F32 && (!o.kbuf || !o.vbuf)) ||
        ((mode == FE_MEM || mode == FE_MEMQ) && (!o.kbm || !o.vbm || !o.kinvm || !o.validm)) ||
        (mode == FE_CODES && (!o.kcode || !o.kscale || !o.vcode || !o.vscale)) || (kr && nch > 1 && !o.kcarry))
        return fail(SLOTSCAN_ERR_NULL, "slotscan_fwd: a required pointer is NULL");
    if (kr)
        if (int r = check_q(o.bits, o.group, D, mode == FE_CODES)) return r;
    if ((kold == nullptr) != (oold == nullptr) || (kold == nullptr) != (vold == nullptr) ||
        (kold == nullptr) != (cslog == nullptr))
        return fail(SLOTSCAN_ERR_NULL, "slotscan_fwd: kold, vold, oold and cslog must be all set or all NULL");
    if (!al16(k) || !al16(q) || !al16(v) || !al16(o.kbuf) || !al16(o.vbuf) || !al16(o.kbm) || !al16(o.vbm) ||
        !al16(o.kcode) || !al16(o.vcode) || !al16(o.kcarry) ||
        !al16(kfin) || !al16(vfin) || (kold && (!al16(kold) || !al16(vold))) || (k0 && !al16(k0)) || (v0 && !al16(v0)))
        return fail(SLOTSCAN_ERR_ALIGN, "slotscan_fwd: row buffers must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    const int NB = (int)((T + G - 1) / G);
    const bool f32 = mode == FE_F32;
    ChainFwdArgs ca{q, k, gate, fr, temp, k0, o0, f32 ? o.kbuf : nullptr, am, kold, oold, cslog, kfin, ofin,
                    (int)T, (int)H, (int)N, (int)G, NB, eps, fr_per_token ? 1 : 0, occ_bin ? 1 : 0, 0, (int)T,
                    mode == FE_MEM ? o.kbm : nullptr, o.kinvm, o.validm, (int)H, (int)H, 0};
    RowsFwdArgs ra{v, gate, am, v0, f32 ? o.vbuf : nullptr, vold, vfin, (int)T, (int)H, (int)N, (int)G, NB, 0,
                   (int)T, o.vbm, (int)H, (int)H, 0,
                   k, k0, nullptr, o.bits, o.group, o.kbm, o.kinvm, o.validm, o.kcode, o.kscale, o.vcode, o.vscale};
    // Long sequences run as a two-stream pipeline over step chunks of a multiple of G: the key chain of
    // chunk c + 1 (latency-bound, caller's stream) overlaps the row replay of chunk c (HBM-bound, the
    // library's side stream); the last chunk's replay has no chain to overlap and runs on the caller's stream
    // behind its chain, after the side stream's replays.  fp32 contract: the state crosses an inner chunk boundary te as the snapshot
    // of block te / G, which is exactly the state there -- a chunk ends by writing it (it is its next block's
    // PRE-write snapshot) and the next chunk starts from it without storing it again.  The other contracts
    // emit no fp32 state, so the chain carries its keys in kfin, the value replay its values in vfin, and a
    // key replay its keys in kcarry (the chain may already be overwriting kfin while the replay of an
    // earlier chunk runs).  The occupancy crosses through ofin; the last chunk writes kfin, vfin, ofin.
    hipStream_t side = nullptr;
    hipEvent_t* ev = nullptr;
    if (nch > 1)
        if (int r = slothost::side_stream(&side, &ev, nch + 1)) return r;
    dim3 grid((unsigned)(B * H), (unsigned)((N + 31) / 32)), block(512);
    hipError_t e;
    for (int c = 0; c < nch; c++) {
        ca.ts = ra.ts = (int)cb[c];
        ca.te = ra.te = (int)cb[c + 1];
        const bool inner_end = ca.te < T;
        if (c > 0) {
            ca.o0 = ofin;
            if (!f32) {
                ca.k0 = kfin;
                ra.v0 = vfin;
                if (kr) ra.k0 = o.kcarry;
            } else {                                     // from the snapshot slab of block ts / G
                ca.k0 = o.kbuf + (size_t)(ca.ts / G) * H * N * D;
                ra.v0 = o.vbuf + (size_t)(ra.ts / G) * H * N * D;
                ca.k0bs = ra.v0bs = NB * (int)H;
                ca.skip0 = ra.skip0 = 1;
            }
        }
        if (kr) ra.kfin = inner_end ? o.kcarry : nullptr;
        if (f32) {                                       // an inner chunk ends in the next block's slab
            ca.kfin = inner_end ? o.kbuf + (size_t)(ca.te / G) * H * N * D : kfin;
            ra.vfin = inner_end ? o.vbuf + (size_t)(ra.te / G) * H * N * D : vfin;
            ca.kfbs = ra.vfbs = inner_end ? NB * (int)H : (int)H;
        }
        {
            slothost::Scope sc(SLOTSCAN_K_CHAIN_FWD, st);
            if (D == 128) e = dtype == SLOTSCAN_BF16 ? launch_chain_fwd<128, bf16_t>(ca, (int)B, st) : launch_chain_fwd<128, float>(ca, (int)B, st);
            else e = dtype == SLOTSCAN_BF16 ? launch_chain_fwd<64, bf16_t>(ca, (int)B, st) : launch_chain_fwd<64, float>(ca, (int)B, st);
        }
        if (e != hipSuccess) return hip_fail(e, "chain_fwd launch");
        hipStream_t rs = st;
        if (nch > 1 && c + 1 < nch) {
            if ((e = hipEventRecord(ev[c], st)) != hipSuccess) return hip_fail(e, "hipEventRecord");
            if ((e = hipStreamWaitEvent(side, ev[c], 0)) != hipSuccess) return hip_fail(e, "hipStreamWaitEvent");
            rs = side;
        } else if (nch > 1) {
            // the last chunk's replay follows its chain on the caller's stream, behind the side stream's
            // replays (its value carry): no cross-stream wait between the chain and it, and no join after it
            if ((e = hipEventRecord(ev[c], side)) != hipSuccess) return hip_fail(e, "hipEventRecord");
            if ((e = hipStreamWaitEvent(st, ev[c], 0)) != hipSuccess) return hip_fail(e, "hipStreamWaitEvent");
        }
        {
            slothost::Scope sc(SLOTSCAN_K_ROWS_FWD, rs);
#define SLOT_RF(DD, TT) { if (mode == FE_MEM) slothost::launch((rows_fwd<DD, TT, RF_BF>), grid, block, 0, rs, ra); \
                          else if (mode == FE_MEMQ) slothost::launch((rows_fwd<DD, TT, RF_MEMQ>), grid, block, 0, rs, ra); \
                          else if (mode == FE_CODES) slothost::launch((rows_fwd<DD, TT, RF_CODES>), grid, block, 0, rs, ra); \
                          else slothost::launch((rows_fwd<DD, TT, RF_F32>), grid, block, 0, rs, ra); }
            if (D == 128) {
                if (dtype == SLOTSCAN_BF16) SLOT_RF(128, bf16_t) else SLOT_RF(128, float)
            } else {
                if (dtype == SLOTSCAN_BF16) SLOT_RF(64, bf16_t) else SLOT_RF(64, float)
            }
#undef SLOT_RF
            e = hipGetLastError();
        }
        if (e != hipSuccess) return hip_fail(e, "rows_fwd launch");
    }
    return 0;                                            // the caller's stream has every chunk behind it
}

extern "C" int slotscan_fwd(const void* k, const void* q, const void* v, int dtype,
                            const float* gate, const float* fr, int fr_per_token, const float* temp,
                            int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                            float eps, int occ_bin,
                            const float* k0, const float* v0, const float* o0,
                            float* kbuf, float* vbuf, int32_t* am,
                            float* kold, float* vold, float* oold, float* cslog,
                            float* kfin, float* vfin, float* ofin, void* stream) {
    FwdOut o{};
    o.mode = FE_F32; o.kbuf = kbuf; o.vbuf = vbuf;
    return scan_fwd(k, q, v, dtype, gate, fr, fr_per_token, temp, B, T, H, N, D, G, eps, occ_bin, k0, v0, o0,
                    o, am, kold, vold, oold, cslog, kfin, vfin, ofin, stream);
}

extern "C" int slotscan_fwd_mem(const void* k, const void* q, const void* v, int dtype,
                                const float* gate, const float* fr, int fr_per_token, const float* temp,
                                int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                                float eps, int occ_bin,
                                const float* k0, const float* v0, const float* o0,
                                void* kb, void* vb, float* kinv, uint8_t* valid, int32_t* am,
                                float* kold, float* vold, float* oold, float* cslog,
                                float* kfin, float* vfin, float* ofin, void* stream) {
    FwdOut o{};
    o.mode = FE_MEM; o.kbm = (bf16_t*)kb; o.vbm = (bf16_t*)vb; o.kinvm = kinv; o.validm = valid;
    return scan_fwd(k, q, v, dtype, gate, fr, fr_per_token, temp, B, T, H, N, D, G, eps, occ_bin, k0, v0, o0,
                    o, am, kold, vold, oold, cslog, kfin, vfin, ofin, stream);
}

extern "C" size_t slotscan_fwd_carry_bytes(int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G) {
    if (B < 1 || T < 1 || H < 1 || N < 1 || D < 1 || G < 1) return 0;
    return fwd_chunk_len(T, G) < T ? (size_t)B * H * N * D * sizeof(float) : 0;
}

extern "C" int slotscan_fwd_memq(const void* k, const void* q, const void* v, int dtype,
                                 const float* gate, const float* fr, int fr_per_token, const float* temp,
                                 int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                                 float eps, int occ_bin, int bits, int64_t group,
                                 const float* k0, const float* v0, const float* o0,
                                 void* kb, void* vb, float* kinv, uint8_t* valid, int32_t* am,
                                 float* kold, float* vold, float* oold, float* cslog,
                                 float* kfin, float* vfin, float* ofin, float* kcarry, void* stream) {
    FwdOut o{};
    o.mode = FE_MEMQ; o.kbm = (bf16_t*)kb; o.vbm = (bf16_t*)vb; o.kinvm = kinv; o.validm = valid;
    o.bits = bits; o.group = (int)group; o.kcarry = kcarry;
    return scan_fwd(k, q, v, dtype, gate, fr, fr_per_token, temp, B, T, H, N, D, G, eps, occ_bin, k0, v0, o0,
                    o, am, kold, vold, oold, cslog, kfin, vfin, ofin, stream);
}

extern "C" int slotscan_fwd_codes(const void* k, const void* q, const void* v, int dtype,
                                  const float* gate, const float* fr, int fr_per_token, const float* temp,
                                  int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                                  float eps, int occ_bin, int bits, int64_t group,
                                  const float* k0, const float* v0, const float* o0,
                                  int8_t* kcode, float* kscale, int8_t* vcode, float* vscale, int32_t* am,
                                  float* kfin, float* vfin, float* ofin, float* kcarry, void* stream) {
    FwdOut o{};
    o.mode = FE_CODES; o.kcode = kcode; o.kscale = kscale; o.vcode = vcode; o.vscale = vscale;
    o.bits = bits; o.group = (int)group; o.kcarry = kcarry;
    return scan_fwd(k, q, v, dtype, gate, fr, fr_per_token, temp, B, T, H, N, D, G, eps, occ_bin, k0, v0, o0,
                    o, am, nullptr, nullptr, nullptr, nullptr, kfin, vfin, ofin, stream);
}

// The untracked G = 8 row kernel (rows_bwd<.., G8 = true, ..>) needs two snapshot boundaries at fixed
// positions in every 16-step chunk, and it addresses a batch row's snapshot gradients as 32-bit byte
// offsets from the row's base: it runs only where every such offset fits (NB * H * N * D elements of 4 B,
// or 2 B for the bf16 gradients of the fused contract, which is built for D = 128 only).
static bool rows_bwd_untracked(int64_t T, int64_t H, int64_t N, int64_t D, int64_t G, bool mem) {
    if (G != 8 || T % 16 != 0 || (mem && D != 128)) return false;
    const int64_t NB = (T + G - 1) / G;
    return (uint64_t)NB * (uint64_t)H * (uint64_t)N * (uint64_t)D * (mem ? 2u : 4u) <= 0xffffffffull;
}

extern "C" int slotscan_bwd_plan(int64_t T, int64_t H, int64_t N, int64_t D, int64_t G, int mem) {
    if (T < 1 || H < 1 || N < 1 || G < 1) {
        fail(SLOTSCAN_ERR_SHAPE, "T, H, N and G must be >= 1");
        return -1;
    }
    return rows_bwd_untracked(T, H, N, D, G, mem != 0) ? SLOTSCAN_PLAN_ROWS_UNTRACKED : 0;
}

extern "C" size_t slotscan_bwd_workspace(int64_t B, int64_t T, int64_t H, int64_t N) {
    // Dn (B*H, N, T) fp32, then the partials (B*H*chunks, 2) fp32 of the address backward, 256-byte aligned
    const size_t dn = (size_t)B * H * N * T * sizeof(float);
    return ((dn + 255) & ~(size_t)255) + (size_t)B * H * chain_bwd_chunks(B * H, T) * 2 * sizeof(float);
}

// The backward of both contracts: fp32 snapshot gradients (dkbuf, dvbuf) or, when dkbm is set, the
// gradients of the writer epilogue's bf16 copies and of kinv (dkbm, dvbm, dkinvm).
static int scan_bwd(const void* k, const void* q, const void* v, int dtype,
                    const float* gate, const float* fr, int fr_per_token, const float* temp,
                    int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                    float eps, int occ_bin,
                    const int32_t* am, const float* kold, const float* vold, const float* oold,
                    const float* cslog, const float* kfin, const float* vfin, const float* ofin,
                    const float* dkbuf, const float* dvbuf, const bf16_t* dkbm, const bf16_t* dvbm,
                    const float* dkinvm, int qbits, int qgroup, void* workspace,
                    void* dk, void* dq, void* dv, float* dgate, float* dfr, float* dtemp,
                    void* stream) {
    if (int r = check_common(B, T, H, N, D, G, dtype)) return r;
    const bool mem = dkbm != nullptr;
    if (mem && qbits)
        if (int r = check_q(qbits, qgroup, D, false)) return r;
    if (!k || !q || !v || !gate || !fr || !temp || !am || !kold || !vold || !oold || !cslog || !kfin || !vfin || !ofin ||
        (mem ? (!dvbm || !dkinvm) : (!dkbuf || !dvbuf)) || !workspace || !dk || !dq || !dv || !dgate || !dfr || !dtemp)
        return fail(SLOTSCAN_ERR_NULL, "slotscan_bwd: a required pointer is NULL");
    if (mem) { dkbuf = dvbuf = nullptr; }
    if (!al16(k) || !al16(q) || !al16(v) || !al16(kold) || !al16(vold) || !al16(kfin) || !al16(vfin) ||
        !al16(dkbuf) || !al16(dvbuf) || !al16(dkbm) || !al16(dvbm) || !al16(dk) || !al16(dv) ||
        ((uintptr_t)workspace & 255u))
        return fail(SLOTSCAN_ERR_ALIGN, "slotscan_bwd: row buffers must be 16-byte aligned (workspace 256)");
    hipStream_t st = (hipStream_t)stream;
    const int NB = (int)((T + G - 1) / G);
    float* dn = (float*)workspace;
    const size_t dnb = (size_t)B * H * N * T * sizeof(float);
    float* part = (float*)((char*)workspace + ((dnb + 255) & ~(size_t)255));
    RowsBwdArgs ra{k, v, gate, am, kold, vold, kfin, vfin, dkbuf, dvbuf, dk, dv, dn,
                   (int)T, (int)H, (int)N, (int)G, NB, dkbm, dvbm, dkinvm, mem ? qbits : 0, qgroup};
    dim3 grid((unsigned)(B * H), (unsigned)((N + 31) / 32)), block(512);
    hipError_t e;
    {
        slothost::Scope sc(SLOTSCAN_K_ROWS_BWD, st);
        const bool g8 = rows_bwd_untracked(T, H, N, D, G, mem);
#define SLOT_RB(DD, TT) { if (mem) { if (g8 && DD == 128) slothost::launch((rows_bwd<DD, TT, DD == 128, true>), grid, block, 0, st, ra); \
                                     else slothost::launch((rows_bwd<DD, TT, false, true>), grid, block, 0, st, ra); } \
                          else if (g8) slothost::launch((rows_bwd<DD, TT, true, false>), grid, block, 0, st, ra); \
                          else slothost::launch((rows_bwd<DD, TT, false, false>), grid, block, 0, st, ra); }
        if (D == 128) {
            if (dtype == SLOTSCAN_BF16) SLOT_RB(128, bf16_t) else SLOT_RB(128, float)
        } else {
            if (dtype == SLOTSCAN_BF16) SLOT_RB(64, bf16_t) else SLOT_RB(64, float)
        }
#undef SLOT_RB
        e = hipGetLastError();
    }
    if (e != hipSuccess) return hip_fail(e, "rows_bwd launch");
    ChainBwdArgs ca{q, gate, fr, temp, am, kold, oold, cslog, kfin, ofin, dn, dq, dgate, dfr, part,
                    (int)T, (int)H, (int)N, eps, fr_per_token ? 1 : 0, occ_bin ? 1 : 0,
                    chain_bwd_wpc(B * H, T)};
    const int nparts = (int)(occ_bin ? B * H * chain_bwd_chunks(B * H, T) : B * H);
    {
        slothost::Scope sc(SLOTSCAN_K_CHAIN_BWD, st);
        if (D == 128) e = dtype == SLOTSCAN_BF16 ? launch_chain_bwd<128, bf16_t>(ca, (int)B, st) : launch_chain_bwd<128, float>(ca, (int)B, st);
        else e = dtype == SLOTSCAN_BF16 ? launch_chain_bwd<64, bf16_t>(ca, (int)B, st) : launch_chain_bwd<64, float>(ca, (int)B, st);
    }
    if (e != hipSuccess) return hip_fail(e, "chain_bwd launch");
    {
        slothost::Scope sc(SLOTSCAN_K_REDUCE, st);
        slothost::launch(reduce_parts, dim3(1), dim3(256), 0, st, part, nparts, dtemp,
                           fr_per_token ? (float*)nullptr : dfr);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return hip_fail(e, "reduce_parts launch");
    return 0;
}

extern "C" int slotscan_bwd(const void* k, const void* q, const void* v, int dtype,
                            const float* gate, const float* fr, int fr_per_token, const float* temp,
                            int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                            float eps, int occ_bin,
                            const int32_t* am, const float* kold, const float* vold, const float* oold,
                            const float* cslog, const float* kfin, const float* vfin, const float* ofin,
                            const float* dkbuf, const float* dvbuf, void* workspace,
                            void* dk, void* dq, void* dv, float* dgate, float* dfr, float* dtemp,
                            void* stream) {
    if (!dkbuf || !dvbuf) return fail(SLOTSCAN_ERR_NULL, "slotscan_bwd: a required pointer is NULL");
    return scan_bwd(k, q, v, dtype, gate, fr, fr_per_token, temp, B, T, H, N, D, G, eps, occ_bin, am, kold, vold,
                    oold, cslog, kfin, vfin, ofin, dkbuf, dvbuf, nullptr, nullptr, nullptr, 0, 0, workspace,
                    dk, dq, dv, dgate, dfr, dtemp, stream);
}

// ------------------------------------------------------------------ allocation-free backward
// The backward's workspace (Dn and the per-chain partials) in a file-scope device array, for callers that
// cannot allocate.  Each device holds its own copy for the life of the process; its address is fetched once
// per device (with that device current) and kept, because in host code the array's name is not a device
// address.  Every element the kernels read is written earlier in the same call (Dn by rows_bwd for every
// (row, step) that chain_bwd reads; each chain's partials by chain_bwd before reduce_parts), so nothing has
// to start at zero, and calls that overlap on one device race on the array.
static __device__ __align__(256) unsigned char scratch[SLOTSCAN_NOALLOC_SCRATCH_BYTES];
static std::mutex scratch_mu;
static void* scratch_dev[64];

static int scratch_ptr(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= 64) return fail(SLOTSCAN_ERR_HIP, "device id out of range");
    std::lock_guard<std::mutex> g(scratch_mu);
    if (!scratch_dev[dev]) {
        void* p = nullptr;
        if ((e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess) return hip_fail(e, "hipGetSymbolAddress");
        if (!p || ((uintptr_t)p & 255u)) return fail(SLOTSCAN_ERR_HIP, "scratch array address is not 256-byte aligned");
        scratch_dev[dev] = p;
    }
    *out = scratch_dev[dev];
    return 0;
}

extern "C" int slotscan_bwd_noalloc(const void* k, const void* q, const void* v, int dtype,
                                    const float* gate, const float* fr, int fr_per_token, const float* temp,
                                    int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                                    float eps, int occ_bin,
                                    const int32_t* am, const float* kold, const float* vold, const float* oold,
                                    const float* cslog, const float* kfin, const float* vfin, const float* ofin,
                                    const float* dkbuf, const float* dvbuf,
                                    void* dk, void* dq, void* dv, float* dgate, float* dfr, float* dtemp,
                                    void* stream) {
    if (int r = check_common(B, T, H, N, D, G, dtype)) return r;
    const unsigned __int128 need = (unsigned __int128)(uint64_t)(B * H) * (uint64_t)N * (uint64_t)T * 4u + 255u +
                                   (unsigned __int128)(uint64_t)(B * H) * (uint64_t)chain_bwd_chunks(B * H, T) * 8u;
    if (need > (unsigned __int128)SLOTSCAN_NOALLOC_SCRATCH_BYTES)
        return fail(SLOTSCAN_ERR_SHAPE, "slotscan_bwd_noalloc: B*H*N*T*4 (+ partials) exceeds the static scratch of "
                                        "SLOTSCAN_NOALLOC_SCRATCH_BYTES; use slotscan_bwd with a workspace");
    if (!dkbuf || !dvbuf) return fail(SLOTSCAN_ERR_NULL, "slotscan_bwd_noalloc: a required pointer is NULL");
    void* ws = nullptr;
    if (int r = scratch_ptr(&ws)) return r;
    return scan_bwd(k, q, v, dtype, gate, fr, fr_per_token, temp, B, T, H, N, D, G, eps, occ_bin, am, kold, vold,
                    oold, cslog, kfin, vfin, ofin, dkbuf, dvbuf, nullptr, nullptr, nullptr, 0, 0, ws,
                    dk, dq, dv, dgate, dfr, dtemp, stream);
}

extern "C" int slotscan_bwd_mem(const void* k, const void* q, const void* v, int dtype,
                                const float* gate, const float* fr, int fr_per_token, const float* temp,
                                int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                                float eps, int occ_bin,
                                const int32_t* am, const float* kold, const float* vold, const float* oold,
                                const float* cslog, const float* kfin, const float* vfin, const float* ofin,
                                const void* dkb, const void* dvb, const float* dkinv, void* workspace,
                                void* dk, void* dq, void* dv, float* dgate, float* dfr, float* dtemp,
                                void* stream) {
    if (!dkb || !dvb || !dkinv) return fail(SLOTSCAN_ERR_NULL, "slotscan_bwd_mem: a required pointer is NULL");
    return scan_bwd(k, q, v, dtype, gate, fr, fr_per_token, temp, B, T, H, N, D, G, eps, occ_bin, am, kold, vold,
                    oold, cslog, kfin, vfin, ofin, nullptr, nullptr, (const bf16_t*)dkb, (const bf16_t*)dvb, dkinv,
                    0, 0, workspace, dk, dq, dv, dgate, dfr, dtemp, stream);
}

extern "C" int slotscan_bwd_memq(const void* k, const void* q, const void* v, int dtype,
                                 const float* gate, const float* fr, int fr_per_token, const float* temp,
                                 int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                                 float eps, int occ_bin, int bits, int64_t group,
                                 const int32_t* am, const float* kold, const float* vold, const float* oold,
                                 const float* cslog, const float* kfin, const float* vfin, const float* ofin,
                                 const void* dkb, const void* dvb, const float* dkinv, void* workspace,
                                 void* dk, void* dq, void* dv, float* dgate, float* dfr, float* dtemp,
                                 void* stream) {
    if (!dkb || !dvb || !dkinv) return fail(SLOTSCAN_ERR_NULL, "slotscan_bwd_memq: a required pointer is NULL");
    return scan_bwd(k, q, v, dtype, gate, fr, fr_per_token, temp, B, T, H, N, D, G, eps, occ_bin, am, kold, vold,
                    oold, cslog, kfin, vfin, ofin, nullptr, nullptr, (const bf16_t*)dkb, (const bf16_t*)dvb, dkinv,
                    bits, (int)group, workspace, dk, dq, dv, dgate, dfr, dtemp, stream);
}
