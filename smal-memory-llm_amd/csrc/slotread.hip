// Cosine slot read with per-token sharpness, for MI355X (gfx950), as bf16 MFMA contractions.
//
// Semantics (reference: /root/reference/gqa25/memlm_sh.py:362-397).  The G tokens of block j share the
// block's PRE-write copy (kbuf_j, vbuf_j); every token has NQ unit read queries.  For query m of block j:
//   raw_n = bf16(<q_m, K_n>)                 the bf16 einsum's output rounding    (memlm_sh.py:383)
//   sc_n  = raw_n * kinv_n * scale_m         kinv, exp(log_rsel), exp(C tanh(s/C)) (memlm_sh.py:383-393)
//   a     = softmax over valid n; no valid row -> a = 0 (masked_fill + nan_to_num, memlm_sh.py:394)
//   rd_m  = bf16(sum_n bf16(a_n) V_n)        att.to(bf16) then the bf16 einsum    (memlm_sh.py:395)
//
// gfx950 mapping.  One workgroup = 4 waves per (b, j, h) block and a range of up to MC query rows.  The
// slots are SPLIT across the waves (wave w owns the 16-row key tiles w*TPW .. w*TPW+TPW-1, TPW <= 3 for
// N <= 192), so a wave's share of the keys and values is loaded ONCE into VGPRs as MFMA operands and then
// reused for every 16-query tile of the range:
//   scores   S^T (16 slots x 16 queries) = K_tile Q^T   v_mfma_f32_16x16x32_bf16, K as the A operand
//            (lane row = slot), Q as the B operand (lane column = query), D/32 k-steps;
//   softmax  the D layout of S^T puts one query column in every lane (4 slots per lane per tile), so the
//            max / sum over slots is 4*TPW values per lane, a cross-row permlane reduction and one LDS
//            exchange between the 4 waves;
//   output   O^T (16 dims x 16 queries) = V^T P^T       v_mfma_f32_16x16x16_bf16: the B operand (P^T,
//            lane column = query, 4 slots per lane) is EXACTLY the D layout of the score tile, so the
//            probabilities never move; V^T is the A operand, built once from LDS-staged value rows;
//   reduce   the 4 waves' partial O (their slot ranges) are summed in a fixed order through LDS and
//            written as bf16, 16 contiguous bytes per lane, in token-major order.
// Three workgroup barriers per 16-query tile; no atomics, so the result is bitwise reproducible.
#include <algorithm>

#include "slot_common.h"
#include "slotscan.h"
#include "slotread.h"
#include "slot_host.h"

using namespace slot;
using slothost::fail;
using slothost::hip_fail;
using slothost::al16;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define READ_WAVES 4
#define READ_THREADS (64 * READ_WAVES)
#define READ_TPW 3                       // 16-slot tiles per wave at most: 4 x 3 x 16 = 192 slots

namespace {

__device__ __forceinline__ f32x4 mfma_k32(const uint4& a, const uint4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_k16(const uint2& a, const uint2& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                     0, 0, 0);
}
__device__ __forceinline__ float bf16r(float x) { return bf16_round(x); }
__device__ __forceinline__ uint32_t pack2(float lo, float hi) { return pack_bf16x2(lo, hi); }
#define LOG2E_F 1.4426950408889634f

// max over the 4 row groups of a wave (lanes c, c+16, c+32, c+48); same permlane pattern as sum4rows
__device__ __forceinline__ float max4rows(float v) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    float s = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// order LDS writes of this wave before later LDS reads by other lanes of the same wave
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct ReadFwdArgs {
    const bf16_t* q;
    const bf16_t* kb;
    const bf16_t* vb;
    const float* kinv;
    const uint8_t* valid;
    const float* scale;
    bf16_t* rd;
    int T, H, NQ, N, G, NB, MC;   // MC: query rows per workgroup (read_fwd, a multiple of 16) or per chunk (read_fwd_wide)
    int slabs, parts;             // read_fwd_wide: parts chunks of MC queries per slab, slabs x parts chunks in all
};

// a 16-byte streaming store: the backward's gradient rows are written once and not read by this layer again
// (read_train 2.89 -> 2.80 ms/step A/B in one process, mostly from the dK / dV rows)
__device__ __forceinline__ void st16_stream(bf16_t* p, uint4 v) {
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    const u32x4v y = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(y, reinterpret_cast<u32x4v*>(p));
}

template <int D>
struct ReadSmem {
    static constexpr int VST = D + 8;   // staged value row stride (bf16): rows 4 apart land 16 banks apart
    static constexpr int OST = D + 4;   // output-partial row stride (floats)
    static constexpr int VBYTES = READ_WAVES * READ_TPW * 16 * VST * 2;
    static constexpr int OBYTES = READ_WAVES * 16 * OST * 4;
    static constexpr int BIG = VBYTES > OBYTES ? VBYTES : OBYTES;
};

template <int D>
__global__ __launch_bounds__(READ_THREADS) __attribute__((amdgpu_waves_per_eu(3))) void read_fwd(ReadFwdArgs a) {
    constexpr int KK = D / 32;
    constexpr int DT = D / 16;
    constexpr int VST = ReadSmem<D>::VST;
    constexpr int OST = ReadSmem<D>::OST;
    __shared__ __align__(16) unsigned char s_big[ReadSmem<D>::BIG];   // staged values, then output partials
    __shared__ float s_max[READ_WAVES][16];
    __shared__ float s_sum[READ_WAVES][16];

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int slab = blockIdx.x;                                // (b * NB + j) * H + h: the kbuf slab
    const int h = slab % a.H;
    const int j = (slab / a.H) % a.NB;
    const int b = slab / (a.H * a.NB);
    const int t0 = j * a.G;
    const int Mblk = min(a.G, a.T - t0) * a.NQ;
    const int mlo = blockIdx.y * a.MC;
    const int mhi = min(Mblk, mlo + a.MC);
    if (mlo >= mhi) return;                                     // uniform over the workgroup

    const int N = a.N;
    const int NT16 = (N + 15) >> 4;
    const int TPW = (NT16 + READ_WAVES - 1) / READ_WAVES;
    const bf16_t* Kb = a.kb + (size_t)slab * N * D;
    const bf16_t* Vb = a.vb + (size_t)slab * N * D;
    const float* KI = a.kinv + (size_t)slab * N;
    const uint8_t* VA = a.valid + (size_t)slab * N;

    // the first query tile's B operand and sharpness, issued before the slab's loads so that its latency
    // overlaps theirs (a block's queries usually fit one tile)
    auto load_q = [&](int m0, uint4* qf, float& scl) {
        const int m = m0 + c;
        const bool mok = m < mhi;
        size_t qrow = 0;
        if (mok) qrow = (((size_t)b * a.T + t0 + m / a.NQ) * a.H + h) * a.NQ + (m % a.NQ);
#pragma unroll
        for (int kk = 0; kk < KK; kk++)
            qf[kk] = mok ? *reinterpret_cast<const uint4*>(a.q + qrow * D + kk * 32 + 8 * g) : make_uint4(0, 0, 0, 0);
        scl = mok ? a.scale[qrow] : 0.f;
    };
    uint4 qn[KK];
    float scn;
    load_q(mlo, qn, scn);

    // ---- this wave's keys (A operand of the score product), kinv and validity, values (A of the output)
    // Every load is issued unconditionally from a clamped in-range address and masked by a select, in
    // straight-line code: a load behind a branch waits for itself (and the next load reused its address
    // registers, so the 24 validity and kinv loads went out one at a time)
    uint4 kf[READ_TPW][KK];
    float kv[READ_TPW][4];
    uint32_t vmask = 0;
#pragma unroll
    for (int u = 0; u < READ_TPW; u++) {
        const int nt = w * TPW + u;
        const bool tile = u < TPW && nt < NT16;
        const int nr = nt * 16 + c;                              // A-operand row of this lane
#pragma unroll
        for (int kk = 0; kk < KK; kk++) {
            const uint4 x = *reinterpret_cast<const uint4*>(Kb + (size_t)min(nr, N - 1) * D + kk * 32 + 8 * g);
            kf[u][kk] = (tile && nr < N) ? x : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = nt * 16 + 4 * g + i;                     // D-layout row of item i
            const uint8_t va = VA[min(n, N - 1)];
            const float ki = KI[min(n, N - 1)];
            const bool ok = tile && n < N && va != 0;
            kv[u][i] = ok ? ki : 0.f;
            vmask |= (ok ? 1u : 0u) << (u * 4 + i);
        }
    }
    bf16_t* sV = reinterpret_cast<bf16_t*>(s_big) + w * (READ_TPW * 16 * VST);
    {
        // this wave's value rows straight into its LDS rows (direct global -> LDS loads, no data registers):
        // 16-byte chunk L of the padded region is row L / CPR, chunk L % CPR; the pad chunk is not written,
        // and rows past N or past this wave's tiles get zeros from an ordinary LDS store (the V^T tiles read
        // all READ_TPW tiles)
        constexpr int CPR = VST * 2 / 16;                           // 16-byte chunks per padded row
        constexpr int NI = (READ_TPW * 16 * CPR + 63) / 64;         // load instructions for the whole region
        const int nbase = w * TPW * 16;
        const int rows = TPW * 16;
        const unsigned l0 = lds_addr(sV);
#pragma unroll
        for (int it = 0; it < NI; it++) {
            const int e = lane + 64 * it;
            const int r = e / CPR, cc = e - (e / CPR) * CPR;
            const int n = nbase + r;
            if (r < READ_TPW * 16 && cc < D / 8) {
                if (r < rows && n < N) dma16(Vb + (size_t)n * D + cc * 8, l0 + 1024u * it);
                else *reinterpret_cast<uint4*>(sV + r * VST + cc * 8) = make_uint4(0, 0, 0, 0);
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");           // the direct loads are not tracked
    }
    wave_lds_sync();
    uint2 vf[READ_TPW][DT];                                      // V^T tile: row = dim 16dt + c, k = slot 4g + i
#pragma unroll
    for (int u = 0; u < READ_TPW; u++)
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {                       // rows past this wave's tiles are zero
            const bf16_t* p = sV + (u * 16 + 4 * g) * VST + dt * 16 + c;
            vf[u][dt].x = (uint32_t)p[0] | ((uint32_t)p[VST] << 16);
            vf[u][dt].y = (uint32_t)p[2 * VST] | ((uint32_t)p[3 * VST] << 16);
        }

    float* sO = reinterpret_cast<float*>(s_big);
    for (int m0 = mlo; m0 < mhi; m0 += 16) {
        // ---- queries of this tile: B operand, lane column = query m0 + c (the next tile's in flight)
        uint4 qf[KK];
#pragma unroll
        for (int kk = 0; kk < KK; kk++) qf[kk] = qn[kk];
        const float scl = scn;
        if (m0 + 16 < mhi) load_q(m0 + 16, qn, scn);

        f32x4 acc[READ_TPW];
#pragma unroll
        for (int u = 0; u < READ_TPW; u++) {
            acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KK; kk++) acc[u] = mfma_k32(kf[u][kk], qf[kk], acc[u]);   // zero keys past N
        }
        // ---- masked softmax over the slots of this lane's query column
        float sc[READ_TPW][4];
        float mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < READ_TPW; u++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float s = bf16r(acc[u][i]) * kv[u][i] * scl;
                sc[u][i] = s;
                if ((vmask >> (u * 4 + i)) & 1u) mx = fmaxf(mx, s);
            }
        mx = max4rows(mx);
        if (g == 0) s_max[w][c] = mx;
        __syncthreads();
        const float M = fmaxf(fmaxf(s_max[0][c], s_max[1][c]), fmaxf(s_max[2][c], s_max[3][c]));
        float sum = 0.f;
#pragma unroll
        for (int u = 0; u < READ_TPW; u++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float e = ((vmask >> (u * 4 + i)) & 1u) ? __expf(sc[u][i] - M) : 0.f;
                sc[u][i] = e;
                sum += e;
            }
        sum = sum4rows(sum);
        if (g == 0) s_sum[w][c] = sum;
        __syncthreads();
        const float S = ((s_sum[0][c] + s_sum[1][c]) + s_sum[2][c]) + s_sum[3][c];
        const float inv = S > 0.f ? 1.f / S : 0.f;
        uint2 pf[READ_TPW];
#pragma unroll
        for (int u = 0; u < READ_TPW; u++) {
            pf[u].x = pack2(sc[u][0] * inv, sc[u][1] * inv);
            pf[u].y = pack2(sc[u][2] * inv, sc[u][3] * inv);
        }
        // ---- O^T partial over this wave's slots
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < READ_TPW; u++)
                o = mfma_k16(vf[u][dt], pf[u], o);
            *reinterpret_cast<f32x4*>(sO + (w * 16 + c) * OST + dt * 16 + 4 * g) = o;
        }
        __syncthreads();
        // ---- fixed-order sum of the 4 partials, bf16, token-major store
        {
            constexpr int EPT = D / 16;
            const int mr = threadIdx.x >> 4, dc = (threadIdx.x & 15) * EPT;
            const int mm = m0 + mr;
            if (mm < mhi) {
                float r[EPT];
#pragma unroll
                for (int e = 0; e < EPT; e++) r[e] = sO[mr * OST + dc + e];
#pragma unroll
                for (int ww = 1; ww < READ_WAVES; ww++)
#pragma unroll
                    for (int e = 0; e < EPT; e++) r[e] += sO[(ww * 16 + mr) * OST + dc + e];
                const size_t orow = (((size_t)b * a.T + t0 + mm / a.NQ) * a.H + h) * a.NQ + (mm % a.NQ);
                bf16_t* dst = a.rd + orow * D + dc;
                if constexpr (EPT == 8) {
                    uint4 x;
                    x.x = pack2(r[0], r[1]); x.y = pack2(r[2], r[3]); x.z = pack2(r[4], r[5]); x.w = pack2(r[6], r[7]);
                    *reinterpret_cast<uint4*>(dst) = x;
                } else {
                    uint2 x;
                    x.x = pack2(r[0], r[1]); x.y = pack2(r[2], r[3]);
                    *reinterpret_cast<uint2*>(dst) = x;
                }
            }
        }
    }
}


// ------------------------------------------------------------------------------------ wide query blocks
// Blocks with many queries (the frozen-store fan-out: one block of T*NQ queries per head) invert the split:
// the workgroup stages the block's keys and values in LDS once, and each of its 8 waves owns whole pairs of
// 16-query tiles against ALL slots, so the softmax is wave-local; every key and value operand read from LDS
// feeds one MFMA of each tile of the pair (half the LDS reads per query of one tile per wave, at 2 waves per
// SIMD and up to 256 registers).  Per tile and wave:
//   S^T = K Q^T     12 x D/32 MFMA 16x16x32, A = key rows from LDS (16 B per lane), B = queries from HBM
//                   (loaded one pair ahead, across unit boundaries);
//   softmax         48 scores per lane (its query column), cross-row permlane max / sum;
//   O^T = V^T P^T   D/16 x 6 MFMA 16x16x32: B = the probabilities straight from the score tiles (slots
//                   4g+i of tile 2c and 16+4g+i of tile 2c+1 as the 8 k-slots of lane group g), A = the
//                   same 8 slots of one value dimension, read TRANSPOSED from the row-major value rows by two
//                   ds_read_b64_tr_b16 (a 16-lane group reads 4 slot rows x 16 dims; lane l receives dim l);
//   store           4 consecutive dims of one query per lane and tile (8 bytes), token-major.
// The grid is persistent: one workgroup per CU walks a contiguous range of the blocks' 256-query chunks (6 at
// config 4: one and a half blocks), a unit being the part of the range inside one block, so that staging
// overlaps compute and a workgroup restages the store only where its range crosses into the next block.  Keys are staged in two ping-pong buffers: the NEXT unit's
// keys are fetched by direct global -> LDS loads (no registers) during the current unit, after its first
// tile's softmax.  Values are staged row-major (as the keys: no transposition, so they too are direct loads)
// into one buffer, fetched when every wave is done with the current unit's values; the next unit's first
// tile waits for them only before its value product, behind its scores and softmax.  147 KB of LDS at
// D = 128.  The 16-byte chunks
// of a staged row are XOR-swizzled (kpos, vpos) so that the key operand reads (16 consecutive rows at one
// chunk) and the transposed value reads (4 rows x 2 chunks per 16-lane group) hit distinct banks.
// Rows past N are copies of row N - 1 with kinv 0 and mask -inf: their probability is exactly 0.
#define WIDE_WAVES 8
#define WIDE_THREADS (64 * WIDE_WAVES)
#define WIDE_NP 192                              // staged slots (N <= 192)

template <int D>
struct WideSmem {
    static constexpr int ROWB = 2 * D;           // bytes of a staged key / value row
    static constexpr int OPB = WIDE_NP * ROWB;   // bytes of one staged operand (48 KB at D = 128)
    static constexpr int NDMA = OPB / 1024;      // 1-KB direct loads per operand
    static constexpr int PWD = NDMA / WIDE_WAVES;   // direct loads per wave and operand (6 at D = 128)
    static constexpr int CH = D / 8;             // 16-byte chunks per row
    static constexpr int RP = 256 / ROWB;        // rows per 256 bytes (64 banks)
    static_assert(NDMA % WIDE_WAVES == 0 && PWD < 16, "direct-load split");
};
// chunk position of logical 16-byte chunk c of staged key row r / value row s (XOR: its own inverse)
template <int D> __device__ __forceinline__ int kpos(int r, int c) {
    return c ^ ((r / WideSmem<D>::RP) & (WideSmem<D>::CH - 1));
}
template <int D> __device__ __forceinline__ int vpos(int r, int c) {
    return c ^ (2 * ((r / WideSmem<D>::RP) & (WideSmem<D>::CH / 2 - 1)));
}

typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
__device__ __forceinline__ uint2 ld_tr16(const unsigned char* p) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((const lds_void*)p)));
}
// an empty use of a register: the load that produced it is waited for here, not later
__device__ __forceinline__ void wide_keep(uint4& x) { asm volatile("" : "+v"(x.x), "+v"(x.y), "+v"(x.z), "+v"(x.w)); }
// wait until at most n of this wave's vector-memory operations are outstanding.  The direct loads are not
// tracked by the compiler; the kernel's other vector-memory operations -- query loads, output stores, any
// scratch access -- are tracked by it or younger, so they can only make these waits longer, never shorter.
template <int n> __device__ __forceinline__ void wide_wait_vm() {
    static_assert(n >= 0 && n < 16, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt(0x0F70 | n);
}

template <int D>
__global__ __launch_bounds__(WIDE_THREADS) void read_fwd_wide(ReadFwdArgs a) {
    using S = WideSmem<D>;
    constexpr int KK = D / 32;
    constexpr int DT = D / 16;
    constexpr int NT = WIDE_NP / 16;                       // slot tiles
    __shared__ __align__(1024) unsigned char sKb[2][S::OPB];
    __shared__ __align__(1024) unsigned char sVb[S::OPB];
    __shared__ __align__(16) float sKV[2][WIDE_NP];       // kinv of a valid slot, 0 otherwise
    __shared__ __align__(16) float sMK[2][WIDE_NP];       // 0 for a valid slot, -inf otherwise

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int N = a.N;
    // The work is the sequence of query chunks (slab, CH queries), a.parts chunks per slab; workgroup i takes the
    // contiguous range [c0, c1) of it, so it crosses as few slab boundaries as it can (one per 1.5 slabs at
    // config 4, against one per 512-query unit when the units were dealt round-robin): a unit is a maximal run of
    // the range inside one slab, and only a change of unit restages the slot store behind two barriers.
    constexpr int CH = 32 * WIDE_WAVES;                    // queries per chunk: one tile pair per wave
    const int64_t nch = (int64_t)a.slabs * a.parts;
    const int c0 = (int)(nch * blockIdx.x / gridDim.x), c1 = (int)(nch * (blockIdx.x + 1) / gridDim.x);

    struct Unit { int slab, b, h, t0, mlo, mhi, tpw, cnext; };
    auto unit = [&](int u) {
        Unit x;                                            // (every field wave-uniform: scalar registers)
        u = __builtin_amdgcn_readfirstlane(u);
        x.slab = u / a.parts;
        const int p0 = u - x.slab * a.parts;
        const int p1 = min(a.parts, p0 + (c1 - u));        // this unit: chunks [p0, p1) of the slab
        x.tpw = p1 - p0;                                   // tile pairs per wave
        x.cnext = u + x.tpw;
        x.h = x.slab % a.H;
        const int j = (x.slab / a.H) % a.NB;
        x.b = x.slab / (a.H * a.NB);
        x.t0 = j * a.G;
        const int Mblk = min(a.G, a.T - x.t0) * a.NQ;
        x.mlo = p0 * CH;
        x.mhi = min(Mblk, p1 * CH);
        x.slab = __builtin_amdgcn_readfirstlane(x.slab); x.b = __builtin_amdgcn_readfirstlane(x.b);
        x.h = __builtin_amdgcn_readfirstlane(x.h); x.t0 = __builtin_amdgcn_readfirstlane(x.t0);
        x.mlo = __builtin_amdgcn_readfirstlane(x.mlo); x.mhi = __builtin_amdgcn_readfirstlane(x.mhi);
        x.tpw = __builtin_amdgcn_readfirstlane(x.tpw); x.cnext = __builtin_amdgcn_readfirstlane(x.cnext);
        return x;
    };
    // this wave's direct loads of one staged operand (keys: kpos, values: vpos): lane L of block b fills LDS
    // bytes 1024 b + 16 L, i.e. row (1024 b + 16 L) / ROWB at chunk position p, from the chunk stored there
    // The per-lane source offsets are derived from an opaque copy of the lane index at every call: hoisted out of
    // the unit loop they were spilled, and each reload's wait (the compiler cannot count the direct loads) then
    // waited for every direct load issued before it, one round trip per load.
    auto stage = [&](const bf16_t* src, unsigned char* dst, bool val) {
        uint32_t lo;
        asm volatile("v_mov_b32 %0, %1" : "=v"(lo) : "v"((uint32_t)lane));
#pragma unroll
        for (int i = 0; i < S::PWD; i++) {
            const int blk = w * S::PWD + i, byte = blk * 1024 + 16 * (int)lo;
            const int r = byte / S::ROWB, p = (byte % S::ROWB) / 16;
            const int cc = val ? vpos<D>(r, p) : kpos<D>(r, p);
            dma16(src + (size_t)min(r, N - 1) * D + 8 * cc, lds_addr(dst + blk * 1024));
        }
    };
    auto load_kv = [&](const Unit& x, float& ki, uint32_t& va) {
        const int nc = min((int)threadIdx.x, N - 1);
        ki = a.kinv[(size_t)x.slab * N + nc];
        va = a.valid[(size_t)x.slab * N + nc];
    };
    auto publish_kv = [&](int buf, float ki, uint32_t va) {
        if (threadIdx.x < WIDE_NP) {
            const bool ok = (int)threadIdx.x < N && va != 0;
            sKV[buf][threadIdx.x] = ok ? ki : 0.f;
            sMK[buf][threadIdx.x] = ok ? 0.f : -INFINITY;
        }
    };
    // the queries of the 16-query tile at m0: lane column m0 + c, dims kk * 32 + 8 g
    auto load_q = [&](const Unit& x, int m0, uint4* qf, float& scl) {
        const int m = m0 + c;
        const bool mok = m < x.mhi;
        size_t qrow = 0;
        if (mok) qrow = (((size_t)x.b * a.T + x.t0 + m / a.NQ) * a.H + x.h) * a.NQ + (m % a.NQ);
#pragma unroll
        for (int kk = 0; kk < KK; kk++)
            qf[kk] = mok ? *reinterpret_cast<const uint4*>(a.q + qrow * D + kk * 32 + 8 * g) : make_uint4(0, 0, 0, 0);
        scl = mok ? a.scale[qrow] : 0.f;
    };
    auto load_pair = [&](const Unit& x, int m0, uint4 (&qf)[2][KK], float (&scl)[2]) {
        load_q(x, m0, qf[0], scl[0]);
        load_q(x, m0 + 16, qf[1], scl[1]);
    };

    // per-lane swizzles: key operand rows nt * 16 + c; value rows (tile) 4 g + ((c >> 2) & 3) (+ 32 cc, + 16)
    const int ksw = (c / S::RP) & (S::CH - 1);
    const int rq = (c >> 2) & 3;
    const int vsw = 2 * (((4 * g + rq) / S::RP) & (S::CH / 2 - 1));
    const int vch = (c & 3) >> 1, vhb = 8 * (c & 1);

    // ---- prologue: the first unit's keys, values, kinv / valid and first query tile pair
    int u = c0;
    Unit cur = unit(u);
    stage(a.kb + (size_t)cur.slab * N * D, sKb[0], false);
    stage(a.vb + (size_t)cur.slab * N * D, sVb, true);
    {
        float ki;
        uint32_t va;
        load_kv(cur, ki, va);
        publish_kv(0, ki, va);
    }
    uint4 qn[2][KK];
    float scn[2] = {0.f, 0.f};
    load_pair(cur, cur.mlo + 32 * w, qn, scn);
    wide_wait_vm<0>();
    __syncthreads();
    int kb = 0;
    for (;;) {
        const int un = cur.cnext;
        const bool hasn = un < c1;
        Unit nx = cur;
        float kin = 0.f;
        uint32_t van = 0;
        if (hasn) nx = unit(un);
        const unsigned char* Kc = sKb[kb];
        const int TPW = cur.tpw;
        for (int t = 0; t < TPW; t++) {
            // a pair of 16-query tiles, A = [m0, m0 + 16) and B = [m0 + 16, m0 + 32): every key and value operand
            // read from LDS feeds one MFMA of each
            const int m0 = cur.mlo + 32 * (w + WIDE_WAVES * t);
            const bool live = m0 < cur.mhi;
            int lo0 = 0;                                   // opaque zero: no hoisting of the invariant key reads
            asm volatile("" : "+v"(lo0));
            uint4 qf[2][KK];
            float scl[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
#pragma unroll
                for (int kk = 0; kk < KK; kk++) qf[e][kk] = qn[e][kk];
                scl[e] = scn[e];
            }
            if (t + 1 < TPW) load_pair(cur, m0 + 32 * WIDE_WAVES, qn, scn);
            else if (hasn) load_pair(nx, nx.mlo + 32 * w, qn, scn);

            f32x4 acc[2][NT];
            uint4 pB[2][WIDE_NP / 32];
            if (live) {
                // ---- scores S^T for all slot tiles: lane column = query m0 (+16) + c, items = slots 16 nt + 4 g + i
#pragma unroll
                for (int e = 0; e < 2; e++)
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) acc[e][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ng = 0; ng < NT / 4; ng++) {                      // 3 groups of 4 slot tiles
#pragma unroll
                    for (int kk = 0; kk < KK; kk++)
#pragma unroll
                        for (int nt = 4 * ng; nt < 4 * ng + 4; nt++) {
                            const uint4 ka = *reinterpret_cast<const uint4*>(
                                Kc + lo0 + (nt * 16 + c) * S::ROWB + 16 * ((4 * kk + g) ^ ksw));
                            acc[0][nt] = mfma_k32(ka, qf[0][kk], acc[0][nt]);
                            acc[1][nt] = mfma_k32(ka, qf[1][kk], acc[1][nt]);
                        }
                    __builtin_amdgcn_sched_barrier(0);                    // bound the operand prefetch window
                }
                // v = raw * kinv (+ -inf for an invalid slot), raw the bf16-rounded dot product; with the
                // per-query scale s > 0 the softmax is exp(s (v - max v)) = exp2(fma(v, s log2(e), -max v s log2(e))):
                // the shift rides in the fma, one v_exp_f32 per score
                float mxt[2][NT];                                         // per slot tile, then a tree
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {                          // kinv and mask read once per pair
                    const float4 kv = *reinterpret_cast<const float4*>(&sKV[kb][lo0 + nt * 16 + 4 * g]);
                    const float4 mk = *reinterpret_cast<const float4*>(&sMK[kb][lo0 + nt * 16 + 4 * g]);
                    const float kvs[4] = {kv.x, kv.y, kv.z, kv.w};
                    const float mks[4] = {mk.x, mk.y, mk.z, mk.w};
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const uint32_t r01 = pack2(acc[e][nt][0], acc[e][nt][1]);
                        const uint32_t r23 = pack2(acc[e][nt][2], acc[e][nt][3]);
                        const float raw[4] = {__uint_as_float(r01 << 16), __uint_as_float(r01 & 0xffff0000u),
                                              __uint_as_float(r23 << 16), __uint_as_float(r23 & 0xffff0000u)};
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[e][nt][i] = fmaf(raw[i], kvs[i], mks[i]);
                        mxt[e][nt] = fmaxf(fmaxf(acc[e][nt][0], acc[e][nt][1]), fmaxf(acc[e][nt][2], acc[e][nt][3]));
                    }
                }
#pragma unroll
                for (int e = 0; e < 2; e++) {
#pragma unroll
                    for (int st = 1; st < NT; st *= 2)                     // pairwise tree over the slot tiles
#pragma unroll
                        for (int nt = 0; nt + st < NT; nt += 2 * st) mxt[e][nt] = fmaxf(mxt[e][nt], mxt[e][nt + st]);
                    const float mx = max4rows(mxt[e][0]);
                    const float s2 = scl[e] * LOG2E_F;
                    const float sh = mx == -INFINITY ? 0.f : -mx * s2;    // no valid slot: every term exp2(-inf) = 0
                    float st4[NT];
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[e][nt][i] = __builtin_amdgcn_exp2f(fmaf(acc[e][nt][i], s2, sh));
                        st4[nt] = (acc[e][nt][0] + acc[e][nt][1]) + (acc[e][nt][2] + acc[e][nt][3]);
                    }
#pragma unroll
                    for (int st = 1; st < NT; st *= 2)
#pragma unroll
                        for (int nt = 0; nt + st < NT; nt += 2 * st) st4[nt] += st4[nt + st];
                    const float sum = sum4rows(st4[0]);
                    const float inv = sum > 0.f ? 1.f / sum : 0.f;
#pragma unroll
                    for (int cc = 0; cc < WIDE_NP / 32; cc++) {
                        pB[e][cc].x = pack2(acc[e][2 * cc][0] * inv, acc[e][2 * cc][1] * inv);
                        pB[e][cc].y = pack2(acc[e][2 * cc][2] * inv, acc[e][2 * cc][3] * inv);
                        pB[e][cc].z = pack2(acc[e][2 * cc + 1][0] * inv, acc[e][2 * cc + 1][1] * inv);
                        pB[e][cc].w = pack2(acc[e][2 * cc + 1][2] * inv, acc[e][2 * cc + 1][3] * inv);
                    }
                }
            }
            if (t == 0) {
                // this unit's values (their loads went out at the end of the previous unit, behind its last
                // tile): wait for everything this wave issued, then the next unit's keys and kinv / valid go out,
                // behind the rest of this unit.  The first unit's values were published by the prologue.
                if (u != c0) {
                    wide_wait_vm<0>();
                    __syncthreads();
                }
                if (hasn) {
                    stage(a.kb + (size_t)nx.slab * N * D, sKb[kb ^ 1], false);
                    load_kv(nx, kin, van);
                }
            }
            // the unit's last pair: wait here for everything this wave has issued -- the next unit's keys and
            // kinv / valid among it, long done -- so that no wait is needed after this pair's output stores
            // (gfx9 counts stores on the same counter: a wait behind them would wait for their round trip)
            if (t == TPW - 1) wide_wait_vm<0>();
            if (live) {
                // ---- O^T = V^T P^T, one 16-dim tile at a time (both query tiles per value operand), stored as 4
                // dims x 1 query per lane
                f32x4 o[2][DT];
#pragma unroll
                for (int e = 0; e < 2; e++)
#pragma unroll
                    for (int dt = 0; dt < DT; dt++) o[e][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int cc = 0; cc < WIDE_NP / 32; cc++) {
#pragma unroll
                    for (int dt = 0; dt < DT; dt++) {
                        const unsigned char* vr = sVb + (cc * 32 + 4 * g + rq) * S::ROWB + 16 * ((2 * dt + vch) ^ vsw) + vhb;
                        const uint2 lo = ld_tr16(vr);
                        const uint2 hi = ld_tr16(vr + 16 * S::ROWB);
                        const uint4 va = make_uint4(lo.x, lo.y, hi.x, hi.y);
                        o[0][dt] = mfma_k32(va, pB[0][cc], o[0][dt]);
                        o[1][dt] = mfma_k32(va, pB[1][cc], o[1][dt]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (t == TPW - 1) {
                    // the next unit's first query registers, waited for here (their loads went out at this pair's
                    // start, nothing else is in flight): the direct loads are invisible to the compiler's counts,
                    // so its wait for these registers at the unit's turn would also wait for the unit's values
#pragma unroll
                    for (int e = 0; e < 2; e++) {
#pragma unroll
                        for (int kk = 0; kk < KK; kk++) wide_keep(qn[e][kk]);
                        asm volatile("" : "+v"(scn[e]));
                    }
                }
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const int m = m0 + 16 * e + c;
                    if (m < cur.mhi) {
                        bf16_t* dst = a.rd + ((((size_t)cur.b * a.T + cur.t0 + m / a.NQ) * a.H + cur.h) * a.NQ + (m % a.NQ)) * D;
#pragma unroll
                        for (int dt = 0; dt < DT; dt++) {
                            uint2 x;
                            x.x = pack2(o[e][dt][0], o[e][dt][1]);
                            x.y = pack2(o[e][dt][2], o[e][dt][3]);
                            *reinterpret_cast<uint2*>(dst + dt * 16 + 4 * g) = x;
                        }
                    }
                }
            }
        }
        __syncthreads();                                     // every wave is done with this unit's keys and values
        if (!hasn) break;
        stage(a.vb + (size_t)nx.slab * N * D, sVb, true);     // the next unit's values
        publish_kv(kb ^ 1, kin, van);                        // (its keys landed before the last pair's stores)
        __syncthreads();
        u = un;
        cur = nx;
        kb ^= 1;
    }
}

// ---------------------------------------------------------------------------------------------- backward
// Adjoint of read_fwd, the straight derivative of the reference's ops (memlm_sh.py:383-395) with the same
// bf16 roundings autograd makes there: d(att_bf16) = bf16(dO V^T), the softmax adjoint in fp32 from the fp32
// probabilities, d raw = bf16(dsc * kinv * scale) (the .float() of a bf16 einsum casts its gradient back),
// and bf16 outputs of the three gradient contractions.
//   S     (16 queries x 16 slots) = Q K^T        16x16x32, Q tile from LDS as A, K rows from L2 as B;
//         queries are the ROWS here, so the softmax max / sums over slots are DPP row reductions
//   datt  = bf16(dO V^T)                         16x16x32, same shapes
//   dK^T  (16 dims x 16 slots) = Q^T draw        16x16x16: the B operand is exactly the D layout of draw
//   dV^T  = dO^T P                               16x16x16: the B operand is exactly the D layout of P
//   dQ^T  (16 dims x 16 queries) = K^T draw^T    16x16x16, partial over the wave's slots, fixed-order sum
// The transposed operands (Q^T, dO^T, K^T) are gathered as 16-bit elements from LDS or L2; draw^T goes
// through a per-wave LDS tile.  ACC = the block has more than one 16-query tile, so dK, dV accumulate in
// registers across tiles; otherwise every output tile is finished by one MFMA and stored at once.
struct ReadBwdArgs {
    const bf16_t* q;
    const bf16_t* kb;
    const bf16_t* vb;
    const float* kinv;
    const uint8_t* valid;
    const float* scale;
    const bf16_t* drd;
    bf16_t* dq;
    bf16_t* dkb;
    bf16_t* dvb;
    float* dkinv;
    float* dscale;
    int T, H, NQ, N, G, NB;
};

template <int D>
struct ReadBwdSmem {
    static constexpr int TST = D + 8;               // Q / dO tile row stride (bf16)
    static constexpr int RST = READ_TPW * 16 + 8;   // draw^T tile row stride (bf16)
    static constexpr int OST = D + 4;               // dQ partial row stride (floats)
};

__device__ __forceinline__ uint2 gather4(const bf16_t* p, int stride) {
    uint2 r;
    r.x = (uint32_t)p[0] | ((uint32_t)p[stride] << 16);
    r.y = (uint32_t)p[2 * stride] | ((uint32_t)p[3 * stride] << 16);
    return r;
}

// read_bwd's score and datt products load their key and value operands RBWD_KBATCH k-steps at a time per
// operand before the MFMAs that use them: 2 keeps the non-accumulating form within 168 VGPRs (3 workgroups
// per CU) without spills, where one load pair per k-step made every MFMA wait for its own loads
#ifndef RBWD_KBATCH
#define RBWD_KBATCH 2
#endif
template <int D, bool ACC>
__global__ __launch_bounds__(READ_THREADS) __attribute__((amdgpu_waves_per_eu(ACC ? 1 : 3))) void read_bwd(ReadBwdArgs a) {
    constexpr int KK = D / 32;
    constexpr int DT = D / 16;
    constexpr int TST = ReadBwdSmem<D>::TST;
    constexpr int RST = ReadBwdSmem<D>::RST;
    constexpr int OST = ReadBwdSmem<D>::OST;
    __shared__ __align__(16) bf16_t s_q[16 * TST];
    __shared__ __align__(16) bf16_t s_do[16 * TST];
    __shared__ __align__(16) bf16_t s_dr[READ_WAVES][16 * RST];
    __shared__ __align__(16) float s_part[READ_WAVES * 16 * OST];
    __shared__ float s_scl[16];
    __shared__ float s_red[3][READ_WAVES][16];
    __shared__ float s_dsc[READ_WAVES][16];

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int slab = blockIdx.x;
    const int h = slab % a.H;
    const int j = (slab / a.H) % a.NB;
    const int b = slab / (a.H * a.NB);
    const int t0 = j * a.G;
    const int Mblk = min(a.G, a.T - t0) * a.NQ;
    const int N = a.N;
    const int NT16 = (N + 15) >> 4;
    const int TPW = (NT16 + READ_WAVES - 1) / READ_WAVES;
    const bf16_t* Kb = a.kb + (size_t)slab * N * D;
    const bf16_t* Vb = a.vb + (size_t)slab * N * D;
    const float* KI = a.kinv + (size_t)slab * N;
    const uint8_t* VA = a.valid + (size_t)slab * N;
    bf16_t* dKb = a.dkb + (size_t)slab * N * D;
    bf16_t* dVb = a.dvb + (size_t)slab * N * D;

    // this lane's slot column in the S layout: n = 16 nt + c.  Validity and kinv are loaded unconditionally
    // from clamped rows and masked where first used (after the query tile's barrier), so no load here waits
    float kvc[READ_TPW];
    uint32_t vraw[READ_TPW];
    bool tile[READ_TPW];
#pragma unroll
    for (int u = 0; u < READ_TPW; u++) {
        const int nt = w * TPW + u;
        tile[u] = u < TPW && nt < NT16;
        const int n = min(nt * 16 + c, N - 1);
        vraw[u] = VA[n];
        kvc[u] = KI[n];
    }
    uint32_t vmask = 0;
    bool masked = false;
    float dkinv_acc[READ_TPW] = {};
    f32x4 acc_dk[ACC ? READ_TPW : 1][ACC ? DT : 1];
    f32x4 acc_dv[ACC ? READ_TPW : 1][ACC ? DT : 1];
    if constexpr (ACC) {
#pragma unroll
        for (int u = 0; u < READ_TPW; u++)
#pragma unroll
            for (int dt = 0; dt < DT; dt++) { acc_dk[u][dt] = f32x4{0.f, 0.f, 0.f, 0.f}; acc_dv[u][dt] = f32x4{0.f, 0.f, 0.f, 0.f}; }
    }

    // The dK / dV output rows of this wave's slots, one matrix and PD dims per pass (64 at D = 128, 32 at
    // D = 64: what the wave's rows of s_part hold): the D layout of a (slot tile u, dim tile dt) fragment
    // (row dim 16dt + 4g + i, column slot 16nt + c, so 4 consecutive dims of one slot per lane) goes to LDS as
    // row-major bf16, PD * 2 bytes per slot with the 8-byte pieces XOR-swizzled by the row, and comes back as
    // whole 16-byte pieces of each row, so that the stores fill whole lines (8-byte stores of 16 rows per
    // instruction had cost half the kernel).  frag(u, dt) gives the fragment; the caller owns s_part.
    constexpr int PD = READ_TPW * 16 * 128 <= 16 * OST * 4 ? 64 : 32;
    constexpr int RB = 2 * PD, S8 = RB / 8, C16 = RB / 16;   // row bytes, 8-byte slots, 16-byte chunks
    static_assert(READ_TPW * 16 * RB <= 16 * OST * 4, "a pass fits the wave's partial rows");
    unsigned char* tw = reinterpret_cast<unsigned char*>(s_part + w * 16 * OST);
    auto emit_rows = [&](bf16_t* dst, int hf, auto frag) {
#pragma unroll
        for (int dd = 0; dd < PD / 16; dd++) {
#pragma unroll
            for (int u = 0; u < READ_TPW; u++) {              // tiles past N carry zero draw and P
                const f32x4 r = frag(u, (PD / 16) * hf + dd);
                const int row = u * 16 + c, s8 = 4 * dd + g;
                *reinterpret_cast<uint2*>(tw + row * RB + 8 * (s8 ^ (row & (S8 - 1)))) =
                    make_uint2(pack2(r[0], r[1]), pack2(r[2], r[3]));
            }
        }
        wave_lds_sync();
#pragma unroll
        for (int k = 0; k < READ_TPW * 16 * C16 / 64; k++) {
            const int idx = 64 * k + lane, row = idx / C16, ch = idx % C16, x = row & (S8 - 1);
            uint4 v = *reinterpret_cast<const uint4*>(tw + row * RB + 16 * (ch ^ (x >> 1)));
            if (x & 1) v = make_uint4(v.z, v.w, v.x, v.y);
            const int n = w * TPW * 16 + row;
            if (row < TPW * 16 && n < N) st16_stream(dst + (size_t)n * D + PD * hf + 8 * ch, v);
        }
        wave_lds_sync();                                      // the reads are done before the next pass writes
    };

    for (int m0 = 0; m0 < Mblk; m0 += 16) {
        // ---- (a) the 16-query tile of Q and dO, and the multipliers, into LDS
        for (int e = threadIdx.x; e < 16 * (D / 8); e += READ_THREADS) {
            const int r = e / (D / 8), cc = e % (D / 8);
            const int m = m0 + r;
            uint4 xq = make_uint4(0, 0, 0, 0), xd = make_uint4(0, 0, 0, 0);
            if (m < Mblk) {
                const size_t row = (((size_t)b * a.T + t0 + m / a.NQ) * a.H + h) * a.NQ + (m % a.NQ);
                xq = *reinterpret_cast<const uint4*>(a.q + row * D + cc * 8);
                xd = *reinterpret_cast<const uint4*>(a.drd + row * D + cc * 8);
            }
            *reinterpret_cast<uint4*>(s_q + r * TST + cc * 8) = xq;
            *reinterpret_cast<uint4*>(s_do + r * TST + cc * 8) = xd;
        }
        if (threadIdx.x < 16) {
            const int m = m0 + threadIdx.x;
            float sv = 0.f;
            if (m < Mblk) sv = a.scale[(((size_t)b * a.T + t0 + m / a.NQ) * a.H + h) * a.NQ + (m % a.NQ)];
            s_scl[threadIdx.x] = sv;
        }
        __syncthreads();
        if (!masked) {                                     // once: the slot masks of the raw loads above
            masked = true;
#pragma unroll
            for (int u = 0; u < READ_TPW; u++) {
                const bool ok = tile[u] && (w * TPW + u) * 16 + c < N && vraw[u] != 0u;
                kvc[u] = ok ? kvc[u] : 0.f;
                vmask |= (ok ? 1u : 0u) << u;
            }
        }
        float scl[4];
#pragma unroll
        for (int i = 0; i < 4; i++) scl[i] = s_scl[4 * g + i];

        // ---- (b) scores S = Q K^T and datt = dO V^T, D layout: rows m = 4g + i, column n = 16 nt + c
        f32x4 sacc[READ_TPW], dacc[READ_TPW];
        {
            uint4 qa[KK], da[KK];
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                qa[kk] = *reinterpret_cast<const uint4*>(s_q + c * TST + kk * 32 + 8 * g);
                da[kk] = *reinterpret_cast<const uint4*>(s_do + c * TST + kk * 32 + 8 * g);
            }
#pragma unroll
            for (int u = 0; u < READ_TPW; u++) {
                sacc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
                dacc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
                const int n = (w * TPW + u) * 16 + c;
                const bool in = tile[u] && n < N;
                const size_t nc = (size_t)min(n, N - 1) * D;          // clamped address, then select
                constexpr int KB = RBWD_KBATCH < KK ? RBWD_KBATCH : KK;   // loads per batch, per operand
#pragma unroll
                for (int k0 = 0; k0 < KK; k0 += KB) {
                    uint4 kx[KB], vx[KB];
#pragma unroll
                    for (int kk = 0; kk < KB; kk++) {
                        kx[kk] = *reinterpret_cast<const uint4*>(Kb + nc + (k0 + kk) * 32 + 8 * g);
                        vx[kk] = *reinterpret_cast<const uint4*>(Vb + nc + (k0 + kk) * 32 + 8 * g);
                    }
#pragma unroll
                    for (int kk = 0; kk < KB; kk++) {
                        sacc[u] = mfma_k32(qa[k0 + kk], in ? kx[kk] : make_uint4(0, 0, 0, 0), sacc[u]);
                        dacc[u] = mfma_k32(da[k0 + kk], in ? vx[kk] : make_uint4(0, 0, 0, 0), dacc[u]);
                    }
                }
            }
        }
        // ---- (c) softmax statistics per query row over all slots (DPP rows, then the 4 waves)
        float raw[READ_TPW][4], sc[READ_TPW][4];
        float mx[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            mx[i] = -INFINITY;
#pragma unroll
            for (int u = 0; u < READ_TPW; u++) {
                raw[u][i] = bf16r(sacc[u][i]);
                sc[u][i] = raw[u][i] * kvc[u] * scl[i];
                if ((vmask >> u) & 1u) mx[i] = fmaxf(mx[i], sc[u][i]);
            }
            mx[i] = rowmax16(mx[i]);
        }
        if (c == 0) {
#pragma unroll
            for (int i = 0; i < 4; i++) s_red[0][w][4 * g + i] = mx[i];
        }
        __syncthreads();
        float inv[4];
        {
            float sm[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = 4 * g + i;
                const float M = fmaxf(fmaxf(s_red[0][0][m], s_red[0][1][m]), fmaxf(s_red[0][2][m], s_red[0][3][m]));
                sm[i] = 0.f;
#pragma unroll
                for (int u = 0; u < READ_TPW; u++) {
                    const float e = ((vmask >> u) & 1u) ? __expf(sc[u][i] - M) : 0.f;
                    sc[u][i] = e;
                    sm[i] += e;
                }
                sm[i] = rowsum16(sm[i]);
            }
            if (c == 0) {
#pragma unroll
                for (int i = 0; i < 4; i++) s_red[1][w][4 * g + i] = sm[i];
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = 4 * g + i;
                const float S = ((s_red[1][0][m] + s_red[1][1][m]) + s_red[1][2][m]) + s_red[1][3][m];
                inv[i] = S > 0.f ? 1.f / S : 0.f;
            }
        }
        // att (fp32) in sc, datt = bf16(dO V^T), delta = sum_n att * datt
        float dat[READ_TPW][4];
        {
            float dl[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                dl[i] = 0.f;
#pragma unroll
                for (int u = 0; u < READ_TPW; u++) {
                    sc[u][i] *= inv[i];
                    dat[u][i] = bf16r(dacc[u][i]);
                    dl[i] += sc[u][i] * dat[u][i];
                }
                dl[i] = rowsum16(dl[i]);
            }
            if (c == 0) {
#pragma unroll
                for (int i = 0; i < 4; i++) s_red[2][w][4 * g + i] = dl[i];
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = 4 * g + i;
                const float delta = ((s_red[2][0][m] + s_red[2][1][m]) + s_red[2][2][m]) + s_red[2][3][m];
#pragma unroll
                for (int u = 0; u < READ_TPW; u++) dat[u][i] = sc[u][i] * (dat[u][i] - delta);   // dsc
            }
        }
        // draw = bf16(dsc * kinv * scale), P = bf16(att); dkinv / dscale partials
        uint2 drB[READ_TPW], pB[READ_TPW];
        float dsl[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < READ_TPW; u++) {
            float dr[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float dsc = dat[u][i];
                dr[i] = dsc * kvc[u] * scl[i];
                dkinv_acc[u] += dsc * raw[u][i] * scl[i];
                dsl[i] += dsc * raw[u][i] * kvc[u];
            }
            drB[u].x = pack2(dr[0], dr[1]);
            drB[u].y = pack2(dr[2], dr[3]);
            pB[u].x = pack2(sc[u][0], sc[u][1]);
            pB[u].y = pack2(sc[u][2], sc[u][3]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) dsl[i] = rowsum16(dsl[i]);
        if (c == 0) {
#pragma unroll
            for (int i = 0; i < 4; i++) s_dsc[w][4 * g + i] = dsl[i];
        }
        // ---- (d) dK^T = Q^T draw and dV^T = dO^T P, per (slot tile, dim tile)
        if constexpr (ACC) {
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                const uint2 qT = gather4(s_q + (4 * g) * TST + dt * 16 + c, TST);    // A: row dim 16dt + c, k = query 4g + i
                const uint2 dT = gather4(s_do + (4 * g) * TST + dt * 16 + c, TST);
#pragma unroll
                for (int u = 0; u < READ_TPW; u++) {            // tiles past N carry zero draw and P
                    acc_dk[u][dt] = mfma_k16(qT, drB[u], acc_dk[u][dt]);
                    acc_dv[u][dt] = mfma_k16(dT, pB[u], acc_dv[u][dt]);
                }
            }
        } else {
            // one matrix and PD dims per pass through the wave's rows of s_part (free until (e))
#pragma unroll
            for (int hf = 0; hf < D / PD; hf++)
                emit_rows(dKb, hf, [&](int u, int dt) {
                    const uint2 aT = gather4(s_q + (4 * g) * TST + dt * 16 + c, TST);   // A: row dim 16dt + c, k = query
                    return mfma_k16(aT, drB[u], f32x4{0.f, 0.f, 0.f, 0.f});
                });
#pragma unroll
            for (int hf = 0; hf < D / PD; hf++)
                emit_rows(dVb, hf, [&](int u, int dt) {
                    const uint2 aT = gather4(s_do + (4 * g) * TST + dt * 16 + c, TST);
                    return mfma_k16(aT, pB[u], f32x4{0.f, 0.f, 0.f, 0.f});
                });
        }
        // ---- (e) dQ^T partial = K^T draw^T over this wave's slots
        bf16_t* dr_t = s_dr[w];
#pragma unroll
        for (int u = 0; u < READ_TPW; u++) {                 // draw tile [query m][slot], row = m
            const uint32_t v2[2] = {drB[u].x, drB[u].y};
#pragma unroll
            for (int i = 0; i < 4; i++)
                dr_t[(4 * g + i) * RST + u * 16 + c] = (bf16_t)(v2[i >> 1] >> (16 * (i & 1)));
        }
        wave_lds_sync();
        // K^T (A: row dim 16dt + c, k = slot 16 nt + 4g + i) goes through this wave's own rows of s_part,
        // which are free until its partials are written, half the dims at a time: the key rows are read
        // again as 16-byte loads (cache hits: (b) just read them) and written transposed.  Gathering the
        // operand as 2-byte loads from the key rows cost more than the rest of the kernel.
        constexpr int KTS = READ_TPW * 16 + 4;              // K^T row stride (bf16): 8-byte aligned rows
        constexpr int HD = D / 2;
        static_assert(HD * KTS * 2 <= 16 * OST * 4, "a K^T half fits the wave's partial rows");
        bf16_t* kt_w = reinterpret_cast<bf16_t*>(s_part + w * 16 * OST);
        f32x4 o[DT];
#pragma unroll
        for (int dt = 0; dt < DT; dt++) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            if (hh) wave_lds_sync();                          // the first half's reads are done
#pragma unroll
            for (int u = 0; u < READ_TPW; u++) {
                const int n = (w * TPW + u) * 16 + c;
                const bool in = tile[u] && n < N;
                const size_t nc = (size_t)min(n, N - 1) * D;  // clamped address, then select
#pragma unroll
                for (int k2 = 0; k2 < HD / 32; k2++) {
                    const uint4 kx = *reinterpret_cast<const uint4*>(Kb + nc + (hh * (HD / 32) + k2) * 32 + 8 * g);
                    const uint32_t w4[4] = {in ? kx.x : 0u, in ? kx.y : 0u, in ? kx.z : 0u, in ? kx.w : 0u};
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        kt_w[(k2 * 32 + 8 * g + e) * KTS + u * 16 + c] = (bf16_t)(w4[e >> 1] >> (16 * (e & 1)));
                }
            }
            wave_lds_sync();
#pragma unroll
            for (int d2 = 0; d2 < HD / 16; d2++) {
                const int dt = hh * (HD / 16) + d2;
#pragma unroll
                for (int u = 0; u < READ_TPW; u++) {
                    const uint2 kT = *reinterpret_cast<const uint2*>(kt_w + (d2 * 16 + c) * KTS + u * 16 + 4 * g);
                    const uint2 drT = *reinterpret_cast<const uint2*>(dr_t + c * RST + u * 16 + 4 * g);   // B: k = slot, column m = c
                    o[dt] = mfma_k16(kT, drT, o[dt]);
                }
            }
        }
        wave_lds_sync();                                      // every lane's K^T reads are done
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
            *reinterpret_cast<f32x4*>(s_part + (w * 16 + c) * OST + dt * 16 + 4 * g) = o[dt];
        __syncthreads();
        {
            constexpr int EPT = D / 16;
            const int mr = threadIdx.x >> 4, dc = (threadIdx.x & 15) * EPT;
            const int mm = m0 + mr;
            if (mm < Mblk) {
                float r[EPT];
#pragma unroll
                for (int e = 0; e < EPT; e++) r[e] = s_part[mr * OST + dc + e];
#pragma unroll
                for (int ww = 1; ww < READ_WAVES; ww++)
#pragma unroll
                    for (int e = 0; e < EPT; e++) r[e] += s_part[(ww * 16 + mr) * OST + dc + e];
                const size_t row = (((size_t)b * a.T + t0 + mm / a.NQ) * a.H + h) * a.NQ + (mm % a.NQ);
                bf16_t* dst = a.dq + row * D + dc;
                if constexpr (EPT == 8) {
                    uint4 x;
                    x.x = pack2(r[0], r[1]); x.y = pack2(r[2], r[3]); x.z = pack2(r[4], r[5]); x.w = pack2(r[6], r[7]);
                    st16_stream(dst, x);
                } else {
                    uint2 x;
                    x.x = pack2(r[0], r[1]); x.y = pack2(r[2], r[3]);
                    *reinterpret_cast<uint2*>(dst) = x;
                }
                if ((threadIdx.x & 15) == 0)
                    a.dscale[row] = ((s_dsc[0][mr] + s_dsc[1][mr]) + s_dsc[2][mr]) + s_dsc[3][mr];
            }
        }
    }
    // ---- dkinv per slot: this lane's column, summed over the 4 query row groups
#pragma unroll
    for (int u = 0; u < READ_TPW; u++) {
        const float v = sum4rows(dkinv_acc[u]);
        const int n = (w * TPW + u) * 16 + c;
        if (tile[u] && g == 0 && n < N) a.dkinv[(size_t)slab * N + n] = v;
    }
    if constexpr (ACC) {
        __syncthreads();                                      // every wave's reads of the last partials are done
#pragma unroll
        for (int hf = 0; hf < D / PD; hf++) emit_rows(dKb, hf, [&](int u, int dt) { return acc_dk[u][dt]; });
#pragma unroll
        for (int hf = 0; hf < D / PD; hf++) emit_rows(dVb, hf, [&](int u, int dt) { return acc_dv[u][dt]; });
    }
}

}  // namespace

// ======================================================================================== C-ABI

static int check_read(int64_t B, int64_t T, int64_t H, int64_t NQ, int64_t N, int64_t D, int64_t G) {
    if (B < 1 || T < 1 || H < 1 || NQ < 1 || N < 1 || G < 1)
        return fail(SLOTSCAN_ERR_SHAPE, "slotread: B, T, H, NQ, N and G must be >= 1");
    if (D != 64 && D != 128) return fail(SLOTSCAN_ERR_SHAPE, "slotread: D must be 64 or 128");
    if (N > READ_WAVES * READ_TPW * 16) return fail(SLOTSCAN_ERR_SHAPE, "slotread: N must be <= 192");
    const int64_t NB = (T + G - 1) / G;
    if (B * NB * H > 0x7fffffffLL || G * NQ > 0x7fffffffLL)
        return fail(SLOTSCAN_ERR_SHAPE, "slotread: B*NB*H and G*NQ must fit in int32");
    return 0;
}

// query rows per workgroup: enough workgroups to fill 256 CUs a few times over, at least one 16-row tile
#ifndef READ_TARGET_WGS
#define READ_TARGET_WGS 768
#endif
#ifndef READ_WIDE_MIN_M
#define READ_WIDE_MIN_M 256                      // queries per block from which the wide kernel is used
#endif
static int read_rows_per_wg(int64_t slabs, int64_t Mfull) {
    const int64_t tiles = (Mfull + 15) / 16;
    int64_t split = (READ_TARGET_WGS + slabs - 1) / slabs;
    if (split > tiles) split = tiles;
    if (split < 1) split = 1;
    const int64_t per = (tiles + split - 1) / split;
    return (int)(per * 16);
}

// compute units of the current device (cached per device)
static int cu_count() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cache[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

extern "C" int slotread_fwd(const void* q, const void* kbuf, const void* vbuf, const float* kinv,
                            const uint8_t* valid, const float* scale, int64_t B, int64_t T, int64_t H, int64_t NQ,
                            int64_t N, int64_t D, int64_t G, void* rd, void* stream) {
    if (int r = check_read(B, T, H, NQ, N, D, G)) return r;
    if (!q || !kbuf || !vbuf || !kinv || !valid || !scale || !rd)
        return fail(SLOTSCAN_ERR_NULL, "slotread_fwd: a required pointer is NULL");
    if (!al16(q) || !al16(kbuf) || !al16(vbuf) || !al16(rd))
        return fail(SLOTSCAN_ERR_ALIGN, "slotread_fwd: q, kbuf, vbuf and rd must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    const int64_t NB = (T + G - 1) / G;
    const int64_t slabs = B * NB * H;
    const int MC = read_rows_per_wg(slabs, G * NQ);
    const int64_t ysplit = (G * NQ + MC - 1) / MC;
    ReadFwdArgs ra{(const bf16_t*)q, (const bf16_t*)kbuf, (const bf16_t*)vbuf, kinv, valid, scale, (bf16_t*)rd,
                   (int)T, (int)H, (int)NQ, (int)N, (int)G, (int)NB, MC, (int)slabs, 1};
    dim3 grid((unsigned)slabs, (unsigned)ysplit), block(READ_THREADS);
    hipError_t e;
    {
        slothost::Scope sc(SLOTSCAN_K_READ_FWD, st);
        if (G * NQ >= READ_WIDE_MIN_M) {
            // many queries per block, persistent: one workgroup per CU (the 147 KB of LDS hold one), each walking
            // a contiguous range of the query chunks (32 queries per wave)
            ra.MC = 32 * WIDE_WAVES;
            ra.parts = (int)((G * NQ + ra.MC - 1) / ra.MC);   // chunks per slab
            const int64_t chunks = slabs * ra.parts;
            if (chunks > 0x7fffffffLL) return fail(SLOTSCAN_ERR_SHAPE, "slotread_fwd: B*NB*H*ceil(G*NQ/256) must fit in int32");
            dim3 wgrid((unsigned)std::min<int64_t>(chunks, cu_count())), wblock(WIDE_THREADS);
            if (D == 128) slothost::launch(read_fwd_wide<128>, wgrid, wblock, 0, st, ra);
            else slothost::launch(read_fwd_wide<64>, wgrid, wblock, 0, st, ra);
        } else {
            if (D == 128) slothost::launch(read_fwd<128>, grid, block, 0, st, ra);
            else slothost::launch(read_fwd<64>, grid, block, 0, st, ra);
        }
        e = hipGetLastError();
    }
    if (e != hipSuccess) return hip_fail(e, "read_fwd launch");
    return 0;
}

extern "C" int slotread_bwd(const void* q, const void* kbuf, const void* vbuf, const float* kinv,
                            const uint8_t* valid, const float* scale, const void* drd, int64_t B, int64_t T,
                            int64_t H, int64_t NQ, int64_t N, int64_t D, int64_t G, void* dq, void* dkbuf,
                            void* dvbuf, float* dkinv, float* dscale, void* stream) {
    if (int r = check_read(B, T, H, NQ, N, D, G)) return r;
    if (!q || !kbuf || !vbuf || !kinv || !valid || !scale || !drd || !dq || !dkbuf || !dvbuf || !dkinv || !dscale)
        return fail(SLOTSCAN_ERR_NULL, "slotread_bwd: a required pointer is NULL");
    if (!al16(q) || !al16(kbuf) || !al16(vbuf) || !al16(drd) || !al16(dq) || ((uintptr_t)dkbuf & 7u) ||
        ((uintptr_t)dvbuf & 7u))
        return fail(SLOTSCAN_ERR_ALIGN, "slotread_bwd: q, kbuf, vbuf, drd, dq must be 16-byte aligned (dkbuf, dvbuf 8)");
    hipStream_t st = (hipStream_t)stream;
    const int64_t NB = (T + G - 1) / G;
    ReadBwdArgs ra{(const bf16_t*)q, (const bf16_t*)kbuf, (const bf16_t*)vbuf, kinv, valid, scale,
                   (const bf16_t*)drd, (bf16_t*)dq, (bf16_t*)dkbuf, (bf16_t*)dvbuf, dkinv, dscale,
                   (int)T, (int)H, (int)NQ, (int)N, (int)G, (int)NB};
    dim3 grid((unsigned)(B * NB * H)), block(READ_THREADS);
    const bool acc = G * NQ > 16;
    hipError_t e;
    {
        slothost::Scope sc(SLOTSCAN_K_READ_BWD, st);
        if (D == 128) {
            if (acc) slothost::launch((read_bwd<128, true>), grid, block, 0, st, ra);
            else slothost::launch((read_bwd<128, false>), grid, block, 0, st, ra);
        } else {
            if (acc) slothost::launch((read_bwd<64, true>), grid, block, 0, st, ra);
            else slothost::launch((read_bwd<64, false>), grid, block, 0, st, ra);
        }
        e = hipGetLastError();
    }
    if (e != hipSuccess) return hip_fail(e, "read_bwd launch");
    return 0;
}
