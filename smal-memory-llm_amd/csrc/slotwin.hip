// Rolling-window attention (the exact short-term window every layer runs beside the slot memory) for
// MI355X (gfx950), as bf16 MFMA contractions.
//
// Semantics (reference: /root/reference/gqa25/memlm_sh.py:340-359, SharedMixer._window): scaled dot-product
// attention over the last W tokens, allowed[i, j] = (i >= j) & (i - j < W), scale 1/sqrt(D) by default:
//   s[i, j] = scale <q_i, k_j>,  p[i, :] = softmax over the allowed j,  o_i = sum_j p[i, j] v_j.
// Query head hq reads key/value head hq / (Hq / Hk): the kv_nq path attends its extra queries to
// repeat_interleave'd keys and values (memlm_sh.py:488-492), which is the same mapping without the copies.
// Tensors are token-major (B, T, H, D) bf16, the layout the reference's (B, H, T, D) views are transposed
// from (memlm_sh.py:482-484).  W <= 16, so a 16-query tile sees at most two 16-key tiles.
//
// gfx950 mapping.  One wave per 16-row tile, 4 waves per workgroup:
//   forward   per 64-token tile and key/value head, the staged values and each wave's key operands serve
//             every query head of the group; S^T (keys x queries) = K Q^T with v_mfma_f32_16x16x32_bf16
//             (keys as the A rows, queries as the B columns, D/32 k-steps) for the two key tiles; the D
//             layout puts one query column in every lane (4 keys per lane per tile), so the band softmax
//             is 8 values per lane and one cross-row reduction; O^T = V^T P^T with
//             v_mfma_f32_16x16x16_bf16, whose B operand is exactly the score tile's D layout (the
//             exponentials are rounded to bf16 unnormalised and the sum divides at the end).  V^T is
//             gathered from value rows staged in LDS.  The log-sum-exp of every query is kept for the
//             backward.
//   backward  one pass per 128-key run: per key tile, queries as the A rows, S and dP (queries x keys) for
//             the two query tiles that see the keys, dS = P (dP - rowsum(dO o O)), then dV^T = dO^T P and
//             dK^T = Q^T dS, whose B operands are again the D layout; the dS tiles go through LDS transposed
//             for dQ^T = K^T dS^T.  The query heads of a key/value head are summed in the kernel: no
//             atomics, bitwise reproducible.
#include "slot_common.h"
#include "slotscan.h"
#include "slotwin.h"
#include "slot_host.h"

using namespace slot;
using slothost::fail;
using slothost::hip_fail;
using slothost::al16;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

#define WIN_WAVES 4
#define WIN_THREADS (64 * WIN_WAVES)
#define WIN_TILE (16 * WIN_WAVES)                    // query (or key) rows per workgroup
#define WIN_STAGE (WIN_TILE + 16)                    // staged rows: the tile plus the 16 rows the band reaches
#ifndef WIN_BWD_WAVES
#define WIN_BWD_WAVES 4                              // backward: waves (16-key tiles) per workgroup; 4 fits two
#endif                                               // workgroups (75 KB of LDS each) on a CU

namespace {

__device__ __forceinline__ f32x4 mfma_k32(const uint4& a, const uint4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_k16(const uint2& a, const uint2& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                     0, 0, 0);
}
// max over the 4 row groups of a wave (lanes c, c+16, c+32, c+48), at every lane
__device__ __forceinline__ float max4rows(float v) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    float s = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ uint4 ld16(const bf16_t* p) { return *reinterpret_cast<const uint4*>(p); }
// 4 bf16 down a staged column: rows r, r+1, r+2, r+3 of column col -> one k16 operand (k = row)
template <int ST>
__device__ __forceinline__ uint2 gather4(const bf16_t* s, int r, int col) {
    const bf16_t* p = s + r * ST + col;
    uint2 x;
    x.x = (uint32_t)p[0] | ((uint32_t)p[ST] << 16);
    x.y = (uint32_t)p[2 * ST] | ((uint32_t)p[3 * ST] << 16);
    return x;
}
// Wave-local LDS ordering (DS instructions of a wave execute in order; the fences keep the compiler from
// moving the accesses across)
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// 16 rows of D bf16 from a wave's MFMA D-layout fragments (lane (c, g) holds dims 16 dt + 4 g .. + 3 of row c:
// frag(dt)) through 32 D bytes of the wave's LDS (row-major, 8-byte pieces XOR-swizzled by the row), stored as
// whole 16-byte pieces of each row (rowp(r): the row's address, or nullptr to skip it), so that a store
// instruction writes 4 whole rows instead of 32 bytes of each of 16 rows
template <int D, class F, class R>
__device__ __forceinline__ void emit_rows16(unsigned char* lw, int lane, F frag, R rowp) {
    constexpr int RBY = 2 * D, C16 = RBY / 16;           // row bytes, 16-byte chunks per row
    const int c = lane & 15, g = lane >> 4;
#pragma unroll
    for (int dt = 0; dt < D / 16; dt++) {
        const f32x4 o = frag(dt);
        const int s8 = 4 * dt + g;                        // the 8-byte piece of row c
        *reinterpret_cast<uint2*>(lw + c * RBY + 8 * (s8 ^ c)) = make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
    }
    wave_lds_sync();
#pragma unroll
    for (int k = 0; k < 16 * C16 / 64; k++) {
        const int idx = 64 * k + lane, r = idx / C16, ch = idx % C16;
        uint4 v = *reinterpret_cast<const uint4*>(lw + r * RBY + 16 * (ch ^ (r >> 1)));
        if (r & 1) v = make_uint4(v.z, v.w, v.x, v.y);
        bf16_t* q = rowp(r);
        if (q) {                                         // written once: a streaming store (window_train 0.736 -> 0.717 ms/step)
            const u32x4v y = {v.x, v.y, v.z, v.w};
            __builtin_nontemporal_store(y, reinterpret_cast<u32x4v*>(q + 8 * ch));
        }
    }
    wave_lds_sync();                                      // the reads are done before the region is reused
}
__device__ __forceinline__ float dot8(uint4 x, uint4 y) {     // <x, y> of 8 bf16 pairs, fp32
    const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, ys[4] = {y.x, y.y, y.z, y.w};
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        s = fmaf(__uint_as_float(xs[i] << 16), __uint_as_float(ys[i] << 16), s);
        s = fmaf(__uint_as_float(xs[i] & 0xffff0000u), __uint_as_float(ys[i] & 0xffff0000u), s);
    }
    return s;
}

struct WinArgs {
    const bf16_t* q; const bf16_t* k; const bf16_t* v; const bf16_t* o; const float* lse; const bf16_t* dO;
    bf16_t* out; float* lse_out; bf16_t* dq; bf16_t* dk; bf16_t* dv; float* dsum;
    int T, Hq, Hk, W;
    float scale;
};

// Rows [r0, r0 + NR) of head h of x (B, T, H, D), staged by NT threads into s (row stride ST, zeros outside
// [0, T)).  load() issues every piece of a lane back to back, unconditionally, from in-range addresses (a
// piece past the rows or outside [0, T) reads row clamp(t)), so they are in flight together and nothing
// waits for them before store(), which zeroes those pieces and writes the rest to LDS.  A load per piece
// behind a branch, or a select right after it, would wait for each piece in turn.
template <int D, int ST, int NR = WIN_STAGE, int NT = WIN_THREADS>
struct StagedRows {
    static constexpr int RU = D / 8, NE = NR * RU, NI = (NE + NT - 1) / NT;
    uint4 v[NI];
    __device__ __forceinline__ void load(const bf16_t* x, int b, int T, int H, int h, int r0, int tid) {
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int e = tid + NT * i, r = e / RU, cc = e - (e / RU) * RU;
            const int tc = min(max(r0 + r, 0), T - 1);
            v[i] = ld16(x + (((size_t)b * T + tc) * H + h) * D + cc * 8);
        }
    }
    __device__ __forceinline__ void store(bf16_t* s, int T, int r0, int tid) const {
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int e = tid + NT * i, r = e / RU, cc = e - (e / RU) * RU, t = r0 + r;
            if (e < NE) *reinterpret_cast<uint4*>(s + r * ST + cc * 8) = (t >= 0 && t < T) ? v[i] : make_uint4(0u, 0u, 0u, 0u);
        }
    }
};
template <int D, int ST, int NR = WIN_STAGE, int NT = WIN_THREADS>
__device__ __forceinline__ void stage_rows(bf16_t* s, const bf16_t* x, int b, int T, int H, int h, int r0, int tid) {
    StagedRows<D, ST, NR, NT> rows;
    rows.load(x, b, T, H, h, r0, tid);
    rows.store(s, T, r0, tid);
}

__device__ __forceinline__ bool allowed(int tq, int j, int T, int W) {
    return tq < T && j >= 0 && j <= tq && tq - j < W;
}

// ------------------------------------------------------------------------------------------- forward
template <int D>
__global__ __launch_bounds__(WIN_THREADS) void win_fwd(WinArgs a) {
    constexpr int KK = D / 32, DT = D / 16, ST = D + 8;
    __shared__ __align__(16) bf16_t sV[WIN_STAGE * ST];
    __shared__ __align__(16) unsigned char sO[WIN_WAVES][32 * D];   // a wave's output rows on their way out
    const int T = a.T, Hq = a.Hq, Hk = a.Hk, W = a.W, R = Hq / Hk;
    const int b = blockIdx.z, hk = blockIdx.y;        // every query head of key/value head hk
    const int t0 = blockIdx.x * WIN_TILE;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
    // this wave's first query and key operands first, so that their latency overlaps the value staging's;
    // the keys and staged values serve every query head of the group
    const int qt = t0 + 16 * w;
    const int tq = qt + c;                            // this lane's query column
    const bool qok = tq < T;
    const size_t qrow0 = ((size_t)b * T + (qok ? tq : 0)) * Hq + hk * R;    // (b, tq, first head of the group)
    auto load_q = [&](int r, uint4* qf) {
#pragma unroll
        for (int kk = 0; kk < KK; kk++) qf[kk] = qok ? ld16(a.q + (qrow0 + r) * D + 32 * kk + 8 * g) : make_uint4(0u, 0u, 0u, 0u);
    };
    uint4 qn[KK], kf[2][KK];
    load_q(0, qn);
#pragma unroll
    for (int u = 0; u < 2; u++) {                      // key tile u: keys qt - 16 + 16 u + (0..15)
        const int j = qt - 16 + 16 * u + c;
        const bool jok = j >= 0 && j < T;
        const bf16_t* krow = a.k + (((size_t)b * T + (jok ? j : 0)) * Hk + hk) * D;
#pragma unroll
        for (int kk = 0; kk < KK; kk++) kf[u][kk] = jok ? ld16(krow + 32 * kk + 8 * g) : make_uint4(0u, 0u, 0u, 0u);
    }
    stage_rows<D, ST>(sV, a.v, b, T, Hk, hk, t0 - 16, tid);
    __syncthreads();
    if (qt >= T) return;                              // no barrier follows
    for (int r = 0; r < R; r++) {
        const int hq = hk * R + r;
        uint4 qf[KK];
#pragma unroll
        for (int kk = 0; kk < KK; kk++) qf[kk] = qn[kk];
        if (r + 1 < R) load_q(r + 1, qn);             // the next head's queries in flight
        f32x4 acc[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KK; kk++) acc[u] = mfma_k32(kf[u][kk], qf[kk], acc[u]);
        }
        // band softmax of query column tq: lane (c, g) holds keys qt - 16 + 16 u + 4 g + i
        float s[2][4];
        float mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int j = qt - 16 + 16 * u + 4 * g + i;
                s[u][i] = allowed(tq, j, T, W) ? acc[u][i] * a.scale : -INFINITY;
                mx = fmaxf(mx, s[u][i]);
            }
        mx = max4rows(mx);
        float l = 0.f;
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float e = s[u][i] == -INFINITY ? 0.f : __expf(s[u][i] - mx);
                s[u][i] = e;
                l += e;
            }
        l = sum4rows(l);
        uint2 pf[2];                                   // bf16 exponentials: the B operand (k = key, col = query)
#pragma unroll
        for (int u = 0; u < 2; u++) pf[u] = make_uint2(pack_bf16x2(s[u][0], s[u][1]), pack_bf16x2(s[u][2], s[u][3]));
        const float inv = l > 0.f ? 1.f / l : 0.f;
        emit_rows16<D>(sO[w], lane, [&](int dt) {
            f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < 2; u++) o = mfma_k16(gather4<ST>(sV, 16 * w + 16 * u + 4 * g, 16 * dt + c), pf[u], o);
            return f32x4{o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv};
        }, [&](int rr) { return qt + rr < T ? a.out + ((((size_t)b * T + qt + rr) * Hq + hq) * D) : (bf16_t*)nullptr; });
        if (qok && g == 0) a.lse_out[((size_t)b * Hq + hq) * T + tq] = mx + __logf(l);
    }
}

// ------------------------------------------------------------------------------------ backward, one pass
// One workgroup of NW waves per run of 16 NW keys [k0, k0 + 16 NW) of key/value head hk; wave w owns key tile
// kt = k0 + 16 w and query tile kt (the same token rows).  Per query head of the group:
//   stage   q and dout rows [k0, k0 + 16 NW + 16) (the query tiles kt and kt + 16 that see key tile kt), their
//           log-sum-exp, and D = rowsum(dout o out), reduced across the 16-byte chunks of a row as the
//           staging loads arrive;
//   dk, dv  per wave and u in {0, 1}: S and dP (queries kt + 16 u x keys kt, queries as the A rows), P and
//           dS, then dV^T += dO^T P and dK^T += Q^T dS (B operands = the D layout), summed over the heads;
//   dq      every dS tile goes to LDS transposed (queries x keys, keys contiguous), so that dQ^T = K^T dS^T
//           over key tiles kt - 16 and kt reads its B operand as one 8-byte load: wave w's own u = 0 tile
//           and wave w - 1's u = 1 tile; wave 0 computes the pair (query tile k0, key tile k0 - 16) itself.
// S and dP are computed once per (query tile, key tile) pair for all three gradients.
template <int D, int NW>
// At most 256 VGPRs (2 waves per SIMD): two 4-wave workgroups share a CU, one staging while the other computes
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void win_bwd(WinArgs a) {
    constexpr int NTH = 64 * NW, TILE = 16 * NW, STG = TILE + 16;   // threads, keys per workgroup, staged rows
    constexpr int KK = D / 32, DT = D / 16, ST = D + 8, RU = D / 8;
    constexpr int TS = 20;                             // transposed dS row (bf16): 10 dwords, 16 rows on 32 banks
    __shared__ __align__(16) bf16_t sK[STG * ST];   // key rows [k0 - 16, k0 + 64)
    __shared__ __align__(16) bf16_t sQ[STG * ST];   // query rows [k0, k0 + 80) of the current head
    __shared__ __align__(16) bf16_t sD[STG * ST];   // dout rows, the same
    __shared__ __align__(16) bf16_t sVx[16 * ST];   // value rows [k0 - 16, k0)
    __shared__ float sL[STG], sDs[STG];        // their log-sum-exp and rowsum(dout o out)
    __shared__ __align__(16) bf16_t sT[NW + 1][2][16 * TS];   // dS tiles [query][key]; [WAVES] = wave 0's extra
    const int T = a.T, Hq = a.Hq, Hk = a.Hk, W = a.W, R = Hq / Hk;
    const int b = blockIdx.z, hk = blockIdx.y;
    const int k0 = blockIdx.x * TILE;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
    const int kt = k0 + 16 * w;                        // this wave's key tile and query tile
    unsigned char* ow = reinterpret_cast<unsigned char*>(sQ) + w * 32 * D;   // output rows, once sQ is read
    static_assert(NW * 32 * D <= STG * ST * 2, "every wave's output rows fit in sQ");
    const int j = kt + c;                              // lane column = key j (key/value pass)
    const bool jok = j < T;
    const size_t krow = ((size_t)b * T + (jok ? j : 0)) * Hk + hk;
    StagedRows<D, ST, STG, NTH> krows;                 // key rows [k0 - 16, k0 + 16 NW)
    krows.load(a.k, b, T, Hk, hk, k0 - 16, tid);
    StagedRows<D, ST, 16, NTH> vxrows;                 // value rows [k0 - 16, k0): wave 0's extra tile
    vxrows.load(a.v, b, T, Hk, hk, k0 - 16, tid);
    uint4 kb[KK], vb[KK];
#pragma unroll
    for (int kk = 0; kk < KK; kk++) {
        const uint4 z = make_uint4(0u, 0u, 0u, 0u);
        kb[kk] = jok ? ld16(a.k + krow * D + 32 * kk + 8 * g) : z;
        vb[kk] = jok ? ld16(a.v + krow * D + 32 * kk + 8 * g) : z;
    }
    f32x4 dkt[DT], dvt[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++) dkt[dt] = dvt[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // the dS of query tile u (rows 4 g + i) against this lane's key column, into the transposed tile
    auto put_ds = [&](bf16_t* tile, const float* ds) {
#pragma unroll
        for (int i = 0; i < 4; i++) tile[(4 * g + i) * TS + c] = f2bf(ds[i]);
    };
    // A head's rows [k0, k0 + 16 NW + 16) (the query tiles kt and kt + 16 that see key tile kt) are loaded one
    // head ahead, during the previous head's dq pass: the q rows and the log-sum-exp into registers, the dout
    // rows straight into sD by direct global -> LDS loads (its last reads are done by then; sQ is still the
    // dq rows' way out).  Pieces past T are zero.  The out rows, needed only for D = rowsum(dout o out), are
    // loaded in one batch when the head starts.
    constexpr int CPR = ST / 8;                         // 16-byte chunks of a padded row (the pad is not loaded)
    constexpr int NDI = (STG * CPR + NTH - 1) / NTH;    // direct loads per lane for the dout rows
    constexpr int NIT = (STG * RU + NTH - 1) / NTH;
    StagedRows<D, ST, STG, NTH> qrows;
    float lsev = 0.f;
    const unsigned sD0 = lds_addr(sD);
    // Every per-head index is derived from an opaque copy of the thread index, so the compiler does not hoist
    // dozens of loop-invariant 64-bit lane addresses and masks out of the head loop (they spilled)
    auto opaque_tid = [&]() { int x = tid; asm volatile("" : "+v"(x)); return x; };
    auto load_head = [&](int hq) {
        const int tl = opaque_tid();
        qrows.load(a.q, b, T, Hq, hq, k0, tl);
#pragma unroll
        for (int it = 0; it < NDI; it++) {
            const int L = NTH * it + tl, r = L / CPR, cc = L - (L / CPR) * CPR, t = k0 + r;
            if (r < STG && cc < RU) {                   // chunk L of sD: row r, 16-byte piece cc
                if (t < T) dma16(a.dO + (((size_t)b * T + t) * Hq + hq) * D + cc * 8, sD0 + 16u * (NTH * it + 64 * w));
                else *reinterpret_cast<uint4*>(sD + r * ST + cc * 8) = make_uint4(0u, 0u, 0u, 0u);
            }
        }
        lsev = a.lse[((size_t)b * Hq + hq) * T + min(k0 + min(tl, STG - 1), T - 1)];   // zeroed past T when stored
    };
    load_head(hk * R);
    krows.store(sK, T, k0 - 16, tid);
    vxrows.store(sVx, T, k0 - 16, tid);
    for (int r = 0; r < R; r++) {
        const int hq = hk * R + r;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this lane's direct loads into sD have landed
        __syncthreads();                               // sD complete; the previous head's dq rows are out of sQ
        const int tl = opaque_tid();
        uint4 orows[NIT];                              // out rows, in the order of the D reduction below
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int e = tl + NTH * it, rr = e / RU, cc = e - (e / RU) * RU, t = k0 + rr;
            const uint4 ov = ld16(a.o + (((size_t)b * T + min(t, T - 1)) * Hq + hq) * D + cc * 8);
            orows[it] = (e < STG * RU && t < T) ? ov : make_uint4(0u, 0u, 0u, 0u);
        }
        qrows.store(sQ, T, k0, tl);
        if (tl < STG) sL[tl] = k0 + tl < T ? lsev : 0.f;
        // D: the RU chunks of a row are RU consecutive lanes of one DPP row
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int e = tl + NTH * it;
            const bool ev = e < STG * RU;
            const int rr = min(e / RU, STG - 1), cc = e - (e / RU) * RU, t = k0 + rr;
            float di = dot8(ld16(sD + rr * ST + cc * 8), orows[it]);
            di += dppf<SLOT_DPP_XOR1>(di);
            di += dppf<SLOT_DPP_XOR2>(di);
            di += dppf<SLOT_DPP_HMIR>(di);
            if constexpr (RU == 16) di += dppf<SLOT_DPP_MIR>(di);
            if (ev && cc == 0) {
                sDs[rr] = di;
                if (rr < TILE && t < T) a.dsum[((size_t)b * Hq + hq) * T + t] = di;
            }
        }
        __syncthreads();
        // ---- S, dP per (query tile kt + 16 u, key tile kt); dk, dv; dS tiles for dq
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int rq = 16 * w + 16 * u;            // the query tile's first staged row
            f32x4 sa = {0.f, 0.f, 0.f, 0.f}, pa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                sa = mfma_k32(ld16(sQ + (rq + c) * ST + 32 * kk + 8 * g), kb[kk], sa);
                pa = mfma_k32(ld16(sD + (rq + c) * ST + 32 * kk + 8 * g), vb[kk], pa);
            }
            float p[4], ds[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {              // query kt + 16 u + 4 g + i, key j
                const int tq = kt + 16 * u + 4 * g + i;
                const bool ok = allowed(tq, j, T, W);
                p[i] = ok ? __expf(sa[i] * a.scale - sL[rq + 4 * g + i]) : 0.f;
                ds[i] = p[i] * (pa[i] - sDs[rq + 4 * g + i]);
            }
            const uint2 pB = make_uint2(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]));
            const uint2 dB = make_uint2(pack_bf16x2(ds[0], ds[1]), pack_bf16x2(ds[2], ds[3]));
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                dvt[dt] = mfma_k16(gather4<ST>(sD, rq + 4 * g, 16 * dt + c), pB, dvt[dt]);
                dkt[dt] = mfma_k16(gather4<ST>(sQ, rq + 4 * g, 16 * dt + c), dB, dkt[dt]);
            }
            put_ds(&sT[w][u][0], ds);
        }
        if (w == 0) {                                  // query tile k0 against key tile k0 - 16 (dq only)
            const int jx = k0 - 16 + c;
            f32x4 sa = {0.f, 0.f, 0.f, 0.f}, pa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                const uint4 kx = ld16(sK + c * ST + 32 * kk + 8 * g);   // staged rows 0..15 = keys k0 - 16..
                sa = mfma_k32(ld16(sQ + c * ST + 32 * kk + 8 * g), kx, sa);
                pa = mfma_k32(ld16(sD + c * ST + 32 * kk + 8 * g), ld16(sVx + c * ST + 32 * kk + 8 * g), pa);
            }
            float ds[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tq = k0 + 4 * g + i;
                const bool ok = allowed(tq, jx, T, W);
                const float p = ok ? __expf(sa[i] * a.scale - sL[4 * g + i]) : 0.f;
                ds[i] = p * (pa[i] - sDs[4 * g + i]);
            }
            put_ds(&sT[NW][1][0], ds);
        }
        __syncthreads();
        if (r + 1 < R) load_head(hq + 1);              // the next head's rows in flight during the dq pass
        // ---- dQ^T (dims x queries of tile kt) = K^T dS^T over key tiles kt - 16 and kt
        const bf16_t* t0p = w > 0 ? &sT[w - 1][1][0] : &sT[NW][1][0];
        const bf16_t* t1p = &sT[w][0][0];
        const uint2 b0 = *reinterpret_cast<const uint2*>(t0p + c * TS + 4 * g);
        const uint2 b1 = *reinterpret_cast<const uint2*>(t1p + c * TS + 4 * g);
        // the rows go out through this wave's slice of sQ: every wave's reads of the head's q rows are done
        emit_rows16<D>(ow, lane, [&](int dt) {
            f32x4 o = {0.f, 0.f, 0.f, 0.f};
            o = mfma_k16(gather4<ST>(sK, 16 * w + 4 * g, 16 * dt + c), b0, o);
            o = mfma_k16(gather4<ST>(sK, 16 * w + 16 + 4 * g, 16 * dt + c), b1, o);
            return f32x4{o[0] * a.scale, o[1] * a.scale, o[2] * a.scale, o[3] * a.scale};
        }, [&](int rr) { return kt + rr < T ? a.dq + ((((size_t)b * T + kt + rr) * Hq + hq) * D) : (bf16_t*)nullptr; });
    }
    auto krowp = [&](bf16_t* base, int rr) { return kt + rr < T ? base + ((((size_t)b * T + kt + rr) * Hk + hk) * D) : (bf16_t*)nullptr; };
    emit_rows16<D>(ow, lane, [&](int dt) {
        return f32x4{dkt[dt][0] * a.scale, dkt[dt][1] * a.scale, dkt[dt][2] * a.scale, dkt[dt][3] * a.scale};
    }, [&](int rr) { return krowp(a.dk, rr); });
    emit_rows16<D>(ow, lane, [&](int dt) { return dvt[dt]; }, [&](int rr) { return krowp(a.dv, rr); });
}

}  // namespace

// ======================================================================================== C-ABI
static int check_win(int64_t B, int64_t T, int64_t Hq, int64_t Hk, int64_t D, int64_t W) {
    if (B < 1 || T < 1 || Hq < 1 || Hk < 1) return fail(SLOTSCAN_ERR_SHAPE, "slotwin: B, T, Hq, Hk must be >= 1");
    if (Hq % Hk) return fail(SLOTSCAN_ERR_SHAPE, "slotwin: Hq must be a multiple of Hk");
    if (D != 64 && D != 128) return fail(SLOTSCAN_ERR_SHAPE, "slotwin: D must be 64 or 128");
    if (W < 1 || W > SLOTWIN_MAX_W) return fail(SLOTSCAN_ERR_SHAPE, "slotwin: W must be in [1, 16]");
    if (B > 65535 || Hq > 65535 || (T + WIN_TILE - 1) / WIN_TILE > 0x7fffffffLL || B * T * Hq * D > 0x7fffffffffffLL)
        return fail(SLOTSCAN_ERR_SHAPE, "slotwin: shape too large");
    return 0;
}

extern "C" int slotwin_fwd(const void* q, const void* k, const void* v, int64_t B, int64_t T, int64_t Hq,
                           int64_t Hk, int64_t D, int64_t W, float scale, void* out, float* lse, void* stream) {
    if (int r = check_win(B, T, Hq, Hk, D, W)) return r;
    if (!q || !k || !v || !out || !lse) return fail(SLOTSCAN_ERR_NULL, "slotwin_fwd: a required pointer is NULL");
    if (!al16(q) || !al16(k) || !al16(v) || !al16(out))                // out is written in 16-byte row pieces
        return fail(SLOTSCAN_ERR_ALIGN, "slotwin_fwd: q, k, v and out must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    WinArgs a{(const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, nullptr, nullptr, nullptr,
              (bf16_t*)out, lse, nullptr, nullptr, nullptr, nullptr, (int)T, (int)Hq, (int)Hk, (int)W, scale};
    const dim3 grid((unsigned)((T + WIN_TILE - 1) / WIN_TILE), (unsigned)Hk, (unsigned)B), block(WIN_THREADS);
    hipError_t e;
    {
        slothost::Scope sc(SLOTSCAN_K_WIN_FWD, st);
        if (D == 128) slothost::launch(win_fwd<128>, grid, block, 0, st, a);
        else slothost::launch(win_fwd<64>, grid, block, 0, st, a);
        e = hipGetLastError();
    }
    return e == hipSuccess ? 0 : hip_fail(e, "win_fwd launch");
}

extern "C" int slotwin_bwd(const void* q, const void* k, const void* v, const void* out, const float* lse,
                           const void* dout, int64_t B, int64_t T, int64_t Hq, int64_t Hk, int64_t D, int64_t W,
                           float scale, float* dsum, void* dq, void* dk, void* dv, void* stream) {
    if (int r = check_win(B, T, Hq, Hk, D, W)) return r;
    if (!q || !k || !v || !out || !lse || !dout || !dsum || !dq || !dk || !dv)
        return fail(SLOTSCAN_ERR_NULL, "slotwin_bwd: a required pointer is NULL");
    if (!al16(q) || !al16(k) || !al16(v) || !al16(out) || !al16(dout) || !al16(dq) || !al16(dk) || !al16(dv))
        return fail(SLOTSCAN_ERR_ALIGN, "slotwin_bwd: q, k, v, out, dout, dq, dk and dv must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    WinArgs a{(const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, (const bf16_t*)out, lse, (const bf16_t*)dout,
              nullptr, nullptr, (bf16_t*)dq, (bf16_t*)dk, (bf16_t*)dv, dsum, (int)T, (int)Hq, (int)Hk, (int)W, scale};
    const unsigned nt = (unsigned)((T + 16 * WIN_BWD_WAVES - 1) / (16 * WIN_BWD_WAVES));
    hipError_t e;
    {
        slothost::Scope sc(SLOTSCAN_K_WIN_BWD, st);
        if (D == 128) slothost::launch(win_bwd<128, WIN_BWD_WAVES>, dim3(nt, (unsigned)Hk, (unsigned)B), dim3(64 * WIN_BWD_WAVES), 0, st, a);
        else slothost::launch(win_bwd<64, WIN_BWD_WAVES>, dim3(nt, (unsigned)Hk, (unsigned)B), dim3(64 * WIN_BWD_WAVES), 0, st, a);
        e = hipGetLastError();
    }
    return e == hipSuccess ? 0 : hip_fail(e, "win_bwd launch");
}
