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
//   forward   S^T (keys x queries) = K Q^T with v_mfma_f32_16x16x32_bf16 (keys as the A rows, queries as
//             the B columns, D/32 k-steps) for the two key tiles; the D layout puts one query column in
//             every lane (4 keys per lane per tile), so the band softmax is 8 values per lane and one
//             cross-row reduction; O^T = V^T P^T with v_mfma_f32_16x16x16_bf16, whose B operand is exactly
//             the score tile's D layout (the exponentials are rounded to bf16 unnormalised and the sum
//             divides at the end).  V^T is gathered from value rows staged in LDS.  The log-sum-exp of
//             every query is kept for the backward.
//   dq        per query tile: S^T and dP^T = V dO^T as above, dS = P (dP - rowsum(dO o O)), dQ^T = K^T dS^T;
//             it also stores rowsum(dO o O) for the key pass.
//   dk, dv    per key tile, queries as the A rows: S and dP (queries x keys) for the two query tiles that
//             see the keys, then dV^T = dO^T P and dK^T = Q^T dS, whose B operands are again the D layout.
//             The query heads of a key/value head are summed in the kernel: no atomics, bitwise
//             reproducible.
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

#define WIN_WAVES 4
#define WIN_THREADS (64 * WIN_WAVES)
#define WIN_TILE (16 * WIN_WAVES)                    // query (or key) rows per workgroup
#define WIN_STAGE (WIN_TILE + 16)                    // staged rows: the tile plus the 16 rows the band reaches

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
__device__ __forceinline__ void st4bf(bf16_t* p, float a0, float a1, float a2, float a3) {
    *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(a0, a1), pack_bf16x2(a2, a3));
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

// stage rows [r0, r0 + WIN_STAGE) of head h of x (B, T, H, D) into s (zeros outside [0, T))
template <int D, int ST>
__device__ __forceinline__ void stage_rows(bf16_t* s, const bf16_t* x, int b, int T, int H, int h, int r0, int tid) {
    constexpr int RU = D / 8;
    for (int e = tid; e < WIN_STAGE * RU; e += WIN_THREADS) {
        const int r = e / RU, cc = e - (e / RU) * RU, t = r0 + r;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (t >= 0 && t < T) v = ld16(x + (((size_t)b * T + t) * H + h) * D + cc * 8);
        *reinterpret_cast<uint4*>(s + r * ST + cc * 8) = v;
    }
}

__device__ __forceinline__ bool allowed(int tq, int j, int T, int W) {
    return tq < T && j >= 0 && j <= tq && tq - j < W;
}

// ------------------------------------------------------------------------------------------- forward
template <int D>
__global__ __launch_bounds__(WIN_THREADS) void win_fwd(WinArgs a) {
    constexpr int KK = D / 32, DT = D / 16, ST = D + 8;
    __shared__ __align__(16) bf16_t sV[WIN_STAGE * ST];
    const int T = a.T, Hq = a.Hq, Hk = a.Hk, W = a.W;
    const int b = blockIdx.z, hq = blockIdx.y, hk = hq / (Hq / Hk);
    const int t0 = blockIdx.x * WIN_TILE;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
    stage_rows<D, ST>(sV, a.v, b, T, Hk, hk, t0 - 16, tid);
    __syncthreads();
    const int qt = t0 + 16 * w;
    if (qt >= T) return;                              // no barrier follows
    const int tq = qt + c;                            // this lane's query column
    const bool qok = tq < T;
    const bf16_t* qrow = a.q + (((size_t)b * T + (qok ? tq : 0)) * Hq + hq) * D;
    uint4 qf[KK];
#pragma unroll
    for (int kk = 0; kk < KK; kk++) qf[kk] = qok ? ld16(qrow + 32 * kk + 8 * g) : make_uint4(0u, 0u, 0u, 0u);
    f32x4 acc[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {                      // key tile u: keys qt - 16 + 16 u + (0..15)
        const int j = qt - 16 + 16 * u + c;
        const bool jok = j >= 0 && j < T;
        const bf16_t* krow = a.k + (((size_t)b * T + (jok ? j : 0)) * Hk + hk) * D;
        acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KK; kk++)
            acc[u] = mfma_k32(jok ? ld16(krow + 32 * kk + 8 * g) : make_uint4(0u, 0u, 0u, 0u), qf[kk], acc[u]);
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
    uint2 pf[2];                                       // bf16 exponentials: the B operand (k = key, col = query)
#pragma unroll
    for (int u = 0; u < 2; u++) pf[u] = make_uint2(pack_bf16x2(s[u][0], s[u][1]), pack_bf16x2(s[u][2], s[u][3]));
    const float inv = l > 0.f ? 1.f / l : 0.f;
    bf16_t* orow = a.out + (((size_t)b * T + (qok ? tq : 0)) * Hq + hq) * D;
#pragma unroll
    for (int dt = 0; dt < DT; dt++) {
        f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 2; u++) o = mfma_k16(gather4<ST>(sV, 16 * w + 16 * u + 4 * g, 16 * dt + c), pf[u], o);
        if (qok) st4bf(orow + 16 * dt + 4 * g, o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv);
    }
    if (qok && g == 0) a.lse_out[((size_t)b * Hq + hq) * T + tq] = mx + __logf(l);
}

// --------------------------------------------------------------------------------------- backward dq
template <int D>
__global__ __launch_bounds__(WIN_THREADS) void win_bwd_q(WinArgs a) {
    constexpr int KK = D / 32, DT = D / 16, ST = D + 8;
    __shared__ __align__(16) bf16_t sK[WIN_STAGE * ST];
    const int T = a.T, Hq = a.Hq, Hk = a.Hk, W = a.W;
    const int b = blockIdx.z, hq = blockIdx.y, hk = hq / (Hq / Hk);
    const int t0 = blockIdx.x * WIN_TILE;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
    stage_rows<D, ST>(sK, a.k, b, T, Hk, hk, t0 - 16, tid);
    __syncthreads();
    const int qt = t0 + 16 * w;
    if (qt >= T) return;
    const int tq = qt + c;
    const bool qok = tq < T;
    const size_t qrow = ((size_t)b * T + (qok ? tq : 0)) * Hq + hq;
    uint4 qf[KK], df[KK];
    float di = 0.f;                                    // rowsum(dO o O) of query tq, over this lane's dims
#pragma unroll
    for (int kk = 0; kk < KK; kk++) {
        const uint4 z = make_uint4(0u, 0u, 0u, 0u);
        qf[kk] = qok ? ld16(a.q + qrow * D + 32 * kk + 8 * g) : z;
        df[kk] = qok ? ld16(a.dO + qrow * D + 32 * kk + 8 * g) : z;
        di += dot8(df[kk], qok ? ld16(a.o + qrow * D + 32 * kk + 8 * g) : z);
    }
    di = sum4rows(di);
    const float lq = qok ? a.lse[((size_t)b * Hq + hq) * T + tq] : 0.f;
    uint2 dsf[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int j = qt - 16 + 16 * u + c;
        const bool jok = j >= 0 && j < T;
        const size_t krow = ((size_t)b * T + (jok ? j : 0)) * Hk + hk;
        f32x4 sa = {0.f, 0.f, 0.f, 0.f}, pa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KK; kk++) {
            const uint4 z = make_uint4(0u, 0u, 0u, 0u);
            sa = mfma_k32(jok ? ld16(a.k + krow * D + 32 * kk + 8 * g) : z, qf[kk], sa);
            pa = mfma_k32(jok ? ld16(a.v + krow * D + 32 * kk + 8 * g) : z, df[kk], pa);
        }
        float ds[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int jj = qt - 16 + 16 * u + 4 * g + i;
            const float p = allowed(tq, jj, T, W) ? __expf(sa[i] * a.scale - lq) : 0.f;
            ds[i] = p * (pa[i] - di);
        }
        dsf[u] = make_uint2(pack_bf16x2(ds[0], ds[1]), pack_bf16x2(ds[2], ds[3]));
    }
#pragma unroll
    for (int dt = 0; dt < DT; dt++) {
        f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 2; u++) o = mfma_k16(gather4<ST>(sK, 16 * w + 16 * u + 4 * g, 16 * dt + c), dsf[u], o);
        if (qok) st4bf(a.dq + qrow * D + 16 * dt + 4 * g, o[0] * a.scale, o[1] * a.scale, o[2] * a.scale, o[3] * a.scale);
    }
    if (qok && g == 0) a.dsum[((size_t)b * Hq + hq) * T + tq] = di;
}

// ----------------------------------------------------------------------------------- backward dk, dv
template <int D>
__global__ __launch_bounds__(WIN_THREADS) void win_bwd_kv(WinArgs a) {
    constexpr int KK = D / 32, DT = D / 16, ST = D + 8;
    __shared__ __align__(16) bf16_t sQ[WIN_STAGE * ST];
    __shared__ __align__(16) bf16_t sD[WIN_STAGE * ST];
    const int T = a.T, Hq = a.Hq, Hk = a.Hk, W = a.W, R = Hq / Hk;
    const int b = blockIdx.z, hk = blockIdx.y;
    const int k0 = blockIdx.x * WIN_TILE;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
    const int kt = k0 + 16 * w;                        // this wave's key tile; lane column = key kt + c
    const int j = kt + c;
    const bool jok = j < T;
    const size_t krow = ((size_t)b * T + (jok ? j : 0)) * Hk + hk;
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
    for (int r = 0; r < R; r++) {
        const int hq = hk * R + r;
        __syncthreads();                               // the previous head's staged rows are consumed
        stage_rows<D, ST>(sQ, a.q, b, T, Hq, hq, k0, tid);
        stage_rows<D, ST>(sD, a.dO, b, T, Hq, hq, k0, tid);
        __syncthreads();
        if (kt >= T) continue;
        const float* lse = a.lse + ((size_t)b * Hq + hq) * T;
        const float* dsm = a.dsum + ((size_t)b * Hq + hq) * T;
#pragma unroll
        for (int u = 0; u < 2; u++) {                  // query tile u: queries kt + 16 u + (0..15), A rows
            const int rq = 16 * w + 16 * u;            // its first staged row
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
                const float lq = ok ? lse[tq] : 0.f, dq = ok ? dsm[tq] : 0.f;
                p[i] = ok ? __expf(sa[i] * a.scale - lq) : 0.f;
                ds[i] = p[i] * (pa[i] - dq);
            }
            const uint2 pB = make_uint2(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]));
            const uint2 dB = make_uint2(pack_bf16x2(ds[0], ds[1]), pack_bf16x2(ds[2], ds[3]));
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                dvt[dt] = mfma_k16(gather4<ST>(sD, rq + 4 * g, 16 * dt + c), pB, dvt[dt]);
                dkt[dt] = mfma_k16(gather4<ST>(sQ, rq + 4 * g, 16 * dt + c), dB, dkt[dt]);
            }
        }
    }
    if (!jok || kt >= T) return;
#pragma unroll
    for (int dt = 0; dt < DT; dt++) {
        st4bf(a.dk + krow * D + 16 * dt + 4 * g, dkt[dt][0] * a.scale, dkt[dt][1] * a.scale, dkt[dt][2] * a.scale,
              dkt[dt][3] * a.scale);
        st4bf(a.dv + krow * D + 16 * dt + 4 * g, dvt[dt][0], dvt[dt][1], dvt[dt][2], dvt[dt][3]);
    }
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
    if (!al16(q) || !al16(k) || !al16(v) || ((uintptr_t)out & 7u))
        return fail(SLOTSCAN_ERR_ALIGN, "slotwin_fwd: q, k, v must be 16-byte aligned, out 8-byte");
    hipStream_t st = (hipStream_t)stream;
    WinArgs a{(const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, nullptr, nullptr, nullptr,
              (bf16_t*)out, lse, nullptr, nullptr, nullptr, nullptr, (int)T, (int)Hq, (int)Hk, (int)W, scale};
    const dim3 grid((unsigned)((T + WIN_TILE - 1) / WIN_TILE), (unsigned)Hq, (unsigned)B), block(WIN_THREADS);
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
    if (!al16(q) || !al16(k) || !al16(v) || !al16(out) || !al16(dout) || ((uintptr_t)dq & 7u) ||
        ((uintptr_t)dk & 7u) || ((uintptr_t)dv & 7u))
        return fail(SLOTSCAN_ERR_ALIGN, "slotwin_bwd: q, k, v, out, dout must be 16-byte aligned, dq, dk, dv 8-byte");
    hipStream_t st = (hipStream_t)stream;
    WinArgs a{(const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, (const bf16_t*)out, lse, (const bf16_t*)dout,
              nullptr, nullptr, (bf16_t*)dq, (bf16_t*)dk, (bf16_t*)dv, dsum, (int)T, (int)Hq, (int)Hk, (int)W, scale};
    const unsigned nt = (unsigned)((T + WIN_TILE - 1) / WIN_TILE);
    hipError_t e;
    {
        slothost::Scope sc(SLOTSCAN_K_WIN_BWD, st);
        if (D == 128) slothost::launch(win_bwd_q<128>, dim3(nt, (unsigned)Hq, (unsigned)B), dim3(WIN_THREADS), 0, st, a);
        else slothost::launch(win_bwd_q<64>, dim3(nt, (unsigned)Hq, (unsigned)B), dim3(WIN_THREADS), 0, st, a);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return hip_fail(e, "win_bwd_q launch");
    {
        slothost::Scope sc(SLOTSCAN_K_WIN_BWD, st);
        if (D == 128) slothost::launch(win_bwd_kv<128>, dim3(nt, (unsigned)Hk, (unsigned)B), dim3(WIN_THREADS), 0, st, a);
        else slothost::launch(win_bwd_kv<64>, dim3(nt, (unsigned)Hk, (unsigned)B), dim3(WIN_THREADS), 0, st, a);
        e = hipGetLastError();
    }
    return e == hipSuccess ? 0 : hip_fail(e, "win_bwd_kv launch");
}
