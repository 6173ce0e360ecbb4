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
// gfx950 mapping.  A chain workgroup is 256 lanes = 4 waves = 16 row groups of 16 lanes (one DPP row per
// slot row); row n lives in row group n % 16 as register slice i = n / 16.  Row dot products reduce with 4
// DPP stages, the argmax reduces the 4 row groups of a wave with readlane and the 4 waves through one
// ping-pong LDS slot, so a step costs ONE workgroup barrier.  Token inputs (q, k, gate, fr, and in the
// backward the undo log and Dn) are staged in LDS 16 steps ahead in double-buffered chunks.  Row norms are
// kept per row and recomputed only for the written row.
#include "slot_common.h"

using namespace slot;
typedef uint64_t u64;
typedef uint32_t u32;

#define SLOT_CT 16          // tokens per staged chunk in the chain kernels
#define SLOT_BIGI 0x7fffffff

#define CHAIN_ATTR __global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(2)))
#define ROWS_ATTR __global__ __attribute__((amdgpu_flat_work_group_size(512, 512)))

namespace {

constexpr int CT = SLOT_CT;

__device__ __forceinline__ u64 umax64(u64 a, u64 b) { return a > b ? a : b; }
__device__ __forceinline__ float readlanef(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ u32 readlaneu(u32 v, int l) { return (u32)__builtin_amdgcn_readlane((int)v, l); }
__device__ __forceinline__ u64 readlane64(u64 v, int l) {
    return ((u64)readlaneu((u32)(v >> 32), l) << 32) | readlaneu((u32)v, l);
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
template <int EPL>
__device__ __forceinline__ void st_slice_nt(float* row, const float* s, int c) {
#pragma unroll
    for (int jj = 0; jj < EPL / 4; jj++)
        st4_nt(row + 4 * c + 64 * jj, make_float4(s[4 * jj], s[4 * jj + 1], s[4 * jj + 2], s[4 * jj + 3]));
}
template <int EPL>
__device__ __forceinline__ float norm_inv(const float* x) {
    float kk = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; e++) kk = fmaf(x[e], x[e], kk);
    kk = rowsum16(kk);
    return 1.f / fmaxf(sqrtf(kk), 1e-6f);
}

// online-softmax merge of (max, sum e^(z-max), sum e^(z-max) w)
__device__ __forceinline__ void smerge(float& M, float& S, float& SD, float m2, float s2, float sd2) {
    if (m2 == -INFINITY) return;
    if (M == -INFINITY) { M = m2; S = s2; SD = sd2; return; }
    const float m = fmaxf(M, m2);
    const float a1 = expf(M - m), a2 = expf(m2 - m);
    S = S * a1 + s2 * a2;
    SD = SD * a1 + sd2 * a2;
    M = m;
}

// =========================================================================================== chain_fwd
struct ChainFwdArgs {
    const void* q; const void* k; const float* gate; const float* fr; const float* temp;
    const float* k0; const float* o0;
    float* kbuf; int32_t* am; float* kold; float* oold; float* kfin; float* ofin;
    int T, H, N, G, NB; float eps; int frt, occb;
};

template <int D, int RPT, typename TI>
CHAIN_ATTR void chain_fwd(ChainFwdArgs a) {
    constexpr int CT = (sizeof(TI) == 4 && RPT >= 12) ? 8 : SLOT_CT;   // fewer staging registers at N > 128
    constexpr int EPL = D / 16;
    constexpr int RU = D * (int)sizeof(TI) / 16;      // uint4 per token row
    constexpr int NU = CT * 2 * RU;                    // uint4 per staged chunk: (q row, k row) per token
    constexpr int UPT = (NU + 255) / 256;
    __shared__ __align__(16) TI s_tok[2][CT][2][D];
    __shared__ float s_g[2][CT], s_fr[2][CT];
    __shared__ uint4 s_red[2][4];

    const int T = a.T, H = a.H, N = a.N, G = a.G;
    const int bh = blockIdx.x, b = bh / H, h = bh - b * H;
    const int tid = threadIdx.x, rg = tid >> 4, c = tid & 15, wave = tid >> 6, lane = tid & 63;
    const TI* __restrict__ qp = (const TI*)a.q;
    const TI* __restrict__ kp = (const TI*)a.k;
    const size_t tok0 = (size_t)b * T * H + h;         // token (b, t, h) = tok0 + t * H

    float K[RPT][EPL], o[RPT], kinv[RPT];
#pragma unroll
    for (int i = 0; i < RPT; i++) {
        const int n = rg + 16 * i;
        o[i] = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) K[i][e] = 0.f;
        if (n < N) {
            if (a.k0) ld_slice<EPL>(K[i], a.k0 + ((size_t)bh * N + n) * D, c);
            if (a.o0) o[i] = a.o0[(size_t)bh * N + n];
        }
        kinv[i] = norm_inv<EPL>(K[i]);
    }

    uint4 rq[UPT];
    float rs = 0.f;
    auto load_chunk = [&](int ch) {
#pragma unroll
        for (int m = 0; m < UPT; m++) {
            const int u = tid + 256 * m;
            rq[m] = make_uint4(0u, 0u, 0u, 0u);
            if (u < NU) {
                const int j = u / (2 * RU), arr = (u / RU) & 1, w = u % RU;
                const int t = ch * CT + j;
                if (t < T) rq[m] = reinterpret_cast<const uint4*>((arr ? kp : qp) + (tok0 + (size_t)t * H) * D)[w];
            }
        }
        if (tid < 2 * CT) {
            const int t = ch * CT + (tid & (CT - 1));
            rs = 0.f;
            if (t < T) rs = (tid < CT) ? a.gate[tok0 + (size_t)t * H] : (a.frt ? a.fr[tok0 + (size_t)t * H] : 0.f);
        }
    };
    auto store_chunk = [&](int buf) {
        uint4* dst = reinterpret_cast<uint4*>(&s_tok[buf][0][0][0]);
#pragma unroll
        for (int m = 0; m < UPT; m++) {
            const int u = tid + 256 * m;
            if (u < NU) dst[u] = rq[m];
        }
        if (tid < CT) s_g[buf][tid] = rs;
        else if (tid < 2 * CT) s_fr[buf][tid - CT] = rs;
    };

    const float temp = a.temp[0];
    const float fr_s = a.frt ? 0.f : a.fr[0];
    const float eps = a.eps;
    const bool occb = a.occb != 0, frt = a.frt != 0;

    load_chunk(0);
    store_chunk(0);
    __syncthreads();
    load_chunk(1);
    int par = 0, j = 0, buf = 0;
    for (int t = 0; t < T; t++) {
        if (t % G == 0) {                                   // the PRE-write key state of block t / G
            float* kb = a.kbuf + ((size_t)(b * a.NB + t / G) * H + h) * N * D;
#pragma unroll
            for (int i = 0; i < RPT; i++) {
                const int n = rg + 16 * i;
                if (n < N) st_slice_nt<EPL>(kb + (size_t)n * D, K[i], c);
            }
        }
        float qv[EPL];
        ld_slice<EPL>(qv, &s_tok[buf][j][0][0], c);
        float qq = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) qq = fmaf(qv[e], qv[e], qq);
        qq = rowsum16(qq);
        const float qinv = 1.f / fmaxf(sqrtf(qq), 1e-6f);
        const float g = s_g[buf][j];
        const float frv = frt ? s_fr[buf][j] : fr_s;

        // per-row score and this thread's candidates: best occupied (z, -n) and lowest free n (with its z)
        u64 bo = 0, bfr = 0;
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            const int n = rg + 16 * i;
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < EPL; e++) d = fmaf(K[i][e], qv[e], d);
            d = rowsum16(d);
            const float s = temp * ((d * kinv[i]) * qinv);
            const bool taken = o[i] >= eps;
            const float occ = occb ? (taken ? 1.f : 0.f) : o[i];
            const float z = s - frv * occ;
            if (n < N) {
                if (taken) bo = umax64(bo, ((u64)fkey(z) << 32) | (u32)(~n));
                else bfr = umax64(bfr, ((u64)(u32)(~n) << 32) | fkey(z));
            }
        }
        {   // the 4 row groups of this wave sit at lanes 0, 16, 32, 48
            u64 wo = 0, wf = 0;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                wo = umax64(wo, readlane64(bo, 16 * r));
                wf = umax64(wf, readlane64(bfr, 16 * r));
            }
            if (lane == 0) s_red[par][wave] = make_uint4((u32)(wo >> 32), (u32)wo, (u32)(wf >> 32), (u32)wf);
        }
        if (j == CT - 1) {                                  // refill: chunk t/CT+1 -> LDS, fetch t/CT+2
            store_chunk(buf ^ 1);
            load_chunk(t / CT + 2);
        }
        __syncthreads();
        u64 BO = 0, BF = 0;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint4 x = s_red[par][w];
            BO = umax64(BO, ((u64)x.x << 32) | x.y);
            BF = umax64(BF, ((u64)x.z << 32) | x.w);
        }
        par ^= 1;
        // the lowest free row competes as (its z, -its index)
        const u64 fc = BF ? (((u64)(u32)BF << 32) | (BF >> 32)) : 0;
        const int amv = (int)(~(u32)umax64(BO, fc));
        const size_t ix = tok0 + (size_t)t * H;
        if (tid == 0) a.am[ix] = amv;
        const float omw = 1.f - g;
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            const int n = rg + 16 * i;
            if (n == amv) {
                if (a.kold) {
                    st_slice<EPL>(a.kold + ix * D, K[i], c);
                    if (c == 0) a.oold[ix] = o[i];
                }
                float kv[EPL];
                ld_slice<EPL>(kv, &s_tok[buf][j][1][0], c);
#pragma unroll
                for (int e = 0; e < EPL; e++) K[i][e] = omw * K[i][e] + g * kv[e];
                o[i] = omw * o[i] + g;
                kinv[i] = norm_inv<EPL>(K[i]);
            }
        }
        if (++j == CT) { j = 0; buf ^= 1; }
    }
#pragma unroll
    for (int i = 0; i < RPT; i++) {
        const int n = rg + 16 * i;
        if (n < N) {
            st_slice<EPL>(a.kfin + ((size_t)bh * N + n) * D, K[i], c);
            if (c == 0) a.ofin[(size_t)bh * N + n] = o[i];
        }
    }
}

// =========================================================================================== rows_fwd
struct RowsFwdArgs {
    const void* v; const float* gate; const int32_t* am; const float* v0;
    float* vbuf; float* vold; float* vfin;
    int T, H, N, G, NB;
};

// 512 lanes = 32 rows of one chain per workgroup; grid (B*H, ceil(N/32)).
template <int D, typename TI>
ROWS_ATTR void rows_fwd(RowsFwdArgs a) {
    constexpr int EPL = D / 16;
    constexpr int TC = 2048;
    __shared__ int s_am[TC];
    __shared__ float s_g[TC];
    const int T = a.T, H = a.H, N = a.N, G = a.G;
    const int bh = blockIdx.x, b = bh / H, h = bh - b * H;
    const int tid = threadIdx.x, rg = tid >> 4, c = tid & 15;
    const int n = blockIdx.y * 32 + rg;
    const bool live = n < N;
    const TI* __restrict__ vp = (const TI*)a.v;
    const size_t tok0 = (size_t)b * T * H + h;
    float V[EPL];
#pragma unroll
    for (int e = 0; e < EPL; e++) V[e] = 0.f;
    if (live && a.v0) ld_slice<EPL>(V, a.v0 + ((size_t)bh * N + n) * D, c);
    float* vb0 = a.vbuf + ((size_t)b * a.NB * H + h) * N * D + (size_t)n * D;
    const size_t vbstride = (size_t)H * N * D;
    for (int t0 = 0; t0 < T; t0 += TC) {
        const int tn = min(TC, T - t0);
        __syncthreads();
        for (int u = tid; u < tn; u += 512) {
            const size_t ix = tok0 + (size_t)(t0 + u) * H;
            s_am[u] = a.am[ix];
            s_g[u] = a.gate[ix];
        }
        __syncthreads();
        if (!live) continue;
        for (int jt = 0; jt < tn; jt++) {
            const int t = t0 + jt;
            if (t % G == 0) st_slice_nt<EPL>(vb0 + (size_t)(t / G) * vbstride, V, c);
            if (s_am[jt] == n) {
                const size_t ix = tok0 + (size_t)t * H;
                const float g = s_g[jt], omw = 1.f - g;
                float vv[EPL];
                ld_slice<EPL>(vv, vp + ix * D, c);
                if (a.vold) st_slice<EPL>(a.vold + ix * D, V, c);
#pragma unroll
                for (int e = 0; e < EPL; e++) V[e] = omw * V[e] + g * vv[e];
            }
        }
    }
    if (live) st_slice<EPL>(a.vfin + ((size_t)bh * N + n) * D, V, c);
}

// =========================================================================================== rows_bwd
struct RowsBwdArgs {
    const void* k; const void* v; const float* gate; const int32_t* am;
    const float* kold; const float* vold; const float* kfin; const float* vfin;
    const float* dkbuf; const float* dvbuf;
    void* dk; void* dv; float* dn;
    int T, H, N, G, NB;
};

// 512 lanes = 32 rows per workgroup, grid (B*H, ceil(N/32)); reverse in t.  The chain's k_t, v_t are
// staged through LDS in chunks of CT tokens, double buffered one chunk ahead.  Dn is written (B*H, N, T):
// lane c of a row group keeps Dn for t with t % 16 == c and the group stores 16 consecutive t at once.
template <int D, typename TI>
ROWS_ATTR void rows_bwd(RowsBwdArgs a) {
    constexpr int EPL = D / 16;
    constexpr int RU = D * (int)sizeof(TI) / 16;
    constexpr int NU = CT * 2 * RU;
    constexpr int UPT = (NU + 511) / 512;
    __shared__ __align__(16) TI s_tok[2][CT][2][D];
    __shared__ int s_am[2][CT];
    __shared__ float s_g[2][CT];

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

    uint4 rq[UPT];
    int ram = 0;
    float rgt = 0.f;
    auto load_chunk = [&](int ch) {
#pragma unroll
        for (int m = 0; m < UPT; m++) {
            const int u = tid + 512 * m;
            rq[m] = make_uint4(0u, 0u, 0u, 0u);
            if (u < NU) {
                const int j = u / (2 * RU), arr = (u / RU) & 1, w = u % RU;
                const int t = T - 1 - (ch * CT + j);
                if (t >= 0) rq[m] = reinterpret_cast<const uint4*>((arr ? vp : kp) + (tok0 + (size_t)t * H) * D)[w];
            }
        }
        if (tid < CT) {
            const int t = T - 1 - (ch * CT + tid);
            ram = -1; rgt = 0.f;
            if (t >= 0) { ram = a.am[tok0 + (size_t)t * H]; rgt = a.gate[tok0 + (size_t)t * H]; }
        }
    };
    auto store_chunk = [&](int buf) {
        uint4* dst = reinterpret_cast<uint4*>(&s_tok[buf][0][0][0]);
#pragma unroll
        for (int m = 0; m < UPT; m++) {
            const int u = tid + 512 * m;
            if (u < NU) dst[u] = rq[m];
        }
        if (tid < CT) { s_am[buf][tid] = ram; s_g[buf][tid] = rgt; }
    };

    float K[EPL], V[EPL], dK[EPL], dV[EPL], pk[EPL], pv[EPL];
    ld_slice<EPL>(K, a.kfin + ((size_t)bh * N + n) * D, c);
    ld_slice<EPL>(V, a.vfin + ((size_t)bh * N + n) * D, c);
#pragma unroll
    for (int e = 0; e < EPL; e++) { dK[e] = 0.f; dV[e] = 0.f; }
    const size_t sbstride = (size_t)H * N * D;
    const float* dkb0 = a.dkbuf + ((size_t)b * a.NB * H + h) * N * D + (size_t)n * D;
    const float* dvb0 = a.dvbuf + ((size_t)b * a.NB * H + h) * N * D + (size_t)n * D;
    {   // prefetch the gradient of the last emitted block
        const int blk = (T - 1) / G;
        ld_slice<EPL>(pk, dkb0 + (size_t)blk * sbstride, c);
        ld_slice<EPL>(pv, dvb0 + (size_t)blk * sbstride, c);
    }
    float dnk = 0.f;
    load_chunk(0);
    store_chunk(0);
    __syncthreads();
    load_chunk(1);
    int j = 0, buf = 0;
    for (int s = 0; s < T; s++) {
        const int t = T - 1 - s;
        float kt[EPL], vt[EPL];
        ld_slice<EPL>(kt, &s_tok[buf][j][0][0], c);
        ld_slice<EPL>(vt, &s_tok[buf][j][1][0], c);
        const bool hit = live && (s_am[buf][j] == n);
        const float g = s_g[buf][j];
        const size_t ix = tok0 + (size_t)t * H;
        if (hit) {                                          // undo: the row before this step's write
            ld_slice<EPL>(K, a.kold + ix * D, c);
            ld_slice<EPL>(V, a.vold + ix * D, c);
        }
        float p = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) p = fmaf(kt[e] - K[e], dK[e], p);
#pragma unroll
        for (int e = 0; e < EPL; e++) p = fmaf(vt[e] - V[e], dV[e], p);
        p = rowsum16(p);
        if ((t & 15) == c) dnk = p;
        if ((t & 15) == 0 && live) {
            const int tt = t + c;
            if (tt < T) a.dn[((size_t)bh * N + n) * T + tt] = dnk;
        }
        if (hit) {
            const float omw = 1.f - g;
            float x[EPL], y[EPL];
#pragma unroll
            for (int e = 0; e < EPL; e++) { x[e] = g * dK[e]; y[e] = g * dV[e]; dK[e] *= omw; dV[e] *= omw; }
            st_slice<EPL>(dkp + ix * D, x, c);
            st_slice<EPL>(dvp + ix * D, y, c);
        }
        if (t % G == 0) {                                   // the copy emitted at t is the pre-write state
#pragma unroll
            for (int e = 0; e < EPL; e++) { dK[e] += pk[e]; dV[e] += pv[e]; }
            const int blk = t / G - 1;
            if (blk >= 0) {
                ld_slice<EPL>(pk, dkb0 + (size_t)blk * sbstride, c);
                ld_slice<EPL>(pv, dvb0 + (size_t)blk * sbstride, c);
            }
        }
        if (j == CT - 1) {
            store_chunk(buf ^ 1);
            load_chunk(s / CT + 2);
        }
        __syncthreads();
        if (++j == CT) { j = 0; buf ^= 1; }
    }
}

// =========================================================================================== chain_bwd
struct ChainBwdArgs {
    const void* q; const float* gate; const float* fr; const float* temp;
    const int32_t* am; const float* kold; const float* oold; const float* kfin; const float* ofin;
    const float* dn;                                     // (B*H, N, T)
    void* dq; float* dg; float* dfr; float* part;        // part (B*H, 2): dtemp and scalar-dfr partials
    int T, H, N; float eps; int frt, occb;
};

// OCCB (occ_bin) is a template flag here: with it the occupancy enters only through [o >= eps], so the
// kernel keeps one taken-bit per row instead of o and the (identically zero) occupancy adjoint dO.
template <int D, int RPT, typename TI, bool OCCB>
CHAIN_ATTR void chain_bwd(ChainBwdArgs a) {
    constexpr int CT = RPT >= 12 ? 8 : SLOT_CT;                         // fewer staging registers at N > 128
    constexpr int EPL = D / 16;
    constexpr int RUQ = D * (int)sizeof(TI) / 16, RUK = D / 4;
    constexpr int NUQ = CT * RUQ, NU = NUQ + CT * RUK;
    constexpr int UPT = (NU + 255) / 256;
    constexpr int NMAX = 16 * RPT;
    constexpr int DPT = (CT * NMAX + 255) / 256;
    constexpr int EPW = D / 64;                          // q elements per lane in the dq finaliser
    __shared__ __align__(16) TI s_q[2][CT][D];
    __shared__ __align__(16) float s_ko[2][CT][D];
    __shared__ float s_dn[2][CT][NMAX];
    __shared__ float s_g[2][CT], s_fr[2][CT], s_oo[2][CT];
    __shared__ int s_am[2][CT];
    __shared__ float s_st[2][4][8];
    __shared__ float s_pq[2][4][D];
    __shared__ float s_pfr[2][4];
    __shared__ float s_qn[2][2];
    __shared__ float s_fin[2][4];

    const int T = a.T, H = a.H, N = a.N;
    const int bh = blockIdx.x, b = bh / H, h = bh - b * H;
    const int tid = threadIdx.x, rg = tid >> 4, c = tid & 15, wave = tid >> 6, lane = tid & 63;
    const TI* __restrict__ qp = (const TI*)a.q;
    const size_t tok0 = (size_t)b * T * H + h;
    const float temp = a.temp[0];
    const float fr_s = a.frt ? 0.f : a.fr[0];
    const float eps = a.eps;
    const bool frt = a.frt != 0;

    float K[RPT][EPL], o[RPT], kinv[RPT], dO[RPT];
    u32 tk = 0;                                          // OCCB: bit i = row slice i is taken (o >= eps)
#pragma unroll
    for (int i = 0; i < RPT; i++) {
        const int n = rg + 16 * i;
        o[i] = 0.f; dO[i] = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) K[i][e] = 0.f;
        if (n < N) {
            ld_slice<EPL>(K[i], a.kfin + ((size_t)bh * N + n) * D, c);
            o[i] = a.ofin[(size_t)bh * N + n];
            if (o[i] >= eps) tk |= 1u << i;
        }
        kinv[i] = norm_inv<EPL>(K[i]);
    }
    auto taken_of = [&](int i) -> bool { if constexpr (OCCB) return (tk >> i) & 1u; else return o[i] >= eps; };

    uint4 rq[UPT];
    float rdn[DPT];
    float rs = 0.f;
    auto load_chunk = [&](int ch) {
#pragma unroll
        for (int m = 0; m < UPT; m++) {
            const int u = tid + 256 * m;
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
            const int u = tid + 256 * m;
            rdn[m] = 0.f;
            if (u < CT * N) {
                const int nn = u / CT, jj = u % CT, t = T - 1 - (ch * CT + jj);
                if (t >= 0) rdn[m] = a.dn[((size_t)bh * N + nn) * T + t];
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
        uint4* dq_ = reinterpret_cast<uint4*>(&s_q[buf][0][0]);
        uint4* dk_ = reinterpret_cast<uint4*>(&s_ko[buf][0][0]);
#pragma unroll
        for (int m = 0; m < UPT; m++) {
            const int u = tid + 256 * m;
            if (u < NUQ) dq_[u] = rq[m];
            else if (u < NU) dk_[u - NUQ] = rq[m];
        }
#pragma unroll
        for (int m = 0; m < DPT; m++) {
            const int u = tid + 256 * m;
            if (u < CT * N) s_dn[buf][u % CT][u / CT] = rdn[m];
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
        const float qn = s_qn[pp][0], qi = s_qn[pp][1];
        float dqn[EPW], qh[EPW];
        float pr = 0.f;
#pragma unroll
        for (int m = 0; m < EPW; m++) {
            const int e = lane + 64 * m;
            dqn[m] = temp * ((s_pq[pp][0][e] + s_pq[pp][1][e]) + (s_pq[pp][2][e] + s_pq[pp][3][e]));
            qh[m] = ld1<TI>(&s_q[bp][jp][e]) * qi;
            pr = fmaf(dqn[m], qh[m], pr);
        }
        pr = wavesum(pr);
        TI* dqp = (TI*)a.dq + (tok0 + (size_t)tp * H) * D;
#pragma unroll
        for (int m = 0; m < EPW; m++) {
            const float r = qn < 1e-6f ? qi * dqn[m] : qi * (dqn[m] - qh[m] * pr);
            st1<TI>(dqp + lane + 64 * m, r);
        }
        if (frt && lane == 0)
            a.dfr[tok0 + (size_t)tp * H] = (s_pfr[pp][0] + s_pfr[pp][1]) + (s_pfr[pp][2] + s_pfr[pp][3]);
    };

    float dtemp_acc = 0.f, dfr_acc = 0.f;
    load_chunk(0);
    store_chunk(0);
    __syncthreads();
    load_chunk(1);
    int par = 0, j = 0, buf = 0;
    for (int s = 0; s < T; s++) {
        const int t = T - 1 - s;
        const int amv = s_am[buf][j];
        const float g = s_g[buf][j];
        const float frv = frt ? s_fr[buf][j] : fr_s;
        // undo this step's write: the written row goes back to its logged pre-write key and occupancy
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            const int n = rg + 16 * i;
            if (n == amv) {
                ld_slice<EPL>(K[i], &s_ko[buf][j][0], c);
                const float oo = s_oo[buf][j];
                if constexpr (OCCB) tk = (tk & ~(1u << i)) | ((oo >= eps ? 1u : 0u) << i);
                else o[i] = oo;
                kinv[i] = norm_inv<EPL>(K[i]);
            }
        }
        float qv[EPL];
        ld_slice<EPL>(qv, &s_q[buf][j][0], c);
        float qq = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) qq = fmaf(qv[e], qv[e], qq);
        qq = rowsum16(qq);
        const float qnorm = sqrtf(qq), qinv = 1.f / fmaxf(qnorm, 1e-6f);

        float cs[RPT], dw[RPT], ex[RPT];
        float mloc = -INFINITY;
        int ei = SLOT_BIGI;
        float ez = 0.f, ed = 0.f;
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            const int n = rg + 16 * i;
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < EPL; e++) d = fmaf(K[i][e], qv[e], d);
            d = rowsum16(d);
            cs[i] = (d * kinv[i]) * qinv;
            const bool taken = taken_of(i);
            float z;
            if constexpr (OCCB) {
                z = temp * cs[i] - (taken ? frv : 0.f);
                dw[i] = n < N ? s_dn[buf][j][n] : 0.f;
            } else {
                z = temp * cs[i] - frv * o[i];
                dw[i] = (n < N ? s_dn[buf][j][n] : 0.f) + (1.f - o[i]) * dO[i];
            }
            ex[i] = z;
            if (n < N && taken) mloc = fmaxf(mloc, z);
            if (n < N && !taken && n < ei) { ei = n; ez = z; ed = dw[i]; }
        }
        float S = 0.f, SD = 0.f;
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            const int n = rg + 16 * i;
            const bool taken = n < N && taken_of(i);
            ex[i] = taken ? expf(ex[i] - mloc) : 0.f;
            S += ex[i];
            SD = fmaf(ex[i], dw[i], SD);
        }
        {
            float M = -INFINITY, SS = 0.f, SSD = 0.f, EZ = 0.f, ED = 0.f;
            int EI = SLOT_BIGI;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                smerge(M, SS, SSD, readlanef(mloc, 16 * r), readlanef(S, 16 * r), readlanef(SD, 16 * r));
                const int e2 = __builtin_amdgcn_readlane(ei, 16 * r);
                if (e2 < EI) { EI = e2; EZ = readlanef(ez, 16 * r); ED = readlanef(ed, 16 * r); }
            }
            if (lane == 0) {
                s_st[par][wave][0] = M; s_st[par][wave][1] = SS; s_st[par][wave][2] = SSD;
                s_st[par][wave][3] = __int_as_float(EI); s_st[par][wave][4] = EZ; s_st[par][wave][5] = ED;
            }
        }
        if (j == CT - 1) {
            store_chunk(buf ^ 1);
            load_chunk(s / CT + 2);
        }
        __syncthreads();
        if (s > 0 && wave == ((s - 1) & 3)) finalize(s - 1);
        float M = -INFINITY, SS = 0.f, SSD = 0.f, EZ = 0.f, ED = 0.f;
        int EI = SLOT_BIGI;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            smerge(M, SS, SSD, s_st[par][w][0], s_st[par][w][1], s_st[par][w][2]);
            const int e2 = __float_as_int(s_st[par][w][3]);
            if (e2 < EI) { EI = e2; EZ = s_st[par][w][4]; ED = s_st[par][w][5]; }
        }
        if (EI != SLOT_BIGI) smerge(M, SS, SSD, EZ, 1.f, ED);   // the first free row competes too
        const float sa = g * SSD / SS;                          // sum_n asoft_n * g * dw_n
        const float sloc = mloc == -INFINITY ? 0.f : expf(mloc - M) / SS;
        const float afree = EI != SLOT_BIGI ? expf(EZ - M) / SS : 0.f;   // soft address of the first free row
        float pq[EPL];
#pragma unroll
        for (int e = 0; e < EPL; e++) pq[e] = 0.f;
        float frp = 0.f;
        const float omw = 1.f - g;
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            const int n = rg + 16 * i;
            const bool taken = n < N && taken_of(i);
            const bool first_free = n == EI;
            const float as = taken ? ex[i] * sloc : (first_free ? afree : 0.f);
            const float dz = (taken || first_free) ? as * (g * dw[i] - sa) : 0.f;
            if (n == amv && c == 0) a.dg[tok0 + (size_t)t * H] = dw[i];
            dtemp_acc = fmaf(dz, cs[i], dtemp_acc);
            if constexpr (OCCB) frp -= taken ? dz : 0.f;
            else frp = fmaf(-o[i], dz, frp);
            const float cf = dz * kinv[i];
#pragma unroll
            for (int e = 0; e < EPL; e++) pq[e] = fmaf(cf, K[i][e], pq[e]);
            if constexpr (!OCCB) dO[i] = (n == amv ? omw : 1.f) * dO[i] - frv * dz;
        }
#pragma unroll
        for (int e = 0; e < EPL; e++) pq[e] = sum4rows(pq[e]);
        frp = sum4rows(frp);
        if (lane < 16) {
#pragma unroll
            for (int jj = 0; jj < EPL / 4; jj++)
#pragma unroll
                for (int r = 0; r < 4; r++) s_pq[par][wave][4 * c + 64 * jj + r] = pq[4 * jj + r];
        }
        if (lane == 0) { s_pfr[par][wave] = frp; dfr_acc += frp; }
        if (tid == 0) { s_qn[par][0] = qnorm; s_qn[par][1] = qinv; }
        par ^= 1;
        if (++j == CT) { j = 0; buf ^= 1; }
    }
    __syncthreads();
    if (wave == ((T - 1) & 3)) finalize(T - 1);
    dtemp_acc = sum4rows(dtemp_acc);
    if (lane == 0) { s_fin[0][wave] = dtemp_acc; s_fin[1][wave] = dfr_acc; }
    __syncthreads();
    if (tid == 0) {
        a.part[2 * (size_t)bh + 0] = (s_fin[0][0] + s_fin[0][1]) + (s_fin[0][2] + s_fin[0][3]);
        a.part[2 * (size_t)bh + 1] = (s_fin[1][0] + s_fin[1][1]) + (s_fin[1][2] + s_fin[1][3]);
    }
}

// fixed-order sum of the per-chain partials: dtemp = sum_bh part[bh][0]; scalar dfr = sum_bh part[bh][1]
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
    const int rpt_need = (a.N + 15) / 16;
    dim3 grid(B * a.H), block(256);
#define SLOT_CF(R) if (rpt_need <= R) { hipLaunchKernelGGL((chain_fwd<D, R, TI>), grid, block, 0, st, a); return hipGetLastError(); }
    SLOT_CF(2) SLOT_CF(4) SLOT_CF(6) SLOT_CF(8) SLOT_CF(12)
#undef SLOT_CF
    return hipErrorInvalidValue;
}
template <int D, typename TI>
hipError_t launch_chain_bwd(const ChainBwdArgs& a, int B, hipStream_t st) {
    const int rpt_need = (a.N + 15) / 16;
    dim3 grid(B * a.H), block(256);
#define SLOT_CB(R) if (rpt_need <= R) { \
        if (a.occb) hipLaunchKernelGGL((chain_bwd<D, R, TI, true>), grid, block, 0, st, a); \
        else hipLaunchKernelGGL((chain_bwd<D, R, TI, false>), grid, block, 0, st, a); \
        return hipGetLastError(); }
    SLOT_CB(2) SLOT_CB(4) SLOT_CB(6) SLOT_CB(8) SLOT_CB(12)
#undef SLOT_CB
    return hipErrorInvalidValue;
}

}  // namespace

// ======================================================================================== C-ABI
#include "slotscan.h"
#include <mutex>
#include <vector>

// Optional per-kernel timing with HIP events recorded on the launch stream around every kernel (the
// reference times its compiled kernels the same way with CUDA events, kvu/prof_cuda.py:9-20).
namespace slotprof {
std::mutex mu;
bool on = false;
std::vector<hipEvent_t> pool;
struct Rec { int kid; hipEvent_t a, b; };
std::vector<Rec> recs;
hipEvent_t get() {
    if (!pool.empty()) { hipEvent_t e = pool.back(); pool.pop_back(); return e; }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}
struct Scope {
    int kid; hipStream_t st; hipEvent_t a = nullptr;
    Scope(int k, hipStream_t s) : kid(k), st(s) {
        if (!on) return;
        std::lock_guard<std::mutex> g(mu);
        a = get();
        if (a) hipEventRecord(a, st);
    }
    ~Scope() {
        if (!a) return;
        std::lock_guard<std::mutex> g(mu);
        hipEvent_t b = get();
        if (!b) return;
        hipEventRecord(b, st);
        recs.push_back({kid, a, b});
    }
};
}  // namespace slotprof

extern "C" int slotscan_profile(int enable) {
    std::lock_guard<std::mutex> g(slotprof::mu);
    slotprof::on = enable != 0;
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

static thread_local char g_err[512];
static int fail(int code, const char* msg) {
    snprintf(g_err, sizeof g_err, "%s", msg);
    return code;
}
static int hip_fail(hipError_t e, const char* where) {
    snprintf(g_err, sizeof g_err, "%s: %s", where, hipGetErrorString(e));
    return SLOTSCAN_ERR_HIP;
}

extern "C" const char* slotscan_last_error(void) { return g_err; }
extern "C" int slotscan_max_slots(int64_t D) { (void)D; return SLOTSCAN_MAX_SLOTS; }

static int check_common(int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G, int dtype) {
    if (B < 1 || T < 1 || H < 1 || N < 1 || G < 1) return fail(SLOTSCAN_ERR_SHAPE, "B, T, H, N and G must be >= 1");
    if (D != 64 && D != 128) return fail(SLOTSCAN_ERR_SHAPE, "the scan supports DK == DV in {64, 128}");
    if (N > SLOTSCAN_MAX_SLOTS) return fail(SLOTSCAN_ERR_SHAPE, "N exceeds SLOTSCAN_MAX_SLOTS (192)");
    if (dtype != SLOTSCAN_F32 && dtype != SLOTSCAN_BF16) return fail(SLOTSCAN_ERR_DTYPE, "token dtype must be f32 or bf16");
    if (B * H > 0x7fffffffLL || T > 0x7fffffffLL) return fail(SLOTSCAN_ERR_SHAPE, "B*H and T must fit in int32");
    return 0;
}
static bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

extern "C" int slotscan_fwd(const void* k, const void* q, const void* v, int dtype,
                            const float* gate, const float* fr, int fr_per_token, const float* temp,
                            int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                            float eps, int occ_bin,
                            const float* k0, const float* v0, const float* o0,
                            float* kbuf, float* vbuf, int32_t* am,
                            float* kold, float* vold, float* oold,
                            float* kfin, float* vfin, float* ofin, void* stream) {
    if (int r = check_common(B, T, H, N, D, G, dtype)) return r;
    if (!k || !q || !v || !gate || !fr || !temp || !kbuf || !vbuf || !am || !kfin || !vfin || !ofin)
        return fail(SLOTSCAN_ERR_NULL, "slotscan_fwd: a required pointer is NULL");
    if ((kold == nullptr) != (oold == nullptr) || (kold == nullptr) != (vold == nullptr))
        return fail(SLOTSCAN_ERR_NULL, "slotscan_fwd: kold, vold and oold must be all set or all NULL");
    if (!al16(k) || !al16(q) || !al16(v) || !al16(kbuf) || !al16(vbuf) || !al16(kfin) || !al16(vfin) ||
        (kold && (!al16(kold) || !al16(vold))) || (k0 && !al16(k0)) || (v0 && !al16(v0)))
        return fail(SLOTSCAN_ERR_ALIGN, "slotscan_fwd: row buffers must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    const int NB = (int)((T + G - 1) / G);
    ChainFwdArgs ca{q, k, gate, fr, temp, k0, o0, kbuf, am, kold, oold, kfin, ofin,
                    (int)T, (int)H, (int)N, (int)G, NB, eps, fr_per_token ? 1 : 0, occ_bin ? 1 : 0};
    hipError_t e;
    {
        slotprof::Scope sc(SLOTSCAN_K_CHAIN_FWD, st);
        if (D == 128) e = dtype == SLOTSCAN_BF16 ? launch_chain_fwd<128, bf16_t>(ca, (int)B, st) : launch_chain_fwd<128, float>(ca, (int)B, st);
        else e = dtype == SLOTSCAN_BF16 ? launch_chain_fwd<64, bf16_t>(ca, (int)B, st) : launch_chain_fwd<64, float>(ca, (int)B, st);
    }
    if (e != hipSuccess) return hip_fail(e, "chain_fwd launch");
    RowsFwdArgs ra{v, gate, am, v0, vbuf, vold, vfin, (int)T, (int)H, (int)N, (int)G, NB};
    dim3 grid((unsigned)(B * H), (unsigned)((N + 31) / 32)), block(512);
    {
        slotprof::Scope sc(SLOTSCAN_K_ROWS_FWD, st);
        if (D == 128) {
            if (dtype == SLOTSCAN_BF16) hipLaunchKernelGGL((rows_fwd<128, bf16_t>), grid, block, 0, st, ra);
            else hipLaunchKernelGGL((rows_fwd<128, float>), grid, block, 0, st, ra);
        } else {
            if (dtype == SLOTSCAN_BF16) hipLaunchKernelGGL((rows_fwd<64, bf16_t>), grid, block, 0, st, ra);
            else hipLaunchKernelGGL((rows_fwd<64, float>), grid, block, 0, st, ra);
        }
        e = hipGetLastError();
    }
    if (e != hipSuccess) return hip_fail(e, "rows_fwd launch");
    return 0;
}

extern "C" size_t slotscan_bwd_workspace(int64_t B, int64_t T, int64_t H, int64_t N) {
    // Dn (B*H, N, T) fp32, then the per-chain partials (B*H, 2) fp32, 256-byte aligned
    const size_t dn = (size_t)B * H * N * T * sizeof(float);
    return ((dn + 255) & ~(size_t)255) + (size_t)B * H * 2 * sizeof(float);
}

extern "C" int slotscan_bwd(const void* k, const void* q, const void* v, int dtype,
                            const float* gate, const float* fr, int fr_per_token, const float* temp,
                            int64_t B, int64_t T, int64_t H, int64_t N, int64_t D, int64_t G,
                            float eps, int occ_bin,
                            const int32_t* am, const float* kold, const float* vold, const float* oold,
                            const float* kfin, const float* vfin, const float* ofin,
                            const float* dkbuf, const float* dvbuf, void* workspace,
                            void* dk, void* dq, void* dv, float* dgate, float* dfr, float* dtemp,
                            void* stream) {
    if (int r = check_common(B, T, H, N, D, G, dtype)) return r;
    if (!k || !q || !v || !gate || !fr || !temp || !am || !kold || !vold || !oold || !kfin || !vfin || !ofin ||
        !dkbuf || !dvbuf || !workspace || !dk || !dq || !dv || !dgate || !dfr || !dtemp)
        return fail(SLOTSCAN_ERR_NULL, "slotscan_bwd: a required pointer is NULL");
    if (!al16(k) || !al16(q) || !al16(v) || !al16(kold) || !al16(vold) || !al16(kfin) || !al16(vfin) ||
        !al16(dkbuf) || !al16(dvbuf) || !al16(dk) || !al16(dv) || ((uintptr_t)workspace & 255u))
        return fail(SLOTSCAN_ERR_ALIGN, "slotscan_bwd: row buffers must be 16-byte aligned (workspace 256)");
    hipStream_t st = (hipStream_t)stream;
    const int NB = (int)((T + G - 1) / G);
    float* dn = (float*)workspace;
    const size_t dnb = (size_t)B * H * N * T * sizeof(float);
    float* part = (float*)((char*)workspace + ((dnb + 255) & ~(size_t)255));
    RowsBwdArgs ra{k, v, gate, am, kold, vold, kfin, vfin, dkbuf, dvbuf, dk, dv, dn,
                   (int)T, (int)H, (int)N, (int)G, NB};
    dim3 grid((unsigned)(B * H), (unsigned)((N + 31) / 32)), block(512);
    hipError_t e;
    {
        slotprof::Scope sc(SLOTSCAN_K_ROWS_BWD, st);
        if (D == 128) {
            if (dtype == SLOTSCAN_BF16) hipLaunchKernelGGL((rows_bwd<128, bf16_t>), grid, block, 0, st, ra);
            else hipLaunchKernelGGL((rows_bwd<128, float>), grid, block, 0, st, ra);
        } else {
            if (dtype == SLOTSCAN_BF16) hipLaunchKernelGGL((rows_bwd<64, bf16_t>), grid, block, 0, st, ra);
            else hipLaunchKernelGGL((rows_bwd<64, float>), grid, block, 0, st, ra);
        }
        e = hipGetLastError();
    }
    if (e != hipSuccess) return hip_fail(e, "rows_bwd launch");
    ChainBwdArgs ca{q, gate, fr, temp, am, kold, oold, kfin, ofin, dn, dq, dgate, dfr, part,
                    (int)T, (int)H, (int)N, eps, fr_per_token ? 1 : 0, occ_bin ? 1 : 0};
    {
        slotprof::Scope sc(SLOTSCAN_K_CHAIN_BWD, st);
        if (D == 128) e = dtype == SLOTSCAN_BF16 ? launch_chain_bwd<128, bf16_t>(ca, (int)B, st) : launch_chain_bwd<128, float>(ca, (int)B, st);
        else e = dtype == SLOTSCAN_BF16 ? launch_chain_bwd<64, bf16_t>(ca, (int)B, st) : launch_chain_bwd<64, float>(ca, (int)B, st);
    }
    if (e != hipSuccess) return hip_fail(e, "chain_bwd launch");
    {
        slotprof::Scope sc(SLOTSCAN_K_REDUCE, st);
        hipLaunchKernelGGL(reduce_parts, dim3(1), dim3(256), 0, st, part, (int)(B * H), dtemp,
                           fr_per_token ? (float*)nullptr : dfr);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return hip_fail(e, "reduce_parts launch");
    return 0;
}
