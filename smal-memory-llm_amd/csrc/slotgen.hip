// General-mode slot scan for MI355X (gfx950): soft write addresses (hard = false) and the attached address
// gradient (detach_addr = false), any DK, DV in {64, 128}, N <= 192.  The hard + detached mode has its own
// row-sparse kernels (slotscan.hip); every other mode runs here, as the reference runs every other mode on
// its general Triton scan (/root/reference/gqa25/slotkern_cuda.py:539-542 -> slotkern_kvg.py:257-265).
//
// Semantics (reference: slotkern_kv.py:66-123; the adjoints of slotkern_kvt.py:157-171 with the stride-G
// gradient entry of slotkern_kvg.py:165-168).  Per (b, h) chain, state K (N, DK), V (N, DV), o (N) from zero;
// for t = 0..T-1:
//   t % G == 0: emit (K, V, o), the PRE-write state
//   s_n = temp <K_n / max(|K_n|, 1e-6), q_t / max(|q_t|, 1e-6)>,  z_n = s_n - fr_t (occ_bin ? [o_n >= eps] : o_n)
//   only occupied rows (o_n >= eps) and the lowest-index free row compete
//   a = softmax(z) (soft) or onehot(argmax z), first maximum wins (hard; the gradient is straight-through
//   the softmax, slotkern_kv.py:108-110);  w = g_t a
//   K <- (1-w) K + w k_t,  V <- (1-w) V + w v_t,  o <- (1-w) o + w
// The forward logs, per step, every row's pre-write occupancy o, soft address a_s, scaled cosine s and |K|,
// and 1 / max(|q_t|, 1e-6) (the address log, rlog).
// Backward, per stride-G segment in reverse: replay the segment's keys from its emitted copy with the logged
// addresses (key checkpoints and one value row scalar per step into per-chain scratch; the scores and the
// address are not recomputed, so the replay has no cross-wave exchange), then walk it backward:
//   dw_n = <k_t - K_n, dK_n> + <v_t - V_n, dV_n> + (1 - o_n) do_n
//   dk_t = sum_n w_n dK_n,  dv_t = sum_n w_n dV_n,  dgate_t = sum_n a_n dw_n
//   dz_n = a_s,n (g dw_n - sum_m a_s,m g dw_m)                       (a_s the soft address, 0 off the mask)
//   dfr_t = -sum_n occ_n dz_n,  dtemp += sum_n dz_n s_n / temp,  dq_t = qinv (dqn - qn <qn, dqn>),
//   dqn = temp sum_n dz_n kn_n  (qinv dqn where |q_t| < 1e-6)
//   attached address only: dK_n += dz_n kinv_n (temp qn - s_n kn_n)  (temp dz_n kinv_n qn where |K_n| < 1e-6)
//   pin (the reference's ref_scan_kv default, slotkern_kv.py:88-101): s_n = 0 where |K_n| < 1e-6, and those
//   rows' dz is cut from dtemp, dq and the attached key gradient (dfr and the occupancy carry keep it)
//   carry: dK = (1-w) dK, dV = (1-w) dV, do = (1-w) do - fr_t dz (no -fr dz under occ_bin);
//   at a segment's first step the emitted copy's gradient (dkbuf, dvbuf) joins dK, dV.
// Inside a segment dV only scales (dV(t+) = c(t) D, c the product of (1 - w) over the later steps), so the
// value term of dw is c(t) (<v_t, D> - <V(t), D>), and <V(t), D> follows the forward recurrence from the
// emitted copy: the value state is never replayed or stored.
//
// gfx950 mapping.  One workgroup of 8 waves per chain; the state lives in registers.  Lane = 4 row-lanes
// (the wave's 16-lane DPP rows) x 16 dim-lanes: a lane holds RPL rows x DK/16 key dims (and DV/16 value
// dims), wave w rows w*4*RPL .. (w+1)*4*RPL - 1, so a row dot product is a 16-lane DPP reduction and a sum
// over rows is a 4-row permlane reduction plus one LDS exchange across the waves.  Each step of the
// forward needs one workgroup barrier: every wave posts its (max, sum) of the competing scores, its first
// free row and its best row to a double-buffered LDS slot, and all waves combine the 8 posts.  The
// backward's replay needs none (the address comes from the log).  Each step of its walk needs one: the waves post the
// address-gradient sums and their dk/dv partials; the previous step's dq/dfr/dtemp partials ride along on
// the same exchange.  The scratch is written and read in 16-byte units, each row by its 16 dim-lanes.
// The step is bound by its VALU instruction count (2 waves per SIMD), so the clamped inverse norms and the
// softmax normaliser use the hardware v_rsq / v_rcp / v_sqrt (1 ulp) instead of IEEE division sequences.
#include <type_traits>

#include "slot_common.h"
#include "slotscan.h"
#include "slot_host.h"

using namespace slot;
using slothost::fail;
using slothost::hip_fail;
using slothost::al16;

namespace {

#define GEN_WAVES 8
#define GEN_THREADS (64 * GEN_WAVES)
constexpr float GEN_NORM_EPS = 1e-6f;

struct GenArgs {
    const void* k; const void* q; const void* v;
    const float* gate; const float* fr; const float* temp;
    int frt, T, H, N, G, NB, occ_bin, hard, detach, pin;
    float eps;
    float* kbuf; float* vbuf; float* obuf; int32_t* am;          // forward outputs (am: hard only)
    float* wb;                                                    // optional: the address of every step
    float* rlog;                                                  // the address log (written by the forward)
    const float* dkbuf; const float* dvbuf;                       // backward inputs
    float* scr; int64_t scr_chain;                                 // replay scratch, floats per chain
    void* dk; void* dq; void* dv; float* dg; float* dfr; float* part;
};

// ---- gate and fr of 64 consecutive steps [base, base + 64) of one chain, step base + l in lane l of every
// wave: one vector load per 64 steps, read per step with a readlane, instead of two scalar loads per step
// (each a cache miss on the step's critical path).
struct StepPar {
    float g, f;
    int am;                                   // the written row (hard mode, backward), else -1
    int base;
};
__device__ __forceinline__ StepPar load_steppar(const float* gate, const float* fr, int frt, const int32_t* am,
                                                int T, int H, size_t tok0, int base, int lane) {
    StepPar p;
    p.base = base;
    const int t = base + lane;
    const bool ok = t >= 0 && t < T;
    const size_t ti = tok0 + (size_t)(ok ? t : 0) * H;
    p.g = ok ? gate[ti] : 0.f;
    p.f = frt ? (ok ? fr[ti] : 0.f) : fr[0];
    p.am = (am && ok) ? am[ti] : -1;
    return p;
}
__device__ __forceinline__ float steppar_g(const StepPar& p, int t) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p.g), t - p.base));
}
__device__ __forceinline__ float steppar_f(const StepPar& p, int t) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p.f), t - p.base));
}
__device__ __forceinline__ int steppar_am(const StepPar& p, int t) { return __builtin_amdgcn_readlane(p.am, t - p.base); }

// ---- token loads (f32 or bf16 tokens, always fp32 registers)
template <typename TI, int N> __device__ __forceinline__ void ldtok(const TI* p, float* x) {
    if constexpr (sizeof(TI) == 4) {
#pragma unroll
        for (int i = 0; i < N; i += 4) {
            const float4 f = ld4(reinterpret_cast<const float*>(p) + i);
            x[i] = f.x; x[i + 1] = f.y; x[i + 2] = f.z; x[i + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; i += 4) {
            const float4 f = ld4(reinterpret_cast<const bf16_t*>(p) + i);
            x[i] = f.x; x[i + 1] = f.y; x[i + 2] = f.z; x[i + 3] = f.w;
        }
    }
}
// Raw token bytes of a lane's N elements (8 or a multiple of 16 bytes), loaded one step ahead and converted
// only where used: a prefetch held as converted fp32 registers took twice the registers, and the compiler
// then converted (and waited for) each load right after issuing it.  `base` is uniform, `off` the lane's
// byte offset, so the loads use a scalar base with a 32-bit lane offset.
template <typename TI, int N> struct RawTok {
    static constexpr int BYTES = N * (int)sizeof(TI);
    static constexpr int NW = BYTES / 4;   // 32-bit words
    static_assert(BYTES == 8 || BYTES % 16 == 0, "token slice must be 8 bytes or whole 16-byte pieces");
    uint32_t w[NW];
    __device__ __forceinline__ void load(const void* base, uint32_t off) {
        const char* p = (const char*)base + off;
        if constexpr (BYTES == 8) {
            const uint2 v = *reinterpret_cast<const uint2*>(p);
            w[0] = v.x; w[1] = v.y;
        } else {
#pragma unroll
            for (int u = 0; u < NW / 4; u++) {
                const uint4 v = *reinterpret_cast<const uint4*>(p + 16 * u);
                w[4 * u] = v.x; w[4 * u + 1] = v.y; w[4 * u + 2] = v.z; w[4 * u + 3] = v.w;
            }
        }
    }
    __device__ __forceinline__ void cvt(float* x) const {
#pragma unroll
        for (int i = 0; i < NW; i++) {
            if constexpr (sizeof(TI) == 4) {
                x[i] = __uint_as_float(w[i]);
            } else {
                x[2 * i] = __uint_as_float(w[i] << 16);
                x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
            }
        }
    }
};

template <typename TI> __device__ __forceinline__ void sttok4(TI* p, float4 v) {
    if constexpr (sizeof(TI) == 4) st4(reinterpret_cast<float*>(p), v);
    else st4(reinterpret_cast<bf16_t*>(p), v);
}

// The two lanes' copies a permlane swap returns: [0] from the lower 16-lane row (or 32-lane half), [1] from
// the upper one, at every lane -- so pairs of values swapped separately stay matched.
__device__ __forceinline__ void swap16(float x, float& lo, float& hi) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    lo = __uint_as_float(p[0]); hi = __uint_as_float(p[1]);
}
__device__ __forceinline__ void swap32(float x, float& lo, float& hi) {
    auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    lo = __uint_as_float(p[0]); hi = __uint_as_float(p[1]);
}

// (max, sum of exp(z - max)) of two partial softmax sums; an empty part has sum 0.
__device__ __forceinline__ void ms_merge(float m0, float s0, float m1, float s1, float& m, float& s) {
    m = fmaxf(m0, m1);
    s = (s0 > 0.f ? s0 * __expf(m0 - m) : 0.f) + (s1 > 0.f ? s1 * __expf(m1 - m) : 0.f);
}
// Lower (index, value) wins; index INT_MAX = none.
__device__ __forceinline__ void idx_merge(int i0, float v0, int i1, float v1, int& i, float& v) {
    const bool lo = i0 <= i1;
    i = lo ? i0 : i1; v = lo ? v0 : v1;
}
// Larger value wins, the lower index on a tie (first maximum); index INT_MAX = none.
__device__ __forceinline__ void best_merge(float z0, int i0, float z1, int i1, float& z, int& i) {
    const bool first = (i1 == INT_MAX) || (i0 != INT_MAX && (z0 > z1 || (z0 == z1 && i0 < i1)));
    z = first ? z0 : z1; i = first ? i0 : i1;
}

// Workgroup barrier for an exchange through LDS only: this wave's LDS accesses complete, then s_barrier.
// __syncthreads() would also wait for every global store the wave has in flight (its release fence), and the
// per-step exchanges below do not need that: what they publish is in LDS.  Global data another wave reads
// (the replay scratch) is published with __syncthreads().
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// rowsum16 whose result is materialised where it is formed: its last DPP add then folds into one
// instruction (when the sum's uses sit in later blocks the compiler had sunk that add behind a separate DPP
// move and a zero-initialised register)
__device__ __forceinline__ float rowsum16p(float v) {
    v = rowsum16(v);
    asm volatile("" : "+v"(v));
    return v;
}
// Sum over the 4 row-lanes (lanes c, c+16, c+32, c+48).
__device__ __forceinline__ float rows4_sum(float x) { return sum4rows(x); }

// Reduce-scatter of NV per-lane values over the 4 row-lanes: row-lane rl ends with the totals of values
// rows4_rs_base<NV>(rl) .. + NV / 4 - 1.  The 16-lane swap first, then the 32-lane one, each adding its
// two returned copies in the same order as sum4rows, so every total is bitwise sum4rows' result; 3 NV / 4
// swaps instead of 2 NV.
template <int NV> __device__ __forceinline__ void rows4_rs(const float (&x)[NV], float (&y)[NV / 4]) {
    float a[NV / 2];
#pragma unroll
    for (int k = 0; k < NV / 2; k++) {   // rows 0, 2 keep values k, rows 1, 3 values NV / 2 + k
        auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x[k]), __float_as_uint(x[NV / 2 + k]), false, false);
        a[k] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
#pragma unroll
    for (int k = 0; k < NV / 4; k++) {   // the lower half keeps a[k], the upper half a[NV / 4 + k]
        auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[k]), __float_as_uint(a[NV / 4 + k]), false, false);
        y[k] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
}
template <int NV> __device__ __forceinline__ int rows4_rs_base(int rl) { return (NV / 4) * (rl >> 1) + (NV / 2) * (rl & 1); }

// One step's address over the chain: every lane gets its rows' soft address a_s, the address a used for the
// write (a_s, or the one-hot of `hard_row`), and the winning row of the hard argmax.  xf is the workgroup
// exchange slot of this step: [wave][8] = {softmax max, sum, first-free index, its z, best z, best index}.
// shadow() runs between the wave's post and the barrier: work that no other wave waits for fills the wait.
template <int RPL, typename F>
__device__ __forceinline__ int gen_address(const float (&z)[RPL], const float (&o)[RPL], int nbase, int N,
                                           float eps, bool hard, int hard_row, float* xf, int w, int lane,
                                           float (&as)[RPL], float (&ad)[RPL], F&& shadow) {
    // Short dependency chains: maxima first, then independent exponentials summed in trees (the lane's rows,
    // its 4 row-lanes, the 8 waves' posts), instead of an online softmax carried row by row.
    float m = -INFINITY;
    int ff = INT_MAX; float zff = 0.f;
    float bz = 0.f; int bi = INT_MAX;
    bool cmp[RPL];
#pragma unroll
    for (int j = 0; j < RPL; j++) {
        const int n = nbase + j;
        cmp[j] = n < N && o[j] >= eps;
        if (cmp[j]) {
            m = fmaxf(m, z[j]);
            if (bi == INT_MAX || z[j] > bz) { bz = z[j]; bi = n; }
        } else if (n < N && ff == INT_MAX) {
            ff = n; zff = z[j];
        }
    }
    {   // the max and the index reductions over the 4 row-lanes
        float m0, m1, a0, a1, b0, b1, c0, c1, d0, d1;
        swap16(m, m0, m1); m = fmaxf(m0, m1);
        swap16(__int_as_float(ff), a0, a1); swap16(zff, b0, b1);
        idx_merge(__float_as_int(a0), b0, __float_as_int(a1), b1, ff, zff);
        swap16(bz, c0, c1); swap16(__int_as_float(bi), d0, d1);
        best_merge(c0, __float_as_int(d0), c1, __float_as_int(d1), bz, bi);
        swap32(m, m0, m1); m = fmaxf(m0, m1);
        swap32(__int_as_float(ff), a0, a1); swap32(zff, b0, b1);
        idx_merge(__float_as_int(a0), b0, __float_as_int(a1), b1, ff, zff);
        swap32(bz, c0, c1); swap32(__int_as_float(bi), d0, d1);
        best_merge(c0, __float_as_int(d0), c1, __float_as_int(d1), bz, bi);
    }
    float s = 0.f;                            // sum of exp(z - m) over the wave's competing rows
    {
        float e[RPL];
#pragma unroll
        for (int j = 0; j < RPL; j++) e[j] = cmp[j] ? __expf(z[j] - m) : 0.f;
#pragma unroll
        for (int j = 0; j < RPL; j++) s += e[j];
        float s0, s1;
        swap16(s, s0, s1); s = s0 + s1;
        swap32(s, s0, s1); s = s0 + s1;
    }
    if (lane == 0) {
        float4* p = reinterpret_cast<float4*>(xf + w * 8);
        p[0] = make_float4(m, s, __int_as_float(ff), zff);
        p[1] = make_float4(bz, __int_as_float(bi), 0.f, 0.f);
    }
    shadow();
    lds_barrier();
    // The 8 waves' posts are merged across the lanes of each 8-lane group (lane l reads wave l & 7's post) and
    // taken as scalars from lane 0: the maxima and the index selections are order-free, and the exponential
    // sum uses the tree of a loop over the waves, ((0 + 4) + (2 + 6)) + ((1 + 5) + (3 + 7)), so the results
    // are bitwise those of every lane merging all 8 posts (16 LDS reads and 8 exponentials per lane before)
    static_assert(GEN_WAVES == 8, "one post per lane of an 8-lane group");
    const int pw = lane & 7;
    const float4 q0 = reinterpret_cast<const float4*>(xf + pw * 8)[0];
    const float4 q1 = reinterpret_cast<const float4*>(xf + pw * 8)[1];
    float mx = q0.x;
    mx = fmaxf(mx, dppf<SLOT_DPP_XOR1>(mx));
    mx = fmaxf(mx, dppf<SLOT_DPP_XOR2>(mx));
    mx = fmaxf(mx, dppf<SLOT_DPP_HMIR>(mx));
    int ffl = __float_as_int(q0.z), bil = __float_as_int(q1.y);
    float zfl = q0.w, bzl = q1.x;
    auto merge_stage = [&](auto ctrl) {
        constexpr int C = decltype(ctrl)::value;
        const int fi = (int)dppu<C>((uint32_t)ffl), bi1 = (int)dppu<C>((uint32_t)bil);
        const float fz = dppf<C>(zfl), bz1 = dppf<C>(bzl);
        idx_merge(ffl, zfl, fi, fz, ffl, zfl);
        best_merge(bzl, bil, bz1, bi1, bzl, bil);
    };
    merge_stage(std::integral_constant<int, SLOT_DPP_XOR1>{});
    merge_stage(std::integral_constant<int, SLOT_DPP_XOR2>{});
    merge_stage(std::integral_constant<int, SLOT_DPP_HMIR>{});
    float M = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(mx)));
    const int FF = __builtin_amdgcn_readfirstlane(ffl);
    const float Z = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(zfl)));
    float BZ = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(bzl)));
    int BI = __builtin_amdgcn_readfirstlane(bil);
    if (FF != INT_MAX) {                      // the first free row competes too
        M = fmaxf(M, Z);
        best_merge(BZ, BI, Z, FF, BZ, BI);
    }
    float S = FF != INT_MAX ? __expf(Z - M) : 0.f;
    {
        float sw = q0.y > 0.f ? q0.y * __expf(q0.x - M) : 0.f;
        sw += dppf<0x12C>(sw);                // row_ror:12: lanes 0..3 add the posts of waves 4..7
        sw += dppf<SLOT_DPP_XOR2>(sw);        // lanes 0, 1 add lanes 2, 3
        sw += dppf<SLOT_DPP_XOR1>(sw);        // lane 0 adds lane 1
        S += __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sw)));
    }
    const float rS = __builtin_amdgcn_rcpf(S);
    const int row = hard ? (hard_row >= 0 ? hard_row : BI) : -1;
#pragma unroll
    for (int j = 0; j < RPL; j++) {
        const int n = nbase + j;
        const bool comp = n < N && (o[j] >= eps || n == FF);
        as[j] = comp ? __expf(z[j] - M) * rS : 0.f;
        ad[j] = hard ? (n == row ? 1.f : 0.f) : as[j];
    }
    return BI;
}

// Scores of one step: z, the raw scaled cosine s, |K_n| and 1 / max(|q|, 1e-6).
template <int RPL, int DPK>
__device__ __forceinline__ void gen_scores(const float (&K)[RPL][DPK], const float (&o)[RPL], const float* qt,
                                           float temp, float frt, float eps, bool occ_bin, bool pin,
                                           float (&z)[RPL], float (&sr)[RPL], float (&kn)[RPL], float& qinv) {
    float qq = 0.f;
#pragma unroll
    for (int i = 0; i < DPK; i++) qq = fmaf(qt[i], qt[i], qq);
    qq = rowsum16p(qq);
    qinv = __builtin_amdgcn_rsqf(fmaxf(qq, GEN_NORM_EPS * GEN_NORM_EPS));   // 1 / max(|q|, 1e-6)
#pragma unroll
    for (int j = 0; j < RPL; j++) {
        float d = 0.f, n2 = 0.f;
#pragma unroll
        for (int i = 0; i < DPK; i++) { d = fmaf(K[j][i], qt[i], d); n2 = fmaf(K[j][i], K[j][i], n2); }
        d = rowsum16p(d);
        n2 = rowsum16p(n2);
        kn[j] = __builtin_amdgcn_sqrtf(n2);
        const float kinv = __builtin_amdgcn_rsqf(fmaxf(n2, GEN_NORM_EPS * GEN_NORM_EPS));   // 1 / max(|K|, 1e-6)
        sr[j] = temp * (d * kinv * qinv);
        if (pin && kn[j] < GEN_NORM_EPS) sr[j] = 0.f;   // pinned: a (near-)zero row scores 0
        const float occ = occ_bin ? (o[j] >= eps ? 1.f : 0.f) : o[j];
        z[j] = sr[j] - frt * occ;
    }
}

// a <- fmaf(m, a, p), the result in a's own register.  The compiler's v_fmac form ties the destination to the
// addend p, so a state updated that way in a loop moved to new registers every step and was copied back at the
// loop's end (about 140 register moves per forward step at RPL 6).  The same single-rounding fma.
__device__ __forceinline__ void fma_in(float& a, float m, float p) {
    asm("v_fma_f32 %0, %1, %0, %2" : "+v"(a) : "v"(m), "v"(p));
}

// The write of one step into this lane's rows: X <- (1 - wr) X + wr x (keys, or values), o likewise.
template <int RPL, int DP>
__device__ __forceinline__ void gen_update(float (&X)[RPL][DP], const float (&wr)[RPL], const float* x) {
#pragma unroll
    for (int j = 0; j < RPL; j++) {
        const float omw = 1.f - wr[j];
#pragma unroll
        for (int i = 0; i < DP; i++) fma_in(X[j][i], omw, wr[j] * x[i]);
    }
}

// X[j] <- this lane's slice of rows nbase + j of an fp32 (rows, DP * 16) slab at `base` (uniform), `off` the
// lane's byte offset of row nbase; `nv` rows of the lane exist (the rest read 0).  All rows exist in the
// common case (full): the loads are then unconditional, a scalar base plus one 32-bit lane offset.
template <int RPL, int DP>
__device__ __forceinline__ void ld_rows(float (&X)[RPL][DP], const float* base, uint32_t off, bool full, int nv) {
    const char* p = reinterpret_cast<const char*>(base) + off;
#pragma unroll
    for (int j = 0; j < RPL; j++) {
#pragma unroll
        for (int i = 0; i < DP; i += 4) {
            const float4 f = (full || j < nv) ? *reinterpret_cast<const float4*>(p + (j * DP * 16 + i) * 4)
                                              : make_float4(0.f, 0.f, 0.f, 0.f);
            X[j][i] = f.x; X[j][i + 1] = f.y; X[j][i + 2] = f.z; X[j][i + 3] = f.w;
        }
    }
}

// ------------------------------------------------------------------------------------------- forward
// Per step, in this order: the step's token rows (loaded during the previous step) are converted; the
// stores are issued (the snapshot at t % G == 0, the previous step's address log); the next step's token
// rows are loaded; then the scores, the address exchange and the update run.  No store is issued between a
// token load and its use, so the wait for the tokens never waits for stores, and the loads have a whole
// step to arrive.  Every global access is a uniform (scalar) base plus a 32-bit lane offset.
template <typename TI, int DK, int DV, int RPL>
__global__ __launch_bounds__(GEN_THREADS) void gen_fwd(GenArgs a) {
    constexpr int DPK = DK / 16, DPV = DV / 16, RPW = 4 * RPL;
    __shared__ __align__(16) float xf[2][GEN_WAVES * 8];
    const int chain = blockIdx.x, b = chain / a.H, h = chain % a.H;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, dl = lane & 15;
    const int nbase = w * RPW + (lane >> 4) * RPL;
    const float temp = a.temp[0];
    float K[RPL][DPK], V[RPL][DPV], o[RPL];
#pragma unroll
    for (int j = 0; j < RPL; j++) {
#pragma unroll
        for (int i = 0; i < DPK; i++) K[j][i] = 0.f;
#pragma unroll
        for (int i = 0; i < DPV; i++) V[j][i] = 0.f;
        o[j] = 0.f;
    }
    auto tok = [&](int t) { return ((size_t)b * a.T + t) * a.H + h; };
    const size_t tok0 = tok(0);
    const uint32_t tk_off = (uint32_t)(dl * DPK * sizeof(TI)), tv_off = (uint32_t)(dl * DPV * sizeof(TI));
    auto krow = [&](int t) { return (const char*)a.k + tok(t) * DK * sizeof(TI); };
    auto qrow = [&](int t) { return (const char*)a.q + tok(t) * DK * sizeof(TI); };
    auto vrow = [&](int t) { return (const char*)a.v + tok(t) * DV * sizeof(TI); };
    // this lane's slice of row nbase in a snapshot slab (bytes); row nbase + j is j * D * 4 further
    const uint32_t sk_off = (uint32_t)((nbase * DK + dl * DPK) * 4), sv_off = (uint32_t)((nbase * DV + dl * DPV) * 4);
    StepPar spc = load_steppar(a.gate, a.fr, a.frt, nullptr, a.T, a.H, tok0, 0, lane);   // steps [64 i, 64 i + 64)
    StepPar spn = load_steppar(a.gate, a.fr, a.frt, nullptr, a.T, a.H, tok0, 64, lane);  // the next 64, in flight
    RawTok<TI, DPK> rk, rq;
    RawTok<TI, DPV> rv;
    rk.load(krow(0), tk_off); rq.load(qrow(0), tk_off); rv.load(vrow(0), tv_off);
    // the previous step's address log, stored at the top of the next step
    float lo = 0.f, la = 0.f, ls = 0.f, lk = 0.f, lq = 0.f;
    float lw[RPL];
    int lbest = -1;
    // nb, d, tid: this lane's nbase, dim-lane and thread index (taken from the step's opaque copy)
    auto store_log = [&](int t, int nb, int d, uint32_t tid) {
        const size_t ti = tok(t);
        if (a.hard && tid == 0) a.am[ti] = lbest;
        if (a.wb && d == 0) {
#pragma unroll
            for (int j = 0; j < RPL; j++)
                if (nb + j < a.N) a.wb[ti * a.N + nb + j] = lw[j];
        }
        if (a.rlog) {                         // dim-lane j < RPL stores row nbase + j
            const int n = nb + d;
            float* rec = a.rlog + ((size_t)chain * a.T + t) * 4 * a.N;
            if (d < RPL && n < a.N) { rec[n] = lo; rec[a.N + n] = la; rec[2 * a.N + n] = ls; rec[3 * a.N + n] = lk; }
            if (tid == 0) a.rlog[(size_t)gridDim.x * a.T * 4 * a.N + (size_t)chain * a.T + t] = lq;
        }
    };
    // The value rows are not read by the step's scores: step t's value write is applied during step t + 1's
    // address exchange (between the wave's post and the barrier), or before the snapshot when step t + 1
    // emits one.  pvt, pwr: the pending write's value token and weights.
    float pvt[DPV], pwr[RPL];
#pragma unroll
    for (int i = 0; i < DPV; i++) pvt[i] = 0.f;
#pragma unroll
    for (int j = 0; j < RPL; j++) pwr[j] = 0.f;
    for (int t = 0; t < a.T; t++) {
        // the lane indices re-derived from an opaque copy every step: comparisons on them are then not loop
        // invariant, so the compiler does not hoist the per-row and per-lane masks into scalar registers
        // (they had spilled to VGPR lanes, reloaded by readlane every step)
        uint32_t tido;
        asm volatile("v_mov_b32 %0, %1" : "=v"(tido) : "v"((uint32_t)threadIdx.x));
        const int lane_s = (int)(tido & 63u), dl_s = lane_s & 15, nb_s = w * RPW + (lane_s >> 4) * RPL;
        float kt[DPK], qt[DPK], vt[DPV];
        rk.cvt(kt); rq.cvt(qt); rv.cvt(vt);
        // converted here, so that the raw words are dead before the next step's loads reuse their registers
        // (converted where used, they were live across those loads, which then went to other registers and
        // were copied back at the loop's end: 24 moves per step)
#pragma unroll
        for (int i = 0; i < DPK; i++) asm volatile("" : "+v"(kt[i]), "+v"(qt[i]));
#pragma unroll
        for (int i = 0; i < DPV; i++) asm volatile("" : "+v"(vt[i]));
        if (t > 0 && (t & 63) == 0) {
            spc = spn;
            spn = load_steppar(a.gate, a.fr, a.frt, nullptr, a.T, a.H, tok0, t + 64, lane);
        }
        const bool snap = t % a.G == 0;
        if (snap) {                           // emit the pre-write state
            if (t > 0) gen_update<RPL, DPV>(V, pwr, pvt);
            const size_t slab = (((size_t)b * a.NB + t / a.G) * a.H + h) * a.N;
            char* kb = (char*)(a.kbuf + slab * DK);
            char* vb = (char*)(a.vbuf + slab * DV);
#pragma unroll
            for (int j = 0; j < RPL; j++) {
                if (nb_s + j < a.N) {
#pragma unroll
                    for (int i = 0; i < DPK; i += 4)
                        *reinterpret_cast<float4*>(kb + sk_off + (j * DK + i) * 4) = make_float4(K[j][i], K[j][i + 1], K[j][i + 2], K[j][i + 3]);
#pragma unroll
                    for (int i = 0; i < DPV; i += 4)
                        *reinterpret_cast<float4*>(vb + sv_off + (j * DV + i) * 4) = make_float4(V[j][i], V[j][i + 1], V[j][i + 2], V[j][i + 3]);
                    if (dl_s == 0) a.obuf[slab + nb_s + j] = o[j];
                }
            }
        }
        if (t + 1 < a.T) { rk.load(krow(t + 1), tk_off); rq.load(qrow(t + 1), tk_off); rv.load(vrow(t + 1), tv_off); }
        const float g = steppar_g(spc, t);
        const float frt = steppar_f(spc, t);
        float z[RPL], sr[RPL], knr[RPL], qinv, as[RPL], ad[RPL], wr[RPL];
        gen_scores<RPL, DPK>(K, o, qt, temp, frt, a.eps, a.occ_bin, a.pin, z, sr, knr, qinv);
        lbest = gen_address<RPL>(z, o, nb_s, a.N, a.eps, a.hard, -1, xf[t & 1], w, lane_s, as, ad, [&] {
            if (t > 0) {                      // the previous step's log and (between snapshots) its value write
                store_log(t - 1, nb_s, dl_s, tido);
                if (!snap) gen_update<RPL, DPV>(V, pwr, pvt);
            }
        });
        lo = o[0]; la = as[0]; ls = sr[0]; lk = knr[0]; lq = qinv;
#pragma unroll
        for (int j = 1; j < RPL; j++) {
            const bool me = dl_s == j;
            lo = me ? o[j] : lo; la = me ? as[j] : la; ls = me ? sr[j] : ls; lk = me ? knr[j] : lk;
        }
#pragma unroll
        for (int j = 0; j < RPL; j++) { lw[j] = ad[j]; wr[j] = g * ad[j]; }
        gen_update<RPL, DPK>(K, wr, kt);
#pragma unroll
        for (int j = 0; j < RPL; j++) { o[j] = fmaf(1.f - wr[j], o[j], wr[j]); pwr[j] = wr[j]; }
#pragma unroll
        for (int i = 0; i < DPV; i++) pvt[i] = vt[i];
    }
    store_log(a.T - 1, nbase, dl, threadIdx.x);
}

// ------------------------------------------------------------------------------------------- backward
// The address log (rlog): per chain and step the four row scalars o, a_s, s, |K| of rows 0..N-1 (4 N
// floats, each quantity N-contiguous), then, after every chain's records, qinv per chain and step.
__host__ __device__ inline size_t gen_log_floats(int64_t BH, int64_t T, int64_t N) {
    return (size_t)BH * T * (4 * N + 1);
}

// Scratch per chain: for every segment step s the row scalar e - P = <v_t, D> - <V, D> (NP floats), then
// the pre-write keys (NP, DK) of every GC-th step after the first (the first step's are the emitted copy).
// NP = 32 * RPL.  The first GL steps of a
// segment keep their row scalars (the four logged ones and e - P), key and query token rows and qinv in
// LDS instead (gen_bwd), so the walk reads them at LDS latency; later steps read the logged ones from the
// log.  The walk rebuilds the keys of any step from the checkpoint at or before it with the updates in
// between (at most GC - 1), the same fmaf sequence, weights and token values as the replay, so bitwise the
// replay's keys.
template <int DK, int DV, int RPL>
struct GenScr {
    static constexpr int NP = 32 * RPL;
    static constexpr int GC = 4;
    __host__ __device__ static int64_t nck(int G) { return (G - 1) / GC; }
    __host__ __device__ static int64_t chain(int G) { return (int64_t)G * NP + nck(G) * NP * DK; }
};

template <typename TI, int DK, int DV, int RPL>
__global__ __launch_bounds__(GEN_THREADS) void gen_bwd(GenArgs a) {
    constexpr int DPK = DK / 16, DPV = DV / 16, RPW = 4 * RPL;
    using SC = GenScr<DK, DV, RPL>;
    constexpr int NP = SC::NP;
    constexpr int P1W = DK + DV + 4;          // per wave: dk, dv partials, then {sum a dw, sum a_s g dw}
    constexpr int P2W = DK + 4;               // per wave: dqn partial, then {sum occ dz, sum dz s}
    constexpr int GL = 8;                     // a segment's first GL steps keep their per-step data in LDS
    constexpr int TU = DK * (int)sizeof(TI) / 16;   // 16-byte pieces of a key / query token row
    __shared__ __align__(16) float p1[2][GEN_WAVES * P1W];
    __shared__ __align__(16) float p2[2][GEN_WAVES * P2W];
    // The value adjoint lives in LDS: inside a segment it only scales, dV(t+) = cV(t) D, so the walk reads
    // D and keeps the per-row factors cV in registers; D is rewritten once per segment (at its first step).
    // Each lane reads and writes only its own rows and dims.
    __shared__ __align__(16) float sD[NP * DV];
    // a segment's first GL steps: row scalars [step][5][NP] (o, a_s, s, |K| from the log, then e - P),
    // key and query token rows [step][2][DK] in the token dtype, qinv [step]
    __shared__ __align__(16) float lsc[GL * 5 * NP];
    __shared__ __align__(16) uint4 ltq[GL * 2 * TU];
    __shared__ float lqinv[GL];
    const int chain = blockIdx.x, b = chain / a.H, h = chain % a.H;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, dl = lane & 15, rl = lane >> 4;
    const int nbase = w * RPW + rl * RPL;
    TI* dkp = static_cast<TI*>(a.dk);
    TI* dqp = static_cast<TI*>(a.dq);
    TI* dvp = static_cast<TI*>(a.dv);
    const float temp = a.temp[0];
    float* scr = a.scr + (size_t)chain * a.scr_chain;
    float* scr_e = scr;                                        // e - P, NP per step
    float* scr_k = scr_e + (size_t)a.G * NP;                   // key checkpoints, NP DK each
    const float* rlog = a.rlog + (size_t)chain * a.T * 4 * a.N;                 // this chain's records
    const float* qlog = a.rlog + (size_t)gridDim.x * a.T * 4 * a.N + (size_t)chain * a.T;
    auto tok = [&](int t) { return ((size_t)b * a.T + t) * a.H + h; };
    const size_t tok0 = tok(0);
    // lane byte offsets: in a token row, and of row nbase in (rows, DK) / (rows, DV) fp32 slabs
    const uint32_t tk_off = (uint32_t)(dl * DPK * sizeof(TI)), tv_off = (uint32_t)(dl * DPV * sizeof(TI));
    const uint32_t rk_off = (uint32_t)((nbase * DK + dl * DPK) * 4), rv_off = (uint32_t)((nbase * DV + dl * DPV) * 4);
    const bool full = a.N == NP;                               // every row of every lane exists
    const int nv = min(max(a.N - nbase, 0), RPL);              // this lane's rows that exist
    // gate and fr through a 64-step window that ends at the current segment's end, so that the next (earlier)
    // segments find their steps in it too: reloaded once per 64 steps (per step where G > 64)
    const int32_t* amlog = a.hard ? a.am : nullptr;
    StepPar sp = load_steppar(a.gate, a.fr, a.frt, amlog, a.T, a.H, tok0, max(a.T - 64, 0), lane);
    auto steppar = [&](int t, float& g, float& f) {
        if (t < sp.base || t >= sp.base + 64) sp = load_steppar(a.gate, a.fr, a.frt, amlog, a.T, a.H, tok0, max(t - 63, 0), lane);
        g = steppar_g(sp, t);
        f = steppar_f(sp, t);
    };
    // the key (which = 0) or query (1) token row of segment step s (at t), this lane's dims, as fp32
    auto tokrow = [&](int which, int s, int t, float* x) {
        if (s < GL) {
            RawTok<TI, DPK> r;
            r.load(ltq + (s * 2 + which) * TU, (uint32_t)(dl * DPK * sizeof(TI)));
            r.cvt(x);
        } else {
            const TI* p = static_cast<const TI*>(which ? a.q : a.k);
            ldtok<TI, DPK>(p + tok(t) * DK + dl * DPK, x);
        }
    };
    float* dvr = sD + nbase * DV + dl * DPV;
    float dK[RPL][DPK], dO[RPL];
#pragma unroll
    for (int j = 0; j < RPL; j++) {
#pragma unroll
        for (int i = 0; i < DPK; i++) dK[j][i] = 0.f;
#pragma unroll
        for (int i = 0; i < DPV; i += 4) *reinterpret_cast<float4*>(dvr + j * DV + i) = make_float4(0.f, 0.f, 0.f, 0.f);
        dO[j] = 0.f;
    }
    float dfr_acc = 0.f, dtemp_acc = 0.f;     // wave 1, every lane the same
    int pend_t = -1;                          // the walk step whose dq/dfr/dtemp partials are in p2
    float pend_qinv = 0.f;                    // and its 1 / max(|q|, 1e-6)
    int par = 0;                              // exchange-slot parity, flipped once per barrier

    // Wave 1 finishes a walk step (segment step ps) from the p2 posts: dq_t, dfr_t (per token) and the
    // dfr/dtemp sums.
    auto finish_q = [&](int t, int ps, float qinv, const float* q2) {
        if (w != 1) return;
        const size_t ti = tok(t);
        float qt[DPK];
        tokrow(1, ps, t, qt);
        float dqn[DPK];
#pragma unroll
        for (int i = 0; i < DPK; i++) dqn[i] = 0.f;
        float sfo = 0.f, sds = 0.f;
#pragma unroll
        for (int u = 0; u < 2; u++) {           // row-lane rl sums waves 2 rl, 2 rl + 1; then over the 4 rows
            const int ww = 2 * rl + u;
#pragma unroll
            for (int i = 0; i < DPK; i += 4) {
                const float4 f = *reinterpret_cast<const float4*>(q2 + ww * P2W + dl * DPK + i);
                dqn[i] += f.x; dqn[i + 1] += f.y; dqn[i + 2] += f.z; dqn[i + 3] += f.w;
            }
            sfo += q2[ww * P2W + DK];
            sds += q2[ww * P2W + DK + 1];
        }
#pragma unroll
        for (int i = 0; i < DPK; i++) dqn[i] = rows4_sum(dqn[i]);
        sfo = rows4_sum(sfo);
        sds = rows4_sum(sds);
        float pr = 0.f, qq = 0.f;
#pragma unroll
        for (int i = 0; i < DPK; i++) { pr = fmaf(qt[i] * qinv, dqn[i], pr); qq = fmaf(qt[i], qt[i], qq); }
        pr = rowsum16p(pr);
        qq = rowsum16p(qq);
        const bool small = qq < GEN_NORM_EPS * GEN_NORM_EPS;
        if (rl == 0) {
            float r[DPK];
#pragma unroll
            for (int i = 0; i < DPK; i++) r[i] = small ? qinv * dqn[i] : qinv * (dqn[i] - qt[i] * qinv * pr);
#pragma unroll
            for (int i = 0; i < DPK; i += 4)
                sttok4<TI>(dqp + ti * DK + dl * DPK + i, make_float4(r[i], r[i + 1], r[i + 2], r[i + 3]));
        }
        if (a.frt) { if (lane == 0) a.dfr[ti] = -sfo; }
        else dfr_acc -= sfo;
        dtemp_acc += sds / temp;
    };

    for (int tb = a.NB - 1; tb >= 0; tb--) {
        const int t0 = tb * a.G, t1 = min(t0 + a.G, a.T);
        const int ns = min(t1 - t0, GL);
        if (t0 < sp.base) sp = load_steppar(a.gate, a.fr, a.frt, amlog, a.T, a.H, tok0, max(t1 - 64, 0), lane);
        // ---- the segment's logged row scalars (o, a_s, s, |K|), qinv, and key and query token rows of its
        // first GL steps into LDS.  Direct global -> LDS loads where the layouts allow (no data registers: the
        // dK state is live here), waited for explicitly before the barrier.
        {
            const float* rec = rlog + (size_t)t0 * 4 * a.N;
            if (full) {                       // a step's record (4 N floats) is N / 64 KB pieces, contiguous in lsc
                const int pps = a.N / 64;
                for (int k = w; k < ns * pps; k += GEN_WAVES) {
                    const int st = k / pps, pc = k - st * pps;
                    dma16((const char*)(rec + (size_t)st * 4 * a.N) + pc * 1024 + lane * 16,
                          lds_addr(lsc + st * 5 * NP) + pc * 1024);
                }
            } else {
                for (int x = threadIdx.x; x < ns * 4 * NP; x += GEN_THREADS) {
                    const int st = x / (4 * NP), r = x - st * 4 * NP, f = r / NP, n = r - f * NP;
                    lsc[(st * 5 + f) * NP + n] = n < a.N ? rec[((size_t)st * 4 + f) * a.N + n] : 0.f;
                }
            }
            if (threadIdx.x < ns) lqinv[threadIdx.x] = qlog[t0 + threadIdx.x];
            {                                 // token rows (st, key / query): 1 KB of them per load instruction
                constexpr int LPR = DK * (int)sizeof(TI) / 16;        // lanes per token row
                constexpr int RPI = 64 / LPR;                          // rows per instruction
                for (int k = w; k * RPI < 2 * ns; k += GEN_WAVES) {
                    const int row = k * RPI + lane / LPR, st = row >> 1;
                    const char* g = (const char*)((row & 1) ? a.q : a.k) + tok(t0 + st) * DK * sizeof(TI) + (lane % LPR) * 16;
                    if (row < 2 * ns) dma16(g, lds_addr(ltq) + k * 1024);
                }
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __syncthreads();                      // the replay reads the logged addresses of every row group
        // ---- replay the segment's keys from its emitted copy, keeping every step's pre-write state
        {
            // The value state itself is not replayed: inside a segment the value adjoint only scales,
            // dV(t+) = c(t) D with D the adjoint entering the segment, so the walk needs just the row
            // scalars P(t) = <V(t), D> (P <- (1-w) P + w e from the emitted copy) and e(t) = <v_t, D>.
            // The addresses come from the forward's log, so a step needs no exchange between the waves.
            // The next step's value row is loaded once this step's stores are issued.
            const size_t slab = (((size_t)b * a.NB + tb) * a.H + h) * a.N;
            float K[RPL][DPK], P[RPL];
            ld_rows<RPL, DPK>(K, a.kbuf + slab * DK, rk_off, full, nv);
            {
                float Vs[RPL][DPV];
                ld_rows<RPL, DPV>(Vs, a.vbuf + slab * DV, rv_off, full, nv);
#pragma unroll
                for (int j = 0; j < RPL; j++) {
                    float x = 0.f;
#pragma unroll
                    for (int i = 0; i < DPV; i += 4) {
                        const float4 d = *reinterpret_cast<const float4*>(dvr + j * DV + i);
                        x = fmaf(Vs[j][i], d.x, x); x = fmaf(Vs[j][i + 1], d.y, x);
                        x = fmaf(Vs[j][i + 2], d.z, x); x = fmaf(Vs[j][i + 3], d.w, x);
                    }
                    P[j] = rowsum16p(x);
                }
            }
            RawTok<TI, DPV> rv;
            rv.load((const char*)a.v + tok(t0) * DV * sizeof(TI), tv_off);
            for (int t = t0; t < t1; t++) {
                // lane indices from an opaque copy every step: comparisons on them are then not loop invariant, so
                // the compiler does not hoist the per-row and per-lane masks into (spilled) scalar registers
                uint32_t tido;
                asm volatile("v_mov_b32 %0, %1" : "=v"(tido) : "v"((uint32_t)threadIdx.x));
                const int lane_s = (int)(tido & 63u), dl_s = lane_s & 15, rl_s = lane_s >> 4;
                const int nb_s = w * RPW + rl_s * RPL;
                const int s = t - t0;
                float vt[DPV];
                rv.cvt(vt);
                if (s > 0 && s % SC::GC == 0) {             // a key checkpoint
                    char* sk = (char*)(scr_k + (size_t)(s / SC::GC - 1) * NP * DK) + rk_off;
#pragma unroll
                    for (int j = 0; j < RPL; j++)
#pragma unroll
                        for (int i = 0; i < DPK; i += 4)
                            *reinterpret_cast<float4*>(sk + (j * DK + i) * 4) = make_float4(K[j][i], K[j][i + 1], K[j][i + 2], K[j][i + 3]);
                }
                if (t + 1 < t1) rv.load((const char*)a.v + tok(t + 1) * DV * sizeof(TI), tv_off);
                float kt[DPK];
                tokrow(0, s, t, kt);
                float g, frt;
                steppar(t, g, frt);
                float ad[RPL];                                  // the write address (pre-gate)
                if (a.hard) {
                    const int amt = steppar_am(sp, t);
#pragma unroll
                    for (int j = 0; j < RPL; j++) ad[j] = nb_s + j == amt ? 1.f : 0.f;
                } else if (s < GL) {
#pragma unroll
                    for (int j = 0; j < RPL; j++) ad[j] = lsc[(s * 5 + 1) * NP + nb_s + j];
                } else {
#pragma unroll
                    for (int j = 0; j < RPL; j++) ad[j] = nb_s + j < a.N ? rlog[((size_t)t * 4 + 1) * a.N + nb_s + j] : 0.f;
                }
                float e[RPL];
#pragma unroll
                for (int j = 0; j < RPL; j++) {
                    float x = 0.f;
#pragma unroll
                    for (int i = 0; i < DPV; i += 4) {
                        const float4 d = *reinterpret_cast<const float4*>(dvr + j * DV + i);
                        x = fmaf(vt[i], d.x, x); x = fmaf(vt[i + 1], d.y, x);
                        x = fmaf(vt[i + 2], d.z, x); x = fmaf(vt[i + 3], d.w, x);
                    }
                    e[j] = rowsum16p(x);
                }
                if (dl_s == 0) {
#pragma unroll
                    for (int j = 0; j < RPL; j++) {
                        const int n = nb_s + j;
                        // explicit branches (s is uniform): a select between the LDS and the global pointer
                        // would make every access a flat one, which waits on both counters
                        if (s < GL) lsc[(s * 5 + 4) * NP + n] = e[j] - P[j];
                        else scr_e[(size_t)s * NP + n] = e[j] - P[j];
                    }
                }
#pragma unroll
                for (int j = 0; j < RPL; j++) {
                    const float wr = g * ad[j];
                    const float omw = 1.f - wr;
#pragma unroll
                    for (int i = 0; i < DPK; i++) fma_in(K[j][i], omw, wr * kt[i]);
                    fma_in(P[j], omw, wr * e[j]);
                }
            }
        }
        __syncthreads();                      // the replay's scratch is visible to every wave
        // ---- walk the segment backward
        float cV[RPL];                        // dV(t+) = cV D: the product of (1 - w) over the steps walked
#pragma unroll
        for (int j = 0; j < RPL; j++) cV[j] = 1.f;
        for (int t = t1 - 1; t >= t0; t--) {
            // lane indices from an opaque copy every step: comparisons on them are then not loop invariant, so
            // the compiler does not hoist the per-row and per-lane masks into (spilled) scalar registers
            uint32_t tido;
            asm volatile("v_mov_b32 %0, %1" : "=v"(tido) : "v"((uint32_t)threadIdx.x));
            const int lane_s = (int)(tido & 63u), dl_s = lane_s & 15, rl_s = lane_s >> 4;
            const int nb_s = w * RPW + rl_s * RPL;
            const int s = t - t0;
            const size_t ti = tok(t);
            // The pre-write keys of step s: the checkpoint at or before it, then the replay's updates of the
            // steps in between.  Built once per step and held across the step's barrier (with the addresses
            // held as scalar bases and lane_s offsets there is room for them; rebuilding them after the barrier
            // cost more).
            auto load_K = [&](float (&K)[RPL][DPK]) {
                const int c = (s / SC::GC) * SC::GC;
                if (c == 0) ld_rows<RPL, DPK>(K, a.kbuf + ((((size_t)b * a.NB + tb) * a.H + h) * a.N) * DK, rk_off, full, nv);
                else ld_rows<RPL, DPK>(K, scr_k + (size_t)(c / SC::GC - 1) * NP * DK, rk_off, true, RPL);
                // at most GC - 1 updates, unrolled with a uniform test: a rolled loop rotated the 8 RPL key
                // registers through copies at every iteration
#pragma unroll
                for (int uu = 0; uu < SC::GC - 1; uu++) {
                    const int u = c + uu;
                    if (u >= s) break;
                    float ku[DPK];
                    tokrow(0, u, t0 + u, ku);
                    const float gu = steppar_g(sp, t0 + u);
                    const int amu = a.hard ? steppar_am(sp, t0 + u) : -1;
                    float asu[RPL];                                 // a_s of step u
                    if (u < GL) {
#pragma unroll
                        for (int j = 0; j < RPL; j++) asu[j] = lsc[(u * 5 + 1) * NP + nb_s + j];
                    } else {
#pragma unroll
                        for (int j = 0; j < RPL; j++)
                            asu[j] = nb_s + j < a.N ? rlog[((size_t)(t0 + u) * 4 + 1) * a.N + nb_s + j] : 0.f;
                    }
#pragma unroll
                    for (int j = 0; j < RPL; j++) {
                        const float adu = a.hard ? (nb_s + j == amu ? 1.f : 0.f) : asu[j];
                        const float wr = gu * adu;
                        const float omw = 1.f - wr;
#pragma unroll
                        for (int i = 0; i < DPK; i++) fma_in(K[j][i], omw, wr * ku[i]);
                    }
                }
            };
            // the row scalars: read where they are used, on each side of the barrier
            auto load_s = [&](float (&x)[RPL], int f) {
                if (s < GL) {
#pragma unroll
                    for (int j = 0; j < RPL; j++) x[j] = lsc[(s * 5 + f) * NP + nb_s + j];
                } else if (f < 4) {                            // logged by the forward
#pragma unroll
                    for (int j = 0; j < RPL; j++)
                        x[j] = nb_s + j < a.N ? rlog[((size_t)t * 4 + f) * a.N + nb_s + j] : 0.f;
                } else {
#pragma unroll
                    for (int j = 0; j < RPL; j++) x[j] = scr_e[(size_t)s * NP + nb_s + j];
                }
            };
            float kt[DPK];
            tokrow(0, s, t, kt);
            float g, frt;
            steppar(t, g, frt);
            float qinv;
            if (s < GL) qinv = lqinv[s];
            else qinv = qlog[t];

            // dw per row; dk_t, dv_t partials; the two address sums
            float dw[RPL], wr[RPL];
            float pg = 0.f, pa = 0.f;
            float K[RPL][DPK];
            load_K(K);
            {
            float o[RPL], as[RPL], ad[RPL], ep[RPL];
            load_s(o, 0); load_s(as, 1); load_s(ep, 4);
            {
                const int amt = a.hard ? steppar_am(sp, t) : -1;
#pragma unroll
                for (int j = 0; j < RPL; j++) ad[j] = a.hard ? (nb_s + j == amt ? 1.f : 0.f) : as[j];
            }
#pragma unroll
            for (int j = 0; j < RPL; j++) {
                float x = 0.f;
#pragma unroll
                for (int i = 0; i < DPK; i++) x = fmaf(kt[i] - K[j][i], dK[j][i], x);
                x = rowsum16p(x);
                x = fmaf(cV[j], ep[j], x);              // <v_t - V(t), dV(t+)> = cV (e - P)
                dw[j] = fmaf(1.f - o[j], dO[j], x);
                wr[j] = g * ad[j];
                pg = fmaf(ad[j], dw[j], pg);
                pa = fmaf(as[j], g * dw[j], pa);
            }
            }
            pg = rows4_sum(pg);
            pa = rows4_sum(pa);
            float* q1 = p1[par];
            {   // the wave's dk, dv partials: summed over its rows, reduce-scattered over the row-lanes
                float pk[DPK], pv[DPV];
#pragma unroll
                for (int i = 0; i < DPK; i++) {
                    float x = 0.f;
#pragma unroll
                    for (int j = 0; j < RPL; j++) x = fmaf(wr[j], dK[j][i], x);
                    pk[i] = x;
                }
#pragma unroll
                for (int i = 0; i < DPV; i += 4) {             // dV(t+) = cV D
                    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                    for (int j = 0; j < RPL; j++) {
                        const float c = wr[j] * cV[j];
                        const float4 d = *reinterpret_cast<const float4*>(dvr + j * DV + i);
                        x.x = fmaf(c, d.x, x.x); x.y = fmaf(c, d.y, x.y); x.z = fmaf(c, d.z, x.z); x.w = fmaf(c, d.w, x.w);
                    }
                    pv[i] = x.x; pv[i + 1] = x.y; pv[i + 2] = x.z; pv[i + 3] = x.w;
                }
                float yk[DPK / 4], yv[DPV / 4];
                rows4_rs<DPK>(pk, yk);
                rows4_rs<DPV>(pv, yv);
                float* ok = q1 + w * P1W + dl_s * DPK + rows4_rs_base<DPK>(rl_s);
                float* ov = q1 + w * P1W + DK + dl_s * DPV + rows4_rs_base<DPV>(rl_s);
#pragma unroll
                for (int i = 0; i < DPK / 4; i++) ok[i] = yk[i];
#pragma unroll
                for (int i = 0; i < DPV / 4; i++) ov[i] = yv[i];
                if (lane_s == 0) { q1[w * P1W + DK + DV] = pg; q1[w * P1W + DK + DV + 1] = pa; }
            }
            lds_barrier();
            if (pend_t >= 0) finish_q(pend_t, pend_t - t0, pend_qinv, p2[par ^ 1]);
            float SG, SA;
            {                                 // the 8 waves' {sum a dw, sum a_s g dw}: lane l holds wave l & 7's
                const float2 gp = *reinterpret_cast<const float2*>(q1 + (lane & 7) * P1W + DK + DV);
                float sg = gp.x, sa = gp.y;
                sg += dppf<SLOT_DPP_XOR1>(sg); sa += dppf<SLOT_DPP_XOR1>(sa);
                sg += dppf<SLOT_DPP_XOR2>(sg); sa += dppf<SLOT_DPP_XOR2>(sa);
                sg += dppf<SLOT_DPP_HMIR>(sg); sa += dppf<SLOT_DPP_HMIR>(sa);
                SG = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sg)));
                SA = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sa)));
            }
            if (w == 0) {                     // dk_t, dv_t and dgate_t
                constexpr int CK = DK / 4, CV = DV / 4;
                if (lane_s < CK + CV) {
                    const int off = lane_s < CK ? 4 * lane_s : DK + 4 * (lane_s - CK);
                    float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                    for (int ww = 0; ww < GEN_WAVES; ww++) {
                        const float4 f = *reinterpret_cast<const float4*>(q1 + ww * P1W + off);
                        r.x += f.x; r.y += f.y; r.z += f.z; r.w += f.w;
                    }
                    if (lane_s < CK) sttok4<TI>(dkp + ti * DK + off, r);
                    else sttok4<TI>(dvp + ti * DV + (off - DK), r);
                }
                if (lane_s == 0) a.dg[ti] = SG;
            }
            // dz and the search-side partials
            float o[RPL], as[RPL], sr[RPL], knr[RPL], qt[DPK];
            load_s(o, 0); load_s(as, 1); load_s(sr, 2); load_s(knr, 3);
            tokrow(1, s, t, qt);
            float dz[RPL], ds[RPL], kinv[RPL];      // ds: dz with the pinned rows' score path cut
            float sfo = 0.f, sds = 0.f;
#pragma unroll
            for (int j = 0; j < RPL; j++) {
                dz[j] = as[j] * (g * dw[j] - SA);
                ds[j] = (a.pin && knr[j] < GEN_NORM_EPS) ? 0.f : dz[j];
                kinv[j] = __builtin_amdgcn_rcpf(fmaxf(knr[j], GEN_NORM_EPS));
                const float occ = a.occ_bin ? (o[j] >= a.eps ? 1.f : 0.f) : o[j];
                sfo = fmaf(occ, dz[j], sfo);
                sds = fmaf(ds[j], sr[j], sds);
            }
            sfo = rows4_sum(sfo);
            sds = rows4_sum(sds);
            float* q2 = p2[par];
            {   // the wave's dqn partial, reduce-scattered over the row-lanes
                float pq[DPK];
#pragma unroll
                for (int i = 0; i < DPK; i++) {
                    float x = 0.f;
#pragma unroll
                    for (int j = 0; j < RPL; j++) x = fmaf(ds[j] * kinv[j], K[j][i], x);
                    pq[i] = temp * x;
                }
                float yq[DPK / 4];
                rows4_rs<DPK>(pq, yq);
                float* oq = q2 + w * P2W + dl_s * DPK + rows4_rs_base<DPK>(rl_s);
#pragma unroll
                for (int i = 0; i < DPK / 4; i++) oq[i] = yq[i];
                if (lane_s == 0) { q2[w * P2W + DK] = sfo; q2[w * P2W + DK + 1] = sds; }
            }
            pend_t = t;
            pend_qinv = qinv;
            par ^= 1;
            // carry to the pre-write adjoint; attached: dK += c (temp qn - s kinv K), c = ds kinv (the second
            // term dropped where |K| < 1e-6)
            float tq[DPK];
#pragma unroll
            for (int i = 0; i < DPK; i++) tq[i] = temp * (qt[i] * qinv);
#pragma unroll
            for (int j = 0; j < RPL; j++) {
                const float omw = 1.f - wr[j];
                if (!a.detach) {
                    const float c = ds[j] * kinv[j];
                    const float cs = knr[j] < GEN_NORM_EPS ? 0.f : c * (sr[j] * kinv[j]);
#pragma unroll
                    for (int i = 0; i < DPK; i++) dK[j][i] = fmaf(-cs, K[j][i], fmaf(c, tq[i], omw * dK[j][i]));
                } else {
#pragma unroll
                    for (int i = 0; i < DPK; i++) dK[j][i] *= omw;
                }
                cV[j] *= omw;
                dO[j] = a.occ_bin ? omw * dO[j] : fmaf(omw, dO[j], -frt * dz[j]);
            }
            if (t == t0) {                    // the emitted copy's gradient enters at the segment's first step
                const size_t slab = (((size_t)b * a.NB + tb) * a.H + h) * a.N;
                float X[RPL][DPK];
                ld_rows<RPL, DPK>(X, a.dkbuf + slab * DK, rk_off, full, nv);
#pragma unroll
                for (int j = 0; j < RPL; j++)
#pragma unroll
                    for (int i = 0; i < DPK; i++) dK[j][i] += X[j][i];
                float Y[RPL][DPV];
                ld_rows<RPL, DPV>(Y, a.dvbuf + slab * DV, rv_off, full, nv);
#pragma unroll
                for (int j = 0; j < RPL; j++) {
#pragma unroll
                    for (int i = 0; i < DPV; i += 4) {      // the next segment's D = cV D + dvbuf
                        float4* d = reinterpret_cast<float4*>(dvr + j * DV + i);
                        const float4 x = *d;
                        *d = make_float4(fmaf(cV[j], x.x, Y[j][i]), fmaf(cV[j], x.y, Y[j][i + 1]),
                                         fmaf(cV[j], x.z, Y[j][i + 2]), fmaf(cV[j], x.w, Y[j][i + 3]));
                    }
                }
            }
        }
        __syncthreads();                      // the last walk step's posts are visible
        if (pend_t >= 0) { finish_q(pend_t, pend_t - t0, pend_qinv, p2[par ^ 1]); pend_t = -1; }
        __syncthreads();                      // every read of this segment's LDS data is done before the next
                                              // segment's staging overwrites it
    }
    if (w == 1 && lane == 0) {
        a.part[2 * chain] = dfr_acc;
        a.part[2 * chain + 1] = dtemp_acc;
    }
}

// dfr (scalar fr) and dtemp: the sums of the per-chain partials, in a fixed order.
__global__ __launch_bounds__(256) void gen_reduce(const float* part, int chains, int frt, float* dfr, float* dtemp) {
    __shared__ float sh[2][4];
    float x = 0.f, y = 0.f;
    for (int c = threadIdx.x; c < chains; c += 256) { x += part[2 * c]; y += part[2 * c + 1]; }
    x = wavesum(x);
    y = wavesum(y);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sh[0][w] = x; sh[1][w] = y; }
    __syncthreads();
    if (threadIdx.x == 0) {
        if (!frt) dfr[0] = sh[0][0] + sh[0][1] + sh[0][2] + sh[0][3];
        dtemp[0] = sh[1][0] + sh[1][1] + sh[1][2] + sh[1][3];
    }
}

static int gen_rpl(int64_t N) { return N <= 64 ? 2 : (N <= 128 ? 4 : 6); }

template <typename TI, int DK, int DV>
static void launch_fwd(int rpl, dim3 grid, hipStream_t st, const GenArgs& a) {
    if (rpl == 2) slothost::launch(gen_fwd<TI, DK, DV, 2>, grid, dim3(GEN_THREADS), 0, st, a);
    else if (rpl == 4) slothost::launch(gen_fwd<TI, DK, DV, 4>, grid, dim3(GEN_THREADS), 0, st, a);
    else slothost::launch(gen_fwd<TI, DK, DV, 6>, grid, dim3(GEN_THREADS), 0, st, a);
}
template <typename TI, int DK, int DV>
static void launch_bwd(int rpl, dim3 grid, hipStream_t st, const GenArgs& a) {
    if (rpl == 2) slothost::launch(gen_bwd<TI, DK, DV, 2>, grid, dim3(GEN_THREADS), 0, st, a);
    else if (rpl == 4) slothost::launch(gen_bwd<TI, DK, DV, 4>, grid, dim3(GEN_THREADS), 0, st, a);
    else slothost::launch(gen_bwd<TI, DK, DV, 6>, grid, dim3(GEN_THREADS), 0, st, a);
}
template <typename TI>
static void dispatch(bool bwd, int64_t DK, int64_t DV, int rpl, dim3 grid, hipStream_t st, const GenArgs& a) {
    if (DK == 64 && DV == 64) (bwd ? launch_bwd<TI, 64, 64> : launch_fwd<TI, 64, 64>)(rpl, grid, st, a);
    else if (DK == 64) (bwd ? launch_bwd<TI, 64, 128> : launch_fwd<TI, 64, 128>)(rpl, grid, st, a);
    else if (DV == 64) (bwd ? launch_bwd<TI, 128, 64> : launch_fwd<TI, 128, 64>)(rpl, grid, st, a);
    else (bwd ? launch_bwd<TI, 128, 128> : launch_fwd<TI, 128, 128>)(rpl, grid, st, a);
}

static int64_t scr_chain(int64_t DK, int64_t DV, int rpl, int64_t G) {
    const int64_t NP = 32 * rpl;
    (void)DV;
    return G * NP + ((G - 1) / 4) * NP * DK;                           // GenScr<...>::chain
}

}  // namespace

// ======================================================================================== C-ABI
static int check_gen(int64_t B, int64_t T, int64_t H, int64_t N, int64_t DK, int64_t DV, int64_t G, int dtype) {
    if (B < 1 || T < 1 || H < 1 || N < 1 || G < 1) return fail(SLOTSCAN_ERR_SHAPE, "slotscan_gen: B, T, H, N and G must be >= 1");
    if ((DK != 64 && DK != 128) || (DV != 64 && DV != 128))
        return fail(SLOTSCAN_ERR_SHAPE, "slotscan_gen: DK and DV must each be 64 or 128");
    if (N > SLOTSCAN_MAX_SLOTS) return fail(SLOTSCAN_ERR_SHAPE, "slotscan_gen: N exceeds SLOTSCAN_MAX_SLOTS (192)");
    if (dtype != SLOTSCAN_F32 && dtype != SLOTSCAN_BF16) return fail(SLOTSCAN_ERR_DTYPE, "token dtype must be f32 or bf16");
    if (B * H > 0x7fffffffLL || T > 0x7fffffffLL || G > 0x7fffffffLL)
        return fail(SLOTSCAN_ERR_SHAPE, "slotscan_gen: B*H and T must fit in int32");
    return 0;
}

extern "C" int slotscan_gen_fwd(const void* k, const void* q, const void* v, int dtype, const float* gate,
                                const float* fr, int fr_per_token, const float* temp, int64_t B, int64_t T,
                                int64_t H, int64_t N, int64_t DK, int64_t DV, int64_t G, float eps, int occ_bin,
                                int hard, int pin, float* kbuf, float* vbuf, float* obuf, int32_t* am, float* wb,
                                float* rlog, void* stream) {
    if (int r = check_gen(B, T, H, N, DK, DV, G, dtype)) return r;
    if (!k || !q || !v || !gate || !fr || !temp || !kbuf || !vbuf || !obuf || (hard && !am))
        return fail(SLOTSCAN_ERR_NULL, "slotscan_gen_fwd: a required pointer is NULL");
    if (!al16(k) || !al16(q) || !al16(v) || !al16(kbuf) || !al16(vbuf) || !al16(rlog))
        return fail(SLOTSCAN_ERR_ALIGN, "slotscan_gen_fwd: k, q, v, kbuf, vbuf, rlog must be 16-byte aligned");
    GenArgs a{};
    a.k = k; a.q = q; a.v = v; a.gate = gate; a.fr = fr; a.temp = temp;
    a.frt = fr_per_token != 0; a.T = (int)T; a.H = (int)H; a.N = (int)N; a.G = (int)G;
    a.NB = (int)((T + G - 1) / G); a.occ_bin = occ_bin != 0; a.hard = hard != 0; a.detach = 1; a.eps = eps;
    a.pin = pin != 0;
    a.kbuf = kbuf; a.vbuf = vbuf; a.obuf = obuf; a.am = am; a.wb = wb; a.rlog = rlog;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)(B * H));
    hipError_t e;
    {
        slothost::Scope sc(SLOTSCAN_K_GEN_FWD, st);
        if (dtype == SLOTSCAN_BF16) dispatch<bf16_t>(false, DK, DV, gen_rpl(N), grid, st, a);
        else dispatch<float>(false, DK, DV, gen_rpl(N), grid, st, a);
        e = hipGetLastError();
    }
    return e == hipSuccess ? 0 : hip_fail(e, "gen_fwd launch");
}

extern "C" size_t slotscan_gen_log_bytes(int64_t B, int64_t T, int64_t H, int64_t N) {
    if (B < 1 || T < 1 || H < 1 || N < 1) return 0;
    return gen_log_floats(B * H, T, N) * sizeof(float);
}

extern "C" size_t slotscan_gen_bwd_workspace(int64_t B, int64_t H, int64_t N, int64_t DK, int64_t DV, int64_t G) {
    const int64_t per = scr_chain(DK, DV, gen_rpl(N), G);
    const size_t scr = (size_t)B * H * per * sizeof(float);
    return ((scr + 255) & ~(size_t)255) + (size_t)B * H * 2 * sizeof(float);
}

extern "C" int slotscan_gen_bwd(const void* k, const void* q, const void* v, int dtype, const float* gate,
                                const float* fr, int fr_per_token, const float* temp, int64_t B, int64_t T,
                                int64_t H, int64_t N, int64_t DK, int64_t DV, int64_t G, float eps, int occ_bin,
                                int hard, int detach_addr, int pin, const float* kbuf, const float* vbuf,
                                const float* obuf, const int32_t* am, const float* rlog, const float* dkbuf,
                                const float* dvbuf, void* workspace, void* dk, void* dq, void* dv, float* dgate,
                                float* dfr, float* dtemp, void* stream) {
    if (int r = check_gen(B, T, H, N, DK, DV, G, dtype)) return r;
    if (!k || !q || !v || !gate || !fr || !temp || !kbuf || !vbuf || !obuf || (hard && !am) || !rlog || !dkbuf ||
        !dvbuf || !workspace || !dk || !dq || !dv || !dgate || !dfr || !dtemp)
        return fail(SLOTSCAN_ERR_NULL, "slotscan_gen_bwd: a required pointer is NULL");
    if (!al16(k) || !al16(q) || !al16(v) || !al16(kbuf) || !al16(vbuf) || !al16(dkbuf) || !al16(dvbuf) ||
        !al16(workspace) || ((uintptr_t)dk & 7u) || ((uintptr_t)dq & 7u) || ((uintptr_t)dv & 7u))
        return fail(SLOTSCAN_ERR_ALIGN, "slotscan_gen_bwd: 16-byte aligned inputs and workspace, 8-byte aligned dk, dq, dv");
    const int rpl = gen_rpl(N);
    GenArgs a{};
    a.k = k; a.q = q; a.v = v; a.gate = gate; a.fr = fr; a.temp = temp;
    a.frt = fr_per_token != 0; a.T = (int)T; a.H = (int)H; a.N = (int)N; a.G = (int)G;
    a.NB = (int)((T + G - 1) / G); a.occ_bin = occ_bin != 0; a.hard = hard != 0; a.detach = detach_addr != 0;
    a.eps = eps; a.pin = pin != 0;
    a.kbuf = const_cast<float*>(kbuf); a.vbuf = const_cast<float*>(vbuf); a.obuf = const_cast<float*>(obuf);
    a.am = const_cast<int32_t*>(am); a.rlog = const_cast<float*>(rlog); a.dkbuf = dkbuf; a.dvbuf = dvbuf;
    a.scr = (float*)workspace; a.scr_chain = scr_chain(DK, DV, rpl, G);
    const size_t scr = (size_t)B * H * a.scr_chain * sizeof(float);
    a.part = (float*)((char*)workspace + ((scr + 255) & ~(size_t)255));
    a.dk = dk; a.dq = dq; a.dv = dv; a.dg = dgate; a.dfr = dfr;
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    {
        slothost::Scope sc(SLOTSCAN_K_GEN_BWD, st);
        if (dtype == SLOTSCAN_BF16) dispatch<bf16_t>(true, DK, DV, rpl, dim3((unsigned)(B * H)), st, a);
        else dispatch<float>(true, DK, DV, rpl, dim3((unsigned)(B * H)), st, a);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return hip_fail(e, "gen_bwd launch");
    {
        slothost::Scope sc(SLOTSCAN_K_REDUCE, st);
        slothost::launch(gen_reduce, dim3(1), dim3(256), 0, st, (const float*)a.part, (int)(B * H),
                         (int)a.frt, dfr, dtemp);
        e = hipGetLastError();
    }
    return e == hipSuccess ? 0 : hip_fail(e, "gen_reduce launch");
}
