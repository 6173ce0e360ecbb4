// Writer epilogue and storage quantiser of the shared slot memory, for MI355X (gfx950).
//
// Semantics (reference: /root/reference/gqa25/memlm_sh.py).  The scan emits fp32 snapshot copies kbuf, vbuf
// (rows of D channels).  The writer turns them into what the readers see:
//   full precision (memlm_sh.py:474-475): nsq = sum K^2, kinv = rsqrt(max(nsq, 1e-12)), valid = nsq > 1e-12,
//                                          copies cast to the activation dtype;
//   quantised (memlm_sh.py:221-234, 468-471): per group of `group` channels, a = absmax, s = max(a / 2^(b-1),
//       1e-30), q = (clamp(floor(x / s), -2^(b-1), 2^(b-1) - 1) + 0.5) s, q = 0 where a == 0; the returned
//       value is the straight-through x + (q - x); kinv / valid from the quantised keys.
// Backward (autograd of the same expressions): d kbuf = d kout + 2 K dnsq with dnsq = -0.5 kinv^3 dkinv
// where nsq >= 1e-12 (the clamp passes the gradient there), d vbuf = d vout; the quantiser is the identity
// (straight-through).
// Storage codes (config 5's int8 + per-row scale is b = 8, group = D): code = clamp(floor(x / s), ...),
// scale = s, or 0 for an all-zero group so that (code + 0.5) * scale decodes it to exactly 0.
//
// Mapping: a row of D fp32 channels is owned by D/8 consecutive lanes (8 channels = two 16-byte loads per
// lane), so a wave streams 8 (D=64) or 4 (D=128) rows per instruction, fully coalesced.  Group maxima and
// the row norm are DPP reductions inside the lane group; the kernels are pure HBM streams.
#include "slot_common.h"
#include "slotscan.h"
#include "slotmem.h"
#include "slot_host.h"

using namespace slot;
using slothost::fail;
using slothost::hip_fail;
using slothost::al16;

#define MEM_THREADS 256

namespace {

struct MemFwdArgs {
    const float* kb;
    const float* vb;
    void* kout;
    void* vout;
    float* kinv;
    uint8_t* valid;
    int64_t rows;
    int bits, group;
};

struct MemBwdArgs {
    const float* kb;
    const void* dkout;
    const void* dvout;
    const float* dkinv;
    float* dkb;
    float* dvb;
    int64_t rows;
    int bits, group;
};

struct MemCodeArgs {
    const float* x;
    int8_t* codes;
    float* scales;
    int64_t rows;
    int bits, group;
};

// max over the `lanes` consecutive lanes of a group (lanes in {1, 2, 4, 8, 16}); every lane gets the result
__device__ __forceinline__ float group_max(float v, int lanes) {
    if (lanes >= 2) v = fmaxf(v, dppf<SLOT_DPP_XOR1>(v));
    if (lanes >= 4) v = fmaxf(v, dppf<SLOT_DPP_XOR2>(v));
    if (lanes >= 8) v = fmaxf(v, dppf<SLOT_DPP_HMIR>(v));
    if (lanes >= 16) v = fmaxf(v, dppf<SLOT_DPP_MIR>(v));
    return v;
}
// sum over the LPR lanes of a row (LPR in {8, 16})
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
    v += dppf<SLOT_DPP_XOR1>(v);
    v += dppf<SLOT_DPP_XOR2>(v);
    v += dppf<SLOT_DPP_HMIR>(v);
    if constexpr (LPR == 16) v += dppf<SLOT_DPP_MIR>(v);
    return v;
}

__device__ __forceinline__ void load8(const float* p, float* x) {
    const float4 a = ld4(p), b = ld4(p + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

// the quantiser over this lane's 8 channels; a group spans group/8 lanes (group >= 8) or part of the 8
// (group 4: two groups per lane).  Returns the straight-through value x + (q - x); code / scale optional.
__device__ __forceinline__ void quantise8(float* x, int bits, int group, int8_t* code, float* scale2) {
    const float half = (float)(1 << (bits - 1));
    float a[2];
    if (group >= 8) {
        float m = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) m = fmaxf(m, fabsf(x[e]));
        a[0] = a[1] = group_max(m, group / 8);
    } else {                                   // group == 4
        float m0 = 0.f, m1 = 0.f;
#pragma unroll
        for (int e = 0; e < 4; e++) { m0 = fmaxf(m0, fabsf(x[e])); m1 = fmaxf(m1, fabsf(x[4 + e])); }
        a[0] = m0; a[1] = m1;
    }
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float ag = a[e >> 2];
        const float s = fmaxf(ag / half, 1e-30f);
        const float c = fminf(fmaxf(floorf(x[e] / s), -half), half - 1.f);
        float q = (c + 0.5f) * s;
        q = ag > 0.f ? q : 0.f;
        if (code) code[e] = (int8_t)c;
        x[e] = x[e] + (q - x[e]);
    }
    if (scale2) {
        const float s0 = fmaxf(a[0] / half, 1e-30f), s1 = fmaxf(a[1] / half, 1e-30f);
        scale2[0] = a[0] > 0.f ? s0 : 0.f;
        scale2[1] = a[1] > 0.f ? s1 : 0.f;
    }
}

template <typename OT>
__device__ __forceinline__ void store8(OT* p, const float* x);
template <>
__device__ __forceinline__ void store8<float>(float* p, const float* x) {
    st4(p, make_float4(x[0], x[1], x[2], x[3]));
    st4(p + 4, make_float4(x[4], x[5], x[6], x[7]));
}
template <>
__device__ __forceinline__ void store8<bf16_t>(bf16_t* p, const float* x) {
    uint4 r;
    r.x = pack_bf16x2(x[0], x[1]); r.y = pack_bf16x2(x[2], x[3]);
    r.z = pack_bf16x2(x[4], x[5]); r.w = pack_bf16x2(x[6], x[7]);
    *reinterpret_cast<uint4*>(p) = r;
}
template <typename OT>
__device__ __forceinline__ void load8g(const OT* p, float* x);
template <>
__device__ __forceinline__ void load8g<float>(const float* p, float* x) { load8(p, x); }
template <>
__device__ __forceinline__ void load8g<bf16_t>(const bf16_t* p, float* x) {
    const uint4 r = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 4; e++) { x[2 * e] = __uint_as_float(w[e] << 16); x[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u); }
}

template <int D, typename OT>
__global__ __launch_bounds__(MEM_THREADS) void mem_epilogue(MemFwdArgs a) {
    constexpr int LPR = D / 8;
    constexpr int RPB = MEM_THREADS / LPR;                   // rows per workgroup pass
    const int lr = threadIdx.x % LPR, rr = threadIdx.x / LPR;
    for (int64_t row = (int64_t)blockIdx.x * RPB + rr; row < a.rows; row += (int64_t)gridDim.x * RPB) {
        const size_t off = (size_t)row * D + lr * 8;
        float k[8], v[8];
        load8(a.kb + off, k);
        load8(a.vb + off, v);
        if (a.bits > 0) {
            quantise8(k, a.bits, a.group, nullptr, nullptr);
            quantise8(v, a.bits, a.group, nullptr, nullptr);
        }
        float sq = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) sq = fmaf(k[e], k[e], sq);
        const float nsq = row_sum<LPR>(sq);
        store8<OT>(reinterpret_cast<OT*>(a.kout) + off, k);
        store8<OT>(reinterpret_cast<OT*>(a.vout) + off, v);
        if (lr == 0) {
            a.kinv[row] = rsqrtf(fmaxf(nsq, 1e-12f));
            a.valid[row] = nsq > 1e-12f ? 1 : 0;
        }
    }
}

template <int D, typename OT>
__global__ __launch_bounds__(MEM_THREADS) void mem_epilogue_bwd(MemBwdArgs a) {
    constexpr int LPR = D / 8;
    constexpr int RPB = MEM_THREADS / LPR;
    const int lr = threadIdx.x % LPR, rr = threadIdx.x / LPR;
    for (int64_t row = (int64_t)blockIdx.x * RPB + rr; row < a.rows; row += (int64_t)gridDim.x * RPB) {
        const size_t off = (size_t)row * D + lr * 8;
        float k[8], gk[8], gv[8];
        load8(a.kb + off, k);
        if (a.bits > 0) quantise8(k, a.bits, a.group, nullptr, nullptr);
        float sq = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) sq = fmaf(k[e], k[e], sq);
        const float nsq = row_sum<LPR>(sq);
        const float ki = rsqrtf(fmaxf(nsq, 1e-12f));
        const float dnsq = nsq >= 1e-12f ? a.dkinv[row] * (ki * ki * ki * -0.5f) : 0.f;
        load8g<OT>(reinterpret_cast<const OT*>(a.dkout) + off, gk);
        load8g<OT>(reinterpret_cast<const OT*>(a.dvout) + off, gv);
#pragma unroll
        for (int e = 0; e < 8; e++) gk[e] = gk[e] + (2.f * k[e]) * dnsq;
        store8<float>(a.dkb + off, gk);
        store8<float>(a.dvb + off, gv);
    }
}

template <int D>
__global__ __launch_bounds__(MEM_THREADS) void mem_codes(MemCodeArgs a) {
    constexpr int LPR = D / 8;
    constexpr int RPB = MEM_THREADS / LPR;
    const int lr = threadIdx.x % LPR, rr = threadIdx.x / LPR;
    const int gpr = D / a.group;                             // groups per row
    for (int64_t row = (int64_t)blockIdx.x * RPB + rr; row < a.rows; row += (int64_t)gridDim.x * RPB) {
        const size_t off = (size_t)row * D + lr * 8;
        float x[8], sc[2];
        int8_t cd[8];
        load8(a.x + off, x);
        quantise8(x, a.bits, a.group, cd, sc);
        uint2 pk;
        pk.x = (uint32_t)(uint8_t)cd[0] | ((uint32_t)(uint8_t)cd[1] << 8) | ((uint32_t)(uint8_t)cd[2] << 16) | ((uint32_t)(uint8_t)cd[3] << 24);
        pk.y = (uint32_t)(uint8_t)cd[4] | ((uint32_t)(uint8_t)cd[5] << 8) | ((uint32_t)(uint8_t)cd[6] << 16) | ((uint32_t)(uint8_t)cd[7] << 24);
        *reinterpret_cast<uint2*>(a.codes + off) = pk;
        float* srow = a.scales + (size_t)row * gpr;
        if (a.group >= 8) {
            if (lr % (a.group / 8) == 0) srow[(lr * 8) / a.group] = sc[0];
        } else {
            srow[lr * 2] = sc[0];
            srow[lr * 2 + 1] = sc[1];
        }
    }
}

unsigned mem_grid(int64_t rows, int D) {
    const int64_t rpb = MEM_THREADS / (D / 8);
    int64_t g = (rows + rpb - 1) / rpb;
    if (g > 256 * 64) g = 256 * 64;                          // grid-stride beyond 64 workgroups per CU
    return (unsigned)(g < 1 ? 1 : g);
}

}  // namespace

// ======================================================================================== C-ABI

static int check_mem(int64_t rows, int64_t D, int bits, int64_t group) {
    if (rows < 1) return fail(SLOTSCAN_ERR_SHAPE, "slotmem: rows must be >= 1");
    if (D != 64 && D != 128) return fail(SLOTSCAN_ERR_SHAPE, "slotmem: D must be 64 or 128");
    if (bits != 0 && (bits < 2 || bits > 8)) return fail(SLOTSCAN_ERR_SHAPE, "slotmem: bits must be 0 or 2..8");
    if (bits != 0 && (group < 4 || group > D || (group & (group - 1)) != 0 || D % group != 0))
        return fail(SLOTSCAN_ERR_SHAPE, "slotmem: group must be a power of two in [4, D] dividing D");
    return 0;
}

extern "C" int slotmem_epilogue_fwd(const float* kbuf, const float* vbuf, int64_t rows, int64_t D, int bits,
                                    int64_t group, int out_dtype, void* kout, void* vout, float* kinv,
                                    uint8_t* valid, void* stream) {
    if (int r = check_mem(rows, D, bits, group)) return r;
    if (out_dtype != SLOTSCAN_F32 && out_dtype != SLOTSCAN_BF16) return fail(SLOTSCAN_ERR_DTYPE, "slotmem: out dtype must be f32 or bf16");
    if (!kbuf || !vbuf || !kout || !vout || !kinv || !valid) return fail(SLOTSCAN_ERR_NULL, "slotmem_epilogue_fwd: NULL pointer");
    if (!al16(kbuf) || !al16(vbuf) || !al16(kout) || !al16(vout)) return fail(SLOTSCAN_ERR_ALIGN, "slotmem_epilogue_fwd: rows must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    MemFwdArgs a{kbuf, vbuf, kout, vout, kinv, valid, rows, bits, (int)group};
    const dim3 grid(mem_grid(rows, (int)D)), block(MEM_THREADS);
    hipError_t e;
    {
        slothost::Scope sc(SLOTSCAN_K_MEM, st);
        if (D == 128) {
            if (out_dtype == SLOTSCAN_BF16) slothost::launch((mem_epilogue<128, bf16_t>), grid, block, 0, st, a);
            else slothost::launch((mem_epilogue<128, float>), grid, block, 0, st, a);
        } else {
            if (out_dtype == SLOTSCAN_BF16) slothost::launch((mem_epilogue<64, bf16_t>), grid, block, 0, st, a);
            else slothost::launch((mem_epilogue<64, float>), grid, block, 0, st, a);
        }
        e = hipGetLastError();
    }
    return e == hipSuccess ? 0 : hip_fail(e, "mem_epilogue launch");
}

extern "C" int slotmem_epilogue_bwd(const float* kbuf, const void* dkout, const void* dvout, const float* dkinv,
                                    int64_t rows, int64_t D, int bits, int64_t group, int grad_dtype,
                                    float* dkbuf, float* dvbuf, void* stream) {
    if (int r = check_mem(rows, D, bits, group)) return r;
    if (grad_dtype != SLOTSCAN_F32 && grad_dtype != SLOTSCAN_BF16) return fail(SLOTSCAN_ERR_DTYPE, "slotmem: grad dtype must be f32 or bf16");
    if (!kbuf || !dkout || !dvout || !dkinv || !dkbuf || !dvbuf) return fail(SLOTSCAN_ERR_NULL, "slotmem_epilogue_bwd: NULL pointer");
    if (!al16(kbuf) || !al16(dkout) || !al16(dvout) || !al16(dkbuf) || !al16(dvbuf))
        return fail(SLOTSCAN_ERR_ALIGN, "slotmem_epilogue_bwd: rows must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    MemBwdArgs a{kbuf, dkout, dvout, dkinv, dkbuf, dvbuf, rows, bits, (int)group};
    const dim3 grid(mem_grid(rows, (int)D)), block(MEM_THREADS);
    hipError_t e;
    {
        slothost::Scope sc(SLOTSCAN_K_MEM_BWD, st);
        if (D == 128) {
            if (grad_dtype == SLOTSCAN_BF16) slothost::launch((mem_epilogue_bwd<128, bf16_t>), grid, block, 0, st, a);
            else slothost::launch((mem_epilogue_bwd<128, float>), grid, block, 0, st, a);
        } else {
            if (grad_dtype == SLOTSCAN_BF16) slothost::launch((mem_epilogue_bwd<64, bf16_t>), grid, block, 0, st, a);
            else slothost::launch((mem_epilogue_bwd<64, float>), grid, block, 0, st, a);
        }
        e = hipGetLastError();
    }
    return e == hipSuccess ? 0 : hip_fail(e, "mem_epilogue_bwd launch");
}

extern "C" int slotmem_codes(const float* x, int64_t rows, int64_t D, int bits, int64_t group, int8_t* codes,
                             float* scales, void* stream) {
    if (int r = check_mem(rows, D, bits, group)) return r;
    if (bits == 0) return fail(SLOTSCAN_ERR_SHAPE, "slotmem_codes: bits must be 2..8");
    if (!x || !codes || !scales) return fail(SLOTSCAN_ERR_NULL, "slotmem_codes: NULL pointer");
    if (!al16(x) || ((uintptr_t)codes & 7u)) return fail(SLOTSCAN_ERR_ALIGN, "slotmem_codes: x 16-byte, codes 8-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    MemCodeArgs a{x, codes, scales, rows, bits, (int)group};
    const dim3 grid(mem_grid(rows, (int)D)), block(MEM_THREADS);
    hipError_t e;
    {
        slothost::Scope sc(SLOTSCAN_K_MEM, st);
        if (D == 128) slothost::launch(mem_codes<128>, grid, block, 0, st, a);
        else slothost::launch(mem_codes<64>, grid, block, 0, st, a);
        e = hipGetLastError();
    }
    return e == hipSuccess ? 0 : hip_fail(e, "mem_codes launch");
}
