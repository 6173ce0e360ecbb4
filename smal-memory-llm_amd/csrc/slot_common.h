// Shared device helpers for the slot-scan and slot-read kernels (gfx950, wave64).
//
// Row layout used by every scan kernel: a slot row of D floats is owned by a ROW GROUP of 16 consecutive
// lanes (one DPP row).  Lane c of the group holds D/16 elements as D/64 chunks of 4 consecutive floats at
// offsets 4c + 64j, so one dwordx4 access by the 16 lanes covers 256 contiguous bytes of the row.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace slot {

typedef uint16_t bf16_t;

__device__ __forceinline__ float bf2f(bf16_t x) { return __uint_as_float((uint32_t)x << 16); }

// float -> bfloat16, round to nearest even (torch's .to(torch.bfloat16) rounding); gfx950 converts in
// hardware (v_cvt_pk_bf16_f32)
__device__ __forceinline__ bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

// two floats -> packed bfloat16 pair (lo in bits 0-15), one v_cvt_pk_bf16_f32
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
// float rounded to the nearest bfloat16, returned as float
__device__ __forceinline__ float bf16_round(float x) { return __uint_as_float((uint32_t)f2bf(x) << 16); }

// ---- 4-element vector access in the input / output element type --------------------------------------
__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 ld4(const bf16_t* p) {
    uint2 r = *reinterpret_cast<const uint2*>(p);
    return make_float4(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u),
                       __uint_as_float(r.y << 16), __uint_as_float(r.y & 0xffff0000u));
}
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
__device__ __forceinline__ void st4(bf16_t* p, float4 v) {
    uint2 r;
    r.x = pack_bf16x2(v.x, v.y);
    r.y = pack_bf16x2(v.z, v.w);
    *reinterpret_cast<uint2*>(p) = r;
}
// streaming (write-once) store of a float4: non-temporal, so the snapshot stream does not evict the
// working set from L2
__device__ __forceinline__ void st4_nt(float* p, float4 v) {
    __builtin_nontemporal_store(v.x, p + 0);
    __builtin_nontemporal_store(v.y, p + 1);
    __builtin_nontemporal_store(v.z, p + 2);
    __builtin_nontemporal_store(v.w, p + 3);
}
__device__ __forceinline__ float4 ld4_nt(const float* p) {
    return make_float4(__builtin_nontemporal_load(p + 0), __builtin_nontemporal_load(p + 1),
                       __builtin_nontemporal_load(p + 2), __builtin_nontemporal_load(p + 3));
}

template <typename T> __device__ __forceinline__ float ld1(const T* p);
template <> __device__ __forceinline__ float ld1<float>(const float* p) { return *p; }
template <> __device__ __forceinline__ float ld1<bf16_t>(const bf16_t* p) { return bf2f(*p); }
template <typename T> __device__ __forceinline__ void st1(T* p, float v);
template <> __device__ __forceinline__ void st1<float>(float* p, float v) { *p = v; }
template <> __device__ __forceinline__ void st1<bf16_t>(bf16_t* p, float v) { *p = f2bf(v); }

// ---- cross-lane primitives ------------------------------------------------------------------------------
// DPP controls (GFX9 encoding): quad_perm [1,0,3,2] = lane^1, quad_perm [2,3,0,1] = lane^2,
// row_half_mirror (lane i <-> 7-i inside each 8), row_mirror (lane i <-> 15-i inside each 16).
#define SLOT_DPP_XOR1 0xB1
#define SLOT_DPP_XOR2 0x4E
#define SLOT_DPP_HMIR 0x141
#define SLOT_DPP_MIR 0x140

template <int CTRL> __device__ __forceinline__ float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL> __device__ __forceinline__ uint32_t dppu(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

// Sum over the 16 lanes of a DPP row; every lane of the row receives the bitwise-same result (each stage
// adds the same two partial sums, and IEEE addition is commutative).
__device__ __forceinline__ float rowsum16(float v) {
    v += dppf<SLOT_DPP_XOR1>(v);
    v += dppf<SLOT_DPP_XOR2>(v);
    v += dppf<SLOT_DPP_HMIR>(v);
    v += dppf<SLOT_DPP_MIR>(v);
    return v;
}
__device__ __forceinline__ float rowmax16(float v) {
    v = fmaxf(v, dppf<SLOT_DPP_XOR1>(v));
    v = fmaxf(v, dppf<SLOT_DPP_XOR2>(v));
    v = fmaxf(v, dppf<SLOT_DPP_HMIR>(v));
    v = fmaxf(v, dppf<SLOT_DPP_MIR>(v));
    return v;
}

// Sum over the 4 row groups of a wave (lanes c, c+16, c+32, c+48), result at every lane.  The gfx950
// permlane swaps exchange 16-lane rows (odd rows of the first operand with even rows of the second) and
// 32-lane halves; with both operands the same register the two returned copies hold the two partners'
// values at every lane, in the same order everywhere, so the sum is symmetric and bitwise uniform.
__device__ __forceinline__ float sum4rows(float v) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    float s = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Full wave64 sum (result at every lane).
__device__ __forceinline__ float wavesum(float v) { return sum4rows(rowsum16(v)); }

// ---- ordered keys for a deterministic argmax ----------------------------------------------------------
// Monotone map float -> uint32 (larger float -> larger key).  -0 is folded into +0 first so that the key
// order is exactly IEEE's order on non-NaN values.
__device__ __forceinline__ uint32_t fkey(float z) {
    uint32_t u = __float_as_uint(z + 0.0f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float fkey_inv(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

typedef __attribute__((address_space(3))) void lds_void;

// LDS byte address of a __shared__ object (for m0)
__device__ __forceinline__ unsigned lds_addr(const void* p) {
    return (unsigned)reinterpret_cast<uintptr_t>((const lds_void*)p);
}

// One direct global -> LDS load: 16 bytes per active lane from g into LDS at lds + 16 * lane (lds
// wave-uniform, in m0).  Issued as inline assembly, so the compiler does not track it: the caller waits for
// it explicitly (a vmcnt wait) before the barrier that publishes the data.  It holds no data register.
__device__ __forceinline__ void dma16(const void* g, unsigned lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, off" : : "{m0}"(lds), "v"(g) : "memory");
}

}  // namespace slot
