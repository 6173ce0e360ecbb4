// The reader layer's output projection into the residual on MI355X (gfx950): out = delta + rd wo^T, the wo_tk
// Linear of SharedMixer (bias-free, /root/reference/gqa25/memlm_sh.py:313) applied to the read and added to the
// window output (memlm_sh.py:499-501), as one bf16 MFMA GEMM whose epilogue is the add.
//   rd    (M, K) bf16 row-major: M = B*T tokens, K = H*NQ*dv, the read kernel's output layout, no copy
//   wo    (N, K) bf16 row-major: N = d_model (nn.Linear weight layout)
//   delta (M, N) bf16 or NULL;  out (M, N) bf16.  Rounding as in the reference: the product (fp32
//         accumulation) is rounded to bf16 -- the bf16 Linear output -- and, with delta, added to it in fp32 and
//         rounded again -- the bf16 residual add (round to nearest even both times)
//
// gfx950 mapping.  A workgroup of 4 waves (one per SIMD, each with the whole 512-register file) owns a
// 256 x 256 output tile; wave (wm, wn) = (w >> 1, w & 1) owns rows 128 wm .. + 128 and columns 128 wn .. + 128
// as 4 x 4 tiles of v_mfma_f32_32x32x16_bf16 (256 fp32 accumulators per lane, 16 independent chains; 8
// 16-byte operand reads per 16 MFMAs).  The MFMA's A operand is the weight (output columns) and its B operand
// the read (output rows), so a lane's 4 consecutive accumulators are 4 consecutive output columns of one row.
// The epilogue passes the bf16 tile through LDS so that delta is read and out written in row-contiguous
// 16-byte accesses.
// K is staged 32 at a time through LDS in a ring of 4 stages (128 KB), filled by direct global -> LDS loads
// (global_load_lds_dwordx4: no registers hold the prefetch) issued 2-3 stages ahead, one workgroup barrier
// per stage.  The loop is software-pipelined: loads, the barrier and the next stage's LDS operand reads are
// interleaved with the current stage's MFMAs, so the MFMA pipe is not left idle while a wave issues them.  A load instruction fills 1 KB of LDS = 16 rows of 64 bytes, lane L at byte 16 L; the
// lane fetches the row's 16-byte chunk c = (L & 3) ^ ((row >> 2) & 3).  gfx950's LDS has 64 4-byte banks and
// serves a 16-byte read 16 lanes at a time, so the operand reads of 16 consecutive rows at one k chunk must
// cover 256 bytes of distinct banks: rows r, r + 4, r + 8, r + 12 share banks modulo 256 bytes and the XOR puts
// their chunk in 4 different places (a swizzle in place of padding, which a direct load cannot leave).  Workgroup order is XCD-aware: the 8 column tiles of a row block run on
// one XCD (workgroup i goes to XCD i mod 8), so that block's read rows are fetched into one L2 once.
#include <type_traits>

#include "slot_common.h"
#include "slotscan.h"
#include "slotproj.h"
#include "slot_host.h"

using namespace slot;
using slothost::fail;
using slothost::hip_fail;

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int PT = 256;            // output tile edge (rows and columns)
constexpr int PK = 32;             // K per stage: 64-byte LDS rows
constexpr int NST = 4;             // stages in the LDS ring
constexpr int PTHREADS = 256;
constexpr int STAGE = PT * PK * 2; // bytes of one operand's stage (16 KB)
constexpr int PLD = STAGE / 1024 / (PTHREADS / 64);   // 1-KB load instructions per wave, operand and stage (4)
constexpr int PXCD = 8;            // XCDs of an MI355X: consecutive workgroups go to consecutive XCDs

struct ProjArgs {
    const bf16_t* a; const bf16_t* w; const bf16_t* d; bf16_t* out;
    int M, N, K, mblocks, nblocks;
};

__device__ __forceinline__ f32x16 mfma32(const uint4& a, const uint4& b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

// wait until at most n of this wave's vector-memory operations are outstanding (n constant: the count is an
// instruction immediate; the other counters are left unconstrained)
template <int n>
__device__ __forceinline__ void wait_vm() {
    static_assert(n >= 0 && n < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (n & 15) | ((n >> 4) << 14));
}

// The ring's direct global -> LDS loads (dma16) are not tracked by the compiler: its own tracking cannot tell
// the ring's buffers apart and would drain every load in flight before each stage's first LDS read.  The kernel
// waits for these loads itself (wait_vm before the barrier that publishes a stage), and issues no other
// vector-memory load while any is in flight, so the compiler's counts for its own loads stay exact.

// workgroup barrier that orders LDS for the compiler but adds no hardware wait for the direct loads still in
// flight (those are waited for explicitly, per stage, before the barrier that publishes them)
__device__ __forceinline__ void stage_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

__global__ __launch_bounds__(PTHREADS) void proj_gemm(ProjArgs p) {
    // the k ring: stage s of rd at sA + (s % NST) STAGE, of wo at sW + (s % NST) STAGE; after the k loop the
    // same 128 KB hold the workgroup's bf16 output tile (256 rows x 512 bytes) for the epilogue
    __shared__ __align__(1024) unsigned char smem[2 * NST * STAGE];
    unsigned char* const sA = smem;
    unsigned char* const sW = smem + NST * STAGE;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // XCD-aware tile order: workgroup i runs on XCD i % 8; the column tiles of one row block share an XCD
    const int bid = blockIdx.x, xcd = bid % PXCD, k8 = bid / PXCD;
    const int nb = k8 % p.nblocks, mb = (k8 / p.nblocks) * PXCD + xcd;
    if (mb >= p.mblocks) return;                           // padding workgroups of the last row-block group
    const int m0 = mb * PT, n0 = nb * PT;
    const int M = p.M, K = p.K, KT = K / PK;

    // direct loads: instruction i of wave w fills rows 16 (4 i + w) .. + 15 of a stage; lane L takes row
    // + (L >> 2) and the chunk that belongs at its LDS position L & 3.  Rows of rd past M repeat row M - 1
    // (their outputs are never stored; every output row depends on its own rd row only).
    const bf16_t* ga[PLD];
    const bf16_t* gw[PLD];
#pragma unroll
    for (int i = 0; i < PLD; i++) {
        const int r = 16 * (PLD * i + wave) + (lane >> 2);
        const int c = (lane & 3) ^ ((r >> 2) & 3);
        ga[i] = p.a + (size_t)min(m0 + r, M - 1) * K + 8 * c;
        gw[i] = p.w + (size_t)(n0 + r) * K + 8 * c;
    }
    // load q (0..7) of stage kt: q < 4 the rd instruction q, else the wo instruction q - 4
    auto dma = [&](int kt, int q) {
        const int buf = kt % NST, k0 = kt * PK;
        if (q < PLD) dma16(ga[q] + k0, lds_addr(sA + buf * STAGE + (PLD * q + wave) * 1024));
        else dma16(gw[q - PLD] + k0, lds_addr(sW + buf * STAGE + (PLD * (q - PLD) + wave) * 1024));
    };

    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31;
    // byte offset of this lane's operand chunk in a 32-row tile: row lr, logical chunk 2 ks + (lane >> 5)
    int off[2];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) off[ks] = lr * 64 + 16 * ((2 * ks + (lane >> 5)) ^ ((lr >> 2) & 3));
    // a stage's MFMA operands: op[ks][j] = wo rows 32 j + lr (A operand), op[ks][4 + i] = rd rows 32 i + lr
    // (B operand), k step ks; read in 4 groups of 4 (wo ks 0, rd ks 0, wo ks 1, rd ks 1)
    auto read_ops = [&](int kt, uint4 (&op)[2][8], int r) {
        const int buf = kt % NST, ks = r >> 1;
        if ((r & 1) == 0) {
            const unsigned char* Ws = sW + buf * STAGE + 128 * wn * 64 + off[ks];
#pragma unroll
            for (int j = 0; j < 4; j++) op[ks][j] = *reinterpret_cast<const uint4*>(Ws + 32 * j * 64);
        } else {
            const unsigned char* As = sA + buf * STAGE + 128 * wm * 64 + off[ks];
#pragma unroll
            for (int i = 0; i < 4; i++) op[ks][4 + i] = *reinterpret_cast<const uint4*>(As + 32 * i * 64);
        }
    };
    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    // One k stage = 8 groups of 4 MFMAs (k step g >> 2, rd tile g & 3, the 4 wo tiles).  Behind group g the
    // wave issues load g of stage kt + 3 (into the buffer stage kt - 1 used: every wave finished reading it
    // before the previous stage's barrier), so the loads trickle out between MFMAs instead of stalling the
    // wave in a burst.  Behind group 4 it waits for stage kt + 1 (its loads, issued two stages earlier, are
    // complete when at most stage kt + 2's 8 and stage kt + 3's first 5 loads are outstanding), drains its own
    // LDS reads, and passes the barrier that publishes stage kt + 1; behind groups 4..7 it reads stage kt + 1's
    // operands into the other register set, in flight while the remaining MFMAs run.
    constexpr int PER = 2 * PLD;                           // loads per wave and stage (8)
    auto stage = [&](int kt, uint4 (&cur)[2][8], uint4 (&nxt)[2][8]) {
        const bool more = kt + 1 < KT, pre = kt + 3 < KT;
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const int ks = g >> 2, i = g & 3;
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = mfma32(cur[ks][j], cur[ks][4 + i], acc[i][j]);
            __builtin_amdgcn_sched_barrier(0);
            if (pre) dma(kt + 3, g);
            if (g == 4 && more) {
                if (pre) wait_vm<PER + 5>();
                else if (kt + 2 < KT) wait_vm<PER>();
                else wait_vm<0>();
                wait_lgkm0();
                stage_barrier();
            }
            if (g >= 4 && more) read_ops(kt + 1, nxt, g - 4);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    uint4 opA[2][8], opB[2][8];
#pragma unroll
    for (int st = 0; st < NST - 1; st++)
        if (st < KT)
#pragma unroll
            for (int q = 0; q < PER; q++) dma(st, q);
    if (KT > 2) wait_vm<2 * PER>();
    else if (KT > 1) wait_vm<PER>();
    else wait_vm<0>();
    stage_barrier();
#pragma unroll
    for (int r = 0; r < 4; r++) read_ops(0, opA, r);
    int kt = 0;
    for (; kt + 1 < KT; kt += 2) {
        stage(kt, opA, opB);
        stage(kt + 1, opB, opA);
    }
    if (kt < KT) stage(kt, opA, opB);

    // epilogue.  acc[i][j] lane l, register r holds D[n][m] with m = 32 i + (l & 31) (output row) and
    // n = 32 j + 8 (r >> 2) + 4 (l >> 5) + (r & 3) (output column).  The product is rounded to bf16 (the
    // reference's Linear output) and written to LDS as 8-byte column quads: row m at byte 512 m, quad s at
    // slot s ^ (m & 31), so the 32 rows of one store land on 32 distinct 8-byte bank slots.  Then every thread
    // moves 16-byte row chunks: the 2 quads of a chunk sit in one aligned 16-byte slot pair (swapped when
    // m is odd), are added to delta in fp32 and rounded again (the reference's bf16 residual add), and stored
    // with row-contiguous 16-byte accesses.
    wait_lgkm0();
    stage_barrier();                                       // every wave is done with the ring
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int m = 128 * wm + 32 * i + lr;
                const int sq = 32 * wn + 8 * j + 2 * g + (lane >> 5);
                uint2 o;
                o.x = pack_bf16x2(acc[i][j][4 * g], acc[i][j][4 * g + 1]);
                o.y = pack_bf16x2(acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
                *reinterpret_cast<uint2*>(smem + m * 512 + 8 * (sq ^ lr)) = o;
            }
    stage_barrier();
    auto epilogue = [&](auto with_delta) {
        constexpr int CH = PT * PT * 2 / 16 / PTHREADS;   // 16-byte chunks per thread (32)
        constexpr int BATCH = 16;
#pragma unroll
        for (int b0 = 0; b0 < CH; b0 += BATCH) {
            uint4 dv[BATCH];
            if constexpr (decltype(with_delta)::value) {
#pragma unroll
                for (int u = 0; u < BATCH; u++) {
                    const int idx = (b0 + u) * PTHREADS + tid, r = idx >> 5, c = idx & 31;
                    dv[u] = *reinterpret_cast<const uint4*>(p.d + (size_t)min(m0 + r, M - 1) * p.N + n0 + 8 * c);
                }
            }
#pragma unroll
            for (int u = 0; u < BATCH; u++) {
                const int idx = (b0 + u) * PTHREADS + tid, r = idx >> 5, c = idx & 31;
                uint4 v = *reinterpret_cast<const uint4*>(smem + r * 512 + 16 * (c ^ ((r & 31) >> 1)));
                if (r & 1) v = make_uint4(v.z, v.w, v.x, v.y);
                if constexpr (decltype(with_delta)::value) {
                    auto add2 = [](unsigned x, unsigned d) {
                        return pack_bf16x2(__uint_as_float(x << 16) + __uint_as_float(d << 16),
                                           __uint_as_float(x & 0xffff0000u) + __uint_as_float(d & 0xffff0000u));
                    };
                    v = make_uint4(add2(v.x, dv[u].x), add2(v.y, dv[u].y), add2(v.z, dv[u].z), add2(v.w, dv[u].w));
                }
                if (m0 + r < M) *reinterpret_cast<uint4*>(p.out + (size_t)(m0 + r) * p.N + n0 + 8 * c) = v;
            }
        }
    };
    if (p.d) epilogue(std::true_type{});
    else epilogue(std::false_type{});
}

}  // namespace

extern "C" int slotproj_fwd(const void* rd, const void* wo, const void* delta, int64_t M, int64_t N, int64_t K,
                            void* out, void* stream) {
    if (M < 1 || N < 1 || K < 1) return fail(SLOTSCAN_ERR_SHAPE, "slotproj_fwd: M, N and K must be >= 1");
    if (N % PT != 0 || K % PK != 0)
        return fail(SLOTSCAN_ERR_SHAPE, "slotproj_fwd: N must be a multiple of 256 and K a multiple of 32");
    if (M > 0x7fffffffLL || N * K > 0x7fffffffLL || M * N > ((int64_t)1 << 40))
        return fail(SLOTSCAN_ERR_SHAPE, "slotproj_fwd: shape too large");
    if (!rd || !wo || !out) return fail(SLOTSCAN_ERR_NULL, "slotproj_fwd: a required pointer is NULL");
    if (!slothost::al16(rd) || !slothost::al16(wo) || !slothost::al16(delta) || !slothost::al16(out))
        return fail(SLOTSCAN_ERR_ALIGN, "slotproj_fwd: rd, wo, delta and out must be 16-byte aligned");
    ProjArgs a{(const bf16_t*)rd, (const bf16_t*)wo, (const bf16_t*)delta, (bf16_t*)out, (int)M, (int)N, (int)K,
               (int)((M + PT - 1) / PT), (int)(N / PT)};
    const int groups = (a.mblocks + PXCD - 1) / PXCD;
    hipStream_t st = (hipStream_t)stream;
    {
        slothost::Scope sc(SLOTSCAN_K_PROJ, st);
        slothost::launch(proj_gemm, dim3((unsigned)(groups * PXCD * a.nblocks)), dim3(PTHREADS), 0, st, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "proj_gemm launch");
    return 0;
}
