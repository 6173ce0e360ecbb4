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
#include <algorithm>
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
typedef uint32_t u32;
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

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
    // with delta (the forward's residual add) delta is read once and out written once, 2 x 268 MB at config4_wo:
    // streaming accesses (config4_wo 2.036 -> 1.933 ms/step A/B in one process)
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
                    const u32x4v x = __builtin_nontemporal_load(
                        reinterpret_cast<const u32x4v*>(p.d + (size_t)min(m0 + r, M - 1) * p.N + n0 + 8 * c));
                    dv[u] = make_uint4(x.x, x.y, x.z, x.w);
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
                if (m0 + r < M) {
                    uint4* dst = reinterpret_cast<uint4*>(p.out + (size_t)(m0 + r) * p.N + n0 + 8 * c);
                    if constexpr (decltype(with_delta)::value) {
                        const u32x4v x = {v.x, v.y, v.z, v.w};
                        __builtin_nontemporal_store(x, reinterpret_cast<u32x4v*>(dst));
                    } else {
                        *dst = v;                          // the backward's drd, read by read_bwd right after
                    }
                }
            }
        }
    };
    if (p.d) epilogue(std::true_type{});
    else epilogue(std::false_type{});
}

// ------------------------------------------------------------------------------------ the backward's GEMMs
// dWo = dDelta^T rd: C (N, K) = A^T B with A = dDelta (M, N) and B = rd (M, K), both token-major, the tokens
// the reduction.  The same 256 x 256 tile, 4 waves and 4-stage ring of direct global -> LDS loads as
// proj_gemm, a stage now being 32 TOKEN rows of the tile's 256 columns of each operand (512-byte LDS rows,
// the 16-byte chunk c of row t at chunk position c ^ 2 (t & 3)).  The MFMA operands need 8 consecutive
// tokens of one column per lane, which gfx950's transposing LDS read delivers: ds_read_b64_tr_b16 lets each
// 16-lane group read a 4 x 16 block of 16-bit values -- lane l supplying the address of 4 consecutive
// elements of row (l >> 2) & 3 -- and hands lane l the 4 rows of column l; two such reads (tokens t..t+3,
// t+4..t+7) are one operand.  The chunk swizzle puts the 4 rows x 2 chunks of one group's read on 8 distinct
// 16-byte bank groups.  The tokens are split over `splits` workgroups per output tile (24 tiles at
// d_model 2048 and K 768 would not fill 256 CUs); each writes its fp32 partial tile and proj_reduce sums the
// partials in split order and rounds the sum to bf16 once (the bf16 matmul's one rounding of its fp32
// accumulation) -- fixed order, no atomics.
struct ProjTArgs {
    const bf16_t* a; const bf16_t* b; float* part;
    int M, N, K, nblocks, kblocks, tps;                   // tps: tokens per split (a multiple of PK)
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ uint2 ld_tr(const unsigned char* p) {
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((const lds_void*)p));
    return __builtin_bit_cast(uint2, v);
}

__global__ __launch_bounds__(PTHREADS) void projt_gemm(ProjTArgs p) {
    __shared__ __align__(1024) unsigned char smem[2 * NST * STAGE];
    unsigned char* const sA = smem;
    unsigned char* const sB = smem + NST * STAGE;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tiles = p.nblocks * p.kblocks;
    const int split = blockIdx.x / tiles, tile = blockIdx.x % tiles;
    const int nb = tile / p.kblocks, kb = tile % p.kblocks;
    const int n0 = nb * PT, k0 = kb * PT;
    const int m_lo = split * p.tps, m_hi = min(p.M, m_lo + p.tps);
    const int KT = (m_hi - m_lo) / PK;                    // full stages (the pipelined loop)
    const int tail = (m_hi - m_lo) - KT * PK;             // tokens of a last partial stage (0 .. 31)

    // direct loads: instruction i of wave w fills token rows 2 (4 i + w) and + 1 of a stage (lane L: row
    // + (L >> 5), chunk position L & 31, global chunk (L & 31) ^ 2 (row & 3))
    const bf16_t* ga[PLD];
    const bf16_t* gb[PLD];
#pragma unroll
    for (int i = 0; i < PLD; i++) {
        const int r = 2 * (PLD * i + wave) + (lane >> 5);
        const int c = (lane & 31) ^ (2 * (r & 3));
        ga[i] = p.a + (size_t)(m_lo + r) * p.N + n0 + 8 * c;
        gb[i] = p.b + (size_t)(m_lo + r) * p.K + k0 + 8 * c;
    }
    auto dma = [&](int kt, int q) {
        const int buf = kt % NST;
        if (q < PLD) dma16(ga[q] + (size_t)kt * PK * p.N, lds_addr(sA + buf * STAGE + (PLD * q + wave) * 1024));
        else dma16(gb[q - PLD] + (size_t)kt * PK * p.K, lds_addr(sB + buf * STAGE + (PLD * (q - PLD) + wave) * 1024));
    };

    const int wm = wave >> 1, wn = wave & 1;
    // this lane's part of a transposed read: token row 8 (g >> 1) + ((l >> 2) & 3) (+ 16 ks + 4 half), chunk
    // 2 (g & 1) + ((l & 3) >> 1) of the operand tile's 32 columns, byte 8 (l & 1) of the chunk; g = l >> 4
    const int g4 = lane >> 4, rq = (lane >> 2) & 3;
    const int rowb = (8 * (g4 >> 1) + rq) * 512, cl = 2 * (g4 & 1) + ((lane & 3) >> 1), hb = 8 * (lane & 1);
    int offA[4], offB[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        offA[t] = rowb + 16 * ((16 * wm + 4 * t + cl) ^ (2 * rq)) + hb;
        offB[t] = rowb + 16 * ((16 * wn + 4 * t + cl) ^ (2 * rq)) + hb;
    }
    // op[ks][t]: A operand of n tile t (dDelta), op[ks][4 + t]: B operand of k tile t (rd); groups of 4 reads
    // as in proj_gemm (A ks 0, B ks 0, A ks 1, B ks 1)
    auto read_ops_at = [&](const unsigned char* bufA, const unsigned char* bufB, uint4 (&op)[2][8], int r) {
        const int ks = r >> 1;
        const unsigned char* base = (r & 1) ? bufB : bufA;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const unsigned char* q0 = base + ((r & 1) ? offB[t] : offA[t]) + 16 * ks * 512;
            const uint2 lo = ld_tr(q0), hi = ld_tr(q0 + 4 * 512);
            op[ks][4 * (r & 1) + t] = make_uint4(lo.x, lo.y, hi.x, hi.y);
        }
    };
    auto read_ops = [&](int kt, uint4 (&op)[2][8], int r) {
        const int buf = kt % NST;
        read_ops_at(sA + buf * STAGE, sB + buf * STAGE, op, r);
    };
    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    // the k loop of proj_gemm (same load trickle, counted waits and barrier placement), with the A operand
    // the n tile i and the B operand the k tile j
    constexpr int PER = 2 * PLD;
    auto stage = [&](int kt, uint4 (&cur)[2][8], uint4 (&nxt)[2][8]) {
        const bool more = kt + 1 < KT, pre = kt + 3 < KT;
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const int ks = g >> 2, i = g & 3;
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = mfma32(cur[ks][i], cur[ks][4 + j], acc[i][j]);
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
    // (not wrapped in a test of KT > 0: with no full stage nothing is loaded, the operand reads below read
    // whatever the ring holds and no MFMA uses them; a branch here made the compiler spill the accumulators)
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
    if (tail) {
        // the last, partial stage: plain loads of the valid token rows (zeros past them, so they add
        // nothing), written to ring buffer 0 in the swizzled layout, then one stage of MFMAs
        wait_lgkm0();
        stage_barrier();                                   // every wave is done reading the ring
        const int t0 = m_lo + KT * PK;
#pragma unroll
        for (int i = 0; i < PLD; i++) {
            const int r = 2 * (PLD * i + wave) + (lane >> 5);
            const int c = (lane & 31) ^ (2 * (r & 3));
            const int m = min(t0 + r, p.M - 1);
            uint4 va = *reinterpret_cast<const uint4*>(p.a + (size_t)m * p.N + n0 + 8 * c);
            uint4 vb = *reinterpret_cast<const uint4*>(p.b + (size_t)m * p.K + k0 + 8 * c);
            if (r >= tail) va = vb = make_uint4(0u, 0u, 0u, 0u);
            *reinterpret_cast<uint4*>(sA + (PLD * i + wave) * 1024 + 16 * lane) = va;
            *reinterpret_cast<uint4*>(sB + (PLD * i + wave) * 1024 + 16 * lane) = vb;
        }
        wait_lgkm0();
        stage_barrier();
#pragma unroll
        for (int r = 0; r < 4; r++) read_ops_at(sA, sB, opA, r);
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const int ks = g >> 2, i = g & 3;
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = mfma32(opA[ks][i], opA[ks][4 + j], acc[i][j]);
        }
    }
    // epilogue: acc[i][j] lane l, register r holds C[n][k] with n = 128 wm + 32 i + 8 (r >> 2) + 4 (l >> 5) +
    // (r & 3) and k = 128 wn + 32 j + (l & 31): 32 lanes store 128 contiguous bytes of one partial row
    // (a wave-uniform base and one 32-bit lane offset: no per-element 64-bit addresses; the lane id is formed
    // anew with mbcnt, so that nothing computed before the k loop has to stay live across it)
    const int ln = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    const float* out0 = p.part + (size_t)split * p.N * p.K + (size_t)(n0 + 128 * wm) * p.K + k0 + 128 * wn;
    const u32 loff = (u32)((4 * (ln >> 5)) * p.K + (ln & 31)) * 4u;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int dr = 32 * i + 8 * (r >> 2) + (r & 3);
            char* rowp = (char*)(out0 + (size_t)dr * p.K);
#pragma unroll
            for (int j = 0; j < 4; j++)
                __builtin_nontemporal_store(acc[i][j][r], reinterpret_cast<float*>(rowp + loff + 128 * j));
        }
}

// dWo = bf16(sum over the splits, in split order, of the fp32 partials): 4 elements per thread
__global__ __launch_bounds__(256) void proj_reduce(const float* __restrict__ part, int splits, int64_t nk,
                                                   bf16_t* __restrict__ out) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= nk) return;
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    f32x4 s = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(part + i));
    for (int q = 1; q < splits; q++) {
        const f32x4 x = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(part + (size_t)q * nk + i));
        s.x += x.x; s.y += x.y; s.z += x.z; s.w += x.w;
    }
    uint2 r;
    r.x = pack_bf16x2(s.x, s.y);
    r.y = pack_bf16x2(s.z, s.w);
    *reinterpret_cast<uint2*>(out + i) = r;
}

// woT (K, N) = wo (N, K)^T, bf16, 64 x 64 tiles through LDS (the 2 x 64 x 64 staging reads / writes whole
// 128-byte rows on both sides)
__global__ __launch_bounds__(256) void proj_transpose(const bf16_t* __restrict__ w, int N, int K,
                                                      bf16_t* __restrict__ wt) {
    __shared__ bf16_t t[64][66];
    const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64, tid = threadIdx.x;
    for (int u = tid; u < 64 * 64; u += 256) {
        const int r = u >> 6, c = u & 63;
        if (r0 + r < N && c0 + c < K) t[r][c] = w[(size_t)(r0 + r) * K + c0 + c];
    }
    __syncthreads();
    for (int u = tid; u < 64 * 64; u += 256) {
        const int c = u >> 6, r = u & 63;
        if (r0 + r < N && c0 + c < K) wt[(size_t)(c0 + c) * N + r0 + r] = t[r][c];
    }
}

// the token splits of projt_gemm for an (N, K) output: about two rounds of workgroups on 256 CUs, each split
// a multiple of the 32-token stage
static void projt_plan(int64_t M, int64_t N, int64_t K, int* splits, int* tps) {
    const int64_t tiles = (N / PT) * (K / PT);
    int64_t s = std::max<int64_t>(1, (512 + tiles - 1) / tiles);
    int64_t t = ((M + s - 1) / s + PK - 1) / PK * PK;
    s = (M + t - 1) / t;
    *splits = (int)s;
    *tps = (int)t;
}

}  // namespace

extern "C" size_t slotproj_bwd_workspace(int64_t M, int64_t N, int64_t K) {
    if (M < 1 || N < 1 || K < 1) return 0;
    int splits = 0, tps = 0;
    projt_plan(M, N, K, &splits, &tps);
    const size_t wt = ((size_t)N * K * 2 + 255) & ~(size_t)255;
    return wt + (size_t)splits * N * K * 4;
}

extern "C" int slotproj_bwd(const void* dout, const void* rd, const void* wo, int64_t M, int64_t N, int64_t K,
                            void* drd, void* dwo, void* workspace, void* stream) {
    if (M < 1 || N < 1 || K < 1) return fail(SLOTSCAN_ERR_SHAPE, "slotproj_bwd: M, N and K must be >= 1");
    if (N % PT != 0 || K % PT != 0)
        return fail(SLOTSCAN_ERR_SHAPE, "slotproj_bwd: N and K must be multiples of 256");
    if (M > 0x7fffffffLL || N * K > 0x7fffffffLL || M * N > ((int64_t)1 << 40) || M * K > ((int64_t)1 << 40))
        return fail(SLOTSCAN_ERR_SHAPE, "slotproj_bwd: shape too large");
    if (!dout || !rd || !wo || !drd || !dwo || !workspace)
        return fail(SLOTSCAN_ERR_NULL, "slotproj_bwd: a required pointer is NULL");
    if (!slothost::al16(dout) || !slothost::al16(rd) || !slothost::al16(wo) || !slothost::al16(drd) ||
        !slothost::al16(dwo) || ((uintptr_t)workspace & 255u))
        return fail(SLOTSCAN_ERR_ALIGN, "slotproj_bwd: operands 16-byte, workspace 256-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    bf16_t* wt = (bf16_t*)workspace;
    float* part = (float*)((char*)workspace + (((size_t)N * K * 2 + 255) & ~(size_t)255));
    // dRD (M, K) = dout (M, N) wo (N, K): proj_gemm with the transposed weight as its (K, N) operand
    slothost::launch(proj_transpose, dim3((unsigned)((K + 63) / 64), (unsigned)((N + 63) / 64)), dim3(256), 0, st,
                     (const bf16_t*)wo, (int)N, (int)K, wt);
    {
        slothost::Scope sc(SLOTSCAN_K_PROJ_DRD, st);
        ProjArgs a{(const bf16_t*)dout, wt, nullptr, (bf16_t*)drd, (int)M, (int)K, (int)N,
                   (int)((M + PT - 1) / PT), (int)(K / PT)};
        const int groups = (a.mblocks + PXCD - 1) / PXCD;
        slothost::launch(proj_gemm, dim3((unsigned)(groups * PXCD * a.nblocks)), dim3(PTHREADS), 0, st, a);
    }
    // dWo (N, K) = dout^T rd: the transposing GEMM over token splits, then the fixed-order reduction
    int splits = 0, tps = 0;
    projt_plan(M, N, K, &splits, &tps);
    {
        slothost::Scope sc(SLOTSCAN_K_PROJ_DWO, st);
        ProjTArgs t{(const bf16_t*)dout, (const bf16_t*)rd, part, (int)M, (int)N, (int)K, (int)(N / PT), (int)(K / PT),
                    tps};
        slothost::launch(projt_gemm, dim3((unsigned)(splits * t.nblocks * t.kblocks)), dim3(PTHREADS), 0, st, t);
    }
    {
        slothost::Scope sc(SLOTSCAN_K_PROJ_RED, st);
        const int64_t nk = N * K;
        slothost::launch(proj_reduce, dim3((unsigned)((nk / 4 + 255) / 256)), dim3(256), 0, st, (const float*)part,
                         splits, nk, (bf16_t*)dwo);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "slotproj_bwd launch");
    return 0;
}

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
