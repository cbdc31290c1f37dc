// gemm_i8.hip - MATMUL_I8 prefill path on the gfx950 int8 matrix cores.
//
// Replaces the reference's AVX2 packed-panel / 2x32 tiles
// (src/kernels/kernels.cpp:635-869) for M > 8.  Same semantics as the
// reference's store_i8_c (kernels.cpp:526-535): exact int32 accumulation,
// then C = epi(((float)acc * scale_a[m]) * scale_b[n] + bias[n]).
//
// Kernels, chosen by gemm_i8() at the end of the file:
//   * gemm_i8_wide   - 256 x 256 (or 192) tiles, M % 256 == 0,
//                      K % 128 == 0, when whole rounds of tiles favour them;
//   * gemm_i8_k128w8 - 256 x 128 tiles, 8 waves, K % 128 == 0;
//   * gemm_i8_pipe   - 256 x 128 tiles, 64-deep stages, K % 64 == 0;
//   * gemm_i8_generic - any shape and alignment (below).
// All of them multiply int8 fragments read from the packed weight layout and
// accumulate exactly in int32.
//
// Generic kernel: workgroup tile BM x BN = 128 x 128, 4 waves in a 2 x 2
// grid, wave tile 64 x 64 = 4 x 4 v_mfma_i32_16x16x64_i8 blocks; A staged
// through LDS (rows padded to 80 bytes, conflict-free ds_read_b128), B loaded
// straight from the packed layout (one 16-byte load per lane per 1 KiB
// operand block).  Fragment convention (both operands use the same k order,
// so the integer result is exact whatever order the hardware sums in):
// lane l = 16*g + r holds row/column r and k = 16*g .. 16*g + 15 of the
// 64-deep block.  Output: lane l holds C[4*(l/16) + i][l%16], i = 0..3.
#include "kernels.hpp"

#include <atomic>
#include <type_traits>
#include "device_math.hpp"
#include "lds_dma.hpp"

namespace vnpu {
namespace k {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kThreads = 256;
constexpr int kPitch = 80;  // LDS row pitch for A (64 data + 16 pad bytes)

__device__ __forceinline__ v4i load_a_chunk(const I8Gemm &p, uint32_t m, uint32_t k, bool vec)
{
    v4i v = {0, 0, 0, 0};
    if (m >= p.M) return v;
    const int8_t *src = p.A + static_cast<uint64_t>(m) * p.lda + k;
    if (vec && k + 16 <= p.K) return *reinterpret_cast<const v4i *>(src);
    union {
        int8_t b[16];
        v4i v;
    } u;
#pragma unroll
    for (int j = 0; j < 16; ++j) u.b[j] = (k + j < p.K) ? src[j] : 0;
    return u.v;
}

__global__ __launch_bounds__(kThreads) void gemm_i8_generic(I8Gemm p)
{
    __shared__ __attribute__((aligned(16))) int8_t a_lds[2][BM * kPitch];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t m0 = blockIdx.y * BM;
    const uint32_t n0 = blockIdx.x * BN;
    const uint32_t NT = p.Np >> 4;
    const uint32_t KT = p.Kp >> 6;
    const bool vec_a = ((p.lda & 15u) == 0) && ((reinterpret_cast<uintptr_t>(p.A) & 15u) == 0);

    // A staging: 128 rows x 4 chunks of 16 B = 512 chunks, 2 per thread.
    const uint32_t ar0 = tid >> 2, ac = (tid & 3) * 16;
    const uint32_t ar1 = ar0 + 64;

    // B blocks this wave multiplies: n16 blocks nbase + j, j < 4.
    const uint32_t nbase = (n0 >> 4) + wn * 4;

    v4i acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (v4i){0, 0, 0, 0};

    auto load_b = [&](uint32_t kt, v4i (&b)[4], bool (&z)[4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t nb = nbase + j;
            z[j] = nb >= NT;
            b[j] = (v4i){0, 0, 0, 0};
            if (!z[j])
                b[j] = *reinterpret_cast<const v4i *>(p.frag + ((static_cast<uint64_t>(nb) * KT + kt) << 10) + lane * 16);
        }
    };

    v4i ra0 = load_a_chunk(p, m0 + ar0, ac, vec_a);
    v4i ra1 = load_a_chunk(p, m0 + ar1, ac, vec_a);
    v4i b[4];
    bool z[4];
    load_b(0, b, z);
    *reinterpret_cast<v4i *>(&a_lds[0][ar0 * kPitch + ac]) = ra0;
    *reinterpret_cast<v4i *>(&a_lds[0][ar1 * kPitch + ac]) = ra1;
    __syncthreads();

    const int fr = lane & 15, fg = lane >> 4;
    for (uint32_t kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        v4i nb[4];
        bool nz[4];
        const bool more = kt + 1 < KT;
        if (more) {
            ra0 = load_a_chunk(p, m0 + ar0, (kt + 1) * BK + ac, vec_a);
            ra1 = load_a_chunk(p, m0 + ar1, (kt + 1) * BK + ac, vec_a);
            load_b(kt + 1, nb, nz);
        }
        v4i a[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            a[i] = *reinterpret_cast<const v4i *>(&a_lds[cur][(wm * 64 + i * 16 + fr) * kPitch + fg * 16]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (z[j]) continue;  // wave-uniform
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            *reinterpret_cast<v4i *>(&a_lds[cur ^ 1][ar0 * kPitch + ac]) = ra0;
            *reinterpret_cast<v4i *>(&a_lds[cur ^ 1][ar1 * kPitch + ac]) = ra1;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                b[j] = nb[j];
                z[j] = nz[j];
            }
        }
        __syncthreads();
    }

    // Epilogue: lane holds rows 4*fg + r of column fr in each 16 x 16 block.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t n = n0 + wn * 64 + j * 16 + fr;
        if (n >= p.N) continue;
        const float sb = p.scale_b[n];
        const float bias = p.bias ? p.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t m = m0 + wm * 64 + i * 16 + fg * 4 + r;
                if (m >= p.M) continue;
                const float sa = p.scale_a ? p.scale_a[m] : 1.0f;
                float out = dev::mul_rn(dev::mul_rn(static_cast<float>(acc[i][j][r]), sa), sb);
                if (p.bias) out = dev::add_rn(out, bias);
                p.C[static_cast<uint64_t>(m) * p.ldc + n] = dev::epilogue(out, p.epilogue);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Pipelined kernel (K % 64 == 0, 16-byte aligned rows of A).
//
//   * workgroup tile 256 x 128, 4 waves of 128 x 64 (8 x 4 MFMA blocks, 32
//     independent accumulators per wave - enough to keep the matrix pipe
//     issuing back to back);
//   * a ring of kStages LDS stages, each holding one 64-deep k step of both
//     operands as 1 KiB fragment blocks (16 of A, 8 of B), filled by
//     global_load_lds_dwordx4: lane l of a wave writes bytes [16l, 16l+16) of
//     a block, so A is fetched directly in fragment order (lane l reads row
//     l%16, k 16*(l/16)..+16) and B is copied as packed;
//   * kStages-1 k steps of DMA are in flight; each wave waits with an
//     explicit vmcnt for only its own oldest stage and one s_barrier per k
//     step publishes it;
//   * fragments are software-pipelined through two register sets: the 12
//     ds_read_b128 of step k+1 are in flight while the 32 MFMAs of step k
//     issue, so LDS latency is hidden at one wave per SIMD;
//   * the accumulators leave through LDS: a compact loop then applies the
//     dequant epilogue with row-contiguous, coalesced stores (a fully
//     unrolled per-lane epilogue would be tens of KiB of code per wave);
//   * rows past M and column blocks past N are clamped to valid addresses
//     (their results are never stored), so every DMA stays in bounds.
// ---------------------------------------------------------------------------
namespace pipe {
constexpr int TM = 256, TN = 128;
constexpr int kStages = 6;
constexpr int kABlocks = TM / 16;                    // 16
constexpr int kBBlocks = TN / 16;                    // 8
constexpr int kBlocks = kABlocks + kBBlocks;         // 24 x 1 KiB per stage
constexpr int kLoads = kBlocks / 4;                  // per wave per stage
constexpr int kStageBytes = kBlocks * 1024;
constexpr int kRing = kStages * kStageBytes;         // 144 KiB
constexpr int kOutPitch = TN + 4;                    // int32 per staged row (pad vs bank conflicts)
constexpr int kOut = TM * kOutPitch * 4;             // 132 KiB, row-major staged tile
constexpr int kScaleOff = kOut;                      // 256 row scales after the tile
constexpr size_t kLds = kRing;                       // 144 KiB (>= kOut + 1 KiB)
static_assert(kOut + TM * 4 <= kRing, "staged tile + row scales fit in the ring");
}  // namespace pipe

using lds::block_barrier;
using lds::dma16;
using lds::dma16_s;
using lds::wait_vmcnt;
using lds::waitcnt_imm;

typedef int v16i __attribute__((ext_vector_type(16)));

// One stage's operands for v_mfma_i32_32x32x32_i8, per 32-deep k half h:
// lane l holds row (col) l%32 and k 16*(l/32)..+16 of that half.
struct Frags {
    v4i a[2][4], b[2][2];
};

// Dequant epilogue over a row-major staged tile of kRows x kCols int32 (row
// pitch kPitch): each thread writes 4 consecutive columns per row (one
// 16-byte store), kT/(kCols/4) rows per pass.  One instantiation per
// activation keeps the loop body small.  No contraction:
// ((float)acc * sa) * sb + bias rounds each step, as the reference's
// store_i8_c does.
template <int EPI, int kT = kThreads, int kCols = pipe::TN, int kPitch = pipe::kOutPitch, int kRows = pipe::TM>
__device__ void store_tile(const I8Gemm &p, const int32_t *tile, const float *sa_lds, uint32_t m0,
                           uint32_t n0, int tid)
{
#pragma clang fp contract(off)
    constexpr int kPerRow = kCols / 4;   // threads per row
    constexpr int kRowStep = kT / kPerRow;
    if (tid >= kRowStep * kPerRow) return;    // kT need not be a multiple of kPerRow
    const uint32_t c4 = (tid % kPerRow) * 4;  // first of this thread's 4 columns
    const uint32_t n = n0 + c4;
    float sb[4], bias[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const bool ok = n + q < p.N;
        sb[q] = ok ? p.scale_b[n + q] : 0.0f;
        bias[q] = (ok && p.bias) ? p.bias[n + q] : 0.0f;
    }
    const bool vec = (n + 3 < p.N) && ((p.ldc & 3u) == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 15u) == 0);
    const uint32_t rows = min(static_cast<uint32_t>(kRows), p.M - m0);
#pragma unroll 4
    for (uint32_t r = tid / kPerRow; r < rows; r += kRowStep) {
        const v4i acc = *reinterpret_cast<const v4i *>(tile + r * kPitch + c4);
        const float sa = sa_lds[r];
        float o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float v = (static_cast<float>(acc[q]) * sa) * sb[q];
            if (p.bias) v = v + bias[q];
            o[q] = dev::epilogue(v, EPI);
        }
        float *dst = p.C + static_cast<uint64_t>(m0 + r) * p.ldc + n;
        if (vec) {
            // Streaming store: C is written once and not re-read by this kernel.
            __builtin_nontemporal_store((v4f){o[0], o[1], o[2], o[3]}, reinterpret_cast<v4f *>(dst));
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (n + q < p.N) dst[q] = o[q];
        }
    }
}

__global__ __launch_bounds__(kThreads) void gemm_i8_pipe(I8Gemm p, uint32_t tiles_m, uint32_t tiles_n)
{
    using pipe::kABlocks;
    using pipe::kBBlocks;
    using pipe::kLoads;
    using pipe::kStageBytes;
    using pipe::kStages;
    extern __shared__ __attribute__((aligned(1024))) int8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 15, fg = lane >> 4;

    // XCD-aware tile order: workgroup g runs on XCD g % 8; give each XCD a
    // contiguous run of tiles, M-fastest, so an XCD's L2 keeps its B columns.
    const uint32_t total = tiles_m * tiles_n;
    uint32_t g = blockIdx.x;
    if ((total & 7u) == 0) g = (g & 7u) * (total >> 3) + (g >> 3);
    const uint32_t tmi = g % tiles_m, tni = g / tiles_m;
    const uint32_t m0 = tmi * pipe::TM, n0 = tni * pipe::TN;
    const uint32_t NT = p.Np >> 4;
    const uint32_t KT = p.K >> 6;

    // This wave's kLoads blocks of every stage: base address + per-k-step stride.
    const int8_t *src[kLoads];
    uint64_t stride[kLoads];
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const int b = wave * kLoads + j;
        if (b < kABlocks) {
            const uint32_t row = min(m0 + b * 16 + fr, p.M - 1);
            src[j] = p.A + static_cast<uint64_t>(row) * p.lda + fg * 16;
            stride[j] = 64;
        } else {
            const uint32_t nb = min((n0 >> 4) + (b - kABlocks), NT - 1);
            src[j] = p.frag + ((static_cast<uint64_t>(nb) * (p.Kp >> 6)) << 10) + lane * 16;
            stride[j] = 1024;
        }
    }
    auto issue = [&](uint32_t kt) {
        int8_t *st = smem + (kt % kStages) * kStageBytes;
#pragma unroll
        for (int j = 0; j < kLoads; ++j) dma16(src[j] + kt * stride[j], st + (wave * kLoads + j) * 1024);
    };
    // A 32-row (32-column) operand is two 16-row fragment blocks of the
    // stage: lane l takes block (l/16)%2, row l%16, k group 2h + l/32.
    const int sub = (lane >> 4) & 1;
    auto read_frags = [&](uint32_t kt, Frags &f) {
        const int8_t *st = smem + (kt % kStages) * kStageBytes;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int off = ((2 * h + (lane >> 5)) * 16 + (lane & 15)) * 16;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
                f.b[h][nb] = *reinterpret_cast<const v4i *>(st + (kABlocks + wn * 4 + 2 * nb + sub) * 1024 + off);
#pragma unroll
            for (int mb = 0; mb < 4; ++mb)
                f.a[h][mb] = *reinterpret_cast<const v4i *>(st + (wm * 8 + 2 * mb + sub) * 1024 + off);
        }
    };

    v16i acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (v16i){0};

    // 32x32x32 rather than 16x16x64: at one wave per SIMD it keeps the int8
    // matrix pipe ~85% busy where the 16x16 shape issues at ~55%.
    auto mma = [&](const Frags &f) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[h][i], f.b[h][j], acc[i][j], 0, 0, 0);
    };

    // Prologue: DMA every stage buffer, then stage 0's fragments.
    const uint32_t pre = min(KT, static_cast<uint32_t>(kStages));
    for (uint32_t s = 0; s < pre; ++s) issue(s);
    if (KT > static_cast<uint32_t>(kStages)) wait_vmcnt<(kStages - 1) * kLoads>();
    else wait_vmcnt<0>();
    block_barrier();
    Frags f0, f1;
    read_frags(0, f0);

    // Steady state, two k steps per trip so the fragment sets swap without
    // copies, and no branch around the MFMAs.  Step kt: wait for this wave's
    // DMA of stage kt+1 (kStages-2 later stages may stay in flight), barrier
    // (stage kt+1 landed everywhere; every wave holds stage kt in registers,
    // so its buffer is free), DMA stage kt+kStages into it, read stage kt+1,
    // then issue stage kt's 32 MFMAs.
    // sched_barrier(0) keeps the three phases of a step in order: the
    // compiler would otherwise pull the next stage's reads into the MFMA
    // sequence and stall it on lgkmcnt.
    uint32_t kt = 0;
    for (; kt + kStages + 1 < KT; kt += 2) {
        wait_vmcnt<(kStages - 2) * kLoads>();
        block_barrier();
        issue(kt + kStages);
        read_frags(kt + 1, f1);
        __builtin_amdgcn_sched_barrier(0);
        mma(f0);
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<(kStages - 2) * kLoads>();
        block_barrier();
        issue(kt + 1 + kStages);
        read_frags(kt + 2, f0);
        __builtin_amdgcn_sched_barrier(0);
        mma(f1);
        __builtin_amdgcn_sched_barrier(0);
    }
    // Drain.  The loop has issued stages up to kt + 5; with an odd KT (every
    // K % 128 == 64 this kernel takes) stage kt + 6 = KT - 1 is still to be
    // copied, into the slot of stage kt once every wave has read stage kt's
    // fragments.  Then wait for all of it once.
    if (kt + kStages < KT) {
        block_barrier();
        issue(kt + kStages);
    }
    wait_vmcnt<0>();
    block_barrier();
    mma(f0);
    for (++kt; kt < KT; ++kt) {
        read_frags(kt, f1);
        mma(f1);
    }

    // Stage the accumulators row-major (32x32 block: lane l holds column
    // l%32, rows 8j + 4(l/32) + q in register 4j + q) and the row scales.
    __syncthreads();
    int32_t *tile = reinterpret_cast<int32_t *>(smem);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                tile[(wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * pipe::kOutPitch + wn * 64 +
                     j * 32 + (lane & 31)] = acc[i][j][r];
    float *sa_lds = reinterpret_cast<float *>(smem + pipe::kScaleOff);
    {
        const uint32_t m = m0 + tid;
        sa_lds[tid] = (p.scale_a && m < p.M) ? p.scale_a[m] : 1.0f;
    }
    __syncthreads();
    switch (p.epilogue) {
    case 1: store_tile<1>(p, tile, sa_lds, m0, n0, tid); break;
    case 2: store_tile<2>(p, tile, sa_lds, m0, n0, tid); break;
    case 3:
    case 4: store_tile<3>(p, tile, sa_lds, m0, n0, tid); break;
    default: store_tile<0>(p, tile, sa_lds, m0, n0, tid); break;
    }
}

// ---------------------------------------------------------------------------
// Strip kernel for weights with all-zero 64 x 64 tiles (the Wildcat cull
// geometry of config 5; the reference's int8 culled tile, kernels.cpp:927-931,
// is never reached).  A workgroup owns TM = 512 rows x one group of four
// 16-column strips (64 columns) and walks only that group's nonzero 64-deep
// k blocks, from the list built at pack time (tile_lists): stage s holds
// k block list[s] of both operands, A gathered from its 64 columns, so a
// zero tile costs neither copies nor MFMAs, and every wave of the workgroup
// takes the same stages (no per-MFMA test).  Otherwise the pipelined
// kernel's scheme: 8 waves of 64 x 64 (2 x 2 v_mfma_i32_32x32x32_i8 blocks;
// two waves per SIMD, so one wave's stage overhead overlaps the other's
// MFMAs), stages copied into an LDS ring by global_load_lds_dwordx4 (A from
// its fragment-block copy, B as packed), three stages in flight, fragments
// double-buffered in registers, the accumulators leaving through LDS for the
// dequant epilogue.
// The list sits in registers: lane l holds entry 64q + l of register q, and a
// stage's k block is a readlane, so no load waits on it.
// ---------------------------------------------------------------------------
// A in fragment blocks for the strip kernel: block (rb, kb) is 1 KiB, lane
// l's 16 bytes = A[16 rb + l % 16][64 kb + 16 (l / 16) .. +16] (rows past M
// zero), so a stage's copy of a 16-row block is one contiguous 1 KiB read
// (whole cache lines) instead of 16 half lines of row-major A.
__global__ __launch_bounds__(256) void a_blocks_kernel(const int8_t *__restrict__ A, uint32_t lda, uint32_t M,
                                                       uint32_t KTp, uint64_t chunks, int8_t *__restrict__ out)
{
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= chunks) return;
    const uint32_t l = idx & 63;
    const uint64_t blk = idx >> 6;
    const uint32_t kb = static_cast<uint32_t>(blk % KTp), rb = static_cast<uint32_t>(blk / KTp);
    const uint32_t row = rb * 16 + (l & 15);
    v4i v = {0, 0, 0, 0};
    if (row < M) v = *reinterpret_cast<const v4i *>(A + static_cast<uint64_t>(row) * lda + kb * 64 + (l >> 4) * 16);
    reinterpret_cast<v4i *>(out)[idx] = v;
}

namespace strip {
constexpr int TM = 512, TN = 64;
constexpr int kStages = 4;
constexpr int kABlocks = TM / 16;                    // 32
constexpr int kBBlocks = TN / 16;                    // 4
constexpr int kBlocks = kABlocks + kBBlocks;         // 36 x 1 KiB per stage
constexpr int kThreads = 512;                        // 8 waves
constexpr int kLoadsLo = 5, kLoadsHi = 4;            // copies per stage: waves 0-3, waves 4-7
constexpr int kStageBytes = kBlocks * 1024;
constexpr int kRing = kStages * kStageBytes;         // 144 KiB
constexpr int kOutPitch = TN + 4;
constexpr int kOut = TM * kOutPitch * 4;             // 136 KiB
constexpr int kScaleOff = kOut;
constexpr uint32_t kMaxKBlocks = 256;                // list registers: 4 x 64
constexpr size_t kLds = kRing;
static_assert(kOut + TM * 4 <= kRing, "staged tile + row scales fit in the ring");
static_assert(4 * kLoadsLo + 4 * kLoadsHi == kBlocks, "every block of a stage has one copy");
}  // namespace strip

__global__ __launch_bounds__(strip::kThreads) void gemm_i8_strip(I8Gemm p, uint32_t tiles_m, uint32_t groups,
                                                                 const int8_t *__restrict__ ablk)
{
    using strip::kABlocks;
    using strip::kLoadsHi;
    using strip::kLoadsLo;
    using strip::kStageBytes;
    using strip::kStages;
    extern __shared__ __attribute__((aligned(1024))) int8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // XCD-aware order: each XCD takes a contiguous run of tiles, column
    // groups fastest, so its L2 keeps the run's row tiles of A (512 rows x K)
    // while the groups' weights stream past.
    const uint32_t total = tiles_m * groups;
    uint32_t g = blockIdx.x;
    if ((total & 7u) == 0) g = (g & 7u) * (total >> 3) + (g >> 3);
    const uint32_t tmi = g / groups, grp = g % groups;
    const uint32_t m0 = tmi * strip::TM, n0 = grp * strip::TN;
    const uint32_t NT = p.Np >> 4;
    const uint32_t KTp = p.Kp >> 6;
    const uint32_t NS = p.nz_count[grp];   // stages: the group's nonzero k blocks
    const uint32_t *lst = p.nz_list + static_cast<uint64_t>(grp) * KTp;
    uint32_t lv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t i = 64u * q + lane;
        lv[q] = i < NS ? lst[i] : 0u;
    }
    auto kblock = [&](uint32_t s) -> uint32_t {
        const uint32_t q = s >> 6;
        const uint32_t v = q == 0 ? lv[0] : q == 1 ? lv[1] : q == 2 ? lv[2] : lv[3];
        return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), static_cast<int>(s & 63)));
    };

    // This wave's blocks of every stage (5 for waves 0-3, 4 for waves 4-7):
    // a block's run of k blocks (A blocks and packed B strips are both
    // k-block-major, 1 KiB apart).  The fifth slot of waves 4-7 is unused.
    const bool lo = wave < 4;
    const int b0 = lo ? wave * kLoadsLo : 4 * kLoadsLo + (wave - 4) * kLoadsHi;
    const int8_t *src[kLoadsLo];
#pragma unroll
    for (int j = 0; j < kLoadsLo; ++j) {
        const int b = min(b0 + j, strip::kBlocks - 1);
        if (b < kABlocks) {
            const uint32_t rb = min((m0 >> 4) + b, (p.M + 15) / 16 - 1);
            src[j] = ablk + ((static_cast<uint64_t>(rb) * KTp) << 10) + lane * 16;
        } else {
            const uint32_t nb = min((n0 >> 4) + (b - kABlocks), NT - 1);
            src[j] = p.frag + ((static_cast<uint64_t>(nb) * KTp) << 10) + lane * 16;
        }
    }
    auto issue = [&](uint32_t s) {
        int8_t *st = smem + (s % kStages) * kStageBytes;
        const uint64_t kb = kblock(s);
#pragma unroll
        for (int j = 0; j < kLoadsHi; ++j) dma16(src[j] + (kb << 10), st + (b0 + j) * 1024);
        if (lo) dma16(src[kLoadsHi] + (kb << 10), st + (b0 + kLoadsHi) * 1024);
    };
    // Waits for all but this wave's last n stages of copies.
    auto wait_stages = [&](auto n) {
        constexpr int N = decltype(n)::value;
        if (lo) wait_vmcnt<N * kLoadsLo>();
        else wait_vmcnt<N * kLoadsHi>();
    };
    // A 32-row (32-column) operand is two 16-row fragment blocks of the
    // stage: lane l takes block (l/16)%2, row l%16, k group 2h + l/32.
    const int sub = (lane >> 4) & 1;
    struct SFrags {
        v4i a[2][2], b[2][2];
    };
    auto read_frags = [&](uint32_t s, SFrags &f) {
        const int8_t *st = smem + (s % kStages) * kStageBytes;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int off = ((2 * h + (lane >> 5)) * 16 + (lane & 15)) * 16;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
                f.b[h][nb] = *reinterpret_cast<const v4i *>(st + (kABlocks + 2 * nb + sub) * 1024 + off);
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
                f.a[h][mb] = *reinterpret_cast<const v4i *>(st + (wave * 4 + 2 * mb + sub) * 1024 + off);
        }
    };

    v16i acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (v16i){0};
    auto mma = [&](const SFrags &f) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[h][i], f.b[h][j], acc[i][j], 0, 0, 0);
    };

    if (NS) {
        // The pipelined kernel's schedule over the NS listed stages.
        const uint32_t pre = min(NS, static_cast<uint32_t>(kStages));
        for (uint32_t s = 0; s < pre; ++s) issue(s);
        if (NS > static_cast<uint32_t>(kStages)) wait_stages(std::integral_constant<int, kStages - 1>{});
        else wait_vmcnt<0>();
        block_barrier();
        SFrags f0, f1;
        read_frags(0, f0);
        uint32_t s = 0;
        for (; s + kStages + 1 < NS; s += 2) {
            wait_stages(std::integral_constant<int, kStages - 2>{});
            block_barrier();
            issue(s + kStages);
            read_frags(s + 1, f1);
            __builtin_amdgcn_sched_barrier(0);
            mma(f0);
            __builtin_amdgcn_sched_barrier(0);
            wait_stages(std::integral_constant<int, kStages - 2>{});
            block_barrier();
            issue(s + 1 + kStages);
            read_frags(s + 2, f0);
            __builtin_amdgcn_sched_barrier(0);
            mma(f1);
            __builtin_amdgcn_sched_barrier(0);
        }
        // Drain: at most stage s + kStages is still to be copied, into the
        // slot of stage s once every wave holds stage s's fragments.
        if (s + kStages < NS) {
            block_barrier();
            issue(s + kStages);
        }
        wait_vmcnt<0>();
        block_barrier();
        mma(f0);
        for (++s; s < NS; ++s) {
            read_frags(s, f1);
            mma(f1);
        }
    }

    // Stage the accumulators row-major (32x32 block: lane l holds column
    // l%32, rows 8j + 4(l/32) + q in register 4j + q) and the row scales.
    __syncthreads();
    int32_t *tile = reinterpret_cast<int32_t *>(smem);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                tile[(wave * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * strip::kOutPitch + j * 32 +
                     (lane & 31)] = acc[i][j][r];
    float *sa_lds = reinterpret_cast<float *>(smem + strip::kScaleOff);
    for (int r = tid; r < strip::TM; r += strip::kThreads) {
        const uint32_t m = m0 + r;
        sa_lds[r] = (p.scale_a && m < p.M) ? p.scale_a[m] : 1.0f;
    }
    __syncthreads();
    using strip::kOutPitch;
    using strip::TM;
    using strip::TN;
    constexpr int kT = strip::kThreads;
    switch (p.epilogue) {
    case 1: store_tile<1, kT, TN, kOutPitch, TM>(p, tile, sa_lds, m0, n0, tid); break;
    case 2: store_tile<2, kT, TN, kOutPitch, TM>(p, tile, sa_lds, m0, n0, tid); break;
    case 3:
    case 4: store_tile<3, kT, TN, kOutPitch, TM>(p, tile, sa_lds, m0, n0, tid); break;
    default: store_tile<0, kT, TN, kOutPitch, TM>(p, tile, sa_lds, m0, n0, tid); break;
    }
}

// ---------------------------------------------------------------------------
// 128-deep LDS stages (K % 128 == 0) for the 256 x 128 tile: each stage holds
// a 128-deep k slab, so every row of A is fetched as one full 128-byte line
// (64-deep stages fetched half lines and doubled the L2 requests for A):
//   * stage = A 256 rows x 128 B (32 KiB) + B 16 fragment blocks (2 k
//     blocks x 8 column blocks, 16 KiB); 3 stages = 144 KiB of LDS;
//   * one DMA instruction moves 8 rows of A (lane l: row l/8, 16-byte slot
//     l%8); the lane fetches k chunk slot ^ ((row >> 1) & 7), so chunk c of
//     row r sits at r*128 + 16*(c ^ ((r >> 1) & 7)) and the fragment reads
//     (16 rows at one chunk per quarter wave) hit 16 distinct bank groups.
// ---------------------------------------------------------------------------
namespace pipe128 {
constexpr int TM = 256, TN = 128, SK = 128;  // k depth of one stage
constexpr int kStages = 3;
constexpr int kAInstr = TM / 8;                      // 32 x 1 KiB of A per stage
constexpr int kBInstr = (TN / 16) * (SK / 64);       // 16 x 1 KiB of B per stage
constexpr int kStageBytes = (kAInstr + kBInstr) * 1024;  // 48 KiB
constexpr int kBOff = kAInstr * 1024;
constexpr size_t kLds = static_cast<size_t>(kStages) * kStageBytes;  // 144 KiB
static_assert(pipe::kOut + TM * 4 <= static_cast<int>(kLds), "staged tile + row scales fit");
}  // namespace pipe128

// ---------------------------------------------------------------------------
// Two waves per SIMD (K % 128 == 0): the 256 x 128 tile over the 128-deep
// LDS stages above, with 8 waves.  Waves w and w+4 own the same
// 128 x 64 output block and split every stage by k half (wave group gk takes
// the 64-deep half gk), so LDS traffic per MFMA is unchanged while each SIMD
// has a second wave to issue MFMAs whenever the other waits on its fragment
// reads or the barrier.  The two partial accumulators are summed through LDS
// (exact int32) before the shared epilogue.
//   * 3 LDS stages; stage s+3 is copied while stage s is multiplied (two
//     stages in flight); each wave issues 6 of the 48 DMA instructions of a
//     stage;
//   * per stage and wave: vmcnt wait for its own copy of the stage to be
//     read, one barrier, 12 fragment reads, 16 MFMAs that each wait only
//     for their own operands.
// ---------------------------------------------------------------------------
namespace w8 {
constexpr int kThreads8 = 512;
constexpr int kAPer = 4;                 // A DMA instructions per wave per stage
constexpr int kBPer = 2;                 // B DMA instructions per wave per stage
constexpr int kLoads = kAPer + kBPer;
constexpr int kStages = pipe128::kStages;
}  // namespace w8

// ---------------------------------------------------------------------------
// Epilogue from registers (8-wave and wide tiles).  A 32 x 32 MFMA
// accumulator leaves column l % 32 and rows 8q + 4(l / 32) + rr in register
// 4q + rr of lane l, so one dword store covers 32 columns of two rows (two
// full 128-byte lines).  The stores go through a buffer over the wave's 128
// rows of C: rows past M fall outside it and columns past N get an offset
// past its end, so the buffer's range check drops out-of-range results
// without branches (the whole offset is in the per-lane operand, which the
// range check covers).  Needs
// ldc <= kRegStoreMaxLdc (128 rows of C within a 31-bit byte range).
// ---------------------------------------------------------------------------
constexpr uint32_t kRegStoreMaxLdc = (1u << 22) - 1;
constexpr int kCBufferWord3 = 0x00020000;   // raw buffer, 32-bit data format
constexpr int kCStorePolicy = 2;            // nontemporal: C is written once
constexpr uint32_t kDropOffset = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t c_rows(const I8Gemm &p, uint32_t mrow)
{
    const uint32_t rows = mrow < p.M ? min(128u, p.M - mrow) : 0u;
    return __builtin_amdgcn_make_buffer_rsrc(p.C + static_cast<uint64_t>(mrow) * p.ldc, 0,
                                             static_cast<int>(rows * p.ldc * 4u), kCBufferWord3);
}

// Column scales and bias of the NB 32-column tiles of lane l (column ncol +
// 32j), and the lane's store offsets (row half l / 32 included).
template <int NB>
struct ColEpi {
    float sb[NB], bias[NB];
    uint32_t off[NB];
    __device__ __forceinline__ ColEpi(const I8Gemm &p, uint32_t ncol, int lane)
    {
        const uint32_t h4 = static_cast<uint32_t>(lane >> 5) * 4u;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const uint32_t n = ncol + 32 * j;
            const bool ok = n < p.N;
            sb[j] = ok ? p.scale_b[n] : 0.0f;
            bias[j] = (ok && p.bias) ? p.bias[n] : 0.0f;
            off[j] = ok ? (h4 * p.ldc + n) * 4u : kDropOffset;
        }
    }
};

// Row tiles I0 .. I0+NI-1 of a wave's accumulators (plus, with kXch, the
// partner wave's partial sums of the same tiles from LDS), stored in the
// reference's order ((float)acc * sa) * sb + bias -> epi.  sa: the row scales
// of the wave's 128 rows (LDS).
template <int EPI, int NB, int I0, int NI, bool kXch>
__device__ __forceinline__ void reg_store(const I8Gemm &p, const v16i (&acc)[4][NB], const v4i *theirs,
                                          const float *sa, uint32_t mrow, const ColEpi<NB> &ce, int lane)
{
#pragma clang fp contract(off)
    const __amdgpu_buffer_rsrc_t rs = c_rows(p, mrow);
    const uint32_t ld4 = p.ldc * 4u;
    const int h = lane >> 5;
#pragma unroll
    for (int ii = 0; ii < NI; ++ii)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r0 = (I0 + ii) * 32 + 8 * q;
            const v4f s4 = *reinterpret_cast<const v4f *>(sa + r0 + 4 * h);
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                v4i o = (v4i){0, 0, 0, 0};
                if (kXch) o = theirs[((ii * NB + j) * 4 + q) * 64 + lane];
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int32_t v = acc[I0 + ii][j][4 * q + rr] + o[rr];
                    float f = (static_cast<float>(v) * s4[rr]) * ce.sb[j];
                    if (p.bias) f = f + ce.bias[j];
                    f = dev::epilogue(f, EPI);
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, f), rs,
                                                          static_cast<int>(ce.off[j] + (r0 + rr) * ld4), 0,
                                                          kCStorePolicy);
                }
            }
        }
}

// Epilogue exchange of the 8-wave tile: a wave's two MFMA row tiles x two
// column tiles x 16 accumulators, as [tile][column tile][4 registers][lane]
// 16-byte slots (lane-contiguous, so conflict-free), 16 KiB per wave.
constexpr int kXchBytes = 2 * 2 * 4 * 64 * 16;
static_assert(8 * kXchBytes + pipe128::TM * 4 <= static_cast<int>(pipe128::kLds), "exchange + row scales fit");

template <int I0>
__device__ __forceinline__ void xchg_put(const v16i (&acc)[4][2], v4i *dst, int lane)
{
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const v16i &a = acc[I0 + ii][j];
                dst[((ii * 2 + j) * 4 + q) * 64 + lane] = (v4i){a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]};
            }
}

__global__ __launch_bounds__(w8::kThreads8) void gemm_i8_k128w8(I8Gemm p, uint32_t tiles_m, uint32_t tiles_n)
{
    using pipe128::kBOff;
    using pipe128::kStageBytes;
    using pipe128::SK;
    using pipe128::TM;
    using pipe128::TN;
    using w8::kAPer;
    using w8::kBPer;
    using w8::kLoads;
    using w8::kStages;
    extern __shared__ __attribute__((aligned(1024))) int8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gk = wave >> 2;                    // k half of every stage
    const int wm = (wave >> 1) & 1, wn = wave & 1;

    const uint32_t total = tiles_m * tiles_n;
    uint32_t g = blockIdx.x;
    if ((total & 7u) == 0) g = (g & 7u) * (total >> 3) + (g >> 3);
    const uint32_t tmi = g % tiles_m, tni = g / tiles_m;
    const uint32_t m0 = tmi * TM, n0 = tni * TN;
    const uint32_t NT = p.Np >> 4;
    const uint32_t KS = p.K / SK;
    const uint64_t KTp = p.Kp >> 6;

    // Fragment reads of half gk of a stage, in MFMA consumption order.
    const int sub = (lane >> 4) & 1;
    int a_off[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
        const uint32_t r = wm * 128 + mb * 32 + (lane & 31);
        a_off[mb] = r * 128;
    }

    v16i acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (v16i){0};

    // Software-pipelined: stage s's 16 MFMAs run from fragments read
    // during stage s-1; after the first four, one wait + barrier makes
    // stage s+1 visible (its copy was issued two stages earlier; stage
    // s+2's copy stays in flight), and the remaining twelve MFMA slots
    // each carry one fragment read of stage s+1 and, in the first six,
    // one copy instruction of stage s+3.  That copy refills the ring slot
    // of stage s itself: every wave read stage s's fragments during stage
    // s-1 and waited for them before this barrier.
    //
    // Copy addresses: wave-uniform bases (SGPRs, advanced per stage by
    // scalar adds) plus one 32-bit per-lane offset each.  A instruction j
    // copies rows rb .. rb+7 (rb = 8(4 wave + j) in the tile); lane rows
    // past M are clamped to M - 1 and so is the base row, so a lane's
    // offset stays below 8 lda.
    const int8_t *a_base[kAPer];
    uint32_t a_lo[kAPer];
#pragma unroll
    for (int j = 0; j < kAPer; ++j) {
        const uint32_t rb = (wave * kAPer + j) * 8;
        const uint32_t r = rb + (lane >> 3);
        const uint32_t brow = min(m0 + rb, p.M - 1);
        const uint32_t row = min(m0 + r, p.M - 1);
        a_base[j] = p.A + static_cast<uint64_t>(brow) * p.lda;
        a_lo[j] = (row - brow) * p.lda + 16 * ((lane & 7) ^ ((r >> 1) & 7));
    }
    const int8_t *b_base[kBPer];
#pragma unroll
    for (int j = 0; j < kBPer; ++j) {
        const int bi = wave * kBPer + j;
        const uint32_t nb = min((n0 >> 4) + (bi >> 1), NT - 1);
        b_base[j] = p.frag + ((static_cast<uint64_t>(nb) * KTp + (bi & 1)) << 10);
    }
    const uint32_t b_lo = lane * 16;
    // Copy instruction j of stage st_i into ring slot `slot`.
    auto issue_one = [&](uint32_t st_i, uint32_t slot, int j) {
        int8_t *st = smem + slot * kStageBytes;
        if (j < kAPer)
            dma16_s(a_base[j] + st_i * SK, a_lo[j], st + (wave * kAPer + j) * 1024);
        else
            dma16_s(b_base[j - kAPer] + static_cast<uint64_t>(st_i) * 2048, b_lo,
                    st + kBOff + (wave * kBPer + j - kAPer) * 1024);
    };
    auto read_one = [&](uint32_t slot, Frags &f, int k) {
        const int8_t *st = smem + slot * kStageBytes;
        const int h = k / 6, r = k % 6;
        if (r == 0 || r == 5) {
            const int nb = r == 5;
            const int boff = kBOff + (((wn * 4 + sub) * 2 + gk) << 10) +
                             (((2 * h + (lane >> 5)) * 16 + (lane & 15)) << 4);
            f.b[h][nb] = *reinterpret_cast<const v4i *>(st + boff + nb * 2 * 2 * 1024);
        } else {
            const int mb = r - 1;
            const uint32_t row = wm * 128 + mb * 32 + (lane & 31);
            const uint32_t c = 4 * gk + 2 * h + (lane >> 5);
            f.a[h][mb] = *reinterpret_cast<const v4i *>(st + a_off[mb] + ((c ^ ((row >> 1) & 7)) << 4));
        }
    };
    // Stage s: multiply `cur`, read stage s+1 (ring slot rd) into `nxt`
    // and copy stage s+3 into ring slot s % 3 (cp).  more: s+1 < KS;
    // ahead: stage s+2 was copied (s+2 < KS), so its copy may stay in
    // flight while stage s+1's is waited for; dma: s+3 < KS.  All three
    // are compile-time true in the steady-state loops, which then have no
    // branch.
    auto step = [&](const Frags &cur, Frags &nxt, uint32_t s, uint32_t rd, uint32_t cp, bool more, bool ahead,
                    bool dma) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int h = k >> 3, j = (k >> 2) & 1, i = k & 3;
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.a[h][i], cur.b[h][j], acc[i][j], 0, 0, 0);
            if (k == 3 && more) {
                if (ahead)
                    wait_vmcnt<kLoads>();
                else
                    wait_vmcnt<0>();
                block_barrier();
            }
            if (k >= 4 && more) {
                if (dma && k - 4 < kLoads) issue_one(s + 3, cp, k - 4);
                read_one(rd, nxt, k - 4);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    Frags f0, f1;
    const uint32_t pre = min(KS, static_cast<uint32_t>(kStages));
    for (uint32_t st_i = 0; st_i < pre; ++st_i) {
#pragma unroll
        for (int j = 0; j < kLoads; ++j) issue_one(st_i, st_i, j);
    }
    if (pre == 3)
        wait_vmcnt<2 * kLoads>();
    else if (pre == 2)
        wait_vmcnt<kLoads>();
    else
        wait_vmcnt<0>();
    block_barrier();
#pragma unroll
    for (int k = 0; k < 12; ++k) read_one(0, f0, k);
    // Six stages per trip (a multiple of both the ring depth and the two
    // fragment sets), so every ring slot is a constant; then pairs of
    // stages with every flag still true; then the last stages.
    uint32_t s = 0;
    for (; s + 8 < KS; s += 6) {
        step(f0, f1, s, 1, 0, true, true, true);
        step(f1, f0, s + 1, 2, 1, true, true, true);
        step(f0, f1, s + 2, 0, 2, true, true, true);
        step(f1, f0, s + 3, 1, 0, true, true, true);
        step(f0, f1, s + 4, 2, 1, true, true, true);
        step(f1, f0, s + 5, 0, 2, true, true, true);
    }
    for (; s + 4 < KS; s += 2) {
        step(f0, f1, s, (s + 1) % kStages, s % kStages, true, true, true);
        step(f1, f0, s + 1, (s + 2) % kStages, (s + 1) % kStages, true, true, true);
    }
    for (; s + 1 < KS; s += 2) {
        step(f0, f1, s, (s + 1) % kStages, s % kStages, true, s + 2 < KS, s + 3 < KS);
        step(f1, f0, s + 1, (s + 2) % kStages, (s + 1) % kStages, s + 2 < KS, s + 3 < KS, s + 4 < KS);
    }
    if (s < KS) step(f0, f1, s, 0, 0, false, false, false);

    // Waves w and w+4 hold the two k halves of the same 128 x 64 block.
    // Wave group gk finishes MFMA row tiles 2gk and 2gk+1: it hands the other
    // two tiles' partial sums to its partner through LDS and takes the
    // partner's partials of its own two, then converts and stores them from
    // registers.  One exchange barrier, half the tile through LDS each way.
    const ColEpi<2> ce(p, n0 + wn * 64 + (lane & 31), lane);
    const float sa_g = (tid < TM && p.scale_a && m0 + tid < p.M) ? p.scale_a[m0 + tid] : 1.0f;
    __syncthreads();   // every wave's last fragment reads are done: the ring is free
    v4i *xch = reinterpret_cast<v4i *>(smem);                      // [wave][2 x 2 x 4][64 lanes]
    float *sa_lds = reinterpret_cast<float *>(smem + 8 * kXchBytes);
    if (gk == 0)
        xchg_put<2>(acc, xch + wave * (kXchBytes / 16), lane);
    else
        xchg_put<0>(acc, xch + wave * (kXchBytes / 16), lane);
    if (tid < TM) sa_lds[tid] = sa_g;
    __syncthreads();
    const v4i *theirs = xch + (wave ^ 4) * (kXchBytes / 16);
    const float *sa = sa_lds + wm * 128;
    const uint32_t mrow = m0 + wm * 128;
#define VNPU_W8_STORE(E)                                                   \
    (gk ? reg_store<E, 2, 2, 2, true>(p, acc, theirs, sa, mrow, ce, lane) \
        : reg_store<E, 2, 0, 2, true>(p, acc, theirs, sa, mrow, ce, lane))
    switch (p.epilogue) {
    case 1: VNPU_W8_STORE(1); break;
    case 2: VNPU_W8_STORE(2); break;
    case 3:
    case 4: VNPU_W8_STORE(3); break;
    default: VNPU_W8_STORE(0); break;
    }
#undef VNPU_W8_STORE
}

// ---------------------------------------------------------------------------
// Wide tiles (K % 128 == 0, dense weights, M % 256 == 0): 256 x TN per
// workgroup with TN = 256 or 192, 4 waves of 128 x TN/2 (4 x TN/64 MFMA
// tiles; 256 or 192 accumulator registers at one wave per SIMD).  Per MFMA
// the 256 x 256 tile copies a third fewer bytes from L2 into LDS and reads a
// third fewer fragment bytes from LDS than the 256 x 128 tile; 256 x 192 sits
// between them and fills whole rounds of 256 CUs where 256-wide tiles leave a
// half-empty last round (N = 11008 and 12288 at M = 2048).
//   * stage = A 256 x 128 B (32 KiB, swizzled as above) + B TN/8 fragment
//     blocks (TN/16 column blocks x 2 k blocks); 2 stages (128 or 112 KiB);
//   * per stage: the MFMAs of k half 0 with half 1's fragment reads threaded
//     between them; vmcnt(0) (stage s+1 landed) and one barrier (stage s
//     fully read); the MFMAs of half 1 with stage s+2's DMA instructions and
//     stage s+1's half-0 reads threaded between them;
//   * the epilogue stores each wave's block from registers; its row and
//     column scales load during the last stage's MFMAs.
// ---------------------------------------------------------------------------
namespace wide {
constexpr int TM = 256, SK = 128;
constexpr int kALoads = 8;                            // A DMA per wave per stage
constexpr int kBOff = 32 * 1024;                      // B's offset in a stage
template <int TN>
struct Cfg {
    static constexpr int NB = TN / 64;                // 32-column MFMA tiles per wave
    static constexpr int kBBlocks = TN / 8;           // 1 KiB B blocks per stage
    static constexpr int kBLoads = kBBlocks / 4;      // B DMA per wave per stage
    static constexpr int kLoads = kALoads + kBLoads;
    static constexpr int kStageBytes = kBOff + kBBlocks * 1024;
    static constexpr int kRing = 2 * kStageBytes;
    static constexpr int kScaleOff = kRing;           // 256 row scales after the ring
    static constexpr size_t kLds = static_cast<size_t>(kRing + TM * 4);
    static constexpr int kReads = 2 * (4 + NB);       // fragment reads per 64-deep half
    static constexpr int kMfma = 2 * 4 * NB;          // MFMAs per 64-deep half
    static_assert(kLds <= 160 * 1024, "LDS plan");
    static_assert(kLoads + kReads <= 2 * kMfma, "side work fits the MFMA slots");
};
}  // namespace wide

template <int NB>
struct FragsW {
    v4i a[2][4], b[2][NB];
};

// ps[0] and ps[1]: up to two independent problems with the same M in one
// grid (tiles_n0 and tiles_n1 column tiles; tiles_n1 = 0 for one problem),
// so the tiles of both fill whole rounds of CUs together.
template <int TN>
__device__ __forceinline__ void wide_tile(const I8Gemm &p, uint32_t tmi, uint32_t tni)
{
    using namespace wide;
    using G = Cfg<TN>;
    constexpr int NB = G::NB;
    extern __shared__ __attribute__((aligned(1024))) int8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t m0 = tmi * TM, n0 = tni * TN;
    const uint32_t NT = p.Np >> 4;
    const uint32_t KS = p.K / SK;
    const uint64_t KTp = p.Kp >> 6;

    // DMA: A instruction 8*wave + j copies rows 64*wave + 8j + l/8 (M is a
    // multiple of 256 here, so no row clamp); lane l fetches k chunk
    // (l%8) ^ ((row >> 1) & 7) = (l%8) ^ (l/16) ^ 4(j%2).  B block
    // bi = kBLoads*wave + j is column block bi/2, k block bi%2 (column blocks
    // past N are clamped: their results are never stored).  Bases are
    // wave-uniform (SGPRs); per-lane parts are 32-bit offsets.
    const int q = lane >> 3;
    const int8_t *a_base = p.A + static_cast<uint64_t>(m0 + wave * 64) * p.lda;
    const uint32_t a_lo = q * p.lda + 16 * ((lane & 7) ^ (q >> 1));
    const uint32_t a_lo_odd = q * p.lda + 16 * ((lane & 7) ^ (q >> 1) ^ 4);
    const uint32_t b_lo = lane * 16;
    auto issue_one = [&](uint32_t s, int k) {
        int8_t *st = smem + (s & 1) * G::kStageBytes;
        if (k < kALoads) {
            dma16_s(a_base + static_cast<uint64_t>(8 * k) * p.lda + s * SK, (k & 1) ? a_lo_odd : a_lo,
                    st + (wave * kALoads + k) * 1024);
        } else {
            const int bi = wave * G::kBLoads + (k - kALoads);
            const uint32_t nb = min((n0 >> 4) + (bi >> 1), NT - 1);
            dma16_s(p.frag + ((static_cast<uint64_t>(nb) * KTp + (bi & 1)) << 10) + static_cast<uint64_t>(s) * 2048,
                    b_lo, st + kBOff + bi * 1024);
        }
    };

    // Fragment read k of half hh of the stage at byte offset st, in MFMA
    // order: per 32-deep h, b[h][0], a[h][0..3], b[h][1..NB-1].  A row
    // wm*128 + 32i + l%32 has swizzle ((l%32) >> 1) & 7 whatever i is, so one
    // per-lane base per (hh, h) plus the constant 4096 i addresses it; B needs
    // one per-lane base plus constants.  With st a constant every read is
    // base + immediate.
    const int sub = (lane >> 4) & 1;
    uint32_t a_rd[2][2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int h = 0; h < 2; ++h)
            a_rd[hh][h] = (wm * 128 + (lane & 31)) * 128 +
                          (((4 * hh + 2 * h + (lane >> 5)) ^ (((lane & 31) >> 1) & 7)) << 4);
    const uint32_t b_lane = ((2 * sub) << 10) + (((lane >> 5) * 16 + (lane & 15)) << 4);
    const uint32_t b_rd = kBOff + ((wn * (TN / 16)) << 10) + b_lane;
    auto read_one = [&](uint32_t st, int hh, FragsW<NB> &f, int k) {
        const int h = k / (4 + NB), r = k % (4 + NB);
        if (r >= 1 && r <= 4) {
            const int i = r - 1;
            f.a[h][i] = *reinterpret_cast<const v4i *>(smem + st + a_rd[hh][h] + i * 4096);
        } else {
            const int j = r == 0 ? 0 : r - 4;
            f.b[h][j] = *reinterpret_cast<const v4i *>(smem + st + b_rd + j * 4096 + hh * 1024 + h * 512);
        }
    };

    v16i acc[4][NB];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = (v16i){0};
    // The MFMAs of one 64-deep half; side(k) runs after MFMA k.
    auto mma = [&](const FragsW<NB> &f, auto &&side) {
#pragma unroll
        for (int k = 0; k < G::kMfma; ++k) {
            const int h = k / (4 * NB), j = (k / 4) % NB, i = k % 4;
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[h][i], f.b[h][j], acc[i][j], 0, 0, 0);
            side(k);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // Second half's side work: the stage s+2 DMA, one per MFMA slot, then the
    // next stage's half-0 reads spread over the remaining slots.
    constexpr int kTail = G::kMfma - G::kLoads;
    auto side2 = [&](int k, uint32_t s, uint32_t nxt, FragsW<NB> &f, bool dma) {
        if (dma && k < G::kLoads) issue_one(s, k);
#pragma unroll
        for (int r = 0; r < G::kReads; ++r)
            if (G::kLoads + (r * kTail) / G::kReads == k) read_one(nxt, 0, f, r);
    };

    // Prologue: stages 0 and 1 in flight, wait for 0, read its first half.
#pragma unroll
    for (int k = 0; k < G::kLoads; ++k) issue_one(0, k);
    if (KS > 1) {
#pragma unroll
        for (int k = 0; k < G::kLoads; ++k) issue_one(1, k);
        wait_vmcnt<G::kLoads>();
    } else {
        wait_vmcnt<0>();
    }
    block_barrier();
    FragsW<NB> f0, f1;
#pragma unroll
    for (int k = 0; k < G::kReads; ++k) read_one(0, 0, f0, k);

    uint32_t s = 0;
    for (; s + 2 < KS; ++s) {
        const uint32_t cur = (s & 1) * G::kStageBytes, nxt = G::kStageBytes - cur;
        __builtin_amdgcn_sched_barrier(0);
        mma(f0, [&](int k) { if (k < G::kReads) read_one(cur, 1, f1, k); });
        wait_vmcnt<0>();
        block_barrier();
        mma(f1, [&](int k) { side2(k, s + 2, nxt, f0, true); });
    }
    if (s + 1 < KS) {
        const uint32_t cur = (s & 1) * G::kStageBytes, nxt = ((s + 1) & 1) * G::kStageBytes;
        __builtin_amdgcn_sched_barrier(0);
        mma(f0, [&](int k) { if (k < G::kReads) read_one(cur, 1, f1, k); });
        wait_vmcnt<0>();
        block_barrier();
        mma(f1, [&](int k) { side2(k, 0, nxt, f0, false); });
        ++s;
    }
    // The epilogue's row and column scales load during the last stage.
    const float sa_g = p.scale_a ? p.scale_a[m0 + tid] : 1.0f;   // M % 256 == 0: row m0 + tid exists
    const ColEpi<NB> ce(p, n0 + wn * (TN / 2) + (lane & 31), lane);
    {
        const uint32_t cur = (s & 1) * G::kStageBytes;
        __builtin_amdgcn_sched_barrier(0);
        mma(f0, [&](int k) { if (k < G::kReads) read_one(cur, 1, f1, k); });
        mma(f1, [](int) {});
    }

    // Epilogue: each wave stores its own 128 x TN/2 block from registers.
    float *sa_lds = reinterpret_cast<float *>(smem + G::kScaleOff);
    sa_lds[tid] = sa_g;
    __syncthreads();
    const float *sa = sa_lds + wm * 128;
    const uint32_t mrow = m0 + wm * 128;
    switch (p.epilogue) {
    case 1: reg_store<1, NB, 0, 4, false>(p, acc, nullptr, sa, mrow, ce, lane); break;
    case 2: reg_store<2, NB, 0, 4, false>(p, acc, nullptr, sa, mrow, ce, lane); break;
    case 3:
    case 4: reg_store<3, NB, 0, 4, false>(p, acc, nullptr, sa, mrow, ce, lane); break;
    default: reg_store<0, NB, 0, 4, false>(p, acc, nullptr, sa, mrow, ce, lane); break;
    }
}

// Workgroup g (XCD-aware order) -> problem and tile: the first
// tiles_m * tiles_n0 tiles belong to ps.p[0], the rest to ps.p[1].
__device__ __forceinline__ bool wide_tile_of(uint32_t tiles_m, uint32_t tiles_n0, uint32_t tiles_n1, uint32_t &tmi,
                                             uint32_t &tni)
{
    const uint32_t first = tiles_m * tiles_n0, total = first + tiles_m * tiles_n1;
    uint32_t g = blockIdx.x;
    if ((total & 7u) == 0) g = (g & 7u) * (total >> 3) + (g >> 3);
    const bool second = g >= first;
    if (second) g -= first;
    tmi = g % tiles_m;
    tni = g / tiles_m;
    return second;
}

template <int TN>
__global__ __launch_bounds__(kThreads) void gemm_i8_wide(I8GemmPair ps, uint32_t tiles_m, uint32_t tiles_n0,
                                                         uint32_t tiles_n1)
{
    uint32_t tmi, tni;
    const bool second = wide_tile_of(tiles_m, tiles_n0, tiles_n1, tmi, tni);
    wide_tile<TN>(ps.p[second ? 1 : 0], tmi, tni);
}

// One problem in two column ranges: ps.p[0] (the first columns) on 256-wide
// tiles, ps.p[1] (the rest) on 192-wide tiles, sized so the grid fills whole
// rounds of one tile per CU (N = 14336 at M = 2048: 32 + 32 tile columns, 512
// tiles = two rounds, where 256-wide tiles alone are 448 = 1.75 rounds).
// Each range fills whole rounds, and workgroups are dispatched in index
// order, so the first rounds run the 256-wide tiles and the last ones the
// 192-wide tiles (every CU one of each); the XCD-aware order applies within
// each range.
__global__ __launch_bounds__(kThreads) void gemm_i8_wide_mix(I8GemmPair ps, uint32_t tiles_m, uint32_t tiles_n0,
                                                             uint32_t tiles_n1)
{
    const uint32_t first = tiles_m * tiles_n0;
    const bool second = blockIdx.x >= first;
    const uint32_t n = second ? tiles_m * tiles_n1 : first;
    uint32_t g = second ? blockIdx.x - first : blockIdx.x;
    if ((n & 7u) == 0) g = (g & 7u) * (n >> 3) + (g >> 3);
    if (second)
        wide_tile<192>(ps.p[1], g % tiles_m, g / tiles_m);
    else
        wide_tile<256>(ps.p[0], g % tiles_m, g / tiles_m);
}

}  // namespace

uint32_t gemm_i8_variant_for_tiles(uint32_t tile_m, uint32_t tile_k, uint32_t tile_n)
{
    if (tile_m == 256 && tile_k == 128 && tile_n == 256) return kI8Wide;
    if (tile_m == 256 && tile_k == 128 && tile_n == 192) return kI8Wide192;
    if (tile_m == 256 && tile_k == 128 && tile_n == 128) return kI8Wave8;
    if (tile_m == 256 && tile_k == 64 && tile_n == 128) return kI8Pipe;
    if (tile_m == 128 && tile_k == 64 && tile_n == 128) return kI8Generic;
    return kI8Auto;
}

namespace {


// Estimated time of a grid of `tiles` tiles of area tm x tn on `cus` CUs:
// whole rounds of one tile per CU, each tile costing its area times the
// kernel's measured time per unit area (relative: 256 x 256 tile 1.0,
// 256 x 192 1.2, 256 x 128 8-wave 1.4; from 2048 x 4096 x N runs).
double tile_cost(uint64_t tiles, uint32_t cus, uint32_t tm, uint32_t tn, double per_area)
{
    const uint64_t rounds = (tiles + cus - 1) / cus;
    return static_cast<double>(rounds) * tm * tn * per_area;
}

}  // namespace

uint32_t cu_count()
{
    static const uint32_t n = [] {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
            (void)hipGetLastError();
            return 256u;
        }
        return static_cast<uint32_t>(cus);
    }();
    return n;
}

// Largest share of nonzero 64 x 64 weight tiles at which the strip kernel
// (with its copy of A in fragment blocks) beats the dense ones.  Measured at
// 4096^3 against the 256 x 256 dense kernel on the same weights: 1.06x the
// dense time at 50% nonzero tiles, 0.88x at 37.5%, 0.77x at 25%, 0.63x at
// 12.5%.  The int8 GEMM is bound by operand traffic into LDS, not by the
// matrix cores: at 50% zero tiles the skip removes half the MFMAs, but A is
// read once per 64-column group instead of once per 256-column tile.
constexpr double kStripDensity = 0.4;

// The strip kernel takes the call: packed weights with nonzero-tile lists,
// the pipelined kernels' alignment, at most 256 k blocks, and at most
// kStripDensity of the tiles nonzero (unless another kernel was requested).
static bool use_strip(const I8Gemm &p)
{
    const uint32_t KTp = p.Kp / 64, groups = (p.Np / 16 + 3) / 4;
    const bool aligned = (p.K % 64 == 0) && (p.lda % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(p.A) % 16 == 0) && p.M >= 64;
    if (!aligned || !p.nz_list || !p.nz_count || KTp > strip::kMaxKBlocks) return false;
    if (p.variant != kI8Auto && p.variant != kI8Strip) return false;
    return p.variant == kI8Strip || static_cast<double>(p.nz_tiles) <= kStripDensity * groups * KTp;
}

size_t gemm_i8_ws_bytes(const I8Gemm &p)
{
    return use_strip(p) ? static_cast<size_t>((p.M + 15) / 16) * 16 * p.Kp : 0;
}

void gemm_i8(hipStream_t s, const I8Gemm &p, int8_t *ws)
{
    const bool aligned = (p.K % 64 == 0) && (p.lda % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(p.A) % 16 == 0) && p.M >= 64;
    // The 128-deep kernels address 8 rows of A per copy as a 32-bit lane
    // offset from a uniform base (below 8 lda).
    const bool k128 = aligned && p.K % pipe128::SK == 0 && p.ldc <= kRegStoreMaxLdc && p.lda < (1u << 29);
    const bool wide_ok = k128 && p.M % wide::TM == 0;
    const uint32_t wm_ = p.M / wide::TM;
    const uint32_t wn256 = (p.N + 255) / 256, wn192 = (p.N + 191) / 192;
    const uint32_t tm = (p.M + pipe::TM - 1) / pipe::TM;
    const uint32_t tn = (p.N + pipe::TN - 1) / pipe::TN;
    // A requested kernel that cannot take this shape falls back to the
    // automatic choice.
    // The strip kernel walks only the nonzero 64 x 64 weight tiles (ws holds
    // gemm_i8_ws_bytes(p): A in fragment blocks).
    const uint32_t KTp = p.Kp / 64, groups = (p.Np / 16 + 3) / 4;
    uint32_t v = p.variant;
    if (ws && use_strip(p)) v = kI8Strip;
    if (((v == kI8Wide || v == kI8Wide192) && !wide_ok) || (v == kI8Wave8 && !k128) || (v == kI8Pipe && !aligned) ||
        (v == kI8Strip && !(ws && use_strip(p))))
        v = kI8Auto;
    uint32_t mix_a = 0, mix_b = 0;   // tile columns of 256 and 192 (mixed grid)
    if (v == kI8Auto) {
        // The tile that finishes first: whole rounds of one tile per CU times
        // the tile's cost (a 256-wide grid of 344 or 384 tiles runs two
        // rounds, the second half empty; 256 x 192 tiles fill both).
        v = k128 ? kI8Wave8 : aligned ? kI8Pipe : kI8Generic;
        if (wide_ok) {
            const uint32_t cus = cu_count();
            const double c8 = tile_cost(static_cast<uint64_t>(tm) * tn, cus, 256, 128, 1.4);
            const double c256 = tile_cost(static_cast<uint64_t>(wm_) * wn256, cus, 256, 256, 1.0);
            const double c192 = tile_cost(static_cast<uint64_t>(wm_) * wn192, cus, 256, 192, 1.2);
            double best = c8;
            if (c256 <= c192 && c256 < c8) v = kI8Wide, best = c256;
            else if (c192 < c8) v = kI8Wide192, best = c192;
            // Mixed widths (dense weights): r1 whole rounds of 256-wide tiles
            // on the first columns, r2 of 192-wide tiles on the rest.
            if (cus % wm_ == 0) {
                const uint32_t per = cus / wm_;   // tile columns per round
                for (uint32_t r1 = 1; r1 <= 3; ++r1)
                    for (uint32_t r2 = 1; r2 <= 3; ++r2) {
                        const uint64_t n256 = 256ull * per * r1, ncols = n256 + 192ull * per * r2;
                        if (n256 >= p.N || ncols < p.N || ncols - 192ull * per >= p.N) continue;
                        const double c = r1 * 65536.0 * 1.0 + r2 * 49152.0 * 1.2;
                        if (c < best) {
                            best = c;
                            v = kI8Wide;
                            mix_a = per * r1;
                            mix_b = per * r2;
                        }
                    }
            }
        }
    }
    if (v != kI8Generic) {
        static std::atomic<bool> lds_optin{false};  // launches may come from several host threads
        if (!lds_optin) {
            bool ok = true;
            for (const void *fn : {reinterpret_cast<const void *>(gemm_i8_pipe),
                                   reinterpret_cast<const void *>(gemm_i8_strip),
                                   reinterpret_cast<const void *>(gemm_i8_k128w8),
                                   reinterpret_cast<const void *>(gemm_i8_wide<256>),
                                   reinterpret_cast<const void *>(gemm_i8_wide<192>),
                                   reinterpret_cast<const void *>(gemm_i8_wide_mix)})
                ok = ok && hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               160 * 1024) == hipSuccess;
            lds_optin = ok;
        }
    }
    if (mix_a) {
        // Column split of one problem: the packed weights are strip-major, so
        // columns from nsplit on start nsplit / 16 strips into the fragments.
        const uint32_t nsplit = 256 * mix_a;
        I8Gemm p0 = p, p1 = p;
        p0.N = p0.Np = nsplit;
        p1.N = p.N - nsplit;
        p1.Np = p.Np - nsplit;
        p1.frag = p.frag + static_cast<uint64_t>(nsplit / 16) * (p.Kp / 64) * 1024;
        p1.scale_b = p.scale_b + nsplit;
        p1.bias = p.bias ? p.bias + nsplit : nullptr;
        p1.C = p.C + nsplit;
        gemm_i8_wide_mix<<<dim3(wm_ * (mix_a + mix_b)), kThreads, wide::Cfg<256>::kLds, s>>>(I8GemmPair{{p0, p1}},
                                                                                             wm_, mix_a, mix_b);
        return;
    }
    switch (v) {
    case kI8Strip: {
        const uint32_t tiles_m = (p.M + strip::TM - 1) / strip::TM;
        const uint64_t chunks = static_cast<uint64_t>((p.M + 15) / 16) * KTp * 64;
        a_blocks_kernel<<<dim3(static_cast<uint32_t>((chunks + 255) / 256)), 256, 0, s>>>(p.A, p.lda, p.M, KTp,
                                                                                          chunks, ws);
        gemm_i8_strip<<<dim3(tiles_m * groups), strip::kThreads, strip::kLds, s>>>(p, tiles_m, groups, ws);
        return;
    }
    case kI8Wide:
        gemm_i8_wide<256><<<dim3(wm_ * wn256), kThreads, wide::Cfg<256>::kLds, s>>>(I8GemmPair{{p, p}}, wm_,
                                                                                   wn256, 0);
        return;
    case kI8Wide192:
        gemm_i8_wide<192><<<dim3(wm_ * wn192), kThreads, wide::Cfg<192>::kLds, s>>>(I8GemmPair{{p, p}}, wm_,
                                                                                   wn192, 0);
        return;
    case kI8Wave8:
        gemm_i8_k128w8<<<dim3(tm * tn), w8::kThreads8, pipe128::kLds, s>>>(p, tm, tn);
        return;
    case kI8Pipe:
        gemm_i8_pipe<<<dim3(tm * tn), kThreads, pipe::kLds, s>>>(p, tm, tn);
        return;
    default: {
        dim3 grid((p.N + BN - 1) / BN, (p.M + BM - 1) / BM);
        gemm_i8_generic<<<grid, kThreads, 0, s>>>(p);
        return;
    }
    }
}

bool gemm_i8_pair(hipStream_t s, const I8Gemm &p0, const I8Gemm &p1)
{
    auto wide_ok = [](const I8Gemm &p) {
        return p.K % 64 == 0 && p.lda % 16 == 0 && reinterpret_cast<uintptr_t>(p.A) % 16 == 0 && p.M >= 64 &&
               p.K % pipe128::SK == 0 && p.M % wide::TM == 0 &&
               p.ldc <= kRegStoreMaxLdc &&
               p.variant == kI8Auto;
    };
    if (p0.M != p1.M || !wide_ok(p0) || !wide_ok(p1)) return false;
    // One grid of 256 x 256 tiles only when its whole rounds beat the two
    // grids the automatic choice would run one after the other.
    const uint32_t cus = cu_count();
    const uint32_t wm_ = p0.M / wide::TM;
    auto alone = [&](const I8Gemm &p) {
        const uint32_t tm = (p.M + pipe::TM - 1) / pipe::TM, tn = (p.N + pipe::TN - 1) / pipe::TN;
        const double c8 = tile_cost(static_cast<uint64_t>(tm) * tn, cus, 256, 128, 1.4);
        const double c256 = tile_cost(static_cast<uint64_t>(wm_) * ((p.N + 255) / 256), cus, 256, 256, 1.0);
        const double c192 = tile_cost(static_cast<uint64_t>(wm_) * ((p.N + 191) / 192), cus, 256, 192, 1.2);
        return std::min(c8, std::min(c256, c192));
    };
    const uint32_t tn0 = (p0.N + 255) / 256, tn1 = (p1.N + 255) / 256;
    const double together = tile_cost(static_cast<uint64_t>(wm_) * (tn0 + tn1), cus, 256, 256, 1.0);
    if (together >= alone(p0) + alone(p1)) return false;
    static std::atomic<bool> lds_optin{false};  // launches may come from several host threads
    if (!lds_optin)
        lds_optin = hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_i8_wide<256>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
    gemm_i8_wide<256><<<dim3(wm_ * (tn0 + tn1)), kThreads, wide::Cfg<256>::kLds, s>>>(I8GemmPair{{p0, p1}}, wm_,
                                                                                      tn0, tn1);
    return true;
}

}  // namespace k
}  // namespace vnpu
