// gemv_i8.hip - MATMUL_I8 decode path (M <= 8): HBM-streaming GEMV.
//
// Replaces the reference's rank-1/rank-R AVX2 decode kernels
// (src/kernels/kernels.cpp:581-632, 702-767) and their tile rules
// (src/core/scheduler.cpp:76-167).  Semantics are the reference's
// store_i8_c (kernels.cpp:526-535):
//   C[m][n] = epi(((float)acc * scale_a[m]) * scale_b[n] + bias[n]),
//   acc = sum_k A[m][k] * B[k][n] in int32 (exact, so any order is bit-exact).
//
// Design (HBM-bound: every weight byte is read once, ~K*N bytes per call):
//   * one workgroup of W waves owns T 16-column strips (T = 1, or 4 for many
//     rows and strips) over all of K; the packed layout stores a strip's
//     Kp/64 blocks of 1 KiB contiguously, so each strip is one sequential
//     run;
//   * lane l = 16*kg + c loads 16 bytes = 16 consecutive k of column c
//     (one fully coalesced 1 KiB load per wave per block); waves interleave
//     over the blocks (wave w takes blocks w, w+W, ...), with U blocks in
//     flight per wave and the next U issued before the current U are used;
//   * weight loads are raw buffer loads: the bounds check of the buffer
//     resource turns loads past the wave's last block into zeros, so the
//     load stream has no branches (branches around loads force the waitcnt
//     pass into full drains), and they are nontemporal: the weights are read
//     once and are not worth an L2 allocation;
//   * the activations (M x K int8, tiny) are staged in LDS as [k/16][m][16]
//     (dynamic LDS sized to the chunk actually used), so lane kg reads its
//     16 bytes of every row with one ds_read_b128 per row; the matrix-core
//     kernel for up to 16 rows instead reads them from global memory with
//     each weight block when the rows are 16-byte aligned
//     (gemv_i8_mfma_direct);
//   * v_dot4_i32_i8 (4 per 16 bytes per row) accumulates in int32 for up
//     to four rows; from five rows one v_mfma_i32_16x16x64_i8 per block
//     does it (gemv_i8_mfma below);
//   * lanes of equal c reduce over kg with two cross-lane shuffles, waves
//     reduce through LDS, and 16*M threads apply the fused epilogue.
// Blocks flagged all-zero by PACK_WEIGHTS_I8 are streamed like any other: the
// zero bytes are in memory, so skipping them would only save bandwidth.
#include "kernels.hpp"
#include "device_math.hpp"

#include <atomic>

namespace vnpu {
namespace k {
namespace {

constexpr uint32_t kLdsA = 32768;   // max bytes of staged activations per chunk
// The same for grids of 16-wave workgroups with at most one workgroup per CU:
// a whole 8 x 11008 activation block (the decode down projection) fits in
// one chunk, so the weight stream is not drained at chunk boundaries.
constexpr uint32_t kLdsAOwnCu = 128 * 1024;
constexpr int kBufferWord3 = 0x00020000;  // raw buffer, 32-bit data format
constexpr int kNontemporal = 2;           // cache policy bits of the weight loads

__device__ __forceinline__ int dot16(const int4 a, const int4 b, int acc)
{
    acc = __builtin_amdgcn_sdot4(a.x, b.x, acc, false);
    acc = __builtin_amdgcn_sdot4(a.y, b.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a.z, b.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a.w, b.w, acc, false);
    return acc;
}

// The epilogue's scales and bias for the outputs this thread stores (o = tid,
// tid + NTH, ... below NO), loaded when the workgroup starts so their memory
// latency overlaps the weight stream instead of following it.  The store
// keeps the reference's order ((float)acc * sa) * sb (+ bias) -> epilogue.
template <int NO, int NTH>
struct EpiOperands {
    static constexpr int S = (NO + NTH - 1) / NTH;
    float sa[S], sb[S], bias[S], res[S];
    __device__ __forceinline__ EpiOperands(const I8Gemm &p, uint32_t nt0, int M, int tid)
    {
        const uint32_t NT = p.Np >> 4;
#pragma unroll
        for (int j = 0; j < S; ++j) {
            const int o = tid + j * NTH;
            const int c = o & 15, m = (o >> 4) % M, t = (o >> 4) / M;
            const uint32_t n = (nt0 + t) * 16 + c;
            const bool live = o < NO && nt0 + t < NT && n < p.N && static_cast<uint32_t>(m) < p.M;
            sa[j] = live && p.scale_a ? p.scale_a[m] : 1.0f;
            sb[j] = live ? p.scale_b[n] : 1.0f;
            bias[j] = live && p.bias ? p.bias[n] : 0.0f;
            // the fused ADD's other operand, read before any output is written
            // (it may be the ADD's own output buffer)
            res[j] = live && p.res ? p.res[static_cast<uint64_t>(m) * p.N + n] : 0.0f;
        }
    }
    template <int W, int T, int M>
    __device__ __forceinline__ void store(const I8Gemm &p, const int (&red)[W][T][M][16], uint32_t nt0,
                                          uint32_t NT, int tid) const
    {
#pragma unroll
        for (int j = 0; j < S; ++j) {
            const int o = tid + j * NTH;
            const int c = o & 15, m = (o >> 4) % M, t = (o >> 4) / M;
            const uint32_t n = (nt0 + t) * 16 + c;
            if (o >= NO || nt0 + t >= NT || n >= p.N || static_cast<uint32_t>(m) >= p.M) continue;
            int s = 0;
#pragma unroll
            for (int w = 0; w < W; ++w) s += red[w][t][m][c];
            float out = dev::mul_rn(dev::mul_rn(static_cast<float>(s), sa[j]), sb[j]);
            if (p.bias) out = dev::add_rn(out, bias[j]);
            out = dev::epilogue(out, p.epilogue);
            p.C[static_cast<uint64_t>(m) * p.ldc + n] = out;
            if (p.res) {
                // ADD_F32's fma(a, alpha, b * beta), a and b in command order
                const float x = p.res_c_first ? out : res[j], y = p.res_c_first ? res[j] : out;
                p.res_out[static_cast<uint64_t>(m) * p.N + n] = fmaf(x, p.res_alpha, dev::mul_rn(y, p.res_beta));
            }
        }
    }
};

// M rows, W waves, U blocks in flight per wave, T strips per workgroup (each
// activation read from LDS feeds T weight blocks); chunk_k = k extent
// (multiple of 64) of the activations staged at a time.
template <int M, int W, int U, int T>
__global__ __launch_bounds__(64 * W) void gemv_i8_kernel(I8Gemm p, uint32_t chunk_k)
{
    extern __shared__ __attribute__((aligned(16))) int8_t a_lds[];  // [chunk_k/16][M][16]
    __shared__ int red[W][T][M][16];

    const int tid = threadIdx.x, lane = tid & 63;
    // wave-uniform by construction; readfirstlane lets the compiler know
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kg = lane >> 4;
    const uint32_t NT = p.Np >> 4;
    const uint32_t nt0 = blockIdx.x * T;
    const uint32_t KT = p.Kp >> 6;
    const bool vec_a = ((p.lda & 15u) == 0) && ((reinterpret_cast<uintptr_t>(p.A) & 15u) == 0);

    int acc[T][M];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[t][m] = 0;
    const EpiOperands<T * M * 16, 64 * W> epi(p, nt0, M, tid);

    for (uint32_t kc = 0; kc < p.Kp; kc += chunk_k) {
        const uint32_t kt0 = kc >> 6, kt1 = min(KT, (kc + chunk_k) >> 6);
        const uint32_t first = kt0 + wave;
        const uint32_t cnt = first < kt1 ? (kt1 - first + W - 1) / W : 0;
        // This wave's blocks first, first + W, ... of each strip as one
        // bounds-checked buffer (empty for a strip past the last one).
        __amdgpu_buffer_rsrc_t rs[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const uint32_t nt = min(nt0 + t, NT - 1);
            const int8_t *strip = p.frag + static_cast<uint64_t>(nt) * KT * 1024;
            const int bytes = (cnt && nt0 + t < NT) ? static_cast<int>(((cnt - 1) * W + 1) * 1024) : 0;
            rs[t] = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(strip) + static_cast<uint64_t>(first) * 1024,
                                                      0, bytes, kBufferWord3);
        }
        auto ld = [&](int t, uint32_t i) {
            return __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(
                rs[t], i * W * 1024 + lane * 16, 0, kNontemporal));
        };
        // The weight stream does not depend on the activations: put the first
        // batch in flight before staging them.
        int4 bc[U][T], bn[U][T];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int t = 0; t < T; ++t) bc[u][t] = ld(t, u);

        if (kc) __syncthreads();  // previous chunk fully consumed
        const uint32_t chunks = (kt1 - kt0) * 4 * M;
        for (uint32_t i = tid; i < chunks; i += 64 * W) {
            const uint32_t m = i % M, k16 = i / M;
            const uint32_t k = kc + k16 * 16;
            const int8_t *src = p.A + static_cast<uint64_t>(m) * p.lda + k;
            int4 v;
            if (vec_a && k + 16 <= p.K) {
                v = *reinterpret_cast<const int4 *>(src);
            } else {
                union {
                    int8_t b[16];
                    int4 v;
                } u;
#pragma unroll
                for (int j = 0; j < 16; ++j) u.b[j] = (k + j < p.K) ? src[j] : 0;
                v = u.v;
            }
            *reinterpret_cast<int4 *>(a_lds + (k16 * M + m) * 16) = v;
        }
        __syncthreads();

        for (uint32_t i = 0; i < cnt; i += U) {
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int t = 0; t < T; ++t) bn[u][t] = ld(t, i + U + u);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                // past the last block the weights read as zero; clamp the
                // activation index so it stays inside the staged chunk
                const uint32_t ktl = first + W * min(i + u, cnt - 1) - kt0;
                const int8_t *arow = a_lds + ((ktl * 4 + kg) * M) * 16;
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const int4 a = *reinterpret_cast<const int4 *>(arow + m * 16);
#pragma unroll
                    for (int t = 0; t < T; ++t) acc[t][m] = dot16(a, bc[u][t], acc[t][m]);
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int t = 0; t < T; ++t) bc[u][t] = bn[u][t];
        }
    }

    // Reduce the four k groups (lanes c, c+16, c+32, c+48).
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            int v = acc[t][m];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            acc[t][m] = v;
        }
    if (lane < 16) {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int m = 0; m < M; ++m) red[wave][t][m][lane] = acc[t][m];
    }
    __syncthreads();
    epi.template store<W, T, M>(p, red, nt0, NT, tid);
}

// The same stream for 3..64 rows with the int8 matrix core doing the math: a
// packed 1 KiB weight block is exactly the B operand of one
// v_mfma_i32_16x16x64_i8 (lane 16kg + c holds k 16kg..16kg+15 of column c),
// and the A operand is the staged activations (lane l: row l%16 of a group of
// 16 rows, the same 16 k; rows past M are zero).  One MFMA per block and row
// group replaces 4M v_dot4 and M ds_read_b128 per lane, which at M = 8 made
// the VALU the bottleneck.  The 16 x 16 result leaves row 4(l/16) + i, column
// l%16 in lane l, register i.  M is the row capacity: the kernels for up to
// 8 rows are built per row count, those for 16, 32 and 64 take any p.M up to
// it (the staged layout uses p.M; rows past it are zero and not stored), and
// above 16 rows the wave sums go through the activation LDS once it is free.
template <int M, int W, int U, int T>
__global__ __launch_bounds__(64 * W) void gemv_i8_mfma(I8GemmPair ps, uint32_t grid0, uint32_t chunk_k)
{
    // Workgroups from grid0 on serve the second problem of a pair (same M
    // and K, so the same chunk_k and LDS size).
    const bool second = blockIdx.x >= grid0;
    const I8Gemm &p = ps.p[second ? 1 : 0];
    const uint32_t bx = second ? blockIdx.x - grid0 : blockIdx.x;
    static_assert(M <= 64, "at most four 16-row groups");
    constexpr int MG = (M + 15) / 16;
    typedef int v4i __attribute__((ext_vector_type(4)));
    extern __shared__ __attribute__((aligned(16))) int8_t a_lds[];  // [chunk_k/16][Mr][16]
    __shared__ int red_s[M <= 16 ? W * T * M * 16 : 1];
    // rows present: the template's count up to 8 rows, else the call's
    const uint32_t Mr = M <= 8 ? static_cast<uint32_t>(M) : ps.p[0].M;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kg = lane >> 4, row = lane & 15;
    const uint32_t NT = p.Np >> 4;
    const uint32_t nt0 = bx * T;
    const uint32_t KT = p.Kp >> 6;
    const bool vec_a = ((p.lda & 15u) == 0) && ((reinterpret_cast<uintptr_t>(p.A) & 15u) == 0);

    v4i acc[MG][T];
#pragma unroll
    for (int g = 0; g < MG; ++g)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[g][t] = (v4i){0, 0, 0, 0};
    const EpiOperands<T * M * 16, 64 * W> epi(p, nt0, M, tid);

    for (uint32_t kc = 0; kc < p.Kp; kc += chunk_k) {
        const uint32_t kt0 = kc >> 6, kt1 = min(KT, (kc + chunk_k) >> 6);
        const uint32_t first = kt0 + wave;
        const uint32_t cnt = first < kt1 ? (kt1 - first + W - 1) / W : 0;
        __amdgpu_buffer_rsrc_t rs[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const uint32_t nt = min(nt0 + t, NT - 1);
            const int8_t *strip = p.frag + static_cast<uint64_t>(nt) * KT * 1024;
            const int bytes = (cnt && nt0 + t < NT) ? static_cast<int>(((cnt - 1) * W + 1) * 1024) : 0;
            rs[t] = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(strip) + static_cast<uint64_t>(first) * 1024,
                                                      0, bytes, kBufferWord3);
        }
        auto ld = [&](int t, uint32_t i) {
            return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                rs[t], i * W * 1024 + lane * 16, 0, kNontemporal));
        };
        v4i bc[U][T], bn[U][T];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int t = 0; t < T; ++t) bc[u][t] = ld(t, u);

        if (kc) __syncthreads();  // previous chunk fully consumed
        const uint32_t chunks = (kt1 - kt0) * 4 * Mr;
        for (uint32_t i = tid; i < chunks; i += 64 * W) {
            const uint32_t m = i % Mr, k16 = i / Mr;
            const uint32_t k = kc + k16 * 16;
            const int8_t *src = p.A + static_cast<uint64_t>(m) * p.lda + k;
            int4 v;
            if (vec_a && k + 16 <= p.K) {
                v = *reinterpret_cast<const int4 *>(src);
            } else {
                union {
                    int8_t b[16];
                    int4 v;
                } u;
#pragma unroll
                for (int j = 0; j < 16; ++j) u.b[j] = (k + j < p.K) ? src[j] : 0;
                v = u.v;
            }
            *reinterpret_cast<int4 *>(a_lds + (k16 * Mr + m) * 16) = v;
        }
        __syncthreads();

        for (uint32_t i = 0; i < cnt; i += U) {
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int t = 0; t < T; ++t) bn[u][t] = ld(t, i + U + u);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t ktl = first + W * min(i + u, cnt - 1) - kt0;
#pragma unroll
                for (int g = 0; g < MG; ++g) {
                    const uint32_t r = 16 * g + row;
                    v4i a = (v4i){0, 0, 0, 0};
                    if (r < Mr) a = *reinterpret_cast<const v4i *>(a_lds + ((ktl * 4 + kg) * Mr + r) * 16);
#pragma unroll
                    for (int t = 0; t < T; ++t)
                        acc[g][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bc[u][t], acc[g][t], 0, 0, 0);
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int t = 0; t < T; ++t) bc[u][t] = bn[u][t];
        }
    }

    // Lane l holds rows 16g + 4(l/16) + i of column l%16; sum the waves in LDS
    // (above 16 rows in the activation area, once every wave is done with it).
    if constexpr (M > 16) __syncthreads();
    auto &red = *reinterpret_cast<int (*)[W][T][M][16]>(M <= 16 ? static_cast<void *>(red_s)
                                                                 : static_cast<void *>(a_lds));
#pragma unroll
    for (int g = 0; g < MG; ++g)
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 16 * g + 4 * kg + i;
                if (m < M) red[wave][t][m][row] = acc[g][t][i];
            }
    __syncthreads();
    epi.template store<W, T, M>(p, red, nt0, NT, tid);
}

// The matrix-core GEMV with the activations read straight from global memory
// instead of staged in LDS: lane (kg, row) loads its 16 bytes of row `row`
// for each k block alongside that block's weights (one A load serves the T
// strips), so no staging pass and barrier sit between the first weight loads
// and the first MFMA.  Needs 16-byte aligned rows (lda % 16 == 0,
// K % 16 == 0); rows past p.M and k past K read as zeros through the
// buffer's range check.
template <int M, int W, int U, int T>
__global__ __launch_bounds__(64 * W) void gemv_i8_mfma_direct(I8GemmPair ps, uint32_t grid0)
{
    static_assert(M <= 16, "one 16-row group");
    const bool second = blockIdx.x >= grid0;
    const I8Gemm &p = ps.p[second ? 1 : 0];
    const uint32_t nt0 = (second ? blockIdx.x - grid0 : blockIdx.x) * T;
    typedef int v4i __attribute__((ext_vector_type(4)));
    __shared__ int red[W][T][M][16];
    const uint32_t Mr = M <= 8 ? static_cast<uint32_t>(M) : p.M;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kg = lane >> 4, row = lane & 15;
    const uint32_t NT = p.Np >> 4;
    const uint32_t KT = p.Kp >> 6;
    const EpiOperands<T * M * 16, 64 * W> epi(p, nt0, M, tid);

    const uint32_t first = wave;
    const uint32_t cnt = first < KT ? (KT - first + W - 1) / W : 0;
    __amdgpu_buffer_rsrc_t rw[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int8_t *strip = p.frag + static_cast<uint64_t>(min(nt0 + t, NT - 1)) * KT * 1024;
        const int bytes = (cnt && nt0 + t < NT) ? static_cast<int>(((cnt - 1) * W + 1) * 1024) : 0;
        rw[t] = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(strip) + static_cast<uint64_t>(first) * 1024,
                                                  0, bytes, kBufferWord3);
    }
    // A: one buffer over the Mr rows; the lane's offset is past the end for a
    // row past Mr, a block past the wave's last or k past K
    const auto ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(p.A), 0,
                                                      static_cast<int>((Mr - 1) * p.lda + p.K), kBufferWord3);
    const bool row_live = static_cast<uint32_t>(row) < Mr;
    const uint32_t a_row = row_live ? row * p.lda : 0u;
    auto ldb = [&](int t, uint32_t i) {
        return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rw[t], i * W * 1024 + lane * 16, 0,
                                                                             kNontemporal));
    };
    auto lda_ = [&](uint32_t i) {
        const uint32_t k = (first + W * i) * 64 + kg * 16;
        const bool live = row_live && i < cnt && k < p.K;
        return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(ra, live ? a_row + k : 0x80000000u, 0,
                                                                             0));
    };
    v4i acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = (v4i){0, 0, 0, 0};
    v4i bc[U][T], bn[U][T], ac[U], an[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int t = 0; t < T; ++t) bc[u][t] = ldb(t, u);
        ac[u] = lda_(u);
    }
    for (uint32_t i = 0; i < cnt; i += U) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int t = 0; t < T; ++t) bn[u][t] = ldb(t, i + U + u);
            an[u] = lda_(i + U + u);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int t = 0; t < T; ++t) acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ac[u], bc[u][t], acc[t], 0, 0, 0);
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int t = 0; t < T; ++t) bc[u][t] = bn[u][t];
            ac[u] = an[u];
        }
    }
    // lane l holds rows 4(l/16) + i of column l%16
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * kg + i;
            if (m < M) red[wave][t][m][row] = acc[t][i];
        }
    __syncthreads();
    epi.template store<W, T, M>(p, red, nt0, NT, tid);
}

// Launch shapes (swept on MI355X at K = 4096 with the weights streamed from
// HBM; waves W x blocks in flight U per wave).  Fewer registers per wave buy
// more resident waves, which matters more than deeper per-wave prefetch:
//   * v_dot4 kernel (M <= 4), from 512 strips: M = 1, 3, 4 eight waves with two
//     blocks (M=1 N=32000 21.7 -> 20.4 us, N=11008 9.7 -> 8.5 us; M=4 N=32000
//     25.5 -> 22.2 us), M = 1 with two strips per workgroup (N=32000 a further
//     1.6%: 21.8-22.1 -> 21.4-21.7 us on one box; 4 waves with 8 blocks, or 4
//     strips, were slower), M = 2 four waves with two; below 512 strips (one
//     workgroup per strip, at most 256 workgroups) sixteen waves with four
//     (M = 1) or two blocks (M=1 N=4096 5.2 -> 4.8 us).
//   * matrix-core kernel (M >= 5; at three and four rows v_dot4 is as fast):
//     from 1024 strips four strips per workgroup so one staged activation
//     chunk serves four weight streams, <W,U,T> = <4,4,4>; 512-1023 strips
//     two strips per workgroup, <8,2,2> (M=8 N=11008 11.9 -> 11.1 us with
//     <8,4,1>, then N=12288 11.8 -> 11.5 us and N=8200 10.6 -> 9.9 us with two
//     strips); below, <16,2,1> (M=8 N=4096 6.9 -> 6.2 us).
//   * one problem whose two-strip grid has more workgroups than CUs but
//     whose three-strip grid has no more (513-768 strips on 256 CUs): three
//     strips per workgroup, <8,2,3>, so no CU streams twice the bytes of
//     another (768 strips at N = 12288: 384 workgroups of two strips leave
//     half the CUs with two of them).  M=8 N=12288 11.8 -> 11.3 us, N=11008
//     11.4 -> 10.7 us, M=16 N=12288 14.1 -> 12.6 us; the pair grids keep two
//     strips (two problems of 688 strips balance no better with three).
int mfma_variant(uint32_t NT) { return NT >= 1024 ? 0 : NT >= 512 ? 1 : 2; }
int mfma_variant_one(uint32_t NT)
{
    const int v = mfma_variant(NT);
    return v == 1 && (NT + 1) / 2 > cu_count() && (NT + 2) / 3 <= cu_count() ? 3 : v;
}

// k extent (a multiple of 64) of one staged chunk of M activation rows: below
// 512 strips both kernels run one 16-wave workgroup per strip, and when those
// fit one per CU the chunk may take up to kLdsAOwnCu bytes.
uint32_t chunk_k_for(uint32_t Kp, int M, uint32_t NT)
{
    const uint32_t budget = (NT < 512 && NT <= cu_count()) ? kLdsAOwnCu : kLdsA;
    return std::min<uint32_t>(Kp, (budget / M) & ~63u);
}

// Dynamic LDS above 64 KiB needs the kernel's opt-in (once per kernel).
template <auto Kernel>
void lds_optin()
{
    static std::atomic<bool> done{false};
    if (!done)
        done = hipFuncSetAttribute(reinterpret_cast<const void *>(Kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                   static_cast<int>(kLdsAOwnCu)) == hipSuccess;
}
uint32_t mfma_grid(uint32_t NT, int v)
{
    return v == 0 ? (NT + 3) / 4 : v == 1 ? (NT + 1) / 2 : v == 3 ? (NT + 2) / 3 : NT;
}

// The activations can be read straight from global memory by the direct
// kernel: 16-byte aligned rows and K.
bool direct_a(const I8Gemm &p)
{
    return (p.lda % 16 == 0) && (p.K % 16 == 0) && (reinterpret_cast<uintptr_t>(p.A) % 16 == 0) &&
           static_cast<uint64_t>(p.M - 1) * p.lda + p.K < (1ull << 31);
}

template <int M>
void launch_mfma_pair(hipStream_t s, const I8GemmPair &ps, int variant, uint32_t grid0, uint32_t grid1,
                      uint32_t chunk_k)
{
    // above 16 rows the wave sums ([W][T][M][16] int32, 64 W T M bytes; W T =
    // 24 for <8,2,3>, 16 in the other variants) reuse the activation LDS
    const size_t wt = variant == 3 ? 24u : 16u;
    const size_t lds = std::max<size_t>(static_cast<size_t>(chunk_k) * M, M > 16 ? 64u * wt * M : 0u);
    const dim3 grid(grid0 + grid1);
    const bool direct = M <= 16 && direct_a(ps.p[0]) && (grid1 == 0 || direct_a(ps.p[1]));
    if (direct) {
        if constexpr (M <= 16) {
            if (variant == 0)
                gemv_i8_mfma_direct<M, 4, 4, 4><<<grid, 256, 0, s>>>(ps, grid0);
            else if (variant == 1)
                gemv_i8_mfma_direct<M, 8, 2, 2><<<grid, 512, 0, s>>>(ps, grid0);
            else if (variant == 3)
                gemv_i8_mfma_direct<M, 8, 2, 3><<<grid, 512, 0, s>>>(ps, grid0);
            else
                gemv_i8_mfma_direct<M, 16, 2, 1><<<grid, 1024, 0, s>>>(ps, grid0);
        }
    } else if (variant == 0) {
        if (M > 16) lds_optin<gemv_i8_mfma<M, 4, 4, 4>>();
        gemv_i8_mfma<M, 4, 4, 4><<<grid, 256, lds, s>>>(ps, grid0, chunk_k);
    } else if (variant == 1) {
        if (M > 16) lds_optin<gemv_i8_mfma<M, 8, 2, 2>>();
        gemv_i8_mfma<M, 8, 2, 2><<<grid, 512, lds, s>>>(ps, grid0, chunk_k);
    } else if (variant == 3) {
        if (M > 16) lds_optin<gemv_i8_mfma<M, 8, 2, 3>>();
        gemv_i8_mfma<M, 8, 2, 3><<<grid, 512, lds, s>>>(ps, grid0, chunk_k);
    } else {
        lds_optin<gemv_i8_mfma<M, 16, 2, 1>>();
        gemv_i8_mfma<M, 16, 2, 1><<<grid, 1024, lds, s>>>(ps, grid0, chunk_k);
    }
}

template <int M>
void launch_m(hipStream_t s, const I8Gemm &p)
{
    const uint32_t NT = p.Np >> 4;
    const uint32_t chunk_k = chunk_k_for(p.Kp, M, NT);
    const size_t lds = static_cast<size_t>(chunk_k) * M;
    // Four rows below 512 strips on the matrix core with direct activation
    // reads (M=4 K=11008 N=4096 10.7 -> 9.8 us, K=4096 6.0 -> 5.8 us; from
    // 512 strips, and for three rows, v_dot4 stays 3-8% faster).
    if constexpr (M >= 4) {
        if (M >= 5 || (NT < 512 && direct_a(p))) {
            I8GemmPair ps;
            ps.p[0] = ps.p[1] = p;
            const int v = mfma_variant_one(NT);
            launch_mfma_pair<M>(s, ps, v, mfma_grid(NT, v), 0, chunk_k);
            return;
        }
    }
    if constexpr (M == 2) {
        if (NT >= 512) {
            gemv_i8_kernel<M, 4, 2, 1><<<dim3(NT), 256, lds, s>>>(p, chunk_k);
        } else {
            lds_optin<gemv_i8_kernel<M, 16, 2, 1>>();
            gemv_i8_kernel<M, 16, 2, 1><<<dim3(NT), 1024, lds, s>>>(p, chunk_k);
        }
    } else if constexpr (M <= 4) {
        if (NT >= 512) {
            // One row: two strips per workgroup (half the workgroups, each
            // wave's loads alternating between them).
            // (three strips where two would put two workgroups on some CUs
            // and one on others: M=1 N=11008 9.7 -> 9.0 us; three and four
            // rows were slower with three strips)
            if constexpr (M == 1) {
                if ((NT + 1) / 2 > cu_count() && (NT + 2) / 3 <= cu_count())
                    gemv_i8_kernel<M, 8, 2, 3><<<dim3((NT + 2) / 3), 512, lds, s>>>(p, chunk_k);
                else
                    gemv_i8_kernel<M, 8, 2, 2><<<dim3((NT + 1) / 2), 512, lds, s>>>(p, chunk_k);
            } else {
                gemv_i8_kernel<M, 8, 2, 1><<<dim3(NT), 512, lds, s>>>(p, chunk_k);
            }
        } else if constexpr (M == 1) {
            lds_optin<gemv_i8_kernel<M, 16, 4, 1>>();
            gemv_i8_kernel<M, 16, 4, 1><<<dim3(NT), 1024, lds, s>>>(p, chunk_k);
        } else {
            lds_optin<gemv_i8_kernel<M, 16, 2, 1>>();
            gemv_i8_kernel<M, 16, 2, 1><<<dim3(NT), 1024, lds, s>>>(p, chunk_k);
        }
    }
}

}  // namespace

void gemv_i8(hipStream_t s, const I8Gemm &p)
{
    switch (p.M) {
    case 1: launch_m<1>(s, p); break;
    case 2: launch_m<2>(s, p); break;
    case 3: launch_m<3>(s, p); break;
    case 4: launch_m<4>(s, p); break;
    case 5: launch_m<5>(s, p); break;
    case 6: launch_m<6>(s, p); break;
    case 7: launch_m<7>(s, p); break;
    case 8: launch_m<8>(s, p); break;
    default:
        // 9..64 rows: the matrix-core kernel with a row capacity of 16, 32 or 64
        if (p.M <= 16) launch_m<16>(s, p);
        else if (p.M <= 32) launch_m<32>(s, p);
        else if (p.M <= kGemvMaxRows) launch_m<64>(s, p);
        break;
    }
}

bool gemv_i8_pair(hipStream_t s, const I8Gemm &p0, const I8Gemm &p1)
{
    if (p0.M != p1.M || p0.M < 5 || p0.M > 8 || p0.Kp != p1.Kp) return false;
    const uint32_t nt0 = p0.Np >> 4, nt1 = p1.Np >> 4;
    if (mfma_variant(nt0) != mfma_variant(nt1)) return false;
    const uint32_t chunk_k = chunk_k_for(p0.Kp, p0.M, mfma_variant(nt0) == 2 ? nt0 + nt1 : 512);
    const I8GemmPair ps{{p0, p1}};
    const int v = mfma_variant(nt0);
    const uint32_t g0 = mfma_grid(nt0, v), g1 = mfma_grid(nt1, v);
    switch (p0.M) {
    case 5: launch_mfma_pair<5>(s, ps, v, g0, g1, chunk_k); break;
    case 6: launch_mfma_pair<6>(s, ps, v, g0, g1, chunk_k); break;
    case 7: launch_mfma_pair<7>(s, ps, v, g0, g1, chunk_k); break;
    default: launch_mfma_pair<8>(s, ps, v, g0, g1, chunk_k); break;
    }
    return true;
}

}  // namespace k
}  // namespace vnpu
