// gemv_i8.hip - MATMUL_I8 decode path (M <= 8): HBM-streaming GEMV, no MFMA.
//
// Replaces the reference's rank-1/rank-R AVX2 decode kernels
// (src/kernels/kernels.cpp:581-632, 702-767) and their tile rules
// (src/core/scheduler.cpp:76-167).  Semantics are the reference's
// store_i8_c (kernels.cpp:526-535):
//   C[m][n] = epi(((float)acc * scale_a[m]) * scale_b[n] + bias[n]),
//   acc = sum_k A[m][k] * B[k][n] in int32 (exact, so any order is bit-exact).
//
// Design (HBM-bound: every weight byte is read once, ~K*N bytes per call):
//   * one workgroup = 4 waves owns T 16-column blocks over all of K;
//   * the weights are read in the packed fragment layout: for each 64-deep
//     k block one 1 KiB run per 16 columns; lane l = 16*kg + c loads 16 bytes
//     = 16 consecutive k of column c (fully coalesced 16-byte loads);
//   * waves stride over the k blocks (wave w takes kt = w, w+4, ...), with
//     U k blocks of loads in flight per lane before any arithmetic;
//   * the activations (M x K int8, tiny) are staged once per workgroup in LDS
//     as [k/16][m][16], so lane kg reads its 16 bytes of every row with one
//     ds_read_b128 per row;
//   * v_dot4_i32_i8 (4 per 16 bytes per row) accumulates in int32;
//   * lanes of equal c reduce over kg with two cross-lane shuffles, waves
//     reduce through LDS, and 16*T*M threads apply the fused epilogue.
#include "kernels.hpp"
#include "device_math.hpp"

namespace vnpu {
namespace k {
namespace {

constexpr int kUnroll = 8;           // k blocks per batch in flight per wave
constexpr uint32_t kLdsA = 32768;    // bytes of LDS for staged activations

__device__ __forceinline__ int dot16(const int4 a, const int4 b, int acc)
{
    acc = __builtin_amdgcn_sdot4(a.x, b.x, acc, false);
    acc = __builtin_amdgcn_sdot4(a.y, b.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a.z, b.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a.w, b.w, acc, false);
    return acc;
}

// M rows, T 16-column blocks per workgroup, W waves splitting K.
template <int M, int T, int W>
__global__ __launch_bounds__(64 * W) void gemv_i8_kernel(I8Gemm p)
{
    constexpr int kThreads = 64 * W;
    constexpr uint32_t kChunkK = (kLdsA / M) & ~63u;  // whole 64-deep k blocks
    __shared__ __attribute__((aligned(16))) int8_t a_lds[kChunkK * M];
    __shared__ int red[W][T][M][16];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int kg = lane >> 4;
    const uint32_t NT = p.Np >> 4;
    const uint32_t nt0 = blockIdx.x * T;
    const bool vec_a = ((p.lda & 15u) == 0) && ((reinterpret_cast<uintptr_t>(p.A) & 15u) == 0);

    int acc[T][M];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[t][m] = 0;

    for (uint32_t kc = 0; kc < p.Kp; kc += kChunkK) {
        const uint32_t kc_len = min(kChunkK, p.Kp - kc);
        const uint32_t kt_begin = kc >> 6, kt_end = (kc + kc_len) >> 6;
        const uint32_t first = kt_begin + wave;
        const uint32_t nsteps = first < kt_end ? (kt_end - first + W - 1) / W : 0;

        // The weight stream does not depend on the activations: put the first
        // batch in flight before staging them.
        int4 bc[kUnroll][T], bn[kUnroll][T];
        auto load_batch = [&](int4 (&b)[kUnroll][T], uint32_t i0) {
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const uint32_t step = i0 + u;
                const uint32_t kt = first + step * W;
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    b[u][t] = make_int4(0, 0, 0, 0);
                    if (step < nsteps && nt0 + t < NT) {
                        const uint64_t blk = static_cast<uint64_t>(kt) * NT + nt0 + t;
                        if (!p.zero_blocks || !p.zero_blocks[blk])
                            b[u][t] = *reinterpret_cast<const int4 *>(p.frag + (blk << 10) + lane * 16);
                    }
                }
            }
        };
        load_batch(bc, 0);

        __syncthreads();  // previous chunk fully consumed
        const uint32_t chunks = (kc_len >> 4) * M;
        for (uint32_t i = tid; i < chunks; i += kThreads) {
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

        for (uint32_t i = 0; i < nsteps; i += kUnroll) {
            if (i + kUnroll < nsteps) load_batch(bn, i + kUnroll);
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const uint32_t step = i + u;
                if (step >= nsteps) break;
                const uint32_t ktl = first + step * W - kt_begin;
                const int8_t *arow = a_lds + ((ktl * 4 + kg) * M) * 16;
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const int4 a = *reinterpret_cast<const int4 *>(arow + m * 16);
#pragma unroll
                    for (int t = 0; t < T; ++t) acc[t][m] = dot16(a, bc[u][t], acc[t][m]);
                }
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u)
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
    for (int o = tid; o < T * M * 16; o += kThreads) {
        const int c = o & 15;
        const int m = (o >> 4) % M;
        const int t = (o >> 4) / M;
        const uint32_t n = (nt0 + t) * 16 + c;
        if (n < p.N) {
            int s = 0;
#pragma unroll
            for (int w = 0; w < W; ++w) s += red[w][t][m][c];
            const float sa = p.scale_a ? p.scale_a[m] : 1.0f;
            float out = __fmul_rn(__fmul_rn(static_cast<float>(s), sa), p.scale_b[n]);
            if (p.bias) out = __fadd_rn(out, p.bias[n]);
            p.C[static_cast<uint64_t>(m) * p.ldc + n] = dev::epilogue(out, p.epilogue);
        }
    }
}

// Launch shape from the column count: two column blocks per workgroup once
// there are enough of them, and eight waves when workgroups are scarce.
template <int M>
void launch_m(hipStream_t s, const I8Gemm &p)
{
    const uint32_t NT = p.Np >> 4;
    if (NT >= 1024)
        gemv_i8_kernel<M, 2, 4><<<dim3((NT + 1) / 2), 256, 0, s>>>(p);
    else if (NT >= 512)
        gemv_i8_kernel<M, 1, 4><<<dim3(NT), 256, 0, s>>>(p);
    else
        gemv_i8_kernel<M, 1, 8><<<dim3(NT), 512, 0, s>>>(p);
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
    default: break;
    }
}

}  // namespace k
}  // namespace vnpu
