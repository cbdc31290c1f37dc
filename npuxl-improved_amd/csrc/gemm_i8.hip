// gemm_i8.hip - MATMUL_I8 prefill path on the gfx950 int8 matrix cores.
//
// Replaces the reference's AVX2 packed-panel / 2x32 tiles
// (src/kernels/kernels.cpp:635-869) for M > 8.  Same semantics as the
// reference's store_i8_c (kernels.cpp:526-535): exact int32 accumulation,
// then C = epi(((float)acc * scale_a[m]) * scale_b[n] + bias[n]).
//
// Structure:
//   * workgroup tile BM x BN = 128 x 128, 4 waves in a 2 x 2 grid, wave tile
//     64 x 64 = 4 x 4 v_mfma_i32_16x16x64_i8 blocks (64 accumulator VGPRs);
//   * k step 64 = one MFMA depth;
//   * A (row-major int8 from QUANTIZE_I8) is staged through LDS, double
//     buffered, rows padded to 80 bytes so each ds_read_b128 fragment read is
//     bank-conflict free;
//   * B needs no LDS: the packed fragment layout stores each 16 x 64 operand
//     block as the 1 KiB a wave loads with one 16-byte load per lane;
//   * the next k step's global loads are issued before the current step's
//     MFMAs, one barrier per k step;
//   * a 1 KiB weight block known to be all zero (PACK_WEIGHTS_I8's zero map)
//     is neither loaded nor multiplied: exact, it only adds zeros.
//
// Fragment convention (both operands use the same k order, so the integer
// result is exact whatever order the hardware sums in): lane l = 16*g + r
// holds row/column r and k = 16*g .. 16*g + 15 of the 64-deep block.
// Output: lane l holds C[4*(l/16) + i][l%16], i = 0..3.
#include "kernels.hpp"
#include "device_math.hpp"

namespace vnpu {
namespace k {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

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

__global__ __launch_bounds__(kThreads) void gemm_i8_kernel(I8Gemm p)
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
            if (!z[j] && p.zero_blocks) z[j] = p.zero_blocks[static_cast<uint64_t>(kt) * NT + nb] != 0;
            b[j] = (v4i){0, 0, 0, 0};
            if (!z[j])
                b[j] = *reinterpret_cast<const v4i *>(p.frag + ((static_cast<uint64_t>(kt) * NT + nb) << 10) + lane * 16);
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
                float out = __fmul_rn(__fmul_rn(static_cast<float>(acc[i][j][r]), sa), sb);
                if (p.bias) out = __fadd_rn(out, bias);
                p.C[static_cast<uint64_t>(m) * p.ldc + n] = dev::epilogue(out, p.epilogue);
            }
        }
    }
}

}  // namespace

void gemm_i8(hipStream_t s, const I8Gemm &p)
{
    dim3 grid((p.N + BN - 1) / BN, (p.M + BM - 1) / BM);
    gemm_i8_kernel<<<grid, kThreads, 0, s>>>(p);
}

}  // namespace k
}  // namespace vnpu
