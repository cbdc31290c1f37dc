// pack.hip - PACK_WEIGHTS_I8: int8 weights -> HBM-resident fragment layout.
//
// The reference packs into a VNNI panel [Npad/16][Kpad/4][16][4] that its
// AVX2 kernels never read (src/core/scheduler.cpp:763-836).  This backend
// packs into the layout its gfx950 kernels consume directly:
//
//   frag[kt][nt][kg][c][j] = B[k = 64*kt + 16*kg + j][n = 16*nt + c]
//
// with kt < Kp/64, nt < Np/16, kg < 4, c < 16, j < 16 (zero padded).  One
// (kt, nt) block is 1 KiB and is exactly the B operand of one
// v_mfma_i32_16x16x64_i8: lane l = 16*kg + c loads the 16 bytes at 16*l.
// For a fixed kt the Np/16 blocks are contiguous, so a workgroup's B tile of
// BN columns is one contiguous BN*64-byte run per k step.
//
// Also produced: per-column sums (reference scheduler.cpp:798-800) and a
// per-block all-zero map that lets MATMUL_I8 skip zero weight blocks exactly.
#include "kernels.hpp"

namespace vnpu {
namespace k {
namespace {

__global__ __launch_bounds__(256) void pack_frag_kernel(const int8_t *__restrict__ B, uint32_t K,
                                                        uint32_t N, uint32_t ldb, uint32_t trans_b,
                                                        int8_t *__restrict__ frag, uint32_t NT,
                                                        uint64_t chunks)
{
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= chunks) return;
    // idx = ((kt * NT + nt) * 4 + kg) * 16 + c
    const uint32_t c = idx & 15;
    const uint32_t kg = (idx >> 4) & 3;
    const uint64_t blk = idx >> 6;
    const uint32_t nt = static_cast<uint32_t>(blk % NT);
    const uint32_t kt = static_cast<uint32_t>(blk / NT);
    const uint32_t n = nt * 16 + c;
    const uint32_t k0 = kt * 64 + kg * 16;
    union {
        int8_t b[16];
        int4 v;
    } u;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const uint32_t k = k0 + j;
        int8_t v = 0;
        if (n < N && k < K)
            v = trans_b ? B[static_cast<uint64_t>(n) * ldb + k] : B[static_cast<uint64_t>(k) * ldb + n];
        u.b[j] = v;
    }
    reinterpret_cast<int4 *>(frag)[idx] = u.v;
}

__global__ __launch_bounds__(256) void column_sums_kernel(const int8_t *__restrict__ B, uint32_t K,
                                                          uint32_t N, uint32_t ldb,
                                                          uint32_t trans_b,
                                                          int32_t *__restrict__ sums)
{
    const uint32_t n = blockIdx.x * 256 + threadIdx.x;
    if (n >= N) return;
    int32_t s = 0;
    if (trans_b) {
        const int8_t *row = B + static_cast<uint64_t>(n) * ldb;
        for (uint32_t k = 0; k < K; ++k) s += row[k];
    } else {
        for (uint32_t k = 0; k < K; ++k) s += B[static_cast<uint64_t>(k) * ldb + n];
    }
    sums[n] = s;
}

// One wave per 1 KiB block: 1 if every byte is zero.
__global__ __launch_bounds__(64) void zero_block_kernel(const int8_t *__restrict__ frag,
                                                        uint8_t *__restrict__ zero_blocks)
{
    const uint64_t blk = blockIdx.x;
    const int4 v = reinterpret_cast<const int4 *>(frag + blk * 1024)[threadIdx.x];
    const int any = (v.x | v.y | v.z | v.w) != 0;
    const unsigned long long nz = __ballot(any);
    if (threadIdx.x == 0) zero_blocks[blk] = nz == 0ull ? 1 : 0;
}

}  // namespace

void pack_fragments(hipStream_t s, const int8_t *B, uint32_t K, uint32_t N, uint32_t ldb,
                    uint32_t trans_b, int8_t *frag, uint32_t Kp, uint32_t Np,
                    int32_t *column_sums, uint8_t *zero_blocks)
{
    const uint32_t NT = Np / 16;
    const uint64_t blocks = static_cast<uint64_t>(Kp / 64) * NT;
    const uint64_t chunks = blocks * 64;
    pack_frag_kernel<<<dim3(static_cast<uint32_t>((chunks + 255) / 256)), 256, 0, s>>>(
        B, K, N, ldb, trans_b, frag, NT, chunks);
    column_sums_kernel<<<dim3((N + 255) / 256), 256, 0, s>>>(B, K, N, ldb, trans_b, column_sums);
    zero_block_kernel<<<dim3(static_cast<uint32_t>(blocks)), 64, 0, s>>>(frag, zero_blocks);
}

}  // namespace k
}  // namespace vnpu
