// pack.hip - PACK_WEIGHTS_I8: int8 weights -> HBM-resident fragment layout.
//
// The reference packs into a VNNI panel [Npad/16][Kpad/4][16][4] that its
// AVX2 kernels never read (src/core/scheduler.cpp:763-836).  This backend
// packs into the layout its gfx950 kernels consume directly:
//
//   frag[nt][kt][kg][c][j] = B[k = 64*kt + 16*kg + j][n = 16*nt + c]
//
// with nt < Np/16, kt < Kp/64, kg < 4, c < 16, j < 16 (zero padded).  One
// (kt, nt) block is 1 KiB: lane l = 16*kg + c of a wave loads the 16 bytes
// at 16*l, i.e. 16 consecutive k of one column, which is the per-lane B
// operand of the int8 MFMAs and four v_dot4 of the GEMV.  Blocks are stored
// column-strip-major: the Kp/64 blocks of one 16-column strip are one
// contiguous run, so the decode GEMV streams each strip sequentially.
//
// With a Wildcat weight-tile mask (tile_mask[kb * mask_ld + g], one byte per
// 64 x 64 tile: k block kb, columns 64 g .. 64 g + 63), a zero byte packs its
// tile as zeros whatever B holds there.
//
// Also produced: per-column sums (reference scheduler.cpp:798-800), and for
// each group of four strips (64 columns, the reference's 64 x 64 cull tile
// width) the list of its 64-deep k blocks that hold a nonzero weight, which
// the strip GEMM walks instead of every k block.
#include "kernels.hpp"

namespace vnpu {
namespace k {
namespace {

__global__ __launch_bounds__(256) void pack_frag_kernel(const int8_t *__restrict__ B, uint32_t K,
                                                        uint32_t N, uint32_t ldb, uint32_t trans_b,
                                                        const uint8_t *__restrict__ tile_mask, uint32_t mask_ld,
                                                        int8_t *__restrict__ frag, uint32_t KT,
                                                        uint64_t chunks)
{
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= chunks) return;
    // idx = ((nt * KT + kt) * 4 + kg) * 16 + c
    const uint32_t c = idx & 15;
    const uint32_t kg = (idx >> 4) & 3;
    const uint64_t blk = idx >> 6;
    const uint32_t kt = static_cast<uint32_t>(blk % KT);
    const uint32_t nt = static_cast<uint32_t>(blk / KT);
    const uint32_t n = nt * 16 + c;
    const uint32_t k0 = kt * 64 + kg * 16;
    // The 16 k of this chunk lie in k block kt, its column in group n / 64.
    const bool culled = tile_mask && n < N && tile_mask[static_cast<uint64_t>(kt) * mask_ld + n / 64] == 0;
    union {
        int8_t b[16];
        int4 v;
    } u;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const uint32_t k = k0 + j;
        int8_t v = 0;
        if (n < N && k < K && !culled)
            v = trans_b ? B[static_cast<uint64_t>(n) * ldb + k] : B[static_cast<uint64_t>(k) * ldb + n];
        u.b[j] = v;
    }
    reinterpret_cast<int4 *>(frag)[idx] = u.v;
}

// One workgroup per 16-column strip: the strip's blocks are contiguous, lane
// 16*kg + c sums its 16 bytes of column c with one v_dot4 against ones, the
// four k groups reduce by shuffles and the waves through LDS.  Padding is
// zero, so the sums equal those over the K x N weights.
__global__ __launch_bounds__(256) void column_sums_kernel(const int8_t *__restrict__ frag,
                                                          uint32_t KT, uint32_t N,
                                                          int32_t *__restrict__ sums)
{
    __shared__ int red[4][16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t nt = blockIdx.x;
    const int4 *strip = reinterpret_cast<const int4 *>(frag + static_cast<uint64_t>(nt) * KT * 1024);
    const int ones = 0x01010101;
    int s = 0;
    for (uint32_t kt = wave; kt < KT; kt += 4) {
        const int4 v = strip[static_cast<uint64_t>(kt) * 64 + lane];
        s = __builtin_amdgcn_sdot4(v.x, ones, s, false);
        s = __builtin_amdgcn_sdot4(v.y, ones, s, false);
        s = __builtin_amdgcn_sdot4(v.z, ones, s, false);
        s = __builtin_amdgcn_sdot4(v.w, ones, s, false);
    }
    s += __shfl_xor(s, 16, 64);
    s += __shfl_xor(s, 32, 64);
    if (lane < 16) red[wave][lane] = s;
    __syncthreads();
    if (tid < 16) {
        const uint32_t n = nt * 16 + tid;
        if (n < N) sums[n] = red[0][tid] + red[1][tid] + red[2][tid] + red[3][tid];
    }
}

// Which 64 x 64 weight tiles hold a nonzero: one wave per (k block, group
// of four 16-column strips); flag[g][kt] = 1 when any of the group's four
// 1 KiB blocks at k block kt is nonzero.
__global__ __launch_bounds__(64) void tile_nz_kernel(const int8_t *__restrict__ frag, uint32_t KT, uint32_t NT,
                                                     uint8_t *__restrict__ flag)
{
    const uint32_t kt = blockIdx.x, g = blockIdx.y;
    const int lane = threadIdx.x;
    int any = 0;
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        const uint32_t nt = 4 * g + j;
        if (nt >= NT) break;   // uniform
        const int4 v = reinterpret_cast<const int4 *>(frag + (static_cast<uint64_t>(nt) * KT + kt) * 1024)[lane];
        any |= v.x | v.y | v.z | v.w;
    }
    const uint64_t nz = __ballot(any != 0);
    if (lane == 0) flag[static_cast<uint64_t>(g) * KT + kt] = nz != 0 ? 1 : 0;
}

// Each group's nonzero k blocks in ascending order: list[g][0 .. count[g]).
__global__ __launch_bounds__(64) void tile_list_kernel(const uint8_t *__restrict__ flag, uint32_t KT, uint32_t NG,
                                                       uint32_t *__restrict__ list, uint32_t *__restrict__ count)
{
    const uint32_t g = blockIdx.x * 64 + threadIdx.x;
    if (g >= NG) return;
    uint32_t n = 0;
    for (uint32_t kt = 0; kt < KT; ++kt)
        if (flag[static_cast<uint64_t>(g) * KT + kt]) list[static_cast<uint64_t>(g) * KT + n++] = kt;
    count[g] = n;
}

}  // namespace

void tile_lists(hipStream_t s, const int8_t *frag, uint32_t Kp, uint32_t Np, uint8_t *flag, uint32_t *list,
                uint32_t *count)
{
    const uint32_t KT = Kp / 64, NT = Np / 16, NG = (NT + 3) / 4;
    tile_nz_kernel<<<dim3(KT, NG), 64, 0, s>>>(frag, KT, NT, flag);
    tile_list_kernel<<<dim3((NG + 63) / 64), 64, 0, s>>>(flag, KT, NG, list, count);
}

void pack_fragments(hipStream_t s, const int8_t *B, uint32_t K, uint32_t N, uint32_t ldb,
                    uint32_t trans_b, const uint8_t *tile_mask, uint32_t mask_ld, int8_t *frag,
                    uint32_t Kp, uint32_t Np, int32_t *column_sums)
{
    const uint32_t NT = Np / 16, KT = Kp / 64;
    const uint64_t blocks = static_cast<uint64_t>(KT) * NT;
    const uint64_t chunks = blocks * 64;
    pack_frag_kernel<<<dim3(static_cast<uint32_t>((chunks + 255) / 256)), 256, 0, s>>>(
        B, K, N, ldb, trans_b, tile_mask, mask_ld, frag, KT, chunks);
    column_sums_kernel<<<dim3(NT), 256, 0, s>>>(frag, KT, N, column_sums);
}

}  // namespace k
}  // namespace vnpu
