// quantize.hip - QUANTIZE_I8 on gfx950 (symmetric int8, bit-exact).
//
// Semantics (reference src/kernels/llm.cpp:387-436, scheduler.cpp:430-473):
//   scale = max|x| / 127 (zero or non-finite -> 1), inv = 1 / scale,
//   q = clamp(round_half_away(x * inv), -128, 127).
// Every step is an IEEE single operation with the reference's rounding:
// __fdiv_rn / __fmul_rn pin the correctly rounded divide and multiply, and
// roundf lowers to trunc + half-away adjust on AMDGPU.  Max ignores NaN
// exactly as std::max(m, NaN) does (fmaxf returns the non-NaN operand).
//
// HBM-bound: per-row reads each element once (kept in registers between the
// max pass and the quantize pass) and writes one byte, 5 bytes per element.
#include "kernels.hpp"
#include "device_math.hpp"

#include <algorithm>

namespace vnpu {
namespace k {
namespace {

constexpr int kThreads = 256;

using dev::q8;
using dev::scale_from_max;

__device__ __forceinline__ float block_max(float v, float *red)
{
    v = dev::wave_max(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) r = fmaxf(r, red[w]);
    return r;
}

// One workgroup per row; the row stays in registers (VPT float4 per thread).
template <int VPT>
__global__ __launch_bounds__(kThreads) void quant_rows_reg(const float *__restrict__ X,
                                                           int8_t *__restrict__ Y,
                                                           float *__restrict__ scales,
                                                           uint32_t cols)
{
    __shared__ float red[kThreads / 64];
    const uint64_t r = blockIdx.x;
    // The row through raw buffers: slots past it read zeros and their stores
    // are dropped, so no branch sits around a load or a store.
    const auto rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(X + r * cols), 0,
                                                      static_cast<int>(cols * 4u), 0x00020000);
    const auto ry = __builtin_amdgcn_make_buffer_rsrc(Y + r * cols, 0, static_cast<int>(cols), 0x00020000);
    float4 v[VPT];
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t j = threadIdx.x + i * kThreads;
        v[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rx, j * 16u, 0, 0));
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    }
    const float scale = scale_from_max(block_max(m, red));
    const float inv = __fdiv_rn(1.0f, scale);
    if (threadIdx.x == 0) scales[r] = scale;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t j = threadIdx.x + i * kThreads;
        const char4 q = make_char4(q8(v[i].x, inv), q8(v[i].y, inv), q8(v[i].z, inv), q8(v[i].w, inv));
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, q), ry, j * 4u, 0, 0);
    }
}

// Any row length / alignment: two passes over the row (second from cache).
__global__ __launch_bounds__(kThreads) void quant_rows_any(const float *__restrict__ X,
                                                           int8_t *__restrict__ Y,
                                                           float *__restrict__ scales,
                                                           uint64_t cols)
{
    __shared__ float red[kThreads / 64];
    const uint64_t r = blockIdx.x;
    const float *row = X + r * cols;
    float m = 0.0f;
    for (uint64_t j = threadIdx.x; j < cols; j += kThreads) m = fmaxf(m, fabsf(row[j]));
    const float scale = scale_from_max(block_max(m, red));
    const float inv = __fdiv_rn(1.0f, scale);
    if (threadIdx.x == 0) scales[r] = scale;
    for (uint64_t j = threadIdx.x; j < cols; j += kThreads) Y[r * cols + j] = q8(row[j], inv);
}

// Per-column quantization in two bandwidth-shaped passes over a grid of
// (256-column chunk) x (row range): every thread owns one column, so each
// row of a chunk is one coalesced 1 KiB read.
//   1. partial maxima of |x| (fmaxf ignores NaN, as the reference's max does)
//      folded into colmax[] with an integer atomicMax on the float's bits,
//      which orders non-negative floats exactly - the result does not depend
//      on the order the row ranges arrive in;
//   2. scale = max/127 (0 or non-finite -> 1), q = round(x * (1/scale)).
__global__ __launch_bounds__(kThreads) void quant_cols_max(const float *__restrict__ X,
                                                           uint64_t rows, uint64_t cols,
                                                           uint64_t rows_per,
                                                           uint32_t *__restrict__ colmax)
{
    const uint64_t c = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (c >= cols) return;
    const uint64_t r0 = static_cast<uint64_t>(blockIdx.y) * rows_per;
    const uint64_t r1 = min(rows, r0 + rows_per);
    float m0 = 0.0f, m1 = 0.0f, m2 = 0.0f, m3 = 0.0f;
    uint64_t r = r0;
    for (; r + 4 <= r1; r += 4) {
        m0 = fmaxf(m0, fabsf(X[(r + 0) * cols + c]));
        m1 = fmaxf(m1, fabsf(X[(r + 1) * cols + c]));
        m2 = fmaxf(m2, fabsf(X[(r + 2) * cols + c]));
        m3 = fmaxf(m3, fabsf(X[(r + 3) * cols + c]));
    }
    for (; r < r1; ++r) m0 = fmaxf(m0, fabsf(X[r * cols + c]));
    const float m = fmaxf(fmaxf(m0, m1), fmaxf(m2, m3));
    atomicMax(colmax + c, __float_as_uint(m));
}

__global__ __launch_bounds__(kThreads) void quant_cols_apply(const float *__restrict__ X,
                                                             int8_t *__restrict__ Y,
                                                             float *__restrict__ scales,
                                                             uint64_t rows, uint64_t cols,
                                                             uint64_t rows_per,
                                                             const uint32_t *__restrict__ colmax)
{
    const uint64_t c = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (c >= cols) return;
    const float scale = scale_from_max(__uint_as_float(colmax[c]));
    const float inv = __fdiv_rn(1.0f, scale);
    if (blockIdx.y == 0) scales[c] = scale;
    const uint64_t r0 = static_cast<uint64_t>(blockIdx.y) * rows_per;
    const uint64_t r1 = min(rows, r0 + rows_per);
#pragma unroll 4
    for (uint64_t r = r0; r < r1; ++r) Y[r * cols + c] = q8(X[r * cols + c], inv);
}

constexpr int kTensorBlocks = 1024;

__global__ __launch_bounds__(kThreads) void tensor_partial_max(const float *__restrict__ X,
                                                               uint64_t n, float *__restrict__ ws)
{
    __shared__ float red[kThreads / 64];
    float m = 0.0f;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * kThreads)
        m = fmaxf(m, fabsf(X[i]));
    m = block_max(m, red);
    if (threadIdx.x == 0) ws[blockIdx.x] = m;
}

__global__ __launch_bounds__(kThreads) void tensor_scale(const float *__restrict__ ws,
                                                         float *__restrict__ scales)
{
    __shared__ float red[kThreads / 64];
    float m = 0.0f;
    for (int i = threadIdx.x; i < kTensorBlocks; i += kThreads) m = fmaxf(m, ws[i]);
    m = block_max(m, red);
    if (threadIdx.x == 0) scales[0] = scale_from_max(m);
}

// reference llm.cpp:430-436: inv = 1 / (scale > 0 ? scale : 1)
__global__ __launch_bounds__(kThreads) void tensor_quant(const float *__restrict__ X,
                                                         int8_t *__restrict__ Y, uint64_t n,
                                                         const float *__restrict__ scales)
{
    const float s = scales[0];
    const float inv = __fdiv_rn(1.0f, s > 0.0f ? s : 1.0f);
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * kThreads)
        Y[i] = q8(X[i], inv);
}

}  // namespace

void quantize_rows(hipStream_t s, const float *X, int8_t *Y, float *scales, uint64_t rows,
                   uint64_t cols)
{
    const bool aligned = (cols % 4 == 0) && (reinterpret_cast<uintptr_t>(X) % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(Y) % 4 == 0);
    const uint64_t n4 = cols / 4;
    for (uint64_t r0 = 0; r0 < rows; r0 += 0x7fffffffull) {
        const uint64_t nr = rows - r0 < 0x7fffffffull ? rows - r0 : 0x7fffffffull;
        const float *x = X + r0 * cols;
        int8_t *y = Y + r0 * cols;
        float *sc = scales + r0;
        dim3 grid(static_cast<uint32_t>(nr));
        if (aligned && n4 <= kThreads * 1)
            quant_rows_reg<1><<<grid, kThreads, 0, s>>>(x, y, sc, static_cast<uint32_t>(cols));
        else if (aligned && n4 <= kThreads * 4)
            quant_rows_reg<4><<<grid, kThreads, 0, s>>>(x, y, sc, static_cast<uint32_t>(cols));
        else if (aligned && n4 <= kThreads * 12)
            quant_rows_reg<12><<<grid, kThreads, 0, s>>>(x, y, sc, static_cast<uint32_t>(cols));
        else
            quant_rows_any<<<grid, kThreads, 0, s>>>(x, y, sc, cols);
    }
}

size_t quantize_cols_ws_bytes(uint64_t cols) { return static_cast<size_t>(cols) * sizeof(uint32_t); }

void quantize_cols(hipStream_t s, const float *X, int8_t *Y, float *scales, uint64_t rows,
                   uint64_t cols, uint32_t *ws)
{
    // ~2048 workgroups, at least 16 rows each.
    const uint64_t chunks = (cols + kThreads - 1) / kThreads;
    const uint64_t max_splits = (rows + 15) / 16;
    const uint64_t splits = std::max<uint64_t>(1, std::min<uint64_t>(max_splits, (2048 + chunks - 1) / chunks));
    const uint64_t rows_per = (rows + splits - 1) / splits;
    const uint64_t ysplits = (rows + rows_per - 1) / rows_per;
    fill_u8(s, ws, 0, quantize_cols_ws_bytes(cols));   // a kernel, not a memset
    const dim3 grid(static_cast<uint32_t>(chunks), static_cast<uint32_t>(ysplits));
    quant_cols_max<<<grid, kThreads, 0, s>>>(X, rows, cols, rows_per, ws);
    quant_cols_apply<<<grid, kThreads, 0, s>>>(X, Y, scales, rows, cols, rows_per, ws);
}

size_t quantize_tensor_ws_bytes() { return kTensorBlocks * sizeof(float); }

void quantize_tensor(hipStream_t s, const float *X, int8_t *Y, float *scales, uint64_t count,
                     float *ws)
{
    tensor_partial_max<<<kTensorBlocks, kThreads, 0, s>>>(X, count, ws);
    tensor_scale<<<1, kThreads, 0, s>>>(ws, scales);
    tensor_quant<<<kTensorBlocks, kThreads, 0, s>>>(X, Y, count, scales);
}

}  // namespace k
}  // namespace vnpu
