// ops.hip - bandwidth-bound transformer ops on gfx950.
//
// RMSNORM, SOFTMAX, ROPE, SWIGLU, ADD, MUL, GELU with the reference's
// semantics and defaults (src/kernels/llm.cpp:64-330, 576-602;
// src/core/scheduler.cpp:475-581).  Row ops use one workgroup per row with
// wave-shuffle + LDS reductions; elementwise ops are grid-stride float4
// streams.  All are HBM-bound: the algorithmic bytes are the reads and writes
// of each element once (rows are re-read from cache between passes).
#include "kernels.hpp"
#include "device_math.hpp"

namespace vnpu {
namespace k {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float block_sum(float v, float *red)
{
    v = dev::wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = 0.0f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) r += red[w];
    return r;
}

__device__ __forceinline__ float block_max(float v, float *red)
{
    v = dev::wave_max(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) r = fmaxf(r, red[w]);
    return r;
}

// reference llm.cpp:64-108: inv = 1/sqrt(sum(x^2)/cols + eps); y = x*inv*w
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const float *__restrict__ X,
                                                           const float *__restrict__ W,
                                                           float *__restrict__ Y, uint32_t cols,
                                                           float eps)
{
    __shared__ float red[kThreads / 64];
    const uint64_t r = blockIdx.x;
    const float *x = X + r * cols;
    float *y = Y + r * cols;
    float ss = 0.0f;
    for (uint32_t j = threadIdx.x; j < cols; j += kThreads) ss = fmaf(x[j], x[j], ss);
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
    for (uint32_t j = threadIdx.x; j < cols; j += kThreads) y[j] = x[j] * inv * (W ? W[j] : 1.0f);
}

__global__ __launch_bounds__(kThreads) void rmsnorm_vec_kernel(const float *__restrict__ X,
                                                               const float *__restrict__ W,
                                                               float *__restrict__ Y,
                                                               uint32_t cols, float eps)
{
    __shared__ float red[kThreads / 64];
    const uint64_t r = blockIdx.x;
    const float4 *x = reinterpret_cast<const float4 *>(X + r * cols);
    float4 *y = reinterpret_cast<float4 *>(Y + r * cols);
    const float4 *w = reinterpret_cast<const float4 *>(W);
    const uint32_t n4 = cols >> 2;
    float ss = 0.0f;
    for (uint32_t j = threadIdx.x; j < n4; j += kThreads) {
        const float4 v = x[j];
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
    for (uint32_t j = threadIdx.x; j < n4; j += kThreads) {
        const float4 v = x[j];
        const float4 g = W ? w[j] : make_float4(1.f, 1.f, 1.f, 1.f);
        y[j] = make_float4(v.x * inv * g.x, v.y * inv * g.y, v.z * inv * g.z, v.w * inv * g.w);
    }
}

// Rows of up to VPT*1024 floats, 16-byte aligned: the row stays in registers
// between the sum of squares and the scaling (one HBM read instead of two).
template <int VPT>
__global__ __launch_bounds__(kThreads) void rmsnorm_reg_kernel(const float *__restrict__ X,
                                                               const float *__restrict__ W,
                                                               float *__restrict__ Y, uint32_t cols,
                                                               float eps)
{
    __shared__ float red[kThreads / 64];
    const uint64_t r = blockIdx.x;
    const float4 *x = reinterpret_cast<const float4 *>(X + r * cols);
    float4 *y = reinterpret_cast<float4 *>(Y + r * cols);
    const float4 *w = reinterpret_cast<const float4 *>(W);
    const uint32_t n4 = cols >> 2;
    float4 v[VPT];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t j = threadIdx.x + i * kThreads;
        v[i] = j < n4 ? x[j] : make_float4(0.f, 0.f, 0.f, 0.f);
        ss = fmaf(v[i].x, v[i].x, ss);
        ss = fmaf(v[i].y, v[i].y, ss);
        ss = fmaf(v[i].z, v[i].z, ss);
        ss = fmaf(v[i].w, v[i].w, ss);
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t j = threadIdx.x + i * kThreads;
        if (j >= n4) continue;
        const float4 g = W ? w[j] : make_float4(1.f, 1.f, 1.f, 1.f);
        y[j] = make_float4(v[i].x * inv * g.x, v[i].y * inv * g.y, v[i].z * inv * g.z, v[i].w * inv * g.w);
    }
}

// reference llm.cpp:116-180 (exp is the reference's polynomial)
__global__ __launch_bounds__(kThreads) void softmax_kernel(const float *__restrict__ X,
                                                           float *__restrict__ Y, uint32_t cols,
                                                           float inv_t)
{
    __shared__ float red[kThreads / 64];
    const uint64_t r = blockIdx.x;
    const float *x = X + r * cols;
    float *y = Y + r * cols;
    float mx = -__builtin_inff();
    for (uint32_t j = threadIdx.x; j < cols; j += kThreads) mx = fmaxf(mx, x[j]);
    mx = block_max(mx, red);
    float sum = 0.0f;
    for (uint32_t j = threadIdx.x; j < cols; j += kThreads) sum += dev::fast_expf((x[j] - mx) * inv_t);
    sum = block_sum(sum, red);
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (uint32_t j = threadIdx.x; j < cols; j += kThreads) y[j] = dev::fast_expf((x[j] - mx) * inv_t) * inv;
}

// Few long rows (e.g. the MTP head's [4, 32000] logits): each row is split
// into chunks over many workgroups, in three passes that keep the
// reference's terms exactly: chunk maxima -> the row max M; chunk sums of
// fast_expf((x - M) * inv_t) -> the row sum L; y = fast_expf((x - M) * inv_t)
// * (1 / L).  ws holds rows x chunks x 2 floats.
__device__ __forceinline__ float row_max_of(const float *part, uint32_t chunks, float *red)
{
    float m = -__builtin_inff();
    for (uint32_t c = threadIdx.x; c < chunks; c += kThreads) m = fmaxf(m, part[2 * c]);
    return block_max(m, red);
}

__device__ __forceinline__ float row_sum_of(const float *part, uint32_t chunks, float *red)
{
    float s = 0.0f;
    for (uint32_t c = threadIdx.x; c < chunks; c += kThreads) s += part[2 * c + 1];
    return block_sum(s, red);
}

__global__ __launch_bounds__(kThreads) void softmax_chunk_max(const float *__restrict__ X,
                                                              uint32_t cols, uint32_t chunk,
                                                              float *__restrict__ ws)
{
    __shared__ float red[kThreads / 64];
    const uint64_t r = blockIdx.y;
    const uint32_t c0 = blockIdx.x * chunk, c1 = min(cols, c0 + chunk);
    const float *x = X + r * cols;
    float mx = -__builtin_inff();
    for (uint32_t j = c0 + threadIdx.x; j < c1; j += kThreads) mx = fmaxf(mx, x[j]);
    mx = block_max(mx, red);
    if (threadIdx.x == 0) ws[(r * gridDim.x + blockIdx.x) * 2] = mx;
}

__global__ __launch_bounds__(kThreads) void softmax_chunk_sum(const float *__restrict__ X,
                                                              uint32_t cols, uint32_t chunk,
                                                              float inv_t, float *__restrict__ ws)
{
    __shared__ float red[kThreads / 64];
    const uint64_t r = blockIdx.y;
    const uint32_t c0 = blockIdx.x * chunk, c1 = min(cols, c0 + chunk);
    const float *x = X + r * cols;
    const float mx = row_max_of(ws + r * gridDim.x * 2, gridDim.x, red);
    float sum = 0.0f;
    for (uint32_t j = c0 + threadIdx.x; j < c1; j += kThreads) sum += dev::fast_expf((x[j] - mx) * inv_t);
    sum = block_sum(sum, red);
    if (threadIdx.x == 0) ws[(r * gridDim.x + blockIdx.x) * 2 + 1] = sum;
}

__global__ __launch_bounds__(kThreads) void softmax_chunk_norm(const float *__restrict__ X,
                                                               float *__restrict__ Y, uint32_t cols,
                                                               uint32_t chunk, float inv_t,
                                                               const float *__restrict__ ws)
{
    __shared__ float red[kThreads / 64];
    const uint64_t r = blockIdx.y;
    const uint32_t c0 = blockIdx.x * chunk, c1 = min(cols, c0 + chunk);
    const float *part = ws + r * gridDim.x * 2;
    const float mx = row_max_of(part, gridDim.x, red);
    const float sum = row_sum_of(part, gridDim.x, red);
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    const float *x = X + r * cols;
    float *y = Y + r * cols;
    for (uint32_t j = c0 + threadIdx.x; j < c1; j += kThreads) y[j] = dev::fast_expf((x[j] - mx) * inv_t) * inv;
}

// reference llm.cpp:188-217, 576-602: one thread per rotated pair.
__global__ __launch_bounds__(kThreads) void rope_kernel(float *__restrict__ Q, float *__restrict__ K,
                                                        const int32_t *__restrict__ positions,
                                                        uint64_t bh_count, uint32_t q_seq,
                                                        uint32_t k_seq, uint32_t seq,
                                                        uint32_t head_dim, uint32_t offset,
                                                        uint32_t interleaved, float scaling,
                                                        const float *__restrict__ inv_freq)
{
    const uint32_t half = head_dim / 2;
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const uint64_t total = bh_count * seq * half;
    if (idx >= total) return;
    const uint32_t j = static_cast<uint32_t>(idx % half);
    const uint64_t tok = idx / half;
    const uint32_t t = static_cast<uint32_t>(tok % seq);
    const uint64_t bh = tok / seq;
    const float pos = static_cast<float>(positions ? positions[t] : static_cast<int32_t>(t + offset));
    const float angle = (pos * scaling) * inv_freq[j];
    const float c = cosf(angle), s = sinf(angle);
    const uint32_t i0 = interleaved ? 2 * j : j;
    const uint32_t i1 = interleaved ? 2 * j + 1 : j + half;
    if (Q && t < q_seq) {
        float *x = Q + (bh * q_seq + t) * head_dim;
        const float x0 = x[i0], x1 = x[i1];
        x[i0] = x0 * c - x1 * s;
        x[i1] = x0 * s + x1 * c;
    }
    if (K && t < k_seq) {
        float *x = K + (bh * k_seq + t) * head_dim;
        const float x0 = x[i0], x1 = x[i1];
        x[i0] = x0 * c - x1 * s;
        x[i1] = x0 * s + x1 * c;
    }
}

// Half-rotation layout with head_dim % 8 == 0 and 16-byte aligned rows: one
// thread rotates pairs j..j+3 with one float4 from each half of the row.
__device__ __forceinline__ void rotate4(float *row, uint32_t j4, uint32_t half4, const float (&c)[4],
                                        const float (&s)[4])
{
    float4 *x = reinterpret_cast<float4 *>(row);
    const float4 a = x[j4], b = x[half4 + j4];
    x[j4] = make_float4(a.x * c[0] - b.x * s[0], a.y * c[1] - b.y * s[1], a.z * c[2] - b.z * s[2],
                        a.w * c[3] - b.w * s[3]);
    x[half4 + j4] = make_float4(a.x * s[0] + b.x * c[0], a.y * s[1] + b.y * c[1], a.z * s[2] + b.z * c[2],
                                a.w * s[3] + b.w * c[3]);
}

__global__ __launch_bounds__(kThreads) void rope_vec_kernel(float *__restrict__ Q, float *__restrict__ K,
                                                            const int32_t *__restrict__ positions,
                                                            uint64_t bh_count, uint32_t q_seq,
                                                            uint32_t k_seq, uint32_t seq,
                                                            uint32_t head_dim, uint32_t offset,
                                                            float scaling,
                                                            const float *__restrict__ inv_freq)
{
    const uint32_t half4 = head_dim / 8;
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (idx >= bh_count * seq * half4) return;
    const uint32_t j4 = static_cast<uint32_t>(idx % half4);
    const uint64_t tok = idx / half4;
    const uint32_t t = static_cast<uint32_t>(tok % seq);
    const uint64_t bh = tok / seq;
    const float pos = static_cast<float>(positions ? positions[t] : static_cast<int32_t>(t + offset));
    float c[4], s[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float angle = (pos * scaling) * inv_freq[4 * j4 + e];
        c[e] = cosf(angle);
        s[e] = sinf(angle);
    }
    if (Q && t < q_seq) rotate4(Q + (bh * q_seq + t) * head_dim, j4, half4, c, s);
    if (K && t < k_seq) rotate4(K + (bh * k_seq + t) * head_dim, j4, half4, c, s);
}

enum EwOp { EW_SWIGLU = 0, EW_ADD = 1, EW_MUL = 2, EW_GELU = 3 };

template <int OP>
__device__ __forceinline__ float ew(float a, float b, float alpha, float beta)
{
    if (OP == EW_SWIGLU) return dev::silu(a) * b * alpha;        // llm.cpp:240-246
    if (OP == EW_ADD) return fmaf(a, alpha, b * beta);           // llm.cpp:256-271
    if (OP == EW_MUL) return fmaf(a * b, alpha, beta);           // llm.cpp:273-287
    return dev::gelu_tanh(a);                                    // llm.cpp:248-253
}

template <int OP>
__global__ __launch_bounds__(kThreads) void ew_vec_kernel(const float4 *__restrict__ A,
                                                          const float4 *__restrict__ B,
                                                          float4 *__restrict__ Y, uint64_t n4,
                                                          float alpha, float beta)
{
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n4;
         i += static_cast<uint64_t>(gridDim.x) * kThreads) {
        const float4 a = A[i];
        const float4 b = (OP == EW_GELU) ? a : B[i];
        Y[i] = make_float4(ew<OP>(a.x, b.x, alpha, beta), ew<OP>(a.y, b.y, alpha, beta),
                           ew<OP>(a.z, b.z, alpha, beta), ew<OP>(a.w, b.w, alpha, beta));
    }
}

template <int OP>
__global__ __launch_bounds__(kThreads) void ew_kernel(const float *__restrict__ A,
                                                      const float *__restrict__ B,
                                                      float *__restrict__ Y, uint64_t n,
                                                      float alpha, float beta)
{
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * kThreads)
        Y[i] = ew<OP>(A[i], (OP == EW_GELU) ? 0.0f : B[i], alpha, beta);
}

template <int OP>
void launch_ew(hipStream_t s, const float *A, const float *B, float *Y, uint64_t n, float alpha,
               float beta)
{
    const bool vec = (n % 4 == 0) && ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(Y) |
                                       (B ? reinterpret_cast<uintptr_t>(B) : 0)) % 16 == 0);
    const uint64_t work = vec ? n / 4 : n;
    uint64_t blocks = (work + kThreads - 1) / kThreads;
    if (blocks > 8192) blocks = 8192;
    if (blocks == 0) blocks = 1;
    if (vec)
        ew_vec_kernel<OP><<<dim3(static_cast<uint32_t>(blocks)), kThreads, 0, s>>>(
            reinterpret_cast<const float4 *>(A), reinterpret_cast<const float4 *>(B),
            reinterpret_cast<float4 *>(Y), n / 4, alpha, beta);
    else
        ew_kernel<OP><<<dim3(static_cast<uint32_t>(blocks)), kThreads, 0, s>>>(A, B, Y, n, alpha, beta);
}

template <int NT>
__device__ __forceinline__ float block_max_n(float v, float *red)
{
    v = dev::wave_max(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) r = fmaxf(r, red[w]);
    return r;
}

template <int NT>
__device__ __forceinline__ float block_sum_n(float v, float *red)
{
    v = dev::wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = 0.0f;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) r += red[w];
    return r;
}

// Softmax of few long rows (the MTP head's [gamma, vocab] logits) in one
// launch: a 1024-thread workgroup per row keeps the row in registers, takes
// the max, then each e = fast_expf((x - max) * inv_t) once (kept for the
// output) and their sum; y = e * (1 / sum), the reference's terms
// (llm.cpp:116-134) with a tree sum.
template <int VPT>
__global__ __launch_bounds__(1024) void softmax_reg_kernel(const float *__restrict__ X, float *__restrict__ Y,
                                                          uint32_t cols, float inv_t)
{
    __shared__ float red[1024 / 64];
    const uint64_t r = blockIdx.x;
    const float4 *x = reinterpret_cast<const float4 *>(X + r * cols);
    float4 *y = reinterpret_cast<float4 *>(Y + r * cols);
    const uint32_t n4 = cols >> 2;
    const float ninf = -__builtin_inff();
    float4 v[VPT];
    float mx = ninf;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t j = threadIdx.x + i * 1024;
        v[i] = j < n4 ? x[j] : make_float4(ninf, ninf, ninf, ninf);
        mx = fmaxf(mx, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
    }
    mx = block_max_n<1024>(mx, red);
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t j = threadIdx.x + i * 1024;
        if (j >= n4) continue;
        v[i] = make_float4(dev::fast_expf((v[i].x - mx) * inv_t), dev::fast_expf((v[i].y - mx) * inv_t),
                           dev::fast_expf((v[i].z - mx) * inv_t), dev::fast_expf((v[i].w - mx) * inv_t));
        sum += v[i].x;
        sum += v[i].y;
        sum += v[i].z;
        sum += v[i].w;
    }
    sum = block_sum_n<1024>(sum, red);
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t j = threadIdx.x + i * 1024;
        if (j < n4) y[j] = make_float4(v[i].x * inv, v[i].y * inv, v[i].z * inv, v[i].w * inv);
    }
}


// One row of a RowChain per workgroup (no __restrict__: a stage's output may
// be the very buffer an input row came from; every thread reads its elements
// of the row before it writes them, and writes the stages in command order).
// The RMSNORM sum runs over the same thread/element mapping and block_sum as
// rmsnorm_reg_kernel, hence the same float sum; the max of the quantize stage
// does not depend on order.
// NT threads per row: 256 whenever the chain has an RMSNORM (its sum order is
// rmsnorm_reg_kernel's); SWIGLU -> QUANTIZE_I8 (a max, any order) uses 1024,
// four times the lanes for the SiLU of a long row.
template <int VPT, uint32_t PRE, bool NORM, bool QUANT, int NT = kThreads>
__global__ __launch_bounds__(NT) void row_chain_kernel(RowChain p)
{
    static_assert(!NORM || NT == kThreads, "RMSNORM sums in rmsnorm_reg_kernel's order");
    __shared__ float red[NT / 64];
    const uint32_t n4 = p.cols >> 2;
    const uint64_t off = static_cast<uint64_t>(blockIdx.x) * n4;
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 v[VPT];
    if (PRE == kChainNone) {
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const uint32_t j = threadIdx.x + i * NT;
            v[i] = j < n4 ? reinterpret_cast<const float4 *>(p.A)[off + j] : zero;
        }
    } else {
        float4 b[VPT];
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const uint32_t j = threadIdx.x + i * NT;
            v[i] = j < n4 ? reinterpret_cast<const float4 *>(p.A)[off + j] : zero;
            b[i] = j < n4 ? reinterpret_cast<const float4 *>(p.B)[off + j] : zero;
        }
        constexpr int OP = PRE == kChainAdd ? EW_ADD : EW_SWIGLU;
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const uint32_t j = threadIdx.x + i * NT;
            if (j >= n4) continue;
            v[i] = make_float4(ew<OP>(v[i].x, b[i].x, p.alpha, p.beta), ew<OP>(v[i].y, b[i].y, p.alpha, p.beta),
                               ew<OP>(v[i].z, b[i].z, p.alpha, p.beta), ew<OP>(v[i].w, b[i].w, p.alpha, p.beta));
            reinterpret_cast<float4 *>(p.Y)[off + j] = v[i];
        }
    }
    if (NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            ss = fmaf(v[i].x, v[i].x, ss);
            ss = fmaf(v[i].y, v[i].y, ss);
            ss = fmaf(v[i].z, v[i].z, ss);
            ss = fmaf(v[i].w, v[i].w, ss);
        }
        ss = block_sum(ss, red);
        const float inv = 1.0f / sqrtf(ss / static_cast<float>(p.cols) + p.eps);
        const float4 *w = reinterpret_cast<const float4 *>(p.W);
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const uint32_t j = threadIdx.x + i * NT;
            if (j >= n4) continue;
            const float4 g = w ? w[j] : make_float4(1.f, 1.f, 1.f, 1.f);
            v[i] = make_float4(v[i].x * inv * g.x, v[i].y * inv * g.y, v[i].z * inv * g.z, v[i].w * inv * g.w);
            reinterpret_cast<float4 *>(p.Nrm)[off + j] = v[i];
        }
    }
    if (QUANT) {
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < VPT; ++i)
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
        const float scale = dev::scale_from_max(block_max_n<NT>(m, red));
        const float inv = __fdiv_rn(1.0f, scale);
        if (threadIdx.x == 0) p.scales[blockIdx.x] = scale;
        char4 *out = reinterpret_cast<char4 *>(p.Q) + off;
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const uint32_t j = threadIdx.x + i * NT;
            if (j < n4)
                out[j] = make_char4(dev::q8(v[i].x, inv), dev::q8(v[i].y, inv), dev::q8(v[i].z, inv),
                                    dev::q8(v[i].w, inv));
        }
    }
}

template <int VPT>
bool launch_row_chain(hipStream_t s, const RowChain &p)
{
    const dim3 grid(p.rows), block(kThreads);
    const bool norm = p.Nrm != nullptr, quant = p.Q != nullptr;
    if (p.pre == kChainAdd && norm && quant)
        row_chain_kernel<VPT, kChainAdd, true, true><<<grid, block, 0, s>>>(p);
    else if (p.pre == kChainAdd && norm)
        row_chain_kernel<VPT, kChainAdd, true, false><<<grid, block, 0, s>>>(p);
    else if (p.pre == kChainNone && norm && quant)
        row_chain_kernel<VPT, kChainNone, true, true><<<grid, block, 0, s>>>(p);
    else
        return false;
    return true;
}

bool launch_swiglu_chain(hipStream_t s, const RowChain &p)
{
    const dim3 grid(p.rows), block(1024);
    if (p.cols / 4 <= 1024)
        row_chain_kernel<1, kChainSwiglu, false, true, 1024><<<grid, block, 0, s>>>(p);
    else
        row_chain_kernel<3, kChainSwiglu, false, true, 1024><<<grid, block, 0, s>>>(p);
    return true;
}

__global__ void fill_kernel(uint8_t *dst, uint8_t v, uint64_t n)
{
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * kThreads)
        dst[i] = v;
}

}  // namespace

void rmsnorm(hipStream_t s, const float *X, const float *W, float *Y, uint32_t rows,
             uint32_t cols, float eps)
{
    const bool vec = (cols % 4 == 0) &&
                     ((reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(Y) |
                       (W ? reinterpret_cast<uintptr_t>(W) : 0)) % 16 == 0);
    const uint32_t n4 = cols / 4;
    if (vec && n4 <= kThreads * 4)
        rmsnorm_reg_kernel<4><<<dim3(rows), kThreads, 0, s>>>(X, W, Y, cols, eps);
    else if (vec && n4 <= kThreads * 12)
        rmsnorm_reg_kernel<12><<<dim3(rows), kThreads, 0, s>>>(X, W, Y, cols, eps);
    else if (vec)
        rmsnorm_vec_kernel<<<dim3(rows), kThreads, 0, s>>>(X, W, Y, cols, eps);
    else
        rmsnorm_kernel<<<dim3(rows), kThreads, 0, s>>>(X, W, Y, cols, eps);
}

// Rows below this count leave most CUs idle with one workgroup per row.
constexpr uint32_t kSplitRows = 512;
constexpr uint32_t kSplitChunk = 1024;  // columns per workgroup (4 per thread)

static uint32_t softmax_chunks(uint32_t rows, uint32_t cols)
{
    if (rows >= kSplitRows || cols < 2 * kSplitChunk) return 1;
    return (cols + kSplitChunk - 1) / kSplitChunk;
}

size_t softmax_ws_bytes(uint32_t rows, uint32_t cols)
{
    const uint32_t chunks = softmax_chunks(rows, cols);
    return chunks > 1 ? static_cast<size_t>(rows) * chunks * 2 * sizeof(float) : 0;
}

void softmax(hipStream_t s, const float *X, float *Y, uint32_t rows, uint32_t cols, float inv_t,
             float *ws)
{
    const uint32_t chunks = softmax_chunks(rows, cols);
    if (chunks == 1) {
        softmax_kernel<<<dim3(rows), kThreads, 0, s>>>(X, Y, cols, inv_t);
        return;
    }
    const bool vec = cols % 4 == 0 && ((reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(Y)) % 16 == 0);
    if (vec && cols / 4 <= 1024 * 8) {
        softmax_reg_kernel<8><<<dim3(rows), 1024, 0, s>>>(X, Y, cols, inv_t);
        return;
    }
    const dim3 grid(chunks, rows);
    softmax_chunk_max<<<grid, kThreads, 0, s>>>(X, cols, kSplitChunk, ws);
    softmax_chunk_sum<<<grid, kThreads, 0, s>>>(X, cols, kSplitChunk, inv_t, ws);
    softmax_chunk_norm<<<grid, kThreads, 0, s>>>(X, Y, cols, kSplitChunk, inv_t, ws);
}

void rope(hipStream_t s, float *Q, float *K, const int32_t *positions, uint32_t batch,
          uint32_t heads, uint32_t q_seq, uint32_t k_seq, uint32_t head_dim,
          uint32_t position_offset, uint32_t interleaved, float scaling, const float *inv_freq)
{
    const uint32_t seq = q_seq > k_seq ? q_seq : k_seq;
    const uint64_t bh = static_cast<uint64_t>(batch) * heads;
    const uint64_t total = bh * seq * (head_dim / 2);
    if (!total) return;
    const bool vec = !interleaved && head_dim % 8 == 0 &&
                     ((reinterpret_cast<uintptr_t>(Q) | reinterpret_cast<uintptr_t>(K)) % 16 == 0);
    if (vec) {
        const uint64_t t4 = total / 4;
        rope_vec_kernel<<<dim3(static_cast<uint32_t>((t4 + kThreads - 1) / kThreads)), kThreads, 0, s>>>(
            Q, K, positions, bh, q_seq, k_seq, seq, head_dim, position_offset, scaling, inv_freq);
        return;
    }
    rope_kernel<<<dim3(static_cast<uint32_t>((total + kThreads - 1) / kThreads)), kThreads, 0, s>>>(
        Q, K, positions, bh, q_seq, k_seq, seq, head_dim, position_offset, interleaved, scaling,
        inv_freq);
}

void swiglu(hipStream_t s, const float *g, const float *u, float *Y, uint64_t n, float alpha)
{
    launch_ew<EW_SWIGLU>(s, g, u, Y, n, alpha, 0.0f);
}

void add(hipStream_t s, const float *A, const float *B, float *Y, uint64_t n, float alpha, float beta)
{
    launch_ew<EW_ADD>(s, A, B, Y, n, alpha, beta);
}

void mul(hipStream_t s, const float *A, const float *B, float *Y, uint64_t n, float alpha, float beta)
{
    launch_ew<EW_MUL>(s, A, B, Y, n, alpha, beta);
}

void gelu(hipStream_t s, const float *X, float *Y, uint64_t n)
{
    launch_ew<EW_GELU>(s, X, nullptr, Y, n, 0.0f, 0.0f);
}

bool row_chain(hipStream_t s, const RowChain &p)
{
    auto al = [](const void *q, uintptr_t a) { return reinterpret_cast<uintptr_t>(q) % a == 0; };
    if (!p.rows || !p.cols || p.cols % 4 || p.cols / 4 > kRowChainMaxVec4 || p.rows > (1u << 22))
        return false;
    if (!p.A || !al(p.A, 16) || (p.pre != kChainNone && (!p.B || !p.Y || !al(p.B, 16) || !al(p.Y, 16))))
        return false;
    if ((p.W && !al(p.W, 16)) || (p.Nrm && !al(p.Nrm, 16)) || (p.Q && (!al(p.Q, 4) || !p.scales)))
        return false;
    if (p.pre == kChainSwiglu) return !p.Nrm && p.Q && launch_swiglu_chain(s, p);
    return p.cols / 4 <= kThreads * 4 ? launch_row_chain<4>(s, p) : launch_row_chain<12>(s, p);
}

void fill_u8(hipStream_t s, void *dst, uint8_t value, uint64_t bytes)
{
    uint64_t blocks = (bytes + kThreads - 1) / kThreads;
    if (blocks > 8192) blocks = 8192;
    if (!blocks) return;
    fill_kernel<<<dim3(static_cast<uint32_t>(blocks)), kThreads, 0, s>>>(static_cast<uint8_t *>(dst), value, bytes);
}

}  // namespace k
}  // namespace vnpu
