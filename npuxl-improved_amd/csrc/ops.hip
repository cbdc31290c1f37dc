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
constexpr int kRawBuf = 0x00020000;   // raw buffer resource word 3: 32-bit data, no swizzle
typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));

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

// RMSNORM in the rounding order of the reference's AVX2 build
// (rmsnorm_avx2_rows, llm.cpp:80-108), so the result is the reference's bit
// for bit:
//   * the sum of squares runs as eight FMA chains, chain c over elements c,
//     c + 8, c + 16, ... in order; the eight sums combine as
//     ((s0 + s4) + (s1 + s5)) + ((s2 + s6) + (s3 + s7)) (hsum256), and the
//     cols % 8 tail elements follow as the reference's build adds them
//     (dev::tail_dot: four rounded products first when four or more remain,
//     then FMAs);
//   * inv = 1 / sqrt(sum / cols + eps), correctly rounded;
//   * y = (x * w) * inv on the 8-wide part, (x * inv) * w on the tail.
// A chain is one sequential dependency (cols / 8 FMAs), so eight lanes walk
// the row staged in LDS while the other lanes wait; rows run in parallel
// across workgroups.  kChainFloats bounds the LDS staging of one pass.
constexpr uint32_t kChainFloats = 12288;

// The row's 8-wide part is staged in LDS chain-major: element e at
// (e % 8) * P + e / 8, so chain c is one contiguous run its lane reads with
// 16-byte loads.  P = chain_pitch(elements per chain) is a multiple of 4,
// and P = 4 (mod 64) puts the eight lanes' reads of one step in distinct
// 16-byte bank slots.
__host__ __device__ constexpr uint32_t chain_pitch(uint32_t len) { return (len + 63) / 64 * 64 + 4; }
// Floats of LDS for a row of `cols`: the chain-major part plus the tail.
__host__ __device__ constexpr uint32_t chain_floats(uint32_t cols)
{
    return 8 * chain_pitch((cols & ~7u) / 8) + 8;
}

// Elements e0 .. e0+3 (e0 a multiple of 4) of the 8-wide part.
__device__ __forceinline__ void chain_put4(float *rowt, uint32_t P, uint32_t e0, float4 v)
{
    const uint32_t c = e0 & 4u, s = e0 >> 3;
    rowt[c * P + s] = v.x;
    rowt[(c + 1) * P + s] = v.y;
    rowt[(c + 2) * P + s] = v.z;
    rowt[(c + 3) * P + s] = v.w;
}

// Eight chain lanes accumulate len elements each (chain c at rowt + c * P)
// into acc in element order.  A chain is one dependent FMA after another, so
// the LDS reads must run ahead of it: the next kChainGroup float4s are
// issued before the current ones are summed, and a scheduling barrier keeps
// the compiler from sinking those reads below the FMAs (it did, and each
// float4 then waited out a whole LDS round trip: about 16 cycles per
// element).  Call with every thread, between barriers.
constexpr uint32_t kChainGroup = 4;
__device__ __forceinline__ void chain_sumsq(const float *rowt, uint32_t P, uint32_t len, float &acc)
{
    const uint32_t c = threadIdx.x;
    if (c >= 8) return;
    const float *r = rowt + c * P;
    const float4 *r4 = reinterpret_cast<const float4 *>(r);
    const uint32_t n4 = len / 4, groups = n4 / kChainGroup;
    auto sum4 = [&](const float4 &v) {
        acc = fmaf(v.x, v.x, acc);
        acc = fmaf(v.y, v.y, acc);
        acc = fmaf(v.z, v.z, acc);
        acc = fmaf(v.w, v.w, acc);
    };
    auto load = [&](float4 (&x)[kChainGroup], uint32_t g) {
#pragma unroll
        for (uint32_t u = 0; u < kChainGroup; ++u) x[u] = r4[g * kChainGroup + u];
        __builtin_amdgcn_sched_barrier(0);
    };
    auto sum = [&](const float4 (&x)[kChainGroup]) {
#pragma unroll
        for (uint32_t u = 0; u < kChainGroup; ++u) sum4(x[u]);
        __builtin_amdgcn_sched_barrier(0);
    };
    if (groups) {
        float4 x0[kChainGroup], x1[kChainGroup];   // ping-pong: group g + 1 loads while g is summed
        load(x0, 0);
        uint32_t g = 1;
        for (; g + 1 < groups; g += 2) {
            load(x1, g);
            sum(x0);
            load(x0, g + 1);
            sum(x1);
        }
        if (g < groups) {
            load(x1, g);
            sum(x0);
            sum(x1);
        } else {
            sum(x0);
        }
    }
    for (uint32_t i = groups * kChainGroup; i < n4; ++i) sum4(r4[i]);
    for (uint32_t i = 4 * n4; i < len; ++i) acc = fmaf(r[i], r[i], acc);
}

// Combines the chain sums (red8, written by lanes 0..7) and the tail
// row_tail[0 .. tail) the way hsum256 and the scalar tail do; every thread
// gets the result.  Call after a barrier that follows the chains' writes.
__device__ __forceinline__ float chain_total(const float *red8, const float *row_tail, uint32_t tail)
{
    const float sum = ((red8[0] + red8[4]) + (red8[1] + red8[5])) + ((red8[2] + red8[6]) + (red8[3] + red8[7]));
    return dev::tail_dot(row_tail, row_tail, tail, sum);
}

__device__ __forceinline__ float rms_inv(float sum, uint32_t cols, float eps)
{
    return 1.0f / sqrtf(sum / static_cast<float>(cols) + eps);
}

// Element e of a row of `cols`: (x*w)*inv inside the 8-wide part, else
// (x*inv)*w.
__device__ __forceinline__ float rms_scale(float x, float w, float inv, uint32_t e, uint32_t cols8)
{
    return e < cols8 ? dev::mul_rn(dev::mul_rn(x, w), inv) : dev::mul_rn(dev::mul_rn(x, inv), w);
}

// Any row length and alignment: the row streams through LDS in passes of
// kChainFloats for the sum, then is read again for the scaling.
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const float *__restrict__ X,
                                                           const float *__restrict__ W,
                                                           float *__restrict__ Y, uint32_t cols,
                                                           float eps)
{
    extern __shared__ float row_lds[];   // chain_floats(min(cols, kChainFloats)) floats
    __shared__ float red8[8];
    const uint64_t r = blockIdx.x;
    const float *x = X + r * cols;
    float *y = Y + r * cols;
    const uint32_t cols8 = cols & ~7u;
    float acc = 0.0f;
    for (uint32_t c0 = 0; c0 < cols8; c0 += kChainFloats) {
        const uint32_t n = min(kChainFloats, cols8 - c0), P = chain_pitch(n / 8);
        __syncthreads();
        for (uint32_t j = threadIdx.x; j < n; j += kThreads) row_lds[(j & 7u) * P + (j >> 3)] = x[c0 + j];
        __syncthreads();
        chain_sumsq(row_lds, P, n / 8, acc);
    }
    __syncthreads();
    if (threadIdx.x < 8) red8[threadIdx.x] = acc;
    __syncthreads();
    const float inv = rms_inv(chain_total(red8, x + cols8, cols - cols8), cols, eps);
    for (uint32_t j = threadIdx.x; j < cols; j += kThreads) y[j] = rms_scale(x[j], W ? W[j] : 1.0f, inv, j, cols8);
}

// Rows of up to VPT*1024 floats, 16-byte aligned: the row stays in registers
// between the sum of squares and the scaling (one HBM read instead of two)
// and is staged once in LDS for the chain lanes.
template <int VPT>
__global__ __launch_bounds__(kThreads) void rmsnorm_reg_kernel(const float *__restrict__ X,
                                                               const float *__restrict__ W,
                                                               float *__restrict__ Y, uint32_t cols,
                                                               float eps)
{
    extern __shared__ float4 row4[];   // chain_floats(cols) floats
    __shared__ float red8[8];
    const uint64_t r = blockIdx.x;
    const float4 *x = reinterpret_cast<const float4 *>(X + r * cols);
    float4 *y = reinterpret_cast<float4 *>(Y + r * cols);
    const float4 *w = reinterpret_cast<const float4 *>(W);
    const uint32_t n4 = cols >> 2, cols8 = cols & ~7u, P = chain_pitch(cols8 / 8);
    float *rowt = reinterpret_cast<float *>(row4), *tail = rowt + 8 * P;
    float4 v[VPT], g[VPT];   // the weights load while the sum runs
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t j = threadIdx.x + i * kThreads;
        g[i] = (W && j < n4) ? w[j] : make_float4(1.f, 1.f, 1.f, 1.f);
        v[i] = j < n4 ? x[j] : make_float4(0.f, 0.f, 0.f, 0.f);
        if (j < n4) {
            if (4 * j < cols8) chain_put4(rowt, P, 4 * j, v[i]);
            else *reinterpret_cast<float4 *>(tail) = v[i];   // the one float4 past cols8
        }
    }
    __syncthreads();
    float acc = 0.0f;
    chain_sumsq(rowt, P, cols8 / 8, acc);
    if (threadIdx.x < 8) red8[threadIdx.x] = acc;
    __syncthreads();
    const float inv = rms_inv(chain_total(red8, tail, cols - cols8), cols, eps);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t j = threadIdx.x + i * kThreads;
        if (j >= n4) continue;
        const uint32_t e = 4 * j;
        y[j] = make_float4(rms_scale(v[i].x, g[i].x, inv, e, cols8), rms_scale(v[i].y, g[i].y, inv, e + 1, cols8),
                           rms_scale(v[i].z, g[i].z, inv, e + 2, cols8), rms_scale(v[i].w, g[i].w, inv, e + 3, cols8));
    }
}

// The weight of element j as the reference's AVX2 build computes it
// (softmax_avx2_rows, llm.cpp:137-180): exp256 (clamped to [-80, 80]) of
// the separately rounded (x - max) * inv_t over the 8-wide steps, j below
// cols & ~7; the scalar fast_expf (Horner steps contracted, 0 below -80) in
// the tail.  Each weight is the reference's bit for bit; the sums below add
// them in tree order, not in the reference's eight lanes.
__device__ __forceinline__ float softmax_exp(float x, float mx, float inv_t, uint32_t j, uint32_t cols8)
{
#pragma clang fp contract(off)
    const float t = (x - mx) * inv_t;
    return j < cols8 ? dev::exp_avx2(t) : dev::fast_expf(t);
}

// reference llm.cpp:137-180
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
    const uint32_t cols8 = cols & ~7u;
    float sum = 0.0f;
    for (uint32_t j = threadIdx.x; j < cols; j += kThreads) sum += softmax_exp(x[j], mx, inv_t, j, cols8);
    sum = block_sum(sum, red);
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (uint32_t j = threadIdx.x; j < cols; j += kThreads) y[j] = softmax_exp(x[j], mx, inv_t, j, cols8) * inv;
}

// Few long rows (e.g. the MTP head's [4, 32000] logits): each row is split
// into chunks over many workgroups, in three passes that keep the
// reference's terms exactly: chunk maxima -> the row max M; chunk sums of
// the weights (softmax_exp) -> the row sum L; y = weight * (1 / L).  ws
// holds rows x chunks x 2 floats.
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
    const uint32_t cols8 = cols & ~7u;
    float sum = 0.0f;
    for (uint32_t j = c0 + threadIdx.x; j < c1; j += kThreads) sum += softmax_exp(x[j], mx, inv_t, j, cols8);
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
    const uint32_t cols8 = cols & ~7u;
    for (uint32_t j = c0 + threadIdx.x; j < c1; j += kThreads) y[j] = softmax_exp(x[j], mx, inv_t, j, cols8) * inv;
}

// reference llm.cpp:188-217, 576-602: one thread per rotated pair.
// cos and sin of pair j at position p: from the host table (the reference's
// libm cosf/sinf of (p * scaling) * inv[j], llm.cpp:195-211) where it covers
// p, else computed here (positions the table does not cover: a device-side
// position array beyond the positions seen so far, or a negative position).
__device__ __forceinline__ void rope_cos_sin(int32_t p, uint32_t j, uint32_t half, float scaling,
                                             const float *inv_freq, const float2 *cs, uint32_t cs_rows,
                                             float &c, float &s)
{
    if (cs && p >= 0 && static_cast<uint32_t>(p) < cs_rows) {
        const float2 v = cs[static_cast<uint64_t>(p) * half + j];
        c = v.x;
        s = v.y;
        return;
    }
    const float angle = dev::mul_rn(dev::mul_rn(static_cast<float>(p), scaling), inv_freq[j]);
    c = cosf(angle);
    s = sinf(angle);
}

// rotate_vector's pair update (llm.cpp:202-213): products and the
// difference / sum round separately.
__device__ __forceinline__ void rotate_pair(float *x, uint32_t i0, uint32_t i1, float c, float s)
{
#pragma clang fp contract(off)
    const float x0 = x[i0], x1 = x[i1];
    x[i0] = x0 * c - x1 * s;
    x[i1] = x0 * s + x1 * c;
}

__global__ __launch_bounds__(kThreads) void rope_kernel(float *__restrict__ Q, float *__restrict__ K,
                                                        const int32_t *__restrict__ positions,
                                                        uint64_t bh_count, uint32_t q_seq,
                                                        uint32_t k_seq, uint32_t seq,
                                                        uint32_t head_dim, uint32_t offset,
                                                        uint32_t interleaved, float scaling,
                                                        const float *__restrict__ inv_freq,
                                                        const float2 *__restrict__ cs, uint32_t cs_rows)
{
    const uint32_t half = head_dim / 2;
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const uint64_t total = bh_count * seq * half;
    if (idx >= total) return;
    const uint32_t j = static_cast<uint32_t>(idx % half);
    const uint64_t tok = idx / half;
    const uint32_t t = static_cast<uint32_t>(tok % seq);
    const uint64_t bh = tok / seq;
    const int32_t p = positions ? positions[t] : static_cast<int32_t>(t + offset);
    float c, s;
    rope_cos_sin(p, j, half, scaling, inv_freq, cs, cs_rows, c, s);
    const uint32_t i0 = interleaved ? 2 * j : j;
    const uint32_t i1 = interleaved ? 2 * j + 1 : j + half;
    if (Q && t < q_seq) rotate_pair(Q + (bh * q_seq + t) * head_dim, i0, i1, c, s);
    if (K && t < k_seq) rotate_pair(K + (bh * k_seq + t) * head_dim, i0, i1, c, s);
}

// cos and sin of pairs 4 j4 .. 4 j4 + 3 at position p: two 16-byte table
// reads where the table covers p (half is a multiple of 4 on the vector
// path, so they are aligned), rope_cos_sin per pair otherwise.
__device__ __forceinline__ void rope_cos_sin4(int32_t p, uint32_t j4, uint32_t half, float scaling,
                                              const float *inv_freq, const float2 *cs, uint32_t cs_rows,
                                              float (&c)[4], float (&s)[4])
{
    if (cs && p >= 0 && static_cast<uint32_t>(p) < cs_rows) {
        const float4 *t = reinterpret_cast<const float4 *>(cs + static_cast<uint64_t>(p) * half + 4 * j4);
        const float4 a = t[0], b = t[1];
        c[0] = a.x; s[0] = a.y; c[1] = a.z; s[1] = a.w;
        c[2] = b.x; s[2] = b.y; c[3] = b.z; s[3] = b.w;
        return;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) rope_cos_sin(p, 4 * j4 + e, half, scaling, inv_freq, cs, cs_rows, c[e], s[e]);
}

// Half-rotation layout with head_dim % 8 == 0 and 16-byte aligned rows: one
// thread rotates pairs j..j+3 with one float4 from each half of the row.
__device__ __forceinline__ void rotate4(const float4 a, const float4 b, const float (&c)[4], const float (&s)[4],
                                        float4 &lo, float4 &hi)
{
#pragma clang fp contract(off)
    lo = make_float4(a.x * c[0] - b.x * s[0], a.y * c[1] - b.y * s[1], a.z * c[2] - b.z * s[2],
                     a.w * c[3] - b.w * s[3]);
    hi = make_float4(a.x * s[0] + b.x * c[0], a.y * s[1] + b.y * c[1], a.z * s[2] + b.z * c[2],
                     a.w * s[3] + b.w * c[3]);
}

// Grid: x = chunks of kThreads (token, pair group) items of one (batch, head),
// y = (batch, head) pairs (those past gridDim.y take further trips), so the
// index math is 32-bit (seq * head_dim / 8 < 2^32 is required).
__global__ __launch_bounds__(kThreads) void rope_vec_kernel(float *__restrict__ Q, float *__restrict__ K,
                                                            const int32_t *__restrict__ positions,
                                                            uint64_t bh_count, uint32_t q_seq,
                                                            uint32_t k_seq, uint32_t seq,
                                                            uint32_t head_dim, uint32_t offset,
                                                            float scaling,
                                                            const float *__restrict__ inv_freq,
                                                            const float2 *__restrict__ cs, uint32_t cs_rows)
{
    const uint32_t half4 = head_dim / 8;
    const uint32_t idx = blockIdx.x * kThreads + threadIdx.x;
    if (idx >= seq * half4) return;
    const uint32_t t = idx / half4, j4 = idx - t * half4;
    const int32_t p = positions ? positions[t] : static_cast<int32_t>(t + offset);
    float c[4], s[4];
    rope_cos_sin4(p, j4, head_dim / 2, scaling, inv_freq, cs, cs_rows, c, s);
    for (uint64_t bh = blockIdx.y; bh < bh_count; bh += gridDim.y) {
        // Q's and K's pairs load before anything is stored, through raw buffers
        // over the row (an empty range when the row is absent: zero in, writes
        // dropped), so no branch sits between the loads and the stores and the
        // K loads do not wait behind the Q stores.
        const bool has_q = Q && t < q_seq, has_k = K && t < k_seq;
        const uint32_t row_bytes = head_dim * 4u;
        float *qrow = has_q ? Q + (bh * q_seq + t) * head_dim : Q, *krow = has_k ? K + (bh * k_seq + t) * head_dim : K;
        const auto rq = __builtin_amdgcn_make_buffer_rsrc(qrow, 0, static_cast<int>(has_q ? row_bytes : 0u), kRawBuf);
        const auto rk = __builtin_amdgcn_make_buffer_rsrc(krow, 0, static_cast<int>(has_k ? row_bytes : 0u), kRawBuf);
        const uint32_t o0 = j4 * 16u, o1 = (half4 + j4) * 16u;
        auto ld = [](__amdgpu_buffer_rsrc_t r, uint32_t o) {
            return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, o, 0, 0));
        };
        const float4 qa = ld(rq, o0), qb = ld(rq, o1), ka = ld(rk, o0), kb = ld(rk, o1);
        auto st = [](__amdgpu_buffer_rsrc_t r, uint32_t o, float4 x) {
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u32, x), r, o, 0, 0);
        };
        float4 lo, hi;
        rotate4(qa, qb, c, s, lo, hi);
        st(rq, o0, lo);
        st(rq, o1, hi);
        // Q and K the same row: K is rotated again, from Q's result, as in
        // command order
        const bool same = has_q && qrow == krow;
        const float4 ka2 = same ? lo : ka, kb2 = same ? hi : kb;
        rotate4(ka2, kb2, c, s, lo, hi);
        st(rk, o0, lo);
        st(rk, o1, hi);
    }
}

enum EwOp { EW_SWIGLU = 0, EW_ADD = 1, EW_MUL = 2, EW_GELU = 3 };

// The reference's AVX2 builds (llm.cpp:256-330), rounding for rounding.  They
// run 8-wide steps from the start of a range and the last count % 8 elements
// in a scalar tail loop whose expressions contract differently (MUL:
// fma(alpha*a, b, beta)) or use the scalar exp without the clamp (SWIGLU);
// `tail` marks those elements (the elements from count - count % 8 on, the
// reference's single range per command whenever its chunk size is a multiple
// of 8).  ADD's tail contracts to the same fma and GELU's gives the same
// values.
template <int OP>
__device__ __forceinline__ float ew(float a, float b, float alpha, float beta, bool tail)
{
    if (OP == EW_SWIGLU) return tail ? dev::swiglu_tail(a, b, alpha) : dev::swiglu_avx2(a, b, alpha);
    if (OP == EW_ADD) return fmaf(a, alpha, dev::mul_rn(b, beta));
    if (OP == EW_MUL) return tail ? fmaf(dev::mul_rn(alpha, a), b, beta) : fmaf(dev::mul_rn(a, b), alpha, beta);
    return dev::gelu_avx2(a);
}

// Which elements of an elementwise command fall in a scalar tail.  The
// reference runs a command over n elements as ranges [c*grain, (c+1)*grain)
// (scheduler.cpp:536-581: grain = max(4096, n / (4 * num_threads));
// ThreadPool::parallel_for, internal.h:273-340), each as 8-wide steps from
// its own start and a scalar tail of (length % 8) elements.  When only the
// last range can have a tail (grain % 8 == 0, or one range) the tail is the
// last n % 8 elements: grain is then 0 and t0 = n - n % 8.
struct EwTail {
    uint64_t n = 0, grain = 0, t0 = 0;
    __device__ __forceinline__ bool operator()(uint64_t x) const
    {
        if (grain == 0) return x >= t0;
        const uint64_t b = x / grain * grain;
        const uint64_t len = n - b < grain ? n - b : grain;
        return x - b >= (len & ~7ull);
    }
    // bit k: element e + k (all four < n); one division per call
    __device__ __forceinline__ uint32_t mask4(uint64_t e) const
    {
        uint32_t m = 0;
        if (grain == 0) {
#pragma unroll
            for (int k = 0; k < 4; ++k) m |= uint32_t(e + k >= t0) << k;
            return m;
        }
        uint64_t b = e / grain * grain;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (e + k >= b + grain) b += grain;   // grain >= 4096: one step at most
            const uint64_t len = n - b < grain ? n - b : grain;
            m |= uint32_t(e + k - b >= (len & ~7ull)) << k;
        }
        return m;
    }
};

__host__ __device__ inline EwTail ew_tail(uint64_t n, uint64_t grain)
{
    EwTail t;
    t.n = n;
    if (grain == 0 || grain >= n || grain % 8 == 0) t.t0 = n - n % 8;
    else t.grain = grain;
    return t;
}

template <int OP>
__global__ __launch_bounds__(kThreads) void ew_vec_kernel(const float4 *__restrict__ A,
                                                          const float4 *__restrict__ B,
                                                          float4 *__restrict__ Y, uint64_t n4,
                                                          float alpha, float beta, EwTail tl)
{
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n4;
         i += static_cast<uint64_t>(gridDim.x) * kThreads) {
        const float4 a = A[i];
        const float4 b = (OP == EW_GELU) ? a : B[i];
        const uint32_t t = tl.mask4(4 * i);
        Y[i] = make_float4(ew<OP>(a.x, b.x, alpha, beta, t & 1), ew<OP>(a.y, b.y, alpha, beta, t & 2),
                           ew<OP>(a.z, b.z, alpha, beta, t & 4), ew<OP>(a.w, b.w, alpha, beta, t & 8));
    }
}

template <int OP>
__global__ __launch_bounds__(kThreads) void ew_kernel(const float *__restrict__ A,
                                                      const float *__restrict__ B,
                                                      float *__restrict__ Y, uint64_t n,
                                                      float alpha, float beta, EwTail tl)
{
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * kThreads)
        Y[i] = ew<OP>(A[i], (OP == EW_GELU) ? 0.0f : B[i], alpha, beta, tl(i));
}

template <int OP>
void launch_ew(hipStream_t s, const float *A, const float *B, float *Y, uint64_t n, float alpha,
               float beta, uint64_t grain)
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
            reinterpret_cast<float4 *>(Y), n / 4, alpha, beta, ew_tail(n, grain));
    else
        ew_kernel<OP><<<dim3(static_cast<uint32_t>(blocks)), kThreads, 0, s>>>(A, B, Y, n, alpha, beta,
                                                                              ew_tail(n, grain));
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
// the max, then each weight once (softmax_exp, kept for the output) and
// their sum; y = e * (1 / sum), the reference's terms with a tree sum.
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
    const uint32_t cols8 = cols & ~7u;
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const uint32_t j = threadIdx.x + i * 1024;
        if (j >= n4) continue;
        // four consecutive elements lie on one side of cols & ~7
        v[i] = make_float4(softmax_exp(v[i].x, mx, inv_t, 4 * j, cols8), softmax_exp(v[i].y, mx, inv_t, 4 * j, cols8),
                           softmax_exp(v[i].z, mx, inv_t, 4 * j, cols8), softmax_exp(v[i].w, mx, inv_t, 4 * j, cols8));
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
    static_assert(!NORM || NT == kThreads, "RMSNORM as rmsnorm_reg_kernel computes it");
    __shared__ float red[NT / 64];
    const uint32_t n4 = p.cols >> 2, row_bytes = p.cols * 4u;
    const uint64_t off = static_cast<uint64_t>(blockIdx.x) * n4;
    float4 v[VPT];
    // Every global access goes through a raw buffer over this row, so float4
    // slots past the row need no branch (reads return zero, writes are
    // dropped).  With a branch around each load the compiler could not tell
    // which loads were still in flight and waited for all memory operations,
    // stores included, before later uses of those registers: a memory round
    // trip on the row's critical path after each store.
    const uint32_t lane_off = threadIdx.x * 16u;
    auto rsrc = [&](const void *base, uint32_t bytes) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, static_cast<int>(bytes), kRawBuf);
    };
    auto ld4 = [&](__amdgpu_buffer_rsrc_t r, int i) {
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, lane_off + i * NT * 16u, 0, 0));
    };
    auto st4 = [&](__amdgpu_buffer_rsrc_t r, int i, float4 x) {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u32, x), r, lane_off + i * NT * 16u, 0, 0);
    };
    // The RMSNORM weights are read up front: loaded after the sum, each load
    // would wait behind the previous element's Nrm store (the buffers may
    // alias, so the compiler keeps them in order).
    float4 g[NORM ? VPT : 1];
    if (NORM) {
        const bool has_w = p.W != nullptr;
        const auto rw = rsrc(p.W, has_w ? row_bytes : 0u);
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const float4 x = ld4(rw, i);
            g[i] = has_w ? x : make_float4(1.f, 1.f, 1.f, 1.f);
        }
    }
    const auto ra = rsrc(p.A + off * 4, row_bytes);
#pragma unroll
    for (int i = 0; i < VPT; ++i) v[i] = ld4(ra, i);
    if (PRE != kChainNone) {
        float4 b[VPT];
        const auto rb = rsrc(p.B + off * 4, row_bytes);
#pragma unroll
        for (int i = 0; i < VPT; ++i) b[i] = ld4(rb, i);
        constexpr int OP = PRE == kChainAdd ? EW_ADD : EW_SWIGLU;
        // the elementwise command spans all rows: its ranges and tails are
        // those of rows * cols elements
        const EwTail tl = ew_tail(static_cast<uint64_t>(p.rows) * p.cols, p.grain);
        const auto ry = rsrc(p.Y + off * 4, row_bytes);
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const uint32_t j = threadIdx.x + i * NT;
            const uint32_t t = OP == EW_ADD ? 0u : tl.mask4(4 * (off + j));   // ADD: tail = body
            v[i] = make_float4(ew<OP>(v[i].x, b[i].x, p.alpha, p.beta, t & 1),
                               ew<OP>(v[i].y, b[i].y, p.alpha, p.beta, t & 2),
                               ew<OP>(v[i].z, b[i].z, p.alpha, p.beta, t & 4),
                               ew<OP>(v[i].w, b[i].w, p.alpha, p.beta, t & 8));
            // slots past the row: zero in, so the max below is unchanged
            if (j >= n4) v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            st4(ry, i, v[i]);
        }
    }
    auto local_absmax = [](const float4 (&x)[VPT]) {
        float r = 0.0f;
#pragma unroll
        for (int i = 0; i < VPT; ++i)
            r = fmaxf(r, fmaxf(fmaxf(fabsf(x[i].x), fabsf(x[i].y)), fmaxf(fabsf(x[i].z), fabsf(x[i].w))));
        return r;
    };
    float m = 0.0f;   // this thread's max |v| for the quantize stage
    if (NORM) {
        // rmsnorm_reg_kernel's arithmetic (the reference's AVX2 order)
        extern __shared__ float4 row4[];   // chain_floats(cols) floats
        __shared__ float red8[8];
        const uint32_t cols8 = p.cols & ~7u, P = chain_pitch(cols8 / 8);
        float *rowt = reinterpret_cast<float *>(row4), *tail = rowt + 8 * P;
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const uint32_t j = threadIdx.x + i * NT;
            if (j >= n4) continue;
            if (4 * j < cols8) chain_put4(rowt, P, 4 * j, v[i]);
            else *reinterpret_cast<float4 *>(tail) = v[i];
        }
        __syncthreads();
        float acc = 0.0f;
        chain_sumsq(rowt, P, cols8 / 8, acc);
        if (threadIdx.x < 8) red8[threadIdx.x] = acc;
        __syncthreads();
        const float inv = rms_inv(chain_total(red8, tail, p.cols - cols8), p.cols, p.eps);
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const uint32_t j = threadIdx.x + i * NT;
            if (j >= n4) continue;
            const uint32_t e = 4 * j;
            v[i] = make_float4(rms_scale(v[i].x, g[i].x, inv, e, cols8), rms_scale(v[i].y, g[i].y, inv, e + 1, cols8),
                               rms_scale(v[i].z, g[i].z, inv, e + 2, cols8),
                               rms_scale(v[i].w, g[i].w, inv, e + 3, cols8));
        }
        // The quantize stage's max is taken before the Nrm stores: the
        // compiler waits for every outstanding memory operation (stores
        // included) before the first use of these registers after them.
        if (QUANT) m = local_absmax(v);
        const auto rn = rsrc(p.Nrm + off * 4, row_bytes);
#pragma unroll
        for (int i = 0; i < VPT; ++i) st4(rn, i, v[i]);
    }
    if (QUANT) {
        if (!NORM) m = local_absmax(v);
        const float scale = dev::scale_from_max(block_max_n<NT>(m, red));
        const float inv = __fdiv_rn(1.0f, scale);
        if (threadIdx.x == 0) p.scales[blockIdx.x] = scale;
        const auto rq = rsrc(p.Q + off * 4, p.cols);
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const char4 q = make_char4(dev::q8(v[i].x, inv), dev::q8(v[i].y, inv), dev::q8(v[i].z, inv),
                                       dev::q8(v[i].w, inv));
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, q), rq,
                                                  threadIdx.x * 4u + i * NT * 4u, 0, 0);
        }
    }
}

template <int VPT>
bool launch_row_chain(hipStream_t s, const RowChain &p)
{
    const dim3 grid(p.rows), block(kThreads);
    const bool norm = p.Nrm != nullptr, quant = p.Q != nullptr;
    const size_t lds = norm ? static_cast<size_t>(chain_floats(p.cols)) * sizeof(float) : 0;
    if (p.pre == kChainAdd && norm && quant)
        row_chain_kernel<VPT, kChainAdd, true, true><<<grid, block, lds, s>>>(p);
    else if (p.pre == kChainAdd && norm)
        row_chain_kernel<VPT, kChainAdd, true, false><<<grid, block, lds, s>>>(p);
    else if (p.pre == kChainNone && norm && quant)
        row_chain_kernel<VPT, kChainNone, true, true><<<grid, block, lds, s>>>(p);
    else
        return false;
    return true;
}

bool launch_swiglu_chain(hipStream_t s, const RowChain &p)
{
    const dim3 grid(p.rows);
    // many rows: 256 threads, as few float4 slots per thread as the row needs
    // (unused slots still hold registers and cut the waves per SIMD)
    if (p.rows >= 256 && p.cols / 4 <= 4 * 256)
        row_chain_kernel<4, kChainSwiglu, false, true, 256><<<grid, dim3(256), 0, s>>>(p);
    else if (p.rows >= 256 && p.cols / 4 <= 8 * 256)
        row_chain_kernel<8, kChainSwiglu, false, true, 256><<<grid, dim3(256), 0, s>>>(p);
    else if (p.rows >= 256)
        row_chain_kernel<12, kChainSwiglu, false, true, 256><<<grid, dim3(256), 0, s>>>(p);
    else if (p.cols / 4 <= 1024)
        row_chain_kernel<1, kChainSwiglu, false, true, 1024><<<grid, dim3(1024), 0, s>>>(p);
    else
        row_chain_kernel<3, kChainSwiglu, false, true, 1024><<<grid, dim3(1024), 0, s>>>(p);
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
    const size_t row_bytes = static_cast<size_t>(chain_floats(cols)) * sizeof(float);
    if (vec && n4 <= kThreads * 4)
        rmsnorm_reg_kernel<4><<<dim3(rows), kThreads, row_bytes, s>>>(X, W, Y, cols, eps);
    else if (vec && n4 <= kThreads * 12)
        rmsnorm_reg_kernel<12><<<dim3(rows), kThreads, row_bytes, s>>>(X, W, Y, cols, eps);
    else
        rmsnorm_kernel<<<dim3(rows), kThreads, chain_floats(std::min(cols, kChainFloats)) * sizeof(float), s>>>(
            X, W, Y, cols, eps);
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
          uint32_t position_offset, uint32_t interleaved, float scaling, const float *inv_freq,
          const float2 *cs, uint32_t cs_rows)
{
    const uint32_t seq = q_seq > k_seq ? q_seq : k_seq;
    const uint64_t bh = static_cast<uint64_t>(batch) * heads;
    const uint64_t total = bh * seq * (head_dim / 2);
    if (!total) return;
    const bool vec = !interleaved && head_dim % 8 == 0 &&
                     ((reinterpret_cast<uintptr_t>(Q) | reinterpret_cast<uintptr_t>(K)) % 16 == 0);
    const uint64_t per_bh4 = static_cast<uint64_t>(seq) * (head_dim / 8);
    if (vec && per_bh4 + kThreads < (1ull << 32)) {
        const dim3 grid(static_cast<uint32_t>((per_bh4 + kThreads - 1) / kThreads),
                        static_cast<uint32_t>(bh < 65535 ? bh : 65535));
        rope_vec_kernel<<<grid, kThreads, 0, s>>>(Q, K, positions, bh, q_seq, k_seq, seq, head_dim, position_offset,
                                                  scaling, inv_freq, cs, cs_rows);
        return;
    }
    rope_kernel<<<dim3(static_cast<uint32_t>((total + kThreads - 1) / kThreads)), kThreads, 0, s>>>(
        Q, K, positions, bh, q_seq, k_seq, seq, head_dim, position_offset, interleaved, scaling,
        inv_freq, cs, cs_rows);
}

void swiglu(hipStream_t s, const float *g, const float *u, float *Y, uint64_t n, float alpha,
            uint64_t grain)
{
    launch_ew<EW_SWIGLU>(s, g, u, Y, n, alpha, 0.0f, grain);
}

void add(hipStream_t s, const float *A, const float *B, float *Y, uint64_t n, float alpha, float beta)
{
    launch_ew<EW_ADD>(s, A, B, Y, n, alpha, beta, 0);   // tail = body (fma(a, alpha, b * beta))
}

void mul(hipStream_t s, const float *A, const float *B, float *Y, uint64_t n, float alpha, float beta,
         uint64_t grain)
{
    launch_ew<EW_MUL>(s, A, B, Y, n, alpha, beta, grain);
}

void gelu(hipStream_t s, const float *X, float *Y, uint64_t n)
{
    launch_ew<EW_GELU>(s, X, nullptr, Y, n, 0.0f, 0.0f, 0);   // tail = body
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
