// attention.hip - ATTENTION_F32 (streaming online softmax) on gfx950.
//
// Semantics of the reference's attention_range (src/kernels/llm.cpp:442-546):
//   s = (q . k) * scale (+ mask[b,h,qi,ki]); causal masks ki > qi + (sk - sq);
//   online softmax over 64-key blocks, a block whose max is not finite is
//   skipped; O = sum(p v) / l, and a row with l == 0 is written as 0.
//   scale <= 0 means 1/sqrt(D) (resolved by the caller).
//
// Structure: one workgroup = 4 waves x 4 queries (16 query rows) of one
// (batch, head); the key range may be split across workgroups (flash-decoding
// style) when there are too few (b, h, q-block) tiles to fill the GPU, with a
// second pass that merges the partial (m, l, acc) triples.  Per 64-key block
// the workgroup stages K transposed ([d][key], conflict-free per-lane key
// reads) and V ([key][d]) in LDS; lane j scores key j for the wave's 4
// queries, the wave's max/sum use cross-lane reductions, and the P.V update
// runs with lanes over the head dimension.  Keys past a query block's causal
// limit are never loaded.
#include "kernels.hpp"

#include <atomic>
#include "device_math.hpp"
#include "lds_dma.hpp"
#include "vnpu_internal.hpp"

#include <algorithm>
#include <mutex>

// Device scratch of vnpu_attention_f32_noalloc (partial (m, l, acc) triples of
// split decode, the split K / V^T blocks of prefill): 64 MiB, the prefill
// need of B1 x 32 heads x 2048 keys at head_dim 128.  Each GPU holds its own
// copy for the life of the process; host code uses only the address
// hipGetSymbolAddress returns for the current device, never this name.
static __device__ __align__(256) float scratch[vnpu::k::kAttnScratchBytes / sizeof(float)];

namespace vnpu {
namespace k {
namespace {

constexpr int kThreads = 256;
constexpr int QW = 4;            // queries per wave
constexpr int BQ = 4 * QW;       // queries per workgroup
constexpr int BKEY = 64;         // keys per block

__global__ __launch_bounds__(kThreads) void attn_kernel(Attn a, uint32_t keys_per_split,
                                                        uint32_t splits, float *ws_acc,
                                                        float *ws_ml)
{
    extern __shared__ float smem[];
    const uint32_t D = a.head_dim;
    float *Kt = smem;               // [D][64]
    float *Vs = Kt + D * BKEY;      // [64][D]
    float *Qs = Vs + BKEY * D;      // [16][D]
    float *Ps = Qs + BQ * D;        // [4][QW][64]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t bh = blockIdx.y;
    const uint32_t q0 = blockIdx.x * BQ;
    const uint32_t split = blockIdx.z;
    const uint32_t sq = a.seq_q, sk = a.seq_k;
    const uint32_t off = sk > sq ? sk - sq : 0;
    const float *Qh = a.Q + bh * sq * D;
    const float *Kh = a.K + bh * sk * D;
    const float *Vh = a.V + bh * sk * D;
    const float *Mh = a.mask ? a.mask + bh * sq * sk : nullptr;

    for (uint32_t i = tid; i < BQ * D; i += kThreads) {
        const uint32_t qi = q0 + i / D;
        Qs[i] = qi < sq ? Qh[static_cast<uint64_t>(qi) * D + (i % D)] : 0.0f;
    }

    uint32_t kbeg = split * keys_per_split;
    uint32_t kend = min(sk, kbeg + keys_per_split);
    if (a.causal) {
        const uint32_t qlast = min(q0 + BQ, sq) - 1;
        kend = min(kend, qlast + off + 1);
    }

    const uint32_t DL = (D + 63) / 64;  // head-dim values per lane (<= 4)
    float m[QW], l[QW], acc[QW][4];
#pragma unroll
    for (int i = 0; i < QW; ++i) {
        m[i] = -__builtin_inff();
        l[i] = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[i][t] = 0.0f;
    }

    for (uint32_t k0 = kbeg; k0 < kend; k0 += BKEY) {
        __syncthreads();
        for (uint32_t i = tid; i < BKEY * D; i += kThreads) {
            const uint32_t j = i / D, d = i % D;
            const uint32_t key = k0 + j;
            float kv = 0.0f, vv = 0.0f;
            if (key < kend) {
                kv = Kh[static_cast<uint64_t>(key) * D + d];
                vv = Vh[static_cast<uint64_t>(key) * D + d];
            }
            Kt[d * BKEY + j] = kv;
            Vs[j * D + d] = vv;
        }
        __syncthreads();

        const uint32_t key = k0 + lane;
        float s[QW];
#pragma unroll
        for (int i = 0; i < QW; ++i) s[i] = 0.0f;
        const float *qw = Qs + wave * QW * D;
        for (uint32_t d = 0; d < D; ++d) {
            const float kv = Kt[d * BKEY + lane];
#pragma unroll
            for (int i = 0; i < QW; ++i) s[i] = fmaf(qw[i * D + d], kv, s[i]);
        }
#pragma unroll
        for (int i = 0; i < QW; ++i) {
            const uint32_t qi = q0 + wave * QW + i;
            float sc;
            if (key >= kend || qi >= sq || (a.causal && key > qi + off)) {
                sc = -__builtin_inff();
            } else {
                sc = s[i] * a.scale;
                if (Mh) sc += Mh[static_cast<uint64_t>(qi) * sk + key];
            }
            const float bmax = dev::wave_max(sc);
            float p = 0.0f;
            if (isfinite(bmax)) {  // wave-uniform
                const float new_m = fmaxf(m[i], bmax);
                const float alpha = dev::fast_expf(m[i] - new_m);
                p = dev::fast_expf(sc - new_m);
                l[i] = l[i] * alpha + dev::wave_sum(p);
#pragma unroll
                for (int t = 0; t < 4; ++t) acc[i][t] *= alpha;
                m[i] = new_m;
            }
            Ps[(wave * QW + i) * BKEY + lane] = p;
        }
        __syncthreads();
        for (int j = 0; j < BKEY; ++j) {
            float pj[QW];
#pragma unroll
            for (int i = 0; i < QW; ++i) pj[i] = Ps[(wave * QW + i) * BKEY + j];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t d = lane + 64 * t;
                if (t < static_cast<int>(DL) && d < D) {
                    const float v = Vs[j * D + d];
#pragma unroll
                    for (int i = 0; i < QW; ++i) acc[i][t] = fmaf(pj[i], v, acc[i][t]);
                }
            }
        }
    }

#pragma unroll
    for (int i = 0; i < QW; ++i) {
        const uint32_t qi = q0 + wave * QW + i;
        if (qi >= sq) continue;
        if (splits == 1) {
            const float inv = l[i] > 0.0f ? 1.0f / l[i] : 0.0f;
            float *o = a.O + (bh * sq + qi) * D;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t d = lane + 64 * t;
                if (t < static_cast<int>(DL) && d < D) o[d] = acc[i][t] * inv;
            }
        } else {
            const uint64_t row = (static_cast<uint64_t>(split) * gridDim.y + bh) * sq + qi;
            float *o = ws_acc + row * D;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t d = lane + 64 * t;
                if (t < static_cast<int>(DL) && d < D) o[d] = acc[i][t];
            }
            if (lane == 0) {
                ws_ml[row * 2 + 0] = m[i];
                ws_ml[row * 2 + 1] = l[i];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Decode kernel (seq_q <= 4, head_dim a multiple of 32): streams K and V.
//
// Eight lanes own one key at a time: lane r of a group reads float4 r, r+8,
// r+16, ... of the key's K and V rows (one contiguous 128-byte segment per
// float4 index), so a wave reads 8 whole rows per step.  Every group runs its
// own online softmax (m, l, acc) over the keys it owns (keys kbeg + 32*i +
// its stream index), so steps need no cross-group reduction; the 32 streams
// of the workgroup are merged once at the end.  Loads are clamped and
// flagged rather than branched, and the next key's rows are in flight while
// the current key is consumed.
// ---------------------------------------------------------------------------
constexpr int kStreams = 32;   // 4 waves x 8 groups

__device__ __forceinline__ void merge_stream(float &m, float &l, float &mo, float &lo, float &a,
                                             float &b)
{
    const float M = fmaxf(m, mo);
    a = (m == -__builtin_inff()) ? 0.0f : dev::fast_expf(m - M);
    b = (mo == -__builtin_inff()) ? 0.0f : dev::fast_expf(mo - M);
    l = l * a + lo * b;
    m = M;
}

// K and V rows are read once per call: nontemporal loads keep them from
// displacing the L2's reusable lines.
__device__ __forceinline__ float4 load_stream(const float4 *p)
{
    typedef float nv4 __attribute__((ext_vector_type(4)));
    const nv4 v = __builtin_nontemporal_load(reinterpret_cast<const nv4 *>(p));
    return make_float4(v[0], v[1], v[2], v[3]);
}

// A stream's reference point m moves only when a score exceeds it by more
// than this (weights stay below e^5.5 ~ 256), so acc is rescaled on rare
// keys only; softmax is invariant to the reference point.
constexpr float kDecodeLazy = 5.5f;

template <int QN, int V4>
__global__ __launch_bounds__(kThreads) void attn_decode_kernel(Attn a, uint32_t keys_per_split,
                                                               uint32_t splits, float *ws_acc,
                                                               float *ws_ml)
{
    __shared__ float red_ml[4][QN][2];
    __shared__ float4 red_acc[4][QN][8][V4];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 3, r = lane & 7;
    const uint32_t D = a.head_dim;
    const uint64_t bh = blockIdx.y;
    const uint32_t q0 = blockIdx.x * QN, split = blockIdx.z;
    const uint32_t sq = a.seq_q, sk = a.seq_k;
    const uint32_t off = sk > sq ? sk - sq : 0;
    const uint32_t nq = min(static_cast<uint32_t>(QN), sq - q0);
    const float4 *Kh = reinterpret_cast<const float4 *>(a.K + bh * sk * D);
    const float4 *Vh = reinterpret_cast<const float4 *>(a.V + bh * sk * D);
    const uint32_t D4 = D >> 2;

    float4 q[QN][V4];
#pragma unroll
    for (int i = 0; i < QN; ++i)
#pragma unroll
        for (int t = 0; t < V4; ++t) {
            const uint32_t qi = min(q0 + i, sq - 1);
            q[i][t] = reinterpret_cast<const float4 *>(a.Q + (bh * sq + qi) * D)[r + 8 * t];
        }

    const uint32_t kbeg = split * keys_per_split;
    uint32_t kend = min(sk, kbeg + keys_per_split);
    if (a.causal) kend = min(kend, q0 + nq - 1 + off + 1);
    const uint32_t stream = wave * 8 + g;
    const uint32_t nsteps = kend > kbeg ? (kend - kbeg + kStreams - 1) / kStreams : 0;

    float m[QN], l[QN];
    float4 acc[QN][V4];
#pragma unroll
    for (int i = 0; i < QN; ++i) {
        m[i] = -__builtin_inff();
        l[i] = 0.0f;
#pragma unroll
        for (int t = 0; t < V4; ++t) acc[i][t] = make_float4(0.f, 0.f, 0.f, 0.f);
    }

    auto load = [&](uint32_t step, float4 (&kr)[V4], float4 (&vr)[V4]) {
        const uint32_t key = min(kbeg + stream + step * kStreams, kend - 1);
#pragma unroll
        for (int t = 0; t < V4; ++t) {
            kr[t] = load_stream(Kh + static_cast<uint64_t>(key) * D4 + r + 8 * t);
            vr[t] = load_stream(Vh + static_cast<uint64_t>(key) * D4 + r + 8 * t);
        }
    };
    // One key step: this stream's key kbeg + stream + 32 step.
    auto consume = [&](uint32_t step, const float4 (&kc)[V4], const float4 (&vc)[V4]) {
        const uint32_t key = kbeg + stream + step * kStreams;
#pragma unroll
        for (int i = 0; i < QN; ++i) {
            float dot = 0.0f;
#pragma unroll
            for (int t = 0; t < V4; ++t) {
                dot = fmaf(q[i][t].x, kc[t].x, dot);
                dot = fmaf(q[i][t].y, kc[t].y, dot);
                dot = fmaf(q[i][t].z, kc[t].z, dot);
                dot = fmaf(q[i][t].w, kc[t].w, dot);
            }
            dot += __shfl_xor(dot, 1, 64);
            dot += __shfl_xor(dot, 2, 64);
            dot += __shfl_xor(dot, 4, 64);
            const uint32_t qi = q0 + i;
            const bool live = key < kend && i < static_cast<int>(nq) && !(a.causal && key > qi + off);
            if (live) {   // uniform over the 8 lanes of the group
                float s = dot * a.scale;
                if (a.mask) s += a.mask[(bh * sq + qi) * sk + key];
                if (s > m[i] + kDecodeLazy) {   // also the first key (m = -inf)
                    const float al = (m[i] == -__builtin_inff()) ? 0.0f : dev::fast_expf(m[i] - s);
                    l[i] *= al;
#pragma unroll
                    for (int t = 0; t < V4; ++t) {
                        acc[i][t].x *= al;
                        acc[i][t].y *= al;
                        acc[i][t].z *= al;
                        acc[i][t].w *= al;
                    }
                    m[i] = s;
                }
                // m is still -inf only if every key so far, this one included,
                // scored -inf (an additive -inf mask): such a key weighs 0, as
                // fast_expf(-inf - m) does for any finite m.
                const float p = (m[i] == -__builtin_inff()) ? 0.0f : dev::fast_expf(s - m[i]);
                l[i] += p;
#pragma unroll
                for (int t = 0; t < V4; ++t) {
                    acc[i][t].x = fmaf(p, vc[t].x, acc[i][t].x);
                    acc[i][t].y = fmaf(p, vc[t].y, acc[i][t].y);
                    acc[i][t].z = fmaf(p, vc[t].z, acc[i][t].z);
                    acc[i][t].w = fmaf(p, vc[t].w, acc[i][t].w);
                }
            }
        }
    };
    // Three register sets in rotation: while one step is consumed the next
    // two are in flight.
    float4 k0[V4], v0[V4], k1[V4], v1[V4], k2[V4], v2[V4];
    if (nsteps > 0) load(0, k0, v0);
    if (nsteps > 1) load(1, k1, v1);
    if (nsteps > 2) load(2, k2, v2);
    for (uint32_t step = 0; step < nsteps; step += 3) {
        consume(step, k0, v0);
        if (step + 3 < nsteps) load(step + 3, k0, v0);
        if (step + 1 >= nsteps) break;
        consume(step + 1, k1, v1);
        if (step + 4 < nsteps) load(step + 4, k1, v1);
        if (step + 2 >= nsteps) break;
        consume(step + 2, k2, v2);
        if (step + 5 < nsteps) load(step + 5, k2, v2);
    }

    // Merge the 8 groups of the wave (lanes differing in bits 3..5), then
    // the 4 waves through LDS.
#pragma unroll
    for (int i = 0; i < QN; ++i) {
#pragma unroll
        for (int sh = 8; sh < 64; sh <<= 1) {
            float mo = __shfl_xor(m[i], sh, 64), lo = __shfl_xor(l[i], sh, 64), wa, wb;
            merge_stream(m[i], l[i], mo, lo, wa, wb);
#pragma unroll
            for (int t = 0; t < V4; ++t) {
                float4 o;
                o.x = __shfl_xor(acc[i][t].x, sh, 64);
                o.y = __shfl_xor(acc[i][t].y, sh, 64);
                o.z = __shfl_xor(acc[i][t].z, sh, 64);
                o.w = __shfl_xor(acc[i][t].w, sh, 64);
                acc[i][t].x = acc[i][t].x * wa + o.x * wb;
                acc[i][t].y = acc[i][t].y * wa + o.y * wb;
                acc[i][t].z = acc[i][t].z * wa + o.z * wb;
                acc[i][t].w = acc[i][t].w * wa + o.w * wb;
            }
        }
        if (g == 0) {
            if (r == 0) {
                red_ml[wave][i][0] = m[i];
                red_ml[wave][i][1] = l[i];
            }
#pragma unroll
            for (int t = 0; t < V4; ++t) red_acc[wave][i][r][t] = acc[i][t];
        }
    }
    __syncthreads();
    if (wave != 0 || g != 0) return;
#pragma unroll
    for (int i = 0; i < QN; ++i) {
        if (i >= static_cast<int>(nq)) break;
        for (int w = 1; w < 4; ++w) {
            float mo = red_ml[w][i][0], lo = red_ml[w][i][1], wa, wb;
            merge_stream(m[i], l[i], mo, lo, wa, wb);
#pragma unroll
            for (int t = 0; t < V4; ++t) {
                const float4 o = red_acc[w][i][r][t];
                acc[i][t].x = acc[i][t].x * wa + o.x * wb;
                acc[i][t].y = acc[i][t].y * wa + o.y * wb;
                acc[i][t].z = acc[i][t].z * wa + o.z * wb;
                acc[i][t].w = acc[i][t].w * wa + o.w * wb;
            }
        }
        const uint32_t qi = q0 + i;
        if (splits == 1) {
            const float inv = l[i] > 0.0f ? 1.0f / l[i] : 0.0f;
            float4 *o = reinterpret_cast<float4 *>(a.O + (bh * sq + qi) * D);
#pragma unroll
            for (int t = 0; t < V4; ++t)
                o[r + 8 * t] = make_float4(acc[i][t].x * inv, acc[i][t].y * inv, acc[i][t].z * inv,
                                           acc[i][t].w * inv);
        } else {
            const uint64_t row = (static_cast<uint64_t>(split) * gridDim.y + bh) * sq + qi;
            float4 *o = reinterpret_cast<float4 *>(ws_acc + row * D);
#pragma unroll
            for (int t = 0; t < V4; ++t) o[r + 8 * t] = acc[i][t];
            if (r == 0) {
                ws_ml[row * 2 + 0] = m[i];
                ws_ml[row * 2 + 1] = l[i];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Prefill (head_dim 64 or 128, seq_q > 4) on the bf16 matrix cores with
// three-term split products.
//
// gfx950 multiplies bf16 ~11x faster than f32 on its matrix cores (measured
// with random operands: v_mfma_f32_32x32x16_bf16 1.8 PFLOP/s against
// v_mfma_f32_16x16x4_f32 157 TFLOP/s).  Every f32 operand x is split into
// hi = bf16(x) and lo = bf16(x - hi) (x - hi is exact in f32), and a product
// is taken as hi*hi + hi*lo + lo*hi with f32 accumulation: the dropped lo*lo
// term and the rounding of lo leave a relative error of about 2^-16 per
// product, far inside the attention bar of 2e-3 (the f32 kernel's own
// softmax exponent differs from the reference's by 1.5e-4).
//
// A pre-pass (attn_split_kv) writes K and V of every 32-key block, split and
// laid out for the fragment reads, as one contiguous 32 KiB (D = 128) block:
//   K hi | K lo : [key][d] bf16, 16-byte chunk c of key k at slot
//                 c ^ k_swizzle(k);
//   V^T hi | lo : [d][position] bf16, 32 positions per row in the key order
//                 that the PV step consumes (vt_key), chunk c of row d at
//                 slot c ^ ((d >> 2) & 3).
// ds_read_b128 serves 16 lanes at a time from one 256-byte window of banks;
// the swizzles put the 16 rows a quarter wave reads at one chunk in 16
// distinct 16-byte slots of that window.
// Keys past seq_k are written as zeros (their scores are masked anyway).
//
// Main kernel: a workgroup of 8 waves owns 128 queries of one (batch, head):
// waves w and w+4 own queries q0 + 32(w%4) .. +31 and take the even and the
// odd 32-key blocks of every 64-key super block (two waves per SIMD, one
// barrier per super block, the next super block's 64 KiB in flight by DMA
// while this one is multiplied).  Per 32-key block a wave runs
// v_mfma_f32_32x32x16_bf16:
//   S^T (32 keys x 32 queries) = K . Q^T      (Q^T hi/lo in VGPRs)
//   O^T (D x 32 queries)      += V^T . P^T    (P^T from the lane's scores)
// The 32 x 32 accumulator puts query l%32 and keys 8j + 4(l/32) + i
// (register 4j + i) in lane l, so a query's block max and sum combine two
// lanes (l, l^32), and the PV step over keys 16t..16t+15 takes the lane's
// score registers 8t..8t+7 as its P^T operand when V^T's positions follow
// the same key order.  The two key halves are merged through LDS at the end,
// O leaves through LDS so every global row write is coalesced.
// Online softmax as in the reference (a query whose block is fully masked
// skips the block).
// ---------------------------------------------------------------------------
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
constexpr int XQ = 32;           // queries per wave
constexpr int XK = 32;           // keys per block
constexpr int PQ = 128;          // queries per workgroup
constexpr int PThreads = 512;    // 8 waves: 4 query groups x 2 key halves

template <int D>
struct SplitBlk {
    static constexpr int kHalfK = XK * D * 2;                    // bytes of K hi (or lo)
    static constexpr int kHalfV = D * XK * 2;                    // bytes of V^T hi (or lo)
    static constexpr int kVOff = 2 * kHalfK;
    static constexpr int kBytes = 2 * kHalfK + 2 * kHalfV;       // one 32-key block
    static constexpr int kChunks = D / 8;                        // 16-byte chunks per K row
    static constexpr size_t kLds = 4 * static_cast<size_t>(kBytes);  // 2 super blocks of 2 blocks
    static constexpr int kOPitch = D + 4;                        // floats per staged row
    static_assert(4 * XQ * kOPitch * 4 + 4 * XQ * 2 * 4 <= static_cast<int>(kLds), "merge staging fits");
};

// Key (within its 32-key block) at V^T position p: the PV step t = p/16 of
// lane half h = (p/8)%2 multiplies element e = p%8 with the lane's score
// register 8t + e, which holds key 16t + 4h + e (e < 4) or 16t + 8 + 4h +
// e - 4 (e >= 4).
// K rows are 2D bytes: 256 (D = 128) rows differ in all 16 slots of a
// window by k % 16; 128-byte rows (D = 64) pair up in a window, so the slot
// varies with k / 2.
template <int D>
__device__ __forceinline__ uint32_t k_swizzle(uint32_t k)
{
    return D == 128 ? (k & 15) : ((k >> 1) & 7);
}

__device__ __forceinline__ uint32_t vt_key(uint32_t p)
{
    const uint32_t t = p >> 4, h = (p >> 3) & 1, e = p & 7;
    return 16 * t + (e < 4 ? 4 * h + e : 8 + 4 * h + (e - 4));
}

__device__ __forceinline__ void split_bf16(const float (&x)[8], v8bf &hi, v8bf &lo)
{
    // hi rounded to nearest even, two per v_cvt_pk_bf16_f32; its f32 value is
    // the packed word's halves moved to the top; lo = bf16(x - hi).
    typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
    typedef float v2f __attribute__((ext_vector_type(2)));
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        hw[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){x[2 * e], x[2 * e + 1]}, v2bf));
        const float h0 = __builtin_bit_cast(float, hw[e] << 16);
        const float h1 = __builtin_bit_cast(float, hw[e] & 0xFFFF0000u);
        lw[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){x[2 * e] - h0, x[2 * e + 1] - h1}, v2bf));
    }
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    hi = __builtin_bit_cast(v8bf, (v4u){hw[0], hw[1], hw[2], hw[3]});
    lo = __builtin_bit_cast(v8bf, (v4u){lw[0], lw[1], lw[2], lw[3]});
}

// One (32-key block, batch*head) per workgroup of 256 threads.  Every load
// is issued before the first split, through raw buffers over the block's
// keys (keys past seq_k read as zero, which is what the layout holds for
// them), so no branch separates loads from stores: with loads under
// branches the compiler waited for all memory operations, the previous
// item's stores included, before each item.
//   * K: item (key, 16-byte chunk c), C = D / 8 chunks per key, 4D items;
//   * V^T: item (position chunk ch, column pair d2): 8 keys' float2 at
//     columns 2 d2, 2 d2 + 1 give rows 2 d2 and 2 d2 + 1 of chunk ch; 2D
//     items, so every thread has one at D = 128.
template <int D>
__global__ __launch_bounds__(256) void attn_split_kv(Attn a, uint32_t nkb, int8_t *split)
{
    using S = SplitBlk<D>;
    constexpr int C = S::kChunks;
    constexpr int KItems = XK * C, VItems = (XK / 8) * (D / 2);
    constexpr int NK = (KItems + 255) / 256, NV = (VItems + 255) / 256;
    const uint32_t kb = blockIdx.x, tid = threadIdx.x;
    const uint64_t bh = blockIdx.y;
    const uint32_t sk = a.seq_k, key0 = kb * XK, nk = min(static_cast<uint32_t>(XK), sk - key0);
    int8_t *blk = split + (bh * nkb + kb) * S::kBytes;
    const uint64_t base = (bh * sk + key0) * D;
    const int bytes = static_cast<int>(nk * D * 4u);
    const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(a.K + base), 0, bytes, 0x00020000);
    const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(a.V + base), 0, bytes, 0x00020000);
    float kx[NK][8];
    float2 vx[NV][8];
#pragma unroll
    for (int i = 0; i < NK; ++i) {
        const uint32_t it = tid + 256 * i, key = it / C, c = it % C;
        const int off = static_cast<int>((key * D + 8 * c) * 4);
        const float4 u = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
        const float4 v = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, off + 16, 0, 0));
        kx[i][0] = u.x; kx[i][1] = u.y; kx[i][2] = u.z; kx[i][3] = u.w;
        kx[i][4] = v.x; kx[i][5] = v.y; kx[i][6] = v.z; kx[i][7] = v.w;
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const uint32_t it = tid + 256 * i, d2 = it % (D / 2), ch = it / (D / 2);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int off = static_cast<int>((vt_key(8 * ch + e) * D + 2 * d2) * 4);
            vx[i][e] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rv, off, 0, 0));
        }
    }
#pragma unroll
    for (int i = 0; i < NK; ++i) {
        const uint32_t it = tid + 256 * i, key = it / C, c = it % C;
        if (it >= KItems) continue;
        v8bf hi, lo;
        split_bf16(kx[i], hi, lo);
        const uint32_t off = key * (D * 2) + ((c ^ k_swizzle<D>(key)) << 4);
        *reinterpret_cast<v8bf *>(blk + off) = hi;
        *reinterpret_cast<v8bf *>(blk + S::kHalfK + off) = lo;
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const uint32_t it = tid + 256 * i, d2 = it % (D / 2), ch = it / (D / 2);
        if (it >= VItems) continue;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint32_t d = 2 * d2 + q;
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = q ? vx[i][e].y : vx[i][e].x;
            v8bf hi, lo;
            split_bf16(x, hi, lo);
            const uint32_t off = d * (XK * 2) + ((ch ^ ((d >> 2) & 3)) << 4);
            *reinterpret_cast<v8bf *>(blk + S::kVOff + off) = hi;
            *reinterpret_cast<v8bf *>(blk + S::kVOff + S::kHalfV + off) = lo;
        }
    }
}

using lds::dma16;

// Softmax weights use the hardware exp2 (v_exp_f32) on base-2 scores (Q is
// pre-scaled by log2 e).  The reference's degree-5 polynomial
// (dev::fast_expf) spends ~10 VALU ops per weight; the two differ by at most
// ~1.5e-4 relative (the polynomial's own truncation error), far inside the
// attention bar of 2e-3; the decode kernel keeps the polynomial.
__device__ __forceinline__ v16f mfma_bf16(const v8bf &a, const v8bf &b, const v16f &c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// One block of PQ queries starting at q0, for (batch, head) bh.
template <int D>
__device__ __forceinline__ void prefill_block(const Attn &a, uint32_t q0, uint64_t bh, uint32_t nkb,
                                              const int8_t *split, int8_t *lds)
{
    using S = SplitBlk<D>;
    constexpr int NS = D / 16;          // QK steps (16 d each)
    constexpr int DT = D / 32;          // 32-row tiles of O^T
    constexpr int kInstr = 2 * S::kBytes / 1024;   // DMA instructions per super block

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wq = wave & 3, wk = wave >> 2;
    const int h = lane >> 5, col = lane & 31;
    const uint32_t sq = a.seq_q, sk = a.seq_k;
    const uint32_t off = sk > sq ? sk - sq : 0;
    const float *Mh = a.mask ? a.mask + bh * sq * sk : nullptr;
    const uint32_t qw = q0 + wq * XQ;                         // this wave's first query
    const uint32_t myq = qw + col;                            // this lane's query
    const int8_t *src = split + bh * nkb * S::kBytes;

    uint32_t kend = sk;
    if (a.causal) kend = min(sk, min(q0 + PQ, sq) - 1 + off + 1);
    const uint32_t nblk = (kend + XK - 1) / XK;
    const uint32_t nsb = (nblk + 1) / 2;
    const uint32_t wave_kend = a.causal ? min(kend, min(qw + XQ, sq) - 1 + off + 1) : kend;

    // Q^T operand of step s: lane (query col, half h) holds d = 16s + 8h .. +8,
    // pre-multiplied by scale * log2(e) so scores come out in base-2 units
    // (softmax weights are exp2(s - m); m, alpha and the merge use base 2).
    constexpr float kLog2e = 1.4426950408889634f;
    v8bf qh[NS], ql[NS];
    {
        const float qs = a.scale * kLog2e;
        const float4 *qrow = reinterpret_cast<const float4 *>(a.Q + (bh * sq + min(myq, sq - 1)) * D + 8 * h);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const float4 u = qrow[4 * s], v = qrow[4 * s + 1];
            const float x[8] = {u.x * qs, u.y * qs, u.z * qs, u.w * qs, v.x * qs, v.y * qs, v.z * qs, v.w * qs};
            split_bf16(x, qh[s], ql[s]);
        }
    }

    // LDS slot of block 2sb + wk: super block sb sits in ring slot sb % 2.
    auto slot = [&](uint32_t sb) -> int8_t * {
        return lds + ((sb & 1) * 2 + wk) * S::kBytes;
    };
    // DMA of block 2sb + wk: waves 0-3 copy the even block, 4-7 the odd one
    // (skipped past nblk).
    auto issue = [&](uint32_t sb) {
        const uint32_t blk = 2 * sb + wk;
        if (blk >= nblk) return;                                  // wave-uniform
        int8_t *dst = slot(sb);
        const int8_t *from = src + static_cast<uint64_t>(blk) * S::kBytes + lane * 16;
#pragma unroll
        for (int i = 0; i < kInstr / 8; ++i) {
            const int ins = wq * (kInstr / 8) + i;                // 1 KiB piece of the block
            dma16(from + ins * 1024, dst + ins * 1024);
        }
    };

    v16f o[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] = (v16f){0.f};
    float m = -__builtin_inff(), l = 0.0f;

    // S^T = K . Q^T, one accumulator chain (the cross terms first).
    auto qk = [&](const int8_t *blk, v16f &sa) {
        sa = (v16f){0.f};
        const int8_t *krow = blk + col * (D * 2);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const uint32_t koff = ((2 * s + h) ^ k_swizzle<D>(col)) << 4;
            const v8bf kh = *reinterpret_cast<const v8bf *>(krow + koff);
            const v8bf kl = *reinterpret_cast<const v8bf *>(krow + S::kHalfK + koff);
            sa = mfma_bf16(kl, qh[s], sa);
            sa = mfma_bf16(kh, ql[s], sa);
            sa = mfma_bf16(kh, qh[s], sa);
        }
    };

    // Online softmax of block kb: scores of query myq for keys kb*32 + 8j +
    // 4h + i (register 4j + i) -> split weights ph/pl, rescaled O^T.  A block
    // whose keys are all below every query's causal limit and kend (wave-
    // uniform) needs no masking.
    auto softmax = [&](uint32_t kb, const v16f &sa, v8bf (&ph)[2], v8bf (&pl)[2]) {
        const bool interior = (kb + 1) * XK <= kend && qw + XQ - 1 < sq &&
                              (!a.causal || (kb + 1) * XK - 1 <= qw + off);
        float sc[16];
        float bmax = -__builtin_inff();
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float v = sa[r];
            if (!interior || Mh) {
                const uint32_t key = kb * XK + 8 * (r >> 2) + 4 * h + (r & 3);
                if (Mh) v += Mh[static_cast<uint64_t>(min(myq, sq - 1)) * sk + min(key, sk - 1)] * kLog2e;
                const bool dead = key >= kend || myq >= sq || (a.causal && key > myq + off);
                v = dead ? -__builtin_inff() : v;
            }
            sc[r] = v;
            bmax = fmaxf(bmax, v);
        }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
        // Lazy reference point: weights are exp2(s - m) with m moved only when
        // the block max exceeds it by more than 8 (weights stay <= 256), so
        // O^T is rescaled only on those rare blocks; softmax is invariant to
        // the reference point.  A block whose max is not finite adds nothing.
        const bool grow = bmax > m + 8.0f;                // also the first live block (m = -inf)
        const float mn = grow ? bmax : m;
        const float alpha = grow ? __builtin_amdgcn_exp2f(m - mn) : 1.0f;   // 0 when m = -inf
        const float ref = mn == -__builtin_inff() ? 0.0f : mn;             // exp2(-inf - 0) = 0
        float psum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float p = __builtin_amdgcn_exp2f(sc[r] - ref);
            sc[r] = p;
            psum += p;
        }
        psum += __shfl_xor(psum, 32, 64);
        l = l * alpha + psum;
        if (__ballot(grow && m != -__builtin_inff())) {   // wave-uniform; O^T is 0 before the first
#pragma unroll
            for (int t = 0; t < DT; ++t) o[t] *= alpha;
        }
        m = mn;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const float x[8] = {sc[8 * t], sc[8 * t + 1], sc[8 * t + 2], sc[8 * t + 3],
                                sc[8 * t + 4], sc[8 * t + 5], sc[8 * t + 6], sc[8 * t + 7]};
            split_bf16(x, ph[t], pl[t]);
        }
    };

    // O^T += V^T . P^T over keys 16t..16t+15: P^T = score registers 8t..8t+7.
    auto pv = [&](const int8_t *vt, const v8bf (&ph)[2], const v8bf (&pl)[2]) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const uint32_t d = 32 * dt + col;
                const uint32_t voff = d * (XK * 2) + (((2 * t + h) ^ ((d >> 2) & 3)) << 4);
                const v8bf vh = *reinterpret_cast<const v8bf *>(vt + voff);
                const v8bf vl = *reinterpret_cast<const v8bf *>(vt + S::kHalfV + voff);
                o[dt] = mfma_bf16(vl, ph[t], o[dt]);
                o[dt] = mfma_bf16(vh, pl[t], o[dt]);
                o[dt] = mfma_bf16(vh, ph[t], o[dt]);
            }
    };

    if (nsb) issue(0);
    for (uint32_t sb = 0; sb < nsb; ++sb) {
        __builtin_amdgcn_s_waitcnt(0xF70);   // vmcnt(0): this wave's DMA of super block sb
        __syncthreads();                     // landed everywhere; super block sb-1's slot free
        if (sb + 1 < nsb) issue(sb + 1);
        const uint32_t kb = 2 * sb + wk;
        if (kb * XK >= wave_kend) continue;  // wave-uniform: past this wave's causal limit
        const int8_t *blk = slot(sb);
        v16f sa;
        qk(blk, sa);
        v8bf ph[2], pl[2];
        softmax(kb, sa, ph, pl);
        pv(blk + S::kVOff, ph, pl);
    }

    // Merge the two key halves: waves 4-7 stage (m, l, O^T) in LDS, waves 0-3
    // combine them with their own, normalise, and stage O row-major; then all
    // waves write the 128 rows.  Lane (query col, half h) holds O^T rows
    // d = 32dt + 8j + 4h + i in register 4j + i of tile dt: one float4 per
    // (dt, j), stored at row col of the wave's [32][D + 4] tile.
    __syncthreads();
    float *ot = reinterpret_cast<float *>(lds) + wq * XQ * S::kOPitch;
    float *ml = reinterpret_cast<float *>(lds) + 4 * XQ * S::kOPitch + wq * XQ * 2;
    if (wk == 1) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<v4f *>(ot + col * S::kOPitch + 32 * dt + 8 * j + 4 * h) =
                    (v4f){o[dt][4 * j], o[dt][4 * j + 1], o[dt][4 * j + 2], o[dt][4 * j + 3]};
        if (h == 0) {
            ml[2 * col] = m;
            ml[2 * col + 1] = l;
        }
    }
    __syncthreads();
    if (wk == 0) {
        const float m1 = ml[2 * col], l1 = ml[2 * col + 1];
        const float M = fmaxf(m, m1);
        const float a0 = m == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m - M);
        const float a1 = m1 == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m1 - M);
        const float L = a0 * l + a1 * l1;
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        const float w0 = a0 * inv, w1 = a1 * inv;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v4f *p = reinterpret_cast<v4f *>(ot + col * S::kOPitch + 32 * dt + 8 * j + 4 * h);
                const v4f other = *p;
                *p = (v4f){o[dt][4 * j] * w0 + other[0] * w1, o[dt][4 * j + 1] * w0 + other[1] * w1,
                           o[dt][4 * j + 2] * w0 + other[2] * w1, o[dt][4 * j + 3] * w0 + other[3] * w1};
            }
    }
    __syncthreads();
    const float *stage = reinterpret_cast<const float *>(lds);
    for (uint32_t i = tid; i < PQ * D / 4; i += PThreads) {
        const uint32_t row = i / (D / 4), c4 = i % (D / 4);
        const uint32_t q = q0 + row;
        if (q < sq)
            *reinterpret_cast<v4f *>(a.O + (bh * sq + q) * D + 4 * c4) =
                *reinterpret_cast<const v4f *>(stage + row * S::kOPitch + 4 * c4);
    }
}

// Causal blocks cost in proportion to their position, so with nqb blocks per
// head the grid has ceil(nqb/2) workgroups per head and workgroup x takes
// block nqb-1-x and then block x: every workgroup does the same work (the
// grid otherwise runs as long as its last, heaviest block).  Without a
// causal mask every block costs the same and each workgroup takes one.
template <int D>
__global__ __launch_bounds__(PThreads) void attn_prefill_kernel(Attn a, uint32_t nqb, uint32_t nkb,
                                                                const int8_t *split)
{
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];
    // Workgroup g runs on XCD g % 8: give each XCD a contiguous run of
    // (query block, head) pairs, so the workgroups of one head share its
    // split K / V blocks through one L2 instead of fetching them once per XCD.
    const uint32_t nx = gridDim.x, total = nx * gridDim.y;
    uint32_t g = blockIdx.x + nx * blockIdx.y;
    if ((total & 7u) == 0) g = (g & 7u) * (total >> 3) + (g >> 3);
    const uint32_t bx = g % nx;
    const uint64_t bh = g / nx;
    const uint32_t heavy = nqb - 1 - bx;
    prefill_block<D>(a, heavy * PQ, bh, nkb, split, lds);
    if (nx < nqb && bx != heavy) {
        __syncthreads();  // the output staging of the first block is read out
        prefill_block<D>(a, bx * PQ, bh, nkb, split, lds);
    }
}

// Merge split partials: O = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s.
__global__ __launch_bounds__(kThreads) void attn_merge(Attn a, uint32_t splits, uint64_t rows,
                                                       const float *ws_acc, const float *ws_ml)
{
    const uint32_t D = a.head_dim;
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (idx >= rows * D) return;
    const uint64_t row = idx / D;
    const uint32_t d = static_cast<uint32_t>(idx % D);
    // Splits in groups of eight whose loads are all issued before any is used
    // (one L2 round trip per group, not two per split); the sums run in split
    // order, skipping splits with no unmasked key.
    constexpr uint32_t G = 8;
    float M = -__builtin_inff();
    for (uint32_t s0 = 0; s0 < splits; s0 += G) {
        float ms[G];
#pragma unroll
        for (uint32_t u = 0; u < G; ++u)
            ms[u] = s0 + u < splits ? ws_ml[((s0 + u) * rows + row) * 2] : -__builtin_inff();
#pragma unroll
        for (uint32_t u = 0; u < G; ++u) M = fmaxf(M, ms[u]);
    }
    float num = 0.0f, den = 0.0f;
    if (isfinite(M)) {
        for (uint32_t s0 = 0; s0 < splits; s0 += G) {
            float ms[G], acc[G], l[G];
#pragma unroll
            for (uint32_t u = 0; u < G; ++u) {
                const bool in = s0 + u < splits;
                const uint64_t r = static_cast<uint64_t>(s0 + u) * rows + row;
                ms[u] = in ? ws_ml[r * 2] : -__builtin_inff();
                acc[u] = in ? ws_acc[r * D + d] : 0.0f;
                l[u] = in ? ws_ml[r * 2 + 1] : 0.0f;
            }
#pragma unroll
            for (uint32_t u = 0; u < G; ++u) {
                if (!isfinite(ms[u])) continue;
                const float w = dev::fast_expf(ms[u] - M);
                num = fmaf(w, acc[u], num);
                den = fmaf(w, l[u], den);
            }
        }
    }
    a.O[row * D + d] = den > 0.0f ? num / den : 0.0f;
}

template <int QN>
void decode_launch_v(int v4, dim3 grid, hipStream_t s, const Attn &a, uint32_t kps,
                     uint32_t splits, float *ws_acc, float *ws_ml)
{
    switch (v4) {
    case 1: attn_decode_kernel<QN, 1><<<grid, kThreads, 0, s>>>(a, kps, splits, ws_acc, ws_ml); break;
    case 2: attn_decode_kernel<QN, 2><<<grid, kThreads, 0, s>>>(a, kps, splits, ws_acc, ws_ml); break;
    case 3: attn_decode_kernel<QN, 3><<<grid, kThreads, 0, s>>>(a, kps, splits, ws_acc, ws_ml); break;
    case 4: attn_decode_kernel<QN, 4><<<grid, kThreads, 0, s>>>(a, kps, splits, ws_acc, ws_ml); break;
    case 5: attn_decode_kernel<QN, 5><<<grid, kThreads, 0, s>>>(a, kps, splits, ws_acc, ws_ml); break;
    case 6: attn_decode_kernel<QN, 6><<<grid, kThreads, 0, s>>>(a, kps, splits, ws_acc, ws_ml); break;
    case 7: attn_decode_kernel<QN, 7><<<grid, kThreads, 0, s>>>(a, kps, splits, ws_acc, ws_ml); break;
    default: attn_decode_kernel<QN, 8><<<grid, kThreads, 0, s>>>(a, kps, splits, ws_acc, ws_ml); break;
    }
}

void decode_launch(int qn, int v4, dim3 grid, hipStream_t s, const Attn &a, uint32_t kps,
                   uint32_t splits, float *ws_acc, float *ws_ml)
{
    if (qn == 1) decode_launch_v<1>(v4, grid, s, a, kps, splits, ws_acc, ws_ml);
    else if (qn == 2) decode_launch_v<2>(v4, grid, s, a, kps, splits, ws_acc, ws_ml);
    else decode_launch_v<4>(v4, grid, s, a, kps, splits, ws_acc, ws_ml);
}

// ---------------------------------------------------------------------------
// Reference-order attention: the reference's attention_range
// (llm.cpp:442-546) rounding for rounding, so the output is its output bit
// for bit.  Per query row, keys in 64-key blocks from key 0:
//   * s = dot(q, k) * scale (+ mask), dot in dot_avx2's order (eight FMA
//     chains over the 8-wide steps, hsum256, then the tail unfused);
//   * block max m_b; a block whose max is not finite is skipped; new_m =
//     max(m, m_b), alpha = fast_expf(m - new_m), p_j = fast_expf(s_j - new_m)
//     with the reference's unfused scalar polynomial (dev::fast_expf_unfused);
//   * sum_p adds the block's p_j in key order, l = l * alpha + sum_p;
//   * acc = acc * alpha, then acc = fma(v_j, p_j, acc) in key order (p_j != 0);
//   * out = acc * (1 / l), 0 when l == 0.
// The sums over keys are sequential chains: lanes split the score work and
// the head dimension, never a chain.
// ---------------------------------------------------------------------------
constexpr int RK = 64;   // keys per block (the reference's BK)

// Any head_dim and any number of (batch, head) pairs: one workgroup per
// query row (a 1-D grid), the scores of a block by the lanes of wave 0 (one
// key each), the running output in the output row itself (no bound on
// head_dim; every thread owns the same elements throughout).
__global__ __launch_bounds__(kThreads) void attn_rowwise_kernel(Attn a, uint64_t row0)
{
#pragma clang fp contract(off)
    __shared__ float pw[RK];
    const int tid = threadIdx.x;
    const uint64_t row = row0 + blockIdx.x;
    const uint32_t sq = a.seq_q, sk = a.seq_k, D = a.head_dim;
    const uint64_t bh = row / sq;
    const uint32_t qi = static_cast<uint32_t>(row % sq);
    const uint32_t off = sk > sq ? sk - sq : 0;
    const float *q = a.Q + row * D;
    const float *Kh = a.K + bh * sk * D;
    const float *Vh = a.V + bh * sk * D;
    float *o = a.O + row * D;
    for (uint32_t d = tid; d < D; d += kThreads) o[d] = 0.0f;
    float m = -__builtin_inff(), l = 0.0f;
    uint32_t kend = sk;
    if (a.causal) kend = min(sk, qi + off + 1);
    for (uint32_t k0 = 0; k0 < kend; k0 += RK) {
        const uint32_t kc = min(static_cast<uint32_t>(RK), kend - k0);
        __syncthreads();   // the previous block's weights are consumed
        if (tid < static_cast<int>(kc)) {
            float sc = dev::dot_ref(q, Kh + static_cast<uint64_t>(k0 + tid) * D, D) * a.scale;
            if (a.mask) sc = sc + a.mask[row * sk + k0 + tid];
            pw[tid] = sc;
        }
        __syncthreads();
        float bmax = -__builtin_inff();
        for (uint32_t j = 0; j < kc; ++j) bmax = bmax < pw[j] ? pw[j] : bmax;
        if (!isfinite(bmax)) continue;   // uniform over the workgroup
        const float nm = m < bmax ? bmax : m;
        const float alpha = dev::fast_expf_unfused(m - nm);
        __syncthreads();   // every thread has read the scores
        if (tid < static_cast<int>(kc)) pw[tid] = dev::fast_expf_unfused(pw[tid] - nm);
        __syncthreads();
        float psum = 0.0f;
        for (uint32_t j = 0; j < kc; ++j) psum = psum + pw[j];
        l = l * alpha + psum;
        for (uint32_t d = tid; d < D; d += kThreads) {
            float acc = o[d] * alpha;
            for (uint32_t j = 0; j < kc; ++j) {
                const float p = pw[j];
                if (p != 0.0f) acc = fmaf(Vh[static_cast<uint64_t>(k0 + j) * D + d], p, acc);
            }
            o[d] = acc;
        }
        m = nm;
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    for (uint32_t d = tid; d < D; d += kThreads) o[d] = o[d] * inv;
}

bool use_rowwise(const Attn &a)
{
    return a.head_dim > 256 || static_cast<uint64_t>(a.batch) * a.heads > 65535u ||
           (a.exact && a.head_dim != 64 && a.head_dim != 128);
}

// Reference-order tiled kernel (exact mode, head_dim 64 or 128).
bool use_exact_tiled(const Attn &a)
{
    return a.exact && !use_rowwise(a);
}

bool use_decode(const Attn &a)
{
    return a.seq_q <= 4 && (a.head_dim % 32) == 0 && a.head_dim <= 256;
}

bool use_prefill(const Attn &a)
{
    return !use_decode(a) && (a.head_dim == 64 || a.head_dim == 128);
}

void plan(const Attn &a, uint32_t &qblocks, uint32_t &splits, uint32_t &kps)
{
    if (use_rowwise(a)) {
        qblocks = 1;
        splits = 1;
        kps = a.seq_k;
        return;
    }
    if (use_prefill(a)) {
        qblocks = (a.seq_q + PQ - 1) / PQ;
        splits = 1;
        kps = a.seq_k;
        return;
    }
    if (use_decode(a)) {
        // One workgroup per (batch, head) and key range: enough ranges for
        // ~1024 workgroups (four per CU), each at least 256 keys (8 per
        // stream).  B8 x 32 heads x 4096 keys: 161.6 us at 1024, 163.0 at
        // 2048, 167.5 at 4096 workgroups.
        qblocks = 1;
        const uint64_t bh = static_cast<uint64_t>(a.batch) * a.heads;
        const uint32_t max_splits = std::max<uint32_t>(1, (a.seq_k + 255) / 256);
        splits = static_cast<uint32_t>(std::min<uint64_t>(max_splits, std::max<uint64_t>(1, (1024 + bh - 1) / bh)));
        kps = ((a.seq_k + splits - 1) / splits + kStreams - 1) / kStreams * kStreams;
        splits = (a.seq_k + kps - 1) / kps;
        return;
    }
    qblocks = (a.seq_q + BQ - 1) / BQ;
    const uint64_t tiles = static_cast<uint64_t>(qblocks) * a.batch * a.heads;
    splits = 1;
    const uint32_t kblocks = (a.seq_k + BKEY - 1) / BKEY;
    while (tiles * splits < 2048 && splits * 2 <= kblocks && kblocks / (splits * 2) >= 2) splits *= 2;
    kps = ((kblocks + splits - 1) / splits) * BKEY;
    splits = (a.seq_k + kps - 1) / kps;
}

}  // namespace

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
float *g_scratch[kMaxScratchDevices] = {};
}  // namespace

void attention_scratch_setup(int hip_device)
{
    if (hip_device < 0 || hip_device >= kMaxScratchDevices)
        throw HipError("attention scratch: device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[hip_device]) return;
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
        throw HipError(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch[hip_device] = static_cast<float *>(ptr);
}

float *attention_scratch(int hip_device)
{
    if (hip_device < 0 || hip_device >= kMaxScratchDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return g_scratch[hip_device];
}

size_t attention_ws_bytes(const Attn &a)
{
    if (use_exact_tiled(a)) return a.seq_q <= 4 ? attention_exact_decode_ws_bytes(a) : 0;
    if (use_rowwise(a)) return 0;
    uint32_t qb, splits, kps;
    plan(a, qb, splits, kps);
    if (use_prefill(a)) {
        // the split K / V^T blocks of the bf16 prefill kernel
        const uint64_t nkb = (a.seq_k + XK - 1) / XK;
        const uint64_t blk = a.head_dim == 128 ? SplitBlk<128>::kBytes : SplitBlk<64>::kBytes;
        return static_cast<size_t>(static_cast<uint64_t>(a.batch) * a.heads * nkb * blk);
    }
    if (splits <= 1) return 0;
    const uint64_t rows = static_cast<uint64_t>(a.batch) * a.heads * a.seq_q;
    return static_cast<size_t>(splits) * rows * (a.head_dim + 2) * sizeof(float);
}

void attention(hipStream_t s, const Attn &a, float *ws)
{
    if (use_exact_tiled(a)) {
        const bool decode = a.seq_q <= 4;
        if (decode) attention_exact_decode(s, a, ws);
        else attention_exact_prefill(s, a);
        return;
    }
    if (use_rowwise(a)) {
        const uint64_t rows = static_cast<uint64_t>(a.batch) * a.heads * a.seq_q;
        for (uint64_t r0 = 0; r0 < rows; r0 += 0x7fffffffull) {
            const uint32_t n = static_cast<uint32_t>(std::min<uint64_t>(rows - r0, 0x7fffffffull));
            attn_rowwise_kernel<<<n, kThreads, 0, s>>>(a, r0);
        }
        return;
    }
    uint32_t qb, splits, kps;
    plan(a, qb, splits, kps);
    const uint32_t D = a.head_dim;
    const size_t lds = (static_cast<size_t>(D) * BKEY * 2 + BQ * D + 4 * QW * BKEY) * sizeof(float);
    const uint64_t rows = static_cast<uint64_t>(a.batch) * a.heads * a.seq_q;
    float *ws_acc = ws;
    float *ws_ml = ws ? ws + static_cast<uint64_t>(splits) * rows * D : nullptr;
    dim3 grid(qb, a.batch * a.heads, splits);
    if (use_prefill(a)) {
        // ws holds attention_ws_bytes(a): the split K / V^T blocks.
        int8_t *split = reinterpret_cast<int8_t *>(ws);
        const uint32_t nqb = qb;
        const uint32_t nkb = (a.seq_k + XK - 1) / XK;
        const dim3 sgrid(nkb, a.batch * a.heads);
        if (a.causal) grid.x = (nqb + 1) / 2;
        static std::atomic<bool> lds_optin{false};  // launches may come from several host threads
        if (!lds_optin)
            lds_optin = hipFuncSetAttribute(reinterpret_cast<const void *>(attn_prefill_kernel<128>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize,
                                            static_cast<int>(SplitBlk<128>::kLds)) == hipSuccess &&
                        hipFuncSetAttribute(reinterpret_cast<const void *>(attn_prefill_kernel<64>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize,
                                            static_cast<int>(SplitBlk<64>::kLds)) == hipSuccess;
        if (D == 128) {
            attn_split_kv<128><<<sgrid, 256, 0, s>>>(a, nkb, split);
            attn_prefill_kernel<128><<<grid, PThreads, SplitBlk<128>::kLds, s>>>(a, nqb, nkb, split);
        } else {
            attn_split_kv<64><<<sgrid, 256, 0, s>>>(a, nkb, split);
            attn_prefill_kernel<64><<<grid, PThreads, SplitBlk<64>::kLds, s>>>(a, nqb, nkb, split);
        }
        return;
    }
    if (use_decode(a)) {
        const int qn = a.seq_q == 1 ? 1 : a.seq_q == 2 ? 2 : 4;
        const int v4 = static_cast<int>(D / 32);
        decode_launch(qn, v4, grid, s, a, kps, splits, ws_acc, ws_ml);
    } else {
        // Above 64 KiB of dynamic LDS the kernel must opt in (CDNA4 has 160 KiB).
        static thread_local size_t lds_optin = 0;
        if (lds > 65536 && lds > lds_optin) {
            if (hipFuncSetAttribute(reinterpret_cast<const void *>(attn_kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                    static_cast<int>(lds)) == hipSuccess)
                lds_optin = lds;
        }
        attn_kernel<<<grid, kThreads, lds, s>>>(a, kps, splits, ws_acc, ws_ml);
    }
    if (splits > 1) {
        const uint64_t total = rows * D;
        attn_merge<<<dim3(static_cast<uint32_t>((total + kThreads - 1) / kThreads)), kThreads, 0, s>>>(
            a, splits, rows, ws_acc, ws_ml);
    }
}

}  // namespace k
}  // namespace vnpu
