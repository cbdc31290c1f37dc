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
#include "device_math.hpp"

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

// Merge split partials: O = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s.
__global__ __launch_bounds__(kThreads) void attn_merge(Attn a, uint32_t splits, uint64_t rows,
                                                       const float *ws_acc, const float *ws_ml)
{
    const uint32_t D = a.head_dim;
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (idx >= rows * D) return;
    const uint64_t row = idx / D;
    const uint32_t d = static_cast<uint32_t>(idx % D);
    float M = -__builtin_inff();
    for (uint32_t s = 0; s < splits; ++s) M = fmaxf(M, ws_ml[(s * rows + row) * 2]);
    float num = 0.0f, den = 0.0f;
    if (isfinite(M)) {
        for (uint32_t s = 0; s < splits; ++s) {
            const float ms = ws_ml[(s * rows + row) * 2];
            if (!isfinite(ms)) continue;
            const float w = dev::fast_expf(ms - M);
            num = fmaf(w, ws_acc[(s * rows + row) * D + d], num);
            den = fmaf(w, ws_ml[(s * rows + row) * 2 + 1], den);
        }
    }
    a.O[row * D + d] = den > 0.0f ? num / den : 0.0f;
}

void plan(const Attn &a, uint32_t &qblocks, uint32_t &splits, uint32_t &kps)
{
    qblocks = (a.seq_q + BQ - 1) / BQ;
    const uint64_t tiles = static_cast<uint64_t>(qblocks) * a.batch * a.heads;
    splits = 1;
    const uint32_t kblocks = (a.seq_k + BKEY - 1) / BKEY;
    while (tiles * splits < 2048 && splits * 2 <= kblocks && kblocks / (splits * 2) >= 2) splits *= 2;
    kps = ((kblocks + splits - 1) / splits) * BKEY;
    splits = (a.seq_k + kps - 1) / kps;
}

}  // namespace

size_t attention_ws_bytes(const Attn &a)
{
    uint32_t qb, splits, kps;
    plan(a, qb, splits, kps);
    if (splits <= 1) return 0;
    const uint64_t rows = static_cast<uint64_t>(a.batch) * a.heads * a.seq_q;
    return static_cast<size_t>(splits) * rows * (a.head_dim + 2) * sizeof(float);
}

void attention(hipStream_t s, const Attn &a, float *ws)
{
    uint32_t qb, splits, kps;
    plan(a, qb, splits, kps);
    const uint32_t D = a.head_dim;
    const size_t lds = (static_cast<size_t>(D) * BKEY * 2 + BQ * D + 4 * QW * BKEY) * sizeof(float);
    const uint64_t rows = static_cast<uint64_t>(a.batch) * a.heads * a.seq_q;
    float *ws_acc = ws;
    float *ws_ml = ws ? ws + static_cast<uint64_t>(splits) * rows * D : nullptr;
    dim3 grid(qb, a.batch * a.heads, splits);
    // Above 64 KiB of dynamic LDS the kernel must opt in (CDNA4 has 160 KiB).
    static thread_local size_t lds_optin = 0;
    if (lds > 65536 && lds > lds_optin) {
        if (hipFuncSetAttribute(reinterpret_cast<const void *>(attn_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(lds)) == hipSuccess)
            lds_optin = lds;
    }
    attn_kernel<<<grid, kThreads, lds, s>>>(a, kps, splits, ws_acc, ws_ml);
    if (splits > 1) {
        const uint64_t total = rows * D;
        attn_merge<<<dim3(static_cast<uint32_t>((total + kThreads - 1) / kThreads)), kThreads, 0, s>>>(
            a, splits, rows, ws_acc, ws_ml);
    }
}

}  // namespace k
}  // namespace vnpu
