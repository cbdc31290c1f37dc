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

#include <algorithm>

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
            kr[t] = Kh[static_cast<uint64_t>(key) * D4 + r + 8 * t];
            vr[t] = Vh[static_cast<uint64_t>(key) * D4 + r + 8 * t];
        }
    };
    float4 kc[V4], vc[V4], kn[V4], vn[V4];
    if (nsteps) load(0, kc, vc);
    for (uint32_t step = 0; step < nsteps; ++step) {
        if (step + 1 < nsteps) load(step + 1, kn, vn);
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
                const float mn = fmaxf(m[i], s);
                const float al = (m[i] == -__builtin_inff()) ? 0.0f : dev::fast_expf(m[i] - mn);
                const float p = dev::fast_expf(s - mn);
                l[i] = fmaf(l[i], al, p);
#pragma unroll
                for (int t = 0; t < V4; ++t) {
                    acc[i][t].x = fmaf(p, vc[t].x, acc[i][t].x * al);
                    acc[i][t].y = fmaf(p, vc[t].y, acc[i][t].y * al);
                    acc[i][t].z = fmaf(p, vc[t].z, acc[i][t].z * al);
                    acc[i][t].w = fmaf(p, vc[t].w, acc[i][t].w * al);
                }
                m[i] = mn;
            }
        }
#pragma unroll
        for (int t = 0; t < V4; ++t) {
            kc[t] = kn[t];
            vc[t] = vn[t];
        }
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
// Prefill kernel on the f32 matrix cores (head_dim 64 or 128, seq_q > 4).
//
// A workgroup of 8 waves owns 128 queries of one (batch, head); wave w owns
// queries q0 + 16w .. +15 (two waves per SIMD).  Keys stream through LDS in
// blocks of 32, double buffered and filled by 16-byte DMA of whole rows: V as
// [key][d], K as [key][d] with 16-byte chunk c of key k at slot c ^ k (mod the
// chunks per row).  Per block each wave runs v_mfma_f32_16x16x4_f32:
//   S^T (16 keys x 16 queries, two tiles) = K . Q^T   (Q^T in VGPRs)
//   O^T (D x 16 queries)                += V^T . P^T
// Index maps chosen so every lane's operands are contiguous (one
// ds_read_b128 feeds four MFMAs):
//   * QK step st of lane group g = l/16 sums d = (D/4)g + st, so a lane reads
//     its key's K row in 16-byte chunks (the swizzle keeps the 16 keys of a
//     quarter wave in distinct banks) and holds Q[q][(D/4)g .. +D/4];
//   * O^T tile dt, row i stands for d = 64(dt/4) + 4i + dt%4, so one chunk of
//     a V row feeds four tiles;
//   * the accumulator layout puts query l%16 and keys 4g + q of a tile in
//     lane l, so a query's block max and sum combine four lanes (l^16, l^32),
//     and the P^T operand of PV step s of tile t is the lane's own score
//     register s when that product's key order is 16t + 4g + s.
// Online softmax as in the reference (a query whose block is fully masked
// skips the block), with the reference's fast_expf.  Keys past the range are
// clamped to a valid row and masked in the scores.  O leaves through LDS so
// every global row write is coalesced.
// ---------------------------------------------------------------------------
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int PQ = 128;          // queries per workgroup
constexpr int PK = 32;           // keys per block
constexpr int PThreads = 512;    // 8 waves

// 16-byte-per-lane global->LDS copy (lane l writes lds_dst + 16 l bytes).
// Written as asm on purpose: for the builtin form the compiler cannot tell the
// in-flight copy of the next key block from the buffer being read, and waits
// vmcnt(0) before the first ds_read of every block, which serialises the copy
// with the compute.  The kernel's own vmcnt(0) + barrier at the top of each
// key block is what orders the copy before its readers.
__device__ __forceinline__ void lds_dma16(const void *src, float *lds_dst)
{
    const uint32_t lds = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) float *)(lds_dst)));
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(src), "s"(lds)
                 : "memory", "m0");
}

template <int D>
struct PrefillLds {
    static constexpr int kK = PK * D;            // floats
    static constexpr int kBuf = 2 * PK * D;      // K + V
    static constexpr size_t kBytes = static_cast<size_t>(2 * kBuf) * 4;
    static_assert(8 * 16 * D <= 2 * kBuf, "output staging fits in the key buffers");
};

// e^x through the hardware exp2 (v_exp_f32).  The prefill kernel is matrix-
// bound and this is its softmax's cost: the reference's degree-5 polynomial
// (dev::fast_expf) spends ~10 VALU ops per weight.  The two differ by at most
// ~1.5e-4 relative (the polynomial's own truncation error), far inside the
// attention bar of 2e-3; the decode kernel keeps the polynomial.
__device__ __forceinline__ float fast_exp_hw(float x)
{
    return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// One block of PQ queries starting at q0, for (batch, head) bh.
template <int D>
__device__ __forceinline__ void prefill_block(const Attn &a, uint32_t q0, uint64_t bh, float *lds)
{
    using L = PrefillLds<D>;
    constexpr int NS = D / 4;          // QK MFMA steps per tile (4 d each)
    constexpr int NCH = D / 4;         // 16-byte chunks per row
    constexpr int DT = D / 16;         // 16-wide d tiles of O^T
    constexpr int HI = DT / 4;         // V chunks read per key

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, qc = lane & 15;
    const uint32_t sq = a.seq_q, sk = a.seq_k;
    const uint32_t off = sk > sq ? sk - sq : 0;
    const float *Kh = a.K + bh * sk * D;
    const float *Vh = a.V + bh * sk * D;
    const float *Mh = a.mask ? a.mask + bh * sq * sk : nullptr;
    const uint32_t qw = q0 + wave * 16;                      // this wave's first query
    const uint32_t myq = qw + qc;                            // this lane's query

    uint32_t kend = sk;
    if (a.causal) kend = min(sk, min(q0 + PQ, sq) - 1 + off + 1);
    const uint32_t nblk = (kend + PK - 1) / PK;
    const uint32_t wave_kend = a.causal ? min(kend, min(qw + 16, sq) - 1 + off + 1) : kend;

    // Q^T operand: lane (query qc, group g) holds Q[myq][NS*g .. NS*g + NS).
    float qf[NS];
    {
        const float4 *qrow = reinterpret_cast<const float4 *>(a.Q + (bh * sq + min(myq, sq - 1)) * D + NS * g);
#pragma unroll
        for (int u = 0; u < NS / 4; ++u) {
            const float4 v = qrow[u];
            qf[4 * u] = v.x;
            qf[4 * u + 1] = v.y;
            qf[4 * u + 2] = v.z;
            qf[4 * u + 3] = v.w;
        }
    }

    // DMA of key block kb into buffer buf: K and V, 16-byte chunks, 64 per
    // instruction, PK*NCH/64 instructions each, spread over the 8 waves.
    auto issue = [&](uint32_t kb, int buf) {
        float *ks = lds + buf * L::kBuf;
        float *vs = ks + L::kK;
        constexpr int kInstr = PK * NCH / 64;
#pragma unroll
        for (int i = 0; i < kInstr / 8; ++i) {
            const int ins = wave * (kInstr / 8) + i;
            const uint32_t f = ins * 64 + lane;              // chunk slot in the block
            const uint32_t k = f / NCH, slot = f % NCH;
            const uint32_t key = min(kb * PK + k, kend - 1);
            const uint32_t c = slot ^ (k & (NCH - 1));       // K chunk stored in this slot
            lds_dma16(Kh + static_cast<uint64_t>(key) * D + 4 * c, ks + ins * 256);
            lds_dma16(Vh + static_cast<uint64_t>(key) * D + 4 * slot, vs + ins * 256);
        }
    };
    if (nblk) issue(0, 0);

    v4f o[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] = (v4f){0.f, 0.f, 0.f, 0.f};
    float m = -__builtin_inff(), l = 0.0f;

    for (uint32_t kb = 0; kb < nblk; ++kb) {
        const int buf = kb & 1;
        __builtin_amdgcn_s_waitcnt(0xF70);   // vmcnt(0): this wave's DMA of block kb
        __syncthreads();                     // block kb landed everywhere; block kb-1's buffer free
        if (kb + 1 < nblk) issue(kb + 1, buf ^ 1);
        if (kb * PK >= wave_kend) continue;  // wave-uniform: past this wave's causal limit
        const float *ks = lds + buf * L::kBuf;
        const float *vs = ks + L::kK;

        // S^T tiles (keys 16t + row) = K . Q^T
        v4f sc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int kk = 16 * t + qc;
            const float *krow = ks + kk * D;
            sc[t] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < NS / 4; ++u) {
                const int c = (NS / 4) * g + u;
                const float4 kv = *reinterpret_cast<const float4 *>(krow + 4 * (c ^ (kk & (NCH - 1))));
                sc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.x, qf[4 * u + 0], sc[t], 0, 0, 0);
                sc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.y, qf[4 * u + 1], sc[t], 0, 0, 0);
                sc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.z, qf[4 * u + 2], sc[t], 0, 0, 0);
                sc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.w, qf[4 * u + 3], sc[t], 0, 0, 0);
            }
        }
        // Scores of query myq for keys kb*32 + 16t + 4g + q.  A block whose
        // keys are all below every query's causal limit and kend (wave-
        // uniform) needs no masking.
        const bool interior = (kb + 1) * PK <= kend && qw + 15 < sq &&
                              (!a.causal || (kb + 1) * PK - 1 <= qw + off);
        float bmax = -__builtin_inff();
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t key = kb * PK + 16 * t + 4 * g + r;
                float v = sc[t][r] * a.scale;
                if (Mh) v += Mh[static_cast<uint64_t>(min(myq, sq - 1)) * sk + min(key, sk - 1)];
                if (!interior) {
                    const bool dead = key >= kend || myq >= sq || (a.causal && key > myq + off);
                    v = dead ? -__builtin_inff() : v;
                }
                sc[t][r] = v;
                bmax = fmaxf(bmax, v);
            }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 16, 64));
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
        const bool live = bmax != -__builtin_inff();      // else the block is skipped for this query
        const float mn = live ? fmaxf(m, bmax) : m;
        const float alpha = (!live || m == -__builtin_inff()) ? (live ? 0.0f : 1.0f) : fast_exp_hw(m - mn);
        float psum = 0.0f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = (sc[t][r] == -__builtin_inff()) ? 0.0f : fast_exp_hw(sc[t][r] - mn);
                sc[t][r] = p;
                psum += p;
            }
        psum += __shfl_xor(psum, 16, 64);
        psum += __shfl_xor(psum, 32, 64);
        m = mn;
        l = l * alpha + psum;
#pragma unroll
        for (int t = 0; t < DT; ++t) o[t] *= alpha;
        // O^T += V^T . P^T, key 16t + 4g + st: P^T is the lane's register st;
        // tile dt row qc is d = 64(dt/4) + 4qc + dt%4.
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const float *vrow = vs + (16 * t + 4 * g + st) * D + 4 * qc;
#pragma unroll
                for (int hi = 0; hi < HI; ++hi) {
                    const float4 vv = *reinterpret_cast<const float4 *>(vrow + 64 * hi);
                    o[4 * hi + 0] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.x, sc[t][st], o[4 * hi + 0], 0, 0, 0);
                    o[4 * hi + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.y, sc[t][st], o[4 * hi + 1], 0, 0, 0);
                    o[4 * hi + 2] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.z, sc[t][st], o[4 * hi + 2], 0, 0, 0);
                    o[4 * hi + 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.w, sc[t][st], o[4 * hi + 3], 0, 0, 0);
                }
            }
    }

    // O = O^T / l through LDS (the key buffers): this wave's 16 x D tile; the
    // lane holds query qc, d = 64(dt/4) + 16g + 4r + dt%4 (register r of tile
    // dt); column c of row q stored at c ^ q (distinct banks per register).
    __syncthreads();
    float *ot = lds + wave * 16 * D;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            ot[qc * D + ((64 * (dt >> 2) + 16 * g + 4 * r + (dt & 3)) ^ qc)] = o[dt][r] * inv;
    __syncthreads();
    for (int i = lane; i < 16 * D; i += 64) {
        const uint32_t row = i / D, col = i % D;
        const uint32_t q = qw + row;
        if (q < sq) a.O[(bh * sq + q) * D + col] = ot[row * D + (col ^ row)];
    }
}

// Causal blocks cost in proportion to their position, so with nqb blocks per
// head the grid has ceil(nqb/2) workgroups per head and workgroup x takes
// block nqb-1-x and then block x: every workgroup does the same work (the
// grid otherwise runs as long as its last, heaviest block).  Without a
// causal mask every block costs the same and each workgroup takes one.
template <int D>
__global__ __launch_bounds__(PThreads) void attn_prefill_kernel(Attn a, uint32_t nqb)
{
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const uint64_t bh = blockIdx.y;
    const uint32_t heavy = nqb - 1 - blockIdx.x;
    prefill_block<D>(a, heavy * PQ, bh, lds);
    if (gridDim.x < nqb && blockIdx.x != heavy) {
        __syncthreads();  // the output staging of the first block is read out
        prefill_block<D>(a, blockIdx.x * PQ, bh, lds);
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
    if (use_prefill(a)) {
        qblocks = (a.seq_q + PQ - 1) / PQ;
        splits = 1;
        kps = a.seq_k;
        return;
    }
    if (use_decode(a)) {
        // One workgroup per (batch, head) and key range: enough ranges for
        // ~2048 workgroups, each at least 256 keys (8 per stream).
        qblocks = 1;
        const uint64_t bh = static_cast<uint64_t>(a.batch) * a.heads;
        const uint32_t max_splits = std::max<uint32_t>(1, (a.seq_k + 255) / 256);
        splits = static_cast<uint32_t>(std::min<uint64_t>(max_splits, std::max<uint64_t>(1, (2048 + bh - 1) / bh)));
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
    if (use_prefill(a)) {
        const uint32_t nqb = qb;
        if (a.causal) grid.x = (nqb + 1) / 2;
        if (D == 128)
            attn_prefill_kernel<128><<<grid, PThreads, PrefillLds<128>::kBytes, s>>>(a, nqb);
        else
            attn_prefill_kernel<64><<<grid, PThreads, PrefillLds<64>::kBytes, s>>>(a, nqb);
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
