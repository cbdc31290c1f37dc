// attn_exact.hip - ATTENTION_F32 prefill (seq_q > 4) in the reference's
// order of roundings, on the fp32 matrix cores.
//
// The reference's attention_range (src/kernels/llm.cpp:442-546) computes,
// per query row and 64-key block:
//   s_j = dot_avx2(q, k_j) * scale (+ mask)   eight FMA chains over
//         d = 8i + c, i ascending, then hsum256 ((c0+c4)+(c1+c5)) +
//         ((c2+c6)+(c3+c7)) (llm.cpp:332-343);
//   a block whose max is not finite is skipped; new_m = max(m, block max),
//   alpha = fast_expf(m - new_m), p_j = fast_expf(s_j - new_m), the weight
//   sum in key order, l = l * alpha + sum;
//   acc = acc * alpha, then acc = fma(v_j, p_j, acc) in key order for every
//   p_j != 0 (axpy_avx2, llm.cpp:345-355); out = acc * (1 / l).
//
// gfx950's fp32 MFMA with K = 1 (v_mfma_f32_32x32x1_2b_f32) computes
// D = A * B + C with one rounding, the same result as fmaf for every input
// (normal, denormal, infinite, NaN; checked against v_fma_f32 on MI355X over
// 8.4 million outputs per operand class, chains included).  Both sequential
// chains of the reference therefore run on the matrix core, one rank-1 step
// per instruction, in the reference's order:
//   scores   S^T[key][q] over a 32-key x 32-row tile: block 0 of the
//            instruction is chain c, block 1 chain c + 4, step i of both
//            chains per instruction (A = K, B = Q); the lane that holds
//            (key, row) in block 0 holds it in block 1, so hsum256's
//            pairing is in-lane;
//   output   O^T[d][q] += V^T[d][key] * P[key][q], one key per instruction,
//            keys ascending (A = V, B = P), 64 head elements per instruction.
// Every lane owns one query row in both products (column = lane % 32): the
// softmax state, alpha and the row's weights stay in the lane.  The weights
// of a key sit in one half of the wave; one exchange with the other half
// gives every lane its row's 64 weights, in key order for the sum and as the
// B operand of each key's instruction.
//
// The one difference from the reference is the p_j == 0 skip: the
// instruction adds v * 0 instead of skipping, which equals skipping unless
// acc is -0 (it becomes +0) or v is infinite or NaN (the sum becomes NaN).
// A sign-of-zero difference either vanishes at the next nonzero product or
// leaves a zero output element; a non-finite v leaves a NaN.  So every
// output element that is neither NaN nor zero is the reference's bit for
// bit, and a wave that finds a NaN, or a zero in a row with l > 0, among its
// outputs recomputes its rows in the reference's order on the vector ALUs.
//
// Structure: one workgroup of four waves per (batch, head) and 128 query
// rows, wave w owning rows 32w .. 32w + 31; the 64-key K and V tiles are
// copied from HBM straight into LDS (double-buffered, the next block's copy
// in flight during this block's work); the workgroups of the longest causal
// rows are dispatched first.
#include "kernels.hpp"

#include <algorithm>
#include <atomic>
#include "device_math.hpp"
#include "lds_dma.hpp"
#include "vnpu_internal.hpp"

namespace vnpu {
namespace k {
namespace {

typedef float f32x32 __attribute__((ext_vector_type(32)));

constexpr int XT = 256;          // threads per workgroup (four waves)
constexpr int XQW = 32;          // query rows per wave
constexpr int XQ = 4 * XQW;      // query rows per workgroup
constexpr int XB = 64;           // keys per block (the reference's BK)

template <int D>
struct XL {
    static constexpr int KCH = D / 4 + 1;              // 16-byte slots per K row (one pad slot)
    static constexpr int KP = 4 * KCH;                 // K row pitch (floats): conflict-free 16-byte row reads
    static constexpr int KTILE = XB * KP;              // floats per K tile
    static constexpr int VTILE = XB * D;               // floats per V tile
    static constexpr int KI = XB * KCH / 64;           // wave copies (64 slots each) per K tile
    static constexpr int VI = XB * D / 4 / 64;         // per V tile
    static constexpr size_t kLds = static_cast<size_t>(2 * KTILE + 2 * VTILE) * sizeof(float);
    static_assert((XB * KCH) % 64 == 0, "K tile copies are whole waves");
};

__device__ __forceinline__ f32x32 mfma1(float a, float b, f32x32 c)
{
    return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c, 0, 0, 0);
}

// Both halves' values of a lane's column: lo[l] = v of lane l % 32, hi[l] =
// v of lane 32 + l % 32 (one v_permlane32_swap_b32).
__device__ __forceinline__ void halves(float v, float &lo, float &hi)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    lo = __uint_as_float(r[0]);
    hi = __uint_as_float(r[1]);
}

// The weights and the output chain of one 64-key block for the lane's row
// (keys 32t + 8g + 4h + j of S[t][4g + j] in half h): per group of eight keys,
// the weights of both halves, the weight sum in key order, then one
// instruction per key and 64 head elements, keys ascending.  FULL: every key
// of the block is seen by some row of the wave (no per-key test).  Returns
// the block's weight sum.  Every S - nm is <= 0 or NaN (nm is the max).
template <int D, bool FULL>
__device__ __forceinline__ float weights_output(f32x32 (&oacc)[D / 64], const float (&S)[2][16], float nm,
                                                bool live, uint32_t kc_w, int lane, const float *Vb)
{
#pragma clang fp contract(off)
    float psum = 0.0f;
    float lo[4], hi[4], nlo[4], nhi[4];
    auto weights = [&](int t, int g, float (&wl)[4], float (&wh)[4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float e = dev::fast_expf_nonpos(S[t][4 * g + j] - nm);
            halves(live ? e : 0.0f, wl[j], wh[j]);
        }
    };
    weights(0, 0, nlo, nhi);
#pragma unroll
    for (int q = 0; q < 8; ++q) {   // group q: keys 8q .. 8q + 7
        // One group's V operands in registers at a time (without the fence
        // the scheduler hoists every V read of the block); the next group's
        // weights are computed while this group's instructions run.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            lo[j] = nlo[j];
            hi[j] = nhi[j];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) psum = psum + lo[j];
#pragma unroll
        for (int j = 0; j < 4; ++j) psum = psum + hi[j];
        if (q < 7) weights((q + 1) / 4, (q + 1) % 4, nlo, nhi);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int kk = 8 * q + j;
            if (FULL || kk < static_cast<int>(kc_w)) {   // uniform
#pragma unroll
                for (int mm = 0; mm < D / 64; ++mm)
                    oacc[mm] = mfma1(Vb[kk * D + 64 * mm + lane], j < 4 ? lo[j] : hi[j - 4], oacc[mm]);
            }
        }
    }
    return psum;
}

// One query row in the reference's order on the vector ALUs, by one wave:
// lane j scores key k0 + j of each block, lane e owns head elements e,
// e + 64, ... of the output row.
template <int D>
__device__ __noinline__ void exact_row_wave(Attn a, uint64_t bh, uint32_t qi, int lane)
{
#pragma clang fp contract(off)
    constexpr int E = D / 64;
    const uint32_t sq = a.seq_q, sk = a.seq_k;
    const uint32_t off = sk > sq ? sk - sq : 0;
    const uint64_t row = bh * sq + qi;
    const float *q = a.Q + row * D;
    const float *Kh = a.K + bh * sk * D;
    const float *Vh = a.V + bh * sk * D;
    const float *Mr = a.mask ? a.mask + row * sk : nullptr;
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = 0.0f;
    float m = -__builtin_inff(), l = 0.0f;
    const uint32_t kend = a.causal ? min(sk, qi + off + 1) : sk;
    for (uint32_t k0 = 0; k0 < kend; k0 += XB) {
        const uint32_t kc = min(static_cast<uint32_t>(XB), kend - k0);
        float sc = -__builtin_inff();
        if (lane < static_cast<int>(kc)) {
            sc = dev::dot_ref(q, Kh + static_cast<uint64_t>(k0 + lane) * D, D) * a.scale;
            if (Mr) sc = sc + Mr[k0 + lane];
        }
        const float bmax = dev::wave_max(sc);
        if (!isfinite(bmax)) continue;   // uniform
        const float nm = m < bmax ? bmax : m;
        const float alpha = dev::fast_expf_unfused(m - nm);
        const float p = dev::fast_expf_unfused(sc - nm);
        float psum = 0.0f;
        for (uint32_t j = 0; j < kc; ++j)
            psum = psum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), static_cast<int>(j)));
        l = l * alpha + psum;
#pragma unroll
        for (int e = 0; e < E; ++e) acc[e] = acc[e] * alpha;
        for (uint32_t j = 0; j < kc; ++j) {
            const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), static_cast<int>(j)));
            if (pj == 0.0f) continue;
            const float *vr = Vh + static_cast<uint64_t>(k0 + j) * D + lane;
#pragma unroll
            for (int e = 0; e < E; ++e) acc[e] = fmaf(vr[64 * e], pj, acc[e]);
        }
        m = nm;
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) a.O[row * D + lane + 64 * e] = acc[e] * inv;
}

template <int D>
__global__ __launch_bounds__(XT) __attribute__((amdgpu_waves_per_eu(1, 1))) void attn_exact_mfma_kernel(Attn a)
{
#pragma clang fp contract(off)
    using L = XL<D>;
    constexpr int NI = D / 8;    // steps of each dot chain
    constexpr int NM = D / 64;   // output instructions per key
    extern __shared__ float4 sm4[];
    float *Kt = reinterpret_cast<float *>(sm4);   // [2][64][KP]
    float *Vt = Kt + 2 * L::KTILE;               // [2][64][D]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, c32 = lane & 31;
    const uint64_t bh = blockIdx.x;
    const uint32_t sq = a.seq_q, sk = a.seq_k;
    const uint32_t off = sk > sq ? sk - sq : 0;
    const uint32_t q0 = (gridDim.y - 1 - blockIdx.y) * XQ;
    const uint32_t nq = min(static_cast<uint32_t>(XQ), sq - q0);
    const uint32_t qw0 = q0 + wave * XQW;       // the wave's first row
    const uint32_t qi = qw0 + c32;              // the lane's row
    const bool qvalid = qi < sq;
    const float *Kh = a.K + bh * sk * D;
    const float *Vh = a.V + bh * sk * D;
    const float *Mh = a.mask ? a.mask + bh * sq * sk : nullptr;

    const uint32_t kend = a.causal ? min(sk, q0 + nq - 1 + off + 1) : sk;   // keys of any row here
    uint32_t kend_w = 0;                                                    // keys of any row of the wave
    if (qw0 < sq) kend_w = a.causal ? min(sk, min(qw0 + XQW - 1, sq - 1) + off + 1) : sk;
    const uint32_t nblk = (kend + XB - 1) / XB;

    auto copy = [&](uint32_t b) {
        int8_t *kd = reinterpret_cast<int8_t *>(Kt + (b & 1) * L::KTILE);
        int8_t *vd = reinterpret_cast<int8_t *>(Vt + (b & 1) * L::VTILE);
        for (int i = wave; i < L::KI; i += 4) {
            const uint32_t sl = static_cast<uint32_t>(i) * 64 + lane;
            const uint32_t r = sl / L::KCH, c = sl % L::KCH;
            const uint32_t key = min(b * XB + r, kend - 1);
            lds::dma16(Kh + static_cast<uint64_t>(key) * D + (c < D / 4 ? 4 * c : 0), kd + i * 1024);
        }
        for (int i = wave; i < L::VI; i += 4) {
            const uint32_t sl = static_cast<uint32_t>(i) * 64 + lane;
            const uint32_t key = min(b * XB + sl / (D / 4), kend - 1);
            lds::dma16(Vh + static_cast<uint64_t>(key) * D + 4 * (sl % (D / 4)), vd + i * 1024);
        }
    };
    if (nblk) copy(0);

    // B operands of the score products: lane (h, c32) holds the row's
    // elements 8i + 4h .. 8i + 4h + 3 (chains 4h .. 4h + 3 at step i).
    float4 qop[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i)
        qop[i] = qvalid ? *reinterpret_cast<const float4 *>(a.Q + (bh * sq + qi) * D + 8 * i + 4 * h)
                        : make_float4(0.f, 0.f, 0.f, 0.f);

    float m = -__builtin_inff(), l = 0.0f;
    f32x32 oacc[NM];
#pragma unroll
    for (int mm = 0; mm < NM; ++mm)
#pragma unroll
        for (int r = 0; r < 32; ++r) oacc[mm][r] = 0.0f;

    for (uint32_t b = 0; b < nblk; ++b) {
        lds::wait_vmcnt<0>();
        lds::block_barrier();                  // block b's tiles are in; block b-1's buffers are free
        if (b + 1 < nblk) copy(b + 1);
        const uint32_t k0 = b * XB;
        if (k0 >= kend_w) continue;           // no row of this wave sees these keys (uniform)
        const uint32_t kc_w = min(static_cast<uint32_t>(XB), kend_w - k0);
        const float *Kb = Kt + (b & 1) * L::KTILE;
        const float *Vb = Vt + (b & 1) * L::VTILE;

        // Scores: S[t][r] is (key k0 + 32t + 8(r/4) + 4h + r%4, row qi).  Both
        // 32-key tiles are computed (a tile no row sees is masked below), so
        // the two tiles' products and sums share one scheduling region.
        float S[2][16];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            // Two passes of two chain pairs each: (0,4) and (1,5), then (2,6)
            // and (3,7); hsum256's ((c0+c4) + (c1+c5)) + ((c2+c6) + (c3+c7)).
            const float *kr = Kb + (32 * t + c32) * L::KP + 4 * h;
            float s01[16];
            f32x32 acc0, acc1;
#pragma unroll
            for (int r = 0; r < 32; ++r) acc0[r] = acc1[r] = 0.0f;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const float2 kv = *reinterpret_cast<const float2 *>(kr + 8 * i);
                acc0 = mfma1(kv.x, qop[i].x, acc0);
                acc1 = mfma1(kv.y, qop[i].y, acc1);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) s01[r] = (acc0[r] + acc0[r + 16]) + (acc1[r] + acc1[r + 16]);
#pragma unroll
            for (int r = 0; r < 32; ++r) acc0[r] = acc1[r] = 0.0f;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const float2 kv = *reinterpret_cast<const float2 *>(kr + 8 * i + 2);
                acc0 = mfma1(kv.x, qop[i].z, acc0);
                acc1 = mfma1(kv.y, qop[i].w, acc1);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r)
                S[t][r] = (s01[r] + ((acc0[r] + acc0[r + 16]) + (acc1[r] + acc1[r + 16]))) * a.scale;
        }
        // Every row of the wave sees every key of the block: no masking.
        const bool dense = qw0 + XQW <= sq && k0 + XB <= kend && (!a.causal || k0 + XB - 1 <= qw0 + off);
        if (!dense) {   // uniform
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t key = k0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
                    const bool valid = qvalid && key < kend && !(a.causal && key > qi + off);
                    S[t][r] = valid ? S[t][r] : -__builtin_inff();
                }
        }
        if (Mh) {   // the additive mask on the scores the row sees (uniform)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t key = k0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (qvalid && key < kend && !(a.causal && key > qi + off))
                        S[t][r] = S[t][r] + Mh[static_cast<uint64_t>(qi) * sk + key];
                }
        }

        // Softmax state of the lane's row (both halves hold the same).
        float bmax = -__builtin_inff();
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) bmax = fmaxf(bmax, S[t][r]);
        {
            float b0, b1;
            halves(bmax, b0, b1);
            bmax = fmaxf(b0, b1);
        }
        const bool live = isfinite(bmax);
        const float nm = m < bmax ? bmax : m;
        const float alpha = live ? dev::fast_expf_unfused(m - nm) : 1.0f;
        if (__ballot(alpha != 1.0f)) {   // acc * 1 is acc: skipped when no row's max moved
#pragma unroll
            for (int mm = 0; mm < NM; ++mm)
#pragma unroll
                for (int r = 0; r < 32; ++r) oacc[mm][r] = oacc[mm][r] * alpha;
        }

        // Keys in groups of eight (32t + 8g .. +7); keys no row of the wave
        // sees are skipped.
        const float psum = kc_w == XB ? weights_output<D, true>(oacc, S, nm, live, kc_w, lane, Vb)
                                      : weights_output<D, false>(oacc, S, nm, live, kc_w, lane, Vb);
        if (live) {
            l = l * alpha + psum;
            m = nm;
        }
    }

    // Output: oacc[mm][r] is element 64mm + 32(r/16) + 8((r%16)/4) + 4h + r%4 of row qi.
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    bool bad = false;
#pragma unroll
    for (int mm = 0; mm < NM; ++mm)
#pragma unroll
        for (int r = 0; r < 32; ++r) {
            const float o = oacc[mm][r] * inv;
            oacc[mm][r] = o;
            bad |= (o != o) || (o == 0.0f && l > 0.0f);
        }
    bad = bad && qvalid;
    if (__ballot(bad) == 0) {
        if (qvalid) {
            float *orow = a.O + (bh * sq + qi) * D + 4 * h;
#pragma unroll
            for (int mm = 0; mm < NM; ++mm)
#pragma unroll
                for (int g = 0; g < 8; ++g)
                    *reinterpret_cast<float4 *>(orow + 64 * mm + 32 * (g >> 2) + 8 * (g & 3)) =
                        make_float4(oacc[mm][4 * g], oacc[mm][4 * g + 1], oacc[mm][4 * g + 2], oacc[mm][4 * g + 3]);
        }
    } else {
        for (uint32_t j = 0; j < XQW && qw0 + j < sq; ++j) exact_row_wave<D>(a, bh, qw0 + j, lane);
    }
}

template <int D>
void launch(hipStream_t s, const Attn &a)
{
    using L = XL<D>;
    static std::atomic<bool> lds_optin{false};
    if (!lds_optin && L::kLds > 65536)
        lds_optin = hipFuncSetAttribute(reinterpret_cast<const void *>(attn_exact_mfma_kernel<D>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        static_cast<int>(L::kLds)) == hipSuccess;
    const dim3 grid(a.batch * a.heads, (a.seq_q + XQ - 1) / XQ);
    attn_exact_mfma_kernel<D><<<grid, XT, L::kLds, s>>>(a);
}

// ---------------------------------------------------------------------------
// Reference-order decode (seq_q <= 4).  In attention_range only the output
// chain is sequential over keys; the scores are independent per key and the
// chain is independent per head element.  So decode runs as two kernels:
//   attn_dec_scores  s[row][key] = dot_avx2(q_row, k_key) * scale, then -inf
//                    for a causally masked key or + mask, every key in
//                    parallel (one lane per key running its eight chains);
//   attn_dec_chain   one wave per (row, 64 head elements): per 64-key block
//                    the block max, m, alpha and the weights from the saved
//                    scores (every wave of a row derives the same ones), the
//                    weight sum and acc = fma(v_j, p_j, acc) in key order for
//                    p_j != 0, with the V slices and the scores of the next
//                    three blocks copied from HBM into LDS meanwhile.
// The scores live in a workspace of rows x pitch floats (pitch = seq_k
// rounded up to 64); calls whose scores exceed kDecScoreCap run over
// consecutive (batch, head) ranges.
// ---------------------------------------------------------------------------
constexpr int DTPW = 4;                     // 64-key K tiles per scores wave
constexpr int DNB = 4;                      // blocks in flight per chain wave
constexpr int DTV = XB * 64;                // floats per V tile (64 keys x 64 head elements)
constexpr int DOPS = 17;                    // copies per block: 16 of V, one of scores
constexpr size_t kDecLds = static_cast<size_t>(DNB) * (DTV + XB) * sizeof(float) + XB * sizeof(float);
constexpr uint64_t kDecScoreCap = 32ull << 20;

uint32_t dec_pitch(const Attn &a) { return (a.seq_k + XB - 1) / XB * XB; }

template <int D>
constexpr size_t dec_scores_lds() { return (static_cast<size_t>(XB) * XL<D>::KP + 4 * D) * sizeof(float); }

// Maximum over the wave's 64 lanes, in every lane (order-free: NaN operands
// are ignored as by fmaxf, and the sign of a zero maximum never matters).
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_f(float x)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), CTRL, ROWS, 0xf, false));
}

__device__ __forceinline__ float wave_max_dpp(float v)
{
    v = fmaxf(v, dpp_f<0xB1, 0xf>(v));    // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f<0x4E, 0xf>(v));    // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f<0x141, 0xf>(v));   // row_half_mirror
    v = fmaxf(v, dpp_f<0x140, 0xf>(v));   // row_mirror: every lane holds its row's max
    v = fmaxf(v, dpp_f<0x142, 0xa>(v));   // row_bcast15 into rows 1 and 3
    v = fmaxf(v, dpp_f<0x143, 0xc>(v));   // row_bcast31 into rows 2 and 3: lane 63 holds the max
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Scores: one wave per (batch, head) and DTPW tiles of 64 keys (four such
// workgroups per CU by LDS); the wave copies a tile's K rows into LDS (row
// pitch D + 4 floats: lane j's 16-byte reads of key j are conflict-free) and
// lane j runs key j's eight chains for every query row (the rows' elements
// as broadcast reads).
template <int D>
__global__ __launch_bounds__(64) void attn_dec_scores(Attn a, float *S, uint32_t pitch)
{
#pragma clang fp contract(off)
    using L = XL<D>;
    constexpr int NI = D / 8;
    extern __shared__ float4 sm4[];
    const int lane = threadIdx.x;
    float *Kt = reinterpret_cast<float *>(sm4);          // [64][KP]
    float *Qs = Kt + XB * L::KP;                         // [sq][D]
    const uint64_t bh = blockIdx.y;
    const uint32_t sq = a.seq_q, sk = a.seq_k;
    const uint32_t off = sk > sq ? sk - sq : 0;
    const float *Kh = a.K + bh * sk * D;
    for (uint32_t i = lane; i < sq * D; i += 64) Qs[i] = a.Q[bh * sq * D + i];
    __syncthreads();
    const uint32_t t0 = blockIdx.x * DTPW;
    for (uint32_t tt = 0; tt < DTPW; ++tt) {
        const uint32_t k0 = (t0 + tt) * XB;
        if (k0 >= sk) break;   // uniform over the wave; no barrier follows
        for (int i = 0; i < L::KCH; ++i) {
            const uint32_t sl = static_cast<uint32_t>(i) * 64 + lane;
            const uint32_t r = sl / L::KCH, c = sl % L::KCH;
            const uint32_t key = min(k0 + r, sk - 1);
            lds::dma16_nt(Kh + static_cast<uint64_t>(key) * D + (c < D / 4 ? 4 * c : 0),
                          reinterpret_cast<int8_t *>(Kt) + i * 1024);
        }
        lds::wait_vmcnt<0>();
        asm volatile("" ::: "memory");
        const uint32_t key = k0 + lane;
        const float *kr = Kt + lane * L::KP;
        for (uint32_t r = 0; r < sq; ++r) {
            const float *qr = Qs + r * D;
            float c8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const float4 ka = *reinterpret_cast<const float4 *>(kr + 8 * i);
                const float4 kb = *reinterpret_cast<const float4 *>(kr + 8 * i + 4);
                const float4 qa = *reinterpret_cast<const float4 *>(qr + 8 * i);
                const float4 qb = *reinterpret_cast<const float4 *>(qr + 8 * i + 4);
                c8[0] = fmaf(qa.x, ka.x, c8[0]);
                c8[1] = fmaf(qa.y, ka.y, c8[1]);
                c8[2] = fmaf(qa.z, ka.z, c8[2]);
                c8[3] = fmaf(qa.w, ka.w, c8[3]);
                c8[4] = fmaf(qb.x, kb.x, c8[4]);
                c8[5] = fmaf(qb.y, kb.y, c8[5]);
                c8[6] = fmaf(qb.z, kb.z, c8[6]);
                c8[7] = fmaf(qb.w, kb.w, c8[7]);
            }
            const float dot = ((c8[0] + c8[4]) + (c8[1] + c8[5])) + ((c8[2] + c8[6]) + (c8[3] + c8[7]));
            const uint64_t row = bh * sq + r;
            if (key < sk) {
                float sc = dot * a.scale;
                if (a.causal && key > r + off) sc = -__builtin_inff();
                else if (a.mask) sc = sc + a.mask[row * sk + key];
                S[row * pitch + key] = sc;
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the tile is read before the next copy
    }
}

// Output chain: one wave per (row, 64 head elements).
template <int D>
__global__ __launch_bounds__(64) void attn_dec_chain(Attn a, const float *S, uint32_t pitch)
{
#pragma clang fp contract(off)
    extern __shared__ float4 sm4[];
    float *Vt = reinterpret_cast<float *>(sm4);   // [DNB][64 keys][64]
    float *St = Vt + DNB * DTV;                   // [DNB][64] scores
    float *Pw = St + DNB * XB;                    // [64] weights of the current block
    const int lane = threadIdx.x;
    const uint64_t row = blockIdx.x;
    const uint32_t sq = a.seq_q, sk = a.seq_k;
    const uint32_t off = sk > sq ? sk - sq : 0;
    const uint64_t bh = row / sq;
    const uint32_t qi = static_cast<uint32_t>(row % sq);
    const uint32_t kend = a.causal ? min(sk, qi + off + 1) : sk;
    const uint32_t nblk = (kend + XB - 1) / XB;
    const float *Vh = a.V + bh * sk * D + blockIdx.y * 64;
    const float *Sr = S + row * pitch;

    // Block t's copies: 16 of four keys x 64 head elements each, then the
    // block's 64 scores by lanes 0-15 (the row pitch keeps them in the row).
    auto copy = [&](uint32_t t) {
        int8_t *vd = reinterpret_cast<int8_t *>(Vt + (t % DNB) * DTV);
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const uint32_t key = min(t * XB + 4 * u + (lane >> 4), kend - 1);
            lds::dma16_nt(Vh + static_cast<uint64_t>(key) * D + 4 * (lane & 15), vd + u * 1024);
        }
        if (lane < 16) lds::dma16(Sr + t * XB + 4 * lane, reinterpret_cast<int8_t *>(St + (t % DNB) * XB));
    };
    for (uint32_t t = 0; t < DNB - 1 && t < nblk; ++t) copy(t);

    float m = -__builtin_inff(), l = 0.0f, acc = 0.0f;
    for (uint32_t t = 0; t < nblk; ++t) {
        if (t + DNB - 1 < nblk) {
            copy(t + DNB - 1);
            lds::wait_vmcnt<DOPS * (DNB - 1)>();
        } else {
            lds::wait_vmcnt<0>();
        }
        asm volatile("" ::: "memory");
        const uint32_t k0 = t * XB, kc = min(static_cast<uint32_t>(XB), kend - k0);
        const float *vt = Vt + (t % DNB) * DTV + lane;
        const float sc = lane < static_cast<int>(kc) ? St[(t % DNB) * XB + lane] : -__builtin_inff();
        const float bmax = wave_max_dpp(sc);
        if (isfinite(bmax)) {   // uniform
            const float nm = m < bmax ? bmax : m;
            const float alpha = dev::fast_expf_unfused(m - nm);
            const float p = dev::fast_expf_unfused(sc - nm);   // 0 past kc
            Pw[lane] = p;
            const uint64_t nz = __ballot(p != 0.0f);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            float psum = 0.0f;
            acc = acc * alpha;
            if (kc == XB && nz == ~0ull) {
                // Every weight of a whole block is nonzero: the chains without
                // a test, every read of the block issued up front.
                float v[XB], pj[XB];
#pragma unroll
                for (int j = 0; j < XB; j += 4) {
                    const float4 w4 = *reinterpret_cast<const float4 *>(Pw + j);
                    pj[j] = w4.x; pj[j + 1] = w4.y; pj[j + 2] = w4.z; pj[j + 3] = w4.w;
                }
#pragma unroll
                for (int j = 0; j < XB; ++j) v[j] = vt[j * 64];
#pragma unroll
                for (int j = 0; j < XB; ++j) {
                    psum = psum + pj[j];
                    acc = fmaf(v[j], pj[j], acc);
                }
            } else {
                for (uint32_t j = 0; j < kc; j += 4) {
                    const float4 w4 = *reinterpret_cast<const float4 *>(Pw + j);
                    const float pq[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        if (j + u < kc) psum = psum + pq[u];
                        if ((nz >> (j + u)) & 1ull) acc = fmaf(vt[(j + u) * 64], pq[u], acc);
                    }
                }
            }
            l = l * alpha + psum;
            m = nm;
        }
        // This wave's reads of slot t % DNB are done before block t + DNB's
        // copies land in it.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    a.O[row * D + blockIdx.y * 64 + lane] = acc * inv;
}

template <int D>
void launch_decode(hipStream_t s, const Attn &a, float *ws)
{
    static std::atomic<bool> lds_optin{false};
    if (!lds_optin)
        lds_optin = hipFuncSetAttribute(reinterpret_cast<const void *>(attn_dec_chain<D>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        static_cast<int>(kDecLds)) == hipSuccess &&
                    hipFuncSetAttribute(reinterpret_cast<const void *>(attn_dec_scores<D>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        static_cast<int>(dec_scores_lds<D>())) == hipSuccess;
    const uint32_t pitch = dec_pitch(a);
    const uint64_t per_bh = static_cast<uint64_t>(a.seq_q) * pitch * sizeof(float);
    const uint64_t nbh = static_cast<uint64_t>(a.batch) * a.heads;
    const uint64_t step = std::max<uint64_t>(1, kDecScoreCap / per_bh);
    for (uint64_t b0 = 0; b0 < nbh; b0 += step) {
        const uint32_t n = static_cast<uint32_t>(std::min(step, nbh - b0));
        Attn c = a;   // the (batch, head) range [b0, b0 + n) as a batch of n single heads
        const uint64_t qo = b0 * a.seq_q * D, ko = b0 * a.seq_k * D;
        c.Q = a.Q + qo; c.K = a.K + ko; c.V = a.V + ko; c.O = a.O + qo;
        c.mask = a.mask ? a.mask + b0 * a.seq_q * a.seq_k : nullptr;
        c.batch = n;
        c.heads = 1;
        const uint32_t tiles = (a.seq_k + XB - 1) / XB;
        attn_dec_scores<D><<<dim3((tiles + DTPW - 1) / DTPW, n), 64, dec_scores_lds<D>(), s>>>(c, ws, pitch);
        attn_dec_chain<D><<<dim3(n * a.seq_q, D / 64), 64, kDecLds, s>>>(c, ws, pitch);
    }
}

}  // namespace

void attention_exact_prefill(hipStream_t s, const Attn &a)
{
    if (a.head_dim == 128) launch<128>(s, a);
    else launch<64>(s, a);
}

size_t attention_exact_decode_ws_bytes(const Attn &a)
{
    const uint64_t per_bh = static_cast<uint64_t>(a.seq_q) * dec_pitch(a) * sizeof(float);
    const uint64_t nbh = static_cast<uint64_t>(a.batch) * a.heads;
    const uint64_t step = std::max<uint64_t>(1, kDecScoreCap / per_bh);
    return static_cast<size_t>(std::min(step, nbh) * per_bh);
}

void attention_exact_decode(hipStream_t s, const Attn &a, float *ws)
{
    if (a.head_dim == 128) launch_decode<128>(s, a, ws);
    else launch_decode<64>(s, a, ws);
}

}  // namespace k
}  // namespace vnpu
