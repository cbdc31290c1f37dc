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

        // Scores: S[t][r] is (key k0 + 32t + 8(r/4) + 4h + r%4, row qi).
        float S[2][16];
#pragma unroll
        for (int r = 0; r < 16; ++r) S[1][r] = -__builtin_inff();
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            if (t == 1 && kc_w <= 32) continue;   // uniform: no key of the second tile is seen
            f32x32 acc0, acc1, acc2, acc3;
#pragma unroll
            for (int r = 0; r < 32; ++r) acc0[r] = acc1[r] = acc2[r] = acc3[r] = 0.0f;
            const float *kr = Kb + (32 * t + c32) * L::KP + 4 * h;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const float4 kv = *reinterpret_cast<const float4 *>(kr + 8 * i);
                acc0 = mfma1(kv.x, qop[i].x, acc0);
                acc1 = mfma1(kv.y, qop[i].y, acc1);
                acc2 = mfma1(kv.z, qop[i].z, acc2);
                acc3 = mfma1(kv.w, qop[i].w, acc3);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float dot = ((acc0[r] + acc0[r + 16]) + (acc1[r] + acc1[r + 16])) +
                                  ((acc2[r] + acc2[r + 16]) + (acc3[r] + acc3[r + 16]));
                const uint32_t key = k0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
                const float sc = dot * a.scale;
                const bool valid = qvalid && key < kend && !(a.causal && key > qi + off);
                S[t][r] = valid ? sc : -__builtin_inff();
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
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
        const bool live = isfinite(bmax);
        const float nm = m < bmax ? bmax : m;
        const float alpha = live ? dev::fast_expf_unfused(m - nm) : 1.0f;
        // Weights in key order: Plo[t][r] is key 32t + 8(r/4) + r%4, Phi[t][r]
        // key 32t + 8(r/4) + 4 + r%4 (the other half's keys by exchange).
        float Plo[2][16], Phi[2][16];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = live ? dev::fast_expf_unfused(S[t][r] - nm) : 0.0f;
                const float x = __shfl_xor(p, 32, 64);
                Plo[t][r] = h ? x : p;
                Phi[t][r] = h ? p : x;
            }
        if (live) {
            float psum = 0.0f;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int a4 = 0; a4 < 4; ++a4) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) psum = psum + Plo[t][4 * a4 + j];
#pragma unroll
                    for (int j = 0; j < 4; ++j) psum = psum + Phi[t][4 * a4 + j];
                }
            l = l * alpha + psum;
            m = nm;
        }
#pragma unroll
        for (int mm = 0; mm < NM; ++mm)
#pragma unroll
            for (int r = 0; r < 32; ++r) oacc[mm][r] = oacc[mm][r] * alpha;

        // Output chain, keys ascending; keys no row of the wave sees are skipped.
#pragma unroll
        for (int kk = 0; kk < XB; ++kk) {
            const int t = kk >> 5, r = 4 * ((kk & 31) >> 3) + (kk & 3);
            const float p = (kk & 4) ? Phi[t][r] : Plo[t][r];
            if (kk < static_cast<int>(kc_w)) {   // uniform
#pragma unroll
                for (int mm = 0; mm < NM; ++mm) oacc[mm] = mfma1(Vb[kk * D + 64 * mm + lane], p, oacc[mm]);
            }
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

}  // namespace

void attention_exact_prefill(hipStream_t s, const Attn &a)
{
    if (a.head_dim == 128) launch<128>(s, a);
    else launch<64>(s, a);
}

}  // namespace k
}  // namespace vnpu
