// gemm_f32.hip - MATMUL_F32 / MTP_HEAD_F32 on gfx950.
//
// Semantics: the reference's store_c / zero_c_tile (src/kernels/kernels.cpp:
// 43-62) with the defaults of prepare_matmul_f32 (src/core/scheduler.cpp:
// 274-318):
//   C = epi(alpha * op(A) op(B) + bias + beta * C_in)        (computed tile)
//   C = epi(bias + beta * C_in)                             (Wildcat-culled)
// applied once over the full K sum.  (The reference's default AVX2 packed NN
// path applies the epilogue after the first 128-deep K block only,
// kernels.cpp:313-323; this backend implements the documented semantics,
// which its scalar, NT, row-stream and VNPU_PACK=0 paths also compute.)
//
// Two kernels:
//   * gemm_f32_kernel: 128 x 128 workgroup tile, 2 x 2 waves of 64 x 64,
//     v_mfma_f32_16x16x4_f32, both operands staged k-major in LDS (double
//     buffered; row pitch 144 floats keeps fragment reads conflict free).
//     trans_a / trans_b only change how a tile is fetched from HBM.
//   * gemv_f32_kernel: M <= 8, NN (the MTP head and f32 decode GEMMs).  HBM
//     bound: 256 columns x float4 per workgroup, waves and workgroups split K,
//     weights streamed with branch-free bounds-checked buffer loads,
//     activations read as wave-uniform scalars; partial sums reduced in a
//     second deterministic pass when K is split across workgroups.
//   * gemv_f32_wide: the same for N of 200 x 128 columns and more (the MTP
//     head's vocabulary): 128 columns x all of K per 16-wave workgroup, one
//     pass, no partials.
#include "kernels.hpp"

#include <atomic>
#include "device_math.hpp"

#include <algorithm>
#include <type_traits>

namespace vnpu {
namespace k {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 16;
constexpr int kThreads = 256;
constexpr int kPitch = 144;

// Loads 4 consecutive elements along the contiguous dimension of a matrix
// stored with leading dimension ld: element (r, c0 + i), zero outside
// rows x cols.
__device__ __forceinline__ float4 load4(const float *base, uint32_t ld, uint32_t r, uint32_t c0,
                                        uint32_t rows, uint32_t cols, bool vec)
{
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (r >= rows) return v;
    const float *p = base + static_cast<uint64_t>(r) * ld + c0;
    if (vec && c0 + 4 <= cols) return *reinterpret_cast<const float4 *>(p);
    if (c0 + 0 < cols) v.x = p[0];
    if (c0 + 1 < cols) v.y = p[1];
    if (c0 + 2 < cols) v.z = p[2];
    if (c0 + 3 < cols) v.w = p[3];
    return v;
}

struct Stage {
    float4 a0, a1, b0, b1;
};

// Fetch the (k0 .. k0+15) x tile slices of A (BM rows) and B (BN cols).
// Thread mapping depends on which dimension is contiguous in memory.
__device__ __forceinline__ void fetch(const F32Gemm &p, uint32_t m0, uint32_t n0, uint32_t k0,
                                      int tid, bool va, bool vb, Stage &s)
{
    if (!p.trans_a) {  // A[m][k]: 128 rows x 4 float4 along k
        const uint32_t r = tid >> 2, c = (tid & 3) * 4;
        s.a0 = load4(p.A, p.lda, m0 + r, k0 + c, p.M, p.K, va);
        s.a1 = load4(p.A, p.lda, m0 + r + 64, k0 + c, p.M, p.K, va);
    } else {           // A[k][m]: 16 rows x 32 float4 along m
        const uint32_t r = tid >> 5, c = (tid & 31) * 4;
        s.a0 = load4(p.A, p.lda, k0 + r, m0 + c, p.K, p.M, va);
        s.a1 = load4(p.A, p.lda, k0 + r + 8, m0 + c, p.K, p.M, va);
    }
    if (!p.trans_b) {  // B[k][n]: 16 rows x 32 float4 along n
        const uint32_t r = tid >> 5, c = (tid & 31) * 4;
        s.b0 = load4(p.B, p.ldb, k0 + r, n0 + c, p.K, p.N, vb);
        s.b1 = load4(p.B, p.ldb, k0 + r + 8, n0 + c, p.K, p.N, vb);
    } else {           // B[n][k]: 128 rows x 4 float4 along k
        const uint32_t r = tid >> 2, c = (tid & 3) * 4;
        s.b0 = load4(p.B, p.ldb, n0 + r, k0 + c, p.N, p.K, vb);
        s.b1 = load4(p.B, p.ldb, n0 + r + 64, k0 + c, p.N, p.K, vb);
    }
}

// Store a fetched stage k-major: As[k][m], Bs[k][n].
__device__ __forceinline__ void stash(const F32Gemm &p, int tid, const Stage &s, float *As,
                                      float *Bs)
{
    if (!p.trans_a) {
        const uint32_t r = tid >> 2, c = (tid & 3) * 4;
        As[(c + 0) * kPitch + r] = s.a0.x; As[(c + 1) * kPitch + r] = s.a0.y;
        As[(c + 2) * kPitch + r] = s.a0.z; As[(c + 3) * kPitch + r] = s.a0.w;
        As[(c + 0) * kPitch + r + 64] = s.a1.x; As[(c + 1) * kPitch + r + 64] = s.a1.y;
        As[(c + 2) * kPitch + r + 64] = s.a1.z; As[(c + 3) * kPitch + r + 64] = s.a1.w;
    } else {
        const uint32_t r = tid >> 5, c = (tid & 31) * 4;
        *reinterpret_cast<float4 *>(&As[r * kPitch + c]) = s.a0;
        *reinterpret_cast<float4 *>(&As[(r + 8) * kPitch + c]) = s.a1;
    }
    if (!p.trans_b) {
        const uint32_t r = tid >> 5, c = (tid & 31) * 4;
        *reinterpret_cast<float4 *>(&Bs[r * kPitch + c]) = s.b0;
        *reinterpret_cast<float4 *>(&Bs[(r + 8) * kPitch + c]) = s.b1;
    } else {
        const uint32_t r = tid >> 2, c = (tid & 3) * 4;
        Bs[(c + 0) * kPitch + r] = s.b0.x; Bs[(c + 1) * kPitch + r] = s.b0.y;
        Bs[(c + 2) * kPitch + r] = s.b0.z; Bs[(c + 3) * kPitch + r] = s.b0.w;
        Bs[(c + 0) * kPitch + r + 64] = s.b1.x; Bs[(c + 1) * kPitch + r + 64] = s.b1.y;
        Bs[(c + 2) * kPitch + r + 64] = s.b1.z; Bs[(c + 3) * kPitch + r + 64] = s.b1.w;
    }
}

__device__ __forceinline__ bool culled(const F32Gemm &p, uint32_t m, uint32_t n)
{
    return p.cull[static_cast<uint64_t>(m / p.cull_tm) * p.cull_nt + n / p.cull_tn] != 0;
}

__device__ __forceinline__ void store_out(const F32Gemm &p, uint32_t m, uint32_t n, float acc,
                                          bool cull)
{
    float *dst = p.C + static_cast<uint64_t>(m) * p.ldc + n;
    float out;
    if (cull) {
        out = p.bias ? p.bias[n] : 0.0f;
        if (p.beta != 0.0f) out += p.beta * *dst;
    } else {
        out = p.alpha * acc;
        if (p.bias) out += p.bias[n];
        if (p.beta != 0.0f) out += p.beta * *dst;
    }
    *dst = dev::epilogue(out, p.epilogue);
}

// blockIdx.z selects a k range of k_per_split (a multiple of BK) when K is
// split over workgroups; then the raw sums go to ws[z][m][n] and
// gemm_f32_splitk_reduce applies alpha, bias, beta and the epilogue once.
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(F32Gemm p, uint32_t k_per_split, float *ws)
{
    __shared__ __attribute__((aligned(16))) float As[2][BK * kPitch];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK * kPitch];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int fr = lane & 15, fg = lane >> 4;

    uint8_t state = 0;
    if (p.ktile_state) state = p.ktile_state[blockIdx.y * gridDim.x + blockIdx.x];

    v4f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

    if (state != 1) {
        const bool va = ((p.lda & 3u) == 0) && ((reinterpret_cast<uintptr_t>(p.A) & 15u) == 0);
        const bool vb = ((p.ldb & 3u) == 0) && ((reinterpret_cast<uintptr_t>(p.B) & 15u) == 0);
        const uint32_t kb = blockIdx.z * k_per_split;
        const uint32_t ke = min(p.K, kb + k_per_split);
        const uint32_t KT = (ke - kb + BK - 1) / BK;
        Stage st;
        fetch(p, m0, n0, kb, tid, va, vb, st);
        stash(p, tid, st, As[0], Bs[0]);
        __syncthreads();
        for (uint32_t kt = 0; kt < KT; ++kt) {
            const int cur = kt & 1;
            const bool more = kt + 1 < KT;
            if (more) fetch(p, m0, n0, kb + (kt + 1) * BK, tid, va, vb, st);
            const float *as = As[cur];
            const float *bs = Bs[cur];
#pragma unroll
            for (int kk = 0; kk < BK / 4; ++kk) {
                float a[4], b[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) a[i] = as[(kk * 4 + fg) * kPitch + wm * 64 + i * 16 + fr];
#pragma unroll
                for (int j = 0; j < 4; ++j) b[j] = bs[(kk * 4 + fg) * kPitch + wn * 64 + j * 16 + fr];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
            }
            if (more) stash(p, tid, st, As[cur ^ 1], Bs[cur ^ 1]);
            __syncthreads();
        }
    }

#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t n = n0 + wn * 64 + j * 16 + fr;
        if (n >= p.N) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t m = m0 + wm * 64 + i * 16 + fg * 4 + r;
                if (m >= p.M) continue;
                if (ws) {
                    ws[(static_cast<uint64_t>(blockIdx.z) * p.M + m) * p.N + n] = acc[i][j][r];
                    continue;
                }
                const bool c = state == 1 ? true : (state == 2 ? culled(p, m, n) : false);
                store_out(p, m, n, acc[i][j][r], c);
            }
    }
}

__global__ __launch_bounds__(kThreads) void gemm_f32_splitk_reduce(F32Gemm p, const float *ws, uint32_t splits)
{
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const uint64_t total = static_cast<uint64_t>(p.M) * p.N;
    if (idx >= total) return;
    const uint32_t m = static_cast<uint32_t>(idx / p.N), n = static_cast<uint32_t>(idx % p.N);
    // Partials in groups of eight whose loads are issued together (one round
    // trip per group), summed in split order.
    constexpr uint32_t G = 8;
    float s = 0.0f;
    for (uint32_t i0 = 0; i0 < splits; i0 += G) {
        float v[G];
#pragma unroll
        for (uint32_t u = 0; u < G; ++u)
            v[u] = i0 + u < splits ? ws[static_cast<uint64_t>(i0 + u) * total + idx] : 0.0f;
#pragma unroll
        for (uint32_t u = 0; u < G; ++u)
            if (i0 + u < splits) s += v[u];
    }
    store_out(p, m, n, s, false);
}

// ---------------------------------------------------------------------------
// Split-bf16 prefill kernel (no cull, 16-byte aligned operands).
//
// gfx950's bf16 matrix cores run ~11x faster than its f32 ones (measured with
// random operands: v_mfma_f32_32x32x16_bf16 1.8 PFLOP/s, v_mfma_f32_16x16x4_f32
// 157 TFLOP/s).  Each f32 element x is split into hi = bf16(x) and
// lo = bf16(x - hi) (x - hi is exact) and every product is taken as
// hi*hi + hi*lo + lo*hi in f32 accumulation: the dropped lo*lo term and the
// rounding of lo leave ~2^-16 relative error per product, an order of
// magnitude inside the MATMUL_F32 bar (1e-4 of the output's largest value).
//   * 128 x 128 workgroup tile, 2 x 2 waves of 64 x 64 (2 x 2 tiles of
//     32 x 32), 32-deep k stages, two workgroups per CU;
//   * the next stage's f32 slices are loaded into registers while the
//     current stage is multiplied, then split and written to the other LDS
//     buffer: per operand row (m for A, n for B) 32 k of bf16 as 4 chunks of
//     16 bytes, hi and lo in separate planes, chunk c of row r at slot
//     c ^ ((r >> 2) & 3): ds_read_b128 serves 16 lanes at a time from one
//     256-byte window of banks, and the 16 rows of a quarter wave at one
//     chunk then hit 16 distinct 16-byte slots of it (measured: the
//     (r >> 1) & 3 swizzle that only separates 8 rows costs 1.6x);
//   * an operand stored k-contiguous (A, or B with trans_b) is fetched as 8
//     consecutive k of one row per item; one stored the other way (B, or A
//     with trans_a) as 8 rows of k by 2 adjacent columns, so a lane's chunk
//     is one column's 8 k either way.
// ---------------------------------------------------------------------------
namespace x3 {
constexpr int TN = 128, BK = 32;
// Two stages of A hi, A lo (64*WM rows) and B hi, B lo (128 rows), 32 k of
// bf16 per row: 64 KiB for WM = 2, 96 KiB for WM = 4.
constexpr int lds_bytes(int wm) { return 2 * (2 * 64 * wm + 2 * TN) * BK * 2; }
}  // namespace x3

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

// hi = bf16(x) rounded to nearest even, lo = bf16(x - hi).  hi is rounded
// from x clamped to the largest finite bf16 (3.3895e38), so it is finite for
// every finite x and x - hi stays exact; an infinite x leaves its infinity in
// lo (hi*b + hi*lo_b + lo*b is then +-inf with the sign of x*b, as the f32
// product), and a NaN x gives lo = NaN, which propagates.
__device__ __forceinline__ void split8(const float (&x)[8], v8bf &hi, v8bf &lo)
{
    typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
    typedef float v2f __attribute__((ext_vector_type(2)));
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    constexpr float kBf16Max = 3.38953139e38f;   // 0x7F7F0000
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        // one v_med3 each (fminf(fmaxf()) adds a NaN-quieting max per input)
        const float c0 = __builtin_amdgcn_fmed3f(x[2 * e], -kBf16Max, kBf16Max);
        const float c1 = __builtin_amdgcn_fmed3f(x[2 * e + 1], -kBf16Max, kBf16Max);
        hw[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){c0, c1}, v2bf));
        const float h0 = __builtin_bit_cast(float, hw[e] << 16);
        const float h1 = __builtin_bit_cast(float, hw[e] & 0xFFFF0000u);
        lw[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){x[2 * e] - h0, x[2 * e + 1] - h1}, v2bf));
    }
    hi = __builtin_bit_cast(v8bf, (v4u){hw[0], hw[1], hw[2], hw[3]});
    lo = __builtin_bit_cast(v8bf, (v4u){lw[0], lw[1], lw[2], lw[3]});
}

// One operand's share of a stage: up to two chunks (8 k of one row each).
struct X3Slice {
    float x[2][8];
};

// Operand op(X) viewed as R rows (m of A, n of B) x k, fetched by NT
// threads.  KCONTIG: X[row][k] with leading dimension ld, item i = (row i/4,
// chunk i%4), 4R/NT items per thread.  Otherwise X[k][row]: item i = (rows
// 2p, 2p+1 with p = i % (R/2), chunk i / (R/2)), two chunks per item, one item
// per thread for the first 2R threads.
template <bool KCONTIG, int R, int NT>
__device__ __forceinline__ constexpr int x3_chunks()
{
    return KCONTIG ? 4 * R / NT : 2;
}

template <bool KCONTIG, int R, int NT>
__device__ __forceinline__ bool x3_active(int tid)
{
    return KCONTIG || tid < 2 * R;
}

template <bool KCONTIG, int R, int NT>
__device__ __forceinline__ void x3_chunk(int tid, int u, uint32_t &row, uint32_t &c)
{
    if (KCONTIG) {
        const uint32_t item = tid + NT * u;
        row = item >> 2;
        c = item & 3;
    } else {
        row = 2 * (tid % (R / 2)) + u;
        c = tid / (R / 2);
    }
}

template <bool KCONTIG, int R, int NT>
__device__ __forceinline__ void x3_fetch(const float *X, uint32_t ld, uint32_t rows, uint32_t K,
                                         uint32_t r0, uint32_t k0, int tid, X3Slice &s)
{
    static_assert(x3_chunks<KCONTIG, R, NT>() >= 1 && x3_chunks<KCONTIG, R, NT>() <= 2, "slice size");
    if (!x3_active<KCONTIG, R, NT>(tid)) return;
    if (KCONTIG) {
#pragma unroll
        for (int u = 0; u < x3_chunks<KCONTIG, R, NT>(); ++u) {
            uint32_t row, c;
            x3_chunk<KCONTIG, R, NT>(tid, u, row, c);
            const uint32_t r = r0 + row, k = k0 + 8 * c;
            const float *p = X + static_cast<uint64_t>(r) * ld + k;
            if (r < rows && k + 8 <= K) {
                const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
                s.x[u][0] = a.x; s.x[u][1] = a.y; s.x[u][2] = a.z; s.x[u][3] = a.w;
                s.x[u][4] = b.x; s.x[u][5] = b.y; s.x[u][6] = b.z; s.x[u][7] = b.w;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) s.x[u][e] = (r < rows && k + e < K) ? p[e] : 0.0f;
            }
        }
    } else {
        uint32_t row, c;
        x3_chunk<KCONTIG, R, NT>(tid, 0, row, c);
        const uint32_t r = r0 + row, k = k0 + 8 * c;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float *p = X + static_cast<uint64_t>(k + e) * ld + r;
            if (k + e < K && r + 1 < rows) {
                const float2 v = *reinterpret_cast<const float2 *>(p);
                s.x[0][e] = v.x;
                s.x[1][e] = v.y;
            } else {
                s.x[0][e] = (k + e < K && r < rows) ? p[0] : 0.0f;
                s.x[1][e] = (k + e < K && r + 1 < rows) ? p[1] : 0.0f;
            }
        }
    }
}

// hi plane at hi_plane, lo plane plane_bytes after it.
template <bool KCONTIG, int R, int NT>
__device__ __forceinline__ void x3_stash(const X3Slice &s, int tid, int8_t *hi_plane, int plane_bytes)
{
    if (!x3_active<KCONTIG, R, NT>(tid)) return;
#pragma unroll
    for (int u = 0; u < x3_chunks<KCONTIG, R, NT>(); ++u) {
        uint32_t row, c;
        x3_chunk<KCONTIG, R, NT>(tid, u, row, c);
        v8bf h, l;
        split8(s.x[u], h, l);
        const uint32_t off = row * (x3::BK * 2) + ((c ^ ((row >> 2) & 3)) << 4);
        *reinterpret_cast<v8bf *>(hi_plane + off) = h;
        *reinterpret_cast<v8bf *>(hi_plane + plane_bytes + off) = l;
    }
}

// WM wave rows: the tile is 64*WM x 128 (WM = 2: four waves, two workgroups
// per CU; WM = 4: eight waves, one workgroup per CU, each A slice converted
// once for twice the columns... the B slice once for twice the rows).
// The epilogue of a wave's 64 x 64 block straight from its accumulators
// (store_out's arithmetic: alpha * acc + bias + beta * C_in -> epi).  The
// wave's 64 rows of C are one buffer whose range check drops rows past M,
// and columns past N get an offset past its end, so loads and stores need
// no branches; the column's bias is loaded once and every C_in value of the
// block is in flight before the first is used.  Needs ldc <= kX3MaxLdc (64
// rows of C within a 31-bit byte range).
constexpr uint32_t kX3MaxLdc = (1u << 23) - 1;
constexpr int kCBufferWord3 = 0x00020000;   // raw buffer, 32-bit data format
constexpr int kCStorePolicy = 2;            // nontemporal: C is written once

// EPI: the epilogue (0 none, 1 ReLU, 2 SiLU, 3 GELU); NB: C_in batches (the
// loads of one batch of row tiles are all in flight before the first is used).
template <int EPI, int NB>
__device__ __forceinline__ void x3_store_rows(const F32Gemm &p, const v16f (&acc)[2][2], uint32_t mrow,
                                              uint32_t ncol, int h)
{
    const uint32_t rows = mrow < p.M ? min(64u, p.M - mrow) : 0u;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        p.C + static_cast<uint64_t>(mrow) * p.ldc, 0, static_cast<int>(rows * p.ldc * 4u), kCBufferWord3);
    const uint32_t ld4 = p.ldc * 4u;
    float bv[2];
    uint32_t off[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t n = ncol + 32 * j;
        const bool ok = n < p.N;
        bv[j] = (ok && p.bias) ? p.bias[n] : 0.0f;
        off[j] = ok ? (static_cast<uint32_t>(4 * h) * p.ldc + n) * 4u : 0x80000000u;
    }
    auto at = [&](int i, int j, int r) {
        return static_cast<int>(off[j] + static_cast<uint32_t>(32 * i + 8 * (r >> 2) + (r & 3)) * ld4);
    };
    constexpr int PER = 2 / NB;   // row tiles per batch
#pragma unroll
    for (int bt = 0; bt < NB; ++bt) {
        float cin[PER][2][16];
        if (p.beta != 0.0f) {
#pragma unroll
            for (int ii = 0; ii < PER; ++ii)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        cin[ii][j][r] = __builtin_bit_cast(
                            float, __builtin_amdgcn_raw_buffer_load_b32(rs, at(bt * PER + ii, j, r), 0, 0));
        }
#pragma unroll
        for (int ii = 0; ii < PER; ++ii)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int i = bt * PER + ii;
                    float out = p.alpha * acc[i][j][r];
                    if (p.bias) out += bv[j];
                    if (p.beta != 0.0f) out += p.beta * cin[ii][j][r];
                    out = dev::epilogue(out, EPI);
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, out), rs, at(i, j, r), 0,
                                                          kCStorePolicy);
                }
    }
}

// x3_store_rows with the epilogue chosen once per call.
template <int NB>
__device__ __forceinline__ void x3_store_rows_epi(const F32Gemm &p, const v16f (&acc)[2][2], uint32_t mrow,
                                                  uint32_t ncol, int h)
{
    switch (p.epilogue) {
    case 1: x3_store_rows<1, NB>(p, acc, mrow, ncol, h); break;
    case 2: x3_store_rows<2, NB>(p, acc, mrow, ncol, h); break;
    case 3:
    case 4: x3_store_rows<3, NB>(p, acc, mrow, ncol, h); break;
    default: x3_store_rows<0, NB>(p, acc, mrow, ncol, h); break;
    }
}

// blockIdx.y selects the k range [y * k_per_split, + k_per_split) (a
// multiple of the 32-deep stage) when K is split over workgroups; then the
// raw sums go to ws[y][m][n] and gemm_f32_splitk_reduce applies alpha, bias,
// beta and the epilogue once.
template <bool TA, bool TB, int WM>
__global__ __launch_bounds__(128 * WM) void gemm_f32_x3(F32Gemm p, uint32_t k_per_split, float *ws)
{
    constexpr uint32_t TM = 64 * WM, TN = x3::TN, XBK = x3::BK;
    constexpr int NT = 128 * WM;
    constexpr int kPlaneA = TM * XBK * 2, kPlaneB = TN * XBK * 2;
    constexpr int kStage = 2 * kPlaneA + 2 * kPlaneB;
    extern __shared__ __attribute__((aligned(1024))) int8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    // Tiles run M-fastest, and each XCD (workgroup g runs on XCD g % 8) takes
    // a contiguous run of them: the XCD's resident workgroups share A's rows
    // and a few of B's column tiles through its L2.
    const uint32_t tiles_m = (p.M + TM - 1) / TM, total = tiles_m * ((p.N + TN - 1) / TN);
    uint32_t g = blockIdx.x;
    if ((total & 7u) == 0) g = (g & 7u) * (total >> 3) + (g >> 3);
    const uint32_t m0 = (g % tiles_m) * TM, n0 = (g / tiles_m) * TN;
    const uint32_t kb = blockIdx.y * k_per_split;
    const uint32_t KT = (min(p.K, kb + k_per_split) - kb + XBK - 1) / XBK;
    const int h = lane >> 5, col = lane & 31;

    // The next stage's f32 slices load into registers while this stage is
    // multiplied, then are split into the other LDS buffer.
    X3Slice sa, sb;
    auto fetch = [&](uint32_t kt) {
        x3_fetch<!TA, TM, NT>(p.A, p.lda, p.M, p.K, m0, kb + kt * XBK, tid, sa);
        x3_fetch<TB, TN, NT>(p.B, p.ldb, p.N, p.K, n0, kb + kt * XBK, tid, sb);
    };
    auto stash = [&](uint32_t kt) {
        int8_t *st = smem + (kt & 1) * kStage;
        x3_stash<!TA, TM, NT>(sa, tid, st, kPlaneA);
        x3_stash<TB, TN, NT>(sb, tid, st + 2 * kPlaneA, kPlaneB);
    };

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (v16f){0.f};

    fetch(0);
    stash(0);
    __syncthreads();
    for (uint32_t kt = 0; kt < KT; ++kt) {
        const bool more = kt + 1 < KT;
        if (more) fetch(kt + 1);
        const int8_t *st = smem + (kt & 1) * kStage;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            // lane (row l%32, half h) reads k 16s + 8h .. +8 of its row
            v8bf ah[2], al[2], bh[2], bl[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint32_t r = wm * 64 + 32 * i + col;
                const uint32_t off = r * (XBK * 2) + (((2 * s + h) ^ ((r >> 2) & 3)) << 4);
                ah[i] = *reinterpret_cast<const v8bf *>(st + off);
                al[i] = *reinterpret_cast<const v8bf *>(st + kPlaneA + off);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t r = wn * 64 + 32 * j + col;
                const uint32_t off = r * (XBK * 2) + (((2 * s + h) ^ ((r >> 2) & 3)) << 4);
                bh[j] = *reinterpret_cast<const v8bf *>(st + 2 * kPlaneA + off);
                bl[j] = *reinterpret_cast<const v8bf *>(st + 2 * kPlaneA + kPlaneB + off);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bl[j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bh[j], acc[i][j], 0, 0, 0);
        }
        // The other buffer was last read in step kt-1, before the barrier
        // that ended it; the next barrier publishes the new stage.
        if (more) stash(kt + 1);
        __syncthreads();
    }

    // 32 x 32 accumulator: lane l holds column l%32, rows 8j' + 4(l/32) + i'
    // in register 4j' + i'; a store instruction writes two 128-byte row runs.
    // (The four-wave tile keeps the per-element stores: the direct epilogue's
    // registers slowed its main loop, which small and split grids run.)
    if constexpr (WM == 4) {
        if (!ws && p.ldc <= kX3MaxLdc) {
            x3_store_rows_epi<1>(p, acc, m0 + wm * 64, n0 + wn * 64 + col, h);
            return;
        }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t n = n0 + wn * 64 + 32 * j + col;
        if (n >= p.N) continue;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t m = m0 + wm * 64 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                if (m >= p.M) continue;
                if (ws)
                    ws[(static_cast<uint64_t>(blockIdx.y) * p.M + m) * p.N + n] = acc[i][j][r];
                else
                    store_out(p, m, n, acc[i][j][r], false);
            }
    }
}

// ---------------------------------------------------------------------------
// Warp-specialised split-bf16 kernel (op(A) = A, 256 x 128 tiles).
//
// The lock-step kernel above has every wave load, split and store a stage
// and then multiply between two barriers, so the matrix cores idle while the
// splits run.  Here four producer waves (one per SIMD) load the f32 slices of
// stage s + 2 and s + 1 into registers while they split stage s into a ring
// of three LDS stages (the layout above), and four consumer waves (one per
// SIMD) run only fragment reads and MFMAs, each owning a 128 x 64 block.
// The two sides meet through per-wave LDS flags instead of barriers:
// producer p sets prod[slot][p] = s + 1 once stage s is in the slot,
// consumer c sets cons[slot][c] = s + 1 once it has read stage s, and a
// producer refills a slot only when every consumer has released the stage
// three before.  Every wait is bounded: after p.max_spin polls (kMaxSpin when
// 0) the wave goes on, so a protocol error never hangs a wave; it stores 1
// into p.err (the stream's error word in host-coherent memory), which the
// stream's sync turns into a sticky device error, so the wrong C it leaves
// is never reported as success.
// Operand loads are raw buffer loads over the whole matrix (out of range
// reads return zero), rows past M / N are clamped and k past K is zeroed
// with selects: no branch around a load, so the three stages of loads stay
// in flight.
// ---------------------------------------------------------------------------
namespace ws {
constexpr int TM = 256, TN = 128, BK = 32, kSlots = 3;
constexpr int kPlaneA = TM * BK * 2, kPlaneB = TN * BK * 2;   // bytes of one bf16 plane
constexpr int kSlotBytes = 2 * kPlaneA + 2 * kPlaneB;        // 48 KiB
constexpr int kFlagOff = kSlots * kSlotBytes;                 // 144 KiB
constexpr int kLds = kFlagOff + 2 * 4 * kSlots * 4;
constexpr uint32_t kMaxSpin = 1u << 22;
constexpr int kBufWord3 = 0x00020000;
static_assert(kLds <= 160 * 1024, "ring + flags fit in LDS");
}  // namespace ws

// Flag words are read and written with asm: a volatile C++ access makes the
// compiler drain every outstanding global load first (vmcnt(0)), which would
// empty the producers' load pipeline at each poll.  The "memory" clobber keeps
// the compiler from moving LDS accesses across them; one wave's LDS operations
// execute in order, so data written before a flag is in place when the flag
// is seen, and a consumer's reads of a stage precede its release.
__device__ __forceinline__ uint32_t lds_addr(const uint32_t *p)
{
    return static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint32_t *)(p)));
}

// Waits until the four flags f[0..3] (one per wave of the other side) are at
// least `target`, at most p.max_spin polls (kMaxSpin when 0); a wait that
// gives up marks the launch failed in p.err.
__device__ __forceinline__ void ws_wait(const F32Gemm &p, const uint32_t *f, uint32_t target)
{
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    const uint32_t a = lds_addr(f);
    const uint32_t limit = p.max_spin ? p.max_spin : ws::kMaxSpin;
    for (uint32_t spin = 0; spin < limit; ++spin) {
        v4u v;
        asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
        const uint32_t lo = min(min(v.x, v.y), min(v.z, v.w));
        // No s_sleep: each poll already waits for its LDS read, and a sleep
        // measured 3-5% slower (the waiter reacts later).
        if (__builtin_amdgcn_readfirstlane(lo) >= target) return;
    }
    if (p.err) __hip_atomic_store(p.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Publishes `v` after this wave's earlier LDS reads and writes completed.
__device__ __forceinline__ void ws_release(uint32_t *f, uint32_t v)
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\tds_write_b32 %0, %1" : : "v"(lds_addr(f)), "v"(v) : "memory");
}

// One producer thread's share of a stage: A (k-contiguous) 4 chunks of 8 k,
// B 2 chunks (k-contiguous, TB) or 8 k x 2 adjacent columns (!TB).
struct WsSlice {
    float a[4][8];
    float b[2][8];
};

__device__ __forceinline__ void put4(float *d, const float4 v)
{
    d[0] = v.x;
    d[1] = v.y;
    d[2] = v.z;
    d[3] = v.w;
}

// Tile of workgroup b: the first `full` workgroups take tiles [0, full) one
// each; the rest split the remaining T2 = total - full tiles over K,
// workgroup full + sp * T2 + t taking k-slice sp of split tile t.  Within each
// part the tiles are remapped so that the workgroups of one XCD (b % 8, as
// they are dispatched round-robin) get a contiguous run of tiles, whose A
// rows and B columns then meet in that XCD's L2.
__host__ __device__ inline uint32_t ws_tile_of(uint32_t b, uint32_t full, uint32_t total, uint32_t *slice)
{
    if (b < full) {
        *slice = 0;
        return (full & 7u) == 0 ? (b & 7u) * (full >> 3) + (b >> 3) : b;
    }
    const uint32_t t2 = total - full, r = b - full, t = r % t2;
    *slice = r / t2;
    return full + ((t2 & 7u) == 0 ? (t & 7u) * (t2 >> 3) + (t >> 3) : t);
}

// Workgroups from `full` on split the remaining tiles over K, `splits` per
// tile, slice sp taking k stages [sp * ks_per, + ks_per) (the last one the
// rest); each writes its raw sums as a 256 x 128 row-major tile into part
// (workgroup full + r at part + r * 256 * 128) and gemm_f32_tail_reduce adds
// the slices in order and finishes them.  Used when the last round of tiles
// would leave at least half the CUs idle (two slices) and for grids of fewer
// tiles than CUs (as many slices as fill the CUs).
template <bool TB>
__global__ __launch_bounds__(512) void gemm_f32_ws(F32Gemm p, uint32_t full, uint32_t ks_per, float *part)
{
    using ws::kSlots;
    using ws::kSlotBytes;
    using ws::kPlaneA;
    using ws::kPlaneB;
    using ws::kFlagOff;
    using ws::TM;
    using ws::TN;
    constexpr uint32_t WBK = ws::BK;
    extern __shared__ __attribute__((aligned(1024))) int8_t smem[];
    uint32_t *flags = reinterpret_cast<uint32_t *>(smem + kFlagOff);   // prod[slot][4], cons[slot][4]
    uint32_t *prod = flags, *cons = flags + 4 * kSlots;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t tiles_m = (p.M + TM - 1) / TM, total = tiles_m * ((p.N + TN - 1) / TN);
    const bool split = blockIdx.x >= full;
    uint32_t sp;
    const uint32_t g = ws_tile_of(blockIdx.x, full, total, &sp);
    const uint32_t m0 = (g % tiles_m) * TM, n0 = (g / tiles_m) * TN;
    const uint32_t KTall = (p.K + WBK - 1) / WBK;
    // This workgroup's k stages: [ks0, ks0 + KT); the host gives every slice
    // at least one stage
    const uint32_t ks0 = split ? sp * ks_per : 0u;
    const uint32_t KT = split ? min(ks_per, KTall - ks0) : KTall;
    if (tid < 2 * 4 * kSlots) flags[tid] = 0;
    __syncthreads();

    if (wave >= 4) {
        // ---------------- producers ----------------
        const int pw = wave - 4, pt = tid - 256;
        const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float *>(p.A), 0, static_cast<int>(static_cast<uint64_t>(p.M) * p.lda * 4), ws::kBufWord3);
        const uint32_t brows = TB ? p.N : p.K;
        const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float *>(p.B), 0, static_cast<int>(static_cast<uint64_t>(brows) * p.ldb * 4), ws::kBufWord3);
        // A item u: row pt/4 + 64u, chunk pt%4 (a wave reads 16 whole 128-byte row runs)
        uint32_t a_off[4];
        bool a_ok[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t r = (pt >> 2) + 64 * u, m = m0 + r;
            a_ok[u] = m < p.M;
            a_off[u] = (min(m, p.M - 1) * p.lda + 8 * (pt & 3)) * 4;
        }
        // B items: TB as A (rows pt/4 + 64u, u < 2); !TB rows 2(pt%64), +1 at chunk pt/64
        uint32_t b_off[2];
        bool b_ok[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (TB) {
                const uint32_t n = n0 + (pt >> 2) + 64 * u;
                b_ok[u] = n < p.N;
                b_off[u] = (min(n, p.N - 1) * p.ldb + 8 * (pt & 3)) * 4;
            } else {
                // the float2 load starts at an even column (8-byte aligned rows: ldb % 4 == 0)
                const uint32_t n = n0 + 2 * (pt & 63) + u;
                b_ok[u] = n < p.N;
                b_off[u] = min(n0 + 2 * (pt & 63), (p.N - 1) & ~1u) * 4;
            }
        }
        auto load = [&](WsSlice &x, uint32_t s) {
            const uint32_t k0 = (ks0 + min(s, KT - 1)) * WBK;
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int v = 0; v < 2; ++v)
                    put4(&x.a[u][4 * v], __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                       ra, a_off[u] + (k0 + 4 * v) * 4, 0, 0)));
            if (TB) {
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int v = 0; v < 2; ++v)
                        put4(&x.b[u][4 * v], __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                           rb, b_off[u] + (k0 + 4 * v) * 4, 0, 0)));
            } else {
                // rows k0 + 8c + e (c = pt/64), columns 2(pt%64) and +1: a float2 per k
                const uint32_t kc = k0 + 8 * (pt >> 6);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t kk = min(kc + e, p.K - 1);
                    const float2 v2 = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(
                                                                     rb, kk * p.ldb * 4 + b_off[0], 0, 0));
                    x.b[0][e] = v2.x;
                    x.b[1][e] = v2.y;
                }
            }
        };
        // LDS byte offsets within a slot.  A rows pt/4 + 64u all have the
        // swizzle (pt/16) & 3, so one base plus immediates (4096 u, the lo
        // plane) places every chunk; B likewise (TB: rows pt/4 + 64u; !TB:
        // rows 2(pt%64) + u, swizzle (pt%64)/2 & 3, 64 bytes apart).
        const uint32_t a_lds = (pt >> 2) * (WBK * 2) + (((pt & 3) ^ ((pt >> 4) & 3)) << 4);
        const uint32_t b_lds = TB ? a_lds
                                  : 2 * (pt & 63) * (WBK * 2) + (((pt >> 6) ^ (((pt & 63) >> 1) & 3)) << 4);
        constexpr uint32_t kBStep = TB ? 4096 : 64;
        auto write = [&](const WsSlice &x, uint32_t slot) {
            int8_t *sa = smem + slot * kSlotBytes + a_lds;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                v8bf h, l;
                split8(x.a[u], h, l);
                *reinterpret_cast<v8bf *>(sa + 4096 * u) = h;
                *reinterpret_cast<v8bf *>(sa + kPlaneA + 4096 * u) = l;
            }
            int8_t *sb = smem + slot * kSlotBytes + 2 * kPlaneA + b_lds;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                v8bf h, l;
                split8(x.b[u], h, l);
                *reinterpret_cast<v8bf *>(sb + kBStep * u) = h;
                *reinterpret_cast<v8bf *>(sb + kPlaneB + kBStep * u) = l;
            }
        };
        // Rows past M / N and k past K read as zero: selects only on edge
        // tiles and the last stage (uniform branch, no load inside it).
        const bool edge = m0 + TM > p.M || n0 + TN > p.N;
        auto put = [&](const WsSlice &x, uint32_t s) {
            const uint32_t slot = s % kSlots;
            const uint32_t k0 = (ks0 + s) * WBK;
            if (s >= kSlots) ws_wait(p, cons + 4 * slot, s - kSlots + 1);
            if (edge || k0 + WBK > p.K) {
                WsSlice y;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const uint32_t kb = k0 + 8 * (pt & 3);
#pragma unroll
                    for (int e = 0; e < 8; ++e) y.a[u][e] = (a_ok[u] && kb + e < p.K) ? x.a[u][e] : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const uint32_t kb = k0 + 8 * (TB ? (pt & 3) : (pt >> 6));
#pragma unroll
                    for (int e = 0; e < 8; ++e) y.b[u][e] = (b_ok[u] && kb + e < p.K) ? x.b[u][e] : 0.0f;
                }
                write(y, slot);
            } else {
                write(x, slot);
            }
            ws_release(prod + 4 * slot + pw, s + 1);
        };
        WsSlice x0, x1, x2;
        load(x0, 0);
        load(x1, 1);
        for (uint32_t s = 0; s < KT; s += 3) {
            load(x2, s + 2);
            put(x0, s);
            load(x0, s + 3);
            if (s + 1 < KT) put(x1, s + 1);
            load(x1, s + 4);
            if (s + 2 < KT) put(x2, s + 2);
        }
        return;
    }

    // ---------------- consumers ----------------
    const int cw = wave, wm = cw >> 1, wn = cw & 1;
    const int h = lane >> 5, col = lane & 31;
    struct Frag {
        v8bf ah[4], al[4], bh[2], bl[2];
    };
    // Rows wm*128 + 32i + col of A and wn*64 + 32j + col of B all have the
    // swizzle (col/4) & 3: per k16 step one lane base each, row tiles and
    // planes are immediates.
    uint32_t a_lane[2], b_lane[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
        const uint32_t sw = (((2 * s2 + h) ^ ((col >> 2) & 3)) << 4);
        a_lane[s2] = (wm * 128 + col) * (WBK * 2) + sw;
        b_lane[s2] = 2 * kPlaneA + (wn * 64 + col) * (WBK * 2) + sw;
    }
    auto read = [&](Frag &f, uint32_t s, int s2) {
        const int8_t *pa = smem + (s % kSlots) * kSlotBytes + a_lane[s2];
        const int8_t *pb = smem + (s % kSlots) * kSlotBytes + b_lane[s2];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f.ah[i] = *reinterpret_cast<const v8bf *>(pa + 2048 * i);
            f.al[i] = *reinterpret_cast<const v8bf *>(pa + kPlaneA + 2048 * i);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            f.bh[j] = *reinterpret_cast<const v8bf *>(pb + 2048 * j);
            f.bl[j] = *reinterpret_cast<const v8bf *>(pb + kPlaneB + 2048 * j);
        }
    };
    v16f acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (v16f){0.f};
    // Three passes over the eight accumulators (cross terms first): an MFMA
    // never waits for the one just issued into the same accumulator.
    auto mma = [&](const Frag &f) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.al[i], f.bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.ah[i], f.bl[j], acc[i][j], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.ah[i], f.bh[j], acc[i][j], 0, 0, 0);
    };
    Frag f0, f1;
    ws_wait(p, prod, 1);
    read(f0, 0, 0);
    for (uint32_t s = 0; s < KT; ++s) {
        read(f1, s, 1);
        mma(f0);
        ws_release(cons + 4 * (s % kSlots) + cw, s + 1);
        if (s + 1 < KT) {
            ws_wait(p, prod + 4 * ((s + 1) % kSlots), s + 2);
            read(f0, s + 1, 0);
        }
        mma(f1);
    }
    // Rows wm*128 + 64q .. +63 of the block: the split-bf16 kernel's register
    // epilogue, twice; a K-split workgroup stores its raw sums (alpha 1, no
    // bias, beta 0, no activation) into its 256 x 128 partial tile instead.
    if (split) {
        F32Gemm t = p;
        t.C = part + static_cast<uint64_t>(blockIdx.x - full) * TM * TN;
        t.M = TM;
        t.N = TN;
        t.ldc = TN;
        t.alpha = 1.0f;
        t.beta = 0.0f;
        t.bias = nullptr;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const v16f pq[2][2] = {{acc[2 * q][0], acc[2 * q][1]}, {acc[2 * q + 1][0], acc[2 * q + 1][1]}};
            x3_store_rows<0, 2>(t, pq, wm * 128 + 64 * q, wn * 64 + col, h);
        }
        return;
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const v16f pq[2][2] = {{acc[2 * q][0], acc[2 * q][1]}, {acc[2 * q + 1][0], acc[2 * q + 1][1]}};
        x3_store_rows_epi<2>(p, pq, m0 + wm * 128 + 64 * q, n0 + wn * 64 + col, h);
    }
}

// The tiles gemm_f32_ws split over K: C = epi(alpha (s_0 + s_1 + ...) +
// bias + beta C), the slices added in order, for split tile blockIdx.y,
// 1024 elements (four per thread) per workgroup.
__global__ __launch_bounds__(kThreads) void gemm_f32_tail_reduce(F32Gemm p, const float *part, uint32_t full,
                                                                 uint32_t splits)
{
    using ws::TM;
    using ws::TN;
    const uint32_t tiles_m = (p.M + TM - 1) / TM, total = tiles_m * ((p.N + TN - 1) / TN);
    uint32_t sp;
    const uint32_t g = ws_tile_of(full + blockIdx.y, full, total, &sp);   // slice 0 of tile blockIdx.y
    const uint32_t m0 = (g % tiles_m) * TM, n0 = (g / tiles_m) * TN;
    const uint32_t e = (blockIdx.x * kThreads + threadIdx.x) * 4;   // element of the 256 x 128 tile
    const uint64_t t2 = total - full, stride = t2 * TM * TN;
    const float *p0 = part + static_cast<uint64_t>(blockIdx.y) * TM * TN + e;
    const uint32_t m = m0 + e / TN, n = n0 + e % TN;
    if (m >= p.M) return;
    float4 a = *reinterpret_cast<const float4 *>(p0);
    for (uint32_t i = 1; i < splits; ++i) {
        const float4 b = *reinterpret_cast<const float4 *>(p0 + i * stride);
        a = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
    }
    const float s4[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (n + i < p.N) store_out(p, m, n + i, s4[i], false);
}

// ---------------------------------------------------------------------------
// Skinny NN path (M <= 8).
// ---------------------------------------------------------------------------
constexpr int kSkinnyCols = 256;  // 64 lanes x float4
constexpr int kSkinnyUnroll = 8;
constexpr int kBufferWord3 = 0x00020000;  // raw buffer, 32-bit data format
constexpr int kNontemporal = 2;           // weights are streamed once

// Rows kb..ke of B in this workgroup's 256 columns, as one bounds-checked
// buffer: lane l of wave w reads row kb + w + 4i at byte (row - kb) * ldb * 4
// + 16 l.  Rows past ke and columns past N in the last row read as zero, so
// the load stream has no branches (a branch around a load makes the waitcnt
// pass drain every load in flight).  Activations are wave-uniform scalars,
// zero for rows past ke.
template <int M>
__global__ __launch_bounds__(kThreads) void gemv_f32_kernel(F32Gemm p, uint32_t k_per_split,
                                                            float *ws, uint32_t splits)
{
    __shared__ float4 red[4][M][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t n0 = blockIdx.x * kSkinnyCols;
    const uint32_t n = n0 + lane * 4;
    const uint32_t kb = blockIdx.y * k_per_split;
    const uint32_t ke = min(p.K, kb + k_per_split);

    const uint64_t row_bytes = static_cast<uint64_t>(p.ldb) * 4;
    const uint64_t span = ke > kb ? (ke - kb - 1) * row_bytes + static_cast<uint64_t>(p.N - n0) * 4 : 0;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(p.B) + static_cast<uint64_t>(kb) * p.ldb + n0, 0,
        static_cast<int>(span), kBufferWord3);

    float4 acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = make_float4(0.f, 0.f, 0.f, 0.f);

    for (uint32_t k = kb + wave; k < ke; k += 4 * kSkinnyUnroll) {
        float4 b[kSkinnyUnroll];
#pragma unroll
        for (int u = 0; u < kSkinnyUnroll; ++u) {
            const uint32_t off = static_cast<uint32_t>((k - kb + u * 4) * row_bytes) + lane * 16;
            b[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kNontemporal));
        }
#pragma unroll
        for (int u = 0; u < kSkinnyUnroll; ++u) {
            const uint32_t kk = k + u * 4;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float a = kk < ke ? p.A[static_cast<uint64_t>(m) * p.lda + kk] : 0.0f;
                acc[m].x = fmaf(a, b[u].x, acc[m].x);
                acc[m].y = fmaf(a, b[u].y, acc[m].y);
                acc[m].z = fmaf(a, b[u].z, acc[m].z);
                acc[m].w = fmaf(a, b[u].w, acc[m].w);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) red[tid >> 6][m][lane] = acc[m];
    __syncthreads();
    if (tid < 64) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float4 s = red[0][m][lane];
#pragma unroll
            for (int w = 1; w < 4; ++w) {
                const float4 t = red[w][m][lane];
                s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
            }
            const float v[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t nn = n + i;
                if (nn >= p.N) continue;
                if (splits > 1)
                    ws[(static_cast<uint64_t>(blockIdx.y) * M + m) * p.N + nn] = v[i];
                else
                    store_out(p, m, nn, v[i], false);
            }
        }
    }
}

__global__ __launch_bounds__(kThreads) void gemv_f32_reduce(F32Gemm p, const float *ws,
                                                            uint32_t splits)
{
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const uint64_t total = static_cast<uint64_t>(p.M) * p.N;
    if (idx >= total) return;
    const uint32_t m = static_cast<uint32_t>(idx / p.N), n = static_cast<uint32_t>(idx % p.N);
    // Partials in groups of eight whose loads are issued together (one round
    // trip per group), summed in split order.
    constexpr uint32_t G = 8;
    float s = 0.0f;
    for (uint32_t i0 = 0; i0 < splits; i0 += G) {
        float v[G];
#pragma unroll
        for (uint32_t u = 0; u < G; ++u)
            v[u] = i0 + u < splits ? ws[static_cast<uint64_t>(i0 + u) * total + idx] : 0.0f;
#pragma unroll
        for (uint32_t u = 0; u < G; ++u)
            if (i0 + u < splits) s += v[u];
    }
    store_out(p, m, n, s, false);
}

// Wide-N variant (N >= 200 x 128): one workgroup of 16 waves per 128 columns
// and the whole of K, so no split partials and no second pass.  For M > 1 the
// activations are staged once in LDS as at[k][MP] (MP = M rounded up to 4,
// zero padded), so each row's M values are one or two broadcast ds_read_b128
// instead of M scalar loads from a 32-128 KiB region the scalar cache cannot
// hold; one row (16 KiB at K = 4096) stays on scalar loads.  Lane l of wave
// w reads float2 columns n0 + 2l .. +1 of rows w + 16i (kWideUnroll of them
// in flight per wave); rows past K and columns past N in the last row read as
// zero through the buffer's bounds check.  The 16 wave sums are added in wave
// order in LDS, over the staged activations.
constexpr int kWideCols = 128;  // 64 lanes x float2
constexpr int kWideWaves = 16;
constexpr int kWideUnroll = 16;
constexpr uint32_t kWideMinBlocks = 200;
constexpr uint32_t kWideMaxLds = 128 * 1024;

__host__ __device__ constexpr uint32_t wide_mp(int M) { return (M + 3) & ~3; }

template <int M>
__host__ __device__ constexpr uint32_t wide_red_bytes() { return kWideWaves * M * 64 * 8; }

template <int M>
__global__ __launch_bounds__(64 * kWideWaves) void gemv_f32_wide(F32Gemm p)
{
    constexpr uint32_t MP = wide_mp(M);
    extern __shared__ float4 wide_lds[];
    float *at = reinterpret_cast<float *>(wide_lds);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t n0 = blockIdx.x * kWideCols;
    const uint64_t row_bytes = static_cast<uint64_t>(p.ldb) * 4;
    const uint64_t span = (p.K - 1) * row_bytes + static_cast<uint64_t>(p.N - n0) * 4;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(p.B) + n0, 0, static_cast<int>(span), kBufferWord3);

    if constexpr (M > 1) {
#pragma unroll
        for (uint32_t m = 0; m < MP; ++m)
            for (uint32_t k = tid; k < p.K; k += 64 * kWideWaves)
                at[k * MP + m] = m < M ? p.A[static_cast<uint64_t>(m) * p.lda + k] : 0.0f;
        __syncthreads();
    }

    float2 acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = make_float2(0.f, 0.f);
    auto load_rows = [&](float2 (&b)[kWideUnroll], uint32_t k) {
#pragma unroll
        for (int u = 0; u < kWideUnroll; ++u) {
            const uint32_t off = static_cast<uint32_t>((k + u * kWideWaves) * row_bytes) + lane * 8;
            b[u] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, kNontemporal));
        }
    };
    // all_in: every row of the set is below K (no per-row selects).
    auto fma_rows = [&](const float2 (&b)[kWideUnroll], uint32_t k, auto all_in) {
#pragma unroll
        for (int u = 0; u < kWideUnroll; ++u) {
            const uint32_t kk = k + u * kWideWaves;
            const bool in = decltype(all_in)::value || kk < p.K;
            if constexpr (M == 1) {
                const float a = in ? p.A[kk] : 0.0f;
                acc[0].x = fmaf(a, b[u].x, acc[0].x);
                acc[0].y = fmaf(a, b[u].y, acc[0].y);
                continue;
            }
            const float4 *ar = reinterpret_cast<const float4 *>(at + (in ? kk : p.K - 1) * MP);
            float av[MP];
#pragma unroll
            for (uint32_t q = 0; q < MP / 4; ++q) {
                const float4 t = ar[q];
                av[4 * q] = t.x; av[4 * q + 1] = t.y; av[4 * q + 2] = t.z; av[4 * q + 3] = t.w;
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float a = in ? av[m] : 0.0f;
                acc[m].x = fmaf(a, b[u].x, acc[m].x);
                acc[m].y = fmaf(a, b[u].y, acc[m].y);
            }
        }
    };
    // Two register sets of kWideUnroll rows: the next set's loads are issued
    // before the current set's FMAs.
    constexpr uint32_t kStep = kWideWaves * kWideUnroll;
    float2 b0[kWideUnroll], b1[kWideUnroll];
    uint32_t k = wave;
    if (k < p.K) load_rows(b0, k);
    using yes = std::true_type;
    using no = std::false_type;
    for (; k < p.K; k += 2 * kStep) {
        load_rows(b1, k + kStep);
        if (k + kStep <= p.K) fma_rows(b0, k, yes{}); else fma_rows(b0, k, no{});
        if (k + kStep >= p.K) break;
        load_rows(b0, k + 2 * kStep);
        if (k + 2 * kStep <= p.K) fma_rows(b1, k + kStep, yes{}); else fma_rows(b1, k + kStep, no{});
    }
    __syncthreads();  // every wave is done with at[] before red[] reuses it
    float2 *red = reinterpret_cast<float2 *>(wide_lds);  // [wave][m][lane]
#pragma unroll
    for (int m = 0; m < M; ++m) red[(wave * M + m) * 64 + lane] = acc[m];
    __syncthreads();
    if (tid < M * kWideCols) {
        const uint32_t m = tid / kWideCols, c = tid % kWideCols;
        const float *r = reinterpret_cast<const float *>(red) + m * kWideCols + c;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kWideWaves; ++w) v += r[static_cast<size_t>(w) * M * kWideCols];
        if (n0 + c < p.N) store_out(p, m, n0 + c, v, false);
    }
}

template <int M>
uint32_t wide_lds_bytes(const F32Gemm &p)
{
    const uint32_t a = M > 1 ? p.K * wide_mp(M) * 4 : 0;
    return a > wide_red_bytes<M>() ? a : wide_red_bytes<M>();
}

template <int M>
bool wide_lds_optin()
{
    static std::atomic<bool> done{false};  // launches may come from several host threads
    if (!done)
        done = hipFuncSetAttribute(reinterpret_cast<const void *>(gemv_f32_wide<M>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
    return done;
}

bool wide_lds_optin(uint32_t M)
{
    switch (M) {
    case 1: return wide_lds_optin<1>();
    case 2: return wide_lds_optin<2>();
    case 3: return wide_lds_optin<3>();
    case 4: return wide_lds_optin<4>();
    case 5: return wide_lds_optin<5>();
    case 6: return wide_lds_optin<6>();
    case 7: return wide_lds_optin<7>();
    case 8: return wide_lds_optin<8>();
    default: return false;
    }
}

// The wide variant needs float2-aligned rows (even N and ldb, 8-byte B),
// enough column blocks to fill the chip, the staged activations within
// kWideMaxLds (K <= 8192 for M of 2 to 4, 4096 above), and its last two
// batches of rows (up to 2 * kWideWaves * kWideUnroll past K) addressable with
// 32-bit offsets; LDS above 64 KiB is opted into once per kernel.
bool use_wide(const F32Gemm &p)
{
    const uint64_t row_bytes = static_cast<uint64_t>(p.ldb) * 4;
    return p.N % 2 == 0 && p.ldb % 2 == 0 && reinterpret_cast<uintptr_t>(p.B) % 8 == 0 &&
           (p.N + kWideCols - 1) / kWideCols >= kWideMinBlocks &&
           (p.M == 1 || static_cast<uint64_t>(p.K) * wide_mp(p.M) * 4 <= kWideMaxLds) &&
           (static_cast<uint64_t>(p.K) + 2 * kWideWaves * kWideUnroll) * row_bytes < 0x7fffffffull &&
           wide_lds_optin(p.M);
}

// K split: enough workgroups to keep the weight stream in flight, and each
// workgroup's buffer (its rows of B, plus the rows a final partial batch
// reads past them) addressable with 32-bit offsets.
struct SkinnyPlan {
    uint32_t splits, kps;
};

SkinnyPlan skinny_plan(const F32Gemm &p)
{
    const uint32_t col_blocks = (p.N + kSkinnyCols - 1) / kSkinnyCols;
    uint32_t want = 1;
    while (col_blocks * want < 1024 && p.K / (want * 2) >= 256) want *= 2;
    const uint64_t row_bytes = static_cast<uint64_t>(p.ldb) * 4;
    const uint64_t max_rows = (0x7fffffffull / row_bytes) - 4 * kSkinnyUnroll;
    uint64_t kps = (p.K + want - 1) / want;
    if (kps > max_rows) kps = max_rows;
    SkinnyPlan plan;
    plan.kps = static_cast<uint32_t>(kps);
    plan.splits = static_cast<uint32_t>((p.K + kps - 1) / kps);
    return plan;
}

template <int M>
void launch_skinny(hipStream_t s, const F32Gemm &p, float *ws)
{
    if (use_wide(p)) {
        gemv_f32_wide<M><<<dim3((p.N + kWideCols - 1) / kWideCols), 64 * kWideWaves, wide_lds_bytes<M>(p), s>>>(p);
        return;
    }
    const SkinnyPlan plan = skinny_plan(p);
    dim3 grid((p.N + kSkinnyCols - 1) / kSkinnyCols, plan.splits);
    gemv_f32_kernel<M><<<grid, kThreads, 0, s>>>(p, plan.kps, ws, plan.splits);
    if (plan.splits > 1) {
        const uint64_t total = static_cast<uint64_t>(p.M) * p.N;
        gemv_f32_reduce<<<dim3(static_cast<uint32_t>((total + kThreads - 1) / kThreads)), kThreads, 0, s>>>(
            p, ws, plan.splits);
    }
}

}  // namespace

void gemm_f32_tile_dims(uint32_t &bm, uint32_t &bn)
{
    bm = BM;
    bn = BN;
}

namespace {

// Cull grid tile (mi, ni) samples the mask at (mi * mask_m / mt,
// ni * mask_n / nt), as the host path and the reference's geometry do; one
// count per wave goes to *culled.
__global__ __launch_bounds__(kThreads) void cull_map_kernel(const uint8_t *__restrict__ mask, uint32_t mask_m,
                                                            uint32_t mask_n, uint32_t mt, uint32_t nt,
                                                            uint8_t *__restrict__ cull,
                                                            unsigned long long *__restrict__ culled)
{
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    bool c = false;
    if (i < static_cast<uint64_t>(mt) * nt) {
        const uint32_t mi = static_cast<uint32_t>(i / nt), ni = static_cast<uint32_t>(i % nt);
        const uint32_t mm = min(mask_m - 1, static_cast<uint32_t>((static_cast<uint64_t>(mi) * mask_m) / mt));
        const uint32_t nn = min(mask_n - 1, static_cast<uint32_t>((static_cast<uint64_t>(ni) * mask_n) / nt));
        c = mask[static_cast<uint64_t>(mm) * mask_n + nn] == 0;
        cull[i] = c ? 1 : 0;
    }
    const uint64_t n = __popcll(__ballot(c));
    if ((threadIdx.x & 63) == 0 && n) atomicAdd(culled, static_cast<unsigned long long>(n));
}

// Kernel tile (gi, gj) of BM x BN outputs: compute (0), all culled (1) or
// mixed (2) over the cull tiles it overlaps.
__global__ __launch_bounds__(kThreads) void cull_state_kernel(const uint8_t *__restrict__ cull, uint32_t nt,
                                                              uint32_t M, uint32_t N, uint32_t tm, uint32_t tn,
                                                              uint32_t gm, uint32_t gn, uint8_t *__restrict__ state)
{
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= static_cast<uint64_t>(gm) * gn) return;
    const uint32_t gi = static_cast<uint32_t>(i / gn), gj = static_cast<uint32_t>(i % gn);
    const uint32_t r0 = gi * BM / tm, r1 = (min(M, (gi + 1) * BM) - 1) / tm;
    const uint32_t c0 = gj * BN / tn, c1 = (min(N, (gj + 1) * BN) - 1) / tn;
    bool any_c = false, any_k = false;
    for (uint32_t r = r0; r <= r1; ++r)
        for (uint32_t c = c0; c <= c1; ++c) {
            if (cull[static_cast<uint64_t>(r) * nt + c]) any_c = true;
            else any_k = true;
        }
    state[i] = any_c ? (any_k ? 2 : 1) : 0;
}

}  // namespace

void cull_classify(hipStream_t s, const uint8_t *mask, uint32_t mask_m, uint32_t mask_n, uint32_t M, uint32_t N,
                   uint32_t tm, uint32_t tn, uint8_t *cull, uint8_t *state, unsigned long long *culled)
{
    const uint32_t mt = (M + tm - 1) / tm, nt = (N + tn - 1) / tn;
    const uint32_t gm = (M + BM - 1) / BM, gn = (N + BN - 1) / BN;
    const uint64_t n1 = static_cast<uint64_t>(mt) * nt, n2 = static_cast<uint64_t>(gm) * gn;
    cull_map_kernel<<<dim3(static_cast<uint32_t>((n1 + kThreads - 1) / kThreads)), kThreads, 0, s>>>(
        mask, mask_m, mask_n, mt, nt, cull, culled);
    cull_state_kernel<<<dim3(static_cast<uint32_t>((n2 + kThreads - 1) / kThreads)), kThreads, 0, s>>>(
        cull, nt, M, N, tm, tn, gm, gn, state);
}

// Grids of fewer than 128 tiles leave most CUs idle: split K over up to
// 256 workgroups, at least 64 deep each (not with a cull map, whose per-tile
// state is read by the single-pass kernel).
// A requested K depth (device tiles 128 x depth x 128) is honoured up to a
// split-K workspace of kMaxSplitWs bytes; deeper slices beyond that.
constexpr uint64_t kMaxSplitWs = 256ull << 20;

static uint32_t gemm_f32_splits(const F32Gemm &p)
{
    if (p.ktile_state || p.cull) return 1;
    if (p.k_split_depth >= BK && p.k_split_depth < p.K) {
        const uint64_t per_split = static_cast<uint64_t>(p.M) * p.N * sizeof(float);
        const uint64_t cap = std::max<uint64_t>(1, kMaxSplitWs / per_split);
        return static_cast<uint32_t>(
            std::min<uint64_t>(std::min<uint64_t>(256, cap), (p.K + p.k_split_depth - 1) / p.k_split_depth));
    }
    if (p.k_split_depth >= p.K) return 1;
    const uint32_t tiles = ((p.N + BN - 1) / BN) * ((p.M + BM - 1) / BM);
    uint32_t splits = 1;
    while (tiles * splits < 256 && p.K / (splits * 2) >= 64) splits *= 2;
    return tiles >= 128 ? 1 : splits;
}

// The split-bf16 kernel takes every MATMUL_F32 without a cull map or a
// requested K depth on 16-byte aligned operands.  Grids of fewer than 128
// tiles of 128 x 128 split K over workgroups (32-deep stages, at least two
// per slice) until the grid has 128 or more, with the partial sums reduced
// in slice order by a second pass.
// Grid targets (swept on MI355X, 256 CUs).  The lock-step four-wave kernel
// splits K until it has kX3Grid workgroups (two per CU): against 128, at
// 1024x4096x2048 206 -> 97 us, 2048^3 109 -> 100 us, 1024x1024x2048 78 -> 40
// us (256 and 1024 were slower).  The warp-specialised kernel takes grids of
// fewer 256 x 128 tiles than CUs when slices of K of at least kWsMinStages
// stages bring them to kWsMinGrid workgroups.
constexpr uint64_t kX3Grid = 512;
constexpr uint32_t kWsMinStages = 16;
constexpr uint64_t kWsMinGrid = 192;

// K slices per tile for a grid of `tiles` 256 x 128 tiles below the CU count:
// as many as fill the CUs, each of at least kWsMinStages stages (1: none).
static uint32_t ws_slices(uint64_t tiles, uint32_t K)
{
    const uint32_t cus = std::max<uint32_t>(1, cu_count());
    const uint32_t kt = (K + ws::BK - 1) / ws::BK;
    if (!tiles || tiles >= cus) return 1;
    return std::max<uint32_t>(1, std::min<uint32_t>(static_cast<uint32_t>(cus / tiles), kt / kWsMinStages));
}

// How the warp-specialised kernel covers its tiles: the first `full` whole,
// the rest as `splits` K slices of ks_per stages each.  A last round that
// would fill at most half the CUs is split in two (its round then takes half
// as long); a grid of fewer tiles than CUs is split by ws_slices.
struct WsSplit {
    uint32_t total, full, splits, ks_per, kt;
};
static WsSplit ws_split(const F32Gemm &p)
{
    WsSplit w;
    w.total = ((p.M + ws::TM - 1) / ws::TM) * ((p.N + ws::TN - 1) / ws::TN);
    w.kt = (p.K + ws::BK - 1) / ws::BK;
    w.full = w.total;
    w.splits = 1;
    const uint32_t cus = std::max<uint32_t>(1, cu_count()), rest = w.total % cus;
    if (w.total < cus) {
        w.splits = ws_slices(w.total, p.K);
        if (w.splits > 1) w.full = 0;
    } else if (rest && rest <= cus / 2 && w.kt >= 16) {
        w.full = w.total - rest;
        w.splits = 2;
    }
    w.ks_per = (w.kt + w.splits - 1) / w.splits;
    w.splits = (w.kt + w.ks_per - 1) / w.ks_per;   // every slice has at least one stage
    if (w.splits == 1) w.full = w.total;
    return w;
}

struct X3Plan {
    bool x3 = false;
    bool ws = false;   // the warp-specialised 256 x 128 kernel (op(A) = A)
    int wm = 2;
    uint32_t splits = 1, kps = 0;
};

static X3Plan x3_plan(const F32Gemm &p)
{
    X3Plan x;
    const bool al = (p.lda % 4 == 0) && (p.ldb % 4 == 0) && (reinterpret_cast<uintptr_t>(p.A) % 16 == 0) &&
                    (reinterpret_cast<uintptr_t>(p.B) % 16 == 0);
    if (p.cull || p.ktile_state || p.k_split_depth != 0 || !al) return x;
    x.x3 = true;
    x.kps = p.K;
    const uint64_t tiles = static_cast<uint64_t>((p.M + 127) / 128) * ((p.N + x3::TN - 1) / x3::TN);
    // 256 x 128 tiles (eight waves) when they still give every CU one: each
    // workgroup splits an A slice once for 128 columns and a B slice once
    // for 256 rows (a quarter less conversion per MFMA).
    const uint64_t tiles256 = static_cast<uint64_t>((p.M + 255) / 256) * ((p.N + x3::TN - 1) / x3::TN);
    const uint64_t a_bytes = static_cast<uint64_t>(p.M) * p.lda * 4;
    const uint64_t b_bytes = static_cast<uint64_t>(p.trans_b ? p.N : p.K) * p.ldb * 4;
    // The warp-specialised kernel reads A and B through 31-bit buffer ranges.
    const bool ws_ok = !p.trans_a && a_bytes < (1ull << 31) && b_bytes < (1ull << 31);
    if (tiles256 >= 256) {
        x.wm = 4;
        x.ws = ws_ok;
    } else if (ws_ok && tiles256 * ws_slices(tiles256, p.K) >= kWsMinGrid) {
        // fewer tiles than CUs, but K slices of at least kWsMinStages fill
        // three quarters of the CUs or more
        x.wm = 4;
        x.ws = true;
        return x;
    }
    // The lock-step kernel splits K until the grid has two workgroups per CU.
    if (x.ws || tiles >= kX3Grid) return x;
    uint32_t want = 1;
    while (tiles * want < kX3Grid && p.K / (want * 2) >= 2 * x3::BK) want *= 2;
    const uint64_t per_split = static_cast<uint64_t>(p.M) * p.N * sizeof(float);
    want = static_cast<uint32_t>(std::min<uint64_t>(want, std::max<uint64_t>(1, kMaxSplitWs / per_split)));
    if (want > 1) {
        x.kps = ((p.K + want - 1) / want + x3::BK - 1) / x3::BK * x3::BK;
        x.splits = (p.K + x.kps - 1) / x.kps;   // every slice starts below K
    }
    return x;
}

template <int WM>
static void launch_x3(hipStream_t s, const F32Gemm &p, const X3Plan &x, float *ws)
{
    static std::atomic<bool> lds_optin{false};  // launches may come from several host threads
    constexpr int lds = x3::lds_bytes(WM);
    if (!lds_optin)
        lds_optin = hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_f32_x3<false, false, WM>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, lds) == hipSuccess &&
                    hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_f32_x3<false, true, WM>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, lds) == hipSuccess &&
                    hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_f32_x3<true, false, WM>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, lds) == hipSuccess &&
                    hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_f32_x3<true, true, WM>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, lds) == hipSuccess;
    const dim3 grid(((p.N + x3::TN - 1) / x3::TN) * ((p.M + 64 * WM - 1) / (64 * WM)), x.splits);
    const dim3 block(128 * WM);
    float *out = x.splits > 1 ? ws : nullptr;
    if (!p.trans_a && !p.trans_b) gemm_f32_x3<false, false, WM><<<grid, block, lds, s>>>(p, x.kps, out);
    else if (!p.trans_a) gemm_f32_x3<false, true, WM><<<grid, block, lds, s>>>(p, x.kps, out);
    else if (!p.trans_b) gemm_f32_x3<true, false, WM><<<grid, block, lds, s>>>(p, x.kps, out);
    else gemm_f32_x3<true, true, WM><<<grid, block, lds, s>>>(p, x.kps, out);
}

size_t gemm_f32_ws_bytes(const F32Gemm &p)
{
    const X3Plan x = x3_plan(p);
    if (x.ws) {
        const WsSplit w = ws_split(p);
        return static_cast<size_t>(w.total - w.full) * w.splits * ws::TM * ws::TN * sizeof(float);
    }
    const uint32_t splits = x.x3 ? x.splits : gemm_f32_splits(p);
    return splits > 1 ? static_cast<size_t>(splits) * p.M * p.N * sizeof(float) : 0;
}

static void splitk_reduce(hipStream_t s, const F32Gemm &p, const float *ws, uint32_t splits)
{
    const uint64_t total = static_cast<uint64_t>(p.M) * p.N;
    gemm_f32_splitk_reduce<<<dim3(static_cast<uint32_t>((total + kThreads - 1) / kThreads)), kThreads, 0, s>>>(
        p, ws, splits);
}

void gemm_f32(hipStream_t s, const F32Gemm &p, float *ws)
{
    const X3Plan x = x3_plan(p);
    if (x.ws) {
        static std::atomic<bool> lds_optin{false};  // launches may come from several host threads
        if (!lds_optin)
            lds_optin = hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_f32_ws<false>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, ws::kLds) == hipSuccess &&
                        hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_f32_ws<true>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, ws::kLds) == hipSuccess;
        WsSplit w = ws_split(p);
        if (!ws) w = WsSplit{w.total, w.total, 1, w.kt};   // no workspace: every tile whole
        const uint32_t tail = w.total - w.full;
        const dim3 grid(w.full + tail * w.splits);
        if (p.trans_b) gemm_f32_ws<true><<<grid, 512, ws::kLds, s>>>(p, w.full, w.ks_per, ws);
        else gemm_f32_ws<false><<<grid, 512, ws::kLds, s>>>(p, w.full, w.ks_per, ws);
        if (tail)
            gemm_f32_tail_reduce<<<dim3(ws::TM * ws::TN / (4 * kThreads), tail), kThreads, 0, s>>>(p, ws, w.full,
                                                                                                    w.splits);
        return;
    }
    if (x.x3) {
        if (x.wm == 4) launch_x3<4>(s, p, x, ws);
        else launch_x3<2>(s, p, x, ws);
        if (x.splits > 1) splitk_reduce(s, p, ws, x.splits);
        return;
    }
    const uint32_t want = gemm_f32_splits(p);
    const uint32_t kps = want > 1 ? ((p.K + want - 1) / want + BK - 1) / BK * BK : p.K;
    // Every z slice starts below K (rounding kps up may leave fewer slices).
    const uint32_t splits = want > 1 ? (p.K + kps - 1) / kps : 1;
    dim3 grid((p.N + BN - 1) / BN, (p.M + BM - 1) / BM, splits);
    gemm_f32_kernel<<<grid, kThreads, 0, s>>>(p, kps, splits > 1 ? ws : nullptr);
    if (splits > 1) splitk_reduce(s, p, ws, splits);
}

size_t gemv_f32_ws_bytes(const F32Gemm &p)
{
    if (use_wide(p)) return 0;
    const SkinnyPlan plan = skinny_plan(p);
    return plan.splits > 1 ? static_cast<size_t>(plan.splits) * p.M * p.N * sizeof(float) : 0;
}

bool gemv_f32_supported(const F32Gemm &p)
{
    // 33 rows of B must be addressable with 32-bit offsets
    return static_cast<uint64_t>(p.ldb) * 4 * (4 * kSkinnyUnroll + 1) < 0x7fffffffull;
}

void gemv_f32(hipStream_t s, const F32Gemm &p, float *ws)
{
    switch (p.M) {
    case 1: launch_skinny<1>(s, p, ws); break;
    case 2: launch_skinny<2>(s, p, ws); break;
    case 3: launch_skinny<3>(s, p, ws); break;
    case 4: launch_skinny<4>(s, p, ws); break;
    case 5: launch_skinny<5>(s, p, ws); break;
    case 6: launch_skinny<6>(s, p, ws); break;
    case 7: launch_skinny<7>(s, p, ws); break;
    case 8: launch_skinny<8>(s, p, ws); break;
    default: break;
    }
}

}  // namespace k
}  // namespace vnpu
