// kernels.hpp - host-side launchers for the gfx950 kernels.
//
// Every launcher only enqueues work on the given stream; the command
// processor (dispatch.cpp) has already validated shapes, so each launcher's
// grid covers exactly the buffers described by its arguments.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace vnpu {
namespace k {

// ---- QUANTIZE_I8 (quantize.hip) ----
void quantize_rows(hipStream_t s, const float *X, int8_t *Y, float *scales, uint64_t rows,
                   uint64_t cols);
// ws must hold quantize_cols_ws_bytes(cols) bytes (per-column maxima).
size_t quantize_cols_ws_bytes(uint64_t cols);
void quantize_cols(hipStream_t s, const float *X, int8_t *Y, float *scales, uint64_t rows,
                   uint64_t cols, uint32_t *ws);
// ws must hold quantize_tensor_ws_bytes() bytes.
size_t quantize_tensor_ws_bytes();
void quantize_tensor(hipStream_t s, const float *X, int8_t *Y, float *scales, uint64_t count,
                     float *ws);

// ---- PACK_WEIGHTS_I8 (pack.hip) ----
// Writes the fragment layout [Np/16][Kp/64][4][16][16] (zero padded) and the
// per-column sums [N].  A non-null tile_mask ([Kp/64][mask_ld] bytes, device
// memory) packs the 64 x 64 tiles whose byte is zero as zeros.
void pack_fragments(hipStream_t s, const int8_t *B, uint32_t K, uint32_t N, uint32_t ldb,
                    uint32_t trans_b, const uint8_t *tile_mask, uint32_t mask_ld, int8_t *frag,
                    uint32_t Kp, uint32_t Np, int32_t *column_sums);
// The nonzero 64 x 64 weight tiles of packed fragments: for each group g of
// four 16-column strips, list[g][0 .. count[g]) = its k blocks (64 deep)
// holding a nonzero, ascending (flag: [groups][Kp/64] bytes of scratch;
// list: [groups][Kp/64], count: [groups], groups = ceil(Np / 64)).
void tile_lists(hipStream_t s, const int8_t *frag, uint32_t Kp, uint32_t Np, uint8_t *flag, uint32_t *list,
                uint32_t *count);

// Compute units of the current device (read once per process; 256 if the
// query fails).  Launch shapes are chosen in whole rounds of these.
uint32_t cu_count();

// ---- MATMUL_I8 (gemv_i8.hip, gemm_i8.hip) ----
struct I8Gemm {
    const int8_t *A = nullptr;   // [M][lda]
    uint32_t lda = 0;
    const int8_t *frag = nullptr;
    uint32_t Kp = 0, Np = 0;
    const float *scale_a = nullptr;  // [M] or null
    const float *scale_b = nullptr;  // [Np]
    const float *bias = nullptr;     // [N] or null
    float *C = nullptr;              // [M][ldc]
    uint32_t ldc = 0;
    uint32_t M = 0, N = 0, K = 0;
    uint32_t epilogue = 0;
    uint32_t variant = 0;            // kI8*: which prefill kernel (0 = choose)
    // Nonzero 64 x 64 weight tiles (tile_lists): per group of four strips,
    // the k blocks the strip kernel walks; nz_tiles of (groups x Kp/64) are
    // nonzero.  Null lists: every block is walked (dense kernels).
    const uint32_t *nz_list = nullptr, *nz_count = nullptr;
    uint64_t nz_tiles = 0;
    // An ADD_F32 of the output fused into the store (GEMV path, M <= 8, C
    // contiguous): res_out[m*N + n] = fma(x, res_alpha, y * res_beta) with
    // (x, y) = (res[m*N + n], c), or (c, res[...]) when res_c_first; C is
    // stored as well.  Null res: no fused add.
    const float *res = nullptr;
    float *res_out = nullptr;
    float res_alpha = 1.0f, res_beta = 1.0f;
    uint32_t res_c_first = 0;
};
struct I8GemmPair {
    I8Gemm p[2];
};
// Prefill kernels (gemm_i8.hip): a requested one that cannot take the shape
// falls back to the automatic choice.
enum : uint32_t { kI8Auto = 0, kI8Wide = 1, kI8Wave8 = 2, kI8Pipe = 3, kI8Generic = 4, kI8Wide192 = 5, kI8Strip = 6 };
// vnpu_device_set_tiles / autotune: tile triples (M, K, N) that name a kernel
// select it: 256x128x256 wide, 256x128x128 8-wave, 256x64x128 64-deep,
// 128x64x128 generic; anything else chooses automatically.
uint32_t gemm_i8_variant_for_tiles(uint32_t tile_m, uint32_t tile_k, uint32_t tile_n);
// Weight-streaming path for few rows: v_dot4 up to 4 rows, the int8 matrix
// core from 5 to kGemvMaxRows rows.  It takes every MATMUL_I8 below 64 rows
// (the GEMM kernels' 64-row tiles need M >= 64; below that they fell back to
// the generic kernel, 9..48 rows 71-77 us where this runs 6-12 us at
// 4096 x 4096) and 64 rows below 512 column strips (at 11008 and 32000
// columns the 256 x 128 GEMM tiles are faster: 24 / 33 against 33 / 79 us).
constexpr uint32_t kGemvMaxRows = 64;
inline bool gemv_i8_takes(uint32_t M, uint32_t N)
{
    return M < kGemvMaxRows || (M == kGemvMaxRows && N < 512 * 16);
}
void gemv_i8(hipStream_t s, const I8Gemm &p);
// Any M, int8 MFMA; ws holds gemm_i8_ws_bytes(p) (the strip kernel's A in
// fragment blocks; nothing for the dense kernels, where ws may be null).
size_t gemm_i8_ws_bytes(const I8Gemm &p);
void gemm_i8(hipStream_t s, const I8Gemm &p, int8_t *ws);
// Two independent MATMUL_I8 problems with the same M in one wide-tile grid
// when that runs fewer whole rounds of tiles; false (nothing launched) when
// either cannot take the wide kernel or one grid would not be faster.
bool gemm_i8_pair(hipStream_t s, const I8Gemm &p0, const I8Gemm &p1);
// Two M <= 8 problems with the same M (5..8) and K, whose strip counts take
// the same matrix-core GEMV variant, in one grid; false: nothing launched.
bool gemv_i8_pair(hipStream_t s, const I8Gemm &p0, const I8Gemm &p1);

// ---- MATMUL_F32 (gemm_f32.hip) ----
struct F32Gemm {
    const float *A = nullptr, *B = nullptr, *bias = nullptr;
    float *C = nullptr;
    uint32_t M = 0, K = 0, N = 0;
    uint32_t lda = 0, ldb = 0, ldc = 0;
    uint32_t trans_a = 0, trans_b = 0;
    float alpha = 1.0f, beta = 0.0f;
    uint32_t epilogue = 0;
    // Wildcat cull: a grid of (cull_tm x cull_tn) output tiles, cull_nt tiles
    // per row of the grid, one byte per tile (1 = culled).  Null = no cull.
    const uint8_t *cull = nullptr;
    uint32_t cull_tm = 0, cull_tn = 0, cull_nt = 0;
    // Per kernel-tile state derived from the cull grid: 0 compute, 1 fully
    // culled (skip the K loop), 2 mixed.  Null when cull is null.
    const uint8_t *ktile_state = nullptr;
    // K depth per workgroup when a 128 x 128 x depth tile was requested
    // (vnpu_device_set_tiles / autotune); 0 = choose the split automatically.
    uint32_t k_split_depth = 0;
    // The warp-specialised kernel's bounded waits: at most max_spin polls
    // (0 = the kernel's default); a wait that gives up stores 1 into *err
    // (host-coherent, read at the stream's sync).  err may be null.
    uint32_t *err = nullptr;
    uint32_t max_spin = 0;
};
void gemm_f32_tile_dims(uint32_t &bm, uint32_t &bn);
// The Wildcat cull of MATMUL_F32 built on the GPU from a device-resident
// mask (the same sampling and kernel-tile classification as the host path):
// cull[mt][nt] (1 = culled), state[gm][gn] (0 compute, 1 all culled, 2
// mixed); the number of culled tiles is added to *culled.
void cull_classify(hipStream_t s, const uint8_t *mask, uint32_t mask_m, uint32_t mask_n, uint32_t M, uint32_t N,
                   uint32_t tm, uint32_t tn, uint8_t *cull, uint8_t *state, unsigned long long *culled);
// Grids of few tiles split K over workgroups: ws holds gemm_f32_ws_bytes(p)
// bytes (0 when the single-pass kernel is used).
size_t gemm_f32_ws_bytes(const F32Gemm &p);
void gemm_f32(hipStream_t s, const F32Gemm &p, float *ws);
// Skinny path: M <= 8, trans_a == 0, trans_b == 0, no cull, and
// gemv_f32_supported(p) (rows of B short enough for 32-bit buffer offsets).
// ws holds gemv_f32_ws_bytes(p) bytes.
size_t gemv_f32_ws_bytes(const F32Gemm &p);
bool gemv_f32_supported(const F32Gemm &p);
void gemv_f32(hipStream_t s, const F32Gemm &p, float *ws);

// ---- transformer ops (ops.hip) ----
void rmsnorm(hipStream_t s, const float *X, const float *W, float *Y, uint32_t rows,
             uint32_t cols, float eps);
// Few long rows are split over workgroups: ws holds softmax_ws_bytes(rows,
// cols) bytes (0 when one workgroup per row is used).
size_t softmax_ws_bytes(uint32_t rows, uint32_t cols);
void softmax(hipStream_t s, const float *X, float *Y, uint32_t rows, uint32_t cols, float inv_t,
             float *ws);
// inv_freq: device table [head_dim/2] (half-rotation) or [head_dim/2] for the
// interleaved pairs, computed on the host with the reference's powf expression.
void rope(hipStream_t s, float *Q, float *K, const int32_t *positions, uint32_t batch,
          uint32_t heads, uint32_t q_seq, uint32_t k_seq, uint32_t head_dim,
          uint32_t position_offset, uint32_t interleaved, float scaling, const float *inv_freq,
          const float2 *cs, uint32_t cs_rows);
// SWIGLU and MUL round their scalar tails differently: `grain` is the length
// of the reference's ranges (each with its own tail; 0 = one range).  ADD and
// GELU give the same bits in a tail.
void swiglu(hipStream_t s, const float *g, const float *u, float *Y, uint64_t n, float alpha,
            uint64_t grain);
void add(hipStream_t s, const float *A, const float *B, float *Y, uint64_t n, float alpha,
         float beta);
void mul(hipStream_t s, const float *A, const float *B, float *Y, uint64_t n, float alpha,
         float beta, uint64_t grain);
void gelu(hipStream_t s, const float *X, float *Y, uint64_t n);

// A run of row-wise commands over the same rows x cols float rows, executed
// per row in one workgroup with the row held in registers: an optional first
// stage (ADD: Y = A*alpha + B*beta, or SWIGLU: Y = silu(A)*B*alpha), an
// optional RMSNORM (Nrm = X*inv*W, X being Y or, without a first stage, A),
// and an optional per-row QUANTIZE_I8 of the last stage's output.  Every
// stage's output is written, and each stage is the arithmetic of its own
// kernel in the same order, so the results equal the commands run one by one.
// Needs cols % 4 == 0, cols / 4 <= kRowChainMaxVec4, 16-byte aligned float
// rows and W, a 4-byte aligned Q; returns false (nothing launched) otherwise.
enum RowChainPre : uint32_t { kChainNone = 0, kChainAdd = 1, kChainSwiglu = 2 };
constexpr uint32_t kRowChainMaxVec4 = 3072;
struct RowChain {
    uint32_t pre = kChainNone;
    const float *A = nullptr, *B = nullptr;
    float *Y = nullptr;
    float alpha = 1.0f, beta = 1.0f;
    uint64_t grain = 0;    // SWIGLU: range length of the rows * cols command (as k::swiglu)
    const float *W = nullptr;
    float *Nrm = nullptr;  // null: no RMSNORM
    float eps = 1e-5f;
    int8_t *Q = nullptr;   // null: no QUANTIZE_I8
    float *scales = nullptr;
    uint32_t rows = 0, cols = 0;
};
bool row_chain(hipStream_t s, const RowChain &p);

// ---- ATTENTION_F32 (attention.hip) ----
struct Attn {
    const float *Q = nullptr, *K = nullptr, *V = nullptr, *mask = nullptr;
    float *O = nullptr;
    uint32_t batch = 0, heads = 0, seq_q = 0, seq_k = 0, head_dim = 0, causal = 0;
    float scale = 1.0f;
    bool exact = false;   // the reference's order of roundings (bit for bit)
};
size_t attention_ws_bytes(const Attn &a);
void attention(hipStream_t s, const Attn &a, float *ws);
// Reference-order prefill (exact, seq_q > 4, head_dim 64 or 128) on the fp32
// matrix cores (attn_exact.hip).
void attention_exact_prefill(hipStream_t s, const Attn &a);
// Reference-order decode (exact, seq_q <= 4, head_dim 64 or 128): scores,
// then the output chain (attn_exact.hip); ws holds
// attention_exact_decode_ws_bytes(a).
size_t attention_exact_decode_ws_bytes(const Attn &a);
void attention_exact_decode(hipStream_t s, const Attn &a, float *ws);
// The allocation-free attention entry point's device scratch: a file-scope
// array of kAttnScratchBytes in attention.hip, one copy per GPU.  Setup looks
// its address up once per device (that device current) and keeps it;
// attention_scratch returns it (nullptr before setup).
constexpr size_t kAttnScratchBytes = 64ull << 20;
void attention_scratch_setup(int hip_device);
float *attention_scratch(int hip_device);

// ---- fills (ops.hip) ----
void fill_u8(hipStream_t s, void *dst, uint8_t value, uint64_t bytes);

}  // namespace k
}  // namespace vnpu
