// block_harness.hip - the synthetic Llama-style block (libvnpu_block.so).
//
// Harness, not product: it composes vnpu commands exactly as the
// reference's block benchmark does (tools/llm_bench.cpp:213-326), submitted
// in three batches through the backend's vtable, and does the layout work
// the vnpu ABI has no op for - the QKV split into head-major q/k/v
// (llm_bench.cpp:255-268, to_head_major :189-199), the token-major merge of
// the attention output (from_head_major :200-210) and the KV-cache append of
// a decode step - with the HIP kernels below on the same stream, or on the
// host when no hipStream_t is given (the reference's CPU build).
#include <hip/hip_runtime.h>

#include <cstring>
#include <vector>

#include "block_harness.h"

namespace {

// qkv [rows][3d] (row r = b*T + t) -> q, k, v [B][H][T][D]; one float4 per
// thread, grid (chunks of 256 float4 of a row, row groups): a row's index is
// the grid's y (rows past gridDim.y take further trips), so the index math
// is 32-bit with no 64-bit division.
__global__ __launch_bounds__(256) void split_qkv_kernel(const float4 *__restrict__ qkv,
                                                        float4 *__restrict__ q, float4 *__restrict__ k,
                                                        float4 *__restrict__ v, uint32_t rows, uint32_t T,
                                                        uint32_t H, uint32_t D)
{
    const uint32_t d4 = (H * D) >> 2, D4 = D >> 2;   // float4s per q/k/v row part, per head
    const uint32_t c4 = blockIdx.x * 256 + threadIdx.x;
    if (c4 >= 3 * d4) return;
    const uint32_t which = c4 / d4, w4 = c4 - which * d4;
    const uint32_t h = w4 / D4, dd4 = w4 - h * D4;
    float4 *out = which == 0 ? q : which == 1 ? k : v;
    for (uint32_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const uint32_t b = r / T, t = r - b * T;
        out[(static_cast<uint64_t>(b * H + h) * T + t) * D4 + dd4] = qkv[static_cast<uint64_t>(r) * 3 * d4 + c4];
    }
}

// o [B][H][T][D] -> y [rows][H*D]; one float4 per thread (coalesced writes),
// the same grid as split_qkv_kernel.
__global__ __launch_bounds__(256) void merge_heads_kernel(const float4 *__restrict__ o,
                                                          float4 *__restrict__ y, uint32_t rows, uint32_t T,
                                                          uint32_t H, uint32_t D)
{
    const uint32_t d4 = (H * D) >> 2, D4 = D >> 2;
    const uint32_t w4 = blockIdx.x * 256 + threadIdx.x;
    if (w4 >= d4) return;
    const uint32_t h = w4 / D4, dd4 = w4 - h * D4;
    for (uint32_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const uint32_t b = r / T, t = r - b * T;
        y[static_cast<uint64_t>(r) * d4 + w4] = o[(static_cast<uint64_t>(b * H + h) * T + t) * D4 + dd4];
    }
}

// k, v [B][H][T][D] -> caches [B][H][S][D] at rows past .. past+T-1.
__global__ __launch_bounds__(256) void kv_append_kernel(const float4 *__restrict__ k,
                                                        const float4 *__restrict__ v,
                                                        float4 *__restrict__ kc, float4 *__restrict__ vc,
                                                        uint32_t bh_count, uint32_t T, uint32_t S, uint32_t D,
                                                        uint32_t past)
{
    // grid: x = chunks of one (batch, head)'s T x D/4 float4, y = (batch,
    // head) pairs (those past gridDim.y take further trips)
    const uint32_t D4 = D >> 2;
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= T * D4) return;
    const uint32_t t = i / D4, dd4 = i - t * D4;
    for (uint32_t bh = blockIdx.y; bh < bh_count; bh += gridDim.y) {
        const uint64_t src = static_cast<uint64_t>(bh) * T * D4 + i;
        const uint64_t dst = (static_cast<uint64_t>(bh) * S + past + t) * D4 + dd4;
        kc[dst] = k[src];
        vc[dst] = v[src];
    }
}

inline uint32_t blocks_for(uint64_t n) { return static_cast<uint32_t>((n + 255) / 256); }
// Grid of the row-layout kernels: chunks of 256 float4 per row, up to 65535 row groups.
inline dim3 row_grid(uint64_t f4_per_row, uint64_t rows)
{
    return dim3(blocks_for(f4_per_row), static_cast<uint32_t>(rows < 65535 ? rows : 65535));
}

// Host twins of the three layout kernels (reference CPU build).
void split_qkv_host(const float *qkv, float *q, float *k, float *v, uint64_t rows, uint32_t T,
                    uint32_t H, uint32_t D)
{
    const uint64_t d = static_cast<uint64_t>(H) * D;
    for (uint64_t r = 0; r < rows; ++r) {
        const uint64_t b = r / T, t = r % T;
        for (uint32_t h = 0; h < H; ++h) {
            const uint64_t dst = ((b * H + h) * T + t) * D;
            const float *src = qkv + r * 3 * d + static_cast<uint64_t>(h) * D;
            std::memcpy(q + dst, src, D * sizeof(float));
            std::memcpy(k + dst, src + d, D * sizeof(float));
            std::memcpy(v + dst, src + 2 * d, D * sizeof(float));
        }
    }
}

void merge_heads_host(const float *o, float *y, uint64_t rows, uint32_t T, uint32_t H, uint32_t D)
{
    const uint64_t d = static_cast<uint64_t>(H) * D;
    for (uint64_t r = 0; r < rows; ++r) {
        const uint64_t b = r / T, t = r % T;
        for (uint32_t h = 0; h < H; ++h)
            std::memcpy(y + r * d + static_cast<uint64_t>(h) * D, o + ((b * H + h) * T + t) * D,
                        D * sizeof(float));
    }
}

void kv_append_host(const float *k, const float *v, float *kc, float *vc, uint64_t BH, uint32_t T,
                    uint32_t S, uint32_t D, uint32_t past)
{
    for (uint64_t bh = 0; bh < BH; ++bh)
        for (uint32_t t = 0; t < T; ++t) {
            std::memcpy(kc + (bh * S + past + t) * D, k + (bh * T + t) * D, D * sizeof(float));
            std::memcpy(vc + (bh * S + past + t) * D, v + (bh * T + t) * D, D * sizeof(float));
        }
}

vnpu_command_t rmsnorm(const float *X, const float *W, float *Y, uint32_t rows, uint32_t cols,
                       float eps)
{
    vnpu_command_t c{};
    c.opcode = VNPU_OP_RMSNORM_F32;
    c.args.rmsnorm.X = X;
    c.args.rmsnorm.W = W;
    c.args.rmsnorm.Y = Y;
    c.args.rmsnorm.rows = rows;
    c.args.rmsnorm.cols = cols;
    c.args.rmsnorm.eps = eps;
    return c;
}

// run_gemm (llm_bench.cpp:213-238): per-row QUANTIZE_I8, then MATMUL_I8.
void gemm_i8(std::vector<vnpu_command_t> &cmds, const float *X, int8_t *a8, float *sa,
             vnpu_packed_weights_t *W, float *C, uint32_t M, uint32_t K, uint32_t N, bool quantize)
{
    if (quantize) {
        vnpu_command_t q{};
        q.opcode = VNPU_OP_QUANTIZE_I8;
        q.args.quantize_i8.X = X;
        q.args.quantize_i8.Y = a8;
        q.args.quantize_i8.scales = sa;
        q.args.quantize_i8.rows = M;
        q.args.quantize_i8.cols = K;
        q.args.quantize_i8.axis = VNPU_QUANT_PER_ROW;
        cmds.push_back(q);
    }
    vnpu_command_t g{};
    g.opcode = VNPU_OP_MATMUL_I8;
    g.args.matmul_i8.A = a8;
    g.args.matmul_i8.B = W;
    g.args.matmul_i8.scale_a = sa;
    g.args.matmul_i8.C = C;
    g.args.matmul_i8.M = M;
    g.args.matmul_i8.K = K;
    g.args.matmul_i8.N = N;
    cmds.push_back(g);
}

vnpu_command_t add(const float *A, const float *B, float *Y, uint64_t n)
{
    vnpu_command_t c{};
    c.opcode = VNPU_OP_ADD_F32;
    c.args.binary.A = A;
    c.args.binary.B = B;
    c.args.binary.Y = Y;
    c.args.binary.count = n;
    c.args.binary.alpha = 1.0f;
    c.args.binary.beta = 1.0f;
    return c;
}

}  // namespace

extern "C" vnpu_status_t vnpu_block_run(const vnpu_backend_v1_t *api, vnpu_stream_t *stream,
                                        void *hip_stream, const vnpu_block_config_t *cfg,
                                        const vnpu_block_weights_t *w, const vnpu_block_buffers_t *b)
{
    if (!api || !stream || !cfg || !w || !b) return VNPU_ERR_INVALID_ARGUMENT;
    const uint32_t B = cfg->batch, T = cfg->tokens, d = cfg->d_model, H = cfg->heads,
                   D = cfg->head_dim, F = cfg->ffn;
    if (!B || !T || !d || !H || !D || !F || H * D != d || (D & 3)) return VNPU_ERR_INVALID_ARGUMENT;
    const bool decode = b->k_cache != nullptr;
    if (decode && (!b->v_cache || cfg->cache_len != cfg->past + T)) return VNPU_ERR_INVALID_ARGUMENT;
    const uint32_t rows = B * T;
    const uint64_t rd = static_cast<uint64_t>(rows) * d;
    hipStream_t hs = static_cast<hipStream_t>(hip_stream);
    vnpu_status_t rc;
    auto submit = [&](std::vector<vnpu_command_t> &cmds) {
        rc = api->stream_submit(stream, cmds.data(), cmds.size(), nullptr);
        cmds.clear();
        if (rc == VNPU_OK && !hs) rc = api->stream_sync(stream);
        return rc == VNPU_OK;
    };
    auto launched = [&]() {
        if (hipGetLastError() != hipSuccess) {
            rc = VNPU_ERR_DEVICE_ERROR;
            return false;
        }
        return true;
    };
    std::vector<vnpu_command_t> cmds;
    cmds.reserve(16);

    // Batch 1: attention RMSNorm, QKV projection.
    cmds.push_back(rmsnorm(b->x, w->norm_attn, b->xn, rows, d, cfg->eps));
    gemm_i8(cmds, b->xn, b->a8, b->scale_a, w->qkv, b->qkv, rows, d, 3 * d, true);
    if (!submit(cmds)) return rc;
    if (hs) {
        split_qkv_kernel<<<row_grid(3 * d / 4, rows), 256, 0, hs>>>(
            reinterpret_cast<const float4 *>(b->qkv), reinterpret_cast<float4 *>(b->q),
            reinterpret_cast<float4 *>(b->k), reinterpret_cast<float4 *>(b->v), static_cast<uint32_t>(rows), T, H,
            D);
        if (!launched()) return rc;
    } else {
        split_qkv_host(b->qkv, b->q, b->k, b->v, rows, T, H, D);
    }

    // Batch 2: RoPE at positions past .. past+T-1; decode appends to the caches.
    vnpu_command_t rope{};
    rope.opcode = VNPU_OP_ROPE_F32;
    rope.args.rope.Q = b->q;
    rope.args.rope.K = b->k;
    rope.args.rope.batch = B;
    rope.args.rope.heads = H;
    rope.args.rope.q_seq = T;
    rope.args.rope.k_seq = T;
    rope.args.rope.head_dim = D;
    rope.args.rope.position_offset = cfg->past;
    rope.args.rope.theta_base = cfg->theta;
    rope.args.rope.scaling = 1.0f;
    cmds.push_back(rope);
    if (!submit(cmds)) return rc;
    if (decode) {
        if (hs) {
            const dim3 grid = row_grid(static_cast<uint64_t>(T) * D / 4, static_cast<uint64_t>(B) * H);
            kv_append_kernel<<<grid, 256, 0, hs>>>(
                reinterpret_cast<const float4 *>(b->k), reinterpret_cast<const float4 *>(b->v),
                reinterpret_cast<float4 *>(b->k_cache), reinterpret_cast<float4 *>(b->v_cache), B * H, T,
                cfg->cache_len, D, cfg->past);
            if (!launched()) return rc;
        } else {
            kv_append_host(b->k, b->v, b->k_cache, b->v_cache, static_cast<uint64_t>(B) * H, T,
                           cfg->cache_len, D, cfg->past);
        }
    }

    // Batch 3: causal attention.
    vnpu_command_t att{};
    att.opcode = VNPU_OP_ATTENTION_F32;
    att.args.attention.Q = b->q;
    att.args.attention.K = decode ? b->k_cache : b->k;
    att.args.attention.V = decode ? b->v_cache : b->v;
    att.args.attention.O = b->o;
    att.args.attention.batch = B;
    att.args.attention.heads = H;
    att.args.attention.seq_q = T;
    att.args.attention.seq_k = decode ? cfg->cache_len : T;
    att.args.attention.head_dim = D;
    att.args.attention.causal = 1;
    cmds.push_back(att);
    // One token per sequence: [B][H][1][D] is already the token-major
    // [B][H*D] layout, so the O projection reads the attention output as is.
    const float *att_rows = b->att;
    if (T == 1) {
        att_rows = b->o;
    } else {
        if (!submit(cmds)) return rc;
        if (hs) {
            merge_heads_kernel<<<row_grid(d / 4, rows), 256, 0, hs>>>(
                reinterpret_cast<const float4 *>(b->o), reinterpret_cast<float4 *>(b->att),
                static_cast<uint32_t>(rows), T, H, D);
            if (!launched()) return rc;
        } else {
            merge_heads_host(b->o, b->att, rows, T, H, D);
        }
    }

    // Batch 4 (with the attention when T = 1): O projection + residual, FFN
    // RMSNorm, gate/up, SwiGLU, down + residual.
    gemm_i8(cmds, att_rows, b->a8, b->scale_a, w->o, b->proj, rows, d, d, true);
    cmds.push_back(add(b->x, b->proj, b->x, rd));
    cmds.push_back(rmsnorm(b->x, w->norm_ffn, b->xn, rows, d, cfg->eps));
    gemm_i8(cmds, b->xn, b->a8, b->scale_a, w->gate, b->gate, rows, d, F, true);
    gemm_i8(cmds, b->xn, b->a8, b->scale_a, w->up, b->up, rows, d, F, false);
    vnpu_command_t sg{};
    sg.opcode = VNPU_OP_SWIGLU_F32;
    sg.args.swiglu.gate = b->gate;
    sg.args.swiglu.up = b->up;
    sg.args.swiglu.Y = b->ff;
    sg.args.swiglu.count = static_cast<uint64_t>(rows) * F;
    sg.args.swiglu.alpha = 1.0f;
    cmds.push_back(sg);
    gemm_i8(cmds, b->ff, b->a8, b->scale_a, w->down, b->proj, rows, F, d, true);
    cmds.push_back(add(b->x, b->proj, b->x, rd));
    submit(cmds);
    return rc;
}
