/* block_harness.h - the synthetic Llama-style decoder block, driven through
 * any vnpu backend's v1 vtable (libvnpu_block.so).
 *
 * This is the harness side of the workload, not part of the vnpu ABI: the
 * reference's own block benchmark (tools/llm_bench.cpp:213-326 run_gemm /
 * run_block) composes ABI calls the same way and does the layout work the
 * ABI has no op for (head-major transposes, KV-cache append) on the host.
 * Here the layout work runs as small HIP kernels on the vnpu stream when a
 * hipStream_t is given, or on the host (after a stream sync) when it is not,
 * so the same sequence drives the MI355X backend and the reference's CPU
 * build.
 *
 * One block on rows = batch * tokens hidden states x [rows][d_model]:
 *   xn = RMSNORM(x, norm_attn, eps)
 *   qkv = MATMUL_I8(QUANTIZE_I8(xn), W_qkv)            [rows][3 d_model]
 *   q, k, v = head-major split of qkv                  [batch][heads][tokens][head_dim]
 *   ROPE(q, k, position_offset = past, theta)
 *   decode (k_cache != NULL): k, v appended to the caches at slot past;
 *     o = ATTENTION(q, k_cache, v_cache, seq_k = cache_len, causal)
 *   prefill: o = ATTENTION(q, k, v, seq_k = tokens, causal)
 *   x += MATMUL_I8(QUANTIZE_I8(token-major o), W_o)
 *   xn = RMSNORM(x, norm_ffn, eps)
 *   ff = SWIGLU(MATMUL_I8(QUANTIZE_I8(xn), W_gate), MATMUL_I8(.., W_up))
 *   x += MATMUL_I8(QUANTIZE_I8(ff), W_down)
 */
#ifndef VNPU_BLOCK_HARNESS_H
#define VNPU_BLOCK_HARNESS_H

#include "vnpu.h"
#include "vnpu_backend.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct vnpu_block_config_t {
    uint32_t batch;
    uint32_t tokens;     /* new tokens per sequence */
    uint32_t d_model;
    uint32_t heads;
    uint32_t head_dim;   /* heads * head_dim == d_model */
    uint32_t ffn;
    uint32_t past;       /* positions already in the cache; RoPE offset */
    uint32_t cache_len;  /* decode: cache rows per (b, h); must equal past + tokens */
    float eps;
    float theta;
} vnpu_block_config_t;

typedef struct vnpu_block_weights_t {
    vnpu_packed_weights_t *qkv;   /* [d_model][3 d_model] */
    vnpu_packed_weights_t *o;     /* [d_model][d_model] */
    vnpu_packed_weights_t *gate;  /* [d_model][ffn] */
    vnpu_packed_weights_t *up;    /* [d_model][ffn] */
    vnpu_packed_weights_t *down;  /* [ffn][d_model] */
    const float *norm_attn;       /* [d_model] */
    const float *norm_ffn;        /* [d_model] */
} vnpu_block_weights_t;

/* Every pointer addresses memory the backend's commands accept (device
 * memory for the MI355X backend, host memory for the reference). */
typedef struct vnpu_block_buffers_t {
    float *x;            /* [rows][d_model], updated in place */
    float *xn;           /* [rows][d_model] */
    int8_t *a8;          /* [rows][max(d_model, ffn)] */
    float *scale_a;      /* [rows] */
    float *qkv;          /* [rows][3 d_model] */
    float *q, *k, *v;    /* [batch][heads][tokens][head_dim] each */
    float *o;            /* [batch][heads][tokens][head_dim] */
    float *att;          /* [rows][d_model] */
    float *proj;         /* [rows][d_model] */
    float *gate, *up;    /* [rows][ffn] */
    float *ff;           /* [rows][ffn] */
    float *k_cache;      /* decode: [batch][heads][cache_len][head_dim], else NULL */
    float *v_cache;
} vnpu_block_buffers_t;

/* Enqueues one block on stream.  hip_stream: the hipStream_t behind stream
 * (vnpu_stream_hip_handle) to run the layout kernels on the GPU, or NULL to
 * run them on the host after syncing the stream.  Returns VNPU_OK once
 * everything is enqueued (GPU) or done (host). */
vnpu_status_t vnpu_block_run(const vnpu_backend_v1_t *api, vnpu_stream_t *stream, void *hip_stream,
                             const vnpu_block_config_t *cfg, const vnpu_block_weights_t *w,
                             const vnpu_block_buffers_t *b);

#ifdef __cplusplus
}
#endif

#endif /* VNPU_BLOCK_HARNESS_H */
