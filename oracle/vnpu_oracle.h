/*
 * vnpu_oracle.h - CPU restatement of the reference vnpu kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the
 * MI355X backend: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product (libvnpu.so) never links it.
 *
 * Every function restates one reference routine in plain C (file:line in the
 * definition).  Arithmetic is single precision in the reference's operation
 * order, built with -ffp-contract=off so no multiply-add is fused.
 */
#ifndef VNPU_ORACLE_H
#define VNPU_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float vo_fast_expf(float x);
float vo_silu(float x);
float vo_gelu_tanh(float x);
float vo_apply_epilogue(float v, uint32_t epilogue);

void vo_quantize_rows(const float *X, int8_t *Y, float *scales, uint64_t rows, uint64_t cols);
void vo_quantize_columns(const float *X, int8_t *Y, float *scales, uint64_t rows, uint64_t cols);
void vo_quantize_tensor(const float *X, int8_t *Y, float *scales, uint64_t rows, uint64_t cols);

void vo_pack_canonical(const int8_t *B, uint32_t K, uint32_t N, uint32_t ldb, uint32_t trans_b,
                       int8_t *orig, int32_t *column_sums);

void vo_gemm_i8_acc(const int8_t *A, uint32_t lda, const int8_t *Bkn, uint32_t M, uint32_t K,
                    uint32_t N, int32_t *acc);
void vo_matmul_i8(const int8_t *A, uint32_t lda, const int8_t *Bkn, const float *scale_a,
                  const float *scale_b, const float *bias, float *C, uint32_t ldc, uint32_t M,
                  uint32_t K, uint32_t N, uint32_t epilogue);

void vo_store_i8(const int32_t *acc, const float *scale_a, const float *scale_b,
                 const float *bias, float *C, uint32_t M, uint32_t N, uint32_t epilogue);
void vo_store_f32(const double *acc, const float *bias, float *C, uint32_t M, uint32_t N,
                  float alpha, float beta, uint32_t epilogue);

void vo_matmul_f32(const float *A, const float *B, const float *bias, float *C, uint32_t M,
                   uint32_t K, uint32_t N, uint32_t lda, uint32_t ldb, uint32_t ldc,
                   uint32_t trans_a, uint32_t trans_b, float alpha, float beta, uint32_t epilogue,
                   const uint8_t *cull);
void vo_matmul_f32_acc64(const float *A, const float *B, const float *bias, float *C, uint32_t M,
                         uint32_t K, uint32_t N, uint32_t lda, uint32_t ldb, uint32_t ldc,
                         uint32_t trans_a, uint32_t trans_b, float alpha, float beta,
                         uint32_t epilogue);
uint64_t vo_cull_map(uint32_t M, uint32_t N, uint32_t unit, uint32_t tile_m, uint32_t tile_n,
                     uint32_t threads, uint32_t pack_b, const uint8_t *tile_mask,
                     uint32_t mask_tile_m, uint32_t mask_tile_n, uint8_t *elem_cull);

void vo_rmsnorm(const float *X, const float *W, float *Y, uint32_t rows, uint32_t cols, float eps);
void vo_softmax(const float *X, float *Y, uint32_t rows, uint32_t cols, float temperature);
void vo_rope(float *Q, float *K, const int32_t *positions, uint32_t batch, uint32_t heads,
             uint32_t q_seq, uint32_t k_seq, uint32_t head_dim, uint32_t position_offset,
             uint32_t interleaved, float theta_base, float scaling);
void vo_swiglu(const float *gate, const float *up, float *Y, uint64_t count, float alpha);
void vo_add(const float *A, const float *B, float *Y, uint64_t count, float alpha, float beta);
void vo_mul(const float *A, const float *B, float *Y, uint64_t count, float alpha, float beta);
void vo_gelu(const float *X, float *Y, uint64_t count);
void vo_attention(const float *Q, const float *K, const float *V, const float *mask, float *O,
                  uint32_t batch, uint32_t heads, uint32_t seq_q, uint32_t seq_k,
                  uint32_t head_dim, uint32_t causal, float scale);

#ifdef __cplusplus
}
#endif

/* The reference's AVX2 builds of the block's f32 ops, rounding for rounding. */
void vo_rmsnorm_avx2(const float *X, const float *W, float *Y, uint32_t rows, uint32_t cols, float eps);
float vo_exp_avx2(float x);
/* SWIGLU and MUL round differently in each range's scalar tail: ranges of
 * `grain` elements (0: one range), as the reference's command splits them. */
void vo_swiglu_avx2(const float *gate, const float *up, float *Y, uint64_t count, float alpha,
                    uint64_t grain);
void vo_softmax_avx2(const float *X, float *Y, uint32_t rows, uint32_t cols, float temperature);
void vo_gelu_avx2(const float *X, float *Y, uint64_t count);
void vo_add_avx2(const float *A, const float *B, float *Y, uint64_t count, float alpha, float beta);
void vo_mul_avx2(const float *A, const float *B, float *Y, uint64_t count, float alpha, float beta,
                 uint64_t grain);
void vo_attention_avx2(const float *Q, const float *K, const float *V, const float *mask, float *O,
                       uint32_t batch, uint32_t heads, uint32_t seq_q, uint32_t seq_k,
                       uint32_t head_dim, uint32_t causal, float scale);

#endif
