/*
 * vnpu_oracle.c - CPU restatement of the reference vnpu kernels.
 *
 * TEST INFRASTRUCTURE ONLY (see vnpu_oracle.h).  Plain C, single precision,
 * the reference's operation order, built with -ffp-contract=off.  Each
 * function cites the reference routine it restates; paths are relative to
 * the reference repository root.
 */
#include "vnpu_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define VO_EPI_NONE 0u
#define VO_EPI_RELU 1u
#define VO_EPI_SILU 2u
#define VO_EPI_GELU_TANH 3u
#define VO_EPI_GELU_ERF 4u

/* src/internal.h:87-110: exp(x) = 2^floor(z) * P5(z - floor(z)), z = x*log2(e),
 * P5 the degree-5 Taylor polynomial of 2^f in f, clamped at |x| > 80. */
float vo_fast_expf(float x)
{
    if (x < -80.0f) return 0.0f;
    if (x > 80.0f) return INFINITY;
    const float log2e = 1.4426950408889634f;
    float z = x * log2e;
    float zi = floorf(z);
    float f = z - zi;
    float p = 1.0f + f * (0.6931471805599453f +
              f * (0.2402265069591007f +
              f * (0.05550410866482158f +
              f * (0.009618129107628477f +
              f * 0.0013333558146428443f))));
    return ldexpf(p, (int)zi);
}

/* src/internal.h:112 */
float vo_silu(float x) { return x / (1.0f + vo_fast_expf(-x)); }

/* src/internal.h:114-121 */
float vo_gelu_tanh(float x)
{
    const float k0 = 0.7978845608028654f;
    const float k1 = 0.035677408136300125f;
    float x3 = x * x * x;
    float inner = k0 * (x + k1 * x3);
    float t = 2.0f / (1.0f + vo_fast_expf(-2.0f * inner)) - 1.0f;
    return 0.5f * x * (1.0f + t);
}

/* src/internal.h:123-136; GELU_ERF is evaluated as tanh-GELU. */
float vo_apply_epilogue(float v, uint32_t epilogue)
{
    switch (epilogue) {
    case VO_EPI_RELU: return v > 0.0f ? v : 0.0f;
    case VO_EPI_SILU: return vo_silu(v);
    case VO_EPI_GELU_TANH:
    case VO_EPI_GELU_ERF: return vo_gelu_tanh(v);
    default: return v;
    }
}

/* ----------------------------------------------------------------------- */
/* Quantization: src/kernels/llm.cpp:387-436, src/core/scheduler.cpp:430-473 */
/* ----------------------------------------------------------------------- */

/* llm.cpp:387-393: round half away from zero, clamp, truncate to int8.  A NaN
 * product converts to 0, as x86 cvttss2si's 0x80000000 truncated to 8 bits. */
static int8_t quantize_value(float x, float inv_scale)
{
    float q = roundf(x * inv_scale);
    if (q > 127.0f) q = 127.0f;
    if (q < -128.0f) q = -128.0f;
    if (q != q) return 0;
    return (int8_t)(int)q;
}

/* std::max(m, v) keeps m when v is NaN (llm.cpp:400-401). */
static float max_keep(float m, float v) { return (m < v) ? v : m; }

/* llm.cpp:402-404: scale = max|x|/127, zero or non-finite -> 1, inv = 1/scale. */
static float scale_from_max(float maxabs)
{
    float scale = maxabs / 127.0f;
    if (scale <= 0.0f || !isfinite(scale)) scale = 1.0f;
    return scale;
}

/* llm.cpp:395-411 */
void vo_quantize_rows(const float *X, int8_t *Y, float *scales, uint64_t rows, uint64_t cols)
{
    for (uint64_t r = 0; r < rows; ++r) {
        const float *row = X + r * cols;
        float maxabs = 0.0f;
        for (uint64_t j = 0; j < cols; ++j) maxabs = max_keep(maxabs, fabsf(row[j]));
        float scale = scale_from_max(maxabs);
        float inv = 1.0f / scale;
        scales[r] = scale;
        for (uint64_t j = 0; j < cols; ++j) Y[r * cols + j] = quantize_value(row[j], inv);
    }
}

/* llm.cpp:413-428 */
void vo_quantize_columns(const float *X, int8_t *Y, float *scales, uint64_t rows, uint64_t cols)
{
    float *mx = (float *)calloc(cols, sizeof(float));
    for (uint64_t r = 0; r < rows; ++r)
        for (uint64_t c = 0; c < cols; ++c) mx[c] = max_keep(mx[c], fabsf(X[r * cols + c]));
    float *inv = (float *)malloc(cols * sizeof(float));
    for (uint64_t c = 0; c < cols; ++c) {
        scales[c] = scale_from_max(mx[c]);
        inv[c] = 1.0f / scales[c];
    }
    for (uint64_t r = 0; r < rows; ++r)
        for (uint64_t c = 0; c < cols; ++c)
            Y[r * cols + c] = quantize_value(X[r * cols + c], inv[c]);
    free(inv);
    free(mx);
}

/* scheduler.cpp:441-465 (max over all elements; max is order independent)
 * then llm.cpp:430-436. */
void vo_quantize_tensor(const float *X, int8_t *Y, float *scales, uint64_t rows, uint64_t cols)
{
    uint64_t n = rows * cols;
    float maxabs = 0.0f;
    for (uint64_t i = 0; i < n; ++i) maxabs = max_keep(maxabs, fabsf(X[i]));
    scales[0] = scale_from_max(maxabs);
    float inv = 1.0f / (scales[0] > 0.0f ? scales[0] : 1.0f);
    for (uint64_t i = 0; i < n; ++i) Y[i] = quantize_value(X[i], inv);
}

/* ----------------------------------------------------------------------- */
/* Packed weights: scheduler.cpp:787-806 (canonical KxN copy + column sums). */
/* ----------------------------------------------------------------------- */

void vo_pack_canonical(const int8_t *B, uint32_t K, uint32_t N, uint32_t ldb, uint32_t trans_b,
                       int8_t *orig, int32_t *column_sums)
{
    uint32_t ld = ldb ? ldb : (trans_b ? K : N);
    for (uint32_t n = 0; n < N; ++n) column_sums[n] = 0;
    for (uint32_t k = 0; k < K; ++k)
        for (uint32_t n = 0; n < N; ++n) {
            int8_t v = trans_b ? B[(size_t)n * ld + k] : B[(size_t)k * ld + n];
            orig[(size_t)k * N + n] = v;
            column_sums[n] += v;
        }
}

/* ----------------------------------------------------------------------- */
/* INT8 GEMM: kernels.cpp:537-550 (scalar tile) + store_i8_c :526-535.        */
/* ----------------------------------------------------------------------- */

void vo_gemm_i8_acc(const int8_t *A, uint32_t lda, const int8_t *Bkn, uint32_t M, uint32_t K,
                    uint32_t N, int32_t *acc)
{
    for (uint32_t m = 0; m < M; ++m) {
        int32_t *row = acc + (size_t)m * N;
        for (uint32_t n = 0; n < N; ++n) row[n] = 0;
        for (uint32_t k = 0; k < K; ++k) {
            int32_t a = A[(size_t)m * lda + k];
            if (!a) continue;
            const int8_t *b = Bkn + (size_t)k * N;
            for (uint32_t n = 0; n < N; ++n) row[n] += a * (int32_t)b[n];
        }
    }
}

/* store_i8_c: out = ((float)dot * sa) * sb; out += bias; epilogue. */
void vo_matmul_i8(const int8_t *A, uint32_t lda, const int8_t *Bkn, const float *scale_a,
                  const float *scale_b, const float *bias, float *C, uint32_t ldc, uint32_t M,
                  uint32_t K, uint32_t N, uint32_t epilogue)
{
    int32_t *acc = (int32_t *)malloc((size_t)N * sizeof(int32_t));
    for (uint32_t m = 0; m < M; ++m) {
        vo_gemm_i8_acc(A + (size_t)m * lda, lda, Bkn, 1, K, N, acc);
        float sa = scale_a ? scale_a[m] : 1.0f;
        for (uint32_t n = 0; n < N; ++n) {
            float sb = scale_b ? scale_b[n] : 1.0f;
            float out = (float)acc[n] * sa;
            out = out * sb;
            if (bias) out += bias[n];
            C[(size_t)m * ldc + n] = vo_apply_epilogue(out, epilogue);
        }
    }
    free(acc);
}

/* The store_i8_c step above for accumulators computed elsewhere (an exact
 * float64 product of int8 matrices is the int32 accumulator): lets the tests
 * check full-size GEMMs through BLAS with this file's rounding order. */
void vo_store_i8(const int32_t *acc, const float *scale_a, const float *scale_b,
                 const float *bias, float *C, uint32_t M, uint32_t N, uint32_t epilogue)
{
    for (uint32_t m = 0; m < M; ++m) {
        float sa = scale_a ? scale_a[m] : 1.0f;
        for (uint32_t n = 0; n < N; ++n) {
            float sb = scale_b ? scale_b[n] : 1.0f;
            float out = (float)acc[(size_t)m * N + n] * sa;
            out = out * sb;
            if (bias) out += bias[n];
            C[(size_t)m * N + n] = vo_apply_epilogue(out, epilogue);
        }
    }
}

/* ----------------------------------------------------------------------- */
/* F32 GEMM: kernels.cpp:43-75 (store_c, zero_c_tile, scalar tile) with the   */
/* defaults of scheduler.cpp:274-318 (alpha 0 -> 1, ld 0 -> dense).           */
/* ----------------------------------------------------------------------- */

static float load_a(const float *A, uint32_t lda, uint32_t trans_a, uint32_t m, uint32_t k)
{
    return trans_a ? A[(size_t)k * lda + m] : A[(size_t)m * lda + k];
}

static float load_b(const float *B, uint32_t ldb, uint32_t trans_b, uint32_t k, uint32_t n)
{
    return trans_b ? B[(size_t)n * ldb + k] : B[(size_t)k * ldb + n];
}

static void f32_defaults(uint32_t M, uint32_t K, uint32_t N, uint32_t *lda, uint32_t *ldb,
                         uint32_t *ldc, uint32_t trans_a, uint32_t trans_b, float *alpha)
{
    if (!*lda) *lda = trans_a ? M : K;
    if (!*ldb) *ldb = trans_b ? K : N;
    if (!*ldc) *ldc = N;
    if (*alpha == 0.0f) *alpha = 1.0f;
}

/* store_c (kernels.cpp:43-50): out = alpha*acc; += bias; += beta*C; epi.
 * A culled element (cull[m*N+n] != 0) is zero_c_tile (:52-62): epi(bias + beta*C). */
void vo_matmul_f32(const float *A, const float *B, const float *bias, float *C, uint32_t M,
                   uint32_t K, uint32_t N, uint32_t lda, uint32_t ldb, uint32_t ldc,
                   uint32_t trans_a, uint32_t trans_b, float alpha, float beta, uint32_t epilogue,
                   const uint8_t *cull)
{
    f32_defaults(M, K, N, &lda, &ldb, &ldc, trans_a, trans_b, &alpha);
    for (uint32_t m = 0; m < M; ++m)
        for (uint32_t n = 0; n < N; ++n) {
            float *dst = C + (size_t)m * ldc + n;
            if (cull && cull[(size_t)m * N + n]) {
                float out = bias ? bias[n] : 0.0f;
                if (beta != 0.0f) out += beta * *dst;
                *dst = vo_apply_epilogue(out, epilogue);
                continue;
            }
            float acc = 0.0f;
            for (uint32_t k = 0; k < K; ++k)
                acc += load_a(A, lda, trans_a, m, k) * load_b(B, ldb, trans_b, k, n);
            float out = alpha * acc;
            if (bias) out += bias[n];
            if (beta != 0.0f) out += beta * *dst;
            *dst = vo_apply_epilogue(out, epilogue);
        }
}

/* Same semantics with a double accumulator, the reference's conformance
 * oracle (tools/conformance.cpp:75-91) for large K. */
void vo_matmul_f32_acc64(const float *A, const float *B, const float *bias, float *C, uint32_t M,
                         uint32_t K, uint32_t N, uint32_t lda, uint32_t ldb, uint32_t ldc,
                         uint32_t trans_a, uint32_t trans_b, float alpha, float beta,
                         uint32_t epilogue)
{
    f32_defaults(M, K, N, &lda, &ldb, &ldc, trans_a, trans_b, &alpha);
    for (uint32_t m = 0; m < M; ++m)
        for (uint32_t n = 0; n < N; ++n) {
            double acc = 0.0;
            for (uint32_t k = 0; k < K; ++k)
                acc += (double)load_a(A, lda, trans_a, m, k) *
                       (double)load_b(B, ldb, trans_b, k, n);
            float *dst = C + (size_t)m * ldc + n;
            float out = alpha * (float)acc;
            if (bias) out += bias[n];
            if (beta != 0.0f) out += beta * *dst;
            *dst = vo_apply_epilogue(out, epilogue);
        }
}

/* The store step of vo_matmul_f32_acc64 for double accumulators computed
 * elsewhere (float64 BLAS in the tests): C = epi(alpha*(float)acc + bias +
 * beta*C), C dense [M][N]. */
void vo_store_f32(const double *acc, const float *bias, float *C, uint32_t M, uint32_t N,
                  float alpha, float beta, uint32_t epilogue)
{
    if (alpha == 0.0f) alpha = 1.0f;
    for (uint32_t m = 0; m < M; ++m)
        for (uint32_t n = 0; n < N; ++n) {
            float *dst = C + (size_t)m * N + n;
            float out = alpha * (float)acc[(size_t)m * N + n];
            if (bias) out += bias[n];
            if (beta != 0.0f) out += beta * *dst;
            *dst = vo_apply_epilogue(out, epilogue);
        }
}

/* ----------------------------------------------------------------------- */
/* Wildcat cull geometry: choose_unit scheduler.cpp:43-59, tile_geometry      */
/* :96-206 (the f32 branches), build_tiles_generic :208-262.  Writes a per-   */
/* element cull map and returns the number of culled tiles.                  */
/* ----------------------------------------------------------------------- */

static uint32_t cdiv(uint32_t a, uint32_t b) { return b ? (a + b - 1) / b : 0; }
static uint32_t umin(uint32_t a, uint32_t b) { return a < b ? a : b; }
static uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

uint64_t vo_cull_map(uint32_t M, uint32_t N, uint32_t unit, uint32_t tile_m, uint32_t tile_n,
                     uint32_t threads, uint32_t pack_b, const uint8_t *tile_mask,
                     uint32_t mask_tile_m, uint32_t mask_tile_n, uint8_t *elem_cull)
{
    /* choose_unit with no batch flags: an explicit unit wins, AUTO with a mask
     * becomes WILDCAT. */
    if (unit == 0) unit = tile_mask ? 2u : 1u;
    uint32_t tm = umax(1, tile_m), tn = umax(1, tile_n);
    uint32_t units = umax(1, threads);
    int done = 0;
    if (M <= 8 && (unit == 1 || unit == 0)) {
        tm = M;
        tn = umin(umax(32, tn), 64);
        if (tn > N) tn = N;
        done = 1;
    }
    if (!done && pack_b && (unit == 1 || unit == 0)) {
        uint32_t nt64 = cdiv(N, 64);
        if (M >= 3 && nt64 >= 2 * units) {
            tm = M;
            tn = 64;
            done = 1;
        }
    }
    if (!done) {
        if (unit == 2) {
            tm = umin(tm, 32);
            tn = umin(tn, 64);
        } else if (unit == 3) {
            tm = umin(tm, 16);
            tn = umin(tn, 64);
        }
        uint64_t tiles = (uint64_t)cdiv(M, tm) * cdiv(N, tn);
        uint64_t target = (uint64_t)threads * 64;
        while (tiles > target && (tm < M || tn < N)) {
            if (tm < M) tm = umin(M, tm * 2);
            if (tn < N) tn = umin(N, tn * 2);
            tiles = (uint64_t)cdiv(M, tm) * cdiv(N, tn);
        }
    }
    uint32_t mt = cdiv(M, tm), nt = cdiv(N, tn);
    uint64_t culled = 0;
    memset(elem_cull, 0, (size_t)M * N);
    if (!tile_mask || !mask_tile_m || !mask_tile_n) return 0;
    for (uint32_t mi = 0; mi < mt; ++mi)
        for (uint32_t ni = 0; ni < nt; ++ni) {
            uint32_t mm = umin(mask_tile_m - 1, (uint32_t)(((uint64_t)mi * mask_tile_m) / mt));
            uint32_t nn = umin(mask_tile_n - 1, (uint32_t)(((uint64_t)ni * mask_tile_n) / nt));
            if (tile_mask[(size_t)mm * mask_tile_n + nn] != 0) continue;
            ++culled;
            uint32_t m0 = mi * tm, n0 = ni * tn;
            uint32_t m1 = umin(M, m0 + tm), n1 = umin(N, n0 + tn);
            for (uint32_t m = m0; m < m1; ++m) memset(elem_cull + (size_t)m * N + n0, 1, n1 - n0);
        }
    return culled;
}

/* ----------------------------------------------------------------------- */
/* Transformer ops: src/kernels/llm.cpp                                      */
/* ----------------------------------------------------------------------- */

/* llm.cpp:64-77: ss = sum x^2 (sequential); inv = 1/sqrt(ss/C + eps);
 * y = x*inv*w.  eps <= 0 -> 1e-5. */
void vo_rmsnorm(const float *X, const float *W, float *Y, uint32_t rows, uint32_t cols, float eps)
{
    if (!(eps > 0.0f)) eps = 1e-5f;
    for (uint32_t r = 0; r < rows; ++r) {
        const float *x = X + (size_t)r * cols;
        float *y = Y + (size_t)r * cols;
        float ss = 0.0f;
        for (uint32_t j = 0; j < cols; ++j) ss += x[j] * x[j];
        float inv = 1.0f / sqrtf(ss / (float)cols + eps);
        for (uint32_t j = 0; j < cols; ++j) y[j] = x[j] * inv * (W ? W[j] : 1.0f);
    }
}

/* llm.cpp:116-134 */
void vo_softmax(const float *X, float *Y, uint32_t rows, uint32_t cols, float temperature)
{
    float inv_t = temperature > 0.0f ? 1.0f / temperature : 1.0f;
    for (uint32_t r = 0; r < rows; ++r) {
        const float *x = X + (size_t)r * cols;
        float *y = Y + (size_t)r * cols;
        float maxv = -INFINITY;
        for (uint32_t j = 0; j < cols; ++j) maxv = (maxv < x[j]) ? x[j] : maxv;
        float sum = 0.0f;
        for (uint32_t j = 0; j < cols; ++j) {
            float e = vo_fast_expf((x[j] - maxv) * inv_t);
            y[j] = e;
            sum += e;
        }
        float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (uint32_t j = 0; j < cols; ++j) y[j] *= inv;
    }
}

/* llm.cpp:188-217 (rotate_vector) */
static void rotate_vector(float *x, uint32_t dim, float position, float theta, float scaling,
                          int interleaved)
{
    if (!x || dim < 2) return;
    position *= scaling;
    if (interleaved) {
        for (uint32_t j = 0; j + 1 < dim; j += 2) {
            float inv = 1.0f / powf(theta, (float)j / (float)dim);
            float angle = position * inv;
            float c = cosf(angle), s = sinf(angle);
            float x0 = x[j], x1 = x[j + 1];
            x[j] = x0 * c - x1 * s;
            x[j + 1] = x0 * s + x1 * c;
        }
    } else {
        uint32_t half = dim / 2;
        for (uint32_t j = 0; j < half; ++j) {
            float inv = 1.0f / powf(theta, 2.0f * (float)j / (float)dim);
            float angle = position * inv;
            float c = cosf(angle), s = sinf(angle);
            float x0 = x[j], x1 = x[j + half];
            x[j] = x0 * c - x1 * s;
            x[j + half] = x0 * s + x1 * c;
        }
    }
}

/* llm.cpp:576-602 (kernel_rope_tokens): token t of every (b,h) rotates by
 * positions[t] or t + offset. */
void vo_rope(float *Q, float *K, const int32_t *positions, uint32_t batch, uint32_t heads,
             uint32_t q_seq, uint32_t k_seq, uint32_t head_dim, uint32_t position_offset,
             uint32_t interleaved, float theta_base, float scaling)
{
    uint32_t seq = q_seq > k_seq ? q_seq : k_seq;
    float theta = theta_base > 0.0f ? theta_base : 10000.0f;
    float sc = scaling > 0.0f ? scaling : 1.0f;
    uint64_t total = (uint64_t)batch * heads * seq;
    for (uint64_t idx = 0; idx < total; ++idx) {
        uint64_t bh = idx / seq;
        uint32_t t = (uint32_t)(idx % seq);
        float pos = (float)(positions ? positions[t] : (int32_t)(t + position_offset));
        if (Q && t < q_seq)
            rotate_vector(Q + (bh * q_seq + t) * head_dim, head_dim, pos, theta, sc, interleaved != 0);
        if (K && t < k_seq)
            rotate_vector(K + (bh * k_seq + t) * head_dim, head_dim, pos, theta, sc, interleaved != 0);
    }
}

/* llm.cpp:240-246 */
void vo_swiglu(const float *gate, const float *up, float *Y, uint64_t count, float alpha)
{
    float a = alpha == 0.0f ? 1.0f : alpha;
    for (uint64_t i = 0; i < count; ++i) Y[i] = vo_silu(gate[i]) * up[i] * a;
}

/* llm.cpp:223-230: alpha = beta = 0 means 1, 1. */
void vo_add(const float *A, const float *B, float *Y, uint64_t count, float alpha, float beta)
{
    float a = (alpha == 0.0f && beta == 0.0f) ? 1.0f : alpha;
    float b = (alpha == 0.0f && beta == 0.0f) ? 1.0f : beta;
    for (uint64_t i = 0; i < count; ++i) Y[i] = a * A[i] + b * B[i];
}

/* llm.cpp:232-238 */
void vo_mul(const float *A, const float *B, float *Y, uint64_t count, float alpha, float beta)
{
    float a = alpha == 0.0f ? 1.0f : alpha;
    for (uint64_t i = 0; i < count; ++i) Y[i] = a * A[i] * B[i] + beta;
}

/* llm.cpp:248-253 */
void vo_gelu(const float *X, float *Y, uint64_t count)
{
    for (uint64_t i = 0; i < count; ++i) Y[i] = vo_gelu_tanh(X[i]);
}

/* llm.cpp:442-546: per (b, h, 16-query block), online softmax over 64-key
 * blocks; causal masks ki > qi + (seq_k - seq_q); a block whose max is not
 * finite is skipped; fully masked rows give 0. */
void vo_attention(const float *Q, const float *K, const float *V, const float *mask, float *O,
                  uint32_t batch, uint32_t heads, uint32_t seq_q, uint32_t seq_k,
                  uint32_t head_dim, uint32_t causal, float scale)
{
    enum { BQ = 16, BK = 64 };
    const uint32_t D = head_dim;
    if (!(scale > 0.0f)) scale = 1.0f / sqrtf((float)D);
    float scores[BQ * BK], probs[BQ * BK], m[BQ], l[BQ];
    float *acc = (float *)malloc((size_t)BQ * D * sizeof(float));
    const uint32_t off = seq_k > seq_q ? seq_k - seq_q : 0;
    for (uint64_t bh = 0; bh < (uint64_t)batch * heads; ++bh) {
        const float *Qh = Q + bh * seq_q * D;
        const float *Kh = K + bh * seq_k * D;
        const float *Vh = V + bh * seq_k * D;
        const float *Mh = mask ? mask + bh * seq_q * seq_k : NULL;
        float *Oh = O + bh * seq_q * D;
        for (uint32_t q0 = 0; q0 < seq_q; q0 += BQ) {
            uint32_t qc = umin(BQ, seq_q - q0);
            for (uint32_t i = 0; i < qc; ++i) {
                m[i] = -INFINITY;
                l[i] = 0.0f;
                for (uint32_t d = 0; d < D; ++d) acc[i * D + d] = 0.0f;
            }
            for (uint32_t k0 = 0; k0 < seq_k; k0 += BK) {
                uint32_t kc = umin(BK, seq_k - k0);
                for (uint32_t i = 0; i < qc; ++i) {
                    uint32_t qi = q0 + i;
                    for (uint32_t j = 0; j < kc; ++j) {
                        uint32_t ki = k0 + j;
                        float s;
                        if (causal && ki > qi + off) {
                            s = -INFINITY;
                        } else {
                            float dot = 0.0f;
                            for (uint32_t d = 0; d < D; ++d)
                                dot += Qh[(size_t)qi * D + d] * Kh[(size_t)ki * D + d];
                            s = dot * scale;
                            if (Mh) s += Mh[(size_t)qi * seq_k + ki];
                        }
                        scores[i * BK + j] = s;
                    }
                }
                for (uint32_t i = 0; i < qc; ++i) {
                    float bmax = -INFINITY;
                    for (uint32_t j = 0; j < kc; ++j)
                        bmax = (bmax < scores[i * BK + j]) ? scores[i * BK + j] : bmax;
                    if (!isfinite(bmax)) continue;
                    float new_m = (m[i] < bmax) ? bmax : m[i];
                    float alpha = vo_fast_expf(m[i] - new_m);
                    float sum_p = 0.0f;
                    for (uint32_t j = 0; j < kc; ++j) {
                        float p = vo_fast_expf(scores[i * BK + j] - new_m);
                        probs[i * BK + j] = p;
                        sum_p += p;
                    }
                    l[i] = l[i] * alpha + sum_p;
                    for (uint32_t d = 0; d < D; ++d) acc[i * D + d] *= alpha;
                    for (uint32_t j = 0; j < kc; ++j) {
                        float p = probs[i * BK + j];
                        if (p == 0.0f) continue;
                        const float *v = Vh + (size_t)(k0 + j) * D;
                        for (uint32_t d = 0; d < D; ++d) acc[i * D + d] += p * v[d];
                    }
                    m[i] = new_m;
                }
            }
            for (uint32_t i = 0; i < qc; ++i) {
                float inv = l[i] > 0.0f ? 1.0f / l[i] : 0.0f;
                for (uint32_t d = 0; d < D; ++d) Oh[(size_t)(q0 + i) * D + d] = acc[i * D + d] * inv;
            }
        }
    }
    free(acc);
}

/* ----------------------------------------------------------------------- */
/* The reference's AVX2 builds of the block's f32 ops, in their exact order  */
/* of roundings (what the reference computes on an AVX2 host).  fmaf marks   */
/* each fused multiply-add of the reference's intrinsics; everything else   */
/* rounds separately (this file is built with -ffp-contract=off).           */
/* ----------------------------------------------------------------------- */

/* hsum256 (llm.cpp:20-28): (lo + hi), then two horizontal adds. */
static float vo_hsum8(const float a[8])
{
    float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    return (s0 + s1) + (s2 + s3);
}

/* The scalar tail loop `sum += a[i] * b[i]` of the reference's AVX2 reductions
 * (rmsnorm_avx2_rows llm.cpp:91, dot_avx2 :342) as its build compiles it: g++
 * -O3 gives the loop a 4-wide vector epilogue, so with four or more elements
 * left the first four products are rounded as one vector multiply and added to
 * the sum in order, and the remaining one to three (or all of a shorter tail)
 * are contracted into FMAs. */
static float vo_tail_dot(const float *a, const float *b, uint32_t n, float sum)
{
    uint32_t i = 0;
    if (n >= 4)
        for (; i < 4; ++i) {
            const float p = a[i] * b[i];
            sum = sum + p;
        }
    for (; i < n; ++i) sum = fmaf(a[i], b[i], sum);
    return sum;
}

/* rmsnorm_avx2_rows (llm.cpp:80-108): eight running sums of x*x (FMA) over
 * each 8-wide step, hsum256, then the tail; y = (x*w)*inv over the 8-wide
 * part and (x*inv)*w on the tail. */
void vo_rmsnorm_avx2(const float *X, const float *W, float *Y, uint32_t rows, uint32_t cols, float eps)
{
    if (!(eps > 0.0f)) eps = 1e-5f;
    for (uint32_t r = 0; r < rows; ++r) {
        const float *x = X + (size_t)r * cols;
        float *y = Y + (size_t)r * cols;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        uint32_t j = 0;
        for (; j + 8 <= cols; j += 8)
            for (int l = 0; l < 8; ++l) acc[l] = fmaf(x[j + l], x[j + l], acc[l]);
        float sum = vo_tail_dot(x + j, x + j, cols - j, vo_hsum8(acc));
        float inv = 1.0f / sqrtf(sum / (float)cols + eps);
        j = 0;
        for (; j + 8 <= cols; j += 8)
            for (int l = 0; l < 8; ++l) y[j + l] = (x[j + l] * (W ? W[j + l] : 1.0f)) * inv;
        for (; j < cols; ++j) y[j] = x[j] * inv * (W ? W[j] : 1.0f);
    }
}

/* exp256_ps (llm.cpp:31-56): x clamped to [-80, 80], z = x*log2e,
 * f = z - floor(z), P5 by FMA Horner, times 2^floor(z). */
float vo_exp_avx2(float x)
{
    /* _mm256_max_ps(-80, _mm256_min_ps(x, 80)): each returns its second
     * operand unless the comparison holds, so a NaN becomes 80. */
    x = x < 80.0f ? x : 80.0f;
    x = -80.0f > x ? -80.0f : x;
    float z = x * 1.4426950408889634f;
    float zi = floorf(z);
    float f = z - zi;
    float p = fmaf(0.0013333558146428443f, f, 0.009618129107628477f);
    p = fmaf(p, f, 0.05550410866482158f);
    p = fmaf(p, f, 0.2402265069591007f);
    p = fmaf(p, f, 0.6931471805599453f);
    p = fmaf(p, f, 1.0f);
    return ldexpf(p, (int)zi);
}

/* swiglu_avx2_range (llm.cpp:289-306): s = g / (1 + exp256(-g)),
 * y = (s*u)*alpha; the scalar tail of a thread's range uses silu with the
 * same FMA polynomial (its AVX2 function contracts it). */
/* The scalar fast_expf (internal.h:87-110) as inlined into the reference's
 * AVX2-target functions: the Horner steps contract to FMAs; x beyond
 * [-80, 80] gives 0 or +inf (no clamp to the bound). */
static float vo_fast_expf_fma(float x)
{
    if (x < -80.0f) return 0.0f;
    if (x > 80.0f) return INFINITY;
    float z = x * 1.4426950408889634f;
    float zi = floorf(z);
    float f = z - zi;
    float p = fmaf(0.0013333558146428443f, f, 0.009618129107628477f);
    p = fmaf(p, f, 0.05550410866482158f);
    p = fmaf(p, f, 0.2402265069591007f);
    p = fmaf(p, f, 0.6931471805599453f);
    p = fmaf(p, f, 1.0f);
    return ldexpf(p, (int)zi);
}

/* softmax_avx2_rows (llm.cpp:137-180), one row at a time as each of the
 * reference's threads takes whole rows: lane maxima over the 8-wide steps by
 * _mm256_max_ps(m, x) = m > x ? m : x (a NaN element becomes the lane's
 * running max, and the next element replaces it), the eight lanes then the
 * tail by std::max (a < b ? b : a); over the 8-wide steps e = exp256 of the
 * separately rounded (x - max) * inv_t, summed per lane and combined as
 * hsum256 does, ((s0+s4) + (s1+s5)) + ((s2+s6) + (s3+s7)); the tail with the
 * scalar fast_expf as inlined into the AVX2 function, added in order;
 * y = e * (1 / sum), 0 when sum is 0. */
void vo_softmax_avx2(const float *X, float *Y, uint32_t rows, uint32_t cols, float temperature)
{
    const float inv_t = temperature > 0.0f ? 1.0f / temperature : 1.0f;
    const uint32_t c8 = cols & ~7u;
    for (uint32_t r = 0; r < rows; ++r) {
        const float *x = X + (size_t)r * cols;
        float *y = Y + (size_t)r * cols;
        float vm[8], s[8];
        for (int c = 0; c < 8; ++c) { vm[c] = -INFINITY; s[c] = 0.0f; }
        for (uint32_t j = 0; j < c8; j += 8)
            for (int c = 0; c < 8; ++c) vm[c] = vm[c] > x[j + c] ? vm[c] : x[j + c];
        float maxv = -INFINITY;
        for (int c = 0; c < 8; ++c) maxv = maxv < vm[c] ? vm[c] : maxv;
        for (uint32_t j = c8; j < cols; ++j) maxv = maxv < x[j] ? x[j] : maxv;
        for (uint32_t j = 0; j < c8; j += 8)
            for (int c = 0; c < 8; ++c) {
                const float e = vo_exp_avx2((x[j + c] - maxv) * inv_t);
                y[j + c] = e;
                s[c] = s[c] + e;
            }
        float sum = ((s[0] + s[4]) + (s[1] + s[5])) + ((s[2] + s[6]) + (s[3] + s[7]));
        for (uint32_t j = c8; j < cols; ++j) {
            const float e = vo_fast_expf_fma((x[j] - maxv) * inv_t);
            y[j] = e;
            sum = sum + e;
        }
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (uint32_t j = 0; j < cols; ++j) y[j] = y[j] * inv;
    }
}

/* The elementwise commands run as ranges [c * grain, min(count, (c + 1) *
 * grain)) (scheduler.cpp:536-581 with grain = max(4096, count / (4 *
 * num_threads)); ThreadPool::parallel_for, internal.h:273-340, hands each
 * range to a *_avx2_range call), and each range runs 8-wide steps from its
 * own start and the last (length % 8) elements in its scalar tail.  grain 0
 * (or >= count) is one range.  The hybrid-core weighted split of
 * parallel_for (internal.h:301-340: a device whose units run at different
 * speeds and few chunks) is host-specific and not restated. */
static int vo_in_tail(uint64_t i, uint64_t count, uint64_t grain)
{
    if (grain == 0 || grain > count) grain = count;
    const uint64_t b = i / grain * grain;
    const uint64_t len = count - b < grain ? count - b : grain;
    return i - b >= (len & ~(uint64_t)7);
}

void vo_swiglu_avx2(const float *gate, const float *up, float *Y, uint64_t count, float alpha,
                    uint64_t grain)
{
    float a = alpha == 0.0f ? 1.0f : alpha;
    for (uint64_t i = 0; i < count; ++i) {
        float g = gate[i];
        /* vector: exp256_ps clamps to [-80, 80]; tail: silu() with the
         * scalar fast_expf (llm.cpp:240-246 inlined into swiglu_avx2_range) */
        float s = g / (1.0f + (vo_in_tail(i, count, grain) ? vo_fast_expf_fma(-g) : vo_exp_avx2(-g)));
        Y[i] = (s * up[i]) * a;
    }
}

/* gelu_avx2_range (llm.cpp:308-330): inner = k0 * fma(k1, x^3, x),
 * t = 2 / (1 + exp256(-2 inner)) - 1, y = (0.5 x)(1 + t). */
void vo_gelu_avx2(const float *X, float *Y, uint64_t count)
{
    for (uint64_t i = 0; i < count; ++i) {
        float x = X[i];
        float x3 = (x * x) * x;
        float inner = 0.7978845608028654f * fmaf(0.035677408136300125f, x3, x);
        float e = vo_exp_avx2(-2.0f * inner);
        float t = 2.0f / (1.0f + e) - 1.0f;
        Y[i] = (0.5f * x) * (1.0f + t);
    }
}

/* mul_avx2_range (llm.cpp:273-287): y = fma(a*b, alpha, beta) in the 8-wide
 * steps; the tail's alpha * a * b + beta contracts to fma(alpha*a, b, beta). */
void vo_mul_avx2(const float *A, const float *B, float *Y, uint64_t count, float alpha, float beta,
                 uint64_t grain)
{
    float a = alpha == 0.0f ? 1.0f : alpha;
    for (uint64_t i = 0; i < count; ++i)
        Y[i] = vo_in_tail(i, count, grain) ? fmaf(a * A[i], B[i], beta) : fmaf(A[i] * B[i], a, beta);
}

/* add_avx2_range (llm.cpp:256-271): y = fma(a, alpha, b*beta); the tail's
 * alpha * a + beta * b contracts to the same fma. */
void vo_add_avx2(const float *A, const float *B, float *Y, uint64_t count, float alpha, float beta)
{
    float al = (alpha == 0.0f && beta == 0.0f) ? 1.0f : alpha;
    float be = (alpha == 0.0f && beta == 0.0f) ? 1.0f : beta;
    for (uint64_t i = 0; i < count; ++i) Y[i] = fmaf(A[i], al, B[i] * be);
}

/* dot_avx2 (llm.cpp:332-343): eight FMA chains over 8-wide steps, hsum256,
 * then the tail (vo_tail_dot). */
static float vo_dot_avx2(const float *a, const float *b, uint32_t n)
{
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint32_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
    return vo_tail_dot(a + i, b + i, n - i, vo_hsum8(acc));
}

/* attention_range (llm.cpp:442-546) with its AVX2 helpers: scores by
 * dot_avx2, the online softmax in the function's own (non-AVX2, so unfused)
 * scalar arithmetic with the scalar fast_expf, acc by axpy_avx2 (FMA). */
void vo_attention_avx2(const float *Q, const float *K, const float *V, const float *mask, float *O,
                       uint32_t batch, uint32_t heads, uint32_t seq_q, uint32_t seq_k,
                       uint32_t head_dim, uint32_t causal, float scale)
{
    enum { BQ = 16, BK = 64 };
    const uint32_t D = head_dim;
    if (!(scale > 0.0f)) scale = 1.0f / sqrtf((float)D);
    float scores[BQ * BK], probs[BQ * BK], m[BQ], l[BQ];
    float *acc = (float *)malloc((size_t)BQ * D * sizeof(float));
    const uint32_t off = seq_k > seq_q ? seq_k - seq_q : 0;
    for (uint64_t bh = 0; bh < (uint64_t)batch * heads; ++bh) {
        const float *Qh = Q + bh * seq_q * D;
        const float *Kh = K + bh * seq_k * D;
        const float *Vh = V + bh * seq_k * D;
        const float *Mh = mask ? mask + bh * seq_q * seq_k : NULL;
        float *Oh = O + bh * seq_q * D;
        for (uint32_t q0 = 0; q0 < seq_q; q0 += BQ) {
            uint32_t qc = umin(BQ, seq_q - q0);
            for (uint32_t i = 0; i < qc; ++i) {
                m[i] = -INFINITY;
                l[i] = 0.0f;
                for (uint32_t d = 0; d < D; ++d) acc[i * D + d] = 0.0f;
            }
            for (uint32_t k0 = 0; k0 < seq_k; k0 += BK) {
                uint32_t kc = umin(BK, seq_k - k0);
                for (uint32_t i = 0; i < qc; ++i) {
                    uint32_t qi = q0 + i;
                    for (uint32_t j = 0; j < kc; ++j) {
                        uint32_t ki = k0 + j;
                        float s;
                        if (causal && ki > qi + off) {
                            s = -INFINITY;
                        } else {
                            s = vo_dot_avx2(Qh + (size_t)qi * D, Kh + (size_t)ki * D, D) * scale;
                            if (Mh) s += Mh[(size_t)qi * seq_k + ki];
                        }
                        scores[i * BK + j] = s;
                    }
                }
                for (uint32_t i = 0; i < qc; ++i) {
                    float bmax = -INFINITY;
                    for (uint32_t j = 0; j < kc; ++j)
                        bmax = (bmax < scores[i * BK + j]) ? scores[i * BK + j] : bmax;
                    if (!isfinite(bmax)) continue;
                    float new_m = (m[i] < bmax) ? bmax : m[i];
                    float alpha = vo_fast_expf(m[i] - new_m);
                    float sum_p = 0.0f;
                    for (uint32_t j = 0; j < kc; ++j) {
                        float p = vo_fast_expf(scores[i * BK + j] - new_m);
                        probs[i * BK + j] = p;
                        sum_p += p;
                    }
                    l[i] = l[i] * alpha + sum_p;
                    for (uint32_t d = 0; d < D; ++d) acc[i * D + d] *= alpha;
                    for (uint32_t j = 0; j < kc; ++j) {
                        float p = probs[i * BK + j];
                        if (p == 0.0f) continue;
                        const float *v = Vh + (size_t)(k0 + j) * D;
                        for (uint32_t d = 0; d < D; ++d) acc[i * D + d] = fmaf(v[d], p, acc[i * D + d]);
                    }
                    m[i] = new_m;
                }
            }
            for (uint32_t i = 0; i < qc; ++i) {
                float inv = l[i] > 0.0f ? 1.0f / l[i] : 0.0f;
                for (uint32_t d = 0; d < D; ++d) Oh[(size_t)(q0 + i) * D + d] = acc[i * D + d] * inv;
            }
        }
    }
    free(acc);
}
