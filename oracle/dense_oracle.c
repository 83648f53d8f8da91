/*
 * dense_oracle.c — scalar CPU restatement of the dense part of a koaWood/M1MoE
 * decoder step (the layers around the MoE block).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP implementation.  Only the
 * test-suite, the smoke check and the benchmark's CPU-baseline leg may load
 * it; nothing in the product library links or calls it.
 *
 * Semantics restated (reference paths relative to the koaWood/M1MoE tree):
 *   token embedding          InferenceEngine.swift:482-488
 *   RMSNorm                  Shaders.metal:96-134, InferenceEngine.swift:298-320
 *   bf16 matvec              Shaders.metal:328-358, InferenceEngine.swift:322-335
 *   residual add             Shaders.metal:152-162
 *   per-head q/k RMSNorm     InferenceEngine.swift:538-548
 *   RoPE (half-split pairs)  InferenceEngine.swift:521-536
 *   attention                Shaders.metal:209-326, InferenceEngine.swift:349-399
 *   greedy argmax            InferenceEngine.swift:550-555
 *
 * Refinement (as for the router logits): every sum — sum of squares, dot
 * product, softmax denominator, weighted V sum — is accumulated in f64 and
 * rounded once to f32 where the reference stores an f32, so the oracle does
 * not depend on a summation order.  Exponentials, powers and trigonometric
 * functions are the reference's f32 ones (expf, powf, cosf, sinf), on the
 * same f32 arguments.
 */
#include <math.h>
#include <string.h>

#include "m1moe_oracle.h"

void orc_embed(const uint16_t* embed_bf16, int32_t token, int32_t hidden,
               float* out) {
    const uint16_t* row = embed_bf16 + (size_t)token * hidden; /* :484 */
    for (int32_t d = 0; d < hidden; ++d) out[d] = orc_bf16_to_f32(row[d]);
}

void orc_rmsnorm(const float* x, const uint16_t* w_bf16, float* out, int32_t n,
                 float eps) {
    double ss = 0.0;
    for (int32_t i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i]; /* :105-108 */
    const float ms = (float)ss / (float)n + eps; /* :131, sumSq stored as f32 */
    const float rms = (float)(1.0 / sqrt((double)ms));
    for (int32_t i = 0; i < n; ++i)
        out[i] = x[i] * rms * orc_bf16_to_f32(w_bf16[i]); /* :132 */
}

void orc_matvec_bf16(const uint16_t* w_bf16, const float* x,
                     const float* residual, float* y, int32_t rows,
                     int32_t cols) {
    for (int32_t r = 0; r < rows; ++r) {
        const uint16_t* wr = w_bf16 + (size_t)r * cols; /* :341 */
        double acc = 0.0;
        for (int32_t c = 0; c < cols; ++c)
            acc += (double)orc_bf16_to_f32(wr[c]) * (double)x[c]; /* :344 */
        const float v = (float)acc;
        y[r] = residual ? residual[r] + v : v; /* residualAdd :161 */
    }
}

void orc_head_rmsnorm(float* buf, int32_t num_heads, int32_t head_dim,
                      const uint16_t* w_bf16, float eps) {
    for (int32_t h = 0; h < num_heads; ++h) {
        float* v = buf + (size_t)h * head_dim;
        double ss = 0.0;
        for (int32_t d = 0; d < head_dim; ++d) ss += (double)v[d] * (double)v[d]; /* :543 */
        const float rms = 1.0f / sqrtf((float)ss / (float)head_dim + eps);      /* :544 */
        for (int32_t d = 0; d < head_dim; ++d)
            v[d] *= rms * orc_bf16_to_f32(w_bf16[d]); /* :545 */
    }
}

void orc_rope(float* buf, int32_t num_heads, int32_t head_dim, float theta,
              int32_t pos) {
    const int32_t half = head_dim / 2;
    for (int32_t h = 0; h < num_heads; ++h) {
        float* v = buf + (size_t)h * head_dim;
        for (int32_t p = 0; p < half; ++p) {
            const float freq = 1.0f / powf(theta, (float)(2 * p) / (float)head_dim); /* :527 */
            const float angle = (float)pos * freq;                                 /* :528 */
            const float c = cosf(angle), s = sinf(angle);
            const float x0 = v[p], x1 = v[p + half];
            v[p] = x0 * c - x1 * s; /* :532 */
            v[p + half] = x0 * s + x1 * c;
        }
    }
}

int32_t orc_attention(const float* q, const float* kcache, const float* vcache,
                      float* out, int32_t num_heads, int32_t num_kv_heads,
                      int32_t head_dim, int32_t seq_len, double* scratch) {
    if (num_kv_heads <= 0 || num_heads % num_kv_heads || seq_len <= 0) return -1;
    const int32_t hpkv = num_heads / num_kv_heads;
    const size_t kvd = (size_t)num_kv_heads * head_dim;
    const float scale = 1.0f / sqrtf((float)head_dim); /* :354 */
    for (int32_t h = 0; h < num_heads; ++h) {
        const float* qh = q + (size_t)h * head_dim;
        const int32_t kvh = h / hpkv; /* :225 */
        double mx = -INFINITY;
        for (int32_t p = 0; p < seq_len; ++p) {
            const float* kp = kcache + (size_t)p * kvd + (size_t)kvh * head_dim;
            double acc = 0.0;
            for (int32_t d = 0; d < head_dim; ++d) acc += (double)qh[d] * (double)kp[d];
            const float sc = (float)acc * scale; /* :242 */
            scratch[p] = sc;
            if (sc > mx) mx = sc;
        }
        double sum = 0.0;
        for (int32_t p = 0; p < seq_len; ++p) { /* :265-273 */
            const float e = expf((float)scratch[p] - (float)mx);
            scratch[p] = e;
            sum += e;
        }
        for (int32_t d = 0; d < head_dim; ++d) { /* :318-324 */
            double acc = 0.0;
            for (int32_t p = 0; p < seq_len; ++p)
                acc += scratch[p] * (double)vcache[(size_t)p * kvd + (size_t)kvh * head_dim + d];
            out[(size_t)h * head_dim + d] = (float)(acc / sum);
        }
    }
    return 0;
}

int32_t orc_argmax(const float* x, int32_t n) {
    int32_t best = 0;
    float bv = x[0];
    for (int32_t i = 1; i < n; ++i) /* :552-553 */
        if (x[i] > bv) {
            bv = x[i];
            best = i;
        }
    return best;
}
