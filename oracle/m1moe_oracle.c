/*
 * m1moe_oracle.c — scalar CPU restatement of the MoE-layer decode path of
 * koaWood/M1MoE.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP implementation.  Only the
 * test-suite, the smoke check and the benchmark's CPU-baseline leg may load
 * it; nothing in the product library links or calls it.
 *
 * Semantics restated (reference paths relative to the koaWood/M1MoE tree):
 *   expert block layout     ModelSpec.swift:36-52, InferenceEngine.swift:84-97,
 *                           scripts/extract_olmoe.py:20-32,145-150,321-338
 *   4-bit dequant matvec    Shaders.metal:39-92
 *   SwiGLU                  Shaders.metal:138-149
 *   router + softmax        InferenceEngine.swift:490-508
 *   top-K (+ renorm)        InferenceEngine.swift:510-519
 *   expert FFN sequence     InferenceEngine.swift:401-444
 *   combine + residual      Shaders.metal:360-376
 *   MoE block               InferenceEngine.swift:240-266
 *
 * Two deliberate refinements, both pinned by tests:
 *   - router logits: exact products accumulated in f64 and rounded once to
 *     f32, so that the value does not depend on summation order (the
 *     reference's sequential f32 sum is kept as orc_router_logits_seq_f32);
 *   - top-K key: descending logit, ties to the lower index.  Softmax is
 *     monotone, so this equals the reference's stable sort on probabilities
 *     except where two distinct logits round to the same f32 probability.
 */
#include "m1moe_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

float orc_bf16_to_f32(uint16_t v) {
    uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

void orc_expert_offsets(const orc_shape* s, orc_offsets* o) {
    const uint64_t h = (uint64_t)s->hidden, i = (uint64_t)s->intermediate;
    const uint64_t gs = (uint64_t)s->group_size;
    const uint64_t gw = i * (h / 8) * 4;   /* gate/up packed words */
    const uint64_t gsb = i * (h / gs) * 2; /* gate/up scales or biases */
    const uint64_t dw = h * (i / 8) * 4;   /* down packed words */
    const uint64_t dsb = h * (i / gs) * 2; /* down scales or biases */
    o->gate_w = 0;
    o->gate_s = o->gate_w + gw;
    o->gate_b = o->gate_s + gsb;
    o->up_w = o->gate_b + gsb;
    o->up_s = o->up_w + gw;
    o->up_b = o->up_s + gsb;
    o->down_w = o->up_b + gsb;
    o->down_s = o->down_w + dw;
    o->down_b = o->down_s + dsb;
    o->expert_bytes = o->down_b + dsb;
}

static void proj_ptrs(const orc_shape* s, const uint8_t* blk, int32_t proj,
                      const uint32_t** w, const uint16_t** sc,
                      const uint16_t** bi, int32_t* rows, int32_t* cols) {
    orc_offsets o;
    orc_expert_offsets(s, &o);
    if (proj == 0) {
        *w = (const uint32_t*)(blk + o.gate_w);
        *sc = (const uint16_t*)(blk + o.gate_s);
        *bi = (const uint16_t*)(blk + o.gate_b);
        *rows = s->intermediate;
        *cols = s->hidden;
    } else if (proj == 1) {
        *w = (const uint32_t*)(blk + o.up_w);
        *sc = (const uint16_t*)(blk + o.up_s);
        *bi = (const uint16_t*)(blk + o.up_b);
        *rows = s->intermediate;
        *cols = s->hidden;
    } else {
        *w = (const uint32_t*)(blk + o.down_w);
        *sc = (const uint16_t*)(blk + o.down_s);
        *bi = (const uint16_t*)(blk + o.down_b);
        *rows = s->hidden;
        *cols = s->intermediate;
    }
}

void orc_dequant_proj(const orc_shape* s, const uint8_t* blk, int32_t proj,
                      float* out) {
    const uint32_t* w;
    const uint16_t *sc, *bi;
    int32_t rows, cols;
    proj_ptrs(s, blk, proj, &w, &sc, &bi, &rows, &cols);
    const int32_t words = cols / 8, groups = cols / s->group_size;
    for (int32_t r = 0; r < rows; ++r) {
        for (int32_t c = 0; c < cols; ++c) {
            const uint32_t packed = w[(size_t)r * words + c / 8];
            const uint32_t n = (packed >> (4 * (c % 8))) & 0xFu; /* :74 */
            const int32_t g = c / s->group_size;                 /* :67 */
            const float scale = orc_bf16_to_f32(sc[(size_t)r * groups + g]);
            const float bias = orc_bf16_to_f32(bi[(size_t)r * groups + g]);
            /* n*scale has at most 12 significant bits, so it is exact in
             * f32 and the sum is the only rounding. */
            out[(size_t)r * cols + c] = (float)n * scale + bias;
        }
    }
}

/* The restatement itself: lane by lane, one row at a time. */
void orc_matvec4bit_lanes(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                          const float* x, float* y, int32_t out_dim, int32_t in_dim,
                          int32_t gs) {
    const uint32_t num_words = (uint32_t)in_dim / 8;   /* :55 */
    const uint32_t num_groups = (uint32_t)in_dim / gs; /* :56 */
    float shared[64];
    for (int32_t row = 0; row < out_dim; ++row) {
        const uint32_t* w_row = w + (size_t)row * num_words;  /* :59 */
        const uint16_t* s_row = s + (size_t)row * num_groups; /* :60 */
        const uint16_t* b_row = b + (size_t)row * num_groups; /* :61 */
        for (uint32_t lid = 0; lid < 64; ++lid) {
            float acc = 0.0f;
            for (uint32_t wi = lid; wi < num_words; wi += 64) { /* :65 */
                const uint32_t packed = w_row[wi];
                const uint32_t g = (wi * 8) / (uint32_t)gs;
                const float scale = orc_bf16_to_f32(s_row[g]);
                const float bias = orc_bf16_to_f32(b_row[g]);
                const uint32_t base = wi * 8;
                for (uint32_t bb = 0; bb < 8; ++bb) { /* :73-78 */
                    const float nib = (float)((packed >> (bb * 4)) & 0xFu);
                    const float xv = x[base + bb];
                    acc = fmaf(nib, scale * xv, fmaf(bias, xv, acc));
                }
            }
            shared[lid] = acc; /* :83 */
        }
        for (uint32_t st = 32; st > 0; st >>= 1) /* :86-89 */
            for (uint32_t lid = 0; lid < st; ++lid)
                shared[lid] += shared[lid + st];
        y[row] = shared[0]; /* :91 */
    }
}

/* The same arithmetic with eight lanes per AVX2 register: lane l of the
 * restatement is element l % 8 of accumulator l / 8, and every lane performs
 * exactly the restatement's operations in its order (the same fused
 * multiply-adds and the same f32 product scale * x), so the result is equal
 * bit for bit (pinned by a test against orc_matvec4bit_lanes).  Eight
 * consecutive lanes read eight consecutive packed words; x is transposed
 * once so that the eight x values of nibble bb of those words are
 * contiguous. */
__attribute__((target("avx2,fma"))) static void matvec4bit_avx2(
    const uint32_t* w, const uint16_t* s, const uint16_t* b, const float* x, float* y,
    int32_t out_dim, int32_t in_dim, int32_t gs, float* xt) {
    const uint32_t num_words = (uint32_t)in_dim / 8;
    const uint32_t num_groups = (uint32_t)in_dim / (uint32_t)gs;
    for (uint32_t wi = 0; wi < num_words; ++wi)
        for (uint32_t bb = 0; bb < 8; ++bb) xt[(size_t)bb * num_words + wi] = x[wi * 8 + bb];
    const __m256i mask = _mm256_set1_epi32(0xF);
    /* words per scale group: gs is a multiple of 8 (32, 64 or 128), and a
     * lane block starts at a multiple of 8 words */
    const uint32_t wpg = (uint32_t)gs / 8;
    float shared[64];
    for (int32_t row = 0; row < out_dim; ++row) {
        const uint32_t* w_row = w + (size_t)row * num_words;
        const uint16_t* s_row = s + (size_t)row * num_groups;
        const uint16_t* b_row = b + (size_t)row * num_groups;
        __m256 acc[8];
        for (int lb = 0; lb < 8; ++lb) acc[lb] = _mm256_setzero_ps();
        for (uint32_t k0 = 0; k0 < num_words; k0 += 64) {
            for (uint32_t lb = 0; lb < 8; ++lb) {
                const uint32_t wi0 = k0 + lb * 8;   /* lanes lb*8 .. lb*8+7 */
                if (wi0 >= num_words) break;
                __m256 scale, bias;
                if (wpg >= 8) {   /* the eight words share one group */
                    const uint32_t g = wi0 / wpg;
                    scale = _mm256_set1_ps(orc_bf16_to_f32(s_row[g]));
                    bias = _mm256_set1_ps(orc_bf16_to_f32(b_row[g]));
                } else {
                    float sv[8], bv[8];
                    for (uint32_t j = 0; j < 8; ++j) {
                        const uint32_t g = (wi0 + j) / wpg;
                        sv[j] = orc_bf16_to_f32(s_row[g]);
                        bv[j] = orc_bf16_to_f32(b_row[g]);
                    }
                    scale = _mm256_loadu_ps(sv);
                    bias = _mm256_loadu_ps(bv);
                }
                const __m256i packed = _mm256_loadu_si256((const __m256i*)(w_row + wi0));
                __m256 a = acc[lb];
                for (uint32_t bb = 0; bb < 8; ++bb) {
                    const __m256 nib = _mm256_cvtepi32_ps(
                        _mm256_and_si256(_mm256_srli_epi32(packed, (int)(bb * 4)), mask));
                    const __m256 xv = _mm256_loadu_ps(xt + (size_t)bb * num_words + wi0);
                    a = _mm256_fmadd_ps(nib, _mm256_mul_ps(scale, xv),
                                        _mm256_fmadd_ps(bias, xv, a));
                }
                acc[lb] = a;
            }
        }
        for (int lb = 0; lb < 8; ++lb) _mm256_storeu_ps(shared + lb * 8, acc[lb]);
        for (uint32_t st = 32; st > 0; st >>= 1)
            for (uint32_t lid = 0; lid < st; ++lid) shared[lid] += shared[lid + st];
        y[row] = shared[0];
    }
}

/* Set by orc_set_scalar(): every matvec4bit runs the lane-by-lane
 * restatement (the benchmark's scalar CPU baseline).  Set it before any
 * thread uses the oracle. */
static int g_scalar_only = 0;

void orc_set_scalar(int32_t on) { g_scalar_only = on != 0; }

/* Shaders.metal:39-92 (matvec4bit): the AVX2 form where the CPU has it and
 * the row length is a whole number of eight-word lane blocks, else the
 * lane-by-lane restatement. */
void orc_matvec4bit(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                    const float* x, float* y, int32_t out_dim, int32_t in_dim,
                    int32_t gs) {
    const int have_avx2 = !g_scalar_only && __builtin_cpu_supports("avx2") &&
                          __builtin_cpu_supports("fma");
    float* xt = NULL;
    if (have_avx2 && in_dim % 64 == 0) xt = (float*)malloc((size_t)in_dim * sizeof(float));
    if (xt) {
        matvec4bit_avx2(w, s, b, x, y, out_dim, in_dim, gs, xt);
        free(xt);
    } else {
        orc_matvec4bit_lanes(w, s, b, x, y, out_dim, in_dim, gs);
    }
}

void orc_matvec4bit_f64(const uint32_t* w, const uint16_t* s,
                        const uint16_t* b, const float* x, double* y,
                        int32_t out_dim, int32_t in_dim, int32_t gs) {
    const int32_t words = in_dim / 8, groups = in_dim / gs;
    for (int32_t r = 0; r < out_dim; ++r) {
        double acc = 0.0;
        for (int32_t c = 0; c < in_dim; ++c) {
            const uint32_t n = (w[(size_t)r * words + c / 8] >> (4 * (c % 8))) & 0xFu;
            const double sc = orc_bf16_to_f32(s[(size_t)r * groups + c / gs]);
            const double bi = orc_bf16_to_f32(b[(size_t)r * groups + c / gs]);
            acc += ((double)n * sc + bi) * (double)x[c];
        }
        y[r] = acc;
    }
}

void orc_swiglu(const float* gate, const float* up, float* act, int32_t n) {
    for (int32_t i = 0; i < n; ++i) {
        const float g = gate[i];
        act[i] = (g / (1.0f + expf(-g))) * up[i]; /* Shaders.metal:147-148 */
    }
}

void orc_router_logits(const uint16_t* router_bf16, const float* x,
                       int32_t num_experts, int32_t hidden, float* logits) {
    for (int32_t e = 0; e < num_experts; ++e) {
        const uint16_t* row = router_bf16 + (size_t)e * hidden;
        double acc = 0.0;
        for (int32_t d = 0; d < hidden; ++d) {
            /* bf16 (8 significant bits) x f32 (24 bits) is exact in f64 */
            acc += (double)orc_bf16_to_f32(row[d]) * (double)x[d];
        }
        logits[e] = (float)acc;
    }
}

void orc_router_logits_seq_f32(const uint16_t* router_bf16, const float* x,
                               int32_t num_experts, int32_t hidden,
                               float* logits) {
    for (int32_t e = 0; e < num_experts; ++e) {
        const uint16_t* row = router_bf16 + (size_t)e * hidden;
        float dot = 0.0f; /* InferenceEngine.swift:496-498 (no contraction) */
        for (int32_t d = 0; d < hidden; ++d) {
            const float p = orc_bf16_to_f32(row[d]) * x[d];
            dot = dot + p;
        }
        logits[e] = dot;
    }
}

void orc_softmax(const float* logits, int32_t n, float* probs) {
    float mx = logits[0]; /* :502 */
    for (int32_t e = 1; e < n; ++e)
        if (logits[e] > mx) mx = logits[e];
    float sum = 0.0f;
    for (int32_t e = 0; e < n; ++e) { /* :504 */
        probs[e] = expf(logits[e] - mx);
        sum += probs[e];
    }
    const float inv = 1.0f / sum; /* :505 */
    for (int32_t e = 0; e < n; ++e) probs[e] *= inv;
}

void orc_select_topk(const float* logits, const float* probs, int32_t n,
                     int32_t k, int32_t norm_topk_prob, int32_t key_mode,
                     int32_t* idx, float* w) {
    const float* key = (key_mode == ORC_KEY_PROB) ? probs : logits;
    unsigned char* taken = (unsigned char*)calloc((size_t)n, 1);
    for (int32_t slot = 0; slot < k; ++slot) {
        int32_t best = -1;
        for (int32_t e = 0; e < n; ++e) {
            if (taken[e]) continue;
            /* strict '>' keeps the lowest index among equal keys, which is
             * the order a stable descending sort produces */
            if (best < 0 || key[e] > key[best]) best = e;
        }
        taken[best] = 1;
        idx[slot] = best;
        w[slot] = probs[best];
    }
    free(taken);
    if (norm_topk_prob) { /* :514-517 */
        float ssum = 0.0f;
        for (int32_t slot = 0; slot < k; ++slot) ssum = ssum + w[slot];
        for (int32_t slot = 0; slot < k; ++slot) w[slot] = w[slot] / ssum;
    }
}

void orc_combine(const float* expert_outs, const float* w,
                 const float* residual, float* out, int32_t k, int32_t hidden) {
    for (int32_t d = 0; d < hidden; ++d) {
        float acc = residual ? residual[d] : 0.0f; /* Shaders.metal:371 */
        for (int32_t j = 0; j < k; ++j)            /* :372-374 */
            acc = fmaf(w[j], expert_outs[(size_t)j * hidden + d], acc);
        out[d] = acc;
    }
}

void orc_expert_forward(const orc_shape* s, const uint8_t* blk,
                        const float* x, float* out) {
    const int32_t h = s->hidden, I = s->intermediate, gs = s->group_size;
    orc_offsets o;
    orc_expert_offsets(s, &o);
    float* gate = (float*)malloc(sizeof(float) * (size_t)I);
    float* up = (float*)malloc(sizeof(float) * (size_t)I);
    float* act = (float*)malloc(sizeof(float) * (size_t)I);
    /* InferenceEngine.swift:408-414 gate_proj */
    orc_matvec4bit((const uint32_t*)(blk + o.gate_w),
                   (const uint16_t*)(blk + o.gate_s),
                   (const uint16_t*)(blk + o.gate_b), x, gate, I, h, gs);
    /* :417-423 up_proj */
    orc_matvec4bit((const uint32_t*)(blk + o.up_w),
                   (const uint16_t*)(blk + o.up_s),
                   (const uint16_t*)(blk + o.up_b), x, up, I, h, gs);
    orc_swiglu(gate, up, act, I); /* :426-433 */
    /* :436-443 down_proj */
    orc_matvec4bit((const uint32_t*)(blk + o.down_w),
                   (const uint16_t*)(blk + o.down_s),
                   (const uint16_t*)(blk + o.down_b), act, out, h, I, gs);
    free(gate);
    free(up);
    free(act);
}

int32_t orc_moe_decode_given_topk(const orc_shape* s,
                                  const uint8_t* layer_image, const float* x,
                                  const int32_t* idx, const float* w,
                                  const float* residual, float* out) {
    orc_offsets o;
    orc_expert_offsets(s, &o);
    const int32_t K = s->top_k, h = s->hidden;
    for (int32_t j = 0; j < K; ++j)
        if (idx[j] < 0 || idx[j] >= s->num_experts) return 1;
    float* eo = (float*)malloc(sizeof(float) * (size_t)K * h);
    for (int32_t j = 0; j < K; ++j) /* :252-260, expert base = idx*expertBytes */
        orc_expert_forward(s, layer_image + (size_t)idx[j] * o.expert_bytes, x,
                           eo + (size_t)j * h);
    orc_combine(eo, w, residual, out, K, h); /* :261 */
    free(eo);
    return 0;
}

int32_t orc_moe_decode(const orc_shape* s, const uint8_t* layer_image,
                       const uint16_t* router_bf16, const float* logit_bias,
                       const float* x, const float* residual, float* out,
                       int32_t* idx, float* w, float* logits) {
    const int32_t E = s->num_experts, K = s->top_k;
    if (K < 1 || K > E) return 1;
    float* lg = (float*)malloc(sizeof(float) * (size_t)E);
    float* pr = (float*)malloc(sizeof(float) * (size_t)E);
    int32_t* li = (int32_t*)malloc(sizeof(int32_t) * (size_t)K);
    float* lw = (float*)malloc(sizeof(float) * (size_t)K);
    orc_router_logits(router_bf16, x, E, s->hidden, lg); /* :243 */
    if (logit_bias)
        for (int32_t e = 0; e < E; ++e) lg[e] = lg[e] + logit_bias[e];
    orc_softmax(lg, E, pr);
    orc_select_topk(lg, pr, E, K, s->norm_topk_prob, ORC_KEY_LOGIT, li, lw);
    const int32_t rc =
        orc_moe_decode_given_topk(s, layer_image, x, li, lw, residual, out);
    if (idx) memcpy(idx, li, sizeof(int32_t) * (size_t)K);
    if (w) memcpy(w, lw, sizeof(float) * (size_t)K);
    if (logits) memcpy(logits, lg, sizeof(float) * (size_t)E);
    free(lg);
    free(pr);
    free(li);
    free(lw);
    return rc;
}

typedef struct {
    const orc_shape* s;
    const uint8_t* img;
    const uint16_t* router;
    const float* bias;
    const float* x;
    const float* res;
    float* out;
    int32_t* idx;
    float* w;
    int32_t t0, t1;
    int32_t rc;
} prefill_job;

static void* prefill_worker(void* arg) {
    prefill_job* j = (prefill_job*)arg;
    const size_t h = (size_t)j->s->hidden, K = (size_t)j->s->top_k;
    j->rc = 0;
    for (int32_t t = j->t0; t < j->t1; ++t) {
        const int32_t rc = orc_moe_decode(
            j->s, j->img, j->router, j->bias, j->x + t * h,
            j->res ? j->res + t * h : NULL, j->out + t * h,
            j->idx ? j->idx + t * K : NULL, j->w ? j->w + t * K : NULL, NULL);
        if (rc) j->rc = rc;
    }
    return NULL;
}

int32_t orc_moe_prefill(const orc_shape* s, const uint8_t* layer_image,
                        const uint16_t* router_bf16, const float* logit_bias,
                        int32_t T, const float* x, const float* residual,
                        float* out, int32_t* idx, float* w, int32_t nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > T) nthreads = T > 0 ? T : 1;
    prefill_job* jobs = (prefill_job*)calloc((size_t)nthreads, sizeof *jobs);
    pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof *th);
    for (int32_t i = 0; i < nthreads; ++i) {
        prefill_job j = {s, layer_image, router_bf16, logit_bias, x, residual,
                         out, idx, w, (int32_t)((int64_t)T * i / nthreads),
                         (int32_t)((int64_t)T * (i + 1) / nthreads), 0};
        jobs[i] = j;
    }
    for (int32_t i = 1; i < nthreads; ++i)
        pthread_create(&th[i], NULL, prefill_worker, &jobs[i]);
    prefill_worker(&jobs[0]);
    int32_t rc = jobs[0].rc;
    for (int32_t i = 1; i < nthreads; ++i) {
        pthread_join(th[i], NULL);
        if (jobs[i].rc) rc = jobs[i].rc;
    }
    free(jobs);
    free(th);
    return rc;
}
