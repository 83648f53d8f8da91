/*
 * m1moe_oracle.h — scalar CPU oracle for the MoE-layer decode path of
 * koaWood/M1MoE (router softmax/top-K, expert dispatch, 4-bit group affine
 * dequant + SwiGLU gate/up/down matvec, weighted combine).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP
 * implementation is compared against.  Only the test-suite, the smoke check
 * and the CPU-baseline leg of the benchmark may load it; the product library
 * (libm1moe_hip.so) never links, loads or calls it.
 *
 * Every function cites the reference file:line whose arithmetic it restates.
 * Reference paths are relative to the koaWood/M1MoE checkout.
 */
#ifndef M1MOE_ORACLE_H
#define M1MOE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int32_t hidden;        /* ModelSpec.hiddenDim */
    int32_t num_experts;   /* MoESpec.numExperts */
    int32_t top_k;         /* MoESpec.topK */
    int32_t intermediate;  /* MoESpec.intermediateDim */
    int32_t group_size;    /* QuantSpec.groupSize */
    int32_t norm_topk_prob;/* MoESpec.normTopkProb */
} orc_shape;

/* Byte offsets of the nine planar sub-blocks of one expert block.
 * InferenceEngine.swift:84-97; scripts/extract_olmoe.py:20-32,321-338. */
typedef struct {
    uint64_t gate_w, gate_s, gate_b;
    uint64_t up_w, up_s, up_b;
    uint64_t down_w, down_s, down_b;
    uint64_t expert_bytes;
} orc_offsets;

/* Top-K selection key.  ORC_KEY_LOGIT: descending logit, ties to the lower
 * expert index (the pinned semantics the GPU implements).  ORC_KEY_PROB:
 * descending softmax probability with a stable order, i.e. the reference's
 * literal `indexed.sort { $0.1 > $1.1 }` (InferenceEngine.swift:511-513). */
enum { ORC_KEY_LOGIT = 0, ORC_KEY_PROB = 1 };

/* InferenceEngine.swift:603-606 / Shaders.metal:11-14 */
float orc_bf16_to_f32(uint16_t v);

/* ModelSpec.swift:36-52 and InferenceEngine.swift:84-97 */
void orc_expert_offsets(const orc_shape* s, orc_offsets* out);

/* Dequantised weights of one projection (0=gate, 1=up, 2=down) of one expert
 * block, row-major [rows x cols], value f32(n)*f32(s) + f32(b).
 * Shaders.metal:66-77; scripts/extract_olmoe.py:145-150. */
void orc_dequant_proj(const orc_shape* s, const uint8_t* expert_block,
                      int32_t proj, float* out);

/* matvec4bit, Shaders.metal:39-92: 64 lane-strided partial sums of
 * fma(n, s*x, fma(b, x, acc)) followed by the threadgroup tree reduction.
 * orc_matvec4bit_lanes is the restatement, lane by lane; orc_matvec4bit
 * computes the same bits eight lanes at a time where the CPU has AVX2. */
void orc_matvec4bit_lanes(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                          const float* x, float* y, int32_t out_dim, int32_t in_dim,
                          int32_t gs);
void orc_matvec4bit(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                    const float* x, float* y, int32_t out_dim, int32_t in_dim,
                    int32_t gs);
/* on != 0: orc_matvec4bit always runs the lane-by-lane restatement. */
void orc_set_scalar(int32_t on);

/* Double-precision brute force of the same matvec: sum_c (n*s+b)*x_c. */
void orc_matvec4bit_f64(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                        const float* x, double* y, int32_t out_dim,
                        int32_t in_dim, int32_t gs);

/* swiGLU, Shaders.metal:138-149 */
void orc_swiglu(const float* gate, const float* up, float* act, int32_t n);

/* computeRouterScores, InferenceEngine.swift:490-500 (logits).  Products are
 * formed exactly and accumulated in f64, then rounded once to f32. */
void orc_router_logits(const uint16_t* router_bf16, const float* x,
                       int32_t num_experts, int32_t hidden, float* logits);

/* The reference's literal f32 sequential dot (InferenceEngine.swift:495-499),
 * kept to quantify the f64-accumulation refinement. */
void orc_router_logits_seq_f32(const uint16_t* router_bf16, const float* x,
                               int32_t num_experts, int32_t hidden,
                               float* logits);

/* softmax, InferenceEngine.swift:501-507 */
void orc_softmax(const float* logits, int32_t n, float* probs);

/* selectTopK, InferenceEngine.swift:510-519 (see ORC_KEY_*). */
void orc_select_topk(const float* logits, const float* probs, int32_t n,
                     int32_t k, int32_t norm_topk_prob, int32_t key_mode,
                     int32_t* idx, float* w);

/* moeCombine, Shaders.metal:360-376 (residual may be NULL = zeros). */
void orc_combine(const float* expert_outs, const float* w,
                 const float* residual, float* out, int32_t k, int32_t hidden);

/* One expert's FFN, InferenceEngine.swift:401-444:
 * gate/up matvec, SwiGLU, down matvec. */
void orc_expert_forward(const orc_shape* s, const uint8_t* expert_block,
                        const float* x, float* out /* [hidden] */);

/* The whole MoE block for one token, InferenceEngine.swift:240-266.
 * layer_image = E expert blocks (layer_NN.bin), router = bf16 [E x hidden].
 * logit_bias [E] (may be NULL) is added to the logits before softmax/top-K;
 * NULL is the reference's semantics (the reference has no router bias).
 * Outputs: out[hidden]; idx/w [K] (may be NULL); logits [E] (may be NULL,
 * bias included). */
int32_t orc_moe_decode(const orc_shape* s, const uint8_t* layer_image,
                       const uint16_t* router_bf16, const float* logit_bias,
                       const float* x, const float* residual, float* out,
                       int32_t* idx, float* w, float* logits);

/* Same, with the routing supplied (expert dispatch + FFN + combine only). */
int32_t orc_moe_decode_given_topk(const orc_shape* s,
                                  const uint8_t* layer_image,
                                  const float* x, const int32_t* idx,
                                  const float* w, const float* residual,
                                  float* out);

/* T tokens, each through orc_moe_decode independently (the reference's
 * prefill is token-by-token forward, Sources/bench/main.swift:139-141).
 * x [T x hidden], residual [T x hidden] or NULL, out [T x hidden],
 * idx/w [T x K] (may be NULL).  nthreads>1 splits tokens over threads. */
int32_t orc_moe_prefill(const orc_shape* s, const uint8_t* layer_image,
                        const uint16_t* router_bf16, const float* logit_bias,
                        int32_t T, const float* x,
                        const float* residual, float* out, int32_t* idx,
                        float* w, int32_t nthreads);


/* ---- dense decoder step (dense_oracle.c) ---------------------------------- */

/* embedToken, InferenceEngine.swift:482-488: row `token` of the bf16 table. */
void orc_embed(const uint16_t* embed_bf16, int32_t token, int32_t hidden,
               float* out);

/* rmsNormSum + rmsNormApply, Shaders.metal:96-134:
 * out = x * rsqrt(sum(x^2)/n + eps) * w. */
void orc_rmsnorm(const float* x, const uint16_t* w_bf16, float* out, int32_t n,
                 float eps);

/* matvecBF16, Shaders.metal:328-358, then residualAdd (:152-162) when
 * residual is not NULL: y = W x (+ residual), W bf16 [rows x cols]. */
void orc_matvec_bf16(const uint16_t* w_bf16, const float* x,
                     const float* residual, float* y, int32_t rows,
                     int32_t cols);

/* applyHeadRMSNorm, InferenceEngine.swift:538-548 (in place; w has head_dim
 * entries shared by all heads). */
void orc_head_rmsnorm(float* buf, int32_t num_heads, int32_t head_dim,
                      const uint16_t* w_bf16, float eps);

/* applyRoPE, InferenceEngine.swift:521-536 (in place; pairs (p, p+hd/2)). */
void orc_rope(float* buf, int32_t num_heads, int32_t head_dim, float theta,
              int32_t pos);

/* attnScores + attnSoftmax + attnValues, Shaders.metal:209-326 with the
 * dispatch of InferenceEngine.swift:349-399: caches [seq_len x kv_dim] f32,
 * GQA head h reads kv head h / (num_heads / num_kv_heads), scale
 * 1/sqrt(head_dim).  scratch: seq_len doubles.  Returns 0, or -1 on bad
 * dimensions. */
int32_t orc_attention(const float* q, const float* kcache, const float* vcache,
                      float* out, int32_t num_heads, int32_t num_kv_heads,
                      int32_t head_dim, int32_t seq_len, double* scratch);

/* sampleToken at temperature 0, InferenceEngine.swift:550-555: scan from
 * x[0] with a strict >, so ties go to the lower index and NaN never replaces
 * (nor is replaced at index 0). */
int32_t orc_argmax(const float* x, int32_t n);

#ifdef __cplusplus
}
#endif

#endif
