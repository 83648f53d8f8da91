/*
 * m1moe_hip.h — C ABI of the MI355X (gfx950) MoE-layer decode library
 * libm1moe_hip.so.
 *
 * This is the boundary that replaces the Metal backend of koaWood/M1MoE for
 * the MoE block of a decoder layer (Sources/M1MoE/InferenceEngine.swift:240-266:
 * CPU router + top-K, pread expert dispatch, matvec4bit x3 + swiGLU per slot,
 * moeCombine).  It is plain C99: no HIP, C++ or torch types cross it, so a
 * SwiftPM .systemLibrary target (or ctypes, cgo, ...) can bind it directly.
 *
 * Conventions
 *  - Every call returns int32_t status; M1MOE_OK (0) is success.  On failure
 *    m1moe_last_error() returns a thread-local message for the last failing
 *    call on this thread.
 *  - A context owns all device memory it allocates (expert arena, routers,
 *    scratch, m1moe_alloc buffers) and one HIP stream.  Every compute call is
 *    enqueued asynchronously on that stream; m1moe_sync() waits for it.  A
 *    context is single-threaded (the reference engine is driven from one
 *    serial queue, Sources/bench/main.swift:58); separate contexts are
 *    independent.
 *  - Arguments (shapes, layer/expert ranges, image sizes, dtypes, null
 *    pointers) are validated on the host before anything is enqueued.
 *    Expert indices that arrive in device memory are checked by the kernels;
 *    a bad one sets a sticky device error flag that the next m1moe_sync()
 *    reports (the kernels never read outside the arena).
 *  - Expert weights use the reference's on-disk expert block layout
 *    unchanged (layer_NN.bin): per expert, planar
 *    [gate W|S|B][up W|S|B][down W|S|B]; W = u32 [rows, cols/8] with column
 *    8w+j in bits 4j..4j+3, S/B = bf16 [rows, cols/group_size];
 *    value = nibble*scale + bias (scripts/extract_olmoe.py:20-38,145-150;
 *    ModelSpec.swift:36-52).
 */
#ifndef M1MOE_HIP_H
#define M1MOE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define M1MOE_ABI_VERSION 1

/* status codes */
enum {
    M1MOE_OK = 0,
    M1MOE_ERR_INVALID = 1, /* bad argument: shape, range, size, null pointer */
    M1MOE_ERR_HIP = 2,     /* the HIP runtime reported an error */
    M1MOE_ERR_OOM = 3,     /* device allocation failed */
    M1MOE_ERR_DEVICE = 4   /* a kernel flagged bad device-side input */
};

/* activation dtypes */
enum { M1MOE_F32 = 0, M1MOE_BF16 = 1 };

/* projections of one expert block */
enum { M1MOE_PROJ_GATE = 0, M1MOE_PROJ_UP = 1, M1MOE_PROJ_DOWN = 2 };

typedef struct m1moe_ctx* m1moe_ctx_t;
typedef struct m1moe_graph* m1moe_graph_t;
typedef struct m1moe_event* m1moe_event_t;

/* MoE dimensions of a model.  Mirrors ModelSpec.hiddenDim/numLayers and
 * MoESpec {numExperts, topK, intermediateDim, normTopkProb} and
 * QuantSpec.groupSize (ModelSpec.swift:19-21,82-94).
 * Constraints: hidden and intermediate are multiples of 64; group_size is
 * 32, 64 or 128 and divides both; 1 <= top_k <= num_experts <= 256;
 * top_k <= 32; hidden <= 16384; intermediate <= 32768. */
typedef struct {
    int32_t hidden;
    int32_t num_experts;
    int32_t top_k;
    int32_t intermediate;
    int32_t group_size;
    int32_t num_layers;
    int32_t norm_topk_prob;
} m1moe_moe_shape;

/* ---- host-only queries (no device needed) ----------------------------- */

int32_t m1moe_abi_version(void);

/* Message of the last failing call on the calling thread ("" if none). */
const char* m1moe_last_error(void);

/* Validates a shape against the constraints above. */
int32_t m1moe_check_shape(const m1moe_moe_shape* shape);

/* ModelSpec.expertBytes4Bit (ModelSpec.swift:36-52). */
int32_t m1moe_expert_bytes(const m1moe_moe_shape* shape, uint64_t* out);

/* Byte offsets of the nine sub-blocks inside one expert block, in the order
 * gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s, down_b
 * (InferenceEngine.swift:84-97). */
int32_t m1moe_expert_offsets(const m1moe_moe_shape* shape, uint64_t out[9]);

/* ---- context (replaces MetalContext, MetalContext.swift:69-185) -------- */

/* Creates a context on HIP device `device`: allocates the resident expert
 * arena for num_layers layers (num_layers * num_experts * expert_bytes), the
 * bf16 routers and all scratch.  All experts stay resident in HBM; there is
 * no expert cache or streaming (replaces the pread dispatch,
 * InferenceEngine.swift:62-77,271-280). */
int32_t m1moe_create(int32_t device, const m1moe_moe_shape* shape,
                     m1moe_ctx_t* out);

/* Frees everything the context owns.  NULL is a no-op. */
void m1moe_destroy(m1moe_ctx_t ctx);

/* Copies one layer_NN.bin image (num_experts expert blocks, exactly
 * num_experts * expert_bytes bytes) from host memory into the arena.  The
 * reference zero-fills a missing or short expert read
 * (InferenceEngine.swift:274-279); here a wrong size is an error. */
int32_t m1moe_upload_layer_experts(m1moe_ctx_t ctx, int32_t layer,
                                   const void* host_image, uint64_t bytes);

/* Copies one layer's router (mlp.gate / block_sparse_moe.gate weight, bf16
 * [num_experts x hidden], InferenceEngine.swift:99-113) from host memory.
 * `count` must be num_experts * hidden.  It stays bf16 in HBM. */
int32_t m1moe_upload_router(m1moe_ctx_t ctx, int32_t layer,
                            const uint16_t* host_router, uint64_t count);

/* Optional per-expert f32 logit bias of one layer, added to the router
 * logits before softmax and top-K.  Absent (the default, or host_bias ==
 * NULL) is the reference's semantics; the reference has no router bias. */
int32_t m1moe_set_logit_bias(m1moe_ctx_t ctx, int32_t layer,
                             const float* host_bias, int32_t count);

/* Device pointer to the first byte of (layer, expert)'s block, for callers
 * that fill the arena on the device. */
int32_t m1moe_expert_block(m1moe_ctx_t ctx, int32_t layer, int32_t expert,
                           void** dev_ptr);

/* ---- memory, streams, events, graphs (so callers never include HIP) ---- */

int32_t m1moe_alloc(m1moe_ctx_t ctx, uint64_t bytes, void** dev_ptr);
int32_t m1moe_free(m1moe_ctx_t ctx, void* dev_ptr);
/* Stream-ordered on the context stream; both return after the copy ends. */
int32_t m1moe_copy_h2d(m1moe_ctx_t ctx, void* dev_dst, const void* host_src,
                       uint64_t bytes);
int32_t m1moe_copy_d2h(m1moe_ctx_t ctx, void* host_dst, const void* dev_src,
                       uint64_t bytes);
int32_t m1moe_copy_d2d(m1moe_ctx_t ctx, void* dev_dst, const void* dev_src,
                       uint64_t bytes);

/* Replaces the context stream with a caller-owned hipStream_t (passed as
 * void*); NULL restores the context's own stream. */
int32_t m1moe_set_stream(m1moe_ctx_t ctx, void* hip_stream);
int32_t m1moe_get_stream(m1moe_ctx_t ctx, void** hip_stream);

/* Waits for all work enqueued on the context stream (the reference's
 * commitSync, InferenceEngine.swift:289-294), then reports any sticky device
 * error flag raised by a kernel since the last sync as M1MOE_ERR_DEVICE. */
int32_t m1moe_sync(m1moe_ctx_t ctx);

int32_t m1moe_event_create(m1moe_ctx_t ctx, m1moe_event_t* out);
int32_t m1moe_event_record(m1moe_ctx_t ctx, m1moe_event_t ev);
/* Milliseconds between two recorded events (waits for `end`). */
int32_t m1moe_event_elapsed_ms(m1moe_event_t start, m1moe_event_t end,
                               float* ms);
void m1moe_event_destroy(m1moe_event_t ev);

/* Captures every call enqueued on the context stream between begin and end
 * into a HIP graph (no device work runs during capture). */
int32_t m1moe_graph_begin(m1moe_ctx_t ctx);
int32_t m1moe_graph_end(m1moe_ctx_t ctx, m1moe_graph_t* out);
int32_t m1moe_graph_launch(m1moe_ctx_t ctx, m1moe_graph_t graph);
void m1moe_graph_destroy(m1moe_graph_t graph);

/* ---- the MoE block ------------------------------------------------------ */

/* Router logits, softmax and top-K for T tokens (computeRouterScores +
 * selectTopK, InferenceEngine.swift:490-519, moved on-GPU).
 * d_x: [T x hidden] in x_dtype.  Logits are exact products accumulated in
 * f64 and rounded once to f32 (plus the optional logit bias); experts are
 * ranked by descending logit with ties to the lower index; weights are the
 * softmax probabilities of the selected experts, renormalised over the
 * selection when norm_topk_prob is set (:514-517).
 * Outputs: d_topk_idx int32 [T x top_k], d_topk_w f32 [T x top_k],
 * d_logits f32 [T x num_experts] (nullable). */
int32_t m1moe_router_topk(m1moe_ctx_t ctx, int32_t layer, int32_t T,
                          const void* d_x, int32_t x_dtype,
                          int32_t* d_topk_idx, float* d_topk_w,
                          float* d_logits);

/* One token through the MoE block of `layer` (batch-1 decode):
 *   out[d] = residual[d] + sum_k w_k * down_k(silu(gate_k x) * up_k x)[d]
 * d_x: [hidden] in x_dtype; d_residual: f32 [hidden] or NULL (zeros);
 * d_out: f32 [hidden].  d_topk_idx / d_topk_w (nullable) receive the routing.
 * Replaces InferenceEngine.swift:240-266 (router, dispatch, the 4K+1 Metal
 * dispatches and the residual hand-off).  Asynchronous. */
int32_t m1moe_moe_decode(m1moe_ctx_t ctx, int32_t layer, const void* d_x,
                         int32_t x_dtype, const float* d_residual,
                         float* d_out, int32_t* d_topk_idx, float* d_topk_w);

/* Same, with the routing given in device memory: d_topk_idx int32 [top_k],
 * d_topk_w f32 [top_k] (InferenceEngine.swift:247-263 without the router). */
int32_t m1moe_moe_decode_given_topk(m1moe_ctx_t ctx, int32_t layer,
                                    const void* d_x, int32_t x_dtype,
                                    const int32_t* d_topk_idx,
                                    const float* d_topk_w,
                                    const float* d_residual, float* d_out);

/* T tokens at once (prefill): routing per token as m1moe_router_topk, the
 * (token, slot) pairs grouped by expert, gate/up/down as MFMA f16 grouped
 * GEMMs with the 4-bit dequant fused, and a deterministic weighted combine.
 * Results equal T independent m1moe_moe_decode calls up to bf16 operand
 * rounding.  d_x [T x hidden], d_residual f32 [T x hidden] or NULL,
 * d_out f32 [T x hidden], d_topk_idx/d_topk_w [T x top_k] nullable.
 * T <= the context's prefill capacity (4096 tokens). */
int32_t m1moe_moe_prefill(m1moe_ctx_t ctx, int32_t layer, int32_t T,
                          const void* d_x, int32_t x_dtype,
                          const float* d_residual, float* d_out,
                          int32_t* d_topk_idx, float* d_topk_w);

/* Writes the dequantised f32 weights of one projection of one expert,
 * row-major [rows x cols] (gate/up: intermediate x hidden; down: hidden x
 * intermediate), value f32(n)*f32(s)+f32(b), for the bit-exact weight check
 * (Shaders.metal:66-77). */
int32_t m1moe_dequant_debug(m1moe_ctx_t ctx, int32_t layer, int32_t expert,
                            int32_t proj, float* d_out);

/* ---- seeded synthetic inputs (host-only; bench and test data) ----------
 * Counter-based: value i of tensor `tensor_id` under `seed` is a function of
 * (seed, tensor_id, i) only, so any slice can be generated independently.
 * Normals are Box-Muller in f64, scaled by sigma, rounded to f32, then
 * (bf16 variants) rounded to nearest-even bf16. */
int32_t m1moe_synth_normal_bf16(uint64_t seed, uint64_t tensor_id,
                                uint64_t n, float sigma, int32_t absval,
                                uint16_t* out);
int32_t m1moe_synth_normal_f32(uint64_t seed, uint64_t tensor_id, uint64_t n,
                               float sigma, float* out);
/* One layer_NN.bin image: nibbles uniform in 0..15 (8 per u32), scales
 * bf16 |N(0, scale_sigma)|, biases bf16 N(0, bias_sigma), per expert block.
 * `bytes` must be num_experts * expert_bytes.  Uses up to `threads` host
 * threads (<=0: one). */
int32_t m1moe_synth_layer_image(const m1moe_moe_shape* shape, uint64_t seed,
                                int32_t layer, float scale_sigma,
                                float bias_sigma, void* out, uint64_t bytes,
                                int32_t threads);

#ifdef __cplusplus
}
#endif

#endif /* M1MOE_HIP_H */
