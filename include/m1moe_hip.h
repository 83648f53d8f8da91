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
 *    scratch, m1moe_alloc buffers).  Every compute call is enqueued
 *    asynchronously on the context's stream; m1moe_sync() waits for it.  A
 *    context is single-threaded (the reference engine is driven from one
 *    serial queue, Sources/bench/main.swift:58).
 *  - All contexts on one device share one library stream, so the library's
 *    launches on a device never overlap: on a device with at least 256 CUs
 *    the per-CU decode kernels (hidden 2048 and 4096 shapes, see
 *    m1moe_decode_kernel_for) run one workgroup on every CU and each
 *    workgroup waits for every other one, so they need the whole device.
 *    Work of another stream or process on the same GPU can keep some of
 *    their workgroups from starting; the waiting ones then give up after
 *    about a second, and the next m1moe_sync() reports M1MOE_ERR_DEVICE.
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

/* The decode kernel a shape runs on a device with `cus` compute units, each
 * holding `blocks_per_cu` workgroups of the per-CU kernels (1 on an
 * MI355X): *kernel = 1 (moe_decode_cu_kernel: hidden 2048, K * I 8192 or
 * 16384) or 2 (moe_decode_cuw_kernel: hidden 4096, K <= 2) when all 256 of
 * the per-CU kernel's workgroups fit on the device at once — these need the
 * whole device (conventions above) — else 0 (moe_decode_kernel, which only
 * waits for lower workgroup ids and shares the device safely).  m1moe_create
 * makes the same choice from the device's CU count and occupancy.  No
 * counterpart in the reference (one Metal path); host only. */
int32_t m1moe_decode_kernel_for(const m1moe_moe_shape* shape, int32_t cus,
                                int32_t blocks_per_cu, int32_t* kernel);

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
 * (InferenceEngine.swift:274-279); here a wrong size is an error, and so is
 * a non-finite group scale or bias (the layer then stays unloaded). */
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
 * that fill the arena on the device.  The decode and prefill kernels also
 * read repacked copies of each layer's blocks; this call marks the layer's
 * copies stale and the next decode or prefill of the layer rebuilds them
 * from the arena (refused during graph capture).  So every write through
 * the pointer must be complete, in order on the context stream (or
 * synchronised), before the next decode or prefill of the layer, and a
 * later write needs this call again first: a write after the rebuild is
 * seen by the arena's gate/up rows but not by the copies. */
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
 * void*); NULL restores the library stream of the device.  Refused
 * (M1MOE_ERR_INVALID) while another context is live on the same device, and
 * m1moe_create on a device refuses a second context while the first runs on
 * a caller stream: launches on one device stay on one stream. */
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
 * into a HIP graph (no device work runs during capture).  A graph is
 * launched on the context it was captured on; its launch is refused
 * (M1MOE_ERR_INVALID) once a call has reallocated a scratch buffer of the
 * context since the capture (a prefill, decoder prefill or attention call
 * larger than any before), since the graph holds the freed addresses:
 * capture it again. */
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
 * Results equal T independent m1moe_moe_decode calls up to f16 operand
 * rounding (the SwiGLU products in blocks of 32 with a power of two each
 * where they pass the f16 range; a non-finite one is clamped and reported
 * by the next m1moe_sync).  d_x [T x hidden], d_residual f32 [T x hidden]
 * or NULL, d_out f32 [T x hidden], d_topk_idx/d_topk_w [T x top_k]
 * nullable.  T <= the context's prefill capacity (4096 tokens). */
int32_t m1moe_moe_prefill(m1moe_ctx_t ctx, int32_t layer, int32_t T,
                          const void* d_x, int32_t x_dtype,
                          const float* d_residual, float* d_out,
                          int32_t* d_topk_idx, float* d_topk_w);

/* m1moe_moe_prefill with the same arguments, kernels and results, that
 * allocates nothing: no counterpart in the reference.  It is for callers that
 * cannot allocate device memory (code under HIP graph capture without a
 * warm-up call, tight serving loops, harnesses that forbid hipMalloc).  Its
 * scratch is a fixed 64 MiB static device array per GPU (looked up by
 * m1moe_create, held until the process ends) instead of the context's
 * buffers that m1moe_moe_prefill grows; a T whose scratch would not fit is
 * rejected with M1MOE_ERR_INVALID naming the largest T that fits (776
 * tokens at hidden 2048, 8 x 1024 experts; 676 at hidden 4096,
 * 2 x 14336).  Every call on one GPU shares that array, so calls that overlap
 * on one GPU (two streams, or two contexts on one device) race. */
int32_t m1moe_moe_prefill_noalloc(m1moe_ctx_t ctx, int32_t layer, int32_t T,
                                  const void* d_x, int32_t x_dtype,
                                  const float* d_residual, float* d_out,
                                  int32_t* d_topk_idx, float* d_topk_w);

/* Writes the dequantised f32 weights of one projection of one expert,
 * row-major [rows x cols] (gate/up: intermediate x hidden; down: hidden x
 * intermediate), value f32(n)*f32(s)+f32(b), for the bit-exact weight check
 * (Shaders.metal:66-77). */
int32_t m1moe_dequant_debug(m1moe_ctx_t ctx, int32_t layer, int32_t expert,
                            int32_t proj, float* d_out);

/* ---- dense decoder step around the MoE block ---------------------------- */

/* Building blocks (each asynchronous on the context stream; all vectors f32
 * unless stated, weights bf16 row-major). */

/* out[i] = x[i] * rsqrt(sum(x^2)/n + eps) * w[i]   (rmsNormSum + rmsNormApply,
 * Shaders.metal:96-134; InferenceEngine.swift:298-320).  n <= 65536. */
int32_t m1moe_rmsnorm(m1moe_ctx_t ctx, const float* d_x, const uint16_t* d_w,
                      float* d_out, int32_t n, float eps);

/* y[r] = sum_c W[r][c] * x[c] (+ residual[r] when d_residual is non-null)
 * (matvecBF16, Shaders.metal:328-358; residualAdd :152-162).
 * cols % 8 == 0, cols <= 65536. */
int32_t m1moe_matvec_bf16(m1moe_ctx_t ctx, const uint16_t* d_w,
                          const float* d_x, const float* d_residual,
                          float* d_y, int32_t rows, int32_t cols);

/* Decode attention of one query position over seq_len cached positions
 * (attnScores + attnSoftmax + attnValues, Shaders.metal:209-326, dispatched as
 * InferenceEngine.swift:349-399): per head h,
 * s_p = (q_h . k_p[h / hpkv]) / sqrt(head_dim), p_s = softmax(s), out_h =
 * sum_p p_p v_p[h / hpkv].  q f32 [num_heads x head_dim]; caches f32
 * [>= seq_len x num_kv_heads*head_dim]; out f32 [num_heads x head_dim].
 * head_dim is 64, 128 or 256; num_heads % num_kv_heads == 0;
 * 1 <= seq_len <= 65536. */
int32_t m1moe_attention_decode(m1moe_ctx_t ctx, const float* d_q,
                               const float* d_kcache, const float* d_vcache,
                               float* d_out, int32_t num_heads,
                               int32_t num_kv_heads, int32_t head_dim,
                               int32_t seq_len);

/* Index of the largest of n values, ties to the lower index, written to
 * d_idx (greedy sampling, InferenceEngine.swift:550-555: a scan from x[0]
 * with a strict >, so NaN never wins except at index 0). */
int32_t m1moe_argmax(m1moe_ctx_t ctx, const float* d_x, int32_t n,
                     int32_t* d_idx);

/* The whole decode step (InferenceEngine.forward and runLayer,
 * InferenceEngine.swift:125-266, which ran norms/projections/attention on
 * Metal and q/k norms, RoPE, the KV store, router and top-K on the CPU with
 * three syncs per layer): token embedding; per layer input RMSNorm, q/k/v
 * matvecs, per-head q/k RMSNorm (when the model has it), RoPE, f32 KV cache
 * store, attention, o_proj + residual, post-attention RMSNorm, the MoE block
 * of the context; final RMSNorm, lm_head, greedy argmax — all on the GPU with
 * no host sync.  The token and the position live in device memory, so each
 * step reads the previous step's argmax and a greedy loop can be captured in
 * a graph and replayed. */
typedef struct m1moe_dec* m1moe_dec_t;

/* Attention and vocabulary of a model (ModelSpec.swift AttentionSpec and
 * vocabSize).  hidden and num_layers come from the MoE context.
 * head_dim is 64, 128 or 256 (even); num_heads % num_kv_heads == 0;
 * 1 <= max_seq <= 65536; vocab >= 1. */
typedef struct {
    int32_t vocab;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t max_seq;   /* KV cache positions */
    int32_t qk_norm;   /* per-head q/k RMSNorm before RoPE (OLMoE) */
    float rope_theta;
    float rms_eps;
} m1moe_dec_shape;

/* dense tensors of a model (bf16, row-major) */
enum {
    M1MOE_W_EMBED = 0,      /* [vocab x hidden]                 model.embed_tokens */
    M1MOE_W_LM_HEAD = 1,    /* [vocab x hidden]                 lm_head */
    M1MOE_W_FINAL_NORM = 2, /* [hidden]                         model.norm */
    M1MOE_W_IN_NORM = 3,    /* [hidden]       per layer         input_layernorm */
    M1MOE_W_POST_NORM = 4,  /* [hidden]       per layer         post_attention_layernorm */
    M1MOE_W_Q = 5,          /* [heads*hd x hidden]   per layer  self_attn.q_proj */
    M1MOE_W_K = 6,          /* [kv_heads*hd x hidden]           self_attn.k_proj */
    M1MOE_W_V = 7,          /* [kv_heads*hd x hidden]           self_attn.v_proj */
    M1MOE_W_O = 8,          /* [hidden x heads*hd]              self_attn.o_proj */
    M1MOE_W_Q_NORM = 9,     /* [head_dim]     per layer         self_attn.q_norm (first head_dim
                               values, applied to every head: applyHeadRMSNorm, InferenceEngine.swift:538-548) */
    M1MOE_W_K_NORM = 10     /* [head_dim]     per layer         self_attn.k_norm */
};

/* The decoder uses the MoE context's layers, stream and error flag; destroy
 * it before the context. */
int32_t m1moe_dec_create(m1moe_ctx_t moe, const m1moe_dec_shape* shape,
                         m1moe_dec_t* out);
void m1moe_dec_destroy(m1moe_dec_t dec);
/* count must be the tensor's element count (above); layer is ignored for
 * the model-level tensors. */
int32_t m1moe_dec_upload(m1moe_dec_t dec, int32_t which, int32_t layer,
                         const uint16_t* host_bf16, uint64_t count);
/* Position 0 and an empty KV cache (InferenceEngine.reset, :159-163; the
 * positions past the new one are never read, so only the position is
 * rewritten).  Enqueued on the context stream. */
int32_t m1moe_dec_reset(m1moe_dec_t dec);
/* One step at the current device-side position: reads the token from
 * d_token_in (int32 device), writes the greedy next token to d_token_out
 * (may be the same address) and advances the position.  d_logits (nullable)
 * receives f32 [vocab].  A prompt is fed as steps with d_token_in =
 * &prompt[i]; a greedy loop passes out = in, or &toks[i+1] to keep them.  A token outside
 * [0, vocab) is embedded as token 0, and with the cache full (position ==
 * max_seq) nothing is stored and the position stays; either sets the device
 * error flag, reported by the next m1moe_sync. */
int32_t m1moe_dec_step(m1moe_dec_t dec, const int32_t* d_token_in,
                       int32_t* d_token_out, float* d_logits);
/* Sequence mode: d_seq int32 [seq_cap] holds the prompt in [0, n_prompt).
 * The step at device-side position p embeds d_seq[p] and, when p + 1 >=
 * n_prompt, stores its greedy token at d_seq[p + 1] (if p + 1 < seq_cap).
 * After m1moe_dec_reset, n_prompt + n_gen calls (or replays of one graph
 * captured around one call) run the reference's prefill-then-generate loop
 * (Sources/bench/main.swift:136-163): the prompt forwarded token by token,
 * then each generated token fed back, d_seq[n_prompt .. n_prompt + n_gen]
 * receiving the n_gen + 1 greedy tokens.  p >= seq_cap sets the device error
 * flag (as a token outside the vocabulary). */
int32_t m1moe_dec_step_seq(m1moe_dec_t dec, int32_t* d_seq, int32_t n_prompt,
                           int32_t seq_cap, float* d_logits);
/* The prompt at once: the T tokens d_tokens (int32 device) at positions
 * pos .. pos + T - 1 through every layer in one batch per layer (the
 * reference forwards a prompt token by token, Sources/bench/main.swift:
 * 139-141): q/k/v and o_proj as f32 GEMMs over the T rows, causal attention,
 * the MoE block through the grouped prefill (m1moe_moe_prefill; its f16
 * activations make this path agree with T m1moe_dec_step calls to ~1e-3).
 * Their K/V rows enter the cache, the position advances by T, d_token_out
 * receives the greedy token after the last one and d_logits (nullable) its
 * logits.  1 <= T <= max_seq (prompts longer than 4096 tokens go through in
 * pieces of 4096, each from the position the previous one reached);
 * positions past max_seq set the device error flag.  The first call with a
 * larger piece than any before grows the scratch (make it before capturing a
 * graph). */
int32_t m1moe_dec_prefill(m1moe_dec_t dec, const int32_t* d_tokens, int32_t T,
                          int32_t* d_token_out, float* d_logits);
/* The current position (waits for the context stream). */
int32_t m1moe_dec_position(m1moe_dec_t dec, int32_t* pos);

/* ---- the converted model directory on disk (host-side) -----------------
 * scripts/extract_olmoe.py writes model_weights.bin (non-expert tensors,
 * 4-byte aligned) + model_weights.json ({name: {offset, shape, dtype}}) and
 * packed_experts/layer_NN.bin (E expert blocks per layer). */
typedef struct m1moe_store* m1moe_store_t;
enum { M1MOE_DT_BF16 = 0, M1MOE_DT_F32 = 1, M1MOE_DT_U32 = 2 };

/* WeightStore.init (WeightStore.swift:47-76): maps the .bin read-only and
 * reads the manifest; every tensor must lie inside the file.  Host only. */
int32_t m1moe_store_open(const char* bin_path, const char* json_path,
                         m1moe_store_t* out);
void m1moe_store_close(m1moe_store_t store);
int32_t m1moe_store_count(m1moe_store_t store, int32_t* n);
/* WeightStore.info / pointer (:86-100): the tensor's bytes inside the
 * mapping, dtype (M1MOE_DT_*), shape (4 entries, unused ones 0) and rank.
 * Each output is nullable. */
int32_t m1moe_store_tensor(m1moe_store_t store, const char* name,
                           const void** data, int32_t* dtype, int64_t* shape,
                           int32_t* ndim);

/* Uploads a converted model directory: every layer_NN.bin of the context's
 * layers (m1moe_upload_layer_experts; the size must be E x expert_bytes),
 * each layer's router (mlp.gate.weight, or block_sparse_moe.gate.weight,
 * InferenceEngine.swift:593-598) and, when dec is non-null, the dense
 * tensors under the reference's weight keys (:580-599; f32 tensors are
 * rounded to bf16; q/k norms: the first head_dim values).  Shapes are
 * checked against the context and decoder.  threads: parallel reads per
 * layer file. */
int32_t m1moe_load_model(m1moe_ctx_t ctx, m1moe_dec_t dec, const char* model_dir,
                         int32_t threads);

/* ---- the converters' 4-bit quantizer (host-only; offline) ---------------
 * quantize_4bit of scripts/extract_olmoe.py:116-159 (extract_mixtral.py
 * :93-116 is the same): per row and group of group_size columns, in f32,
 * lo = min, s = (max - lo) / 15 (1 where that is 0), nibble =
 * clamp(round-half-even((w - lo) / s), 0, 15); scales = bf16(s), biases =
 * bf16(lo), nibbles 8 per u32 (column 8w+j in bits 4j..4j+3).  cols must be
 * a multiple of group_size and of 8 (:130-131); a non-finite weight is
 * refused (M1MOE_ERR_INVALID).  threads: host threads over rows (<= 0: 1). */
int32_t m1moe_quantize_4bit(const float* w, int64_t rows, int64_t cols,
                            int32_t group_size, uint32_t* packed,
                            uint16_t* scales, uint16_t* biases,
                            int32_t threads);
/* One expert block of layer_NN.bin from f32 gate [I, h], up [I, h] and
 * down [h, I] (the per-expert loop of extract_olmoe.py:322-338):
 * [gate W|S|B][up W|S|B][down W|S|B].  block_bytes must be expert_bytes. */
int32_t m1moe_quantize_expert(const m1moe_moe_shape* shape, const float* gate,
                              const float* up, const float* down, void* block,
                              uint64_t block_bytes, int32_t threads);
/* f32_to_bf16 of extract_olmoe.py:104-111: (bits + 0x7FFF + lsb) >> 16. */
int32_t m1moe_f32_to_bf16(const float* x, uint64_t n, uint16_t* out);

/* ---- BPE tokenizer (host-only) -------------------------------------------
 * Tokenizer (Sources/M1MoE/Tokenizer.swift) over a HuggingFace
 * tokenizer.json: byte-level BPE (GPT-2 / OLMoE) or, when
 * model.byte_fallback is true, SentencePiece BPE (Mistral / Mixtral).
 * Text crosses the boundary as UTF-8 bytes (not NUL-terminated). */
typedef struct m1moe_tokenizer* m1moe_tokenizer_t;

/* Tokenizer.init(url:) (:35-62).  M1MOE_ERR_INVALID when the file cannot be
 * read or lacks model.vocab / model.merges (TokenizerError.invalidFormat). */
int32_t m1moe_tokenizer_load(const char* path, m1moe_tokenizer_t* out);
void m1moe_tokenizer_free(m1moe_tokenizer_t tok);
/* Mode (1 = SentencePiece BPE, 0 = byte-level), vocabulary entries and merge
 * pairs.  Each output is nullable. */
int32_t m1moe_tokenizer_info(m1moe_tokenizer_t tok, int32_t* sentencepiece,
                             uint64_t* vocab_size, uint64_t* merges);
/* encode(_:addBOS:bos:) (:66-72): bos first when add_bos.  *n_ids gets the
 * count; ids == NULL only asks for it; a count above cap is an error. */
int32_t m1moe_tokenizer_encode(m1moe_tokenizer_t tok, const char* text,
                               uint64_t text_len, int32_t add_bos,
                               uint32_t bos, uint32_t* ids, uint64_t cap,
                               uint64_t* n_ids);
/* decode(_:skipSpecial:) (:76-81): UTF-8 bytes into out (NUL added when
 * there is room); *out_len gets the length; out == NULL only asks for it. */
int32_t m1moe_tokenizer_decode(m1moe_tokenizer_t tok, const uint32_t* ids,
                               uint64_t n, int32_t skip_special, char* out,
                               uint64_t cap, uint64_t* out_len);

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
