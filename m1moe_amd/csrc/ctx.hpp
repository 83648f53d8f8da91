// ctx.hpp — the context object behind the C ABI and the host helpers shared
// by the translation units that implement the ABI (ctx.cpp, decoder.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <set>
#include <vector>

#include "internal.hpp"
#include "m1moe_hip.h"

namespace m1moe {
int32_t fail(int32_t code, const char* fmt, ...);
}  // namespace m1moe
using m1moe::fail;

struct m1moe_event {
    hipEvent_t ev;
};

struct m1moe_graph {
    hipGraph_t graph;
    hipGraphExec_t exec;
    m1moe_ctx_t owner;       // the context whose stream was captured
    uint64_t scratch_gen;    // owner->scratch_gen when the capture ended
    bool uses_scratch;       // a captured call used the context's growable scratch
};

struct m1moe_ctx {
    int32_t device = 0;
    int32_t cus = 0;                 // compute units of the device
    m1moe_moe_shape shape{};
    m1moe::Geom g{};
    // every context on a device enqueues on the device's one library stream
    // (lib_stream, shared and reference-counted across the process), or on a
    // caller stream set by m1moe_set_stream while it is the device's only
    // context: the per-CU decode kernels need all their workgroups resident
    // at once, so no two launches of the library may overlap on one device
    hipStream_t lib_stream = nullptr;
    hipStream_t stream = nullptr;
    bool registered = false;         // counted in the device's stream share
    // bumped whenever a scratch buffer is reallocated: a graph captured
    // before then holds the freed addresses and is refused at launch
    uint64_t scratch_gen = 0;
    // set by every call that uses the growable scratch (prefill, decoder
    // prefill, attention), cleared when a capture begins
    bool capture_uses_scratch = false;
    uint8_t* arena = nullptr;        // [L][E] expert blocks
    uint16_t* routers = nullptr;     // [L][E][h] bf16
    float* biases = nullptr;         // [L][E]
    std::vector<bool> has_bias;
    std::vector<bool> layer_loaded;
    std::vector<bool> router_loaded;
    // scratch
    float* logits = nullptr;         // [cap][E]
    int32_t* topk_idx = nullptr;     // [cap][K]
    float* topk_w = nullptr;         // [cap][K]
    uint32_t* counters = nullptr;    // [cap]
    float* act = nullptr;            // [K][I]
    uint8_t* sync = nullptr;         // decode hand-off state: slots | gu_cnt | seen |
                                     // cu_seen | cu_cnt | cu_part | xl
    uint64_t sync_bytes = 0, sync_gu_cnt = 0, sync_seen = 0;
    uint64_t sync_cu_seen = 0, sync_cu_cnt = 0, sync_cu_part = 0, sync_xl = 0;
    // decode launches use the one-workgroup-per-CU kernel (decode_cu.hip):
    // the shape fits it and the device has the CUs to hold all its
    // workgroups at once.  That kernel reads a repacked copy of every expert
    // block (dec, [L][E][dec_bytes]), made at upload; a layer whose canonical
    // blocks were handed out for writing (m1moe_expert_block) is repacked
    // again before its next decode (dec_stale).
    bool decode_cu = false;
    uint8_t* dec = nullptr;
    uint64_t dec_bytes = 0;
    std::vector<bool> dec_stale;
    // the prefill GEMMs' copy of every expert block, operand tiles as the
    // GEMM's LDS images with f16 scale/bias pairs and a power of two per row
    // (pft, [L][E][pft_bytes], PfTileLayout), made at upload and, like the
    // decode copy, again after m1moe_expert_block (pft_stale)
    uint8_t* pft = nullptr;
    uint64_t pft_bytes = 0;
    std::vector<bool> pft_stale;
    uint32_t* err = nullptr;         // sticky device error flag
    // prefill scratch, grown on demand to the largest T seen (pf_cap tokens)
    int32_t pf_cap = 0;
    _Float16* pf_xq = nullptr;       // [cap][h]
    float* pf_xinv = nullptr;        // [cap]
    int32_t* pf_pos = nullptr;       // [cap*K]
    m1moe::PfPair* pf_sorted = nullptr;       // [cap*K]
    int32_t* pf_eoff = nullptr;      // [E+1]
    int32_t* pf_toff = nullptr;      // [E+1]
    m1moe::PfTile* pf_tdesc = nullptr;        // [cap*K/kPfTN + E + 1]
    _Float16* pf_act = nullptr;      // [cap*K][I]
    float* pf_y = nullptr;           // [cap*K][h]
    uint8_t* pf_aexp = nullptr;      // [cap*K][I/32]
    uint32_t* pf_aflag = nullptr;    // [1]
    // this device's static scratch (scratch.hip), for m1moe_moe_prefill_noalloc;
    // shared with every other context on the device, never freed
    uint8_t* static_scratch = nullptr;
    // attention scratch of m1moe_attention_decode, grown on demand
    float* attn_part = nullptr;
    uint64_t attn_part_floats = 0;
    uint32_t* attn_cnt = nullptr;    // [kAttnCounters], zero between launches
    std::set<void*> allocs;
};

namespace m1moe {

#define HIP_TRY(expr)                                                                        \
    do {                                                                                     \
        hipError_t e_ = (expr);                                                              \
        if (e_ != hipSuccess)                                                                \
            return fail(M1MOE_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_));      \
    } while (0)

inline int32_t device_alloc(void** p, uint64_t bytes, const char* what) {
    hipError_t e = hipMalloc(p, bytes ? bytes : 1);
    if (e != hipSuccess) {
        *p = nullptr;
        return fail(M1MOE_ERR_OOM, "hipMalloc(%s, %llu bytes) failed: %s", what,
                    (unsigned long long)bytes, hipGetErrorString(e));
    }
    return M1MOE_OK;
}

// Scratch that must grow is reallocated (synchronise, free, allocate): not
// possible while the stream is being captured into a graph, and a graph
// captured earlier would point at the freed buffers.  Growth under capture is
// refused; the caller grows it first with one eager call at the largest size.
inline int32_t refuse_growth_in_capture(hipStream_t stream, const char* what) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return fail(M1MOE_ERR_INVALID, "%s must grow, which cannot happen during stream capture: "
                    "make one eager call at the largest size before capturing", what);
    return M1MOE_OK;
}

inline int32_t check_ctx(m1moe_ctx_t ctx) {
    if (!ctx) return fail(M1MOE_ERR_INVALID, "null context");
    return M1MOE_OK;
}

inline int32_t set_device(m1moe_ctx_t ctx) {
    HIP_TRY(hipSetDevice(ctx->device));
    return M1MOE_OK;
}

inline int32_t check_layer(m1moe_ctx_t ctx, int32_t layer) {
    if (layer < 0 || layer >= ctx->shape.num_layers)
        return fail(M1MOE_ERR_INVALID, "layer %d out of range [0, %d)", layer,
                    ctx->shape.num_layers);
    return M1MOE_OK;
}

inline int32_t check_dev_ptr(const void* p, const char* what, bool nullable) {
    if (!p) {
        if (nullable) return M1MOE_OK;
        return fail(M1MOE_ERR_INVALID, "%s is null", what);
    }
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
        return fail(M1MOE_ERR_INVALID, "%s must be 16-byte aligned", what);
    return M1MOE_OK;
}

inline int32_t check_dtype(int32_t dt) {
    if (dt != M1MOE_F32 && dt != M1MOE_BF16)
        return fail(M1MOE_ERR_INVALID, "x_dtype %d is not M1MOE_F32 or M1MOE_BF16", dt);
    return M1MOE_OK;
}

// The decode entry with the post-attention RMSNorm applied to the f32 input
// in the kernel (sum of squares given as n_ssq partials); for the decoder.
int32_t moe_decode_normed(m1moe_ctx_t ctx, int32_t layer, const float* d_x, const float* d_ssq,
                          int32_t n_ssq, const uint16_t* d_norm_w, float eps,
                          const float* d_residual, float* d_out);

// A decoder's vocabulary and attention dimensions (for the loader).
int32_t dec_dims(m1moe_dec_t dec, int32_t* vocab, int32_t* num_heads, int32_t* num_kv_heads,
                 int32_t* head_dim, int32_t* qk_norm);

inline int32_t launched(int rc, const char* what) {
    if (rc != (int)hipSuccess)
        return fail(M1MOE_ERR_HIP, "launch of %s failed: %s", what,
                    hipGetErrorString((hipError_t)rc));
    return M1MOE_OK;
}

}  // namespace m1moe
