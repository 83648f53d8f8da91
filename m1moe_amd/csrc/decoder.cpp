// decoder.cpp — C ABI of the dense decoder step around the MoE block.
//
// Replaces InferenceEngine.forward / runLayer (InferenceEngine.swift:125-266)
// on the GPU: the reference encodes norms, projections and attention on Metal
// and does the q/k norms, RoPE, the KV store, the router and top-K on the CPU
// with three command-buffer syncs per layer; here a step is a fixed sequence
// of kernels on the context stream with no host sync, the token and the
// position in device memory (so a greedy loop can be graph-captured).
#include <hip/hip_runtime.h>

#include <cmath>
#include <vector>

#include "ctx.hpp"
#include "internal.hpp"
#include "m1moe_hip.h"

using namespace m1moe;

namespace {

int32_t check_f32_vec(const void* p, const char* what) { return check_dev_ptr(p, what, false); }

int32_t ensure_attn_scratch(m1moe_ctx_t ctx, uint64_t floats) {
    if (floats <= ctx->attn_part_floats) return M1MOE_OK;
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    if (ctx->attn_part) HIP_TRY(hipFree(ctx->attn_part));
    ctx->attn_part = nullptr;
    ctx->attn_part_floats = 0;
    int32_t rc = device_alloc((void**)&ctx->attn_part, floats * 4, "attention scratch");
    if (rc) return rc;
    ctx->attn_part_floats = floats;
    return M1MOE_OK;
}

int32_t check_attn_dims(int32_t nh, int32_t nkv, int32_t hd) {
    if (hd != 64 && hd != 128 && hd != 256)
        return fail(M1MOE_ERR_INVALID, "head_dim %d is not 64, 128 or 256", hd);
    if (nh <= 0 || nkv <= 0 || nh % nkv)
        return fail(M1MOE_ERR_INVALID, "num_heads %d must be a positive multiple of num_kv_heads %d",
                    nh, nkv);
    return M1MOE_OK;
}

}  // namespace

struct m1moe_dec {
    m1moe_ctx_t moe = nullptr;
    int32_t device = 0;  // the context's, kept so destroy never reads the context
    m1moe_dec_shape sh{};
    int32_t h = 0, L = 0, qd = 0, kvd = 0;
    // weights (bf16)
    uint16_t *embed = nullptr, *lm_head = nullptr, *final_norm = nullptr;
    uint16_t *in_norm = nullptr, *post_norm = nullptr;  // [L][h]
    uint16_t *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr;  // [L][rows][cols]
    uint16_t *q_norm = nullptr, *k_norm = nullptr;  // [L][head_dim]
    std::vector<bool> loaded;                        // [which][layer]
    // state
    float *kcache = nullptr, *vcache = nullptr;  // [L][max_seq][kvd]
    int32_t* pos = nullptr;
    // step scratch
    float *res = nullptr, *res2 = nullptr, *xn = nullptr, *hmid = nullptr;
    float *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr;
    float *logits = nullptr, *part = nullptr;
    std::vector<void*> allocs;
};

namespace {

constexpr int kNumW = 11;

bool per_layer(int32_t which) { return which >= M1MOE_W_IN_NORM; }

uint64_t w_count(const m1moe_dec* d, int32_t which) {
    const uint64_t h = d->h, V = d->sh.vocab, qd = d->qd, kvd = d->kvd, hd = d->sh.head_dim;
    switch (which) {
        case M1MOE_W_EMBED:
        case M1MOE_W_LM_HEAD: return V * h;
        case M1MOE_W_FINAL_NORM:
        case M1MOE_W_IN_NORM:
        case M1MOE_W_POST_NORM: return h;
        case M1MOE_W_Q: return qd * h;
        case M1MOE_W_K:
        case M1MOE_W_V: return kvd * h;
        case M1MOE_W_O: return h * qd;
        case M1MOE_W_Q_NORM:
        case M1MOE_W_K_NORM: return hd;
        default: return 0;
    }
}

uint16_t* w_base(const m1moe_dec* d, int32_t which) {
    switch (which) {
        case M1MOE_W_EMBED: return d->embed;
        case M1MOE_W_LM_HEAD: return d->lm_head;
        case M1MOE_W_FINAL_NORM: return d->final_norm;
        case M1MOE_W_IN_NORM: return d->in_norm;
        case M1MOE_W_POST_NORM: return d->post_norm;
        case M1MOE_W_Q: return d->wq;
        case M1MOE_W_K: return d->wk;
        case M1MOE_W_V: return d->wv;
        case M1MOE_W_O: return d->wo;
        case M1MOE_W_Q_NORM: return d->q_norm;
        case M1MOE_W_K_NORM: return d->k_norm;
        default: return nullptr;
    }
}

int32_t dec_alloc(m1moe_dec* d, void** p, uint64_t bytes, const char* what) {
    int32_t rc = device_alloc(p, bytes, what);
    if (rc == M1MOE_OK) d->allocs.push_back(*p);
    return rc;
}

DenseStepArgs step_args(const m1moe_dec* d, const int32_t* token) {
    DenseStepArgs a{};
    a.token = token;
    a.pos = d->pos;
    a.embed = d->embed;
    a.x_out = d->res;
    a.q = d->q;
    a.k = d->k;
    a.v = d->v;
    a.q_norm = d->q_norm;
    a.k_norm = d->k_norm;
    a.kcache = d->kcache;
    a.vcache = d->vcache;
    a.err = d->moe->err;
    a.vocab = d->sh.vocab;
    a.h = d->h;
    a.num_heads = d->sh.num_heads;
    a.num_kv_heads = d->sh.num_kv_heads;
    a.head_dim = d->sh.head_dim;
    a.max_seq = d->sh.max_seq;
    a.qk_norm = d->sh.qk_norm;
    a.rope_theta = d->sh.rope_theta;
    a.eps = d->sh.rms_eps;
    return a;
}

MvArgs mv_one(const uint16_t* w, const float* x, const float* res, float* y, int32_t rows, int32_t cols) {
    MvArgs m{};
    m.seg[0] = MvSeg{w, y, res, rows};
    m.x = x;
    m.rows = rows;
    m.cols = cols;
    return m;
}

}  // namespace

extern "C" {

// ---- building blocks -----------------------------------------------------------------

int32_t m1moe_rmsnorm(m1moe_ctx_t ctx, const float* d_x, const uint16_t* d_w, float* d_out,
                      int32_t n, float eps) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = check_f32_vec(d_x, "d_x")) || (rc = check_f32_vec(d_w, "d_w")) ||
        (rc = check_f32_vec(d_out, "d_out")))
        return rc;
    if (n <= 0 || n > 65536) return fail(M1MOE_ERR_INVALID, "n %d out of range [1, 65536]", n);
    if (!(eps >= 0.f)) return fail(M1MOE_ERR_INVALID, "eps must be >= 0");
    if ((rc = set_device(ctx))) return rc;
    return launched(launch_rmsnorm(d_x, d_w, d_out, n, eps, ctx->stream), "rmsnorm");
}

int32_t m1moe_matvec_bf16(m1moe_ctx_t ctx, const uint16_t* d_w, const float* d_x,
                          const float* d_residual, float* d_y, int32_t rows, int32_t cols) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = check_f32_vec(d_w, "d_w")) || (rc = check_f32_vec(d_x, "d_x")) ||
        (rc = check_dev_ptr(d_residual, "d_residual", true)) || (rc = check_f32_vec(d_y, "d_y")))
        return rc;
    if (rows <= 0 || cols <= 0 || cols % 8 || cols > 65536)
        return fail(M1MOE_ERR_INVALID, "rows %d / cols %d: need rows > 0, cols a positive multiple of 8 <= 65536",
                    rows, cols);
    if ((rc = set_device(ctx))) return rc;
    return launched(launch_matvec_bf16(mv_one(d_w, d_x, d_residual, d_y, rows, cols), ctx->stream),
                    "matvec_bf16");
}

int32_t m1moe_attention_decode(m1moe_ctx_t ctx, const float* d_q, const float* d_kcache,
                               const float* d_vcache, float* d_out, int32_t num_heads,
                               int32_t num_kv_heads, int32_t head_dim, int32_t seq_len) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = check_f32_vec(d_q, "d_q")) ||
        (rc = check_f32_vec(d_kcache, "d_kcache")) || (rc = check_f32_vec(d_vcache, "d_vcache")) ||
        (rc = check_f32_vec(d_out, "d_out")) || (rc = check_attn_dims(num_heads, num_kv_heads, head_dim)))
        return rc;
    if (seq_len <= 0 || seq_len > 65536)
        return fail(M1MOE_ERR_INVALID, "seq_len %d out of range [1, 65536]", seq_len);
    if ((rc = set_device(ctx))) return rc;
    if ((rc = ensure_attn_scratch(ctx, attention_partial_floats(num_heads, head_dim, seq_len)))) return rc;
    AttnArgs a{};
    a.q = d_q;
    a.kcache = d_kcache;
    a.vcache = d_vcache;
    a.out = d_out;
    a.partial = ctx->attn_part;
    a.seq_ptr = nullptr;
    a.seq_len = seq_len;
    a.max_seq = seq_len;
    a.num_heads = num_heads;
    a.num_kv_heads = num_kv_heads;
    a.hpkv = num_heads / num_kv_heads;
    a.head_dim = head_dim;
    a.scale = 1.0f / sqrtf((float)head_dim);
    return launched(launch_attention(a, seq_len, ctx->stream), "attention");
}

int32_t m1moe_argmax(m1moe_ctx_t ctx, const float* d_x, int32_t n, int32_t* d_idx) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = check_f32_vec(d_x, "d_x"))) return rc;
    if (!d_idx) return fail(M1MOE_ERR_INVALID, "d_idx is null");
    if (n <= 0) return fail(M1MOE_ERR_INVALID, "n %d must be positive", n);
    if ((rc = set_device(ctx))) return rc;
    return launched(launch_argmax(d_x, n, d_idx, nullptr, 0, ctx->stream), "argmax");
}

// ---- the decoder ---------------------------------------------------------------------

void m1moe_dec_destroy(m1moe_dec_t dec) {
    if (!dec) return;
    (void)hipSetDevice(dec->device);
    for (void* p : dec->allocs) (void)hipFree(p);
    delete dec;
}

int32_t m1moe_dec_create(m1moe_ctx_t moe, const m1moe_dec_shape* s, m1moe_dec_t* out) {
    int32_t rc;
    if (!out) return fail(M1MOE_ERR_INVALID, "out is null");
    *out = nullptr;
    if ((rc = check_ctx(moe))) return rc;
    if (!s) return fail(M1MOE_ERR_INVALID, "shape is null");
    if ((rc = check_attn_dims(s->num_heads, s->num_kv_heads, s->head_dim))) return rc;
    if (s->vocab <= 0) return fail(M1MOE_ERR_INVALID, "vocab %d must be positive", s->vocab);
    if (s->max_seq <= 0 || s->max_seq > 65536)
        return fail(M1MOE_ERR_INVALID, "max_seq %d out of range [1, 65536]", s->max_seq);
    if (!(s->rope_theta > 0.f) || !(s->rms_eps >= 0.f))
        return fail(M1MOE_ERR_INVALID, "rope_theta must be > 0 and rms_eps >= 0");
    if (s->num_heads * s->head_dim > 65536)
        return fail(M1MOE_ERR_INVALID, "num_heads * head_dim exceeds 65536");
    if ((rc = set_device(moe))) return rc;
    m1moe_dec* d = new (std::nothrow) m1moe_dec;
    if (!d) return fail(M1MOE_ERR_OOM, "out of host memory");
    d->moe = moe;
    d->device = moe->device;
    d->sh = *s;
    d->h = moe->g.h;
    d->L = moe->g.L;
    d->qd = s->num_heads * s->head_dim;
    d->kvd = s->num_kv_heads * s->head_dim;
    d->loaded.assign((size_t)kNumW * d->L, false);
    const uint64_t h = d->h, L = d->L, V = s->vocab, qd = d->qd, kvd = d->kvd, hd = s->head_dim;
    const uint64_t ms = s->max_seq;
    const uint64_t part = (uint64_t)attention_partial_floats(s->num_heads, s->head_dim, s->max_seq);
    if ((rc = dec_alloc(d, (void**)&d->embed, V * h * 2, "embedding")) ||
        (rc = dec_alloc(d, (void**)&d->lm_head, V * h * 2, "lm_head")) ||
        (rc = dec_alloc(d, (void**)&d->final_norm, h * 2, "final norm")) ||
        (rc = dec_alloc(d, (void**)&d->in_norm, L * h * 2, "input norms")) ||
        (rc = dec_alloc(d, (void**)&d->post_norm, L * h * 2, "post-attention norms")) ||
        (rc = dec_alloc(d, (void**)&d->wq, L * qd * h * 2, "q_proj")) ||
        (rc = dec_alloc(d, (void**)&d->wk, L * kvd * h * 2, "k_proj")) ||
        (rc = dec_alloc(d, (void**)&d->wv, L * kvd * h * 2, "v_proj")) ||
        (rc = dec_alloc(d, (void**)&d->wo, L * h * qd * 2, "o_proj")) ||
        (rc = dec_alloc(d, (void**)&d->q_norm, L * hd * 2, "q norms")) ||
        (rc = dec_alloc(d, (void**)&d->k_norm, L * hd * 2, "k norms")) ||
        (rc = dec_alloc(d, (void**)&d->kcache, L * ms * kvd * 4, "K cache")) ||
        (rc = dec_alloc(d, (void**)&d->vcache, L * ms * kvd * 4, "V cache")) ||
        (rc = dec_alloc(d, (void**)&d->pos, 16, "position")) ||
        (rc = dec_alloc(d, (void**)&d->res, h * 4, "residual")) ||
        (rc = dec_alloc(d, (void**)&d->res2, h * 4, "residual 2")) ||
        (rc = dec_alloc(d, (void**)&d->xn, h * 4, "normed input")) ||
        (rc = dec_alloc(d, (void**)&d->hmid, h * 4, "MoE input")) ||
        (rc = dec_alloc(d, (void**)&d->q, qd * 4, "q")) ||
        (rc = dec_alloc(d, (void**)&d->k, kvd * 4, "k")) ||
        (rc = dec_alloc(d, (void**)&d->v, kvd * 4, "v")) ||
        (rc = dec_alloc(d, (void**)&d->attn, qd * 4, "attention output")) ||
        (rc = dec_alloc(d, (void**)&d->logits, V * 4, "logits")) ||
        (rc = dec_alloc(d, (void**)&d->part, part * 4, "attention scratch"))) {
        m1moe_dec_destroy(d);
        return rc;
    }
    if (hipMemset(d->pos, 0, 16) != hipSuccess) {
        m1moe_dec_destroy(d);
        return fail(M1MOE_ERR_HIP, "hipMemset(position) failed");
    }
    *out = d;
    return M1MOE_OK;
}

int32_t m1moe_dec_upload(m1moe_dec_t dec, int32_t which, int32_t layer, const uint16_t* host_bf16,
                         uint64_t count) {
    int32_t rc;
    if (!dec) return fail(M1MOE_ERR_INVALID, "null decoder");
    if (which < 0 || which >= kNumW) return fail(M1MOE_ERR_INVALID, "tensor id %d out of range", which);
    if (!host_bf16) return fail(M1MOE_ERR_INVALID, "host_bf16 is null");
    if (per_layer(which) && (layer < 0 || layer >= dec->L))
        return fail(M1MOE_ERR_INVALID, "layer %d out of range [0, %d)", layer, dec->L);
    const uint64_t n = w_count(dec, which);
    if (count != n)
        return fail(M1MOE_ERR_INVALID, "tensor %d: count %llu != expected %llu", which,
                    (unsigned long long)count, (unsigned long long)n);
    if ((rc = set_device(dec->moe))) return rc;
    uint16_t* dst = w_base(dec, which) + (per_layer(which) ? (uint64_t)layer * n : 0);
    HIP_TRY(hipMemcpyAsync(dst, host_bf16, n * 2, hipMemcpyHostToDevice, dec->moe->stream));
    HIP_TRY(hipStreamSynchronize(dec->moe->stream));
    dec->loaded[(size_t)which * dec->L + (per_layer(which) ? layer : 0)] = true;
    return M1MOE_OK;
}

int32_t m1moe_dec_reset(m1moe_dec_t dec) {
    int32_t rc;
    if (!dec) return fail(M1MOE_ERR_INVALID, "null decoder");
    if ((rc = set_device(dec->moe))) return rc;
    return launched(launch_set_i32(dec->pos, 0, dec->moe->stream), "reset");
}

int32_t m1moe_dec_position(m1moe_dec_t dec, int32_t* pos) {
    int32_t rc;
    if (!dec || !pos) return fail(M1MOE_ERR_INVALID, "null decoder or pos");
    if ((rc = set_device(dec->moe))) return rc;
    HIP_TRY(hipStreamSynchronize(dec->moe->stream));
    HIP_TRY(hipMemcpy(pos, dec->pos, 4, hipMemcpyDeviceToHost));
    return M1MOE_OK;
}

int32_t m1moe_dec_step(m1moe_dec_t dec, const int32_t* d_token_in, int32_t* d_token_out,
                       float* d_logits) {
    int32_t rc;
    if (!dec) return fail(M1MOE_ERR_INVALID, "null decoder");
    if (!d_token_in || reinterpret_cast<uintptr_t>(d_token_in) % 4 || !d_token_out ||
        reinterpret_cast<uintptr_t>(d_token_out) % 4)
        return fail(M1MOE_ERR_INVALID, "d_token_in / d_token_out must be 4-byte aligned device pointers");
    if ((rc = check_dev_ptr(d_logits, "d_logits", true))) return rc;
    const bool needs_qk = dec->sh.qk_norm != 0;
    for (int w = 0; w < kNumW; ++w) {
        if (!needs_qk && (w == M1MOE_W_Q_NORM || w == M1MOE_W_K_NORM)) continue;
        for (int l = 0; l < (per_layer(w) ? dec->L : 1); ++l)
            if (!dec->loaded[(size_t)w * dec->L + l])
                return fail(M1MOE_ERR_INVALID, "tensor %d of layer %d was not uploaded", w, l);
    }
    m1moe_ctx_t ctx = dec->moe;
    for (int l = 0; l < dec->L; ++l)
        if (!ctx->layer_loaded[l] || !ctx->router_loaded[l])
            return fail(M1MOE_ERR_INVALID, "MoE layer %d was not uploaded", l);
    if ((rc = set_device(ctx))) return rc;
    void* st = ctx->stream;
    const int32_t h = dec->h, qd = dec->qd, kvd = dec->kvd, V = dec->sh.vocab;
    const float eps = dec->sh.rms_eps;
    const DenseStepArgs a = step_args(dec, d_token_in);
    if ((rc = launched(launch_embed(a, st), "embed"))) return rc;
    AttnArgs at{};
    at.q = dec->q;
    at.out = dec->attn;
    at.partial = dec->part;
    at.seq_ptr = dec->pos;
    at.max_seq = dec->sh.max_seq;
    at.num_heads = dec->sh.num_heads;
    at.num_kv_heads = dec->sh.num_kv_heads;
    at.hpkv = dec->sh.num_heads / dec->sh.num_kv_heads;
    at.head_dim = dec->sh.head_dim;
    at.scale = 1.0f / sqrtf((float)dec->sh.head_dim);
    const uint64_t cache_layer = (uint64_t)dec->sh.max_seq * kvd;
    for (int l = 0; l < dec->L; ++l) {
        // input norm, q/k/v in one launch (InferenceEngine.swift:177-192)
        if ((rc = launched(launch_rmsnorm(dec->res, dec->in_norm + (size_t)l * h, dec->xn, h, eps, st),
                           "input norm")))
            return rc;
        MvArgs m{};
        m.seg[0] = MvSeg{dec->wq + (size_t)l * qd * h, dec->q, nullptr, qd};
        m.seg[1] = MvSeg{dec->wk + (size_t)l * kvd * h, dec->k, nullptr, kvd};
        m.seg[2] = MvSeg{dec->wv + (size_t)l * kvd * h, dec->v, nullptr, kvd};
        m.x = dec->xn;
        m.rows = qd + 2 * kvd;
        m.cols = h;
        if ((rc = launched(launch_matvec_bf16(m, st), "qkv"))) return rc;
        // q/k norms, RoPE, KV store (:194-220), attention (:226)
        if ((rc = launched(launch_qk_rope_kv(a, l, st), "qk norm / rope / kv store"))) return rc;
        at.kcache = dec->kcache + l * cache_layer;
        at.vcache = dec->vcache + l * cache_layer;
        if ((rc = launched(launch_attention(at, dec->sh.max_seq, st), "attention"))) return rc;
        // o_proj + residual, post-attention norm (:227-236)
        if ((rc = launched(launch_matvec_bf16(
                               mv_one(dec->wo + (size_t)l * h * qd, dec->attn, dec->res, dec->res2, h, qd), st),
                           "o_proj")))
            return rc;
        if ((rc = launched(launch_rmsnorm(dec->res2, dec->post_norm + (size_t)l * h, dec->hmid, h, eps, st),
                           "post-attention norm")))
            return rc;
        // the MoE block with the residual, its output the next residual (:240-266)
        if ((rc = m1moe_moe_decode(ctx, l, dec->hmid, M1MOE_F32, dec->res2, dec->res, nullptr, nullptr)))
            return rc;
    }
    // final norm, lm_head, greedy token, next position (:138-155)
    float* logits = d_logits ? d_logits : dec->logits;
    if ((rc = launched(launch_rmsnorm(dec->res, dec->final_norm, dec->xn, h, eps, st), "final norm")))
        return rc;
    if ((rc = launched(launch_matvec_bf16(mv_one(dec->lm_head, dec->xn, nullptr, logits, V, h), st),
                       "lm_head")))
        return rc;
    return launched(launch_argmax(logits, V, d_token_out, dec->pos, dec->sh.max_seq, st), "argmax");
}

}  // extern "C"
