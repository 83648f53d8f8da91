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

constexpr int kAttnCounters = 1024;  // >= num_heads (num_heads * 64 <= 65536); then the
                                     // synchronous merge's launch number and, 32 words on,
                                     // its finish counts (kCountWords)
constexpr int kAttnCntWords = kAttnCounters + 32 + kCountWords;
// the decoder's counters: 2 + num_heads + 1 words, then, 32-word aligned, the
// attention's finish counts and lm_head's (kCountWords each)
uint64_t dec_fin_offset(int num_heads) { return 32 * ((3 + (uint64_t)num_heads + 31) / 32); }
uint64_t dec_lm_offset(int num_heads) { return dec_fin_offset(num_heads) + kCountWords; }
uint64_t dec_cnt_words(int num_heads) { return dec_lm_offset(num_heads) + kCountWords; }

int32_t ensure_attn_scratch(m1moe_ctx_t ctx, uint64_t floats) {
    ctx->capture_uses_scratch = true;
    if (!ctx->attn_cnt || floats > ctx->attn_part_floats)
        if (int32_t rc = refuse_growth_in_capture(ctx->stream, "the attention scratch")) return rc;
    if (!ctx->attn_cnt) {
        int32_t rc = device_alloc((void**)&ctx->attn_cnt, kAttnCntWords * 4, "attention counters");
        if (rc) return rc;
        HIP_TRY(hipMemset(ctx->attn_cnt, 0, kAttnCntWords * 4));
    }
    if (floats <= ctx->attn_part_floats) return M1MOE_OK;
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    if (ctx->attn_part) ++ctx->scratch_gen;  // earlier graphs hold the old buffer
    if (ctx->attn_part) HIP_TRY(hipFree(ctx->attn_part));
    ctx->attn_part = nullptr;
    ctx->attn_part_floats = 0;
    int32_t rc = device_alloc((void**)&ctx->attn_part, floats * 4, "attention scratch");
    if (rc) return rc;
    // (zeroed: the synchronous merge accepts a value carrying the current
    // launch number, and reused device memory may hold one)
    HIP_TRY(hipMemset(ctx->attn_part, 0, floats * 4));
    ctx->attn_part_floats = floats;
    return M1MOE_OK;
}

int32_t check_attn_dims(int32_t nh, int32_t nkv, int32_t hd) {
    if (hd != 64 && hd != 128 && hd != 256)
        return fail(M1MOE_ERR_INVALID, "head_dim %d is not 64, 128 or 256", hd);
    if (nh <= 0 || nkv <= 0 || nh % nkv)
        return fail(M1MOE_ERR_INVALID, "num_heads %d must be a positive multiple of num_kv_heads %d",
                    nh, nkv);
    // the attention launch keeps one counter per group of q heads (at most
    // num_heads groups), kAttnCounters of them; with head_dim >= 64 this
    // bound keeps num_heads <= 1024
    if ((int64_t)nh * hd > 65536)
        return fail(M1MOE_ERR_INVALID, "num_heads * head_dim = %lld exceeds 65536",
                    (long long)nh * hd);
    if (nh > kAttnCounters)
        return fail(M1MOE_ERR_INVALID, "num_heads %d exceeds %d", nh, kAttnCounters);
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
    float *res = nullptr, *res2 = nullptr;
    float *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr;
    float *logits = nullptr, *part = nullptr;
    // prefill scratch for up to pf_cap tokens (grown on demand)
    int32_t pf_cap = 0;
    float *pf_res = nullptr, *pf_res2 = nullptr, *pf_xn = nullptr, *pf_qkv = nullptr, *pf_attn = nullptr;
    float* pf_part = nullptr;  // split-K partials of the prefill GEMMs (kGemmPartFloats)
    uint32_t* cnt = nullptr;   // [dec_cnt_words]: (unused) x 2, attention groups, the
                               // attention's launch number, then (dec_fin_offset) its
                               // finish counts and (dec_lm_offset) lm_head's
    float* ssq = nullptr;      // o_proj's per-workgroup sums of squares
    float* rope = nullptr;     // [max_seq][head_dim / 2] (cos, sin) of every position
    float* am_val = nullptr;   // lm_head's per-workgroup best logit
    int32_t* am_idx = nullptr;
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
    a.fused = 0;
    a.q = d_q;
    a.kcache = const_cast<float*>(d_kcache);  // read only when fused = 0
    a.vcache = const_cast<float*>(d_vcache);
    a.out = d_out;
    a.partial = ctx->attn_part;
    a.counters = ctx->attn_cnt;
    a.err = ctx->err;
    a.seq_len = seq_len;
    a.max_seq = seq_len;
    a.num_heads = num_heads;
    a.num_kv_heads = num_kv_heads;
    a.hpkv = num_heads / num_kv_heads;
    a.head_dim = head_dim;
    a.qh = attention_qh(a.hpkv);
    a.cus = ctx->cus;
    a.chunk = attention_chunk(seq_len, num_heads / a.qh, a.cus);
    a.kv_pos = (int64_t)num_kv_heads * head_dim;   // the caller's [seq_len][num_kv_heads][head_dim]
    a.kv_head = head_dim;
    a.scale = 1.0f / sqrtf((float)head_dim);
    a.gen = ctx->attn_cnt + kAttnCounters;
    a.fin = ctx->attn_cnt + kAttnCounters + 32;
    a.spin_limit = kAttnSpinLimit;
    a.sync_merge = attention_grid_fits(a) ? 1 : 0;
    return launched(launch_attention(a, ctx->stream), "attention");
}

int32_t m1moe_argmax(m1moe_ctx_t ctx, const float* d_x, int32_t n, int32_t* d_idx) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = check_f32_vec(d_x, "d_x"))) return rc;
    if (!d_idx) return fail(M1MOE_ERR_INVALID, "d_idx is null");
    if (n <= 0) return fail(M1MOE_ERR_INVALID, "n %d must be positive", n);
    if ((rc = set_device(ctx))) return rc;
    return launched(launch_argmax(d_x, n, d_idx, ctx->stream), "argmax");
}

// ---- the decoder ---------------------------------------------------------------------

void m1moe_dec_destroy(m1moe_dec_t dec) {
    if (!dec) return;
    (void)hipSetDevice(dec->device);
    for (void* p : dec->allocs) (void)hipFree(p);
    for (void* p : {(void*)dec->pf_res, (void*)dec->pf_res2, (void*)dec->pf_xn, (void*)dec->pf_qkv,
                    (void*)dec->pf_attn, (void*)dec->pf_part})
        if (p) (void)hipFree(p);
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
    if (moe->g.h > kMvStageMax)
        return fail(M1MOE_ERR_INVALID, "hidden %d exceeds the decoder's %d (normalised inputs are "
                    "staged in LDS)", moe->g.h, kMvStageMax);
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
        (rc = dec_alloc(d, (void**)&d->q, qd * 4, "q")) ||
        (rc = dec_alloc(d, (void**)&d->k, kvd * 4, "k")) ||
        (rc = dec_alloc(d, (void**)&d->v, kvd * 4, "v")) ||
        (rc = dec_alloc(d, (void**)&d->attn, qd * 4, "attention output")) ||
        (rc = dec_alloc(d, (void**)&d->logits, V * 4, "logits")) ||
        (rc = dec_alloc(d, (void**)&d->part, part * 4, "attention scratch")) ||
        (rc = dec_alloc(d, (void**)&d->cnt, dec_cnt_words(s->num_heads) * 4, "counters")) ||
        (rc = dec_alloc(d, (void**)&d->ssq, (uint64_t)matvec_workgroups(d->h) * 4, "o_proj sums")) ||
        (rc = dec_alloc(d, (void**)&d->rope, ms * hd * 4, "RoPE table")) ||
        (rc = dec_alloc(d, (void**)&d->am_val, (uint64_t)matvec_workgroups(s->vocab) * 4, "argmax scratch")) ||
        (rc = dec_alloc(d, (void**)&d->am_idx, (uint64_t)matvec_workgroups(s->vocab) * 4, "argmax scratch"))) {
        m1moe_dec_destroy(d);
        return rc;
    }
    // (the partials are zeroed: the synchronous merge accepts a value by its
    // launch number, which starts at 1, and reused device memory may hold any)
    if (hipMemset(d->pos, 0, 16) != hipSuccess ||
        hipMemset(d->cnt, 0, dec_cnt_words(s->num_heads) * 4) != hipSuccess ||
        hipMemset(d->part, 0, part * 4) != hipSuccess ||
        launch_rope_table(d->rope, s->max_seq, s->head_dim, s->rope_theta, moe->stream) != 0 ||
        hipStreamSynchronize(moe->stream) != hipSuccess) {
        m1moe_dec_destroy(d);
        return fail(M1MOE_ERR_HIP, "decoder state initialisation failed");
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

}  // extern "C"

namespace {

// Every dense tensor of the decoder and every MoE layer of its context uploaded.
int32_t check_loaded(const m1moe_dec* dec) {
    const bool needs_qk = dec->sh.qk_norm != 0;
    for (int w = 0; w < kNumW; ++w) {
        if (!needs_qk && (w == M1MOE_W_Q_NORM || w == M1MOE_W_K_NORM)) continue;
        for (int l = 0; l < (per_layer(w) ? dec->L : 1); ++l)
            if (!dec->loaded[(size_t)w * dec->L + l])
                return fail(M1MOE_ERR_INVALID, "tensor %d of layer %d was not uploaded", w, l);
    }
    for (int l = 0; l < dec->L; ++l)
        if (!dec->moe->layer_loaded[l] || !dec->moe->router_loaded[l])
            return fail(M1MOE_ERR_INVALID, "MoE layer %d was not uploaded", l);
    return M1MOE_OK;
}

// One step; seq_cap == 0: token from *tok_in, greedy token to *tok_out;
// seq_cap > 0: sequence mode over tok_out[0 .. seq_cap) (tok_in == tok_out).
int32_t dec_step(m1moe_dec_t dec, const int32_t* tok_in, int32_t* tok_out, int32_t n_prompt,
                 int32_t seq_cap, float* d_logits) {
    int32_t rc;
    if (!dec) return fail(M1MOE_ERR_INVALID, "null decoder");
    if ((rc = check_dev_ptr(d_logits, "d_logits", true))) return rc;
    if ((rc = check_loaded(dec))) return rc;
    m1moe_ctx_t ctx = dec->moe;
    if ((rc = set_device(ctx))) return rc;
    void* st = ctx->stream;
    const int32_t h = dec->h, qd = dec->qd, kvd = dec->kvd, V = dec->sh.vocab, hd = dec->sh.head_dim;
    const float eps = dec->sh.rms_eps;
    const bool qk = dec->sh.qk_norm != 0;
    AttnArgs at{};
    at.fused = 1;
    at.q = dec->q;
    at.k_new = dec->k;
    at.v_new = dec->v;
    at.out = dec->attn;
    at.partial = dec->part;
    at.counters = dec->cnt + 2;
    at.pos = dec->pos;
    at.err = ctx->err;
    at.max_seq = dec->sh.max_seq;
    at.num_heads = dec->sh.num_heads;
    at.num_kv_heads = dec->sh.num_kv_heads;
    at.hpkv = dec->sh.num_heads / dec->sh.num_kv_heads;
    at.head_dim = hd;
    at.qh = attention_qh(at.hpkv);
    at.cus = ctx->cus;
    at.chunk = attention_chunk(dec->sh.max_seq, at.num_heads / at.qh, at.cus);
    at.kv_pos = kvd;
    at.kv_head = hd;
    at.scale = 1.0f / sqrtf((float)hd);
    at.rope_theta = dec->sh.rope_theta;
    at.eps = eps;
    at.gen = dec->cnt + 2 + dec->sh.num_heads;
    at.fin = dec->cnt + dec_fin_offset(dec->sh.num_heads);
    at.spin_limit = kAttnSpinLimit;
    at.sync_merge = attention_grid_fits(at) ? 1 : 0;
    at.rope = dec->rope;
    // short contexts: o_proj merges the attention partials while staging its
    // input (only a staged input can: q widths up to kMvStageMax)
    at.defer = qd <= kMvStageMax ? 1 : 0;
    const uint64_t cache_layer = (uint64_t)dec->sh.max_seq * kvd;
    for (int l = 0; l < dec->L; ++l) {
        // input RMSNorm and q/k/v in one launch (InferenceEngine.swift:177-192); layer 0
        // takes its input from the embedding table at the step's token (:129-131)
        MvArgs m{};
        m.seg[0] = MvSeg{dec->wq + (size_t)l * qd * h, dec->q, nullptr, qd};
        m.seg[1] = MvSeg{dec->wk + (size_t)l * kvd * h, dec->k, nullptr, kvd};
        m.seg[2] = MvSeg{dec->wv + (size_t)l * kvd * h, dec->v, nullptr, kvd};
        m.rows = qd + 2 * kvd;
        m.cols = h;
        m.norm_w = dec->in_norm + (size_t)l * h;
        m.eps = eps;
        m.err = ctx->err;
        if (l == 0) {
            m.embed = dec->embed;
            m.token = tok_in;
            m.seq_cap = seq_cap;
            m.pos = dec->pos;
            m.vocab = V;
            m.x_copy = dec->res;
        } else {
            m.x = dec->res;
        }
        if ((rc = launched(launch_matvec_bf16(m, st), "qkv"))) return rc;
        // q/k norms, RoPE, KV store (:194-220) and attention (:226)
        at.q_norm = qk ? dec->q_norm + (size_t)l * hd : nullptr;
        at.k_norm = qk ? dec->k_norm + (size_t)l * hd : nullptr;
        at.kcache = dec->kcache + l * cache_layer;
        at.vcache = dec->vcache + l * cache_layer;
        // o_proj's weights into the caches while the attention runs (piece b:
        // the rows of o_proj's workgroup b)
        at.pf = reinterpret_cast<const uint8_t*>(dec->wo + (size_t)l * h * qd);
        at.pf_unit = (int64_t)matvec_rows_per_workgroup(h) * qd * 2;
        at.pf_bytes = (int64_t)h * qd * 2;
        at.pf_units = matvec_workgroups(h);
        if ((rc = launched(launch_attention(at, st), "attention"))) return rc;
        // o_proj + residual (:227-233), with the sums of squares of its rows
        MvArgs o = mv_one(dec->wo + (size_t)l * h * qd, dec->attn, dec->res, dec->res2, h, qd);
        o.ssq_out = dec->ssq;
        // its input from the attention partials when that launch deferred their merge
        o.attn_part = at.defer ? dec->part : nullptr;
        o.attn_heads = at.num_heads;
        o.attn_qh = at.qh;
        o.attn_hd = hd;
        o.attn_chunk = at.chunk;
        o.attn_nch = (at.max_seq + at.chunk - 1) / at.chunk;
        o.pos = dec->pos;
        o.max_seq = at.max_seq;
        if ((rc = launched(launch_matvec_bf16(o, st), "o_proj"))) return rc;
        // the post-attention RMSNorm (:234-236) applied by the MoE kernel to its
        // input, the MoE block with the residual, its output the next residual
        // (:240-266)
        if ((rc = moe_decode_normed(ctx, l, dec->res2, dec->ssq, matvec_workgroups(h),
                                    dec->post_norm + (size_t)l * h, eps, dec->res2, dec->res)))
            return rc;
    }
    // final RMSNorm, lm_head, greedy token, next position (:138-155)
    MvArgs f = mv_one(dec->lm_head, dec->res, nullptr, d_logits ? d_logits : dec->logits, V, h);
    f.norm_w = dec->final_norm;
    f.eps = eps;
    f.counter = dec->cnt + dec_lm_offset(dec->sh.num_heads);
    f.am_val = dec->am_val;
    f.am_idx = dec->am_idx;
    f.tok_out = tok_out;
    f.n_prompt = n_prompt;
    f.seq_cap = seq_cap;
    f.pos = dec->pos;
    f.max_seq = dec->sh.max_seq;
    f.err = ctx->err;
    return launched(launch_matvec_bf16(f, st), "lm_head");
}

bool aligned_i32(const void* p) { return p && reinterpret_cast<uintptr_t>(p) % 4 == 0; }

}  // namespace

int32_t m1moe::dec_dims(m1moe_dec_t dec, int32_t* vocab, int32_t* num_heads, int32_t* num_kv_heads,
                        int32_t* head_dim, int32_t* qk_norm) {
    if (!dec) return fail(M1MOE_ERR_INVALID, "null decoder");
    *vocab = dec->sh.vocab;
    *num_heads = dec->sh.num_heads;
    *num_kv_heads = dec->sh.num_kv_heads;
    *head_dim = dec->sh.head_dim;
    *qk_norm = dec->sh.qk_norm;
    return M1MOE_OK;
}

extern "C" {

int32_t m1moe_dec_step(m1moe_dec_t dec, const int32_t* d_token_in, int32_t* d_token_out,
                       float* d_logits) {
    if (!aligned_i32(d_token_in) || !aligned_i32(d_token_out))
        return fail(M1MOE_ERR_INVALID, "d_token_in / d_token_out must be 4-byte aligned device pointers");
    return dec_step(dec, d_token_in, d_token_out, 0, 0, d_logits);
}

namespace {
constexpr int32_t kPrefillPiece = 4096;  // tokens per batched pass (the MoE prefill's cap)

int32_t dec_prefill_piece(m1moe_dec_t dec, const int32_t* d_tokens, int32_t T,
                          int32_t* d_token_out, float* d_logits);
}  // namespace

int32_t m1moe_dec_prefill(m1moe_dec_t dec, const int32_t* d_tokens, int32_t T, int32_t* d_token_out,
                          float* d_logits) {
    int32_t rc;
    if (!dec) return fail(M1MOE_ERR_INVALID, "null decoder");
    if (!aligned_i32(d_tokens) || !aligned_i32(d_token_out))
        return fail(M1MOE_ERR_INVALID, "d_tokens / d_token_out must be 4-byte aligned device pointers");
    if ((rc = check_dev_ptr(d_logits, "d_logits", true))) return rc;
    if (T < 1 || T > dec->sh.max_seq)
        return fail(M1MOE_ERR_INVALID, "T=%d must be in [1, max_seq=%d]", T, dec->sh.max_seq);
    if ((rc = check_loaded(dec))) return rc;
    // longer prompts in pieces: each continues from the device position the
    // previous one advanced; the last one gives the greedy token and logits
    for (int32_t off = 0; off < T; off += kPrefillPiece) {
        const int32_t n = T - off < kPrefillPiece ? T - off : kPrefillPiece;
        const bool last = off + n == T;
        if ((rc = dec_prefill_piece(dec, d_tokens + off, n, d_token_out, last ? d_logits : nullptr)))
            return rc;
    }
    return M1MOE_OK;
}

namespace {
int32_t dec_prefill_piece(m1moe_dec_t dec, const int32_t* d_tokens, int32_t T,
                          int32_t* d_token_out, float* d_logits) {
    int32_t rc;
    m1moe_ctx_t ctx = dec->moe;
    if ((rc = set_device(ctx))) return rc;
    ctx->capture_uses_scratch = true;
    const int32_t h = dec->h, qd = dec->qd, kvd = dec->kvd, hd = dec->sh.head_dim;
    const int32_t N = qd + 2 * kvd;
    if (T > dec->pf_cap) {
        if ((rc = refuse_growth_in_capture(ctx->stream, "the decoder prefill scratch"))) return rc;
        HIP_TRY(hipStreamSynchronize(ctx->stream));
        if (dec->pf_cap > 0) ++ctx->scratch_gen;  // earlier graphs hold the old buffers
        for (float** b : {&dec->pf_res, &dec->pf_res2, &dec->pf_xn, &dec->pf_qkv, &dec->pf_attn, &dec->pf_part}) {
            if (*b) (void)hipFree(*b);
            *b = nullptr;
        }
        dec->pf_cap = 0;
        const uint64_t t = (uint64_t)T;
        if ((rc = device_alloc((void**)&dec->pf_res, t * h * 4, "prefill residual")) ||
            (rc = device_alloc((void**)&dec->pf_res2, t * h * 4, "prefill residual 2")) ||
            (rc = device_alloc((void**)&dec->pf_xn, t * h * 4, "prefill normed rows")) ||
            (rc = device_alloc((void**)&dec->pf_qkv, t * N * 4, "prefill q/k/v")) ||
            (rc = device_alloc((void**)&dec->pf_attn, t * qd * 4, "prefill attention")) ||
            (rc = device_alloc((void**)&dec->pf_part, kGemmPartFloats * 4, "prefill split-K partials")))
            return rc;
        dec->pf_cap = T;
    }
    void* st = ctx->stream;
    const float eps = dec->sh.rms_eps;
    const bool qk = dec->sh.qk_norm != 0;
    PfDenseArgs a{};
    a.tokens = d_tokens;
    a.embed = dec->embed;
    a.res = dec->pf_res;
    a.qkv = dec->pf_qkv;
    a.attn = dec->pf_attn;
    a.pos = dec->pos;
    a.err = ctx->err;
    a.T = T;
    a.vocab = dec->sh.vocab;
    a.h = h;
    a.ldqkv = N;
    a.qd = qd;
    a.kvd = kvd;
    a.num_heads = dec->sh.num_heads;
    a.num_kv_heads = dec->sh.num_kv_heads;
    a.hpkv = dec->sh.num_heads / dec->sh.num_kv_heads;
    a.head_dim = hd;
    a.max_seq = dec->sh.max_seq;
    a.scale = 1.0f / sqrtf((float)hd);
    a.rope_theta = dec->sh.rope_theta;
    a.eps = eps;
    auto gemm = [&](const float* A, int lda, const uint16_t* W, const float* R, float* C, int ldc, int n,
                    int k, const char* what) {
        GemmArgs g{};
        g.A = A;
        g.lda = lda;
        g.W = W;
        g.R = R;
        g.C = C;
        g.ldc = ldc;
        g.M = T;
        g.N = n;
        g.K = k;
        g.part = dec->pf_part;
        return launched(launch_gemm(g, st), what);
    };
    // q, k and v: one launch over the three weight segments when the prompt
    // is short (each alone would leave most CUs idle), three launches else
    const bool merge_qkv = h % 64 == 0 && (long)((N + 127) / 128) * ((T + 127) / 128) < 256;
    auto qkv_gemm = [&](int l) -> int32_t {
        const uint16_t* wq = dec->wq + (size_t)l * qd * h;
        const uint16_t* wk = dec->wk + (size_t)l * kvd * h;
        const uint16_t* wv = dec->wv + (size_t)l * kvd * h;
        if (merge_qkv) {
            GemmArgs g{};
            g.A = dec->pf_xn;
            g.lda = h;
            g.W = wq;
            g.W1 = wk;
            g.W2 = wv;
            g.n1 = qd;
            g.n2 = qd + kvd;
            g.C = dec->pf_qkv;
            g.ldc = N;
            g.M = T;
            g.N = N;
            g.K = h;
            g.part = dec->pf_part;
            return launched(launch_gemm(g, st), "prefill q/k/v");
        }
        int32_t r;
        if ((r = gemm(dec->pf_xn, h, wq, nullptr, dec->pf_qkv, N, qd, h, "prefill q")) ||
            (r = gemm(dec->pf_xn, h, wk, nullptr, dec->pf_qkv + qd, N, kvd, h, "prefill k")) ||
            (r = gemm(dec->pf_xn, h, wv, nullptr, dec->pf_qkv + qd + kvd, N, kvd, h, "prefill v")))
            return r;
        return M1MOE_OK;
    };
    if ((rc = launched(launch_pf_embed(a, st), "prefill embedding"))) return rc;  // :129-131
    const uint64_t cache_layer = (uint64_t)dec->sh.max_seq * kvd;
    for (int l = 0; l < dec->L; ++l) {
        // input RMSNorm, q/k/v for all T tokens (InferenceEngine.swift:177-192)
        if ((rc = launched(launch_rmsnorm_rows(dec->pf_res, dec->in_norm + (size_t)l * h, dec->pf_xn, T, h,
                                               eps, st),
                           "prefill input norm")) ||
            (rc = qkv_gemm(l)))
            return rc;
        // q/k norms, RoPE, KV rows (:194-220); causal attention (:226)
        a.q_norm = qk ? dec->q_norm + (size_t)l * hd : nullptr;
        a.k_norm = qk ? dec->k_norm + (size_t)l * hd : nullptr;
        a.kcache = dec->kcache + l * cache_layer;
        a.vcache = dec->vcache + l * cache_layer;
        if ((rc = launched(launch_pf_rope_kv(a, st), "prefill rope / kv rows")) ||
            (rc = launched(launch_pf_attention(a, st), "prefill attention")))
            return rc;
        // o_proj + residual (:227-233), post-attention RMSNorm (:234-236)
        // (the norm is made by the GEMM's split-K sum when it has one)
        GemmArgs o{};
        o.A = dec->pf_attn;
        o.lda = qd;
        o.W = dec->wo + (size_t)l * h * qd;
        o.R = dec->pf_res;
        o.C = dec->pf_res2;
        o.ldc = h;
        o.M = T;
        o.N = h;
        o.K = qd;
        o.part = dec->pf_part;
        o.norm_w = dec->post_norm + (size_t)l * h;
        o.norm_out = dec->pf_xn;
        o.norm_eps = eps;
        if ((rc = launched(launch_gemm(o, st), "prefill o_proj + post-attention norm"))) return rc;
        // the MoE block for the T tokens, its output the next residual (:240-266)
        if ((rc = m1moe_moe_prefill(ctx, l, T, dec->pf_xn, M1MOE_F32, dec->pf_res2, dec->pf_res, nullptr,
                                    nullptr)))
            return rc;
    }
    // the position moves past the prompt; the last token's final norm, lm_head
    // and greedy token advance it by the last one (:138-155)
    if ((rc = launched(launch_advance_pos(dec->pos, T - 1, dec->sh.max_seq, st), "prefill position")))
        return rc;
    MvArgs f = mv_one(dec->lm_head, dec->pf_res + (size_t)(T - 1) * h, nullptr,
                      d_logits ? d_logits : dec->logits, dec->sh.vocab, h);
    f.norm_w = dec->final_norm;
    f.eps = eps;
    f.counter = dec->cnt + dec_lm_offset(dec->sh.num_heads);
    f.am_val = dec->am_val;
    f.am_idx = dec->am_idx;
    f.tok_out = d_token_out;
    f.pos = dec->pos;
    f.max_seq = dec->sh.max_seq;
    f.err = ctx->err;
    return launched(launch_matvec_bf16(f, st), "prefill lm_head");
}
}  // namespace

int32_t m1moe_dec_step_seq(m1moe_dec_t dec, int32_t* d_seq, int32_t n_prompt, int32_t seq_cap,
                           float* d_logits) {
    if (!aligned_i32(d_seq)) return fail(M1MOE_ERR_INVALID, "d_seq must be a 4-byte aligned device pointer");
    if (seq_cap <= 0 || n_prompt < 1 || n_prompt > seq_cap)
        return fail(M1MOE_ERR_INVALID, "need 1 <= n_prompt (%d) <= seq_cap (%d)", n_prompt, seq_cap);
    return dec_step(dec, d_seq, d_seq, n_prompt, seq_cap, d_logits);
}

}  // extern "C"
