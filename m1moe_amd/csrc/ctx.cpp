// ctx.cpp — the C ABI of libm1moe_hip.so: context, validation, uploads,
// memory/stream/event/graph plumbing, and the MoE-block entry points.
//
// The context replaces the reference's MetalContext (MetalContext.swift:
// 69-185) for the MoE block: it owns the resident expert arena (every
// expert of every layer in HBM, replacing the pread dispatch and the K
// expert slots, InferenceEngine.swift:62-77,271-280, MetalContext.swift:
// 154-172), the bf16 routers (kept bf16, unlike the f32 pre-conversion at
// InferenceEngine.swift:99-113) and all scratch.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <set>
#include <string>
#include <vector>

#include "ctx.hpp"
#include "internal.hpp"
#include "m1moe_hip.h"

namespace m1moe {

namespace {
thread_local std::string g_last_error;
constexpr int32_t kPrefillCap = 4096;  // tokens per m1moe_moe_prefill call
}  // namespace

int32_t fail(int32_t code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

Geom make_geom(const m1moe_moe_shape& s) {
    Geom g{};
    g.h = s.hidden;
    g.E = s.num_experts;
    g.K = s.top_k;
    g.I = s.intermediate;
    g.gs = s.group_size;
    g.L = s.num_layers;
    g.norm = s.norm_topk_prob;
    const uint64_t h = (uint64_t)s.hidden, i = (uint64_t)s.intermediate;
    const uint64_t gs = (uint64_t)s.group_size;
    const uint64_t gw = i * (h / 8) * 4, gsb = i * (h / gs) * 2;
    const uint64_t dw = h * (i / 8) * 4, dsb = h * (i / gs) * 2;
    const uint64_t sizes[9] = {gw, gsb, gsb, gw, gsb, gsb, dw, dsb, dsb};
    uint64_t o = 0;
    for (int k = 0; k < 9; ++k) {
        g.off[k] = o;
        o += sizes[k];
    }
    g.expert_bytes = o;
    return g;
}

}  // namespace m1moe

namespace {
using namespace m1moe;

constexpr int32_t kSpinLimit = 1 << 20;  // bounded waits in the decode kernel (~1 s)

// The one library stream of each device, shared by every context on it, so
// that no two launches of the library overlap on a device (the per-CU decode
// kernels wait for all 256 of their workgroups, which must be resident
// together; the reference drives its engine from one serial queue,
// MetalContext.swift:73-77, Sources/bench/main.swift:58).  A caller stream
// (m1moe_set_stream) is accepted only while its context is the device's only
// one, and no second context is created on the device until it is unset.
struct DeviceShare {
    hipStream_t stream = nullptr;
    int users = 0;
    m1moe_ctx_t on_caller_stream = nullptr;
};
std::mutex g_share_mu;
std::map<int32_t, DeviceShare> g_share;

int32_t share_join(m1moe_ctx_t c) {
    std::lock_guard<std::mutex> lk(g_share_mu);
    DeviceShare& d = g_share[c->device];
    if (d.users > 0 && d.on_caller_stream)
        return fail(M1MOE_ERR_INVALID,
                    "device %d's other context enqueues on a caller stream (m1moe_set_stream); "
                    "set it back to NULL before creating another context on the device (all "
                    "contexts on one device share one stream)", c->device);
    if (!d.stream) {
        hipError_t e = hipStreamCreateWithFlags(&d.stream, hipStreamNonBlocking);
        if (e != hipSuccess) {
            d.stream = nullptr;
            if (d.users == 0) g_share.erase(c->device);
            return fail(M1MOE_ERR_HIP, "hipStreamCreate failed: %s", hipGetErrorString(e));
        }
    }
    ++d.users;
    c->registered = true;
    c->lib_stream = d.stream;
    c->stream = d.stream;
    return M1MOE_OK;
}

void share_leave(m1moe_ctx_t c) {
    if (!c->registered) return;
    std::lock_guard<std::mutex> lk(g_share_mu);
    auto it = g_share.find(c->device);
    if (it == g_share.end()) return;
    DeviceShare& d = it->second;
    if (d.on_caller_stream == c) d.on_caller_stream = nullptr;
    if (--d.users == 0) {
        if (d.stream) (void)hipStreamDestroy(d.stream);
        g_share.erase(it);
    }
    c->registered = false;
}

m1moe::FusedArgs fused_args(m1moe_ctx_t ctx, int32_t layer, const void* x, int32_t x_dtype,
                            const float* residual, float* out) {
    const m1moe::Geom& g = ctx->g;
    m1moe::FusedArgs a{};
    a.layer_base = ctx->arena + (uint64_t)layer * g.E * g.expert_bytes;
    a.expert_bytes = g.expert_bytes;
    a.router = ctx->routers + (uint64_t)layer * g.E * g.h;
    a.next_router = ctx->routers + (uint64_t)((layer + 1) % ctx->shape.num_layers) * g.E * g.h;
    a.bias = ctx->has_bias[layer] ? ctx->biases + (uint64_t)layer * g.E : nullptr;
    a.x = x;
    a.residual = residual;
    a.out = out;
    a.slots = reinterpret_cast<unsigned long long*>(ctx->sync);
    a.act = ctx->act;
    a.gu_cnt = reinterpret_cast<uint32_t*>(ctx->sync + ctx->sync_gu_cnt);
    a.seen = reinterpret_cast<uint32_t*>(ctx->sync + ctx->sync_seen);
    a.cu_seen = reinterpret_cast<uint32_t*>(ctx->sync + ctx->sync_cu_seen);
    a.cu_cnt = reinterpret_cast<uint32_t*>(ctx->sync + ctx->sync_cu_cnt);
    a.cu_part = reinterpret_cast<uint32_t*>(ctx->sync + ctx->sync_cu_part);
    a.xl = reinterpret_cast<unsigned long long*>(ctx->sync + ctx->sync_xl);
    a.dec_base = ctx->dec ? ctx->dec + (uint64_t)layer * g.E * ctx->dec_bytes : nullptr;
    a.dec_bytes = ctx->dec_bytes;
    a.err = ctx->err;
    a.h = g.h;
    a.E = g.E;
    a.K = g.K;
    a.I = g.I;
    a.gs = g.gs;
    a.norm = g.norm;
    a.x_bf16 = (x_dtype == M1MOE_BF16);
    a.spin_limit = kSpinLimit;
    return a;
}

// Rebuilds a layer's repacked copy when its canonical blocks may have been
// written through m1moe_expert_block since it was made (enqueued before the
// decode on the context stream; refused while the stream is captured).
int32_t refresh_decode_copy(m1moe_ctx_t ctx, int32_t layer) {
    if (!ctx->decode_cu || !ctx->dec_stale[layer]) return M1MOE_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(ctx->stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return fail(M1MOE_ERR_INVALID,
                    "layer %d's expert blocks were handed out for writing since its repacked "
                    "copy was made; decode it once outside stream capture first", layer);
    const uint64_t lb = (uint64_t)ctx->g.E * ctx->g.expert_bytes;
    HIP_TRY((hipError_t)m1moe::launch_decode_copy(
        ctx->arena + (uint64_t)layer * lb, ctx->g.expert_bytes,
        ctx->dec + (uint64_t)layer * ctx->g.E * ctx->dec_bytes, ctx->g.E, ctx->g.h, ctx->g.I,
        ctx->g.gs,
        ctx->stream));
    ctx->dec_stale[layer] = false;
    return M1MOE_OK;
}

int32_t launch_pft_copy(m1moe_ctx_t ctx, int32_t layer) {
    const uint64_t lb = (uint64_t)ctx->g.E * ctx->g.expert_bytes;
    HIP_TRY((hipError_t)m1moe::launch_pf_tile_copy(
        ctx->arena + (uint64_t)layer * lb, ctx->g.expert_bytes,
        ctx->pft + (uint64_t)layer * ctx->g.E * ctx->pft_bytes, ctx->g.E, ctx->g.h, ctx->g.I,
        ctx->g.gs, ctx->err, ctx->stream));
    ctx->pft_stale[layer] = false;
    return M1MOE_OK;
}

// The prefill copies of a layer whose expert blocks were handed out for
// writing since they were made.
int32_t refresh_pft_copy(m1moe_ctx_t ctx, int32_t layer) {
    if (!ctx->pft_stale[layer]) return M1MOE_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(ctx->stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return fail(M1MOE_ERR_INVALID,
                    "layer %d's expert blocks were handed out for writing since its prefill "
                    "copy was made; run its prefill once outside stream capture first", layer);
    return launch_pft_copy(ctx, layer);
}

int enqueue_decode(m1moe_ctx_t ctx, const m1moe::FusedArgs& a) {
    return ctx->decode_cu ? m1moe::launch_moe_decode_cu(a, ctx->stream)
                          : m1moe::launch_moe_decode(a, ctx->stream);
}

// (xq / xinv: the prefill's f16 copy of x, made by the logits kernel, or null)
int32_t enqueue_router(m1moe_ctx_t ctx, int32_t layer, int32_t T, const void* x,
                       int32_t x_dtype, int32_t* uidx, float* uw, float* ulogits,
                       _Float16* xq = nullptr, float* xinv = nullptr) {
    const m1moe::Geom& g = ctx->g;
    m1moe::RouterArgs r{};
    r.router = ctx->routers + (uint64_t)layer * g.E * g.h;
    r.bias = ctx->has_bias[layer] ? ctx->biases + (uint64_t)layer * g.E : nullptr;
    r.x = x;
    r.x_bf16 = (x_dtype == M1MOE_BF16);
    r.T = T;
    r.E = g.E;
    r.h = g.h;
    r.K = g.K;
    r.norm = g.norm;
    r.logits = ctx->logits;
    r.idx = ctx->topk_idx;
    r.w = ctx->topk_w;
    r.user_idx = uidx;
    r.user_w = uw;
    r.user_logits = ulogits;
    r.counters = ctx->counters;
    r.xq = xq;
    r.xinv = xinv;
    return launched(m1moe::launch_router_topk(r, ctx->stream), "router_topk");
}

// Sizes in bytes of the kPfBufs prefill scratch buffers for T tokens, in the
// order of PrefillArgs: xq, xinv, pos, sorted_tok, expert_off, tile_off,
// tile_desc, act, y, act_exp, act_flag.
void prefill_scratch_sizes(const m1moe::Geom& g, int32_t T, uint64_t sz[m1moe::kPfBufs]) {
    const uint64_t t = (uint64_t)T, P = t * (uint64_t)g.K, E = (uint64_t)g.E;
    sz[0] = t * g.h * 2;
    sz[1] = t * 4;
    sz[2] = P * 4;
    sz[3] = P * 8;
    sz[4] = (E + 1) * 4;
    sz[5] = (E + 1) * 4;
    sz[6] = (P / m1moe::kPfTN + E + 1) * 16;
    sz[7] = P * g.I * 2;
    sz[8] = P * g.h * 4;
    sz[9] = P * (g.I / 32) + 4;   // (+4: the down GEMM reads E as a whole aligned word)
    sz[10] = 4 * (m1moe::kPfFlagWords + (P + 31) / 32);
}

// Bytes of the kPfBufs buffers carved from one block, each 256-byte aligned.
uint64_t prefill_scratch_packed(const m1moe::Geom& g, int32_t T) {
    uint64_t sz[m1moe::kPfBufs], total = 0;
    prefill_scratch_sizes(g, T, sz);
    for (uint64_t b : sz) total += (b + 255) / 256 * 256;
    return total;
}

// Grows the prefill scratch to exactly T tokens when a call needs more than
// it holds.  Growth frees the old buffers, so it is refused during stream
// capture, and a graph captured before a call with a larger T must be
// captured again.
int32_t ensure_prefill_scratch(m1moe_ctx_t ctx, int32_t T) {
    ctx->capture_uses_scratch = true;
    if (T <= ctx->pf_cap) return M1MOE_OK;
    if (int32_t rc = m1moe::refuse_growth_in_capture(ctx->stream, "the prefill scratch")) return rc;
    void** bufs[m1moe::kPfBufs] = {
        (void**)&ctx->pf_xq,    (void**)&ctx->pf_xinv, (void**)&ctx->pf_pos,
        (void**)&ctx->pf_sorted, (void**)&ctx->pf_eoff, (void**)&ctx->pf_toff,
        (void**)&ctx->pf_tdesc, (void**)&ctx->pf_act,  (void**)&ctx->pf_y,
        (void**)&ctx->pf_aexp,  (void**)&ctx->pf_aflag};
    static const char* const names[m1moe::kPfBufs] = {
        "prefill x",       "prefill x scales",   "prefill positions",
        "prefill sorted tokens", "prefill expert offsets", "prefill tile offsets",
        "prefill tile descriptors", "prefill act",        "prefill expert outputs",
        "prefill act exponents", "prefill act flag"};
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    if (ctx->pf_cap > 0) ++ctx->scratch_gen;  // earlier graphs hold the old buffers
    for (void** b : bufs) {
        if (*b) (void)hipFree(*b);
        *b = nullptr;
    }
    ctx->pf_cap = 0;
    uint64_t sz[m1moe::kPfBufs];
    prefill_scratch_sizes(ctx->g, T, sz);
    for (int i = 0; i < m1moe::kPfBufs; ++i)
        if (int32_t rc = device_alloc(bufs[i], sz[i], names[i])) return rc;
    ctx->pf_cap = T;
    return M1MOE_OK;
}

int32_t require_loaded(m1moe_ctx_t ctx, int32_t layer, bool router) {
    if (!ctx->layer_loaded[layer])
        return fail(M1MOE_ERR_INVALID, "layer %d experts were never uploaded", layer);
    if (router && !ctx->router_loaded[layer])
        return fail(M1MOE_ERR_INVALID, "layer %d router was never uploaded", layer);
    return M1MOE_OK;
}

// m1moe_moe_prefill and its allocation-free variant: the same kernels, with
// the scratch either grown in the context (allocates when T exceeds every
// earlier call) or carved from this device's fixed static scratch (allocates
// nothing; T is limited by its size).
int32_t prefill_common(m1moe_ctx_t ctx, int32_t layer, int32_t T, const void* d_x,
                       int32_t x_dtype, const float* d_residual, float* d_out,
                       int32_t* d_topk_idx, float* d_topk_w, bool use_static) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = check_layer(ctx, layer))) return rc;
    if (T < 1 || T > m1moe::kPrefillCap)
        return fail(M1MOE_ERR_INVALID, "T=%d must be in [1, %d]", T, m1moe::kPrefillCap);
    if ((rc = check_dtype(x_dtype)) || (rc = check_dev_ptr(d_x, "d_x", false)) ||
        (rc = check_dev_ptr(d_residual, "d_residual", true)) ||
        (rc = check_dev_ptr(d_out, "d_out", false)) ||
        (rc = check_dev_ptr(d_topk_idx, "d_topk_idx", true)) ||
        (rc = check_dev_ptr(d_topk_w, "d_topk_w", true)))
        return rc;
    if ((rc = require_loaded(ctx, layer, true))) return rc;
    if ((rc = set_device(ctx)) || (rc = refresh_pft_copy(ctx, layer))) return rc;
    uint8_t* sbase = nullptr;
    if (use_static) {
        const uint64_t need = prefill_scratch_packed(ctx->g, T);
        if (need > m1moe::kStaticScratchBytes) {
            int32_t tmax = 0;
            for (int32_t lo = 1, hi = T; lo <= hi;) {   // bytes grow with T
                const int32_t mid = lo + (hi - lo) / 2;
                if (prefill_scratch_packed(ctx->g, mid) <= m1moe::kStaticScratchBytes) {
                    tmax = mid;
                    lo = mid + 1;
                } else {
                    hi = mid - 1;
                }
            }
            return fail(M1MOE_ERR_INVALID,
                        "T=%d needs %llu bytes of static prefill scratch, more than its %llu; "
                        "at this shape T <= %d",
                        T, (unsigned long long)need,
                        (unsigned long long)m1moe::kStaticScratchBytes, tmax);
        }
        if (!ctx->static_scratch)
            return fail(M1MOE_ERR_HIP, "the static scratch of device %d is not attached",
                        ctx->device);
        sbase = ctx->static_scratch;
    } else if ((rc = ensure_prefill_scratch(ctx, T))) {
        return rc;
    }
    const m1moe::Geom& g = ctx->g;
    m1moe::PrefillArgs a{};
    a.layer_base = ctx->arena + (uint64_t)layer * g.E * g.expert_bytes;
    a.expert_bytes = g.expert_bytes;
    a.pft_base = ctx->pft + (uint64_t)layer * g.E * ctx->pft_bytes;
    a.pft_bytes = ctx->pft_bytes;
    a.x = d_x;
    a.x_bf16 = (x_dtype == M1MOE_BF16);
    a.residual = d_residual;
    a.out = d_out;
    a.idx = ctx->topk_idx;
    a.w = ctx->topk_w;
    a.T = T;
    a.h = g.h;
    a.E = g.E;
    a.K = g.K;
    a.I = g.I;
    a.gs = g.gs;
    if (sbase) {
        // carve the kPfBufs buffers, 256-byte aligned; every one is written
        // before it is read, so nothing left by an earlier call is used
        uint64_t sz[m1moe::kPfBufs];
        void* p[m1moe::kPfBufs];
        prefill_scratch_sizes(g, T, sz);
        for (int i = 0; i < m1moe::kPfBufs; ++i) {
            p[i] = sbase;
            sbase += (sz[i] + 255) / 256 * 256;
        }
        a.xq = static_cast<_Float16*>(p[0]);
        a.xinv = static_cast<float*>(p[1]);
        a.pos = static_cast<int32_t*>(p[2]);
        a.sorted_tok = static_cast<m1moe::PfPair*>(p[3]);
        a.expert_off = static_cast<int32_t*>(p[4]);
        a.tile_off = static_cast<int32_t*>(p[5]);
        a.tile_desc = static_cast<m1moe::PfTile*>(p[6]);
        a.act = static_cast<_Float16*>(p[7]);
        a.y = static_cast<float*>(p[8]);
        a.act_exp = static_cast<uint8_t*>(p[9]);
        a.act_flag = static_cast<uint32_t*>(p[10]);
    } else {
        a.xq = ctx->pf_xq;
        a.xinv = ctx->pf_xinv;
        a.pos = ctx->pf_pos;
        a.sorted_tok = ctx->pf_sorted;
        a.expert_off = ctx->pf_eoff;
        a.tile_off = ctx->pf_toff;
        a.tile_desc = ctx->pf_tdesc;
        a.act = ctx->pf_act;
        a.y = ctx->pf_y;
        a.act_exp = ctx->pf_aexp;
        a.act_flag = ctx->pf_aflag;
    }
    a.err = ctx->err;
    a.cus = ctx->cus;
    if ((rc = enqueue_router(ctx, layer, T, d_x, x_dtype, d_topk_idx, d_topk_w, nullptr, a.xq,
                             a.xinv)))
        return rc;
    return launched(m1moe::launch_prefill(a, ctx->stream),
                    use_static ? "moe_prefill_noalloc" : "moe_prefill");
}

}  // namespace

extern "C" {

int32_t m1moe_abi_version(void) { return M1MOE_ABI_VERSION; }

const char* m1moe_last_error(void) { return m1moe::g_last_error.c_str(); }

int32_t m1moe_check_shape(const m1moe_moe_shape* s) {
    if (!s) return fail(M1MOE_ERR_INVALID, "null shape");
    if (s->hidden <= 0 || s->hidden % 64 || s->hidden > 16384)
        return fail(M1MOE_ERR_INVALID, "hidden=%d must be a positive multiple of 64, <= 16384",
                    s->hidden);
    if (s->intermediate <= 0 || s->intermediate % 64 || s->intermediate > 16384)
        return fail(M1MOE_ERR_INVALID,
                    "intermediate=%d must be a positive multiple of 64, <= 16384",
                    s->intermediate);
    if (s->group_size != 32 && s->group_size != 64 && s->group_size != 128)
        return fail(M1MOE_ERR_INVALID, "group_size=%d must be 32, 64 or 128", s->group_size);
    if (s->hidden % s->group_size || s->intermediate % s->group_size)
        return fail(M1MOE_ERR_INVALID, "group_size=%d must divide hidden=%d and intermediate=%d",
                    s->group_size, s->hidden, s->intermediate);
    if (s->num_experts < 1 || s->num_experts > 256)
        return fail(M1MOE_ERR_INVALID, "num_experts=%d must be in [1, 256]", s->num_experts);
    if (s->top_k < 1 || s->top_k > s->num_experts || s->top_k > 32)
        return fail(M1MOE_ERR_INVALID, "top_k=%d must be in [1, min(num_experts, 32)]",
                    s->top_k);
    if (s->num_layers < 1)
        return fail(M1MOE_ERR_INVALID, "num_layers=%d must be >= 1", s->num_layers);
    if (s->norm_topk_prob != 0 && s->norm_topk_prob != 1)
        return fail(M1MOE_ERR_INVALID, "norm_topk_prob=%d must be 0 or 1", s->norm_topk_prob);
    return M1MOE_OK;
}

int32_t m1moe_expert_bytes(const m1moe_moe_shape* s, uint64_t* out) {
    int32_t rc = m1moe_check_shape(s);
    if (rc) return rc;
    if (!out) return fail(M1MOE_ERR_INVALID, "null output");
    *out = m1moe::make_geom(*s).expert_bytes;
    return M1MOE_OK;
}

int32_t m1moe_expert_offsets(const m1moe_moe_shape* s, uint64_t out[9]) {
    int32_t rc = m1moe_check_shape(s);
    if (rc) return rc;
    if (!out) return fail(M1MOE_ERR_INVALID, "null output");
    const m1moe::Geom g = m1moe::make_geom(*s);
    for (int k = 0; k < 9; ++k) out[k] = g.off[k];
    return M1MOE_OK;
}

int32_t m1moe_decode_kernel_for(const m1moe_moe_shape* s, int32_t cus, int32_t blocks_per_cu,
                                int32_t* kernel) {
    int32_t rc = m1moe_check_shape(s);
    if (rc) return rc;
    if (!kernel) return fail(M1MOE_ERR_INVALID, "null output");
    if (cus < 0 || blocks_per_cu < 0)
        return fail(M1MOE_ERR_INVALID, "cus=%d and blocks_per_cu=%d must be >= 0", cus,
                    blocks_per_cu);
    const bool fits = m1moe::decode_cu_fits(s->hidden, s->num_experts, s->top_k,
                                            s->intermediate, s->group_size);
    *kernel = m1moe::decode_kernel_choice(fits, s->hidden, cus, blocks_per_cu);
    return M1MOE_OK;
}

void m1moe_destroy(m1moe_ctx_t ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->lib_stream && ctx->lib_stream != ctx->stream)
        (void)hipStreamSynchronize(ctx->lib_stream);
    for (void* p : ctx->allocs) (void)hipFree(p);
    void* owned[] = {ctx->arena,   ctx->dec,      ctx->pft,      ctx->routers,  ctx->biases,  ctx->logits,  ctx->topk_idx,
                     ctx->topk_w,  ctx->counters, ctx->act,     ctx->sync,    ctx->err,
                     ctx->pf_xq,   ctx->pf_xinv,  ctx->pf_pos,  ctx->pf_sorted, ctx->pf_eoff,
                     ctx->pf_toff, ctx->pf_tdesc,  ctx->pf_act,  ctx->pf_y,     ctx->pf_aexp,
                     ctx->pf_aflag, ctx->attn_part, ctx->attn_cnt};
    for (void* p : owned)
        if (p) (void)hipFree(p);
    share_leave(ctx);
    delete ctx;
}

int32_t m1moe_create(int32_t device, const m1moe_moe_shape* s, m1moe_ctx_t* out) {
    if (!out) return fail(M1MOE_ERR_INVALID, "null output handle");
    *out = nullptr;
    int32_t rc = m1moe_check_shape(s);
    if (rc) return rc;
    int ndev = 0;
    HIP_TRY(hipGetDeviceCount(&ndev));
    if (device < 0 || device >= ndev)
        return fail(M1MOE_ERR_INVALID, "device %d out of range [0, %d)", device, ndev);
    m1moe_ctx* c = new (std::nothrow) m1moe_ctx();
    if (!c) return fail(M1MOE_ERR_OOM, "host allocation failed");
    c->device = device;
    c->shape = *s;
    c->g = m1moe::make_geom(*s);
    c->has_bias.assign(s->num_layers, false);
    c->layer_loaded.assign(s->num_layers, false);
    c->router_loaded.assign(s->num_layers, false);
    const m1moe::Geom& g = c->g;
    const uint64_t L = (uint64_t)s->num_layers, E = (uint64_t)g.E;
    auto cleanup = [&](int32_t code) {
        m1moe_destroy(c);
        return code;
    };
    if (hipSetDevice(device) != hipSuccess) return cleanup(fail(M1MOE_ERR_HIP, "hipSetDevice"));
    if ((rc = share_join(c))) return cleanup(rc);
    if (int e = m1moe::static_scratch_attach(device, &c->static_scratch))
        return cleanup(fail(M1MOE_ERR_HIP, "static scratch address of device %d: %s", device,
                            hipGetErrorString((hipError_t)e)));
    const uint64_t cap = m1moe::kPrefillCap;
    {
        // hand-off state of the fused decode kernel: kLogitRep replicas of
        // the tagged logits, kNRep replicas of n_cnt padded tile counters, one
        // launch counter per workgroup
        m1moe::FusedArgs fa{};
        fa.h = g.h;
        fa.E = g.E;
        fa.K = g.K;
        fa.I = g.I;
        const int grid = m1moe::decode_grid(fa);
        c->sync_gu_cnt = (uint64_t)m1moe::kLogitRep * m1moe::kRepStride * 8;
        c->sync_seen =
            c->sync_gu_cnt + (uint64_t)m1moe::kNRep * fa.n_cnt * m1moe::kCntStride * 4;
        c->sync_cu_seen = c->sync_seen + ((uint64_t)grid * 4 + 255) / 256 * 256;
        c->sync_cu_cnt = c->sync_cu_seen + (uint64_t)m1moe::kCuWorkgroups * 4;
        c->sync_cu_part =
            c->sync_cu_cnt + (uint64_t)m1moe::kCuRep * m1moe::kCuParts * m1moe::kCntStride * 4;
        // per-CU kernels: [256 row blocks][256 sources][8 or 16 rows] f32 partials
        c->sync_xl = c->sync_cu_part + (uint64_t)m1moe::kCuWorkgroups *
                                           m1moe::kCuWorkgroups * (g.h > 2048 ? 16 : 8) * 4;
        // per-CU kernels: XCD-local logit slots, [8][kRepStride] u64
        c->sync_bytes = c->sync_xl + (uint64_t)8 * m1moe::kRepStride * 8;
    }
    {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
            return cleanup(fail(M1MOE_ERR_HIP, "hipDeviceGetAttribute(multiprocessor count)"));
        c->cus = cus;
        // the per-CU kernels only when all of their workgroups fit on the
        // device at once (CUs x workgroups per CU, from the occupancy query)
        const bool fits = m1moe::decode_cu_fits(g.h, g.E, g.K, g.I, g.gs);
        int blocks = 0;
        if (fits && m1moe::decode_cu_blocks_per_cu(g.h, g.K, g.I, g.gs, &blocks) != 0)
            blocks = 0;
        c->decode_cu = m1moe::decode_kernel_choice(fits, g.h, cus, blocks) != 0;
        c->dec_stale.assign(s->num_layers, false);
        if (c->decode_cu) {
            c->dec_bytes = m1moe::decode_copy_bytes(g.h, g.I, g.gs);
            if ((rc = device_alloc((void**)&c->dec, L * E * c->dec_bytes, "repacked expert copy")))
                return cleanup(rc);
        }
    }
    c->pft_bytes = m1moe::PfTileLayout(g.h, g.I, g.gs).bytes;
    c->pft_stale.assign(s->num_layers, false);
    if ((rc = device_alloc((void**)&c->arena, L * E * g.expert_bytes, "expert arena")) ||
        (rc = device_alloc((void**)&c->pft, L * E * c->pft_bytes, "prefill expert copy")) ||
        (rc = device_alloc((void**)&c->routers, L * E * g.h * 2, "routers")) ||
        (rc = device_alloc((void**)&c->biases, L * E * 4, "logit biases")) ||
        (rc = device_alloc((void**)&c->logits, cap * E * 4, "logits")) ||
        (rc = device_alloc((void**)&c->topk_idx, cap * g.K * 4, "topk idx")) ||
        (rc = device_alloc((void**)&c->topk_w, cap * g.K * 4, "topk w")) ||
        (rc = device_alloc((void**)&c->counters, cap * 4, "counters")) ||
        (rc = device_alloc((void**)&c->act, (uint64_t)g.K * g.I * 4, "act")) ||
        (rc = device_alloc((void**)&c->sync, c->sync_bytes, "decode hand-off state")) ||
        (rc = device_alloc((void**)&c->err, 4, "error flag")))
        return cleanup(rc);
    // act starts with tag bits 0, which no launch (tags start at 1) takes for current
    if (hipMemset(c->act, 0, (uint64_t)g.K * g.I * 4) != hipSuccess ||
        hipMemset(c->counters, 0, cap * 4) != hipSuccess ||
        hipMemset(c->err, 0, 4) != hipSuccess || hipMemset(c->biases, 0, L * E * 4) != hipSuccess ||
        hipMemset(c->sync, 0, c->sync_bytes) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess)
        return cleanup(fail(M1MOE_ERR_HIP, "scratch initialisation failed"));
    *out = c;
    return M1MOE_OK;
}

int32_t m1moe_upload_layer_experts(m1moe_ctx_t ctx, int32_t layer, const void* host_image,
                                   uint64_t bytes) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = check_layer(ctx, layer))) return rc;
    if (!host_image) return fail(M1MOE_ERR_INVALID, "null layer image");
    const uint64_t want = (uint64_t)ctx->g.E * ctx->g.expert_bytes;
    if (bytes != want)
        return fail(M1MOE_ERR_INVALID,
                    "layer %d image is %llu bytes; num_experts * expert_bytes = %llu", layer,
                    (unsigned long long)bytes, (unsigned long long)want);
    if ((rc = set_device(ctx))) return rc;
    HIP_TRY(hipMemcpyAsync(ctx->arena + (uint64_t)layer * want, host_image, bytes,
                           hipMemcpyHostToDevice, ctx->stream));
    if (ctx->decode_cu) {
        HIP_TRY((hipError_t)m1moe::launch_decode_copy(
            ctx->arena + (uint64_t)layer * want, ctx->g.expert_bytes,
            ctx->dec + (uint64_t)layer * ctx->g.E * ctx->dec_bytes, ctx->g.E, ctx->g.h, ctx->g.I,
            ctx->g.gs,
            ctx->stream));
        ctx->dec_stale[layer] = false;
    }
    if ((rc = launch_pft_copy(ctx, layer))) return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    // the prefill copy kernel flags a non-finite group scale or bias (bit 8):
    // report it here, take the bit back, and leave the layer unloaded
    uint32_t flag = 0;
    HIP_TRY(hipMemcpy(&flag, ctx->err, 4, hipMemcpyDeviceToHost));
    if (flag & 8u) {
        const uint32_t rest = flag & ~8u;
        HIP_TRY(hipMemcpy(ctx->err, &rest, 4, hipMemcpyHostToDevice));
        ctx->layer_loaded[layer] = false;
        return fail(M1MOE_ERR_INVALID,
                    "layer %d image has a non-finite group scale or bias; the layer is not "
                    "loaded", layer);
    }
    ctx->layer_loaded[layer] = true;
    return M1MOE_OK;
}

int32_t m1moe_upload_router(m1moe_ctx_t ctx, int32_t layer, const uint16_t* host_router,
                            uint64_t count) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = check_layer(ctx, layer))) return rc;
    if (!host_router) return fail(M1MOE_ERR_INVALID, "null router");
    const uint64_t want = (uint64_t)ctx->g.E * ctx->g.h;
    if (count != want)
        return fail(M1MOE_ERR_INVALID, "router count %llu != num_experts * hidden = %llu",
                    (unsigned long long)count, (unsigned long long)want);
    if ((rc = set_device(ctx))) return rc;
    HIP_TRY(hipMemcpyAsync(ctx->routers + (uint64_t)layer * want, host_router, want * 2,
                           hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    ctx->router_loaded[layer] = true;
    return M1MOE_OK;
}

int32_t m1moe_set_logit_bias(m1moe_ctx_t ctx, int32_t layer, const float* host_bias,
                             int32_t count) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = check_layer(ctx, layer))) return rc;
    if (!host_bias) {
        ctx->has_bias[layer] = false;
        return M1MOE_OK;
    }
    if (count != ctx->g.E)
        return fail(M1MOE_ERR_INVALID, "bias count %d != num_experts %d", count, ctx->g.E);
    if ((rc = set_device(ctx))) return rc;
    HIP_TRY(hipMemcpyAsync(ctx->biases + (uint64_t)layer * ctx->g.E, host_bias,
                           (uint64_t)count * 4, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    ctx->has_bias[layer] = true;
    return M1MOE_OK;
}

int32_t m1moe_expert_block(m1moe_ctx_t ctx, int32_t layer, int32_t expert, void** dev_ptr) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = check_layer(ctx, layer))) return rc;
    if (expert < 0 || expert >= ctx->g.E)
        return fail(M1MOE_ERR_INVALID, "expert %d out of range [0, %d)", expert, ctx->g.E);
    if (!dev_ptr) return fail(M1MOE_ERR_INVALID, "null output");
    *dev_ptr = ctx->arena + ((uint64_t)layer * ctx->g.E + (uint64_t)expert) * ctx->g.expert_bytes;
    if (ctx->decode_cu) ctx->dec_stale[layer] = true;  // the caller may write the block
    ctx->pft_stale[layer] = true;
    return M1MOE_OK;
}

int32_t m1moe_alloc(m1moe_ctx_t ctx, uint64_t bytes, void** dev_ptr) {
    int32_t rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!dev_ptr) return fail(M1MOE_ERR_INVALID, "null output");
    if ((rc = set_device(ctx))) return rc;
    if ((rc = device_alloc(dev_ptr, bytes, "m1moe_alloc"))) return rc;
    ctx->allocs.insert(*dev_ptr);
    return M1MOE_OK;
}

int32_t m1moe_free(m1moe_ctx_t ctx, void* dev_ptr) {
    int32_t rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!dev_ptr) return M1MOE_OK;
    auto it = ctx->allocs.find(dev_ptr);
    if (it == ctx->allocs.end())
        return fail(M1MOE_ERR_INVALID, "pointer was not allocated by m1moe_alloc on this context");
    if ((rc = set_device(ctx))) return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    HIP_TRY(hipFree(dev_ptr));
    ctx->allocs.erase(it);
    return M1MOE_OK;
}

static int32_t copy_common(m1moe_ctx_t ctx, void* dst, const void* src, uint64_t bytes,
                           hipMemcpyKind kind) {
    int32_t rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (bytes == 0) return M1MOE_OK;
    if (!dst || !src) return fail(M1MOE_ERR_INVALID, "null copy pointer");
    if ((rc = set_device(ctx))) return rc;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, kind, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return M1MOE_OK;
}

int32_t m1moe_copy_h2d(m1moe_ctx_t ctx, void* d, const void* h, uint64_t n) {
    return copy_common(ctx, d, h, n, hipMemcpyHostToDevice);
}
int32_t m1moe_copy_d2h(m1moe_ctx_t ctx, void* h, const void* d, uint64_t n) {
    return copy_common(ctx, h, d, n, hipMemcpyDeviceToHost);
}
int32_t m1moe_copy_d2d(m1moe_ctx_t ctx, void* d, const void* s, uint64_t n) {
    return copy_common(ctx, d, s, n, hipMemcpyDeviceToDevice);
}

int32_t m1moe_set_stream(m1moe_ctx_t ctx, void* hip_stream) {
    int32_t rc;
    if ((rc = check_ctx(ctx))) return rc;
    std::lock_guard<std::mutex> lk(g_share_mu);
    DeviceShare& d = g_share[ctx->device];
    if (hip_stream && d.users > 1)
        return fail(M1MOE_ERR_INVALID,
                    "%d contexts share device %d and its one stream; a caller stream is accepted "
                    "only while a context is the device's only one", d.users, ctx->device);
    ctx->stream = hip_stream ? static_cast<hipStream_t>(hip_stream) : ctx->lib_stream;
    d.on_caller_stream = hip_stream ? ctx : nullptr;
    return M1MOE_OK;
}

int32_t m1moe_get_stream(m1moe_ctx_t ctx, void** hip_stream) {
    int32_t rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!hip_stream) return fail(M1MOE_ERR_INVALID, "null output");
    *hip_stream = ctx->stream;
    return M1MOE_OK;
}

int32_t m1moe_sync(m1moe_ctx_t ctx) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = set_device(ctx))) return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    uint32_t flag = 0;
    HIP_TRY(hipMemcpy(&flag, ctx->err, 4, hipMemcpyDeviceToHost));
    if (flag) {
        // a failed launch leaves the workgroups' launch counters out of step:
        // restart them all from zero
        HIP_TRY(hipMemset(ctx->err, 0, 4));
        HIP_TRY(hipMemset(ctx->sync, 0, ctx->sync_bytes));
        HIP_TRY(hipMemset(ctx->act, 0, (uint64_t)ctx->g.K * ctx->g.I * 4));
        HIP_TRY(hipDeviceSynchronize());
        if (flag & 1u)
            return fail(M1MOE_ERR_DEVICE,
                        "a kernel saw an expert index outside [0, %d) (device flag 0x%x)",
                        ctx->g.E, flag);
        if (flag & 8u)
            return fail(M1MOE_ERR_DEVICE,
                        "an uploaded expert block has a non-finite group scale or bias (device "
                        "flag 0x%x)", flag);
        if (flag & 16u)
            return fail(M1MOE_ERR_DEVICE,
                        "a decoder step read a token id outside the vocabulary; token 0 was "
                        "embedded (device flag 0x%x)", flag);
        if (flag & 64u)
            return fail(M1MOE_ERR_DEVICE,
                        "a prefill's SwiGLU product was not finite; it was clamped to +-65504 "
                        "(device flag 0x%x)", flag);
        if (flag & 128u)
            return fail(M1MOE_ERR_DEVICE,
                        "a prefill's down GEMM timed out waiting for its workgroups (another "
                        "kernel held compute units); the layer output is not valid (device flag "
                        "0x%x)", flag);
        if (flag & 32u)
            return fail(M1MOE_ERR_DEVICE,
                        "a decoder step ran with the KV cache full (position == max_seq); "
                        "nothing was stored (device flag 0x%x)", flag);
        return fail(M1MOE_ERR_DEVICE,
                    "a decode hand-off wait timed out (device flag 0x%x); state was reset", flag);
    }
    return M1MOE_OK;
}

int32_t m1moe_event_create(m1moe_ctx_t ctx, m1moe_event_t* out) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = set_device(ctx))) return rc;
    if (!out) return fail(M1MOE_ERR_INVALID, "null output");
    m1moe_event* e = new (std::nothrow) m1moe_event();
    if (!e) return fail(M1MOE_ERR_OOM, "host allocation failed");
    if (hipEventCreate(&e->ev) != hipSuccess) {
        delete e;
        return fail(M1MOE_ERR_HIP, "hipEventCreate failed");
    }
    *out = e;
    return M1MOE_OK;
}

int32_t m1moe_event_record(m1moe_ctx_t ctx, m1moe_event_t ev) {
    int32_t rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!ev) return fail(M1MOE_ERR_INVALID, "null event");
    HIP_TRY(hipEventRecord(ev->ev, ctx->stream));
    return M1MOE_OK;
}

int32_t m1moe_event_elapsed_ms(m1moe_event_t start, m1moe_event_t end, float* ms) {
    if (!start || !end || !ms) return fail(M1MOE_ERR_INVALID, "null argument");
    HIP_TRY(hipEventSynchronize(end->ev));
    HIP_TRY(hipEventElapsedTime(ms, start->ev, end->ev));
    return M1MOE_OK;
}

void m1moe_event_destroy(m1moe_event_t ev) {
    if (!ev) return;
    (void)hipEventDestroy(ev->ev);
    delete ev;
}

int32_t m1moe_graph_begin(m1moe_ctx_t ctx) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = set_device(ctx))) return rc;
    HIP_TRY(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capture_uses_scratch = false;
    return M1MOE_OK;
}

int32_t m1moe_graph_end(m1moe_ctx_t ctx, m1moe_graph_t* out) {
    int32_t rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!out) return fail(M1MOE_ERR_INVALID, "null output");
    m1moe_graph* gr = new (std::nothrow) m1moe_graph();
    if (!gr) return fail(M1MOE_ERR_OOM, "host allocation failed");
    hipError_t e = hipStreamEndCapture(ctx->stream, &gr->graph);
    if (e != hipSuccess) {
        delete gr;
        return fail(M1MOE_ERR_HIP, "hipStreamEndCapture failed: %s", hipGetErrorString(e));
    }
    e = hipGraphInstantiate(&gr->exec, gr->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(gr->graph);
        delete gr;
        return fail(M1MOE_ERR_HIP, "hipGraphInstantiate failed: %s", hipGetErrorString(e));
    }
    gr->owner = ctx;
    gr->scratch_gen = ctx->scratch_gen;
    gr->uses_scratch = ctx->capture_uses_scratch;
    *out = gr;
    return M1MOE_OK;
}

int32_t m1moe_graph_launch(m1moe_ctx_t ctx, m1moe_graph_t graph) {
    int32_t rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!graph) return fail(M1MOE_ERR_INVALID, "null graph");
    if (graph->owner != ctx)
        return fail(M1MOE_ERR_INVALID, "the graph was captured on another context");
    if (graph->uses_scratch && graph->scratch_gen != ctx->scratch_gen)
        return fail(M1MOE_ERR_INVALID,
                    "a scratch buffer was reallocated (a call with a larger size) since the "
                    "graph was captured, so it holds freed addresses; capture it again");
    HIP_TRY(hipGraphLaunch(graph->exec, ctx->stream));
    return M1MOE_OK;
}

void m1moe_graph_destroy(m1moe_graph_t graph) {
    if (!graph) return;
    (void)hipGraphExecDestroy(graph->exec);
    (void)hipGraphDestroy(graph->graph);
    delete graph;
}

int32_t m1moe_router_topk(m1moe_ctx_t ctx, int32_t layer, int32_t T, const void* d_x,
                          int32_t x_dtype, int32_t* d_topk_idx, float* d_topk_w,
                          float* d_logits) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = check_layer(ctx, layer))) return rc;
    if (T < 1 || T > m1moe::kPrefillCap)
        return fail(M1MOE_ERR_INVALID, "T=%d must be in [1, %d]", T, m1moe::kPrefillCap);
    if ((rc = check_dtype(x_dtype)) || (rc = check_dev_ptr(d_x, "d_x", false)) ||
        (rc = check_dev_ptr(d_topk_idx, "d_topk_idx", false)) ||
        (rc = check_dev_ptr(d_topk_w, "d_topk_w", false)) ||
        (rc = check_dev_ptr(d_logits, "d_logits", true)))
        return rc;
    if (!ctx->router_loaded[layer])
        return fail(M1MOE_ERR_INVALID, "layer %d router was never uploaded", layer);
    if ((rc = set_device(ctx))) return rc;
    return enqueue_router(ctx, layer, T, d_x, x_dtype, d_topk_idx, d_topk_w, d_logits);
}

int32_t m1moe_moe_decode_given_topk(m1moe_ctx_t ctx, int32_t layer, const void* d_x,
                                    int32_t x_dtype, const int32_t* d_topk_idx,
                                    const float* d_topk_w, const float* d_residual,
                                    float* d_out) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = check_layer(ctx, layer))) return rc;
    if ((rc = check_dtype(x_dtype)) || (rc = check_dev_ptr(d_x, "d_x", false)) ||
        (rc = check_dev_ptr(d_topk_idx, "d_topk_idx", false)) ||
        (rc = check_dev_ptr(d_topk_w, "d_topk_w", false)) ||
        (rc = check_dev_ptr(d_residual, "d_residual", true)) ||
        (rc = check_dev_ptr(d_out, "d_out", false)))
        return rc;
    if ((rc = require_loaded(ctx, layer, false))) return rc;
    if ((rc = set_device(ctx)) || (rc = refresh_decode_copy(ctx, layer))) return rc;
    m1moe::FusedArgs a = fused_args(ctx, layer, d_x, x_dtype, d_residual, d_out);
    a.given_idx = d_topk_idx;
    a.given_w = d_topk_w;
    return launched(enqueue_decode(ctx, a), "moe_decode (given routing)");
}

int32_t m1moe_moe_decode(m1moe_ctx_t ctx, int32_t layer, const void* d_x, int32_t x_dtype,
                         const float* d_residual, float* d_out, int32_t* d_topk_idx,
                         float* d_topk_w) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = check_layer(ctx, layer))) return rc;
    if ((rc = check_dtype(x_dtype)) || (rc = check_dev_ptr(d_x, "d_x", false)) ||
        (rc = check_dev_ptr(d_residual, "d_residual", true)) ||
        (rc = check_dev_ptr(d_out, "d_out", false)) ||
        (rc = check_dev_ptr(d_topk_idx, "d_topk_idx", true)) ||
        (rc = check_dev_ptr(d_topk_w, "d_topk_w", true)))
        return rc;
    if ((rc = require_loaded(ctx, layer, true))) return rc;
    if ((rc = set_device(ctx)) || (rc = refresh_decode_copy(ctx, layer))) return rc;
    m1moe::FusedArgs a = fused_args(ctx, layer, d_x, x_dtype, d_residual, d_out);
    a.user_idx = d_topk_idx;
    a.user_w = d_topk_w;
    return launched(enqueue_decode(ctx, a), "moe_decode");
}

}  // extern "C"

namespace m1moe {
int32_t moe_decode_normed(m1moe_ctx_t ctx, int32_t layer, const float* d_x, const float* d_ssq,
                          int32_t n_ssq, const uint16_t* d_norm_w, float eps,
                          const float* d_residual, float* d_out) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = check_layer(ctx, layer))) return rc;
    if ((rc = require_loaded(ctx, layer, true))) return rc;
    if ((rc = set_device(ctx)) || (rc = refresh_decode_copy(ctx, layer))) return rc;
    m1moe::FusedArgs a = fused_args(ctx, layer, d_x, M1MOE_F32, d_residual, d_out);
    a.x_ssq = d_ssq;
    a.n_ssq = n_ssq;
    a.x_norm_w = d_norm_w;
    a.x_eps = eps;
    return launched(enqueue_decode(ctx, a), "moe_decode (normed input)");
}
}  // namespace m1moe

extern "C" {

int32_t m1moe_moe_prefill(m1moe_ctx_t ctx, int32_t layer, int32_t T, const void* d_x,
                          int32_t x_dtype, const float* d_residual, float* d_out,
                          int32_t* d_topk_idx, float* d_topk_w) {
    return prefill_common(ctx, layer, T, d_x, x_dtype, d_residual, d_out, d_topk_idx, d_topk_w,
                          false);
}

int32_t m1moe_moe_prefill_noalloc(m1moe_ctx_t ctx, int32_t layer, int32_t T, const void* d_x,
                                  int32_t x_dtype, const float* d_residual, float* d_out,
                                  int32_t* d_topk_idx, float* d_topk_w) {
    return prefill_common(ctx, layer, T, d_x, x_dtype, d_residual, d_out, d_topk_idx, d_topk_w,
                          true);
}

int32_t m1moe_dequant_debug(m1moe_ctx_t ctx, int32_t layer, int32_t expert, int32_t proj,
                            float* d_out) {
    int32_t rc;
    if ((rc = check_ctx(ctx)) || (rc = check_layer(ctx, layer))) return rc;
    if (expert < 0 || expert >= ctx->g.E)
        return fail(M1MOE_ERR_INVALID, "expert %d out of range [0, %d)", expert, ctx->g.E);
    if (proj < 0 || proj > 2) return fail(M1MOE_ERR_INVALID, "proj %d must be 0, 1 or 2", proj);
    if ((rc = check_dev_ptr(d_out, "d_out", false))) return rc;
    if ((rc = require_loaded(ctx, layer, false))) return rc;
    if ((rc = set_device(ctx))) return rc;
    const m1moe::Geom& g = ctx->g;
    const uint8_t* blk = ctx->arena + ((uint64_t)layer * g.E + (uint64_t)expert) * g.expert_bytes;
    const m1moe::ProjView p = {g.off[3 * proj], g.off[3 * proj + 1], g.off[3 * proj + 2],
                               g.rows(proj), g.cols(proj)};
    return launched(m1moe::launch_dequant(blk, p, g.gs, d_out, ctx->stream), "dequant");
}

}  // extern "C"
