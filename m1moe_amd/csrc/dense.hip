// dense.hip — the dense part of a decoder step on the GPU.
//
// The reference runs these on Metal one threadgroup per row or per dot
// product (Shaders.metal:96-358) and the q/k norms, RoPE and the KV store on
// the CPU between syncs (InferenceEngine.swift:194-228, 521-548).  Here a
// layer is four launches, the MoE block's included:
//
//   matvec_kernel  y = W x over up to three weight segments (q, k, v share
//                  the input).  The input is staged in LDS once per
//                  workgroup, RMS-normalised there (the layer's input norm,
//                  the final norm) or taken from the embedding table at the
//                  step's token.  o_proj also stores per-workgroup sums of
//                  squares of its output, from which the MoE kernel applies
//                  the post-attention RMSNorm to its input; lm_head's last
//                  workgroup to finish takes the greedy argmax (and advances
//                  the device-side position).
//   attn_kernel    one workgroup per (kv head, 64 positions): the per-head
//                  q/k RMSNorm and RoPE of the current token, its K/V row
//                  stored, scores, a chunk softmax and the weighted V sum;
//                  the last workgroup of each kv head merges the chunks (the
//                  reference's softmax, computed in pieces)
//   rmsnorm_kernel, argmax_kernel   the standalone building blocks
//
// Cross-workgroup results (attention partials, per-workgroup maxima) are
// written with agent-scope (coherent) stores; every thread waits
// for its stores to complete, then after a barrier thread 0 counts the
// workgroup in with a relaxed agent-scope add (a release fence instead would
// write back the whole L2 once per workgroup).  The last workgroup reads
// the results with coherent loads, issued in batches, and puts the counter
// back to 0, so a captured graph can replay the kernels.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>

#include "device.hpp"
#include "internal.hpp"

namespace m1moe {
namespace {

// Sum over a workgroup of `nw` waves; every thread gets the result (waves
// combined in order).
__device__ __forceinline__ float block_sum(float v, float* s_red, int nw) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    v = wave_sum(v);
    if (lane == 0) s_red[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int w = 0; w < nw; ++w) t += s_red[w];
    __syncthreads();
    return t;
}

__device__ __forceinline__ void st_coh(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh(int32_t* p, int32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coh(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_coh(const int32_t* p) {
    return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// True in the workgroup that finishes last of `total` (counter: one word).
// Every thread's coherent stores have completed before the barrier, so they
// are visible to coherent loads once the counter shows the workgroup.
__device__ __forceinline__ bool last_workgroup(uint32_t* counter, uint32_t total, int* s_flag) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t old =
            __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *s_flag = old == total - 1;
    }
    __syncthreads();
    return *s_flag != 0;
}
__device__ __forceinline__ void reset_counter(uint32_t* c) {
    __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Counts workgroup b of `total` out (one thread); true for the last one.
// Above 64 workgroups in two levels: b counts on part b % 8 (words 32 x),
// the last of each part on word 256 (kCountWords words in all), so that no
// address takes more than total / 8 counts (one address taking every
// workgroup's count serialises them: ~1 us at 264 workgroups).  Each counter
// is put back to 0 by its last count.
__device__ __forceinline__ bool count_out(uint32_t* c, uint32_t total, uint32_t b) {
    const uint32_t np = total > 64u ? 8u : 1u, x = b % np, per = (total + np - 1u - x) / np;
    if (__hip_atomic_fetch_add(c + 32 * x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) !=
        per - 1u)
        return false;
    reset_counter(c + 32 * x);
    if (np == 1u) return true;
    if (__hip_atomic_fetch_add(c + 256, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != np - 1u)
        return false;
    reset_counter(c + 256);
    return true;
}

// last_workgroup over a kCountWords counter (count_out), workgroup blockIdx.x
// of a one-dimensional grid.
__device__ __forceinline__ bool last_workgroup_wide(uint32_t* counter, uint32_t total, int* s_flag) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) *s_flag = count_out(counter, total, blockIdx.x) ? 1 : 0;
    __syncthreads();
    return *s_flag != 0;
}

// (value, index) pairs: the larger value wins, ties to the lower index; NaN
// never wins.
__device__ __forceinline__ bool am_better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

// ---- RMSNorm (standalone) ------------------------------------------------------------

// Shaders.metal:96-134: the sum of squares in f32, rms = rsqrt(ss / n + eps),
// out = x * rms * w.
__global__ __launch_bounds__(1024) void rmsnorm_kernel(const float* x, const uint16_t* w,
                                                       float* out, int n, float eps) {
    __shared__ float s_red[16];
    float acc = 0.f;
    for (int i = threadIdx.x; i < n; i += 1024) {
        const float v = x[i];
        acc = fmaf(v, v, acc);
    }
    const float ss = block_sum(acc, s_red, 16);
    const float rms = rsqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 1024) out[i] = x[i] * rms * bf16_to_f32(w[i]);
}

// ---- bf16 matvec ----------------------------------------------------------------------

// Row `row` of the concatenated segments: its weight row, output and
// residual slots.  Fields are picked with constant indices (a reference into
// the argument array with a computed index would copy it to scratch).
struct RowRef {
    const uint16_t* w;
    float* y;
    const float* res;
};
__device__ __forceinline__ RowRef mv_row(const MvArgs& a, int row) {
    const int e0 = a.seg[0].rows, e1 = e0 + a.seg[1].rows;
    RowRef r;
    int loc;
    if (row < e0) {
        loc = row;
        r.w = a.seg[0].w, r.y = a.seg[0].y, r.res = a.seg[0].res;
    } else if (row < e1) {
        loc = row - e0;
        r.w = a.seg[1].w, r.y = a.seg[1].y, r.res = a.seg[1].res;
    } else {
        loc = row - e1;
        r.w = a.seg[2].w, r.y = a.seg[2].y, r.res = a.seg[2].res;
    }
    r.w += (size_t)loc * a.cols;
    r.y += loc;
    if (r.res) r.res += loc;
    return r;
}

// Stages the input in LDS: x, or the embedding row of the step's token
// (InferenceEngine.swift:482-488), then (norm_w) RMS-normalised
// (Shaders.metal:96-134).  Workgroup 0 stores the un-normalised input to
// x_copy.
// Active chunks of a fused decode-attention launch at position p if it
// leaves their merge to the next launch, else 0 (one chunk: the attention
// launch writes the output itself; many: the merge stays there, where the
// partials are read once per kv head rather than once per matvec workgroup).
// The attention launch and the matvec that stages its output both decide
// with this function.
__device__ __forceinline__ int attn_defer_nact(int p, int max_seq, int chunk, int num_heads) {
    const int seq = p < max_seq ? p + 1 : max_seq;
    const int nact = (seq + chunk - 1) / chunk;
    return (nact > 1 && nact <= kAttnDeferChunks && nact * num_heads <= kAttnDeferHeadChunks)
               ? nact
               : 0;
}

// x[h * hd + d] of the deferred attention merge: per head M = max_c m_c,
// x = sum_c acc_c[d] e^(m_c - M) / sum_c l_c e^(m_c - M) (chunks in order),
// over the partials [groups][chunks][qh][hd + 2] of the attention launch.
// Each thread takes 4 consecutive elements (one head); all of its loads are
// issued before they are used.
__device__ float mv_stage_attn(const MvArgs& a, int nact, float* s_x) {
    const int n4 = a.cols >> 2;
    const int hs = a.attn_hd + 2;
    const size_t cstride = (size_t)a.attn_qh * hs;
    float ss = 0.f;
    for (int i4 = threadIdx.x; i4 < n4; i4 += 256) {
        const int i = 4 * i4, h = i / a.attn_hd, d = i - h * a.attn_hd;
        const int g = h / a.attn_qh, hq = h - g * a.attn_qh;
        const float* base = a.attn_part + (size_t)g * a.attn_nch * cstride + (size_t)hq * hs;
        float m[kAttnDeferChunks], l[kAttnDeferChunks], v[kAttnDeferChunks][4];
#pragma unroll
        for (int c = 0; c < kAttnDeferChunks; ++c) {
            if (c >= nact) break;  // (nact is uniform)
            const float* pc = base + (size_t)c * cstride;
            m[c] = pc[0];
            l[c] = pc[1];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[c][e] = pc[2 + d + e];
        }
        float M = -INFINITY;
#pragma unroll
        for (int c = 0; c < kAttnDeferChunks; ++c)
            if (c < nact) M = fmaxf(M, m[c]);
        float L = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < kAttnDeferChunks; ++c) {
            if (c >= nact) break;
            const float f = expf(m[c] - M);
            L = fmaf(l[c], f, L);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] = fmaf(v[c][e], f, acc[e]);
        }
        const float4 o = {acc[0] / L, acc[1] / L, acc[2] / L, acc[3] / L};
        reinterpret_cast<float4*>(s_x)[i4] = o;
        ss += o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w;
    }
    return ss;
}

__device__ void mv_stage(const MvArgs& a, float* s_x, float* s_red) {
    const int n4 = a.cols >> 2;
    float ss = 0.f;
    if (a.embed) {
        int t;
        if (a.seq_cap > 0) {
            const int p = *a.pos;
            t = p < a.seq_cap ? a.token[p] : -1;
        } else {
            t = *a.token;
        }
        if (t < 0 || t >= a.vocab) {
            if (blockIdx.x == 0 && threadIdx.x == 0) flag_error(a.err, 16u);
            t = 0;
        }
        const uint2* row = reinterpret_cast<const uint2*>(a.embed + (size_t)t * a.cols);
        for (int i = threadIdx.x; i < n4; i += 256) {
            const uint2 b = row[i];
            const float4 v = {bf16_to_f32(b.x & 0xFFFFu), bf16_to_f32(b.x >> 16),
                              bf16_to_f32(b.y & 0xFFFFu), bf16_to_f32(b.y >> 16)};
            reinterpret_cast<float4*>(s_x)[i] = v;
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
    } else if (a.attn_part &&
               attn_defer_nact(*a.pos, a.max_seq, a.attn_chunk, a.attn_heads) > 0) {
        ss = mv_stage_attn(a, attn_defer_nact(*a.pos, a.max_seq, a.attn_chunk, a.attn_heads),
                           s_x);
    } else {
        const float4* x4 = reinterpret_cast<const float4*>(a.x);
        for (int i = threadIdx.x; i < n4; i += 256) {
            const float4 v = x4[i];
            reinterpret_cast<float4*>(s_x)[i] = v;
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
    }
    if (a.x_copy && blockIdx.x == 0) {
        // each thread copies the elements it staged itself
        for (int i = threadIdx.x; i < n4; i += 256)
            reinterpret_cast<float4*>(a.x_copy)[i] = reinterpret_cast<const float4*>(s_x)[i];
    }
    if (a.norm_w) {
        const float tot = block_sum(ss, s_red, 4);
        const float rms = rsqrtf(tot / (float)a.cols + a.eps);
        const uint2* w = reinterpret_cast<const uint2*>(a.norm_w);
        for (int i = threadIdx.x; i < n4; i += 256) {
            const uint2 b = w[i];
            float4 v = reinterpret_cast<float4*>(s_x)[i];
            v.x = v.x * rms * bf16_to_f32(b.x & 0xFFFFu);
            v.y = v.y * rms * bf16_to_f32(b.x >> 16);
            v.z = v.z * rms * bf16_to_f32(b.y & 0xFFFFu);
            v.w = v.w * rms * bf16_to_f32(b.y >> 16);
            reinterpret_cast<float4*>(s_x)[i] = v;
        }
    }
    __syncthreads();
}

// mv_stage for an input x of at most 1024 XF floats whose loads (x and the
// norm weights: XF float4 / uint2 per thread) were issued before the weight
// rows': the same arithmetic in the same order as mv_stage.
template <int XF>
__device__ void mv_stage_early(const MvArgs& a, float* s_x, float* s_red, const float4 (&xv)[XF],
                               const uint2 (&nw)[XF]) {
    const int n4 = a.cols >> 2;
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < XF; ++k) {
        const float4 v = xv[k];
        if (threadIdx.x + 256 * k < n4) ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    if (a.x_copy && blockIdx.x == 0) {
#pragma unroll
        for (int k = 0; k < XF; ++k) {
            const int i = threadIdx.x + 256 * k;
            if (i < n4) reinterpret_cast<float4*>(a.x_copy)[i] = xv[k];
        }
    }
    float rms = 1.f;
    if (a.norm_w) rms = rsqrtf(block_sum(ss, s_red, 4) / (float)a.cols + a.eps);
#pragma unroll
    for (int k = 0; k < XF; ++k) {
        const int i = threadIdx.x + 256 * k;
        if (i >= n4) continue;
        float4 v = xv[k];
        if (a.norm_w) {
            const uint2 b = nw[k];
            v.x = v.x * rms * bf16_to_f32(b.x & 0xFFFFu);
            v.y = v.y * rms * bf16_to_f32(b.x >> 16);
            v.z = v.z * rms * bf16_to_f32(b.y & 0xFFFFu);
            v.w = v.w * rms * bf16_to_f32(b.y >> 16);
        }
        reinterpret_cast<float4*>(s_x)[i] = v;
    }
    __syncthreads();
}

// Workgroup = 4 waves x RPW rows.  Lane l takes columns 8l .. 8l+7 of each
// 512-column block; U blocks of every row are loaded per group, the next
// group's loads issued before the current one is used.  The first group is
// in flight while the input is staged.  XF > 0 (inputs of at most 1024 XF
// floats): the input x, its norm weights and the rows' residuals are
// requested before the weight rows, so that the input is staged as soon as
// they land (the loads complete in order) while the weights stream, and the
// residual is no round trip at the end.
template <int RPW, bool STAGE, int XF>
__global__ __launch_bounds__(256) void matvec_kernel(MvArgs a) {
    constexpr int U = 8 / RPW;
    extern __shared__ __attribute__((aligned(16))) float s_x[];
    __shared__ float s_red[4];
    __shared__ float s_bv[4];
    __shared__ int s_bi[4];
    __shared__ int s_flag;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r0 = (blockIdx.x * 4 + wave) * RPW;
    // (XF: the embedded input of layer 0 waits for its token and takes the
    // staging below; x is requested anyway when the staging turns out to be
    // the deferred attention merge, whose output buffer it is)
    constexpr int XN = XF > 0 ? XF : 1;
    const bool early = STAGE && XF > 0 && !a.embed;
    float4 xv[XN];
    uint2 nwv[XN];
    if (early) {
#pragma unroll
        for (int k = 0; k < XN; ++k) {
            const int i = threadIdx.x + 256 * k;
            xv[k] = i < (a.cols >> 2) ? reinterpret_cast<const float4*>(a.x)[i] : float4{0.f, 0.f, 0.f, 0.f};
            nwv[k] = (a.norm_w && i < (a.cols >> 2)) ? reinterpret_cast<const uint2*>(a.norm_w)[i]
                                                     : uint2{0u, 0u};
        }
    }
    float resv[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        resv[i] = 0.f;
        if (r0 + i < a.rows) {
            const RowRef rr = mv_row(a, r0 + i);
            if (rr.res) resv[i] = *rr.res;
        }
    }
    const uint16_t* wr[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) wr[i] = mv_row(a, min(r0 + i, a.rows - 1)).w;
    const int ngroups = (a.cols + 512 * U - 1) / (512 * U);
    uint4 cur[U][RPW], nxt[U][RPW];
    auto load = [&](int gi, uint4 (&dst)[U][RPW]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = min(gi * 512 * U + 512 * u + 8 * lane, a.cols - 8);
#pragma unroll
            for (int i = 0; i < RPW; ++i) dst[u][i] = *reinterpret_cast<const uint4*>(wr[i] + c);
        }
    };
    // two groups in flight from the start (both before the input is staged),
    // each refilled as soon as it is used
    load(0, cur);
    if (ngroups > 1) load(1, nxt);
    if (STAGE) {
        if (early && !(a.attn_part &&
                       attn_defer_nact(*a.pos, a.max_seq, a.attn_chunk, a.attn_heads) > 0))
            mv_stage_early<XN>(a, s_x, s_red, xv, nwv);
        else
            mv_stage(a, s_x, s_red);
    }
    float acc[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) acc[i] = 0.f;
    auto use = [&](int gi, const uint4 (&buf)[U][RPW]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = gi * 512 * U + 512 * u + 8 * lane;
            if (c >= a.cols) continue;
            float4 x0, x1;
            if (STAGE) {
                x0 = *reinterpret_cast<const float4*>(s_x + c);
                x1 = *reinterpret_cast<const float4*>(s_x + c + 4);
            } else {
                x0 = *reinterpret_cast<const float4*>(a.x + c);
                x1 = *reinterpret_cast<const float4*>(a.x + c + 4);
            }
            const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int i = 0; i < RPW; ++i)
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[i] = fmaf(bf16x8_at(buf[u][i], k), xs[k], acc[i]);
        }
    };
    for (int gi = 0; gi < ngroups; gi += 2) {
        use(gi, cur);
        if (gi + 2 < ngroups) load(gi + 2, cur);
        if (gi + 1 < ngroups) {
            use(gi + 1, nxt);
            if (gi + 3 < ngroups) load(gi + 3, nxt);
        }
    }
    float bv = -INFINITY, ssq = 0.f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const float v = wave_sum(acc[i]);
        const int row = r0 + i;
        if (row < a.rows) {
            const RowRef rr = mv_row(a, row);
            const float y = rr.res ? resv[i] + v : v;
            if (lane == 0) {
                if (a.counter)
                    st_coh(rr.y, y);  // the last workgroup reads it
                else
                    *rr.y = y;
            }
            ssq = fmaf(y, y, ssq);
            if (am_better(y, row, bv, bi)) {
                bv = y;
                bi = row;
            }
        }
    }
    if (a.ssq_out) {
        if (lane == 0) s_red[wave] = ssq;
        __syncthreads();
        if (threadIdx.x == 0)
            a.ssq_out[blockIdx.x] = ((s_red[0] + s_red[1]) + s_red[2]) + s_red[3];
    }
    if (!a.counter) return;

    {
        // this workgroup's best row, then the last workgroup's reduction
        if (lane == 0) {
            s_bv[wave] = bv;
            s_bi[wave] = bi;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int w = 1; w < 4; ++w)
                if (am_better(s_bv[w], s_bi[w], bv, bi)) {
                    bv = s_bv[w];
                    bi = s_bi[w];
                }
            st_coh(a.am_val + blockIdx.x, bv);
            st_coh(a.am_idx + blockIdx.x, bi);
        }
        if (!last_workgroup_wide(a.counter, gridDim.x, &s_flag)) return;
        bv = -INFINITY;
        bi = 0x7fffffff;
        const int nwg = (int)gridDim.x;
        for (int w0 = 0; w0 < nwg; w0 += 256 * 16) {
            float vv[16];
            int ii[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int w = w0 + threadIdx.x + 256 * j;
                vv[j] = w < nwg ? ld_coh(a.am_val + w) : -INFINITY;
                ii[j] = w < nwg ? ld_coh(a.am_idx + w) : 0x7fffffff;
            }
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (am_better(vv[j], ii[j], bv, bi)) {
                    bv = vv[j];
                    bi = ii[j];
                }
        }
        wave_argmax(bv, bi);
        if (lane == 0) {
            s_bv[wave] = bv;
            s_bi[wave] = bi;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int w = 1; w < 4; ++w)
                if (am_better(s_bv[w], s_bi[w], bv, bi)) {
                    bv = s_bv[w];
                    bi = s_bi[w];
                }
            // the reference's scan starts from y[0] with a strict > (its
            // sampleToken, InferenceEngine.swift:550-555): a NaN there is
            // never replaced; all NaN also gives 0
            const int n = a.seg[0].rows;
            const int best = (bi < n && !__builtin_isnan(ld_coh(a.seg[0].y))) ? bi : 0;
            const int p = *a.pos;
            if (a.seq_cap > 0) {
                if (p + 1 >= a.n_prompt && p + 1 < a.seq_cap) a.tok_out[p + 1] = best;
            } else {
                *a.tok_out = best;
            }
            if (p < a.max_seq) *a.pos = p + 1;
        }
        return;
    }
}

// ---- attention --------------------------------------------------------------------------

// Sum over aligned groups of LP lanes (8, 16 or 32), the total in every lane
// of the group: quad sums on DPP quad permutes, then the half-row mirror
// (LP 8) or two row rotations (LP 16, 32), then the neighbouring row by a
// row swap (LP 32).  No LDS crossbar round trips.
__device__ __forceinline__ float rows_pair_sum(float v) {  // rows 0+1 and 2+3
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float halves_sum(float v) {  // lanes l and l ^ 32
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
template <int LP>
__device__ __forceinline__ float lane_group_sum(float v) {
    static_assert(LP == 8 || LP == 16 || LP == 32, "8, 16 or 32 lanes");
    v += dpp_f32<kDppXor1>(v, v);
    v += dpp_f32<kDppXor2>(v, v);
    if (LP == 8) {
        v += dpp_f32<0x141>(v, v);  // row_half_mirror: the other quad of the 8
    } else {
        v += dpp_f32<kDppRor4>(v, v);
        v += dpp_f32<kDppRor8>(v, v);
        if (LP == 32) v = rows_pair_sum(v);
    }
    return v;
}
// Sum of the lanes l, l ^ LP, l ^ 2 LP, ... (every lane of the wave with the
// same l % LP), the total in all of them.
template <int LP>
__device__ __forceinline__ float lane_stride_sum(float v) {
    if (LP == 8) v += dpp_f32<kDppRor8>(v, v);  // l ^ 8 within the 16-lane row
    if (LP <= 16) v = rows_pair_sum(v);
    return halves_sum(v);
}

__device__ __forceinline__ uint32_t ld_coh_u32(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh_u64(unsigned long long* p, unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_coh_u64(const unsigned long long* p) {
    return __hip_atomic_load(const_cast<unsigned long long*>(p), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long tagged64(uint32_t tag, float v) {
    return ((unsigned long long)tag << 32) | __float_as_uint(v);
}

// Lanes per output in a synchronous-merge share of S outputs (R S <= 256,
// R <= 16, so the R lanes of an output lie in one 16-lane row).
__host__ __device__ constexpr int attn_share_lanes(int S) {
    return S <= 16 ? 16 : S <= 32 ? 8 : S <= 64 ? 4 : S <= 128 ? 2 : 1;
}
// Chunks per lane the share handles at most: (the merge is used only when
// the share of nact chunks fits, attn_sync_fits)
template <int HD, int QH>
__host__ __device__ constexpr int attn_share_max() { return QH * HD / 128 + 2; }
template <int HD, int QH>
__host__ __device__ constexpr bool attn_sync_fits(int nact) {
    return nact > 1 && nact <= kAttnMaxChunks && QH * HD <= 256 * nact &&
           (nact + attn_share_lanes((QH * HD + nact - 1) / nact) - 1) /
                   attn_share_lanes((QH * HD + nact - 1) / nact) <=
               attn_share_max<HD, QH>();
}

// The synchronous merge, workgroup (g, c)'s share: outputs o0 .. o0 + S - 1 of
// its group's QH * HD (S = ceil(QH HD / nact), o0 = c S), each taken by R
// lanes (R S <= 256, R <= 16) that add every R-th chunk; per head M = max_c
// m_c, f_c = e^(m_c - M), L = sum_c l_c f_c (from the chunk statistics,
// staged in LDS), out = sum_c acc_c f_c / L.  Every value is read until it
// carries this launch's number (the other workgroups' stores are not
// waited for); the waits are bounded (a timeout raises device flag 4).
template <int HD, int QH>
__device__ void attn_merge_share(const AttnArgs& a, int g, int c, int nch, int nact, uint32_t tag,
                                 float (*s_st)[QH][kAttnMaxChunks], float* s_l) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t cstride = (size_t)QH * (HD + 2);
    const unsigned long long* base =
        reinterpret_cast<const unsigned long long*>(a.partial) + (size_t)g * nch * cstride;
    // this lane's share (below) is requested first, with the statistics: one
    // memory round trip when every chunk is in
    const int S = (QH * HD + nact - 1) / nact;
    const int R = attn_share_lanes(S);
    const int oi = tid / R, r = tid - oi * R, o = c * S + oi;
    const bool mine = oi < S && o < QH * HD;
    const int i = mine ? o / HD : 0, d = mine ? o - i * HD : 0;
    constexpr int kMaxPer = attn_share_max<HD, QH>();
    const int nper = mine ? (nact - r + R - 1) / R : 0;  // chunks r, r + R, ...
    unsigned long long u0[kMaxPer];
#pragma unroll
    for (int j = 0; j < kMaxPer; ++j)
        u0[j] = j < nper ? ld_coh_u64(base + (size_t)(r + R * j) * cstride + i * (HD + 2) + 2 + d)
                         : 0ull;
    // the statistics of every (head, chunk): 2 QH nact pairs, up to 4 per thread
    constexpr int kSt = (2 * QH * kAttnMaxChunks + 255) / 256;
    bool ok = true;
    for (int it = 0;; ++it) {
        bool cur = true;
        unsigned long long u[kSt];
#pragma unroll
        for (int s = 0; s < kSt; ++s) {
            const int e = tid + 256 * s;  // (head i, chunk k, m or l)
            const int i = e / (2 * nact), r = e - i * 2 * nact, k = r >> 1;
            u[s] = (e < 2 * QH * nact) ? ld_coh_u64(base + k * cstride + i * (HD + 2) + (r & 1))
                                       : ((unsigned long long)tag << 32);
        }
#pragma unroll
        for (int s = 0; s < kSt; ++s) {
            const int e = tid + 256 * s;
            const int i = e / (2 * nact), r = e - i * 2 * nact, k = r >> 1;
            if ((uint32_t)(u[s] >> 32) != tag) cur = false;
            else if (e < 2 * QH * nact) s_st[r & 1][i][k] = __uint_as_float((uint32_t)u[s]);
        }
        if (__syncthreads_and(cur)) break;
        if (it >= a.spin_limit) {
            if (tid == 0) flag_error(a.err, 4u);
            ok = false;
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    // per head: M, the factors (in place of m), L
    for (int i = wave; i < QH; i += 4) {
        const bool on = lane < nact;
        const float m = on ? s_st[0][i][lane] : -INFINITY;
        const float mx = wave_max(m);
        const float f = on ? expf(m - mx) : 0.f;
        const float l = wave_sum(on ? s_st[1][i][lane] * f : 0.f);
        if (on) s_st[0][i][lane] = f;
        if (lane == 0) s_l[i] = l;
    }
    __syncthreads();
    float vals[kMaxPer];
    bool have[kMaxPer];
#pragma unroll
    for (int j = 0; j < kMaxPer; ++j) {
        vals[j] = 0.f;
        have[j] = !(ok && j < nper);
    }
    for (int it = 0; ok; ++it) {
        // every missing value of the lane is requested before any is examined
        // (the first round's were requested with the statistics)
        unsigned long long u[kMaxPer];
#pragma unroll
        for (int j = 0; j < kMaxPer; ++j)
            u[j] = it == 0 ? u0[j]
                   : have[j] ? 0ull
                             : ld_coh_u64(base + (size_t)(r + R * j) * cstride + i * (HD + 2) + 2 + d);
        bool cur = true;
#pragma unroll
        for (int j = 0; j < kMaxPer; ++j) {
            if (!have[j]) {
                if ((uint32_t)(u[j] >> 32) == tag) {
                    have[j] = true;
                    vals[j] = __uint_as_float((uint32_t)u[j]);
                } else {
                    cur = false;
                }
            }
        }
        if (__all(cur)) break;
        if (it >= a.spin_limit) {
            flag_error(a.err, 4u);
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    float acc = 0.f;  // the chunks in order
#pragma unroll
    for (int j = 0; j < kMaxPer; ++j)
        if (j < nper) acc = fmaf(vals[j], s_st[0][i][r + R * j], acc);
    // the R lanes of an output (aligned in a 16-lane row), in a fixed order
    for (int off = R >> 1; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (mine && r == 0) a.out[(size_t)(g * QH + i) * HD + d] = acc / s_l[i];
}


// Workgroup (g, c): q heads g*QH .. g*QH+QH-1 (one kv head), positions
// c*a.chunk .. (c+1)*a.chunk - 1, walked SCH at a time with a running max
// and sum (the softmax of attnSoftmax, Shaders.metal:245-289, in pieces).
// Lanes take 8 dims of one position each (HD/8 lanes per position), so every
// K or V row is one coalesced read shared by the QH heads.  V: 0 one set of
// K/V registers, 64-position sub-chunks; 1 two sets (chunks of several
// sub-chunks); 2 one wide sub-chunk of up to attn_wide_sub<HD>() positions
// (chunks of 65..kAttnWideChunk positions, so that the grid fits the CUs).
template <int HD>
__host__ __device__ constexpr int attn_wide_sub() { return HD == 64 ? 96 : 80; }

// The planes z >= 1 of an attention grid: workgroup p of the P in them
// (linear dispatch number A + p after the A attention workgroups, so XCD
// p mod 8 when A and P are multiples of 8)
// reads pieces p, p + P, ... of the next launch's bytes, whose workgroup b
// runs on XCD b mod 8: each piece lands in the L2 of the XCD that reads it
// (and in the memory-side cache).  Nothing waits on this plane.
__device__ void attn_prefetch(const AttnArgs& a) {
    const int P = (int)(gridDim.x * gridDim.y * (gridDim.z - 1));
    const int p = (int)(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * (blockIdx.z - 1)));
    uint32_t acc = 0u;
    for (int b = p; b < a.pf_units; b += P) {
        const int64_t lo = (int64_t)b * a.pf_unit;
        const int64_t hi = min(lo + a.pf_unit, a.pf_bytes);
        const uint4* src = reinterpret_cast<const uint4*>(a.pf + lo);
        const int n = (int)((hi - lo) >> 4);
        for (int i0 = 0; i0 < n; i0 += 256 * 16) {
            uint4 v[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int i = i0 + (int)threadIdx.x + 256 * j;
                v[j] = i < n ? src[i] : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
        }
    }
    asm volatile("" ::"v"(acc));
}

template <int HD, int QH, int V>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
    if (blockIdx.z) {
        attn_prefetch(a);
        return;
    }
    constexpr bool TWO = V == 1;
    constexpr int SCH = V == 2 ? attn_wide_sub<HD>() : kAttnChunk;   // positions per sub-chunk
    constexpr int LP = HD / 8;                 // lanes per position
    constexpr int PPI = 64 / LP;               // positions per wave and iteration
    constexpr int PW = SCH / 4;                // positions per wave per sub-chunk
    constexpr int IT = PW / PPI;               // iterations
    static_assert(PW % PPI == 0 && SCH <= 128, "whole iterations, at most two positions per softmax lane");
    constexpr int HALF = HD / 2;
    __shared__ __attribute__((aligned(16))) float s_q[QH][HD];
    __shared__ __attribute__((aligned(16))) float s_kv[2][HD];
    __shared__ float s_p[QH][SCH];
    __shared__ __attribute__((aligned(16))) float s_acc[4][QH][HD];
    __shared__ float s_m[QH], s_l[QH], s_f[QH];
    __shared__ float s_st[2][QH][kAttnMaxChunks];  // merge: chunk max and sum
    __shared__ int s_flag;
    __shared__ uint32_t s_tag;

    const int g = blockIdx.x, c = blockIdx.y, nch = gridDim.y;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lp = lane % LP, pg = lane / LP;
    const int h0 = g * QH, kvh = h0 / a.hpkv;
    // this wave's q heads it = wave, wave + 4, ... (it == QH: the new k row)
    // and the new v row, requested before the position they wait on
    constexpr int QW = (QH + 4) / 4;   // items per wave at most
    float qpre[QW][HD / 64];
#pragma unroll
    for (int j = 0; j < QW; ++j) {
        const int it = wave + 4 * j;
        const float* src = it < QH ? a.q + (size_t)(h0 + it) * HD
                                   : (it == QH && a.fused ? a.k_new + (size_t)kvh * HD : nullptr);
#pragma unroll
        for (int e = 0; e < HD / 64; ++e) qpre[j][e] = src ? src[lane + 64 * e] : 0.f;
    }
    float vpre[(HD + 255) / 256];
#pragma unroll
    for (int e = 0; e < (HD + 255) / 256; ++e)
        vpre[e] = (a.fused && tid + 256 * e < HD) ? a.v_new[(size_t)kvh * HD + tid + 256 * e] : 0.f;
    int p = -1, seq;
    if (a.fused) {
        p = *a.pos;
        if (p >= a.max_seq) {
            if (g == 0 && c == 0 && tid == 0) flag_error(a.err, 32u);
            seq = a.max_seq;
        } else {
            seq = p + 1;
        }
    } else {
        seq = a.seq_len;
    }
    const bool has_new = a.fused && p < a.max_seq;  // row p comes from k_new / v_new
    const int c0 = c * a.chunk, c1 = min(c0 + a.chunk, seq);
    const int nact = min(nch, (seq + a.chunk - 1) / a.chunk);  // workgroups with positions
    const bool defer = a.defer && attn_defer_nact(p, a.max_seq, a.chunk, a.num_heads) > 0;
    const bool sync = a.sync_merge && !defer && attn_sync_fits<HD, QH>(nact);
    float* part = a.partial + ((size_t)g * nch + c) * QH * (HD + 2);
    unsigned long long* part64 =
        reinterpret_cast<unsigned long long*>(a.partial) + ((size_t)g * nch + c) * QH * (HD + 2);
    if (sync && tid == 0) s_tag = ld_coh_u32(a.gen) + 1u;

    if (c0 < seq) {
        // this lane's K and V rows of a 64-position sub-chunk (row p, not yet
        // in the cache, comes from LDS once it is prepared)
        // two sub-chunks of rows in flight (A, B alternate)
        struct KVRows {
            float k[IT][8], v[IT][8];
        };
        KVRows A, B;
        auto load_rows = [&](int p0, KVRows& R) {
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const int pp = p0 + wave * PW + it * PPI + pg;
                float4 k0 = {0.f, 0.f, 0.f, 0.f}, k1 = k0, v0 = k0, v1 = k0;
                if (pp < c1 && !(has_new && pp == p)) {
                    const size_t off = (size_t)pp * a.kv_pos + (size_t)kvh * a.kv_head + 8 * lp;
                    k0 = *reinterpret_cast<const float4*>(a.kcache + off);
                    k1 = *reinterpret_cast<const float4*>(a.kcache + off + 4);
                    v0 = *reinterpret_cast<const float4*>(a.vcache + off);
                    v1 = *reinterpret_cast<const float4*>(a.vcache + off + 4);
                }
                R.k[it][0] = k0.x, R.k[it][1] = k0.y, R.k[it][2] = k0.z, R.k[it][3] = k0.w;
                R.k[it][4] = k1.x, R.k[it][5] = k1.y, R.k[it][6] = k1.z, R.k[it][7] = k1.w;
                R.v[it][0] = v0.x, R.v[it][1] = v0.y, R.v[it][2] = v0.z, R.v[it][3] = v0.w;
                R.v[it][4] = v1.x, R.v[it][5] = v1.y, R.v[it][6] = v1.z, R.v[it][7] = v1.w;
            }
        };
        // (TWO: chunks of several sub-chunks; head_dim 256 has the registers
        // for one sub-chunk only)
        constexpr bool kTwo = TWO && HD <= 128;
        load_rows(c0, A);
        if (kTwo && c0 + SCH < c1) load_rows(c0 + SCH, B);
        // keep both sub-chunks' loads here (the compiler may otherwise sink
        // the second to its first use, a memory round trip later)
        asm volatile("" ::: "memory");

        // q heads (and the new k when this workgroup holds row p): per-head
        // RMSNorm (InferenceEngine.swift:538-548), then RoPE (:521-536)
        const bool mine_new = has_new && p >= c0 && p < c1;
        const int items = QH + (mine_new ? 1 : 0);
#pragma unroll
        for (int jw = 0; jw < QW; ++jw) {
            const int it = wave + 4 * jw;
            if (it >= items) break;
            const bool is_k = it == QH;
            float* dst = is_k ? s_kv[0] : s_q[it];
            const uint16_t* nw = is_k ? a.k_norm : a.q_norm;
            float v[HD / 64];
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < HD / 64; ++j) {
                v[j] = qpre[jw][j];
                ss = fmaf(v[j], v[j], ss);
            }
            if (a.fused && nw) {
                const float rms = 1.0f / sqrtf(wave_sum(ss) / (float)HD + a.eps);
#pragma unroll
                for (int j = 0; j < HD / 64; ++j) v[j] *= rms * bf16_to_f32(nw[lane + 64 * j]);
            }
#pragma unroll
            for (int j = 0; j < HD / 64; ++j) dst[lane + 64 * j] = v[j];
        }
        if (mine_new) {
#pragma unroll
            for (int e = 0; e < (HD + 255) / 256; ++e)
                if (tid + 256 * e < HD) s_kv[1][tid + 256 * e] = vpre[e];
        }
        __syncthreads();
        if (a.fused) {
            for (int t = tid; t < items * HALF; t += 256) {
                const int it = t / HALF, d = t - it * HALF;
                float* vec = it == QH ? s_kv[0] : s_q[it];
                float cs, sn;
                if (a.rope && p < a.max_seq) {  // rope_table_kernel's table (the same arithmetic)
                    const float2 r = reinterpret_cast<const float2*>(a.rope)[(size_t)p * HALF + d];
                    cs = r.x;
                    sn = r.y;
                } else {
                    const float freq = 1.0f / powf(a.rope_theta, (float)(2 * d) / (float)HD);
                    const float ang = (float)p * freq;
                    cs = cosf(ang);
                    sn = sinf(ang);
                }
                const float x0 = vec[d], x1 = vec[d + HALF];
                vec[d] = x0 * cs - x1 * sn;
                vec[d + HALF] = x0 * sn + x1 * cs;
            }
            __syncthreads();
            // the new row into the caches, by the first group of its kv head
            if (mine_new && h0 % a.hpkv == 0) {
                for (int d = tid; d < HD; d += 256) {
                    a.kcache[(size_t)p * a.kv_pos + (size_t)kvh * a.kv_head + d] = s_kv[0][d];
                    a.vcache[(size_t)p * a.kv_pos + (size_t)kvh * a.kv_head + d] = s_kv[1][d];
                }
            }
        }
        float qv[QH][8];
#pragma unroll
        for (int i = 0; i < QH; ++i) {
            const float4 q0 = *reinterpret_cast<const float4*>(&s_q[i][8 * lp]);
            const float4 q1 = *reinterpret_cast<const float4*>(&s_q[i][8 * lp + 4]);
            qv[i][0] = q0.x, qv[i][1] = q0.y, qv[i][2] = q0.z, qv[i][3] = q0.w;
            qv[i][4] = q1.x, qv[i][5] = q1.y, qv[i][6] = q1.z, qv[i][7] = q1.w;
        }
        float acc[QH][8];
#pragma unroll
        for (int i = 0; i < QH; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[i][e] = 0.f;
        if (tid < QH) {
            s_m[tid] = -INFINITY;
            s_l[tid] = 0.f;
        }

        auto sub = [&](int p0, KVRows& R) {
            if (mine_new && p >= p0 && p < p0 + SCH) {
#pragma unroll
                for (int it = 0; it < IT; ++it) {
                    if (p0 + wave * PW + it * PPI + pg != p) continue;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        R.k[it][e] = s_kv[0][8 * lp + e];
                        R.v[it][e] = s_kv[1][8 * lp + e];
                    }
                }
            }
            // scores (attnScores, Shaders.metal:209-243)
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const int pl = wave * PW + it * PPI + pg;
#pragma unroll
                for (int i = 0; i < QH; ++i) {
                    float d = 0.f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) d = fmaf(qv[i][e], R.k[it][e], d);
                    d = lane_group_sum<LP>(d);
                    if (lp == 0) s_p[i][pl] = p0 + pl < c1 ? d * a.scale : -INFINITY;
                }
            }
            __syncthreads();
            // running max and sum per head; lane = position of the sub-chunk
            // (and lane + 64 in a wide one)
            for (int i = wave; i < QH; i += 4) {
                constexpr bool W2 = SCH > 64;
                const float sc = s_p[i][lane];
                const float sc2 = (W2 && lane + 64 < SCH) ? s_p[i][W2 ? lane + 64 : lane] : -INFINITY;
                const float m_old = s_m[i];
                const float m = fmaxf(m_old, wave_max(fmaxf(sc, sc2)));
                const float e = sc == -INFINITY ? 0.f : expf(sc - m);
                const float e2 = sc2 == -INFINITY ? 0.f : expf(sc2 - m);
                const float f = m_old == -INFINITY ? 0.f : expf(m_old - m);
                const float l = wave_sum(W2 ? e + e2 : e);
                s_p[i][lane] = e;
                if (W2 && lane + 64 < SCH) s_p[i][W2 ? lane + 64 : lane] = e2;
                if (lane == 0) {
                    s_m[i] = m;
                    s_l[i] = fmaf(s_l[i], f, l);
                    s_f[i] = f;
                }
            }
            __syncthreads();
            // weighted V sum (attnValues, :291-326), earlier sub-chunks rescaled
#pragma unroll
            for (int i = 0; i < QH; ++i) {
                const float f = s_f[i];
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[i][e] *= f;
            }
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const int pl = wave * PW + it * PPI + pg;
#pragma unroll
                for (int i = 0; i < QH; ++i) {
                    const float w = s_p[i][pl];
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[i][e] = fmaf(w, R.v[it][e], acc[i][e]);
                }
            }
            if (p0 + SCH < c1) __syncthreads();  // s_p is rewritten by the next sub-chunk
        };
        if (!kTwo) {
            for (int p0 = c0; p0 < c1; p0 += SCH) {
                sub(p0, A);
                if (p0 + SCH < c1) load_rows(p0 + SCH, A);
            }
        }
        for (int p0 = c0; kTwo && p0 < c1; p0 += 2 * SCH) {
            sub(p0, A);
            if (p0 + 2 * SCH < c1) load_rows(p0 + 2 * SCH, A);
            if (p0 + SCH < c1) {
                sub(p0 + SCH, B);
                if (p0 + 3 * SCH < c1) load_rows(p0 + 3 * SCH, B);
            }
        }
#pragma unroll
        for (int i = 0; i < QH; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[i][e] = lane_stride_sum<LP>(acc[i][e]);
        if (pg == 0) {
#pragma unroll
            for (int i = 0; i < QH; ++i) {
                *reinterpret_cast<float4*>(&s_acc[wave][i][8 * lp]) =
                    float4{acc[i][0], acc[i][1], acc[i][2], acc[i][3]};
                *reinterpret_cast<float4*>(&s_acc[wave][i][8 * lp + 4]) =
                    float4{acc[i][4], acc[i][5], acc[i][6], acc[i][7]};
            }
        }
        __syncthreads();
        if (nact == 1) {
            // the only workgroup with positions: no merge
            for (int t = tid; t < QH * HD; t += 256) {
                const int i = t / HD, d = t - i * HD;
                a.out[(size_t)(h0 + i) * HD + d] =
                    (((s_acc[0][i][d] + s_acc[1][i][d]) + s_acc[2][i][d]) + s_acc[3][i][d]) / s_l[i];
            }
            return;
        }
        // (a deferred merge reads the partials in the next launch: plain stores;
        // the synchronous merge: (launch number, value) pairs)
        const uint32_t tag = s_tag;
        for (int t = tid; t < QH * HD; t += 256) {
            const int i = t / HD, d = t - i * HD;
            const float v = ((s_acc[0][i][d] + s_acc[1][i][d]) + s_acc[2][i][d]) + s_acc[3][i][d];
            if (sync)
                st_coh_u64(part64 + i * (HD + 2) + 2 + d, tagged64(tag, v));
            else if (defer)
                part[i * (HD + 2) + 2 + d] = v;
            else
                st_coh(part + i * (HD + 2) + 2 + d, v);
        }
        if (tid < QH) {
            if (sync) {
                st_coh_u64(part64 + tid * (HD + 2), tagged64(tag, s_m[tid]));
                st_coh_u64(part64 + tid * (HD + 2) + 1, tagged64(tag, s_l[tid]));
            } else if (defer) {
                part[tid * (HD + 2)] = s_m[tid];
                part[tid * (HD + 2) + 1] = s_l[tid];
            } else {
                st_coh(part + tid * (HD + 2), s_m[tid]);
                st_coh(part + tid * (HD + 2) + 1, s_l[tid]);
            }
        }
    }
    if (nact == 1) return;  // (workgroups past the sequence are not read by the merge)
    if (defer) return;      // merged by the next launch (mv_stage_attn)
    if (sync) {
        if (c < nact) attn_merge_share<HD, QH>(a, g, c, nch, nact, s_tag, s_st, s_l);
        // count this workgroup out; the last one advances the launch number
        // (every workgroup read it before counting itself out)
        __syncthreads();
        if (tid == 0 && count_out(a.fin, gridDim.x * gridDim.y, blockIdx.y * gridDim.x + blockIdx.x))
            __hip_atomic_store(a.gen, s_tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }

    // the last workgroup of the group merges the nact partials:
    // out = sum_c acc_c e^(m_c - M) / sum_c l_c e^(m_c - M)
    if (!last_workgroup(a.counters + g, nch, &s_flag)) return;
    const size_t cstride = (size_t)QH * (HD + 2);
    const float* base = a.partial + (size_t)g * nch * cstride;
    // The chunk statistics (one (max, sum) pair per thread, staged in LDS)
    // and the first kMB chunks of each of the thread's OPT outputs are loaded
    // together: one memory round trip for up to kMB chunks.
    static_assert(kAttnMaxChunks <= 64, "the merge takes one chunk per lane");
    constexpr int OPT = (QH * HD + 255) / 256;  // outputs per thread
    constexpr int kMB = OPT <= 2 ? 34 : OPT <= 4 ? 12 : 6;
    // (head, chunk) statistics: QH * nact <= QH * kAttnMaxChunks entries,
    // entry tid + 256 s for s < kSt
    constexpr int kSt = (QH * kAttnMaxChunks + 255) / 256;
    bool has_st[kSt];
    int st_i[kSt], st_c[kSt];
    float st_m[kSt], st_l[kSt];
#pragma unroll
    for (int s = 0; s < kSt; ++s) {
        const int e = tid + 256 * s;
        has_st[s] = e < QH * nact;
        st_i[s] = has_st[s] ? e / nact : 0;
        st_c[s] = has_st[s] ? e - st_i[s] * nact : 0;
        st_m[s] = 0.f;
        st_l[s] = 0.f;
        if (has_st[s]) {
            st_m[s] = ld_coh(base + st_c[s] * cstride + st_i[s] * (HD + 2));
            st_l[s] = ld_coh(base + st_c[s] * cstride + st_i[s] * (HD + 2) + 1);
        }
    }
    float acc[OPT];
#pragma unroll
    for (int o = 0; o < OPT; ++o) acc[o] = 0.f;
    for (int cb = 0; cb < nact; cb += kMB) {
        float vals[OPT][kMB];
#pragma unroll
        for (int o = 0; o < OPT; ++o) {
            const int t = tid + 256 * o;
            const int i = t < QH * HD ? t / HD : 0, d = t < QH * HD ? t - i * HD : 0;
#pragma unroll
            for (int j = 0; j < kMB; ++j)
                vals[o][j] = (t < QH * HD && cb + j < nact)
                                 ? ld_coh(base + (cb + j) * cstride + i * (HD + 2) + 2 + d)
                                 : 0.f;
        }
        if (cb == 0) {
            // per head: M = max_c m_c, factors f_c = e^(m_c - M) (in place of
            // m_c), L = sum_c l_c f_c -- once per (head, chunk), not per output
#pragma unroll
            for (int s = 0; s < kSt; ++s) {
                if (has_st[s]) {
                    s_st[0][st_i[s]][st_c[s]] = st_m[s];
                    s_st[1][st_i[s]][st_c[s]] = st_l[s];
                }
            }
            __syncthreads();
            for (int i = wave; i < QH; i += 4) {  // lane = chunk (nact <= 64)
                const bool ok = lane < nact;
                const float m = ok ? s_st[0][i][lane] : -INFINITY;
                const float mx = wave_max(m);
                const float f = ok ? expf(m - mx) : 0.f;
                const float l = wave_sum(ok ? s_st[1][i][lane] * f : 0.f);
                if (ok) s_st[0][i][lane] = f;
                if (lane == 0) s_l[i] = l;
            }
            __syncthreads();
        }
#pragma unroll
        for (int o = 0; o < OPT; ++o) {
            const int i = min((tid + 256 * o) / HD, QH - 1);
#pragma unroll
            for (int j = 0; j < kMB; ++j) {
                if (cb + j >= nact) break;
                acc[o] = fmaf(vals[o][j], s_st[0][i][cb + j], acc[o]);
            }
        }
    }
#pragma unroll
    for (int o = 0; o < OPT; ++o) {
        const int t = tid + 256 * o;
        if (t < QH * HD) a.out[(size_t)(h0 + t / HD) * HD + (t % HD)] = acc[o] / s_l[t / HD];
    }
    if (tid == 0) reset_counter(a.counters + g);
}

// ---- argmax (standalone) -------------------------------------------------------------

__global__ __launch_bounds__(1024) void argmax_kernel(const float* x, int n, int32_t* out) {
    __shared__ float s_v[16];
    __shared__ int s_i[16];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += 1024) {
        const float v = x[i];
        if (am_better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
    wave_argmax(bv, bi);
    if (lane == 0) {
        s_v[wave] = bv;
        s_i[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; ++w)
            if (am_better(s_v[w], s_i[w], bv, bi)) {
                bv = s_v[w];
                bi = s_i[w];
            }
        // InferenceEngine.swift:550-555 scans from x[0] with a strict >
        *out = (bi < n && !__builtin_isnan(x[0])) ? bi : 0;
    }
}

// RoPE (InferenceEngine.swift:521-536) factors of every position and pair:
// table[p][d] = (cos, sin) of p / theta^(2d / head_dim), the arithmetic of
// the in-kernel form of attn_kernel, made once per decoder.
__global__ __launch_bounds__(256) void rope_table_kernel(float* table, int max_seq, int half,
                                                         float theta, int hd) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= max_seq * half) return;
    const int p = i / half, d = i - p * half;
    const float freq = 1.0f / powf(theta, (float)(2 * d) / (float)hd);
    const float ang = (float)p * freq;
    table[2 * i] = cosf(ang);
    table[2 * i + 1] = sinf(ang);
}

__global__ void set_i32_kernel(int32_t* p, int32_t v) { *p = v; }

// Rows per wave: more rows per workgroup for taller matrices (each workgroup
// stages, and may normalise, the whole input; lm_head of a 50k vocabulary
// reads 1% faster at 8 than at 4).
// Rows per wave by row count.  Tall matrices (the lm_heads) take 3: 12 rows
// per workgroup, three workgroups per CU at once, the grid many rounds deep
// (50304 x 2048: 44.1 us at 8 rows per wave, whose 1572 workgroups of two
// per CU left a last round of 36; 38.1-39.2 at 4, 36.1 at 3, 36.3 at 2;
// 32000 x 4096: 46.6 at 4, 45.9-46.2 at 3).
int mv_rpw(int rows) { return rows >= 8192 ? 3 : rows >= 2048 ? 2 : 1; }

template <int RPW>
int launch_mv(const MvArgs& a, hipStream_t st) {
    const unsigned grid = (unsigned)((a.rows + 4 * RPW - 1) / (4 * RPW));
    const size_t lds = (size_t)a.cols * 4;
    if (a.cols <= 2048)
        hipLaunchKernelGGL((matvec_kernel<RPW, true, 2>), dim3(grid), dim3(256), lds, st, a);
    else if (a.cols <= 4096)
        hipLaunchKernelGGL((matvec_kernel<RPW, true, 4>), dim3(grid), dim3(256), lds, st, a);
    else if (a.cols <= kMvStageMax)
        hipLaunchKernelGGL((matvec_kernel<RPW, true, 0>), dim3(grid), dim3(256), lds, st, a);
    else
        hipLaunchKernelGGL((matvec_kernel<RPW, false, 0>), dim3(grid), dim3(256), 0, st, a);
    return (int)hipGetLastError();
}

// The kernel's variant for a chunk of `chunk` positions (attn_kernel's V).
int attn_variant(int chunk) {
    return chunk <= kAttnChunk ? 0 : (chunk <= kAttnWideChunk ? 2 : 1);
}

template <int HD, int V>
int launch_attn_v(const AttnArgs& a, dim3 grid, hipStream_t st) {
    switch (a.qh) {
        case 1: hipLaunchKernelGGL((attn_kernel<HD, 1, V>), grid, dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL((attn_kernel<HD, 2, V>), grid, dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL((attn_kernel<HD, 4, V>), grid, dim3(256), 0, st, a); break;
        case 8: hipLaunchKernelGGL((attn_kernel<HD, 8, V>), grid, dim3(256), 0, st, a); break;
        default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

template <int HD>
int launch_attn_hd(const AttnArgs& a, dim3 grid, hipStream_t st) {
    // one-sub-chunk workgroups keep no second set of K/V registers, so two of
    // them fit on a CU (more than 256 workgroups then run at once)
    switch (attn_variant(a.chunk)) {
        case 0: return launch_attn_v<HD, 0>(a, grid, st);
        case 2: return launch_attn_v<HD, 2>(a, grid, st);
        default: return launch_attn_v<HD, 1>(a, grid, st);
    }
}

}  // namespace

int launch_set_i32(int32_t* p, int32_t v, void* stream) {
    hipLaunchKernelGGL(set_i32_kernel, dim3(1), dim3(1), 0, static_cast<hipStream_t>(stream), p, v);
    return (int)hipGetLastError();
}

int launch_rmsnorm(const float* x, const uint16_t* w, float* out, int n, float eps, void* stream) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream), x, w,
                       out, n, eps);
    return (int)hipGetLastError();
}

int matvec_workgroups(int rows) {
    const int per = 4 * mv_rpw(rows);
    return (rows + per - 1) / per;
}

int matvec_rows_per_workgroup(int rows) { return 4 * mv_rpw(rows); }

int launch_matvec_bf16(const MvArgs& a, void* stream) {
    if (a.cols % 8 || a.rows <= 0 || a.cols <= 0) return (int)hipErrorInvalidValue;
    if ((a.embed || a.norm_w) && a.cols > kMvStageMax) return (int)hipErrorInvalidValue;
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (mv_rpw(a.rows)) {
        case 3: return launch_mv<3>(a, st);
        case 2: return launch_mv<2>(a, st);
        default: return launch_mv<1>(a, st);
    }
}

int attention_qh(int hpkv) {
    for (int q = kAttnMaxQH; q > 1; q >>= 1)
        if (hpkv % q == 0) return q;
    return 1;
}

// The fewest 64-position sub-chunks per workgroup that keep at most
// kAttnMaxChunks workgroups per group.
int attention_chunk_min(int max_positions) {
    const int sub = (max_positions + kAttnChunk - 1) / kAttnChunk;  // 64-position sub-chunks
    return kAttnChunk * ((sub + kAttnMaxChunks - 1) / kAttnMaxChunks);
}

// When that grid has more workgroups than the device has CUs: if chunks
// of at most kAttnWideChunk positions fit the groups on the CUs, those (one
// wide sub-chunk each: 2113 positions x 8 groups on 256 CUs, 67-position
// chunks, 12.4 -> ~9.8 us); else, from two workgroups per CU on, one
// workgroup per CU taking more 64-position sub-chunks (32 q / 8 kv heads of
// 128, 256 CUs: 19.8 -> 16.1 us at 4096 positions, 34.5 -> 25.7 us at 8192).
// Between the two (one round and a bit, wide chunks too short) the 64-position
// chunks stay: 256 workgroups of 66 positions in two sub-chunks measured 14.4
// against 13.5 us for 264 of 64.
int attention_chunk(int max_positions, int groups, int cus) {
    const int c = attention_chunk_min(max_positions);
    const long wgs = (long)groups * ((max_positions + c - 1) / c);
    const int per = std::min(kAttnMaxChunks, groups > 0 ? cus / groups : 0);   // chunks per group
    if (per < 1 || wgs <= cus) return c;
    const int wide = (max_positions + per - 1) / per;
    if (c == kAttnChunk && wide <= kAttnWideChunk) return wide;
    if (wgs < 2L * cus) return c;
    const int sub = (max_positions + kAttnChunk - 1) / kAttnChunk;
    return std::max(c, kAttnChunk * ((sub + per - 1) / per));
}

// (sized for attention_chunk_min, whose chunk count bounds attention_chunk's)
int attention_partial_floats(int num_heads, int head_dim, int max_positions) {
    const int chunk = attention_chunk_min(max_positions);
    return 2 * num_heads * ((max_positions + chunk - 1) / chunk) * (head_dim + 2);
}

namespace {
template <int HD, int V>
int attn_occupancy_v(int qh) {
    int n = 0;
    hipError_t e = hipErrorInvalidValue;
    switch (qh) {
        case 1: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, attn_kernel<HD, 1, V>, 256, 0); break;
        case 2: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, attn_kernel<HD, 2, V>, 256, 0); break;
        case 4: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, attn_kernel<HD, 4, V>, 256, 0); break;
        case 8: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, attn_kernel<HD, 8, V>, 256, 0); break;
        default: break;
    }
    return e == hipSuccess ? n : 0;
}
template <int HD>
int attn_occupancy_hd(int qh, int v) {
    return v == 0 ? attn_occupancy_v<HD, 0>(qh) : (v == 2 ? attn_occupancy_v<HD, 2>(qh) : attn_occupancy_v<HD, 1>(qh));
}

// Workgroups of the attention kernel of (head_dim, qh, variant) one CU
// holds, from the occupancy query, kept after the first ask.
std::atomic<int> g_attn_occ[3][9][3];

int attn_blocks_per_cu(int hd, int qh, int v) {
    const int hi = hd == 64 ? 0 : hd == 128 ? 1 : 2;
    std::atomic<int>& slot = g_attn_occ[hi][qh][v];
    int n = slot.load(std::memory_order_relaxed);
    if (n == 0) {
        n = hd == 64 ? attn_occupancy_hd<64>(qh, v)
                     : hd == 128 ? attn_occupancy_hd<128>(qh, v) : attn_occupancy_hd<256>(qh, v);
        n = n > 0 ? n : -1;
        slot.store(n, std::memory_order_relaxed);
    }
    return n > 0 ? n : 0;
}
}  // namespace

bool attention_grid_fits(const AttnArgs& a) {
    if (a.qh <= 0 || a.qh > 8 || a.cus <= 0) return false;
    const int64_t grid = (int64_t)(a.num_heads / a.qh) * ((a.max_seq + a.chunk - 1) / a.chunk);
    return (int64_t)attn_blocks_per_cu(a.head_dim, a.qh, attn_variant(a.chunk)) * a.cus >= grid;
}

int launch_attention(const AttnArgs& a, void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (a.qh <= 0 || a.num_heads % a.qh || a.hpkv % a.qh ||
        a.chunk != attention_chunk(a.max_seq, a.num_heads / a.qh, a.cus))
        return (int)hipErrorInvalidValue;
    if (a.kv_pos <= 0 || a.kv_head <= 0) return (int)hipErrorInvalidValue;
    if (a.sync_merge && !(a.gen && a.fin && attention_grid_fits(a))) return (int)hipErrorInvalidValue;
    if (a.pf && (a.pf_unit <= 0 || a.pf_units <= 0 || a.pf_bytes <= 0 || a.pf_unit % 16 ||
                 a.pf_bytes % 16 || (int64_t)a.pf_units * a.pf_unit < a.pf_bytes))
        return (int)hipErrorInvalidValue;
    // (the prefetch planes only where the attention leaves most CUs idle: on a
    // full grid they compete with it, cfg4 2615 -> 2670 us per token)
    const unsigned gx = (unsigned)(a.num_heads / a.qh), gy = (unsigned)((a.max_seq + a.chunk - 1) / a.chunk);
    const bool pf = a.pf && 2 * (int64_t)gx * gy <= a.cus;
    const dim3 grid(gx, gy, pf ? 1u + (unsigned)kAttnPfPlanes : 1u);
    switch (a.head_dim) {
        case 64: return launch_attn_hd<64>(a, grid, st);
        case 128: return launch_attn_hd<128>(a, grid, st);
        case 256: return launch_attn_hd<256>(a, grid, st);
        default: return (int)hipErrorInvalidValue;
    }
}

int launch_rope_table(float* table, int max_seq, int head_dim, float theta, void* stream) {
    const int n = max_seq * (head_dim / 2);
    hipLaunchKernelGGL(rope_table_kernel, dim3((n + 255) / 256), dim3(256), 0,
                       static_cast<hipStream_t>(stream), table, max_seq, head_dim / 2, theta,
                       head_dim);
    return (int)hipGetLastError();
}

int launch_argmax(const float* x, int n, int32_t* out, void* stream) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream), x, n,
                       out);
    return (int)hipGetLastError();
}

}  // namespace m1moe
