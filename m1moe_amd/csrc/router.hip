// router.hip — router logits, softmax and top-K for T tokens on the GPU.
//
// Replaces the CPU router of the reference (computeRouterScores and
// selectTopK, InferenceEngine.swift:490-519), which ran after a full GPU
// sync.  Two kernels:
//
//   router_logits   logits[t][e] = sum_d W[e][d] * x[t][d]: a wave computes
//                   4 tokens x 4 experts with its lanes across the columns
//                   (coalesced 128-bit loads, all of a 2048-column row in
//                   flight at once), a workgroup 4 tokens x 16 experts.  For
//                   a prefill an extra row of workgroups writes x's f16 copy
//                   (prep_token): wave w takes token t0 + w.
//                   Every product bf16 * x is exact in f64; each lane sums
//                   its columns in f64, the lanes are added by a fixed DPP
//                   tree, then one rounding to f32 (+ the optional logit
//                   bias), so the value is independent of the summation
//                   order in practice.
//   router_rank     one wave per token: experts ranked by descending logit,
//                   ties to the lower index (softmax is monotone; this is the
//                   order of the reference's stable sort on probabilities),
//                   softmax weights exp(l - max) * (1 / sum) (:501-506),
//                   renormalised over the selection in slot order when
//                   norm_topk_prob is set (:514-517).
#include <hip/hip_runtime.h>

#include "device.hpp"
#include "internal.hpp"

namespace m1moe {
namespace {

constexpr int kTT = 4;       // tokens per logits wave and workgroup
constexpr int kTEw = 4;      // experts per logits wave
constexpr int kTE = 16;      // experts per logits workgroup (four waves)
constexpr int kMaxE = 256;   // 4 logits per lane in the ranking wave
constexpr int kMaxK = 32;    // one selection per lane

// Lane l takes columns blk * 512 + 8 l .. + 7 of each 512-column block; DB
// blocks have their loads in flight together.  Rows past T / E are clamped
// (loaded, never stored); columns past h are skipped.
template <bool XBF16, int DB>
__device__ __forceinline__ void logits_wave(const RouterArgs& a, int t0, int e0, int lane,
                                            double (&acc)[kTT][kTEw]) {
    const int h = a.h, nb = (h + 511) / 512;
    const uint16_t* wr[kTEw];
#pragma unroll
    for (int j = 0; j < kTEw; ++j) wr[j] = a.router + (size_t)min(e0 + j, a.E - 1) * h;
    for (int b0 = 0; b0 < nb; b0 += DB) {
        uint4 wv[DB][kTEw];
        float4 xv[DB][kTT][2];  // f32 x, or bf16 x in xv[][][0] as raw bits
#pragma unroll
        for (int u = 0; u < DB; ++u) {
            const int c = min((b0 + u) * 512 + lane * 8, h - 8);
#pragma unroll
            for (int j = 0; j < kTEw; ++j) wv[u][j] = *reinterpret_cast<const uint4*>(wr[j] + c);
#pragma unroll
            for (int i = 0; i < kTT; ++i) {
                const size_t row = (size_t)min(t0 + i, a.T - 1) * h + c;
                if (XBF16) {
                    const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.x) + row);
                    xv[u][i][0] = __builtin_bit_cast(float4, q);
                } else {
                    const float* xr = static_cast<const float*>(a.x) + row;
                    xv[u][i][0] = *reinterpret_cast<const float4*>(xr);
                    xv[u][i][1] = *reinterpret_cast<const float4*>(xr + 4);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < DB; ++u) {
            if ((b0 + u) * 512 + lane * 8 >= h) continue;
#pragma unroll
            for (int i = 0; i < kTT; ++i) {
                float x8[8];
                if (XBF16) {
                    const uint4 q = __builtin_bit_cast(uint4, xv[u][i][0]);
#pragma unroll
                    for (int k = 0; k < 8; ++k) x8[k] = bf16x8_at(q, k);
                } else {
                    const float4 p = xv[u][i][0], r = xv[u][i][1];
                    x8[0] = p.x; x8[1] = p.y; x8[2] = p.z; x8[3] = p.w;
                    x8[4] = r.x; x8[5] = r.y; x8[6] = r.z; x8[7] = r.w;
                }
#pragma unroll
                for (int j = 0; j < kTEw; ++j)
#pragma unroll
                    for (int k = 0; k < 8; ++k)
                        acc[i][j] = fma((double)bf16x8_at(wv[u][j], k), (double)x8[k], acc[i][j]);
            }
        }
    }
}

// The prefill's f16 copy of token t's x row (when a.xq is set): the row times
// a per-token power of two that maps max|x| into [2^13, 2^14), each 8-column
// group stored in the column order perm8 of the GEMM's A fragments, and the
// inverse power in xinv[t].  One wave; h % 64 == 0.
__device__ void prep_token(const RouterArgs& a, int t, int lane) {
    if (t >= a.T) return;
    const int units = a.h / 8;
    auto load8 = [&](int u, float (&v)[8]) {
        if (a.x_bf16) {
            const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.x) +
                                                            (size_t)t * a.h + 8 * u);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = bf16x8_at(q, i);
        } else {
            const float* xr = static_cast<const float*>(a.x) + (size_t)t * a.h + 8 * u;
            const float4 q0 = *reinterpret_cast<const float4*>(xr);
            const float4 q1 = *reinterpret_cast<const float4*>(xr + 4);
            v[0] = q0.x; v[1] = q0.y; v[2] = q0.z; v[3] = q0.w;
            v[4] = q1.x; v[5] = q1.y; v[6] = q1.z; v[7] = q1.w;
        }
    };
    float mx = 0.f;
    for (int u = lane; u < units; u += 64) {
        float v[8];
        load8(u, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(v[i]));
    }
    mx = wave_max(mx);
    float scale, inv;
    pow2_scale(mx, scale, inv);
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    for (int u = lane; u < units; u += 64) {
        float v[8];
        load8(u, v);
        h8 o;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (_Float16)(v[perm8(i)] * scale);
        *reinterpret_cast<h8*>(a.xq + (size_t)t * a.h + 8 * u) = o;
    }
    if (lane == 0) a.xinv[t] = inv;
}

static_assert(kTT == 4, "one wave of the 256-thread workgroup per token");

__global__ __launch_bounds__(256) void router_logits_kernel(RouterArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t0 = blockIdx.x * kTT, e0 = blockIdx.y * kTE + wave * kTEw;
    // for a prefill, an extra row of workgroups (the last) makes the f16 copy:
    // wave w takes token t0 + w, beside the logits of the other rows
    if (a.xq && blockIdx.y == gridDim.y - 1) {
        prep_token(a, t0 + wave, lane);
        return;
    }
    if (e0 >= a.E) return;
    double acc[kTT][kTEw];
#pragma unroll
    for (int i = 0; i < kTT; ++i)
#pragma unroll
        for (int j = 0; j < kTEw; ++j) acc[i][j] = 0.0;
    if (a.x_bf16)
        logits_wave<true, 4>(a, t0, e0, lane, acc);
    else
        logits_wave<false, 2>(a, t0, e0, lane, acc);
#pragma unroll
    for (int i = 0; i < kTT; ++i)
#pragma unroll
        for (int j = 0; j < kTEw; ++j) {
            const double v = wave_sum_f64_last(acc[i][j]);  // lane 63
            const int t = t0 + i, e = e0 + j;
            if (lane == 63 && t < a.T && e < a.E) {
                float l = (float)v;
                if (a.bias) l = l + a.bias[e];
                a.logits[(size_t)t * a.E + e] = l;
                if (a.user_logits) a.user_logits[(size_t)t * a.E + e] = l;
            }
        }
}

// Orders this wave's LDS accesses before / after the call (lanes exchange
// values through LDS; the waves of a workgroup are independent).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One wave per token (four tokens per workgroup); MB = experts per lane
// (E <= 64 * MB).
template <int MB>
__global__ __launch_bounds__(256) void router_rank_kernel(RouterArgs a) {
    __shared__ __attribute__((aligned(16))) float s_v[4][64 * MB];
    __shared__ int s_sel[4][kMaxK];
    __shared__ float s_p[4][kMaxK];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + wave;
    if (t >= a.T) return;
    const int E = a.E, K = a.K;
    const float* lg = a.logits + (size_t)t * E;
    float v[MB];
#pragma unroll
    for (int j = 0; j < MB; ++j) {
        const int e = lane + 64 * j;
        float x = -INFINITY;
        if (e < E) {
            x = lg[e];
            if (x != x) x = -INFINITY;  // NaN ranks last
        }
        v[j] = x;
        s_v[wave][e] = x;  // -inf beyond E
    }
    wave_lds_sync();
    // rank of expert i = experts ahead of it (padding: -inf at a higher index)
    const int Ep = (E + 3) & ~3;
    int rank[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) rank[m] = 0;
    for (int j0 = 0; j0 < Ep; j0 += 4) {
        const float4 w4 = *reinterpret_cast<const float4*>(&s_v[wave][j0]);
        const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int j = j0 + q;
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                const int i = lane + 64 * m;
                rank[m] += (int)(wv[q] > v[m]) | ((int)(wv[q] == v[m]) & (int)(j < i));
            }
        }
    }
    float mx = v[0];
#pragma unroll
    for (int m = 1; m < MB; ++m) mx = fmaxf(mx, v[m]);
    mx = wave_max(mx);
    float ex[MB], sum = 0.f;
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        ex[m] = (lane + 64 * m < E) ? expf(v[m] - mx) : 0.f;
        sum += ex[m];
    }
    const float inv = 1.0f / wave_sum(sum);
    // selected (expert, probability) by slot
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        const int i = lane + 64 * m;
        if (i < E && rank[m] < K) {
            s_sel[wave][rank[m]] = i;
            s_p[wave][rank[m]] = ex[m] * inv;
        }
    }
    wave_lds_sync();
    if (lane < K) {
        const int e = s_sel[wave][lane];
        float w = s_p[wave][lane];
        if (a.norm) {
            float ssum = 0.f;
            for (int r = 0; r < K; ++r) ssum = ssum + s_p[wave][r];
            w = w / ssum;
        }
        a.idx[(size_t)t * K + lane] = e;
        a.w[(size_t)t * K + lane] = w;
        if (a.user_idx) a.user_idx[(size_t)t * K + lane] = e;
        if (a.user_w) a.user_w[(size_t)t * K + lane] = w;
    }
}

}  // namespace

int launch_router_topk(const RouterArgs& a, void* stream) {
    if (a.E > kMaxE || a.K > kMaxK || a.h % 64) return (int)hipErrorInvalidValue;
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(router_logits_kernel,
                       dim3((unsigned)((a.T + kTT - 1) / kTT),
                            (unsigned)((a.E + kTE - 1) / kTE + (a.xq ? 1 : 0))),
                       dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    const dim3 g((unsigned)((a.T + 3) / 4));
    if (a.E <= 64)
        hipLaunchKernelGGL(router_rank_kernel<1>, g, dim3(256), 0, st, a);
    else if (a.E <= 128)
        hipLaunchKernelGGL(router_rank_kernel<2>, g, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL(router_rank_kernel<4>, g, dim3(256), 0, st, a);
    return (int)hipGetLastError();
}

}  // namespace m1moe
