// router.hip — router logits, softmax and top-K for T tokens on the GPU.
//
// Replaces the CPU router of the reference (computeRouterScores and
// selectTopK, InferenceEngine.swift:490-519), which ran after a full GPU
// sync.  Two kernels:
//
//   router_logits   logits[t][e] = sum_d W[e][d] * x[t][d] for a tile of
//                   8 tokens x 16 experts per workgroup.  Every product
//                   bf16 * x is exact in f64; each thread sums half a row in
//                   f64 and the two halves are added in a fixed order before
//                   one rounding to f32 (+ the optional logit bias), so the
//                   value is independent of the summation order in practice.
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

constexpr int kTT = 8;       // tokens per logits workgroup
constexpr int kTE = 16;      // experts per logits workgroup
constexpr int kMaxE = 256;   // 4 logits per lane in the ranking wave
constexpr int kMaxK = 32;    // one selection per lane

// thread -> (token tt = tid / 32, expert te = (tid / 2) % 16, half = tid % 2)
__global__ __launch_bounds__(256) void router_logits_kernel(RouterArgs a) {
    __shared__ double s_half[256];
    const int tid = threadIdx.x;
    const int tt = tid >> 5, te = (tid >> 1) & (kTE - 1), half = tid & 1;
    const int t = blockIdx.x * kTT + tt, e = blockIdx.y * kTE + te;
    const int h = a.h;
    double acc = 0.0;
    if (t < a.T && e < a.E) {
        const uint16_t* wr = a.router + (size_t)e * h;
        const int d0 = half * (h / 2), d1 = d0 + h / 2;
        if (a.x_bf16) {
            const uint16_t* xr = static_cast<const uint16_t*>(a.x) + (size_t)t * h;
            for (int d = d0; d < d1; d += 8) {
                const uint4 wv = *reinterpret_cast<const uint4*>(wr + d);
                const uint4 xv = *reinterpret_cast<const uint4*>(xr + d);
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    acc += (double)bf16x8_at(wv, i) * (double)bf16x8_at(xv, i);
            }
        } else {
            const float* xr = static_cast<const float*>(a.x) + (size_t)t * h;
            for (int d = d0; d < d1; d += 8) {
                const uint4 wv = *reinterpret_cast<const uint4*>(wr + d);
                const float4 x0 = *reinterpret_cast<const float4*>(xr + d);
                const float4 x1 = *reinterpret_cast<const float4*>(xr + d + 4);
                const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int i = 0; i < 8; ++i) acc += (double)bf16x8_at(wv, i) * (double)xs[i];
            }
        }
    }
    s_half[tid] = acc;
    __syncthreads();
    if (half == 0 && t < a.T && e < a.E) {
        float l = (float)(s_half[tid] + s_half[tid + 1]);
        if (a.bias) l = l + a.bias[e];
        a.logits[(size_t)t * a.E + e] = l;
        if (a.user_logits) a.user_logits[(size_t)t * a.E + e] = l;
    }
}

// Orders this wave's LDS accesses before / after the call (lanes exchange
// values through LDS; the waves of a workgroup are independent).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One wave per token (four tokens per workgroup).
__global__ __launch_bounds__(256) void router_rank_kernel(RouterArgs a) {
    __shared__ __attribute__((aligned(16))) float s_v[4][kMaxE];
    __shared__ int s_sel[4][kMaxK];
    __shared__ float s_p[4][kMaxK];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + wave;
    if (t >= a.T) return;
    const int E = a.E, K = a.K;
    const float* lg = a.logits + (size_t)t * E;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
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
    int rank[4] = {0, 0, 0, 0};
    for (int j0 = 0; j0 < E; j0 += 4) {
        const float4 w4 = *reinterpret_cast<const float4*>(&s_v[wave][j0]);
        const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int j = j0 + q;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int i = lane + 64 * m;
                rank[m] += (int)(wv[q] > v[m]) | ((int)(wv[q] == v[m]) & (int)(j < i));
            }
        }
    }
    float mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
    mx = wave_max(mx);
    float ex[4], sum = 0.f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        ex[m] = (lane + 64 * m < E) ? expf(v[m] - mx) : 0.f;
        sum += ex[m];
    }
    const float inv = 1.0f / wave_sum(sum);
    // selected (expert, probability) by slot
#pragma unroll
    for (int m = 0; m < 4; ++m) {
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
    if (a.E > kMaxE || a.K > kMaxK || a.h % 16) return (int)hipErrorInvalidValue;
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(router_logits_kernel,
                       dim3((unsigned)((a.T + kTT - 1) / kTT), (unsigned)((a.E + kTE - 1) / kTE)),
                       dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL(router_rank_kernel, dim3((unsigned)((a.T + 3) / 4)), dim3(256), 0, st, a);
    return (int)hipGetLastError();
}

}  // namespace m1moe
