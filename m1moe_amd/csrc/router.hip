// router.hip — router logits, softmax and top-K on the GPU.
//
// Replaces the CPU router of the reference (computeRouterScores and
// selectTopK, InferenceEngine.swift:490-519), which ran after a full GPU
// sync.  One wave per (token, expert) forms the logit; the last block of a
// token (counter-based) ranks the experts and writes the routing.
//
// Logit: every product bf16(W) * x is exact in f64 and the 64 per-lane
// partial sums are combined in f64 before one rounding to f32, so the value
// is independent of the summation order in practice.  Ranking: descending
// logit, ties to the lower expert index (softmax is monotone; this is the
// order of the reference's stable sort on probabilities).  Weights:
// softmax probabilities exp(l - max) * (1 / sum) (:501-506), renormalised
// over the selection when norm_topk_prob is set (:514-517).
#include <hip/hip_runtime.h>

#include <cfloat>

#include "device.hpp"
#include "internal.hpp"

namespace m1moe {
namespace {

constexpr int kRouterWaves = 4;  // experts (waves) per block
constexpr int kMaxE = 256;       // 4 logits per lane in the ranking wave
constexpr int kMaxK = 32;  // one selection per lane

__global__ __launch_bounds__(256) void router_topk_kernel(RouterArgs a, int blocks_per_token) {
    const int t = blockIdx.x / blocks_per_token;
    const int b = blockIdx.x - t * blocks_per_token;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int e = b * kRouterWaves + wave;
    const int h = a.h, E = a.E, K = a.K;

    if (e < E) {
        const uint16_t* wr = a.router + (size_t)e * h;
        double acc = 0.0;
        if (a.x_bf16) {
            const uint16_t* xr = static_cast<const uint16_t*>(a.x) + (size_t)t * h;
            for (int d = lane * 8; d < h; d += 512) {
                const uint4 wv = *reinterpret_cast<const uint4*>(wr + d);
                const uint4 xv = *reinterpret_cast<const uint4*>(xr + d);
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    acc += (double)bf16x8_at(wv, i) * (double)bf16x8_at(xv, i);
            }
        } else {
            const float* xr = static_cast<const float*>(a.x) + (size_t)t * h;
            for (int d = lane * 8; d < h; d += 512) {
                const uint4 wv = *reinterpret_cast<const uint4*>(wr + d);
                const float4 x0 = *reinterpret_cast<const float4*>(xr + d);
                const float4 x1 = *reinterpret_cast<const float4*>(xr + d + 4);
                const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int i = 0; i < 8; ++i) acc += (double)bf16x8_at(wv, i) * (double)xs[i];
            }
        }
        acc = wave_sum_f64_last(acc);
        if (lane == 63) {
            float l = (float)acc;
            if (a.bias) l = l + a.bias[e];
            a.logits[(size_t)t * E + e] = l;
            if (a.user_logits) a.user_logits[(size_t)t * E + e] = l;
        }
    }

    // last block of this token ranks the experts
    __shared__ int s_last;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = atomicAdd(&a.counters[t], 1u);
        s_last = (prev == (uint32_t)blocks_per_token - 1u);
    }
    __syncthreads();
    if (!s_last || wave != 0) return;
    __threadfence();

    const float* lg = a.logits + (size_t)t * E;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int ee = lane + 64 * j;
        float x = -INFINITY;
        if (ee < E) {
            x = lg[ee];
            if (x != x) x = -INFINITY;  // NaN ranks last
        }
        v[j] = x;
    }

    int my_idx;
    float wr;
    topk_softmax(v, E, K, a.norm, lane, my_idx, wr);
    if (lane < K) {
        a.idx[(size_t)t * K + lane] = my_idx;
        a.w[(size_t)t * K + lane] = wr;
        if (a.user_idx) a.user_idx[(size_t)t * K + lane] = my_idx;
        if (a.user_w) a.user_w[(size_t)t * K + lane] = wr;
    }
    // re-arm the counter for the next launch
    if (lane == 0)
        __hip_atomic_store(&a.counters[t], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

int launch_router_topk(const RouterArgs& a, void* stream) {
    if (a.E > kMaxE || a.K > kMaxK) return (int)hipErrorInvalidValue;
    const int bpt = (a.E + kRouterWaves - 1) / kRouterWaves;
    hipLaunchKernelGGL(router_topk_kernel, dim3((unsigned)(a.T * bpt)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), a, bpt);
    return (int)hipGetLastError();
}

}  // namespace m1moe
