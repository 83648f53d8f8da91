// dense.hip — the dense part of a decoder step on the GPU.
//
// The reference runs these on Metal one threadgroup per row or per dot
// product (Shaders.metal:96-358) and the q/k norms, RoPE and the KV store on
// the CPU between syncs (InferenceEngine.swift:196-228, 521-548).  Here:
//
//   embed          token row of the bf16 embedding -> f32
//                  (InferenceEngine.swift:482-488)
//   rmsnorm        one workgroup: sum of squares, then x * rsqrt(ss/n + eps) * w
//   matvec_bf16    y = W x (+ residual): a wave takes kMvRows rows, its lanes
//                  128-bit loads across the columns; up to three weight
//                  segments per launch (q, k, v share the input)
//   qk_rope_kv     one workgroup per q or k head: optional per-head RMSNorm,
//                  RoPE on (d, d + hd/2) pairs, k and v stored at the
//                  device-side position
//   attn_partial   one workgroup per (head, 256 positions): scores, their
//   attn_combine   max and exp-sum, the weighted V sum; then the chunks are
//                  merged per head (the softmax of the reference, computed in
//                  pieces)
//   argmax         one workgroup; ties to the lower index, NaN never wins
//                  except at index 0 (InferenceEngine.swift:550-555);
//                  advances the device-side position
#include <hip/hip_runtime.h>

#include "device.hpp"
#include "internal.hpp"

namespace m1moe {
namespace {

constexpr int kMvRows = 2;        // matvec rows per wave
constexpr int kAttnChunk = 256;   // positions per attention workgroup

// Sum over a workgroup of `nw` waves; every thread gets the total (waves
// added in order).
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
__device__ __forceinline__ float block_max(float v, float* s_red, int nw) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    v = wave_max(v);
    if (lane == 0) s_red[wave] = v;
    __syncthreads();
    float t = -INFINITY;
    for (int w = 0; w < nw; ++w) t = fmaxf(t, s_red[w]);
    __syncthreads();
    return t;
}

// ---- embedding ----------------------------------------------------------------------

__global__ __launch_bounds__(256) void embed_kernel(DenseStepArgs a) {
    int t = *a.token;
    if (t < 0 || t >= a.vocab) {
        if (blockIdx.x == 0 && threadIdx.x == 0) flag_error(a.err, 16u);
        t = 0;
    }
    const uint16_t* row = a.embed + (size_t)t * a.h;
    for (int d = blockIdx.x * 256 + threadIdx.x; d < a.h; d += gridDim.x * 256)
        a.x_out[d] = bf16_to_f32(row[d]);
}

// ---- RMSNorm ------------------------------------------------------------------------

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

// ---- bf16 matvec --------------------------------------------------------------------

// Row `row` of the concatenated segments: its weight row, output and residual.
__device__ __forceinline__ const MvSeg& mv_seg(const MvArgs& a, int row, int& local) {
    if (row < a.seg[0].rows) {
        local = row;
        return a.seg[0];
    }
    if (row < a.seg[0].rows + a.seg[1].rows) {
        local = row - a.seg[0].rows;
        return a.seg[1];
    }
    local = row - a.seg[0].rows - a.seg[1].rows;
    return a.seg[2];
}

// Lane l takes columns 8l .. 8l+7 of each 512-column block; four blocks of
// loads are in flight together.
__global__ __launch_bounds__(256) void matvec_bf16_kernel(MvArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r0 = (blockIdx.x * 4 + wave) * kMvRows;
    if (r0 >= a.rows) return;
    const uint16_t* wr[kMvRows];
    int loc[kMvRows];
#pragma unroll
    for (int i = 0; i < kMvRows; ++i) {
        const int row = min(r0 + i, a.rows - 1);
        const MvSeg& sg = mv_seg(a, row, loc[i]);
        wr[i] = sg.w + (size_t)loc[i] * a.cols;
    }
    float acc[kMvRows];
#pragma unroll
    for (int i = 0; i < kMvRows; ++i) acc[i] = 0.f;
    constexpr int U = 4;
    for (int c0 = 0; c0 < a.cols; c0 += 512 * U) {
        uint4 wv[U][kMvRows];
        float4 x0[U], x1[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = min(c0 + 512 * u + 8 * lane, a.cols - 8);
#pragma unroll
            for (int i = 0; i < kMvRows; ++i) wv[u][i] = *reinterpret_cast<const uint4*>(wr[i] + c);
            x0[u] = *reinterpret_cast<const float4*>(a.x + c);
            x1[u] = *reinterpret_cast<const float4*>(a.x + c + 4);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c0 + 512 * u + 8 * lane >= a.cols) continue;
            const float xs[8] = {x0[u].x, x0[u].y, x0[u].z, x0[u].w, x1[u].x, x1[u].y, x1[u].z, x1[u].w};
#pragma unroll
            for (int i = 0; i < kMvRows; ++i)
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[i] = fmaf(bf16x8_at(wv[u][i], k), xs[k], acc[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < kMvRows; ++i) {
        const float v = wave_sum(acc[i]);
        const int row = r0 + i;
        if (lane == 0 && row < a.rows) {
            int l;
            const MvSeg& sg = mv_seg(a, row, l);
            sg.y[l] = sg.res ? sg.res[l] + v : v;
        }
    }
}

// ---- q/k norm, RoPE, KV store --------------------------------------------------------

// Workgroup b < num_heads: q head b; else k head (and v head) b - num_heads.
// Thread d < head_dim holds element d.
__global__ __launch_bounds__(256) void qk_rope_kv_kernel(DenseStepArgs a, int layer) {
    __shared__ float s_x[256];
    __shared__ float s_red[4];
    const int pos = *a.pos;
    if (pos >= a.max_seq) {
        if (blockIdx.x == 0 && threadIdx.x == 0) flag_error(a.err, 32u);
        return;
    }
    const int hd = a.head_dim, half = hd / 2;
    const bool is_q = (int)blockIdx.x < a.num_heads;
    const int head = is_q ? blockIdx.x : blockIdx.x - a.num_heads;
    float* vec = (is_q ? a.q : a.k) + (size_t)head * hd;
    const int d = threadIdx.x;
    float x = d < hd ? vec[d] : 0.f;
    if (a.qk_norm) {
        // InferenceEngine.swift:538-548: x *= rms * w[d], w of length head_dim
        const float ss = block_sum(x * x, s_red, 4);
        const float rms = 1.0f / sqrtf(ss / (float)hd + a.eps);
        const uint16_t* w = (is_q ? a.q_norm : a.k_norm) + (size_t)layer * hd;
        if (d < hd) x *= rms * bf16_to_f32(w[d]);
    }
    if (d < hd) s_x[d] = x;
    __syncthreads();
    // RoPE (InferenceEngine.swift:521-536): pairs (p, p + hd/2)
    const size_t kvd = (size_t)a.num_kv_heads * hd;
    if (d < half) {
        const float freq = 1.0f / powf(a.rope_theta, (float)(2 * d) / (float)hd);
        const float angle = (float)pos * freq;
        const float c = cosf(angle), s = sinf(angle);
        const float x0 = s_x[d], x1 = s_x[d + half];
        const float y0 = x0 * c - x1 * s, y1 = x0 * s + x1 * c;
        if (is_q) {
            vec[d] = y0;
            vec[d + half] = y1;
        } else {
            float* kc = a.kcache + (size_t)layer * a.max_seq * kvd + (size_t)pos * kvd + (size_t)head * hd;
            kc[d] = y0;
            kc[d + half] = y1;
        }
    }
    if (!is_q && d < hd) {
        float* vc = a.vcache + (size_t)layer * a.max_seq * kvd + (size_t)pos * kvd + (size_t)head * hd;
        vc[d] = a.v[(size_t)head * hd + d];
    }
}

// ---- attention ----------------------------------------------------------------------

// Workgroup (head, chunk): positions chunk*256 .. +255 of the first seq.
// Thread t scores position p0 + t; thread d < head_dim sums V column d.
// Writes (max, exp-sum, acc[head_dim]) of the chunk, or max = -inf if empty.
__global__ __launch_bounds__(256) void attn_partial_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) float s_q[256];
    __shared__ float s_e[kAttnChunk];
    __shared__ float s_red[4];
    const int head = blockIdx.x, chunk = blockIdx.y;
    const int seq = a.seq_ptr ? min(*a.seq_ptr + 1, a.max_seq) : a.seq_len;
    const int hd = a.head_dim;
    const int p0 = chunk * kAttnChunk;
    float* part = a.partial + ((size_t)head * gridDim.y + chunk) * (hd + 2);
    if (p0 >= seq) {
        if (threadIdx.x == 0) {
            part[0] = -INFINITY;
            part[1] = 0.f;
        }
        return;
    }
    const int kvh = head / a.hpkv;
    const size_t kvd = (size_t)a.num_kv_heads * hd;
    if ((int)threadIdx.x < hd) s_q[threadIdx.x] = a.q[(size_t)head * hd + threadIdx.x];
    __syncthreads();
    const int p = p0 + threadIdx.x;
    float s = -INFINITY;
    if (p < seq) {
        const float4* kp = reinterpret_cast<const float4*>(a.kcache + (size_t)p * kvd + (size_t)kvh * hd);
        const float4* qp = reinterpret_cast<const float4*>(s_q);
        float acc = 0.f;
        for (int i = 0; i < hd / 4; ++i) {
            const float4 k4 = kp[i], q4 = qp[i];
            acc = fmaf(q4.x, k4.x, acc);
            acc = fmaf(q4.y, k4.y, acc);
            acc = fmaf(q4.z, k4.z, acc);
            acc = fmaf(q4.w, k4.w, acc);
        }
        s = acc * a.scale;
    }
    const float m = block_max(s, s_red, 4);
    const float e = p < seq ? expf(s - m) : 0.f;
    s_e[threadIdx.x] = e;
    const float l = block_sum(e, s_red, 4);  // (its barriers also publish s_e)
    if ((int)threadIdx.x < hd) {
        const int np = min(kAttnChunk, seq - p0);
        const float* vp = a.vcache + (size_t)p0 * kvd + (size_t)kvh * hd + threadIdx.x;
        float acc = 0.f;
        for (int t = 0; t < np; ++t) acc = fmaf(s_e[t], vp[(size_t)t * kvd], acc);
        part[2 + threadIdx.x] = acc;
    }
    if (threadIdx.x == 0) {
        part[0] = m;
        part[1] = l;
    }
}

// Workgroup per head, thread d < head_dim: out = sum_c acc_c e^(m_c - M) / L.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a, int nchunks) {
    const int head = blockIdx.x, d = threadIdx.x, hd = a.head_dim;
    if (d >= hd) return;
    const float* part = a.partial + (size_t)head * nchunks * (hd + 2);
    float M = -INFINITY;
    for (int c = 0; c < nchunks; ++c) M = fmaxf(M, part[(size_t)c * (hd + 2)]);
    float L = 0.f, acc = 0.f;
    for (int c = 0; c < nchunks; ++c) {
        const float* pc = part + (size_t)c * (hd + 2);
        if (pc[0] == -INFINITY) continue;
        const float f = expf(pc[0] - M);
        L = fmaf(pc[1], f, L);
        acc = fmaf(pc[2 + d], f, acc);
    }
    a.out[(size_t)head * hd + d] = acc / L;
}

// ---- argmax -------------------------------------------------------------------------

// (value, index) pairs: larger value wins, ties to the lower index.
__device__ __forceinline__ bool am_better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

__global__ __launch_bounds__(1024) void argmax_kernel(const float* x, int n, int32_t* out,
                                                      int32_t* pos, int max_seq) {
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
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (am_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
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
        // the reference's scan starts from x[0] with a strict >, so a NaN
        // there is never replaced; all NaN also gives 0
        *out = (bi < n && !__builtin_isnan(x[0])) ? bi : 0;
        if (pos && *pos < max_seq) *pos += 1;
    }
}

__global__ void set_i32_kernel(int32_t* p, int32_t v) { *p = v; }

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

int launch_matvec_bf16(const MvArgs& a, void* stream) {
    if (a.cols % 8 || a.rows <= 0) return (int)hipErrorInvalidValue;
    const int per_wg = 4 * kMvRows;
    hipLaunchKernelGGL(matvec_bf16_kernel, dim3((unsigned)((a.rows + per_wg - 1) / per_wg)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), a);
    return (int)hipGetLastError();
}

int launch_attention(const AttnArgs& a, int max_positions, void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int nchunks = (max_positions + kAttnChunk - 1) / kAttnChunk;
    hipLaunchKernelGGL(attn_partial_kernel, dim3((unsigned)a.num_heads, (unsigned)nchunks), dim3(256), 0,
                       st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)a.num_heads), dim3(256), 0, st, a, nchunks);
    return (int)hipGetLastError();
}

int attention_partial_floats(int num_heads, int head_dim, int max_positions) {
    return num_heads * ((max_positions + kAttnChunk - 1) / kAttnChunk) * (head_dim + 2);
}

int launch_argmax(const float* x, int n, int32_t* out, int32_t* pos, int max_seq, void* stream) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream), x, n, out,
                       pos, max_seq);
    return (int)hipGetLastError();
}

int launch_embed(const DenseStepArgs& a, void* stream) {
    hipLaunchKernelGGL(embed_kernel, dim3((unsigned)((a.h + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), a);
    return (int)hipGetLastError();
}

int launch_qk_rope_kv(const DenseStepArgs& a, int layer, void* stream) {
    hipLaunchKernelGGL(qk_rope_kv_kernel, dim3((unsigned)(a.num_heads + a.num_kv_heads)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), a, layer);
    return (int)hipGetLastError();
}

}  // namespace m1moe
