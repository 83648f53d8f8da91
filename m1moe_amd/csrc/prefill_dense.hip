// prefill_dense.hip — the dense part of the decoder for T prompt tokens at once.
//
// The reference forwards a prompt token by token (Sources/bench/main.swift:
// 139-141, Sources/chat/main.swift:143-149), so every weight is read once
// per token.  Here each layer's dense work for the T tokens is one pass over
// its weights:
//
//   embed_rows     the token rows of the bf16 embedding -> f32 [T][h]
//                  (InferenceEngine.swift:482-488)
//   rmsnorm_rows   x * rsqrt(mean(x^2) + eps) * w per row (Shaders.metal:96-134)
//   gemm_kernel    Y[T][N] = X[T][K] W[N][K]^T (+ R) on v_mfma_f32_16x16x4f32:
//                  bf16 weights widened to f32 in LDS, f32 activations, f32
//                  accumulation (the arithmetic of matvecBF16, Shaders.metal:
//                  328-358, in another order)
//   rope_kv_rows   per token and head: the per-head q/k RMSNorm and RoPE at
//                  the token's position (InferenceEngine.swift:521-548), k and
//                  v rows into the caches (:215-220)
//   attn_mfma      causal attention of the T queries over positions 0 .. their
//                  own (Shaders.metal:209-326 for every token) on f32 MFMA,
//                  online softmax over key blocks staged in LDS (head_dim 64,
//                  128; attn_causal, on the SIMD units, for head_dim 256)
//
// The MoE block runs through the grouped prefill (prefill.hip).
#include <hip/hip_runtime.h>

#include "device.hpp"
#include "internal.hpp"

namespace m1moe {
namespace {

typedef float f32x4v __attribute__((ext_vector_type(4)));

// ---- embedding and row norms ----------------------------------------------------------

__global__ __launch_bounds__(256) void embed_rows_kernel(PfDenseArgs a) {
    const int t = blockIdx.x;
    int tok = a.tokens[t];
    if (tok < 0 || tok >= a.vocab) {
        if (threadIdx.x == 0) flag_error(a.err, 16u);
        tok = 0;
    }
    const uint16_t* row = a.embed + (size_t)tok * a.h;
    float* out = a.res + (size_t)t * a.h;
    for (int d = threadIdx.x; d < a.h; d += 256) out[d] = bf16_to_f32(row[d]);
}

// One workgroup per row: out = x * rsqrt(sum(x^2) / n + eps) * w.
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float* x, const uint16_t* w,
                                                           float* out, int n, float eps) {
    __shared__ float s_red[4];
    const float* xr = x + (size_t)blockIdx.x * n;
    float* o = out + (size_t)blockIdx.x * n;
    float acc = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) acc = fmaf(xr[i], xr[i], acc);
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = acc;
    __syncthreads();
    const float ss = ((s_red[0] + s_red[1]) + s_red[2]) + s_red[3];
    const float rms = rsqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256) o[i] = xr[i] * rms * bf16_to_f32(w[i]);
}

// ---- GEMM on f32 MFMA -------------------------------------------------------------------

// v_mfma_f32_16x16x4f32: A 16x4 (lane l: row l%16, k l/16), B 4x16 (lane l:
// column l%16, k l/16), D 16x16 (lane l: column l%16, rows 4(l/16) .. +3).
// Workgroup tile 64 (tokens) x 64 (weight rows), k-steps of 32; wave w owns
// the 32 x 32 quarter (w/2, w%2) as 2 x 2 MFMA tiles.  The next k-step's
// global loads are issued before the current one is computed.
constexpr int kGM = 64, kGN = 64, kGK = 32;

__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g) {
    __shared__ float sA[kGM][kGK + 1];
    __shared__ float sB[kGN][kGK + 1];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int m0 = blockIdx.y * kGM, n0 = blockIdx.x * kGN;
    const int lr = tid >> 2, lc = (tid & 3) * 8;  // loader: row, 8 columns
    const float* arow = g.A + (size_t)min(m0 + lr, g.M - 1) * g.lda + lc;
    const uint16_t* brow = g.W + (size_t)min(n0 + lr, g.N - 1) * g.K + lc;
    float4 a0, a1;
    uint4 b;
    auto load = [&](int k0) {
        a0 = *reinterpret_cast<const float4*>(arow + k0);
        a1 = *reinterpret_cast<const float4*>(arow + k0 + 4);
        b = *reinterpret_cast<const uint4*>(brow + k0);
    };
    f32x4v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    const int r16 = lane & 15, k4 = lane >> 4;
    load(0);
    for (int k0 = 0; k0 < g.K; k0 += kGK) {
        sA[lr][lc + 0] = a0.x, sA[lr][lc + 1] = a0.y, sA[lr][lc + 2] = a0.z, sA[lr][lc + 3] = a0.w;
        sA[lr][lc + 4] = a1.x, sA[lr][lc + 5] = a1.y, sA[lr][lc + 6] = a1.z, sA[lr][lc + 7] = a1.w;
#pragma unroll
        for (int e = 0; e < 8; ++e) sB[lr][lc + e] = bf16x8_at(b, e);
        __syncthreads();
        if (k0 + kGK < g.K) load(k0 + kGK);
#pragma unroll
        for (int kk = 0; kk < kGK; kk += 4) {
            float av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) av[i] = sA[wm + 16 * i + r16][kk + k4];
#pragma unroll
            for (int j = 0; j < 2; ++j) bv[j] = sB[wn + 16 * j + r16][kk + k4];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn + 16 * j + r16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm + 16 * i + 4 * k4 + r;
                if (m < g.M && n < g.N) {
                    float v = acc[i][j][r];
                    if (g.R) v += g.R[(size_t)m * g.ldc + n];
                    g.C[(size_t)m * g.ldc + n] = v;
                }
            }
        }
}

// ---- q/k norm, RoPE, KV rows ----------------------------------------------------------

// Workgroup (t, head): head < num_heads: q head, rotated in place; else kv
// head: k normalised and rotated, k and v stored at cache row p0 + t.
template <int HD>
__global__ __launch_bounds__(64) void rope_kv_rows_kernel(PfDenseArgs a) {
    __shared__ float s_v[HD];
    const int t = blockIdx.x, head = blockIdx.y, lane = threadIdx.x;
    const int p = *a.pos + t;
    const bool is_q = head < a.num_heads;
    const int kvh = head - a.num_heads;
    float* row = a.qkv + (size_t)t * a.ldqkv;
    float* vec = is_q ? row + (size_t)head * HD : row + a.qd + (size_t)kvh * HD;
    const uint16_t* nw = is_q ? a.q_norm : a.k_norm;
    if (p >= a.max_seq) {
        if (lane == 0 && head == 0) flag_error(a.err, 32u);
        return;
    }
    float v[HD / 64];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < HD / 64; ++j) {
        v[j] = vec[lane + 64 * j];
        ss = fmaf(v[j], v[j], ss);
    }
    if (nw) {
        const float rms = 1.0f / sqrtf(wave_sum(ss) / (float)HD + a.eps);
#pragma unroll
        for (int j = 0; j < HD / 64; ++j) v[j] *= rms * bf16_to_f32(nw[lane + 64 * j]);
    }
#pragma unroll
    for (int j = 0; j < HD / 64; ++j) s_v[lane + 64 * j] = v[j];
    __syncthreads();
    float* dst = is_q ? vec : a.kcache + (size_t)p * a.kvd + (size_t)kvh * HD;
    for (int d = lane; d < HD / 2; d += 64) {
        const float freq = 1.0f / powf(a.rope_theta, (float)(2 * d) / (float)HD);
        const float ang = (float)p * freq;
        const float cs = cosf(ang), sn = sinf(ang);
        const float x0 = s_v[d], x1 = s_v[d + HD / 2];
        dst[d] = x0 * cs - x1 * sn;
        dst[d + HD / 2] = x0 * sn + x1 * cs;
    }
    if (!is_q) {
        const float* vsrc = row + a.qd + a.kvd + (size_t)kvh * HD;
        float* vdst = a.vcache + (size_t)p * a.kvd + (size_t)kvh * HD;
        for (int d = lane; d < HD; d += 64) vdst[d] = vsrc[d];
    }
}

// ---- causal attention ------------------------------------------------------------------

// Workgroup (head, 16 queries): thread (q = tid/16, j = tid%16).  Key blocks
// of KB = 4096/HD positions are staged in LDS; thread j scores keys j, j+16,
// ... of its query, the 16 threads of a query reduce max and sum, then
// accumulate dims j, j+16, ... of the output.  Queries at positions p0+t see
// keys 0 .. p0+t.
template <int HD>
__global__ __launch_bounds__(256) void attn_causal_kernel(PfDenseArgs a) {
    constexpr int QB = 16, KB = 4096 / HD, KPT = KB / 16, DPT = HD / 16;
    __shared__ __attribute__((aligned(16))) float sQ[QB][HD];
    __shared__ float sK[KB][HD + 1];
    __shared__ __attribute__((aligned(16))) float sV[KB][HD];
    __shared__ float sP[QB][KB];
    const int h = blockIdx.x, tb = blockIdx.y * QB;
    const int tid = threadIdx.x, qi = tid >> 4, j = tid & 15;
    const int p0 = *a.pos;
    const int kvh = h / a.hpkv;
    const int t = tb + qi;
    const bool live = t < a.T;
    const int qpos = min(p0 + t, a.max_seq - 1);
    const int last = min(p0 + min(tb + QB, a.T) - 1, a.max_seq - 1);  // the block's last query position
    for (int e = tid; e < QB * HD; e += 256) {
        const int r = e / HD, d = e - r * HD;
        sQ[r][d] = tb + r < a.T ? a.qkv[(size_t)(tb + r) * a.ldqkv + (size_t)h * HD + d] : 0.f;
    }
    float m = -INFINITY, l = 0.f, acc[DPT];
#pragma unroll
    for (int e = 0; e < DPT; ++e) acc[e] = 0.f;
    for (int k0 = 0; k0 <= last; k0 += KB) {
        __syncthreads();  // (sQ published; the previous block's sK/sV/sP consumed)
        for (int e = tid; e < KB * HD / 4; e += 256) {
            const int r = e / (HD / 4), d = (e - r * (HD / 4)) * 4;
            const int kp = min(k0 + r, last);
            const size_t off = (size_t)kp * a.kvd + (size_t)kvh * HD + d;
            const float4 kv = *reinterpret_cast<const float4*>(a.kcache + off);
            const float4 vv = *reinterpret_cast<const float4*>(a.vcache + off);
            sK[r][d] = kv.x, sK[r][d + 1] = kv.y, sK[r][d + 2] = kv.z, sK[r][d + 3] = kv.w;
            *reinterpret_cast<float4*>(&sV[r][d]) = vv;
        }
        __syncthreads();
        float s[KPT];
        float bm = -INFINITY;
#pragma unroll
        for (int e = 0; e < KPT; ++e) {
            const int kk = j + 16 * e;
            float d = 0.f;
#pragma unroll 8
            for (int c = 0; c < HD; ++c) d = fmaf(sQ[qi][c], sK[kk][c], d);
            s[e] = (live && k0 + kk <= qpos) ? d * a.scale : -INFINITY;
            bm = fmaxf(bm, s[e]);
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) bm = fmaxf(bm, __shfl_xor(bm, o));
        const float mn = fmaxf(m, bm);
        const float f = m == -INFINITY ? 0.f : expf(m - mn);
        float ls = 0.f;
#pragma unroll
        for (int e = 0; e < KPT; ++e) {
            const float pe = s[e] == -INFINITY ? 0.f : expf(s[e] - mn);
            sP[qi][j + 16 * e] = pe;
            ls += pe;
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) ls += __shfl_xor(ls, o);
        l = fmaf(l, f, ls);
        m = mn;
#pragma unroll
        for (int e = 0; e < DPT; ++e) acc[e] *= f;
        __syncthreads();  // sP complete
        for (int kk = 0; kk < KB; ++kk) {
            const float pk = sP[qi][kk];
#pragma unroll
            for (int e = 0; e < DPT; ++e) acc[e] = fmaf(pk, sV[kk][j + 16 * e], acc[e]);
        }
    }
    if (live) {
        float* out = a.attn + (size_t)t * a.qd + (size_t)h * HD;
#pragma unroll
        for (int e = 0; e < DPT; ++e) out[j + 16 * e] = acc[e] / l;
    }
}

__global__ void advance_pos_kernel(int32_t* pos, int32_t by, int32_t max_seq) {
    *pos = min(*pos + by, max_seq);
}

}  // namespace

int launch_pf_embed(const PfDenseArgs& a, void* stream) {
    hipLaunchKernelGGL(embed_rows_kernel, dim3((unsigned)a.T), dim3(256), 0, static_cast<hipStream_t>(stream), a);
    return (int)hipGetLastError();
}

int launch_rmsnorm_rows(const float* x, const uint16_t* w, float* out, int rows, int n, float eps,
                        void* stream) {
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3((unsigned)rows), dim3(256), 0, static_cast<hipStream_t>(stream),
                       x, w, out, n, eps);
    return (int)hipGetLastError();
}

int launch_gemm(const GemmArgs& g, void* stream) {
    if (g.K % kGK || g.M <= 0 || g.N <= 0 || g.lda % 4) return (int)hipErrorInvalidValue;
    const dim3 grid((unsigned)((g.N + kGN - 1) / kGN), (unsigned)((g.M + kGM - 1) / kGM));
    hipLaunchKernelGGL(gemm_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), g);
    return (int)hipGetLastError();
}

int launch_pf_rope_kv(const PfDenseArgs& a, void* stream) {
    const dim3 grid((unsigned)a.T, (unsigned)(a.num_heads + a.num_kv_heads));
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (a.head_dim) {
        case 64: hipLaunchKernelGGL(rope_kv_rows_kernel<64>, grid, dim3(64), 0, st, a); break;
        case 128: hipLaunchKernelGGL(rope_kv_rows_kernel<128>, grid, dim3(64), 0, st, a); break;
        case 256: hipLaunchKernelGGL(rope_kv_rows_kernel<256>, grid, dim3(64), 0, st, a); break;
        default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

// Causal attention on v_mfma_f32_16x16x4f32 (f32 operands and accumulation;
// head_dim 64 or 128).  Workgroup = (head, 64 queries), wave = 16 queries.
// Keys go in blocks of 32 through LDS, shared by the four waves: K row-major,
// V transposed.  Per block a wave computes S = Q K^T (16 x 32), updates each
// query row's running max and sum (the softmax of Shaders.metal:245-289 in
// pieces), writes P = e^(S - m) to LDS and reads it back as the A operand of
// O += P V.  Contraction orders: in k-step 4t+u lane (r, kq) supplies dim (or
// key) 16t + 4kq + u, so each lane's four steps read 16 contiguous bytes.
template <int HD>
__global__ __launch_bounds__(256) void attn_mfma_kernel(PfDenseArgs a) {
    constexpr int QW = 16, QB = 64, KB = 32;
    constexpr int NT = HD / 16;  // 16-wide dim groups: Q K^T k-step groups, output blocks
    __shared__ __attribute__((aligned(16))) float sK[KB][HD + 4];
    __shared__ __attribute__((aligned(16))) float sVt[HD][KB + 4];
    __shared__ __attribute__((aligned(16))) float sP[4][QW][KB + 4];
    const int h = blockIdx.x, tb = blockIdx.y * QB;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, kq = lane >> 4;
    const int p0 = *a.pos;
    const int kvh = h / a.hpkv;
    const int qw0 = tb + wave * QW;  // the wave's first query (token index)
    // the workgroup's last query position (keys beyond it are never needed)
    const int last = min(p0 + min(tb + QB, a.T) - 1, a.max_seq - 1);

    // Q as the A operand: row lr, dims 16t + 4kq .. +3
    f32x4v qa[NT];
    {
        const int t = min(qw0 + lr, a.T - 1);
        const float* q = a.qkv + (size_t)t * a.ldqkv + (size_t)h * HD + 4 * kq;
#pragma unroll
        for (int t4 = 0; t4 < NT; ++t4) qa[t4] = *reinterpret_cast<const f32x4v*>(q + 16 * t4);
    }
    // this lane's output rows: queries qw0 + 4kq + i
    int qpos[4];
    bool qlive[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = qw0 + 4 * kq + i;
        qlive[i] = t < a.T;
        qpos[i] = min(p0 + t, a.max_seq - 1);
    }
    float m[4], l[4];
    f32x4v acc[NT];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m[i] = -INFINITY;
        l[i] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[j] = f32x4v{0.f, 0.f, 0.f, 0.f};
    const int wlast = min(p0 + min(qw0 + QW, a.T) - 1, a.max_seq - 1);  // this wave's last

    for (int k0 = 0; k0 <= last; k0 += KB) {
        __syncthreads();  // the previous block's sK / sVt consumed
        // K rows: thread -> (key r, 4 dims c); V: (key r fastest) -> sVt[dims][r]
        for (int e = tid; e < KB * HD / 4; e += 256) {
            const int r = e / (HD / 4), c = (e - r * (HD / 4)) * 4;
            const int kp = min(k0 + r, last);
            *reinterpret_cast<float4*>(&sK[r][c]) = *reinterpret_cast<const float4*>(
                a.kcache + (size_t)kp * a.kvd + (size_t)kvh * HD + c);
            const int rv = e % KB, cv = (e / KB) * 4;
            const int kv = min(k0 + rv, last);
            const float4 v = *reinterpret_cast<const float4*>(a.vcache + (size_t)kv * a.kvd +
                                                              (size_t)kvh * HD + cv);
            sVt[cv + 0][rv] = v.x;
            sVt[cv + 1][rv] = v.y;
            sVt[cv + 2][rv] = v.z;
            sVt[cv + 3][rv] = v.w;
        }
        __syncthreads();
        if (k0 > wlast) continue;  // (uniform per wave) keys after every query of the wave

        // S = Q K^T: 2 blocks of 16 keys; lane: key 16nb + lr, queries 4kq + i
        f32x4v s[2];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            s[nb] = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t4 = 0; t4 < NT; ++t4) {
                const f32x4v kb = *reinterpret_cast<const f32x4v*>(&sK[16 * nb + lr][16 * t4 + 4 * kq]);
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    s[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[t4][u], kb[u], s[nb], 0, 0, 0);
            }
        }
        // online softmax per query row (the 16 lanes of a kq group hold its keys)
        float f[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float sv[2];
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                const int kp = k0 + 16 * nb + lr;
                sv[nb] = (qlive[i] && kp <= qpos[i]) ? s[nb][i] * a.scale : -INFINITY;
            }
            float bm = fmaxf(sv[0], sv[1]);
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) bm = fmaxf(bm, __shfl_xor(bm, o));
            const float mn = fmaxf(m[i], bm);
            f[i] = m[i] == -INFINITY ? 0.f : expf(m[i] - mn);
            float ls = 0.f;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                const float pe = sv[nb] == -INFINITY ? 0.f : expf(sv[nb] - mn);
                sP[wave][4 * kq + i][16 * nb + lr] = pe;
                ls += pe;
            }
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) ls += __shfl_xor(ls, o);
            l[i] = fmaf(l[i], f[i], ls);
            m[i] = mn;
        }
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[j][i] *= f[i];
        // O += P V: A = P (row lr, keys 16t + 4kq + u), B = V^T rows (dim 16j + lr)
#pragma unroll
        for (int t2 = 0; t2 < KB / 16; ++t2) {
            const f32x4v pa = *reinterpret_cast<const f32x4v*>(&sP[wave][lr][16 * t2 + 4 * kq]);
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const f32x4v vb = *reinterpret_cast<const f32x4v*>(&sVt[16 * j + lr][16 * t2 + 4 * kq]);
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[u], vb[u], acc[j], 0, 0, 0);
            }
        }
    }
    // lane: dims 16j + lr of queries 4kq + i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (!qlive[i]) continue;
        float* out = a.attn + (size_t)(qw0 + 4 * kq + i) * a.qd + (size_t)h * HD;
#pragma unroll
        for (int j = 0; j < NT; ++j) out[16 * j + lr] = acc[j][i] / l[i];
    }
}

int launch_pf_attention(const PfDenseArgs& a, void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid_m((unsigned)a.num_heads, (unsigned)((a.T + 63) / 64));
    const dim3 grid((unsigned)a.num_heads, (unsigned)((a.T + 15) / 16));
    switch (a.head_dim) {
        case 64: hipLaunchKernelGGL(attn_mfma_kernel<64>, grid_m, dim3(256), 0, st, a); break;
        case 128: hipLaunchKernelGGL(attn_mfma_kernel<128>, grid_m, dim3(256), 0, st, a); break;
        case 256: hipLaunchKernelGGL(attn_causal_kernel<256>, grid, dim3(256), 0, st, a); break;
        default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

int launch_advance_pos(int32_t* pos, int32_t by, int32_t max_seq, void* stream) {
    hipLaunchKernelGGL(advance_pos_kernel, dim3(1), dim3(1), 0, static_cast<hipStream_t>(stream), pos, by, max_seq);
    return (int)hipGetLastError();
}

}  // namespace m1moe
