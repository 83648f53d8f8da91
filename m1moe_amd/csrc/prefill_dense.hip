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
//   gemm_bf3       Y[T][N] = X[T][K] W[N][K]^T (+ R): f32 activations split
//                  exactly into three bf16 parts, each multiplied with the
//                  bf16 weights on v_mfma_f32_32x32x16_bf16 (exact products,
//                  f32 accumulation: the arithmetic of matvecBF16,
//                  Shaders.metal:328-358, in another order); gemm_kernel does
//                  the same on v_mfma_f32_16x16x4f32 for a K that is not a
//                  multiple of 64
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
// ---- GEMM on bf16 MFMA with the f32 input split three ways ---------------------------

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16v __attribute__((ext_vector_type(16)));

// Y[M][N] = X[M][K] W[N][K]^T (+ R), X f32, W bf16.  Each x is split exactly
// into three bf16 values, hi = x with the low 16 bits cleared, mid = (x - hi)
// likewise, lo = x - hi - mid (x has 24 significant bits: 8 + 8 + 8), when the
// X tile is staged in LDS; each part is multiplied with the bf16 weights on
// v_mfma_f32_32x32x16_bf16, whose products are exact, and accumulated in f32:
// the arithmetic of the f32 GEMM (exact products, f32 sums) at the bf16 rate.
// Tile BM tokens x BN weight rows (128 x 128, 64 x 128 or 64 x 64), k-blocks
// of 64; the next k-block's global loads are issued before the current one
// is multiplied.  Four waves, each TI x TJ tiles of 32 x 32.  MFMA operands:
// A = tokens (lane l: row l % 32, k 8 (l / 32) .. + 7), B = weight rows
// likewise; D element 4 v + i of lane l is token 8 v + 4 (l / 32) + i, weight
// row l % 32 of the tile.
constexpr int kBK = 64, kBP = kBK + 8;  // LDS rows padded to 144 bytes

template <int BM, int BN>
__global__ __launch_bounds__(256, 2) void gemm_bf3_kernel(GemmArgs g) {
    constexpr int TI = BM == 128 ? 2 : (BN == 128 ? 2 : 1);
    constexpr int TJ = BM == 128 ? 2 : 1;
    constexpr int WN = BN / (32 * TJ);              // waves along the weight rows
    static_assert((BM / (32 * TI)) * WN == 4, "four waves");
    constexpr int EA = BM * kBK / 256;              // X values staged per thread (32 or 16)
    constexpr int EW = BN * kBK / 256;              // W values staged per thread (32 or 16)
    __shared__ __attribute__((aligned(16))) uint16_t sX[3][BM][kBP];
    __shared__ __attribute__((aligned(16))) uint16_t sW[BN][kBP];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    // loaders: X row xr, columns xc .. xc + EA - 1; W row wr, columns wc .. wc + EW - 1
    const int xr = tid / (kBK / EA), xc = (tid % (kBK / EA)) * EA;
    const int wr = tid / (kBK / EW), wc = (tid % (kBK / EW)) * EW;
    const float* xrow = g.A + (size_t)min(m0 + xr, g.M - 1) * g.lda + xc;
    const int wrow_n = min(n0 + wr, g.N - 1);
    const uint16_t* wrow = !g.W1 || wrow_n < g.n1 ? g.W + (size_t)wrow_n * g.K + wc
                           : wrow_n < g.n2        ? g.W1 + (size_t)(wrow_n - g.n1) * g.K + wc
                                                  : g.W2 + (size_t)(wrow_n - g.n2) * g.K + wc;
    typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
    float4 xv[EA / 4];
    u32x4v wv[EW / 8];
    // hi / mid / lo parts of eight values, as bf16 bits packed two per word
    auto split8 = [&](const float (&v)[8], uint4& h, uint4& m, uint4& l) {
        uint32_t hb[8], mb[8], lb[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t u = __float_as_uint(v[e]);
            const float hi = __uint_as_float(u & 0xffff0000u);
            const float r = v[e] - hi;
            const float mid = __uint_as_float(__float_as_uint(r) & 0xffff0000u);
            const float lo = r - mid;
            hb[e] = __float_as_uint(hi) >> 16;
            mb[e] = __float_as_uint(mid) >> 16;
            lb[e] = __float_as_uint(lo) >> 16;
        }
        h = make_uint4(hb[0] | hb[1] << 16, hb[2] | hb[3] << 16, hb[4] | hb[5] << 16, hb[6] | hb[7] << 16);
        m = make_uint4(mb[0] | mb[1] << 16, mb[2] | mb[3] << 16, mb[4] | mb[5] << 16, mb[6] | mb[7] << 16);
        l = make_uint4(lb[0] | lb[1] << 16, lb[2] | lb[3] << 16, lb[4] | lb[5] << 16, lb[6] | lb[7] << 16);
    };
    f32x16v acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    const int wm = (wave / WN) * 32 * TI, wn = (wave % WN) * 32 * TJ;
    const int r32 = lane & 31, k8 = (lane >> 5) * 8;
    // this workgroup's k range: split blockIdx.z of gridDim.z, whole k-blocks
    const int nkb = g.K / kBK, S = (int)gridDim.z, z = (int)blockIdx.z;
    const int kbeg = (z * nkb / S) * kBK, kend = ((z + 1) * nkb / S) * kBK;
#pragma unroll
    for (int i = 0; i < EA / 4; ++i) xv[i] = *reinterpret_cast<const float4*>(xrow + kbeg + 4 * i);
#pragma unroll
    for (int i = 0; i < EW / 8; ++i) wv[i] = *reinterpret_cast<const u32x4v*>(wrow + kbeg + 8 * i);
    for (int k0 = kbeg; k0 < kend; k0 += kBK) {
#pragma unroll
        for (int c = 0; c < EA / 8; ++c) {
            float v[8];
            v[0] = xv[2 * c].x, v[1] = xv[2 * c].y, v[2] = xv[2 * c].z, v[3] = xv[2 * c].w;
            v[4] = xv[2 * c + 1].x, v[5] = xv[2 * c + 1].y, v[6] = xv[2 * c + 1].z, v[7] = xv[2 * c + 1].w;
            uint4 h, m, l;
            split8(v, h, m, l);
            *reinterpret_cast<uint4*>(&sX[0][xr][xc + 8 * c]) = h;
            *reinterpret_cast<uint4*>(&sX[1][xr][xc + 8 * c]) = m;
            *reinterpret_cast<uint4*>(&sX[2][xr][xc + 8 * c]) = l;
        }
#pragma unroll
        for (int c = 0; c < EW / 8; ++c) *reinterpret_cast<u32x4v*>(&sW[wr][wc + 8 * c]) = wv[c];
        __syncthreads();
        if (k0 + kBK < kend) {
            const int k1 = k0 + kBK;
#pragma unroll
            for (int i = 0; i < EA / 4; ++i) xv[i] = *reinterpret_cast<const float4*>(xrow + k1 + 4 * i);
#pragma unroll
            for (int i = 0; i < EW / 8; ++i) wv[i] = *reinterpret_cast<const u32x4v*>(wrow + k1 + 8 * i);
        }
#pragma unroll
        for (int ks = 0; ks < kBK; ks += 16) {
            bf16x8 b[TJ];
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                b[j] = *reinterpret_cast<const bf16x8*>(&sW[wn + 32 * j + r32][ks + k8]);
#pragma unroll
            for (int p = 0; p < 3; ++p)
#pragma unroll
                for (int i = 0; i < TI; ++i) {
                    const bf16x8 a = *reinterpret_cast<const bf16x8*>(&sX[p][wm + 32 * i + r32][ks + k8]);
#pragma unroll
                    for (int j = 0; j < TJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b[j], acc[i][j], 0, 0, 0);
                }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int n = n0 + wn + 32 * j + r32;
#pragma unroll
            for (int v = 0; v < 4; ++v)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = m0 + wm + 32 * i + 8 * v + 4 * (lane >> 5) + r;
                    if (m < g.M && n < g.N) {
                        float y = acc[i][j][4 * v + r];
                        if (S > 1) {
                            g.part[((size_t)z * g.M + m) * g.N + n] = y;
                        } else {
                            if (g.R) y += g.R[(size_t)m * g.ldc + n];
                            g.C[(size_t)m * g.ldc + n] = y;
                        }
                    }
                }
        }
}

// C = sum over s = 0 .. S-1 of the split-K partials (in that order) + R; four
// columns per thread (N, ldc and the C / R addresses are multiples of 4).
__global__ __launch_bounds__(256) void splitk_sum_kernel(GemmArgs g) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t mn4 = (size_t)g.M * g.N / 4;
    if (i >= mn4) return;
    const float4* p = reinterpret_cast<const float4*>(g.part);
    float4 y = p[i];
    for (int z = 1; z < g.splits; ++z) {
        const float4 q = p[(size_t)z * mn4 + i];
        y.x += q.x, y.y += q.y, y.z += q.z, y.w += q.w;
    }
    const size_t m = 4 * i / g.N, n = 4 * i % g.N;
    if (g.R) {
        const float4 r = *reinterpret_cast<const float4*>(g.R + m * g.ldc + n);
        y.x += r.x, y.y += r.y, y.z += r.z, y.w += r.w;
    }
    *reinterpret_cast<float4*>(g.C + m * g.ldc + n) = y;
}

// The same sum for one output row per workgroup (at most kSumNormSplits
// splits), then that row's RMSNorm with the arithmetic of rmsnorm_rows_kernel
// (each thread's squares summed in its own column order, four at a time).
constexpr int kSumNormSplits = 8;
__global__ __launch_bounds__(256) void splitk_sum_norm_kernel(GemmArgs g) {
    __shared__ float s_red[4];
    const size_t m = blockIdx.x, mn4 = (size_t)g.M * g.N / 4;
    const float4* p = reinterpret_cast<const float4*>(g.part) + m * (g.N / 4);
    float* c = g.C + m * g.ldc;
    float acc = 0.f;
    for (int i = threadIdx.x; i < g.N / 4; i += 256) {
        float4 v[kSumNormSplits];  // every split's load in flight together
#pragma unroll
        for (int z = 0; z < kSumNormSplits; ++z)
            if (z < g.splits) v[z] = p[(size_t)z * mn4 + i];
        float4 y = v[0];
#pragma unroll
        for (int z = 1; z < kSumNormSplits; ++z)
            if (z < g.splits) y.x += v[z].x, y.y += v[z].y, y.z += v[z].z, y.w += v[z].w;
        if (g.R) {
            const float4 r = *reinterpret_cast<const float4*>(g.R + m * g.ldc + 4 * i);
            y.x += r.x, y.y += r.y, y.z += r.z, y.w += r.w;
        }
        *reinterpret_cast<float4*>(c + 4 * i) = y;
        acc = fmaf(y.x, y.x, acc);
        acc = fmaf(y.y, y.y, acc);
        acc = fmaf(y.z, y.z, acc);
        acc = fmaf(y.w, y.w, acc);
    }
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = acc;
    __syncthreads();
    const float ss = ((s_red[0] + s_red[1]) + s_red[2]) + s_red[3];
    const float rms = rsqrtf(ss / (float)g.N + g.norm_eps);
    float* o = g.norm_out + m * g.ldc;
    for (int i = threadIdx.x; i < g.N; i += 256) o[i] = c[i] * rms * bf16_to_f32(g.norm_w[i]);
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
    if (g.W1 && (g.K % kBK || !g.W2 || g.n1 < 0 || g.n1 > g.n2 || g.n2 > g.N))
        return (int)hipErrorInvalidValue;
    if (g.norm_w && (!g.norm_out || g.ldc != g.N)) return (int)hipErrorInvalidValue;
    hipStream_t st = static_cast<hipStream_t>(stream);
    int splits = 1;
    if (g.K % kBK) {  // f32 MFMA for a K that is not a multiple of 64
        const dim3 grid((unsigned)((g.N + kGN - 1) / kGN), (unsigned)((g.M + kGM - 1) / kGM));
        hipLaunchKernelGGL(gemm_kernel, grid, dim3(256), 0, st, g);
    } else {
        // the largest tile that still gives at least one workgroup per CU
        const long gm128 = (g.M + 127) / 128, gm64 = (g.M + 63) / 64;
        const long gn128 = (g.N + 127) / 128, gn64 = (g.N + 63) / 64;
        if (gn128 * gm128 >= 256) {
            hipLaunchKernelGGL((gemm_bf3_kernel<128, 128>), dim3((unsigned)gn128, (unsigned)gm128),
                               dim3(256), 0, st, g);
        } else if (gn128 * gm64 >= 256) {
            hipLaunchKernelGGL((gemm_bf3_kernel<64, 128>), dim3((unsigned)gn128, (unsigned)gm64),
                               dim3(256), 0, st, g);
        } else {
            // Too few 64 x 64 tiles to fill the chip: split the k-blocks over
            // gridDim.z (at least 4 per split, at most 512 workgroups in all)
            // and sum the partials in a fixed order, so results do not depend
            // on timing.
            const long tiles = gn64 * gm64, nkb = g.K / kBK;
            long S = 768 / tiles < nkb / 4 ? 768 / tiles : nkb / 4;
            const bool aligned = g.N % 4 == 0 && g.ldc % 4 == 0 && (uintptr_t)g.C % 16 == 0 &&
                                 (uintptr_t)g.R % 16 == 0;
            if (!g.part || !aligned || S < 2 || S * g.M * g.N > kGemmPartFloats) S = 1;
            GemmArgs gs = g;
            gs.splits = splits = (int)S;
            hipLaunchKernelGGL((gemm_bf3_kernel<64, 64>),
                               dim3((unsigned)gn64, (unsigned)gm64, (unsigned)S), dim3(256), 0, st, gs);
            if (S > 1 && S <= kSumNormSplits && g.norm_w) {  // the sum makes the row norm too
                hipLaunchKernelGGL(splitk_sum_norm_kernel, dim3((unsigned)g.M), dim3(256), 0, st, gs);
            } else if (S > 1) {
                const size_t mn4 = (size_t)g.M * g.N / 4;
                hipLaunchKernelGGL(splitk_sum_kernel, dim3((unsigned)((mn4 + 255) / 256)), dim3(256), 0,
                                   st, gs);
            }
        }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !g.norm_w || (splits > 1 && splits <= kSumNormSplits)) return (int)e;
    return launch_rmsnorm_rows(g.C, g.norm_w, g.norm_out, g.M, g.N, g.norm_eps, stream);
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
