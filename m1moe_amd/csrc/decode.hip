// decode.hip — batch-1 MoE expert FFN for gfx950: fused 4-bit group-affine
// dequant + gate/up matvec + SwiGLU, then fused dequant + down matvec +
// weighted combine + residual.
//
// Replaces, per token and layer, the reference's 4K+1 Metal dispatches
// (matvec4bit gate, matvec4bit up, swiGLU, matvec4bit down per slot, then
// moeCombine: InferenceEngine.swift:401-478, Shaders.metal:39-92,138-149,
// 360-376) with two kernels.  Experts are addressed in the resident arena
// as layer_base + idx * expert_bytes (replacing the pread dispatch,
// InferenceEngine.swift:271-280).
//
// Work mapping: a row of a projection is split into 32-column chunks (one
// 128-bit load of nibbles per lane).  A lane keeps the same chunk(s) for
// every row it visits, so its slice of the input vector is converted once
// into f16 pairs in registers.  Rows shorter than 64 chunks are packed
// several to a wave; longer rows give each lane several chunks.
//
// Arithmetic: sum_c (n_c*s_g + b_g) x_c is evaluated as
// sum_g [ s_g * sum_{c in g} n_c x_c + b_g * sum_{c in g} x_c ] with the
// inner nibble sums on v_dot2_f32_f16 (exact f16*f16 products, f32
// accumulation).  The input is first scaled by a power of two so that its
// largest element is in [2^13, 2^14) and then rounded to f16; the result is
// scaled back exactly.  That input rounding (relative 2^-11) is the only
// difference from f32 arithmetic beyond summation order.
#include <hip/hip_runtime.h>

#include "device.hpp"
#include "internal.hpp"

namespace m1moe {
namespace {

struct LaneMap {
    int q;      // row slot within one wave step
    int c0;     // first chunk index
    bool ok;    // lane participates
    int seg;    // reduction segment width (power of two)
};

// C = chunks per row.  C < 64 packs rpi = 64/C rows per wave step.
__device__ __forceinline__ LaneMap lane_map(int lane, int C, int rpi) {
    LaneMap m;
    if (C >= 64) {
        m.q = 0;
        m.c0 = lane;
        m.ok = true;
        m.seg = 64;
    } else {
        m.q = lane / C;
        m.c0 = lane - m.q * C;
        m.ok = m.q < rpi;
        m.seg = (rpi > 1) ? C : 64;  // rpi > 1 only when C divides 64
    }
    return m;
}

// Loads 32-element chunk c of an f32 or bf16 vector as f32 (zeros if !ok).
__device__ __forceinline__ void load_chunk(const void* x, int x_bf16, int c, bool ok, float (&v)[32]) {
    if (x_bf16) {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + c * 32);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 q = ok ? p[i] : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[8 * i + e] = bf16x8_at(q, e);
        }
    } else {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + c * 32);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 q = ok ? p[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            v[4 * i + 0] = q.x;
            v[4 * i + 1] = q.y;
            v[4 * i + 2] = q.z;
            v[4 * i + 3] = q.w;
        }
    }
}

// Loads one lane's chunks of an f32 or bf16 vector, scales them by a
// wave-wide power of two and prepares the f16 pairs.  All 64 lanes must call
// it (wave-wide max).  Returns the inverse scale.  With more than two chunks
// per lane the vector is read twice (max, then convert) instead of being
// held in registers; the second read hits the cache.
template <int CPL>
__device__ __forceinline__ float load_prep_x(const void* x, int x_bf16, const LaneMap& m, int C,
                                             XChunk (&xc)[CPL]) {
    constexpr bool kHold = CPL <= 2;
    float v[kHold ? CPL : 1][32];
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = m.c0 + 64 * j;
        float (&vj)[32] = v[kHold ? j : 0];
        load_chunk(x, x_bf16, c, m.ok && c < C, vj);
#pragma unroll
        for (int e = 0; e < 32; ++e) mx = fmaxf(mx, fabsf(vj[e]));
    }
    mx = wave_max(mx);
    float scale, inv;
    pow2_scale(mx, scale, inv);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = m.c0 + 64 * j;
        float (&vj)[32] = v[kHold ? j : 0];
        if (!kHold) load_chunk(x, x_bf16, c, m.ok && c < C, vj);
#pragma unroll
        for (int e = 0; e < 32; ++e) vj[e] *= scale;
        prep_chunk(vj, xc[j]);
    }
    return inv;
}

// Gate/up + SwiGLU.  Grid: K * blocks_per_expert blocks of 4 waves; each wave
// covers U steps of rpi rows of one selected expert.
template <int CPL, int U>
__global__ __launch_bounds__(256) void gate_up_kernel(DecodeArgs a, int C, int rpi,
                                                      int blocks_per_expert) {
    const int k = blockIdx.x / blocks_per_expert;
    const int rb = blockIdx.x - k * blocks_per_expert;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int e = a.topk_idx[k];
    if (e < 0 || e >= a.E) {
        if (threadIdx.x == 0) flag_error(a.err, 1u);
        return;
    }
    const uint8_t* blk = a.layer_base + (uint64_t)e * a.expert_bytes;
    const LaneMap m = lane_map(lane, C, rpi);
    const int groups = a.h / a.gs;
    const int row_bytes = a.h / 2;
    const int row0 = (rb * 4 + wave) * U * rpi + m.q;

    uint4 gw[U][CPL], uw[U][CPL];
    uint32_t gs_[U][CPL], gb_[U][CPL], us_[U][CPL], ub_[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int row = row0 + u * rpi;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = m.c0 + 64 * j;
            const bool ok = m.ok && row < a.I && c < C;
            const uint64_t wo = (uint64_t)row * row_bytes + (uint64_t)c * 16;
            const uint64_t so = ((uint64_t)row * groups + (uint64_t)(c * 32) / a.gs) * 2;
            gw[u][j] = ok ? *reinterpret_cast<const uint4*>(blk + a.gate.w_off + wo) : make_uint4(0, 0, 0, 0);
            uw[u][j] = ok ? *reinterpret_cast<const uint4*>(blk + a.up.w_off + wo) : make_uint4(0, 0, 0, 0);
            gs_[u][j] = ok ? *reinterpret_cast<const uint16_t*>(blk + a.gate.s_off + so) : 0u;
            gb_[u][j] = ok ? *reinterpret_cast<const uint16_t*>(blk + a.gate.b_off + so) : 0u;
            us_[u][j] = ok ? *reinterpret_cast<const uint16_t*>(blk + a.up.s_off + so) : 0u;
            ub_[u][j] = ok ? *reinterpret_cast<const uint16_t*>(blk + a.up.b_off + so) : 0u;
        }
    }

    XChunk xc[CPL];
    const float inv = load_prep_x<CPL>(a.x, a.x_bf16, m, C, xc);

#pragma unroll
    for (int u = 0; u < U; ++u) {
        float pg = 0.f, pu = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const float dg = nib_dot32(gw[u][j], xc[j]) - xc[j].off;
            const float du = nib_dot32(uw[u][j], xc[j]) - xc[j].off;
            pg = fmaf(bf16_to_f32(gs_[u][j]), dg, fmaf(bf16_to_f32(gb_[u][j]), xc[j].xs, pg));
            pu = fmaf(bf16_to_f32(us_[u][j]), du, fmaf(bf16_to_f32(ub_[u][j]), xc[j].xs, pu));
        }
        pg = seg_sum(pg, m.seg);
        pu = seg_sum(pu, m.seg);
        const int row = row0 + u * rpi;
        if (m.ok && m.c0 == 0 && row < a.I) {
            const float g = pg * inv, up = pu * inv;
            a.act[(size_t)k * a.I + row] = (g / (1.0f + expf(-g))) * up;  // Shaders.metal:147-148
        }
    }
}

// Down + combine.  Grid: ceil(h / (S*rpi)) blocks of W waves; wave w handles
// the selected experts w, w+W, ...; the block combines all K experts of its
// rows in slot order (no atomics, deterministic).
template <int CPL, int S>
__global__ __launch_bounds__(512) void down_combine_kernel(DecodeArgs a, int C, int rpi, int W) {
    extern __shared__ float part[];  // [K][S*rpi]
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rows_blk = S * rpi;
    const int row_base = blockIdx.x * rows_blk;
    const LaneMap m = lane_map(lane, C, rpi);
    const int groups = a.I / a.gs;
    const int row_bytes = a.I / 2;

    for (int k = wave; k < a.K; k += W) {
        const int e = a.topk_idx[k];
        const bool valid = (e >= 0 && e < a.E);
        if (!valid) {
            if (lane == 0) flag_error(a.err, 1u);
            for (int r = lane; r < rows_blk; r += 64) part[k * rows_blk + r] = 0.f;
            continue;
        }
        const uint8_t* blk = a.layer_base + (uint64_t)e * a.expert_bytes;
        uint4 dw[S][CPL];
        uint32_t ds_[S][CPL], db_[S][CPL];
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int row = row_base + s * rpi + m.q;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = m.c0 + 64 * j;
                const bool ok = m.ok && row < a.h && c < C;
                const uint64_t wo = (uint64_t)row * row_bytes + (uint64_t)c * 16;
                const uint64_t so = ((uint64_t)row * groups + (uint64_t)(c * 32) / a.gs) * 2;
                dw[s][j] = ok ? *reinterpret_cast<const uint4*>(blk + a.down.w_off + wo) : make_uint4(0, 0, 0, 0);
                ds_[s][j] = ok ? *reinterpret_cast<const uint16_t*>(blk + a.down.s_off + so) : 0u;
                db_[s][j] = ok ? *reinterpret_cast<const uint16_t*>(blk + a.down.b_off + so) : 0u;
            }
        }
        XChunk xc[CPL];
        const float inv = load_prep_x<CPL>(a.act + (size_t)k * a.I, 0, m, C, xc);
#pragma unroll
        for (int s = 0; s < S; ++s) {
            float p = 0.f;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const float d = nib_dot32(dw[s][j], xc[j]) - xc[j].off;
                p = fmaf(bf16_to_f32(ds_[s][j]), d, fmaf(bf16_to_f32(db_[s][j]), xc[j].xs, p));
            }
            p = seg_sum(p, m.seg);
            if (m.ok && m.c0 == 0) part[k * rows_blk + s * rpi + m.q] = p * inv;
        }
    }
    __syncthreads();
    for (int r = threadIdx.x; r < rows_blk; r += blockDim.x) {
        const int row = row_base + r;
        if (row >= a.h) continue;
        float acc = a.residual ? a.residual[row] : 0.f;  // Shaders.metal:371-374
        for (int k = 0; k < a.K; ++k) acc = fmaf(a.topk_w[k], part[k * rows_blk + r], acc);
        a.out[row] = acc;
    }
}

// Dequantised weights of one projection: one thread per packed word.
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* blk, ProjView p, int gs,
                                                     float* out) {
    const uint64_t words = (uint64_t)p.rows * (p.cols / 8);
    const uint64_t wi = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (wi >= words) return;
    const uint64_t row = wi / (p.cols / 8), wc = wi - row * (p.cols / 8);
    const uint32_t packed = reinterpret_cast<const uint32_t*>(blk + p.w_off)[wi];
    const uint64_t g = row * (p.cols / gs) + (wc * 8) / gs;
    const float s = bf16_to_f32(reinterpret_cast<const uint16_t*>(blk + p.s_off)[g]);
    const float b = bf16_to_f32(reinterpret_cast<const uint16_t*>(blk + p.b_off)[g]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        // n*s is exact in f32 (<= 12 significant bits): one rounding, in the add
        const float n = (float)((packed >> (4 * j)) & 0xFu);
        out[row * p.cols + wc * 8 + j] = __fadd_rn(__fmul_rn(n, s), b);
    }
}

inline int chunks_per_lane(int C) { return (C + 63) / 64; }
// Several rows share a wave step only when the row's chunk count divides 64
// (a power of two), so each row owns an aligned power-of-two lane segment.
inline int rows_per_step(int C) { return (C < 64 && 64 % C == 0) ? 64 / C : 1; }

template <int CPL>
int launch_gu(const DecodeArgs& a, hipStream_t st) {
    constexpr int U = CPL == 1 ? 4 : CPL == 2 ? 2 : 1;
    const int C = a.h / 32, rpi = rows_per_step(C);
    const int rows_per_block = 4 * U * rpi;
    const int bpe = (a.I + rows_per_block - 1) / rows_per_block;
    hipLaunchKernelGGL((gate_up_kernel<CPL, U>), dim3((unsigned)(a.K * bpe)), dim3(256), 0, st, a,
                       C, rpi, bpe);
    return (int)hipGetLastError();
}

template <int CPL>
int launch_dc(const DecodeArgs& a, hipStream_t st) {
    constexpr int S = CPL <= 2 ? 4 : CPL <= 4 ? 2 : 1;
    const int C = a.I / 32, rpi = rows_per_step(C);
    const int W = a.K < 8 ? a.K : 8;
    const int rows_blk = S * rpi;
    const int blocks = (a.h + rows_blk - 1) / rows_blk;
    const size_t lds = sizeof(float) * (size_t)a.K * rows_blk;
    hipLaunchKernelGGL((down_combine_kernel<CPL, S>), dim3((unsigned)blocks), dim3(64 * W), lds,
                       st, a, C, rpi, W);
    return (int)hipGetLastError();
}

}  // namespace

int launch_decode_gate_up(const DecodeArgs& a, void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (chunks_per_lane(a.h / 32)) {
        case 1: return launch_gu<1>(a, st);
        case 2: return launch_gu<2>(a, st);
        case 3: return launch_gu<3>(a, st);
        case 4: return launch_gu<4>(a, st);
        case 5: return launch_gu<5>(a, st);
        case 6: return launch_gu<6>(a, st);
        case 7: return launch_gu<7>(a, st);
        case 8: return launch_gu<8>(a, st);
        default: return (int)hipErrorInvalidValue;
    }
}

int launch_decode_down_combine(const DecodeArgs& a, void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (chunks_per_lane(a.I / 32)) {
        case 1: return launch_dc<1>(a, st);
        case 2: return launch_dc<2>(a, st);
        case 3: return launch_dc<3>(a, st);
        case 4: return launch_dc<4>(a, st);
        case 5: return launch_dc<5>(a, st);
        case 6: return launch_dc<6>(a, st);
        case 7: return launch_dc<7>(a, st);
        case 8: return launch_dc<8>(a, st);
        default: return (int)hipErrorInvalidValue;
    }
}

int launch_dequant(const uint8_t* expert_base, const ProjView& p, int32_t gs, float* out,
                   void* stream) {
    const uint64_t words = (uint64_t)p.rows * (p.cols / 8);
    const unsigned blocks = (unsigned)((words + 255) / 256);
    hipLaunchKernelGGL(dequant_kernel, dim3(blocks), dim3(256), 0,
                       static_cast<hipStream_t>(stream), expert_base, p, gs, out);
    return (int)hipGetLastError();
}

}  // namespace m1moe
