// device.hpp — gfx950 device helpers shared by the MoE kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace m1moe {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_to_f32(uint32_t v16) {
    return __uint_as_float(v16 << 16);
}

// Element i (0..7) of eight bf16 values packed in a uint4.
__device__ __forceinline__ float bf16x8_at(const uint4& v, int i) {
    const uint32_t w = (i < 2) ? v.x : (i < 4) ? v.y : (i < 6) ? v.z : v.w;
    return (i & 1) ? __uint_as_float(w & 0xFFFF0000u) : __uint_as_float(w << 16);
}

__device__ __forceinline__ float dot2_f16(uint32_t a, half2_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), b, c, false);
}

// One lane's 32-column chunk of the input vector, prepared for the nibble
// dot product.  The f16 "magic" conversion turns a nibble n in the low 4
// mantissa bits of 0x6400 into 1024+n, and one at bits 4..7 into 1024+16n,
// so a word is expanded with two masks and one shift, no per-nibble
// conversion.  Pairs are ordered to match those masks:
//   X[4i+0] = (x[8i+0],    x[8i+4])      against (1024+n0,    1024+n4)
//   X[4i+1] = (x[8i+1]/16, x[8i+5]/16)   against (1024+16n1,  1024+16n5)
//   X[4i+2] = (x[8i+2],    x[8i+6])      against (1024+n2,    1024+n6)
//   X[4i+3] = (x[8i+3]/16, x[8i+7]/16)   against (1024+16n3,  1024+16n7)
// so sum over the chunk of dot2 = sum_c n_c x_c + off, off = 1024*sum(X).
// xs = sum_c x_c (the values the dot products see), for the bias term.
struct XChunk {
    half2_t X[16];
    float off;
    float xs;
};

// v[0..31]: the chunk's inputs already multiplied by the power-of-two scale.
__device__ __forceinline__ void prep_chunk(const float* v, XChunk& c) {
    float off = 0.f, xs = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float* b = v + 8 * i;
        const _Float16 e0 = (_Float16)b[0], e4 = (_Float16)b[4];
        const _Float16 e2 = (_Float16)b[2], e6 = (_Float16)b[6];
        const _Float16 o1 = (_Float16)(b[1] * 0.0625f), o5 = (_Float16)(b[5] * 0.0625f);
        const _Float16 o3 = (_Float16)(b[3] * 0.0625f), o7 = (_Float16)(b[7] * 0.0625f);
        c.X[4 * i + 0] = half2_t{e0, e4};
        c.X[4 * i + 1] = half2_t{o1, o5};
        c.X[4 * i + 2] = half2_t{e2, e6};
        c.X[4 * i + 3] = half2_t{o3, o7};
        const float se = (float)e0 + (float)e4 + (float)e2 + (float)e6;
        const float so = (float)o1 + (float)o5 + (float)o3 + (float)o7;
        off += se + so;
        xs += se + 16.f * so;
    }
    c.off = 1024.f * off;
    c.xs = xs;
}

// The same chunk with each input split as hi + lo, hi = f16(x), lo =
// f16(x - hi): 22 significant bits instead of 11.  Both halves go through the
// same nibble dot products (twice the v_dot2, 16 more VGPRs per chunk); off
// and xs are those of hi + lo.  Used for the gate/up input, whose rounding
// the SwiGLU and the down projection can amplify when their sums cancel.
struct XChunk2 {
    half2_t X[16];  // hi pairs, ordered as XChunk::X
    half2_t L[16];  // lo pairs
    float off;
    float xs;
};

__device__ __forceinline__ void split_f16(float x, _Float16& hi, _Float16& lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);  // x - hi is exact in f32
}

__device__ __forceinline__ void prep_chunk(const float* v, XChunk2& c) {
    float off = 0.f, xs = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float* b = v + 8 * i;
        _Float16 h[8], l[8];
        split_f16(b[0], h[0], l[0]);
        split_f16(b[4], h[4], l[4]);
        split_f16(b[2], h[2], l[2]);
        split_f16(b[6], h[6], l[6]);
        split_f16(b[1] * 0.0625f, h[1], l[1]);
        split_f16(b[5] * 0.0625f, h[5], l[5]);
        split_f16(b[3] * 0.0625f, h[3], l[3]);
        split_f16(b[7] * 0.0625f, h[7], l[7]);
        c.X[4 * i + 0] = half2_t{h[0], h[4]};
        c.X[4 * i + 1] = half2_t{h[1], h[5]};
        c.X[4 * i + 2] = half2_t{h[2], h[6]};
        c.X[4 * i + 3] = half2_t{h[3], h[7]};
        c.L[4 * i + 0] = half2_t{l[0], l[4]};
        c.L[4 * i + 1] = half2_t{l[1], l[5]};
        c.L[4 * i + 2] = half2_t{l[2], l[6]};
        c.L[4 * i + 3] = half2_t{l[3], l[7]};
        float se = 0.f, so = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            se += (float)h[e] + (float)l[e];
            so += (float)h[e + 1] + (float)l[e + 1];
        }
        off += se + so;
        xs += se + 16.f * so;
    }
    c.off = 1024.f * off;
    c.xs = xs;
}

// Masks and the f16 magic of the nibble expansion, held in registers so that
// each expansion is one v_and_or_b32 (masks in SGPRs, magic in a VGPR; with
// literal operands the compiler emits a separate AND and OR).
struct NibK {
    uint32_t lo, hi, mg;
};
__device__ __forceinline__ NibK nib_consts() {
    NibK k;
    k.lo = __builtin_amdgcn_readfirstlane(0x000F000Fu);
    k.hi = __builtin_amdgcn_readfirstlane(0x00F000F0u);
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(k.mg));
    return k;
}

// sum over 32 columns of (1024+n)*x-pairs, i.e. sum n_c x_c + c.off
__device__ __forceinline__ float nib_dot32(const uint4& w, const XChunk& c, const NibK& k) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t v = ws[i], v8 = v >> 8;
        a0 = dot2_f16((v & k.lo) | k.mg, c.X[4 * i + 0], a0);
        a1 = dot2_f16((v & k.hi) | k.mg, c.X[4 * i + 1], a1);
        a0 = dot2_f16((v8 & k.lo) | k.mg, c.X[4 * i + 2], a0);
        a1 = dot2_f16((v8 & k.hi) | k.mg, c.X[4 * i + 3], a1);
    }
    return a0 + a1;
}

// The same over a split chunk: hi and lo pairs against the same expansions
// (LO = false: hi only, for inputs that are exact in f16, whose lo is 0).
template <bool LO>
__device__ __forceinline__ float nib_dot32(const uint4& w, const XChunk2& c, const NibK& k) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t v = ws[i], v8 = v >> 8;
        const uint32_t n0 = (v & k.lo) | k.mg, n1 = (v & k.hi) | k.mg;
        const uint32_t n2 = (v8 & k.lo) | k.mg, n3 = (v8 & k.hi) | k.mg;
        a0 = dot2_f16(n0, c.X[4 * i + 0], a0);
        a1 = dot2_f16(n1, c.X[4 * i + 1], a1);
        if (LO) a2 = dot2_f16(n0, c.L[4 * i + 0], a2);
        if (LO) a3 = dot2_f16(n1, c.L[4 * i + 1], a3);
        a0 = dot2_f16(n2, c.X[4 * i + 2], a0);
        a1 = dot2_f16(n3, c.X[4 * i + 3], a1);
        if (LO) a2 = dot2_f16(n2, c.L[4 * i + 2], a2);
        if (LO) a3 = dot2_f16(n3, c.L[4 * i + 3], a3);
    }
    return LO ? (a0 + a1) + (a2 + a3) : a0 + a1;
}

// Nibble dot product on exact f16 subnormals: masking a word's nibble pairs
// (bits 0..3 / 16..19 and 4..7 / 20..23, then the same of the word >> 8)
// leaves f16 bit patterns whose values are n * 2^-24 (or 16 n * 2^-24 for
// the upper nibble of a byte, which meets the /16 of the odd chunk
// elements).  The products with the scaled chunk are exact in f32, so the
// result is sum_c n_c x_c * 2^-24 with no offset to cancel; the caller
// multiplies by 2^24 (exact).  LO: the lo pairs of a split chunk take part.
template <bool LO>
__device__ __forceinline__ float nib_dot32_sub(const uint4& w, const XChunk2& c, uint32_t mlo,
                                               uint32_t mhi) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t v = ws[i], v8 = v >> 8;
        const uint32_t n0 = v & mlo, n1 = v & mhi, n2 = v8 & mlo, n3 = v8 & mhi;
        a0 = dot2_f16(n0, c.X[4 * i + 0], a0);
        a1 = dot2_f16(n1, c.X[4 * i + 1], a1);
        if (LO) a2 = dot2_f16(n0, c.L[4 * i + 0], a2);
        if (LO) a3 = dot2_f16(n1, c.L[4 * i + 1], a3);
        a0 = dot2_f16(n2, c.X[4 * i + 2], a0);
        a1 = dot2_f16(n3, c.X[4 * i + 3], a1);
        if (LO) a2 = dot2_f16(n2, c.L[4 * i + 2], a2);
        if (LO) a3 = dot2_f16(n3, c.L[4 * i + 3], a3);
    }
    return LO ? (a0 + a1) + (a2 + a3) : a0 + a1;
}

// v_perm_b32 selectors that move the low / high bf16 of a dword into the
// upper half of an f32 and zero the lower half (selector byte 0x0C = 0x00).
constexpr uint32_t kSelLo = 0x01000C0Cu, kSelHi = 0x03020C0Cu;
__device__ __forceinline__ float bf16_pick(uint32_t w, uint32_t sel) {
    return __uint_as_float(__builtin_amdgcn_perm(w, w, sel));
}

// Position i of a permuted 8-column group holds column perm8(i):
// 0, 4, 1, 5, 2, 6, 3, 7 (the column order of the prefill GEMM's A fragments).
__host__ __device__ constexpr int perm8(int i) { return (i >> 1) | ((i & 1) << 2); }

// Power-of-two scale that maps max|x| into [2^13, 2^14), so every scaled
// input is a normal-range f16 with headroom (max f16 is 65504).  The scale
// is at most 2^126 so both factors stay finite, normal f32 values: a max|x|
// below 2^-112 is scaled by 2^126 only (its chunk then sits below 2^14 with
// fewer f16 bits; finite f32 inputs never need the lower bound).
__device__ __forceinline__ void pow2_scale(float maxabs, float& scale, float& inv) {
    if (!(maxabs > 0.f) || !(maxabs < 3.0e38f)) {
        scale = 1.f;
        inv = 1.f;
        return;
    }
    int e;
    frexpf(maxabs, &e);  // maxabs = m * 2^e, m in [0.5, 1)
    const int k = min(max(14 - e, -126), 126);
    scale = ldexpf(1.f, k);
    inv = ldexpf(1.f, -k);
}

// ---- cross-lane reductions on DPP (full-rate VALU lane moves) ---------------
// gfx9 DPP controls: quad_perm [1,0,3,2] / [2,3,0,1], rotate right within a
// row of 16 lanes by 4 / 8, broadcast lane 15 of each row to the next row,
// broadcast lane 31 to rows 2 and 3.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppRor4 = 0x124, kDppRor8 = 0x128;
constexpr int kDppBcast15 = 0x142, kDppBcast31 = 0x143;

// Lanes of rows outside ROWS get `old`.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t old, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROWS, 0xF, false);
}
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp_f32(float old, float v) {
    return __uint_as_float(dpp_u32<CTRL, ROWS>(__float_as_uint(old), __float_as_uint(v)));
}
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ double dpp_f64(double old, double v) {
    const unsigned long long o = __double_as_longlong(old), x = __double_as_longlong(v);
    const uint32_t lo = dpp_u32<CTRL, ROWS>((uint32_t)o, (uint32_t)x);
    const uint32_t hi = dpp_u32<CTRL, ROWS>((uint32_t)(o >> 32), (uint32_t)(x >> 32));
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ float readlane_f32(float v, int lane) {
    return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), lane));
}

// Sum over aligned segments of `seg` lanes (a power of two, 2..64).  The
// segment's total lands in its last lane (lane % seg == seg - 1); other lanes
// keep partial sums.  The order is fixed, so results are deterministic.
// Branch-free: every step runs and the steps beyond `seg` add a term masked
// to +0 (a run-time width would otherwise compile to a branch per step).
__device__ __forceinline__ float seg_sum(float v, int seg) {
    const uint32_t m4 = seg >= 4 ? ~0u : 0u, m8 = seg >= 8 ? ~0u : 0u;
    const uint32_t m16 = seg >= 16 ? ~0u : 0u, m32 = seg >= 32 ? ~0u : 0u;
    const uint32_t m64 = seg >= 64 ? ~0u : 0u;
    v += dpp_f32<kDppXor1>(v, v);
    v += __uint_as_float(dpp_u32<kDppXor2>(__float_as_uint(v), __float_as_uint(v)) & m4);
    v += __uint_as_float(dpp_u32<kDppRor4>(__float_as_uint(v), __float_as_uint(v)) & m8);
    v += __uint_as_float(dpp_u32<kDppRor8>(__float_as_uint(v), __float_as_uint(v)) & m16);
    v += __uint_as_float(dpp_u32<kDppBcast15, 0xA>(0u, __float_as_uint(v)) & m32);
    v += __uint_as_float(dpp_u32<kDppBcast31, 0xC>(0u, __float_as_uint(v)) & m64);
    return v;
}

// Sum over aligned segments of SEG lanes, SEG known at compile time.
template <int SEG>
__device__ __forceinline__ float seg_sum_c(float v) {
    v += dpp_f32<kDppXor1>(v, v);
    if (SEG >= 4) v += dpp_f32<kDppXor2>(v, v);
    if (SEG >= 8) v += dpp_f32<kDppRor4>(v, v);
    if (SEG >= 16) v += dpp_f32<kDppRor8>(v, v);
    if (SEG >= 32) v += dpp_f32<kDppBcast15, 0xA>(0.f, v);
    if (SEG >= 64) v += dpp_f32<kDppBcast31, 0xC>(0.f, v);
    return v;
}

// Sum over the wave, total in lane 63.
__device__ __forceinline__ double wave_sum_f64_last(double v) {
    v += dpp_f64<kDppXor1>(v, v);
    v += dpp_f64<kDppXor2>(v, v);
    v += dpp_f64<kDppRor4>(v, v);
    v += dpp_f64<kDppRor8>(v, v);
    v += dpp_f64<kDppBcast15, 0xA>(0.0, v);
    v += dpp_f64<kDppBcast31, 0xC>(0.0, v);
    return v;
}

// Sum over the wave, returned to every lane (uniform).
__device__ __forceinline__ float wave_sum(float v) {
    return readlane_f32(seg_sum_c<64>(v), 63);
}

// Max over the wave, returned to every lane (uniform).
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<kDppXor1>(v, v));
    v = fmaxf(v, dpp_f32<kDppXor2>(v, v));
    v = fmaxf(v, dpp_f32<kDppRor4>(v, v));
    v = fmaxf(v, dpp_f32<kDppRor8>(v, v));
    v = fmaxf(v, dpp_f32<kDppBcast15, 0xA>(v, v));
    v = fmaxf(v, dpp_f32<kDppBcast31, 0xC>(v, v));
    return readlane_f32(v, 63);
}

// (value desc, index asc) maximum over the wave, returned to every lane.
__device__ __forceinline__ void wave_argmax(float& bv, int& bi) {
#define M1MOE_ARGMAX_STEP(CTRL)                                                   \
    {                                                                             \
        const float ov = dpp_f32<CTRL>(bv, bv);                                   \
        const int oi = (int)dpp_u32<CTRL>((uint32_t)bi, (uint32_t)bi);            \
        if (ov > bv || (ov == bv && oi < bi)) {                                   \
            bv = ov;                                                              \
            bi = oi;                                                              \
        }                                                                         \
    }
    M1MOE_ARGMAX_STEP(kDppXor1)
    M1MOE_ARGMAX_STEP(kDppXor2)
    M1MOE_ARGMAX_STEP(kDppRor4)
    M1MOE_ARGMAX_STEP(kDppRor8)
#undef M1MOE_ARGMAX_STEP
    // every lane of a row now holds the row's best; combine the four rows
    float v = readlane_f32(bv, 0);
    int i = __builtin_amdgcn_readlane(bi, 0);
#pragma unroll
    for (int r = 1; r < 4; ++r) {
        const float rv = readlane_f32(bv, 16 * r);
        const int ri = __builtin_amdgcn_readlane(bi, 16 * r);
        if (rv > v || (rv == v && ri < i)) {
            v = rv;
            i = ri;
        }
    }
    bv = v;
    bi = i;
}

// Ranks the logits of up to 256 experts held 4 per lane (expert lane + 64j;
// pass -inf beyond E) by descending value with ties to the lower index, and
// computes softmax weights over all E experts (InferenceEngine.swift:501-506),
// renormalised over the selection when `norm` (:514-517, summed in slot
// order).  Lane r < K receives slot r's expert and weight.
__device__ __forceinline__ void topk_softmax(const float (&v)[4], int E, int K, int norm, int lane,
                                             int& my_idx, float& my_w) {
    bool taken[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) taken[j] = (lane + 64 * j >= E);
    float my_val = -INFINITY, mx = -INFINITY;
    my_idx = 0;
    for (int r = 0; r < K; ++r) {
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int ee = lane + 64 * j;
            if (!taken[j] && (v[j] > bv || (v[j] == bv && ee < bi))) {
                bv = v[j];
                bi = ee;
            }
        }
        wave_argmax(bv, bi);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (lane + 64 * j == bi) taken[j] = true;
        if (r == 0) mx = bv;
        if (lane == r) {
            my_idx = bi;
            my_val = bv;
        }
    }
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (lane + 64 * j < E) sum += expf(v[j] - mx);
    const float inv = 1.0f / wave_sum(sum);
    const float p = (lane < K) ? expf(my_val - mx) * inv : 0.f;
    my_w = p;
    if (norm) {
        float ssum = 0.f;
        for (int r = 0; r < K; ++r) ssum = ssum + readlane_f32(p, r);
        my_w = p / ssum;
    }
}

// Byte offsets of the planar sub-blocks (ModelSpec.swift:36-52,
// InferenceEngine.swift:84-97), from the MoE dimensions.
struct Layout {
    uint64_t gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s, down_b;
    __device__ Layout(int h, int I, int gs) {
        const uint64_t gw = (uint64_t)I * (uint64_t)(h / 2);
        const uint64_t gsb = (uint64_t)I * (uint64_t)(h / gs) * 2;
        const uint64_t dw = (uint64_t)h * (uint64_t)(I / 2);
        const uint64_t dsb = (uint64_t)h * (uint64_t)(I / gs) * 2;
        gate_w = 0;
        gate_s = gw;
        gate_b = gate_s + gsb;
        up_w = gate_b + gsb;
        up_s = up_w + gw;
        up_b = up_s + gsb;
        down_w = up_b + gsb;
        down_s = down_w + dw;
        down_b = down_s + dsb;
    }
};

// Byte offsets within one expert's repacked block (h = 2048 or 4096), the copy the
// decode_cu.hip kernels read instead of the canonical scales and down matrix:
//   gsb: [I/4 row quads][h/gs groups][4 rows][gate s | gate b << 16, up s | up b << 16]
//   dw:  [I/32 column chunks][h rows][4 words]  (the down matrix, chunk-major)
//   dsb: [I/gs groups][512][h/512]: entry (t, r) = down s | down b << 16 of row t + 512 r
struct DecLayout {
    uint64_t gsb, dw, dsb, bytes;
    __host__ __device__ DecLayout(int h, int I, int gs) {
        gsb = 0;
        dw = (uint64_t)I * (uint64_t)(h / gs) * 8;
        dsb = dw + (uint64_t)h * (uint64_t)(I / 2);
        bytes = (dsb + (uint64_t)(I / gs) * (uint64_t)h * 4 + 255) / 256 * 256;
    }
};

// silu(g) = g / (1 + e^-g) (Shaders.metal:148, fast-math there) on the
// hardware exp2 and reciprocal.
__device__ __forceinline__ float silu_fast(float g) {
    return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.44269504088896341f));
}

__device__ __forceinline__ void flag_error(uint32_t* err, uint32_t code) {
    if (err) atomicOr(err, code);
}

}  // namespace m1moe
