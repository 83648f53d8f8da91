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

// sum over 32 columns of (1024+n)*x-pairs, i.e. sum n_c x_c + c.off
__device__ __forceinline__ float nib_dot32(const uint4& w, const XChunk& c) {
    constexpr uint32_t kLo = 0x000F000Fu, kHi = 0x00F000F0u, kMagic = 0x64006400u;
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t v = ws[i], v8 = v >> 8;
        a0 = dot2_f16((v & kLo) | kMagic, c.X[4 * i + 0], a0);
        a1 = dot2_f16((v & kHi) | kMagic, c.X[4 * i + 1], a1);
        a0 = dot2_f16((v8 & kLo) | kMagic, c.X[4 * i + 2], a0);
        a1 = dot2_f16((v8 & kHi) | kMagic, c.X[4 * i + 3], a1);
    }
    return a0 + a1;
}

// Power-of-two scale that maps max|x| into [2^13, 2^14), so every scaled
// input is a normal-range f16 with headroom (max f16 is 65504).
__device__ __forceinline__ void pow2_scale(float maxabs, float& scale, float& inv) {
    if (!(maxabs > 0.f) || !(maxabs < 3.0e38f)) {
        scale = 1.f;
        inv = 1.f;
        return;
    }
    int e;
    frexpf(maxabs, &e);  // maxabs = m * 2^e, m in [0.5, 1)
    scale = ldexpf(1.f, 14 - e);
    inv = ldexpf(1.f, e - 14);
}

template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int m) {
    return __shfl_xor(v, m, 64);
}

// Butterfly sum inside aligned segments of `seg` lanes (seg a power of two).
__device__ __forceinline__ float seg_sum(float v, int seg) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        if (o < seg) v += shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ void flag_error(uint32_t* err, uint32_t code) {
    if (err) atomicOr(err, code);
}

}  // namespace m1moe
