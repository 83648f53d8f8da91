// decode_common.hpp — device helpers shared by the batch-1 MoE decode
// kernels: streaming and hand-off memory accesses, the nibble-chunk terms
// and the input RMS of a normalised input.
#pragma once

#include <hip/hip_runtime.h>

#include "device.hpp"
#include "internal.hpp"

namespace m1moe {

// Expert weights are read once per launch: non-temporal loads keep them from
// displacing the hand-off lines and router rows in the caches.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const uint8_t* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// ---- hand-off primitives ------------------------------------------------------

__device__ __forceinline__ unsigned long long ld_u64(const unsigned long long* p) {
    return __hip_atomic_load(const_cast<unsigned long long*>(p), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_u64(unsigned long long* p, unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_u32(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_u32(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_f32(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void add_u32(uint32_t* p, uint32_t v) {
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Loads 32-element chunk c of an f32 or bf16 vector as f32.  The caller
// passes an in-range chunk index (clamped for idle lanes) so the loads are
// unconditional; ok = false zeroes them.
__device__ __forceinline__ void load_chunk(const void* x, int x_bf16, int c, bool ok,
                                           float (&v)[32]) {
    if (x_bf16) {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + c * 32);
        uint4 q[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = p[i];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) v[8 * i + e] = ok ? bf16x8_at(q[i], e) : 0.f;
    } else {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + c * 32);
        float4 q[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = p[i];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[4 * i + 0] = ok ? q[i].x : 0.f;
            v[4 * i + 1] = ok ? q[i].y : 0.f;
            v[4 * i + 2] = ok ? q[i].z : 0.f;
            v[4 * i + 3] = ok ? q[i].w : 0.f;
        }
    }
}

// f32 chunk written by other workgroups in this launch: eight 128-bit
// agent-coherent loads (sc1: they bypass the non-coherent L2 copies), all in
// flight together, then one wait (which also covers this wave's earlier
// loads).  The chunk address must be in range.
__device__ __forceinline__ void load_chunk_coherent(const float* x, int c, float (&v)[32]) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const float* p = x + c * 32;
    // the asm writes these locals themselves (writing the array through a
    // vector-typed view would let the compiler assume the array unchanged)
    f4 q0, q1, q2, q3, q4, q5, q6, q7;
    asm volatile(
        "global_load_dwordx4 %0, %8, off sc1\n\t"
        "global_load_dwordx4 %1, %8, off offset:16 sc1\n\t"
        "global_load_dwordx4 %2, %8, off offset:32 sc1\n\t"
        "global_load_dwordx4 %3, %8, off offset:48 sc1\n\t"
        "global_load_dwordx4 %4, %8, off offset:64 sc1\n\t"
        "global_load_dwordx4 %5, %8, off offset:80 sc1\n\t"
        "global_load_dwordx4 %6, %8, off offset:96 sc1\n\t"
        "global_load_dwordx4 %7, %8, off offset:112 sc1\n\t"
        "s_waitcnt vmcnt(0)"
        : "=&v"(q0), "=&v"(q1), "=&v"(q2), "=&v"(q3), "=&v"(q4), "=&v"(q5), "=&v"(q6), "=&v"(q7)
        : "v"(p)
        : "memory");
    const f4 q[8] = {q0, q1, q2, q3, q4, q5, q6, q7};
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int k = 0; k < 4; ++k) v[4 * j + k] = q[j][k];
}

// Scale and bias of one group, loaded as the aligned dword holding the bf16
// (a 32-bit load keeps the compiler from merging halves with ordered d16
// loads); `elem` is the bf16 index in the row-major [rows][groups] array.
__device__ __forceinline__ uint32_t sb_word(uint32_t elem) { return (elem >> 1) << 2; }
__device__ __forceinline__ uint32_t sb_sel(uint32_t elem) { return (elem & 1u) ? kSelHi : kSelLo; }

// Scales each of a lane's chunks by one power of two (its largest element
// into [2^13, 2^14)) and converts them to the f16 pairs of the nibble dot
// product.  Returns the inverse scale.
template <int N, class XC>
__device__ __forceinline__ float lane_scale_prep(float (&v)[N][32], XC (&xc)[N]) {
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < N; ++j)
#pragma unroll
        for (int e = 0; e < 32; ++e) mx = fmaxf(mx, fabsf(v[j][e]));
    float scale, inv;
    pow2_scale(mx, scale, inv);
#pragma unroll
    for (int j = 0; j < N; ++j) {
#pragma unroll
        for (int e = 0; e < 32; ++e) v[j][e] *= scale;
        prep_chunk(v[j], xc[j]);
    }
    return inv;
}

// One 32-column chunk of one row: s * sum(n x) + b * sum(x), in the lane's
// scaled units.
// (LO: the split chunk's lo half takes part; without it the split chunk's
// hi half alone, exact for bf16 inputs.)
template <bool LO = false>
__device__ __forceinline__ float chunk_term(const uint4& w, uint32_t sw, uint32_t bw,
                                            uint32_t sel, const XChunk& xc, const NibK& nk) {
    const float d = nib_dot32(w, xc, nk) - xc.off;
    return fmaf(bf16_pick(sw, sel), d, bf16_pick(bw, sel) * xc.xs);
}
template <bool LO>
__device__ __forceinline__ float chunk_term(const uint4& w, uint32_t sw, uint32_t bw,
                                            uint32_t sel, const XChunk2& xc, const NibK& nk) {
    const float d = nib_dot32<LO>(w, xc, nk) - xc.off;
    return fmaf(bf16_pick(sw, sel), d, bf16_pick(bw, sel) * xc.xs);
}

// rsqrt(sum(x^2) / h + eps) of a normalised input, from its n_ssq partial
// sums added in the same order in every wave (lane l takes partials l,
// l + 64, ..., then the wave sum), so every wave of every role gets the same
// value.
__device__ __forceinline__ float input_rms(const FusedArgs& a, int lane) {
    float s = 0.f;
    for (int i0 = 0; i0 < a.n_ssq; i0 += 256) {
        float t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = i0 + lane + 64 * j;
            t[j] = i < a.n_ssq ? a.x_ssq[i] : 0.f;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) s += t[j];
    }
    return rsqrtf(wave_sum(s) / (float)a.h + a.x_eps);
}

}  // namespace m1moe
