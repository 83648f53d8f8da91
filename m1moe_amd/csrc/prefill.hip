// prefill.hip — T tokens through the MoE block of one layer at once.
//
// The reference has no batched path: prefill is T independent token-by-token
// forwards (Sources/bench/main.swift:139-141, Sources/chat/main.swift:
// 143-149), each running the router + selectTopK (InferenceEngine.swift:
// 490-519) and matvec4bit x3 + swiGLU + moeCombine (:401-478,
// Shaders.metal:39-92,138-149,360-376).  Here the T*K (token, slot) pairs
// are grouped by expert and each expert's pairs go through f16 MFMA GEMMs
// with the 4-bit dequantisation fused into the operand load:
//
//   router_topk (router.hip)   routing of all T tokens
//   prep_x                     x_t * 2^e_t in f16, one power of two per token
//                              (largest |x| into [2^13, 2^14): exact for bf16
//                              inputs, no f16 overflow)
//   group                      pairs sorted by expert; N-tiles of kPfTN pairs
//   gemm<2>                    gate and up for a (64 rows x 64 pairs) tile,
//                              epilogue act = silu(g) * u  -> f16 [pair][I]
//   gemm<1>                    down for a (64 rows x 64 pairs) tile -> f32 y
//   combine                    out[t] = residual[t] + sum_k w_tk y[pair(t,k)]
//                              in slot order (deterministic, no atomics)
//
// Dequantisation into MFMA operands.  A lane's A fragment is one packed
// word (8 nibbles = 8 columns of one weight row).  Each nibble is moved to
// f16 mantissa bits 6..9, which makes it the exact subnormal n * 2^-18; one
// v_pk_fma_f16 with (s * 2^(18-k), b * 2^-k) then gives f16((n * s + b) *
// 2^-k), a single rounding of the exact value (n * s has at most 12
// significant bits and the FMA is fused).  k is a per-row power of two
// (0 unless the row has a group scale |s| >= 0.25 or a weight beyond f16
// range), made at upload with the f16 scale/bias pairs (PfScaleLayout) and
// undone on the row's f32 accumulator.  The pairs come out in column order
// (0,4), (1,5), (2,6), (3,7); the B fragments are stored in LDS in the same
// permuted order (the sum over k does not depend on the order).
//
// MFMA v_mfma_f32_16x16x32_f16: A 16x32 (lane l: row l%16, k 8(l/16)..+7),
// B 32x16 (lane l: column l%16, the same k), D 16x16 (lane l: column l%16,
// rows 4(l/16)..+3).
#include <hip/hip_runtime.h>

#include "device.hpp"
#include "internal.hpp"

namespace m1moe {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kTN = kPfTN;
constexpr int kMaxE = 256;
constexpr uint32_t kNibMask = 0x03C003C0u;  // f16 mantissa bits 6..9 of both halves

// ---- x: per-token power-of-two scale, f16 copy ----------------------------------

// One workgroup per token; h <= 16384 (eight groups of 8 values per thread).
__global__ __launch_bounds__(256) void prep_x_kernel(PrefillArgs a) {
    __shared__ float s_max[4];
    const int t = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float v[8][8];
    float mx = 0.f;
#pragma unroll
    for (int it = 0; it < 8; ++it) {
        const int d = (it * 256 + (int)threadIdx.x) * 8;
        if (d < a.h) {
            if (a.x_bf16) {
                const uint4 q = *reinterpret_cast<const uint4*>(
                    static_cast<const uint16_t*>(a.x) + (size_t)t * a.h + d);
#pragma unroll
                for (int i = 0; i < 8; ++i) v[it][i] = bf16x8_at(q, i);
            } else {
                const float* xr = static_cast<const float*>(a.x) + (size_t)t * a.h + d;
                const float4 q0 = *reinterpret_cast<const float4*>(xr);
                const float4 q1 = *reinterpret_cast<const float4*>(xr + 4);
                v[it][0] = q0.x; v[it][1] = q0.y; v[it][2] = q0.z; v[it][3] = q0.w;
                v[it][4] = q1.x; v[it][5] = q1.y; v[it][6] = q1.z; v[it][7] = q1.w;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(v[it][i]));
        }
    }
    mx = wave_max(mx);
    if (lane == 0) s_max[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
    float scale, inv;
    pow2_scale(mx, scale, inv);
#pragma unroll
    for (int it = 0; it < 8; ++it) {
        const int d = (it * 256 + (int)threadIdx.x) * 8;
        if (d < a.h) {
            f16x8 o;
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = (_Float16)(v[it][i] * scale);
            *reinterpret_cast<f16x8*>(a.xq + (size_t)t * a.h + d) = o;
        }
    }
    if (threadIdx.x == 0) a.xinv[t] = inv;
}

// ---- grouping of (token, slot) pairs by expert ----------------------------------

// One workgroup.  Pair p = t*K + k gets the sorted position pos[p]; the order
// of pairs within an expert is arbitrary (each pair's GEMM column is computed
// independently of the others, so results do not depend on it).
__global__ __launch_bounds__(1024) void group_kernel(PrefillArgs a) {
    __shared__ int cnt[kMaxE];
    __shared__ int sc[kMaxE], st[kMaxE];
    __shared__ int off[kMaxE + 1], toff[kMaxE + 1];
    const int tid = threadIdx.x;
    const int E = a.E, P = a.T * a.K;
    if (tid < kMaxE) cnt[tid] = 0;
    __syncthreads();
    for (int p = tid; p < P; p += 1024) a.pos[p] = atomicAdd(&cnt[a.idx[p]], 1);
    __syncthreads();
    // inclusive scans of the pair and N-tile counts
    if (tid < kMaxE) {
        const int c = tid < E ? cnt[tid] : 0;
        sc[tid] = c;
        st[tid] = (c + kTN - 1) / kTN;
    }
    __syncthreads();
    for (int o = 1; o < kMaxE; o <<= 1) {
        int vc = 0, vt = 0;
        if (tid < kMaxE && tid >= o) {
            vc = sc[tid - o];
            vt = st[tid - o];
        }
        __syncthreads();
        if (tid < kMaxE) {
            sc[tid] += vc;
            st[tid] += vt;
        }
        __syncthreads();
    }
    if (tid <= E) {
        const int o = tid == 0 ? 0 : sc[tid - 1], to = tid == 0 ? 0 : st[tid - 1];
        off[tid] = o;
        toff[tid] = to;
        a.expert_off[tid] = o;
        a.tile_off[tid] = to;
    }
    __syncthreads();
    if (tid < E)
        for (int j = toff[tid]; j < toff[tid + 1]; ++j) a.tile_expert[j] = tid;
    for (int p = tid; p < P; p += 1024) {
        const int q = off[a.idx[p]] + a.pos[p];
        a.pos[p] = q;
        a.sorted_tok[q] = p / a.K;
    }
}

// ---- grouped GEMM with fused dequantisation ---------------------------------------

// 8 f16 of one row in column order c0..c7 (four u32 pairs) -> the permuted
// order (c0,c4), (c1,c5), (c2,c6), (c3,c7) of the A fragments.
__device__ __forceinline__ uint4 permute8(const uint4& x) {
    uint4 y;
    y.x = __builtin_amdgcn_perm(x.z, x.x, 0x05040100u);
    y.y = __builtin_amdgcn_perm(x.z, x.x, 0x07060302u);
    y.z = __builtin_amdgcn_perm(x.w, x.y, 0x05040100u);
    y.w = __builtin_amdgcn_perm(x.w, x.y, 0x07060302u);
    return y;
}

// A fragment of one packed word: f16(n*s + b) for its 8 columns, permuted.
__device__ __forceinline__ f16x8 dequant_word(uint32_t w, f16x2 s2, f16x2 b2) {
    const f16x2 p0 = __builtin_bit_cast(f16x2, (w << 6) & kNibMask);
    const f16x2 p1 = __builtin_bit_cast(f16x2, (w << 2) & kNibMask);
    const f16x2 p2 = __builtin_bit_cast(f16x2, (w >> 2) & kNibMask);
    const f16x2 p3 = __builtin_bit_cast(f16x2, (w >> 6) & kNibMask);
    const f16x2 q0 = __builtin_elementwise_fma(p0, s2, b2);
    const f16x2 q1 = __builtin_elementwise_fma(p1, s2, b2);
    const f16x2 q2 = __builtin_elementwise_fma(p2, s2, b2);
    const f16x2 q3 = __builtin_elementwise_fma(p3, s2, b2);
    return f16x8{q0[0], q0[1], q1[0], q1[1], q2[0], q2[1], q3[0], q3[1]};
}

// NMAT = 2: gate and up (K = h, rows = I), B = xq rows of the pairs' tokens,
//           epilogue act = silu(g) * u.
// NMAT = 1: down (K = I, rows = h), B = act rows, epilogue y.
// KB = k per block (64, 128 or 256; K % KB == 0), GSL = log2(group_size / 32).
// Lane (r = row in the wave's 16, kq = lane / 16) owns the KB/4 contiguous
// columns kq*KB/4.. of its row in each block (KB/32 packed words, one
// scale group since KB/4 <= group size); MFMA k-step s uses word s.
// Blocks are pipelined two deep: the loads of block kb+2 are issued while
// block kb is multiplied; B tiles go through a double-buffered LDS tile.
template <int NMAT, int KB, int NW>
struct PfStage {
    static constexpr int W = KB / 32;  // packed words per lane per block
    static constexpr int NB = KB * kTN / (8 * 64 * NW);  // uint4 of the B tile per thread
    uint32_t aw[NMAT][W];
    uint32_t sb[NMAT];                 // f16 s * 2^(18-k) | f16 b * 2^-k << 16
    uint4 b[NB];                       // this thread's share of the B tile
};

template <int NMAT, int KB, int GSL, int NW>
__global__ __launch_bounds__(64 * NW) void pf_gemm_kernel(PrefillArgs a, int m_tiles) {
    constexpr int W = KB / 32;
    constexpr int TM = 16 * NW;               // weight rows per workgroup
    constexpr int TPP = 64 * NW / kTN;        // B-staging threads per pair
    constexpr int NB = PfStage<NMAT, KB, NW>::NB;
    constexpr int kRow = KB * 2 + 16;  // LDS bytes per pair row (padded)
    __shared__ __attribute__((aligned(16))) unsigned char s_b[2][kTN * kRow];
    __shared__ int s_tok[kTN];
    __shared__ float s_inv[kTN];
    // all M-tiles of one N-tile read the same B tile: give them block ids with
    // the same residue mod 8, i.e. the same XCD (and L2)
    const int blk = blockIdx.x;
    const int slot = blk >> 3;
    const int mt = slot % m_tiles;
    const int nt = (slot / m_tiles) * 8 + (blk & 7);
    if (nt >= a.tile_off[a.E]) return;
    const int e = a.tile_expert[nt];
    const int p0 = a.expert_off[e] + (nt - a.tile_off[e]) * kTN;
    const int np = min(kTN, a.expert_off[e + 1] - p0);

    const int K = NMAT == 2 ? a.h : a.I;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r = lane & 15, kq = lane >> 4;
    const int row = mt * TM + wave * 16 + r;  // this lane's A row
    const int nblk = K / KB;
    const uint32_t groups = (uint32_t)K >> (5 + GSL);

    // expert sub-blocks (planar [gate W|S|B][up W|S|B][down W|S|B])
    const uint8_t* ex = a.layer_base + (uint64_t)e * a.expert_bytes;
    const uint8_t* px = a.pfs_base + (uint64_t)e * a.pfs_bytes;
    const Layout L(a.h, a.I, a.gs);
    const PfScaleLayout PL(a.h, a.I, a.gs);
    const uint32_t* wrow[NMAT];
    const uint32_t* sbrow[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
        const uint64_t wo = NMAT == 2 ? (m == 0 ? L.gate_w : L.up_w) : L.down_w;
        const uint64_t so = NMAT == 2 ? (m == 0 ? PL.gate : PL.up) : PL.down;
        wrow[m] = reinterpret_cast<const uint32_t*>(ex + wo) + (size_t)row * (K / 8) + kq * W;
        sbrow[m] = reinterpret_cast<const uint32_t*>(px + so) + (size_t)row * groups;
    }

    if (tid < kTN) {
        const bool ok = tid < np;
        const int tok = (NMAT == 2 && ok) ? a.sorted_tok[p0 + tid] : 0;
        s_tok[tid] = tok;
        if (NMAT == 2) s_inv[tid] = ok ? a.xinv[tok] : 0.f;
    }
    __syncthreads();

    // B staging: thread -> (pair j = tid / TPP, part q = tid % TPP: KB/TPP elements)
    const int bj = tid / TPP, bq = tid % TPP;
    const bool b_ok = bj < np;
    const _Float16* b_src =
        (NMAT == 2 ? a.xq + (size_t)s_tok[bj] * a.h : a.act + (size_t)(p0 + (b_ok ? bj : 0)) * a.I) +
        bq * (KB / TPP);
    auto load = [&](int kb, PfStage<NMAT, KB, NW>& st) {
        const uint4* pb = reinterpret_cast<const uint4*>(b_src + kb * KB);
#pragma unroll
        for (int i = 0; i < NB; ++i) st.b[i] = b_ok ? pb[i] : make_uint4(0, 0, 0, 0);
        const uint32_t g = ((uint32_t)kb * KB + (uint32_t)kq * (KB / 4)) >> (5 + GSL);
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            const uint32_t* pw = wrow[m] + (size_t)kb * (KB / 8);
            if constexpr (W % 4 == 0) {
#pragma unroll
                for (int v = 0; v < W / 4; ++v) {
                    const uint4 q = *reinterpret_cast<const uint4*>(pw + 4 * v);
                    st.aw[m][4 * v] = q.x; st.aw[m][4 * v + 1] = q.y;
                    st.aw[m][4 * v + 2] = q.z; st.aw[m][4 * v + 3] = q.w;
                }
            } else {
                const uint2 q = *reinterpret_cast<const uint2*>(pw);
                st.aw[m][0] = q.x; st.aw[m][W > 1 ? 1 : 0] = q.y;
            }
            st.sb[m] = sbrow[m][g];
        }
    };
    auto store_b = [&](int buf, const PfStage<NMAT, KB, NW>& st) {
        uint4* d = reinterpret_cast<uint4*>(&s_b[buf][bj * kRow + bq * (KB / TPP) * 2]);
#pragma unroll
        for (int i = 0; i < NB; ++i) d[i] = permute8(st.b[i]);
    };

    f32x4 acc[NMAT][kTN / 16];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int j = 0; j < kTN / 16; ++j) acc[m][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int buf, const PfStage<NMAT, KB, NW>& st) {
        f16x2 s2[NMAT], b2[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            const uint32_t lo = st.sb[m] & 0xffffu, hi = st.sb[m] >> 16;
            s2[m] = __builtin_bit_cast(f16x2, lo | (lo << 16));
            b2[m] = __builtin_bit_cast(f16x2, hi | (hi << 16));
        }
        // two k-steps at a time: their B fragments are read from LDS and their
        // A fragments unpacked before the 2 * 4 * NMAT MFMAs that use them
        constexpr int SP = W >= 2 ? 2 : 1;
#pragma unroll
        for (int s0 = 0; s0 < W; s0 += SP) {
            f16x8 bf[SP][kTN / 16];
#pragma unroll
            for (int t = 0; t < SP; ++t)
#pragma unroll
                for (int j = 0; j < kTN / 16; ++j)
                    bf[t][j] = *reinterpret_cast<const f16x8*>(
                        &s_b[buf][(j * 16 + r) * kRow + (kq * W + s0 + t) * 16]);
            f16x8 af[SP][NMAT];
#pragma unroll
            for (int t = 0; t < SP; ++t)
#pragma unroll
                for (int m = 0; m < NMAT; ++m) af[t][m] = dequant_word(st.aw[m][s0 + t], s2[m], b2[m]);
#pragma unroll
            for (int t = 0; t < SP; ++t)
#pragma unroll
                for (int j = 0; j < kTN / 16; ++j)
#pragma unroll
                    for (int m = 0; m < NMAT; ++m)
                        acc[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t][m], bf[t][j], acc[m][j], 0, 0, 0);
        }
    };

    PfStage<NMAT, KB, NW> S0, S1;
    load(0, S0);
    if (nblk > 1) load(1, S1);
    store_b(0, S0);
    __syncthreads();
    // iteration kb: LDS holds B(kb); S(kb%2) holds A(kb), S((kb+1)%2) holds block kb+1
    for (int kb = 0; kb < nblk; kb += 2) {
        compute(0, S0);
        if (kb + 2 < nblk) load(kb + 2, S0);
        if (kb + 1 < nblk) store_b(1, S1);
        __syncthreads();
        if (kb + 1 >= nblk) break;
        compute(1, S1);
        if (kb + 3 < nblk) load(kb + 3, S1);
        if (kb + 2 < nblk) store_b(0, S0);
        __syncthreads();
    }
    // epilogue: lane holds column (pair) j*16 + r, rows 4*kq..4*kq+3 of the wave's 16;
    // each row's 2^k comes back on its accumulator
    const int row0 = mt * TM + wave * 16 + 4 * kq;
    float rs[NMAT][4];
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
        const uint64_t ko = NMAT == 2 ? (m == 0 ? PL.kg : PL.ku) : PL.kd;
        const uint32_t k4 = *reinterpret_cast<const uint32_t*>(px + ko + row0);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            rs[m][i] = __uint_as_float((uint32_t)(127 + ((k4 >> (8 * i)) & 0xffu)) << 23);
    }
#pragma unroll
    for (int j = 0; j < kTN / 16; ++j) {
        const int n = j * 16 + r;
        if (n >= np) continue;
        if (NMAT == 2) {
            const float inv = s_inv[n];
            _Float16 o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float g = acc[0][j][i] * rs[0][i] * inv;
                const float u = acc[NMAT - 1][j][i] * rs[NMAT - 1][i] * inv;
                float v = (g / (1.0f + expf(-g))) * u;  // Shaders.metal:148
                v = fminf(fmaxf(v, -65504.f), 65504.f);
                o[i] = (_Float16)v;
            }
            *reinterpret_cast<uint2*>(a.act + (size_t)(p0 + n) * a.I + row0) =
                __builtin_bit_cast(uint2, o);
        } else {
            const f32x4 y = acc[0][j];
            *reinterpret_cast<f32x4*>(a.y + (size_t)(p0 + n) * a.h + row0) =
                f32x4{y[0] * rs[0][0], y[1] * rs[0][1], y[2] * rs[0][2], y[3] * rs[0][3]};
        }
    }
}

// ---- the scale blocks of the prefill GEMMs (PfScaleLayout), made at upload -----------

// One thread per (expert, weight row): the row's power of two k and its
// groups' f16 (s * 2^(18-k), b * 2^-k) pairs.
__global__ __launch_bounds__(256) void pf_scale_copy_kernel(const uint8_t* src, uint64_t src_bytes,
                                                            uint8_t* dst, uint64_t dst_bytes, int E,
                                                            int h, int I, int gs, uint32_t* err) {
    const int rows = 2 * I + h;
    const uint64_t gid = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= (uint64_t)E * rows) return;
    const int e = (int)(gid / rows), ri = (int)(gid - (uint64_t)e * rows);
    const int m = ri < I ? 0 : (ri < 2 * I ? 1 : 2);
    const int row = m == 2 ? ri - 2 * I : ri - m * I;
    const int groups = (m == 2 ? I : h) / gs;
    const Layout L(h, I, gs);
    const PfScaleLayout P(h, I, gs);
    const uint8_t* b = src + (uint64_t)e * src_bytes;
    const uint16_t* sp = reinterpret_cast<const uint16_t*>(
        b + (m == 0 ? L.gate_s : (m == 1 ? L.up_s : L.down_s))) + (size_t)row * groups;
    const uint16_t* bp = reinterpret_cast<const uint16_t*>(
        b + (m == 0 ? L.gate_b : (m == 1 ? L.up_b : L.down_b))) + (size_t)row * groups;
    float ms = 0.f, mw = 0.f;
    bool finite = true;
    for (int g = 0; g < groups; ++g) {
        const float sf = bf16_to_f32(sp[g]), bf = bf16_to_f32(bp[g]);
        finite = finite && isfinite(sf) && isfinite(bf);
        ms = fmaxf(ms, fabsf(sf));
        mw = fmaxf(mw, 15.f * fabsf(sf) + fabsf(bf));
    }
    int k = 0;
    if (!finite) {
        flag_error(err, 8u);
    } else {
        while (k < 100 && (ldexpf(ms, 18 - k) > 65504.f || ldexpf(mw, -k) > 65504.f)) ++k;
    }
    uint8_t* d = dst + (uint64_t)e * dst_bytes;
    d[(m == 0 ? P.kg : (m == 1 ? P.ku : P.kd)) + row] = (uint8_t)k;
    uint32_t* o = reinterpret_cast<uint32_t*>(d + (m == 0 ? P.gate : (m == 1 ? P.up : P.down))) +
                  (size_t)row * groups;
    for (int g = 0; g < groups; ++g) {
        const _Float16 s16 = (_Float16)ldexpf(bf16_to_f32(sp[g]), 18 - k);
        const _Float16 b16 = (_Float16)ldexpf(bf16_to_f32(bp[g]), -k);
        o[g] = (uint32_t)__builtin_bit_cast(uint16_t, s16) |
               ((uint32_t)__builtin_bit_cast(uint16_t, b16) << 16);
    }
}

// ---- combine ----------------------------------------------------------------------

// out[t][d] = residual[t][d] + sum_k w[t][k] * y[pos[t,k]][d], k ascending
// (Shaders.metal:371-374); four columns per thread.
__global__ __launch_bounds__(256) void pf_combine_kernel(PrefillArgs a) {
    const int t = blockIdx.y;
    const int d = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (d >= a.h) return;
    float4 acc = a.residual ? *reinterpret_cast<const float4*>(a.residual + (size_t)t * a.h + d)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k = 0; k < a.K; ++k) {
        const float w = a.w[(size_t)t * a.K + k];
        const float4 y = *reinterpret_cast<const float4*>(
            a.y + (size_t)a.pos[(size_t)t * a.K + k] * a.h + d);
        acc.x = fmaf(w, y.x, acc.x);
        acc.y = fmaf(w, y.y, acc.y);
        acc.z = fmaf(w, y.z, acc.z);
        acc.w = fmaf(w, y.w, acc.w);
    }
    *reinterpret_cast<float4*>(a.out + (size_t)t * a.h + d) = acc;
}

template <int NMAT, int GSL, int NW>
void launch_gemm_nw(const PrefillArgs& a, hipStream_t st, int groups8, int rows) {
    const int K = NMAT == 2 ? a.h : a.I;
    const int m_tiles = rows / (16 * NW);
    const dim3 grid((unsigned)(8 * groups8 * m_tiles));
    // Eight-wave gate/up (two matrices: two waves per SIMD at any k-block)
    // streams 256-wide k-blocks, twice the weight bytes in flight per wave at
    // the same occupancy.  The down GEMM stays at 128: at 256 its registers
    // would leave room for one workgroup per CU instead of two.  A lane's 64
    // columns then still sit in one scale group (group size >= 64).
    if constexpr (NMAT == 2 && NW == 8 && GSL >= 1) {
        if (K % 256 == 0) {
            hipLaunchKernelGGL((pf_gemm_kernel<NMAT, 256, GSL, NW>), grid, dim3(64 * NW), 0, st,
                               a, m_tiles);
            return;
        }
    }
    if (K % 128 == 0)
        hipLaunchKernelGGL((pf_gemm_kernel<NMAT, 128, GSL, NW>), grid, dim3(64 * NW), 0, st, a,
                           m_tiles);
    else
        hipLaunchKernelGGL((pf_gemm_kernel<NMAT, 64, GSL, NW>), grid, dim3(64 * NW), 0, st, a,
                           m_tiles);
}

// Eight waves (128 weight rows) per workgroup where the rows allow it: the
// workgroup's B tile in LDS then feeds twice the rows, halving the B reads.
template <int NMAT, int GSL>
void launch_gemm(const PrefillArgs& a, hipStream_t st, int groups8, int rows) {
    if (rows % 128 == 0)
        launch_gemm_nw<NMAT, GSL, 8>(a, st, groups8, rows);
    else
        launch_gemm_nw<NMAT, GSL, 4>(a, st, groups8, rows);
}

template <int GSL>
int launch_gemms(const PrefillArgs& a, hipStream_t st) {
    const int P = a.T * a.K;
    const int ntiles_max = (P + kTN - 1) / kTN + a.E;
    const int groups8 = (ntiles_max + 7) / 8;
    launch_gemm<2, GSL>(a, st, groups8, a.I);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    launch_gemm<1, GSL>(a, st, groups8, a.h);
    return (int)hipGetLastError();
}

}  // namespace

int launch_pf_scale_copy(const uint8_t* layer, uint64_t expert_bytes, uint8_t* dst, int E,
                         int h, int I, int gs, uint32_t* err, void* stream) {
    const PfScaleLayout P(h, I, gs);
    const uint64_t threads = (uint64_t)E * (uint64_t)(2 * I + h);
    hipLaunchKernelGGL(pf_scale_copy_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256),
                       0, static_cast<hipStream_t>(stream), layer, expert_bytes, dst, P.bytes, E,
                       h, I, gs, err);
    return (int)hipGetLastError();
}

int launch_prefill(const PrefillArgs& a, void* stream) {
    if (a.E > kMaxE || a.h > 16384 || a.h % 64 || a.I % 64) return (int)hipErrorInvalidValue;
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(prep_x_kernel, dim3((unsigned)a.T), dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL(group_kernel, dim3(1), dim3(1024), 0, st, a);
    if ((e = hipGetLastError()) != hipSuccess) return (int)e;
    int rc;
    switch (a.gs) {
        case 32: rc = launch_gemms<0>(a, st); break;
        case 64: rc = launch_gemms<1>(a, st); break;
        case 128: rc = launch_gemms<2>(a, st); break;
        default: return (int)hipErrorInvalidValue;
    }
    if (rc != (int)hipSuccess) return rc;
    hipLaunchKernelGGL(pf_combine_kernel, dim3((unsigned)((a.h / 4 + 255) / 256), (unsigned)a.T),
                       dim3(256), 0, st, a);
    return (int)hipGetLastError();
}

}  // namespace m1moe
