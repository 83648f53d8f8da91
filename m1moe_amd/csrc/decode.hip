// decode.hip — batch-1 MoE block for gfx950 in ONE kernel: router logits and
// top-K, expert dispatch, fused 4-bit group-affine dequant + gate/up matvec +
// SwiGLU, fused dequant + down matvec, weighted combine + residual.
//
// Replaces, per token and layer, the reference's CPU router + selectTopK
// (InferenceEngine.swift:490-519), pread dispatch (:271-280) and the 4K+1
// Metal dispatches (matvec4bit x3 + swiGLU per slot, then moeCombine:
// InferenceEngine.swift:401-478, Shaders.metal:39-92,138-149,360-376).
//
// Roles (by workgroup id; lower ids are dispatched first, and a workgroup
// only waits for lower-id workgroups or for router logits, which the lowest
// ids produce before they wait for anything, so the grid cannot deadlock):
//   [0, n_gu)          gate/up workgroups: (slot k, block of rows) of the
//                      k-th selected expert -> act[k][rows] = silu(g)*u
//   [n_gu, n_gu+n_dn)  down workgroups: a block of output rows for all K
//                      slots; they load their down-weight tiles as soon as
//                      the routing is known, then wait for act[k].
//   Workgroup e < E (wave 0) first publishes router logit e.
//
// Cross-workgroup hand-off uses relaxed agent-scope atomics (sc1 loads and
// stores, coherent across the XCDs' L2s), never release/acquire fences
// (their L2 write-back/invalidate costs microseconds per use).  Logits are
// published as (launch tag, value) pairs that consumers poll directly.
// Finished gate/up workgroups bump one of kActSub spread counters of their
// slot after their act stores have completed (s_waitcnt), so no address sees
// more than a handful of atomics per launch.  Nothing is reset between
// launches: every workgroup counts its own launches (seen[wg]), so all agree
// on the launch number `tag` and on the counters' targets (graph replay
// needs no memset).  Every wait is bounded: on timeout the workgroup raises
// the device error flag and skips its work, so a broken hand-off ends the
// kernel instead of hanging it.
//
// Matvec arithmetic: sum_c (n_c*s_g + b_g) x_c is evaluated as
// sum_g [ s_g * sum_{c in g} n_c x_c + b_g * sum_{c in g} x_c ], the inner
// nibble sums on v_dot2_f32_f16 (exact f16*f16 products, f32 accumulation).
// The input vector is scaled by a power of two (largest element in
// [2^13, 2^14)) and rounded to f16 once; results are scaled back exactly.
#include <hip/hip_runtime.h>

#include "device.hpp"
#include "internal.hpp"

namespace m1moe {
namespace {

constexpr int kWaves = 4;  // waves per workgroup
constexpr int kMaxK = 32;
constexpr int kMaxE = 256;
constexpr int kRS = 2;     // down: wave steps per tile

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
// All of this wave's memory operations have completed (stores acknowledged
// at their scope) before anything after it is issued.
__device__ __forceinline__ void wait_all_mem() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// ---- expert block layout -----------------------------------------------------------

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

// ---- lane maps -------------------------------------------------------------------

struct LaneMap {
    int q;        // row slot within one wave step
    int c0;       // first chunk index
    bool ok;      // lane participates
    int seg;      // reduction segment width (power of two)
    bool writer;  // last lane of its segment: holds the row total
    int wq;       // row slot whose total the writer holds
};

// Chunk = 32 columns = one 128-bit load of nibbles.  C = chunks per row; a
// row with C < 64 dividing 64 shares a wave step with rpi-1 others.
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
        m.seg = (rpi > 1) ? C : 64;
    }
    m.writer = (lane & (m.seg - 1)) == m.seg - 1;
    m.wq = (m.seg < 64) ? lane / m.seg : 0;
    return m;
}

// Loads 32-element chunk c of an f32 or bf16 vector as f32.  The caller
// passes an in-range chunk index (clamped for idle lanes) so the loads are
// unconditional and can all be in flight together; ok = false zeroes them.
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

// f32 chunk written by other workgroups in this launch: coherent 64-bit loads
// (same in-range/ok convention as load_chunk).
__device__ __forceinline__ void load_chunk_coherent(const float* x, int c, bool ok,
                                                    float (&v)[32]) {
    const unsigned long long* p = reinterpret_cast<const unsigned long long*>(x + c * 32);
    unsigned long long u[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) u[i] = ld_u64(p + i);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        v[2 * i] = ok ? __uint_as_float((uint32_t)u[i]) : 0.f;
        v[2 * i + 1] = ok ? __uint_as_float((uint32_t)(u[i] >> 32)) : 0.f;
    }
}

// Scale and bias of one group as the aligned dword holding the bf16 (a 32-bit
// load keeps the compiler from merging halves with ordered d16 loads).
struct SBIdx {
    uint32_t word;  // byte offset of the dword
    bool hi;        // the bf16 is the upper half
};
__device__ __forceinline__ SBIdx sb_index(uint32_t elem) {
    return SBIdx{(elem >> 1) << 2, (elem & 1u) != 0};
}
__device__ __forceinline__ float sb_pick(uint32_t w, bool hi) {
    return hi ? __uint_as_float(w & 0xFFFF0000u) : __uint_as_float(w << 16);
}

// Scale a lane's chunks by the wave-wide power of two and convert to the f16
// pairs of the nibble dot product.  All 64 lanes must call it.
template <int N>
__device__ __forceinline__ float scale_and_prep(float (&v)[N][32], XChunk (&xc)[N]) {
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < N; ++j)
#pragma unroll
        for (int e = 0; e < 32; ++e) mx = fmaxf(mx, fabsf(v[j][e]));
    mx = wave_max(mx);
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

// ---- router --------------------------------------------------------------------

template <bool XBF16>
__device__ __forceinline__ double logit_partial(const FusedArgs& a, const uint16_t* wr, int lane) {
    double acc = 0.0;
    // 8 columns per lane per step; 4 steps' loads in flight at once
    for (int d0 = lane * 8; d0 < a.h; d0 += 4 * 512) {
        uint4 wv[4];
        uint4 xb[4];
        float4 xf[4][2];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int d = min(d0 + s * 512, a.h - 8);
            wv[s] = *reinterpret_cast<const uint4*>(wr + d);
            if (XBF16) {
                xb[s] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.x) + d);
            } else {
                const float* xr = static_cast<const float*>(a.x) + d;
                xf[s][0] = *reinterpret_cast<const float4*>(xr);
                xf[s][1] = *reinterpret_cast<const float4*>(xr + 4);
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            if (d0 + s * 512 < a.h) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    float xv;
                    if (XBF16) {
                        xv = bf16x8_at(xb[s], i);
                    } else {
                        const float4 q = xf[s][i >> 2];
                        xv = (i & 3) == 0 ? q.x : (i & 3) == 1 ? q.y : (i & 3) == 2 ? q.z : q.w;
                    }
                    acc += (double)bf16x8_at(wv[s], i) * (double)xv;
                }
            }
        }
    }
    return acc;
}

// Logit e (exact bf16*x products, f64 sum, one rounding, + bias), published
// by lane 0 as (tag << 32 | bits).  seen_raw: this workgroup's launch count as
// loaded by lane 0 (the load stays in flight behind the logit's own loads).
__device__ __forceinline__ void produce_logit(const FusedArgs& a, int e, int lane,
                                              uint32_t seen_raw) {
    const uint16_t* wr = a.router + (size_t)e * a.h;
    double acc = a.x_bf16 ? logit_partial<true>(a, wr, lane) : logit_partial<false>(a, wr, lane);
    acc = wave_sum_f64_last(acc);
    const uint32_t tag = __builtin_amdgcn_readfirstlane(seen_raw) + 1u;
    if (lane == 63) {
        float l = (float)acc;
        if (a.bias) l = l + a.bias[e];
        st_u64(a.slots + e, ((unsigned long long)tag << 32) | __float_as_uint(l));
    }
}

// Wave 0: obtain the routing (poll the published logits, rank, softmax) or
// read the given one; writes s_idx/s_w.  Returns false on timeout.
__device__ bool routing(const FusedArgs& a, int lane, uint32_t tag, int* s_idx, float* s_w) {
    const int E = a.E, K = a.K;
    if (a.given_idx) {
        if (lane < K) {
            int e = a.given_idx[lane];
            if (e < 0 || e >= E) {
                flag_error(a.err, 1u);
                e = -1;
            }
            s_idx[lane] = e;
            s_w[lane] = a.given_w[lane];
        }
        return true;
    }
    float v[4];
    bool have[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        have[j] = (lane + 64 * j >= E);
        v[j] = -INFINITY;
    }
    for (int it = 0;; ++it) {
        bool all = true;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (!have[j]) {
                const unsigned long long u = ld_u64(a.slots + lane + 64 * j);
                if ((uint32_t)(u >> 32) == tag) {
                    have[j] = true;
                    const float f = __uint_as_float((uint32_t)u);
                    v[j] = (f != f) ? -INFINITY : f;  // NaN ranks last
                } else {
                    all = false;
                }
            }
        }
        if (__all(all)) break;
        if (it >= a.spin_limit) {
            flag_error(a.err, 2u);
            return false;
        }
        __builtin_amdgcn_s_sleep(4);
    }
    int my_idx;
    float w;
    topk_softmax(v, E, K, a.norm, lane, my_idx, w);
    if (lane < K) {
        s_idx[lane] = my_idx;
        s_w[lane] = w;
    }
    return true;
}

// ---- gate/up ---------------------------------------------------------------------

// GSL = log2(group_size / 32): group of chunk c is c >> GSL.
template <int CPL, int U, int GSL>
__device__ void gate_up_role(const FusedArgs& a, const Layout& L, int k, int rb, int wave,
                             int lane, const XChunk (&xc)[CPL], float inv, int e) {
    const uint8_t* blk = a.layer_base + (uint64_t)e * a.expert_bytes;
    const uint8_t* gw_p = blk + L.gate_w;
    const uint8_t* uw_p = blk + L.up_w;
    const uint8_t* gs_p = blk + L.gate_s;
    const uint8_t* gb_p = blk + L.gate_b;
    const uint8_t* us_p = blk + L.up_s;
    const uint8_t* ub_p = blk + L.up_b;
    const LaneMap m = lane_map(lane, a.Cg, a.rpi_g);
    const uint32_t groups = (uint32_t)a.h >> (5 + GSL);
    const uint32_t row_bytes = (uint32_t)a.h / 2;
    const int row0 = (rb * kWaves + wave) * U * a.rpi_g + m.q;

    uint4 gw[U][CPL], uw[U][CPL];
    uint32_t gsc[U][CPL], gbi[U][CPL], usc[U][CPL], ubi[U][CPL];
    bool okv[U][CPL], hi[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int row = row0 + u * a.rpi_g;
        const uint32_t rc = (uint32_t)min(row, a.I - 1);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = m.c0 + 64 * j;
            const uint32_t cc = (uint32_t)min(c, a.Cg - 1);
            okv[u][j] = m.ok && row < a.I && c < a.Cg;
            const uint64_t wo = (uint64_t)(rc * row_bytes + cc * 16u);
            const SBIdx sb = sb_index(rc * groups + (cc >> GSL));
            hi[u][j] = sb.hi;
            gw[u][j] = *reinterpret_cast<const uint4*>(gw_p + wo);
            uw[u][j] = *reinterpret_cast<const uint4*>(uw_p + wo);
            gsc[u][j] = *reinterpret_cast<const uint32_t*>(gs_p + sb.word);
            gbi[u][j] = *reinterpret_cast<const uint32_t*>(gb_p + sb.word);
            usc[u][j] = *reinterpret_cast<const uint32_t*>(us_p + sb.word);
            ubi[u][j] = *reinterpret_cast<const uint32_t*>(ub_p + sb.word);
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        float pg = 0.f, pu = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const float dg = nib_dot32(gw[u][j], xc[j]) - xc[j].off;
            const float du = nib_dot32(uw[u][j], xc[j]) - xc[j].off;
            const float tg = fmaf(sb_pick(gsc[u][j], hi[u][j]), dg,
                                  sb_pick(gbi[u][j], hi[u][j]) * xc[j].xs);
            const float tu = fmaf(sb_pick(usc[u][j], hi[u][j]), du,
                                  sb_pick(ubi[u][j], hi[u][j]) * xc[j].xs);
            pg += okv[u][j] ? tg : 0.f;
            pu += okv[u][j] ? tu : 0.f;
        }
        pg = seg_sum(pg, m.seg);
        pu = seg_sum(pu, m.seg);
        // the segment's total is in its last lane; that lane's row slot is
        // m.q when rows share the wave, else 0
        const int row = row0 - m.q + m.wq + u * a.rpi_g;
        if (m.writer && row < a.I) {
            const float gv = pg * inv, uv = pu * inv;
            st_f32(a.act + (size_t)k * a.I + row, (gv / (1.0f + expf(-gv))) * uv);  // Shaders.metal:148
        }
    }
}

// ---- down + combine ----------------------------------------------------------------

struct DownTile {
    uint4 w[kRS];
    uint32_t s[kRS], b[kRS];
    bool hi[kRS], ok[kRS];
};

// task t = (slot k = t / Sc, column slice j = t % Sc) over this block's rows;
// loads are unconditional at clamped addresses, invalid lanes masked later
template <int GSL>
__device__ __forceinline__ void load_down_tile(const FusedArgs& a, const Layout& L, int t, int T,
                                               int row_base, const LaneMap& m, const int* s_idx,
                                               DownTile& d) {
    const int tt = min(t, T - 1);
    const int k = tt / a.Sc, j = tt - k * a.Sc;
    const int e = s_idx[k];
    const int c = m.c0 + 64 * j;
    const uint32_t cc = (uint32_t)min(c, a.Cd - 1);
    const bool ok0 = (t < T) && (e >= 0) && m.ok && c < a.Cd;
    const uint8_t* blk = a.layer_base + (uint64_t)(e < 0 ? 0 : e) * a.expert_bytes;
    const uint8_t* w_p = blk + L.down_w;
    const uint8_t* s_p = blk + L.down_s;
    const uint8_t* b_p = blk + L.down_b;
    const uint32_t groups = (uint32_t)a.I >> (5 + GSL);
    const uint32_t row_bytes = (uint32_t)a.I / 2;
#pragma unroll
    for (int s = 0; s < kRS; ++s) {
        const int row = row_base + s * a.rpi_d + m.q;
        const uint32_t rc = (uint32_t)min(row, a.h - 1);
        d.ok[s] = ok0 && row < a.h;
        const SBIdx sb = sb_index(rc * groups + (cc >> GSL));
        d.hi[s] = sb.hi;
        d.w[s] = *reinterpret_cast<const uint4*>(w_p + (uint64_t)(rc * row_bytes + cc * 16u));
        d.s[s] = *reinterpret_cast<const uint32_t*>(s_p + sb.word);
        d.b[s] = *reinterpret_cast<const uint32_t*>(b_p + sb.word);
    }
}

// Waits until every gate/up workgroup of slot k has finished: sub-counter i
// gains the number of those workgroups with rb % kActSub == i per launch.
__device__ __forceinline__ bool wait_slot(const FusedArgs& a, int k, int lane, uint32_t tag) {
    const uint32_t n = (uint32_t)a.gu_per_slot;
    const uint32_t per = n / kActSub + ((uint32_t)lane < n % kActSub ? 1u : 0u);
    const uint32_t want = tag * per;
    const uint32_t* p = a.act_cnt + ((size_t)k * kActSub + (lane & (kActSub - 1))) * kActCntStride;
    for (int it = 0;; ++it) {
        const bool done = lane >= kActSub || ld_u32(p) == want;
        if (__all(done)) return true;
        if (it >= a.spin_limit) return false;
        __builtin_amdgcn_s_sleep(4);
    }
}

__device__ __forceinline__ void compute_down_tile(const FusedArgs& a, int t, int lane,
                                                  const LaneMap& m, const int* s_idx,
                                                  const DownTile& d, float* s_part, uint32_t tag,
                                                  bool& ok_run) {
    const int k = t / a.Sc, j = t - k * a.Sc;
    const int R2 = kRS * a.rpi_d;
    float* part = s_part + (k * a.Sc + j) * R2;
    if (s_idx[k] < 0 || !ok_run || !wait_slot(a, k, lane, tag)) {
        if (ok_run && s_idx[k] >= 0) {
            flag_error(a.err, 4u);
            ok_run = false;
        }
        for (int r = lane; r < R2; r += 64) part[r] = 0.f;
        return;
    }
    const int c = m.c0 + 64 * j;
    float v[1][32];
    load_chunk_coherent(a.act + (size_t)k * a.I, min(c, a.Cd - 1), m.ok && c < a.Cd, v[0]);
    XChunk xc[1];
    const float inv = scale_and_prep<1>(v, xc);
#pragma unroll
    for (int s = 0; s < kRS; ++s) {
        const float dd = nib_dot32(d.w[s], xc[0]) - xc[0].off;
        float p = fmaf(sb_pick(d.s[s], d.hi[s]), dd, sb_pick(d.b[s], d.hi[s]) * xc[0].xs);
        p = d.ok[s] ? p : 0.f;
        p = seg_sum(p, m.seg);
        if (m.writer) part[s * a.rpi_d + m.wq] = p * inv;
    }
}

template <int GSL>
__device__ void down_role(const FusedArgs& a, const Layout& L, int dblk, int wave, int lane,
                          const int* s_idx, const float* s_w, float* s_part, uint32_t tag,
                          bool ok_run) {
    const int R2 = kRS * a.rpi_d;
    const int row_base = dblk * R2;
    const int T = a.K * a.Sc;
    const LaneMap m = lane_map(lane, a.Cd, a.rpi_d);
    // two tiles in flight per wave: tasks wave, wave+4, wave+8, ...
    DownTile A, B;
    load_down_tile<GSL>(a, L, wave, T, row_base, m, s_idx, A);
    load_down_tile<GSL>(a, L, wave + kWaves, T, row_base, m, s_idx, B);
    for (int t = wave; t < T; t += 2 * kWaves) {
        compute_down_tile(a, t, lane, m, s_idx, A, s_part, tag, ok_run);
        load_down_tile<GSL>(a, L, t + 2 * kWaves, T, row_base, m, s_idx, A);
        if (t + kWaves < T) {
            compute_down_tile(a, t + kWaves, lane, m, s_idx, B, s_part, tag, ok_run);
            load_down_tile<GSL>(a, L, t + 3 * kWaves, T, row_base, m, s_idx, B);
        }
    }
    __syncthreads();
    // combine in slot order, column slices summed in order (Shaders.metal:371-374)
    for (int r = threadIdx.x; r < R2; r += blockDim.x) {
        const int row = row_base + r;
        if (row >= a.h) continue;
        float acc = a.residual ? a.residual[row] : 0.f;
        for (int k = 0; k < a.K; ++k) {
            float y = 0.f;
            for (int j = 0; j < a.Sc; ++j) y += s_part[(k * a.Sc + j) * R2 + r];
            acc = fmaf(s_w[k], y, acc);
        }
        a.out[row] = acc;
    }
}

// ---- the kernel --------------------------------------------------------------------

template <int CPL, int U, int GSL>
__global__ __launch_bounds__(256, CPL == 1 ? 4 : 1) void moe_decode_kernel(FusedArgs a) {
    __shared__ int s_idx[kMaxK];
    __shared__ float s_w[kMaxK];
    __shared__ int s_ok;
    __shared__ uint32_t s_tag;
    extern __shared__ float s_part[];  // down role: [K][Sc][R2]
    const int wg = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const bool is_gu = wg < a.n_gu;

    // this launch's number, as counted by this workgroup (all agree)
    uint32_t tag = 0;
    if (wave == 0) {
        uint32_t s = 0;
        if (lane == 0) s = ld_u32(a.seen + wg);
        if (!a.given_idx)
            for (int e = wg; e < a.E; e += gridDim.x) produce_logit(a, e, lane, s);
        tag = __builtin_amdgcn_readfirstlane(s) + 1u;
    }

    // the input vector does not depend on the routing: prepare it meanwhile
    XChunk xc[CPL];
    float inv = 1.f;
    if (is_gu) {
        const LaneMap m = lane_map(lane, a.Cg, a.rpi_g);
        float v[CPL][32];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = m.c0 + 64 * j;
            load_chunk(a.x, a.x_bf16, min(c, a.Cg - 1), m.ok && c < a.Cg, v[j]);
        }
        inv = scale_and_prep<CPL>(v, xc);
    }

    if (wave == 0) {
        const bool ok = routing(a, lane, tag, s_idx, s_w);
        if (lane == 0) {
            s_ok = ok ? 1 : 0;
            s_tag = tag;
        }
        if (ok && wg == 0 && lane < a.K) {
            if (a.user_idx) a.user_idx[lane] = s_idx[lane];
            if (a.user_w) a.user_w[lane] = s_w[lane];
        }
    }
    __syncthreads();
    const bool ok_run = s_ok != 0;
    tag = s_tag;
    const Layout L(a.h, a.I, a.gs);

    if (is_gu) {
        const int k = wg / a.gu_per_slot, rb = wg - k * a.gu_per_slot;
        const int e = s_idx[k];
        if (ok_run && e >= 0) gate_up_role<CPL, U, GSL>(a, L, k, rb, wave, lane, xc, inv, e);
        wait_all_mem();
        __syncthreads();
        if (threadIdx.x == 0)
            add_u32(a.act_cnt + ((size_t)k * kActSub + (rb & (kActSub - 1))) * kActCntStride, 1u);
    } else {
        down_role<GSL>(a, L, wg - a.n_gu, wave, lane, s_idx, s_w, s_part, tag, ok_run);
    }
    if (threadIdx.x == 0) st_u32(a.seen + wg, tag);
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

// Several rows share a wave step only when the row's chunk count divides 64
// (a power of two), so each row owns an aligned power-of-two lane segment.
inline int rows_per_step(int C) { return (C < 64 && 64 % C == 0) ? 64 / C : 1; }
constexpr int gu_steps(int cpl) { return cpl == 1 ? 4 : cpl == 2 ? 2 : 1; }

template <int CPL, int GSL>
int launch_shape(const FusedArgs& a, hipStream_t st) {
    const int R2 = kRS * a.rpi_d;
    const size_t lds = sizeof(float) * (size_t)a.K * a.Sc * R2;
    if (lds > 64 * 1024) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL((moe_decode_kernel<CPL, gu_steps(CPL), GSL>),
                       dim3((unsigned)(a.n_gu + a.n_dn)), dim3(64 * kWaves), lds, st, a);
    return (int)hipGetLastError();
}

template <int CPL>
int launch_cpl(const FusedArgs& a, hipStream_t st) {
    switch (a.gs) {
        case 32: return launch_shape<CPL, 0>(a, st);
        case 64: return launch_shape<CPL, 1>(a, st);
        case 128: return launch_shape<CPL, 2>(a, st);
        default: return (int)hipErrorInvalidValue;
    }
}

}  // namespace

int decode_grid(FusedArgs& a) {
    const int cpl = (a.h / 32 + 63) / 64;
    a.Cg = a.h / 32;
    a.rpi_g = rows_per_step(a.Cg);
    const int rows_gu = kWaves * gu_steps(cpl) * a.rpi_g;
    a.gu_per_slot = (a.I + rows_gu - 1) / rows_gu;
    a.n_gu = a.K * a.gu_per_slot;
    a.Cd = a.I / 32;
    a.rpi_d = rows_per_step(a.Cd);
    a.Sc = a.Cd >= 64 ? (a.Cd + 63) / 64 : 1;
    const int R2 = kRS * a.rpi_d;
    a.n_dn = (a.h + R2 - 1) / R2;
    return a.n_gu + a.n_dn;
}

int launch_moe_decode(const FusedArgs& a_in, void* stream) {
    if (a_in.E > kMaxE || a_in.K > kMaxK) return (int)hipErrorInvalidValue;
    FusedArgs a = a_in;
    decode_grid(a);
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch ((a.h / 32 + 63) / 64) {
        case 1: return launch_cpl<1>(a, st);
        case 2: return launch_cpl<2>(a, st);
        case 3: return launch_cpl<3>(a, st);
        case 4: return launch_cpl<4>(a, st);
        case 5: return launch_cpl<5>(a, st);
        case 6: return launch_cpl<6>(a, st);
        case 7: return launch_cpl<7>(a, st);
        case 8: return launch_cpl<8>(a, st);
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
