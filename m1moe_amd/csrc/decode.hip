// decode.hip — batch-1 MoE block for gfx950 in ONE kernel: router logits and
// top-K, expert dispatch, fused 4-bit group-affine dequant + gate/up matvec +
// SwiGLU, fused dequant + down matvec, weighted combine + residual.
//
// Replaces, per token and layer, the reference's CPU router + selectTopK
// (InferenceEngine.swift:490-519), pread dispatch (:271-280) and the 4K+1
// Metal dispatches (matvec4bit x3 + swiGLU per slot, then moeCombine:
// InferenceEngine.swift:401-478, Shaders.metal:39-92,138-149,360-376).
//
// Roles by workgroup id (lower ids are dispatched first; a workgroup only
// waits for lower-id workgroups or for router logits, which the lowest ids
// publish before they wait for anything, so the grid cannot deadlock):
//   [0, n_gu)          gate/up workgroups: (slot k, block of rows) of the
//                      k-th selected expert, slot-major.  All of a
//                      workgroup's weight loads are issued at once (for a
//                      few-MB working set the whole layer must be in flight
//                      to cover the loaded HBM latency); it writes
//                      act[k][rows] = silu(g) * u, then counts the tile
//                      for the down unit that reads those rows.
//   [n_gu, grid)       down workgroups: Rd output rows for all K slots.  Each
//                      lane owns one (slot, 32-column chunk) of the down
//                      projection; its weights for all Rd rows are loaded as
//                      soon as the routing is known, then it waits for its
//                      unit's counters, converts its chunk of act once and
//                      sweeps the rows.  Slots are combined in slot order in
//                      LDS (deterministic, no atomics), plus the residual.
//   Workgroup e < E first publishes router logit e (all four waves).
//
// Hand-off.  Relaxed agent-scope atomics and 128-bit sc1 loads of act (sc1
// accesses are coherent across the XCDs' L2s), never release/acquire fences
// (an L2 write-back or invalidate costs microseconds).  Logits are published as (launch tag,
// value) pairs into kLogitRep replicas, and a workgroup polls replica
// wg % kLogitRep; tile counters have kNRep replicas.  Nothing is
// reset between launches: every workgroup counts its own launches (seen[wg]),
// so all agree on the launch number `tag` and on the counters' targets
// (graph replay needs no memset).  Every wait is bounded: on timeout the
// workgroup raises the device error flag and skips its work but still does
// all of its counter updates, so the kernel always ends and the counters stay
// in step.
//
// Matvec arithmetic: sum_c (n_c*s_g + b_g) x_c is evaluated as
// sum_g [ s_g * sum_{c in g} n_c x_c + b_g * sum_{c in g} x_c ], the inner
// nibble sums on v_dot2_f32_f16 (exact f16*f16 products, f32 accumulation).
// Each lane scales its 32-element input chunk by a power of two (largest
// element in [2^13, 2^14)) and rounds it to f16 once; its partial sum is
// scaled back exactly before the cross-lane reduction.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "decode_common.hpp"
#include "device.hpp"
#include "internal.hpp"

namespace m1moe {
namespace {

constexpr int kWaves = kDecodeWaves;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxK = 32;
constexpr int kMaxE = 256;
constexpr int kRT = 4;          // down rows per sub-tile
constexpr int kDnTarget = 256;  // down workgroups
constexpr int kGuMax = 512;     // gate/up workgroups (persistent beyond that many tiles)

static_assert(kWaves >= 4, "the router splits a logit over four waves");

// ---- router --------------------------------------------------------------------

// Logit e: exact bf16*x products summed in f64, rounded once to f32, plus the
// bias.  Wave w < 4 sums columns 8w..8w+7 of every 32-column chunk; the wave
// partials are added in wave order.  Published to every replica as
// (tag << 32 | bits).  Every thread of the workgroup calls it; s_tag must be
// visible (a barrier after it was written) before the call.
// rms / need_rms: a normalised input's scale, computed at the first call.
// All of a wave's loads (router row, x, norm weights, the partial sums of
// squares) are issued before any is used: one memory round trip.  CPL =
// ceil(h / 2048) column blocks per lane.
template <int CPL>
__device__ void produce_logit(const FusedArgs& a, int e, int wave, int lane, uint32_t* s_tag,
                              uint32_t tag_reg, double* s_lp, float& rms, bool& need_rms) {
    if (wave < 4) {
        const uint16_t* wr = a.router + (size_t)e * a.h;
        const int C = a.h / 32;
        const bool norm = !a.x_bf16 && a.x_norm_w;
        uint4 wv[CPL], xb[CPL], nw[CPL];
        float4 xf[CPL][2];
        int dd[CPL];
#pragma unroll
        for (int it = 0; it < CPL; ++it) {
            const int c = lane + 64 * it;
            dd[it] = (c < C ? c : 0) * 32 + wave * 8;
            wv[it] = *reinterpret_cast<const uint4*>(wr + dd[it]);
            if (a.x_bf16) {
                xb[it] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.x) + dd[it]);
            } else {
                const float* xr = static_cast<const float*>(a.x) + dd[it];
                xf[it][0] = *reinterpret_cast<const float4*>(xr);
                xf[it][1] = *reinterpret_cast<const float4*>(xr + 4);
                if (norm) nw[it] = *reinterpret_cast<const uint4*>(a.x_norm_w + dd[it]);
            }
        }
        if (norm && need_rms) {  // uniform: every lane of the wave is here
            rms = input_rms(a, lane);
            need_rms = false;
        }
        double acc = 0.0;
#pragma unroll
        for (int it = 0; it < CPL; ++it) {
            float xv[8];
            if (a.x_bf16) {
#pragma unroll
                for (int i = 0; i < 8; ++i) xv[i] = bf16x8_at(xb[it], i);
            } else {
                xv[0] = xf[it][0].x; xv[1] = xf[it][0].y; xv[2] = xf[it][0].z; xv[3] = xf[it][0].w;
                xv[4] = xf[it][1].x; xv[5] = xf[it][1].y; xv[6] = xf[it][1].z; xv[7] = xf[it][1].w;
                if (norm) {  // the norm of Shaders.metal:121-134
#pragma unroll
                    for (int i = 0; i < 8; ++i) xv[i] = xv[i] * rms * bf16x8_at(nw[it], i);
                }
            }
            if (lane + 64 * it < C) {
#pragma unroll
                for (int i = 0; i < 8; ++i) acc += (double)bf16x8_at(wv[it], i) * (double)xv[i];
            }
        }
        acc = wave_sum_f64_last(acc);
        if (lane == 63) s_lp[wave] = acc;
    }
    if (threadIdx.x == 0) *s_tag = tag_reg;  // after the row loads were issued
    __syncthreads();
    if (wave == 0 && lane < kLogitRep) {
        double t = s_lp[0];
        t += s_lp[1];
        t += s_lp[2];
        t += s_lp[3];
        float l = (float)t;
        if (a.bias) l = l + a.bias[e];
        st_u64(a.slots + (size_t)lane * kRepStride + e,
               ((unsigned long long)*s_tag << 32) | __float_as_uint(l));
    }
    __syncthreads();  // s_lp is reused by the next logit
}

// Routing state shared by the workgroup.
struct RouteLDS {
    alignas(16) float v[kMaxE];  // logits, NaN as -inf (kMaxE is a multiple of 16)
    int rk[kWaves][kMaxE];    // partial ranks
    int idx[kMaxK];           // expert of each slot (-1: invalid)
    float w[kMaxK];           // probability of each slot (not renormalised)
    int ok;
};

// Obtains the routing (wave 0 polls the published logits; the ranks are
// counted by all waves; wave 0 ranks and computes the softmax) or reads the
// given one.  Every thread calls it; r.idx / r.w / r.ok are valid after it.
__device__ void routing(const FusedArgs& a, int wg, int wave, int lane, uint32_t tag,
                        RouteLDS& r) {
    const int E = a.E, K = a.K;
    if (a.given_idx) {
        if (threadIdx.x < (unsigned)K) {
            int e = a.given_idx[threadIdx.x];
            if (e < 0 || e >= E) {
                flag_error(a.err, 1u);
                e = -1;
            }
            r.idx[threadIdx.x] = e;
            r.w[threadIdx.x] = a.given_w[threadIdx.x];
        }
        if (threadIdx.x == 0) r.ok = 1;
        __syncthreads();
        return;
    }
    if (wave == 0) {
        const unsigned long long* rep = a.slots + (size_t)(wg & (kLogitRep - 1)) * kRepStride;
        float v[4];
        bool have[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            have[j] = (lane + 64 * j >= E);
            v[j] = -INFINITY;
        }
        bool ok = true;
        for (int it = 0;; ++it) {
            bool all = true;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (!have[j]) {
                    const unsigned long long u = ld_u64(rep + lane + 64 * j);
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
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) r.v[lane + 64 * j] = v[j];  // -inf beyond E
        if (lane == 0) r.ok = ok ? 1 : 0;
    }
    __syncthreads();
    // rank of expert i = experts ahead of it (descending logit, ties to the
    // lower index); wave w counts over experts [j0, j1)
    // (windows of 16 logits, read four at a time into registers)
    for (int j0 = wave * 16; j0 < E; j0 += kWaves * 16) {
        float4 win[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) win[q] = *reinterpret_cast<const float4*>(&r.v[j0 + 4 * q]);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int i = lane + 64 * m;
            if (i < E) {
                const float my = r.v[i];
                int cnt = j0 == wave * 16 ? 0 : r.rk[wave][i];
                // padding beyond E is -inf at an index above i: never ahead
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float wv[4] = {win[q].x, win[q].y, win[q].z, win[q].w};
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int j = j0 + 4 * q + t;
                        cnt += (int)(wv[t] > my) | ((int)(wv[t] == my) & (int)(j < i));
                    }
                }
                r.rk[wave][i] = cnt;
            }
        }
    }
    if (wave * 16 >= E)
        for (int m = 0; m < 4; ++m)
            if (lane + 64 * m < E) r.rk[wave][lane + 64 * m] = 0;
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int i = lane + 64 * m;
            if (i < E) {
                int rank = 0;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) rank += r.rk[w][i];
                if (rank < K) r.idx[rank] = i;
            }
        }
    }
    __syncthreads();
}

// Softmax probabilities of the selected experts (InferenceEngine.swift:
// 501-506) into r.w, from the logits left in r.v by routing().  Wave 0 of
// the workgroups that need the weights calls it (a barrier must follow before
// other waves read r.w); given weights are kept as supplied.
__device__ void routing_weights(const FusedArgs& a, int lane, RouteLDS& r) {
    if (a.given_idx) return;
    const int E = a.E, K = a.K;
    float v[4], mx = -INFINITY;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        v[m] = (lane + 64 * m < E) ? r.v[lane + 64 * m] : -INFINITY;
        mx = fmaxf(mx, v[m]);
    }
    mx = wave_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int m = 0; m < 4; ++m) sum += (lane + 64 * m < E) ? expf(v[m] - mx) : 0.f;
    const float inv = 1.0f / wave_sum(sum);
    if (lane < K) {
        const int e = r.idx[lane];
        r.w[lane] = expf(r.v[e] - mx) * inv;
    }
}

// Weight of slot k: the probability, renormalised over the selection in slot
// order when norm_topk_prob is set (InferenceEngine.swift:514-517).  Given
// weights are used as supplied.
__device__ __forceinline__ float slot_weight(const FusedArgs& a, const float* s_w, int k) {
    if (!a.norm || a.given_idx) return s_w[k];
    float ssum = 0.f;
    for (int r = 0; r < a.K; ++r) ssum = ssum + s_w[r];
    return s_w[k] / ssum;
}

// ---- gate/up ---------------------------------------------------------------------

// Lane geometry of a gate/up row: rows of C >= 64 chunks give a lane chunks
// lane, lane+64, ...; shorter rows share a wave step, seg lanes (a power of
// two) per row.
struct GUGeo {
    int q;       // row slot within a wave step
    int c0;      // first chunk
    bool ok;     // lane has a chunk
    bool writer; // last lane of its segment (holds the row total)
};
__device__ __forceinline__ GUGeo gu_geo(int lane, int C, int seg) {
    GUGeo m;
    m.q = lane / seg;
    m.c0 = lane - m.q * seg;
    m.ok = m.c0 < C;
    m.writer = (lane & (seg - 1)) == seg - 1;
    return m;
}

template <int CPL, int UG>
struct GUTile {
    uint4 gw[UG][CPL], uw[UG][CPL];
    uint32_t gs[UG][CPL], gb[UG][CPL], us[UG][CPL], ub[UG][CPL];
};

// GSL = log2(group_size / 32): the group of chunk c is c >> GSL.  A load that
// is not `real` (a prefetch past the last tile) reads the first 16 bytes of
// the layer in every lane instead: one line, an L2 hit after its first use.
template <int CPL, int UG, int GSL>
__device__ __forceinline__ void gu_load(const FusedArgs& a, const Layout& L, int e, int row0,
                                        bool real, const GUGeo& m, GUTile<CPL, UG>& t) {
    // e is wave-uniform: keep the sub-block bases in scalar registers and
    // address with 32-bit lane offsets
    const uint8_t* blk = a.layer_base +
        (real ? (uint64_t)__builtin_amdgcn_readfirstlane(e) * a.expert_bytes : 0);
    const uint8_t* gw_b = blk + (real ? L.gate_w : 0);
    const uint8_t* uw_b = blk + (real ? L.up_w : 0);
    const uint8_t* gs_b = blk + (real ? L.gate_s : 0);
    const uint8_t* gb_b = blk + (real ? L.gate_b : 0);
    const uint8_t* us_b = blk + (real ? L.up_s : 0);
    const uint8_t* ub_b = blk + (real ? L.up_b : 0);
    const uint32_t groups = (uint32_t)a.h >> (5 + GSL);
    const uint32_t row_bytes = (uint32_t)a.h / 2;
#pragma unroll
    for (int u = 0; u < UG; ++u) {
        const uint32_t rc = (uint32_t)min(row0 + u * a.rpi_g, a.I - 1);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint32_t cc = (uint32_t)min(m.c0 + 64 * j, a.Cg - 1);
            const uint32_t wo = real ? rc * row_bytes + cc * 16u : 0u;
            const uint32_t sbw = real ? sb_word(rc * groups + (cc >> GSL)) : 0u;
            t.gw[u][j] = ld_stream(gw_b + wo);
            t.uw[u][j] = ld_stream(uw_b + wo);
            t.gs[u][j] = *reinterpret_cast<const uint32_t*>(gs_b + sbw);
            t.gb[u][j] = *reinterpret_cast<const uint32_t*>(gb_b + sbw);
            t.us[u][j] = *reinterpret_cast<const uint32_t*>(us_b + sbw);
            t.ub[u][j] = *reinterpret_cast<const uint32_t*>(ub_b + sbw);
        }
    }
}

// act values carry the launch number's parity in their lowest mantissa bit:
// every launch rewrites every act entry (tagged zeros for a slot without an
// expert), so an entry holds this launch's value or the previous launch's,
// and the parity tells them apart.  The consumer clears the bit before use (a
// relative change below 2^-22, the same in every launch) and splits the value
// into hi + lo f16 halves (22 significant bits).
#ifndef M1MOE_ACT_TAG_BITS
#define M1MOE_ACT_TAG_BITS 1
#endif
constexpr uint32_t kActTagMask = (1u << M1MOE_ACT_TAG_BITS) - 1u;
__device__ __forceinline__ float act_tagged(float v, uint32_t tag) {
    return __uint_as_float((__float_as_uint(v) & ~kActTagMask) | (tag & kActTagMask));
}

// The gate/up input chunk: split hi + lo (f32 inputs keep 22 significant
// bits) for up to two chunks per lane, within the 256 VGPRs of two waves per
// SIMD; wider inputs keep single f16 chunks.
template <int CPL>
using GUChunk = typename std::conditional<CPL <= 2, XChunk2, XChunk>::type;

template <int CPL, int UG, int GSL, bool LO>
__device__ __forceinline__ void gu_compute(const FusedArgs& a, int k, int row0, const GUGeo& m,
                                           const GUTile<CPL, UG>& t, const GUChunk<CPL> (&xc)[CPL],
                                           float inv, uint32_t tag) {
    const uint32_t groups = (uint32_t)a.h >> (5 + GSL);
    const NibK nk = nib_consts();
#pragma unroll
    for (int u = 0; u < UG; ++u) {
        const int row = row0 + u * a.rpi_g;
        const uint32_t rc = (uint32_t)min(row, a.I - 1);
        float pg = 0.f, pu = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = m.c0 + 64 * j;
            const uint32_t cc = (uint32_t)min(c, a.Cg - 1);
            const uint32_t sel = sb_sel(rc * groups + (cc >> GSL));
            const float tg = chunk_term<LO>(t.gw[u][j], t.gs[u][j], t.gb[u][j], sel, xc[j], nk);
            const float tu = chunk_term<LO>(t.uw[u][j], t.us[u][j], t.ub[u][j], sel, xc[j], nk);
            const bool ok = m.ok && c < a.Cg;
            pg += ok ? tg : 0.f;
            pu += ok ? tu : 0.f;
        }
        pg = seg_sum(pg * inv, a.seg_g);
        pu = seg_sum(pu * inv, a.seg_g);
        if (m.writer && row < a.I)
            st_f32(a.act + (size_t)k * a.I + row,
                   act_tagged((pg / (1.0f + expf(-pg))) * pu, tag));  // Shaders.metal:148
    }
}

// Counted unit of gate/up tile T (slot-major tiles of rows_tile act rows,
// a power of two <= 1024): its slot (Cp < 64), or (slot, 2048-row block of
// act) = the down unit that reads those rows (Cp >= 64).
__device__ __forceinline__ int count_unit(const FusedArgs& a, int T) {
    const int k = T / a.tiles_per_slot;
    if (a.Cp < 64) return k;
    return k * a.nb + (((T - k * a.tiles_per_slot) * a.rows_tile) >> 11);
}
// Tiles of counted unit c (what its parts add up to in one launch).
__device__ __forceinline__ uint32_t count_tiles(const FusedArgs& a, int c) {
    if (a.Cp < 64) return (uint32_t)a.tiles_per_slot;
    const int tpb = 2048 / a.rows_tile;
    const int b = c % a.nb;
    return (uint32_t)min(tpb, a.tiles_per_slot - b * tpb);
}

// gate/up workgroup g: tiles T = g, g + n_gu, ... of the K * tiles_per_slot
// (slot-major, so slot 0 completes first and its down work can start while
// later slots stream), each tile = rows_tile rows of one slot; the next
// tile's loads are in flight while a tile is computed.  When the workgroup
// moves on to another counted unit (and at its end) it adds the number of
// tiles it finished of the previous one to its part of every copy of that
// unit's counter (a consumer polls one copy): one add per unit, not per tile,
// since adds to one counter serialise in the memory system and, being counted
// with the loads, stall the next tile's wait.  With several tiles per
// workgroup each tile is its own unit (down units are 2048 act rows, tiles
// are 512 tiles apart); there the count has kCntParts parts, so each counter
// takes a quarter of the adds and a consumer adds four.  Counts do not wait
// for the act stores to be acknowledged (that wait costs µs under the expert
// stream): the consumer checks the tag bits of what it reads and reads again
// until they are current.
template <int CPL, int UG, int GSL>
__device__ void gu_role(const FusedArgs& a, const Layout& L, int g, int wave, int lane,
                        const RouteLDS& r, const GUChunk<CPL> (&xc)[CPL], float inv,
                        uint32_t tag) {
    const GUGeo m = gu_geo(lane, a.Cg, a.seg_g);
    const int tps = a.tiles_per_slot;
    const int total = a.K * tps;
    const int wave_row = wave * a.rpi_g * UG + m.q;
    auto expert_of = [&](int T) {
        const int e = r.idx[T / tps];
        return (r.ok && e >= 0) ? e : -1;
    };
    auto row_of = [&](int T) { return (T % tps) * a.rows_tile + wave_row; };
    int cnt_c = count_unit(a, g);  // counted unit of the current tiles
    uint32_t cnt_n = 0;            // its tiles finished by this workgroup
    auto flush = [&]() {
        __syncthreads();
        if (threadIdx.x < (unsigned)(kNRep / a.cnt_parts))
            add_u32(a.gu_cnt + (((size_t)threadIdx.x * a.cnt_parts + g % a.cnt_parts) * a.n_cnt +
                                cnt_c) * kCntStride,
                    cnt_n);
    };
    // this workgroup's tiles: i = 0 .. n_mine-1 -> T = g + i * n_gu.  Two
    // tiles are in flight from the start; every prefetch is issued (past the
    // last tile it reads a dummy line), so the compiler's in-order load
    // counting stays exact and a tile's compute waits only for its own loads.
    const int n_mine = (total - 1 - g) / a.n_gu + 1;  // g < n_gu <= total
    auto load = [&](int i, GUTile<CPL, UG>& t) {
        const bool real = i < n_mine;
        const int T = g + (real ? i : 0) * a.n_gu;
        gu_load<CPL, UG, GSL>(a, L, expert_of(T), row_of(T), real && expert_of(T) >= 0, m, t);
    };
    auto step = [&](int i, const GUTile<CPL, UG>& t) {
        const int T = g + i * a.n_gu;
        const int k = T / tps;
        const int c = count_unit(a, T);
        if (c != cnt_c) {
            flush();
            cnt_c = c;
            cnt_n = 0;
        }
        if (expert_of(T) >= 0) {
            // bf16 inputs are exact in f16: the lo half of a split chunk is 0
            if (std::is_same<GUChunk<CPL>, XChunk2>::value && !a.x_bf16)
                gu_compute<CPL, UG, GSL, true>(a, k, row_of(T), m, t, xc, inv, tag);
            else
                gu_compute<CPL, UG, GSL, false>(a, k, row_of(T), m, t, xc, inv, tag);
        } else if (m.writer) {
            // no expert for this slot (a bad index or a failed hand-off, both
            // flagged): its act rows still get this launch's tag, so every
            // act entry is rewritten in every launch
#pragma unroll
            for (int u = 0; u < UG; ++u) {
                const int row = row_of(T) + u * a.rpi_g;
                if (row < a.I) st_f32(a.act + (size_t)k * a.I + row, act_tagged(0.f, tag));
            }
        }
        ++cnt_n;
    };
    GUTile<CPL, UG> A, B;
    load(0, A);
    load(1, B);
    for (int i = 0; i < n_mine; i += 2) {
        step(i, A);
        if (i + 1 >= n_mine) break;
        load(i + 2, A);
        step(i + 1, B);
        load(i + 3, B);
    }
    flush();
}

// ---- down + combine ----------------------------------------------------------------

struct DNTile {
    uint4 w[kRT];
    uint32_t s[kRT], b[kRT];
};

// Lane geometry of one 64-lane unit of the down projection: the unit covers
// spu whole slots of Cp (< 64) padded chunks, or 64-chunk block `blk` of one
// slot (Cp >= 64).
struct DNUnit {
    int k;        // slot
    int blk;      // 64-chunk block within the slot
    int c;        // chunk
    bool ok;      // real (slot, chunk)
    bool writer;  // last lane of its segment
};
__device__ __forceinline__ DNUnit dn_unit(const FusedArgs& a, int u, int lane) {
    DNUnit d;
    if (a.Cp < 64) {
        d.k = u * a.spu + (lane >> a.cp_log2);
        d.blk = 0;
        d.c = lane & (a.Cp - 1);
    } else {
        d.k = u / a.nb;
        d.blk = u - d.k * a.nb;
        d.c = d.blk * 64 + lane;
    }
    d.ok = d.k < a.K && d.c < a.Cd;
    d.writer = (lane & (a.seg_d - 1)) == a.seg_d - 1;
    return d;
}

// A load that is not `real` (a prefetch past the wave's last item) reads the
// first 16 bytes of the layer in every lane instead.
template <int GSL>
__device__ __forceinline__ void dn_load(const FusedArgs& a, const Layout& L, const DNUnit& d,
                                        int e, int row0, bool real, DNTile& t) {
    const uint8_t* blk = a.layer_base + (real ? (uint64_t)(e < 0 ? 0 : e) * a.expert_bytes : 0);
    const uint8_t* w_b = blk + (real ? L.down_w : 0);
    const uint8_t* s_b = blk + (real ? L.down_s : 0);
    const uint8_t* b_b = blk + (real ? L.down_b : 0);
    const uint32_t groups = (uint32_t)a.I >> (5 + GSL);
    const uint32_t row_bytes = (uint32_t)a.I / 2;
    const uint32_t cc = (uint32_t)min(d.c, a.Cd - 1);
#pragma unroll
    for (int r = 0; r < kRT; ++r) {
        const uint32_t rc = (uint32_t)min(row0 + r, a.h - 1);
        const uint32_t sbw = real ? sb_word(rc * groups + (cc >> GSL)) : 0u;
        const uint64_t wo = real ? (uint64_t)rc * row_bytes + cc * 16u : 0u;
        t.w[r] = ld_stream(w_b + wo);
        t.s[r] = *reinterpret_cast<const uint32_t*>(s_b + sbw);
        t.b[r] = *reinterpret_cast<const uint32_t*>(b_b + sbw);
    }
}

// Waits until every gate/up tile of counted units [c0, c0 + n) has been
// counted (n * cnt_parts <= 64), polling copy wg % (kNRep / cnt_parts): lane
// j reads part j % cnt_parts of unit c0 + j / cnt_parts, the parts are added
// across their lanes.
__device__ bool wait_counts(const FusedArgs& a, int c0, int n, int lane, uint32_t tag) {
    const int P = a.cnt_parts;
    const bool mine = lane < n * P;
    const int c = c0 + (mine ? lane / P : 0);
    const uint32_t want = tag * count_tiles(a, c);
    const uint32_t* p = a.gu_cnt +
        (((size_t)(blockIdx.x % (kNRep / P)) * P + (lane & (P - 1))) * a.n_cnt + c) * kCntStride;
    for (int it = 0;; ++it) {
        uint32_t v = ld_u32(p);
        for (int m = 1; m < P; m <<= 1) v += __shfl_xor(v, m);
        const bool done = !mine || v == want;
        if (__all(done)) return true;
        if (it >= a.spin_limit) return false;
        __builtin_amdgcn_s_sleep(2);
    }
}

// Items of a down workgroup: (unit u, sub-tile st of kRT rows), unit-major;
// wave w takes a contiguous block of them, so consecutive items of a wave
// mostly share a unit (and its converted act chunk).
struct ItemPos {
    int u, st;
    __device__ ItemPos(int g, int nsub) : u(g / nsub), st(g - (g / nsub) * nsub) {}
};

template <int GSL>
__device__ void dn_role(const FusedArgs& a, const Layout& L, int dblk, int wave, int lane,
                        RouteLDS& r, float* s_part, uint32_t tag) {
    const bool ok_run = r.ok != 0;
    const int Rd = a.Rd;
    const int row_base = dblk * Rd;
    const int nsub = Rd / kRT;
    const int total = a.units * nsub;
    const int per = (total + kWaves - 1) / kWaves;
    const int g0 = wave * per;
    const int n_items = max(0, min(total, g0 + per) - g0);
    const uint32_t groups = (uint32_t)a.I >> (5 + GSL);
    auto expert_at = [&](const DNUnit& d) {
        const int e = d.ok ? r.idx[d.k] : -1;
        return (ok_run && e >= 0) ? e : -1;
    };
    // two items in flight: the first two are loaded as soon as the routing is
    // known.  (Unlike the gate/up role, prefetches past the wave's last item
    // are skipped: waves here end the kernel, and even an L2 hit at the end
    // shows in its duration.)
    auto load = [&](int i, DNTile& t) {
        const bool real = i < n_items;
        const ItemPos p(real ? g0 + i : 0, nsub);
        const DNUnit d = dn_unit(a, p.u, lane);
        dn_load<GSL>(a, L, d, expert_at(d), row_base + p.st * kRT, real, t);
    };
    DNTile A, B;
    if (n_items > 0) load(0, A);
    if (n_items > 1) load(1, B);
    // keep the weight loads above the waits below (the compiler may otherwise
    // sink them to their first use)
    asm volatile("" ::: "memory");
    if (wave == 0) routing_weights(a, lane, r);  // read by the combine after a barrier
    float res = 0.f;
    if ((int)threadIdx.x < Rd && row_base + (int)threadIdx.x < a.h && a.residual)
        res = a.residual[row_base + threadIdx.x];
    const NibK nk = nib_consts();
    int cur = -1;
    DNUnit d{};
    XChunk2 xc[1];
    float inv = 1.f;
    bool live = false;  // this lane's unit is ready and routed
    auto process = [&](const ItemPos& p, const DNTile& t) {
        if (p.u != cur) {
            cur = p.u;
            d = dn_unit(a, p.u, lane);
            int c0, n;
            if (a.Cp < 64) {  // the unit's slots
                c0 = p.u * a.spu;
                n = min(a.spu, a.K - c0);
            } else {          // (slot, block) = the unit itself
                c0 = p.u;
                n = 1;
            }
            bool ready = ok_run;
            if (ready && !wait_counts(a, c0, n, lane, tag)) {
                flag_error(a.err, 4u);
                ready = false;
            }
            live = ready && expert_at(d) >= 0;
            float v[1][32];
            const float* src = a.act + (size_t)(d.k < a.K ? d.k : 0) * a.I;
            const int cc = min(d.c, a.Cd - 1);
            for (int it = 0;; ++it) {
                load_chunk_coherent(src, cc, v[0]);
                uint32_t bad = 0;
#pragma unroll
                for (int i = 0; i < 32; ++i) bad |= (__float_as_uint(v[0][i]) ^ tag) & kActTagMask;
                if (__all(!live || bad == 0)) break;
                if (it >= a.spin_limit) {
                    flag_error(a.err, 4u);
                    live = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            // the value without its tag bits (the same in every launch), or 0
            const uint32_t keep = live ? ~kActTagMask : 0u;
#pragma unroll
            for (int i = 0; i < 32; ++i) v[0][i] = __uint_as_float(__float_as_uint(v[0][i]) & keep);
            inv = lane_scale_prep<1>(v, xc);
        }
        const uint32_t cc = (uint32_t)min(d.c, a.Cd - 1);
        float* part = s_part + (d.k * a.nb + d.blk) * Rd + p.st * kRT;
#pragma unroll
        for (int rr = 0; rr < kRT; ++rr) {
            const uint32_t rc = (uint32_t)min(row_base + p.st * kRT + rr, a.h - 1);
            float q = chunk_term<true>(t.w[rr], t.s[rr], t.b[rr], sb_sel(rc * groups + (cc >> GSL)),
                                       xc[0], nk) * inv;
            q = live ? q : 0.f;
            q = seg_sum(q, a.seg_d);
            if (d.writer && d.k < a.K) part[rr] = q;
        }
    };
    for (int i = 0; i < n_items; i += 2) {
        process(ItemPos(g0 + i, nsub), A);
        if (i + 2 < n_items) load(i + 2, A);
        if (i + 1 < n_items) process(ItemPos(g0 + i + 1, nsub), B);
        if (i + 3 < n_items) load(i + 3, B);
    }
    __syncthreads();
    // combine in slot order, 64-chunk blocks summed in order (Shaders.metal:371-374)
    for (int rr = threadIdx.x; rr < Rd; rr += kThreads) {
        const int row = row_base + rr;
        if (row >= a.h) continue;
        float acc = (rr == (int)threadIdx.x) ? res : (a.residual ? a.residual[row] : 0.f);
        for (int k = 0; k < a.K; ++k) {
            float y = 0.f;
            for (int b = 0; b < a.nb; ++b) y += s_part[(k * a.nb + b) * Rd + rr];
            acc = fmaf(slot_weight(a, r.w, k), y, acc);
        }
        a.out[row] = acc;
    }
}

// The f32 gate/up input of one workgroup (h <= CPL * 2048, CPL <= 2): x is
// read from memory once per workgroup, normalised if asked (x * rms * w, rms
// from the partial sums of squares), and staged in LDS; each wave then takes
// its lanes' 32-element chunks from there.  (Every wave reading x itself put
// 4x the bytes through L2 at the start of the launch.)  Chunks are padded to
// 36 floats against LDS bank conflicts.
template <int CPL>
__device__ __forceinline__ void stage_x(const FusedArgs& a, int wave, int lane, const GUGeo& m,
                                        float (&v)[CPL][32]) {
    constexpr int kG = CPL * 2048 / (4 * kThreads);  // groups of 4 elements per thread
    __shared__ __attribute__((aligned(16))) float s_x[CPL * 64 * 36];
    __shared__ float s_rms;
    float4 xv[kG];
    uint2 nw[kG];
#pragma unroll
    for (int q = 0; q < kG; ++q) {
        const int e = 4 * ((int)threadIdx.x + kThreads * q);
        const int ec = e < a.h ? e : 0;
        xv[q] = *reinterpret_cast<const float4*>(static_cast<const float*>(a.x) + ec);
        if (a.x_norm_w) nw[q] = *reinterpret_cast<const uint2*>(a.x_norm_w + ec);
    }
    if (a.x_norm_w && wave == 0) {
        const float r = input_rms(a, lane);
        if (lane == 0) s_rms = r;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kG; ++q) {
        const int e = 4 * ((int)threadIdx.x + kThreads * q);
        if (e >= a.h) continue;
        float4 t = xv[q];
        if (a.x_norm_w) {  // the norm of Shaders.metal:121-134
            const float rms = s_rms;
            t.x = t.x * rms * __uint_as_float(nw[q].x << 16);
            t.y = t.y * rms * __uint_as_float(nw[q].x & 0xffff0000u);
            t.z = t.z * rms * __uint_as_float(nw[q].y << 16);
            t.w = t.w * rms * __uint_as_float(nw[q].y & 0xffff0000u);
        }
        *reinterpret_cast<float4*>(&s_x[(e >> 5) * 36 + (e & 31)]) = t;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = m.c0 + 64 * j;
        const bool ok = m.ok && c < a.Cg;
        const float* src = &s_x[(ok ? c : 0) * 36];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 t = *reinterpret_cast<const float4*>(src + 4 * i);
            v[j][4 * i + 0] = ok ? t.x : 0.f;
            v[j][4 * i + 1] = ok ? t.y : 0.f;
            v[j][4 * i + 2] = ok ? t.z : 0.f;
            v[j][4 * i + 3] = ok ? t.w : 0.f;
        }
    }
}

// ---- the kernel --------------------------------------------------------------------

template <int CPL, int UG, int GSL>
__global__ __launch_bounds__(kThreads, (CPL <= 2 ? 2 : 1)) void moe_decode_kernel(FusedArgs a) {
    __shared__ RouteLDS r;
    __shared__ uint32_t s_tag;
    __shared__ double s_lp[4];
    extern __shared__ float s_part[];  // down role: [K][nb][Rd]
    const int wg = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const bool is_gu = wg < a.n_gu;

    // this launch's number, as counted by this workgroup (all agree); its
    // load overlaps the router row loads of the producers
    const uint32_t tag_reg = threadIdx.x == 0 ? ld_u32(a.seen + wg) + 1u : 0u;
    if (!a.given_idx && wg < a.E) {
        float rms = 1.f;
        bool need_rms = a.x_norm_w != nullptr;
        for (int e = wg; e < a.E; e += gridDim.x)
            produce_logit<CPL>(a, e, wave, lane, &s_tag, tag_reg, s_lp, rms, need_rms);
    } else {
        if (threadIdx.x == 0) s_tag = tag_reg;
        __syncthreads();
    }
    const uint32_t tag = s_tag;

    // the input vector does not depend on the routing: prepare it meanwhile
    GUChunk<CPL> xc[CPL];
    float inv = 1.f;
    if (is_gu) {
        const GUGeo m = gu_geo(lane, a.Cg, a.seg_g);
        float v[CPL][32];
        bool staged = false;
        if constexpr (CPL <= 2) {
            if (!a.x_bf16) {  // (a bf16 x is half the bytes: read per wave)
                stage_x<CPL>(a, wave, lane, m, v);
                staged = true;
            }
        }
        if (!staged) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = m.c0 + 64 * j;
            load_chunk(a.x, a.x_bf16, min(c, a.Cg - 1), m.ok && c < a.Cg, v[j]);
        }
        if (a.x_norm_w) {
            // the norm weights are loaded before the partial sums are waited for
            uint4 nw[CPL][4];
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = min(m.c0 + 64 * j, a.Cg - 1);
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    nw[j][q] = *reinterpret_cast<const uint4*>(a.x_norm_w + 32 * c + 8 * q);
            }
            const float rms = input_rms(a, lane);
#pragma unroll
            for (int j = 0; j < CPL; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        v[j][8 * q + i] = v[j][8 * q + i] * rms * bf16x8_at(nw[j][q], i);
        }
        }
        inv = lane_scale_prep<CPL>(v, xc);
    }

    routing(a, wg, wave, lane, tag, r);
    const bool ok_run = r.ok != 0;
    if (wg == 0 && ok_run && (a.user_idx || a.user_w)) {
        if (wave == 0) routing_weights(a, lane, r);
        __syncthreads();
        if ((int)threadIdx.x < a.K) {
            if (a.user_idx) a.user_idx[threadIdx.x] = r.idx[threadIdx.x];
            if (a.user_w) a.user_w[threadIdx.x] = slot_weight(a, r.w, threadIdx.x);
        }
    }
    const Layout L(a.h, a.I, a.gs);
    if (is_gu) {
        gu_role<CPL, UG, GSL>(a, L, wg, wave, lane, r, xc, inv, tag);
    } else {
        dn_role<GSL>(a, L, wg - a.n_gu, wave, lane, r, s_part, tag);
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

inline int pow2_ceil(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}
// gate/up rows per wave: about eight 128-bit weight loads per lane
constexpr int gu_rows(int cpl) { return cpl == 1 ? 4 : cpl == 2 ? 2 : 1; }

template <int CPL, int GSL>
int launch_shape(const FusedArgs& a, hipStream_t st) {
    const size_t lds = sizeof(float) * (size_t)a.K * a.nb * a.Rd;
    if (lds > 64 * 1024) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL((moe_decode_kernel<CPL, gu_rows(CPL), GSL>),
                       dim3((unsigned)(a.n_gu + a.n_dn)), dim3(kThreads), lds, st, a);
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
    // gate/up
    a.Cg = a.h / 32;
    if (a.Cg >= 64) {
        a.seg_g = 64;
        a.rpi_g = 1;
    } else {
        a.seg_g = pow2_ceil(a.Cg);
        a.rpi_g = 64 / a.seg_g;
    }
    const int cpl = (a.Cg + 63) / 64;
    a.rows_tile = kWaves * a.rpi_g * gu_rows(cpl);
    a.tiles_per_slot = (a.I + a.rows_tile - 1) / a.rows_tile;
    a.n_gu = min(a.K * a.tiles_per_slot, kGuMax);
    // down
    a.Cd = a.I / 32;
    if (a.Cd < 64) {
        a.Cp = pow2_ceil(a.Cd);
        a.cp_log2 = __builtin_ctz(a.Cp);
        a.seg_d = a.Cp;
        a.nb = 1;
        a.spu = 64 / a.Cp;
        a.units = (a.K + a.spu - 1) / a.spu;
    } else {
        a.Cp = (a.Cd + 63) / 64 * 64;
        a.seg_d = 64;
        a.nb = a.Cp / 64;
        a.spu = 1;
        a.units = a.K * a.nb;
    }
    const int nsub = max(1, (a.h + kDnTarget * kRT - 1) / (kDnTarget * kRT));
    a.Rd = kRT * nsub;
    a.n_dn = (a.h + a.Rd - 1) / a.Rd;
    a.n_cnt = a.Cp < 64 ? a.K : a.K * a.nb;
    a.cnt_parts = a.n_gu < a.K * a.tiles_per_slot ? kCntParts : 1;
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
