// decode_cu.hip — batch-1 MoE block for gfx950 with one workgroup per CU:
// router logits and top-K, expert dispatch, fused 4-bit group-affine dequant +
// gate/up matvec + SwiGLU, fused dequant + down matvec, weighted combine +
// residual, in ONE launch of 256 workgroups of eight waves (all resident at
// once on the 256 CUs).
//
// Replaces, per token and layer, the reference's CPU router + selectTopK
// (InferenceEngine.swift:490-519), pread dispatch (:271-280) and the 4K+1
// Metal dispatches (matvec4bit x3 + swiGLU per slot, then moeCombine:
// InferenceEngine.swift:401-478, Shaders.metal:39-92,138-149,360-376), for
// hidden width 2048 with K * I = 8192 or 16384 (OLMoE: K = 8, I = 1024).
//
// Every workgroup g does the same four things:
//   1. router: every XCD computes all E logits (exact bf16*x products
//      summed in f64, rounded once; workgroup j of an XCD takes experts
//      j + 32 i) and hands them to its own workgroups through its L2; every
//      workgroup polls the logits and ranks them (descending, ties to the
//      lower index);
//   2. gate/up: 8 * UG consecutive act rows of one slot (UG rows per wave,
//      one 32-column chunk of each row per lane), SwiGLU into LDS.  These
//      rows are whole 32-row chunks of act, i.e. whole 32-column chunks of
//      the slot's down matrix;
//   3. down, split over the intermediate dimension: the workgroup multiplies
//      ITS act chunks (never sent to another workgroup) by those columns of
//      the down matrix for all 2048 output rows (four per lane), and writes
//      the 2048 partial sums;
//   4. reduce: output rows 8g .. 8g+7, once every workgroup's partials for
//      them are readable: for each slot the partials of its workgroups are
//      summed in a fixed tree order, then the slots are combined in slot
//      order with the residual.
//
// The down weights and all scales/biases are read from a repacked copy of
// each expert block made at upload (make_decode_copy): down columns
// chunk-major (a workgroup's columns are one contiguous 32 KiB run), the
// gate/up scales and biases of four rows interleaved (one 32-byte load per
// lane instead of sixteen 4-byte ones), the down scales/biases group-major.
// The gate/up weights are read from the canonical arena.
//
// Hand-off.  Published logits are (launch number, value) pairs: in the
// XCD's local slots (plain stores, read with non-temporal loads through the
// XCD's L2) and in one global replica per XCD (sc1), read only when the local
// slots stay incomplete (workgroups not placed on the XCDs in turn).  Partial sums carry the parity of the launch number in their
// lowest mantissa bit: the reader checks every value it loads, reads the
// stale ones again until all are current, and clears the bit (the value used
// is the same in every launch: a relative change below 2^-23), so no counter
// or store acknowledgement is waited for.  Nothing is reset between launches:
// each workgroup counts its launches in cu_seen[g], so all workgroups agree
// on the launch number.  Every wait is bounded (a timeout raises the
// device error flag and the workgroup still stores all of its partials, so
// the kernel always ends).  Every workgroup waits for every other one, so
// all 256 must be resident together: the host uses this kernel only on a
// device with at least 256 CUs.
#include <hip/hip_runtime.h>

#include "decode_common.hpp"
#include "device.hpp"
#include "internal.hpp"

namespace m1moe {
namespace {

// Phase stamps of the per-CU kernels, compiled only when M1MOE_DECODE_TRACE
// is defined (never in libm1moe_hip.so): s_memrealtime (100 MHz) per
// workgroup into LDS, written at the end of the launch to the buffer that
// m1moe_trace_decode() set ([workgroup][64 slots]; none set: nothing is
// written).  The slot numbers are the arguments of the DTR_* calls below.
#ifdef M1MOE_DECODE_TRACE
__device__ unsigned long long* g_decode_trace;
__shared__ unsigned long long s_dtr[64];
#define DTR_BEGIN()                                      \
    do {                                                 \
        if (threadIdx.x < 64) s_dtr[threadIdx.x] = 0ull; \
        __syncthreads();                                 \
    } while (0)
#define DTR_WAVE(slot)                                                                   \
    do {                                                                                 \
        if ((threadIdx.x & 63) == 0) s_dtr[(slot)] = __builtin_amdgcn_s_memrealtime();  \
    } while (0)
#define DTR_WG(slot)                                                          \
    do {                                                                      \
        if (threadIdx.x == 0) s_dtr[(slot)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#define DTR_END()                                                                          \
    do {                                                                                   \
        __syncthreads();                                                                   \
        if (g_decode_trace && threadIdx.x < 64)                                            \
            g_decode_trace[(size_t)blockIdx.x * 64 + threadIdx.x] = s_dtr[threadIdx.x];    \
    } while (0)
#else
#define DTR_BEGIN() do {} while (0)
#define DTR_WAVE(slot) do {} while (0)
#define DTR_WG(slot) do {} while (0)
#define DTR_END() do {} while (0)
#endif

constexpr int kW = 8;               // waves per workgroup
constexpr int kT = 64 * kW;         // threads per workgroup
constexpr int kNG = kCuWorkgroups;  // workgroups
constexpr int kH = 2048;            // hidden width: 64 chunks of 32 columns, one per lane
constexpr int kRows = kH / kNG;     // output rows per workgroup
constexpr int kMaxE = 256;
constexpr int kMaxK = 8;
constexpr int kChunkWords = 34;     // prepared act chunk: 16 hi pairs, 16 lo pairs, sum, 2^-e
constexpr int kMaxLoc = 8;          // router logits per workgroup (E <= 256, 32 per XCD)
constexpr int kLocalPolls = 64;     // XCD-local logit polls before the global replicas are read

// The XCD (and L2) the calling workgroup runs on.
__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 7u;
}

// XCD-local hand-off words: a plain store lands in the XCD's L2 (the CU's L1
// writes through), and a non-temporal load reads that L2 without the CU's
// L1, so workgroups of one XCD see each other's stores in ~0.25 us (an sc1
// store and load pair, which goes through memory and works between XCDs,
// takes ~0.6 us).  Other XCDs cannot rely on seeing such a store.
__device__ __forceinline__ void st_l2_u64(unsigned long long* p, unsigned long long v) {
    asm volatile("global_store_dwordx2 %0, %1, off" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ unsigned long long ld_l2_u64(const unsigned long long* p) {
    unsigned long long v;
    asm volatile("global_load_dwordx2 %0, %1, off nt\n\ts_waitcnt vmcnt(0)"
                 : "=v"(v)
                 : "v"(p)
                 : "memory");
    return v;
}

static_assert(kRows == 8 && kT * 4 == kH, "one x quad and four down rows per thread");

struct CuLDS {
    alignas(16) float x[64 * 36];   // staged input, chunk c at 36c (padded against bank conflicts)
    alignas(16) float v[kMaxE];     // logits (NaN and beyond E: -inf)
    alignas(16) uint32_t xp[2][36]; // this workgroup's prepared act chunks
    alignas(16) uint32_t xq[64][36];// gate/up input chunk of each lane: 16 hi pairs, 16 lo
                                    // pairs, sum, 2^-e (prepared once per workgroup)
    double lp[kMaxLoc][kW];         // wave partials of this workgroup's logits
    float act[64];                  // this workgroup's act rows
    float y[kMaxK][kRows];          // per slot: reduced down outputs of rows 8g .. 8g+7
    int idx[kMaxK];                 // expert of each slot (-1: none)
    float w[kMaxK];                 // combine weight of each slot
    float rms;
    uint32_t tag;
    int ok;
};

// ---- routing ---------------------------------------------------------------------

// Expert i's rank = the number of experts ahead of it (a larger logit, or an
// equal one at a lower index), counted by P = 2^LP lanes over M = 2^LEP / P
// experts each (the 512 threads cover the 2^LEP experts exactly); the
// segment's last lane writes s.idx[rank] = i for the K first ranks.
template <int LEP, class S>
__device__ __forceinline__ void rank_cu(int t, int E, int K, S& s) {
    constexpr int LP = LEP == 6 ? 3 : (LEP == 7 ? 2 : 1);
    constexpr int P = 1 << LP, M = 1 << (LEP - LP);
    static_assert((1 << LEP) * P == kT, "one thread per (expert, part)");
    const int i = t >> LP, q = t & (P - 1), j0 = q * M;
    const float my = s.v[i];
    float cnt = 0.f;
#pragma unroll
    for (int m = 0; m < M; m += 4) {
        const float4 v4 = *reinterpret_cast<const float4*>(&s.v[j0 + m]);
        const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u)
            cnt += ((vv[u] > my) || (vv[u] == my && j0 + m + u < i)) ? 1.f : 0.f;
    }
    cnt = seg_sum_c<P>(cnt);  // total in the segment's last lane
    if (i < E && q == P - 1 && (int)cnt < K) s.idx[(int)cnt] = i;
}

// Router logits (InferenceEngine.swift:490-500) computed on every XCD: the
// workgroup with local index j = g / 8 (one per workgroup of an XCD when the
// workgroups are placed on the XCDs in turn) takes experts j + 32 i < E, each
// the exact products of its bf16 router row and x summed in f64 (NX
// consecutive columns per thread, a fixed wave tree, the waves in order) and
// rounded once, plus the optional bias.  Stage 1 (before the barrier that
// follows): the wave partials into lp.  Stage 2: published as (launch tag,
// value) to the XCD's local slots (plain stores) and to the XCD's global
// replica (sc1 stores).
template <int NX, class RW>
__device__ __forceinline__ void logits_partial(int nloc, int wave, int lane, const RW (&rw)[kMaxLoc],
                                               const float (&xv)[NX], double (*lp)[kW]) {
#pragma unroll
    for (int i = 0; i < kMaxLoc; ++i) {
        if (i < nloc) {
            const uint32_t* r = reinterpret_cast<const uint32_t*>(&rw[i]);
            double acc = 0.0;
#pragma unroll
            for (int k = 0; k < NX / 2; ++k) {
                acc += (double)__uint_as_float(r[k] << 16) * (double)xv[2 * k];
                acc += (double)__uint_as_float(r[k] & 0xffff0000u) * (double)xv[2 * k + 1];
            }
            acc = wave_sum_f64_last(acc);
            if (lane == 63) lp[i][wave] = acc;
        }
    }
}

__device__ __forceinline__ void logits_publish(const FusedArgs& a, int t, int jl, int nloc,
                                               uint32_t tag, const double (*lp)[kW]) {
    if (t < nloc) {
        const int e = jl + 32 * t;
        double sum = lp[t][0];
#pragma unroll
        for (int w = 1; w < kW; ++w) sum += lp[t][w];
        float l = (float)sum;
        if (a.bias) l = l + a.bias[e];
        const unsigned long long u = ((unsigned long long)tag << 32) | __float_as_uint(l);
        const uint32_t x = xcc_id();
        st_l2_u64(a.xl + (size_t)x * kRepStride + e, u);
        st_u64(a.slots + (size_t)x * kRepStride + e, u);
    }
}

// Obtains the routing: the given one, or the published logits (wave 0 polls
// replica g % kLogitRep) ranked by all threads: expert i's rank is the
// number of experts ahead of it (larger logit, or equal logit and lower
// index), counted by P lanes over ep / P experts each (ep = E rounded up to
// a power of two, padding at -inf).  Ends with a barrier; s.idx and s.ok are
// valid after it (and s.w for a given routing).
template <class S>
__device__ void route_cu(const FusedArgs& a, int g, int t, int wave, int lane, uint32_t tag,
                         S& s) {
    const int E = a.E, K = a.K;
    if (a.given_idx) {
        if (t < K) {
            int e = a.given_idx[t];
            if (e < 0 || e >= E) {
                flag_error(a.err, 1u);
                e = -1;
            }
            s.idx[t] = e;
            s.w[t] = a.given_w[t];
        }
        if (t == 0) s.ok = 1;
        __syncthreads();
        return;
    }
    if (wave == 0) {
        // this XCD's own slots first (its workgroups compute every logit, see
        // publish_logits); after kLocalPolls rounds, for workgroups placed on
        // the XCDs other than in turn, the global replicas, one per XCD,
        // rotating over them (every logit is in at least one)
        const unsigned long long* loc = a.xl + (size_t)xcc_id() * kRepStride;
        const int nj = (E + 63) >> 6;  // logits per lane (wave-uniform)
        float v[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        bool have[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) have[j] = (lane + 64 * j >= E);
        bool ok = true;
        for (int it = 0;; ++it) {
            const bool local = it < kLocalPolls;
            unsigned long long u[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = lane + 64 * j;
                u[j] = 0ull;
                if (j < nj && !have[j])
                    u[j] = local ? ld_l2_u64(loc + e)
                                 : ld_u64(a.slots + (size_t)((it + e) & 7) * kRepStride + e);
            }
            bool all = true;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (j < nj && !have[j]) {
                    if ((uint32_t)(u[j] >> 32) == tag) {
                        have[j] = true;
                        const float f = __uint_as_float((uint32_t)u[j]);
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
            __builtin_amdgcn_s_sleep(1);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) s.v[lane + 64 * j] = v[j];
        if (lane == 0) s.ok = ok ? 1 : 0;
        DTR_WAVE(4);
    }
    __syncthreads();
    DTR_WG(5);
    // ranks over ep = 2^LEP experts (E rounded up, at least 64; the padding
    // is -inf at indices above every expert)
    const int lep = E <= 64 ? 6 : (E <= 128 ? 7 : 8);
    if (lep == 6)
        rank_cu<6>(t, E, K, s);
    else if (lep == 7)
        rank_cu<7>(t, E, K, s);
    else
        rank_cu<8>(t, E, K, s);
    DTR_WG(7);
    __syncthreads();
}

// Softmax probabilities of the selected experts (InferenceEngine.swift:
// 501-506), renormalised over the selection in slot order when
// norm_topk_prob is set (:514-517), into s.w.  One wave; a given routing
// keeps the supplied weights.
template <class S>
__device__ void weights_cu(const FusedArgs& a, int lane, S& s) {
    if (a.given_idx) return;
    const int E = a.E, K = a.K;
    float v[4], mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[j] = (lane + 64 * j < E) ? s.v[lane + 64 * j] : -INFINITY;
        mx = fmaxf(mx, v[j]);
    }
    mx = wave_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) sum += (lane + 64 * j < E) ? expf(v[j] - mx) : 0.f;
    const float inv = 1.0f / wave_sum(sum);
    float p = 0.f;
    if (lane < K) p = expf(s.v[s.idx[lane]] - mx) * inv;
    if (a.norm) {
        float ssum = 0.f;
        for (int r = 0; r < K; ++r) ssum = ssum + readlane_f32(p, r);
        p = p / ssum;
    }
    if (lane < K) s.w[lane] = p;
}

// ---- the repacked copy of an expert block ---------------------------------------------

// One thread per 16 bytes of the repacked block, all experts of a layer
// (H = hidden width: 2048, or 4096 for moe_decode_cuw_kernel).
template <int H>
__global__ __launch_bounds__(256) void decode_copy_kernel(const uint8_t* src, uint64_t src_bytes,
                                                          uint8_t* dst, uint64_t dst_bytes,
                                                          int E, int I, int gs) {
    constexpr int RPT = H / 512;  // down rows per thread: t + 512 r, r < RPT
    const Layout L(H, I, gs);
    const DecLayout D(H, I, gs);
    const uint64_t n16 = D.bytes / 16;
    const uint64_t gi = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (gi >= n16 * (uint64_t)E) return;
    const uint64_t e = gi / n16, o = (gi - e * n16) * 16;
    const uint8_t* b = src + e * src_bytes;
    uint8_t* d = dst + e * dst_bytes;
    const int groups_h = H / gs, groups_i = I / gs;
    auto bf = [&](uint64_t off, uint64_t elem) {
        return (uint32_t)reinterpret_cast<const uint16_t*>(b + off)[elem];
    };
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (o < D.dw) {
        // two rows of one (quad, group): 16 bytes = rows 2p, 2p + 1
        const uint64_t i8 = o / 8;                 // (quad, group, row) index
        const uint64_t r4 = i8 % 4, qg = i8 / 4;
        const uint64_t grp = qg % groups_h, quad = qg / groups_h;
        uint32_t w[4];
        for (int k = 0; k < 2; ++k) {
            const uint64_t row = quad * 4 + r4 + k;
            const uint64_t el = row * groups_h + grp;
            w[2 * k] = bf(L.gate_s, el) | (bf(L.gate_b, el) << 16);
            w[2 * k + 1] = bf(L.up_s, el) | (bf(L.up_b, el) << 16);
        }
        v = make_uint4(w[0], w[1], w[2], w[3]);
    } else if (o < D.dsb) {
        const uint64_t k16 = (o - D.dw) / 16;      // (chunk, row)
        const uint64_t row = k16 % H, c = k16 / H;
        v = *reinterpret_cast<const uint4*>(b + L.down_w + row * (uint64_t)(I / 2) + c * 16);
    } else if (o < D.dsb + (uint64_t)groups_i * H * 4) {
        // (group, t, quarter): rows t + 512 r, r = 4 quarter .. 4 quarter + 3
        const uint64_t k16 = (o - D.dsb) / 16;
        const uint64_t qt = k16 % (RPT / 4), t = (k16 / (RPT / 4)) % 512;
        const uint64_t grp = k16 / (RPT / 4) / 512;
        uint32_t w[4];
        for (int k = 0; k < 4; ++k) {
            const uint64_t el = (t + (uint64_t)512 * (4 * qt + k)) * groups_i + grp;
            w[k] = bf(L.down_s, el) | (bf(L.down_b, el) << 16);
        }
        v = make_uint4(w[0], w[1], w[2], w[3]);
    }
    *reinterpret_cast<uint4*>(d + o) = v;
}

// ---- cross-lane reductions --------------------------------------------------------

// Eight values per lane summed over the wave: a butterfly of exchanges
// (quad_perm xor 1, then xor 2) leaves two values per lane, indexed by the
// lane's low bits, then those are summed over the quads of each 16-lane row
// (row_ror 4 and 8) and over the four rows.  Lane l ends with the totals of
// v[2 r] and v[2 r + 1], r = ((l >> 1) & 1) + 2 (l & 1).  Fixed order.
__device__ __forceinline__ void reduce8_wave(const float (&v)[8], int lane, float& r0, float& r1) {
    const bool b0 = lane & 1, b1 = (lane >> 1) & 1;
    float k[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float send = b0 ? v[j] : v[j + 4];
        const float keep = b0 ? v[j + 4] : v[j];
        k[j] = keep + dpp_f32<kDppXor1>(0.f, send);
    }
    float m[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const float send = b1 ? k[j] : k[j + 2];
        const float keep = b1 ? k[j + 2] : k[j];
        m[j] = keep + dpp_f32<kDppXor2>(0.f, send);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        m[j] += dpp_f32<kDppRor4>(0.f, m[j]);
        m[j] += dpp_f32<kDppRor8>(0.f, m[j]);
        m[j] += __shfl_xor(m[j], 16);
        m[j] += __shfl_xor(m[j], 32);
    }
    r0 = m[0];
    r1 = m[1];
}

// Four values per lane summed over aligned segments of SEG lanes (32 or
// 64), the same butterfly: lane l ends with the segment total of v[r],
// r = ((l >> 1) & 1) + 2 (l & 1).  Fixed order.
__device__ __forceinline__ float reduce4_seg(const float (&v)[4], int lane, int seg) {
    const bool b0 = lane & 1, b1 = (lane >> 1) & 1;
    float k[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const float send = b0 ? v[j] : v[j + 2];
        const float keep = b0 ? v[j + 2] : v[j];
        k[j] = keep + dpp_f32<kDppXor1>(0.f, send);
    }
    float m = (b1 ? k[1] : k[0]) + dpp_f32<kDppXor2>(0.f, b1 ? k[0] : k[1]);
    m += dpp_f32<kDppRor4>(0.f, m);
    m += dpp_f32<kDppRor8>(0.f, m);
    m += __shfl_xor(m, 16);
    if (seg == 64) m += __shfl_xor(m, 32);
    return m;
}


// ---- gate/up ---------------------------------------------------------------------

template <int UG>
struct GUTileCU {
    uint4 gw[UG], uw[UG];
    uint4 sb[UG / 2];  // row u: word 2u = gate s | b << 16, 2u + 1 = up s | b << 16
};

__device__ __forceinline__ uint32_t word_of(const uint4* v, int i) {
    const uint4 q = v[i >> 2];
    const int k = i & 3;
    return k == 0 ? q.x : k == 1 ? q.y : k == 2 ? q.z : q.w;
}

// Rows row0 .. row0+UG-1 of expert e's gate and up projections, chunk `lane`
// of each, with their scales/biases.  e < 0: every lane reads the first 16
// bytes of the layer instead.
template <int UG, int GSL>
__device__ __forceinline__ void gu_load_cu(const FusedArgs& a, const Layout& L, int e, int row0,
                                           int lane, GUTileCU<UG>& t) {
    const bool real = e >= 0;
    const uint64_t eu = real ? (uint64_t)__builtin_amdgcn_readfirstlane(e) : 0;
    const uint8_t* blk = a.layer_base + eu * a.expert_bytes;
    const uint8_t* gw_b = blk + (real ? L.gate_w : 0);
    const uint8_t* uw_b = blk + (real ? L.up_w : 0);
    const uint8_t* sb_b = a.dec_base + eu * a.dec_bytes;
    constexpr uint32_t groups = kH >> (5 + GSL);
    // the scales and biases first: loads return in issue order, so the
    // compute of row 0 can start once its own words are in, while the
    // later rows are still arriving
#pragma unroll
    for (int q = 0; q < UG / 4; ++q) {
        const uint32_t so = real ? (((uint32_t)(row0 / 4 + q) * groups + ((uint32_t)lane >> GSL)) * 32u) : 0u;
        t.sb[2 * q] = ld_stream(sb_b + so);
        t.sb[2 * q + 1] = ld_stream(sb_b + so + 16);
    }
#pragma unroll
    for (int u = 0; u < UG; ++u) {
        const uint32_t wo = real ? (uint32_t)(row0 + u) * (kH / 2) + (uint32_t)lane * 16u : 0u;
        t.gw[u] = ld_stream(gw_b + wo);
        t.uw[u] = ld_stream(uw_b + wo);
    }
}

// act = silu(gate) * up for the UG rows of this wave (Shaders.metal:138-149),
// into s.act: four rows at a time, reduced together, their SwiGLU in four
// lanes at once.
template <int UG, bool LO>
__device__ __forceinline__ void gu_compute_cu(int wave, int lane, const GUTileCU<UG>& t,
                                              const XChunk2& xc, float inv, CuLDS& s) {
    const uint32_t mlo = __builtin_amdgcn_readfirstlane(0x000F000Fu);
    const uint32_t mhi = __builtin_amdgcn_readfirstlane(0x00F000F0u);
    const float sc = inv * 16777216.f;  // undoes the lane's 2^e and the subnormal 2^-24
#pragma unroll
    for (int u0 = 0; u0 < UG; u0 += 4) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t gsb = word_of(t.sb, 2 * (u0 + u)), usb = word_of(t.sb, 2 * (u0 + u) + 1);
            const float dg = nib_dot32_sub<LO>(t.gw[u0 + u], xc, mlo, mhi);
            const float du = nib_dot32_sub<LO>(t.uw[u0 + u], xc, mlo, mhi);
            v[2 * u] = fmaf(bf16_pick(gsb, kSelLo) * sc, dg, bf16_pick(gsb, kSelHi) * xc.xs * inv);
            v[2 * u + 1] =
                fmaf(bf16_pick(usb, kSelLo) * sc, du, bf16_pick(usb, kSelHi) * xc.xs * inv);
            // row by row as the rows arrive (the scheduler would otherwise
            // gather every row's wait ahead of the first row's arithmetic)
            __builtin_amdgcn_sched_barrier(0);
        }
        float pg, pu;
        reduce8_wave(v, lane, pg, pu);
        if (lane < 4) s.act[wave * UG + u0 + ((lane >> 1) & 1) + 2 * (lane & 1)] = silu_fast(pg) * pu;
    }
}

// Max over aligned 32-lane halves, returned to every lane of the half.
__device__ __forceinline__ float half_max(float v) {
    v = fmaxf(v, dpp_f32<kDppXor1>(v, v));
    v = fmaxf(v, dpp_f32<kDppXor2>(v, v));
    v = fmaxf(v, dpp_f32<kDppRor4>(v, v));
    v = fmaxf(v, dpp_f32<kDppRor8>(v, v));
    v = fmaxf(v, dpp_f32<kDppBcast15, 0xA>(v, v));  // rows 1 and 3: the half's max
    const float m0 = readlane_f32(v, 31), m1 = readlane_f32(v, 63);
    return (threadIdx.x & 32) ? m1 : m0;
}

// Prepares the workgroup's act chunks for the down dot products (lanes
// 32h .. 32h+31 take chunk h): chunk element i scaled by 2^e (largest into
// [2^13, 2^14)), divided by 16 at odd i, split into f16 hi + lo and paired
// (i, i + 4) for i % 8 < 4: pair p = 4 (i / 8) + i % 8 at words 2p (hi) and
// 2p + 1 (lo); word 32 = the sum of the chunk's values as the dot products
// see them (hi + lo, times 16 at odd i), word 33 = 2^-e.  One wave, into
// s.xp.
template <int UG>
__device__ __forceinline__ void prep_chunks(int lane, CuLDS& s) {
    constexpr int kChunks = UG / 4;
    const int h = lane >> 5, i = lane & 31;
    const bool on = h < kChunks;
    const float x = on ? s.act[32 * h + i] : 0.f;
    const float mx = half_max(fabsf(x));
    float scale, inv;
    pow2_scale(mx, scale, inv);
    _Float16 hi, lo;
    split_f16(x * scale * ((i & 1) ? 0.0625f : 1.f), hi, lo);
    const uint32_t hb = __builtin_bit_cast(uint16_t, hi), lb = __builtin_bit_cast(uint16_t, lo);
    // element i + 4 of the same group of eight (row_shl:4 stays in the 16-lane row for i % 8 < 4)
    const uint32_t hb4 = dpp_u32<0x104>(0u, hb), lb4 = dpp_u32<0x104>(0u, lb);
    const float vs = ((float)hi + (float)lo) * ((i & 1) ? 16.f : 1.f);
    const float xs = seg_sum_c<32>(vs);  // total in lanes 31 and 63
    if (!on) return;
    if ((i & 7) < 4) {
        const int p = 4 * (i >> 3) + (i & 7);
        s.xp[h][2 * p] = hb | (hb4 << 16);
        s.xp[h][2 * p + 1] = lb | (lb4 << 16);
    }
    if (i == 31) {
        s.xp[h][32] = __float_as_uint(xs);
        s.xp[h][33] = __float_as_uint(inv);
    }
}

// ---- down (split over the intermediate dimension) -------------------------------------

template <int NC>
struct DNTileCU {
    uint4 w[NC][4];   // chunk c, row t + 512 r
    uint4 sb[NC];     // chunk c's group: (s | b << 16) of rows t + 512 r
};

// Columns of chunks c0 .. c0+NC-1 of expert e's down matrix, rows t + 512 r
// (each load is one contiguous run across the lanes).
template <int NC, int GSL>
__device__ __forceinline__ void dn_load_cu(const FusedArgs& a, int e, int c0, int t,
                                           DNTileCU<NC>& d) {
    const bool real = e >= 0;
    const uint64_t eu = real ? (uint64_t)__builtin_amdgcn_readfirstlane(e) : 0;
    const DecLayout D(kH, a.I, a.gs);
    const uint8_t* blk = a.dec_base + eu * a.dec_bytes;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t wo = real ? (uint32_t)(((c0 + c) * kH + t + (kH / 4) * r) * 16) : 0u;
            d.w[c][r] = ld_stream(blk + (real ? D.dw : 0) + wo);
        }
        const uint32_t so = real ? (uint32_t)((((c0 + c) >> GSL) * (kH / 4) + t) * 16) : 0u;
        d.sb[c] = ld_stream(blk + (real ? D.dsb : 0) + so);
    }
}

// The down tile with its nibbles expanded to exact f16 subnormals (n * 2^-24,
// or 16 n * 2^-24 at bits 4..7 of a byte, matching the /16 of the odd chunk
// elements; see nib_dot32_sub): word q of a row gives pairs 4q .. 4q+3.
// Done while the act chunks are awaited.
template <int NC>
struct DNExpCU {
    uint32_t n[NC][4][16];
    float s[NC][4], b[NC][4];
};

template <int NC>
__device__ __forceinline__ void dn_expand_cu(const DNTileCU<NC>& d, DNExpCU<NC>& x) {
    const uint32_t mlo = __builtin_amdgcn_readfirstlane(0x000F000Fu);
    const uint32_t mhi = __builtin_amdgcn_readfirstlane(0x00F000F0u);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const uint32_t sbw[4] = {d.sb[c].x, d.sb[c].y, d.sb[c].z, d.sb[c].w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t ws[4] = {d.w[c][r].x, d.w[c][r].y, d.w[c][r].z, d.w[c][r].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t v = ws[q], v8 = v >> 8;
                x.n[c][r][4 * q + 0] = v & mlo;
                x.n[c][r][4 * q + 1] = v & mhi;
                x.n[c][r][4 * q + 2] = v8 & mlo;
                x.n[c][r][4 * q + 3] = v8 & mhi;
            }
            x.s[c][r] = bf16_pick(sbw[r], kSelLo);
            x.b[c][r] = bf16_pick(sbw[r], kSelHi);
        }
    }
}

// Rows t + 512 r of the workgroup's down columns: per chunk, s * sum(n x)
// + b * sum(x) in the chunk's scaled units, times 2^-e, summed over the
// chunks; the hi and lo pairs go through the same expanded nibbles.
template <int NC>
__device__ __forceinline__ void dn_compute_cu(const DNExpCU<NC>& x, const CuLDS& s,
                                              float (&out)[4]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) out[r] = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        uint32_t p[kChunkWords];
#pragma unroll
        for (int k = 0; k < kChunkWords; k += 2) {
            const uint2 q = *reinterpret_cast<const uint2*>(&s.xp[c][k]);
            p[k] = q.x;
            p[k + 1] = q.y;
        }
        const float xs = __uint_as_float(p[32]), sc = __uint_as_float(p[33]) * 16777216.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
            for (int k = 0; k < 16; k += 2) {  // pair k: hi at word 2k, lo at 2k + 1
                const half2_t n0 = __builtin_bit_cast(half2_t, x.n[c][r][k]);
                const half2_t n1 = __builtin_bit_cast(half2_t, x.n[c][r][k + 1]);
                a0 = __builtin_amdgcn_fdot2(n0, __builtin_bit_cast(half2_t, p[2 * k]), a0, false);
                a1 = __builtin_amdgcn_fdot2(n1, __builtin_bit_cast(half2_t, p[2 * k + 2]), a1, false);
                a2 = __builtin_amdgcn_fdot2(n0, __builtin_bit_cast(half2_t, p[2 * k + 1]), a2, false);
                a3 = __builtin_amdgcn_fdot2(n1, __builtin_bit_cast(half2_t, p[2 * k + 3]), a3, false);
            }
            const float dsum = (a0 + a1) + (a2 + a3);
            out[r] += fmaf(x.s[c][r] * sc, dsum, x.b[c][r] * xs * __uint_as_float(p[33]));
        }
    }
}

// An f32 carrying the launch parity in its lowest mantissa bit.
__device__ __forceinline__ uint32_t tagged(float v, uint32_t parity) {
    return (__float_as_uint(v) & ~1u) | parity;
}

// 16 bytes of partial sums written by other workgroups in this launch
// (agent-coherent load).
__device__ __forceinline__ uint4 ld_coherent16(const uint32_t* p) {
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    u4 q;
    asm volatile("global_load_dwordx4 %0, %1, off sc1\n\ts_waitcnt vmcnt(0)"
                 : "=v"(q)
                 : "v"(p)
                 : "memory");
    return make_uint4(q[0], q[1], q[2], q[3]);
}

// ---- the kernel ------------------------------------------------------------------

// UG = K * I / 2048: gate/up rows per wave; the workgroup's 8 * UG act rows
// are UG / 4 chunks of 32.
template <int UG, int GSL, bool LO>
__global__ __launch_bounds__(kT, 1) void moe_decode_cu_kernel(FusedArgs a) {
    constexpr int NC = UG / 4;
    __shared__ CuLDS s;
    DTR_BEGIN();
    DTR_WG(0);
    const int g = blockIdx.x, t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int E = a.E, K = a.K, I = a.I;
    // router logits jl + 32 i < E, computed on every XCD (logits_partial)
    const int jl = g >> 3;
    const int nloc = (a.given_idx || jl >= E) ? 0 : (E - jl + 31) / 32;

    // ---- input, launch number, router row --------------------------------------
    if (t == 0) s.tag = ld_u32(a.cu_seen + g) + 1u;
    float res = 0.f;
    if (t < kRows && a.residual) res = a.residual[g * kRows + t];
    const bool normed = !a.x_bf16 && a.x_norm_w;
    float xv[4];
    uint2 nw = make_uint2(0u, 0u);
    if (a.x_bf16) {
        const uint2 q = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.x) + 4 * t);
        xv[0] = __uint_as_float(q.x << 16);
        xv[1] = __uint_as_float(q.x & 0xffff0000u);
        xv[2] = __uint_as_float(q.y << 16);
        xv[3] = __uint_as_float(q.y & 0xffff0000u);
    } else {
        const float4 q = *reinterpret_cast<const float4*>(static_cast<const float*>(a.x) + 4 * t);
        xv[0] = q.x;
        xv[1] = q.y;
        xv[2] = q.z;
        xv[3] = q.w;
        if (normed) nw = *reinterpret_cast<const uint2*>(a.x_norm_w + 4 * t);
    }
    uint2 rw[kMaxLoc];
#pragma unroll
    for (int i = 0; i < kMaxLoc; ++i)
        rw[i] = i < nloc ? *reinterpret_cast<const uint2*>(a.router + (size_t)(jl + 32 * i) * kH + 4 * t)
                         : make_uint2(0u, 0u);
    if (normed && wave == 0) {
        const float r = input_rms(a, lane);
        if (lane == 0) s.rms = r;
    }
    __syncthreads();
    if (normed) {  // the norm of Shaders.metal:121-134
        const float rms = s.rms;
        xv[0] = xv[0] * rms * __uint_as_float(nw.x << 16);
        xv[1] = xv[1] * rms * __uint_as_float(nw.x & 0xffff0000u);
        xv[2] = xv[2] * rms * __uint_as_float(nw.y << 16);
        xv[3] = xv[3] * rms * __uint_as_float(nw.y & 0xffff0000u);
    }
    *reinterpret_cast<float4*>(&s.x[(t >> 3) * 36 + (t & 7) * 4]) = float4{xv[0], xv[1], xv[2], xv[3]};
    logits_partial<4>(nloc, wave, lane, rw, xv, s.lp);
    __syncthreads();
    const uint32_t tag = s.tag, parity = tag & 1u;
    logits_publish(a, t, jl, nloc, tag, s.lp);
    DTR_WG(1);

    // the gate/up input, chunk c of x for lane c of every wave: prepared once
    // per workgroup by wave 1 while wave 0 awaits the logits
    if (wave == 1) {
        float v[1][32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 q = *reinterpret_cast<const float4*>(&s.x[lane * 36 + 4 * i]);
            v[0][4 * i + 0] = q.x;
            v[0][4 * i + 1] = q.y;
            v[0][4 * i + 2] = q.z;
            v[0][4 * i + 3] = q.w;
        }
        XChunk2 c1[1];
        const float vinv = lane_scale_prep<1>(v, c1);
        uint32_t* d = s.xq[lane];
#pragma unroll
        for (int p = 0; p < 16; ++p) {
            d[p] = __builtin_bit_cast(uint32_t, c1[0].X[p]);
            d[16 + p] = __builtin_bit_cast(uint32_t, c1[0].L[p]);
        }
        d[32] = __float_as_uint(c1[0].xs);
        d[33] = __float_as_uint(vinv);
        DTR_WAVE(2);
    }

    route_cu(a, g, t, wave, lane, tag, s);
    const bool ok_run = s.ok != 0;
    DTR_WG(3);
    XChunk2 xc;
    float inv;
    {
        const uint32_t* d = s.xq[lane];
#pragma unroll
        for (int p = 0; p < 16; p += 4) {
            const uint4 q = *reinterpret_cast<const uint4*>(d + p);
            xc.X[p] = __builtin_bit_cast(half2_t, q.x);
            xc.X[p + 1] = __builtin_bit_cast(half2_t, q.y);
            xc.X[p + 2] = __builtin_bit_cast(half2_t, q.z);
            xc.X[p + 3] = __builtin_bit_cast(half2_t, q.w);
        }
        if (!a.x_bf16) {  // (a bf16 input is exact in f16: its lo half is 0 and unused)
#pragma unroll
            for (int p = 0; p < 16; p += 4) {
                const uint4 q = *reinterpret_cast<const uint4*>(d + 16 + p);
                xc.L[p] = __builtin_bit_cast(half2_t, q.x);
                xc.L[p + 1] = __builtin_bit_cast(half2_t, q.y);
                xc.L[p + 2] = __builtin_bit_cast(half2_t, q.z);
                xc.L[p + 3] = __builtin_bit_cast(half2_t, q.w);
            }
        }
        const uint2 m = *reinterpret_cast<const uint2*>(d + 32);
        xc.xs = __uint_as_float(m.x);
        xc.off = 0.f;
        inv = __uint_as_float(m.y);
    }

    // ---- all of this workgroup's expert bytes: gate/up rows, then down columns -----
    const Layout L(kH, I, a.gs);
    const int wps = kNG / K;                 // workgroups per slot
    const int kg = g / wps;                  // the slot of this workgroup's act rows
    const int eg = ok_run ? s.idx[kg] : -1;
    const int wg_row0 = (g - kg * wps) * (kW * UG);
    GUTileCU<UG> gt;
    gu_load_cu<UG, GSL>(a, L, eg, wg_row0 + wave * UG, lane, gt);
    // every wave's gate/up requests leave the CU before any down request (a
    // barrier without a memory fence: nothing is waited for)
    __builtin_amdgcn_s_barrier();
    DNTileCU<NC> dt;
    dn_load_cu<NC, GSL>(a, eg, wg_row0 / 32, t, dt);

    // ---- gate/up + SwiGLU, then the act chunks ----------------------------------------
    // (LO: an f32 input's lo halves take part; a bf16 input is exact in f16)
    if (eg >= 0) gu_compute_cu<UG, LO>(wave, lane, gt, xc, inv, s);
    DTR_WAVE(8 + wave);
    // the act chunks are prepared (wave 0) while the other waves expand their
    // down nibbles (the down bytes, requested last, are the last to arrive)
    __syncthreads();
    if (wave == 0 && eg >= 0) prep_chunks<UG>(lane, s);
    if (wave == 0) DTR_WAVE(16);
    DNExpCU<NC> dx;
    if (eg >= 0) dn_expand_cu<NC>(dt, dx);  // (waits for this wave's down loads)
    DTR_WAVE(40 + wave);
    __syncthreads();

    // ---- down partials of all 2048 rows from this workgroup's columns ------------------
    float pr[4] = {0.f, 0.f, 0.f, 0.f};
    if (eg >= 0) dn_compute_cu<NC>(dx, s, pr);
    DTR_WAVE(24 + wave);
    // row t + 512 r goes to output block (t + 512 r) / 8, position t % 8, at this
    // workgroup's place; eight lanes fill one 32-byte run
#pragma unroll
    for (int r = 0; r < 4; ++r)
        st_u32(a.cu_part + ((size_t)((t + (kH / 4) * r) >> 3) * kNG + g) * kRows + (t & 7),
               tagged(pr[r], parity));
    DTR_WG(17);
    // the next layer's router rows that this workgroup's successor (the same
    // index, so the same XCD) reads first, requested now so that they wait in
    // the XCD's L2 (consumed by an empty asm at the end: the loads complete
    // while the partials are awaited)
    uint32_t pf = 0u;
    if (a.next_router) {
#pragma unroll
        for (int i = 0; i < kMaxLoc; ++i)
            if (i < nloc) {
                const uint2 v =
                    *reinterpret_cast<const uint2*>(a.next_router + (size_t)(jl + 32 * i) * kH + 4 * t);
                pf ^= v.x ^ v.y;
            }
    }

    // the combine weights, off the path to the partial stores (read after the
    // barrier that follows the reduction)
    if (wave == kW - 1) {
        weights_cu(a, lane, s);
        if (g == 0 && ok_run && lane < K) {
            if (a.user_idx) a.user_idx[lane] = s.idx[lane];
            if (a.user_w) a.user_w[lane] = s.w[lane];
        }
    }

    // ---- reduce: thread t takes source workgroup t % 256, rows 4 (t / 256) .. +3, ------
    // reading until every value carries this launch's parity (a source still
    // computing is read again after a pause; only the stale lanes reload)
    const int src = t & (kNG - 1), half = t >> 8;
    uint4 q = make_uint4(0u, 0u, 0u, 0u);
    {
        const uint32_t* p = a.cu_part + ((size_t)g * kNG + src) * kRows + half * 4;
        bool cur = false;
        for (int it = 0;; ++it) {
            if (!cur) {
                q = ld_coherent16(p);
                cur = ((q.x & q.y & q.z & q.w & 1u) == parity) &&
                      (((q.x | q.y | q.z | q.w) & 1u) == parity);
            }
            if (__all(cur)) break;
            if (it >= a.spin_limit) {
                flag_error(a.err, 4u);
                break;
            }
            __builtin_amdgcn_s_sleep(4);
        }
    }
    DTR_WAVE(32 + wave);
    // the values without their tag bit (the same in every launch); the
    // sources of one slot are wps consecutive lanes (32 or 64)
    const float yv[4] = {__uint_as_float(q.x & ~1u), __uint_as_float(q.y & ~1u),
                         __uint_as_float(q.z & ~1u), __uint_as_float(q.w & ~1u)};
    const float ysum = reduce4_seg(yv, lane, wps);
    if ((src & (wps - 1)) < 4)
        s.y[src / wps][half * 4 + ((lane >> 1) & 1) + 2 * (lane & 1)] = ysum;
    __syncthreads();

    // ---- combine in slot order with the residual (Shaders.metal:360-376) --------------
    if (t < kRows) {
        float acc = res;
        if (ok_run) {
            int iv[kMaxK];
            float wv[kMaxK], yv[kMaxK];
#pragma unroll
            for (int k = 0; k < kMaxK; ++k) {
                iv[k] = s.idx[k];
                wv[k] = s.w[k];
                yv[k] = s.y[k][t];
            }
#pragma unroll
            for (int k = 0; k < kMaxK; ++k)
                if (k < K && iv[k] >= 0) acc = fmaf(wv[k], yv[k], acc);
        }
        a.out[g * kRows + t] = acc;
    }
    DTR_WG(56);
    if (t == 0) st_u32(a.cu_seen + g, tag);
    asm volatile("" ::"v"(pf));
    DTR_END();
}

template <int UG, int GSL>
void launch_lo(const FusedArgs& a, hipStream_t st) {
    if (a.x_bf16)
        hipLaunchKernelGGL((moe_decode_cu_kernel<UG, GSL, false>), dim3(kNG), dim3(kT), 0, st, a);
    else
        hipLaunchKernelGGL((moe_decode_cu_kernel<UG, GSL, true>), dim3(kNG), dim3(kT), 0, st, a);
}

template <int UG>
int launch_ug(const FusedArgs& a, hipStream_t st) {
    switch (a.gs) {
        case 32: launch_lo<UG, 0>(a, st); break;
        case 64: launch_lo<UG, 1>(a, st); break;
        case 128: launch_lo<UG, 2>(a, st); break;
        default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

// ---- hidden 4096 (Mixtral): moe_decode_cuw_kernel ------------------------------------
//
// The same one-launch, one-workgroup-per-CU scheme for hidden width 4096 and
// top-K <= 2: working workgroup g < K * I / 128 owns 128 consecutive act rows
// of one slot (4 chunks of 32; wave w: rows 16 w .. 16 w + 15), streams their
// gate/up rows in batches of 4 rows x one 32-column chunk per lane (one
// batch in flight while the previous one is multiplied), then its down
// columns chunk by chunk (rows t + 512 r, r
// < 8, per thread), and stores 4096 partial sums.  Every workgroup (working
// or not) then reduces output rows 16 g .. 16 g + 15 over the working
// workgroups of each slot, in a fixed order, and combines the slots.

constexpr int kHW = 4096;
constexpr int kRowsW = kHW / kNG;   // output rows per workgroup in the reduce
constexpr int kRPT = kHW / kT;      // down rows per thread
constexpr int kWRows = 128;         // act rows per working workgroup
constexpr int kWChunks = kWRows / 32;
constexpr int kMaxKW = 2;
constexpr int kWInFlight = 1;   // gate/up batches in flight per wave (two: 43.9 against
                                // 43.3 us per cfg2 layer-token, more queueing in the memory system)
constexpr int kWEarlyDown = 2;  // down chunks requested during the last batches

struct CuwLDS {
    alignas(16) float x[128 * 36];      // staged input, chunk c at 36 c
    alignas(16) float v[kMaxE];         // logits
    alignas(16) uint32_t xq[128][36];   // prepared gate/up input chunks (hi, lo, sum, 2^-e)
    alignas(16) uint32_t xp[kWChunks][36];  // this workgroup's prepared act chunks
    double lp[kMaxLoc][kW];
    float act[kWRows];
    float y[kMaxKW][kRowsW];
    int idx[kMaxK];
    float w[kMaxK];
    float rms;
    uint32_t tag;
    int ok;
};

// One batch: 4 act rows x one 32-column chunk per lane, gate and up, and the
// (4-row, group) scale/bias quad of that chunk.
struct GUBatchW {
    uint4 gw[4], uw[4];
    uint4 sb[2];
};

template <int GSL>
__device__ __forceinline__ void guw_load(const FusedArgs& a, const Layout& L, int e, int row0,
                                         int c, GUBatchW& b) {
    const bool real = e >= 0;
    const uint64_t eu = real ? (uint64_t)__builtin_amdgcn_readfirstlane(e) : 0;
    const uint8_t* blk = a.layer_base + eu * a.expert_bytes;
    const uint8_t* sb_b = a.dec_base + eu * a.dec_bytes;
    constexpr uint32_t groups = kHW >> (5 + GSL);
    const uint32_t so = ((uint32_t)(row0 / 4) * groups + ((uint32_t)c >> GSL)) * 32u;
    b.sb[0] = ld_stream(sb_b + so);
    b.sb[1] = ld_stream(sb_b + so + 16);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const uint32_t wo = (uint32_t)(row0 + u) * (kHW / 2) + (uint32_t)c * 16u;
        b.gw[u] = ld_stream(blk + L.gate_w + wo);
        b.uw[u] = ld_stream(blk + L.up_w + wo);
    }
}

// The down columns of one chunk for rows t + 512 r: nibble words and the
// (scale | bias) words of the chunk's group.
struct DNChunkW {
    uint4 w[kRPT];
    uint4 sb[kRPT / 4];
};

template <int GSL>
__device__ __forceinline__ void dnw_load(const FusedArgs& a, int e, int cg, int t, DNChunkW& d) {
    const bool real = e >= 0;
    const uint64_t eu = real ? (uint64_t)__builtin_amdgcn_readfirstlane(e) : 0;
    const DecLayout D(kHW, a.I, a.gs);
    const uint8_t* blk = a.dec_base + eu * a.dec_bytes;
#pragma unroll
    for (int r = 0; r < kRPT; ++r)
        d.w[r] = ld_stream(blk + D.dw + ((uint64_t)cg * kHW + t + 512 * r) * 16);
    const uint64_t so = D.dsb + (((uint64_t)(cg >> GSL) * 512 + t) * (kRPT / 4)) * 16;
#pragma unroll
    for (int q = 0; q < kRPT / 4; ++q) d.sb[q] = ld_stream(blk + so + 16 * q);
}

// acc[r] += the chunk's contribution to row t + 512 r (act chunk prepared in xp).
__device__ __forceinline__ void dnw_compute(const DNChunkW& d, const uint32_t* xp, float (&acc)[kRPT]) {
    const uint32_t mlo = __builtin_amdgcn_readfirstlane(0x000F000Fu);
    const uint32_t mhi = __builtin_amdgcn_readfirstlane(0x00F000F0u);
    uint32_t p[kChunkWords];
#pragma unroll
    for (int k = 0; k < kChunkWords; k += 2) {
        const uint2 q = *reinterpret_cast<const uint2*>(&xp[k]);
        p[k] = q.x;
        p[k + 1] = q.y;
    }
    const float xs = __uint_as_float(p[32]), inv = __uint_as_float(p[33]);
    const float sc = inv * 16777216.f;
    const uint32_t sbw[kRPT] = {d.sb[0].x, d.sb[0].y, d.sb[0].z, d.sb[0].w,
                                d.sb[1].x, d.sb[1].y, d.sb[1].z, d.sb[1].w};
#pragma unroll
    for (int r = 0; r < kRPT; ++r) {
        const uint32_t ws[4] = {d.w[r].x, d.w[r].y, d.w[r].z, d.w[r].w};
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {  // word q: pairs 4q .. 4q + 3 (hi at 2k, lo at 2k + 1)
            const uint32_t v = ws[q], v8 = v >> 8;
            const uint32_t n[4] = {v & mlo, v & mhi, v8 & mlo, v8 & mhi};
#pragma unroll
            for (int j = 0; j < 4; j += 2) {
                const int k = 4 * q + j;
                const half2_t n0 = __builtin_bit_cast(half2_t, n[j]);
                const half2_t n1 = __builtin_bit_cast(half2_t, n[j + 1]);
                a0 = __builtin_amdgcn_fdot2(n0, __builtin_bit_cast(half2_t, p[2 * k]), a0, false);
                a1 = __builtin_amdgcn_fdot2(n1, __builtin_bit_cast(half2_t, p[2 * k + 2]), a1, false);
                a2 = __builtin_amdgcn_fdot2(n0, __builtin_bit_cast(half2_t, p[2 * k + 1]), a2, false);
                a3 = __builtin_amdgcn_fdot2(n1, __builtin_bit_cast(half2_t, p[2 * k + 3]), a3, false);
            }
        }
        const float dsum = (a0 + a1) + (a2 + a3);
        acc[r] += fmaf(bf16_pick(sbw[r], kSelLo) * sc, dsum, bf16_pick(sbw[r], kSelHi) * xs * inv);
    }
}

template <int GSL, bool LO>
__global__ __launch_bounds__(kT, 1) void moe_decode_cuw_kernel(FusedArgs a) {
    __shared__ CuwLDS s;
    DTR_BEGIN();
    DTR_WG(0);
    const int g = blockIdx.x, t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int E = a.E, K = a.K, I = a.I;
    const int wps = I / kWRows;               // working workgroups per slot
    const int nwork = K * wps;
    const int jl = g >> 3;  // router logits jl + 32 i < E (logits_partial)
    const int nloc = (a.given_idx || jl >= E) ? 0 : (E - jl + 31) / 32;

    // ---- input, launch number, router row --------------------------------------------
    if (t == 0) s.tag = ld_u32(a.cu_seen + g) + 1u;
    float res = 0.f;
    if (t < kRowsW && a.residual) res = a.residual[g * kRowsW + t];
    const bool normed = !a.x_bf16 && a.x_norm_w;
    float xv[8];
    uint4 nw = make_uint4(0u, 0u, 0u, 0u);
    if (a.x_bf16) {
        const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.x) + 8 * t);
        const uint32_t qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xv[2 * i] = __uint_as_float(qq[i] << 16);
            xv[2 * i + 1] = __uint_as_float(qq[i] & 0xffff0000u);
        }
    } else {
        const float4 q0 = *reinterpret_cast<const float4*>(static_cast<const float*>(a.x) + 8 * t);
        const float4 q1 = *reinterpret_cast<const float4*>(static_cast<const float*>(a.x) + 8 * t + 4);
        xv[0] = q0.x; xv[1] = q0.y; xv[2] = q0.z; xv[3] = q0.w;
        xv[4] = q1.x; xv[5] = q1.y; xv[6] = q1.z; xv[7] = q1.w;
        if (normed) nw = *reinterpret_cast<const uint4*>(a.x_norm_w + 8 * t);
    }
    uint4 rw[kMaxLoc];
#pragma unroll
    for (int i = 0; i < kMaxLoc; ++i)
        rw[i] = i < nloc ? *reinterpret_cast<const uint4*>(a.router + (size_t)(jl + 32 * i) * kHW + 8 * t)
                         : make_uint4(0u, 0u, 0u, 0u);
    if (normed && wave == 0) {
        const float r = input_rms(a, lane);
        if (lane == 0) s.rms = r;
    }
    __syncthreads();
    if (normed) {  // the norm of Shaders.metal:121-134
        const float rms = s.rms;
        const uint32_t ww[4] = {nw.x, nw.y, nw.z, nw.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xv[2 * i] = xv[2 * i] * rms * __uint_as_float(ww[i] << 16);
            xv[2 * i + 1] = xv[2 * i + 1] * rms * __uint_as_float(ww[i] & 0xffff0000u);
        }
    }
    {
        float* dx = &s.x[(t >> 2) * 36 + (t & 3) * 8];
        *reinterpret_cast<float4*>(dx) = float4{xv[0], xv[1], xv[2], xv[3]};
        *reinterpret_cast<float4*>(dx + 4) = float4{xv[4], xv[5], xv[6], xv[7]};
    }
    logits_partial<8>(nloc, wave, lane, rw, xv, s.lp);
    __syncthreads();
    const uint32_t tag = s.tag, parity = tag & 1u;
    logits_publish(a, t, jl, nloc, tag, s.lp);
    DTR_WG(1);
    // the gate/up input chunks (lane l of every wave uses chunks l and l + 64),
    // prepared once per workgroup by waves 1 and 2 while wave 0 awaits the logits
    if (wave == 1 || wave == 2) {
        const int c = lane + 64 * (wave - 1);
        float v[1][32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 q = *reinterpret_cast<const float4*>(&s.x[c * 36 + 4 * i]);
            v[0][4 * i + 0] = q.x;
            v[0][4 * i + 1] = q.y;
            v[0][4 * i + 2] = q.z;
            v[0][4 * i + 3] = q.w;
        }
        XChunk2 c1[1];
        const float vinv = lane_scale_prep<1>(v, c1);
        uint32_t* d = s.xq[c];
#pragma unroll
        for (int p = 0; p < 16; ++p) {
            d[p] = __builtin_bit_cast(uint32_t, c1[0].X[p]);
            d[16 + p] = __builtin_bit_cast(uint32_t, c1[0].L[p]);
        }
        d[32] = __float_as_uint(c1[0].xs);
        d[33] = __float_as_uint(vinv);
    }

    route_cu(a, g, t, wave, lane, tag, s);
    const bool ok_run = s.ok != 0;
    DTR_WG(3);

    // ---- working workgroups: gate/up of 128 act rows, then their down columns ------
    const bool working = g < nwork;
    const int kg = working ? g / wps : 0;
    const int eg = (working && ok_run) ? s.idx[kg] : -1;
    const int r0 = working ? (g - kg * wps) * kWRows : 0;
    const Layout L(kHW, I, a.gs);
    float pr[kRPT];
#pragma unroll
    for (int r = 0; r < kRPT; ++r) pr[r] = 0.f;
    DNChunkW D0, D1;
    const int cg0 = r0 / 32;
    if (eg >= 0) {
        // batch b: row quad b / 2 of this wave's 16 rows, chunk half b % 2 (lane
        // l: chunk l, then chunk l + 64); kWInFlight batches in flight
        const int wrow = r0 + 16 * wave;
        GUBatchW Bq[kWInFlight];
#pragma unroll
        for (int bi = 0; bi < kWInFlight; ++bi)
            guw_load<GSL>(a, L, eg, wrow + 4 * (bi >> 1), lane + 64 * (bi & 1), Bq[bi]);
        const uint32_t mlo = __builtin_amdgcn_readfirstlane(0x000F000Fu);
        const uint32_t mhi = __builtin_amdgcn_readfirstlane(0x00F000F0u);
        float pg[4], pu[4];
#pragma unroll
        for (int bi = 0; bi < 8; ++bi) {
            const int q = bi >> 1, ch = bi & 1;
            GUBatchW& B = Bq[bi % kWInFlight];
            const uint32_t* d = s.xq[lane + 64 * ch];
            XChunk2 xc;
#pragma unroll
            for (int p = 0; p < 16; p += 4) {
                const uint4 qh = *reinterpret_cast<const uint4*>(d + p);
                xc.X[p] = __builtin_bit_cast(half2_t, qh.x);
                xc.X[p + 1] = __builtin_bit_cast(half2_t, qh.y);
                xc.X[p + 2] = __builtin_bit_cast(half2_t, qh.z);
                xc.X[p + 3] = __builtin_bit_cast(half2_t, qh.w);
                if (LO) {
                    const uint4 ql = *reinterpret_cast<const uint4*>(d + 16 + p);
                    xc.L[p] = __builtin_bit_cast(half2_t, ql.x);
                    xc.L[p + 1] = __builtin_bit_cast(half2_t, ql.y);
                    xc.L[p + 2] = __builtin_bit_cast(half2_t, ql.z);
                    xc.L[p + 3] = __builtin_bit_cast(half2_t, ql.w);
                }
            }
            const uint2 m2 = *reinterpret_cast<const uint2*>(d + 32);
            xc.xs = __uint_as_float(m2.x);
            xc.off = 0.f;
            const float inv = __uint_as_float(m2.y);
            const float sc = inv * 16777216.f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t gsb = word_of(B.sb, 2 * u), usb = word_of(B.sb, 2 * u + 1);
                const float dg = nib_dot32_sub<LO>(B.gw[u], xc, mlo, mhi);
                const float du = nib_dot32_sub<LO>(B.uw[u], xc, mlo, mhi);
                const float tg = fmaf(bf16_pick(gsb, kSelLo) * sc, dg, bf16_pick(gsb, kSelHi) * xc.xs * inv);
                const float tu = fmaf(bf16_pick(usb, kSelLo) * sc, du, bf16_pick(usb, kSelHi) * xc.xs * inv);
                pg[u] = ch ? pg[u] + tg : tg;
                pu[u] = ch ? pu[u] + tu : tu;
                __builtin_amdgcn_sched_barrier(0);
            }
            const int nb = bi + kWInFlight;
            if (nb < 8) guw_load<GSL>(a, L, eg, wrow + 4 * (nb >> 1), lane + 64 * (nb & 1), B);
            if (nb == 7) {  // every gate/up byte requested: the first down chunks next
                if (kWEarlyDown >= 1) dnw_load<GSL>(a, eg, cg0, t, D0);
                if (kWEarlyDown >= 2) dnw_load<GSL>(a, eg, cg0 + 1, t, D1);
            }
            if (ch) {
                const float v8[8] = {pg[0], pu[0], pg[1], pu[1], pg[2], pu[2], pg[3], pu[3]};
                float gg, uu;
                reduce8_wave(v8, lane, gg, uu);
                if (lane < 4)
                    s.act[16 * wave + 4 * q + ((lane >> 1) & 1) + 2 * (lane & 1)] = silu_fast(gg) * uu;
            }
        }
    }
    DTR_WAVE(8 + wave);
    if (eg >= 0) {  // the down chunks not yet requested
        if (kWEarlyDown < 1) dnw_load<GSL>(a, eg, cg0, t, D0);
        if (kWEarlyDown < 2) dnw_load<GSL>(a, eg, cg0 + 1, t, D1);
    }
    __syncthreads();
    if (eg >= 0 && wave < kWChunks / 2) {
        // act chunks 2 w and 2 w + 1 (lanes 0-31, 32-63)
        const int h = lane >> 5, i = lane & 31, c = 2 * wave + h;
        const float x = s.act[32 * c + i];
        const float mx = half_max(fabsf(x));
        float scale, inv;
        pow2_scale(mx, scale, inv);
        _Float16 hi, lo;
        split_f16(x * scale * ((i & 1) ? 0.0625f : 1.f), hi, lo);
        const uint32_t hb = __builtin_bit_cast(uint16_t, hi), lb = __builtin_bit_cast(uint16_t, lo);
        const uint32_t hb4 = dpp_u32<0x104>(0u, hb), lb4 = dpp_u32<0x104>(0u, lb);
        const float vs = ((float)hi + (float)lo) * ((i & 1) ? 16.f : 1.f);
        const float xs = seg_sum_c<32>(vs);
        if ((i & 7) < 4) {
            const int p = 4 * (i >> 3) + (i & 7);
            s.xp[c][2 * p] = hb | (hb4 << 16);
            s.xp[c][2 * p + 1] = lb | (lb4 << 16);
        }
        if (i == 31) {
            s.xp[c][32] = __float_as_uint(xs);
            s.xp[c][33] = __float_as_uint(inv);
        }
    }
    __syncthreads();
    DTR_WG(16);
    if (eg >= 0) {
        dnw_compute(D0, s.xp[0], pr);
        dnw_load<GSL>(a, eg, cg0 + 2, t, D0);
        dnw_compute(D1, s.xp[1], pr);
        dnw_load<GSL>(a, eg, cg0 + 3, t, D1);
        dnw_compute(D0, s.xp[2], pr);
        dnw_compute(D1, s.xp[3], pr);
    }
    DTR_WAVE(24 + wave);
    if (working) {
        // row t + 512 r -> block (t + 512 r) / 16, position t % 16, at this workgroup's place
#pragma unroll
        for (int r = 0; r < kRPT; ++r)
            st_u32(a.cu_part + ((size_t)((t + 512 * r) >> 4) * kNG + g) * kRowsW + (t & 15),
                   tagged(pr[r], parity));
    }
    DTR_WG(17);
    if (wave == kW - 1) {
        weights_cu(a, lane, s);
        if (g == 0 && ok_run && lane < K) {
            if (a.user_idx) a.user_idx[lane] = s.idx[lane];
            if (a.user_w) a.user_w[lane] = s.w[lane];
        }
    }

    // ---- reduce rows 16 g .. 16 g + 15: thread t < nwork reads source t's 16 ---------
    // partials (re-reading the stale ones), then per slot and row 16 lanes each
    // add every 16th source of the slot, and the 16 lanes are summed
    uint4 q4[4];
    if (t < nwork) {
        const uint32_t* p = a.cu_part + ((size_t)g * kNG + t) * kRowsW;
        bool cur[4] = {false, false, false, false};
        for (int it = 0;; ++it) {
            bool all = true;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (!cur[j]) {
                    q4[j] = ld_coherent16(p + 4 * j);
                    const uint4 q = q4[j];
                    cur[j] = ((q.x & q.y & q.z & q.w & 1u) == parity) &&
                             (((q.x | q.y | q.z | q.w) & 1u) == parity);
                }
                all = all && cur[j];
            }
            if (all) break;
            if (it >= a.spin_limit) {
                flag_error(a.err, 4u);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    DTR_WAVE(32 + wave);
    // stage the sources in LDS (x is no longer used): src[t][16]
    float* stage = s.x;
    if (t < nwork) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint4 q = q4[j];
            *reinterpret_cast<float4*>(&stage[t * 16 + 4 * j]) =
                float4{__uint_as_float(q.x & ~1u), __uint_as_float(q.y & ~1u),
                       __uint_as_float(q.z & ~1u), __uint_as_float(q.w & ~1u)};
        }
    }
    __syncthreads();
    {
        const int j = t & 15, row = (t >> 4) & 15, k = t >> 8;
        float sum = 0.f;
        if (k < K)
            for (int src = k * wps + j; src < (k + 1) * wps; src += 16) sum += stage[src * 16 + row];
        sum = seg_sum_c<16>(sum);  // total in lane j = 15
        if (k < K && j == 15) s.y[k][row] = sum;
    }
    __syncthreads();

    // ---- combine in slot order with the residual (Shaders.metal:360-376) -------------
    if (t < kRowsW) {
        float acc = res;
        if (ok_run) {
#pragma unroll
            for (int k = 0; k < kMaxKW; ++k)
                if (k < K && s.idx[k] >= 0) acc = fmaf(s.w[k], s.y[k][t], acc);
        }
        a.out[g * kRowsW + t] = acc;
    }
    DTR_WG(56);
    if (t == 0) st_u32(a.cu_seen + g, tag);
    DTR_END();
}

template <int GSL>
void launch_w(const FusedArgs& a, hipStream_t st) {
    if (a.x_bf16)
        hipLaunchKernelGGL((moe_decode_cuw_kernel<GSL, false>), dim3(kNG), dim3(kT), 0, st, a);
    else
        hipLaunchKernelGGL((moe_decode_cuw_kernel<GSL, true>), dim3(kNG), dim3(kT), 0, st, a);
}

}  // namespace

#ifdef M1MOE_DECODE_TRACE
// Tracing build only: sets (or, with NULL, clears) the device buffer that
// moe_decode_cu_kernel writes its phase stamps to.
extern "C" int32_t m1moe_trace_decode(void* dev_buf) {
    return hipMemcpyToSymbol(HIP_SYMBOL(g_decode_trace), &dev_buf, sizeof(dev_buf)) == hipSuccess
               ? 0
               : M1MOE_ERR_HIP;
}
#endif

bool decode_cu_fits(int h, int E, int K, int I, int gs) {
    if (E > kMaxE || K < 1 || (gs != 32 && gs != 64 && gs != 128)) return false;
    if (h == kH) {  // moe_decode_cu_kernel
        if (K > kMaxK || (kMaxK % K) != 0 || (I != 1024 && I != 2048)) return false;
        const int ug = K * I / 2048;
        return ug == 4 || ug == 8;
    }
    if (h == kHW)  // moe_decode_cuw_kernel
        return K <= kMaxKW && I % kWRows == 0 && K * (I / kWRows) <= kNG;
    return false;
}

namespace {
template <class F>
int occupancy_min(F f0, F f1, int* blocks) {
    int b0 = 0, b1 = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&b0, f0, kT, 0);
    if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&b1, f1, kT, 0);
    *blocks = e == hipSuccess ? min(b0, b1) : 0;
    return (int)e;
}
template <int UG, int GSL>
int occupancy_ug(int* blocks) {
    return occupancy_min(moe_decode_cu_kernel<UG, GSL, false>, moe_decode_cu_kernel<UG, GSL, true>,
                         blocks);
}
template <int UG>
int occupancy_gs(int gs, int* blocks) {
    return gs == 32 ? occupancy_ug<UG, 0>(blocks)
                    : (gs == 64 ? occupancy_ug<UG, 1>(blocks) : occupancy_ug<UG, 2>(blocks));
}
}  // namespace

int decode_cu_blocks_per_cu(int h, int K, int I, int gs, int* blocks) {
    *blocks = 0;
    if (h == kHW) {
        switch (gs) {
            case 32: return occupancy_min(moe_decode_cuw_kernel<0, false>, moe_decode_cuw_kernel<0, true>, blocks);
            case 64: return occupancy_min(moe_decode_cuw_kernel<1, false>, moe_decode_cuw_kernel<1, true>, blocks);
            default: return occupancy_min(moe_decode_cuw_kernel<2, false>, moe_decode_cuw_kernel<2, true>, blocks);
        }
    }
    return K * I == 8192 ? occupancy_gs<4>(gs, blocks) : occupancy_gs<8>(gs, blocks);
}

uint64_t decode_copy_bytes(int h, int I, int gs) { return DecLayout(h, I, gs).bytes; }

int launch_decode_copy(const uint8_t* layer, uint64_t expert_bytes, uint8_t* dst, int E, int h,
                       int I, int gs, void* stream) {
    const DecLayout D(h, I, gs);
    const uint64_t threads = D.bytes / 16 * (uint64_t)E;
    const dim3 grid((unsigned)((threads + 255) / 256));
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (h == kHW)
        hipLaunchKernelGGL(decode_copy_kernel<kHW>, grid, dim3(256), 0, st, layer, expert_bytes,
                           dst, D.bytes, E, I, gs);
    else
        hipLaunchKernelGGL(decode_copy_kernel<kH>, grid, dim3(256), 0, st, layer, expert_bytes,
                           dst, D.bytes, E, I, gs);
    return (int)hipGetLastError();
}

int launch_moe_decode_cu(const FusedArgs& a, void* stream) {
    if (!decode_cu_fits(a.h, a.E, a.K, a.I, a.gs)) return (int)hipErrorInvalidValue;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (a.h == kHW) {
        switch (a.gs) {
            case 32: launch_w<0>(a, st); break;
            case 64: launch_w<1>(a, st); break;
            default: launch_w<2>(a, st); break;
        }
        return (int)hipGetLastError();
    }
    return a.K * a.I == 8192 ? launch_ug<4>(a, st) : launch_ug<8>(a, st);
}

}  // namespace m1moe
