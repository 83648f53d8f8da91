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
//   gemm<2>                    gate and up for a (rows x 64 pairs) tile,
//                              epilogue act = silu(g) * u  -> f16 [pair][I],
//                              each 32-value block times 2^-e (e = 0 unless
//                              the block passes the f16 range)
//   gemm<1>                    down for a (rows x 64 pairs) tile -> f32 y; only
//                              when some e > 0, first each pair's blocks
//                              brought to its largest e, E, and y times 2^E
//   combine                    out[t] = residual[t] + sum_k w_tk y[pair(t,k)]
//                              in slot order (deterministic, no atomics)
//
// Dequantisation into MFMA operands.  A lane's A fragment is one packed
// word (8 nibbles = 8 columns of one weight row, column 2i in the low nibble
// of byte i).  Masking the word with 0x000F000F leaves columns 0 and 4 as the
// exact f16 subnormals n * 2^-24, masking with 0x00F000F0 columns 1 and 5 as
// n * 2^-20, and the same two masks on the word shifted right by 8 give
// columns 2, 6 and 3, 7.  One v_pk_fma_f16 per pair with (s * 2^(24-k) or
// s * 2^(20-k), b * 2^-k) then gives f16((n * s + b) * 2^-k), a single
// rounding of the exact value (n * s has at most 15 significant bits and
// the FMA is fused).  k is a per-row power of two (the smallest k >= 0 that
// keeps s * 2^(24-k) and the row's weights within f16 range), made at upload
// with the f16 (s * 2^(20-k), b * 2^-k) pairs (PfTileLayout) and undone on
// the row's f32 accumulator.  The columns come out in the order 0, 4, 1, 5,
// 2, 6, 3, 7; the B operands are stored in that order in memory (every
// 8-column group of xq and act is permuted by its producer, prep_x and the
// gate/up epilogue), so both operands agree and no permutation is done in
// the GEMMs (the sum over k does not depend on the order).
//
// The GEMM kernel, pf_mma_kernel: 4 waves, a (128 gate and 128 up rows, or
// 256 down rows) x 64 pairs tile, v_mfma_f32_32x32x16_f16, 64-column
// k-blocks copied global -> LDS by the loads themselves (global_load_lds)
// into a ring of four stages, three blocks ahead: B gathered from the pairs'
// xq or act rows, A and the scale words from the expert's prefill copy
// (PfTileLayout, made at upload), stored as the LDS image of a stage.
//
// MFMA v_mfma_f32_32x32x16_f16: A 32x16 (lane l: row l%32, k 8(l/32)..+7),
// B 16x32 (lane l: column l%32, the same k), D 32x32 (lane l: column l%32,
// element v: row 8(v/4) + 4(l/32) + v%4).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "device.hpp"
#include "internal.hpp"

namespace m1moe {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTN = kPfTN;
constexpr int kMaxE = 256;


// ---- grouping of (token, slot) pairs by expert ----------------------------------

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(v, o, 64);
        if (lane >= o) v += u;
    }
    return v;
}

constexpr int kGP = 8;  // pairs per thread per pass of group_kernel

// One workgroup.  Pair p = t*K + k gets the sorted position pos[p]; the order
// of pairs within an expert is arbitrary (each pair's GEMM column is computed
// independently of the others, so results do not depend on it).  A thread
// takes kGP pairs per pass with all their loads in flight; when one pass
// covers every pair (P <= 1024 kGP) their experts and ranks stay in
// registers until the positions are written.  One wave computes the prefix
// sums (4 experts per lane).
__global__ __launch_bounds__(1024) void group_kernel(PrefillArgs a) {
    __shared__ int cnt[kMaxE];
    __shared__ int off[kMaxE + 1], toff[kMaxE + 1], qoff[4][kMaxE + 1], qtot[4];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int E = a.E, P = a.T * a.K;
    if (tid < kMaxE) cnt[tid] = 0;
    // the down GEMM's flag (set by gate/up), barrier words and bitmap of
    // rewritten act rows (act_fix)
    for (int j = tid; j < kPfFlagWords + (P + 31) / 32; j += 1024) a.act_flag[j] = 0u;
    __syncthreads();
    const bool one_pass = P <= 1024 * kGP;
    int pe[kGP], pr[kGP];
    for (int base = 0; base < P; base += 1024 * kGP) {
#pragma unroll
        for (int j = 0; j < kGP; ++j) {
            const int p = base + j * 1024 + tid;
            pe[j] = p < P ? a.idx[p] : -1;
        }
#pragma unroll
        for (int j = 0; j < kGP; ++j) pr[j] = pe[j] >= 0 ? atomicAdd(&cnt[pe[j]], 1) : 0;
        if (!one_pass) {
#pragma unroll
            for (int j = 0; j < kGP; ++j) {
                const int p = base + j * 1024 + tid;
                if (p < P) a.pos[p] = pr[j];
            }
        }
    }
    __syncthreads();
    // exclusive prefix sums of the pair and N-tile counts, and of the tiles of
    // each size class (c + 1 quarters of 32 pairs: every full tile has 4, an
    // expert's last tile ceil(rest / 32)); entry E holds the totals
    if (wave == 0) {
        int c[4], tl[4], qq[4][4];
        int sc = 0, st = 0, sq[4] = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = 4 * lane + j;
            c[j] = i < E ? cnt[i] : 0;
            tl[j] = (c[j] + kTN - 1) / kTN;
            const int r = c[j] % kTN, last = r ? (r + 31) / 32 - 1 : -1;
#pragma unroll
            for (int k = 0; k < 4; ++k) qq[k][j] = (k == 3 ? c[j] / kTN : 0) + (last == k ? 1 : 0);
            sc += c[j];
            st += tl[j];
#pragma unroll
            for (int k = 0; k < 4; ++k) sq[k] += qq[k][j];
        }
        int ec = wave_incl_scan(sc, lane) - sc, et = wave_incl_scan(st, lane) - st, eq[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) eq[k] = wave_incl_scan(sq[k], lane) - sq[k];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = 4 * lane + j;
            if (i <= E) {
                off[i] = ec;
                toff[i] = et;
#pragma unroll
                for (int k = 0; k < 4; ++k) qoff[k][i] = eq[k];
                a.expert_off[i] = ec;
                a.tile_off[i] = et;
            }
            ec += c[j];
            et += tl[j];
#pragma unroll
            for (int k = 0; k < 4; ++k) eq[k] += qq[k][j];
        }
        if (lane == 63) {
#pragma unroll
            for (int k = 0; k < 4; ++k) qtot[k] = eq[k];
            if (E == kMaxE) {  // entry E lies past the lanes' 4 x 64 experts
                off[E] = ec;
                toff[E] = et;
                a.expert_off[E] = ec;
                a.tile_off[E] = et;
            }
        }
    }
    // one descriptor per N-tile the GEMMs may see ((P + kTN - 1) / kTN + E of
    // them): expert, first sorted position, pairs; none past the last.  The
    // tiles are ordered by size class, 4 quarters first, then 3, 2, 1
    // (experts in order within a class), so that the GEMMs, which deal
    // their queues out forwards and backwards in turn, give the long work
    // out first and even out each workgroup's total.
    const int nt_max = (P + kTN - 1) / kTN + E;
    for (int j = tid; j < nt_max; j += 1024) a.tile_desc[j] = PfTile{0, 0, 0, 0};
    __syncthreads();
    if (tid < E) {
        int base[4];
        base[3] = 0;
        base[2] = qtot[3];
        base[1] = base[2] + qtot[2];
        base[0] = base[1] + qtot[1];
        for (int j = 0; j < toff[tid + 1] - toff[tid]; ++j) {
            const int p0 = off[tid] + j * kTN;
            const int np = min(kTN, off[tid + 1] - p0);
            const int q = (np + 31) / 32 - 1;
            // full tiles of the expert first in its class-4 run, its last
            // tile after them (class 4) or alone in its class
            const int at = base[q] + qoff[q][tid] + (q == 3 ? j : 0);
            a.tile_desc[at] = PfTile{tid, p0, np, 0};
        }
    }
    if (one_pass) {
#pragma unroll
        for (int j = 0; j < kGP; ++j) {
            const int p = j * 1024 + tid;
            if (p < P) {
                const int q = off[pe[j]] + pr[j];
                const int t = p / a.K;
                a.pos[p] = q;
                a.sorted_tok[q] = PfPair{t, a.xinv[t]};
            }
        }
    } else {
        for (int p = tid; p < P; p += 1024) {
            const int q = off[a.idx[p]] + a.pos[p];
            const int t = p / a.K;
            a.pos[p] = q;
            a.sorted_tok[q] = PfPair{t, a.xinv[t]};
        }
    }
}

// ---- grouped GEMM with fused dequantisation ---------------------------------------

// A fragment of one packed word: f16((n * s + b) * 2^-k) for its 8 columns in
// the order 0, 4, 1, 5, 2, 6, 3, 7 (s24 = s * 2^(24-k), s20 = s * 2^(20-k),
// b2 = b * 2^-k, each in both halves).
__device__ __forceinline__ f16x8 dequant_word(uint32_t w, f16x2 s24, f16x2 s20, f16x2 b2) {
    const uint32_t w8 = w >> 8;
    const f16x2 p0 = __builtin_bit_cast(f16x2, w & 0x000F000Fu);   // columns 0, 4: n * 2^-24
    const f16x2 p1 = __builtin_bit_cast(f16x2, w & 0x00F000F0u);   // columns 1, 5: n * 2^-20
    const f16x2 p2 = __builtin_bit_cast(f16x2, w8 & 0x000F000Fu);  // columns 2, 6
    const f16x2 p3 = __builtin_bit_cast(f16x2, w8 & 0x00F000F0u);  // columns 3, 7
    const f16x2 q0 = __builtin_elementwise_fma(p0, s24, b2);
    const f16x2 q1 = __builtin_elementwise_fma(p1, s20, b2);
    const f16x2 q2 = __builtin_elementwise_fma(p2, s24, b2);
    const f16x2 q3 = __builtin_elementwise_fma(p3, s20, b2);
    return f16x8{q0[0], q0[1], q1[0], q1[1], q2[0], q2[1], q3[0], q3[1]};
}

// The three operands of dequant_word from a PfTileLayout scale word
// (f16 s * 2^(20-k) | f16 b * 2^-k << 16).
__device__ __forceinline__ void scale_ops(uint32_t sb, f16x2& s24, f16x2& s20, f16x2& b2) {
    const uint32_t lo = sb & 0xffffu, hi = sb >> 16;
    s20 = __builtin_bit_cast(f16x2, lo | (lo << 16));
    s24 = s20 * (f16x2){(_Float16)16.f, (_Float16)16.f};
    b2 = __builtin_bit_cast(f16x2, hi | (hi << 16));
}

// 2^k of a row from its PfTileLayout exponent byte.
__device__ __forceinline__ float row_scale(uint32_t k) {
    return __uint_as_float((127u + (k & 0xffu)) << 23);
}

// ---- pipelined grouped GEMM: operands copied to LDS by the loads themselves -------

// Workgroup: 4 waves, one (TM weight rows x kTN = 128 pairs) tile of one expert.
// NMAT = 2: TM = 128; wave w owns rows 32 w .. 32 w + 31 of gate (row-mat 0)
//           and of up (row-mat 1), B = xq rows of the pairs' tokens.
// NMAT = 1: TM = 256; wave w owns rows 64 w .. 64 w + 63 of down (row-mats 0
//           and 1: its two halves of 32), B = act rows of the pairs.
// Lane l: c = l % 32 (the A row within a row-mat, the B pair within each
// 32-pair quarter), kh = l / 32; in a 64-column k-block the lane owns columns
// 32 kh .. 32 kh + 31 of its rows (4 packed words) and MFMA step s (0..3)
// takes word s and the B columns 32 kh + 8 s .. + 7.  Every dequantised A
// fragment feeds one MFMA per quarter of the tile's pairs; a tile copies and
// multiplies only the NQ = ceil(pairs / 32) quarters it has.
//
// A stage (one k-block) in LDS, every byte copied from global memory by
// global_load_lds (no registers, no VALU):
//   A, S  the (M-tile, k-block) chunk of the expert's prefill copy
//      (PfTileLayout), copied as it is: it is stored as this LDS image
//   B  [128 pairs][8 units of 16 bytes]   unit u of pair p at position
//      u ^ (p & 7) ^ ((p >> 3) & 1), gathered from the pairs' xq or act rows
// The swizzles put the 8 (or 16) lanes served together by one ds_read_b128
// on distinct banks.  Per stage a wave copies 2 KB of A, 256 bytes (512 at
// group size 32) of S and NQ KB of B, each copy addressed by
// a wave-uniform base in SGPRs, advanced per block by scalar adds, plus a
// fixed per-lane offset (lane j of a B copy fetching the unit that belongs
// at its position).
//
// Pipeline: NS ring slots (3 for tiles of 3 or 4 quarters, 4 for 2, 5 for
// 1: the LDS of three full stages); block kb's copies are issued NS - 1
// blocks ahead into slot kb % NS.  Before block kb is multiplied each wave
// waits until only the copies of blocks kb + 1 .. kb + NS - 2 are
// outstanding (memory loads complete in issue order), then a barrier makes
// every wave's copies of block kb visible; the slot of block kb - 1, read by
// every wave before that barrier, is then refilled with block kb + NS - 1.
constexpr int kMK = 64;                       // k per block
constexpr int kMA = 256 * kMK / 2;            // 8 KB of A
constexpr int kMB = kTN * kMK * 2;            // 16 KB of B
// scale words (two groups per block at gs 32) and a whole stage
template <int GSL>
constexpr int mma_sbytes() { return (GSL == 0 ? 2 : 1) * 256 * 4; }
template <int GSL>
constexpr int mma_stage() { return kMA + mma_sbytes<GSL>() + kMB; }
constexpr int kMSlots = 3;
// A tile of NQ quarters uses stages of NQ quarters of B, and as many of them
// as the LDS of three full stages holds (3, 3, 4, 5 for NQ = 4, 3, 2, 1): a
// narrow tile keeps more k-blocks of A in flight, which is what bounds it.
template <int GSL, int NQ>
constexpr int mma_stage_q() { return kMA + mma_sbytes<GSL>() + NQ * (kMB / 4); }
template <int GSL, int NQ>
constexpr int mma_slots() { return kMSlots * mma_stage<GSL>() / mma_stage_q<GSL, NQ>(); }

// Copy sources (per block kb: base + kb * stride, plus the lane's offset) and
// the lane's LDS read offsets within a stage.
struct MmaSrc {
    const uint8_t* bbase;                     // first B row (xq or act), block 0
    const uint8_t* abase;                     // the M-tile's chunk of block 0
    uint32_t chunk;                           // bytes per block of the prefill copy
    uint32_t boff[4];                         // B copy i: the lane's unit of its pair's row
    uint32_t aoff[2];                         // A copy i
    uint32_t soff[2];                         // S copy i (second only at gs 32)
    uint32_t bread[4];                        // B operand of step s, pairs 0..31
    uint32_t aread[2];                        // A unit of row-mat rm
    uint32_t sread[2];                        // scale word of row-mat rm
    uint32_t wave;
};

// vmcnt(n) alone (expcnt and lgkmcnt at their maxima, no wait on them).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt field is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// global -> LDS copy of 16 (or 4) bytes per lane from sbase + voff (sbase in
// SGPRs, voff the lane's 32-bit offset): lane j's bytes land at LDS byte
// address lds + 16 j (4 j); lds is the same for the whole wave.  Written as
// inline assembly: the compiler, which cannot tell the ring slots apart,
// would otherwise wait for every copy in flight before each LDS read.  The
// kernel waits for the copies itself (vmcnt, which counts them in issue
// order with every other load) before the barrier that publishes a slot; the
// compiler's own vmcnt waits for its loads stay safe, as copies it does not
// know of only make them wait longer.  M0 is not listed as clobbered (the
// compiler reserves it and warns): these kernels contain no instruction of
// the compiler's that reads M0 (no LDS-DMA builtins, indexed lane reads or
// messages; the generated code sets M0 only in these statements).
__device__ __forceinline__ void lds_copy16(uint32_t voff, const uint8_t* sbase, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds)
                 : "memory");
}
// The same, coherent across the XCDs (sc1: the line is read from memory, not
// from this XCD's L2): the down GEMM's B when act_fix rewrote act in this launch.
__device__ __forceinline__ void lds_copy16_coh(uint32_t voff, const uint8_t* sbase, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 sc1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds)
                 : "memory");
}
__device__ __forceinline__ void lds_copy4(uint32_t voff, const uint8_t* sbase, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds)
                 : "memory");
}

// LDS byte address of a pointer into LDS.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Copies one wave issues per block: A 2, S 1 or 2, B NQ.
template <int GSL, int NQ>
constexpr int mma_ops() { return 2 + (GSL == 0 ? 2 : 1) + NQ; }

// Block kb's copies into ring slot SLOT (ring: LDS address of slot 0).
// Issued for every step, also past the last block (kb is then clamped: the
// last block is read again into a slot no step reads), so that every wave
// always has the same number of copies issued after any block's.
template <int GSL, int NQ, int SLOT, bool COH>
__device__ __forceinline__ void mma_issue(const MmaSrc& src, int kb, int nblk, uint32_t ring) {
    kb = min(kb, nblk - 1);
    const uint32_t st = ring + SLOT * mma_stage_q<GSL, NQ>();
    const uint8_t* ab = src.abase + (size_t)kb * src.chunk;
#pragma unroll
    for (int i = 0; i < 2; ++i) lds_copy16(src.aoff[i], ab, st + (2 * src.wave + i) * 1024);
#pragma unroll
    for (int i = 0; i < (GSL == 0 ? 2 : 1); ++i)
        lds_copy4(src.soff[i], ab, st + kMA + i * 1024 + src.wave * 256);
    const uint8_t* bb = src.bbase + (size_t)kb * (kMK * 2);
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
        if (COH)
            lds_copy16_coh(src.boff[i], bb, st + kMA + mma_sbytes<GSL>() + (NQ * src.wave + i) * 1024);
        else
            lds_copy16(src.boff[i], bb, st + kMA + mma_sbytes<GSL>() + (NQ * src.wave + i) * 1024);
    }
}

template <int GSL, int NQ>
__device__ __forceinline__ void mma_compute(const MmaSrc& src, const uint8_t* lds,
                                            f32x16 (&acc)[2][4]) {
    constexpr int kB = kMA + mma_sbytes<GSL>();   // B's offset in a stage
    uint4 aw[2];
    f16x2 s24[2], s20[2], b2[2];
#pragma unroll
    for (int rm = 0; rm < 2; ++rm) {
        aw[rm] = *reinterpret_cast<const uint4*>(lds + src.aread[rm]);
        scale_ops(*reinterpret_cast<const uint32_t*>(lds + kMA + src.sread[rm]), s24[rm],
                  s20[rm], b2[rm]);
    }
    // the B operands of step s + 1 are read while step s is multiplied
    f16x8 bf[2][NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q)
        bf[0][q] = *reinterpret_cast<const f16x8*>(lds + kB + src.bread[0] + q * (32 * kMK * 2));
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        if (s + 1 < 4) {
#pragma unroll
            for (int q = 0; q < NQ; ++q)
                bf[(s + 1) & 1][q] = *reinterpret_cast<const f16x8*>(
                    lds + kB + src.bread[s + 1] + q * (32 * kMK * 2));
        }
        f16x8 af[2];
#pragma unroll
        for (int rm = 0; rm < 2; ++rm) {
            const uint32_t w = s == 0 ? aw[rm].x : s == 1 ? aw[rm].y : s == 2 ? aw[rm].z : aw[rm].w;
            af[rm] = dequant_word(w, s24[rm], s20[rm], b2[rm]);
        }
#pragma unroll
        for (int rm = 0; rm < 2; ++rm)
#pragma unroll
            for (int q = 0; q < NQ; ++q)
                acc[rm][q] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[rm], bf[s & 1][q],
                                                                    acc[rm][q], 0, 0, 0);
    }
}

// Steps I .. NS - 1 of one round of the ring (every slot's LDS offsets are
// constants).
template <int I, int NS, class F>
__device__ __forceinline__ void mma_round(int kb, F& step) {
    if constexpr (I < NS) {
        step(kb + I, std::integral_constant<int, I>{});
        mma_round<I + 1, NS>(kb, step);
    }
}

// The k loop over the NS = mma_slots ring slots of ring: blocks 0 .. NS - 2
// are issued first; step kb waits for block kb (NS - 2 younger blocks may be
// in flight), passes the barrier after which every wave is done with block
// kb - 1's slot, issues block kb + NS - 1 into that slot and multiplies
// block kb.
// (COH: B copied with lds_copy16_coh)
template <int GSL, int NQ, bool COH>
__device__ __forceinline__ void mma_loop(const MmaSrc& src, int nblk, const uint8_t* ring,
                                         f32x16 (&acc)[2][4]) {
    constexpr int ops = mma_ops<GSL, NQ>();
    constexpr int stage = mma_stage_q<GSL, NQ>();
    constexpr int NS = mma_slots<GSL, NQ>();
    static_assert(NS >= 3 && ops * (NS - 2) < 64, "ring depth");
    const uint32_t rl = lds_addr(ring);
    auto first = [&](int kb, auto slot) {
        constexpr int S = decltype(slot)::value;
        if constexpr (S < NS - 1) mma_issue<GSL, NQ, S, COH>(src, kb, nblk, rl);
    };
    mma_round<0, NS>(0, first);
    auto step = [&](int kb, auto slot) {
        constexpr int S = decltype(slot)::value;
        if (kb >= nblk) return;
        wait_vm<ops * (NS - 2)>();  // block kb's copies are in (the next NS - 2 may not be)
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        mma_issue<GSL, NQ, (S + NS - 1) % NS, COH>(src, kb + NS - 1, nblk, rl);
        __builtin_amdgcn_sched_barrier(0);
        mma_compute<GSL, NQ>(src, ring + S * stage, acc);
    };
    for (int kb = 0; kb < nblk; kb += NS) mma_round<0, NS>(kb, step);
    // no copy into LDS may still be in flight when the workgroup ends
    wait_vm<0>();
}

// Stores coherent across the XCDs (sc1: written through to memory), for
// what act_fix hands to other workgroups.
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void st_coh16(void* p, u32x4v v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st_coh_u8(uint8_t* p, uint32_t v) {
    asm volatile("global_store_byte %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}

// act blocks to one exponent per pair (the down GEMM's prologue when
// act_flag[0] is set; every workgroup of the launch, all of them resident):
// wave w of the grid takes pairs w, w + 4 grid, ...; a block with e < E, E
// the pair's largest e, is multiplied by 2^(e - E) in place (in f16), and E
// goes to the pair's first act exponent byte, where the epilogue reads it.
// Those writes are coherent (st_coh16, st_coh_u8) and so are their readers
// (lds_copy16_coh for the tiles with a rewritten row, agent-scope loads of
// the E words): no cache
// write-back or invalidation.  Bit p of the bitmap after the barrier words
// marks pair p's row as rewritten.  Then a grid barrier in two levels (one
// address taking every workgroup's count and poll costs microseconds): the
// workgroups of residue x = block id % 8 count themselves on word x, the
// last of them counts residue x on the second-level word, and the last of
// those releases the 8 replicas that the workgroups of each residue poll
// (all zeroed by group_kernel); the waits are bounded (device flag 128).
__device__ __forceinline__ void act_fix(const PrefillArgs& a) {
    const int P = a.T * a.K, nb = a.I >> 5, lane = threadIdx.x & 63;
    for (int p = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6); p < P; p += (int)gridDim.x * 4) {
        uint8_t* ep = a.act_exp + (size_t)p * nb;
        int E = 0;
        for (int b = lane; b < nb; b += 64) E = max(E, (int)ep[b]);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) E = max(E, __shfl_xor(E, o));
        if (E == 0) continue;
        _Float16* row = a.act + (size_t)p * a.I;
        bool rewrote = false;
        for (int j = lane * 8; j < a.I; j += 512) {
            const int e = ep[j >> 5];
            if (e == E) continue;
            rewrote = true;
            const float f = __builtin_bit_cast(float, (127 + e - E) << 23);   // e - E >= -113
            _Float16 v[8];
            *reinterpret_cast<uint4*>(v) = *reinterpret_cast<const uint4*>(row + j);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = (_Float16)((float)v[i] * f);
            st_coh16(row + j, __builtin_bit_cast(u32x4v, v));
        }
        // every lane has read ep[] (the loop above ends in its last read)
        __builtin_amdgcn_wave_barrier();
        const bool any = __any(rewrote);
        if (lane == 0) {
            st_coh_u8(ep, (uint32_t)E);
            if (any)
                __hip_atomic_fetch_or(a.act_flag + kPfFlagWords + (p >> 5), 1u << (p & 31),
                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);   // this thread's stores are complete
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t x = blockIdx.x & 7u, per = gridDim.x >> 3;   // (the grid is a multiple of 8)
        uint32_t* rel = a.act_flag + 32 * (10 + x);
        if (__hip_atomic_fetch_add(a.act_flag + 32 * (1 + x), 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT) == per - 1 &&
            __hip_atomic_fetch_add(a.act_flag + 32 * 9, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT) == 7u) {
            for (int r = 0; r < 8; ++r)
                __hip_atomic_store(a.act_flag + 32 * (10 + r), 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        for (int it = 0;; ++it) {
            if (__hip_atomic_load(rel, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) break;
            if (it >= kPfSpinLimit) {
                flag_error(a.err, 128u);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __syncthreads();
}

// Persistent: the workgroups of an XCD take the (N-tile, M-tile) items of
// their queue in rounds of W (W workgroups on the queue), workgroup j taking
// item j of the even rounds and item W - 1 - j of the odd ones.  Queue x
// (block id % 8, modulo the M-tile count when there are fewer than 8
// M-tiles) holds M-tiles x, x + 8, ... of every N-tile, the N-tiles by size
// class (4 quarters of 32 pairs first, then 3, 2, 1) and, per N-tile, its
// M-tiles in a row: the long items start first, every workgroup's total
// work evens out (a large first item is followed by a small second one),
// and the N-tiles of one expert run together on one XCD and share the
// expert's A rows through its L2.
template <int NMAT, int GSL>
__global__ __launch_bounds__(256, 2) void pf_mma_kernel(PrefillArgs a, int m_tiles) {
    constexpr int TM = NMAT == 2 ? 128 : 256;
    __shared__ __attribute__((aligned(1024))) uint8_t s_ring[kMSlots * mma_stage<GSL>()];
    __shared__ int s_tok[kTN];
    __shared__ float s_inv[kTN];
    const int K = NMAT == 2 ? a.h : a.I;
    const int M = NMAT == 2 ? a.I : a.h;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c = lane & 31, kh = lane >> 5;
    const int nq = min(8, m_tiles);
    const int queue = (int)(blockIdx.x & 7) % nq;
    const int n_mg = (m_tiles - queue + nq - 1) / nq;
    const int items = a.tile_off[a.E] * n_mg;
    const int xcds = (8 - queue + nq - 1) / nq;               // block id residues on this queue
    const int per_queue = (int)(gridDim.x >> 3) * xcds;       // workgroups taking this queue
    const int first = (int)(blockIdx.x >> 3) * xcds + (int)(blockIdx.x & 7) / nq;
    // down, only when the gate/up GEMM stored some block of act times 2^-e,
    // e > 0: every pair brought to one exponent first, by all workgroups
    const bool scaled = NMAT == 1 && a.act_flag[0] != 0u;
    if (NMAT == 1 && scaled) act_fix(a);
    for (int r = 0;; ++r) {
        // the queue is dealt out forwards in even rounds and backwards in odd
        // ones: the workgroups that took the largest items of a round take
        // the smallest of the next
        const int item = r * per_queue + ((r & 1) ? per_queue - 1 - first : first);
        if (item >= items) break;
        // every wave is done with the previous item's LDS before the next starts
        __syncthreads();
        const int mt = (item % n_mg) * nq + queue;
        const PfTile desc = a.tile_desc[item / n_mg];
        const int e = desc.e, p0 = desc.p0, np = desc.np;

        if (NMAT == 2 && tid < kTN) {
            const PfPair ti = tid < np ? a.sorted_tok[p0 + tid] : PfPair{0, 0.f};
            s_tok[tid] = ti.tok;
            s_inv[tid] = ti.inv;
        }
        __syncthreads();

        // the expert's prefill copy: this M-tile's chunks (block 0) and row exponents
        const PfTileLayout PT(a.h, a.I, a.gs);
        const uint8_t* px = a.pft_base + (uint64_t)e * a.pft_bytes;
        const int wrow0 = mt * TM + wave * (TM / 4);
        // the exponents of this lane's accumulator rows, loaded now so that their
        // latency passes with the first blocks': gate/up 8 bytes per (matrix, q)
        // (the 8-row group 8 q of the wave's rows), down 4 bytes per (row-mat, q)
        uint2 kx[2][4];
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (NMAT == 2) {
                    kx[m][q] = *reinterpret_cast<const uint2*>(
                        px + (m == 0 ? PT.kg : PT.ku) + wrow0 + 8 * q);
                } else {
                    kx[m][q].x = *reinterpret_cast<const uint32_t*>(px + PT.kd + wrow0 + 32 * m +
                                                                    8 * q + 4 * kh);
                    kx[m][q].y = 0;
                }
            }
        const int nq4 = (np + 31) >> 5;       // NQ, quarters of 32 pairs
        MmaSrc src;
        src.wave = __builtin_amdgcn_readfirstlane(wave);
        src.chunk = (uint32_t)PT.chunk;
        src.abase = px + (NMAT == 2 ? PT.gu + (uint64_t)mt * PT.kbg * PT.chunk
                                    : PT.dn + (uint64_t)mt * PT.kbd * PT.chunk);
        src.bbase = reinterpret_cast<const uint8_t*>(NMAT == 2 ? a.xq : a.act + (size_t)p0 * a.I);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            // A: the chunk's piece 2 w + i as it is; S: its words of tile rows 64 w + lane
            src.aoff[i] = (uint32_t)((2 * wave + i) * 1024 + lane * 16);
            src.soff[i] = (uint32_t)(kMA + i * 1024 + wave * 256 + lane * 4);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // B: piece (NQ w + i) holds pairs 8 piece .. + 7, 128 bytes each
            const int piece = nq4 * wave + i;
            const int pair = 8 * piece + (lane >> 3);
            const int u = (lane & 7) ^ (pair & 7) ^ ((pair >> 3) & 1);
            const int pc = pair < np ? pair : 0;
            const uint64_t row = NMAT == 2 ? (uint64_t)s_tok[pc] * a.h : (uint64_t)pc * a.I;
            src.boff[i] = (uint32_t)(row * 2 + u * 16);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint32_t u =
                (uint32_t)(kh * 4 + s) ^ (uint32_t)(c & 7) ^ (uint32_t)((c >> 3) & 1);
            src.bread[s] = (uint32_t)c * (kMK * 2) + (u << 4);
        }
#pragma unroll
        for (int rm = 0; rm < 2; ++rm) {
            // gate/up: weight row perm8 within each 8 (the accumulator rows of a lane
            // are then 4 consecutive positions of act's permuted groups)
            const int r = NMAT == 2 ? rm * 128 + 32 * wave + ((c & ~7) | perm8(c & 7))
                                    : 64 * wave + 32 * rm + c;
            const int ua = kh ^ ((r >> 2) & 1) ^ ((r >> 3) & 1);
            src.aread[rm] = (uint32_t)r * 32 + (uint32_t)ua * 16;
            src.sread[rm] = (GSL == 0 ? (uint32_t)kh * 1024 : 0u) + (uint32_t)r * 4;
        }

        f32x16 acc[2][4];
#pragma unroll
        for (int rm = 0; rm < 2; ++rm)
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[rm][q][v] = 0.f;
        // (scaled) B read coherently when a row of the tile was rewritten;
        // the E of the lane's pair of quarter q (act_fix): the aligned word
        // Ew[q] holding it is requested now, taken apart in the epilogue
        // (byte Esh[q] / 8), so that its load's latency passes with the GEMM
        bool coh = false;
        uint32_t Ew[4] = {0u, 0u, 0u, 0u}, Esh = 0u;
        if (NMAT == 1 && scaled) {
            for (int wi = p0 >> 5; wi <= (p0 + np - 1) >> 5; ++wi) {
                const uint32_t m = __hip_atomic_load(a.act_flag + kPfFlagWords + wi,
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const int lo = max(p0 - 32 * wi, 0), hi = min(p0 + np - 32 * wi, 32);   // bits [lo, hi)
                const uint32_t mask = (hi >= 32 ? ~0u : (1u << hi) - 1u) & ~((1u << lo) - 1u);
                coh = coh || (m & mask) != 0u;
            }
            // (act_exp is 256-byte aligned: byte offset o lies in word o / 4)
            uint32_t* xw = reinterpret_cast<uint32_t*>(a.act_exp);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const size_t o = (size_t)(p0 + min(q * 32 + c, np - 1)) * (a.I >> 5);
                Ew[q] = __hip_atomic_load(xw + (o >> 2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                Esh |= (uint32_t)(o & 3) << (8 * q);
            }
        }
        if (NMAT == 1 && coh) {
            switch (nq4) {
                case 1: mma_loop<GSL, 1, true>(src, K / kMK, s_ring, acc); break;
                case 2: mma_loop<GSL, 2, true>(src, K / kMK, s_ring, acc); break;
                case 3: mma_loop<GSL, 3, true>(src, K / kMK, s_ring, acc); break;
                default: mma_loop<GSL, 4, true>(src, K / kMK, s_ring, acc); break;
            }
        } else {
            switch (nq4) {
                case 1: mma_loop<GSL, 1, false>(src, K / kMK, s_ring, acc); break;
                case 2: mma_loop<GSL, 2, false>(src, K / kMK, s_ring, acc); break;
                case 3: mma_loop<GSL, 3, false>(src, K / kMK, s_ring, acc); break;
                default: mma_loop<GSL, 4, false>(src, K / kMK, s_ring, acc); break;
            }
        }

        // epilogue: lane holds pair q * 32 + c and, per row-mat, accumulator rows
        // 8 v + 4 kh + i (element 4 v + i); each row's 2^k comes back on it
        if (NMAT == 2 && wrow0 < M) {
            // the row's 2^k, taken from kx where it is used (a table of all 32
            // would stay live through the epilogue)
            auto rs = [&](int m, int v, int i) {
                const int col = perm8(4 * kh + i);
                return row_scale((col < 4 ? kx[m][v].x : kx[m][v].y) >> (8 * (col & 3)));
            };
            // act goes out in blocks of 32 values, this wave's 32 rows of one pair
            // (16 on each lane of c and c + 32): a block whose largest |value|
            // is past the f16 range is stored times 2^-e, e >= 1 the least that
            // fits, and e is kept per block (0 for the others).  A value that is
            // not finite is clamped and reported (device flag 64).
            bool bad = false, scaled = false;
            const int nb = a.I >> 5;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = q * 32 + c;
                if (n >= np) continue;   // both lanes of the pair's block skip together
                const float inv = s_inv[n];
                float y[4][4], mx = 0.f;
#pragma unroll
                for (int v = 0; v < 4; ++v)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float g = acc[0][q][4 * v + i] * rs(0, v, i) * inv;
                        const float u = acc[1][q][4 * v + i] * rs(1, v, i) * inv;
                        y[v][i] = silu_fast(g) * u;  // Shaders.metal:148
                        const bool fin = isfinite(y[v][i]);
                        bad |= !fin;
                        mx = fin ? fmaxf(mx, fabsf(y[v][i])) : mx;
                    }
                mx = fmaxf(mx, __shfl_xor(mx, 32));
                // r = mx / 65504 > 1 is m 2^e with m in [0.5, 1) (e its exponent
                // field - 126): mx 2^-e < 65504
                const float r = mx * (1.f / 65504.f);
                const int e = mx > 65504.f ? (int)((__float_as_uint(r) >> 23) & 255u) - 126 : 0;
                scaled |= e > 0;
                const float sc = __builtin_bit_cast(float, (127 - e) << 23);   // 2^-e, e <= 113
                _Float16* dst = a.act + (size_t)(p0 + n) * a.I + wrow0 + 4 * kh;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    _Float16 o[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        o[i] = (_Float16)fminf(fmaxf(y[v][i] * sc, -65504.f), 65504.f);
                    *reinterpret_cast<uint2*>(dst + 8 * v) = __builtin_bit_cast(uint2, o);
                }
                if (kh == 0) a.act_exp[(size_t)(p0 + n) * nb + (wrow0 >> 5)] = (uint8_t)e;
            }
            if (__any(bad) && lane == 0) flag_error(a.err, 64u);
            if (__any(scaled) && lane == 0) a.act_flag[0] = 1u;
        } else if (NMAT == 1) {
#pragma unroll
            for (int rm = 0; rm < 2; ++rm) {
                const int rb = wrow0 + 32 * rm;
                if (rb >= M) continue;
                float rs[4][4];
#pragma unroll
                for (int v = 0; v < 4; ++v)
#pragma unroll
                    for (int i = 0; i < 4; ++i) rs[v][i] = row_scale(kx[rm][v].x >> (8 * i));
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int n = q * 32 + c;
                    if (n >= np) continue;
                    float* dst = a.y + (size_t)(p0 + n) * a.h + rb + 4 * kh;
                    // the pair's 2^E (1 unless scaled; exact): E in the first
                    // byte of its act exponents (act_fix)
                    const int pE = (int)((Ew[q] >> (8 * ((Esh >> (8 * q)) & 3u))) & 255u);
                    const float pe = __builtin_bit_cast(float, (127 + pE) << 23);
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        *reinterpret_cast<f32x4*>(dst + 8 * v) = f32x4{
                            acc[rm][q][4 * v] * rs[v][0] * pe, acc[rm][q][4 * v + 1] * rs[v][1] * pe,
                            acc[rm][q][4 * v + 2] * rs[v][2] * pe, acc[rm][q][4 * v + 3] * rs[v][3] * pe};
                }
            }
        }
    }
}

// ---- the prefill copy of the expert blocks (PfTileLayout), made at upload -----------

// One thread per (expert, row of the padded gate, up and down row ranges): the
// row's power of two k (0 past the matrix).  A non-finite scale or bias sets
// error flag 8.
__global__ __launch_bounds__(256) void pf_row_exp_kernel(const uint8_t* src, uint64_t src_bytes,
                                                         uint8_t* dst, uint64_t dst_bytes, int E,
                                                         int h, int I, int gs, uint32_t* err) {
    const PfTileLayout P(h, I, gs);
    const int rows = 2 * P.mg * 128 + P.md * 256;
    const uint64_t gid = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= (uint64_t)E * rows) return;
    const int e = (int)(gid / rows), ri = (int)(gid - (uint64_t)e * rows);
    const int m = ri < P.mg * 128 ? 0 : (ri < 2 * P.mg * 128 ? 1 : 2);
    const int row = m == 2 ? ri - 2 * P.mg * 128 : ri - m * P.mg * 128;
    uint8_t* d = dst + (uint64_t)e * dst_bytes + (m == 0 ? P.kg : (m == 1 ? P.ku : P.kd)) + row;
    if (row >= (m == 2 ? h : I)) {
        *d = 0;
        return;
    }
    const int groups = (m == 2 ? I : h) / gs;
    const Layout L(h, I, gs);
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
        while (k < 100 && (ldexpf(ms, 24 - k) > 65504.f || ldexpf(mw, -k) > 65504.f)) ++k;
    }
    *d = (uint8_t)k;
}

// One thread per 16 bytes of the chunks of E experts (after pf_row_exp_kernel
// on the same stream): an A unit (16 packed bytes of one row) or four rows'
// scale words of one group.
__global__ __launch_bounds__(256) void pf_tile_copy_kernel(const uint8_t* src, uint64_t src_bytes,
                                                           uint8_t* dst, uint64_t dst_bytes, int E,
                                                           int h, int I, int gs) {
    const PfTileLayout P(h, I, gs);
    const uint64_t per_chunk = P.chunk / 16;
    const uint64_t chunks = (uint64_t)P.mg * P.kbg + (uint64_t)P.md * P.kbd;
    const uint64_t gid = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= (uint64_t)E * chunks * per_chunk) return;
    const uint64_t e = gid / (chunks * per_chunk), uo = gid - e * chunks * per_chunk;
    const uint64_t ci = uo / per_chunk;
    const int within = (int)(uo - ci * per_chunk) * 16;
    const bool gu = ci < (uint64_t)P.mg * P.kbg;
    const int mt = gu ? (int)(ci / P.kbg) : (int)((ci - (uint64_t)P.mg * P.kbg) / P.kbd);
    const int kb = gu ? (int)(ci % P.kbg) : (int)((ci - (uint64_t)P.mg * P.kbg) % P.kbd);
    const Layout L(h, I, gs);
    const uint8_t* b = src + e * src_bytes;
    uint8_t* d = dst + e * dst_bytes;
    // tile row r -> (matrix, row); false past the matrix
    auto tile_row = [&](int r, int& m, int& row) {
        m = gu ? r >> 7 : 2;
        row = gu ? mt * 128 + (r & 127) : mt * 256 + r;
        return row < (gu ? I : h);
    };
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (within < 256 * 32) {
        const int r = within >> 5;
        const int kh = ((within >> 4) & 1) ^ ((r >> 2) & 1) ^ ((r >> 3) & 1);
        int m, row;
        if (tile_row(r, m, row)) {
            const int K = m == 2 ? I : h;
            const uint64_t wo = m == 0 ? L.gate_w : (m == 1 ? L.up_w : L.down_w);
            v = *reinterpret_cast<const uint4*>(b + wo + (uint64_t)row * (K / 2) + kb * 32 +
                                                kh * 16);
        }
    } else {
        const int so = within - 256 * 32, j = so >> 10, r0 = (so & 1023) >> 2;
        const int g = gs == 32 ? 2 * kb + j : (gs == 64 ? kb : kb >> 1);
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int m, row;
            w[i] = 0u;
            if (!tile_row(r0 + i, m, row)) continue;
            const int groups = (m == 2 ? I : h) / gs;
            const int k = d[(m == 0 ? P.kg : (m == 1 ? P.ku : P.kd)) + row];
            const uint64_t o = ((uint64_t)row * groups + g) * 2;
            const float sf = bf16_to_f32(*reinterpret_cast<const uint16_t*>(
                b + (m == 0 ? L.gate_s : (m == 1 ? L.up_s : L.down_s)) + o));
            const float bf = bf16_to_f32(*reinterpret_cast<const uint16_t*>(
                b + (m == 0 ? L.gate_b : (m == 1 ? L.up_b : L.down_b)) + o));
            const _Float16 s16 = (_Float16)ldexpf(sf, 20 - k);
            const _Float16 b16 = (_Float16)ldexpf(bf, -k);
            w[i] = (uint32_t)__builtin_bit_cast(uint16_t, s16) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, b16) << 16);
        }
        v = make_uint4(w[0], w[1], w[2], w[3]);
    }
    *reinterpret_cast<uint4*>(d + (gu ? P.gu : P.dn) +
                              ((gu ? (uint64_t)mt * P.kbg : (uint64_t)mt * P.kbd) + kb) * P.chunk +
                              within) = v;
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

// Workgroups of pf_mma_kernel<NMAT, GSL> one compute unit holds at once (2
// by its launch bounds and LDS; asked of the runtime once per process).
template <int NMAT, int GSL>
int pf_resident_per_cu() {
    static const int n = [] {
        int b = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, pf_mma_kernel<NMAT, GSL>, 256, 0) !=
                hipSuccess ||
            b < 1)
            b = 1;
        return std::min(b, 2);
    }();
    return n;
}

// Persistent workgroups, as many as the compute units hold at once (two per
// CU; at most one per item), a multiple of 8 so that every XCD holds the
// same number.  All of them resident is what the down GEMM's rare grid
// barrier (act_fix) needs.
template <int NMAT, int GSL>
void launch_one(const PrefillArgs& a, hipStream_t st, int ntiles_max) {
    const int M = NMAT == 2 ? a.I : a.h;
    constexpr int TM = NMAT == 2 ? 128 : 256;
    const int m_tiles = (M + TM - 1) / TM;
    const long items = (long)ntiles_max * m_tiles;
    const long cap = (long)pf_resident_per_cu<NMAT, GSL>() * (a.cus > 0 ? a.cus : 256);
    const int grid = (int)std::min((std::min(items, cap) + 7) / 8 * 8, std::max(cap / 8 * 8, 8L));
    hipLaunchKernelGGL((pf_mma_kernel<NMAT, GSL>), dim3((unsigned)grid), dim3(256), 0, st, a,
                       m_tiles);
}

template <int GSL>
int launch_gemms(const PrefillArgs& a, hipStream_t st) {
    const int P = a.T * a.K;
    const int ntiles_max = (P + kTN - 1) / kTN + a.E;
    launch_one<2, GSL>(a, st, ntiles_max);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    launch_one<1, GSL>(a, st, ntiles_max);
    return (int)hipGetLastError();
}

}  // namespace

int launch_pf_tile_copy(const uint8_t* layer, uint64_t expert_bytes, uint8_t* dst, int E, int h,
                        int I, int gs, uint32_t* err, void* stream) {
    const PfTileLayout P(h, I, gs);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const uint64_t rows = (uint64_t)E * (uint64_t)(2 * P.mg * 128 + P.md * 256);
    hipLaunchKernelGGL(pf_row_exp_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st,
                       layer, expert_bytes, dst, P.bytes, E, h, I, gs, err);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    const uint64_t units = (uint64_t)E * ((uint64_t)P.mg * P.kbg + (uint64_t)P.md * P.kbd) *
                           (P.chunk / 16);
    hipLaunchKernelGGL(pf_tile_copy_kernel, dim3((unsigned)((units + 255) / 256)), dim3(256), 0,
                       st, layer, expert_bytes, dst, P.bytes, E, h, I, gs);
    return (int)hipGetLastError();
}

int launch_prefill(const PrefillArgs& a, void* stream) {
    if (a.E > kMaxE || a.h > 16384 || a.h % 64 || a.I % 64) return (int)hipErrorInvalidValue;
    hipStream_t st = static_cast<hipStream_t>(stream);
    // (x's f16 copy xq / xinv was made by the router's logits kernel)
    hipLaunchKernelGGL(group_kernel, dim3(1), dim3(1024), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
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
