// internal.hpp — shared host-side definitions of libm1moe_hip.so.
#pragma once

#include <cstdint>

#include "m1moe_hip.h"

// constructors shared by host code and kernels
#if defined(__HIPCC__)
#define M1MOE_HD __host__ __device__
#else
#define M1MOE_HD
#endif

namespace m1moe {

// Geometry of one expert block in the reference's planar layout
// (ModelSpec.swift:36-52, InferenceEngine.swift:84-97):
// off[0..8] = gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s, down_b.
struct Geom {
    int32_t h, E, K, I, gs, L, norm;
    uint64_t off[9];
    uint64_t expert_bytes;
    int32_t rows(int proj) const { return proj == 2 ? h : I; }
    int32_t cols(int proj) const { return proj == 2 ? I : h; }
};

Geom make_geom(const m1moe_moe_shape& s);

// Records a printf-style message as the thread's last error; returns code.
int32_t fail(int32_t code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// One projection of an expert block: packed words, scales and biases are
// reached from the block base by these byte offsets.
struct ProjView {
    uint64_t w_off, s_off, b_off;
    int32_t rows, cols;
};

// Arguments of the fused decode kernel (one token through one layer).  The
// nine sub-block offsets of an expert block are derived in the kernel from
// (h, I, gs) rather than passed.
struct FusedArgs {
    const uint8_t* layer_base;   // first expert block of the layer
    uint64_t expert_bytes;
    const uint16_t* router;      // [E][h] bf16
    const uint16_t* next_router; // the next layer's router (read into the XCD's L2 near the
                                 // end of the launch, for the next layer's launch), or null
    const float* bias;           // [E] or null
    const void* x;               // [h] f32 or bf16
    const float* residual;       // [h] or null
    float* out;                  // [h]
    const int32_t* given_idx;    // [K] routing supplied by the caller, or null
    const float* given_w;        // [K]
    int32_t* user_idx;           // optional copies of the routing
    float* user_w;
    // optional RMSNorm of an f32 input (the decoder's post-attention norm):
    // x <- x * rsqrt(sum(x^2) / h + x_eps) * x_norm_w, sum(x^2) given as
    // n_ssq partial sums (added in a fixed order, so every wave gets the same
    // value)
    const float* x_ssq;
    const uint16_t* x_norm_w;
    int32_t n_ssq;
    float x_eps;
    // hand-off state.  It starts at zero and is never reset between launches:
    // every workgroup counts its own launches in seen[wg], so all workgroups
    // agree on the launch number ("tag") without communicating.
    unsigned long long* slots;   // [kLogitRep][kRepStride] logits tagged with the launch number
    unsigned long long* xl;      // [8 XCDs][kRepStride] the same, XCD-local (decode_cu.hip)
    float* act;                  // [K][I] silu(gate) * up
    uint32_t* gu_cnt;            // [kNRep][n_cnt] monotonic counters of finished gate/up
                                 // tiles, kCntStride apart
    uint32_t* seen;              // [grid] launches completed by each workgroup
    // the one-workgroup-per-CU kernel (decode_cu.hip): the layer's repacked
    // expert blocks, its own launch counters, counters and partial sums
    const uint8_t* dec_base;     // [E][dec_bytes] repacked copy of the layer's experts
    uint64_t dec_bytes;
    uint32_t* cu_seen;           // [kCuWorkgroups]
    uint32_t* cu_cnt;            // [kCuRep][kCuParts] counters, kCntStride apart
    uint32_t* cu_part;           // [kCuWorkgroups][kCuWorkgroups][8] tagged partial sums
    uint32_t* err;               // sticky device error flag
    int32_t h, E, K, I, gs, norm, x_bf16, spin_limit;
    // work decomposition (filled by decode_grid)
    int32_t n_gu;                // gate/up workgroups (persistent over all slots)
    int32_t Cg, seg_g, rpi_g;    // gate/up: 32-column chunks per row, lanes per row, rows per wave step
    int32_t rows_tile, tiles_per_slot;
    int32_t n_dn, Rd;            // down workgroups, rows per down workgroup
    int32_t Cd, Cp, seg_d, nb;   // down: chunks per row, padded chunks per slot, lanes per
                                 // segment, 64-lane blocks per slot (Cp >= 64)
    int32_t spu, units;          // slots per 64-lane unit (Cp < 64), units per row block
    int32_t cp_log2;             // log2(Cp) when Cp < 64
    // counted units of gate/up tiles: one per slot (Cp < 64) or one per
    // (slot, 64-chunk block of the down input) (Cp >= 64), so a down unit
    // waits only for the act rows it reads.  Replica r = copy * cnt_parts +
    // part: a gate/up workgroup adds to part (wg % cnt_parts) of every copy,
    // a consumer sums the cnt_parts parts of one copy.
    int32_t n_cnt, cnt_parts;
};

// Replicas of the hand-off words (published logits, slot counters), so that
// each line has few pollers.  Counter (replica r, slot k) is word
// (r * K + k) * kCntStride: consecutive 128-byte lines, which spreads them over
// the L2 channels (replicas exactly 4 KiB apart would share one channel).
constexpr int kNRep = 32;            // counter replicas
constexpr int kCntParts = 4;         // parts of a count when gate/up workgroups take several tiles
constexpr int kLogitRep = 8;         // logit replicas
constexpr int kRepStride = 544;      // u64 words between logit replicas (4352 B)
constexpr int kCntStride = 32;       // u32 words between counters (128 B)
constexpr int kDecodeWaves = 4;    // waves per decode workgroup
constexpr int kCuWorkgroups = 256; // decode_cu.hip: workgroups (one per CU)
constexpr int kCuRep = 4;          // decode_cu.hip: replicas of the counter
constexpr int kCuParts = 16;       // decode_cu.hip: parts of the counter

// Fills the work decomposition of the fused decode kernel for a shape and
// returns its grid size (workgroups).
int decode_grid(FusedArgs& a);

struct RouterArgs {
    const uint16_t* router;      // [E][h] bf16
    const float* bias;           // [E] or null
    const void* x;               // [T][h]
    int32_t x_bf16;
    int32_t T, E, h, K, norm;
    float* logits;               // [T][E] scratch
    int32_t* idx;                // [T][K]
    float* w;                    // [T][K]
    int32_t* user_idx;           // optional copies
    float* user_w;
    float* user_logits;
    uint32_t* counters;          // [T] zero-initialised, self-resetting
    _Float16* xq;                // optional: the prefill's f16 copy of x [T][h] and
    float* xinv;                 // its per-token 2^-e (PrefillArgs xq / xinv)
};

// Per-expert prefill copy of an expert block, made on the device at upload
// (launch_pf_tile_copy): the operand tiles of the prefill GEMMs stored as the
// LDS images the GEMM copies, one contiguous chunk per (M-tile, 64-column
// k-block):
//   gate/up: mg = ceil(I/128) M-tiles x h/64 blocks, rows 0..127 of a tile
//            gate rows, 128..255 the same up rows;
//   down:    md = ceil(h/256) M-tiles x I/64 blocks, 256 down rows a tile;
//   chunk  = A [256 rows][2 units of 16 bytes]: unit kh (the row's packed
//            columns 32 kh .. 32 kh + 31 of the block) of tile row r at
//            position kh ^ ((r >> 2) & 1) ^ ((r >> 3) & 1); rows past the
//            matrix zero
//          + S [2 groups at gs 32, else 1][256 rows]: u32 f16(s * 2^(20-k))
//            | f16(b * 2^-k) << 16 of the block's group(s) (at gs 128 the
//            group the block lies in);
// then one int8 k per row: gate [mg*128], up [mg*128], down [md*256] (zero
// past the matrix).  k, the smallest k >= 0 that keeps s * 2^(24 - k) and
// every dequantised weight (15|s| + |b|) * 2^-k within f16 range, is undone
// on the row's accumulator (x 2^k, exact).
struct PfTileLayout {
    int mg, md, kbg, kbd;        // M-tiles and k-blocks of gate/up and of down
    uint64_t chunk, gu, dn, kg, ku, kd, bytes;
    M1MOE_HD PfTileLayout(int h, int I, int gs) {
        mg = (I + 127) / 128;
        md = (h + 255) / 256;
        kbg = h / 64;
        kbd = I / 64;
        chunk = 256 * 32 + (gs == 32 ? 2 : 1) * 256 * 4;
        gu = 0;
        dn = (uint64_t)mg * kbg * chunk;
        kg = dn + (uint64_t)md * kbd * chunk;
        ku = kg + (uint64_t)mg * 128;
        kd = ku + (uint64_t)mg * 128;
        bytes = (kd + (uint64_t)md * 256 + 255) / 256 * 256;
    }
};

// Prefill grouping results: a sorted (token, slot) pair, and an N-tile of
// one expert's pairs (np = 0: no tile).
struct alignas(8) PfPair {
    int32_t tok;
    float inv;                   // the token's 2^-e_t
};
struct alignas(16) PfTile {
    int32_t e, p0, np, pad;      // expert, first sorted position, pairs
};

// Arguments of the prefill kernels (T tokens through one layer).
struct PrefillArgs {
    const uint8_t* layer_base;   // first expert block of the layer
    uint64_t expert_bytes;
    const uint8_t* pft_base;     // the layer's first prefill copy (PfTileLayout)
    uint64_t pft_bytes;          // bytes per expert of those copies
    const void* x;               // [T][h] f32 or bf16
    int32_t x_bf16;
    const float* residual;       // [T][h] or null
    float* out;                  // [T][h]
    const int32_t* idx;          // [T][K] routing
    const float* w;              // [T][K]
    int32_t T, h, E, K, I, gs;
    // scratch
    _Float16* xq;                // [T][h] x * 2^e_t in f16
    float* xinv;                 // [T] 2^-e_t
    int32_t* pos;                // [T*K] sorted position of pair (t, k)
    PfPair* sorted_tok;          // [T*K] per sorted position
    int32_t* expert_off;         // [E+1] first sorted position of each expert
    int32_t* tile_off;           // [E+1] first N-tile of each expert
    PfTile* tile_desc;           // [T*K/kPfTN + E + 1] per N-tile (np = 0 past the last):
                                 // tiles of more than kPfTN / 2 pairs first
    int32_t cus;                 // compute units of the device
    _Float16* act;               // [T*K][I] silu(gate)*up per sorted pair (per block: act_exp)
    float* y;                    // [T*K][h] expert outputs per sorted pair
    uint8_t* act_exp;            // [T*K][I/32] e >= 0 of each 32-value block: act held act * 2^-e
    uint32_t* act_flag;          // [kPfFlagWords + ceil(T*K/32)]: word 0 is 1 when some e > 0
                                 // (the down GEMM then reads act_exp); words 32 .. 32 * 18 - 1
                                 // the down GEMM's barrier; then a bit per pair whose act
                                 // row its prologue rewrote
    uint32_t* err;               // sticky device error flag
};

// Prefill scratch buffers (in the order of PrefillArgs: xq, xinv, pos,
// sorted_tok, expert_off, tile_off, tile_desc, act, y, act_exp, act_flag).
constexpr int kPfBufs = 11;

constexpr int kPfTN = 128;  // prefill GEMM: (token, slot) pairs per workgroup tile
constexpr int kPfSpinLimit = 1 << 20;   // bounded wait of the down GEMM's rare grid barrier
constexpr int kPfFlagWords = 32 * 18;    // act_flag words before the rewritten-row bitmap

// m1moe_moe_prefill_noalloc: bytes of the per-GPU static scratch (scratch.hip)
// that holds its prefill buffers.  64 MiB: 776 tokens at hidden 2048,
// 8 x 1024 experts, 676 at hidden 4096, 2 x 14336.
constexpr uint64_t kStaticScratchBytes = 64ull << 20;
// Device address of this GPU's static scratch; `device` must be current.
// Looks it up on the first call per device and returns the kept address
// after that.  Returns a hipError_t as int.
int static_scratch_attach(int device, uint8_t** out);

// launchers (defined next to their kernels); return a hipError_t as int
int launch_router_topk(const RouterArgs& a, void* stream);
int launch_moe_decode(const FusedArgs& a, void* stream);
// The one-workgroup-per-CU decode kernel: the shapes it takes (hidden 2048,
// K * I = 8192 or 16384, I = 1024 or 2048, K <= 8 dividing 8) and its
// launcher (all kCuWorkgroups workgroups must be resident together).
bool decode_cu_fits(int h, int E, int K, int I, int gs);
int launch_moe_decode_cu(const FusedArgs& a, void* stream);
// Workgroups of the per-CU kernel of this shape one CU of the current device
// holds (the occupancy query; the smaller of the bf16 and f32 input
// variants).  Returns a hipError_t as int.
int decode_cu_blocks_per_cu(int h, int K, int I, int gs, int* blocks);
// The decode kernel of a shape (fits: decode_cu_fits) on a device of `cus`
// CUs holding `blocks` per-CU workgroups each: 1 = moe_decode_cu_kernel
// (hidden 2048), 2 = moe_decode_cuw_kernel (hidden 4096), when all
// kCuWorkgroups workgroups fit at once; else 0 = moe_decode_kernel.
inline int decode_kernel_choice(bool fits, int h, int cus, int blocks) {
    if (!fits || (int64_t)cus * blocks < kCuWorkgroups) return 0;
    return h == 2048 ? 1 : 2;
}
// Bytes of one expert's repacked block (decode_cu.hip) and the launch that
// builds a layer's repacked blocks from its canonical ones.
uint64_t decode_copy_bytes(int h, int I, int gs);
int launch_decode_copy(const uint8_t* layer, uint64_t expert_bytes, uint8_t* dst, int E, int h,
                       int I, int gs, void* stream);
int launch_prefill(const PrefillArgs& a, void* stream);
// Writes the PfTileLayout copies of E experts (layer image at `layer`) to
// dst; a non-finite scale or bias raises device error flag 8.
int launch_pf_tile_copy(const uint8_t* layer, uint64_t expert_bytes, uint8_t* dst, int E, int h,
                        int I, int gs, uint32_t* err, void* stream);
int launch_dequant(const uint8_t* expert_base, const ProjView& p, int32_t gs, float* out,
                   void* stream);

// ---- dense decoder step (dense.hip) ----

// One weight segment of a bf16 matvec: y[r] = W[r] . x (+ res[r]).
struct MvSeg {
    const uint16_t* w;   // [rows][cols] bf16
    float* y;            // [rows]
    const float* res;    // [rows] or null
    int32_t rows;
};

// y = W x over up to three segments sharing the input x.
//   input:    x (f32), or row *token (or token[*pos] with seq_cap > 0) of the
//             bf16 table `embed` (a token outside [0, vocab) embeds row 0
//             and sets error flag 16); x_copy: workgroup 0 stores the f32
//             input there; norm_w: the input is RMS-normalised first,
//             x * rsqrt(mean(x^2) + eps) * w (the input is staged in LDS)
//   outputs:  ssq_out non-null: each workgroup stores the sum of squares of
//             its output rows (after the residual) at ssq_out[workgroup];
//             counter non-null (argmax): the last workgroup to finish reduces
//             the per-workgroup best (am_val, am_idx) to the greedy token of
//             segment 0's output and advances *pos; the counter is back at 0
//             when the kernel ends.
struct MvArgs {
    MvSeg seg[3];
    const float* x;
    int32_t rows, cols;
    const uint16_t* embed;
    const int32_t* token;
    int32_t seq_cap;
    int32_t vocab;
    float* x_copy;
    const uint16_t* norm_w;
    float eps;
    float* ssq_out;              // [workgroups]
    uint32_t* counter;           // [kCountWords] (dense.hip count_out)
    float* am_val;               // [workgroups]
    int32_t* am_idx;             // [workgroups]
    int32_t* tok_out;            // single mode: *tok_out; sequence mode: tok_out[p + 1]
    int32_t n_prompt;
    int32_t* pos;                // device position (read for the embedding, advanced by argmax)
    int32_t max_seq;
    uint32_t* err;
    // x given as decode-attention partials when the attention launch left
    // their merge to this one (attention_defers): attn_part is that launch's
    // partial buffer, the other fields its AttnArgs geometry; null: x given
    const float* attn_part;
    int32_t attn_heads, attn_qh, attn_hd, attn_chunk, attn_nch;
};

// Decode attention of one query position.  Workgroup (g, c): q heads
// g*qh .. g*qh+qh-1 (one kv head) over positions c*chunk .. (c+1)*chunk - 1
// (chunk = attention_chunk(max_seq, groups, cus): a multiple of 64 or 65 ..
// kAttnWideChunk, at most kAttnMaxChunks workgroups per kv head).
//   fused = 1: q, k_new, v_new are the raw projections of the current token;
//     q and k get the per-head RMSNorm (q_norm/k_norm non-null) and RoPE at
//     p = *pos, the new k/v row is stored at cache row p (flag 32 and no
//     store when p >= max_seq), positions 0..p attended;
//   fused = 0: q final, positions 0..seq_len-1 all from the caches.
// The last workgroup of each group merges the chunks into out; counters
// ([groups]) are back at 0 when the kernel ends.
struct AttnArgs {
    int32_t fused;
    const float* q;              // [num_heads][head_dim]
    const float* k_new;          // [num_kv_heads][head_dim] (fused)
    const float* v_new;
    const uint16_t* q_norm;      // [head_dim] or null
    const uint16_t* k_norm;
    float* kcache;               // row (position pp, kv head h) at pp * kv_pos + h * kv_head
    float* vcache;
    int64_t kv_pos, kv_head;     // floats between positions and between kv heads
    float* out;                  // [num_heads][head_dim]
    float* partial;              // [groups][chunks][qh][head_dim + 2]
    uint32_t* counters;          // [groups]
    const int32_t* pos;
    uint32_t* err;
    int32_t seq_len;             // fused = 0
    int32_t max_seq;             // cache rows (fused) / seq_len
    int32_t num_heads, num_kv_heads, hpkv, head_dim, qh;
    int32_t chunk;               // positions per workgroup
    float scale, rope_theta, eps;
    // fused only: for 2 .. kAttnDeferChunks active chunks and num_heads x chunks
    // <= kAttnDeferHeadChunks, write the partials and leave their merge to the
    // next launch (the o_proj matvec, which stages them as its input)
    int32_t defer;
    // 1 when the whole grid fits on the device at once (set by the launcher
    // from the occupancy query): the partials are stored as (launch number,
    // value) pairs in `partial` read as u64, and every workgroup with
    // positions merges a share of its group's outputs, waiting for the
    // current launch number instead of a completion count.  gen holds the
    // launch number, fin counts finished workgroups (the last one advances
    // gen and puts fin back to 0).
    int32_t sync_merge;
    const float* rope;           // fused: [max_seq][head_dim / 2] (cos, sin) table, or null
    uint32_t* gen;
    uint32_t* fin;               // [kCountWords] (dense.hip count_out)
    int32_t cus;                 // compute units of the device
    int32_t spin_limit;
    // optional: bytes the next launch streams (the decoder's o_proj weights),
    // read by a second plane of workgroups (grid z = 1) into the caches while
    // the attention runs: pf_units pieces of pf_unit bytes (piece b is what
    // workgroup b of that launch reads, so it goes to that XCD's L2), pf_bytes
    // in all; null: no second plane
    const uint8_t* pf;
    int64_t pf_unit, pf_bytes;
    int32_t pf_units;
};

constexpr int kAttnChunk = 64;   // positions per attention sub-chunk
constexpr int kAttnPfPlanes = 1;  // prefetch planes of an attention grid (AttnArgs::pf)
constexpr int kAttnWideChunk = 80;   // chunks of 65 .. this many positions: one wide sub-chunk
constexpr int kAttnMaxQH = 8;    // q heads per attention workgroup
constexpr int kAttnMaxChunks = 64;   // workgroups per kv head
constexpr int kAttnDeferChunks = 8;        // deferred merge: at most this many chunks
constexpr int kAttnDeferHeadChunks = 64;   // and heads x chunks (the partials staged per matvec workgroup)
constexpr int kMvStageMax = 8192;   // largest staged (normalised / embedded) input, floats

// ---- decoder prefill (prefill_dense.hip) ----

// C[M][N] = A[M][K] W[N][K]^T (+ R[M][N]); A f32 (row stride lda, lda % 4 ==
// 0), W bf16 row-major, C and R with row stride ldc; K % 32 == 0.
struct GemmArgs {
    const float* A;
    int32_t lda;
    const uint16_t* W;
    const float* R;
    float* C;
    int32_t ldc;
    int32_t M, N, K;
    // split-K workspace ([S][M][N] f32 partials, summed in order s = 0 .. S-1)
    // or null; with it a GEMM whose tiles leave the CUs idle splits its k range
    float* part;
    int32_t splits;              // set by launch_gemm
    // optional second and third weight segments: rows [n1, n2) are rows
    // 0 .. of W1, rows [n2, N) rows 0 .. of W2 (q, k and v in one launch);
    // null W1: every row from W.  Needs K % 64 == 0.
    const uint16_t* W1;
    const uint16_t* W2;
    int32_t n1, n2;
    // optional RMSNorm of each output row (ldc == N): norm_out[m] =
    // C[m] * rsqrt(mean(C[m]^2) + norm_eps) * norm_w (bf16), made by the
    // split-K sum when there is one, else by a row-norm launch
    const uint16_t* norm_w;
    float* norm_out;
    float norm_eps;
};
constexpr int64_t kGemmPartFloats = 768LL * 64 * 64;  // the workspace launch_gemm may use

// The T prompt tokens of a decoder prefill at positions *pos .. *pos + T - 1.
struct PfDenseArgs {
    const int32_t* tokens;       // [T]
    const uint16_t* embed;       // [vocab][h]
    float* res;                  // [T][h] residual stream
    float* qkv;                  // [T][ldqkv]: q | k | v
    float* attn;                 // [T][qd]
    const uint16_t* q_norm;      // [head_dim] or null
    const uint16_t* k_norm;
    float* kcache;               // this layer's [max_seq][kvd]
    float* vcache;
    const int32_t* pos;
    uint32_t* err;
    int32_t T, vocab, h, ldqkv, qd, kvd;
    int32_t num_heads, num_kv_heads, hpkv, head_dim, max_seq;
    float scale, rope_theta, eps;
};

int launch_pf_embed(const PfDenseArgs& a, void* stream);
int launch_rmsnorm_rows(const float* x, const uint16_t* w, float* out, int rows, int n, float eps,
                        void* stream);
int launch_gemm(const GemmArgs& g, void* stream);
int launch_pf_rope_kv(const PfDenseArgs& a, void* stream);
int launch_pf_attention(const PfDenseArgs& a, void* stream);
int launch_advance_pos(int32_t* pos, int32_t by, int32_t max_seq, void* stream);

int launch_set_i32(int32_t* p, int32_t v, void* stream);
int launch_rmsnorm(const float* x, const uint16_t* w, float* out, int n, float eps, void* stream);
// Workgroups of a matvec launch (the size of am_val / am_idx).
int matvec_workgroups(int rows);
int matvec_rows_per_workgroup(int rows);
int launch_matvec_bf16(const MvArgs& a, void* stream);
// q heads per attention workgroup (0: unsupported hpkv).
int attention_qh(int hpkv);
// Positions per attention workgroup for a cache of max_positions, groups
// (num_heads / qh) workgroups per chunk and cus compute units: a multiple of
// 64, or 65 .. kAttnWideChunk; at most kAttnMaxChunks chunks.
int attention_chunk(int max_positions, int groups, int cus);
// The whole attention grid of `a` fits on the device at once (a.cus CUs, the
// occupancy of the kernel instance it launches): the synchronous merge may
// be used.
bool attention_grid_fits(const AttnArgs& a);
// The RoPE table of attn_kernel: [max_seq][head_dim / 2] (cos, sin) pairs.
int launch_rope_table(float* table, int max_seq, int head_dim, float theta, void* stream);
constexpr int32_t kAttnSpinLimit = 1 << 20;  // bounded waits of the synchronous merge (~1 s)
constexpr int kCountWords = 32 * 9;   // a two-level completion counter (dense.hip count_out)
// floats of the partials buffer (room for the u64 pairs of the synchronous merge)
int attention_partial_floats(int num_heads, int head_dim, int max_positions);
int launch_attention(const AttnArgs& a, void* stream);
// Greedy token of x[0..n) to *out (ties to the lower index; x[0] NaN gives 0).
int launch_argmax(const float* x, int n, int32_t* out, void* stream);

}  // namespace m1moe
