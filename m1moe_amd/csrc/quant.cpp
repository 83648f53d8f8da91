// quant.cpp — the converters' 4-bit group quantizer, on the host.
//
// Restates quantize_4bit and f32_to_bf16 of the reference's converters
// (scripts/extract_olmoe.py:104-111 and :116-159; scripts/extract_mixtral.py
// carries the same two functions) so that a real checkpoint's f32/bf16/f16
// expert matrices become the layer_NN.bin blocks the library uploads.  Per
// row and group of `group_size` consecutive columns, all in f32:
//   lo = min, hi = max, s = (hi - lo) / 15, s = 1 where s == 0,
//   nibble = clamp(round_half_even((w - lo) / s), 0, 15),
//   stored: nibbles 8 per u32 (column 8w + j in bits 4j..4j+3), bf16(s),
//   bf16(lo), bf16 = round-to-nearest-even of the f32 bits (0x7FFF + lsb).
// The nibbles come from the f32 scale, not from its bf16 rounding, as in the
// reference.  Non-finite weights are refused (the reference would write
// meaningless groups for them).  Offline work: no device is touched.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "internal.hpp"
#include "m1moe_hip.h"

using namespace m1moe;

namespace {

inline uint16_t bf16_rne(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// Rows [r0, r1) of one matrix; returns the first row holding a non-finite
// value, or -1.
int64_t quantize_rows(const float* w, int64_t r0, int64_t r1, int64_t cols, int32_t gs,
                      uint32_t* packed, uint16_t* scales, uint16_t* biases) {
    const int64_t ng = cols / gs;
    std::vector<uint8_t> q((size_t)cols);
    for (int64_t r = r0; r < r1; ++r) {
        const float* row = w + r * cols;
        for (int64_t g = 0; g < ng; ++g) {
            const float* v = row + g * gs;
            // min, max and a finiteness check in eight independent lanes (so
            // the loop vectorizes): x * 0 is 0 for a finite x and NaN for an
            // infinite or NaN one, so chk ends 0 or NaN
            float lo8[8], hi8[8], chk8[8];
            for (int j = 0; j < 8; ++j) lo8[j] = hi8[j] = v[0], chk8[j] = 0.f;
            const int32_t g8 = gs - gs % 8;
            for (int32_t i = 0; i < g8; i += 8)
                for (int j = 0; j < 8; ++j) {
                    const float x = v[i + j];
                    lo8[j] = x < lo8[j] ? x : lo8[j];
                    hi8[j] = x > hi8[j] ? x : hi8[j];
                    chk8[j] += x * 0.f;
                }
            for (int32_t i = g8; i < gs; ++i) {
                lo8[0] = v[i] < lo8[0] ? v[i] : lo8[0];
                hi8[0] = v[i] > hi8[0] ? v[i] : hi8[0];
                chk8[0] += v[i] * 0.f;
            }
            float lo = lo8[0], hi = hi8[0], chk = chk8[0];
            for (int j = 1; j < 8; ++j) {
                lo = lo8[j] < lo ? lo8[j] : lo;
                hi = hi8[j] > hi ? hi8[j] : hi;
                chk += chk8[j];
            }
            if (!(chk == 0.f)) return r;
            float s = (hi - lo) / 15.0f;
            if (s == 0.0f) s = 1.0f;
            uint8_t* qg = q.data() + g * gs;
            for (int32_t i = 0; i < gs; ++i) {
                // t >= 0; adding and taking away 1.5 * 2^23 rounds it to an
                // integer half to even (the default rounding mode) for t < 2^22,
                // as nearbyint; larger values clamp to 15 either way
                float t = (v[i] - lo) / s;
                t = (t + 12582912.0f) - 12582912.0f;
                t = t > 0.f ? t : 0.f;  // (NaN from an overflowed range: 0)
                t = t < 15.f ? t : 15.f;
                qg[i] = (uint8_t)(int32_t)t;
            }
            scales[r * ng + g] = bf16_rne(s);
            biases[r * ng + g] = bf16_rne(lo);
        }
        uint32_t* pw = packed + r * (cols / 8);
        for (int64_t c = 0; c < cols / 8; ++c) {
            uint32_t word = 0;
            for (int j = 0; j < 8; ++j) word |= (uint32_t)q[(size_t)(8 * c + j)] << (4 * j);
            pw[c] = word;
        }
    }
    return -1;
}

// Rows split over up to `threads` host threads (the result does not depend
// on the split).  Returns the first bad row found, or -1.
int64_t quantize_matrix(const float* w, int64_t rows, int64_t cols, int32_t gs, uint32_t* packed,
                        uint16_t* scales, uint16_t* biases, int32_t threads) {
    int64_t nt = threads < 1 ? 1 : threads;
    if (nt > 64) nt = 64;
    if (nt > rows) nt = rows;
    if (nt <= 1) return quantize_rows(w, 0, rows, cols, gs, packed, scales, biases);
    std::vector<int64_t> bad((size_t)nt, -1);
    std::vector<std::thread> pool;
    for (int64_t t = 0; t < nt; ++t)
        pool.emplace_back([&, t] {
            bad[(size_t)t] = quantize_rows(w, rows * t / nt, rows * (t + 1) / nt, cols, gs, packed,
                                           scales, biases);
        });
    for (auto& th : pool) th.join();
    for (int64_t b : bad)
        if (b >= 0) return b;
    return -1;
}

int32_t check_matrix(int64_t rows, int64_t cols, int32_t gs) {
    if (rows < 0 || cols <= 0 || gs <= 0)
        return fail(M1MOE_ERR_INVALID, "quantize_4bit: rows %lld, cols %lld, group_size %d",
                    (long long)rows, (long long)cols, gs);
    // extract_olmoe.py:130-131
    if (cols % gs)
        return fail(M1MOE_ERR_INVALID, "quantize_4bit: cols %lld not divisible by group_size %d",
                    (long long)cols, gs);
    if (cols % 8)
        return fail(M1MOE_ERR_INVALID, "quantize_4bit: cols %lld not divisible by 8",
                    (long long)cols);
    return M1MOE_OK;
}

}  // namespace

extern "C" {

int32_t m1moe_f32_to_bf16(const float* x, uint64_t n, uint16_t* out) {
    if (n && (!x || !out)) return fail(M1MOE_ERR_INVALID, "f32_to_bf16: null pointer");
    for (uint64_t i = 0; i < n; ++i) out[i] = bf16_rne(x[i]);
    return M1MOE_OK;
}

int32_t m1moe_quantize_4bit(const float* w, int64_t rows, int64_t cols, int32_t group_size,
                            uint32_t* packed, uint16_t* scales, uint16_t* biases,
                            int32_t threads) {
    int32_t rc = check_matrix(rows, cols, group_size);
    if (rc) return rc;
    if (rows && (!w || !packed || !scales || !biases))
        return fail(M1MOE_ERR_INVALID, "quantize_4bit: null pointer");
    const int64_t bad = quantize_matrix(w, rows, cols, group_size, packed, scales, biases, threads);
    if (bad >= 0)
        return fail(M1MOE_ERR_INVALID, "quantize_4bit: row %lld holds a non-finite value",
                    (long long)bad);
    return M1MOE_OK;
}

int32_t m1moe_quantize_expert(const m1moe_moe_shape* shape, const float* gate, const float* up,
                              const float* down, void* block, uint64_t block_bytes,
                              int32_t threads) {
    int32_t rc = m1moe_check_shape(shape);
    if (rc) return rc;
    if (!gate || !up || !down || !block)
        return fail(M1MOE_ERR_INVALID, "quantize_expert: null pointer");
    const Geom g = make_geom(*shape);
    if (block_bytes != g.expert_bytes)
        return fail(M1MOE_ERR_INVALID, "quantize_expert: %llu bytes given, an expert block is %llu",
                    (unsigned long long)block_bytes, (unsigned long long)g.expert_bytes);
    uint8_t* base = static_cast<uint8_t*>(block);
    const float* src[3] = {gate, up, down};
    static const char* names[3] = {"gate", "up", "down"};
    // extract_olmoe.py:322-338: gate_proj, up_proj, down_proj, each W|S|B
    for (int proj = 0; proj < 3; ++proj) {
        const int64_t bad = quantize_matrix(
            src[proj], g.rows(proj), g.cols(proj), g.gs,
            reinterpret_cast<uint32_t*>(base + g.off[3 * proj + 0]),
            reinterpret_cast<uint16_t*>(base + g.off[3 * proj + 1]),
            reinterpret_cast<uint16_t*>(base + g.off[3 * proj + 2]), threads);
        if (bad >= 0)
            return fail(M1MOE_ERR_INVALID, "quantize_expert: %s row %lld holds a non-finite value",
                        names[proj], (long long)bad);
    }
    return M1MOE_OK;
}

}  // extern "C"
