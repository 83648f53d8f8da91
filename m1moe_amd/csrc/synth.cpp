// synth.cpp — seeded, counter-based synthetic inputs for the MoE block.
//
// Value i of tensor `tensor_id` under `seed` depends only on (seed,
// tensor_id, i): a SplitMix64 finaliser over a Weyl sequence keyed by the
// pair.  Normals come from Box-Muller in f64 over two consecutive draws.
// bf16 rounding is round-to-nearest-even of the f32 value, the rounding the
// reference's converter applies (scripts/extract_olmoe.py:104-111).
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "m1moe_hip.h"
#include "internal.hpp"

namespace {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

inline uint64_t fmix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t stream_key(uint64_t seed, uint64_t tensor_id) {
    return fmix64(seed * kGamma ^ fmix64(tensor_id + kGamma));
}

inline uint64_t draw(uint64_t key, uint64_t i) { return fmix64(key + (i + 1) * kGamma); }

inline float normal_at(uint64_t key, uint64_t i, float sigma) {
    const double u1 = ((double)(draw(key, 2 * i) >> 11) + 0.5) * 0x1.0p-53;
    const double u2 = (double)(draw(key, 2 * i + 1) >> 11) * 0x1.0p-53;
    const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
    return (float)(z * (double)sigma);
}

inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void fill_bf16(uint64_t key, uint64_t n, float sigma, bool absval, uint16_t* out) {
    for (uint64_t i = 0; i < n; ++i) {
        float v = normal_at(key, i, sigma);
        if (absval) v = std::fabs(v);
        out[i] = f32_to_bf16_rne(v);
    }
}

// Runs body(i0, i1) over [0, n) on up to 16 threads (values depend only on
// the index, so the split does not change them).
template <class F>
void parallel_range(uint64_t n, F body) {
    constexpr uint64_t kMinPerThread = 1u << 20;
    unsigned hw = std::thread::hardware_concurrency();
    uint64_t nt = hw ? hw : 1;
    if (nt > 16) nt = 16;
    if (nt > n / kMinPerThread) nt = n / kMinPerThread;
    if (nt <= 1) {
        body((uint64_t)0, n);
        return;
    }
    std::vector<std::thread> pool;
    for (uint64_t t = 1; t < nt; ++t) pool.emplace_back(body, n * t / nt, n * (t + 1) / nt);
    body((uint64_t)0, n / nt);
    for (auto& th : pool) th.join();
}

void fill_words(uint64_t key, uint64_t n, uint32_t* out) {
    // every nibble of a uniform 32-bit word is uniform in 0..15
    for (uint64_t i = 0; i < n; ++i) out[i] = (uint32_t)(draw(key, i) >> 32);
}

// tensor ids of the sub-blocks of expert (layer, expert): kind 0 = packed
// words, 1 = scales, 2 = biases; proj 0 = gate, 1 = up, 2 = down
inline uint64_t expert_tensor_id(int32_t layer, int32_t expert, int proj, int kind) {
    return (1ull << 62) | ((uint64_t)(uint32_t)layer << 24) |
           ((uint64_t)(uint32_t)expert << 8) | ((uint64_t)proj << 4) | (uint64_t)kind;
}

}  // namespace

extern "C" int32_t m1moe_synth_normal_bf16(uint64_t seed, uint64_t tensor_id, uint64_t n,
                                           float sigma, int32_t absval, uint16_t* out) {
    if (!out && n) return m1moe::fail(M1MOE_ERR_INVALID, "synth_normal_bf16: null output");
    const uint64_t key = stream_key(seed, tensor_id);
    parallel_range(n, [&](uint64_t i0, uint64_t i1) {
        for (uint64_t i = i0; i < i1; ++i) {
            float v = normal_at(key, i, sigma);
            if (absval) v = std::fabs(v);
            out[i] = f32_to_bf16_rne(v);
        }
    });
    return M1MOE_OK;
}

extern "C" int32_t m1moe_synth_normal_f32(uint64_t seed, uint64_t tensor_id, uint64_t n,
                                          float sigma, float* out) {
    if (!out && n) return m1moe::fail(M1MOE_ERR_INVALID, "synth_normal_f32: null output");
    const uint64_t key = stream_key(seed, tensor_id);
    parallel_range(n, [&](uint64_t i0, uint64_t i1) {
        for (uint64_t i = i0; i < i1; ++i) out[i] = normal_at(key, i, sigma);
    });
    return M1MOE_OK;
}

extern "C" int32_t m1moe_synth_layer_image(const m1moe_moe_shape* shape, uint64_t seed,
                                           int32_t layer, float scale_sigma, float bias_sigma,
                                           void* out, uint64_t bytes, int32_t threads) {
    int32_t rc = m1moe_check_shape(shape);
    if (rc) return rc;
    if (!out) return m1moe::fail(M1MOE_ERR_INVALID, "synth_layer_image: null output");
    const m1moe::Geom g = m1moe::make_geom(*shape);
    const uint64_t want = (uint64_t)shape->num_experts * g.expert_bytes;
    if (bytes != want)
        return m1moe::fail(M1MOE_ERR_INVALID,
                           "synth_layer_image: %llu bytes given, layer image is %llu",
                           (unsigned long long)bytes, (unsigned long long)want);
    const int32_t E = shape->num_experts;
    uint8_t* base = static_cast<uint8_t*>(out);
    auto work = [&](int32_t e0, int32_t e1) {
        for (int32_t e = e0; e < e1; ++e) {
            uint8_t* blk = base + (uint64_t)e * g.expert_bytes;
            for (int proj = 0; proj < 3; ++proj) {
                const uint64_t rows = (uint64_t)g.rows(proj), cols = (uint64_t)g.cols(proj);
                const uint64_t nw = rows * cols / 8, nsb = rows * (cols / (uint64_t)g.gs);
                fill_words(stream_key(seed, expert_tensor_id(layer, e, proj, 0)), nw,
                           reinterpret_cast<uint32_t*>(blk + g.off[3 * proj + 0]));
                fill_bf16(stream_key(seed, expert_tensor_id(layer, e, proj, 1)), nsb,
                          scale_sigma, true, reinterpret_cast<uint16_t*>(blk + g.off[3 * proj + 1]));
                fill_bf16(stream_key(seed, expert_tensor_id(layer, e, proj, 2)), nsb,
                          bias_sigma, false, reinterpret_cast<uint16_t*>(blk + g.off[3 * proj + 2]));
            }
        }
    };
    int32_t nt = threads < 1 ? 1 : threads;
    if (nt > E) nt = E;
    std::vector<std::thread> pool;
    for (int32_t t = 1; t < nt; ++t)
        pool.emplace_back(work, (int32_t)((int64_t)E * t / nt), (int32_t)((int64_t)E * (t + 1) / nt));
    work(0, (int32_t)((int64_t)E / nt));
    for (auto& th : pool) th.join();
    return M1MOE_OK;
}
