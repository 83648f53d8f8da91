// internal.hpp — shared host-side definitions of libm1moe_hip.so.
#pragma once

#include <cstdint>

#include "m1moe_hip.h"

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

// Kernel-side view of one projection: packed words, scales, biases are
// reached from the expert block base by the byte offsets below.
struct ProjView {
    uint64_t w_off, s_off, b_off;
    int32_t rows, cols;
};

// Arguments shared by the decode kernels.
struct DecodeArgs {
    const uint8_t* layer_base;   // first expert block of the layer
    uint64_t expert_bytes;
    int32_t h, E, K, I, gs;
    const void* x;               // [h] f32 or bf16
    int32_t x_bf16;
    const int32_t* topk_idx;     // [K]
    const float* topk_w;         // [K]
    const float* residual;       // [h] or null
    float* out;                  // [h]
    float* act;                  // [K][I] scratch
    uint32_t* err;               // sticky device error flag
    ProjView gate, up, down;
};

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
};

// launchers (defined next to their kernels); return a hipError_t as int
int launch_router_topk(const RouterArgs& a, void* stream);
int launch_decode_gate_up(const DecodeArgs& a, void* stream);
int launch_decode_down_combine(const DecodeArgs& a, void* stream);
int launch_dequant(const uint8_t* expert_base, const ProjView& p, int32_t gs, float* out,
                   void* stream);

}  // namespace m1moe
