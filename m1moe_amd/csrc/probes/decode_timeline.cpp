// decode_timeline — where the time of one per-CU MoE decode launch goes
// (moe_decode_cu_kernel at hidden 2048, moe_decode_cuw_kernel at 4096).
//
// Not part of the library.  Built by `make -C m1moe_amd/csrc probes` into
// m1moe_amd/_probes/decode_timeline, linked against the tracing build of the
// library (m1moe_amd/_probes/libm1moe_hip_trace.so: decode_cu.hip compiled
// with -DM1MOE_DECODE_TRACE, every other object as in libm1moe_hip.so).  The
// tracing kernel stamps s_memrealtime (100 MHz, one clock for the whole GPU)
// into LDS at the phase boundaries below and writes the stamps of each
// workgroup at its end to the buffer set by m1moe_trace_decode().
//
// Workload: cfg0, the OLMoE-shaped layer (h 2048, 64 experts, top-8, I 1024,
// 4-bit group 64), or cfg2, the Mixtral-shaped one (h 4096, 8 experts, top-2,
// I 14336), with R synthetic replicas, one token per replica, the R launches
// captured in one graph as in bench.py.  Prints the launch time of the
// tracing build with no buffer set, then per phase the spread over all
// workgroups of 5 traced replays (the graph's last replica), in us from the
// first workgroup's start.
//
// usage: decode_timeline [bf16|f32] [R] [cfg0|cfg2]
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "m1moe_hip.h"

extern "C" int32_t m1moe_trace_decode(void* dev_buf);

#define HIPCHK(x)                                                                      \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));             \
            exit(1);                                                                   \
        }                                                                              \
    } while (0)
#define M1CHK(x)                                                                       \
    do {                                                                               \
        int32_t r_ = (x);                                                              \
        if (r_ != M1MOE_OK) {                                                          \
            fprintf(stderr, "%s failed (%d): %s\n", #x, r_, m1moe_last_error());       \
            exit(1);                                                                   \
        }                                                                              \
    } while (0)

int main(int argc, char** argv) {
    const bool f32 = argc > 1 && strcmp(argv[1], "f32") == 0;
    const bool mixtral = argc > 3 && strcmp(argv[3], "cfg2") == 0;
    const int R = argc > 2 ? atoi(argv[2]) : (mixtral ? 8 : 38);
    m1moe_moe_shape sh = mixtral ? m1moe_moe_shape{4096, 8, 2, 14336, 64, R, 0}
                                 : m1moe_moe_shape{2048, 64, 8, 1024, 64, R, 0};
    m1moe_ctx_t ctx;
    M1CHK(m1moe_create(0, &sh, &ctx));
    uint64_t eb;
    M1CHK(m1moe_expert_bytes(&sh, &eb));
    const int h = sh.hidden;
    {
        std::vector<uint8_t> img((size_t)sh.num_experts * eb);
        std::vector<uint16_t> router((size_t)sh.num_experts * h);
        for (int r = 0; r < R; ++r) {
            M1CHK(m1moe_synth_layer_image(&sh, 77, r, 0.02f, 0.01f, img.data(), img.size(), 8));
            M1CHK(m1moe_upload_layer_experts(ctx, r, img.data(), img.size()));
            M1CHK(m1moe_synth_normal_bf16(77, 1000 + r, router.size(), 0.02f, 0, router.data()));
            M1CHK(m1moe_upload_router(ctx, r, router.data(), router.size()));
        }
    }
    void *dx, *dx32, *dres, *dy;
    M1CHK(m1moe_alloc(ctx, (uint64_t)h * 2 * R, &dx));
    M1CHK(m1moe_alloc(ctx, (uint64_t)h * 4 * R, &dx32));
    M1CHK(m1moe_alloc(ctx, (uint64_t)h * 4 * R, &dres));
    M1CHK(m1moe_alloc(ctx, (uint64_t)h * 4 * R, &dy));
    {
        std::vector<uint16_t> hx((size_t)h * R);
        M1CHK(m1moe_synth_normal_bf16(5, 5, hx.size(), 1.f, 0, hx.data()));
        std::vector<float> fx(hx.size());
        for (size_t i = 0; i < hx.size(); ++i) {
            const uint32_t u = (uint32_t)hx[i] << 16;
            memcpy(&fx[i], &u, 4);
        }
        M1CHK(m1moe_copy_h2d(ctx, dx, hx.data(), hx.size() * 2));
        M1CHK(m1moe_copy_h2d(ctx, dx32, fx.data(), fx.size() * 4));
        M1CHK(m1moe_copy_h2d(ctx, dres, fx.data(), fx.size() * 4));
    }
    M1CHK(m1moe_graph_begin(ctx));
    for (int r = 0; r < R; ++r) {
        float* res = (float*)dres + (size_t)h * r;
        float* y = (float*)dy + (size_t)h * r;
        if (f32)
            M1CHK(m1moe_moe_decode(ctx, r, (float*)dx32 + (size_t)h * r, M1MOE_F32, res, y,
                                   nullptr, nullptr));
        else
            M1CHK(m1moe_moe_decode(ctx, r, (uint16_t*)dx + (size_t)h * r, M1MOE_BF16, res, y,
                                   nullptr, nullptr));
    }
    m1moe_graph_t gr;
    M1CHK(m1moe_graph_end(ctx, &gr));
    for (int i = 0; i < 20; ++i) M1CHK(m1moe_graph_launch(ctx, gr));
    M1CHK(m1moe_sync(ctx));
    m1moe_event_t e0, e1;
    M1CHK(m1moe_event_create(ctx, &e0));
    M1CHK(m1moe_event_create(ctx, &e1));
    M1CHK(m1moe_event_record(ctx, e0));
    for (int i = 0; i < 30; ++i) M1CHK(m1moe_graph_launch(ctx, gr));
    M1CHK(m1moe_event_record(ctx, e1));
    float ms = 0.f;
    M1CHK(m1moe_event_elapsed_ms(e0, e1, &ms));
    printf("%s, %s input, %d replicas: %.3f us per launch (tracing build, no buffer set)\n",
           mixtral ? "cfg2" : "cfg0", f32 ? "f32" : "bf16", R, ms * 1000.0 / (30.0 * R));

    constexpr int G = 256, S = 64, NT = 5;
    unsigned long long* tb;
    HIPCHK(hipMalloc(&tb, G * S * 8));
    std::vector<std::vector<double>> acc(S);
    for (int rep = 0; rep < NT; ++rep) {
        HIPCHK(hipMemset(tb, 0, G * S * 8));
        HIPCHK(hipDeviceSynchronize());
        M1CHK(m1moe_trace_decode(tb));
        M1CHK(m1moe_graph_launch(ctx, gr));
        M1CHK(m1moe_sync(ctx));
        std::vector<unsigned long long> t((size_t)G * S);
        HIPCHK(hipMemcpy(t.data(), tb, t.size() * 8, hipMemcpyDeviceToHost));
        unsigned long long t0 = ~0ull;
        for (int w = 0; w < G; ++w)
            if (t[(size_t)w * S]) t0 = std::min(t0, t[(size_t)w * S]);
        // (cfg2: the 224 workgroups that multiply; the other 32 only route and reduce)
        const int gw = mixtral ? sh.top_k * sh.intermediate / 128 : G;
        for (int w = 0; w < gw; ++w)
            for (int s = 0; s < S; ++s)
                if (t[(size_t)w * S + s]) acc[s].push_back((double)(t[(size_t)w * S + s] - t0) * 0.01);
    }
    M1CHK(m1moe_trace_decode(nullptr));
    printf("phase stamps over %d traced replays (%s), us from the first workgroup's start\n\n"
           "| phase | n | min | p10 | median | p90 | max |\n|---|---|---|---|---|---|---|\n",
           NT, mixtral ? "the 224 working workgroups" : "all 256 workgroups");
    auto stat = [&](const char* name, int s) {
        std::vector<double> v = acc[s];
        if (v.empty()) return;
        std::sort(v.begin(), v.end());
        printf("| %s | %zu | %.2f | %.2f | %.2f | %.2f | %.2f |\n", name, v.size(), v[0],
               v[v.size() / 10], v[v.size() / 2], v[v.size() * 9 / 10], v.back());
    };
    char name[96];
    stat("start", 0);
    stat("router logit published (workgroups < E)", 1);
    if (!mixtral) stat("x chunks prepared (wave 1)", 2);
    stat("logits polled (wave 0)", 4);
    stat("rank: logits in LDS", 5);
    stat("rank: top-K written", 7);
    stat("routed (after barrier)", 3);
    for (int w = 0; w < 8; ++w) {
        snprintf(name, sizeof name, "gate/up + SwiGLU done, wave %d", w);
        stat(name, 8 + w);
    }
    stat(mixtral ? "act chunks prepared (after barrier)" : "act chunks prepared (wave 0)", 16);
    for (int w = 0; w < 8; ++w) {
        snprintf(name, sizeof name, "down nibbles expanded, wave %d", w);
        stat(name, 40 + w);
    }
    for (int w = 0; w < 8; ++w) {
        snprintf(name, sizeof name, "down partials computed, wave %d", w);
        stat(name, 24 + w);
    }
    stat("partials stored", 17);
    for (int w = 0; w < 8; ++w) {
        snprintf(name, sizeof name, "all partials of its rows in, wave %d", w);
        stat(name, 32 + w);
    }
    stat("end (rows combined and stored)", 56);
    m1moe_destroy(ctx);
    return 0;
}
