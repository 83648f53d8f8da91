// stream_floor — what one launch costs on this GPU before any arithmetic: the
// floor under the per-CU MoE decode kernels (decode_cu.hip).
//
// Not part of the library.  Built by `make -C m1moe_amd/csrc probes` into
// m1moe_amd/_probes/stream_floor; prints one table row per probe.  Every probe
// is a graph of R launches, one per resident replica of the expert arena, so
// each launch reads bytes that are not in the 256 MB Infinity Cache:
//   * empty: an empty 256 x 512 kernel (launch and drain only);
//   * stream: a grid-stride read of the selected experts' canonical blocks
//     (16-byte nontemporal loads, as the kernels use), several grid sizes;
//   * cfg0 pattern: the exact loads of moe_decode_cu_kernel<4, 1> for an
//     OLMoE-shaped layer (h 2048, 64 experts, top-8, I 1024, group 64): per
//     workgroup g and wave w the scale/bias quad and the gate and up rows of
//     act rows 32 g + 4 w .. + 3, a barrier, then the down chunk g % 32 of
//     expert g / 32 (rows t + 512 r) and its scale/bias group, no compute.
// The Mixtral-shaped layer (h 4096, 8 experts, top-2, I 14336) gets the
// stream probe only.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#include "device.hpp"

#define CHECK(x)                                                                       \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            fprintf(stderr, "%s failed: %s (line %d)\n", #x, hipGetErrorString(e_),   \
                    __LINE__);                                                         \
            exit(1);                                                                   \
        }                                                                              \
    } while (0)

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t ld_fold(const uint8_t* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return v.x ^ v.y ^ v.z ^ v.w;
}

// The loaded words are folded into one value that is stored only if it equals
// a constant no data here produces, so no load can be dropped.
__device__ __forceinline__ void keep(uint32_t acc, uint32_t* sink) {
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

__global__ __launch_bounds__(512) void k_empty() {}

// Bytes [0, K * block) of the K selected blocks, block-contiguous, grid-stride,
// four independent loads per thread per step.
__global__ __launch_bounds__(256) void k_stream(const uint8_t* arena, uint64_t block,
                                                const int32_t* sel, int K, uint32_t* sink) {
    const uint64_t per = block / 16, total = per * (uint64_t)K;
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    uint32_t acc = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += 4 * stride) {
        uint32_t v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint64_t j = i + u * stride;
            const uint64_t jj = j < total ? j : total - 1;
            const uint64_t k = jj / per;
            v[u] = ld_fold(arena + (uint64_t)sel[k] * block + (jj - k * per) * 16);
        }
        acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
    keep(acc, sink);
}

// moe_decode_cu_kernel<4, 1>'s loads for h 2048, I 1024, group 64, top-8.
__global__ __launch_bounds__(512) void k_cfg0_pattern(const uint8_t* arena, uint64_t block,
                                                      const uint8_t* dec, uint64_t dec_block,
                                                      const int32_t* sel, uint32_t* sink) {
    constexpr int H = 2048, I = 1024, GS = 64;
    const m1moe::Layout L(H, I, GS);
    const m1moe::DecLayout D(H, I, GS);
    const int g = blockIdx.x, t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int k = g / (I / 32), row0 = (g % (I / 32)) * 32 + wave * 4;
    const uint8_t* blk = arena + (uint64_t)sel[k] * block;
    const uint8_t* dblk = dec + (uint64_t)sel[k] * dec_block;
    uint32_t v[18];
    const uint64_t so = ((uint64_t)(row0 / 4) * (H / GS) + (lane >> 1)) * 32;
    v[0] = ld_fold(dblk + D.gsb + so);
    v[1] = ld_fold(dblk + D.gsb + so + 16);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const uint64_t wo = (uint64_t)(row0 + u) * (H / 2) + lane * 16;
        v[2 + 2 * u] = ld_fold(blk + L.gate_w + wo);
        v[3 + 2 * u] = ld_fold(blk + L.up_w + wo);
    }
    __builtin_amdgcn_s_barrier();
    const int c = g % (I / 32);
#pragma unroll
    for (int r = 0; r < 4; ++r)
        v[10 + r] = ld_fold(dblk + D.dw + ((uint64_t)c * H + t + 512 * r) * 16);
    v[14] = ld_fold(dblk + D.dsb + ((uint64_t)(c / 2) * 512 + t) * 16);
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < 15; ++i) acc ^= v[i];
    keep(acc, sink);
}

struct Timer {
    hipStream_t st;
    hipEvent_t e0, e1;
    Timer() {
        CHECK(hipStreamCreate(&st));
        CHECK(hipEventCreate(&e0));
        CHECK(hipEventCreate(&e1));
    }
    // us per launch of a graph of R launches (5 warm-up replays, 20 timed)
    template <class F>
    double per_launch(int R, F launch) {
        hipGraph_t gr;
        hipGraphExec_t ex;
        CHECK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        for (int r = 0; r < R; ++r) launch(r, st);
        CHECK(hipStreamEndCapture(st, &gr));
        CHECK(hipGraphInstantiate(&ex, gr, nullptr, nullptr, 0));
        for (int i = 0; i < 5; ++i) CHECK(hipGraphLaunch(ex, st));
        CHECK(hipStreamSynchronize(st));
        CHECK(hipEventRecord(e0, st));
        for (int i = 0; i < 20; ++i) CHECK(hipGraphLaunch(ex, st));
        CHECK(hipEventRecord(e1, st));
        CHECK(hipEventSynchronize(e1));
        float ms = 0.f;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        CHECK(hipGraphExecDestroy(ex));
        CHECK(hipGraphDestroy(gr));
        return ms * 1000.0 / (20.0 * R);
    }
};

void row(const char* name, double us, double bytes) {
    if (bytes > 0)
        printf("| %s | %.2f | %.1f | %.2f | %.1f%% |\n", name, us, bytes / 1e6, bytes / us / 1e6,
               100.0 * bytes / us / 1e6 / 8.0);
    else
        printf("| %s | %.2f | - | - | - |\n", name, us);
    fflush(stdout);
}

uint64_t expert_bytes(int h, int I, int gs) {
    return (uint64_t)I * h / 2 * 3 + ((uint64_t)I * (h / gs) * 2 * 2) * 2 +
           (uint64_t)h * (I / gs) * 2 * 2;
}

}  // namespace

int main(int argc, char** argv) {
    const int R0 = argc > 1 ? atoi(argv[1]) : 38;  // cfg0 replicas (8.6 GB of canonical blocks)
    Timer tm;
    uint32_t* sink;
    CHECK(hipMalloc(&sink, 256));
    printf("| probe | us per launch | MB per launch | TB/s | of 8 TB/s |\n|---|---|---|---|---|\n");
    row("empty kernel, 256 x 512 threads", tm.per_launch(R0, [&](int, hipStream_t s) {
            hipLaunchKernelGGL(k_empty, dim3(256), dim3(512), 0, s);
        }), 0);

    {  // cfg0: 64 experts, top-8
        const int H = 2048, I = 1024, GS = 64, E = 64, K = 8, R = R0;
        const uint64_t eb = expert_bytes(H, I, GS);
        const uint64_t db = m1moe::DecLayout(H, I, GS).bytes;
        uint8_t *arena, *dec;
        int32_t* sel;
        CHECK(hipMalloc(&arena, (size_t)R * E * eb));
        CHECK(hipMalloc(&dec, (size_t)R * E * db));
        CHECK(hipMemset(arena, 0x11, (size_t)R * E * eb));
        CHECK(hipMemset(dec, 0x22, (size_t)R * E * db));
        std::vector<int32_t> hs((size_t)R * K);
        for (int r = 0; r < R; ++r)
            for (int k = 0; k < K; ++k) hs[(size_t)r * K + k] = (r * 7 + k * 8 + k * k) % E;
        CHECK(hipMalloc(&sel, hs.size() * 4));
        CHECK(hipMemcpy(sel, hs.data(), hs.size() * 4, hipMemcpyHostToDevice));
        const double stream_bytes = (double)K * eb;
        // the per-CU kernel's expert bytes: gate/up rows + the decode copy
        const double pattern_bytes = (double)K * ((double)I * H + (double)db);
        for (int grid : {512, 1024, 2048, 4096}) {
            char name[96];
            snprintf(name, sizeof name, "cfg0 stream, 8 selected blocks, grid %d x 256", grid);
            row(name, tm.per_launch(R, [&](int r, hipStream_t s) {
                    hipLaunchKernelGGL(k_stream, dim3(grid), dim3(256), 0, s,
                                       arena + (size_t)r * E * eb, eb, sel + r * K, K, sink);
                }), stream_bytes);
        }
        row("cfg0 per-CU kernel's loads, 256 x 512 threads, no compute",
            tm.per_launch(R, [&](int r, hipStream_t s) {
                hipLaunchKernelGGL(k_cfg0_pattern, dim3(256), dim3(512), 0, s,
                                   arena + (size_t)r * E * eb, eb, dec + (size_t)r * E * db, db,
                                   sel + r * K, sink);
            }), pattern_bytes);
        CHECK(hipFree(arena));
        CHECK(hipFree(dec));
        CHECK(hipFree(sel));
    }
    {  // cfg2: 8 experts, top-2 (8 replicas: 5.7 GB)
        const int H = 4096, I = 14336, GS = 64, E = 8, K = 2, R = 8;
        const uint64_t eb = expert_bytes(H, I, GS);
        uint8_t* arena;
        int32_t* sel;
        CHECK(hipMalloc(&arena, (size_t)R * E * eb));
        CHECK(hipMemset(arena, 0x33, (size_t)R * E * eb));
        std::vector<int32_t> hs((size_t)R * K);
        for (int r = 0; r < R; ++r)
            for (int k = 0; k < K; ++k) hs[(size_t)r * K + k] = (r + 3 * k) % E;
        CHECK(hipMalloc(&sel, hs.size() * 4));
        CHECK(hipMemcpy(sel, hs.data(), hs.size() * 4, hipMemcpyHostToDevice));
        for (int grid : {1024, 2048, 4096, 8192}) {
            char name[96];
            snprintf(name, sizeof name, "cfg2 stream, 2 selected blocks, grid %d x 256", grid);
            row(name, tm.per_launch(R, [&](int r, hipStream_t s) {
                    hipLaunchKernelGGL(k_stream, dim3(grid), dim3(256), 0, s,
                                       arena + (size_t)r * E * eb, eb, sel + r * K, K, sink);
                }), (double)K * eb);
        }
        CHECK(hipFree(arena));
        CHECK(hipFree(sel));
    }
    CHECK(hipDeviceSynchronize());
    printf("stream_floor done\n");
    return 0;
}
