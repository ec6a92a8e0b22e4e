// Stand-alone driver of the decode step through the C ABI (no Python), for
// profilers: builds the 48-layer resident context of the benchmark workload
// (H=2048, I=512, E=512, K=10, Is=512, synthetic weights), runs warm-up and
// timed steps on one stream and prints the mean step time. With
// --copy-calibration it also runs three 1 GiB plain copies (k_copy_bytes), whose
// traffic is known exactly, to scale hardware traffic counters.
//
//   fw_decode_bench [--layers L] [--tokens T] [--steps N] [--warmup W]
//                   [--seed S] [--copy-calibration]
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "firewing_hip_moe.h"

namespace {

void die(const char* what) {
    std::fprintf(stderr, "fw_decode_bench: %s: %s\n", what, firewing_hip_last_error());
    std::exit(1);
}

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        std::fprintf(stderr, "fw_decode_bench: %s: %s\n", what, hipGetErrorString(e));
        std::exit(1);
    }
}

}  // namespace

int main(int argc, char** argv) {
    size_t layers = 48, tokens = 1;
    int steps = 20, warmup = 3;
    uint64_t seed = 0x46495245ULL;
    bool copy_calibration = false;
    for (int i = 1; i < argc; ++i) {
        std::string a = argv[i];
        auto next = [&]() -> const char* {
            if (i + 1 >= argc) {
                std::fprintf(stderr, "missing value for %s\n", a.c_str());
                std::exit(2);
            }
            return argv[++i];
        };
        if (a == "--layers") layers = std::strtoull(next(), nullptr, 0);
        else if (a == "--tokens") tokens = std::strtoull(next(), nullptr, 0);
        else if (a == "--steps") steps = std::atoi(next());
        else if (a == "--warmup") warmup = std::atoi(next());
        else if (a == "--seed") seed = std::strtoull(next(), nullptr, 0);
        else if (a == "--copy-calibration") copy_calibration = true;
        else {
            std::fprintf(stderr, "unknown argument %s\n", a.c_str());
            return 2;
        }
    }
    firewing_hip_shape shape{2048, 512, 512, 10, 512, layers};
    firewing_hip_context* ctx = nullptr;
    if (!firewing_hip_create(&shape, &ctx)) die("create");
    if (!firewing_hip_generate_layers(ctx, 0, layers, seed, true)) die("generate_layers");
    std::vector<uint16_t> x(tokens * shape.hidden);
    firewing_hip_synth_hidden(seed, 0, (uint32_t)tokens, (uint32_t)shape.hidden, true, x.data());
    void *dx = nullptr, *dr = nullptr;
    hip_check(hipMalloc(&dx, x.size() * 2), "hipMalloc");
    hip_check(hipMalloc(&dr, x.size() * 2), "hipMalloc");
    hip_check(hipMemcpy(dx, x.data(), x.size() * 2, hipMemcpyHostToDevice), "hipMemcpy");
    hipStream_t s;
    hip_check(hipStreamCreate(&s), "hipStreamCreate");
    auto step = [&] {
        if (!firewing_hip_moe_step_dev(ctx, static_cast<const uint16_t*>(dx), tokens, FIREWING_HIP_LOGITS_TREE32,
                                       true, static_cast<uint16_t*>(dr), nullptr, nullptr, nullptr, s))
            die("moe_step_dev");
    };
    for (int i = 0; i < warmup; ++i) step();
    hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    hipEvent_t a, b;
    hip_check(hipEventCreate(&a), "hipEventCreate");
    hip_check(hipEventCreate(&b), "hipEventCreate");
    hip_check(hipEventRecord(a, s), "hipEventRecord");
    for (int i = 0; i < steps; ++i) step();
    hip_check(hipEventRecord(b, s), "hipEventRecord");
    hip_check(hipEventSynchronize(b), "hipEventSynchronize");
    if (!firewing_hip_synchronize(ctx)) die("synchronize");
    float ms = 0.0f;
    hip_check(hipEventElapsedTime(&ms, a, b), "hipEventElapsedTime");
    std::printf("decode step: %zu layers, %zu token(s): %.1f us/step over %d steps\n", layers, tokens,
                ms * 1000.0 / steps, steps);
    std::fflush(stdout);
    if (copy_calibration) {
        const size_t bytes = size_t(1) << 30;
        void *src = nullptr, *dst = nullptr;
        hip_check(hipMalloc(&src, bytes), "hipMalloc");
        hip_check(hipMalloc(&dst, bytes), "hipMalloc");
        for (int i = 0; i < 3; ++i)
            if (!firewing_hip_copy_bytes(dst, src, bytes, s)) die("copy_bytes");
        hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        std::printf("copy calibration: 3 x %zu bytes\n", bytes);
        std::fflush(stdout);
        hip_check(hipFree(src), "hipFree");
        hip_check(hipFree(dst), "hipFree");
    }
    hip_check(hipEventDestroy(a), "hipEventDestroy");
    hip_check(hipEventDestroy(b), "hipEventDestroy");
    hip_check(hipStreamDestroy(s), "hipStreamDestroy");
    hip_check(hipFree(dx), "hipFree");
    hip_check(hipFree(dr), "hipFree");
    firewing_hip_destroy(ctx);
    return 0;
}
