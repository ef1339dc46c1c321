// ops::Mul timed end to end, as the reference's own benchmark does (tests/mul.cpp:16-31: 100 x
// RUNNING_TIME(ops::Mul(a, b)) on the README shape [2592,2048] @ [2048,4096] fp32, the result a
// temporary destroyed after each call; its published figure is README.md:154-163).
//
// Besides the per-call wall time of ops::Mul (result allocation, kernel, the op's synchronisation
// and the result's release), it times the parts on their own:
//   alloc_free_ms  construct + destroy the result tensor alone (HIPContext::alloc / release);
//   kernel_ms      tv_hip_gemm on the same operands into one preallocated C, back to back, HIP
//                  events on the context stream around the launches;
//   launch_sync_ms the rest: host-side packing, the launch and the synchronisation round trip.
// Run once with the context's block cache (default) and once without (TV_HIP_CACHE_LIMIT_MB=0,
// every result hipMalloc'd and hipFree'd as the reference's CUDA backend does), each in its own
// process.  Prints one JSON object.
//
// usage: ops_mul_time [iters] [M K N] [dtype]   (defaults 100, 2592 2048 4096, 6 = FLOAT32)
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <string>

#include "tensorvia/hip_backend.h"
#include "tensorvia/ops.h"
#include "tensorvia_hip.h"

using via::DataType;
using clk = std::chrono::steady_clock;

namespace {
double ms_since(clk::time_point t0) { return std::chrono::duration<double, std::milli>(clk::now() - t0).count(); }

void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
} // namespace

int main(int argc, char** argv) {
    const int iters = argc > 1 ? std::atoi(argv[1]) : 100;
    const int64_t M = argc > 4 ? std::atoll(argv[2]) : 2592, K = argc > 4 ? std::atoll(argv[3]) : 2048,
                  N = argc > 4 ? std::atoll(argv[4]) : 4096;
    const auto dt = static_cast<DataType>(argc > 5 ? std::atoi(argv[5]) : static_cast<int>(DataType::FLOAT32));
    if (iters <= 0 || M <= 0 || K <= 0 || N <= 0) {
        std::fprintf(stderr, "usage: %s [iters] [M K N] [dtype]\n", argv[0]);
        return 2;
    }
    try {
        // The reference's operands: Tensor::Random({2592,2048}, -10, 10, FLOAT32) and {2048,4096}.
        Tensor a = ops::Random({M, K}, dt, -10.0f, 10.0f, 1);
        Tensor b = ops::Random({K, N}, dt, -10.0f, 10.0f, 2);
        auto ctx = HIPContext::get();
        const DataType rt = via::compute_type(dt, dt);

        // Settle: the GPU's clocks take tens of milliseconds of load to settle.
        const auto settle = clk::now();
        while (ms_since(settle) < 200.0) (void)ops::Mul(a, b);

        // 1. ops::Mul end to end (the reference's loop, without its per-call print).
        auto t0 = clk::now();
        for (int i = 0; i < iters; ++i) (void)ops::Mul(a, b);
        const double mul_ms = ms_since(t0) / iters;

        // 2. the result tensor's allocation and release alone.
        t0 = clk::now();
        for (int i = 0; i < iters; ++i) {
            Tensor c({M, N}, rt, via::Device::HIP);
            (void)c;
        }
        const double alloc_ms = ms_since(t0) / iters;

        // 3. the kernel: tv_hip_gemm into one C, back to back, events on the context stream.
        Tensor c({M, N}, rt, via::Device::HIP);
        tv_gemm_args g{};
        g.dtype_a = g.dtype_b = static_cast<int32_t>(dt);
        g.dtype_c = static_cast<int32_t>(rt);
        g.batch = 1;
        g.M = M; g.N = N; g.K = K;
        g.A = a.data(); g.sa_m = K; g.sa_k = 1;
        g.B = b.data(); g.sb_k = N; g.sb_n = 1;
        g.C = c.data(); g.sc_m = N; g.sc_n = 1;
        hipEvent_t e0, e1;
        check_hip(hipEventCreate(&e0), "hipEventCreate");
        check_hip(hipEventCreate(&e1), "hipEventCreate");
        check_hip(hipEventRecord(e0, ctx->stream()), "hipEventRecord");
        for (int i = 0; i < iters; ++i) {
            const int rc = tv_hip_gemm(&g, ctx->stream());
            if (rc) throw std::runtime_error(std::string("tv_hip_gemm: ") + tv_hip_strerror(rc));
        }
        check_hip(hipEventRecord(e1, ctx->stream()), "hipEventRecord");
        check_hip(hipEventSynchronize(e1), "hipEventSynchronize");
        float kern = 0.0f;
        check_hip(hipEventElapsedTime(&kern, e0, e1), "hipEventElapsedTime");
        const double kernel_ms = kern / iters;
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);

        std::printf("{\"shape\": [%lld, %lld, %lld], \"dtype\": \"%s\", \"iters\": %d, \"cache_limit_mb\": %zu, "
                    "\"ops_mul_ms\": %.4f, \"alloc_free_ms\": %.4f, \"kernel_ms\": %.4f, \"launch_sync_ms\": %.4f}\n",
                    static_cast<long long>(M), static_cast<long long>(K), static_cast<long long>(N),
                    std::string(via::dtype_to_string(dt)).c_str(), iters, ctx->cache_limit() >> 20, mul_ms, alloc_ms, kernel_ms,
                    mul_ms - alloc_ms - kernel_ms);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ops_mul_time: %s\n", e.what());
        return 1;
    }
    return 0;
}
