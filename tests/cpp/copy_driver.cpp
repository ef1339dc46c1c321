// GPU driver for the host <-> device boundary: Tensor(ptr, shape, dtype, Device::HIP) (host ->
// device through HIPContext::copy_h2d) and Tensor::to_host() (device -> host through copy_d2h),
// at sizes below, at and across the direct-copy threshold (4 MiB) and the pinned staging chunk
// (16 MiB).  Each round trip must return the host bytes unchanged: prints "ok <bytes>" or
// "mismatch <bytes> at <index>".
//
// With --time <MiB> it also times, for one buffer of that size: the API's host -> device and
// device -> host copies (the latter into a new host tensor, as to_host() makes), and plain hipMemcpy
// from and to the same pageable buffer, into a new untouched host buffer, and from and to pinned
// (hipHostMalloc) memory, printing "time <path> <GB/s>" lines (best of 5).
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "tensorvia/ops.h"

using via::DataType;

namespace {
void fill_pattern(std::vector<uint8_t>& v, uint32_t seed) {
    uint32_t x = seed * 2654435761u + 1u;
    for (auto& b : v) {
        x ^= x << 13;
        x ^= x >> 17;
        x ^= x << 5;
        b = static_cast<uint8_t>(x >> 24);
    }
}

bool round_trip(size_t bytes, uint32_t seed) {
    std::vector<uint8_t> host(bytes);
    fill_pattern(host, seed);
    Tensor dev(static_cast<void*>(host.data()), {static_cast<int64_t>(bytes)}, DataType::INT8, via::Device::HIP);
    dev.to_host();
    const auto* back = static_cast<const uint8_t*>(dev.data());
    for (size_t i = 0; i < bytes; ++i)
        if (back[i] != host[i]) {
            std::printf("mismatch %zu at %zu\n", bytes, i);
            return false;
        }
    std::printf("ok %zu\n", bytes);
    return true;
}

template <typename F> double best_gbs(size_t bytes, F&& f) {
    double best = 0;
    for (int r = 0; r < 5; ++r) {
        const auto t0 = std::chrono::steady_clock::now();
        f();
        const double s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        best = std::max(best, bytes / s / 1e9);
    }
    return best;
}

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
} // namespace

int main(int argc, char** argv) {
    int failures = 0;
    const size_t MiB = size_t(1) << 20;
    // 24 MiB + 5 and 17 MiB + 4 end in a staged chunk whose length over the 8 memcpy threads has a
    // page-aligned quotient (8 MiB + 5, 1 MiB + 4): the sizes whose tail a floor-rounded part size
    // would drop.
    for (size_t bytes : {size_t(1), size_t(1000), 4 * MiB - 1, 4 * MiB, 16 * MiB, 16 * MiB + 3, 32 * MiB + 17,
                         40 * MiB + 12345, 24 * MiB + 5, 17 * MiB + 4})
        failures += round_trip(bytes, static_cast<uint32_t>(bytes)) ? 0 : 1;

    if (argc == 3 && std::string(argv[1]) == "--time") {
        const size_t bytes = static_cast<size_t>(std::stoul(argv[2])) * MiB;
        std::vector<uint8_t> host(bytes);
        fill_pattern(host, 7);
        Tensor dev(static_cast<void*>(host.data()), {static_cast<int64_t>(bytes)}, DataType::INT8, via::Device::HIP);
        std::printf("time api_h2d %.2f\n", best_gbs(bytes, [&] {
            Tensor t(static_cast<void*>(host.data()), {static_cast<int64_t>(bytes)}, DataType::INT8, via::Device::HIP);
        }));
        std::printf("time api_d2h %.2f\n", best_gbs(bytes, [&] {
            Tensor t = dev.clone();
            t.to_host();
        }));
        void* d = nullptr;
        void* pinned = nullptr;
        check(hipMalloc(&d, bytes), "hipMalloc");
        check(hipHostMalloc(&pinned, bytes, hipHostMallocDefault), "hipHostMalloc");
        std::memcpy(pinned, host.data(), bytes);
        std::printf("time pageable_h2d %.2f\n", best_gbs(bytes, [&] { check(hipMemcpy(d, host.data(), bytes, hipMemcpyHostToDevice), "h2d"); }));
        std::printf("time pageable_d2h %.2f\n", best_gbs(bytes, [&] { check(hipMemcpy(host.data(), d, bytes, hipMemcpyDeviceToHost), "d2h"); }));
        std::printf("time pageable_d2h_new_buffer %.2f\n", best_gbs(bytes, [&] {
            std::unique_ptr<char[]> fresh(new char[bytes]);
            check(hipMemcpy(fresh.get(), d, bytes, hipMemcpyDeviceToHost), "d2h");
        }));
        std::printf("time pinned_h2d %.2f\n", best_gbs(bytes, [&] { check(hipMemcpy(d, pinned, bytes, hipMemcpyHostToDevice), "h2d"); }));
        std::printf("time pinned_d2h %.2f\n", best_gbs(bytes, [&] { check(hipMemcpy(pinned, d, bytes, hipMemcpyDeviceToHost), "d2h"); }));
        check(hipHostFree(pinned), "hipHostFree");
        check(hipFree(d), "hipFree");
    }
    std::printf("failures %d\n", failures);
    return failures ? 1 : 0;
}
