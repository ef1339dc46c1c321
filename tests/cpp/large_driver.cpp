// GPU driver for the C++ API at sizes past 4 GiB:
//  * a host -> device -> host round trip of 4 GiB + 12,345 bytes (Tensor(ptr, shape, dtype,
//    Device::HIP) and to_host(), through HIPContext's pinned staging chunks);
//  * ops::Mul of an int8 A [131072, 40960] (5.4 GB) made by the device ops::Random with B [40960,
//    256]: A, B and C come back with to_host(), and sampled rows of C (the first rows, the rows on
//    either side of byte offset 2^32 of A, the last rows) must equal the low byte of the exact
//    int64 sums, the reference CPU backend's int8 result.
// Prints "ok <what>" or "mismatch <what> ..." lines; exit status 1 on any mismatch or exception.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "tensorvia/ops.h"

using via::DataType;

namespace {
bool round_trip() {
    const size_t bytes = (size_t(1) << 32) + 12345;
    std::vector<uint8_t> host(bytes);
    uint64_t x = 0x9E3779B97F4A7C15ull;
    for (size_t i = 0; i < bytes; i += 8) {
        x ^= x << 13;
        x ^= x >> 7;
        x ^= x << 17;
        std::memcpy(&host[i], &x, std::min<size_t>(8, bytes - i));
    }
    Tensor dev(static_cast<void*>(host.data()), {static_cast<int64_t>(bytes)}, DataType::INT8, via::Device::HIP);
    dev.to_host();
    const auto* back = static_cast<const uint8_t*>(dev.data());
    if (std::memcmp(back, host.data(), bytes) != 0) {
        size_t i = 0;
        while (back[i] == host[i]) ++i;
        std::printf("mismatch round_trip %zu bytes: first at %zu\n", bytes, i);
        return false;
    }
    std::printf("ok round_trip %zu bytes\n", bytes);
    return true;
}

bool mul_int8() {
    const int64_t M = 131072, K = 40960, N = 256;
    Tensor a = ops::Random({M, K}, DataType::INT8, -3, 3, 21);
    Tensor b = ops::Random({K, N}, DataType::INT8, -3, 3, 22);
    Tensor c = ops::Mul(a, b);
    if (c.dtype() != DataType::INT8 || c.shape(0) != M || c.shape(1) != N) {
        std::printf("mismatch mul: result dtype or shape\n");
        return false;
    }
    a.to_host();
    b.to_host();
    c.to_host();
    const auto* A = static_cast<const int8_t*>(a.data());
    const auto* B = static_cast<const int8_t*>(b.data());
    const auto* C = static_cast<const int8_t*>(c.data());
    // Row 104,858 is the first whose bytes of A start past 2^32 (104,858 * 40,960 > 2^32).
    const int64_t rows[] = {0, 1, 2, 65535, 65536, 104856, 104857, 104858, 104859, 131069, 131070, 131071};
    std::vector<int64_t> acc(N);
    for (int64_t m : rows) {
        std::fill(acc.begin(), acc.end(), 0);
        for (int64_t k = 0; k < K; ++k) {
            const int64_t av = A[m * K + k];
            const int8_t* brow = B + k * N;
            for (int64_t n = 0; n < N; ++n) acc[n] += av * brow[n];
        }
        for (int64_t n = 0; n < N; ++n)
            if (C[m * N + n] != static_cast<int8_t>(static_cast<uint8_t>(acc[n] & 0xFF))) {
                std::printf("mismatch mul: row %ld column %ld: %d, exact sum %ld\n", static_cast<long>(m), static_cast<long>(n),
                            static_cast<int>(C[m * N + n]), static_cast<long>(acc[n]));
                return false;
            }
    }
    std::printf("ok mul int8 [%ld,%ld]@[%ld,%ld]: %zu sampled rows\n", static_cast<long>(M), static_cast<long>(K),
                static_cast<long>(K), static_cast<long>(N), sizeof(rows) / sizeof(rows[0]));
    return true;
}
} // namespace

int main() {
    int failures = 0;
    try {
        failures += round_trip() ? 0 : 1;
        std::fflush(stdout);
        failures += mul_int8() ? 0 : 1;
    } catch (const std::exception& e) {
        std::printf("error: %s\n", e.what());
        ++failures;
    }
    std::fflush(stdout);
    return failures ? 1 : 0;
}
