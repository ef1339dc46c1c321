// GPU driver for the C++ API used from several host threads at once.  The HIP context is shared:
// one stream, the block cache and the pinned staging chunks, each behind its own mutex.  Four
// threads each run 12 iterations of ops::Random -> ops::Mul -> to_host() on their own operands
// (int8, bf16, fp32 and int8 again, different shapes); every iteration must give the same bytes as
// the thread's first iteration, and the int8 threads' sampled rows must equal the low byte of the exact
// sums.  Prints "ok thread <t> ..." or "mismatch thread <t> ..." lines; exit status 1 on any failure.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "tensorvia/ops.h"

using via::DataType;

namespace {
std::mutex g_print;

struct Job {
    DataType dt;
    int64_t M, K, N;
    uint64_t seed;
};

std::vector<uint8_t> bytes_of(Tensor t) {
    t.to_host();
    const size_t n = static_cast<size_t>(t.numel()) * via::calc_dtype_size(t.dtype());
    const auto* p = static_cast<const uint8_t*>(t.data());
    return std::vector<uint8_t>(p, p + n);
}

bool run(int t, const Job& j) {
    std::vector<uint8_t> first;
    for (int it = 0; it < 12; ++it) {
        Tensor a = ops::Random({j.M, j.K}, j.dt, -10, 10, j.seed);
        Tensor b = ops::Random({j.K, j.N}, j.dt, -10, 10, j.seed + 1);
        Tensor c = ops::Mul(a, b);
        std::vector<uint8_t> got = bytes_of(c);
        if (it == 0) {
            first = got;
            if (j.dt == DataType::INT8) {
                const std::vector<uint8_t> A = bytes_of(a), B = bytes_of(b);
                for (int64_t m : {int64_t(0), j.M / 2, j.M - 1})
                    for (int64_t n = 0; n < j.N; ++n) {
                        int64_t s = 0;
                        for (int64_t k = 0; k < j.K; ++k)
                            s += int64_t(int8_t(A[m * j.K + k])) * int64_t(int8_t(B[k * j.N + n]));
                        if (int8_t(got[m * j.N + n]) != int8_t(uint8_t(s & 0xFF))) {
                            std::lock_guard<std::mutex> lk(g_print);
                            std::printf("mismatch thread %d: row %ld column %ld\n", t, long(m), long(n));
                            return false;
                        }
                    }
            }
        } else if (got != first) {
            std::lock_guard<std::mutex> lk(g_print);
            std::printf("mismatch thread %d: iteration %d differs from iteration 0\n", t, it);
            return false;
        }
    }
    std::lock_guard<std::mutex> lk(g_print);
    std::printf("ok thread %d: 12 iterations of [%ld,%ld]@[%ld,%ld] dtype %d\n", t, long(j.M), long(j.K), long(j.K), long(j.N),
                static_cast<int>(j.dt));
    return true;
}
} // namespace

int main() {
    const Job jobs[] = {{DataType::INT8, 512, 1024, 768, 11}, {DataType::BFLOAT16, 300, 2048, 1000, 21},
                        {DataType::FLOAT32, 1, 4096, 4096, 31}, {DataType::INT8, 8, 4096, 2048, 41}};
    int failures = 0;
    std::mutex mu;
    std::vector<std::thread> threads;
    for (int t = 0; t < 4; ++t)
        threads.emplace_back([&, t] {
            bool ok = false;
            try {
                ok = run(t, jobs[t]);
            } catch (const std::exception& e) {
                std::lock_guard<std::mutex> lk(g_print);
                std::printf("error thread %d: %s\n", t, e.what());
            }
            if (!ok) {
                std::lock_guard<std::mutex> lk(mu);
                ++failures;
            }
        });
    for (auto& th : threads) th.join();
    std::fflush(stdout);
    return failures ? 1 : 0;
}
