// Host-side checks of the C++ API that need no GPU: views and offsets, CPU gathers, ops::Mul
// validation, Typecast, the staging copies' threaded memcpy, and the seeded generator (its stream is written to <outdir> for the
// Python side to compare against tensorvia_amd/rng.py).
//
// Usage: host_api_test <outdir>.  Prints "ok <name>" per check; exits non-zero on the first failure.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <string>
#include <vector>

#include "tensorvia/hip_backend.h"
#include "tensorvia/ops.h"

using via::DataType;
using via::Device;

namespace {
int g_fail = 0;

void check(bool cond, const std::string& name, const std::string& what) {
    if (!cond) {
        std::printf("FAIL %s: %s\n", name.c_str(), what.c_str());
        g_fail = 1;
    }
}

void run(const std::string& name, const std::function<void()>& body) {
    try {
        const int before = g_fail;
        body();
        if (g_fail == before) std::printf("ok %s\n", name.c_str());
    } catch (const std::exception& e) {
        std::printf("FAIL %s: exception %s\n", name.c_str(), e.what());
        g_fail = 1;
    }
    std::fflush(stdout);
}

// Runs f, which must throw std::runtime_error whose message contains `needle`.
void expect_throw(const std::string& name, const std::function<void()>& f, const std::string& needle) {
    try {
        f();
    } catch (const std::exception& e) {
        check(std::string(e.what()).find(needle) != std::string::npos, name,
              std::string("message '") + e.what() + "' lacks '" + needle + "'");
        return;
    }
    check(false, name, "no exception");
}

Tensor iota_cpu(std::vector<int64_t> shape) {
    Tensor t(shape, DataType::INT32, Device::CPU);
    auto* p = static_cast<int32_t*>(t.data());
    for (size_t i = 0; i < t.numel(); ++i) p[i] = static_cast<int32_t>(i);
    return t;
}

std::vector<int32_t> values(const Tensor& t) {
    Tensor c = t.contiguous();
    const auto* p = static_cast<const int32_t*>(c.data());
    return std::vector<int32_t>(p, p + c.numel());
}

void dump(const std::string& path, const void* p, size_t bytes) {
    std::ofstream f(path, std::ios::binary);
    f.write(static_cast<const char*>(p), static_cast<std::streamsize>(bytes));
}
} // namespace

int main(int argc, char** argv) {
    const std::string outdir = argc > 1 ? argv[1] : ".";

    run("transpose_view_strides", [] {
        Tensor a = iota_cpu({4, 6});
        Tensor t = a.t();
        check(t.shape() == std::vector<int64_t>{6, 4}, "transpose_view_strides", "shape");
        check(t.strides() == std::vector<int64_t>{1, 6}, "transpose_view_strides", "strides");
        check(!t.is_contiguous(), "transpose_view_strides", "is_contiguous");
        auto v = values(t);
        bool good = true;
        for (int i = 0; i < 6; ++i)
            for (int j = 0; j < 4; ++j) good &= v[i * 4 + j] == j * 6 + i;
        check(good, "transpose_view_strides", "gathered values");
    });

    run("slice_offset_and_gather", [] {
        Tensor a = iota_cpu({5, 7});
        Tensor s = a.slice({{1, 4}, {2, 6}});
        check(s.offset() == 1 * 7 + 2, "slice_offset_and_gather", "offset");
        check(s.strides() == std::vector<int64_t>{7, 1}, "slice_offset_and_gather", "strides");
        auto v = values(s);
        bool good = v.size() == 12;
        for (int i = 0; good && i < 3; ++i)
            for (int j = 0; j < 4; ++j) good &= v[i * 4 + j] == (i + 1) * 7 + (j + 2);
        check(good, "slice_offset_and_gather", "values");
        // A view of a slice keeps the slice's offset (the reference would reset it to 0).
        Tensor st = s.t();
        check(st.offset() == s.offset(), "slice_offset_and_gather", "t() keeps offset");
        auto w = values(st);
        bool good2 = true;
        for (int i = 0; i < 4; ++i)
            for (int j = 0; j < 3; ++j) good2 &= w[i * 3 + j] == (j + 1) * 7 + (i + 2);
        check(good2, "slice_offset_and_gather", "t() of slice values");
    });

    run("permute_021_like_config4", [] {
        Tensor k = iota_cpu({3, 5, 4});
        Tensor p = k.permute({0, 2, 1});
        check(p.shape() == std::vector<int64_t>{3, 4, 5}, "permute_021_like_config4", "shape");
        check(p.strides() == std::vector<int64_t>{20, 1, 4}, "permute_021_like_config4", "strides");
        auto v = values(p);
        bool good = true;
        for (int b = 0; b < 3; ++b)
            for (int i = 0; i < 4; ++i)
                for (int j = 0; j < 5; ++j) good &= v[(b * 4 + i) * 5 + j] == b * 20 + j * 4 + i;
        check(good, "permute_021_like_config4", "values");
        Tensor m = ops::Transpose(k, {0, 2, 1});
        check(m.is_contiguous() && values(m) == v, "permute_021_like_config4", "Transpose materialises");
    });

    run("copy_of_view_is_contiguous", [] {
        Tensor a = iota_cpu({4, 6});
        Tensor t = a.t();
        Tensor c(t);
        check(c.is_contiguous() && c.offset() == 0, "copy_of_view_is_contiguous", "layout");
        check(values(c) == values(t), "copy_of_view_is_contiguous", "values");
    });

    run("mul_validation_messages", [] {
        Tensor a2({4, 5}, DataType::FLOAT32, Device::CPU), b2({5, 3}, DataType::FLOAT32, Device::CPU);
        Tensor bad_k({6, 3}, DataType::FLOAT32, Device::CPU);
        Tensor a3({2, 4, 5}, DataType::FLOAT32, Device::CPU), b3({3, 5, 3}, DataType::FLOAT32, Device::CPU);
        Tensor a4({1, 2, 4, 5}, DataType::FLOAT32, Device::CPU);
        Tensor bad_k3({2, 6, 3}, DataType::FLOAT32, Device::CPU);
        // Messages and their order are the reference's (src/ops.cpp:542-556): the rank check comes
        // before the 2-or-3 check, and the 2-d message names dimension 0 of both operands.
        expect_throw("mul_validation_messages", [&] { ops::Mul(a2, bad_k); },
                     "Tensors common dim must match,but 4 and 6");
        expect_throw("mul_validation_messages", [&] { ops::Mul(a3, bad_k3); },
                     "Tensors common dim must match,but 5 and 6");
        expect_throw("mul_validation_messages", [&] { ops::Mul(a2, a3); },
                     "Tensors a and b must have the same rank,but got 2 and 3");
        expect_throw("mul_validation_messages", [&] { ops::Mul(a4, a2); },
                     "Tensors a and b must have the same rank,but got 4 and 2");
        expect_throw("mul_validation_messages", [&] { ops::Mul(a4, a4); }, "Tensors a and b dims must be 2 or 3,but got 4");
        expect_throw("mul_validation_messages", [&] { ops::Mul(a3, b3); }, "Tensors a and b must have the same batch size");
        expect_throw("mul_validation_messages", [&] { ops::Mul(a2, a4); }, "same rank");
        // The broadcast extension: rank-3 A with rank-2 B passes validation (then needs the device).
        expect_throw("mul_validation_messages", [&] { ops::Mul(a3, b2); }, "to_device");
        // A zero-sized dimension is rejected when the tensor is built (type_traits.h:296), so K = 0
        // never reaches ops::Mul.
        expect_throw("mul_validation_messages", [&] { Tensor k0({4, 0}, DataType::FLOAT32, Device::CPU); },
                     "Invalid tensor dimension");
        Tensor dst({7}, DataType::FLOAT32, Device::CPU);
        expect_throw("mul_validation_messages", [&] { ops::Transpose(a2, dst, {1, 0}); }, "dst numel not enough");
        expect_throw("mul_validation_messages", [&] { ops::Transpose(a2, dst, {1, 0, 2}); },
                     "transpose shape and axes size not match");
        // Valid shapes on CPU tensors: the CPU backend is not part of this build.
        expect_throw("mul_validation_messages", [&] { ops::Mul(a2, b2); }, "to_device");
    });

    run("parallel_memcpy", [] {
        // The staging copies' threaded memcpy: every byte copied, nothing written past the end, at
        // sizes around the split threshold and the page-aligned part boundaries.
        for (int threads : {1, 2, 3, 8}) {
            ParallelMemcpy mc(threads);
            for (size_t n : {size_t(0), size_t(1), size_t(4095), ParallelMemcpy::kMinSplit - 1, ParallelMemcpy::kMinSplit,
                             ParallelMemcpy::kMinSplit + 7, (size_t(3) << 20) + 123, (size_t(16) << 20) + 5}) {
                std::vector<unsigned char> src(n + 64), dst(n + 64, 0xA5);
                for (size_t i = 0; i < src.size(); ++i) src[i] = static_cast<unsigned char>(i * 131 + 7);
                mc.copy(dst.data(), src.data(), n);
                bool ok = std::equal(src.begin(), src.begin() + static_cast<std::ptrdiff_t>(n), dst.begin());
                for (size_t i = n; i < n + 64; ++i) ok = ok && dst[i] == 0xA5;
                check(ok, "parallel_memcpy", "threads " + std::to_string(threads) + " bytes " + std::to_string(n));
            }
        }
    });

    run("typecast_widening_exact", [] {
        std::vector<bfloat16> h = {bfloat16(1.5f), bfloat16(-0.375f), bfloat16(3.0e38f)};
        Tensor b(static_cast<void*>(h.data()), {3}, DataType::BFLOAT16, Device::CPU);
        Tensor f = ops::Typecast(static_cast<const Tensor&>(b), DataType::FLOAT32);
        const float* p = static_cast<const float*>(f.data());
        check(f.dtype() == DataType::FLOAT32 && p[0] == 1.5f && p[1] == -0.375f &&
                  p[2] == static_cast<float>(h[2]),
              "typecast_widening_exact", "values");
        expect_throw("typecast_widening_exact", [&] { ops::Typecast(static_cast<const Tensor&>(f), DataType::INT8); }, "Invalid typecast");
    });

    run("random_streams_dumped", [&] {
        struct Case { const char* tag; DataType dt; float lo, hi; uint64_t seed; size_t n; };
        const Case cases[] = {{"f32", DataType::FLOAT32, -1.f, 1.f, 1, 4099},
                              {"bf16", DataType::BFLOAT16, -1.f, 1.f, 5, 4099},
                              {"f16", DataType::FLOAT16, -0.05f, 0.05f, 10, 4099},
                              {"i8", DataType::INT8, -10.f, 10.f, 3, 4099},
                              {"i8full", DataType::INT8, -128.f, 127.f, 77, 4099},
                              {"i32", DataType::INT32, -1000.f, 999.f, 42, 4099}};
        for (const Case& c : cases) {
            std::vector<char> buf(c.n * via::calc_dtype_size(c.dt));
            ops::detail::random_fill(buf.data(), c.n, c.dt, c.lo, c.hi, c.seed);
            dump(outdir + "/random_" + c.tag + ".bin", buf.data(), buf.size());
        }
    });

    return g_fail;
}
