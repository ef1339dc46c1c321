// GPU driver for the C++ API's device initialisers and casts: ops::Random, ops::Fill / Zeros /
// Ones and ops::Typecast, all run on the HIP device (RandomImpl / FillImpl / TypecastImpl<HIP>).
// Writes each result's host storage bytes to <outdir>/<name>.bin and prints "done <name>"; the
// Python side regenerates the expected bytes with tensorvia_amd/rng.py and numpy.
//
//   rand_<dt>        ops::Random({3, 1001}, dt, lo, hi, seed 40 + dt)
//   fill_<dt>        ops::Fill({517}, dt, 2.75)
//   zeros_<dt>       ops::Zeros({9, 7}, dt);   ones_<dt>  ops::Ones({9, 7}, dt)
//   cast_<s>_<d>     ops::Typecast(ops::Random({257, 33}, s, lo, hi, seed 70 + 8 s + d).t(), d)
//                    (a transposed view, made contiguous on the device first)
// with [lo, hi] = [-100, 100] for integer and [-300, 300] for floating-point dtypes.
//   fused_<act>      ops::MulBiasAct(Random({2,64,96}, bf16, -1, 1, 90), Random({96,80}, bf16, -1, 1, 91),
//                    &Random({80}, bf16, -2, 2, 92), act)          (B and the bias broadcast)
//   fused_f32_full   ops::MulBiasAct(Random({64,96}, fp32, -1, 1, 93), Random({96,80}, fp32, -1, 1, 94),
//                    &Random({64,80}, fp32, -2, 2, 95), Silu)
//   tdst_<i>         ops::Transpose(src, dst, axes) into a 1-d dst of the same element count
//                    (dst reshaped to the permuted shape): i = 0..2 permute an int32
//                    Random({4, 6, 10}, -1000, 999, seed 100) by {2,0,1}, {0,2,1}, {1,0,2};
//                    i = 3 permutes fp16 Random({3, 40, 16}, -1, 1, seed 101) by {0,2,1} (config c4's
//                    materialised K^T); i = 4 permutes the slice [1:3, 2:6, :] of the int32 source by
//                    {2,1,0} (a view with an offset)
//   "threw <name>" lines: calls that must throw (bias of the wrong dtype or shape; Transpose into a
//   dst of another dtype or into a's own storage; a 2^60-byte device tensor).
//   mul_after_oom    ops::Mul(Random({64,96}, int8, -3, 3, 5), Random({96,80}, int8, -3, 3, 6)) right
//                    after the failed allocation
#include <cstdio>
#include <fstream>
#include <string>
#include <utility>
#include <vector>

#include "tensorvia/ops.h"

using via::DataType;

namespace {
void dump(const std::string& path, const Tensor& src) {
    Tensor t = src.contiguous();
    t.to_host();
    std::ofstream f(path, std::ios::binary);
    f.write(static_cast<const char*>(t.data()),
            static_cast<std::streamsize>(t.numel() * via::calc_dtype_size(t.dtype())));
    if (!f) throw std::runtime_error("cannot write " + path);
}

bool is_int(DataType d) { return static_cast<int>(d) <= static_cast<int>(DataType::INT64); }
float lo_of(DataType d) { return is_int(d) ? -100.0f : -300.0f; }
float hi_of(DataType d) { return is_int(d) ? 100.0f : 300.0f; }
} // namespace

int main(int argc, char** argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s <outdir>\n", argv[0]);
        return 2;
    }
    const std::string out = std::string(argv[1]) + "/";
    int failures = 0;
    auto run = [&](const std::string& name, auto&& make) {
        try {
            dump(out + name + ".bin", make());
            std::printf("done %s\n", name.c_str());
        } catch (const std::exception& e) {
            std::printf("FAIL %s: %s\n", name.c_str(), e.what());
            ++failures;
        }
        std::fflush(stdout);
    };
    for (int i = 0; i < 8; ++i) {
        const DataType dt = static_cast<DataType>(i);
        const std::string n = std::to_string(i);
        run("rand_" + n, [&] { return ops::Random({3, 1001}, dt, lo_of(dt), hi_of(dt), 40 + i); });
        run("fill_" + n, [&] { return ops::Fill({517}, dt, 2.75f); });
        run("zeros_" + n, [&] { return ops::Zeros({9, 7}, dt); });
        run("ones_" + n, [&] { return ops::Ones({9, 7}, dt); });
    }
    for (int s = 0; s < 8; ++s)
        for (int d = 0; d < 8; ++d) {
            const DataType sd = static_cast<DataType>(s), dd = static_cast<DataType>(d);
            if (s == d || !via::is_cast_valid(sd, dd)) continue;
            run("cast_" + std::to_string(s) + "_" + std::to_string(d), [&] {
                Tensor src = ops::Random({257, 33}, sd, lo_of(sd), hi_of(sd), 70 + 8 * s + d);
                return ops::Typecast(src.t(), dd);
            });
        }
    for (int act = 0; act <= 4; ++act)
        run("fused_" + std::to_string(act), [&] {
            const Tensor bias = ops::Random({80}, DataType::BFLOAT16, -2.0f, 2.0f, 92);
            return ops::MulBiasAct(ops::Random({2, 64, 96}, DataType::BFLOAT16, -1.0f, 1.0f, 90),
                                   ops::Random({96, 80}, DataType::BFLOAT16, -1.0f, 1.0f, 91), &bias,
                                   static_cast<ops::Activation>(act));
        });
    run("fused_f32_full", [&] {
        const Tensor bias = ops::Random({64, 80}, DataType::FLOAT32, -2.0f, 2.0f, 95);
        return ops::MulBiasAct(ops::Random({64, 96}, DataType::FLOAT32, -1.0f, 1.0f, 93),
                               ops::Random({96, 80}, DataType::FLOAT32, -1.0f, 1.0f, 94), &bias, ops::Activation::Silu);
    });
    const std::vector<std::vector<int64_t>> perms = {{2, 0, 1}, {0, 2, 1}, {1, 0, 2}};
    for (int i = 0; i < 3; ++i)
        run("tdst_" + std::to_string(i), [&] {
            const Tensor src = ops::Random({4, 6, 10}, DataType::INT32, -1000.0f, 999.0f, 100);
            Tensor dst = ops::Zeros({240}, DataType::INT32);
            const auto& p = perms[i];
            ops::Transpose(src, dst, {p[0], p[1], p[2]});
            if (dst.dims() != 3 || dst.shape(0) != src.shape(p[0]) || dst.shape(2) != src.shape(p[2]))
                throw std::runtime_error("dst not reshaped to the permuted shape");
            return dst;
        });
    run("tdst_3", [&] {
        const Tensor src = ops::Random({3, 40, 16}, DataType::FLOAT16, -1.0f, 1.0f, 101);
        Tensor dst = ops::Zeros({1920}, DataType::FLOAT16);
        ops::Transpose(src, dst, {0, 2, 1});
        return dst;
    });
    run("tdst_4", [&] {
        const Tensor src = ops::Random({4, 6, 10}, DataType::INT32, -1000.0f, 999.0f, 100);
        const Tensor view = src.slice({{1, 3}, {2, 6}});
        Tensor dst = ops::Zeros({80}, DataType::INT32);
        ops::Transpose(view, dst, {2, 1, 0});
        return dst;
    });
    auto must_throw = [&](const std::string& name, auto&& f) {
        try {
            f();
            std::printf("FAIL %s: no exception\n", name.c_str());
            ++failures;
        } catch (const std::exception& e) {
            std::printf("threw %s: %s\n", name.c_str(), e.what());
        }
    };
    const Tensor a = ops::Random({64, 96}, DataType::BFLOAT16, -1.0f, 1.0f, 1);
    const Tensor b = ops::Random({96, 80}, DataType::BFLOAT16, -1.0f, 1.0f, 2);
    const Tensor bias_f32 = ops::Random({80}, DataType::FLOAT32, -1.0f, 1.0f, 3);
    const Tensor bias_short = ops::Random({40}, DataType::BFLOAT16, -1.0f, 1.0f, 4);
    must_throw("bias_dtype", [&] { ops::MulBiasAct(a, b, &bias_f32, ops::Activation::Relu); });
    must_throw("bias_shape", [&] { ops::MulBiasAct(a, b, &bias_short, ops::Activation::Relu); });
    const Tensor ai = ops::Random({64, 96}, DataType::INT8, -3.0f, 3.0f, 5);
    const Tensor bi = ops::Random({96, 80}, DataType::INT8, -3.0f, 3.0f, 6);
    must_throw("int8_output", [&] { ops::MulBiasAct(ai, bi, nullptr, ops::Activation::Relu); });
    Tensor tdst_f32 = ops::Zeros({64 * 96}, DataType::FLOAT32);
    must_throw("transpose_dst_dtype", [&] { ops::Transpose(a, tdst_f32, {1, 0}); });
    Tensor self = ops::Random({8, 8}, DataType::FLOAT32, -1.0f, 1.0f, 7);
    must_throw("transpose_dst_self", [&] { ops::Transpose(self, self, {1, 0}); });
    // A device allocation that cannot fit throws, and leaves nothing behind that the next op would
    // report: ops::Mul right after it must succeed.
    must_throw("alloc_too_large", [&] { Tensor huge({int64_t(1) << 58}, DataType::FLOAT32, via::Device::HIP); });
    run("mul_after_oom", [&] { return ops::Mul(ai, bi); });
    std::printf("failures %d\n", failures);
    return failures ? 1 : 0;
}
