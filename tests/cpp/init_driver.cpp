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
    std::printf("failures %d\n", failures);
    return failures ? 1 : 0;
}
