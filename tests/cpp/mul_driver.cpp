// GPU driver for the C++ API parity tests: for each case line of <casefile>, builds the operands
// with the seeded ops::Random on the HIP device, forms the requested views, runs ops::Mul, and
// writes the base operands and the result (host storage bytes) to <outdir>/<name>_{a,b,c}.bin.
// The Python side regenerates the operands, checks them bit for bit, and checks C against the
// CPU oracle.
//
// Case line: name dtype_a dtype_b layout batch M K N lo hi seed_a seed_b
//   batch 0: rank-2 operands.  layout:
//     contig  A [b,M,K] @ B [b,K,N]
//     bcast   A [b,M,K] @ B [K,N]                     (B broadcast over the batch)
//     bt      B = base [b,N,K] permuted to [b,K,N]   (the strided config-4 operand)
//     at      A = base [b,K,M] permuted to [b,M,K]
//     slice   A = base [b,M+3,K+5][.., 1:M+1, 2:K+2], B = base [b,K+2,N+4][.., 1:K+1, 3:N+3]
#include <cstdio>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "tensorvia/ops.h"

using via::DataType;

namespace {
std::vector<int64_t> dims(int64_t batch, int64_t r, int64_t c) {
    return batch ? std::vector<int64_t>{batch, r, c} : std::vector<int64_t>{r, c};
}

Tensor swap_last2(const Tensor& t) {
    return t.dims() == 3 ? t.permute({0, 2, 1}) : t.permute({1, 0});
}

Tensor slice_last2(const Tensor& t, int64_t r0, int64_t r1, int64_t c0, int64_t c1) {
    if (t.dims() == 3) return t.slice({{0, t.shape(0)}, {r0, r1}, {c0, c1}});
    return t.slice({{r0, r1}, {c0, c1}});
}

void dump(const std::string& path, const Tensor& src) {
    Tensor t = src.contiguous(); // shares the storage of a dense tensor
    t.to_host();
    std::ofstream f(path, std::ios::binary);
    f.write(static_cast<const char*>(t.data()),
            static_cast<std::streamsize>(t.numel() * via::calc_dtype_size(t.dtype())));
    if (!f) throw std::runtime_error("cannot write " + path);
}
} // namespace

int main(int argc, char** argv) {
    if (argc != 3) {
        std::fprintf(stderr, "usage: %s <casefile> <outdir>\n", argv[0]);
        return 2;
    }
    std::ifstream cases(argv[1]);
    const std::string outdir = argv[2];
    std::string line;
    int failures = 0;
    while (std::getline(cases, line)) {
        if (line.empty() || line[0] == '#') continue;
        std::istringstream in(line);
        std::string name, layout;
        int dta, dtb;
        int64_t batch, M, K, N;
        float lo, hi;
        uint64_t sa, sb;
        in >> name >> dta >> dtb >> layout >> batch >> M >> K >> N >> lo >> hi >> sa >> sb;
        std::printf("case %s (%s, dtypes %d x %d, batch %ld, %ldx%ldx%ld)\n", name.c_str(), layout.c_str(), dta, dtb,
                    static_cast<long>(batch), static_cast<long>(M), static_cast<long>(K), static_cast<long>(N));
        std::fflush(stdout);
        try {
            const auto ta = static_cast<DataType>(dta), tb = static_cast<DataType>(dtb);
            Tensor abase, bbase, a, b;
            if (layout == "contig" || layout == "bcast") {
                abase = ops::Random(dims(batch, M, K), ta, lo, hi, sa);
                bbase = ops::Random(dims(layout == "bcast" ? 0 : batch, K, N), tb, lo, hi, sb);
                a = abase.permute(batch ? std::vector<int64_t>{0, 1, 2} : std::vector<int64_t>{0, 1});
                b = bbase.permute(bbase.dims() == 3 ? std::vector<int64_t>{0, 1, 2} : std::vector<int64_t>{0, 1});
            } else if (layout == "bt") {
                abase = ops::Random(dims(batch, M, K), ta, lo, hi, sa);
                bbase = ops::Random(dims(batch, N, K), tb, lo, hi, sb);
                a = abase.permute(batch ? std::vector<int64_t>{0, 1, 2} : std::vector<int64_t>{0, 1});
                b = swap_last2(bbase);
            } else if (layout == "at") {
                abase = ops::Random(dims(batch, K, M), ta, lo, hi, sa);
                bbase = ops::Random(dims(batch, K, N), tb, lo, hi, sb);
                a = swap_last2(abase);
                b = bbase.permute(batch ? std::vector<int64_t>{0, 1, 2} : std::vector<int64_t>{0, 1});
            } else if (layout == "slice") {
                abase = ops::Random(dims(batch, M + 3, K + 5), ta, lo, hi, sa);
                bbase = ops::Random(dims(batch, K + 2, N + 4), tb, lo, hi, sb);
                a = slice_last2(abase, 1, M + 1, 2, K + 2);
                b = slice_last2(bbase, 1, K + 1, 3, N + 3);
            } else {
                throw std::runtime_error("unknown layout " + layout);
            }
            Tensor c = ops::Mul(a, b);
            dump(outdir + "/" + name + "_a.bin", abase);
            dump(outdir + "/" + name + "_b.bin", bbase);
            dump(outdir + "/" + name + "_c.bin", c);
            std::printf("done %s dtype %d\n", name.c_str(), static_cast<int>(c.dtype()));
        } catch (const std::exception& e) {
            std::printf("error %s: %s\n", name.c_str(), e.what());
            ++failures;
        }
        std::fflush(stdout);
    }
    return failures ? 1 : 0;
}
