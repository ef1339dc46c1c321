// float instantiation of the MFMA GEMM kernels (gemm_mfma_impl.h).
#include "gemm_mfma_impl.h"

namespace tvk {
// fp32 matrix cores are 16x slower than the 16-bit ones, so a tile's wasted rows and columns cost
// real time (a 128-row tile computes 128 rows however few are real), and few large tiles leave CUs
// idle that the stream-K split only partly recovers.  Each of the four fp32 tiles is priced as
//   padded MACs / rate / sqrt(min(1, tiles / 128))
// with rates 1.0 (128x128), 0.96 (64x128), 0.94 (128x64) and 0.83 (32x128): the relative speeds
// on fp32 A[2592, 2048] @ B[2048, 4096] (2,688 / 2,624 / 2,592 padded rows: 353 / 363 / 376 /
// 425 us), and a fill term fitted to 23 fp32 shapes (M 100-4096, N 64-10000, K 1000-8192, batch
// 1 and 8) timed on every tile; the cheapest is launched.  E.g. A[3000, 4096] @ B[4096, 129]:
// 128x128 84.5 us, 128x64 61.4 us; A[300, 4096] @ B[4096, 4096]: 116.1 us, 64x128 99.7 us.
namespace {
struct F32Tile {
    int bm, bn;
    double rate;
};
constexpr F32Tile kF32Tiles[4] = {{128, 128, 1.0}, {64, 128, 0.96}, {128, 64, 0.94}, {32, 128, 0.83}};

int pick_f32_tile(const GemmDesc& d) {
    int best = 0;
    double best_cost = 0;
    for (int i = 0; i < 4; ++i) {
        const F32Tile& t = kF32Tiles[i];
        const double tm = (double)((d.M + t.bm - 1) / t.bm), tn = (double)((d.N + t.bn - 1) / t.bn);
        const double tiles = (double)d.batch * tm * tn;
        const double fill = tiles >= 128 ? 1.0 : std::sqrt(tiles / 128.0);
        const double cost = tiles * t.bm * t.bn / t.rate / fill;
        if (i == 0 || cost < best_cost) {
            best = i;
            best_cost = cost;
        }
    }
    return best;
}
} // namespace

int launch_gemm_mfma_f32(const GemmDesc& d, hipStream_t stream, bool may_alloc) {
    switch (pick_f32_tile(d)) {
        case 0: return run_modes<float, 128, 128, 2, 2>(d, stream, 8, may_alloc);
        case 1: return run_modes<float, 64, 128, 2, 2>(d, stream, 8, may_alloc);
        case 2: return run_modes<float, 128, 64, 2, 2>(d, stream, 8, may_alloc);
        default: return run_modes<float, 32, 128, 1, 4>(d, stream, 8, may_alloc);
    }
}
} // namespace tvk
