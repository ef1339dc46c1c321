// float instantiation of the MFMA GEMM kernels (gemm_mfma_impl.h).
#include "gemm_mfma_impl.h"

namespace tvk {
// fp32 matrix cores are 16x slower than the 16-bit ones, so a tile's wasted rows and columns cost
// real time (a 128-row tile computes 128 rows however few are real), and few large tiles leave CUs
// idle that the stream-K split only partly recovers.  Each of the five fp32 tiles is priced as
//   padded MACs / rate / sqrt(min(1, tiles / 128))
// with rates 1.0 (128x128), 0.96 (64x128), 0.94 (128x64), 0.83 (32x128) and 0.77 (128x32): the
// relative speeds on fp32 A[2592, 2048] @ B[2048, 4096] (2,688 / 2,624 / 2,592 padded rows: 353 /
// 363 / 376 / 425 us) and, for 128x32, against 128x64 on shapes of several hundred tiles; the fill
// term was fitted to 50 fp32 shapes (M 20-10000, N 32-11008, K 1000-16384, batch 1, 2, 4, 8 and
// 16) timed on every tile, where the cheapest lands 0.8 % from the fastest on average.  E.g. A[3000, 4096] @
// B[4096, 129]: 128x128 84.5 us, 128x64 60.6 us, 128x32 56.6 us; A[8192, 4096] @ B[4096, 32]:
// 128x64 51.4 us, 128x32 34.8 us; A[300, 4096] @ B[4096, 4096]: 128x128 116.1 us, 64x128 99.7 us.
// A sixth tile, 96x128 (rate 0.984), serves row counts that 96 divides better than 128: on
// A[2592, 2048] @ B[2048, 4096] it computes 2,592 rows instead of 2,688 and ran 341.5-342.7 us
// against 348.5-349.1 us for 128x128 (same box, same process).  Its loaders need A k-contiguous
// (96 rows of an m-contiguous A do not split into whole 16-byte chunks per thread).
namespace {
struct F32Tile {
    int bm, bn;
    double rate;
};
constexpr int kF32TileCount = 6;
constexpr F32Tile kF32Tiles[kF32TileCount] = {{128, 128, 1.0}, {64, 128, 0.96}, {128, 64, 0.94},
                                              {32, 128, 0.83}, {128, 32, 0.77}, {96, 128, 0.984}};

int f32_a_mode_96(const GemmDesc& d) { return pick_mode(d.A, d.M, d.K, d.sa_m, d.sa_k, d.sa_b, d.batch, 4, 96, d.pad_a); }
int f32_b_mode(const GemmDesc& d) { return pick_mode(d.B, d.N, d.K, d.sb_n, d.sb_k, d.sb_b, d.batch, 4, 128, d.pad_b); }

// A 256x256 tile (8 waves of 128x64, one workgroup per CU) reads half the operand bytes per FLOP
// of the 128x128 tile.  It serves shapes whose 256x256 tiles fill whole rounds of the CUs with no
// padded rows or columns: A[4096,4096] @ B[4096,4096] 979.4 against 1,003.9 us, [8192]^3 7,702
// against 7,980 us, [4096,2048] @ [2048,4096] 499.1 against 507.2 us (same box, same process; both
// on the persistent stream-K kernel, before whole rounds took the plain kernel); with
// fewer tiles than CUs the stream-K split it would need measured slower ([2048,8192] @
// [8192,2048], 64 tiles: 533.7 against 518.4 us).
bool f32_whole_rounds_256(const GemmDesc& d) {
    if (d.M % 256 || d.N % 256) return false;
    const int64_t tiles = (int64_t)(d.M / 256) * (d.N / 256) * d.batch;
    const int cus = device_cus();
    return tiles >= cus && tiles % cus == 0;
}

int pick_f32_tile(const GemmDesc& d) {
    const int bm = f32_b_mode(d);
    const bool t96_ok = f32_a_mode_96(d) == LOAD_KCONTIG && (bm == LOAD_MNCONTIG || bm == LOAD_KCONTIG);
    int best = 0;
    double best_cost = 0;
    for (int i = 0; i < kF32TileCount; ++i) {
        if (i == 5 && !t96_ok) continue;
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
        case 0:
            if (f32_whole_rounds_256(d)) return run_modes<float, 256, 256, 2, 4>(d, stream, 8, may_alloc);
            return run_modes<float, 128, 128, 2, 2>(d, stream, 8, may_alloc);
        case 1: return run_modes<float, 64, 128, 2, 2>(d, stream, 8, may_alloc);
        case 2: return run_modes<float, 128, 64, 2, 2>(d, stream, 8, may_alloc);
        case 3: return run_modes<float, 32, 128, 1, 4>(d, stream, 8, may_alloc);
        case 4: return run_modes<float, 128, 32, 4, 1>(d, stream, 8, may_alloc);
        default:
            if (f32_b_mode(d) == LOAD_MNCONTIG)
                return run_cfg<GemmCfg<float, 96, 128, 2, 2, LOAD_KCONTIG, LOAD_MNCONTIG>>(d, stream, 8, may_alloc);
            return run_cfg<GemmCfg<float, 96, 128, 2, 2, LOAD_KCONTIG, LOAD_KCONTIG>>(d, stream, 8, may_alloc);
    }
}
} // namespace tvk
