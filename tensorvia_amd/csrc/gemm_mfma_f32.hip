// float instantiation of the MFMA GEMM kernels (gemm_mfma_impl.h).
#include "gemm_mfma_impl.h"

namespace tvk {
// fp32 matrix cores are 16x slower than the 16-bit ones, so a tile's wasted rows cost real time: a
// 128-row tile computes 128 rows however few are real.  Few rows (or columns) take a smaller tile.
int launch_gemm_mfma_f32(const GemmDesc& d, hipStream_t stream, bool may_alloc) {
    if (d.M <= 32) return run_modes<float, 32, 128, 1, 4>(d, stream, 8, may_alloc);
    if (d.M <= 64) return run_modes<float, 64, 128, 2, 2>(d, stream, 8, may_alloc);
    if (d.N <= 64) return run_modes<float, 128, 64, 2, 2>(d, stream, 8, may_alloc);
    return run_modes<float, 128, 128, 2, 2>(d, stream, 8, may_alloc);
}
} // namespace tvk
