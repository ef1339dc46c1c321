// float instantiation of the MFMA GEMM kernels (gemm_mfma_impl.h).
#include "gemm_mfma_impl.h"

namespace tvk {
int launch_gemm_mfma_f32(const GemmDesc& d, hipStream_t stream, bool may_alloc) {
    return run_modes<float, 128, 128, 2, 2>(d, stream, 8, may_alloc);
}
} // namespace tvk
