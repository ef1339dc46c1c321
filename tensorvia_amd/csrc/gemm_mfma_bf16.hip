// __bf16 instantiation of the GEMM kernels: the direct-load kernels of gemm_dma_impl.h and, for the
// operand layouts they do not take, the register-staged kernels of gemm_mfma_impl.h (which it includes).
#include "gemm_dma_impl.h"

namespace tvk {
int launch_gemm_mfma_bf16(const GemmDesc& d, hipStream_t stream, bool may_alloc) {
    return run_modes_dma<__bf16, 256, 256, 2, 4>(d, stream, 8, may_alloc);
}
} // namespace tvk
