// Routes a validated descriptor to the MFMA GEMM instantiation of its input dtype.
#include "tv_kernels.h"

namespace tvk {
int launch_gemm_mfma_f32(const GemmDesc& d, hipStream_t stream, bool may_alloc);
int launch_gemm_mfma_bf16(const GemmDesc& d, hipStream_t stream, bool may_alloc);
int launch_gemm_mfma_f16(const GemmDesc& d, hipStream_t stream, bool may_alloc);
int launch_gemm_mfma_i8(const GemmDesc& d, hipStream_t stream, bool may_alloc);

int launch_gemm_mfma(const GemmDesc& d, hipStream_t stream, bool may_alloc) {
    switch (d.dtype_a) {
        case TV_FLOAT32: return launch_gemm_mfma_f32(d, stream, may_alloc);
        case TV_BFLOAT16: return launch_gemm_mfma_bf16(d, stream, may_alloc);
        case TV_FLOAT16: return launch_gemm_mfma_f16(d, stream, may_alloc);
        case TV_INT8: return launch_gemm_mfma_i8(d, stream, may_alloc);
        default: return TV_E_DTYPE;
    }
}
} // namespace tvk
