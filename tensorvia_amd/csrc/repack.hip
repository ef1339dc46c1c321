// Strided view -> contiguous copy (TensorImpl::clone_as_contiguous of the HIP backend).
// Restates RepackImpl<Device::CUDA> (reference src/backend/cuda/repack.cu:5-54) without its
// per-call device allocations: shape and strides travel in the kernel arguments.  Each thread
// copies one element; consecutive threads write consecutive destination elements.
#include "tv_kernels.h"

namespace tvk {

struct RepackDesc {
    int64_t shape[TV_MAX_DIMS];
    int64_t strides[TV_MAX_DIMS];
    int ndim;
    int64_t numel;
    const void* src;
    void* dst;
};

template <typename E>
__global__ __launch_bounds__(256) void repack_kernel(RepackDesc r) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < r.numel; i += stride) {
        int64_t rem = i, off = 0;
        for (int d = r.ndim - 1; d >= 0; --d) {
            const int64_t c = rem % r.shape[d];
            rem /= r.shape[d];
            off += c * r.strides[d];
        }
        static_cast<E*>(r.dst)[i] = static_cast<const E*>(r.src)[off];
    }
}

int launch_repack(const tv_repack_args* a, hipStream_t stream) {
    RepackDesc r;
    r.ndim = a->ndim;
    r.numel = 1;
    for (int d = 0; d < a->ndim; ++d) {
        r.shape[d] = a->shape[d];
        r.strides[d] = a->strides[d];
        r.numel *= a->shape[d];
    }
    r.src = a->src;
    r.dst = a->dst;
    if (r.numel == 0) return 0;
    int64_t blocks = (r.numel + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    switch (a->elem_size) {
        case 1: hipLaunchKernelGGL(repack_kernel<uint8_t>, dim3((unsigned)blocks), dim3(256), 0, stream, r); break;
        case 2: hipLaunchKernelGGL(repack_kernel<uint16_t>, dim3((unsigned)blocks), dim3(256), 0, stream, r); break;
        case 4: hipLaunchKernelGGL(repack_kernel<uint32_t>, dim3((unsigned)blocks), dim3(256), 0, stream, r); break;
        case 8: hipLaunchKernelGGL(repack_kernel<uint64_t>, dim3((unsigned)blocks), dim3(256), 0, stream, r); break;
        default: return TV_E_DTYPE;
    }
    return hipGetLastError();
}

} // namespace tvk
