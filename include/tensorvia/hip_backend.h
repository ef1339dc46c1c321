// The HIP (MI355X) backend: context, storage and the matmul plugin, mirroring the reference's
// CUDA backend interfaces (include/backend/cuda/cuda_context.h:8-68, cuda_tensor.h:12-47,
// include/backend/cuda/ops/mul.h:6-15).
#pragma once

#include <hip/hip_runtime_api.h>

#include <condition_variable>
#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "context.h"
#include "ops.h"
#include "tensor.h"

// memcpy split over a small pool of host threads in page-aligned parts (the host side of the
// pinned staging copies; one thread moves pageable memory at about half the DMA engines' rate).
class ParallelMemcpy {
public:
    static constexpr size_t kMinSplit = size_t(1) << 20; // smaller copies stay on the calling thread
    explicit ParallelMemcpy(int threads = 0);            // 0: min(8, hardware threads)
    ~ParallelMemcpy();
    ParallelMemcpy(const ParallelMemcpy&) = delete;
    ParallelMemcpy& operator=(const ParallelMemcpy&) = delete;
    // Returns when all n bytes are copied.  One copy at a time per object.
    void copy(void* dst, const void* src, size_t n);
    int threads() const { return m_threads; }

private:
    void work(int i);
    void copy_part(int i) const;
    int m_threads = 1;
    std::vector<std::thread> m_workers;
    std::mutex m_mu;
    std::condition_variable m_go, m_fin;
    char* m_dst = nullptr;
    const char* m_src = nullptr;
    size_t m_len = 0, m_part = 0;
    unsigned m_gen = 0;
    int m_left = 0;
    bool m_stop = false;
};

// One HIP device (the one with the most memory, as CUDAContext picks, cuda_context.h:14-36) and
// one stream.  Ops enqueue on the stream and synchronise it before returning.
class HIPContext : public ContextImpl {
    int m_device_id = 0;
    hipStream_t m_stream = nullptr;
    // Pinned staging for copies of pageable host memory (allocated on first use).
    struct Staging;
    std::unique_ptr<Staging> m_staging;
    std::mutex m_staging_mu;
    Staging& staging();
    // Device blocks of released tensors, by capacity (see alloc()).
    std::multimap<size_t, void*> m_free;
    size_t m_cached = 0;
    size_t m_cache_limit = 0;
    mutable std::mutex m_cache_mu;

public:
    HIPContext();
    ~HIPContext() override;
    void* ctx_raw_ptr() override { return &m_stream; }
    hipStream_t stream() const { return m_stream; }
    int device_id() const { return m_device_id; }
    void wait() const;
    // Copies between pageable host memory and device memory on the context stream; they return
    // once the copy has completed.  Large copies go through two pinned chunks, the host-side
    // memcpy of one chunk overlapping the DMA of the other; small ones are direct.
    void copy_h2d(void* dst, const void* src, size_t bytes);
    void copy_d2h(void* dst, const void* src, size_t bytes);
    // The process-wide context, created on first use (no GPU is touched at library load).
    static std::shared_ptr<HIPContext> get();

    // Device memory of this context's tensors.  A released block is kept and handed to the next
    // tensor of about its size, so an op that returns a new tensor (ops::Mul's result) costs no
    // hipMalloc / hipFree once the sizes repeat; the reference's CUDA backend allocates every result
    // with cudaMalloc and frees it with cudaFree (src/backend/cuda/mul.cu:64,
    // include/backend/cuda/cuda_tensor.cpp:14-30).  All work of the context is on its one stream,
    // so a block released after its last use was enqueued there can serve later work on that
    // stream without a synchronisation.  Requests are rounded up (512 bytes below 1 MiB, 2 MiB
    // above) and served from a cached block at most a quarter larger.  Cached bytes are capped
    // (TV_HIP_CACHE_LIMIT_MB, default a quarter of the device's memory; 0 turns the cache off):
    // past the cap a released block is freed after a stream synchronisation, as without a cache.
    // When hipMalloc fails the cache is emptied and the allocation tried once more.
    // Work that a caller queues on another stream with a tensor's data() is outside that order:
    // it must have completed before the tensor is destroyed (hipFree waited for the whole device;
    // a cached block goes straight to the next tensor of the context).
    // alloc() returns nullptr for 0 bytes and sets *capacity to the block's size.
    void* alloc(size_t bytes, size_t* capacity);
    void release(void* p, size_t capacity);
    void empty_cache();
    size_t cached_bytes() const;
    size_t cache_limit() const { return m_cache_limit; }
};

// Device storage from the context's block cache (reference CUDATensor,
// include/backend/cuda/cuda_tensor.cpp:14-70, which calls cudaMalloc / cudaFree directly).
class HIPTensor : public TensorImpl {
    size_t m_numel = 0;
    via::DataType m_dtype = via::DataType::FLOAT32;
    std::shared_ptr<HIPContext> m_context;
    void* m_data = nullptr;
    size_t m_capacity = 0; // bytes of the context block holding the data

public:
    HIPTensor(void* host_ptr, size_t numel, via::DataType dtype, std::shared_ptr<HIPContext> ctx);
    ~HIPTensor() override;
    HIPTensor(const HIPTensor&) = delete;
    HIPTensor& operator=(const HIPTensor&) = delete;
    void* data() override { return m_data; }
    const void* data() const override { return m_data; }
    size_t numel() const override { return m_numel; }
    void copy_to(std::shared_ptr<TensorImpl> dst) const override;
    std::unique_ptr<TensorImpl> clone() const override;
    std::unique_ptr<TensorImpl> clone_as_contiguous(const Metadata& meta) const override;
    std::shared_ptr<ContextImpl> context() const override { return m_context; }
    std::shared_ptr<HIPContext> hip_context() const { return m_context; }
};

// Host storage (reference CPUTensor, include/backend/cpu/cpu_tensor.cpp:9-69): the staging side
// of to_host() / to_device().
class CPUTensor : public TensorImpl {
    size_t m_numel = 0;
    via::DataType m_dtype = via::DataType::FLOAT32;
    std::unique_ptr<char[]> m_data;

public:
    CPUTensor(void* ptr, size_t numel, via::DataType dtype);
    void* data() override { return m_data.get(); }
    const void* data() const override { return m_data.get(); }
    size_t numel() const override { return m_numel; }
    void copy_to(std::shared_ptr<TensorImpl> dst) const override;
    std::unique_ptr<TensorImpl> clone() const override;
    std::unique_ptr<TensorImpl> clone_as_contiguous(const Metadata& meta) const override;
    std::shared_ptr<ContextImpl> context() const override { return nullptr; }
};

namespace ops {
template <via::Device D> struct MulImpl;

// The HIP matmul plugin: packs the two views into the C-ABI descriptor (include/tensorvia_hip.h)
// and runs tv_hip_gemm on the context stream (replaces MulImpl<Device::CUDA>,
// src/backend/cuda/mul.cu:52-124).
template <> struct MulImpl<via::Device::HIP> {
    static Tensor execute(const Tensor& a, const Tensor& b);
};
// As the reference declares its backends' plugins (include/backend/cpu/ops/mul.h:15,
// include/backend/cuda/ops/mul.h:15): the definition lives in libtensorvia.so.
extern template struct MulImpl<via::Device::HIP>;

template <via::Device D> struct MulBiasActImpl;
// The fused matmul + bias + activation (tv_hip_gemm_ex).
template <> struct MulBiasActImpl<via::Device::HIP> {
    static Tensor execute(const Tensor& a, const Tensor& b, const Tensor* bias, Activation act);
};

template <via::Device D> struct TransposeImpl;
// Materialising permutation on the device (tv_hip_repack; replaces TransposeImpl<Device::CUDA>,
// src/backend/cuda/transpose.cu:129-174).  The dst overload reshapes dst to the permuted shape and
// writes into its storage, as the reference's does.
template <> struct TransposeImpl<via::Device::HIP> {
    static Tensor execute(const Tensor& a, std::initializer_list<int64_t> axes);
    static void execute(const Tensor& a, Tensor& dst, std::initializer_list<int64_t> axes);
};

template <via::Device D> struct TypecastImpl;
template <via::Device D> struct FillImpl;
template <via::Device D> struct RandomImpl;

// Element-wise cast on the device (tv_hip_typecast; replaces TypecastImpl<Device::CUDA>,
// src/backend/cuda/typecast.cu:29+).  Views are made contiguous on the device first.
template <> struct TypecastImpl<via::Device::HIP> {
    static Tensor execute(const Tensor& a, via::DataType dst_type);
};
// Constant fill on the device (tv_hip_fill; replaces FillImpl/ZerosImpl/OnesImpl<Device::CUDA>,
// src/backend/cuda/initializer.cu:39-98).
template <> struct FillImpl<via::Device::HIP> {
    static Tensor execute(const std::vector<int64_t>& shape, via::DataType dtype, float value);
};
// Seeded uniform values generated on the device (tv_hip_random; replaces RandomImpl<Device::CUDA>,
// src/backend/cuda/initializer.cu:99+), bit-identical to ops::detail::random_fill.
template <> struct RandomImpl<via::Device::HIP> {
    static Tensor execute(const std::vector<int64_t>& shape, via::DataType dtype, float min, float max, uint64_t seed);
};
} // namespace ops
