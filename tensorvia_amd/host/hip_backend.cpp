// HIP backend: context, device/host storage, copies, registration and the matmul plugin.
// Mirrors the reference CUDA backend's roles (include/backend/cuda/cuda_context.h:8-68,
// cuda_tensor.cpp:14-70, cuda_copy.cpp:9-26, src/init.cpp:18-34, src/backend/cuda/mul.cu:52-124)
// on the C-ABI of include/tensorvia_hip.h.
#include <algorithm>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "tensorvia/factory.h"
#include "tensorvia/hip_backend.h"
#include "tensorvia_hip.h"

using namespace via;

namespace {

// Throws on a failed HIP call.  The runtime also keeps the failure as its last error, which the
// kernel library's launchers read after each launch: it is cleared here so that a caught exception
// (an allocation that did not fit, say) is not reported again by the next, successful call.
void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        (void)hipGetLastError();
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
    }
}

void tv_check(int rc, const char* what) {
    if (rc != TV_OK) throw std::runtime_error(std::string(what) + ": " + tv_hip_strerror(rc));
}

std::shared_ptr<HIPContext> hip_ctx_of(const std::shared_ptr<TensorImpl>& t) {
    auto h = std::dynamic_pointer_cast<HIPTensor>(t);
    if (!h) throw std::runtime_error("expected a HIP tensor");
    return h->hip_context();
}

} // namespace

// ---- HIPContext --------------------------------------------------------------------------------

HIPContext::HIPContext() {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) throw std::runtime_error("No HIP devices found");
    size_t best_mem = 0;
    for (int i = 0; i < count; ++i) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, i) == hipSuccess && prop.totalGlobalMem > best_mem) {
            best_mem = prop.totalGlobalMem;
            m_device_id = i;
        }
    }
    hip_check(hipSetDevice(m_device_id), "hipSetDevice");
    hip_check(hipStreamCreate(&m_stream), "hipStreamCreate");
    size_t free_b = 0, total_b = 0;
    m_cache_limit = hipMemGetInfo(&free_b, &total_b) == hipSuccess ? total_b / 4 : (size_t(1) << 30);
    if (const char* env = std::getenv("TV_HIP_CACHE_LIMIT_MB")) {
        char* end = nullptr;
        const unsigned long long mb = std::strtoull(env, &end, 10);
        if (end != env) m_cache_limit = static_cast<size_t>(mb) << 20;
    }
}

// ---- device block cache ----------------------------------------------------------------------------

namespace {
size_t round_block(size_t bytes) {
    const size_t g = bytes < (size_t(1) << 20) ? 512 : (size_t(2) << 20);
    return (bytes + g - 1) / g * g;
}
} // namespace

void* HIPContext::alloc(size_t bytes, size_t* capacity) {
    *capacity = 0;
    if (bytes == 0) return nullptr;
    const size_t want = round_block(bytes);
    {
        std::lock_guard<std::mutex> lk(m_cache_mu);
        auto it = m_free.lower_bound(want);
        if (it != m_free.end() && it->first <= want + want / 4) {
            void* p = it->second;
            *capacity = it->first;
            m_cached -= it->first;
            m_free.erase(it);
            return p;
        }
    }
    hip_check(hipSetDevice(m_device_id), "hipSetDevice");
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        empty_cache();
        e = hipMalloc(&p, want);
    }
    hip_check(e, "hipMalloc");
    *capacity = want;
    return p;
}

void HIPContext::release(void* p, size_t capacity) {
    if (!p) return;
    {
        std::lock_guard<std::mutex> lk(m_cache_mu);
        if (m_cached + capacity <= m_cache_limit) {
            m_free.emplace(capacity, p);
            m_cached += capacity;
            return;
        }
    }
    (void)hipStreamSynchronize(m_stream); // work queued on the block finishes before it is freed
    (void)hipFree(p);
}

void HIPContext::empty_cache() {
    std::multimap<size_t, void*> blocks;
    {
        std::lock_guard<std::mutex> lk(m_cache_mu);
        blocks.swap(m_free);
        m_cached = 0;
    }
    if (blocks.empty()) return;
    (void)hipStreamSynchronize(m_stream);
    for (auto& b : blocks) (void)hipFree(b.second);
}

size_t HIPContext::cached_bytes() const {
    std::lock_guard<std::mutex> lk(m_cache_mu);
    return m_cached;
}

// ---- ParallelMemcpy ------------------------------------------------------------------------------

ParallelMemcpy::ParallelMemcpy(int threads) {
    if (threads <= 0) {
        const unsigned hw = std::thread::hardware_concurrency();
        threads = static_cast<int>(std::min(8u, hw ? hw : 1u));
    }
    m_threads = threads;
    for (int i = 1; i < m_threads; ++i) m_workers.emplace_back([this, i] { work(i); });
}

ParallelMemcpy::~ParallelMemcpy() {
    {
        std::lock_guard<std::mutex> lk(m_mu);
        m_stop = true;
    }
    m_go.notify_all();
    for (auto& t : m_workers) t.join();
}

// Part i of the current job: [i * part, (i + 1) * part) clipped to the job's length.
void ParallelMemcpy::copy_part(int i) const {
    const size_t b = std::min(m_len, i * m_part), e = std::min(m_len, (i + 1) * m_part);
    if (e > b) std::memcpy(m_dst + b, m_src + b, e - b);
}

void ParallelMemcpy::work(int i) {
    unsigned seen = 0;
    std::unique_lock<std::mutex> lk(m_mu);
    for (;;) {
        m_go.wait(lk, [&] { return m_stop || m_gen != seen; });
        if (m_stop) return;
        seen = m_gen;
        lk.unlock();
        copy_part(i);
        lk.lock();
        if (--m_left == 0) m_fin.notify_one();
    }
}

void ParallelMemcpy::copy(void* dst, const void* src, size_t n) {
    if (m_threads == 1 || n < kMinSplit) {
        if (n) std::memcpy(dst, src, n);
        return;
    }
    std::unique_lock<std::mutex> lk(m_mu);
    m_dst = static_cast<char*>(dst);
    m_src = static_cast<const char*>(src);
    m_len = n;
    // ceil(n / threads) rounded up to whole pages, so the parts cover all n bytes.
    m_part = ((n + m_threads - 1) / m_threads + 4095) & ~size_t(4095);
    m_left = m_threads - 1;
    ++m_gen;
    lk.unlock();
    m_go.notify_all();
    copy_part(0);
    lk.lock();
    m_fin.wait(lk, [&] { return m_left == 0; });
}

// Two pinned chunks, the events that mark the DMA last issued from each, and the host threads that
// split each chunk's memcpy (one thread copies a pageable buffer at about half the rate the DMA
// engines move a pinned one).
struct HIPContext::Staging {
    static constexpr size_t kChunk = size_t(16) << 20;
    void* buf[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    ParallelMemcpy mc;

    ~Staging() {
        for (int i = 0; i < 2; ++i) {
            if (done[i]) (void)hipEventDestroy(done[i]);
            if (buf[i]) (void)hipHostFree(buf[i]);
        }
    }
    void copy(void* dst, const void* src, size_t n) { mc.copy(dst, src, n); }
};

// Copies below this size go straight through hipMemcpyAsync.
static constexpr size_t kStagingMin = size_t(4) << 20;

HIPContext::~HIPContext() {
    if (m_stream) (void)hipStreamSynchronize(m_stream);
    for (auto& b : m_free) (void)hipFree(b.second);
    m_free.clear();
    m_staging.reset();
    if (m_stream) (void)hipStreamDestroy(m_stream);
}

void HIPContext::wait() const { hip_check(hipStreamSynchronize(m_stream), "hipStreamSynchronize"); }

HIPContext::Staging& HIPContext::staging() {
    if (!m_staging) {
        auto st = std::make_unique<Staging>();
        for (int i = 0; i < 2; ++i) {
            hip_check(hipHostMalloc(&st->buf[i], Staging::kChunk, hipHostMallocDefault), "hipHostMalloc (staging)");
            hip_check(hipEventCreateWithFlags(&st->done[i], hipEventDisableTiming), "hipEventCreate (staging)");
        }
        m_staging = std::move(st);
    }
    return *m_staging;
}

void HIPContext::copy_h2d(void* dst, const void* src, size_t bytes) {
    if (bytes < kStagingMin) {
        hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, m_stream), "hipMemcpyAsync H2D");
        wait();
        return;
    }
    std::lock_guard<std::mutex> lk(m_staging_mu);
    Staging& st = staging();
    size_t i = 0;
    for (size_t off = 0; off < bytes; off += Staging::kChunk, ++i) {
        const size_t n = std::min(Staging::kChunk, bytes - off);
        const int b = static_cast<int>(i & 1);
        // The DMA that last read this chunk (two chunks ago) has finished; then refill it while
        // the other chunk's DMA runs.
        hip_check(hipEventSynchronize(st.done[b]), "hipEventSynchronize (staging)");
        st.copy(st.buf[b], static_cast<const char*>(src) + off, n);
        hip_check(hipMemcpyAsync(static_cast<char*>(dst) + off, st.buf[b], n, hipMemcpyHostToDevice, m_stream),
                  "hipMemcpyAsync H2D (staged)");
        hip_check(hipEventRecord(st.done[b], m_stream), "hipEventRecord (staging)");
    }
    wait();
}

void HIPContext::copy_d2h(void* dst, const void* src, size_t bytes) {
    if (bytes < kStagingMin) {
        hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, m_stream), "hipMemcpyAsync D2H");
        wait();
        return;
    }
    std::lock_guard<std::mutex> lk(m_staging_mu);
    Staging& st = staging();
    // Chunk i's DMA is issued before chunk i-1 is copied out of its pinned buffer.
    int prev = -1;
    size_t prev_off = 0, prev_n = 0, i = 0;
    auto drain = [&] {
        hip_check(hipEventSynchronize(st.done[prev]), "hipEventSynchronize (staging)");
        st.copy(static_cast<char*>(dst) + prev_off, st.buf[prev], prev_n);
    };
    for (size_t off = 0; off < bytes; off += Staging::kChunk, ++i) {
        const size_t n = std::min(Staging::kChunk, bytes - off);
        const int b = static_cast<int>(i & 1);
        hip_check(hipMemcpyAsync(st.buf[b], static_cast<const char*>(src) + off, n, hipMemcpyDeviceToHost, m_stream),
                  "hipMemcpyAsync D2H (staged)");
        hip_check(hipEventRecord(st.done[b], m_stream), "hipEventRecord (staging)");
        if (prev >= 0) drain();
        prev = b;
        prev_off = off;
        prev_n = n;
    }
    if (prev >= 0) drain();
    wait();
}

std::shared_ptr<HIPContext> HIPContext::get() {
    static std::mutex mu;
    static std::shared_ptr<HIPContext> ctx;
    std::lock_guard<std::mutex> lk(mu);
    if (!ctx) ctx = std::make_shared<HIPContext>();
    return ctx;
}

// ---- HIPTensor ---------------------------------------------------------------------------------

HIPTensor::HIPTensor(void* host_ptr, size_t numel, DataType dtype, std::shared_ptr<HIPContext> ctx)
    : m_numel(numel), m_dtype(dtype), m_context(std::move(ctx)) {
    const size_t bytes = numel * calc_dtype_size(dtype);
    m_data = m_context->alloc(bytes, &m_capacity);
    if (host_ptr && bytes) m_context->copy_h2d(m_data, host_ptr, bytes);
}

HIPTensor::~HIPTensor() { m_context->release(m_data, m_capacity); }

void HIPTensor::copy_to(std::shared_ptr<TensorImpl> dst) const {
    const size_t bytes = m_numel * calc_dtype_size(m_dtype);
    hip_check(hipMemcpyAsync(dst->data(), m_data, bytes, hipMemcpyDeviceToDevice, m_context->stream()), "hipMemcpyAsync D2D");
    m_context->wait();
}

std::unique_ptr<TensorImpl> HIPTensor::clone() const {
    auto out = std::make_unique<HIPTensor>(nullptr, m_numel, m_dtype, m_context);
    const size_t bytes = m_numel * calc_dtype_size(m_dtype);
    hip_check(hipMemcpyAsync(out->data(), m_data, bytes, hipMemcpyDeviceToDevice, m_context->stream()), "hipMemcpyAsync D2D");
    m_context->wait();
    return out;
}

std::unique_ptr<TensorImpl> HIPTensor::clone_as_contiguous(const Metadata& meta) const {
    auto out = std::make_unique<HIPTensor>(nullptr, meta.numel, m_dtype, m_context);
    if (meta.shape.size() > TV_MAX_DIMS) throw std::runtime_error("clone_as_contiguous: too many dimensions");
    tv_repack_args a{};
    a.ndim = static_cast<int32_t>(meta.shape.size());
    a.elem_size = static_cast<int32_t>(calc_dtype_size(m_dtype));
    for (int d = 0; d < a.ndim; ++d) {
        a.shape[d] = meta.shape[d];
        a.strides[d] = meta.strides[d];
    }
    a.src = static_cast<const char*>(m_data) + meta.offset * a.elem_size;
    a.dst = out->data();
    tv_check(tv_hip_repack(&a, m_context->stream()), "tv_hip_repack");
    m_context->wait();
    return out;
}

// ---- CPUTensor ---------------------------------------------------------------------------------

CPUTensor::CPUTensor(void* ptr, size_t numel, DataType dtype) : m_numel(numel), m_dtype(dtype) {
    const size_t bytes = numel * calc_dtype_size(dtype);
    m_data.reset(new char[bytes]);
    if (ptr) std::memcpy(m_data.get(), ptr, bytes);
}

void CPUTensor::copy_to(std::shared_ptr<TensorImpl> dst) const {
    std::memcpy(dst->data(), m_data.get(), m_numel * calc_dtype_size(m_dtype));
}

std::unique_ptr<TensorImpl> CPUTensor::clone() const {
    return std::make_unique<CPUTensor>(m_data.get(), m_numel, m_dtype);
}

// Gather of a strided view into row-major order (reference include/backend/cpu/cpu_tensor.cpp:32-63).
std::unique_ptr<TensorImpl> CPUTensor::clone_as_contiguous(const Metadata& meta) const {
    auto out = std::make_unique<CPUTensor>(nullptr, meta.numel, m_dtype);
    const size_t es = calc_dtype_size(m_dtype);
    const char* src = m_data.get() + meta.offset * es;
    char* dst = static_cast<char*>(out->data());
    const size_t nd = meta.shape.size();
    std::vector<int64_t> idx(nd, 0);
    for (size_t i = 0; i < meta.numel; ++i) {
        int64_t off = 0;
        for (size_t d = 0; d < nd; ++d) off += idx[d] * meta.strides[d];
        std::memcpy(dst + i * es, src + off * es, es);
        for (size_t d = nd; d-- > 0;) {
            if (++idx[d] < meta.shape[d]) break;
            idx[d] = 0;
        }
    }
    return out;
}

// ---- host <-> device ---------------------------------------------------------------------------

void copy_device_to_host(std::shared_ptr<TensorImpl> src, std::shared_ptr<TensorImpl> dst, DataType dtype) {
    auto ctx = hip_ctx_of(src);
    // dst is sized to the tensor; src may be a larger storage whose leading elements are the tensor.
    const size_t bytes = dst->numel() * calc_dtype_size(dtype);
    ctx->copy_d2h(dst->data(), src->data(), bytes);
}

void copy_host_to_device(std::shared_ptr<TensorImpl> src, std::shared_ptr<TensorImpl> dst, DataType dtype) {
    auto ctx = hip_ctx_of(dst);
    const size_t bytes = dst->numel() * calc_dtype_size(dtype);
    ctx->copy_h2d(dst->data(), src->data(), bytes);
}

// ---- registration (no GPU is touched until the first HIP tensor) --------------------------------

namespace {
struct HIPRegistrar {
    HIPRegistrar() {
        register_tensor_impl(Device::HIP, [](void* ptr, size_t numel, DataType dtype) -> std::shared_ptr<TensorImpl> {
            return std::make_shared<HIPTensor>(ptr, numel, dtype, HIPContext::get());
        });
        register_tensor_impl(Device::CPU, [](void* ptr, size_t numel, DataType dtype) -> std::shared_ptr<TensorImpl> {
            return std::make_shared<CPUTensor>(ptr, numel, dtype);
        });
    }
} hip_registrar;
} // namespace

// ---- MulImpl<HIP> ------------------------------------------------------------------------------

namespace ops {

namespace {
// Output tensor plus the C-ABI descriptor of a @ b (views through their strides and offsets).
Tensor pack_gemm(const Tensor& a, const Tensor& b, tv_gemm_args& args) {
    const bool a3 = a.dims() == 3, b3 = b.dims() == 3;
    const int64_t batch = a3 ? a.shape(0) : 1;
    const int64_t M = a.shape(-2), K = a.shape(-1), N = b.shape(-1);
    const DataType res = compute_type(a.dtype(), b.dtype());
    std::vector<int64_t> shape = a3 ? std::vector<int64_t>{batch, M, N} : std::vector<int64_t>{M, N};
    Tensor c(shape, res, Device::HIP);

    const std::vector<int64_t> sa = a.strides(), sb = b.strides(), sc = c.strides();
    args = tv_gemm_args{};
    args.dtype_a = static_cast<int32_t>(a.dtype());
    args.dtype_b = static_cast<int32_t>(b.dtype());
    args.dtype_c = static_cast<int32_t>(res);
    args.batch = batch;
    args.M = M;
    args.N = N;
    args.K = K;
    args.A = static_cast<const char*>(a.data()) + a.offset() * calc_dtype_size(a.dtype());
    args.sa_b = a3 ? sa[0] : 0;
    args.sa_m = sa[a3 ? 1 : 0];
    args.sa_k = sa[a3 ? 2 : 1];
    args.B = static_cast<const char*>(b.data()) + b.offset() * calc_dtype_size(b.dtype());
    args.sb_b = b3 ? sb[0] : 0; // rank-2 B with rank-3 A: broadcast over the batch
    args.sb_k = sb[b3 ? 1 : 0];
    args.sb_n = sb[b3 ? 2 : 1];
    args.C = c.data();
    args.sc_b = a3 ? sc[0] : 0;
    args.sc_m = sc[a3 ? 1 : 0];
    args.sc_n = sc[a3 ? 2 : 1];
    return c;
}
} // namespace

Tensor MulImpl<Device::HIP>::execute(const Tensor& a, const Tensor& b) {
    tv_gemm_args args{};
    Tensor c = pack_gemm(a, b, args);
    auto ctx = hip_ctx_of(c.get_impl());
    tv_check(tv_hip_gemm(&args, ctx->stream()), "ops::Mul");
    ctx->wait(); // the reference's op is synchronous (src/backend/cuda/mul.cu:122)
    return c;
}

Tensor MulBiasActImpl<Device::HIP>::execute(const Tensor& a, const Tensor& b, const Tensor* bias, Activation act) {
    tv_gemm_args args{};
    Tensor c = pack_gemm(a, b, args);
    tv_epilogue ep{};
    ep.act = static_cast<int32_t>(act);
    if (bias) {
        if (bias->device() != Device::HIP) throw std::runtime_error("MulBiasAct: bias must be on the HIP device");
        if (bias->dtype() != c.dtype())
            throw std::runtime_error("MulBiasAct: bias dtype must be the result dtype " +
                                     std::string(dtype_to_string(c.dtype())));
        // Align the bias's dimensions with C's trailing ones; missing leading dimensions broadcast.
        const size_t cd = c.dims(), bd = bias->dims();
        if (bd < 1 || bd > cd) throw std::runtime_error("MulBiasAct: bias must have 1 to rank(C) dimensions");
        const std::vector<int64_t> st = bias->strides();
        int64_t s3[3] = {0, 0, 0}; // batch, m, n strides of C's [b?, m, n]
        for (size_t i = 0; i < bd; ++i) {
            const size_t ci = cd - bd + i;
            if (bias->shape(i) != c.shape(ci))
                throw std::runtime_error("MulBiasAct: bias shape does not match the result's trailing dimensions");
            s3[3 - cd + ci] = bias->shape(i) == 1 ? 0 : st[i];
        }
        ep.bias = static_cast<const char*>(bias->data()) + bias->offset() * calc_dtype_size(bias->dtype());
        ep.sbias_b = s3[0];
        ep.sbias_m = s3[1];
        ep.sbias_n = s3[2];
    }
    auto ctx = hip_ctx_of(c.get_impl());
    tv_check(tv_hip_gemm_ex(&args, &ep, ctx->stream()), "ops::MulBiasAct");
    ctx->wait();
    return c;
}

// ---- TypecastImpl / FillImpl / RandomImpl<HIP> ---------------------------------------------------

Tensor TypecastImpl<Device::HIP>::execute(const Tensor& a, DataType dst_type) {
    const Tensor src = a.contiguous(); // device repack of a view; a dense tensor is shared as is
    Tensor out(src.shape(), dst_type, Device::HIP);
    auto ctx = hip_ctx_of(out.get_impl());
    const char* sp = static_cast<const char*>(src.data()) + src.offset() * calc_dtype_size(src.dtype());
    tv_check(tv_hip_typecast(sp, static_cast<int32_t>(src.dtype()), out.data(), static_cast<int32_t>(dst_type),
                             static_cast<int64_t>(src.numel()), ctx->stream()),
             "ops::Typecast");
    ctx->wait();
    return out;
}

// ---- TransposeImpl<HIP> --------------------------------------------------------------------------

Tensor TransposeImpl<Device::HIP>::execute(const Tensor& a, std::initializer_list<int64_t> axes) {
    return a.permute(std::vector<int64_t>(axes)).contiguous(); // clone_as_contiguous: tv_hip_repack
}

void TransposeImpl<Device::HIP>::execute(const Tensor& a, Tensor& dst, std::initializer_list<int64_t> axes) {
    if (a.device() != Device::HIP || dst.device() != Device::HIP)
        throw std::runtime_error("Transpose: a and dst must be HIP tensors");
    if (a.dtype() != dst.dtype())
        throw std::runtime_error("Transpose: dst dtype " + std::string(dtype_to_string(dst.dtype())) +
                                 " differs from the input's " + std::string(dtype_to_string(a.dtype())));
    const Tensor view = a.permute(std::vector<int64_t>(axes));
    // Both checks come before dst is touched: a caller that catches the error keeps dst as it was.
    if (view.dims() > TV_MAX_DIMS) throw std::runtime_error("Transpose: too many dimensions");
    // A permutation written over its own source would read elements it has already overwritten.
    if (dst.get_impl() == a.get_impl()) throw std::runtime_error("Transpose: dst shares storage with a");
    std::vector<int64_t> shape = view.shape();
    dst.reshape(shape); // as the reference (src/backend/cuda/transpose.cu:129-134); dst is dense after it
    const size_t es = calc_dtype_size(a.dtype());
    tv_repack_args r{};
    r.ndim = static_cast<int32_t>(view.dims());
    r.elem_size = static_cast<int32_t>(es);
    const std::vector<int64_t> st = view.strides();
    for (int d = 0; d < r.ndim; ++d) {
        r.shape[d] = shape[d];
        r.strides[d] = st[d];
    }
    r.src = static_cast<const char*>(view.data()) + view.offset() * es;
    r.dst = static_cast<char*>(dst.data()) + dst.offset() * es;
    auto ctx = hip_ctx_of(dst.get_impl());
    tv_check(tv_hip_repack(&r, ctx->stream()), "ops::Transpose");
    ctx->wait();
}

Tensor FillImpl<Device::HIP>::execute(const std::vector<int64_t>& shape, DataType dtype, float value) {
    Tensor out(shape, dtype, Device::HIP);
    auto ctx = hip_ctx_of(out.get_impl());
    tv_check(tv_hip_fill(out.data(), static_cast<int32_t>(dtype), static_cast<int64_t>(out.numel()), value, ctx->stream()),
             "ops::Fill");
    ctx->wait();
    return out;
}

Tensor RandomImpl<Device::HIP>::execute(const std::vector<int64_t>& shape, DataType dtype, float min, float max,
                                        uint64_t seed) {
    Tensor out(shape, dtype, Device::HIP);
    auto ctx = hip_ctx_of(out.get_impl());
    tv_check(tv_hip_random(out.data(), static_cast<int32_t>(dtype), static_cast<int64_t>(out.numel()), min, max, seed,
                           ctx->stream()),
             "ops::Random");
    ctx->wait();
    return out;
}

} // namespace ops
