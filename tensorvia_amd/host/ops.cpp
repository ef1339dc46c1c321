// Operator entry points of the HIP backend (reference src/ops.cpp): validation, then dispatch.
#include <cstring>
#include <string>

#include "tensorvia/factory.h"
#include "tensorvia/hip_backend.h"
#include "tensorvia/ops.h"

using namespace via;

namespace ops {

// Validation restates the reference's (src/ops.cpp:540-556), in its order and with its messages,
// with one extension: a rank-3 A may multiply a rank-2 B (B broadcast over the batch), which the
// reference rejects as a rank mismatch.
namespace {
void check_mul_operands(const Tensor& a, const Tensor& b) {
    if (a.device() != b.device()) throw std::runtime_error("Tensors a and b device mismatch!"); // :542-543
    const size_t ra = a.dims(), rb = b.dims();
    if (rb != ra && !(ra == 3 && rb == 2)) // :544-545
        throw std::runtime_error("Tensors a and b must have the same rank,but got " + std::to_string(ra) + " and " +
                                 std::to_string(rb));
    if (ra != 2 && ra != 3) throw std::runtime_error("Tensors a and b dims must be 2 or 3,but got " + std::to_string(ra)); // :546-547
    if (ra == 3) { // :548-552
        if (rb == 3 && a.shape(0) != b.shape(0)) throw std::runtime_error("Tensors a and b must have the same batch size");
        if (a.shape(2) != b.shape(-2))
            throw std::runtime_error("Tensors common dim must match,but " + std::to_string(a.shape(2)) + " and " +
                                     std::to_string(b.shape(-2)));
    } else if (a.shape(1) != b.shape(0)) { // :553-556; the reference's message names dimension 0 of both
        throw std::runtime_error("Tensors common dim must match,but " + std::to_string(a.shape(0)) + " and " +
                                 std::to_string(b.shape(0)));
    }
    if (a.device() == Device::CPU)
        throw std::runtime_error("ops::Mul on CPU tensors runs the reference CPU backend, which is not part of the "
                                 "HIP build; move both tensors with to_device()");
}
} // namespace

Tensor Mul(const Tensor& a, const Tensor& b) {
    check_mul_operands(a, b);
    return MulImpl<Device::HIP>::execute(a, b);
}

Tensor matmul(const Tensor& a, const Tensor& b) { return Mul(a, b); }

Tensor MulBiasAct(const Tensor& a, const Tensor& b, const Tensor* bias, Activation act) {
    check_mul_operands(a, b);
    return MulBiasActImpl<Device::HIP>::execute(a, b, bias, act);
}

Tensor transpose(const Tensor& a, std::initializer_list<int64_t> axes) {
    if (a.dims() != axes.size()) throw std::runtime_error("transpose shape and axes size not match");
    return a.permute(std::vector<int64_t>(axes));
}

// Validation as the reference's (src/ops.cpp:1380-1385); device tensors are permuted on the device.
Tensor Transpose(const Tensor& a, std::initializer_list<int64_t> axes) {
    if (a.dims() == 0) throw std::runtime_error("Input tensor must be not null.");
    if (a.dims() != axes.size()) throw std::runtime_error("transpose shape and axes size not match");
    if (a.device() == Device::HIP) return TransposeImpl<Device::HIP>::execute(a, axes);
    return a.permute(std::vector<int64_t>(axes)).contiguous(); // host tensors: host gather
}

// Validation as the reference's (src/ops.cpp:1354-1361): dst is reshaped to the permuted shape and
// receives the permuted elements.
void Transpose(const Tensor& a, Tensor& dst, std::initializer_list<int64_t> axes) {
    if (a.dims() == 0) throw std::runtime_error("Input tensor must be not null.");
    if (a.dims() != axes.size()) throw std::runtime_error("transpose shape and axes size not match");
    if (a.numel() != dst.numel()) throw std::runtime_error("dst numel not enough");
    if (a.device() != Device::HIP)
        throw std::runtime_error("ops::Transpose into dst runs on HIP tensors; move both with to_device()");
    TransposeImpl<Device::HIP>::execute(a, dst, axes);
}

void Transpose(Tensor& a) {
    if (a.numel() == 0) throw std::runtime_error("tensor a is null");
    if (a.dims() != 2) throw std::runtime_error("transpose only support 2D tensor");
    a = a.t().contiguous();
}

// ---- typecasts (host conversion; reference src/backend/cpu/typecast.cpp:48-98) ----------------

namespace {
template <typename S, typename D> void cast_n(const void* src, void* dst, size_t n) {
    const S* s = static_cast<const S*>(src);
    D* d = static_cast<D*>(dst);
    for (size_t i = 0; i < n; ++i) d[i] = static_cast<D>(static_cast<compute_type_t<S>>(s[i]));
}

Tensor cast_tensor(const Tensor& a, DataType dst) {
    Tensor host = a.contiguous();
    const Device dev = a.device();
    host.to_host();
    Tensor out(host.shape(), dst, Device::CPU);
    dispatch_dtype(a.dtype(), [&](auto sid) {
        using S = typename decltype(sid)::type;
        dispatch_dtype(dst, [&](auto did) {
            using D = typename decltype(did)::type;
            cast_n<S, D>(host.data(), out.data(), host.numel());
        });
    });
    if (dev != Device::CPU) out.to_device();
    return out;
}
} // namespace

// Validation as the reference's (src/ops.cpp:1277-1300); device tensors cast on the device,
// host tensors on the host.
Tensor Typecast(const Tensor& a, DataType dst_type) {
    if (a.numel() == 0) throw std::runtime_error("tensor a is null");
    if (!is_cast_valid(a.dtype(), dst_type))
        throw std::runtime_error("Invalid typecast from " + std::string(dtype_to_string(a.dtype())) + " to " +
                                 std::string(dtype_to_string(dst_type)));
    if (a.dtype() == dst_type) return a;
    if (a.device() == Device::HIP) return TypecastImpl<Device::HIP>::execute(a, dst_type);
    return cast_tensor(a, dst_type);
}

void Typecast(Tensor& a, DataType dst_type) { a = Typecast(static_cast<const Tensor&>(a), dst_type); }

// ---- initialisers ------------------------------------------------------------------------------
// Values are produced on the device (tv_hip_fill / tv_hip_random).  The host generator below
// (detail::random_fill) produces the same stream for host buffers.

namespace {
constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;
inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t g_next_seed = 0x5EEDull;
} // namespace

Tensor Fill(const std::vector<int64_t>& shape, DataType dtype, float value) {
    if (shape.empty()) throw std::runtime_error("ops::Fill: shape is empty");
    return FillImpl<Device::HIP>::execute(shape, dtype, value);
}
Tensor Zeros(const std::vector<int64_t>& shape, DataType dtype) {
    if (shape.empty()) throw std::runtime_error("ops::Zeros: shape is empty");
    return FillImpl<Device::HIP>::execute(shape, dtype, 0.0f);
}
Tensor Ones(const std::vector<int64_t>& shape, DataType dtype) {
    if (shape.empty()) throw std::runtime_error("ops::Ones: shape is empty");
    return FillImpl<Device::HIP>::execute(shape, dtype, 1.0f);
}

// Counter-based SplitMix64 stream: element i of stream `seed` is mix64(mix64(seed + G) + (i+1) G).
// Reals: min + (max - min) * u in fp32, u = top 24 bits / 2^24, then rounded to the element type
// (round to nearest even for half types).  Integers: inclusive [min, max] by multiply-shift of
// the top 32 bits.  The same stream is produced by tensorvia_amd/rng.py.
namespace detail {
void random_fill(void* p, size_t n, DataType dtype, float min, float max, uint64_t seed) {
    const uint64_t key = mix64(seed + kGamma);
    dispatch_dtype(dtype, [&](auto id) {
        using E = typename decltype(id)::type;
        E* e = static_cast<E*>(p);
        if constexpr (std::is_integral_v<E>) {
            const int64_t lo = static_cast<int64_t>(min), hi = static_cast<int64_t>(max);
            const uint64_t span = static_cast<uint64_t>(hi - lo + 1);
            for (size_t i = 0; i < n; ++i) {
                const uint64_t top = mix64(key + (i + 1) * kGamma) >> 32;
                e[i] = static_cast<E>(lo + static_cast<int64_t>((top * span) >> 32));
            }
        } else {
#pragma clang fp contract(off)
            const float span = static_cast<float>(static_cast<double>(max) - static_cast<double>(min));
            for (size_t i = 0; i < n; ++i) {
                const float u = static_cast<float>(mix64(key + (i + 1) * kGamma) >> 40) * 0x1p-24f;
                e[i] = static_cast<E>(min + span * u);
            }
        }
    });
}
} // namespace detail

Tensor Random(const std::vector<int64_t>& shape, DataType dtype, float min, float max, uint64_t seed) {
    if (shape.empty()) throw std::runtime_error("ops::Random: shape is empty");
    if (min > max) throw std::runtime_error("Random: min must not exceed max");
    return RandomImpl<Device::HIP>::execute(shape, dtype, min, max, seed);
}

Tensor Random(const std::vector<int64_t>& shape, DataType dtype, float min, float max) {
    return Random(shape, dtype, min, max, g_next_seed++);
}

} // namespace ops
