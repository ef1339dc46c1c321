// Tensor: construction, strided views and device moves (reference src/tensor.cpp).
#include <algorithm>
#include <string>

#include "tensorvia/factory.h"
#include "tensorvia/ops.h"
#include "tensorvia/tensor.h"

using namespace via;

namespace {
void check_shape(const std::vector<int64_t>& shape) {
    if (shape.empty()) throw std::runtime_error("Tensor shape cannot be empty");
}
} // namespace

Tensor::Tensor() {
    m_meta.numel = 0;
    m_meta.device = Device::HIP;
    m_meta.dtype = DataType::FLOAT32;
    m_impl = nullptr;
}

Tensor::Tensor(std::vector<int64_t> shape, DataType dtype, Device device) {
    check_shape(shape);
    m_meta.device = device;
    m_meta.dtype = dtype;
    m_meta.shape = std::move(shape);
    m_meta.calculate_strides();
    m_meta.numel = calc_numel(m_meta.shape);
    m_impl = create_tensor_impl(m_meta.numel, dtype, device);
}
Tensor::Tensor(std::initializer_list<int64_t> shape, DataType dtype, Device device)
    : Tensor(std::vector<int64_t>(shape), dtype, device) {}
Tensor::Tensor(std::vector<int64_t> shape, DataType dtype) : Tensor(std::move(shape), dtype, Device::HIP) {}
Tensor::Tensor(std::initializer_list<int64_t> shape, DataType dtype)
    : Tensor(std::vector<int64_t>(shape), dtype, Device::HIP) {}

Tensor::Tensor(void* ptr, std::vector<int64_t> shape, DataType dtype, Device device) {
    check_shape(shape);
    if (ptr == nullptr) throw std::runtime_error("ptr can not nullptr");
    m_meta.device = device;
    m_meta.dtype = dtype;
    m_meta.shape = std::move(shape);
    m_meta.calculate_strides();
    m_meta.numel = calc_numel(m_meta.shape);
    m_impl = create_tensor_impl(ptr, m_meta.numel, dtype, device);
}
Tensor::Tensor(void* ptr, std::initializer_list<int64_t> shape, DataType dtype, Device device)
    : Tensor(ptr, std::vector<int64_t>(shape), dtype, device) {}

// A copy of a view is a contiguous tensor holding the view's elements.
Tensor::Tensor(const Tensor& other) {
    if (!other.m_impl) {
        m_meta = other.m_meta;
        return;
    }
    Tensor c = other.clone();
    m_meta = std::move(c.m_meta);
    m_impl = std::move(c.m_impl);
}
Tensor::Tensor(Tensor&& other) noexcept : m_meta(std::move(other.m_meta)), m_impl(std::move(other.m_impl)) {}

Tensor& Tensor::operator=(const Tensor& other) {
    if (this != &other) {
        Tensor c(other);
        m_meta = std::move(c.m_meta);
        m_impl = std::move(c.m_impl);
    }
    return *this;
}
Tensor& Tensor::operator=(Tensor&& other) noexcept {
    if (this != &other) {
        m_meta = std::move(other.m_meta);
        m_impl = std::move(other.m_impl);
    }
    return *this;
}

void* Tensor::data() { return m_impl ? m_impl->data() : nullptr; }
const void* Tensor::data() const { return m_impl ? m_impl->data() : nullptr; }
Device Tensor::device() const { return m_meta.device; }
DataType Tensor::dtype() const { return m_meta.dtype; }
size_t Tensor::dims() const { return m_meta.shape.size(); }
std::vector<int64_t> Tensor::shape() const { return m_meta.shape; }
int64_t Tensor::shape(int i) const {
    const int n = static_cast<int>(m_meta.shape.size());
    if (i < -n || i >= n) throw std::out_of_range("shape: dimension index out of range");
    return m_meta.shape[i < 0 ? i + n : i];
}
int64_t Tensor::shape(int i) { return static_cast<const Tensor&>(*this).shape(i); }
int64_t Tensor::strides(int i) const {
    const int n = static_cast<int>(m_meta.strides.size());
    if (i < -n || i >= n) throw std::out_of_range("strides: dimension index out of range");
    return m_meta.strides[i < 0 ? i + n : i];
}
std::vector<int64_t> Tensor::strides() const { return m_meta.strides; }
std::shared_ptr<TensorImpl> Tensor::get_impl() const { return m_impl; }
void Tensor::set_impl(std::shared_ptr<TensorImpl> impl, DataType new_dtype) {
    m_impl = std::move(impl);
    m_meta.dtype = new_dtype;
    m_meta.offset = 0;
    m_meta.calculate_strides();
}
Tensor Tensor::empty_like(Tensor& tensor) const { return Tensor(tensor.shape(), tensor.dtype(), tensor.device()); }

bool Tensor::is_contiguous() const {
    if (m_meta.shape.empty()) return true;
    int64_t expect = 1;
    for (int i = static_cast<int>(m_meta.shape.size()) - 1; i >= 0; --i) {
        if (m_meta.shape[i] != 1 && m_meta.strides[i] != expect) return false;
        expect *= m_meta.shape[i];
    }
    return true;
}

Tensor Tensor::clone() const {
    if (!m_impl) return Tensor();
    Metadata meta = m_meta;
    meta.offset = 0;
    meta.calculate_strides();
    if (is_contiguous() && m_meta.offset == 0 && m_impl->numel() == m_meta.numel)
        return Tensor(std::shared_ptr<TensorImpl>(m_impl->clone()), std::move(meta));
    return Tensor(std::shared_ptr<TensorImpl>(m_impl->clone_as_contiguous(m_meta)), std::move(meta));
}

Tensor Tensor::contiguous() const {
    if (is_contiguous() && m_meta.offset == 0) return Tensor(m_impl, m_meta);
    return clone();
}
Tensor& Tensor::to_contiguous() {
    if (!(is_contiguous() && m_meta.offset == 0)) *this = clone();
    return *this;
}

Tensor Tensor::_make_view(std::vector<int64_t> shape, std::vector<int64_t> strides, int64_t offset) const {
    Metadata meta;
    meta.numel = calc_numel(shape);
    meta.dtype = m_meta.dtype;
    meta.device = m_meta.device;
    meta.offset = offset;
    meta.shape = std::move(shape);
    meta.strides = std::move(strides);
    return Tensor(m_impl, std::move(meta));
}

Tensor Tensor::t() {
    if (m_meta.shape.size() != 2) throw std::invalid_argument("t() needs a 2-d tensor");
    return _make_view({m_meta.shape[1], m_meta.shape[0]}, {m_meta.strides[1], m_meta.strides[0]}, m_meta.offset);
}

Tensor Tensor::permute(std::initializer_list<int64_t> dims) const { return permute(std::vector<int64_t>(dims)); }
Tensor Tensor::permute(const std::vector<int64_t>& dims) const {
    const int64_t nd = static_cast<int64_t>(m_meta.shape.size());
    if (static_cast<int64_t>(dims.size()) != nd)
        throw std::invalid_argument("permute: number of dims (" + std::to_string(dims.size()) +
                                    ") doesn't match tensor dim (" + std::to_string(nd) + ")");
    std::vector<bool> seen(nd, false);
    std::vector<int64_t> shape, strides;
    for (int64_t d : dims) {
        const int64_t n = d >= 0 ? d : d + nd;
        if (n < 0 || n >= nd) throw std::invalid_argument("Dimension out of range");
        if (seen[n]) throw std::invalid_argument("Duplicate dimension in permute");
        seen[n] = true;
        shape.push_back(m_meta.shape[n]);
        strides.push_back(m_meta.strides[n]);
    }
    return _make_view(std::move(shape), std::move(strides), m_meta.offset);
}

Tensor Tensor::slice(const std::vector<std::pair<int64_t, int64_t>>& ranges) const {
    if (ranges.size() > m_meta.shape.size()) throw std::invalid_argument("Too many slice ranges");
    std::vector<int64_t> shape = m_meta.shape;
    int64_t offset = m_meta.offset;
    for (size_t i = 0; i < ranges.size(); ++i) {
        const int64_t n = m_meta.shape[i];
        int64_t s = ranges[i].first < 0 ? ranges[i].first + n : ranges[i].first;
        int64_t e = ranges[i].second < 0 ? ranges[i].second + n : ranges[i].second;
        s = std::clamp<int64_t>(s, 0, n);
        e = std::clamp<int64_t>(e, s, n);
        shape[i] = e - s;
        offset += s * m_meta.strides[i];
    }
    return _make_view(std::move(shape), m_meta.strides, offset);
}

Tensor Tensor::view(std::initializer_list<int64_t> new_shape) { return view(std::vector<int64_t>(new_shape)); }
Tensor Tensor::view(std::vector<int64_t> new_shape) {
    if (!is_contiguous()) throw std::invalid_argument("view: tensor is not contiguous. Call .contiguous() first.");
    int64_t infer = -1, known = 1;
    for (size_t i = 0; i < new_shape.size(); ++i) {
        if (new_shape[i] == -1) {
            if (infer != -1) throw std::invalid_argument("Only one dimension can be -1");
            infer = static_cast<int64_t>(i);
        } else if (new_shape[i] < 0) {
            throw std::invalid_argument("Negative dimension size not allowed (except -1)");
        } else {
            known *= new_shape[i];
        }
    }
    if (infer != -1) {
        if (known == 0 || static_cast<int64_t>(numel()) % known != 0)
            throw std::invalid_argument("view: invalid inferred size for -1 (numel mismatch)");
        new_shape[infer] = static_cast<int64_t>(numel()) / known;
        known = static_cast<int64_t>(numel());
    }
    if (known != static_cast<int64_t>(numel())) throw std::invalid_argument("view: new shape numel does not match original numel");
    Metadata m;
    m.shape = new_shape;
    m.calculate_strides();
    return _make_view(std::move(new_shape), std::move(m.strides), m_meta.offset);
}

void Tensor::reshape(std::vector<int64_t>& newshape) {
    if (calc_numel(newshape) != m_meta.numel)
        throw std::runtime_error("new elements count must be equal to old elements count. " +
                                 std::to_string(m_meta.numel) + " != " + std::to_string(calc_numel(newshape)));
    if (!is_contiguous()) to_contiguous();
    m_meta.shape = newshape;
    m_meta.calculate_strides();
}
void Tensor::reshape(std::initializer_list<int64_t> newshape) {
    std::vector<int64_t> s(newshape);
    reshape(s);
}

Tensor& Tensor::squeeze(int dim) {
    std::vector<int64_t> shape, strides;
    const int nd = static_cast<int>(m_meta.shape.size());
    for (int i = 0; i < nd; ++i) {
        const bool drop = m_meta.shape[i] == 1 && (dim == -1 || i == dim);
        if (!drop) {
            shape.push_back(m_meta.shape[i]);
            strides.push_back(m_meta.strides[i]);
        }
    }
    if (shape.empty()) {
        shape.push_back(1);
        strides.push_back(1);
    }
    m_meta.shape = std::move(shape);
    m_meta.strides = std::move(strides);
    return *this;
}
Tensor& Tensor::unsqueeze(size_t dim) {
    if (dim > m_meta.shape.size()) throw std::out_of_range("unsqueeze: dimension out of range");
    const int64_t stride = dim < m_meta.shape.size() ? m_meta.strides[dim] * m_meta.shape[dim] : 1;
    m_meta.shape.insert(m_meta.shape.begin() + dim, 1);
    m_meta.strides.insert(m_meta.strides.begin() + dim, stride);
    return *this;
}

// HIP -> CPU: the view's elements become a contiguous host tensor.
void Tensor::to_host() {
    if (m_meta.device == Device::CPU) return;
    Tensor dense = contiguous();
    auto host = create_tensor_impl(m_meta.numel, m_meta.dtype, Device::CPU);
    copy_device_to_host(dense.m_impl, host, m_meta.dtype);
    m_impl = std::move(host);
    m_meta.device = Device::CPU;
    m_meta.offset = 0;
    m_meta.calculate_strides();
}

// CPU -> HIP.
void Tensor::to_device(uint32_t) {
    if (m_meta.device != Device::CPU) return;
    Tensor dense = contiguous();
    auto dev = create_tensor_impl(m_meta.numel, m_meta.dtype, Device::HIP);
    copy_host_to_device(dense.m_impl, dev, m_meta.dtype);
    m_impl = std::move(dev);
    m_meta.device = Device::HIP;
    m_meta.offset = 0;
    m_meta.calculate_strides();
}

void Tensor::to_type(DataType dst) { ops::Typecast(*this, dst); }
Tensor Tensor::to_type_(DataType dst) { return ops::Typecast(static_cast<const Tensor&>(*this), dst); }

template <typename T> T Tensor::at(std::initializer_list<int64_t> idxs) {
    if (m_meta.device != Device::CPU) throw std::runtime_error("Tensor device must be CPU");
    if (idxs.size() != m_meta.shape.size()) throw std::runtime_error("Tensor index size must be equal to tensor shape size");
    int64_t index = m_meta.offset;
    int d = 0;
    for (int64_t i : idxs) {
        if (i < 0 || i >= m_meta.shape[d]) throw std::runtime_error("index out of range");
        index += i * m_meta.strides[d++];
    }
    T out{};
    dispatch_dtype(m_meta.dtype, [&](auto id) {
        using E = typename decltype(id)::type;
        out = static_cast<T>(static_cast<const E*>(m_impl->data())[index]);
    });
    return out;
}
template <typename T> T Tensor::operator[](std::initializer_list<int64_t> idxs) { return at<T>(idxs); }

#define TV_AT(T) template T Tensor::at<T>(std::initializer_list<int64_t>); \
                 template T Tensor::operator[]<T>(std::initializer_list<int64_t>);
TV_AT(int8_t) TV_AT(int16_t) TV_AT(int32_t) TV_AT(int64_t) TV_AT(float) TV_AT(double)
#undef TV_AT

Tensor Tensor::Zeros(std::initializer_list<int64_t> shape, DataType dtype) { return ops::Zeros(shape, dtype); }
Tensor Tensor::Zeros(std::vector<int64_t> shape, DataType dtype) { return ops::Zeros(shape, dtype); }
Tensor Tensor::Ones(std::initializer_list<int64_t> shape, DataType dtype) { return ops::Ones(shape, dtype); }
Tensor Tensor::Ones(std::vector<int64_t> shape, DataType dtype) { return ops::Ones(shape, dtype); }
Tensor Tensor::Fill(std::initializer_list<int64_t> shape, float value, DataType dtype) { return ops::Fill(shape, dtype, value); }
Tensor Tensor::Fill(std::vector<int64_t> shape, float value, DataType dtype) { return ops::Fill(shape, dtype, value); }
Tensor Tensor::Random(std::initializer_list<int64_t> shape, float min, float max, DataType dtype) {
    return ops::Random(shape, dtype, min, max);
}
Tensor Tensor::Random(std::vector<int64_t> shape, float min, float max, DataType dtype) {
    return ops::Random(shape, dtype, min, max);
}
Tensor Tensor::Random(std::vector<int64_t> shape, float min, float max, DataType dtype, uint64_t seed) {
    return ops::Random(shape, dtype, min, max, seed);
}
