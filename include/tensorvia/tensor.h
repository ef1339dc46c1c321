// Tensor with strided views, API-compatible with the reference's include/core/tensor.h:12-156.
//
// Differences, each deliberate:
//  * Device::HIP is the default device of this build (the reference picks its compiled backend,
//    src/tensor.cpp:10-28);
//  * offset() is public: ops::Mul passes view offsets to the kernels (Metadata is private);
//  * views keep their offset through t() / permute() (the reference resets it to 0,
//    src/tensor.cpp:220,282), and copying a view copies the view's elements into a contiguous
//    tensor (the reference clones the whole storage and resets the strides, tensor.cpp:396-403);
//  * Random takes an optional seed and is reproducible (the reference seeds from the clock,
//    src/backend/cpu/initializer.cpp:22-24).
#pragma once

#include <array>
#include <cstddef>
#include <cstring>
#include <initializer_list>
#include <memory>
#include <vector>

#include "type_traits.h"

class ContextImpl;

struct Metadata {
    size_t numel = 0;             // elements of the view
    int64_t offset = 0;           // first element of the view inside the storage
    via::Device device = via::Device::HIP;
    via::DataType dtype = via::DataType::FLOAT32;
    std::vector<int64_t> shape;
    std::vector<int64_t> strides; // element strides
    void calculate_strides() {
        strides.assign(shape.size(), 1);
        for (int i = static_cast<int>(shape.size()) - 2; i >= 0; --i) strides[i] = strides[i + 1] * shape[i + 1];
    }
};

class TensorImpl {
public:
    virtual ~TensorImpl() = default;
    virtual void* data() = 0;
    virtual size_t numel() const = 0;
    virtual const void* data() const = 0;
    virtual void copy_to(std::shared_ptr<TensorImpl> dst) const = 0;
    virtual std::unique_ptr<TensorImpl> clone() const = 0;
    // Contiguous copy of the view `meta` describes (offset and strides honoured).
    virtual std::unique_ptr<TensorImpl> clone_as_contiguous(const Metadata&) const = 0;
    virtual std::shared_ptr<ContextImpl> context() const = 0;
};

class Tensor {
private:
    Metadata m_meta;
    std::shared_ptr<TensorImpl> m_impl;

    Tensor(std::shared_ptr<TensorImpl> impl, Metadata meta) : m_meta(std::move(meta)), m_impl(std::move(impl)) {}
    Tensor _make_view(std::vector<int64_t> shape, std::vector<int64_t> strides, int64_t offset) const;

public:
    // Storage base pointer (without the view offset, as in the reference); see offset().
    void* data();
    const void* data() const;
    int64_t offset() const { return m_meta.offset; }

    Tensor clone() const;
    via::Device device() const;
    via::DataType dtype() const;

    void to_type(via::DataType);
    Tensor to_type_(via::DataType);

    void to_host();
    void to_device(uint32_t id = 0);

    int64_t strides(int i) const;
    std::vector<int64_t> strides() const;

    Tensor& to_contiguous();
    Tensor contiguous() const;
    bool is_contiguous() const;

    size_t dims() const;
    size_t numel() const { return m_meta.numel; }
    Tensor empty_like(Tensor& tensor) const;

    std::shared_ptr<TensorImpl> get_impl() const;
    void set_impl(std::shared_ptr<TensorImpl> impl, via::DataType new_dtype);

    Tensor view(std::vector<int64_t> new_shape_list);
    Tensor view(std::initializer_list<int64_t> new_shape);

    Tensor();
    Tensor(const Tensor& other);
    Tensor(Tensor&& other) noexcept;
    Tensor(std::vector<int64_t> shape, via::DataType dtype);
    Tensor(std::initializer_list<int64_t> shape, via::DataType dtype);
    Tensor(std::vector<int64_t> shape, via::DataType dtype, via::Device device);
    Tensor(std::initializer_list<int64_t> shape, via::DataType dtype, via::Device device);
    // Deep copy of host memory at ptr (numel elements of dtype) into a tensor on `device`.
    Tensor(void* ptr, std::vector<int64_t> shape, via::DataType dtype, via::Device device);
    Tensor(void* ptr, std::initializer_list<int64_t> shape, via::DataType dtype, via::Device device);
    template <typename T> Tensor(std::vector<T>& vec, std::initializer_list<int64_t> shape);
    template <typename T> Tensor(std::vector<T>& vec, std::vector<int64_t> shape);

    Tensor& operator=(const Tensor& other);
    Tensor& operator=(Tensor&& other) noexcept;

    int64_t shape(int i);
    int64_t shape(int i) const;
    std::vector<int64_t> shape() const;

    Tensor t();
    Tensor permute(const std::vector<int64_t>& dims) const;
    Tensor permute(std::initializer_list<int64_t> dims) const;
    Tensor slice(const std::vector<std::pair<int64_t, int64_t>>& ranges) const;

    // Shape changes of a contiguous tensor (the data layout does not change).
    void reshape(std::vector<int64_t>& newshape);
    void reshape(std::initializer_list<int64_t> newshape);

    Tensor& squeeze(int dim = -1);
    Tensor& unsqueeze(size_t dim);

    // Element access (CPU tensors).
    template <typename T> T at(std::initializer_list<int64_t> idxs);
    template <typename T> T operator[](std::initializer_list<int64_t> idxs);

    static Tensor Zeros(std::initializer_list<int64_t> shape, via::DataType dtype = via::DataType::FLOAT32);
    static Tensor Zeros(std::vector<int64_t> shape, via::DataType dtype = via::DataType::FLOAT32);
    static Tensor Ones(std::initializer_list<int64_t> shape, via::DataType dtype = via::DataType::FLOAT32);
    static Tensor Ones(std::vector<int64_t> shape, via::DataType dtype = via::DataType::FLOAT32);
    static Tensor Fill(std::initializer_list<int64_t> shape, float value, via::DataType dtype = via::DataType::FLOAT32);
    static Tensor Fill(std::vector<int64_t> shape, float value, via::DataType dtype);
    static Tensor Random(std::initializer_list<int64_t> shape, float min = 0.0f, float max = 1.0f,
                         via::DataType dtype = via::DataType::FLOAT32);
    static Tensor Random(std::vector<int64_t> shape, float min = 0.0f, float max = 1.0f,
                         via::DataType dtype = via::DataType::FLOAT32);
    // Seeded form: element i depends only on (seed, i); uniform reals / inclusive integers.
    static Tensor Random(std::vector<int64_t> shape, float min, float max, via::DataType dtype, uint64_t seed);
};

// Tensor(std::vector<T>&, shape): dtype from T, storage on the default device.
namespace via::detail {
template <typename T> constexpr DataType dtype_of() {
    if constexpr (std::is_same_v<T, float32>) return DataType::FLOAT32;
    else if constexpr (std::is_same_v<T, float64>) return DataType::FLOAT64;
    else if constexpr (std::is_same_v<T, int64_t>) return DataType::INT64;
    else if constexpr (std::is_same_v<T, int32_t>) return DataType::INT32;
    else if constexpr (std::is_same_v<T, int16_t>) return DataType::INT16;
    else if constexpr (std::is_same_v<T, int8_t>) return DataType::INT8;
    else if constexpr (std::is_same_v<T, bfloat16>) return DataType::BFLOAT16;
    else if constexpr (std::is_same_v<T, float16>) return DataType::FLOAT16;
    else static_assert(sizeof(T) == 0, "unsupported element type");
}
} // namespace via::detail

template <typename T>
Tensor::Tensor(std::vector<T>& vec, std::vector<int64_t> shape)
    : Tensor(static_cast<void*>(vec.data()), std::move(shape), via::detail::dtype_of<T>(), via::Device::HIP) {
    if (vec.size() != m_meta.numel) throw std::runtime_error("Tensor: vector size does not match the shape");
}
template <typename T>
Tensor::Tensor(std::vector<T>& vec, std::initializer_list<int64_t> shape)
    : Tensor(vec, std::vector<int64_t>(shape)) {}
