// Operators of the HIP backend's hot path, API-compatible with the reference's
// include/core/ops.h (ops::Mul :57-59, Transpose :102-104, Typecast :99-100, initialisers :27-30).
#pragma once

#include <initializer_list>
#include <vector>

#include "tensor.h"
#include "types.h"

#define OPS_API

namespace ops {

// [m,k] @ [k,n] -> [m,n];  [b,m,k] @ [b,k,n] -> [b,m,n];  and, beyond the reference,
// [b,m,k] @ [k,n] -> [b,m,n] with B broadcast over the batch.  Views (slices, permutes, t())
// are consumed through their strides.  The result dtype is compute_type(a, b); synchronous.
OPS_API Tensor Mul(const Tensor& a, const Tensor& b);
// Spelling used by the reference README (README.md:116); same operation.
OPS_API Tensor matmul(const Tensor& a, const Tensor& b);

// Beyond the reference: act(Mul(a, b) + bias) in one pass, the bias added and the activation
// applied to the fp32 accumulator before the single rounding to the result dtype (the reference
// composes ops::Mul, ops::Add and ops::Relu/Silu/Tanh/Sigmoid, src/ops.cpp:330-352, 678-780).
// bias: nullptr, or a tensor of the result dtype shaped [n], [m, n] or [b, m, n] (broadcast over
// the missing leading dimensions).  Float results only (fp32, bf16, fp16 inputs).
enum class Activation { None = 0, Relu = 1, Silu = 2, Sigmoid = 3, Tanh = 4 };
OPS_API Tensor MulBiasAct(const Tensor& a, const Tensor& b, const Tensor* bias, Activation act);

// Materialising N-d transpose (reference src/ops.cpp:1380-1402).
OPS_API Tensor Transpose(const Tensor& a, std::initializer_list<int64_t> axes);
// Into an existing tensor (reference include/core/ops.h:105, src/ops.cpp:1354-1378): dst must hold
// as many elements as a; it is reshaped to the permuted shape and overwritten.  HIP tensors, dst of
// a's dtype and not sharing a's storage.
OPS_API void Transpose(const Tensor& a, Tensor& dst, std::initializer_list<int64_t> axes);
OPS_API void Transpose(Tensor& a); // 2-d, in place
// Zero-copy spelling used by the reference README (README.md:137): the permuted view.
OPS_API Tensor transpose(const Tensor& a, std::initializer_list<int64_t> axes);

OPS_API void Typecast(Tensor& a, via::DataType dst_type);
OPS_API Tensor Typecast(const Tensor& a, via::DataType dst_type);

OPS_API Tensor Ones(const std::vector<int64_t>& shape, via::DataType dtype);
OPS_API Tensor Zeros(const std::vector<int64_t>& shape, via::DataType dtype);
OPS_API Tensor Fill(const std::vector<int64_t>& shape, via::DataType dtype, float value);
OPS_API Tensor Random(const std::vector<int64_t>& shape, via::DataType dtype, float min, float max);
OPS_API Tensor Random(const std::vector<int64_t>& shape, via::DataType dtype, float min, float max, uint64_t seed);

namespace detail {
// The host generator behind the seeded Random: n elements of stream `seed` into dst, stored as
// `dtype`.
OPS_API void random_fill(void* dst, size_t n, via::DataType dtype, float min, float max, uint64_t seed);
} // namespace detail

} // namespace ops
