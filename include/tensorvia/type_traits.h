// Tensorvia core enums and dtype rules, API-compatible with the reference's
// include/core/type_traits.h, plus Device::HIP for the MI355X backend.
//
// Reference counterparts: OpType / op_to_string (type_traits.h:49-115), Device (116-121),
// DataType (123-132), device_to_string / dtype_to_string (134-158), calc_dtype_size (162-174),
// data_as_const_variant / dispatch_dtype (177-234), valid_casts / is_cast_valid (237-291),
// compute_type (270-287), calc_numel (292-299), LOG_* and RUNNING_TIME (21-45).
// The reference builds these on C++23 <format>/<print>/<stdfloat>; this header keeps the same
// names and behaviour on C++20 library features.
#pragma once

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <ctime>
#include <iomanip>
#include <iostream>
#include <set>
#include <stdexcept>
#include <string>
#include <string_view>
#include <type_traits>
#include <utility>
#include <variant>
#include <vector>

#include "types.h"

#define TV_COLOR_RESET "\033[0m"
#define TV_COLOR_RED "\033[31m"
#define TV_COLOR_YELLOW "\033[33m"
#define TV_COLOR_CYAN "\033[36m"

#define LOG_BASE(level, color, msg)                                                                       \
    do {                                                                                                  \
        const std::time_t tv_log_t_ = std::chrono::system_clock::to_time_t(std::chrono::system_clock::now()); \
        std::tm tv_log_tm_;                                                                               \
        localtime_r(&tv_log_t_, &tv_log_tm_);                                                             \
        std::cerr << color << "[" << level << "] " << std::put_time(&tv_log_tm_, "%Y-%m-%d %H:%M:%S")    \
                  << " [" << __FILE__ << ":" << __LINE__ << "] (" << __func__ << "): " << msg             \
                  << TV_COLOR_RESET << std::endl;                                                         \
    } while (0)

#define LOG_INFO(msg) LOG_BASE("INFO", TV_COLOR_CYAN, msg)
#define LOG_WARN(msg) LOG_BASE("WARN", TV_COLOR_YELLOW, msg)
#define LOG_ERROR(msg) LOG_BASE("ERROR", TV_COLOR_RED, msg)

// Wall time of one expression, printed in milliseconds (reference type_traits.h:38-45).
#define RUNNING_TIME(expr)                                                                   \
    do {                                                                                     \
        const auto tv_rt_start_ = std::chrono::steady_clock::now();                          \
        expr;                                                                                \
        const std::chrono::duration<double, std::milli> tv_rt_ms_ =                          \
            std::chrono::steady_clock::now() - tv_rt_start_;                                 \
        std::cout << "Execution time: " << tv_rt_ms_.count() << "ms" << std::endl;           \
    } while (0)

namespace via {

enum class OpType {
    Fill, Random,
    Slice,
    Matmul,
    Add, Sub, Dot, Div,
    AddVec, SubVec, DotVec, DivVec,
    Abs, Repack,
    Sin, Cos, Tan, Exp, Relu, Silu, Tanh, Sqrt, Sidmoid, Pow, Log, Softmax,
    Clamp, Sum, SumVec, Min, MinVec, Max, MaxVec, Mean, Concat,
    Transpose2d, TransposeNd, Equal, NotEqual, Greater, Less, GreaterEqual, LessEqual,
    All, Any, Nonzero, Argmax, Argmin
};

inline const char* op_to_string(OpType op) {
    static const char* const names[] = {
        "fill", "random", "slice", "matmul", "add", "sub", "dot", "div", "addvec", "subvec", "dotvec", "divvec",
        "abs", "repack", "sin", "cos", "tan", "exp", "relu", "silu", "tanh", "sqrt", "sigmoid", "pow", "log",
        "softmax", "clamp", "sum", "sumvec", "min", "minvec", "max", "maxvec", "mean", "concat", "transpose2d",
        "transposeNd", "equal", "not_equal", "greater", "less", "greater_equal", "less_equal", "all", "any",
        "nonzero", "argmax", "argmin"};
    const auto i = static_cast<size_t>(op);
    if (i >= sizeof(names) / sizeof(names[0])) throw std::invalid_argument("Unknown OpType");
    return names[i];
}

enum class Device { CPU, CUDA, SYCL, VULKAN, HIP };

enum class DataType {
    INT8 = 0,
    INT16,
    INT32,
    INT64,
    BFLOAT16,
    FLOAT16,
    FLOAT32,
    FLOAT64
};

constexpr std::string_view device_to_string(Device d) {
    switch (d) {
        case Device::CPU: return "CPU";
        case Device::CUDA: return "CUDA";
        case Device::SYCL: return "SYCL";
        case Device::VULKAN: return "VULKAN";
        case Device::HIP: return "HIP";
        default: return "UNKNOWN";
    }
}

constexpr std::string_view dtype_to_string(DataType t) {
    switch (t) {
        case DataType::INT8: return "int8";
        case DataType::INT16: return "int16";
        case DataType::INT32: return "int32";
        case DataType::INT64: return "int64";
        case DataType::FLOAT16: return "float16";
        case DataType::FLOAT32: return "float32";
        case DataType::FLOAT64: return "float64";
        case DataType::BFLOAT16: return "bfloat16";
        default: return "UNKNOWN";
    }
}

inline size_t calc_dtype_size(DataType dtype) {
    switch (dtype) {
        case DataType::INT8: return 1;
        case DataType::INT16: return 2;
        case DataType::INT32: return 4;
        case DataType::INT64: return 8;
        case DataType::FLOAT16: return 2;
        case DataType::FLOAT32: return 4;
        case DataType::FLOAT64: return 8;
        case DataType::BFLOAT16: return 2;
        default: throw std::runtime_error("Unsupported DataType");
    }
}

using CppDTypeVariant = std::variant<int8_t*, int16_t*, int32_t*, int64_t*, float16*, bfloat16*, float*, double*>;
using ConstCppDTypeVariant = std::variant<const int8_t*, const int16_t*, const int32_t*, const int64_t*,
                                          const float16*, const bfloat16*, const float32*, const float64*>;

template <typename T> ConstCppDTypeVariant make_variant(const void* src) {
    ConstCppDTypeVariant var;
    var.emplace<const T*>(static_cast<const T*>(src));
    return var;
}

inline ConstCppDTypeVariant data_as_const_variant(DataType type, const void* src) {
    switch (type) {
        case DataType::INT8: return make_variant<int8_t>(src);
        case DataType::INT16: return make_variant<int16_t>(src);
        case DataType::INT32: return make_variant<int32_t>(src);
        case DataType::INT64: return make_variant<int64_t>(src);
        case DataType::FLOAT16: return make_variant<float16>(src);
        case DataType::BFLOAT16: return make_variant<bfloat16>(src);
        case DataType::FLOAT32: return make_variant<float32>(src);
        case DataType::FLOAT64: return make_variant<float64>(src);
        default: throw std::runtime_error("Unsupported dtype for variant");
    }
}

template <typename Func> void dispatch_dtype(DataType type, Func&& f) {
    switch (type) {
        case DataType::INT8: f(std::type_identity<int8_t>{}); break;
        case DataType::INT16: f(std::type_identity<int16_t>{}); break;
        case DataType::INT32: f(std::type_identity<int32_t>{}); break;
        case DataType::INT64: f(std::type_identity<int64_t>{}); break;
        case DataType::FLOAT16: f(std::type_identity<float16>{}); break;
        case DataType::BFLOAT16: f(std::type_identity<bfloat16>{}); break;
        case DataType::FLOAT32: f(std::type_identity<float>{}); break;
        case DataType::FLOAT64: f(std::type_identity<double>{}); break;
        default: throw std::runtime_error("Unsupported dtype");
    }
}

// Permitted casts (reference type_traits.h:237-260).
inline const std::set<std::pair<DataType, DataType>> valid_casts = {
    {DataType::INT8, DataType::FLOAT32},     {DataType::INT16, DataType::FLOAT32},
    {DataType::INT16, DataType::FLOAT64},    {DataType::INT32, DataType::FLOAT32},
    {DataType::INT32, DataType::FLOAT64},    {DataType::INT64, DataType::FLOAT64},
    {DataType::FLOAT32, DataType::FLOAT16},  {DataType::FLOAT32, DataType::INT32},
    {DataType::FLOAT32, DataType::INT64},    {DataType::INT8, DataType::INT16},
    {DataType::INT8, DataType::INT32},       {DataType::INT8, DataType::INT64},
    {DataType::INT16, DataType::INT32},      {DataType::INT32, DataType::INT64},
    {DataType::FLOAT16, DataType::FLOAT32},  {DataType::FLOAT16, DataType::FLOAT64},
    {DataType::FLOAT16, DataType::BFLOAT16}, {DataType::BFLOAT16, DataType::FLOAT32},
    {DataType::BFLOAT16, DataType::FLOAT64}, {DataType::BFLOAT16, DataType::FLOAT16},
    {DataType::FLOAT32, DataType::FLOAT64},  {DataType::FLOAT64, DataType::FLOAT32}};

// Result dtype of a binary op (reference type_traits.h:270-287; the code, not its comments).
inline DataType compute_type(DataType type0, DataType type1) {
    if (type0 == type1) return type0;
    if (type0 <= DataType::INT64 && type1 <= DataType::INT64) return std::max(type0, type1);
    if (type0 > DataType::INT64 && type1 > DataType::INT64)
        return std::max(std::max(type0, DataType::FLOAT32), std::max(type1, DataType::FLOAT32));
    if (type0 == DataType::INT64 || type1 == DataType::INT64) return DataType::FLOAT64;
    return std::max(std::max(type0, DataType::FLOAT32), std::max(type1, DataType::FLOAT32));
}

inline bool is_cast_valid(DataType src, DataType dst) { return src == dst || valid_casts.count({src, dst}) != 0; }

// Element count of a shape; every dimension must be positive (reference type_traits.h:292-299).
inline size_t calc_numel(const std::vector<int64_t>& shape) {
    size_t numel = 1;
    for (int64_t dim : shape) {
        if (dim <= 0) throw std::runtime_error("Invalid tensor dimension");
        numel *= static_cast<size_t>(dim);
    }
    return numel;
}

} // namespace via
