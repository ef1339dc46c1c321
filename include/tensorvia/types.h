// Element types of the Tensorvia API (reference include/core/types.h).
//
// float16 / bfloat16 are the compiler's IEEE binary16 and bfloat16 types, whose conversions from
// float round to nearest even (the reference's C++23 std::float16_t / std::bfloat16_t behaviour,
// types.h:56-62).  Arithmetic on them is carried out in float (compute_type_t).
#pragma once

#include <cstdint>

using float32 = float;
using float64 = double;
using float16 = _Float16;
using bfloat16 = __bf16;

template <typename T> struct compute_type_helper { using type = T; };
template <> struct compute_type_helper<float16> { using type = float; };
template <> struct compute_type_helper<bfloat16> { using type = float; };

template <typename T> using compute_type_t = typename compute_type_helper<T>::type;

#ifndef RESTRICT
#define RESTRICT __restrict__
#endif
