// SIMT slow path for the dtype pairs the matrix cores do not serve (int16/int32/int64/fp64 and
// mixed pairs).  It restates the reference CPU backend's arithmetic exactly, one thread per
// output element, reading operands through their strides:
//   * fp16/bf16 inputs are widened to fp32 first (src/backend/cpu/mul.cpp:110-111);
//   * the result type is compute_type of the widened types (mul.cpp:112,
//     include/core/type_traits.h:270-287);
//   * batch*M*N < 2^20 selects mul_kernel_basic (mul.cpp:87-96): the sum runs in
//     decltype(T + R) (mul.cpp:13-18) and is converted to the result type once (mul.cpp:21);
//   * otherwise mul_kernel_tiled<.., 64> (mul.cpp:27-85): each 64-wide k-chunk is summed in A's
//     type T with B's values converted to T (mul.cpp:64-71), and chunk sums are converted to the
//     result type and added into it (mul.cpp:74-78).
// Integer arithmetic wraps (two's complement), as the reference's does on its targets; float to
// integer conversion of out-of-range values yields the x86 "integer indefinite" value.
#include "tv_kernels.h"

namespace tvk {
namespace simt {

template <typename X> struct Promote { using type = X; };
template <> struct Promote<int8_t> { using type = int; };
template <> struct Promote<int16_t> { using type = int; };
template <typename A, typename B>
using Common = decltype(typename Promote<A>::type{} + typename Promote<B>::type{});

template <typename X> struct Unsigned;
template <> struct Unsigned<int8_t> { using type = uint8_t; };
template <> struct Unsigned<int16_t> { using type = uint16_t; };
template <> struct Unsigned<int> { using type = unsigned; };
template <> struct Unsigned<long> { using type = unsigned long; };
template <> struct Unsigned<long long> { using type = unsigned long long; };

template <typename X> __device__ constexpr bool is_int() { return !__is_same(X, float) && !__is_same(X, double); }

// static_cast<To>(from) with the reference targets' behaviour for every case.
template <typename To, typename From> __device__ inline To cvt(From v) {
    if constexpr (is_int<To>() && !is_int<From>()) {
        const double x = (double)v;
        if constexpr (sizeof(To) == 8) {
            if (!(x > -9223372036854775808.0 - 1.0 && x < 9223372036854775808.0)) return (To)(int64_t)(-9223372036854775807LL - 1);
            return (To)(int64_t)x;
        } else {
            if (!(x > -2147483649.0 && x < 2147483648.0)) return (To)(int32_t)(-2147483647 - 1);
            return (To)(int32_t)x;
        }
    } else {
        return static_cast<To>(v);
    }
}

template <typename X> __device__ inline X add(X a, X b) {
    if constexpr (is_int<X>()) {
        using U = typename Unsigned<X>::type;
        return (X)(U)((U)a + (U)b);
    } else {
        return a + b;
    }
}
template <typename X> __device__ inline X mul(X a, X b) {
    if constexpr (is_int<X>()) {
        using U = typename Unsigned<X>::type;
        return (X)(U)((U)a * (U)b);
    } else {
        return a * b;
    }
}

// acc (type Acc) += x * y with the C++ promotions of `Acc += P * P`.
template <typename Acc, typename P> __device__ inline Acc mac(Acc acc, P x, P y) {
    using Prod = typename Promote<P>::type;
    const Prod p = mul<Prod>((Prod)x, (Prod)y);
    using Sum = Common<Acc, Prod>;
    return cvt<Acc>(add<Sum>((Sum)acc, (Sum)p));
}

// Load element `idx` of a tensor of storage dtype `dt` as compute type X (fp16/bf16 widened).
template <typename X> __device__ inline X load_as(const void* p, int dt, int64_t idx) {
    switch (dt) {
        case TV_INT8: return cvt<X>(static_cast<const int8_t*>(p)[idx]);
        case TV_INT16: return cvt<X>(static_cast<const int16_t*>(p)[idx]);
        case TV_INT32: return cvt<X>(static_cast<const int32_t*>(p)[idx]);
        case TV_INT64: return cvt<X>(static_cast<const long*>(p)[idx]);
        case TV_BFLOAT16: return cvt<X>((float)static_cast<const __bf16*>(p)[idx]);
        case TV_FLOAT16: return cvt<X>((float)static_cast<const _Float16*>(p)[idx]);
        case TV_FLOAT32: return cvt<X>(static_cast<const float*>(p)[idx]);
        default: return cvt<X>(static_cast<const double*>(p)[idx]);
    }
}

template <typename S> __device__ inline void store_as(void* p, int dt, int64_t idx, S v) {
    switch (dt) {
        case TV_INT8: static_cast<int8_t*>(p)[idx] = cvt<int8_t>(v); break;
        case TV_INT16: static_cast<int16_t*>(p)[idx] = cvt<int16_t>(v); break;
        case TV_INT32: static_cast<int32_t*>(p)[idx] = cvt<int32_t>(v); break;
        case TV_INT64: static_cast<long*>(p)[idx] = cvt<long>(v); break;
        case TV_FLOAT32: static_cast<float*>(p)[idx] = cvt<float>(v); break;
        default: static_cast<double*>(p)[idx] = cvt<double>(v); break;
    }
}

template <int DT> struct CType;
template <> struct CType<TV_INT8> { using type = int8_t; };
template <> struct CType<TV_INT16> { using type = int16_t; };
template <> struct CType<TV_INT32> { using type = int; };
template <> struct CType<TV_INT64> { using type = long; };
template <> struct CType<TV_FLOAT32> { using type = float; };
template <> struct CType<TV_FLOAT64> { using type = double; };

// T, R: widened input types; S: result type.
template <typename T, typename R, typename S>
__global__ __launch_bounds__(256) void gemm_simt_kernel(GemmDesc d, int tiled) {
    const int64_t total = (int64_t)d.batch * d.M * d.N;
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += (int64_t)gridDim.x * blockDim.x) {
        const int64_t n = o % d.N;
        const int64_t m = (o / d.N) % d.M;
        const int64_t b = o / ((int64_t)d.N * d.M);
        const int64_t ia = b * d.sa_b + m * d.sa_m;
        const int64_t ib = b * d.sb_b + n * d.sb_n;
        S res;
        if (!tiled) {
            using P = Common<T, R>;
            P sum = 0;
            for (int64_t k = 0; k < d.K; ++k) {
                const P x = cvt<P>(load_as<T>(d.A, d.dtype_a, ia + k * d.sa_k));
                const P y = cvt<P>(load_as<R>(d.B, d.dtype_b, ib + k * d.sb_k));
                sum = mac<P, P>(sum, x, y);
            }
            res = cvt<S>(sum);
        } else {
            res = 0;
            for (int64_t k0 = 0; k0 < d.K; k0 += 64) {
                const int64_t k1 = k0 + 64 < d.K ? k0 + 64 : d.K;
                T sum = 0;
                for (int64_t k = k0; k < k1; ++k) {
                    const T x = load_as<T>(d.A, d.dtype_a, ia + k * d.sa_k);
                    const T y = cvt<T>(load_as<R>(d.B, d.dtype_b, ib + k * d.sb_k));
                    sum = mac<T, T>(sum, x, y);
                }
                if (k0 == 0) res = cvt<S>(sum);
                else res = cvt<S>(add<Common<S, S>>((Common<S, S>)res, (Common<S, S>)cvt<S>(sum)));
            }
        }
        store_as<S>(d.C, d.dtype_c, b * d.sc_b + m * d.sc_m + n * d.sc_n, res);
    }
}

static int widen(int dt) { return (dt == TV_BFLOAT16 || dt == TV_FLOAT16) ? TV_FLOAT32 : dt; }

template <typename T, typename R>
static int launch_tr(const GemmDesc& d, hipStream_t stream) {
    const int64_t total = (int64_t)d.batch * d.M * d.N;
    const int tiled = total >= (int64_t)1024 * 1024;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    switch (d.dtype_c) {
#define TV_S(DT)                                                                                                      \
    case DT:                                                                                                          \
        hipLaunchKernelGGL((gemm_simt_kernel<T, R, typename CType<DT>::type>), dim3((unsigned)blocks), dim3(256), 0, \
                           stream, d, tiled);                                                                          \
        return hipGetLastError();
        TV_S(TV_INT8) TV_S(TV_INT16) TV_S(TV_INT32) TV_S(TV_INT64) TV_S(TV_FLOAT32) TV_S(TV_FLOAT64)
#undef TV_S
        default: return TV_E_DTYPE;
    }
}

template <typename T>
static int launch_t(const GemmDesc& d, hipStream_t stream) {
    switch (widen(d.dtype_b)) {
        case TV_INT8: return launch_tr<T, int8_t>(d, stream);
        case TV_INT16: return launch_tr<T, int16_t>(d, stream);
        case TV_INT32: return launch_tr<T, int>(d, stream);
        case TV_INT64: return launch_tr<T, long>(d, stream);
        case TV_FLOAT32: return launch_tr<T, float>(d, stream);
        case TV_FLOAT64: return launch_tr<T, double>(d, stream);
        default: return TV_E_DTYPE;
    }
}

// K = 0: every output is the empty sum, through the fused epilogue when one is given (act(bias)).
__global__ __launch_bounds__(256) void gemm_k0_kernel(GemmDesc d) {
    const int64_t total = (int64_t)d.batch * d.M * d.N;
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += (int64_t)gridDim.x * blockDim.x) {
        const int64_t n = o % d.N;
        const int64_t m = (o / d.N) % d.M;
        const int64_t b = o / ((int64_t)d.N * d.M);
        const float v = has_epilogue(d) ? epilogue_value(0.0f, d, b, m, n) : 0.0f;
        const int64_t i = b * d.sc_b + m * d.sc_m + n * d.sc_n;
        switch (d.dtype_c) {
            case TV_BFLOAT16: static_cast<__bf16*>(d.C)[i] = static_cast<__bf16>(v); break;
            case TV_FLOAT16: static_cast<_Float16*>(d.C)[i] = static_cast<_Float16>(v); break;
            case TV_FLOAT32: static_cast<float*>(d.C)[i] = v; break;
            default: store_as<int>(d.C, d.dtype_c, i, 0); break;
        }
    }
}

} // namespace simt

int launch_gemm_k0(const GemmDesc& d, hipStream_t stream) {
    const int64_t total = (int64_t)d.batch * d.M * d.N;
    if (total == 0) return 0;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(simt::gemm_k0_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, d);
    return hipGetLastError();
}

int launch_gemm_simt(const GemmDesc& d, hipStream_t stream) {
    if ((int64_t)d.batch * d.M * d.N == 0) return 0;
    switch (simt::widen(d.dtype_a)) {
        case TV_INT8: return simt::launch_t<int8_t>(d, stream);
        case TV_INT16: return simt::launch_t<int16_t>(d, stream);
        case TV_INT32: return simt::launch_t<int>(d, stream);
        case TV_INT64: return simt::launch_t<long>(d, stream);
        case TV_FLOAT32: return simt::launch_t<float>(d, stream);
        case TV_FLOAT64: return simt::launch_t<double>(d, stream);
        default: return TV_E_DTYPE;
    }
}

} // namespace tvk
