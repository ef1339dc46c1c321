// Element-wise materialisation ops of the HIP backend: dtype casts (TypecastImpl), constant fills
// (FillImpl / ZerosImpl / OnesImpl) and the seeded counter-based generator behind ops::Random
// (RandomImpl).  All three are HBM-bound streams over contiguous buffers.
//
// Layout of the work: a workgroup owns 2048 consecutive elements, a thread 8 of them.  When both
// buffers are 16-byte aligned, a thread's 8 elements are 8 / V runs of V = 16 / (widest element size)
// (at most 8) consecutive elements, and run a of thread t starts at element a * 256 V + t V of the
// workgroup's range: every vector access of a wave covers one contiguous span (64 x 16 bytes on the
// wider side), so each store instruction writes whole cache lines.  The ragged end and misaligned
// buffers take an element loop.  Grid: enough 256-thread workgroups for 8 waves per SIMD,
// grid-striding beyond that.
#include "tv_kernels.h"

namespace tvk {

// Element type of each DataType value (reference include/core/type_traits.h:123-132).
template <int DT> struct Elem;
template <> struct Elem<TV_INT8> { using type = int8_t; };
template <> struct Elem<TV_INT16> { using type = int16_t; };
template <> struct Elem<TV_INT32> { using type = int32_t; };
template <> struct Elem<TV_INT64> { using type = int64_t; };
template <> struct Elem<TV_BFLOAT16> { using type = __bf16; };
template <> struct Elem<TV_FLOAT16> { using type = _Float16; };
template <> struct Elem<TV_FLOAT32> { using type = float; };
template <> struct Elem<TV_FLOAT64> { using type = double; };

// Half types compute in float (reference compute_type_t, include/core/types.h:111-117); a cast
// from a half type goes through its exact float value.
template <typename S> struct Widen { using type = S; };
template <> struct Widen<__bf16> { using type = float; };
template <> struct Widen<_Float16> { using type = float; };

template <typename S, typename D> __device__ inline D cast_elem(S s) {
    return static_cast<D>(static_cast<typename Widen<S>::type>(s));
}

constexpr int kEwGroup = 8; // elements per thread
constexpr int kEwThreads = 256;
constexpr int64_t kEwBlock = (int64_t)kEwGroup * kEwThreads; // elements per workgroup step

// V consecutive elements moved by one access (V * sizeof(E) bytes, aligned to that).
template <typename E, int V> struct alignas(V * sizeof(E)) Run {
    E v[V];
};
// Elements per run: 16 bytes of the wider element type, at most a thread's 8.
template <int A, int B> constexpr int ew_run() {
    constexpr int w = A > B ? A : B;
    return 16 / w < kEwGroup ? 16 / w : kEwGroup;
}

static unsigned ew_blocks(int64_t n) {
    const int64_t groups = (n + kEwGroup - 1) / kEwGroup;
    int64_t b = (groups + kEwThreads - 1) / kEwThreads;
    const int64_t cap = 256 * 8 * 4; // 8 waves per SIMD on 256 CUs, then grid-stride
    if (b > cap) b = cap;
    return (unsigned)(b < 1 ? 1 : b);
}


// ---- typecast ----------------------------------------------------------------------------------

template <typename S, typename D, bool VEC>
__global__ __launch_bounds__(kEwThreads) void cast_kernel(const S* __restrict__ src, D* __restrict__ dst, int64_t n) {
    constexpr int V = ew_run<sizeof(S), sizeof(D)>();
    const int64_t stride = (int64_t)gridDim.x * kEwBlock;
    for (int64_t b0 = (int64_t)blockIdx.x * kEwBlock; b0 < n; b0 += stride) {
#pragma unroll
        for (int a = 0; a < kEwGroup / V; ++a) {
            const int64_t i0 = b0 + (int64_t)a * kEwThreads * V + (int64_t)threadIdx.x * V;
            if (VEC && i0 + V <= n) {
                const Run<S, V> g = *reinterpret_cast<const Run<S, V>*>(src + i0);
                Run<D, V> o;
#pragma unroll
                for (int e = 0; e < V; ++e) o.v[e] = cast_elem<S, D>(g.v[e]);
                // Streaming (nt sc1) stores when a run is 16 bytes: a wave's store is whole lines,
                // and the output does not evict the source from the caches (cast_c3a 140 -> 134 us;
                // the same policy on fill measured 2 % slower and is not used there).
                if constexpr (sizeof(Run<D, V>) == 16) store_stream16(dst + i0, __builtin_bit_cast(u32x4, o));
                else *reinterpret_cast<Run<D, V>*>(dst + i0) = o;
            } else {
                for (int64_t i = i0; i < n && i < i0 + V; ++i) dst[i] = cast_elem<S, D>(src[i]);
            }
        }
    }
}

template <typename S, typename D>
static int cast_launch(const void* src, void* dst, int64_t n, hipStream_t stream) {
    const bool vec = aligned16(src) && aligned16(dst);
    if (vec)
        hipLaunchKernelGGL((cast_kernel<S, D, true>), dim3(ew_blocks(n)), dim3(kEwThreads), 0, stream,
                           static_cast<const S*>(src), static_cast<D*>(dst), n);
    else
        hipLaunchKernelGGL((cast_kernel<S, D, false>), dim3(ew_blocks(n)), dim3(kEwThreads), 0, stream,
                           static_cast<const S*>(src), static_cast<D*>(dst), n);
    return hipGetLastError();
}

// The pairs of the reference's valid_casts table (include/core/type_traits.h:237-260).
int launch_typecast(const void* src, int src_dt, void* dst, int dst_dt, int64_t n, hipStream_t stream) {
#define TV_CAST(S_, D_) \
    if (src_dt == S_ && dst_dt == D_) return cast_launch<Elem<S_>::type, Elem<D_>::type>(src, dst, n, stream);
    TV_CAST(TV_INT8, TV_FLOAT32)
    TV_CAST(TV_INT16, TV_FLOAT32)
    TV_CAST(TV_INT16, TV_FLOAT64)
    TV_CAST(TV_INT32, TV_FLOAT32)
    TV_CAST(TV_INT32, TV_FLOAT64)
    TV_CAST(TV_INT64, TV_FLOAT64)
    TV_CAST(TV_FLOAT32, TV_FLOAT16)
    TV_CAST(TV_FLOAT32, TV_INT32)
    TV_CAST(TV_FLOAT32, TV_INT64)
    TV_CAST(TV_INT8, TV_INT16)
    TV_CAST(TV_INT8, TV_INT32)
    TV_CAST(TV_INT8, TV_INT64)
    TV_CAST(TV_INT16, TV_INT32)
    TV_CAST(TV_INT32, TV_INT64)
    TV_CAST(TV_FLOAT16, TV_FLOAT32)
    TV_CAST(TV_FLOAT16, TV_FLOAT64)
    TV_CAST(TV_FLOAT16, TV_BFLOAT16)
    TV_CAST(TV_BFLOAT16, TV_FLOAT32)
    TV_CAST(TV_BFLOAT16, TV_FLOAT64)
    TV_CAST(TV_BFLOAT16, TV_FLOAT16)
    TV_CAST(TV_FLOAT32, TV_FLOAT64)
    TV_CAST(TV_FLOAT64, TV_FLOAT32)
#undef TV_CAST
    return TV_E_DTYPE;
}

// ---- fill --------------------------------------------------------------------------------------

template <typename E, bool VEC>
__global__ __launch_bounds__(kEwThreads) void fill_kernel(E* __restrict__ dst, int64_t n, float value) {
    constexpr int V = ew_run<sizeof(E), sizeof(E)>();
    const E v = static_cast<E>(value); // T(val), reference initializer.cpp:14-17
    const int64_t stride = (int64_t)gridDim.x * kEwBlock;
    for (int64_t b0 = (int64_t)blockIdx.x * kEwBlock; b0 < n; b0 += stride) {
#pragma unroll
        for (int a = 0; a < kEwGroup / V; ++a) {
            const int64_t i0 = b0 + (int64_t)a * kEwThreads * V + (int64_t)threadIdx.x * V;
            if (VEC && i0 + V <= n) {
                Run<E, V> o;
#pragma unroll
                for (int e = 0; e < V; ++e) o.v[e] = v;
                *reinterpret_cast<Run<E, V>*>(dst + i0) = o;
            } else {
                for (int64_t i = i0; i < n && i < i0 + V; ++i) dst[i] = v;
            }
        }
    }
}

// ---- seeded uniform generator --------------------------------------------------------------------
// Element i of stream `seed` is mix64(key + (i + 1) * G) with key = mix64(seed + G) (SplitMix64).
// Reals: min + span * u in fp32 without contraction, u = (top 24 bits) / 2^24, then rounded to the
// element type (round to nearest even for the half types).  Integers: lo + ((top32 * (hi - lo + 1))
// >> 32), inclusive [lo, hi].  The same stream as the host generator (ops::detail::random_fill) and
// tensorvia_amd/rng.py.

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

__host__ __device__ inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct RandomArgs {
    uint64_t key;
    float min, span; // reals
    int64_t lo;      // integers
    uint64_t range;  // hi - lo + 1
};

// Element whose SplitMix64 state (key + (i + 1) * G) is z0.
template <typename E> __device__ inline E random_from_state(const RandomArgs& r, uint64_t z0) {
    const uint64_t z = mix64(z0);
    if constexpr (__is_same(E, int8_t) || __is_same(E, int16_t) || __is_same(E, int32_t) || __is_same(E, int64_t)) {
        return static_cast<E>(r.lo + (int64_t)(((z >> 32) * r.range) >> 32));
    } else {
#pragma clang fp contract(off)
        // A separate multiply and add (a fused multiply-add would round once and differ from the
        // host stream).
        const float u = (float)(z >> 40) * 0x1p-24f;
        const float su = r.span * u;
        return static_cast<E>(r.min + su);
    }
}

template <typename E> __device__ inline E random_elem(const RandomArgs& r, int64_t i) {
    return random_from_state<E>(r, r.key + (uint64_t)(i + 1) * kGamma);
}

template <typename E, bool VEC>
__global__ __launch_bounds__(kEwThreads) void random_kernel(E* __restrict__ dst, int64_t n, RandomArgs r) {
    constexpr int V = ew_run<sizeof(E), sizeof(E)>();
    const int64_t stride = (int64_t)gridDim.x * kEwBlock;
    for (int64_t b0 = (int64_t)blockIdx.x * kEwBlock; b0 < n; b0 += stride) {
#pragma unroll
        for (int a = 0; a < kEwGroup / V; ++a) {
            const int64_t i0 = b0 + (int64_t)a * kEwThreads * V + (int64_t)threadIdx.x * V;
            if (VEC && i0 + V <= n) {
                // Consecutive states differ by G: one 64-bit multiply per run, then additions.
                Run<E, V> o;
                uint64_t z0 = r.key + (uint64_t)(i0 + 1) * kGamma;
#pragma unroll
                for (int e = 0; e < V; ++e, z0 += kGamma) o.v[e] = random_from_state<E>(r, z0);
                *reinterpret_cast<Run<E, V>*>(dst + i0) = o;
            } else {
                for (int64_t i = i0; i < n && i < i0 + V; ++i) dst[i] = random_elem<E>(r, i);
            }
        }
    }
}

template <typename E>
static int fill_or_random(void* dst, int64_t n, bool random, float value, const RandomArgs& r, hipStream_t stream) {
    E* p = static_cast<E*>(dst);
    const dim3 grid(ew_blocks(n)), block(kEwThreads);
    if (random) {
        if (aligned16(dst)) hipLaunchKernelGGL((random_kernel<E, true>), grid, block, 0, stream, p, n, r);
        else hipLaunchKernelGGL((random_kernel<E, false>), grid, block, 0, stream, p, n, r);
    } else {
        if (aligned16(dst)) hipLaunchKernelGGL((fill_kernel<E, true>), grid, block, 0, stream, p, n, value);
        else hipLaunchKernelGGL((fill_kernel<E, false>), grid, block, 0, stream, p, n, value);
    }
    return hipGetLastError();
}

static int dispatch_init(void* dst, int dt, int64_t n, bool random, float value, const RandomArgs& r, hipStream_t s) {
    switch (dt) {
        case TV_INT8: return fill_or_random<int8_t>(dst, n, random, value, r, s);
        case TV_INT16: return fill_or_random<int16_t>(dst, n, random, value, r, s);
        case TV_INT32: return fill_or_random<int32_t>(dst, n, random, value, r, s);
        case TV_INT64: return fill_or_random<int64_t>(dst, n, random, value, r, s);
        case TV_BFLOAT16: return fill_or_random<__bf16>(dst, n, random, value, r, s);
        case TV_FLOAT16: return fill_or_random<_Float16>(dst, n, random, value, r, s);
        case TV_FLOAT32: return fill_or_random<float>(dst, n, random, value, r, s);
        case TV_FLOAT64: return fill_or_random<double>(dst, n, random, value, r, s);
        default: return TV_E_DTYPE;
    }
}

int launch_fill(void* dst, int dt, int64_t n, float value, hipStream_t stream) {
    return dispatch_init(dst, dt, n, false, value, RandomArgs{}, stream);
}

int launch_random(void* dst, int dt, int64_t n, float min, float max, uint64_t seed, hipStream_t stream) {
    RandomArgs r;
    r.key = mix64(seed + kGamma);
    r.min = min;
    r.span = static_cast<float>(static_cast<double>(max) - static_cast<double>(min));
    r.lo = static_cast<int64_t>(min);
    r.range = static_cast<uint64_t>(static_cast<int64_t>(max) - r.lo + 1);
    return dispatch_init(dst, dt, n, true, 0.0f, r, stream);
}

} // namespace tvk
