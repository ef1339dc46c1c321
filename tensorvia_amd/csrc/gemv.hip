// Skinny-M (M <= 8) matmul for decode-shaped calls: x[b, M, K] @ W[b, K, N], W row-major
// (N-contiguous).  HBM-bound: W is streamed exactly once with 16-byte loads and no matrix cores.
//
// The reference computes these shapes with mul_kernel_basic (src/backend/cpu/mul.cpp:7-25), chosen
// because batch*M*N < 2^20 (mul.cpp:87-96), on one OpenMP thread when M = 1.
//
// Work split:
//  * a workgroup of 256 threads owns NB = 16 * VEC columns (16 lanes x 16 bytes = 256 bytes of each
//    W row) and one K-slice; its 16 k-lanes walk contiguous row ranges of that slice;
//  * each step reads VEC rows of W (VEC x 16 bytes per thread in flight, double-buffered in
//    registers) and one 16-byte chunk of x per row of x, which holds the same VEC k values;
//  * products use the packed dot instructions: v_dot2_f32_bf16 / v_dot2_f32_f16 over pairs of
//    rows, v_dot4_i32_i8 over quads of rows, plain fp32 FMA for fp32 — fp32 (int32) accumulation;
//  * k-lanes are reduced with lane shuffles and LDS; when the grid splits K over S > 1 workgroups,
//    each writes its fp32/int32 partial to a workspace and the last one to arrive for a column
//    block (agent-scope atomic counter, release/acquire fences) sums the S partials in slice order
//    — deterministic — converts and stores C, then re-arms the counter for the next call.
#include "tv_kernels.h"

namespace tvk {

template <typename T> struct GemvTraits;
template <> struct GemvTraits<float> { using Acc = float; static constexpr int P = 1; };
template <> struct GemvTraits<__bf16> { using Acc = float; static constexpr int P = 2; };
template <> struct GemvTraits<_Float16> { using Acc = float; static constexpr int P = 2; };
template <> struct GemvTraits<int8_t> { using Acc = int; static constexpr int P = 4; };

constexpr int GEMV_NL = 16;      // lanes across columns
constexpr int GEMV_THREADS = 256;
constexpr int GEMV_KL = GEMV_THREADS / GEMV_NL; // k-lanes per workgroup (4 per wave)

struct GemvArgs {
    GemmDesc d;
    int kslice;      // rows per K-slice (multiple of GEMV_KL * VEC)
    int nslices;     // S
    void* ws;        // [batch][S][MR][N] partials (S > 1)
    unsigned* cnt;   // [batch][n-blocks] arrival counters (S > 1)
};

// Accumulate VEC rows (one 16-byte W chunk per row) against the matching x chunks.
template <typename T, int MR>
__device__ inline void gemv_step(const u32x4 (&w)[16 / sizeof(T)], const u32x4 (&x)[MR],
                                 typename GemvTraits<T>::Acc (&acc)[MR][16 / sizeof(T)]) {
    constexpr int VEC = 16 / sizeof(T);
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int r = 0; r < VEC; ++r)
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const float xv = __builtin_bit_cast(float, x[m][r]);
#pragma unroll
                for (int e = 0; e < VEC; ++e) acc[m][e] = __builtin_fmaf(xv, __builtin_bit_cast(float, w[r][e]), acc[m][e]);
            }
    } else if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int r = 0; r < VEC; r += 2) {
            unsigned wp[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const unsigned lo = (w[r][e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
                const unsigned hi = (w[r + 1][e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
                wp[e] = lo | (hi << 16);
            }
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const unsigned xp = x[m][r >> 1];
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    if constexpr (__is_same(T, __bf16))
                        acc[m][e] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, xp),
                                                                    __builtin_bit_cast(bf16x2, wp[e]), acc[m][e], false);
                    else
                        acc[m][e] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, xp),
                                                           __builtin_bit_cast(f16x2, wp[e]), acc[m][e], false);
                }
            }
        }
    } else {
#pragma unroll
        for (int r = 0; r < VEC; r += 4) {
            unsigned wq[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const int sh = 8 * (e & 3), dw = e >> 2;
                wq[e] = ((w[r][dw] >> sh) & 0xFFu) | (((w[r + 1][dw] >> sh) & 0xFFu) << 8) |
                        (((w[r + 2][dw] >> sh) & 0xFFu) << 16) | (((w[r + 3][dw] >> sh) & 0xFFu) << 24);
            }
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const int xq = (int)x[m][r >> 2];
#pragma unroll
                for (int e = 0; e < VEC; ++e) acc[m][e] = __builtin_amdgcn_sdot4(xq, (int)wq[e], acc[m][e], false);
            }
        }
    }
}

template <typename Acc>
__device__ inline void gemv_store(void* C, int64_t idx, int dtype_c, Acc v) {
    if constexpr (__is_same(Acc, int)) {
        if (dtype_c == TV_INT8) static_cast<int8_t*>(C)[idx] = static_cast<int8_t>(v);
        else static_cast<int32_t*>(C)[idx] = v;
    } else {
        if (dtype_c == TV_BFLOAT16) static_cast<__bf16*>(C)[idx] = static_cast<__bf16>(v);
        else if (dtype_c == TV_FLOAT16) static_cast<_Float16*>(C)[idx] = static_cast<_Float16>(v);
        else static_cast<float*>(C)[idx] = v;
    }
}

template <typename T, int MR>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_ncontig_kernel(GemvArgs g) {
    using Acc = typename GemvTraits<T>::Acc;
    constexpr int ES = sizeof(T);
    constexpr int VEC = 16 / ES;
    constexpr int NB = GEMV_NL * VEC;
    constexpr int NWAVES = GEMV_THREADS / 64;
    const GemmDesc& d = g.d;

    __shared__ Acc part[NWAVES][MR][NB];
    __shared__ int last_flag;

    const int tid = threadIdx.x;
    const int nl = tid % GEMV_NL, kl = tid / GEMV_NL;
    const int b = blockIdx.z, s = blockIdx.y;
    const int n0 = blockIdx.x * NB;
    const int col = n0 + nl * VEC;
    const bool col_ok = col < d.N; // N % VEC == 0 is a launch precondition

    const int kbeg_slice = s * g.kslice;
    const int kend_slice = min(d.K, kbeg_slice + g.kslice);
    const int per_lane = g.kslice / GEMV_KL; // multiple of VEC
    const int kbeg = kbeg_slice + kl * per_lane;
    const int kend = min(kend_slice, kbeg + per_lane);

    const char* W = static_cast<const char*>(d.B) + ((int64_t)b * d.sb_b + col) * ES;
    const char* X = static_cast<const char*>(d.A) + (int64_t)b * d.sa_b * ES;

    Acc acc[MR][VEC];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[m][e] = 0;

    auto load_w = [&](int k, u32x4 (&w)[VEC]) {
#pragma unroll
        for (int r = 0; r < VEC; ++r) {
            if (col_ok && k + r < kend)
                w[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(W + (int64_t)(k + r) * d.sb_k * ES));
            else
                w[r] = u32x4{0, 0, 0, 0};
        }
    };
    auto load_x = [&](int k, u32x4 (&x)[MR]) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            if (m < d.M && k < kend)
                x[m] = *reinterpret_cast<const u32x4*>(X + ((int64_t)m * d.sa_m + k) * ES);
            else
                x[m] = u32x4{0, 0, 0, 0};
        }
    };

    if (kbeg < kend) {
        u32x4 w0[VEC], w1[VEC], x0[MR], x1[MR];
        load_w(kbeg, w0);
        load_x(kbeg, x0);
        int k = kbeg;
        for (; k + VEC < kend; k += 2 * VEC) {
            load_w(k + VEC, w1);
            load_x(k + VEC, x1);
            gemv_step<T, MR>(w0, x0, acc);
            if (k + 2 * VEC < kend) {
                load_w(k + 2 * VEC, w0);
                load_x(k + 2 * VEC, x0);
            }
            gemv_step<T, MR>(w1, x1, acc);
        }
        if (k < kend) gemv_step<T, MR>(w0, x0, acc);
    }

    // Reduce the 4 k-lanes of each wave (lanes nl, nl+16, nl+32, nl+48), then the waves via LDS.
    const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            Acc v = acc[m][e];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            acc[m][e] = v;
        }
    if (lane < GEMV_NL) {
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int e = 0; e < VEC; ++e) part[wave][m][lane * VEC + e] = acc[m][e];
    }
    __syncthreads();

    const int64_t c_b = (int64_t)b * d.sc_b;
    const size_t csz = dtype_size(d.dtype_c);
    if (g.nslices == 1) {
        for (int i = tid; i < MR * NB; i += GEMV_THREADS) {
            const int m = i / NB, c = i % NB;
            if (m < d.M && n0 + c < d.N) {
                Acc v = part[0][m][c];
#pragma unroll
                for (int w = 1; w < NWAVES; ++w) v += part[w][m][c];
                gemv_store(static_cast<char*>(d.C) + c_b * csz, (int64_t)m * d.sc_m + (int64_t)(n0 + c) * d.sc_n, d.dtype_c, v);
            }
        }
        return;
    }

    // Split-K: publish this slice's partial, the last workgroup of the column block reduces.
    Acc* ws = static_cast<Acc*>(g.ws) + ((int64_t)b * g.nslices) * MR * d.N;
    for (int i = tid; i < MR * NB; i += GEMV_THREADS) {
        const int m = i / NB, c = i % NB;
        if (n0 + c < d.N) {
            Acc v = part[0][m][c];
#pragma unroll
            for (int w = 1; w < NWAVES; ++w) v += part[w][m][c];
            ws[((int64_t)s * MR + m) * d.N + n0 + c] = v;
        }
    }
    __threadfence();
    __syncthreads();
    unsigned* counter = g.cnt + (int64_t)b * gridDim.x + blockIdx.x;
    if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last_flag = (prev == (unsigned)g.nslices - 1);
    }
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
    for (int i = tid; i < MR * NB; i += GEMV_THREADS) {
        const int m = i / NB, c = i % NB;
        if (m < d.M && n0 + c < d.N) {
            Acc v = 0;
            for (int ss = 0; ss < g.nslices; ++ss)
                v += __hip_atomic_load(&ws[((int64_t)ss * MR + m) * d.N + n0 + c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            gemv_store(static_cast<char*>(d.C) + c_b * csz, (int64_t)m * d.sc_m + (int64_t)(n0 + c) * d.sc_n, d.dtype_c, v);
        }
    }
    if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------------------
// Host side.

// Per-stream workspace for the split-K partials and counters.  Calls on one stream are ordered by
// the stream, so they can share it; the counters are zero whenever no kernel of the stream runs.
struct GemvWorkspace {
    void* base = nullptr;
    size_t bytes = 0;
};
}

#include <map>
#include <mutex>

namespace tvk {
static std::mutex g_ws_mu;
static std::map<std::pair<int, hipStream_t>, GemvWorkspace> g_ws;

static int get_workspace(hipStream_t stream, size_t need, void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    GemvWorkspace& w = g_ws[{dev, stream}];
    if (w.bytes < need) {
        if (w.base) {
            // The old buffer may still be in use by queued work of this stream.
            e = hipStreamSynchronize(stream);
            if (e != hipSuccess) return e;
            hipFree(w.base);
            w.base = nullptr;
            w.bytes = 0;
        }
        size_t sz = need < (1u << 20) ? (1u << 20) : need;
        e = hipMalloc(&w.base, sz);
        if (e != hipSuccess) return TV_E_NOMEM;
        e = hipMemsetAsync(w.base, 0, sz, stream);
        if (e != hipSuccess) return e;
        w.bytes = sz;
    }
    *out = w.base;
    return 0;
}

// Whether the vectorised GEMV serves this call.
static bool gemv_layout_ok(const GemmDesc& d) {
    if (d.dtype_a != d.dtype_b) return false;
    const int es = (int)dtype_size(d.dtype_a);
    const int64_t vec = 16 / es;
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (d.M < 1 || d.M > 8) return false;
    if (d.sb_n != 1 || !al(d.B) || d.N % vec || (d.K > 1 && d.sb_k % vec) || (d.batch > 1 && d.sb_b % vec)) return false;
    if (d.sa_k != 1 || !al(d.A) || d.K % vec || (d.M > 1 && d.sa_m % vec) || (d.batch > 1 && d.sa_b % vec)) return false;
    return true;
}

template <typename T, int MR>
static int gemv_run(const GemmDesc& d, hipStream_t stream) {
    constexpr int VEC = 16 / sizeof(T);
    constexpr int NB = GEMV_NL * VEC;
    using Acc = typename GemvTraits<T>::Acc;
    const int nblk = (d.N + NB - 1) / NB;
    // Aim for >= 4 workgroups per CU (256 CUs) while keeping >= 4 steps per k-lane.
    const int unit = GEMV_KL * VEC;                 // rows one slice step covers
    const int max_s = (d.K + 4 * unit - 1) / (4 * unit);
    int S = (1024 + nblk * d.batch - 1) / (nblk * d.batch);
    S = S < 1 ? 1 : (S > max_s ? max_s : S);
    if (S < 1) S = 1;
    int kslice = (d.K + S - 1) / S;
    kslice = (kslice + unit - 1) / unit * unit;
    S = (d.K + kslice - 1) / kslice;
    if (S < 1) S = 1;

    GemvArgs g;
    g.d = d;
    g.kslice = kslice;
    g.nslices = S;
    g.ws = nullptr;
    g.cnt = nullptr;
    if (S > 1) {
        const size_t part_bytes = (size_t)d.batch * S * MR * d.N * sizeof(Acc);
        const size_t cnt_bytes = (size_t)d.batch * nblk * sizeof(unsigned);
        void* ws = nullptr;
        int rc = get_workspace(stream, part_bytes + cnt_bytes + 256, &ws);
        if (rc) return rc;
        g.cnt = static_cast<unsigned*>(ws);
        g.ws = static_cast<char*>(ws) + ((cnt_bytes + 255) / 256) * 256;
    }
    hipLaunchKernelGGL((gemv_ncontig_kernel<T, MR>), dim3(nblk, S, d.batch), dim3(GEMV_THREADS), 0, stream, g);
    return hipGetLastError();
}

template <typename T>
static int gemv_dispatch_mr(const GemmDesc& d, hipStream_t stream) {
    if (d.M <= 1) return gemv_run<T, 1>(d, stream);
    if (d.M <= 2) return gemv_run<T, 2>(d, stream);
    if (d.M <= 4) return gemv_run<T, 4>(d, stream);
    return gemv_run<T, 8>(d, stream);
}

int launch_gemv(const GemmDesc& d, hipStream_t stream) {
    if (!gemv_layout_ok(d)) return TV_E_UNSUPPORTED;
    if (d.N == 0 || d.batch == 0) return 0;
    switch (d.dtype_a) {
        case TV_FLOAT32: return gemv_dispatch_mr<float>(d, stream);
        case TV_BFLOAT16: return gemv_dispatch_mr<__bf16>(d, stream);
        case TV_FLOAT16: return gemv_dispatch_mr<_Float16>(d, stream);
        case TV_INT8: return gemv_dispatch_mr<int8_t>(d, stream);
        default: return TV_E_UNSUPPORTED;
    }
}

} // namespace tvk
