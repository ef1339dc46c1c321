// Skinny-M (M <= 8) matmul for decode-shaped calls: x[b, M, K] @ W[b, K, N], W row-major
// (N-contiguous).  HBM-bound: W is streamed exactly once with 16-byte loads and no matrix cores.
//
// The reference computes these shapes with mul_kernel_basic (src/backend/cpu/mul.cpp:7-25), chosen
// because batch*M*N < 2^20 (mul.cpp:87-96), on one OpenMP thread when M = 1.
//
// Work split:
//  * a workgroup owns a strip of NB = NL * VEC columns (NL lanes x 16 bytes of each W row) and, by
//    default, the whole K range; its KL = THREADS / NL k-lanes walk contiguous row ranges;
//  * narrow strips (64 bytes of a 128-byte line for bf16) give every CU a workgroup; workgroup ids
//    are remapped so that neighbouring strips run on the same XCD and share W's lines in its L2;
//  * each step reads VEC rows of W (VEC x 16 bytes per thread, double-buffered in registers) and
//    one 16-byte chunk of x per row of x, which holds the same VEC k values;
//  * products use the packed dot instructions: v_dot2_f32_bf16 / v_dot2_f32_f16 over pairs of
//    rows, v_dot4_i32_i8 over quads of rows, plain fp32 FMA for fp32 — fp32 (int32) accumulation;
//  * k-lanes are reduced with lane shuffles, then across waves through LDS, in a fixed order;
//  * only when the strips cannot fill the GPU is K split over S workgroups: each writes its partial
//    to a workspace and a second kernel sums the S partials in slice order (deterministic).  No
//    cross-workgroup fences or atomics are used: an agent-scope release costs an L2 writeback per
//    workgroup on this part.
#include "tv_kernels.h"

namespace tvk {

template <typename T> struct GemvTraits;
template <> struct GemvTraits<float> { using Acc = float; static constexpr int P = 1; };
template <> struct GemvTraits<__bf16> { using Acc = float; static constexpr int P = 2; };
template <> struct GemvTraits<_Float16> { using Acc = float; static constexpr int P = 2; };
template <> struct GemvTraits<int8_t> { using Acc = int; static constexpr int P = 4; };

// A workgroup owns NB = NL * VEC columns of W and one K-slice; NL lanes span the columns and
// KL = THREADS / NL "k-lanes" walk contiguous row ranges of the slice.
struct GemvArgs {
    GemmDesc d;
    int kslice;      // rows per K-slice (a multiple of KL * VEC)
    int nslices;     // S: K-slices; S > 1 writes partials for gemv_reduce_kernel
    int nblk;        // column blocks per batch
    void* ws;        // [S][batch][MR][N] partials (S > 1)
};

// Accumulate VEC rows (one 16-byte W chunk per row) against the matching x chunks.
template <typename T, int MR>
__device__ inline void gemv_step(const u32x4 (&w)[16 / sizeof(T)], const u32x4 (&x)[MR],
                                 typename GemvTraits<T>::Acc (&acc)[MR][16 / sizeof(T)]) {
    constexpr int VEC = 16 / sizeof(T);
    if constexpr (sizeof(T) == 4) {
        // Whole-vector casts: clang's __builtin_bit_cast of a vector *element* reads element 0.
#pragma unroll
        for (int r = 0; r < VEC; ++r) {
            const f32x4 wf = __builtin_bit_cast(f32x4, w[r]);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const float xv = __builtin_bit_cast(f32x4, x[m])[r];
#pragma unroll
                for (int e = 0; e < VEC; ++e) acc[m][e] = __builtin_fmaf(xv, wf[e], acc[m][e]);
            }
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

// Workgroup ids are remapped so that neighbouring column blocks (which share 128-byte lines of W
// when NB * sizeof(T) < 128) run on the same XCD and meet in its L2.
__device__ inline int xcd_remap(int bid, int nwg) {
    return (nwg & 7) == 0 ? (bid & 7) * (nwg >> 3) + (bid >> 3) : bid;
}

template <typename T, int MR, int NL, int THREADS>
__global__ __launch_bounds__(THREADS) void gemv_ncontig_kernel(GemvArgs g) {
    using Acc = typename GemvTraits<T>::Acc;
    constexpr int ES = sizeof(T);
    constexpr int VEC = 16 / ES;
    constexpr int NB = NL * VEC;
    constexpr int KL = THREADS / NL;
    constexpr int NWAVES = THREADS / 64;
    constexpr int LPW = 64 / NL; // k-lanes per wave
    static_assert(64 % NL == 0 && THREADS % 64 == 0, "n-lanes must tile a wave");
    const GemmDesc& d = g.d;

    __shared__ Acc part[NWAVES][MR][NB];

    const int tid = threadIdx.x;
    const int nl = tid % NL, kl = tid / NL;
    const int lin = xcd_remap(blockIdx.x, gridDim.x);
    const int b = lin / g.nblk;
    const int n0 = (lin - b * g.nblk) * NB;
    const int s = blockIdx.y;
    const int col = n0 + nl * VEC;
    const bool col_ok = col < d.N; // N % VEC == 0 is a launch precondition

    const int kbeg_slice = s * g.kslice;
    const int kend_slice = min(d.K, kbeg_slice + g.kslice);
    const int per_lane = g.kslice / KL; // multiple of VEC
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

    // Reduce the LPW k-lanes of each wave (lanes nl + NL*j), then the waves through LDS.
    const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            Acc v = acc[m][e];
#pragma unroll
            for (int off = NL; off < 64; off <<= 1) v += __shfl_xor(v, off);
            acc[m][e] = v;
        }
    (void)LPW;
    if (lane < NL) {
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int e = 0; e < VEC; ++e) part[wave][m][lane * VEC + e] = acc[m][e];
    }
    __syncthreads();

    const size_t csz = dtype_size(d.dtype_c);
    char* Cb = static_cast<char*>(d.C) + (int64_t)b * d.sc_b * csz;
    Acc* ws = g.nslices > 1 ? static_cast<Acc*>(g.ws) + (((int64_t)s * d.batch + b) * MR) * d.N : nullptr;
    for (int i = tid; i < MR * NB; i += THREADS) {
        const int m = i / NB, c = i % NB;
        if (m < d.M && n0 + c < d.N) {
            Acc v = part[0][m][c];
#pragma unroll
            for (int w = 1; w < NWAVES; ++w) v += part[w][m][c];
            if (ws) ws[(int64_t)m * d.N + n0 + c] = v;
            else gemv_store(Cb, (int64_t)m * d.sc_m + (int64_t)(n0 + c) * d.sc_n, d.dtype_c, v);
        }
    }
}

// Split-K epilogue: C[b, m, n] = sum over slices s = 0..S-1, in slice order (deterministic).
template <typename Acc>
__global__ __launch_bounds__(256) void gemv_reduce_kernel(GemvArgs g, int mr) {
    const GemmDesc& d = g.d;
    const int64_t total = (int64_t)d.batch * d.M * d.N;
    const int64_t stride_s = (int64_t)d.batch * mr * d.N;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t n = i % d.N;
        const int64_t m = (i / d.N) % d.M;
        const int64_t b = i / ((int64_t)d.N * d.M);
        const Acc* p = static_cast<const Acc*>(g.ws) + (b * mr + m) * d.N + n;
        Acc v = 0;
        for (int s = 0; s < g.nslices; ++s) v += p[s * stride_s];
        const size_t csz = dtype_size(d.dtype_c);
        gemv_store(static_cast<char*>(d.C) + b * d.sc_b * csz, m * d.sc_m + n * d.sc_n, d.dtype_c, v);
    }
}

// ---------------------------------------------------------------------------------------------
// Host side.
}

#include <map>
#include <mutex>

namespace tvk {

// Per-(device, stream) workspace for split-K partials.  Calls on one stream are ordered by the
// stream, so they can share it.
struct GemvWorkspace {
    void* base = nullptr;
    size_t bytes = 0;
};
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
            (void)hipFree(w.base);
            w.base = nullptr;
            w.bytes = 0;
        }
        const size_t sz = need < ((size_t)1 << 20) ? ((size_t)1 << 20) : need;
        e = hipMalloc(&w.base, sz);
        if (e != hipSuccess) return TV_E_NOMEM;
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

struct GemvPlan {
    int nl, threads, nslices;
};

// Column strip width and K split (measured on MI355X for x[1|8,4096] @ W[4096,11008] bf16):
// 128-byte strips (NL = 8) over the whole K with 512 threads stream W best for M <= 2; wider
// strips with a 2-way K split suit M > 2, whose 8 accumulator rows limit occupancy.  K is split
// further only when the strips cannot give every CU a workgroup.
static GemvPlan gemv_plan(const GemmDesc& d) {
    const int vec = 16 / (int)dtype_size(d.dtype_a);
    GemvPlan p = d.M <= 2 ? GemvPlan{8, 512, 1} : GemvPlan{16, 256, 2};
    const int64_t nblk = ((int64_t)d.N + p.nl * vec - 1) / (p.nl * vec) * d.batch;
    const int unit = (p.threads / p.nl) * vec;
    const int max_s = (d.K + 2 * unit - 1) / (2 * unit);
    int s = p.nslices;
    if (nblk * s < 128) s = (int)((256 + nblk - 1) / nblk);
    p.nslices = s < max_s ? s : max_s;
    if (p.nslices < 1) p.nslices = 1;
    return p;
}

template <typename T, int MR, int NL, int THREADS>
static int gemv_run(const GemmDesc& d, hipStream_t stream, int nslices) {
    constexpr int VEC = 16 / sizeof(T);
    constexpr int NB = NL * VEC;
    constexpr int KL = THREADS / NL;
    using Acc = typename GemvTraits<T>::Acc;
    const int nblk = (d.N + NB - 1) / NB;
    const int unit = KL * VEC;
    int S = nslices < 1 ? 1 : nslices;
    int kslice = (d.K + S - 1) / S;
    kslice = (kslice + unit - 1) / unit * unit;
    if (kslice < unit) kslice = unit;
    S = (d.K + kslice - 1) / kslice;
    if (S < 1) S = 1;

    GemvArgs g;
    g.d = d;
    g.kslice = kslice;
    g.nslices = S;
    g.nblk = nblk;
    g.ws = nullptr;
    if (S > 1) {
        int rc = get_workspace(stream, (size_t)S * d.batch * MR * d.N * sizeof(Acc), &g.ws);
        if (rc) return rc;
    }
    const int64_t nwg = (int64_t)nblk * d.batch;
    if (nwg > 0x7FFFFFFF) return TV_E_SHAPE;
    hipLaunchKernelGGL((gemv_ncontig_kernel<T, MR, NL, THREADS>), dim3((unsigned)nwg, S), dim3(THREADS), 0, stream, g);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || S == 1) return e;
    const int64_t total = (int64_t)d.batch * d.M * d.N;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL((gemv_reduce_kernel<Acc>), dim3((unsigned)blocks), dim3(256), 0, stream, g, MR);
    return hipGetLastError();
}

template <typename T, int MR>
static int gemv_dispatch_cfg(const GemmDesc& d, hipStream_t stream, const GemvPlan& p) {
    if (p.nl == 4 && p.threads == 256) return gemv_run<T, MR, 4, 256>(d, stream, p.nslices);
    if (p.nl == 8 && p.threads == 512) return gemv_run<T, MR, 8, 512>(d, stream, p.nslices);
    if (p.nl == 8 && p.threads == 1024) return gemv_run<T, MR, 8, 1024>(d, stream, p.nslices);
    if (p.nl == 16 && p.threads == 256) return gemv_run<T, MR, 16, 256>(d, stream, p.nslices);
    return TV_E_UNSUPPORTED;
}

template <typename T>
static int gemv_dispatch_mr(const GemmDesc& d, hipStream_t stream, const GemvPlan& p) {
    if (d.M <= 1) return gemv_dispatch_cfg<T, 1>(d, stream, p);
    if (d.M <= 2) return gemv_dispatch_cfg<T, 2>(d, stream, p);
    if (d.M <= 4) return gemv_dispatch_cfg<T, 4>(d, stream, p);
    return gemv_dispatch_cfg<T, 8>(d, stream, p);
}

int launch_gemv_plan(const GemmDesc& d, hipStream_t stream, int nl, int threads, int nslices) {
    if (!gemv_layout_ok(d)) return TV_E_UNSUPPORTED;
    if (d.N == 0 || d.batch == 0) return 0;
    const GemvPlan p{nl, threads, nslices};
    switch (d.dtype_a) {
        case TV_FLOAT32: return gemv_dispatch_mr<float>(d, stream, p);
        case TV_BFLOAT16: return gemv_dispatch_mr<__bf16>(d, stream, p);
        case TV_FLOAT16: return gemv_dispatch_mr<_Float16>(d, stream, p);
        case TV_INT8: return gemv_dispatch_mr<int8_t>(d, stream, p);
        default: return TV_E_UNSUPPORTED;
    }
}

int launch_gemv(const GemmDesc& d, hipStream_t stream) {
    if (!gemv_layout_ok(d)) return TV_E_UNSUPPORTED;
    const GemvPlan p = gemv_plan(d);
    return launch_gemv_plan(d, stream, p.nl, p.threads, p.nslices);
}

} // namespace tvk
