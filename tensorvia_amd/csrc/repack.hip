// Strided view -> contiguous copy (TensorImpl::clone_as_contiguous of the HIP backend, and the
// materialising ops::Transpose).  Restates RepackImpl<Device::CUDA> (reference
// src/backend/cuda/repack.cu:5-54) without its per-call device allocations: shape and strides travel
// in the kernel arguments.  Three kernels, by the view's layout:
//  * rows: the innermost dimension is contiguous in the source and rows are 16-byte aligned; each
//    thread moves 16 bytes, so reads and writes are whole 16-byte accesses;
//  * transpose: the last two dimensions are swapped (source stride 1 on the next-to-last dimension,
//    as K.permute(0, 2, 1)); 64 x 64 element tiles go through LDS, so reads run along the source's
//    contiguous dimension and writes along the destination's (16-bit elements in 4-byte pairs when
//    the view allows);
//  * element: anything else, one element per thread, consecutive threads writing consecutive
//    destination elements.
#include "tv_kernels.h"

namespace tvk {

struct RepackDesc {
    int64_t shape[TV_MAX_DIMS];
    int64_t strides[TV_MAX_DIMS];
    int ndim;
    int64_t numel;
    const void* src;
    void* dst;
};

// Source element offset of the first element of "outer" index o over dimensions [0, nd).
__device__ inline int64_t outer_offset(const RepackDesc& r, int nd, int64_t o) {
    int64_t off = 0;
    for (int d = nd - 1; d >= 0; --d) {
        const int64_t c = o % r.shape[d];
        o /= r.shape[d];
        off += c * r.strides[d];
    }
    return off;
}

template <typename E>
__global__ __launch_bounds__(256) void repack_kernel(RepackDesc r) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < r.numel; i += stride)
        static_cast<E*>(r.dst)[i] = static_cast<const E*>(r.src)[outer_offset(r, r.ndim, i)];
}

// Rows of CPR 16-byte chunks: chunk c of destination row w comes from the row's source offset.
__global__ __launch_bounds__(256) void repack_rows_kernel(RepackDesc r, int64_t rows, int cpr, int es) {
    const int64_t total = rows * cpr;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t w = i / cpr;
        const int c = (int)(i - w * cpr);
        const char* s = static_cast<const char*>(r.src) + outer_offset(r, r.ndim - 1, w) * es + (int64_t)c * 16;
        *reinterpret_cast<u32x4*>(static_cast<char*>(r.dst) + i * 16) = *reinterpret_cast<const u32x4*>(s);
    }
}

// dst[o][i][j] = src[outer(o) + i + j * sC]: tiles of 64 (i) x 64 (j) elements.  Loads: lane l of a
// tile row reads i = i0 + l % 64 (contiguous in the source); stores: lane l writes j = j0 + l % 64
// (contiguous in the destination).  The LDS tile is padded by one element per row.
template <typename E>
__global__ __launch_bounds__(256) void repack_transpose_kernel(RepackDesc r, int64_t tiles_i, int64_t tiles_j) {
    __shared__ E tile[64][65];
    const int nd = r.ndim;
    const int64_t R = r.shape[nd - 2], C = r.shape[nd - 1], sC = r.strides[nd - 1];
    const int64_t per_outer = tiles_i * tiles_j;
    const int64_t total = per_outer * (r.numel / (R * C));
    const int l = threadIdx.x & 63, q = threadIdx.x >> 6;
    const E* src = static_cast<const E*>(r.src);
    E* dst = static_cast<E*>(r.dst);
    for (int64_t t = blockIdx.x; t < total; t += gridDim.x) {
        const int64_t o = t / per_outer;
        const int64_t rem = t - o * per_outer;
        const int64_t i0 = (rem / tiles_j) * 64, j0 = (rem % tiles_j) * 64;
        const int64_t base = outer_offset(r, nd - 2, o);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int jj = q + 4 * k;
            if (i0 + l < R && j0 + jj < C) tile[jj][l] = src[base + (i0 + l) + (j0 + jj) * sC];
        }
        __syncthreads();
        E* out = dst + o * R * C;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int ii = q + 4 * k;
            if (i0 + ii < R && j0 + l < C) out[(i0 + ii) * C + j0 + l] = tile[l][ii];
        }
        __syncthreads();
    }
}

// 16-bit elements moved in pairs: the same tiles, with 4-byte loads of two consecutive i and 4-byte
// stores of two consecutive j.  Requires even R and C, even outer strides and 4-byte aligned
// buffers (checked by the launcher), so every pair lies inside the view and is aligned.
__global__ __launch_bounds__(256) void repack_transpose16_kernel(RepackDesc r, int64_t tiles_i, int64_t tiles_j) {
    __shared__ uint16_t tile[64][66];
    const int nd = r.ndim;
    const int64_t R = r.shape[nd - 2], C = r.shape[nd - 1], sC = r.strides[nd - 1];
    const int64_t per_outer = tiles_i * tiles_j;
    const int64_t total = per_outer * (r.numel / (R * C));
    const int p = threadIdx.x & 31, q = threadIdx.x >> 5; // pair index, row group (8)
    const uint16_t* src = static_cast<const uint16_t*>(r.src);
    uint16_t* dst = static_cast<uint16_t*>(r.dst);
    for (int64_t t = blockIdx.x; t < total; t += gridDim.x) {
        const int64_t o = t / per_outer;
        const int64_t rem = t - o * per_outer;
        const int64_t i0 = (rem / tiles_j) * 64, j0 = (rem % tiles_j) * 64;
        const int64_t base = outer_offset(r, nd - 2, o);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int jj = q + 8 * k;
            if (i0 + 2 * p < R && j0 + jj < C) {
                const unsigned v = *reinterpret_cast<const unsigned*>(src + base + (i0 + 2 * p) + (j0 + jj) * sC);
                tile[jj][2 * p] = (uint16_t)(v & 0xFFFFu);
                tile[jj][2 * p + 1] = (uint16_t)(v >> 16);
            }
        }
        __syncthreads();
        uint16_t* out = dst + o * R * C;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int ii = q + 8 * k;
            if (i0 + ii < R && j0 + 2 * p < C) {
                const unsigned v = (unsigned)tile[2 * p][ii] | ((unsigned)tile[2 * p + 1][ii] << 16);
                *reinterpret_cast<unsigned*>(out + (i0 + ii) * C + j0 + 2 * p) = v;
            }
        }
        __syncthreads();
    }
}

static unsigned grid_for(int64_t items, int64_t per_block) {
    int64_t blocks = (items + per_block - 1) / per_block;
    if (blocks > 65536) blocks = 65536;
    return (unsigned)(blocks < 1 ? 1 : blocks);
}

template <typename E>
static int launch_transpose(const RepackDesc& r, hipStream_t stream) {
    const int nd = r.ndim;
    const int64_t R = r.shape[nd - 2], C = r.shape[nd - 1];
    const int64_t tiles_i = (R + 63) / 64, tiles_j = (C + 63) / 64;
    const int64_t total = tiles_i * tiles_j * (r.numel / (R * C));
    if constexpr (sizeof(E) == 2) {
        bool pairs = R % 2 == 0 && C % 2 == 0 && r.strides[nd - 1] % 2 == 0 &&
                     (reinterpret_cast<uintptr_t>(r.src) % 4) == 0 && (reinterpret_cast<uintptr_t>(r.dst) % 4) == 0;
        for (int d = 0; d < nd - 2; ++d)
            if (r.shape[d] > 1 && r.strides[d] % 2 != 0) pairs = false;
        if (pairs) {
            hipLaunchKernelGGL(repack_transpose16_kernel, dim3(grid_for(total, 1)), dim3(256), 0, stream, r, tiles_i, tiles_j);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL(repack_transpose_kernel<E>, dim3(grid_for(total, 1)), dim3(256), 0, stream, r, tiles_i, tiles_j);
    return hipGetLastError();
}

// Zero-padded row copy of a GEMM operand (launch_gemm_mfma uses it for operands contiguous along
// one dimension whose rows are not whole 16-byte chunks): destination row w = batch * rows + row
// holds the source row's L elements, then zeros up to P.  One thread per 16-byte destination
// chunk, consecutive threads on consecutive chunks (rows run on one after the other).  A chunk
// wholly inside its row is read with the widest loads the row start's alignment allows (16, 8 or
// 4 bytes; the same for every chunk of a row, since chunks are 16 bytes apart); a row's last,
// partial chunk element by element.  IDX: 32-bit index arithmetic when the chunk count allows.
template <typename E, typename IDX>
__global__ __launch_bounds__(256) void pad_rows_kernel(const E* src, E* dst, int64_t rows, int64_t nrows, int64_t s_row,
                                                       int64_t s_batch, int64_t L, int64_t P) {
    constexpr int V = 16 / (int)sizeof(E);
    struct Chunk {
        E e[V];
    };
    const IDX cpr = (IDX)(P / V);
    const IDX total = (IDX)nrows * cpr;
    const IDX rws = (IDX)rows;
    const IDX stride = (IDX)gridDim.x * blockDim.x;
    for (IDX i = (IDX)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const IDX w = i / cpr, c = i - w * cpr;
        const IDX b = rws == (IDX)nrows ? 0 : w / rws, r = w - b * rws;
        const E* s = src + (int64_t)b * s_batch + (int64_t)r * s_row;
        const int64_t x0 = (int64_t)c * V;
        const char* q = reinterpret_cast<const char*>(s + x0);
        const unsigned al = (unsigned)(reinterpret_cast<uintptr_t>(s) & 15);
        u32x4 v;
        if (x0 + V <= L && al == 0) {
            v = *reinterpret_cast<const u32x4*>(q);
        } else if (x0 + V <= L && (al & 7) == 0) {
            const uint2 lo = reinterpret_cast<const uint2*>(q)[0], hi = reinterpret_cast<const uint2*>(q)[1];
            v = u32x4{lo.x, lo.y, hi.x, hi.y};
        } else if (x0 + V <= L && (al & 3) == 0) {
            const unsigned* u = reinterpret_cast<const unsigned*>(q);
            v = u32x4{u[0], u[1], u[2], u[3]};
        } else {
            Chunk t;
#pragma unroll
            for (int e = 0; e < V; ++e) t.e[e] = x0 + e < L ? s[x0 + e] : E(0);
            v = __builtin_bit_cast(u32x4, t);
        }
        *reinterpret_cast<u32x4*>(dst + (int64_t)w * P + x0) = v;
    }
}

int launch_pad_rows(const void* src, void* dst, int es, int64_t nb, int64_t rows, int64_t s_row, int64_t s_batch, int64_t L,
                    int64_t P, hipStream_t stream) {
    const int64_t nrows = nb * rows;
    if (nrows <= 0 || L <= 0 || P < L || (P * es) % 16 != 0) return TV_E_SHAPE;
    const int64_t chunks = nrows * (P * es / 16);
    const unsigned grid = grid_for(chunks, 256);
    const bool small = chunks < ((int64_t)1 << 31);
#define TV_PAD(E)                                                                                                      \
    if (small)                                                                                                         \
        hipLaunchKernelGGL((pad_rows_kernel<E, uint32_t>), dim3(grid), dim3(256), 0, stream, static_cast<const E*>(src), \
                           static_cast<E*>(dst), rows, nrows, s_row, s_batch, L, P);                                  \
    else                                                                                                               \
        hipLaunchKernelGGL((pad_rows_kernel<E, int64_t>), dim3(grid), dim3(256), 0, stream, static_cast<const E*>(src),  \
                           static_cast<E*>(dst), rows, nrows, s_row, s_batch, L, P);
    switch (es) {
        case 1: TV_PAD(uint8_t) break;
        case 2: TV_PAD(uint16_t) break;
        case 4: TV_PAD(uint32_t) break;
        default: return TV_E_DTYPE;
    }
#undef TV_PAD
    return hipGetLastError();
}

int launch_repack(const tv_repack_args* a, hipStream_t stream) {
    RepackDesc r;
    r.ndim = a->ndim;
    r.numel = 1;
    for (int d = 0; d < a->ndim; ++d) {
        r.shape[d] = a->shape[d];
        r.strides[d] = a->strides[d];
        r.numel *= a->shape[d];
    }
    r.src = a->src;
    r.dst = a->dst;
    if (r.numel == 0) return 0;
    const int es = a->elem_size;
    if (es != 1 && es != 2 && es != 4 && es != 8) return TV_E_DTYPE;
    const int nd = r.ndim;

    // Rows: contiguous innermost dimension in whole, aligned 16-byte chunks.
    if (nd >= 1 && r.strides[nd - 1] == 1 && (r.shape[nd - 1] * es) % 16 == 0 &&
        (reinterpret_cast<uintptr_t>(r.src) % 16) == 0 && (reinterpret_cast<uintptr_t>(r.dst) % 16) == 0) {
        bool aligned = true;
        for (int d = 0; d < nd - 1; ++d)
            if (r.shape[d] > 1 && (r.strides[d] * es) % 16 != 0) aligned = false;
        const int64_t cpr = r.shape[nd - 1] * es / 16;
        if (aligned && cpr <= 0x7FFFFFFF) {
            const int64_t rows = r.numel / r.shape[nd - 1];
            hipLaunchKernelGGL(repack_rows_kernel, dim3(grid_for(rows * cpr, 256)), dim3(256), 0, stream, r, rows, (int)cpr, es);
            return hipGetLastError();
        }
    }
    // Transpose of the last two dimensions.
    if (nd >= 2 && r.strides[nd - 2] == 1 && r.strides[nd - 1] != 1 && r.shape[nd - 2] > 1 && r.shape[nd - 1] > 1) {
        switch (es) {
            case 1: return launch_transpose<uint8_t>(r, stream);
            case 2: return launch_transpose<uint16_t>(r, stream);
            case 4: return launch_transpose<uint32_t>(r, stream);
            default: return launch_transpose<uint64_t>(r, stream);
        }
    }
    const unsigned blocks = grid_for(r.numel, 256);
    switch (es) {
        case 1: hipLaunchKernelGGL(repack_kernel<uint8_t>, dim3(blocks), dim3(256), 0, stream, r); break;
        case 2: hipLaunchKernelGGL(repack_kernel<uint16_t>, dim3(blocks), dim3(256), 0, stream, r); break;
        case 4: hipLaunchKernelGGL(repack_kernel<uint32_t>, dim3(blocks), dim3(256), 0, stream, r); break;
        default: hipLaunchKernelGGL(repack_kernel<uint64_t>, dim3(blocks), dim3(256), 0, stream, r); break;
    }
    return hipGetLastError();
}

} // namespace tvk
