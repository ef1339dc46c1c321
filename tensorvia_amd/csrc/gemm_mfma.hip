// MFMA GEMM kernels for gfx950 (CDNA4): fp32, bf16, fp16 and int8 inputs.
//
// Replaces the 16x16 shared-memory tile kernel mul_cuda_3d (reference src/backend/cuda/mul.cu:8-48)
// and computes what MulImpl<CPU> computes (src/backend/cpu/mul.cpp:27-85) for these dtypes:
//   C[b,m,n] = sum_k A[b,m,k] * B[b,k,n]
// with fp32 accumulation for the float types and exact int32 accumulation for int8.
//
// Design:
//  * One workgroup computes a BM x BN output tile; its waves are laid out WAVES_M x WAVES_N and
//    each wave owns a (BM/WAVES_M) x (BN/WAVES_N) sub-tile made of 16x16 MFMA blocks.
//  * Every dtype streams 128-byte k-slices: an LDS tile row holds BK = 128/sizeof(T) consecutive
//    k values of one m (A) or one n (B).  A lane feeds the matrix core one 16-byte fragment per
//    operand per "k-group" (4 lane groups x 16 bytes = 64 bytes of k); a BK slice is 2 k-groups.
//      fp32 : 4 x v_mfma_f32_16x16x4_f32 per fragment pair
//      bf16 : 1 x v_mfma_f32_16x16x32_bf16
//      fp16 : 1 x v_mfma_f32_16x16x32_f16
//      int8 : 1 x v_mfma_i32_16x16x64_i8
//    A and B lanes use the same (lane group, element) -> k assignment, so the k order inside a
//    fragment does not affect the dot product.
//  * LDS rows are 128 bytes; the eight 16-byte chunks of row r are XOR-swizzled with
//    (r ^ (r >> 4)) & 7 so that the MFMA fragment reads (16 consecutive rows, one chunk) and the
//    transposing stores (rows 4/8/16 apart) spread over the banks.
//  * Two LDS stages: tile k+1 is fetched from HBM into registers while tile k is multiplied,
//    then written to the other stage; one barrier per k-tile.
//  * Operands are read through their element strides (views are never repacked):
//      K-contiguous rows          -> 16-byte loads straight into the LDS layout
//      M/N-contiguous (transposed) -> 16-byte loads of 4 k-rows, transposed in registers
//      any other strides          -> element gathers
//  * Batch and broadcast: the batch offset is b*s_b, so s_b = 0 broadcasts an operand.
//  * Workgroup ids are remapped so that tiles that share A rows / B columns run on the same XCD
//    (workgroups are dealt round-robin over the 8 XCDs, each with its own L2).
#include "tv_kernels.h"

namespace tvk {

// ---------------------------------------------------------------------------------------------
// Matrix-core step per input dtype.
template <typename T> struct Mfma;

template <> struct Mfma<float> {
    using Acc = f32x4;
    __device__ static inline void run(const u32x4& a, const u32x4& b, Acc& c) {
        const f32x4 av = __builtin_bit_cast(f32x4, a);
        const f32x4 bv = __builtin_bit_cast(f32x4, b);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(av[0], bv[0], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(av[1], bv[1], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(av[2], bv[2], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(av[3], bv[3], c, 0, 0, 0);
    }
};
template <> struct Mfma<__bf16> {
    using Acc = f32x4;
    __device__ static inline void run(const u32x4& a, const u32x4& b, Acc& c) {
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
};
template <> struct Mfma<_Float16> {
    using Acc = f32x4;
    __device__ static inline void run(const u32x4& a, const u32x4& b, Acc& c) {
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
};
template <> struct Mfma<int8_t> {
    using Acc = i32x4;
    __device__ static inline void run(const u32x4& a, const u32x4& b, Acc& c) {
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a),
                                                  __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
    }
};

// ---------------------------------------------------------------------------------------------
// Raw element access inside a 16-byte register chunk.
template <int ES> __device__ inline unsigned elem_bits(const u32x4& r, int e) {
    if constexpr (ES == 4) return r[e];
    else if constexpr (ES == 2) return (r[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
    else return (r[e >> 2] >> (8 * (e & 3))) & 0xFFu;
}
template <int ES> __device__ inline void set_elem_bits(u32x4& r, int e, unsigned v) {
    if constexpr (ES == 4) r[e] = v;
    else if constexpr (ES == 2) r[e >> 1] |= (v & 0xFFFFu) << (16 * (e & 1));
    else r[e >> 2] |= (v & 0xFFu) << (8 * (e & 3));
}
template <int ES> __device__ inline unsigned load_bits(const char* p) {
    if constexpr (ES == 4) return *reinterpret_cast<const unsigned*>(p);
    else if constexpr (ES == 2) return *reinterpret_cast<const unsigned short*>(p);
    else return *reinterpret_cast<const unsigned char*>(p);
}

__device__ inline int lds_swz(int row) { return (row ^ (row >> 4)) & 7; }
__device__ inline int lds_off(int row, int chunk) { return row * 128 + ((chunk ^ lds_swz(row)) << 4); }

// ---------------------------------------------------------------------------------------------
// One operand's global -> register -> LDS path.  ROWS is BM (operand A, rows = m) or BN
// (operand B, rows = n); s_r / s_k are the element strides along rows and along k.
template <int MODE, int ROWS, int THREADS, int ES>
struct TileLoader {
    static constexpr int VEC = 16 / ES;   // elements per 16-byte chunk
    static constexpr int BK = 128 / ES;   // k extent of one LDS row
    static constexpr int NCH = ROWS * 8 / THREADS; // 16-byte registers per thread
    static_assert(NCH >= 1 && ROWS * 8 % THREADS == 0, "tile rows do not divide over the threads");
    static_assert(MODE != LOAD_MNCONTIG || NCH % 4 == 0, "transposing loads need 4 k-rows");

    const char* base; // element (row0, k = 0) of this tile, as bytes
    int64_t s_r, s_k;  // element strides
    int rows_valid;    // rows of this tile inside the matrix
    int K;

    __device__ inline void load(int tid, int k0, u32x4 (&r)[NCH]) const {
        if constexpr (MODE == LOAD_KCONTIG) {
#pragma unroll
            for (int j = 0; j < NCH; ++j) {
                const int lin = tid + j * THREADS;
                const int row = lin >> 3, c = lin & 7;
                const int k = k0 + c * VEC;
                if (row < rows_valid && k < K)
                    r[j] = *reinterpret_cast<const u32x4*>(base + ((int64_t)row * s_r + k) * ES);
                else
                    r[j] = u32x4{0, 0, 0, 0};
            }
        } else if constexpr (MODE == LOAD_MNCONTIG) {
#pragma unroll
            for (int blk = 0; blk < NCH / 4; ++blk) {
                const int lin = tid + blk * THREADS;
                const int rc = lin % (ROWS / VEC), kb = lin / (ROWS / VEC);
                const int row = rc * VEC;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int k = k0 + kb * 4 + q;
                    if (row < rows_valid && k < K)
                        r[blk * 4 + q] = *reinterpret_cast<const u32x4*>(base + ((int64_t)k * s_k + row) * ES);
                    else
                        r[blk * 4 + q] = u32x4{0, 0, 0, 0};
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < NCH; ++j) {
                const int lin = tid + j * THREADS;
                const int row = lin >> 3, c = lin & 7;
                u32x4 v = {0, 0, 0, 0};
                if (row < rows_valid) {
                    const char* p = base + (int64_t)row * s_r * ES;
#pragma unroll
                    for (int e = 0; e < VEC; ++e) {
                        const int k = k0 + c * VEC + e;
                        if (k < K) set_elem_bits<ES>(v, e, load_bits<ES>(p + (int64_t)k * s_k * ES));
                    }
                }
                r[j] = v;
            }
        }
    }

    __device__ inline void store(int tid, char* lds, const u32x4 (&r)[NCH]) const {
        if constexpr (MODE == LOAD_MNCONTIG) {
#pragma unroll
            for (int blk = 0; blk < NCH / 4; ++blk) {
                const int lin = tid + blk * THREADS;
                const int rc = lin % (ROWS / VEC), kb = lin / (ROWS / VEC);
                const u32x4& r0 = r[blk * 4 + 0];
                const u32x4& r1 = r[blk * 4 + 1];
                const u32x4& r2 = r[blk * 4 + 2];
                const u32x4& r3 = r[blk * 4 + 3];
                const int byte_in_row = kb * 4 * ES; // 4 consecutive k per piece
                const int chunk = byte_in_row >> 4, within = byte_in_row & 15;
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const int row = rc * VEC + e;
                    char* dst = lds + lds_off(row, chunk) + within;
                    if constexpr (ES == 4) {
                        *reinterpret_cast<u32x4*>(dst) = u32x4{r0[e], r1[e], r2[e], r3[e]};
                    } else if constexpr (ES == 2) {
                        const unsigned lo = elem_bits<2>(r0, e) | (elem_bits<2>(r1, e) << 16);
                        const unsigned hi = elem_bits<2>(r2, e) | (elem_bits<2>(r3, e) << 16);
                        *reinterpret_cast<uint2*>(dst) = uint2{lo, hi};
                    } else {
                        *reinterpret_cast<unsigned*>(dst) = elem_bits<1>(r0, e) | (elem_bits<1>(r1, e) << 8) |
                                                            (elem_bits<1>(r2, e) << 16) | (elem_bits<1>(r3, e) << 24);
                    }
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < NCH; ++j) {
                const int lin = tid + j * THREADS;
                const int row = lin >> 3, c = lin & 7;
                *reinterpret_cast<u32x4*>(lds + lds_off(row, c)) = r[j];
            }
        }
    }
};

// ---------------------------------------------------------------------------------------------
template <typename T_, int BM_, int BN_, int WAVES_M_, int WAVES_N_, int AMODE_, int BMODE_>
struct GemmCfg {
    using T = T_;
    static constexpr int BM = BM_, BN = BN_, WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
    static constexpr int AMODE = AMODE_, BMODE = BMODE_;
    static constexpr int ES = sizeof(T);
    static constexpr int BK = 128 / ES;
    static constexpr int THREADS = WAVES_M * WAVES_N * 64;
    static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    static constexpr int FM = WM / 16, FN = WN / 16;
    static constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile must be whole 16x16 blocks");
};

template <typename TC> __device__ inline TC to_out(float v) { return static_cast<TC>(v); }

// Output conversion + store of one accumulator element.  int8 output keeps the low byte of the
// exact int32 sum (two's-complement wrap), the reference CPU backend's int8 result.
template <typename Acc>
__device__ inline void store_out(void* C, int64_t idx, int dtype_c, Acc v) {
    if constexpr (__is_same(Acc, int)) {
        if (dtype_c == TV_INT8) static_cast<int8_t*>(C)[idx] = static_cast<int8_t>(v);
        else static_cast<int32_t*>(C)[idx] = v;
    } else {
        if (dtype_c == TV_BFLOAT16) static_cast<__bf16*>(C)[idx] = static_cast<__bf16>(v);
        else if (dtype_c == TV_FLOAT16) static_cast<_Float16*>(C)[idx] = static_cast<_Float16>(v);
        else static_cast<float*>(C)[idx] = v;
    }
}

template <class C>
__global__ __launch_bounds__(C::THREADS) void gemm_mfma_kernel(GemmDesc d, int tiles_m, int tiles_n, int group_m) {
    using T = typename C::T;
    using Op = Mfma<T>;
    using Acc = typename Op::Acc;
    constexpr int ES = C::ES;

    __shared__ __attribute__((aligned(16))) char smem[2 * C::STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;

    // Workgroup -> tile.  The hardware deals workgroup ids round-robin over the 8 XCDs; undo that
    // so that a contiguous range of logical tiles lands on one XCD, then walk tiles in groups of
    // `group_m` tile-rows so neighbouring workgroups share A rows and B columns in that XCD's L2.
    int bid = blockIdx.x;
    const int nwg = gridDim.x;
    if ((nwg & 7) == 0) bid = (bid & 7) * (nwg >> 3) + (bid >> 3);
    const int per_batch = tiles_m * tiles_n;
    const int b = bid / per_batch;
    int r = bid - b * per_batch;
    const int span = group_m * tiles_n;
    const int g = r / span;
    const int first_m = g * group_m;
    const int gsz = min(tiles_m - first_m, group_m);
    r -= g * span;
    const int tm = first_m + r % gsz;
    const int tn = r / gsz;
    const int m0 = tm * C::BM, n0 = tn * C::BN;

    TileLoader<C::AMODE, C::BM, C::THREADS, ES> la;
    la.base = static_cast<const char*>(d.A) + ((int64_t)b * d.sa_b + (int64_t)m0 * d.sa_m) * ES;
    la.s_r = d.sa_m; la.s_k = d.sa_k; la.rows_valid = d.M - m0; la.K = d.K;
    TileLoader<C::BMODE, C::BN, C::THREADS, ES> lb;
    lb.base = static_cast<const char*>(d.B) + ((int64_t)b * d.sb_b + (int64_t)n0 * d.sb_n) * ES;
    lb.s_r = d.sb_n; lb.s_k = d.sb_k; lb.rows_valid = d.N - n0; lb.K = d.K;

    Acc acc[C::FM][C::FN];
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j) acc[i][j] = Acc{0, 0, 0, 0};

    u32x4 ra[decltype(la)::NCH];
    u32x4 rb[decltype(lb)::NCH];

    const int nk = (d.K + C::BK - 1) / C::BK;
    la.load(tid, 0, ra);
    lb.load(tid, 0, rb);
    la.store(tid, smem, ra);
    lb.store(tid, smem + C::A_BYTES, rb);
    __syncthreads();

    const int frag_row = lane & 15, frag_grp = lane >> 4;
    for (int kt = 0; kt < nk; ++kt) {
        char* sa = smem + (kt & 1) * C::STAGE;
        char* sb = sa + C::A_BYTES;
        const bool more = kt + 1 < nk;
        if (more) {
            la.load(tid, (kt + 1) * C::BK, ra);
            lb.load(tid, (kt + 1) * C::BK, rb);
        }
#pragma unroll
        for (int kg = 0; kg < 2; ++kg) {
            const int chunk = kg * 4 + frag_grp;
            u32x4 af[C::FM], bf[C::FN];
#pragma unroll
            for (int i = 0; i < C::FM; ++i) {
                const int row = wm * C::WM + i * 16 + frag_row;
                af[i] = *reinterpret_cast<const u32x4*>(sa + lds_off(row, chunk));
            }
#pragma unroll
            for (int j = 0; j < C::FN; ++j) {
                const int row = wn * C::WN + j * 16 + frag_row;
                bf[j] = *reinterpret_cast<const u32x4*>(sb + lds_off(row, chunk));
            }
#pragma unroll
            for (int i = 0; i < C::FM; ++i)
#pragma unroll
                for (int j = 0; j < C::FN; ++j) Op::run(af[i], bf[j], acc[i][j]);
        }
        if (more) {
            char* na = smem + ((kt + 1) & 1) * C::STAGE;
            la.store(tid, na, ra);
            lb.store(tid, na + C::A_BYTES, rb);
        }
        __syncthreads();
    }

    // Epilogue: 16x16 block (i, j): lane holds rows 4*(lane/16)+q, column lane%16.
    char* cbase = static_cast<char*>(d.C);
    const size_t csz = dtype_size(d.dtype_c);
    void* Cb = cbase + (int64_t)b * d.sc_b * csz;
#pragma unroll
    for (int i = 0; i < C::FM; ++i) {
#pragma unroll
        for (int j = 0; j < C::FN; ++j) {
            const int col = n0 + wn * C::WN + j * 16 + (lane & 15);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int row = m0 + wm * C::WM + i * 16 + (lane >> 4) * 4 + q;
                if (row < d.M && col < d.N)
                    store_out(Cb, (int64_t)row * d.sc_m + (int64_t)col * d.sc_n, d.dtype_c, acc[i][j][q]);
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Host side: pick the operand load modes and the tile configuration.
static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Mode for one operand.  `rows` extent R, strides s_r (along rows), s_k (along k), s_b (batch).
static int pick_mode(const void* p, int64_t R, int64_t K, int64_t s_r, int64_t s_k, int64_t s_b, int64_t batch, int es) {
    const int64_t vec = 16 / es;
    const bool ok_ptr = aligned16(p);
    const bool ok_b = batch <= 1 || s_b % vec == 0;
    if (s_k == 1 && ok_ptr && ok_b && K % vec == 0 && (R <= 1 || s_r % vec == 0)) return LOAD_KCONTIG;
    if (s_r == 1 && ok_ptr && ok_b && R % vec == 0 && (K <= 1 || s_k % vec == 0)) return LOAD_MNCONTIG;
    return LOAD_GENERIC;
}

template <class C>
static int run_cfg(const GemmDesc& d, hipStream_t stream, int group_m) {
    const int tiles_m = (d.M + C::BM - 1) / C::BM;
    const int tiles_n = (d.N + C::BN - 1) / C::BN;
    const int64_t nwg = (int64_t)tiles_m * tiles_n * d.batch;
    if (nwg <= 0) return 0;
    if (nwg > 0x7FFFFFFF) return TV_E_SHAPE;
    hipLaunchKernelGGL(gemm_mfma_kernel<C>, dim3((unsigned)nwg), dim3(C::THREADS), 0, stream, d, tiles_m, tiles_n, group_m);
    return hipGetLastError();
}

template <typename T, int BM, int BN, int WMW, int WNW>
static int run_modes(const GemmDesc& d, hipStream_t stream, int am, int bm, int group_m) {
#define TV_CASE(A_, B_) \
    if (am == A_ && bm == B_) return run_cfg<GemmCfg<T, BM, BN, WMW, WNW, A_, B_>>(d, stream, group_m);
    TV_CASE(LOAD_KCONTIG, LOAD_MNCONTIG)
    TV_CASE(LOAD_KCONTIG, LOAD_KCONTIG)
    TV_CASE(LOAD_KCONTIG, LOAD_GENERIC)
    TV_CASE(LOAD_MNCONTIG, LOAD_MNCONTIG)
    TV_CASE(LOAD_MNCONTIG, LOAD_KCONTIG)
    TV_CASE(LOAD_MNCONTIG, LOAD_GENERIC)
    TV_CASE(LOAD_GENERIC, LOAD_MNCONTIG)
    TV_CASE(LOAD_GENERIC, LOAD_KCONTIG)
    TV_CASE(LOAD_GENERIC, LOAD_GENERIC)
#undef TV_CASE
    return TV_E_UNSUPPORTED;
}

int launch_gemm_mfma(const GemmDesc& d, hipStream_t stream) {
    const int es = (int)dtype_size(d.dtype_a);
    const int am = pick_mode(d.A, d.M, d.K, d.sa_m, d.sa_k, d.sa_b, d.batch, es);
    const int bm = pick_mode(d.B, d.N, d.K, d.sb_n, d.sb_k, d.sb_b, d.batch, es);
    switch (d.dtype_a) {
        case TV_FLOAT32: return run_modes<float, 128, 128, 2, 2>(d, stream, am, bm, 8);
        case TV_BFLOAT16: return run_modes<__bf16, 256, 256, 2, 4>(d, stream, am, bm, 8);
        case TV_FLOAT16: return run_modes<_Float16, 256, 256, 2, 4>(d, stream, am, bm, 8);
        case TV_INT8: return run_modes<int8_t, 256, 256, 2, 4>(d, stream, am, bm, 8);
        default: return TV_E_DTYPE;
    }
}

} // namespace tvk
