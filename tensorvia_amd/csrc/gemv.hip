// Skinny-M (M <= 8) matmul for decode-shaped calls: x[b, M, K] @ W[b, K, N], W row-major
// (N-contiguous).  HBM-bound: W is streamed exactly once with 16-byte buffer loads.  Two kernels:
// a packed-dot-product kernel (gemv_kernel, no matrix cores) and a matrix-core kernel
// (gemv_mfma_kernel) that serves 16-bit W of 64 or more columns at every M and int8 W of 128 or
// more columns at M >= 3, where the dot products would make the VALU, not HBM, the bound.  A third
// kernel (gemv_kt_kernel, below) serves 16-bit and int8 W stored K-contiguous (x @ W^T, W[N, K])
// at M <= 16.
//
// The reference computes these shapes with mul_kernel_basic (src/backend/cpu/mul.cpp:7-25), chosen
// because batch*M*N < 2^20 (mul.cpp:87-96), on one OpenMP thread when M = 1.
//
// Work split (measured on MI355X for W[4096, 11008] bf16; one CU alone streams only about
// 29 GB/s, so W reaches HBM speed only when every CU streams, and partial 128-byte lines shared by
// two workgroups cost more than they save):
//  * a workgroup owns a strip of NB = NL * VEC columns (NL lanes x 16 bytes of each W row; 128-byte
//    strips when N allows) and one K-slice; K is cut into S slices so that there are several
//    hundred workgroups (W[4096, 11008]: 172 strips x 4 slices), which the dispatcher balances
//    over the CUs;
//  * the KL = THREADS / NL k-lanes of a workgroup take groups of GR = 4 consecutive rows in turn
//    (group q goes to k-lane q mod KL), keeping DEPTH groups (16 loads) in flight per thread; loads
//    past the end of the slice or right of column N use an out-of-range buffer offset and return
//    zeros, so the loop has no branches;
//  * x's slice is staged in LDS once per workgroup (while the first W loads are in flight);
//  * products use the packed dot instructions over row pairs / quads of W, with the pairs built by
//    v_perm_b32: v_dot2_f32_bf16 / v_dot2_f32_f16 (fp32 accumulation), v_dot4_i32_i8 (exact int32
//    accumulation); fp32 uses fp32 FMA.  16-bit W with N >= 64, and int8 W with N >= 128 at
//    M >= 3, go to gemv_mfma_kernel instead (matrix cores, W transposed through LDS);
//  * the k-lanes are summed through LDS in a fixed order;
//  * with S > 1 each workgroup publishes its strip partial to slot s (agent-scope atomic stores,
//    waited for before the workgroup counts itself in with an agent-scope atomic, see
//    publish_and_count); the workgroup that arrives last sums slots 0..S-1 in order
//    (deterministic), writes C and resets the counter.  No workgroup waits for another, and there
//    is no second kernel.
#include "gemm_mfma_impl.h"
#include "tv_kernels.h"

namespace tvk {

template <typename T> struct GemvTraits;
template <> struct GemvTraits<float> { using Acc = float; };
template <> struct GemvTraits<__bf16> { using Acc = float; };
template <> struct GemvTraits<_Float16> { using Acc = float; };
template <> struct GemvTraits<int8_t> { using Acc = int; };

constexpr int kGemvThreads = 256;
constexpr int kGemvGroupRows = 4;  // GR
constexpr int kGemvDepth = 4;      // groups in flight per thread
constexpr int kGemvXBytes = 65536; // LDS for x's slice at MR = 8
constexpr int kGemvMaxSlices = 16; // K slices combined in-kernel

// Rows of x staged per slice: MR * kslice * sizeof(T) <= kGemvXBytes at MR = 8.
template <typename T> constexpr int gemv_kcap() { return kGemvXBytes / (8 * (int)sizeof(T)); }

struct GemvArgs {
    GemmDesc d;
    int kslice;  // rows per K-slice (a multiple of VEC, at most gemv_kcap<T>())
    int nslices; // S
    int nblk;    // strips per batch
    int* cnt;    // [batch * nblk] arrival counters (S > 1), zero between launches
    void* part;  // [batch * nblk][S][MR][NB] strip partials (S > 1)
};

template <typename T, int MR>
__device__ inline void gemv_group(const u32x4 (&w)[kGemvGroupRows], const char* xs, int xstride,
                                  typename GemvTraits<T>::Acc (&acc)[MR][16 / sizeof(T)]) {
    constexpr int VEC = 16 / sizeof(T);
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const f32x4 xv = *reinterpret_cast<const f32x4*>(xs + m * xstride);
#pragma unroll
            for (int r = 0; r < kGemvGroupRows; ++r) {
                const f32x4 wf = __builtin_bit_cast(f32x4, w[r]);
#pragma unroll
                for (int e = 0; e < VEC; ++e) acc[m][e] = __builtin_fmaf(xv[r], wf[e], acc[m][e]);
            }
        }
    } else if constexpr (sizeof(T) == 2) {
        // pair p = rows (2p, 2p+1); dword t of a row holds columns 2t, 2t+1
        unsigned lo[2][4], hi[2][4];
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                lo[p][t] = __builtin_amdgcn_perm(w[2 * p + 1][t], w[2 * p][t], 0x05040100u);
                hi[p][t] = __builtin_amdgcn_perm(w[2 * p + 1][t], w[2 * p][t], 0x07060302u);
            }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            // x rows (0,1) and (2,3) as two scalars: clang's __builtin_bit_cast of a vector
            // *element* reads element 0, so no vector type is indexed here.
            const unsigned* xr = reinterpret_cast<const unsigned*>(xs + m * xstride);
            const unsigned xp[2] = {xr[0], xr[1]};
#pragma unroll
            for (int p = 0; p < 2; ++p)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    if constexpr (__is_same(T, __bf16)) {
                        acc[m][2 * t] = __builtin_amdgcn_fdot2_f32_bf16(
                            __builtin_bit_cast(bf16x2, xp[p]), __builtin_bit_cast(bf16x2, lo[p][t]), acc[m][2 * t], false);
                        acc[m][2 * t + 1] = __builtin_amdgcn_fdot2_f32_bf16(
                            __builtin_bit_cast(bf16x2, xp[p]), __builtin_bit_cast(bf16x2, hi[p][t]), acc[m][2 * t + 1], false);
                    } else {
                        acc[m][2 * t] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, xp[p]),
                                                               __builtin_bit_cast(f16x2, lo[p][t]), acc[m][2 * t], false);
                        acc[m][2 * t + 1] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, xp[p]),
                                                                   __builtin_bit_cast(f16x2, hi[p][t]), acc[m][2 * t + 1], false);
                    }
                }
        }
    } else {
        // the four rows' bytes of column c gathered into one dword (row r in byte r)
        unsigned q[16];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const unsigned a01l = __builtin_amdgcn_perm(w[1][t], w[0][t], 0x05010400u); // r0.b0 r1.b0 r0.b1 r1.b1
            const unsigned a01h = __builtin_amdgcn_perm(w[1][t], w[0][t], 0x07030602u); // r0.b2 r1.b2 r0.b3 r1.b3
            const unsigned a23l = __builtin_amdgcn_perm(w[3][t], w[2][t], 0x05010400u);
            const unsigned a23h = __builtin_amdgcn_perm(w[3][t], w[2][t], 0x07030602u);
            q[4 * t + 0] = __builtin_amdgcn_perm(a23l, a01l, 0x05040100u);
            q[4 * t + 1] = __builtin_amdgcn_perm(a23l, a01l, 0x07060302u);
            q[4 * t + 2] = __builtin_amdgcn_perm(a23h, a01h, 0x05040100u);
            q[4 * t + 3] = __builtin_amdgcn_perm(a23h, a01h, 0x07060302u);
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const int xq = *reinterpret_cast<const int*>(xs + m * xstride);
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[m][e] = __builtin_amdgcn_sdot4(xq, (int)q[e], acc[m][e], false);
        }
    }
}

// Output value of C[b, m, n] through the fused epilogue (float accumulators only).
template <typename Acc> __device__ inline Acc gemv_epilogue(Acc v, const GemmDesc& d, int b, int m, int n) {
    if constexpr (__is_same(Acc, float))
        if (has_epilogue(d)) return epilogue_value(v, d, b, m, n);
    return v;
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

// Workgroup ids are remapped so that neighbouring column strips (which share 128-byte lines of W)
// run on the same XCD and meet in its L2 (workgroups are dealt round-robin over the 8 XCDs).
__device__ inline int xcd_remap(int bid, int nwg) {
    return (nwg & 7) == 0 ? (bid & 7) * (nwg >> 3) + (bid >> 3) : bid;
}

template <typename T, int MR, int NL, int THREADS> struct GemvShape {
    static constexpr int ES = sizeof(T);
    static constexpr int VEC = 16 / ES;
    static constexpr int NB = NL * VEC;     // columns per strip
    static constexpr int KL = THREADS / NL; // k-lanes
    static constexpr int P = KL / VEC;      // threads that sum one output
    static constexpr int KCAP = gemv_kcap<T>();
    static_assert(P >= 1 && 64 % P == 0 && P * NB == THREADS, "reduction lanes");
};

template <typename T, int MR, int NL, int THREADS>
__global__ __launch_bounds__(THREADS) void gemv_kernel(GemvArgs g) {
    using Acc = typename GemvTraits<T>::Acc;
    using S = GemvShape<T, MR, NL, THREADS>;
    constexpr int ES = S::ES, VEC = S::VEC, NB = S::NB, KL = S::KL, P = S::P;
    constexpr int GR = kGemvGroupRows, DEPTH = kGemvDepth;
    static_assert(64 % NL == 0, "n-lanes must tile a wave");
    const GemmDesc& d = g.d;

    extern __shared__ __attribute__((aligned(16))) char xs[]; // MR * kslice * ES bytes (launch size)
    __shared__ Acc red[NB * (KL + 1)];
    __shared__ int last_flag;

    const int tid = threadIdx.x;
    const int nl = tid % NL, kl = tid / NL;
    const int lin = xcd_remap(blockIdx.x, gridDim.x);
    const int b = lin / g.nblk;
    const int n0 = (lin - b * g.nblk) * NB;
    const int s = blockIdx.y;
    const int col = n0 + nl * VEC;
    const bool col_ok = col < d.N; // N % VEC == 0 is a launch precondition

    const int k0 = s * g.kslice;
    const int ks = min(d.K - k0, g.kslice); // rows of this slice, a multiple of GR
    const int ngroups = ks / GR;
    const int niter = (ngroups + KL - 1) / KL;

    // W rows [k0, k0 + ks) of batch b; row r of the slice, this lane's columns at r * rowb + colb.
    const int64_t rowb = d.sb_k * ES;
    const char* wbase = static_cast<const char*>(d.B) + ((int64_t)b * d.sb_b + (int64_t)k0 * d.sb_k) * ES;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wbase, (int64_t)(ks - 1) * rowb + (int64_t)d.N * ES);
    const unsigned colb = (unsigned)(col * ES);

    u32x4 w[DEPTH][GR];
    auto issue = [&](int slot, int j) {
        const int q = kl + j * KL;
        const bool ok = col_ok && q < ngroups;
        const unsigned base = (unsigned)(q * GR * rowb) + colb;
#pragma unroll
        for (int r = 0; r < GR; ++r) w[slot][r] = buf_load16_nt(wr, ok ? base + (unsigned)(r * rowb) : kOOB);
    };
#pragma unroll
    for (int j = 0; j < DEPTH; ++j) issue(j, j);

    // Stage x[b][0..MR)[k0 .. k0 + ks) in LDS (rows m >= M are zero).
    {
        const char* xb = static_cast<const char*>(d.A) + ((int64_t)b * d.sa_b + k0) * ES;
        const int cpr = ks * ES / 16; // 16-byte chunks per row
        for (int i = tid; i < MR * cpr; i += THREADS) {
            const int m = i / cpr, c = i - m * cpr;
            u32x4 v = {0, 0, 0, 0};
            if (m < d.M) v = *reinterpret_cast<const u32x4*>(xb + (int64_t)m * d.sa_m * ES + c * 16);
            *reinterpret_cast<u32x4*>(xs + m * ks * ES + c * 16) = v;
        }
    }
    __syncthreads();

    Acc acc[MR][VEC];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[m][e] = 0;

    const int xstride = ks * ES;
    for (int j0 = 0; j0 < niter; j0 += DEPTH) {
#pragma unroll
        for (int dd = 0; dd < DEPTH; ++dd) {
            const int j = j0 + dd;
            if (j < niter) {
                int q = kl + j * KL;
                q = q < ngroups ? q : 0; // past the end: w is zero, keep the x read in range
                gemv_group<T, MR>(w[dd], xs + q * GR * ES, xstride, acc);
                if (j + DEPTH < niter) issue(dd, j + DEPTH);
            }
        }
    }

    // Sum the k-lanes one row of x at a time: red[c * (KL + 1) + kl]; output c is summed by the P
    // consecutive threads c * P .. c * P + P - 1 (VEC partials each, in k-lane order), then a fixed
    // shuffle tree.  Thread c * P keeps the strip's result for row m in v[m].
    const int oc = tid / P, part = tid % P;
    Acc v[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        v[m] = 0;
        if (m >= d.M) break;
        __syncthreads();
#pragma unroll
        for (int e = 0; e < VEC; ++e) red[(nl * VEC + e) * (KL + 1) + kl] = acc[m][e];
        __syncthreads();
        const Acc* p = red + oc * (KL + 1) + part * VEC;
        Acc t = p[0];
#pragma unroll
        for (int i = 1; i < VEC; ++i) t += p[i];
#pragma unroll
        for (int off = 1; off < P; off <<= 1) t += __shfl_xor(t, off);
        v[m] = t;
    }

    const size_t csz = dtype_size(d.dtype_c);
    char* Cb = static_cast<char*>(d.C) + (int64_t)b * d.sc_b * csz;
    const bool writer = part == 0 && n0 + oc < d.N;
    if (g.nslices == 1) {
        if (writer)
#pragma unroll
            for (int m = 0; m < MR; ++m)
                if (m < d.M)
                    gemv_store(Cb, (int64_t)m * d.sc_m + (int64_t)(n0 + oc) * d.sc_n, d.dtype_c,
                               gemv_epilogue(v[m], d, b, m, n0 + oc));
        return;
    }

    // Publish slot s of this strip, count in; the last arriver sums the slots in order.
    const int strip = lin;
    Acc* slots = static_cast<Acc*>(g.part) + (int64_t)strip * g.nslices * MR * NB;
    if (part == 0)
#pragma unroll
        for (int m = 0; m < MR; ++m)
            if (m < d.M) slot_store(slots + ((int64_t)s * MR + m) * NB + oc, v[m]);
    publish_and_count(g.cnt + strip, g.nslices, &last_flag);
    if (!last_flag) return;
    for (int o = tid; o < MR * NB; o += THREADS) {
        const int m = o / NB, c = o - m * NB;
        if (m < d.M && n0 + c < d.N) {
            // All slot loads are issued before the first add (S <= kGemvMaxSlices).
            Acc part_v[kGemvMaxSlices];
#pragma unroll
            for (int k = 0; k < kGemvMaxSlices; ++k)
                part_v[k] = k < g.nslices ? slot_load(slots + ((int64_t)k * MR + m) * NB + c) : Acc(0);
            Acc t = part_v[0];
#pragma unroll
            for (int k = 1; k < kGemvMaxSlices; ++k)
                if (k < g.nslices) t += part_v[k];
            gemv_store(Cb, (int64_t)m * d.sc_m + (int64_t)(n0 + c) * d.sc_n, d.dtype_c, gemv_epilogue(t, d, b, m, n0 + c));
        }
    }
    slot_count_reset(g.cnt + strip);
}

// Matrix-core variant for 16-bit and int8 W (the dot-product loop above is VALU-bound at larger M:
// 16 v_dot2 or v_dot4 per x row per 64 bytes of W).  Described here for 16 bits; int8 has 128-column
// strips, 64-row chunks, v_mfma_i32_16x16x64_i8, ds_read_b64_tr_b8 and exact int32 sums.  Same
// strips (128 bytes of each W row), K slices and slot combine; inside a workgroup, the WAVES waves
// take 32-row chunks of the slice in turn (chunk c goes to wave c mod WAVES):
//  * a chunk is 4 KB: 4 nontemporal 16-byte buffer loads per lane (lane l: rows l/8 + 8q, columns
//    8 (l mod 8) ..), DEPTH chunks in flight per wave;
//  * the wave writes it to its own LDS tile (32 rows x 64 columns, row pitch 144 bytes) and reads it
//    back with ds_read_b64_tr_b16, which hands lane l the 8 consecutive rows of one column that the
//    matrix core's B operand wants (column 16 f + l mod 16, rows 8 (l / 16) ..);
//  * one v_mfma_f32_16x16x32 per 16 columns and 16-row block of x: XR = 8 stages x rows 0..7 (the
//    block's rows 8..15 are zero), XR = 16 or 32 one or two whole blocks (9 <= M <= 32), rows >= M
//    zero; D[m][n] of a block lands in lane n mod 16 + 16 (m / 4), element m mod 4, and each W
//    fragment read from LDS serves every block;
//  * the waves' partials are summed through LDS in wave order, then published as in gemv_kernel.
// A wave's LDS tile is private to it: LDS instructions of one wave execute in order, so the next
// chunk's stores cannot overtake the previous chunk's reads.
constexpr int kGemvMfmaPitch = 144;
// 4 waves with 8 KB of loads in flight each (2 chunks at 16 bits, 1 at 8): the best of 2/4/8 waves
// x 1-8 chunks on c5's W, and of 4/8 waves x 1-2 chunks on the same shape in int8.
constexpr int kGemvMfmaWaves = 4;
template <typename T> constexpr int gemv_mfma_depth() { return sizeof(T) == 2 ? 2 : 1; }

template <typename T, int WAVES, int DEPTH, int XR>
__global__ __launch_bounds__(WAVES * 64) void gemv_mfma_kernel(GemvArgs g) {
    using Acc = typename GemvTraits<T>::Acc;
    static_assert(XR == 8 || XR == 16 || XR == 32, "x rows staged: 8 (M <= 8), 16 or 32");
    constexpr int MB = XR < 16 ? 1 : XR / 16; // 16-row blocks of x
    // 16-bit: 64-column strips, 32-row chunks (v_mfma_f32_16x16x32, ds_read_b64_tr_b16); int8:
    // 128-column strips, 64-row chunks (v_mfma_i32_16x16x64_i8, ds_read_b64_tr_b8).
    constexpr int ES = sizeof(T), VEC = 16 / ES, NB = 8 * VEC, CH = 64 / ES, NQ = CH / 8, NF = NB / 16;
    constexpr int PITCH = kGemvMfmaPitch, THREADS = WAVES * 64;
    static_assert(ES == 1 || ES == 2, "16-bit or 8-bit W");
    static_assert(XR * NB % THREADS == 0, "outputs per thread");
    const GemmDesc& d = g.d;

    // x's rows (XR x kpad x ES, the launch size), and for XR > 8 also the wave partials after the
    // loop (the launch sizes the area for both: gemv_mfma_dyn_lds); XR = 8 keeps its own array.
    extern __shared__ __attribute__((aligned(16))) char xs[];
    __shared__ __attribute__((aligned(16))) char wt[WAVES][CH * PITCH];
    constexpr bool kRedInX = XR > 8;
    __shared__ Acc red_own[kRedInX ? 1 : WAVES][kRedInX ? 1 : XR][NB];
    __shared__ int last_flag;

    // The wave index from the first lane: wave-uniform to the compiler, so the loop below has scalar
    // control flow.  With a per-lane index the per-chunk guard became an exec-mask branch, and the
    // compiler waited for every load of the next chunk inside each chunk (one chunk in flight, not
    // DEPTH) and moved the accumulators between register files every chunk.
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lin = xcd_remap(blockIdx.x, gridDim.x);
    const int b = lin / g.nblk;
    const int n0 = (lin - b * g.nblk) * NB;
    const int s = blockIdx.y;
    const int k0 = s * g.kslice;
    const int ks = min(d.K - k0, g.kslice);  // a multiple of VEC, except the last slice of a padded x
    const int nch = (ks + CH - 1) / CH;
    const int kpad = nch * CH;
    const int niter = (nch - wave + WAVES - 1) / WAVES; // chunks wave, wave + WAVES, ...
    const int nsteps = (niter + DEPTH - 1) / DEPTH * DEPTH; // the loop's count: chunks past niter are zeros

    const int64_t rowb = d.sb_k * ES;
    const char* wbase = static_cast<const char*>(d.B) + ((int64_t)b * d.sb_b + (int64_t)k0 * d.sb_k) * ES;
    // The last row's range ends at N rounded up to whole chunks (N itself unless W is a padded copy).
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wbase, (int64_t)(ks - 1) * rowb + (int64_t)((d.N + VEC - 1) / VEC * VEC) * ES);
    const int r0 = lane >> 3, cc = lane & 7;
    const int col = n0 + cc * VEC;
    const bool col_ok = col < d.N; // a chunk straddling N (padded copy) reads the zero padding
    const unsigned colb = (unsigned)(col * ES);

    u32x4 w[DEPTH][NQ];
    auto issue = [&](int slot, int j) {
        const int c = wave + WAVES * j;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int r = c * CH + r0 + 8 * q;
            const bool ok = col_ok && j < niter && r < ks; // rows past the slice read as zeros
            w[slot][q] = buf_load16_nt(wr, ok ? (unsigned)(r * rowb) + colb : kOOB);
        }
    };
#pragma unroll
    for (int j = 0; j < DEPTH; ++j) issue(j, j);

    // x[b][0..XR)[k0 .. k0 + kpad) in LDS; rows >= M and columns >= ks are zero.  Four chunks per
    // thread are loaded before any is stored: each wait for an x load also waits for the W loads
    // issued before it, so the loads go out together and pay that wait once.
    {
        const char* xb = static_cast<const char*>(d.A) + ((int64_t)b * d.sa_b + k0) * ES;
        const int cpr = kpad * ES / 16;
        for (int i0 = tid; i0 < XR * cpr; i0 += 4 * THREADS) {
            u32x4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * THREADS, m = i / cpr, c = i - m * cpr;
                v[u] = u32x4{0, 0, 0, 0};
                if (i < XR * cpr && m < d.M && c * 16 < ks * ES)
                    v[u] = *reinterpret_cast<const u32x4*>(xb + (int64_t)m * d.sa_m * ES + c * 16);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * THREADS;
                if (i < XR * cpr) *reinterpret_cast<u32x4*>(xs + i * 16) = v[u];
            }
        }
    }
    __syncthreads();

    typename Mfma<T>::Acc acc[MB][NF];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int f = 0; f < NF; ++f) acc[mb][f] = typename Mfma<T>::Acc{0, 0, 0, 0};
    char* wl = wt[wave];
    const int wr_off = r0 * PITCH + cc * 16;
    // transpose reads: 16-bit, lanes 4r + c of a 16-lane group read row kb + r, columns 4c .. 4c + 3
    // (then rows + 4); 8-bit, lanes 2r + c read row kb + r, columns 8c .. 8c + 7 (then rows + 8)
    const int fr = lane & 15, kb = (lane >> 4) * (CH / 4);
    const int rd_off = ES == 2 ? (kb + (fr >> 2)) * PITCH + 8 * (fr & 3) : (kb + (fr >> 1)) * PITCH + 8 * (fr & 1);
    const bool arow = XR > 8 || fr < 8;
    const char* xa = xs + (XR > 8 ? fr : (lane & 7)) * kpad * ES + kb * ES; // block mb: + 16 mb rows
    // No per-chunk guard: the step count is a multiple of DEPTH, and a chunk past niter multiplies
    // zeros (its W loads are out of range, its x fragment is zeroed).
    for (int j0 = 0; j0 < nsteps; j0 += DEPTH) {
#pragma unroll
        for (int dd = 0; dd < DEPTH; ++dd) {
            const int j = j0 + dd;
            {
                const int c = wave + WAVES * j;
#pragma unroll
                for (int q = 0; q < NQ; ++q) *reinterpret_cast<u32x4*>(wl + wr_off + q * 8 * PITCH) = w[dd][q];
                u32x4 a[MB];
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    a[mb] = *reinterpret_cast<const u32x4*>(xa + (mb * 16 * kpad + (j < niter ? c : 0) * CH) * ES);
                    if (!arow || j >= niter) a[mb] = u32x4{0, 0, 0, 0};
                }
#pragma unroll
                for (int f = 0; f < NF; ++f) {
                    const lds_char* p = (const lds_char*)(wl + rd_off + f * 16 * ES);
                    u32x4 bf;
                    if constexpr (ES == 2) {
                        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p);
                        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 4 * PITCH));
                        const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
                        bf = u32x4{l2.x, l2.y, h2.x, h2.y};
                    } else {
                        const i32x2_t lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)p);
                        const i32x2_t hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(p + 8 * PITCH));
                        bf = u32x4{(unsigned)lo.x, (unsigned)lo.y, (unsigned)hi.x, (unsigned)hi.y};
                    }
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) Mfma<T>::run(a[mb], bf, acc[mb][f]);
                }
                issue(dd, j + DEPTH); // out of range past niter: zeros
            }
        }
    }

    // Wave partials D[m][n] (XR = 8: rows 0..7, lanes 0..31) to red, then sum the waves in order.
    if constexpr (kRedInX) __syncthreads(); // every wave is done reading x
    Acc(*red)[XR][NB] = kRedInX ? reinterpret_cast<Acc(*)[XR][NB]>(xs) : reinterpret_cast<Acc(*)[XR][NB]>(&red_own[0][0][0]);
    if (XR > 8 || lane < 32)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int f = 0; f < NF; ++f)
#pragma unroll
                for (int r = 0; r < 4; ++r) red[wave][16 * mb + 4 * (lane >> 4) + r][16 * f + (lane & 15)] = acc[mb][f][r];
    __syncthreads();
    constexpr int OPT = XR * NB / THREADS; // outputs per thread
    Acc v[OPT];
#pragma unroll
    for (int i = 0; i < OPT; ++i) {
        const int o = tid + THREADS * i, m = o / NB, c = o % NB;
        Acc t = red[0][m][c];
#pragma unroll
        for (int wv = 1; wv < WAVES; ++wv) t += red[wv][m][c];
        v[i] = t;
    }

    const size_t csz = dtype_size(d.dtype_c);
    char* Cb = static_cast<char*>(d.C) + (int64_t)b * d.sc_b * csz;
    if (g.nslices == 1) {
#pragma unroll
        for (int i = 0; i < OPT; ++i) {
            const int o = tid + THREADS * i, m = o / NB, c = o % NB;
            if (m < d.M && n0 + c < d.N)
                gemv_store(Cb, (int64_t)m * d.sc_m + (int64_t)(n0 + c) * d.sc_n, d.dtype_c, gemv_epilogue(v[i], d, b, m, n0 + c));
        }
        return;
    }

    // Publish slot s of this strip ([XR][NB] accumulators, fp32 or int32, rows < M), count in; the
    // last arriver sums the slots in order.
    const int strip = lin;
    Acc* slots = static_cast<Acc*>(g.part) + (int64_t)strip * g.nslices * XR * NB;
#pragma unroll
    for (int i = 0; i < OPT; ++i)
        if ((tid + THREADS * i) / NB < d.M)
            slot_store(slots + (int64_t)s * XR * NB + tid + THREADS * i, v[i]);
    publish_and_count(g.cnt + strip, g.nslices, &last_flag);
    if (!last_flag) return;
#pragma unroll
    for (int i = 0; i < OPT; ++i) {
        const int o = tid + THREADS * i, m = o / NB, c = o % NB;
        if (m < d.M && n0 + c < d.N) {
            Acc part_v[kGemvMaxSlices];
#pragma unroll
            for (int k = 0; k < kGemvMaxSlices; ++k)
                part_v[k] = k < g.nslices ? slot_load(slots + (int64_t)k * XR * NB + o) : Acc(0);
            Acc t = part_v[0];
#pragma unroll
            for (int k = 1; k < kGemvMaxSlices; ++k)
                if (k < g.nslices) t += part_v[k];
            gemv_store(Cb, (int64_t)m * d.sc_m + (int64_t)(n0 + c) * d.sc_n, d.dtype_c, gemv_epilogue(t, d, b, m, n0 + c));
        }
    }
    slot_count_reset(g.cnt + strip);
}


// Matrix-core GEMV for K-contiguous W (W stored [N, K] row-major, used as x @ W^T: the usual
// linear-layer layout).  The matrix core's B fragment is 8 consecutive k of one W row, so each lane
// loads it straight from memory as one 16-byte load, with no LDS transpose:
//  * a workgroup owns a strip of 16 x WAVES W rows and one K slice, and wave w the rows n0 + 16 w ..
//    n0 + 16 w + 15 over the whole slice, so x's slice is staged in LDS once for all of them (x's
//    bytes from L2 are XR / (16 WAVES) of W's);
//  * the slice is walked in 256-byte chunks of each row (128 k at 16 bits, 256 in int8), DEPTH
//    chunks in flight per wave; per chunk a lane issues 4 loads, k-steps of 4 VEC (VEC = 16 bytes
//    of k): lane l reads its row (l mod 16) at k 4 VEC q + VEC (l / 16), so each wave instruction
//    reads 64 contiguous bytes of each of 16 rows and the 4 instructions of a chunk 256 contiguous
//    bytes of each (rows >= N and k >= the slice read zeros);
//  * one v_mfma_f32_16x16x32 (int8: v_mfma_i32_16x16x64_i8, exact int32 sums) per k-step and 16-row block of x (src0 x: lane l holds x[l mod 16][VEC (l / 16)
//    ..], row pitch padded by 16 bytes; src1 W), D[m][n] landing in lane n + 16 (m / 4), element m mod 4, which the lane
//    stores, or publishes to slot s for the last-arriving slice to sum in slot order as in
//    gemv_mfma_kernel.
template <typename T> constexpr int gemv_kt_chunk() { return 256 / (int)sizeof(T); }
template <typename T, int WAVES, int DEPTH, int XR>
__global__ __launch_bounds__(WAVES * 64) void gemv_kt_kernel(GemvArgs g) {
    using Acc = typename GemvTraits<T>::Acc;
    constexpr int ES = sizeof(T), VEC = 16 / ES, KSTEP = 4 * VEC, NB = 16 * WAVES, CK = gemv_kt_chunk<T>(), NQ = CK / KSTEP;
    constexpr int MB = XR < 16 ? 1 : XR / 16;
    static_assert(ES == 1 || ES == 2, "8- or 16-bit W");
    const GemmDesc& d = g.d;

    extern __shared__ __attribute__((aligned(16))) char xs[]; // XR rows of kpad * ES + 16 bytes
    __shared__ int last_flag;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lin = xcd_remap(blockIdx.x, gridDim.x);
    const int b = lin / g.nblk;
    const int n0 = (lin - b * g.nblk) * NB;
    const int s = blockIdx.y;
    const int k0 = s * g.kslice;
    const int ks = min(d.K - k0, g.kslice); // a multiple of VEC
    const int nch = (ks + CK - 1) / CK;
    const int kpad = nch * CK;
    const int xpitch = kpad * ES + 16;
    const int nsteps = (nch + DEPTH - 1) / DEPTH * DEPTH; // chunks past nch multiply zeros

    const int fr = lane & 15, kg = lane >> 4;
    const int wrow0 = n0 + 16 * wave; // this wave's first W row
    const bool row_ok = wrow0 + fr < d.N;
    const int64_t rowb = d.sb_n * ES;
    const int nrows = max(1, min(16, d.N - wrow0));
    const char* wbase = static_cast<const char*>(d.B) + ((int64_t)b * d.sb_b + (int64_t)min(wrow0, d.N - 1) * d.sb_n + k0) * ES;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wbase, (int64_t)(nrows - 1) * rowb + (int64_t)ks * ES);
    const unsigned lane_off = (unsigned)(fr * rowb) + (unsigned)(kg * 16);

    u32x4 w[DEPTH][NQ];
    auto issue = [&](int slot, int c) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int k = c * CK + KSTEP * q + VEC * kg;
            const bool ok = row_ok && c < nch && k < ks;
            w[slot][q] = buf_load16_nt(wr, ok ? lane_off + (unsigned)((c * CK + KSTEP * q) * ES) : kOOB);
        }
    };
#pragma unroll
    for (int j = 0; j < DEPTH; ++j) issue(j, j);

    // x[b][0..XR)[k0 .. k0 + kpad) in LDS; rows >= M and columns >= ks are zero.
    {
        const char* xb = static_cast<const char*>(d.A) + ((int64_t)b * d.sa_b + k0) * ES;
        const int cpr = kpad * ES / 16;
        for (int i = tid; i < XR * cpr; i += WAVES * 64) {
            const int m = i / cpr, c = i - m * cpr;
            u32x4 v = u32x4{0, 0, 0, 0};
            if (m < d.M && c * 16 < ks * ES) v = *reinterpret_cast<const u32x4*>(xb + (int64_t)m * d.sa_m * ES + c * 16);
            *reinterpret_cast<u32x4*>(xs + m * xpitch + c * 16) = v;
        }
    }
    __syncthreads();

    typename Mfma<T>::Acc acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = typename Mfma<T>::Acc{0, 0, 0, 0};
    const bool arow = XR > 8 || fr < 8;
    const char* xa = xs + (XR > 8 ? fr : (fr & 7)) * xpitch + kg * 16; // block mb: + 16 mb rows
    for (int c0 = 0; c0 < nsteps; c0 += DEPTH) {
#pragma unroll
        for (int dd = 0; dd < DEPTH; ++dd) {
            const int c = c0 + dd;
            const int cx = c < nch ? c : 0;
#pragma unroll
            for (int q = 0; q < NQ; ++q)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    u32x4 a = *reinterpret_cast<const u32x4*>(xa + mb * 16 * xpitch + (cx * CK + KSTEP * q) * ES);
                    if (!arow || c >= nch) a = u32x4{0, 0, 0, 0};
                    Mfma<T>::run(a, w[dd][q], acc[mb]);
                }
            issue(dd, c + DEPTH); // out of range past nch: zeros
        }
    }

    // Lane (fr, kg) holds D[16 mb + 4 kg + r][wrow0 + fr], r = 0..3.
    const int n = wrow0 + fr;
    const size_t csz = dtype_size(d.dtype_c);
    char* Cb = static_cast<char*>(d.C) + (int64_t)b * d.sc_b * csz;
    if (g.nslices == 1) {
        if (n < d.N)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = 16 * mb + 4 * kg + r;
                    if (m < d.M) gemv_store(Cb, (int64_t)m * d.sc_m + (int64_t)n * d.sc_n, d.dtype_c, gemv_epilogue(acc[mb][r], d, b, m, n));
                }
        return;
    }

    // Slots [strip][S][XR][NB]: rows < M published; the last-arriving slice sums them in order.
    const int strip = lin;
    Acc* slots = static_cast<Acc*>(g.part) + (int64_t)strip * g.nslices * XR * NB;
    const int col = 16 * wave + fr;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 16 * mb + 4 * kg + r;
            if (m < d.M && m < XR)
                slot_store(slots + ((int64_t)s * XR + m) * NB + col, acc[mb][r]);
        }
    publish_and_count(g.cnt + strip, g.nslices, &last_flag);
    if (!last_flag) return;
    if (n < d.N)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 16 * mb + 4 * kg + r;
                if (m < d.M && m < XR) {
                    Acc part_v[kGemvMaxSlices];
#pragma unroll
                    for (int k = 0; k < kGemvMaxSlices; ++k)
                        part_v[k] = k < g.nslices ? slot_load(slots + ((int64_t)k * XR + m) * NB + col) : Acc(0);
                    Acc t = part_v[0];
#pragma unroll
                    for (int k = 1; k < kGemvMaxSlices; ++k)
                        if (k < g.nslices) t += part_v[k];
                    gemv_store(Cb, (int64_t)m * d.sc_m + (int64_t)n * d.sc_n, d.dtype_c, gemv_epilogue(t, d, b, m, n));
                }
            }
    slot_count_reset(g.cnt + strip);
}

__global__ __launch_bounds__(256) void gemv_zero_kernel(int* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0;
}

// ---------------------------------------------------------------------------------------------
// Host side.
}

#include <map>
#include <mutex>
#include <tuple>

namespace tvk {

// Per-(device, stream, kind) workspace.  Calls on one stream are ordered by the stream, so they
// can share it.
struct GemvWorkspace {
    void* base = nullptr;
    size_t bytes = 0;
};
static std::mutex g_ws_mu;
static std::map<std::tuple<int, hipStream_t, int>, GemvWorkspace> g_ws;

// Test hook (tv_hip_inject_alloc_failure): while armed, each workspace request allocates, asking the
// runtime for more memory than any device has, so it fails as it would under memory pressure (a
// buffer the stream already holds is kept for later requests).
static std::atomic<int> g_alloc_fail{0};
constexpr size_t kImpossibleBytes = (size_t)1 << 60;
static bool alloc_failure_armed() {
    int n = g_alloc_fail.load();
    while (n > 0)
        if (g_alloc_fail.compare_exchange_weak(n, n - 1)) return true;
    return false;
}
void inject_alloc_failure(int count) { g_alloc_fail.store(count < 0 ? 0 : count); }

// kind 1: the GEMV's split-K arrival counters (every launch leaves them at zero); kind 2: its strip
// partial slots; kinds 3 and 4: the same for the stream-K GEMM schedule (gemm_sk_workspace); kinds
// 5 and 6: the zero-padded copies of GEMM operands A and B (gemm_pad_workspace).
static int get_workspace(hipStream_t stream, size_t need, void** out, int kind) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    GemvWorkspace& w = g_ws[{dev, stream, kind}];
    const bool fail = alloc_failure_armed(); // test hook: this request fails as an allocation would
    if (w.bytes < need || fail) {
        if (w.base && !fail) {
            // The old buffer may still be in use by queued work of this stream.
            e = hipStreamSynchronize(stream);
            if (e != hipSuccess) return e;
            (void)hipFree(w.base);
            w.base = nullptr;
            w.bytes = 0;
        }
        const size_t sz = need < ((size_t)1 << 20) ? ((size_t)1 << 20) : need;
        void* p = nullptr;
        e = hipMalloc(&p, fail ? kImpossibleBytes : sz);
        if (e != hipSuccess) {
            // The caller may carry on without the buffer (another kernel, the gather loader): the
            // failed allocation must not stay behind as the runtime's last error, which the
            // launchers report after their launch.
            (void)hipGetLastError();
            return TV_E_NOMEM;
        }
        w.base = p;
        w.bytes = sz;
        // The arrival counters must start at zero (each launch leaves them at zero again).  This
        // workspace is not meant for stream capture: growing it synchronises the stream.
        hipLaunchKernelGGL(gemv_zero_kernel, dim3(256), dim3(256), 0, stream, static_cast<int*>(w.base),
                           (int64_t)(sz / sizeof(int)));
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    *out = w.base;
    return 0;
}

// Split-K buffers of one launch: the per-stream workspace (allocated and grown on demand), or the
// caller's fixed buffers (the static scratch of tv_hip_gemm_noalloc), which must hold them.
static int split_buffers(hipStream_t stream, const GemvScratch* fixed, int64_t nwg, size_t part_bytes, GemvArgs& g) {
    if (fixed) {
        if ((size_t)nwg > fixed->cnt_ints || part_bytes > fixed->part_bytes) return TV_E_SCRATCH;
        g.cnt = fixed->cnt;
        g.part = fixed->part;
        return 0;
    }
    void* cnt = nullptr;
    int rc = get_workspace(stream, (size_t)nwg * sizeof(int), &cnt, 1);
    if (rc) return rc;
    rc = get_workspace(stream, part_bytes, &g.part, 2);
    if (rc) return rc;
    g.cnt = static_cast<int*>(cnt);
    return 0;
}

// Buffers of the stream-K GEMM schedule (workspace kinds 3 and 4; the counters start at zero and
// every launch leaves them at zero).
int gemm_sk_workspace(hipStream_t stream, size_t cnt_ints, size_t slot_bytes, int** cnt, char** slots) {
    void* c = nullptr;
    void* p = nullptr;
    int rc = get_workspace(stream, cnt_ints * sizeof(int), &c, 3);
    if (rc) return rc;
    rc = get_workspace(stream, slot_bytes, &p, 4);
    if (rc) return rc;
    *cnt = static_cast<int*>(c);
    *slots = static_cast<char*>(p);
    return 0;
}

// Buffer of the zero-padded copy of GEMM operand A (workspace kind 5) or B (kind 6).
int gemm_pad_workspace(hipStream_t stream, size_t bytes, int operand, void** out) {
    return get_workspace(stream, bytes, out, operand == 0 ? 5 : 6);
}

// Whether the vectorised GEMV serves this call.
static bool gemv_layout_ok(const GemmDesc& d) {
    if (d.dtype_a != d.dtype_b) return false;
    if (d.dtype_a != TV_FLOAT32 && d.dtype_a != TV_BFLOAT16 && d.dtype_a != TV_FLOAT16 && d.dtype_a != TV_INT8) return false;
    const int es = (int)dtype_size(d.dtype_a);
    const int64_t vec = 16 / es;
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (d.M < 1 || d.M > 32) return false; // M > 8: the matrix-core kernel only (launch_gemv)
    // N and K need not be whole chunks on zero-padded copies (pad_b / pad_a); launch_gemv keeps such
    // calls on the matrix-core kernel.
    if (d.sb_n != 1 || !al(d.B) || (d.N % vec && !d.pad_b) || (d.K > 1 && d.sb_k % vec) || (d.batch > 1 && d.sb_b % vec)) return false;
    if (d.sa_k != 1 || !al(d.A) || (d.K % vec && !d.pad_a) || (d.M > 1 && d.sa_m % vec) || (d.batch > 1 && d.sa_b % vec)) return false;
    if (d.K > 1 && d.sb_k < d.N) return false;
    return true;
}

struct GemvPlan {
    int nl, threads, nslices;
};

// Strip width: 128 bytes (8 lanes) unless N has fewer 16-byte chunks.
static int gemv_nl(const GemmDesc& d) {
    const int nch = d.N / (16 / (int)dtype_size(d.dtype_a));
    return nch >= 8 ? 8 : (nch >= 4 ? 4 : 2);
}

// K slices: enough for about 1376 workgroups in all at M <= 2, 688 at M <= 4 and 344 above
// (W[4096, 11008] bf16: 172 strips x 8, x 4 or x 2, measured best; larger M has a longer
// per-workgroup reduction), at least what x's LDS slice needs, and no more than leaves every
// k-lane two row groups per slice.
static GemvPlan gemv_plan(const GemmDesc& d) {
    const int nl = gemv_nl(d);
    const int vec = 16 / (int)dtype_size(d.dtype_a);
    const int64_t strips = (d.N / vec + nl - 1) / nl * (int64_t)d.batch;
    const int kcap = kGemvXBytes / (8 * (int)dtype_size(d.dtype_a));
    const int min_s = (d.K + kcap - 1) / kcap;
    const int rows_min = 2 * kGemvGroupRows * (kGemvThreads / nl);
    const int max_s = d.K / rows_min > 1 ? d.K / rows_min : 1;
    const int64_t target = d.M <= 2 ? 1376 : (d.M <= 4 ? 688 : 344);
    int s = (int)((target + strips - 1) / strips);
    // fp32 W: slices of about 1024 rows, 2048 from 512 strips up, unless that leaves fewer than 512
    // workgroups (a sweep of 1-16 slices over ten fp32 W shapes, K 2048-14336, N 4096-30000, M 1-8,
    // W rotated over 4 copies: e.g. x[7, 4096] @ W[4096, 10000] 58.1 us at the workgroup target
    // above, 48.0 at 4 slices; x[4, 2048] @ W[2048, 2048] 11.7 us at the target, 12.5 at 2).
    if (d.dtype_a == TV_FLOAT32) {
        const int rows = strips >= 512 ? 2048 : 1024;
        const int s_rows = (d.K + rows - 1) / rows;
        if (strips * s_rows >= 512) s = s_rows;
        else if (s < s_rows) s = s_rows;
    }
    if (s > max_s) s = max_s;
    if (s > kGemvMaxSlices) s = kGemvMaxSlices;
    if (s < min_s) s = min_s;
    return GemvPlan{nl, kGemvThreads, s < 1 ? 1 : s};
}

template <typename T, int MR, int NL, int THREADS>
static int gemv_run(const GemmDesc& d, hipStream_t stream, int nslices, const GemvScratch* fixed) {
    using Sh = GemvShape<T, MR, NL, THREADS>;
    using Acc = typename GemvTraits<T>::Acc;
    const int vec = Sh::VEC;
    if (d.K < 1) return TV_E_UNSUPPORTED; // K = 0 is served by the zero-sum kernel
    const int nblk = (d.N + Sh::NB - 1) / Sh::NB;
    int S = nslices < 1 ? 1 : nslices;
    const int min_s = (d.K + Sh::KCAP - 1) / Sh::KCAP;
    if (S < min_s) S = min_s;
    int kslice = (d.K + S - 1) / S;
    kslice = (kslice + vec - 1) / vec * vec;
    if (kslice > Sh::KCAP) kslice = Sh::KCAP; // KCAP is a multiple of every VEC
    S = (d.K + kslice - 1) / kslice;
    if (S > kGemvMaxSlices) return TV_E_UNSUPPORTED; // K beyond 16 LDS slices: the GEMM path serves it
    // Buffer offsets of one slice stay below 2^30.
    if ((int64_t)(kslice - 1) * d.sb_k * Sh::ES + (int64_t)d.N * Sh::ES >= ((int64_t)1 << 30)) return TV_E_UNSUPPORTED;
    const int64_t nwg = (int64_t)nblk * d.batch;
    if (nwg > 0x7FFFFFFF || S > 65535) return TV_E_SHAPE;

    GemvArgs g;
    g.d = d;
    g.kslice = kslice;
    g.nslices = S;
    g.nblk = nblk;
    g.cnt = nullptr;
    g.part = nullptr;
    if (S > 1) {
        const int rc = split_buffers(stream, fixed, nwg, (size_t)nwg * S * MR * Sh::NB * sizeof(Acc), g);
        if (rc) return rc;
    }
    hipLaunchKernelGGL((gemv_kernel<T, MR, NL, THREADS>), dim3((unsigned)nwg, S), dim3(THREADS),
                       (size_t)MR * kslice * Sh::ES, stream, g);
    return hipGetLastError();
}

// Dynamic LDS of the matrix-core GEMV: x's XR rows of kpad, and for XR > 8 at least the wave
// partials, which reuse that area after the loop.
template <typename T, int XR, int WAVES = kGemvMfmaWaves>
static size_t gemv_mfma_dyn_lds(int kpad) {
    const size_t x = (size_t)XR * kpad * sizeof(T);
    const size_t red = XR > 8 ? (size_t)WAVES * XR * (128 / sizeof(T)) * sizeof(typename GemvTraits<T>::Acc) : 0;
    return x > red ? x : red;
}

// K slices of the matrix-core GEMV asked for as `nslices`: at least what x's LDS slice needs, rows
// per slice a multiple of the 16-byte vector; S is what the rounding leaves.
struct GemvSlices {
    int S, kslice, kpad;
};
template <typename T, int XR, int WAVES = kGemvMfmaWaves, int DEPTH = gemv_mfma_depth<T>()>
static GemvSlices gemv_mfma_slices(const GemmDesc& d, int nslices) {
    using Acc = typename GemvTraits<T>::Acc;
    constexpr int ES = sizeof(T), VEC = 16 / ES, NB = 8 * VEC, CH = 64 / ES;
    // A workgroup's LDS (at most 160 KB) holds the kernel's static arrays and x's XR rows of a
    // slice: x rows per slice are capped by kGemvXBytes and by what the static arrays leave.
    constexpr int kLds = 160 * 1024;
    constexpr int kStatic = WAVES * CH * kGemvMfmaPitch + (XR > 8 ? 0 : WAVES * XR * NB * (int)sizeof(Acc)) + 16;
    static_assert(kStatic + XR * ES * CH <= kLds, "static LDS leaves no room for x");
    constexpr int kFit = (kLds - kStatic) / (XR * ES) / CH * CH;
    constexpr int kX = kGemvXBytes / (XR * ES) / CH * CH;
    constexpr int KCAP = kX < kFit ? kX : kFit; // a multiple of CH
    int S = nslices < 1 ? 1 : nslices;
    const int min_s = (d.K + KCAP - 1) / KCAP;
    if (S < min_s) S = min_s;
    int kslice = (d.K + S - 1) / S;
    kslice = (kslice + VEC - 1) / VEC * VEC;
    if (kslice > KCAP) kslice = KCAP;
    S = (d.K + kslice - 1) / kslice;
    return GemvSlices{S, kslice, (kslice + CH - 1) / CH * CH};
}

// The matrix-core GEMV (bf16 / fp16 with 64-column strips, int8 with 128-column strips).
template <typename T, int XR, int WAVES = kGemvMfmaWaves, int DEPTH = gemv_mfma_depth<T>()>
static int gemv_mfma_run(const GemmDesc& d, hipStream_t stream, int nslices, const GemvScratch* fixed) {
    using Acc = typename GemvTraits<T>::Acc;
    constexpr int ES = sizeof(T), VEC = 16 / ES, NB = 8 * VEC;
    if (d.K < 1) return TV_E_UNSUPPORTED;
    const int nblk = (d.N + NB - 1) / NB;
    const GemvSlices sl = gemv_mfma_slices<T, XR, WAVES, DEPTH>(d, nslices);
    const int S = sl.S, kslice = sl.kslice;
    if (S > kGemvMaxSlices) return TV_E_UNSUPPORTED;
    if ((int64_t)(kslice - 1) * d.sb_k * ES + (int64_t)d.N * ES >= ((int64_t)1 << 30)) return TV_E_UNSUPPORTED;
    const int64_t nwg = (int64_t)nblk * d.batch;
    if (nwg > 0x7FFFFFFF || S > 65535) return TV_E_SHAPE;

    GemvArgs g;
    g.d = d;
    g.kslice = kslice;
    g.nslices = S;
    g.nblk = nblk;
    g.cnt = nullptr;
    g.part = nullptr;
    if (S > 1) {
        const int rc = split_buffers(stream, fixed, nwg, (size_t)nwg * S * XR * NB * sizeof(Acc), g);
        if (rc) return rc;
    }
    const size_t lds = gemv_mfma_dyn_lds<T, XR, WAVES>(sl.kpad);
    hipLaunchKernelGGL((gemv_mfma_kernel<T, WAVES, DEPTH, XR>), dim3((unsigned)nwg, S), dim3(WAVES * 64), lds, stream, g);
    return hipGetLastError();
}

// Workgroups of the matrix-core GEMV that the current device holds at once: resident workgroups
// per CU at the launch's LDS size (the occupancy API) times the CUs.  Cached per device and LDS
// size (x's slice is the only part that varies); 0 if the runtime cannot tell.
template <typename T, int XR, int WAVES = kGemvMfmaWaves, int DEPTH = gemv_mfma_depth<T>()>
static int64_t gemv_mfma_capacity(int kpad) {
    static std::mutex mu;
    static std::map<std::pair<int, int>, int64_t> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lk(mu);
    const auto key = std::make_pair(dev, kpad);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(gemv_mfma_kernel<T, WAVES, DEPTH, XR>),
                                                     WAVES * 64, gemv_mfma_dyn_lds<T, XR, WAVES>(kpad)) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    const int64_t cap = (int64_t)(per_cu > 0 ? per_cu : 0) * (cus > 0 ? cus : 0);
    cache[key] = cap;
    return cap;
}

template <typename T, int MR>
static int gemv_dispatch_nl(const GemmDesc& d, hipStream_t stream, const GemvPlan& p, const GemvScratch* fixed) {
    if (p.threads == 256) {
        switch (p.nl) {
            case 2: return gemv_run<T, MR, 2, 256>(d, stream, p.nslices, fixed);
            case 4: return gemv_run<T, MR, 4, 256>(d, stream, p.nslices, fixed);
            case 8: return gemv_run<T, MR, 8, 256>(d, stream, p.nslices, fixed);
        }
    } else if (p.threads == 512) {
        switch (p.nl) {
            case 8: return gemv_run<T, MR, 8, 512>(d, stream, p.nslices, fixed);
        }
    }
    return TV_E_UNSUPPORTED;
}

template <typename T>
static int gemv_dispatch_mr(const GemmDesc& d, hipStream_t stream, const GemvPlan& p, const GemvScratch* fixed) {
    if (d.M <= 1) return gemv_dispatch_nl<T, 1>(d, stream, p, fixed);
    if (d.M <= 2) return gemv_dispatch_nl<T, 2>(d, stream, p, fixed);
    if (d.M <= 4) return gemv_dispatch_nl<T, 4>(d, stream, p, fixed);
    return gemv_dispatch_nl<T, 8>(d, stream, p, fixed);
}

static int launch_gemv_plan_with(const GemmDesc& d, hipStream_t stream, const GemvPlan& p, const GemvScratch* fixed) {
    switch (d.dtype_a) {
        case TV_FLOAT32: return gemv_dispatch_mr<float>(d, stream, p, fixed);
        case TV_BFLOAT16: return gemv_dispatch_mr<__bf16>(d, stream, p, fixed);
        case TV_FLOAT16: return gemv_dispatch_mr<_Float16>(d, stream, p, fixed);
        case TV_INT8: return gemv_dispatch_mr<int8_t>(d, stream, p, fixed);
        default: return TV_E_UNSUPPORTED;
    }
}

// The matrix-core kernel serves 16-bit W at every M and int8 W at M >= 3, with whole 128-byte
// strips (N >= 64 columns at 16 bits, N >= 128 at 8).  On c5's W shape, against the dot-product
// kernel: bf16 18.7 / 19.3 / 20.2 us at M = 1 / 4 / 8 (dot 19.2 / 20.9 / 25.7); int8 13.7 us at
// M = 8 (dot 20.5) but 12.1 us at M = 1 (dot 11.5).
//
// Slices: about 688 workgroups at 16 bits and 344 in int8 (4 slices of c5's W, the best of 1-16 at
// every M), unless that count lands where a sweep of 1-16 slices over nine W shapes (bf16 M = 1
// and 8, int8 M = 8; K 2048-14336, N 4096-32768) found launches slow:
//  * workgroups / resident capacity in (1.0, 1.4): a second round that is mostly empty
//    (W[4096, 14336]: 4 slices 27.9 us, 3 slices 24.5 us, 2 slices 23.7 us);
//  * fewer resident workgroups per CU than the shape allows elsewhere, up to 3 (x's LDS slice of
//    few, long slices leaves room for one: W[8192, 28672], 2 slices 119 us, 5 slices 81 us);
//  * under 0.6 of a round.
// It then takes the nearest slice count (more slices first) that avoids all three.  The resident
// capacity comes from the occupancy API at the launch's LDS size.
template <typename T, int XR>
static int gemv_mfma_pick(const GemmDesc& d) {
    constexpr int ES = sizeof(T), NB = 128 / ES, CH = 64 / ES;
    const int64_t strips = (int64_t)(d.N + NB - 1) / NB * d.batch;
    int max_s = d.K / (8 * CH) > 1 ? d.K / (8 * CH) : 1; // each wave at least two chunks per slice
    if (max_s > kGemvMaxSlices) max_s = kGemvMaxSlices;
    const int64_t target = ES == 2 ? 688 : 344;
    int s0 = (int)((target + strips - 1) / strips);
    if (s0 > max_s) s0 = max_s;
    s0 = gemv_mfma_slices<T, XR>(d, s0).S; // raised to what x's LDS slice needs

    static std::mutex mu;
    static std::map<std::tuple<int, int64_t, int>, int> picked; // (device, strips, K) -> S, per XR
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return s0;
    const auto key = std::make_tuple(dev, strips, d.K);
    {
        std::lock_guard<std::mutex> lk(mu);
        const auto it = picked.find(key);
        if (it != picked.end()) return it->second;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return s0;
    const int top = s0 > max_s ? s0 : max_s;
    int64_t cap[kGemvMaxSlices + 2] = {};
    int s_of[kGemvMaxSlices + 2] = {};
    int occ_best = 0;
    for (int s = 1; s <= top && s <= kGemvMaxSlices; ++s) {
        const GemvSlices sl = gemv_mfma_slices<T, XR>(d, s);
        s_of[s] = sl.S;
        cap[s] = gemv_mfma_capacity<T, XR>(sl.kpad);
        if (cap[s] <= 0) return s0;
        const int occ = (int)(cap[s] / cus);
        if (occ > occ_best) occ_best = occ;
    }
    const int occ_req = occ_best < 3 ? occ_best : 3;
    auto good = [&](int s) {
        if (s < 1 || s > top || s > kGemvMaxSlices || s_of[s] != s) return false;
        const double r = (double)(strips * s) / (double)cap[s];
        return cap[s] / cus >= occ_req && r >= 0.6 && !(r > 1.0 && r < 1.4);
    };
    int S = s0;
    if (!good(s0)) {
        for (int dist = 1; dist <= kGemvMaxSlices; ++dist) {
            if (good(s0 + dist)) { S = s0 + dist; break; }
            if (good(s0 - dist)) { S = s0 - dist; break; }
        }
    }
    std::lock_guard<std::mutex> lk(mu);
    picked[key] = S;
    return S;
}

template <typename T, int XR>
static int gemv_mfma_go(const GemmDesc& d, hipStream_t stream, const GemvScratch* fixed) {
    return gemv_mfma_run<T, XR>(d, stream, gemv_mfma_pick<T, XR>(d), fixed);
}
// x rows staged: 8 up to M = 8 (c5's kernel), then whole 16-row blocks: 16, and 32 at 16 bits (in
// int8 the 128-column strips' wave partials for 32 rows would take 64 KB of LDS).
static int launch_gemv_mfma(const GemmDesc& d, hipStream_t stream, const GemvScratch* fixed) {
    switch (d.dtype_a) {
        case TV_BFLOAT16:
            return d.M <= 8 ? gemv_mfma_go<__bf16, 8>(d, stream, fixed) : d.M <= 16 ? gemv_mfma_go<__bf16, 16>(d, stream, fixed)
                                                                                    : gemv_mfma_go<__bf16, 32>(d, stream, fixed);
        case TV_FLOAT16:
            return d.M <= 8 ? gemv_mfma_go<_Float16, 8>(d, stream, fixed) : d.M <= 16 ? gemv_mfma_go<_Float16, 16>(d, stream, fixed)
                                                                                      : gemv_mfma_go<_Float16, 32>(d, stream, fixed);
        default: return d.M <= 8 ? gemv_mfma_go<int8_t, 8>(d, stream, fixed) : gemv_mfma_go<int8_t, 16>(d, stream, fixed);
    }
}

// The K-contiguous-W GEMV (gemv_kt_kernel): 16-bit or int8 x and W, W rows 16-byte aligned with K
// a multiple of the 16-byte vector and no padded copy, x K-contiguous with aligned rows, 1 <= M <= 16.
static bool gemv_kt_layout_ok(const GemmDesc& d) {
    if (d.dtype_a != d.dtype_b) return false;
    // fp32 W stays on the GEMM: through this kernel (four v_mfma_f32_16x16x4f32 per 16 bytes) it
    // measured slower at large N (x[8,4096] @ W^T[4096,32000] 129.4 us against 105.3).
    if (d.dtype_a != TV_BFLOAT16 && d.dtype_a != TV_FLOAT16 && d.dtype_a != TV_INT8) return false;
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const int64_t v = 16 / (int64_t)dtype_size(d.dtype_a);
    if (d.M < 1 || d.M > 16 || d.K < v || d.K % v || d.pad_a || d.pad_b) return false;
    if (d.sb_k != 1 || !al(d.B) || (d.N > 1 && (d.sb_n % v || d.sb_n < d.K)) || (d.batch > 1 && d.sb_b % v)) return false;
    if (d.sa_k != 1 || !al(d.A) || (d.M > 1 && d.sa_m % v) || (d.batch > 1 && d.sa_b % v)) return false;
    return true;
}

// K slices of the K-contiguous-W GEMV: about 688 workgroups in all (strips of 16 x WAVES rows x
// slices), at least two 256-byte chunks per slice, x's slice within 64 KB of LDS; at most
// kGemvMaxSlices.
template <typename T, int XR, int WAVES = kGemvMfmaWaves, int DEPTH = gemv_mfma_depth<T>()>
static int gemv_kt_run(const GemmDesc& d, hipStream_t stream, const GemvScratch* fixed) {
    using Acc = typename GemvTraits<T>::Acc;
    constexpr int ES = sizeof(T), NB = 16 * WAVES, CK = gemv_kt_chunk<T>();
    constexpr int KCAP = ((kGemvXBytes / XR - 16) / ES) / CK * CK;
    const int nblk = (d.N + NB - 1) / NB;
    const int64_t strips = (int64_t)nblk * d.batch;
    int S = (int)((688 + strips - 1) / strips);
    const int max_s = d.K / (2 * CK) > 1 ? d.K / (2 * CK) : 1;
    if (S > max_s) S = max_s;
    const int min_s = (d.K + KCAP - 1) / KCAP;
    if (S < min_s) S = min_s;
    // Whole 256-byte chunks per slice: a slice then starts 256-byte aligned in every W row, so each
    // lane group's 64-byte piece is half of one 128-byte line (x[1,4096] @ W^T[4096,10000] with
    // 824-k slices: 26.8 us, the pieces straddling lines).
    int kslice = (d.K + S - 1) / S;
    kslice = (kslice + CK - 1) / CK * CK;
    if (kslice > KCAP) kslice = KCAP;
    S = (d.K + kslice - 1) / kslice;
    if (S > kGemvMaxSlices) return TV_E_UNSUPPORTED;
    if ((int64_t)15 * d.sb_n * ES + (int64_t)kslice * ES >= ((int64_t)1 << 30)) return TV_E_UNSUPPORTED;
    if (strips > 0x7FFFFFFF) return TV_E_SHAPE;

    GemvArgs g;
    g.d = d;
    g.kslice = kslice;
    g.nslices = S;
    g.nblk = nblk;
    g.cnt = nullptr;
    g.part = nullptr;
    if (S > 1) {
        // A caller's fixed split buffers too small for this split: the GEMM serves the call, as it
        // did for this layout before this kernel existed.
        const int rc = split_buffers(stream, fixed, strips, (size_t)strips * S * XR * NB * sizeof(Acc), g);
        if (rc) return rc == TV_E_SCRATCH ? TV_E_UNSUPPORTED : rc;
    }
    const int kpad = (kslice + CK - 1) / CK * CK;
    const size_t lds = (size_t)XR * (kpad * ES + 16);
    hipLaunchKernelGGL((gemv_kt_kernel<T, WAVES, DEPTH, XR>), dim3((unsigned)strips, S), dim3(WAVES * 64), lds, stream, g);
    return hipGetLastError();
}

// M <= 16 (8 or 16 rows of x staged); from 17 rows the GEMM is faster (x[32,4096] @ W^T[4096,11008]:
// 44.0 us here with 32 rows staged).
static int launch_gemv_kt(const GemmDesc& d, hipStream_t stream, const GemvScratch* fixed) {
    if (d.M > 16) return TV_E_UNSUPPORTED;
    if (d.N == 0 || d.batch == 0) return 0;
    if (d.dtype_a == TV_BFLOAT16)
        return d.M <= 8 ? gemv_kt_run<__bf16, 8>(d, stream, fixed) : gemv_kt_run<__bf16, 16>(d, stream, fixed);
    if (d.dtype_a == TV_INT8)
        return d.M <= 8 ? gemv_kt_run<int8_t, 8>(d, stream, fixed) : gemv_kt_run<int8_t, 16>(d, stream, fixed);
    return d.M <= 8 ? gemv_kt_run<_Float16, 8>(d, stream, fixed) : gemv_kt_run<_Float16, 16>(d, stream, fixed);
}

int launch_gemv(const GemmDesc& d, hipStream_t stream, const GemvScratch* fixed) {
    if (!gemv_layout_ok(d)) return gemv_kt_layout_ok(d) ? launch_gemv_kt(d, stream, fixed) : TV_E_UNSUPPORTED;
    if (d.N == 0 || d.batch == 0) return 0;
    const bool mfma = (d.dtype_a == TV_BFLOAT16 || d.dtype_a == TV_FLOAT16 || (d.dtype_a == TV_INT8 && d.M >= 3)) && gemv_nl(d) == 8;
    const int64_t vec = 16 / (int64_t)dtype_size(d.dtype_a);
    if ((d.N % vec || d.K % vec) && !mfma) return TV_E_UNSUPPORTED; // padded ragged N / K: matrix-core kernel only
    if (d.M > 8) // 9 <= M <= 32: the matrix-core kernel only (16-bit up to 32 rows, int8 up to 16)
        return mfma && (d.dtype_a != TV_INT8 || d.M <= 16) ? launch_gemv_mfma(d, stream, fixed) : TV_E_UNSUPPORTED;
    if (mfma) return launch_gemv_mfma(d, stream, fixed);
    return launch_gemv_plan_with(d, stream, gemv_plan(d), fixed);
}

// ---- Static split-K scratch of tv_hip_gemm_noalloc ---------------------------------------------
// One array per GPU, held until the process ends: the arrival counters (kScratchCounters ints,
// zero between launches) followed by the partial slots (kScratchSlotBytes).  Host code never
// passes `scratch` itself to a kernel (in host code the name is a host-side stand-in); it passes
// the device address hipGetSymbolAddress returns for the current device, kept per device.
constexpr size_t kScratchCounters = 16384;
constexpr size_t kScratchCounterBytes = kScratchCounters * sizeof(int); // 64 KiB, a multiple of 256
constexpr size_t kScratchSlotBytes = (size_t)4 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchCounterBytes + kScratchSlotBytes];

constexpr int kScratchMaxDevices = 64;
static std::mutex g_scratch_mu;
static unsigned char* g_scratch_ptr[kScratchMaxDevices]; // device address of `scratch` per device

int gemv_static_scratch(hipStream_t stream, GemvScratch* out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kScratchMaxDevices) return TV_E_UNSUPPORTED;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!ptr) return TV_E_NULL;
        // The counters must start at zero; every launch leaves them at zero again.  A fill kernel
        // (not a memset node), so a caller capturing its first call records a harmless clear.
        hipLaunchKernelGGL(gemv_zero_kernel, dim3(16), dim3(256), 0, stream, static_cast<int*>(ptr),
                           (int64_t)kScratchCounters);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        g_scratch_ptr[dev] = static_cast<unsigned char*>(ptr);
    }
    out->cnt = reinterpret_cast<int*>(g_scratch_ptr[dev]);
    out->cnt_ints = kScratchCounters;
    out->part = g_scratch_ptr[dev] + kScratchCounterBytes;
    out->part_bytes = kScratchSlotBytes;
    return 0;
}

} // namespace tvk
