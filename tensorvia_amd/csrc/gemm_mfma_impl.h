// MFMA GEMM kernels for gfx950 (CDNA4): fp32, bf16, fp16 and int8 inputs (template code; one
// translation unit per input dtype instantiates it: gemm_mfma_{f32,bf16,f16,i8}.hip).
//
// Replaces the 16x16 shared-memory tile kernel mul_cuda_3d (reference src/backend/cuda/mul.cu:8-48)
// and computes what MulImpl<CPU> computes (src/backend/cpu/mul.cpp:27-85) for these dtypes:
//   C[b,m,n] = sum_k A[b,m,k] * B[b,k,n]
// with fp32 accumulation for the float types and exact int32 accumulation for int8.
//
// Design:
//  * One workgroup computes a BM x BN output tile; its waves are laid out WAVES_M x WAVES_N and
//    each wave owns a (BM/WAVES_M) x (BN/WAVES_N) sub-tile made of 16x16 MFMA blocks.  The 16-bit
//    and int8 tiles run 8 waves (two per SIMD, 256 registers each) so one wave's LDS and HBM
//    latency hides behind the other's MFMAs.
//  * Every dtype streams 128-byte k-slices (BK = 128/sizeof(T) values of k per tile step).  A lane
//    feeds the matrix core one 16-byte fragment per operand per "k-group" (4 lane groups x 16
//    bytes = 64 bytes of k); a k-slice is 2 k-groups.
//      fp32 : 4 x v_mfma_f32_16x16x4_f32 per fragment pair
//      bf16 : 1 x v_mfma_f32_16x16x32_bf16
//      fp16 : 1 x v_mfma_f32_16x16x32_f16
//      int8 : 1 x v_mfma_i32_16x16x64_i8
//    A and B lanes use the same (lane group, element) -> k assignment, so the k order inside a
//    fragment does not affect the dot product.  The B fragment is the instruction's first operand,
//    so each lane's 4 results are 4 consecutive n of one m (vector stores).
//  * Each operand is copied into LDS in its own memory order, 16 bytes per lane, never
//    transposed in registers:
//      K-contiguous operand   -> LDS rows of 128 bytes of k (one row per m or n); fragments are
//                                ds_read_b128; 16-byte chunk c of row r sits at c ^ ((r >> 1) & 7),
//                                so the 16 rows of a fragment read cover all 64 banks once.
//      M/N-contiguous operand -> LDS rows of one k each (all m or n of the tile, padded by 16/32
//                                bytes so consecutive k rows start in different banks); fragments
//                                are gathered by the gfx950 transpose reads ds_read_b64_tr_b16 /
//                                ds_read_b64_tr_b8 (fp32: four ds_read_b32), which hand each lane
//                                the k values of one column.
//      any other strides      -> element gathers into the K-contiguous layout
//    Buffer loads return zero outside the resource's range, which zero-fills the M/N/K tails
//    without branches.
//  * Software pipeline, one barrier per k-tile (two LDS stages):
//      phase A: MFMAs on k-group 0 of tile t, interleaved with the LDS stores of tile t+1 (from
//               registers), the buffer loads of tile t+2 and the fragment reads of k-group 1;
//      barrier (LDS-only fence: the global prefetches stay in flight);
//      phase B: MFMAs on k-group 1, interleaved with the fragment reads of k-group 0 of tile t+1.
//  * Batch and broadcast: the batch offset is b*s_b, so s_b = 0 broadcasts an operand.
//  * Workgroup ids are remapped so that tiles that share A rows / B columns run on the same XCD
//    (workgroups are dealt round-robin over the 8 XCDs, each with its own L2).
#pragma once
#include "tv_kernels.h"

namespace tvk {

// ---------------------------------------------------------------------------------------------
// Matrix-core step per input dtype: c += a (x) b with a = B fragment, b = A fragment.
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
    static constexpr int kInstr = 4;
};
template <> struct Mfma<__bf16> {
    using Acc = f32x4;
    __device__ static inline void run(const u32x4& a, const u32x4& b, Acc& c) {
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
    static constexpr int kInstr = 1;
};
template <> struct Mfma<_Float16> {
    using Acc = f32x4;
    __device__ static inline void run(const u32x4& a, const u32x4& b, Acc& c) {
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
    static constexpr int kInstr = 1;
};
template <> struct Mfma<int8_t> {
    using Acc = i32x4;
    __device__ static inline void run(const u32x4& a, const u32x4& b, Acc& c) {
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a),
                                                  __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
    }
    static constexpr int kInstr = 1;
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

// K-contiguous LDS layout: row r holds 128 bytes of k; 16-byte chunk c is stored at c ^ ((r>>1)&7).
__device__ inline int kc_off(int row, int chunk) { return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4); }

// Keeps the compiler from hoisting values derived from `v` out of a loop (they are cheaper to
// recompute than to hold in registers across the MFMA loop).
__device__ inline int opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
typedef __attribute__((address_space(3))) i32x2_t lds_i32x2;
typedef __attribute__((address_space(3))) char lds_char;

// ---------------------------------------------------------------------------------------------
// One operand's global -> register -> LDS -> fragment path.  ROWS is BM (operand A, rows = m) or
// BN (operand B, rows = n); s_r / s_k are the element strides along rows and along k.
//
// Vector modes: a lane loads chunk j at  lane_off + j * (wave-uniform stride)  from the k-tile
// origin.  Tails are zero-filled by the buffer range check: the resource ends where the valid
// rows (K-contiguous) or the valid k rows (M/N-contiguous) end, and a lane whose k range
// (K-contiguous) or row range (M/N-contiguous) lies outside gets an offset >= 2^31.
template <int MODE, int ROWS, int THREADS, int ES>
struct TileLoader {
    static constexpr int VEC = 16 / ES;            // elements per 16-byte chunk
    static constexpr int BK = 128 / ES;            // k extent of one k-tile
    static constexpr int NCH = ROWS * 8 / THREADS; // 16-byte registers per thread
    static constexpr int RCH = ROWS / VEC;         // 16-byte chunks across one k row (MN layout)
    static constexpr int PITCH = ROWS * ES + (ES == 4 ? 16 : 32); // MN layout: bytes per k row
    static constexpr int BYTES = MODE == LOAD_MNCONTIG ? BK * PITCH : ROWS * 128;
    static_assert(NCH >= 1 && ROWS * 8 % THREADS == 0, "tile rows do not divide over the threads");
    static_assert(MODE != LOAD_MNCONTIG || THREADS % RCH == 0, "k rows must divide over the threads");

    const char* base;  // element (row0, k = 0) of this tile, as bytes
    int64_t s_r, s_k;  // element strides
    int rows_valid;    // rows of this tile inside the matrix
    int K;

    // K-contiguous: chunk j = tile row (t>>3) + j*THREADS/8, k = (t&7)*VEC.
    // M/N-contiguous: chunk j = k row t/RCH + j*THREADS/RCH, rows (t%RCH)*VEC ...
    __device__ inline unsigned lane_off(int t) const {
        if constexpr (MODE == LOAD_MNCONTIG) return (unsigned)(((int64_t)(t / RCH) * s_k + (t % RCH) * VEC) * ES);
        else return (unsigned)(((int64_t)(t >> 3) * s_r + (t & 7) * VEC) * ES);
    }
    __device__ inline int64_t chunk_stride(int j) const {
        if constexpr (MODE == LOAD_MNCONTIG) return (int64_t)j * (THREADS / RCH) * s_k * ES;
        else return (int64_t)j * (THREADS / 8) * s_r * ES;
    }

    __device__ inline void load(int t, int k0, u32x4 (&r)[NCH]) const {
        if constexpr (MODE == LOAD_GENERIC) {
#pragma unroll
            for (int j = 0; j < NCH; ++j) {
                const int lin = t + j * THREADS;
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
        } else {
            const int rows = rows_valid < ROWS ? rows_valid : ROWS;
            const char* kbase;
            int64_t bytes;
            unsigned lo;
            if constexpr (MODE == LOAD_MNCONTIG) {
                kbase = base + (int64_t)k0 * s_k * ES;
                bytes = (int64_t)(K - k0) * s_k * ES;                   // k rows k0..K-1
                lo = (t % RCH) * VEC < rows ? lane_off(t) : kOOB;       // whole chunk of rows valid or not
            } else {
                kbase = base + (int64_t)k0 * ES;
                bytes = (int64_t)rows * s_r * ES;                       // rows 0..rows-1
                lo = k0 + (t & 7) * VEC < K ? lane_off(t) : kOOB;
            }
            const __amdgpu_buffer_rsrc_t rs = make_rsrc(kbase, bytes);
#pragma unroll
            for (int j = 0; j < NCH; ++j) r[j] = buf_load16(rs, lo + (unsigned)chunk_stride(j));
        }
    }

    __device__ inline void store(int t, char* lds, const u32x4 (&r)[NCH]) const {
        if constexpr (MODE == LOAD_MNCONTIG) {
            char* dst = lds + (t / RCH) * PITCH + (t % RCH) * 16;
#pragma unroll
            for (int j = 0; j < NCH; ++j) *reinterpret_cast<u32x4*>(dst + j * (THREADS / RCH) * PITCH) = r[j];
        } else {
#pragma unroll
            for (int j = 0; j < NCH; ++j) {
                const int lin = t + j * THREADS;
                *reinterpret_cast<u32x4*>(lds + kc_off(lin >> 3, lin & 7)) = r[j];
            }
        }
    }

    // Fragment addressing.  Fragment f of a wave covers the 16 tile rows w0 + 16f .. w0 + 16f + 15;
    // lane (row = lane%16, group = lane/16) receives the 16 bytes of k-group kg that the matrix
    // core expects: k = kg*4*VEC + group*VEC + (0..VEC-1).
    int fbase[2]; // per k-group: lane byte offset inside a stage (fragment f adds f * frag_step)
    static constexpr int frag_step = MODE == LOAD_MNCONTIG ? 16 * ES : 16 * 128;

    __device__ inline void frag_init(int lane, int w0) {
        const int fr = lane & 15, grp = lane >> 4;
#pragma unroll
        for (int kg = 0; kg < 2; ++kg) {
            if constexpr (MODE == LOAD_MNCONTIG) {
                const int kb = kg * 4 * VEC + grp * VEC; // first k of this lane group
                if constexpr (ES == 2)      // tr16: lanes 4r+c read k row kb+r, rows w0+4c..+3
                    fbase[kg] = (kb + (fr >> 2)) * PITCH + (w0 + 4 * (fr & 3)) * 2;
                else if constexpr (ES == 1) // tr8: lanes 2r+c read k row kb+r, rows w0+8c..+7
                    fbase[kg] = (kb + (fr >> 1)) * PITCH + (w0 + 8 * (fr & 1));
                else                        // fp32: lane reads k rows kb..kb+3 at row w0+fr
                    fbase[kg] = kb * PITCH + (w0 + fr) * 4;
            } else {
                fbase[kg] = kc_off(w0 + fr, kg * 4 + grp);
            }
        }
    }

    __device__ inline u32x4 frag(const char* stage, int kg, int f) const {
        const char* p = stage + fbase[kg] + f * frag_step;
        if constexpr (MODE != LOAD_MNCONTIG) {
            return *reinterpret_cast<const u32x4*>(p);
        } else if constexpr (ES == 2) {
            const lds_char* q = (const lds_char*)p;
            const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)q);
            const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(q + 4 * PITCH));
            const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
            return u32x4{l2.x, l2.y, h2.x, h2.y};
        } else if constexpr (ES == 1) {
            const lds_char* q = (const lds_char*)p;
            const i32x2_t lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)q);
            const i32x2_t hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(q + 8 * PITCH));
            return u32x4{(unsigned)lo.x, (unsigned)lo.y, (unsigned)hi.x, (unsigned)hi.y};
        } else {
            const unsigned* u = reinterpret_cast<const unsigned*>(p);
            return u32x4{u[0], u[PITCH / 4], u[2 * PITCH / 4], u[3 * PITCH / 4]};
        }
    }

    // LDS instructions per thread: stores per tile, reads per fragment.
    static constexpr int kStores = NCH;
    static constexpr int kFragReads = MODE == LOAD_MNCONTIG ? (ES == 4 ? 4 : 2) : 1;
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
    static constexpr int A_BYTES = (TileLoader<AMODE_, BM_, WAVES_M_ * WAVES_N_ * 64, sizeof(T_)>::BYTES + 15) / 16 * 16;
    static constexpr int B_BYTES = (TileLoader<BMODE_, BN_, WAVES_M_ * WAVES_N_ * 64, sizeof(T_)>::BYTES + 15) / 16 * 16;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile must be whole 16x16 blocks");
};

// Output conversion.  int8 output keeps the low byte of the exact int32 sum (two's-complement
// wrap), the reference CPU backend's int8 result; half outputs round to nearest even.
template <typename TC, typename V> __device__ inline TC cvt_out(V v) { return static_cast<TC>(v); }

// Store the wave's accumulators as TC: acc[i][j][q] is C[row0 + 16i][col0 + 16j + q] (the lane's
// row and first column are folded into row0 / col0), four consecutive columns per vector store.
template <typename TC, class C, typename Acc>
__device__ inline void write_tile(const Acc (&acc)[C::FM][C::FN], char* Cb, int row0, int col0, bool vec_ok,
                                  const GemmDesc& d) {
    typedef TC vec_t __attribute__((__vector_size__(4 * sizeof(TC))));
#pragma unroll
    for (int i = 0; i < C::FM; ++i) {
        const int row = row0 + 16 * i;
        if (row >= d.M) continue;
        TC* crow = reinterpret_cast<TC*>(Cb) + (int64_t)row * d.sc_m;
#pragma unroll
        for (int j = 0; j < C::FN; ++j) {
            const int col = col0 + 16 * j;
            if (vec_ok && col + 4 <= d.N) {
                vec_t v;
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = cvt_out<TC>(acc[i][j][q]);
                *reinterpret_cast<vec_t*>(crow + col) = v;
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (col + q < d.N) crow[(int64_t)(col + q) * d.sc_n] = cvt_out<TC>(acc[i][j][q]);
            }
        }
    }
}

// LDS bytes each wave gets for staging its output tile.
constexpr int kEpiWaveBytes = 18432;

// Staged store: the wave writes its accumulators (as TC) into its own LDS area, rows padded by 16
// bytes (the 16 rows x 4 column groups of one write land on distinct banks), then copies them out
// in 16-byte row chunks, so every global store covers whole row segments.  Rows are processed in
// passes of RPP (all WM rows for 1- and 2-byte outputs).  Requires a contiguous row (sc_n == 1)
// with 16-byte aligned row starts at the tile's column origin.
// Rows per staging pass: the largest multiple of 16 that divides WM (a pass takes whole 16-row
// fragment blocks) and whose padded rows fit in the wave's staging bytes; 16 when none does, which
// the callers' static_asserts then reject.  (Halving WM instead would give 24 rows for WM = 48.)
template <int WM, int PITCH, int WAVE_BYTES> constexpr int staged_rows() {
    for (int r = WM - WM % 16; r > 16; r -= 16)
        if (WM % r == 0 && r * PITCH <= WAVE_BYTES) return r;
    return 16;
}

// Value transform of the staged store: identity for a plain matmul.
struct NoTransform {
    template <typename V> __device__ V operator()(V v, int, int) const { return v; }
};

template <typename TC, class C, typename Acc, int WAVE_BYTES = kEpiWaveBytes, class F = NoTransform>
__device__ inline void write_tile_staged(const Acc (&acc)[C::FM][C::FN], char* lds_wave, char* Cb, int lane, int mrow0,
                                         int ncol0, const GemmDesc& d, const F& f = F()) {
    constexpr int ROWB = C::WN * (int)sizeof(TC);            // bytes per output row of the wave tile
    constexpr int PITCH = ROWB + 16;
    constexpr int RPP = staged_rows<C::WM, PITCH, WAVE_BYTES>(); // rows per pass
    constexpr int CPR = ROWB / 16;                            // 16-byte chunks per row
    static_assert(RPP % 16 == 0 && C::WM % RPP == 0 && RPP * PITCH <= WAVE_BYTES, "staging area too small");
    typedef TC vec_t __attribute__((__vector_size__(4 * sizeof(TC))));
#pragma unroll
    for (int pass = 0; pass < C::WM / RPP; ++pass) {
        // accumulators -> LDS: acc[i][j][q] is tile row 16i + lane%16, column 16j + 4*(lane/16) + q
#pragma unroll
        for (int i = pass * (RPP / 16); i < (pass + 1) * (RPP / 16); ++i) {
            char* rowp = lds_wave + (16 * (i - pass * (RPP / 16)) + (lane & 15)) * PITCH + (lane >> 4) * 4 * sizeof(TC);
#pragma unroll
            for (int j = 0; j < C::FN; ++j) {
                vec_t v;
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = cvt_out<TC>(f(acc[i][j][q], j, q));
                *reinterpret_cast<vec_t*>(rowp + j * 16 * sizeof(TC)) = v;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        // LDS -> global, 16 bytes per lane, CPR lanes per row
#pragma unroll
        for (int idx = lane; idx < RPP * CPR; idx += 64) {
            const int r = idx / CPR, c = idx % CPR;
            const int row = mrow0 + pass * RPP + r;
            const int col = ncol0 + c * (16 / (int)sizeof(TC));
            if (row >= d.M) continue;
            const u32x4 v = *reinterpret_cast<const u32x4*>(lds_wave + r * PITCH + c * 16);
            TC* dst = reinterpret_cast<TC*>(Cb) + (int64_t)row * d.sc_m + col;
            if (col + 16 / (int)sizeof(TC) <= d.N) {
                if constexpr (ROWB % 128 == 0) store_stream16(dst, v); // whole lines per row
                else *reinterpret_cast<u32x4*>(dst) = v;
            } else {
                const TC* e = reinterpret_cast<const TC*>(&v);
#pragma unroll
                for (int q = 0; q < 16 / (int)sizeof(TC); ++q)
                    if (col + q < d.N) dst[q] = e[q];
            }
        }
        if (pass + 1 < C::WM / RPP) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        }
    }
}

// Staged store with the fused epilogue (float accumulators): the wave stages its fp32 accumulators
// in its LDS area (rows padded by 16 bytes), then each lane takes 4 consecutive columns of a row,
// adds their bias values, applies the activation and stores them rounded once to TC.  The
// accumulators are dead before the bias is read, so the epilogue adds no register pressure to the
// k-loop.  Requires row-contiguous C (sc_n == 1); vec_ok: rows aligned for 4-element stores.
template <typename TC, class C, int WAVE_BYTES = kEpiWaveBytes>
__device__ inline void write_tile_staged_epi(const f32x4 (&acc)[C::FM][C::FN], char* lds_wave, char* Cb, int lane,
                                             int mrow0, int ncol0, const GemmDesc& d, int b, bool vec_ok) {
    constexpr int ROWB = C::WN * 4;
    constexpr int PITCH = ROWB + 16;
    constexpr int RPP = staged_rows<C::WM, PITCH, WAVE_BYTES>();
    constexpr int CPR = ROWB / 16; // 4-column float chunks per row
    static_assert(RPP % 16 == 0 && C::WM % RPP == 0 && RPP * PITCH <= WAVE_BYTES, "staging area too small");
    typedef TC out4 __attribute__((__vector_size__(4 * sizeof(TC))));
    const bool has_bias = d.bias != nullptr;
    const __amdgpu_buffer_rsrc_t br = make_rsrc(static_cast<const char*>(d.bias), has_bias ? d.bias_bytes : 0);
    const int64_t base = (int64_t)b * d.sbias_b;
    const bool logistic = d.act == TV_ACT_SILU || d.act == TV_ACT_SIGMOID || d.act == TV_ACT_TANH;
    const ActCoef k = act_coef(d.act);
    auto bias_elem = [&](int row, int col) {
        const unsigned bi = row < d.M && col < d.N ? (unsigned)(base + (int64_t)row * d.sbias_m + (int64_t)col * d.sbias_n)
                                                   : kOOB;
        return d.dtype_c == TV_FLOAT32 ? bias_load32(br, bi) : bias_load16(br, bi, d.dtype_c == TV_BFLOAT16);
    };
    // A bias with no row stride (one value per column, as a per-channel bias): every chunk a lane
    // writes has the same 4 columns (64 lanes cover whole rows of chunks), so the lane loads its 4
    // values once instead of once per row.
    static_assert(64 % CPR == 0, "a lane's chunk column is the same in every pass");
    const bool col_bias = has_bias && d.sbias_m == 0;
    float cbias[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (col_bias)
#pragma unroll
        for (int q = 0; q < 4; ++q) cbias[q] = bias_elem(0, ncol0 + (lane % CPR) * 4 + q);
#pragma unroll
    for (int pass = 0; pass < C::WM / RPP; ++pass) {
#pragma unroll
        for (int i = pass * (RPP / 16); i < (pass + 1) * (RPP / 16); ++i) {
            char* rowp = lds_wave + (16 * (i - pass * (RPP / 16)) + (lane & 15)) * PITCH + (lane >> 4) * 16;
#pragma unroll
            for (int j = 0; j < C::FN; ++j) *reinterpret_cast<f32x4*>(rowp + j * 64) = acc[i][j];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
        for (int idx = lane; idx < RPP * CPR; idx += 64) {
            const int r = idx / CPR, c = idx % CPR;
            const int row = mrow0 + pass * RPP + r;
            const int col = ncol0 + c * 4;
            f32x4 v = *reinterpret_cast<const f32x4*>(lds_wave + r * PITCH + c * 16);
            if (col_bias) {
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] += cbias[q];
            } else if (has_bias) {
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] += bias_elem(row, col + q);
            }
            // One uniform branch per chunk, not one per value.
            if (logistic) {
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = act_logistic(v[q], k);
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = act_simple(v[q], d.act);
            }
            if (row >= d.M) continue;
            TC* dst = reinterpret_cast<TC*>(Cb) + (int64_t)row * d.sc_m + col;
            if (vec_ok && col + 4 <= d.N) {
                out4 o;
#pragma unroll
                for (int q = 0; q < 4; ++q) o[q] = cvt_out<TC>(v[q]);
                if constexpr (C::WN * sizeof(TC) % 128 != 0) *reinterpret_cast<out4*>(dst) = o; // part lines
                else if constexpr (sizeof(out4) == 16) store_stream16(dst, __builtin_bit_cast(u32x4, o));
                else store_stream8(dst, __builtin_bit_cast(uint2, o));
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (col + q < d.N) dst[q] = cvt_out<TC>(v[q]);
            }
        }
        if (pass + 1 < C::WM / RPP) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        }
    }
}

// Fused epilogue applied while the accumulators are staged (write_tile_staged's transform), for a
// bias without a row stride or no bias: acc[i][j][q] is tile row 16i + lane%16, column
// 16j + 4*(lane/16) + q, so the lane's FN x 4 bias values serve every row it holds.  16-bit outputs
// then stage half the LDS bytes of the fp32 staging in write_tile_staged_epi, in half the passes.
// LOGISTIC selects the activation family at compile time, so no value carries a branch.
template <int FN, bool LOGISTIC>
struct ColBiasAct {
    float cb[FN][4];
    ActCoef k;
    int act;
    __device__ ColBiasAct(const GemmDesc& d, int b, int ncol0, int lane) : k(act_coef(d.act)), act(d.act) {
        if (d.bias != nullptr) {
            const __amdgpu_buffer_rsrc_t br = make_rsrc(static_cast<const char*>(d.bias), d.bias_bytes);
            const int64_t base = (int64_t)b * d.sbias_b;
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int col = ncol0 + 16 * j + 4 * (lane >> 4) + q;
                    const unsigned bi = col < d.N ? (unsigned)(base + (int64_t)col * d.sbias_n) : kOOB;
                    cb[j][q] = d.dtype_c == TV_FLOAT32 ? bias_load32(br, bi) : bias_load16(br, bi, d.dtype_c == TV_BFLOAT16);
                }
        } else {
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) cb[j][q] = 0.0f;
        }
    }
    __device__ float operator()(float v, int j, int q) const {
        v += cb[j][q];
        return LOGISTIC ? act_logistic(v, k) : act_simple(v, act);
    }
};

// Scheduling hints for the interleaved phases (LLVM AMDGPU sched_group_barrier masks).
constexpr int SG_MFMA = 0x008, SG_VMEM_READ = 0x020, SG_DS_READ = 0x100, SG_DS_WRITE = 0x200, SG_VALU = 0x002;

// Workgroup barrier that orders LDS only (global prefetches stay in flight).  The scheduling
// fences keep each phase's MFMAs on their side of the barrier.
__device__ inline void lds_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    __builtin_amdgcn_sched_barrier(0);
}

// The k-loop of one output tile over k-tiles [kt0, kt1), accumulating into acc (the caller zeroes
// it).  b, m0, n0: the tile's batch and origin.
template <class C>
__device__ inline void mfma_tile_kloop(const GemmDesc& d, char* smem, int b, int m0, int n0, int kt0, int kt1,
                                       typename Mfma<typename C::T>::Acc (&acc)[C::FM][C::FN]) {
    using T = typename C::T;
    using Op = Mfma<T>;
    constexpr int ES = C::ES;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;

    TileLoader<C::AMODE, C::BM, C::THREADS, ES> la;
    la.base = static_cast<const char*>(d.A) + ((int64_t)b * d.sa_b + (int64_t)m0 * d.sa_m) * ES;
    la.s_r = d.sa_m; la.s_k = d.sa_k; la.rows_valid = d.M - m0; la.K = d.K;
    TileLoader<C::BMODE, C::BN, C::THREADS, ES> lb;
    lb.base = static_cast<const char*>(d.B) + ((int64_t)b * d.sb_b + (int64_t)n0 * d.sb_n) * ES;
    lb.s_r = d.sb_n; lb.s_k = d.sb_k; lb.rows_valid = d.N - n0; lb.K = d.K;

    u32x4 ra[decltype(la)::NCH];
    u32x4 rb[decltype(lb)::NCH];
    // B fragments of a k-group are held for the whole group; A fragments stream one 16-row block at
    // a time, one block ahead of the MFMAs that use them.
    u32x4 fb[C::FN];
    u32x4 fa;

    la.frag_init(lane, wm * C::WM);
    lb.frag_init(lane, wn * C::WN);
    auto a_frag = [&](const char* stage, int kg, int i) { return la.frag(stage, kg, i); };
    auto b_frag = [&](const char* stage, int kg, int j) { return lb.frag(stage + C::A_BYTES, kg, j); };
    // MFMAs of one k-group (B fragments in fb, first A fragment already in `fa`).  While A block i
    // is multiplied, A block i+1 is read; in the last block each B fragment is refilled with the
    // following group's right after its last use, and the first A block of that group is read.
    auto kgroup = [&](const char* stage, int kg, const char* nstage, int nkg) {
#pragma unroll
        for (int i = 0; i < C::FM; ++i) {
            const u32x4 a_cur = fa;
            fa = (i + 1 < C::FM) ? a_frag(stage, kg, i + 1) : a_frag(nstage, nkg, 0);
#pragma unroll
            for (int j = 0; j < C::FN; ++j) {
                Op::run(fb[j], a_cur, acc[i][j]);
                if (i + 1 == C::FM) fb[j] = b_frag(nstage, nkg, j);
            }
        }
    };

    // Prologue: k-tile kt0 -> LDS stage 0, kt0 + 1 -> registers, k-group 0 fragments of kt0.
    la.load(tid, kt0 * C::BK, ra);
    lb.load(tid, kt0 * C::BK, rb);
    la.store(tid, smem, ra);
    lb.store(tid, smem + C::A_BYTES, rb);
    la.load(tid, (kt0 + 1) * C::BK, ra);
    lb.load(tid, (kt0 + 1) * C::BK, rb);
    lds_barrier();
#pragma unroll
    for (int j = 0; j < C::FN; ++j) fb[j] = b_frag(smem, 0, j);
    fa = a_frag(smem, 0, 0);

    constexpr int NMF = C::FM * C::FN * Op::kInstr;                  // MFMAs per k-group
    constexpr int NST = decltype(la)::kStores + decltype(lb)::kStores; // LDS stores per tile
    constexpr int NRD = C::FM * decltype(la)::kFragReads + C::FN * decltype(lb)::kFragReads; // LDS reads per k-group
    constexpr int NLD = decltype(la)::NCH + decltype(lb)::NCH;        // buffer loads per tile

    // k-tiles past kt1 are loaded ahead (zeros past K) but never multiplied.
    for (int kt = kt0; kt < kt1; ++kt) {
        char* cur = smem + ((kt - kt0) & 1) * C::STAGE;
        char* nxt = smem + ((kt - kt0 + 1) & 1) * C::STAGE;
        // Phase A: tile kt+1 -> LDS, tile kt+2 -> registers, MFMAs of k-group 0 of tile kt
        // (reading k-group 1's fragments of tile kt on the way).
        const int t = opaque(tid);
        la.store(t, nxt, ra);
        lb.store(t, nxt + C::A_BYTES, rb);
        la.load(t, (kt + 2) * C::BK, ra);
        lb.load(t, (kt + 2) * C::BK, rb);
        kgroup(cur, 0, cur, 1);
        if constexpr (NMF >= NRD + NLD + 1) {
            constexpr int slots = NMF - NRD - NLD;            // MFMAs left for the LDS stores
            constexpr int wper = (NST + slots - 1) / slots;   // stores per MFMA
            constexpr int wgroups = (NST + wper - 1) / wper;
#pragma unroll
            for (int i = 0; i < wgroups; ++i) {
                __builtin_amdgcn_sched_group_barrier(SG_DS_WRITE, wper, 0);
                __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
            }
#pragma unroll
            for (int i = 0; i < NLD; ++i) {
                __builtin_amdgcn_sched_group_barrier(SG_VMEM_READ, 1, 0);
                __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
            }
#pragma unroll
            for (int i = 0; i < NRD; ++i) {
                __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
                __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
            }
            if constexpr (NMF - wgroups - NRD - NLD > 0)
                __builtin_amdgcn_sched_group_barrier(SG_MFMA, NMF - wgroups - NRD - NLD, 0);
        }
        lds_barrier();
        // Phase B: MFMAs of k-group 1 of tile kt, reading k-group 0's fragments of tile kt+1.
        kgroup(cur, 1, nxt, 0);
        if constexpr (NMF >= NRD) {
#pragma unroll
            for (int i = 0; i < NRD; ++i) {
                __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
                __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(SG_MFMA, NMF - NRD, 0);
        }
    }
}

// Epilogue of one output tile: acc[i][j][q] = C[m0 + wm*WM + 16i + lane%16][n0 + wn*WN + 16j +
// 4*(lane/16) + q].  The output type is chosen once; each branch is straight-line code over the
// accumulators.
template <class C, bool FUSED>
__device__ inline void mfma_tile_store(const GemmDesc& d, char* smem, int b, int m0, int n0, int c_vec,
                                       const typename Mfma<typename C::T>::Acc (&acc)[C::FM][C::FN]) {
    using Acc = typename Mfma<typename C::T>::Acc;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
    const size_t csz = dtype_size(d.dtype_c);
    char* Cb = static_cast<char*>(d.C) + (int64_t)b * d.sc_b * csz;
    const int row0 = m0 + wm * C::WM + (lane & 15);
    const int col0 = n0 + wn * C::WN + (lane >> 4) * 4;
    const bool vec_ok = c_vec != 0;
    if constexpr (FUSED && !__is_same(Acc, i32x4)) {
        // Fused epilogue: fp32 staging, bias and activation after the accumulators are dead.
        lds_barrier();
        char* lw = smem + wave * kEpiWaveBytes;
        const int mrow0 = m0 + wm * C::WM, ncol0 = n0 + wn * C::WN;
        if (d.dtype_c == TV_BFLOAT16) write_tile_staged_epi<__bf16, C>(acc, lw, Cb, lane, mrow0, ncol0, d, b, vec_ok);
        else if (d.dtype_c == TV_FLOAT16) write_tile_staged_epi<_Float16, C>(acc, lw, Cb, lane, mrow0, ncol0, d, b, vec_ok);
        else write_tile_staged_epi<float, C>(acc, lw, Cb, lane, mrow0, ncol0, d, b, vec_ok);
        return;
    }
    if (c_vec == 2) {
        // All waves are done with the k-loop's LDS stages before any wave reuses them.
        lds_barrier();
        char* lw = smem + wave * kEpiWaveBytes;
        const int mrow0 = m0 + wm * C::WM, ncol0 = n0 + wn * C::WN;
        if constexpr (__is_same(Acc, i32x4)) {
            if (d.dtype_c == TV_INT8) write_tile_staged<int8_t, C>(acc, lw, Cb, lane, mrow0, ncol0, d);
            else write_tile_staged<int32_t, C>(acc, lw, Cb, lane, mrow0, ncol0, d);
        } else {
            if (d.dtype_c == TV_BFLOAT16) write_tile_staged<__bf16, C>(acc, lw, Cb, lane, mrow0, ncol0, d);
            else if (d.dtype_c == TV_FLOAT16) write_tile_staged<_Float16, C>(acc, lw, Cb, lane, mrow0, ncol0, d);
            else write_tile_staged<float, C>(acc, lw, Cb, lane, mrow0, ncol0, d);
        }
        return;
    }
    if constexpr (__is_same(Acc, i32x4)) {
        if (d.dtype_c == TV_INT8) write_tile<int8_t, C>(acc, Cb, row0, col0, vec_ok, d);
        else write_tile<int32_t, C>(acc, Cb, row0, col0, vec_ok, d);
    } else {
        if (d.dtype_c == TV_BFLOAT16) write_tile<__bf16, C>(acc, Cb, row0, col0, vec_ok, d);
        else if (d.dtype_c == TV_FLOAT16) write_tile<_Float16, C>(acc, Cb, row0, col0, vec_ok, d);
        else write_tile<float, C>(acc, Cb, row0, col0, vec_ok, d);
    }
}

// Workgroup id -> (batch, tile row, tile column).  The hardware deals workgroup ids round-robin over
// the 8 XCDs; the id is first remapped so that a contiguous range of logical tiles lands on one XCD,
// then tiles are walked in groups of `group_m` tile-rows so that neighbouring workgroups share A rows
// and B columns in that XCD's L2.
__device__ inline void mfma_tile_of(int lin, int tiles_m, int tiles_n, int group_m, int& b, int& tm, int& tn) {
    const int per_batch = tiles_m * tiles_n;
    b = lin / per_batch;
    int r = lin - b * per_batch;
    const int span = group_m * tiles_n;
    const int g = r / span;
    const int first_m = g * group_m;
    const int gsz = min(tiles_m - first_m, group_m);
    r -= g * span;
    tm = first_m + r % gsz;
    tn = r / gsz;
}

// Waves per SIMD the kernels are compiled for: two, as the 8-wave tiles run.  For the 4-wave tiles
// this is a register bound (at most 256 per wave) rather than an occupancy need: bound to one wave
// per SIMD, the fp32 k-loop kept its accumulators in AGPRs and spent 28-32 v_accvgpr moves per
// k-tile (324 instructions against 293); with the bound, 512 fp32 tiles ran 273 us against 311.
template <class C> constexpr int mfma_waves_per_eu() { return C::THREADS == 256 ? 2 : C::THREADS / 256; }

template <class C, bool FUSED = false>
__global__ __attribute__((amdgpu_flat_work_group_size(C::THREADS, C::THREADS),
                          amdgpu_waves_per_eu(mfma_waves_per_eu<C>(), mfma_waves_per_eu<C>())))
void gemm_mfma_kernel(GemmDesc d, int tiles_m, int tiles_n, int group_m, int c_vec) {
    using Acc = typename Mfma<typename C::T>::Acc;
    constexpr int SMEM = 2 * C::STAGE > kEpiWaveBytes * C::THREADS / 64 ? 2 * C::STAGE : kEpiWaveBytes * C::THREADS / 64;
    __shared__ __attribute__((aligned(16))) char smem[SMEM];

    int bid = blockIdx.x;
    const int nwg = gridDim.x;
    if ((nwg & 7) == 0) bid = (bid & 7) * (nwg >> 3) + (bid >> 3);
    int b, tm, tn;
    mfma_tile_of(bid, tiles_m, tiles_n, group_m, b, tm, tn);
    const int m0 = tm * C::BM, n0 = tn * C::BN;

    Acc acc[C::FM][C::FN];
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j) acc[i][j] = Acc{0, 0, 0, 0};
    mfma_tile_kloop<C>(d, smem, b, m0, n0, 0, (d.K + C::BK - 1) / C::BK, acc);
    mfma_tile_store<C, FUSED>(d, smem, b, m0, n0, c_vec, acc);
}

// ---------------------------------------------------------------------------------------------
// Stream-K schedule (fp32): G resident workgroups share the work instead of one workgroup per
// tile.  Every CU then does the same work however the tiles divide over the CUs (c1: 864 tiles of
// 96x128 on 256 CUs, 3.375 per CU, which the one-per-tile launch runs in the time of 4), and fewer
// tiles than CUs still use every CU.  Whole rounds of G tiles run whole (workgroup w takes tiles
// w, w + G, ...), so the workgroups running side by side take neighbouring tiles at the same k and
// share their operands in L2; the last, partial round is split: the first `wgs` workgroups take
// equal contiguous ranges of its (tile, k-tile) iteration space, workgroup w iterations
// [w*I/wgs, (w+1)*I/wgs), and a tile cut by a range boundary is computed in segments by
// consecutive workgroups.  Each segment stores its accumulators in a slot (register order, 16 bytes a lane),
// counts itself in (publish_and_count), and the last segment to arrive sums the slots in segment
// order (deterministic) and writes the tile.  Workgroup w's slots: 2w for the segment that continues
// a tile begun before its range, 2w + 1 for the one that begins a tile that runs past it (a range
// holds at most one of each).  No workgroup waits for another.
struct SkArgs {
    int64_t iters; // split tiles x k-tiles
    int nk;        // k-tiles per tile
    int dp_tiles;  // tiles [0, dp_tiles) run whole, workgroup w taking w, w + G, ...; the rest split
    int wgs;       // workgroups sharing the split tiles' iterations (the first wgs, at most G)
    int* cnt;      // [tiles] arrival counters, zero between launches
    char* slots;   // [2 x workgroups][slot bytes]
};

template <class C> constexpr int sk_slot_bytes() { return C::THREADS / 64 * C::FM * C::FN * 64 * 16; }

template <class C, bool FUSED = false>
__global__ __attribute__((amdgpu_flat_work_group_size(C::THREADS, C::THREADS),
                          amdgpu_waves_per_eu(mfma_waves_per_eu<C>(), mfma_waves_per_eu<C>())))
void gemm_mfma_sk_kernel(GemmDesc d, int tiles_m, int tiles_n, int group_m, int c_vec, SkArgs sk) {
    using Acc = typename Mfma<typename C::T>::Acc;
    static_assert(__is_same(Acc, f32x4), "stream-K slots hold fp32 accumulators");
    constexpr int SMEM = 2 * C::STAGE > kEpiWaveBytes * C::THREADS / 64 ? 2 * C::STAGE : kEpiWaveBytes * C::THREADS / 64;
    constexpr int SLOT = sk_slot_bytes<C>();
    __shared__ __attribute__((aligned(16))) char smem[SMEM];
    __shared__ int last_flag;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int w = blockIdx.x;
    if ((gridDim.x & 7) == 0) w = (w & 7) * (gridDim.x >> 3) + (w >> 3); // consecutive ids on one XCD
    const int nk = sk.nk;

    // Whole tiles first, in the grouped tile order: the workgroups side by side on an XCD take
    // neighbouring tiles and start them together, so they share A and B k-slices in its L2.
    for (int tile = w; tile < sk.dp_tiles; tile += (int)gridDim.x) {
        int b, tm, tn;
        mfma_tile_of(tile, tiles_m, tiles_n, group_m, b, tm, tn);
        const int m0 = tm * C::BM, n0 = tn * C::BN;
        Acc acc[C::FM][C::FN];
#pragma unroll
        for (int i = 0; i < C::FM; ++i)
#pragma unroll
            for (int j = 0; j < C::FN; ++j) acc[i][j] = Acc{0, 0, 0, 0};
        lds_barrier(); // the previous tile's epilogue is done with the LDS
        mfma_tile_kloop<C>(d, smem, b, m0, n0, 0, nk, acc);
        mfma_tile_store<C, FUSED>(d, smem, b, m0, n0, c_vec, acc);
    }

    // Then the split tiles [dp_tiles, tiles): the first sk.wgs workgroups take equal ranges of their
    // iterations.
    const int G = sk.wgs;
    if (w >= G) return;
    const int64_t I = sk.iters;
    const int64_t it_end = (int64_t)(w + 1) * I / G;
    // The workgroup whose range holds iteration it: the largest v with floor(v * I / G) <= it.
    auto owner = [&](int64_t it) { return (int)(((it + 1) * G - 1) / I); };
    auto slot_rsrc = [&](int slot) { return make_rsrc(sk.slots + (int64_t)slot * SLOT, SLOT); };

    for (int64_t it = (int64_t)w * I / G; it < it_end;) {
        const int rel = (int)(it / nk); // split tile index; its k-tiles are iterations rel*nk ..
        const int tile = sk.dp_tiles + rel;
        const int kt0 = (int)(it - (int64_t)rel * nk);
        const int kt1 = (int)min((int64_t)nk, kt0 + (it_end - it));
        it += kt1 - kt0;
        int b, tm, tn;
        mfma_tile_of(tile, tiles_m, tiles_n, group_m, b, tm, tn);
        const int m0 = tm * C::BM, n0 = tn * C::BN;
        Acc acc[C::FM][C::FN];
#pragma unroll
        for (int i = 0; i < C::FM; ++i)
#pragma unroll
            for (int j = 0; j < C::FN; ++j) acc[i][j] = Acc{0, 0, 0, 0};
        lds_barrier(); // the previous segment's epilogue is done with the LDS
        mfma_tile_kloop<C>(d, smem, b, m0, n0, kt0, kt1, acc);
        if (kt0 != 0 || kt1 != nk) {
            const int64_t t0 = (int64_t)rel * nk;
            const int first = owner(t0), last = owner(t0 + nk - 1);
            {
                const __amdgpu_buffer_rsrc_t r = slot_rsrc(w == first ? 2 * w + 1 : 2 * w);
#pragma unroll
                for (int i = 0; i < C::FM; ++i)
#pragma unroll
                    for (int j = 0; j < C::FN; ++j)
                        slot_store16(r, (((wave * C::FM + i) * C::FN + j) * 64 + lane) * 16, acc[i][j]);
            }
            publish_and_count(sk.cnt + tile, last - first + 1, &last_flag);
            if (!last_flag) continue;
            // Sum the segments' slots in segment order (this workgroup's own included).
            for (int v = first; v <= last; ++v) {
                const __amdgpu_buffer_rsrc_t r = slot_rsrc(v == first ? 2 * v + 1 : 2 * v);
#pragma unroll
                for (int i = 0; i < C::FM; ++i)
#pragma unroll
                    for (int j = 0; j < C::FN; ++j) {
                        const f32x4 p = slot_load16<f32x4>(r, (((wave * C::FM + i) * C::FN + j) * 64 + lane) * 16);
                        acc[i][j] = v == first ? p : acc[i][j] + p;
                    }
            }
            slot_count_reset(sk.cnt + tile);
        }
        mfma_tile_store<C, FUSED>(d, smem, b, m0, n0, c_vec, acc);
    }
}

// ---------------------------------------------------------------------------------------------
// Host side: pick the operand load modes and the tile configuration.
// Workgroups of the stream-K kernel resident at once on the current device (occupancy API x CUs),
// cached per device; 0 if the runtime cannot tell.
template <class C>
static int sk_grid() {
    static std::atomic<int> cached[kMaxDevices];
    return cached_per_device(cached, [](int dev) {
        int per_cu = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(gemm_mfma_sk_kernel<C, false>),
                                                         C::THREADS, 0) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu <= 0 || cus <= 0)
            return 0;
        return per_cu * cus;
    });
}

// The stream-K launch: K of at least 32 k-tiles (8 when the tiles do not fill the CUs), at least 8
// k-tiles per workgroup, and a last round that the resident workgroups do not fill.  Measured
// against one workgroup per tile with random fp32 inputs (same box, settled clocks): c1
// [2592,2048]@[2048,4096] 349 against 380 us; 768 tiles 411 against 432 us; [1024]^3 (64 tiles)
// 37.9 against 68.0 us; but 363 tiles at K = 512 (16 k-tiles) 78.7 against 75.0 us, the combines
// outweighing the balance.  Tile counts of whole rounds run one workgroup per tile, which measured
// faster than this kernel's persistent loop over them and needs no slots: [4096]^3 on 256x256
// tiles 948.3 against 972.6 us, [8192]^3 7,534 against 7,649, [8][1024,1024]@[1024,1024] (512
// tiles of 128x128) 130.1 against 132.6, [16][128,4096]@[4096,8192] (1,024 tiles) 995.6 against
// 998.8.  Returns 1 if it did not launch.
template <class C, bool FUSED>
static int run_cfg_sk(const GemmDesc& d, hipStream_t stream, int group_m, int tiles_m, int tiles_n, int64_t ntiles, int c_vec) {
    const int nk = (d.K + C::BK - 1) / C::BK;
    if (nk < 8) return 1;
    int G = sk_grid<C>();
    if (G <= 0) return 1;
    if (nk < 32 && ntiles >= G / 2) return 1; // G / 2: about one tile per CU
    if (ntiles % G == 0) return 1;            // whole rounds: nothing to split
    // Whole rounds of G tiles run whole; only the last, partial round is split.
    const int64_t dp = ntiles > G ? ntiles / G * G : 0;
    const int64_t iters = (ntiles - dp) * nk;
    int wgs = (int)(iters / 8 < G ? iters / 8 : G);
    // At most 32 segments per split tile: a tile's last-arriving workgroup sums its slots alone.
    if (32 * (ntiles - dp) < wgs) wgs = (int)(32 * (ntiles - dp));
    if (dp == 0) G = wgs;
    if (G < 1) return 1;
    SkArgs sk;
    sk.iters = iters;
    sk.nk = nk;
    sk.dp_tiles = (int)dp;
    sk.wgs = wgs;
    const int rc = gemm_sk_workspace(stream, (size_t)ntiles, (size_t)2 * G * sk_slot_bytes<C>(), &sk.cnt, &sk.slots);
    if (rc == TV_E_NOMEM) return 1; // no room for the slots: one workgroup per tile serves the call
    if (rc) return rc;
    hipLaunchKernelGGL((gemm_mfma_sk_kernel<C, FUSED>), dim3((unsigned)G), dim3(C::THREADS), 0, stream, d, tiles_m, tiles_n,
                       group_m, c_vec, sk);
    return hipGetLastError();
}

template <class C>
static int run_cfg(const GemmDesc& d, hipStream_t stream, int group_m, bool may_alloc = true) {
    const int tiles_m = (d.M + C::BM - 1) / C::BM;
    const int tiles_n = (d.N + C::BN - 1) / C::BN;
    const int64_t nwg = (int64_t)tiles_m * tiles_n * d.batch;
    if (nwg <= 0) return 0;
    if (nwg > 0x7FFFFFFF) return TV_E_SHAPE;
    const size_t csz = dtype_size(d.dtype_c);
    // c_vec = 1: 4-element vector stores along rows of C (aligned to 4 elements);
    // c_vec = 2: LDS-staged 16-byte row chunks (rows 16-byte aligned at every tile origin).
    int c_vec = d.sc_n == 1 && d.sc_m % 4 == 0 && (d.batch <= 1 || d.sc_b % 4 == 0) &&
                (reinterpret_cast<uintptr_t>(d.C) % (4 * csz)) == 0;
    const int64_t v16 = 16 / (int64_t)csz;
    if (c_vec && d.sc_m % v16 == 0 && (d.batch <= 1 || d.sc_b % v16 == 0) &&
        (reinterpret_cast<uintptr_t>(d.C) % 16) == 0 && (C::WN * (int64_t)csz) % 16 == 0)
        c_vec = 2;
    // The fused epilogue runs in the staged store only (16-byte aligned rows of C).
    const bool epi = d.bias != nullptr || d.act != TV_ACT_NONE;
    if (epi && d.sc_n != 1) return TV_E_UNSUPPORTED; // the fused store writes rows of C
    if constexpr (__is_same(typename C::T, float))
        if (may_alloc) {
            const int rc = epi ? run_cfg_sk<C, true>(d, stream, group_m, tiles_m, tiles_n, nwg, c_vec)
                               : run_cfg_sk<C, false>(d, stream, group_m, tiles_m, tiles_n, nwg, c_vec);
            if (rc != 1) return rc;
        }
    if constexpr (!__is_same(typename C::T, int8_t))
        if (epi) {
            hipLaunchKernelGGL((gemm_mfma_kernel<C, true>), dim3((unsigned)nwg), dim3(C::THREADS), 0, stream, d, tiles_m, tiles_n,
                               group_m, c_vec);
            return hipGetLastError();
        }
    hipLaunchKernelGGL(gemm_mfma_kernel<C>, dim3((unsigned)nwg), dim3(C::THREADS), 0, stream, d, tiles_m, tiles_n,
                       group_m, c_vec);
    return hipGetLastError();
}

// Tile shapes: the large tile serves the vector load modes; any operand that needs element
// gathers runs a 128x128 tile (fewer registers, faster to build, rarely used).
template <typename T, int BM, int BN, int WMW, int WNW>
static int run_modes(const GemmDesc& d, hipStream_t stream, int group_m, bool may_alloc = true) {
    const int es = (int)sizeof(T);
    const int am = pick_mode(d.A, d.M, d.K, d.sa_m, d.sa_k, d.sa_b, d.batch, es, BM, d.pad_a);
    const int bm = pick_mode(d.B, d.N, d.K, d.sb_n, d.sb_k, d.sb_b, d.batch, es, BN, d.pad_b);
#define TV_CASE(A_, B_) \
    if (am == A_ && bm == B_) return run_cfg<GemmCfg<T, BM, BN, WMW, WNW, A_, B_>>(d, stream, group_m, may_alloc);
    TV_CASE(LOAD_KCONTIG, LOAD_MNCONTIG)
    TV_CASE(LOAD_KCONTIG, LOAD_KCONTIG)
    TV_CASE(LOAD_MNCONTIG, LOAD_MNCONTIG)
    TV_CASE(LOAD_MNCONTIG, LOAD_KCONTIG)
#undef TV_CASE
    // Gather paths: re-pick the modes for the small tile's row count.
    const int am2 = pick_mode(d.A, d.M, d.K, d.sa_m, d.sa_k, d.sa_b, d.batch, es, 128, d.pad_a);
    const int bm2 = pick_mode(d.B, d.N, d.K, d.sb_n, d.sb_k, d.sb_b, d.batch, es, 128, d.pad_b);
#define TV_CASE(A_, B_) \
    if (am2 == A_ && bm2 == B_) return run_cfg<GemmCfg<T, 128, 128, 2, 2, A_, B_>>(d, stream, group_m, may_alloc);
    TV_CASE(LOAD_KCONTIG, LOAD_GENERIC)
    TV_CASE(LOAD_MNCONTIG, LOAD_GENERIC)
    TV_CASE(LOAD_GENERIC, LOAD_MNCONTIG)
    TV_CASE(LOAD_GENERIC, LOAD_KCONTIG)
    TV_CASE(LOAD_GENERIC, LOAD_GENERIC)
    TV_CASE(LOAD_KCONTIG, LOAD_MNCONTIG)
    TV_CASE(LOAD_KCONTIG, LOAD_KCONTIG)
    TV_CASE(LOAD_MNCONTIG, LOAD_MNCONTIG)
    TV_CASE(LOAD_MNCONTIG, LOAD_KCONTIG)
#undef TV_CASE
    return TV_E_UNSUPPORTED;
}

} // namespace tvk
