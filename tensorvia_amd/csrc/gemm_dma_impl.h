// MFMA GEMM with global -> LDS direct loads (gfx950 buffer_load_dwordx4 ... lds) for the 16-bit and
// int8 inputs when both operands have a vector layout (K- or M/N-contiguous).  Same tile math as
// gemm_mfma_kernel (gemm_mfma_impl.h); what changes is how a k-tile reaches LDS and the pipeline:
//
//  * Loads go straight from HBM/L2 into LDS: no staging registers, no ds_write, no wait for the
//    loaded data in the wave that issued it.  Each wave instruction fills one contiguous 1 KB block
//    of LDS (lane l writes bytes 16l..16l+15 of the block), so the layouts are chosen so that every
//    1 KB block is a set of whole rows and the swizzle is applied by choosing which global chunk each
//    lane loads:
//      K-contiguous operand   -> rows of 128 bytes of k, chunk c of row r at c ^ ((r >> 1) & 7)
//                                (as gemm_mfma_kernel); a block is 8 rows;
//      M/N-contiguous operand -> k rows of ROWS elements (256 or 512 bytes, no padding), 16-byte
//                                chunk q of k row r at q ^ swz(r); a block is 4 (int8) or 2 (16-bit)
//                                k rows.  swz spreads the k rows that one ds_read_b64_tr_b8/_b16
//                                pass reads over all 64 banks.
//    Lanes past the matrix edge (rows, columns or k) get an out-of-range buffer offset; the load then
//    writes zeros into LDS.
//  * Two LDS stages; a stage is one 128-byte k-tile of A and of B.  The main kernel lays LDS out as
//    [A stage 0 | A stage 1 | B stage 0 | B stage 1] and addresses every fragment of a lane from
//    one base address per operand (XOR for the swizzled bits, ds_read immediates for the stage,
//    k-group and fragment offsets), so the loop holds few address registers.
//  * Per k-tile and wave (two k-groups, 2 x FM x FN MFMAs), one workgroup barrier:
//        region 1: rows of MFMAs on k-group 0; after row i, fragment A[i] is reloaded with
//                  k-group 1, and the B fragments of k-group 1 are read;
//        wait for tile t+1's loads; barrier (tile t+1 visible everywhere, stage of tile t free);
//        region 2: rows on k-group 1; the loads of tile t+2 into the freed stage go out one per
//                  row; after row i, A[i] is reloaded with k-group 0 of tile t+1, and the B
//                  fragments of tile t+1 are read.
//    sched_group_barrier fixes the interleave (a row of MFMAs, then its reads).  The loads inside
//    the loop are inline assembly that the compiler does not see as LDS writes, so it adds no
//    waits of its own for them; every wait for them is an explicit vmcnt count.
#pragma once
#include "gemm_mfma_impl.h"

namespace tvk {

typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt on vector-memory operations only (gfx9 encoding: vmcnt in bits 3:0 and 15:14; expcnt
// and lgkmcnt at their maxima, i.e. not waited for).
template <int N> __device__ inline void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// s_waitcnt on LDS / scalar-memory operations only.
template <int N> __device__ inline void wait_lgkmcnt() {
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4) | (N << 8));
}

// Workgroup barrier for the direct-load pipeline: this wave's LDS reads have completed (lgkmcnt)
// and no memory access moves across it.  Loads into LDS are waited for explicitly (vmcnt), so
// other memory operations stay in flight (a release fence on LDS would wait for all of them).
__device__ inline void dma_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// The direct load (buffer_load_dwordx4 ... lds: 16 bytes per lane into LDS at M0 + 16 * lane) in
// inline assembly, hidden from the compiler: it then adds no waits of its own for the LDS it writes
// (callers wait with explicit vmcnt counts).  M0 is written right before the load; the s_nop covers
// the M0 and descriptor-register read-after-write wait states.
__device__ inline void dma_load16_asm(__amdgpu_buffer_rsrc_t r, char* lds_dst, unsigned off) {
    const unsigned m0v = (unsigned)(uintptr_t)(lds_void*)lds_dst;
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0v), "v"(off), "s"(r)
                 : "memory", "m0");
}

// The same load for the main k-loop.  No memory clobber: the loop's LDS reads may be scheduled
// around it (they read the other stage; the workgroup barriers order the stages).  FIRST: the
// descriptor was just written by v_readfirstlane (5 wait states before a VMEM reads it); later
// loads of the same k-tile need only the M0 wait state.
template <bool FIRST>
__device__ inline void dma_load16_loop(__amdgpu_buffer_rsrc_t r, unsigned m0v, unsigned off) {
    if constexpr (FIRST)
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0v), "v"(off), "s"(r) : "m0");
    else
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0v), "v"(off), "s"(r) : "m0");
}

template <int MODE, int ROWS, int THREADS, int ES>
struct DmaOperand {
    static constexpr int VEC = 16 / ES;            // elements per 16-byte chunk
    static constexpr int BK = 128 / ES;            // k extent of one k-tile
    static constexpr int BYTES = ROWS * 128;       // LDS bytes of one k-tile
    static constexpr int NWAVES = THREADS / 64;
    static constexpr int NBLK = BYTES / 1024;      // 1 KB load blocks per k-tile
    static constexpr int PER_WAVE = NBLK / NWAVES; // load instructions per wave per k-tile
    static constexpr int RB = ROWS * ES;           // M/N layout: bytes per k row
    static constexpr int CPR = RB / 16;            // M/N layout: chunks per k row
    static constexpr int KRB = 1024 / RB;          // M/N layout: k rows per block
    // M/N layout: LDS bytes between the k-groups of a k-tile (64 int8 / 32 16-bit k rows) and
    // between the two transposed reads of a fragment (8 / 4 k rows).
    static constexpr int KGB = (ES == 1 ? 64 : 32) * RB;
    static constexpr int RD2 = (ES == 1 ? 8 : 4) * RB;
    static_assert(NBLK % NWAVES == 0, "load blocks must divide over the waves");
    static_assert(MODE == LOAD_KCONTIG || (MODE == LOAD_MNCONTIG && ES <= 2 && (ROWS == 256 || ROWS == 128)),
                  "M/N layout is laid out for 256- and 128-row int8 / 16-bit tiles");

    const char* base; // element (row0, k = 0) of this tile, as bytes
    int64_t s_r, s_k; // element strides
    int rows_valid;   // rows of this tile inside the matrix
    int K;
    unsigned loff[PER_WAVE]; // lane byte offsets from the k-tile origin (kOOB past the matrix rows)
    int kc[PER_WAVE];        // K layout: first k of the lane's chunk inside the k-tile

    // M/N layout swizzle: distinct 16-byte bank groups for the k rows one transpose-read pass reads.
    // int8 with 128-byte k rows (128-row tiles): a k row covers half of the 64 banks, the row's
    // parity picks the half, so the 16 rows of a 32-lane pass (k rows r..r+7 and r+16..r+23) need
    // distinct chunks among the 8 rows of each parity: (kr >> 1) & 3 and bit 4 of kr; it is the same
    // for the rows 8 and 64 apart that a lane's second read and k-group 1 read, and below 8, the
    // row's chunk count.
    __device__ static inline int swz(int kr) {
        if constexpr (ES == 1 && ROWS == 128) return ((kr >> 1) & 3) | (((kr >> 4) & 1) << 2);
        else if constexpr (ES == 1) return (kr & 7) | (((kr >> 4) & 1) << 3);
        else return ((kr & 3) | (((kr >> 3) & 1) << 2)) << 1;
    }

    __device__ inline void init(int wave, int lane) {
#pragma unroll
        for (int j = 0; j < PER_WAVE; ++j) {
            const int blk = wave * PER_WAVE + j;
            if constexpr (MODE == LOAD_KCONTIG) {
                const int row = blk * 8 + (lane >> 3);
                const int c = (lane & 7) ^ ((row >> 1) & 7);
                loff[j] = row < rows_valid ? (unsigned)((int64_t)row * s_r * ES + c * 16) : kOOB;
                kc[j] = c * VEC;
            } else {
                const int kr = blk * KRB + lane / CPR;
                const int q = (lane % CPR) ^ swz(kr);
                loff[j] = q * VEC < rows_valid ? (unsigned)((int64_t)kr * s_k * ES + q * 16) : kOOB;
                kc[j] = 0;
            }
        }
    }

    // Loads k-tile k0 into `stage` (this wave's PER_WAVE blocks).  Through inline assembly: the
    // compiler then adds no waits of its own for the LDS it writes (callers wait with explicit
    // vmcnt counts).
    __device__ inline void issue(char* stage, int wave, int k0) const {
        const __amdgpu_buffer_rsrc_t rs = rsrc(k0);
#pragma unroll
        for (int j = 0; j < PER_WAVE; ++j) {
            unsigned off = loff[j];
            if constexpr (MODE == LOAD_KCONTIG) off = k0 + kc[j] < K ? off : kOOB;
            dma_load16_asm(rs, stage + (wave * PER_WAVE + j) * 1024, off);
        }
    }

    // Buffer descriptor of k-tile k0.  It lives in scalar registers and its values are
    // workgroup-uniform; reading them from the first lane states that to the compiler, which
    // otherwise may treat them as per-lane values (the inline-assembly load would then get vector
    // registers).
    __device__ inline __amdgpu_buffer_rsrc_t rsrc(int k0) const {
        const char* p;
        int64_t bytes;
        if constexpr (MODE == LOAD_KCONTIG) {
            const int rows = rows_valid < ROWS ? rows_valid : ROWS;
            p = base + (int64_t)k0 * ES;
            bytes = (int64_t)rows * s_r * ES;
        } else {
            p = base + (int64_t)k0 * s_k * ES;
            bytes = (int64_t)(K - k0) * s_k * ES;
        }
        const uint64_t u = reinterpret_cast<uint64_t>(p);
        p = reinterpret_cast<const char*>(
            (uint64_t)(unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)u) |
            ((uint64_t)(unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)(u >> 32)) << 32));
        const int nr = __builtin_amdgcn_readfirstlane(bytes <= 0 ? 0 : (bytes > 0x40000000 ? 0x40000000 : (int)bytes));
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(p), (short)0, nr, 0x00020000);
    }
    // Load j of this wave for k-tile k0 into the k-tile at LDS address `stage` (see issue()); j is
    // a constant after unrolling, and load 0 is the first use of a fresh descriptor.
    __device__ inline void issue_one(int j, __amdgpu_buffer_rsrc_t rs, unsigned stage, int wave, int k0) const {
        unsigned off = loff[j];
        if constexpr (MODE == LOAD_KCONTIG) off = k0 + kc[j] < K ? off : kOOB;
        const unsigned m0v = stage + (unsigned)((wave * PER_WAVE + j) * 1024);
        if (j == 0) dma_load16_loop<true>(rs, m0v, off);
        else dma_load16_loop<false>(rs, m0v, off);
    }

    // Main-loop fragment addressing: one per-lane LDS address `xf` (fragment 0, k-group 0, first
    // read, stage 0); every other fragment differs from it by an XOR that the lane's own bits do
    // not use and an offset that fits a ds_read immediate:
    //  K layout:   kc_off(w0 + 16f + lane%16, 4kg + lane/16) = (xf ^ 64kg) + 2048f  (the row
    //              swizzle (row >> 1) & 7 does not depend on f; k-group 1 flips chunk bit 2);
    //  M/N layout: chunk (q0 + step f) ^ swz(kr) = (q0 ^ swz(kr)) ^ (step f) because q0 has no bits
    //              below the fragment count times `step`; swz is the same for both reads of a lane
    //              (k rows kr and kr + 8 / kr + 4) and both k-groups (kr + 64 / kr + 32), so
    //              address = (xf ^ (f << FSH)) + KGB kg + RD2 (second read).  A k row's bytes (RB,
    //              256 or 512) are a whole multiple of the 64 banks, so the swizzle spreads the
    //              rows of a transposed read over the banks the same way for either.
    unsigned xf;
    static constexpr int FSH = ES == 1 ? 4 : 5;
    __device__ inline void xinit(unsigned op_base, int lane, int w0) {
        const int fr = lane & 15, grp = lane >> 4;
        if constexpr (MODE == LOAD_KCONTIG) {
            xf = op_base + kc_off(w0 + fr, grp);
        } else if constexpr (ES == 1) {
            const int kr = grp * 16 + (fr >> 1);
            xf = op_base + kr * RB + (fr & 1) * 8 + (((w0 / 16) ^ swz(kr)) << 4);
        } else {
            const int kr = grp * 8 + (fr >> 2);
            const int c = fr & 3;
            xf = op_base + kr * RB + (c >> 1) * 16 + (c & 1) * 8 + (((w0 / 8) ^ swz(kr)) << 4);
        }
    }
    // Fragment f of k-group kg in stage `st` (stage stride BYTES).
    __device__ inline u32x4 frag_at(int st, int kg, int f) const {
        if constexpr (MODE == LOAD_KCONTIG) {
            const lds_char* p = (const lds_char*)(uintptr_t)(xf ^ (unsigned)(kg << 6)) + st * BYTES + f * 2048;
            return *(const __attribute__((address_space(3))) u32x4*)p;
        } else {
            const lds_char* p = (const lds_char*)(uintptr_t)(xf ^ (unsigned)(f << FSH)) + st * BYTES + kg * KGB;
            if constexpr (ES == 1) {
                const i32x2_t a = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)p);
                const i32x2_t b = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(p + RD2));
                return u32x4{(unsigned)a.x, (unsigned)a.y, (unsigned)b.x, (unsigned)b.y};
            } else {
                const i16x4_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p);
                const i16x4_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + RD2));
                const uint2 l2 = __builtin_bit_cast(uint2, a), h2 = __builtin_bit_cast(uint2, b);
                return u32x4{l2.x, l2.y, h2.x, h2.y};
            }
        }
    }

    // Fragment addressing (see TileLoader::frag for the lane -> k assignment).
    //  K layout: b128 at kc_off(w0 + 16f + lane%16, 4kg + lane/16).
    //  M/N layout, int8:  lanes 2r+c of group g read k row 64kg + 16g + r (+8 for the second read),
    //                     bytes 8c..8c+7 of chunk w0/16 + f;
    //  M/N layout, 16-bit: lanes 4r+c of group g read k row 32kg + 8g + r (+4), bytes 8c..8c+7 of the
    //                     32-byte pair of chunks starting at w0/8 + 2f.
    int fb_lo[2], fb_hi[2]; // byte offset of the lane's k row (+ in-chunk offset), first / second read
    int sw_lo[2], sw_hi[2]; // swizzle of those k rows
    int q0;                 // first chunk of the wave's rows (M/N layout)
    int fbase[2];           // K layout

    __device__ inline void frag_init(int lane, int w0) {
        const int fr = lane & 15, grp = lane >> 4;
#pragma unroll
        for (int kg = 0; kg < 2; ++kg) {
            if constexpr (MODE == LOAD_KCONTIG) {
                fbase[kg] = kc_off(w0 + fr, kg * 4 + grp);
            } else if constexpr (ES == 1) {
                const int kr = kg * 64 + grp * 16 + (fr >> 1);
                fb_lo[kg] = kr * RB + (fr & 1) * 8;
                fb_hi[kg] = (kr + 8) * RB + (fr & 1) * 8;
                sw_lo[kg] = swz(kr);
                sw_hi[kg] = swz(kr + 8);
            } else {
                const int kr = kg * 32 + grp * 8 + (fr >> 2);
                const int c = fr & 3;
                fb_lo[kg] = kr * RB + (c >> 1) * 16 + (c & 1) * 8;
                fb_hi[kg] = (kr + 4) * RB + (c >> 1) * 16 + (c & 1) * 8;
                sw_lo[kg] = swz(kr);
                sw_hi[kg] = swz(kr + 4);
            }
        }
        q0 = ES == 1 ? w0 / 16 : w0 / 8;
    }

    __device__ inline u32x4 frag(const char* stage, int kg, int f) const {
        if constexpr (MODE == LOAD_KCONTIG) {
            return *reinterpret_cast<const u32x4*>(stage + fbase[kg] + f * 2048);
        } else if constexpr (ES == 1) {
            const int q = q0 + f;
            const lds_char* lo = (const lds_char*)(stage + fb_lo[kg] + ((q ^ sw_lo[kg]) << 4));
            const lds_char* hi = (const lds_char*)(stage + fb_hi[kg] + ((q ^ sw_hi[kg]) << 4));
            const i32x2_t a = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)lo);
            const i32x2_t b = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)hi);
            return u32x4{(unsigned)a.x, (unsigned)a.y, (unsigned)b.x, (unsigned)b.y};
        } else {
            const int q = q0 + 2 * f;
            const lds_char* lo = (const lds_char*)(stage + fb_lo[kg] + ((q ^ sw_lo[kg]) << 4));
            const lds_char* hi = (const lds_char*)(stage + fb_hi[kg] + ((q ^ sw_hi[kg]) << 4));
            const i16x4_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)lo);
            const i16x4_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)hi);
            const uint2 l2 = __builtin_bit_cast(uint2, a), h2 = __builtin_bit_cast(uint2, b);
            return u32x4{l2.x, l2.y, h2.x, h2.y};
        }
    }

    static constexpr int kFragReads = MODE == LOAD_MNCONTIG ? 2 : 1;
};

// int8 output of a whole BM x BN tile.  A wave's own block is 64-byte rows (half a cache line), so
// the per-wave staged store writes half lines; staged through LDS as one tile (rows padded by 16
// bytes), every wave instead stores whole rows of the tile, 16 bytes per lane, with the streaming
// policy.  The low byte of each exact int32 sum is kept (as the per-wave store does).  Entered with
// the k-loop's LDS free (after a workgroup barrier); L holds at least BM * (BN + 16) bytes.
template <class C>
__device__ inline void write_tile_wg_i8(const i32x4 (&acc)[C::FM][C::FN], char* L, char* Cb, int lane, int wave, int wm,
                                        int wn, int m0, int n0, const GemmDesc& d) {
    constexpr int PITCH = C::BN + 16;
    constexpr int NWAVES = C::THREADS / 64;
    constexpr int CPR = C::BN / 16;               // 16-byte chunks per tile row
    constexpr int RPW = C::BM / NWAVES;           // tile rows each wave stores
    static_assert((RPW * CPR) % 64 == 0, "whole wave stores per row group");
    // accumulators -> LDS: acc[i][j][q] is tile row wm*WM + 16i + lane%16, column
    // wn*WN + 16j + 4*(lane/16) + q; the 4 bytes of one (i, j) are one dword.
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j) {
            const int r = wm * C::WM + 16 * i + (lane & 15);
            const int c = wn * C::WN + 16 * j + 4 * (lane >> 4);
            unsigned w = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) w |= (unsigned)(uint8_t)cvt_out<int8_t>(acc[i][j][q]) << (8 * q);
            *reinterpret_cast<unsigned*>(L + r * PITCH + c) = w;
        }
    lds_barrier();
#pragma unroll
    for (int it = 0; it < RPW * CPR / 64; ++it) {
        const int idx = it * 64 + lane;
        const int r = wave * RPW + idx / CPR, c = idx % CPR;
        const u32x4 v = *reinterpret_cast<const u32x4*>(L + r * PITCH + c * 16);
        const int row = m0 + r, col = n0 + c * 16;
        if (row >= d.M) continue;
        int8_t* dst = reinterpret_cast<int8_t*>(Cb) + (int64_t)row * d.sc_m + col;
        if (col + 16 <= d.N) {
            store_stream16(dst, v);
        } else {
            const int8_t* e = reinterpret_cast<const int8_t*>(&v);
            for (int q = 0; q < 16 && col + q < d.N; ++q) dst[q] = e[q];
        }
    }
}

// Waves per SIMD the direct-load kernels' registers must allow: two for the 256x256 tile (8
// waves a workgroup, one workgroup per CU); four for the 128x128 tile (8 waves of 64x32, 64 KB of
// LDS, so two workgroups per CU).
template <class C> constexpr int dma_waves_per_eu() { return C::BM * C::BN <= 128 * 128 ? 4 : C::THREADS / 256; }

// LDS of the direct-load kernels: [A stage 0 | A stage 1 | B stage 0 | B stage 1]; the epilogue
// reuses all of it.
template <class C> constexpr int dma_lds_bytes() {
    return 2 * (DmaOperand<C::AMODE, C::BM, C::THREADS, C::ES>::BYTES + DmaOperand<C::BMODE, C::BN, C::THREADS, C::ES>::BYTES);
}

// One k-tile of the direct-load pipeline for one wave.  Stage `cs` holds k-tile t, whose k-group 0
// is already in fa / fb0; stage 1 - cs holds k-tile t + 1 once the barrier has passed.
//   Region 1: rows on k-group 0; after row i reload fa[i] with k-group 1 and read fb1[i].
//   Wait for this wave's vector-memory operations (tile t + 1's loads, and anything issued before
//   them), barrier (tile t + 1 visible, stage cs free).
//   Region 2: rows on k-group 1; one load of the k-tile at k offset k2 into stage cs per row;
//   after row i reload fa[i] with k-group 0 of tile t + 1 and read its fb0[i].
template <class C, class LA, class LB, class Acc>
__device__ __attribute__((always_inline)) inline void dma_kstep(int cs, int k2, const LA& la, const LB& lb, u32x4 (&fa)[C::FM],
                                                                u32x4 (&fb0)[C::FN], u32x4 (&fb1)[C::FN], Acc (&acc)[C::FM][C::FN],
                                                                unsigned LA0, unsigned LB0, int wave) {
    using Op = Mfma<typename C::T>;
    constexpr int NA = LA::PER_WAVE, NB = LB::PER_WAVE, NDMA = NA + NB;
    static_assert(NDMA <= C::FM, "one load per row of MFMAs");
    // Reads after each row: the row's A reload, plus B fragment i after rows i < FN.
    static_assert(C::FN <= C::FM, "one B fragment per row");
    constexpr int RD_B = 1 + LB::kFragReads;
    auto row = [&](int i, const u32x4 (&fb)[C::FN]) {
#pragma unroll
        for (int j = 0; j < C::FN; ++j) Op::run(fb[j], fa[i], acc[i][j]); // B fragment first: lanes hold 4 columns
    };
    // Interleave of a region: each row's FN MFMAs, then the reads that follow that row.
    auto sched_rows = [] {
#pragma unroll
        for (int i = 0; i < C::FN; ++i) {
            __builtin_amdgcn_sched_group_barrier(SG_MFMA, C::FN, 0);
            __builtin_amdgcn_sched_group_barrier(SG_DS_READ, RD_B, 0);
        }
#pragma unroll
        for (int i = C::FN; i < C::FM; ++i) {
            __builtin_amdgcn_sched_group_barrier(SG_MFMA, C::FN, 0);
            __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    const int ns = 1 - cs;
#pragma unroll
    for (int i = 0; i < C::FM; ++i) {
        row(i, fb0);
        fa[i] = la.frag_at(cs, 1, i);
        if (i < C::FN) fb1[i] = lb.frag_at(cs, 1, i);
    }
    sched_rows();
    const __amdgpu_buffer_rsrc_t ra = la.rsrc(k2);
    const __amdgpu_buffer_rsrc_t rb = lb.rsrc(k2);
    wait_vmcnt<0>();
    dma_barrier();
    const unsigned sa = LA0 + (unsigned)(cs * LA::BYTES), sb = LB0 + (unsigned)(cs * LB::BYTES);
#pragma unroll
    for (int i = 0; i < C::FM; ++i) {
        row(i, fb1);
        if (i < NA) la.issue_one(i, ra, sa, wave, k2);
        else if (i < NDMA) lb.issue_one(i - NA, rb, sb, wave, k2);
        if (i < C::FN) fb0[i] = lb.frag_at(ns, 0, i);
        fa[i] = la.frag_at(ns, 0, i);
    }
    sched_rows();
    // Row 0 of the next step needs fb0 and fa[0]: only the A reloads after the last B read
    // may still be in flight.
    wait_lgkmcnt<C::FM - C::FN + 1>();
}

// The k-loop of one output tile over k-tiles [kt0, kt1) into acc (zeroed by the caller).  L: the
// kernel's LDS (dma_lds_bytes).  The loaders see K as the range's end, so every load past it
// returns zeros.
template <class C>
__device__ __attribute__((always_inline)) inline void dma_tile_kloop(const GemmDesc& d, char* L, int b, int m0, int n0, int kt0,
                                                                     int kt1, typename Mfma<typename C::T>::Acc (&acc)[C::FM][C::FN]) {
    constexpr int ES = C::ES;
    using LA = DmaOperand<C::AMODE, C::BM, C::THREADS, ES>;
    using LB = DmaOperand<C::BMODE, C::BN, C::THREADS, ES>;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
    const unsigned LA0 = (unsigned)(uintptr_t)(lds_void*)L;
    const unsigned LB0 = LA0 + 2 * LA::BYTES;
    static_assert(LA::BYTES + LA::KGB + LA::RD2 < 65536 && LB::BYTES + LB::KGB + LB::RD2 < 65536 &&
                      LA::BYTES + (C::FM - 1) * 2048 < 65536 && LB::BYTES + (C::FN - 1) * 2048 < 65536,
                  "stage 1 and fragment offsets must fit a ds_read immediate");
    const int K_eff = min(d.K, kt1 * C::BK);

    LA la;
    la.base = static_cast<const char*>(d.A) + ((int64_t)b * d.sa_b + (int64_t)m0 * d.sa_m) * ES;
    la.s_r = d.sa_m; la.s_k = d.sa_k; la.rows_valid = d.M - m0; la.K = K_eff;
    LB lb;
    lb.base = static_cast<const char*>(d.B) + ((int64_t)b * d.sb_b + (int64_t)n0 * d.sb_n) * ES;
    lb.s_r = d.sb_n; lb.s_k = d.sb_k; lb.rows_valid = d.N - n0; lb.K = K_eff;
    la.init(wave, lane);
    lb.init(wave, lane);
    la.xinit(LA0, lane, wm * C::WM);
    lb.xinit(LB0, lane, wn * C::WN);

    // A fragments: one set, each reloaded with the next k-group's right after its row of MFMAs.
    // B fragments: one set per k-group of the k-tile (every row of a k-group uses all of them).
    u32x4 fa[C::FM], fb0[C::FN], fb1[C::FN];
    constexpr int NDMA = LA::PER_WAVE + LB::PER_WAVE;
    auto step = [&](int cs, int kt) {
        dma_kstep<C>(cs, (kt + 2) * C::BK, la, lb, fa, fb0, fb1, acc, LA0, LB0, wave);
    };

    // Prologue: k-tiles kt0 and kt0 + 1 in flight, then k-group 0 of kt0.
    la.issue(L, wave, kt0 * C::BK);
    lb.issue(L + 2 * LA::BYTES, wave, kt0 * C::BK);
    la.issue(L + LA::BYTES, wave, (kt0 + 1) * C::BK); // all out of range (zeros) past the range
    lb.issue(L + 2 * LA::BYTES + LB::BYTES, wave, (kt0 + 1) * C::BK);
    wait_vmcnt<NDMA>();
    lds_barrier();
#pragma unroll
    for (int j = 0; j < C::FN; ++j) fb0[j] = lb.frag_at(0, 0, j);
#pragma unroll
    for (int i = 0; i < C::FM; ++i) fa[i] = la.frag_at(0, 0, i);
    wait_lgkmcnt<C::FM - 1>();

    // The step count is rounded up to even: a step past the range multiplies the zeros loaded there
    // (the loaders' K is the range's end), and the loop has no conditional tail (the accumulators
    // stay in place across the loop).
    for (int kt = kt0; kt < kt1; kt += 2) {
        step(0, kt);
        step(1, kt + 1);
    }
    // The zero-filling loads issued by the last steps land before anything else (no load into LDS
    // is left in flight when the range ends).
    wait_vmcnt<0>();
}

// Store of one output tile (the epilogue).  acc[i][j][q] is tile row wm*WM + 16i + lane%16,
// column wn*WN + 16j + 4*(lane/16) + q.
template <class C, bool FUSED>
__device__ __attribute__((always_inline)) inline void dma_tile_store(const GemmDesc& d, char* L, int b, int m0, int n0, int c_vec,
                                                                     const typename Mfma<typename C::T>::Acc (&acc)[C::FM][C::FN]) {
    using T = typename C::T;
    using Op = Mfma<T>;
    using Acc = typename Op::Acc;
    constexpr int ES = C::ES;
    using LA = DmaOperand<C::AMODE, C::BM, C::THREADS, ES>;
    using LB = DmaOperand<C::BMODE, C::BN, C::THREADS, ES>;
    constexpr int STAGE = LA::BYTES + LB::BYTES;
    constexpr int NWAVES = C::THREADS / 64;
    static_assert(NWAVES % 2 == 0, "the epilogue gives half of the waves to each stage array");
    constexpr int EPI = STAGE / (NWAVES / 2) / 16 * 16; // staging bytes per wave in the epilogue
    char* const S0 = L;
    char* const S1 = L + STAGE;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
    (void)S0; (void)S1; (void)EPI; (void)tid;
    // All waves leave the k-loop's LDS before any wave stages its output there (the barriers below).
    const size_t csz = dtype_size(d.dtype_c);
    char* Cb = static_cast<char*>(d.C) + (int64_t)b * d.sc_b * csz;
    if constexpr (FUSED && !__is_same(Acc, i32x4)) {
        // Fused epilogue: fp32 staging, bias and activation after the accumulators are dead.
        lds_barrier();
        char* lw = (wave < NWAVES / 2 ? S0 : S1) + (wave % (NWAVES / 2)) * EPI;
        const int mrow0 = m0 + wm * C::WM, ncol0 = n0 + wn * C::WN;
        if (c_vec == 2 && (d.bias == nullptr || d.sbias_m == 0)) {
            // per-column (or no) bias: applied as the accumulators are staged by the plain store
            auto store = [&](const auto& f) {
                if (d.dtype_c == TV_BFLOAT16) write_tile_staged<__bf16, C, Acc, EPI>(acc, lw, Cb, lane, mrow0, ncol0, d, f);
                else if (d.dtype_c == TV_FLOAT16) write_tile_staged<_Float16, C, Acc, EPI>(acc, lw, Cb, lane, mrow0, ncol0, d, f);
                else write_tile_staged<float, C, Acc, EPI>(acc, lw, Cb, lane, mrow0, ncol0, d, f);
            };
            if (d.act == TV_ACT_SILU || d.act == TV_ACT_SIGMOID || d.act == TV_ACT_TANH) store(ColBiasAct<C::FN, true>(d, b, ncol0, lane));
            else store(ColBiasAct<C::FN, false>(d, b, ncol0, lane));
            return;
        }
        if (d.dtype_c == TV_BFLOAT16) write_tile_staged_epi<__bf16, C, EPI>(acc, lw, Cb, lane, mrow0, ncol0, d, b, c_vec != 0);
        else if (d.dtype_c == TV_FLOAT16) write_tile_staged_epi<_Float16, C, EPI>(acc, lw, Cb, lane, mrow0, ncol0, d, b, c_vec != 0);
        else write_tile_staged_epi<float, C, EPI>(acc, lw, Cb, lane, mrow0, ncol0, d, b, c_vec != 0);
        return;
    }
    if (c_vec == 2) {
        lds_barrier();
        char* lw = (wave < NWAVES / 2 ? S0 : S1) + (wave % (NWAVES / 2)) * EPI;
        const int mrow0 = m0 + wm * C::WM, ncol0 = n0 + wn * C::WN;
        if constexpr (__is_same(Acc, i32x4)) {
            static_assert(C::BM * (C::BN + 16) <= 2 * STAGE, "the int8 tile staging fits the k-loop's LDS");
            if (d.dtype_c == TV_INT8) write_tile_wg_i8<C>(acc, L, Cb, lane, wave, wm, wn, m0, n0, d);
            else write_tile_staged<int32_t, C, Acc, EPI>(acc, lw, Cb, lane, mrow0, ncol0, d);
        } else {
            if (d.dtype_c == TV_BFLOAT16) write_tile_staged<__bf16, C, Acc, EPI>(acc, lw, Cb, lane, mrow0, ncol0, d);
            else if (d.dtype_c == TV_FLOAT16) write_tile_staged<_Float16, C, Acc, EPI>(acc, lw, Cb, lane, mrow0, ncol0, d);
            else write_tile_staged<float, C, Acc, EPI>(acc, lw, Cb, lane, mrow0, ncol0, d);
        }
        return;
    }
    const int row0 = m0 + wm * C::WM + (lane & 15);
    const int col0 = n0 + wn * C::WN + (lane >> 4) * 4;
    const bool vec_ok = c_vec != 0;
    if constexpr (__is_same(Acc, i32x4)) {
        if (d.dtype_c == TV_INT8) write_tile<int8_t, C>(acc, Cb, row0, col0, vec_ok, d);
        else write_tile<int32_t, C>(acc, Cb, row0, col0, vec_ok, d);
    } else {
        if (d.dtype_c == TV_BFLOAT16) write_tile<__bf16, C>(acc, Cb, row0, col0, vec_ok, d);
        else if (d.dtype_c == TV_FLOAT16) write_tile<_Float16, C>(acc, Cb, row0, col0, vec_ok, d);
        else write_tile<float, C>(acc, Cb, row0, col0, vec_ok, d);
    }
}

template <class C, bool FUSED = false>
__global__ __attribute__((amdgpu_flat_work_group_size(C::THREADS, C::THREADS),
                          amdgpu_waves_per_eu(dma_waves_per_eu<C>(), dma_waves_per_eu<C>())))
void gemm_dma_kernel(GemmDesc d, int tiles_m, int tiles_n, int group_m, int c_vec) {
    using Acc = typename Mfma<typename C::T>::Acc;
    __shared__ __attribute__((aligned(1024))) char L[dma_lds_bytes<C>()];
    // Workgroup -> tile (XCD-aware, groups of group_m tile-rows), as gemm_mfma_kernel.
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
    dma_tile_kloop<C>(d, L, b, m0, n0, 0, (d.K + C::BK - 1) / C::BK, acc);
    dma_tile_store<C, FUSED>(d, L, b, m0, n0, c_vec, acc);
}

// Stream-K schedule of the direct-load kernel, as gemm_mfma_sk_kernel (same iteration ranges, slots
// and hand-over; int32 accumulators of int8 sum exactly in any order).
template <class C, bool FUSED = false>
__global__ __attribute__((amdgpu_flat_work_group_size(C::THREADS, C::THREADS),
                          amdgpu_waves_per_eu(dma_waves_per_eu<C>(), dma_waves_per_eu<C>())))
void gemm_dma_sk_kernel(GemmDesc d, int tiles_m, int tiles_n, int group_m, int c_vec, SkArgs sk) {
    using Acc = typename Mfma<typename C::T>::Acc;
    constexpr int SLOT = sk_slot_bytes<C>();
    __shared__ __attribute__((aligned(1024))) char L[dma_lds_bytes<C>()];
    __shared__ int last_flag;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = gridDim.x;
    int w = blockIdx.x;
    if ((G & 7) == 0) w = (w & 7) * (G >> 3) + (w >> 3);
    const int64_t I = sk.iters;
    const int nk = sk.nk;
    const int64_t it_end = (int64_t)(w + 1) * I / G;
    auto owner = [&](int64_t it) { return (int)(((it + 1) * G - 1) / I); };
    auto slot_rsrc = [&](int slot) { return make_rsrc(sk.slots + (int64_t)slot * SLOT, SLOT); };

    for (int64_t it = (int64_t)w * I / G; it < it_end;) {
        const int tile = (int)(it / nk);
        const int kt0 = (int)(it - (int64_t)tile * nk);
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
        dma_tile_kloop<C>(d, L, b, m0, n0, kt0, kt1, acc);
        if (kt0 != 0 || kt1 != nk) {
            const int64_t t0 = (int64_t)tile * nk;
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
            for (int v = first; v <= last; ++v) {
                const __amdgpu_buffer_rsrc_t r = slot_rsrc(v == first ? 2 * v + 1 : 2 * v);
#pragma unroll
                for (int i = 0; i < C::FM; ++i) {
#pragma unroll
                    for (int j = 0; j < C::FN; ++j) {
                        const Acc p = slot_load16<Acc>(r, (((wave * C::FM + i) * C::FN + j) * 64 + lane) * 16);
                        acc[i][j] = v == first ? p : acc[i][j] + p;
                    }
                    // one row of slot loads at a time: with all of them hoisted, the loads and the
                    // 128 accumulator registers exceed the 256 a wave has
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            slot_count_reset(sk.cnt + tile);
        }
        dma_tile_store<C, FUSED>(d, L, b, m0, n0, c_vec, acc);
    }
}

// ---------------------------------------------------------------------------------------------
// Small K (at most two 128-byte k-tiles, e.g. attention scores Q @ K^T with head dim 128): the
// output dominates, and a workgroup per tile would load, compute and store one after the other.
// Persistent workgroups (one per CU) take contiguous runs of tiles; A stays in LDS while the run
// stays in one block of rows, and B of the next tile loads while the current tile's output leaves
// through a separate staging area.
constexpr int kSmallKEpiBytes = 2304; // per wave: 16 rows of a 64-column 16-bit or 8-bit output row

// Staged store for the small-K kernel: as write_tile_staged, but every wave issues the same number
// of 16-byte buffer stores (chunks outside the matrix get an out-of-range offset and are dropped),
// so a later vmcnt wait can count them.  Requires N and the row pitch in whole 16-byte chunks.
// The stores are nontemporal (cache-policy bit nt = 2), and also sc1 (16) when a wave row is whole
// 128-byte lines: the output is written once and never re-read by this launch, and streaming it
// past the caches keeps them for the next tile's B and the resident A (c4 fp16: plain 99.7 us,
// nt 73.1 us, nt sc1 68-69 us).
template <typename TC, class C, typename Acc, int WAVE_BYTES>
__device__ inline void write_tile_fixed(const Acc (&acc)[C::FM][C::FN], char* lds_wave, __amdgpu_buffer_rsrc_t cr,
                                        int lane, int mrow0, int ncol0, const GemmDesc& d) {
    constexpr int ROWB = C::WN * (int)sizeof(TC);
    constexpr int PITCH = ROWB + 16;
    constexpr int RPP = staged_rows<C::WM, PITCH, WAVE_BYTES>();
    constexpr int CPR = ROWB / 16;
    static_assert(RPP % 16 == 0 && C::WM % RPP == 0 && RPP * PITCH <= WAVE_BYTES && (RPP * CPR) % 64 == 0,
                  "staging pass must be whole wave stores");
    typedef TC vec_t __attribute__((__vector_size__(4 * sizeof(TC))));
#pragma unroll
    for (int pass = 0; pass < C::WM / RPP; ++pass) {
#pragma unroll
        for (int i = pass * (RPP / 16); i < (pass + 1) * (RPP / 16); ++i) {
            char* rowp = lds_wave + (16 * (i - pass * (RPP / 16)) + (lane & 15)) * PITCH + (lane >> 4) * 4 * sizeof(TC);
#pragma unroll
            for (int j = 0; j < C::FN; ++j) {
                vec_t v;
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = cvt_out<TC>(acc[i][j][q]);
                *reinterpret_cast<vec_t*>(rowp + j * 16 * sizeof(TC)) = v;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
        for (int u = 0; u < RPP * CPR / 64; ++u) {
            const int idx = lane + 64 * u;
            const int r = idx / CPR, c = idx % CPR;
            const int row = mrow0 + pass * RPP + r;
            const int col = ncol0 + c * (16 / (int)sizeof(TC));
            const u32x4 v = *reinterpret_cast<const u32x4*>(lds_wave + r * PITCH + c * 16);
            const unsigned off = row < d.M && col < d.N ? (unsigned)(((int64_t)row * d.sc_m + col) * (int64_t)sizeof(TC)) : kOOB;
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), cr, (int)off, 0, ROWB % 128 == 0 ? 18 : 2);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    }
}

template <class C>
__global__ __attribute__((amdgpu_flat_work_group_size(C::THREADS, C::THREADS),
                          amdgpu_waves_per_eu(C::THREADS / 256, C::THREADS / 256)))
void gemm_smallk_kernel(GemmDesc d, int tiles_m, int tiles_n) {
    using T = typename C::T;
    using Op = Mfma<T>;
    using Acc = typename Op::Acc;
    constexpr int ES = C::ES;
    using LA = DmaOperand<C::AMODE, C::BM, C::THREADS, ES>;
    using LB = DmaOperand<C::BMODE, C::BN, C::THREADS, ES>;
    constexpr int NWAVES = C::THREADS / 64;
    constexpr int EPI = kSmallKEpiBytes;

    // A's two k-tiles stay resident while consecutive tiles share them (same batch and rows); B's
    // two k-tiles are reloaded per tile.
    __shared__ __attribute__((aligned(1024))) char SA[2 * LA::BYTES];
    __shared__ __attribute__((aligned(1024))) char SB[2 * LB::BYTES];
    __shared__ __attribute__((aligned(16))) char E[EPI * NWAVES];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
    const int per_batch = tiles_m * tiles_n;
    const int ntiles = per_batch * d.batch;

    LA la;
    LB lb;
    la.s_r = d.sa_m; la.s_k = d.sa_k; la.K = d.K;
    lb.s_r = d.sb_n; lb.s_k = d.sb_k; lb.K = d.K;
    la.frag_init(lane, wm * C::WM);
    lb.frag_init(lane, wn * C::WN);

    // Workgroup w takes the contiguous tiles [w*ntiles/G, (w+1)*ntiles/G) in (batch, m, n) order, so
    // consecutive tiles share A; ids are remapped so that neighbouring ranges (same batch, sharing
    // B) run on one XCD.
    const int G = gridDim.x;
    int w = blockIdx.x;
    if ((G & 7) == 0) w = (w & 7) * (G >> 3) + (w >> 3);
    const int t_end = (int)((int64_t)(w + 1) * ntiles / G);

    // Points the loaders at tile t and loads its k-tiles (A only when it changes).  Past t_end every
    // lane is out of range and nothing is read.
    int cur_b = -1, cur_m0 = -1;
    auto start = [&](int t, int& b, int& m0, int& n0) {
        const bool live = t < t_end;
        const int tt = live ? t : t_end - 1;
        b = tt / per_batch;
        const int r = tt - b * per_batch;
        m0 = (r / tiles_n) * C::BM;
        n0 = (r % tiles_n) * C::BN;
        lb.base = static_cast<const char*>(d.B) + ((int64_t)b * d.sb_b + (int64_t)n0 * d.sb_n) * ES;
        lb.rows_valid = live ? d.N - n0 : 0;
        lb.init(wave, lane);
        lb.issue(SB, wave, 0);
        lb.issue(SB + LB::BYTES, wave, C::BK); // zeros when K fits in one k-tile
        if (live && (b != cur_b || m0 != cur_m0)) { // uniform over the workgroup
            cur_b = b;
            cur_m0 = m0;
            la.base = static_cast<const char*>(d.A) + ((int64_t)b * d.sa_b + (int64_t)m0 * d.sa_m) * ES;
            la.rows_valid = d.M - m0;
            la.init(wave, lane);
            la.issue(SA, wave, 0);
            la.issue(SA + LA::BYTES, wave, C::BK);
        }
    };

    int t = (int)((int64_t)w * ntiles / G), b, m0, n0;
    start(t, b, m0, n0);
    const size_t csz = dtype_size(d.dtype_c);
    constexpr int NST = C::WM * (C::WN * ES / 16) / 64; // epilogue stores per wave (output type = input size)
    wait_vmcnt<0>();
    for (;;) {
        dma_barrier(); // this tile's operands have landed everywhere
        Acc acc[C::FM][C::FN];
#pragma unroll
        for (int i = 0; i < C::FM; ++i)
#pragma unroll
            for (int j = 0; j < C::FN; ++j) acc[i][j] = Acc{0, 0, 0, 0};
        // Both k-tiles, always (the second holds zeros when K fits in one).
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int kg = 0; kg < 2; ++kg) {
                u32x4 fa[C::FM], fb[C::FN];
#pragma unroll
                for (int j = 0; j < C::FN; ++j) fb[j] = lb.frag(SB + kt * LB::BYTES, kg, j);
#pragma unroll
                for (int i = 0; i < C::FM; ++i) fa[i] = la.frag(SA + kt * LA::BYTES, kg, i);
#pragma unroll
                for (int i = 0; i < C::FM; ++i)
#pragma unroll
                    for (int j = 0; j < C::FN; ++j) Op::run(fb[j], fa[i], acc[i][j]);
            }
        }
        dma_barrier(); // every wave is done reading the operands
        const int cb = b, cm0 = m0, cn0 = n0;
        const int next = t + 1;
        start(next, b, m0, n0);
        // The output of tile t leaves while the next tile's operands load.
        const char* Cb = static_cast<const char*>(d.C) + (int64_t)cb * d.sc_b * csz;
        const __amdgpu_buffer_rsrc_t cr = make_rsrc(Cb, ((int64_t)(d.M - 1) * d.sc_m + d.N) * (int64_t)csz);
        char* lw = E + wave * EPI;
        const int mrow0 = cm0 + wm * C::WM, ncol0 = cn0 + wn * C::WN;
        if constexpr (__is_same(Acc, i32x4)) {
            write_tile_fixed<int8_t, C, Acc, EPI>(acc, lw, cr, lane, mrow0, ncol0, d);
        } else {
            if (d.dtype_c == TV_BFLOAT16) write_tile_fixed<__bf16, C, Acc, EPI>(acc, lw, cr, lane, mrow0, ncol0, d);
            else write_tile_fixed<_Float16, C, Acc, EPI>(acc, lw, cr, lane, mrow0, ncol0, d);
        }
        if (next >= t_end) break;
        t = next;
        // The next tile's operands were loaded before this tile's NST stores (vmcnt retires in issue
        // order), so waiting down to NST outstanding operations leaves only the stores in flight.
        wait_vmcnt<NST>();
    }
    wait_vmcnt<0>();
}

// Small K, 16-bit: each tile's stores spread over the next tile's MFMAs, and the tiles ordered so
// that the workgroups running at any moment write whole runs of rows of C.  At small K the output
// stores are the work (c4: 268 MB of C against 34 MB of operands); what they cost depends on their
// order: with each workgroup taking a contiguous run of (batch, m, n) tiles, the 256 workgroups
// write 256-byte pieces of 128 rows each, 4 KB apart and scattered over C, and c4's stores run at
// 3.8 TB/s; with the 16 column tiles of a row block taken by 16 workgroups at the same time, the
// same stores run at about 5.5 TB/s (c4 72 against 49 us with the operand loads dropped).
//  * Workgroups form groups of P = ceil(tiles_n / 2); workgroup p of a group stores column tiles p
//    and p + P of each row block (batch, m) in the group's contiguous range, one after the other,
//    so one load of A serves two tiles (A's loads compete with the stores for the CU's memory
//    path: c4 loading A for every tile ran 9 % slower).  The group writes the left half of the
//    row block's rows, then the right half.
//  * LDS: A double-buffered (2 x 32 KB, loaded one row block ahead), one B per column tile
//    (2 x 32 KB, reloaded at a new batch in the iteration after its last use), and the output
//    tile (128 rows of 256 bytes, the 16-byte chunks of row r XOR-ed with r % 16, so neither the
//    fragment writes nor the row reads conflict): 160 KB.
//  * The output of a tile waits in LDS; the next iteration issues one store per wave after each
//    k-group of 8 MFMAs.  That iteration's loads were issued before those stores, so the wait at
//    its end leaves the 4 stores in flight (vmcnt retires in issue order).
//  * Each wave stores 16 whole rows of the tile, 4 rows per instruction, with the streaming
//    policy (nt sc1): whole 128-byte lines.  Stores outside C (the first iteration's, which has no
//    previous tile, and column tile p + P where it is past N) get an out-of-range offset, so every
//    wave issues the same count.
template <class C, typename TC>
__global__ __attribute__((amdgpu_flat_work_group_size(C::THREADS, C::THREADS), amdgpu_waves_per_eu(2, 2)))
void gemm_smallk_pipe_kernel(GemmDesc d, int tiles_m, int tiles_n, int ngroups) {
    using T = typename C::T;
    using Op = Mfma<T>;
    using Acc = typename Op::Acc;
    constexpr int ES = C::ES;
    static_assert(ES == 2 && sizeof(TC) == 2 && C::BM == 128 && C::BN == 128 && C::THREADS == 512,
                  "16-bit inputs and output, 128x128 tiles, 8 waves");
    using LA = DmaOperand<C::AMODE, C::BM, C::THREADS, ES>;
    using LB = DmaOperand<C::BMODE, C::BN, C::THREADS, ES>;
    constexpr int NWAVES = C::THREADS / 64;
    constexpr int OROW = C::BN * ES;               // bytes of one output row (16 chunks)
    constexpr int RPW = C::BM / NWAVES;            // output rows each wave stores
    constexpr int CPR = OROW / 16;                 // 16-byte chunks per output row
    constexpr int NST = RPW * CPR / 64;            // store instructions per wave and tile
    constexpr int RPS = 64 / CPR;                  // rows per store instruction
    static_assert(NST == 4 && CPR == 16 && C::FM * C::FN == 8, "one store after each k-group of 8 MFMAs");

    __shared__ __attribute__((aligned(1024))) char SA[2][2 * LA::BYTES];
    __shared__ __attribute__((aligned(1024))) char SB[2][2 * LB::BYTES]; // SB[s]: B of column tile s
    __shared__ __attribute__((aligned(1024))) char SO[C::BM * OROW];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;

    LA la;
    LB lb;
    la.s_r = d.sa_m; la.s_k = d.sa_k; la.K = d.K;
    lb.s_r = d.sb_n; lb.s_k = d.sb_k; lb.K = d.K;
    la.frag_init(lane, wm * C::WM);
    lb.frag_init(lane, wn * C::WN);

    // The grid is ngroups * P workgroups; ids are remapped so that neighbouring ids (one group,
    // sharing A) run on one XCD.
    const int P = (tiles_n + 1) >> 1;
    const int G = gridDim.x;
    int w = blockIdx.x;
    if ((G & 7) == 0) w = (w & 7) * (G >> 3) + (w >> 3);
    const int grp = w / P;
    const int p = w - grp * P;
    const int n0_0 = p * C::BN, n0_1 = (p + P) * C::BN; // the second may lie past N: no reads, no stores
    const int R = tiles_m * d.batch; // row blocks (batch, m)
    const int r_begin = (int)((int64_t)grp * R / ngroups);
    const int r_end = (int)((int64_t)(grp + 1) * R / ngroups);
    if (r_begin >= r_end) return; // uniform

    auto load_a = [&](int r, char* dst) {
        const int b = r / tiles_m, m0 = (r - b * tiles_m) * C::BM;
        la.base = static_cast<const char*>(d.A) + ((int64_t)b * d.sa_b + (int64_t)m0 * d.sa_m) * ES;
        la.rows_valid = d.M - m0;
        la.init(wave, lane);
        la.issue(dst, wave, 0);
        la.issue(dst + LA::BYTES, wave, C::BK); // zeros when K fits in one k-tile
    };
    auto load_b = [&](int b, int n0, char* dst) {
        lb.base = static_cast<const char*>(d.B) + ((int64_t)b * d.sb_b + (int64_t)n0 * d.sb_n) * ES;
        lb.rows_valid = d.N - n0; // <= 0: every lane out of range, zeros
        lb.init(wave, lane);
        lb.issue(dst, wave, 0);
        lb.issue(dst + LB::BYTES, wave, C::BK);
    };

    const int64_t cbytes = ((int64_t)(d.M - 1) * d.sc_m + d.N) * ES;
    // This lane's output chunks: rows wave*RPW + s*RPS + lane/CPR, chunk lane%CPR.
    const int srow = wave * RPW + lane / CPR;
    const int schunk = lane % CPR;
    // Reads this lane's rows of the staged output (row block pr, column tile origin pn0) from LDS and
    // makes their global offsets.
    auto stage_out = [&](int pr, int pn0, u32x4 (&v)[NST], unsigned (&off)[NST]) {
        const int pb = pr < 0 ? 0 : pr / tiles_m;
        const int pm0 = pr < 0 ? 0 : (pr - pb * tiles_m) * C::BM;
#pragma unroll
        for (int s = 0; s < NST; ++s) {
            const int lr = srow + s * RPS;
            v[s] = *reinterpret_cast<const u32x4*>(SO + lr * OROW + ((schunk ^ (lr & 15)) << 4));
            const int row = pm0 + lr;
            const int col = pn0 + schunk * (16 / ES);
            off[s] = pr >= 0 && row < d.M && col < d.N ? (unsigned)(((int64_t)row * d.sc_m + col) * ES) : kOOB;
        }
        return make_rsrc(static_cast<const char*>(d.C) + (int64_t)pb * d.sc_b * ES, cbytes);
    };

    {
        const int b = r_begin / tiles_m;
        load_a(r_begin, SA[0]);
        load_b(b, n0_0, SB[0]);
        load_b(b, n0_1, SB[1]);
    }
    wait_vmcnt<0>();
    dma_barrier();

    int pr = -1, pn0 = 0; // the tile whose output is in SO (pr < 0: none yet)
    int ca = 0;
    for (int r = r_begin; r < r_end; ++r) {
        const int b = r / tiles_m;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            // Operands of later tiles into buffers that no later MFMA of this row block reads
            // (uniform conditions): A of the next row block; at a new batch, B of column tile 1
            // (last read by the previous row block) and then B of column tile 0 for the next row
            // block (last read by this row block's first tile).
            if (s == 0) {
                if (r + 1 < r_end) load_a(r + 1, SA[ca ^ 1]);
                if (r > r_begin && b != (r - 1) / tiles_m) load_b(b, n0_1, SB[1]);
            } else if (r + 1 < r_end && (r + 1) / tiles_m != b) {
                load_b((r + 1) / tiles_m, n0_0, SB[0]);
            }
            u32x4 sv[NST];
            unsigned soff[NST];
            const __amdgpu_buffer_rsrc_t cr = stage_out(pr, pn0, sv, soff);

            Acc acc[C::FM][C::FN];
#pragma unroll
            for (int i = 0; i < C::FM; ++i)
#pragma unroll
                for (int j = 0; j < C::FN; ++j) acc[i][j] = Acc{0, 0, 0, 0};
            const char* sa = SA[ca];
            const char* sb = SB[s];
            u32x4 fa[2][C::FM], fb[2][C::FN];
#pragma unroll
            for (int j = 0; j < C::FN; ++j) fb[0][j] = lb.frag(sb, 0, j);
#pragma unroll
            for (int i = 0; i < C::FM; ++i) fa[0][i] = la.frag(sa, 0, i);
            // k-group g = 2 * k-tile + group inside the k-tile; the next group's fragments are
            // read while this group's MFMAs run, and one store goes out after each group.
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int x = g & 1;
                if (g < 3) {
                    const int kt = (g + 1) >> 1, kg = (g + 1) & 1;
#pragma unroll
                    for (int j = 0; j < C::FN; ++j) fb[x ^ 1][j] = lb.frag(sb + kt * LB::BYTES, kg, j);
#pragma unroll
                    for (int i = 0; i < C::FM; ++i) fa[x ^ 1][i] = la.frag(sa + kt * LA::BYTES, kg, i);
                }
#pragma unroll
                for (int i = 0; i < C::FM; ++i)
#pragma unroll
                    for (int j = 0; j < C::FN; ++j) Op::run(fb[x][j], fa[x][i], acc[i][j]);
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, sv[g]), cr, (int)soff[g], 0, 18);
                __builtin_amdgcn_sched_barrier(0);
            }
            dma_barrier(); // every wave is done with these operands and with the staged output

            // This tile's output into SO: acc[i][j][q] is tile row wm*WM + 16i + lane%16, column
            // wn*WN + 16j + 4*(lane/16) + q; 8 bytes at byte 2*column of the row, chunk-swizzled.
#pragma unroll
            for (int i = 0; i < C::FM; ++i)
#pragma unroll
                for (int j = 0; j < C::FN; ++j) {
                    const int row = wm * C::WM + 16 * i + (lane & 15);
                    const int cbyte = (wn * C::WN + 16 * j + 4 * (lane >> 4)) * ES;
                    typedef TC v4 __attribute__((__vector_size__(4 * sizeof(TC))));
                    const v4 h = {cvt_out<TC>(acc[i][j][0]), cvt_out<TC>(acc[i][j][1]), cvt_out<TC>(acc[i][j][2]),
                                  cvt_out<TC>(acc[i][j][3])};
                    *reinterpret_cast<uint2*>(SO + row * OROW + (((cbyte >> 4) ^ (row & 15)) << 4) + (cbyte & 15)) =
                        __builtin_bit_cast(uint2, h);
                }
            wait_vmcnt<NST>(); // this iteration's loads (issued before its stores)
            dma_barrier();     // ... and this tile's staged output are visible to every wave
            pr = r;
            pn0 = s ? n0_1 : n0_0;
        }
        ca ^= 1;
    }
    {
        u32x4 sv[NST];
        unsigned soff[NST];
        const __amdgpu_buffer_rsrc_t cr = stage_out(pr, pn0, sv, soff);
#pragma unroll
        for (int s = 0; s < NST; ++s)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, sv[s]), cr, (int)soff[s], 0, 18);
    }
    wait_vmcnt<0>();
}

// Persistent direct-load GEMM for launches of several tiles per CU (one resident workgroup per
// CU).  The k-loop runs on from one tile into the next: the last two k-steps of a tile load
// k-tiles 0 and 1 of the workgroup's next tile, so when a tile's output is stored the next tile's
// first k-tile has landed, its k-group-0 fragments are in registers, and its second k-tile is
// loading.  One workgroup per tile instead loads its first two k-tiles only after the previous
// workgroup on the CU has stored its output.
//  * The output is staged through an LDS area of its own (the k-loop's stages hold the next
//    tile's operands), 16 rows per pass and wave.  The next tile's first step waits for the
//    stores along with its k-tile 1 loads (vmcnt retires in issue order), after a region of
//    MFMAs.
//  * Workgroup s of XCD x (ids x, x + 8, ...) takes the tiles lo + s, lo + s + S, ... of its XCD's
//    range [lo, hi) (S: the XCD's workgroups), the order in which one workgroup per tile would run
//    them, so the tiles in flight on an XCD share A and B rows in its L2 as before.
//  * 16-bit inputs and outputs, with 16-byte aligned rows (an fp32 staging area does not fit
//    beside the stages; int8 outputs keep the one-per-tile kernel, whose store writes whole
//    256-byte rows of the tile: 1 % faster there than this kernel's 64-byte wave rows).
//  * Same bits as one workgroup per tile (the same k-loop per tile).  Measured on one box against
//    it: c3 829 against 830 us, [8192]^3 788 against 806, [4096,1024] @ [1024,32768] 241 against
//    260 (the fixed cost per tile saved is a larger share at short K).
template <class C>
__global__ __attribute__((amdgpu_flat_work_group_size(C::THREADS, C::THREADS),
                          amdgpu_waves_per_eu(C::THREADS / 256, C::THREADS / 256)))
void gemm_dma_chain_kernel(GemmDesc d, int tiles_m, int tiles_n, int group_m, int ntiles) {
    using T = typename C::T;
    using Acc = typename Mfma<T>::Acc;
    static_assert(!__is_same(T, int8_t), "16-bit inputs");
    constexpr int ES = C::ES;
    using LA = DmaOperand<C::AMODE, C::BM, C::THREADS, ES>;
    using LB = DmaOperand<C::BMODE, C::BN, C::THREADS, ES>;
    constexpr int NWAVES = C::THREADS / 64;
    constexpr int EPI = kSmallKEpiBytes; // 16 rows of a 64-column 16-bit row, padded
    constexpr int NDMA = LA::PER_WAVE + LB::PER_WAVE;
    __shared__ __attribute__((aligned(1024))) char L[dma_lds_bytes<C>()];
    __shared__ __attribute__((aligned(16))) char E[EPI * NWAVES];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
    const unsigned LA0 = (unsigned)(uintptr_t)(lds_void*)L;
    const unsigned LB0 = LA0 + 2 * LA::BYTES;

    int s = blockIdx.x, S = gridDim.x, lo = 0, hi = ntiles;
    if ((gridDim.x & 7) == 0) {
        const int x = blockIdx.x & 7;
        s = blockIdx.x >> 3;
        S = gridDim.x >> 3;
        lo = (int)((int64_t)x * ntiles / 8);
        hi = (int)((int64_t)(x + 1) * ntiles / 8);
    }
    int t = lo + s;
    if (t >= hi) return;

    LA la;
    LB lb;
    la.s_r = d.sa_m; la.s_k = d.sa_k; la.K = d.K;
    lb.s_r = d.sb_n; lb.s_k = d.sb_k; lb.K = d.K;
    la.xinit(LA0, lane, wm * C::WM);
    lb.xinit(LB0, lane, wn * C::WN);
    // Points the loaders at tile u; past the range every lane is out of range and loads zeros.
    // Lane-derived values of the loaders' and the store's addressing are computed where they are
    // used, from a copy of the lane id that the compiler cannot hoist: kept live across the k-loop
    // they would not fit the 256 registers of a wave.
    auto lane_here = [&] {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        return ln;
    };
    auto point = [&](int u) {
        const int ln = lane_here();
        const bool live = u < hi;
        int b, tm, tn;
        mfma_tile_of(live ? u : t, tiles_m, tiles_n, group_m, b, tm, tn);
        const int m0 = tm * C::BM, n0 = tn * C::BN;
        la.base = static_cast<const char*>(d.A) + ((int64_t)b * d.sa_b + (int64_t)m0 * d.sa_m) * ES;
        la.rows_valid = live ? d.M - m0 : 0;
        lb.base = static_cast<const char*>(d.B) + ((int64_t)b * d.sb_b + (int64_t)n0 * d.sb_n) * ES;
        lb.rows_valid = live ? d.N - n0 : 0;
        la.init(wave, ln);
        lb.init(wave, ln);
    };

    u32x4 fa[C::FM], fb0[C::FN], fb1[C::FN];
    // Prologue: k-tiles 0 and 1 of the first tile.
    point(t);
    la.issue(L, wave, 0);
    lb.issue(L + 2 * LA::BYTES, wave, 0);
    la.issue(L + LA::BYTES, wave, C::BK);
    lb.issue(L + 2 * LA::BYTES + LB::BYTES, wave, C::BK);
    wait_vmcnt<NDMA>();
    lds_barrier();
#pragma unroll
    for (int j = 0; j < C::FN; ++j) fb0[j] = lb.frag_at(0, 0, j);
#pragma unroll
    for (int i = 0; i < C::FM; ++i) fa[i] = la.frag_at(0, 0, i);
    wait_lgkmcnt<C::FM - 1>();

    const int nk = (d.K + C::BK - 1) / C::BK;
    const int P = (nk + 1) & ~1; // steps per tile (a step past K multiplies zeros)
    for (;;) {
        int b, tm, tn;
        mfma_tile_of(t, tiles_m, tiles_n, group_m, b, tm, tn);
        const int next = t + S;
        Acc acc[C::FM][C::FN];
#pragma unroll
        for (int i = 0; i < C::FM; ++i)
#pragma unroll
            for (int j = 0; j < C::FN; ++j) acc[i][j] = Acc{0, 0, 0, 0};
        // Step k loads k-tile k + 2; the last two steps (k = P - 2, P - 1) load the next tile's
        // k-tiles 0 and 1.  The first step's wait for k-tile 1 also waits for the previous tile's
        // stores (issued after those loads), which have had the step's first region to land.
        for (int kt = 0; kt < P; kt += 2) {
            const bool last = kt + 2 == P;
            if (last) point(next);
            const int k2 = last ? 0 : (kt + 2) * C::BK;
            dma_kstep<C>(0, k2, la, lb, fa, fb0, fb1, acc, LA0, LB0, wave);
            dma_kstep<C>(1, k2 + C::BK, la, lb, fa, fb0, fb1, acc, LA0, LB0, wave);
        }
        char* Cb = static_cast<char*>(d.C) + (int64_t)b * d.sc_b * (int64_t)dtype_size(d.dtype_c);
        char* lw = E + wave * EPI;
        const int ln = lane_here(), mrow0 = tm * C::BM + wm * C::WM, ncol0 = tn * C::BN + wn * C::WN;
        if (d.dtype_c == TV_BFLOAT16) write_tile_staged<__bf16, C, Acc, EPI>(acc, lw, Cb, ln, mrow0, ncol0, d);
        else write_tile_staged<_Float16, C, Acc, EPI>(acc, lw, Cb, ln, mrow0, ncol0, d);
        if (next >= hi) break;
        t = next;
    }
    // The last tile's zero-filling loads and its stores land before the workgroup ends.
    wait_vmcnt<0>();
}

// Workgroups of `kernel` (THREADS threads, static LDS only) resident at once on device dev: the
// occupancy API's count per CU times the CUs; 0 if the runtime cannot tell.
static int resident_grid(const void* kernel, int threads, int dev) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu <= 0 || cus <= 0)
        return 0;
    return per_cu * cus;
}

// Chained launch: one workgroup per CU walking several tiles.  Returns 1 if it did not launch:
// fewer than two tiles per CU, or an output other than 16-bit with 16-byte aligned rows.
template <class C>
static int run_dma_chain(const GemmDesc& d, hipStream_t stream, int group_m, int tiles_m, int tiles_n, int64_t ntiles, int c_vec) {
    if (c_vec != 2 || !(d.dtype_c == TV_BFLOAT16 || d.dtype_c == TV_FLOAT16)) return 1;
    static std::atomic<int> grid[kMaxDevices];
    const int G = cached_per_device(grid, [](int dev) { return resident_grid(reinterpret_cast<const void*>(gemm_dma_chain_kernel<C>), C::THREADS, dev); });
    if (G <= 0) return 1;
    if (ntiles < 2 * (int64_t)G) return 1;
    hipLaunchKernelGGL(gemm_dma_chain_kernel<C>, dim3((unsigned)G), dim3(C::THREADS), 0, stream, d, tiles_m, tiles_n, group_m, (int)ntiles);
    return hipGetLastError();
}

// Stream-K launch of the direct-load kernel for few, long tiles: at most a quarter as many 256x256
// tiles (half as many 128x128 tiles) as resident workgroups, and K of at least 64 k-tiles.  A split tile moves its fp32 partial sums
// through the slots once per segment, which costs more than the balance gains once the tiles are
// many.  Measured (settled clocks, same box, against one workgroup per tile) on int8 256x256 tiles
// (one resident per CU): [512,8192]@[8192,8192] 52.0 against 75.5 us; and on bf16 256x256 tiles
// before 16-bit GEMMs this small moved to 128x128 tiles: [512,8192]@[8192,8192] 88.9 against
// 146.7 us, but 192 tiles (M = 3000, K = 4096) 121.5 against 83.0 us.  bf16 [128,8192]@[8192,8192]
// (64 tiles of 128x128, two resident per CU) runs 43.5 us split.  c2 (256 tiles) and c3 (2048)
// keep one workgroup per tile.  128x128 tiles split at up to half the resident workgroups: bf16
// [512,8192]@[8192,8192] (256 tiles on 512 slots) 74.2 against 79.2 us, [1024,8192]@[8192,4096]
// 74.5 against 80.1, [1024,4096]@[4096,4096] 43.0 against 45.1.  Returns 1 if it did not launch.
template <class C, bool FUSED>
static int run_dma_sk(const GemmDesc& d, hipStream_t stream, int group_m, int tiles_m, int tiles_n, int64_t ntiles, int c_vec) {
    const int nk = (d.K + C::BK - 1) / C::BK;
    if (nk < (__is_same(typename C::T, int8_t) ? 16 : 64)) return 1;
    static std::atomic<int> grid[kMaxDevices];
    int G = cached_per_device(grid, [](int dev) { return resident_grid(reinterpret_cast<const void*>(gemm_dma_sk_kernel<C, false>), C::THREADS, dev); });
    if (G <= 0) return 1;
    if (ntiles * (C::BM == 128 ? 2 : 4) > G) return 1;
    // 16-bit 128x128 tiles above a quarter of the resident workgroups split only into segments of
    // at least 32 k-tiles, or when the tile grid is one row or one column (each tile then streams
    // its own rows of A or columns of B, HBM-bound, and the split adds streams).  Shorter segments
    // of tiles whose operands are reused from L2 cost more in prologues and slot traffic than the
    // idle CUs: bf16 [3000,4096]@[4096,1000] (192 tiles, 24 k-tiles per segment) 58.0 -> 47.3 us
    // unsplit, [300,4096]@[4096,10000] 63.8 -> 59.2, [600,4096]@[4096,4096] 47.3 -> 43.0; but
    // [8][3000,4096]@[4096,64] (192 tiles, one column each) 61.2 us split against 69.8,
    // [300,4096]@[4096,4096] (96 tiles) 29.1 against 41.9, and [2048,8192]@[8192,2048] (256 tiles,
    // 64 k-tiles per segment) 77.8 against 81.7.
    if constexpr (!__is_same(typename C::T, int8_t) && C::BM == 128)
        if (ntiles * 4 > G && tiles_m >= 2 && tiles_n >= 2 && ntiles * nk < 32 * (int64_t)G) return 1;
    // int8 256x256 tiles split from 16 k-tiles (K >= 2048) when they are few (at most a fifth of
    // the resident workgroups): one such tile takes a CU about 40 us at K = 4096, so a few of them
    // leave the chip idle (int8 [512,4096]@[4096,4096] 41.0 -> 33.3 us, [256,4096]@[4096,4096]
    // 40.5 -> 31.6, [16,4096]@[4096,4096] 40.2 -> 31.0); 64 tiles were slower split
    // ([2048,2048]^3 24.2 against 28.5 us).  16-bit tiles split from 64 k-tiles.
    if (nk < 64 && ntiles * 5 > G) return 1;
    const int64_t iters = ntiles * nk;
    if (iters / 8 < G) G = (int)(iters / 8);
    // At most about four segments per tile, unless the segments stay at least 32 k-tiles long:
    // bf16 [256,4096]@[4096,4096] (64 tiles of 128x128) 24.5 us in 4 against 32.0 in 8 and 28.7 in
    // 2, [128,8192]@[8192,8192] 39.7 against 44.9 in 8; a single tile over K = 65536 keeps 32
    // workgroups rather than 4.
    const int64_t cap = 4 * ntiles > iters / 32 ? 4 * ntiles : iters / 32;
    if (cap < G) G = (int)cap;
    if (G < 1) return 1;
    SkArgs sk;
    sk.iters = iters;
    sk.nk = nk;
    sk.dp_tiles = 0; // every tile is split here (at most a quarter as many tiles as workgroups)
    sk.wgs = G;
    const int rc = gemm_sk_workspace(stream, (size_t)ntiles, (size_t)2 * G * sk_slot_bytes<C>(), &sk.cnt, &sk.slots);
    if (rc == TV_E_NOMEM) return 1; // no room for the slots: one workgroup per tile serves the call
    if (rc) return rc;
    hipLaunchKernelGGL((gemm_dma_sk_kernel<C, FUSED>), dim3((unsigned)G), dim3(C::THREADS), 0, stream, d, tiles_m, tiles_n, group_m,
                       c_vec, sk);
    return hipGetLastError();
}

template <class C>
static int run_dma_cfg(const GemmDesc& d, hipStream_t stream, int group_m, bool may_alloc) {
    const int tiles_m = (d.M + C::BM - 1) / C::BM;
    const int tiles_n = (d.N + C::BN - 1) / C::BN;
    const int64_t nwg = (int64_t)tiles_m * tiles_n * d.batch;
    if (nwg <= 0) return 0;
    if (nwg > 0x7FFFFFFF) return TV_E_SHAPE;
    const size_t csz = dtype_size(d.dtype_c);
    int c_vec = d.sc_n == 1 && d.sc_m % 4 == 0 && (d.batch <= 1 || d.sc_b % 4 == 0) &&
                (reinterpret_cast<uintptr_t>(d.C) % (4 * csz)) == 0;
    const int64_t v16 = 16 / (int64_t)csz;
    if (c_vec && d.sc_m % v16 == 0 && (d.batch <= 1 || d.sc_b % v16 == 0) &&
        (reinterpret_cast<uintptr_t>(d.C) % 16) == 0 && (C::WN * (int64_t)csz) % 16 == 0)
        c_vec = 2;
    // The fused epilogue runs in the staged store only (16-byte aligned rows of C).
    const bool epi = d.bias != nullptr || d.act != TV_ACT_NONE;
    if (epi && d.sc_n != 1) return TV_E_UNSUPPORTED; // the fused store writes rows of C
    if (may_alloc) {
        // 16-bit GEMMs few enough to split (at most a quarter as many 256x256 tiles as CUs) always
        // take 128x128 tiles in run_modes_dma, so the 256x256 16-bit configurations never split.
        int rc = 1;
        if constexpr (__is_same(typename C::T, int8_t))
            rc = run_dma_sk<C, false>(d, stream, group_m, tiles_m, tiles_n, nwg, c_vec);
        else if constexpr (C::BM == 128)
            rc = epi ? run_dma_sk<C, true>(d, stream, group_m, tiles_m, tiles_n, nwg, c_vec)
                     : run_dma_sk<C, false>(d, stream, group_m, tiles_m, tiles_n, nwg, c_vec);
        if (rc != 1) return rc;
    }
    if constexpr (!__is_same(typename C::T, int8_t) && C::BM == 256)
        if (!epi) {
            const int rc = run_dma_chain<C>(d, stream, group_m, tiles_m, tiles_n, nwg, c_vec);
            if (rc != 1) return rc;
        }
    if constexpr (!__is_same(typename C::T, int8_t))
        if (epi) {
            hipLaunchKernelGGL((gemm_dma_kernel<C, true>), dim3((unsigned)nwg), dim3(C::THREADS), 0, stream, d, tiles_m, tiles_n,
                               group_m, c_vec);
            return hipGetLastError();
        }
    hipLaunchKernelGGL(gemm_dma_kernel<C>, dim3((unsigned)nwg), dim3(C::THREADS), 0, stream, d, tiles_m, tiles_n,
                       group_m, c_vec);
    return hipGetLastError();
}

// Small-K path: K within two 128-byte k-tiles, an 8- or 16-bit output (int8 inputs: int8 output;
// half inputs: half output) with 16-byte aligned rows, and enough tiles to keep every CU busy.
template <class C>
static int run_smallk_cfg(const GemmDesc& d, hipStream_t stream) {
    const int tiles_m = (d.M + C::BM - 1) / C::BM;
    const int tiles_n = (d.N + C::BN - 1) / C::BN;
    const int64_t nt = (int64_t)tiles_m * tiles_n * d.batch;
    if (nt > 0x7FFFFFFF) return TV_E_SHAPE;
    const int cus = device_cus();
    const int grid = (int)(nt < cus ? nt : cus);
    hipLaunchKernelGGL(gemm_smallk_kernel<C>, dim3((unsigned)grid), dim3(C::THREADS), 0, stream, d, tiles_m, tiles_n);
    return hipGetLastError();
}

// The 16-bit small-K path: 128x128 tiles, groups of ceil(tiles_n / 2) persistent workgroups (one
// per CU: its LDS admits one) that store runs of whole rows of C together
// (gemm_smallk_pipe_kernel).  Returns 1 if the groups do not fill the CUs well (more than an
// eighth of them would idle).
template <class C>
static int run_smallk_pipe_cfg(const GemmDesc& d, hipStream_t stream) {
    const int64_t tiles_m = (d.M + C::BM - 1) / C::BM;
    const int64_t tiles_n = (d.N + C::BN - 1) / C::BN;
    const int64_t rows = tiles_m * d.batch;
    if (rows * tiles_n > 0x7FFFFFFF) return TV_E_SHAPE;
    const int cus = device_cus();
    const int64_t P = (tiles_n + 1) / 2;
    if (P > cus || (cus % P) * 8 > cus) return 1;
    const int64_t ngroups = cus / P < rows ? cus / P : rows;
    const int grid = (int)(ngroups * P);
    if (d.dtype_c == TV_BFLOAT16)
        hipLaunchKernelGGL((gemm_smallk_pipe_kernel<C, __bf16>), dim3((unsigned)grid), dim3(C::THREADS), 0, stream, d, (int)tiles_m,
                           (int)tiles_n, (int)ngroups);
    else
        hipLaunchKernelGGL((gemm_smallk_pipe_kernel<C, _Float16>), dim3((unsigned)grid), dim3(C::THREADS), 0, stream, d, (int)tiles_m,
                           (int)tiles_n, (int)ngroups);
    return hipGetLastError();
}

static bool smallk_ok(const GemmDesc& d, int es, int bm_rows, int bn_rows) {
    const size_t csz = dtype_size(d.dtype_c);
    if (d.K > 2 * (128 / es) || csz != (size_t)es) return false;
    if (d.N % (16 / (int64_t)csz) != 0) return false;
    if (((int64_t)(d.M - 1) * d.sc_m + d.N) * (int64_t)csz >= ((int64_t)1 << 30)) return false;
    if (!(d.sc_n == 1 && (reinterpret_cast<uintptr_t>(d.C) % 16) == 0 && d.sc_m % (16 / (int64_t)csz) == 0 &&
          (d.batch <= 1 || d.sc_b % (16 / (int64_t)csz) == 0)))
        return false;
    const int64_t tiles = (int64_t)((d.M + bm_rows - 1) / bm_rows) * ((d.N + bn_rows - 1) / bn_rows) * d.batch;
    return tiles >= 1024;
}


// 16-bit / int8 inputs: direct-to-LDS kernel for the vector layouts, gemm_mfma_kernel otherwise.
template <typename T, int BM, int BN, int WMW, int WNW>
static int run_modes_dma(const GemmDesc& d, hipStream_t stream, int group_m, bool may_alloc) {
    const int es = (int)sizeof(T);
    const int am = pick_mode(d.A, d.M, d.K, d.sa_m, d.sa_k, d.sa_b, d.batch, es, BM, d.pad_a);
    const int bm = pick_mode(d.B, d.N, d.K, d.sb_n, d.sb_k, d.sb_b, d.batch, es, BN, d.pad_b);
    // The small-K kernel has no fused epilogue (its staging area holds the output type only).
    const bool epi = d.bias != nullptr || d.act != TV_ACT_NONE;
    if (!epi && am != LOAD_GENERIC && bm != LOAD_GENERIC && smallk_ok(d, es, BM, BN)) {
#define TV_CASE(A_, B_)                                                                                      \
    if (am == A_ && bm == B_) {                                                                              \
        if constexpr (sizeof(T) == 2) {                                                                      \
            const int rc = run_smallk_pipe_cfg<GemmCfg<T, 128, 128, 2, 4, A_, B_>>(d, stream);               \
            if (rc != 1) return rc;                                                                          \
        }                                                                                                    \
        return run_smallk_cfg<GemmCfg<T, BM, BN, WMW, WNW, A_, B_>>(d, stream);                              \
    }
        TV_CASE(LOAD_KCONTIG, LOAD_MNCONTIG)
        TV_CASE(LOAD_KCONTIG, LOAD_KCONTIG)
        TV_CASE(LOAD_MNCONTIG, LOAD_MNCONTIG)
        TV_CASE(LOAD_MNCONTIG, LOAD_KCONTIG)
#undef TV_CASE
    }
    // 16-bit and int8 GEMMs whose 128x128 tiles all fit one round of resident workgroups (two per
    // CU) run 128x128 tiles: few 256x256 tiles leave CUs idle.  Measured against 256x256 tiles (and their
    // stream-K schedule) on one box: bf16 [1024,4096]@[4096,4096] 45.5 against 62.7 us,
    // [128,8192]@[8192,8192] 43.5 against 79.3, [2048]^3 25.6 against 41.6, [2048,4096]@[4096,4096]
    // 67.4 against 78.6 (512 tiles of 128x128); but [3000,4096]@[4096,4096] (768 of them) 102.6
    // against 83.7.
    if constexpr (BM == 256 && BN == 256) {
        const int64_t tiles128 = (int64_t)((d.M + 127) / 128) * ((d.N + 127) / 128) * d.batch;
        if (am != LOAD_GENERIC && bm != LOAD_GENERIC && tiles128 <= 2 * (int64_t)device_cus()) {
#define TV_CASE(A_, B_) \
    if (am == A_ && bm == B_) return run_dma_cfg<GemmCfg<T, 128, 128, 2, 4, A_, B_>>(d, stream, group_m, may_alloc);
            TV_CASE(LOAD_KCONTIG, LOAD_MNCONTIG)
            TV_CASE(LOAD_KCONTIG, LOAD_KCONTIG)
            TV_CASE(LOAD_MNCONTIG, LOAD_MNCONTIG)
            TV_CASE(LOAD_MNCONTIG, LOAD_KCONTIG)
#undef TV_CASE
        }
    }
#define TV_CASE(A_, B_) \
    if (am == A_ && bm == B_) return run_dma_cfg<GemmCfg<T, BM, BN, WMW, WNW, A_, B_>>(d, stream, group_m, may_alloc);
    TV_CASE(LOAD_KCONTIG, LOAD_MNCONTIG)
    TV_CASE(LOAD_KCONTIG, LOAD_KCONTIG)
    TV_CASE(LOAD_MNCONTIG, LOAD_MNCONTIG)
    TV_CASE(LOAD_MNCONTIG, LOAD_KCONTIG)
#undef TV_CASE
    return run_modes<T, BM, BN, WMW, WNW>(d, stream, group_m, may_alloc);
}

} // namespace tvk
