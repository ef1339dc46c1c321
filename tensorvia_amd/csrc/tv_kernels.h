// Shared declarations of the gfx950 matmul kernels (device side and launchers).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "tensorvia_hip.h"

namespace tvk {

// 16-byte vector types used for global loads, LDS traffic and MFMA operands.
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 f16x2;
typedef __attribute__((__vector_size__(4 * sizeof(unsigned)))) unsigned u32x4;

// Global stores with the streaming write policy (nt sc1) for output tiles that are written once.
// Used only where every wave instruction writes whole 128-byte lines (rows of a staged tile): there
// the policy saves the L2 the output's lines (c3 bf16 epilogue -3 %, c4 -6 %); on stores that
// cover half lines per instruction it is several times slower than a plain store.
// A store of more than 8 bytes reads its data VGPRs after it issues: a VALU write to them needs 2
// wait states first (gfx950; the compiler puts `s_nop 1` after its own such stores).  The compiler
// cannot see inside the asm, and with no wait it was measured to schedule the next chunk's address
// computation into v[0] of the data right behind the store: the store then wrote that value
// instead of element 0, now and then.  The `s_nop 1` is part of the asm for that reason.
__device__ inline void store_stream16(void* p, u32x4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1 nt\n\ts_nop 1" ::"v"(p), "v"(v) : "memory");
}
__device__ inline void store_stream8(void* p, uint2 v) {
    asm volatile("global_store_dwordx2 %0, %1, off sc1 nt" ::"v"(p), "v"(v) : "memory");
}

// Descriptor the launchers receive: tv_gemm_args after validation, with sizes narrowed to the
// ranges the kernels index with.
struct GemmDesc {
    const void* A;
    const void* B;
    void* C;
    int64_t sa_b, sa_m, sa_k;
    int64_t sb_b, sb_k, sb_n;
    int64_t sc_b, sc_m, sc_n;
    int32_t M, N, K, batch;
    int32_t dtype_a, dtype_b, dtype_c;
    // Fused epilogue (float outputs): C = act(acc + bias[b, m, n]) on the fp32 accumulator, rounded
    // once to dtype_c.  bias == nullptr: no bias; act == TV_ACT_NONE: identity.
    // Defaults: no epilogue, so a descriptor filled field by field without them is a plain matmul.
    const void* bias = nullptr;                    // element type dtype_c
    int64_t sbias_b = 0, sbias_m = 0, sbias_n = 0; // element strides (0 broadcasts), non-negative
    int64_t bias_bytes = 0;                        // extent of the bias read (below 2^30)
    int32_t act = TV_ACT_NONE;
    // 1: the operand is a copy made by pad_gemm_operands whose rows are whole 16-byte chunks, zero
    // past the valid extent, so a chunk that straddles the end of the valid extent may be read.
    int32_t pad_a = 0, pad_b = 0;
};

__device__ inline bool has_epilogue(const GemmDesc& d) { return d.bias != nullptr || d.act != TV_ACT_NONE; }

// The reference's activations on float values (src/backend/cpu/activate.cpp:8-40,
// src/backend/cuda/activate.cu:8-36): relu x > 0 ? x : 0, silu x / (1 + exp(-x)),
// sigmoid 1 / (1 + exp(-x)), tanh(x).  The three logistic ones are one formula,
// (a*x + c) * s + e with s = 1 / (1 + 2^(l*x)) and l = -g * log2(e):
//   silu    a = 1, c = 0, e = 0,  g = 1
//   sigmoid a = 0, c = 1, e = 0,  g = 1
//   tanh    a = 0, c = 2, e = -1, g = 2      (tanh x = 2 / (1 + exp(-2x)) - 1)
// evaluated with the hardware's exp2 and reciprocal (v_exp_f32, v_rcp_f32, about 1 ulp each):
// a few ulp relative for silu / sigmoid, about 1e-7 absolute for tanh near 0.  (__fdividef and
// the / operator compile to the full IEEE division sequence here, about 11 instructions per value,
// which made the activation the largest part of a fused epilogue.)
struct ActCoef {
    float a, c, e, l;
};
__host__ __device__ inline ActCoef act_coef(int act) {
    constexpr float kLog2e = 1.4426950408889634f;
    if (act == TV_ACT_SIGMOID) return ActCoef{0.0f, 1.0f, 0.0f, -kLog2e};
    if (act == TV_ACT_TANH) return ActCoef{0.0f, 2.0f, -1.0f, -2.0f * kLog2e};
    return ActCoef{1.0f, 0.0f, 0.0f, -kLog2e}; // silu
}
__device__ inline float act_logistic(float x, const ActCoef& k) {
    // 2^(l*x) overflows to +inf for large -x: s = rcp(inf) = 0, the limit.
    const float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(k.l * x));
    // sigmoid and tanh have a = 0: the a*x term is left out rather than multiplied, since 0 * inf
    // would turn their limits at x = +-inf (1 and 0, +-1) into NaN.
    const float ax = k.a != 0.0f ? k.a * x : 0.0f;
    return (ax + k.c) * s + k.e;
}
__device__ inline float act_simple(float x, int act) { return act == TV_ACT_RELU ? (x > 0.0f ? x : 0.0f) : x; }
__device__ inline float act_apply(float x, int act) {
    if (act == TV_ACT_SILU || act == TV_ACT_SIGMOID || act == TV_ACT_TANH) return act_logistic(x, act_coef(act));
    return act_simple(x, act);
}

__device__ inline float bias_at(const GemmDesc& d, int64_t b, int64_t m, int64_t n) {
    const int64_t i = b * d.sbias_b + m * d.sbias_m + n * d.sbias_n;
    if (d.dtype_c == TV_BFLOAT16) return (float)static_cast<const __bf16*>(d.bias)[i];
    if (d.dtype_c == TV_FLOAT16) return (float)static_cast<const _Float16*>(d.bias)[i];
    return static_cast<const float*>(d.bias)[i];
}

// One output value through the epilogue (m, n inside C).
__device__ inline float epilogue_value(float v, const GemmDesc& d, int64_t b, int64_t m, int64_t n) {
    if (d.bias) v += bias_at(d, b, m, n);
    return act_apply(v, d.act);
}

// Split-K hand-over between the workgroups that share one output block (a GEMV strip, a GEMM tile
// split by the stream-K schedule).  Called by every thread after its partial-slot stores, which
// carry the agent-scope cache policy (sc1: written through the XCD's L2 to the agent's coherence
// point, never left dirty in an L2; the GEMV's agent-scope atomic stores compile to such stores, the
// GEMM issues 16-byte buffer stores with the same bit).
//  * Each wave waits until its own slot stores are acknowledged (s_waitcnt vmcnt(0); for a store
//    the count drops when the write is complete at the scope it was issued with).  The asm's
//    memory clobber keeps the compiler from moving the stores below the wait.
//  * After the barrier every slot store of the workgroup is complete; thread 0 then counts the
//    workgroup in with an agent-scope atomic add, so a count that completes the block is taken
//    after every publisher's stores are complete.
//  * The combining workgroup reads the slots with sc1 loads, which are served from the coherence
//    point, issued after the count returned (through the barrier).
// This is the ordering-only release that rocPRIM's look-back scan uses on this architecture for
// data published through agent-scope atomics: a C++ release/acquire fence pair at agent scope
// also writes back and invalidates the XCD's whole L2 (buffer_wbl2 sc1, buffer_inv sc1) once per
// wave, which measured 104 us on c5 (x[1,4096] @ W[4096,11008] bf16) against 18.5 us with this
// hand-over; there is no dirty non-atomic data here for those to write back.
// *last is 1 in the workgroup that must combine the slots.  Every slot access and the count's reset
// go through the slot_* helpers below, which carry that policy.
__device__ inline void publish_and_count(int* cnt, int nslices, int* last) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) *last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nslices - 1;
    __syncthreads();
}

// Partial-slot stores and loads of the hand-over above: scalar slots as agent-scope relaxed
// atomics, 16-byte slots through a buffer resource with the sc1 cache-policy bit (16).
constexpr int kSlotPolicy = 16;
template <typename T> __device__ inline void slot_store(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T> __device__ inline T slot_load(const T* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename V> __device__ inline void slot_store16(__amdgpu_buffer_rsrc_t r, int off, V v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), r, off, 0, kSlotPolicy);
}
template <typename V> __device__ inline V slot_load16(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSlotPolicy));
}
// The combining workgroup leaves the block's count at zero for the next launch.
__device__ inline void slot_count_reset(int* cnt) {
    if (threadIdx.x == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Operand load modes for one GEMM operand (A: rows m, B: rows n; "K-contiguous" means the
// reduction index has stride 1).
enum LoadMode : int {
    LOAD_KCONTIG = 0,  // stride 1 along k, 16-byte aligned rows: 16B vector loads
    LOAD_MNCONTIG = 1, // stride 1 along m (A) / n (B), 16-byte aligned: 16B loads + register transpose
    LOAD_GENERIC = 2   // anything else: element gathers
};

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Mode for one operand.  `rows` extent R, strides s_r (along rows), s_k (along k), s_b (batch).
// The vector modes also need every per-lane offset inside one k-tile panel to fit in 31 bits.
// padded: a zero-padded copy (GemmDesc::pad_a / pad_b), whose valid extent need not be whole chunks.
inline int pick_mode(const void* p, int64_t R, int64_t K, int64_t s_r, int64_t s_k, int64_t s_b, int64_t batch, int es,
                     int rows_tile, bool padded) {
    const int64_t vec = 16 / es;
    const int64_t bk = 128 / es;
    const bool ok_ptr = aligned16(p);
    const bool ok_b = batch <= 1 || s_b % vec == 0;
    const int64_t lim = (int64_t)1 << 30;
    // Tails are masked by the buffer range check, which needs rows (k rows) that do not overlap;
    // a chunk past the valid extent would read the next row, unless that tail is zero padding.
    if (s_k == 1 && ok_ptr && ok_b && (padded || K % vec == 0) && (R <= 1 || (s_r % vec == 0 && s_r >= K)) &&
        ((int64_t)rows_tile * s_r + bk) * es < lim)
        return LOAD_KCONTIG;
    if (s_r == 1 && ok_ptr && ok_b && (padded || R % vec == 0) && (K <= 1 || (s_k % vec == 0 && s_k >= R)) &&
        (bk * s_k + rows_tile) * es < lim)
        return LOAD_MNCONTIG;
    return LOAD_GENERIC;
}

// Launchers (return hipError_t, or a negative TV_E_* code).
// may_alloc = false: no launch path that needs a grown workspace (the stream-K schedule of the fp32
// kernel); the plain data-parallel kernels serve the call.
int launch_gemm_mfma(const GemmDesc& d, hipStream_t stream, bool may_alloc = true);
// Copies operands that are contiguous along one dimension but not in whole 16-byte rows into
// zero-padded rows in the per-stream workspace (calls of at least 2^20 multiply-adds or K >= 256) and points d
// at the copies (pad_a / pad_b).  0 with d unchanged when nothing needs or gets a copy.
int pad_gemm_operands(GemmDesc& d, hipStream_t stream);
// The next `count` workspace allocations fail (tv_hip_inject_alloc_failure).
void inject_alloc_failure(int count);
// Per-(device, stream) buffers of the stream-K GEMM schedule: `cnt_ints` arrival counters (zero
// between launches) and `slot_bytes` of partial-accumulator slots.
int gemm_sk_workspace(hipStream_t stream, size_t cnt_ints, size_t slot_bytes, int** cnt, char** slots);
int launch_gemm_simt(const GemmDesc& d, hipStream_t stream);
int launch_gemm_k0(const GemmDesc& d, hipStream_t stream); // K = 0: C = epilogue(0)
int launch_repack(const tv_repack_args* a, hipStream_t stream);
int launch_typecast(const void* src, int src_dt, void* dst, int dst_dt, int64_t n, hipStream_t stream);
int launch_fill(void* dst, int dt, int64_t n, float value, hipStream_t stream);
int launch_random(void* dst, int dt, int64_t n, float min, float max, uint64_t seed, hipStream_t stream);
// Split-K buffers supplied by the caller instead of the per-stream workspace: cnt_ints arrival
// counters (zero between launches) and part_bytes of partial slots.
struct GemvScratch {
    int* cnt;
    size_t cnt_ints;
    void* part;
    size_t part_bytes;
};
// TV_E_UNSUPPORTED if it does not serve d.  fixed = nullptr: the split-K partials live in a
// per-(device, stream) workspace that grows by hipMalloc; otherwise in *fixed (TV_E_SCRATCH when
// they do not fit).
int launch_gemv(const GemmDesc& d, hipStream_t stream, const GemvScratch* fixed = nullptr);
// The static split-K scratch of the current device (set up on its first use: its address is looked
// up and its counters cleared on `stream`).
int gemv_static_scratch(hipStream_t stream, GemvScratch* out);
// Zero-padded row copy of a GEMM operand: nb batches (source stride s_batch) of `rows` rows (source
// stride s_row) of L contiguous elements of `es` bytes, written densely as rows of P elements (P a
// multiple of 16 bytes), zero in [L, P).
int launch_pad_rows(const void* src, void* dst, int es, int64_t nb, int64_t rows, int64_t s_row, int64_t s_batch,
                    int64_t L, int64_t P, hipStream_t stream);
// Per-(device, stream) buffer for the padded copy of operand A (operand 0) or B (operand 1).
int gemm_pad_workspace(hipStream_t stream, size_t bytes, int operand, void** out);

// A value computed once per device by host code (a resident-workgroup grid, a CU count), 0 while it
// is not known.  Relaxed atomic loads and stores: host threads making their first calls at the same
// time may each compute it, and each stores the same value.  Returns 0 if the device cannot be
// named or compute() fails (returns 0 or less).
constexpr int kMaxDevices = 64;
template <class F> inline int cached_per_device(std::atomic<int> (&slot)[kMaxDevices], F&& compute) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
    int v = slot[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    v = compute(dev);
    if (v <= 0) return 0;
    slot[dev].store(v, std::memory_order_relaxed);
    return v;
}

// Compute units of the current device (cached per device; 256 if the runtime cannot tell).
inline int device_cus() {
    static std::atomic<int> cached[kMaxDevices];
    const int v = cached_per_device(cached, [](int dev) {
        int cus = 0;
        return hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0 ? cus : 0;
    });
    return v > 0 ? v : 256;
}

// Buffer loads: a lane offset at or above 2^31 is outside every buffer resource built by make_rsrc
// (num_records <= 2^30), also after a stride multiple below 2^30 is added to it, and such a load
// returns zeros.
constexpr unsigned kOOB = 0x80000000u;

__device__ inline u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
// Streaming variant (nontemporal: the lines are not kept in the caches for reuse).
__device__ inline u32x4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2));
}
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const char* base, int64_t bytes) {
    const int nr = bytes <= 0 ? 0 : (bytes > 0x40000000 ? 0x40000000 : (int)bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, nr, 0x00020000);
}

// Bias element `idx` as float: fp32 storage, or 16-bit storage (bf16 when bf, else fp16); idx = kOOB
// reads zero.
__device__ inline float bias_load32(__amdgpu_buffer_rsrc_t r, unsigned idx) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)(idx == kOOB ? kOOB : idx * 4), 0, 0));
}
__device__ inline float bias_load16(__amdgpu_buffer_rsrc_t r, unsigned idx, bool bf) {
    const unsigned short h = __builtin_amdgcn_raw_buffer_load_b16(r, (int)(idx == kOOB ? kOOB : idx * 2), 0, 0);
    return bf ? (float)__builtin_bit_cast(__bf16, h) : (float)__builtin_bit_cast(_Float16, h);
}

__host__ __device__ inline size_t dtype_size(int dt) {
    switch (dt) {
        case TV_INT8: return 1;
        case TV_INT16: return 2;
        case TV_INT32: return 4;
        case TV_INT64: return 8;
        case TV_BFLOAT16: return 2;
        case TV_FLOAT16: return 2;
        case TV_FLOAT32: return 4;
        case TV_FLOAT64: return 8;
        default: return 0;
    }
}

} // namespace tvk
