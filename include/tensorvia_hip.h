/*
 * tensorvia_hip.h — C-ABI of the MI355X (gfx950) HIP matmul backend.
 *
 * This is the boundary between Tensorvia's C++ op layer and the hand-written HIP kernels.
 * It carries plain pointers, sizes and element strides only: no C++ types, no exceptions,
 * no tensor allocation.  Every entry point returns 0 on success, a positive hipError_t value
 * when the HIP runtime failed, or a negative TV_E_* code when the arguments were rejected.
 * Launch errors are read from the HIP runtime's last error of the calling thread, which each call
 * that launches work clears on entry: an error that earlier, unrelated HIP calls left there is
 * discarded, not reported as this call's.
 *
 * Reference interfaces replaced (paths into Aimol-l/Tensorvia):
 *   tv_hip_gemm   <- template<> struct MulImpl<Device::CUDA> { static Tensor execute(a, b); }
 *                    (include/backend/cuda/ops/mul.h:6-15, src/backend/cuda/mul.cu:52-124) and its
 *                    kernel launch mul_cuda_3d<<<...>>> (src/backend/cuda/mul.cu:8-48,77-91).
 *                    The descriptor also covers the view metadata that ops::Mul receives through
 *                    Tensor (Metadata, include/core/tensor.h:12-27) so strided and broadcast
 *                    operands are consumed without a repack.
 *   tv_hip_gemv   <- the batch*M*N < 2^20 "basic" branch of mul_kernel (src/backend/cpu/mul.cpp:7-25,
 *                    87-96) that decode-shaped calls (M <= 8) take; no CUDA counterpart exists.
 *   tv_hip_gemm_ex <- ops::Mul followed by ops::Add(C, bias) (src/ops.cpp:330-352,
 *                    src/backend/cpu/arithmetic.cpp:308-330) and ops::Relu / Silu / Sigmoid / Tanh
 *                    (src/backend/cpu/activate.cpp:8-40, src/backend/cuda/activate.cu:8-36), fused
 *                    into the matmul's epilogue; no single reference function does this.
 *   tv_hip_strerror <- the std::runtime_error texts the reference throws (src/ops.cpp:542-556,
 *                    include/backend/cuda/cuda_tensor.cpp:20-23).
 *   tv_hip_typecast <- TypecastImpl<Device::CUDA>::execute (src/backend/cuda/typecast.cu:7-27,29+),
 *                    restating the CPU cast (src/backend/cpu/typecast.cpp:48-98) over the pairs of
 *                    valid_casts (include/core/type_traits.h:237-260).
 *   tv_hip_fill     <- FillImpl / ZerosImpl / OnesImpl<Device::CUDA> (src/backend/cuda/initializer.cu:16-20,
 *                    39-98; CPU src/backend/cpu/initializer.cpp:14-17,39-66) behind ops::Fill/Zeros/Ones
 *                    (src/ops.cpp:85-138).
 *   tv_hip_random   <- RandomImpl<Device::CUDA> (src/backend/cuda/initializer.cu:22-37,99+; CPU
 *                    src/backend/cpu/initializer.cpp:18-36,69-77) behind ops::Random (src/ops.cpp:139-156),
 *                    with a seeded counter-based stream in place of the reference's clock-seeded
 *                    generators.
 *
 * Semantics (matching the reference CPU backend, src/backend/cpu/mul.cpp:97-145):
 *   C[b, m, n] = sum_k A[b, m, k] * B[b, k, n]
 *   - element (b, m, k) of A lives at  A + b*sa_b + m*sa_m + k*sa_k  (element units);
 *     sa_b == 0 broadcasts A over the batch, likewise sb_b for B (and a zero row or k stride
 *     repeats a row or column); the stride of a dimension of extent 1 is ignored;
 *   - strides along extents above 1 must not be negative, C's must not be zero (no two outputs in
 *     one element), and each operand's elements must lie within 2^56 bytes of its first element;
 *     other descriptors return TV_E_SHAPE;
 *   - int8 x int8: exact int32 accumulation; dtype_c INT8 stores the low byte of the exact sum
 *     (the reference's wrap-around result), dtype_c INT32 stores the full sum;
 *   - bf16/fp16 inputs: fp32 accumulation, output bf16/fp16 (GPU-backend convention) or FLOAT32
 *     (the CPU backend's widened result);
 *   - fp32: fp32 accumulation on the fp32 matrix cores;
 *   - any other dtype pair: exact restatement of the reference CPU accumulation rules on a
 *     SIMT kernel (slow path, provided for completeness).
 *
 * Calls are asynchronous on `hip_stream` (a hipStream_t, NULL = default stream).  The caller
 * keeps A, B and C alive until the stream has executed the work.  The split-K schedules keep their
 * partial sums, and large GEMMs their zero-padded copies of operands whose rows are not whole
 * 16-byte chunks, in a workspace per (device, stream): calls on one stream are ordered by that
 * stream, and calls on different streams use different workspaces, so concurrent streams are safe.
 * Growing a stream's workspace synchronises that stream once.  When the workspace cannot be
 * allocated (device memory exhausted), the call runs on kernels that need none (the unsplit GEMM,
 * the element-gather loader), more slowly, and still returns 0.
 */
#ifndef TENSORVIA_HIP_H
#define TENSORVIA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* via::DataType values (reference include/core/type_traits.h:123-132). */
enum tv_dtype {
    TV_INT8 = 0,
    TV_INT16 = 1,
    TV_INT32 = 2,
    TV_INT64 = 3,
    TV_BFLOAT16 = 4,
    TV_FLOAT16 = 5,
    TV_FLOAT32 = 6,
    TV_FLOAT64 = 7
};

/* Negative error codes; positive codes are hipError_t values. */
enum tv_status {
    TV_OK = 0,
    TV_E_NULL = -1,        /* a required pointer is NULL */
    TV_E_SHAPE = -2,       /* batch/M/N/K negative or above TV_MAX_EXTENT, a size overflows the kernels' index range, or a
                              stride is not allowed (see the semantics above) */
    TV_E_DTYPE = -3,       /* dtype value out of range or output dtype not allowed for the inputs */
    TV_E_UNSUPPORTED = -4, /* valid request that this entry point does not serve (e.g. gemv with M > 8) */
    TV_E_INJECTED = -5,    /* returned by the fault-injection hook (tests only) */
    TV_E_NOMEM = -6,       /* workspace allocation failed */
    TV_E_SCRATCH = -7      /* tv_hip_gemm_noalloc: the call needs more split-K scratch than the static buffer holds */
};

/* Largest batch, M, N or K the GEMM entry points accept: 2^31 - 2^20 - 1.  Tile, k-tile and slice
 * counts are 32-bit; the margin keeps their rounded-up sums in range.  Operands and outputs may
 * span up to 2^56 bytes: every address is formed in 64 bits. */
#define TV_MAX_EXTENT 2146435071

typedef struct tv_gemm_args {
    int32_t dtype_a, dtype_b, dtype_c; /* enum tv_dtype */
    int32_t flags;                     /* reserved, must be 0 */
    int64_t batch, M, N, K;
    const void* A; int64_t sa_b, sa_m, sa_k; /* element strides; A already includes the view offset */
    const void* B; int64_t sb_b, sb_k, sb_n; /* K.permute({0,2,1}) of a [b,n,k] tensor: sb_k = 1, sb_n = k */
    void*       C; int64_t sc_b, sc_m, sc_n;
} tv_gemm_args;

/* General batched matmul.  Routes M <= 8 shapes to the GEMV kernels when they serve the
 * dtype/layout, and 9 <= M <= 32 to the matrix-core GEMV (16-bit W up to 32 rows, int8 W up to 16,
 * whole 128-byte strips), everything else to the MFMA GEMM kernels (or the SIMT slow path). */
int tv_hip_gemm(const tv_gemm_args* args, void* hip_stream);

/* Activations of the fused epilogue (the reference's ops::Relu / Silu / Sigmoid / Tanh). */
enum tv_act {
    TV_ACT_NONE = 0,
    TV_ACT_RELU = 1,    /* x > 0 ? x : 0 */
    TV_ACT_SILU = 2,    /* x / (1 + exp(-x)) */
    TV_ACT_SIGMOID = 3, /* 1 / (1 + exp(-x)) */
    TV_ACT_TANH = 4     /* tanh(x) */
};

/* Fused epilogue: C[b, m, n] = act(sum_k A*B + bias[b, m, n]), computed on the fp32 accumulator and
 * rounded once to dtype_c.  Element (b, m, n) of the bias lives at bias + b*sbias_b + m*sbias_m +
 * n*sbias_n (element units, dtype = dtype_c); zero strides broadcast (sbias_b = sbias_m = 0,
 * sbias_n = 1 is a per-column bias vector).  bias = NULL adds nothing.  Strides are non-negative
 * and the bias elements read span at most 2^30 bytes (TV_E_SHAPE / TV_E_UNSUPPORTED otherwise).
 * silu and sigmoid use the hardware's approximate exp2 and reciprocal (a few ulp in fp32). */
typedef struct tv_epilogue {
    int32_t act;        /* enum tv_act */
    int32_t reserved;   /* must be 0 */
    const void* bias;
    int64_t sbias_b, sbias_m, sbias_n;
} tv_epilogue;

/* tv_hip_gemm with a fused epilogue (ep = NULL: same as tv_hip_gemm).  Served for the float-output
 * matrix-core pairs (fp32 -> fp32, bf16 -> bf16/fp32, fp16 -> fp16/fp32) with row-contiguous C
 * (sc_n = 1; any C layout when M <= 8); integer outputs, a column-strided C and an act outside
 * enum tv_act return TV_E_UNSUPPORTED. */
int tv_hip_gemm_ex(const tv_gemm_args* args, const tv_epilogue* ep, void* hip_stream);

/* tv_hip_gemm that allocates nothing.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments and routing as tv_hip_gemm.  The split-K partials of the
 * M <= 8 GEMV kernels come from a static device array of 4 MiB of partial slots plus 16,384 arrival
 * counters per GPU, held until the process ends, instead of tv_hip_gemm's workspace.  GEMMs
 * (M > 8) that tv_hip_gemm splits with its stream-K schedule, whose partial tiles need a
 * workspace, run unsplit here, so their fp32 and 16-bit results can differ from tv_hip_gemm's in
 * the last bits (summation order).  So can float calls with an operand whose rows are not whole
 * 16-byte chunks (e.g. bf16 W[4096,129]): tv_hip_gemm copies such an operand into padded rows (a
 * skinny call then runs on the matrix-core GEMV), while this entry point reads it in place with
 * the GEMM's element-gather loader, which sums K in another order.  Every other call, and every
 * int8 call, gives tv_hip_gemm's results bit for bit.  A call whose split needs more returns TV_E_SCRATCH at M <= 8 (e.g. M = 8
 * bf16 needs 2 KiB per (64-column strip, K-slice) pair: c5's x[8,4096] @ W[4096,11008] needs
 * 1.4 MiB); at 9 <= M <= 32 it runs the GEMM instead (e.g. M = 32 bf16 on c5's W needs 11 MiB of
 * partials), whose fp32 and 16-bit results can then differ from tv_hip_gemm's in the last bits.
 * The first call on a GPU looks the array up (hipGetSymbolAddress) and clears its counters with a
 * kernel on hip_stream.  All calls on one GPU share its array: calls that overlap on one GPU (on
 * different streams, or from different threads) race and must be serialised by the caller.  Under
 * graph capture, make a shape's first call outside the capture (it sets up the array and the
 * shape's launch plan); the captured calls then replay exactly. */
int tv_hip_gemm_noalloc(const tv_gemm_args* args, void* hip_stream);

/* Skinny-M (M <= 8) matrix-vector path, HBM-streaming.  W N-contiguous (x @ W, W[K, N] row-major):
 * matrix cores for bf16/fp16 W of 64 or more columns and int8 W of 128 or more columns at M >= 3,
 * packed dot products otherwise.  W K-contiguous (x @ W^T, W[N, K] row-major, K a multiple of the
 * 16-byte vector, rows 16-byte aligned): matrix cores for bf16, fp16 and int8.  Returns
 * TV_E_UNSUPPORTED for M > 8 or for a dtype pair or layout it does not serve (tv_hip_gemm serves
 * every layout). */
int tv_hip_gemv(const tv_gemm_args* args, void* hip_stream);

/* Strided -> contiguous copy of one tensor view on the device (ndim <= TV_MAX_DIMS).  Element
 * (i0, .., i{n-1}) of the view lives at src + sum_d i_d*strides[d] (element units, src already
 * includes the view offset); dst receives the elements in row-major order.
 * Replaces RepackImpl<Device::CUDA>::execute (reference src/backend/cuda/repack.cu:5-54), which
 * backs TensorImpl::clone_as_contiguous (include/core/tensor.h:38) for Tensor::contiguous() /
 * clone() of views (src/tensor.cpp:284-309). */
#define TV_MAX_DIMS 8
typedef struct tv_repack_args {
    int32_t ndim;
    int32_t elem_size;                 /* bytes per element: 1, 2, 4 or 8 */
    int64_t shape[TV_MAX_DIMS];
    int64_t strides[TV_MAX_DIMS];      /* element strides of the view */
    const void* src;
    void* dst;
} tv_repack_args;
int tv_hip_repack(const tv_repack_args* args, void* hip_stream);

/* Element-wise cast of n contiguous elements, dst[i] = static_cast<dst>(src[i]) with half types
 * going through their float value (round to nearest even into fp16/bf16, truncation toward zero
 * into integers).  Serves the pairs of the reference's valid_casts table and same-dtype copies;
 * any other pair returns TV_E_DTYPE. */
int tv_hip_typecast(const void* src, int32_t src_dtype, void* dst, int32_t dst_dtype, int64_t n, void* hip_stream);

/* dst[0..n) = static_cast<dtype>(value). */
int tv_hip_fill(void* dst, int32_t dtype, int64_t n, float value, void* hip_stream);

/* dst[0..n) = elements 0..n-1 of the seeded uniform stream: element i is SplitMix64 output
 * mix64(mix64(seed + G) + (i + 1) * G), G = 0x9E3779B97F4A7C15.  Integer dtypes take
 * lo + ((top 32 bits * (hi - lo + 1)) >> 32) in [lo, hi] = [(int64)min, (int64)max]; the others take
 * min + (max - min) * u in fp32 (no fused multiply-add), u = top 24 bits / 2^24, rounded to the
 * dtype.  Bit-identical to the host generator for the same (seed, dtype, min, max).  min > max
 * returns TV_E_SHAPE. */
int tv_hip_random(void* dst, int32_t dtype, int64_t n, float min, float max, uint64_t seed, void* hip_stream);

/* Human-readable text for any return code of this library. */
const char* tv_hip_strerror(int code);

/* ABI version of this header (bumped on any change of tv_gemm_args or the entry points). */
int tv_hip_abi_version(void);

/* Test hook: the next `count` calls of any compute entry point return `code` without touching
 * the device.  Lets host code prove error propagation without a GPU.  count = 0 disarms. */
void tv_hip_inject_fault(int code, int count);

/* Test hook: the next `count` requests for the library's per-stream workspace (split-K slots,
 * padded operand copies) allocate, asking the HIP runtime for more memory than any device has, so
 * they fail as they would when device memory is exhausted, and the calls take their no-workspace
 * paths.  count = 0 disarms. */
void tv_hip_inject_alloc_failure(int count);

#define TV_HIP_ABI_VERSION 6

#ifdef __cplusplus
}
#endif

#endif /* TENSORVIA_HIP_H */
