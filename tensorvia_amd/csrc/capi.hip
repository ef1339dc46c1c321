// extern "C" entry points of libtv_hip.so: argument validation and kernel routing.
// The argument checks restate the ones ops::Mul performs before dispatch (reference
// src/ops.cpp:540-556) at the level of a strided descriptor.
#include <atomic>

#include "tv_kernels.h"

namespace {

std::atomic<int> g_fault_code{0};
std::atomic<int> g_fault_count{0};

// Entry of every C-ABI call that launches work.  A launch's error is read back from the HIP
// runtime's last error after the launch, so a failure that earlier, unrelated HIP calls of this
// thread left there (and nobody read) is cleared first: the call's return code then reports its
// own launches only.  Then the test hook: *code is set and true returned while injected faults
// remain.
bool enter_call(int* code) {
    (void)hipGetLastError();
    int n = g_fault_count.load();
    while (n > 0) {
        if (g_fault_count.compare_exchange_weak(n, n - 1)) {
            *code = g_fault_code.load();
            return true;
        }
    }
    return false;
}

// Output dtypes each input pair may produce.  For the matrix-core dtypes the GPU-backend result
// type (compute_type(a, b), reference include/core/type_traits.h:270-287) and the widened CPU
// backend result (src/backend/cpu/mul.cpp:110-112) are both served; other pairs produce exactly
// the CPU backend's result type.
int cpu_result_type(int a, int b) {
    // CPU widens fp16/bf16 to fp32 first (mul.cpp:110-111), then applies compute_type.
    if (a == TV_FLOAT16 || a == TV_BFLOAT16) a = TV_FLOAT32;
    if (b == TV_FLOAT16 || b == TV_BFLOAT16) b = TV_FLOAT32;
    if (a == b) return a;
    const bool ai = a <= TV_INT64, bi = b <= TV_INT64;
    if (ai && bi) return a > b ? a : b;
    if (!ai && !bi) {
        int m = a > b ? a : b;
        return m < TV_FLOAT32 ? TV_FLOAT32 : m;
    }
    if (a == TV_INT64 || b == TV_INT64) return TV_FLOAT64;
    int m = a > b ? a : b;
    return m < TV_FLOAT32 ? TV_FLOAT32 : m;
}

bool mfma_pair(const tv_gemm_args* a) {
    if (a->dtype_a != a->dtype_b) return false;
    switch (a->dtype_a) {
        case TV_FLOAT32: return a->dtype_c == TV_FLOAT32;
        case TV_BFLOAT16: return a->dtype_c == TV_BFLOAT16 || a->dtype_c == TV_FLOAT32;
        case TV_FLOAT16: return a->dtype_c == TV_FLOAT16 || a->dtype_c == TV_FLOAT32;
        case TV_INT8: return a->dtype_c == TV_INT8 || a->dtype_c == TV_INT32;
        default: return false;
    }
}

// Bytes from a strided operand's first element to its last: (extent - 1) * stride summed over its
// three dimensions, times the element size.  A dimension of extent 0 or 1 never steps, so its
// stride counts nothing.  -1 when a stride along an extent above 1 is negative.
__int128 span_bytes(const int64_t (&ext)[3], const int64_t (&str)[3], size_t es) {
    __int128 span = 0;
    for (int i = 0; i < 3; ++i) {
        if (ext[i] <= 1) continue;
        if (str[i] < 0) return -1;
        span += (__int128)(ext[i] - 1) * str[i];
    }
    return span * (__int128)es;
}

// Largest span accepted: 2^56 bytes, above any device's memory, so that every address a kernel
// forms (base + offsets, in 64 bits) stays in range.
constexpr __int128 kMaxSpan = (__int128)1 << 56;

int validate(const tv_gemm_args* a, tvk::GemmDesc* d) {
    if (!a) return TV_E_NULL;
    if (a->flags != 0) return TV_E_UNSUPPORTED;
    for (int dt : {a->dtype_a, a->dtype_b, a->dtype_c})
        if (dt < TV_INT8 || dt > TV_FLOAT64) return TV_E_DTYPE;
    if (a->batch < 0 || a->M < 0 || a->N < 0 || a->K < 0) return TV_E_SHAPE;
    // The launchers count tiles, k-tiles and K slices in 32-bit arithmetic from these sizes (tile
    // rows rounded up, the k offset two k-tiles ahead of the last one): staying 2^20 below INT32_MAX
    // keeps every such sum in range.
    const int64_t lim = TV_MAX_EXTENT;
    if (a->batch > lim || a->M > lim || a->N > lim || a->K > lim) return TV_E_SHAPE;
    if (!mfma_pair(a) && a->dtype_c != cpu_result_type(a->dtype_a, a->dtype_b)) return TV_E_DTYPE;
    const bool empty = a->batch == 0 || a->M == 0 || a->N == 0;
    if (!empty) {
        // Strides along extents above 1: not negative (the loaders and stores add 32-bit offsets
        // to a row's or tile's base), and C's not zero either (two outputs in one element).  A and
        // B are not read when K = 0.
        const __int128 sa = span_bytes({a->batch, a->M, a->K}, {a->sa_b, a->sa_m, a->sa_k}, tvk::dtype_size(a->dtype_a));
        const __int128 sb = span_bytes({a->batch, a->K, a->N}, {a->sb_b, a->sb_k, a->sb_n}, tvk::dtype_size(a->dtype_b));
        const __int128 sc = span_bytes({a->batch, a->M, a->N}, {a->sc_b, a->sc_m, a->sc_n}, tvk::dtype_size(a->dtype_c));
        if ((a->K > 0 && (sa < 0 || sa >= kMaxSpan || sb < 0 || sb >= kMaxSpan)) || sc < 0 || sc >= kMaxSpan)
            return TV_E_SHAPE;
        if ((a->batch > 1 && a->sc_b == 0) || (a->M > 1 && a->sc_m == 0) || (a->N > 1 && a->sc_n == 0)) return TV_E_SHAPE;
        if (!a->C) return TV_E_NULL;
        if (a->K > 0 && (!a->A || !a->B)) return TV_E_NULL;
    }
    d->A = a->A; d->B = a->B; d->C = a->C;
    d->sa_b = a->sa_b; d->sa_m = a->sa_m; d->sa_k = a->sa_k;
    d->sb_b = a->sb_b; d->sb_k = a->sb_k; d->sb_n = a->sb_n;
    d->sc_b = a->sc_b; d->sc_m = a->sc_m; d->sc_n = a->sc_n;
    d->M = (int32_t)a->M; d->N = (int32_t)a->N; d->K = (int32_t)a->K; d->batch = (int32_t)a->batch;
    d->dtype_a = a->dtype_a; d->dtype_b = a->dtype_b; d->dtype_c = a->dtype_c;
    d->bias = nullptr;
    d->sbias_b = d->sbias_m = d->sbias_n = 0;
    d->bias_bytes = 0;
    d->act = TV_ACT_NONE;
    return TV_OK;
}

// Routing shared by tv_hip_gemm, tv_hip_gemm_ex and tv_hip_gemm_noalloc (fixed: the GEMV's
// split-K buffers, nullptr for the per-stream workspace; with fixed buffers the GEMM takes no
// schedule that needs a workspace either).
int run_gemm(const tv_gemm_args* args, const tvk::GemmDesc& d0, hipStream_t s, const tvk::GemvScratch* fixed = nullptr) {
    if (d0.batch == 0 || d0.M == 0 || d0.N == 0) return TV_OK;
    if (mfma_pair(args) && d0.K == 0) return tvk::launch_gemm_k0(d0, s);
    tvk::GemmDesc d = d0;
    if (mfma_pair(args) && fixed == nullptr) { // misaligned operands into padded rows (workspace)
        const int rc = tvk::pad_gemm_operands(d, s);
        if (rc) return rc;
    }
    if (mfma_pair(args)) {
        // Skinny M: the GEMV streams W once (M <= 8 always; 9 <= M <= 32 on the matrix-core GEMV,
        // which the tiled GEMM is about 1.7x slower than there).  Where it declines the call, or
        // the caller's fixed split-K buffers are too small above M = 8, the GEMM serves it.
        if (d.M <= 32) {
            const int rc = tvk::launch_gemv(d, s, fixed);
            // No room for the split-K slots (TV_E_NOMEM): the GEMM needs none in its plain form.
            if (rc != TV_E_UNSUPPORTED && rc != TV_E_NOMEM && !(rc == TV_E_SCRATCH && d.M > 8)) return rc;
        }
        return tvk::launch_gemm_mfma(d, s, fixed == nullptr);
    }
    return tvk::launch_gemm_simt(d, s);
}

} // namespace

extern "C" {

int tv_hip_abi_version(void) { return TV_HIP_ABI_VERSION; }

void tv_hip_inject_fault(int code, int count) {
    g_fault_code.store(code);
    g_fault_count.store(count < 0 ? 0 : count);
}

void tv_hip_inject_alloc_failure(int count) { tvk::inject_alloc_failure(count); }

int tv_hip_gemm(const tv_gemm_args* args, void* hip_stream) {
    int code;
    if (enter_call(&code)) return code;
    tvk::GemmDesc d;
    int rc = validate(args, &d);
    if (rc) return rc;
    return run_gemm(args, d, static_cast<hipStream_t>(hip_stream));
}

int tv_hip_gemm_noalloc(const tv_gemm_args* args, void* hip_stream) {
    int code;
    if (enter_call(&code)) return code;
    tvk::GemmDesc d;
    int rc = validate(args, &d);
    if (rc) return rc;
    hipStream_t s = static_cast<hipStream_t>(hip_stream);
    tvk::GemvScratch sc;
    rc = tvk::gemv_static_scratch(s, &sc);
    if (rc) return rc;
    return run_gemm(args, d, s, &sc);
}

int tv_hip_gemm_ex(const tv_gemm_args* args, const tv_epilogue* ep, void* hip_stream) {
    int code;
    if (enter_call(&code)) return code;
    tvk::GemmDesc d;
    int rc = validate(args, &d);
    if (rc) return rc;
    if (ep) {
        if (ep->act < TV_ACT_NONE || ep->act > TV_ACT_TANH || ep->reserved != 0) return TV_E_UNSUPPORTED;
        const bool float_out = args->dtype_c == TV_FLOAT32 || args->dtype_c == TV_BFLOAT16 || args->dtype_c == TV_FLOAT16;
        if (!mfma_pair(args) || !float_out) return TV_E_UNSUPPORTED;
        if (ep->bias) {
            if (ep->sbias_b < 0 || ep->sbias_m < 0 || ep->sbias_n < 0) return TV_E_SHAPE;
            // Extent of the elements read, in bytes: every offset stays below 2^30 (one buffer
            // resource, 32-bit offsets).
            const size_t es = tvk::dtype_size(args->dtype_c);
            const __int128 span = span_bytes({d.batch, d.M, d.N}, {ep->sbias_b, ep->sbias_m, ep->sbias_n}, es);
            if (span + (__int128)es > ((__int128)1 << 30)) return TV_E_UNSUPPORTED;
            const int64_t bytes = (int64_t)span + (int64_t)es;
            d.bias = ep->bias;
            d.sbias_b = ep->sbias_b;
            d.sbias_m = ep->sbias_m;
            d.sbias_n = ep->sbias_n;
            d.bias_bytes = bytes;
        }
        d.act = ep->act;
    }
    return run_gemm(args, d, static_cast<hipStream_t>(hip_stream));
}

int tv_hip_gemv(const tv_gemm_args* args, void* hip_stream) {
    int code;
    if (enter_call(&code)) return code;
    tvk::GemmDesc d;
    int rc = validate(args, &d);
    if (rc) return rc;
    if (d.M > 8) return TV_E_UNSUPPORTED;
    if (!mfma_pair(args)) return TV_E_UNSUPPORTED;
    if (d.batch == 0 || d.M == 0 || d.N == 0) return TV_OK;
    if (d.K == 0) return tvk::launch_gemm_k0(d, static_cast<hipStream_t>(hip_stream));
    return tvk::launch_gemv(d, static_cast<hipStream_t>(hip_stream));
}

int tv_hip_repack(const tv_repack_args* args, void* hip_stream) {
    int code;
    if (enter_call(&code)) return code;
    if (!args) return TV_E_NULL;
    if (args->ndim < 0 || args->ndim > TV_MAX_DIMS) return TV_E_SHAPE;
    if (args->elem_size != 1 && args->elem_size != 2 && args->elem_size != 4 && args->elem_size != 8) return TV_E_DTYPE;
    for (int d = 0; d < args->ndim; ++d)
        if (args->shape[d] < 0) return TV_E_SHAPE;
    for (int d = 0; d < args->ndim; ++d)
        if (args->shape[d] == 0) return TV_OK; // empty view
    int64_t n = 1; // element count: must fit in 64 bits
    for (int d = 0; d < args->ndim; ++d)
        if (__builtin_mul_overflow(n, args->shape[d], &n)) return TV_E_SHAPE;
    if (!args->src || !args->dst) return TV_E_NULL;
    return tvk::launch_repack(args, static_cast<hipStream_t>(hip_stream));
}

int tv_hip_typecast(const void* src, int32_t src_dtype, void* dst, int32_t dst_dtype, int64_t n, void* hip_stream) {
    int code;
    if (enter_call(&code)) return code;
    if (src_dtype < TV_INT8 || src_dtype > TV_FLOAT64 || dst_dtype < TV_INT8 || dst_dtype > TV_FLOAT64) return TV_E_DTYPE;
    if (n < 0) return TV_E_SHAPE;
    if (n == 0) return TV_OK;
    if (!src || !dst) return TV_E_NULL;
    hipStream_t s = static_cast<hipStream_t>(hip_stream);
    if (src_dtype == dst_dtype)
        return hipMemcpyAsync(dst, src, (size_t)n * tvk::dtype_size(src_dtype), hipMemcpyDeviceToDevice, s);
    return tvk::launch_typecast(src, src_dtype, dst, dst_dtype, n, s);
}

int tv_hip_fill(void* dst, int32_t dtype, int64_t n, float value, void* hip_stream) {
    int code;
    if (enter_call(&code)) return code;
    if (dtype < TV_INT8 || dtype > TV_FLOAT64) return TV_E_DTYPE;
    if (n < 0) return TV_E_SHAPE;
    if (n == 0) return TV_OK;
    if (!dst) return TV_E_NULL;
    return tvk::launch_fill(dst, dtype, n, value, static_cast<hipStream_t>(hip_stream));
}

int tv_hip_random(void* dst, int32_t dtype, int64_t n, float min, float max, uint64_t seed, void* hip_stream) {
    int code;
    if (enter_call(&code)) return code;
    if (dtype < TV_INT8 || dtype > TV_FLOAT64) return TV_E_DTYPE;
    if (n < 0 || !(min <= max)) return TV_E_SHAPE;
    if (n == 0) return TV_OK;
    if (!dst) return TV_E_NULL;
    return tvk::launch_random(dst, dtype, n, min, max, seed, static_cast<hipStream_t>(hip_stream));
}

const char* tv_hip_strerror(int code) {
    switch (code) {
        case TV_OK: return "success";
        case TV_E_NULL: return "tensorvia-hip: a required pointer is NULL";
        case TV_E_SHAPE: return "tensorvia-hip: invalid or too large batch/M/N/K";
        case TV_E_DTYPE: return "tensorvia-hip: dtype out of range or output dtype not allowed for the input dtypes";
        case TV_E_UNSUPPORTED: return "tensorvia-hip: request not served by this entry point";
        case TV_E_INJECTED: return "tensorvia-hip: injected fault";
        case TV_E_NOMEM: return "tensorvia-hip: workspace allocation failed";
        case TV_E_SCRATCH:
            return "tensorvia-hip: the call needs more split-K scratch than tv_hip_gemm_noalloc's static buffer "
                   "holds (4 MiB of partial slots, 16384 counters); use tv_hip_gemm";
        default: break;
    }
    if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
    return "tensorvia-hip: unknown error";
}

} // extern "C"
