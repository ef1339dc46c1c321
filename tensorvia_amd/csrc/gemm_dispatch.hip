// Routes a validated descriptor to the MFMA GEMM instantiation of its input dtype.
#include "tv_kernels.h"

namespace tvk {
int launch_gemm_mfma_f32(const GemmDesc& d, hipStream_t stream, bool may_alloc);
int launch_gemm_mfma_bf16(const GemmDesc& d, hipStream_t stream, bool may_alloc);
int launch_gemm_mfma_f16(const GemmDesc& d, hipStream_t stream, bool may_alloc);
int launch_gemm_mfma_i8(const GemmDesc& d, hipStream_t stream, bool may_alloc);

// An operand contiguous along one dimension whose rows are not whole 16-byte chunks (row length,
// pitch, batch stride or base address) would be read by the element-gather loader, one load per
// element: bf16 [2048,4096] @ [4096,4100] took 1.18 ms that way, against about 0.1 ms on the
// vector loaders.  With a workspace, such an operand is copied once into rows of whole chunks, zero
// past its valid extent (pad_a / pad_b tell the load-mode choice, and the matrix-core GEMV, that
// the tail may be read), and the call runs on the copy.  Small calls keep the gather.
static int pad_operand(GemmDesc& d, bool is_a, hipStream_t stream) {
    const int es = (int)dtype_size(is_a ? d.dtype_a : d.dtype_b);
    if (es != 1 && es != 2 && es != 4) return 0;
    const int64_t vec = 16 / es;
    const void* p = is_a ? d.A : d.B;
    const int64_t R = is_a ? d.M : d.N, K = d.K;
    const int64_t s_r = is_a ? d.sa_m : d.sb_n, s_k = is_a ? d.sa_k : d.sb_k, s_b = is_a ? d.sa_b : d.sb_b;
    if (is_a ? d.pad_a : d.pad_b) return 0; // already a padded copy
    if (pick_mode(p, R, K, s_r, s_k, s_b, d.batch, es, 256, false) != LOAD_GENERIC) return 0;
    int64_t L, rows, s_row;
    if (s_k == 1) { // rows (m / n) of L = K contiguous elements
        L = K;
        rows = R;
        s_row = s_r;
    } else if (s_r == 1) { // k rows of L = M / N contiguous elements
        L = R;
        rows = K;
        s_row = s_k;
    } else {
        return 0; // no contiguous dimension: the gather stays
    }
    if (L <= 0 || rows <= 0) return 0;
    const int64_t P = (L + vec - 1) / vec * vec;
    const int64_t nb = d.batch > 1 && s_b != 0 ? d.batch : 1;
    // The copy's layout must itself pass (a k-tile panel's offsets within 31 bits); nullptr stands
    // for the workspace's 16-byte aligned base.
    const int64_t ps_r = s_k == 1 ? P : 1, ps_k = s_k == 1 ? 1 : P, ps_b = nb > 1 ? rows * P : 0;
    if (pick_mode(nullptr, R, K, ps_r, ps_k, ps_b, d.batch, es, 256, true) == LOAD_GENERIC) return 0;
    void* ws = nullptr;
    if (gemm_pad_workspace(stream, (size_t)(nb * rows * P * es), is_a ? 0 : 1, &ws) != 0) return 0; // no room: gather
    const int rc = launch_pad_rows(p, ws, es, nb, rows, s_row, s_b, L, P, stream);
    if (rc) return rc;
    if (is_a) {
        d.A = ws;
        (s_k == 1 ? d.sa_m : d.sa_k) = P;
        d.sa_b = nb > 1 ? rows * P : 0;
        d.pad_a = 1;
    } else {
        d.B = ws;
        (s_k == 1 ? d.sb_n : d.sb_k) = P;
        d.sb_b = nb > 1 ? rows * P : 0;
        d.pad_b = 1;
    }
    return 0;
}

// Calls of at least this many multiply-adds, or of K at least kPadMinK, copy misaligned operands
// (pad_operand): below both the gather is cheaper than a second launch.  The gather's cost grows
// with K per output tile (about 4 us per 64 k of bf16), not with the work: bf16 x[1,4096] @
// W[4096,129] (0.5 M) took 276 us gathered, against about 20 us copied onto the matrix-core GEMV.
constexpr int64_t kPadMinMacs = (int64_t)1 << 20;
constexpr int kPadMinK = 256;

int pad_gemm_operands(GemmDesc& d, hipStream_t stream) {
    if ((int64_t)d.M * d.N * d.K * (d.batch > 1 ? d.batch : 1) < kPadMinMacs && d.K < kPadMinK) return 0;
    const int rc = pad_operand(d, true, stream);
    return rc ? rc : pad_operand(d, false, stream);
}

// The stride of a dimension of extent 1 (A's rows when M = 1, B's columns when N = 1, either
// operand's k when K = 1) never steps between two elements a kernel reads, and the caller may pass
// any value there (torch gives a [K, 1] tensor strides (1, 1)).  The vector loaders size each
// buffer range from it, as rows x row stride (k-contiguous) or k rows x k stride (m/n-contiguous),
// so a stride below the row's length cut the one row short, and the elements past the cut read as
// zeros.  Such a stride is replaced by the row's length rounded up to whole 16-byte chunks; the
// zero-padded copies (pad_a / pad_b) already have row strides of that kind.
static GemmDesc with_unit_extent_strides(GemmDesc d) {
    auto up = [](int64_t x, int64_t v) { return ((x > 1 ? x : 1) + v - 1) / v * v; };
    const int64_t va = 16 / (int64_t)dtype_size(d.dtype_a), vb = 16 / (int64_t)dtype_size(d.dtype_b);
    if (!d.pad_a) {
        if (d.M <= 1) d.sa_m = up(d.K, va);
        if (d.K <= 1) d.sa_k = up(d.M, va);
    }
    if (!d.pad_b) {
        if (d.N <= 1) d.sb_n = up(d.K, vb);
        if (d.K <= 1) d.sb_k = up(d.N, vb);
    }
    return d;
}

int launch_gemm_mfma(const GemmDesc& d0, hipStream_t stream, bool may_alloc) {
    const GemmDesc d = with_unit_extent_strides(d0);
    switch (d.dtype_a) {
        case TV_FLOAT32: return launch_gemm_mfma_f32(d, stream, may_alloc);
        case TV_BFLOAT16: return launch_gemm_mfma_bf16(d, stream, may_alloc);
        case TV_FLOAT16: return launch_gemm_mfma_f16(d, stream, may_alloc);
        case TV_INT8: return launch_gemm_mfma_i8(d, stream, may_alloc);
        default: return TV_E_DTYPE;
    }
}
} // namespace tvk
