// ORACLE — TEST INFRASTRUCTURE ONLY.
//
// A CPU restatement of the reference CPU backend's matmul path, MulImpl<Device::CPU>
// (Aimol-l/Tensorvia src/backend/cpu/mul.cpp:7-145), used as the parity checker by tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg.  It is never linked into, loaded by,
// or called from the product libraries (libtv_hip.so, libtensorvia.so).
//
// Restated parts (each function cites the reference lines it follows):
//   oracle_mul          MulImpl<CPU>::execute          mul.cpp:97-145  (widening, result type,
//                       16-thread cap, (T,R) dispatch, S switch)
//   mul_basic           mul_kernel_basic               mul.cpp:7-25
//   mul_tiled           mul_kernel_tiled<T,R,S,64>     mul.cpp:27-85
//   choose              mul_kernel                     mul.cpp:87-96
//   oracle_result_type  compute_type                   include/core/type_traits.h:270-287
//   oracle_widen_f32    cast_kernel (fp16/bf16->fp32)  src/backend/cpu/typecast.cpp:48-53,79-98
//   oracle_transpose_last2  transpose_nd_kernel with axes {0..,d-1,d-2}
//                       src/backend/cpu/transpose.cpp:8-28,69-93,113-126
//
// Build: oracle/Makefile (g++ -O2 -mavx2 -mfma -fopenmp -fwrapv, the reference's CPU flags of
// CMakeLists.txt:37-41 plus -fwrapv so that the integer wrap-around the reference relies on is
// defined behaviour here).
//
// Pinning: every function is checked in tests/test_oracle.py against closed forms and brute force
// (exact int64 sums for integers, exactly representable fp32 sums, numpy transposes, RNE
// conversion tables) and against the committed golden vectors under tests/golden/.
#include <omp.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <type_traits>
#include <vector>

namespace {

enum Dt { I8 = 0, I16, I32, I64, BF16, F16, F32, F64 };

// fp16 / bf16 -> fp32, exact (the reference's static_cast from std::float16_t / std::bfloat16_t).
float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t u;
    if (exp == 0x1F) {
        u = sign | 0x7F800000u | (man << 13);
    } else if (exp != 0) {
        u = sign | ((exp + 112) << 23) | (man << 13);
    } else if (man == 0) {
        u = sign;
    } else {
        // subnormal: normalise
        int e = -1;
        do {
            ++e;
            man <<= 1;
        } while ((man & 0x400u) == 0);
        u = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3FFu) << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// compute_type (include/core/type_traits.h:270-287).
int result_type(int a, int b) {
    if (a == b) return a;
    if (a <= I64 && b <= I64) return std::max(a, b);
    if (a > I64 && b > I64) return std::max(std::max(a, (int)F32), std::max(b, (int)F32));
    if (a == I64 || b == I64) return F64;
    return std::max(std::max(a, (int)F32), std::max(b, (int)F32));
}

// mul_kernel_basic (mul.cpp:7-25): one pass over k per output, accumulator decltype(T + R).
template <typename T, typename R, typename S>
void mul_basic(const T* a, const R* b, S* c, size_t batch, size_t rows, size_t common, size_t cols) {
#pragma omp parallel for collapse(2)
    for (size_t bb = 0; bb < batch; ++bb) {
        for (size_t i = 0; i < rows; ++i) {
            const T* arow = a + bb * rows * common + i * common;
            const R* bmat = b + bb * common * cols;
            S* crow = c + bb * rows * cols + i * cols;
            for (size_t j = 0; j < cols; ++j) {
                using P = decltype(std::declval<T>() + std::declval<R>());
                P acc = 0;
                for (size_t k = 0; k < common; ++k)
                    acc += static_cast<P>(arow[k]) * static_cast<P>(bmat[k * cols + j]);
                crow[j] = static_cast<S>(acc);
            }
        }
    }
}

// mul_kernel_tiled<T,R,S,64> (mul.cpp:27-85): per 64x64 output tile, 64-wide k-chunks staged in
// tile buffers; each chunk is summed in A's element type T with B's values converted to T
// (mul.cpp:64-71), the first chunk's sum is stored into C and later ones are added (mul.cpp:74-78).
template <typename T, typename R, typename S, int TILE = 64>
void mul_tiled(const T* a, const R* b, S* c, size_t batch, size_t rows, size_t common, size_t cols) {
#pragma omp parallel for collapse(3)
    for (size_t bb = 0; bb < batch; ++bb) {
        for (size_t i0 = 0; i0 < rows; i0 += TILE) {
            for (size_t j0 = 0; j0 < cols; j0 += TILE) {
                const size_t i1 = std::min(i0 + TILE, rows);
                const size_t j1 = std::min(j0 + TILE, cols);
                std::vector<T> at(TILE * TILE);
                std::vector<R> bt(TILE * TILE);
                const T* amat = a + bb * rows * common;
                const R* bmat = b + bb * common * cols;
                S* cmat = c + bb * rows * cols;
                for (size_t k0 = 0; k0 < common; k0 += TILE) {
                    const size_t k1 = std::min(k0 + TILE, common);
                    const size_t kn = k1 - k0;
                    for (size_t i = i0; i < i1; ++i)
                        for (size_t k = k0; k < k1; ++k) at[(i - i0) * TILE + (k - k0)] = amat[i * common + k];
                    for (size_t k = k0; k < k1; ++k)
                        for (size_t j = j0; j < j1; ++j) bt[(k - k0) * TILE + (j - j0)] = bmat[k * cols + j];
                    for (size_t i = i0; i < i1; ++i) {
                        for (size_t j = j0; j < j1; ++j) {
                            T acc = 0;
                            for (size_t k = 0; k < kn; ++k)
                                acc += static_cast<T>(at[(i - i0) * TILE + k]) * static_cast<T>(bt[k * TILE + (j - j0)]);
                            S& out = cmat[i * cols + j];
                            if (k0 == 0) out = static_cast<S>(acc);
                            else out += static_cast<S>(acc);
                        }
                    }
                }
            }
        }
    }
}

// mul_kernel (mul.cpp:87-96): basic below 2^20 outputs, tiled otherwise.  variant: 0 = as the
// reference chooses, 1 = force basic, 2 = force tiled.
template <typename T, typename R, typename S>
void choose(const T* a, const R* b, S* c, size_t batch, size_t rows, size_t common, size_t cols, int variant) {
    const bool basic = variant == 1 || (variant == 0 && batch * rows * cols < 1024 * 1024);
    if (basic) mul_basic(a, b, c, batch, rows, common, cols);
    else mul_tiled<T, R, S, 64>(a, b, c, batch, rows, common, cols);
}

template <typename T, typename R>
int dispatch_s(const T* a, const R* b, void* c, int rt, size_t batch, size_t rows, size_t common, size_t cols, int variant) {
    switch (rt) {
        case I8: choose(a, b, static_cast<int8_t*>(c), batch, rows, common, cols, variant); break;
        case I16: choose(a, b, static_cast<int16_t*>(c), batch, rows, common, cols, variant); break;
        case I32: choose(a, b, static_cast<int32_t*>(c), batch, rows, common, cols, variant); break;
        case I64: choose(a, b, static_cast<int64_t*>(c), batch, rows, common, cols, variant); break;
        case F32: choose(a, b, static_cast<float*>(c), batch, rows, common, cols, variant); break;
        case F64: choose(a, b, static_cast<double*>(c), batch, rows, common, cols, variant); break;
        default: return -1;
    }
    return rt;
}

template <typename T>
int dispatch_r(const T* a, int dtb, const void* b, void* c, int rt, size_t batch, size_t rows, size_t common, size_t cols, int variant) {
    switch (dtb) {
        case I8: return dispatch_s(a, static_cast<const int8_t*>(b), c, rt, batch, rows, common, cols, variant);
        case I16: return dispatch_s(a, static_cast<const int16_t*>(b), c, rt, batch, rows, common, cols, variant);
        case I32: return dispatch_s(a, static_cast<const int32_t*>(b), c, rt, batch, rows, common, cols, variant);
        case I64: return dispatch_s(a, static_cast<const int64_t*>(b), c, rt, batch, rows, common, cols, variant);
        case F32: return dispatch_s(a, static_cast<const float*>(b), c, rt, batch, rows, common, cols, variant);
        case F64: return dispatch_s(a, static_cast<const double*>(b), c, rt, batch, rows, common, cols, variant);
        default: return -1;
    }
}

int g_threads_used = 0;

} // namespace

extern "C" {

// compute_type after the CPU backend's fp16/bf16 -> fp32 widening (mul.cpp:110-112).
int oracle_result_type(int dta, int dtb) {
    if (dta == BF16 || dta == F16) dta = F32;
    if (dtb == BF16 || dtb == F16) dtb = F32;
    return result_type(dta, dtb);
}

int oracle_compute_type(int dta, int dtb) { return result_type(dta, dtb); }

// cast_kernel for fp16/bf16 -> fp32 (typecast.cpp:48-53): serial, element by element.
void oracle_widen_f32(int dt, const void* src, float* dst, int64_t n) {
    const uint16_t* s = static_cast<const uint16_t*>(src);
    if (dt == BF16)
        for (int64_t i = 0; i < n; ++i) dst[i] = bf16_to_f32(s[i]);
    else
        for (int64_t i = 0; i < n; ++i) dst[i] = f16_to_f32(s[i]);
}

// MulImpl<CPU>::execute (mul.cpp:97-145) over dense row-major buffers A[batch,rows,common] and
// B[batch,common,cols] (the reference indexes .data() densely, mul.cpp:49,57).  C must have room for
// batch*rows*cols elements of the returned dtype.  Returns the result dtype, or -1.
int oracle_mul(int dta, const void* a, int dtb, const void* b, void* c, int64_t batch, int64_t rows,
               int64_t common, int64_t cols, int variant) {
    std::vector<float> wa, wb;
    if (dta == BF16 || dta == F16) {
        wa.resize((size_t)(batch * rows * common));
        oracle_widen_f32(dta, a, wa.data(), batch * rows * common);
        a = wa.data();
        dta = F32;
    }
    if (dtb == BF16 || dtb == F16) {
        wb.resize((size_t)(batch * common * cols));
        oracle_widen_f32(dtb, b, wb.data(), batch * common * cols);
        b = wb.data();
        dtb = F32;
    }
    const int rt = result_type(dta, dtb);
    omp_set_num_threads(std::min(omp_get_max_threads(), 16));
    g_threads_used = std::min(omp_get_max_threads(), 16);
    const size_t B = (size_t)batch, M = (size_t)rows, K = (size_t)common, N = (size_t)cols;
    switch (dta) {
        case I8: return dispatch_r(static_cast<const int8_t*>(a), dtb, b, c, rt, B, M, K, N, variant);
        case I16: return dispatch_r(static_cast<const int16_t*>(a), dtb, b, c, rt, B, M, K, N, variant);
        case I32: return dispatch_r(static_cast<const int32_t*>(a), dtb, b, c, rt, B, M, K, N, variant);
        case I64: return dispatch_r(static_cast<const int64_t*>(a), dtb, b, c, rt, B, M, K, N, variant);
        case F32: return dispatch_r(static_cast<const float*>(a), dtb, b, c, rt, B, M, K, N, variant);
        case F64: return dispatch_r(static_cast<const double*>(a), dtb, b, c, rt, B, M, K, N, variant);
        default: return -1;
    }
}

// OpenMP threads the last oracle_mul ran with (min(omp_get_max_threads(), 16), mul.cpp:114).
int oracle_threads_used(void) { return g_threads_used; }

// Materialising transpose of the last two dims of a dense [batch, rows, cols] buffer, as
// ops::Transpose(a, {0, 2, 1}) does on the CPU (transpose.cpp:69-93 with prefix = dim-2, which runs
// the 64x64-blocked transpose_2d_kernel, transpose.cpp:8-28, per batch).
void oracle_transpose_last2(int esize, const void* src, void* dst, int64_t batch, int64_t rows, int64_t cols) {
    const char* s = static_cast<const char*>(src);
    char* d = static_cast<char*>(dst);
    const int64_t T = 64;
#pragma omp parallel for collapse(2)
    for (int64_t bb = 0; bb < batch; ++bb) {
        for (int64_t j0 = 0; j0 < cols; j0 += T) {
            const char* sb = s + bb * rows * cols * esize;
            char* db = d + bb * rows * cols * esize;
            const int64_t j1 = std::min(j0 + T, cols);
            for (int64_t i0 = 0; i0 < rows; i0 += T) {
                const int64_t i1 = std::min(i0 + T, rows);
                for (int64_t j = j0; j < j1; ++j)
                    for (int64_t i = i0; i < i1; ++i)
                        std::memcpy(db + (j * rows + i) * esize, sb + (i * cols + j) * esize, esize);
            }
        }
    }
}

} // extern "C"
