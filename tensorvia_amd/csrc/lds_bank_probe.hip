// LDS bank-conflict probe for gfx950: one LDS access pattern per launch, as the GEMM kernels issue
// them, so that rocprofv3's SQ_LDS_BANK_CONFLICT / SQ_INSTS_LDS give the conflict cycles of one
// instruction of that pattern.  Each launch is 256 workgroups of one wave; every wave issues
// kReps instructions of the pattern, each followed by a wait, so the counters divide exactly.
// Every address lies inside the 64 KB shared array.  Prints the patterns in launch order.
//
// usage: lds_bank_probe
#include <hip/hip_runtime.h>

#include <cstdio>

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr int kReps = 1024;
constexpr int kWaves = 256;

enum Kind { READ_B128 = 0, WRITE_B32 = 1, WRITE_B64 = 2 };

struct Pattern {
    const char* name;
    Kind kind;
    int id;
};

// Byte address of lane l for pattern id (all below 4 KB).
__device__ inline unsigned lane_addr(int id, int l) {
    const int r = l % 16;
    switch (id) {
    case 0: return 16 * l;                                            // contiguous 1 KB
    case 1: return r * 128 + 16 * ((l / 16) ^ ((r >> 1) & 7));        // k-loop A fragment (k-contiguous layout)
    case 2: return (l / 16) * 272 + 16 * (l % 16);                    // int8 tile staging, rows of 256 + 16 bytes
    case 3: return (l / 8) * 144 + 16 * (l % 8);                      // 16-bit wave staging, rows of 128 + 16 bytes
    case 4: return (l / 16) * 256 + 16 * (l % 16);                    // rows of 256 bytes
    case 5: return (l / 16) * 256 + 16 * ((l % 16) ^ (l / 16));       // rows of 256 bytes, chunk ^ row
    case 6: return (l / 8) * 128 + 16 * ((l % 8) ^ (l / 8));          // rows of 128 bytes, chunk ^ row
    case 7: return 4 * l;                                             // contiguous 256 bytes
    case 8: return r * 272 + 4 * (l / 16);                            // int8 tile staging: lane l%16 = row
    case 9: return r * 256 + 16 * (0 ^ r) + 4 * (l / 16);             // rows of 256 bytes, chunk ^ row
    case 10: return 8 * l;                                            // contiguous 512 bytes
    case 11: return r * 144 + 8 * (l / 16);                           // 16-bit wave staging: lane l%16 = row
    case 12: return r * 128 + 16 * ((l >> 5) ^ (r & 7)) + 8 * ((l >> 4) & 1); // rows of 128 bytes, chunk ^ row
    default: return 0;
    }
}

template <int KIND>
__global__ __launch_bounds__(64) void lds_probe(int id, unsigned* sink) {
    __shared__ __attribute__((aligned(1024))) char L[65536];
    const int l = threadIdx.x;
    const unsigned a = (unsigned)(uintptr_t)(__attribute__((address_space(3))) char*)L + lane_addr(id, l);
    u32x4 acc = {0, 0, 0, 0};
    for (int i = 0; i < kReps; ++i) {
        if constexpr (KIND == READ_B128) {
            u32x4 v;
            asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
            acc ^= v;
        } else if constexpr (KIND == WRITE_B32) {
            asm volatile("ds_write_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" ::"v"(a), "v"(i) : "memory");
        } else {
            const u32x2 v = {(unsigned)i, (unsigned)l};
            asm volatile("ds_write_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" ::"v"(a), "v"(v) : "memory");
        }
    }
    if (acc.x == 0x9E3779B9u) sink[blockIdx.x] = acc.y; // keeps the reads live
}

const Pattern kPatterns[] = {
    {"ds_read_b128 contiguous", READ_B128, 0},
    {"ds_read_b128 k-loop A fragment (k-contiguous layout)", READ_B128, 1},
    {"ds_read_b128 int8 tile staging (272-byte rows)", READ_B128, 2},
    {"ds_read_b128 16-bit wave staging (144-byte rows)", READ_B128, 3},
    {"ds_read_b128 256-byte rows", READ_B128, 4},
    {"ds_read_b128 256-byte rows, chunk ^ row", READ_B128, 5},
    {"ds_read_b128 128-byte rows, chunk ^ row", READ_B128, 6},
    {"ds_write_b32 contiguous", WRITE_B32, 7},
    {"ds_write_b32 int8 tile staging (272-byte rows, lane % 16 = row)", WRITE_B32, 8},
    {"ds_write_b32 256-byte rows, chunk ^ row", WRITE_B32, 9},
    {"ds_write_b64 contiguous", WRITE_B64, 10},
    {"ds_write_b64 16-bit wave staging (144-byte rows, lane % 16 = row)", WRITE_B64, 11},
    {"ds_write_b64 128-byte rows, chunk ^ row", WRITE_B64, 12},
};

} // namespace

int main() {
    unsigned* sink = nullptr;
    if (hipMalloc(&sink, kWaves * sizeof(unsigned)) != hipSuccess) {
        std::fprintf(stderr, "lds_bank_probe: hipMalloc failed\n");
        return 1;
    }
    int n = 0;
    for (const Pattern& p : kPatterns) {
        if (p.kind == READ_B128) hipLaunchKernelGGL(lds_probe<READ_B128>, dim3(kWaves), dim3(64), 0, 0, p.id, sink);
        else if (p.kind == WRITE_B32) hipLaunchKernelGGL(lds_probe<WRITE_B32>, dim3(kWaves), dim3(64), 0, 0, p.id, sink);
        else hipLaunchKernelGGL(lds_probe<WRITE_B64>, dim3(kWaves), dim3(64), 0, 0, p.id, sink);
        const hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) {
            std::fprintf(stderr, "lds_bank_probe: %s: %s\n", p.name, hipGetErrorString(e));
            return 1;
        }
        std::printf("dispatch %d: %s (%d waves x %d instructions)\n", n++, p.name, kWaves, kReps);
    }
    (void)hipFree(sink);
    return 0;
}
