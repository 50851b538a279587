// Measures the LDS atomic-add rate of the GPU for the address patterns that bound the
// histogram fills.  Every thread computes its addresses before the timed loop (8 per thread,
// reused every iteration), so the loop issues back-to-back LDS atomics and nothing else: the
// rate is the LDS pipe's, not the address arithmetic's.  1024-thread workgroups, 128 KB of LDS
// each (16384 64-bit cells), two workgroups per CU in the grid.
// Patterns (a DPP row is a group of 16 consecutive lanes):
//   contiguous_u64 / _u32        64 lanes on 64 neighbouring cells (the best case)
//   scattered_u64 / _u32 / _rtn  every lane a random cell (with return: the old value used)
//   contiguous_u64_16of64_lanes  contiguous, only lanes 0-15 of a wave active (printed as
//                                instructions per second x 64: an instruction's cost does not
//                                shrink with its active lanes)
//   dpp_rows_same_pairs_u64      the four DPP rows on the same 16 bank pairs at other addresses
//   dpp_row_pairs_random_rows_u64 the fills' pattern: lane l of a DPP row at column l of a
//                                random 256-byte bin row (16 distinct bank pairs, random rows)
//   dpp_row_mod16_pairs_u64      columns (r + 2 l) mod 32 of random bin rows: 8 pairs of lanes
//                                of a DPP row on the same bank pair (column mod 16)
//   *_160k_lo / *_160k_hi        160 KiB workgroups (the whole LDS), addresses in the low 128 KiB
//                                or in the top 32 KiB: contiguous, and the folded narrow words'
//                                pattern (lane l: cell bin * 16 + 8 (l >> 3) + ... 16 distinct
//                                bank pairs of random bin rows of 16 cells)
// Prints one line per pattern: "<pattern> <lane-atomics per second>".
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#define CK(x)                                                                   \
    do {                                                                        \
        hipError_t e = (x);                                                     \
        if (e != hipSuccess) {                                                  \
            std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e));        \
            return 1;                                                           \
        }                                                                       \
    } while (0)

constexpr int kIters = 2048;
constexpr int kAddr = 8;        // addresses per thread
constexpr int kCells = 16384;   // 128 KB of u64 cells
constexpr int kBigCells = 20480;   // 160 KB

__device__ __forceinline__ uint32_t mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

enum Pattern : int {
    kContiguous = 0,
    kScattered = 1,
    kDppSamePairs = 2,
    kDppPairsRandomRows = 3,
    kDppMod16Pairs = 4,
    kFoldRows = 5,
};

// T: cell type (u64 or u32); kRtn: use the returned old value (an atomic with return);
// kQuarter: only lanes 0-15 of every wave issue.
// kBig: a 160 KiB workgroup; kBase: the first cell the addresses use (16384 = the top 32 KiB)
template <int kPattern, typename T, int kRtn, int kQuarter = 0, int kBig = 0, uint32_t kBase = 0>
__global__ __launch_bounds__(1024) void rate_kernel(unsigned long long* out, uint32_t seed) {
    extern __shared__ unsigned long long cells_raw[];
    T* cells = (T*)(cells_raw + kBase);
    constexpr uint32_t all_cells = (kBig ? kBigCells : kCells) * 8 / sizeof(T);
    constexpr uint32_t n_cells = (kBase ? 4096u : kCells) * 8 / sizeof(T);   // the cells the addresses span
    for (uint32_t i = threadIdx.x; i < all_cells; i += blockDim.x) ((T*)cells_raw)[i] = 0;
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u, l = threadIdx.x & 15u, row = threadIdx.x >> 4;
    uint32_t idx[kAddr];
#pragma unroll
    for (int q = 0; q < kAddr; ++q) {
        const uint32_t h = mix32(threadIdx.x * 7919u + blockIdx.x * 104729u + seed * 31u + (uint32_t)q * 1000003u);
        const uint32_t hr = mix32(row * 7919u + blockIdx.x * 104729u + seed * 31u + (uint32_t)q * 1000003u);
        uint32_t c;
        if (kPattern == kContiguous) c = (uint32_t)q * 64u + lane + 512u * (threadIdx.x >> 6);
        else if (kPattern == kScattered) c = h;
        else if (kPattern == kDppSamePairs) c = l + 32u * ((threadIdx.x >> 4) & 3u) + 128u * (uint32_t)q;
        else if (kPattern == kDppPairsRandomRows) c = (h & 255u) * 32u + l;
        else if (kPattern == kDppMod16Pairs) c = (h & 255u) * 32u + (((hr & 31u) + 2u * l) & 31u);
        else c = (h & 255u) * 16u + 8u * (l >> 3) + (((uint32_t)q + (l & 7u)) & 3u) + 4u * ((l >> 2) & 1u);
        idx[q] = c % n_cells;
    }
    T carry = 0;
    const bool issue = !(kQuarter && lane >= 16);
    for (int it = 0; issue && it < kIters; ++it) {
#pragma unroll
        for (int q = 0; q < kAddr; ++q) {
            if (kRtn) carry += atomicAdd(&cells[idx[q]], (T)1) >> 31;
            else atomicAdd(&cells[idx[q]], (T)1);
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = (unsigned long long)cells[0] + (unsigned long long)carry;
}

template <int kPattern, typename T, int kRtn, int kQuarter = 0, int kBig = 0, uint32_t kBase = 0>
int measure(const char* name, int blocks, unsigned long long* d) {
    constexpr int bytes = (kBig ? kBigCells : kCells) * 8;
    CK(hipFuncSetAttribute((const void*)rate_kernel<kPattern, T, kRtn, kQuarter, kBig, kBase>,
                           hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
    rate_kernel<kPattern, T, kRtn, kQuarter, kBig, kBase><<<blocks, 1024, bytes>>>(d, 1u);
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
    hipEvent_t a, b;
    CK(hipEventCreate(&a));
    CK(hipEventCreate(&b));
    CK(hipEventRecord(a));
    rate_kernel<kPattern, T, kRtn, kQuarter, kBig, kBase><<<blocks, 1024, bytes>>>(d, 2u);
    CK(hipEventRecord(b));
    CK(hipEventSynchronize(b));
    float ms = 0.f;
    CK(hipEventElapsedTime(&ms, a, b));
    // lane-atomics per second; with kQuarter the wave-level instruction rate x 64 (each
    // instruction counted as if all 64 lanes were active), comparable with the full-lane line
    const double lanes = (double)blocks * 1024.0 * kIters * kAddr;
    std::printf("%s %.6e\n", name, lanes / (ms * 1e-3));
    CK(hipEventDestroy(a));
    CK(hipEventDestroy(b));
    return 0;
}

int main() {
    int dev = 0, cus = 0;
    CK(hipGetDevice(&dev));
    CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    unsigned long long* d = nullptr;
    const int blocks = 2 * cus;
    CK(hipMalloc(&d, sizeof(unsigned long long) * blocks));
    using u64 = unsigned long long;
    if (measure<kScattered, u64, 0>("scattered_u64", blocks, d)) return 1;
    if (measure<kContiguous, u64, 0>("contiguous_u64", blocks, d)) return 1;
    if (measure<kScattered, unsigned int, 0>("scattered_u32", blocks, d)) return 1;
    if (measure<kScattered, unsigned int, 1>("scattered_u32_rtn", blocks, d)) return 1;
    if (measure<kContiguous, unsigned int, 0>("contiguous_u32", blocks, d)) return 1;
    if (measure<kContiguous, u64, 0, 1>("contiguous_u64_16of64_lanes", blocks, d)) return 1;
    if (measure<kDppSamePairs, u64, 0>("dpp_rows_same_pairs_u64", blocks, d)) return 1;
    if (measure<kDppPairsRandomRows, u64, 0>("dpp_row_pairs_random_rows_u64", blocks, d)) return 1;
    if (measure<kDppMod16Pairs, u64, 0>("dpp_row_mod16_pairs_u64", blocks, d)) return 1;
    if (measure<kContiguous, u64, 0, 0, 1>("contiguous_u64_160k_lo", blocks, d)) return 1;
    if (measure<kContiguous, u64, 0, 0, 1, 16384>("contiguous_u64_160k_hi", blocks, d)) return 1;
    if (measure<kFoldRows, u64, 0, 0, 1>("fold_rows_u64_160k_lo", blocks, d)) return 1;
    if (measure<kFoldRows, u64, 0, 0, 1, 16384>("fold_rows_u64_160k_hi", blocks, d)) return 1;
    if (measure<kDppPairsRandomRows, u64, 0, 0, 1>("dpp_row_pairs_random_rows_u64_160k_lo", blocks, d)) return 1;
    CK(hipFree(d));
    return 0;
}
