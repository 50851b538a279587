// Measures the LDS atomic-add rate of the GPU for the address patterns that bound the
// histogram fill: scattered cells (the fill's pattern: every lane a random bin) and
// contiguous cells (64 lanes on 64 neighbouring cells, the best case), for 64-bit cells
// (the fill's) and 32-bit cells with and without a returned value, and contiguous 64-bit
// atomics with 16 of every 64 lanes active (an instruction's cost does not shrink with its
// active lanes: the fills are bound by the wave-level atomic instruction rate).  1024-thread
// workgroups, 128 KB of LDS each, every address reduced into the array.
// Prints one line per pattern: "<pattern> <lane-atomics per second>" (the 16-of-64 pattern:
// instructions per second x 64).
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

constexpr int kIters = 4096;
constexpr int kCells = 16384;  // 128 KB of u64 cells

__device__ __forceinline__ uint32_t mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// T: cell type (u64 or u32); kRtn: use the returned old value (an atomic with return);
// kQuarter: only lanes 0-15 of every wave issue (an instruction with 16 of 64 lanes active).
// kScattered 2 (u64): the 16 lanes of each DPP row hit 16 distinct bank pairs, and the four DPP
// rows the same 16 pairs at other addresses (cells (l & 15) + 32 (l >> 4) + 128 it), which
// shows whether an instruction's conflicts count within 16 or within 32 lanes.
template <int kScattered, typename T, int kRtn, int kQuarter = 0>
__global__ __launch_bounds__(1024) void rate_kernel(unsigned long long* out, uint32_t seed) {
    extern __shared__ unsigned long long cells_raw[];
    T* cells = (T*)cells_raw;
    constexpr uint32_t n_cells = kCells * 8 / sizeof(T);
    for (uint32_t i = threadIdx.x; i < n_cells; i += blockDim.x) cells[i] = 0;
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t h = mix32(threadIdx.x * 7919u + blockIdx.x * 104729u + seed);
    T carry = 0;
    const bool issue = !(kQuarter && lane >= 16);
    for (int it = 0; issue && it < kIters; ++it) {
        uint32_t idx;
        if (kScattered == 2) {
            idx = ((lane & 15u) + 32u * (lane >> 4) + 128u * (uint32_t)it) % n_cells;
        } else if (kScattered) {
            h = mix32(h + (uint32_t)it);
            idx = h % n_cells;
        } else {
            idx = ((uint32_t)it * 64u + lane) % n_cells;
        }
        if (kRtn) carry += atomicAdd(&cells[idx], (T)1) >> 31;
        else atomicAdd(&cells[idx], (T)1);
    }
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = (unsigned long long)cells[0] + (unsigned long long)carry;
}

template <int kScattered, typename T, int kRtn, int kQuarter = 0>
int measure(const char* name, int blocks, unsigned long long* d) {
    CK(hipFuncSetAttribute((const void*)rate_kernel<kScattered, T, kRtn, kQuarter>,
                           hipFuncAttributeMaxDynamicSharedMemorySize, kCells * 8));
    rate_kernel<kScattered, T, kRtn, kQuarter><<<blocks, 1024, kCells * 8>>>(d, 1u);
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
    hipEvent_t a, b;
    CK(hipEventCreate(&a));
    CK(hipEventCreate(&b));
    CK(hipEventRecord(a));
    rate_kernel<kScattered, T, kRtn, kQuarter><<<blocks, 1024, kCells * 8>>>(d, 2u);
    CK(hipEventRecord(b));
    CK(hipEventSynchronize(b));
    float ms = 0.f;
    CK(hipEventElapsedTime(&ms, a, b));
    // lane-atomics per second; with kQuarter the wave-level instruction rate x 64 (each
    // instruction counted as if all 64 lanes were active), comparable with the full-lane line
    const double lanes = (double)blocks * 1024.0 * kIters;
    std::printf("%s %.6e\n", name, lanes / (ms * 1e-3));
    return 0;
}

int main() {
    int dev = 0, cus = 0;
    CK(hipGetDevice(&dev));
    CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    unsigned long long* d = nullptr;
    const int blocks = 2 * cus;
    CK(hipMalloc(&d, sizeof(unsigned long long) * blocks));
    if (measure<1, unsigned long long, 0>("scattered_u64", blocks, d)) return 1;
    if (measure<0, unsigned long long, 0>("contiguous_u64", blocks, d)) return 1;
    if (measure<1, unsigned int, 0>("scattered_u32", blocks, d)) return 1;
    if (measure<1, unsigned int, 1>("scattered_u32_rtn", blocks, d)) return 1;
    if (measure<0, unsigned int, 0>("contiguous_u32", blocks, d)) return 1;
    if (measure<0, unsigned long long, 0, 1>("contiguous_u64_16of64_lanes", blocks, d)) return 1;
    if (measure<2, unsigned long long, 0>("dpp_rows_same_pairs_u64", blocks, d)) return 1;
    CK(hipFree(d));
    return 0;
}
