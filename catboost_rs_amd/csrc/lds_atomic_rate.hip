// Measures the 64-bit LDS atomic-add rate of the GPU for the address patterns that bound
// the histogram fill: scattered cells (the fill's pattern: every lane a random bin) and
// contiguous cells (64 lanes on 64 neighbouring cells, the best case).  One 1024-thread
// workgroup per CU-slot, 128 KB of LDS, every address masked into the array.
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

template <int kScattered>
__global__ __launch_bounds__(1024) void rate_kernel(unsigned long long* out, uint32_t seed) {
    extern __shared__ unsigned long long cells[];
    for (int i = threadIdx.x; i < kCells; i += blockDim.x) cells[i] = 0;
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t h = mix32(threadIdx.x * 7919u + blockIdx.x * 104729u + seed);
    for (int it = 0; it < kIters; ++it) {
        uint32_t idx;
        if (kScattered) {
            h = mix32(h + (uint32_t)it);
            idx = h % kCells;
        } else {
            idx = ((uint32_t)it * 64u + lane) % kCells;
        }
        atomicAdd(&cells[idx], 1ull);
    }
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = cells[0];
}

template <int kScattered>
int measure(const char* name, int blocks, unsigned long long* d) {
    CK(hipFuncSetAttribute((const void*)rate_kernel<kScattered>,
                           hipFuncAttributeMaxDynamicSharedMemorySize, kCells * 8));
    rate_kernel<kScattered><<<blocks, 1024, kCells * 8>>>(d, 1u);
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
    hipEvent_t a, b;
    CK(hipEventCreate(&a));
    CK(hipEventCreate(&b));
    CK(hipEventRecord(a));
    rate_kernel<kScattered><<<blocks, 1024, kCells * 8>>>(d, 2u);
    CK(hipEventRecord(b));
    CK(hipEventSynchronize(b));
    float ms = 0.f;
    CK(hipEventElapsedTime(&ms, a, b));
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
    if (measure<1>("scattered_u64", blocks, d)) return 1;
    if (measure<0>("contiguous_u64", blocks, d)) return 1;
    CK(hipFree(d));
    return 0;
}
