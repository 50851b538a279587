// Stand-alone C-ABI entry points: compute_gradients and the kernel-level entry points
// that run one kernel of the training path on host buffers (used to check each kernel
// alone against the CPU restatement).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/cbhip.h"
#include "common.hpp"
#include "kernels.hpp"

using namespace cbh;

int cbh_internal_fail(int code, const std::string& msg);  // session.hip

namespace {

int fail2(int code, const std::string& msg);

#define HIP_OK(expr)                                                                        \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess) return fail2(CBH_ERR_DEVICE, std::string(#expr ": ") + hipGetErrorString(e_)); \
    } while (0)

// RAII device buffer
template <typename T>
struct DBuf {
    T* p = nullptr;
    size_t n = 0;
    ~DBuf() {
        if (p) (void)hipFree(p);
    }
    hipError_t alloc(size_t count) {
        n = count;
        return hipMalloc((void**)&p, std::max<size_t>(count, 1) * sizeof(T));
    }
};

__global__ void ders_kernel(int loss, const double* __restrict__ a, const double* __restrict__ t,
                            uint64_t n, double* __restrict__ d1, double* __restrict__ d2) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        double g, h;
        scalar_ders(loss, a[i], t[i], g, h);
        d1[i] = g;
        d2[i] = h;
    }
}

template <int K>
__global__ void softmax_ders_kernel(const double* __restrict__ a, const double* __restrict__ t,
                                    uint64_t n, double* __restrict__ d1, double* __restrict__ d2) {
    constexpr int PK = K * (K + 1) / 2;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        double x[K], p[K];
        for (int d = 0; d < K; ++d) x[d] = a[(size_t)d * n + i];
        softmax_probs<K>(x, p);
        int j = 0;
        for (int y = 0; y < K; ++y) {
            d2[i * PK + j++] = p[y] * (p[y] - 1.0);
            for (int z = y + 1; z < K; ++z) d2[i * PK + j++] = p[y] * p[z];
        }
        const int tc = (int)t[i];
        for (int d = 0; d < K; ++d) d1[(size_t)d * n + i] = (d == tc ? 1.0 : 0.0) - p[d];
    }
}

__global__ void bootstrap_kernel(SampleParams smp, JumpTabs jt, uint64_t n, double* __restrict__ sw,
                                 uint8_t* __restrict__ ctrl) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        double s;
        bool c;
        sample_row(smp, jt, i, s, c);
        sw[i] = s;
        ctrl[i] = c ? 1 : 0;
    }
}

__global__ void pack_stats_kernel(const double* __restrict__ der, const double* __restrict__ w,
                                  uint64_t n, uint32_t K, double* __restrict__ sstat) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        for (uint32_t d = 0; d < K; ++d) sstat[i * (K + 1) + d] = der[(size_t)d * n + i];
        sstat[i * (K + 1) + K] = w[i];
    }
}

// ---- histogram build without allocation (cbh_hist_build_noalloc) ----
// Device scratch of the no-allocation entry: one copy per GPU, alive until the process
// ends.  Host code never passes `scratch` itself (its host-side name is no device address):
// it uses the per-device address hipGetSymbolAddress returns.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr unsigned kBoundBlocks = 256;

// Per-block sums of max_d |der[d][i]| and |w[i]| (the bounds cbh_hist_build takes on the
// host), in a fixed order so the result does not depend on scheduling.
__global__ __launch_bounds__(256) void bound_partials_kernel(const double* __restrict__ der,
                                                             const double* __restrict__ w, uint64_t n,
                                                             uint32_t K, double* __restrict__ part) {
    __shared__ double sd[256], sw[256];
    double ad = 0.0, aw = 0.0;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        double m = 0.0;
        for (uint32_t d = 0; d < K; ++d) m = fmax(m, fabs(der[(size_t)d * n + i]));
        ad += m;
        aw += fabs(w[i]);
    }
    sd[threadIdx.x] = ad;
    sw[threadIdx.x] = aw;
    __syncthreads();
    for (unsigned o = 128; o > 0; o >>= 1) {
        if (threadIdx.x < o) {
            sd[threadIdx.x] += sd[threadIdx.x + o];
            sw[threadIdx.x] += sw[threadIdx.x + o];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        part[2 * blockIdx.x] = sd[0];
        part[2 * blockIdx.x + 1] = sw[0];
    }
}

// The scales of cbh_hist_build from the partial bounds (one thread, blocks in order).
__global__ void bound_scales_kernel(const double* __restrict__ part, unsigned n_part, Scales* __restrict__ sc) {
    if (blockIdx.x != 0 || threadIdx.x != 0) return;
    double b[2] = {0.0, 0.0};
    for (unsigned k = 0; k < n_part; ++k) {
        b[0] += part[2 * k];
        b[1] += part[2 * k + 1];
    }
    for (int k = 0; k < kNumScales; ++k) {
        int e = -20;
        if (k < 2 && b[k] > 0.0) frexp(b[k] * 1.0000001 + 1e-300, &e);
        const int s = min(61 - e, 100);
        sc->shift[k] = s;
        sc->mul[k] = ldexp(1.0, s);
        sc->inv[k] = ldexp(1.0, -s);
    }
}

std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};   // per device: the address of that GPU's `scratch`

// The calling device's scratch address, looked up once per device.
int scratch_address(void** out) {
    int dev = 0;
    HIP_OK(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return fail2(CBH_ERR_UNSUPPORTED, "device index beyond 63");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        HIP_OK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail2(CBH_ERR_DEVICE, "no device address for the scratch array");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return CBH_OK;
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

unsigned grid_of(uint64_t work, unsigned block) {
    uint64_t g = (work + block - 1) / block;
    return (unsigned)std::max<uint64_t>(1, std::min<uint64_t>(g, 65535u * 4));
}

int fail2(int code, const std::string& msg) { return cbh_internal_fail(code, msg); }

template <int C>
int run_fill(const uint32_t* rows, uint32_t W, uint64_t n, const uint32_t* idx,
             const LevelPlan* plan, double* sstat, const Scales* sc, const FillTiles& ft, uint32_t F,
             uint32_t B, long long* hist) {
    quantize_stats_kernel<C><<<grid_of(n * C, 256), 256>>>(sstat, n, sc);
    HIP_OK(hipFuncSetAttribute((const void*)fill_kernel<C, false>, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)ft.lds_bytes));
    const uint32_t G = 64;
    fill_kernel<C, false><<<G * ft.n_tiles, 1024, ft.lds_bytes, 0>>>(rows, W, W, n, idx, plan,
                                                             (const long long*)sstat, ft.n_tiles, ft.tw,
                                                             F, B, G, hist, nullptr, (int)ft.bin_major);
    HIP_OK(hipGetLastError());
    return CBH_OK;
}

template <int C>
int run_fill_on(const uint32_t* rows, uint32_t W, uint64_t n, double* sstat, const Scales* sc, const FillTiles& ft,
                uint32_t F, uint32_t B, long long* hist, hipStream_t st) {
    quantize_stats_kernel<C><<<grid_of(n * C, 256), 256, 0, st>>>(sstat, n, sc);
    HIP_OK(hipFuncSetAttribute((const void*)fill_kernel<C, false>, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)ft.lds_bytes));
    const uint32_t G = 64;
    fill_kernel<C, false><<<G * ft.n_tiles, 1024, ft.lds_bytes, st>>>(rows, W, W, n, nullptr, nullptr,
                                                                     (const long long*)sstat, ft.n_tiles, ft.tw,
                                                                     F, B, G, hist, nullptr, (int)ft.bin_major);
    HIP_OK(hipGetLastError());
    return CBH_OK;
}

}  // namespace

extern "C" {

int cbh_compute_gradients(int32_t loss, const double* approx, const double* target, uint64_t n,
                          uint32_t approx_dim, double* der1, double* der2) {
    if (!approx || !target || !der1 || !der2) return fail2(CBH_ERR_INVALID_ARG, "null argument");
    const uint32_t K = approx_dim;
    if (loss == CBH_LOSS_MULTICLASS ? (K < 2 || K > 16) : K != 1)
        return fail2(CBH_ERR_UNSUPPORTED, "approx_dim not covered");
    const size_t pk = loss == CBH_LOSS_MULTICLASS ? (size_t)K * (K + 1) / 2 : 1;
    DBuf<double> a, t, d1, d2;
    HIP_OK(a.alloc(n * K));
    HIP_OK(t.alloc(n));
    HIP_OK(d1.alloc(n * K));
    HIP_OK(d2.alloc(n * (loss == CBH_LOSS_MULTICLASS ? pk : 1)));
    HIP_OK(hipMemcpy(a.p, approx, sizeof(double) * n * K, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(t.p, target, sizeof(double) * n, hipMemcpyHostToDevice));
    if (loss == CBH_LOSS_MULTICLASS) {
        switch (K) {
#define CASE(k) case k: softmax_ders_kernel<k><<<grid_of(n, 256), 256>>>(a.p, t.p, n, d1.p, d2.p); break;
            CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7) CASE(8) CASE(9) CASE(10) CASE(11) CASE(12)
            CASE(13) CASE(14) CASE(15) CASE(16)
#undef CASE
            default: return fail2(CBH_ERR_UNSUPPORTED, "approx_dim has no compiled variant");
        }
    } else {
        ders_kernel<<<grid_of(n, 256), 256>>>(loss == CBH_LOSS_RMSE ? 0 : 1, a.p, t.p, n, d1.p, d2.p);
    }
    HIP_OK(hipGetLastError());
    HIP_OK(hipMemcpy(der1, d1.p, sizeof(double) * n * K, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(der2, d2.p, sizeof(double) * n * (loss == CBH_LOSS_MULTICLASS ? pk : 1),
                     hipMemcpyDeviceToHost));
    return CBH_OK;
}

int cbh_bootstrap(const cbh_tree_sampling* sampling, uint64_t n, double* sample_weight, uint8_t* control) {
    if (!sampling || !sample_weight || !control) return fail2(CBH_ERR_INVALID_ARG, "null argument");
    SampleParams smp{};
    smp.kind = sampling->kind;
    smp.temperature = sampling->bagging_temperature;
    smp.rate = (double)(float)sampling->subsample;
    smp.bayes_seed = sampling->bayesian_seed;
    smp.bern = Rng{sampling->bernoulli_state[0], sampling->bernoulli_state[1],
                   sampling->bernoulli_state[2], sampling->bernoulli_state[3]};
    if (smp.kind == CBH_BOOT_BERNOULLI && sampling->subsample >= 1.0) smp.kind = 0;
    if (smp.kind == CBH_BOOT_BAYESIAN && sampling->bagging_temperature == 0.0f) smp.kind = 0;
    DBuf<double> sw;
    DBuf<uint8_t> c;
    DBuf<uint64_t> jump;
    const uint64_t n_coarse = (n >> 10) + 2;
    std::vector<uint64_t> h(2048 + 2 * n_coarse);
    make_jump_tables(n_coarse, h.data(), h.data() + 1024, h.data() + 2048, h.data() + 2048 + n_coarse);
    HIP_OK(jump.alloc(h.size()));
    HIP_OK(hipMemcpy(jump.p, h.data(), sizeof(uint64_t) * h.size(), hipMemcpyHostToDevice));
    const JumpTabs jt{jump.p, jump.p + 1024, jump.p + 2048, jump.p + 2048 + n_coarse};
    HIP_OK(sw.alloc(n));
    HIP_OK(c.alloc(n));
    bootstrap_kernel<<<grid_of(n, 256), 256>>>(smp, jt, n, sw.p, c.p);
    HIP_OK(hipGetLastError());
    HIP_OK(hipMemcpy(sample_weight, sw.p, sizeof(double) * n, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(control, c.p, n, hipMemcpyDeviceToHost));
    return CBH_OK;
}

int cbh_hist_build(const uint8_t* bins_fm, uint64_t n, uint32_t F, uint32_t B, const double* der,
                   const double* w, uint32_t K, const uint32_t* slot_of_row, uint32_t n_slots,
                   double* hist_out) {
    if (!bins_fm || !der || !w || !hist_out) return fail2(CBH_ERR_INVALID_ARG, "null argument");
    if (K < 1 || K > 16 || B < 1 || B > 256 || n == 0 || F == 0 || n_slots == 0)
        return fail2(CBH_ERR_INVALID_ARG, "bad shape");
    for (uint64_t i = 0; i < n * F; ++i)
        if (bins_fm[i] >= B) return fail2(CBH_ERR_OUT_OF_RANGE, "bin >= n_bins");
    const uint32_t C = K + 1, W = (F + 3) / 4;
    // scales from sum |v| bounds (same rule as the session)
    double bd = 0.0, bw = 0.0;
    for (uint64_t i = 0; i < n; ++i) {
        double m = 0.0;
        for (uint32_t d = 0; d < K; ++d) m = std::max(m, std::fabs(der[(size_t)d * n + i]));
        bd += m;
        bw += std::fabs(w[i]);
    }
    Scales sc{};
    const double bounds[2] = {bd, bw};
    for (int k = 0; k < kNumScales; ++k) {
        int e = -20;
        if (k < 2 && bounds[k] > 0.0) std::frexp(bounds[k] * 1.0000001 + 1e-300, &e);
        const int s = std::min(61 - e, 100);
        sc.shift[k] = s;
        sc.mul[k] = std::ldexp(1.0, s);
        sc.inv[k] = std::ldexp(1.0, -s);
    }
    // rows grouped by slot, ascending row order (the layout the partition kernels produce)
    std::vector<uint32_t> idx;
    LevelPlan plan{};
    if (slot_of_row) {
        if (n_slots > kMaxLeaves / 2) return fail2(CBH_ERR_INVALID_ARG, "at most 128 slots");
        std::vector<std::vector<uint32_t>> per(n_slots);
        for (uint64_t i = 0; i < n; ++i)
            if (slot_of_row[i] < n_slots) per[slot_of_row[i]].push_back((uint32_t)i);
        for (uint32_t s = 0; s < n_slots; ++s) {
            plan.seg_begin[s] = (uint32_t)idx.size();
            plan.built[s] = s;
            idx.insert(idx.end(), per[s].begin(), per[s].end());
        }
        plan.n_parent = n_slots;
        plan.rows = (uint32_t)idx.size();
    }
    int lds_max = 0, dev = 0;
    HIP_OK(hipGetDevice(&dev));
    HIP_OK(hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
    const FillTiles ft = plan_fill_tiles(F, B, C, std::min<size_t>((size_t)lds_max, 160 * 1024), 1, n);
    if (ft.n_tiles == 0) return fail2(CBH_ERR_UNSUPPORTED, "histogram line too wide for LDS");

    DBuf<uint8_t> cols;
    DBuf<uint32_t> rows, didx;
    DBuf<double> dder, dw, sstat, dout;
    DBuf<LevelPlan> dplan;
    DBuf<Scales> dsc;
    DBuf<long long> hist;
    const size_t cells = (size_t)n_slots * F * B * C;
    HIP_OK(cols.alloc(n * F));
    HIP_OK(rows.alloc(n * W));
    HIP_OK(dder.alloc(n * K));
    HIP_OK(dw.alloc(n));
    HIP_OK(sstat.alloc(n * C));
    HIP_OK(dsc.alloc(1));
    HIP_OK(hist.alloc(cells));
    HIP_OK(dout.alloc(cells));
    HIP_OK(hipMemcpy(cols.p, bins_fm, n * F, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dder.p, der, sizeof(double) * n * K, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dw.p, w, sizeof(double) * n, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dsc.p, &sc, sizeof(Scales), hipMemcpyHostToDevice));
    HIP_OK(hipMemset(hist.p, 0, cells * sizeof(long long)));
    pack_rows_kernel<<<grid_of(n * W, 256), 256>>>(cols.p, n, F, W, rows.p);
    pack_stats_kernel<<<grid_of(n, 256), 256>>>(dder.p, dw.p, n, K, sstat.p);
    HIP_OK(hipGetLastError());
    if (slot_of_row) {
        HIP_OK(didx.alloc(std::max<size_t>(idx.size(), 1)));
        HIP_OK(dplan.alloc(1));
        if (!idx.empty()) HIP_OK(hipMemcpy(didx.p, idx.data(), sizeof(uint32_t) * idx.size(), hipMemcpyHostToDevice));
        HIP_OK(hipMemcpy(dplan.p, &plan, sizeof(LevelPlan), hipMemcpyHostToDevice));
    }
    int rc;
    switch (C) {
#define CASE(c) case c: rc = run_fill<c>(rows.p, W, n, slot_of_row ? didx.p : nullptr, dplan.p, sstat.p, dsc.p, ft, F, B, hist.p); break;
        CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7) CASE(8) CASE(9) CASE(11) CASE(13) CASE(17)
#undef CASE
        default: return fail2(CBH_ERR_UNSUPPORTED, "K has no compiled fill variant");
    }
    if (rc != CBH_OK) return rc;
    hist_to_f64_kernel<<<grid_of(cells, 256), 256>>>(hist.p, cells, C, F, B, dsc.p, dout.p);
    HIP_OK(hipGetLastError());
    HIP_OK(hipMemcpy(hist_out, dout.p, sizeof(double) * cells, hipMemcpyDeviceToHost));
    return CBH_OK;
}

int cbh_hist_build_noalloc(const uint8_t* bins_fm, uint64_t n, uint32_t n_features, uint32_t n_bins,
                           const double* der, const double* w, uint32_t K, double* hist_out, void* stream) {
    if (!bins_fm || !der || !w || !hist_out) return fail2(CBH_ERR_INVALID_ARG, "null argument");
    const uint32_t F = n_features, B = n_bins;
    if (K < 1 || K > 16 || B < 1 || B > 256 || n == 0 || F == 0) return fail2(CBH_ERR_INVALID_ARG, "bad shape");
    const uint32_t C = K + 1, W = (F + 3) / 4;
    // scratch layout: bound partials | scales | packed rows | row statistics | int64 histogram
    const size_t off_sc = align256(sizeof(double) * 2 * kBoundBlocks);
    const size_t off_rows = off_sc + align256(sizeof(Scales));
    const size_t off_sstat = off_rows + align256(sizeof(uint32_t) * (size_t)n * W);
    const size_t off_hist = off_sstat + align256(sizeof(double) * (size_t)n * C);
    const size_t cells = (size_t)F * B * C;
    const size_t need = off_hist + sizeof(long long) * cells;
    if (n >= ((size_t)1 << 32) || need > kNoAllocScratchBytes)
        return fail2(CBH_ERR_OUT_OF_RANGE, "n x (4 ceil(F/4) + 8 (K+1)) + 8 F n_bins (K+1) bytes exceed the " +
                                               std::to_string(kNoAllocScratchBytes >> 20) + " MiB scratch (" +
                                               std::to_string(need) + " bytes asked)");
    int lds_max = 0, dev = 0;
    HIP_OK(hipGetDevice(&dev));
    HIP_OK(hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
    const FillTiles ft = plan_fill_tiles(F, B, C, std::min<size_t>((size_t)lds_max, 160 * 1024), 1, n);
    if (ft.n_tiles == 0) return fail2(CBH_ERR_UNSUPPORTED, "histogram line too wide for LDS");
    if (!(C <= 9 || C == 11 || C == 13 || C == 17)) return fail2(CBH_ERR_UNSUPPORTED, "K has no compiled fill variant");
    void* base = nullptr;
    int rc = scratch_address(&base);
    if (rc != CBH_OK) return rc;
    unsigned char* sp = (unsigned char*)base;
    double* part = (double*)sp;
    Scales* sc = (Scales*)(sp + off_sc);
    uint32_t* rows = (uint32_t*)(sp + off_rows);
    double* sstat = (double*)(sp + off_sstat);
    long long* hist = (long long*)(sp + off_hist);
    hipStream_t st = (hipStream_t)stream;
    bound_partials_kernel<<<kBoundBlocks, 256, 0, st>>>(der, w, n, K, part);
    bound_scales_kernel<<<1, 64, 0, st>>>(part, kBoundBlocks, sc);
    zero_i64_kernel<<<grid_of(cells, 256), 256, 0, st>>>(hist, cells);
    pack_rows_kernel<<<grid_of((uint64_t)n * W, 256), 256, 0, st>>>(bins_fm, n, F, W, rows);
    pack_stats_kernel<<<grid_of(n, 256), 256, 0, st>>>(der, w, n, K, sstat);
    HIP_OK(hipGetLastError());
    switch (C) {
#define CASE(c) case c: rc = run_fill_on<c>(rows, W, n, sstat, sc, ft, F, B, hist, st); break;
        CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7) CASE(8) CASE(9) CASE(11) CASE(13) CASE(17)
#undef CASE
        default: return fail2(CBH_ERR_UNSUPPORTED, "K has no compiled fill variant");
    }
    if (rc != CBH_OK) return rc;
    hist_to_f64_kernel<<<grid_of(cells, 256), 256, 0, st>>>(hist, cells, C, F, B, sc, hist_out);
    HIP_OK(hipGetLastError());
    return CBH_OK;
}

}  // extern "C"
