// Model apply on the device: raw predictions of an oblivious float ensemble.
//
// Mirrors the reference's device apply (crates/cb-backend/src/kernels.rs:629
// apply_oblivious_float_kernel, launched by launch_apply_oblivious_f64,
// crates/cb-backend/src/gpu_runtime/mod.rs:337) and its CPU twin predict_raw
// (crates/cb-model/src/apply.rs): one object per thread over a feature-major matrix, each
// tree's leaf from its float splits (value > border, forward bit order), contributions
// summed in tree order from 0, the bias added once after the trees.  A split on a feature
// the matrix does not have is absent (bit 0); a NaN value fails every split unless its
// feature is flagged nan_as_true (borders of nan_mode=Max, apply.rs:160-166); a leaf index
// beyond the tree's leaves contributes 0.  Multi-output models (approx_dim K) store the K
// values of a leaf contiguously; the output is dim-major [K][n].
#include <hip/hip_runtime.h>

#include <string>

#include "../../include/cbhip.h"
#include "common.hpp"

int cbh_internal_fail(int code, const std::string& msg);  // session.hip

namespace {

template <int K>
__global__ __launch_bounds__(256) void apply_oblivious_kernel(
    const float* __restrict__ x, uint64_t n, uint32_t F, const uint32_t* __restrict__ split_features,
    const double* __restrict__ split_borders, const uint32_t* __restrict__ tree_split_offsets,
    const double* __restrict__ leaf_values, const uint32_t* __restrict__ tree_leaf_offsets,
    uint32_t n_trees, const double* __restrict__ bias, const uint8_t* __restrict__ nan_as_true,
    double* __restrict__ out) {
    for (uint64_t obj = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; obj < n;
         obj += (uint64_t)gridDim.x * blockDim.x) {
        double acc[K];
#pragma unroll
        for (int d = 0; d < K; ++d) acc[d] = 0.0;
        for (uint32_t t = 0; t < n_trees; ++t) {
            uint32_t leaf = 0, bit = 0;
            for (uint32_t s = tree_split_offsets[t]; s < tree_split_offsets[t + 1]; ++s, ++bit) {
                const uint32_t f = split_features[s];
                bool pass = false;
                if (f < F) {
                    const float v = x[(size_t)f * n + obj];
                    pass = isnan(v) ? (nan_as_true != nullptr && nan_as_true[f] != 0)
                                    : ((double)v > split_borders[s]);
                }
                leaf |= (uint32_t)pass << bit;
            }
            const uint32_t li = tree_leaf_offsets[t] + leaf;
            const bool in = li < tree_leaf_offsets[t + 1];
#pragma unroll
            for (int d = 0; d < K; ++d) acc[d] += in ? leaf_values[(size_t)li * K + d] : 0.0;
        }
#pragma unroll
        for (int d = 0; d < K; ++d) out[(size_t)d * n + obj] = acc[d] + (bias ? bias[d] : 0.0);
    }
}

template <typename T>
struct Buf {
    T* p = nullptr;
    ~Buf() {
        if (p) (void)hipFree(p);
    }
    hipError_t alloc(size_t count) { return hipMalloc((void**)&p, (count ? count : 1) * sizeof(T)); }
};

#define APPLY_TRY(expr)                                                                          \
    do {                                                                                         \
        hipError_t e_ = (expr);                                                                  \
        if (e_ != hipSuccess)                                                                    \
            return cbh_internal_fail(CBH_ERR_DEVICE, std::string(#expr ": ") + hipGetErrorString(e_)); \
    } while (0)

template <int K>
int launch(const float* x, uint64_t n, uint32_t F, const uint32_t* sf, const double* sb, const uint32_t* so,
           const double* lv, const uint32_t* lo, uint32_t T, const double* bias, const uint8_t* nan_true,
           double* out) {
    uint64_t g = (n + 255) / 256;
    if (g > 65535ull * 16) g = 65535ull * 16;
    if (g < 1) g = 1;
    apply_oblivious_kernel<K><<<(unsigned)g, 256>>>(x, n, F, sf, sb, so, lv, lo, T, bias, nan_true, out);
    APPLY_TRY(hipGetLastError());
    return CBH_OK;
}

}  // namespace

extern "C" int cbh_apply_oblivious(const float* features_fm, uint64_t n_objects, uint32_t n_features,
                                   const uint32_t* split_features, const double* split_borders,
                                   const uint32_t* tree_split_offsets, const double* leaf_values,
                                   const uint32_t* tree_leaf_offsets, uint32_t n_trees, uint32_t approx_dim,
                                   const double* bias, const uint8_t* nan_as_true, double* out) {
    if (!tree_split_offsets || !tree_leaf_offsets || !out)
        return cbh_internal_fail(CBH_ERR_INVALID_ARG, "offset arrays and out are required");
    if (n_objects > 0 && n_features > 0 && !features_fm)
        return cbh_internal_fail(CBH_ERR_INVALID_ARG, "features are null");
    // CSR offsets: start at 0, non-decreasing (gpu_runtime/mod.rs:306-330); a leaf index has
    // one bit per split, so a tree has at most 31 splits
    if (tree_split_offsets[0] != 0 || tree_leaf_offsets[0] != 0)
        return cbh_internal_fail(CBH_ERR_OUT_OF_RANGE, "CSR offsets must start at 0");
    for (uint32_t t = 0; t < n_trees; ++t) {
        if (tree_split_offsets[t + 1] < tree_split_offsets[t] || tree_leaf_offsets[t + 1] < tree_leaf_offsets[t])
            return cbh_internal_fail(CBH_ERR_OUT_OF_RANGE, "CSR offsets must be non-decreasing");
        if (tree_split_offsets[t + 1] - tree_split_offsets[t] > 31)
            return cbh_internal_fail(CBH_ERR_OUT_OF_RANGE, "a tree has more than 31 splits");
    }
    const uint32_t n_splits = tree_split_offsets[n_trees];
    const uint32_t n_leaves = tree_leaf_offsets[n_trees];
    if ((n_splits && (!split_features || !split_borders)) || (n_leaves && !leaf_values))
        return cbh_internal_fail(CBH_ERR_INVALID_ARG, "model arrays are null");
    const uint32_t K = approx_dim;
    if (n_objects == 0) return CBH_OK;
    Buf<float> x;
    Buf<uint32_t> sf, so, lo;
    Buf<double> sb, lv, db, dout;
    Buf<uint8_t> na;
    APPLY_TRY(x.alloc(n_objects * n_features));
    APPLY_TRY(sf.alloc(n_splits));
    APPLY_TRY(sb.alloc(n_splits));
    APPLY_TRY(so.alloc((size_t)n_trees + 1));
    APPLY_TRY(lv.alloc((size_t)n_leaves * K));
    APPLY_TRY(lo.alloc((size_t)n_trees + 1));
    APPLY_TRY(dout.alloc(n_objects * K));
    if (n_features)
        APPLY_TRY(hipMemcpy(x.p, features_fm, sizeof(float) * n_objects * n_features, hipMemcpyHostToDevice));
    if (n_splits) {
        APPLY_TRY(hipMemcpy(sf.p, split_features, sizeof(uint32_t) * n_splits, hipMemcpyHostToDevice));
        APPLY_TRY(hipMemcpy(sb.p, split_borders, sizeof(double) * n_splits, hipMemcpyHostToDevice));
    }
    APPLY_TRY(hipMemcpy(so.p, tree_split_offsets, sizeof(uint32_t) * ((size_t)n_trees + 1), hipMemcpyHostToDevice));
    APPLY_TRY(hipMemcpy(lo.p, tree_leaf_offsets, sizeof(uint32_t) * ((size_t)n_trees + 1), hipMemcpyHostToDevice));
    if (n_leaves) APPLY_TRY(hipMemcpy(lv.p, leaf_values, sizeof(double) * n_leaves * K, hipMemcpyHostToDevice));
    if (bias) {
        APPLY_TRY(db.alloc(K));
        APPLY_TRY(hipMemcpy(db.p, bias, sizeof(double) * K, hipMemcpyHostToDevice));
    }
    if (nan_as_true && n_features) {
        APPLY_TRY(na.alloc(n_features));
        APPLY_TRY(hipMemcpy(na.p, nan_as_true, n_features, hipMemcpyHostToDevice));
    }
    int rc;
    switch (K) {
#define CASE(k) case k: rc = launch<k>(x.p, n_objects, n_features, sf.p, sb.p, so.p, lv.p, lo.p, n_trees, bias ? db.p : nullptr, na.p, dout.p); break;
        CASE(1) CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7) CASE(8) CASE(10) CASE(12) CASE(16)
#undef CASE
        default: return cbh_internal_fail(CBH_ERR_UNSUPPORTED, "approx_dim " + std::to_string(K) + " has no apply variant");
    }
    if (rc != CBH_OK) return rc;
    APPLY_TRY(hipMemcpy(out, dout.p, sizeof(double) * n_objects * K, hipMemcpyDeviceToHost));
    return CBH_OK;
}
