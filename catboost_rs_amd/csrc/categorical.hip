// Categorical inputs on the device: first-seen bins of category keys (PerfectHash,
// crates/cb-data/src/cat_hash.rs:389-479) and online (ordered) CTR columns
// (materialize_ctr_feature, crates/cb-train/src/ctr/ctr_feature.rs; the reference's device
// twin is ordered_ctr_prefix_kernel, crates/cb-backend/src/kernels/ctr_device.rs:164-399,
// a single-thread serial scan).
//
// The ordered statistic of an object is a count over its PREDECESSORS in the learn
// permutation that share its bucket (read before increment).  Here that prefix is computed
// data-parallel and exactly: the positions 0..n-1 are radix-sorted by bucket (the sort is
// stable, so each bucket's positions stay ascending), after which an object's predecessor
// count is its rank inside its bucket segment and its predecessor class-1 count is a
// difference of one exclusive prefix sum of the classes.  Counter CTRs use whole-set bucket
// sizes (segment lengths) and their maximum.  No step counts through an atomic on a shared
// address: device atomics on one address serialize at about a microsecond each on this GPU,
// and category frequencies are heavily skewed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <string>
#include <vector>

#include "../../include/cbhip.h"
#include "common.hpp"
#include "prim.hpp"

int cbh_internal_fail(int code, const std::string& msg);  // session.hip

namespace {

#define CAT_TRY(expr)                                                                           \
    do {                                                                                        \
        hipError_t e_ = (expr);                                                                 \
        if (e_ != hipSuccess)                                                                   \
            return cbh_internal_fail(CBH_ERR_DEVICE, std::string(#expr ": ") + hipGetErrorString(e_)); \
    } while (0)

template <typename T>
struct Buf {
    T* p = nullptr;
    ~Buf() {
        if (p) (void)hipFree(p);
    }
    hipError_t alloc(size_t count) { return hipMalloc((void**)&p, (count ? count : 1) * sizeof(T)); }
};

constexpr uint32_t kMaxCtrSpecs = 16;

struct SpecArgs {   // per spec: type, numerator selector, prior, normalization
    int32_t type[kMaxCtrSpecs];
    uint32_t tbi[kMaxCtrSpecs];
    double prior[kMaxCtrSpecs];
    double shift[kMaxCtrSpecs];
    double norm[kMaxCtrSpecs];
};

unsigned grid_for(uint64_t n, uint64_t cap = 16384) {
    uint64_t g = (n + 255) / 256;
    return (unsigned)std::max<uint64_t>(1, std::min<uint64_t>(g, cap));
}

uint32_t bits_for(uint64_t max_value) {   // radix bits to sort keys in [0, max_value]
    uint32_t b = 1;
    while (b < 32 && (max_value >> b) != 0) ++b;
    return b;
}

__global__ void iota_kernel(uint32_t* __restrict__ v, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        v[i] = (uint32_t)i;
}

// keys in permutation order: key[p] = bucket[perm[p]], value p
__global__ void gather_keys_kernel(const uint32_t* __restrict__ bucket, const uint32_t* __restrict__ perm,
                                   uint64_t n, uint32_t* __restrict__ key, uint32_t* __restrict__ pos) {
    for (uint64_t p = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; p < n; p += (uint64_t)gridDim.x * blockDim.x) {
        key[p] = bucket[perm[p]];
        pos[p] = (uint32_t)p;
    }
}

// per sorted slot: the object's class and the slot index if it opens a bucket segment
__global__ void segment_prep_kernel(const uint32_t* __restrict__ skey, const uint32_t* __restrict__ spos,
                                    const uint32_t* __restrict__ perm, const uint8_t* __restrict__ cls,
                                    uint64_t n, uint32_t* __restrict__ c, uint32_t* __restrict__ head) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
        c[i] = cls[perm[spos[i]]] == 1 ? 1u : 0u;
        head[i] = (i == 0 || skey[i] != skey[i - 1]) ? (uint32_t)i : 0u;
    }
}

// bucket sizes from the last slot of every segment (each bucket written once)
__global__ void segment_size_kernel(const uint32_t* __restrict__ skey, const uint32_t* __restrict__ start,
                                    uint64_t n, uint32_t* __restrict__ size) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        if (i + 1 == n || skey[i + 1] != skey[i]) size[skey[i]] = (uint32_t)(i - start[i] + 1);
}

__device__ __forceinline__ uint8_t clamp_bin(double bin_f, uint32_t border_count) {
    const double t = trunc(bin_f);
    if (t < 0.0) return 0;
    if (t > (double)border_count) return (uint8_t)border_count;
    return (uint8_t)t;
}

// Every spec's value and bin of every object (ctr_feature.rs materialize_ctr_feature):
//   Borders @ b: total - sum_{c<=b} N_c;  Buckets @ b: N_b;  BTMV: the f32 running sum of the
//   classes (exact: a sum of ones, which an f32 holds up to 2^24); Counter: bucket size over
//   the maximum bucket size.  value = (num + prior) / (total + 1); bin = trunc of
//   (value + shift) / norm * border_count clamped to [0, border_count], in f32 for BTMV.
__global__ void ctr_finalize_kernel(const uint32_t* __restrict__ skey, const uint32_t* __restrict__ spos,
                                    const uint32_t* __restrict__ perm, const uint32_t* __restrict__ excl,
                                    const uint32_t* __restrict__ start, const uint32_t* __restrict__ bsize,
                                    const uint32_t* __restrict__ max_size, uint64_t n, SpecArgs sp,
                                    uint32_t n_specs, uint32_t border_count, uint8_t* __restrict__ bins,
                                    double* __restrict__ values, uint32_t* __restrict__ counts) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t obj = perm[spos[i]];
        const uint32_t s = start[i];
        const uint32_t total = (uint32_t)(i - s);
        const uint32_t n1 = excl[i] - excl[s];
        const uint32_t n0 = total - n1;
        if (counts) {
            counts[obj] = n0;
            counts[n + obj] = n1;
        }
        for (uint32_t k = 0; k < n_specs; ++k) {
            double num, den;
            bool f32_bin = false;
            switch (sp.type[k]) {
                case CBH_CTR_BUCKETS:
                    num = sp.tbi[k] == 0 ? (double)n0 : (sp.tbi[k] == 1 ? (double)n1 : 0.0);
                    den = (double)total;
                    break;
                case CBH_CTR_BTMV:
                    num = (double)(n1 < 16777216u ? (float)n1 : 16777216.0f);
                    den = (double)total;
                    f32_bin = true;
                    break;
                case CBH_CTR_COUNTER:
                    num = (double)bsize[skey[i]];
                    den = (double)*max_size;
                    break;
                default:   // Borders
                    num = sp.tbi[k] == 0 ? (double)n1 : 0.0;
                    den = (double)total;
                    break;
            }
            const double v = (num + sp.prior[k]) / (den + 1.0);
            double bf;
            if (f32_bin) {
                const float d = (float)den + 1.0f;
                const float c = ((float)num + (float)sp.prior[k]) / d;
                bf = (double)(((c + (float)sp.shift[k]) / (float)sp.norm[k]) * (float)border_count);
            } else {
                bf = sp.norm[k] == 0.0 ? 0.0 : (v + sp.shift[k]) / sp.norm[k] * (double)border_count;
            }
            bins[(size_t)k * n + obj] = clamp_bin(bf, border_count);
            if (values) values[(size_t)k * n + obj] = v;
        }
    }
}

// One CTR column of a session (build_ctr_cindex_columns, gpu_runtime/session.rs:262-360):
// the spec's value of every object (as ctr_finalize_kernel) binarized by the column's own
// border table, bin = the number of borders strictly below the value (binarize_ctr_kernel,
// kernels/ctr_device.rs:399-413; a NaN border never counts).  The table sits in LDS.
__global__ __launch_bounds__(256) void ctr_table_kernel(
    const uint32_t* __restrict__ skey, const uint32_t* __restrict__ spos, const uint32_t* __restrict__ perm,
    const uint32_t* __restrict__ excl, const uint32_t* __restrict__ start, const uint32_t* __restrict__ bsize,
    const uint32_t* __restrict__ max_size, uint64_t n, int32_t type, uint32_t tbi, double prior,
    const double* __restrict__ borders, uint32_t n_borders, uint8_t* __restrict__ bins) {
    __shared__ double bd[256];
    for (uint32_t j = threadIdx.x; j < n_borders; j += blockDim.x) bd[j] = borders[j];
    __syncthreads();
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t obj = perm[spos[i]];
        const uint32_t s = start[i];
        const uint32_t total = (uint32_t)(i - s);
        const uint32_t n1 = excl[i] - excl[s];
        const uint32_t n0 = total - n1;
        double num, den;
        switch (type) {
            case CBH_CTR_BUCKETS:
                num = tbi == 0 ? (double)n0 : (tbi == 1 ? (double)n1 : 0.0);
                den = (double)total;
                break;
            case CBH_CTR_BTMV:   // the f32 running sum of the classes
                num = (double)(n1 < 16777216u ? (float)n1 : 16777216.0f);
                den = (double)total;
                break;
            case CBH_CTR_COUNTER:
                num = (double)bsize[skey[i]];
                den = (double)*max_size;
                break;
            default:   // Borders
                num = tbi == 0 ? (double)n1 : 0.0;
                den = (double)total;
                break;
        }
        const double v = (num + prior) / (den + 1.0);
        uint32_t b = 0;
        for (uint32_t j = 0; j < n_borders; ++j) b += v > bd[j] ? 1u : 0u;
        bins[obj] = (uint8_t)b;
    }
}

// ---- first-seen bins ----
__global__ void head_flag_kernel(const uint32_t* __restrict__ skey, uint64_t n, uint32_t* __restrict__ flag) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        flag[i] = (i == 0 || skey[i] != skey[i - 1]) ? 1u : 0u;
}

// every segment's first object index (the smallest: the stable sort keeps index order)
__global__ void segment_first_kernel(const uint32_t* __restrict__ skey, const uint32_t* __restrict__ sidx,
                                     const uint32_t* __restrict__ segid1, uint64_t n,
                                     uint32_t* __restrict__ first, uint32_t* __restrict__ seg) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        if (i == 0 || skey[i] != skey[i - 1]) {
            first[segid1[i] - 1] = sidx[i];
            seg[segid1[i] - 1] = segid1[i] - 1;
        }
}

__global__ void rank_kernel(const uint32_t* __restrict__ sseg, uint64_t d, uint32_t* __restrict__ rank) {
    for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < d; r += (uint64_t)gridDim.x * blockDim.x)
        rank[sseg[r]] = (uint32_t)r;
}

__global__ void assign_bins_kernel(const uint32_t* __restrict__ sidx, const uint32_t* __restrict__ segid1,
                                   const uint32_t* __restrict__ rank, uint64_t n, uint32_t* __restrict__ bins) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        bins[sidx[i]] = rank[segid1[i] - 1];
}

}  // namespace

// The CTR bins of m session columns under one permutation, written to the device array
// dst [m][n] on stream st (the caller has validated every input: a permutation of 0..n-1,
// classes 0/1, member codes below n_buckets[c], at most 255 borders per column).  Columns
// that share a member column share its sort: the sorted bucket segments do not depend on
// the spec.
int cbh_internal_ctr_bins(const cbh_device_ctr_column* cols, uint32_t m, const uint64_t* n_buckets,
                          const uint32_t* permutation, const uint32_t* target_class, uint64_t n,
                          uint8_t* dst, hipStream_t st) {
    if (m == 0 || n == 0) return CBH_OK;
    Buf<uint32_t> db, dperm, key, pos, skey, spos, c, head, excl, start, bsize, maxsz;
    Buf<uint8_t> dcls;
    Buf<double> dbord;
    for (Buf<uint32_t>* b : {&db, &dperm, &key, &pos, &skey, &spos, &c, &head, &excl, &start})
        CAT_TRY(b->alloc(n));
    uint64_t nb_max = 1;
    for (uint32_t k = 0; k < m; ++k) nb_max = std::max<uint64_t>(nb_max, n_buckets[k]);
    CAT_TRY(bsize.alloc(nb_max));
    CAT_TRY(maxsz.alloc(1));
    CAT_TRY(dcls.alloc(n));
    CAT_TRY(dbord.alloc(256));
    {
        std::vector<uint8_t> cls(n);
        for (uint64_t i = 0; i < n; ++i) cls[i] = (uint8_t)target_class[i];
        CAT_TRY(hipMemcpyAsync(dcls.p, cls.data(), n, hipMemcpyHostToDevice, st));
        CAT_TRY(hipMemcpyAsync(dperm.p, permutation, sizeof(uint32_t) * n, hipMemcpyHostToDevice, st));
        CAT_TRY(hipStreamSynchronize(st));
    }
    const int N = (int)n;
    Buf<uint8_t> tmp;
    size_t tb = 0;
    std::vector<bool> done(m, false);
    for (uint32_t c0 = 0; c0 < m; ++c0) {
        if (done[c0]) continue;
        const uint32_t* member = cols[c0].member_bins[0];
        const uint64_t nb = n_buckets[c0];
        const int kbits = (int)bits_for(nb ? nb - 1 : 0);
        size_t t1 = 0, t2 = 0, t3 = 0, t4 = 0;
        CAT_TRY(cbh::prim::sort_pairs(nullptr, t1, key.p, skey.p, pos.p, spos.p, N, 0, kbits, st));
        CAT_TRY(cbh::prim::exclusive_sum(nullptr, t2, c.p, excl.p, N, st));
        CAT_TRY(cbh::prim::inclusive_max(nullptr, t3, head.p, start.p, N, st));
        CAT_TRY(cbh::prim::reduce_max(nullptr, t4, bsize.p, maxsz.p, (int)nb, st));
        const size_t need = std::max(std::max(t1, t2), std::max(t3, t4));
        if (need > tb) {
            CAT_TRY(hipStreamSynchronize(st));
            if (tmp.p) (void)hipFree(tmp.p);
            tmp.p = nullptr;
            CAT_TRY(tmp.alloc(need));
            tb = need;
        }
        CAT_TRY(hipMemcpyAsync(db.p, member, sizeof(uint32_t) * n, hipMemcpyHostToDevice, st));
        gather_keys_kernel<<<grid_for(n), 256, 0, st>>>(db.p, dperm.p, n, key.p, pos.p);
        CAT_TRY(hipGetLastError());
        size_t tbx = tb;
        CAT_TRY(cbh::prim::sort_pairs(tmp.p, tbx, key.p, skey.p, pos.p, spos.p, N, 0, kbits, st));
        segment_prep_kernel<<<grid_for(n), 256, 0, st>>>(skey.p, spos.p, dperm.p, dcls.p, n, c.p, head.p);
        CAT_TRY(hipGetLastError());
        tbx = tb;
        CAT_TRY(cbh::prim::exclusive_sum(tmp.p, tbx, c.p, excl.p, N, st));
        tbx = tb;
        CAT_TRY(cbh::prim::inclusive_max(tmp.p, tbx, head.p, start.p, N, st));
        CAT_TRY(hipMemsetAsync(bsize.p, 0, sizeof(uint32_t) * nb, st));
        segment_size_kernel<<<grid_for(n), 256, 0, st>>>(skey.p, start.p, n, bsize.p);
        CAT_TRY(hipGetLastError());
        tbx = tb;
        CAT_TRY(cbh::prim::reduce_max(tmp.p, tbx, bsize.p, maxsz.p, (int)nb, st));
        for (uint32_t k = c0; k < m; ++k) {
            if (done[k] || cols[k].member_bins[0] != member) continue;
            done[k] = true;
            const cbh_device_ctr_column& col = cols[k];
            if (col.n_borders)
                CAT_TRY(hipMemcpyAsync(dbord.p, col.borders, sizeof(double) * col.n_borders,
                                       hipMemcpyHostToDevice, st));
            ctr_table_kernel<<<grid_for(n), 256, 0, st>>>(skey.p, spos.p, dperm.p, excl.p, start.p, bsize.p,
                                                          maxsz.p, n, col.ctr_type, col.target_border_idx,
                                                          col.prior, dbord.p, col.n_borders, dst + (size_t)k * n);
            CAT_TRY(hipGetLastError());
            // the border table is reused by the next column: wait for this launch
            CAT_TRY(hipStreamSynchronize(st));
        }
    }
    return CBH_OK;
}

extern "C" {

int cbh_shuffled_indices(uint64_t n, uint64_t seed, uint32_t count, uint32_t* out) {
    if (n && !out) return cbh_internal_fail(CBH_ERR_INVALID_ARG, "out is null");
    if (n >= (1ull << 32)) return cbh_internal_fail(CBH_ERR_UNSUPPORTED, "more than 2^32 objects");
    // count Fisher-Yates shuffles drawn one after another off one TFastRng64 stream: for i in
    // 1..n swap(i, uniform(i + 1)) (permutation.rs:131-160, :236); a sequential host loop, every
    // swap depends on the previous ones
    cbh::Rng r = cbh::rng_from_seed(seed);
    for (uint32_t k = 0; k < count; ++k) {
        uint32_t* v = out + (size_t)k * n;
        for (uint64_t i = 0; i < n; ++i) v[i] = (uint32_t)i;
        for (uint64_t i = 1; i < n; ++i) {
            const uint64_t j = cbh::rng_uniform(r, i + 1);
            std::swap(v[i], v[j]);
        }
    }
    return CBH_OK;
}

int cbh_perfect_hash(const uint32_t* keys, uint64_t n, uint32_t* bins_out, uint32_t* n_distinct_out) {
    if ((n && (!keys || !bins_out)) || !n_distinct_out) return cbh_internal_fail(CBH_ERR_INVALID_ARG, "null argument");
    if (n >= (1ull << 31)) return cbh_internal_fail(CBH_ERR_UNSUPPORTED, "more than 2^31 objects");
    *n_distinct_out = 0;
    if (n == 0) return CBH_OK;
    Buf<uint32_t> k, ks, idx, sidx, flag, segid1, first, seg, sfirst, sseg, rank, out;
    for (Buf<uint32_t>* b : {&k, &ks, &idx, &sidx, &flag, &segid1, &first, &seg, &sfirst, &sseg, &rank, &out})
        CAT_TRY(b->alloc(n));
    CAT_TRY(hipMemcpy(k.p, keys, sizeof(uint32_t) * n, hipMemcpyHostToDevice));
    const int N = (int)n;
    size_t t1 = 0, t2 = 0, t3 = 0;
    CAT_TRY(cbh::prim::sort_pairs(nullptr, t1, k.p, ks.p, idx.p, sidx.p, N, 0, 32));
    CAT_TRY(cbh::prim::inclusive_sum(nullptr, t2, flag.p, segid1.p, N));
    CAT_TRY(cbh::prim::sort_pairs(nullptr, t3, first.p, sfirst.p, seg.p, sseg.p, N, 0,
                                               (int)bits_for(n)));
    Buf<uint8_t> tmp;
    size_t tb = std::max(t1, std::max(t2, t3));
    CAT_TRY(tmp.alloc(tb));
    iota_kernel<<<grid_for(n), 256>>>(idx.p, n);
    CAT_TRY(hipGetLastError());
    CAT_TRY(cbh::prim::sort_pairs(tmp.p, tb, k.p, ks.p, idx.p, sidx.p, N, 0, 32));
    head_flag_kernel<<<grid_for(n), 256>>>(ks.p, n, flag.p);
    CAT_TRY(hipGetLastError());
    CAT_TRY(cbh::prim::inclusive_sum(tmp.p, tb, flag.p, segid1.p, N));
    uint32_t d = 0;
    CAT_TRY(hipMemcpy(&d, segid1.p + (n - 1), sizeof(uint32_t), hipMemcpyDeviceToHost));
    segment_first_kernel<<<grid_for(n), 256>>>(ks.p, sidx.p, segid1.p, n, first.p, seg.p);
    CAT_TRY(hipGetLastError());
    CAT_TRY(cbh::prim::sort_pairs(tmp.p, tb, first.p, sfirst.p, seg.p, sseg.p, (int)d, 0,
                                               (int)bits_for(n)));
    rank_kernel<<<grid_for(d), 256>>>(sseg.p, d, rank.p);
    CAT_TRY(hipGetLastError());
    assign_bins_kernel<<<grid_for(n), 256>>>(sidx.p, segid1.p, rank.p, n, out.p);
    CAT_TRY(hipGetLastError());
    CAT_TRY(hipMemcpy(bins_out, out.p, sizeof(uint32_t) * n, hipMemcpyDeviceToHost));
    *n_distinct_out = d;
    return CBH_OK;
}

int cbh_ctr_columns(const uint32_t* buckets, uint32_t n_buckets, uint64_t n, const uint32_t* permutation,
                    const uint8_t* target_class, const cbh_ctr_spec* specs, uint32_t n_specs,
                    uint32_t border_count, uint8_t* bins_out, double* values_out, uint32_t* class_counts_out) {
    if (n && (!buckets || !permutation || !target_class || !bins_out))
        return cbh_internal_fail(CBH_ERR_INVALID_ARG, "null argument");
    if (!specs || n_specs == 0 || n_specs > kMaxCtrSpecs)
        return cbh_internal_fail(CBH_ERR_OUT_OF_RANGE, "1..16 CTR specs per call");
    if (border_count == 0 || border_count > 255)
        return cbh_internal_fail(CBH_ERR_OUT_OF_RANGE, "border_count must be 1..255 (u8 bins)");
    if (n >= (1ull << 31)) return cbh_internal_fail(CBH_ERR_UNSUPPORTED, "more than 2^31 objects");
    SpecArgs sp{};
    for (uint32_t k = 0; k < n_specs; ++k) {
        const cbh_ctr_spec& s = specs[k];
        if (s.ctr_type != CBH_CTR_BORDERS && s.ctr_type != CBH_CTR_BUCKETS && s.ctr_type != CBH_CTR_BTMV &&
            s.ctr_type != CBH_CTR_COUNTER)
            return cbh_internal_fail(CBH_ERR_UNSUPPORTED, "CTR type not covered (FloatTargetMeanValue / "
                                                          "FeatureFreq are not CPU types either)");
        if (s.prior_denom == 0.0) return cbh_internal_fail(CBH_ERR_DEGENERATE, "prior_denom must be non-zero");
        sp.type[k] = s.ctr_type;
        sp.tbi[k] = s.target_border_idx;
        sp.prior[k] = s.prior_num / s.prior_denom;
        const double left = std::min(0.0, sp.prior[k]), right = std::max(1.0, sp.prior[k]);
        sp.shift[k] = -left;
        sp.norm[k] = right - left;
    }
    if (n == 0) return CBH_OK;
    // host validation: buckets in range, the permutation a permutation, classes binary
    {
        std::vector<uint8_t> seen(n, 0);
        for (uint64_t p = 0; p < n; ++p) {
            const uint32_t o = permutation[p];
            if (o >= n || seen[o]) return cbh_internal_fail(CBH_ERR_OUT_OF_RANGE, "permutation is not a permutation of 0..n-1");
            seen[o] = 1;
        }
        for (uint64_t i = 0; i < n; ++i) {
            if (buckets[i] >= n_buckets) return cbh_internal_fail(CBH_ERR_OUT_OF_RANGE, "bucket >= n_buckets");
            if (target_class[i] > 1) return cbh_internal_fail(CBH_ERR_OUT_OF_RANGE, "target_class must be 0 or 1");
        }
    }
    Buf<uint32_t> db, dperm, key, pos, skey, spos, c, head, excl, start, bsize, maxsz, counts;
    Buf<uint8_t> dcls, dbins;
    Buf<double> dvals;
    for (Buf<uint32_t>* b : {&db, &dperm, &key, &pos, &skey, &spos, &c, &head, &excl, &start})
        CAT_TRY(b->alloc(n));
    CAT_TRY(bsize.alloc(n_buckets));
    CAT_TRY(maxsz.alloc(1));
    CAT_TRY(dcls.alloc(n));
    CAT_TRY(dbins.alloc((size_t)n_specs * n));
    if (values_out) CAT_TRY(dvals.alloc((size_t)n_specs * n));
    if (class_counts_out) CAT_TRY(counts.alloc(2 * n));
    CAT_TRY(hipMemcpy(db.p, buckets, sizeof(uint32_t) * n, hipMemcpyHostToDevice));
    CAT_TRY(hipMemcpy(dperm.p, permutation, sizeof(uint32_t) * n, hipMemcpyHostToDevice));
    CAT_TRY(hipMemcpy(dcls.p, target_class, n, hipMemcpyHostToDevice));
    const int N = (int)n;
    const int kbits = (int)bits_for(n_buckets ? n_buckets - 1 : 0);
    size_t t1 = 0, t2 = 0, t3 = 0, t4 = 0;
    CAT_TRY(cbh::prim::sort_pairs(nullptr, t1, key.p, skey.p, pos.p, spos.p, N, 0, kbits));
    CAT_TRY(cbh::prim::exclusive_sum(nullptr, t2, c.p, excl.p, N));
    CAT_TRY(cbh::prim::inclusive_max(nullptr, t3, head.p, start.p, N));
    CAT_TRY(cbh::prim::reduce_max(nullptr, t4, bsize.p, maxsz.p, (int)n_buckets));
    Buf<uint8_t> tmp;
    const size_t tb = std::max(std::max(t1, t2), std::max(t3, t4));
    CAT_TRY(tmp.alloc(tb));
    gather_keys_kernel<<<grid_for(n), 256>>>(db.p, dperm.p, n, key.p, pos.p);
    CAT_TRY(hipGetLastError());
    size_t tbx = tb;
    CAT_TRY(cbh::prim::sort_pairs(tmp.p, tbx, key.p, skey.p, pos.p, spos.p, N, 0, kbits));
    segment_prep_kernel<<<grid_for(n), 256>>>(skey.p, spos.p, dperm.p, dcls.p, n, c.p, head.p);
    CAT_TRY(hipGetLastError());
    tbx = tb;
    CAT_TRY(cbh::prim::exclusive_sum(tmp.p, tbx, c.p, excl.p, N));
    tbx = tb;
    CAT_TRY(cbh::prim::inclusive_max(tmp.p, tbx, head.p, start.p, N));
    // bucket sizes: zero-filled (empty buckets stay 0), the last slot of each segment writes
    CAT_TRY(hipMemset(bsize.p, 0, sizeof(uint32_t) * n_buckets));
    segment_size_kernel<<<grid_for(n), 256>>>(skey.p, start.p, n, bsize.p);
    CAT_TRY(hipGetLastError());
    tbx = tb;
    CAT_TRY(cbh::prim::reduce_max(tmp.p, tbx, bsize.p, maxsz.p, (int)n_buckets));
    ctr_finalize_kernel<<<grid_for(n), 256>>>(skey.p, spos.p, dperm.p, excl.p, start.p, bsize.p, maxsz.p, n, sp,
                                              n_specs, border_count, dbins.p, values_out ? dvals.p : nullptr,
                                              class_counts_out ? counts.p : nullptr);
    CAT_TRY(hipGetLastError());
    CAT_TRY(hipMemcpy(bins_out, dbins.p, (size_t)n_specs * n, hipMemcpyDeviceToHost));
    if (values_out) CAT_TRY(hipMemcpy(values_out, dvals.p, sizeof(double) * n_specs * n, hipMemcpyDeviceToHost));
    if (class_counts_out) CAT_TRY(hipMemcpy(class_counts_out, counts.p, sizeof(uint32_t) * 2 * n, hipMemcpyDeviceToHost));
    return CBH_OK;
}

}  // extern "C"
