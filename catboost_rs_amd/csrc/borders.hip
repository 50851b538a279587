// Float-feature preparation: greedy border selection (GreedyLogSum / GreedyMinEntropy,
// crates/cb-data/src/borders.rs) and device quantization of float columns into u8 bins
// (bin_of, crates/cb-compute/src/histogram.rs:563-569; device twin quantize_pack_feature_kernel,
// crates/cb-backend/src/kernels.rs:2852).
//
// Border selection keeps the reference's split of work: the object subset (200000 rows
// drawn by a fixed-seed partial Fisher-Yates, borders.rs:504-516) is gathered on the host
// with its NaNs made the positive quiet NaN, the values of every column are sorted on the
// GPU in one segmented radix sort (NaNs land after +inf and are cut off; the sort dominates
// border selection at scale), and the greedy bin heap -- at most border_count pops per
// column -- runs on the host, one worker per column.  Device atomics on one address cost
// about a microsecond each in series here, so no step counts through a shared counter.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <queue>
#include <string>
#include <thread>
#include <vector>

#include "../../include/cbhip.h"
#include "common.hpp"
#include "prim.hpp"

int cbh_internal_fail(int code, const std::string& msg);  // session.hip

namespace {

constexpr uint64_t kMaxSubsetForBorders = 200000;   // borders.rs:48

#define BRD_TRY(expr)                                                                           \
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

// ---- greedy split over sorted values (borders.rs:120-270, 572-640) ----
struct GBin {
    uint64_t start, end, best;
    double score;
    uint64_t seq;
};

double penalty(int kind, double w) { return kind == 0 ? -std::log(w + 1e-8) : w * std::log(w + 1e-8); }

double split_score(const GBin& b, uint64_t pos, int kind) {
    if (pos == b.start || pos == b.end) return -INFINITY;
    const double left = -penalty(kind, (double)(pos - b.start));
    const double right = -penalty(kind, (double)(b.end - pos));
    const double curr = -penalty(kind, (double)(b.end - b.start));
    return left + right - curr;
}

void update_best(GBin& b, const float* v, int kind) {
    const uint64_t mid = b.start + (b.end - b.start) / 2;
    const float mv = v[mid];
    const uint64_t lb = (uint64_t)(std::lower_bound(v + b.start, v + mid, mv) - v);
    const uint64_t ub = (uint64_t)(std::upper_bound(v + mid, v + b.end, mv) - v);
    const double sl = split_score(b, lb, kind), sr = split_score(b, ub, kind);
    if (sl >= sr) {
        b.best = lb;
        b.score = sl;
    } else {
        b.best = ub;
        b.score = sr;
    }
}

struct ByScore {   // max-heap: higher score first, earlier insertion first on ties
    bool operator()(const GBin& a, const GBin& b) const {
        if (a.score != b.score) return a.score < b.score;
        return a.seq > b.seq;
    }
};

// One column: sorted non-NaN values v[0..m) -> borders (sentinel first when asked).
uint32_t greedy_borders(const float* v, uint64_t m, uint32_t border_count, bool sentinel, int kind,
                        double* out) {
    const uint32_t budget = sentinel ? (border_count ? border_count - 1 : 0) : border_count;
    std::vector<float> b32;
    if (m >= 2) {
        std::priority_queue<GBin, std::vector<GBin>, ByScore> q;
        uint64_t seq = 0;
        GBin root{0, m, 0, 0.0, seq++};
        update_best(root, v, kind);
        q.push(root);
        while (q.size() <= budget) {
            const GBin& top = q.top();
            if (!(top.start != top.best && top.end != top.best)) break;
            GBin t = top;
            q.pop();
            GBin left{t.start, t.best, 0, 0.0, seq++};
            update_best(left, v, kind);
            t.start = t.best;
            t.seq = seq++;
            update_best(t, v, kind);
            q.push(left);
            q.push(t);
        }
        while (!q.empty()) {
            const GBin& b = q.top();
            if (b.start != 0) {   // LeftBorder in f32: 0.5f * prev, then += 0.5f * cur
                float border = 0.5f * v[b.start - 1];
                border += 0.5f * v[b.start];
                if (border == 0.0f) border = 0.0f;
                b32.push_back(border);
            }
            q.pop();
        }
    }
    std::sort(b32.begin(), b32.end());
    b32.erase(std::unique(b32.begin(), b32.end()), b32.end());
    uint32_t k = 0;
    if (sentinel) out[k++] = (double)(-3.40282346638528859812e+38F);
    for (float b : b32) out[k++] = (double)b;
    return k;
}

// ---- device quantization (bin_of) ----
// One block per (row chunk, feature); the feature's borders are staged in LDS.  NaN goes to
// the top bin when the borders end with the nan_mode=Max sentinel f32::MAX, else to bin 0.
__global__ __launch_bounds__(256) void quantize_kernel(const float* __restrict__ col, uint64_t n,
                                                       const double* __restrict__ borders, uint32_t nb,
                                                       uint8_t* __restrict__ out) {
    __shared__ double bs[256];
    for (uint32_t i = threadIdx.x; i < nb; i += blockDim.x) bs[i] = borders[i];
    __syncthreads();
    const bool nan_top = nb > 0 && bs[nb - 1] == (double)3.40282346638528859812e+38F;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const float v = col[i];
        uint32_t bin;
        if (isnan(v)) {
            bin = nan_top ? nb : 0u;
        } else {   // number of borders strictly below v (lower bound)
            const double dv = (double)v;
            uint32_t lo = 0, hi = nb;
            while (lo < hi) {
                const uint32_t mid = (lo + hi) >> 1;
                if (bs[mid] < dv) lo = mid + 1;
                else hi = mid;
            }
            bin = lo;
        }
        out[i] = (uint8_t)bin;
    }
}

}  // namespace

// Device quantization of one column on a stream (used by the raw session open).
int cbh_internal_quantize(const float* d_col, uint64_t n, const double* d_borders, uint32_t nb, uint8_t* d_out,
                          hipStream_t st) {
    uint64_t g = (n + 255) / 256;
    if (g > 8192) g = 8192;
    quantize_kernel<<<(unsigned)std::max<uint64_t>(g, 1), 256, 0, st>>>(d_col, n, d_borders, nb, d_out);
    BRD_TRY(hipGetLastError());
    return CBH_OK;
}

// Host worker threads: the hardware's, at most 16 (the CPU share a GPU of a shared host gets)
// and at most OMP_NUM_THREADS when the environment sets it.
static unsigned host_threads() {
    unsigned t = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (const char* e = std::getenv("OMP_NUM_THREADS")) {
        const long v = std::strtol(e, nullptr, 10);
        if (v >= 1 && (unsigned long)v < t) t = (unsigned)v;
    }
    return t;
}

extern "C" {

int cbh_quantize(const float* column, uint64_t n, const double* borders, uint32_t n_borders, uint8_t* bins_out) {
    if ((n && (!column || !bins_out)) || (n_borders && !borders))
        return cbh_internal_fail(CBH_ERR_INVALID_ARG, "null argument");
    if (n_borders > 255) return cbh_internal_fail(CBH_ERR_OUT_OF_RANGE, "more than 255 borders do not fit u8 bins");
    for (uint32_t k = 1; k < n_borders; ++k)
        if (!(borders[k - 1] < borders[k])) return cbh_internal_fail(CBH_ERR_OUT_OF_RANGE, "borders must ascend");
    if (n == 0) return CBH_OK;
    Buf<float> c;
    Buf<double> b;
    Buf<uint8_t> o;
    BRD_TRY(c.alloc(n));
    BRD_TRY(b.alloc(n_borders));
    BRD_TRY(o.alloc(n));
    BRD_TRY(hipMemcpy(c.p, column, sizeof(float) * n, hipMemcpyHostToDevice));
    if (n_borders) BRD_TRY(hipMemcpy(b.p, borders, sizeof(double) * n_borders, hipMemcpyHostToDevice));
    const int rc = cbh_internal_quantize(c.p, n, b.p, n_borders, o.p, nullptr);
    if (rc != CBH_OK) return rc;
    BRD_TRY(hipMemcpy(bins_out, o.p, n, hipMemcpyDeviceToHost));
    return CBH_OK;
}

int cbh_select_borders(const float* const* columns, uint64_t n, uint32_t n_features, uint32_t border_count,
                       int32_t nan_mode, int32_t border_type, double* borders_out, uint32_t* n_borders_out) {
    if (!columns || !borders_out || !n_borders_out) return cbh_internal_fail(CBH_ERR_INVALID_ARG, "null argument");
    if (border_type != CBH_BORDERS_GREEDY_LOGSUM && border_type != CBH_BORDERS_GREEDY_MIN_ENTROPY)
        return cbh_internal_fail(CBH_ERR_UNSUPPORTED, "border type not covered");
    if (nan_mode != CBH_NAN_MIN && nan_mode != CBH_NAN_MAX && nan_mode != CBH_NAN_FORBIDDEN)
        return cbh_internal_fail(CBH_ERR_INVALID_ARG, "unknown nan_mode");
    // u8 bins: at most 255 borders per feature, the Max sentinel included
    if (border_count == 0 || border_count > (nan_mode == CBH_NAN_MAX ? 254u : 255u))
        return cbh_internal_fail(CBH_ERR_OUT_OF_RANGE, "border_count must leave at most 255 borders (u8 bins)");
    const uint32_t F = n_features;
    if (F == 0) return CBH_OK;
    for (uint32_t f = 0; f < F; ++f)
        if (n && !columns[f]) return cbh_internal_fail(CBH_ERR_INVALID_ARG, "column is null");
    // object subset: every row, or the fixed-seed 200000-row sample (ascending)
    std::vector<uint32_t> sample;
    const bool sampled = n > kMaxSubsetForBorders;
    if (n >= (1ull << 32)) return cbh_internal_fail(CBH_ERR_UNSUPPORTED, "more than 2^32 rows");
    if (sampled) {
        std::vector<uint32_t> idx(n);
        for (uint64_t i = 0; i < n; ++i) idx[i] = (uint32_t)i;
        cbh::Rng r = cbh::rng_from_seed(0);
        for (uint64_t i = 0; i < kMaxSubsetForBorders; ++i) {
            const uint64_t off = cbh::rng_uniform(r, n - i);
            std::swap(idx[i], idx[i + off]);
        }
        // the subset in ascending order: a bitmap of the drawn rows, read back in order
        std::vector<uint64_t> bits((n + 63) / 64, 0);
        for (uint64_t i = 0; i < kMaxSubsetForBorders; ++i) bits[idx[i] >> 6] |= 1ull << (idx[i] & 63);
        sample.reserve(kMaxSubsetForBorders);
        for (uint64_t w = 0; w < bits.size(); ++w)
            for (uint64_t b = bits[w]; b; b &= b - 1) sample.push_back((uint32_t)(w * 64 + __builtin_ctzll(b)));
    }
    const uint64_t S = sampled ? kMaxSubsetForBorders : n;
    if (S == 0 || (uint64_t)F * S >= (1ull << 31)) {
        if (S == 0) {
            for (uint32_t f = 0; f < F; ++f) n_borders_out[f] = 0;
            return CBH_OK;
        }
        return cbh_internal_fail(CBH_ERR_UNSUPPORTED, "n_features x sample rows exceeds 2^31 values");
    }
    // gather the subset and find the NaN-bearing columns (over every row), a worker per column
    const unsigned nt = std::max(1u, std::min<unsigned>(host_threads(), F));
    std::vector<float> vals((size_t)F * S);
    std::vector<uint8_t> has_nan(F, 0);
    {
        std::vector<std::thread> pool;
        for (unsigned w = 0; w < nt; ++w)
            pool.emplace_back([&, w]() {
                for (uint32_t f = w; f < F; f += nt) {
                    const float* c = columns[f];
                    // every NaN becomes the positive quiet NaN, which the radix sort puts
                    // after +inf: each sorted segment is its non-NaN values, then the NaNs
                    float* dst = vals.data() + (size_t)f * S;
                    const float qnan = std::numeric_limits<float>::quiet_NaN();
                    for (uint64_t i = 0; i < S; ++i) {
                        const float x = c[sampled ? sample[i] : i];
                        dst[i] = x != x ? qnan : x;
                    }
                    // NaN scan over the whole column, in blocks the compiler vectorizes
                    bool any = false;
                    for (uint64_t b0 = 0; b0 < n && !any; b0 += 4096) {
                        const uint64_t b1 = std::min<uint64_t>(n, b0 + 4096);
                        int acc = 0;
                        for (uint64_t i = b0; i < b1; ++i) acc |= (c[i] != c[i]);
                        any = acc != 0;
                    }
                    has_nan[f] = any;
                }
            });
        for (auto& t : pool) t.join();
    }
    // device: sort the values of every column (one segmented radix sort)
    Buf<float> dv, ds;
    Buf<int> dbeg, dend;
    BRD_TRY(dv.alloc(vals.size()));
    BRD_TRY(ds.alloc(vals.size()));
    BRD_TRY(dbeg.alloc(F));
    BRD_TRY(dend.alloc(F));
    BRD_TRY(hipMemcpy(dv.p, vals.data(), sizeof(float) * vals.size(), hipMemcpyHostToDevice));
    std::vector<int> beg(F), end(F);
    for (uint32_t f = 0; f < F; ++f) {
        beg[f] = (int)((uint64_t)f * S);
        end[f] = beg[f] + (int)S;
    }
    BRD_TRY(hipMemcpy(dbeg.p, beg.data(), sizeof(int) * F, hipMemcpyHostToDevice));
    BRD_TRY(hipMemcpy(dend.p, end.data(), sizeof(int) * F, hipMemcpyHostToDevice));
    size_t tmp_bytes = 0;
    BRD_TRY(cbh::prim::segmented_sort_keys(nullptr, tmp_bytes, dv.p, ds.p, (int)vals.size(), (int)F,
                                                       dbeg.p, dend.p, 0, 32));
    Buf<uint8_t> tmp;
    BRD_TRY(tmp.alloc(tmp_bytes));
    BRD_TRY(cbh::prim::segmented_sort_keys(tmp.p, tmp_bytes, dv.p, ds.p, (int)vals.size(), (int)F,
                                                       dbeg.p, dend.p, 0, 32));
    BRD_TRY(hipMemcpy(vals.data(), ds.p, sizeof(float) * vals.size(), hipMemcpyDeviceToHost));
    std::vector<uint64_t> cnt(F);
    for (uint32_t f = 0; f < F; ++f) {
        const float* seg = vals.data() + (size_t)f * S;
        cnt[f] = (uint64_t)(std::partition_point(seg, seg + S, [](float x) { return x == x; }) - seg);
    }
    // host: the greedy heap of every column, then the NaN sentinel of its mode
    const int kind = border_type == CBH_BORDERS_GREEDY_LOGSUM ? 0 : 1;
    const uint32_t stride = border_count + 1;
    std::vector<std::thread> pool;
    for (unsigned w = 0; w < nt; ++w)
        pool.emplace_back([&, w]() {
            for (uint32_t f = w; f < F; f += nt) {
                double* o = borders_out + (size_t)f * stride;
                const bool min_sentinel = has_nan[f] && nan_mode == CBH_NAN_MIN;
                uint32_t k = greedy_borders(vals.data() + (size_t)f * S, cnt[f], border_count, min_sentinel, kind, o);
                if (has_nan[f] && nan_mode == CBH_NAN_MAX) o[k++] = (double)3.40282346638528859812e+38F;
                n_borders_out[f] = k;
            }
        });
    for (auto& t : pool) t.join();
    return CBH_OK;
}

}  // extern "C"
