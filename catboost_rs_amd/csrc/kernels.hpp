// HIP kernels of the gfx950 oblivious-tree training path.
//
// Data layout in HBM (per session):
//   rows   u32 [n][W]      row-major packed bins, 4 features per word (byte k of word w is
//                          feature 4w+k); a fill reads only the words of its feature tile
//   cols   u8  [F][n]      feature-major bins, read once per level by the split kernel
//   sstat  f64 [n][K+1]    score channels per row: K weighted, sampled derivatives, then the
//                          sampled weight (zero for rows outside the bootstrap sample);
//                          quantized in place to int64 fixed point once the tree's scales
//                          are known
//   leaf   u16 [n]         leaf index, bit 15 set for rows outside the score sample
//   idx    u32 [<= n]      row ids of the directly built children, grouped by parent leaf,
//                          ascending row order inside each group (stable partition)
//   hist   i64 [2^l][K+1][F][B]  exact fixed-point histograms of level l (channel planes)
#pragma once
#include <algorithm>

#include "common.hpp"

namespace cbh {

struct SplitRec {
    uint32_t feature;
    uint32_t bin;
    uint32_t one_hot;
    uint32_t valid;
    double score;
};

struct LevelPlan {            // written by compact (block 0), read by fill/derive
    uint32_t pad0;
    uint32_t n_parent;
    uint32_t rows;            // rows visited by the next fill (sum of built segments)
    uint32_t pad;
    uint32_t built[kMaxLeaves / 2];
    uint32_t seg_begin[kMaxLeaves / 2];
};

// Row range g of G over the idx list of a gathered level, balanced by cost rather than rows:
// position x costs C(x) = x + lambda * s(x), s(x) the segment holding x, so a range pays lambda
// rows' worth for every segment boundary it crosses (each costs a flush of its LDS tile), and
// ranges over many small segments get fewer rows.  Range g is [C^-1(g T / G), C^-1((g+1) T / G))
// with T = V + lambda (n_seg - 1); C^-1 by binary search over the segments.
__device__ __forceinline__ uint32_t cost_inverse(const LevelPlan* __restrict__ plan, uint32_t n_seg, uint32_t V,
                                                 uint64_t lambda, uint64_t target) {
    uint32_t lo = 0, hi = n_seg;   // last s with seg_begin[s] + lambda * s <= target
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) / 2;
        if ((uint64_t)plan->seg_begin[mid] + lambda * mid <= target) lo = mid;
        else hi = mid;
    }
    const uint64_t seg_end = lo + 1 < n_seg ? plan->seg_begin[lo + 1] : V;
    const uint64_t x = target - lambda * lo;
    return (uint32_t)(x < seg_end ? x : seg_end);
}

__device__ __forceinline__ void balanced_range(const LevelPlan* __restrict__ plan, uint32_t n_seg, uint32_t V,
                                               uint32_t g, uint32_t G, uint32_t lambda, uint32_t& rb, uint32_t& re) {
    const uint64_t T = (uint64_t)V + (uint64_t)lambda * (n_seg - 1);
    rb = g == 0 ? 0u : cost_inverse(plan, n_seg, V, lambda, T * g / G);
    re = g + 1 == G ? V : cost_inverse(plan, n_seg, V, lambda, T * (g + 1) / G);
}

// The segment of the idx list that position rb falls in: the last s with seg_begin[s] <= rb
// (seg_begin is non-decreasing, seg_begin[0] = 0), by binary search -- a few dependent loads of
// the plan instead of one per segment before rb.
__device__ __forceinline__ uint32_t first_segment(const LevelPlan* __restrict__ plan, uint32_t n_seg, uint32_t rb) {
    uint32_t lo = 0, hi = n_seg;   // answer in [lo, hi)
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) / 2;
        if (plan->seg_begin[mid] <= rb) lo = mid;
        else hi = mid;
    }
    return lo;
}

struct SampleParams {
    int32_t kind;             // 0 none, 1 Bayesian, 2 Bernoulli
    float temperature;
    double rate;              // (double)(float)subsample
    uint64_t bayes_seed;
    Rng bern;                 // main-stream state before the n Bernoulli draws
};

// ---------------------------------------------------------------------------------
// wave64 helpers
// ---------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

__device__ __forceinline__ uint32_t mbcnt64(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ unsigned long long wave_sum_u64(unsigned long long v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// ---------------------------------------------------------------------------------
// zero fill (graph-safe replacement for memset)
// ---------------------------------------------------------------------------------
static __global__ void zero_u32_kernel(uint32_t* __restrict__ p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

static __global__ void zero_i64_kernel(long long* __restrict__ p, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) p[i] = 0;
}

// ---------------------------------------------------------------------------------
// Bin packing: feature-major u8 [F][n] -> row-major words [n][W].
// ---------------------------------------------------------------------------------
static __global__ void pack_rows_kernel(const uint8_t* __restrict__ cols, uint64_t n, uint32_t F,
                                 uint32_t W, uint32_t* __restrict__ rows) {
    uint64_t total = n * W;
    for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (uint64_t)gridDim.x * blockDim.x) {
        uint64_t i = t / W;
        uint32_t w = (uint32_t)(t % W);
        uint32_t word = 0;
        for (uint32_t k = 0; k < 4; ++k) {
            uint32_t f = 4 * w + k;
            if (f < F) word |= (uint32_t)cols[(size_t)f * n + i] << (8 * k);
        }
        rows[t] = word;
    }
}

// Tile-major packing for the tiled fills: tile t (words [M t, M t + TW_t), TW_t = min(M,
// W - M t), M the words of a full tile) of row r at trows[n * M t + r * TS_t + w], so a
// workgroup of a tile streams its rows contiguously.  TS_t = 2^(shift - 2) words: M for a full
// tile, the next power of two of TW for a narrow last tile (its padding words are zero), so a
// row's offset is one shift whatever the tile.
__host__ __device__ inline uint32_t packed_slice_shift(uint32_t TW) {
    uint32_t sh = 2;
    while ((1u << sh) < 4u * TW) ++sh;
    return sh;
}
__host__ __device__ inline uint32_t packed_slice_words(uint32_t TW) { return 1u << (packed_slice_shift(TW) - 2); }

// TWM: words of a full tile (16 for the packed fill's 64-feature tiles, 8 for the exact fill's
// 32-feature tiles).
static __global__ void pack_tiles_kernel(const uint8_t* __restrict__ cols, uint64_t n, uint32_t F, uint32_t W,
                                         uint32_t* __restrict__ trows, uint64_t total /* words of trows */,
                                         uint32_t TWM) {
    for (uint64_t o = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total;
         o += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t t = (uint32_t)(o / (n * TWM));
        const uint32_t w0 = TWM * t;
        const uint32_t TS = packed_slice_words(min(TWM, W - w0));   // words per row in the slice
        const uint64_t rem = o - (uint64_t)n * w0;
        const uint64_t r = rem / TS;
        const uint32_t w = (uint32_t)(rem - r * TS) + w0;
        uint32_t word = 0;
        for (uint32_t k = 0; k < 4; ++k) {
            const uint32_t f = 4 * w + k;
            if (w < W && f < F) word |= (uint32_t)cols[(size_t)f * n + r] << (8 * k);
        }
        trows[o] = word;
    }
}

// ---------------------------------------------------------------------------------
// Derivatives (crates/cb-compute/src/loss.rs:35-80, 424-486).
// ---------------------------------------------------------------------------------
__device__ __forceinline__ void scalar_ders(int loss, double a, double t, double& d1, double& d2) {
    if (loss == 0) {          // RMSE
        d1 = t - a;
        d2 = -1.0;
    } else {                  // Logloss / CrossEntropy: p = 1 - 1/(1+e^a)
        double e = exp(a);
        double p = 1.0 - 1.0 / (1.0 + e);
        d1 = t - p;
        d2 = -p * (1.0 - p);
    }
}

template <int K>
__device__ __forceinline__ void softmax_probs(const double* a, double* p) {
    double mx = -INFINITY;
#pragma unroll
    for (int d = 0; d < K; ++d) mx = a[d] > mx ? a[d] : mx;
    double sum = 0.0;
#pragma unroll
    for (int d = 0; d < K; ++d) p[d] = exp(a[d] - mx);
#pragma unroll
    for (int d = 0; d < K; ++d) sum += p[d];
#pragma unroll
    for (int d = 0; d < K; ++d) p[d] = p[d] / sum;
}

// ---------------------------------------------------------------------------------
// RNG stream positions.  Advancing a PCG/LCG stream by j draws is the affine map
// x -> A^j x + c (A^j - 1)/(A - 1); the session precomputes (A^j, (A^j-1)/(A-1)) for
// j < 1024 (fine) and for j = 1024 q (coarse), so a row's stream position costs two
// table lookups and four 64-bit multiplies instead of a log-time jump.
// ---------------------------------------------------------------------------------
struct JumpTabs {
    const uint64_t* fine_a;
    const uint64_t* fine_d;
    const uint64_t* coarse_a;
    const uint64_t* coarse_d;
};

__device__ __forceinline__ void rng_jump(Rng& r, uint64_t a, uint64_t d) {
    r.x1 = a * r.x1 + r.c1 * d;
    r.x2 = a * r.x2 + r.c2 * d;
}

// Bootstrap sample of row i (bootstrap.rs:141-184): Bayesian rows of block b = i / 1000
// draw from TFastRng64(seed + b) advanced by 10 + (i % 1000); Bernoulli row i is draw i of
// the main stream.
__device__ __forceinline__ void sample_row(const SampleParams& smp, const JumpTabs& jt, uint64_t i,
                                           double& s, bool& ctrl) {
    s = 1.0;
    ctrl = true;
    if (smp.kind == 1) {
        Rng r = rng_from_seed(smp.bayes_seed + i / 1000);
        const uint32_t j = 10u + (uint32_t)(i % 1000);
        rng_jump(r, jt.fine_a[j], jt.fine_d[j]);
        const double u = rng_real1(r);
        const float bw = -fast_logf((float)u + 0.0f);  // 1e-100f rounds to 0 in f32
        s = smp.temperature == 1.0f ? (double)bw : (double)powf(bw, smp.temperature);
    } else if (smp.kind == 2) {
        Rng r = smp.bern;
        rng_jump(r, jt.fine_a[i & 1023u], jt.fine_d[i & 1023u]);
        rng_jump(r, jt.coarse_a[i >> 10], jt.coarse_d[i >> 10]);
        ctrl = rng_real1(r) < smp.rate;
    }
}

// ---------------------------------------------------------------------------------
// Per-tree preparation: apply the previous tree (approx += lr * leaf), derivatives,
// bootstrap sample, score channels, leaf flags, and per-block partial bounds for the
// fixed-point scales (summed deterministically by scales_kernel).
// ---------------------------------------------------------------------------------
constexpr int kPrepBlocks = 2048;
constexpr int kPartials = 8;   // per block: 4 bounds, sampled rows, 3 spare

template <int K>
static __global__ __launch_bounds__(256) void prepare_kernel(
    uint64_t n, int loss, double* __restrict__ approx, const double* __restrict__ target,
    const double* __restrict__ weight, uint16_t* __restrict__ leaf,
    const double* __restrict__ pending /* [leaves][K] lr-scaled, nullable */,
    const SampleParams* __restrict__ smpp, JumpTabs jt, const double* __restrict__ host_sample,
    double* __restrict__ sstat /* [n][K+1] */, int newton,
    unsigned long long* __restrict__ partials /* [gridDim.x][kPartials] */,
    const double* __restrict__ ext_der /* nullable [2][n]: der1, der2 of a pair loss */,
    const double* __restrict__ score_w /* nullable [n]: histogram weight (pairwise weights) */) {
    constexpr int C = K + 1;
    __shared__ unsigned long long red[4][kPartials];
    unsigned long long acc[kPartials] = {0, 0, 0, 0, 0, 0, 0, 0};
    const double bscale = (double)(1 << kBoundShift);
    // the tree's sampling parameters live in device memory, so a recorded launch sequence
    // replays unchanged from tree to tree
    const SampleParams smp = *smpp;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        double a[K];
#pragma unroll
        for (int d = 0; d < K; ++d) a[d] = approx[(size_t)d * n + i];
        if (pending) {
            const uint32_t l = leaf[i] & 0x7FFFu;
#pragma unroll
            for (int d = 0; d < K; ++d) {
                a[d] += pending[(size_t)l * K + d];
                approx[(size_t)d * n + i] = a[d];
            }
        }
        const double t = target[i];
        const double w = weight ? weight[i] : 1.0;
        double d1[K];
        double h_leaf;  // leaf weight channel bound: w (Gradient) or |der2 * w| (Newton)
        // histogram / Gradient-leaf weight: the pairwise weight for a pair loss
        // (eff_weights, boosting.rs:7575-7579), else the object weight
        const double hw = score_w ? score_w[i] : w;
        if (K == 1) {
            double g, h;
            if (ext_der) {
                g = ext_der[i];
                h = ext_der[n + i];
            } else {
                scalar_ders(loss, a[0], t, g, h);
            }
            d1[0] = g;
            h_leaf = newton ? fabs(h * w) : fabs(hw);
        } else {
            double p[K];
            softmax_probs<K>(a, p);
#pragma unroll
            for (int d = 0; d < K; ++d) d1[d] = -p[d];
            const int tc = (int)t;
            if (tc >= 0 && tc < K) d1[tc] += 1.0;
            h_leaf = fabs(w);
        }
        double s;
        bool ctrl;
        if (host_sample) {
            s = host_sample[i];
            ctrl = true;
        } else {
            sample_row(smp, jt, i, s, ctrl);
        }
        double mx_sd = 0.0, mx_ld = 0.0;
#pragma unroll
        for (int d = 0; d < K; ++d) {
            const double wd = d1[d] * w;             // weighted_der1 (boosting.rs:7479)
            const double sd = ctrl ? wd * s : 0.0;   // score_weighted_der1 (:7709)
            sstat[i * C + d] = sd;
            mx_sd = fmax(mx_sd, fabs(sd));
            mx_ld = fmax(mx_ld, fabs(wd));
        }
        const double sw = ctrl ? hw * s : 0.0;       // score_weights (:7728)
        sstat[i * C + K] = sw;
        leaf[i] = sw == 0.0 ? (uint16_t)0x8000u : (uint16_t)0;
        const unsigned long long qsd = (unsigned long long)ceil(mx_sd * bscale);
        const unsigned long long qsw = (unsigned long long)ceil(fabs(sw) * bscale);
        acc[kScoreDer] += qsd;
        acc[kScoreW] += qsw;
        acc[kLeafDer] += (unsigned long long)ceil(mx_ld * bscale);
        acc[kLeafW] += (unsigned long long)ceil(h_leaf * bscale);
        acc[4] += sw != 0.0;
        acc[5] = qsd > acc[5] ? qsd : acc[5];   // per-row maxima (the packed fill's scales)
        acc[6] = qsw > acc[6] ? qsw : acc[6];
    }
    const uint32_t wave = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < kPartials; ++k) {
        unsigned long long v = acc[k];
        if (k == 5 || k == 6) {
            for (int o = 32; o > 0; o >>= 1) {
                const unsigned long long u = __shfl_xor(v, o, 64);
                v = u > v ? u : v;
            }
        } else {
            v = wave_sum_u64(v);
        }
        if (lane_id() == 0) red[wave][k] = v;
    }
    __syncthreads();
    if (threadIdx.x < kPartials) {
        unsigned long long v = 0;
        const bool mx = threadIdx.x == 5 || threadIdx.x == 6;
        for (int w = 0; w < 4; ++w) {
            const unsigned long long u = red[w][threadIdx.x];
            v = mx ? (u > v ? u : v) : v + u;
        }
        partials[(size_t)blockIdx.x * kPartials + threadIdx.x] = v;
    }
}

// Count-packed fill (K == 1, integer score weights).  A row's two score channels travel in
// one 64-bit word p = q_der * 2^k + q_w (mod 2^64): q_w the row's integer score weight (0 or 1
// without object weights) in the low k bits, q_der = round(der * w * s * 2^S) in the high
// 64 - k bits.  A cell decodes as lo = p mod 2^k (a sum of non-negative weights: it never
// borrows from the der field) and der = (p - lo) / 2^k, exactly, while at most D rows have
// landed since the cell was emptied: D * wmax < 2^k and D * max|q_der| < 2^(63 - k).  With
// swaps every `swap` blocks of 1024 rows, D = 2 * 1024 * swap (atomics of the next period may
// land before a swap).  The plan takes the longest swap period of 4, 2, 1 blocks whose der
// scale S = 62 - k - log2 D - e is at least 30 -- the reference's per-row resolution 2^-30
// (kernels.rs:4145-4150) -- for the largest row |der * w * s| < 2^e; failing that, one block
// and its S (every sum stays exact; only the per-row step is coarser).
struct CountPack {
    int k, swap, shift;
};
__host__ __device__ inline CountPack count_pack_plan(int e, unsigned long long wmax) {
    CountPack cp{1, 1, 0};
    for (int sw = 4; sw >= 1; sw >>= 1) {
        const int lg = sw == 4 ? 13 : sw == 2 ? 12 : 11;   // log2 D
        int k = 1;
        while (k < 40 && (1ull << k) <= (wmax << lg)) ++k;   // D * wmax < 2^k
        cp = CountPack{k, sw, 62 - k - lg - e};
        if (cp.shift >= 30) break;
    }
    return cp;
}

// Sum the per-block partials (integers: exact in any order) and pick S per slot so that
// 2^S * sum|v| <= 2^61: no partial sum of rounded values can overflow int64.  With
// pack_bits > 0 the two score slots instead take S = pack_bits - e for the largest row
// bound M < 2^e, so every rounded row value fits pack_bits bits (|q| <= 2^pack_bits): the
// rounded packed fill's 32-bit fields.  With count set (the count-packed fill: integer score
// weights) the weight slot takes S = 0 (the weights themselves) and the der slot the finest
// scale whose packed cells stay decodable (count_pack_plan).
static __global__ __launch_bounds__(256) void scales_kernel(const unsigned long long* __restrict__ partials,
                                                           uint32_t n_blocks, Bounds* __restrict__ b,
                                                           Scales* __restrict__ sc, int pack_bits, int count) {
    __shared__ unsigned long long red[4][7];   // per wave (256 threads)
    unsigned long long acc[7] = {0, 0, 0, 0, 0, 0, 0};
    for (uint32_t i = threadIdx.x; i < n_blocks; i += blockDim.x) {
        for (int k = 0; k < 5; ++k) acc[k] += partials[(size_t)i * kPartials + k];
        for (int k = 5; k < 7; ++k) {
            const unsigned long long u = partials[(size_t)i * kPartials + k];
            acc[k] = u > acc[k] ? u : acc[k];
        }
    }
    // integer sums and maxima: any order gives the same values
    const uint32_t wave = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < 7; ++k) {
        unsigned long long v = acc[k];
        if (k < 5) {
            v = wave_sum_u64(v);
        } else {
            for (int o = 32; o > 0; o >>= 1) {
                const unsigned long long u = __shfl_xor(v, o, 64);
                v = u > v ? u : v;
            }
        }
        if (lane_id() == 0) red[wave][k] = v;
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (int k = 0; k < 7; ++k) {
        unsigned long long v = 0;
        for (uint32_t w = 0; w < blockDim.x / 64; ++w) {
            const unsigned long long u = red[w][k];
            v = k < 5 ? v + u : (u > v ? u : v);
        }
        acc[k] = v;
    }
    for (int k = 0; k < kNumScales; ++k) b->sum_abs[k] = acc[k];
    b->sampled_rows = acc[4];
    b->device_err = 0;   // the tree's kernels after this one report a failed bounded wait here
    for (int k = 0; k < kNumScales; ++k) {
        const bool packed = pack_bits > 0 && (k == kScoreDer || k == kScoreW);
        const double bound = (double)acc[packed ? 5 + k : k] / (double)(1 << kBoundShift);
        int e = -20;
        if (bound > 0.0) frexp(bound, &e);   // bound < 2^e
        int s = (packed ? pack_bits : 61) - e;
        if (s > 100) s = 100;
        if (count && k == kScoreW) s = 0;
        if (count && k == kScoreDer) {
            int mx = -20;   // largest row |der * w * s| < 2^mx
            const double mb = (double)acc[5] / (double)(1 << kBoundShift);
            if (mb > 0.0) frexp(mb, &mx);
            const CountPack cp = count_pack_plan(mx, acc[6] >> kBoundShift);
            s = min(s, cp.shift);
            sc->pk_k = cp.k;
            sc->pk_swap = cp.swap;
        }
        sc->shift[k] = s;
        sc->mul[k] = ldexp(1.0, s);
        sc->inv[k] = ldexp(1.0, -s);
    }
}

// Score channels f64 -> fixed point, in place ([n][C] doubles become [n][C] int64), once
// per tree, so the fill's inner loop only moves integers.
template <int C>
static __global__ void quantize_stats_kernel(double* __restrict__ sstat, uint64_t n,
                                             const Scales* __restrict__ sc) {
    const double md = sc->mul[kScoreDer], mw = sc->mul[kScoreW];
    long long* out = (long long*)sstat;
    const uint64_t total = n * C;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t ch = (uint32_t)(i % C);
        out[i] = to_fixed(sstat[i], ch == C - 1 ? mw : md);
    }
}

// ---------------------------------------------------------------------------------
// Histogram fill.  One workgroup = (feature tile, row range); it accumulates
// round(v * 2^S) of its rows into an LDS histogram of its feature tile with 64-bit integer
// LDS atomics, then flushes non-zero cells into the level histogram with 64-bit global
// atomics (integer adds: any order gives the same bits).  The blockIdx -> (tile, range)
// map keeps all tiles of a range on one XCD (blocks are dealt to the 8 XCDs round-robin),
// so the rows a range reads are fetched into that XCD's L2 once and shared by its tiles.
//
// Lane layout (word per lane): a lane takes one 4-byte word (4 features) of a row; the
// TW lanes of a row cover the tile's words and a 1024-thread workgroup covers
// 1024 / TW rows per pass.  The VALU work per LDS atomic is a byte extract and an address
// add, so the loop runs at the LDS atomic rate: 64-bit LDS atomics with scattered
// addresses are the bound of this kernel on gfx950 (the stats are pre-quantized int64
// per row, so nothing is converted in the loop).  LDS histogram layout is [ch][f][bin].
// Every lane keeps kFillRows rows in flight.
// ---------------------------------------------------------------------------------
constexpr int kFillRows = 4;
constexpr uint32_t kFillSegmentCost = 1024;   // rows' worth of time a segment's flush costs (ranges)

struct FillTiles {       // host-side plan of the feature tiles
    uint32_t n_tiles;
    uint32_t tw;         // words (4 features) per tile
    uint32_t bin_major;  // LDS [ch][bin][f] with rotated visits (tw == 8)
    uint32_t pad2;
    size_t lds_bytes;
};

// layout: 0 feature-major, 1 bin-major where it pays (>= 4 channels, or many rows), 2 bin-major
// whenever it fits
inline FillTiles plan_fill_tiles(uint32_t F, uint32_t B, uint32_t C, size_t budget, int layout,
                                 uint64_t n_rows) {
    FillTiles t{0, 0, 0, 0, 0};
    const uint32_t W = (F + 3) / 4;
    const size_t per_word = (size_t)4 * B * C * sizeof(long long);
    const size_t max_words = budget / per_word;
    if (max_words == 0) return t;
    const bool pays = C >= 4 || n_rows >= (4u << 20);
    if ((layout == 2 || (layout == 1 && pays)) && max_words >= 8) {   // 32-feature tiles, bin-major
        t.tw = std::min<uint32_t>(8, W);
        t.n_tiles = (W + t.tw - 1) / t.tw;
        t.bin_major = 1;
        t.lds_bytes = (size_t)std::min<uint32_t>(4 * t.tw, F) * B * C * sizeof(long long);
        return t;
    }
    t.n_tiles = (uint32_t)((W + max_words - 1) / max_words);
    t.tw = (W + t.n_tiles - 1) / t.n_tiles;       // balanced tiles
    t.n_tiles = (W + t.tw - 1) / t.tw;
    t.lds_bytes = (size_t)std::min<uint32_t>(4 * t.tw, F) * B * C * sizeof(long long);
    return t;
}

// One workgroup per (feature tile, row range): the rows to histogram (all n rows at level
// 0, else the concatenated segments of the directly built children listed in idx) are
// split into G equal contiguous ranges; a workgroup walks its range and flushes its LDS
// histogram only when it crosses into the next segment (leaf) and at the end, so the
// global-atomic flush traffic is about G * tiles * cells per launch instead of one flush
// per small chunk.  G * tiles is sized to the number of workgroups the CUs hold at once.
// What a lane does with the 4 bytes of its word, fixed for the whole launch: visit order,
// byte shift, LDS cell offset, validity and dominant bin per visit.  Feature-major layout
// [ch][f][bin]: cell = f * B + bin, visits in byte order.  Bin-major layout [ch][bin][f]
// (tiles of 32 features, 8 lanes per row, 8 rows per wave): cell = bin * 32 + f, and each lane
// rotates its visit order by a function of (row, word), so one atomic instruction of a wave
// covers the 32 features of the tile twice and any 16 consecutive lanes hit 16 distinct
// features modulo 16 -- every bank pair takes the fewest lanes whatever the bins (the
// conflict-free rate of 64-bit LDS atomics, against scattered bins over [f][bin]).
struct FillLane {
    uint32_t sh[4], off[4], skip[4];
    bool ok[4];
    uint32_t bin_stride;
};

// CU: the channels filled, 0 .. CU-1 of the C a row holds (the others stay as they are)
template <int C, bool kSkip, int CU = C>
__device__ __forceinline__ void fill_range(const uint32_t* __restrict__ rows, uint32_t W,
                                           const uint32_t* __restrict__ idx,
                                           const long long* __restrict__ sfix, uint32_t beg,
                                           uint32_t end, uint32_t w0, uint32_t TW, uint32_t plane,
                                           unsigned long long* __restrict__ lds64,
                                           const FillLane& fl) {
    // rows in flight per lane: more for few channels (latency), fewer for many (registers)
    constexpr int U = C <= 3 ? 2 * kFillRows : (C > 12 ? 2 : kFillRows);
    const uint32_t rows_per_pass = blockDim.x / TW;
    const uint32_t r0 = threadIdx.x / TW;
    const uint32_t wl = threadIdx.x - r0 * TW;
    if (r0 >= rows_per_pass) return;
    for (uint32_t p0 = beg + r0; p0 < end; p0 += U * rows_per_pass) {
        uint32_t doc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t p = p0 + (uint32_t)u * rows_per_pass;
            doc[u] = p < end ? (idx ? idx[p] : p) : 0xFFFFFFFFu;
        }
        long long st[U][CU];
        uint32_t word[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (doc[u] != 0xFFFFFFFFu) {
                const long long* sp_ = sfix + (size_t)doc[u] * C;
#pragma unroll
                for (int ch = 0; ch < CU; ++ch) st[u][ch] = sp_[ch];
                word[u] = rows[(size_t)doc[u] * W + w0 + wl];
            } else {
#pragma unroll
                for (int ch = 0; ch < CU; ++ch) st[u][ch] = 0;
                word[u] = 0;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            bool zero = true;  // a row of zeros (outside the sample, padding) adds nothing
#pragma unroll
            for (int ch = 0; ch < CU; ++ch) zero &= st[u][ch] == 0;
            if (zero) continue;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (fl.ok[k]) {
                    const uint32_t bin = (word[u] >> fl.sh[k]) & 0xFFu;
                    if (kSkip && bin == fl.skip[k]) continue;   // dominant bin: rebuilt from the totals
                    unsigned long long* cell = lds64 + bin * fl.bin_stride + fl.off[k];
#pragma unroll
                    for (int ch = 0; ch < CU; ++ch)
                        atomicAdd(cell + (size_t)ch * plane, (unsigned long long)st[u][ch]);
                }
            }
        }
    }
}

template <int C, bool kSkip, int CU = C>   // CU: channels filled (hist keeps C per leaf)
static __global__ __launch_bounds__(1024) void fill_kernel(
    const uint32_t* __restrict__ rows, uint32_t W, uint32_t stride /* words per row in memory, >= W */,
    uint64_t n,
    const uint32_t* __restrict__ idx,                  // null: dense rows [0, n), leaf 0
    const LevelPlan* __restrict__ plan, const long long* __restrict__ sfix, uint32_t n_tiles,
    uint32_t tw, uint32_t F, uint32_t B, uint32_t G, long long* __restrict__ hist,
    const uint32_t* __restrict__ skip_bin /* nullable [F]: dominant bin left out, or >= B */,
    int bin_major /* LDS [ch][bin][f] with rotated visits (tw == 8), else [ch][f][bin] */) {
    extern __shared__ long long lds[];
    const uint32_t b = blockIdx.x;
    const uint32_t xcd = b & 7u, q = b >> 3;
    const uint32_t t = q % n_tiles;
    const uint32_t g = (q / n_tiles) * 8u + xcd;       // row range
    const uint32_t w0 = t * tw;
    const uint32_t TW = min(tw, W - w0);
    const uint32_t f0 = 4u * w0;
    const uint32_t TF = min(4u * TW, F - f0);
    const uint32_t plane = TF * B;                      // cells of one channel plane
    const uint32_t cells = plane * CU;
    for (uint32_t i = threadIdx.x; i < cells; i += blockDim.x) lds[i] = 0;
    __syncthreads();
    const uint32_t r0 = threadIdx.x / TW;
    const uint32_t wl = threadIdx.x - r0 * TW;
    const uint32_t nf = min(4u, TF - min(TF, 4u * wl));   // valid features of this lane's word
    FillLane fl;
    fl.bin_stride = bin_major ? TF : 1u;
    // visit rotation: within every 16 lanes (2 rows x 8 words) and every 32 lanes (4 rows)
    // the features of one step are distinct modulo 16 and 32 (bank pairs at 32 and 64 banks)
    const uint32_t rot = bin_major ? ((2u * (r0 & 1u) + ((wl >> 2) ^ ((r0 >> 1) & 1u))) & 3u) : 0u;
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) {   // constant indices: the tables stay in registers
        const uint32_t kb = (k + rot) & 3u;   // byte visited at step k
        const uint32_t f = 4u * wl + kb;
        fl.sh[k] = 8u * kb;
        fl.off[k] = bin_major ? f : f * B;
        fl.ok[k] = kb < nf;
        fl.skip[k] = (kSkip && kb < nf) ? skip_bin[f0 + f] : 256u;
    }
    const uint32_t V = idx ? plan->rows : (uint32_t)n;
    const uint32_t n_seg = idx ? plan->n_parent : 1u;
    uint32_t rb = (uint32_t)(((uint64_t)V * g) / G), re = (uint32_t)(((uint64_t)V * (g + 1)) / G);
    if (idx) balanced_range(plan, n_seg, V, g, G, kFillSegmentCost, rb, re);
    uint32_t seg = 0;
    if (idx)
        seg = first_segment(plan, n_seg, rb);
    uint32_t pos = rb;
    while (pos < re) {
        const uint32_t seg_end = (idx && seg + 1 < n_seg) ? plan->seg_begin[seg + 1] : V;
        const uint32_t end = min(re, seg_end);
        const uint32_t slot = idx ? plan->built[seg] : 0u;
        if (end > pos) {
            fill_range<C, kSkip, CU>(rows, stride, idx, sfix, pos, end, w0, TW, plane, (unsigned long long*)lds, fl);
            __syncthreads();
            // flush LDS -> hist[leaf][ch][f0 + f][bin]
            if (!bin_major) {   // [ch][f][bin]: i is the global order (coalesced atomics)
                for (uint32_t i = threadIdx.x; i < cells; i += blockDim.x) {
                    const long long v = lds[i];
                    if (v != 0) {
                        const uint32_t ch = i / plane;
                        const uint32_t r = i - ch * plane;
                        unsigned long long* dst = (unsigned long long*)hist +
                            (((size_t)slot * C + ch) * F + f0) * B + r;
                        atomicAdd(dst, (unsigned long long)v);
                        lds[i] = 0;
                    }
                }
            } else {   // [ch][bin][f]: a wave takes 8 features x 8 bins (8-way LDS conflicts,
                       // 64-byte runs of bins in the global histogram)
                const uint32_t nfb = (TF + 7) / 8, nbb = (B + 7) / 8;
                const uint32_t vcells = CU * nfb * nbb * 64;
                for (uint32_t i = threadIdx.x; i < vcells; i += blockDim.x) {
                    const uint32_t l = i & 63u, j = i >> 6;
                    const uint32_t ch = j / (nfb * nbb), jb = j - ch * (nfb * nbb);
                    const uint32_t f = (jb / nbb) * 8 + (l >> 3), bin = (jb % nbb) * 8 + (l & 7u);
                    if (f >= TF || bin >= B) continue;
                    const uint32_t li = ch * plane + bin * TF + f;
                    const long long v = lds[li];
                    if (v != 0) {
                        unsigned long long* dst = (unsigned long long*)hist +
                            (((size_t)slot * C + ch) * F + f0 + f) * B + bin;
                        atomicAdd(dst, (unsigned long long)v);
                        lds[li] = 0;
                    }
                }
            }
            __syncthreads();
        }
        pos = end;
        ++seg;
    }
}

// ---------------------------------------------------------------------------------
// Packed fill (two score channels, K == 1).  A row's two fixed-point channels travel in one
// 64-bit word, p = q_der * 2^32 + q_w (mod 2^64) with |q| <= 2^pack_bits - 1 (rounded on a scale
// set by the largest row, then clamped), so ONE 64-bit LDS atomic per (row, feature) adds both
// channels.  The 32-bit fields of an LDS cell stay exactly decodable while the contributions
// that landed since the cell was last emptied sum to less than 2^31 in magnitude (q_w >= 0, so
// the weight field never borrows).  Every thread owns kPackOwn cells of the tile and swaps them
// with zero (ds_wrxchg) after the barrier that ends every swap period of swap_every blocks of
// kPackIterRows rows; atomics of threads already in the next period may land before the swap,
// so at most R = 2 * swap_every * kPackIterRows rows fall between two swaps of a cell, and
// pack_bits = 31 - log2(R) keeps every field sum within R * (2^pack_bits - 1) < 2^31.  The
// swapped words are decoded into int64 registers, which flush to the level histogram at
// segment ends.  Every sum stays an exact integer (order-free, reproducible); only the per-row
// quantization step is coarser than the two-atomic fill's (2^-pack_bits of the largest row
// instead of 2^-61 of the sum).
//
// Tiles are 64 features (16 words): a workgroup reads one aligned 64-byte sector of every
// 256-byte padded row it visits, so no two tiles share a sector and the gathers of the deeper
// levels fetch no bytes they do not use.  LDS layout [bin][64] (stride 64 whatever the tile
// width): a wave covers 4 rows x 16 words; the lane of word w of row r visits the bytes of its
// word starting at byte (w / 4 + r) mod 4, so every 16 consecutive lanes of an atomic
// instruction touch 16 distinct features mod 16 (32 lanes: 32 distinct mod 32), i.e. distinct
// bank pairs -- the conflict-free rate whatever the bins.
// ---------------------------------------------------------------------------------
constexpr uint32_t kPackTileWords = 16;
constexpr uint32_t kPackStride = 64;        // LDS cells per bin row
constexpr uint32_t kPackThreads = 1024;     // 16 waves, one workgroup per CU
constexpr uint32_t kPackIterRows = 1024;    // rows of the workgroup per block (between two swaps)
constexpr int kPackOwn = 16;                // cells per thread: 64 x 256 / 1024
constexpr uint32_t kPackCells = kPackStride * 256;   // LDS cells of a packed tile (any B <= 256)
static_assert(kPackOwn * kPackThreads == kPackCells, "every thread owns kPackOwn cells");
// pack_bits for swap_every = 1 (2 * 1024 rows between swaps): 2^11 * (2^20 - 1) < 2^31; each
// doubling of swap_every takes one bit
constexpr int kPackBitsSwap1 = 20;
constexpr int kPackHalf = 8;                // passes per half block of a full tile (64 rows each)
constexpr uint32_t kPackSegmentCost = 2048;  // rows' worth of time a segment's flush costs (ranges)

// Decode a swapped cell: no weight is negative (the session checks), so the weight field is a
// sum of non-negative values below 2^31 that never borrows from the der field.
__device__ __forceinline__ void unpack_add_nonneg(unsigned long long v, long long& acc_d, long long& acc_w) {
    acc_w += (long long)(uint32_t)v;
    acc_d += (long long)(int32_t)(uint32_t)(v >> 32);
}

// Level histogram flush of one channel: every thread stages its registers into the cells it
// owns, then the workgroup walks the tile 8 features x 8 bins per wave (64-byte runs of bins in
// the global histogram) with integer global atomics.
__device__ __forceinline__ void packed_flush_channel(unsigned long long* __restrict__ pk, const long long* acc,
                                                    uint32_t TF, uint32_t B, uint32_t F, uint32_t f0,
                                                    long long* __restrict__ dst_plane /* hist + ((slot*C+ch)*F)*B */,
                                                    uint32_t copies = 1, uint32_t cstride = 0 /* narrow tile */) {
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kPackOwn; ++k) pk[threadIdx.x + (uint32_t)k * kPackThreads] = (unsigned long long)acc[k];
    __syncthreads();
    const uint32_t nfb = (TF + 7) / 8, nbb = (B + 7) / 8;
    const uint32_t vcells = nfb * nbb * 64;
    for (uint32_t i = threadIdx.x; i < vcells; i += kPackThreads) {
        const uint32_t l = i & 63u, j = i >> 6;
        const uint32_t f = (j / nbb) * 8 + (l >> 3), bin = (j % nbb) * 8 + (l & 7u);
        if (f >= TF || bin >= B) continue;
        unsigned long long v = 0;
        for (uint32_t c = 0; c < copies; ++c) v += pk[bin * kPackStride + c * cstride + f];
        if (v != 0) atomicAdd((unsigned long long*)dst_plane + ((size_t)(f0 + f) * B + bin), v);
    }
}

// The four byte visits of one row's word.  Step k adds to the cell column at byte offset
// off8[k] = 8 (4 wl + b) the byte b of the word, b = (k + rot) & 3: v_bfe reads the low 5 bits
// of its offset operand, which are 8 b, so off8 doubles as the bit shift.  The lane's visit
// order (rotated by lane) spreads the lanes of an instruction over distinct bank pairs.
__device__ __forceinline__ void packed_row_atomics(unsigned long long* __restrict__ pk, uint32_t word,
                                                   const uint32_t* off8 /* byte offsets of the 4 columns */,
                                                   unsigned long long st) {
    char* base = (char*)pk;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t bin = __builtin_amdgcn_ubfe(word, off8[k], 8);   // bits [off8 & 31, +8)
        atomicAdd((unsigned long long*)(base + ((bin << 9) + off8[k])), st);   // [bin][64] x 8 bytes
    }
}

// Buffer loads at 32-bit byte offsets from a workgroup-uniform resource (one address register
// per load, no 64-bit address arithmetic; an offset past the resource's size reads 0).  The
// session keeps each buffer of the packed fill under 4 GiB.
constexpr int kBufWord3 = 0x00020000;   // gfx9 raw-buffer resource word 3
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                             (int)(uint32_t)(bytes < 0xFFFFFFFFull ? bytes : 0xFFFFFFFFull), kBufWord3);
}
__device__ __forceinline__ uint32_t ldw(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
constexpr uint32_t kPastEnd = 0xFFFFFFF0u;   // a byte offset past every packed-fill buffer

// A buffer load at a per-lane offset plus a workgroup-uniform one (soffset); callers keep the
// sum inside the resource.
__device__ __forceinline__ uint32_t ldw_s(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, (int)soff, 0);
}

__device__ __forceinline__ unsigned long long ldq(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
    return (unsigned long long)v[0] | ((unsigned long long)v[1] << 32);
}

// Decode a swapped cell of the count-packed fill: the weight field's low kb bits, the der
// field the rest (an arithmetic shift of the signed difference).
__device__ __forceinline__ void unpack_add_count(unsigned long long v, uint32_t kb, long long& acc_d,
                                                 long long& acc_w) {
    const unsigned long long lo = v & ((1ull << kb) - 1ull);
    acc_w += (long long)lo;
    acc_d += (long long)(v - lo) >> kb;
}

// Swap the cells a thread owns with zero and add their decoded fields to its registers.
// The cells of thread t are t + k * kPackThreads, k < kPackOwn: the LDS always holds 256 bin
// rows, so every thread owns kPackOwn cells and the swaps carry no per-cell branch (the LDS
// exchanges issue back to back and return together).  Cells of bins >= B, or of columns
// >= TF (the zero padding of a partial last word), are swapped too and never flushed.
// kCount: the count-packed encoding (weight field of kb bits), else the rounded one.
template <bool kCount>
__device__ __forceinline__ void packed_swap(unsigned long long* __restrict__ pk, uint32_t kb,
                                            long long (&acc_d)[kPackOwn], long long (&acc_w)[kPackOwn]) {
    unsigned long long* c = pk + threadIdx.x;
    constexpr int kBatch = 4;   // exchanges in flight: few registers beyond the accumulators
#pragma unroll
    for (int k0 = 0; k0 < kPackOwn; k0 += kBatch) {
        unsigned long long v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) v[j] = atomicExch(c + (uint32_t)(k0 + j) * kPackThreads, 0ull);
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            if (kCount) unpack_add_count(v[j], kb, acc_d[k0 + j], acc_w[k0 + j]);
            else unpack_add_nonneg(v[j], acc_d[k0 + j], acc_w[k0 + j]);
        }
    }
}

// Broadcast lane U of each 16-lane DPP row to the row (row_newbcast).
template <int U>
__device__ __forceinline__ uint32_t row_bcast(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x150 + U, 0xF, 0xF, true);
}
template <int U>
__device__ __forceinline__ unsigned long long row_bcast64(unsigned long long v) {   // one v_mov_b64_dpp
    return __builtin_amdgcn_update_dpp(0ull, v, 0x150 + U, 0xF, 0xF, true);
}

// The rows [pos, end) of a tile (up to 16 words: the 16 lanes of a row are one 16-lane DPP row
// of the wave), in blocks of kPackIterRows rows: DPP row r of the workgroup takes the 16
// consecutive positions q = base + 16 r .. q + 15 of a block, in two halves of 8.  Lane w of a
// DPP row loads the packed statistic (and, gathered, the row index) of position q + w; row u of
// the half broadcasts lane u to the DPP row's 16 lanes (row_newbcast), so statistics and indices
// cost one load per row and no LDS round trip -- the atomics of consecutive rows issue back to
// back.  At the dense level the 16 rows of a DPP row are consecutive in memory, so their word
// loads share one per-lane offset and differ by a uniform one: no per-row address arithmetic.
// Software pipeline: block j+1's statistics and indices are loaded when block j starts (indices
// two blocks ahead), and the words of a half of block j+1 right after that half of block j is
// consumed, so they are in flight across the other half, the barrier and the swap.  Positions
// past the range carry a zero statistic (their atomics add nothing).
template <bool kGather, bool kCount>
__device__ __forceinline__ void packed_range(unsigned long long* __restrict__ pk,
                                             __amdgpu_buffer_rsrc_t rbase, uint32_t sh, uint32_t wl4,
                                             uint32_t wl, __amdgpu_buffer_rsrc_t idx,
                                             __amdgpu_buffer_rsrc_t sbase, uint32_t pos, uint32_t end,
                                             uint32_t n, uint32_t r0, const uint32_t* off8,
                                             uint32_t swap_every, uint32_t kb,
                                             long long (&acc_d)[kPackOwn], long long (&acc_w)[kPackOwn]) {
    static_assert(2 * kPackHalf * 64 == kPackIterRows && kPackHalf == 8, "block layout");
    uint32_t six = 0, six_n = 0, six_nn = 0;
    unsigned long long ssv, ssv_n = 0;
    // the first position of this DPP row's 16 in the block at bb; at the dense level the rows
    // read are clamped to [0, n) as a group (q - qc positions before q are re-read with a zero
    // statistic), so every word load stays inside the tile's rows
    auto dense_q = [&](uint32_t bb) -> uint32_t {
        const uint32_t q = bb + 16u * r0;
        return q + 16u <= n ? q : n - 16u;
    };
    // this lane's position in the block at bb: gathered, its row index is staged two blocks
    // ahead, so the word loads that depend on it never wait for it; the statistic (stored in
    // position order) one block ahead.  A position outside the range reads its statistic from
    // past the end of the buffer, which returns 0 (buffer range checking), so no select waits on
    // the load
    auto stage_ix = [&](uint32_t bb) -> uint32_t {
        const uint32_t p = bb + 16u * r0 + wl;
        return ldw(idx, 4u * (p < end ? p : bb));
    };
    auto stage_sv = [&](uint32_t bb) -> unsigned long long {
        if (kGather) {
            const uint32_t p = bb + 16u * r0 + wl;
            return ldq(sbase, p < end ? 8u * p : kPastEnd);
        }
        const uint32_t q = bb + 16u * r0, p = dense_q(bb) + wl;
        return ldq(sbase, (p >= q && p < end) ? 8u * p : kPastEnd);
    };
    uint32_t wA[kPackHalf], wB[kPackHalf];
    uint32_t base = pos;
    if (kGather) {
        six = stage_ix(base);
        if (base + kPackIterRows < end) six_n = stage_ix(base + kPackIterRows);
    }
    ssv = stage_sv(base);
#define CBH_GLOAD(W, I, U, SIX) W[I] = ldw(rbase, (row_bcast<U>(SIX) << sh) + wl4);
#define CBH_DLOAD(W, I, U, OFF) W[I] = ldw_s(rbase, OFF, (uint32_t)(U) << sh);
#define CBH_LOADA(SIX, BB)                                                                    \
    if (kGather) {                                                                            \
        CBH_GLOAD(wA, 0, 0, SIX) CBH_GLOAD(wA, 1, 1, SIX) CBH_GLOAD(wA, 2, 2, SIX) CBH_GLOAD(wA, 3, 3, SIX) \
        CBH_GLOAD(wA, 4, 4, SIX) CBH_GLOAD(wA, 5, 5, SIX) CBH_GLOAD(wA, 6, 6, SIX) CBH_GLOAD(wA, 7, 7, SIX) \
    } else {                                                                                  \
        const uint32_t o = (dense_q(BB) << sh) + wl4;                                         \
        CBH_DLOAD(wA, 0, 0, o) CBH_DLOAD(wA, 1, 1, o) CBH_DLOAD(wA, 2, 2, o) CBH_DLOAD(wA, 3, 3, o) \
        CBH_DLOAD(wA, 4, 4, o) CBH_DLOAD(wA, 5, 5, o) CBH_DLOAD(wA, 6, 6, o) CBH_DLOAD(wA, 7, 7, o) \
    }
#define CBH_LOADB(SIX, BB)                                                                    \
    if (kGather) {                                                                            \
        CBH_GLOAD(wB, 0, 8, SIX) CBH_GLOAD(wB, 1, 9, SIX) CBH_GLOAD(wB, 2, 10, SIX) CBH_GLOAD(wB, 3, 11, SIX) \
        CBH_GLOAD(wB, 4, 12, SIX) CBH_GLOAD(wB, 5, 13, SIX) CBH_GLOAD(wB, 6, 14, SIX) CBH_GLOAD(wB, 7, 15, SIX) \
    } else {                                                                                  \
        const uint32_t o = (dense_q(BB) << sh) + wl4;                                         \
        CBH_DLOAD(wB, 0, 8, o) CBH_DLOAD(wB, 1, 9, o) CBH_DLOAD(wB, 2, 10, o) CBH_DLOAD(wB, 3, 11, o) \
        CBH_DLOAD(wB, 4, 12, o) CBH_DLOAD(wB, 5, 13, o) CBH_DLOAD(wB, 6, 14, o) CBH_DLOAD(wB, 7, 15, o) \
    }
#define CBH_ATOMS(W, U0, SSV)                                                                \
    packed_row_atomics(pk, W[0], off8, row_bcast64<U0 + 0>(SSV));                         \
    packed_row_atomics(pk, W[1], off8, row_bcast64<U0 + 1>(SSV));                         \
    packed_row_atomics(pk, W[2], off8, row_bcast64<U0 + 2>(SSV));                         \
    packed_row_atomics(pk, W[3], off8, row_bcast64<U0 + 3>(SSV));                         \
    packed_row_atomics(pk, W[4], off8, row_bcast64<U0 + 4>(SSV));                         \
    packed_row_atomics(pk, W[5], off8, row_bcast64<U0 + 5>(SSV));                         \
    packed_row_atomics(pk, W[6], off8, row_bcast64<U0 + 6>(SSV));                         \
    packed_row_atomics(pk, W[7], off8, row_bcast64<U0 + 7>(SSV));
    CBH_LOADA(six, base)
    CBH_LOADB(six, base)
    uint32_t blk = 0;
    for (;;) {   // workgroup-uniform
        const uint32_t nb = base + kPackIterRows;
        const bool more = nb < end;
        if (kGather && nb + kPackIterRows < end) six_nn = stage_ix(nb + kPackIterRows);
        if (more) ssv_n = stage_sv(nb);
        CBH_ATOMS(wA, 0, ssv)
        if (more) { CBH_LOADA(six_n, nb) }
        CBH_ATOMS(wB, 8, ssv)
        if (more) { CBH_LOADB(six_n, nb) }
        six_n = six_nn;
        ssv = ssv_n;
        if (++blk >= swap_every || !more) {
            blk = 0;
            __syncthreads();
            packed_swap<kCount>(pk, kb, acc_d, acc_w);
        }
        if (!more) break;
        base = nb;
    }
#undef CBH_ATOMS
#undef CBH_LOADB
#undef CBH_LOADA
#undef CBH_DLOAD
#undef CBH_GLOAD
}

// Broadcast lane 2 (i / 2) + U of each group of four lanes to lane i (DPP quad_perm
// [U, U, 2 + U, 2 + U]).
template <int U>
__device__ __forceinline__ uint32_t quad_pair_bcast(uint32_t v) {
    constexpr int ctrl = U | (U << 2) | ((2 + U) << 4) | ((2 + U) << 6);
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, ctrl, 0xF, 0xF, true);
}
template <int U>
__device__ __forceinline__ unsigned long long quad_pair_bcast64(unsigned long long v) {
    return (unsigned long long)quad_pair_bcast<U>((uint32_t)v) |
           ((unsigned long long)quad_pair_bcast<U>((uint32_t)(v >> 32)) << 32);
}

// The rows [pos, end) of a narrow last tile of 2 words at the dense level (a tile-major slice of
// 2 words per row): a 16-lane DPP row takes 8 rows per pass, lane wl = 2 j + w word w of row
// j, so every atomic instruction carries 64 useful lanes (the full tiles' loop would leave 14 of
// every 16 lanes on padding).  The LDS columns are the full tiles' (lane wl, step k: column
// 4 wl + ((k + rot) & 3)), i.e. 8 copies of the tile's 8 feature columns, one per row of a pass
// -- the same conflict-free bank pairs; the flush sums the copies.  The positions a DPP row
// covers in a block are the full tiles' (q .. q + 15, clamped into [0, n)), in 2 passes of 8:
// lane 2 j + w stages the statistic of position q + 8 w + j, and pass u broadcasts lane
// 2 j + u to lanes 2 j, 2 j + 1 (DPP quad_perm).  A block holds only 8 atomics per lane, so
// four blocks are in flight: four fixed register sets (words and statistic of a block), each
// reloaded right after its block is consumed.  Positions past the range read a zero statistic,
// so the loads of blocks past the end need no guard.  (At the gathered levels every listed row
// costs its own random line whatever the tile's width, so the narrow tile keeps the 16-lane
// loop there, in as many ranges as a full tile.)
struct NarrowSet {
    uint32_t w[2];                 // words of the set's block (passes 0, 1)
    unsigned long long sv;         // statistic of the staged position of the set's block
};

template <bool kCount>
__device__ __forceinline__ void packed_range_narrow(unsigned long long* __restrict__ pk,
                                                    __amdgpu_buffer_rsrc_t rbase, uint32_t sh,
                                                    __amdgpu_buffer_rsrc_t sbase, uint32_t pos, uint32_t end,
                                                    uint32_t n, uint32_t r0, uint32_t wl, const uint32_t* off8,
                                                    uint32_t swap_every, uint32_t kb,
                                                    long long (&acc_d)[kPackOwn], long long (&acc_w)[kPackOwn]) {
    constexpr uint32_t D = 4 * kPackIterRows;   // rows of four blocks
    const uint32_t j = wl >> 1, w = wl & 1u, w4 = 4u * w;
    auto qbase = [&](uint32_t bb) -> uint32_t {   // first row of this DPP row's 16, clamped into [0, n)
        const uint32_t q = bb + 16u * r0;
        return q + 16u <= n ? q : n - 16u;
    };
    auto stage_sv = [&](uint32_t bb) -> unsigned long long {   // this lane's staged position
        const uint32_t p = qbase(bb) + 8u * w + j;
        return ldq(sbase, (p < end && p >= bb + 16u * r0) ? 8u * p : kPastEnd);
    };
    auto load = [&](NarrowSet& S, uint32_t bb) {
        S.sv = stage_sv(bb);
        const uint32_t o = ((qbase(bb) + j) << sh) + w4;
        S.w[0] = ldw(rbase, o);
        S.w[1] = ldw(rbase, o + (8u << sh));
    };
    NarrowSet S0, S1, S2, S3;
    // the sets load in the loop's order (compiler memory barriers between them): the loop's first
    // use, set 0, then waits for set 0's loads only, on entry as on every later round
    load(S0, pos);
    asm volatile("" ::: "memory");
    load(S1, pos + kPackIterRows);
    asm volatile("" ::: "memory");
    load(S2, pos + 2 * kPackIterRows);
    asm volatile("" ::: "memory");
    load(S3, pos + 3 * kPackIterRows);
    asm volatile("" ::: "memory");
    // one block of a set: its atomics, then the set reloaded for the block four later.  The loop
    // runs whole rounds of four blocks (blocks past the range add zero statistics), so its body
    // has no exit between blocks and the loads of every set stay in flight across the round;
    // swaps come every swap_every blocks (a multiple of 4) and once after the last round.
    auto step = [&](NarrowSet& S, uint32_t bb) {
        packed_row_atomics(pk, S.w[0], off8, quad_pair_bcast64<0>(S.sv));
        packed_row_atomics(pk, S.w[1], off8, quad_pair_bcast64<1>(S.sv));
        load(S, bb + D);
    };
    const uint32_t rounds = (end - pos + D - 1) / D;
    const uint32_t swap_rounds = swap_every / 4;
    uint32_t base = pos;
    for (uint32_t rd = 0, since = 0; rd < rounds; ++rd, base += D) {
        step(S0, base);
        __builtin_amdgcn_sched_barrier(0);   // keep every set's reload in its own step
        step(S1, base + kPackIterRows);
        __builtin_amdgcn_sched_barrier(0);
        step(S2, base + 2 * kPackIterRows);
        __builtin_amdgcn_sched_barrier(0);
        step(S3, base + 3 * kPackIterRows);
        __builtin_amdgcn_sched_barrier(0);
        if (++since >= swap_rounds && rd + 1 < rounds) {
            since = 0;
            __syncthreads();
            packed_swap<kCount>(pk, kb, acc_d, acc_w);
        }
    }
    __syncthreads();
    packed_swap<kCount>(pk, kb, acc_d, acc_w);
}

template <bool kGather, bool kCount>
static __global__ __launch_bounds__(kPackThreads) void fill_packed_kernel(
    const uint32_t* __restrict__ rows /* tile-major (pack_tiles_kernel) */, uint32_t W,
    uint64_t n, const uint32_t* __restrict__ idx /* kGather: rows listed by the partition */,
    const LevelPlan* __restrict__ plan, const unsigned long long* __restrict__ spack /* [n] */,
    const unsigned long long* __restrict__ sseq /* nullable [V]: packed stats in idx order */,
    uint32_t n_tiles, uint32_t F, uint32_t B, uint32_t G, uint32_t Gn, long long* __restrict__ hist,
    uint32_t swap_every /* rounded: blocks of rows between two swaps: 2 * swap_every * kPackIterRows * 2^pack_bits <= 2^30 */,
    const uint32_t* __restrict__ rows_rm /* nullable, kGather: row-major words, 2^rm_sh bytes per row */,
    uint32_t rm_sh, const Scales* __restrict__ sc /* kCount: the tree's swap period and weight-field bits */) {
    constexpr uint32_t C = 2;
    extern __shared__ unsigned long long pk[];   // [B][64] packed cells
    // blocks: n_tiles tiles of the 16-lane row loop (64 features; the last one narrower when W
    // is not a multiple of 16 words and its slice is wider than 2 words: its row costs about as
    // much as a full one's), G row ranges each.  Workgroups go to the 8 XCDs round robin (block
    // b to XCD b % 8), so the (range, tile) pairs are numbered range-major and XCD x takes the
    // x-th run of per = ceil(n_tiles G / 8) of them: every tile of one range sits on one XCD, so
    // at the gathered levels the row-major lines of a listed row come from HBM once and from that
    // L2 for the other tiles, and no XCD holds more pairs than its CUs when n_tiles G fits the
    // resident slots (pairs past the last exit).  Then, when Gn > 0 (the dense level only), the
    // narrow last tile (tile n_tiles, 2 words) in Gn ranges of the narrow loop.
    const uint32_t pairs = n_tiles * G;
    const uint32_t per = (pairs + 7u) / 8u;
    const uint32_t b = blockIdx.x;
    const bool narrow = b >= 8u * per;
    uint32_t t, g, GR;
    if (!narrow) {
        const uint32_t i = (b & 7u) * per + (b >> 3);
        if (i >= pairs) return;   // workgroup-uniform, before any barrier
        t = i % n_tiles;
        g = i / n_tiles;
        GR = G;
    } else {
        t = n_tiles;
        g = b - 8u * per;
        GR = Gn;
        if (g >= Gn) return;
    }
    const uint32_t w0 = t * kPackTileWords;
    const uint32_t TW = min(kPackTileWords, W - w0);
    const uint32_t f0 = 4u * w0;
    const uint32_t TF = min(4u * TW, F - f0);
    // a row of this tile's tile-major slice: 2^sh bytes; gathered from row-major words: 2^rm_sh
    const bool rm = kGather && rows_rm != nullptr;
    const uint32_t sh = rm ? rm_sh : packed_slice_shift(TW);
    for (uint32_t i = threadIdx.x; i < kPackCells; i += kPackThreads) pk[i] = 0ull;
    // lanes: a 16-lane DPP row per row (the narrow loop: 16 / TW rows); in the 16-lane loop, a
    // tile narrower than 16 words has lanes past its words read the zero padding of the slice
    // (or the next row's words) and add to LDS columns >= TF, never read
    const uint32_t r0 = threadIdx.x / kPackTileWords;
    const uint32_t wl = threadIdx.x % kPackTileWords;
    // step k of a row visits byte (k + rot) & 3 of the lane's word: feature 4 * wl + ((k + rot) & 3).
    // rot = (wl / 4 + r) mod 4 makes the 16 lanes of a DPP row hit 16 distinct features mod 16
    // and any two DPP rows 32 distinct features mod 32, i.e. distinct bank pairs of the
    // [bin][64] cells whatever the bins.
    const uint32_t rot = ((wl >> 2) + (r0 & 1u)) & 3u;
    uint32_t off8[4];   // byte offset of the column of step k (its low 5 bits: the byte's bit shift)
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) off8[k] = 8u * (4u * wl + ((k + rot) & 3u));
    long long acc_d[kPackOwn], acc_w[kPackOwn];
#pragma unroll
    for (int k = 0; k < kPackOwn; ++k) acc_d[k] = acc_w[k] = 0;
    // the swap period and the weight field's bits: the count-packed fill takes the tree's (set on
    // the device by scales_kernel, so a replayed tree follows its own data)
    const uint32_t swap = kCount ? (uint32_t)sc->pk_swap : swap_every;
    const uint32_t kb = kCount ? (uint32_t)sc->pk_k : 0u;
    __syncthreads();
    const uint32_t V = kGather ? plan->rows : (uint32_t)n;
    const uint32_t n_seg = kGather ? plan->n_parent : 1u;
    uint32_t rb = (uint32_t)(((uint64_t)V * g) / GR), re = (uint32_t)(((uint64_t)V * (g + 1)) / GR);
    if (kGather) balanced_range(plan, n_seg, V, g, GR, kPackSegmentCost, rb, re);
    uint32_t seg = 0;
    if (kGather)
        seg = first_segment(plan, n_seg, rb);
    // tile-major rows: this tile's slice starts at word n * w0, 2^sh bytes per row; row-major:
    // word w0 of row 0, rows 2^sh bytes apart (a narrow tile's lanes past W read the row's zero
    // padding: rows are padded to whole 16-word multiples)
    const __amdgpu_buffer_rsrc_t rbase =
        rm ? make_rsrc(rows_rm + w0, ((uint64_t)n << sh) - 4ull * w0) : make_rsrc(rows + n * w0, (uint64_t)n << sh);
    const uint32_t wl4 = 4u * wl;
    const __amdgpu_buffer_rsrc_t sbase = make_rsrc(kGather ? sseq : spack, n * 8u);
    const __amdgpu_buffer_rsrc_t ibase = make_rsrc(kGather ? (const void*)idx : (const void*)spack, kGather ? n * 4u : 0u);
    uint32_t pos = rb;
    while (pos < re) {
        const uint32_t seg_end = (kGather && seg + 1 < n_seg) ? plan->seg_begin[seg + 1] : V;
        const uint32_t end = min(re, seg_end);
        const uint32_t slot = kGather ? plan->built[seg] : 0u;
        if (end > pos) {
            if (kGather || !narrow)
                packed_range<kGather, kCount>(pk, rbase, sh, wl4, wl, ibase, sbase, pos, end, (uint32_t)n, r0, off8,
                                              swap, kb, acc_d, acc_w);
            else   // a cell takes 1/8 of the rows a full tile's does: swaps 8x rarer
                packed_range_narrow<kCount>(pk, rbase, sh, sbase, pos, end, (uint32_t)n, r0, wl, off8, 8u * swap,
                                            kb, acc_d, acc_w);
            // every contribution of the segment is in the registers now (the last swap follows
            // the last barrier); flush both channels (a narrow tile's 16 / TW copies summed), then
            // clear the cells and registers
            long long* hd = hist + (size_t)slot * C * F * B;
            const uint32_t copies = narrow ? 16u / TW : 1u, cstride = 4u * TW;
            packed_flush_channel(pk, acc_d, TF, B, F, f0, hd, copies, cstride);
            packed_flush_channel(pk, acc_w, TF, B, F, f0, hd + (size_t)F * B, copies, cstride);
            __syncthreads();
#pragma unroll
            for (int k = 0; k < kPackOwn; ++k) {
                pk[threadIdx.x + (uint32_t)k * kPackThreads] = 0ull;
                acc_d[k] = acc_w[k] = 0;
            }
            __syncthreads();
        }
        pos = end;
        ++seg;
    }
}

// ---------------------------------------------------------------------------------
// Tiled exact fill (K == 1).  Both score channels keep the tree's full fixed-point scale
// (round(v * 2^S), S = 61 - ceil(log2 sum|v|) per channel, 2^-37 at config 2), one 64-bit LDS
// atomic per (row, feature, channel).  The LDS cells are exact int64 sums: nothing is rounded
// beyond the per-row quantization, no cell is swapped, and the tile flushes straight from LDS to
// the level histogram at segment ends.
//
// Tiles of 32 features (8 words); LDS [bin][ch][32] of u64, 512 bytes per bin, the weight cell
// of a column 256 bytes past its der cell (one immediate offset apart).  A 16-lane DPP row
// takes two rows per pass, lane 8 j + w word w of row j.  The 16 positions a DPP row covers in
// a block of 1024 are staged one per lane (16 bytes of statistics; gathered, the row index), and
// pass u broadcasts lane u to lanes 0-7 and lane 8 + u to lanes 8-15 (row_newbcast, the second
// under a bank mask), so a row's statistics cost one load and no LDS round trip.  Step k of a
// lane visits byte (k + rot) & 3 of its word, rot = (2 j + w / 4) mod 4: the 16 lanes of every
// atomic hit 16 distinct columns mod 16, i.e. distinct bank pairs whatever the bins.
//
// A last tile of at most 2 words runs the narrow loop: 8 rows per DPP row (lane 2 j + w word w
// of row j), four LDS copies of its 8 feature columns (copy j mod 4, summed at the flush), the
// statistics of a pass broadcast within lane quads (quad_perm), so its atomics carry 64 useful
// lanes instead of 16.
//
// Rows: the dense level streams each tile's tile-major slice, the gathered levels read the
// row-major words through the partition's index list (all tiles of a range on one XCD: a listed
// row's lines come from HBM once); statistics in position order ([n][2] f64, or the listed
// rows' copy in idx order written by the compaction), rounded onto the tree's fixed-point
// scales as a block's set is consumed (to_fixed, the score channels' rounding everywhere).
// ---------------------------------------------------------------------------------
constexpr uint32_t kExThreads = 1024;           // 16 waves, one workgroup per CU
constexpr uint32_t kExTileWords = 8;
constexpr uint32_t kExCells = 256u * 2u * 32u;   // [bin][ch][32] u64: 128 KiB
constexpr uint32_t kExBlockRows = 1024;         // positions of a block: 16 per DPP row
constexpr uint32_t kExSegmentCost = 1024;       // rows' worth of time a segment's flush costs (ranges)

// Lanes 0-7 of every DPP row take lane U of the row, lanes 8-15 lane 8 + U.
template <int U>
__device__ __forceinline__ unsigned long long half_bcast64(unsigned long long v) {
    const unsigned long long a = __builtin_amdgcn_update_dpp(0ull, v, 0x150 + U, 0xF, 0xF, true);
    return __builtin_amdgcn_update_dpp(a, v, 0x150 + 8 + U, 0xF, 0xC, false);
}
template <int U>
__device__ __forceinline__ uint32_t half_bcast32(uint32_t v) {
    const int a = __builtin_amdgcn_update_dpp(0, (int)v, 0x150 + U, 0xF, 0xF, true);
    return (uint32_t)__builtin_amdgcn_update_dpp(a, (int)v, 0x150 + 8 + U, 0xF, 0xC, false);
}

// The four byte visits of one row's word, both channels: off8[k] = 8 * column (its low 5 bits
// are the byte's bit shift, the v_bfe offset); der cell at bin * 512 + off8, weight cell 256
// bytes further.
__device__ __forceinline__ void exact_row_atomics(unsigned long long* __restrict__ ex, uint32_t word,
                                                  const uint32_t* off8, unsigned long long sd,
                                                  unsigned long long sw) {
    char* base = (char*)ex;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t bin = __builtin_amdgcn_ubfe(word, off8[k], 8);
        unsigned long long* c = (unsigned long long*)(base + ((bin << 9) + off8[k]));
        atomicAdd(c, sd);
        atomicAdd(c + 32, sw);
    }
}

// A 16-byte load at kPastEnd16 lies wholly past every buffer of the tiled exact fill (whose
// sizes the session keeps below 2^31 bytes) without wrapping the 32-bit offset: it returns 0.
constexpr uint32_t kPastEnd16 = 0xFFFFFFE0u;
__device__ __forceinline__ void ldq2(__amdgpu_buffer_rsrc_t r, uint32_t off, unsigned long long& a,
                                     unsigned long long& b) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    a = (unsigned long long)v[0] | ((unsigned long long)v[1] << 32);
    b = (unsigned long long)v[2] | ((unsigned long long)v[3] << 32);
}

// One block's worth of a DPP row in flight: the words of its 8 passes, the staged statistics and,
// gathered, the staged row index of the set's next block.
struct ExSet {
    uint32_t w[8];
    unsigned long long sd, sw;
    uint32_t ix;
};

template <int U>
__device__ __forceinline__ void exact_pass(unsigned long long* __restrict__ ex, const ExSet& S, const uint32_t* off8,
                                           unsigned long long qd, unsigned long long qw) {
    exact_row_atomics(ex, S.w[U], off8, half_bcast64<U>(qd), half_bcast64<U>(qw));
}

// A staged row's score channels: the f64 values (their bits as loaded) on the tree's fixed-point
// scales, round(v * 2^S) as the score channels are everywhere (to_fixed); a position past the
// range loaded 0 and stays 0.
__device__ __forceinline__ unsigned long long stat_fixed(unsigned long long bits, double mul) {
    return (unsigned long long)to_fixed(__longlong_as_double((long long)bits), mul);
}

// Positions [pos, end) of a full tile.  Two sets alternate: while one block's atomics issue, the
// next block's words and statistics are in flight; gathered, a set's row indices are staged a
// round (two blocks) before its words need them.  Blocks past the range read zero statistics
// (a buffer load past the resource returns 0) and, at the dense level, rows clamped into
// [0, n) in groups of 16; gathered, the indices of positions past the range repeat idx[pos].
template <bool kGather, int NS>
__device__ __forceinline__ void exact_range(unsigned long long* __restrict__ ex, __amdgpu_buffer_rsrc_t rbase,
                                            uint32_t sh, uint32_t wl4, uint32_t j8, uint32_t l,
                                            __amdgpu_buffer_rsrc_t ibase, __amdgpu_buffer_rsrc_t sbase,
                                            bool seq, uint32_t pos, uint32_t end, uint32_t n, uint32_t r0,
                                            const uint32_t* off8, double md, double mw) {
    auto q_of = [&](uint32_t bb) -> uint32_t { return bb + 16u * r0; };
    auto dense_q = [&](uint32_t bb) -> uint32_t {
        const uint32_t q = q_of(bb);
        return q + 16u <= n ? q : n - 16u;
    };
    auto stage_ix = [&](uint32_t bb) -> uint32_t {
        const uint32_t p = q_of(bb) + l;
        return ldw(ibase, 4u * (p < end ? p : pos));
    };
    auto load = [&](ExSet& S, uint32_t bb) {
        uint32_t p;
        bool ok;
        if (kGather) {
            p = q_of(bb) + l;
            ok = p < end;
        } else {
            p = dense_q(bb) + l;
            ok = p >= q_of(bb) && p < end;
        }
        // gathered: the statistics of the staged position, in idx order (seq) or through its row
        // index
        const uint32_t sp = (kGather && !seq) ? S.ix : p;
        ldq2(sbase, ok ? 16u * sp : kPastEnd16, S.sd, S.sw);
        if (kGather) {
            const uint32_t ix = S.ix;
            S.w[0] = ldw(rbase, (half_bcast32<0>(ix) << sh) + wl4);
            S.w[1] = ldw(rbase, (half_bcast32<1>(ix) << sh) + wl4);
            S.w[2] = ldw(rbase, (half_bcast32<2>(ix) << sh) + wl4);
            S.w[3] = ldw(rbase, (half_bcast32<3>(ix) << sh) + wl4);
            S.w[4] = ldw(rbase, (half_bcast32<4>(ix) << sh) + wl4);
            S.w[5] = ldw(rbase, (half_bcast32<5>(ix) << sh) + wl4);
            S.w[6] = ldw(rbase, (half_bcast32<6>(ix) << sh) + wl4);
            S.w[7] = ldw(rbase, (half_bcast32<7>(ix) << sh) + wl4);
            S.ix = stage_ix(bb + NS * kExBlockRows);
        } else {
            const uint32_t o = ((dense_q(bb) + j8) << sh) + wl4;
#pragma unroll
            for (uint32_t u = 0; u < 8; ++u) S.w[u] = ldw_s(rbase, o, u << sh);
        }
    };
    auto consume = [&](const ExSet& S) {
        const unsigned long long qd = stat_fixed(S.sd, md), qw = stat_fixed(S.sw, mw);
        exact_pass<0>(ex, S, off8, qd, qw);
        exact_pass<1>(ex, S, off8, qd, qw);
        exact_pass<2>(ex, S, off8, qd, qw);
        exact_pass<3>(ex, S, off8, qd, qw);
        exact_pass<4>(ex, S, off8, qd, qw);
        exact_pass<5>(ex, S, off8, qd, qw);
        exact_pass<6>(ex, S, off8, qd, qw);
        exact_pass<7>(ex, S, off8, qd, qw);
    };
    static_assert(NS >= 2 && NS <= 4, "two to four sets");
    ExSet S0, S1, S2, S3;
    if (kGather) {
        S0.ix = stage_ix(pos);
        S1.ix = stage_ix(pos + kExBlockRows);
        if (NS >= 3) S2.ix = stage_ix(pos + 2u * kExBlockRows);
        if (NS >= 4) S3.ix = stage_ix(pos + 3u * kExBlockRows);
    }
    load(S0, pos);
    load(S1, pos + kExBlockRows);
    if (NS >= 3) load(S2, pos + 2u * kExBlockRows);
    if (NS >= 4) load(S3, pos + 3u * kExBlockRows);
    for (uint32_t bb = pos;; bb += NS * kExBlockRows) {   // workgroup-uniform
        consume(S0);
        if (bb + kExBlockRows >= end) break;
        load(S0, bb + NS * kExBlockRows);
        consume(S1);
        if (bb + 2u * kExBlockRows >= end) break;
        load(S1, bb + (NS + 1) * kExBlockRows);
        if (NS >= 3) {
            consume(S2);
            if (bb + 3u * kExBlockRows >= end) break;
            load(S2, bb + (NS + 2) * kExBlockRows);
        }
        if (NS >= 4) {
            consume(S3);
            if (bb + 4u * kExBlockRows >= end) break;
            load(S3, bb + (NS + 3) * kExBlockRows);
        }
    }
}

// The narrow loop's set: the words of its 2 passes, staged statistics and row index.
struct ExNarrowSet {
    uint32_t w[2];
    unsigned long long sd, sw;
    uint32_t ix;
};

template <int U>
__device__ __forceinline__ void exact_narrow_pass(unsigned long long* __restrict__ ex, const ExNarrowSet& S,
                                                  const uint32_t* off8, unsigned long long qd, unsigned long long qw) {
    exact_row_atomics(ex, S.w[U], off8, quad_pair_bcast64<U>(qd), quad_pair_bcast64<U>(qw));
}

// Positions [pos, end) of a narrow last tile (at most 2 words).  A DPP row covers the same 16
// positions q .. q + 15 per block as in the full loop, in 2 passes of 8 rows: lane 2 j + w stages
// position q + 8 w + j, so pass u broadcasts lane 2 j + u to lanes 2 j, 2 j + 1 (quad_perm).  A
// block holds 16 atomics per lane, so four sets are in flight, each reloaded right after its
// block is consumed; gathered, a set's indices are staged a round (four blocks) ahead.
template <bool kGather>
__device__ __forceinline__ void exact_range_narrow(unsigned long long* __restrict__ ex, __amdgpu_buffer_rsrc_t rbase,
                                                   uint32_t sh, uint32_t wl4, uint32_t l,
                                                   __amdgpu_buffer_rsrc_t ibase, __amdgpu_buffer_rsrc_t sbase,
                                                   bool seq, uint32_t pos, uint32_t end, uint32_t n, uint32_t r0,
                                                   const uint32_t* off8, double md, double mw) {
    constexpr uint32_t NS = 4;
    const uint32_t j = l >> 1, stg = 8u * (l & 1u) + j;   // this lane's staged position in a block
    auto q_of = [&](uint32_t bb) -> uint32_t { return bb + 16u * r0; };
    auto dense_q = [&](uint32_t bb) -> uint32_t {
        const uint32_t q = q_of(bb);
        return q + 16u <= n ? q : n - 16u;
    };
    auto stage_ix = [&](uint32_t bb) -> uint32_t {
        const uint32_t p = q_of(bb) + stg;
        return ldw(ibase, 4u * (p < end ? p : pos));
    };
    auto load = [&](ExNarrowSet& S, uint32_t bb) {
        uint32_t p;
        bool ok;
        if (kGather) {
            p = q_of(bb) + stg;
            ok = p < end;
        } else {
            p = dense_q(bb) + stg;
            ok = p >= q_of(bb) && p < end;
        }
        const uint32_t sp = (kGather && !seq) ? S.ix : p;
        ldq2(sbase, ok ? 16u * sp : kPastEnd16, S.sd, S.sw);
        if (kGather) {
            const uint32_t ix = S.ix;
            S.w[0] = ldw(rbase, (quad_pair_bcast<0>(ix) << sh) + wl4);
            S.w[1] = ldw(rbase, (quad_pair_bcast<1>(ix) << sh) + wl4);
            S.ix = stage_ix(bb + NS * kExBlockRows);
        } else {
            const uint32_t o = ((dense_q(bb) + j) << sh) + wl4;
            S.w[0] = ldw(rbase, o);
            S.w[1] = ldw_s(rbase, o, 8u << sh);
        }
    };
    ExNarrowSet S0, S1, S2, S3;
    static_assert(NS == 4, "four sets");
    if (kGather) {
        S0.ix = stage_ix(pos);
        S1.ix = stage_ix(pos + kExBlockRows);
        S2.ix = stage_ix(pos + 2u * kExBlockRows);
        S3.ix = stage_ix(pos + 3u * kExBlockRows);
    }
    // the sets load in the loop's order (compiler memory barriers between them), so the loop's
    // first use waits for that set's loads only
    load(S0, pos);
    asm volatile("" ::: "memory");
    load(S1, pos + kExBlockRows);
    asm volatile("" ::: "memory");
    load(S2, pos + 2u * kExBlockRows);
    asm volatile("" ::: "memory");
    load(S3, pos + 3u * kExBlockRows);
    asm volatile("" ::: "memory");
    // one block of a set: its atomics, then (unless the range ends) the set reloaded for the block
    // four later
    auto step = [&](ExNarrowSet& S, uint32_t bb) -> bool {
        const unsigned long long qd = stat_fixed(S.sd, md), qw = stat_fixed(S.sw, mw);
        exact_narrow_pass<0>(ex, S, off8, qd, qw);
        exact_narrow_pass<1>(ex, S, off8, qd, qw);
        if (bb + kExBlockRows >= end) return true;
        load(S, bb + NS * kExBlockRows);
        return false;
    };
    for (uint32_t bb = pos;; bb += NS * kExBlockRows) {   // workgroup-uniform
        if (step(S0, bb)) break;
        if (step(S1, bb + kExBlockRows)) break;
        if (step(S2, bb + 2u * kExBlockRows)) break;
        if (step(S3, bb + 3u * kExBlockRows)) break;
    }
}

// Level histogram flush of the tile: a wave takes 8 features x 8 bins of one channel (64-byte
// runs of bins in the histogram); every cell is read and cleared by one thread (a narrow tile's
// copies summed).  Columns >= TF (lanes past a short tile's words) are never read.
__device__ __forceinline__ void exact_flush(unsigned long long* __restrict__ ex, uint32_t TF, uint32_t B,
                                            uint32_t F, uint32_t f0, long long* __restrict__ hd /* hist + slot*2*F*B */,
                                            uint32_t copies) {
    const uint32_t nfb = (TF + 7) / 8, nbb = (B + 7) / 8;
    const uint32_t per_ch = nfb * nbb;
    for (uint32_t i = threadIdx.x; i < 2u * per_ch * 64u; i += kExThreads) {
        const uint32_t lane = i & 63u, jj = i >> 6;
        const uint32_t ch = jj >= per_ch ? 1u : 0u, jb = jj - ch * per_ch;
        const uint32_t f = (jb / nbb) * 8 + (lane >> 3), bin = (jb % nbb) * 8 + (lane & 7u);
        if (f >= TF || bin >= B) continue;
        unsigned long long v = 0;
        for (uint32_t c = 0; c < copies; ++c) {
            unsigned long long* cell = ex + bin * 64u + ch * 32u + c * 8u + f;
            v += *cell;
            *cell = 0ull;
        }
        if (v != 0) atomicAdd((unsigned long long*)hd + ((size_t)(ch * F + f0 + f) * B + bin), v);
    }
}

template <bool kGather>
static __global__ __launch_bounds__(kExThreads) void fill_exact_kernel(
    const uint32_t* __restrict__ trows /* tile-major 8-word slices (pack_tiles_kernel) */, uint32_t W,
    uint64_t n, const uint32_t* __restrict__ idx /* kGather: rows listed by the partition */,
    const LevelPlan* __restrict__ plan, const long long* __restrict__ sfix /* [n][2] f64 score channels */,
    const long long* __restrict__ sseq /* kGather, nullable: [V][2], the listed rows' channels in idx order */,
    uint32_t n_tiles, uint32_t F, uint32_t B, uint32_t G, uint32_t Gn, long long* __restrict__ hist,
    const uint32_t* __restrict__ rows_rm /* nullable, kGather: row-major words, 2^rm_sh bytes per row */,
    uint32_t rm_sh, uint32_t sets /* blocks in flight of the full loop: 2 to 4 */,
    const Scales* __restrict__ sc /* the score channels' scales: sfix and sseq hold f64 values */) {
    extern __shared__ unsigned long long ex[];
    const double md = sc->mul[kScoreDer], mw = sc->mul[kScoreW];
    // blocks: n_tiles tiles of the 8-lane loop in G row ranges each, numbered range-major and
    // dealt to the 8 XCDs in runs (block b to XCD b % 8: XCD x takes pairs [x per, (x + 1) per)),
    // so all tiles of a range share one L2; then, when Gn > 0, the narrow last tile (tile
    // n_tiles) in Gn ranges of the narrow loop
    const uint32_t pairs = n_tiles * G;
    const uint32_t per = (pairs + 7u) / 8u;
    const uint32_t b = blockIdx.x;
    const bool narrow = b >= 8u * per;
    uint32_t t, g, GR;
    if (!narrow) {
        const uint32_t i = (b & 7u) * per + (b >> 3);
        if (i >= pairs) return;   // workgroup-uniform, before any barrier
        t = i % n_tiles;
        g = i / n_tiles;
        GR = G;
    } else {
        t = n_tiles;
        g = b - 8u * per;
        GR = Gn;
        if (g >= Gn) return;
    }
    const uint32_t w0 = t * kExTileWords;
    const uint32_t TW = min(kExTileWords, W - w0);
    const uint32_t f0 = 4u * w0;
    const uint32_t TF = min(4u * TW, F - f0);
    const bool rm = kGather && rows_rm != nullptr;
    const uint32_t sh = rm ? rm_sh : packed_slice_shift(TW);
    for (uint32_t i = threadIdx.x; i < kExCells; i += kExThreads) ex[i] = 0ull;
    const uint32_t r0 = threadIdx.x >> 4;   // DPP row of the workgroup
    const uint32_t l = threadIdx.x & 15u;   // lane in the DPP row
    uint32_t off8[4], wl4;
    if (!narrow) {
        const uint32_t j = l >> 3, w = l & 7u;
        const uint32_t rot = (2u * j + (w >> 2)) & 3u;
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) off8[k] = 8u * (4u * w + ((k + rot) & 3u));
        wl4 = 4u * w;
    } else {
        // lane 2 j + w: copy j mod 4 of the 8 columns, rot = j / 2, so the 16 lanes of an
        // atomic still hit 16 distinct columns mod 16
        const uint32_t j = l >> 1, w = l & 1u;
        const uint32_t rot = j >> 1;
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) off8[k] = 8u * (8u * (j & 3u) + 4u * w + ((k + rot) & 3u));
        wl4 = 4u * w;
    }
    __syncthreads();
    const uint32_t V = kGather ? plan->rows : (uint32_t)n;
    const uint32_t n_seg = kGather ? plan->n_parent : 1u;
    uint32_t rb = (uint32_t)(((uint64_t)V * g) / GR), re = (uint32_t)(((uint64_t)V * (g + 1)) / GR);
    if (kGather) balanced_range(plan, n_seg, V, g, GR, kExSegmentCost, rb, re);
    uint32_t seg = 0;
    if (kGather)
        seg = first_segment(plan, n_seg, rb);
    const __amdgpu_buffer_rsrc_t rbase = rm ? make_rsrc(rows_rm + w0, ((uint64_t)n << sh) - 4ull * w0)
                                            : make_rsrc(trows + n * w0, (uint64_t)n << sh);
    // gathered: statistics in idx order when the compaction wrote them (sseq), else through the
    // listed rows' indices
    const bool seq = kGather && sseq != nullptr;
    const __amdgpu_buffer_rsrc_t sbase = make_rsrc(seq ? (const void*)sseq : (const void*)sfix, n * 16u);
    const __amdgpu_buffer_rsrc_t ibase =
        make_rsrc(kGather ? (const void*)idx : (const void*)sfix, kGather ? n * 4u : 0u);
    uint32_t pos = rb;
    while (pos < re) {
        const uint32_t seg_end = (kGather && seg + 1 < n_seg) ? plan->seg_begin[seg + 1] : V;
        const uint32_t end = min(re, seg_end);
        const uint32_t slot = kGather ? plan->built[seg] : 0u;
        if (end > pos) {
            if (!narrow && sets == 4)
                exact_range<kGather, 4>(ex, rbase, sh, wl4, 8u * (l >> 3), l, ibase, sbase, seq, pos, end,
                                        (uint32_t)n, r0, off8, md, mw);
            else if (!narrow && sets == 3)
                exact_range<kGather, 3>(ex, rbase, sh, wl4, 8u * (l >> 3), l, ibase, sbase, seq, pos, end,
                                        (uint32_t)n, r0, off8, md, mw);
            else if (!narrow)
                exact_range<kGather, 2>(ex, rbase, sh, wl4, 8u * (l >> 3), l, ibase, sbase, seq, pos, end,
                                        (uint32_t)n, r0, off8, md, mw);
            else
                exact_range_narrow<kGather>(ex, rbase, sh, wl4, l, ibase, sbase, seq, pos, end, (uint32_t)n, r0,
                                            off8, md, mw);
            __syncthreads();
            exact_flush(ex, TF, B, F, f0, hist + (size_t)slot * 2u * F * B, narrow ? 4u : 1u);
            __syncthreads();
        }
        pos = end;
        ++seg;
    }
}

// ---------------------------------------------------------------------------------
// Packed multi-channel fill (K > 1, NP * B <= 512 with NP = ceil(C / 2) planes).  The score
// channels 2j and 2j + 1 of a row travel in one 64-bit word, p_j = q_{2j+1} * 2^32 + q_{2j}
// (mod 2^64), each |q| <= 2^kPkkBits - 1 (rounded on the scale of the largest row, clamped), so
// a (row, feature) costs NP = 6 LDS atomics at C = 11 instead of 11 -- the fill of a many-class
// session is bound by the LDS atomic instruction rate, whatever share of lanes the dominant-bin
// skip leaves active.  Both fields are signed: a cell decodes as lo = sext(low 32 bits),
// hi = (cell - lo) / 2^32, exact while each field's sum stays below 2^31 in magnitude.  Every
// thread owns kPkkOwn cells and swaps them with zero after the barrier that ends every
// kPkkSwapBlocks blocks of kPkkBlockRows rows; atomics of threads already in the next period
// may land before the swap, so at most R = 2 * kPkkSwapBlocks * kPkkBlockRows rows fall between
// two swaps of a cell and R * (2^kPkkBits - 1) < 2^31.  The swapped fields are added to int64
// registers, flushed to the level histogram at segment ends: every sum is an exact integer of
// the rounded rows (order-free, reproducible).  Tiles of 32 features (8 words), LDS
// [plane][bin][32] with the two-channel bin-major fill's rotated visits (any 16 consecutive
// lanes hit 16 distinct features mod 16: distinct bank pairs whatever the bins), 8 lanes per
// row.  A lane past the tile's words reads the row's zero
// padding and adds to columns >= TF, which are never flushed.
// ---------------------------------------------------------------------------------
constexpr uint32_t kPkkThreads = 1024;
constexpr int kPkkOwn = 16;                                            // cells per thread
constexpr uint32_t kPkkCells = (uint32_t)kPkkOwn * kPkkThreads;        // NP * B * 32 <= 16384
constexpr uint32_t kPkkBlockRows = kPkkThreads / 8;                   // 128 rows per block
constexpr uint32_t kPkkSwapBlocks = 8;                                 // 1024 rows per swap period
constexpr int kPkkBits = 20;                                           // 2048 * (2^20 - 1) < 2^31
constexpr uint32_t kPkkSegmentCost = 512;   // rows' worth of time a segment's flush costs (ranges)
static_assert(2ull * kPkkSwapBlocks * kPkkBlockRows * ((1ull << kPkkBits) - 1) < (1ull << 31),
              "packed multi-channel fields stay below 2^31");

__device__ __forceinline__ void unpack_add_signed(unsigned long long v, long long& lo_acc, long long& hi_acc) {
    const int32_t lo = (int32_t)(uint32_t)v;
    lo_acc += lo;
    hi_acc += (long long)(int32_t)(uint32_t)((v - (unsigned long long)(long long)lo) >> 32);
}

// Score channels f64 -> clamped fixed point in place ([n][C] doubles become int64, which the
// dominant-bin segment totals read) and the NP packed words of every row [n][NP] the fill reads.
template <int C>
static __global__ void quantize_pack_kernel(double* __restrict__ sstat, uint64_t n, const Scales* __restrict__ sc,
                                            unsigned long long* __restrict__ spk, long long qmax) {
    constexpr int NP = (C + 1) / 2;
    const double md = sc->mul[kScoreDer], mw = sc->mul[kScoreW];
    long long* out = (long long*)sstat;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        long long q[2 * NP];
#pragma unroll
        for (int ch = 0; ch < C; ++ch) {
            q[ch] = max(-qmax, min(qmax, to_fixed(sstat[i * C + ch], ch == C - 1 ? mw : md)));
            out[i * C + ch] = q[ch];
        }
        if (C & 1) q[C] = 0;
#pragma unroll
        for (int j = 0; j < NP; ++j)
            spk[i * NP + j] = ((unsigned long long)(uint32_t)q[2 * j + 1] << 32) + (unsigned long long)q[2 * j];
    }
}

template <int C, bool kSkip, bool kGather>
static __global__ __launch_bounds__(kPkkThreads) void fill_pkk_kernel(
    const uint32_t* __restrict__ rows, uint32_t W, uint32_t stride /* words per row in memory */, uint64_t n,
    const uint32_t* __restrict__ idx, const LevelPlan* __restrict__ plan,
    const unsigned long long* __restrict__ spk /* [n][NP] */, uint32_t n_tiles, uint32_t F, uint32_t B, uint32_t G, long long* __restrict__ hist,
    const uint32_t* __restrict__ skip_bin /* kSkip: [F] */,
    uint32_t np_fill /* planes filled: NP, or NP - 1 when the last (the weight alone) comes from elsewhere */) {
    constexpr int NP = (C + 1) / 2;
    extern __shared__ unsigned long long pk[];   // [NP][B][32], kPkkCells cells
    const uint32_t b = blockIdx.x;
    const uint32_t xcd = b & 7u, q = b >> 3;
    const uint32_t t = q % n_tiles;
    const uint32_t g = (q / n_tiles) * 8u + xcd;   // row range (ranges of a tile spread over the XCDs)
    const uint32_t w0 = t * 8u;
    const uint32_t TW = min(8u, W - w0);
    const uint32_t f0 = 4u * w0;
    const uint32_t TF = min(4u * TW, F - f0);
    const uint32_t plane = B * 32u;
    // cells in use: NP planes of B bins x 32 features; a thread's cells past them stay zero, so
    // the swaps, staging and clears skip them (kc of its kPkkOwn slots)
    const uint32_t kc = ((uint32_t)NP * plane + kPkkThreads - 1) / kPkkThreads;
    for (uint32_t i = threadIdx.x; i < kPkkCells; i += kPkkThreads) pk[i] = 0ull;
    const uint32_t r0 = threadIdx.x >> 3, wl = threadIdx.x & 7u;   // 128 rows per pass
    const uint32_t rot = (2u * (r0 & 1u) + ((wl >> 2) ^ ((r0 >> 1) & 1u))) & 3u;
    uint32_t off8[4], skp[4];   // byte offset of the step's column (low 5 bits: the byte's bit shift)
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) {
        const uint32_t kb = (k + rot) & 3u;
        const uint32_t f = 4u * wl + kb;
        off8[k] = 8u * f;
        skp[k] = (kSkip && f < TF) ? skip_bin[f0 + f] : 256u;
    }
    long long acc_lo[kPkkOwn], acc_hi[kPkkOwn];
#pragma unroll
    for (int k = 0; k < kPkkOwn; ++k) acc_lo[k] = acc_hi[k] = 0;
    __syncthreads();
    const uint32_t V = kGather ? plan->rows : (uint32_t)n;
    const uint32_t n_seg = kGather ? plan->n_parent : 1u;
    uint32_t rb = (uint32_t)(((uint64_t)V * g) / G), re = (uint32_t)(((uint64_t)V * (g + 1)) / G);
    if (kGather) balanced_range(plan, n_seg, V, g, G, kPkkSegmentCost, rb, re);
    uint32_t seg = 0;
    if (kGather)
        seg = first_segment(plan, n_seg, rb);
    auto swap_cells = [&]() {
#pragma unroll
        for (int k = 0; k < kPkkOwn; ++k) {
            if ((uint32_t)k < kc) {
                const unsigned long long v = atomicExch(pk + threadIdx.x + (uint32_t)k * kPkkThreads, 0ull);
                unpack_add_signed(v, acc_lo[k], acc_hi[k]);
            }
        }
    };
    uint32_t pos = rb;
    while (pos < re) {
        const uint32_t seg_lo = kGather ? plan->seg_begin[seg] : 0u;
        const uint32_t seg_end = (kGather && seg + 1 < n_seg) ? plan->seg_begin[seg + 1] : V;
        const uint32_t end = min(re, seg_end);
        const uint32_t slot = kGather ? plan->built[seg] : 0u;
        if (end > pos) {
            // blocks of 128 rows (one per row slot), two register sets SA and SB in flight: the
            // words and statistics of a block are loaded two blocks ahead, gathered row indices
            // four, so a block's atomics never wait for its loads (fixed set roles: no register
            // moves that would wait on loads in flight)
            struct Set {
                uint32_t word;
                unsigned long long st[NP];
            } SA, SB;
            auto ldix = [&](uint32_t bb) -> uint32_t {
                const uint32_t p = bb + r0;
                return kGather ? idx[p < end ? p : pos] : (p < end ? p : pos);
            };
            auto load_set = [&](Set& S, uint32_t bb, uint32_t doc) {
                const uint32_t p = bb + r0;
                const bool ok = p < end;
                S.word = rows[(size_t)doc * stride + w0 + wl];
#pragma unroll
                for (int j = 0; j < NP; ++j) {
                    const unsigned long long v = spk[(size_t)doc * NP + j];
                    S.st[j] = ok ? v : 0ull;
                }
            };
            auto atoms = [&](const Set& S) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t bin = __builtin_amdgcn_ubfe(S.word, off8[k], 8);
                    if (kSkip && bin == skp[k]) continue;   // dominant bin: rebuilt from the totals
                    unsigned long long* cell = (unsigned long long*)((char*)pk + ((bin << 8) + off8[k]));
#pragma unroll
                    for (int j = 0; j < NP; ++j)
                        if (j + 1 < NP || np_fill == (uint32_t)NP) atomicAdd(cell + (size_t)j * plane, S.st[j]);
                }
            };
            uint32_t blk = 0;
            auto after_block = [&](uint32_t bb) {   // swap at the end of a period and of the segment
                if (++blk >= kPkkSwapBlocks || bb + kPkkBlockRows >= end) {
                    blk = 0;
                    __syncthreads();
                    swap_cells();
                }
            };
            uint32_t ixA = ldix(pos), ixB = ldix(pos + kPkkBlockRows);
            load_set(SA, pos, ixA);
            asm volatile("" ::: "memory");
            load_set(SB, pos + kPkkBlockRows, ixB);
            asm volatile("" ::: "memory");
            if (kGather) {
                ixA = ldix(pos + 2 * kPkkBlockRows);
                ixB = ldix(pos + 3 * kPkkBlockRows);
            }
            asm volatile("" ::: "memory");
            for (uint32_t bb = pos;; bb += 2 * kPkkBlockRows) {   // workgroup-uniform
                atoms(SA);
                load_set(SA, bb + 2 * kPkkBlockRows, kGather ? ixA : ldix(bb + 2 * kPkkBlockRows));
                if (kGather) ixA = ldix(bb + 4 * kPkkBlockRows);
                after_block(bb);
                if (bb + kPkkBlockRows >= end) break;
                atoms(SB);
                load_set(SB, bb + 3 * kPkkBlockRows, kGather ? ixB : ldix(bb + 3 * kPkkBlockRows));
                if (kGather) ixB = ldix(bb + 5 * kPkkBlockRows);
                after_block(bb + kPkkBlockRows);
                if (bb + 2 * kPkkBlockRows >= end) break;
            }
            // every contribution of the segment is in the registers now: flush each plane's two
            // channels (stage the registers in the cells, then write the non-zero cells).  A segment
            // that lies wholly in this workgroup's range is this tile's only writer of its rows: its
            // cells are stored (the level histogram starts zeroed); a segment shared with the
            // neighbouring range is added with global atomics
            const bool owned = pos == seg_lo && end == seg_end;
            long long* hd = hist + (size_t)slot * C * F * B;
            for (int half = 0; half < 2; ++half) {
                __syncthreads();
#pragma unroll
                for (int k = 0; k < kPkkOwn; ++k)
                    if ((uint32_t)k < kc)
                        pk[threadIdx.x + (uint32_t)k * kPkkThreads] = (unsigned long long)(half ? acc_hi[k] : acc_lo[k]);
                __syncthreads();
                // a wave takes 8 features x 8 bins of one plane (64-byte runs of bins in the histogram)
                const uint32_t nfb = (TF + 7) / 8, nbb = (B + 7) / 8;
                const uint32_t vcells = (uint32_t)NP * nfb * nbb * 64;
                for (uint32_t i = threadIdx.x; i < vcells; i += kPkkThreads) {
                    const uint32_t l = i & 63u, jj = i >> 6;
                    const uint32_t j = jj / (nfb * nbb), jb = jj - j * (nfb * nbb);
                    const uint32_t f = (jb / nbb) * 8 + (l >> 3), bin = (jb % nbb) * 8 + (l & 7u);
                    const uint32_t ch = 2u * j + (uint32_t)half;
                    if (f >= TF || bin >= B || ch >= (uint32_t)C || j >= np_fill) continue;
                    const unsigned long long v = pk[j * plane + bin * 32u + f];
                    unsigned long long* d = (unsigned long long*)hd + (((size_t)ch * F + f0 + f) * B + bin);
                    if (v != 0) {
                        if (owned) *d = v;
                        else atomicAdd(d, v);
                    }
                }
            }
            __syncthreads();
#pragma unroll
            for (int k = 0; k < kPkkOwn; ++k) {
                if ((uint32_t)k < kc) pk[threadIdx.x + (uint32_t)k * kPkkThreads] = 0ull;
                acc_lo[k] = acc_hi[k] = 0;
            }
            __syncthreads();
        }
        pos = end;
        ++seg;
    }
}

// ---------------------------------------------------------------------------------
// Packed multi-channel fill over sparse entries (sessions whose features mostly sit in their
// dominant bin).  An instruction of 64-bit LDS atomics costs the same whatever lanes are active,
// and its bank conflicts count within each 16-lane DPP row only (a DPP row whose lanes hit
// distinct bank pairs runs at the full rate whatever the other rows hit).  So a DPP row takes
// one row of a 32-feature tile and lane e its e-th non-dominant (feature, bin) entry, in feature
// order: distinct features, i.e. distinct bank pairs of the [plane][bin][32] cells, and about
// twice the active lanes of the dense fill's 8-lanes-per-row visit when 30% of the entries are
// non-dominant.  The entries are built once per session (pack_sparse_kernel): per (tile, row)
// 16 codes in slots A and the rest (a row with more than 16 entries in a tile) in slots B, a
// code being the entry's byte offset in a plane, bin * 256 + 8 * feature, bit 0 of A's last
// code flagging the overflow, 0xFFFF an empty lane.  Statistics, swaps, flushes and the cells'
// bound are the packed multi-channel fill's (64 rows per block, swaps every 16 blocks: at most
// 2048 rows between two swaps of a cell).
// ---------------------------------------------------------------------------------
// sv[j] = lane j's v in every lane of its DPP row (row_newbcast), j < NP
template <int NP, int J = 0>
__device__ __forceinline__ void bcast_planes(unsigned long long v, unsigned long long* sv) {
    if constexpr (J < NP) {
        sv[J] = row_bcast64<J>(v);
        bcast_planes<NP, J + 1>(v, sv);
    }
}

constexpr uint32_t kPksBlockRows = kPkkThreads / 16;   // 64 rows per block
constexpr uint32_t kPksSwapBlocks = 16;                // 1024 rows per swap period
constexpr uint16_t kPksEmpty = 0xFFFFu;
static_assert(2ull * kPksSwapBlocks * kPksBlockRows * ((1ull << kPkkBits) - 1) < (1ull << 31),
              "packed multi-channel fields stay below 2^31");

// Entries of every (tile, row): thread per (tile, row), rows consecutive (coalesced column reads).
static __global__ __launch_bounds__(256) void pack_sparse_kernel(const uint8_t* __restrict__ cols /* [F][n] */,
                                                                 uint64_t n, uint32_t F, uint32_t n_tiles,
                                                                 const uint32_t* __restrict__ skip_bin,
                                                                 uint16_t* __restrict__ A, uint16_t* __restrict__ Bo) {
    for (uint64_t q = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; q < (uint64_t)n_tiles * n;
         q += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t t = (uint32_t)(q / n);
        const uint64_t i = q - (uint64_t)t * n;
        uint16_t* a = A + q * 16;
        uint16_t* bo = Bo + q * 16;
        for (uint32_t k = 0; k < 16; ++k) {
            a[k] = kPksEmpty;
            bo[k] = kPksEmpty;
        }
        uint32_t cnt = 0;
        uint16_t last_a = kPksEmpty;
        for (uint32_t fl = 0; fl < 32; ++fl) {
            const uint32_t f = 32u * t + fl;
            if (f >= F) break;
            const uint32_t bin = cols[(size_t)f * n + i];
            if (bin == skip_bin[f]) continue;
            const uint16_t code = (uint16_t)((bin << 8) | (fl << 3));
            if (cnt < 16) a[cnt] = code;
            else bo[cnt - 16] = code;
            if (cnt == 15) last_a = code;
            ++cnt;
        }
        if (cnt > 16) a[15] = (uint16_t)(last_a | 1u);
    }
}

// kOwn: cells per thread (NP * B * 32 <= kOwn * 1024; the registers holding their int64 partial
// sums are sized by it); kSets: blocks in flight per wave.
template <int C, bool kGather, int kOwn = kPkkOwn, int kSets = 4>
static __global__ __launch_bounds__(kPkkThreads) void fill_pks_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ Bo /* [n_tiles][n][16] each */, uint64_t n,
    const uint32_t* __restrict__ idx, const LevelPlan* __restrict__ plan,
    const unsigned long long* __restrict__ spk /* [n][NP] */, uint32_t n_tiles, uint32_t F, uint32_t B, uint32_t G,
    long long* __restrict__ hist,
    uint32_t np_fill /* planes filled: NP, or NP - 1 when the last (the weight alone) comes from elsewhere */) {
    constexpr int NP = (C + 1) / 2;
    const bool fill_last = np_fill == (uint32_t)NP;   // workgroup-uniform
    extern __shared__ unsigned long long pk[];   // [NP][B][32], kOwn * 1024 cells
    const uint32_t b = blockIdx.x;
    const uint32_t xcd = b & 7u, q = b >> 3;
    const uint32_t t = q % n_tiles;
    const uint32_t g = (q / n_tiles) * 8u + xcd;   // row range (ranges of a tile spread over the XCDs)
    const uint32_t f0 = 32u * t;
    const uint32_t TF = min(32u, F - f0);
    const uint32_t plane = B * 32u;
    const uint32_t kc = ((uint32_t)NP * plane + kPkkThreads - 1) / kPkkThreads;
    for (uint32_t i = threadIdx.x; i < (uint32_t)kOwn * kPkkThreads; i += kPkkThreads) pk[i] = 0ull;
    const uint32_t r0 = threadIdx.x >> 4, e = threadIdx.x & 15u;   // 64 rows per pass, lane e: entry e
    const uint16_t* At = A + (size_t)t * n * 16 + e;
    const uint16_t* Bt = Bo + (size_t)t * n * 16 + e;
    static_assert(kOwn >= 1 && kOwn <= kPkkOwn, "owned cells");
    long long acc_lo[kOwn], acc_hi[kOwn];
#pragma unroll
    for (int k = 0; k < kOwn; ++k) acc_lo[k] = acc_hi[k] = 0;
    __syncthreads();
    const uint32_t V = kGather ? plan->rows : (uint32_t)n;
    const uint32_t n_seg = kGather ? plan->n_parent : 1u;
    uint32_t rb = (uint32_t)(((uint64_t)V * g) / G), re = (uint32_t)(((uint64_t)V * (g + 1)) / G);
    if (kGather) balanced_range(plan, n_seg, V, g, G, kPkkSegmentCost, rb, re);
    uint32_t seg = 0;
    if (kGather)
        seg = first_segment(plan, n_seg, rb);
    auto swap_cells = [&]() {
#pragma unroll
        for (int k = 0; k < kOwn; ++k) {
            if ((uint32_t)k < kc) {
                const unsigned long long v = atomicExch(pk + threadIdx.x + (uint32_t)k * kPkkThreads, 0ull);
                unpack_add_signed(v, acc_lo[k], acc_hi[k]);
            }
        }
    };
    uint32_t pos = rb;
    while (pos < re) {
        const uint32_t seg_lo = kGather ? plan->seg_begin[seg] : 0u;
        const uint32_t seg_end = (kGather && seg + 1 < n_seg) ? plan->seg_begin[seg + 1] : V;
        const uint32_t end = min(re, seg_end);
        const uint32_t slot = kGather ? plan->built[seg] : 0u;
        if (end > pos) {
            // blocks of 64 rows (one per DPP row); lane j < NP of a DPP row loads plane j of the
            // row's statistics
            // (one load instruction for all planes; lane j broadcasts plane j at use)
            struct Set {
                uint32_t code, doc;
                unsigned long long st;
            };
            auto ldix = [&](uint32_t bb) -> uint32_t {
                const uint32_t p = bb + r0;
                return kGather ? idx[p < end ? p : pos] : (p < end ? p : pos);
            };
            auto load_set = [&](Set& S, uint32_t bb, uint32_t doc) {
                const bool ok = bb + r0 < end;
                S.doc = doc;
                const uint32_t c = At[(size_t)doc * 16];
                S.code = ok ? c : (uint32_t)kPksEmpty;
                const unsigned long long v = spk[(size_t)doc * NP + (e < (uint32_t)NP ? e : 0u)];
                S.st = ok ? v : 0ull;
            };
            auto atoms = [&](const Set& S) {
                unsigned long long sv[NP];
                bcast_planes<NP>(S.st, sv);
                // a row with more than 16 entries flags A's last code: its DPP row reads B too
                const uint32_t over = row_bcast<15>(S.code != kPksEmpty ? (S.code & 1u) : 0u);
                if (S.code != kPksEmpty) {
                    unsigned long long* cell = (unsigned long long*)((char*)pk + (S.code & ~7u));
#pragma unroll
                    for (int j = 0; j < NP; ++j)
                        if (j + 1 < NP || fill_last) atomicAdd(cell + (size_t)j * plane, sv[j]);
                }
                if (__any(over != 0u)) {   // rare: wave-uniform branch
                    const uint32_t c2 = over ? (uint32_t)Bt[(size_t)S.doc * 16] : (uint32_t)kPksEmpty;
                    if (c2 != kPksEmpty) {
                        unsigned long long* cell = (unsigned long long*)((char*)pk + (c2 & ~7u));
#pragma unroll
                        for (int j = 0; j < NP; ++j)
                            if (j + 1 < NP || fill_last) atomicAdd(cell + (size_t)j * plane, sv[j]);
                    }
                }
            };
            uint32_t blk = 0;
            auto after_block = [&](uint32_t bb) {   // swap at the end of a period and of the segment
                if (++blk >= kPksSwapBlocks || bb + kPksBlockRows >= end) {
                    blk = 0;
                    __syncthreads();
                    swap_cells();
                }
            };
            // kSets sets in flight (a block's atomics are few: the loads need several blocks'
            // time), gathered row indices kSets blocks ahead of their set's loads; named sets
            // (an array of them indexed in the loop went to scratch)
            static_assert(kSets == 4 || kSets == 8, "four or eight sets");
            constexpr uint32_t R = kPksBlockRows;
            Set S0, S1, S2, S3, S4, S5, S6, S7;
            uint32_t ix0 = 0, ix1 = 0, ix2 = 0, ix3 = 0, ix4 = 0, ix5 = 0, ix6 = 0, ix7 = 0;
#define CBH_PKS_SET(Q, X)                                                                   \
    if constexpr (kSets > Q) X
            CBH_PKS_SET(0, ix0 = ldix(pos);)
            CBH_PKS_SET(1, ix1 = ldix(pos + R);)
            CBH_PKS_SET(2, ix2 = ldix(pos + 2 * R);)
            CBH_PKS_SET(3, ix3 = ldix(pos + 3 * R);)
            CBH_PKS_SET(4, ix4 = ldix(pos + 4 * R);)
            CBH_PKS_SET(5, ix5 = ldix(pos + 5 * R);)
            CBH_PKS_SET(6, ix6 = ldix(pos + 6 * R);)
            CBH_PKS_SET(7, ix7 = ldix(pos + 7 * R);)
#define CBH_PKS_LOAD(Q)                                                                     \
    if constexpr (kSets > Q) {                                                              \
        load_set(S##Q, pos + Q * R, ix##Q);                                                 \
        asm volatile("" ::: "memory");                                                      \
    }
            CBH_PKS_LOAD(0) CBH_PKS_LOAD(1) CBH_PKS_LOAD(2) CBH_PKS_LOAD(3)
            CBH_PKS_LOAD(4) CBH_PKS_LOAD(5) CBH_PKS_LOAD(6) CBH_PKS_LOAD(7)
#undef CBH_PKS_LOAD
            if (kGather) {
                CBH_PKS_SET(0, ix0 = ldix(pos + kSets * R);)
                CBH_PKS_SET(1, ix1 = ldix(pos + (kSets + 1) * R);)
                CBH_PKS_SET(2, ix2 = ldix(pos + (kSets + 2) * R);)
                CBH_PKS_SET(3, ix3 = ldix(pos + (kSets + 3) * R);)
                CBH_PKS_SET(4, ix4 = ldix(pos + (kSets + 4) * R);)
                CBH_PKS_SET(5, ix5 = ldix(pos + (kSets + 5) * R);)
                CBH_PKS_SET(6, ix6 = ldix(pos + (kSets + 6) * R);)
                CBH_PKS_SET(7, ix7 = ldix(pos + (kSets + 7) * R);)
            }
#undef CBH_PKS_SET
            asm volatile("" ::: "memory");
            auto step = [&](Set& Sq, uint32_t& ixq, uint32_t bb) {   // block bb: atomics, reload for bb + kSets R
                atoms(Sq);
                load_set(Sq, bb + kSets * R, kGather ? ixq : ldix(bb + kSets * R));
                if (kGather) ixq = ldix(bb + 2u * kSets * R);
                after_block(bb);
            };
            for (uint32_t bb = pos;; bb += kSets * R) {   // workgroup-uniform
#define CBH_PKS_STEP(Q)                                                                     \
    if constexpr (kSets > Q) {                                                              \
        step(S##Q, ix##Q, bb + Q * R);                                                      \
        if (bb + (Q + 1) * R >= end) break;                                                 \
    }
                CBH_PKS_STEP(0) CBH_PKS_STEP(1) CBH_PKS_STEP(2) CBH_PKS_STEP(3)
                CBH_PKS_STEP(4) CBH_PKS_STEP(5) CBH_PKS_STEP(6) CBH_PKS_STEP(7)
#undef CBH_PKS_STEP
            }
            // flush: as the dense multi-channel fill's (same cells, same ownership rule)
            const bool owned = pos == seg_lo && end == seg_end;
            long long* hd = hist + (size_t)slot * C * F * B;
            for (int half = 0; half < 2; ++half) {
                __syncthreads();
#pragma unroll
                for (int k = 0; k < kOwn; ++k)
                    if ((uint32_t)k < kc)
                        pk[threadIdx.x + (uint32_t)k * kPkkThreads] = (unsigned long long)(half ? acc_hi[k] : acc_lo[k]);
                __syncthreads();
                const uint32_t nfb = (TF + 7) / 8, nbb = (B + 7) / 8;
                const uint32_t vcells = (uint32_t)NP * nfb * nbb * 64;
                for (uint32_t i = threadIdx.x; i < vcells; i += kPkkThreads) {
                    const uint32_t l = i & 63u, jj = i >> 6;
                    const uint32_t j = jj / (nfb * nbb), jb = jj - j * (nfb * nbb);
                    const uint32_t f = (jb / nbb) * 8 + (l >> 3), bin = (jb % nbb) * 8 + (l & 7u);
                    const uint32_t ch = 2u * j + (uint32_t)half;
                    if (f >= TF || bin >= B || ch >= (uint32_t)C || j >= np_fill) continue;
                    const unsigned long long v = pk[j * plane + bin * 32u + f];
                    unsigned long long* d = (unsigned long long*)hd + (((size_t)ch * F + f0 + f) * B + bin);
                    if (v != 0) {
                        if (owned) *d = v;
                        else atomicAdd(d, v);
                    }
                }
            }
            __syncthreads();
#pragma unroll
            for (int k = 0; k < kOwn; ++k) {
                if ((uint32_t)k < kc) pk[threadIdx.x + (uint32_t)k * kPkkThreads] = 0ull;
                acc_lo[k] = acc_hi[k] = 0;
            }
            __syncthreads();
        }
        pos = end;
        ++seg;
    }
}

// Score channels f64 [n][2] -> one packed word per row (der in the high field, weight in the
// low field), each channel rounded with its own scale.
static __global__ void pack_stats_fixed_kernel(const double* __restrict__ sstat, uint64_t n,
                                               const Scales* __restrict__ sc,
                                               unsigned long long* __restrict__ spack,
                                               long long qmax /* 2^pack_bits - 1 */) {
    const double md = sc->mul[kScoreDer], mw = sc->mul[kScoreW];
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        // |v * 2^S| < 2^pack_bits, so rounding reaches 2^pack_bits at most: clamped one unit down
        const long long qd = max(-qmax, min(qmax, to_fixed(sstat[2 * i], md)));
        const long long qw = max(-qmax, min(qmax, to_fixed(sstat[2 * i + 1], mw)));
        spack[i] = ((unsigned long long)qd << 32) + (unsigned long long)qw;
    }
}

// Score channels f64 [n][2] -> one count-packed word per row: the der channel rounded at the
// tree's scale in the high field, the integer score weight (w * s, an integer in a session that
// takes this fill) in the low pk_k bits.
static __global__ void pack_stats_count_kernel(const double* __restrict__ sstat, uint64_t n,
                                               const Scales* __restrict__ sc,
                                               unsigned long long* __restrict__ spack) {
    const double md = sc->mul[kScoreDer];
    const uint32_t kb = (uint32_t)sc->pk_k;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const long long qd = to_fixed(sstat[2 * i], md);
        const unsigned long long qw = (unsigned long long)sstat[2 * i + 1];
        spack[i] = ((unsigned long long)qd << kb) + qw;
    }
}

// Histograms are kept in PREFIX form over bins (cell b holds the sum of bins 0..b): the
// split scorer then reads FALSE = prefix[b], TRUE = prefix[B-1] - prefix[b] directly, and
// the sibling subtraction stays valid because the prefix is linear.  This pass turns the
// directly built children of a level (raw sums from the fill) into prefix form: one wave per
// (child, channel, feature) row, each lane scanning up to 4 consecutive bins.
// With `parent` given (levels >= 1) the same wave then writes the sibling row, parent - built,
// both in prefix form (the subtraction is linear), so no separate derive pass is needed.
static __global__ __launch_bounds__(256) void hist_prefix_kernel(long long* __restrict__ hist,
                                                                 const LevelPlan* __restrict__ plan,
                                                                 uint32_t n_built, uint32_t C, uint32_t F,
                                                                 uint32_t B,
                                                                 const long long* __restrict__ parent,
                                                                 const uint32_t* __restrict__ skip_bin,
                                                                 const long long* __restrict__ seg_tot) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t row = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint64_t rows = (uint64_t)n_built * C * F;
    if (row >= rows) return;   // wave-uniform
    const uint32_t seg = (uint32_t)(row / ((uint64_t)C * F));
    const uint32_t rem = (uint32_t)(row - (uint64_t)seg * C * F);
    const uint32_t slot = plan ? plan->built[seg] : 0u;
    long long* h = hist + ((size_t)slot * C * F + rem) * B;
    const uint32_t E = (B + 63) / 64;   // bins per lane, <= 4
    const uint32_t b0 = lane * E;
    long long v[4];
    long long run = 0;
#pragma unroll
    for (uint32_t e = 0; e < 4; ++e) {
        const uint32_t b = b0 + e;
        v[e] = (e < E && b < B) ? h[b] : 0;
        run += v[e];
        v[e] = run;
    }
    long long incl = run;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const long long u = __shfl_up(incl, o, 64);
        if (lane >= (uint32_t)o) incl += u;
    }
    const long long off = incl - run;
    // a dominant bin the fill left out (its cell still 0) is rebuilt as the segment's channel
    // total minus the other bins, i.e. every prefix from that bin on grows by it
    long long dv = 0;
    uint32_t d = B;
    if (skip_bin) {
        const uint32_t ch = rem / F, f = rem - ch * F;
        d = skip_bin[f];
        if (d < B) dv = seg_tot[(size_t)seg * C + ch] - __shfl(incl, 63, 64);
    }
#pragma unroll
    for (uint32_t e = 0; e < 4; ++e) {
        const uint32_t b = b0 + e;
        v[e] += off + (b >= d ? dv : 0);
        if (e < E && b < B) h[b] = v[e];
    }
    if (!parent) return;
    // sibling of the built child: parent segment seg has children seg and seg + n_built
    const uint32_t other = slot == seg ? seg + n_built : seg;
    const long long* pr = parent + ((size_t)seg * C * F + rem) * B;
    long long* sib = hist + ((size_t)other * C * F + rem) * B;
#pragma unroll
    for (uint32_t e = 0; e < 4; ++e) {
        const uint32_t b = b0 + e;
        if (e < E && b < B) sib[b] = pr[b] - v[e];
    }
}

// The same pass for few bins: a group of GL lanes (32 or 16, up to EM bins each) per row, 64 / GL
// rows per wave (fewer waves than the 64-lane form, whose lanes past 33 idle at 65 bins).
template <uint32_t GL, uint32_t EM>
static __global__ __launch_bounds__(256) void hist_prefix_group_kernel(long long* __restrict__ hist,
                                                                       const LevelPlan* __restrict__ plan,
                                                                       uint32_t n_built, uint32_t C, uint32_t F,
                                                                       uint32_t B,
                                                                       const long long* __restrict__ parent,
                                                                       const uint32_t* __restrict__ skip_bin,
                                                                       const long long* __restrict__ seg_tot) {
    const uint32_t hl = threadIdx.x & (GL - 1u);
    const uint64_t row = (uint64_t)blockIdx.x * (256 / GL) + (threadIdx.x / GL);
    const uint64_t rows = (uint64_t)n_built * C * F;
    const bool valid = row < rows;   // the shuffles below run in every lane of the wave
    const uint64_t rc = valid ? row : rows - 1;
    const uint32_t seg = (uint32_t)(rc / ((uint64_t)C * F));
    const uint32_t rem = (uint32_t)(rc - (uint64_t)seg * C * F);
    const uint32_t slot = plan ? plan->built[seg] : 0u;
    long long* h = hist + ((size_t)slot * C * F + rem) * B;
    const uint32_t E = (B + GL - 1) / GL;   // bins per lane, <= EM
    const uint32_t b0 = hl * E;
    long long v[EM];
    long long run = 0;
#pragma unroll
    for (uint32_t e = 0; e < EM; ++e) {
        const uint32_t b = b0 + e;
        v[e] = (e < E && b < B) ? h[b] : 0;
        run += v[e];
        v[e] = run;
    }
    long long incl = run;
#pragma unroll
    for (int o = 1; o < (int)GL; o <<= 1) {
        const long long u = __shfl_up(incl, o, GL);
        if (hl >= (uint32_t)o) incl += u;
    }
    const long long off = incl - run;
    long long dv = 0;
    uint32_t d = B;
    const long long tot = __shfl(incl, GL - 1, GL);
    if (skip_bin) {
        const uint32_t ch = rem / F, f = rem - ch * F;
        d = skip_bin[f];
        if (d < B) dv = seg_tot[(size_t)seg * C + ch] - tot;
    }
    if (!valid) return;
#pragma unroll
    for (uint32_t e = 0; e < EM; ++e) {
        const uint32_t b = b0 + e;
        v[e] += off + (b >= d ? dv : 0);
        if (e < E && b < B) h[b] = v[e];
    }
    if (!parent) return;
    const uint32_t other = slot == seg ? seg + n_built : seg;
    const long long* pr = parent + ((size_t)seg * C * F + rem) * B;
    long long* sib = hist + ((size_t)other * C * F + rem) * B;
#pragma unroll
    for (uint32_t e = 0; e < EM; ++e) {
        const uint32_t b = b0 + e;
        if (e < E && b < B) sib[b] = pr[b] - v[e];
    }
}

// ---------------------------------------------------------------------------------
// Dominant-bin skip.  A feature whose most frequent bin holds a large share of the rows
// (sparse columns: 70% exact zeros put 70% of the rows in one bin) makes the fill's LDS
// atomics collide on one cell.  The fill leaves that bin out; the per-segment channel totals
// are summed apart (seg_totals_kernel) and the bin is rebuilt as total - sum(other bins),
// exact in int64 (hist_prefix_kernel).
// ---------------------------------------------------------------------------------
constexpr int kMaxC = kMaxK + 1;

// Per-feature bin counts over the feature-major columns: grid (row chunks, features); a
// block counts its chunk in LDS with 16-byte loads over the aligned body of the chunk.
static __global__ __launch_bounds__(256) void bin_census_kernel(const uint8_t* __restrict__ cols, uint64_t n,
                                                                uint64_t chunk,
                                                                unsigned long long* __restrict__ counts) {
    __shared__ unsigned int c[256];
    c[threadIdx.x] = 0;
    __syncthreads();
    const uint8_t* col = cols + (size_t)blockIdx.y * n;
    const uint64_t lo = (uint64_t)blockIdx.x * chunk;
    const uint64_t hi = lo + chunk < n ? lo + chunk : n;
    if (lo < hi) {
        const uint64_t mis = (uint64_t)(uintptr_t)(col + lo) & 15u;
        uint64_t head = mis ? 16u - mis : 0u;
        if (head > hi - lo) head = hi - lo;
        const uint64_t nvec = (hi - lo - head) / 16;
        const uint64_t body = lo + head, tail = body + nvec * 16;
        for (uint64_t i = lo + threadIdx.x; i < body; i += blockDim.x) atomicAdd(&c[col[i]], 1u);
        const uint4* v = reinterpret_cast<const uint4*>(col + body);
        for (uint64_t j = threadIdx.x; j < nvec; j += blockDim.x) {
            const uint4 w = v[j];
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int b = 0; b < 4; ++b) atomicAdd(&c[(ws[q] >> (8 * b)) & 0xffu], 1u);
        }
        for (uint64_t i = tail + threadIdx.x; i < hi; i += blockDim.x) atomicAdd(&c[col[i]], 1u);
    }
    __syncthreads();
    if (c[threadIdx.x])
        atomicAdd(counts + (size_t)blockIdx.y * 256 + threadIdx.x, (unsigned long long)c[threadIdx.x]);
}

// Entries a row adds to the level histograms when the fill leaves out the dominant bins: the
// features with no dominant bin plus those whose bin is not it ([n], counted once).
static __global__ __launch_bounds__(256) void row_entries_kernel(const uint8_t* __restrict__ cols /* [F][n] */,
                                                                 uint64_t n, uint32_t F,
                                                                 const uint32_t* __restrict__ skip_bin,
                                                                 uint16_t* __restrict__ out) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
        uint32_t c = 0;
        for (uint32_t f = 0; f < F; ++f) c += cols[(size_t)f * n + i] != skip_bin[f];
        out[i] = (uint16_t)c;
    }
}

// The entries one fill launch adds (profiling only): the sum of the visited rows' entry counts
// (idx: the partition's listed rows, plan->rows of them; else rows [0, n)).
static __global__ __launch_bounds__(256) void fill_entries_kernel(const uint32_t* __restrict__ idx,
                                                                  const LevelPlan* __restrict__ plan, uint64_t n,
                                                                  const uint16_t* __restrict__ ent,
                                                                  unsigned long long* __restrict__ total /* [2] */,
                                                                  uint32_t atomics_per_entry) {
    const uint32_t V = idx ? plan->rows : (uint32_t)n;
    unsigned long long c = 0;
    for (uint32_t p = blockIdx.x * blockDim.x + threadIdx.x; p < V; p += gridDim.x * blockDim.x)
        c += ent[idx ? idx[p] : p];
    c = wave_sum_u64(c);
    if (lane_id() == 0 && c != 0) {
        atomicAdd(total, c);
        atomicAdd(total + 1, c * atomics_per_entry);
    }
}

// Channel totals of the rows of every directly built segment: tot [segment][C].
static __global__ __launch_bounds__(256) void seg_totals_kernel(const uint32_t* __restrict__ idx,
                                                                const LevelPlan* __restrict__ plan, uint64_t n,
                                                                const long long* __restrict__ sfix, uint32_t C,
                                                                long long* __restrict__ tot) {
    __shared__ unsigned long long acc[(kMaxLeaves / 2) * kMaxC];
    const uint32_t V = idx ? plan->rows : (uint32_t)n;
    const uint32_t n_seg = idx ? plan->n_parent : 1u;
    for (uint32_t i = threadIdx.x; i < n_seg * C; i += blockDim.x) acc[i] = 0;
    __syncthreads();
    // block-uniform loop; a wave whose rows all lie in one segment reduces in registers
    for (uint32_t base = blockIdx.x * blockDim.x; base < V; base += gridDim.x * blockDim.x) {
        const uint32_t p = base + threadIdx.x;
        const bool act = p < V;
        uint32_t seg = 0;
        if (act && idx) {   // last segment whose begin <= p
            uint32_t lo = 0, hi = n_seg - 1;
            while (lo < hi) {
                const uint32_t mid = (lo + hi + 1) >> 1;
                if (plan->seg_begin[mid] <= p) lo = mid;
                else hi = mid - 1;
            }
            seg = lo;
        }
        const long long* st = act ? sfix + (size_t)(idx ? idx[p] : p) * C : nullptr;
        const uint32_t seg0 = __shfl(seg, 0, 64);
        const bool uniform = __all(!act || seg == seg0);
        for (uint32_t ch = 0; ch < C; ++ch) {
            const long long v = act ? st[ch] : 0;
            if (uniform) {
                const unsigned long long u = wave_sum_u64((unsigned long long)v);
                if (lane_id() == 0 && u != 0) atomicAdd(acc + seg0 * C + ch, u);
            } else if (v != 0) {
                atomicAdd(acc + seg * C + ch, (unsigned long long)v);
            }
        }
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n_seg * C; i += blockDim.x)
        if (acc[i] != 0) atomicAdd((unsigned long long*)tot + i, acc[i]);
}


// ---------------------------------------------------------------------------------
// Split scoring.  One workgroup per feature, one thread per border; for every leaf the
// exact integer prefix over bins gives FALSE = prefix, TRUE = total - prefix (one-hot:
// TRUE = the bin, FALSE = total - bin).  Scores fold in the reference order
// (crates/cb-compute/src/score.rs:192-265): dimension-major, FALSE children 0..P-1 then
// TRUE children 0..P-1; Cosine = num / sqrt(1e-100 + sum avg^2 w).  The block argmax keeps
// the highest score, ties to the lowest border (strict first-wins, tree.rs:355-366).
// ---------------------------------------------------------------------------------
// The score terms of candidate border b of feature f over all parents, folded into num and
// den in the reference order (d, side, p): score.rs:192-265.  The cells of kPre parents are
// loaded ahead of their terms, from clamped (always valid) addresses with the values of parents
// past P (and, for one-hot, bin -1) replaced by zero, so the loads need no branches; zero cells
// give s = w = 0, avg = 0 and terms of exactly 0 (num and den only hold non-negative sums).  The
// quotient is computed for every term and kept only where w > 0 (branch-free).  Lanes past the
// bins read bin B-1 (their score is discarded).
// One leaf's additive term of the SolarL2 / LOOL2 / SatL2 calcers (score.rs:283-350,
// kernels.rs:3338-3390): der sum s, weight sum w, no L2 regularizer.
__device__ __forceinline__ double leaf_score_term(int sf, double s, double w) {
    if (sf == 2) return w > 1e-20 ? (-s * s) * (1.0 + 2.0 * log(w + 1.0)) / w : 0.0;
    if (sf == 3) {
        double adjust = w > 1.0 ? w / (w - 1.0) : 0.0;
        adjust *= adjust;
        return w > 0.0 ? adjust * (-s * s) / w : 0.0;
    }
    const double adjust = w > 2.0 ? w * (w - 2.0) / (w * w - 3.0 * w + 1.0) : 0.0;
    return w > 0.0 ? adjust * (-s * s) / w : 0.0;
}

// sf (CBH_SCORE_*): Cosine and L2 fold avg * s into num and avg^2 * w into den; SolarL2, LOOL2 and
// SatL2 fold their per-leaf terms into num, in the same (d, side, p) order.
template <int K, bool kOneHot, bool kTerms /* SolarL2 / LOOL2 / SatL2 (sf) */>
__device__ __forceinline__ void score_fold(const long long* __restrict__ hist, uint32_t P, uint32_t F, uint32_t B,
                                           uint32_t f, uint32_t b, double inv_d, double inv_w, double l2, int sf,
                                           double& num, double& den) {
    constexpr int C = K + 1;
    constexpr uint32_t kPre = 8;   // parents whose cells are loaded ahead of their terms
    const uint32_t bc = min(b, B - 1);
    const uint32_t bq = bc > 0 ? bc - 1 : 0;
    for (int d = 0; d < K; ++d) {
        for (int side = 0; side < 2; ++side) {
            for (uint32_t p0 = 0; p0 < P; p0 += kPre) {
                long long pdv[kPre], pwv[kPre], tdv[kPre], twv[kPre], qdv[kPre], qwv[kPre];
#pragma unroll
                for (uint32_t u = 0; u < kPre; ++u) {
                    const uint32_t p = p0 + u;
                    const bool ok = p < P;
                    const uint32_t pc = ok ? p : P - 1;
                    const long long* hd = hist + (((size_t)pc * C + d) * F + f) * B;
                    const long long* hw = hist + (((size_t)pc * C + K) * F + f) * B;
                    const long long a = hd[bc], c = hw[bc], e = hd[B - 1], g = hw[B - 1];
                    pdv[u] = ok ? a : 0;
                    pwv[u] = ok ? c : 0;
                    tdv[u] = ok ? e : 0;
                    twv[u] = ok ? g : 0;
                    if (kOneHot) {
                        const long long qa = hd[bq], qc = hw[bq];
                        qdv[u] = (ok && b > 0) ? qa : 0;
                        qwv[u] = (ok && b > 0) ? qc : 0;
                    }
                }
#pragma unroll
                for (uint32_t u = 0; u < kPre; ++u) {
                    const long long pd = pdv[u], pw = pwv[u], td = tdv[u], tw = twv[u];
                    long long xd, xw;
                    if (!kOneHot) {
                        xd = side == 0 ? pd : td - pd;
                        xw = side == 0 ? pw : tw - pw;
                    } else {
                        const long long vd = pd - qdv[u], vw = pw - qwv[u];
                        xd = side == 0 ? td - vd : vd;
                        xw = side == 0 ? tw - vw : vw;
                    }
                    const double s = (double)xd * inv_d;
                    const double w = (double)xw * inv_w;
                    if (kTerms) {
                        num += leaf_score_term(sf, s, w);
                        continue;
                    }
                    const double q = s / (w + l2);
                    const double avg = w > 0.0 ? q : 0.0;
                    num += avg * s;
                    den += avg * avg * w;
                }
            }
        }
    }
}

template <int K, int NW>
__global__ __launch_bounds__(64 * NW) void score_kernel(
    long long* __restrict__ zero_buf, uint32_t zero_leaves, uint32_t HC,   // next level's histogram
    const long long* __restrict__ hist, uint32_t P, uint32_t F, uint32_t B,
    const uint32_t* __restrict__ n_cand, const uint8_t* __restrict__ one_hot,
    const Scales* __restrict__ sc, double l2, int sf /* CBH_SCORE_* */, double* __restrict__ best_score,
    uint32_t* __restrict__ best_bin, const double* __restrict__ fweight /* nullable [F] */) {
    __shared__ double red_s[NW];
    __shared__ uint32_t red_b[NW];
    const uint32_t f = blockIdx.x;
    const uint32_t b = threadIdx.x;
    // clear feature f's cells of the next level's histogram [leaf][HC][F][B] (its fill adds)
    for (uint32_t i = threadIdx.x; i < zero_leaves * HC * B; i += blockDim.x) {
        const uint32_t lc = i / B, bb = i - lc * B;
        zero_buf[((size_t)lc * F + f) * B + bb] = 0;
    }
    const uint32_t nc = n_cand[f];
    if (nc == 0) {
        if (b == 0) {
            best_score[f] = -INFINITY;
            best_bin[f] = 0;
        }
        return;
    }
    const bool oh = one_hot != nullptr && one_hot[f] != 0;
    const double inv_d = sc->inv[kScoreDer], inv_w = sc->inv[kScoreW];
    double num = 0.0;
    double den = 0.0;
    den += 1e-100;
    // the histograms are in prefix form over bins: prefix = cell b, total = cell B-1, the
    // bin itself (one-hot) = cell b - cell b-1; the fold order over (d, side, p) is the reference's
    if (sf > 1 && oh)
        score_fold<K, true, true>(hist, P, F, B, f, b, inv_d, inv_w, l2, sf, num, den);
    else if (sf > 1)
        score_fold<K, false, true>(hist, P, F, B, f, b, inv_d, inv_w, l2, sf, num, den);
    else if (oh)
        score_fold<K, true, false>(hist, P, F, B, f, b, inv_d, inv_w, l2, sf, num, den);
    else
        score_fold<K, false, false>(hist, P, F, B, f, b, inv_d, inv_w, l2, sf, num, den);
    double score = sf == 0 ? num / sqrt(den) : num;
    // the model_size_reg weight of a CTR column multiplies every candidate's score
    // (weight * score, tree.rs:3340-3346)
    if (fweight) score = fweight[f] * score;
    if (b >= nc || score != score) score = -INFINITY;
    // block argmax: max score, ties -> lowest border
    uint32_t bb = b;
    for (int o = 32; o > 0; o >>= 1) {
        double os = __shfl_xor(score, o, 64);
        uint32_t ob = __shfl_xor(bb, o, 64);
        if (os > score || (os == score && ob < bb)) {
            score = os;
            bb = ob;
        }
    }
    const uint32_t wave = threadIdx.x >> 6;
    if (lane_id() == 0) {
        red_s[wave] = score;
        red_b[wave] = bb;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double s0 = red_s[0];
        uint32_t b0 = red_b[0];
        for (int k = 1; k < NW; ++k)
            if (red_s[k] > s0 || (red_s[k] == s0 && red_b[k] < b0)) {
                s0 = red_s[k];
                b0 = red_b[k];
            }
        best_score[f] = s0;
        best_bin[f] = b0;
    }
}

// ---------------------------------------------------------------------------------
// Split scoring with the parents split over waves (many parents, K > 1, <= 64 candidates).
// The fold of score_fold is, per border, one chain of additions in the order (d, side, p).
// Here wave j of the workgroup owns parents [j*PW, j*PW + PW) and the chain passes from wave to
// wave: wave j adds its parents' terms of slab (d, side) to the running (num, den) it takes from
// LDS and hands them on; wave 0 takes slab (d, side) + 1 from the last wave.  Each wave keeps its
// parents' weight terms of both sides in registers for every dimension and loads each of its
// der cells once (the next dimension's while the chain is elsewhere), and computes a slab's
// terms before its turn comes, so the serial part is only the additions, in exactly the order
// of score_fold.
// Hand-off: every wave has an outbox of (num, den) per lane in LDS, read by the next wave
// (wave 0 reads the last wave's); an empty entry holds an all-ones NaN pattern, which num >= 0
// and den > 0 never take.  A hop polls its lanes' den in the previous wave's outbox until all are
// set, reads num (written before den), marks both empty again and writes its own outbox, num
// first.  An outbox holds one hop at a time: its reader is the only wave that clears it, and its
// writer's next hop comes after the reader's hop that cleared it (a wave's LDS operations
// complete in order).
// ---------------------------------------------------------------------------------
constexpr uint32_t kChainSpinLimit = 1u << 22;   // default bound on a wave's wait for its turn

// A wave-uniform row pointer kept in SGPRs (loads then take a per-lane 32-bit offset), and a
// wave-uniform cell read through the scalar cache (constant address space): the level's
// histogram is read-only in the scorer.
using GlobalI64 = const long long __attribute__((address_space(1)))*;
using GlobalU8 = const char __attribute__((address_space(1)))*;
using ConstI64 = const long long __attribute__((address_space(4)))*;
__device__ __forceinline__ GlobalI64 uniform_ptr(const long long* p) {
    const uint64_t a = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    return (GlobalI64)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ long long uniform_cell(GlobalI64 p) { return *(ConstI64)(uintptr_t)p; }
__device__ __forceinline__ long long readlane64(long long v, int lane) {
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)(unsigned long long)v, lane);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((unsigned long long)v >> 32), lane);
    return (long long)(((unsigned long long)hi << 32) | lo);
}

constexpr unsigned long long kChainEmpty = ~0ull;

// Take the previous hop's (num, den).  The hop before runs in another wave of this workgroup
// (or this one), each of which reaches every hop it owns; the bound (spin polls) only keeps a
// broken schedule from hanging the GPU.  The poll reads den alone with acquire ordering at
// workgroup scope, paired with the writer's release store of den, so num (stored before den)
// is visible once den is; it sleeps between reads (a polling wave would otherwise take VALU
// issue from the waves computing terms).  A wait that runs out leaves den NaN and sets the
// tree's device error word, which the host turns into an error for the tree.
__device__ __forceinline__ void chain_take(unsigned long long* slot, uint32_t lane, double& num, double& den,
                                           uint32_t spin, unsigned long long* err) {
    unsigned long long b = kChainEmpty;
    for (uint32_t k = 0; k < spin; ++k) {
        b = __hip_atomic_load(slot + 64 + lane, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (__all(b != kChainEmpty)) break;
        __builtin_amdgcn_s_sleep(1);
    }
    if (!__all(b != kChainEmpty) && lane == 0) atomicOr(err, 1ull);
    const unsigned long long a = __hip_atomic_load(slot + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    num = __longlong_as_double((long long)a);
    den = __longlong_as_double((long long)b);
    // the clearing precedes this wave's release of its own outbox (chain_give), so the wave
    // that writes this outbox next -- after the chain has passed through this wave -- sees it
    __hip_atomic_store(slot + lane, kChainEmpty, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_store(slot + 64 + lane, kChainEmpty, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void chain_give(unsigned long long* slot, uint32_t lane, double num, double den) {
    __hip_atomic_store(slot + lane, (unsigned long long)__double_as_longlong(num), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_WORKGROUP);
    // release: num and every earlier LDS write of this wave are visible before den
    __hip_atomic_store(slot + 64 + lane, (unsigned long long)__double_as_longlong(den), __ATOMIC_RELEASE,
                       __HIP_MEMORY_SCOPE_WORKGROUP);
}

// One term of the fold (score_fold): s = der sum, w = weight sum of one child.
__device__ __forceinline__ void score_term(double s, double w, double l2, double& x, double& y) {
    const double q = s / (w + l2);
    const double avg = w > 0.0 ? q : 0.0;
    x = avg * s;
    y = avg * avg * w;
}

// The launcher passes P = PW * (waves of the workgroup), every wave owning a full block, or
// (kPartial) one wave with P < PW parents: its blocks' parents past P read parent P-1's cells
// and add exact zeros (num >= +0 and den > 0 are unchanged by them).
// A workgroup scores nf features f, f + 1, ... (nf * B <= 64; nf > 1 only without one-hot
// features): lane gi * B + b is border b of feature f + gi, lanes past the groups (or past F) read
// border B-1 of feature f and their scores are discarded.
template <int K, int PW, bool kPartial, bool kOneHot>
__device__ __forceinline__ void score_chain(const long long* __restrict__ hist, uint32_t P, uint32_t F,
                                            uint32_t B, uint32_t f, uint32_t nf, double inv_d, double inv_w,
                                            double l2, unsigned long long* ring /* [waves][2][64] */, double& num,
                                            double& den, uint32_t spin, unsigned long long* err) {
    constexpr int C = K + 1;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
    const uint32_t gr = lane / B;
    const bool lane_on = gr < nf && f + gr < F;
    const uint32_t gi = lane_on ? gr : 0u;                 // feature f + gi
    const uint32_t bc = lane_on ? lane - gr * B : B - 1;   // border
    const uint32_t off_c = gi * B + bc;                    // cells from feature f's row
    const uint32_t off_tot = gi * B + (B - 1);             // feature f + gi's total
    const uint32_t p0 = wv * PW;
    auto pu = [&](uint32_t u) { return kPartial ? min(u, P - 1) : u; };   // block slot -> parent offset
    // weight sums of both children of every parent of this wave (FALSE side 0, TRUE side 1)
    double w0[PW], w1[PW];
#pragma unroll
    for (int u = 0; u < PW; ++u) {
        const GlobalI64 hw = uniform_ptr(hist + (((size_t)(p0 + pu(u)) * C + K) * F + f) * B);
        const long long pw = hw[off_c], tw = nf == 1 ? uniform_cell(hw + (B - 1)) : hw[off_tot];
        long long x0, x1;
        if (kOneHot) {   // the bin itself = prefix[b] - prefix[b-1]; TRUE = the bin
            long long qw = __shfl_up(pw, 1, 64);
            if (lane == 0) qw = 0;
            x1 = pw - qw;
            x0 = tw - x1;
        } else {
            x0 = pw;
            x1 = tw - pw;
        }
        w0[u] = (double)x0 * inv_w;
        w1[u] = (double)x1 * inv_w;
    }
    // a dimension's cells: the prefixes of every parent (one vector load each), and the
    // totals of all PW parents of all nf features in one vector load (lane g * PW + u holds
    // feature f + g's total of parent u), read out per parent with readlane (nf == 1: wave-uniform
    // values) or a lane shuffle
    long long pd[PW], tdv;
    // byte offsets from the row of (parent p0, dimension d): parent p0 + u is u * C * F * B
    // cells further (the launcher keeps PW of those strides below 2^31 bytes)
    const uint32_t pstride = (uint32_t)C * F * B * 8u;
    const uint32_t off_d = off_c * 8u;
    const uint32_t nfe = min(nf, F - f);   // features of this workgroup (the last may hold fewer)
    const uint32_t tg = min(lane / (uint32_t)PW, nfe - 1), tu = nf == 1 ? min(lane, (uint32_t)PW - 1) : lane % PW;
    const uint32_t off_t = pu(tu) * pstride + (tg * B + (B - 1)) * 8u;
    // wave-uniform byte addresses (kept in SGPRs, 64-bit scalar adds): the row of (parent p0,
    // dimension d) is row0 + d * dstride; parent p0 + u is u parent strides further
    const uint64_t pstride64 = (uint64_t)C * F * B * 8u, dstride64 = (uint64_t)F * B * 8u;
    const uint64_t row0 = (uint64_t)(uintptr_t)uniform_ptr(hist + ((size_t)p0 * C * F + f) * B);
    auto load_der = [&](int d) {
        uint64_t a = row0 + (uint64_t)d * dstride64;
        tdv = *(GlobalI64)((GlobalU8)(uintptr_t)a + off_t);
#pragma unroll
        for (int u = 0; u < PW; ++u) {
            if (u > 0 && (!kPartial || (uint32_t)u < P)) a += pstride64;   // parent p0 + pu(u)
            pd[u] = *(GlobalI64)((GlobalU8)(uintptr_t)a + off_d);
        }
    };
    load_der(0);
    uint32_t hop = wv;   // this wave's hop of slab t is t * nw + wv
    double x[PW], y[PW];
    for (int d = 0; d < K; ++d) {
#pragma unroll
        for (int side = 0; side < 2; ++side) {
#pragma unroll
            for (int u = 0; u < PW; ++u) {
                long long xd;
                const long long td = nf == 1 ? readlane64(tdv, u) : __shfl(tdv, (int)(gi * PW + u), 64);
                if (kOneHot) {
                    long long qd = __shfl_up(pd[u], 1, 64);
                    if (lane == 0) qd = 0;
                    xd = side == 0 ? td - (pd[u] - qd) : pd[u] - qd;
                } else {
                    xd = side == 0 ? pd[u] : td - pd[u];
                }
                score_term((double)xd * inv_d, side == 0 ? w0[u] : w1[u], l2, x[u], y[u]);
            }
            if (kPartial) {
#pragma unroll
                for (int u = 0; u < PW; ++u)
                    if ((uint32_t)u >= P) x[u] = y[u] = 0.0;
            }
            // the terms are computed here, before the wait for this wave's turn (the compiler
            // would otherwise sink them past it, into the serial part)
#pragma unroll
            for (int u = 0; u < PW; ++u) asm volatile("" ::"v"(x[u]), "v"(y[u]) : "memory");
            // the next dimension's cells load while the chain is in other waves
            if (side == 1 && d + 1 < K) load_der(d + 1);
            if (hop > 0) chain_take(ring + 128 * (wv == 0 ? nw - 1 : wv - 1), lane, num, den, spin, err);
#pragma unroll
            for (int u = 0; u < PW; ++u) {
                num += x[u];
                den += y[u];
            }
            chain_give(ring + 128 * wv, lane, num, den);
            // nothing of the next slab (whose first use of the prefetched cells waits for
            // them) is scheduled before the hand-off
            __builtin_amdgcn_sched_barrier(0);
            hop += nw;
        }
    }
}

template <int K, int PW, bool kPartial>
__global__ __launch_bounds__(512) void score_chain_kernel(
    long long* __restrict__ zero_buf, uint32_t zero_leaves, uint32_t HC,   // next level's histogram
    const long long* __restrict__ hist, uint32_t P, uint32_t F, uint32_t B,
    const uint32_t* __restrict__ n_cand, const uint8_t* __restrict__ one_hot,
    const Scales* __restrict__ sc, double l2, int sf /* CBH_SCORE_COSINE or _L2 */, double* __restrict__ best_score,
    uint32_t* __restrict__ best_bin, const double* __restrict__ fweight /* nullable [F] */,
    uint32_t spin /* polls a wave's wait for its turn may take */,
    unsigned long long* __restrict__ err /* the tree's device error word */, uint32_t nf /* features per workgroup */) {
    __shared__ unsigned long long ring[8 * 2 * 64];   // outboxes [wave][num, den][lane]
    __shared__ double red[64];
    // features f .. f + nf - 1 (nf > 1: B <= 64 / nf and no one-hot features)
    const uint32_t f = blockIdx.x * nf;
    const uint32_t nfe = min(nf, F - f);
    // clear the features' cells of the next level's histogram [leaf][HC][F][B] (its fill adds)
    for (uint32_t i = threadIdx.x; i < zero_leaves * HC * nfe * B; i += blockDim.x) {
        const uint32_t lc = i / (nfe * B), fb = i - lc * (nfe * B);
        zero_buf[((size_t)lc * F + f) * B + fb] = 0;
    }
    uint32_t any_cand = 0;
    for (uint32_t g = 0; g < nfe; ++g) any_cand |= n_cand[f + g];
    if (any_cand == 0) {   // workgroup-uniform: no wave enters the chain
        if (threadIdx.x < nfe) {
            best_score[f + threadIdx.x] = -INFINITY;
            best_bin[f + threadIdx.x] = 0;
        }
        return;
    }
    for (uint32_t i = threadIdx.x; i < 8 * 2 * 64; i += blockDim.x) ring[i] = kChainEmpty;
    __syncthreads();
    const double inv_d = sc->inv[kScoreDer], inv_w = sc->inv[kScoreW];
    double num = 0.0;
    double den = 0.0;
    den += 1e-100;
    if (one_hot != nullptr && one_hot[f] != 0)
        score_chain<K, PW, kPartial, true>(hist, P, F, B, f, 1u, inv_d, inv_w, l2, ring, num, den, spin, err);
    else
        score_chain<K, PW, kPartial, false>(hist, P, F, B, f, nf, inv_d, inv_w, l2, ring, num, den, spin, err);
    // the last wave made the last hop: its (num, den) are the full fold
    if ((threadIdx.x >> 6) != (blockDim.x >> 6) - 1) return;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t gr = lane / B, b = lane - gr * B;
    const bool on = gr < nfe;
    double score = sf == 0 ? num / sqrt(den) : num;
    if (on && fweight) score = fweight[f + gr] * score;
    if (!on || b >= n_cand[f + gr] || score != score) score = -INFINITY;
    if (nf == 1) {
        uint32_t bb = lane;
        for (int o = 32; o > 0; o >>= 1) {
            double os = __shfl_xor(score, o, 64);
            uint32_t ob = __shfl_xor(bb, o, 64);
            if (os > score || (os == score && ob < bb)) {
                score = os;
                bb = ob;
            }
        }
        if (lane == 0) {
            best_score[f] = score;
            best_bin[f] = bb;
        }
        return;
    }
    // nf > 1: lane g scans feature f + g's B borders in order (strict first-wins)
    red[lane] = score;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < nfe) {
        double best = -INFINITY;
        uint32_t bb = 0;
        for (uint32_t k = 0; k < B; ++k) {
            const double v = red[lane * B + k];
            if (v > best) {
                best = v;
                bb = k;
            }
        }
        best_score[f + lane] = best;
        best_bin[f + lane] = bb;
    }
}

// Level argmax over features in enumeration order (floats ascending, then one-hot
// columns ascending); strict first-wins.  One workgroup of 1024 threads.
static __global__ __launch_bounds__(1024) void argmax_kernel(const double* __restrict__ best_score,
                                                      const uint32_t* __restrict__ best_bin,
                                                      const uint8_t* __restrict__ one_hot,
                                                      uint32_t F, SplitRec* __restrict__ out) {
    __shared__ double rs[16];
    __shared__ uint32_t rk[16];
    double s = -INFINITY;
    uint32_t key = 0xFFFFFFFFu;
    for (uint32_t f = threadIdx.x; f < F; f += blockDim.x) {
        const double v = best_score[f];
        const uint32_t k = f + ((one_hot && one_hot[f]) ? F : 0u);
        if (v > s || (v == s && k < key)) {
            s = v;
            key = k;
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        double os = __shfl_xor(s, o, 64);
        uint32_t ok = __shfl_xor(key, o, 64);
        if (os > s || (os == s && ok < key)) {
            s = os;
            key = ok;
        }
    }
    const uint32_t wave = threadIdx.x >> 6;
    if (lane_id() == 0) {
        rs[wave] = s;
        rk[wave] = key;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t nw = (blockDim.x + 63) / 64;
        for (uint32_t k = 1; k < nw; ++k)
            if (rs[k] > s || (rs[k] == s && rk[k] < key)) {
                s = rs[k];
                key = rk[k];
            }
        SplitRec r;
        r.valid = (s > -INFINITY) ? 1u : 0u;
        r.feature = key == 0xFFFFFFFFu ? 0u : (key >= F ? key - F : key);
        r.one_hot = (key != 0xFFFFFFFFu && key >= F) ? 1u : 0u;
        r.bin = r.valid ? best_bin[r.feature] : 0u;
        r.score = s;
        *out = r;
    }
}

// ---------------------------------------------------------------------------------
// Stable partition by leaf.
//   split_count: leaf |= pass << level for every row; per-block counts of sampled rows
//                per new leaf -> cnt[leaf][block]
//   plan_scan:   per leaf, exclusive scan over blocks (in place) + total
//   compact:     the plan (smaller child per parent, ties -> the TRUE child, tree.rs:1109,
//                and the segment offsets of the next fill) from the totals, then the rows
//                of the built children written in ascending row order per segment;
//                inside a block, ranks come from wave ballots (match on the key bits) and
//                mbcnt, across waves from per-wave counts in LDS.
// ---------------------------------------------------------------------------------
constexpr uint32_t kPartRows = 4096;   // rows per partition block (4 waves)
constexpr uint32_t kPartWaveRows = kPartRows / 4;

// Lanes of this wave whose key equals mine (valid lanes only): one ballot per key bit.
__device__ __forceinline__ uint64_t wave_peers(uint32_t key, bool valid, uint32_t nbits) {
    uint64_t mask = __ballot(valid);
    for (uint32_t bit = 0; bit < nbits; ++bit) {
        const uint64_t m = __ballot((key >> bit) & 1u);
        mask &= ((key >> bit) & 1u) ? m : ~m;
    }
    return mask;
}

// Leaf update of one level and the per-wave row counts of every new leaf.  Each wave owns
// kPartWaveRows consecutive rows; its counts go to cnt[leaf][wave].  Up to 4 new leaves a
// leader per distinct leaf adds the popcount of its peers (one ballot per key bit, so no LDS
// cell takes more than one add per 64 rows); with more leaves every row adds 1 to its leaf's
// LDS counter (few lanes share a counter, and the ballots would grow with the level).
static __global__ __launch_bounds__(256) void split_count_kernel(
    const uint8_t* __restrict__ cols, uint64_t n, const SplitRec* __restrict__ split,
    uint32_t level, uint16_t* __restrict__ leaf, uint32_t* __restrict__ cnt, uint32_t n_waves,
    int write_counts) {
    __shared__ uint32_t c[4][kMaxLeaves];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t n_new = 2u << level;
    for (uint32_t k = lane; k < n_new; k += 64) c[wave][k] = 0;
    __syncthreads();
    const SplitRec s = *split;
    const uint8_t* col = cols + (size_t)s.feature * n;
    const uint64_t wid = (uint64_t)blockIdx.x * 4 + wave;
    const uint64_t beg = wid * kPartWaveRows;
    const uint64_t end = min(beg + kPartWaveRows, n);
    // every load of the wave's rows is issued before any is used (one memory round trip
    // per wave instead of one per 64 rows)
    constexpr int U = kPartWaveRows / 64;
    uint32_t bin[U], lf[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint64_t i = beg + (uint64_t)u * 64 + lane;
        bin[u] = i < end ? col[i] : 0u;
        lf[u] = i < end ? leaf[i] : 0x8000u;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint64_t i = beg + (uint64_t)u * 64 + lane;
        const bool in = i < end;
        const bool pass = s.one_hot ? bin[u] == s.bin : bin[u] > s.bin;
        lf[u] |= (uint32_t)pass << level;
        if (in) leaf[i] = (uint16_t)lf[u];
        if (write_counts) {
            const bool valid = in && !(lf[u] & 0x8000u);
            if (level >= 2) {   // uniform
                if (valid) atomicAdd(&c[wave][lf[u]], 1u);
            } else {
                const uint64_t mask = wave_peers(lf[u], valid, level + 1);
                if (valid && mbcnt64(mask) == 0) c[wave][lf[u]] += (uint32_t)__popcll(mask);
            }
        }
    }
    if (!write_counts) return;
    for (uint32_t k = lane; k < n_new; k += 64) cnt[(size_t)k * n_waves + wid] = c[wave][k];
}

static __global__ __launch_bounds__(1024) void plan_scan_kernel(uint32_t* __restrict__ cnt,
                                                         uint32_t n_blocks,
                                                         uint32_t* __restrict__ totals) {
    __shared__ uint32_t sh[128];   // [0, 16): wave totals, [64, 80): their exclusive prefix
    uint32_t* row = cnt + (size_t)blockIdx.x * n_blocks;
    const uint32_t per = (n_blocks + blockDim.x - 1) / blockDim.x;
    const uint32_t b0 = threadIdx.x * per;
    uint32_t local = 0;
    constexpr uint32_t kBatch = 8;   // loads in flight per thread
    for (uint32_t k0 = 0; k0 < per; k0 += kBatch) {
        uint32_t v[kBatch];
#pragma unroll
        for (uint32_t q = 0; q < kBatch; ++q) {
            const uint32_t k = k0 + q;
            v[q] = (k < per && b0 + k < n_blocks) ? row[b0 + k] : 0u;
        }
#pragma unroll
        for (uint32_t q = 0; q < kBatch; ++q) local += v[q];
    }
    // inclusive scan of the threads' sums: within each wave by shuffles, then over the wave
    // totals by wave 0 (two barriers)
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, n_waves = blockDim.x >> 6;
    uint32_t inc = local;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t u = __shfl_up(inc, o, 64);
        if (lane >= (uint32_t)o) inc += u;
    }
    if (lane == 63) sh[wave] = inc;
    __syncthreads();
    if (wave == 0) {
        const uint32_t t = lane < n_waves ? sh[lane] : 0u;
        uint32_t wi = t;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t u = __shfl_up(wi, o, 64);
            if (lane >= (uint32_t)o) wi += u;
        }
        if (lane < n_waves) sh[64 + lane] = wi - t;   // exclusive prefix of the wave totals
    }
    __syncthreads();
    uint32_t run = sh[64 + wave] + inc - local;  // exclusive prefix of this thread's range
    for (uint32_t k0 = 0; k0 < per; k0 += kBatch) {
        uint32_t v[kBatch];
#pragma unroll
        for (uint32_t q = 0; q < kBatch; ++q) {
            const uint32_t k = k0 + q;
            v[q] = (k < per && b0 + k < n_blocks) ? row[b0 + k] : 0u;
        }
#pragma unroll
        for (uint32_t q = 0; q < kBatch; ++q) {
            const uint32_t k = k0 + q;
            if (k < per && b0 + k < n_blocks) {
                row[b0 + k] = run;
                run += v[q];
            }
        }
    }
    if (threadIdx.x == blockDim.x - 1) totals[blockIdx.x] = sh[64 + wave] + inc;
}

// Stable compaction of the rows of every directly built child into idx (grouped by parent in
// plan order, object order inside each group).  Each wave walks its own rows with per-leaf
// running offsets in its LDS slice (seeded from the scanned per-wave counts), so the loop
// needs no block barrier: lanes read their group's offset, then one leader per group
// advances it.
// With SPW > 0, the SPW score words of every listed row ([n][SPW] in row order) are written
// beside its index (sp_out[k] = sp_in[idx[k]], [V][SPW]), so the next fill reads the statistics
// of its rows in order instead of gathering them.
// The level's plan (the smaller child of every parent, ties to the TRUE child, tree.rs:1109, and
// the segment offsets of the next fill) comes from the children's totals: every block derives it
// (at most 128 parents, one wave) and block 0 stores it for the kernels after.
template <int SPW>
static __global__ __launch_bounds__(256) void compact_kernel(const uint16_t* __restrict__ leaf, uint64_t n,
                                                      uint32_t level, const uint32_t* __restrict__ cnt,
                                                      uint32_t n_waves, const uint32_t* __restrict__ totals,
                                                      LevelPlan* __restrict__ plan,
                                                      uint32_t* __restrict__ idx,
                                                      const unsigned long long* __restrict__ sp_in,
                                                      unsigned long long* __restrict__ sp_out) {
    __shared__ uint32_t run[4][kMaxLeaves / 2];
    __shared__ uint32_t built[kMaxLeaves / 2];
    __shared__ uint32_t segb[kMaxLeaves / 2];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t n_parent = 1u << level;
    const uint64_t wid = (uint64_t)blockIdx.x * 4 + wave;
    static_assert(kMaxLeaves / 2 <= 128, "two parents per lane of one wave");
    if (wave == 0) {
        uint32_t sz[2], inc[2];
#pragma unroll
        for (uint32_t q = 0; q < 2; ++q) {
            const uint32_t p = lane + 64u * q;
            sz[q] = 0;
            if (p < n_parent) {
                const uint32_t nf = totals[p], nt = totals[p + n_parent];
                const bool true_smaller = nt <= nf;
                built[p] = true_smaller ? p + n_parent : p;
                sz[q] = true_smaller ? nt : nf;
            }
            inc[q] = sz[q];
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t u = __shfl_up(inc[q], o, 64);
                if (lane >= (uint32_t)o) inc[q] += u;
            }
        }
        const uint32_t tot0 = __shfl(inc[0], 63, 64), tot1 = __shfl(inc[1], 63, 64);
        const uint32_t b0 = inc[0] - sz[0], b1 = tot0 + inc[1] - sz[1];
        if (lane < n_parent) segb[lane] = b0;
        if (lane + 64u < n_parent) segb[lane + 64u] = b1;
        if (blockIdx.x == 0) {
            if (lane < n_parent) {
                plan->built[lane] = built[lane];
                plan->seg_begin[lane] = b0;
            }
            if (lane + 64u < n_parent) {
                plan->built[lane + 64u] = built[lane + 64u];
                plan->seg_begin[lane + 64u] = b1;
            }
            if (lane == 0) {
                plan->n_parent = n_parent;
                plan->rows = tot0 + tot1;
            }
        }
    }
    __syncthreads();
    for (uint32_t p = lane; p < n_parent; p += 64)
        run[wave][p] = segb[p] + cnt[(size_t)built[p] * n_waves + wid];
    __syncthreads();
    const uint64_t beg = wid * kPartWaveRows;
    const uint64_t end = min(beg + kPartWaveRows, n);
    constexpr int U = kPartWaveRows / 64;
    uint32_t lfs[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {   // all loads in flight before the first use
        const uint64_t i = beg + (uint64_t)u * 64 + lane;
        lfs[u] = i < end ? leaf[i] : 0x8000u;
    }
    // listed rows: key = parent, valid = the row lies in its parent's directly built child
    uint32_t vmask = 0;   // validity bit per u
    uint32_t key_of[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t lf = lfs[u];
        const uint32_t p = lf & (n_parent - 1u);
        const bool valid = !(lf & 0x8000u) && built[p] == lf;
        key_of[u] = valid ? p : 0u;
        vmask |= (valid ? 1u : 0u) << u;
    }
    // the statistics: every listed row's words are loaded before the first store, so the wave
    // waits for memory once, not once per 64 rows
    constexpr int SW = SPW > 0 ? SPW : 1;
    unsigned long long spv[U][SW];
    if (SPW > 0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t i = beg + (uint64_t)u * 64 + lane;
            const bool valid = (vmask >> u) & 1u;
#pragma unroll
            for (int c = 0; c < SW; ++c) spv[u][c] = valid ? sp_in[i * SW + c] : 0ull;
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint64_t i = beg + (uint64_t)u * 64 + lane;
        const bool valid = (vmask >> u) & 1u;
        const uint32_t key = key_of[u];
        const uint64_t mask = wave_peers(key, valid, level);
        const uint32_t rank = mbcnt64(mask);
        const uint32_t base = valid ? run[wave][key] : 0u;
        if (valid) idx[base + rank] = (uint32_t)i;
        if (SPW > 0 && valid) {
#pragma unroll
            for (int c = 0; c < SW; ++c) sp_out[(size_t)(base + rank) * SW + c] = spv[u][c];
        }
        if (valid && rank == 0) run[wave][key] = base + (uint32_t)__popcll(mask);
    }
}

// ---------------------------------------------------------------------------------
// CTR columns.  (1) The model_size_reg weight needs, once the tree holds a float split, the
// number of distinct (float-partition leaf, bucket) pairs of every CTR-eligible categorical
// column (phantom_mixed_bucket_count, tree.rs:3093-3178): a bitmap [bucket][leaf] per column,
// set per block in LDS and OR-ed into the global bitmap once per block (a hot category would
// otherwise put every one of its rows on one global word), then popcounted.  (2) Leaf values
// and the approximant use the partition in which each CTR level re-tests the column built
// under the averaging permutation (assign_leaf_over_ctr_columns, boosting.rs:2905).
// ---------------------------------------------------------------------------------
constexpr uint32_t kPhantomLdsWords = 16384;   // 64 KiB of bitmap per block
constexpr uint32_t kPhantomBlocks = 32;        // row chunks per column
constexpr uint32_t kPhantomThreads = 1024;     // a block's rows in flight: its loop is latency-bound

// Block g of column c sets its rows' (bucket, float leaf) bits in an LDS bitmap and stores
// it whole into its own slice of part (no global atomics: a hot category would otherwise
// put thousands of atomics on one word); a column too large for LDS sets its slice directly.
// Leaf bits of the splits before `level` on float columns (features below fc0).
__device__ __forceinline__ uint32_t float_split_mask(const SplitRec* __restrict__ splits, uint32_t level,
                                                     uint32_t fc0) {
    uint32_t m = 0;
    for (uint32_t l = 0; l < level; ++l)
        if (splits[l].feature < fc0) m |= 1u << l;
    return m;
}

// float_mask < 0: taken from the device splits (float_split_mask); a level with no float split
// yet sets nothing (its phantom count is not used).  Buckets are 16-bit (every column under
// 65536 buckets) or 32-bit (TB).  Block (0, c) first clears cnt[c], which phantom_count_kernel's
// blocks then add into.
template <typename TB>
static __global__ __launch_bounds__(kPhantomThreads) void phantom_bits_kernel(
    const uint16_t* __restrict__ leaf, uint64_t n, int64_t float_mask_arg, uint32_t L,
    const TB* __restrict__ cat_bk, const uint32_t* __restrict__ cat_nb,
    const uint64_t* __restrict__ word_off, uint32_t* __restrict__ part, const SplitRec* __restrict__ splits,
    uint32_t level, uint32_t fc0, const uint8_t* __restrict__ skip /* nullable: set = no count needed */,
    uint64_t m_lo, unsigned long long* __restrict__ cnt) {
    extern __shared__ uint32_t lbits[];
    if (blockIdx.x == 0 && threadIdx.x == 0) cnt[blockIdx.y] = 0;
    if (skip && *skip) return;
    const uint32_t float_mask =
        float_mask_arg >= 0 ? (uint32_t)float_mask_arg : float_split_mask(splits, level, fc0);
    if (float_mask == 0) return;
    const uint32_t c = blockIdx.y, g = blockIdx.x;
    // a column with at most m_lo possible pairs cannot raise the max count above m_lo
    if ((uint64_t)cat_nb[c] << __popc(float_mask) <= m_lo) return;
    const uint64_t words = ((uint64_t)cat_nb[c] * L + 31) / 32;
    const bool lds = words <= kPhantomLdsWords;
    uint32_t* slice = part + word_off[c] + (uint64_t)g * words;
    uint32_t* bits = lds ? lbits : slice;   // a block owns its slice: it clears it itself
    for (uint64_t w = threadIdx.x; w < words; w += blockDim.x) bits[w] = 0;
    __syncthreads();
    const TB* bk = cat_bk + (size_t)c * n;
    const uint64_t per = (n + gridDim.x - 1) / gridDim.x;
    const uint64_t beg = (uint64_t)g * per;
    const uint64_t end = min(beg + per, n);
    // a bit already set is only read (reads of one word broadcast; the atomic, which a hot
    // category would serialize across the lanes of a wave, runs only for a first occurrence)
    // rows are loaded kU at a time before any is used (the loop is otherwise one memory
    // round trip per row)
    constexpr int kU = 16;
    for (uint64_t i0 = beg + threadIdx.x; i0 < end; i0 += (uint64_t)kU * blockDim.x) {
        uint32_t b[kU], lf[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const uint64_t i = i0 + (uint64_t)u * blockDim.x;
            b[u] = i < end ? (uint32_t)bk[i] : 0xFFFFFFFFu;
            lf[u] = i < end ? (uint32_t)leaf[i] : 0u;
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            if (b[u] == 0xFFFFFFFFu) continue;
            const uint64_t bit = (uint64_t)b[u] * L + (lf[u] & float_mask);
            const uint32_t m = 1u << (bit & 31u);
            uint32_t* wp = lds ? &lbits[bit >> 5] : &slice[bit >> 5];
            if (!(*wp & m)) atomicOr(wp, m);
        }
    }
    if (!lds) return;
    __syncthreads();
    for (uint32_t w = threadIdx.x; w < words; w += blockDim.x) slice[w] = lbits[w];
}

// distinct pairs of every column: OR of its kPhantomBlocks slices, popcounted; grid (column,
// kPhantomCountSplit word ranges), each block adding its popcount to cnt[c] (cleared by
// phantom_bits_kernel)
constexpr uint32_t kPhantomCountSplit = 16;
static __global__ __launch_bounds__(256) void phantom_count_kernel(const uint32_t* __restrict__ part,
                                                                   const uint64_t* __restrict__ word_off,
                                                                   const uint32_t* __restrict__ cat_nb, uint32_t L,
                                                                   unsigned long long* __restrict__ cnt,
                                                                   const SplitRec* __restrict__ splits,
                                                                   uint32_t level, uint32_t fc0,
                                                                   const uint8_t* __restrict__ skip,
                                                                   int64_t float_mask_arg, uint64_t m_lo) {
    __shared__ unsigned long long red[4];
    const uint32_t c = blockIdx.x;
    const uint32_t fm = float_mask_arg >= 0 ? (uint32_t)float_mask_arg : float_split_mask(splits, level, fc0);
    if ((skip && *skip) || fm == 0 || ((uint64_t)cat_nb[c] << __popc(fm)) <= m_lo) return;   // no count
    const uint64_t words = ((uint64_t)cat_nb[c] * L + 31) / 32;
    const uint64_t per = (words + gridDim.y - 1) / gridDim.y;
    const uint64_t w0 = (uint64_t)blockIdx.y * per, w1 = min(w0 + per, words);
    const uint32_t* base = part + word_off[c];
    unsigned long long acc = 0;
    for (uint64_t w = w0 + threadIdx.x; w < w1; w += blockDim.x) {
        uint32_t v[kPhantomBlocks];
#pragma unroll
        for (uint32_t g = 0; g < kPhantomBlocks; ++g) v[g] = base[(uint64_t)g * words + w];
        uint32_t o = 0;
#pragma unroll
        for (uint32_t g = 0; g < kPhantomBlocks; ++g) o |= v[g];
        acc += (unsigned long long)__popc(o);
    }
    for (int d = 32; d > 0; d >>= 1) acc += __shfl_xor(acc, d, 64);
    if (lane_id() == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned long long t = red[0] + red[1] + red[2] + red[3];
        if (t) atomicAdd(cnt + c, t);
    }
}

// model_size_reg weights of the CTR columns for one level, on the device: a column whose
// (type, projection) group is in the model (group_used, from earlier trees) or in this tree's
// earlier levels scores with weight 1; any other with pow_table[c][max_count - m_lo], the
// host's pow(1 + bc_c / m, -model_size_reg) for every m in [m_lo, m_hi], where max_count is
// the larger of the eligible maximum m_lo and the phantom counts once a float split is in the
// tree (tree.rs:3093-3178, 3340-3346).
static __global__ __launch_bounds__(64) void ctr_weights_kernel(
    const SplitRec* __restrict__ splits, uint32_t level, uint32_t fc0, uint32_t ctr_n,
    const uint32_t* __restrict__ group, const uint8_t* __restrict__ group_used,
    const unsigned long long* __restrict__ phantom_cnt, uint32_t cat_n, const double* __restrict__ pow_table,
    uint64_t m_lo, uint64_t m_hi, int msr_zero, double* __restrict__ fweight) {
    uint64_t max_count = m_lo;
    if (cat_n && float_split_mask(splits, level, fc0) != 0)
        for (uint32_t c = 0; c < cat_n; ++c) max_count = max(max_count, (uint64_t)phantom_cnt[c]);
    max_count = min(max_count, m_hi);   // the table covers every reachable count
    const uint64_t span = m_hi - m_lo + 1;
    for (uint32_t c = threadIdx.x; c < ctr_n; c += blockDim.x) {
        bool used = group_used[group[c]] != 0;
        for (uint32_t l = 0; l < level; ++l)
            if (splits[l].feature >= fc0 && group[splits[l].feature - fc0] == group[c]) used = true;
        fweight[fc0 + c] = (used || msr_zero) ? 1.0 : pow_table[(size_t)c * span + (max_count - m_lo)];
    }
}

static __global__ __launch_bounds__(256) void averaging_leaf_kernel(uint16_t* __restrict__ leaf, uint64_t n,
                                                                    const SplitRec* __restrict__ splits,
                                                                    uint32_t depth, uint32_t fc0,
                                                                    const uint8_t* __restrict__ avg) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
        uint32_t lf = leaf[i];
        for (uint32_t l = 0; l < depth; ++l) {
            const SplitRec sp = splits[l];
            if (sp.feature < fc0) continue;
            const uint32_t bit = avg[(size_t)(sp.feature - fc0) * n + i] > sp.bin ? 1u : 0u;
            lf = (lf & ~(1u << l)) | (bit << l);
        }
        leaf[i] = (uint16_t)lf;
    }
}

// ---------------------------------------------------------------------------------
// Leaf statistics on the UNSAMPLED derivatives (boosting.rs:2470-2560, :2634): per leaf
// sum(w * der1[d]) and sum(w) (Gradient) / sum(w * der2) (Newton) / packed sum(w * H)
// (MultiClass), exact in fixed point.  LDS accumulators per block, global atomics.
// ---------------------------------------------------------------------------------
// Per-leaf sums over ALL rows (unsampled, boosting.rs:2470-2560), int64 fixed point.
// K == 1 cells: [sum w der1, sum (Newton: w der2 | Gradient: weight), document count];
// the count is filled for pair losses (centring of the leaf values), else left 0.
template <int K>
constexpr int leaf_cells() { return K == 1 ? 3 : K + K * (K + 1) / 2; }

constexpr uint32_t kLeafThreads = 1024;
template <int K>
static __global__ __launch_bounds__(kLeafThreads) void leaf_reduce_kernel(
    uint64_t n, int loss, int newton, const double* __restrict__ approx,
    const double* __restrict__ target, const double* __restrict__ weight,
    const uint16_t* __restrict__ leaf, const Scales* __restrict__ sc, uint32_t n_leaves,
    long long* __restrict__ out, const double* __restrict__ ext_der,
    const double* __restrict__ score_w) {
    constexpr int CL = leaf_cells<K>();
    extern __shared__ long long acc[];
    const uint32_t cells = n_leaves * CL;
    for (uint32_t i = threadIdx.x; i < cells; i += blockDim.x) acc[i] = 0;
    __syncthreads();
    const double md = sc->mul[kLeafDer], mw = sc->mul[kLeafW];
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t l = leaf[i] & 0x7FFFu;
        const double w = weight ? weight[i] : 1.0;
        unsigned long long* cell = (unsigned long long*)(acc + (size_t)l * CL);
        if (K == 1) {
            double g, h;
            if (ext_der) {
                g = ext_der[i];
                h = ext_der[n + i];
            } else {
                scalar_ders(loss, approx[i], target[i], g, h);
            }
            const double hw = score_w ? score_w[i] : w;
            atomicAdd(cell, (unsigned long long)to_fixed(g * w, md));
            atomicAdd(cell + 1, (unsigned long long)to_fixed(newton ? h * w : hw, mw));
            if (ext_der) atomicAdd(cell + 2, 1ull);
        } else {
            double a[K], p[K];
#pragma unroll
            for (int d = 0; d < K; ++d) a[d] = approx[(size_t)d * n + i];
            softmax_probs<K>(a, p);
            const int tc = (int)target[i];
#pragma unroll
            for (int d = 0; d < K; ++d) {
                double g = -p[d];
                if (d == tc) g += 1.0;
                atomicAdd(cell + d, (unsigned long long)to_fixed(g * w, md));
            }
            int j = 0;
#pragma unroll
            for (int y = 0; y < K; ++y) {
                atomicAdd(cell + K + j, (unsigned long long)to_fixed((p[y] * (p[y] - 1.0)) * w, mw));
                ++j;
                for (int x = y + 1; x < K; ++x) {
                    atomicAdd(cell + K + j, (unsigned long long)to_fixed((p[y] * p[x]) * w, mw));
                    ++j;
                }
            }
        }
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < cells; i += blockDim.x)
        if (acc[i] != 0) atomicAdd((unsigned long long*)(out + i), (unsigned long long)acc[i]);
}

__device__ inline int cholesky_solve_dev(int k, double* a, const double* b, double* x) {
    double l[kMaxK * kMaxK];
    double y[kMaxK];
    for (int i = 0; i < k * k; ++i) l[i] = 0.0;
    for (int i = 0; i < k; ++i) {
        for (int j = 0; j <= i; ++j) {
            double sum = a[i * k + j];
            for (int p = 0; p < j; ++p) sum -= l[i * k + p] * l[j * k + p];
            if (i == j) {
                if (sum <= 0.0) return 0;
                l[i * k + j] = sqrt(sum);
            } else {
                double ljj = l[j * k + j];
                if (ljj == 0.0) return 0;
                l[i * k + j] = sum / ljj;
            }
        }
    }
    for (int i = 0; i < k; ++i) {
        double sum = b[i];
        for (int p = 0; p < i; ++p) sum -= l[i * k + p] * y[p];
        y[i] = sum / l[i * k + i];
    }
    for (int i = k - 1; i >= 0; --i) {
        double sum = y[i];
        for (int p = i + 1; p < k; ++p) sum -= l[p * k + i] * x[p];
        x[i] = sum / l[i * k + i];
    }
    return 1;
}

// Leaf values (leaf.rs:161-335): one thread per leaf.  raw[leaf][d] unscaled, scaled =
// raw * learning_rate (NormalizeLeafValues, boosting.rs:2879-2881).
template <int K>
static __global__ void leaf_values_kernel(const long long* __restrict__ sums, const Scales* __restrict__ sc,
                                   uint32_t n_leaves, int newton, double l2, double lr,
                                   double* __restrict__ raw, double* __restrict__ scaled) {
    constexpr int CL = leaf_cells<K>();
    const uint32_t l = blockIdx.x * blockDim.x + threadIdx.x;
    if (l >= n_leaves) return;
    const long long* s = sums + (size_t)l * CL;
    const double id = sc->inv[kLeafDer], iw = sc->inv[kLeafW];
    if (K == 1) {
        const double sd = (double)s[0] * id;
        const double sw = (double)s[1] * iw;
        double v;
        if (newton) {
            const double den = -sw + l2;
            v = den == 0.0 ? 0.0 : sd / den;
        } else {
            v = sw > 0.0 ? sd / (sw + l2) : 0.0;
        }
        raw[l] = v;
        scaled[l] = v * lr;
        return;
    }
    double h[kMaxK * kMaxK], nd[kMaxK], x[kMaxK];
    int idx = 0;
    for (int i = 0; i < K; ++i)
        for (int j = i; j < K; ++j) {
            const double v = (double)s[K + idx] * iw;
            h[i * K + j] = v;
            h[j * K + i] = v;
            ++idx;
        }
    float max_trace = (float)l2;
    for (int d = 0; d < K; ++d) max_trace = fmaxf(max_trace, (float)(-h[d * K + d]));
    const double adj = (double)fmaxf((float)l2, max_trace * 1.1920928955078125e-7f);
    for (int d = 0; d < K; ++d) h[d * K + d] -= adj;
    for (int i = 0; i < K * K; ++i) h[i] = -h[i];
    for (int d = 0; d < K; ++d) nd[d] = -((double)s[d] * id);
    const int ok = cholesky_solve_dev(K, h, nd, x);
    for (int d = 0; d < K; ++d) {
        const double v = ok ? -x[d] : 0.0;
        raw[(size_t)l * K + d] = v;
        scaled[(size_t)l * K + d] = v * lr;
    }
}

// Exact fixed-point histogram -> f64 (kernel-level entry point and tests).
// h is [slot][ch][f][bin]; out is [slot][f][bin][ch].
static __global__ void hist_to_f64_kernel(const long long* __restrict__ h, size_t n_cells, uint32_t C,
                                          uint32_t F, uint32_t B, const Scales* __restrict__ sc,
                                          double* __restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_cells;
         i += (size_t)gridDim.x * blockDim.x) {
        const uint32_t ch = (uint32_t)(i % C);
        size_t r = i / C;
        const uint32_t bin = (uint32_t)(r % B);
        r /= B;
        const uint32_t f = (uint32_t)(r % F);
        const size_t slot = r / F;
        const long long v = h[((slot * C + ch) * F + f) * B + bin];
        out[i] = (double)v * (ch == C - 1 ? sc->inv[kScoreW] : sc->inv[kScoreDer]);
    }
}

}  // namespace cbh
