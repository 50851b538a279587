// Ranking kernels of the gfx950 path: PairLogit derivatives over explicit pairs, and the
// pairwise split scoring and leaf solve of PairLogitPairwise.
//
// Pairs are resident in the reference's competitor order (query group ascending, winner
// ascending, input order per winner; crates/cb-train/src/query_info.rs:205-250):
//   comp_win, comp_los  u32 [m]   winner / loser row of pair k
//   comp_w              f64 [m]   pair weight
//   comp_wq             i64 [m]   pair weight in fixed point (x 2^pair_shift, exact sums)
//   comp_off            u32 [n+1] pairs of winner row i are comp_off[i] .. comp_off[i+1]
//   group_off           u32 [G+1] query groups (contiguous rows)
//
// Pairwise statistics of a level (compute_pair_weight_statistics,
// crates/cb-compute/src/pairwise_scoring.rs:163-196) are int64 fixed point, laid out
//   st  i64 [F][P][P][B][2]   (first leaf, second leaf, bucket, {smaller, greater_right})
// and turned into inclusive prefix sums over the bucket axis, so the running per-border
// state of calculate_pairwise_score (:450-560) is read directly at border s.  The bucket runs
// of one (feature, leaf pair) are contiguous: the producers write whole runs.
#pragma once
#include "kernels.hpp"

namespace cbh {

constexpr uint32_t kPairMaxParents = 128;  // pairwise scoring: 2P <= 256 unknowns (depth <= 8)
constexpr uint32_t kPairWaveParents = 32;  // levels of up to 32 leaves: one system per wavefront
constexpr size_t kPairLdsMax = 160 * 1024;   // LDS of one workgroup (gfx950)
constexpr uint32_t kPairCandGlobalWgs = 1024; // persistent workgroups of the 128-leaf candidate solves
constexpr uint32_t kPairChunk = 65536;     // pairs per workgroup of the LDS statistics kernel
constexpr uint32_t kPairLoadAhead = 8;      // pairs whose gathers one thread issues together
constexpr uint32_t kKeyLoadAhead = 8;       // the same for the keyed statistics
constexpr uint32_t kKeyWords = 4;           // row words of one pair loaded together

__device__ __forceinline__ uint32_t tri(uint32_t r, uint32_t c) {   // packed lower triangle
    return r >= c ? r * (r + 1) / 2 + c : c * (c + 1) / 2 + r;
}

// pairlogit_pair_prob (crates/cb-compute/src/loss.rs:640-651).
__device__ __forceinline__ double pairlogit_p(double winner_approx, double loser_approx) {
    const double el = exp(loser_approx), ew = exp(winner_approx);
    const double den = el + ew;
    return den > 0.0 ? el / den : 0.5;
}

// PairLogit derivatives, one thread per query group (pairlogit_group_der,
// crates/cb-compute/src/ranking_der.rs:408-445): rows of the group ascending, each winner's
// pairs in order, a loser's derivatives decremented as its winners are visited and a
// winner's own sums added after its pair loop -- the reference's accumulation order.  The
// thread first applies the previous tree's leaf values to its rows (the rows of a group
// belong to it alone).
static __global__ __launch_bounds__(256) void pairlogit_ders_kernel(
    const uint32_t* __restrict__ group_off, uint32_t n_groups, const uint32_t* __restrict__ comp_off,
    const uint32_t* __restrict__ comp_los, const double* __restrict__ comp_w,
    double* __restrict__ approx, const uint16_t* __restrict__ leaf,
    const double* __restrict__ pending /* [leaves] lr-scaled, nullable */,
    double* __restrict__ der1, double* __restrict__ der2) {
    const uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n_groups) return;
    const uint32_t b = group_off[g], e = group_off[g + 1];
    if (pending)
        for (uint32_t i = b; i < e; ++i) approx[i] += pending[leaf[i] & 0x7FFFu];
    for (uint32_t i = b; i < e; ++i) {
        der1[i] = 0.0;
        der2[i] = 0.0;
    }
    for (uint32_t doc = b; doc < e; ++doc) {
        const double wa = approx[doc];
        double wd = 0.0, wd2 = 0.0;
        for (uint32_t k = comp_off[doc]; k < comp_off[doc + 1]; ++k) {
            const uint32_t l = comp_los[k];
            const double p = pairlogit_p(wa, approx[l]);
            const double w = comp_w[k];
            wd += w * p;
            wd2 += w * p * (p - 1.0);
            der1[l] -= w * p;
            der2[l] += w * p * (p - 1.0);
        }
        der1[doc] += wd;
        der2[doc] += wd2;
    }
}

// Leaves of both rows of every pair for one level: pair_lv[k] = winner leaf | loser leaf << 16.
static __global__ __launch_bounds__(256) void pair_leaves_kernel(const uint32_t* __restrict__ comp_win,
                                                                 const uint32_t* __restrict__ comp_los, uint64_t m,
                                                                 const uint16_t* __restrict__ leaf,
                                                                 uint32_t* __restrict__ pair_lv) {
    for (uint64_t k = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; k < m; k += (uint64_t)gridDim.x * blockDim.x)
        pair_lv[k] = (leaf[comp_win[k]] & 0x7FFFu) | ((uint32_t)(leaf[comp_los[k]] & 0x7FFFu) << 16);
}

// Pair-weight statistics of one level for every feature.  For a
// pair with winner bucket > loser bucket the cells [loserLeaf][winnerLeaf] are decremented at
// (loser bucket, smaller) and (winner bucket, greater); otherwise [winnerLeaf][loserLeaf] at
// (winner bucket, smaller) and (loser bucket, greater).  The P*P*B*2 cells of the feature fit
// in LDS (P <= 4): a workgroup accumulates its chunk there, then adds it to st.  In LDS the
// two channels of a leaf pair are separate runs of B ([P][P][2][B]), so a wave's atomics on
// random buckets spread over every bank.
static __global__ __launch_bounds__(256) void pair_stats_kernel(
    const uint8_t* __restrict__ cols, uint64_t n, const uint32_t* __restrict__ pair_lv,
    const uint32_t* __restrict__ comp_win, const uint32_t* __restrict__ comp_los,
    const long long* __restrict__ comp_wq, uint64_t m, uint32_t n_chunks, uint32_t F, uint32_t P, uint32_t B,
    long long* __restrict__ st) {
    extern __shared__ long long sh_st[];
    // 1-D grid of 8 * n_chunks * ceil(F / 8) blocks, round-robin over the 8 XCDs: all chunks of
    // a feature run on one XCD, which keeps its bucket column in that XCD's L2
    const uint32_t xcd = blockIdx.x & 7u, q = blockIdx.x >> 3;
    const uint32_t f = xcd + 8u * (q / n_chunks), chunk = q % n_chunks;
    if (f >= F) return;
    const size_t cells = (size_t)B * P * P * 2;
    unsigned long long* out = (unsigned long long*)(st + (size_t)f * cells);
    unsigned long long* acc = (unsigned long long*)sh_st;
    for (size_t i = threadIdx.x; i < cells; i += blockDim.x) sh_st[i] = 0;
    __syncthreads();
    const uint8_t* col = cols + (size_t)f * n;
    const uint64_t k0 = (uint64_t)chunk * kPairChunk;
    const uint64_t k1 = min(k0 + kPairChunk, m);
    // kPairLoadAhead pairs per thread at a time: their indices, then all their bucket and leaf
    // gathers, are in flight together (the loop is latency-bound otherwise)
    for (uint64_t kb = k0 + threadIdx.x; kb < k1; kb += (uint64_t)blockDim.x * kPairLoadAhead) {
        uint32_t wi[kPairLoadAhead], lo[kPairLoadAhead], lv[kPairLoadAhead];
        long long wq[kPairLoadAhead];
#pragma unroll
        for (uint32_t u = 0; u < kPairLoadAhead; ++u) {
            const uint64_t k = kb + (uint64_t)u * blockDim.x;
            const bool ok = k < k1;
            wi[u] = ok ? comp_win[k] : 0u;
            lo[u] = ok ? comp_los[k] : 0u;
            lv[u] = ok ? pair_lv[k] : 0u;
            wq[u] = ok ? comp_wq[k] : 0;
        }
        uint32_t wb[kPairLoadAhead], lb[kPairLoadAhead], wl[kPairLoadAhead], ll[kPairLoadAhead];
#pragma unroll
        for (uint32_t u = 0; u < kPairLoadAhead; ++u) {
            wb[u] = col[wi[u]];
            lb[u] = col[lo[u]];
            wl[u] = lv[u] & 0x7FFFu;
            ll[u] = (lv[u] >> 16) & 0x7FFFu;
        }
#pragma unroll
        for (uint32_t u = 0; u < kPairLoadAhead; ++u) {
            if (kb + (uint64_t)u * blockDim.x >= k1 || wi[u] == lo[u]) continue;
            const unsigned long long neg = (unsigned long long)(-wq[u]);
            const bool wg = wb[u] > lb[u];
            const size_t run = ((size_t)(wg ? ll[u] : wl[u]) * P + (wg ? wl[u] : ll[u])) * 2 * B;
            atomicAdd(acc + run + (wg ? lb[u] : wb[u]), neg);
            atomicAdd(acc + run + B + (wg ? wb[u] : lb[u]), neg);
        }
    }
    __syncthreads();
    for (size_t i = threadIdx.x; i < cells; i += blockDim.x) {   // st index i = (pair, bucket, c)
        const size_t pr = i / (2 * B), rem = i % (2 * B);
        const long long v = sh_st[(pr * 2 + (rem & 1)) * B + (rem >> 1)];
        if (v != 0) atomicAdd(out + i, (unsigned long long)v);
    }
}

// ---- statistics with many parents (P >= 8): pairs grouped by their unordered leaf pair
// {a, b}; one workgroup per (feature, leaf pair) owns the cells [a][b][*][*] and [b][a][*][*]
// of that feature, accumulates them in LDS, takes the prefix over buckets and writes the
// cumulative values (no zeroing, no global atomics, no separate scan).

__device__ __forceinline__ uint32_t pair_key(uint32_t wl, uint32_t ll, uint32_t P) {
    return wl < ll ? wl * P + ll : ll * P + wl;
}

// Count the pairs of every key (P*P keys, those with a > b stay 0).
static __global__ __launch_bounds__(256) void pair_key_count_kernel(
    const uint32_t* __restrict__ comp_win, const uint32_t* __restrict__ comp_los, uint64_t m,
    const uint16_t* __restrict__ leaf, uint32_t P, uint32_t* __restrict__ cnt) {
    extern __shared__ uint32_t c[];   // [P * P]
    for (uint32_t i = threadIdx.x; i < P * P; i += blockDim.x) c[i] = 0;
    __syncthreads();
    for (uint64_t k = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; k < m;
         k += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t wi = comp_win[k], lo = comp_los[k];
        if (wi == lo) continue;
        atomicAdd(&c[pair_key(leaf[wi] & 0x7FFFu, leaf[lo] & 0x7FFFu, P)], 1u);
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < P * P; i += blockDim.x)
        if (c[i]) atomicAdd(cnt + i, c[i]);
}

// Exclusive scan of the P*P key counts (one workgroup of 1024 threads, each over a run of
// ceil(nk / 1024) consecutive keys): key_off[P*P + 1], cursor = key_off[0 .. P*P).
static __global__ __launch_bounds__(1024) void pair_key_scan_kernel(const uint32_t* __restrict__ cnt, uint32_t nk,
                                                                    uint32_t* __restrict__ key_off,
                                                                    uint32_t* __restrict__ cursor) {
    __shared__ uint32_t sh[1024];
    const uint32_t t = threadIdx.x;
    const uint32_t per = (nk + 1023) / 1024;
    const uint32_t k0 = min(t * per, nk), k1 = min(k0 + per, nk);
    uint32_t v = 0;
    for (uint32_t k = k0; k < k1; ++k) v += cnt[k];
    sh[t] = v;
    __syncthreads();
    for (uint32_t o = 1; o < 1024; o <<= 1) {
        const uint32_t a = t >= o ? sh[t - o] : 0u;
        __syncthreads();
        sh[t] += a;
        __syncthreads();
    }
    uint32_t run = sh[t] - v;
    for (uint32_t k = k0; k < k1; ++k) {
        key_off[k] = run;
        cursor[k] = run;
        run += cnt[k];
    }
    if (t == 1023) key_off[nk] = sh[t];
}

// Scatter the pairs by key as compact records (order inside a key is free: the sums are
// exact integers): rec = (winner, loser | winner-in-leaf-a << 31), weight in fixed point.
// Each workgroup takes kScatterItems pairs per thread, ranks them per key in LDS, reserves one
// range per key with a single global atomic, then writes.
constexpr uint32_t kScatterItems = 8;
static __global__ __launch_bounds__(256) void pair_key_scatter_kernel(
    const uint32_t* __restrict__ comp_win, const uint32_t* __restrict__ comp_los,
    const long long* __restrict__ comp_wq, uint64_t m, const uint16_t* __restrict__ leaf, uint32_t P,
    uint32_t* __restrict__ cursor, uint2* __restrict__ rec, long long* __restrict__ rec_wq) {
    extern __shared__ uint32_t lcnt[];   // [P * P]
    const uint32_t nk = P * P;
    for (uint32_t i = threadIdx.x; i < nk; i += blockDim.x) lcnt[i] = 0;
    __syncthreads();
    const uint64_t base = (uint64_t)blockIdx.x * blockDim.x * kScatterItems;
    uint32_t key[kScatterItems], slot[kScatterItems];
    for (uint32_t r = 0; r < kScatterItems; ++r) {
        const uint64_t k = base + (uint64_t)r * blockDim.x + threadIdx.x;
        key[r] = 0xFFFFFFFFu;
        if (k < m) {
            const uint32_t wi = comp_win[k], lo = comp_los[k];
            if (wi != lo) {
                key[r] = pair_key(leaf[wi] & 0x7FFFu, leaf[lo] & 0x7FFFu, P);
                slot[r] = atomicAdd(&lcnt[key[r]], 1u);
            }
        }
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < nk; i += blockDim.x)
        if (lcnt[i]) lcnt[i] = atomicAdd(cursor + i, lcnt[i]);   // count -> reserved base
    __syncthreads();
    for (uint32_t r = 0; r < kScatterItems; ++r) {
        if (key[r] == 0xFFFFFFFFu) continue;
        const uint64_t k = base + (uint64_t)r * blockDim.x + threadIdx.x;
        const uint32_t wi = comp_win[k], lo = comp_los[k];
        const uint32_t pos = lcnt[key[r]] + slot[r];
        const uint32_t wl = leaf[wi] & 0x7FFFu, ll = leaf[lo] & 0x7FFFu;
        rec[pos] = make_uint2(wi, lo | ((wl <= ll ? 1u : 0u) << 31));
        rec_wq[pos] = comp_wq[k];
    }
}

// Feature tiles of the keyed statistics: tf features (a multiple of 4, whole row words) whose
// cells [tf][2][B][2] fit the LDS budget.
inline uint32_t pair_tile_features(uint32_t F, uint32_t B, size_t budget) {
    const size_t per_f = (size_t)2 * B * 2 * sizeof(long long);
    uint32_t tf = (uint32_t)(budget / per_f) & ~3u;
    if (tf < 4) tf = 4;
    return std::min<uint32_t>(tf, (F + 3) / 4 * 4);
}

// Inclusive prefix, in place, of nseq contiguous runs of B values in LDS (run q starts at
// base + q B): a workgroup-wide two-level scan, tps threads per run.
__device__ inline void lds_runs_prefix(unsigned long long* base, uint32_t nseq, uint32_t B,
                                       unsigned long long* part /* [blockDim.x] */) {
    uint32_t tps = 1;
    while (tps * 2 * nseq <= blockDim.x && tps * 2 <= 64) tps *= 2;
    const uint32_t t = threadIdx.x, q = t / tps, j = t % tps;
    const uint32_t chunk = (B + tps - 1) / tps;
    const uint32_t b0 = min(j * chunk, B), b1 = min(b0 + chunk, B);
    unsigned long long* p = q < nseq ? base + (size_t)q * B : nullptr;
    unsigned long long run = 0;
    if (p)
        for (uint32_t bb = b0; bb < b1; ++bb) {
            run += p[bb];
            p[bb] = run;
        }
    part[t] = run;
    __syncthreads();
    if (p && j > 0) {
        unsigned long long off = 0;
        for (uint32_t i = 0; i < j; ++i) off += part[q * tps + i];
        for (uint32_t bb = b0; bb < b1; ++bb) p[bb] += off;
    }
    __syncthreads();
}

// One workgroup per (leaf pair {a <= b}, feature tile).  Each pair reads the row words of its
// winner and loser once for the whole tile.  Writes the cumulative statistics of the cells [a][b] and
// [b][a] of the tile's features, whole bucket runs (every cell of st is written once per
// level: no zeroing, no global atomics, no separate scan).
static __global__ __launch_bounds__(256) void pair_stats_key_kernel(
    const uint32_t* __restrict__ rows, uint32_t W, const uint2* __restrict__ rec,
    const long long* __restrict__ rec_wq, const uint32_t* __restrict__ key_off, uint32_t F,
    uint32_t P, uint32_t B, uint32_t tf, uint32_t n_tiles, long long* __restrict__ st) {
    extern __shared__ unsigned long long cell_k[];   // [tf][blk][c][bucket]
    // block ids go round-robin over the 8 XCDs: the tiles of one leaf pair run on one XCD,
    // consecutively, so the rows its pairs gather come from that XCD's L2 after the first tile
    const uint32_t bid = blockIdx.x;
    const uint32_t xcd = bid & 7u, q = bid >> 3;
    const uint32_t tile = q % n_tiles;
    const uint32_t idx = (q / n_tiles) * 8u + xcd;   // leaf pair {a <= b}: idx = b (b + 1) / 2 + a
    if (idx >= P * (P + 1) / 2) return;
    uint32_t b = (uint32_t)((sqrtf(8.0f * (float)idx + 1.0f) - 1.0f) * 0.5f);
    while (b * (b + 1) / 2 > idx) --b;
    while ((b + 1) * (b + 2) / 2 <= idx) ++b;
    const uint32_t a = idx - b * (b + 1) / 2;
    const uint32_t key = a * P + b;
    const uint32_t f0 = tile * tf;
    const uint32_t nf = min(tf, F - f0);
    const uint32_t w0 = f0 / 4, nw = (nf + 3) / 4;
    const size_t per_f = (size_t)2 * B * 2;
    for (size_t i = threadIdx.x; i < (size_t)nf * per_f; i += blockDim.x) cell_k[i] = 0;
    __syncthreads();
    const uint32_t j0 = key_off[key], j1 = key_off[key + 1];
    for (uint32_t jb = j0 + threadIdx.x; jb < j1; jb += blockDim.x * kKeyLoadAhead) {
        // kKeyLoadAhead pairs per thread at a time: records first, then kKeyWords row words
        // of each winner and loser, all in flight together
        uint2 r[kKeyLoadAhead];
        long long wq[kKeyLoadAhead];
#pragma unroll
        for (uint32_t u = 0; u < kKeyLoadAhead; ++u) {
            const uint32_t j = jb + u * blockDim.x;
            const bool ok = j < j1;
            r[u] = ok ? rec[j] : make_uint2(0u, 0u);
            wq[u] = ok ? rec_wq[j] : 0;
        }
        for (uint32_t wc = 0; wc < nw; wc += kKeyWords) {
            uint32_t ww[kKeyLoadAhead][kKeyWords], wlw[kKeyLoadAhead][kKeyWords];
#pragma unroll
            for (uint32_t u = 0; u < kKeyLoadAhead; ++u)
#pragma unroll
                for (uint32_t w = 0; w < kKeyWords; ++w) {
                    const uint32_t wa = wc + w < nw ? w0 + wc + w : w0;   // in-row, in-bounds
                    ww[u][w] = rows[(size_t)r[u].x * W + wa];
                    wlw[u][w] = rows[(size_t)(r[u].y & 0x7FFFFFFFu) * W + wa];
                }
#pragma unroll
            for (uint32_t u = 0; u < kKeyLoadAhead; ++u) {
                if (jb + u * blockDim.x >= j1) continue;
                const bool win_in_a = (r[u].y >> 31) != 0;
                const unsigned long long neg = (unsigned long long)(-wq[u]);
#pragma unroll
                for (uint32_t w = 0; w < kKeyWords; ++w) {
                    if (wc + w >= nw) break;
                    for (uint32_t k = 0; k < 4; ++k) {
                        const uint32_t f = 4 * (wc + w) + k;
                        if (f >= nf) break;
                        const uint32_t wb = (ww[u][w] >> (8 * k)) & 0xFFu, lb = (wlw[u][w] >> (8 * k)) & 0xFFu;
                        // first index x = loser leaf when wb > lb, else winner leaf; block 0 = [a][b]
                        const uint32_t blk = a == b ? 0u : ((wb > lb) == win_in_a ? 1u : 0u);
                        const uint32_t bs = wb > lb ? lb : wb, bg = wb > lb ? wb : lb;
                        unsigned long long* c = cell_k + (size_t)f * per_f + (size_t)blk * B * 2;
                        atomicAdd(c + bs, neg);
                        atomicAdd(c + B + bg, neg);
                    }
                }
            }
        }
    }
    __syncthreads();
    // prefix over buckets of every (f, blk, c) run
    __shared__ unsigned long long part[256];
    lds_runs_prefix(cell_k, nf * 4, B, part);
    const uint32_t nblk = a == b ? 1u : 2u;
    for (uint32_t fb = 0; fb < nf * nblk; ++fb) {   // whole contiguous runs of 2B values
        const uint32_t f = fb / nblk, blk = fb % nblk;
        const uint32_t x = blk == 0 ? a : b, y = blk == 0 ? b : a;
        const unsigned long long* src = cell_k + (size_t)f * per_f + (size_t)blk * B * 2;
        long long* dst = st + (((size_t)(f0 + f) * P + x) * P + y) * B * 2;
        for (uint32_t i = threadIdx.x; i < 2 * B; i += blockDim.x) dst[i] = (long long)src[(i & 1u) * B + (i >> 1)];
    }
}

// Inclusive prefix over the bucket axis, in place: one wavefront per (f, x, y, c) run of B
// values at stride 2; lane l takes buckets [l k, l k + k), k = ceil(B / 64), and the lane
// totals are scanned across the wave.
static __global__ __launch_bounds__(256) void pair_scan_kernel(long long* __restrict__ st, uint32_t n_runs,
                                                               uint32_t B) {
    const uint32_t run = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (run >= n_runs) return;
    long long* p = st + (size_t)(run >> 1) * B * 2 + (run & 1u);
    const uint32_t k = (B + 63) / 64;
    const uint32_t b0 = min(lane * k, B), b1 = min(b0 + k, B);
    long long v[4];   // B <= 256
    long long tot = 0;
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
        v[i] = b0 + i < b1 ? p[(size_t)(b0 + i) * 2] : 0;
        tot += v[i];
        v[i] = tot;
    }
    long long incl = tot;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const long long t = __shfl_up(incl, o, 64);
        if ((int)lane >= o) incl += t;
    }
    const long long off = incl - tot;
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i)
        if (b0 + i < b1) p[(size_t)(b0 + i) * 2] = v[i] + off;
}

// MakeZeroAverage (pairwise_scoring.rs:255-265), sequential sum as the reference; every
// thread of the workgroup takes part.
__device__ inline void zero_average_block(double* r, int n) {
    __shared__ double avg_s;
    if (threadIdx.x == 0) {
        double avg = 0.0;
        for (int i = 0; i < n; ++i) avg += r[i];
        avg_s = avg / (double)n;
    }
    __syncthreads();
    const double avg = avg_s;
    for (int i = threadIdx.x; i < n; i += blockDim.x) r[i] -= avg;
    __syncthreads();
}

// In-place Cholesky of the m x m packed system M (right-looking, the reference's row order)
// and the forward / back substitutions of y, by every thread of the workgroup (rows strided
// over the threads); M may be in LDS or global memory.  The forward pass writes its result
// to fwd (y[p] is read by every thread of step p while other rows of y change), the back
// pass to res[0..m); res[m] = 0.  A non-positive pivot gives the zero solution
// (cholesky_solve's failure arm).
__device__ inline void pairwise_factor_solve_block(double* __restrict__ M, int m, double* __restrict__ cj,
                                                   double* __restrict__ y, double* __restrict__ fwd,
                                                   double* __restrict__ res) {
    const int t = threadIdx.x, nt = blockDim.x;
    bool good = true;
    for (int j = 0; j < m; ++j) {
        const double d = M[tri(j, j)];   // the same value in every thread: a uniform exit
        if (d <= 0.0) {
            good = false;
            break;
        }
        const double ljj = sqrt(d);
        for (int i = j + 1 + t; i < m; i += nt) {
            const double v = M[tri(i, j)] / ljj;
            M[tri(i, j)] = v;
            cj[i] = v;
        }
        __syncthreads();
        if (t == 0) M[tri(j, j)] = ljj;
        // trailing update of row i: M[i][k] -= L[i][j] L[k][j], k in (j, i]; the row is
        // contiguous in the packed layout and the pivot column is a separate array
        for (int i = j + 1 + t; i < m; i += nt) {
            const double lij = cj[i];
            double* __restrict__ row = M + i * (i + 1) / 2;
            int k = j + 1;
            for (; k + 3 <= i; k += 4) {
                const double r0 = row[k], r1 = row[k + 1], r2 = row[k + 2], r3 = row[k + 3];
                const double c0 = cj[k], c1 = cj[k + 1], c2 = cj[k + 2], c3 = cj[k + 3];
                row[k] = r0 - lij * c0;
                row[k + 1] = r1 - lij * c1;
                row[k + 2] = r2 - lij * c2;
                row[k + 3] = r3 - lij * c3;
            }
            for (; k <= i; ++k) row[k] = row[k] - lij * cj[k];
        }
        __syncthreads();
    }
    if (good) {
        for (int p = 0; p < m; ++p) {   // forward: y[i] -= L[i][p] y[p], p ascending
            const double yp = y[p] / M[tri(p, p)];
            if (t == 0) fwd[p] = yp;
            for (int i = p + 1 + t; i < m; i += nt) y[i] -= M[tri(i, p)] * yp;
            __syncthreads();
        }
        for (int p = m - 1; p >= 0; --p) {   // back: L^T x = y
            const double xp = fwd[p] / M[tri(p, p)];
            if (t == 0) res[p] = xp;
            for (int i = t; i < p; i += nt) fwd[i] -= M[tri(p, i)] * xp;
            __syncthreads();
        }
    } else {
        for (int i = t; i < m; i += nt) res[i] = 0.0;
    }
    if (t == 0) res[m] = 0.0;
    __syncthreads();
}

// The workgroup solves the pairwise leaf system of n unknowns (calculate_pairwise_leaf_values,
// pairwise_scoring.rs:283-345, pairwise_leaves.rs:120-200): W (packed lower triangle, n x n)
// plus the bucket-weight prior gives the (n-1)x(n-1) SPD matrix M; right-looking Cholesky
// (every element receives its pivot subtractions in ascending order, as the reference's
// left-looking loop applies them), forward and back substitution, res[n-1] = 0, zero
// average.  A non-positive pivot yields zeros.  M holds (n-1) n / 2 doubles (packed);
// cj / y / fwd / res n doubles each.
__device__ inline void pairwise_solve_block(const double* __restrict__ W, const double* __restrict__ der, int n,
                                            double l2, double prior, double* __restrict__ M,
                                            double* __restrict__ cj, double* __restrict__ y,
                                            double* __restrict__ fwd, double* __restrict__ res) {
    const int t = threadIdx.x, nt = blockDim.x;
    const double cell_prior = 1.0 / (double)n;
    const double non_diag = -prior * cell_prior;
    const double diag = prior * (1.0 - cell_prior) + l2;
    if (n <= 2) {
        if (t == 0) {
            if (n == 1) {
                res[0] = 0.0;
            } else {
                const double den = W[0] + diag;
                res[0] = den != 0.0 ? der[0] / den : 0.0;
                res[1] = 0.0;
            }
        }
        __syncthreads();
        if (n == 2) zero_average_block(res, 2);
        return;
    }
    const int m = n - 1;
    for (int r = t; r < m; r += nt) {
        const double* wr = W + r * (r + 1) / 2;
        double* mr = M + r * (r + 1) / 2;
        for (int c = 0; c < r; ++c) mr[c] = wr[c] + non_diag;
        mr[r] = wr[r] + diag;
        y[r] = der[r];
    }
    __syncthreads();
    pairwise_factor_solve_block(M, m, cj, y, fwd, res);
    zero_average_block(res, n);
}

// Doubles of the leaf solve of L leaves: W L (L+1) / 2 | M (L-1) L / 2 | der, cj, y, fwd, res L
// each.  In LDS up to 128 leaves (136 KB), else in a global workspace.
__host__ __device__ constexpr size_t pair_leaf_solve_doubles(uint32_t L) { return (size_t)L * L + 5 * (size_t)L; }

// LDS of the candidate solve (8-byte words): L (packed lower triangle, up to 63 rows; the
// border's statistics once the solve is done) | der, res, part, dgs 64 each.  ~18 KB, so eight
// waves share a CU.
constexpr size_t kPairCandLds = (2080 + 4 * 64) * sizeof(double);
// Leaf pairs whose statistics one lane loads before using any of them.
constexpr uint32_t kPairBatch = 8;

// Entries of row r = 2a + u of the 2P x 2P pairwise weight matrix of one border, read from the
// cumulative statistics R = [P][P][2] at the border and T (the last border's, i.e. totals):
// wp(b) gives (W[r][2b], W[r][2b+1]) for b != a in fixed point; the diagonal block of row r is
// (dg, da) (u == 0) or (da, dg) (u == 1).  Integer sums are exact, so every entry equals the
// staged assembly's bit for bit whatever the order.
struct PairRow {
    const long long* R;   // cell (x, y) at R + (x P + y) rs: {smaller, greater}
    const long long* T;   // cell (x, y) at T + (x P + y) ts: smaller at the last border
    uint32_t rs, ts, P, a, u;
    __device__ inline long long da() const { return R[(a * P + a) * rs] - R[(a * P + a) * rs + 1]; }
    __device__ inline void wp(uint32_t b, long long& e0, long long& e1, long long& dg_part) const {
        const uint32_t yv_ = a < b ? a : b, xv = a < b ? b : a;
        const long long xs = R[(xv * P + yv_) * rs], xg = R[(xv * P + yv_) * rs + 1];
        const long long ys = R[(yv_ * P + xv) * rs], yg = R[(yv_ * P + xv) * rs + 1];
        const long long total = T[(xv * P + yv_) * ts] + T[(yv_ * P + xv) * ts];
        const long long w00 = xg + yg, w01 = xs - xg, w10 = ys - yg, w11 = -(xs + ys);
        if (u == 0) {
            e0 = w00;
            e1 = a > b ? w01 : w10;
            dg_part = a < b ? (w00 + w10) : (w00 + w01);
        } else {
            e0 = a > b ? w10 : w01;
            e1 = w11 + total;
            dg_part = (a < b ? (w01 + w11) : (w10 + w11)) + total;
        }
    }
    __device__ inline long long dg() const {
        long long d = -da();
        for (uint32_t b = 0; b < P; ++b) {
            if (b == a) continue;
            long long e0, e1, part;
            wp(b, e0, e1, part);
            d -= part;
        }
        return d;
    }
};

// Cells (x, y) of one border, {smaller, greater} 16 bytes at stride 2B in st, into Rs[2 PP].
__device__ inline void stage_pair_cells(long long* Rs, const long long* R, uint32_t PP, uint32_t B) {
    for (uint32_t i = threadIdx.x; i < PP; i += blockDim.x) {
        const longlong2 v = *reinterpret_cast<const longlong2*>(R + (size_t)i * 2 * B);
        Rs[2 * i] = v.x;
        Rs[2 * i + 1] = v.y;
    }
}

// The double of lane l (uniform l) on every lane.
__device__ inline double readlane_f64(double v, int l) {
    const long long bits = __double_as_longlong(v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)bits, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(bits >> 32), l);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// One wavefront per (border s, feature f) at a level of P_ leaves: the weight matrix of border
// s from the cumulative pair statistics (calculate_pairwise_score's leaf system,
// pairwise_scoring.rs:471-581), the prior terms, the 2P-1 Cholesky solve, MakeZeroAverage and
// the score.  Lane r holds row r of the system in registers (entries above the diagonal are
// don't-care), so the factorization runs without LDS traffic: the pivot and the pivot column
// come from the owning lanes by readlane, and every element still receives its pivot
// subtractions in ascending order with the reference's roundings (pairwise_factor_solve_block
// is the same arithmetic over memory).  The back substitution reads L^T from LDS; the score
// rebuilds each row of W from the statistics staged over that buffer afterwards.
template <uint32_t P_>
static __global__ __launch_bounds__(64) void pairwise_candidate_kernel(
    const long long* __restrict__ st, const long long* __restrict__ hist, uint32_t C, uint32_t F,
    const uint32_t* __restrict__ n_cand, uint32_t B, const Scales* __restrict__ sc, double pair_inv,
    double l2, double prior, double* __restrict__ scores /* [F][B] */) {
    constexpr uint32_t P = P_;
    constexpr int n = 2 * (int)P_, m = n - 1;
    static_assert(n <= 64, "one row per lane");
    extern __shared__ double sh_pw[];
    // gridDim.x = 8 * ceil((B - 1) / 8): consecutive borders of a feature run on one XCD (block
    // ids go round-robin over the 8 XCDs), where their statistics share L2 lines
    const uint32_t s = (blockIdx.x & 7u) * (gridDim.x >> 3) + (blockIdx.x >> 3), f = blockIdx.y;
    const int lane = threadIdx.x;
    if (s >= B - 1) return;
    if (s >= n_cand[f]) {
        if (lane == 0) scores[(size_t)f * B + s] = -INFINITY;
        return;
    }
    double* M = sh_pw;   // L for the back substitution, then the staged statistics
    double* der = M + 2080;
    double* res = der + 64;
    double* part = res + 64;
    long long* dgs = (long long*)(part + 64);   // W[r][r] per row, kept for the score
    constexpr uint32_t PP = P * P;
    const long long* R = st + (size_t)f * PP * B * 2 + (size_t)s * 2;          // cell stride 2B
    const long long* T = st + (size_t)f * PP * B * 2 + (size_t)(B - 1) * 2;
    const double inv_d = sc->inv[kScoreDer];
    for (uint32_t yl = lane; yl < P; yl += 64) {
        // der channel of the level histogram hist [P][C][F][B], kept as a prefix over bins
        const long long* h = hist + ((size_t)yl * C * F + f) * B;
        const long long dp = h[s], dt = h[B - 1];
        der[2 * yl] = (double)dp * inv_d;
        der[2 * yl + 1] = (double)(dt - dp) * inv_d;
    }
    const double cell_prior = 1.0 / (double)n;
    const double non_diag = -prior * cell_prior;
    const double diag = prior * (1.0 - cell_prior) + l2;
    // this border's cells, one 16-byte load each, staged in LDS (the L buffer is free until
    // the back substitution)
    long long* Rs = (long long*)M;
    stage_pair_cells(Rs, R, PP, B);
    __syncthreads();
    // row r of M = W + prior terms (lanes past the system repeat row 0 and write nothing)
    const int r = lane < n ? lane : 0;
    const PairRow pr{Rs, T, 2, 2 * B, P, (uint32_t)r >> 1, (uint32_t)r & 1u};
    const long long da = pr.da();
    long long dg = -da;
    double row[m];
#pragma unroll
    for (uint32_t b = 0; b < P; ++b) {
        long long e0, e1, dpart;
        pr.wp(b, e0, e1, dpart);   // b == a reads in-bounds cells; its values are replaced below
        if (b != pr.a) dg -= dpart;
        if ((int)(2 * b) < m) row[2 * b] = (double)e0 * pair_inv + non_diag;
        if ((int)(2 * b + 1) < m) row[2 * b + 1] = (double)e1 * pair_inv + non_diag;
    }
    {
        const double diag_v = (double)dg * pair_inv + diag;
        const double da_v = (double)da * pair_inv + non_diag;
#pragma unroll
        for (int c = 0; c < m; ++c) {
            if (c == r) row[c] = diag_v;
            else if (c == r - 1 && (r & 1)) row[c] = da_v;
        }
    }
    if (lane < n) dgs[lane] = dg;
    __syncthreads();
    double x;   // this lane's component of the solution
    if constexpr (m == 1) {   // one leaf pair: a 1 x 1 system
        const double den = readlane_f64(row[0], 0);
        x = lane == 0 && den != 0.0 ? der[0] / den : 0.0;
    } else {
        bool good = true;
#pragma unroll
        for (int j = 0; j < m; ++j) {
            const double d = readlane_f64(row[j], j);
            if (d <= 0.0) {
                good = false;
                break;
            }
            const double ljj = sqrt(d);
            row[j] = lane == j ? ljj : row[j] / ljj;
#pragma unroll
            for (int k = j + 1; k < m; ++k) row[k] = row[k] - row[j] * readlane_f64(row[j], k);
        }
        double y = lane < m ? der[lane] : 0.0;
        if (good) {
#pragma unroll
            for (int p = 0; p < m; ++p) {   // forward: y[i] -= L[i][p] y[p], p ascending
                const double yp = readlane_f64(y, p) / readlane_f64(row[p], p);
                y = lane == p ? yp : (lane > p ? y - row[p] * yp : y);
            }
            if (lane < m) {
#pragma unroll
                for (int c = 0; c < m; ++c)
                    if (c <= lane) M[tri(lane, c)] = row[c];
            }
            __syncthreads();
#pragma unroll
            for (int p = m - 1; p >= 0; --p) {   // back: L^T x = y
                const double xp = readlane_f64(y, p) / readlane_f64(row[p], p);
                const double lpi = lane < p ? M[tri(p, lane)] : 0.0;
                y = lane == p ? xp : (lane < p ? y - lpi * xp : y);
            }
        }
        x = good && lane < m ? y : 0.0;
    }
    if (lane < n) res[lane] = x;
    __syncthreads();
    zero_average_block(res, n);
    // the statistics replace L again for the score's pass over the rows of W
    stage_pair_cells(Rs, R, PP, B);
    __syncthreads();
    // score (calculate_score, pairwise_scoring.rs:352-375): inner and outer sums sequential
    if (lane < n) {
        const PairRow ps{Rs, T, 2, 2 * B, P, (uint32_t)lane >> 1, (uint32_t)lane & 1u};
        const long long dgx = dgs[lane], dax = ps.da();
        double inner = 0.0;
        for (uint32_t b0 = 0; b0 < P; b0 += kPairBatch) {
            long long e0[kPairBatch], e1[kPairBatch];
#pragma unroll
            for (uint32_t q = 0; q < kPairBatch; ++q) {
                const uint32_t b = b0 + q;
                if (b >= P) continue;
                if (b == ps.a) {
                    e0[q] = ps.u == 0 ? dgx : dax;
                    e1[q] = ps.u == 0 ? dax : dgx;
                } else {
                    long long dpart;
                    ps.wp(b, e0[q], e1[q], dpart);
                }
            }
#pragma unroll
            for (uint32_t q = 0; q < kPairBatch; ++q) {
                const uint32_t b = b0 + q;
                if (b >= P) continue;
                inner += res[2 * b] * ((double)e0[q] * pair_inv);
                inner += res[2 * b + 1] * ((double)e1[q] * pair_inv);
            }
        }
        part[lane] = res[lane] * (der[lane] - 0.5 * inner);
    }
    __syncthreads();
    if (lane == 0) {
        double outer = 0.0;
        for (int i = 0; i < n; ++i) outer += part[i];
        scores[(size_t)f * B + s] = outer;
    }
}

// Best border of each feature: maximum score, lowest border on ties (strict first-wins over
// border ascending, select_level_pairwise tree.rs:3852-3900).
static __global__ __launch_bounds__(256) void pairwise_best_kernel(const double* __restrict__ scores,
                                                                   const uint32_t* __restrict__ n_cand,
                                                                   uint32_t B, double* __restrict__ best_score,
                                                                   uint32_t* __restrict__ best_bin) {
    __shared__ double rs[4];
    __shared__ uint32_t rb[4];
    const uint32_t f = blockIdx.x;
    double s = -INFINITY;
    uint32_t bb = 0xFFFFFFFFu;
    for (uint32_t b = threadIdx.x; b < n_cand[f]; b += blockDim.x) {
        const double v = scores[(size_t)f * B + b];
        if (v > s || (v == s && b < bb)) {
            s = v;
            bb = b;
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const double os = __shfl_xor(s, o, 64);
        const uint32_t ob = __shfl_xor(bb, o, 64);
        if (os > s || (os == s && ob < bb)) {
            s = os;
            bb = ob;
        }
    }
    if (lane_id() == 0) {
        rs[threadIdx.x >> 6] = s;
        rb[threadIdx.x >> 6] = bb;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 4; ++k)
            if (rs[k] > s || (rs[k] == s && rb[k] < bb)) {
                s = rs[k];
                bb = rb[k];
            }
        best_score[f] = s;
        best_bin[f] = bb == 0xFFFFFFFFu ? 0u : bb;
    }
}

// Pairwise weight sums of the final leaves (compute_pairwise_weight_sums,
// pairwise_leaves.rs:47-88): out [L][L] int64, same-leaf pairs skipped.  The L x L sums are
// privatized in LDS up to 128 leaves (in_lds), else added to out directly.
static __global__ __launch_bounds__(256) void pair_leaf_weights_kernel(
    const uint32_t* __restrict__ comp_win, const uint32_t* __restrict__ comp_los,
    const long long* __restrict__ comp_wq, uint64_t m, const uint16_t* __restrict__ leaf, uint32_t L,
    long long* __restrict__ out, int in_lds) {
    extern __shared__ long long sh_lw[];
    if (in_lds)
        for (uint32_t i = threadIdx.x; i < L * L; i += blockDim.x) sh_lw[i] = 0;
    __syncthreads();
    unsigned long long* acc = in_lds ? (unsigned long long*)sh_lw : (unsigned long long*)out;
    for (uint64_t k = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; k < m;
         k += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t wl = leaf[comp_win[k]] & 0x7FFFu, ll = leaf[comp_los[k]] & 0x7FFFu;
        if (wl == ll) continue;
        const long long q = comp_wq[k];
        atomicAdd(acc + (size_t)wl * L + ll, (unsigned long long)(-q));
        atomicAdd(acc + (size_t)ll * L + wl, (unsigned long long)(-q));
        atomicAdd(acc + (size_t)wl * L + wl, (unsigned long long)q);
        atomicAdd(acc + (size_t)ll * L + ll, (unsigned long long)q);
    }
    __syncthreads();
    if (in_lds)
        for (uint32_t i = threadIdx.x; i < L * L; i += blockDim.x)
            if (sh_lw[i] != 0) atomicAdd((unsigned long long*)out + i, (unsigned long long)sh_lw[i]);
}

// normalize_leaf_values for pairwise-weight losses (boosting.rs:2844-2882): subtract the
// document-weighted mean leaf value (leaves with |weight| <= 1e-9 become 0), then scale by
// the learning rate.  counts are the per-leaf document weights (integers).  Lane 0 only.
__device__ inline void pairwise_center_lane0(double* raw, const long long* sums, uint32_t CL, uint32_t L,
                                             double lr, double* scaled) {
    double total = 0.0;
    for (uint32_t l = 0; l < L; ++l) total += (double)sums[(size_t)l * CL + 2];
    if (fabs(total) > 1e-9) {
        double weighted = 0.0;
        for (uint32_t l = 0; l < L; ++l) weighted += raw[l] * (double)sums[(size_t)l * CL + 2];
        const double avg = weighted / total;
        for (uint32_t l = 0; l < L; ++l) {
            if (fabs((double)sums[(size_t)l * CL + 2]) > 1e-9) raw[l] -= avg;
            else raw[l] = 0.0;
        }
    }
    for (uint32_t l = 0; l < L; ++l) scaled[l] = raw[l] * lr;
}

// PairLogit leaves: centring of the Newton / Gradient values of leaf_values_kernel.
static __global__ void pairwise_center_kernel(double* __restrict__ raw, const long long* __restrict__ sums,
                                              uint32_t CL, uint32_t L, double lr, double* __restrict__ scaled) {
    if (threadIdx.x == 0 && blockIdx.x == 0) pairwise_center_lane0(raw, sums, CL, L, lr, scaled);
}

// PairLogitPairwise leaves (compute_pairwise_leaf_deltas, pairwise_leaves.rs:219-238): one
// workgroup solves the L-leaf system from the pair weight sums and the per-leaf der sums,
// then the centring.  Its pair_leaf_solve_doubles(L) doubles are in LDS (ws null) or at ws.
static __global__ __launch_bounds__(256) void pairwise_leaf_kernel(
    const long long* __restrict__ lw, uint32_t L, const long long* __restrict__ sums, uint32_t CL,
    const Scales* __restrict__ sc, double pair_inv, double l2, double prior, double lr,
    double* __restrict__ raw, double* __restrict__ scaled, double* __restrict__ ws) {
    extern __shared__ double sh_pl[];
    double* W = ws ? ws : sh_pl;
    double* M = W + (size_t)L * (L + 1) / 2;
    double* der = M + (size_t)(L - 1) * L / 2;
    double* cj = der + L;
    double* yv = cj + L;
    double* fwd = yv + L;
    double* res = fwd + L;
    const double inv_d = sc->inv[kLeafDer];
    for (uint32_t r = threadIdx.x; r < L; r += blockDim.x) {
        for (uint32_t c = 0; c <= r; ++c) W[tri(r, c)] = (double)lw[(size_t)r * L + c] * pair_inv;
        der[r] = (double)sums[(size_t)r * CL] * inv_d;
    }
    __syncthreads();
    pairwise_solve_block(W, der, (int)L, l2, prior, M, cj, yv, fwd, res);
    for (uint32_t l = threadIdx.x; l < L; l += blockDim.x) raw[l] = res[l];
    __syncthreads();
    if (threadIdx.x == 0) pairwise_center_lane0(raw, sums, CL, L, lr, scaled);
}

// Doubles of one candidate solve of the workgroup kernel at a level of P leaves (n = 2P
// unknowns, m = n - 1): M m (m + 1) / 2 | der, y, fwd, res, cj, part n each | dgs n (int64).
__host__ __device__ constexpr size_t pair_cand_block_doubles(uint32_t P) {
    return (size_t)(2 * P - 1) * (2 * P) / 2 + 7 * (size_t)(2 * P);
}

static_assert(pair_cand_block_doubles(64) * sizeof(double) <= kPairLdsMax, "64-leaf candidates solve in LDS");
static_assert(pair_cand_block_doubles(128) * sizeof(double) > kPairLdsMax, "128-leaf candidates solve in memory");

// Candidate solves of levels with more than 32 leaves (2P = 128 or 256 unknowns): one
// workgroup per (border s, feature f) at a time, looping over the F (B - 1) candidates with
// a stride of the grid.  The same arithmetic as pairwise_candidate_kernel (calculate_pairwise_score,
// pairwise_scoring.rs:471-581): rows of M = W + prior terms assembled from the cumulative
// statistics (threads over rows), the right-looking Cholesky and substitutions of
// pairwise_factor_solve_block, MakeZeroAverage, then the score with sequential inner and outer
// sums.  The workspace of a candidate is in LDS (ws null) or at ws + blockIdx.x * doubles.
static __global__ __launch_bounds__(256) void pairwise_candidate_block_kernel(
    const long long* __restrict__ st, const long long* __restrict__ hist, uint32_t C, uint32_t F,
    const uint32_t* __restrict__ n_cand, uint32_t B, uint32_t P, const Scales* __restrict__ sc, double pair_inv,
    double l2, double prior, double* __restrict__ scores /* [F][B] */, double* __restrict__ ws) {
    extern __shared__ double sh_pb[];
    const int n = 2 * (int)P, m = n - 1;
    double* M = ws ? ws + (size_t)blockIdx.x * pair_cand_block_doubles(P) : sh_pb;
    double* der = M + (size_t)m * (m + 1) / 2;
    double* y = der + n;
    double* fwd = y + n;
    double* res = fwd + n;
    double* cj = res + n;
    double* part = cj + n;
    long long* dgs = (long long*)(part + n);
    const int t = threadIdx.x, nt = blockDim.x;
    const double inv_d = sc->inv[kScoreDer];
    const double cell_prior = 1.0 / (double)n;
    const double non_diag = -prior * cell_prior;
    const double diag = prior * (1.0 - cell_prior) + l2;
    const uint64_t per_f = B - 1, total = (uint64_t)F * per_f;
    for (uint64_t cand = blockIdx.x; cand < total; cand += gridDim.x) {
        const uint32_t f = (uint32_t)(cand / per_f), s = (uint32_t)(cand % per_f);
        if (s >= n_cand[f]) {   // uniform over the workgroup
            if (t == 0) scores[(size_t)f * B + s] = -INFINITY;
            continue;
        }
        const long long* R = st + (size_t)f * P * P * B * 2 + (size_t)s * 2;   // cell stride 2B
        const long long* T = st + (size_t)f * P * P * B * 2 + (size_t)(B - 1) * 2;
        for (uint32_t yl = t; yl < P; yl += nt) {
            const long long* h = hist + ((size_t)yl * C * F + f) * B;
            const long long dp = h[s], dt = h[B - 1];
            der[2 * yl] = (double)dp * inv_d;
            der[2 * yl + 1] = (double)(dt - dp) * inv_d;
        }
        // rows of M (r < m) and the diagonal entries of W (every row, kept for the score)
        for (int r = t; r < n; r += nt) {
            const PairRow pr{R, T, 2 * B, 2 * B, P, (uint32_t)r >> 1, (uint32_t)r & 1u};
            const long long da = pr.da();
            long long dg = -da;
            double* mr = M + (size_t)r * (r + 1) / 2;
            for (uint32_t b = 0; b < P; ++b) {
                if (b == pr.a) continue;
                long long e0, e1, dpart;
                pr.wp(b, e0, e1, dpart);
                dg -= dpart;
                if (r < m && (int)(2 * b) <= r) mr[2 * b] = (double)e0 * pair_inv + non_diag;
                if (r < m && (int)(2 * b + 1) <= r) mr[2 * b + 1] = (double)e1 * pair_inv + non_diag;
            }
            dgs[r] = dg;
            if (r < m) {
                mr[r] = (double)dg * pair_inv + diag;
                if (r & 1) mr[r - 1] = (double)da * pair_inv + non_diag;
            }
        }
        __syncthreads();
        for (int r = t; r < m; r += nt) y[r] = der[r];   // der is complete after the barrier
        __syncthreads();
        pairwise_factor_solve_block(M, m, cj, y, fwd, res);
        zero_average_block(res, n);
        // score (calculate_score, pairwise_scoring.rs:352-375): inner and outer sums sequential
        for (int r = t; r < n; r += nt) {
            const PairRow ps{R, T, 2 * B, 2 * B, P, (uint32_t)r >> 1, (uint32_t)r & 1u};
            const long long dgx = dgs[r], dax = ps.da();
            double inner = 0.0;
            for (uint32_t b = 0; b < P; ++b) {
                long long e0, e1;
                if (b == ps.a) {
                    e0 = ps.u == 0 ? dgx : dax;
                    e1 = ps.u == 0 ? dax : dgx;
                } else {
                    long long dpart;
                    ps.wp(b, e0, e1, dpart);
                }
                inner += res[2 * b] * ((double)e0 * pair_inv);
                inner += res[2 * b + 1] * ((double)e1 * pair_inv);
            }
            part[r] = res[r] * (der[r] - 0.5 * inner);
        }
        __syncthreads();
        if (t == 0) {
            double outer = 0.0;
            for (int i = 0; i < n; ++i) outer += part[i];
            scores[(size_t)f * B + s] = outer;
        }
        __syncthreads();   // the workspace is rewritten by the next candidate
    }
}

}  // namespace cbh
