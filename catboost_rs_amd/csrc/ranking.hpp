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

__device__ __forceinline__ uint32_t tri(uint32_t r, uint32_t c) {   // packed lower triangle
    return r >= c ? r * (r + 1) / 2 + c : c * (c + 1) / 2 + r;
}

// pairlogit_pair_prob (crates/cb-compute/src/loss.rs:640-651).
__device__ __forceinline__ double pairlogit_p(double winner_approx, double loser_approx) {
    const double el = exp(loser_approx), ew = exp(winner_approx);
    const double den = el + ew;
    return den > 0.0 ? el / den : 0.5;
}

// The previous tree's leaf values (lr-scaled) applied to every row (pair losses: their
// derivatives need every row's updated approximant, so this runs before them).
static __global__ __launch_bounds__(256) void apply_leaves_kernel(double* __restrict__ approx,
                                                                  const uint16_t* __restrict__ leaf,
                                                                  const double* __restrict__ pending, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        approx[i] += pending[leaf[i] & 0x7FFFu];
}

// PairLogit derivatives, one thread per row (pairlogit_group_der,
// crates/cb-compute/src/ranking_der.rs:408-445).  The reference walks a query group's rows
// ascending, each winner's pairs in order: a loser's derivatives are decremented as its
// winners are visited, and a winner adds its own sums after its pair loop.  Row i receives
// exactly those operations in that order: its decrements as a loser from the winners before
// it (its pairs as a loser, los_idx, ascend in competitor order, i.e. by winner), then its own
// pair loop (a pair with itself as loser decremented inside it, as there), then its sums, then
// the decrements from the winners after it -- the same sequential f64 values, with no atomics.
static __global__ __launch_bounds__(256) void pairlogit_row_ders_kernel(
    uint64_t n, const uint32_t* __restrict__ comp_off, const uint32_t* __restrict__ comp_win,
    const uint32_t* __restrict__ comp_los, const double* __restrict__ comp_w, const uint32_t* __restrict__ los_off,
    const uint32_t* __restrict__ los_idx, const double* __restrict__ approx, double* __restrict__ der1,
    double* __restrict__ der2) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const double ai = approx[i];
    const uint32_t own0 = comp_off[i], own1 = comp_off[i + 1];
    const uint32_t l0 = los_off[i], l1 = los_off[i + 1];
    double d1 = 0.0, d2 = 0.0;
    uint32_t q = l0;
    for (; q < l1 && los_idx[q] < own0; ++q) {   // winners before row i
        const uint32_t k = los_idx[q];
        const double p = pairlogit_p(approx[comp_win[k]], ai), w = comp_w[k];
        d1 -= w * p;
        d2 += w * p * (p - 1.0);
    }
    double wd = 0.0, wd2 = 0.0;
    for (uint32_t k = own0; k < own1; ++k) {   // row i's own pairs
        const uint32_t l = comp_los[k];
        const double p = pairlogit_p(ai, approx[l]), w = comp_w[k];
        wd += w * p;
        wd2 += w * p * (p - 1.0);
        if (l == i) {
            d1 -= w * p;
            d2 += w * p * (p - 1.0);
        }
    }
    d1 += wd;
    d2 += wd2;
    for (; q < l1; ++q) {   // winners after row i (its own pairs with itself were taken above)
        const uint32_t k = los_idx[q];
        if (k < own1) continue;
        const double p = pairlogit_p(approx[comp_win[k]], ai), w = comp_w[k];
        d1 -= w * p;
        d2 += w * p * (p - 1.0);
    }
    der1[i] = d1;
    der2[i] = d2;
}

// ---- pairs grouped by their unordered leaf pair {a <= b} (levels of 2 leaves and more)

__device__ __forceinline__ uint32_t pair_key(uint32_t wl, uint32_t ll, uint32_t P) {
    return wl < ll ? wl * P + ll : ll * P + wl;
}

// Count the pairs of every key (P*P keys, those with a > b stay 0).  Each thread takes
// kCountItems pairs (their loads and leaf lookups all in flight at once) and each workgroup
// adds its nonzero counts once: few workgroups, so few global atomics per key.
constexpr uint32_t kCountItems = 16;
static __global__ __launch_bounds__(256) void pair_key_count_kernel(
    const uint32_t* __restrict__ comp_win, const uint32_t* __restrict__ comp_los, uint64_t m,
    const uint16_t* __restrict__ leaf, uint32_t P, uint32_t* __restrict__ cnt) {
    extern __shared__ uint32_t c[];   // [P * P]
    for (uint32_t i = threadIdx.x; i < P * P; i += blockDim.x) c[i] = 0;
    __syncthreads();
    const uint64_t base = (uint64_t)blockIdx.x * blockDim.x * kCountItems + threadIdx.x;
    uint32_t wi[kCountItems], lo[kCountItems];
#pragma unroll
    for (uint32_t r = 0; r < kCountItems; ++r) {
        const uint64_t k = base + (uint64_t)r * blockDim.x;
        wi[r] = k < m ? comp_win[k] : 0u;
        lo[r] = k < m ? comp_los[k] : 0u;   // k past m: winner == loser, not counted
    }
    uint32_t wl[kCountItems], ll[kCountItems];
#pragma unroll
    for (uint32_t r = 0; r < kCountItems; ++r) {
        wl[r] = leaf[wi[r]] & 0x7FFFu;
        ll[r] = leaf[lo[r]] & 0x7FFFu;
    }
#pragma unroll
    for (uint32_t r = 0; r < kCountItems; ++r)
        if (wi[r] != lo[r]) atomicAdd(&c[pair_key(wl[r], ll[r], P)], 1u);
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < P * P; i += blockDim.x)
        if (c[i]) atomicAdd(cnt + i, c[i]);
}

// Scatter the pairs by key as compact records (order inside a key is free: the sums are
// exact integers): rec = (winner, loser | winner-in-leaf-a << 31), weight in fixed point.
// Each workgroup takes kScatterItems pairs per thread, ranks them per key in LDS, reserves one
// range per key with a single global atomic, then writes.
constexpr uint32_t kScatterItems = 8;
// Zero the statistics runs of multi-chunk key mk[i] of feature f (pair_multi_zero_kernel's work).
__device__ __forceinline__ void pair_multi_zero_runs(const uint32_t* __restrict__ mk, uint32_t i, uint32_t f,
                                                     uint32_t P, uint32_t B, long long* __restrict__ st) {
    const uint32_t k = mk[i], a = k / P, b = k % P;
    long long* r0 = st + (((size_t)f * P + a) * P + b) * B * 2;
    long long* r1 = st + (((size_t)f * P + b) * P + a) * B * 2;
    for (uint32_t j = threadIdx.x; j < 2 * B; j += blockDim.x) {
        r0[j] = 0;
        r1[j] = 0;
    }
}

// Workgroups past n_sc zero the runs of the multi-chunk keys (one per (key, feature), F per
// key): the zeroing rides in the scatter's launch.
static __global__ __launch_bounds__(256) void pair_key_scatter_kernel(
    const uint32_t* __restrict__ comp_win, const uint32_t* __restrict__ comp_los,
    const long long* __restrict__ comp_wq, uint64_t m, const uint16_t* __restrict__ leaf, uint32_t P,
    uint32_t* __restrict__ cursor, uint2* __restrict__ rec, long long* __restrict__ rec_wq, uint32_t n_sc,
    const uint32_t* __restrict__ mk, const uint32_t* __restrict__ n_multi, uint32_t F, uint32_t B,
    long long* __restrict__ st) {
    if (blockIdx.x >= n_sc) {   // uniform over the workgroup, before any barrier
        const uint32_t z = blockIdx.x - n_sc, i = z / F;
        if (i < *n_multi) pair_multi_zero_runs(mk, i, z % F, P, B, st);
        return;
    }
    extern __shared__ uint32_t lcnt[];   // [P * P]
    const uint32_t nk = P * P;
    for (uint32_t i = threadIdx.x; i < nk; i += blockDim.x) lcnt[i] = 0;
    __syncthreads();
    const uint64_t base = (uint64_t)blockIdx.x * blockDim.x * kScatterItems + threadIdx.x;
    // every item's loads and leaf lookups in flight at once; the records are kept for the write
    uint32_t wi[kScatterItems], lo[kScatterItems], key[kScatterItems], slot[kScatterItems];
#pragma unroll
    for (uint32_t r = 0; r < kScatterItems; ++r) {
        const uint64_t k = base + (uint64_t)r * blockDim.x;
        wi[r] = k < m ? comp_win[k] : 0u;
        lo[r] = k < m ? comp_los[k] : 0u;   // k past m: winner == loser, skipped
    }
#pragma unroll
    for (uint32_t r = 0; r < kScatterItems; ++r) {
        const uint32_t wl = leaf[wi[r]] & 0x7FFFu, ll = leaf[lo[r]] & 0x7FFFu;
        key[r] = wi[r] != lo[r] ? pair_key(wl, ll, P) : 0xFFFFFFFFu;
        lo[r] |= (wl <= ll ? 1u : 0u) << 31;
    }
#pragma unroll
    for (uint32_t r = 0; r < kScatterItems; ++r)
        if (key[r] != 0xFFFFFFFFu) slot[r] = atomicAdd(&lcnt[key[r]], 1u);
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < nk; i += blockDim.x)
        if (lcnt[i]) lcnt[i] = atomicAdd(cursor + i, lcnt[i]);   // count -> reserved base
    __syncthreads();
#pragma unroll
    for (uint32_t r = 0; r < kScatterItems; ++r) {
        if (key[r] == 0xFFFFFFFFu) continue;
        const uint64_t k = base + (uint64_t)r * blockDim.x;
        const uint32_t pos = lcnt[key[r]] + slot[r];
        rec[pos] = make_uint2(wi[r], lo[r]);
        rec_wq[pos] = comp_wq[k];
    }
}

// ---- statistics with feature lanes: one workgroup per (leaf-pair key, chunk of its pairs,
// tile of 16 features).  16 lanes take the 16 features of one pair, so the two atomics of a
// (pair, feature) land in LDS cells laid out [bucket][channel][block][16 features]: the 16 lanes
// of a pair always hit 16 distinct bank pairs (the block and feature give the bank; the bucket
// only the row).  A key whose pairs fit one chunk writes its cumulative runs straight into the
// statistics; the chunks of a larger key add their cells into a zeroed region that
// pair_multi_scan_kernel then turns into prefix form.

constexpr uint32_t kStatTileF = 16;       // features per tile (lanes of one pair)
constexpr uint32_t kStatThreads = 1024;   // 64 pairs per pass of a workgroup
constexpr uint32_t kStatChunkMin = 4096;  // pairs per chunk: at least, the session picks per level

// Chunk plan of one level (one workgroup of 1024 threads, each over a run of consecutive keys):
// key_off / cursor = exclusive scan of the pair counts of the P*P keys (pair_key_scatter), and
// per key {a <= b}: max(1, ceil(count / chunk)) chunk descriptors {key, first pair, pairs,
// multi}; keys of several chunks are also listed in mk.  direct: one key (a single leaf) over
// the m pairs in input order.  Once read, the counts [0, n_zero) are cleared for the next
// level's pair_key_count_kernel (cnt_next: the same buffer).
static __global__ __launch_bounds__(1024) void pair_plan_kernel(
    const uint32_t* cnt, uint32_t P, int direct, uint32_t m, uint32_t chunk, uint32_t* __restrict__ key_off,
    uint32_t* __restrict__ cursor, uint4* __restrict__ desc, uint32_t* __restrict__ n_desc,
    uint32_t* __restrict__ mk, uint32_t* __restrict__ n_multi, uint32_t* cnt_next, uint32_t n_zero) {
    __shared__ uint32_t sc[32], sn[32], sm[32];   // wave totals [0, 16), then their exclusive prefixes
    const uint32_t t = threadIdx.x;
    const uint32_t nk = direct ? 1u : P * P;
    const uint32_t per = (nk + 1023) / 1024;
    const uint32_t k0 = min(t * per, nk), k1 = min(k0 + per, nk);
    auto count_of = [&](uint32_t k) -> uint32_t { return direct ? m : cnt[k]; };
    auto chunks_of = [&](uint32_t k, uint32_t c) -> uint32_t {
        if (!direct && k / P > k % P) return 0u;   // keys are {min, max}
        return c == 0 ? 1u : (c + chunk - 1) / chunk;
    };
    uint32_t vc = 0, vn = 0, vm = 0;
    for (uint32_t k = k0; k < k1; ++k) {
        const uint32_t c = count_of(k), nc = chunks_of(k, c);
        vc += c;
        vn += nc;
        vm += nc > 1 ? 1u : 0u;
    }
    // exclusive prefixes of the three sums over the threads: within each wave by shuffles, then
    // over the 16 wave totals by wave 0 (two barriers)
    const uint32_t lane = t & 63u, wave = t >> 6;
    uint32_t ic = vc, in_ = vn, im = vm;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t uc = __shfl_up(ic, o, 64), un = __shfl_up(in_, o, 64), um = __shfl_up(im, o, 64);
        if (lane >= (uint32_t)o) {
            ic += uc;
            in_ += un;
            im += um;
        }
    }
    if (lane == 63) {
        sc[wave] = ic;
        sn[wave] = in_;
        sm[wave] = im;
    }
    __syncthreads();
    if (wave == 0) {
        const uint32_t tc = lane < 16 ? sc[lane] : 0u, tn = lane < 16 ? sn[lane] : 0u, tm = lane < 16 ? sm[lane] : 0u;
        uint32_t wc = tc, wn = tn, wm = tm;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
            const uint32_t uc = __shfl_up(wc, o, 64), un = __shfl_up(wn, o, 64), um = __shfl_up(wm, o, 64);
            if (lane >= (uint32_t)o) {
                wc += uc;
                wn += un;
                wm += um;
            }
        }
        if (lane < 16) {
            sc[16 + lane] = wc - tc;
            sn[16 + lane] = wn - tn;
            sm[16 + lane] = wm - tm;
        }
        if (lane == 15) {   // the grand totals
            if (!direct) key_off[nk] = wc;
            *n_desc = wn;
            *n_multi = wm;
        }
    }
    __syncthreads();
    uint32_t oc = sc[16 + wave] + ic - vc, on = sn[16 + wave] + in_ - vn, om = sm[16 + wave] + im - vm;
    for (uint32_t k = k0; k < k1; ++k) {
        const uint32_t c = count_of(k), nc = chunks_of(k, c);
        if (!direct) {
            key_off[k] = oc;
            cursor[k] = oc;
        }
        for (uint32_t j = 0; j < nc; ++j)
            desc[on + j] = make_uint4(k, oc + j * chunk, min(chunk, c - j * chunk), nc > 1 ? 1u : 0u);
        if (nc > 1) mk[om++] = k;
        oc += c;
        on += nc;
    }
    __syncthreads();   // every count read
    for (uint32_t i = t; i < n_zero; i += 1024) cnt_next[i] = 0;
}

// Zero the statistics runs of the keys of several chunks (grid: (max multi keys, F)).
static __global__ __launch_bounds__(256) void pair_multi_zero_kernel(const uint32_t* __restrict__ mk,
                                                                     const uint32_t* __restrict__ n_multi, uint32_t P,
                                                                     uint32_t B, long long* __restrict__ st) {
    if (blockIdx.x >= *n_multi) return;
    pair_multi_zero_runs(mk, blockIdx.x, blockIdx.y, P, B, st);
}

// Inclusive prefix over buckets of the runs of the keys of several chunks: one wavefront per
// (block, channel) run of a (key, feature); lane l takes buckets [l k, l k + k), k = ceil(B / 64).
static __global__ __launch_bounds__(256) void pair_multi_scan_kernel(const uint32_t* __restrict__ mk,
                                                                     const uint32_t* __restrict__ n_multi, uint32_t P,
                                                                     uint32_t B, long long* __restrict__ st) {
    if (blockIdx.x >= *n_multi) return;
    const uint32_t k = mk[blockIdx.x], a = k / P, b = k % P, f = blockIdx.y;
    const uint32_t w = threadIdx.x >> 6, lane = threadIdx.x & 63;   // w = block * 2 + channel
    const uint32_t blk = w >> 1, c = w & 1u;
    if (blk == 1 && a == b) return;
    const uint32_t x = blk == 0 ? a : b, y = blk == 0 ? b : a;
    long long* p = st + (((size_t)f * P + x) * P + y) * B * 2 + c;
    const uint32_t kk = (B + 63) / 64;
    const uint32_t b0 = min(lane * kk, B), b1 = min(b0 + kk, B);
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
        const long long tt = __shfl_up(incl, o, 64);
        if ((int)lane >= o) incl += tt;
    }
    const long long off = incl - tot;
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i)
        if (b0 + i < b1) p[(size_t)(b0 + i) * 2] = v[i] + off;
}

// Words of one (block, feature) row of the pair statistics' flush in LDS: 2B (bucket, channel)
// padded to 2 mod 32, so that the 64 runs' writes of one bucket spread over the banks.
__host__ __device__ constexpr uint32_t pair_stat_row_words(uint32_t B) { return 2 * B + (34u - (2 * B) % 32u) % 32u; }
// LDS of pair_stats_feature_kernel: the cells [B][channel][block][16], then the flush rows.
__host__ __device__ constexpr size_t pair_stat_lds(uint32_t B) {
    return (B * 64 > 32 * pair_stat_row_words(B) ? B * 64 : 32 * pair_stat_row_words(B)) * sizeof(unsigned long long);
}

// Accumulate one chunk of one key's pairs for one tile of 16 features.  Grid: 8 * tiles *
// ceil(max descriptors / 8) workgroups; workgroup g runs descriptor 8 (q / tiles) + g mod 8 and
// tile q mod tiles (q = g / 8), so the tiles of a descriptor share an XCD (workgroups go to the 8
// XCDs round-robin) and start together: the pairs' rows they all gather come from HBM into that
// XCD's L2 once rather than once per tile.  Records come grouped by key (rec: winner, loser |
// winner-in-leaf-a << 31), or, at a level of one leaf, straight from the pair arrays (direct).  For a pair with winner
// bucket > loser bucket the cells [loserLeaf][winnerLeaf] receive -w at (loser bucket, smaller)
// and (winner bucket, greater), otherwise [winnerLeaf][loserLeaf] at (winner bucket, smaller)
// and (loser bucket, greater) (compute_pair_weight_statistics, pairwise_scoring.rs:163-196);
// block 0 of a key {a <= b} is [a][b], block 1 is [b][a].
template <bool kBuf>   // row words by 32-bit buffer offsets (row buffer under 4 GiB, rows < 2^24)
static __global__ __launch_bounds__(kStatThreads) void pair_stats_feature_kernel(
    const uint32_t* __restrict__ rows, uint32_t Ws, const uint4* __restrict__ desc, const uint32_t* __restrict__ n_desc,
    const uint2* __restrict__ rec, const long long* __restrict__ rec_wq, const uint32_t* __restrict__ comp_win,
    const uint32_t* __restrict__ comp_los, const long long* __restrict__ comp_wq, int direct, uint32_t F, uint32_t P,
    uint32_t B, long long* __restrict__ st, uint32_t tiles) {
    extern __shared__ unsigned long long cells[];   // [B][channel][block][16]
    const uint32_t qg = blockIdx.x >> 3, tile = qg % tiles, di = (qg / tiles) * 8u + (blockIdx.x & 7u);
    if (di >= *n_desc) return;   // workgroup-uniform, before any barrier
    const uint4 ds = desc[di];
    const uint32_t key = ds.x, a = key / P, b = key % P;
    const uint32_t t = threadIdx.x, fl = t & 15;
    const uint32_t f = tile * kStatTileF + fl;
    const bool fok = f < F;
    // a lane past the last feature reads feature F - 1's bins (< B) into its own cells, which
    // are never flushed
    const uint32_t word = (fok ? f : F - 1) >> 2, sh = ((fok ? f : F - 1) & 3u) * 8u;
    for (uint32_t i = t; i < B * 64; i += kStatThreads) cells[i] = 0;
    __syncthreads();
    // each 16-lane row takes 16 consecutive pairs per pass: lane fl loads the record of pair
    // fl (one coalesced load for the row, the next pass's prefetched), the records reach the
    // row's lanes by row_newbcast, and the 32 row words of the 16 pairs are loaded together
    const uint32_t first = ds.y, cnt = ds.z;
    constexpr uint32_t kRows = kStatThreads / 16, kPass = kRows * 16;
    // A pair past the chunk or with winner == loser adds nothing: its weight is zeroed here and
    // its two atomics add 0 (no per-pair branch).  The weight is kept negated.
    auto load_rec = [&](uint32_t j, uint32_t& wi, uint32_t& lo, uint32_t& wa, long long& wq) {
        const bool ok = j < cnt;
        const size_t k = (size_t)first + (ok ? j : 0u);
        long long q;
        if (direct) {
            wi = comp_win[k];
            lo = comp_los[k];
            wa = 0;
            q = comp_wq[k];
        } else {
            const uint2 r = rec[k];
            wi = r.x;
            lo = r.y & 0x7FFFFFFFu;
            wa = r.y >> 31;
            q = rec_wq[k];
        }
        wq = ok && wi != lo ? -q : 0;
    };
    const uint32_t row = t >> 4;
    // cell (bucket, channel, block, lane) at byte 512 bucket + 256 channel + 128 block + 8 lane
    char* const cl0 = (char*)cells + fl * 8u;                    // block 0 of lane fl
    char* const cl1 = cl0 + (a == b ? 0u : 128u);               // block 1 (a == b: block 0)
    const uint32_t Ws4 = Ws * 4u, word4 = word * 4u;
    uint32_t n_wi, n_lo, n_wa;
    long long n_wq;
    load_rec(row * 16 + fl, n_wi, n_lo, n_wa, n_wq);
    for (uint32_t base = row * 16; base < cnt; base += kPass) {
        const uint32_t c_wi = n_wi, c_lo = n_lo, c_wa = n_wa;
        const long long c_wq = n_wq;
        load_rec(base + kPass + fl, n_wi, n_lo, n_wa, n_wq);   // the next pass's records
        uint32_t ww[16], lw[16];
#define CBH_STAT_GATHER(U)                                                                                   \
    {                                                                                                         \
        const uint32_t wiu = row_bcast<U>(c_wi), lou = row_bcast<U>(c_lo);                                   \
        if constexpr (kBuf) {   /* rows < 2^24 and 4 Ws < 2^24: one 24-bit multiply-add per offset */        \
            const __amdgpu_buffer_rsrc_t rr = make_rsrc(rows, 0xFFFFFFFFull);                                 \
            ww[U] = ldw(rr, __umul24(wiu, Ws4) + word4);                                                      \
            lw[U] = ldw(rr, __umul24(lou, Ws4) + word4);                                                      \
        } else {                                                                                              \
            ww[U] = rows[(size_t)wiu * Ws + word];                                                            \
            lw[U] = rows[(size_t)lou * Ws + word];                                                            \
        }                                                                                                     \
    }
        CBH_STAT_GATHER(0) CBH_STAT_GATHER(1) CBH_STAT_GATHER(2) CBH_STAT_GATHER(3)
        CBH_STAT_GATHER(4) CBH_STAT_GATHER(5) CBH_STAT_GATHER(6) CBH_STAT_GATHER(7)
        CBH_STAT_GATHER(8) CBH_STAT_GATHER(9) CBH_STAT_GATHER(10) CBH_STAT_GATHER(11)
        CBH_STAT_GATHER(12) CBH_STAT_GATHER(13) CBH_STAT_GATHER(14) CBH_STAT_GATHER(15)
#undef CBH_STAT_GATHER
        // block 1 when (winner bucket > loser bucket) == winner-in-leaf-a, block 0 when a == b
#define CBH_STAT_PAIR(U)                                                                                     \
    {                                                                                                         \
        const uint32_t wau = row_bcast<U>(c_wa);                                                              \
        const unsigned long long neg = row_bcast64<U>((unsigned long long)c_wq);                              \
        const uint32_t wb = (ww[U] >> sh) & 0xFFu, lb = (lw[U] >> sh) & 0xFFu;                                \
        char* const cl = (wb > lb) == (wau != 0) ? cl1 : cl0;                                                 \
        const uint32_t bs = wb > lb ? lb : wb, bg = wb > lb ? wb : lb;                                        \
        atomicAdd((unsigned long long*)(cl + (bs << 9)), neg);                                                \
        atomicAdd((unsigned long long*)(cl + (bg << 9) + 256u), neg);                                         \
    }
        CBH_STAT_PAIR(0) CBH_STAT_PAIR(1) CBH_STAT_PAIR(2) CBH_STAT_PAIR(3)
        CBH_STAT_PAIR(4) CBH_STAT_PAIR(5) CBH_STAT_PAIR(6) CBH_STAT_PAIR(7)
        CBH_STAT_PAIR(8) CBH_STAT_PAIR(9) CBH_STAT_PAIR(10) CBH_STAT_PAIR(11)
        CBH_STAT_PAIR(12) CBH_STAT_PAIR(13) CBH_STAT_PAIR(14) CBH_STAT_PAIR(15)
#undef CBH_STAT_PAIR
    }
    __syncthreads();
    // Flush.  The key's only chunk writes its cumulative runs straight into the statistics; one
    // chunk of several adds its raw cells into the zeroed runs (pair_multi_scan_kernel takes the
    // prefix).  Thread t takes run t & 63 (= channel, block, feature: consecutive lanes read
    // consecutive cells) and the 16 buckets of segment t >> 6, the segment totals giving each
    // segment its offset; the values go back to LDS as one row per (block, feature) of 2B
    // words (bucket, channel), which each wavefront then copies out 1 KB at a time.
    const bool single = ds.w == 0;
    __shared__ unsigned long long seg_tot[16][64];
    {
        const uint32_t run = t & 63u, seg = t >> 6, c = run >> 5;
        unsigned long long v[16];
#pragma unroll
        for (uint32_t i = 0; i < 16; ++i) {
            const uint32_t bk = seg * 16 + i;
            v[i] = bk < B ? cells[(size_t)bk * 64 + run] : 0ull;
        }
        if (single) {
#pragma unroll
            for (uint32_t i = 1; i < 16; ++i) v[i] += v[i - 1];
            seg_tot[seg][run] = v[15];
        }
        __syncthreads();   // every cell read before the rows overwrite them
        unsigned long long off = 0;
        if (single)
            for (uint32_t g = 0; g < seg; ++g) off += seg_tot[g][run];
        unsigned long long* trow = cells + (size_t)(run & 31u) * pair_stat_row_words(B);
#pragma unroll
        for (uint32_t i = 0; i < 16; ++i) {
            const uint32_t bk = seg * 16 + i;
            if (bk < B) trow[bk * 2 + c] = v[i] + off;
        }
    }
    __syncthreads();
    {
        const uint32_t w = t >> 6, lane = t & 63u;
        for (uint32_t q = w; q < 32; q += kStatThreads / 64) {   // row q: block q >> 4, feature q & 15
            const uint32_t blk = q >> 4, ff = tile * kStatTileF + (q & 15u);
            if (ff >= F || (blk == 1 && a == b)) continue;   // uniform over the wavefront
            const uint32_t x = blk == 0 ? a : b, y = blk == 0 ? b : a;
            long long* dst = st + (((size_t)ff * P + x) * P + y) * B * 2;
            const unsigned long long* src = cells + (size_t)q * pair_stat_row_words(B);
            for (uint32_t e = lane * 2; e < 2 * B; e += 128) {
                const ulonglong2 v2 = *reinterpret_cast<const ulonglong2*>(src + e);
                if (single) {
                    *reinterpret_cast<longlong2*>(dst + e) = make_longlong2((long long)v2.x, (long long)v2.y);
                } else {
                    if (v2.x) atomicAdd((unsigned long long*)(dst + e), v2.x);
                    if (v2.y) atomicAdd((unsigned long long*)(dst + e + 1), v2.y);
                }
            }
        }
    }
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

// In-place Cholesky of the m x m packed system M (right-looking: every element receives its
// pivot subtractions in ascending order, as the reference's left-looking loop applies them)
// and the forward / back substitutions of y, by the threads of the workgroup (rows strided
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
        // back, right-looking: x[p] = y[p] / L[p][p], then y[i] -= L[p][i] x[p] for i < p.  Row i
        // receives its subtractions p descending where the reference's left-looking loop sums
        // them p ascending (leaf.rs:409-415): the last bits of x may differ, as they do anyway
        // from the fixed-point der sums; the chain of the reference's order would serialize
        // m^2 / 2 steps
        for (int p = m - 1; p >= 0; --p) {
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

// LDS of the candidate solve at P leaves (8-byte words): L (packed lower triangle of the 2P-1
// rows; the border's 2 P^2 statistics once the solve is done) | der, res, part, dgs 64 each.
// 18 KB at 32 leaves (eight waves a CU, as its 243 VGPRs allow), 6 KB at 16 (its 115 VGPRs:
// four waves a SIMD).
__host__ __device__ constexpr uint32_t pair_cand_l_words(uint32_t P) {
    return (2 * P - 1) * 2 * P / 2 > 2 * P * P ? (2 * P - 1) * 2 * P / 2 : 2 * P * P;
}
__host__ __device__ constexpr size_t pair_cand_lds(uint32_t P) {
    return ((size_t)pair_cand_l_words(P) + 4 * 64) * sizeof(double);
}
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

// The weight-matrix entries between the rows of two different leaves lo < hi at one border,
// from the cumulative statistics at that border (R, cell stride rs) and at the last border
// (T, stride ts): one load of the four cells PairRow::wp reads.
struct PairCells {
    long long w00, w01, w10, w11, total;
};
__device__ __forceinline__ PairCells pair_cells(const long long* R, uint32_t rs, const long long* T, uint32_t ts,
                                                uint32_t P, uint32_t lo, uint32_t hi) {
    const long long xs = R[(size_t)(hi * P + lo) * rs], xg = R[(size_t)(hi * P + lo) * rs + 1];
    const long long ys = R[(size_t)(lo * P + hi) * rs], yg = R[(size_t)(lo * P + hi) * rs + 1];
    const long long total = T[(size_t)(hi * P + lo) * ts] + T[(size_t)(lo * P + hi) * ts];
    return {xg + yg, xs - xg, ys - yg, -(xs + ys), total};
}
// Row (a, u) of the system at the columns (2b, 2b + 1) of another leaf b, and that block's part
// of the row's diagonal entry (PairRow::wp with a > b given as a_gt_b).
__device__ __forceinline__ void pair_row_entries(const PairCells& c, bool a_gt_b, uint32_t u, long long& e0,
                                                 long long& e1, long long& dpart) {
    if (u == 0) {
        e0 = c.w00;
        e1 = a_gt_b ? c.w01 : c.w10;
        dpart = a_gt_b ? (c.w00 + c.w01) : (c.w00 + c.w10);
    } else {
        e0 = a_gt_b ? c.w10 : c.w01;
        e1 = c.w11 + c.total;
        dpart = (a_gt_b ? (c.w10 + c.w11) : (c.w01 + c.w11)) + c.total;
    }
}

// Levels of up to 8 leaves (2P <= 16 unknowns): one border per lane, 64 consecutive borders of
// one feature per wavefront, the whole system in the lane's registers (calculate_pairwise_score,
// pairwise_scoring.rs:471-581).  Every IEEE operation is the reference's, in its order:
// the matrix M = W + prior terms, the Cholesky factorization (leaf.rs:363-389, here
// right-looking: every element receives its pivot subtractions in ascending order), the
// forward and back substitutions with their sums taken p ascending (:390-423), a non-positive
// pivot giving zeros, MakeZeroAverage, and the score with sequential inner and outer sums
// (calculate_score :352-375).  A lane's statistics of one cell are 16 bytes at stride 16 bytes
// from its neighbour's: every load is one contiguous 1 KB run per wavefront.
template <uint32_t P_>
static __global__ __launch_bounds__(64) void pairwise_candidate_lane_kernel(
    const long long* __restrict__ st, const long long* __restrict__ hist, uint32_t C, uint32_t F,
    const uint32_t* __restrict__ n_cand, uint32_t B, const Scales* __restrict__ sc, double pair_inv,
    double l2, double prior, double* __restrict__ scores /* [F][B] */) {
    constexpr uint32_t P = P_;
    constexpr int n = 2 * (int)P, m = n - 1;
    constexpr int nL = m * (m + 1) / 2;
    static_assert(P >= 1 && P <= 8, "register-resident systems up to 15 unknowns");
    const uint32_t f = blockIdx.y;
    const uint32_t s = blockIdx.x * 64 + threadIdx.x;
    if (s >= B - 1) return;
    if (s >= n_cand[f]) {
        scores[(size_t)f * B + s] = -INFINITY;
        return;
    }
    const long long* base = st + (size_t)f * P * P * B * 2;
    const long long* R = base + (size_t)s * 2;
    const long long* T = base + (size_t)(B - 1) * 2;
    const uint32_t rs = 2 * B;
    const double inv_d = sc->inv[kScoreDer];
    double der[n];
#pragma unroll
    for (uint32_t yl = 0; yl < P; ++yl) {   // der channel of the level histogram, prefix over bins
        const long long* h = hist + ((size_t)yl * C * F + f) * B;
        const long long dp = h[s], dt = h[B - 1];
        der[2 * yl] = (double)dp * inv_d;
        der[2 * yl + 1] = (double)(dt - dp) * inv_d;
    }
    const double cell_prior = 1.0 / (double)n;
    const double non_diag = -prior * cell_prior;
    const double diag = prior * (1.0 - cell_prior) + l2;
    // ---- M (packed lower triangle, rows < m) and the diagonal entries of W (every row) ----
    double L[nL];
    long long dg[n], da[P];
#pragma unroll
    for (uint32_t a = 0; a < P; ++a) {
        da[a] = R[(size_t)(a * P + a) * rs] - R[(size_t)(a * P + a) * rs + 1];
        dg[2 * a] = -da[a];
        dg[2 * a + 1] = -da[a];
    }
#pragma unroll
    for (uint32_t hi = 1; hi < P; ++hi)
#pragma unroll
        for (uint32_t lo = 0; lo < hi; ++lo) {
            const PairCells c = pair_cells(R, rs, T, rs, P, lo, hi);
#pragma unroll
            for (uint32_t u = 0; u < 2; ++u) {
                long long e0, e1, dp;
                pair_row_entries(c, true, u, e0, e1, dp);   // row of leaf hi, columns of lo (below the diagonal)
                dg[2 * hi + u] -= dp;
                const int r = 2 * (int)hi + (int)u;
                if (r < m) {
                    L[tri(r, 2 * lo)] = (double)e0 * pair_inv + non_diag;
                    L[tri(r, 2 * lo + 1)] = (double)e1 * pair_inv + non_diag;
                }
                pair_row_entries(c, false, u, e0, e1, dp);  // row of leaf lo: above the diagonal
                dg[2 * lo + u] -= dp;
            }
        }
#pragma unroll
    for (int r = 0; r < m; ++r) {
        L[tri(r, r)] = (double)dg[r] * pair_inv + diag;
        if (r & 1) L[tri(r, r - 1)] = (double)da[r >> 1] * pair_inv + non_diag;
    }
    // ---- solve ----
    double x[n];
    x[m] = 0.0;
    if constexpr (m == 1) {   // one leaf: the 1 x 1 system (the reference's n == 2 case)
        const double den = L[0];
        x[0] = den != 0.0 ? der[0] / den : 0.0;
    } else {
        bool good = true;
#pragma unroll
        for (int j = 0; j < m; ++j) {
            const double d = L[tri(j, j)];
            if (d <= 0.0) good = false;   // the reference returns None; the rest is discarded
            const double ljj = sqrt(d);
#pragma unroll
            for (int i = j + 1; i < m; ++i) L[tri(i, j)] = L[tri(i, j)] / ljj;
            L[tri(j, j)] = ljj;
#pragma unroll
            for (int i = j + 1; i < m; ++i)
#pragma unroll
                for (int k = j + 1; k <= i; ++k) L[tri(i, k)] = L[tri(i, k)] - L[tri(i, j)] * L[tri(k, j)];
        }
        double y[m];
#pragma unroll
        for (int i = 0; i < m; ++i) {   // forward: L y = der
            double sum = der[i];
#pragma unroll
            for (int p = 0; p < i; ++p) sum -= L[tri(i, p)] * y[p];
            y[i] = sum / L[tri(i, i)];
        }
#pragma unroll
        for (int i = m - 1; i >= 0; --i) {   // back: L^T x = y
            double sum = y[i];
#pragma unroll
            for (int p = i + 1; p < m; ++p) sum -= L[tri(p, i)] * x[p];
            x[i] = sum / L[tri(i, i)];
        }
        if (!good)
#pragma unroll
            for (int i = 0; i < m; ++i) x[i] = 0.0;
    }
    {   // MakeZeroAverage (pairwise_scoring.rs:255-265)
        double avg = 0.0;
#pragma unroll
        for (int i = 0; i < n; ++i) avg += x[i];
        avg = avg / (double)n;
#pragma unroll
        for (int i = 0; i < n; ++i) x[i] -= avg;
    }
    // ---- score: rows of W in column order (b ascending), inner sums per row ----
    double inner[n];
#pragma unroll
    for (int i = 0; i < n; ++i) inner[i] = 0.0;
#pragma unroll
    for (uint32_t b = 0; b < P; ++b)
#pragma unroll
        for (uint32_t a = 0; a < P; ++a) {
#pragma unroll
            for (uint32_t u = 0; u < 2; ++u) {
                const int r = 2 * (int)a + (int)u;
                long long e0, e1;
                if (a == b) {
                    e0 = u == 0 ? dg[r] : da[a];
                    e1 = u == 0 ? da[a] : dg[r];
                } else {
                    const PairCells c = pair_cells(R, rs, T, rs, P, a < b ? a : b, a < b ? b : a);
                    long long dp;
                    pair_row_entries(c, a > b, u, e0, e1, dp);
                }
                inner[r] += x[2 * b] * ((double)e0 * pair_inv);
                inner[r] += x[2 * b + 1] * ((double)e1 * pair_inv);
            }
        }
    double outer = 0.0;
#pragma unroll
    for (int i = 0; i < n; ++i) outer += x[i] * (der[i] - 0.5 * inner[i]);
    scores[(size_t)f * B + s] = outer;
}

// The m x m SPD system of one wavefront, row r in lane r's registers (entries above the
// diagonal are don't-care) and the right-hand side y in lane r: right-looking Cholesky (the
// pivot and the pivot column come from the owning lanes by readlane; every element receives
// its pivot subtractions in ascending order with the reference's roundings, as
// pairwise_factor_solve_block), the forward substitution p ascending, then the back
// substitution reading L^T from Lbuf (m (m + 1) / 2 doubles of LDS).  Returns the lane's
// component of the solution: 0 past m, and 0 everywhere when a pivot is not positive.
template <int m>
__device__ __forceinline__ double pairwise_rows_solve(double (&row)[m], double y, double* __restrict__ Lbuf,
                                                      int lane) {
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
    if (good) {
#pragma unroll
        for (int p = 0; p < m; ++p) {   // forward: y[i] -= L[i][p] y[p], p ascending
            const double yp = readlane_f64(y, p) / readlane_f64(row[p], p);
            y = lane == p ? yp : (lane > p ? y - row[p] * yp : y);
        }
        if (lane < m) {
#pragma unroll
            for (int c = 0; c < m; ++c)
                if (c <= lane) Lbuf[tri(lane, c)] = row[c];
        }
        __syncthreads();
#pragma unroll
        for (int p = m - 1; p >= 0; --p) {   // back: L^T x = y
            const double xp = readlane_f64(y, p) / readlane_f64(row[p], p);
            const double lpi = lane < p ? Lbuf[tri(p, lane)] : 0.0;
            y = lane == p ? xp : (lane < p ? y - lpi * xp : y);
        }
    }
    return good && lane < m ? y : 0.0;
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
    double* der = M + pair_cand_l_words(P);
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
        x = pairwise_rows_solve<m>(row, lane < m ? der[lane] : 0.0, M, lane);
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
// privatized in LDS up to 128 leaves (in_lds), else added to out directly.  Launched as one
// 1024-thread workgroup a CU, so that few LDS images are flushed.
static __global__ __launch_bounds__(1024) void pair_leaf_weights_kernel(
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

// PairLogitPairwise leaves of 3 to 64 leaves in one wavefront (the arithmetic of
// pairwise_leaf_kernel, whose steps here need no barrier): lane r < L - 1 holds row r of
// M = W + prior terms in registers, lanes L - 1 .. 62 rows of the identity, so that the
// 63 x 63 system factors as blockdiag(M, I) with M's elements getting exactly their own
// operations (the identity rows contribute 0 * x terms and unit pivots).  LDS: the L^T buffer
// (2016 doubles) and the L doubles of the solution.
constexpr uint32_t kPairLeafWaveDoubles = 63 * 64 / 2 + 64;
static __global__ __launch_bounds__(64) void pairwise_leaf_wave_kernel(
    const long long* __restrict__ lw, uint32_t L, const long long* __restrict__ sums, uint32_t CL,
    const Scales* __restrict__ sc, double pair_inv, double l2, double prior, double lr,
    double* __restrict__ raw, double* __restrict__ scaled) {
    constexpr int m = 63;
    __shared__ double Lbuf[kPairLeafWaveDoubles];
    double* res = Lbuf + 63 * 64 / 2;
    const int lane = threadIdx.x, mm = (int)L - 1;
    const double cell_prior = 1.0 / (double)L;
    const double non_diag = -prior * cell_prior;
    const double diag = prior * (1.0 - cell_prior) + l2;
    const double inv_d = sc->inv[kLeafDer];
    double row[m];
#pragma unroll
    for (int c = 0; c < m; ++c) {
        double v;
        if (lane < mm) {
            const double wrc = c <= lane ? (double)lw[(size_t)lane * L + c] * pair_inv : 0.0;
            v = c < lane ? wrc + non_diag : (c == lane ? wrc + diag : 0.0);
        } else {
            v = c == lane ? 1.0 : 0.0;
        }
        row[c] = v;
    }
    const double y = lane < mm ? (double)sums[(size_t)lane * CL] * inv_d : 0.0;
    const double x = pairwise_rows_solve<m>(row, y, Lbuf, lane);
    __syncthreads();
    if (lane < (int)L) res[lane] = lane < mm ? x : 0.0;
    __syncthreads();
    zero_average_block(res, (int)L);
    if (lane < (int)L) raw[lane] = res[lane];
    __syncthreads();
    if (lane == 0) pairwise_center_lane0(raw, sums, CL, L, lr, scaled);
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
