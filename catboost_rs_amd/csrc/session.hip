// Host side of the gfx950 training path: the C-ABI declared in include/cbhip.h.
//
// A session keeps every per-fit buffer resident in HBM (bins in two layouts, target,
// weights, approximant, score channels, leaf ids, level histograms) and grows each tree
// with a fixed sequence of kernel launches on one stream, with no host synchronisation
// between levels: the split of every level is chosen, applied and planned on the device.
// The only per-tree transfer is the tree itself (depth splits + 2^depth leaf values).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../include/cbhip.h"
#include "common.hpp"
#include "kernels.hpp"
#include "ranking.hpp"

using namespace cbh;

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

#define HIP_TRY(expr)                                                                     \
    do {                                                                                  \
        hipError_t e_ = (expr);                                                           \
        if (e_ != hipSuccess)                                                             \
            return fail(CBH_ERR_DEVICE, std::string(#expr " failed: ") + hipGetErrorString(e_)); \
    } while (0)

template <typename T>
int dalloc(T** p, size_t count) {
    *p = nullptr;
    if (count == 0) return CBH_OK;
    hipError_t e = hipMalloc((void**)p, count * sizeof(T));
    if (e != hipSuccess) {
        *p = nullptr;
        return fail(CBH_ERR_DEVICE, std::string("hipMalloc failed: ") + hipGetErrorString(e));
    }
    return CBH_OK;
}

template <typename T>
void dfree(T*& p) {
    if (p) (void)hipFree(p);
    p = nullptr;
}

#define CHECK(expr)              \
    do {                         \
        int rc_ = (expr);        \
        if (rc_ != CBH_OK) return rc_; \
    } while (0)

unsigned grid_for(uint64_t work, unsigned block, unsigned cap = 65535u * 4) {
    uint64_t g = (work + block - 1) / block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (unsigned)g;
}

// Dispatch a runtime approx dimension to a compile-time K.
template <typename F>
int with_k(int k, F&& f) {
    switch (k) {
        case 1: return f(std::integral_constant<int, 1>{});
        case 2: return f(std::integral_constant<int, 2>{});
        case 3: return f(std::integral_constant<int, 3>{});
        case 4: return f(std::integral_constant<int, 4>{});
        case 5: return f(std::integral_constant<int, 5>{});
        case 6: return f(std::integral_constant<int, 6>{});
        case 7: return f(std::integral_constant<int, 7>{});
        case 8: return f(std::integral_constant<int, 8>{});
        case 10: return f(std::integral_constant<int, 10>{});
        case 12: return f(std::integral_constant<int, 12>{});
        case 16: return f(std::integral_constant<int, 16>{});
        default: return fail(CBH_ERR_UNSUPPORTED, "approx_dim " + std::to_string(k) +
                                                      " has no compiled kernel variant");
    }
}


struct StageTimer {
    hipEvent_t a = nullptr, b = nullptr;
};

}  // namespace

int cbh_internal_fail(int code, const std::string& msg) { return fail(code, msg); }
int cbh_internal_ctr_bins(const cbh_device_ctr_column* cols, uint32_t m, const uint64_t* n_buckets,
                          const uint32_t* permutation, const uint32_t* target_class, uint64_t n,
                          uint8_t* dst, hipStream_t st);   // categorical.hip
int cbh_internal_quantize(const float* d_col, uint64_t n, const double* d_borders, uint32_t nb, uint8_t* d_out,
                          hipStream_t st);  // borders.hip

struct cbh_session {
    cbh_config cfg{};
    std::vector<uint8_t> one_hot_host;
    uint64_t n = 0;
    uint32_t F = 0, B = 0, W = 0, Ws = 0, K = 1, C = 2, depth = 0;   // Ws: words per packed row in memory
    double lr = 0.0, l2 = 0.0;
    bool has_weight = false, target_set = false, pending = false;
    // host work that the caller runs while the device grows the tree (between the launch and the
    // wait of cbh_session_grow; cbh_internal_set_overlap)
    void (*overlap_fn)(void*) = nullptr;
    void* overlap_arg = nullptr;
    hipStream_t stream = nullptr;
    int device = 0;

    // resident buffers
    uint32_t* rows = nullptr;
    uint8_t* cols = nullptr;
    double* weight = nullptr;
    double* target = nullptr;
    double* approx = nullptr;
    double* sstat = nullptr;         // [n][C] score channels (f64; int64 in place for the generic fill)
    double* host_sample = nullptr;
    uint16_t* leaf = nullptr;
    uint32_t* idx = nullptr;
    long long* hist[2] = {nullptr, nullptr};
    size_t hist_cells_max = 0;
    uint32_t* cnt = nullptr;
    uint32_t* totals = nullptr;
    uint32_t n_part_blocks = 0;
    LevelPlan* plans = nullptr;   // [depth]
    SplitRec* splits = nullptr;   // [depth]
    double* best_score = nullptr;
    uint32_t* best_bin = nullptr;
    uint32_t* n_cand = nullptr;
    uint32_t max_cand = 0;           // most candidates of any feature (threads of the scorer)
    bool score_chain = true;         // parents split over waves for K > 1 (CBH_SCORE_CHAIN=off: one wave)
    uint32_t chain_spin = kChainSpinLimit;   // polls of a chained scorer wave's wait (CBH_CHAIN_SPIN: a test knob)
    uint32_t chain_nf = 0;   // features per chained-scorer workgroup at most (CBH_CHAIN_FEATURES; 0: no cap)
    uint8_t* one_hot = nullptr;
    Scales* scales = nullptr;
    Bounds* bounds = nullptr;
    long long* leaf_sums = nullptr;
    double* leaf_raw = nullptr;
    double* leaf_scaled = nullptr;
    FillTiles tiles{};
    uint32_t fill_ranges = 8;   // row ranges per tile (multiple of 8)
    uint64_t* jump = nullptr;               // [2048 + 2 * n_coarse]: fine a, fine d, coarse a, coarse d
    uint64_t n_coarse = 0;
    unsigned long long* partials = nullptr; // [kPrepBlocks][kPartials]

    // pair losses (PairLogit: pointwise scoring over pairwise weights; PairLogitPairwise:
    // pairwise statistics scoring and Cholesky leaves)
    bool ranking = false, pairwise = false, pairs_set = false;
    double prior = 0.1;
    uint32_t n_groups = 0;
    uint64_t n_pairs = 0;
    double pair_inv = 1.0;
    uint32_t* group_off = nullptr;   // [n_groups + 1]
    uint32_t* los_off = nullptr;     // [n + 1] pairs of each row as a loser: los_idx[los_off[i] ..]
    uint32_t* los_idx = nullptr;     // [m] their indices in competitor order, ascending
    uint32_t* comp_off = nullptr;    // [n + 1]
    uint32_t* comp_win = nullptr;    // [m]
    uint32_t* comp_los = nullptr;    // [m]
    double* comp_w = nullptr;        // [m]
    long long* comp_wq = nullptr;    // [m]
    double* ext_der = nullptr;       // [2][n] der1, der2
    double* score_w = nullptr;       // [n] pairwise weights
    long long* pair_st = nullptr;    // [F][Pmax][Pmax][B][2]
    double* cand_scores = nullptr;   // [F][B]
    long long* leaf_w = nullptr;     // [L][L]
    uint32_t* key_cnt = nullptr;     // [Pmax^2] pairs per unordered leaf pair
    uint32_t* key_off = nullptr;     // [Pmax^2 + 1]
    uint32_t* key_cur = nullptr;     // [Pmax^2]
    uint2* key_rec = nullptr;        // [m] pair records grouped by leaf pair
    long long* key_wq = nullptr;     // [m]
    uint4* pair_desc = nullptr;      // chunk descriptors of a level's statistics (pair_plan_kernel)
    uint32_t pair_cus = 256;         // CUs of the device: a level's chunks are sized to fill them once
    uint32_t cus = 256;              // CUs of the device (the leaf reduction's grid)
    uint32_t* pair_mk = nullptr;     // keys of several chunks
    uint32_t* pair_nd = nullptr;     // [2] descriptors, keys of several chunks
    double* pair_ws = nullptr;       // global workspace of the 256-leaf solves (depth 8)
    uint32_t pair_cand_wgs = 0;      // workgroups of the 128-leaf-level candidate solves (global workspace)
    size_t pair_leaf_lds = 0;        // LDS of the leaf solve (0: global workspace)

    // dominant-bin skip of the fill (features whose most frequent bin holds >= 1/8 of rows)
    uint32_t* skip_bin = nullptr;    // [F] dominant bin, or 256 (no skip)
    long long* seg_tot = nullptr;    // [kMaxLeaves / 2][C] channel totals per built segment
    bool use_skip = false;
    uint64_t n_skip = 0;
    double nd_per_tile = 32.0;       // mean non-dominant (feature, bin) entries of a row per 32-feature tile
    uint16_t* row_ent = nullptr;     // profiling with the dominant-bin skip: entries per row
    unsigned long long* fill_ent = nullptr;   // profiling: entries the fill launches added (device)
    bool pks = false;                // packed multi-channel fill over sparse entries
    uint16_t* pks_a = nullptr;       // [pkk_tiles][n][16] entry codes 0..15 of every (tile, row)
    uint16_t* pks_b = nullptr;       // [pkk_tiles][n][16] entry codes 16..31

    // K == 1 tiled fills: the tiled exact fill (32-feature tiles, both channels at the tree's
    // full fixed-point scale, one 64-bit LDS atomic per (row, feature, channel)) or the rounded
    // packed fill (64-feature tiles, both channels rounded to 18-bit rows in one 64-bit word,
    // one LDS atomic per (row, feature); a measurement knob)
    bool packed = false, tiled = false;
    // count-packed fill (K == 1, integer score weights: bootstrap No or Bernoulli over integer
    // object weights): the der channel at >= 2^-30 and the integer weight in one 64-bit word per
    // row, one LDS atomic per (row, feature), 64-feature tiles (the rounded packed fill's loops)
    bool count = false;
    bool int_w = true;                         // every object weight is an integer in [0, 2^20]
    uint32_t ex_sets = 3;                      // tiled: blocks in flight of the full loop
    // packed multi-channel fill (K > 1: two score channels per 64-bit word, NP = ceil(C/2) planes)
    bool pkk = false;
    uint32_t pkk_tiles = 0, pkk_ranges = 8;
    bool pks_small = false;          // sparse entries, NP * B * 32 <= 4096: 4 cells per thread
    bool w_static = false;           // packed multi-channel fill, the weight alone in the last plane and
    bool w0_ready = false;           // the same every tree: its level-0 cells cached after the first tree
    long long* w0_cache = nullptr;   // [F][B] (the fill's cells, before the dominant-bin rebuild)
    bool l0_cached = false;          // the last recorded or enqueued tree took the weight's level-0 cells
                                     // from the cache (its level-0 fill one plane short)
    int pack_bits = 0;
    unsigned long long* spack = nullptr;   // packed: [n] words
    unsigned long long* sseq = nullptr;    // the listed rows' statistics in idx order (packed: [V]; tiled: [V][2] f64)
    uint32_t* trows = nullptr;             // tiled fills: tile-major row words (pack_tiles_kernel)
    uint32_t pk_tiles = 0, pk_ranges = 8, pk_swap = 1;
    struct PackPlan {                          // tiled fill launch: tiles of the full loop, ranges
        uint32_t tiles16 = 0, ranges = 0, ranges_n = 0, blocks = 0;   // of each, narrow-tile ranges, workgroups
    } pk_dense, pk_gath;                       // the dense level; the gathered levels
    uint32_t pk_rm_sh = 0;                     // tiled fills: log2 bytes of a row-major row (0: tile-major gathers)
    bool pk_signed_w = false;              // some object or pair weight is negative
    // level histograms of the last tree kept for inspection (cbh_session_capture_hists): level l
    // at hist_cap + hist_cap_off[l], the level's 2^l leaves in prefix form, as the scorer read them
    long long* hist_cap = nullptr;
    size_t hist_cap_off[kMaxDepth + 1] = {};
    size_t pk_lds = 0;
    JumpTabs jt() const {
        return JumpTabs{jump, jump + 1024, jump + 2048, jump + 2048 + n_coarse};
    }

    // CTR columns: the last ctr_n features, scored with the model_size_reg weight of a
    // (ctr type, projection) group not used yet; leaves over the averaging-permutation bins
    uint32_t ctr_n = 0;
    uint8_t* ctr_avg = nullptr;                 // [ctr_n][n]
    std::vector<uint32_t> ctr_bc, ctr_group;    // bucket count, group of every CTR column
    std::vector<uint8_t> ctr_used;              // [ctr_n] groups chosen by an earlier tree
    uint64_t ctr_eligible_max = 1;
    uint32_t cat_n = 0;
    uint32_t* cat_bk = nullptr;                 // [cat_n][n] first-seen buckets (32-bit) ...
    uint16_t* cat_bk16 = nullptr;               // ... or 16-bit, when every column has < 65536
    uint32_t* cat_nb_dev = nullptr;             // [cat_n]
    std::vector<uint32_t> cat_nb;
    uint64_t* phantom_off = nullptr;            // [cat_n] word offsets of the bitmaps
    uint32_t* phantom_bits = nullptr;
    unsigned long long* phantom_cnt = nullptr;  // [cat_n]
    double msr = 0.5;
    double* fweight = nullptr;                  // [F] score multiplier (1 except CTR columns)
    std::vector<double> fweight_host;
    bool fweight_one = false;                   // the device weights are all 1
    // device-side weights (ctr_dev): pow(1 + bc_c / m, -model_size_reg) tabulated on the host
    // for every reachable max count m in [ctr_m_lo, ctr_m_hi], per-level bitmap offsets, and
    // the model's used groups mirrored before every tree
    bool ctr_dev = false;
    double* ctr_pow = nullptr;                  // [ctr_n][m_hi - m_lo + 1]
    uint64_t ctr_m_lo = 0, ctr_m_hi = 0;
    uint32_t* ctr_group_dev = nullptr;          // [ctr_n]
    uint8_t* ctr_used_dev = nullptr;            // [ctr_n] by group
    uint8_t* pin_ctr_used = nullptr;
    uint64_t* phantom_off_lv = nullptr;         // [depth][cat_n] word offsets at each level

    // per-tree launch sequence recorded once and replayed (index: host sample given or not)
    hipGraphExec_t tree_graph[2] = {nullptr, nullptr};
    bool graph_off = false;          // recording failed once: stay eager
    SampleParams* smp_dev = nullptr; // [2]: the tree's sampling parameters, an inert set
    // pinned staging of the per-tree results (the recorded copies land here)
    SampleParams* pin_smp = nullptr;
    // the per-tree results (splits, plans, bounds, raw leaves) live in one device block and come
    // back in one copy into its pinned mirror; the pointers below are views into the blocks
    unsigned char* out_dev = nullptr;
    unsigned char* pin_out = nullptr;
    size_t out_bytes = 0;
    SplitRec* pin_splits = nullptr;
    LevelPlan* pin_plans = nullptr;
    Bounds* pin_bounds = nullptr;
    double* pin_leaves = nullptr;

    // profiling
    cbh_stats stats{};
    std::vector<std::pair<int, StageTimer>> timers;
    size_t timer_used = 0;

    ~cbh_session() { release(); }

    void release() {
        dfree(rows); dfree(cols); dfree(weight); dfree(target); dfree(approx); dfree(sstat);
        dfree(host_sample); dfree(leaf); dfree(idx); dfree(hist[0]); dfree(hist[1]); dfree(cnt);
        dfree(totals); dfree(best_score);
        dfree(best_bin); dfree(n_cand); dfree(one_hot); dfree(scales);
        dfree(leaf_sums); dfree(leaf_scaled); dfree(jump);
        dfree(out_dev);
        plans = nullptr; splits = nullptr; bounds = nullptr; leaf_raw = nullptr;
        dfree(partials);
        dfree(group_off); dfree(los_off); dfree(los_idx); dfree(comp_off); dfree(comp_win); dfree(comp_los); dfree(comp_w);
        dfree(comp_wq); dfree(ext_der); dfree(score_w); dfree(pair_st);
        dfree(cand_scores); dfree(leaf_w); dfree(skip_bin); dfree(seg_tot); dfree(spack); dfree(sseq); dfree(trows); dfree(pks_a); dfree(pks_b); dfree(row_ent); dfree(fill_ent); dfree(w0_cache);
        dfree(key_cnt); dfree(key_off); dfree(key_cur); dfree(key_rec); dfree(key_wq); dfree(pair_ws);
        dfree(pair_desc); dfree(pair_mk); dfree(pair_nd);
        dfree(ctr_avg); dfree(cat_bk); dfree(cat_bk16); dfree(cat_nb_dev); dfree(phantom_off); dfree(phantom_bits);
        dfree(phantom_cnt); dfree(fweight); dfree(ctr_pow); dfree(ctr_group_dev); dfree(ctr_used_dev);
        dfree(phantom_off_lv); dfree(hist_cap);
        if (pin_ctr_used) (void)hipHostFree(pin_ctr_used);
        pin_ctr_used = nullptr;
        for (auto& g : tree_graph)
            if (g) (void)hipGraphExecDestroy(g);
        tree_graph[0] = tree_graph[1] = nullptr;
        dfree(smp_dev);
        for (void* p : {(void*)pin_smp, (void*)pin_out})
            if (p) (void)hipHostFree(p);
        pin_smp = nullptr; pin_out = nullptr;
        pin_splits = nullptr; pin_plans = nullptr; pin_bounds = nullptr; pin_leaves = nullptr;
        for (auto& t : timers) {
            if (t.second.a) (void)hipEventDestroy(t.second.a);
            if (t.second.b) (void)hipEventDestroy(t.second.b);
        }
        timers.clear();
        if (stream) (void)hipStreamDestroy(stream);
        stream = nullptr;
    }

    // Stage timing: begin() records the start event of a stage, end() the stop event.
    int stage_begin(int stage) {
        if (!cfg.profile) return CBH_OK;
        if (timer_used == timers.size()) {
            StageTimer t;
            HIP_TRY(hipEventCreate(&t.a));
            HIP_TRY(hipEventCreate(&t.b));
            timers.push_back({stage, t});
        }
        timers[timer_used].first = stage;
        HIP_TRY(hipEventRecord(timers[timer_used].second.a, stream));
        return CBH_OK;
    }
    int stage_end() {
        if (!cfg.profile) return CBH_OK;
        HIP_TRY(hipEventRecord(timers[timer_used].second.b, stream));
        ++timer_used;
        return CBH_OK;
    }
    int collect_timers() {
        for (size_t i = 0; i < timer_used; ++i) {
            float ms = 0.f;
            HIP_TRY(hipEventElapsedTime(&ms, timers[i].second.a, timers[i].second.b));
            double* dst = nullptr;
            switch (timers[i].first) {
                case 0: dst = &stats.fill_ms; break;
                case 1: dst = &stats.derive_ms; break;
                case 2: dst = &stats.score_ms; break;
                case 3: dst = &stats.partition_ms; break;
                case 4: dst = &stats.leaf_ms; break;
                default: dst = &stats.prepare_ms; break;
            }
            *dst += ms;
            stats.total_ms += ms;
        }
        timer_used = 0;
        return CBH_OK;
    }
};

namespace {

enum { kStFill = 0, kStDerive = 1, kStScore = 2, kStPartition = 3, kStLeaf = 4, kStPrepare = 5 };

int validate_config(const cbh_config* cfg, uint32_t n_bins, uint64_t n, uint32_t F) {
    if (!cfg) return fail(CBH_ERR_INVALID_ARG, "config is null");
    if (cfg->boosting_type_is_plain != 1 || cfg->fold_count != 1)
        return fail(CBH_DECLINED, "ordered boosting / several folds are not covered on device");
    if (cfg->depth < 1 || cfg->depth > kMaxDepth)
        return fail(CBH_DECLINED, "depth outside 1..8 is not covered on device");
    if (cfg->loss < CBH_LOSS_RMSE || cfg->loss > CBH_LOSS_PAIRLOGIT_PAIRWISE)
        return fail(CBH_DECLINED, "loss not covered on device");
    if (cfg->loss == CBH_LOSS_MULTICLASS) {
        const int k = cfg->approx_dim;
        if (k < 2 || k > kMaxK) return fail(CBH_DECLINED, "MultiClass approx_dim must be 2..16");
        if (!(k <= 8 || k == 10 || k == 12 || k == 16))   // the compiled variants (with_k)
            return fail(CBH_DECLINED, "MultiClass approx_dim " + std::to_string(k) + " has no compiled kernel variant");
        // the leaf reduction keeps 2^depth leaves x (K + K(K+1)/2) int64 cells in one
        // workgroup's LDS (160 KiB on gfx950)
        const uint64_t lds = ((uint64_t)1 << cfg->depth) * (uint64_t)(k + k * (k + 1) / 2) * 8u;
        if (lds > 160u * 1024u)
            return fail(CBH_DECLINED, "MultiClass leaf statistics of approx_dim " + std::to_string(k) + " at depth " +
                                          std::to_string(cfg->depth) + " exceed the LDS of one workgroup");
        if (cfg->leaf_method != CBH_LEAF_NEWTON)
            return fail(CBH_DECLINED, "MultiClass needs Newton leaves (boosting.rs:2169-2186)");
    } else if (cfg->approx_dim != 1) {
        return fail(CBH_ERR_INVALID_ARG, "approx_dim must be 1 for scalar losses");
    }
    // Cosine, L2, SolarL2, LOOL2, SatL2 (map_score_fn, session.rs:1118-1128); the pairwise
    // scorer of PairLogitPairwise has its own score
    if (cfg->score_function < CBH_SCORE_COSINE || cfg->score_function > CBH_SCORE_SAT_L2)
        return fail(CBH_DECLINED, "score function not covered on device");
    if (cfg->score_function > CBH_SCORE_L2 && cfg->loss == CBH_LOSS_PAIRLOGIT_PAIRWISE)
        return fail(CBH_DECLINED, "SolarL2 / LOOL2 / SatL2 are pointwise score calcers");
    if (n_bins < 2 || n_bins > 256)
        return fail(CBH_DECLINED, "n_bins must be in 2..256 (u8 bins)");
    if (n == 0 || F == 0) return fail(CBH_ERR_DEGENERATE, "empty dataset");
    if (n >= (1ull << 32)) return fail(CBH_DECLINED, "more than 2^32-1 rows");
    return CBH_OK;
}

int session_alloc(cbh_session* s) {
    const uint64_t n = s->n;
    CHECK(dalloc(&s->rows, (size_t)n * s->Ws));
    CHECK(dalloc(&s->cols, (size_t)n * s->F));
    if (s->has_weight) CHECK(dalloc(&s->weight, n));
    CHECK(dalloc(&s->target, n));
    CHECK(dalloc(&s->approx, (size_t)n * s->K));
    CHECK(dalloc(&s->sstat, (size_t)n * s->C));
    CHECK(dalloc(&s->leaf, n));
    CHECK(dalloc(&s->idx, n));
    const size_t per_leaf = (size_t)s->F * s->B * s->C;
    s->hist_cells_max = per_leaf << (s->depth - 1);
    CHECK(dalloc(&s->hist[0], s->hist_cells_max));
    CHECK(dalloc(&s->hist[1], s->hist_cells_max));
    s->n_part_blocks = (uint32_t)((n + kPartRows - 1) / kPartRows);
    CHECK(dalloc(&s->cnt, ((size_t)s->n_part_blocks * 4) << s->depth));   // [leaf][wave]
    CHECK(dalloc(&s->totals, (size_t)1 << s->depth));
    {   // one block for the per-tree results, sections 256-byte aligned
        auto up = [](size_t b) { return (b + 255) / 256 * 256; };
        const size_t o_plans = up(sizeof(SplitRec) * s->depth);
        const size_t o_bounds = o_plans + up(sizeof(LevelPlan) * s->depth);
        const size_t o_leaves = o_bounds + up(sizeof(Bounds));
        s->out_bytes = o_leaves + sizeof(double) * ((size_t)1 << s->depth) * s->K;
        CHECK(dalloc(&s->out_dev, s->out_bytes));
        HIP_TRY(hipHostMalloc((void**)&s->pin_out, s->out_bytes, hipHostMallocDefault));
        s->splits = (SplitRec*)s->out_dev;
        s->plans = (LevelPlan*)(s->out_dev + o_plans);
        s->bounds = (Bounds*)(s->out_dev + o_bounds);
        s->leaf_raw = (double*)(s->out_dev + o_leaves);
        s->pin_splits = (SplitRec*)s->pin_out;
        s->pin_plans = (LevelPlan*)(s->pin_out + o_plans);
        s->pin_bounds = (Bounds*)(s->pin_out + o_bounds);
        s->pin_leaves = (double*)(s->pin_out + o_leaves);
    }
    CHECK(dalloc(&s->best_score, s->F));
    CHECK(dalloc(&s->best_bin, s->F));
    CHECK(dalloc(&s->n_cand, s->F));
    CHECK(dalloc(&s->scales, 1));
    const uint32_t CL = s->K == 1 ? 3 : s->K + s->K * (s->K + 1) / 2;
    CHECK(dalloc(&s->leaf_sums, ((size_t)1 << s->depth) * CL));
    if (s->ranking) {
        CHECK(dalloc(&s->ext_der, 2 * n));
        CHECK(dalloc(&s->score_w, n));
        CHECK(dalloc(&s->comp_off, n + 1));
    }
    if (s->pairwise) {
        const size_t pmax = (size_t)1 << (s->depth - 1);
        CHECK(dalloc(&s->pair_st, (size_t)s->F * s->B * pmax * pmax * 2));
        CHECK(dalloc(&s->cand_scores, (size_t)s->F * s->B));
        CHECK(dalloc(&s->leaf_w, ((size_t)1 << s->depth) << s->depth));
        CHECK(dalloc(&s->key_cnt, pmax * pmax));
        CHECK(dalloc(&s->key_off, pmax * pmax + 1));
        CHECK(dalloc(&s->key_cur, pmax * pmax));
        CHECK(dalloc(&s->pair_nd, 2));
        int cus = 0;
        HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, s->device));
        s->pair_cus = (uint32_t)std::max(cus, 1);
        // every LDS size a level can ask for is set here, before any tree is recorded as a graph
        HIP_TRY(hipFuncSetAttribute((const void*)pair_stats_feature_kernel<true>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)pair_stat_lds(s->B)));
        HIP_TRY(hipFuncSetAttribute((const void*)pair_stats_feature_kernel<false>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)pair_stat_lds(s->B)));
        HIP_TRY(hipFuncSetAttribute((const void*)pair_key_count_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)(pmax * pmax * sizeof(uint32_t))));
        HIP_TRY(hipFuncSetAttribute((const void*)pair_key_scatter_kernel,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)(pmax * pmax * sizeof(uint32_t))));
        const uint32_t L = 1u << s->depth;
        const size_t leaf_bytes = pair_leaf_solve_doubles(L) * sizeof(double);
        size_t ws_doubles = 0;
        if (leaf_bytes <= kPairLdsMax) {
            s->pair_leaf_lds = leaf_bytes;
            HIP_TRY(hipFuncSetAttribute((const void*)pairwise_leaf_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)leaf_bytes));
        } else {
            ws_doubles = pair_leaf_solve_doubles(L);
        }
        if ((size_t)L * L * sizeof(long long) <= kPairLdsMax)
            HIP_TRY(hipFuncSetAttribute((const void*)pair_leaf_weights_kernel,
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)((size_t)L * L * sizeof(long long))));
        // levels of 64 leaves solve their candidates in LDS, the level of 128 in a global
        // workspace, one slot per workgroup of a persistent grid
        if (pmax >= 64)
            HIP_TRY(hipFuncSetAttribute((const void*)pairwise_candidate_block_kernel,
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)(pair_cand_block_doubles(64) * sizeof(double))));
        if (pmax >= 128) {
            const uint64_t total = (uint64_t)s->F * (s->B - 1);
            s->pair_cand_wgs = (uint32_t)std::min<uint64_t>(std::max<uint64_t>(total, 1), kPairCandGlobalWgs);
            ws_doubles = std::max(ws_doubles, (size_t)s->pair_cand_wgs * pair_cand_block_doubles(128));
        }
        if (ws_doubles) CHECK(dalloc(&s->pair_ws, ws_doubles));
    }
    CHECK(dalloc(&s->smp_dev, 2));
    HIP_TRY(hipMemset(s->smp_dev, 0, 2 * sizeof(SampleParams)));
    HIP_TRY(hipHostMalloc((void**)&s->pin_smp, sizeof(SampleParams), hipHostMallocDefault));
    CHECK(dalloc(&s->leaf_scaled, ((size_t)1 << s->depth) * s->K));
    CHECK(dalloc(&s->partials, (size_t)kPrepBlocks * kPartials));
    s->n_coarse = (n >> 10) + 2;
    CHECK(dalloc(&s->jump, 2048 + 2 * s->n_coarse));
    {
        std::vector<uint64_t> h(2048 + 2 * s->n_coarse);
        make_jump_tables(s->n_coarse, h.data(), h.data() + 1024, h.data() + 2048,
                         h.data() + 2048 + s->n_coarse);
        HIP_TRY(hipMemcpy(s->jump, h.data(), sizeof(uint64_t) * h.size(), hipMemcpyHostToDevice));
    }
    return CBH_OK;
}

// Row ranges per feature tile: (tile, range) workgroups for one or two rounds of the CUs'
// resident slots, ranges a multiple of 8: one round when it fills >= 97% of the slots, else
// the better of the two (config 2: 7 tiles on 256 one-workgroup CUs -> 1 round uses 224
// slots, 2 rounds 504 of 512: fill 0.594 -> 0.563 ms per launch; more rounds add flushes and
// lose).  CBH_FILL_WAVES overrides the workgroups per CU (a tuning knob).
uint32_t pick_ranges(uint32_t cus, uint32_t per_cu, uint32_t nt, uint64_t n) {
    const uint32_t cap = cus * std::max<uint32_t>(per_cu, 1);
    auto ranges_for = [&](uint32_t slots) { return std::max<uint32_t>(8, slots / nt / 8 * 8); };
    auto fill_frac = [&](uint32_t G, uint32_t rounds) { return (double)G * nt / ((double)rounds * cap); };
    uint32_t G = ranges_for(cap);
    const uint32_t G2 = ranges_for(2 * cap);
    // (two rounds only with long ranges: each workgroup's flush is a fixed cost, and at 1M rows
    // the second round's extra flushes lose: config 3 fill 0.060 -> 0.083 ms)
    if (fill_frac(G, 1) < 0.97 && fill_frac(G2, 2) > fill_frac(G, 1) && n / G2 >= 65536) G = G2;
    if (const char* e = std::getenv("CBH_FILL_WAVES")) {
        const long m = std::strtol(e, nullptr, 10);
        if (m >= 1 && m <= 16) G = ranges_for(cus * (uint32_t)m);
    }
    return G;
}

// Row ranges of the tiled fills.  Tiles of the full loop (TWM words: 16 for the packed fill, 8
// for the tiled exact fill; a shorter last tile runs the same loop, its lanes past TW adding to
// columns that are never read, so its row costs about as much as a full one's) get G ranges
// each.  A narrow last tile (the packed fill: exactly 2 words, at the dense level only; the
// exact fill: at most 2 words, at every level) runs the narrow loop (8 rows per DPP row) in
// Gn = G * r ranges, r its cost per row relative to a full tile's (CBH_PACK_NARROW_COST, a
// measurement knob; CBH_PACK_NARROW=off keeps the full loop).  One round of workgroups fills
// the resident slots.  The gathered levels read row-major words (2^rm_sh bytes per row) when
// the padded row is a power of two under 4 GiB in all: the tiles of a range run on one XCD, so
// a listed row's lines come from HBM once for all its tiles (CBH_PACK_GATHER=tiles keeps the
// tile-major slices there, a measurement knob).
void pick_tile_ranges(cbh_session* s, uint32_t cus, uint32_t per_cu, uint32_t TWM) {
    const uint32_t cap = cus * std::max<uint32_t>(per_cu, 1);
    const bool exact = TWM == kExTileWords;
    double r = exact ? 0.3 : 0.2;
    if (const char* e = std::getenv("CBH_PACK_NARROW_COST")) {
        const double v = std::strtod(e, nullptr);
        if (v > 0.0 && v <= 1.0) r = v;
    }
    const uint32_t n_tiles = (s->W + TWM - 1) / TWM;
    auto plan = [&](bool narrow) {
        cbh_session::PackPlan pl;
        const uint32_t nt = narrow ? s->W / TWM : n_tiles;
        auto gn_of = [&](uint32_t g) { return narrow ? std::max<uint32_t>(1, (uint32_t)std::ceil(g * r)) : 0u; };
        uint32_t G = 0, Gn = 0;
        if (nt == 0) {   // one narrow tile: every slot
            Gn = cap;
        } else {
            G = std::max<uint32_t>(1, cap / nt);
            while (G > 1 && nt * G + gn_of(G) > cap) --G;
            Gn = gn_of(G);
            // blocks go to the 8 XCDs round robin: the full tiles' pairs fill per = nt G / 8 slots
            // of each XCD (G a multiple of 8), the narrow ranges the rest, so no XCD holds more
            // workgroups than its resident slots (one more would wait for a second round)
            const uint32_t per_xcd = cap / 8;
            if (narrow && cap % 8 == 0) {
                for (uint32_t g8 = (cap / nt) / 8 * 8; g8 >= 8; g8 -= 8) {
                    const uint32_t per = nt * g8 / 8;
                    if (per < per_xcd && 8 * (per_xcd - per) >= gn_of(g8)) {
                        G = g8;
                        Gn = 8 * (per_xcd - per);
                        break;
                    }
                }
            }
        }
        // short inputs: at least min_rows rows per range, so the per-workgroup flush stays small
        // (CBH_FILL_MIN_ROWS, a measurement knob)
        uint64_t min_rows = 2048;
        if (const char* mr = std::getenv("CBH_FILL_MIN_ROWS")) min_rows = std::max<uint64_t>(256, std::strtoull(mr, nullptr, 10));
        while (G > 1 && s->n / G < min_rows) G = G / 2;
        while (Gn > 1 && s->n / Gn < min_rows) Gn = Gn / 2;
        pl.tiles16 = nt;
        pl.ranges = G;
        pl.ranges_n = Gn;
        pl.blocks = 8 * ((nt * G + 7) / 8) + Gn;
        return pl;
    };
    const char* ne = std::getenv("CBH_PACK_NARROW");
    const bool off = ne && std::string(ne) == "off";
    const uint32_t last = s->W % TWM;
    const bool narrow = !off && (exact ? (last == 1 || last == 2) : last == 2);
    s->pk_dense = plan(narrow);
    // (the exact fill's narrow loop at the gathered levels measured 2x slower there: 760 against
    // 360 us per level at config 2, each of its workgroups' few 8-byte gathers waiting on random
    // lines; CBH_PACK_NARROW_GATHER=on takes it, a measurement knob)
    const char* ng = std::getenv("CBH_PACK_NARROW_GATHER");
    s->pk_gath = plan(exact && narrow && ng && std::string(ng) == "on");
    s->pk_ranges = s->pk_gath.ranges;
    const uint64_t rb = 4ull * s->Ws;
    s->pk_rm_sh = 0;
    const char* e = std::getenv("CBH_PACK_GATHER");
    if ((rb & (rb - 1)) == 0 && s->n * rb < (1ull << 32) && !(e && std::string(e) == "tiles"))
        while ((1ull << s->pk_rm_sh) < rb) ++s->pk_rm_sh;
}

// Feature tiles of the fill: the widest LDS slot stride whose histogram fits the budget.
int plan_tiles(cbh_session* s) {
    int lds_max = 0;
    HIP_TRY(hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, s->device));
    size_t budget = std::min<size_t>((size_t)lds_max, 160 * 1024);
    // CBH_FILL_LDS_KB lowers the per-workgroup LDS budget (a tuning knob; the default uses
    // the whole LDS of a CU)
    if (const char* e = std::getenv("CBH_FILL_LDS_KB")) {
        const long kb = std::strtol(e, nullptr, 10);
        if (kb >= 8) budget = std::min<size_t>(budget, (size_t)kb * 1024);
    }
    // bin-major LDS with rotated visits (conflict-free atomics) for >= 4 channels, where the
    // atomics per loaded word dominate (config 5: 31 -> 38 iters/s), and for >= 4M rows
    // (config 2: fill 0.654 -> 0.621 ms per launch); at 1M rows and 2 channels its extra
    // 32-feature tiles cost more than the bank conflicts they remove (config 3: 0.060 ->
    // 0.073 ms).
    // CBH_FILL_LAYOUT=feature|bin forces one layout (a measurement knob)
    const char* lv = std::getenv("CBH_FILL_LAYOUT");
    const std::string lay = lv ? lv : "";
    const int layout = lay == "feature" ? 0 : lay == "bin" ? 2 : 1;
    s->tiles = plan_fill_tiles(s->F, s->B, s->C, budget, layout, s->n);
    if (s->tiles.n_tiles == 0) return fail(CBH_DECLINED, "histogram of 4 features does not fit in LDS");
    // (tile, range) workgroups for one or two rounds of the CUs' resident slots, ranges a
    // multiple of 8: one round when it fills >= 97% of the slots, else the better of the two
    // (config 2: 7 tiles on 256 one-workgroup CUs -> 1 round uses 224 slots, 2 rounds 504 of
    // 512: fill 0.594 -> 0.563 ms per launch; more rounds add flushes and lose)
    int cus = 0;
    HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, s->device));
    const uint32_t per_cu = std::max<uint32_t>(1, (uint32_t)((size_t)lds_max / s->tiles.lds_bytes));
    s->fill_ranges = pick_ranges((uint32_t)cus, std::min<uint32_t>(per_cu, 2), s->tiles.n_tiles, s->n);
    return CBH_OK;
}

template <int C>
int set_pkk_attr(size_t lds) {
    for (const void* k : {(const void*)fill_pkk_kernel<C, false, false>, (const void*)fill_pkk_kernel<C, false, true>,
                          (const void*)fill_pkk_kernel<C, true, false>, (const void*)fill_pkk_kernel<C, true, true>,
                          (const void*)fill_pks_kernel<C, false>, (const void*)fill_pks_kernel<C, true>,
                          (const void*)fill_pks_kernel<C, false, 4, 8>, (const void*)fill_pks_kernel<C, true, 4, 8>})
        HIP_TRY(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    return CBH_OK;
}

// Packed multi-channel fill plan (K > 1): from 500000 rows (CBH_FILL=packed at any size,
// CBH_FILL=exact keeps the two-channel fill) when the NP planes of a 32-feature tile fit the
// per-thread cells (NP * B * 32 <= kPkkCells).
int plan_pkk(cbh_session* s, const std::string& v) {
    const uint32_t NP = (s->C + 1) / 2;
    const bool want = v == "packed" || (v.empty() && s->n >= 500000);
    if (!want || (uint64_t)NP * s->B * 32u > kPkkCells) return CBH_OK;
    int lds_max = 0, cus = 0;
    HIP_TRY(hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, s->device));
    HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, s->device));
    const size_t lds = (size_t)kPkkCells * sizeof(unsigned long long);
    if (lds > (size_t)lds_max) return CBH_OK;
    CHECK(with_k((int)s->K, [&](auto kc) { return set_pkk_attr<decltype(kc)::value + 1>(lds); }));
    s->pkk_tiles = (s->W + 7) / 8;
    s->pkk_ranges = pick_ranges((uint32_t)cus, 1u, s->pkk_tiles, s->n);
    CHECK(dalloc(&s->spack, (size_t)s->n * NP));
    s->pack_bits = kPkkBits;
    s->pkk = true;
    // the score weight alone in the last plane (C odd) and the same every tree (no bootstrap, no
    // per-tree sample from the host): level 0 fills it once (CBH_PKK_W0=off, a measurement knob,
    // fills it every tree)
    const char* w0e = std::getenv("CBH_PKK_W0");
    s->w_static = (s->C & 1u) && s->cfg.bootstrap_type == CBH_BOOT_NO && !s->cfg.sample_from_host &&
                  !(w0e && std::string(w0e) == "off");
    if (s->w_static) CHECK(dalloc(&s->w0_cache, (size_t)s->F * s->B));
    // sparse entries when the dominant-bin skip leaves at most 12 of a tile's 32 entries per row
    // on average (a DPP row of 16 lanes per row then carries about twice the active lanes of the
    // dense visit); CBH_PKK_SPARSE=off keeps the dense visit, =on takes the entries whatever
    // their count (measurement and test knobs)
    const char* se = std::getenv("CBH_PKK_SPARSE");
    const std::string sv = se ? se : "";
    if (s->use_skip && sv != "off" && (sv == "on" || s->nd_per_tile <= 12.0)) {
        const size_t slots = (size_t)s->pkk_tiles * s->n * 16;
        if (dalloc(&s->pks_a, slots) != CBH_OK || dalloc(&s->pks_b, slots) != CBH_OK) {
            // no room for the entries (64 bytes per row and tile): the dense visit needs none
            dfree(s->pks_a);
            dfree(s->pks_b);
            (void)hipGetLastError();
            return CBH_OK;
        }
        pack_sparse_kernel<<<grid_for((uint64_t)s->pkk_tiles * s->n, 256), 256, 0, s->stream>>>(
            s->cols, s->n, s->F, s->pkk_tiles, s->skip_bin, s->pks_a, s->pks_b);
        if (hipGetLastError() != hipSuccess || hipStreamSynchronize(s->stream) != hipSuccess)
            return fail(CBH_ERR_DEVICE, "sparse entry packing failed");
        s->pks = true;
        // tiles of at most 4096 cells (NP * B * 32: config 5's 6 planes of 20 bins) take the
        // 4-cells-per-thread variant (CBH_PKS_SMALL=off, a measurement knob, keeps the general one)
        const char* sm = std::getenv("CBH_PKS_SMALL");
        s->pks_small = (uint64_t)NP * s->B * 32u <= 4u * kPkkThreads && !(sm && std::string(sm) == "off");
    }
    return CBH_OK;
}

// Fill plan.  The default: K == 1 with integer score weights from 2^22 rows the count-packed
// fill, else from 2^16 rows (2^20 with pairs) the tiled exact fill (which visits every bin: its
// lanes add to distinct features, so a dominant bin does not serialize them); K > 1 from 500000
// rows the packed multi-channel fill; otherwise the generic fill.  CBH_FILL (a measurement and
// test knob) forces one: =generic the generic fill (any K), =tiled the tiled exact fill (K == 1),
// =count the count-packed fill (K == 1, integer score weights), =packed the rounded packed fill
// (K == 1: 18-bit rows) or the packed multi-channel fill (K > 1).
int plan_fill_mode(cbh_session* s) {
    s->packed = s->tiled = s->pkk = s->count = false;
    const char* e = std::getenv("CBH_FILL");
    const std::string v = e ? e : "";
    if (s->K > 1) return (v.empty() || v == "packed") ? plan_pkk(s, v) : CBH_OK;
    if (v == "generic") return CBH_OK;
    // integer score weights: no per-row sample beyond Bernoulli's keep mask, integer object
    // weights, no pair weights (they arrive after the plan)
    const bool count_ok = !s->ranking && !s->cfg.sample_from_host && s->int_w &&
                          (s->cfg.bootstrap_type == CBH_BOOT_NO || s->cfg.bootstrap_type == CBH_BOOT_BERNOULLI);
    // (the packed decodes take non-negative weights: a negative object weight keeps the other fills)
    const bool want_packed = v == "packed" && !s->pk_signed_w;
    // defaults by measurement: the count-packed fill from 4M rows (config 2's data under Bernoulli:
    // 380 against 324 iters/s for the tiled exact fill); below, its per-workgroup swaps and
    // register flush outweigh the halved atomics (config 4 at 2M rows: 861 against 953 iters/s,
    // config 1: 2578 against 2616), so the tiled exact fill takes over from 64k rows (config 1:
    // 2616 against 2234 iters/s for the generic fill) -- from 2^20 rows with pair weights, whose
    // sessions below that ran faster on the generic fill (config 3 at 1M rows: 1419 against 1311)
    const bool want_count = !want_packed && count_ok && (v == "count" || (v.empty() && s->n >= (1ull << 22)));
    const bool want_tiled = !want_packed && !want_count &&
                            (v == "tiled" || v == "count" ||
                             (v.empty() && s->n >= (s->ranking ? (1ull << 20) : (1ull << 16))));
    if (!want_packed && !want_count && !want_tiled) return CBH_OK;
    // the tiled fills address their buffers (a tile's row words, statistics) by 32-bit byte
    // offsets and read the dense level's rows in groups of 16 clamped to [0, n)
    const bool pk64 = want_packed || want_count;   // the 64-feature loops
    const uint32_t TWM = pk64 ? kPackTileWords : kExTileWords;
    if ((uint64_t)s->n * TWM * 4u >= (1ull << 31) || s->n < 1024) return CBH_OK;
    int lds_max = 0, cus = 0, per_cu = 0;
    HIP_TRY(hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, s->device));
    HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, s->device));
    // every thread owns the same cells of a 256-bin tile whatever B
    const size_t lds = (size_t)(pk64 ? kPackCells : kExCells) * sizeof(unsigned long long);
    if (lds > (size_t)lds_max) return CBH_OK;
    const void* kg = want_packed  ? (const void*)fill_packed_kernel<true, false>
                     : want_count ? (const void*)fill_packed_kernel<true, true>
                                  : (const void*)fill_exact_kernel<true>;
    const void* kd = want_packed  ? (const void*)fill_packed_kernel<false, false>
                     : want_count ? (const void*)fill_packed_kernel<false, true>
                                  : (const void*)fill_exact_kernel<false>;
    for (const void* k : {kg, kd})
        HIP_TRY(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kg, (int)kPackThreads, lds));
    if (per_cu < 1) return CBH_OK;
    s->pk_lds = lds;
    s->pk_tiles = (s->W + TWM - 1) / TWM;
    pick_tile_ranges(s, (uint32_t)cus, (uint32_t)per_cu, TWM);
    if (want_packed) {
        // CBH_PACK_SWAP (1, 2, 4, 8): blocks of rows between two swaps; each doubling costs
        // one bit of a row's rounded value (a measurement knob).  Default 4: 18-bit rows (rows
        // clamped to 2^18 - 1, so 8192 of them stay below 2^31), a quarter of the swap work of 1
        s->pk_swap = 4;
        if (const char* sw = std::getenv("CBH_PACK_SWAP")) {
            const long v2 = std::strtol(sw, nullptr, 10);
            if (v2 == 1 || v2 == 2 || v2 == 4 || v2 == 8) s->pk_swap = (uint32_t)v2;
        }
        s->pack_bits = kPackBitsSwap1 - (s->pk_swap >= 2) - (s->pk_swap >= 4) - (s->pk_swap >= 8);
    }
    if (pk64) CHECK(dalloc(&s->spack, (size_t)s->n));
    // the listed rows' statistics in idx order (packed: one word per row; tiled: both channels;
    // CBH_EX_STATS=idx, a measurement knob, has the tiled fill read them through the listed rows'
    // indices instead: gathered levels 360 -> 400-650 us at config 2).  CBH_EX_SETS=2..4: blocks
    // in flight in the tiled fill's full loop (a measurement knob; three instead of two took
    // config 2's fill from 443 to 436 us per launch)
    const char* es = std::getenv("CBH_EX_STATS");
    if (pk64 || !(es && std::string(es) == "idx")) CHECK(dalloc(&s->sseq, (size_t)s->n * (pk64 ? 1u : 2u)));
    if (const char* ns = std::getenv("CBH_EX_SETS")) {
        const long v2 = std::strtol(ns, nullptr, 10);
        if (v2 >= 2 && v2 <= 4) s->ex_sets = (uint32_t)v2;
    }
    // tile-major row words: each tile's rows contiguous (the row-major words stay for the
    // gathered levels and the other fills)
    const uint32_t tw_last = s->W - TWM * (s->pk_tiles - 1);
    const uint64_t words = (uint64_t)s->n * (TWM * (s->pk_tiles - 1) + packed_slice_words(tw_last));
    CHECK(dalloc(&s->trows, words));
    pack_tiles_kernel<<<grid_for(words, 256), 256, 0, s->stream>>>(s->cols, s->n, s->F, s->W, s->trows, words, TWM);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(s->stream) != hipSuccess)
        return fail(CBH_ERR_DEVICE, "tile-major packing failed");
    s->packed = want_packed;
    s->count = want_count;
    s->tiled = want_tiled;
    // the tiled fills visit every bin: the 16 lanes of a DPP row add to 16 distinct features, so
    // rows crowding one bin never meet on one cell within the lanes an atomic's conflicts count
    // over (the generic fill leaves such bins out instead, rebuilding them from the totals)
    s->use_skip = false;
    s->n_skip = 0;
    return CBH_OK;
}

template <int C>
int set_fill_attr(size_t lds) {
    HIP_TRY(hipFuncSetAttribute((const void*)fill_kernel<C, false>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    HIP_TRY(hipFuncSetAttribute((const void*)fill_kernel<C, true>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    if constexpr (C == 2)   // the der-only fill of PairLogitPairwise sessions
        HIP_TRY(hipFuncSetAttribute((const void*)fill_kernel<2, false, 1>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    return CBH_OK;
}

// Dominant bins: a device census of every column, then per feature the most frequent bin
// if it holds at least 1/8 of the rows (the fill leaves it out and rebuilds it exactly).
int plan_skip_bins(cbh_session* s) {
    unsigned long long* cnt = nullptr;
    CHECK(dalloc(&cnt, (size_t)s->F * 256));
    std::vector<unsigned long long> h((size_t)s->F * 256);
    int rc = CBH_OK;
    do {
        zero_i64_kernel<<<grid_for((size_t)s->F * 256, 256, 8192), 256, 0, s->stream>>>((long long*)cnt,
                                                                                       (size_t)s->F * 256);
        if (hipGetLastError() != hipSuccess) { rc = fail(CBH_ERR_DEVICE, "census zero launch failed"); break; }
        // about 4 blocks per CU over all features, chunks of at least 64 KiB
        const uint64_t want = std::max<uint64_t>(1, 1024 / std::max<uint32_t>(s->F, 1));
        const uint64_t chunk = std::max<uint64_t>(65536, ((s->n + want - 1) / want + 15) & ~15ull);
        const uint64_t gx = (s->n + chunk - 1) / chunk;
        bin_census_kernel<<<dim3((unsigned)std::max<uint64_t>(gx, 1), s->F), 256, 0, s->stream>>>(s->cols, s->n,
                                                                                              chunk, cnt);
        if (hipGetLastError() != hipSuccess) { rc = fail(CBH_ERR_DEVICE, "census launch failed"); break; }
        if (hipMemcpyAsync(h.data(), cnt, sizeof(unsigned long long) * h.size(), hipMemcpyDeviceToHost,
                           s->stream) != hipSuccess ||
            hipStreamSynchronize(s->stream) != hipSuccess) {
            rc = fail(CBH_ERR_DEVICE, "census copy failed");
            break;
        }
    } while (false);
    dfree(cnt);
    if (rc != CBH_OK) return rc;
    std::vector<uint32_t> skip(s->F, 256u);
    bool any = false;
    for (uint32_t f = 0; f < s->F; ++f) {
        const unsigned long long* c = h.data() + (size_t)f * 256;
        uint32_t best = 0;
        for (uint32_t b = 1; b < s->B; ++b)
            if (c[b] > c[best]) best = b;
        if (c[best] * 8 >= s->n) {
            skip[f] = best;
            any = true;
        }
    }
    s->use_skip = any;
    s->n_skip = 0;
    for (uint32_t v : skip) s->n_skip += v < 256u;
    {   // mean entries a row keeps per 32-feature tile once dominant bins are left out
        double kept = 0.0;
        for (uint32_t f = 0; f < s->F; ++f)
            kept += skip[f] < 256u ? 1.0 - (double)h[(size_t)f * 256 + skip[f]] / (double)s->n : 1.0;
        s->nd_per_tile = kept / (double)((s->F + 31) / 32);
    }
    if (!any) return CBH_OK;
    CHECK(dalloc(&s->skip_bin, s->F));
    CHECK(dalloc(&s->seg_tot, (size_t)(kMaxLeaves / 2) * s->C));
    HIP_TRY(hipMemcpy(s->skip_bin, skip.data(), sizeof(uint32_t) * s->F, hipMemcpyHostToDevice));
    return CBH_OK;
}

template <typename Load>
int session_open(const cbh_config* cfg, const double* weight, uint64_t n, uint32_t F, uint32_t n_bins,
                 double lr, double l2, cbh_session** out, Load&& load_cols);

// ---- device CTR config at open (DeviceTrainConfig.ctr) ----
struct CtrOpen {
    uint32_t m = 0;                      // CTR columns appended after the base features
    std::vector<uint8_t> one_hot;        // base flags extended with zeros
    std::vector<uint32_t> folds;         // base folds extended with n_borders + 1
    std::vector<uint64_t> nb_struct, nb_avg;   // bucket scratch sizes (largest code + 1)
    std::vector<uint32_t> bucket_count, group;
    std::vector<uint32_t> cat_nb;
};

bool ctr_type_covered(int32_t t) {
    return t == CBH_CTR_BORDERS || t == CBH_CTR_BUCKETS || t == CBH_CTR_BTMV || t == CBH_CTR_COUNTER;
}

// Admission (ctr_covered, gpu_runtime/session.rs:177-215) and host validation of the
// inputs the device build reads.  Fills the extended one-hot flags / folds of the session.
int admit_device_ctr(const cbh_config* cfg, uint64_t n, uint32_t F, uint32_t n_bins, CtrOpen& co) {
    const cbh_device_ctr_config* c = cfg->ctr;
    if (cfg->loss == CBH_LOSS_PAIRLOGIT || cfg->loss == CBH_LOSS_PAIRLOGIT_PAIRWISE)
        return fail(CBH_DECLINED, "CTR columns are not covered with pair losses");
    const cbh_device_ctr_averaging* a = c->averaging;
    if (!a) return fail(CBH_DECLINED, "a CTR config without its averaging half is not covered");
    if (c->n_columns == 0) return fail(CBH_DECLINED, "a CTR config without columns is not covered");
    if (a->n_columns != c->n_columns)
        return fail(CBH_DECLINED, "the averaging half has another column count than the structure half");
    if (!c->permutation || !c->target_class || !c->columns || !a->permutation || !a->target_class || !a->columns)
        return fail(CBH_ERR_INVALID_ARG, "null CTR array");
    if (n >= (1ull << 31)) return fail(CBH_DECLINED, "device CTR columns cover fewer than 2^31 objects");
    if ((uint64_t)F + c->n_columns > (1u << 20)) return fail(CBH_ERR_OUT_OF_RANGE, "too many CTR columns");
    const uint32_t m = c->n_columns;
    // largest code and distinct count of every member column, once per column pointer
    std::vector<std::pair<const uint32_t*, std::pair<uint64_t, uint64_t>>> seen;
    auto census = [&](const uint32_t* col) -> std::pair<uint64_t, uint64_t> {
        for (auto& e : seen)
            if (e.first == col) return e.second;
        uint32_t mx = 0;
        for (uint64_t i = 0; i < n; ++i) mx = std::max(mx, col[i]);
        std::vector<uint8_t> hit((size_t)mx + 1, 0);
        uint64_t d = 0;
        for (uint64_t i = 0; i < n; ++i) {
            d += hit[col[i]] ? 0 : 1;
            hit[col[i]] = 1;
        }
        seen.push_back({col, {(uint64_t)mx + 1, d}});
        return seen.back().second;
    };
    auto check_half = [&](const cbh_device_ctr_column* cols, std::vector<uint64_t>& nb) -> int {
        nb.assign(m, 1);
        for (uint32_t k = 0; k < m; ++k) {
            const cbh_device_ctr_column& col = cols[k];
            if (!ctr_type_covered(col.ctr_type))
                return fail(CBH_DECLINED, "CTR type " + std::to_string(col.ctr_type) + " is not covered on device");
            if (col.n_members == 0) return fail(CBH_DECLINED, "a CTR column without members is not covered");
            if (col.n_members >= 2)
                return fail(CBH_DECLINED, "combination (multi-member) CTR projections are not covered on device");
            if (col.n_borders == 0 || col.n_borders + 1 > n_bins)
                return fail(CBH_DECLINED, "a CTR border table needs 1 .. n_bins - 1 borders");
            if (!col.member_bins || !col.member_bins[0] || !col.borders)
                return fail(CBH_ERR_INVALID_ARG, "null CTR column array");
            if ((col.ctr_type == CBH_CTR_BORDERS || col.ctr_type == CBH_CTR_BUCKETS) && col.target_border_idx > 1)
                return fail(CBH_ERR_OUT_OF_RANGE, "CTR target_border_idx > 1 (binary classes)");
            if (col.weight_group >= m) return fail(CBH_ERR_OUT_OF_RANGE, "CTR weight_group >= n_columns");
            nb[k] = census(col.member_bins[0]).first;
        }
        return CBH_OK;
    };
    CHECK(check_half(c->columns, co.nb_struct));
    CHECK(check_half(a->columns, co.nb_avg));
    for (const uint32_t* perm : {c->permutation, a->permutation}) {
        std::vector<uint8_t> hit(n, 0);
        for (uint64_t p = 0; p < n; ++p) {
            if (perm[p] >= n || hit[perm[p]])
                return fail(CBH_ERR_OUT_OF_RANGE, "a CTR permutation is not a permutation of 0..n-1");
            hit[perm[p]] = 1;
        }
    }
    for (const uint32_t* cls : {c->target_class, a->target_class})
        for (uint64_t i = 0; i < n; ++i)
            if (cls[i] > 1) return fail(CBH_ERR_OUT_OF_RANGE, "CTR target_class must be 0 or 1");
    co.m = m;
    co.bucket_count.resize(m);
    co.group.resize(m);
    for (uint32_t k = 0; k < m; ++k) {
        const cbh_device_ctr_column& col = c->columns[k];
        // 0 = unknown: the column's own observed distinct-bucket count (runtime.rs:1116-1122)
        const uint64_t bc = col.bucket_count ? col.bucket_count : census(col.member_bins[0]).second;
        if (bc > 0xFFFFFFFFull) return fail(CBH_ERR_OUT_OF_RANGE, "CTR bucket_count does not fit u32");
        co.bucket_count[k] = (uint32_t)bc;
        co.group[k] = col.weight_group;
    }
    if (c->n_cat && !c->cat_eligible_buckets) return fail(CBH_ERR_INVALID_ARG, "null cat_eligible_buckets");
    co.cat_nb.resize(c->n_cat);
    for (uint32_t j = 0; j < c->n_cat; ++j) {
        if (!c->cat_eligible_buckets[j]) return fail(CBH_ERR_INVALID_ARG, "null categorical bucket column");
        co.cat_nb[j] = (uint32_t)std::min<uint64_t>(census(c->cat_eligible_buckets[j]).first, 0xFFFFFFFFull);
    }
    if (cfg->one_hot_flags) {
        co.one_hot.assign(cfg->one_hot_flags, cfg->one_hot_flags + F);
        co.one_hot.resize((size_t)F + m, 0);
    }
    co.folds.resize((size_t)F + m);
    for (uint32_t f = 0; f < F; ++f) co.folds[f] = cfg->real_folds ? cfg->real_folds[f] : n_bins;
    for (uint32_t k = 0; k < m; ++k) co.folds[F + k] = c->columns[k].n_borders + 1;
    return CBH_OK;
}

// Both materializations on the device: the structure columns into the session's
// feature-major bins after the F base features, the averaging columns into ctr_avg.
int build_device_ctr(cbh_session* s, uint32_t F, const cbh_device_ctr_config* c, const CtrOpen& co) {
    CHECK(cbh_internal_ctr_bins(c->columns, co.m, co.nb_struct.data(), c->permutation, c->target_class, s->n,
                                s->cols + (size_t)F * s->n, s->stream));
    CHECK(dalloc(&s->ctr_avg, (size_t)co.m * s->n));
    const cbh_device_ctr_averaging* a = c->averaging;
    CHECK(cbh_internal_ctr_bins(a->columns, co.m, co.nb_avg.data(), a->permutation, a->target_class, s->n,
                                s->ctr_avg, s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    return CBH_OK;
}

int install_ctr(cbh_session* s, uint32_t m, const uint32_t* bucket_count, const uint32_t* weight_group,
                uint32_t n_cat, const uint32_t* const* cat_cols, const uint32_t* cat_bucket_count, double msr);

// Open with the device CTR config, if any: admission, the extended session shape, the
// device build inside the load step and the scoring state once the session exists.
template <typename Open>
int open_with_ctr(const cbh_config* cfg, uint64_t n, uint32_t F, uint32_t n_bins, cbh_session** out, Open&& open) {
    if (!cfg->ctr) return open(cfg, F, [](cbh_session*) { return CBH_OK; });
    CtrOpen co;
    CHECK(admit_device_ctr(cfg, n, F, n_bins, co));
    cbh_config c2 = *cfg;
    c2.one_hot_flags = co.one_hot.empty() ? nullptr : co.one_hot.data();
    c2.real_folds = co.folds.data();
    const cbh_device_ctr_config* c = cfg->ctr;
    CHECK(open(&c2, F + co.m, [&](cbh_session* s) { return build_device_ctr(s, F, c, co); }));
    const int rc = install_ctr(*out, co.m, co.bucket_count.data(), co.group.data(), c->n_cat,
                               c->cat_eligible_buckets, co.cat_nb.data(), c->model_size_reg);
    if (rc != CBH_OK) {
        (void)cbh_session_end(*out);
        *out = nullptr;
    }
    return rc;
}

template <typename BinT>
int session_begin_impl(const cbh_config* cfg, const BinT* bins_fm, const double* weight,
                       uint64_t n, uint32_t F, uint32_t n_bins, double lr, double l2,
                       cbh_session** out) {
    if (!out) return fail(CBH_ERR_INVALID_ARG, "out is null");
    *out = nullptr;
    CHECK(validate_config(cfg, n_bins, n, F));
    if (!bins_fm) return fail(CBH_ERR_INVALID_ARG, "bins_fm is null");
    // validate bins (the reference surfaces an out-of-range bin as a typed error)
    for (uint64_t i = 0, total = n * F; i < total; ++i)
        if ((uint32_t)bins_fm[i] >= n_bins)
            return fail(CBH_ERR_OUT_OF_RANGE, "bin value >= n_bins at flat index " + std::to_string(i));
    // upload bins feature-major as u8 (the rows are packed from them on the device)
    return open_with_ctr(cfg, n, F, n_bins, out, [&](const cbh_config* c, uint32_t F_all, auto&& ctr_build) {
        return session_open(c, weight, n, F_all, n_bins, lr, l2, out, [&](cbh_session* s) -> int {
            if (sizeof(BinT) == 1) {
                HIP_TRY(hipMemcpy(s->cols, bins_fm, (size_t)n * F, hipMemcpyHostToDevice));
            } else {
                std::vector<uint8_t> tmp;
                const uint64_t step = 1ull << 26;
                for (uint64_t off = 0, total = n * F; off < total; off += step) {
                    const uint64_t m = std::min(step, total - off);
                    tmp.resize(m);
                    for (uint64_t i = 0; i < m; ++i) tmp[i] = (uint8_t)bins_fm[off + i];
                    HIP_TRY(hipMemcpy(s->cols + off, tmp.data(), m, hipMemcpyHostToDevice));
                }
            }
            return ctr_build(s);
        });
    });
}

// Raw float channel: every column is staged on the device and quantized there into the
// session's feature-major bins (one quantize launch per column on the session stream).
int session_begin_raw_impl(const cbh_config* cfg, const float* const* columns, const double* const* borders,
                           const uint32_t* n_borders, const double* weight, uint64_t n, uint32_t F,
                           uint32_t n_bins, double lr, double l2, cbh_session** out) {
    if (!out) return fail(CBH_ERR_INVALID_ARG, "out is null");
    *out = nullptr;
    CHECK(validate_config(cfg, n_bins, n, F));
    if (!columns || !borders || !n_borders) return fail(CBH_ERR_INVALID_ARG, "columns / borders / n_borders is null");
    if (cfg->one_hot_flags)
        for (uint32_t f = 0; f < F; ++f)
            if (cfg->one_hot_flags[f]) return fail(CBH_ERR_UNSUPPORTED, "the raw float channel carries no one-hot columns");
    std::vector<uint64_t> off(F + 1, 0);
    for (uint32_t f = 0; f < F; ++f) {
        if (n && !columns[f]) return fail(CBH_ERR_INVALID_ARG, "column " + std::to_string(f) + " is null");
        if (n_borders[f] && !borders[f]) return fail(CBH_ERR_INVALID_ARG, "borders of feature " + std::to_string(f) + " are null");
        if (n_borders[f] + 1 > n_bins)
            return fail(CBH_ERR_OUT_OF_RANGE, "feature " + std::to_string(f) + " has more borders than n_bins - 1");
        for (uint32_t k = 1; k < n_borders[f]; ++k)
            if (!(borders[f][k - 1] < borders[f][k]))
                return fail(CBH_ERR_OUT_OF_RANGE, "borders of feature " + std::to_string(f) + " do not ascend");
        off[f + 1] = off[f] + n_borders[f];
    }
    // candidate folds follow the borders (real_folds = borders + 1, boosting.rs:4334-4372)
    // unless the caller gives them
    std::vector<uint32_t> folds(F);
    for (uint32_t f = 0; f < F; ++f) folds[f] = n_borders[f] + 1;
    cbh_config c = *cfg;
    if (!c.real_folds) c.real_folds = folds.data();
    return open_with_ctr(&c, n, F, n_bins, out, [&](const cbh_config* c2, uint32_t F_all, auto&& ctr_build) {
      return session_open(c2, weight, n, F_all, n_bins, lr, l2, out, [&](cbh_session* s) -> int {
        if (n == 0 || F == 0) return CBH_OK;
        std::vector<double> flat(std::max<uint64_t>(off[F], 1));
        for (uint32_t f = 0; f < F; ++f)
            if (n_borders[f]) std::memcpy(flat.data() + off[f], borders[f], sizeof(double) * n_borders[f]);
        double* db = nullptr;
        float* stage = nullptr;
        int rc = CBH_OK;
        if (hipMalloc((void**)&db, sizeof(double) * flat.size()) != hipSuccess ||
            hipMalloc((void**)&stage, sizeof(float) * n) != hipSuccess) {
            rc = fail(CBH_ERR_DEVICE, "staging allocation failed");
        }
        if (rc == CBH_OK && hipMemcpy(db, flat.data(), sizeof(double) * flat.size(), hipMemcpyHostToDevice) != hipSuccess)
            rc = fail(CBH_ERR_DEVICE, "border upload failed");
        // with profiling, every quantize launch is bracketed by its own event pair
        std::vector<hipEvent_t> ev(s->cfg.profile ? 2 * (size_t)F : 0, nullptr);
        for (auto& e : ev)
            if (rc == CBH_OK && hipEventCreate(&e) != hipSuccess) rc = fail(CBH_ERR_DEVICE, "event creation failed");
        for (uint32_t f = 0; rc == CBH_OK && f < F; ++f) {
            if (hipMemcpyAsync(stage, columns[f], sizeof(float) * n, hipMemcpyHostToDevice, s->stream) != hipSuccess) {
                rc = fail(CBH_ERR_DEVICE, "column upload failed");
                break;
            }
            if (!ev.empty()) (void)hipEventRecord(ev[2 * f], s->stream);
            rc = cbh_internal_quantize(stage, n, db + off[f], n_borders[f], s->cols + (size_t)f * n, s->stream);
            if (!ev.empty()) (void)hipEventRecord(ev[2 * f + 1], s->stream);
        }
        if (hipStreamSynchronize(s->stream) != hipSuccess && rc == CBH_OK) rc = fail(CBH_ERR_DEVICE, "quantize failed");
        for (uint32_t f = 0; rc == CBH_OK && !ev.empty() && f < F; ++f) {
            float ms = 0.f;
            if (hipEventElapsedTime(&ms, ev[2 * f], ev[2 * f + 1]) == hipSuccess) {
                s->stats.quantize_ms += ms;
                s->stats.quantize_launches += 1;
                s->stats.quantize_bytes += 5.0 * (double)n + 8.0 * n_borders[f];
            }
        }
        for (auto& e : ev)
            if (e) (void)hipEventDestroy(e);
        if (db) (void)hipFree(db);
        if (stage) (void)hipFree(stage);
        if (rc != CBH_OK) return rc;
        return ctr_build(s);
      });
    });
}

template <typename Load>
int session_open(const cbh_config* cfg, const double* weight, uint64_t n, uint32_t F, uint32_t n_bins,
                 double lr, double l2, cbh_session** out, Load&& load_cols) {
    std::unique_ptr<cbh_session> s(new cbh_session());
    s->cfg = *cfg;
    if (cfg->one_hot_flags) s->one_hot_host.assign(cfg->one_hot_flags, cfg->one_hot_flags + F);
    s->cfg.one_hot_flags = nullptr;
    s->cfg.real_folds = nullptr;
    s->cfg.ctr = nullptr;
    s->n = n;
    s->F = F;
    s->B = n_bins;
    s->W = (F + 3) / 4;
    // packed rows padded to a multiple of 16 words (64 bytes): a feature tile's 32-byte run
    // of a row never straddles a 64-byte sector and a row spans whole 128-byte lines, which
    // the fill's gathers through the partitioned index list fetch (config 2: fill 0.559 ->
    // 0.531 ms per launch; configs 1, 3, 4 unchanged).  CBH_ROW_ALIGN_WORDS sets another
    // multiple, rounded up to 8 words (a measurement knob): the multi-channel fills read a
    // row's words in whole 8-word tiles, which must stay inside the row
    uint32_t align = 16;
    if (const char* e = std::getenv("CBH_ROW_ALIGN_WORDS")) {
        const long a = std::strtol(e, nullptr, 10);
        if (a >= 1 && a <= 64) align = (uint32_t)((a + 7) / 8 * 8);
    }
    s->Ws = (s->W + align - 1) / align * align;
    s->K = (uint32_t)cfg->approx_dim;
    s->C = s->K + 1;
    s->depth = (uint32_t)cfg->depth;
    s->lr = lr;
    s->l2 = l2;
    s->has_weight = weight != nullptr;
    s->ranking = cfg->loss == CBH_LOSS_PAIRLOGIT || cfg->loss == CBH_LOSS_PAIRLOGIT_PAIRWISE;
    s->pairwise = cfg->loss == CBH_LOSS_PAIRLOGIT_PAIRWISE;
    s->prior = cfg->pairwise_non_diag_reg;
    if (s->ranking && weight)
        return fail(CBH_ERR_UNSUPPORTED, "pair losses take their weights from the pairs, not per object");
    if (s->ranking && cfg->one_hot_flags)
        for (uint32_t f = 0; f < F; ++f)
            if (cfg->one_hot_flags[f])
                return fail(CBH_ERR_UNSUPPORTED, "one-hot columns are not covered with pair losses");
    HIP_TRY(hipGetDevice(&s->device));
    HIP_TRY(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking));
    CHECK(session_alloc(s.get()));
    CHECK(plan_tiles(s.get()));
    {
        int cus = 0;
        HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, s->device));
        s->cus = (uint32_t)std::max(cus, 1);
    }
    CHECK(with_k((int)s->K, [&](auto kc) {
        constexpr int K = decltype(kc)::value;
        CHECK(set_fill_attr<K + 1>(s->tiles.lds_bytes));
        const size_t lds = ((size_t)1 << s->depth) * (size_t)leaf_cells<K>() * sizeof(long long);
        HIP_TRY(hipFuncSetAttribute((const void*)leaf_reduce_kernel<K>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        return CBH_OK;
    }));
    // candidates per feature: float -> real_folds-1 borders; one-hot -> real_folds values
    std::vector<uint32_t> nc(F);
    for (uint32_t f = 0; f < F; ++f) {
        const uint32_t folds = cfg->real_folds ? cfg->real_folds[f] : n_bins;
        if (folds > n_bins) return fail(CBH_ERR_OUT_OF_RANGE, "real_folds[f] > n_bins");
        const bool oh = !s->one_hot_host.empty() && s->one_hot_host[f];
        nc[f] = oh ? folds : (folds > 0 ? folds - 1 : 0);
        s->max_cand = std::max(s->max_cand, nc[f]);
    }
    HIP_TRY(hipMemcpy(s->n_cand, nc.data(), sizeof(uint32_t) * F, hipMemcpyHostToDevice));
    if (const char* e = std::getenv("CBH_SCORE_CHAIN")) s->score_chain = std::string(e) != "off";
    // CBH_CHAIN_SPIN (a test knob): the polls a chained scorer wave takes before it gives up its
    // wait for its turn (0: without polling), so the error path runs with every kernel exiting
    if (const char* e = std::getenv("CBH_CHAIN_SPIN")) s->chain_spin = (uint32_t)std::strtoul(e, nullptr, 10);
    // CBH_CHAIN_FEATURES (a measurement and test knob): cap on the features per chained-scorer workgroup
    if (const char* e = std::getenv("CBH_CHAIN_FEATURES")) s->chain_nf = (uint32_t)std::strtoul(e, nullptr, 10);
    bool any_oh = false;
    for (uint8_t v : s->one_hot_host) any_oh |= v != 0;
    if (any_oh) {
        CHECK(dalloc(&s->one_hot, F));
        HIP_TRY(hipMemcpy(s->one_hot, s->one_hot_host.data(), F, hipMemcpyHostToDevice));
    }
    // feature-major u8 bins in place, then pack the row-major words on the device
    CHECK(load_cols(s.get()));
    pack_rows_kernel<<<grid_for((uint64_t)n * s->Ws, 256), 256, 0, s->stream>>>(s->cols, n, F, s->Ws, s->rows);
    HIP_TRY(hipGetLastError());
    CHECK(plan_skip_bins(s.get()));
    if (weight) {
        HIP_TRY(hipMemcpy(s->weight, weight, sizeof(double) * n, hipMemcpyHostToDevice));
        for (uint64_t i = 0; i < n && !s->pk_signed_w; ++i) s->pk_signed_w = weight[i] < 0.0;
        for (uint64_t i = 0; i < n && s->int_w; ++i)
            s->int_w = weight[i] >= 0.0 && weight[i] <= 1048576.0 && weight[i] == std::floor(weight[i]);
    }
    CHECK(plan_fill_mode(s.get()));
    // resident approximant seeded with the bias (DeviceTrainConfig::bias, runtime.rs:1276)
    std::vector<double> a0(std::min<uint64_t>(n * s->K, 1ull << 22), cfg->bias);
    for (uint64_t off = 0, total = n * s->K; off < total; off += a0.size()) {
        const uint64_t m = std::min<uint64_t>(a0.size(), total - off);
        HIP_TRY(hipMemcpyAsync(s->approx + off, a0.data(), sizeof(double) * m, hipMemcpyHostToDevice, s->stream));
        HIP_TRY(hipStreamSynchronize(s->stream));
    }
    HIP_TRY(hipStreamSynchronize(s->stream));
    *out = s.release();
    return CBH_OK;
}

int launch_zero(long long* p, size_t n, hipStream_t st) {
    zero_i64_kernel<<<grid_for(n, 256, 8192), 256, 0, st>>>(p, n);
    HIP_TRY(hipGetLastError());
    return CBH_OK;
}

// Pairs of a pair loss (FamilyTreeArgs::Pairwise, runtime.rs:925-934): validated, put in the
// reference's competitor order (stable by winner, query_info.rs:205-250), pairwise weights per
// row in pair order (calc_pairwise_weights, boosting.rs:1760-1783), pair weights in fixed
// point 2^shift with 2^shift * sum|w| <= 2^60 (every statistic and weight-matrix entry is a
// sum of at most 4 sum|w|), uploaded once.
void drop_tree_graphs(cbh_session* s) {
    for (auto& g : s->tree_graph)
        if (g) (void)hipGraphExecDestroy(g);
    s->tree_graph[0] = s->tree_graph[1] = nullptr;
}

int upload_pairs(cbh_session* s, const cbh_family* fam) {
    const uint64_t n = s->n;
    if (fam->kind != CBH_FAMILY_PAIRWISE) return fail(CBH_ERR_INVALID_ARG, "family kind is not CBH_FAMILY_PAIRWISE");
    if (!fam->group_offsets || fam->n_groups == 0) return fail(CBH_ERR_INVALID_ARG, "group_offsets are missing");
    const uint32_t G = fam->n_groups;
    const uint32_t* go = fam->group_offsets;
    if (go[0] != 0 || go[G] != n) return fail(CBH_ERR_LENGTH_MISMATCH, "group_offsets must run from 0 to n");
    for (uint32_t g = 0; g < G; ++g)
        if (go[g + 1] < go[g]) return fail(CBH_ERR_OUT_OF_RANGE, "group_offsets decrease at group " + std::to_string(g));
    const uint64_t m = fam->n_pairs;
    if (m >= (1ull << 32)) return fail(CBH_ERR_UNSUPPORTED, "more than 2^32-1 pairs");
    if (m && (!fam->pair_winner || !fam->pair_loser)) return fail(CBH_ERR_INVALID_ARG, "pair arrays are null");
    std::vector<uint32_t> grp(n);
    for (uint32_t g = 0; g < G; ++g)
        for (uint32_t i = go[g]; i < go[g + 1]; ++i) grp[i] = g;
    for (uint64_t k = 0; k < m; ++k) {
        const uint32_t w = fam->pair_winner[k], l = fam->pair_loser[k];
        if (w >= n || l >= n || grp[w] != grp[l])
            return fail(CBH_ERR_OUT_OF_RANGE, "pair " + std::to_string(k) + " is out of range or crosses query groups");
        if (fam->pair_weight && !std::isfinite(fam->pair_weight[k]))
            return fail(CBH_ERR_OUT_OF_RANGE, "pair weight " + std::to_string(k) + " is not finite");
    }
    std::vector<uint32_t> off(n + 1, 0);
    for (uint64_t k = 0; k < m; ++k) off[fam->pair_winner[k] + 1]++;
    for (uint64_t i = 0; i < n; ++i) off[i + 1] += off[i];
    std::vector<uint32_t> pos(off.begin(), off.end() - 1), win(m), los(m);
    std::vector<double> w(m);
    for (uint64_t k = 0; k < m; ++k) {
        const uint32_t j = pos[fam->pair_winner[k]]++;
        win[j] = fam->pair_winner[k];
        los[j] = fam->pair_loser[k];
        w[j] = fam->pair_weight ? fam->pair_weight[k] : 1.0;
    }
    std::vector<double> pw(n, 0.0);
    double sum_abs = 0.0;
    bool neg = false;
    for (uint64_t j = 0; j < m; ++j) {
        pw[win[j]] += w[j];
        pw[los[j]] += w[j];
        sum_abs += std::fabs(w[j]);
        neg |= w[j] < 0.0;
    }
    if (neg && s->packed) {   // the packed fill takes non-negative weights only: back to the two-channel fill
        s->packed = false;
        s->pk_signed_w = true;
        drop_tree_graphs(s);
    }
    int e = 0;
    if (sum_abs > 0.0) std::frexp(sum_abs, &e);
    const int shift = std::min(60 - e, 100);
    std::vector<long long> wq(m);
    for (uint64_t j = 0; j < m; ++j) wq[j] = std::llrint(std::ldexp(w[j], shift));
    // the pairs of each row as a loser, ascending in competitor order (a stable counting sort)
    std::vector<uint32_t> loff(n + 1, 0), lidx(m);
    for (uint64_t j = 0; j < m; ++j) loff[los[j] + 1]++;
    for (uint64_t i = 0; i < n; ++i) loff[i + 1] += loff[i];
    {
        std::vector<uint32_t> lpos(loff.begin(), loff.end() - 1);
        for (uint64_t j = 0; j < m; ++j) lidx[lpos[los[j]]++] = (uint32_t)j;
    }
    // a recorded tree holds the pair count, the group count, the weight scale and the pair
    // buffers: a change of any of them records it again
    if (m != s->n_pairs || G != s->n_groups || std::ldexp(1.0, -shift) != s->pair_inv) drop_tree_graphs(s);
    s->pair_inv = std::ldexp(1.0, -shift);
    if (m != s->n_pairs || !s->comp_win) {
        dfree(s->comp_win); dfree(s->comp_los); dfree(s->comp_w); dfree(s->comp_wq); dfree(s->los_idx);
        dfree(s->key_rec); dfree(s->key_wq); dfree(s->pair_desc); dfree(s->pair_mk);
        CHECK(dalloc(&s->comp_win, m));
        CHECK(dalloc(&s->comp_los, m));
        CHECK(dalloc(&s->comp_w, m));
        CHECK(dalloc(&s->comp_wq, m));
        CHECK(dalloc(&s->los_idx, m));
        if (s->pairwise) {   // keyed records, and the chunk plans of the deepest level
            const uint64_t pmax = 1ull << (s->depth - 1), n_tri = pmax * (pmax + 1) / 2;
            CHECK(dalloc(&s->key_rec, m));
            CHECK(dalloc(&s->key_wq, m));
            CHECK(dalloc(&s->pair_desc, n_tri + (m + kStatChunkMin - 1) / kStatChunkMin));
            CHECK(dalloc(&s->pair_mk, n_tri));
        }
    }
    if (!s->los_off) CHECK(dalloc(&s->los_off, n + 1));
    if (G != s->n_groups || !s->group_off) {
        dfree(s->group_off);
        CHECK(dalloc(&s->group_off, (size_t)G + 1));
    }
    s->n_pairs = m;
    s->n_groups = G;
    hipStream_t st = s->stream;
    if (m) {
        HIP_TRY(hipMemcpyAsync(s->comp_win, win.data(), sizeof(uint32_t) * m, hipMemcpyHostToDevice, st));
        HIP_TRY(hipMemcpyAsync(s->comp_los, los.data(), sizeof(uint32_t) * m, hipMemcpyHostToDevice, st));
        HIP_TRY(hipMemcpyAsync(s->comp_w, w.data(), sizeof(double) * m, hipMemcpyHostToDevice, st));
        HIP_TRY(hipMemcpyAsync(s->comp_wq, wq.data(), sizeof(long long) * m, hipMemcpyHostToDevice, st));
        HIP_TRY(hipMemcpyAsync(s->los_idx, lidx.data(), sizeof(uint32_t) * m, hipMemcpyHostToDevice, st));
    }
    HIP_TRY(hipMemcpyAsync(s->comp_off, off.data(), sizeof(uint32_t) * (n + 1), hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync(s->los_off, loff.data(), sizeof(uint32_t) * (n + 1), hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync(s->group_off, go, sizeof(uint32_t) * ((size_t)G + 1), hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync(s->score_w, pw.data(), sizeof(double) * n, hipMemcpyHostToDevice, st));
    HIP_TRY(hipStreamSynchronize(st));
    s->pairs_set = true;
    return CBH_OK;
}

// Pairwise scoring of one level (PairLogitPairwise, tree.rs:3810-3900): statistics, prefix
// sums over buckets, one wavefront per (border, feature), per-feature best, level argmax.
int pairwise_level(cbh_session* s, const long long* cur, uint32_t level) {
    hipStream_t st = s->stream;
    const uint32_t P = 1u << level, B = s->B, F = s->F;
    // statistics: pairs grouped by leaf-pair key (a level of one leaf reads them in input
    // order), one workgroup per (key, chunk, 16-feature tile); keys of one chunk write their
    // cumulative runs, the chunks of larger keys add into zeroed runs that are scanned after
    const bool direct = P == 1;
    const uint32_t n_tri = P * (P + 1) / 2;
    const uint32_t tiles = (F + kStatTileF - 1) / kStatTileF;
    // chunk: the pairs times the tiles spread once over the CUs (one workgroup each: its cells
    // take most of the LDS), in whole 1024-pair passes
    const uint64_t spread = (s->n_pairs * tiles + s->pair_cus - 1) / s->pair_cus;
    const uint32_t chunk = (uint32_t)std::max<uint64_t>(kStatChunkMin, (spread + 1023) / 1024 * 1024);
    const uint32_t nchunk = (uint32_t)((s->n_pairs + chunk - 1) / chunk);
    const uint32_t max_desc = n_tri + nchunk, max_multi = std::min(n_tri, nchunk);
    if (!direct) {
        const uint32_t nk = P * P;   // (the previous level's plan cleared the counts)
        if (s->n_pairs) {
            pair_key_count_kernel<<<(unsigned)((s->n_pairs + 256 * kCountItems - 1) / (256 * kCountItems)), 256,
                                    nk * sizeof(uint32_t), st>>>(
                s->comp_win, s->comp_los, s->n_pairs, s->leaf, P, s->key_cnt);
            HIP_TRY(hipGetLastError());
        }
    }
    const uint32_t pmax = 1u << (s->depth - 1), next = std::min(4 * P * P, pmax * pmax);
    pair_plan_kernel<<<1, 1024, 0, st>>>(s->key_cnt, P, direct ? 1 : 0, (uint32_t)s->n_pairs, chunk, s->key_off, s->key_cur,
                                         s->pair_desc, s->pair_nd, s->pair_mk, s->pair_nd + 1, s->key_cnt,
                                         level + 1 < s->depth ? next : 0u);
    HIP_TRY(hipGetLastError());
    if (!direct && s->n_pairs) {   // the scatter, and in the same launch the multi-chunk runs' zeroing
        const unsigned n_sc = (unsigned)((s->n_pairs + 256 * kScatterItems - 1) / (256 * kScatterItems));
        pair_key_scatter_kernel<<<n_sc + max_multi * F, 256, P * P * sizeof(uint32_t), st>>>(
            s->comp_win, s->comp_los, s->comp_wq, s->n_pairs, s->leaf, P, s->key_cur, s->key_rec, s->key_wq, n_sc,
            s->pair_mk, s->pair_nd + 1, F, B, s->pair_st);
        HIP_TRY(hipGetLastError());
    } else if (max_multi) {
        pair_multi_zero_kernel<<<dim3(max_multi, F), 256, 0, st>>>(s->pair_mk, s->pair_nd + 1, P, B, s->pair_st);
        HIP_TRY(hipGetLastError());
    }
    // 32-bit buffer offsets formed by one 24-bit multiply-add (row < 2^24, 4 Ws < 2^24)
    const bool buf = (uint64_t)s->n * s->Ws * 4 < (1ull << 32) && s->n < (1u << 24) && s->Ws < (1u << 22);
    (buf ? pair_stats_feature_kernel<true> : pair_stats_feature_kernel<false>)
        <<<8u * tiles * ((max_desc + 7) / 8), kStatThreads, pair_stat_lds(B), st>>>(
            s->rows, s->Ws, s->pair_desc, s->pair_nd, s->key_rec, s->key_wq, s->comp_win, s->comp_los, s->comp_wq,
            direct ? 1 : 0, F, P, B, s->pair_st, tiles);
    HIP_TRY(hipGetLastError());
    if (max_multi) {
        pair_multi_scan_kernel<<<dim3(max_multi, F), 256, 0, st>>>(s->pair_mk, s->pair_nd + 1, P, B, s->pair_st);
        HIP_TRY(hipGetLastError());
    }
    {
        const dim3 grid((B - 1 + 7) / 8 * 8, F);
#define CBH_PAIR_CAND(PV)                                                                                \
    pairwise_candidate_kernel<PV><<<grid, 64, pair_cand_lds(PV), st>>>(s->pair_st, cur, s->C, F, s->n_cand, B, s->scales, \
                                                                  s->pair_inv, s->l2, s->prior, s->cand_scores)
        // up to 8 leaves: one border per lane, the system in the lane's registers
        const dim3 lgrid((B - 1 + 63) / 64, F);
#define CBH_PAIR_LANE(PV)                                                                             \
    pairwise_candidate_lane_kernel<PV><<<lgrid, 64, 0, st>>>(s->pair_st, cur, s->C, F, s->n_cand, B, s->scales, \
                                                             s->pair_inv, s->l2, s->prior, s->cand_scores)
        switch (P) {
            case 1: CBH_PAIR_LANE(1); break;
            case 2: CBH_PAIR_LANE(2); break;
            case 4: CBH_PAIR_LANE(4); break;
            case 8: CBH_PAIR_LANE(8); break;
            case 16: CBH_PAIR_CAND(16); break;
            case 32: CBH_PAIR_CAND(32); break;
            case 64:   // one workgroup per candidate, its system in LDS
                pairwise_candidate_block_kernel<<<F * (B - 1), 256, pair_cand_block_doubles(64) * sizeof(double), st>>>(
                    s->pair_st, cur, s->C, F, s->n_cand, B, P, s->scales, s->pair_inv, s->l2, s->prior,
                    s->cand_scores, nullptr);
                break;
            case 128:  // a persistent grid, one global workspace slot per workgroup
                pairwise_candidate_block_kernel<<<s->pair_cand_wgs, 256, 0, st>>>(
                    s->pair_st, cur, s->C, F, s->n_cand, B, P, s->scales, s->pair_inv, s->l2, s->prior,
                    s->cand_scores, s->pair_ws);
                break;
            default: return fail(CBH_ERR_UNSUPPORTED, "pairwise scoring: level of " + std::to_string(P) + " leaves");
        }
#undef CBH_PAIR_CAND
#undef CBH_PAIR_LANE
        HIP_TRY(hipGetLastError());
    }
    pairwise_best_kernel<<<F, 256, 0, st>>>(s->cand_scores, s->n_cand, B, s->best_score, s->best_bin);
    HIP_TRY(hipGetLastError());
    argmax_kernel<<<1, 1024, 0, st>>>(s->best_score, s->best_bin, nullptr, F, s->splits + level);
    HIP_TRY(hipGetLastError());
    return CBH_OK;
}

// model_size_reg weights of the CTR columns for one level (tree.rs:3245-3346): a column whose
// (ctr type, projection) group an earlier tree or an earlier level of this tree used scores at
// weight 1, any other at (1 + buckets / max_count)^(-model_size_reg), max_count the largest
// bucket count of the CTR columns and, once the tree holds a float split, of the distinct
// (float-partition leaf, bucket) pairs of the categorical columns.  The weight is computed on
// the host with the C library's pow, the function the reference calls.
bool ctr_all_used(const cbh_session* s) {
    for (uint32_t c = 0; c < s->ctr_n; ++c)
        if (!s->ctr_used[s->ctr_group[c]]) return false;
    return true;
}

int ctr_level_weights(cbh_session* s, uint32_t level) {
    hipStream_t st = s->stream;
    if (ctr_all_used(s)) {   // every group is in the model already: every weight is 1
        if (!s->fweight_one) {
            std::fill(s->fweight_host.begin(), s->fweight_host.end(), 1.0);
            HIP_TRY(hipMemcpyAsync(s->fweight, s->fweight_host.data(), sizeof(double) * s->F,
                                   hipMemcpyHostToDevice, st));
            s->fweight_one = true;
        }
        return CBH_OK;
    }
    s->fweight_one = false;
    std::vector<SplitRec> prev(level);
    if (level) {
        HIP_TRY(hipMemcpyAsync(prev.data(), s->splits, sizeof(SplitRec) * level, hipMemcpyDeviceToHost, st));
        HIP_TRY(hipStreamSynchronize(st));
    }
    const uint32_t fc0 = s->F - s->ctr_n;
    uint64_t max_count = s->ctr_eligible_max;
    uint32_t float_mask = 0;
    for (uint32_t l = 0; l < level; ++l)
        if (prev[l].feature < fc0) float_mask |= 1u << l;
    if (float_mask && s->cat_n) {
        const uint32_t L = 1u << level;
        std::vector<uint64_t> off(s->cat_n);
        uint64_t words = 0;
        for (uint32_t c = 0; c < s->cat_n; ++c) {   // kPhantomBlocks slices per column
            off[c] = words;
            words += kPhantomBlocks * (((uint64_t)s->cat_nb[c] * L + 31) / 32);
        }
        HIP_TRY(hipMemcpyAsync(s->phantom_off, off.data(), sizeof(uint64_t) * s->cat_n, hipMemcpyHostToDevice, st));
        (void)words;
        const dim3 bg(kPhantomBlocks, s->cat_n);
        const size_t bl = kPhantomLdsWords * sizeof(uint32_t);
        if (s->cat_bk16)
            phantom_bits_kernel<uint16_t><<<bg, kPhantomThreads, bl, st>>>(s->leaf, s->n, (int64_t)float_mask, L, s->cat_bk16,
                                                               s->cat_nb_dev, s->phantom_off, s->phantom_bits, nullptr,
                                                               0u, 0u, nullptr, s->ctr_eligible_max, s->phantom_cnt);
        else
            phantom_bits_kernel<uint32_t><<<bg, kPhantomThreads, bl, st>>>(s->leaf, s->n, (int64_t)float_mask, L, s->cat_bk,
                                                               s->cat_nb_dev, s->phantom_off, s->phantom_bits, nullptr,
                                                               0u, 0u, nullptr, s->ctr_eligible_max, s->phantom_cnt);
        HIP_TRY(hipGetLastError());
        phantom_count_kernel<<<dim3(s->cat_n, kPhantomCountSplit), 256, 0, st>>>(s->phantom_bits, s->phantom_off, s->cat_nb_dev, L,
                                                       s->phantom_cnt, nullptr, 0u, 0u, nullptr, (int64_t)float_mask,
                                                       s->ctr_eligible_max);
        HIP_TRY(hipGetLastError());
        std::vector<unsigned long long> cnt(s->cat_n);
        HIP_TRY(hipMemcpyAsync(cnt.data(), s->phantom_cnt, sizeof(unsigned long long) * s->cat_n,
                               hipMemcpyDeviceToHost, st));
        HIP_TRY(hipStreamSynchronize(st));
        for (unsigned long long v : cnt) max_count = std::max<uint64_t>(max_count, v);
    }
    for (uint32_t c = 0; c < s->ctr_n; ++c) {
        bool used = s->ctr_used[s->ctr_group[c]] != 0;
        for (uint32_t l = 0; l < level; ++l)
            if (prev[l].feature >= fc0 && s->ctr_group[prev[l].feature - fc0] == s->ctr_group[c]) used = true;
        double w = 1.0;
        if (!used && s->msr != 0.0 && max_count != 0)
            w = std::pow(1.0 + (double)s->ctr_bc[c] / (double)max_count, -s->msr);
        s->fweight_host[fc0 + c] = w;
    }
    HIP_TRY(hipMemcpyAsync(s->fweight, s->fweight_host.data(), sizeof(double) * s->F, hipMemcpyHostToDevice, st));
    return CBH_OK;
}

// The same weights without the host: phantom bitmaps and counts read the float splits from the
// device (nothing is set before the first float split), and ctr_weights_kernel picks each
// column's weight from the host-built pow table.  Recordable into the tree graph.
int ctr_level_weights_dev(cbh_session* s, uint32_t level) {
    hipStream_t st = s->stream;
    const uint32_t fc0 = s->F - s->ctr_n;
    if (level >= 1 && s->cat_n) {
        const uint32_t L = 1u << level;
        const uint64_t* off = s->phantom_off_lv + (size_t)level * s->cat_n;
        const dim3 bg(kPhantomBlocks, s->cat_n);
        const size_t bl = kPhantomLdsWords * sizeof(uint32_t);
        if (s->cat_bk16)
            phantom_bits_kernel<uint16_t><<<bg, kPhantomThreads, bl, st>>>(s->leaf, s->n, -1, L, s->cat_bk16, s->cat_nb_dev, off,
                                                               s->phantom_bits, s->splits, level, fc0,
                                                               s->ctr_used_dev + s->ctr_n, s->ctr_m_lo, s->phantom_cnt);
        else
            phantom_bits_kernel<uint32_t><<<bg, kPhantomThreads, bl, st>>>(s->leaf, s->n, -1, L, s->cat_bk, s->cat_nb_dev, off,
                                                               s->phantom_bits, s->splits, level, fc0,
                                                               s->ctr_used_dev + s->ctr_n, s->ctr_m_lo, s->phantom_cnt);
        HIP_TRY(hipGetLastError());
        phantom_count_kernel<<<dim3(s->cat_n, kPhantomCountSplit), 256, 0, st>>>(s->phantom_bits, off, s->cat_nb_dev, L, s->phantom_cnt,
                                                       s->splits, level, fc0, s->ctr_used_dev + s->ctr_n, -1,
                                                       s->ctr_m_lo);
        HIP_TRY(hipGetLastError());
    }
    ctr_weights_kernel<<<1, 64, 0, st>>>(s->splits, level, fc0, s->ctr_n, s->ctr_group_dev, s->ctr_used_dev,
                                         s->phantom_cnt, level >= 1 ? s->cat_n : 0u, s->ctr_pow, s->ctr_m_lo,
                                         s->ctr_m_hi, s->msr == 0.0 ? 1 : 0, s->fweight);
    HIP_TRY(hipGetLastError());
    return CBH_OK;
}

// Every launch of one tree on the session stream, ending with the copies of its results
// into pinned staging.  No host decision happens between launches (the split, partition
// plan and leaf values stay on the device), so the sequence can be recorded once as a graph
// and replayed for every later tree.
// 64-bit LDS atomics a (row, feature) entry of the level's fill issues: one per channel (generic
// and tiled exact fills), one (rounded packed and count-packed fills), one per plane of two
// channels (packed multi-channel fills; the weight's plane left out at level 0 once it is cached).
uint32_t fill_atomics_per_entry(const cbh_session* s, uint32_t level) {
    if (s->packed || s->count) return 1u;
    if (s->pkk) return (s->C + 1) / 2 - ((level == 0 && s->l0_cached) ? 1u : 0u);
    return s->C;
}

template <int K>
int enqueue_tree(cbh_session* s, bool use_host_sample) {
    constexpr int C = K + 1;
    const bool apply_prev = s->pending;   // the previous tree's leaves are applied by prepare
    const uint64_t n = s->n;
    hipStream_t st = s->stream;
    const int newton = s->cfg.leaf_method == CBH_LEAF_NEWTON ? 1 : 0;
    const int sfn = s->cfg.score_function;   // CBH_SCORE_*
    const int loss = s->cfg.loss == CBH_LOSS_RMSE ? 0 : 1;

    // ---- prepare: apply previous tree, ders, sample, score channels, bounds ----
    CHECK(s->stage_begin(kStPrepare));
    if (s->ranking) {   // pair ders need every row's updated approximant: apply, then ders
        if (apply_prev) {
            apply_leaves_kernel<<<grid_for(n, 256, 8192), 256, 0, st>>>(s->approx, s->leaf, s->leaf_scaled, n);
            HIP_TRY(hipGetLastError());
        }
        pairlogit_row_ders_kernel<<<grid_for(n, 256), 256, 0, st>>>(n, s->comp_off, s->comp_win, s->comp_los,
                                                                  s->comp_w, s->los_off, s->los_idx, s->approx,
                                                                  s->ext_der, s->ext_der + n);
        HIP_TRY(hipGetLastError());
    }
    const unsigned pgrid = grid_for(n, 256, kPrepBlocks);
    prepare_kernel<K><<<pgrid, 256, 0, st>>>(
        n, loss, s->approx, s->target, s->weight, s->leaf,
        apply_prev && !s->ranking ? s->leaf_scaled : nullptr,   // a pair loss applied them above
        s->smp_dev, s->jt(), use_host_sample ? s->host_sample : nullptr, s->sstat, newton, s->partials,
        s->ranking ? s->ext_der : nullptr, s->ranking ? s->score_w : nullptr);
    HIP_TRY(hipGetLastError());
    scales_kernel<<<1, 256, 0, st>>>(s->partials, pgrid, s->bounds, s->scales,
                                     (s->packed || s->pkk) ? s->pack_bits : 0, s->count ? 1 : 0);
    HIP_TRY(hipGetLastError());
    if (s->pkk)
        quantize_pack_kernel<C><<<grid_for(n, 256, 8192), 256, 0, st>>>(s->sstat, n, s->scales, s->spack,
                                                                        (1ll << s->pack_bits) - 1);
    else if (s->packed)
        pack_stats_fixed_kernel<<<grid_for(n, 256, 8192), 256, 0, st>>>(s->sstat, n, s->scales, s->spack,
                                                                         (1ll << s->pack_bits) - 1);
    else if (s->count)
        pack_stats_count_kernel<<<grid_for(n, 256, 8192), 256, 0, st>>>(s->sstat, n, s->scales, s->spack);
    else if (!s->tiled)   // (the tiled exact fill rounds the f64 channels as it stages them)
        quantize_stats_kernel<C><<<grid_for(n * C, 256, 8192), 256, 0, st>>>(s->sstat, n, s->scales);
    HIP_TRY(hipGetLastError());
    CHECK(s->stage_end());

    const size_t per_leaf = (size_t)s->F * s->B * C;
    const uint32_t NB = s->n_part_blocks;
    for (uint32_t level = 0; level < s->depth; ++level) {
        long long* cur = s->hist[level & 1];
        long long* par = s->hist[(level + 1) & 1];
        const uint32_t n_leaves = 1u << level;
        // ---- fill (the histogram it accumulates into is zeroed first: here at level 0 and with
        // pairwise scoring, else by the previous level's score kernel) ----
        if (level == 0 || s->pairwise) {
            CHECK(s->stage_begin(kStPrepare));
            CHECK(launch_zero(cur, per_leaf * n_leaves, st));
            CHECK(s->stage_end());
        }
        const uint32_t nt = s->tiles.n_tiles;
        const uint32_t G = s->fill_ranges;
        const uint32_t* lidx = level == 0 ? nullptr : s->idx;
        const LevelPlan* lplan = level == 0 ? nullptr : s->plans + (level - 1);
        const uint32_t n_seg = level == 0 ? 1u : (1u << (level - 1));
        if (s->use_skip) {   // segment totals for the dominant-bin rebuild (timed with the finishing)
            CHECK(s->stage_begin(kStDerive));
            CHECK(launch_zero(s->seg_tot, (size_t)n_seg * C, st));
            seg_totals_kernel<<<grid_for(n, 256, 1024), 256, 0, st>>>(lidx, lplan, n,
                                                                     (const long long*)s->sstat, C, s->seg_tot);
            HIP_TRY(hipGetLastError());
            CHECK(s->stage_end());
        }
        CHECK(s->stage_begin(kStFill));   // the fill kernel alone
        if (s->packed && level == 0)
            fill_packed_kernel<false, false><<<s->pk_dense.blocks, kPackThreads, s->pk_lds, st>>>(
                s->trows, s->W, n, nullptr, nullptr, s->spack, nullptr, s->pk_dense.tiles16, s->F, s->B,
                s->pk_dense.ranges, s->pk_dense.ranges_n, cur, s->pk_swap, nullptr, 0u, s->scales);
        else if (s->packed)
            fill_packed_kernel<true, false><<<s->pk_gath.blocks, kPackThreads, s->pk_lds, st>>>(
                s->trows, s->W, n, lidx, lplan, s->spack, s->sseq, s->pk_gath.tiles16, s->F, s->B,
                s->pk_gath.ranges, 0u, cur, s->pk_swap, s->pk_rm_sh ? s->rows : nullptr, s->pk_rm_sh, s->scales);
        else if (s->count && level == 0)
            fill_packed_kernel<false, true><<<s->pk_dense.blocks, kPackThreads, s->pk_lds, st>>>(
                s->trows, s->W, n, nullptr, nullptr, s->spack, nullptr, s->pk_dense.tiles16, s->F, s->B,
                s->pk_dense.ranges, s->pk_dense.ranges_n, cur, 0u, nullptr, 0u, s->scales);
        else if (s->count)
            fill_packed_kernel<true, true><<<s->pk_gath.blocks, kPackThreads, s->pk_lds, st>>>(
                s->trows, s->W, n, lidx, lplan, s->spack, s->sseq, s->pk_gath.tiles16, s->F, s->B,
                s->pk_gath.ranges, 0u, cur, 0u, s->pk_rm_sh ? s->rows : nullptr, s->pk_rm_sh, s->scales);
        else if (s->tiled && level == 0)
            fill_exact_kernel<false><<<s->pk_dense.blocks, kExThreads, s->pk_lds, st>>>(
                s->trows, s->W, n, nullptr, nullptr, (const long long*)s->sstat, nullptr, s->pk_dense.tiles16, s->F,
                s->B, s->pk_dense.ranges, s->pk_dense.ranges_n, cur, nullptr, 0u, s->ex_sets, s->scales);
        else if (s->tiled)
            fill_exact_kernel<true><<<s->pk_gath.blocks, kExThreads, s->pk_lds, st>>>(
                s->trows, s->W, n, lidx, lplan, (const long long*)s->sstat, (const long long*)s->sseq,
                s->pk_gath.tiles16, s->F, s->B, s->pk_gath.ranges, s->pk_gath.ranges_n, cur,
                s->pk_rm_sh ? s->rows : nullptr, s->pk_rm_sh, s->ex_sets, s->scales);
        else if (s->pkk) {
            const size_t lds = (size_t)kPkkCells * sizeof(unsigned long long);
            const unsigned grid = s->pkk_ranges * s->pkk_tiles;
            // level 0 of a session whose weight channel is the same every tree (alone in the last
            // plane, no per-tree sample): after the first tree the plane's cells come from the
            // cache of its level-0 histogram, copied in before the fill, and the fill adds the
            // other planes only
            const uint32_t NPl = (C + 1) / 2;
            const bool w0_use = level == 0 && s->w_static && s->w0_ready;
            const uint32_t npf = w0_use ? NPl - 1 : NPl;
            if (level == 0) s->l0_cached = w0_use;
            if (w0_use)
                HIP_TRY(hipMemcpyAsync(cur + (size_t)(C - 1) * s->F * s->B, s->w0_cache,
                                       sizeof(long long) * s->F * s->B, hipMemcpyDeviceToDevice, st));
            // (small tiles: 4 cells per thread, their registers leaving room for 8 blocks in flight)
            const size_t lds4 = (size_t)4 * kPkkThreads * sizeof(unsigned long long);
            if (s->pks && s->pks_small && level == 0)
                fill_pks_kernel<C, false, 4, 8><<<grid, kPkkThreads, lds4, st>>>(
                    s->pks_a, s->pks_b, n, nullptr, nullptr, s->spack, s->pkk_tiles, s->F, s->B, s->pkk_ranges, cur, npf);
            else if (s->pks && s->pks_small)
                fill_pks_kernel<C, true, 4, 8><<<grid, kPkkThreads, lds4, st>>>(
                    s->pks_a, s->pks_b, n, lidx, lplan, s->spack, s->pkk_tiles, s->F, s->B, s->pkk_ranges, cur, npf);
            else if (s->pks && level == 0)
                fill_pks_kernel<C, false><<<grid, kPkkThreads, lds, st>>>(
                    s->pks_a, s->pks_b, n, nullptr, nullptr, s->spack, s->pkk_tiles, s->F, s->B, s->pkk_ranges, cur, npf);
            else if (s->pks)
                fill_pks_kernel<C, true><<<grid, kPkkThreads, lds, st>>>(
                    s->pks_a, s->pks_b, n, lidx, lplan, s->spack, s->pkk_tiles, s->F, s->B, s->pkk_ranges, cur, npf);
            else if (s->use_skip && level == 0)
                fill_pkk_kernel<C, true, false><<<grid, kPkkThreads, lds, st>>>(
                    s->rows, s->W, s->Ws, n, nullptr, nullptr, s->spack, s->pkk_tiles, s->F, s->B, s->pkk_ranges, cur,
                    s->skip_bin, npf);
            else if (s->use_skip)
                fill_pkk_kernel<C, true, true><<<grid, kPkkThreads, lds, st>>>(
                    s->rows, s->W, s->Ws, n, lidx, lplan, s->spack, s->pkk_tiles, s->F, s->B, s->pkk_ranges, cur,
                    s->skip_bin, npf);
            else if (level == 0)
                fill_pkk_kernel<C, false, false><<<grid, kPkkThreads, lds, st>>>(
                    s->rows, s->W, s->Ws, n, nullptr, nullptr, s->spack, s->pkk_tiles, s->F, s->B, s->pkk_ranges, cur,
                    nullptr, npf);
            else
                fill_pkk_kernel<C, false, true><<<grid, kPkkThreads, lds, st>>>(
                    s->rows, s->W, s->Ws, n, lidx, lplan, s->spack, s->pkk_tiles, s->F, s->B, s->pkk_ranges, cur,
                    nullptr, npf);
        } else if (s->use_skip)
            fill_kernel<C, true><<<G * nt, 1024, s->tiles.lds_bytes, st>>>(
                s->rows, s->W, s->Ws, n, lidx, lplan, (const long long*)s->sstat, nt, s->tiles.tw, s->F, s->B, G, cur,
                s->skip_bin, (int)s->tiles.bin_major);
        else if (C == 2 && s->pairwise)
            // PairLogitPairwise scores from the der channel and the pair statistics alone: the
            // weight channel is left out of the fill (its cells stay zero; such sessions refuse
            // histogram capture)
            fill_kernel<2, false, 1><<<G * nt, 1024, s->tiles.lds_bytes, st>>>(
                s->rows, s->W, s->Ws, n, lidx, lplan, (const long long*)s->sstat, nt, s->tiles.tw, s->F, s->B, G, cur,
                nullptr, (int)s->tiles.bin_major);
        else
            fill_kernel<C, false><<<G * nt, 1024, s->tiles.lds_bytes, st>>>(
                s->rows, s->W, s->Ws, n, lidx, lplan, (const long long*)s->sstat, nt, s->tiles.tw, s->F, s->B, G, cur,
                nullptr, (int)s->tiles.bin_major);
        HIP_TRY(hipGetLastError());
        CHECK(s->stage_end());
        if (s->pkk && level == 0 && s->w_static && !s->w0_ready) {   // the weight channel's cache
            HIP_TRY(hipMemcpyAsync(s->w0_cache, cur + (size_t)(C - 1) * s->F * s->B, sizeof(long long) * s->F * s->B,
                                   hipMemcpyDeviceToDevice, st));
            s->w0_ready = true;
        }
        if (s->cfg.profile && s->use_skip) {   // the entries this launch added (untimed)
            if (!s->row_ent) {
                CHECK(dalloc(&s->row_ent, n));
                row_entries_kernel<<<grid_for(n, 256), 256, 0, st>>>(s->cols, n, s->F, s->skip_bin, s->row_ent);
                HIP_TRY(hipGetLastError());
            }
            if (!s->fill_ent) {
                CHECK(dalloc(&s->fill_ent, 2));
                HIP_TRY(hipMemsetAsync(s->fill_ent, 0, 2 * sizeof(unsigned long long), st));
            }
            fill_entries_kernel<<<grid_for(n, 256, 1024), 256, 0, st>>>(lidx, lplan, n, s->row_ent, s->fill_ent,
                                                                       fill_atomics_per_entry(s, level));
            HIP_TRY(hipGetLastError());
        }
        // ---- histogram finishing: dominant bins, prefix form, siblings ----
        CHECK(s->stage_begin(kStDerive));
        {   // built children to prefix form over bins (the level's histograms stay in it), with
            // their dominant bins rebuilt from the segment totals, and their siblings = parent -
            // built (levels >= 1)
            const uint64_t rows = (uint64_t)n_seg * C * s->F;
            if (s->B <= 72)   // 8 lanes per row
                hist_prefix_group_kernel<8, 9><<<(unsigned)((rows + 31) / 32), 256, 0, st>>>(
                    cur, lplan, n_seg, C, s->F, s->B, level > 0 ? par : nullptr,
                    s->use_skip ? s->skip_bin : nullptr, s->seg_tot);
            else if (s->B <= 80)   // 16 lanes per row
                hist_prefix_group_kernel<16, 5><<<(unsigned)((rows + 15) / 16), 256, 0, st>>>(
                    cur, lplan, n_seg, C, s->F, s->B, level > 0 ? par : nullptr,
                    s->use_skip ? s->skip_bin : nullptr, s->seg_tot);
            else if (s->B <= 96)   // a half-wave per row
                hist_prefix_group_kernel<32, 3><<<(unsigned)((rows + 7) / 8), 256, 0, st>>>(
                    cur, lplan, n_seg, C, s->F, s->B, level > 0 ? par : nullptr,
                    s->use_skip ? s->skip_bin : nullptr, s->seg_tot);
            else
                hist_prefix_kernel<<<(unsigned)((rows + 3) / 4), 256, 0, st>>>(
                    cur, lplan, n_seg, C, s->F, s->B, level > 0 ? par : nullptr,
                    s->use_skip ? s->skip_bin : nullptr, s->seg_tot);
            HIP_TRY(hipGetLastError());
        }
        CHECK(s->stage_end());
        if (s->hist_cap)   // the level's histograms as the scorer reads them (inspection only)
            HIP_TRY(hipMemcpyAsync(s->hist_cap + s->hist_cap_off[level], cur, sizeof(long long) * per_leaf * n_leaves,
                                   hipMemcpyDeviceToDevice, st));
        // ---- score + argmax ----
        if (s->ctr_n) CHECK(s->ctr_dev ? ctr_level_weights_dev(s, level) : ctr_level_weights(s, level));
        CHECK(s->stage_begin(kStScore));
        // the score also clears the next level's histogram (the parent buffer, dead once the
        // derive above has run)
        long long* zbuf = level + 1 < s->depth ? par : nullptr;
        const uint32_t zleaves = level + 1 < s->depth ? 2u * n_leaves : 0u;
        // K > 1: the parents are split over the (at most 8) waves of a feature's workgroup, 16
        // per wave from 64 parents at K >= 3 (registers), else 8 (fewer than 8: one wave)
        const uint32_t chain_pw = n_leaves >= 64 && K >= 3 ? 16u : 8u;
        const bool chain = K > 1 && s->score_chain && sfn <= CBH_SCORE_L2 && s->max_cand <= 64 &&
                           n_leaves <= 8 * chain_pw &&
                           (n_leaves < 8 || n_leaves % chain_pw == 0) &&
                           (uint64_t)chain_pw * s->C * s->F * s->B * 8u < (1ull << 31);
        if (s->pairwise) {
            CHECK(pairwise_level(s, cur, level));
        } else if (chain) {
            // several features per workgroup when B lanes per feature leave most of a wave idle
            // (config 5's 20 bins: 3 features in 60 lanes) and no feature is one-hot; at most 64 /
            // chain_pw (the lane-per-(feature, parent) totals load)
            uint32_t nf = s->one_hot ? 1u : std::max<uint32_t>(1u, std::min<uint32_t>(64u / s->B, 64u / chain_pw));
            if (s->chain_nf) nf = std::min<uint32_t>(nf, s->chain_nf);
            const uint32_t groups = (s->F + nf - 1) / nf;
            if constexpr (K >= 3) {
                if (chain_pw == 16)
                    score_chain_kernel<K, 16, false><<<groups, 64 * (n_leaves / 16), 0, st>>>(
                        zbuf, zleaves, s->C, cur, n_leaves, s->F, s->B, s->n_cand, s->one_hot, s->scales, s->l2,
                        sfn, s->best_score, s->best_bin, s->ctr_n ? s->fweight : nullptr, s->chain_spin,
                        &s->bounds->device_err, nf);
            }
            if constexpr (K > 1) {
                if (chain_pw == 8 && n_leaves >= 8)
                    score_chain_kernel<K, 8, false><<<groups, 64 * (n_leaves / 8), 0, st>>>(
                        zbuf, zleaves, s->C, cur, n_leaves, s->F, s->B, s->n_cand, s->one_hot, s->scales, s->l2,
                        sfn, s->best_score, s->best_bin, s->ctr_n ? s->fweight : nullptr, s->chain_spin,
                        &s->bounds->device_err, nf);
                else if (chain_pw == 8)
                    score_chain_kernel<K, 8, true><<<groups, 64, 0, st>>>(
                        zbuf, zleaves, s->C, cur, n_leaves, s->F, s->B, s->n_cand, s->one_hot, s->scales, s->l2,
                        sfn, s->best_score, s->best_bin, s->ctr_n ? s->fweight : nullptr, s->chain_spin,
                        &s->bounds->device_err, nf);
            }
        } else if (s->max_cand <= 64)
            score_kernel<K, 1><<<s->F, 64, 0, st>>>(zbuf, zleaves, s->C, cur, n_leaves, s->F, s->B, s->n_cand, s->one_hot,
                                                   s->scales, s->l2, sfn, s->best_score, s->best_bin,
                                                   s->ctr_n ? s->fweight : nullptr);
        else if (s->max_cand <= 128)
            score_kernel<K, 2><<<s->F, 128, 0, st>>>(zbuf, zleaves, s->C, cur, n_leaves, s->F, s->B, s->n_cand, s->one_hot,
                                                    s->scales, s->l2, sfn, s->best_score, s->best_bin,
                                                   s->ctr_n ? s->fweight : nullptr);
        else
            score_kernel<K, 4><<<s->F, 256, 0, st>>>(zbuf, zleaves, s->C, cur, n_leaves, s->F, s->B, s->n_cand, s->one_hot,
                                                    s->scales, s->l2, sfn, s->best_score, s->best_bin,
                                                   s->ctr_n ? s->fweight : nullptr);
        HIP_TRY(hipGetLastError());
        if (!s->pairwise) {
            argmax_kernel<<<1, 1024, 0, st>>>(s->best_score, s->best_bin, s->one_hot, s->F, s->splits + level);
            HIP_TRY(hipGetLastError());
        }
        CHECK(s->stage_end());
        // ---- partition ----
        CHECK(s->stage_begin(kStPartition));
        const bool last = level + 1 == s->depth;
        split_count_kernel<<<NB, 256, 0, st>>>(s->cols, n, s->splits + level, level, s->leaf, s->cnt,
                                               4 * NB, last ? 0 : 1);
        HIP_TRY(hipGetLastError());
        if (!last) {
            plan_scan_kernel<<<2u << level, 1024, 0, st>>>(s->cnt, 4 * NB, s->totals);
            HIP_TRY(hipGetLastError());
            if (s->packed || s->count)   // the listed rows' packed statistic
                compact_kernel<1><<<NB, 256, 0, st>>>(s->leaf, n, level, s->cnt, 4 * NB, s->totals, s->plans + level,
                                                      s->idx, s->spack, s->sseq);
            else if (s->tiled && s->sseq)   // both f64 score channels of the listed rows
                compact_kernel<2><<<NB, 256, 0, st>>>(s->leaf, n, level, s->cnt, 4 * NB, s->totals, s->plans + level,
                                                      s->idx, (const unsigned long long*)s->sstat, s->sseq);
            else
                compact_kernel<0><<<NB, 256, 0, st>>>(s->leaf, n, level, s->cnt, 4 * NB, s->totals, s->plans + level,
                                                      s->idx, nullptr, nullptr);
            HIP_TRY(hipGetLastError());
        }
        CHECK(s->stage_end());
    }

    // ---- leaf statistics + values ----
    if (s->ctr_n) {   // leaves over the averaging-permutation CTR bins
        averaging_leaf_kernel<<<grid_for(n, 256, 8192), 256, 0, st>>>(s->leaf, n, s->splits, s->depth,
                                                                      s->F - s->ctr_n, s->ctr_avg);
        HIP_TRY(hipGetLastError());
    }
    CHECK(s->stage_begin(kStLeaf));
    const uint32_t n_leaves = 1u << s->depth;
    const uint32_t CL = (uint32_t)leaf_cells<K>();
    CHECK(launch_zero(s->leaf_sums, (size_t)n_leaves * CL, st));
    const size_t lds = (size_t)n_leaves * CL * sizeof(long long);   // attribute set at open
    // one workgroup of 1024 threads a CU: each flushes its LDS sums once (n_leaves * CL global
    // atomics a workgroup: 16.6k at K = 10 and 256 leaves, so few workgroups)
    leaf_reduce_kernel<K><<<grid_for(n, kLeafThreads, s->cus), kLeafThreads, lds, st>>>(
        n, loss, newton, s->approx, s->target, s->weight, s->leaf, s->scales, n_leaves, s->leaf_sums,
        s->ranking ? s->ext_der : nullptr, s->ranking ? s->score_w : nullptr);
    HIP_TRY(hipGetLastError());
    if (s->pairwise) {
        CHECK(launch_zero(s->leaf_w, (size_t)n_leaves * n_leaves, st));
        if (s->n_pairs) {
            const size_t lw_bytes = (size_t)n_leaves * n_leaves * sizeof(long long);
            const bool lw_lds = lw_bytes <= kPairLdsMax;
            pair_leaf_weights_kernel<<<grid_for(s->n_pairs, 1024, s->cus), 1024, lw_lds ? lw_bytes : 0, st>>>(
                s->comp_win, s->comp_los, s->comp_wq, s->n_pairs, s->leaf, n_leaves, s->leaf_w, lw_lds ? 1 : 0);
            HIP_TRY(hipGetLastError());
        }
        // 4 to 64 leaves: the system in one wavefront's registers; else the workgroup solve over
        // LDS or the workspace (the solve is a chain of short steps)
        if (n_leaves >= 4 && n_leaves <= 64)
            pairwise_leaf_wave_kernel<<<1, 64, 0, st>>>(s->leaf_w, n_leaves, s->leaf_sums, CL, s->scales, s->pair_inv,
                                                        s->l2, s->prior, s->lr, s->leaf_raw, s->leaf_scaled);
        else
            pairwise_leaf_kernel<<<1, n_leaves <= 64 ? 64 : 256, s->pair_leaf_lds, st>>>(
                s->leaf_w, n_leaves, s->leaf_sums, CL, s->scales, s->pair_inv, s->l2, s->prior, s->lr, s->leaf_raw,
                s->leaf_scaled, s->pair_leaf_lds ? nullptr : s->pair_ws);
        HIP_TRY(hipGetLastError());
    } else {
        leaf_values_kernel<K><<<(n_leaves + 63) / 64, 64, 0, st>>>(s->leaf_sums, s->scales, n_leaves, newton,
                                                                  s->l2, s->lr, s->leaf_raw, s->leaf_scaled);
        HIP_TRY(hipGetLastError());
        if (s->ranking) {
            pairwise_center_kernel<<<1, 64, 0, st>>>(s->leaf_raw, s->leaf_sums, CL, n_leaves, s->lr,
                                                     s->leaf_scaled);
            HIP_TRY(hipGetLastError());
        }
    }
    CHECK(s->stage_end());

    HIP_TRY(hipMemcpyAsync(s->pin_out, s->out_dev, s->out_bytes, hipMemcpyDeviceToHost, st));
    return CBH_OK;
}

// Record the steady-state tree (previous leaves pending) once per host-sample mode.  A
// recording failure leaves the session eager for good; it never fails the tree.
template <int K>
void record_tree(cbh_session* s, bool use_host_sample) {
    hipGraphExec_t& ge = s->tree_graph[use_host_sample ? 1 : 0];
    hipGraph_t g = nullptr;
    if (hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
        (void)hipGetLastError();
        s->graph_off = true;
        return;
    }
    const int rc = enqueue_tree<K>(s, use_host_sample);
    const hipError_t e = hipStreamEndCapture(s->stream, &g);
    if (rc != CBH_OK || e != hipSuccess || !g || hipGraphInstantiateWithFlags(&ge, g, 0) != hipSuccess) {
        (void)hipGetLastError();
        ge = nullptr;
        s->graph_off = true;
    }
    if (g) (void)hipGraphDestroy(g);
}

template <int K>
int grow_impl(cbh_session* s, const SampleParams& smp, bool use_host_sample,
              std::vector<SplitRec>& splits_out, std::vector<LevelPlan>& plans_out,
              Bounds& bounds_out, std::vector<double>& leaf_out) {
    hipStream_t st = s->stream;
    *s->pin_smp = smp;
    HIP_TRY(hipMemcpyAsync(s->smp_dev, s->pin_smp, sizeof(SampleParams), hipMemcpyHostToDevice, st));
    // replay the recorded tree when nothing differs from it: previous leaves pending, no
    // per-stage events
    // a CTR session replays once every CTR group is in the model (no per-level host step left)
    const bool ctr_static = !s->ctr_n || s->ctr_dev || (ctr_all_used(s) && s->fweight_one);
    if (s->ctr_dev) {   // the groups earlier trees used (and whether all are), for this tree
        std::copy(s->ctr_used.begin(), s->ctr_used.end(), s->pin_ctr_used);
        s->pin_ctr_used[s->ctr_n] = ctr_all_used(s) ? 1 : 0;   // then no phantom count is needed
        HIP_TRY(hipMemcpyAsync(s->ctr_used_dev, s->pin_ctr_used, s->ctr_n + 1, hipMemcpyHostToDevice, st));
    }
    const bool replay = s->pending && !s->cfg.profile && !s->graph_off && ctr_static && !s->hist_cap;
    hipGraphExec_t& ge = s->tree_graph[use_host_sample ? 1 : 0];
    if (replay && !ge) record_tree<K>(s, use_host_sample);
    if (replay && ge) {
        HIP_TRY(hipGraphLaunch(ge, st));
    } else {
        CHECK(enqueue_tree<K>(s, use_host_sample));
    }
    s->pending = true;
    if (s->overlap_fn) s->overlap_fn(s->overlap_arg);   // host work while the tree grows
    HIP_TRY(hipStreamSynchronize(st));
    const size_t n_leaves = (size_t)1 << s->depth;
    splits_out.assign(s->pin_splits, s->pin_splits + s->depth);
    plans_out.assign(s->pin_plans, s->pin_plans + s->depth);
    bounds_out = *s->pin_bounds;
    leaf_out.assign(s->pin_leaves, s->pin_leaves + n_leaves * K);
    if (bounds_out.device_err) {   // a bounded wait of the tree gave up: its splits are not valid
        s->pending = false;
        return fail(CBH_ERR_DEVICE, "the chained split scorer's wait for its turn ran out");
    }
    // a level without a candidate split: the tree is not part of the model (CbError::Degenerate
    // leaves it untouched), so its leaves are never applied and its CTR groups stay unused
    for (uint32_t l = 0; l < s->depth; ++l)
        if (!splits_out[l].valid) {
            s->pending = false;
            return fail(CBH_ERR_DEGENERATE, "no candidate split at level " + std::to_string(l));
        }
    for (const SplitRec& sp : splits_out)   // groups used by this tree (ProcessCtrSplit)
        if (s->ctr_n && sp.feature >= s->F - s->ctr_n) s->ctr_used[s->ctr_group[sp.feature - (s->F - s->ctr_n)]] = 1;
    return CBH_OK;
}

// The CTR scoring state of a session whose last m features are CTR columns and whose
// ctr_avg holds the averaging bins (cbh_session_set_ctr and the device CTR config at open).
int install_ctr(cbh_session* s, uint32_t m, const uint32_t* bucket_count, const uint32_t* weight_group,
                uint32_t n_cat, const uint32_t* const* cat_cols, const uint32_t* cat_bucket_count, double msr) {
    const uint64_t n = s->n;
    const uint32_t fc0 = s->F - m;
    for (uint32_t f = fc0; f < s->F; ++f)
        if (!s->one_hot_host.empty() && s->one_hot_host[f])
            return fail(CBH_ERR_UNSUPPORTED, "a CTR column cannot be one-hot");
    for (uint32_t c = 0; c < m; ++c)
        if (weight_group[c] >= m) return fail(CBH_ERR_OUT_OF_RANGE, "weight_group >= n_ctr");
    const uint32_t lmax = 1u << (s->depth - 1);
    uint64_t words = 0;
    for (uint32_t c = 0; c < n_cat; ++c)
        words += kPhantomBlocks * (((uint64_t)cat_bucket_count[c] * lmax + 31) / 32);
    CHECK(dalloc(&s->fweight, s->F));
    s->fweight_host.assign(s->F, 1.0);
    HIP_TRY(hipMemcpy(s->fweight, s->fweight_host.data(), sizeof(double) * s->F, hipMemcpyHostToDevice));
    if (n_cat) {
        // the phantom bitmaps read every bucket of every column once a level: 16-bit buckets
        // when every column has fewer than 65536
        bool narrow = true;
        for (uint32_t c = 0; c < n_cat; ++c) narrow = narrow && cat_bucket_count[c] <= 65536u;
        if (narrow) {
            CHECK(dalloc(&s->cat_bk16, (size_t)n_cat * n));
            std::vector<uint16_t> col(n);
            for (uint32_t c = 0; c < n_cat; ++c) {
                for (uint64_t i = 0; i < n; ++i) col[i] = (uint16_t)cat_cols[c][i];
                HIP_TRY(hipMemcpy(s->cat_bk16 + (size_t)c * n, col.data(), sizeof(uint16_t) * n, hipMemcpyHostToDevice));
            }
        } else {
            CHECK(dalloc(&s->cat_bk, (size_t)n_cat * n));
            for (uint32_t c = 0; c < n_cat; ++c)
                HIP_TRY(hipMemcpy(s->cat_bk + (size_t)c * n, cat_cols[c], sizeof(uint32_t) * n, hipMemcpyHostToDevice));
        }
        CHECK(dalloc(&s->cat_nb_dev, n_cat));
        HIP_TRY(hipMemcpy(s->cat_nb_dev, cat_bucket_count, sizeof(uint32_t) * n_cat, hipMemcpyHostToDevice));
        CHECK(dalloc(&s->phantom_off, n_cat));
        CHECK(dalloc(&s->phantom_bits, std::max<uint64_t>(words, 1)));
        CHECK(dalloc(&s->phantom_cnt, n_cat));
    }
    s->ctr_bc.assign(bucket_count, bucket_count + m);
    s->ctr_group.assign(weight_group, weight_group + m);
    s->ctr_used.assign(m, 0);
    s->ctr_eligible_max = 1;
    for (uint32_t v : s->ctr_bc) s->ctr_eligible_max = std::max<uint64_t>(s->ctr_eligible_max, v);
    HIP_TRY(hipFuncSetAttribute((const void*)phantom_bits_kernel<uint16_t>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)(kPhantomLdsWords * sizeof(uint32_t))));
    HIP_TRY(hipFuncSetAttribute((const void*)phantom_bits_kernel<uint32_t>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)(kPhantomLdsWords * sizeof(uint32_t))));
    s->cat_n = n_cat;
    s->cat_nb.assign(cat_bucket_count, cat_bucket_count + n_cat);
    s->msr = msr;
    s->ctr_n = m;
    // device weights when the pow table stays modest: counts reachable at any level are the
    // eligible maximum and the phantom counts, at most (float leaves) x (buckets)
    {
        uint64_t nb_max = 0;
        for (uint32_t v : s->cat_nb) nb_max = std::max<uint64_t>(nb_max, v);
        const uint64_t m_lo = s->ctr_eligible_max;
        const uint64_t m_hi = std::max<uint64_t>(m_lo, (uint64_t)lmax * nb_max);
        const uint64_t span = m_hi - m_lo + 1;
        // CBH_CTR_WEIGHTS=host keeps the per-level host step (a test knob for that path)
        const char* cw = std::getenv("CBH_CTR_WEIGHTS");
        const bool host_only = cw && std::string(cw) == "host";
        if (!host_only && (uint64_t)m * span <= (32ull << 20)) {
            std::vector<double> table((size_t)m * span);
            for (uint32_t c = 0; c < m; ++c)
                for (uint64_t k = 0; k < span; ++k)
                    table[(size_t)c * span + k] =
                        std::pow(1.0 + (double)s->ctr_bc[c] / (double)(m_lo + k), -s->msr);
            CHECK(dalloc(&s->ctr_pow, table.size()));
            HIP_TRY(hipMemcpy(s->ctr_pow, table.data(), sizeof(double) * table.size(), hipMemcpyHostToDevice));
            CHECK(dalloc(&s->ctr_group_dev, m));
            HIP_TRY(hipMemcpy(s->ctr_group_dev, s->ctr_group.data(), sizeof(uint32_t) * m, hipMemcpyHostToDevice));
            CHECK(dalloc(&s->ctr_used_dev, m + 1));   // [m] by group, then the all-used flag
            HIP_TRY(hipHostMalloc((void**)&s->pin_ctr_used, m + 1, hipHostMallocDefault));
            if (s->cat_n) {
                std::vector<uint64_t> offs((size_t)s->depth * s->cat_n, 0);
                for (uint32_t lv = 1; lv < s->depth; ++lv) {
                    uint64_t w = 0;
                    for (uint32_t c = 0; c < s->cat_n; ++c) {
                        offs[(size_t)lv * s->cat_n + c] = w;
                        w += kPhantomBlocks * (((uint64_t)s->cat_nb[c] * (1u << lv) + 31) / 32);
                    }
                }
                CHECK(dalloc(&s->phantom_off_lv, offs.size()));
                HIP_TRY(hipMemcpy(s->phantom_off_lv, offs.data(), sizeof(uint64_t) * offs.size(), hipMemcpyHostToDevice));
            }
            s->ctr_m_lo = m_lo;
            s->ctr_m_hi = m_hi;
            s->ctr_dev = true;
        }
    }
    return CBH_OK;
}


}  // namespace

extern "C" {

const char* cbh_last_error(void) { return g_last_error.c_str(); }

const char* cbh_version(void) { return "cbhip 0.1 gfx950"; }

int cbh_session_begin(const cbh_config* cfg, const uint32_t* bins_fm, const double* weight,
                      uint64_t n, uint32_t n_features, uint32_t n_bins, double learning_rate,
                      double scaled_l2, cbh_session** out) {
    return session_begin_impl<uint32_t>(cfg, bins_fm, weight, n, n_features, n_bins, learning_rate,
                                        scaled_l2, out);
}

int cbh_session_begin_u8(const cbh_config* cfg, const uint8_t* bins_fm, const double* weight,
                         uint64_t n, uint32_t n_features, uint32_t n_bins, double learning_rate,
                         double scaled_l2, cbh_session** out) {
    return session_begin_impl<uint8_t>(cfg, bins_fm, weight, n, n_features, n_bins, learning_rate,
                                       scaled_l2, out);
}

int cbh_session_begin_raw(const cbh_config* cfg, const float* const* columns, const double* const* borders,
                          const uint32_t* n_borders, const double* weight, uint64_t n, uint32_t n_features,
                          uint32_t n_bins, double learning_rate, double scaled_l2, cbh_session** out) {
    return session_begin_raw_impl(cfg, columns, borders, n_borders, weight, n, n_features, n_bins,
                                  learning_rate, scaled_l2, out);
}

int cbh_session_grow(cbh_session* s, const double* approx, const double* target, uint64_t n,
                     const double* sample, uint64_t n_sample, const cbh_tree_sampling* sampling,
                     const cbh_family* family, cbh_tree_out* out) {
    if (!s) return fail(CBH_ERR_INVALID_ARG, "session is null");
    if (family && family->kind == CBH_FAMILY_MULTI_OUTPUT) {
        // FamilyTreeArgs::MultiOutput (runtime.rs:935-950): the dim-major K x n approximant of
        // this tree, the same upload as the approx argument
        if (!family->approx_k) return fail(CBH_ERR_INVALID_ARG, "MultiOutput approx_k is null");
        if (family->approx_dim != s->K)
            return fail(CBH_ERR_LENGTH_MISMATCH, "MultiOutput approx_dim differs from the session's approx_dim");
        if (approx && approx != family->approx_k)
            return fail(CBH_ERR_INVALID_ARG, "the approximant is given both as approx and as MultiOutput approx_k");
        approx = family->approx_k;
        family = nullptr;
    }
    if (family && family->kind != CBH_FAMILY_PAIRWISE) return fail(CBH_ERR_INVALID_ARG, "unknown family kind");
    if (family && !s->ranking) return fail(CBH_ERR_INVALID_ARG, "a family descriptor is given to a pointwise session");
    if (s->pairwise && (n_sample != 0 || (sampling && sampling->kind != CBH_BOOT_NO)))
        return fail(CBH_ERR_UNSUPPORTED, "PairLogitPairwise scores unsampled derivatives (no bootstrap)");
    if (s->ranking) {
        if (n != s->n) return fail(CBH_ERR_LENGTH_MISMATCH, "n differs from the session's row count");
        if (family) CHECK(upload_pairs(s, family));
        if (!s->pairs_set) return fail(CBH_ERR_INVALID_ARG, "a pair loss needs the pairs (family) on its first grow");
    }
    if (!out || !out->split_feature || !out->split_bin || !out->leaf_values)
        return fail(CBH_ERR_INVALID_ARG, "tree output buffers are null");
    if (n != s->n) return fail(CBH_ERR_LENGTH_MISMATCH, "n differs from the session's row count");
    if (n_sample != 0 && n_sample != n)
        return fail(CBH_ERR_LENGTH_MISMATCH, "sample must be empty or of length n (runtime.rs:1605)");
    if (n_sample != 0 && !sample) return fail(CBH_ERR_INVALID_ARG, "sample is null");
    if (n_sample != 0 && !s->cfg.sample_from_host)
        return fail(CBH_ERR_INVALID_ARG, "host sample given to a session without sample_from_host");
    if (s->count && sampling && sampling->kind == CBH_BOOT_BAYESIAN)
        return fail(CBH_ERR_INVALID_ARG, "a session configured without Bayesian bootstrap got a Bayesian sample");
    if (n_sample != 0 && sampling && sampling->kind != CBH_BOOT_NO)
        return fail(CBH_ERR_INVALID_ARG, "host sample and device sampling are mutually exclusive");
    if (s->w_static && sampling &&
        ((sampling->kind == CBH_BOOT_BAYESIAN && sampling->bagging_temperature != 0.0f) ||
         (sampling->kind == CBH_BOOT_BERNOULLI && sampling->subsample < 1.0))) {
        // a per-tree sample in a session opened without bootstrap: the weight channel changes from
        // tree to tree, so its level-0 cache and the trees recorded with it are dropped
        s->w_static = s->w0_ready = false;
        for (hipGraphExec_t& g : s->tree_graph)
            if (g) {
                (void)hipGraphExecDestroy(g);
                g = nullptr;
            }
    }
    hipStream_t st = s->stream;
    if (target) {
        HIP_TRY(hipMemcpyAsync(s->target, target, sizeof(double) * n, hipMemcpyHostToDevice, st));
        s->target_set = true;
    }
    if (!s->target_set) return fail(CBH_ERR_INVALID_ARG, "target was never provided");
    if (approx) {
        HIP_TRY(hipMemcpyAsync(s->approx, approx, sizeof(double) * n * s->K, hipMemcpyHostToDevice, st));
        s->pending = false;
    }
    if (n_sample) {
        if (!s->host_sample) CHECK(dalloc(&s->host_sample, n));
        HIP_TRY(hipMemcpyAsync(s->host_sample, sample, sizeof(double) * n, hipMemcpyHostToDevice, st));
    }
    SampleParams smp{};
    if (sampling && sampling->kind != CBH_BOOT_NO) {
        smp.kind = sampling->kind;
        smp.temperature = sampling->bagging_temperature;
        smp.rate = (double)(float)sampling->subsample;
        smp.bayes_seed = sampling->bayesian_seed;
        smp.bern.x1 = sampling->bernoulli_state[0];
        smp.bern.c1 = sampling->bernoulli_state[1];
        smp.bern.x2 = sampling->bernoulli_state[2];
        smp.bern.c2 = sampling->bernoulli_state[3];
        if (smp.kind == CBH_BOOT_BERNOULLI && sampling->subsample >= 1.0) smp.kind = 0;
        if (smp.kind == CBH_BOOT_BAYESIAN && sampling->bagging_temperature == 0.0f) smp.kind = 0;
    }
    std::vector<SplitRec> splits;
    std::vector<LevelPlan> plans;
    Bounds bounds{};
    std::vector<double> leaves;
    int rc = with_k((int)s->K, [&](auto kc) {
        constexpr int K = decltype(kc)::value;
        return grow_impl<K>(s, smp, n_sample != 0, splits, plans, bounds, leaves);
    });
    if (rc != CBH_OK) return rc;
    for (uint32_t l = 0; l < s->depth; ++l) {
        out->split_feature[l] = splits[l].feature;
        out->split_bin[l] = splits[l].bin;
        if (out->split_one_hot) out->split_one_hot[l] = (uint8_t)splits[l].one_hot;
        if (out->split_score) out->split_score[l] = splits[l].score;
    }
    std::memcpy(out->leaf_values, leaves.data(), sizeof(double) * leaves.size());
    if (out->leaf_of) {
        std::vector<uint16_t> lf(n);
        HIP_TRY(hipMemcpy(lf.data(), s->leaf, sizeof(uint16_t) * n, hipMemcpyDeviceToHost));
        for (uint64_t i = 0; i < n; ++i) out->leaf_of[i] = lf[i] & 0x7FFFu;
    }
    // traffic accounting of the fill launches (algorithmic bytes per launch)
    // (sparse entries: the first 16 codes of every tile, 32 bytes; second slots not counted)
    const double wbytes = s->pks ? 32.0 * s->pkk_tiles : 4.0 * s->W,
                 sbytes = (s->packed || s->count) ? 8.0 : s->pkk ? 8.0 * ((s->C + 1) / 2) : 8.0 * s->C;
    const double per_leaf_bytes = (double)s->F * s->B * s->C * 8.0;
    for (uint32_t l = 0; l < s->depth; ++l) {
        const uint64_t V = l == 0 ? bounds.sampled_rows : plans[l - 1].rows;
        const uint32_t built = l == 0 ? 1u : (1u << (l - 1));
        s->stats.fill_launches += 1;
        s->stats.fill_rows += V;
        s->stats.fill_row_features += V * s->F;
        if (!s->use_skip) s->stats.fill_lane_atomics += V * s->F * fill_atomics_per_entry(s, l);
        s->stats.fill_bytes += (double)V * (wbytes + sbytes + (l == 0 ? 0.0 : 4.0)) + built * per_leaf_bytes;
    }
    s->stats.trees += 1;
    return s->collect_timers();
}

int cbh_session_read_approx(cbh_session* s, double* approx_out, uint64_t n_times_k) {
    if (!s || !approx_out) return fail(CBH_ERR_INVALID_ARG, "null argument");
    if (n_times_k != s->n * s->K) return fail(CBH_ERR_LENGTH_MISMATCH, "approx buffer size != n*K");
    if (s->pending) {
        // apply the last tree: the prepare kernel does it as part of the next tree, so run
        // just its update arm here with an inert sample
        int rc = with_k((int)s->K, [&](auto kc) {
            constexpr int K = decltype(kc)::value;
            prepare_kernel<K><<<grid_for(s->n, 256, kPrepBlocks), 256, 0, s->stream>>>(
                s->n, s->cfg.loss == CBH_LOSS_RMSE ? 0 : 1, s->approx, s->target, s->weight, s->leaf,
                s->leaf_scaled, s->smp_dev + 1, s->jt(), nullptr, s->sstat, 0, s->partials, nullptr,
                nullptr);
            HIP_TRY(hipGetLastError());
            return CBH_OK;
        });
        if (rc != CBH_OK) return rc;
        s->pending = false;
    }
    HIP_TRY(hipMemcpyAsync(approx_out, s->approx, sizeof(double) * n_times_k, hipMemcpyDeviceToHost, s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    return CBH_OK;
}

int cbh_session_stats(const cbh_session* s, cbh_stats* out) {
    if (!s || !out) return fail(CBH_ERR_INVALID_ARG, "null argument");
    *out = s->stats;
    out->skip_features = s->n_skip;
    out->fill_mode = s->packed ? 1u : s->tiled ? 2u : s->pks ? 4u : s->pkk ? 3u : s->count ? 5u : 0u;
    out->fill_pack_bits = (s->packed || s->pkk) ? s->pack_bits : 0;
    Scales sc{};
    if (s->scales && s->stats.trees) {
        HIP_TRY(hipStreamSynchronize(s->stream));
        HIP_TRY(hipMemcpy(&sc, s->scales, sizeof(Scales), hipMemcpyDeviceToHost));
    }
    out->score_shift_der = sc.shift[kScoreDer];
    out->score_shift_w = sc.shift[kScoreW];
    out->fill_entries = out->fill_row_features;
    if (s->use_skip) {   // counted in profiled trees only (0 without them)
        unsigned long long e[2] = {0, 0};
        if (s->fill_ent) {
            HIP_TRY(hipStreamSynchronize(s->stream));
            HIP_TRY(hipMemcpy(e, s->fill_ent, sizeof(e), hipMemcpyDeviceToHost));
        }
        out->fill_entries = e[0];
        out->fill_lane_atomics = e[1];
    }
    return CBH_OK;
}

void cbh_session_reset_stats(cbh_session* s) {
    if (!s) return;
    s->stats = cbh_stats{};
    if (s->fill_ent) (void)hipMemsetAsync(s->fill_ent, 0, 2 * sizeof(unsigned long long), s->stream);
}

int cbh_session_set_ctr(cbh_session* s, const cbh_ctr_info* info) {
    if (!s || !info) return fail(CBH_ERR_INVALID_ARG, "null argument");
    const uint64_t n = s->n;
    const uint32_t m = info->n_ctr;
    if (m == 0 || m > s->F) return fail(CBH_ERR_OUT_OF_RANGE, "n_ctr must be 1..n_features");
    if (s->ranking) return fail(CBH_ERR_UNSUPPORTED, "CTR columns are not covered with pair losses");
    if (s->ctr_n) return fail(CBH_ERR_INVALID_ARG, "the CTR columns are already set");
    if (!info->averaging_bins || !info->bucket_count || !info->weight_group || (info->n_cat && !info->cat_buckets) ||
        (info->n_cat && !info->cat_bucket_count))
        return fail(CBH_ERR_INVALID_ARG, "null CTR array");
    for (uint64_t i = 0, total = (uint64_t)m * n; i < total; ++i)
        if (info->averaging_bins[i] >= s->B) return fail(CBH_ERR_OUT_OF_RANGE, "averaging bin >= n_bins");
    std::vector<const uint32_t*> cat_cols(info->n_cat);
    for (uint32_t c = 0; c < info->n_cat; ++c) cat_cols[c] = info->cat_buckets + (size_t)c * n;
    for (uint32_t c = 0; c < info->n_cat; ++c)
        for (uint64_t i = 0; i < n; ++i)
            if (cat_cols[c][i] >= info->cat_bucket_count[c])
                return fail(CBH_ERR_OUT_OF_RANGE, "categorical bucket >= its bucket count");
    CHECK(dalloc(&s->ctr_avg, (size_t)m * n));
    HIP_TRY(hipMemcpy(s->ctr_avg, info->averaging_bins, (size_t)m * n, hipMemcpyHostToDevice));
    const int rc = install_ctr(s, m, info->bucket_count, info->weight_group, info->n_cat, cat_cols.data(),
                               info->cat_bucket_count, info->model_size_reg);
    if (rc != CBH_OK) dfree(s->ctr_avg);
    return rc;
}

int cbh_session_read_ctr_bins(const cbh_session* s, int32_t averaging, uint8_t* out, uint64_t n_times_ctr) {
    if (!s || !out) return fail(CBH_ERR_INVALID_ARG, "null argument");
    if (s->ctr_n == 0) return fail(CBH_ERR_INVALID_ARG, "the session has no CTR columns");
    const size_t total = (size_t)s->ctr_n * s->n;
    if (n_times_ctr != total) return fail(CBH_ERR_LENGTH_MISMATCH, "out must hold n_ctr * n bins");
    const uint8_t* src = averaging ? s->ctr_avg : s->cols + (size_t)(s->F - s->ctr_n) * s->n;
    HIP_TRY(hipStreamSynchronize(s->stream));
    HIP_TRY(hipMemcpy(out, src, total, hipMemcpyDeviceToHost));
    return CBH_OK;
}

// The driver's host work for the next cbh_session_grow calls, run once the tree is launched and
// before the wait for it (null: none).
void cbh_internal_set_overlap(cbh_session* s, void (*fn)(void*), void* arg) {
    if (!s) return;
    s->overlap_fn = fn;
    s->overlap_arg = arg;
}

int cbh_session_set_profile(cbh_session* s, int32_t on) {
    if (!s) return fail(CBH_ERR_INVALID_ARG, "session is null");
    s->cfg.profile = on ? 1 : 0;
    return CBH_OK;
}

int cbh_session_capture_hists(cbh_session* s, int32_t on) {
    if (!s) return fail(CBH_ERR_INVALID_ARG, "session is null");
    if (s->pairwise) return fail(CBH_ERR_UNSUPPORTED, "pairwise sessions score pair statistics");
    if (!on) {
        dfree(s->hist_cap);
        return CBH_OK;
    }
    if (s->hist_cap) return CBH_OK;
    const size_t per_leaf = (size_t)s->F * s->B * s->C;
    size_t off = 0;
    for (uint32_t l = 0; l < s->depth; ++l) {
        s->hist_cap_off[l] = off;
        off += per_leaf << l;
    }
    s->hist_cap_off[s->depth] = off;
    return dalloc(&s->hist_cap, off);
}

int cbh_session_level_hist(const cbh_session* s, uint32_t level, double* out, uint64_t n_cells) {
    if (!s || !out) return fail(CBH_ERR_INVALID_ARG, "null argument");
    if (!s->hist_cap) return fail(CBH_ERR_INVALID_ARG, "histogram capture is off");
    if (level >= s->depth) return fail(CBH_ERR_OUT_OF_RANGE, "level >= depth");
    const uint32_t F = s->F, B = s->B, C = s->C;
    const size_t cells = ((size_t)F * B * C) << level;
    if (n_cells != cells) return fail(CBH_ERR_LENGTH_MISMATCH, "n_cells != 2^level * F * n_bins * C");
    HIP_TRY(hipStreamSynchronize(s->stream));
    std::vector<long long> h(cells);
    HIP_TRY(hipMemcpy(h.data(), s->hist_cap + s->hist_cap_off[level], sizeof(long long) * cells, hipMemcpyDeviceToHost));
    Scales sc{};
    HIP_TRY(hipMemcpy(&sc, s->scales, sizeof(Scales), hipMemcpyDeviceToHost));
    // [leaf][ch][f][bin] prefix sums -> [leaf][f][bin][ch] bin sums (the reference's layout,
    // histogram.rs:176-177), channel K the weight
    for (size_t leaf = 0; leaf < ((size_t)1 << level); ++leaf)
        for (uint32_t ch = 0; ch < C; ++ch) {
            const double inv = ch == C - 1 ? sc.inv[kScoreW] : sc.inv[kScoreDer];
            for (uint32_t f = 0; f < F; ++f) {
                const long long* row = h.data() + ((leaf * C + ch) * F + f) * B;
                for (uint32_t b = 0; b < B; ++b) {
                    const long long v = row[b] - (b ? row[b - 1] : 0);
                    out[((leaf * F + f) * B + b) * C + ch] = (double)v * inv;
                }
            }
        }
    return CBH_OK;
}

int cbh_session_end(cbh_session* s) {
    if (!s) return CBH_OK;
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    delete s;
    return CBH_OK;
}

int cbh_compute_gradients(int32_t loss, const double* approx, const double* target, uint64_t n,
                          uint32_t approx_dim, double* der1, double* der2);

}  // extern "C"
