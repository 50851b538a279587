// Host mirror of cb-train's device branch (crates/cb-train/src/boosting.rs:6532-7300),
// driving the session through the public C-ABI (plus one internal hook, which runs the per-tree
// draw replay while the device grows the tree).  It owns the persistent training RNG: the
// device never draws on the main stream, it receives the per-tree sampling phase
// (Bayesian seed / Bernoulli raw state) and the host advances its stream exactly as the
// CPU branch would, including the per-level draws of the perturbed level search that the
// device path does not run (crates/cb-train/src/device_draw_replay.rs).
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "../../include/cbhip.h"
#include "../../include/cbtrain.h"
#include "common.hpp"

int cbh_internal_fail(int code, const std::string& msg);  // session.hip: sets cbh_last_error()
extern "C" void cbh_internal_set_overlap(cbh_session* s, void (*fn)(void*), void* arg);  // session.hip

namespace {

constexpr int kPreTreeDraws = 2;        // boosting.rs:59
constexpr int kPostTreeExtraDraws = 2;  // boosting.rs:69

// StdNormalDistribution, Marsaglia polar (crates/cb-core/src/normal.rs:50-64).
double std_normal(cbh::Rng& r) {
    for (;;) {
        const double x = cbh::rng_real1(r) * 2.0 - 1.0;
        const double y = cbh::rng_real1(r) * 2.0 - 1.0;
        const double rr = x * x + y * y;
        if (!(rr > 1.0 || rr <= 0.0)) return x * std::sqrt(-2.0 * std::log(rr) / rr);
    }
}

}  // namespace

struct cbt_trainer {
    cbt_params p{};
    cbh_session* s = nullptr;
    uint64_t n = 0;
    uint32_t F = 0, K = 1;
    cbh::Rng rng{};
    bool draws_active = false;
    bool draws_done = false;   // this step's draw replay ran (during the device grow)
    bool first = true;
    std::vector<double> target;
    double bias = 0.0;
    std::vector<uint32_t> sf, sb;
    std::vector<uint8_t> so;
    std::vector<double> leaves;
    // pairs of a pair loss, handed to the session with the first tree
    bool ranking = false, pairs_pending = false, ctr = false;
    std::vector<uint32_t> group_off, pair_win, pair_los;
    std::vector<double> pair_w;
    ~cbt_trainer() {
        if (s) cbh_session_end(s);
    }
};

namespace {

// Shared open: validation, starting approx, scaled l2, the session config; `begin` opens
// the device session over whichever input channel the caller has.
template <typename Begin>
int trainer_open(const cbt_params* p, uint64_t n, uint32_t F, const uint32_t* real_folds,
                 const uint8_t* one_hot_flags, const cbh_device_ctr_config* ctr, const double* target,
                 const double* weight, cbt_trainer** out, Begin&& begin) {
    if (!p || !target || !out) return CBH_ERR_INVALID_ARG;
    *out = nullptr;
    bool any_one_hot = false;
    for (uint32_t f = 0; one_hot_flags && f < F; ++f) any_one_hot |= one_hot_flags[f] != 0;
    // one-hot columns with active RNG draws are refused (boosting.rs:5744-5756)
    if (any_one_hot && p->bootstrap_type != CBH_BOOT_NO)
        return cbh_internal_fail(CBH_ERR_UNSUPPORTED,
                                 "one-hot columns are not supported with bootstrap_type != No "
                                 "(the per-level RNG draw accounting of one-hot candidates is unset)");
    // PairLogitPairwise scores the unsampled derivatives (boosting.rs:7877-7905)
    if (p->loss == CBH_LOSS_PAIRLOGIT_PAIRWISE && p->bootstrap_type != CBH_BOOT_NO)
        return cbh_internal_fail(CBH_ERR_UNSUPPORTED, "PairLogitPairwise is covered without bootstrap");
    std::unique_ptr<cbt_trainer> t(new cbt_trainer());
    t->p = *p;
    // the learning rate that multiplies every leaf is the f32-representable one
    // (boosting.rs:4958); the session applies the same value to the resident approx
    t->p.learning_rate = (double)(float)p->learning_rate;
    t->n = n;
    t->F = F;
    t->K = p->loss == CBH_LOSS_MULTICLASS ? (uint32_t)p->approx_dim : 1u;
    t->target.assign(target, target + n);
    // starting approx: RMSE + boost_from_average -> mean target (boosting.rs:1871-1877)
    if (p->boost_from_average && p->loss == CBH_LOSS_RMSE && n > 0) {
        double s = 0.0;
        for (uint64_t i = 0; i < n; ++i) s += target[i];
        t->bias = s / (double)n;
    }
    double sum_w = 0.0;
    for (uint64_t i = 0; i < n; ++i) sum_w += weight ? weight[i] : 1.0;
    const double scaled_l2 = p->l2_leaf_reg * (sum_w / (double)n);  // scale_l2_reg
    cbh_config cfg{};
    cfg.loss = p->loss;
    cfg.score_function = p->score_function;
    cfg.leaf_method = p->leaf_method;
    cfg.depth = p->depth;
    cfg.boosting_type_is_plain = 1;
    cfg.fold_count = 1;
    cfg.approx_dim = (int32_t)t->K;
    cfg.bootstrap_type = p->bootstrap_type;
    cfg.sample_from_host = 0;
    cfg.sample_rate = (float)p->subsample;
    cfg.bagging_temperature = p->bagging_temperature;
    cfg.profile = p->profile;
    cfg.bias = t->bias;
    cfg.rng_seed = p->random_seed;
    cfg.one_hot_flags = one_hot_flags;
    cfg.real_folds = real_folds;
    cfg.pairwise_non_diag_reg = p->pairwise_non_diag_reg;
    cfg.ctr = ctr;
    t->ranking = p->loss == CBH_LOSS_PAIRLOGIT || p->loss == CBH_LOSS_PAIRLOGIT_PAIRWISE;
    int rc = begin(&cfg, t->p.learning_rate, scaled_l2, &t->s);
    if (rc != CBH_OK) return rc;
    if (ctr) {   // the session appended the CTR columns after the F base features
        t->F = F + ctr->n_columns;
        t->ctr = true;
    }
    t->rng = cbh::rng_from_seed(p->random_seed);
    t->draws_active = p->bootstrap_type != CBH_BOOT_NO;
    t->sf.resize(p->depth);
    t->sb.resize(p->depth);
    t->so.resize(p->depth);
    t->leaves.resize(((size_t)1 << p->depth) * t->K);
    *out = t.release();
    return CBH_OK;
}

}  // namespace

extern "C" {

int cbt_open(const cbt_params* p, const uint8_t* bins_fm, uint64_t n, uint32_t F, uint32_t n_bins,
             const uint32_t* real_folds, const uint8_t* one_hot_flags, const double* target,
             const double* weight, cbt_trainer** out) {
    if (!bins_fm) return CBH_ERR_INVALID_ARG;
    return trainer_open(p, n, F, real_folds, one_hot_flags, nullptr, target, weight, out,
                        [&](const cbh_config* cfg, double lr, double l2, cbh_session** s) {
                            return cbh_session_begin_u8(cfg, bins_fm, weight, n, F, n_bins, lr, l2, s);
                        });
}

int cbt_open_raw(const cbt_params* p, const float* const* columns, const double* const* borders,
                 const uint32_t* n_borders, uint64_t n, uint32_t F, const double* target,
                 const double* weight, cbt_trainer** out) {
    if (!columns || !borders || !n_borders) return CBH_ERR_INVALID_ARG;
    uint32_t n_bins = 1;
    for (uint32_t f = 0; f < F; ++f) n_bins = std::max(n_bins, n_borders[f] + 1);
    return trainer_open(p, n, F, nullptr, nullptr, nullptr, target, weight, out,
                        [&](const cbh_config* cfg, double lr, double l2, cbh_session** s) {
                            return cbh_session_begin_raw(cfg, columns, borders, n_borders, weight, n, F,
                                                         n_bins, lr, l2, s);
                        });
}

int cbt_open_ctr(const cbt_params* p, const uint8_t* bins_fm, uint64_t n, uint32_t F, uint32_t n_bins,
                 const uint32_t* real_folds, const uint8_t* one_hot_flags, const cbh_device_ctr_config* ctr,
                 const double* target, const double* weight, cbt_trainer** out) {
    if (!bins_fm || !ctr) return CBH_ERR_INVALID_ARG;
    return trainer_open(p, n, F, real_folds, one_hot_flags, ctr, target, weight, out,
                        [&](const cbh_config* cfg, double lr, double l2, cbh_session** s) {
                            return cbh_session_begin_u8(cfg, bins_fm, weight, n, F, n_bins, lr, l2, s);
                        });
}

int cbt_set_pairs(cbt_trainer* t, const uint32_t* group_offsets, uint32_t n_groups,
                  const uint32_t* pair_winner, const uint32_t* pair_loser, const double* pair_weight,
                  uint64_t n_pairs) {
    if (!t || !group_offsets || (n_pairs && (!pair_winner || !pair_loser))) return CBH_ERR_INVALID_ARG;
    if (!t->ranking) return cbh_internal_fail(CBH_ERR_INVALID_ARG, "pairs given to a pointwise loss");
    t->group_off.assign(group_offsets, group_offsets + (size_t)n_groups + 1);
    t->pair_win.assign(pair_winner, pair_winner + n_pairs);
    t->pair_los.assign(pair_loser, pair_loser + n_pairs);
    if (pair_weight) t->pair_w.assign(pair_weight, pair_weight + n_pairs);
    else t->pair_w.clear();
    t->pairs_pending = true;
    return CBH_OK;
}

int cbt_set_ctr(cbt_trainer* t, const cbh_ctr_info* info) {
    if (!t) return CBH_ERR_INVALID_ARG;
    if (!t->first) return cbh_internal_fail(CBH_ERR_INVALID_ARG, "CTR columns are set before the first step");
    const int rc = cbh_session_set_ctr(t->s, info);
    if (rc == CBH_OK) t->ctr = true;
    return rc;
}

// Step 3 of a tree: the per-level draws of the CPU grower's perturbed level search (none with
// CTR columns), then the post-tree draws (device_draw_replay.rs).
static void replay_draws(void* arg) {
    cbt_trainer* t = (cbt_trainer*)arg;
    for (int level = 0; level < t->p.depth && !t->ctr; ++level) {
        for (uint32_t f = 0; f < t->F; ++f) (void)cbh::rng_real1(t->rng);
        (void)cbh::rng_gen(t->rng);
        for (uint32_t f = 0; f < t->F; ++f) (void)std_normal(t->rng);
    }
    for (int k = 0; k < kPostTreeExtraDraws; ++k) (void)cbh::rng_gen(t->rng);
    t->draws_done = true;
}

int cbt_step(cbt_trainer* t, uint32_t* split_feature, uint32_t* split_bin, uint8_t* split_one_hot,
             double* leaf_values) {
    if (!t) return CBH_ERR_INVALID_ARG;
    if (t->ranking && t->first && !t->pairs_pending)
        return cbh_internal_fail(CBH_ERR_INVALID_ARG, "a pair loss needs cbt_set_pairs before the first step");
    const cbt_params& p = t->p;
    // 1a. pre-bootstrap draws (train.cpp:208,211)
    if (t->draws_active)
        for (int k = 0; k < kPreTreeDraws; ++k) (void)cbh::rng_gen(t->rng);
    // 1b. bootstrap phase on the main stream (bootstrap.rs:402-466)
    cbh_tree_sampling smp{};
    smp.kind = CBH_BOOT_NO;
    if (p.bootstrap_type == CBH_BOOT_BAYESIAN && p.bagging_temperature != 0.0f) {
        smp.kind = CBH_BOOT_BAYESIAN;
        smp.bagging_temperature = p.bagging_temperature;
        smp.bayesian_seed = cbh::rng_gen(t->rng);
    } else if (p.bootstrap_type == CBH_BOOT_BERNOULLI && p.subsample < 1.0) {
        smp.kind = CBH_BOOT_BERNOULLI;
        smp.subsample = p.subsample;
        smp.bernoulli_state[0] = t->rng.x1;
        smp.bernoulli_state[1] = t->rng.c1;
        smp.bernoulli_state[2] = t->rng.x2;
        smp.bernoulli_state[3] = t->rng.c2;
        cbh::rng_advance(t->rng, t->n);  // the n sequential real1 draws
    }
    // 2. grow on the device
    cbh_tree_out out{};
    out.split_feature = t->sf.data();
    out.split_bin = t->sb.data();
    out.split_one_hot = t->so.data();
    out.leaf_values = t->leaves.data();
    cbh_family fam{};
    if (t->pairs_pending) {
        fam.kind = CBH_FAMILY_PAIRWISE;
        fam.n_groups = (uint32_t)(t->group_off.size() - 1);
        fam.group_offsets = t->group_off.data();
        fam.pair_winner = t->pair_win.data();
        fam.pair_loser = t->pair_los.data();
        fam.pair_weight = t->pair_w.empty() ? nullptr : t->pair_w.data();
        fam.n_pairs = t->pair_win.size();
    }
    // 3. the CPU grower's per-level draws, then the post-tree draws: they depend on nothing the
    // tree computes, so they run while the device grows it (kept only if the tree is taken)
    const cbh::Rng rng_before = t->rng;
    if (t->draws_active) cbh_internal_set_overlap(t->s, &replay_draws, t);
    int rc = cbh_session_grow(t->s, nullptr, t->first ? t->target.data() : nullptr, t->n, nullptr, 0,
                              &smp, t->pairs_pending ? &fam : nullptr, &out);
    cbh_internal_set_overlap(t->s, nullptr, nullptr);
    if (rc != CBH_OK) {
        t->rng = rng_before;
        t->draws_done = false;
        return rc;
    }
    if (t->draws_active && !t->draws_done) replay_draws(t);   // (a grow that never launched)
    t->draws_done = false;
    t->first = false;
    t->pairs_pending = false;
    if (split_feature) std::memcpy(split_feature, t->sf.data(), sizeof(uint32_t) * p.depth);
    if (split_bin) std::memcpy(split_bin, t->sb.data(), sizeof(uint32_t) * p.depth);
    if (split_one_hot) std::memcpy(split_one_hot, t->so.data(), p.depth);
    if (leaf_values) {
        // model leaves: dim-major [K][leaves], scaled by the learning rate
        const size_t L = (size_t)1 << p.depth;
        for (size_t l = 0; l < L; ++l)
            for (uint32_t d = 0; d < t->K; ++d)
                leaf_values[(size_t)d * L + l] = t->leaves[l * t->K + d] * p.learning_rate;
    }
    return CBH_OK;
}

int cbt_read_approx(cbt_trainer* t, double* approx_out) {
    if (!t || !approx_out) return CBH_ERR_INVALID_ARG;
    return cbh_session_read_approx(t->s, approx_out, t->n * t->K);
}

int cbt_stats(const cbt_trainer* t, cbh_stats* out) {
    if (!t) return CBH_ERR_INVALID_ARG;
    return cbh_session_stats(t->s, out);
}

void cbt_reset_stats(cbt_trainer* t) {
    if (t) cbh_session_reset_stats(t->s);
}

int cbt_set_profile(cbt_trainer* t, int32_t on) {
    if (!t) return CBH_ERR_INVALID_ARG;
    t->p.profile = on;
    return cbh_session_set_profile(t->s, on);
}

double cbt_bias(const cbt_trainer* t) { return t ? t->bias : 0.0; }

void cbt_close(cbt_trainer* t) { delete t; }

}  // extern "C"

// Row-major f32 matrix -> per-feature columns (ingest_py.rs:157-203): threads over disjoint
// runs of rows; a block of 64 rows (64 * n_features floats, read once) is scattered to each
// column as one run of 64 consecutive floats.
int cbh_columns_from_rows(const float* rows, uint64_t n, uint32_t n_features, float* columns) {
    if (!rows || !columns) return cbh_internal_fail(CBH_ERR_INVALID_ARG, "rows and columns are required");
    if (n == 0 || n_features == 0) return CBH_OK;
    uint32_t hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (const char* e = std::getenv("OMP_NUM_THREADS")) {   // the host's CPU share, when set
        const long v = std::strtol(e, nullptr, 10);
        if (v >= 1 && (unsigned long)v < hw) hw = (uint32_t)v;
    }
    const uint64_t T = std::min<uint64_t>(hw, (n + 65535) / 65536);
    auto run = [&](uint64_t r0, uint64_t r1) {
        constexpr uint64_t kBlock = 64;
        for (uint64_t b = r0; b < r1; b += kBlock) {
            const uint64_t e = std::min(r1, b + kBlock);
            for (uint32_t f = 0; f < n_features; ++f) {
                float* dst = columns + (size_t)f * n;
                for (uint64_t r = b; r < e; ++r) dst[r] = rows[r * n_features + f];
            }
        }
    };
    if (T <= 1) {
        run(0, n);
        return CBH_OK;
    }
    std::vector<std::thread> pool;
    for (uint64_t t = 0; t < T; ++t) pool.emplace_back(run, n * t / T, n * (t + 1) / T);
    for (std::thread& th : pool) th.join();
    return CBH_OK;
}
