/*
 * cbtrain.h -- host mirror of the caller side of the seam: the device branch of
 * cb-train's boosting loop (crates/cb-train/src/boosting.rs:6532-7300) driving the
 * cbhip.h session exactly as cb_train::train does:
 *   starting approx (boosting.rs:1871), scale_l2_reg (leaf.rs:177),
 *   per tree: PRE_TREE_DRAWS, bootstrap phase on the host RNG (bootstrap.rs:402),
 *   grow_tree_on_device, replay of the CPU grower's per-level draws
 *   (crates/cb-train/src/device_draw_replay.rs), POST_TREE_EXTRA_DRAWS, model leaf
 *   values scaled by the learning rate (boosting.rs:2879-2881).
 * The reference's caller is Rust; Rust is not available in this build, so the caller is
 * restated in C++ above the C-ABI.  It only calls functions declared in cbhip.h.
 */
#ifndef CBTRAIN_H
#define CBTRAIN_H
#include <stdint.h>

#include "cbhip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int32_t loss;                 /* CBH_LOSS_* */
    int32_t score_function;       /* CBH_SCORE_* */
    int32_t leaf_method;          /* CBH_LEAF_* */
    int32_t depth;
    int32_t bootstrap_type;       /* CBH_BOOT_* */
    int32_t boost_from_average;
    int32_t approx_dim;           /* class count for MultiClass, else 1 */
    int32_t profile;
    double learning_rate;
    double l2_leaf_reg;
    double subsample;
    float bagging_temperature;
    float pad_;
    uint64_t random_seed;
    double pairwise_non_diag_reg; /* PairLogitPairwise leaf prior (0.1 by default) */
} cbt_params;

typedef struct cbt_trainer cbt_trainer;

/* Open: upload the u8 feature-major bins once (begin_device_training). */
int cbt_open(const cbt_params* p, const uint8_t* bins_fm, uint64_t n, uint32_t n_features,
             uint32_t n_bins, const uint32_t* real_folds, const uint8_t* one_hot_flags,
             const double* target, const double* weight, cbt_trainer** out);

/* Open over the raw float channel (the trainer's float-only first choice,
 * runtime.rs:1530-1545): f32 columns + per-feature borders; the device quantizes.
 * n_bins = max(n_borders) + 1; candidate folds per feature = n_borders[f] + 1. */
int cbt_open_raw(const cbt_params* p, const float* const* columns, const double* const* borders,
                 const uint32_t* n_borders, uint64_t n, uint32_t n_features, const double* target,
                 const double* weight, cbt_trainer** out);

/* Open with the device CTR config (DeviceTrainConfig.ctr, see cbh_device_ctr_config): the
 * session builds both CTR materializations on the device and appends the structure columns
 * after the n_features base features, so split features >= n_features name CTR columns
 * (in config order).  real_folds / one_hot_flags cover the base features only. */
int cbt_open_ctr(const cbt_params* p, const uint8_t* bins_fm, uint64_t n, uint32_t n_features,
                 uint32_t n_bins, const uint32_t* real_folds, const uint8_t* one_hot_flags,
                 const cbh_device_ctr_config* ctr, const double* target, const double* weight,
                 cbt_trainer** out);

/* PairLogit / PairLogitPairwise: the query groups and explicit pairs of the pool (copied;
 * call once after cbt_open, before the first cbt_step).  See cbh_family. */
int cbt_set_pairs(cbt_trainer* t, const uint32_t* group_offsets, uint32_t n_groups,
                  const uint32_t* pair_winner, const uint32_t* pair_loser, const double* pair_weight,
                  uint64_t n_pairs);

/* One boosting iteration.  Outputs (nullable): split_feature/split_bin/split_one_hot
 * [depth]; leaf_values [K][2^depth] as stored in the model (learning-rate scaled). */
/* CTR columns of the fit (cbh_session_set_ctr; call once after cbt_open, before the first
 * cbt_step).  A CTR fit consumes no per-level RNG draws (the reference's CTR-aware search,
 * tree.rs:3445-3470, draws nothing). */
int cbt_set_ctr(cbt_trainer* t, const cbh_ctr_info* info);

int cbt_step(cbt_trainer* t, uint32_t* split_feature, uint32_t* split_bin, uint8_t* split_one_hot,
             double* leaf_values);

int cbt_read_approx(cbt_trainer* t, double* approx_out);     /* [K][n] */
int cbt_stats(const cbt_trainer* t, cbh_stats* out);
void cbt_reset_stats(cbt_trainer* t);
int cbt_set_profile(cbt_trainer* t, int32_t on);   /* cbh_session_set_profile */
double cbt_bias(const cbt_trainer* t);
void cbt_close(cbt_trainer* t);

#ifdef __cplusplus
}
#endif
#endif
