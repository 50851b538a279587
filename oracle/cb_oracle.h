/*
 * cb_oracle.h -- CPU restatement of catboost_rs's oblivious-tree training path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path and the CPU speed baseline in bench.py.  Only tests/, the smoke() entry
 * of __graft_entry__.py and bench.py's cpu_baseline leg may load it; the
 * product library (catboost_rs_amd) never links, loads or calls it.
 *
 * Every function restates the reference algorithm in the same arithmetic order
 * (sequential f64 folds in object order, f32 where the reference uses f32).
 * Citations are relative to the reference checkout (crates/...).
 *
 * Pinning (what proves each part, beyond retyping):
 *   rng / std_normal      fast_ut.cpp known answers (cb-core/src/rng_test.rs)
 *   fast_logf             1206 bit vectors in cb-train/tests/fixtures/fast_approx_ref.txt
 *   grow_tree / leaves    bench/fixtures/expected_depth6_tree.json (numpy generator)
 *                         + brute-force partition scoring on tiny inputs
 *   bootstrap + boosting  upstream catboost 1.2.10 fixtures under
 *                         crates/cb-oracle/fixtures/{bootstrap/{no,bayesian,bernoulli},regression_skeleton,
 *                         binclf_skeleton} (splits, leaf values, staged approx)
 *   multiclass            crates/cb-oracle/fixtures/multiclass_softmax
 *   permutations / CTR    cb-oracle/fixtures/{plain_ctr,ordered_ctr,tensor_ctr,one_hot_cat}
 *                         permutations, cat_hash first-seen bins, the hand scenarios of
 *                         cb-train/tests/{plain,tensor}_ctr_oracle_test.rs, brute-force recounts
 */
#ifndef CB_ORACLE_H
#define CB_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* TFastRng64 state: two PCG-XSH-RR streams (x = LCG state, c = odd addend). */
typedef struct {
    uint64_t x1, c1, x2, c2;
    uint64_t calls;
} orc_rng;

enum { ORC_LOSS_RMSE = 0, ORC_LOSS_LOGLOSS = 1, ORC_LOSS_MULTICLASS = 2, ORC_LOSS_PAIRLOGIT = 3,
       ORC_LOSS_PAIRLOGIT_PAIRWISE = 4 };
enum { ORC_SCORE_COSINE = 0, ORC_SCORE_L2 = 1, ORC_SCORE_SOLAR_L2 = 2, ORC_SCORE_LOO_L2 = 3, ORC_SCORE_SAT_L2 = 4 };

/* One leaf's additive score term of the SolarL2 / LOOL2 / SatL2 calcers (score.rs:236-330):
 * der sum s and weight sum w of the leaf; no L2 regularizer. */
double orc_leaf_score_term(int32_t score_fn, double s, double w);
enum { ORC_BOOT_NO = 0, ORC_BOOT_BAYESIAN = 1, ORC_BOOT_BERNOULLI = 2 };
enum { ORC_LEAF_GRADIENT = 0, ORC_LEAF_NEWTON = 1 };

typedef struct {
    int32_t loss;            /* ORC_LOSS_* */
    int32_t score_function;  /* ORC_SCORE_* */
    int32_t bootstrap_type;  /* ORC_BOOT_* */
    int32_t leaf_method;     /* ORC_LEAF_* */
    int32_t depth;
    int32_t iterations;
    int32_t boost_from_average;
    int32_t n_threads;       /* 0 = OpenMP default */
    int32_t approx_dim;      /* 1 except MultiClass (class count) */
    int32_t pad_;
    double learning_rate;
    double l2_leaf_reg;
    double subsample;        /* Bernoulli rate */
    float bagging_temperature;
    float pad2_;
    uint64_t random_seed;
    const uint8_t* one_hot_flags; /* nullable [F]: one-hot categorical columns */
    /* PairLogit / PairLogitPairwise: explicit pairs (any order; pairs never cross groups) */
    const uint32_t* pair_winner;
    const uint32_t* pair_loser;
    const double* pair_weight;    /* nullable: weight 1 (query_info.rs:236-239) */
    uint64_t n_pairs;
    double pairwise_non_diag_reg; /* bayesian_matrix_reg, 0.1 by default (boosting.rs:1790) */
    /* CTR columns (greedy_tensor_search_oblivious_with_ctr, tree.rs:3445-3520; simple
     * projections, one learning permutation): the LAST n_ctr features of bins_fm are the CTR
     * columns materialized under the structure permutation, scored after the floats with the
     * model_size_reg weight of a projection not yet used (tree.rs:2907, :3290-3340);
     * leaf values and the approximant use the partition in which every CTR level re-tests
     * the column materialized under the averaging permutation (assign_leaf_over_ctr_columns,
     * boosting.rs:2905, :8206).  The CTR search consumes no per-level RNG draws. */
    uint32_t n_ctr;
    const uint8_t* ctr_avg_bins;      /* [n_ctr][n] */
    const uint32_t* ctr_bucket_count; /* [n_ctr] distinct buckets of each column's projection */
    const uint32_t* ctr_group;        /* [n_ctr] (ctr_type, projection) identity, < n_ctr */
    uint32_t n_cat;                   /* CTR-eligible categorical columns (phantom count) */
    const uint32_t* cat_buckets;      /* [n_cat][n] first-seen buckets */
    double model_size_reg;            /* 0.5 by default */
} orc_params;

/* out_splits feature entries of one-hot (equality) splits carry this flag bit */
#define ORC_ONE_HOT_SPLIT 0x40000000

/* ---- RNG (cb-core/src/rng.rs, normal.rs) ---- */
void orc_rng_new(orc_rng* r, uint64_t seed1, uint32_t seq1, uint64_t seed2, uint32_t seq2);
void orc_rng_from_seed(orc_rng* r, uint64_t seed);
uint64_t orc_rng_gen(orc_rng* r);
void orc_rng_advance(orc_rng* r, uint64_t delta);
double orc_rng_real1(orc_rng* r);
uint64_t orc_rng_uniform(orc_rng* r, uint64_t bound);
double orc_std_normal(orc_rng* r);
float orc_fast_logf(float v);

/* ---- bootstrap (cb-train/src/bootstrap.rs) ---- */
int orc_bootstrap(int32_t type, uint64_t n, double subsample, float temperature, orc_rng* rng,
                  double* sample_weight, uint8_t* control);

/* ---- quantization (cb-compute/src/histogram.rs:563 bin_of) ---- */
void orc_quantize(const float* values, uint64_t n, const double* borders, uint32_t n_borders,
                  uint8_t* bins_out);

/* ---- derivatives (cb-compute/src/loss.rs) ---- */
void orc_ders(int32_t loss, const double* approx, const double* target, uint64_t n,
              double* der1, double* der2);

/* ---- one oblivious tree (cb-train/src/tree.rs:704 greedy_tensor_search_oblivious_perturbed)
 *  bins_fm     feature-major u8 bins [F][n]
 *  n_borders   per-feature border count (bins used: 0..n_borders[f])
 *  score_der   dim-major score derivative channel [K][n] (already weight*sample masked)
 *  score_w     score weight channel [n]
 *  perturb_rng NULL -> plain search (no draws); else the draws of the perturbed search at
 *              random_strength = 0 are consumed on it (std_dev 0 keeps scores exact)
 *  out_splits  [depth][2] = (feature, bin_id)
 *  out_scores  [depth] winning score per level
 *  out_leaf_of [n]
 *  out_hists   nullable; per level l, (2^l * F * n_bins * (K+1)) doubles, ch 0..K-1 der, K weight
 *  one_hot     nullable [F]: one-hot columns; their candidates are the distinct bins of the
 *              column (equality splits, scored after every float candidate), reported as
 *              (feature | ORC_ONE_HOT_SPLIT, value); n_borders[f] + 1 bounds their bins
 * returns 0, or <0 on a degenerate level (no candidate). */
int orc_grow_tree(const uint8_t* bins_fm, const uint32_t* n_borders, uint64_t n, uint32_t F,
                  const double* score_der, const double* score_w, int32_t K, int32_t depth,
                  int32_t score_function, double scaled_l2, orc_rng* perturb_rng, int32_t n_threads,
                  int32_t* out_splits, double* out_scores, uint32_t* out_leaf_of,
                  double* out_hists, const uint8_t* one_hot);

/* ---- pairwise ranking (cb-compute/src/ranking_der.rs, pairwise_scoring.rs;
 *      cb-train/src/pairwise_leaves.rs, tree.rs:3790-3974) ----
 * Pair arrays are in the reference's competitor order (stable by winner). */
void orc_pairs_order(const uint32_t* winner, uint64_t m, uint64_t n, uint64_t* out_perm);
void orc_pairlogit_ders(const double* approx, uint64_t n, const uint32_t* winner,
                        const uint32_t* loser, const double* weight, uint64_t m, double* der1,
                        double* der2);
void orc_pairwise_weights(uint64_t n, const uint32_t* winner, const uint32_t* loser,
                          const double* weight, uint64_t m, double* pw);
int orc_grow_tree_pairwise(const uint8_t* bins_fm, const uint32_t* n_borders, uint64_t n,
                           uint32_t F, const double* der, const uint32_t* winner,
                           const uint32_t* loser, const double* weight, uint64_t m,
                           int32_t depth, double l2, double prior, int32_t n_threads,
                           int32_t* out_splits, double* out_scores, uint32_t* out_leaf_of);
void orc_pairwise_feature_scores(const uint8_t* col, const uint32_t* leaf_of, const double* der,
                                 uint64_t n, const uint32_t* winner, const uint32_t* loser,
                                 const double* weight, uint64_t m, int32_t P, int32_t B, double l2,
                                 double prior, double* scores);
void orc_pairwise_leaf_deltas(const uint32_t* leaf_of, uint64_t n, const double* der,
                              const uint32_t* winner, const uint32_t* loser, const double* weight,
                              uint64_t m, uint32_t n_leaves, double l2, double prior, double* out);

/* ---- border selection (cb-data/src/borders.rs) ----
 * out has room for border_count + 1 values; returns the count written. */
void orc_sample_indices_for_borders(uint64_t n, uint64_t sample_size, uint32_t* out);
uint32_t orc_select_borders_greedy(const float* column, uint64_t n, uint32_t border_count,
                                   int32_t nan_sentinel, int32_t kind, double* out);

/* ---- model apply (cb-model/src/apply.rs; device kernels.rs:629) ----
 * Float splits, CSR per tree; leaf values [(tree_leaf_offsets[t] + leaf) * K + d]; out [K][n]. */
int orc_apply_oblivious(const float* x_fm, uint64_t n, uint32_t F, const uint32_t* split_features,
                        const double* split_borders, const uint32_t* tree_split_offsets,
                        const double* leaf_values, const uint32_t* tree_leaf_offsets,
                        uint32_t n_trees, uint32_t K, const double* bias,
                        const uint8_t* nan_as_true, double* out);

/* ---- categorical inputs (cb-train/src/permutation.rs, cb-data/src/cat_hash.rs,
 *      cb-train/src/ctr/{online,calc_ctr,ctr_feature}.rs) ---- */
enum { ORC_CTR_BORDERS = 0, ORC_CTR_BUCKETS = 1, ORC_CTR_BTMV = 2, ORC_CTR_COUNTER = 4 };

/* Fisher-Yates over TFastRng64::from_seed(seed): for i in 1..n swap(i, uniform(i + 1))
 * (permutation.rs:131 create_shuffled_indices / shuffle_in_place). */
void orc_shuffled_indices(uint64_t n, uint64_t seed, uint32_t* out);
/* count permutations drawn one after another off one from_seed(seed) stream
 * (permutation.rs:236 permutations); out [count][n]. */
void orc_permutations(uint64_t n, uint32_t count, uint64_t seed, uint32_t* out);
/* First-seen dense remap of u32 keys (PerfectHash::remap, cat_hash.rs:389-479); returns the
 * number of distinct keys. */
uint32_t orc_perfect_hash(const uint32_t* keys, uint64_t n, uint32_t* bins);
/* One online CTR column (materialize_ctr_feature, ctr_feature.rs, over
 * online_class_prefix_column / online_mean_prefix / online_counter_column, online.rs;
 * value calc_ctr_online, bin calc_ctr_online_bin or its f32 twin for BTMV):
 *   bucket [n] (< n_buckets), permutation [n], target_class [n] in {0,1}
 *   out: good / total [n] (the numerator as f64 -- the f32 sum for BTMV -- and the
 *   denominator), value [n], bin [n] in [0, border_count].  All nullable except bin. */
int orc_ctr_column(int32_t ctr_type, uint32_t target_border_idx, double prior_num, double prior_denom,
                   uint32_t border_count, const uint32_t* bucket, uint32_t n_buckets, uint64_t n,
                   const uint32_t* permutation, const uint8_t* target_class, double* good,
                   int64_t* total, double* value, uint8_t* bin);

/* Per-leaf ordered sums (cb-compute/src/histogram.rs:49 reduce_leaf_stats, :97 reduce_leaf_der2). */
void orc_leaf_sums(const uint32_t* leaf_of, uint64_t n, uint32_t n_leaves, const double* der,
                   const double* weight, double* sum_der, double* sum_w);

/* ---- full boosting loop, CPU branch of cb-train/src/boosting.rs:7300-8900 ----
 *  out_splits       [iterations][depth][2]
 *  out_leaf_values  [iterations][2^depth * K]  learning-rate scaled (model leaf values)
 *  out_approx       [K][n] final raw approx (nullable)
 *  out_staged       [iterations][K][n] (nullable)
 *  out_bias         starting approx (nullable)
 * returns 0, -1 on a degenerate level, -4 for one-hot columns with active RNG draws. */
int orc_train(const orc_params* p, const uint8_t* bins_fm, const uint32_t* n_borders, uint64_t n,
              uint32_t F, const double* target, const double* weight, int32_t* out_splits,
              double* out_leaf_values, double* out_approx, double* out_staged, double* out_bias);

#ifdef __cplusplus
}
#endif
#endif
