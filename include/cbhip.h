/*
 * cbhip.h -- C-ABI of the MI355X (gfx950) oblivious-tree training path.
 *
 * This library is a drop-in device backend behind catboost_rs's compute seam
 * `trait cb_compute::Runtime` (crates/cb-compute/src/runtime.rs:1410-1651).  A thin
 * Rust crate (`HipBackend: Runtime`) binds these symbols one to one.  Plain pointers and sizes only; no HIP or torch types cross the boundary.
 *
 * Status codes: 0 = OK, 1 = DECLINED (the caller falls back to its CPU grower, as a
 * trait default returning Ok(false)/Ok(None) does), negative = error mirroring the
 * CbError variants (crates/cb-core/src/error.rs:17-117).  A thread-local message for
 * the last error is available from cbh_last_error().
 *
 * Threading: a session is driven from one thread at a time (the reference guards its
 * session with a Mutex, crates/cb-backend/src/gpu_backend.rs:53-84).  Different
 * sessions may run concurrently on different streams.
 */
#ifndef CBHIP_H
#define CBHIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes (CbError mirror) ---- */
#define CBH_OK 0
#define CBH_DECLINED 1
#define CBH_ERR_LENGTH_MISMATCH (-1) /* CbError::LengthMismatch */
#define CBH_ERR_OUT_OF_RANGE (-2)    /* CbError::OutOfRange */
#define CBH_ERR_DEGENERATE (-3)      /* CbError::Degenerate (e.g. no candidate split) */
#define CBH_ERR_UNSUPPORTED (-4)     /* CbError::Unsupported */
#define CBH_ERR_INVALID_ARG (-5)     /* CbError::InvalidArgument-style caller bug */
#define CBH_ERR_DEVICE (-6)          /* HIP runtime / allocation failure, or a kernel's bounded wait gave up */

/* ---- enums (cb-compute Loss / EScoreFunction / ELeavesEstimation / bootstrap) ---- */
enum {
    CBH_LOSS_RMSE = 0,
    CBH_LOSS_LOGLOSS = 1,
    CBH_LOSS_MULTICLASS = 2,
    CBH_LOSS_CROSSENTROPY = 3,
    CBH_LOSS_PAIRLOGIT = 4,          /* pointwise scoring over pairwise weights */
    CBH_LOSS_PAIRLOGIT_PAIRWISE = 5  /* pairwise split scoring + Cholesky leaves */
};
enum {   /* EScoreFunction (runtime.rs:834-870) arms of the device session (session.rs:1118-1128) */
    CBH_SCORE_COSINE = 0,
    CBH_SCORE_L2 = 1,
    CBH_SCORE_SOLAR_L2 = 2,   /* per leaf: w > 1e-20 ? -s^2 (1 + 2 ln(w + 1)) / w : 0 (no L2 regularizer) */
    CBH_SCORE_LOO_L2 = 3,     /* (w > 1 ? w / (w - 1) : 0)^2 * -s^2 / w, w > 0 */
    CBH_SCORE_SAT_L2 = 4      /* (w > 2 ? w (w - 2) / (w^2 - 3w + 1) : 0) * -s^2 / w, w > 0 */
};
enum { CBH_LEAF_GRADIENT = 0, CBH_LEAF_NEWTON = 1, CBH_LEAF_SIMPLE = 2 };
enum { CBH_BOOT_NO = 0, CBH_BOOT_BAYESIAN = 1, CBH_BOOT_BERNOULLI = 2 };
/* float-feature preparation (crates/cb-data/src/borders.rs, nan_mode.rs) */
enum { CBH_BORDERS_GREEDY_LOGSUM = 0, CBH_BORDERS_GREEDY_MIN_ENTROPY = 1 };
enum { CBH_NAN_MIN = 0, CBH_NAN_MAX = 1, CBH_NAN_FORBIDDEN = 2 };
/* CTR types (ECtrType, crates/cb-train/src/ctr/mod.rs; the CPU-task subset) */
enum { CBH_CTR_BORDERS = 0, CBH_CTR_BUCKETS = 1, CBH_CTR_BTMV = 2, CBH_CTR_COUNTER = 4 };

/* The device CTR config (DeviceCtrConfig, runtime.rs:1174-1200); defined below. */
typedef struct cbh_device_ctr_config cbh_device_ctr_config;

/* Mirrors DeviceTrainConfig (runtime.rs:1260-1341) plus the scalar arguments of
 * begin_device_training (runtime.rs:1497-1529).  Fields the device path does not cover
 * (non-symmetric policies, ordered boosting, exact leaves) are absent: a caller that needs
 * them must not open a session (the reference declines the same). */
typedef struct {
    int32_t loss;                 /* CBH_LOSS_* */
    int32_t score_function;       /* CBH_SCORE_* */
    int32_t leaf_method;          /* CBH_LEAF_* (Simple == Gradient, leaf.rs:242) */
    int32_t depth;                /* 1..8 */
    int32_t boosting_type_is_plain; /* must be 1 (ordered boosting declines) */
    int32_t fold_count;           /* must be 1 */
    int32_t approx_dim;           /* 1, or the class count for MultiClass */
    int32_t bootstrap_type;       /* CBH_BOOT_* (describes the sampler; see grow) */
    int32_t sample_from_host;     /* 1: grow receives a host multiplier (len n) */
    float sample_rate;            /* Bernoulli subsample */
    float bagging_temperature;    /* Bayesian temperature */
    int32_t profile;              /* 1: time every kernel with HIP events */
    double bias;                  /* starting approximant (boost_from_average) */
    uint64_t rng_seed;            /* informational; draws come from the host RNG phase */
    /* one-hot columns (DeviceTrainConfig.one_hot_flags / real_folds, runtime.rs:1315-1332;
     * real_folds built as in boosting.rs:4334-4372): nullable, length n_features.  A one-hot feature's
     * candidates are the equality splits bin == v for v < real_folds[f]; float features
     * use bin > b for b < real_folds[f]-1.  NULL real_folds: every feature has n_bins. */
    const uint8_t* one_hot_flags;
    const uint32_t* real_folds;
    /* PairLogitPairwise: the bucket-weight prior of the pairwise leaf system
     * (bayesian_matrix_reg, 0.1 by default; boosting.rs:1785-1790) */
    double pairwise_non_diag_reg;
    /* DeviceTrainConfig.ctr (runtime.rs:1174-1230): NULL, or the CTR columns the session
     * builds on the device at open and appends after the n_features given (see
     * cbh_device_ctr_config) */
    const cbh_device_ctr_config* ctr;
} cbh_config;

typedef struct cbh_session cbh_session;

/* Open a device-resident session.  Mirrors begin_device_training (runtime.rs:1497-1529):
 *   bins_fm    feature-major quantized matrix, bins_fm[f * n + i] < n_bins (u32 like the
 *              reference; values must fit a byte: n_bins <= 256)
 *   weight     per-object weight (NULL = unit weights)
 *   scaled_l2  l2_leaf_reg * sum(weight) / n  (scale_l2_reg, leaf.rs:177)
 * Returns CBH_OK and *out, CBH_DECLINED for an uncovered config, or an error. */
int cbh_session_begin(const cbh_config* cfg, const uint32_t* bins_fm, const double* weight,
                      uint64_t n, uint32_t n_features, uint32_t n_bins, double learning_rate,
                      double scaled_l2, cbh_session** out);

/* Same, with a byte-per-bin feature-major matrix (4x less host memory). */
int cbh_session_begin_u8(const cbh_config* cfg, const uint8_t* bins_fm, const double* weight,
                         uint64_t n, uint32_t n_features, uint32_t n_bins, double learning_rate,
                         double scaled_l2, cbh_session** out);

/* Same, over the RAW float channel: the device quantizes the f32 columns with the
 * per-feature borders and packs the resident rows itself, so no host bin matrix exists.
 * Mirrors begin_device_training_raw (runtime.rs:1546-1580; device quantize twin
 * quantize_pack_feature_kernel, crates/cb-backend/src/kernels.rs:2852):
 *   columns   [n_features] pointers to n f32 values
 *   borders   [n_features] pointers to n_borders[f] ascending f64 borders (a border set
 *             ending with f32::MAX sends NaN to the top bin, else NaN goes to bin 0)
 *   n_bins    >= n_borders[f] + 1 for every f, <= 256
 * The resident bins equal bin_of (crates/cb-compute/src/histogram.rs:563-569) of every
 * value.  One-hot columns are not part of this channel (cfg->one_hot_flags must be NULL). */
int cbh_session_begin_raw(const cbh_config* cfg, const float* const* columns,
                          const double* const* borders, const uint32_t* n_borders,
                          const double* weight, uint64_t n, uint32_t n_features, uint32_t n_bins,
                          double learning_rate, double scaled_l2, cbh_session** out);

/* Per-tree device-resident sampling: the device regenerates exactly the sample the host
 * bootstrap() would draw at the current host RNG phase (bootstrap.rs:402-466), so no
 * n-length multiplier crosses PCIe.  bayesian_seed = the main-stream GenRand() the
 * Bayesian sampler consumes; bernoulli_state = TFastRng64 raw state [x1, c1, x2, c2]
 * before the n Bernoulli draws (rng.rs:221 raw_state). */
typedef struct {
    int32_t kind;                 /* CBH_BOOT_* */
    float bagging_temperature;
    double subsample;
    uint64_t bayesian_seed;
    uint64_t bernoulli_state[4];
} cbh_tree_sampling;

/* Per-tree family descriptor; mirrors FamilyTreeArgs (runtime.rs:913-950).
 * CBH_FAMILY_PAIRWISE (FamilyTreeArgs::Pairwise): required on the first grow of a PairLogit /
 * PairLogitPairwise session; NULL later keeps the resident pairs.  Rows of a query group are
 * contiguous (group_offsets, CSR over row order, n_groups + 1 entries, [0] = 0,
 * [n_groups] = n); pairs are (winner, loser, weight) inside one group, in any order (the
 * session orders them as the reference's competitor lists: stable by winner).
 * pair_weight NULL = weight 1 (query_info.rs:236-239).
 * CBH_FAMILY_MULTI_OUTPUT (FamilyTreeArgs::MultiOutput): approx_k is the dim-major
 * [approx_dim][n] approximant of this tree, approx_dim the session's; it is uploaded as the
 * approx argument of cbh_session_grow would be (which must then be NULL or the same
 * pointer).  The pair fields are unused. */
enum { CBH_FAMILY_PAIRWISE = 1, CBH_FAMILY_MULTI_OUTPUT = 2 };
typedef struct {
    int32_t kind;                 /* CBH_FAMILY_* */
    uint32_t n_groups;
    const uint32_t* group_offsets;
    const uint32_t* pair_winner;
    const uint32_t* pair_loser;
    const double* pair_weight;
    uint64_t n_pairs;
    const double* approx_k;       /* MultiOutput: [approx_dim][n] */
    uint32_t approx_dim;          /* MultiOutput: K */
} cbh_family;

/* Output of one grown tree; mirrors DeviceGrownTree (runtime.rs:990-1059).  Buffers are
 * caller-owned and sized by the caller: split_* [depth], leaf_values [2^depth * K]
 * (row-major leaf x dim, UNscaled by the learning rate), leaf_of [n] or NULL. */
typedef struct {
    uint32_t* split_feature;
    uint32_t* split_bin;
    uint8_t* split_one_hot;
    double* leaf_values;
    uint32_t* leaf_of;
    double* split_score;          /* nullable [depth]: winning score per level */
} cbh_tree_out;

/* Grow one oblivious tree.  Mirrors grow_tree_on_device (runtime.rs:1629-1638):
 *   approx   NULL: use the session's resident approximant (the hot path); else [K][n]
 *            host approximant uploaded for this tree
 *   target   NULL after the first call (resident); [n] (class index for MultiClass)
 *   sample   NULL/0, or the host multiplier control ? weight : 0 of length n (session
 *            opened with sample_from_host)
 *   sampling NULL, or device-resident sampling parameters for this tree
 *   family   NULL, or the pairs of a pair loss (see cbh_family)
 * The session applies approx += learning_rate * leaf_value[leaf_of] itself before the
 * next tree (the resident update of the reference's device branch). */
int cbh_session_grow(cbh_session* s, const double* approx, const double* target, uint64_t n,
                     const double* sample, uint64_t n_sample, const cbh_tree_sampling* sampling,
                     const cbh_family* family, cbh_tree_out* out);

/* Copy the resident approximant ([K][n]) to the host (applies any pending tree). */
int cbh_session_read_approx(cbh_session* s, double* approx_out, uint64_t n_times_k);

/* Per-session kernel timing (profile = 1) and fill traffic accounting.  Times are the
 * sums of HIP-event durations measured on the session stream. */
typedef struct {
    double fill_ms;               /* histogram fill kernels */
    double derive_ms;             /* histogram finishing: dominant-bin rebuild, prefix form, siblings */
    double score_ms;              /* split scoring + argmax */
    double partition_ms;          /* leaf update + stable compaction */
    double leaf_ms;               /* leaf reduction + values */
    double prepare_ms;            /* ders, bootstrap, approx update, histogram zeroing */
    double total_ms;              /* all of the above */
    uint64_t fill_launches;
    uint64_t fill_rows;           /* rows visited by fill launches (sum of V) */
    uint64_t fill_row_features;   /* sum of V * n_features */
    double fill_bytes;            /* algorithmic bytes V*(W*4 + S + 4) + H: S bytes of statistics per row,
                                     8*(K+1) for the generic and tiled exact fills, 8 for the rounded packed
                                     and count-packed fills, 8*ceil((K+1)/2) for the packed multi-channel
                                     fills (over sparse entries: 32 bytes of entry codes per 32-feature tile
                                     instead of W*4); the 4 bytes of a row index at the levels that gather
                                     rows through the partition's index list; H the histogram cells built x 8 */
    uint64_t trees;
    uint64_t skip_features;       /* features whose dominant bin the fill leaves out */
    double quantize_ms;           /* raw float channel: device quantize launches at open */
    uint64_t quantize_launches;
    double quantize_bytes;        /* algorithmic bytes: 4 read + 1 written per value + borders */
    uint32_t fill_mode;           /* 0: generic fill (32-feature tiles, one exact 64-bit atomic per channel,
                                     any K); 1: rounded packed fill (K = 1, 64-feature tiles, both channels
                                     rounded to 18-bit rows in one 64-bit atomic); 2: tiled exact fill (K = 1,
                                     32-feature tiles, one exact 64-bit atomic per channel, DPP-broadcast
                                     statistics); 3: packed multi-channel fill (K > 1, 32-feature tiles, two
                                     channels rounded to 20-bit rows per 64-bit atomic); 4: the same cells
                                     over sparse entries (a row per 16-lane DPP row, one lane per
                                     non-dominant (feature, bin)); 5: count-packed fill (K = 1, integer
                                     score weights, 64-feature tiles, a row's der rounded at 2^-30 or
                                     finer and its weight exact in one 64-bit atomic) */
    int32_t fill_pack_bits;       /* packed fills: bits of a row's rounded channel value (|q| < 2^bits) */
    int32_t score_shift_der;      /* the last tree's fixed-point scales S of the score channels: a row's */
    int32_t score_shift_w;        /* value v enters the histogram as round(v * 2^S) (der; weight) */
    uint64_t fill_entries;        /* (row, feature) entries the fill launches added: fill_row_features, or
                                     with the dominant-bin skip those whose bin is not the dominant one,
                                     counted over the trees grown with profiling on */
    uint64_t fill_lane_atomics;   /* 64-bit LDS atomics (lanes) the fill launches issued for those entries:
                                     entries x atomics per entry (one per channel, one, or one per plane of
                                     two channels, by fill) */
} cbh_stats;

int cbh_session_stats(const cbh_session* s, cbh_stats* out);

/* CTR columns of a session (DeviceCtrConfig, runtime.rs:1160-1230, for simple projections and
 * one learning permutation).  The LAST n_ctr features of the session are CTR columns built
 * under the structure (learning) permutation (cbh_ctr_columns).  They are scored after the
 * float columns, each candidate's score multiplied by the model_size_reg weight of its
 * (ctr type, projection) group while no earlier tree and no earlier level of the tree used
 * the group: (1 + bucket_count / max_count)^(-model_size_reg), max_count the largest bucket
 * count of the CTR columns and, once the tree holds a float split, of the distinct
 * (float-partition leaf, bucket) pairs of the categorical columns (tree.rs:2907, :3146-3346).
 * Leaf values and the resident approximant use the partition in which every CTR level
 * re-tests the column built under the averaging permutation (assign_leaf_over_ctr_columns,
 * boosting.rs:2905, :8206).  The weights come from a table of pow values over every
 * reachable max_count (tabulated here at set-up, picked per level on the device), so such
 * trees replay their recorded launch sequence like any other; when the table would pass
 * 32 Mi entries each level takes a host step instead and the trees run eagerly. */
typedef struct {
    uint32_t n_ctr;
    const uint8_t* averaging_bins;    /* [n_ctr][n] */
    const uint32_t* bucket_count;     /* [n_ctr] distinct buckets of each column's projection */
    const uint32_t* weight_group;     /* [n_ctr] group id (< n_ctr) per (ctr type, projection) */
    uint32_t n_cat;                   /* CTR-eligible categorical columns */
    const uint32_t* cat_buckets;      /* [n_cat][n] first-seen buckets */
    const uint32_t* cat_bucket_count; /* [n_cat] */
    double model_size_reg;            /* 0.5 by default; 0 disables the weight */
} cbh_ctr_info;
int cbh_session_set_ctr(cbh_session* s, const cbh_ctr_info* info);

/* The device CTR config given at open (cbh_config.ctr): DeviceCtrColumn,
 * DeviceCtrAveraging and DeviceCtrConfig (runtime.rs:1104-1230).  The session builds both
 * CTR materializations on the device, as build_ctr_cindex_columns does
 * (crates/cb-backend/src/gpu_runtime/session.rs:262-360): for every column, the ordered
 * statistic of its bucket column under the permutation (Borders / Buckets / BTMV read the
 * object's predecessors in its bucket, Counter whole-set bucket sizes), value
 * (num + prior) / (total + 1), binarized by the column's border table: bin = the number of
 * borders strictly below the value (binarize_ctr_kernel, kernels/ctr_device.rs:399-413).
 * The structure columns become features n_features .. n_features + n_columns - 1 of the
 * session (candidate folds n_borders + 1) and are scored as cbh_session_set_ctr describes;
 * the averaging columns re-test the CTR levels for leaf values and the resident
 * approximant.  Admission follows ctr_covered (session.rs:177-215): a NULL averaging half,
 * a column count that differs between the halves, a type outside CBH_CTR_*, a column with
 * no member, or a pair loss DECLINES; so does a projection of two or more members (the
 * combination gate is not built).  A border table may be shorter than n_bins - 1 (the
 * reference asks for equality and declines otherwise). */
typedef struct {
    uint32_t n_members;                  /* 1: a simple projection */
    const uint32_t* const* member_bins;  /* [n_members] pointers to n category codes */
    double prior;                        /* prior numerator (prior_num / prior_denom) */
    const double* borders;               /* [n_borders] */
    uint32_t n_borders;                  /* 1 .. n_bins - 1 */
    uint64_t bucket_count;               /* the projection's distinct buckets; 0 = observed */
    uint32_t weight_group;               /* (ctr type, projection) group id, < n_columns */
    int32_t ctr_type;                    /* CBH_CTR_* */
    uint32_t target_border_idx;          /* Borders / Buckets numerator selector, <= 1 */
    const uint32_t* projection_members;  /* [n_projection_members] sorted absolute cat ids */
    uint32_t n_projection_members;
} cbh_device_ctr_column;

typedef struct {
    const uint32_t* permutation;             /* [n] averaging-fold order */
    const uint32_t* target_class;            /* [n] 0 or 1 */
    const cbh_device_ctr_column* columns;    /* [n_columns], aligned with the structure set */
    uint32_t n_columns;
} cbh_device_ctr_averaging;

struct cbh_device_ctr_config {
    const uint32_t* permutation;             /* [n] learn order: object permutation[p] at position p */
    const uint32_t* target_class;            /* [n] 0 or 1 */
    const cbh_device_ctr_column* columns;    /* [n_columns] */
    uint32_t n_columns;
    const cbh_device_ctr_averaging* averaging;    /* NULL declines */
    uint32_t n_cat;                               /* CTR-eligible categorical columns */
    const uint32_t* const* cat_eligible_buckets;  /* [n_cat] pointers to n first-seen buckets */
    double model_size_reg;                        /* 0.5 by default; 0 disables the weight */
};

/* Test entry: the session's CTR bins, [n_ctr][n] u8, of the structure (averaging = 0) or
 * the averaging (averaging = 1) materialization.  No counterpart in the reference, whose
 * builder returns the bin columns to its caller. */
int cbh_session_read_ctr_bins(const cbh_session* s, int32_t averaging, uint8_t* out, uint64_t n_times_ctr);

/* Per-stage timing switch (cbh_config.profile).  While it is off, every tree after the
 * first whose previous leaves are still pending replays one recorded launch sequence (a
 * HIP graph) instead of launching its ~60 kernels one by one; while it is on, trees run
 * eagerly with HIP events around every stage.  No counterpart in the reference (its
 * per-kernel timing is a build-time diagnostic). */
int cbh_session_set_profile(cbh_session* s, int32_t on);
void cbh_session_reset_stats(cbh_session* s);

/* Inspection entries (no counterpart in the reference): with capture on, every later tree
 * keeps its level histograms as the split scorer read them (trees then run eagerly, not as a
 * recorded graph; pairwise sessions decline).  cbh_session_level_hist returns level `level` of
 * the last tree as f64 bin sums in the reference's layout [2^level leaves][F][n_bins][K+1]
 * (histogram.rs:176-177; channel K the weight), each exact integer sum times 2^-S of its
 * channel; n_cells must be 2^level * F * n_bins * (K+1). */
int cbh_session_capture_hists(cbh_session* s, int32_t on);
int cbh_session_level_hist(const cbh_session* s, uint32_t level, double* out, uint64_t n_cells);

/* Release the session.  Mirrors end_device_training (runtime.rs:1648). */
int cbh_session_end(cbh_session* s);

/* Mirrors compute_gradients (runtime.rs:1431-1437): dim-major der1/der2 on the device.
 * For MultiClass der2 is the packed per-object Hessian [n][K(K+1)/2]. */
int cbh_compute_gradients(int32_t loss, const double* approx, const double* target, uint64_t n,
                          uint32_t approx_dim, double* der1, double* der2);

/* ---- kernel-level entry points (host buffers in/out), each kernel checked alone ---- */

/* Histogram of one leaf set: rows listed in idx (NULL = all n in order) with leaf slot
 * slot_of_row[i] (NULL = 0), score channels der [K][n], w [n].  Output exact sums as f64
 * in [n_slots][F][n_bins][K+1] (channel K = weight). */
int cbh_hist_build(const uint8_t* bins_fm, uint64_t n, uint32_t n_features, uint32_t n_bins,
                   const double* der, const double* w, uint32_t K, const uint32_t* slot_of_row,
                   uint32_t n_slots, double* hist_out);

/* cbh_hist_build of the whole row set (one slot) over DEVICE buffers, allocating nothing.
 * No counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 *   bins_fm [n_features][n] u8, der [K][n], w [n], hist_out [n_features][n_bins][K+1] f64:
 *   device pointers; stream: a hipStream_t (NULL = the default stream).
 * The work is enqueued on stream and not waited for.  Packed rows, quantized statistics,
 * the integer histogram and the scales live in a 32 MiB static device array per GPU, held
 * until the process ends: n * (4 ceil(n_features / 4) + 8 (K + 1)) + 8 n_features n_bins
 * (K + 1) bytes plus 5 KiB must fit, else CBH_ERR_OUT_OF_RANGE.  Every call on one GPU
 * shares that array: calls that overlap on one GPU (other streams, other host threads)
 * race.  The result equals cbh_hist_build's with slot_of_row NULL (the same scale rule
 * from the sums of max_d |der| and |w|, summed on the device).  Precondition: every bin is
 * below n_bins (cbh_hist_build checks this on the host; here the bins are never read by the
 * host, and a larger bin adds to another feature's cells: the result is then undefined). */
int cbh_hist_build_noalloc(const uint8_t* bins_fm, uint64_t n, uint32_t n_features, uint32_t n_bins,
                           const double* der, const double* w, uint32_t K, double* hist_out, void* stream);

/* Device bootstrap (bootstrap.rs:141-184): sample weights and control mask for n rows. */
int cbh_bootstrap(const cbh_tree_sampling* sampling, uint64_t n, double* sample_weight,
                  uint8_t* control);

/* Raw predictions of an oblivious float ensemble (final prediction / model apply).
 * Mirrors launch_apply_oblivious_f64 (crates/cb-backend/src/gpu_runtime/mod.rs:337, kernel
 * crates/cb-backend/src/kernels.rs:629) and predict_raw (crates/cb-model/src/apply.rs):
 *   features_fm        f32 [n_features][n_objects] (the reference widens f32 values to f64,
 *                      as this comparison does)
 *   split_features, split_borders   [tree_split_offsets[n_trees]], pass test value > border
 *   tree_split_offsets [n_trees + 1] CSR, starting at 0; split i of a tree is leaf bit i
 *   leaf_values        [tree_leaf_offsets[n_trees] * approx_dim], the approx_dim values of a
 *                      leaf contiguous (DeviceGrownTree layout); tree_leaf_offsets CSR in leaves
 *   bias               nullable [approx_dim], added once after the trees
 *   nan_as_true        nullable [n_features]: NaN passes every split of the feature (borders
 *                      of nan_mode=Max); otherwise NaN fails
 *   out                [approx_dim][n_objects]
 * A split feature >= n_features is absent (bit 0); a leaf index past the tree adds 0. */
int cbh_apply_oblivious(const float* features_fm, uint64_t n_objects, uint32_t n_features,
                        const uint32_t* split_features, const double* split_borders,
                        const uint32_t* tree_split_offsets, const double* leaf_values,
                        const uint32_t* tree_leaf_offsets, uint32_t n_trees, uint32_t approx_dim,
                        const double* bias, const uint8_t* nan_as_true, double* out);

/* The float columns of a C-contiguous row-major matrix, as the reference's ingest of an
 * (n_rows, n_features) f32 array builds them (crates/catboost-rs-py/src/ingest_py.rs:157-203):
 *   rows     [n][n_features] f32, row-major
 *   columns  [n_features][n] f32 out, feature f's column at columns + f * n
 * A host copy in blocks of rows, over the host's threads (at most 16; the same values in
 * the same order whatever the split).  CBH_ERR_INVALID_ARG on a null pointer. */
int cbh_columns_from_rows(const float* rows, uint64_t n, uint32_t n_features, float* columns);

/* Greedy border selection of float columns; mirrors Pool::quantize's border step
 * (crates/cb-data/src/quantize.rs:74-110) over select_borders_greedy_logsum_f32 and its
 * GreedyMinEntropy twin (crates/cb-data/src/borders.rs:298-420):
 *   columns         [n_features] pointers to n f32 values (NaN allowed)
 *   border_count    budget per feature (the Min sentinel takes one slot); at most 255, 254
 *                   under CBH_NAN_MAX (its f32::MAX sentinel is appended on top)
 *   nan_mode        CBH_NAN_*: applied to a column holding at least one NaN; a NaN-free
 *                   column has no sentinel
 *   border_type     CBH_BORDERS_*
 *   borders_out     [n_features][border_count + 1] f64; feature f's n_borders_out[f]
 *                   ascending borders (f32-exact values) lead its row
 * Columns over 200000 rows use the fixed-seed 200000-row subset of the reference
 * (sample_indices_for_build_borders, borders.rs:504-516).  The subset's values are sorted
 * on the device; the greedy split runs on the host. */
int cbh_select_borders(const float* const* columns, uint64_t n, uint32_t n_features,
                       uint32_t border_count, int32_t nan_mode, int32_t border_type,
                       double* borders_out, uint32_t* n_borders_out);

/* Quantize one f32 column into u8 bins on the device: bin_of (histogram.rs:563-569) --
 * the count of borders strictly below the value; NaN to the top bin when the borders end
 * with f32::MAX, else to bin 0.  At most 255 ascending borders. */
int cbh_quantize(const float* column, uint64_t n, const double* borders, uint32_t n_borders,
                 uint8_t* bins_out);

/* ---- categorical inputs ---- */

/* count learn permutations drawn one after another off TFastRng64::from_seed(seed)
 * (create_shuffled_indices / permutations, crates/cb-train/src/permutation.rs:131, :236):
 * out [count][n].  Host code (each Fisher-Yates swap depends on the previous draws). */
int cbh_shuffled_indices(uint64_t n, uint64_t seed, uint32_t count, uint32_t* out);

/* First-seen dense bins of u32 category keys (the reference hashes a category to a u32 with
 * calc_cat_feature_hash and remaps with PerfectHash, crates/cb-data/src/cat_hash.rs:389-479):
 * bins_out[i] = the rank of keys[i] among the distinct keys ordered by first occurrence. */
int cbh_perfect_hash(const uint32_t* keys, uint64_t n, uint32_t* bins_out, uint32_t* n_distinct_out);

/* One CTR column spec (DeviceCtrColumn's ctr_type / target_border_idx / prior,
 * runtime.rs:1104-1160; prior_denom must be non-zero, the CPU path uses 1). */
typedef struct {
    int32_t ctr_type;             /* CBH_CTR_* */
    uint32_t target_border_idx;   /* Buckets: the class counted; Borders: classes <= it excluded */
    double prior_num;
    double prior_denom;
} cbh_ctr_spec;

/* Online CTR columns of one categorical feature (or one projection, given its combined
 * bucket per object), all specs at once.  Mirrors materialize_ctr_feature
 * (crates/cb-train/src/ctr/ctr_feature.rs) over online_class_prefix_column /
 * online_mean_prefix / online_counter_column (crates/cb-train/src/ctr/online.rs) and the
 * device twin ordered_ctr_prefix_kernel (crates/cb-backend/src/kernels/ctr_device.rs:164):
 *   buckets        [n], each < n_buckets (first-seen bins of the category or projection)
 *   permutation    [n], the learn order: object permutation[p] sits at position p
 *   target_class   [n], 0 or 1 (binclf class; the reference binarizes t > 0.5)
 *   bins_out       [n_specs][n] u8: trunc((value + shift) / norm * border_count) clamped to
 *                  [0, border_count], shift/norm = calc_normalization(prior), in f32 for BTMV
 *   values_out     nullable [n_specs][n] f64: (num + prior) / (total + 1)
 *   class_counts_out nullable [2][n]: the per-object predecessor counts N0, N1
 * Borders / Buckets / BinarizedTargetMeanValue read the counts of the object's bucket over
 * its PREDECESSORS in the permutation (read before increment); Counter uses whole-set bucket
 * sizes over the largest bucket size (counter_calc_method SkipTest). */
int cbh_ctr_columns(const uint32_t* buckets, uint32_t n_buckets, uint64_t n, const uint32_t* permutation,
                    const uint8_t* target_class, const cbh_ctr_spec* specs, uint32_t n_specs,
                    uint32_t border_count, uint8_t* bins_out, double* values_out,
                    uint32_t* class_counts_out);

/* Version / build information. */
const char* cbh_version(void);
const char* cbh_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
