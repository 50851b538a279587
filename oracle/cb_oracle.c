/*
 * cb_oracle.c -- CPU restatement of catboost_rs's oblivious-tree training path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker + CPU baseline); never linked by the
 * product library.  See cb_oracle.h for what pins each function.
 *
 * Arithmetic-order contract: every float sum is a sequential left-to-right f64
 * fold in ascending object (or bin / leaf) order, exactly like the reference's
 * cb_core::sum_f64 (crates/cb-core/src/reduction.rs:32).  Parallelism is only
 * over independent features (crates/cb-train/src/tree.rs:1191-1252), so the
 * result does not depend on the thread count.
 *
 * Build with -ffp-contract=off: the reference never fuses multiply-adds.
 */
#include "cb_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ======================================================================
 * TFastRng64 (crates/cb-core/src/rng.rs:24-292)
 * ==================================================================== */
static const uint64_t LCG_A = 6364136223846793005ULL; /* rng.rs:26 */

static inline uint32_t pcg_mix(uint64_t x) { /* rng.rs:31-38 */
    uint32_t xs = (uint32_t)(((x >> 18) ^ x) >> 27);
    uint32_t rot = (uint32_t)(x >> 59);
    return (xs >> rot) | (xs << ((32 - rot) & 31));
}

/* NPrivate::LcgAdvance, closed-form jump (rng.rs:45-66). */
static uint64_t lcg_advance(uint64_t seed, uint64_t base, uint64_t addend, uint64_t delta) {
    uint64_t mask = 1;
    while (mask != (1ULL << 63) && (mask << 1) <= delta) mask <<= 1;
    uint64_t apow = 1, adiv = 0;
    while (mask != 0) {
        adiv = adiv * (apow + 1);
        apow = apow * apow;
        if (delta & mask) {
            adiv = adiv + apow;
            apow = apow * base;
        }
        mask >>= 1;
    }
    return seed * apow + addend * adiv;
}

static inline uint32_t lcg32_next(uint64_t* x, uint64_t c) { /* rng.rs:103-106 */
    *x = *x * LCG_A + c;
    return pcg_mix(*x);
}

static uint32_t fix_seq(uint32_t seq1, uint32_t seq2) { /* rng.rs:128-135 */
    uint32_t mask = (~0u) >> 1;
    return ((seq1 & mask) == (seq2 & mask)) ? ~seq2 : seq2;
}

void orc_rng_new(orc_rng* r, uint64_t seed1, uint32_t seq1, uint64_t seed2, uint32_t seq2) {
    r->x1 = seed1;
    r->c1 = ((uint64_t)seq1 << 1) | 1;
    r->x2 = seed2;
    r->c2 = ((uint64_t)fix_seq(seq1, seq2) << 1) | 1;
    r->calls = 0;
}

void orc_rng_from_seed(orc_rng* r, uint64_t seed) { /* rng.rs:171-180 */
    uint64_t x = seed;
    uint64_t lo = lcg32_next(&x, 1), hi = lcg32_next(&x, 1);
    uint64_t seed1 = lo | (hi << 32);
    uint32_t seq1 = lcg32_next(&x, 1);
    lo = lcg32_next(&x, 1);
    hi = lcg32_next(&x, 1);
    uint64_t seed2 = lo | (hi << 32);
    uint32_t seq2 = lcg32_next(&x, 1);
    orc_rng_new(r, seed1, seq1, seed2, seq2);
}

uint64_t orc_rng_gen(orc_rng* r) { /* rng.rs:183-189: stream 1 -> high half */
    uint64_t a = lcg32_next(&r->x1, r->c1);
    uint64_t b = lcg32_next(&r->x2, r->c2);
    r->calls++;
    return (a << 32) | b;
}

void orc_rng_advance(orc_rng* r, uint64_t delta) { /* rng.rs:192-197 */
    r->x1 = lcg_advance(r->x1, LCG_A, r->c1, delta);
    r->x2 = lcg_advance(r->x2, LCG_A, r->c2, delta);
    r->calls += delta;
}

double orc_rng_real1(orc_rng* r) { /* rng.rs:256-259 */
    return (double)(orc_rng_gen(r) >> 11) * (1.0 / 9007199254740991.0);
}

uint64_t orc_rng_uniform(orc_rng* r, uint64_t bound) { /* rng.rs:268-280 */
    if (bound == 0) return 0;
    uint64_t randmax = UINT64_MAX - (UINT64_MAX % bound);
    for (;;) {
        uint64_t v = orc_rng_gen(r);
        if (v < randmax) return v % bound;
    }
}

double orc_std_normal(orc_rng* r) { /* cb-core/src/normal.rs:50-64 (Marsaglia polar) */
    for (;;) {
        double x = orc_rng_real1(r) * 2.0 - 1.0;
        double y = orc_rng_real1(r) * 2.0 - 1.0;
        double rr = x * x + y * y;
        if (!(rr > 1.0 || rr <= 0.0)) return x * sqrt(-2.0 * log(rr) / rr);
    }
}

/* FastLogf (crates/cb-train/src/fast_approx.rs:154-177): all-f32 op order. */
float orc_fast_logf(float value) {
    uint32_t vx;
    memcpy(&vx, &value, 4);
    uint32_t mbits = (vx & 0x007FFFFFu) | 0x3f000000u;
    float mx;
    memcpy(&mx, &mbits, 4);
    float y = (float)vx;
    y *= 1.1920928955078125e-7f;
    float l2 = y - 124.22551499f - 1.498030302f * mx - 1.72587999f / (0.3520887068f + mx);
    return 0.69314718f * l2;
}

/* ======================================================================
 * Bootstrap (crates/cb-train/src/bootstrap.rs)
 * ==================================================================== */
#define BAYESIAN_BLOCK 1000 /* bootstrap.rs:81 */

int orc_bootstrap(int32_t type, uint64_t n, double subsample, float temperature, orc_rng* rng,
                  double* sw, uint8_t* control) {
    if (type == ORC_BOOT_NO) { /* BootstrapResult::identity */
        for (uint64_t i = 0; i < n; ++i) { sw[i] = 1.0; control[i] = 1; }
        return 0;
    }
    if (type == ORC_BOOT_BAYESIAN) { /* bootstrap.rs:152-169 + bayesian_weight :141-146 */
        for (uint64_t i = 0; i < n; ++i) control[i] = 1;
        if (temperature == 0.0f) {
            for (uint64_t i = 0; i < n; ++i) sw[i] = 1.0;
            return 0;
        }
        uint64_t seed = orc_rng_gen(rng);
        uint64_t blocks = (n + BAYESIAN_BLOCK - 1) / BAYESIAN_BLOCK;
        for (uint64_t b = 0; b < blocks; ++b) {
            orc_rng br;
            orc_rng_from_seed(&br, seed + b);
            orc_rng_advance(&br, 10);
            uint64_t end = (b + 1) * BAYESIAN_BLOCK;
            if (end > n) end = n;
            for (uint64_t i = b * BAYESIAN_BLOCK; i < end; ++i) {
                double u = orc_rng_real1(&br);
                float w = -orc_fast_logf((float)u + 1e-100f);
                sw[i] = (double)powf(w, temperature);
            }
        }
        return 0;
    }
    if (type == ORC_BOOT_BERNOULLI) { /* bootstrap.rs:178-184 set_sampled_control */
        for (uint64_t i = 0; i < n; ++i) sw[i] = 1.0;
        if (subsample >= 1.0) {
            for (uint64_t i = 0; i < n; ++i) control[i] = 1;
            return 0;
        }
        double rate = (double)(float)subsample;
        for (uint64_t i = 0; i < n; ++i) control[i] = orc_rng_real1(rng) < rate;
        return 0;
    }
    return -1;
}

/* ======================================================================
 * Quantization (crates/cb-compute/src/histogram.rs:563-569 bin_of)
 * ==================================================================== */
void orc_quantize(const float* values, uint64_t n, const double* borders, uint32_t nb,
                  uint8_t* out) {
    int nan_top = nb > 0 && borders[nb - 1] == (double)3.40282346638528859812e+38F;
    for (uint64_t i = 0; i < n; ++i) {
        float v = values[i];
        if (isnan(v) && nan_top) { out[i] = (uint8_t)nb; continue; }
        double dv = (double)v;
        uint32_t c = 0;
        for (uint32_t k = 0; k < nb; ++k) c += borders[k] < dv;
        out[i] = (uint8_t)c;
    }
}

/* ======================================================================
 * Derivatives (crates/cb-compute/src/loss.rs:35-80)
 * ==================================================================== */
void orc_ders(int32_t loss, const double* a, const double* t, uint64_t n, double* d1,
              double* d2) {
    for (uint64_t i = 0; i < n; ++i) {
        if (loss == ORC_LOSS_RMSE) {
            d1[i] = t[i] - a[i];
            if (d2) d2[i] = -1.0;
        } else {
            double e = exp(a[i]);
            double p = 1.0 - 1.0 / (1.0 + e);
            d1[i] = t[i] - p;
            if (d2) d2[i] = -p * (1.0 - p);
        }
    }
}

/* MultiClass softmax ders for one object (loss.rs:424-486): der1[k], packed der2[k(k+1)/2]. */
static void softmax_ders(const double* approx, int k, int target_class, double* der1,
                         double* der2) {
    double mx = -INFINITY;
    for (int d = 0; d < k; ++d)
        if (approx[d] > mx) mx = approx[d];
    double p[64];
    double sum = 0.0;
    for (int d = 0; d < k; ++d) { p[d] = exp(approx[d] - mx); }
    for (int d = 0; d < k; ++d) sum += p[d];
    for (int d = 0; d < k; ++d) p[d] = p[d] / sum;
    int idx = 0;
    for (int y = 0; y < k; ++y) {
        der2[idx++] = p[y] * (p[y] - 1.0);
        for (int x = y + 1; x < k; ++x) der2[idx++] = p[y] * p[x];
    }
    for (int d = 0; d < k; ++d) der1[d] = -p[d];
    if (target_class >= 0 && target_class < k) der1[target_class] += 1.0;
}

/* ======================================================================
 * Leaf estimators (crates/cb-compute/src/leaf.rs)
 * ==================================================================== */
static inline double calc_average(double s, double w, double l2) { /* leaf.rs:161-167 */
    return w > 0.0 ? s / (w + l2) : 0.0;
}

static double newton_leaf_delta(double s, double d2, double l2) { /* leaf.rs:223-233 */
    double den = -d2 + l2;
    return den == 0.0 ? 0.0 : s / den;
}

/* leaf.rs:387-440 cholesky_solve; returns 0 on a non-positive pivot. */
static int cholesky_solve(int k, const double* a, const double* b, double* x) {
    double* l = (double*)calloc((size_t)k * (size_t)k + (size_t)k, sizeof(double));
    double* y = l + (size_t)k * k;
    int ok = 1;
    for (int i = 0; i < k; ++i) {
        for (int j = 0; j <= i; ++j) {
            double sum = a[i * k + j];
            for (int p = 0; p < j; ++p) sum -= l[i * k + p] * l[j * k + p];
            if (i == j) {
                if (sum <= 0.0) { ok = 0; goto done; }
                l[i * k + j] = sqrt(sum);
            } else {
                double ljj = l[j * k + j];
                if (ljj == 0.0) { ok = 0; goto done; }
                l[i * k + j] = sum / ljj;
            }
        }
    }
    for (int i = 0; i < k; ++i) {
        double sum = b[i];
        for (int p = 0; p < i; ++p) sum -= l[i * k + p] * y[p];
        if (l[i * k + i] == 0.0) { ok = 0; goto done; }
        y[i] = sum / l[i * k + i];
    }
    for (int i = k - 1; i >= 0; --i) {
        double sum = y[i];
        for (int p = i + 1; p < k; ++p) sum -= l[p * k + i] * x[p];
        if (l[i * k + i] == 0.0) { ok = 0; goto done; }
        x[i] = sum / l[i * k + i];
    }
done:
    free(l);
    return ok;
}

/* solve_symmetric_newton (leaf.rs:279-335). */
static void solve_symmetric_newton(int k, const double* sum_der, const double* packed,
                                   double l2, double* out) {
    double h[64 * 64];
    int idx = 0;
    for (int i = 0; i < k; ++i)
        for (int j = i; j < k; ++j) {
            h[i * k + j] = packed[idx];
            h[j * k + i] = packed[idx];
            idx++;
        }
    float max_trace = (float)l2;
    for (int d = 0; d < k; ++d) {
        float v = (float)(-h[d * k + d]);
        max_trace = fmaxf(max_trace, v);
    }
    double adj = (double)fmaxf((float)l2, max_trace * 1.1920928955078125e-7f);
    for (int d = 0; d < k; ++d) h[d * k + d] -= adj;
    for (int i = 0; i < k * k; ++i) h[i] = -h[i];
    double nd[64], x[64];
    for (int d = 0; d < k; ++d) nd[d] = -sum_der[d];
    if (cholesky_solve(k, h, nd, x)) {
        for (int d = 0; d < k; ++d) out[d] = -x[d];
    } else {
        for (int d = 0; d < k; ++d) out[d] = 0.0;
    }
}

void orc_leaf_sums(const uint32_t* leaf_of, uint64_t n, uint32_t n_leaves, const double* der,
                   const double* w, double* sum_der, double* sum_w) {
    for (uint32_t l = 0; l < n_leaves; ++l) { sum_der[l] = 0.0; if (sum_w) sum_w[l] = 0.0; }
    for (uint64_t i = 0; i < n; ++i) {
        uint32_t l = leaf_of[i];
        if (l >= n_leaves) continue;
        sum_der[l] += der[i];
        if (sum_w) sum_w[l] += w ? w[i] : 1.0;
    }
}

/* ======================================================================
 * Per-feature histogram (crates/cb-compute/src/histogram.rs:188-698)
 * layout: hist[(leaf * n_bins + bin) * C + ch], C = K + 1, ch K = weight
 * ==================================================================== */

/* build_bucket_histogram_into restricted to one feature (histogram.rs:676-697):
 * object-outer scatter, objects with slot >= n_leaves skipped. */
static void build_hist(double* h, uint32_t n_leaves, uint32_t n_bins, int K, const uint8_t* col,
                       const double* der, const double* w, const uint32_t* slot, uint64_t n) {
    const int C = K + 1;
    memset(h, 0, sizeof(double) * (size_t)n_leaves * n_bins * C);
    for (uint64_t o = 0; o < n; ++o) {
        uint32_t l = slot[o];
        if (l >= n_leaves) continue;
        uint32_t b = col[o];
        if (b >= n_bins) continue;
        double* cell = h + ((size_t)l * n_bins + b) * C;
        for (int d = 0; d < K; ++d) cell[d] += der[(size_t)d * n + o];
        cell[K] += w[o];
    }
}

/* derive_feature_level_hist (tree.rs:1075-1131): build the globally smaller sibling over
 * all objects, derive the larger as parent - smaller (one f64 subtraction per cell). */
static void derive_hist(double* out, const double* parent, uint32_t level, uint32_t n_bins,
                        int K, const uint8_t* col, const double* der, const double* w,
                        const uint32_t* leaf_of, uint64_t n, uint32_t* scratch_slot,
                        uint64_t n_true) {
    const int C = K + 1;
    uint32_t n_parent = 1u << (level - 1);
    uint32_t n_next = 1u << level;
    size_t per_leaf = (size_t)n_bins * C;
    uint64_t n_false = n - n_true;
    int build_true = n_true <= n_false;
    for (uint64_t o = 0; o < n; ++o) {
        uint32_t lf = leaf_of[o];
        int pass = (lf & n_parent) != 0;
        scratch_slot[o] = (pass == build_true) ? (lf & (n_parent - 1)) : 0xFFFFFFFFu;
    }
    /* built sibling lands in the low slots of an n_next-leaf histogram */
    double* built = (double*)malloc(sizeof(double) * per_leaf * n_next);
    build_hist(built, n_next, n_bins, K, col, der, w, scratch_slot, n);
    for (uint32_t p = 0; p < n_parent; ++p) {
        const double* par = parent + p * per_leaf;
        const double* bl = built + p * per_leaf;
        double* fslot = out + p * per_leaf;               /* FALSE child p */
        double* tslot = out + (p + n_parent) * per_leaf;  /* TRUE child p + n_parent */
        for (size_t c = 0; c < per_leaf; ++c) {
            double other = -bl[c] + par[c]; /* relocate_sub: (-minus) + parent */
            if (build_true) { tslot[c] = bl[c]; fslot[c] = other; }
            else { fslot[c] = bl[c]; tslot[c] = other; }
        }
    }
    free(built);
}

/* Per-parent totals of one feature: ordered f64 sums over the bins (histogram.rs:1040-1075
 * and :1207-1235 compute them the same way for the border and the one-hot scans). */
static void parent_totals(const double* h, uint32_t n_parent, uint32_t n_bins, int K,
                          double* total_w, double* total_d) {
    const int C = K + 1;
    for (uint32_t p = 0; p < n_parent; ++p) {
        const double* blk = h + (size_t)p * n_bins * C;
        double t = 0.0;
        for (uint32_t b = 0; b < n_bins; ++b) t += blk[b * C + K];
        total_w[p] = t;
        for (int d = 0; d < K; ++d) {
            double td = 0.0;
            for (uint32_t b = 0; b < n_bins; ++b) td += blk[b * C + d];
            total_d[p * K + d] = td;
        }
    }
}

/* Per-leaf terms of the SolarL2 / LOOL2 / SatL2 calcers, without the L2 regularizer:
 * solar_l2_terms (score.rs:283-299), loo_l2_terms (:304-325), sat_l2_terms (:330-350). */
double orc_leaf_score_term(int32_t score_fn, double s, double w) {
    if (score_fn == ORC_SCORE_SOLAR_L2) return w > 1e-20 ? (-s * s) * (1.0 + 2.0 * log(w + 1.0)) / w : 0.0;
    if (score_fn == ORC_SCORE_LOO_L2) {
        double adjust = w > 1.0 ? w / (w - 1.0) : 0.0;
        adjust *= adjust;
        return w > 0.0 ? adjust * (-s * s) / w : 0.0;
    }
    if (score_fn == ORC_SCORE_SAT_L2) {
        const double adjust = w > 2.0 ? w * (w - 2.0) / (w * w - 3.0 * w + 1.0) : 0.0;
        return w > 0.0 ? adjust * (-s * s) / w : 0.0;
    }
    return 0.0;
}

/* multi_dim_split_score_into (score.rs:192-265): fold in dimension-then-leaf order over the
 * 2P children (leaves 0..P-1 FALSE, P..2P-1 TRUE); sd is [K][2P], sw is [2P].  SolarL2, LOOL2
 * and SatL2 (:236-265) sum their per-leaf terms in the same order. */
static double fold_score(const double* sd, const double* sw, uint32_t n_parent, int K,
                         int score_fn, double l2) {
    if (score_fn >= ORC_SCORE_SOLAR_L2) {
        double acc = 0.0;
        for (int d = 0; d < K; ++d)
            for (uint32_t l = 0; l < 2 * n_parent; ++l)
                acc += orc_leaf_score_term(score_fn, sd[(size_t)d * 2 * n_parent + l], sw[l]);
        return acc;
    }
    double num = 0.0;
    for (int d = 0; d < K; ++d)
        for (uint32_t l = 0; l < 2 * n_parent; ++l) {
            double s = sd[(size_t)d * 2 * n_parent + l];
            double avg = calc_average(s, sw[l], l2);
            num += avg * s;
        }
    if (score_fn == ORC_SCORE_L2) return num;
    double den = 0.0;
    den += 1e-100;
    for (int d = 0; d < K; ++d)
        for (uint32_t l = 0; l < 2 * n_parent; ++l) {
            double s = sd[(size_t)d * 2 * n_parent + l];
            double avg = calc_average(s, sw[l], l2);
            den += avg * avg * sw[l];
        }
    return num / sqrt(den);
}

/* scan_and_score_borders_into (histogram.rs:1007-1149) + multi_dim_split_score_into
 * (score.rs:192-265) for one feature with n_parent = 2^level leaves. */
static void scan_score(const double* h, uint32_t n_parent, uint32_t n_bins, int K,
                       uint32_t n_borders, int score_fn, double l2, double* scores) {
    const int C = K + 1;
    double* total_w = (double*)calloc(n_parent, sizeof(double));
    double* total_d = (double*)calloc((size_t)n_parent * K, sizeof(double));
    double* acc_w = (double*)calloc(n_parent, sizeof(double));
    double* acc_d = (double*)calloc((size_t)n_parent * K, sizeof(double));
    double* sd = (double*)malloc(sizeof(double) * 2 * n_parent * K);
    double* sw = (double*)malloc(sizeof(double) * 2 * n_parent);
    parent_totals(h, n_parent, n_bins, K, total_w, total_d);
    for (uint32_t b = 0; b < n_borders; ++b) {
        for (uint32_t p = 0; p < n_parent; ++p) {
            const double* cell = h + ((size_t)p * n_bins + b) * C;
            acc_w[p] += cell[K];
            sw[p] = acc_w[p];
            sw[p + n_parent] = total_w[p] - acc_w[p];
            for (int d = 0; d < K; ++d) {
                acc_d[p * K + d] += cell[d];
                sd[(size_t)d * 2 * n_parent + p] = acc_d[p * K + d];
                sd[(size_t)d * 2 * n_parent + p + n_parent] = total_d[p * K + d] - acc_d[p * K + d];
            }
        }
        scores[b] = fold_score(sd, sw, n_parent, K, score_fn, l2);
    }
    free(total_w); free(total_d); free(acc_w); free(acc_d); free(sd); free(sw);
}

/* scan_and_score_one_hot_bins_into (histogram.rs:1175-1287): per candidate value the TRUE
 * child is that one bin's cell, the FALSE child the per-parent total minus it (totals are
 * the same ordered bin sums as the border path); no prefix across candidates. */
static void scan_score_one_hot(const double* h, uint32_t n_parent, uint32_t n_bins, int K,
                               const uint32_t* values, uint32_t n_values, int score_fn,
                               double l2, double* scores) {
    const int C = K + 1;
    double* total_w = (double*)calloc(n_parent, sizeof(double));
    double* total_d = (double*)calloc((size_t)n_parent * K, sizeof(double));
    double* sd = (double*)malloc(sizeof(double) * 2 * n_parent * K);
    double* sw = (double*)malloc(sizeof(double) * 2 * n_parent);
    parent_totals(h, n_parent, n_bins, K, total_w, total_d);
    for (uint32_t v = 0; v < n_values; ++v) {
        const uint32_t b = values[v];
        for (uint32_t p = 0; p < n_parent; ++p) {
            const double* cell = h + ((size_t)p * n_bins + b) * C;
            sw[p] = total_w[p] - cell[K];
            sw[p + n_parent] = cell[K];
            for (int d = 0; d < K; ++d) {
                sd[(size_t)d * 2 * n_parent + p] = total_d[p * K + d] - cell[d];
                sd[(size_t)d * 2 * n_parent + p + n_parent] = cell[d];
            }
        }
        scores[v] = fold_score(sd, sw, n_parent, K, score_fn, l2);
    }
    free(total_w); free(total_d); free(sd); free(sw);
}

/* CTR context of one tree (see orc_params) */
typedef struct {
    uint32_t n_ctr;
    const uint32_t* bucket_count;
    const uint32_t* group;
    const uint8_t* used_model;   /* [n_ctr] groups chosen by an earlier tree */
    uint32_t n_cat;
    const uint32_t* cat_buckets;
    double model_size_reg;
} orc_ctr_ctx;

/* number of distinct (float-partition leaf, bucket) pairs (phantom_mixed_bucket_count,
 * tree.rs:3093-3100) */
static uint64_t distinct_pairs(const uint32_t* leaf_of, uint32_t leaf_mask, const uint32_t* bucket,
                               uint64_t n, uint32_t n_leaves) {
    uint32_t nb = 0;
    for (uint64_t i = 0; i < n; ++i) if (bucket[i] + 1 > nb) nb = bucket[i] + 1;
    uint8_t* seen = (uint8_t*)calloc((size_t)n_leaves * nb + 1, 1);
    uint64_t d = 0;
    for (uint64_t i = 0; i < n; ++i) {
        size_t k = (size_t)(leaf_of[i] & leaf_mask) * nb + bucket[i];
        if (!seen[k]) { seen[k] = 1; ++d; }
    }
    free(seen);
    return d;
}

/* (1 + count / max_count)^(-model_size_reg) (cat_feature_weight, tree.rs:2907-2913) */
static double cat_feature_weight(uint64_t count, uint64_t max_count, double msr) {
    if (msr == 0.0 || max_count == 0) return 1.0;
    double ratio = (double)count / (double)max_count;
    return pow(1.0 + ratio, -msr);
}

static int grow_tree_impl(const uint8_t* bins_fm, const uint32_t* n_borders, uint64_t n, uint32_t F,
                          const double* der, const double* w, int32_t K, int32_t depth, int32_t score_fn,
                          double l2, orc_rng* prng, int32_t n_threads, int32_t* out_splits,
                          double* out_scores, uint32_t* out_leaf_of, double* out_hists,
                          const uint8_t* one_hot, const orc_ctr_ctx* ctr);

int orc_grow_tree(const uint8_t* bins_fm, const uint32_t* n_borders, uint64_t n, uint32_t F,
                  const double* der, const double* w, int32_t K, int32_t depth, int32_t score_fn,
                  double l2, orc_rng* prng, int32_t n_threads, int32_t* out_splits,
                  double* out_scores, uint32_t* out_leaf_of, double* out_hists,
                  const uint8_t* one_hot) {
    return grow_tree_impl(bins_fm, n_borders, n, F, der, w, K, depth, score_fn, l2, prng, n_threads,
                          out_splits, out_scores, out_leaf_of, out_hists, one_hot, NULL);
}

static int grow_tree_impl(const uint8_t* bins_fm, const uint32_t* n_borders, uint64_t n, uint32_t F,
                          const double* der, const double* w, int32_t K, int32_t depth, int32_t score_fn,
                          double l2, orc_rng* prng, int32_t n_threads, int32_t* out_splits,
                          double* out_scores, uint32_t* out_leaf_of, double* out_hists,
                          const uint8_t* one_hot, const orc_ctr_ctx* ctr) {
    const int C = K + 1;
    uint32_t n_bins = 1;
    for (uint32_t f = 0; f < F; ++f)
        if (n_borders[f] + 1 > n_bins) n_bins = n_borders[f] + 1;
    uint32_t* leaf_of = out_leaf_of;
    memset(leaf_of, 0, sizeof(uint32_t) * n);
    double** hists = (double**)calloc(F, sizeof(double*));
    double** scores = (double**)calloc(F, sizeof(double*));
    /* one-hot candidates: one per DISTINCT bin of the whole column, ascending
     * (tree.rs:1305-1380 distinct_bins_ascending) */
    uint32_t** oh_values = (uint32_t**)calloc(F, sizeof(uint32_t*));
    uint32_t* n_cand = (uint32_t*)calloc(F, sizeof(uint32_t));
    for (uint32_t f = 0; f < F; ++f) {
        if (!(one_hot && one_hot[f])) { n_cand[f] = n_borders[f]; continue; }
        uint8_t seen[256] = {0};
        const uint8_t* col = bins_fm + (size_t)f * n;
        for (uint64_t o = 0; o < n; ++o) seen[col[o]] = 1;
        oh_values[f] = (uint32_t*)malloc(sizeof(uint32_t) * 256);
        for (uint32_t v = 0; v < 256; ++v)
            if (seen[v]) oh_values[f][n_cand[f]++] = v;
    }
    size_t hist_off = 0;
#ifdef _OPENMP
    int nt = n_threads > 0 ? n_threads : omp_get_max_threads();
#endif
    int rc = 0;
    for (int level = 0; level < depth; ++level) {
        uint32_t n_leaves = 1u << level;
        size_t per_f = (size_t)n_leaves * n_bins * C;
        if (prng) /* per-level rsm reselection draws, one per listed float feature (tree.rs:746-751) */
            for (uint32_t f = 0; f < F; ++f)
                if (!(one_hot && one_hot[f])) (void)orc_rng_real1(prng);
        uint64_t n_true = 0;
        if (level > 0) {
            uint32_t bit = 1u << (level - 1);
            for (uint64_t o = 0; o < n; ++o) n_true += (leaf_of[o] & bit) != 0;
        }
#ifdef _OPENMP
#pragma omp parallel num_threads(nt)
#endif
        {
            uint32_t* slot = level > 0 ? (uint32_t*)malloc(sizeof(uint32_t) * n) : NULL;
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
            for (int64_t fi = 0; fi < (int64_t)F; ++fi) {
                uint32_t f = (uint32_t)fi;
                if (n_cand[f] == 0) continue; /* never scored, never built (WR-04) */
                const uint8_t* col = bins_fm + (size_t)f * n;
                double* h = (double*)malloc(sizeof(double) * per_f);
                if (level == 0) {
                    build_hist(h, 1, n_bins, K, col, der, w, leaf_of, n);
                } else if (ctr) {
                    /* the CTR-aware search builds every leaf of the level directly, in object
                     * order (build_ctr_aware_histogram, tree.rs:3214-3225) */
                    build_hist(h, n_leaves, n_bins, K, col, der, w, leaf_of, n);
                } else {
                    derive_hist(h, hists[f], (uint32_t)level, n_bins, K, col, der, w, leaf_of, n,
                                slot, n_true);
                }
                free(hists[f]);
                hists[f] = h;
                free(scores[f]);
                scores[f] = (double*)malloc(sizeof(double) * n_cand[f]);
                if (oh_values[f])
                    scan_score_one_hot(h, n_leaves, n_bins, K, oh_values[f], n_cand[f], score_fn, l2,
                                       scores[f]);
                else
                    scan_score(h, n_leaves, n_bins, K, n_borders[f], score_fn, l2, scores[f]);
            }
            free(slot);
        }
        if (out_hists) {
            for (uint32_t f = 0; f < F; ++f) {
                double* dst = out_hists + hist_off;
                /* dump as [leaf][f][bin][ch] */
                for (uint32_t l = 0; l < n_leaves; ++l) {
                    double* d = dst + ((size_t)l * F + f) * n_bins * C;
                    if (hists[f]) memcpy(d, hists[f] + (size_t)l * n_bins * C, sizeof(double) * n_bins * C);
                    else memset(d, 0, sizeof(double) * n_bins * C);
                }
            }
            hist_off += per_f * F;
        }
        /* argmax, strict first-wins over (feature asc, border asc) (tree.rs:355-366).  The
         * perturbed search at random_strength 0 picks the same candidate (instance = raw + 0)
         * and consumes 1 gen_rand + one std_normal per listed feature on the main stream
         * (tree.rs:1525-1611); the per-feature sub-streams never touch the main stream. */
        /* one flat candidate list: every float (feature asc, border asc), then every one-hot
         * column (feature asc, value asc) (tree.rs:1261-1290, select_best :355-366) */
        /* CTR columns: score x the model_size_reg weight of a projection no earlier tree
         * and no earlier level of this tree used (tree.rs:3290-3340); max_count over the CTR
         * columns and, once a float split is chosen, over the distinct (float-partition leaf,
         * bucket) pairs of every CTR-eligible categorical column (tree.rs:3146-3178) */
        if (ctr && ctr->n_ctr) {
            uint64_t max_count = 0;
            for (uint32_t c = 0; c < ctr->n_ctr; ++c)
                if (ctr->bucket_count[c] > max_count) max_count = ctr->bucket_count[c];
            if (max_count == 0) max_count = 1;
            uint32_t float_mask = 0;
            for (int l = 0; l < level; ++l)
                if ((uint32_t)out_splits[l * 2] < F - ctr->n_ctr) float_mask |= 1u << l;
            if (float_mask)
                for (uint32_t c = 0; c < ctr->n_cat; ++c) {
                    uint64_t d = distinct_pairs(leaf_of, float_mask, ctr->cat_buckets + (size_t)c * n, n,
                                                1u << level);
                    if (d > max_count) max_count = d;
                }
            for (uint32_t c = 0; c < ctr->n_ctr; ++c) {
                const uint32_t f = F - ctr->n_ctr + c;
                int used = ctr->used_model[ctr->group[c]];
                for (int l = 0; l < level; ++l) {
                    uint32_t lf = (uint32_t)out_splits[l * 2];
                    if (lf >= F - ctr->n_ctr && ctr->group[lf - (F - ctr->n_ctr)] == ctr->group[c]) used = 1;
                }
                if (used || !scores[f]) continue;
                const double wgt = cat_feature_weight(ctr->bucket_count[c], max_count, ctr->model_size_reg);
                for (uint32_t k = 0; k < n_cand[f]; ++k) scores[f][k] = wgt * scores[f][k];
            }
        }
        int best_f = -1, best_b = -1, best_oh = 0;
        double best = -INFINITY;
        for (int pass = 0; pass < 2; ++pass)
            for (uint32_t f = 0; f < F; ++f) {
                if ((oh_values[f] != NULL) != (pass == 1)) continue;
                for (uint32_t c = 0; c < n_cand[f]; ++c)
                    if (scores[f][c] > best) {
                        best = scores[f][c];
                        best_f = (int)f;
                        best_b = pass ? (int)oh_values[f][c] : (int)c;
                        best_oh = pass;
                    }
            }
        if (prng) {
            (void)orc_rng_gen(prng);
            for (uint32_t f = 0; f < F; ++f)
                if (!(one_hot && one_hot[f])) (void)orc_std_normal(prng);
        }
        if (best_f < 0) { rc = -1; break; }
        out_splits[level * 2] = best_oh ? best_f | ORC_ONE_HOT_SPLIT : best_f;
        out_splits[level * 2 + 1] = best_b;
        if (out_scores) out_scores[level] = best;
        const uint8_t* col = bins_fm + (size_t)best_f * n;
        for (uint64_t o = 0; o < n; ++o) { /* advance_leaf_only; one-hot passes on equality */
            const int pass_bit = best_oh ? col[o] == (uint32_t)best_b : col[o] > (uint32_t)best_b;
            if (pass_bit) leaf_of[o] += n_leaves;
        }
    }
    for (uint32_t f = 0; f < F; ++f) { free(hists[f]); free(scores[f]); free(oh_values[f]); }
    free(hists);
    free(scores);
    free(oh_values);
    free(n_cand);
    return rc;
}


/* ======================================================================
 * Pairwise ranking: PairLogit / PairLogitPairwise
 *   pairs are given in the reference's competitor order: group ascending, winner
 *   ascending, insertion order within a winner (query_info.rs:205-250 builds
 *   competitors[winner] in input order; tree.rs:3790-3800 flattens them group by group).
 *   orc_pairs_order() produces that order from an arbitrary input order.
 * ==================================================================== */

/* Stable order of the pairs by winner (counting sort): out_perm[k] = input index. */
void orc_pairs_order(const uint32_t* winner, uint64_t m, uint64_t n, uint64_t* out_perm) {
    uint64_t* cnt = (uint64_t*)calloc(n + 1, sizeof(uint64_t));
    for (uint64_t k = 0; k < m; ++k) cnt[winner[k] + 1]++;
    for (uint64_t i = 0; i < n; ++i) cnt[i + 1] += cnt[i];
    for (uint64_t k = 0; k < m; ++k) out_perm[cnt[winner[k]]++] = k;
    free(cnt);
}

/* pairlogit_pair_prob (loss.rs:640-651). */
static double pairlogit_p(double winner_approx, double loser_approx) {
    double el = exp(loser_approx), ew = exp(winner_approx);
    double den = el + ew;
    return den > 0.0 ? el / den : 0.5;
}

/* pairlogit_group_der (ranking_der.rs:408-445): docs ascending, each winner's competitors
 * in order; a loser's der is decremented as each winner is visited, a winner's own der is
 * added after its competitor loop.  Groups are contiguous and pairs never cross groups,
 * so visiting all docs in global order is the per-group visit order. */
void orc_pairlogit_ders(const double* approx, uint64_t n, const uint32_t* winner,
                        const uint32_t* loser, const double* weight, uint64_t m, double* der1,
                        double* der2) {
    for (uint64_t i = 0; i < n; ++i) { der1[i] = 0.0; der2[i] = 0.0; }
    uint64_t k = 0;
    for (uint64_t doc = 0; doc < n; ++doc) {
        double wd = 0.0, wd2 = 0.0;
        for (; k < m && winner[k] == doc; ++k) {
            double p = pairlogit_p(approx[doc], approx[loser[k]]);
            double w = weight ? weight[k] : 1.0;
            wd += w * p;
            wd2 += w * p * (p - 1.0);
            der1[loser[k]] -= w * p;
            der2[loser[k]] += w * p * (p - 1.0);
        }
        der1[doc] += wd;
        der2[doc] += wd2;
    }
}

/* calc_pairwise_weights (boosting.rs:1760-1783): pw[obj] = sum of the weights of the pairs
 * incident on obj, in pair order. */
void orc_pairwise_weights(uint64_t n, const uint32_t* winner, const uint32_t* loser,
                          const double* weight, uint64_t m, double* pw) {
    for (uint64_t i = 0; i < n; ++i) pw[i] = 0.0;
    for (uint64_t k = 0; k < m; ++k) {
        double w = weight ? weight[k] : 1.0;
        pw[winner[k]] += w;
        pw[loser[k]] += w;
    }
}

/* MakeZeroAverage (pairwise_scoring.rs:255-265). */
static void make_zero_average(double* r, int n) {
    if (n == 0) return;
    double avg = 0.0;
    for (int i = 0; i < n; ++i) avg += r[i];
    avg /= (double)n;
    for (int i = 0; i < n; ++i) r[i] -= avg;
}

/* calculate_pairwise_leaf_values (pairwise_leaves.rs:120-200, pairwise_scoring.rs:283-345):
 * (n-1)x(n-1) SPD system with the bucket-weight prior, last value pinned to 0, then
 * zero-averaged.  w is n x n row-major. */
static void pairwise_leaf_values(const double* w, const double* der, int n, double l2,
                                 double prior, double* res) {
    if (n == 0) return;
    double cell_prior = 1.0 / (double)n;
    double non_diag = -prior * cell_prior;
    double diag = prior * (1.0 - cell_prior) + l2;
    if (n == 1) { res[0] = 0.0; return; }
    if (n == 2) {
        double den = w[0] + diag;
        res[0] = den != 0.0 ? der[0] / den : 0.0;
        res[1] = 0.0;
        make_zero_average(res, 2);
        return;
    }
    int m = n - 1;
    double* a = (double*)calloc((size_t)m * m, sizeof(double));
    for (int y = 0; y < m; ++y) {
        for (int x = 0; x < y; ++x) {
            double v = w[y * n + x] + non_diag;
            a[y * m + x] = v;
            a[x * m + y] = v;
        }
        a[y * m + y] = w[y * n + y] + diag;
    }
    if (!cholesky_solve(m, a, der, res))
        for (int i = 0; i < m; ++i) res[i] = 0.0;
    res[m] = 0.0;
    make_zero_average(res, n);
    free(a);
}

/* CalculateScore (pairwise_scoring.rs:352-375): sum_x a[x] (der[x] - 0.5 sum_y a[y] w[x][y]). */
static double pairwise_score_value(const double* a, const double* der, const double* w, int n) {
    double outer = 0.0;
    for (int x = 0; x < n; ++x) {
        double inner = 0.0;
        for (int y = 0; y < n; ++y) inner += a[y] * w[x * n + y];
        outer += a[x] * (der[x] - 0.5 * inner);
    }
    return outer;
}

static inline void wadd(double* w, int n, int r, int c, double d) { w[r * n + c] += d; }

/* calculate_pairwise_score (pairwise_scoring.rs:450-560) for one feature.
 *  ds     [P][B] der sums (doc-ascending scatter, compute_der_sums :101-135)
 *  st     [P][P][B][2] pair-weight statistics (smaller, greater_right; :163-196)
 *  scores [B-1] */
static void pairwise_scores(const double* ds, const double* st, int P, int B, double l2,
                            double prior, double* scores) {
    const int n = 2 * P;
    double* w = (double*)calloc((size_t)n * n, sizeof(double));
    double* der = (double*)calloc((size_t)n, sizeof(double));
    double* a = (double*)malloc(sizeof(double) * (size_t)n);
#define ST(x, y, b, c) st[((((size_t)(x) * P + (y)) * B + (b)) << 1) + (c)]
    for (int leaf = 0; leaf < P; ++leaf) {
        double t = 0.0;
        for (int b = 0; b < B; ++b) t += ds[(size_t)leaf * B + b];
        der[2 * leaf + 1] += t;
    }
    for (int y = 0; y < P; ++y)
        for (int x = y + 1; x < P; ++x) {
            double total = 0.0; /* buckets interleaved xy, yx (:480-490) */
            for (int b = 0; b < B; ++b) { total += ST(x, y, b, 0); total += ST(y, x, b, 0); }
            wadd(w, n, 2 * y + 1, 2 * x + 1, total);
            wadd(w, n, 2 * x + 1, 2 * y + 1, total);
            wadd(w, n, 2 * x + 1, 2 * x + 1, -total);
            wadd(w, n, 2 * y + 1, 2 * y + 1, -total);
        }
    for (int s = 0; s + 1 < B; ++s) {
        for (int y = 0; y < P; ++y) {
            double dd = ds[(size_t)y * B + s];
            der[2 * y] += dd;
            der[2 * y + 1] += -dd;
            double wd = ST(y, y, s, 0) - ST(y, y, s, 1);
            wadd(w, n, 2 * y, 2 * y + 1, wd);
            wadd(w, n, 2 * y + 1, 2 * y, wd);
            wadd(w, n, 2 * y, 2 * y, -wd);
            wadd(w, n, 2 * y + 1, 2 * y + 1, -wd);
            for (int x = y + 1; x < P; ++x) {
                double xs = ST(x, y, s, 0), xg = ST(x, y, s, 1);
                double ys = ST(y, x, s, 0), yg = ST(y, x, s, 1);
                double w00 = xg + yg, w01 = xs - xg, w10 = ys - yg, w11 = -(xs + ys);
                wadd(w, n, 2 * x, 2 * y, w00);
                wadd(w, n, 2 * y, 2 * x, w00);
                wadd(w, n, 2 * x, 2 * y + 1, w01);
                wadd(w, n, 2 * y + 1, 2 * x, w01);
                wadd(w, n, 2 * x + 1, 2 * y, w10);
                wadd(w, n, 2 * y, 2 * x + 1, w10);
                wadd(w, n, 2 * x + 1, 2 * y + 1, w11);
                wadd(w, n, 2 * y + 1, 2 * x + 1, w11);
                wadd(w, n, 2 * y, 2 * y, -(w00 + w10));
                wadd(w, n, 2 * x, 2 * x, -(w00 + w01));
                wadd(w, n, 2 * x + 1, 2 * x + 1, -(w10 + w11));
                wadd(w, n, 2 * y + 1, 2 * y + 1, -(w01 + w11));
            }
        }
        pairwise_leaf_values(w, der, n, l2, prior, a);
        scores[s] = pairwise_score_value(a, der, w, n);
    }
#undef ST
    free(w); free(der); free(a);
}

/* Pairwise statistics of one feature at one level (compute_der_sums :101-135 and
 * compute_pair_weight_statistics :163-196).  ds [P][B], st [P][P][B][2]. */
static void pairwise_stats(const uint8_t* col, const uint32_t* leaf_of, const double* der,
                           uint64_t n, const uint32_t* winner, const uint32_t* loser,
                           const double* weight, uint64_t m, int P, int B, double* ds,
                           double* st) {
    memset(ds, 0, sizeof(double) * (size_t)P * B);
    memset(st, 0, sizeof(double) * (size_t)P * P * B * 2);
    for (uint64_t i = 0; i < n; ++i) ds[(size_t)leaf_of[i] * B + col[i]] += der[i];
    for (uint64_t k = 0; k < m; ++k) {
        uint32_t wi = winner[k], lo = loser[k];
        if (wi == lo) continue;
        double w = weight ? weight[k] : 1.0;
        int wb = col[wi], lb = col[lo];
        int wl = (int)leaf_of[wi], ll = (int)leaf_of[lo];
        if (wb > lb) {
            st[((((size_t)ll * P + wl) * B + lb) << 1) + 0] -= w;
            st[((((size_t)ll * P + wl) * B + wb) << 1) + 1] -= w;
        } else {
            st[((((size_t)wl * P + ll) * B + wb) << 1) + 0] -= w;
            st[((((size_t)wl * P + ll) * B + lb) << 1) + 1] -= w;
        }
    }
}

/* Pairwise scores of every border of one feature at one level (test entry). */
void orc_pairwise_feature_scores(const uint8_t* col, const uint32_t* leaf_of, const double* der,
                                 uint64_t n, const uint32_t* winner, const uint32_t* loser,
                                 const double* weight, uint64_t m, int32_t P, int32_t B, double l2,
                                 double prior, double* scores) {
    double* ds = (double*)malloc(sizeof(double) * (size_t)P * B);
    double* st = (double*)malloc(sizeof(double) * (size_t)P * P * B * 2);
    pairwise_stats(col, leaf_of, der, n, winner, loser, weight, m, P, B, ds, st);
    pairwise_scores(ds, st, P, B, l2, prior, scores);
    free(ds);
    free(st);
}

int orc_grow_tree_pairwise(const uint8_t* bins_fm, const uint32_t* n_borders, uint64_t n,
                           uint32_t F, const double* der, const uint32_t* winner,
                           const uint32_t* loser, const double* weight, uint64_t m,
                           int32_t depth, double l2, double prior, int32_t n_threads,
                           int32_t* out_splits, double* out_scores, uint32_t* out_leaf_of) {
    uint32_t* leaf_of = out_leaf_of;
    memset(leaf_of, 0, sizeof(uint32_t) * n);
    double** scores = (double**)calloc(F, sizeof(double*));
#ifdef _OPENMP
    int nt = n_threads > 0 ? n_threads : omp_get_max_threads();
#endif
    int rc = 0;
    for (int level = 0; level < depth; ++level) {
        const int P = 1 << level;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#endif
        for (int64_t fi = 0; fi < (int64_t)F; ++fi) {
            uint32_t f = (uint32_t)fi;
            free(scores[f]);
            scores[f] = NULL;
            if (n_borders[f] == 0) continue;
            const int B = (int)n_borders[f] + 1;
            double* ds = (double*)malloc(sizeof(double) * (size_t)P * B);
            double* st = (double*)malloc(sizeof(double) * (size_t)P * P * B * 2);
            pairwise_stats(bins_fm + (size_t)f * n, leaf_of, der, n, winner, loser, weight, m, P, B,
                           ds, st);
            scores[f] = (double*)malloc(sizeof(double) * (size_t)(B - 1));
            pairwise_scores(ds, st, P, B, l2, prior, scores[f]);
            free(ds);
            free(st);
        }
        /* select_level_pairwise (tree.rs:3852-3900): feature asc, border asc, strict > */
        int best_f = -1, best_b = -1;
        double best = -INFINITY;
        for (uint32_t f = 0; f < F; ++f)
            for (uint32_t b = 0; b < n_borders[f]; ++b)
                if (scores[f][b] > best) { best = scores[f][b]; best_f = (int)f; best_b = (int)b; }
        if (best_f < 0) { rc = -1; break; }
        out_splits[level * 2] = best_f;
        out_splits[level * 2 + 1] = best_b;
        if (out_scores) out_scores[level] = best;
        const uint8_t* col = bins_fm + (size_t)best_f * n;
        for (uint64_t o = 0; o < n; ++o)
            if (col[o] > (uint32_t)best_b) leaf_of[o] += (uint32_t)P;
    }
    for (uint32_t f = 0; f < F; ++f) free(scores[f]);
    free(scores);
    return rc;
}

/* compute_pairwise_leaf_deltas (pairwise_leaves.rs:219-238): per-leaf weight sums from the
 * pairs (compute_pairwise_weight_sums :47-88, same-leaf pairs skipped), per-leaf der sums
 * (docs ascending), then the pairwise leaf solve. */
void orc_pairwise_leaf_deltas(const uint32_t* leaf_of, uint64_t n, const double* der,
                              const uint32_t* winner, const uint32_t* loser, const double* weight,
                              uint64_t m, uint32_t n_leaves, double l2, double prior, double* out) {
    double* w = (double*)calloc((size_t)n_leaves * n_leaves, sizeof(double));
    double* ds = (double*)calloc(n_leaves, sizeof(double));
    for (uint64_t k = 0; k < m; ++k) {
        uint32_t wl = leaf_of[winner[k]], ll = leaf_of[loser[k]];
        if (wl == ll) continue;
        double x = weight ? weight[k] : 1.0;
        w[(size_t)wl * n_leaves + ll] -= x;
        w[(size_t)ll * n_leaves + wl] -= x;
        w[(size_t)wl * n_leaves + wl] += x;
        w[(size_t)ll * n_leaves + ll] += x;
    }
    for (uint64_t i = 0; i < n; ++i) ds[leaf_of[i]] += der[i];
    pairwise_leaf_values(w, ds, (int)n_leaves, l2, prior, out);
    free(w);
    free(ds);
}

/* normalize_leaf_values for pairwise losses (boosting.rs:2844-2875): subtract the
 * document-weighted mean leaf value; leaves with |weight| <= 1e-9 become 0. */
static void pairwise_center(double* v, const double* leaf_w, uint32_t n_leaves) {
    double total = 0.0;
    for (uint32_t l = 0; l < n_leaves; ++l) total += leaf_w[l];
    if (!(fabs(total) > 1e-9)) return;
    double weighted = 0.0;
    for (uint32_t l = 0; l < n_leaves; ++l) weighted += v[l] * leaf_w[l];
    double avg = weighted / total;
    for (uint32_t l = 0; l < n_leaves; ++l) {
        if (fabs(leaf_w[l]) > 1e-9) v[l] -= avg;
        else v[l] = 0.0;
    }
}

/* ======================================================================
 * Border selection: GreedyLogSum / GreedyMinEntropy (crates/cb-data/src/borders.rs,
 * restating catboost's library/cpp/grid_creator/binarization.cpp).
 * ==================================================================== */
#define ORC_MAX_SUBSET_FOR_BORDERS 200000 /* borders.rs:48 */

/* sample_indices_for_build_borders (borders.rs:504-516): partial Fisher-Yates with
 * TFastRng64::from_seed(0), ascending index set. */
void orc_sample_indices_for_borders(uint64_t n, uint64_t sample_size, uint32_t* out) {
    uint32_t* idx = (uint32_t*)malloc(sizeof(uint32_t) * (n ? n : 1));
    for (uint64_t i = 0; i < n; ++i) idx[i] = (uint32_t)i;
    orc_rng r;
    orc_rng_from_seed(&r, 0);
    uint64_t take = sample_size < n ? sample_size : n;
    for (uint64_t i = 0; i < take; ++i) {
        uint64_t off = orc_rng_uniform(&r, n - i);
        uint32_t t = idx[i]; idx[i] = idx[i + off]; idx[i + off] = t;
    }
    /* ascending */
    uint8_t* mark = (uint8_t*)calloc(n ? n : 1, 1);
    for (uint64_t i = 0; i < take; ++i) mark[idx[i]] = 1;
    uint64_t k = 0;
    for (uint64_t i = 0; i < n; ++i) if (mark[i]) out[k++] = (uint32_t)i;
    free(mark);
    free(idx);
}

static double border_penalty(int kind, double w) { /* borders.rs:51-62 */
    return kind == 0 ? -log(w + 1e-8) : w * log(w + 1e-8);
}

typedef struct { uint64_t start, end, best; double score; uint64_t seq; } orc_gbin;

static uint64_t lb_f32(const float* v, uint64_t lo, uint64_t hi, float t) { /* borders.rs:228 */
    while (lo < hi) { uint64_t mid = lo + (hi - lo) / 2; if (v[mid] < t) lo = mid + 1; else hi = mid; }
    return lo;
}
static uint64_t ub_f32(const float* v, uint64_t lo, uint64_t hi, float t) { /* borders.rs:244 */
    while (lo < hi) { uint64_t mid = lo + (hi - lo) / 2; if (v[mid] <= t) lo = mid + 1; else hi = mid; }
    return lo;
}
static double gbin_score(const orc_gbin* b, uint64_t pos, int kind) { /* CalcSplitScore */
    if (pos == b->start || pos == b->end) return -INFINITY;
    double left = -border_penalty(kind, (double)(pos - b->start));
    double right = -border_penalty(kind, (double)(b->end - pos));
    double curr = -border_penalty(kind, (double)(b->end - b->start));
    return left + right - curr;
}
static void gbin_update(orc_gbin* b, const float* v, int kind) { /* UpdateBestSplitProperties */
    uint64_t mid = b->start + (b->end - b->start) / 2;
    float mv = v[mid];
    uint64_t lb = lb_f32(v, b->start, mid, mv);
    uint64_t ub = ub_f32(v, mid, b->end, mv);
    double sl = gbin_score(b, lb, kind), sr = gbin_score(b, ub, kind);
    if (sl >= sr) { b->best = lb; b->score = sl; } else { b->best = ub; b->score = sr; }
}

static int cmp_f32(const void* a, const void* b) {
    float x = *(const float*)a, y = *(const float*)b;
    return x < y ? -1 : (x > y ? 1 : 0);
}

/* Greedy border selection of one column (borders.rs:298-345 + 400-470 + 572-640):
 * values with NaNs, sampled when n > 200000; returns the count written to out
 * (<= border_count, sentinel f32::MIN first when nan_sentinel). kind 0 = MaxSumLog
 * (GreedyLogSum), 1 = MinEntropy (GreedyMinEntropy). */
uint32_t orc_select_borders_greedy(const float* column, uint64_t n, uint32_t border_count,
                                   int32_t nan_sentinel, int32_t kind, double* out) {
    float* v = (float*)malloc(sizeof(float) * (n ? n : 1));
    uint64_t m = 0;
    if (n > ORC_MAX_SUBSET_FOR_BORDERS) {
        uint32_t* s = (uint32_t*)malloc(sizeof(uint32_t) * ORC_MAX_SUBSET_FOR_BORDERS);
        orc_sample_indices_for_borders(n, ORC_MAX_SUBSET_FOR_BORDERS, s);
        for (uint64_t i = 0; i < ORC_MAX_SUBSET_FOR_BORDERS; ++i)
            if (!isnan(column[s[i]])) v[m++] = column[s[i]];
        free(s);
    } else {
        for (uint64_t i = 0; i < n; ++i) if (!isnan(column[i])) v[m++] = column[i];
    }
    qsort(v, m, sizeof(float), cmp_f32);
    uint32_t budget = nan_sentinel ? (border_count > 0 ? border_count - 1 : 0) : border_count;
    float* b32 = (float*)malloc(sizeof(float) * (budget + 2));
    uint32_t nb = 0;
    if (m >= 2) {
        orc_gbin* q = (orc_gbin*)malloc(sizeof(orc_gbin) * (budget + 3));
        uint64_t nq = 0, seq = 0;
        q[0].start = 0; q[0].end = m; q[0].seq = seq++;
        gbin_update(&q[0], v, kind);
        nq = 1;
        while (nq <= budget) {
            /* top: highest score, earliest insertion on ties (borders.rs:600-640) */
            uint64_t top = 0;
            for (uint64_t i = 1; i < nq; ++i)
                if (q[i].score > q[top].score || (q[i].score == q[top].score && q[i].seq < q[top].seq)) top = i;
            if (!(q[top].start != q[top].best && q[top].end != q[top].best)) break;
            orc_gbin t = q[top];
            q[top] = q[nq - 1];
            --nq;
            orc_gbin left;
            left.start = t.start; left.end = t.best; left.seq = seq++;
            gbin_update(&left, v, kind);
            t.start = t.best; t.seq = seq++;
            gbin_update(&t, v, kind);
            q[nq++] = left;
            q[nq++] = t;
        }
        for (uint64_t i = 0; i < nq; ++i) {
            if (q[i].start == 0) continue;
            float border = 0.5f * v[q[i].start - 1];
            border += 0.5f * v[q[i].start];
            if (border == 0.0f) border = 0.0f;  /* -0 -> +0 */
            b32[nb++] = border;
        }
        free(q);
    }
    qsort(b32, nb, sizeof(float), cmp_f32);
    uint32_t k = 0;
    if (nan_sentinel) out[k++] = (double)(-3.40282346638528859812e+38F);
    for (uint32_t i = 0; i < nb; ++i)
        if (i == 0 || b32[i] != b32[i - 1]) out[k++] = (double)b32[i];
    free(b32);
    free(v);
    return k;
}

/* ======================================================================
 * Model apply (crates/cb-model/src/apply.rs predict_raw_one; device twin
 * crates/cb-backend/src/kernels.rs:629 apply_oblivious_float_kernel): per object, each
 * tree's leaf from its float splits (value > border, forward bit order; NaN passes only
 * for a feature flagged nan_as_true, apply.rs:160-166), contributions summed in tree order
 * from 0, bias added once after the trees.  Leaf values of tree t are
 * leaf_values[(tree_leaf_offsets[t] + leaf) * K + d]; out is dim-major [K][n].
 * ==================================================================== */
int orc_apply_oblivious(const float* x_fm, uint64_t n, uint32_t F, const uint32_t* split_features,
                        const double* split_borders, const uint32_t* tree_split_offsets,
                        const double* leaf_values, const uint32_t* tree_leaf_offsets,
                        uint32_t n_trees, uint32_t K, const double* bias,
                        const uint8_t* nan_as_true, double* out) {
    for (uint64_t i = 0; i < n; ++i) {
        for (uint32_t d = 0; d < K; ++d) {
            double acc = 0.0;
            for (uint32_t t = 0; t < n_trees; ++t) {
                uint32_t leaf = 0, bit = 0;
                for (uint32_t s = tree_split_offsets[t]; s < tree_split_offsets[t + 1]; ++s, ++bit) {
                    uint32_t f = split_features[s];
                    int pass = 0;
                    if (f < F) {
                        float v = x_fm[(size_t)f * n + i];
                        pass = isnan(v) ? (nan_as_true && nan_as_true[f]) : ((double)v > split_borders[s]);
                    }
                    leaf |= (uint32_t)pass << bit;
                }
                uint32_t li = tree_leaf_offsets[t] + leaf;
                acc += li < tree_leaf_offsets[t + 1] ? leaf_values[(size_t)li * K + d] : 0.0;
            }
            out[(size_t)d * n + i] = acc + (bias ? bias[d] : 0.0);
        }
    }
    return 0;
}

/* ======================================================================
 * Boosting loop -- CPU branch of crates/cb-train/src/boosting.rs:7300-8900
 * (Plain boosting, SymmetricTree, random_strength 0, pointwise losses).
 * ==================================================================== */
#define PRE_TREE_DRAWS 2        /* boosting.rs:59 */
#define POST_TREE_EXTRA_DRAWS 2 /* boosting.rs:69 */

int orc_train(const orc_params* p, const uint8_t* bins_fm, const uint32_t* n_borders, uint64_t n,
              uint32_t F, const double* target, const double* weight, int32_t* out_splits,
              double* out_leaf_values, double* out_approx, double* out_staged,
              double* out_bias) {
    const int K = p->loss == ORC_LOSS_MULTICLASS ? p->approx_dim : 1;
    /* the learning rate that multiplies every leaf is the f32-representable one
     * (boosting.rs:4958) */
    const double lr = (double)(float)p->learning_rate;
    int any_one_hot = 0;
    for (uint32_t f = 0; p->one_hot_flags && f < F; ++f) any_one_hot |= p->one_hot_flags[f] != 0;
    /* one-hot columns with active RNG draws are refused (boosting.rs:5744-5756) */
    if (any_one_hot && p->bootstrap_type != ORC_BOOT_NO) return -4;
    /* ranking losses over explicit pairs (boosting.rs:1716-1783): PairLogit scores with the
     * pointwise histogram over pairwise weights; PairLogitPairwise with the pairwise
     * statistics (tree.rs:3930-3974) and solves its leaves by Cholesky (pairwise_leaves.rs) */
    const int ranking = p->loss == ORC_LOSS_PAIRLOGIT || p->loss == ORC_LOSS_PAIRLOGIT_PAIRWISE;
    const int pairwise_scoring = p->loss == ORC_LOSS_PAIRLOGIT_PAIRWISE;
    if (ranking && (weight || any_one_hot)) return -4;
    if (pairwise_scoring && p->bootstrap_type != ORC_BOOT_NO) return -4;
    const double prior = p->pairwise_non_diag_reg;
    uint32_t *pw_win = NULL, *pw_los = NULL;
    double *pw_wt = NULL, *pw = NULL;
    const uint64_t m = ranking ? p->n_pairs : 0;
    if (ranking) {
        uint64_t* perm = (uint64_t*)malloc(sizeof(uint64_t) * (m + 1));
        orc_pairs_order(p->pair_winner, m, n, perm);
        pw_win = (uint32_t*)malloc(sizeof(uint32_t) * (m + 1));
        pw_los = (uint32_t*)malloc(sizeof(uint32_t) * (m + 1));
        pw_wt = (double*)malloc(sizeof(double) * (m + 1));
        for (uint64_t k = 0; k < m; ++k) {
            pw_win[k] = p->pair_winner[perm[k]];
            pw_los[k] = p->pair_loser[perm[k]];
            pw_wt[k] = p->pair_weight ? p->pair_weight[perm[k]] : 1.0;
        }
        free(perm);
        pw = (double*)malloc(sizeof(double) * n);
        orc_pairwise_weights(n, pw_win, pw_los, pw_wt, m, pw);
    }
    const int depth = p->depth;
    const uint32_t n_leaves = 1u << depth;
    const int pk = K * (K + 1) / 2;
    double* w = (double*)malloc(sizeof(double) * n);
    for (uint64_t i = 0; i < n; ++i) w[i] = weight ? weight[i] : 1.0;
    double* approx = (double*)malloc(sizeof(double) * n * K);
    double bias = 0.0; /* starting_approx (boosting.rs:1871-1877) */
    if (p->boost_from_average && p->loss == ORC_LOSS_RMSE && n > 0) {
        double s = 0.0;
        for (uint64_t i = 0; i < n; ++i) s += target[i];
        bias = s / (double)n;
    }
    for (uint64_t i = 0; i < n * K; ++i) approx[i] = bias;
    if (out_bias) *out_bias = bias;

    double sum_w = 0.0;
    for (uint64_t i = 0; i < n; ++i) sum_w += w[i];
    double scaled_l2 = n == 0 ? p->l2_leaf_reg : p->l2_leaf_reg * (sum_w / (double)n);

    orc_rng rng;
    orc_rng_from_seed(&rng, p->random_seed);
    int draws_active = p->bootstrap_type != ORC_BOOT_NO;

    double* d1 = (double*)malloc(sizeof(double) * n * K);
    double* d2 = (double*)malloc(sizeof(double) * n * (p->loss == ORC_LOSS_MULTICLASS ? pk : 1));
    double* wd = (double*)malloc(sizeof(double) * n * K);
    double* sder = (double*)malloc(sizeof(double) * n * K);
    double* swt = (double*)malloc(sizeof(double) * n);
    double* samp = (double*)malloc(sizeof(double) * n);
    uint8_t* ctrl = (uint8_t*)malloc(n);
    uint32_t* leaf_of = (uint32_t*)malloc(sizeof(uint32_t) * n);
    double* leaf_vals = (double*)malloc(sizeof(double) * n_leaves * K);
    uint8_t* used_groups = (uint8_t*)calloc(p->n_ctr + 1, 1);
    int rc = 0;
    if (p->n_ctr && (any_one_hot || ranking || p->n_ctr > F)) rc = -4;

    for (int it = 0; it < p->iterations; ++it) {
        /* derivatives of the current approx */
        if (p->loss == ORC_LOSS_MULTICLASS) {
            double a[64], dd1[64], dd2[64 * 65 / 2];
            for (uint64_t i = 0; i < n; ++i) {
                for (int d = 0; d < K; ++d) a[d] = approx[(size_t)d * n + i];
                softmax_ders(a, K, (int)target[i], dd1, dd2);
                for (int d = 0; d < K; ++d) d1[(size_t)d * n + i] = dd1[d];
                for (int j = 0; j < pk; ++j) d2[i * pk + j] = dd2[j];
            }
        } else if (ranking) {
            orc_pairlogit_ders(approx, n, pw_win, pw_los, pw_wt, m, d1, d2);
        } else {
            orc_ders(p->loss, approx, target, n, d1, d2);
        }
        for (uint64_t x = 0; x < n * K; ++x) wd[x] = d1[x] * w[x % n];
        if (draws_active)
            for (int k = 0; k < PRE_TREE_DRAWS; ++k) (void)orc_rng_gen(&rng);
        orc_bootstrap(p->bootstrap_type, n, p->subsample, p->bagging_temperature, &rng, samp, ctrl);
        for (uint64_t x = 0; x < n * K; ++x) {
            uint64_t i = x % n;
            sder[x] = ctrl[i] ? wd[x] * samp[i] : 0.0;
        }
        /* the histogram weight of a pairwise-weight loss is the pairwise weight
         * (eff_weights, boosting.rs:7575-7579) */
        for (uint64_t i = 0; i < n; ++i) swt[i] = ctrl[i] ? (ranking ? pw[i] : w[i]) * samp[i] : 0.0;

        int32_t* splits = out_splits + (size_t)it * depth * 2;
        orc_ctr_ctx cctx;
        if (p->n_ctr) {
            cctx.n_ctr = p->n_ctr;
            cctx.bucket_count = p->ctr_bucket_count;
            cctx.group = p->ctr_group;
            cctx.used_model = used_groups;
            cctx.n_cat = p->n_cat;
            cctx.cat_buckets = p->cat_buckets;
            cctx.model_size_reg = p->model_size_reg;
        }
        if (p->n_ctr)   /* the CTR search draws nothing per level */
            rc = grow_tree_impl(bins_fm, n_borders, n, F, sder, swt, K, depth, p->score_function, scaled_l2,
                                NULL, p->n_threads, splits, NULL, leaf_of, NULL, p->one_hot_flags, &cctx);
        else if (pairwise_scoring)
            rc = orc_grow_tree_pairwise(bins_fm, n_borders, n, F, d1, pw_win, pw_los, pw_wt, m, depth,
                                        p->l2_leaf_reg, prior, p->n_threads, splits, NULL, leaf_of);
        else
            rc = orc_grow_tree(bins_fm, n_borders, n, F, sder, swt, K, depth, p->score_function,
                               scaled_l2, draws_active ? &rng : NULL, p->n_threads, splits, NULL,
                               leaf_of, NULL, p->one_hot_flags);
        if (rc) break;
        if (p->n_ctr) {
            /* leaf values and approx over the averaging-permutation columns: every CTR level
             * re-tests its column's averaging bins, float levels keep their bit */
            const uint32_t fc0 = F - p->n_ctr;
            for (int l = 0; l < depth; ++l) {
                uint32_t f = (uint32_t)splits[l * 2];
                if (f < fc0) continue;
                used_groups[p->ctr_group[f - fc0]] = 1;
                const uint8_t* avg = p->ctr_avg_bins + (size_t)(f - fc0) * n;
                const uint32_t b = (uint32_t)splits[l * 2 + 1];
                for (uint64_t i = 0; i < n; ++i)
                    leaf_of[i] = (leaf_of[i] & ~(1u << l)) | ((uint32_t)(avg[i] > b) << l);
            }
        }

        /* leaf values on the UNSAMPLED derivatives (boosting.rs:2470-2560, :2634) */
        if (p->loss == ORC_LOSS_MULTICLASS) {
            double* sd = (double*)calloc((size_t)n_leaves * K, sizeof(double));
            double* s2 = (double*)calloc((size_t)n_leaves * pk, sizeof(double));
            for (uint64_t i = 0; i < n; ++i) {
                uint32_t l = leaf_of[i];
                for (int d = 0; d < K; ++d) sd[(size_t)l * K + d] += wd[(size_t)d * n + i];
                for (int j = 0; j < pk; ++j) s2[(size_t)l * pk + j] += d2[i * pk + j] * w[i];
            }
            for (uint32_t l = 0; l < n_leaves; ++l) {
                double delta[64];
                solve_symmetric_newton(K, sd + (size_t)l * K, s2 + (size_t)l * pk, scaled_l2, delta);
                for (int d = 0; d < K; ++d) leaf_vals[(size_t)d * n_leaves + l] = delta[d];
            }
            free(sd);
            free(s2);
        } else if (pairwise_scoring) {
            orc_pairwise_leaf_deltas(leaf_of, n, d1, pw_win, pw_los, pw_wt, m, n_leaves,
                                     p->l2_leaf_reg, prior, leaf_vals);
        } else {
            double sd[1 << 12], s2[1 << 12];
            for (uint32_t l = 0; l < n_leaves; ++l) { sd[l] = 0.0; s2[l] = 0.0; }
            for (uint64_t i = 0; i < n; ++i) {
                uint32_t l = leaf_of[i];
                sd[l] += wd[i];
                if (p->leaf_method == ORC_LEAF_NEWTON) s2[l] += d2[i] * w[i];
                else s2[l] += ranking ? pw[i] : w[i]; /* Gradient sumWeight (boosting.rs:8352-8380) */
            }
            for (uint32_t l = 0; l < n_leaves; ++l)
                leaf_vals[l] = p->leaf_method == ORC_LEAF_NEWTON
                                   ? newton_leaf_delta(sd[l], s2[l], scaled_l2)
                                   : calc_average(sd[l], s2[l], scaled_l2);
        }
        /* NormalizeLeafValues (boosting.rs:2844-2882): pairwise-weight losses first subtract
         * the document-weighted mean leaf value; every loss is then scaled by the learning
         * rate; then approx += leaf value (boosting.rs:8560-8572) */
        if (ranking) {
            double lw[1 << 12];
            for (uint32_t l = 0; l < n_leaves; ++l) lw[l] = 0.0;
            for (uint64_t i = 0; i < n; ++i) lw[leaf_of[i]] += w[i];
            pairwise_center(leaf_vals, lw, n_leaves);
        }
        for (uint32_t x = 0; x < n_leaves * K; ++x) leaf_vals[x] *= lr;
        for (int d = 0; d < K; ++d)
            for (uint64_t i = 0; i < n; ++i)
                approx[(size_t)d * n + i] += leaf_vals[(size_t)d * n_leaves + leaf_of[i]];
        if (out_leaf_values)
            memcpy(out_leaf_values + (size_t)it * n_leaves * K, leaf_vals,
                   sizeof(double) * n_leaves * K);
        if (out_staged) memcpy(out_staged + (size_t)it * n * K, approx, sizeof(double) * n * K);
        if (draws_active)
            for (int k = 0; k < POST_TREE_EXTRA_DRAWS; ++k) (void)orc_rng_gen(&rng);
    }
    if (out_approx) memcpy(out_approx, approx, sizeof(double) * n * K);
    free(w); free(approx); free(d1); free(d2); free(wd); free(sder); free(swt); free(samp);
    free(ctrl); free(leaf_of); free(leaf_vals); free(used_groups);
    free(pw_win); free(pw_los); free(pw_wt); free(pw);
    return rc;
}


/* ======================================================================
 * Categorical inputs: permutations, first-seen bins, online CTR columns
 * ==================================================================== */
static void shuffle_from(uint64_t n, orc_rng* r, uint32_t* v) { /* permutation.rs shuffle_in_place */
    for (uint64_t i = 0; i < n; ++i) v[i] = (uint32_t)i;
    for (uint64_t i = 1; i < n; ++i) {
        uint64_t j = orc_rng_uniform(r, i + 1);
        uint32_t t = v[i]; v[i] = v[j]; v[j] = t;
    }
}

void orc_shuffled_indices(uint64_t n, uint64_t seed, uint32_t* out) {
    orc_rng r;
    orc_rng_from_seed(&r, seed);
    shuffle_from(n, &r, out);
}

void orc_permutations(uint64_t n, uint32_t count, uint64_t seed, uint32_t* out) {
    orc_rng r;
    orc_rng_from_seed(&r, seed);
    for (uint32_t k = 0; k < count; ++k) shuffle_from(n, &r, out + (size_t)k * n);
}

typedef struct { uint32_t key; uint32_t idx; } orc_key_idx;
static int cmp_key_idx(const void* a, const void* b) {
    const orc_key_idx* x = (const orc_key_idx*)a;
    const orc_key_idx* y = (const orc_key_idx*)b;
    if (x->key != y->key) return x->key < y->key ? -1 : 1;
    return x->idx < y->idx ? -1 : (x->idx > y->idx);
}

uint32_t orc_perfect_hash(const uint32_t* keys, uint64_t n, uint32_t* bins) {
    /* first occurrence of every key, then keys ranked by their first occurrence */
    orc_key_idx* a = (orc_key_idx*)malloc(sizeof(orc_key_idx) * (n ? n : 1));
    for (uint64_t i = 0; i < n; ++i) { a[i].key = keys[i]; a[i].idx = (uint32_t)i; }
    qsort(a, n, sizeof(orc_key_idx), cmp_key_idx);
    uint32_t* first = (uint32_t*)malloc(sizeof(uint32_t) * (n ? n : 1));  /* first idx per object */
    uint64_t d = 0;
    orc_key_idx* heads = (orc_key_idx*)malloc(sizeof(orc_key_idx) * (n ? n : 1));
    for (uint64_t i = 0; i < n; ++i) {
        if (i == 0 || a[i].key != a[i - 1].key) { heads[d].key = a[i].idx; heads[d].idx = (uint32_t)d; ++d; }
        first[a[i].idx] = (uint32_t)(d - 1);  /* segment id of the object */
    }
    qsort(heads, d, sizeof(orc_key_idx), cmp_key_idx);  /* by first index */
    uint32_t* rank = (uint32_t*)malloc(sizeof(uint32_t) * (d ? d : 1));
    for (uint64_t r = 0; r < d; ++r) rank[heads[r].idx] = (uint32_t)r;
    for (uint64_t i = 0; i < n; ++i) bins[i] = rank[first[i]];
    free(a); free(first); free(heads); free(rank);
    return (uint32_t)d;
}

/* calc_normalization (calc_ctr.rs): shift = -min(0, prior), norm = max(1, prior) - min(0, prior) */
static void ctr_norm(double prior, double* shift, double* norm) {
    double left = prior < 0.0 ? prior : 0.0;
    double right = prior > 1.0 ? prior : 1.0;
    *shift = -left;
    *norm = right - left;
}

static uint8_t ctr_clamp_bin(double bin_f, uint32_t border_count) {
    double t = trunc(bin_f);
    if (t < 0.0) return 0;
    if (t > (double)border_count) return (uint8_t)border_count;
    return (uint8_t)t;
}

int orc_ctr_column(int32_t ctr_type, uint32_t target_border_idx, double prior_num, double prior_denom,
                   uint32_t border_count, const uint32_t* bucket, uint32_t n_buckets, uint64_t n,
                   const uint32_t* permutation, const uint8_t* target_class, double* good,
                   int64_t* total, double* value, uint8_t* bin) {
    if (prior_denom == 0.0) return -3;
    if (border_count > 255) return -2;
    const double prior = prior_num / prior_denom;
    double shift, norm;
    ctr_norm(prior, &shift, &norm);
    double* g = (double*)malloc(sizeof(double) * (n ? n : 1));
    int64_t* t = (int64_t*)malloc(sizeof(int64_t) * (n ? n : 1));
    int f32_bins = 0;
    if (ctr_type == ORC_CTR_COUNTER) {  /* whole-set bucket counts, max count denominator */
        int64_t* cnt = (int64_t*)calloc(n_buckets ? n_buckets : 1, sizeof(int64_t));
        for (uint64_t i = 0; i < n; ++i) cnt[bucket[i]] += 1;
        int64_t den = 0;
        for (uint32_t b = 0; b < n_buckets; ++b) if (cnt[b] > den) den = cnt[b];
        for (uint64_t i = 0; i < n; ++i) { g[i] = (double)cnt[bucket[i]]; t[i] = den; }
        free(cnt);
    } else if (ctr_type == ORC_CTR_BTMV) {  /* online_mean_prefix: f32 running sum of class/1 */
        float* sum = (float*)calloc(n_buckets ? n_buckets : 1, sizeof(float));
        int64_t* cnt = (int64_t*)calloc(n_buckets ? n_buckets : 1, sizeof(int64_t));
        for (uint64_t p = 0; p < n; ++p) {
            uint32_t doc = permutation[p], b = bucket[doc];
            g[doc] = (double)sum[b];
            t[doc] = cnt[b];
            sum[b] += (float)target_class[doc] / 1.0f;
            cnt[b] += 1;
        }
        free(sum); free(cnt);
        f32_bins = 1;
    } else if (ctr_type == ORC_CTR_BORDERS || ctr_type == ORC_CTR_BUCKETS) {
        /* online_class_prefix_column: read the bucket's class counts, then increment */
        int64_t* cnt = (int64_t*)calloc((size_t)(n_buckets ? n_buckets : 1) * 2, sizeof(int64_t));
        for (uint64_t p = 0; p < n; ++p) {
            uint32_t doc = permutation[p], b = bucket[doc];
            int64_t n0 = cnt[2 * (size_t)b], n1 = cnt[2 * (size_t)b + 1];
            int64_t tot = n0 + n1, num;
            if (ctr_type == ORC_CTR_BUCKETS) num = target_border_idx == 0 ? n0 : (target_border_idx == 1 ? n1 : 0);
            else num = tot - (target_border_idx == 0 ? n0 : n0 + n1);
            g[doc] = (double)num;
            t[doc] = tot;
            if (target_class[doc] < 2) cnt[2 * (size_t)b + target_class[doc]] += 1;
        }
        free(cnt);
    } else {
        free(g); free(t);
        return -4;
    }
    for (uint64_t i = 0; i < n; ++i) {
        double v = (g[i] + prior) / ((double)t[i] + 1.0);  /* calc_ctr_online */
        if (value) value[i] = v;
        if (good) good[i] = g[i];
        if (total) total[i] = t[i];
        double bf;
        if (f32_bins) {   /* ctr_feature.rs quantize_in_f32 branch */
            float den = (float)t[i] + 1.0f;
            float c = ((float)g[i] + (float)prior) / den;
            bf = (double)(((c + (float)shift) / (float)norm) * (float)border_count);
        } else {          /* calc_ctr_online_bin */
            bf = norm == 0.0 ? 0.0 : (v + shift) / norm * (double)border_count;
        }
        bin[i] = ctr_clamp_bin(bf, border_count);
    }
    free(g); free(t);
    return 0;
}
