// Shared device/host helpers of the gfx950 training path: the TFastRng64 generator,
// FastLogf, and the fixed-point scale record used by every exact reduction.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cbh {

constexpr int kMaxK = 16;          // largest approx dimension handled on device
constexpr int kMaxDepth = 8;       // 256 leaves
constexpr int kMaxLeaves = 1 << kMaxDepth;
constexpr uint64_t kLcgA = 6364136223846793005ULL;  // crates/cb-core/src/rng.rs:26

// ---------------------------------------------------------------------------------
// TFastRng64 (crates/cb-core/src/rng.rs:24-292): two 32-bit PCG-XSH-RR streams whose
// 64-bit LCG states x1/x2 advance as x = x*A + c; GenRand = (mix(x1) << 32) | mix(x2).
// ---------------------------------------------------------------------------------
struct Rng {
    uint64_t x1, c1, x2, c2;
};

__host__ __device__ inline uint32_t pcg_mix(uint64_t x) {
    uint32_t xs = (uint32_t)(((x >> 18) ^ x) >> 27);
    uint32_t rot = (uint32_t)(x >> 59);
    return (xs >> rot) | (xs << ((32u - rot) & 31u));
}

// Closed-form jump x_d = A^d x + c (A^d - 1)/(A - 1), square-and-multiply over the bits
// of delta from the top (rng.rs:45-66).
__host__ __device__ inline uint64_t lcg_advance(uint64_t seed, uint64_t addend, uint64_t delta) {
    uint64_t mask = 1;
    while (mask != (1ULL << 63) && (mask << 1) <= delta) mask <<= 1;
    uint64_t apow = 1, adiv = 0;
    while (mask != 0) {
        adiv = adiv * (apow + 1);
        apow = apow * apow;
        if (delta & mask) {
            adiv = adiv + apow;
            apow = apow * kLcgA;
        }
        mask >>= 1;
    }
    return seed * apow + addend * adiv;
}

__host__ __device__ inline uint32_t lcg_next(uint64_t& x, uint64_t c) {
    x = x * kLcgA + c;
    return pcg_mix(x);
}

__host__ __device__ inline Rng rng_new(uint64_t seed1, uint32_t seq1, uint64_t seed2, uint32_t seq2) {
    const uint32_t mask = (~0u) >> 1;
    uint32_t s2 = ((seq1 & mask) == (seq2 & mask)) ? ~seq2 : seq2;  // FixSeq
    Rng r;
    r.x1 = seed1;
    r.c1 = ((uint64_t)seq1 << 1) | 1;
    r.x2 = seed2;
    r.c2 = ((uint64_t)s2 << 1) | 1;
    return r;
}

// TFastRng64(ui64 seed): parameters drawn from a TReallyFastRng32 (addend 1).
__host__ __device__ inline Rng rng_from_seed(uint64_t seed) {
    uint64_t x = seed;
    uint64_t lo = lcg_next(x, 1), hi = lcg_next(x, 1);
    uint64_t seed1 = lo | (hi << 32);
    uint32_t seq1 = lcg_next(x, 1);
    lo = lcg_next(x, 1);
    hi = lcg_next(x, 1);
    uint64_t seed2 = lo | (hi << 32);
    uint32_t seq2 = lcg_next(x, 1);
    return rng_new(seed1, seq1, seed2, seq2);
}

__host__ __device__ inline uint64_t rng_gen(Rng& r) {
    uint64_t a = lcg_next(r.x1, r.c1);
    uint64_t b = lcg_next(r.x2, r.c2);
    return (a << 32) | b;
}

__host__ __device__ inline void rng_advance(Rng& r, uint64_t d) {
    r.x1 = lcg_advance(r.x1, r.c1, d);
    r.x2 = lcg_advance(r.x2, r.c2, d);
}

__host__ __device__ inline double rng_real1(Rng& r) {
    return (double)(rng_gen(r) >> 11) * (1.0 / 9007199254740991.0);
}

// Uniform draw in [0, bound) by rejection (rng.rs:268-280).
__host__ __device__ inline uint64_t rng_uniform(Rng& r, uint64_t bound) {
    if (bound == 0) return 0;
    const uint64_t randmax = ~0ull - (~0ull % bound);
    for (;;) {
        const uint64_t v = rng_gen(r);
        if (v < randmax) return v % bound;
    }
}

// Affine jump tables of the LCG: fine[j] = (A^j, (A^j-1)/(A-1)) for j < 1024 and
// coarse[q] = the same for j = 1024 q, q < n_coarse.
inline void make_jump_tables(uint64_t n_coarse, uint64_t* fine_a, uint64_t* fine_d,
                             uint64_t* coarse_a, uint64_t* coarse_d) {
    uint64_t a = 1, d = 0;
    for (int j = 0; j < 1024; ++j) {
        fine_a[j] = a;
        fine_d[j] = d;
        d = d + a;
        a = a * kLcgA;
    }
    const uint64_t a1024 = a, d1024 = d;
    uint64_t ca = 1, cd = 0;
    for (uint64_t q = 0; q < n_coarse; ++q) {
        coarse_a[q] = ca;
        coarse_d[q] = cd;
        cd = cd * a1024 + d1024;
        ca = ca * a1024;
    }
}

// FastLogf (crates/cb-train/src/fast_approx.rs:154-177).  Every operation is a single
// IEEE f32 op in the reference order; the library is compiled with -ffp-contract=off so
// no multiply-add is fused.
__host__ __device__ inline float fast_logf(float value) {
    uint32_t vx = __builtin_bit_cast(uint32_t, value);
    float mx = __builtin_bit_cast(float, (vx & 0x007FFFFFu) | 0x3f000000u);
    float y = (float)vx;
    y *= 1.1920928955078125e-7f;
    float l2 = y - 124.22551499f - 1.498030302f * mx - 1.72587999f / (0.3520887068f + mx);
    return 0.69314718f * l2;
}

// ---------------------------------------------------------------------------------
// Fixed-point scales.  Every per-row statistic v is accumulated as the integer
// round(v * 2^S) in int64; sums of integers are exact and order-free, so histogram,
// prefix and sibling (parent - child) values are reproducible bit for bit and equal to
// the correctly rounded sum of the quantized rows.  S is chosen per tree from a bound on
// sum(|v|) so that no partial sum can overflow.
// ---------------------------------------------------------------------------------
enum ScaleSlot { kScoreDer = 0, kScoreW = 1, kLeafDer = 2, kLeafW = 3, kNumScales = 4 };

struct Scales {
    double mul[kNumScales];   // 2^S
    double inv[kNumScales];   // 2^-S
    int32_t shift[kNumScales];
    int32_t pk_k;             // count-packed fill: bits of the weight field of a packed cell
    int32_t pk_swap;          // count-packed fill: blocks of rows between two swaps
};

// Per-tree bound accumulators: sum of ceil(|v| * 2^kBoundShift) per slot (integers, so
// the device reduction is deterministic) and the count of rows with nonzero score weight.
constexpr int kBoundShift = 10;
struct Bounds {
    unsigned long long sum_abs[kNumScales];
    unsigned long long sampled_rows;
    unsigned long long device_err;   // nonzero: a kernel of the tree gave up a bounded wait (cleared per tree)
    unsigned long long pad[2];
};

__device__ __forceinline__ long long to_fixed(double v, double mul) {
    return __double2ll_rn(v * mul);
}

}  // namespace cbh
