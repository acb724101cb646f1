// turbo4_codec.hpp - host-side tables of the Turbo4 (PolarQuant) KV codec:
// the Lloyd-Max codebook and the LCG sign vectors. Plain C++ (no device code)
// so the tables can be built and checked without a GPU.
//
// Reference behaviour followed (cr0sh/qw):
//   codebook: crates/mlxcel-core/src/cache/turbo/codebook.rs:208-240 (b = 1,
//     2 closed forms; b >= 3 Lloyd-Max on N(0, 1/d), 100 iterations from
//     uniform-quantile boundaries), :289-361 (conditional expectations);
//   boundaries: codebook.rs:84-90 (midpoints, in fp32);
//   signs: crates/mlxcel-core/src/cache/turbo/quant.rs:119-139 (32-bit LCG,
//     bit 31, 0 -> -1), :188-236 (V seeds seed / seed + 0x9E3779B9, K seeds
//     the same from seed + 0x4B5F5345).
#pragma once

#include <math.h>
#include <stdint.h>

#include <vector>

namespace qw {
namespace turbo4 {

constexpr uint32_t kDefaultSeed = 0x7B470404u;   // cache.rs:324 TURBO_DEFAULT_SEED
constexpr uint32_t kSubSeed = 0x9E3779B9u;       // second sign vector of a pair
constexpr uint32_t kKSeedOffset = 0x4B5F5345u;   // quant.rs:101 K_SEED_OFFSET

// Standard normal helpers in double precision.
inline double norm_pdf(double x) { return exp(-0.5 * x * x) / sqrt(2.0 * M_PI); }
inline double norm_cdf(double x) { return 0.5 * erfc(-x / sqrt(2.0)); }
inline double norm_sf(double x) { return 0.5 * erfc(x / sqrt(2.0)); }

// Inverse of norm_cdf by bisection to the limit of double precision (the
// initial boundaries only seed the iteration, which then converges).
inline double norm_ppf(double p) {
    double lo = -40.0, hi = 40.0;
    for (int i = 0; i < 200; i++) {
        const double mid = 0.5 * (lo + hi);
        if (mid == lo || mid == hi) break;
        if (norm_cdf(mid) < p)
            lo = mid;
        else
            hi = mid;
    }
    return 0.5 * (lo + hi);
}

// E[X | a < X < b] for X ~ N(0, sigma^2); a = -inf / b = +inf for the tails.
inline double cond_mean(double sigma, double a, double b) {
    const double as = isfinite(a) ? a / sigma : a;
    const double bs = isfinite(b) ? b / sigma : b;
    double prob;
    if (!isfinite(as))
        prob = norm_cdf(bs);
    else if (!isfinite(bs))
        prob = norm_sf(as);
    else
        prob = norm_cdf(bs) - norm_cdf(as);
    if (prob < 1e-15) {
        // a region of no mass: the reference's asymptotic stand-ins
        if (isfinite(a) && !isfinite(b)) return a + sigma;
        if (!isfinite(a) && isfinite(b)) return b - sigma;
        if (isfinite(a) && isfinite(b)) return 0.5 * (a + b);
        return 0.0;
    }
    const double pa = isfinite(as) ? norm_pdf(as) : 0.0;
    const double pb = isfinite(bs) ? norm_pdf(bs) : 0.0;
    return sigma * (pa - pb) / prob;
}

// Sorted centroids for (bits, head_dim), bits in [1, 8].
inline std::vector<float> centroids(int bits, int head_dim) {
    const double d = (double)head_dim;
    if (bits == 1) {
        const double c = sqrt(2.0 / (M_PI * d));
        return {(float)-c, (float)c};
    }
    if (bits == 2) {
        const double s = 1.0 / sqrt(d);
        return {(float)(-1.51 * s), (float)(-0.453 * s), (float)(0.453 * s), (float)(1.51 * s)};
    }
    const int n = 1 << bits;
    const double sigma = 1.0 / sqrt(d);
    std::vector<double> bnd(n - 1), c(n);
    for (int i = 1; i < n; i++) bnd[i - 1] = norm_ppf((double)i / n) * sigma;
    auto update = [&]() {
        c[0] = cond_mean(sigma, -INFINITY, bnd[0]);
        for (int i = 1; i < n - 1; i++) c[i] = cond_mean(sigma, bnd[i - 1], bnd[i]);
        c[n - 1] = cond_mean(sigma, bnd[n - 2], INFINITY);
    };
    update();
    for (int it = 0; it < 100; it++) {
        for (int i = 0; i + 1 < n; i++) bnd[i] = (c[i] + c[i + 1]) * 0.5;
        update();
    }
    std::vector<float> out(n);
    for (int i = 0; i < n; i++) out[i] = (float)c[i];
    return out;
}

// Midpoint boundaries, formed in fp32 from the fp32 centroids.
inline std::vector<float> boundaries(const std::vector<float>& c) {
    std::vector<float> b;
    for (size_t i = 0; i + 1 < c.size(); i++) b.push_back((c[i] + c[i + 1]) * 0.5f);
    return b;
}

// +-1 sign vector: state <- 1664525 state + 1013904223 (mod 2^32) per entry
// (a zero seed starts from 0xDEADBEEF), sign + when bit 31 of the new state
// is set.
inline std::vector<float> signs(int len, uint32_t seed) {
    uint32_t s = seed == 0 ? 0xDEADBEEFu : seed;
    std::vector<float> out(len);
    for (int i = 0; i < len; i++) {
        s = s * 1664525u + 1013904223u;
        out[i] = (s >> 31) ? 1.0f : -1.0f;
    }
    return out;
}

}  // namespace turbo4
}  // namespace qw
