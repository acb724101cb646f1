// rope.hpp - rotary embedding of one pair, shared by the standalone q/k RoPE
// kernel and the RoPE-on-read of the cache appends so both produce the same
// bits.
//
// Math (crates/mlx-cpp/turbo/fused_rope_append.cpp:140-171, the form MLX's own
// RoPE uses): pair p of the rotated prefix R of a head turns by
//   inv_freq = exp2(-(p / (R/2)) * log2(base)),  log2(base) formed on the host
//   theta    = (scale * position) * inv_freq
//   r1 = x1 cos(theta) - x2 sin(theta),  r2 = x1 sin(theta) + x2 cos(theta)
// in fp32 with the library cosf / sinf (the reference's CUDA port calls the
// same two, fused_rope_append.cpp:185-200). Pairs are (2p, 2p+1) when
// `traditional`, else (p, p + R/2); dims past R are copied unchanged.
#pragma once

#include "qw_common.hpp"

namespace qw {

// cos and sin of pair p's angle at `pos`.
__device__ __forceinline__ void rope_cs(int p, int rhalf, float log2_base, float scale, int pos,
                                        float& c, float& s) {
    const float dd = (float)p / (float)rhalf;
    const float inv_freq = exp2f(-dd * log2_base);
    const float theta = (scale * (float)pos) * inv_freq;
    c = cosf(theta);
    s = sinf(theta);
}

// The rotation of one pair by (c, s). The two products of each output are
// combined with one explicit fma so the rounding does not depend on how the
// compiler contracts a given call site.
__device__ __forceinline__ void rope_rot(float x1, float x2, float c, float s, float& r1,
                                         float& r2) {
    r1 = __builtin_fmaf(x1, c, -(x2 * s));
    r2 = __builtin_fmaf(x1, s, x2 * c);
    // The results are rounded to fp32 here, as the reference's float
    // variables are, before any conversion to fp16. Without this the compiler
    // may fold the last fma and the fp16 conversion into one mixed-precision
    // fma that rounds once, which differs from fp32-then-fp16 in about one
    // element of 10^4 and would make call sites disagree.
    asm volatile("" : "+v"(r1), "+v"(r2));
}

__device__ __forceinline__ void rope_pair(float x1, float x2, int p, int rhalf, float log2_base,
                                          float scale, int pos, float& r1, float& r2) {
    float c, s;
    rope_cs(p, rhalf, log2_base, scale, pos, c, s);
    rope_rot(x1, x2, c, s, r1, r2);
}

// Indices of the pair that holds dim d (d < rope_dims): p, the partner dim,
// and whether d is the first member.
__device__ __forceinline__ void rope_pair_of(int d, int rope_dims, int traditional, int& p,
                                             int& partner, bool& first) {
    const int rhalf = rope_dims >> 1;
    if (traditional) {
        p = d >> 1;
        partner = d ^ 1;
        first = (d & 1) == 0;
    } else {
        first = d < rhalf;
        p = first ? d : d - rhalf;
        partner = first ? d + rhalf : d - rhalf;
    }
}

// Rotated value of dim d of `row` (fp32, before rounding to the row's dtype).
__device__ __forceinline__ float rope_elem(const f16* __restrict__ row, int d, int rope_dims,
                                           int traditional, float log2_base, float scale,
                                           int pos) {
    if (d >= rope_dims) return (float)row[d];
    int p, partner;
    bool first;
    rope_pair_of(d, rope_dims, traditional, p, partner, first);
    const float x1 = (float)row[first ? d : partner];
    const float x2 = (float)row[first ? partner : d];
    float r1, r2;
    rope_pair(x1, x2, p, rope_dims >> 1, log2_base, scale, pos, r1, r2);
    return first ? r1 : r2;
}


// Launches that rotate a few query rows in their prologue (the decode and
// block kernels' RoPE launches) share one angle table: (cos, sin) of (row r,
// pair p) at [r * rope_dims / 2 + p], for position rs.position0 + r, formed by
// rope_cs as every RoPE path forms it. nthreads threads of the workgroup fill
// it; the caller's barrier follows.
template <class Src>
__device__ __forceinline__ void rope_fill_table(const Src& rs, int n_rows, float2* tab,
                                                int nthreads) {
    const int rh = rs.rope_dims >> 1;
    for (int i = threadIdx.x; i < n_rows * rh; i += nthreads) {
        const int r = i / rh, p = i - r * rh;
        float c, sn;
        rope_cs(p, rh, rs.log2_base, rs.scale, rs.position0 + r, c, sn);
        tab[i] = float2{c, sn};
    }
}

// Dims d0 .. d0 + N - 1 of query row r rotated as the RoPE kernels rotate
// them (rope_rot on the pair, the result rounded to fp16): x the dims, xp
// their half-split partners (unused for the adjacent pairing). N divides 8
// and d0 is a multiple of N, so with rope_dims a multiple of 16 the N dims sit
// on one side of rope_dims / 2 and of rope_dims.
template <int N, class Src>
__device__ __forceinline__ void rope_rotate_dims(const Src& rs, const float2* tab, int r, int d0,
                                                 const f16 (&x)[N], const f16 (&xp)[N],
                                                 f16 (&y)[N]) {
    const int R = rs.rope_dims, rh = R >> 1;
#pragma unroll
    for (int e = 0; e < N; e++) {
        const int d = d0 + e;
        if (d >= R) {
            y[e] = x[e];
            continue;
        }
        bool first;
        int pr;
        float partner;
        if (rs.traditional) {
            first = (d & 1) == 0;
            pr = d >> 1;
            partner = (float)x[e ^ 1];
        } else {
            first = d < rh;
            pr = first ? d : d - rh;
            partner = (float)xp[e];
        }
        const float2 cs = tab[r * rh + pr];
        const float xs = (float)x[e];
        float r1, r2;
        rope_rot(first ? xs : partner, first ? partner : xs, cs.x, cs.y, r1, r2);
        y[e] = (f16)(first ? r1 : r2);
    }
}

}  // namespace qw
