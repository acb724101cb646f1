// dequant.hpp - in-register affine dequantization for the MFMA kernels.
//
// Every fused kernel must reproduce MLX's composite dequantize bit for bit,
//   v = f16(f16(code * scale) + bias),
// because the fused attention rounds its scores to fp16 the way MLX's SDPA
// does and a one-ulp change in K would move those roundings.
//
// Codes become fp16 through the magic-number trick: a 4-bit field masked into
// bits 0..3 of a half and OR-ed with 0x6400 reads as 1024 + code (the field
// at bits 4..7 reads as 1024 + 16*code); an 8-bit field placed with v_perm
// reads as 1024 + code.
//   FAST: y = fma(x, s, -1024*s) + bias. The fma forms (1024 + code)*s -
//         1024*s = code*s exactly and rounds it once; the add rounds again.
//         For the x16 fields s is scale/16 and the addend -64*scale.
//         Exact when -1024*scale is a finite fp16 (|scale| < 64) and, for the
//         x16 fields, scale/16 is a normal fp16 (|scale| >= 2^-10).
//   SLOW: c = x - 1024 (exact; x16 fields also * 1/16, exact), then a
//         separately rounded multiply and add. Used for a cache whose
//         scales miss the FAST range, and for Int8 caches, whose codes are
//         stored biased by 128: c = x - 1152 is the signed code, bias 0.
#pragma once

#include "qw_common.hpp"

namespace qw {

constexpr uint32_t kMagic = 0x64006400u;

// |scale| bits of one fp16 (low 16 bits of `h`) inside [lo, hi).
__device__ inline bool scale_in_range(uint32_t h, uint32_t lo, uint32_t hi) {
    const uint32_t a = h & 0x7FFFu;
    return a >= lo && a < hi;
}
// Both halves of a (s, s') pair.
__device__ inline bool scales_in_range(uint32_t pair, uint32_t lo, uint32_t hi) {
    return scale_in_range(pair, lo, hi) && scale_in_range(pair >> 16, lo, hi);
}
constexpr uint32_t kFast4Lo = 0x1400u;  // 2^-10
constexpr uint32_t kFast8Lo = 0x0000u;
constexpr uint32_t kFastHi = 0x5400u;   // 64

#pragma clang fp contract(off)

// ADDB = false returns f16(code * scale) only: the fused attention adds the
// bias term of a group separately (scale and bias are per group, so
// sum_d x_d (c_d s + b) = sum_d x_d f16(c_d s) + b sum_d x_d).
template <bool FAST, bool X16, bool ADDB = true>
__device__ __forceinline__ half2v deq_pair(uint32_t magic_bits, half2v s, half2v m, half2v b,
                                           half2v off) {
    const half2v x = h2(magic_bits);
    half2v p;
    if constexpr (FAST) {
        p = __builtin_elementwise_fma(x, s, m);
    } else {
        half2v c = x - off;
        if constexpr (X16) c = c * (half2v){(f16)0.0625f, (f16)0.0625f};
        p = c * s;
    }
    if constexpr (ADDB) p = p + b;
    return p;
}

// Constants of the four pairs a word produces. FAST: s[1], s[3] are scale/16
// (the x16 fields of 4-bit words), m[i] = -1024 * s[i]. SLOW: s[i] plain
// scales, m unused, off the magic offset (1024, or 1152 for Int8 codes).
struct PairConsts {
    half2v s[4], m[4], b[4];
    half2v off;
};

// Builds the constants from the plain (scale, bias) pairs of the four pairs.
template <bool FAST, int BITS>
__device__ __forceinline__ PairConsts make_consts(half2v s0, half2v s1, half2v s2, half2v s3,
                                                  half2v b0, half2v b1, half2v b2, half2v b3,
                                                  uint32_t off2 = kMagic) {
    PairConsts c;
    c.off = h2(off2);
    c.s[0] = s0;
    c.s[1] = s1;
    c.s[2] = s2;
    c.s[3] = s3;
    c.b[0] = b0;
    c.b[1] = b1;
    c.b[2] = b2;
    c.b[3] = b3;
#pragma unroll
    for (int i = 0; i < 4; i++) c.m[i] = half2v{};
    if constexpr (FAST) {
        if constexpr (BITS == 4) {
            const half2v k16 = {(f16)0.0625f, (f16)0.0625f};
            c.s[1] = c.s[1] * k16;
            c.s[3] = c.s[3] * k16;
        }
        // -1024 * (the multiplier of the pair): -1024*s, or -64*s for x16 fields.
        const half2v k1024 = {(f16)-1024.0f, (f16)-1024.0f};
#pragma unroll
        for (int i = 0; i < 4; i++) c.m[i] = c.s[i] * k1024;
    }
    return c;
}

// 4-bit word -> pairs (nibbles 0,4), (1,5), (2,6), (3,7). `magic` is
// kMagic held in a VGPR (vconst) so each field costs one v_and_or_b32.
template <bool FAST, bool ADDB = true>
__device__ __forceinline__ half8 deq4(uint32_t w, const PairConsts& c, uint32_t magic) {
    const uint32_t w8 = w >> 8;
    const half2v y0 = deq_pair<FAST, false, ADDB>((w & 0x000F000Fu) | magic, c.s[0], c.m[0], c.b[0], c.off);
    const half2v y1 = deq_pair<FAST, true, ADDB>((w & 0x00F000F0u) | magic, c.s[1], c.m[1], c.b[1], c.off);
    const half2v y2 = deq_pair<FAST, false, ADDB>((w8 & 0x000F000Fu) | magic, c.s[2], c.m[2], c.b[2], c.off);
    const half2v y3 = deq_pair<FAST, true, ADDB>((w8 & 0x00F000F0u) | magic, c.s[3], c.m[3], c.b[3], c.off);
    return half8{y0.x, y0.y, y1.x, y1.y, y2.x, y2.y, y3.x, y3.y};
}

// Two 8-bit words -> pairs (bytes 0,1), (2,3) of w0, then of w1.
template <bool FAST, bool ADDB = true>
__device__ __forceinline__ half8 deq8(uint32_t w0, uint32_t w1, const PairConsts& c) {
    const half2v y0 = deq_pair<FAST, false, ADDB>(__builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u),
                                                  c.s[0], c.m[0], c.b[0], c.off);
    const half2v y1 = deq_pair<FAST, false, ADDB>(__builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u),
                                                  c.s[1], c.m[1], c.b[1], c.off);
    const half2v y2 = deq_pair<FAST, false, ADDB>(__builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u),
                                                  c.s[2], c.m[2], c.b[2], c.off);
    const half2v y3 = deq_pair<FAST, false, ADDB>(__builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u),
                                                  c.s[3], c.m[3], c.b[3], c.off);
    return half8{y0.x, y0.y, y1.x, y1.y, y2.x, y2.y, y3.x, y3.y};
}

#pragma clang fp contract(on)

}  // namespace qw
