// append.hpp - quantize-on-append of new K/V rows into an affine or Int8
// cache, shared by the append kernel and the block kernel's append
// workgroups (a verify block that appends its rows in the attention launch).
#pragma once

#include "kv_cache.hpp"
#include "quant.hpp"
#include "rope.hpp"
#include "turbo4_device.hpp"

namespace qw {

// ------------------------------------------------ quantize-on-append (A.1)
//
// The work of one (KV head, 8-token V block touched by the append): each wave
// of the workgroup quantizes whole rows (one token of K or V): a lane
// holds D/64 consecutive dims, a 64-dim group is 64/(D/64) lanes and its
// min/max are wave shuffles. The group math is MLX's, in fp32 with IEEE
// division and rint (ties to even):
//   scale = max((max - min) / n_bins, 1e-7), negated unless |min| > |max|
//   edge = larger-magnitude extreme; q0 = rint(edge / scale)
//   if q0 != 0: scale = edge / q0, bias = edge, else bias = 0
//   code = clamp(rint((w - bias) / scale), 0, n_bins)
// Codes go through LDS so the V block words (8 keys per dim) are assembled
// by one thread each: no two threads write the same word.

// Int8 (cache.rs:270-305 quantize_per_token, MLX fp16 ops): absmax over the
// row; scale = f16(absmax / 127), 1 where that is 0; code = clip(round(
// f16(x / scale)), -128, 127), stored as code + 128 with (scale, 0) in every
// group slot. fp16 division rounded once from the fp32 quotient equals the
// correctly rounded fp16 division (24 >= 2*11 + 2 bits).
template <int D>
__device__ inline void quantize_row_int8(const float* x, uint8_t* lds_codes, half2v* sb_out) {
    constexpr int VPL = D / 64;
    const int lane = threadIdx.x & 63;
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; i++) am = fmaxf(am, fabsf(x[i]));
    am = wave_reduce(am, OpMax());
    f16 sc = (f16)(am / 127.0f);
    if ((float)sc == 0.0f) sc = (f16)1.0f;
    const float s = (float)sc;
#pragma unroll
    for (int i = 0; i < VPL; i++) {
        const float c = __builtin_rintf((float)(f16)(x[i] / s));
        lds_codes[lane * VPL + i] = (uint8_t)((int)fminf(fmaxf(c, -128.0f), 127.0f) + 128);
    }
    if (lane < D / kGroup) {
        half2v sb;
        sb.x = sc;
        sb.y = (f16)0.0f;
        sb_out[lane] = sb;
    }
}

// The row is read from `src`; with `rope` (K of a fused RoPE-append) each
// element is rotated first and rounded to fp16, the value the fp16 rotation
// hands to the cache's quantize-on-append.
template <int D>
__device__ inline void quantize_row(const f16* __restrict__ src, int bits, bool int8,
                                    uint8_t* lds_codes,
                                    half2v* sb_out /* [D/64] (scale, bias) */, int* fast_flag,
                                    const RowSrc* rope = nullptr, int pos = 0) {
    constexpr int VPL = D / 64;         // values per lane
    constexpr int LPG = kGroup / VPL;   // lanes per group
    const int lane = threadIdx.x & 63;
    float x[VPL];
    if (rope && rope->rope_dims > 0) {
#pragma unroll
        for (int i = 0; i < VPL; i++) x[i] = (float)(f16)rope_elem(src, lane * VPL + i, rope->rope_dims,
                                                  rope->traditional, rope->log2_base,
                                                  rope->scale, pos);
    } else {
#pragma unroll
        for (int i = 0; i < VPL; i++) x[i] = (float)src[lane * VPL + i];
    }
    if (int8) {
        quantize_row_int8<D>(x, lds_codes, sb_out);
        return;
    }
    float mx = x[0], mn = x[0];
#pragma unroll
    for (int i = 1; i < VPL; i++) {
        mx = mx < x[i] ? x[i] : mx;
        mn = x[i] < mn ? x[i] : mn;
    }
#pragma unroll
    for (int off = 1; off < LPG; off <<= 1) {
        const float omx = __shfl_xor(mx, off);
        const float omn = __shfl_xor(mn, off);
        mx = mx < omx ? omx : mx;
        mn = omn < mn ? omn : mn;
    }
    const AffineGroup q = affine_group(mn, mx, bits);
#pragma unroll
    for (int i = 0; i < VPL; i++) lds_codes[lane * VPL + i] = (uint8_t)affine_code(x[i], q, bits);
    if ((lane % LPG) == 0) {
        half2v sb;
        sb.x = (f16)q.scale;
        sb.y = (f16)q.bias;
        sb_out[lane / LPG] = sb;
        check_fast_scale(sb.x, bits, fast_flag);
    }
}

// LDS of one 8-token block's append: the codes and (scale, bias) pairs of its
// K and V rows.
template <int D>
struct AppendScratch {
    uint8_t kc[8][D];
    uint8_t vc[8][D];
    half2v ksb[8][D / kGroup];
    half2v vsb[8][D / kGroup];
};

// The append of the new tokens that fall in 8-token V block `blk` of head h
// (tokens t_old .. t_old + n_tokens - 1 of the cache), by threads tid of nthr
// (nthr >= D, a multiple of 64; every thread calls it: it holds a barrier).
template <int D>
__device__ inline void append_block(const RowSrc& rs, int n_tokens, int t_old, int bits, bool int8,
                                    int cap, uint32_t* __restrict__ k_codes,
                                    uint32_t* __restrict__ k_params, uint32_t* __restrict__ v_codes,
                                    f16* __restrict__ v_params, int* __restrict__ fast_flag, int blk,
                                    int h, int tid, int nthr, AppendScratch<D>& sc) {
    constexpr int NG = D / kGroup;
    const int wave = tid >> 6, nwaves = nthr >> 6;
    const int t_end = t_old + n_tokens;
    // Codes of earlier tokens in a partly filled block are kept: fetch those
    // words now so their latency overlaps the quantization.
    const int bw = D * bits / 4;  // words per V block (8 keys x D dims)
    uint32_t* vb = v_codes + ((int64_t)h * (cap / 8) + blk) * bw;
    const bool keep_old = blk * 8 < t_old;
    uint32_t old0 = 0, old1 = 0;
    const int d_own = tid;
    const int p_own = d_own < D ? v_phys_dim(d_own, D, bits) : 0;
    if (keep_old && d_own < D) {
        if (bits == 4) {
            old0 = vb[p_own];
        } else {
            old0 = vb[2 * p_own];
            old1 = vb[2 * p_own + 1];
        }
    }
    for (int k = wave; k < 8; k += nwaves) {
        const int t = blk * 8 + k;
        if (t < t_old || t >= t_end) continue;
        const int64_t src = (int64_t)(t - t_old) * rs.row_stride + (int64_t)h * rs.head_stride;
        quantize_row<D>(rs.k + src, bits, int8, sc.kc[k], sc.ksb[k], fast_flag, &rs,
                        rs.position0 + (t - t_old));
        quantize_row<D>(rs.v + src, bits, int8, sc.vc[k], sc.vsb[k], fast_flag);
    }
    __syncthreads();
    // K: row-major MLX packing, words of 32/bits codes LSB-first.
    const int epw = 32 / bits;
    const int nw = D / epw;
    for (int i = tid; i < 8 * nw; i += nthr) {
        const int k = i / nw, w = i % nw;
        const int t = blk * 8 + k;
        if (t < t_old || t >= t_end) continue;
        uint32_t word = 0;
        for (int e = 0; e < epw; e++) word |= (uint32_t)sc.kc[k][w * epw + e] << (e * bits);
        k_codes[((int64_t)h * cap + t) * nw + w] = word;
    }
    for (int i = tid; i < 8 * NG; i += nthr) {
        const int k = i / NG, g = i % NG;
        const int t = blk * 8 + k;
        if (t < t_old || t >= t_end) continue;
        k_params[((int64_t)h * cap + t) * NG + k_param_slot(g, NG)] =
            __builtin_bit_cast(uint32_t, sc.ksb[k][g]);
        f16* vp = v_params + (((int64_t)h * (cap / 8) + blk) * NG + g) * 16;
        vp[k] = sc.vsb[k][g].x;
        vp[8 + k] = sc.vsb[k][g].y;
    }
    // V: one thread per dim assembles the block word(s), keeping the codes of
    // slots before this append (earlier tokens of a partly filled block).
    if (d_own < D) {
        const int d = d_own, p = p_own;
        if (bits == 4) {
            uint32_t word = old0;
            for (int k = 0; k < 8; k++) {
                const int t = blk * 8 + k;
                if (t < t_old || t >= t_end) continue;
                const int sh = 4 * v4_nibble_pos(k);
                word = (word & ~(0xFu << sh)) | ((uint32_t)sc.vc[k][d] << sh);
            }
            vb[p] = word;
        } else {
            uint32_t w0 = old0, w1 = old1;
            for (int k = 0; k < 8; k++) {
                const int t = blk * 8 + k;
                if (t < t_old || t >= t_end) continue;
                const int sh = 8 * (k & 3);
                if (k < 4)
                    w0 = (w0 & ~(0xFFu << sh)) | ((uint32_t)sc.vc[k][d] << sh);
                else
                    w1 = (w1 & ~(0xFFu << sh)) | ((uint32_t)sc.vc[k][d] << sh);
            }
            vb[2 * p] = w0;
            vb[2 * p + 1] = w1;
        }
    }
}

// Turbo4 quantize-on-append of one row by one wave (lane holds D/64
// consecutive coordinates): row i of head h, K (is_k: K signs, RoPE as RowSrc
// asks) or V (V signs), stored as cache row t_old + i. The steps: fp32 L2 norm
// (an all-zero row divides by 1); signs2 . H . signs1 of the unit row (H the
// Walsh-Hadamard transform scaled 1/sqrt(D)); the index = the number of the
// 15 boundaries strictly below the value; rescale = f16(norm / max(|centroid
// vector|, 1e-10)); nibbles packed low = even coordinate; side word K
// (rescale, 0), V (f16 norm, rescale). cb: the 16 centroids. expand (if not
// null, D values): the row's stored values in the rotated basis, f16(centroid
// * rescale), as the attention kernels form them from the cache.
template <int D>
__device__ inline void turbo4_append_row(const RowSrc& rs, int i, int h, bool is_k, int lane,
                                         int t_old, int cap, const float* __restrict__ tab,
                                         const float* cb, uint8_t* __restrict__ k_packed,
                                         uint32_t* __restrict__ k_side,
                                         uint8_t* __restrict__ v_packed,
                                         uint32_t* __restrict__ v_side, f16* expand = nullptr) {
    constexpr int VPL = D / 64;
    using TT = T4Tab<D>;
    const int64_t src = (int64_t)i * rs.row_stride + (int64_t)h * rs.head_stride;
    const f16* row = (is_k ? rs.k : rs.v) + src;
    float x[VPL];
    if (is_k && rs.rope_dims > 0) {
#pragma unroll
        for (int j = 0; j < VPL; j++)
            x[j] = (float)(f16)rope_elem(row, lane * VPL + j, rs.rope_dims, rs.traditional,
                                         rs.log2_base, rs.scale, rs.position0 + i);
    } else {
#pragma unroll
        for (int j = 0; j < VPL; j++) x[j] = (float)row[lane * VPL + j];
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; j++) ss = __builtin_fmaf(x[j], x[j], ss);
    const float norm = sqrtf(t4_wave_sum(ss));
    const float safe = norm > 0.0f ? norm : 1.0f;
    const float* s1 = tab + (is_k ? TT::k_s1 : TT::v_s1);
    const float* s2 = tab + (is_k ? TT::k_s2 : TT::v_s2);
    float y[VPL];
#pragma unroll
    for (int j = 0; j < VPL; j++) y[j] = (x[j] / safe) * s1[lane * VPL + j];
    wht_wave<D>(y, lane);
    uint32_t idx[VPL];
    float csq = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; j++) {
        const float v = (y[j] * wht_scale(D)) * s2[lane * VPL + j];
        uint32_t n = 0;
#pragma unroll
        for (int b = 0; b < 15; b++) n += v > tab[TT::bnd + b] ? 1u : 0u;
        idx[j] = n;
        const float c = cb[n];
        csq = __builtin_fmaf(c, c, csq);
    }
    const float rn = sqrtf(t4_wave_sum(csq));
    const f16 rescale = (f16)(norm / fmaxf(rn, 1e-10f));
    if (expand) {
#pragma unroll
        for (int j = 0; j < VPL; j++) expand[lane * VPL + j] = t4_f16_product(cb[idx[j]], (float)rescale);
    }
    const int t = t_old + i;
    uint8_t* prow = (is_k ? k_packed : v_packed) + ((int64_t)h * cap + t) * (D / 2);
    if constexpr (VPL == 4) {
        const uint32_t b0 = idx[0] | (idx[1] << 4), b1 = idx[2] | (idx[3] << 4);
        *(uint16_t*)(prow + 2 * lane) = (uint16_t)(b0 | (b1 << 8));
    } else {
        prow[lane] = (uint8_t)(idx[0] | (idx[1] << 4));
    }
    if (lane == 0) {
        half2v sv;
        if (is_k) {
            sv.x = rescale;
            sv.y = (f16)0.0f;
            k_side[(int64_t)h * cap + t] = __builtin_bit_cast(uint32_t, sv);
        } else {
            sv.x = (f16)norm;
            sv.y = rescale;
            v_side[(int64_t)h * cap + t] = __builtin_bit_cast(uint32_t, sv);
        }
    }
}

}  // namespace qw
