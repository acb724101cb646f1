// quant.hpp - MLX affine quantization arithmetic shared by the append kernel
// and the fused decode merge-append kernel.
//
// MLX `quantize` per group (restated in the oracle, qwo_affine_quantize):
// min/max of the group; the edge is the larger-magnitude extreme;
// scale = +-max((max - min) / n_bins, 1e-7) (sign: negative unless the edge is
// the minimum); q0 = rint(edge / scale); when q0 != 0 the scale is refit to
// edge / q0 and the bias is the edge. code = clamp(rint((w - bias) / scale)),
// computed with the fp32 scale and bias; fp16(scale), fp16(bias) are stored.
// IEEE division and round-half-even rint throughout (no reciprocal tricks).
#pragma once

#include "qw_common.hpp"

namespace qw {

struct AffineGroup {
    float scale, bias;  // fp32 values the codes are formed with
};

__device__ inline AffineGroup affine_group(float mn, float mx, int bits) {
    const float n_bins = (float)((1 << bits) - 1);
    const float eps = 1e-7f;
    const bool neg_side = fabsf(mn) > fabsf(mx);
    float scale = (mx - mn) / n_bins;
    scale = scale < eps ? eps : scale;
    scale = neg_side ? scale : -scale;
    const float edge = neg_side ? mn : mx;
    const float q0 = __builtin_rintf(edge / scale);
    float bias = 0.0f;
    if (q0 != 0.0f) {
        scale = edge / q0;
        bias = edge;
    }
    return AffineGroup{scale, bias};
}

__device__ inline float affine_code(float x, AffineGroup q, int bits) {
    const float n_bins = (float)((1 << bits) - 1);
    float c = __builtin_rintf((x - q.bias) / q.scale);
    return c < 0.0f ? 0.0f : (c > n_bins ? n_bins : c);
}

// MLX composite dequantize f16(f16(code * scale) + bias), as a float: the
// product (<= 8-bit code times an fp16) and the sum of two fp16 values are
// exact in fp32, so each fp16 cast is the single rounding MLX applies.
__device__ inline float affine_dequant(float code, f16 scale, f16 bias) {
    const f16 p = (f16)(code * (float)scale);
    return (float)(f16)((float)p + (float)bias);
}

// Clears *fast_flag when the stored fp16 scale is outside the exact range of
// the fused kernels' 2-op dequant (dequant.hpp).
__device__ inline void check_fast_scale(f16 scale, int bits, int* fast_flag) {
    const uint32_t a = __builtin_bit_cast(uint16_t, scale) & 0x7FFFu;
    const uint32_t lo = bits == 4 ? 0x1400u : 0u;
    if (a < lo || a >= 0x5400u) *fast_flag = 0;
}

}  // namespace qw
