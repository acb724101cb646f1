// turbo4_device.hpp - device pieces of the Turbo4 mode shared by its own
// kernels (turbo4.hip) and the decode kernel's Turbo4 read (attend_decode.hip):
// the layout of the per-cache device tables and the rotation.
#pragma once

#include "qw_common.hpp"

namespace qw {

// Offsets (floats) into a Turbo4 cache's device tables: the V signs s1, s2,
// the K signs s1, s2 (D each), the 16 centroids and the 15 boundaries.
template <int D>
struct T4Tab {
    static constexpr int v_s1 = 0, v_s2 = D, k_s1 = 2 * D, k_s2 = 3 * D;
    static constexpr int cb = 4 * D, bnd = 4 * D + 16;
    static constexpr int size = 4 * D + 32;
};

// The transform's scale as MLX forms it: 1 / sqrt(n) in double, cast to fp32.
__host__ __device__ constexpr float wht_scale(int D) {
    return D == 256 ? 0.0625f : (D == 128 ? 0.08838834764831845f : 0.0f);
}

// Sum over the wave by an xor butterfly (offsets 32, 16, ..., 1): the order
// every Turbo4 norm is formed in, so all kernels store the same rescales.
__device__ __forceinline__ float t4_wave_sum(float x) {
    const int lane = (int)__lane_id();
    x += lane_xor<32>(x, lane);
    x += lane_xor<16>(x, lane);
    x += lane_xor<8>(x, lane);
    x += lane_xor<4>(x, lane);
    x += lane_xor<2>(x, lane);
    x += lane_xor<1>(x, lane);
    return x;
}

// In-place fp32 Walsh-Hadamard transform of the wave's row (lane holds
// coordinates lane * VPL .. lane * VPL + VPL - 1), unscaled: log2(VPL)
// butterfly stages inside the lane, then six across lanes.
template <int D>
__device__ __forceinline__ void wht_wave(float (&y)[D / 64], int lane) {
    constexpr int VPL = D / 64;
#pragma unroll
    for (int s = 1; s < VPL; s <<= 1) {
#pragma unroll
        for (int j = 0; j < VPL; j++) {
            if ((j & s) == 0) {
                const float a = y[j], b = y[j + s];
                y[j] = a + b;
                y[j + s] = a - b;
            }
        }
    }
    auto stage = [&](auto ls_c) {
        constexpr int LS = decltype(ls_c)::value;
        const bool upper = (lane & LS) != 0;
#pragma unroll
        for (int j = 0; j < VPL; j++) {
            const float p = lane_xor<LS>(y[j], lane);
            y[j] = upper ? p - y[j] : y[j] + p;
        }
    };
    stage(std::integral_constant<int, 1>{});
    stage(std::integral_constant<int, 2>{});
    stage(std::integral_constant<int, 4>{});
    stage(std::integral_constant<int, 8>{});
    stage(std::integral_constant<int, 16>{});
    stage(std::integral_constant<int, 32>{});
}

// f16 of an fp32 product, rounded first to fp32 (the expansion's
// f16(centroid * rescale)); the register pin keeps the compiler from fusing
// the multiply and the conversion into one singly rounded mixed-precision op.
__device__ __forceinline__ f16 t4_f16_product(float c, float r) {
    float p = c * r;
    asm("" : "+v"(p));
    return (f16)p;
}

// One row through a rotation, as the rotation kernel forms it:
// out = f16((H x (s_in . in)) * (1/sqrt(D)) * s_out) in fp32, the wave's lane
// holding coordinates lane * VPL .. + VPL - 1 of `in` (fp32 values) and of
// the signs si, so.
template <int D>
__device__ __forceinline__ void t4_rotate_row(float (&y)[D / 64], int lane,
                                              const float (&si)[D / 64], const float (&so)[D / 64],
                                              f16 (&o)[D / 64]) {
    constexpr int VPL = D / 64;
#pragma unroll
    for (int j = 0; j < VPL; j++) y[j] *= si[j];
    wht_wave<D>(y, lane);
#pragma unroll
    for (int j = 0; j < VPL; j++) o[j] = (f16)((y[j] * wht_scale(D)) * so[j]);
}

// The fused verify pass's q: out = f16(f32(f32(s_out . (H / sqrt(D)) . s_in .
// in) * post)) (post = scale * log2 e), as the scaled rotation kernel forms it.
template <int D>
__device__ __forceinline__ void t4_rotate_row_scaled(float (&y)[D / 64], int lane,
                                                     const float (&si)[D / 64],
                                                     const float (&so)[D / 64], float post,
                                                     f16 (&o)[D / 64]) {
    constexpr int VPL = D / 64;
#pragma unroll
    for (int j = 0; j < VPL; j++) y[j] *= si[j];
    wht_wave<D>(y, lane);
#pragma unroll
    for (int j = 0; j < VPL; j++) {
        float v = (y[j] * wht_scale(D)) * so[j];
        asm("" : "+v"(v));
        o[j] = t4_f16_product(v, post);
    }
}

// The lane's coordinates of a sign vector (D floats).
template <int D>
__device__ __forceinline__ void t4_lane_signs(const float* __restrict__ s, int lane,
                                              float (&r)[D / 64]) {
#pragma unroll
    for (int j = 0; j < D / 64; j++) r[j] = s[lane * (D / 64) + j];
}

template <int D>
__device__ __forceinline__ void t4_rotate_row(float (&y)[D / 64], int lane,
                                              const float* __restrict__ s_in,
                                              const float* __restrict__ s_out, f16 (&o)[D / 64]) {
    float si[D / 64], so[D / 64];
    t4_lane_signs<D>(s_in, lane, si);
    t4_lane_signs<D>(s_out, lane, so);
    t4_rotate_row<D>(y, lane, si, so, o);
}

}  // namespace qw
