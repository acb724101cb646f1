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
#pragma unroll
    for (int ls = 1; ls < 64; ls <<= 1) {
        const bool upper = (lane & ls) != 0;
#pragma unroll
        for (int j = 0; j < VPL; j++) {
            const float p = __shfl_xor(y[j], ls);
            y[j] = upper ? p - y[j] : y[j] + p;
        }
    }
}

// One row through a rotation, as the rotation kernel forms it:
// out = f16((H x (s_in . in)) * (1/sqrt(D)) * s_out) in fp32, the wave's lane
// holding coordinates lane * VPL .. + VPL - 1 of `in` (fp32 values).
template <int D>
__device__ __forceinline__ void t4_rotate_row(float (&y)[D / 64], int lane,
                                              const float* __restrict__ s_in,
                                              const float* __restrict__ s_out, f16 (&o)[D / 64]) {
    constexpr int VPL = D / 64;
#pragma unroll
    for (int j = 0; j < VPL; j++) y[j] *= s_in[lane * VPL + j];
    wht_wave<D>(y, lane);
#pragma unroll
    for (int j = 0; j < VPL; j++) o[j] = (f16)((y[j] * wht_scale(D)) * s_out[lane * VPL + j]);
}

}  // namespace qw
