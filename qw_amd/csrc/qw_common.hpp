// qw_common.hpp - shared device types, helpers and host error plumbing for
// the gfx950 full-attention kernels (libqwattn.so).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "qwattn.h"

namespace qw {

typedef _Float16 f16;
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kGroup = 64;  // affine group size along head_dim
constexpr int kWave = 64;

// Byte layout of one cache mode, shared by every kernel that touches it.
//   K plane, affine:  codes [hkv][cap][D*bits/32] u32, row-major and packed
//                     LSB-first exactly as MLX `quantize` packs a row;
//                     params [hkv][cap][D/64] u32 = half2(scale, bias).
//   V plane, affine:  8-key blocks, codes [hkv][cap/8][D*bits/4 bytes]:
//                     for each dim the 8 keys' codes sit in one u32 (4-bit)
//                     or two u32 (8-bit), so a lane's 128-bit load is
//                     directly the k-contiguous B operand of the P.V MFMA.
//                     Dims are stored in "lane order" (see v_phys_dim) so
//                     the 16 lanes of an MFMA column group read 256
//                     contiguous bytes per load.
//                     params [hkv][cap/8][D/64][16] f16: s0..s7, b0..b7.
//   fp16 mode:        K [hkv][cap][D] f16; V in the same 8-key blocks,
//                     [hkv][cap/8][D][8] f16 with dims in lane order.
struct KvLayout {
    int bits;  // 4, 8, or 16 (fp16 mode)
    int D;
    int hkv;
    int cap;  // rows per head, multiple of 32
    int64_t k_row_words() const { return (int64_t)D * bits / 32; }
    int64_t k_param_words() const { return D / kGroup; }
    int64_t v_block_words() const { return (int64_t)D * bits / 4; }
    int64_t v_block_param_words() const { return (int64_t)(D / kGroup) * 8; }
};

// K params of a row are stored in slot order (0, 2, 1, 3) when a row has four
// 64-dim groups, so that the two groups a 4-bit decode lane dequantizes
// (g/2 and 2 + g/2) are one 8-byte load.
__host__ __device__ inline int k_param_slot(int group, int n_groups) {
    return n_groups == 4 ? ((group & 1) * 2 + (group >> 1)) : group;
}

// 4-bit V block word: key slot k (0..7) of a dim sits at nibble k/2 + 4*(k%2),
// so `(w & 0x000F000F)`, `(w & 0x00F000F0)`, `(w>>8 & ..)` yield the key pairs
// (0,1), (2,3), (4,5), (6,7) as fp16 magic-number halves.
__host__ __device__ inline int v4_nibble_pos(int k) { return (k >> 1) + 4 * (k & 1); }

// Physical slot of dim d inside a V block, in units of one dim's 8 codes
// (4 bytes at 4-bit, 8 bytes at 8-bit, 16 bytes for fp16 values). Lane n of
// an MFMA column group owns dims [n*DPL, (n+1)*DPL), DPL = D/16, and reads
// them with 128-bit loads; E dims fit in 16 bytes.
// Slot = 16*E*j + E*n + (d % E) with j = (d % DPL) / E.
__host__ __device__ inline int v_phys_dim(int d, int D, int bits) {
    const int dpl = D / 16;
    const int e = bits == 4 ? 4 : (bits == 8 ? 2 : 1);
    const int n = d / dpl, r = d % dpl;
    return 16 * e * (r / e) + e * n + (r % e);
}

// Logical dim of physical slot `slot` of a V block (inverse of v_phys_dim).
__host__ __device__ inline int v_logical_dim(int slot, int D, int bits) {
    const int dpl = D / 16;
    const int e = bits == 4 ? 4 : (bits == 8 ? 2 : 1);
    const int i = slot % e, n = (slot / e) % 16, j = slot / (16 * e);
    return n * dpl + e * j + i;
}

// v_phys_dim(64 pp + 4 n + c, D, bits) split into a part that depends only
// on n (0..15, an MFMA column) and one that depends only on (pp, c), so that a
// lane's 4 * D/64 slots are one base plus immediates (same values, by algebra:
// 4n % DPL + c < DPL because DPL = D/16 is a multiple of 4).
__host__ __device__ inline int v_slot_base(int n, int D, int bits) {
    const int dpl = D / 16;
    if (bits == 4) return 64 * (n % (dpl / 4)) + 4 * ((4 * n) / dpl);
    if (bits == 8) return 16 * ((4 * n) % dpl) + 2 * ((4 * n) / dpl);
    return 16 * ((4 * n) % dpl) + (4 * n) / dpl;
}
__host__ __device__ constexpr int v_slot_off(int pp, int c, int D, int bits) {
    return bits == 4 ? c + (256 * pp) / (D / 16)
                     : (bits == 8 ? 32 * (c / 2) + c % 2 + (128 * pp) / (D / 16)
                                  : 16 * c + (64 * pp) / (D / 16));
}

__device__ inline half2v h2(uint32_t x) { return __builtin_bit_cast(half2v, x); }

// A 32-bit constant materialized in a VGPR the compiler cannot see through.
// gfx9 VOP3 encodings take no literal and at most one SGPR, so `(x & m) | k`
// with both constants visible compiles to v_and + v_or; with k in a VGPR it
// becomes one v_and_or_b32.
__device__ __forceinline__ uint32_t vconst(uint32_t x) {
    uint32_t r;
    asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(x));
    return r;
}
__device__ inline half8 as_h8(u32x4 v) { return __builtin_bit_cast(half8, v); }

// Wave-wide reductions. Inside each row of 16 lanes the partners come through
// DPP (quad_perm [1,0,3,2], [2,3,0,1], then row_ror 4 and 8: a VALU operand
// modifier, no LDS round trip); the two cross-row steps use ds_bpermute.
// Every lane ends with the result.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
// The value lane l ^ S holds (S a power of two below 64) without an LDS
// permute: DPP row moves for S < 16 (quad_perm for 1 and 2, a rotate by 8
// within the 16-lane row for 8, the row shift that stays in the row for 4)
// and the permlane swaps for 16 and 32 (after a swap of x with itself, a
// lower-half lane holds its own value in [0] and the partner's in [1], an
// upper-half lane the other way round). Exact copies, so any butterfly built
// on it keeps its arithmetic bit for bit.
template <int S>
__device__ __forceinline__ float lane_xor(float x, int lane) {
    const uint32_t u = __float_as_uint(x);
    if constexpr (S == 1) {
        return __uint_as_float(__builtin_amdgcn_update_dpp(0u, u, 0xB1, 0xF, 0xF, false));
    } else if constexpr (S == 2) {
        return __uint_as_float(__builtin_amdgcn_update_dpp(0u, u, 0x4E, 0xF, 0xF, false));
    } else if constexpr (S == 4) {
        const uint32_t up = __builtin_amdgcn_update_dpp(0u, u, 0x104, 0xF, 0xF, false);  // lane + 4
        const uint32_t dn = __builtin_amdgcn_update_dpp(0u, u, 0x114, 0xF, 0xF, false);  // lane - 4
        return __uint_as_float((lane & 4) ? dn : up);
    } else if constexpr (S == 8) {
        return __uint_as_float(__builtin_amdgcn_update_dpp(0u, u, 0x128, 0xF, 0xF, false));
    } else if constexpr (S == 16) {
        const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        return __uint_as_float((lane & 16) ? a[0] : a[1]);
    } else {
        static_assert(S == 32, "lane_xor: a power of two below 64");
        const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        return __uint_as_float((lane & 32) ? a[0] : a[1]);
    }
}

template <class Op>
__device__ __forceinline__ float wave_reduce(float x, Op op) {
    x = op(x, dpp_mov<0xB1>(x));   // quad_perm [1,0,3,2]
    x = op(x, dpp_mov<0x4E>(x));   // quad_perm [2,3,0,1]
    x = op(x, dpp_mov<0x124>(x));  // row_ror 4
    x = op(x, dpp_mov<0x128>(x));  // row_ror 8
    const int lane = (int)__lane_id();
    x = op(x, lane_xor<16>(x, lane));
    return op(x, lane_xor<32>(x, lane));
}
struct OpSum {
    __device__ float operator()(float a, float b) const { return a + b; }
};
struct OpMax {
    __device__ float operator()(float a, float b) const { return a < b ? b : a; }
};
struct OpMin {
    __device__ float operator()(float a, float b) const { return b < a ? b : a; }
};

// Thread-local last-error string for the C ABI.
void set_error(const std::string& msg);
const char* last_error();

// A device buffer for split-K partials that grows on demand and never frees
// memory a captured HIP graph may still reference: a buffer handed to work
// recorded into a graph is retired, not freed, when it grows, and released
// with the owner. A buffer no graph holds is freed after a synchronization:
// of the one stream that uses it (stream_owned: the per-(device, stream)
// workspaces), else of the device. It cannot grow while its stream is being
// captured (HIP allows no allocation there): such a call returns
// QW_ERR_STATE without touching the capture; one call of that shape before
// capturing sizes it. Growth allocates and frees device memory, which HIP
// forbids while any stream of the process is under a global-mode capture:
// size the buffers (one call of each shape) before such a capture begins.
struct GrowBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    bool captured = false;
    bool stream_owned = false;
    std::vector<void*> retired;
    int get(size_t need, hipStream_t stream, void** out);
    void release();
};

// Raises `kernel`'s dynamic-LDS limit on the current device to at least
// `bytes` (needed above 64 KB); thread safe, once per (kernel, device, size).
int ensure_dynamic_lds(const void* kernel, size_t bytes);

}  // namespace qw

#define QW_HIP_CHECK(expr)                                                          \
    do {                                                                            \
        hipError_t _e = (expr);                                                     \
        if (_e != hipSuccess) {                                                     \
            qw::set_error(std::string(#expr) + ": " + hipGetErrorString(_e));       \
            return QW_ERR_HIP;                                                      \
        }                                                                           \
    } while (0)

#define QW_REQUIRE(cond, code, msg)  \
    do {                             \
        if (!(cond)) {               \
            qw::set_error(msg);      \
            return (code);           \
        }                            \
    } while (0)
