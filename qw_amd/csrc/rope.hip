// rope.hip - fused q/k RoPE out of the fused QKV projection, and the cache
// append that rotates K as it reads it.
//
// Reference behaviour followed (cr0sh/qw):
//   fused_rope_qk_append: crates/mlx-cpp/turbo/fused_rope_append.cpp:80-180
//   (kernel body), :378-420 (argument contract), FFI declaration
//   crates/mlxcel-core/src/lib.rs:1462-1476, caller
//   crates/mlxcel-core/src/layers.rs:2852-2905.
//
// Input  qkv [B][L][(Hq + 2 Hkv) D]: per token the q heads, then the k heads,
//        then the v heads, each D contiguous fp16.
// Output q [B][Hq][L][D]; k, v [B][Hkv][L][D] (dest_layout 0, the dense cache
//        slab order) or [B][L][Hkv][D] (dest_layout 1, paged pool row order).
// q and k are rotated (rope.hpp); v is moved only.
//
// One thread per (token, head slot, pair): a pair is two dims, so a wave
// covers 128 dims of one head and its loads and stores are contiguous runs
// (the half-split layout reads dims p and p + R/2 as two runs). The op is a
// copy with a few VALU ops per pair, bound by HBM at 2 x 2 bytes a dim.
#include <algorithm>
#include <cmath>

#include "kv_cache.hpp"
#include "rope.hpp"

namespace qw {

struct RopeArgs {
    const f16* qkv;
    f16* q_out;
    f16* k_out;
    f16* v_out;
    int batch, seq, hq, hkv, D;
    int rope_dims, traditional, dest_layout;
    int slot_begin, slot_end;  // head slots handled: [0, hq) q, then k, then v
    float log2_base, scale;
    int positions_base;
};

__global__ __launch_bounds__(256) void rope_qkv_kernel(RopeArgs a) {
    const int half = a.D >> 1;
    const int slots = a.hq + 2 * a.hkv;
    const int nsl = a.slot_end - a.slot_begin;
    const int64_t total = (int64_t)a.batch * a.seq * nsl * half;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int p = (int)(i % half);
        const int64_t rest = i / half;
        const int slot = a.slot_begin + (int)(rest % nsl);
        const int64_t row = rest / nsl;  // b * seq + t
        const int b = (int)(row / a.seq), t = (int)(row % a.seq);
        const f16* in = a.qkv + row * ((int64_t)slots * a.D) + (int64_t)slot * a.D;

        int kind, h;  // 0 q, 1 k, 2 v
        if (slot < a.hq) {
            kind = 0;
            h = slot;
        } else if (slot < a.hq + a.hkv) {
            kind = 1;
            h = slot - a.hq;
        } else {
            kind = 2;
            h = slot - a.hq - a.hkv;
        }
        int64_t ob;
        f16* out;
        if (kind == 0) {
            ob = (((int64_t)b * a.hq + h) * a.seq + t) * a.D;
            out = a.q_out;
        } else {
            ob = a.dest_layout == 0 ? (((int64_t)b * a.hkv + h) * a.seq + t) * a.D
                                    : (((int64_t)b * a.seq + t) * a.hkv + h) * a.D;
            out = kind == 1 ? a.k_out : a.v_out;
        }
        const int rhalf = a.rope_dims >> 1;
        int i1, i2;
        const bool rotate = kind != 2 && p < rhalf;
        if (kind == 2) {
            i1 = 2 * p;
            i2 = i1 + 1;
        } else if (rotate) {
            i1 = a.traditional ? 2 * p : p;
            i2 = a.traditional ? 2 * p + 1 : p + rhalf;
        } else {
            // the unrotated tail [R, D): two dims per leftover pair index
            i1 = a.rope_dims + 2 * (p - rhalf);
            i2 = i1 + 1;
        }
        const f16 x1 = in[i1], x2 = in[i2];
        if (rotate) {
            float r1, r2;
            rope_pair((float)x1, (float)x2, p, rhalf, a.log2_base, a.scale,
                      t + a.positions_base, r1, r2);
            out[ob + i1] = (f16)r1;
            out[ob + i2] = (f16)r2;
        } else {
            out[ob + i1] = x1;
            out[ob + i2] = x2;
        }
    }
}

// The same op four pairs a thread, for D and rope_dims multiples of 8 (a
// group of four pairs is then wholly rotated or wholly tail): the dims of a
// group are one 16-byte run (traditional pairs, v, the tail) or two 8-byte
// runs (half-split pairs p and p + R/2), so a wave moves 0.5-1 KB per access.
// Each element's value is the scalar kernel's (same rope_pair).
// One workgroup a token row (grid.x = b * seq + t): the row's cos/sin table
// (one entry a rotated pair, shared by every head) goes to LDS first, then
// the threads walk the row's (slot, group) units, 32-bit index math.
constexpr int kRopeMaxPairs = 256;  // rope_dims / 2 the vector kernel takes

__global__ __launch_bounds__(256) void rope_qkv_vec_kernel(RopeArgs a) {
    const int groups = a.D >> 3;       // 4-pair groups a head
    const int rgroups = a.rope_dims >> 3;
    const int rhalf = a.rope_dims >> 1;
    const int slots = a.hq + 2 * a.hkv;
    const int nsl = a.slot_end - a.slot_begin;
    const int64_t row = blockIdx.x;  // b * seq + t
    __shared__ float2 cs[kRopeMaxPairs];
    {
        const int t = (int)(row % a.seq);
        for (int p = threadIdx.x; p < rhalf; p += blockDim.x) {
            float c, sn;
            rope_cs(p, rhalf, a.log2_base, a.scale, t + a.positions_base, c, sn);
            cs[p] = float2{c, sn};
        }
    }
    __syncthreads();
    for (int u = threadIdx.x; u < nsl * groups; u += blockDim.x) {
        const int gi = u % groups;
        const int slot = a.slot_begin + u / groups;
        const int b = (int)(row / a.seq), t = (int)(row % a.seq);
        const f16* in = a.qkv + row * ((int64_t)slots * a.D) + (int64_t)slot * a.D;
        int kind, h;  // 0 q, 1 k, 2 v
        if (slot < a.hq) {
            kind = 0;
            h = slot;
        } else if (slot < a.hq + a.hkv) {
            kind = 1;
            h = slot - a.hq;
        } else {
            kind = 2;
            h = slot - a.hq - a.hkv;
        }
        int64_t ob;
        f16* out;
        if (kind == 0) {
            ob = (((int64_t)b * a.hq + h) * a.seq + t) * a.D;
            out = a.q_out;
        } else {
            ob = a.dest_layout == 0 ? (((int64_t)b * a.hkv + h) * a.seq + t) * a.D
                                    : (((int64_t)b * a.seq + t) * a.hkv + h) * a.D;
            out = kind == 1 ? a.k_out : a.v_out;
        }
        // Groups [0, R/8) are rotated, groups [R/8, D/8) are the tail, dims
        // 8 gi .. 8 gi + 7 (8 (R/8) = R). A rotated group holds pairs 4 gi ..
        // 4 gi + 3: dims 8 gi .. + 7 when traditional, else dims 4 gi .. + 3
        // and their partners 4 gi + R/2 .. + 3.
        if (kind == 2 || gi >= rgroups) {
            *(u32x4*)(out + ob + 8 * gi) = *(const u32x4*)(in + 8 * gi);
        } else if (a.traditional) {
            const u32x4 w = *(const u32x4*)(in + 8 * gi);
            u32x4 o;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const half2v x = h2(w[j]);
                float r1, r2;
                const float2 c2 = cs[4 * gi + j];
                rope_rot((float)x.x, (float)x.y, c2.x, c2.y, r1, r2);
                half2v y;
                y.x = (f16)r1;
                y.y = (f16)r2;
                o[j] = __builtin_bit_cast(uint32_t, y);
            }
            *(u32x4*)(out + ob + 8 * gi) = o;
        } else {
            const int pg = gi;  // pairs 4 pg .. 4 pg + 3
            const uint2 w1 = *(const uint2*)(in + 4 * pg);
            const uint2 w2 = *(const uint2*)(in + 4 * pg + rhalf);
            const half2v a1[2] = {h2(w1.x), h2(w1.y)}, a2[2] = {h2(w2.x), h2(w2.y)};
            half2v o1[2], o2[2];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float x1 = (float)(j & 1 ? a1[j >> 1].y : a1[j >> 1].x);
                const float x2 = (float)(j & 1 ? a2[j >> 1].y : a2[j >> 1].x);
                float r1, r2;
                const float2 c2 = cs[4 * pg + j];
                rope_rot(x1, x2, c2.x, c2.y, r1, r2);
                if (j & 1) {
                    o1[j >> 1].y = (f16)r1;
                    o2[j >> 1].y = (f16)r2;
                } else {
                    o1[j >> 1].x = (f16)r1;
                    o2[j >> 1].x = (f16)r2;
                }
            }
            *(uint2*)(out + ob + 4 * pg) =
                uint2{__builtin_bit_cast(uint32_t, o1[0]), __builtin_bit_cast(uint32_t, o1[1])};
            *(uint2*)(out + ob + 4 * pg + rhalf) =
                uint2{__builtin_bit_cast(uint32_t, o2[0]), __builtin_bit_cast(uint32_t, o2[1])};
        }
    }
}

static int rope_launch(const RopeArgs& a, hipStream_t stream) {
    const int64_t rows = (int64_t)a.batch * a.seq * (a.slot_end - a.slot_begin);
    if (rows == 0) return QW_OK;
    // the vector form needs 16-byte aligned buffers (the ABI takes any pointers)
    auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    const bool vec = a.D % 8 == 0 && a.rope_dims % 8 == 0 && a.rope_dims / 2 <= kRopeMaxPairs &&
                     al16(a.qkv) && al16(a.q_out) && al16(a.k_out) && al16(a.v_out);
    if (vec) {
        // one workgroup a token row b * seq + t
        const int64_t tokens = (int64_t)a.batch * a.seq;
        QW_REQUIRE(tokens <= 0x7FFFFFFF, QW_ERR_INVALID_ARGUMENT,
                   "fused_rope_qk_append: too many rows");
        hipLaunchKernelGGL(rope_qkv_vec_kernel, dim3((unsigned)tokens), dim3(256), 0, stream, a);
    } else {
        // Grid-stride loop: enough workgroups to fill the chip several times over.
        const int64_t total = rows * (a.D / 2);
        const int64_t blocks = std::min<int64_t>((total + 255) / 256, 256 * 32);
        hipLaunchKernelGGL(rope_qkv_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a);
    }
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

// fused_rope_append.cpp:378-420: the same argument contract and messages.
static int rope_check(int hq, int hkv, int head_dim, int rope_dims) {
    QW_REQUIRE(hq > 0 && hkv > 0 && head_dim > 0, QW_ERR_INVALID_ARGUMENT,
               "fused_rope_qk_append: head counts and head_dim must be positive");
    QW_REQUIRE(head_dim % 2 == 0, QW_ERR_INVALID_ARGUMENT,
               "fused_rope_qk_append: head_dim must be even");
    QW_REQUIRE(rope_dims > 0 && rope_dims % 2 == 0 && rope_dims <= head_dim,
               QW_ERR_INVALID_ARGUMENT,
               "fused_rope_qk_append: rope_dims must be even, positive and <= head_dim");
    return QW_OK;
}

int fused_rope_qk_append(const void* qkv, int batch, int seq, int hq, int hkv, int head_dim,
                         int rope_dims, float rope_base, float rope_scale, int traditional,
                         int positions_base, int dest_layout, void* q_out, void* k_out,
                         void* v_out, hipStream_t stream) {
    int rc = rope_check(hq, hkv, head_dim, rope_dims);
    if (rc) return rc;
    QW_REQUIRE(dest_layout == 0 || dest_layout == 1, QW_ERR_INVALID_ARGUMENT,
               "fused_rope_qk_append: dest_layout must be 0 (dense slab) or 1 (paged pool)");
    QW_REQUIRE(batch >= 0 && seq >= 0, QW_ERR_INVALID_ARGUMENT,
               "fused_rope_qk_append: batch and seq must be >= 0");
    if ((int64_t)batch * seq == 0) return QW_OK;
    QW_REQUIRE(qkv && q_out && k_out && v_out, QW_ERR_INVALID_ARGUMENT,
               "fused_rope_qk_append: null buffer");
    RopeArgs a;
    a.qkv = (const f16*)qkv;
    a.q_out = (f16*)q_out;
    a.k_out = (f16*)k_out;
    a.v_out = (f16*)v_out;
    a.batch = batch;
    a.seq = seq;
    a.hq = hq;
    a.hkv = hkv;
    a.D = head_dim;
    a.rope_dims = rope_dims;
    a.traditional = traditional ? 1 : 0;
    a.dest_layout = dest_layout;
    a.slot_begin = 0;
    a.slot_end = hq + 2 * hkv;
    // MLX forms log2(base) on the host in fp32 (fused_rope_append.cpp:435-441).
    a.log2_base = std::log2(rope_base);
    a.scale = rope_scale;
    a.positions_base = positions_base;
    return rope_launch(a, stream);
}

int KVCache::rope_update(const void* qkv, int n_q_heads, int n_tokens, int rope_dims,
                         int traditional, float rope_base, float rope_scale, int position0,
                         void* q_out, hipStream_t stream) {
    int rc = rope_check(n_q_heads, hkv, D, rope_dims);
    if (rc) return rc;
    QW_REQUIRE(n_tokens >= 0, QW_ERR_INVALID_ARGUMENT, "rope_update: n_tokens must be >= 0");
    if (n_tokens == 0) return QW_OK;
    QW_REQUIRE(qkv && q_out, QW_ERR_INVALID_ARGUMENT, "rope_update: null buffer");
    DeviceGuard dg(device);
    QW_REQUIRE(dg.ok, QW_ERR_HIP, "rope_update: hipSetDevice failed");
    const float log2_base = std::log2(rope_base);
    RopeArgs a;
    a.qkv = (const f16*)qkv;
    a.q_out = (f16*)q_out;
    a.k_out = nullptr;
    a.v_out = nullptr;
    a.batch = 1;
    a.seq = n_tokens;
    a.hq = n_q_heads;
    a.hkv = hkv;
    a.D = D;
    a.rope_dims = rope_dims;
    a.traditional = traditional ? 1 : 0;
    a.dest_layout = 0;
    a.slot_begin = 0;
    a.slot_end = n_q_heads;  // q only: k and v go straight into the cache below
    a.log2_base = log2_base;
    a.scale = rope_scale;
    a.positions_base = position0;
    rc = rope_launch(a, stream);
    if (rc) return rc;
    const int64_t W = (int64_t)(n_q_heads + 2 * hkv) * D;
    RowSrc rs;
    rs.k = (const f16*)qkv + (int64_t)n_q_heads * D;
    rs.v = (const f16*)qkv + (int64_t)(n_q_heads + hkv) * D;
    rs.row_stride = W;
    rs.head_stride = D;
    rs.rope_dims = rope_dims;
    rs.traditional = traditional ? 1 : 0;
    rs.position0 = position0;
    rs.log2_base = log2_base;
    rs.scale = rope_scale;
    return update_rows(rs, n_tokens, stream);
}

}  // namespace qw
