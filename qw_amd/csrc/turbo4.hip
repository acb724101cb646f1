// turbo4.hip - the Turbo4 (symmetric PolarQuant) KV mode on gfx950:
// quantize-on-append, fetch, snapshot tensors and attention.
//
// Reference behaviour followed (cr0sh/qw):
//   quantize: crates/mlxcel-core/src/cache/turbo/quant.rs:270-440
//     (quantize_into_packed: fp32 norm, x / norm, signs1, Walsh-Hadamard,
//     signs2, nearest centroid by boundary count, nibble pack) and the pack
//     kernel crates/mlxcel-core/cpp/mlx_cxx_kernels.cpp:186-212 (index =
//     #boundaries below the value, rescale = f16(norm / max(|y|, 1e-10)));
//   fetch: quant.rs:486-546 (V: centroids, unit-normalised, inverse rotation,
//     times the norm) and :676-691 (K: f16(centroid * k_rescale), inverse
//     rotation);
//   attention: crates/mlxcel-core/src/cache/turbo/sparse_v.rs:1051-1072
//     (attention_turbo4_dequant_sdpa: q rotated into the K basis and cast to
//     fp16, K and V expanded to f16(centroid * rescale) in their rotated
//     bases, fp16 SDPA, output rotated back through the V basis), with the
//     bulk expansion of crates/mlx-cpp/turbo/turbo4_delegated_sdpa.cpp:193-221;
//   storage and growth: crates/mlxcel-core/src/cache.rs:1438-1597
//     (update_turbo4_sym).
//
// The Walsh-Hadamard transform is the orthonormal Sylvester one
// (H[i][j] = (-1)^popcount(i & j) / sqrt(D)), done in fp32 registers: a lane
// holds D/64 consecutive coordinates, the first log2(D/64) butterfly stages
// run inside the lane and the remaining six across lanes.
#include <math.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>

#include <utility>

#include "append.hpp"
#include "kv_cache.hpp"
#include "rope.hpp"
#include "turbo4_device.hpp"

namespace qw {

namespace {


// f16 of an fp32 product, rounded first to fp32 (the reference multiplies in
// fp32 and then casts); the register pin keeps the compiler from fusing the
// multiply and the conversion into one singly rounded mixed-precision op. The
// pin is not volatile: a volatile one is a scheduling barrier, which
// serialized every table lookup feeding a product behind the previous one.
__device__ __forceinline__ f16 f16_of_product(float a, float b) {
    float p = a * b;
    asm("" : "+v"(p));
    return (f16)p;
}

// ------------------------------------------------------------ append
//
// grid (n_tokens, hkv), 2 waves: wave 0 quantizes the K row (K signs), wave 1
// the V row (V signs); turbo4_append_row holds the steps.
template <int D>
__global__ __launch_bounds__(128) void turbo4_append_kernel(
    RowSrc rs, int t_old, int cap, const float* __restrict__ tab, uint8_t* __restrict__ k_packed,
    uint32_t* __restrict__ k_side, uint8_t* __restrict__ v_packed, uint32_t* __restrict__ v_side) {
    __shared__ float s_cb[16];
    if (threadIdx.x < 16) s_cb[threadIdx.x] = tab[T4Tab<D>::cb + threadIdx.x];
    __syncthreads();
    turbo4_append_row<D>(rs, blockIdx.x, blockIdx.y, (threadIdx.x >> 6) == 0, threadIdx.x & 63, t_old,
                         cap, tab, s_cb, k_packed, k_side, v_packed, v_side);
}

// ------------------------------------------------------------ fetch
//
// Rows [start, start + n) back in the original basis: grid (n, hkv), wave 0
// K, wave 1 V; out [hkv][n][D].
template <int D>
__global__ __launch_bounds__(128) void turbo4_fetch_kernel(
    const uint8_t* __restrict__ k_packed, const uint32_t* __restrict__ k_side,
    const uint8_t* __restrict__ v_packed, const uint32_t* __restrict__ v_side,
    const float* __restrict__ tab, int cap, int start, int n, f16* __restrict__ k_out,
    f16* __restrict__ v_out) {
    constexpr int VPL = D / 64;
    using TT = T4Tab<D>;
    __shared__ float s_cb[16];
    if (threadIdx.x < 16) s_cb[threadIdx.x] = tab[TT::cb + threadIdx.x];
    __syncthreads();
    const int i = blockIdx.x, h = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const bool is_k = wave == 0;
    const int t = start + i;
    const uint8_t* prow = (is_k ? k_packed : v_packed) + ((int64_t)h * cap + t) * (D / 2);
    uint32_t idx[VPL];
    if constexpr (VPL == 4) {
        const uint32_t w = *(const uint16_t*)(prow + 2 * lane);
#pragma unroll
        for (int j = 0; j < 4; j++) idx[j] = (w >> (4 * j)) & 15u;
    } else {
        const uint32_t w = prow[lane];
        idx[0] = w & 15u;
        idx[1] = w >> 4;
    }
    const half2v side = __builtin_bit_cast(half2v, (is_k ? k_side : v_side)[(int64_t)h * cap + t]);
    float y[VPL];
    float mul;
    if (is_k) {
        // K: the rotated values as the fp16 expansion holds them
        const float r = (float)side.x;
#pragma unroll
        for (int j = 0; j < VPL; j++) y[j] = (float)f16_of_product(s_cb[idx[j]], r);
        mul = 1.0f;
    } else {
        // V: unit-normalised centroids, scaled by the stored norm at the end
        float csq = 0.0f;
#pragma unroll
        for (int j = 0; j < VPL; j++) {
            y[j] = s_cb[idx[j]];
            csq = __builtin_fmaf(y[j], y[j], csq);
        }
        const float yn = fmaxf(sqrtf(t4_wave_sum(csq)), 1e-10f);
#pragma unroll
        for (int j = 0; j < VPL; j++) y[j] = y[j] / yn;
        mul = (float)side.x;
    }
    // inverse rotation: signs1 . H . signs2
    const float* s1 = tab + (is_k ? TT::k_s1 : TT::v_s1);
    const float* s2 = tab + (is_k ? TT::k_s2 : TT::v_s2);
#pragma unroll
    for (int j = 0; j < VPL; j++) y[j] *= s2[lane * VPL + j];
    wht_wave<D>(y, lane);
    f16* orow = (is_k ? k_out : v_out) + ((int64_t)h * n + i) * D;
#pragma unroll
    for (int j = 0; j < VPL; j++) {
        const float u = (y[j] * wht_scale(D)) * s1[lane * VPL + j];
        orow[lane * VPL + j] = is_k ? (f16)u : (f16)(u * mul);
    }
}

// ------------------------------------------- rotated fp16 expansion (SDPA)
//
// NB 8-key blocks of one head a workgroup of D threads: thread = (key,
// 8 coordinates) of each block, the loads of all NB blocks issued before the
// first is expanded. K_rot rows go to kw [hkv][capv][D]; V_rot to the fp16
// cache's transposed blocks vw [hkv][capv/8][D][8] (dims in lane order)
// through LDS. Keys past `T` are written as zeros (the fp16 kernels read
// whole 8-key blocks).
// 1: Turbo4 calls of up to 16 rows a KV head (decode) read the packed cache in
// the decode kernel; 0: they expand it to fp16 first, as longer blocks do.
#ifndef QW_T4_FUSED_DECODE
#define QW_T4_FUSED_DECODE 1
#endif
// 1: longer Turbo4 blocks (the fused verify pass, and the dequantize-then-SDPA
// route from 17 to kT4BlockRows rows a KV head) run in the block kernel, which
// reads the packed cache in place; 0: the verify kernel and the fp16 expansion.
#ifndef QW_T4_BLOCK
#define QW_T4_BLOCK 1
#endif
constexpr int kT4BlockRows = 1024;
// 1: update-and-attention calls that take the block kernel with one query tile,
// or the decode kernel, append their rows inside its launch; 0: the append
// kernel first.
#ifndef QW_T4_APPEND
#define QW_T4_APPEND 1
#endif
constexpr int kExpandBlocks = 4;  // 8-key blocks a workgroup (capv / 8 is a multiple of 32)

// VROWS: V rows too ([hkv][capv][D], for the general SDPA); else V in the fp16
// cache's 8-key blocks.
template <int D, bool VROWS = false>
__global__ __launch_bounds__(D) void turbo4_expand_kernel(
    const uint8_t* __restrict__ k_packed, const uint32_t* __restrict__ k_side,
    const uint8_t* __restrict__ v_packed, const uint32_t* __restrict__ v_side,
    const float* __restrict__ tab, int cap, int T, int capv, int b0, f16* __restrict__ kw,
    f16* __restrict__ vw) {
    constexpr int CPK = D / 8;  // 8-coordinate chunks a key
    constexpr int NB = kExpandBlocks;
    using TT = T4Tab<D>;
    __shared__ float s_cb[16];
    __shared__ __align__(16) f16 sv[NB][D][8];
    if (threadIdx.x < 16) s_cb[threadIdx.x] = tab[TT::cb + threadIdx.x];
    const int h = blockIdx.y;
    const int k = threadIdx.x / CPK, c = threadIdx.x % CPK;
    uint32_t kb[NB], vb[NB], ks[NB], vs[NB];
#pragma unroll
    for (int n = 0; n < NB; n++) {
        const int t = (b0 + blockIdx.x * NB + n) * 8 + k;
        kb[n] = vb[n] = ks[n] = vs[n] = 0u;
        if (t < T) {
            const int64_t r = (int64_t)h * cap + t;
            kb[n] = *(const uint32_t*)(k_packed + r * (D / 2) + 4 * c);
            vb[n] = *(const uint32_t*)(v_packed + r * (D / 2) + 4 * c);
            ks[n] = k_side[r];
            vs[n] = v_side[r];
        }
    }
    __syncthreads();  // s_cb
#pragma unroll
    for (int n = 0; n < NB; n++) {
        const int blk = b0 + blockIdx.x * NB + n;
        const int t = blk * 8 + k;
        half8 kv8, vv8;
        if (t < T) {
            const float kr = (float)__builtin_bit_cast(half2v, ks[n]).x;
            const float vr = (float)__builtin_bit_cast(half2v, vs[n]).y;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                kv8[j] = f16_of_product(s_cb[(kb[n] >> (4 * j)) & 15u], kr);
                vv8[j] = f16_of_product(s_cb[(vb[n] >> (4 * j)) & 15u], vr);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) kv8[j] = vv8[j] = (f16)0.0f;
        }
        *(half8*)(kw + ((int64_t)h * capv + t) * D + 8 * c) = kv8;
        if constexpr (VROWS) {
            *(half8*)(vw + ((int64_t)h * capv + t) * D + 8 * c) = vv8;
        } else {
            // (the fp16 cache keeps V dims in MFMA lane order, v_phys_dim)
#pragma unroll
            for (int j = 0; j < 8; j++) sv[n][v_phys_dim(8 * c + j, D, 16)][k] = vv8[j];
        }
    }
    if constexpr (VROWS) return;
    __syncthreads();
    const int p = threadIdx.x;  // physical dim slot
#pragma unroll
    for (int n = 0; n < NB; n++) {
        const int blk = blockIdx.x * NB + n;
        *(half8*)(vw + (((int64_t)h * (capv / 8) + blk) * D + p) * 8) = *(const half8*)&sv[n][p][0];
    }
}

// ------------------------------------------------------------ rotation
//
// rows of D fp16 or fp32: out = f16(s_out . (H / sqrt(D)) . s_in . in) in
// fp32, one wave a row.
template <int D, typename TIn = f16>
__global__ __launch_bounds__(256) void turbo4_rotate_kernel(const TIn* __restrict__ in,
                                                            f16* __restrict__ out, int rows,
                                                            const float* __restrict__ s_in,
                                                            const float* __restrict__ s_out) {
    constexpr int VPL = D / 64;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;  // whole waves leave together
    const TIn* r = in + (int64_t)row * D;
    float y[VPL];
#pragma unroll
    for (int j = 0; j < VPL; j++) y[j] = (float)r[lane * VPL + j] * s_in[lane * VPL + j];
    wht_wave<D>(y, lane);
    f16* o = out + (int64_t)row * D;
#pragma unroll
    for (int j = 0; j < VPL; j++)
        o[lane * VPL + j] = (f16)((y[j] * wht_scale(D)) * s_out[lane * VPL + j]);
}

// q for the fused verify kernel: out = f16(f32(f32(s_out . (H / sqrt(D)) .
// s_in . in) * post)), the reference's fp32 rotated q times scale * log2(e),
// then the kernel's fp16 cast (turbo4_attention.cpp:67-79).
template <int D>
__global__ __launch_bounds__(256) void turbo4_rotate_scaled_kernel(
    const f16* __restrict__ in, f16* __restrict__ out, int rows, const float* __restrict__ s_in,
    const float* __restrict__ s_out, float post) {
    constexpr int VPL = D / 64;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;  // whole waves leave together
    const f16* r = in + (int64_t)row * D;
    float y[VPL];
#pragma unroll
    for (int j = 0; j < VPL; j++) y[j] = (float)r[lane * VPL + j] * s_in[lane * VPL + j];
    wht_wave<D>(y, lane);
    f16* o = out + (int64_t)row * D;
#pragma unroll
    for (int j = 0; j < VPL; j++) {
        float v = (y[j] * wht_scale(D)) * s_out[lane * VPL + j];
        asm("" : "+v"(v));
        o[lane * VPL + j] = f16_of_product(v, post);
    }
}

// ------------------------------------------- fused causal verify
//
// The reference's fused Turbo4 verify pass (turbo4_attention.cpp:45-193
// partial, :198-264 merge; gate fused_attention.rs:70-100): causal blocks of
// 1..5 query rows over a cache of more than 2048 tokens, scored straight from
// the packed codes. Semantics: q' = f16(q_rot * scale * log2 e), K and V
// expanded as f16(f32(centroid) * f32(rescale)), fp32 scores in the log2
// domain, an exact running max, fp32 softmax sums and fp32 P.V.
//
// grid (splits, kv_heads), 8 waves. A workgroup walks its key range in
// stages of 64 keys: the stage's K codes are expanded into LDS rows
// [key][D], its V codes transposed into [dim][key] (so the P.V B operand is
// one 8-byte read of 4 consecutive keys), double-buffered, with the codes of
// two stages ahead held in registers. Wave (rt, kq) takes query rows
// 16 rt .. 16 rt + 15 (G heads x rows, row = qr * G + head) against keys
// 16 kq .. 16 kq + 15 of every stage: QK on v_mfma_f32_16x16x32_f16 (A = K
// rows, B = q'), P.V on v_mfma_f32_16x16x16_f16 with P straight from the
// score tile as an fp16 high part plus an fp16 remainder (every product
// exact, sums fp32). The four key quarters merge through LDS at the end and the
// workgroup writes one fp32 partial per row, merged by the block kernels'
// merge kernel.
constexpr int kT4vKeys = 64;     // keys a stage
constexpr int kT4vRows = 32;     // query rows a workgroup (partial row stride)
constexpr int kT4vWaves = 8;     // two row tiles x four 16-key quarters of a stage
constexpr int kT4vThreads = 64 * kT4vWaves;

struct T4VerifyArgs {
    const uint8_t* k_codes;   // [hkv][cap][D/2]
    const uint32_t* k_side;   // [hkv][cap] half2(k_rescale, 0)
    const uint8_t* v_codes;   // [hkv][cap][D/2]
    const uint32_t* v_side;   // [hkv][cap] half2(v_norm, v_rescale)
    const float* cb;          // 16 centroids
    const f16* qs;            // [hq][Tq][D] q' = f16(q_rot * scale * log2 e)
    float* part_o;            // [hkv][nc][kT4vRows][D]
    float2* part_ml;          // [hkv][nc][kT4vRows] (m in natural units, l)
    int cap, T, Tq, G, R, nc, kps;
};

template <int D>
struct T4vShape {
    static constexpr int KROW = D + 8;                 // K row stride in LDS (halves)
    static constexpr int VROW = kT4vKeys + 4;          // V^T row stride (halves), 8-byte rows
    static constexpr int KBUF = kT4vKeys * KROW;       // halves a K buffer
    static constexpr int VBUF = D * VROW;              // halves a V buffer
    static constexpr size_t lds = (size_t)2 * (KBUF + VBUF) * sizeof(f16) + 16 * sizeof(float);
};

template <int D>
__global__ __launch_bounds__(kT4vThreads) void turbo4_verify_kernel(T4VerifyArgs a) {
    using S = T4vShape<D>;
    constexpr int NM = D / 32, NT = D / 16, KS = kT4vKeys;
    constexpr int KROW = S::KROW, VROW = S::VROW;
    constexpr int CH = D / 32;              // 16-byte code chunks a row (32 coordinates each)
    constexpr int NTH = kT4vThreads, NKW = kT4vWaves / 2;
    constexpr int KW = KS / NKW;            // keys a wave a stage (one 16-key MFMA tile)
    static_assert(KW == 16, "one 16-key tile a wave a stage");
    constexpr int NCH = KS * CH;            // K (and V) chunks a stage
    constexpr int NJ = (NCH + NTH - 1) / NTH;  // chunks a thread
    extern __shared__ __attribute__((aligned(16))) char lds_raw[];
    f16* const sK = (f16*)lds_raw;                          // [2][KS][KROW]
    f16* const sV = sK + 2 * S::KBUF;                       // [2][D][VROW]
    float* const s_cb = (float*)(sV + 2 * S::VBUF);         // [16]

    const int c = blockIdx.x, h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int rt = wave & 1, kq = wave >> 1;
    if (tid < 16) s_cb[tid] = a.cb[tid];
    const int k0 = c * a.kps;
    const int k1 = min(a.T, k0 + a.kps);
    const int n_st = (k1 - k0 + KS - 1) / KS;

    // q' as the B operand: column r16 = row 16 rt + r16 (head row % G, query
    // row row / G), dims 32m + 8g .. +7.
    const int row = 16 * rt + r16;
    const bool row_ok = row < a.R;
    const int qr = row_ok ? row / a.G : 0, gh = row_ok ? row % a.G : 0;
    const int lim = row_ok ? a.T - a.Tq + qr : -1;  // last key the row sees
    const bool tile_live = 16 * rt < a.R;            // wave-uniform
    half8 qb[NM];
    {
        const f16* qrow = a.qs + ((int64_t)(h * a.G + gh) * a.Tq + qr) * D;
#pragma unroll
        for (int m = 0; m < NM; m++)
            qb[m] = row_ok ? *(const half8*)(qrow + 32 * m + 8 * g) : half8{};
    }

    // A stage's codes: K chunk j of this thread = key (t / CH), chunk t % CH
    // (8 lanes a 128-byte row); V chunk j = key t % KS, chunk t / KS (a wave
    // covers 64 consecutive keys of one chunk, so the transposed writes hit 32
    // distinct banks). Keys past the range load as zeros.
    struct Stage {
        u32x4 kc[NJ], vc[NJ];
        uint32_t kr[NJ], vr[NJ];
    };
    const int64_t hrow = (int64_t)h * a.cap;
    auto load = [&](Stage& st, int s) {
        const int base = k0 + s * KS;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int t = tid + NTH * j;
            const int kk = base + t / CH, kc = t % CH;
            const int vk = base + t % KS, vcn = t / KS;
            st.kc[j] = u32x4{0u, 0u, 0u, 0u};
            st.vc[j] = u32x4{0u, 0u, 0u, 0u};
            st.kr[j] = st.vr[j] = 0u;
            if (t >= NCH) continue;
            if (kk < k1) {
                st.kc[j] = *(const u32x4*)(a.k_codes + (hrow + kk) * (D / 2) + 16 * kc);
                st.kr[j] = a.k_side[hrow + kk];
            }
            if (vk < k1) {
                st.vc[j] = *(const u32x4*)(a.v_codes + (hrow + vk) * (D / 2) + 16 * vcn);
                st.vr[j] = a.v_side[hrow + vk];
            }
        }
    };
    auto store = [&](const Stage& st, int b) {
        f16* const K = sK + b * S::KBUF;
        f16* const V = sV + b * S::VBUF;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int t = tid + NTH * j;
            if (t >= NCH) continue;
            {
                const int key = t / CH, ch = t % CH;
                const float r = (float)__builtin_bit_cast(half2v, st.kr[j]).x;
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    half8 o;
#pragma unroll
                    for (int n = 0; n < 8; n++) o[n] = f16_of_product(s_cb[(st.kc[j][w] >> (4 * n)) & 15u], r);
                    *(half8*)(K + key * KROW + 32 * ch + 8 * w) = o;
                }
            }
            {
                const int key = t % KS, ch = t / KS;
                const float r = (float)__builtin_bit_cast(half2v, st.vr[j]).y;
#pragma unroll
                for (int w = 0; w < 4; w++)
#pragma unroll
                    for (int n = 0; n < 8; n++)
                        V[(32 * ch + 8 * w + n) * VROW + key] =
                            f16_of_product(s_cb[(st.vc[j][w] >> (4 * n)) & 15u], r);
            }
        }
    };

    float m_run = -INFINITY;  // running max of row r16 (log2 domain)
    float l_run = 0.0f;       // this lane's share of the row's sum
    float4v acc[NT];          // rows 4g + i of the tile, dims 16 mm + r16
#pragma unroll
    for (int mm = 0; mm < NT; mm++) acc[mm] = float4v{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int b, int s) {
        const f16* const K = sK + b * S::KBUF;
        const f16* const V = sV + b * S::VBUF;
        const int kb = k0 + s * KS + KW * kq;  // the wave's first key of the stage
        float sc[1][4];
        {
            constexpr int u = 0;
            float4v sacc = {0.f, 0.f, 0.f, 0.f};
            const f16* krow = K + (KW * kq + r16) * KROW + 8 * g;
#pragma unroll
            for (int m = 0; m < NM; m++)
                sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const half8*)(krow + 32 * m), qb[m],
                                                              sacc, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = kb + 16 * u + 4 * g + i;
                sc[u][i] = key < k1 && key <= lim ? sacc[i] : -INFINITY;
            }
        }
        float mx = fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3]));
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float mref = m_new == -INFINITY ? 0.0f : m_new;
        if (__any(m_new != m_run)) {
            const float corr = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - mref);
            l_run *= corr;
            float f[4];
#pragma unroll
            for (int i = 0; i < 4; i++) f[i] = __shfl(corr, 4 * g + i);
#pragma unroll
            for (int mm = 0; mm < NT; mm++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[mm][i] *= f[i];
        }
        m_run = m_new;
        {
            constexpr int u = 0;
            half4v ph, pl;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float p = __builtin_amdgcn_exp2f(sc[u][i] - mref);
                l_run += p;
                ph[i] = (f16)p;
                pl[i] = (f16)(p - (float)ph[i]);
            }
            const f16* vcol = V + r16 * VROW + KW * kq + 4 * g;
#pragma unroll
            for (int mm = 0; mm < NT; mm++) {
                const half4v vb = *(const half4v*)(vcol + 16 * mm * VROW);
                acc[mm] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, vb, acc[mm], 0, 0, 0);
                acc[mm] = __builtin_amdgcn_mfma_f32_16x16x16f16(pl, vb, acc[mm], 0, 0, 0);
            }
        }
    };

    // Codes of stage s + 1 sit in the stage being stored, those of s + 2 / s + 3
    // are in flight; one barrier a stage.
    Stage s0, s1;
    if (n_st > 0) load(s0, 0);
    if (n_st > 1) load(s1, 1);
    __syncthreads();  // s_cb
    if (n_st > 0) {
        store(s0, 0);
        if (n_st > 2) load(s0, 2);
    }
    __syncthreads();
    auto round = [&](Stage& nx, int s) {
        if (s + 1 < n_st) {
            store(nx, (s + 1) & 1);
            if (s + 3 < n_st) load(nx, s + 3);
        }
        if (tile_live) compute(s & 1, s);
        __syncthreads();
    };
    for (int s = 0; s < n_st; s += 2) {
        round(s1, s);
        if (s + 1 < n_st) round(s0, s + 1);
    }

    // ---- the four key quarters of each row tile: kq > 0 park (m, l, O) in
    // LDS, kq = 0 folds them in and writes the partial.
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    float* const park = (float*)lds_raw;  // [2 row tiles][NKW - 1][NT * 4 + 2][64]
    constexpr int PS = (NT * 4 + 2) * 64;
    static_assert((size_t)2 * (NKW - 1) * PS * sizeof(float) <= T4vShape<D>::lds,
                  "parked quarters fit");
    if (kq > 0) {
        float* pw = park + (rt * (NKW - 1) + kq - 1) * PS;
#pragma unroll
        for (int mm = 0; mm < NT; mm++)
#pragma unroll
            for (int i = 0; i < 4; i++) pw[(mm * 4 + i) * 64 + lane] = acc[mm][i];
        pw[(NT * 4) * 64 + lane] = m_run;
        pw[(NT * 4 + 1) * 64 + lane] = l_run;
    }
    __syncthreads();
    if (kq > 0 || !tile_live) return;
    const float* pws = park + rt * (NKW - 1) * PS;
    float mq[NKW], fq[NKW];
    mq[0] = m_run;
#pragma unroll
    for (int q = 1; q < NKW; q++) mq[q] = pws[(q - 1) * PS + (NT * 4) * 64 + lane];
    float M = mq[0];
#pragma unroll
    for (int q = 1; q < NKW; q++) M = fmaxf(M, mq[q]);
    float L = 0.0f;
#pragma unroll
    for (int q = 0; q < NKW; q++) {
        fq[q] = mq[q] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mq[q] - M);
        L += (q == 0 ? l_run : pws[(q - 1) * PS + (NT * 4 + 1) * 64 + lane]) * fq[q];
    }
    float F[NKW][4];
#pragma unroll
    for (int q = 0; q < NKW; q++)
#pragma unroll
        for (int i = 0; i < 4; i++) F[q][i] = __shfl(fq[q], 4 * g + i);
    const int64_t pbase = ((int64_t)h * a.nc + c) * kT4vRows;
    if (g == 0 && row_ok) a.part_ml[pbase + row] = float2{M * kLn2, L};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int orow = 16 * rt + 4 * g + i;
        if (orow >= a.R) continue;
        float* prow = a.part_o + (pbase + orow) * D;
#pragma unroll
        for (int mm = 0; mm < NT; mm++) {
            float o = acc[mm][i] * F[0][i];
#pragma unroll
            for (int q = 1; q < NKW; q++)
                o = __builtin_fmaf(pws[(q - 1) * PS + (mm * 4 + i) * 64 + lane], F[q][i], o);
            prow[16 * mm + r16] = o;
        }
    }
}

// Snapshot planes <-> the side arrays: [hkv][n] k_rescale, v_norms, v_rescale.
__global__ void turbo4_side_export_kernel(const uint32_t* __restrict__ k_side,
                                          const uint32_t* __restrict__ v_side, int hkv, int cap,
                                          int n, f16* __restrict__ k_rescale,
                                          f16* __restrict__ v_norms, f16* __restrict__ v_rescale) {
    const int64_t total = (int64_t)hkv * n;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int h = (int)(i / n), t = (int)(i % n);
        const half2v ks = __builtin_bit_cast(half2v, k_side[(int64_t)h * cap + t]);
        const half2v vs = __builtin_bit_cast(half2v, v_side[(int64_t)h * cap + t]);
        k_rescale[i] = ks.x;
        v_norms[i] = vs.x;
        v_rescale[i] = vs.y;
    }
}

__global__ void turbo4_side_import_kernel(const f16* __restrict__ k_rescale,
                                          const f16* __restrict__ v_norms,
                                          const f16* __restrict__ v_rescale, int hkv, int cap,
                                          int n, uint32_t* __restrict__ k_side,
                                          uint32_t* __restrict__ v_side) {
    const int64_t total = (int64_t)hkv * n;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int h = (int)(i / n), t = (int)(i % n);
        half2v ks, vs;
        ks.x = k_rescale[i];
        ks.y = (f16)0.0f;
        vs.x = v_norms[i];
        vs.y = v_rescale[i];
        k_side[(int64_t)h * cap + t] = __builtin_bit_cast(uint32_t, ks);
        v_side[(int64_t)h * cap + t] = __builtin_bit_cast(uint32_t, vs);
    }
}

static unsigned grid_for(int64_t work) {
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>((work + 255) / 256, 4096));
}

// Workspace of the attention routes (the rotated fp16 K/V, q, the fp32
// merged rows and split partials), one per (device, stream), shared by the
// Turbo4 caches that attend on that stream as MLX's allocator shares its
// transient buffers: calls on one stream are ordered by the stream, calls on
// different streams never share it. A GrowBuffer, so a call captured in a HIP
// graph keeps its buffer when a later call grows the workspace.
std::mutex g_t4_mu;
std::map<std::pair<int, hipStream_t>, GrowBuffer> g_t4_ws;

int t4_workspace(int device, hipStream_t stream, size_t need, void** out) {
    std::lock_guard<std::mutex> lock(g_t4_mu);
    GrowBuffer& b = g_t4_ws[{device, stream}];
    b.stream_owned = true;  // only calls on `stream` use it
    return b.get(need, stream, out);
}

}  // namespace

// ------------------------------------------------------------ host side

int KVCache::turbo4_setup() {
    QW_REQUIRE(D == 128 || D == 256, QW_ERR_UNSUPPORTED, "turbo4: head_dim must be 128 or 256");
    std::vector<float> tab(4 * D + 32, 0.0f);
    const uint32_t ks = turbo_seed + turbo4::kKSeedOffset;
    const std::vector<float> parts[4] = {
        turbo4::signs(D, turbo_seed), turbo4::signs(D, turbo_seed + turbo4::kSubSeed),
        turbo4::signs(D, ks), turbo4::signs(D, ks + turbo4::kSubSeed)};
    for (int p = 0; p < 4; p++) std::copy(parts[p].begin(), parts[p].end(), tab.begin() + p * D);
    const std::vector<float> cb = turbo4::centroids(4, D);
    const std::vector<float> bd = turbo4::boundaries(cb);
    std::copy(cb.begin(), cb.end(), tab.begin() + 4 * D);
    std::copy(bd.begin(), bd.end(), tab.begin() + 4 * D + 16);
    DeviceGuard dg(device);
    QW_REQUIRE(dg.ok, QW_ERR_HIP, "turbo4: hipSetDevice failed");
    if (!t4_tables) {
        if (hipMalloc(&t4_tables, tab.size() * sizeof(float)) != hipSuccess) {
            (void)hipGetLastError();
            t4_tables = nullptr;
            set_error("turbo4: hipMalloc of the codec tables failed");
            return QW_ERR_OUT_OF_MEMORY;
        }
    }
    QW_HIP_CHECK(hipMemcpy(t4_tables, tab.data(), tab.size() * sizeof(float),
                           hipMemcpyHostToDevice));
    return QW_OK;
}

int KVCache::turbo4_update(const RowSrc& rs, int n_tokens, hipStream_t stream) {
    dim3 grid(n_tokens, hkv);
    if (D == 256)
        hipLaunchKernelGGL(turbo4_append_kernel<256>, grid, dim3(128), 0, stream, rs, offset, cap,
                           t4_tables, (uint8_t*)k_data, k_params, (uint8_t*)v_data, v_params);
    else
        hipLaunchKernelGGL(turbo4_append_kernel<128>, grid, dim3(128), 0, stream, rs, offset, cap,
                           t4_tables, (uint8_t*)k_data, k_params, (uint8_t*)v_data, v_params);
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

int KVCache::turbo4_dequantize(int start, int n, void* k_out, void* v_out,
                               hipStream_t stream) const {
    dim3 grid(n, hkv);
    if (D == 256)
        hipLaunchKernelGGL(turbo4_fetch_kernel<256>, grid, dim3(128), 0, stream,
                           (const uint8_t*)k_data, k_params, (const uint8_t*)v_data, v_params,
                           t4_tables, cap, start, n, (f16*)k_out, (f16*)v_out);
    else
        hipLaunchKernelGGL(turbo4_fetch_kernel<128>, grid, dim3(128), 0, stream,
                           (const uint8_t*)k_data, k_params, (const uint8_t*)v_data, v_params,
                           t4_tables, cap, start, n, (f16*)k_out, (f16*)v_out);
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

int KVCache::turbo4_export(void* kp, void* kr, void* vp, void* vn, void* vr,
                           hipStream_t stream) const {
    QW_REQUIRE(turbo4(), QW_ERR_STATE, "turbo4 snapshot requires a Turbo4 cache");
    QW_REQUIRE(kp && kr && vp && vn && vr, QW_ERR_INVALID_ARGUMENT,
               "turbo4 snapshot: null tensor pointer");
    const int n = offset;
    if (n == 0) return QW_OK;
    DeviceGuard dg(device);
    QW_REQUIRE(dg.ok, QW_ERR_HIP, "turbo4 snapshot: hipSetDevice failed");
    const size_t rb = (size_t)D / 2;
    QW_HIP_CHECK(hipMemcpy2DAsync(kp, n * rb, k_data, cap * rb, n * rb, hkv,
                                  hipMemcpyDeviceToDevice, stream));
    QW_HIP_CHECK(hipMemcpy2DAsync(vp, n * rb, v_data, cap * rb, n * rb, hkv,
                                  hipMemcpyDeviceToDevice, stream));
    hipLaunchKernelGGL(turbo4_side_export_kernel, dim3(grid_for((int64_t)hkv * n)), dim3(256), 0,
                       stream, k_params, v_params, hkv, cap, n, (f16*)kr, (f16*)vn, (f16*)vr);
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

int KVCache::turbo4_import(int n, const void* kp, const void* kr, const void* vp, const void* vn,
                           const void* vr, hipStream_t stream) {
    QW_REQUIRE(turbo4(), QW_ERR_STATE, "turbo4 snapshot requires a Turbo4 cache");
    QW_REQUIRE(n > 0, QW_ERR_INVALID_ARGUMENT, "turbo4 snapshot offset must be positive");
    QW_REQUIRE(kp && kr && vp && vn && vr, QW_ERR_INVALID_ARGUMENT,
               "turbo4 snapshot: null tensor pointer");
    DeviceGuard dg(device);
    QW_REQUIRE(dg.ok, QW_ERR_HIP, "turbo4 snapshot: hipSetDevice failed");
    offset = 0;
    int rc = reserve(n, stream);
    if (rc) return rc;
    const size_t rb = (size_t)D / 2;
    QW_HIP_CHECK(hipMemcpy2DAsync(k_data, cap * rb, kp, n * rb, n * rb, hkv,
                                  hipMemcpyDeviceToDevice, stream));
    QW_HIP_CHECK(hipMemcpy2DAsync(v_data, cap * rb, vp, n * rb, n * rb, hkv,
                                  hipMemcpyDeviceToDevice, stream));
    hipLaunchKernelGGL(turbo4_side_import_kernel, dim3(grid_for((int64_t)hkv * n)), dim3(256), 0,
                       stream, (const f16*)kr, (const f16*)vn, (const f16*)vr, hkv, cap, n,
                       k_params, v_params);
    QW_HIP_CHECK(hipGetLastError());
    offset = n;
    return QW_OK;
}

// Fused causal verify route: rotate q into the K basis (times scale * log2 e),
// the fused kernel's split partials, the merge, the rotation back.
static int turbo4_verify(KVCache& c, const void* q, int n_q_heads, int n_rows, float scale,
                         void* out, hipStream_t stream) {
    const int D = c.D, T = c.offset, G = n_q_heads / c.hkv, R = G * n_rows;
    const int qrows = n_q_heads * n_rows;
    // about one workgroup a CU: splits of whole 64-key stages
    const int want = std::max(1, std::min(256 / c.hkv, (T + kT4vKeys - 1) / kT4vKeys));
    const int kps = ((T + want - 1) / want + kT4vKeys - 1) / kT4vKeys * kT4vKeys;
    const int nc = (T + kps - 1) / kps;
    const size_t q_bytes = (size_t)qrows * D * sizeof(f16);
    const size_t o_bytes = (size_t)qrows * D * sizeof(float);  // merged rows, fp32
    const size_t po_bytes = (size_t)c.hkv * nc * kT4vRows * D * sizeof(float);
    const size_t need = q_bytes + o_bytes + po_bytes + (size_t)c.hkv * nc * kT4vRows * sizeof(float2);

    void* wbuf = nullptr;
    if (int rc0 = t4_workspace(c.device, stream, need, &wbuf)) return rc0;
    // The merge leaves the rotated output in fp32 and the rotation back casts
    // it to fp16 once, as the reference's merge (fp32, turbo4_attention.cpp:
    // 438-446) and turbo4_v_inverse_rotate (quant.rs:764-768) do.
    f16* q_s = (f16*)wbuf;
    float* o_rot = (float*)((char*)wbuf + q_bytes);
    float* part_o = (float*)((char*)wbuf + q_bytes + o_bytes);
    float2* part_ml = (float2*)((char*)wbuf + q_bytes + o_bytes + po_bytes);
    const float* tab = c.t4_tables;
    const float post = scale * 1.4426950408889634f;  // fp32, as the reference forms it

    T4VerifyArgs a;
    a.k_codes = (const uint8_t*)c.k_data;
    a.k_side = c.k_params;
    a.v_codes = (const uint8_t*)c.v_data;
    a.v_side = c.v_params;
    a.qs = q_s;
    a.part_o = part_o;
    a.part_ml = part_ml;
    a.cap = c.cap;
    a.T = T;
    a.Tq = n_rows;
    a.G = G;
    a.R = R;
    a.nc = nc;
    a.kps = kps;
    const dim3 rg((qrows + 3) / 4), vg(nc, c.hkv);
    if (D == 256) {
        using TT = T4Tab<256>;
        a.cb = tab + TT::cb;
        constexpr size_t sh = T4vShape<256>::lds;
        int rc = ensure_dynamic_lds((const void*)turbo4_verify_kernel<256>, sh);
        if (rc) return rc;
        hipLaunchKernelGGL(turbo4_rotate_scaled_kernel<256>, rg, dim3(256), 0, stream,
                           (const f16*)q, q_s, qrows, tab + TT::k_s1, tab + TT::k_s2, post);
        hipLaunchKernelGGL(turbo4_verify_kernel<256>, vg, dim3(kT4vThreads), sh, stream, a);
    } else {
        using TT = T4Tab<128>;
        a.cb = tab + TT::cb;
        constexpr size_t sh = T4vShape<128>::lds;
        int rc = ensure_dynamic_lds((const void*)turbo4_verify_kernel<128>, sh);
        if (rc) return rc;
        hipLaunchKernelGGL(turbo4_rotate_scaled_kernel<128>, rg, dim3(256), 0, stream,
                           (const f16*)q, q_s, qrows, tab + TT::k_s1, tab + TT::k_s2, post);
        hipLaunchKernelGGL(turbo4_verify_kernel<128>, vg, dim3(kT4vThreads), sh, stream, a);
    }
    QW_HIP_CHECK(hipGetLastError());
    int rc = launch_partial_merge(part_o, part_ml, nc, kT4vRows, 0, R, c.hkv, D, G, n_rows, nullptr,
                                  stream, 0, o_rot);
    if (rc) return rc;
    if (D == 256) {
        using TT = T4Tab<256>;
        hipLaunchKernelGGL((turbo4_rotate_kernel<256, float>), rg, dim3(256), 0, stream,
                           (const float*)o_rot, (f16*)out, qrows, tab + TT::v_s2, tab + TT::v_s1);
    } else {
        using TT = T4Tab<128>;
        hipLaunchKernelGGL((turbo4_rotate_kernel<128, float>), rg, dim3(256), 0, stream,
                           (const float*)o_rot, (f16*)out, qrows, tab + TT::v_s2, tab + TT::v_s1);
    }
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

// The same two routes through the block kernel, which rotates q into the K
// basis itself and reads the packed cache in place: fused = true, the fused
// verify pass (q rotated and scaled by scale * log2 e in fp32 then cast to
// fp16, fp32 merged rows rotated back and cast once, by the merge);
// fused = false, the dequantize-then-SDPA route (q rotated to fp16, the fp16
// SDPA arithmetic on the expansion's values, the fp16 rows rotated back here).
// The reference's gate for its fused verify pass (fused_attention.rs:69-110,
// cache.rs:3520-3560): causal, 1..5 query rows, more than 2048 cached tokens,
// at most 32 query heads a KV head. The block kernel runs it for any of those
// shapes (G * rows <= 160: one or two 128-row query tiles, every key split);
// the standalone verify kernel (QW_T4_BLOCK = 0) holds G * rows <= 32.
static bool t4_fused_route(bool causal, int n_rows, int T, int G) {
    return causal && n_rows >= 1 && n_rows <= 5 && T > 2048 && G <= 32 &&
           (QW_T4_BLOCK || G * n_rows <= kT4vRows);
}

static int turbo4_block(KVCache& c, const void* q, int n_q_heads, int n_rows, float scale,
                        bool causal, bool fused, void* out, hipStream_t stream) {
    const int D = c.D, G = n_q_heads / c.hkv;
    const float* tab = c.t4_tables;
    if (fused)
        return launch_block_attention_t4(c, (const f16*)q, G, n_rows, scale, causal, true, tab,
                                         (f16*)out, stream);
    const int qrows = n_q_heads * n_rows;
    void* wbuf = nullptr;
    if (int rc0 = t4_workspace(c.device, stream, (size_t)qrows * D * sizeof(f16), &wbuf)) return rc0;
    f16* o_r = (f16*)wbuf;
    int rc = launch_block_attention_t4(c, (const f16*)q, G, n_rows, scale, causal, false, tab, o_r,
                                       stream);
    if (rc) return rc;
    const dim3 rg((qrows + 3) / 4);
    if (D == 256) {
        using TT = T4Tab<256>;
        hipLaunchKernelGGL(turbo4_rotate_kernel<256>, rg, dim3(256), 0, stream, (const f16*)o_r,
                           (f16*)out, qrows, tab + TT::v_s2, tab + TT::v_s1);
    } else {
        using TT = T4Tab<128>;
        hipLaunchKernelGGL(turbo4_rotate_kernel<128>, rg, dim3(256), 0, stream, (const f16*)o_r,
                           (f16*)out, qrows, tab + TT::v_s2, tab + TT::v_s1);
    }
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

bool turbo4_fused_append_route(const KVCache& c, bool causal, int n_rows, int G) {
    return QW_T4_APPEND && QW_T4_BLOCK && t4_fused_route(causal, n_rows, c.offset + n_rows, G) &&
           block_append_fits_t4(c, G, n_rows);
}

bool turbo4_decode_route(const KVCache& c, bool causal, int n_rows, int G) {
    return !t4_fused_route(causal, n_rows, c.offset + n_rows, G) && QW_T4_FUSED_DECODE &&
           G * n_rows <= 16 && c.offset >= 1;
}

int turbo4_update_and_attention(KVCache& c, const void* q, int n_q_heads, int n_rows,
                                const void* k_new, const void* v_new, float scale, bool causal,
                                void* out, hipStream_t stream) {
    const int G = n_q_heads / c.hkv, T = c.offset + n_rows;
    // the routes of turbo4_attention below: the fused pass and the block
    // kernel's one-tile blocks append in the block launch, the decode route
    // in the decode launch's append unit
    const bool fused = t4_fused_route(causal, n_rows, T, G);
    const bool block = QW_T4_BLOCK && block_append_fits_t4(c, G, n_rows) && (fused || G * n_rows > 16);
    const bool decode = turbo4_decode_route(c, causal, n_rows, G);
    if (!(QW_T4_APPEND && (block || decode))) {
        int rc = c.update(k_new, v_new, n_rows, stream);
        if (rc) return rc;
        return turbo4_attention(c, q, n_q_heads, n_rows, scale, causal, out, stream);
    }
    DeviceGuard dg(c.device);
    QW_REQUIRE(dg.ok, QW_ERR_HIP, "attention: hipSetDevice failed");
    if (T > c.cap) {
        int rc = c.reserve(std::max(T, c.cap + c.cap / 2), stream);
        if (rc) return rc;
    }
    const float* tab = c.t4_tables;
    const f16 *qq = (const f16*)q, *kn = (const f16*)k_new, *vn = (const f16*)v_new;
    if (decode)
        return launch_turbo4_decode_append(c, qq, G, n_rows, kn, vn, scale, causal, tab, (f16*)out,
                                           stream);
    if (fused)
        return launch_block_append_attention_t4(c, qq, G, n_rows, kn, vn, scale, causal, true, tab,
                                                (f16*)out, stream);
    const int D = c.D, qrows = n_q_heads * n_rows;
    void* wbuf = nullptr;
    if (int rc0 = t4_workspace(c.device, stream, (size_t)qrows * D * sizeof(f16), &wbuf)) return rc0;
    f16* o_r = (f16*)wbuf;
    int rc = launch_block_append_attention_t4(c, qq, G, n_rows, kn, vn, scale, causal, false, tab,
                                              o_r, stream);
    if (rc) return rc;
    const dim3 rg((qrows + 3) / 4);
    if (D == 256) {
        using TT = T4Tab<256>;
        hipLaunchKernelGGL(turbo4_rotate_kernel<256>, rg, dim3(256), 0, stream, (const f16*)o_r,
                           (f16*)out, qrows, tab + TT::v_s2, tab + TT::v_s1);
    } else {
        using TT = T4Tab<128>;
        hipLaunchKernelGGL(turbo4_rotate_kernel<128>, rg, dim3(256), 0, stream, (const f16*)o_r,
                           (f16*)out, qrows, tab + TT::v_s2, tab + TT::v_s1);
    }
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

static int turbo4_expansion_route(KVCache& c, const void* q, int n_q_heads, int n_rows,
                                  float scale, bool causal, const SdpaOptions* opts, void* out,
                                  hipStream_t stream);

int turbo4_attention_general(KVCache& c, const void* q, int n_q_heads, int n_rows, float scale,
                             const SdpaOptions& opts, void* out, hipStream_t stream) {
    DeviceGuard dg(c.device);
    QW_REQUIRE(dg.ok, QW_ERR_HIP, "attention: hipSetDevice failed");
    return turbo4_expansion_route(c, q, n_q_heads, n_rows, scale, opts.causal, &opts, out, stream);
}

int turbo4_attention(KVCache& c, const void* q, int n_q_heads, int n_rows, float scale,
                     bool causal, void* out, hipStream_t stream) {
    QW_REQUIRE(q && out, QW_ERR_INVALID_ARGUMENT, "attention: null q/out");
    QW_REQUIRE(n_q_heads > 0 && n_q_heads % c.hkv == 0, QW_ERR_INVALID_ARGUMENT,
               "attention: n_q_heads must be a positive multiple of n_kv_heads");
    QW_REQUIRE(n_rows > 0, QW_ERR_INVALID_ARGUMENT, "attention: n_rows must be > 0");
    QW_REQUIRE(c.offset >= n_rows, QW_ERR_INVALID_ARGUMENT,
               "attention: fewer cached keys than query rows");
    DeviceGuard dg(c.device);
    QW_REQUIRE(dg.ok, QW_ERR_HIP, "attention: hipSetDevice failed");
    const int T = c.offset;
    if (t4_fused_route(causal, n_rows, T, n_q_heads / c.hkv))
        return QW_T4_BLOCK ? turbo4_block(c, q, n_q_heads, n_rows, scale, causal, true, out, stream)
                           : turbo4_verify(c, q, n_q_heads, n_rows, scale, out, stream);
    const float* tab = c.t4_tables;
#if QW_T4_FUSED_DECODE
    if ((n_q_heads / c.hkv) * n_rows <= 16)
        // Up to 16 rows a KV head: the decode kernel rotates q, reads the
        // packed indices in place (the values the fp16 expansion would hold,
        // the fp16 SDPA arithmetic on them) and its merge rotates the output
        // back.
        return launch_turbo4_decode(c, (const f16*)q, n_q_heads / c.hkv, n_rows, scale, causal, tab,
                                    (f16*)out, stream);
#endif
    // Up to 8 query tiles a KV head, the block kernel reads the packed cache in
    // place; past that, its per-tile dequantization (repeated for every query
    // tile) costs more than expanding the cache once for the fp16 kernel
    // (measured at 4 q heads a KV head, depth 8k and 32k: 1024 rows a head
    // 320 against 329 us, 2048 rows 651 against 599 us). From
    // block_image_min_rows() on, the block kernel expands the tiles once into
    // LDS images itself.
    if (QW_T4_BLOCK && ((n_q_heads / c.hkv) * n_rows <= kT4BlockRows ||
                        (n_q_heads / c.hkv) * n_rows >= block_image_min_rows(true)))
        return turbo4_block(c, q, n_q_heads, n_rows, scale, causal, false, out, stream);
    return turbo4_expansion_route(c, q, n_q_heads, n_rows, scale, causal, nullptr, out, stream);
}

// The expansion route: q rotated into the K basis (fp16), the rotated K/V
// expanded to fp16 rows once, attention over them in the rotated basis (the
// fp16 cache's kernels, or with opts the general SDPA: mask, softcap,
// window), and the output rotated back through the V basis
// (attention_turbo4_dequant_sdpa, turbo/sparse_v.rs:1051-1072).
static int turbo4_expansion_route(KVCache& c, const void* q, int n_q_heads, int n_rows,
                                  float scale, bool causal, const SdpaOptions* opts, void* out,
                                  hipStream_t stream) {
    const int D = c.D, T = c.offset;
    const int qrows = n_q_heads * n_rows;
    const float* tab = c.t4_tables;
    const int capv = (T + 255) / 256 * 256;
    // with a sliding window only keys from lo (a multiple of 256) are expanded
    // and attended; the rows keep their places in the [hkv][capv][D] planes
    const int lo = opts ? window_first_key(*opts, T, n_rows, 256) : 0;
    const size_t kv_bytes = (size_t)c.hkv * capv * D * sizeof(f16);
    const size_t q_bytes = (size_t)n_q_heads * n_rows * D * sizeof(f16);
    const size_t need = 2 * kv_bytes + 2 * q_bytes;

    void* wbuf = nullptr;
    if (int rc0 = t4_workspace(c.device, stream, need, &wbuf)) return rc0;
    f16* kw = (f16*)wbuf;
    f16* vw = (f16*)((char*)wbuf + kv_bytes);
    f16* q_rot = (f16*)((char*)wbuf + 2 * kv_bytes);
    f16* o_rot = (f16*)((char*)wbuf + 2 * kv_bytes + q_bytes);
    // Every 8-key block up to capv: rows past T become zeros, as the fp16
    // cache's unused rows are, since the fp16 kernels read whole tiles.
    dim3 eg((capv - lo) / (8 * kExpandBlocks), c.hkv);
    const int b0 = lo / 8;  // first 8-key block expanded
    if (D == 256) {
        using TT = T4Tab<256>;
        hipLaunchKernelGGL(turbo4_rotate_kernel<256>, dim3((qrows + 3) / 4), dim3(256), 0, stream,
                           (const f16*)q, q_rot, qrows, tab + TT::k_s1, tab + TT::k_s2);
        if (opts)
            hipLaunchKernelGGL((turbo4_expand_kernel<256, true>), eg, dim3(256), 0, stream,
                               (const uint8_t*)c.k_data, c.k_params, (const uint8_t*)c.v_data,
                               c.v_params, tab, c.cap, T, capv, b0, kw, vw);
        else
            hipLaunchKernelGGL(turbo4_expand_kernel<256>, eg, dim3(256), 0, stream,
                               (const uint8_t*)c.k_data, c.k_params, (const uint8_t*)c.v_data,
                               c.v_params, tab, c.cap, T, capv, b0, kw, vw);
    } else {
        using TT = T4Tab<128>;
        hipLaunchKernelGGL(turbo4_rotate_kernel<128>, dim3((qrows + 3) / 4), dim3(256), 0, stream,
                           (const f16*)q, q_rot, qrows, tab + TT::k_s1, tab + TT::k_s2);
        if (opts)
            hipLaunchKernelGGL((turbo4_expand_kernel<128, true>), eg, dim3(128), 0, stream,
                               (const uint8_t*)c.k_data, c.k_params, (const uint8_t*)c.v_data,
                               c.v_params, tab, c.cap, T, capv, b0, kw, vw);
        else
            hipLaunchKernelGGL(turbo4_expand_kernel<128>, eg, dim3(128), 0, stream,
                               (const uint8_t*)c.k_data, c.k_params, (const uint8_t*)c.v_data,
                               c.v_params, tab, c.cap, T, capv, b0, kw, vw);
    }
    QW_HIP_CHECK(hipGetLastError());
    int rc;
    if (opts) {
        // rotated K and V rows, [hkv][capv][D]
        rc = sdpa_general(q_rot, n_q_heads, n_rows, kw + (int64_t)lo * D, vw + (int64_t)lo * D,
                          c.hkv, T - lo, D, (int64_t)capv * D, D, (int64_t)capv * D, D, scale,
                          shift_keys(*opts, lo), o_rot, stream);
    } else {
        // The rotated K/V seen as an fp16 cache (not owning its planes); it
        // borrows the Turbo4 cache's split-K workspace.
        KVCache view;
        view.mode = QW_KV_FP16;
        view.bits = 16;
        view.D = D;
        view.hkv = c.hkv;
        view.device = c.device;
        view.offset = T;
        view.cap = capv;
        view.k_data = kw;
        view.v_data = vw;
        view.fast_flag = c.fast_flag;
        std::swap(view.ws, c.ws);
        rc = launch_attention(view, q_rot, n_q_heads, n_rows, scale, causal, o_rot, stream);
        std::swap(view.ws, c.ws);
    }
    if (rc) return rc;
    if (D == 256) {
        using TT = T4Tab<256>;
        hipLaunchKernelGGL(turbo4_rotate_kernel<256>, dim3((qrows + 3) / 4), dim3(256), 0, stream,
                           o_rot, (f16*)out, qrows, tab + TT::v_s2, tab + TT::v_s1);
    } else {
        using TT = T4Tab<128>;
        hipLaunchKernelGGL(turbo4_rotate_kernel<128>, dim3((qrows + 3) / 4), dim3(256), 0, stream,
                           o_rot, (f16*)out, qrows, tab + TT::v_s2, tab + TT::v_s1);
    }
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

}  // namespace qw
