// sdpa_general.hip - attention with the reference's general options: an
// explicit mask array, a logit softcap and a sliding window, over fp16 K/V rows.
//
// Reference path: layers::attention(q, k, v, scale, mask, softcap, window)
// (crates/mlxcel-core/src/layers.rs:4010-4060) and causal_attention(q, k, v,
// scale, softcap, window) (crates/mlxcel-core/src/lib.rs:3185-3275), reached
// from the cache by KVCache::update_and_turbo4_attention(q, k, v, scale, mask)
// (cache.rs:3495) and the runtime's masked branch (qwen3_next.rs:316-324),
// which append, dequantize and run this SDPA on the result.
//
// Semantics (the MLX composites those calls reduce to):
//   softcap == 0 (fast SDPA, mlx_cxx_bridge.cpp:3466-3497): scores
//     S = f16(f16(f16(scale) q) . k); an additive mask is cast to fp16 and
//     added in fp16 (S = f16(S + f16(mask))); a bool mask keeps the scores
//     where it is nonzero; P = softmax in fp32 entering P.V in fp16.
//   softcap > 0 (compiled_softcap_sdpa, mlx_cxx_bridge.cpp:1573-1590):
//     S = f16(q . k) (q unscaled), then in fp32 s = tanh(S scale / cap) cap,
//     plus the additive mask cast to fp16, softmax in fp32, and P.V with the
//     fp32 probabilities (split here into an fp16 high part and an fp16
//     remainder: two MFMAs, fp32-exact products).
//   causal: bottom-right, row r (position p = T - L + r) sees keys t <= p;
//   window > 0 (with causal): also t >= p - window + 1 (the windowed causal
//     mask of create_causal_mask_with_window, utils.rs:95-140; the
//     single-row trailing-window slice of causal_attention is the same set).
// A row with no visible key is zeros here (MLX: the mean of V for a bool mask,
// NaN for an additive -inf mask).
//
// Layout of the work: grid (key splits, row tiles, KV heads), 16 rows a wave,
// 4 waves a workgroup (1 for calls of up to 16 rows a KV head). Rows of a KV head are (query row, head in group)
// pairs, row index r * G + head, as in the other attention kernels. Each
// 32-key (16-key) tile of K (rows) and V (transposed) is loaded into
// registers a tile ahead and staged in LDS; a wave forms
// S^T = K . Q^T with v_mfma_f32_16x16x32_f16, which leaves each lane the
// scores of 8 keys of one query row, exactly the A operand of the P.V MFMA
// (v_mfma_f32_16x16x16f16, B = 4 keys of one V dim from LDS). Several key
// splits write fp32 partials (m, l, O) for the shared merge kernel.
#include <algorithm>
#include <cmath>
#include <map>
#include <mutex>
#include <string>

#include "kv_cache.hpp"
#include "qw_common.hpp"

namespace qw {

namespace {

struct GenArgs {
    const f16* q;  // [hq][L][D]
    const f16* k;
    const f16* v;
    int64_t khs, krs, vhs, vrs;  // element strides of K and V (head, row)
    const void* mask;            // [hq or broadcast][L][T], key stride 1; null: none
    int mask_kind;               // kMaskBool / kMaskF16 / kMaskBf16 / kMaskF32
    int64_t mhs, mrs;            // mask element strides (head, row); mhs 0 broadcasts
    f16* out;                    // [hq][L][D]
    float* part_o;               // [hkv][n_split][R][D]
    float2* part_ml;             // [hkv][n_split][R]
    int G, L, T, R, causal, window, n_split, keys_per_split;
    float scale, scale_h, softcap;
};

constexpr int kMaskBool = 0, kMaskF16 = 1, kMaskBf16 = 2, kMaskF32 = 3;

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
}

// The mask entry of (query head qh, row r, key t): visibility (bool) or the
// additive term cast to fp16 (f16 / bf16 / f32 masks, as the reference casts
// float masks to q's dtype).
__device__ __forceinline__ void mask_at(const GenArgs& a, int64_t off, bool* vis, float* add) {
    switch (a.mask_kind) {
        case kMaskBool:
            *vis = ((const uint8_t*)a.mask)[off] != 0;
            *add = 0.0f;
            break;
        case kMaskF16:
            *add = (float)((const f16*)a.mask)[off];
            break;
        case kMaskBf16:
            *add = (float)(f16)bf16_to_f32(((const uint16_t*)a.mask)[off]);
            break;
        default:
            *add = (float)(f16)((const float*)a.mask)[off];
    }
}

// NWV waves a workgroup (16 rows each): 4 for many rows a KV head, 1 (and
// 16-key tiles) for decode-sized calls, which then spread over four times the
// workgroups.
template <int D, bool SOFTCAP, int NWV>
__global__ __launch_bounds__(64 * NWV) void sdpa_general_kernel(GenArgs a) {
    constexpr int NM = D / 32, NJ = D / 16;
    constexpr int NU = NWV == 1 ? 1 : 2;  // 16-key sub-blocks a tile
    constexpr int KT = 16 * NU;           // keys a tile
    constexpr int KP = D + 8;   // K row pitch (halves)
    constexpr int VP = KT + 8;  // V^T row pitch (halves)
    constexpr int NTH = 64 * NWV, PER = KT * D / 8 / NTH;  // 16-byte chunks a thread a tile
    static_assert(PER * NTH == KT * D / 8, "whole chunks a thread");
    __shared__ __attribute__((aligned(16))) f16 sK[KT * KP];
    __shared__ __attribute__((aligned(16))) f16 sV[D * VP];
    const int sp = blockIdx.x, h = blockIdx.z;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r16 = lane & 15, g = lane >> 4;
    const int tile0 = blockIdx.y * 16 * NWV;
    // this lane's column: row index rho (query row r, head hg of the group)
    const int rho = tile0 + 16 * wave + r16;
    const bool row_ok = rho < a.R;
    const int r = row_ok ? rho / a.G : 0, hg = row_ok ? rho - r * a.G : 0;
    const int qh = h * a.G + hg;
    const int p = a.T - a.L + r;
    int lo = 0, hi = a.T;  // keys [lo, hi) this row may see
    if (a.causal) hi = min(hi, p + 1);
    if (a.window > 0) lo = max(lo, p - a.window + 1);

    // B operand: row r16's dims 32m + 8g .. +7 (q' = f16(f16(scale) q), or q)
    half8 qb[NM];
    {
        const f16* qrow = a.q + ((int64_t)qh * a.L + r) * D;
#pragma unroll
        for (int m = 0; m < NM; m++) {
            half8 x = row_ok ? *(const half8*)(qrow + 32 * m + 8 * g) : half8{};
            if constexpr (!SOFTCAP) {
#pragma unroll
                for (int e = 0; e < 8; e++) x[e] = (f16)(a.scale_h * (float)x[e]);
            }
            qb[m] = x;
        }
    }
    const int64_t moff = (int64_t)qh * a.mhs + (int64_t)r * a.mrs;

    // the workgroup's key range: its split, cut to what any of its rows sees
    const int rho_last = min(a.R, tile0 + 16 * NWV) - 1;
    int k_begin = sp * a.keys_per_split;
    int k_end = min(a.T, k_begin + a.keys_per_split);
    if (a.causal) k_end = min(k_end, a.T - a.L + rho_last / a.G + 1);
    if (a.window > 0) k_begin = max(k_begin, a.T - a.L + tile0 / a.G - a.window + 1);

    float m_run = -INFINITY, l_run = 0.0f;
    float4v acc_o[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) acc_o[j] = float4v{0.f, 0.f, 0.f, 0.f};

    // Tile t0's K and V chunks go through registers: loaded one tile ahead
    // (in flight during the previous tile's math), then stored to LDS (V
    // transposed, [dim][key]).
    // K chunks run along a key's row (contiguous loads and LDS stores); V
    // chunks run along the keys (chunk c: key c % KT, dims 8 (c / KT) ..), so
    // the lanes of a transposed store write consecutive keys of one dim row.
    half8 pk[PER], pv[PER];
    auto load = [&](int t0) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int c = threadIdx.x + i * NTH;
            const int kk = c / (D / 8), d8 = (c % (D / 8)) * 8, t = t0 + kk;
            pk[i] = t < k_end ? *(const half8*)(a.k + h * a.khs + (int64_t)t * a.krs + d8)
                              : half8{};
            const int vk = c % KT, vd = (c / KT) * 8, tv = t0 + vk;
            pv[i] = tv < k_end ? *(const half8*)(a.v + h * a.vhs + (int64_t)tv * a.vrs + vd)
                               : half8{};
        }
    };
    if (k_begin < k_end) load(k_begin);
    for (int t0 = k_begin; t0 < k_end; t0 += KT) {
        __syncthreads();  // the previous tile's reads are done
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int c = threadIdx.x + i * NTH;
            const int kk = c / (D / 8), d8 = (c % (D / 8)) * 8;
            *(half8*)(sK + kk * KP + d8) = pk[i];
            const int vk = c % KT, vd = (c / KT) * 8;
#pragma unroll
            for (int e = 0; e < 8; e++) sV[(vd + e) * VP + vk] = pv[i][e];
        }
        __syncthreads();
        if (t0 + KT < k_end) load(t0 + KT);
        // S^T: lane (g, r16) gets keys t0 + 16u + 4g + i of row r16
        float4v s4[NU];
#pragma unroll
        for (int u = 0; u < NU; u++) {
            s4[u] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int m = 0; m < NM; m++) {
                const half8 ka = *(const half8*)(sK + (16 * u + r16) * KP + 32 * m + 8 * g);
                s4[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[m], s4[u], 0, 0, 0);
            }
        }
        float sv[NU][4];
        float tmax = -INFINITY;
#pragma unroll
        for (int u = 0; u < NU; u++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = t0 + 16 * u + 4 * g + i;
                float s = (float)(f16)s4[u][i];
                if constexpr (SOFTCAP) s = tanhf(s * a.scale / a.softcap) * a.softcap;
                bool vis = row_ok && t >= lo && t < hi && t < k_end;
                if (vis && a.mask) {
                    float add = 0.0f;
                    mask_at(a, moff + t, &vis, &add);
                    if constexpr (SOFTCAP)
                        s += add;
                    else
                        s = (float)(f16)(s + add);
                }
                sv[u][i] = vis ? s : -INFINITY;
                tmax = fmaxf(tmax, sv[u][i]);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float m_new = fmaxf(m_run, tmax);
        const float mref = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m_run - mref) * kLog2e);
        m_run = m_new;
        l_run *= alpha;
        {
            float f[4];
#pragma unroll
            for (int i = 0; i < 4; i++) f[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc_o[j][i] *= f[i];
        }
#pragma unroll
        for (int u = 0; u < NU; u++) {
            half4v ph, pl;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float pv = __builtin_amdgcn_exp2f((sv[u][i] - mref) * kLog2e);
                l_run += pv;
                ph[i] = (f16)pv;
                pl[i] = (f16)(pv - (float)ph[i]);
            }
            // B: V rows t0 + 16u + 4g .. +3 of dim 16j + r16
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const half4v vb = *(const half4v*)(sV + (16 * j + r16) * VP + 16 * u + 4 * g);
                acc_o[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, vb, acc_o[j], 0, 0, 0);
                if constexpr (SOFTCAP)
                    acc_o[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(pl, vb, acc_o[j], 0, 0, 0);
            }
        }
    }
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);

    // acc_o[j][i]: row 4g + i of the wave, dim 16j + r16
    if (a.n_split == 1) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float l = __shfl(l_run, 4 * g + i);
            const int rw = tile0 + 16 * wave + 4 * g + i;
            if (rw >= a.R) continue;
            const int rr = rw / a.G, hh = h * a.G + (rw - rr * a.G);
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
            f16* orow = a.out + ((int64_t)hh * a.L + rr) * D;
#pragma unroll
            for (int j = 0; j < NJ; j++) orow[16 * j + r16] = (f16)(acc_o[j][i] * inv);
        }
    } else {
        const int64_t pbase = ((int64_t)h * a.n_split + sp) * a.R;
        if (g == 0 && row_ok) a.part_ml[pbase + rho] = float2{m_run, l_run};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int rw = tile0 + 16 * wave + 4 * g + i;
            if (rw >= a.R) continue;
            float* prow = a.part_o + (pbase + rw) * D;
#pragma unroll
            for (int j = 0; j < NJ; j++) prow[16 * j + r16] = acc_o[j][i];
        }
    }
}

template <int D, int NWV>
void launch_general(const GenArgs& a, dim3 grid, hipStream_t stream) {
    if (a.softcap > 0.0f)
        hipLaunchKernelGGL((sdpa_general_kernel<D, true, NWV>), grid, dim3(64 * NWV), 0, stream, a);
    else
        hipLaunchKernelGGL((sdpa_general_kernel<D, false, NWV>), grid, dim3(64 * NWV), 0, stream,
                           a);
}

template <int D>
void launch_general(const GenArgs& a, int nwv, dim3 grid, hipStream_t stream) {
    if (nwv == 1)
        launch_general<D, 1>(a, grid, stream);
    else
        launch_general<D, 4>(a, grid, stream);
}

// Split-K partials, one workspace per (device, stream).
std::mutex g_gen_mu;
std::map<std::pair<int, hipStream_t>, GrowBuffer> g_gen_ws;

int gen_workspace(int device, hipStream_t stream, size_t need, void** out) {
    std::lock_guard<std::mutex> lock(g_gen_mu);
    GrowBuffer& b = g_gen_ws[{device, stream}];
    b.stream_owned = true;
    return b.get(need, stream, out);
}

// The dequantized rows of a cache for the general route, one per (device,
// stream).
std::map<std::pair<int, hipStream_t>, GrowBuffer> g_gen_kv;

int gen_kv_workspace(int device, hipStream_t stream, size_t need, void** out) {
    std::lock_guard<std::mutex> lock(g_gen_mu);
    GrowBuffer& b = g_gen_kv[{device, stream}];
    b.stream_owned = true;
    return b.get(need, stream, out);
}

int mask_kind_of(int dtype) {
    switch (dtype) {
        case QW_MASK_BOOL: return kMaskBool;
        case QW_DTYPE_F16: return kMaskF16;
        case QW_DTYPE_BF16: return kMaskBf16;
        case QW_DTYPE_F32: return kMaskF32;
        default: return -1;
    }
}

}  // namespace

int sdpa_general(const void* q, int n_q_heads, int n_rows, const void* k, const void* v,
                 int n_kv_heads, int n_keys, int head_dim, int64_t khs, int64_t krs, int64_t vhs,
                 int64_t vrs, float scale, const SdpaOptions& o, void* out, hipStream_t stream) {
    QW_REQUIRE(q && k && v && out, QW_ERR_INVALID_ARGUMENT, "sdpa: null pointer");
    QW_REQUIRE(n_q_heads > 0 && n_kv_heads > 0 && n_q_heads % n_kv_heads == 0 && n_rows > 0 &&
                   n_keys > 0,
               QW_ERR_INVALID_ARGUMENT, "sdpa: bad head or length geometry");
    QW_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256, QW_ERR_INVALID_ARGUMENT,
               "sdpa: head dim must be 64, 128 or 256");
    QW_REQUIRE(((uintptr_t)q % 16) == 0 && ((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0 &&
                   khs % 8 == 0 && krs % 8 == 0 && vhs % 8 == 0 && vrs % 8 == 0,
               QW_ERR_UNSUPPORTED, "sdpa: q/K/V must be 16-byte aligned with strides % 8 == 0");
    QW_REQUIRE(!o.causal || n_keys >= n_rows, QW_ERR_INVALID_ARGUMENT,
               "sdpa: causal attention needs at least as many keys as query rows");
    QW_REQUIRE(o.window <= 0 || o.causal, QW_ERR_INVALID_ARGUMENT,
               "sdpa: a sliding window is the windowed causal mask (causal must be set)");
    QW_REQUIRE(o.softcap >= 0.0f && std::isfinite(o.softcap), QW_ERR_INVALID_ARGUMENT,
               "sdpa: softcap must be finite and >= 0");
    const int kind = o.mask ? mask_kind_of(o.mask_dtype) : 0;
    QW_REQUIRE(kind >= 0, QW_ERR_INVALID_ARGUMENT, "sdpa: unknown mask dtype");
    QW_REQUIRE(!(o.mask && kind == kMaskBool && o.softcap > 0.0f), QW_ERR_UNSUPPORTED,
               "sdpa: a bool mask with softcap is not supported (the reference casts it to "
               "additive 0/1 offsets); pass an additive mask");
    QW_REQUIRE(!o.mask || (o.mask_head_stride >= 0 && o.mask_row_stride >= 0),
               QW_ERR_INVALID_ARGUMENT, "sdpa: negative mask stride");
    const int G = n_q_heads / n_kv_heads, R = G * n_rows, D = head_dim;
    GenArgs a;
    a.q = (const f16*)q;
    a.k = (const f16*)k;
    a.v = (const f16*)v;
    a.khs = khs;
    a.krs = krs;
    a.vhs = vhs;
    a.vrs = vrs;
    a.mask = o.mask;
    a.mask_kind = kind;
    a.mhs = o.mask_head_stride;
    a.mrs = o.mask_row_stride;
    a.out = (f16*)out;
    a.part_o = nullptr;
    a.part_ml = nullptr;
    a.G = G;
    a.L = n_rows;
    a.T = n_keys;
    a.R = R;
    a.causal = o.causal ? 1 : 0;
    a.window = o.window > 0 ? o.window : 0;
    a.scale = scale;
    a.scale_h = (float)(f16)scale;
    a.softcap = o.softcap;
    // Up to 16 rows a KV head: one-wave workgroups (about 1024 of them);
    // else four-wave ones (about 256). Key splits of whole tiles, at least
    // four tiles each, at most 256 (the merge's limit).
    const int nwv = R <= 16 ? 1 : 4, kt = nwv == 1 ? 16 : 32;
    const int tiles = (R + 16 * nwv - 1) / (16 * nwv), units = tiles * n_kv_heads;
    const int key_tiles = (n_keys + kt - 1) / kt;
    const int target = nwv == 1 ? 1024 : 256;
    int ns = std::max(1, std::min({target / std::max(1, units), (key_tiles + 3) / 4, 256}));
    const int kps = ((key_tiles + ns - 1) / ns) * kt;
    ns = (n_keys + kps - 1) / kps;
    a.n_split = ns;
    a.keys_per_split = kps;
    int dev = 0;
    QW_HIP_CHECK(hipGetDevice(&dev));
    if (ns > 1) {
        const size_t no = (size_t)n_kv_heads * ns * R;
        void* ws = nullptr;
        if (int rc = gen_workspace(dev, stream, no * D * sizeof(float) + no * sizeof(float2), &ws))
            return rc;
        a.part_o = (float*)ws;
        a.part_ml = (float2*)((char*)ws + no * D * sizeof(float));
    }
    const dim3 grid(ns, tiles, n_kv_heads);
    if (D == 256)
        launch_general<256>(a, nwv, grid, stream);
    else if (D == 128)
        launch_general<128>(a, nwv, grid, stream);
    else
        launch_general<64>(a, nwv, grid, stream);
    QW_HIP_CHECK(hipGetLastError());
    if (ns > 1)
        return launch_partial_merge(a.part_o, a.part_ml, ns, R, 0, R, n_kv_heads, D, G, n_rows,
                                    (f16*)out, stream);
    return QW_OK;
}

// 1: a causal sliding window and / or a softcap without a mask over an affine,
// Int8 or fp16 cache runs the fused block kernel; 0: the dequantize-then-SDPA
// route.
#ifndef QW_FUSED_WINDOW
#define QW_FUSED_WINDOW 1
#endif

int window_first_key(const SdpaOptions& o, int T, int n_rows, int align) {
    if (o.window <= 0 || !o.causal) return 0;
    const int lo = std::max(0, T - n_rows - o.window + 1);
    return lo / align * align;
}

SdpaOptions shift_keys(const SdpaOptions& o, int lo) {
    SdpaOptions s = o;
    if (s.mask && lo > 0) {
        const int es = o.mask_dtype == QW_MASK_BOOL ? 1 : o.mask_dtype == QW_DTYPE_F32 ? 4 : 2;
        s.mask = (const char*)o.mask + (int64_t)lo * es;  // key stride 1
    }
    return s;
}

int cache_attention_general(KVCache& c, const void* q, int n_q_heads, int n_rows, float scale,
                            const SdpaOptions& o, void* out, hipStream_t stream) {
    QW_REQUIRE(q && out, QW_ERR_INVALID_ARGUMENT, "attention: null q/out");
    QW_REQUIRE(n_q_heads > 0 && n_q_heads % c.hkv == 0, QW_ERR_INVALID_ARGUMENT,
               "attention: n_q_heads must be a positive multiple of n_kv_heads");
    QW_REQUIRE(n_rows > 0 && c.offset > 0, QW_ERR_INVALID_ARGUMENT,
               "attention: empty query or empty cache");
    QW_REQUIRE(!o.causal || c.offset >= n_rows, QW_ERR_INVALID_ARGUMENT,
               "attention: fewer cached keys than query rows");
    if (!o.mask && o.softcap == 0.0f && o.window <= 0)
        return launch_attention(c, q, n_q_heads, n_rows, scale, o.causal, out, stream);
    if (c.turbo4()) return turbo4_attention_general(c, q, n_q_heads, n_rows, scale, o, out, stream);
    DeviceGuard dg(c.device);
    QW_REQUIRE(dg.ok, QW_ERR_HIP, "attention: hipSetDevice failed");
    // a causal window (the served arithmetic with a lower bound on each row's
    // keys) and / or a softcap, without a mask: the fused block kernel on the
    // codes, no dequantized copy
    if (QW_FUSED_WINDOW && !o.mask && (o.softcap > 0.0f || o.window > 0) &&
        (o.window <= 0 || o.causal) && std::isfinite(o.softcap) && (c.D == 128 || c.D == 256))
        return launch_block_attention_ext(c, (const f16*)q, n_q_heads / c.hkv, n_rows, scale,
                                          o.causal, o.window, o.softcap, (f16*)out, stream);
    const int T = c.offset, D = c.D;
    // A sliding window sees no key below lo (the first row's window start):
    // only keys lo .. T - 1 are dequantized, and the call runs on them with
    // the positions (p - lo) and mask columns shifted alike.
    const int lo = window_first_key(o, T, n_rows);
    const int n = T - lo;
    const size_t bytes = (size_t)c.hkv * n * D * sizeof(f16);
    void* ws = nullptr;
    if (int rc = gen_kv_workspace(c.device, stream, 2 * bytes, &ws)) return rc;
    char* kw = (char*)ws;
    char* vw = kw + bytes;
    if (int rc = c.dequantize(lo, n, kw, vw, stream)) return rc;  // [hkv][n][D] rows
    const SdpaOptions os = shift_keys(o, lo);
    return sdpa_general(q, n_q_heads, n_rows, kw, vw, c.hkv, n, D, (int64_t)n * D, D,
                        (int64_t)n * D, D, scale, os, out, stream);
}

}  // namespace qw
