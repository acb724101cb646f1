// attend_decode.hip - fused dequant-in-attention for decode and short verify
// blocks (G * n_rows <= 16 query rows per KV head), gfx950.
//
// Reference path replaced: KVCache::update_and_turbo4_attention ->
// turbo4_dequant_sdpa_prefix (crates/mlxcel-core/src/cache.rs:3495-3510,
// :3652-3697), which dequantizes the whole cache and then runs SDPA, and the
// fused split-K Turbo4 verify kernel (crates/mlx-cpp/turbo/turbo4_attention.cpp:
// 45-264, partial + merge). Semantics follow MLX's SDPA on the dequantized
// cache (scores f16(q' . k), fp32 softmax, bottom-right causal).
//
// Design (one pass over the packed cache, HBM-bound):
//   grid (chunks, kv_heads), 4 waves a workgroup. The keys of a KV head are
//   cut into 32-key sub-chunks; a workgroup owns a contiguous run of them and
//   its waves take every 4th. A wave issues the loads of all its sub-chunks
//   (K codes, K scale/bias, V codes, V scale/bias) before any math, so the
//   whole per-CU share of the cache is in flight at once.
//   Q.K^T: v_mfma_f32_16x16x32_f16 with A = dequantized K (16 keys x 32
//   dims, one packed 4-bit word or two 8-bit words a lane, dequantized in
//   registers with the fp16 magic-number trick and one v_pk_fma a pair) and
//   B = the G*n_rows query rows of the KV group (GQA: each K row is fetched
//   and dequantized once for all heads of its group).
//   All of a wave's scores are formed before the softmax, so the wave knows
//   its row max up front: no running-max rescale of the accumulators.
//   P.V: the same MFMA with A = P (rows x 32 keys, fp16) and B = V straight
//   out of the 8-key-block V plane (one 128-bit load = 8 keys x 4 dims).
//   The 4 waves merge through LDS; each workgroup writes one fp32 partial
//   (m, l, unnormalized O); a small merge kernel combines the partials.
#include <algorithm>
#include <type_traits>

#include "dequant.hpp"
#include "kv_cache.hpp"

namespace qw {

struct DecodeArgs {
    const uint32_t* k_data;
    const uint32_t* k_params;
    const uint32_t* v_data;
    const uint32_t* v_params;
    const f16* q;      // [hq][Tq][D]
    float* part_o;     // [hkv][nc][16][D]
    float2* part_ml;   // [hkv][nc][16]
    int cap, T, Tq, G, R, causal, n_sub, nc;
    float scale_h;     // f16(scale) as float
};

template <int BITS, int D>
struct DecodeShape {
    static constexpr int NM = D / 32;  // QK MFMAs per 16-key tile
    static constexpr int DPL = D / 16;  // P.V MFMAs (dims per lane)
    static constexpr int NG = D / 64;   // affine groups a row
    // 128-bit loads a lane issues per 16-key K tile and per 8-key V block.
    static constexpr int KL = BITS == 16 ? NM : (D * BITS / 32) / 16;
    static constexpr int VL = (D * BITS / 4) / 64;
};

template <int BITS, int D, int NSUB>
__global__ __launch_bounds__(256, 1) void attend_decode_kernel(DecodeArgs a) {
    using S = DecodeShape<BITS, D>;
    constexpr int NM = S::NM, DPL = S::DPL, NG = S::NG, KL = S::KL, VL = S::VL;
    constexpr bool AFF = BITS != 16;
    const int c = blockIdx.x, h = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, g = lane >> 4;
    const int s_begin = (int)((int64_t)a.n_sub * c / a.nc);
    const int s_end = (int)((int64_t)a.n_sub * (c + 1) / a.nc);

    // ---- issue every load of this wave's sub-chunks
    u32x4 kc[NSUB][2][KL];
    u32x4 kp[NSUB][2];
    u32x4 vc[NSUB][VL];
    u32x4 vp[NSUB][2];
    const int64_t krow_words = (int64_t)D * BITS / 32;
    const int64_t vblk_words = (int64_t)D * BITS / 4;
#pragma unroll
    for (int j = 0; j < NSUB; j++) {
        const int s = s_begin + wave + 4 * j;
        if (s < s_end) {
#pragma unroll
            for (int tile = 0; tile < 2; tile++) {
                const int key = 32 * s + 8 * (r16 >> 2) + 4 * tile + (r16 & 3);
                const int64_t row = (int64_t)h * a.cap + key;
                const u32x4* src = (const u32x4*)(a.k_data + row * krow_words);
#pragma unroll
                for (int cc = 0; cc < KL; cc++) kc[j][tile][cc] = src[4 * cc + g];
                if constexpr (AFF) {
                    if constexpr (NG == 4)
                        kp[j][tile] = *(const u32x4*)(a.k_params + row * NG);
                    else {
                        const u32x2 t2 = *(const u32x2*)(a.k_params + row * NG);
                        kp[j][tile] = u32x4{t2.x, t2.y, 0u, 0u};
                    }
                }
            }
            const int64_t blk = (int64_t)h * (a.cap / 8) + 4 * s + g;
            const u32x4* vsrc = (const u32x4*)(a.v_data + blk * vblk_words);
#pragma unroll
            for (int jj = 0; jj < VL; jj++) vc[j][jj] = vsrc[16 * jj + r16];
            if constexpr (AFF) {
                const int grp = (r16 * DPL) / 64;
                const u32x4* psrc = (const u32x4*)(a.v_params + (blk * NG + grp) * 8);
                vp[j][0] = psrc[0];
                vp[j][1] = psrc[1];
            }
        }
    }

    // ---- Q rows of this KV group as the B operand (col = query row r16)
    const int rho = r16;
    const bool row_ok = rho < a.R;
    half8 qop[NM];
    {
        const int qh = h * a.G + (row_ok ? rho % a.G : 0);
        const int qr = row_ok ? rho / a.G : 0;
        const f16* qrow = a.q + ((int64_t)qh * a.Tq + qr) * D;
        const float sc = a.scale_h;
#pragma unroll
        for (int m = 0; m < NM; m++) {
            int base;
            if constexpr (BITS == 4)
                base = 8 * (16 * (m / 4) + 4 * g + (m % 4));
            else if constexpr (BITS == 8)
                base = 4 * (16 * (m / 2) + 4 * g + 2 * (m % 2));
            else
                base = 32 * m + 8 * g;
            half8 x = row_ok ? *(const half8*)(qrow + base) : half8{};
            half8 y;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                // 4-bit K pairs come out as dims (0,4),(1,5),(2,6),(3,7).
                const int src = BITS == 4 ? ((e >> 1) + 4 * (e & 1)) : e;
                y[e] = (f16)(sc * (float)x[src]);
            }
            qop[m] = y;
        }
    }

    // ---- scores (S^T: lane holds keys 8g+i (tile 0) / 8g+4+i (tile 1) of column r16)
    float sc[NSUB][8];
    const int lim = a.causal ? a.T - a.Tq + (row_ok ? rho / a.G : 0) : a.T - 1;
    // One 16-key tile of Q.K^T; FAST selects the 2-op dequant (dequant.hpp).
    auto qk_tile = [&](auto fast_tag, int j, int tile) -> float4v {
        constexpr bool FAST = decltype(fast_tag)::value;
        float4v acc = {0.f, 0.f, 0.f, 0.f};
        if constexpr (BITS == 4) {
            // load cc covers words 16cc + 4g .. +3, all in group 2cc + g/2
            PairConsts pc[KL];
#pragma unroll
            for (int cc = 0; cc < KL; cc++) {
                const uint32_t raw = (g & 2) ? kp[j][tile][2 * cc + 1] : kp[j][tile][2 * cc];
                const half2v sb = h2(raw);
                const half2v s1 = {sb.x, sb.x}, b1 = {sb.y, sb.y};
                pc[cc] = make_consts<FAST, 4>(s1, s1, s1, s1, b1, b1, b1, b1);
            }
#pragma unroll
            for (int m = 0; m < NM; m++)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    deq4<FAST>(kc[j][tile][m / 4][m % 4], pc[m / 4]), qop[m], acc, 0, 0, 0);
        } else if constexpr (BITS == 8) {
            PairConsts pc[NG];
#pragma unroll
            for (int gi = 0; gi < NG; gi++) {
                const half2v sb = h2(kp[j][tile][gi]);
                const half2v s1 = {sb.x, sb.x}, b1 = {sb.y, sb.y};
                pc[gi] = make_consts<FAST, 8>(s1, s1, s1, s1, b1, b1, b1, b1);
            }
#pragma unroll
            for (int m = 0; m < NM; m++)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    deq8<FAST>(kc[j][tile][m / 2][2 * (m % 2)], kc[j][tile][m / 2][2 * (m % 2) + 1],
                               pc[m / 2]),
                    qop[m], acc, 0, 0, 0);
        } else {
#pragma unroll
            for (int m = 0; m < NM; m++)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(kc[j][tile][m]), qop[m], acc,
                                                             0, 0, 0);
        }
        return acc;
    };
#pragma unroll
    for (int j = 0; j < NSUB; j++) {
        const int s = s_begin + wave + 4 * j;
        bool fast = true;
        if constexpr (AFF) {
            // The FAST dequant needs every scale of this sub-chunk in range.
            const uint32_t lo = BITS == 4 ? kFast4Lo : kFast8Lo;
            bool ok = true;
#pragma unroll
            for (int tile = 0; tile < 2; tile++)
#pragma unroll
                for (int gi = 0; gi < NG; gi++)
                    ok = ok && scale_in_range(kp[j][tile][gi], lo, kFastHi);
            fast = !__any(!ok);
        }
#pragma unroll
        for (int tile = 0; tile < 2; tile++) {
            float4v acc = {0.f, 0.f, 0.f, 0.f};
            if (s < s_end)
                acc = fast ? qk_tile(std::true_type{}, j, tile) : qk_tile(std::false_type{}, j, tile);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = 32 * s + 8 * g + 4 * tile + i;
                const bool ok = row_ok && s < s_end && key <= lim;
                // MLX rounds the score matrix to fp16 before the softmax.
                sc[j][4 * tile + i] = ok ? (float)(f16)acc[i] : -INFINITY;
            }
        }
    }

    // ---- row max over this wave's keys (column r16 lives in lanes r16 + 16g)
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NSUB; j++)
#pragma unroll
        for (int e = 0; e < 8; e++) mx = fmaxf(mx, sc[j][e]);
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mref = mx == -INFINITY ? 0.0f : mx;
    const float mref2 = mref * kLog2e;

    // ---- P and P.V
    float lsum = 0.0f;
    float4v acc_o[DPL];
#pragma unroll
    for (int mm = 0; mm < DPL; mm++) acc_o[mm] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NSUB; j++) {
        const int s = s_begin + wave + 4 * j;
        if (s >= s_end) continue;
        half8 pop;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][e], kLog2e, -mref2));
            lsum += p;
            pop[e] = (f16)p;
        }
        auto pv = [&](auto fast_tag) {
            constexpr bool FAST = decltype(fast_tag)::value;
            PairConsts pc;
            if constexpr (AFF)
                pc = make_consts<FAST, BITS>(h2(vp[j][0][0]), h2(vp[j][0][1]), h2(vp[j][0][2]),
                                             h2(vp[j][0][3]), h2(vp[j][1][0]), h2(vp[j][1][1]),
                                             h2(vp[j][1][2]), h2(vp[j][1][3]));
#pragma unroll
            for (int mm = 0; mm < DPL; mm++) {
                half8 bv;
                if constexpr (BITS == 4)
                    bv = deq4<FAST>(vc[j][mm / 4][mm % 4], pc);
                else if constexpr (BITS == 8)
                    bv = deq8<FAST>(vc[j][mm / 2][2 * (mm % 2)], vc[j][mm / 2][2 * (mm % 2) + 1], pc);
                else
                    bv = as_h8(vc[j][mm]);
                acc_o[mm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pop, bv, acc_o[mm], 0, 0, 0);
            }
        };
        bool fast = true;
        if constexpr (AFF) {
            const uint32_t lo = BITS == 4 ? kFast4Lo : kFast8Lo;
            bool ok = true;
#pragma unroll
            for (int i = 0; i < 4; i++) ok = ok && scales_in_range(vp[j][0][i], lo, kFastHi);
            fast = !__any(!ok);
        }
        if (fast)
            pv(std::true_type{});
        else
            pv(std::false_type{});
    }
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);

    // ---- merge the 4 waves through LDS
    __shared__ float2 sm_ml[4][16];
    __shared__ float4v sm_o[2][16][D / 4];
    if (g == 0) sm_ml[wave][r16] = float2{mx, lsum};
    __syncthreads();
    float fac[4];  // this wave's rescale for its O rows 4g+i
    float Mrow[4], Lrow[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = 4 * g + i;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++) M = fmaxf(M, sm_ml[w][row].x);
        float L = 0.0f, own = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float mw = sm_ml[w][row].x;
            const float f = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((mw - M) * kLog2e);
            L += f * sm_ml[w][row].y;
            if (w == wave) own = f;
        }
        fac[i] = own;
        Mrow[i] = M;
        Lrow[i] = L;
    }
#pragma unroll
    for (int mm = 0; mm < DPL; mm++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc_o[mm][i] *= fac[i];
    // O element (row 4g+i, dim r16*DPL + mm); LDS row-major by dim.
    auto store_o = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = 4 * g + i;
            if (row >= a.R) continue;
#pragma unroll
            for (int q4 = 0; q4 < DPL / 4; q4++)
                sm_o[buf][row][(r16 * DPL) / 4 + q4] =
                    float4v{acc_o[4 * q4][i], acc_o[4 * q4 + 1][i], acc_o[4 * q4 + 2][i],
                            acc_o[4 * q4 + 3][i]};
        }
    };
    auto add_o = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = 4 * g + i;
            if (row >= a.R) continue;
#pragma unroll
            for (int q4 = 0; q4 < DPL / 4; q4++) {
                const float4v t = sm_o[buf][row][(r16 * DPL) / 4 + q4];
                acc_o[4 * q4][i] += t[0];
                acc_o[4 * q4 + 1][i] += t[1];
                acc_o[4 * q4 + 2][i] += t[2];
                acc_o[4 * q4 + 3][i] += t[3];
            }
        }
    };
    if (wave >= 2) store_o(wave - 2);
    __syncthreads();
    if (wave < 2) add_o(wave);
    __syncthreads();
    if (wave == 1) store_o(0);
    __syncthreads();
    if (wave == 0) {
        add_o(0);
        const int64_t pbase = ((int64_t)h * a.nc + c) * 16;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = 4 * g + i;
            if (row >= a.R) continue;
            float4v* dst = (float4v*)(a.part_o + (pbase + row) * D + r16 * DPL);
#pragma unroll
            for (int q4 = 0; q4 < DPL / 4; q4++)
                dst[q4] = float4v{acc_o[4 * q4][i], acc_o[4 * q4 + 1][i], acc_o[4 * q4 + 2][i],
                                  acc_o[4 * q4 + 3][i]};
            if (r16 == 0) a.part_ml[pbase + row] = float2{Mrow[i], Lrow[i]};
        }
    }
}

// Combines the per-workgroup partials of one query row: out = sum_c e^(m_c - M)
// O_c / sum_c e^(m_c - M) l_c, rounded to fp16 (a row with no visible key is 0).
__global__ __launch_bounds__(256) void decode_merge_kernel(const float* __restrict__ part_o,
                                                           const float2* __restrict__ part_ml,
                                                           int nc, int D, int R, int G, int Tq,
                                                           f16* __restrict__ out) {
    const int row = blockIdx.x, h = blockIdx.y;
    const int64_t base = (int64_t)h * nc * 16 + row;
    float M = -INFINITY;
    for (int c = 0; c < nc; c++) M = fmaxf(M, part_ml[base + (int64_t)c * 16].x);
    const int qh = h * G + row % G, qr = row / G;
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float L = 0.0f, O = 0.0f;
#pragma unroll 8
        for (int c = 0; c < nc; c++) {
            const float2 ml = part_ml[base + (int64_t)c * 16];
            const float f = ml.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((ml.x - M) * kLog2e);
            L += f * ml.y;
            O += f * part_o[(base + (int64_t)c * 16) * D + d];
        }
        out[((int64_t)qh * Tq + qr) * D + d] = (f16)(L > 0.0f ? O / L : 0.0f);
    }
}

template <int BITS, int D>
static int launch_decode_bits(KVCache& cc, const f16* q, int G, int Tq, float scale,
                              bool causal, f16* out, hipStream_t stream) {
    const int T = cc.offset;
    const int n_sub = (T + 31) / 32;
    // Sub-chunks a wave owns: 4-bit rows are small enough to keep 4 in flight.
    constexpr int NSUB = BITS == 4 ? 4 : (BITS == 8 ? 2 : 1);
    const int nc = std::max(1, (n_sub + 4 * NSUB - 1) / (4 * NSUB));
    const size_t need = (size_t)cc.hkv * nc * 16 * D * sizeof(float) +
                        (size_t)cc.hkv * nc * 16 * sizeof(float2);
    int rc = cc.ensure_workspace(need);
    if (rc) return rc;
    DecodeArgs a;
    a.k_data = (const uint32_t*)cc.k_data;
    a.k_params = cc.k_params;
    a.v_data = (const uint32_t*)cc.v_data;
    a.v_params = cc.v_params;
    a.q = q;
    a.part_o = (float*)cc.ws;
    a.part_ml = (float2*)((char*)cc.ws + (size_t)cc.hkv * nc * 16 * D * sizeof(float));
    a.cap = cc.cap;
    a.T = T;
    a.Tq = Tq;
    a.G = G;
    a.R = G * Tq;
    a.causal = causal ? 1 : 0;
    a.n_sub = n_sub;
    a.nc = nc;
    a.scale_h = (float)(f16)scale;
    hipLaunchKernelGGL((attend_decode_kernel<BITS, D, NSUB>), dim3(nc, cc.hkv), dim3(256), 0,
                       stream, a);
    QW_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(decode_merge_kernel, dim3(a.R, cc.hkv), dim3(D), 0, stream, a.part_o,
                       a.part_ml, nc, D, a.R, G, Tq, out);
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

int launch_attention(KVCache& cc, const void* q, int n_q_heads, int n_rows, float scale,
                     bool causal, void* out, hipStream_t stream) {
    QW_REQUIRE(q && out, QW_ERR_INVALID_ARGUMENT, "attention: null q/out");
    QW_REQUIRE(n_q_heads > 0 && n_q_heads % cc.hkv == 0, QW_ERR_INVALID_ARGUMENT,
               "attention: n_q_heads must be a positive multiple of n_kv_heads");
    QW_REQUIRE(n_rows > 0, QW_ERR_INVALID_ARGUMENT, "attention: n_rows must be > 0");
    QW_REQUIRE(cc.offset >= n_rows, QW_ERR_INVALID_ARGUMENT,
               "attention: fewer cached keys than query rows");
    const int G = n_q_heads / cc.hkv;
    QW_REQUIRE(G * n_rows <= 16, QW_ERR_UNSUPPORTED,
               "attention: more than 16 query rows per KV head not yet supported");
    DeviceGuard dg(cc.device);
    const f16* qq = (const f16*)q;
    f16* oo = (f16*)out;
    if (cc.D == 256) {
        if (cc.bits == 4) return launch_decode_bits<4, 256>(cc, qq, G, n_rows, scale, causal, oo, stream);
        if (cc.bits == 8) return launch_decode_bits<8, 256>(cc, qq, G, n_rows, scale, causal, oo, stream);
        return launch_decode_bits<16, 256>(cc, qq, G, n_rows, scale, causal, oo, stream);
    }
    if (cc.bits == 4) return launch_decode_bits<4, 128>(cc, qq, G, n_rows, scale, causal, oo, stream);
    if (cc.bits == 8) return launch_decode_bits<8, 128>(cc, qq, G, n_rows, scale, causal, oo, stream);
    return launch_decode_bits<16, 128>(cc, qq, G, n_rows, scale, causal, oo, stream);
}

int KVCache::attention(const void* q, int n_q_heads, int n_rows, float scale, bool causal,
                       void* out, hipStream_t stream) {
    return launch_attention(*this, q, n_q_heads, n_rows, scale, causal, out, stream);
}

int KVCache::update_and_attention(const void* q, int n_q_heads, int n_rows, const void* k_new,
                                  const void* v_new, float scale, bool causal, void* out,
                                  hipStream_t stream) {
    QW_REQUIRE(q && out && k_new && v_new, QW_ERR_INVALID_ARGUMENT,
               "update_and_attention: null pointer");
    QW_REQUIRE(n_q_heads > 0 && n_q_heads % hkv == 0 && n_rows > 0, QW_ERR_INVALID_ARGUMENT,
               "update_and_attention: bad head or row geometry");
    QW_REQUIRE((n_q_heads / hkv) * n_rows <= 16, QW_ERR_UNSUPPORTED,
               "update_and_attention: more than 16 query rows per KV head not yet supported");
    int rc = update(k_new, v_new, n_rows, stream);
    if (rc) return rc;
    return launch_attention(*this, q, n_q_heads, n_rows, scale, causal, out, stream);
}

}  // namespace qw
