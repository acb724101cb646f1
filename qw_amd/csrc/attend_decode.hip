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
    const int* fast_flag;  // != 0: all cached scales in the FAST dequant range
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

// Waves of a workgroup; one workgroup a CU, so NW/4 waves a SIMD. A wave
// holds one sub-chunk's loads at a time and latency is hidden by the other
// waves of its SIMD: 12 waves (3 a SIMD, <= 168 registers each) where one
// stage fits that budget, 8 (2 a SIMD) for the larger 8-bit / fp16 stages.
#ifndef QW_DECODE_WAVES_4BIT
#define QW_DECODE_WAVES_4BIT 8
#endif
template <int BITS, int D>
constexpr int decode_waves() {
    return D == 128 ? 12 : (BITS == 4 ? QW_DECODE_WAVES_4BIT : 8);
}

// Register stages a wave streams through (1: load the next sub-chunk after
// the current one's math; 2: ping-pong, two sub-chunks in flight). Two fit
// the register budget only for the small 4-bit stages.
#ifndef QW_DECODE_STAGES_4BIT
#define QW_DECODE_STAGES_4BIT 1
#endif
template <int BITS>
constexpr int decode_stages() {
    return BITS == 4 ? QW_DECODE_STAGES_4BIT : 1;
}

// FAST: every scale in the cache is inside the 2-op dequant's exact range
// (the cache's fast_flag, maintained by the append and import kernels).
template <int BITS, int D, int NW, bool FAST>
__device__ __forceinline__ void decode_body(const DecodeArgs& a, float2 (*sm_ml)[16],
                                            float* sm_o, half8 (*sm_q)[64]) {
    using S = DecodeShape<BITS, D>;
    constexpr int NM = S::NM, DPL = S::DPL, NG = S::NG, KL = S::KL, VL = S::VL;
    constexpr bool AFF = BITS != 16;
    const int c = blockIdx.x, h = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, g = lane >> 4;
    const int s_begin = (int)((uint32_t)a.n_sub * (uint32_t)c / (uint32_t)a.nc);
    const int s_end = (int)((uint32_t)a.n_sub * (uint32_t)(c + 1) / (uint32_t)a.nc);
    const uint32_t magic = vconst(kMagic);

    // One 32-key sub-chunk's loads; a wave walks its sub-chunks
    // s_begin + wave + NW*k through one of these.
    struct Stage {
        u32x4 kc[2][KL];  // K codes of tiles 0/1 (16 keys each)
        u32x4 kp[2];      // K (scale, bias) of the lane's key, tiles 0/1 (4-bit: the
                          // lane's groups g/2 and 2+g/2 in .x/.y)
        u32x4 vc[VL];     // V block of keys 8g..8g+7, the lane's DPL dims
        u32x4 vp[2];      // V scales / biases of that block and dim group
    };
    const int64_t krow_words = (int64_t)D * BITS / 32;
    const int64_t vblk_words = (int64_t)D * BITS / 4;
    auto load = [&](Stage& st, int s) {
#pragma unroll
        for (int tile = 0; tile < 2; tile++) {
            const int key = 32 * s + 8 * (r16 >> 2) + 4 * tile + (r16 & 3);
            const int64_t row = (int64_t)h * a.cap + key;
            const u32x4* src = (const u32x4*)(a.k_data + row * krow_words);
#pragma unroll
            for (int cc = 0; cc < KL; cc++) st.kc[tile][cc] = src[4 * cc + g];
            if constexpr (BITS == 4 && NG == 4) {
                // groups g/2 and 2 + g/2 sit in slots 2(g/2), 2(g/2)+1 (k_param_slot)
                const u32x2 t2 = *(const u32x2*)(a.k_params + row * NG + 2 * (g >> 1));
                st.kp[tile] = u32x4{t2.x, t2.y, 0u, 0u};
            } else if constexpr (BITS == 4) {
                st.kp[tile] = u32x4{a.k_params[row * NG + (g >> 1)], 0u, 0u, 0u};
            } else if constexpr (AFF) {
                if constexpr (NG == 4)
                    st.kp[tile] = *(const u32x4*)(a.k_params + row * NG);
                else {
                    const u32x2 t2 = *(const u32x2*)(a.k_params + row * NG);
                    st.kp[tile] = u32x4{t2.x, t2.y, 0u, 0u};
                }
            }
        }
        const int64_t blk = (int64_t)h * (a.cap / 8) + 4 * s + g;
        const u32x4* vsrc = (const u32x4*)(a.v_data + blk * vblk_words);
#pragma unroll
        for (int jj = 0; jj < VL; jj++) st.vc[jj] = vsrc[16 * jj + r16];
        if constexpr (AFF) {
            const int grp = (r16 * DPL) / 64;
            const u32x4* psrc = (const u32x4*)(a.v_params + (blk * NG + grp) * 8);
            st.vp[0] = psrc[0];
            st.vp[1] = psrc[1];
        }
    };

    // ---- Q rows of this KV group as the B operand (col = query row r16).
    // The workgroup's waves share one KV head, so the operand is built once
    // into LDS (wave w converts MFMA slice w) and each QK MFMA reads its slice
    // back with one ds_read_b128. Padding rows are zero.
    const int rho = r16;
    const bool row_ok = rho < a.R;
    static_assert(NW >= NM, "one Q slice per wave");
    half8 x[1];
    {
        const int rr = row_ok ? rho : 0;
        const f16* qrow = a.q + ((int64_t)(h * a.G + rr % a.G) * a.Tq + rr / a.G) * D;
#pragma unroll
        for (int i = 0; i < 1; i++) {
            const int m = wave % NM;
            int base;
            if constexpr (BITS == 4)
                base = 8 * (16 * (m / 4) + 4 * g + (m % 4));
            else if constexpr (BITS == 8)
                base = 4 * (16 * (m / 2) + 4 * g + 2 * (m % 2));
            else
                base = 32 * m + 8 * g;
            x[i] = *(const half8*)(qrow + base);
        }
    }
    // The first sub-chunk's loads go out right behind Q (loads return in
    // issue order, so the Q conversion below waits for Q only).
    int s = s_begin + wave;
    Stage A, B;
    if (s < s_end) load(A, s);
    // Second stage in flight from the start: a wave's first two sub-chunks
    // stream in while the first is being computed.
    if constexpr (decode_stages<BITS>() == 2)
        if (s + NW < s_end) load(B, s + NW);
    {
        // q' = f16(f16(scale) * q): one packed fp16 multiply rounds exactly
        // like MLX's fp16 `multiply`. Padding rows get scale 0.
        const f16 sc = row_ok ? (f16)a.scale_h : (f16)0.0f;
        const half2v sc2 = {sc, sc};
        if (wave < NM) {
            const int m = wave;
            const u32x4 w = __builtin_bit_cast(u32x4, x[0]);
            u32x4 o;
            if constexpr (BITS == 4) {
                // 4-bit K pairs come out as dims (0,4),(1,5),(2,6),(3,7).
                o.x = __builtin_amdgcn_perm(w.z, w.x, 0x05040100u);
                o.y = __builtin_amdgcn_perm(w.z, w.x, 0x07060302u);
                o.z = __builtin_amdgcn_perm(w.w, w.y, 0x05040100u);
                o.w = __builtin_amdgcn_perm(w.w, w.y, 0x07060302u);
            } else {
                o = w;
            }
            u32x4 y;
            y.x = __builtin_bit_cast(uint32_t, h2(o.x) * sc2);
            y.y = __builtin_bit_cast(uint32_t, h2(o.y) * sc2);
            y.z = __builtin_bit_cast(uint32_t, h2(o.z) * sc2);
            y.w = __builtin_bit_cast(uint32_t, h2(o.w) * sc2);
            sm_q[m][lane] = __builtin_bit_cast(half8, y);
        }
    }
    __syncthreads();
    const int lim = a.causal ? a.T - a.Tq + (row_ok ? rho / a.G : 0) : a.T - 1;

    float m_run = -INFINITY;  // softmax reference of row r16 (natural units)
    float l_run = 0.0f;       // this lane's share of the row sum
    float4v acc_o[DPL];
#pragma unroll
    for (int mm = 0; mm < DPL; mm++) acc_o[mm] = float4v{0.f, 0.f, 0.f, 0.f};

    // Q.K^T of the two 16-key tiles (S^T: lane holds keys 8g+i / 8g+4+i of
    // column r16); the two MFMA chains interleave to hide each other's latency.
    auto qk = [&](const Stage& st, float4v& acc0, float4v& acc1) {
        acc0 = float4v{0.f, 0.f, 0.f, 0.f};
        acc1 = float4v{0.f, 0.f, 0.f, 0.f};
        if constexpr (BITS == 4) {
            // load cc covers words 16cc + 4g .. +3, all in group 2cc + g/2
#pragma unroll
            for (int cc = 0; cc < KL; cc++) {
                const half2v sb0 = h2(st.kp[0][cc]), sb1 = h2(st.kp[1][cc]);
                const half2v s0 = {sb0.x, sb0.x}, b0 = {sb0.y, sb0.y};
                const half2v s1 = {sb1.x, sb1.x}, b1 = {sb1.y, sb1.y};
                const PairConsts p0 = make_consts<FAST, 4>(s0, s0, s0, s0, b0, b0, b0, b0);
                const PairConsts p1 = make_consts<FAST, 4>(s1, s1, s1, s1, b1, b1, b1, b1);
#pragma unroll
                for (int mi = 0; mi < 4; mi++) {
                    const int m = 4 * cc + mi;
                    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        deq4<FAST>(st.kc[0][cc][mi], p0, magic), sm_q[m][lane], acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        deq4<FAST>(st.kc[1][cc][mi], p1, magic), sm_q[m][lane], acc1, 0, 0, 0);
                }
            }
        } else if constexpr (BITS == 8) {
#pragma unroll
            for (int m = 0; m < NM; m++) {
                const int slot = k_param_slot(m / 2, NG);
                const half2v sb0 = h2(st.kp[0][slot]), sb1 = h2(st.kp[1][slot]);
                const half2v s0 = {sb0.x, sb0.x}, b0 = {sb0.y, sb0.y};
                const half2v s1 = {sb1.x, sb1.x}, b1 = {sb1.y, sb1.y};
                const PairConsts p0 = make_consts<FAST, 8>(s0, s0, s0, s0, b0, b0, b0, b0);
                const PairConsts p1 = make_consts<FAST, 8>(s1, s1, s1, s1, b1, b1, b1, b1);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    deq8<FAST>(st.kc[0][m / 2][2 * (m % 2)], st.kc[0][m / 2][2 * (m % 2) + 1], p0),
                    sm_q[m][lane], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    deq8<FAST>(st.kc[1][m / 2][2 * (m % 2)], st.kc[1][m / 2][2 * (m % 2) + 1], p1),
                    sm_q[m][lane], acc1, 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int m = 0; m < NM; m++) {
                acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(st.kc[0][m]), sm_q[m][lane], acc0, 0,
                                                              0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(st.kc[1][m]), sm_q[m][lane], acc1, 0,
                                                              0, 0);
            }
        }
    };
    auto pv = [&](const Stage& st, const half8& pop) {
        PairConsts pc;
        if constexpr (AFF)
            pc = make_consts<FAST, BITS>(h2(st.vp[0][0]), h2(st.vp[0][1]), h2(st.vp[0][2]),
                                         h2(st.vp[0][3]), h2(st.vp[1][0]), h2(st.vp[1][1]),
                                         h2(st.vp[1][2]), h2(st.vp[1][3]));
#pragma unroll
        for (int mm = 0; mm < DPL; mm++) {
            half8 bv;
            if constexpr (BITS == 4)
                bv = deq4<FAST>(st.vc[mm / 4][mm % 4], pc, magic);
            else if constexpr (BITS == 8)
                bv = deq8<FAST>(st.vc[mm / 2][2 * (mm % 2)], st.vc[mm / 2][2 * (mm % 2) + 1], pc);
            else
                bv = as_h8(st.vc[mm]);
            acc_o[mm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pop, bv, acc_o[mm], 0, 0, 0);
        }
    };

    auto compute = [&](const Stage& st, int s) {
        // ---- scores
        float4v acc0, acc1;
        qk(st, acc0, acc1);
        float sc[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int k0 = 32 * s + 8 * g + i, k1 = k0 + 4;
            // MLX rounds the score matrix to fp16 before the softmax.
            sc[i] = row_ok && k0 <= lim ? (float)(f16)acc0[i] : -INFINITY;
            sc[4 + i] = row_ok && k1 <= lim ? (float)(f16)acc1[i] : -INFINITY;
        }
        // ---- online softmax with a lazy reference: the row reference m_run
        // only moves when a score exceeds it by more than 5.5 (p <= e^5.5 fits
        // fp16 easily), so the accumulators are rarely rescaled.
        float mx = sc[0];
#pragma unroll
        for (int e = 1; e < 8; e++) mx = fmaxf(mx, sc[e]);
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        if (__any(mx > m_run + 5.5f)) {
            const float m_new = fmaxf(m_run, mx);
            if (__any(m_run != -INFINITY)) {
                const float alpha =
                    m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m_run - m_new) * kLog2e);
                l_run *= alpha;
                float f[4];
#pragma unroll
                for (int i = 0; i < 4; i++) f[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
                for (int mm = 0; mm < DPL; mm++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc_o[mm][i] *= f[i];
            }
            m_run = m_new;
        }
        const float mref2 = (m_run == -INFINITY ? 0.0f : m_run) * kLog2e;
        half8 pop;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[e], kLog2e, -mref2));
            l_run += p;
            pop[e] = (f16)p;
        }
        // ---- P.V
        pv(st, pop);
    };

    if constexpr (decode_stages<BITS>() == 2) {
        // Ping-pong: a stage is refilled right after its math, so one stage's
        // loads are always in flight behind the other's compute.
        for (; s < s_end; s += 2 * NW) {
            compute(A, s);
            __builtin_amdgcn_sched_barrier(0);
            if (s + 2 * NW < s_end) load(A, s + 2 * NW);
            if (s + NW >= s_end) break;
            compute(B, s + NW);
            __builtin_amdgcn_sched_barrier(0);
            if (s + 3 * NW < s_end) load(B, s + 3 * NW);
        }
    } else {
        for (; s < s_end; s += NW) {
            compute(A, s);
            // keep the next sub-chunk's loads behind this one's math
            __builtin_amdgcn_sched_barrier(0);
            if (s + NW < s_end) load(A, s + NW);
        }
    }
    float lsum = l_run;
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    const float mx = m_run;

    // ---- merge the NW waves: each wave parks its accumulators (rows < R) in
    // LDS once, then all threads form out[row][d] = sum_w f_w O_w[row][d] with
    // f_w = e^(m_w - M), M the row max over waves, and write the partial.
    if (g == 0) sm_ml[wave][r16] = float2{mx, lsum};
    const int R = a.R;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = 4 * g + i;
        if (row >= R) continue;
        float* dst = sm_o + ((int64_t)wave * R + row) * D + r16 * DPL;
#pragma unroll
        for (int q4 = 0; q4 < DPL / 4; q4++)
            *(float4v*)(dst + 4 * q4) = float4v{acc_o[4 * q4][i], acc_o[4 * q4 + 1][i],
                                                acc_o[4 * q4 + 2][i], acc_o[4 * q4 + 3][i]};
    }
    __syncthreads();
    const int64_t pbase = ((int64_t)h * a.nc + c) * 16;
    for (int o = threadIdx.x; o < R * D; o += 64 * NW) {
        const int row = o / D, d = o % D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, sm_ml[w][row].x);
        float acc = 0.0f, L = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float2 ml = sm_ml[w][row];
            const float f = ml.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((ml.x - M) * kLog2e);
            acc = __builtin_fmaf(f, sm_o[((int64_t)w * R + row) * D + d], acc);
            L = __builtin_fmaf(f, ml.y, L);
        }
        a.part_o[(pbase + row) * D + d] = acc;
        if (d == 0) a.part_ml[pbase + row] = float2{M, L};
    }
}

template <int BITS, int D>
__global__ __launch_bounds__((64 * decode_waves<BITS, D>()), 1) void attend_decode_kernel(
    DecodeArgs a) {
    constexpr int NW = decode_waves<BITS, D>();
    __shared__ float2 sm_ml[NW][16];
    __shared__ half8 sm_q[D / 32][64];
    extern __shared__ float sm_o[];  // [NW][R][D]
    // One uniform branch for the whole launch: the exact 2-op dequant when
    // every cached scale allows it, else the separately rounded path.
    if (BITS == 16 || *a.fast_flag != 0)
        decode_body<BITS, D, NW, true>(a, sm_ml, sm_o, sm_q);
    else
        decode_body<BITS, D, NW, false>(a, sm_ml, sm_o, sm_q);
}

// Combines the per-workgroup partials of one query row (partials of a KV head
// are [nc][rstride] rows, row index = r * G + head-in-group): out = sum_c e^(m_c - M)
// O_c / sum_c e^(m_c - M) l_c, rounded to fp16 (a row with no visible key is 0).
// grid (rows, kv_heads, D/64): a workgroup owns 64 dims of one row; lane =
// dim, wave w sums partials c = w, w+4, ... with every load issued up front.
constexpr int kMergeMaxPer = 64;  // partials a wave sums (nc <= 256)

__global__ __launch_bounds__(256) void decode_merge_kernel(const float* __restrict__ part_o,
                                                           const float2* __restrict__ part_ml,
                                                           int nc, int rstride, int D, int G,
                                                           int Tq, f16* __restrict__ out) {
    const int row = blockIdx.x, h = blockIdx.y, d = blockIdx.z * 64 + (threadIdx.x & 63);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t base = (int64_t)h * nc * rstride + row;
    // One memory round: every (m, l) and O value this lane needs is loaded
    // first; the max is then exchanged through LDS.
    float v[kMergeMaxPer];
    float2 ml[kMergeMaxPer];
#pragma unroll
    for (int i = 0; i < kMergeMaxPer; i++) {
        const int c = wave + 4 * i;
        if (c < nc) {
            ml[i] = part_ml[base + (int64_t)c * rstride];
            v[i] = part_o[(base + (int64_t)c * rstride) * D + d];
        } else {
            ml[i] = float2{-INFINITY, 0.0f};
            v[i] = 0.0f;
        }
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < kMergeMaxPer; i++) m = fmaxf(m, ml[i].x);
    __shared__ float sm_m[4];
    __shared__ float sm[2][4][64];
    if (lane == 0) sm_m[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(sm_m[0], sm_m[1]), fmaxf(sm_m[2], sm_m[3]));
    float o = 0.0f, l = 0.0f;
#pragma unroll
    for (int i = 0; i < kMergeMaxPer; i++) {
        const float w =
            ml[i].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((ml[i].x - m) * kLog2e);
        o = __builtin_fmaf(w, v[i], o);
        l = __builtin_fmaf(w, ml[i].y, l);
    }
    sm[0][wave][lane] = o;
    sm[1][wave][lane] = l;
    __syncthreads();
    if (wave == 0) {
        const float O = (sm[0][0][lane] + sm[0][1][lane]) + (sm[0][2][lane] + sm[0][3][lane]);
        const float L = (sm[1][0][lane] + sm[1][1][lane]) + (sm[1][2][lane] + sm[1][3][lane]);
        const int qh = h * G + row % G, qr = row / G;
        out[((int64_t)qh * Tq + qr) * D + d] = (f16)(L > 0.0f ? O / L : 0.0f);
    }
}

template <int BITS, int D>
static int launch_decode_bits(KVCache& cc, const f16* q, int G, int Tq, float scale,
                              bool causal, f16* out, hipStream_t stream) {
    const int T = cc.offset;
    const int n_sub = (T + 31) / 32;
    // Sub-chunks a wave owns: 4-bit rows are small enough to keep 4 in flight.
    // Sub-chunks a wave keeps in flight per round, and workgroups per KV head:
    // two 4-wave workgroups a CU (256 CUs), each wave one round when the
    // context allows, at most 1024 partials per head.
    // One workgroup a CU (256 CUs), at least a wave's worth of sub-chunks each.
    constexpr int NW = decode_waves<BITS, D>();
    const int per_head = std::max(1, 256 / cc.hkv);
    const int nc = std::max(1, std::min({per_head, (n_sub + NW - 1) / NW, 4 * kMergeMaxPer}));
    const size_t need = (size_t)cc.hkv * nc * 16 * D * sizeof(float) +
                        (size_t)cc.hkv * nc * 16 * sizeof(float2);
    int rc = cc.ensure_workspace(need);
    if (rc) return rc;
    DecodeArgs a;
    a.k_data = (const uint32_t*)cc.k_data;
    a.k_params = cc.k_params;
    a.v_data = (const uint32_t*)cc.v_data;
    a.v_params = cc.v_params;
    a.fast_flag = cc.fast_flag;
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
    const size_t shmem = (size_t)NW * a.R * D * sizeof(float);
    hipLaunchKernelGGL((attend_decode_kernel<BITS, D>), dim3(nc, cc.hkv), dim3(64 * NW), shmem,
                       stream, a);
    QW_HIP_CHECK(hipGetLastError());
    return launch_partial_merge(a.part_o, a.part_ml, nc, 16, a.R, cc.hkv, D, G, Tq, out, stream);
}

int launch_partial_merge(const float* part_o, const float2* part_ml, int nc, int rstride, int R,
                         int hkv, int D, int G, int Tq, f16* out, hipStream_t stream) {
    QW_REQUIRE(nc >= 1 && nc <= 4 * kMergeMaxPer, QW_ERR_INVALID_ARGUMENT,
               "merge: partial count out of range");
    hipLaunchKernelGGL(decode_merge_kernel, dim3(R, hkv, D / 64), dim3(256), 0, stream, part_o,
                       part_ml, nc, rstride, D, G, Tq, out);
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
    DeviceGuard dg(cc.device);
    QW_REQUIRE(dg.ok, QW_ERR_HIP, "attention: hipSetDevice failed");
    const f16* qq = (const f16*)q;
    f16* oo = (f16*)out;
    if (G * n_rows > 16) return launch_block_attention(cc, qq, G, n_rows, scale, causal, oo, stream);
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
    int rc = update(k_new, v_new, n_rows, stream);
    if (rc) return rc;
    return launch_attention(*this, q, n_q_heads, n_rows, scale, causal, out, stream);
}

}  // namespace qw
