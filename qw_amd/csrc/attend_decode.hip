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
//   grid (chunks, kv_heads), 8 waves a workgroup, one workgroup a CU. The
//   keys of a KV head are cut into 32-key sub-chunks dealt round-robin over
//   the head's waves (workgroup c, wave w takes c + nc * (w + 8k)).
//   Each sub-chunk's K half (codes + scale/bias) and V half are requested
//   with raw buffer loads once the previous half has landed, about one
//   sub-chunk a wave in flight.
//   Q.K^T: v_mfma_f32_16x16x32_f16 with A = K dequantized in registers
//   exactly as MLX does (fp16 magic-number conversion, v_pk_fma, v_pk_add)
//   and B = the G*n_rows query rows of the KV group from LDS (GQA: each K row
//   is fetched and dequantized once for all heads of its group).
//   fp16 score rounding, masking and an online softmax whose reference only
//   moves when a score exceeds it by 5.5, so the accumulators are rarely
//   rescaled.
//   P.V: the same MFMA with A = P (rows x 32 keys, fp16) and B = V straight
//   out of the 8-key-block V plane (one 128-bit load = 8 keys x 4 dims),
//   dequantized as f16(code * scale); the biases enter through one MFMA a
//   sub-chunk.
//   The 8 waves merge through LDS; each workgroup writes one fp32 partial
//   (m, l, unnormalized O); a merge kernel combines the partials (and, on the
//   decode-with-append path, quantizes and appends the new token).
#include <algorithm>
#include <type_traits>

#include "append.hpp"
#include "dequant.hpp"
#include "quant.hpp"
#include "kv_cache.hpp"
#include "turbo4_device.hpp"

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
    float inv_g;       // 1 / G
    uint32_t code_off2;  // magic offset pair of the separately rounded dequant
    const float* t4_tab;  // Turbo4 caches: the device tables (signs, centroids); else null
    // ns: workgroups that split the T cached keys (= nc, or nc - 1 with an
    // append unit). app_L > 0: workgroup (ns, h) is the append unit of head h:
    // it appends the app_L new rows read through app (keys T .. T + app_L - 1)
    // and writes their partial, slot ns, with the causal cut when app_causal.
    int ns, app_L, app_causal, app_int8;
    RowSrc app;
    // ROPE launches (RoPE, append and attention in one launch): q holds the
    // projection's unrotated rows, query row r of q head qh at
    // q + r * q_tok_stride + qh * D, rotated with app's RoPE fields at
    // position app.position0 + r (rope_dims a multiple of 16); the append
    // unit writes the rotated rows to q_out [hq][Tq][D].
    int64_t q_tok_stride;
    f16* q_out;
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
#ifndef QW_DECODE_QREG
#define QW_DECODE_QREG 1
#endif
#ifndef QW_DECODE_WAVES_4BIT
#define QW_DECODE_WAVES_4BIT 8
#endif
template <int BITS, int D>
constexpr int decode_waves() {
    return D == 128 ? 12 : (BITS == 4 ? QW_DECODE_WAVES_4BIT : 8);
}

// Word 3 of a raw buffer resource on gfx9-family parts (CDNA): 32-bit data
// format, no swizzle, no index stride.
constexpr int kBufWord3 = 0x00020000;

// Cache policy of the decode kernel's K/V loads (the instruction's sc0 / nt /
// sc1 bits: 1, 2, 16). Non-temporal (2) when a call reads at least
// QW_DECODE_NT_MIN_MB of cache: the streamed cache then leaves the L2 and the
// MALL to what is reused (code, arguments, q, partials); a whole layer stack
// of such calls cannot stay in the 256 MB MALL anyway. Smaller calls keep the
// default policy, so a stack of short caches can stay resident there. A/B in
// one run: config 2 (37.8 MB) 15.9 -> 15.3 us and Int8 at its geometry 21.5
// -> 20.7 us with nt; config 1 (8.9 MB, sixteen caches that fit the MALL)
// 11.4 us without against 12.4 us with.
#ifndef QW_DECODE_NT_MIN_MB
#define QW_DECODE_NT_MIN_MB 16
#endif

// Register stages a wave streams through (1: load the next sub-chunk after
// the current one's math; 2: wait-then-prefetch ping-pong, a stage's
// successor requested once the stage itself has landed). Two fit the register
// budget only for the small 4-bit stages.
template <int BITS>
constexpr int decode_stages() {
    return BITS == 4 ? 2 : 1;
}

// Turbo4: the 256-entry LDS table of centroid pairs (entry b = (centroid of
// the low nibble of b, centroid of its high nibble)) turns one byte of codes
// into two centroids with one 8-byte read (measured ~1.9x the throughput of a
// ds_bpermute per element); the expansion f16(centroid * rescale) rounds the
// product to fp32 first, as the expansion kernel forms it (t4_f16_product).
// 8 consecutive dims (the word's nibbles, LSB first) of one row
__device__ __forceinline__ half8 t4_expand8(uint32_t w, float r, const float2* pt) {
    half8 y;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float2 c = pt[(w >> (8 * k)) & 0xFFu];
        y[2 * k] = t4_f16_product(c.x, r);
        y[2 * k + 1] = t4_f16_product(c.y, r);
    }
    return y;
}

// FAST: every scale in the cache is inside the 2-op dequant's exact range
// (the cache's fast_flag, maintained by the append and import kernels).
//
// K is dequantized exactly as MLX does, f16(f16(code * scale) + bias): the
// scores are rounded to fp16 next, and a key value one rounding off would
// move those roundings. V is dequantized as f16(code * scale) only and the
// bias of each (key, 64-dim group) enters through one more MFMA,
// O_b += P * Vb with B = the biases of the lane's dim group for the 8 keys
// of its block, added to every dim of that group at the end (the bias is
// exact in fp32; only MLX's second rounding of each V element is skipped).
//
// T4 (Turbo4 caches, BITS = 4): K and V rows of D/2 bytes of 4-bit centroid
// indices, row-major, and one side word a row (K rescale in .x of the K side
// plane, V rescale in .y of the V side plane). Every element is formed as the
// fp16 expansion stores it, f16(centroid * rescale) with the product rounded
// to fp32 first, and the attention arithmetic is the fp16 cache's (MLX's SDPA
// on the expansion). Lane group g of a K tile reads dims (D/4) g .. +D/4 - 1 of
// its key (q is laid out to match); the P.V lane (g, r16) reads dims
// DPL r16 .. +DPL - 1 of keys 8g .. 8g+7 (16 lanes cover a row's D/2 bytes).
// The centroid comes from a register table (lane i holds centroid i % 16)
// through ds_bpermute.
template <int BITS, int D, int NW, bool FAST, bool T4 = false, int AUX = 0, bool ROPE = false>
__device__ __forceinline__ void decode_body(const DecodeArgs& a, float2 (*sm_ml)[NW], float* sm_o,
                                            half8 (*sm_q)[64], float2* sm_t4 = nullptr) {
    using S = DecodeShape<BITS, D>;
    constexpr int NM = S::NM, DPL = S::DPL, NG = S::NG, VL = S::VL;
    static_assert(!T4 || BITS == 4, "Turbo4 indices are 4-bit");
    constexpr bool AFF = BITS != 16 && !T4;
    constexpr int KL = T4 ? D / 128 : S::KL;  // 128-bit K loads a lane a tile
    const int c = blockIdx.x, h = blockIdx.y;
    // wave index as a scalar: sub-chunk indices, and so the buffer offsets
    // below, stay in SGPRs
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int r16 = lane & 15, g = lane >> 4;
    // Sub-chunks are dealt round-robin: workgroup c, wave w, round k owns
    // sub-chunk c + ns * (w + NW * k). At any moment the workgroups of a head
    // stream adjacent 4 KB blocks, spreading the reads over all HBM channels
    // (contiguous per-workgroup ranges put the 64 workgroups of a head on a
    // few channel phases at once).
    const int SS = a.ns * NW;  // stride between a wave's sub-chunks
    const int s_end = a.n_sub;
    const uint32_t magic = vconst(kMagic);
    float* const part_o = a.part_o;
    float2* const part_ml = a.part_ml;

    // One 32-key sub-chunk's loads; a wave walks its sub-chunks
    // c + ns * (wave + NW * k) through one of these.
    // T4: vc holds the DPL/2-byte row pieces of keys 8g..8g+7 (two keys a
    // u32x4 at D = 256, four at D = 128), vp the 8 keys' V side words, kp[t].x
    // the K side word of the lane's key.
    constexpr int VLS = T4 ? (D == 256 ? 4 : 2) : VL;
    struct Stage {
        u32x4 kc[2][KL];  // K codes of tiles 0/1 (16 keys each)
        u32x4 kp[2];      // K (scale, bias) of the lane's key, tiles 0/1 (4-bit: the
                          // lane's groups g/2 and 2+g/2 in .x/.y)
        u32x4 vc[VLS];    // V block of keys 8g..8g+7, the lane's DPL dims
        u32x4 vp[2];      // V scales / biases of that block and dim group
    };
    // Raw buffer loads over this KV head's rows of each plane: the lane's
    // byte offset is fixed for the whole kernel (VGPR), the sub-chunk's is a
    // scalar (SGPR), the parts of a stage differ by immediates. A stage past
    // the chunk's end gets num_records = 0, so its loads are issued
    // unconditionally but return zeros without touching memory.
    constexpr int KRB = D * BITS / 8;          // K row bytes
    constexpr int KPB = T4 ? 4 : AFF ? NG * 4 : 0;  // K param bytes a row
    constexpr int VBB = D * BITS;              // V block bytes (8 keys: D*BITS/4 words; T4: 8 rows)
    constexpr int VPB = T4 ? 32 : NG * 32;     // V param bytes a block (T4: 8 side words)
    const int64_t hrow = (int64_t)h * a.cap;
    const char* kbase = (const char*)a.k_data + hrow * KRB;
    const char* kpbase = (const char*)a.k_params + hrow * KPB;
    const char* vbase = (const char*)a.v_data + hrow / 8 * VBB;
    const char* vpbase = (const char*)a.v_params + hrow / 8 * VPB;
    const int kkey = 8 * (r16 >> 2) + (r16 & 3);  // the lane's K row in tile 0
    const int off_k = T4 ? kkey * KRB + (KRB / 4) * g : kkey * KRB + 16 * g;
    const int off_kp = T4                   ? kkey * KPB
                       : BITS == 4 && NG == 4 ? kkey * KPB + 8 * (g >> 1)
                       : BITS == 4          ? kkey * KPB + 4 * (g >> 1)
                                            : kkey * KPB;
    const int off_v = T4 ? g * VBB + (DPL / 2) * r16 : g * VBB + 16 * r16;
    const int off_vp = T4 ? g * VPB : (g * NG + (r16 * DPL) / 64) * 32;
    // K half of a stage (codes + params: 2*KL + 2 loads) and V half (VL + 2).
    auto load_k = [&](Stage& st, int s) {
        const bool ok = s < s_end;
        const int si = ok ? s : 0;
        const __amdgpu_buffer_rsrc_t rk =
            __builtin_amdgcn_make_buffer_rsrc((void*)kbase, 0, ok ? a.cap * KRB : 0, kBufWord3);
#pragma unroll
        for (int tile = 0; tile < 2; tile++) {
#pragma unroll
            for (int cc = 0; cc < KL; cc++)
                st.kc[tile][cc] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                               rk, off_k + tile * 4 * KRB + (T4 ? 16 : 64) * cc, 32 * si * KRB, AUX));
        }
        if constexpr (T4) {
            const __amdgpu_buffer_rsrc_t rkp =
                __builtin_amdgcn_make_buffer_rsrc((void*)kpbase, 0, ok ? a.cap * KPB : 0, kBufWord3);
#pragma unroll
            for (int tile = 0; tile < 2; tile++)
                st.kp[tile] = u32x4{__builtin_amdgcn_raw_buffer_load_b32(rkp, off_kp + tile * 4 * KPB,
                                                                         32 * si * KPB, AUX),
                                    0u, 0u, 0u};
        }
        if constexpr (AFF) {
            const __amdgpu_buffer_rsrc_t rkp =
                __builtin_amdgcn_make_buffer_rsrc((void*)kpbase, 0, ok ? a.cap * KPB : 0, kBufWord3);
#pragma unroll
            for (int tile = 0; tile < 2; tile++) {
                const int o = off_kp + tile * 4 * KPB;
                if constexpr (BITS == 4 && NG == 4) {
                    const auto t2 = __builtin_amdgcn_raw_buffer_load_b64(rkp, o, 32 * si * KPB, AUX);
                    st.kp[tile] = u32x4{t2[0], t2[1], 0u, 0u};
                } else if constexpr (BITS == 4) {
                    st.kp[tile] = u32x4{__builtin_amdgcn_raw_buffer_load_b32(rkp, o, 32 * si * KPB, AUX),
                                        0u, 0u, 0u};
                } else if constexpr (NG == 4) {
                    st.kp[tile] = __builtin_bit_cast(
                        u32x4, __builtin_amdgcn_raw_buffer_load_b128(rkp, o, 32 * si * KPB, AUX));
                } else {
                    const auto t2 = __builtin_amdgcn_raw_buffer_load_b64(rkp, o, 32 * si * KPB, AUX);
                    st.kp[tile] = u32x4{t2[0], t2[1], 0u, 0u};
                }
            }
        }
    };
    auto load_v = [&](Stage& st, int s) {
        const bool ok = s < s_end;
        const int si = ok ? s : 0;
        const __amdgpu_buffer_rsrc_t rv =
            __builtin_amdgcn_make_buffer_rsrc((void*)vbase, 0, ok ? a.cap / 8 * VBB : 0, kBufWord3);
        if constexpr (T4) {
            // key 8g + j: the lane's DPL/2 bytes of that row (row stride KRB)
#pragma unroll
            for (int j = 0; j < 8; j++) {
                if constexpr (D == 256) {
                    const auto t2 = __builtin_amdgcn_raw_buffer_load_b64(rv, off_v + j * KRB, 4 * si * VBB, AUX);
                    st.vc[j / 2][2 * (j % 2)] = t2[0];
                    st.vc[j / 2][2 * (j % 2) + 1] = t2[1];
                } else {
                    st.vc[j / 4][j % 4] = __builtin_amdgcn_raw_buffer_load_b32(rv, off_v + j * KRB, 4 * si * VBB, AUX);
                }
            }
            const __amdgpu_buffer_rsrc_t rvp =
                __builtin_amdgcn_make_buffer_rsrc((void*)vpbase, 0, ok ? a.cap / 8 * VPB : 0, kBufWord3);
            st.vp[0] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rvp, off_vp, 4 * si * VPB, AUX));
            st.vp[1] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rvp, off_vp + 16, 4 * si * VPB, AUX));
        } else {
#pragma unroll
            for (int jj = 0; jj < VL; jj++)
                st.vc[jj] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, off_v + 256 * jj, 4 * si * VBB, AUX));
        }
        if constexpr (AFF) {
            const __amdgpu_buffer_rsrc_t rvp =
                __builtin_amdgcn_make_buffer_rsrc((void*)vpbase, 0, ok ? a.cap / 8 * VPB : 0, kBufWord3);
            st.vp[0] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rvp, off_vp, 4 * si * VPB, AUX));
            st.vp[1] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rvp, off_vp + 16, 4 * si * VPB, AUX));
        }
    };
    auto load = [&](Stage& st, int s) {
        load_k(st, s);
        load_v(st, s);
    };

    // ---- Q rows of this KV group as the B operand (col = query row r16).
    // The workgroup's waves share one KV head, so the operand is built once
    // into LDS (wave w converts MFMA slice w) and each QK MFMA reads its slice
    // back with one ds_read_b128. Padding rows are zero.
    const int rho = r16;
    const bool row_ok = rho < a.R;
    static_assert(NW >= NM, "one Q slice per wave");
    // Turbo4: the rows are rotated into the K basis here (as the rotation
    // kernel does it, one wave a row) and staged as fp16 in the wave merge's
    // LDS area, which is free until the main loop ends.
    f16* const sm_qr = (f16*)sm_o;
    int s = c + a.ns * wave;
    Stage A, B;
    if constexpr (T4) {
        // Every global read of the prologue (the wave's q rows, the lane's
        // signs, a centroid pair a thread) is issued first and the first
        // sub-chunk's loads right behind them, so their latencies overlap;
        // the rotations and the table then wait for the prologue's reads only.
        constexpr int VPL = D / 64;
        static_assert(2 * NW >= 16 && 64 * NW >= 256, "two q rows a wave, a table entry a thread");
        f16 xq[2][VPL], xpq[2][VPL];
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int row = wave + k * NW;
            const int rr = row < a.R ? row : 0;
            const f16* qrow = ROPE ? a.q + (int64_t)(rr / a.G) * a.q_tok_stride + (int64_t)(h * a.G + rr % a.G) * D
                                   : a.q + ((int64_t)(h * a.G + rr % a.G) * a.Tq + rr / a.G) * D;
#pragma unroll
            for (int j = 0; j < VPL; j++) xq[k][j] = qrow[lane * VPL + j];
            if constexpr (ROPE) {
                // the half-split partners of the lane's dims
                const int d0 = lane * VPL, rh = a.app.rope_dims >> 1;
                const int pb = d0 < rh ? d0 + rh : d0 - rh;
                const bool need = !a.app.traditional && d0 < a.app.rope_dims;
#pragma unroll
                for (int j = 0; j < VPL; j++) xpq[k][j] = need ? qrow[pb + j] : (f16)0.0f;
            }
        }
        float si[VPL], so[VPL];
        t4_lane_signs<D>(a.t4_tab + T4Tab<D>::k_s1, lane, si);
        t4_lane_signs<D>(a.t4_tab + T4Tab<D>::k_s2, lane, so);
        const int tb = threadIdx.x & 255;
        const float* cb = a.t4_tab + T4Tab<D>::cb;
        const float2 pair = float2{cb[tb & 15], cb[tb >> 4]};
        load(A, s);
        if (threadIdx.x < 256) sm_t4[threadIdx.x] = pair;
        float yq[2][VPL];
        if constexpr (ROPE) {
            float2* const rtab = (float2*)((char*)sm_o + 16 * D * sizeof(f16));  // behind sm_qr
            rope_fill_table(a.app, a.Tq, rtab, 64 * NW);
            __syncthreads();
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int row = wave + k * NW;
                const int rr = row < a.R ? row : 0;
                f16 yk[VPL];
                rope_rotate_dims<VPL>(a.app, rtab, rr / a.G, lane * VPL, xq[k], xpq[k], yk);
#pragma unroll
                for (int j = 0; j < VPL; j++) yq[k][j] = (float)yk[j];
            }
        } else {
#pragma unroll
            for (int k = 0; k < 2; k++)
#pragma unroll
                for (int j = 0; j < VPL; j++) yq[k][j] = (float)xq[k][j];
        }
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int row = wave + k * NW;
            if (row >= a.R) break;
            f16 o[VPL];
            t4_rotate_row<D>(yq[k], lane, si, so, o);
#pragma unroll
            for (int j = 0; j < VPL; j++) sm_qr[row * D + lane * VPL + j] = o[j];
        }
        __syncthreads();
    }
    half8 x;
    {
        const int rr = row_ok ? rho : 0;
        // rr / G and rr % G for rr < 16 from a float reciprocal (exact here:
        // (rr + 0.5) / G is at least 0.5 / G from an integer)
        const int rq = (int)(((float)rr + 0.5f) * a.inv_g), rg_ = rr - rq * a.G;
        const f16* qrow = T4     ? sm_qr + rr * D
                          : ROPE ? a.q + (int64_t)rq * a.q_tok_stride + (int64_t)(h * a.G + rg_) * D
                                 : a.q + ((int64_t)(h * a.G + rg_) * a.Tq + rq) * D;
        const int m = wave % NM;
        int base;
        if constexpr (T4)
            base = (D / 4) * g + 8 * m;
        else if constexpr (BITS == 4)
            base = 8 * (16 * (m / 4) + 4 * g + (m % 4));
        else if constexpr (BITS == 8)
            base = 4 * (16 * (m / 2) + 4 * g + 2 * (m % 2));
        else
            base = 32 * m + 8 * g;
        x = *(const half8*)(qrow + base);
        if constexpr (ROPE && !T4) {
            // the half-split partners of the 8 dims; rotated once the
            // workgroup's angle table is in
            const int rh = a.app.rope_dims >> 1;
            const int pb = base < rh ? base + rh : base - rh;
            const half8 xp = !a.app.traditional && base < a.app.rope_dims ? *(const half8*)(qrow + pb)
                                                                        : half8{};
            load(A, s);
            float2* const rtab = (float2*)sm_o;
            rope_fill_table(a.app, a.Tq, rtab, 64 * NW);
            __syncthreads();
            f16 xa[8], xpa[8], ya[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                xa[e] = x[e];
                xpa[e] = xp[e];
            }
            rope_rotate_dims<8>(a.app, rtab, rq, base, xa, xpa, ya);
#pragma unroll
            for (int e = 0; e < 8; e++) x[e] = ya[e];
        }
    }
    // The first sub-chunk's loads go out right behind Q (loads return in
    // issue order, so the Q conversion below waits for Q only: the Q barrier
    // holds every wave of the workgroup until the last one's q is in);
    // Turbo4 issued them in its prologue above (and ROPE launches after the
    // partners of q).
    if constexpr (!T4 && !ROPE) load(A, s);
    {
        // q' = f16(f16(scale) * q): one packed fp16 multiply rounds exactly
        // like MLX's fp16 `multiply`. Padding rows get scale 0.
        const f16 sc = row_ok ? (f16)a.scale_h : (f16)0.0f;
        const half2v sc2 = {sc, sc};
        if (wave < NM) {
            const int m = wave;
            const u32x4 w = __builtin_bit_cast(u32x4, x);
            u32x4 o;
            if constexpr (BITS == 4 && !T4) {
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
    // 4-bit: the wave keeps its q' fragments in registers (32 VGPRs fit the
    // budget) instead of reading them from LDS for every 16-key tile.
    constexpr bool kQReg = BITS == 4 && QW_DECODE_QREG;
    half8 qreg[NM];
    if constexpr (kQReg) {
#pragma unroll
        for (int m = 0; m < NM; m++) qreg[m] = sm_q[m][lane];
    }
    auto qop = [&](int m) -> half8 {
        if constexpr (kQReg)
            return qreg[m];
        else
            return sm_q[m][lane];
    };
    const int lim = a.causal ? a.T - a.Tq + (row_ok ? rho / a.G : 0) : a.T - 1;

    float m_run = -INFINITY;  // softmax reference of row r16 (natural units)
    float l_run = 0.0f;       // this lane's share of the row sum
    float4v acc_o[DPL];
#pragma unroll
    for (int mm = 0; mm < DPL; mm++) acc_o[mm] = float4v{0.f, 0.f, 0.f, 0.f};
    float4v acc_b = float4v{0.f, 0.f, 0.f, 0.f};  // P * V biases (rows 4g+i, dim group of r16)

    // Q.K^T of the two 16-key tiles (S^T: lane holds keys 8g+i / 8g+4+i of
    // column r16); the two MFMA chains interleave to hide each other's latency.
    auto qk = [&](const Stage& st, float4v& acc0, float4v& acc1) {
        acc0 = float4v{0.f, 0.f, 0.f, 0.f};
        acc1 = float4v{0.f, 0.f, 0.f, 0.f};
        if constexpr (T4) {
            // step m: dims (D/4) g + 8m .. +7 of the lane's key, word m of its codes
            const float kr0 = (float)h2(st.kp[0][0]).x, kr1 = (float)h2(st.kp[1][0]).x;
#pragma unroll
            for (int m = 0; m < NM; m++) {
                acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(t4_expand8(st.kc[0][m / 4][m % 4], kr0, sm_t4),
                                                              qop(m), acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(t4_expand8(st.kc[1][m / 4][m % 4], kr1, sm_t4),
                                                              qop(m), acc1, 0, 0, 0);
            }
        } else if constexpr (BITS == 4) {
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
                        deq4<FAST>(st.kc[0][cc][mi], p0, magic), qop(m), acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        deq4<FAST>(st.kc[1][cc][mi], p1, magic), qop(m), acc1, 0, 0, 0);
                }
            }
        } else if constexpr (BITS == 8) {
#pragma unroll
            for (int m = 0; m < NM; m++) {
                const int slot = k_param_slot(m / 2, NG);
                const half2v sb0 = h2(st.kp[0][slot]), sb1 = h2(st.kp[1][slot]);
                const half2v s0 = {sb0.x, sb0.x}, b0 = {sb0.y, sb0.y};
                const half2v s1 = {sb1.x, sb1.x}, b1 = {sb1.y, sb1.y};
                const PairConsts p0 = make_consts<FAST, 8>(s0, s0, s0, s0, b0, b0, b0, b0, a.code_off2);
                const PairConsts p1 = make_consts<FAST, 8>(s1, s1, s1, s1, b1, b1, b1, b1, a.code_off2);
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
        if constexpr (T4) {
            // B of output tile mm: dim DPL r16 + mm of keys 8g..8g+7 (nibble mm
            // of each key's row piece)
            float vr[8];
#pragma unroll
            for (int j = 0; j < 8; j++) vr[j] = (float)h2(st.vp[j / 4][j % 4]).y;
            // output tiles 2e, 2e+1: byte e of each key's piece (one pair lookup
            // a key for both)
#pragma unroll
            for (int e = 0; e < DPL / 2; e++) {
                half8 b0, b1;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const uint32_t w = D == 256 ? st.vc[j / 2][2 * (j % 2) + e / 4] : st.vc[j / 4][j % 4];
                    const float2 c = sm_t4[(w >> (8 * (e % 4))) & 0xFFu];
                    b0[j] = t4_f16_product(c.x, vr[j]);
                    b1[j] = t4_f16_product(c.y, vr[j]);
                }
                acc_o[2 * e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pop, b0, acc_o[2 * e], 0, 0, 0);
                acc_o[2 * e + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pop, b1, acc_o[2 * e + 1], 0, 0, 0);
            }
            return;
        }
        PairConsts pc;
        if constexpr (AFF)
            pc = make_consts<FAST, BITS>(h2(st.vp[0][0]), h2(st.vp[0][1]), h2(st.vp[0][2]),
                                         h2(st.vp[0][3]), h2(st.vp[0][0]), h2(st.vp[0][1]),
                                         h2(st.vp[0][2]), h2(st.vp[0][3]), a.code_off2);
#pragma unroll
        for (int mm = 0; mm < DPL; mm++) {
            half8 bv;
            if constexpr (BITS == 4)
                bv = deq4<FAST, false>(st.vc[mm / 4][mm % 4], pc, magic);
            else if constexpr (BITS == 8)
                bv = deq8<FAST, false>(st.vc[mm / 2][2 * (mm % 2)], st.vc[mm / 2][2 * (mm % 2) + 1], pc);
            else
                bv = as_h8(st.vc[mm]);
            acc_o[mm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pop, bv, acc_o[mm], 0, 0, 0);
        }
        if constexpr (AFF)
            acc_b = __builtin_amdgcn_mfma_f32_16x16x32_f16(pop, as_h8(st.vp[1]), acc_b, 0, 0, 0);
    };

    auto scores = [&](const Stage& st, int s) -> half8 {
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
        // The check uses the lane's own maximum: m_run is the same in the four
        // lanes of a row, so some lane's maximum exceeds m_run + 5.5 exactly
        // when some row's does, and the row reduction (two LDS permutes) runs
        // only when the reference moves.
        float mx = sc[0];
#pragma unroll
        for (int e = 1; e < 8; e++) mx = fmaxf(mx, sc[e]);
        if (__any(mx > m_run + 5.5f)) {
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
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
#pragma unroll
                for (int i = 0; i < 4; i++) acc_b[i] *= f[i];
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
        return pop;
    };
    auto compute = [&](const Stage& st, int s) { pv(st, scores(st, s)); };

    if constexpr (decode_stages<BITS>() == 2) {
        // Wait-then-prefetch per plane: each K or V half of a stage is
        // requested once the previous half has landed, and QK starts as soon
        // as the stage's K half is in, so about one stage of a wave is in
        // flight at a time (measured faster than both stages in flight from
        // the start, and than waiting for whole stages).
        // loads a K half and a V half of a stage issue
        constexpr int NK = 2 * KL + (AFF || T4 ? 2 : 0), NV = (T4 ? 8 : VL) + (AFF || T4 ? 2 : 0);
        static_assert(NK < 16 && NV < 16, "vmcnt field");
        // vmcnt(n), expcnt/lgkmcnt untouched: a stage's K half is in while its
        // V half (NV loads) may be in flight; its V half while the next
        // stage's K half (NK loads) may be
        constexpr int kWaitK = 0x0F70 | NV, kWaitV = 0x0F70 | NK;
        for (; s < s_end; s += 2 * SS) {
            __builtin_amdgcn_s_waitcnt(kWaitK);  // K(A) in; V(A) may be in flight
            load_k(B, s + SS);
            const half8 pa = scores(A, s);
            __builtin_amdgcn_s_waitcnt(kWaitV);  // V(A) in; K(B) may be in flight
            load_v(B, s + SS);
            pv(A, pa);
            if (s + SS >= s_end) break;
            __builtin_amdgcn_s_waitcnt(kWaitK);
            load_k(A, s + 2 * SS);
            const half8 pb = scores(B, s + SS);
            __builtin_amdgcn_s_waitcnt(kWaitV);
            load_v(A, s + 2 * SS);
            pv(B, pb);
        }
    } else {
        for (; s < s_end; s += SS) {
            compute(A, s);
            if (s + SS >= s_end) break;
            // keep the next sub-chunk's loads behind this one's math
            __builtin_amdgcn_sched_barrier(0);
            load(A, s + SS);
        }
    }
    float lsum = l_run;
    lsum += lane_xor<16>(lsum, lane);
    lsum += lane_xor<32>(lsum, lane);
    // ---- merge the NW waves into the workgroup's partial. The VALU work of
    // a merge is what sits on the critical path after the last data (two
    // waves a SIMD run it at once), so each step does as little as it can:
    //  1. each wave parks its raw accumulators (lanes g < G4: rows 4g..4g+3
    //     of dims r16*DPL .. +DPL-1, a float4 a dim), its P.V-bias sums
    //     (rows 4g..4g+3, the dim group of column r16) and (m, l) of its
    //     rows; barrier;
    //  2. wave 0 forms each row's M = max m_w, L = sum e^(m_w - M) l_w and
    //     the factors f_w = e^(m_w - M) (lane (g, r16): row r16, waves
    //     g, g+4, ...), and writes (M, L) of the partial; barrier;
    //  3. each thread sums f_w (acc_w + b_w) over the waves for one dim of
    //     four rows and stores them (consecutive threads, consecutive dims).
    const int R = a.R;
    const int G4 = (R + 3) >> 2;  // lane groups holding real rows
    float4v* const sm_acc = (float4v*)sm_o;                    // [NW][G4][16][DPL]
    float4v* const sm_b = sm_acc + (int64_t)NW * G4 * 16 * DPL;  // [NW][G4][16]
    float* const sm_f = (float*)(sm_b + NW * G4 * 16);         // [4 row groups][NW][4 rows]
    if (g == 0) sm_ml[r16][wave] = float2{m_run, lsum};
    if (g < G4) {
        // dim r16*DPL + mm at slot mm ^ (r16 % DPL) of the lane's DPL-slot run:
        // the 16 lanes of a store land in 16 distinct bank groups, and step 3
        // reads whole runs
        float4v* dst = sm_acc + (((int64_t)wave * G4 + g) * 16 + r16) * DPL;
#pragma unroll
        for (int mm = 0; mm < DPL; mm++) dst[mm ^ (r16 % DPL)] = acc_o[mm];
        sm_b[(wave * G4 + g) * 16 + r16] = acc_b;
    }
    __syncthreads();
    if (wave == 0) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, sm_ml[r16][w].x);
        const float Ms = M == -INFINITY ? 0.0f : M;  // a row with no visible key
        float L = 0.0f;
        for (int w = g; w < NW; w += 4) {
            const float2 ml = sm_ml[r16][w];
            const float f = __builtin_amdgcn_exp2f((ml.x - Ms) * kLog2e);
            sm_f[((r16 >> 2) * NW + w) * 4 + (r16 & 3)] = f;
            L = __builtin_fmaf(f, ml.y, L);
        }
        L += lane_xor<16>(L, lane);
        L += lane_xor<32>(L, lane);
        if (g == 0 && r16 < R) part_ml[((int64_t)h * a.nc + c) * 16 + r16] = float2{M, L};
    }
    __syncthreads();
    const int64_t pbase = ((int64_t)h * a.nc + c) * 16;
    for (int t = threadIdx.x; t < G4 * D; t += 64 * NW) {
        // t = (rg, d): dim d of rows 4rg..4rg+3
        const int rg = t / D, d = t % D, rl = d / DPL, mm = d % DPL;
        const float4v* src = sm_acc + ((int64_t)rg * 16 + rl) * DPL + (mm ^ (rl % DPL));
        const float4v* bsrc = sm_b + rg * 16 + rl;
        const float4v* fsrc = (const float4v*)sm_f + rg * NW;
        float4v y = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
        for (int w = 0; w < NW; w++) {
            const float4v x = src[(int64_t)w * G4 * 16 * DPL] + bsrc[w * G4 * 16];
            const float4v f = fsrc[w];
#pragma unroll
            for (int i = 0; i < 4; i++) y[i] = __builtin_fmaf(f[i], x[i], y[i]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (4 * rg + i < R) part_o[(pbase + 4 * rg + i) * D + d] = y[i];
    }
}

// LDS the append unit needs: an 8-token block's append scratch, then the new
// keys' K and V values (fp16, [app_L][D] each).
template <int D>
constexpr size_t decode_append_lds(int L) {
    return (sizeof(AppendScratch<D>) + 15) / 16 * 16 + (size_t)4 * L * D;
}
// (Turbo4 uses the scratch's first 64 bytes for the centroids)
static_assert(sizeof(AppendScratch<128>) >= 16 * sizeof(float), "centroid table fits the scratch");

// The append unit of a decode launch (DecodeArgs::app_L > 0), workgroup
// (ns, h). It appends head h's new rows (the append kernels' work), reads
// them back as the decode kernel would (affine and Int8: f16(f16(c s) + b)
// and f16(c s); Turbo4: f16(centroid rescale) in the rotated basis), and
// writes the new keys' partial for every row of the launch in the decode
// kernel's arithmetic: q' = f16(f16(scale) q) (Turbo4: q rotated first), the
// score rounded to fp16, the weights exp(s - m) summed in fp32 and rounded to
// fp16 for P.V. Wave w takes rows w, w + NW, ... The unit runs while the
// prefix splits keep HBM busy, so its loads are issued up front (q rows and
// rotation signs with the appended rows) and Turbo4 expands the new keys
// from the quantizer's registers: each dependent memory round trip here costs
// microseconds.
template <int BITS, int D, bool T4, bool ROPE = false>
__device__ void decode_append_unit(const DecodeArgs& a, char* lds) {
    constexpr int NW = decode_waves<BITS, D>();
    constexpr int VPL = D / 64, NG = D / 64;
    constexpr int RPW = (16 + NW - 1) / NW;  // rows a wave (R <= 16)
    const int h = blockIdx.y, L = a.app_L, T0 = a.T;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    f16* sk = (f16*)(lds + (sizeof(AppendScratch<D>) + 15) / 16 * 16);
    f16* sv = sk + L * D;
    float qv[RPW][VPL];
#pragma unroll
    for (int k = 0; k < RPW; k++) {
        const int rho = min(wave + NW * k, a.R - 1);
        const int qh = h * a.G + rho % a.G, r = rho / a.G;
        if constexpr (ROPE) {
            // the rows rotated as the RoPE kernels rotate them, and written out
            const f16* qrow = a.q + (int64_t)r * a.q_tok_stride + (int64_t)qh * D;
            const RowSrc& rs = a.app;
#pragma unroll
            for (int i = 0; i < VPL; i++) {
                const f16 y = (f16)rope_elem(qrow, lane * VPL + i, rs.rope_dims, rs.traditional,
                                             rs.log2_base, rs.scale, rs.position0 + r);
                qv[k][i] = (float)y;
                if (wave + NW * k < a.R) a.q_out[((int64_t)qh * a.Tq + r) * D + lane * VPL + i] = y;
            }
        } else {
            const f16* qrow = a.q + ((int64_t)qh * a.Tq + r) * D;
#pragma unroll
            for (int i = 0; i < VPL; i++) qv[k][i] = (float)qrow[lane * VPL + i];
        }
    }
    float si[VPL], so[VPL];
    if constexpr (T4) {
        t4_lane_signs<D>(a.t4_tab + T4Tab<D>::k_s1, lane, si);
        t4_lane_signs<D>(a.t4_tab + T4Tab<D>::k_s2, lane, so);
        float* s_cb = (float*)lds;
        if (tid < 16) s_cb[tid] = a.t4_tab[T4Tab<D>::cb + tid];
        __syncthreads();
        for (int job = wave; job < 2 * L; job += NW) {
            const int j = job >> 1;
            turbo4_append_row<D>(a.app, j, h, (job & 1) == 0, lane, T0, a.cap, a.t4_tab, s_cb,
                                 (uint8_t*)a.k_data, (uint32_t*)a.k_params, (uint8_t*)a.v_data,
                                 (uint32_t*)a.v_params, ((job & 1) == 0 ? sk : sv) + j * D);
        }
    } else {
        auto& sc = *reinterpret_cast<AppendScratch<D>*>(lds);
        for (int blk = T0 / 8; blk <= (T0 + L - 1) / 8; blk++) {
            append_block<D>(a.app, L, T0, BITS, a.app_int8 != 0, a.cap, (uint32_t*)a.k_data,
                            (uint32_t*)a.k_params, (uint32_t*)a.v_data, (f16*)a.v_params,
                            (int*)a.fast_flag, blk, h, tid, 64 * NW, sc);
            __syncthreads();
        }
    }
    __syncthreads();
    // affine and Int8: the new keys' values, read back from the cache
    for (int i = tid; i < (T4 ? 0 : L * D); i += 64 * NW) {
        const int j = i / D, d = i % D, t = T0 + j;
        const int64_t kr = (int64_t)h * a.cap + t;
        const int blk = t / 8, k = t % 8;
        f16 kv = (f16)0.0f, vv = (f16)0.0f;
        if constexpr (!T4) {
            constexpr int EPW = 32 / BITS;
            constexpr uint32_t MASK = (1u << BITS) - 1;
            const uint32_t kw = a.k_data[kr * (D * BITS / 32) + d / EPW];
            const float kc = (float)((kw >> (BITS * (d % EPW))) & MASK);
            const half2v ksb = __builtin_bit_cast(half2v, a.k_params[kr * NG + k_param_slot(d / 64, NG)]);
            const int p = v_phys_dim(d, D, BITS);
            const uint32_t* vbw = a.v_data + ((int64_t)h * (a.cap / 8) + blk) * (D * BITS / 4);
            const float vc = BITS == 4 ? (float)((vbw[p] >> (4 * v4_nibble_pos(k))) & 15u)
                                       : (float)((vbw[2 * p + (k >> 2)] >> (8 * (k & 3))) & 255u);
            const f16* vpp = (const f16*)a.v_params + (((int64_t)h * (a.cap / 8) + blk) * NG + d / 64) * 16;
            if (a.app_int8) {
                kv = (f16)((kc - 128.0f) * (float)ksb.x);
                vv = (f16)((vc - 128.0f) * (float)vpp[k]);
            } else {
                kv = (f16)affine_dequant(kc, ksb.x, ksb.y);
                vv = (f16)affine_dequant(vc, vpp[k], vpp[8 + k]);
            }
        }
        sk[i] = kv;
        sv[i] = vv;
    }
    __syncthreads();
    const int64_t pbase = ((int64_t)h * a.nc + a.ns) * 16;
#pragma unroll
    for (int k = 0; k < RPW; k++) {
        const int rho = wave + NW * k;
        if (rho >= a.R) break;  // wave-uniform
        const int l = rho / a.G;
        float(&q)[VPL] = qv[k];
        if constexpr (T4) {
            f16 o[VPL];
            t4_rotate_row<D>(q, lane, si, so, o);
#pragma unroll
            for (int i = 0; i < VPL; i++) q[i] = (float)o[i];
        }
#pragma unroll
        for (int i = 0; i < VPL; i++) q[i] = (float)(f16)(a.scale_h * q[i]);
        const int n_vis = a.app_causal ? l + 1 : L;
        float sc[16];
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            sc[j] = -INFINITY;
            if (j < n_vis) {
                float dot = 0.0f;
#pragma unroll
                for (int i = 0; i < VPL; i++)
                    dot = __builtin_fmaf(q[i], (float)sk[j * D + lane * VPL + i], dot);
                sc[j] = (float)(f16)t4_wave_sum(dot);
                m = fmaxf(m, sc[j]);
            }
        }
        float o[VPL] = {};
        float lsum = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            if (j < n_vis) {
                const float pj = __builtin_amdgcn_exp2f((sc[j] - m) * kLog2e);
                lsum += pj;
                const float ph = (float)(f16)pj;
#pragma unroll
                for (int i = 0; i < VPL; i++)
                    o[i] = __builtin_fmaf(ph, (float)sv[j * D + lane * VPL + i], o[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < VPL; i++) a.part_o[(pbase + rho) * D + lane * VPL + i] = o[i];
        if (lane == 0) a.part_ml[pbase + rho] = float2{m, lsum};
    }
}

template <int BITS, int D, bool T4 = false, bool APP = false, bool NT = false, bool ROPE = false>
__global__ __launch_bounds__((64 * decode_waves<BITS, D>()), 1) void attend_decode_kernel(
    DecodeArgs a) {
    static_assert(!ROPE || APP, "RoPE launches append their rows");
    constexpr int NW = decode_waves<BITS, D>();
    constexpr int AUX = NT ? 2 : 0;  // the K/V loads' cache policy
    __shared__ __attribute__((aligned(16))) float2 sm_ml[16][NW];
    __shared__ half8 sm_q[D / 32][64];
    __shared__ float2 sm_t4[T4 ? 256 : 1];  // Turbo4 centroid-pair table
    // dynamic LDS: the wave merge's accumulators, bias sums and factors
    extern __shared__ __attribute__((aligned(16))) float sm_o[];
    // The exact 2-op dequant runs first without waiting for the cache's fast
    // flag (a memory round trip ahead of every load). In the rare launch whose
    // cache holds a scale outside that dequant's exact range, the workgroup
    // then redoes its share with the separately rounded dequant, and that
    // pass's partial (same threads, same elements) replaces the first. A
    // null flag (Int8 caches, which always take the separately rounded
    // dequant) goes to that path directly.
    // Turbo4 caches have one dequant (a null flag).
    if constexpr (APP && BITS != 16) {
        if ((int)blockIdx.x == a.ns) {
            decode_append_unit<BITS, D, T4, ROPE>(a, (char*)sm_o);
            return;
        }
    }
    if (!T4 && (BITS == 16 || a.fast_flag != nullptr)) {
        decode_body<BITS, D, NW, true, false, AUX, ROPE>(a, sm_ml, sm_o, sm_q);
        if (BITS != 16 && *a.fast_flag == 0) {
            __syncthreads();
            decode_body<BITS, D, NW, false, false, AUX, ROPE>(a, sm_ml, sm_o, sm_q);
        }
    } else {
        decode_body<BITS, D, NW, false, T4, AUX, ROPE>(a, sm_ml, sm_o, sm_q, sm_t4);
    }
}

// Combines the per-workgroup partials of one query row (partials of a KV head
// are [nc][rstride] rows, row index = r * G + head-in-group): out = sum_c e^(m_c - M)
// O_c / sum_c e^(m_c - M) l_c, rounded to fp16 (a row with no visible key is 0).
// grid (rows, kv_heads, D/64): a workgroup owns 64 dims of one row; lane =
// dim, wave w sums partials c = w, w + kMW, ... with every load issued up
// front.
constexpr int kMergeMaxPer = 64;  // partials a wave of four sums (nc <= 256)

// Partials a wave sums, as a compile-time bound: the smallest power of two
// from 4 to kMergeMaxPer that covers nc / 4.
inline int merge_per(int nc) {
    int per = 4;
    while (4 * per < nc) per *= 2;
    return per;
}

// Waves of the decode merge workgroup, each summing every kMW-th partial:
// eight measured c2 attention 15.25 -> 15.00 us against four, sixteen 15.05 us
// (A/B in one run); the (m, l) loads through the scalar cache gained nothing.
#ifndef QW_MERGE_WAVES
#define QW_MERGE_WAVES 8
#endif
constexpr int kMW = QW_MERGE_WAVES;

template <int PER>
__global__ __launch_bounds__(64 * kMW) void decode_merge_kernel(const float* __restrict__ part_o,
                                                           const float2* __restrict__ part_ml,
                                                           int nc, int rstride, int row0, int D,
                                                           int G, int Tq, int slot_bits,
                                                           f16* __restrict__ out,
                                                           float* __restrict__ out32) {
    // lane = place sd in the partial rows (contiguous loads); it holds dim d
    // (partial rows in slot order: the dim whose slot sd is)
    const int row = blockIdx.x, h = blockIdx.y, sd = blockIdx.z * 64 + (threadIdx.x & 63);
    const int d = slot_bits ? v_logical_dim(sd, D, slot_bits) : sd;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t base = (int64_t)h * nc * rstride + row;
    // One memory round: every (m, l) and O value this lane needs is loaded
    // first.
    float v[PER];
    float2 ml[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int c = wave + kMW * i;
        if (c < nc) {
            ml[i] = part_ml[base + (int64_t)c * rstride];
            v[i] = part_o[(base + (int64_t)c * rstride) * D + sd];
        } else {
            ml[i] = float2{-INFINITY, 0.0f};
            v[i] = 0.0f;
        }
    }
    // each wave reduces its partials against its own maximum; the four
    // (m, l, O) then meet in LDS behind one barrier
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; i++) m = fmaxf(m, ml[i].x);
    float o = 0.0f, l = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const float w =
            ml[i].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((ml[i].x - m) * kLog2e);
        o = __builtin_fmaf(w, v[i], o);
        l = __builtin_fmaf(w, ml[i].y, l);
    }
    __shared__ float2 sm_ml[kMW];
    __shared__ float sm_o[kMW][64];
    if (lane == 0) sm_ml[wave] = float2{m, l};
    sm_o[wave][lane] = o;
    __syncthreads();
    if (wave == 0) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kMW; w++) M = fmaxf(M, sm_ml[w].x);
        float O = 0.0f, L = 0.0f;
#pragma unroll
        for (int w = 0; w < kMW; w++) {
            const float f = sm_ml[w].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((sm_ml[w].x - M) * kLog2e);
            O = __builtin_fmaf(f, sm_o[w][lane], O);
            L = __builtin_fmaf(f, sm_ml[w].y, L);
        }
        const int orow = row0 + row;  // row index r * G + head-in-group
        const int qh = h * G + orow % G, qr = orow / G;
        const float y = L > 0.0f ? O / L : 0.0f;
        if (out32)
            out32[((int64_t)qh * Tq + qr) * D + d] = y;
        else
            out[((int64_t)qh * Tq + qr) * D + d] = (f16)y;
    }
}

// Split-K attention of the Tq rows over the first T cached keys: launches the
// decode kernel and returns its partials (nc per KV head, 16 rows apart).
// rope (a RoPE launch, with app_L > 0): the new rows come through *rope (K
// rotated on load), q is the projection with token stride q_tok_stride, and
// the rotated q rows go to q_out.
template <int BITS, int D, bool T4 = false>
static int launch_decode_partials(KVCache& cc, const f16* q, int G, int Tq, int T, float scale,
                                  bool causal, int* nc_out, float** po, float2** pml,
                                  hipStream_t stream, const float* t4_tab = nullptr,
                                  const f16* k_new = nullptr, const f16* v_new = nullptr,
                                  int app_L = 0, bool app_causal = false,
                                  const RowSrc* rope = nullptr, int64_t q_tok_stride = 0,
                                  f16* q_out = nullptr) {
    const int n_sub = (T + 31) / 32;
    // Sub-chunks a wave owns: 4-bit rows are small enough to keep 4 in flight.
    // Sub-chunks a wave keeps in flight per round, and workgroups per KV head:
    // two 4-wave workgroups a CU (256 CUs), each wave one round when the
    // context allows, at most 1024 partials per head.
    // One workgroup a CU (256 CUs), at least a wave's worth of sub-chunks each.
    constexpr int NW = decode_waves<BITS, D>();
    // an append unit (app_L > 0) takes one workgroup slot a head
    const int app = app_L > 0 ? 1 : 0;
    const int per_head = std::max(1, 256 / cc.hkv - app);
    // Turbo4: at most 128 partials a head (its merge kernel sums up to 32 a thread)
    const int nc_cap = (T4 ? 128 : 4 * kMergeMaxPer) - app;
    const int ns = std::max(1, std::min({per_head, (n_sub + NW - 1) / NW, nc_cap}));
    const int nc = ns + app;
    const size_t need = (size_t)cc.hkv * nc * 16 * D * sizeof(float) +
                        (size_t)cc.hkv * nc * 16 * sizeof(float2);
    int rc = cc.ensure_workspace(need, stream);
    if (rc) return rc;
    DecodeArgs a;
    a.k_data = (const uint32_t*)cc.k_data;
    a.k_params = cc.k_params;
    a.v_data = (const uint32_t*)cc.v_data;
    a.v_params = cc.v_params;
    a.fast_flag = cc.int8() || T4 ? nullptr : cc.fast_flag;  // null: always separately rounded
    a.t4_tab = t4_tab;
    a.q = q;
    a.part_o = (float*)cc.ws_ptr;
    a.part_ml = (float2*)((char*)cc.ws_ptr + (size_t)cc.hkv * nc * 16 * D * sizeof(float));
    a.cap = cc.cap;
    a.T = T;
    a.Tq = Tq;
    a.G = G;
    a.R = G * Tq;
    a.causal = causal ? 1 : 0;
    a.n_sub = n_sub;
    a.nc = nc;
    a.ns = ns;
    a.scale_h = (float)(f16)scale;
    a.inv_g = 1.0f / (float)G;
    a.code_off2 = cc.code_offset2();
    a.app_L = app_L;
    a.app_causal = app_causal ? 1 : 0;
    a.app_int8 = cc.int8() ? 1 : 0;
    a.app = RowSrc{};
    a.app.k = k_new;
    a.app.v = v_new;
    a.app.row_stride = D;
    a.app.head_stride = (int64_t)app_L * D;
    a.q_tok_stride = 0;
    a.q_out = nullptr;
    if (rope) {
        QW_REQUIRE(app_L > 0 && rope->rope_dims % 16 == 0 && rope->rope_dims <= D && q_out,
                   QW_ERR_INVALID_ARGUMENT, "decode: RoPE launch outside its shapes");
        a.app = *rope;
        a.q_tok_stride = q_tok_stride;
        a.q_out = q_out;
    }
    // wave merge: accumulators NW x G4 x D float4, bias sums NW x G4 x 16
    // float4, factors 4 x NW float4
    size_t shmem = (size_t)NW * ((a.R + 3) / 4) * (D + 16) * 16 + 4 * NW * 16;
    // Dynamic LDS above 64 KB must be allowed per kernel and device.
    // KV bytes the call reads: K and V codes plus their params, a key and head
    constexpr int kKeyBytes = 2 * (D * BITS / 8) + (T4 ? 8 : BITS == 16 ? 0 : 2 * (D / 64) * 4);
    const bool nt = (size_t)cc.hkv * T * kKeyBytes >= ((size_t)QW_DECODE_NT_MIN_MB << 20);
    auto go = [&](auto kernel) -> int {
        int rc1 = ensure_dynamic_lds((const void*)kernel, shmem);
        if (rc1) return rc1;
        hipLaunchKernelGGL(kernel, dim3(nc, cc.hkv), dim3(64 * NW), shmem, stream, a);
        return QW_OK;
    };
    if (rope) {
        // the angle table (behind the rotated q rows of Turbo4)
        shmem = std::max({shmem, decode_append_lds<D>(app_L),
                          (size_t)(T4 ? 16 * D * sizeof(f16) : 0) +
                              (size_t)Tq * (rope->rope_dims / 2) * sizeof(float2)});
        rc = nt ? go(attend_decode_kernel<BITS, D, T4, true, true, true>)
                : go(attend_decode_kernel<BITS, D, T4, true, false, true>);
    } else if (app) {
        shmem = std::max(shmem, decode_append_lds<D>(app_L));
        rc = nt ? go(attend_decode_kernel<BITS, D, T4, true, true>)
                : go(attend_decode_kernel<BITS, D, T4, true, false>);
    } else {
        rc = nt ? go(attend_decode_kernel<BITS, D, T4, false, true>)
                : go(attend_decode_kernel<BITS, D, T4, false, false>);
    }
    if (rc) return rc;
    QW_HIP_CHECK(hipGetLastError());
    *nc_out = nc;
    *po = a.part_o;
    *pml = a.part_ml;
    return QW_OK;
}

template <int BITS, int D>
static int launch_decode_bits(KVCache& cc, const f16* q, int G, int Tq, float scale,
                              bool causal, f16* out, hipStream_t stream) {
    int nc = 0;
    float* po = nullptr;
    float2* pml = nullptr;
    int rc = launch_decode_partials<BITS, D>(cc, q, G, Tq, cc.offset, scale, causal, &nc, &po,
                                             &pml, stream);
    if (rc) return rc;
    return launch_partial_merge(po, pml, nc, 16, 0, G * Tq, cc.hkv, D, G, Tq, out, stream);
}

// Turbo4 merge: one workgroup a query row, D/64 x 4 waves (wave w sums
// partials c = w % 4, w % 4 + 4, ... of places 64 (w / 4) .. +63 of the partial
// rows, every load issued first; slot_bits != 0: the rows are in that V
// layout's slot order). The merged row is rounded to fp16 (the rotated-basis
// SDPA output; KEEP32: kept in fp32, the fused verify pass) and rotated back
// through the V basis by wave 0, as the rotation kernels form it.
template <int D, int PER, bool KEEP32>
__global__ __launch_bounds__(D * 4) void t4_merge_rotate_kernel(const float* __restrict__ part_o,
                                                              const float2* __restrict__ part_ml,
                                                              int nc, int rstride, int G, int Tq,
                                                              int slot_bits,
                                                              const float* __restrict__ tab,
                                                              f16* __restrict__ out) {
    const int row = blockIdx.x, h = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int pg = wave & 3, sd = 64 * (wave >> 2) + lane;
    const int d = slot_bits ? v_logical_dim(sd, D, slot_bits) : sd;
    const int64_t base = (int64_t)h * nc * rstride + row;
    // the rotation's signs (wave 0 rotates the merged row): loaded with the
    // partials, so no memory round trip follows the merge
    constexpr int VPL = D / 64;
    float s_in[VPL], s_out[VPL];
    if (wave == 0) {
        t4_lane_signs<D>(tab + T4Tab<D>::v_s2, lane, s_in);
        t4_lane_signs<D>(tab + T4Tab<D>::v_s1, lane, s_out);
    }
    float v[PER];
    float2 ml[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int c = pg + 4 * i;
        if (c < nc) {
            ml[i] = part_ml[base + (int64_t)c * rstride];
            v[i] = part_o[(base + (int64_t)c * rstride) * D + sd];
        } else {
            ml[i] = float2{-INFINITY, 0.0f};
            v[i] = 0.0f;
        }
    }
    // each partial group pg reduces against its own maximum; wave 0 then
    // combines the four groups for the lane's D/64 dims (the rotation's
    // layout), so one barrier separates the loads from the rotation
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; i++) m = fmaxf(m, ml[i].x);
    float o = 0.0f, l = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const float w = ml[i].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((ml[i].x - m) * kLog2e);
        o = __builtin_fmaf(w, v[i], o);
        l = __builtin_fmaf(w, ml[i].y, l);
    }
    __shared__ float2 sm_ml[4];
    __shared__ float sm_o[4][D];
    if (wave < 4 && lane == 0) sm_ml[pg] = float2{m, l};
    sm_o[pg][d] = o;
    __syncthreads();
    if (wave == 0) {
        float M = -INFINITY;
#pragma unroll
        for (int p = 0; p < 4; p++) M = fmaxf(M, sm_ml[p].x);
        float f[4], L = 0.0f;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const float2 gl = sm_ml[p];
            f[p] = gl.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((gl.x - M) * kLog2e);
            L = __builtin_fmaf(f[p], gl.y, L);
        }
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        float y[VPL];
        f16 r[VPL];
#pragma unroll
        for (int j = 0; j < VPL; j++) {
            const int dd = lane * VPL + j;
            float O = 0.0f;
#pragma unroll
            for (int p = 0; p < 4; p++) O = __builtin_fmaf(f[p], sm_o[p][dd], O);
            const float yy = L > 0.0f ? O * inv : 0.0f;
            y[j] = KEEP32 ? yy : (float)(f16)yy;
        }
        t4_rotate_row<D>(y, lane, s_in, s_out, r);
        const int qh = h * G + row % G, qr = row / G;
        f16* orow = out + ((int64_t)qh * Tq + qr) * D;
#pragma unroll
        for (int j = 0; j < VPL; j++) orow[lane * VPL + j] = r[j];
    }
}

template <int D, bool KEEP32>
static int launch_t4_merge_rotate_d(const float* po, const float2* pml, int nc, int rstride, int R,
                                    int hkv, int G, int Tq, int slot_bits, const float* tab,
                                    f16* out, hipStream_t stream) {
    QW_REQUIRE(nc >= 1 && nc <= 128, QW_ERR_INVALID_ARGUMENT, "merge: partial count out of range");
    const dim3 grid(R, hkv), block(D * 4);
    switch (merge_per(nc)) {
        case 4:
            hipLaunchKernelGGL((t4_merge_rotate_kernel<D, 4, KEEP32>), grid, block, 0, stream, po, pml,
                               nc, rstride, G, Tq, slot_bits, tab, out);
            break;
        case 8:
            hipLaunchKernelGGL((t4_merge_rotate_kernel<D, 8, KEEP32>), grid, block, 0, stream, po, pml,
                               nc, rstride, G, Tq, slot_bits, tab, out);
            break;
        case 16:
            hipLaunchKernelGGL((t4_merge_rotate_kernel<D, 16, KEEP32>), grid, block, 0, stream, po, pml,
                               nc, rstride, G, Tq, slot_bits, tab, out);
            break;
        default:  // nc <= 128
            hipLaunchKernelGGL((t4_merge_rotate_kernel<D, 32, KEEP32>), grid, block, 0, stream, po, pml,
                               nc, rstride, G, Tq, slot_bits, tab, out);
    }
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

int launch_t4_merge_rotate(const float* po, const float2* pml, int nc, int rstride, int R, int hkv,
                           int D, int G, int Tq, int slot_bits, bool keep32, const float* tab,
                           f16* out, hipStream_t stream) {
    if (D == 256)
        return keep32 ? launch_t4_merge_rotate_d<256, true>(po, pml, nc, rstride, R, hkv, G, Tq,
                                                            slot_bits, tab, out, stream)
                      : launch_t4_merge_rotate_d<256, false>(po, pml, nc, rstride, R, hkv, G, Tq,
                                                             slot_bits, tab, out, stream);
    return keep32 ? launch_t4_merge_rotate_d<128, true>(po, pml, nc, rstride, R, hkv, G, Tq, slot_bits,
                                                        tab, out, stream)
                  : launch_t4_merge_rotate_d<128, false>(po, pml, nc, rstride, R, hkv, G, Tq,
                                                         slot_bits, tab, out, stream);
}

// Decode-route calls (G * L <= 16 rows a KV head) that append L rows first:
// the decode launch's append unit appends them and attends the new keys, the
// other workgroups split the cached prefix (every row sees all of it).
template <int BITS, int D>
static int launch_decode_append(KVCache& cc, const f16* q, int G, int L, const f16* k_new,
                                const f16* v_new, float scale, bool causal, f16* out,
                                hipStream_t stream) {
    int nc = 0;
    float* po = nullptr;
    float2* pml = nullptr;
    int rc = launch_decode_partials<BITS, D>(cc, q, G, L, cc.offset, scale, false, &nc, &po, &pml,
                                             stream, nullptr, k_new, v_new, L, causal);
    if (rc) return rc;
    cc.offset += L;
    return launch_partial_merge(po, pml, nc, 16, 0, G * L, cc.hkv, D, G, L, out, stream);
}

// RoPE, append and attention in one decode launch (affine and Int8 caches,
// G L <= 16): qkv is the projection [L][(G hkv + 2 hkv) D], rope carries its
// RoPE parameters; the rotated q rows go to q_out.
template <int BITS, int D>
static int launch_decode_rope_append(KVCache& cc, const f16* qkv, int G, int L, const RowSrc& rope,
                                     float scale, bool causal, f16* q_out, f16* out,
                                     hipStream_t stream) {
    int nc = 0;
    float* po = nullptr;
    float2* pml = nullptr;
    const int64_t W = (int64_t)(G + 2) * cc.hkv * D;
    int rc = launch_decode_partials<BITS, D>(cc, qkv, G, L, cc.offset, scale, false, &nc, &po, &pml,
                                             stream, nullptr, rope.k, rope.v, L, causal, &rope, W,
                                             q_out);
    if (rc) return rc;
    cc.offset += L;
    return launch_partial_merge(po, pml, nc, 16, 0, G * L, cc.hkv, D, G, L, out, stream);
}

int launch_turbo4_decode_append(KVCache& cc, const f16* q, int G, int L, const f16* k_new,
                                const f16* v_new, float scale, bool causal, const float* tab,
                                f16* out, hipStream_t stream) {
    QW_REQUIRE(cc.turbo4() && G * L <= 16 && cc.offset >= 1 && cc.offset + L <= cc.cap,
               QW_ERR_INVALID_ARGUMENT, "decode: Turbo4 append outside the decode-route shapes");
    int nc = 0;
    float* po = nullptr;
    float2* pml = nullptr;
    int rc = cc.D == 256 ? launch_decode_partials<4, 256, true>(cc, q, G, L, cc.offset, scale, false,
                                                                &nc, &po, &pml, stream, tab, k_new,
                                                                v_new, L, causal)
                         : launch_decode_partials<4, 128, true>(cc, q, G, L, cc.offset, scale, false,
                                                                &nc, &po, &pml, stream, tab, k_new,
                                                                v_new, L, causal);
    if (rc) return rc;
    cc.offset += L;
    return launch_t4_merge_rotate(po, pml, nc, 16, G * L, cc.hkv, cc.D, G, L, 0, false, tab, out,
                                  stream);
}

static int launch_turbo4_decode_rope_append(KVCache& cc, const f16* qkv, int G, int L,
                                            const RowSrc& rope, float scale, bool causal,
                                            const float* tab, f16* q_out, f16* out,
                                            hipStream_t stream) {
    int nc = 0;
    float* po = nullptr;
    float2* pml = nullptr;
    const int64_t W = (int64_t)(G + 2) * cc.hkv * cc.D;
    int rc = cc.D == 256 ? launch_decode_partials<4, 256, true>(cc, qkv, G, L, cc.offset, scale, false,
                                                                &nc, &po, &pml, stream, tab, rope.k,
                                                                rope.v, L, causal, &rope, W, q_out)
                         : launch_decode_partials<4, 128, true>(cc, qkv, G, L, cc.offset, scale, false,
                                                                &nc, &po, &pml, stream, tab, rope.k,
                                                                rope.v, L, causal, &rope, W, q_out);
    if (rc) return rc;
    cc.offset += L;
    return launch_t4_merge_rotate(po, pml, nc, 16, G * L, cc.hkv, cc.D, G, L, 0, false, tab, out,
                                  stream);
}

int launch_turbo4_decode(KVCache& cc, const f16* q, int G, int Tq, float scale, bool causal,
                         const float* tab, f16* out, hipStream_t stream) {
    int nc = 0;
    float* po = nullptr;
    float2* pml = nullptr;
    if (cc.D == 256) {
        int rc = launch_decode_partials<4, 256, true>(cc, q, G, Tq, cc.offset, scale, causal, &nc,
                                                      &po, &pml, stream, tab);
        if (rc) return rc;
        return launch_t4_merge_rotate(po, pml, nc, 16, G * Tq, cc.hkv, 256, G, Tq, 0, false, tab, out,
                                      stream);
    }
    int rc = launch_decode_partials<4, 128, true>(cc, q, G, Tq, cc.offset, scale, causal, &nc, &po,
                                                  &pml, stream, tab);
    if (rc) return rc;
    return launch_t4_merge_rotate(po, pml, nc, 16, G * Tq, cc.hkv, 128, G, Tq, 0, false, tab, out,
                                  stream);
}

// The same merge for many rows (block kernels' key splits): one thread an
// output element, every (m, l) and O value of its up to MAXN partials loaded
// before the first use (one memory round trip).
template <int MAXN>
__global__ __launch_bounds__(256) void merge_rows_kernel(const float* __restrict__ part_o,
                                                         const float2* __restrict__ part_ml,
                                                         int nc, int rstride, int row0, int R,
                                                         int D, int G, int Tq, int slot_bits,
                                                         f16* __restrict__ out,
                                                         float* __restrict__ out32) {
    const int h = blockIdx.y;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    // thread = place sd in a partial row (contiguous loads), holding dim d
    const int row = (int)(idx / D), sd = (int)(idx % D);
    if (row >= R) return;
    const int d = slot_bits ? v_logical_dim(sd, D, slot_bits) : sd;
    const int64_t base = (int64_t)h * nc * rstride + row;
    float v[MAXN];
    float2 ml[MAXN];
#pragma unroll
    for (int c = 0; c < MAXN; c++) {
        if (c < nc) {
            ml[c] = part_ml[base + (int64_t)c * rstride];
            v[c] = part_o[(base + (int64_t)c * rstride) * D + sd];
        } else {
            ml[c] = float2{-INFINITY, 0.0f};
            v[c] = 0.0f;
        }
    }
    float M = -INFINITY;
#pragma unroll
    for (int c = 0; c < MAXN; c++) M = fmaxf(M, ml[c].x);
    float acc = 0.0f, L = 0.0f;
#pragma unroll
    for (int c = 0; c < MAXN; c++) {
        const float f = ml[c].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((ml[c].x - M) * kLog2e);
        acc = __builtin_fmaf(f, v[c], acc);
        L = __builtin_fmaf(f, ml[c].y, L);
    }
    const int orow = row0 + row;
    const int qh = h * G + orow % G, qr = orow / G;
    const float y = L > 0.0f ? acc / L : 0.0f;
    if (out32)
        out32[((int64_t)qh * Tq + qr) * D + d] = y;
    else
        out[((int64_t)qh * Tq + qr) * D + d] = (f16)y;
}

// The same merge for many rows and many partials (key-split verify blocks):
// one workgroup a (row, KV head), 4 waves; lane n owns the SPL = D/64
// consecutive places SPL*n .. of the partial rows (one 8- or 16-byte load a
// partial) and wave w sums partials w, w + 4, ... with every load issued up
// front; the waves combine through LDS.
template <int D, int PER>
__global__ __launch_bounds__(256) void merge_rows_vec_kernel(const float* __restrict__ part_o,
                                                             const float2* __restrict__ part_ml,
                                                             int nc, int rstride, int row0, int G,
                                                             int Tq, int slot_bits,
                                                             f16* __restrict__ out,
                                                             float* __restrict__ out32) {
    constexpr int SPL = D / 64;
    typedef float vec __attribute__((ext_vector_type(SPL)));
    const int row = blockIdx.x, h = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t base = (int64_t)h * nc * rstride + row;
    vec v[PER];
    float2 ml[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int c = wave + 4 * i;
        if (c < nc) {
            ml[i] = part_ml[base + (int64_t)c * rstride];
            v[i] = *(const vec*)(part_o + (base + (int64_t)c * rstride) * D + SPL * lane);
        } else {
            ml[i] = float2{-INFINITY, 0.0f};
            v[i] = vec{};
        }
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; i++) m = fmaxf(m, ml[i].x);
    vec o = vec{};
    float l = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const float w = ml[i].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((ml[i].x - m) * kLog2e);
        o += w * v[i];
        l = __builtin_fmaf(w, ml[i].y, l);
    }
    __shared__ float2 sm_ml[4];
    __shared__ vec sm_o[4][64];
    if (lane == 0) sm_ml[wave] = float2{m, l};
    sm_o[wave][lane] = o;
    __syncthreads();
    if (wave == 0) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++) M = fmaxf(M, sm_ml[w].x);
        vec O = vec{};
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float f = sm_ml[w].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((sm_ml[w].x - M) * kLog2e);
            O += f * sm_o[w][lane];
            L = __builtin_fmaf(f, sm_ml[w].y, L);
        }
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        const int orow = row0 + row;
        const int qh = h * G + orow % G, qr = orow / G;
        const int64_t obase = ((int64_t)qh * Tq + qr) * D;
#pragma unroll
        for (int j = 0; j < SPL; j++) {
            const int sd = SPL * lane + j;
            const int d = slot_bits ? v_logical_dim(sd, D, slot_bits) : sd;
            if (out32)
                out32[obase + d] = O[j] * inv;
            else
                out[obase + d] = (f16)(O[j] * inv);
        }
    }
}

template <int D>
static void launch_merge_rows_vec(const float* part_o, const float2* part_ml, int nc, int rstride,
                                  int row0, int R, int hkv, int G, int Tq, int slot_bits, f16* out,
                                  float* out32, hipStream_t stream) {
    const dim3 grid(R, hkv);
    switch (merge_per(nc)) {
        case 4:
            hipLaunchKernelGGL((merge_rows_vec_kernel<D, 4>), grid, dim3(256), 0, stream, part_o,
                               part_ml, nc, rstride, row0, G, Tq, slot_bits, out, out32);
            break;
        case 8:
            hipLaunchKernelGGL((merge_rows_vec_kernel<D, 8>), grid, dim3(256), 0, stream, part_o,
                               part_ml, nc, rstride, row0, G, Tq, slot_bits, out, out32);
            break;
        case 16:
            hipLaunchKernelGGL((merge_rows_vec_kernel<D, 16>), grid, dim3(256), 0, stream, part_o,
                               part_ml, nc, rstride, row0, G, Tq, slot_bits, out, out32);
            break;
        case 32:
            hipLaunchKernelGGL((merge_rows_vec_kernel<D, 32>), grid, dim3(256), 0, stream, part_o,
                               part_ml, nc, rstride, row0, G, Tq, slot_bits, out, out32);
            break;
        default:
            hipLaunchKernelGGL((merge_rows_vec_kernel<D, kMergeMaxPer>), grid, dim3(256), 0, stream,
                               part_o, part_ml, nc, rstride, row0, G, Tq, slot_bits, out, out32);
    }
}

// The merge of the block kernel's fp16 partials (normalized rows, place
// NT * r + mm = slot 16 mm + r): one workgroup a (row, KV head), kMRW waves;
// lane n owns places SPL*n .. +SPL-1 (one 4- or 8-byte load a partial), wave
// w sums partials w, w + kMRW, ... weighted by e^(m_c - m) l_c, and the waves
// combine through LDS. Eight waves measured c4 attention 47.9 -> 46.8 us
// against four, the served verify blocks unchanged (A/B in one run).
#ifndef QW_MERGE_ROWS_WAVES
#define QW_MERGE_ROWS_WAVES 8
#endif
constexpr int kMRW = QW_MERGE_ROWS_WAVES;

template <int D, int PER>
__global__ __launch_bounds__(64 * kMRW) void merge_rows_h_kernel(const f16* __restrict__ part_o,
                                                           const float2* __restrict__ part_ml,
                                                           int nc, int rstride, int row0, int G,
                                                           int Tq, int slot_bits,
                                                           f16* __restrict__ out) {
    constexpr int SPL = D / 64, NT = D / 16;
    typedef _Float16 hvec __attribute__((ext_vector_type(SPL)));
    typedef float vec __attribute__((ext_vector_type(SPL)));
    const int row = blockIdx.x, h = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t base = (int64_t)h * nc * rstride + row;
    hvec v[PER];
    float2 ml[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int c = wave + kMRW * i;
        if (c < nc) {
            ml[i] = part_ml[base + (int64_t)c * rstride];
            v[i] = *(const hvec*)(part_o + (base + (int64_t)c * rstride) * D + SPL * lane);
        } else {
            ml[i] = float2{-INFINITY, 0.0f};
            v[i] = hvec{};
        }
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; i++) m = fmaxf(m, ml[i].x);
    vec o = vec{};
    float l = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const float w = ml[i].x == -INFINITY
                            ? 0.0f
                            : __builtin_amdgcn_exp2f((ml[i].x - m) * kLog2e) * ml[i].y;
#pragma unroll
        for (int j = 0; j < SPL; j++) o[j] = __builtin_fmaf(w, (float)v[i][j], o[j]);
        l += w;
    }
    __shared__ float2 sm_ml[kMRW];
    __shared__ vec sm_o[kMRW][64];
    if (lane == 0) sm_ml[wave] = float2{m, l};
    sm_o[wave][lane] = o;
    __syncthreads();
    if (wave == 0) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kMRW; w++) M = fmaxf(M, sm_ml[w].x);
        vec O = vec{};
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < kMRW; w++) {
            const float f = sm_ml[w].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((sm_ml[w].x - M) * kLog2e);
            O += f * sm_o[w][lane];
            L = __builtin_fmaf(f, sm_ml[w].y, L);
        }
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        const int orow = row0 + row;
        const int qh = h * G + orow % G, qr = orow / G;
        const int64_t obase = ((int64_t)qh * Tq + qr) * D;
#pragma unroll
        for (int j = 0; j < SPL; j++) {
            const int p = SPL * lane + j;
            const int sd = 16 * (p % NT) + p / NT;
            const int d = slot_bits ? v_logical_dim(sd, D, slot_bits) : sd;
            out[obase + d] = (f16)(O[j] * inv);
        }
    }
}

template <int D>
static void launch_merge_rows_h(const f16* part_o, const float2* part_ml, int nc, int rstride,
                                int row0, int R, int hkv, int G, int Tq, int slot_bits, f16* out,
                                hipStream_t stream) {
    const dim3 grid(R, hkv);
    switch (std::max(4, merge_per(nc) * 4 / kMRW)) {
        case 4:
            hipLaunchKernelGGL((merge_rows_h_kernel<D, 4>), grid, dim3(64 * kMRW), 0, stream, part_o,
                               part_ml, nc, rstride, row0, G, Tq, slot_bits, out);
            break;
        case 8:
            hipLaunchKernelGGL((merge_rows_h_kernel<D, 8>), grid, dim3(64 * kMRW), 0, stream, part_o,
                               part_ml, nc, rstride, row0, G, Tq, slot_bits, out);
            break;
        case 16:
            hipLaunchKernelGGL((merge_rows_h_kernel<D, 16>), grid, dim3(64 * kMRW), 0, stream, part_o,
                               part_ml, nc, rstride, row0, G, Tq, slot_bits, out);
            break;
        case 32:
            hipLaunchKernelGGL((merge_rows_h_kernel<D, 32>), grid, dim3(64 * kMRW), 0, stream, part_o,
                               part_ml, nc, rstride, row0, G, Tq, slot_bits, out);
            break;
        default:
            hipLaunchKernelGGL((merge_rows_h_kernel<D, kMergeMaxPer>), grid, dim3(64 * kMRW), 0, stream,
                               part_o, part_ml, nc, rstride, row0, G, Tq, slot_bits, out);
    }
}

int launch_partial_merge_h(const f16* part_o, const float2* part_ml, int nc, int rstride, int row0,
                           int R, int hkv, int D, int G, int Tq, f16* out, hipStream_t stream,
                           int slot_bits) {
    QW_REQUIRE(nc >= 1 && nc <= 4 * kMergeMaxPer, QW_ERR_INVALID_ARGUMENT,
               "merge: partial count out of range");
    QW_REQUIRE(D == 128 || D == 256, QW_ERR_INVALID_ARGUMENT, "merge: fp16 partials need D 128/256");
    if (D == 256)
        launch_merge_rows_h<256>(part_o, part_ml, nc, rstride, row0, R, hkv, G, Tq, slot_bits, out,
                                 stream);
    else
        launch_merge_rows_h<128>(part_o, part_ml, nc, rstride, row0, R, hkv, G, Tq, slot_bits, out,
                                 stream);
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

#ifndef QW_MERGE_VEC
#define QW_MERGE_VEC 1
#endif

int launch_partial_merge(const float* part_o, const float2* part_ml, int nc, int rstride, int row0,
                         int R, int hkv, int D, int G, int Tq, f16* out, hipStream_t stream,
                         int slot_bits, float* out32) {
    QW_REQUIRE(nc >= 1 && nc <= 4 * kMergeMaxPer, QW_ERR_INVALID_ARGUMENT,
               "merge: partial count out of range");
    if (QW_MERGE_VEC && R > 16 && nc > 8 && (D == 128 || D == 256)) {
        if (D == 256)
            launch_merge_rows_vec<256>(part_o, part_ml, nc, rstride, row0, R, hkv, G, Tq, slot_bits,
                                       out, out32, stream);
        else
            launch_merge_rows_vec<128>(part_o, part_ml, nc, rstride, row0, R, hkv, G, Tq, slot_bits,
                                       out, out32, stream);
        QW_HIP_CHECK(hipGetLastError());
        return QW_OK;
    }
    if (R > 16 && nc <= 64) {
        const int64_t n = (int64_t)R * D;
        const dim3 grid((unsigned)((n + 255) / 256), hkv);
        if (nc <= 8)
            hipLaunchKernelGGL(merge_rows_kernel<8>, grid, dim3(256), 0, stream, part_o, part_ml, nc,
                               rstride, row0, R, D, G, Tq, slot_bits, out, out32);
        else
            hipLaunchKernelGGL(merge_rows_kernel<64>, grid, dim3(256), 0, stream, part_o, part_ml,
                               nc, rstride, row0, R, D, G, Tq, slot_bits, out, out32);
        QW_HIP_CHECK(hipGetLastError());
        return QW_OK;
    }
    const dim3 grid(R, hkv, D / 64);
    switch (std::max(4, merge_per(nc) * 4 / kMW)) {
        case 4:
            hipLaunchKernelGGL(decode_merge_kernel<4>, grid, dim3(64 * kMW), 0, stream, part_o, part_ml,
                               nc, rstride, row0, D, G, Tq, slot_bits, out, out32);
            break;
        case 8:
            hipLaunchKernelGGL(decode_merge_kernel<8>, grid, dim3(64 * kMW), 0, stream, part_o, part_ml,
                               nc, rstride, row0, D, G, Tq, slot_bits, out, out32);
            break;
        case 16:
            hipLaunchKernelGGL(decode_merge_kernel<16>, grid, dim3(64 * kMW), 0, stream, part_o, part_ml,
                               nc, rstride, row0, D, G, Tq, slot_bits, out, out32);
            break;
        case 32:
            hipLaunchKernelGGL(decode_merge_kernel<32>, grid, dim3(64 * kMW), 0, stream, part_o, part_ml,
                               nc, rstride, row0, D, G, Tq, slot_bits, out, out32);
            break;
        default:
            hipLaunchKernelGGL(decode_merge_kernel<kMergeMaxPer>, grid, dim3(64 * kMW), 0, stream, part_o,
                               part_ml, nc, rstride, row0, D, G, Tq, slot_bits, out, out32);
    }
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

int launch_attention(KVCache& cc, const void* q, int n_q_heads, int n_rows, float scale,
                     bool causal, void* out, hipStream_t stream) {
    if (cc.turbo4()) return turbo4_attention(cc, q, n_q_heads, n_rows, scale, causal, out, stream);
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

// 1: decode-route calls (and Turbo4 decode-route calls) append their rows in
// the decode launch's append unit; 0: a separate append first.
#ifndef QW_DECODE_APPEND
#define QW_DECODE_APPEND 1
#endif

int KVCache::update_and_attention(const void* q, int n_q_heads, int n_rows, const void* k_new,
                                  const void* v_new, float scale, bool causal, void* out,
                                  hipStream_t stream) {
    QW_REQUIRE(q && out && k_new && v_new, QW_ERR_INVALID_ARGUMENT,
               "update_and_attention: null pointer");
    QW_REQUIRE(n_q_heads > 0 && n_q_heads % hkv == 0 && n_rows > 0, QW_ERR_INVALID_ARGUMENT,
               "update_and_attention: bad head or row geometry");
    const int G = n_q_heads / hkv;
    if (turbo4())
        return turbo4_update_and_attention(*this, q, n_q_heads, n_rows, k_new, v_new, scale, causal,
                                           out, stream);
    if (QW_DECODE_APPEND && affine() && G * n_rows <= 16 && offset >= 1) {
        // decode and short verify blocks: the append unit rides in the decode launch
        DeviceGuard dg(device);
        QW_REQUIRE(dg.ok, QW_ERR_HIP, "update_and_attention: hipSetDevice failed");
        if (offset + n_rows > cap) {
            int rc = reserve(std::max(offset + n_rows, cap + cap / 2), stream);
            if (rc) return rc;
        }
        const f16 *qq = (const f16*)q, *kn = (const f16*)k_new, *vn = (const f16*)v_new;
        f16* oo = (f16*)out;
        if (D == 256)
            return bits == 4 ? launch_decode_append<4, 256>(*this, qq, G, n_rows, kn, vn, scale, causal, oo, stream)
                             : launch_decode_append<8, 256>(*this, qq, G, n_rows, kn, vn, scale, causal, oo, stream);
        return bits == 4 ? launch_decode_append<4, 128>(*this, qq, G, n_rows, kn, vn, scale, causal, oo, stream)
                         : launch_decode_append<8, 128>(*this, qq, G, n_rows, kn, vn, scale, causal, oo, stream);
    }
    if (block_append_fits(*this, G, n_rows)) {
        // verify blocks: the append rides in the block kernel's launch
        DeviceGuard dg(device);
        QW_REQUIRE(dg.ok, QW_ERR_HIP, "update_and_attention: hipSetDevice failed");
        if (offset + n_rows > cap) {
            int rc = reserve(std::max(offset + n_rows, cap + cap / 2), stream);
            if (rc) return rc;
        }
        return launch_block_append_attention(*this, (const f16*)q, G, n_rows, (const f16*)k_new,
                                             (const f16*)v_new, scale, causal, (f16*)out, stream);
    }
    int rc = update(k_new, v_new, n_rows, stream);
    if (rc) return rc;
    return launch_attention(*this, q, n_q_heads, n_rows, scale, causal, out, stream);
}

// RoPE, append and attention of one projection: what rope_update (q rotated
// into q_out, K rotated into the cache, V appended) followed by attention on
// q_out computes. With rope_dims a multiple of 16 it runs in one launch plus
// the merge where update_and_attention would append in its attention launch:
// decode-route shapes (affine, Int8 and Turbo4 caches, at most 16 rows a KV
// head: the decode launch) and verify blocks (affine and Int8 blocks of 2..128
// rows a KV head, Turbo4's fused verify pass: the block launch). Its
// workgroups rotate their q rows in the prologue; the append workgroups append
// the rotated K with V and write q_out. Other shapes run the two calls.
int KVCache::rope_update_and_attention(const void* qkv, int n_q_heads, int n_tokens, int rope_dims,
                                       int traditional, float rope_base, float rope_scale,
                                       int position0, float scale, bool causal, void* q_out,
                                       void* out, hipStream_t stream) {
    QW_REQUIRE(qkv && q_out && out, QW_ERR_INVALID_ARGUMENT, "rope_update_and_attention: null buffer");
    QW_REQUIRE(n_q_heads > 0 && n_q_heads % hkv == 0 && n_tokens > 0, QW_ERR_INVALID_ARGUMENT,
               "rope_update_and_attention: bad head or row geometry");
    QW_REQUIRE(rope_dims >= 0 && rope_dims <= D && rope_dims % 2 == 0 && rope_base > 0.0f,
               QW_ERR_INVALID_ARGUMENT, "rope_update_and_attention: bad RoPE parameters");
    const int G = n_q_heads / hkv, T = offset + n_tokens;
    const bool t4_decode = turbo4() && turbo4_decode_route(*this, causal, n_tokens, G);
    const bool decode = QW_DECODE_APPEND && rope_dims % 16 == 0 && G * n_tokens <= 16 &&
                        offset >= 1 && (affine() || t4_decode);
    const bool block = rope_dims % 16 == 0 && !decode &&
                       (block_append_fits(*this, G, n_tokens) ||
                        (turbo4() && turbo4_fused_append_route(*this, causal, n_tokens, G)));
    if (!decode && !block) {
        int rc = rope_update(qkv, n_q_heads, n_tokens, rope_dims, traditional, rope_base, rope_scale,
                             position0, q_out, stream);
        if (rc) return rc;
        return launch_attention(*this, q_out, n_q_heads, n_tokens, scale, causal, out, stream);
    }
    DeviceGuard dg(device);
    QW_REQUIRE(dg.ok, QW_ERR_HIP, "rope_update_and_attention: hipSetDevice failed");
    if (T > cap) {
        int rc = reserve(std::max(T, cap + cap / 2), stream);
        if (rc) return rc;
    }
    const int64_t W = (int64_t)(n_q_heads + 2 * hkv) * D;
    RowSrc rs;
    rs.k = (const f16*)qkv + (int64_t)n_q_heads * D;
    rs.v = (const f16*)qkv + (int64_t)(n_q_heads + hkv) * D;
    rs.row_stride = W;
    rs.head_stride = D;
    rs.rope_dims = rope_dims;
    rs.traditional = traditional ? 1 : 0;
    rs.position0 = position0;
    rs.log2_base = std::log2(rope_base);
    rs.scale = rope_scale;
    const f16* q = (const f16*)qkv;
    f16 *qo = (f16*)q_out, *oo = (f16*)out;
    if (block) {
        if (turbo4())
            return launch_block_append_attention_t4(*this, q, G, n_tokens, rs.k, rs.v, scale, causal,
                                                    true, t4_tables, oo, stream, &rs, qo);
        return launch_block_append_attention(*this, q, G, n_tokens, rs.k, rs.v, scale, causal, oo,
                                             stream, &rs, qo);
    }
    if (turbo4())
        return launch_turbo4_decode_rope_append(*this, q, G, n_tokens, rs, scale, causal, t4_tables,
                                                qo, oo, stream);
    if (D == 256)
        return bits == 4 ? launch_decode_rope_append<4, 256>(*this, q, G, n_tokens, rs, scale, causal, qo, oo, stream)
                         : launch_decode_rope_append<8, 256>(*this, q, G, n_tokens, rs, scale, causal, qo, oo, stream);
    return bits == 4 ? launch_decode_rope_append<4, 128>(*this, q, G, n_tokens, rs, scale, causal, qo, oo, stream)
                     : launch_decode_rope_append<8, 128>(*this, q, G, n_tokens, rs, scale, causal, qo, oo, stream);
}

}  // namespace qw
