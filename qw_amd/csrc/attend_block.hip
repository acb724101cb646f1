// attend_block.hip - fused dequant-in-attention for many query rows per KV
// head (G * n_rows > 16): speculative verify blocks and chunked prefill, gfx950.
//
// Reference path replaced: KVCache::update_and_turbo4_causal_attention
// (crates/mlxcel-core/src/cache.rs:3520-3589) and, for prefill chunks,
// update_and_fetch + layers::attention / chunked_causal_attention
// (cache.rs:2709-2834, crates/mlxcel-core/src/layers.rs:4010-4339), which
// dequantize the whole cache and run MLX SDPA. Semantics are MLX's SDPA on the
// dequantized cache: scores f16(q' . k) with q' = f16(f16(scale) * q), fp32
// softmax, bottom-right causal alignment (row r sees keys <= T - Tq + r,
// cache.rs:3512-3519, turbo4_attention.cpp:96).
//
// Design: the K/V tile of a KV head is dequantized ONCE per workgroup into
// LDS (fp16, MLX-exact values) and shared by all of the workgroup's query
// rows, the GQA heads of the group included:
//   grid (key splits, query tiles, kv heads); NW waves; wave w owns 16 query
//   rows (row index r * G + head-in-group, the decode kernel's order).
//   Per tile of KT = 16384 / D keys (64 at D = 256):
//     every thread loads one 32-dim K slice and one 4-dim V slice of the tile
//     (codes + scale/bias) for the NEXT tile into registers, dequantizes the
//     current one into LDS (K rows, V 8-key blocks), then all waves run
//       S^T = K . Q'^T   v_mfma_f32_16x16x32_f16, A = K rows from LDS,
//                        B = the wave's 16 query rows held in registers,
//       online softmax on the fp16-rounded scores (exp2, lazy reference),
//       O += P . V       A = P straight from the S^T registers, B = 8 keys
//                        of one V dim from LDS (one ds_read_b128 per MFMA).
//   One key split: the workgroup writes normalized fp16 rows. Several:
//   fp32 partials (m, l, O) and the shared split-K merge kernel.
#include <algorithm>

#include "dequant.hpp"
#include "kv_cache.hpp"

namespace qw {

struct BlockArgs {
    const uint32_t* k_data;
    const uint32_t* k_params;
    const uint32_t* v_data;
    const uint32_t* v_params;
    const int* fast_flag;
    const f16* q;       // [hq][Tq][D]
    f16* out;           // [hq][Tq][D], written directly when n_split == 1
    float* part_o;      // [hkv][n_split][R][D]
    float2* part_ml;    // [hkv][n_split][R]
    int cap, T, Tq, G, R, causal, n_split, tiles_per_split;
    float scale_h;      // f16(scale) as float
};

template <int D>
struct BlockShape {
    static constexpr int KT = 16384 / D;  // keys a tile (64 at D=256, 128 at D=128)
    static constexpr int NSUB = KT / 32;  // 32-key sub-blocks a tile
    static constexpr int NM = D / 32;     // QK MFMAs per 16-key tile
    static constexpr int NT = D / 16;     // P.V MFMAs (16-dim output tiles)
    static constexpr int NG = D / 64;     // affine groups a row
    static constexpr int TPR = D / 32;    // threads a K row (32 dims each)
    static constexpr int LTPR = TPR == 8 ? 3 : 2;
    static constexpr int TPB = D / 4;     // threads a V block (4 slots each)
};

// LDS layouts (16-byte chunks, no padding; XOR/rotation swizzles keep every
// 16-lane phase of a ds_read_b128 / ds_write_b128 on 16 distinct bank groups):
//   K  [key][D/8 chunks]: chunk c of key k sits at c ^ kswz(k). The QK A
//      operand reads keys 8(r>>2) + 4t + (r&3) (r = lane & 15) at one chunk,
//      and kswz maps those 16 keys to 16 distinct values.
//   V  [8-key block][D slots][8 keys]: slot s (the V plane's physical dim
//      order) sits at vswz(s) = (s & ~3) | ((s + (s >> 4)) & 3). A lane writes
//      slots 4j..4j+3 of its block; the P.V B operand reads slots 16mm + r.
__device__ __forceinline__ int kswz(int key) { return (key & 3) | (((key >> 3) & 3) << 2); }
__device__ __forceinline__ int vswz(int s) { return (s & ~3) | ((s + (s >> 4)) & 3); }

constexpr int kBlockWaves = 8;  // 128 query rows a workgroup

// Logical dim of physical slot `slot` of a V block (inverse of v_phys_dim).
__device__ __forceinline__ int v_logical_dim(int slot, int D, int bits) {
    const int dpl = D / 16;
    const int e = bits == 4 ? 4 : (bits == 8 ? 2 : 1);
    const int i = slot % e, n = (slot / e) % 16, j = slot / (16 * e);
    return n * dpl + e * j + i;
}

template <int BITS, int D, int NW, bool FAST>
__device__ __forceinline__ void block_body(const BlockArgs& a, f16* sK, f16* sV) {
    using S = BlockShape<D>;
    constexpr int KT = S::KT, NSUB = S::NSUB, NM = S::NM, NT = S::NT, NG = S::NG;
    constexpr int TPR = S::TPR, LTPR = S::LTPR, TPB = S::TPB;
    constexpr bool AFF = BITS != 16;
    constexpr int KU = BITS / 4;  // u32x4 loads a thread's 32-dim K slice / 4-dim V slice
    static_assert(KT * TPR == 64 * NW && (KT / 8) * TPB == 64 * NW, "one slice a thread");

    const int sp = blockIdx.x, qt = blockIdx.y, h = blockIdx.z;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r16 = lane & 15, g = lane >> 4;
    const uint32_t magic = vconst(kMagic);

    // ---- key range of this workgroup: its split, cut at the last key any of
    // its rows can see.
    const int row0 = qt * 16 * NW;
    const int row_last = min(a.R, row0 + 16 * NW) - 1;
    const int wg_lim = a.causal ? a.T - a.Tq + row_last / a.G : a.T - 1;
    const int n_tiles = (a.T + KT - 1) / KT;
    const int t0 = sp * a.tiles_per_split;
    const int t1 = min(min(n_tiles, t0 + a.tiles_per_split), wg_lim / KT + 1);

    // ---- the wave's 16 query rows as the B operand of S^T = K . Q'^T
    // (col = query row r16, k-group g = dims 32m + 8g .. +7 of MFMA step m, in
    // the order the LDS K row holds them).
    const int rho = row0 + 16 * wave + r16;
    const bool row_ok = rho < a.R;
    const int wave_last = min(a.R, row0 + 16 * wave + 16) - 1;
    const bool wave_live = row0 + 16 * wave < a.R;
    const int wave_lim = a.causal ? a.T - a.Tq + wave_last / a.G : a.T - 1;
    const int lim = a.causal ? a.T - a.Tq + (row_ok ? rho / a.G : 0) : a.T - 1;
    half8 qb[NM];
    {
        const int rr = row_ok ? rho : 0;
        const f16* qrow = a.q + ((int64_t)(h * a.G + rr % a.G) * a.Tq + rr / a.G) * D;
        const f16 sc = row_ok ? (f16)a.scale_h : (f16)0.0f;
        const half2v sc2 = {sc, sc};
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const u32x4 w = *(const u32x4*)(qrow + 32 * m + 8 * g);
            u32x4 o;
            if constexpr (BITS == 4) {
                // 4-bit K rows sit in LDS as dim pairs (0,4),(1,5),(2,6),(3,7).
                o.x = __builtin_amdgcn_perm(w.z, w.x, 0x05040100u);
                o.y = __builtin_amdgcn_perm(w.z, w.x, 0x07060302u);
                o.z = __builtin_amdgcn_perm(w.w, w.y, 0x05040100u);
                o.w = __builtin_amdgcn_perm(w.w, w.y, 0x07060302u);
            } else {
                o = w;
            }
            // q' = f16(f16(scale) * q), MLX's fp16 multiply; padding rows are 0.
            u32x4 y;
            y.x = __builtin_bit_cast(uint32_t, h2(o.x) * sc2);
            y.y = __builtin_bit_cast(uint32_t, h2(o.y) * sc2);
            y.z = __builtin_bit_cast(uint32_t, h2(o.z) * sc2);
            y.w = __builtin_bit_cast(uint32_t, h2(o.w) * sc2);
            qb[m] = __builtin_bit_cast(half8, y);
        }
    }

    // ---- tile loads: thread -> (key kk, 32-dim slice q32) of K and
    // (8-key block vb, 4 physical dim slots starting at 4 * vj) of V. Lanes
    // 4i..4i+3 take 4 keys of one slice so a 16-lane phase writes 4 keys x 4
    // slices (distinct banks under kswz).
    const int q32 = (tid >> 2) & (TPR - 1);
    const int kk = (tid & 3) | ((tid >> (2 + LTPR)) << 2);
    const int vb = tid / TPB, vj = tid % TPB;
    struct Stage {
        u32x4 kc[KU];
        uint32_t kp;
        u32x4 vc[KU];
        u32x4 vp[2];
    };
    const int64_t krow_words = (int64_t)D * BITS / 32;
    const int64_t vblk_words = (int64_t)D * BITS / 4;
    const int vgrp = v_logical_dim(4 * vj, D, BITS) / 64;
    auto load = [&](Stage& st, int t) {
        const int64_t row = (int64_t)h * a.cap + (int64_t)t * KT + kk;
        const u32x4* ksrc = (const u32x4*)(a.k_data + row * krow_words) + KU * q32;
#pragma unroll
        for (int u = 0; u < KU; u++) st.kc[u] = ksrc[u];
        if constexpr (AFF) st.kp = a.k_params[row * NG + k_param_slot(q32 >> 1, NG)];
        const int64_t blk = (int64_t)h * (a.cap / 8) + (int64_t)t * (KT / 8) + vb;
        const u32x4* vsrc = (const u32x4*)(a.v_data + blk * vblk_words) + KU * vj;
#pragma unroll
        for (int u = 0; u < KU; u++) st.vc[u] = vsrc[u];
        if constexpr (AFF) {
            const u32x4* psrc = (const u32x4*)(a.v_params + (blk * NG + vgrp) * 8);
            st.vp[0] = psrc[0];
            st.vp[1] = psrc[1];
        }
    };
    // Dequantize a stage into LDS: K row kk, chunks 4 q32 .. +3 (dims in the
    // order of the Q operand); V block vb, slots 4 vj .. +3 (8 keys each).
    half8* const sK8 = (half8*)sK;
    half8* const sV8 = (half8*)sV;
    auto store = [&](const Stage& st) {
        half8* krow = sK8 + kk * (D / 8);
        const int kx = kswz(kk);
        if constexpr (BITS == 4) {
            const half2v sb = h2(st.kp);
            const half2v s = {sb.x, sb.x}, b = {sb.y, sb.y};
            const PairConsts pc = make_consts<FAST, 4>(s, s, s, s, b, b, b, b);
#pragma unroll
            for (int w = 0; w < 4; w++) krow[(4 * q32 + w) ^ kx] = deq4<FAST>(st.kc[0][w], pc, magic);
        } else if constexpr (BITS == 8) {
            const half2v sb = h2(st.kp);
            const half2v s = {sb.x, sb.x}, b = {sb.y, sb.y};
            const PairConsts pc = make_consts<FAST, 8>(s, s, s, s, b, b, b, b);
#pragma unroll
            for (int w = 0; w < 4; w++)
                krow[(4 * q32 + w) ^ kx] =
                    deq8<FAST>(st.kc[w / 2][2 * (w % 2)], st.kc[w / 2][2 * (w % 2) + 1], pc);
        } else {
#pragma unroll
            for (int w = 0; w < 4; w++) krow[(4 * q32 + w) ^ kx] = as_h8(st.kc[w]);
        }
        PairConsts vc;
        if constexpr (AFF)
            vc = make_consts<FAST, BITS>(h2(st.vp[0][0]), h2(st.vp[0][1]), h2(st.vp[0][2]),
                                         h2(st.vp[0][3]), h2(st.vp[1][0]), h2(st.vp[1][1]),
                                         h2(st.vp[1][2]), h2(st.vp[1][3]));
        half8* vblk = sV8 + vb * D;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            half8 y;
            if constexpr (BITS == 4)
                y = deq4<FAST>(st.vc[0][e], vc, magic);
            else if constexpr (BITS == 8)
                y = deq8<FAST>(st.vc[e / 2][2 * (e % 2)], st.vc[e / 2][2 * (e % 2) + 1], vc);
            else
                y = as_h8(st.vc[e]);
            vblk[vswz(4 * vj + e)] = y;
        }
    };

    float m_run = -INFINITY;  // softmax reference of column r16 (natural units)
    float l_run = 0.0f;       // this lane's share of the column sum
    float4v acc_o[NT];
#pragma unroll
    for (int mm = 0; mm < NT; mm++) acc_o[mm] = float4v{0.f, 0.f, 0.f, 0.f};

    // One 32-key sub-block (keys kb .. kb+31, LDS rows 32u ..) of the tile.
    auto sub_block = [&](int u, int kb) {
        // S^T: A row r16 of MFMA tile tt is key 8(r16>>2) + 4tt + (r16&3), so
        // lane (g, r16) ends up with keys 8g + 4tt + i of column r16.
        const int key0 = 32 * u + 8 * (r16 >> 2) + (r16 & 3);  // tile 1: key0 + 4
        const half8* k0 = sK8 + key0 * (D / 8);
        const half8* k1 = k0 + 4 * (D / 8);
        const int kx = kswz(key0);  // == kswz(key0 + 4)
        float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < NM; m++) {
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0[(4 * m + g) ^ kx], qb[m], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1[(4 * m + g) ^ kx], qb[m], acc1, 0, 0, 0);
        }
        float sc[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int ka = kb + 8 * g + i, kc = ka + 4;
            // MLX rounds the score matrix to fp16 before the softmax.
            sc[i] = row_ok && ka <= lim ? (float)(f16)acc0[i] : -INFINITY;
            sc[4 + i] = row_ok && kc <= lim ? (float)(f16)acc1[i] : -INFINITY;
        }
        // Online softmax with a lazy reference: m_run moves only when a score
        // exceeds it by more than 5.5 (so p <= e^5.5 stays well inside fp16).
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
                for (int mm = 0; mm < NT; mm++)
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
        // O += P . V: B = slot 16mm + r16 (column r16 of output tile mm) of
        // V block 4u + g, i.e. keys 8g .. 8g+7 of the sub-block.
        const half8* vb8 = sV8 + (4 * u + g) * D;
#pragma unroll
        for (int mm = 0; mm < NT; mm++)
            acc_o[mm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pop, vb8[vswz(16 * mm + r16)],
                                                               acc_o[mm], 0, 0, 0);
    };

    Stage st;
    if (t0 < t1) load(st, t0);
    for (int t = t0; t < t1; t++) {
        __syncthreads();  // every wave is done reading the previous tile
        store(st);
        if (t + 1 < t1) load(st, t + 1);
        __syncthreads();
        if (wave_live) {
#pragma unroll
            for (int u = 0; u < NSUB; u++) {
                const int kb = t * KT + 32 * u;
                if (kb <= wave_lim) sub_block(u, kb);
            }
        }
    }

    // ---- epilogue: per column, the row sum over the 4 lane groups.
    float lsum = l_run;
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    const int rbase = row0 + 16 * wave + 4 * g;  // rows of acc_o[.][i] are rbase + i
    if (a.n_split == 1) {
        float inv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float l = __shfl(lsum, 4 * g + i);
            inv[i] = l > 0.0f ? 1.0f / l : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = rbase + i;
            if (row >= a.R) continue;
            f16* orow = a.out + ((int64_t)(h * a.G + row % a.G) * a.Tq + row / a.G) * D;
#pragma unroll
            for (int mm = 0; mm < NT; mm++)
                orow[v_logical_dim(16 * mm + r16, D, BITS)] = (f16)(acc_o[mm][i] * inv[i]);
        }
    } else {
        const int64_t pbase = ((int64_t)h * a.n_split + sp) * a.R;
        if (g == 0 && row_ok) a.part_ml[pbase + rho] = float2{m_run, lsum};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = rbase + i;
            if (row >= a.R) continue;
            float* prow = a.part_o + (pbase + row) * D;
#pragma unroll
            for (int mm = 0; mm < NT; mm++) prow[v_logical_dim(16 * mm + r16, D, BITS)] = acc_o[mm][i];
        }
    }
}

template <int BITS, int D>
__global__ __launch_bounds__(64 * kBlockWaves, 1) void attend_block_kernel(BlockArgs a) {
    using S = BlockShape<D>;
    __shared__ __attribute__((aligned(16))) f16 sK[S::KT * D];
    __shared__ __attribute__((aligned(16))) f16 sV[S::KT * D];
    if (BITS == 16 || *a.fast_flag != 0)
        block_body<BITS, D, kBlockWaves, true>(a, sK, sV);
    else
        block_body<BITS, D, kBlockWaves, false>(a, sK, sV);
}

template <int BITS, int D>
static int launch_block_bits(KVCache& cc, const f16* q, int G, int Tq, float scale, bool causal,
                             f16* out, hipStream_t stream) {
    using S = BlockShape<D>;
    constexpr int NW = kBlockWaves;
    const int T = cc.offset;
    const int R = G * Tq;
    const int n_qt = (R + 16 * NW - 1) / (16 * NW);
    const int n_tiles = (T + S::KT - 1) / S::KT;
    // Split the keys only while the (query tile, head) grid leaves CUs idle;
    // at least 4 tiles a split, at most 256 partials a row.
    const int units = n_qt * cc.hkv;
    int n_split = 1;
    if (units < 256)
        n_split = std::max(1, std::min({256 / units, (n_tiles + 3) / 4, 256}));
    const int tps = (n_tiles + n_split - 1) / n_split;
    n_split = (n_tiles + tps - 1) / tps;

    BlockArgs a;
    a.k_data = (const uint32_t*)cc.k_data;
    a.k_params = cc.k_params;
    a.v_data = (const uint32_t*)cc.v_data;
    a.v_params = cc.v_params;
    a.fast_flag = cc.fast_flag;
    a.q = q;
    a.out = out;
    a.part_o = nullptr;
    a.part_ml = nullptr;
    a.cap = cc.cap;
    a.T = T;
    a.Tq = Tq;
    a.G = G;
    a.R = R;
    a.causal = causal ? 1 : 0;
    a.n_split = n_split;
    a.tiles_per_split = tps;
    a.scale_h = (float)(f16)scale;
    if (n_split > 1) {
        const size_t o_bytes = (size_t)cc.hkv * n_split * R * D * sizeof(float);
        const size_t need = o_bytes + (size_t)cc.hkv * n_split * R * sizeof(float2);
        int rc = cc.ensure_workspace(need);
        if (rc) return rc;
        a.part_o = (float*)cc.ws;
        a.part_ml = (float2*)((char*)cc.ws + o_bytes);
    }
    hipLaunchKernelGGL((attend_block_kernel<BITS, D>), dim3(n_split, n_qt, cc.hkv),
                       dim3(64 * NW), 0, stream, a);
    QW_HIP_CHECK(hipGetLastError());
    if (n_split > 1)
        return launch_partial_merge(a.part_o, a.part_ml, n_split, R, R, cc.hkv, D, G, Tq, out,
                                    stream);
    return QW_OK;
}

int launch_block_attention(KVCache& cc, const f16* q, int G, int n_rows, float scale, bool causal,
                           f16* out, hipStream_t stream) {
    if (cc.D == 256) {
        if (cc.bits == 4) return launch_block_bits<4, 256>(cc, q, G, n_rows, scale, causal, out, stream);
        if (cc.bits == 8) return launch_block_bits<8, 256>(cc, q, G, n_rows, scale, causal, out, stream);
        return launch_block_bits<16, 256>(cc, q, G, n_rows, scale, causal, out, stream);
    }
    if (cc.bits == 4) return launch_block_bits<4, 128>(cc, q, G, n_rows, scale, causal, out, stream);
    if (cc.bits == 8) return launch_block_bits<8, 128>(cc, q, G, n_rows, scale, causal, out, stream);
    return launch_block_bits<16, 128>(cc, q, G, n_rows, scale, causal, out, stream);
}

}  // namespace qw
