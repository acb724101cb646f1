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
//   grid (key splits, query tiles, kv heads); 8 waves, two a SIMD; wave w owns
//   RT 16-row MFMA tiles of query rows (row index r * G + head-in-group, the
//   decode kernel's order), so a workgroup owns 128 * RT rows.
//   Tiles of KT = 16384 / D keys (64 at D = 256) go through two LDS buffers:
//   in round t every thread dequantizes tile t+1 (loaded into registers the
//   round before) into the free buffer, issues the loads of tile t+2, and the
//   waves run tile t out of the other buffer:
//     S^T = K . Q'^T   v_mfma_f32_16x16x32_f16, A = K rows from LDS (read once
//                      a wave and used for all RT row tiles), B = query rows
//                      held in registers,
//     online softmax on the fp16-rounded scores (exp2, lazy reference),
//     O += P . V       A = P straight from the S^T registers, B = 8 keys of one
//                      V dim from LDS (one ds_read_b128 per MFMA, shared by the
//                      RT row tiles).
//   One barrier a tile. RT is chosen per launch so the workgroup count fills
//   the 256 CUs in whole rounds where the row count allows.
//   One key split: the workgroup writes normalized fp16 rows. Several:
//   partials (fp32 m and l, the row O / l in fp16; the fused Turbo4 pass
//   keeps O in fp32) and a split-K merge kernel.
#include <algorithm>
#include <map>
#include <mutex>
#include <type_traits>

#include "append.hpp"
#include "dequant.hpp"
#include "kv_cache.hpp"
#include "turbo4_device.hpp"

namespace qw {

struct BlockArgs {
    const uint32_t* k_data;
    const uint32_t* k_params;
    const uint32_t* v_data;
    const uint32_t* v_params;
    const int* fast_flag;
    const f16* q;       // [hq][Tq][D]
    f16* out;           // [hq][Tq][D], written directly when n_split == 1
    float* part_o;      // [hkv][n_split][PR][D], rows from prow0
    float2* part_ml;    // [hkv][n_split][PR]
    int cap, T, Tq, G, R, causal, n_split, tiles_per_split;
    int qt0;            // first query tile of this launch (of its split segment)
    int prow0, PR;      // first row and row count of this launch's partials
    // n_main > 0: a one-dimensional grid whose first n_main workgroups are
    // unsplit query tiles 0 .. n_main / hkv - 1 (unit u: tile u / hkv, head
    // u % hkv, all main_tiles key tiles, rows written directly) and whose
    // others are the split segment described by the fields above (unit t:
    // split t % n_split, head (t / n_split) % hkv, tile qt0 + t / (n_split hkv)).
    // The dispatcher starts the split workgroups as the first ones finish.
    int n_main, main_tiles, hkv;
    // n_app > 0: a verify block that appends its own rows in this launch
    // (affine and Int8 caches, one query tile). Workgroup h < n_app (= hkv)
    // quantizes-and-appends head h's new rows (read through app) and attends
    // them, keys T_pre .. T - 1, as the last of the n_split partial slots; the
    // others are splits 0 .. n_split - 2 of the cached prefix, keys < T_pre.
    int n_app, T_pre, app_int8;
    RowSrc app;
    // ROPE launches (RoPE, append and attention in one launch): q holds the
    // projection's unrotated rows, query row r of q head qh at
    // q + r * q_tok_stride + qh * D, rotated with app's RoPE fields at
    // position app.position0 + r (rope_dims a multiple of 16); the append
    // workgroups write the rotated rows to q_out [hq][Tq][D].
    int64_t q_tok_stride;
    f16* q_out;
    // Tile images (affine and Int8 prefill): img_w / img hold each key tile's
    // dequantized LDS buffer, [hkv][img_tiles][BUF bytes]; the expansion
    // launch writes them and the attention launch copies them into LDS.
    char* img_w;
    const char* img;
    int img_tiles;
    // pair_h > 0 (causal image launches whose units fill whole rounds): the
    // rows come in pair_h half tiles of NW / 2 waves' rows; unit qt holds half
    // tile qt in waves [0, NW/2) and half tile pair_h - 1 - qt in the others,
    // so every workgroup sees about the same number of (row, key) pairs.
    int pair_h;
    const float* t4_tab;  // Turbo4 caches: the device tables (signs, centroids: T4Tab<D>)
    // WIN launches (a causal sliding window): the row at position p sees keys
    // p - window + 1 .. p
    int window = 0;
    // CAP launches (a logit softcap): s = tanh(f16(q . k) scale / softcap) softcap
    float softcap = 0.0f, scale = 0.0f;
    float t4_post;        // Turbo4 fused pass: scale * log2(e) in fp32
    float scale_h;      // f16(scale) as float
    uint32_t code_off2; // magic offset pair of the separately rounded dequant
};

// Register stages of K/V tile loads in flight (1 or 2).
#ifndef QW_BLOCK_STAGES
#define QW_BLOCK_STAGES 2
#endif

// 8 waves, two a SIMD: one wave a SIMD leaves the MFMA, LDS and VALU
// latencies of a wave exposed (measured ~1.6x slower at equal work).
#ifndef QW_BLOCK_WAVES
#define QW_BLOCK_WAVES 8
#endif
constexpr int kBlockWaves = QW_BLOCK_WAVES;
// Waves of the launches that attend from tile images (no register staging:
// three waves a SIMD fit the register budget).
#ifndef QW_IMAGE_WAVES
#define QW_IMAGE_WAVES 12
#endif
constexpr int kImageWaves = QW_IMAGE_WAVES;
template <int PM>
constexpr int block_waves() {
    return PM == 2 ? kImageWaves : kBlockWaves;
}
// LDS reads a wave keeps in flight ahead of its MFMAs (instruction-scheduling
// groups). Left to itself the compiler issues one or two reads ahead, so each
// MFMA waited on its own read; four ahead measured c3 1.25 -> 1.19 ms and c4
// 70 -> 67 us (2, 3, 6 and 8 ahead were slower). 0 leaves the order to the
// compiler.
#ifndef QW_BLOCK_SCHED_QK
#define QW_BLOCK_SCHED_QK 4  // > 0: K reads kept that far ahead of the QK MFMAs
#endif
#ifndef QW_BLOCK_SCHED_PV
#define QW_BLOCK_SCHED_PV 4  // > 0: V reads kept that far ahead of the P.V MFMAs
#endif

// Split partials of the non-fused launches in fp16 (each row O / l rounded
// once, (m, l) in fp32), as the reference's split-K passes keep them
// (turbo4_attention.cpp:180-200); 0: fp32 O and l. Measured (A/B in one
// run): config 4 48.3 -> 46.0 us, served 4-row verify 22.7 -> 21.8 us,
// 5-row 33.6 -> 32.5 us; parity unchanged within the bar.
#ifndef QW_BLOCK_PART16
#define QW_BLOCK_PART16 1
#endif
constexpr bool kPart16 = QW_BLOCK_PART16;

// Wave priority raised over the MFMA phases of a tile (QK and P.V), so a
// SIMD's waves drift apart and one wave's softmax and dequant VALU issue under
// another's MFMAs: 0 never, 1 the launches that dequantize in the loop, 2
// every launch (the fused Turbo4 pass never: 39.25 against 39.39 us at 4 rows
// @ 32k). Measured (A/B in one run): served 4- and 5-row verify blocks
// -0.15 to -0.35 us, config 4 unchanged, the image launches of config 3
// +0.5 % (their three waves a SIMD already overlap).
#ifndef QW_BLOCK_SETPRIO
#define QW_BLOCK_SETPRIO 1
#endif
constexpr bool kSetprio(int pm) {
    return QW_BLOCK_SETPRIO == 2 || (QW_BLOCK_SETPRIO == 1 && pm != 2);
}

// Key-split row tiles (block_body): 1 for workgroups of 5 or 6 row tiles, 2
// also for those of 1 or 2, 3 also for those of 3 or 4 (which the softcap
// launches and the Turbo4 fused pass always split); 0 off.
#ifndef QW_BLOCK_KSPLIT
#define QW_BLOCK_KSPLIT 2
#endif
#ifndef QW_WINDOW_MIN_TILES
#define QW_WINDOW_MIN_TILES 1  // key tiles a split of a window launch takes at least
#endif
#ifndef QW_BLOCK_KSPLIT_APP
#define QW_BLOCK_KSPLIT_APP 0
#endif

template <int D>
struct BlockShape {
    static constexpr int KT = 16384 / D;  // keys a tile (64 at D=256, 128 at D=128)
    static constexpr int NSUB = KT / 32;  // 32-key sub-blocks a tile
    static constexpr int NM = D / 32;     // QK MFMAs per 16-key tile
    static constexpr int NT = D / 16;     // P.V MFMAs (16-dim output tiles)
    static constexpr int NG = D / 64;     // affine groups a row
    static constexpr int TPR = D / 32;    // 32-dim K slices a row
    static constexpr int LTPR = TPR == 8 ? 3 : 2;
    static constexpr int TPB = D / 4;     // 4-slot V slices a block
    static constexpr int KBUF = (D / 8) * KT * 16;  // K tile bytes in LDS (chunk-major)
    static constexpr int VROW = D + D / 16;  // V block stride in chunks (a pad chunk per 16 slots)
    static constexpr int VBUF = (KT / 8) * VROW * 16;               // V tile bytes in LDS
    static constexpr int BUF = KBUF + VBUF;                         // one buffer
};

// LDS layouts (16-byte chunks). Measured on gfx950 (ds_read_b128, 8 waves a
// CU): an instruction runs at full rate (~210 B/clk a CU) when the 16 lanes of
// each quarter-wave hit 16 distinct bank groups (chunk mod 16) AND lane r of
// every quarter-wave hits the same bank group; quarter-waves whose bank groups
// are rotated against each other run at ~125 B/clk, like a 2-way conflict.
//   K  chunk-major [D/8 chunks][KT keys]: chunk c of key k sits at
//      kaddr(k, c) = c * KT + swz(k), swz(k) = k ^ (bit 4 of k) << 2. The QK
//      A operand (lane (g, r), r = lane & 15) reads chunk g + 4m of key
//      8(r>>2) + 4t + (r&3) + 32u: the chunk stride KT keeps the quarter-waves
//      g aligned, and swz maps the 16 keys of a quarter-wave (k mod 16 takes
//      0-3 and 8-11 twice) to 16 distinct bank groups. Every (step, sub-block)
//      is the lane's base (one a 16-key tile t) plus an immediate. The store
//      phase gives each quarter-wave 16 consecutive keys of one 32-dim slice
//      (quarter-waves differ in the slice): also aligned and distinct.
//   V  [8-key block][D slots + D/16 pad][8 keys], slots in the V plane's
//      physical dim order, slot s at s + (s >> 4): the P.V B operand reads 16
//      consecutive slots a phase (slot 16mm + r at 17mm + r, an immediate
//      per mm), and the store phase's lanes (slots 4j + e) land on 16 distinct
//      bank groups.
__device__ __forceinline__ int kswz(int key) { return key ^ (((key >> 4) & 1) << 2); }
template <int KT>
__device__ __forceinline__ int kaddr(int key, int chunk) {
    return chunk * KT + kswz(key);
}


// max / sum of v over the lane pair (l, l ^ 16), then over (l, l ^ 32): row
// swaps in the VALU (v_permlane16/32_swap) instead of LDS permutes.
__device__ __forceinline__ float wave_max_g(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float wave_sum_g(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// T4M: 0 the affine / Int8 / fp16 caches; 1 and 2 a Turbo4 cache (BITS = 4:
// K rows of D/2 bytes of centroid indices, row-major like the 4-bit K plane,
// one side word a row; V row-major too). The store forms f16(centroid *
// rescale) as the fp16 expansion holds it (centroid pairs from an LDS table,
// one 8-byte read a byte of codes) and places V in the fp16 cache's slot
// order. T4M = 1 keeps the fp16 SDPA arithmetic (the reference's
// dequantize-then-SDPA route); T4M = 2 is the reference's fused verify pass
// (turbo4_attention.cpp:45-197): q arrives rotated and scaled by scale *
// log2(e), scores stay fp32 in the log2 domain, P enters P.V as an fp16 high
// part plus an fp16 remainder (fp32-exact products), and the partial maxima are
// stored in natural units for the shared merge.
// PM (tile images): 0 none; 1 the expansion launch (workgroup (t, h) writes
// the image of key tile t of head h and returns); 2 attention from the images
// (each tile's LDS buffer copied in by LDS-DMA, no dequant in the loop).
template <int BITS, int D, int RT, bool FAST, int T4M = 0, bool APP = false, int PM = 0,
          bool ROPE = false, bool WIN = false, bool CAP = false>
__device__ __forceinline__ void block_body(const BlockArgs& a, char* lds) {
    using S = BlockShape<D>;
    constexpr int KT = S::KT, NSUB = S::NSUB, NM = S::NM, NT = S::NT, NG = S::NG;
    constexpr int TPR = S::TPR, LTPR = S::LTPR, TPB = S::TPB, BUF = S::BUF, KBUF = S::KBUF;
    constexpr int VROW = S::VROW;
    constexpr int NW = block_waves<PM>();
    constexpr bool T4 = T4M != 0, FUSED = T4M == 2;
    static_assert(!T4 || BITS == 4, "Turbo4 indices are 4-bit");
    constexpr bool AFF = BITS != 16 && !T4;
    constexpr int VB = T4 ? 16 : BITS;  // the V slot order in LDS (and of the partial rows)
    constexpr int KU = BITS / 4;  // u32x4 loads a 32-dim K slice / a 4-slot V slice
    // slices of each kind a thread owns (the image launches stage nothing)
    constexpr int PER = PM == 2 ? 1 : KT * TPR / (64 * NW);
    static_assert(PM == 2 || (PER * 64 * NW == KT * TPR && (KT / 8) * TPB == KT * TPR),
                  "slices a thread");

    int sp = 0, qt = 0, h = 0, n_split = 1, tiles_per_split = 1;
    // APP (launches with n_app > 0): the keys this workgroup may see are
    // [key_lo, key_hi); other launches compile without the bounds
    int key_lo = 0, key_hi = a.T;
    if constexpr (PM == 1) {
        h = blockIdx.y;
    } else if (APP) {
        const int lin = blockIdx.x;
        qt = 0;
        n_split = a.n_split;
        tiles_per_split = a.tiles_per_split;
        if (lin < a.n_app) {
            h = lin;
            sp = a.n_split - 1;
            key_lo = a.T_pre;
        } else {
            const int t = lin - a.n_app;
            sp = t % (a.n_split - 1);
            h = t / (a.n_split - 1);
            key_hi = a.T_pre;
        }
    } else if (a.n_main > 0) {
        const int lin = blockIdx.x;
        if (lin < a.n_main) {
            sp = 0;
            qt = lin / a.hkv;
            h = lin % a.hkv;
            n_split = 1;
            tiles_per_split = a.main_tiles;
        } else {
            const int t = lin - a.n_main;
            sp = t % a.n_split;
            h = (t / a.n_split) % a.hkv;
            qt = a.qt0 + t / (a.n_split * a.hkv);
            n_split = a.n_split;
            tiles_per_split = a.tiles_per_split;
        }
    } else {
        sp = blockIdx.x;
        qt = blockIdx.y + a.qt0;
        h = blockIdx.z;
        n_split = a.n_split;
        tiles_per_split = a.tiles_per_split;
    }
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar: wave-uniform branches
    const int r16 = lane & 15, g = lane >> 4;
    const uint32_t magic = vconst(kMagic);

    // ---- key range of this workgroup: its split, cut at the last key any of
    // its rows can see.
    constexpr int WROWS = 16 * RT;
    int row0 = qt * WROWS * NW;
    int row_last = min(a.R, row0 + WROWS * NW) - 1;
    int wrow0 = row0 + WROWS * wave;
    if constexpr (PM == 2 && !T4 && NW % 2 == 0) {
        if (a.pair_h > 0) {
            // causal balance: an early half tile and its mirror (a padding
            // wave gets wrow0 = R and no rows)
            constexpr int HR = WROWS * NW / 2;
            const int hb = a.pair_h - 1 - qt;
            const bool b_live = hb > qt;
            row0 = qt * HR;
            row_last = min(a.R, (b_live ? hb : qt) * HR + HR) - 1;
            wrow0 = wave < NW / 2 ? qt * HR + WROWS * wave
                                  : (b_live ? hb * HR + WROWS * (wave - NW / 2) : a.R);
            wrow0 = min(wrow0, a.R);
        }
    }
    // Key-split row tiles: a workgroup of 5 or 6 row tiles (one per wave
    // leaves SIMDs 0 and 1 two tiles each, SIMDs 2 and 3 one) gives its
    // tiles 4 and 5 to waves 4..7, each wave computing half of every key tile
    // (tile 4: waves 4 and 6, SIMDs 0 and 2; tile 5: waves 5 and 7), so each
    // SIMD carries 1.5 tiles; one of 1 or 2 row tiles splits them over waves
    // 0..3, one half a SIMD; in the launches whose tile math is heaviest (the
    // softcap's and the Turbo4 fused pass's), one of 3 or 4 row tiles puts
    // the halves of tile t on waves t and t + 4. The two halves' (m, l, O)
    // meet before the epilogue (the same combine as the split merge).
    // (not in the affine / Int8 launches that append: measured 0.5-1 us slower
    // there, where the attention-only launches gain 1-1.5 us and the Turbo4
    // fused pass 7.7 us at 4 rows; not in the window launches, 0.3 us slower,
    // but in the softcap ones, whose tanh and second P.V MFMA make the tile
    // compute-bound: 35.0 -> 24.0 us for a decode step over 32k keys)
    constexpr bool KS_OK = QW_BLOCK_KSPLIT && PM == 0 && RT == 1 && NW == 8 && NSUB % 2 == 0 &&
                           (!APP || T4 || QW_BLOCK_KSPLIT_APP) && (!WIN || CAP);
    bool ks_any = false, ks_half = false;
    int ks_ub = 0;  // the wave's first sub-block of a tile
    if constexpr (KS_OK) {
        const int n_rt = (row_last - row0) / 16 + 1;
        if (n_rt == 5 || n_rt == 6) {
            ks_any = true;
            if (wave >= 4) {
                ks_half = true;
                wrow0 = row0 + 16 * (4 + (wave & 1));
                ks_ub = ((wave >> 1) & 1) * (NSUB / 2);
            }
        } else if (n_rt <= 2 && QW_BLOCK_KSPLIT >= 2) {
            ks_any = true;
            if (wave < 4) {
                ks_half = true;
                wrow0 = row0 + 16 * (wave & 1);
                ks_ub = ((wave >> 1) & 1) * (NSUB / 2);
            }
        } else if (n_rt <= 4 && (QW_BLOCK_KSPLIT >= 3 || CAP || FUSED)) {
            // 3 or 4 row tiles: tile t on waves t and t + 4 (one SIMD), a half
            // each (softcap launches: 37.2 -> 30.2 us at 8 rows a sequence; the
            // Turbo4 fused pass at G = 8, 5 rows: 41.9 -> 37.2 us; the affine
            // launches and the Turbo4 dequantize route measured 1-3.5 us slower)
            ks_any = true;
            ks_half = true;
            wrow0 = row0 + 16 * (wave & 3);
            ks_ub = (wave >> 2) * (NSUB / 2);
        }
    }
    auto cut = [&](int lim_) { return APP ? min(lim_, key_hi - 1) : lim_; };
    const bool app_unit = APP && key_lo > 0;
    const int wg_lim = cut(a.causal ? a.T - a.Tq + row_last / a.G : a.T - 1);
    const int n_tiles = (a.T + KT - 1) / KT;
    // WIN: the splits cover the keys from the first tile any of the
    // workgroup's rows sees (its first row's window start)
    const int t_win = WIN ? max(0, a.T - a.Tq + row0 / a.G - a.window + 1) / KT : 0;
    const int t0 = app_unit ? key_lo / KT : t_win + sp * tiles_per_split;
    const int t1 = app_unit ? wg_lim / KT + 1 : min(min(n_tiles, t0 + tiles_per_split), wg_lim / KT + 1);

    // ---- the wave's RT x 16 query rows as the B operand of S^T = K . Q'^T
    // (col = query row r16 of row tile rt, k-group g = dims 32m + 8g .. +7 of
    // MFMA step m, in the order the LDS K row holds them).
    const bool wave_live = wrow0 < a.R;
    const int wave_last = min(a.R, wrow0 + WROWS) - 1;
    const int wave_lim = cut(a.causal ? a.T - a.Tq + wave_last / a.G : a.T - 1);
    // the smallest key limit of the wave's live rows (padding rows see nothing
    // and are never written, so they do not count)
    const int wave_first_lim = cut(a.causal ? a.T - a.Tq + wrow0 / a.G : a.T - 1);
    int lim[RT], wlo[RT];  // (WIN) the row's first visible key
    bool row_ok[RT];
    // WIN: the window start of the wave's last row (tiles below it need the
    // mask) and of its first row (tiles wholly below it are skipped)
    const int wave_lo_max = WIN ? a.T - a.Tq + wave_last / a.G - a.window + 1 : 0;
    const int wave_lo_min = WIN ? a.T - a.Tq + wrow0 / a.G - a.window + 1 : 0;
    half8 qb[RT][NM];
    // Turbo4: the workgroup's rows are rotated into the K basis (the rotation
    // kernels' arithmetic; wave w takes rows w, w + NW, ..., four at a time
    // with their loads issued first) and staged as fp16 in the second tile
    // buffer, which the prologue leaves alone; the centroid-pair table goes
    // behind the two buffers. One barrier covers both. (The image launches
    // stage q from the start of the two buffers, one barrier more before the
    // first tile's copy; they need no pair table, the expansion launch no q.)
    f16* const sq = (f16*)(lds + (PM == 2 ? 0 : BUF));
    if constexpr (T4) {
        static_assert(NW * WROWS * D * sizeof(f16) <= (PM == 2 ? 2 : 1) * BUF,
                      "staged q rows exceed the tile buffers");
        if constexpr (PM != 2) {
            float2* const cp = (float2*)(lds + 2 * BUF);
            const float* cb = a.t4_tab + T4Tab<D>::cb;
            for (int bb = tid; bb < 256; bb += 64 * NW) cp[bb] = float2{cb[bb & 15], cb[bb >> 4]};
        }
        constexpr int VPL = D / 64, NB = 4;
        using HV = std::conditional_t<VPL == 4, half4v, half2v>;
        float si[VPL], so[VPL];
        t4_lane_signs<D>(a.t4_tab + T4Tab<D>::k_s1, lane, si);
        t4_lane_signs<D>(a.t4_tab + T4Tab<D>::k_s2, lane, so);
        // ROPE: the angle table in buffer 0, which the prologue leaves alone
        float2* const rtab = (float2*)lds;
        if constexpr (ROPE) {
            rope_fill_table(a.app, a.Tq, rtab, 64 * NW);
            __syncthreads();
        }
        const bool app_writer = ROPE && APP && key_lo > 0;  // writes q_out (one workgroup a head)
        for (int k0 = 0; k0 < (PM == 1 ? 0 : WROWS); k0 += NB) {
            if (row0 + wave + NW * k0 >= a.R) break;  // wave-uniform
            float y[NB][VPL];
#pragma unroll
            for (int kk = 0; kk < NB; kk++) {
                const int rho = min(row0 + wave + NW * (k0 + kk), a.R - 1);
                const int qh = h * a.G + rho % a.G, rq = rho / a.G;
                const f16* qrow = ROPE ? a.q + (int64_t)rq * a.q_tok_stride + (int64_t)qh * D
                                       : a.q + ((int64_t)qh * a.Tq + rq) * D;
                const HV w = *(const HV*)(qrow + lane * VPL);
                if constexpr (ROPE) {
                    // RoPE first (as the reference's q arrives rotated), then
                    // the K basis; the half-split partners of the lane's dims
                    const int d0 = lane * VPL, rh = a.app.rope_dims >> 1;
                    const bool need = !a.app.traditional && d0 < a.app.rope_dims;
                    const HV wp = need ? *(const HV*)(qrow + (d0 < rh ? d0 + rh : d0 - rh)) : HV{};
                    f16 xa[VPL], xpa[VPL], ya[VPL];
#pragma unroll
                    for (int jj = 0; jj < VPL; jj++) {
                        xa[jj] = w[jj];
                        xpa[jj] = wp[jj];
                    }
                    rope_rotate_dims<VPL>(a.app, rtab, rq, d0, xa, xpa, ya);
                    const bool own = row0 + wave + NW * (k0 + kk) < a.R;
#pragma unroll
                    for (int jj = 0; jj < VPL; jj++) {
                        y[kk][jj] = (float)ya[jj];
                        if (app_writer && own) a.q_out[((int64_t)qh * a.Tq + rq) * D + d0 + jj] = ya[jj];
                    }
                } else {
#pragma unroll
                    for (int jj = 0; jj < VPL; jj++) y[kk][jj] = (float)w[jj];
                }
            }
#pragma unroll
            for (int kk = 0; kk < NB; kk++) {
                f16 o[VPL];
                if constexpr (FUSED)
                    t4_rotate_row_scaled<D>(y[kk], lane, si, so, a.t4_post, o);
                else
                    t4_rotate_row<D>(y[kk], lane, si, so, o);
                const int lr = wave + NW * (k0 + kk);
                HV ov;
#pragma unroll
                for (int jj = 0; jj < VPL; jj++) ov[jj] = o[jj];
                if (row0 + lr < a.R) *(HV*)(sq + lr * D + lane * VPL) = ov;
            }
        }
        __syncthreads();
    }
    // ROPE (affine and Int8): the rows rotated first, as the Turbo4 staging
    // above rotates them (angle table in buffer 0, rows staged in buffer 1,
    // both free until the first tile's store), and written out by the head's
    // append workgroup; the conversion below then reads them from LDS
    f16* const sqr = (f16*)(lds + BUF);
    if constexpr (ROPE && !T4) {
        constexpr int VPL = D / 64, NB = 4;
        using HV = std::conditional_t<VPL == 4, half4v, half2v>;
        static_assert(NW * WROWS * D * sizeof(f16) <= BUF, "staged q rows exceed a tile buffer");
        float2* const rtab = (float2*)lds;
        rope_fill_table(a.app, a.Tq, rtab, 64 * NW);
        __syncthreads();
        const bool app_writer = APP && key_lo > 0;
        for (int k0 = 0; k0 < WROWS; k0 += NB) {
            if (row0 + wave + NW * k0 >= a.R) break;  // wave-uniform
#pragma unroll
            for (int kk = 0; kk < NB; kk++) {
                const int lr = wave + NW * (k0 + kk), rho = min(row0 + lr, a.R - 1);
                const int qh = h * a.G + rho % a.G, rq = rho / a.G;
                const f16* qrow = a.q + (int64_t)rq * a.q_tok_stride + (int64_t)qh * D;
                const int d0 = lane * VPL, rh = a.app.rope_dims >> 1;
                const bool need = !a.app.traditional && d0 < a.app.rope_dims;
                const HV w = *(const HV*)(qrow + d0);
                const HV wp = need ? *(const HV*)(qrow + (d0 < rh ? d0 + rh : d0 - rh)) : HV{};
                f16 xa[VPL], xpa[VPL], ya[VPL];
#pragma unroll
                for (int jj = 0; jj < VPL; jj++) {
                    xa[jj] = w[jj];
                    xpa[jj] = wp[jj];
                }
                rope_rotate_dims<VPL>(a.app, rtab, rq, d0, xa, xpa, ya);
                HV y;
#pragma unroll
                for (int jj = 0; jj < VPL; jj++) y[jj] = ya[jj];
                if (row0 + lr < a.R) {
                    *(HV*)(sqr + lr * D + d0) = y;
                    if (app_writer) *(HV*)(a.q_out + ((int64_t)qh * a.Tq + rq) * D + d0) = y;
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int rt = 0; rt < (PM == 1 ? 0 : RT); rt++) {
        const int rho = wrow0 + 16 * rt + r16;
        row_ok[rt] = rho < a.R;
        lim[rt] = row_ok[rt] ? cut(a.causal ? a.T - a.Tq + rho / a.G : a.T - 1) : -1;
        wlo[rt] = WIN && row_ok[rt] ? a.T - a.Tq + rho / a.G - a.window + 1 : 0;
        const int rr = row_ok[rt] ? rho : 0;
        // (Turbo4 padding rows read the workgroup's first staged row; their scale is 0)
        const f16* qrow = T4     ? sq + (row_ok[rt] ? wrow0 - row0 + 16 * rt + r16 : 0) * D
                          : ROPE ? sqr + (row_ok[rt] ? wrow0 - row0 + 16 * rt + r16 : 0) * D
                                 : a.q + ((int64_t)(h * a.G + rr % a.G) * a.Tq + rr / a.G) * D;
        const f16 sc = row_ok[rt] ? (FUSED || CAP ? (f16)1.0f : (f16)a.scale_h) : (f16)0.0f;
        const half2v sc2 = {sc, sc};
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const u32x4 w = *(const u32x4*)(qrow + 32 * m + 8 * g);
            u32x4 o;
            if constexpr (BITS == 4 && !T4) {
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
            qb[rt][m] = __builtin_bit_cast(half8, y);
        }
    }

    if constexpr (T4 && PM == 2) __syncthreads();  // staged q read before the first copy
    if constexpr (ROPE && !T4) __syncthreads();    // the staged rows read before the first store

    // ---- tile loads: thread slice j (of PER) -> (key kk, 32-dim slice q32)
    // of K and (8-key block vb, 4 physical dim slots from 4 vj) of V. A
    // quarter-wave takes 16 consecutive keys of one K slice, the quarter-waves
    // of a wave 4 consecutive slices of the same keys (the LDS writes then hit
    // aligned, distinct bank groups under kaddr; each key row is read as
    // 4-slice runs).
    struct Stage {
        u32x4 kc[PER][KU];
        uint32_t kp[PER];
        u32x4 vc[PER][KU];
        u32x4 vp[PER][2];
        uint32_t vt[PER][T4 ? 8 : 1];  // Turbo4: keys 8 vb + i, the 2 bytes of dims 4 vj .. +3
    };
    int kk[PER], q32[PER], vb[PER], vj[PER], vgrp[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int tt = tid + 64 * NW * j;
        q32[j] = (tt >> 4) & (TPR - 1);
        kk[j] = (tt & 15) | ((tt >> (4 + LTPR)) << 4);
        vb[j] = tt / TPB;
        vj[j] = tt % TPB;
        vgrp[j] = v_logical_dim(4 * vj[j], D, VB) / 64;
    }
    const int64_t krow_words = (int64_t)D * BITS / 32;
    const int64_t vblk_words = (int64_t)D * BITS / 4;
    // the thread's tile-0 addresses; tile t is a scalar multiple of the tile
    // strides further on (one 64-bit add a pointer a tile)
    const u32x4* ksrc0[PER];
    const uint32_t* kpsrc0[PER];
    const u32x4* vsrc0[PER];
    const u32x4* vpsrc0[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int64_t row = (int64_t)h * a.cap + kk[j];
        ksrc0[j] = (const u32x4*)(a.k_data + row * krow_words) + KU * q32[j];
        kpsrc0[j] = T4 ? a.k_params + row : a.k_params + row * NG + k_param_slot(q32[j] >> 1, NG);
        const int64_t blk = (int64_t)h * (a.cap / 8) + vb[j];
        vsrc0[j] = T4 ? (const u32x4*)((const uint16_t*)a.v_data + (8 * blk) * (D / 4) + vj[j])
                      : (const u32x4*)(a.v_data + blk * vblk_words) + KU * vj[j];
        vpsrc0[j] = T4 ? (const u32x4*)(a.v_params + 8 * blk)
                       : (const u32x4*)(a.v_params + (blk * NG + vgrp[j]) * 8);
    }
    auto load = [&](Stage& st, int t) {
        const int64_t t_rows = (int64_t)t * KT, t_blks = (int64_t)t * (KT / 8);
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const u32x4* ksrc = ksrc0[j] + t_rows * (krow_words / 4);
#pragma unroll
            for (int u = 0; u < KU; u++) st.kc[j][u] = ksrc[u];
            if constexpr (AFF) st.kp[j] = kpsrc0[j][t_rows * NG];
            if constexpr (T4) {
                st.kp[j] = kpsrc0[j][t_rows];
                // V: 2 bytes of each of the block's 8 rows (row stride D/4 halfwords)
                const uint16_t* vsrc = (const uint16_t*)vsrc0[j] + t_rows * (D / 4);
#pragma unroll
                for (int i = 0; i < 8; i++) st.vt[j][i] = vsrc[i * (D / 4)];
                const u32x4* psrc = vpsrc0[j] + t_blks * 2;
                st.vp[j][0] = psrc[0];
                st.vp[j][1] = psrc[1];
            } else {
                const u32x4* vsrc = vsrc0[j] + t_blks * (vblk_words / 4);
#pragma unroll
                for (int u = 0; u < KU; u++) st.vc[j][u] = vsrc[u];
            }
            if constexpr (AFF) {
                const u32x4* psrc = vpsrc0[j] + t_blks * (NG * 2);
                st.vp[j][0] = psrc[0];
                st.vp[j][1] = psrc[1];
            }
        }
    };
    // Dequantize a stage into LDS buffer b: K row kk, chunks 4 q32 .. +3 (dims
    // in the order of the Q operand); V block vb, slots 4 vj .. +3 (8 keys each).
    auto store = [&](const Stage& st, int b) {
        half8* const sK8 = (half8*)(lds + BUF * b);
        half8* const sV8 = (half8*)(lds + BUF * b + KBUF);
#pragma unroll
        for (int j = 0; j < PER; j++) {
            // chunks 4 q32 + w of key kk: KT chunks apart
            half8* krow = sK8 + kaddr<KT>(kk[j], 4 * q32[j]);
            if constexpr (T4) {
                const float2* cp = (const float2*)(lds + 2 * BUF);
                const float kr = (float)h2(st.kp[j]).x;
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    half8 y;
#pragma unroll
                    for (int n = 0; n < 4; n++) {
                        const float2 c = cp[(st.kc[j][0][w] >> (8 * n)) & 0xFFu];
                        y[2 * n] = t4_f16_product(c.x, kr);
                        y[2 * n + 1] = t4_f16_product(c.y, kr);
                    }
                    krow[w * KT] = y;
                }
                // V: key i of the block, dims 4 vj + e at the fp16 layout's slot
                half8 yv[4];
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float vr = (float)h2(st.vp[j][i / 4][i % 4]).y;
                    const float2 c0 = cp[st.vt[j][i] & 0xFFu], c1 = cp[(st.vt[j][i] >> 8) & 0xFFu];
                    yv[0][i] = t4_f16_product(c0.x, vr);
                    yv[1][i] = t4_f16_product(c0.y, vr);
                    yv[2][i] = t4_f16_product(c1.x, vr);
                    yv[3][i] = t4_f16_product(c1.y, vr);
                }
                half8* vblk = sV8 + vb[j] * VROW;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int sl = v_phys_dim(4 * vj[j] + e, D, 16);
                    vblk[sl + (sl >> 4)] = yv[e];
                }
                continue;
            }
            if constexpr (BITS == 4) {
                const half2v sb = h2(st.kp[j]);
                const half2v s = {sb.x, sb.x}, bb = {sb.y, sb.y};
                const PairConsts pc = make_consts<FAST, 4>(s, s, s, s, bb, bb, bb, bb);
#pragma unroll
                for (int w = 0; w < 4; w++) krow[w * KT] = deq4<FAST>(st.kc[j][0][w], pc, magic);
            } else if constexpr (BITS == 8) {
                const half2v sb = h2(st.kp[j]);
                const half2v s = {sb.x, sb.x}, bb = {sb.y, sb.y};
                const PairConsts pc = make_consts<FAST, 8>(s, s, s, s, bb, bb, bb, bb, a.code_off2);
#pragma unroll
                for (int w = 0; w < 4; w++)
                    krow[w * KT] = deq8<FAST>(st.kc[j][w / 2][2 * (w % 2)], st.kc[j][w / 2][2 * (w % 2) + 1], pc);
            } else {
#pragma unroll
                for (int w = 0; w < 4; w++) krow[w * KT] = as_h8(st.kc[j][w]);
            }
            PairConsts vc;
            if constexpr (AFF)
                vc = make_consts<FAST, BITS>(h2(st.vp[j][0][0]), h2(st.vp[j][0][1]),
                                             h2(st.vp[j][0][2]), h2(st.vp[j][0][3]),
                                             h2(st.vp[j][1][0]), h2(st.vp[j][1][1]),
                                             h2(st.vp[j][1][2]), h2(st.vp[j][1][3]), a.code_off2);
            half8* vblk = sV8 + vb[j] * VROW;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                half8 y;
                if constexpr (BITS == 4)
                    y = deq4<FAST>(st.vc[j][0][e], vc, magic);
                else if constexpr (BITS == 8)
                    y = deq8<FAST>(st.vc[j][e / 2][2 * (e % 2)], st.vc[j][e / 2][2 * (e % 2) + 1], vc);
                else
                    y = as_h8(st.vc[j][e]);
                vblk[4 * vj[j] + e + (vj[j] >> 2)] = y;  // slot s at s + (s >> 4)
            }
        }
    };

    float m_run[RT], l_run[RT];  // softmax reference / this lane's share of the sum, column r16
    float4v acc_o[RT][NT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        m_run[rt] = -INFINITY;
        l_run[rt] = 0.0f;
#pragma unroll
        for (int mm = 0; mm < NT; mm++) acc_o[rt][mm] = float4v{0.f, 0.f, 0.f, 0.f};
    }

    // One tile (keys kt0 .. kt0 + KT - 1) out of buffer b: the QK MFMAs of all
    // its 32-key sub-blocks first (independent chains), one softmax step over
    // the whole tile (one max reduction, one lazy-rescale check), then P.V.
    // (NU of the tile's NSUB sub-blocks, from sub-block ub: a key-split wave's half)
    auto tile = [&](int b, int kt0, auto nu_c, int ub) {
        constexpr int NU = decltype(nu_c)::value;
        const half8* sK8 = (const half8*)(lds + BUF * b);
        const half8* sV8 = (const half8*)(lds + BUF * b + KBUF);
        // S^T: A row r16 of 16-key MFMA tile (u, tt) is key 32u + 8(r16>>2) +
        // 4tt + (r16&3), so lane (g, r16) ends up with keys 32u + 8g + 4tt + i
        // of column r16.
        const int key0 = 8 * (r16 >> 2) + (r16 & 3);
        // kswz(key0 + 4tt) = key0 + 4 (tt ^ bit 4 of key0): one base a tile tt
        const int b4 = (key0 >> 4) & 1;
        const half8* kbase0 = sK8 + g * KT + key0 + 4 * b4;
        const half8* kbase1 = sK8 + g * KT + key0 + 4 * (b4 ^ 1);
        float4v acc[NU][2][RT];
#pragma unroll
        for (int u = 0; u < NU; u++)
#pragma unroll
            for (int tt = 0; tt < 2; tt++)
#pragma unroll
                for (int rt = 0; rt < RT; rt++) acc[u][tt][rt] = float4v{0.f, 0.f, 0.f, 0.f};
        if constexpr (kSetprio(PM) && !FUSED) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int m = 0; m < NM; m++) {
#pragma unroll
            for (int u = 0; u < NU; u++) {
                // chunk g + 4m of keys key0 + 32u (+4): kswz leaves bits >= 5 alone
                const half8 ka = kbase0[4 * m * KT + 32 * (ub + u)], kb2 = kbase1[4 * m * KT + 32 * (ub + u)];
#pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    acc[u][0][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[rt][m], acc[u][0][rt], 0, 0, 0);
                    acc[u][1][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb2, qb[rt][m], acc[u][1][rt], 0, 0, 0);
                }
            }
        }
#if QW_BLOCK_SCHED_QK
        if constexpr (RT == 1) {
            constexpr int NQ = NM * NU * 2, AH = QW_BLOCK_SCHED_QK;
            __builtin_amdgcn_sched_group_barrier(0x100, AH, 0);
#pragma unroll
            for (int i = 0; i < NQ - AH; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, AH, 0);
        }
#endif
        if constexpr (kSetprio(PM) && !FUSED) __builtin_amdgcn_s_setprio(0);
        half8 pop[NU][RT];
        // Scores -> fp16 rounding -> (mask) -> online softmax -> P; the mask
        // only for tiles some row of the wave cannot fully see (a scalar
        // branch around the compares: the common case carries none).
        const bool mask = kt0 + KT - 1 > wave_first_lim || (APP && kt0 < key_lo) ||
                          (WIN && kt0 < wave_lo_max);
        half8 popl[FUSED || CAP ? NU : 1][RT];  // fp32 P: the remainders p - f16(p)
        auto softmax_fused = [&]() {
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                // fp32 scores in the log2 domain (q carries scale * log2 e)
                float sf[NU][8];
#pragma unroll
                for (int u = 0; u < NU; u++)
#pragma unroll
                    for (int e = 0; e < 8; e++) sf[u][e] = acc[u][e >> 2][rt][e & 3];
                if (mask) {
#pragma unroll
                    for (int u = 0; u < NU; u++)
#pragma unroll
                        for (int e = 0; e < 8; e++) {
                            const int key = kt0 + 32 * (ub + u) + 8 * g + (e & 3) + 4 * (e >> 2);
                            if (key > lim[rt] || (APP && key < key_lo) || (WIN && key < wlo[rt])) sf[u][e] = -INFINITY;
                        }
                }
                float mx_lane = sf[0][0];
#pragma unroll
                for (int u = 0; u < NU; u++)
#pragma unroll
                    for (int e = 0; e < 8; e++) mx_lane = fmaxf(mx_lane, sf[u][e]);
                // lazy reference in log2 units (p <= 2^5.5)
                if (__any(mx_lane > m_run[rt] + 5.5f)) {
                    const float m_new = fmaxf(m_run[rt], wave_max_g(mx_lane));
                    if (__any(m_run[rt] != -INFINITY)) {
                        const float alpha =
                            m_run[rt] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run[rt] - m_new);
                        l_run[rt] *= alpha;
                        float f[4];
#pragma unroll
                        for (int i = 0; i < 4; i++) f[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
                        for (int mm = 0; mm < NT; mm++)
#pragma unroll
                            for (int i = 0; i < 4; i++) acc_o[rt][mm][i] *= f[i];
                    }
                    m_run[rt] = m_new;
                }
                const float mref = m_run[rt] == -INFINITY ? 0.0f : m_run[rt];
#pragma unroll
                for (int u = 0; u < NU; u++)
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const float p = __builtin_amdgcn_exp2f(sf[u][e] - mref);
                        l_run[rt] += p;
                        const f16 ph = (f16)p;
                        pop[u][rt][e] = ph;
                        if constexpr (FUSED) popl[u][rt][e] = (f16)(p - (float)ph);
                    }
            }
        };
        // CAP: the softcap composite's arithmetic (compiled_softcap_sdpa,
        // mlx_cxx_bridge.cpp:1573-1590): S = f16(q . k) with q unscaled, then
        // in fp32 s = tanh(S scale / cap) cap, the softmax in fp32 and P.V
        // with fp32 P (an fp16 high part and an fp16 remainder)
        auto softmax_cap = [&]() {
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                float sf[NU][8];
#pragma unroll
                for (int u = 0; u < NU; u++)
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const float x = (float)(f16)acc[u][e >> 2][rt][e & 3];
                        sf[u][e] = tanhf(x * a.scale / a.softcap) * a.softcap;
                    }
                if (mask) {
#pragma unroll
                    for (int u = 0; u < NU; u++)
#pragma unroll
                        for (int e = 0; e < 8; e++) {
                            const int key = kt0 + 32 * (ub + u) + 8 * g + (e & 3) + 4 * (e >> 2);
                            if (key > lim[rt] || (WIN && key < wlo[rt])) sf[u][e] = -INFINITY;
                        }
                }
                float mx_lane = sf[0][0];
#pragma unroll
                for (int u = 0; u < NU; u++)
#pragma unroll
                    for (int e = 0; e < 8; e++) mx_lane = fmaxf(mx_lane, sf[u][e]);
                if (__any(mx_lane > m_run[rt] + 5.5f)) {
                    const float m_new = fmaxf(m_run[rt], wave_max_g(mx_lane));
                    if (__any(m_run[rt] != -INFINITY)) {
                        const float alpha = m_run[rt] == -INFINITY
                                                ? 0.0f
                                                : __builtin_amdgcn_exp2f((m_run[rt] - m_new) * kLog2e);
                        l_run[rt] *= alpha;
                        float f[4];
#pragma unroll
                        for (int i = 0; i < 4; i++) f[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
                        for (int mm = 0; mm < NT; mm++)
#pragma unroll
                            for (int i = 0; i < 4; i++) acc_o[rt][mm][i] *= f[i];
                    }
                    m_run[rt] = m_new;
                }
                const float mref2 = (m_run[rt] == -INFINITY ? 0.0f : m_run[rt]) * kLog2e;
#pragma unroll
                for (int u = 0; u < NU; u++)
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sf[u][e], kLog2e, -mref2));
                        l_run[rt] += p;
                        const f16 ph = (f16)p;
                        pop[u][rt][e] = ph;
                        if constexpr (CAP) popl[u][rt][e] = (f16)(p - (float)ph);
                    }
            }
        };
        auto softmax = [&]() {
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                // MLX rounds the score matrix to fp16 before the softmax: the
                // scores stay packed in fp16 pairs (element e of pair j is
                // score 2j + e: keys 32u + 8g + (idx & 3) + 4 (idx >> 2)).
                half2v sh[NU][4];
#pragma unroll
                for (int u = 0; u < NU; u++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float4v& av = acc[u][j >> 1][rt];
                        sh[u][j] = half2v{(f16)av[2 * (j & 1)], (f16)av[2 * (j & 1) + 1]};
                    }
                if (mask) {
#pragma unroll
                    for (int u = 0; u < NU; u++)
#pragma unroll
                        for (int j = 0; j < 4; j++)
#pragma unroll
                            for (int e = 0; e < 2; e++) {
                                const int idx = 2 * j + e;
                                const int key = kt0 + 32 * (ub + u) + 8 * g + (idx & 3) + 4 * (idx >> 2);
                                if (key > lim[rt] || (APP && key < key_lo) || (WIN && key < wlo[rt])) sh[u][j][e] = (f16)(-INFINITY);
                            }
                }
                // Online softmax with a lazy reference: m_run moves only when a
                // score exceeds it by more than 5.5 (so p <= e^5.5 stays well
                // inside fp16).
                half2v m2 = sh[0][0];
#pragma unroll
                for (int u = 0; u < NU; u++)
#pragma unroll
                    for (int j = 0; j < 4; j++) m2 = __builtin_elementwise_max(m2, sh[u][j]);
                // the lane's own maximum decides (m_run is the same in the
                // four lanes of a column); the column reduction runs only when
                // the reference moves
                const float mx_lane = fmaxf((float)m2.x, (float)m2.y);
                if (__any(mx_lane > m_run[rt] + 5.5f)) {
                    const float m_new = fmaxf(m_run[rt], wave_max_g(mx_lane));
                    if (__any(m_run[rt] != -INFINITY)) {
                        const float alpha = m_run[rt] == -INFINITY
                                                ? 0.0f
                                                : __builtin_amdgcn_exp2f((m_run[rt] - m_new) * kLog2e);
                        l_run[rt] *= alpha;
                        float f[4];
#pragma unroll
                        for (int i = 0; i < 4; i++) f[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
                        for (int mm = 0; mm < NT; mm++)
#pragma unroll
                            for (int i = 0; i < 4; i++) acc_o[rt][mm][i] *= f[i];
                    }
                    m_run[rt] = m_new;
                }
                const float mref2 = (m_run[rt] == -INFINITY ? 0.0f : m_run[rt]) * kLog2e;
#pragma unroll
                for (int u = 0; u < NU; u++)
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const float x = (float)sh[u][e >> 1][e & 1];
                        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(x, kLog2e, -mref2));
                        l_run[rt] += p;
                        pop[u][rt][e] = (f16)p;
                    }
            }
        };
        if constexpr (FUSED)
            softmax_fused();
        else if constexpr (CAP)
            softmax_cap();
        else
            softmax();
        // O += P . V: B = slot 16mm + r16 (column r16 of output tile mm) of
        // V block 4u + g, i.e. keys 32u + 8g .. +7.
        if constexpr (kSetprio(PM) && !FUSED) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int u = 0; u < NU; u++) {
            const half8* vb8 = sV8 + (4 * (ub + u) + g) * VROW + r16;
#pragma unroll
            for (int mm = 0; mm < NT; mm++) {
                const half8 vv = vb8[17 * mm];  // slot 16mm + r16
#pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    acc_o[rt][mm] =
                        __builtin_amdgcn_mfma_f32_16x16x32_f16(pop[u][rt], vv, acc_o[rt][mm], 0, 0, 0);
                    if constexpr (FUSED || CAP)
                        acc_o[rt][mm] =
                            __builtin_amdgcn_mfma_f32_16x16x32_f16(popl[u][rt], vv, acc_o[rt][mm], 0, 0, 0);
                }
            }
        }
#if QW_BLOCK_SCHED_PV
        if constexpr (RT == 1) {
            constexpr int NQ = NU * NT, AH = QW_BLOCK_SCHED_PV;
            __builtin_amdgcn_sched_group_barrier(0x100, AH, 1);
#pragma unroll
            for (int i = 0; i < NQ - AH; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, AH, 1);
        }
#endif
        if constexpr (kSetprio(PM) && !FUSED) __builtin_amdgcn_s_setprio(0);
    };

    auto run_tile = [&](int b, int kt0) { tile(b, kt0, std::integral_constant<int, NSUB>{}, 0); };

    if constexpr (PM == 1) {
        // the expansion: tile blockIdx.x's buffer, as the main loop stores
        // it, copied out to its image
        Stage st;
        load(st, blockIdx.x);
        store(st, 0);
        __syncthreads();
        char* dst = a.img_w + ((int64_t)h * a.img_tiles + blockIdx.x) * BUF;
        for (int i = 16 * tid; i < BUF; i += 16 * 64 * NW) *(u32x4*)(dst + i) = *(const u32x4*)(lds + i);
        return;
    }
    if constexpr (PM == 2) {
        // tile t's image into buffer b: 1 KB a wave instruction (lane i its
        // 16 bytes at the wave-uniform LDS address + 16 i, which the
        // instruction takes from M0); waited for before the barrier.
        // Issued from asm that saves M0 first and restores it after (each
        // write followed by one wait state), so the compiler's view of M0
        // holds across it. The compiler builtin for this copy
        // (__builtin_amdgcn_global_load_lds) compiles the same instruction,
        // but around it the tile's LDS reads lose their lookahead (21
        // lgkmcnt(0) waits in the kernel against 7, and 4 lgkmcnt(3) against
        // 63): config 3 827 us against 819 us here (A/B in one run; 814 us
        // with an asm that clobbers M0 without restoring it).
        const char* img0 = a.img + (int64_t)h * a.img_tiles * BUF;
        const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds;
        auto dma = [&](int t, int b) {
            const char* src = img0 + (int64_t)t * BUF + 16 * lane;
            for (int c = wave; c < BUF / 1024; c += NW) {
                uint32_t saved;
                asm volatile(
                    "s_mov_b32 %0, m0\n\t"
                    "s_mov_b32 m0, %2\n\t"
                    "s_nop 0\n\t"
                    "global_load_lds_dwordx4 %1, off\n\t"
                    "s_nop 0\n\t"
                    "s_mov_b32 m0, %0"
                    : "=&s"(saved)
                    : "v"(src + 1024 * c),
                      "s"(__builtin_amdgcn_readfirstlane(lds0 + BUF * b + 1024 * c))
                    : "memory");
            }
        };
        static_assert(BUF % 1024 == 0, "a tile buffer is whole 1 KB DMA instructions");
        if (t0 < t1) dma(t0, 0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        for (int t = t0; t < t1; t++) {
            const int b = (t - t0) & 1;
            if (t + 1 < t1) dma(t + 1, b ^ 1);
            if (wave_live && t * KT <= wave_lim) run_tile(b, t * KT);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        }
    } else {
    // (one copy of the loop a tile shape, chosen outside it: a key-split
    // wave's half tile inside the same loop body as the whole tile pushed the
    // kernel to 256 VGPRs with spills; both copies run one barrier a round)
    auto main_loop = [&](auto nu_c, int ub) {
        // ---- main loop: round t dequantizes tile t+1 into LDS buffer (t+1)&1
        // from its register stage, reuses that stage for the loads of tile
        // t + 1 + QW_BLOCK_STAGES, and computes tile t from buffer t&1; one
        // barrier a round. Two register stages keep two tiles of loads in flight
        // behind the tile being computed, which the key-split verify launches
        // (one tile of math a round) need to cover HBM latency.
#if QW_BLOCK_STAGES == 2
        Stage s0, s1;
        if (t0 < t1) {
            load(s0, t0);
            store(s0, 0);
            if (t0 + 1 < t1) load(s0, t0 + 1);
            if (t0 + 2 < t1) load(s1, t0 + 2);
        }
        __syncthreads();
        auto round = [&](Stage& sa, int t, int b) {
            if (t + 1 < t1) {
                store(sa, b ^ 1);
                if (t + 3 < t1) load(sa, t + 3);
            }
            if (wave_live && t * KT <= wave_lim && (!WIN || (t + 1) * KT > wave_lo_min))
                    tile(b, t * KT, nu_c, ub);
            __syncthreads();
        };
        for (int t = t0; t < t1; t += 2) {
            round(s0, t, 0);
            if (t + 1 < t1) round(s1, t + 1, 1);
        }
#else
        Stage st;
        if (t0 < t1) {
            load(st, t0);
            store(st, 0);
            if (t0 + 1 < t1) load(st, t0 + 1);
        }
        __syncthreads();
        for (int t = t0; t < t1; t++) {
            const int b = (t - t0) & 1;
            if (t + 1 < t1) {
                store(st, b ^ 1);
                if (t + 2 < t1) load(st, t + 2);
            }
            if (wave_live && t * KT <= wave_lim && (!WIN || (t + 1) * KT > wave_lo_min))
                    tile(b, t * KT, nu_c, ub);
            __syncthreads();
        }
#endif
    };
    if constexpr (KS_OK) {
        if (ks_half)
            main_loop(std::integral_constant<int, NSUB / 2>{}, ks_ub);
        else
            main_loop(std::integral_constant<int, NSUB>{}, 0);
    } else {
        main_loop(std::integral_constant<int, NSUB>{}, 0);
    }
    }

    // ---- key-split halves: the second half of each split tile (sub-blocks
    // from NSUB/2) parks its (m, l, O) in tile buffer 0, which the loop's
    // last barrier freed; the first half combines them into its own.
    if constexpr (KS_OK) {
        if (ks_any) {
            // slot = the tile's place mod 4: [4][64 lanes] (m, l), then [4][NT][64] O
            float2* const kml = (float2*)lds;
            float4v* const ko = (float4v*)(lds + 4 * 64 * sizeof(float2));
            static_assert(4 * 64 * sizeof(float2) + 4 * NT * 64 * sizeof(float4v) <= BUF,
                          "the split halves' exchange fits tile buffer 0");
            const int slot = ((wrow0 - row0) >> 4) & 3;
            if (ks_half && ks_ub != 0 && wave_live) {
                kml[slot * 64 + lane] = float2{m_run[0], l_run[0]};
#pragma unroll
                for (int mm = 0; mm < NT; mm++) ko[(slot * NT + mm) * 64 + lane] = acc_o[0][mm];
            }
            __syncthreads();
            if (ks_half && ks_ub == 0 && wave_live) {
                const float2 mlb = kml[slot * 64 + lane];
                const float ma = m_run[0], mb = mlb.x, M = fmaxf(ma, mb);
                // (the fused pass's maxima are in log2 units)
                auto fac = [&](float mx) {
                    return mx == -INFINITY ? 0.0f
                                           : __builtin_amdgcn_exp2f(FUSED ? mx - M : (mx - M) * kLog2e);
                };
                const float fa = fac(ma), fb = fac(mb);
                l_run[0] = l_run[0] * fa + mlb.y * fb;
                float fai[4], fbi[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    fai[i] = __shfl(fa, 4 * g + i);
                    fbi[i] = __shfl(fb, 4 * g + i);
                }
#pragma unroll
                for (int mm = 0; mm < NT; mm++) {
                    const float4v ob = ko[(slot * NT + mm) * 64 + lane];
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc_o[0][mm][i] = __builtin_fmaf(acc_o[0][mm][i], fai[i], ob[i] * fbi[i]);
                }
                m_run[0] = M;
            }
            // the second halves write nothing
            if (ks_half && ks_ub != 0) return;
        }
    }

    // ---- epilogue: per column, the row sum over the 4 lane groups.
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        float lsum = l_run[rt];
        lsum = wave_sum_g(lsum);
        const int rbase = wrow0 + 16 * rt + 4 * g;  // rows of acc_o[rt][.][i] are rbase + i
        if (n_split == 1) {
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
                const int64_t obase = ((int64_t)(h * a.G + row % a.G) * a.Tq + row / a.G) * D;
#pragma unroll
                for (int mm = 0; mm < NT; mm++) {
                    const int d = v_logical_dim(16 * mm + r16, D, VB);
                    a.out[obase + d] = (f16)(acc_o[rt][mm][i] * inv[i]);
                }
            }
        } else if constexpr (kPart16 && !FUSED) {
            // fp16 partials: row O / l rounded once, lane r16's NT slots
            // 16 mm + r16 at places NT r16 + mm (whole 16-byte stores), and
            // (m, l) in fp32
            const int64_t pbase = ((int64_t)h * n_split + sp) * a.PR - a.prow0;
            const int rho = wrow0 + 16 * rt + r16;
            if (g == 0 && rho < a.R) a.part_ml[pbase + rho] = float2{m_run[rt], lsum};
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
                f16* prow = (f16*)a.part_o + (pbase + row) * D + NT * r16;
#pragma unroll
                for (int c = 0; c < NT / 8; c++) {
                    half8 y;
#pragma unroll
                    for (int j = 0; j < 8; j++) y[j] = (f16)(acc_o[rt][8 * c + j][i] * inv[i]);
                    *(half8*)(prow + 8 * c) = y;
                }
            }
        } else {
            const int64_t pbase = ((int64_t)h * n_split + sp) * a.PR - a.prow0;
            const int rho = wrow0 + 16 * rt + r16;
            // (the fused pass's maxima are in log2 units; the merge takes natural ones)
            if (g == 0 && rho < a.R) a.part_ml[pbase + rho] = float2{FUSED ? m_run[rt] * kLn2 : m_run[rt], lsum};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = rbase + i;
                if (row >= a.R) continue;
                // partial rows in V slot order (lanes r16 of output tile mm
                // store 16 consecutive floats; the merge kernel reads dim d
                // from slot v_phys_dim(d)): measured c4 56 -> 51.4 us against
                // scattered dim-order stores
                float* prow = a.part_o + (pbase + row) * D;
#pragma unroll
                for (int mm = 0; mm < NT; mm++) prow[16 * mm + r16] = acc_o[rt][mm][i];
            }
        }
    }
}

template <int BITS, int D, int RT, int T4M = 0, bool APP = false, int PM = 0, bool ROPE = false,
          bool WIN = false, bool CAP = false>
__global__ __launch_bounds__(64 * block_waves<PM>(), 1) void attend_block_kernel(BlockArgs a) {
    static_assert(!ROPE || (APP && PM == 0), "RoPE launches are verify blocks that append");
    static_assert(!WIN || (PM == 0 && !APP && T4M == 0), "window launches attend a cache as it is");
    static_assert(!CAP || WIN, "softcap launches are window launches (an unbounded window)");
    // two buffers, each a K and a V tile of KT keys in fp16 (~130 KB)
    extern __shared__ __attribute__((aligned(16))) char lds_buf[];
    // The exact 2-op dequant runs without waiting for the cache's fast flag;
    // a launch whose cache holds a scale outside its exact range redoes the
    // workgroup's share with the separately rounded dequant (same threads,
    // same output elements, so the second pass's writes replace the first's).
    // A null flag (Int8 caches) takes the separately rounded dequant directly.
    // Turbo4 caches have one expansion (a null flag).
    if constexpr (APP && BITS != 16 && T4M == 0) {
        if ((int)blockIdx.x < a.n_app) {
            // the new rows of head blockIdx.x go into the cache first (the
            // append kernel's work, 8-token V block by block); this
            // workgroup's tiles then read them back, and its fast-flag check
            // below sees its own rows' scales
            const int L = a.T - a.T_pre;
            auto& sc = *reinterpret_cast<AppendScratch<D>*>(lds_buf);
            for (int blk = a.T_pre / 8; blk <= (a.T - 1) / 8; blk++) {
                append_block<D>(a.app, L, a.T_pre, BITS, a.app_int8 != 0, a.cap,
                                (uint32_t*)a.k_data, (uint32_t*)a.k_params, (uint32_t*)a.v_data,
                                (f16*)a.v_params, (int*)a.fast_flag, blk, blockIdx.x, threadIdx.x,
                                64 * kBlockWaves, sc);
                __syncthreads();
            }
        }
    }
    if constexpr (APP && T4M != 0) {
        if ((int)blockIdx.x < a.n_app) {
            // Turbo4: the 2L row appends (K and V of each new token) of head
            // blockIdx.x, a wave a row
            const int L = a.T - a.T_pre;
            for (int job = (int)threadIdx.x >> 6; job < 2 * L; job += kBlockWaves)
                turbo4_append_row<D>(a.app, job >> 1, blockIdx.x, (job & 1) == 0, threadIdx.x & 63,
                                     a.T_pre, a.cap, a.t4_tab, a.t4_tab + T4Tab<D>::cb,
                                     (uint8_t*)a.k_data, (uint32_t*)a.k_params, (uint8_t*)a.v_data,
                                     (uint32_t*)a.v_params);
            __syncthreads();
        }
    }
    if constexpr (PM == 2) {
        // the images hold the dequantized tiles: no dequant, no fast flag
        block_body<BITS, D, RT, false, T4M, APP, 2>(a, lds_buf);
    } else if (T4M == 0 && (BITS == 16 || a.fast_flag != nullptr)) {
        block_body<BITS, D, RT, true, 0, APP, PM, ROPE, WIN, CAP>(a, lds_buf);
        if (BITS != 16 && *a.fast_flag == 0) {
            __syncthreads();
            block_body<BITS, D, RT, false, 0, APP, PM, ROPE, WIN, CAP>(a, lds_buf);
        }
    } else {
        block_body<BITS, D, RT, false, T4M, APP, PM, ROPE, WIN, CAP>(a, lds_buf);
    }
}

template <int BITS, int D, int RT, int T4M, bool APP = false, int PM = 0, bool ROPE = false,
          bool WIN = false, bool CAP = false>
static int launch_block_rt(KVCache& cc, BlockArgs& a, int n_qt, hipStream_t stream) {
    // two tile buffers (+ the Turbo4 centroid-pair table)
    const size_t shmem = (size_t)2 * BlockShape<D>::BUF + (T4M ? 256 * sizeof(float2) : 0);
    int rc = ensure_dynamic_lds((const void*)attend_block_kernel<BITS, D, RT, T4M, APP, PM, ROPE, WIN, CAP>, shmem);
    if (rc) return rc;
    const dim3 grid = a.n_app > 0    ? dim3(a.n_app + cc.hkv * (a.n_split - 1))
                      : a.n_main > 0 ? dim3(a.n_main + n_qt * cc.hkv * a.n_split)
                                     : dim3(a.n_split, n_qt, cc.hkv);
    hipLaunchKernelGGL((attend_block_kernel<BITS, D, RT, T4M, APP, PM, ROPE, WIN, CAP>), grid, dim3(64 * block_waves<PM>()), shmem,
                       stream, a);
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

// 1: verify blocks on affine and Int8 caches append their rows inside the
// attention launch (launch_block_append_attention); 0: a separate append.
#ifndef QW_BLOCK_APPEND
#define QW_BLOCK_APPEND 1
#endif

// Row tiles a wave owns: the fewest workgroup rounds on 256 CUs (one
// workgroup a CU), weighing the larger RT's longer rounds.
#ifndef QW_BLOCK_RT
#define QW_BLOCK_RT 0  // 0: automatic; 1..3 forces the row tiles a wave owns
#endif
#ifndef QW_BLOCK_MAX_RT
#define QW_BLOCK_MAX_RT 1  // RT >= 2 exceeds the 256-register budget of two waves a SIMD
#endif
static int pick_rt(int R, int hkv) {
    if (QW_BLOCK_RT > 0) return QW_BLOCK_RT;
    // up to 192 rows a head: one query tile, so the K/V tiles are dequantized
    // once (verify blocks; the key split fills the CUs)
    if (R <= 16 * kBlockWaves * QW_BLOCK_MAX_RT) return (R + 16 * kBlockWaves - 1) / (16 * kBlockWaves);
    int best = 1;
    double best_cost = 1e30;
    for (int rt = 1; rt <= QW_BLOCK_MAX_RT; rt++) {
        const int wg_rows = 16 * kBlockWaves * rt;
        const int units = ((R + wg_rows - 1) / wg_rows) * hkv;
        const int rounds = (units + 255) / 256;
        // a round costs about RT (MFMA work a wave) plus a fixed dequant share
        const double cost = rounds * (rt + 0.5);
        if (cost < best_cost - 1e-9) {
            best_cost = cost;
            best = rt;
        }
    }
    return best;
}

template <int BITS, int D, int T4M, int PM = 0, bool WIN = false, bool CAP = false>
static int launch_one(KVCache& cc, BlockArgs a, int rt, int n_qt, hipStream_t stream) {
    int rc = QW_OK;
    if constexpr (QW_BLOCK_MAX_RT >= 3 || QW_BLOCK_RT == 3) {
        if (rt == 3) rc = launch_block_rt<BITS, D, 3, T4M, false, PM, false, WIN, CAP>(cc, a, n_qt, stream);
    }
    if constexpr (QW_BLOCK_MAX_RT >= 2 || QW_BLOCK_RT == 2) {
        if (rt == 2) rc = launch_block_rt<BITS, D, 2, T4M, false, PM, false, WIN, CAP>(cc, a, n_qt, stream);
    }
    if (rt == 1) rc = launch_block_rt<BITS, D, 1, T4M, false, PM, false, WIN, CAP>(cc, a, n_qt, stream);
    return rc;
}

// 1: unsplit and split query tiles of a call in one launch (see
// launch_block_bits); 0: two launches.
#ifndef QW_BLOCK_ONE_LAUNCH
#define QW_BLOCK_ONE_LAUNCH 1
#endif

// 1: prefill calls with at least kImageMinRows query rows a KV head (affine,
// Int8 and fp16 caches) dequantize (fp16: lay out) each key tile once into an
// image of its LDS buffer and attend from the images; 0: every query tile
// does that work again. The expansion costs about as much as 2200 rows a KV head gain
// (measured at 8k and 18k keys: 512 rows of 6 heads 146 -> 136 us, config 3
// 942 -> 826 us).
#ifndef QW_BLOCK_IMAGES
#define QW_BLOCK_IMAGES 1
#endif
constexpr int kImageMinRows = 3072;
// 1: causal image launches whose query tiles fill whole rounds pair an early
// and a late half tile in each workgroup (equal work a CU); 0: one tile each.
#ifndef QW_BLOCK_PAIR
#define QW_BLOCK_PAIR 1
#endif
// Turbo4 (the block kernel's fp16 arithmetic on the expansion's values): from
// 1025 rows a KV head, where the alternative expands the cache to fp16 rows
// at about the images' cost.
constexpr int kT4ImageMinRows = 1025;

namespace {
std::mutex g_img_mu;
std::map<std::pair<int, hipStream_t>, GrowBuffer> g_img_ws;
// The tile images' buffer, one per (device, stream) like the other
// transient workspaces (stream-ordered reuse; capture-safe growth).
int image_workspace(int device, hipStream_t stream, size_t need, void** out) {
    std::lock_guard<std::mutex> lock(g_img_mu);
    GrowBuffer& b = g_img_ws[{device, stream}];
    b.stream_owned = true;  // only calls on `stream` use it
    return b.get(need, stream, out);
}
}  // namespace

// Splits `n_tiles` key tiles into about `want` parts of at least min_tiles
// tiles (4: a workgroup's fixed costs amortized over its rounds; a window's
// few tiles spread wider).
static void split_keys(int n_tiles, int want, int* n_split, int* tps, int min_tiles = 4) {
    int ns = std::max(1, std::min({want, (n_tiles + min_tiles - 1) / min_tiles, 256}));
    *tps = (n_tiles + ns - 1) / ns;
    *n_split = (n_tiles + *tps - 1) / *tps;
}

// window > 0 (causal, T4M = 0): the WIN kernels, splits over the keys a query
// tile's windows span
template <int BITS, int D, int T4M = 0>
static int launch_block_bits(KVCache& cc, const f16* q, int G, int Tq, float scale, bool causal,
                             f16* out, hipStream_t stream, const float* t4_tab = nullptr,
                             int window = 0, float softcap = 0.0f) {
    using S = BlockShape<D>;
    const int T = cc.offset;
    const int R = G * Tq;
    const int n_tiles = (T + S::KT - 1) / S::KT;
    // long prefill calls dequantize (fp16: lay out) each key tile once into an
    // image of its LDS buffer and attend from the images, in query tiles of
    // 16 kImageWaves rows
    const bool images = QW_BLOCK_IMAGES && T4M != 2 && window <= 0 && softcap <= 0.0f &&
                        R >= (T4M ? kT4ImageMinRows : kImageMinRows) && n_tiles > 0;
    const int rt = images ? 1 : pick_rt(R, cc.hkv);
    const int wg_rows = 16 * (images ? kImageWaves : kBlockWaves) * rt;
    const int n_qt = (R + wg_rows - 1) / wg_rows;
    const int units = n_qt * cc.hkv;

    BlockArgs a;
    a.k_data = (const uint32_t*)cc.k_data;
    a.k_params = cc.k_params;
    a.v_data = (const uint32_t*)cc.v_data;
    a.v_params = cc.v_params;
    a.fast_flag = cc.int8() || T4M ? nullptr : cc.fast_flag;  // null: always separately rounded
    a.q = q;
    a.out = out;
    a.t4_tab = t4_tab;
    a.t4_post = scale * 1.4426950408889634f;
    a.part_o = nullptr;
    a.part_ml = nullptr;
    a.cap = cc.cap;
    a.T = T;
    a.Tq = Tq;
    a.G = G;
    a.R = R;
    a.causal = causal ? 1 : 0;
    a.scale_h = (float)(f16)scale;
    a.code_off2 = cc.code_offset2();
    a.qt0 = 0;
    a.prow0 = 0;
    a.PR = R;
    a.n_main = 0;
    a.main_tiles = n_tiles;
    a.hkv = cc.hkv;
    a.n_app = 0;
    a.T_pre = T;
    a.app_int8 = 0;
    a.app = RowSrc{};
    a.img_w = nullptr;
    a.img = nullptr;
    a.img_tiles = n_tiles;
    a.pair_h = 0;
    // (a softcap launch without a window: one wider than any position)
    a.window = window > 0 ? window : softcap > 0.0f ? (1 << 30) : 0;
    a.softcap = softcap;
    a.scale = scale;
    int rc;
    if constexpr (T4M != 2) {
        if (images) {
            void* img = nullptr;
            rc = image_workspace(cc.device, stream, (size_t)cc.hkv * n_tiles * S::BUF, &img);
            if (rc) return rc;
            a.img_w = (char*)img;
            a.img = (const char*)img;
            // (Turbo4: the store's centroid-pair table sits behind two buffers)
            const size_t shmem = T4M ? 2 * S::BUF + 256 * sizeof(float2) : S::BUF;
            rc = ensure_dynamic_lds((const void*)attend_block_kernel<BITS, D, 1, T4M, false, 1>, shmem);
            if (rc) return rc;
            hipLaunchKernelGGL((attend_block_kernel<BITS, D, 1, T4M, false, 1>), dim3(n_tiles, cc.hkv),
                               dim3(64 * kBlockWaves), shmem, stream, a);
            QW_HIP_CHECK(hipGetLastError());
        }
    }

    // Plan (one workgroup a CU, 256 CUs): query tiles that fill whole rounds
    // run unsplit and write their rows; the rest (all of them when fewer than
    // 256 units) split the keys so that about 256 workgroups run, and go
    // through fp32 partials and the merge kernel.
    // With both parts, one launch: the unsplit tiles first, the split ones
    // behind them, so a CU whose unsplit tile ends early starts a split one
    // (the unsplit tiles' lengths differ with the causal cut) and no kernel
    // boundary separates them.
    // The Turbo4 fused pass splits every row (its merge rotates them back).
    int q_main = 0;
    if (units >= 256 && 256 % cc.hkv == 0 && T4M != 2) q_main = (units / 256) * (256 / cc.hkv);
    q_main = std::min(q_main, n_qt);
    const int q_tail = n_qt - q_main;
    auto launch = [&](BlockArgs& x, int n_qt_) {
        if constexpr (T4M != 2) {
            if (images) return launch_one<BITS, D, T4M, 2>(cc, x, rt, n_qt_, stream);
        }
        if constexpr (T4M == 0) {
            if (softcap > 0.0f) return launch_one<BITS, D, 0, 0, true, true>(cc, x, rt, n_qt_, stream);
            if (window > 0) return launch_one<BITS, D, 0, 0, true>(cc, x, rt, n_qt_, stream);
        }
        return launch_one<BITS, D, T4M>(cc, x, rt, n_qt_, stream);
    };
    if (q_main > 0 && (q_tail == 0 || !QW_BLOCK_ONE_LAUNCH)) {
        BlockArgs m = a;
        m.n_split = 1;
        // causal image launches of whole rounds: balanced half-tile pairs
        if (QW_BLOCK_PAIR && images && causal && T4M == 0 && q_tail == 0 && Tq > 1)
            m.pair_h = (R + wg_rows / 2 - 1) / (wg_rows / 2);
        m.tiles_per_split = n_tiles;
        rc = launch(m, q_main);
        if (rc) return rc;
    }
    if (q_tail == 0) return QW_OK;
    int n_split, tps;
    const int want = std::max(1, 256 / (q_tail * cc.hkv));
    // (a window: the keys from a query tile's first window start to its last row)
    const int plan_tiles =
        window > 0 ? std::min(n_tiles, (window + wg_rows / G + 1 + S::KT - 1) / S::KT + 1) : n_tiles;
    split_keys(plan_tiles, T4M == 2 ? std::min(std::max(want, 2), 128) : want, &n_split, &tps,
               window > 0 ? QW_WINDOW_MIN_TILES : 4);
    QW_REQUIRE(T4M != 2 || n_split > 1, QW_ERR_INVALID_ARGUMENT,
               "block attention: fused Turbo4 pass needs at least 5 key tiles");
    BlockArgs t = a;
    if (q_main > 0 && QW_BLOCK_ONE_LAUNCH) t.n_main = q_main * cc.hkv;
    t.qt0 = q_main;
    t.n_split = n_split;
    t.tiles_per_split = tps;
    t.prow0 = q_main * wg_rows;
    t.PR = R - t.prow0;
    if (n_split > 1) {
        const size_t o_bytes = (size_t)cc.hkv * n_split * t.PR * D * sizeof(float);
        const size_t need = o_bytes + (size_t)cc.hkv * n_split * t.PR * sizeof(float2);
        rc = cc.ensure_workspace(need, stream);
        if (rc) return rc;
        t.part_o = (float*)cc.ws_ptr;
        t.part_ml = (float2*)((char*)cc.ws_ptr + o_bytes);
    }
    rc = launch(t, q_tail);
    if (rc) return rc;
    if (n_split > 1 && T4M == 2)
        return launch_t4_merge_rotate(t.part_o, t.part_ml, n_split, t.PR, R, cc.hkv, D, G, Tq, 16,
                                      true, t4_tab, out, stream);
    if (n_split > 1 && kPart16)
        return launch_partial_merge_h((const f16*)t.part_o, t.part_ml, n_split, t.PR, t.prow0, t.PR,
                                      cc.hkv, D, G, Tq, out, stream, T4M ? 16 : BITS);
    if (n_split > 1)
        return launch_partial_merge(t.part_o, t.part_ml, n_split, t.PR, t.prow0, t.PR, cc.hkv, D,
                                    G, Tq, out, stream, T4M ? 16 : BITS);
    return QW_OK;
}

int launch_block_attention_ext(KVCache& cc, const f16* q, int G, int n_rows, float scale,
                               bool causal, int window, float softcap, f16* out,
                               hipStream_t stream) {
    QW_REQUIRE(cc.affine() || cc.bits == 16, QW_ERR_INVALID_ARGUMENT,
               "block attention: window / softcap route is for affine, Int8 and fp16 caches");
    QW_REQUIRE((window > 0 || softcap > 0.0f) && (window <= 0 || causal) &&
                   (cc.D == 128 || cc.D == 256),
               QW_ERR_INVALID_ARGUMENT, "block attention: window / softcap launch outside its shapes");
    const int w = window > 0 ? window : 0;
    if (cc.D == 256) {
        if (cc.bits == 4) return launch_block_bits<4, 256>(cc, q, G, n_rows, scale, causal, out, stream, nullptr, w, softcap);
        if (cc.bits == 8) return launch_block_bits<8, 256>(cc, q, G, n_rows, scale, causal, out, stream, nullptr, w, softcap);
        return launch_block_bits<16, 256>(cc, q, G, n_rows, scale, causal, out, stream, nullptr, w, softcap);
    }
    if (cc.bits == 4) return launch_block_bits<4, 128>(cc, q, G, n_rows, scale, causal, out, stream, nullptr, w, softcap);
    if (cc.bits == 8) return launch_block_bits<8, 128>(cc, q, G, n_rows, scale, causal, out, stream, nullptr, w, softcap);
    return launch_block_bits<16, 128>(cc, q, G, n_rows, scale, causal, out, stream, nullptr, w, softcap);
}

int launch_block_attention_t4(KVCache& cc, const f16* q, int G, int n_rows, float scale,
                              bool causal, bool fused, const float* tab, f16* out,
                              hipStream_t stream) {
    QW_REQUIRE(cc.turbo4() && cc.bits == 4, QW_ERR_INVALID_ARGUMENT, "block attention: not Turbo4");
    if (cc.D == 256)
        return fused ? launch_block_bits<4, 256, 2>(cc, q, G, n_rows, scale, causal, out, stream, tab)
                     : launch_block_bits<4, 256, 1>(cc, q, G, n_rows, scale, causal, out, stream, tab);
    return fused ? launch_block_bits<4, 128, 2>(cc, q, G, n_rows, scale, causal, out, stream, tab)
                 : launch_block_bits<4, 128, 1>(cc, q, G, n_rows, scale, causal, out, stream, tab);
}

// Verify blocks on affine and Int8 caches: the append rides in the attention
// launch (see BlockArgs::n_app). The prefix splits are planned for the CUs the
// append workgroups leave free; every row sees the whole prefix, so the
// prefix splits need no causal cut and the partial slot of the new keys
// carries it.
template <int BITS, int D, int T4M = 0>
static int launch_block_append_bits(KVCache& cc, const f16* q, int G, int L, const f16* k_new,
                                    const f16* v_new, float scale, bool causal, f16* out,
                                    hipStream_t stream, const float* t4_tab = nullptr,
                                    const RowSrc* rope = nullptr, f16* q_out = nullptr) {
    using S = BlockShape<D>;
    const int T_pre = cc.offset, T = T_pre + L, R = G * L;
    BlockArgs a;
    a.k_data = (const uint32_t*)cc.k_data;
    a.k_params = cc.k_params;
    a.v_data = (const uint32_t*)cc.v_data;
    a.v_params = cc.v_params;
    a.fast_flag = cc.int8() || T4M ? nullptr : cc.fast_flag;
    a.q = q;
    a.out = out;
    a.t4_tab = t4_tab;
    a.t4_post = scale * 1.4426950408889634f;
    a.cap = cc.cap;
    a.T = T;
    a.Tq = L;
    a.G = G;
    a.R = R;
    a.causal = causal ? 1 : 0;
    a.scale_h = (float)(f16)scale;
    a.code_off2 = cc.code_offset2();
    a.qt0 = 0;
    a.prow0 = 0;
    a.PR = R;
    a.n_main = 0;
    a.main_tiles = 0;
    a.hkv = cc.hkv;
    a.n_app = cc.hkv;
    a.T_pre = T_pre;
    a.app_int8 = cc.int8() ? 1 : 0;
    a.app = RowSrc{};
    a.app.k = k_new;
    a.app.v = v_new;
    a.app.row_stride = D;
    a.app.head_stride = (int64_t)L * D;
    a.q_tok_stride = 0;
    a.q_out = nullptr;
    if (rope) {
        // q is the projection [L][(G hkv + 2 hkv) D]; k_new / v_new are inside it
        QW_REQUIRE(rope->rope_dims % 16 == 0 && rope->rope_dims <= D && q_out,
                   QW_ERR_INVALID_ARGUMENT, "block attention: RoPE launch outside its shapes");
        a.app = *rope;
        a.q_tok_stride = (int64_t)(G + 2) * cc.hkv * D;
        a.q_out = q_out;
    }
    a.img_w = nullptr;
    a.img = nullptr;
    a.img_tiles = 0;
    a.pair_h = 0;
    int n_pre, tps;
    // (the Turbo4 fused pass's merge takes up to 128 partials)
    const int want = std::max(1, (256 - cc.hkv) / cc.hkv);
    split_keys((T_pre + S::KT - 1) / S::KT, T4M == 2 ? std::min(want, 127) : want, &n_pre, &tps);
    a.n_split = n_pre + 1;
    a.tiles_per_split = tps;
    const size_t o_bytes = (size_t)cc.hkv * a.n_split * R * D * sizeof(float);
    int rc = cc.ensure_workspace(o_bytes + (size_t)cc.hkv * a.n_split * R * sizeof(float2), stream);
    if (rc) return rc;
    a.part_o = (float*)cc.ws_ptr;
    a.part_ml = (float2*)((char*)cc.ws_ptr + o_bytes);
    rc = rope ? launch_block_rt<BITS, D, 1, T4M, true, 0, true>(cc, a, 1, stream)
              : launch_block_rt<BITS, D, 1, T4M, true>(cc, a, 1, stream);
    if (rc) return rc;
    cc.offset = T;
    if (T4M == 2)
        return launch_t4_merge_rotate(a.part_o, a.part_ml, a.n_split, R, R, cc.hkv, D, G, L, 16, true,
                                      t4_tab, out, stream);
    if (kPart16)
        return launch_partial_merge_h((const f16*)a.part_o, a.part_ml, a.n_split, R, 0, R, cc.hkv, D,
                                      G, L, out, stream, T4M ? 16 : BITS);
    return launch_partial_merge(a.part_o, a.part_ml, a.n_split, R, 0, R, cc.hkv, D, G, L, out,
                                stream, T4M ? 16 : BITS);
}

int block_image_min_rows(bool turbo4) {
    return QW_BLOCK_IMAGES ? (turbo4 ? kT4ImageMinRows : kImageMinRows) : 1 << 30;
}

bool block_append_fits(const KVCache& cc, int G, int L) {
    return QW_BLOCK_APPEND && cc.affine() && (cc.D == 128 || cc.D == 256) && L >= 2 &&
           G * L > 16 && G * L <= 16 * kBlockWaves && cc.offset >= 256;
}

int launch_block_append_attention(KVCache& cc, const f16* q, int G, int L, const f16* k_new,
                                  const f16* v_new, float scale, bool causal, f16* out,
                                  hipStream_t stream, const RowSrc* rope, f16* q_out) {
    QW_REQUIRE(block_append_fits(cc, G, L) && cc.offset + L <= cc.cap, QW_ERR_INVALID_ARGUMENT,
               "block attention: verify block outside the fused-append shapes");
    if (cc.D == 256)
        return cc.bits == 4 ? launch_block_append_bits<4, 256>(cc, q, G, L, k_new, v_new, scale,
                                                               causal, out, stream, nullptr, rope, q_out)
                            : launch_block_append_bits<8, 256>(cc, q, G, L, k_new, v_new, scale,
                                                               causal, out, stream, nullptr, rope, q_out);
    return cc.bits == 4 ? launch_block_append_bits<4, 128>(cc, q, G, L, k_new, v_new, scale, causal,
                                                           out, stream, nullptr, rope, q_out)
                        : launch_block_append_bits<8, 128>(cc, q, G, L, k_new, v_new, scale, causal,
                                                           out, stream, nullptr, rope, q_out);
}

bool block_append_fits_t4(const KVCache& cc, int G, int L) {
    return cc.turbo4() && G * L <= 16 * kBlockWaves && cc.offset >= 256;
}

int launch_block_append_attention_t4(KVCache& cc, const f16* q, int G, int L, const f16* k_new,
                                     const f16* v_new, float scale, bool causal, bool fused,
                                     const float* tab, f16* out, hipStream_t stream,
                                     const RowSrc* rope, f16* q_out) {
    QW_REQUIRE(block_append_fits_t4(cc, G, L) && cc.offset + L <= cc.cap,
               QW_ERR_INVALID_ARGUMENT, "block attention: Turbo4 block outside the fused-append shapes");
    QW_REQUIRE(!rope || fused, QW_ERR_INVALID_ARGUMENT,
               "block attention: Turbo4 RoPE launches take the fused verify pass");
    if (cc.D == 256)
        return fused ? launch_block_append_bits<4, 256, 2>(cc, q, G, L, k_new, v_new, scale, causal,
                                                           out, stream, tab, rope, q_out)
                     : launch_block_append_bits<4, 256, 1>(cc, q, G, L, k_new, v_new, scale, causal,
                                                           out, stream, tab);
    return fused ? launch_block_append_bits<4, 128, 2>(cc, q, G, L, k_new, v_new, scale, causal, out,
                                                       stream, tab, rope, q_out)
                 : launch_block_append_bits<4, 128, 1>(cc, q, G, L, k_new, v_new, scale, causal, out,
                                                       stream, tab);
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
