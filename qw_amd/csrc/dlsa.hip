// dlsa.hip - D-LSA gathered sparse attention (the K2 read), gfx950.
//
// Reference: dlsa_attention::sparse_attention (crates/mlxcel-core/src/
// dlsa_attention.rs:31-63) -> mlx_cxx::dlsa_sparse_attention
// (crates/mlxcel-core/cpp/mlx_cxx_dlsa_attention.cpp:81-330 kernels,
// :379-556 launch policy and validation). Contract: every query row r attends
// over lists[r, 0:lengths[r]] of its KV head (shared by the G heads of the
// group), entries outside [0, T) are skipped, a row with no valid entry is
// zeros, fp32 softmax and accumulation, output in q's dtype (fp16 here),
// K/V read in place through their strides.
//
// Design:
//   grid (parts, rows, kv_heads), 4 waves a workgroup. A part is a contiguous
//   slice of the row's list; waves take 16-entry tiles of it in turn.
//   Q.K^T on MFMA (v_mfma_f32_16x16x32_f16): A = 16 gathered K rows (each
//   lane 16 contiguous bytes of its row per MFMA), B = the G query heads.
//   P.V on MFMA too (v_mfma_f32_16x16x16_f16): the S^T tile already holds P
//   in the A-operand layout, and V is gathered straight into the B layout as
//   8-byte row pieces (16 lanes cover 128 contiguous bytes of a row); P goes
//   in as an fp16 high part plus an fp16 remainder, so every product is exact
//   and the accumulation is fp32.
//   Online softmax in the exp2 domain across tiles; the waves merge through
//   LDS; split-K parts write fp32 partials merged by a second kernel.
#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <type_traits>

#include "dequant.hpp"
#include "kv_cache.hpp"

namespace qw {

struct DlsaArgs {
    const f16* q;
    const int32_t* lists;
    const int32_t* lengths;
    f16* out;
    float* part_o;   // [L][Hq][parts][D]
    float2* part_ml; // [L][Hq][parts]
    int L, W, hq, hkv, G, T, parts;
    float scale2;    // scale * log2(e)
};

constexpr int kDlsaNT = 2;  // tiles per batch a wave keeps in flight

// ---------------------------------------------------------- row sources
//
// Where the gathered K and V rows come from. A source loads the raw registers
// of one 16-entry tile for a lane (g, r16) (the K row of entry r16, the QK A
// operand; entries 4g..4g+3, the P.V B operand) and turns them into MFMA
// operands:
//   k_op(m):     A operand of QK MFMA m, 8 dims of entry r16 (which dims, and
//                in which order, is the source's q layout kQ, shared with the
//                q operand);
//   v_op(pp, c): B operand of P.V tile (pp, c), entries 4g..4g+3 of dim
//                64 pp + 4 r16 + c.
// `aligned` (wave-uniform) says that every lane group's four entries are four
// consecutive keys starting at a multiple of 4: they then sit in one half of
// an 8-key V block, which the cache sources read with whole-word loads.

// q layouts: dims of MFMA m for lane group g
//   kQNatural: 32 m + 8 g .. +7
//   kQGroup:   (D/4) g + 8 m .. +7 (a lane group's dims are one contiguous run)
//   kQGroup4:  as kQGroup, in the pair order (0,4),(1,5),(2,6),(3,7) that the
//              4-bit magic-number dequant produces
enum { kQNatural = 0, kQGroup = 1, kQGroup4 = 2 };

// fp16 K/V views with strides: the K2 contract (strided views of a larger
// cache read in place).
template <int D>
struct SrcStrided {
    static constexpr int kQ = kQNatural;
    static constexpr bool kHasAligned = false;
    static constexpr bool kAffine = false;
    static constexpr int kNT = kDlsaNT;
    static constexpr bool kPairs = true;  // the two-row form fits the registers
    static constexpr int NM = D / 32, NP = D / 64;
    const f16* k;
    const f16* v;
    int64_t khs, krs, vhs, vrs;
    struct Regs {
        u32x4 kc[NM];
        u32x2 vq[4][NP];  // entry 4g + j: dims 64 pp + 4 r16 .. +3
    };
    template <bool ALIGNED>
    __device__ __forceinline__ void load(Regs& r, int h, int key, const int* key4, int r16,
                                         int g) const {
        const u32x4* krow = (const u32x4*)(k + h * khs + (int64_t)key * krs);
#pragma unroll
        for (int m = 0; m < NM; m++) r.kc[m] = krow[4 * m + g];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const f16* vrow = v + h * vhs + (int64_t)key4[j] * vrs + 4 * r16;
#pragma unroll
            for (int pp = 0; pp < NP; pp++) r.vq[j][pp] = *(const u32x2*)(vrow + 64 * pp);
        }
    }
    template <bool FAST>
    __device__ __forceinline__ half8 k_op(const Regs& r, int m) const {
        return as_h8(r.kc[m]);
    }
    template <bool ALIGNED, bool FAST>
    __device__ __forceinline__ half4v v_op(const Regs& r, int pp, int c) const {
        // element c of the four entries' 4-dim pieces
        const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
        uint32_t w0, w1;
        if (c < 2) {
            w0 = __builtin_amdgcn_perm(r.vq[1][pp].x, r.vq[0][pp].x, sel);
            w1 = __builtin_amdgcn_perm(r.vq[3][pp].x, r.vq[2][pp].x, sel);
        } else {
            w0 = __builtin_amdgcn_perm(r.vq[1][pp].y, r.vq[0][pp].y, sel);
            w1 = __builtin_amdgcn_perm(r.vq[3][pp].y, r.vq[2][pp].y, sel);
        }
        return __builtin_bit_cast(half4v, u32x2{w0, w1});
    }
};

// An fp16 KV cache in place: K rows [hkv][cap][D]; V in 8-key blocks
// [hkv][cap/8][D][8] with dims in lane order (v_phys_dim).
template <int D>
struct SrcCacheF16 {
    static constexpr int kQ = kQNatural;
    static constexpr bool kHasAligned = true;
    static constexpr bool kAffine = false;
    static constexpr int kNT = kDlsaNT;
    static constexpr bool kPairs = D <= 128;  // (at D = 256 the two-row form spills)
    static constexpr int NM = D / 32, NP = D / 64;
    const f16* k;
    const f16* v;
    int cap;
    struct Regs {
        u32x4 kc[NM];
        u32x2 vq[NP][4];  // (pp, c): entries 4g..4g+3 of dim 64 pp + 4 r16 + c
    };
    template <bool ALIGNED>
    __device__ __forceinline__ void load(Regs& r, int h, int key, const int* key4, int r16,
                                         int g) const {
        const u32x4* krow = (const u32x4*)(k + ((int64_t)h * cap + key) * D);
#pragma unroll
        for (int m = 0; m < NM; m++) r.kc[m] = krow[4 * m + g];
        const f16* vh = v + ((int64_t)h * (cap / 8) * D + v_slot_base(r16, D, 16)) * 8;
        if constexpr (ALIGNED) {
            const f16* blk = vh + (int64_t)(key4[0] >> 3) * D * 8 + (key4[0] & 4);
#pragma unroll
            for (int pp = 0; pp < NP; pp++)
#pragma unroll
                for (int c = 0; c < 4; c++)
                    r.vq[pp][c] = *(const u32x2*)(blk + v_slot_off(pp, c, D, 16) * 8);
        } else {
#pragma unroll
            for (int pp = 0; pp < NP; pp++)
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const int slot = v_slot_off(pp, c, D, 16) * 8;
                    uint16_t e[4];
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        e[j] = *(const uint16_t*)(vh + (int64_t)(key4[j] >> 3) * D * 8 + slot +
                                                  (key4[j] & 7));
                    r.vq[pp][c] = u32x2{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16)};
                }
        }
    }
    template <bool FAST>
    __device__ __forceinline__ half8 k_op(const Regs& r, int m) const {
        return as_h8(r.kc[m]);
    }
    template <bool ALIGNED, bool FAST>
    __device__ __forceinline__ half4v v_op(const Regs& r, int pp, int c) const {
        return __builtin_bit_cast(half4v, r.vq[pp][c]);
    }
};

// An affine (4/8-bit, group 64) or Int8 KV cache in place, dequantized inside
// the gather exactly as the fetch does it (MLX's composite f16(f16(c s) + b);
// Int8 codes are stored plus 128 with bias 0 and take the separately rounded
// dequant with magic offset 1152):
//   K codes [hkv][cap][D bits/32] u32 (MLX packing), params [hkv][cap][D/64]
//   half2(scale, bias) in k_param_slot order; V blocks of 8 keys,
//   [hkv][cap/8][D bits/4] u32 (dims in lane order, v_phys_dim), params
//   [hkv][cap/8][D/64][16] f16 (s0..s7, b0..b7).
// A lane group's K dims are one contiguous run (kQGroup), so its codes are
// KW contiguous words and one (scale, bias) pair.
template <int D, int BITS>
struct SrcCacheAffine {
    static constexpr int kQ = BITS == 4 ? kQGroup4 : kQGroup;
    static constexpr bool kHasAligned = true;
    static constexpr bool kAffine = true;
    // the dequantized operands and their constants fill the register budget
    // at D = 256 with two tiles in flight: one tile a batch there
    static constexpr int kNT = D == 256 ? 1 : kDlsaNT;
    static constexpr bool kPairs = D <= 128;  // (at D = 256 the two-row form spills)
    static constexpr int NM = D / 32, NP = D / 64, NG = D / 64;
    static constexpr int KW = NM * BITS / 4;   // K words of a lane group's D/4 dims
    static constexpr int RW = D * BITS / 32;   // K words a row
    static constexpr int VBW = D * BITS / 4;   // words of an 8-key V block
    const uint32_t* kc;
    const uint32_t* kp;
    const uint32_t* vc;
    const f16* vp;
    int cap;
    uint32_t off2;  // magic offset pair of the separately rounded dequant
    struct Regs {
        u32x4 kw[KW / 4];
        uint32_t kpar;         // half2(scale, bias) of the lane group's 64-dim group
        uint32_t vw[NP][4];    // (pp, c): codes of dim 64 pp + 4 r16 + c (ALIGNED 4-bit:
                               // the dim's block word; otherwise the four entries' codes,
                               // one a byte)
        u32x2 vs[NP], vb[NP];  // the four entries' V scales and biases of group pp
        int half;              // ALIGNED: keys 4..7 of the block (1) or 0..3 (0)
    };
    template <bool ALIGNED>
    __device__ __forceinline__ void load(Regs& r, int h, int key, const int* key4, int r16,
                                         int g) const {
        const u32x4* krow = (const u32x4*)(kc + ((int64_t)h * cap + key) * RW + KW * g);
#pragma unroll
        for (int i = 0; i < KW / 4; i++) r.kw[i] = krow[i];
        const int grp = (D / 4) * g / 64;
        r.kpar = kp[((int64_t)h * cap + key) * NG + k_param_slot(grp, NG)];
        // slots are in units of a dim's 8 codes: one word at 4-bit, two at 8-bit
        const uint32_t* vh =
            vc + (int64_t)h * (cap / 8) * VBW + v_slot_base(r16, D, BITS) * (BITS / 4);
        const f16* vph = vp + (int64_t)h * (cap / 8) * NG * 16;
        if constexpr (ALIGNED) {
            const int blk = key4[0] >> 3, half = (key4[0] >> 2) & 1;
            r.half = half;
            const uint32_t* bw = vh + (int64_t)blk * VBW + (BITS == 8 ? half : 0);
#pragma unroll
            for (int pp = 0; pp < NP; pp++) {
#pragma unroll
                for (int c = 0; c < 4; c++) r.vw[pp][c] = bw[v_slot_off(pp, c, D, BITS) * (BITS / 4)];
                const f16* pr = vph + ((int64_t)blk * NG + pp) * 16 + 4 * half;
                r.vs[pp] = *(const u32x2*)pr;
                r.vb[pp] = *(const u32x2*)(pr + 8);
            }
        } else {
            r.half = 0;
#pragma unroll
            for (int pp = 0; pp < NP; pp++) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const int slot = v_slot_off(pp, c, D, BITS) * (BITS / 4);
                    uint32_t codes = 0;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int t = key4[j], kk = t & 7;
                        const uint32_t* bw = vh + (int64_t)(t >> 3) * VBW;
                        const uint32_t code =
                            BITS == 4 ? (bw[slot] >> (4 * v4_nibble_pos(kk))) & 0xFu
                                      : (bw[slot + (kk >> 2)] >> (8 * (kk & 3))) & 0xFFu;
                        codes |= code << (8 * j);
                    }
                    r.vw[pp][c] = codes;
                }
                uint32_t sv[4], bv[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int t = key4[j];
                    const uint16_t* pr =
                        (const uint16_t*)(vph + ((int64_t)(t >> 3) * NG + pp) * 16 + (t & 7));
                    sv[j] = pr[0];
                    bv[j] = pr[8];
                }
                r.vs[pp] = u32x2{sv[0] | (sv[1] << 16), sv[2] | (sv[3] << 16)};
                r.vb[pp] = u32x2{bv[0] | (bv[1] << 16), bv[2] | (bv[3] << 16)};
            }
        }
    }
    template <bool FAST>
    __device__ __forceinline__ half8 k_op(const Regs& r, int m) const {
        const half2v sb = h2(r.kpar);
        const half2v s = {sb.x, sb.x}, b = {sb.y, sb.y};
        const PairConsts pc = make_consts<FAST, BITS>(s, s, s, s, b, b, b, b, off2);
        if constexpr (BITS == 4)
            return deq4<FAST>(r.kw[m / 4][m % 4], pc, vconst(kMagic));
        else
            return deq8<FAST>(r.kw[m / 2][2 * (m % 2)], r.kw[m / 2][2 * (m % 2) + 1], pc);
    }
    template <bool ALIGNED, bool FAST>
    __device__ __forceinline__ half4v v_op(const Regs& r, int pp, int c) const {
        // keys (0,1) and (2,3) of the four as magic-number pairs, then
        // f16(f16(code s_k) + b_k) with each key's own scale and bias
        const half2v s01 = h2(r.vs[pp].x), s23 = h2(r.vs[pp].y);
        const half2v b01 = h2(r.vb[pp].x), b23 = h2(r.vb[pp].y);
        const half2v off = h2(off2);
        const half2v k1024 = {(f16)-1024.0f, (f16)-1024.0f};
        half2v y01, y23;
        if constexpr (ALIGNED && BITS == 4) {
            // the dim's block word: key k at nibble k/2 + 4 (k % 2), keys 4..7
            // the same after a shift by 8; (k0, k1) come out of the low nibble
            // fields, (k2, k3) out of the x16 fields
            const uint32_t w = r.half ? r.vw[pp][c] >> 8 : r.vw[pp][c];
            const uint32_t magic = vconst(kMagic);
            const half2v s23x = s23 * (half2v){(f16)0.0625f, (f16)0.0625f};
            y01 = deq_pair<FAST, false>((w & 0x000F000Fu) | magic, s01, s01 * k1024, b01, off);
            y23 = deq_pair<FAST, true>((w & 0x00F000F0u) | magic, FAST ? s23x : s23,
                                       s23x * k1024, b23, off);
        } else {
            // four codes, one a byte
            const uint32_t p01 = __builtin_amdgcn_perm(0x64646464u, r.vw[pp][c], 0x04010400u);
            const uint32_t p23 = __builtin_amdgcn_perm(0x64646464u, r.vw[pp][c], 0x04030402u);
            y01 = deq_pair<FAST, false>(p01, s01, s01 * k1024, b01, off);
            y23 = deq_pair<FAST, false>(p23, s23, s23 * k1024, b23, off);
        }
        return half4v{y01.x, y01.y, y23.x, y23.y};
    }
};

// ---------------------------------------------------------- the kernel
//
// grid (parts, rows, kv_heads), 4 waves a workgroup. A part is a contiguous
// slice of the row's list; waves take 16-entry tiles of it in turn, kDlsaNT
// tiles a batch with all their gathers issued before the first use.
// Q.K^T on MFMA (v_mfma_f32_16x16x32_f16): A = 16 gathered K rows, B = the G
// query heads. P.V on MFMA too (v_mfma_f32_16x16x16_f16, K = the tile's 16
// entries): A = P (row = head r16, entries 4g..4g+3: exactly where the S^T
// tile leaves them), B = V (entries 4g..4g+3 of one dim). Output tile (p, c)
// holds heads 4g + i x dims 64p + 4 r16 + c. P enters as an fp16 high part
// and an fp16 remainder, so p * v is exact and the sums stay fp32 as in the
// reference.
// RP rows a workgroup (2: one-pass prefill calls, 2G <= 16): MFMA column c
// is query head c % G of row r0 + c / G. A tile index whose 16 entries are the
// same keys for both rows (sinks, shared blocks) is gathered once for both;
// otherwise each row's tile runs with the other row's columns masked.
template <int D, int GMAX, class Src, bool FAST, int RP = 1>
__device__ __forceinline__ void dlsa_body(const DlsaArgs& a, const Src& src) {
    constexpr int NM = D / 32;
    constexpr int NP = D / 64;  // 64-dim groups: P.V output tiles (p, c), c < 4
    const int part = blockIdx.x, r0 = blockIdx.y * RP, h = blockIdx.z;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, g = lane >> 4;
    const int G = a.G;
    const int nrow = RP == 1 ? 1 : min(RP, a.L - r0);  // rows this workgroup owns
    const int NC = RP == 1 ? G : nrow * G;              // live columns
    const int crow = RP == 1 ? 0 : r16 / G;             // the lane's column's row
    const int chead = RP == 1 ? r16 : r16 - crow * G;   // and its head in the group
    const bool col_ok = r16 < NC;
    // Parts split the list's width W at multiples of 16 entries, so the list
    // loads depend on the launch arguments only (not on the row's length, a
    // memory round trip of its own) and a list made of aligned key runs gives
    // aligned 4-entry groups in every part. The length, loaded alongside,
    // masks the entries at or past it.
    const int e_begin = (int)((int64_t)a.W * part / a.parts) & ~15;
    const int e_end = part + 1 == a.parts ? a.W : (int)((int64_t)a.W * (part + 1) / a.parts) & ~15;
    const int32_t* list[RP];
    int len[RP];
#pragma unroll
    for (int k = 0; k < RP; k++) {
        const int rk = min(r0 + k, a.L - 1);
        list[k] = a.lists + (int64_t)rk * a.W;
        const int l = a.lengths[rk];
        len[k] = l < 0 ? 0 : (l > a.W ? a.W : l);
    }

    // Q operand: column r16 = head h*G + r16 % G of row r0 + r16 / G (zero
    // past the live columns), 8 dims per MFMA in the source's layout.
    half8 qop[NM];
    {
        const bool ok = col_ok;
        const f16* qrow =
            a.q + ((int64_t)(h * G + (ok ? chead : 0)) * a.L + r0 + (ok ? crow : 0)) * D;
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const int base = Src::kQ == kQNatural ? 32 * m + 8 * g : (D / 4) * g + 8 * m;
            half8 x = ok ? *(const half8*)(qrow + base) : half8{};
            if constexpr (Src::kQ == kQGroup4) {
                const u32x4 w = __builtin_bit_cast(u32x4, x);
                u32x4 o;  // dims (0,4),(1,5),(2,6),(3,7)
                o.x = __builtin_amdgcn_perm(w.z, w.x, 0x05040100u);
                o.y = __builtin_amdgcn_perm(w.z, w.x, 0x07060302u);
                o.z = __builtin_amdgcn_perm(w.w, w.y, 0x05040100u);
                o.w = __builtin_amdgcn_perm(w.w, w.y, 0x07060302u);
                x = __builtin_bit_cast(half8, o);
            }
            qop[m] = x;
        }
    }

    float mrun = -INFINITY;  // running max (log2 domain), column r16
    float lrun = 0.0f;       // running sum, this lane's share
    float4v acc[NP][4];
#pragma unroll
    for (int pp = 0; pp < NP; pp++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[pp][c] = float4v{0.f, 0.f, 0.f, 0.f};

    // One batch of kDlsaNT tiles; ALIGNED: every lane group's four entries
    // are four consecutive keys from a multiple of 4 (checked wave-wide).
    // The general (unaligned) gathers hold many scattered loads: they take
    // one tile at a time (NT = 1).
    auto batch = [&](auto aligned_tag, auto nt_tag, const int* key_a, const bool* ok_a, int colmask) {
        const bool my_col = RP == 1 ? col_ok : col_ok && ((colmask >> crow) & 1) != 0;
        constexpr bool ALIGNED = decltype(aligned_tag)::value;
        constexpr int NT = decltype(nt_tag)::value;
        typename Src::Regs rg[NT];
#pragma unroll
        for (int b = 0; b < NT; b++) {
            int key4[4];
#pragma unroll
            for (int j = 0; j < 4; j++) key4[j] = __shfl(key_a[b], 4 * g + j);
            src.template load<ALIGNED>(rg[b], h, key_a[b], key4, r16, g);
        }
        // Every gather of a multi-tile batch is issued before the first use:
        // without the barrier the scheduler sinks the V gathers below the QK
        // MFMAs, and the batch waits for them there (c5: 17.9 against 14.6 us
        // a call). The one-tile general gathers are left to the scheduler (their
        // many scattered loads would not fit the registers all at once).
        if constexpr (NT > 1) __builtin_amdgcn_sched_barrier(0);
        // ---- scores: S^T tile, lane holds entries 4g+i for head r16
        float sv[NT][4];
        float bmax = -INFINITY;
#pragma unroll
        for (int b = 0; b < NT; b++) {
            float4v sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int m = 0; m < NM; m++)
                sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(src.template k_op<FAST>(rg[b], m),
                                                              qop[m], sacc, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const bool ok = __shfl(ok_a[b] ? 1 : 0, 4 * g + i) != 0 && my_col;
                sv[b][i] = ok ? sacc[i] * a.scale2 : -INFINITY;
                bmax = fmaxf(bmax, sv[b][i]);
            }
        }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 16));
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
        const float mnew = fmaxf(mrun, bmax);
        const float mref = mnew == -INFINITY ? 0.0f : mnew;
        const float alpha = mrun == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mrun - mref);
        mrun = mnew;
        lrun *= alpha;
        // Rescale the accumulators: row i of a tile is head 4g + i, whose
        // factor lives in column 4g + i.
        {
            float f[4];
#pragma unroll
            for (int i = 0; i < 4; i++) f[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
            for (int pp = 0; pp < NP; pp++)
#pragma unroll
                for (int c = 0; c < 4; c++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[pp][c][i] *= f[i];
        }
#pragma unroll
        for (int b = 0; b < NT; b++) {
            half4v ph, pl;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float pv = __builtin_amdgcn_exp2f(sv[b][i] - mref);
                lrun += pv;
                ph[i] = (f16)pv;
                pl[i] = (f16)(pv - (float)ph[i]);
            }
#pragma unroll
            for (int pp = 0; pp < NP; pp++) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const half4v vb = src.template v_op<ALIGNED, FAST>(rg[b], pp, c);
                    acc[pp][c] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, vb, acc[pp][c], 0, 0, 0);
                    acc[pp][c] = __builtin_amdgcn_mfma_f32_16x16x16f16(pl, vb, acc[pp][c], 0, 0, 0);
                }
            }
        }
    };

    // tiles a batch (the two-row form stages one: its three batch forms would
    // not fit the registers with two)
    constexpr int NTB = RP == 2 ? 1 : Src::kNT;
    const int n_tiles = (e_end - e_begin + 15) / 16;
    for (int t0 = wave; t0 < n_tiles; t0 += 4 * NTB) {
        int key_a[RP][NTB];  // the key of list entry tile*16 + r16 (A-operand row), row k
        bool ok_a[RP][NTB];
#pragma unroll
        for (int k = 0; k < RP; k++)
#pragma unroll
            for (int b = 0; b < NTB; b++) {
                const int tile = t0 + 4 * b;
                const int e = e_begin + 16 * tile + r16;
                int key = -1;
                if (tile < n_tiles && e < e_end) key = list[k][e];
                ok_a[k][b] = e < len[k] && key >= 0 && key < a.T;
                key_a[k][b] = ok_a[k][b] ? key : 0;
            }
        using NTall = std::integral_constant<int, NTB>;
        using NT1 = std::integral_constant<int, 1>;
        // row k's tiles for the columns in colmask (k a compile-time tag: the
        // key arrays stay in registers)
        auto run = [&](auto k_tag, int colmask) {
            constexpr int k = decltype(k_tag)::value;
            if constexpr (Src::kHasAligned) {
                bool aligned = true;
#pragma unroll
                for (int b = 0; b < NTB; b++) {
                    // each lane compares with its group's first entry
                    const int first = __shfl(key_a[k][b], r16 & ~3);
                    aligned = aligned && (first & 3) == 0 && key_a[k][b] == first + (r16 & 3);
                }
                if (__all(aligned)) {
                    batch(std::true_type{}, NTall{}, key_a[k], ok_a[k], colmask);
                } else {
#pragma unroll
                    for (int b = 0; b < NTB; b++)
                        batch(std::false_type{}, NT1{}, key_a[k] + b, ok_a[k] + b, colmask);
                }
            } else {
                batch(std::false_type{}, NTall{}, key_a[k], ok_a[k], colmask);
            }
        };
        using K0 = std::integral_constant<int, 0>;
        using K1 = std::integral_constant<int, RP - 1>;
        if constexpr (RP == 1) {
            run(K0{}, 1);
        } else {
            bool same = true;
#pragma unroll
            for (int b = 0; b < NTB; b++)
                same = same && key_a[0][b] == key_a[1][b] && ok_a[0][b] == ok_a[1][b];
            if (nrow == 1 || __all(same)) {
                run(K0{}, 3);
            } else {
                run(K0{}, 1);
                run(K1{}, 2);
            }
        }
    }
    lrun += __shfl_xor(lrun, 16);
    lrun += __shfl_xor(lrun, 32);

    // ---- merge the 4 waves through LDS: each wave parks its (m, l) and its
    // unscaled accumulators (head 4g + i, dims 64p + 4 r16 .. +3 as one
    // float4, i.e. the dims in order); after one barrier thread t owns dim
    // t % D of every 256 / D-th head, forms the factors e^(m_w - M) itself
    // and writes the merged row, so the partial's stores are spread over all
    // four waves. Up to 32 KB of accumulators a round (8 heads at D = 256):
    // G <= 8 takes one round.
    constexpr int HC = GMAX * D <= 2048 ? GMAX : 2048 / D;
    __shared__ float2 sm_ml[4][16];
    __shared__ float4v sm_acc[4][HC][D / 4];
    if (g == 0) sm_ml[wave][r16] = float2{mrun, lrun};
    const float* accf = (const float*)&sm_acc[0][0][0];
    for (int hc0 = 0; hc0 < NC; hc0 += HC) {
        if (hc0 > 0) __syncthreads();  // the previous round's reads are done
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int hd = 4 * g + i;
            if (hd >= hc0 && hd < hc0 + HC && hd < NC)
#pragma unroll
                for (int pp = 0; pp < NP; pp++)
                    sm_acc[wave][hd - hc0][16 * pp + r16] =
                        float4v{acc[pp][0][i], acc[pp][1][i], acc[pp][2][i], acc[pp][3][i]};
        }
        __syncthreads();
        const int nh = min(HC, NC - hc0);
        for (int o = threadIdx.x; o < nh * D; o += 256) {
            const int hl = o / D, d = o % D, hd = hc0 + hl;
            float M = -INFINITY;
#pragma unroll
            for (int w = 0; w < 4; w++) M = fmaxf(M, sm_ml[w][hd].x);
            float O = 0.0f, Ls = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float2 ml = sm_ml[w][hd];
                const float f = ml.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml.x - M);
                O = __builtin_fmaf(f, accf[(w * HC + hl) * D + d], O);
                Ls = __builtin_fmaf(f, ml.y, Ls);
            }
            const int hr = RP == 1 ? 0 : hd / G;  // the column's row
            const int qh = h * G + hd - hr * G, r = r0 + hr;
            if (a.parts == 1) {
                a.out[((int64_t)qh * a.L + r) * D + d] = (f16)(Ls > 0.0f ? O / Ls : 0.0f);
            } else {
                const int64_t pr = ((int64_t)r * a.hq + qh) * a.parts + part;
                a.part_o[pr * D + d] = O;
                if (d == 0) a.part_ml[pr] = float2{M, Ls};
            }
        }
    }
}


// One kernel per (head dim, heads per group, row source). Affine sources use
// the exact 2-op dequant when every cached scale allows it (the cache's
// fast_flag), else the separately rounded one.
template <int D, int GMAX, class Src, int RP = 1>
__global__ __launch_bounds__(256, 2) void dlsa_kernel(DlsaArgs a, Src src, const int* fast_flag) {
    if constexpr (Src::kAffine) {
        // The exact 2-op dequant runs without waiting for the cache's fast
        // flag; a cache holding a scale outside its exact range takes the
        // separately rounded one in a second pass whose writes (same threads,
        // same elements) replace the first's. A null flag (Int8 caches) takes
        // the separately rounded dequant directly.
        if (fast_flag != nullptr) {
            dlsa_body<D, GMAX, Src, true, RP>(a, src);
            if (*fast_flag == 0) {
                __syncthreads();
                dlsa_body<D, GMAX, Src, false, RP>(a, src);
            }
        } else {
            dlsa_body<D, GMAX, Src, false, RP>(a, src);
        }
    } else {
        dlsa_body<D, GMAX, Src, true, RP>(a, src);
    }
}

// out[qh, r] = sum_p e^(m_p - M) O_p / sum_p e^(m_p - M) l_p (m in the log2 domain).
// grid (q heads, rows, D/64), kDMW waves: lane = dim, wave w sums parts w, w + kDMW, ...
// (at most PER of them) with every load issued before the first use (one
// memory round trip).
constexpr int kDlsaMaxParts = 128;

// Waves of the merge, each summing every kDMW-th part: eight measured c5
// 12.89 -> 12.76 us against four (A/B in one run).
#ifndef QW_DLSA_MERGE_WAVES
#define QW_DLSA_MERGE_WAVES 8
#endif
constexpr int kDMW = QW_DLSA_MERGE_WAVES;

template <int PER>
__global__ __launch_bounds__(64 * kDMW) void dlsa_merge_kernel(const float* __restrict__ part_o,
                                                         const float2* __restrict__ part_ml,
                                                         int parts, int D, int L, int hq,
                                                         f16* __restrict__ out) {
    const int qh = blockIdx.x, r = blockIdx.y, d = blockIdx.z * 64 + (threadIdx.x & 63);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t base = ((int64_t)r * hq + qh) * parts;
    float v[PER];
    float2 ml[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int p = wave + kDMW * i;
        if (p < parts) {
            ml[i] = part_ml[base + p];
            v[i] = part_o[(base + p) * D + d];
        } else {
            ml[i] = float2{-INFINITY, 0.0f};
            v[i] = 0.0f;
        }
    }
    // each wave reduces its parts against its own maximum (log2 units); the
    // four (m, l, O) meet in LDS behind one barrier
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; i++) m = fmaxf(m, ml[i].x);
    float o = 0.0f, l = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const float f = ml[i].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml[i].x - m);
        o = __builtin_fmaf(f, v[i], o);
        l = __builtin_fmaf(f, ml[i].y, l);
    }
    __shared__ float2 sm_ml[kDMW];
    __shared__ float sm_o[kDMW][64];
    if (lane == 0) sm_ml[wave] = float2{m, l};
    sm_o[wave][lane] = o;
    __syncthreads();
    if (wave == 0) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kDMW; w++) M = fmaxf(M, sm_ml[w].x);
        float O = 0.0f, Ls = 0.0f;
#pragma unroll
        for (int w = 0; w < kDMW; w++) {
            const float2 gl = sm_ml[w];
            const float f = gl.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(gl.x - M);
            O = __builtin_fmaf(f, sm_o[w][lane], O);
            Ls = __builtin_fmaf(f, gl.y, Ls);
        }
        out[((int64_t)qh * L + r) * D + d] = (f16)(Ls > 0.0f ? O / Ls : 0.0f);
    }
}

// Split-K workspace of the D-LSA calls, one per (device, stream): calls on
// different streams never share partials. Each is a GrowBuffer, so growth
// never frees memory a captured graph may still read.
static std::mutex g_ws_mu;
static std::map<std::pair<int, hipStream_t>, GrowBuffer> g_ws;

static int dlsa_workspace(int device, hipStream_t stream, size_t need, void** out) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    GrowBuffer& b = g_ws[{device, stream}];
    b.stream_owned = true;  // only calls on `stream` use it
    return b.get(need, stream, out);
}

// Launch policy (the reference's auto_parts, mlx_cxx_dlsa_attention.cpp:379-400,
// re-derived for 256 CUs): one pass when rows x kv_heads alone reach 192
// workgroups, else split each list so that about 192 workgroups run (3/4 of
// the CUs still saturate HBM with these gathers, and fewer parts make the
// merge cheaper; measured for one row, 4 KV heads, 4612 entries: 40-48 parts
// 13.0 us, 56 parts 13.2 us, 64 parts 13.4 us, 72 parts 15.5 us), keeping at
// least 16 entries (one tile) a part and at most 128 parts.
static int auto_parts(int units, int width) {
    constexpr int kTargetWorkgroups = 192;
    if (units >= kTargetWorkgroups) return 1;
    int parts = (kTargetWorkgroups + units - 1) / units;
    parts = std::min(parts, std::max(1, width / 16));
    return std::max(1, std::min(parts, 128));
}

// What a read gathers from: fp16 K/V views with strides (cache == nullptr),
// or a KV cache's own storage.
struct DlsaSource {
    const KVCache* cache = nullptr;
    const void* k = nullptr;
    const void* v = nullptr;
    int64_t khs = 0, krs = 0, vhs = 0, vrs = 0;
};

constexpr int kPairMinWorkgroups = 192;

template <int D, int GM, class Src>
static void launch_dlsa_kernel(const Src& src, const DlsaArgs& a, dim3 grid, const int* fast,
                               hipStream_t stream) {
    // one-pass calls with rows to spare: two rows a workgroup (the grid keeps
    // at least kPairMinWorkgroups workgroups)
    if constexpr (Src::kPairs) {
        if (a.parts == 1 && 2 * a.G <= 16 && (int64_t)a.L * a.hkv >= 2 * kPairMinWorkgroups) {
            hipLaunchKernelGGL((dlsa_kernel<D, GM, Src, 2>), dim3(grid.x, (a.L + 1) / 2, grid.z),
                               dim3(256), 0, stream, a, src, fast);
            return;
        }
    }
    hipLaunchKernelGGL((dlsa_kernel<D, GM, Src>), grid, dim3(256), 0, stream, a, src, fast);
}

template <int D, int GM>
static void launch_dlsa_source(const DlsaSource& s, const DlsaArgs& a, dim3 grid,
                               hipStream_t stream) {
    if (!s.cache) {
        const SrcStrided<D> src{(const f16*)s.k, (const f16*)s.v, s.khs, s.krs, s.vhs, s.vrs};
        launch_dlsa_kernel<D, GM>(src, a, grid, nullptr, stream);
        return;
    }
    const KVCache& c = *s.cache;
    if (c.mode == QW_KV_FP16) {
        const SrcCacheF16<D> src{(const f16*)c.k_data, (const f16*)c.v_data, c.cap};
        launch_dlsa_kernel<D, GM>(src, a, grid, nullptr, stream);
        return;
    }
    if constexpr (D == 128 || D == 256) {
        if (c.bits == 4) {
            const SrcCacheAffine<D, 4> src{(const uint32_t*)c.k_data, c.k_params,
                                           (const uint32_t*)c.v_data, (const f16*)c.v_params,
                                           c.cap, c.code_offset2()};
            launch_dlsa_kernel<D, GM>(src, a, grid, c.int8() ? nullptr : c.fast_flag, stream);
        } else {
            const SrcCacheAffine<D, 8> src{(const uint32_t*)c.k_data, c.k_params,
                                           (const uint32_t*)c.v_data, (const f16*)c.v_params,
                                           c.cap, c.code_offset2()};
            launch_dlsa_kernel<D, GM>(src, a, grid, c.int8() ? nullptr : c.fast_flag, stream);
        }
    }
}

// scratch == nullptr: the split-K partials go to the stream's workspace
// (allocated or grown on demand); else to `scratch` (scratch_bytes), and an
// automatic part count is lowered until the partials fit it.
static int dlsa_sparse_attention_impl(const void* q, const DlsaSource& src,
                                      const int32_t* lists, const int32_t* lengths, int n_rows,
                                      int width, int n_q_heads, int n_kv_heads, int head_dim,
                                      int n_keys, float scale, int parts, int waves, void* out,
                                      hipStream_t stream, void* scratch, size_t scratch_bytes) {
    QW_REQUIRE(q && lists && lengths && out && (src.cache || (src.k && src.v)),
               QW_ERR_INVALID_ARGUMENT, "dlsa_sparse_attention: null pointer");
    QW_REQUIRE(n_kv_heads > 0 && n_q_heads > 0 && n_q_heads % n_kv_heads == 0 && n_keys > 0 &&
                   n_rows > 0,
               QW_ERR_INVALID_ARGUMENT, "dlsa_sparse_attention: bad head or length geometry");
    const int G = n_q_heads / n_kv_heads;
    QW_REQUIRE(G <= 16, QW_ERR_INVALID_ARGUMENT,
               "dlsa_sparse_attention: at most 16 query heads per KV head");
    QW_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256, QW_ERR_INVALID_ARGUMENT,
               "dlsa_sparse_attention: head dim must be 64, 128 or 256");
    QW_REQUIRE(width > 0, QW_ERR_INVALID_ARGUMENT, "dlsa_sparse_attention: empty list width");
    QW_REQUIRE(parts >= 0 && waves >= 0 && waves <= 16, QW_ERR_INVALID_ARGUMENT,
               "dlsa_sparse_attention: bad launch knobs");
    QW_REQUIRE(((uintptr_t)q % 16) == 0, QW_ERR_UNSUPPORTED,
               "dlsa_sparse_attention: q must be 16-byte aligned");
    if (!src.cache) {
        // 16-byte row loads: row starts and strides must keep 8-element alignment.
        QW_REQUIRE(((uintptr_t)src.k % 16) == 0 && ((uintptr_t)src.v % 16) == 0 &&
                       src.khs % 8 == 0 && src.krs % 8 == 0 && src.vhs % 8 == 0 &&
                       src.vrs % 8 == 0,
                   QW_ERR_UNSUPPORTED,
                   "dlsa_sparse_attention: K/V/q must be 16-byte aligned with strides % 8 == 0");
    }
    int dev = 0;
    QW_HIP_CHECK(hipGetDevice(&dev));
    // bytes of one part's partials: an fp32 output row and an (m, l) pair per (row, q head)
    const size_t part_bytes = (size_t)n_rows * n_q_heads * (head_dim * sizeof(float) + sizeof(float2));
    if (parts <= 0) {
        parts = auto_parts(n_rows * n_kv_heads, width);
        if (scratch) parts = (int)std::min<size_t>((size_t)parts, scratch_bytes / part_bytes);
    }
    parts = std::max(1, std::min(parts, kDlsaMaxParts));
    QW_REQUIRE(!scratch || parts == 1 || (size_t)parts * part_bytes <= scratch_bytes,
               QW_ERR_INVALID_ARGUMENT,
               "dlsa_sparse_attention_noalloc: the partials of " + std::to_string(parts) +
                   " parts need " + std::to_string((size_t)parts * part_bytes) +
                   " bytes, more than the " + std::to_string(scratch_bytes) +
                   "-byte scratch (use fewer parts or rows)");
    DlsaArgs a;
    a.q = (const f16*)q;
    a.lists = lists;
    a.lengths = lengths;
    a.out = (f16*)out;
    a.part_o = nullptr;
    a.part_ml = nullptr;
    a.L = n_rows;
    a.W = width;
    a.hq = n_q_heads;
    a.hkv = n_kv_heads;
    a.G = G;
    a.T = n_keys;
    a.parts = parts;
    a.scale2 = scale * kLog2e;
    if (parts > 1) {
        const size_t no = (size_t)n_rows * n_q_heads * parts;
        void* ws = scratch;
        if (!ws) {
            int rc = dlsa_workspace(dev, stream, no * head_dim * sizeof(float) + no * sizeof(float2),
                                    &ws);
            if (rc) return rc;
        }
        a.part_o = (float*)ws;
        a.part_ml = (float2*)((char*)ws + no * head_dim * sizeof(float));
    }
    const dim3 grid(parts, n_rows, n_kv_heads);
    if (head_dim == 256) {
        if (G <= 8) launch_dlsa_source<256, 8>(src, a, grid, stream);
        else launch_dlsa_source<256, 16>(src, a, grid, stream);
    } else if (head_dim == 128) {
        if (G <= 8) launch_dlsa_source<128, 8>(src, a, grid, stream);
        else launch_dlsa_source<128, 16>(src, a, grid, stream);
    } else {
        if (G <= 8) launch_dlsa_source<64, 8>(src, a, grid, stream);
        else launch_dlsa_source<64, 16>(src, a, grid, stream);
    }
    QW_HIP_CHECK(hipGetLastError());
    if (parts > 1) {
        // parts a wave sums, rounded up to a power of two (parts <= kDlsaMaxParts)
        const dim3 mg(n_q_heads, n_rows, head_dim / 64);
        auto merge = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, mg, dim3(64 * kDMW), 0, stream, a.part_o, a.part_ml, parts, head_dim,
                               n_rows, n_q_heads, (f16*)out);
        };
        const int per = (parts + kDMW - 1) / kDMW;
        if (per <= 4)
            merge(dlsa_merge_kernel<4>);
        else if (per <= 8)
            merge(dlsa_merge_kernel<8>);
        else if (per <= 16)
            merge(dlsa_merge_kernel<16>);
        else
            merge(dlsa_merge_kernel<kDlsaMaxParts / 4>);
        QW_HIP_CHECK(hipGetLastError());
    }
    (void)waves;  // one 4-wave workgroup shape; the knob is accepted for API parity
    return QW_OK;
}

static DlsaSource strided(const void* k, const void* v, int64_t khs, int64_t krs, int64_t vhs,
                          int64_t vrs) {
    DlsaSource s;
    s.k = k;
    s.v = v;
    s.khs = khs;
    s.krs = krs;
    s.vhs = vhs;
    s.vrs = vrs;
    return s;
}

int dlsa_sparse_attention(const void* q, const void* k, const void* v, int64_t khs, int64_t krs,
                          int64_t vhs, int64_t vrs, const int32_t* lists, const int32_t* lengths,
                          int n_rows, int width, int n_q_heads, int n_kv_heads, int head_dim,
                          int n_keys, float scale, int parts, int waves, void* out,
                          hipStream_t stream) {
    return dlsa_sparse_attention_impl(q, strided(k, v, khs, krs, vhs, vrs), lists, lengths, n_rows,
                                      width, n_q_heads, n_kv_heads, head_dim, n_keys, scale, parts,
                                      waves, out, stream, nullptr, 0);
}

// The read over a KV cache (the qwen3_next/dlsa.rs:161-177 pair
// update_and_fetch + sparse_attention, with the fetch gone): keys are the
// cache's first `offset` rows. fp16 and affine / Int8 caches are read in
// place (quantized rows dequantized inside the gather as the fetch would);
// Turbo4 rows have no in-place form (a rotated codebook basis), so they are
// fetched to fp16 first, as the reference's update_and_fetch does, into a
// buffer the cache keeps.
int KVCache::dlsa_attention(const void* q, int n_q_heads, int n_rows, const int32_t* lists,
                            const int32_t* lengths, int width, float scale, void* out,
                            hipStream_t stream) {
    QW_REQUIRE(offset > 0, QW_ERR_INVALID_ARGUMENT, "dlsa_attention: the cache is empty");
    DeviceGuard dg(device);
    QW_REQUIRE(dg.ok, QW_ERR_HIP, "dlsa_attention: hipSetDevice failed");
    if (turbo4()) {
        const size_t plane = (size_t)hkv * offset * D * sizeof(f16);
        void* buf = nullptr;
        int rc = fetch_ws.get(2 * plane, stream, &buf);
        if (rc) return rc;
        rc = dequantize(0, offset, buf, (char*)buf + plane, stream);
        if (rc) return rc;
        return dlsa_sparse_attention_impl(
            q, strided(buf, (char*)buf + plane, (int64_t)offset * D, D, (int64_t)offset * D, D),
            lists, lengths, n_rows, width, n_q_heads, hkv, D, offset, scale, 0, 0, out, stream,
            nullptr, 0);
    }
    DlsaSource s;
    s.cache = this;
    return dlsa_sparse_attention_impl(q, s, lists, lengths, n_rows, width, n_q_heads, hkv, D,
                                      offset, scale, 0, 0, out, stream, nullptr, 0);
}

int KVCache::update_and_dlsa_attention(const void* q, int n_q_heads, int n_rows,
                                       const void* k_new, const void* v_new, const int32_t* lists,
                                       const int32_t* lengths, int width, float scale, void* out,
                                       hipStream_t stream) {
    int rc = update(k_new, v_new, n_rows, stream);
    if (rc) return rc;
    return dlsa_attention(q, n_q_heads, n_rows, lists, lengths, width, scale, out, stream);
}

// ------------------------------------------------ the no-allocation variant
//
// Split-K partials of qw_dlsa_sparse_attention_noalloc, in a fixed device
// array the library never allocates: each device that loads the library holds
// its own copy until the process ends. In host code `scratch` only names the
// symbol; its device address comes from hipGetSymbolAddress, resolved once
// per device with that device current and kept in g_scratch_ptr. Every call
// on a device shares the array (nothing in it must start at zero: each
// partial is written before it is read), so two calls that overlap on one
// device race.
constexpr size_t kDlsaScratchBytes = (size_t)4 << 20;
static __device__ __align__(256) unsigned char scratch[kDlsaScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];

static int scratch_address(int device, void** out) {
    QW_REQUIRE(device >= 0 && device < 64, QW_ERR_INVALID_ARGUMENT,
               "dlsa_sparse_attention_noalloc: device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void* p = nullptr;
        QW_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        QW_REQUIRE(p != nullptr, QW_ERR_HIP, "dlsa_sparse_attention_noalloc: no scratch address");
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return QW_OK;
}

int dlsa_sparse_attention_noalloc(const void* q, const void* k, const void* v, int64_t khs,
                                  int64_t krs, int64_t vhs, int64_t vrs, const int32_t* lists,
                                  const int32_t* lengths, int n_rows, int width, int n_q_heads,
                                  int n_kv_heads, int head_dim, int n_keys, float scale, int parts,
                                  int waves, void* out, hipStream_t stream) {
    int dev = 0;
    QW_HIP_CHECK(hipGetDevice(&dev));
    void* ws = nullptr;
    int rc = scratch_address(dev, &ws);
    if (rc) return rc;
    return dlsa_sparse_attention_impl(q, strided(k, v, khs, krs, vhs, vrs), lists, lengths, n_rows,
                                      width, n_q_heads, n_kv_heads, head_dim, n_keys, scale, parts,
                                      waves, out, stream, ws, kDlsaScratchBytes);
}

}  // namespace qw
