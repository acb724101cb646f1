// kv_cache.hpp - host-side KV cache object behind the C ABI.
//
// qw::KVCache mirrors the reference's KVCache (crates/mlxcel-core/src/cache.rs:354)
// for one full-attention layer: the same method names (update,
// update_and_fetch, trim, offset, nbytes, snapshot export/import) and the
// same argument meaning, on caller-owned device pointers instead of MLX
// arrays, returning status codes instead of panicking.
#pragma once

#include "qw_common.hpp"
#include "turbo4_codec.hpp"

namespace qw {

// Where an append reads its new rows: row (h, i) of K at k + i * row_stride +
// h * head_stride (V alike), and the RoPE applied to K as it is read
// (rope_dims == 0: none). A plain update reads [hkv][n][D]; the fused
// RoPE-append reads K and V straight out of the fused QKV projection.
struct RowSrc {
    const f16* k;
    const f16* v;
    int64_t row_stride, head_stride;
    int rope_dims;      // rotated prefix of each head (even), 0: no rotation
    int traditional;    // 1: pairs (2p, 2p+1); 0: pairs (p, p + rope_dims/2)
    int position0;      // position of row 0
    float log2_base;    // log2(rope base), formed on the host as MLX does
    float scale;        // rope scale
};

struct KVCache {
    int mode = QW_KV_FP16;  // QW_KV_*
    int bits = 16;          // 4 (affine4, turbo4), 8 (affine8, int8) or 16 (fp16)
    int D = 0;              // head_dim
    int hkv = 0;            // KV heads
    int device = 0;
    int offset = 0;         // cached tokens (cache.rs `offset`)
    int cap = 0;            // allocated rows per head, multiple of 256

    // K plane: affine codes [hkv][cap][D*bits/32] u32 or fp16 [hkv][cap][D];
    // Turbo4: packed indices [hkv][cap][D/2] bytes (low nibble even coord).
    void* k_data = nullptr;
    // K params: [hkv][cap][D/64] half2(scale, bias) (affine);
    // Turbo4: [hkv][cap] half2(k_rescale, 0).
    uint32_t* k_params = nullptr;
    // V plane: affine 8-key blocks [hkv][cap/8][D*bits/4 bytes] or fp16
    // 8-key blocks [hkv][cap/8][D][8] f16 (same transposition, 16 bytes a dim);
    // Turbo4: packed indices [hkv][cap][D/2] bytes, row-major like K.
    void* v_data = nullptr;
    // V params: [hkv][cap/8][D/64][16] f16 (s0..s7, b0..b7) (affine);
    // Turbo4: [hkv][cap] half2(v_norm, v_rescale).
    uint32_t* v_params = nullptr;

    // Turbo4 codec tables on the device (float): V signs1, V signs2, K signs1,
    // K signs2 (D each), then 16 centroids and 15 boundaries.
    uint32_t turbo_seed = turbo4::kDefaultSeed;
    float* t4_tables = nullptr;

    // 1 while every stored scale is inside the exact 2-op dequant range of the
    // fused kernels (dequant.hpp); cleared by an append or import that stores
    // one outside it. Device int, read by each attention launch.
    int* fast_flag = nullptr;

    // Split-K workspace (partial accumulators), grown on demand; ws_ptr is
    // the current buffer (valid after ensure_workspace).
    GrowBuffer ws;
    void* ws_ptr = nullptr;
    // fp16 rows of a Turbo4 cache fetched for the D-LSA read (dlsa.hip)
    GrowBuffer fetch_ws;

    KvLayout layout() const { return KvLayout{bits, D, hkv, cap}; }
    // Codes and per-group (scale, bias) in the affine layout: the affine modes
    // and Int8 (stored as 8-bit codes biased by 128, the token's scale in
    // every group, bias 0).
    bool affine() const {
        return mode == QW_KV_AFFINE8 || mode == QW_KV_AFFINE4 || mode == QW_KV_INT8;
    }
    bool int8() const { return mode == QW_KV_INT8; }
    bool turbo4() const { return mode == QW_KV_TURBO4; }
    // Offset the 8-bit magic-number conversion subtracts to recover a code
    // (fp16 1024 + stored byte): 1024 for unsigned affine codes, 1152 for
    // Int8 codes stored biased by 128.
    uint32_t code_offset2() const { return int8() ? 0x64806480u : 0x64006400u; }

    size_t k_data_bytes(int c) const;
    size_t k_param_bytes(int c) const;
    size_t v_data_bytes(int c) const;
    size_t v_param_bytes(int c) const;

    int init(int mode, int group_size, int n_kv_heads, int head_dim, int capacity, int device);
    // Builds the Turbo4 tables for turbo_seed and D (turbo4.hip).
    int turbo4_setup();
    int release();
    int reserve(int capacity, hipStream_t stream);
    int ensure_workspace(size_t bytes, hipStream_t stream);
    int64_t nbytes() const;
    // cache.rs:3591 demote_fp16_to_turbo4, to an affine mode
    int demote(int target_mode, hipStream_t stream, int* demoted);

    // cache.rs:922 `update`
    int update(const void* k_new, const void* v_new, int n_tokens, hipStream_t stream);
    // Append from a row source (strided rows, optional RoPE on K).
    int update_rows(const RowSrc& src, int n_tokens, hipStream_t stream);
    // fused_rope_append.cpp:80-180 + update: q/k RoPE out of the fused QKV
    // projection, rotated q to q_out, rotated k and v appended.
    int rope_update(const void* qkv, int n_q_heads, int n_tokens, int rope_dims, int traditional,
                    float rope_base, float rope_scale, int position0, void* q_out,
                    hipStream_t stream);
    // fused_rope_append.cpp:80-180 then cache.rs:3495 `update_and_turbo4_attention`
    // on its outputs: rope_update, then attention of q_out over the cache;
    // one decode launch (plus the merge) for decode-route shapes.
    int rope_update_and_attention(const void* qkv, int n_q_heads, int n_tokens, int rope_dims,
                                  int traditional, float rope_base, float rope_scale, int position0,
                                  float scale, bool causal, void* q_out, void* out,
                                  hipStream_t stream);
    // cache.rs:2709 `update_and_fetch`
    int update_and_fetch(const void* k_new, const void* v_new, int n_tokens, void* k_out,
                         void* v_out, hipStream_t stream);
    int dequantize(int start, int n, void* k_out, void* v_out, hipStream_t stream) const;
    // cache.rs:3495 / :3520 `update_and_turbo4_(causal_)attention`, affine codec
    int update_and_attention(const void* q, int n_q_heads, int n_rows, const void* k_new,
                             const void* v_new, float scale, bool causal, void* out,
                             hipStream_t stream);
    // cache.rs:3607 fused prefix attention, no append
    int attention(const void* q, int n_q_heads, int n_rows, float scale, bool causal, void* out,
                  hipStream_t stream);
    // D-LSA K2 over the cache's rows (qwen3_next/dlsa.rs:161-177:
    // update_and_fetch, then dlsa_attention::sparse_attention), dlsa.hip
    int dlsa_attention(const void* q, int n_q_heads, int n_rows, const int32_t* lists,
                       const int32_t* lengths, int width, float scale, void* out,
                       hipStream_t stream);
    int update_and_dlsa_attention(const void* q, int n_q_heads, int n_rows, const void* k_new,
                                  const void* v_new, const int32_t* lists, const int32_t* lengths,
                                  int width, float scale, void* out, hipStream_t stream);
    // cache.rs:2251 `trim`
    int trim(int n);
    // cache.rs:570-626 snapshot tensors
    int export_tensors(void* k_codes, void* k_scales, void* k_biases, void* v_codes,
                       void* v_scales, void* v_biases, hipStream_t stream) const;
    int import_tensors(int n_tokens, const void* k_codes, const void* k_scales,
                       const void* k_biases, const void* v_codes, const void* v_scales,
                       const void* v_biases, hipStream_t stream);

    // Turbo4 parts (turbo4.hip): quantize-on-append, fetch, snapshot tensors
    // (cache.rs:570-626 turbo4_snapshot_tensors / restore_turbo4_snapshot).
    int turbo4_update(const RowSrc& src, int n_tokens, hipStream_t stream);
    int turbo4_dequantize(int start, int n, void* k_out, void* v_out, hipStream_t stream) const;
    int turbo4_export(void* k_packed, void* k_rescale, void* v_packed, void* v_norms,
                      void* v_rescale, hipStream_t stream) const;
    int turbo4_import(int n_tokens, const void* k_packed, const void* k_rescale,
                      const void* v_packed, const void* v_norms, const void* v_rescale,
                      hipStream_t stream);
};

// RAII guard that makes `device` current for the duration of a call.
struct DeviceGuard {
    int prev = -1;
    bool ok = true;
    explicit DeviceGuard(int device) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != device) ok = hipSetDevice(device) == hipSuccess;
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

// Turbo4 attention (turbo4.hip): q rotated into the K basis, attention in the
// rotated basis, the output rotated back. Causal blocks of 1-5 rows past 2048
// tokens with at most 32 query heads a KV head take the fused verify pass (in
// the block kernel); other calls of up to 16 rows a KV head the decode kernel
// reads from the packed indices in place, up to 1024 the block kernel, and
// from block_image_min_rows(true) on the block kernel's tile images; the rest
// expand the rotated K/V to fp16 for the fp16 kernels.
int turbo4_attention(KVCache& c, const void* q, int n_q_heads, int n_rows, float scale,
                     bool causal, void* out, hipStream_t stream);

// Kernel launchers (attend_decode.hip, attend_block.hip).
int launch_attention(KVCache& c, const void* q, int n_q_heads, int n_rows, float scale,
                     bool causal, void* out, hipStream_t stream);
// Turbo4 caches, G * n_rows <= 16: the decode kernel rotates q into the K
// basis, reads the packed indices in place and forms f16(centroid * rescale)
// as the fp16 expansion holds it; the merge rotates the output back. tab: the
// cache's device tables.
int launch_turbo4_decode(KVCache& c, const f16* q, int G, int n_rows, float scale, bool causal,
                         const float* tab, f16* out, hipStream_t stream);
// Turbo4 caches through the block kernel, which rotates q into the K basis
// itself and reads the packed cache in place. fused = false keeps the fp16
// SDPA arithmetic on the expansion's values and writes the rotated-basis rows
// (fp16) to out; fused = true is the reference's fused verify pass (q scaled
// by scale * log2 e, fp32 scores; every row key-split) and its merge writes
// the rows rotated back to out. tab: the cache's device tables.
// A causal sliding window (window > 0: each row's keys p - window + 1 .. p)
// and/or a logit softcap over an affine, Int8 or fp16 cache (D 128 / 256):
// the block kernel reading the codes.
int launch_block_attention_ext(KVCache& c, const f16* q, int G, int n_rows, float scale,
                               bool causal, int window, float softcap, f16* out,
                               hipStream_t stream);
int launch_block_attention_t4(KVCache& c, const f16* q, int G, int n_rows, float scale, bool causal,
                              bool fused, const float* tab, f16* out, hipStream_t stream);
// Turbo4 merge of split partials ([hkv][nc][rstride][D], slot_bits as
// launch_partial_merge): each row merged, rounded to fp16 (keep32: kept fp32),
// rotated back through the V basis and written to out.
int launch_t4_merge_rotate(const float* part_o, const float2* part_ml, int nc, int rstride, int R,
                           int hkv, int D, int G, int Tq, int slot_bits, bool keep32,
                           const float* tab, f16* out, hipStream_t stream);
// G * n_rows > 16 query rows per KV head (verify blocks, prefill chunks).
int launch_block_attention(KVCache& c, const f16* q, int G, int n_rows, float scale, bool causal,
                           f16* out, hipStream_t stream);
// A verify block on an affine or Int8 cache whose append runs inside the block
// kernel's launch: appends n_rows new rows ([hkv][n_rows][D]) and attends q
// over the cache including them, as update + launch_block_attention would.
// block_append_fits: the shapes it takes; the caller reserves the capacity.
bool block_append_fits(const KVCache& c, int G, int n_rows);
// Query rows a KV head from which block attention on an affine or Int8
// (turbo4: a Turbo4) cache expands the key tiles once into LDS images.
int block_image_min_rows(bool turbo4);
// The shapes the Turbo4 form below takes (one query tile, at least 256 cached
// rows; the caller reserves the capacity).
bool block_append_fits_t4(const KVCache& c, int G, int n_rows);

// The D-LSA reads (dlsa.hip, dlsa_typed.hip).
int dlsa_sparse_attention(const void* q, const void* k, const void* v, int64_t k_head_stride,
                          int64_t k_row_stride, int64_t v_head_stride, int64_t v_row_stride,
                          const int32_t* lists, const int32_t* lengths, int n_rows, int width,
                          int n_q_heads, int n_kv_heads, int head_dim, int n_keys, float scale,
                          int parts, int waves, void* out, hipStream_t stream);
int dlsa_sparse_attention_noalloc(const void* q, const void* k, const void* v,
                                  int64_t k_head_stride, int64_t k_row_stride,
                                  int64_t v_head_stride, int64_t v_row_stride,
                                  const int32_t* lists, const int32_t* lengths, int n_rows,
                                  int width, int n_q_heads, int n_kv_heads, int head_dim,
                                  int n_keys, float scale, int parts, int waves, void* out,
                                  hipStream_t stream);
int dlsa_sparse_attention_typed(const void* q, int q_dtype, const void* k, const void* v,
                                int kv_dtype, int64_t k_head_stride, int64_t k_row_stride,
                                int64_t v_head_stride, int64_t v_row_stride,
                                const int32_t* lists, const int32_t* lengths, int n_rows,
                                int width, int n_q_heads, int n_kv_heads, int head_dim,
                                int n_keys, float scale, int parts, int waves, void* out,
                                hipStream_t stream);
// The same for a Turbo4 cache (one query tile, at least 256 cached rows,
// capacity reserved): fused as launch_block_attention_t4's fused pass (out:
// the rows rotated back), else its fp16 arithmetic (out: rotated-basis rows).
int launch_block_append_attention_t4(KVCache& c, const f16* q, int G, int n_rows, const f16* k_new,
                                     const f16* v_new, float scale, bool causal, bool fused,
                                     const float* tab, f16* out, hipStream_t stream,
                                     const RowSrc* rope = nullptr, f16* q_out = nullptr);
// A Turbo4 decode-route call (G * n_rows <= 16, at least one cached row,
// capacity reserved) that appends its n_rows rows in the decode launch (its
// append unit) and attends them with the cached prefix; out as
// launch_turbo4_decode.
int launch_turbo4_decode_append(KVCache& c, const f16* q, int G, int n_rows, const f16* k_new,
                                const f16* v_new, float scale, bool causal, const float* tab,
                                f16* out, hipStream_t stream);
// Whether a Turbo4 update-and-attention of n_rows rows takes the decode route
// (the append unit in the decode launch).
bool turbo4_decode_route(const KVCache& c, bool causal, int n_rows, int G);
// Whether it takes the fused verify pass with the rows appended in its launch.
bool turbo4_fused_append_route(const KVCache& c, bool causal, int n_rows, int G);
// Turbo4 update-and-attention: the append in the block kernel's launch where
// the call takes the block kernel, else turbo4_update then turbo4_attention.
int turbo4_update_and_attention(KVCache& c, const void* q, int n_q_heads, int n_rows,
                                const void* k_new, const void* v_new, float scale, bool causal,
                                void* out, hipStream_t stream);
// rope (a RoPE launch): q is the projection and k_new / v_new point into it
// through *rope; the rotated q rows go to q_out.
int launch_block_append_attention(KVCache& c, const f16* q, int G, int n_rows, const f16* k_new,
                                  const f16* v_new, float scale, bool causal, f16* out,
                                  hipStream_t stream, const RowSrc* rope = nullptr,
                                  f16* q_out = nullptr);
// Split-K merge: out[row0 + row] = sum_c e^(m_c - M) O_c / sum_c e^(m_c - M) l_c
// over nc partials of [rstride][D] fp32 rows per KV head, rows 0 .. R-1.
// slot_bits == 0: partial rows in dim order; 4/8/16: in the V plane's slot
// order of that layout (dim d at v_phys_dim(d, D, slot_bits)). out32 != null:
// the merged rows are written there in fp32 (same indexing) instead of to out.
int launch_partial_merge(const float* part_o, const float2* part_ml, int nc, int rstride, int row0,
                         int R, int hkv, int D, int G, int Tq, f16* out, hipStream_t stream,
                         int slot_bits = 0, float* out32 = nullptr);
// Attention with the reference's general options (sdpa_general.hip):
// layers::attention's mask and softcap and causal_attention's sliding window.
struct SdpaOptions {
    bool causal = false;
    int window = 0;           // > 0 (with causal): keys p - window + 1 .. p
    float softcap = 0.0f;     // > 0: tanh(s / softcap) * softcap on the scores
    const void* mask = nullptr;  // [hq or broadcast][n_rows][n_keys], key stride 1
    int mask_dtype = 0;       // QW_MASK_BOOL or QW_DTYPE_F16 / BF16 / F32 (additive)
    int64_t mask_head_stride = 0, mask_row_stride = 0;  // elements; head stride 0 broadcasts
};
// Over fp16 K/V rows [hkv][n_keys][D] with element strides; q and out
// [hq][n_rows][D] fp16.
int sdpa_general(const void* q, int n_q_heads, int n_rows, const void* k, const void* v,
                 int n_kv_heads, int n_keys, int head_dim, int64_t khs, int64_t krs, int64_t vhs,
                 int64_t vrs, float scale, const SdpaOptions& o, void* out, hipStream_t stream);
// The first key any of n_rows causal windowed rows over T keys sees (0 without
// a window), rounded down to a multiple of align; and the options of a call on
// keys lo .. n_keys - 1 only (the mask's columns shifted by lo).
int window_first_key(const SdpaOptions& o, int T, int n_rows, int align = 1);
SdpaOptions shift_keys(const SdpaOptions& o, int lo);
// Over a cache: without mask, softcap or window the cache's own fused
// attention; else its rows dequantized (Turbo4: expanded in the rotated basis,
// q rotated in and the output rotated back) and sdpa_general.
int cache_attention_general(KVCache& c, const void* q, int n_q_heads, int n_rows, float scale,
                            const SdpaOptions& o, void* out, hipStream_t stream);
int turbo4_attention_general(KVCache& c, const void* q, int n_q_heads, int n_rows, float scale,
                             const SdpaOptions& opts, void* out, hipStream_t stream);

// The same merge over the block kernel's fp16 partials: each partial row is
// O_c / l_c rounded to fp16, place NT * r + mm holding slot 16 mm + r
// (NT = D / 16), with (m_c, l_c) in part_ml; out[row0 + row] =
// sum_c e^(m_c - M) l_c O_c / sum_c e^(m_c - M) l_c.
int launch_partial_merge_h(const f16* part_o, const float2* part_ml, int nc, int rstride, int row0,
                           int R, int hkv, int D, int G, int Tq, f16* out, hipStream_t stream,
                           int slot_bits);


// D-LSA K1 select (dlsa_select.hip).
int dlsa_select(const float* scores, int64_t stride, const int32_t* members, int n_member_rows,
                int bucket_cap, const int32_t* positions, int n_rows, int total_rows, int window,
                int sink, int top_k, int top_p, int buckets_per_block, int threads,
                int32_t* lists, int32_t* lengths, int32_t* picked, int32_t* status,
                hipStream_t stream);

// Fused q/k RoPE + append-layout relayout (rope.hip).
int fused_rope_qk_append(const void* qkv, int batch, int seq, int hq, int hkv, int head_dim,
                         int rope_dims, float rope_base, float rope_scale, int traditional,
                         int positions_base, int dest_layout, void* q_out, void* k_out,
                         void* v_out, hipStream_t stream);

}  // namespace qw
