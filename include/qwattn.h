/*
 * qwattn.h - C ABI of the MI355X (gfx950) full-attention hot path.
 *
 * The ABI is what the reference's Rust runtime would bind in place of its
 * MLX-backed KV cache and attention calls (crates/mlxcel-core). Every entry
 * point names the reference interface it replaces (path:line in the
 * reference tree cr0sh/qw).
 *
 * Conventions
 *   - Plain C: opaque handles, caller-owned device pointers, int status.
 *   - Device pointers live on the device the cache (or call) runs on; the
 *     library sets that device for the duration of a call.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream).
 *     All device work of a call is enqueued on it; no call synchronizes the
 *     stream except where stated.
 *   - Tensors use the reference's layouts with the batch dimension of 1
 *     dropped: q [n_q_heads][n_rows][head_dim], new K/V
 *     [n_kv_heads][n_tokens][head_dim], attention output like q. Element
 *     type is IEEE fp16 unless stated.
 *   - Errors: a non-zero status and a message from qw_last_error() (thread
 *     local). Invalid shapes return QW_ERR_INVALID_ARGUMENT and enqueue
 *     nothing. No C++ exception crosses the ABI. The reference instead
 *     panics (cache.rs:3503-3507) or throws std::invalid_argument
 *     (mlx_cxx_dlsa_attention.cpp:429-470); the status codes carry the
 *     same checks.
 *   - Threading: a cache handle is used by one thread at a time, as the
 *     reference's KVCache is !Send/!Sync (cache.rs:483-497).
 */
#ifndef QWATTN_H
#define QWATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QWATTN_ABI_VERSION 1

/* Status codes. */
#define QW_OK 0
#define QW_ERR_INVALID_ARGUMENT 1
#define QW_ERR_UNSUPPORTED 2
#define QW_ERR_OUT_OF_MEMORY 3
#define QW_ERR_HIP 4
#define QW_ERR_STATE 5

/* KV storage modes. The reference's KVCacheMode (cache.rs:172-205) has
 * Fp16, Int8 and the Turbo family; the affine modes are the codec the
 * reference names at its quantization seam (KvQuantScheme::Uniform,
 * DEFAULT_KV_GROUP_SIZE = 64, batch_quant.rs:109-158) with MLX `quantize`
 * semantics (group 64, fp16 scale and bias per group). */
#define QW_KV_FP16 0
#define QW_KV_AFFINE8 1
#define QW_KV_AFFINE4 2
/* The reference's Int8 mode (quantize_per_token / dequantize,
 * cache.rs:262-316, update_int8 :1042-1157): per (token, KV head) the scale
 * is f16(absmax / 127) (1 for an all-zero token), codes are
 * clip(round(f16(x / scale)), -128, 127) and the fetched value is
 * f16(code * scale). */
#define QW_KV_INT8 3
/* The reference's Turbo4 mode (symmetric PolarQuant, the served default,
 * cache.rs:1438-1597 update_turbo4_sym, turbo/quant.rs:119-769): per
 * (token, KV head) the row is normalised by its L2 norm, rotated by
 * signs2 . H . signs1 (H the orthonormal Walsh-Hadamard transform, signs from
 * a 32-bit LCG on the cache's seed, K and V with independent pairs), and
 * each coordinate stored as the 4-bit index of its nearest Lloyd-Max
 * centroid for N(0, 1/head_dim), two per byte (low nibble = even coord),
 * with fp16 sidecars k_rescale, v_norms and v_rescale (norm / |centroids|).
 * head_dim 128 or 256. */
#define QW_KV_TURBO4 4

typedef struct qw_kv_cache qw_kv_cache;

/* Version of this header the library was built from. */
int qw_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* qw_last_error(void);

/* ---------------------------------------------------------------- cache */

/* KVCache::new_with_mode (cache.rs:526). `capacity` rows per KV head are
 * allocated up front (rounded up to 256, the reference's growth step,
 * cache.rs:354-466 `step`); appends beyond it grow the buffers. group_size
 * must be 64 for the affine modes (ignored for fp16). head_dim: 256 or 128
 * for the affine modes; a multiple of 64 up to 256 for fp16. `device` is the
 * HIP device ordinal. */
int qw_kv_create(int mode, int group_size, int n_kv_heads, int head_dim, int capacity,
                 int device, qw_kv_cache** out);

/* KVCache::new_with_mode_and_seed (cache.rs:537): as qw_kv_create with the
 * seed of the Turbo4 sign vectors (qw_kv_create uses the reference's
 * TURBO_DEFAULT_SEED 0x7B470404, cache.rs:324). Other modes ignore it. */
int qw_kv_create_seeded(int mode, int group_size, int n_kv_heads, int head_dim, int capacity,
                        int device, uint32_t turbo_seed, qw_kv_cache** out);

/* Frees the device buffers (KVCache drop). Waits for the device first. */
int qw_kv_destroy(qw_kv_cache* cache);

/* Grows the allocation to at least `capacity` rows per head, preserving
 * contents (the reference's step-growth concatenate, cache.rs:954-1034). */
int qw_kv_reserve(qw_kv_cache* cache, int capacity, void* stream);

/* KVCache::offset (pub field, cache.rs:354): number of cached tokens. */
int qw_kv_offset(const qw_kv_cache* cache, int* offset);

/* Allocated rows per head. */
int qw_kv_capacity(const qw_kv_cache* cache, int* capacity);

/* KVCache::nbytes (cache.rs:3063): device bytes held by the cache buffers. */
int qw_kv_nbytes(const qw_kv_cache* cache, int64_t* nbytes);

/* KVCache::update (cache.rs:922): quantize-on-append of n_tokens new rows.
 * k_new, v_new: [n_kv_heads][n_tokens][head_dim] fp16 device pointers. */
int qw_kv_update(qw_kv_cache* cache, const void* k_new, const void* v_new, int n_tokens,
                 void* stream);

/* KVCache::update_and_fetch (cache.rs:2709-2834): append, then write the
 * whole visible cache, dequantized to fp16, to k_out / v_out
 * [n_kv_heads][offset][head_dim]. Dequantization is MLX's composite
 * f16(f16(code * scale) + bias). */
int qw_kv_update_and_fetch(qw_kv_cache* cache, const void* k_new, const void* v_new,
                           int n_tokens, void* k_out, void* v_out, void* stream);

/* Dequantized rows [start, start + n) of every head into k_out / v_out
 * [n_kv_heads][n][head_dim] (a window of update_and_fetch without the
 * append; the oracle route of cache.rs:3652-3697). */
int qw_kv_dequantize(const qw_kv_cache* cache, int start, int n, void* k_out, void* v_out,
                     void* stream);

/* KVCache::update_and_turbo4_attention (cache.rs:3495, causal = 0) and
 * update_and_turbo4_causal_attention (cache.rs:3520, causal = 1), with the
 * affine codec: the new rows are quantized and appended first and then
 * attended in their dequantized form (cache.rs:2723, :3508). One fused
 * dequant-in-attention pass over the packed cache, no fp16 K/V copy.
 *   q [n_q_heads][n_rows][head_dim] fp16, n_q_heads % n_kv_heads == 0;
 *   k_new, v_new [n_kv_heads][n_rows][head_dim] fp16 (n_rows new tokens);
 *   causal: bottom-right, row r sees keys t <= offset_after - n_rows + r;
 *   out [n_q_heads][n_rows][head_dim] fp16.
 * Scores are formed as f16(f16(scale) * q) . k and rounded to fp16 before
 * the fp32 softmax, as MLX's SDPA forms them.
 * On a Turbo4 cache the reference's routing applies: causal blocks of 1..5
 * rows over more than 2048 tokens (at most 32 query heads a KV head) take its fused
 * verify pass (turbo4_attention.cpp:45-264: q' = f16(q_rot * scale * log2 e),
 * fp32 scores from the packed codes); every other call takes its
 * dequantize-then-SDPA route (turbo/sparse_v.rs:1051-1072). */
int qw_kv_update_and_attention(qw_kv_cache* cache, const void* q, int n_q_heads, int n_rows,
                               const void* k_new, const void* v_new, float scale, int causal,
                               void* out, void* stream);

/* Attention of q over the cache as it is, without an append (the fused
 * prefix call turbo4_fused_attention_prefix, cache.rs:3607). With causal, row
 * r of n_rows sees keys t <= offset - n_rows + r. */
int qw_kv_attention(qw_kv_cache* cache, const void* q, int n_q_heads, int n_rows, float scale,
                    int causal, void* out, void* stream);

/* Attention with the reference's general options over fp16 K/V views:
 * layers::attention(q, k, v, scale, mask, softcap, window) (layers.rs:4010)
 * and causal_attention(q, k, v, scale, softcap, window) (lib.rs:3185).
 *   q [n_q_heads][n_rows][head_dim] fp16, head_dim 64 / 128 / 256; K and V
 *   rows [n_kv_heads][n_keys][head_dim] with element strides (% 8 == 0);
 *   causal: bottom-right, row r sees keys t <= n_keys - n_rows + r;
 *   window > 0 (causal required): also t >= n_keys - n_rows + r - window + 1,
 *     the windowed causal mask causal_attention builds (utils.rs:95-140);
 *   softcap > 0: the softcap composite (mlx_cxx_bridge.cpp:1573-1590):
 *     S = f16(q . k), s = tanh(S * scale / softcap) * softcap in fp32, fp32
 *     softmax and P.V; softcap == 0: MLX's SDPA, S = f16(f16(f16(scale) q) . k);
 *   mask (null: none) [n_q_heads or broadcast][n_rows][n_keys], key stride 1,
 *     element strides mask_head_stride (0: one mask for every head) and
 *     mask_row_stride: QW_MASK_BOOL (uint8, nonzero attends), or additive
 *     QW_DTYPE_F16 / BF16 / F32, cast to fp16 as the reference casts float
 *     masks to q's dtype (mlx_cxx_bridge.cpp:3466-3497) and added to the
 *     scores (in fp16 without softcap); a bool mask with softcap is refused
 *     (QW_ERR_UNSUPPORTED: the reference would cast it to 0/1 offsets);
 *   out [n_q_heads][n_rows][head_dim] fp16; a row with no visible key is 0.
 * A generic kernel (sdpa_general.hip), not the tuned fused paths. */
int qw_sdpa(const void* q, int n_q_heads, int n_rows, const void* k, const void* v,
            int n_kv_heads, int n_keys, int head_dim, int64_t k_head_stride, int64_t k_row_stride,
            int64_t v_head_stride, int64_t v_row_stride, float scale, int causal, int window,
            float softcap, const void* mask, int mask_dtype, int64_t mask_head_stride,
            int64_t mask_row_stride, void* out, void* stream);

/* The same over a cache (n_keys = its offset): without mask, softcap or
 * window it is qw_kv_attention; otherwise the cache's rows are dequantized
 * into a per-stream workspace and attended as qw_sdpa does, the route of the
 * runtime's masked branch (update_and_fetch + layers::attention,
 * qwen3_next.rs:316-324). On a Turbo4 cache: the rotated expansion, q rotated
 * in and the output rotated back (update_and_turbo4_attention with a mask,
 * cache.rs:3495 -> turbo/sparse_v.rs:1051-1072). The update form appends
 * k_new / v_new ([n_kv_heads][n_rows][head_dim]) first; invalid options are
 * refused before the append. */
int qw_kv_attention_general(qw_kv_cache* cache, const void* q, int n_q_heads, int n_rows,
                            float scale, int causal, int window, float softcap, const void* mask,
                            int mask_dtype, int64_t mask_head_stride, int64_t mask_row_stride,
                            void* out, void* stream);
int qw_kv_update_and_attention_general(qw_kv_cache* cache, const void* q, int n_q_heads,
                                       int n_rows, const void* k_new, const void* v_new,
                                       float scale, int causal, int window, float softcap,
                                       const void* mask, int mask_dtype, int64_t mask_head_stride,
                                       int64_t mask_row_stride, void* out, void* stream);

/* KVCache::trim (cache.rs:2251): drop the last n tokens (clamped to the
 * cached length); *trimmed receives the number removed. No device work. */
int qw_kv_trim(qw_kv_cache* cache, int n, int* trimmed);

/* KVCache::demote_fp16_to_turbo4 (cache.rs:3591-3605), to an affine mode: a
 * QW_KV_FP16 cache holding rows is re-stored as target_mode (QW_KV_AFFINE4 or
 * QW_KV_AFFINE8) by quantize-appending its rows [0, offset) to an empty cache
 * of that mode, exactly as qw_kv_update of the same rows would store them;
 * offset is unchanged. *demoted = 1 when it did so, 0 when the cache is not
 * fp16 or empty (the reference returns false). Synchronizes `stream`; the
 * fp16 rows are staged in a temporary device buffer of 2*hkv*offset*D*2 bytes.
 * The policy deciding when to call it (qwen3_5.rs:929-986) is host code. */
int qw_kv_demote(qw_kv_cache* cache, int target_mode, void* stream, int* demoted);
/* (target_mode may also be QW_KV_TURBO4: the reference's own demote.) */

/* Snapshot export in the reference's tensor layout (the packed-tensor
 * snapshot of cache.rs:570-626): for the affine modes
 *   k_codes, v_codes  [n_kv_heads][offset][head_dim*bits/32] uint32 (MLX
 *                     packing), k_scales/k_biases/v_scales/v_biases
 *                     [n_kv_heads][offset][head_dim/64] fp16;
 * for fp16 mode k_codes/v_codes receive K/V [n_kv_heads][offset][head_dim]
 * fp16 and the scale/bias pointers are ignored (may be NULL); for Int8 mode
 * k_codes/v_codes receive [n_kv_heads][offset][head_dim] int8 codes and
 * k_scales/v_scales [n_kv_heads][offset] fp16 (the reference's keys, values,
 * key_scales, val_scales), the bias pointers are ignored (may be NULL). */
int qw_kv_export(const qw_kv_cache* cache, void* k_codes, void* k_scales, void* k_biases,
                 void* v_codes, void* v_scales, void* v_biases, void* stream);

/* Snapshot import (restore_*_snapshot, cache.rs:570-626): replaces the
 * cache contents with n_tokens rows in the export layout; no requantization. */
int qw_kv_import(qw_kv_cache* cache, int n_tokens, const void* k_codes, const void* k_scales,
                 const void* k_biases, const void* v_codes, const void* v_scales,
                 const void* v_biases, void* stream);

/* Turbo4 snapshot tensors (KVCache::turbo4_snapshot_tensors, cache.rs:570):
 *   k_packed, v_packed [n_kv_heads][offset][head_dim/2] uint8 (two indices a
 *   byte, low nibble = even coord), k_rescale, v_norms, v_rescale
 *   [n_kv_heads][offset] fp16. QW_ERR_STATE unless the cache is Turbo4. */
int qw_kv_export_turbo4(const qw_kv_cache* cache, void* k_packed, void* k_rescale,
                        void* v_packed, void* v_norms, void* v_rescale, void* stream);

/* restore_turbo4_snapshot (cache.rs:581-626): the cache holds exactly the
 * given n_tokens > 0 rows in the export layout; no requantization. */
int qw_kv_import_turbo4(qw_kv_cache* cache, int n_tokens, const void* k_packed,
                        const void* k_rescale, const void* v_packed, const void* v_norms,
                        const void* v_rescale, void* stream);

/* Host-only (no device work) tables of the Turbo4 codec, for inspection and
 * tests. optimal_centroids (turbo/codebook.rs:139): the 2^bits sorted
 * Lloyd-Max centroids for N(0, 1/head_dim) into centroids (bits 1..8);
 * generate_signs (turbo/quant.rs:217): len +-1 floats from the LCG on seed. */
int qw_turbo4_codebook(int bits, int head_dim, float* centroids);
int qw_turbo4_signs(int len, uint32_t seed, float* signs);

/* ---------------------------------------------------------------- D-LSA */

/* dlsa_attention::sparse_attention (crates/mlxcel-core/src/dlsa_attention.rs:31)
 * -> mlx_cxx::dlsa_sparse_attention (mlx_cxx_dlsa_attention.cpp:420-556):
 * every query row r attends over the keys lists[r, 0:lengths[r]] of its KV
 * head (head h reads KV head h / (n_q_heads / n_kv_heads)); list order is
 * irrelevant up to fp32 rounding, entries outside [0, n_keys) are skipped,
 * a row without a valid entry is zeros. Softmax and accumulation in fp32.
 *   q   [n_q_heads][n_rows][head_dim] fp16
 *   k,v fp16, element (h, t, d) at k[h*k_head_stride + t*k_row_stride + d]
 *       (strided views of a larger cache are read in place, never copied)
 *   lists [n_rows][width] int32, lengths [n_rows] int32 (device)
 *   out [n_q_heads][n_rows][head_dim] fp16
 * head_dim in {64, 128, 256}; n_q_heads / n_kv_heads <= 16. */
int qw_dlsa_sparse_attention(const void* q, const void* k, const void* v, int64_t k_head_stride,
                             int64_t k_row_stride, int64_t v_head_stride, int64_t v_row_stride,
                             const int32_t* lists, const int32_t* lengths, int n_rows, int width,
                             int n_q_heads, int n_kv_heads, int head_dim, int n_keys,
                             float scale, void* out, void* stream);

/* The D-LSA read over a KV cache in place: what the reference's caller
 * (crates/runtime/src/qwen3_next/dlsa.rs:161-177) does with
 * KVCache::update_and_fetch (cache.rs:2709) followed by
 * dlsa_attention::sparse_attention (dlsa_attention.rs:31) on the fetched
 * views, without the fetch. Keys are the cache's rows [0, offset); the
 * contract is qw_dlsa_sparse_attention's (q [n_q_heads][n_rows][head_dim],
 * lists [n_rows][width] int32 device, lengths [n_rows], entries outside
 * [0, offset) skipped, fp32 softmax, out like q). fp16, affine and Int8
 * caches are read in place, quantized rows dequantized inside the gather
 * exactly as the fetch would (f16(f16(code * scale) + bias)); a Turbo4 cache
 * is fetched to fp16 first (into a buffer the cache keeps), as the
 * reference's own update_and_fetch does. QW_ERR_INVALID_ARGUMENT on an empty
 * cache. */
int qw_kv_dlsa_attention(qw_kv_cache* cache, const void* q, int n_q_heads, int n_rows,
                         const int32_t* lists, const int32_t* lengths, int width, float scale,
                         void* out, void* stream);

/* update (quantize-on-append of the n_rows new K/V rows, [n_kv_heads][n_rows]
 * [head_dim] fp16), then qw_kv_dlsa_attention: the update_and_fetch +
 * sparse_attention pair of qwen3_next/dlsa.rs:161-177 in one call. */
int qw_kv_update_and_dlsa_attention(qw_kv_cache* cache, const void* q, int n_q_heads,
                                    int n_rows, const void* k_new, const void* v_new,
                                    const int32_t* lists, const int32_t* lengths, int width,
                                    float scale, void* out, void* stream);

/* Element types of the typed D-LSA read. */
#define QW_DTYPE_F16 0
#define QW_DTYPE_BF16 1
#define QW_DTYPE_F32 2
/* Mask dtype of the general attention calls: uint8, nonzero = attend. */
#define QW_MASK_BOOL 3

/* dlsa_attention::sparse_attention_with (dlsa_attention.rs:44) with the
 * reference's full dtype and head-dim contract (mlx_cxx_dlsa_attention.cpp:
 * 429-470): q in q_dtype, K and V alike in kv_dtype, each of QW_DTYPE_F16 /
 * _BF16 / _F32; head_dim 32, 64, 128 or 256; n_q_heads / n_kv_heads <= 8;
 * out [n_q_heads][n_rows][head_dim] in q_dtype. Strides, lists, lengths and
 * the launch knobs as qw_dlsa_sparse_attention_with (waves above 8 run as 8
 * at head_dim 256). Scores, softmax and P.V
 * are fp32 (inputs widened exactly); only the output is rounded. fp16 q with
 * fp16 K/V at head_dim >= 64 is the fp16 read itself (the same result as
 * qw_dlsa_sparse_attention_with, bit for bit). */
int qw_dlsa_sparse_attention_typed(const void* q, int q_dtype, const void* k, const void* v,
                                   int kv_dtype, int64_t k_head_stride, int64_t k_row_stride,
                                   int64_t v_head_stride, int64_t v_row_stride,
                                   const int32_t* lists, const int32_t* lengths, int n_rows,
                                   int width, int n_q_heads, int n_kv_heads, int head_dim,
                                   int n_keys, float scale, int parts, int waves, void* out,
                                   void* stream);

/* dlsa_attention::sparse_attention_with (dlsa_attention.rs:44): the same read
 * with explicit launch knobs; 0 = automatic. parts: split-K partitions of
 * each list (1 = one pass, at most 128); waves: wavefronts per workgroup
 * (1..16). */
int qw_dlsa_sparse_attention_with(const void* q, const void* k, const void* v,
                                  int64_t k_head_stride, int64_t k_row_stride,
                                  int64_t v_head_stride, int64_t v_row_stride,
                                  const int32_t* lists, const int32_t* lengths, int n_rows,
                                  int width, int n_q_heads, int n_kv_heads, int head_dim,
                                  int n_keys, float scale, int parts, int waves, void* out,
                                  void* stream);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). The same read and arguments as
 * qw_dlsa_sparse_attention_with, but its split-K partials live in a fixed
 * 4 MiB device array of the library (each GPU holds its own copy from load
 * until the process ends), so the call allocates nothing. parts = 0 picks
 * the automatic count, lowered until the partials, n_rows * n_q_heads *
 * parts * (head_dim * 4 + 8) bytes, fit the 4 MiB; an explicit parts > 1
 * whose partials do not fit returns QW_ERR_INVALID_ARGUMENT. Every call on a
 * GPU shares that GPU's array: two calls that overlap on one GPU (other
 * streams or threads) race and must be ordered by the caller. */
int qw_dlsa_sparse_attention_noalloc(const void* q, const void* k, const void* v,
                                     int64_t k_head_stride, int64_t k_row_stride,
                                     int64_t v_head_stride, int64_t v_row_stride,
                                     const int32_t* lists, const int32_t* lengths, int n_rows,
                                     int width, int n_q_heads, int n_kv_heads, int head_dim,
                                     int n_keys, float scale, int parts, int waves, void* out,
                                     void* stream);

/* D-LSA K1 select: dlsa_select (crates/mlxcel-core/src/dlsa_kernels.rs:57-84)
 * / dlsa_select_with (:88-117), the device twin of the host select
 * (crates/runtime/src/dlsa/select.rs:65-115). For each of n_rows query rows:
 *   scores    [n_rows][score_stride] f32: row r ranks its first
 *             v = min(floor(positions[r] / window) * buckets_per_block,
 *             total_rows) columns (when v > score_stride only the columns
 *             present: status bit 2), score descending, -0 == +0, a NaN below
 *             every number (status bit 1), ties to the lower bucket;
 *   members   [n_member_rows][bucket_cap] i32, each bucket's key positions
 *             ascending, -1 padded; total_rows <= n_member_rows;
 *   positions [n_rows] i32 >= 0.
 * Outputs (device, i32): picked [n_rows][top_p] (best first, -1 padded);
 * lists [n_rows][top_k + window + sink]: the picked buckets' members in
 * [sink, window_start) (pick order, members ascending, at most top_k), then
 * the window [window_start, p], then the sinks [0, min(sink, window_start,
 * p + 1)), -1 padded, with window_start = max(0, p + 1 - window); lengths
 * [n_rows]; status [n_rows]. top_p <= 2048 (DLSA_TOP_P_MAX). `threads` is the
 * workgroup size (0 = automatic, else a power of two in [64, 1024]); the
 * outputs do not depend on it. */
int qw_dlsa_select(const float* scores, int64_t score_stride, const int32_t* members,
                   int n_member_rows, int bucket_cap, const int32_t* positions, int n_rows,
                   int total_rows, int window, int sink, int top_k, int top_p,
                   int buckets_per_block, int threads, int32_t* lists, int32_t* lengths,
                   int32_t* picked, int32_t* status, void* stream);

/* Fused q/k RoPE + append layout: fused_rope_qk_append
 * (crates/mlxcel-core/src/lib.rs:1462-1476, kernel
 * crates/mlx-cpp/turbo/fused_rope_append.cpp:80-180, contract :378-420).
 *   qkv   [batch][seq][(n_q_heads + 2 n_kv_heads) head_dim] fp16, per token
 *         the q heads, then the k heads, then the v heads;
 *   q_out [batch][n_q_heads][seq][head_dim] fp16, rotated;
 *   k_out, v_out [batch][n_kv_heads][seq][head_dim] (dest_layout 0, dense
 *         slab) or [batch][seq][n_kv_heads][head_dim] (dest_layout 1, paged
 *         pool rows); k rotated, v copied.
 * Token t rotates at position positions_base + t: pair p of the first
 * rope_dims dims of a head ((2p, 2p+1) if traditional, else (p, p +
 * rope_dims/2)) turns by (rope_scale * position) * exp2(-(p / (rope_dims/2))
 * * log2(rope_base)); the other dims are copied. head_dim even, rope_dims
 * even, positive and <= head_dim, else QW_ERR_INVALID_ARGUMENT. */
int qw_fused_rope_qk_append(const void* qkv, int batch, int seq, int n_q_heads, int n_kv_heads,
                            int head_dim, int rope_dims, float rope_base, float rope_scale,
                            int traditional, int positions_base, int dest_layout, void* q_out,
                            void* k_out, void* v_out, void* stream);

/* The same RoPE with the cache append fused in: what
 * Attention::forward_fused_rope_append (crates/mlxcel-core/src/layers.rs:
 * 2852-2905) followed by KVCache::update (cache.rs:922) does, without the
 * k / v round trip through memory. qkv [n_tokens][(n_q_heads + 2 hkv)
 * head_dim] fp16 (one sequence; hkv and head_dim are the cache's); the
 * rotated q goes to q_out [n_q_heads][n_tokens][head_dim]; the rotated k
 * (rounded to fp16) and v are appended as qw_kv_update appends them, token t
 * at position position0 + t. Same argument contract as
 * qw_fused_rope_qk_append. */
int qw_kv_rope_update(qw_kv_cache* cache, const void* qkv, int n_q_heads, int n_tokens,
                      int rope_dims, int traditional, float rope_base, float rope_scale,
                      int position0, void* q_out, void* stream);

/* A decode layer's attention from the projection: what
 * Attention::forward_fused_rope_append (crates/mlxcel-core/src/layers.rs:
 * 2852-2905) followed by KVCache::update_and_turbo4_attention (cache.rs:3495,
 * the served decode call, crates/runtime/src/qwen3_next.rs:297-329) computes,
 * i.e. qw_kv_rope_update then qw_kv_attention(q_out, n_tokens, scale,
 * causal). Arguments as qw_kv_rope_update, plus scale and causal for the
 * attention and out [n_q_heads][n_tokens][head_dim] fp16. q_out receives the
 * rotated q either way. Decode-route shapes (affine, Int8 and Turbo4 caches,
 * at most 16 query rows a KV head, rope_dims a multiple of 16, a non-empty
 * cache) run as one decode launch plus the merge: the attention workgroups
 * rotate their q rows themselves and the launch's append unit appends the
 * rotated k and v; other shapes run the two calls. */
int qw_kv_rope_update_and_attention(qw_kv_cache* cache, const void* qkv, int n_q_heads,
                                    int n_tokens, int rope_dims, int traditional, float rope_base,
                                    float rope_scale, int position0, float scale, int causal,
                                    void* q_out, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QWATTN_H */
