/*
 * qw_oracle.h - CPU restatement of the reference's full-attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker and the
 * reported CPU baseline. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. The product (qw_amd, libqwattn.so) never
 * links, imports or calls it.
 *
 * Every function restates one piece of the reference's semantics:
 *   - affine quantize / dequantize: MLX `quantize` / `dequantize` as called
 *     through crates/mlxcel-core/cpp/mlx_cxx_bridge.cpp:2991-3040, :6347-6393
 *     (MLX pinned at 7ca40033132dae444d45f7fc3daae57e24c13f6c,
 *     crates/mlx-cpp/CMakeLists.txt:83), at the KV seam
 *     crates/mlxcel-core/src/cache/batch_quant.rs:109-158 (group 64).
 *   - SDPA with the MLX CPU-stream fp16 roundings: the unfused fallback of
 *     mlx::core::fast::scaled_dot_product_attention reached through
 *     crates/mlxcel-core/src/layers.rs:4010-4066 and lib.rs:3185-3287,
 *     bottom-right causal as in crates/mlxcel-core/src/cache.rs:3512-3519.
 *   - D-LSA gathered read: crates/mlxcel-core/cpp/mlx_cxx_dlsa_attention.cpp:1-31
 *     (K2 contract) and crates/runtime/src/dlsa/attend.rs:21-160 (MLX read).
 *
 * Pinning status is stated per function in qw_oracle.c.
 */
#ifndef QW_ORACLE_H
#define QW_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 <-> binary32, round-to-nearest-even (own implementation). */
uint16_t qwo_f32_to_f16(float f);
float qwo_f16_to_f32(uint16_t h);
void qwo_f32_to_f16_array(const float* in, uint16_t* out, int64_t n);
void qwo_f16_to_f32_array(const uint16_t* in, float* out, int64_t n);

/* MLX affine quantize of n_rows rows of `dim` fp16 values, groups of `group`
 * along the row, `bits` in {4, 8}. codes: n_rows * dim * bits / 32 words,
 * LSB-first; scales/biases: n_rows * dim / group fp16. Returns 0, or -1 on a
 * bad argument. */
int qwo_affine_quantize(const uint16_t* w, int64_t n_rows, int dim, int group, int bits,
                        uint32_t* codes, uint16_t* scales, uint16_t* biases);

/* MLX composite dequantize: out = f16(f16(code * scale) + bias). */
int qwo_affine_dequantize(const uint32_t* codes, const uint16_t* scales,
                          const uint16_t* biases, int64_t n_rows, int dim, int group,
                          int bits, uint16_t* out);

/* Int8 per-token KV codec (cache.rs:262-316 quantize_per_token / dequantize,
 * MLX fp16 ops): per row of `dim` fp16 values, scale = f16(absmax / 127),
 * replaced by 1 when it is 0; code = clip(round(f16(x / scale)), -128, 127)
 * with round ties-to-even (std::rint). codes: n_rows * dim int8; scales:
 * n_rows fp16. Dequantize: out = f16(code * scale). Return 0, or -1 on a bad
 * argument. */
int qwo_int8_quantize(const uint16_t* w, int64_t n_rows, int dim, int8_t* codes,
                      uint16_t* scales);
int qwo_int8_dequantize(const int8_t* codes, const uint16_t* scales, int64_t n_rows, int dim,
                        uint16_t* out);

/* MLX CPU-stream SDPA over fp16 tensors with the fallback's fp16 roundings.
 *   q   [hq, L, D]   (row r of head h at q + (h * L + r) * D)
 *   k,v [hkv, T, D]
 *   q_pos: NULL for no mask, else the key-space position of each query row;
 *          row r sees keys t <= q_pos[r] (bottom-right causal uses
 *          q_pos[r] = T - L + r).
 *   out [hq, L, D] fp16.  n_threads >= 1. */
int qwo_sdpa_mlx_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, int hq,
                     int hkv, int L, int T, int D, float scale, const int32_t* q_pos,
                     uint16_t* out, int n_threads);

/* The same attention in double precision with no intermediate rounding
 * (closed form, used to bound the fp16-rounding oracle). out fp64. */
int qwo_sdpa_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v, int hq, int hkv,
                 int L, int T, int D, double scale, const int32_t* q_pos, double* out,
                 int n_threads);

/* D-LSA gathered read (K2 contract): every row r of q attends over the keys
 * lists[r, 0:lengths[r]] of its KV head; entries outside [0, T) are skipped,
 * a row with no valid entry yields zeros. Softmax and accumulation in double,
 * result rounded to fp32.
 *   q   [hq, L, D] fp16 contiguous
 *   k,v fp16 with element strides (head_stride, row_stride), unit last stride
 *   lists [L, W] int32, lengths [L] int32
 *   out [hq, L, D] fp32 */
int qwo_dlsa_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                       int64_t k_head_stride, int64_t k_row_stride, int64_t v_head_stride,
                       int64_t v_row_stride, const int32_t* lists, const int32_t* lengths,
                       int L, int W, int hq, int hkv, int D, int T, float scale, float* out,
                       int n_threads);

/* One quantized-cache layer call as the reference composes it
 * (crates/mlxcel-core/src/cache.rs:3495-3510 with the affine codec in place
 * of Turbo4): quantize the new rows, dequantize the whole visible cache with
 * the MLX composite, then MLX SDPA. The cache arrays hold `t_old` quantized
 * rows per head at capacity `cap` (row-major codes, reference layout); the
 * new rows are written at t_old .. t_old + L - 1.
 *   q [hq, L, D], k_new/v_new [hkv, L, D] fp16; causal != 0 -> bottom-right.
 *   Row subset: when n_sel > 0 only the query rows sel[0..n_sel) are
 *   computed and out is [hq, n_sel, D]. */
int qwo_affine_layer_call(uint32_t* k_codes, uint16_t* k_scales, uint16_t* k_biases,
                          uint32_t* v_codes, uint16_t* v_scales, uint16_t* v_biases,
                          int64_t cap, int t_old, const uint16_t* q, const uint16_t* k_new,
                          const uint16_t* v_new, int hq, int hkv, int L, int D, int group,
                          int bits, float scale, int causal, const int32_t* sel, int n_sel,
                          uint16_t* out, int n_threads);

#ifdef __cplusplus
}
#endif

#endif
