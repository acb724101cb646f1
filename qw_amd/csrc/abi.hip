// abi.hip - extern "C" entry points of libqwattn.so (declared in
// include/qwattn.h). Each wrapper validates its handle and forwards to the
// C++ KVCache / D-LSA implementation; no exception crosses the boundary.
#include <new>

#include "kv_cache.hpp"

struct qw_kv_cache {
    qw::KVCache impl;
};


#define QW_HANDLE(c)                                                          \
    do {                                                                      \
        if (!(c)) {                                                           \
            qw::set_error("null qw_kv_cache handle");                         \
            return QW_ERR_INVALID_ARGUMENT;                                   \
        }                                                                     \
    } while (0)

#define QW_GUARDED(expr)                                                      \
    try {                                                                     \
        return (expr);                                                        \
    } catch (const std::bad_alloc&) {                                         \
        qw::set_error("host allocation failed");                              \
        return QW_ERR_OUT_OF_MEMORY;                                          \
    } catch (...) {                                                           \
        qw::set_error("unexpected C++ exception");                            \
        return QW_ERR_STATE;                                                  \
    }

extern "C" {

int qw_abi_version(void) { return QWATTN_ABI_VERSION; }

const char* qw_last_error(void) { return qw::last_error(); }

int qw_kv_create(int mode, int group_size, int n_kv_heads, int head_dim, int capacity,
                 int device, qw_kv_cache** out) {
    return qw_kv_create_seeded(mode, group_size, n_kv_heads, head_dim, capacity, device,
                               qw::turbo4::kDefaultSeed, out);
}

int qw_kv_create_seeded(int mode, int group_size, int n_kv_heads, int head_dim, int capacity,
                        int device, uint32_t turbo_seed, qw_kv_cache** out) {
    if (!out) {
        qw::set_error("qw_kv_create: null out pointer");
        return QW_ERR_INVALID_ARGUMENT;
    }
    *out = nullptr;
    qw_kv_cache* c = new (std::nothrow) qw_kv_cache();
    if (!c) {
        qw::set_error("qw_kv_create: host allocation failed");
        return QW_ERR_OUT_OF_MEMORY;
    }
    int rc;
    c->impl.turbo_seed = turbo_seed;
    try {
        rc = c->impl.init(mode, group_size, n_kv_heads, head_dim, capacity, device);
    } catch (...) {
        rc = QW_ERR_STATE;
        qw::set_error("qw_kv_create: unexpected C++ exception");
    }
    if (rc != QW_OK) {
        c->impl.release();
        delete c;
        return rc;
    }
    *out = c;
    return QW_OK;
}

int qw_kv_destroy(qw_kv_cache* cache) {
    if (!cache) return QW_OK;
    cache->impl.release();
    delete cache;
    return QW_OK;
}

int qw_kv_reserve(qw_kv_cache* cache, int capacity, void* stream) {
    QW_HANDLE(cache);
    QW_GUARDED(cache->impl.reserve(capacity, (hipStream_t)stream));
}

int qw_kv_offset(const qw_kv_cache* cache, int* offset) {
    QW_HANDLE(cache);
    if (!offset) {
        qw::set_error("qw_kv_offset: null out pointer");
        return QW_ERR_INVALID_ARGUMENT;
    }
    *offset = cache->impl.offset;
    return QW_OK;
}

int qw_kv_capacity(const qw_kv_cache* cache, int* capacity) {
    QW_HANDLE(cache);
    if (!capacity) {
        qw::set_error("qw_kv_capacity: null out pointer");
        return QW_ERR_INVALID_ARGUMENT;
    }
    *capacity = cache->impl.cap;
    return QW_OK;
}

int qw_kv_nbytes(const qw_kv_cache* cache, int64_t* nbytes) {
    QW_HANDLE(cache);
    if (!nbytes) {
        qw::set_error("qw_kv_nbytes: null out pointer");
        return QW_ERR_INVALID_ARGUMENT;
    }
    *nbytes = cache->impl.nbytes();
    return QW_OK;
}

int qw_kv_update(qw_kv_cache* cache, const void* k_new, const void* v_new, int n_tokens,
                 void* stream) {
    QW_HANDLE(cache);
    QW_GUARDED(cache->impl.update(k_new, v_new, n_tokens, (hipStream_t)stream));
}

int qw_kv_update_and_fetch(qw_kv_cache* cache, const void* k_new, const void* v_new,
                           int n_tokens, void* k_out, void* v_out, void* stream) {
    QW_HANDLE(cache);
    QW_GUARDED(cache->impl.update_and_fetch(k_new, v_new, n_tokens, k_out, v_out,
                                            (hipStream_t)stream));
}

int qw_kv_dequantize(const qw_kv_cache* cache, int start, int n, void* k_out, void* v_out,
                     void* stream) {
    QW_HANDLE(cache);
    QW_GUARDED(cache->impl.dequantize(start, n, k_out, v_out, (hipStream_t)stream));
}

int qw_kv_update_and_attention(qw_kv_cache* cache, const void* q, int n_q_heads, int n_rows,
                               const void* k_new, const void* v_new, float scale, int causal,
                               void* out, void* stream) {
    QW_HANDLE(cache);
    QW_GUARDED(cache->impl.update_and_attention(q, n_q_heads, n_rows, k_new, v_new, scale,
                                                causal != 0, out, (hipStream_t)stream));
}

int qw_kv_attention(qw_kv_cache* cache, const void* q, int n_q_heads, int n_rows, float scale,
                    int causal, void* out, void* stream) {
    QW_HANDLE(cache);
    QW_GUARDED(cache->impl.attention(q, n_q_heads, n_rows, scale, causal != 0, out,
                                     (hipStream_t)stream));
}

static qw::SdpaOptions sdpa_options(int causal, int window, float softcap, const void* mask,
                                    int mask_dtype, int64_t mask_head_stride,
                                    int64_t mask_row_stride) {
    qw::SdpaOptions o;
    o.causal = causal != 0;
    o.window = window;
    o.softcap = softcap;
    o.mask = mask;
    o.mask_dtype = mask_dtype;
    o.mask_head_stride = mask_head_stride;
    o.mask_row_stride = mask_row_stride;
    return o;
}

// Append, then the general attention (update_and_fetch + layers::attention,
// qwen3_next.rs:316-324; update_and_turbo4_attention, cache.rs:3495). The
// options are checked before the append, so a rejected call leaves the cache
// as it was.
static int update_and_general(qw::KVCache& c, const void* q, int n_q_heads, int n_rows,
                              const void* k_new, const void* v_new, float scale,
                              const qw::SdpaOptions& o, void* out, hipStream_t stream) {
    const bool bad_mask = o.mask && (o.mask_dtype < QW_DTYPE_F16 || o.mask_dtype > QW_MASK_BOOL ||
                                     (o.mask_dtype == QW_MASK_BOOL && o.softcap > 0.0f) ||
                                     o.mask_head_stride < 0 || o.mask_row_stride < 0);
    QW_REQUIRE(q && out && n_rows > 0 && n_q_heads > 0 && n_q_heads % c.hkv == 0,
               QW_ERR_INVALID_ARGUMENT, "attention: bad q geometry");
    QW_REQUIRE(!(o.softcap < 0.0f) && o.softcap == o.softcap && (o.window <= 0 || o.causal) &&
                   !bad_mask,
               QW_ERR_INVALID_ARGUMENT, "attention: invalid general options (see qw_sdpa)");
    int rc = c.update(k_new, v_new, n_rows, stream);
    if (rc) return rc;
    return qw::cache_attention_general(c, q, n_q_heads, n_rows, scale, o, out, stream);
}

int qw_sdpa(const void* q, int n_q_heads, int n_rows, const void* k, const void* v,
            int n_kv_heads, int n_keys, int head_dim, int64_t k_head_stride, int64_t k_row_stride,
            int64_t v_head_stride, int64_t v_row_stride, float scale, int causal, int window,
            float softcap, const void* mask, int mask_dtype, int64_t mask_head_stride,
            int64_t mask_row_stride, void* out, void* stream) {
    QW_GUARDED(qw::sdpa_general(q, n_q_heads, n_rows, k, v, n_kv_heads, n_keys, head_dim,
                                k_head_stride, k_row_stride, v_head_stride, v_row_stride, scale,
                                sdpa_options(causal, window, softcap, mask, mask_dtype,
                                             mask_head_stride, mask_row_stride),
                                out, (hipStream_t)stream));
}

int qw_kv_attention_general(qw_kv_cache* cache, const void* q, int n_q_heads, int n_rows,
                            float scale, int causal, int window, float softcap, const void* mask,
                            int mask_dtype, int64_t mask_head_stride, int64_t mask_row_stride,
                            void* out, void* stream) {
    QW_HANDLE(cache);
    QW_GUARDED(qw::cache_attention_general(
        cache->impl, q, n_q_heads, n_rows, scale,
        sdpa_options(causal, window, softcap, mask, mask_dtype, mask_head_stride, mask_row_stride),
        out, (hipStream_t)stream));
}

int qw_kv_update_and_attention_general(qw_kv_cache* cache, const void* q, int n_q_heads,
                                       int n_rows, const void* k_new, const void* v_new,
                                       float scale, int causal, int window, float softcap,
                                       const void* mask, int mask_dtype, int64_t mask_head_stride,
                                       int64_t mask_row_stride, void* out, void* stream) {
    QW_HANDLE(cache);
    if (!mask && softcap == 0.0f && window <= 0)
        QW_GUARDED(cache->impl.update_and_attention(q, n_q_heads, n_rows, k_new, v_new, scale,
                                                    causal != 0, out, (hipStream_t)stream));
    QW_GUARDED(update_and_general(cache->impl, q, n_q_heads, n_rows, k_new, v_new, scale,
                                  sdpa_options(causal, window, softcap, mask, mask_dtype,
                                               mask_head_stride, mask_row_stride),
                                  out, (hipStream_t)stream));
}

int qw_kv_dlsa_attention(qw_kv_cache* cache, const void* q, int n_q_heads, int n_rows,
                         const int32_t* lists, const int32_t* lengths, int width, float scale,
                         void* out, void* stream) {
    QW_HANDLE(cache);
    QW_GUARDED(cache->impl.dlsa_attention(q, n_q_heads, n_rows, lists, lengths, width, scale, out,
                                          (hipStream_t)stream));
}

int qw_kv_update_and_dlsa_attention(qw_kv_cache* cache, const void* q, int n_q_heads,
                                    int n_rows, const void* k_new, const void* v_new,
                                    const int32_t* lists, const int32_t* lengths, int width,
                                    float scale, void* out, void* stream) {
    QW_HANDLE(cache);
    QW_GUARDED(cache->impl.update_and_dlsa_attention(q, n_q_heads, n_rows, k_new, v_new, lists,
                                                     lengths, width, scale, out,
                                                     (hipStream_t)stream));
}

int qw_kv_trim(qw_kv_cache* cache, int n, int* trimmed) {
    QW_HANDLE(cache);
    const int m = cache->impl.trim(n);
    if (trimmed) *trimmed = m;
    return QW_OK;
}

static int demote_call(qw_kv_cache* cache, int target_mode, void* stream, int* demoted) {
    int d = 0;
    const int rc = cache->impl.demote(target_mode, (hipStream_t)stream, &d);
    if (demoted) *demoted = d;
    return rc;
}

int qw_kv_demote(qw_kv_cache* cache, int target_mode, void* stream, int* demoted) {
    QW_HANDLE(cache);
    QW_GUARDED(demote_call(cache, target_mode, stream, demoted));
}

int qw_kv_export(const qw_kv_cache* cache, void* k_codes, void* k_scales, void* k_biases,
                 void* v_codes, void* v_scales, void* v_biases, void* stream) {
    QW_HANDLE(cache);
    QW_GUARDED(cache->impl.export_tensors(k_codes, k_scales, k_biases, v_codes, v_scales,
                                          v_biases, (hipStream_t)stream));
}

int qw_kv_import(qw_kv_cache* cache, int n_tokens, const void* k_codes, const void* k_scales,
                 const void* k_biases, const void* v_codes, const void* v_scales,
                 const void* v_biases, void* stream) {
    QW_HANDLE(cache);
    QW_GUARDED(cache->impl.import_tensors(n_tokens, k_codes, k_scales, k_biases, v_codes,
                                          v_scales, v_biases, (hipStream_t)stream));
}

int qw_dlsa_sparse_attention(const void* q, const void* k, const void* v, int64_t k_head_stride,
                             int64_t k_row_stride, int64_t v_head_stride, int64_t v_row_stride,
                             const int32_t* lists, const int32_t* lengths, int n_rows, int width,
                             int n_q_heads, int n_kv_heads, int head_dim, int n_keys,
                             float scale, void* out, void* stream) {
    QW_GUARDED(qw::dlsa_sparse_attention(q, k, v, k_head_stride, k_row_stride, v_head_stride,
                                         v_row_stride, lists, lengths, n_rows, width, n_q_heads,
                                         n_kv_heads, head_dim, n_keys, scale, 0, 0, out,
                                         (hipStream_t)stream));
}

int qw_dlsa_sparse_attention_typed(const void* q, int q_dtype, const void* k, const void* v,
                                   int kv_dtype, int64_t k_head_stride, int64_t k_row_stride,
                                   int64_t v_head_stride, int64_t v_row_stride,
                                   const int32_t* lists, const int32_t* lengths, int n_rows,
                                   int width, int n_q_heads, int n_kv_heads, int head_dim,
                                   int n_keys, float scale, int parts, int waves, void* out,
                                   void* stream) {
    QW_GUARDED(qw::dlsa_sparse_attention_typed(q, q_dtype, k, v, kv_dtype, k_head_stride,
                                               k_row_stride, v_head_stride, v_row_stride, lists,
                                               lengths, n_rows, width, n_q_heads, n_kv_heads,
                                               head_dim, n_keys, scale, parts, waves, out,
                                               (hipStream_t)stream));
}

int qw_dlsa_sparse_attention_with(const void* q, const void* k, const void* v,
                                  int64_t k_head_stride, int64_t k_row_stride,
                                  int64_t v_head_stride, int64_t v_row_stride,
                                  const int32_t* lists, const int32_t* lengths, int n_rows,
                                  int width, int n_q_heads, int n_kv_heads, int head_dim,
                                  int n_keys, float scale, int parts, int waves, void* out,
                                  void* stream) {
    QW_GUARDED(qw::dlsa_sparse_attention(q, k, v, k_head_stride, k_row_stride, v_head_stride,
                                         v_row_stride, lists, lengths, n_rows, width, n_q_heads,
                                         n_kv_heads, head_dim, n_keys, scale, parts, waves, out,
                                         (hipStream_t)stream));
}

int qw_dlsa_sparse_attention_noalloc(const void* q, const void* k, const void* v,
                                     int64_t k_head_stride, int64_t k_row_stride,
                                     int64_t v_head_stride, int64_t v_row_stride,
                                     const int32_t* lists, const int32_t* lengths, int n_rows,
                                     int width, int n_q_heads, int n_kv_heads, int head_dim,
                                     int n_keys, float scale, int parts, int waves, void* out,
                                     void* stream) {
    QW_GUARDED(qw::dlsa_sparse_attention_noalloc(q, k, v, k_head_stride, k_row_stride,
                                                 v_head_stride, v_row_stride, lists, lengths,
                                                 n_rows, width, n_q_heads, n_kv_heads, head_dim,
                                                 n_keys, scale, parts, waves, out,
                                                 (hipStream_t)stream));
}

int qw_dlsa_select(const float* scores, int64_t score_stride, const int32_t* members,
                   int n_member_rows, int bucket_cap, const int32_t* positions, int n_rows,
                   int total_rows, int window, int sink, int top_k, int top_p,
                   int buckets_per_block, int threads, int32_t* lists, int32_t* lengths,
                   int32_t* picked, int32_t* status, void* stream) {
    QW_GUARDED(qw::dlsa_select(scores, score_stride, members, n_member_rows, bucket_cap, positions,
                               n_rows, total_rows, window, sink, top_k, top_p, buckets_per_block,
                               threads, lists, lengths, picked, status, (hipStream_t)stream));
}

int qw_kv_export_turbo4(const qw_kv_cache* cache, void* k_packed, void* k_rescale,
                        void* v_packed, void* v_norms, void* v_rescale, void* stream) {
    QW_HANDLE(cache);
    QW_GUARDED(cache->impl.turbo4_export(k_packed, k_rescale, v_packed, v_norms, v_rescale,
                                         (hipStream_t)stream));
}

int qw_kv_import_turbo4(qw_kv_cache* cache, int n_tokens, const void* k_packed,
                        const void* k_rescale, const void* v_packed, const void* v_norms,
                        const void* v_rescale, void* stream) {
    QW_HANDLE(cache);
    QW_GUARDED(cache->impl.turbo4_import(n_tokens, k_packed, k_rescale, v_packed, v_norms,
                                         v_rescale, (hipStream_t)stream));
}

int qw_turbo4_codebook(int bits, int head_dim, float* centroids) {
    if (bits < 1 || bits > 8 || head_dim <= 0 || !centroids) {
        qw::set_error("qw_turbo4_codebook: bits must be 1..8, head_dim > 0, non-null output");
        return QW_ERR_INVALID_ARGUMENT;
    }
    try {
        const std::vector<float> c = qw::turbo4::centroids(bits, head_dim);
        for (size_t i = 0; i < c.size(); i++) centroids[i] = c[i];
    } catch (...) {
        qw::set_error("qw_turbo4_codebook: host allocation failed");
        return QW_ERR_OUT_OF_MEMORY;
    }
    return QW_OK;
}

int qw_turbo4_signs(int len, uint32_t seed, float* signs) {
    if (len < 0 || (len > 0 && !signs)) {
        qw::set_error("qw_turbo4_signs: len must be >= 0 with a non-null output");
        return QW_ERR_INVALID_ARGUMENT;
    }
    try {
        const std::vector<float> s = qw::turbo4::signs(len, seed);
        for (int i = 0; i < len; i++) signs[i] = s[i];
    } catch (...) {
        qw::set_error("qw_turbo4_signs: host allocation failed");
        return QW_ERR_OUT_OF_MEMORY;
    }
    return QW_OK;
}

int qw_fused_rope_qk_append(const void* qkv, int batch, int seq, int n_q_heads, int n_kv_heads,
                            int head_dim, int rope_dims, float rope_base, float rope_scale,
                            int traditional, int positions_base, int dest_layout, void* q_out,
                            void* k_out, void* v_out, void* stream) {
    QW_GUARDED(qw::fused_rope_qk_append(qkv, batch, seq, n_q_heads, n_kv_heads, head_dim,
                                        rope_dims, rope_base, rope_scale, traditional,
                                        positions_base, dest_layout, q_out, k_out, v_out,
                                        (hipStream_t)stream));
}

int qw_kv_rope_update(qw_kv_cache* cache, const void* qkv, int n_q_heads, int n_tokens,
                      int rope_dims, int traditional, float rope_base, float rope_scale,
                      int position0, void* q_out, void* stream) {
    QW_HANDLE(cache);
    QW_GUARDED(cache->impl.rope_update(qkv, n_q_heads, n_tokens, rope_dims, traditional,
                                       rope_base, rope_scale, position0, q_out,
                                       (hipStream_t)stream));
}

int qw_kv_rope_update_and_attention(qw_kv_cache* cache, const void* qkv, int n_q_heads,
                                    int n_tokens, int rope_dims, int traditional, float rope_base,
                                    float rope_scale, int position0, float scale, int causal,
                                    void* q_out, void* out, void* stream) {
    QW_HANDLE(cache);
    QW_GUARDED(cache->impl.rope_update_and_attention(qkv, n_q_heads, n_tokens, rope_dims,
                                                     traditional, rope_base, rope_scale, position0,
                                                     scale, causal != 0, q_out, out,
                                                     (hipStream_t)stream));
}

}  // extern "C"
