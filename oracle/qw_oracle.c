/*
 * qw_oracle.c - CPU restatement of the reference's full-attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the reported CPU baseline.
 * Nothing in the product links or calls this file.
 *
 * Build: see oracle/Makefile (-O3 -ffp-contract=off; no -ffast-math, the
 * quantizer depends on IEEE division and rintf ties-to-even).
 *
 * Pinning (how each function is checked; tests/test_oracle_*.py):
 *   qwo_f32_to_f16 / qwo_f16_to_f32  pinned: exhaustive round trip of all 65536
 *       halves, numpy float16 casts over random and boundary floats.
 *   qwo_affine_quantize  pinned by hand-derived known answers: grid-aligned
 *       groups, and groups that are not grid-aligned, where the refit
 *       scale = edge / q0 moves the stored fp16 scale (4- and 8-bit,
 *       positive and negative edge, exact .5 ties), the invariants the
 *       algorithm fixes (codes in range, the edge decodes exactly, zero in
 *       range decodes to zero, error <= scale/2), brute force (no other code
 *       is nearer), and a numpy restatement. The tie rounding (rintf:
 *       ties-to-even, as MLX's CPU `quantize` uses std::rint) is the one
 *       point only MLX itself could settle (MLX is not vendored and cannot
 *       run here); the exact ties it decides are counted on the seeded
 *       config data (about 1 value in 2,500 at 4-bit, 1 in 1,450 at 8-bit).
 *   qwo_affine_dequantize  pinned by the closed form on every code of
 *       hand-built groups and by the quantize round trip bound.
 *   qwo_int8_quantize / qwo_int8_dequantize  pinned by the reference's own
 *       known-answer test values (cache.rs:7480-7545: every coordinate within
 *       one step absmax/127 after the round trip, the all-zero token), the
 *       closed form on hand-built rows (the absmax element maps to +-127, the
 *       zero-token scale is 1), and brute force (no other code in [-128, 127]
 *       is nearer to x under the stored scale, up to the fp16 rounding of
 *       x / scale). The tie rule of MLX `round` (rint, ties-to-even) is not
 *       pinned against MLX itself.
 *   qwo_sdpa_mlx_f16  pinned against qwo_sdpa_f64 (closed form, fp64)
 *       within the fp16-rounding budget, against the D-LSA fixtures'
 *       dense_out (short_dense, tiny), and by the known answers of
 *       one-key / equal-key / one-hot softmax.
 *   qwo_sdpa_f64  pinned against numpy fp64 softmax attention and the
 *       fixtures' dense_out.
 *   qwo_dlsa_attention  pinned against the reference's golden fixtures
 *       (tests/golden/, extracted from the tests/fixtures/dlsa safetensors): qwen_layer
 *       real/random attention_out, tiny and short_dense attention_out.
 */
#include "qw_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 */

uint16_t qwo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x0200u : 0u));
    }
    if (ax >= 0x477ff000u) { /* >= 65520 rounds to inf under RNE */
        return (uint16_t)(sign | 0x7c00u);
    }
    const int e = (int)(ax >> 23);
    if (e < 113) { /* below 2^-14: fp16 subnormal or zero, unit 2^-24 */
        if (e == 0) {
            return (uint16_t)sign; /* f32 subnormals are far below 2^-25 */
        }
        const int shift = 126 - e; /* value = sig * 2^(e-150) = (sig >> shift) units */
        if (shift >= 25) {
            return (uint16_t)sign;
        }
        const uint32_t sig = (ax & 0x7fffffu) | 0x800000u;
        uint32_t q = sig >> shift;
        const uint32_t rem = sig & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) {
            q++;
        }
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((uint32_t)(e - 112) << 10) | ((ax & 0x7fffffu) >> 13);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
        h++; /* a carry into the exponent is the correct result */
    }
    return (uint16_t)(sign | h);
}

float qwo_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    const uint32_t m = (uint32_t)h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: m * 2^-24, exact in f32 */
            float f = (float)m * (1.0f / 16777216.0f);
            memcpy(&x, &f, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static float g_f16_table[65536];
static pthread_once_t g_table_once = PTHREAD_ONCE_INIT;
static void build_table(void) {
    for (uint32_t i = 0; i < 65536u; i++) {
        g_f16_table[i] = qwo_f16_to_f32((uint16_t)i);
    }
}
static inline float h2f(uint16_t h) { return g_f16_table[h]; }
static inline float round_f16(float f) { return h2f(qwo_f32_to_f16(f)); }

void qwo_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = qwo_f32_to_f16(in[i]);
}
void qwo_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
    pthread_once(&g_table_once, build_table);
    for (int64_t i = 0; i < n; i++) out[i] = h2f(in[i]);
}

/* ------------------------------------------------------- affine codec (A.1)
 * MLX `quantize(w, group_size, bits)` affine mode, CPU stream, as the
 * reference's weight path calls it (mlx_cxx_bridge.cpp:6347-6393) and as the
 * KV seam names it (batch_quant.rs:109-158: Uniform scheme, group 64).
 * Per group: min/max in f32; the larger-magnitude extreme ("edge") becomes the
 * bias and is rescaled so that it lands exactly on an integer code (q0);
 * codes = rint((w - bias) / scale) clamped to [0, 2^bits - 1]; scale and
 * bias are stored as fp16 (RNE). Codes are packed LSB-first, 32/bits per
 * uint32 word. */
int qwo_affine_quantize(const uint16_t* w, int64_t n_rows, int dim, int group, int bits,
                        uint32_t* codes, uint16_t* scales, uint16_t* biases) {
    if (!w || !codes || !scales || !biases || n_rows < 0) return -1;
    if ((bits != 4 && bits != 8) || group <= 0 || dim <= 0 || dim % group != 0) return -1;
    const int el_per_int = 32 / bits;
    if (group % el_per_int != 0) return -1;
    pthread_once(&g_table_once, build_table);
    const float n_bins = (float)((1 << bits) - 1);
    const float eps = 1e-7f;
    const int64_t n_groups = n_rows * (int64_t)(dim / group);
    const int words_per_group = group / el_per_int;
    for (int64_t g = 0; g < n_groups; g++) {
        const uint16_t* src = w + g * group;
        float w_max = -INFINITY, w_min = INFINITY;
        for (int j = 0; j < group; j++) {
            const float x = h2f(src[j]);
            w_max = w_max < x ? x : w_max; /* std::max(w_max, x) */
            w_min = x < w_min ? x : w_min; /* std::min(w_min, x) */
        }
        const int mask = fabsf(w_min) > fabsf(w_max);
        float scale = (w_max - w_min) / n_bins;
        scale = scale < eps ? eps : scale; /* std::max(range / n_bins, eps) */
        scale = mask ? scale : -scale;
        const float edge = mask ? w_min : w_max;
        const float q0 = rintf(edge / scale);
        float bias = 0.0f;
        if (q0 != 0.0f) {
            scale = edge / q0;
            bias = edge;
        }
        uint32_t* dst = codes + g * words_per_group;
        for (int j = 0; j < words_per_group; j++) {
            uint32_t word = 0;
            for (int kk = 0; kk < el_per_int; kk++) {
                float q = rintf((h2f(src[j * el_per_int + kk]) - bias) / scale);
                q = q < 0.0f ? 0.0f : (q > n_bins ? n_bins : q);
                word |= (uint32_t)q << (kk * bits);
            }
            dst[j] = word;
        }
        scales[g] = qwo_f32_to_f16(scale);
        biases[g] = qwo_f32_to_f16(bias);
    }
    return 0;
}

/* MLX `dequantize` composite on the CPU stream: the codes are unpacked to
 * uint32, multiplied by the fp16 scales (uint32 x float16 promotes to
 * float16, so the product is rounded to fp16), then the fp16 biases are
 * added (rounded to fp16 again). The fp16 arithmetic is restated as an f32
 * operation followed by an RNE cast, which is how MLX's CPU float16 type
 * evaluates it. */
/* cache.rs:270-305 quantize_per_token. MLX evaluates each fp16 op as the
 * fp32 result rounded to fp16 (correctly rounded: 24 >= 2*11 + 2 bits), so:
 * absmax is exact, scale = RN16(absmax / 127), x_div = RN16(x / scale). */
int qwo_int8_quantize(const uint16_t* w, int64_t n_rows, int dim, int8_t* codes,
                      uint16_t* scales) {
    if (!w || !codes || !scales || n_rows < 0 || dim <= 0) return -1;
    pthread_once(&g_table_once, build_table);
    for (int64_t r = 0; r < n_rows; r++) {
        const uint16_t* src = w + r * dim;
        float absmax = 0.0f;
        for (int j = 0; j < dim; j++) {
            const float a = fabsf(h2f(src[j]));
            absmax = absmax < a ? a : absmax;
        }
        uint16_t sh = qwo_f32_to_f16(absmax / 127.0f);
        if (h2f(sh) == 0.0f) sh = qwo_f32_to_f16(1.0f); /* zero-token guard, cache.rs:290-295 */
        const float s = h2f(sh);
        scales[r] = sh;
        for (int j = 0; j < dim; j++) {
            const float x_div = round_f16(h2f(src[j]) / s);
            float c = rintf(x_div);
            c = c < -128.0f ? -128.0f : (c > 127.0f ? 127.0f : c);
            codes[r * dim + j] = (int8_t)c;
        }
    }
    return 0;
}

/* cache.rs:313-316 dequantize: astype(f16) is exact, the multiply rounds. */
int qwo_int8_dequantize(const int8_t* codes, const uint16_t* scales, int64_t n_rows, int dim,
                        uint16_t* out) {
    if (!codes || !scales || !out || n_rows < 0 || dim <= 0) return -1;
    pthread_once(&g_table_once, build_table);
    for (int64_t r = 0; r < n_rows; r++) {
        const float s = h2f(scales[r]);
        for (int j = 0; j < dim; j++)
            out[r * dim + j] = qwo_f32_to_f16((float)codes[r * dim + j] * s);
    }
    return 0;
}

int qwo_affine_dequantize(const uint32_t* codes, const uint16_t* scales,
                          const uint16_t* biases, int64_t n_rows, int dim, int group,
                          int bits, uint16_t* out) {
    if (!codes || !scales || !biases || !out || n_rows < 0) return -1;
    if ((bits != 4 && bits != 8) || group <= 0 || dim <= 0 || dim % group != 0) return -1;
    pthread_once(&g_table_once, build_table);
    const int el_per_int = 32 / bits;
    const uint32_t m = (1u << bits) - 1u;
    const int64_t n = n_rows * (int64_t)dim;
    for (int64_t i = 0; i < n; i++) {
        const uint32_t c = (codes[i / el_per_int] >> ((i % el_per_int) * bits)) & m;
        const float s = h2f(scales[i / group]);
        const float b = h2f(biases[i / group]);
        const float prod = round_f16((float)c * s);
        out[i] = qwo_f32_to_f16(prod + b);
    }
    return 0;
}

/* ------------------------------------------------------- threading helper */

typedef void (*task_fn)(void* ctx, int64_t task);
typedef struct {
    task_fn fn;
    void* ctx;
    int64_t n_tasks;
    int64_t next;
    pthread_mutex_t lock;
} pool_t;

static void* pool_worker(void* arg) {
    pool_t* p = (pool_t*)arg;
    for (;;) {
        pthread_mutex_lock(&p->lock);
        const int64_t t = p->next++;
        pthread_mutex_unlock(&p->lock);
        if (t >= p->n_tasks) break;
        p->fn(p->ctx, t);
    }
    return NULL;
}

static void run_tasks(task_fn fn, void* ctx, int64_t n_tasks, int n_threads) {
    if (n_threads <= 1 || n_tasks <= 1) {
        for (int64_t t = 0; t < n_tasks; t++) fn(ctx, t);
        return;
    }
    if (n_threads > 256) n_threads = 256;
    pool_t p = {fn, ctx, n_tasks, 0, PTHREAD_MUTEX_INITIALIZER};
    pthread_t th[256];
    int started = 0;
    for (int i = 0; i < n_threads - 1; i++) {
        if (pthread_create(&th[i], NULL, pool_worker, &p) == 0) started++;
        else break;
    }
    pool_worker(&p);
    for (int i = 0; i < started; i++) pthread_join(th[i], NULL);
    pthread_mutex_destroy(&p.lock);
}

/* ---------------------------------------------------- MLX SDPA (A.2), fp16
 * MLX's CPU fallback of fast::scaled_dot_product_attention:
 *   q' = f16(f16(scale) * q)
 *   S  = f16(q' . K^T)                       (fp32 accumulation)
 *   masked scores = finfo(float16).min = -65504 (bool mask via `where`)
 *   P  = f16(exp(S - max) * (1 / sum exp))   (precise softmax in fp32)
 *   O  = f16(P . V)                          (fp32 accumulation)
 * GQA: query head h reads KV head h / (hq / hkv). The accumulation order
 * inside a dot product is not MLX's (MLX's CPU GEMM order is unknown); it
 * is 8 interleaved fp32 partial sums, which moves results by fp32 rounding
 * only. */

typedef struct {
    const float* qf; /* [hq, L, D], already f16-rounded and pre-scaled */
    const float* kf; /* [hkv, T, D] */
    const float* vf;
    int64_t k_hs, v_hs; /* head strides in elements */
    int hq, hkv, L, T, D;
    const int32_t* q_pos;
    uint16_t* out; /* [hq, L, D] */
} sdpa_ctx;

static float dot8(const float* a, const float* b, int D) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int d = 0;
    for (; d + 8 <= D; d += 8) {
        for (int i = 0; i < 8; i++) acc[i] += a[d + i] * b[d + i];
    }
    for (; d < D; d++) acc[0] += a[d] * b[d];
    return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

static void sdpa_task(void* vctx, int64_t task) {
    const sdpa_ctx* c = (const sdpa_ctx*)vctx;
    const int h = (int)(task / c->L), r = (int)(task % c->L);
    const int kvh = h / (c->hq / c->hkv);
    const int D = c->D, T = c->T;
    const float* q = c->qf + ((int64_t)h * c->L + r) * D;
    const float* kb = c->kf + (int64_t)kvh * c->k_hs;
    const float* vb = c->vf + (int64_t)kvh * c->v_hs;
    float* s = (float*)malloc(sizeof(float) * (size_t)T);
    float* o = (float*)calloc((size_t)D, sizeof(float));
    const int64_t lim = c->q_pos ? (int64_t)c->q_pos[r] : (int64_t)T - 1;
    float mx = -INFINITY;
    for (int t = 0; t < T; t++) {
        float v = (t <= lim) ? round_f16(dot8(q, kb + (int64_t)t * D, D)) : -65504.0f;
        s[t] = v;
        mx = v > mx ? v : mx;
    }
    float sum = 0.0f;
    for (int t = 0; t < T; t++) sum += expf(s[t] - mx);
    const float norm = 1.0f / sum;
    for (int t = 0; t < T; t++) {
        const float p = round_f16(expf(s[t] - mx) * norm);
        if (p == 0.0f) continue;
        const float* vr = vb + (int64_t)t * D;
        for (int d = 0; d < D; d++) o[d] += p * vr[d];
    }
    uint16_t* dst = c->out + ((int64_t)h * c->L + r) * D;
    for (int d = 0; d < D; d++) dst[d] = qwo_f32_to_f16(o[d]);
    free(s);
    free(o);
}

static int sdpa_mlx_core(const uint16_t* q, const float* kf, const float* vf, int64_t k_hs,
                         int64_t v_hs, int hq, int hkv, int L, int T, int D, float scale,
                         const int32_t* q_pos, uint16_t* out, int n_threads) {
    const float sc = h2f(qwo_f32_to_f16(scale));
    const int64_t nq = (int64_t)hq * L * D;
    float* qf = (float*)malloc(sizeof(float) * (size_t)nq);
    if (!qf) return -1;
    for (int64_t i = 0; i < nq; i++) qf[i] = round_f16(sc * h2f(q[i]));
    sdpa_ctx c = {qf, kf, vf, k_hs, v_hs, hq, hkv, L, T, D, q_pos, out};
    run_tasks(sdpa_task, &c, (int64_t)hq * L, n_threads);
    free(qf);
    return 0;
}

int qwo_sdpa_mlx_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, int hq,
                     int hkv, int L, int T, int D, float scale, const int32_t* q_pos,
                     uint16_t* out, int n_threads) {
    if (!q || !k || !v || !out || hq <= 0 || hkv <= 0 || hq % hkv || L <= 0 || T <= 0 ||
        D <= 0)
        return -1;
    pthread_once(&g_table_once, build_table);
    const int64_t nk = (int64_t)hkv * T * D;
    float* kf = (float*)malloc(sizeof(float) * (size_t)nk);
    float* vf = (float*)malloc(sizeof(float) * (size_t)nk);
    if (!kf || !vf) {
        free(kf);
        free(vf);
        return -1;
    }
    for (int64_t i = 0; i < nk; i++) {
        kf[i] = h2f(k[i]);
        vf[i] = h2f(v[i]);
    }
    int rc = sdpa_mlx_core(q, kf, vf, (int64_t)T * D, (int64_t)T * D, hq, hkv, L, T, D, scale,
                           q_pos, out, n_threads);
    free(kf);
    free(vf);
    return rc;
}

/* ------------------------------------------------------ closed form, fp64 */

typedef struct {
    const uint16_t *q, *k, *v;
    int hq, hkv, L, T, D;
    double scale;
    const int32_t* q_pos;
    double* out;
} f64_ctx;

static void f64_task(void* vctx, int64_t task) {
    const f64_ctx* c = (const f64_ctx*)vctx;
    const int h = (int)(task / c->L), r = (int)(task % c->L);
    const int kvh = h / (c->hq / c->hkv);
    const int D = c->D, T = c->T;
    const uint16_t* q = c->q + ((int64_t)h * c->L + r) * D;
    const int64_t lim = c->q_pos ? (int64_t)c->q_pos[r] : (int64_t)T - 1;
    const int n = (int)(lim + 1 < T ? lim + 1 : T);
    double* s = (double*)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1));
    double* o = (double*)calloc((size_t)D, sizeof(double));
    double mx = -INFINITY;
    for (int t = 0; t < n; t++) {
        const uint16_t* kr = c->k + ((int64_t)kvh * T + t) * D;
        double acc = 0.0;
        for (int d = 0; d < D; d++) acc += (double)h2f(q[d]) * (double)h2f(kr[d]);
        s[t] = acc * c->scale;
        mx = s[t] > mx ? s[t] : mx;
    }
    double sum = 0.0;
    for (int t = 0; t < n; t++) {
        s[t] = exp(s[t] - mx);
        sum += s[t];
    }
    for (int t = 0; t < n; t++) {
        const uint16_t* vr = c->v + ((int64_t)kvh * T + t) * D;
        const double p = s[t] / sum;
        for (int d = 0; d < D; d++) o[d] += p * (double)h2f(vr[d]);
    }
    memcpy(c->out + ((int64_t)h * c->L + r) * D, o, sizeof(double) * (size_t)D);
    free(s);
    free(o);
}

int qwo_sdpa_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v, int hq, int hkv,
                 int L, int T, int D, double scale, const int32_t* q_pos, double* out,
                 int n_threads) {
    if (!q || !k || !v || !out || hq <= 0 || hkv <= 0 || hq % hkv || L <= 0 || T <= 0 ||
        D <= 0)
        return -1;
    pthread_once(&g_table_once, build_table);
    f64_ctx c = {q, k, v, hq, hkv, L, T, D, scale, q_pos, out};
    run_tasks(f64_task, &c, (int64_t)hq * L, n_threads);
    return 0;
}

/* ----------------------------------------------------- D-LSA read (A.3)
 * K2 contract (mlx_cxx_dlsa_attention.cpp:1-31, dlsa_attention.rs:1-14):
 * row r of every head of KV group g reads keys lists[r, 0:lengths[r]]; list
 * order is irrelevant; entries outside [0, T) are skipped; a row with no
 * valid entry is all zeros. Softmax over scale * q.k and the weighted sum of
 * V, here in double. */

typedef struct {
    const uint16_t *q, *k, *v;
    int64_t khs, krs, vhs, vrs;
    const int32_t *lists, *lengths;
    int L, W, hq, hkv, D, T;
    double scale;
    float* out;
} dlsa_ctx;

static void dlsa_task(void* vctx, int64_t task) {
    const dlsa_ctx* c = (const dlsa_ctx*)vctx;
    const int h = (int)(task / c->L), r = (int)(task % c->L);
    const int kvh = h / (c->hq / c->hkv);
    const int D = c->D;
    const uint16_t* q = c->q + ((int64_t)h * c->L + r) * D;
    int len = c->lengths[r];
    if (len > c->W) len = c->W;
    double* s = (double*)malloc(sizeof(double) * (size_t)(len > 0 ? len : 1));
    int32_t* keys = (int32_t*)malloc(sizeof(int32_t) * (size_t)(len > 0 ? len : 1));
    double* o = (double*)calloc((size_t)D, sizeof(double));
    int n = 0;
    double mx = -INFINITY;
    for (int i = 0; i < len; i++) {
        const int32_t p = c->lists[(int64_t)r * c->W + i];
        if (p < 0 || p >= c->T) continue;
        const uint16_t* kr = c->k + (int64_t)kvh * c->khs + (int64_t)p * c->krs;
        double acc = 0.0;
        for (int d = 0; d < D; d++) acc += (double)h2f(q[d]) * (double)h2f(kr[d]);
        s[n] = acc * c->scale;
        keys[n] = p;
        mx = s[n] > mx ? s[n] : mx;
        n++;
    }
    float* dst = c->out + ((int64_t)h * c->L + r) * D;
    if (n == 0) {
        for (int d = 0; d < D; d++) dst[d] = 0.0f;
    } else {
        double sum = 0.0;
        for (int i = 0; i < n; i++) {
            s[i] = exp(s[i] - mx);
            sum += s[i];
        }
        for (int i = 0; i < n; i++) {
            const uint16_t* vr = c->v + (int64_t)kvh * c->vhs + (int64_t)keys[i] * c->vrs;
            const double p = s[i] / sum;
            for (int d = 0; d < D; d++) o[d] += p * (double)h2f(vr[d]);
        }
        for (int d = 0; d < D; d++) dst[d] = (float)o[d];
    }
    free(s);
    free(keys);
    free(o);
}

int qwo_dlsa_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                       int64_t k_head_stride, int64_t k_row_stride, int64_t v_head_stride,
                       int64_t v_row_stride, const int32_t* lists, const int32_t* lengths,
                       int L, int W, int hq, int hkv, int D, int T, float scale, float* out,
                       int n_threads) {
    if (!q || !k || !v || !lists || !lengths || !out || hq <= 0 || hkv <= 0 || hq % hkv ||
        L <= 0 || W <= 0 || D <= 0 || T <= 0)
        return -1;
    pthread_once(&g_table_once, build_table);
    dlsa_ctx c = {q,     k,      v, k_head_stride, k_row_stride, v_head_stride, v_row_stride,
                  lists, lengths, L, W,             hq,           hkv,           D,
                  T,     (double)scale, out};
    run_tasks(dlsa_task, &c, (int64_t)hq * L, n_threads);
    return 0;
}

/* ------------------------------------------- quantized layer call (c1-c4)
 * The reference's quantized-cache layer call (cache.rs:3495-3510, :3520,
 * :2709-2723): `update` quantizes and appends the new rows first, then the
 * whole visible cache is dequantized and attended by MLX SDPA, so new rows
 * are attended in their dequantized form. */

typedef struct {
    uint32_t *kc, *vc;
    uint16_t *ks, *kb, *vs, *vb;
    int64_t cap;
    int T, D, group, bits, chunks;
    float *kf, *vf;
} deq_ctx;

/* One task = one (head, row chunk) of K and V. */
static void deq_task(void* vctx, int64_t task) {
    const deq_ctx* c = (const deq_ctx*)vctx;
    const int64_t h = task / c->chunks, ch = task % c->chunks;
    const int wpr = c->D * c->bits / 32, gpr = c->D / c->group;
    const int64_t r0 = (int64_t)c->T * ch / c->chunks, r1 = (int64_t)c->T * (ch + 1) / c->chunks;
    const int64_t nr = r1 - r0;
    if (nr <= 0) return;
    const int64_t n = nr * c->D;
    uint16_t* tmp = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)n);
    const int64_t row = h * c->cap + r0;
    const int64_t dst = (h * (int64_t)c->T + r0) * c->D;
    qwo_affine_dequantize(c->kc + row * wpr, c->ks + row * gpr, c->kb + row * gpr, nr, c->D,
                          c->group, c->bits, tmp);
    for (int64_t i = 0; i < n; i++) c->kf[dst + i] = h2f(tmp[i]);
    qwo_affine_dequantize(c->vc + row * wpr, c->vs + row * gpr, c->vb + row * gpr, nr, c->D,
                          c->group, c->bits, tmp);
    for (int64_t i = 0; i < n; i++) c->vf[dst + i] = h2f(tmp[i]);
    free(tmp);
}

int qwo_affine_layer_call(uint32_t* k_codes, uint16_t* k_scales, uint16_t* k_biases,
                          uint32_t* v_codes, uint16_t* v_scales, uint16_t* v_biases,
                          int64_t cap, int t_old, const uint16_t* q, const uint16_t* k_new,
                          const uint16_t* v_new, int hq, int hkv, int L, int D, int group,
                          int bits, float scale, int causal, const int32_t* sel, int n_sel,
                          uint16_t* out, int n_threads) {
    if (!k_codes || !k_scales || !k_biases || !v_codes || !v_scales || !v_biases || !q ||
        !k_new || !v_new || !out || hq <= 0 || hkv <= 0 || hq % hkv || L <= 0 || t_old < 0 ||
        (int64_t)t_old + L > cap || (bits != 4 && bits != 8) || D % group)
        return -1;
    pthread_once(&g_table_once, build_table);
    const int wpr = D * bits / 32, gpr = D / group;
    const int T = t_old + L;
    for (int h = 0; h < hkv; h++) { /* quantize-on-append */
        const int64_t row0 = (int64_t)h * cap + t_old;
        if (qwo_affine_quantize(k_new + (int64_t)h * L * D, L, D, group, bits,
                                k_codes + row0 * wpr, k_scales + row0 * gpr,
                                k_biases + row0 * gpr) ||
            qwo_affine_quantize(v_new + (int64_t)h * L * D, L, D, group, bits,
                                v_codes + row0 * wpr, v_scales + row0 * gpr,
                                v_biases + row0 * gpr))
            return -1;
    }
    const int64_t n = (int64_t)hkv * T * D;
    float* kf = (float*)malloc(sizeof(float) * (size_t)n);
    float* vf = (float*)malloc(sizeof(float) * (size_t)n);
    if (!kf || !vf) {
        free(kf);
        free(vf);
        return -1;
    }
    const int chunks = n_threads > 1 ? 4 * n_threads : 1;
    deq_ctx dc = {k_codes, v_codes, k_scales, k_biases, v_scales, v_biases, cap, T, D,
                  group,   bits,    chunks,   kf,       vf};
    run_tasks(deq_task, &dc, (int64_t)hkv * chunks, n_threads);
    /* Select the query rows; bottom-right causal position of row r is
     * T - L + r. */
    const int nrows = n_sel > 0 ? n_sel : L;
    uint16_t* qs = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)hq * nrows * D);
    int32_t* pos = (int32_t*)malloc(sizeof(int32_t) * (size_t)nrows);
    int rc = 0;
    if (!qs || !pos) {
        rc = -1;
    } else {
        for (int i = 0; i < nrows; i++) {
            const int r = n_sel > 0 ? sel[i] : i;
            if (r < 0 || r >= L) {
                rc = -1;
                break;
            }
            pos[i] = T - L + r;
            for (int h = 0; h < hq; h++)
                memcpy(qs + ((int64_t)h * nrows + i) * D, q + ((int64_t)h * L + r) * D,
                       sizeof(uint16_t) * (size_t)D);
        }
        if (rc == 0)
            rc = sdpa_mlx_core(qs, kf, vf, (int64_t)T * D, (int64_t)T * D, hq, hkv, nrows, T,
                               D, scale, causal ? pos : NULL, out, n_threads);
    }
    free(qs);
    free(pos);
    free(kf);
    free(vf);
    return rc;
}
