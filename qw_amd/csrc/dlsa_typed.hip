// dlsa_typed.hip - the D-LSA gathered read (K2) for every dtype pair and head
// dim the reference accepts (q f16 / bf16 / f32, K and V alike in one of the
// three, head_dim 32 / 64 / 128 / 256, at most 8 query heads a KV head;
// mlx_cxx_dlsa_attention.cpp:429-470), in fp32 arithmetic.
//
// Reference contract (crates/mlxcel-core/src/dlsa_attention.rs:1-14): every
// query row attends over the cached keys of its own list; entries outside
// [0, n_keys) are skipped; a row without a valid entry is zeros; the output
// has q's dtype. The reference's f32 test holds the result to 1e-5 of an f64
// host softmax (dlsa_attention.rs:213-255), so nothing here rounds below
// fp32: q, K and V are widened to fp32 on load (bf16 and fp16 exactly), the
// dot products, the online softmax (fp32 exp) and P.V accumulate in fp32, and
// only the final row is rounded to the output dtype.
//
// fp16 q with fp16 K/V at head_dim 64..256 is not served here: it takes the
// MFMA kernel of dlsa.hip (the served path), bit for bit what
// qw_dlsa_sparse_attention returns.
//
// Layout of the work: grid (parts, rows, kv heads), NW waves (the reference's
// simdgroups knob, 1..16; at most 8 at head_dim 256). A list entry is handled by LPE = min(64, D) lanes
// (DPL = D / LPE dims each), so a wave takes 64 / LPE entries a step; the
// sub-waves run independent online softmaxes for the G heads of the group and
// are merged through LDS at the end, head by head. With parts > 1 each
// workgroup takes a contiguous share of the list and writes an fp32 partial
// (m, l, unnormalized O); a merge kernel combines the parts.
#include <algorithm>
#include <map>
#include <mutex>
#include <string>

#include "kv_cache.hpp"
#include "qw_common.hpp"

namespace qw {

namespace {

typedef uint16_t bf16_bits;

template <int DT>
struct DType;
template <>
struct DType<QW_DTYPE_F16> {
    typedef _Float16 T;
    __device__ static float load(const T* p) { return (float)*p; }
    __device__ static void store(T* p, float x) { *p = (T)x; }
};
template <>
struct DType<QW_DTYPE_BF16> {
    typedef bf16_bits T;
    __device__ static float load(const T* p) { return __uint_as_float((uint32_t)*p << 16); }
    // round to nearest even; NaN stays NaN
    __device__ static void store(T* p, float x) {
        const uint32_t u = __float_as_uint(x);
        if ((u & 0x7FFFFFFFu) > 0x7F800000u) {
            *p = (T)((u >> 16) | 0x40u);
            return;
        }
        *p = (T)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
    }
};
template <>
struct DType<QW_DTYPE_F32> {
    typedef float T;
    __device__ static float load(const T* p) { return *p; }
    __device__ static void store(T* p, float x) { *p = x; }
};

constexpr int kTypedGMax = 8;
constexpr int kTypedMaxParts = 128;

struct TypedArgs {
    const void* q;  // [hq][L][D], q dtype
    const void* k;  // element (h, t, d) at h * khs + t * krs + d, kv dtype
    const void* v;
    int64_t khs, krs, vhs, vrs;
    const int32_t* lists;    // [L][W]
    const int32_t* lengths;  // [L]
    void* out;               // [hq][L][D], q dtype (parts == 1)
    float* part_o;           // [parts][L][hq][D] (parts > 1)
    float2* part_ml;         // [parts][L][hq]
    int L, W, hq, G, T, parts;
    float scale;
};

// Waves a workgroup at most: 16 (the reference's simdgroups range), 8 at
// head_dim 256, where a lane's fp32 q, O and softmax state for 8 heads need
// more than the 128 registers a 16-wave workgroup leaves.
template <int D>
constexpr int typed_max_waves() {
    return D == 256 ? 8 : 16;
}

template <int DQ, int DKV, int D>
__global__ __launch_bounds__(64 * typed_max_waves<D>()) void dlsa_typed_kernel(TypedArgs a) {
    using TQ = typename DType<DQ>::T;
    using TKV = typename DType<DKV>::T;
    constexpr int LPE = D < 64 ? D : 64;  // lanes an entry
    constexpr int EPW = 64 / LPE;         // entries a wave step
    constexpr int DPL = D / LPE;          // dims a lane
    const int part = blockIdx.x, row = blockIdx.y, h = blockIdx.z;
    const int NW = blockDim.x >> 6, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int sub = lane / LPE, sl = lane % LPE;
    const int G = a.G;
    const int len = max(0, min(a.lengths[row], a.W));
    const int chunk = (len + a.parts - 1) / a.parts;
    const int e0 = part * chunk, e1 = min(len, e0 + chunk);

    // q rows of the group, widened and scaled
    float qv[kTypedGMax][DPL];
#pragma unroll
    for (int g = 0; g < kTypedGMax; g++)
#pragma unroll
        for (int j = 0; j < DPL; j++)
        {
            const int gg = g < G ? g : 0;  // in bounds for every g
            const float x =
                DType<DQ>::load((const TQ*)a.q + ((int64_t)(h * G + gg) * a.L + row) * D + sl * DPL + j);
            qv[g][j] = g < G ? x * a.scale : 0.0f;
        }
    float m[kTypedGMax], l[kTypedGMax], o[kTypedGMax][DPL];
#pragma unroll
    for (int g = 0; g < kTypedGMax; g++) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int j = 0; j < DPL; j++) o[g][j] = 0.0f;
    }
    const TKV* kh = (const TKV*)a.k + (int64_t)h * a.khs + sl * DPL;
    const TKV* vh = (const TKV*)a.v + (int64_t)h * a.vhs + sl * DPL;
    const int32_t* list = a.lists + (int64_t)row * a.W;
    // every lane runs every step (the shuffles stay within the sub-wave):
    // an entry past the share or outside [0, T) scores -inf
    for (int eb = e0; eb < e1; eb += NW * EPW) {
        const int e = eb + wave * EPW + sub;
        const int key = e < e1 ? list[e] : -1;
        const bool ok = key >= 0 && key < a.T;
        const int kk = ok ? key : 0;
        float kv[DPL], vv[DPL];
#pragma unroll
        for (int j = 0; j < DPL; j++) {
            kv[j] = DType<DKV>::load(kh + (int64_t)kk * a.krs + j);
            vv[j] = DType<DKV>::load(vh + (int64_t)kk * a.vrs + j);
        }
#pragma unroll
        for (int g = 0; g < kTypedGMax; g++) {
            if (g >= G) break;  // uniform
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < DPL; j++) s = __builtin_fmaf(qv[g][j], kv[j], s);
#pragma unroll
            for (int x = 1; x < LPE; x <<= 1) s += __shfl_xor(s, x);
            s = ok ? s : -INFINITY;
            const float mn = fmaxf(m[g], s);
            if (mn != -INFINITY) {
                const float alpha = expf(m[g] - mn);  // m = -inf: 0
                const float p = expf(s - mn);
                l[g] = __builtin_fmaf(l[g], alpha, p);
#pragma unroll
                for (int j = 0; j < DPL; j++) o[g][j] = __builtin_fmaf(o[g][j], alpha, p * vv[j]);
                m[g] = mn;
            }
        }
    }

    // merge the NW * EPW sub-waves, head by head: sub-wave u posts (m, l)
    // and its O row; thread d combines dim d
    const int NSUB = NW * EPW, u = wave * EPW + sub;
    __shared__ float2 sm_ml[64];
    __shared__ float sm_o[16 * 2][D];  // NSUB <= 32 (16 waves x 2 at D = 32)
    for (int g = 0; g < G; g++) {
        if (sl == 0) sm_ml[u] = float2{m[g], l[g]};
#pragma unroll
        for (int j = 0; j < DPL; j++) sm_o[u][sl * DPL + j] = o[g][j];
        __syncthreads();
        for (int d = threadIdx.x; d < D; d += blockDim.x) {
            float M = -INFINITY;
            for (int w = 0; w < NSUB; w++) M = fmaxf(M, sm_ml[w].x);
            float acc = 0.0f, Ls = 0.0f;
            if (M != -INFINITY) {
                for (int w = 0; w < NSUB; w++) {
                    const float f = expf(sm_ml[w].x - M);  // m = -inf: 0
                    acc = __builtin_fmaf(f, sm_o[w][d], acc);
                    Ls = __builtin_fmaf(f, sm_ml[w].y, Ls);
                }
            }
            const int hh = h * G + g;
            if (a.parts == 1) {
                DType<DQ>::store((TQ*)a.out + ((int64_t)hh * a.L + row) * D + d, Ls > 0.0f ? acc / Ls : 0.0f);
            } else {
                const int64_t pr = ((int64_t)part * a.L + row) * a.hq + hh;
                a.part_o[pr * D + d] = acc;
                if (d == 0) a.part_ml[pr] = float2{M, Ls};
            }
        }
        __syncthreads();
    }
}

// out[hh][row][d] = sum_p e^(m_p - M) O_p[d] / sum_p e^(m_p - M) l_p, in q's
// dtype (0 when no part saw a valid entry). grid (hq, L), D threads.
template <int DQ>
__global__ __launch_bounds__(256) void dlsa_typed_merge_kernel(const float* __restrict__ part_o,
                                                               const float2* __restrict__ part_ml,
                                                               int parts, int L, int hq, int D,
                                                               void* out) {
    using TQ = typename DType<DQ>::T;
    const int hh = blockIdx.x, row = blockIdx.y, d = threadIdx.x;
    if (d >= D) return;
    float M = -INFINITY;
    for (int p = 0; p < parts; p++) M = fmaxf(M, part_ml[((int64_t)p * L + row) * hq + hh].x);
    float acc = 0.0f, Ls = 0.0f;
    if (M != -INFINITY) {
        for (int p = 0; p < parts; p++) {
            const int64_t pr = ((int64_t)p * L + row) * hq + hh;
            const float2 ml = part_ml[pr];
            const float f = expf(ml.x - M);
            acc = __builtin_fmaf(f, part_o[pr * D + d], acc);
            Ls = __builtin_fmaf(f, ml.y, Ls);
        }
    }
    DType<DQ>::store((TQ*)out + ((int64_t)hh * L + row) * D + d, Ls > 0.0f ? acc / Ls : 0.0f);
}

template <int DQ, int DKV>
static void launch_typed_dq_dkv(const TypedArgs& a, int D, dim3 grid, int nw, hipStream_t stream) {
    const dim3 block(64 * (D == 256 ? std::min(nw, typed_max_waves<256>()) : nw));
    switch (D) {
        case 32: hipLaunchKernelGGL((dlsa_typed_kernel<DQ, DKV, 32>), grid, block, 0, stream, a); break;
        case 64: hipLaunchKernelGGL((dlsa_typed_kernel<DQ, DKV, 64>), grid, block, 0, stream, a); break;
        case 128: hipLaunchKernelGGL((dlsa_typed_kernel<DQ, DKV, 128>), grid, block, 0, stream, a); break;
        default: hipLaunchKernelGGL((dlsa_typed_kernel<DQ, DKV, 256>), grid, block, 0, stream, a);
    }
}

template <int DQ>
static void launch_typed_dq(const TypedArgs& a, int kv_dtype, int D, dim3 grid, int nw,
                            hipStream_t stream) {
    if (kv_dtype == QW_DTYPE_F16)
        launch_typed_dq_dkv<DQ, QW_DTYPE_F16>(a, D, grid, nw, stream);
    else if (kv_dtype == QW_DTYPE_BF16)
        launch_typed_dq_dkv<DQ, QW_DTYPE_BF16>(a, D, grid, nw, stream);
    else
        launch_typed_dq_dkv<DQ, QW_DTYPE_F32>(a, D, grid, nw, stream);
}

// Split-K workspace of the typed calls, one per (device, stream).
static std::mutex g_typed_mu;
static std::map<std::pair<int, hipStream_t>, GrowBuffer> g_typed_ws;

size_t dtype_size(int dt) { return dt == QW_DTYPE_F32 ? 4 : 2; }

}  // namespace

int dlsa_sparse_attention_typed(const void* q, int q_dtype, const void* k, const void* v,
                                int kv_dtype, int64_t khs, int64_t krs, int64_t vhs, int64_t vrs,
                                const int32_t* lists, const int32_t* lengths, int n_rows,
                                int width, int n_q_heads, int n_kv_heads, int head_dim,
                                int n_keys, float scale, int parts, int waves, void* out,
                                hipStream_t stream) {
    QW_REQUIRE(q && k && v && lists && lengths && out, QW_ERR_INVALID_ARGUMENT,
               "dlsa_sparse_attention_typed: null pointer");
    auto dtype_ok = [](int dt) {
        return dt == QW_DTYPE_F16 || dt == QW_DTYPE_BF16 || dt == QW_DTYPE_F32;
    };
    QW_REQUIRE(dtype_ok(q_dtype) && dtype_ok(kv_dtype), QW_ERR_INVALID_ARGUMENT,
               "dlsa_sparse_attention_typed: q/k/v must be f16/bf16/f32, k and v alike");
    QW_REQUIRE(n_kv_heads > 0 && n_q_heads > 0 && n_q_heads % n_kv_heads == 0 && n_keys > 0 &&
                   n_rows > 0,
               QW_ERR_INVALID_ARGUMENT, "dlsa_sparse_attention_typed: bad head or length geometry");
    const int G = n_q_heads / n_kv_heads;
    QW_REQUIRE(G <= kTypedGMax, QW_ERR_INVALID_ARGUMENT,
               "dlsa_sparse_attention_typed: at most 8 query heads per KV head");
    QW_REQUIRE(head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256,
               QW_ERR_INVALID_ARGUMENT,
               "dlsa_sparse_attention_typed: head dim must be 32, 64, 128 or 256");
    QW_REQUIRE(width > 0, QW_ERR_INVALID_ARGUMENT, "dlsa_sparse_attention_typed: empty list width");
    QW_REQUIRE(parts >= 0 && waves >= 0 && waves <= 16, QW_ERR_INVALID_ARGUMENT,
               "dlsa_sparse_attention_typed: bad launch knobs");
    // the served fp16 path, unchanged
    if (q_dtype == QW_DTYPE_F16 && kv_dtype == QW_DTYPE_F16 && head_dim >= 64)
        return dlsa_sparse_attention(q, k, v, khs, krs, vhs, vrs, lists, lengths, n_rows, width,
                                     n_q_heads, n_kv_heads, head_dim, n_keys, scale, parts, waves,
                                     out, stream);
    const size_t es = dtype_size(kv_dtype);
    QW_REQUIRE((uintptr_t)q % dtype_size(q_dtype) == 0 && (uintptr_t)k % es == 0 &&
                   (uintptr_t)v % es == 0 && (uintptr_t)out % dtype_size(q_dtype) == 0,
               QW_ERR_UNSUPPORTED, "dlsa_sparse_attention_typed: misaligned pointer");
    if (parts <= 0) {
        // the reference's policy shape (mlx_cxx_dlsa_attention.cpp:379-400): one pass when
        // the rows and KV heads alone give enough workgroups, else split each list
        const int units = n_rows * n_kv_heads;
        parts = units >= 192 ? 1 : std::min(kTypedMaxParts, std::max(1, std::min(192 / units, width / 16)));
    }
    parts = std::max(1, std::min(parts, kTypedMaxParts));
    const int nw = waves > 0 ? waves : 4;
    int dev = 0;
    QW_HIP_CHECK(hipGetDevice(&dev));
    TypedArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.khs = khs;
    a.krs = krs;
    a.vhs = vhs;
    a.vrs = vrs;
    a.lists = lists;
    a.lengths = lengths;
    a.out = out;
    a.part_o = nullptr;
    a.part_ml = nullptr;
    a.L = n_rows;
    a.W = width;
    a.hq = n_q_heads;
    a.G = G;
    a.T = n_keys;
    a.parts = parts;
    a.scale = scale;
    if (parts > 1) {
        const size_t no = (size_t)parts * n_rows * n_q_heads;
        void* ws = nullptr;
        {
            std::lock_guard<std::mutex> lock(g_typed_mu);
            GrowBuffer& b = g_typed_ws[{dev, stream}];
            b.stream_owned = true;
            int rc = b.get(no * head_dim * sizeof(float) + no * sizeof(float2), stream, &ws);
            if (rc) return rc;
        }
        a.part_o = (float*)ws;
        a.part_ml = (float2*)((char*)ws + no * head_dim * sizeof(float));
    }
    const dim3 grid(parts, n_rows, n_kv_heads);
    if (q_dtype == QW_DTYPE_F16)
        launch_typed_dq<QW_DTYPE_F16>(a, kv_dtype, head_dim, grid, nw, stream);
    else if (q_dtype == QW_DTYPE_BF16)
        launch_typed_dq<QW_DTYPE_BF16>(a, kv_dtype, head_dim, grid, nw, stream);
    else
        launch_typed_dq<QW_DTYPE_F32>(a, kv_dtype, head_dim, grid, nw, stream);
    QW_HIP_CHECK(hipGetLastError());
    if (parts > 1) {
        const dim3 mg(n_q_heads, n_rows), mb(head_dim);
        if (q_dtype == QW_DTYPE_F16)
            hipLaunchKernelGGL(dlsa_typed_merge_kernel<QW_DTYPE_F16>, mg, mb, 0, stream, a.part_o,
                               a.part_ml, parts, n_rows, n_q_heads, head_dim, out);
        else if (q_dtype == QW_DTYPE_BF16)
            hipLaunchKernelGGL(dlsa_typed_merge_kernel<QW_DTYPE_BF16>, mg, mb, 0, stream, a.part_o,
                               a.part_ml, parts, n_rows, n_q_heads, head_dim, out);
        else
            hipLaunchKernelGGL(dlsa_typed_merge_kernel<QW_DTYPE_F32>, mg, mb, 0, stream, a.part_o,
                               a.part_ml, parts, n_rows, n_q_heads, head_dim, out);
        QW_HIP_CHECK(hipGetLastError());
    }
    return QW_OK;
}

}  // namespace qw
