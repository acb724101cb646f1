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

#include "kv_cache.hpp"

namespace qw {

struct DlsaArgs {
    const f16* q;
    const f16* k;
    const f16* v;
    int64_t khs, krs, vhs, vrs;
    const int32_t* lists;
    const int32_t* lengths;
    f16* out;
    float* part_o;   // [L][Hq][parts][D]
    float2* part_ml; // [L][Hq][parts]
    int L, W, hq, hkv, G, T, parts;
    float scale2;    // scale * log2(e)
};

constexpr int kDlsaNT = 2;  // tiles per batch a wave keeps in flight

template <int D, int GMAX>
__global__ __launch_bounds__(256, 2) void dlsa_kernel(DlsaArgs a) {
    constexpr int NM = D / 32;
    constexpr int NP = D / 64;  // 64-dim groups: P.V output tiles (p, c), c < 4
    const int part = blockIdx.x, r = blockIdx.y, h = blockIdx.z;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, g = lane >> 4;
    const int G = a.G;
    int len = a.lengths[r];
    len = len < 0 ? 0 : (len > a.W ? a.W : len);
    const int e_begin = (int)((int64_t)len * part / a.parts);
    const int e_end = (int)((int64_t)len * (part + 1) / a.parts);
    const int32_t* list = a.lists + (int64_t)r * a.W;

    // Q operand: column r16 = head h*G + r16 (zero past G), dims 32m + 8g..+7.
    half8 qop[NM];
    {
        const bool ok = r16 < G;
        const f16* qrow = a.q + ((int64_t)(h * G + (ok ? r16 : 0)) * a.L + r) * D;
#pragma unroll
        for (int m = 0; m < NM; m++) qop[m] = ok ? *(const half8*)(qrow + 32 * m + 8 * g) : half8{};
    }

    // P.V on MFMA (v_mfma_f32_16x16x16_f16, K = the tile's 16 entries): A = P
    // (row = head r16, entries 4g..4g+3: exactly where the S^T tile leaves
    // them), B = V (entries 4g..4g+3 of one dim), gathered as 8-byte row
    // pieces: lane (g, r16) loads dims 64p + 4 r16 .. +3 of entries 4g + j.
    // Output tile (p, c) holds heads 4g + i x dims 64p + 4 r16 + c. P enters
    // as an fp16 high part and an fp16 remainder, so p * v is exact and the
    // sums stay fp32 as in the reference.
    float mrun = -INFINITY;  // running max (log2 domain), column r16
    float lrun = 0.0f;       // running sum, this lane's share
    float4v acc[NP][4];
#pragma unroll
    for (int pp = 0; pp < NP; pp++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[pp][c] = float4v{0.f, 0.f, 0.f, 0.f};

    const int n_tiles = (e_end - e_begin + 15) / 16;
    for (int t0 = wave; t0 < n_tiles; t0 += 4 * kDlsaNT) {
        // ---- gather loads for up to NT tiles
        u32x4 kc[kDlsaNT][NM];
        u32x2 vq[kDlsaNT][4][NP];
        int key_a[kDlsaNT];  // the key of list entry tile*16 + r16 (A-operand row)
        bool ok_a[kDlsaNT];
#pragma unroll
        for (int b = 0; b < kDlsaNT; b++) {
            const int tile = t0 + 4 * b;
            const int e = e_begin + 16 * tile + r16;
            int key = -1;
            if (tile < n_tiles && e < e_end) key = list[e];
            ok_a[b] = key >= 0 && key < a.T;
            key_a[b] = ok_a[b] ? key : 0;
            const u32x4* krow = (const u32x4*)(a.k + h * a.khs + (int64_t)key_a[b] * a.krs);
#pragma unroll
            for (int m = 0; m < NM; m++) kc[b][m] = krow[4 * m + g];
        }
#pragma unroll
        for (int b = 0; b < kDlsaNT; b++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                // entry 4g + j's key sits in lane 4g + j (lane r16 holds entry r16)
                const int key = __shfl(key_a[b], 4 * g + j);
                const f16* vrow = a.v + h * a.vhs + (int64_t)key * a.vrs + 4 * r16;
#pragma unroll
                for (int pp = 0; pp < NP; pp++) vq[b][j][pp] = *(const u32x2*)(vrow + 64 * pp);
            }
        }
        // ---- scores: S^T tile, lane holds entries 4g+i for head r16
        float s[kDlsaNT][4];
        float bmax = -INFINITY;
#pragma unroll
        for (int b = 0; b < kDlsaNT; b++) {
            float4v sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int m = 0; m < NM; m++)
                sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(kc[b][m]), qop[m], sacc, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const bool ok = __shfl(ok_a[b] ? 1 : 0, 4 * g + i) != 0 && r16 < G;
                s[b][i] = ok ? sacc[i] * a.scale2 : -INFINITY;
                bmax = fmaxf(bmax, s[b][i]);
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
        for (int b = 0; b < kDlsaNT; b++) {
            half4v ph, pl;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float pv = __builtin_amdgcn_exp2f(s[b][i] - mref);
                lrun += pv;
                ph[i] = (f16)pv;
                pl[i] = (f16)(pv - (float)ph[i]);
            }
#pragma unroll
            for (int pp = 0; pp < NP; pp++) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    // element c of the four entries' 4-dim pieces
                    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
                    uint32_t w0, w1;
                    if (c < 2) {
                        w0 = __builtin_amdgcn_perm(vq[b][1][pp].x, vq[b][0][pp].x, sel);
                        w1 = __builtin_amdgcn_perm(vq[b][3][pp].x, vq[b][2][pp].x, sel);
                    } else {
                        w0 = __builtin_amdgcn_perm(vq[b][1][pp].y, vq[b][0][pp].y, sel);
                        w1 = __builtin_amdgcn_perm(vq[b][3][pp].y, vq[b][2][pp].y, sel);
                    }
                    const half4v vb = __builtin_bit_cast(half4v, u32x2{w0, w1});
                    acc[pp][c] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, vb, acc[pp][c], 0, 0, 0);
                    acc[pp][c] = __builtin_amdgcn_mfma_f32_16x16x16f16(pl, vb, acc[pp][c], 0, 0, 0);
                }
            }
        }
    }
    lrun += __shfl_xor(lrun, 16);
    lrun += __shfl_xor(lrun, 32);

    // ---- merge the waves: (m, l) per head, then the accumulators
    __shared__ float2 sm_ml[4][16];
    __shared__ float4v sm_acc[2][GMAX][D / 4];
    if (g == 0) sm_ml[wave][r16] = float2{mrun, lrun};
    __syncthreads();
    float Mi[4], Li[4];  // heads 4g + i
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int hd = 4 * g + i;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++) M = fmaxf(M, sm_ml[w][hd].x);
        float L = 0.0f, own = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float mw = sm_ml[w][hd].x;
            const float f = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
            L += f * sm_ml[w][hd].y;
            if (w == wave) own = f;
        }
        Mi[i] = M;
        Li[i] = L;
#pragma unroll
        for (int pp = 0; pp < NP; pp++)
#pragma unroll
            for (int c = 0; c < 4; c++) acc[pp][c][i] *= own;
    }
    // head 4g + i, dims 64p + 4 r16 .. +3 as one float4
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int hd = 4 * g + i;
            if (hd < G && hd < GMAX)
#pragma unroll
                for (int pp = 0; pp < NP; pp++)
                    sm_acc[buf][hd][16 * pp + r16] =
                        float4v{acc[pp][0][i], acc[pp][1][i], acc[pp][2][i], acc[pp][3][i]};
        }
    };
    auto add = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int hd = 4 * g + i;
            if (hd < G && hd < GMAX)
#pragma unroll
                for (int pp = 0; pp < NP; pp++) {
                    const float4v o = sm_acc[buf][hd][16 * pp + r16];
#pragma unroll
                    for (int c = 0; c < 4; c++) acc[pp][c][i] += o[c];
                }
        }
    };
    if (wave >= 2) store(wave - 2);
    __syncthreads();
    if (wave < 2) add(wave);
    __syncthreads();
    if (wave == 1) store(0);
    __syncthreads();
    if (wave != 0) return;
    add(0);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int hd = 4 * g + i;
        if (hd >= G) continue;
        const int qh = h * G + hd;
        if (a.parts == 1) {
            const float inv = Li[i] > 0.0f ? 1.0f / Li[i] : 0.0f;
            f16* dst = a.out + ((int64_t)qh * a.L + r) * D + 4 * r16;
#pragma unroll
            for (int pp = 0; pp < NP; pp++) {
                const half4v o = {(f16)(acc[pp][0][i] * inv), (f16)(acc[pp][1][i] * inv),
                                  (f16)(acc[pp][2][i] * inv), (f16)(acc[pp][3][i] * inv)};
                *(half4v*)(dst + 64 * pp) = o;
            }
        } else {
            const int64_t pr = ((int64_t)r * a.hq + qh) * a.parts + part;
            float* dst = a.part_o + pr * D + 4 * r16;
#pragma unroll
            for (int pp = 0; pp < NP; pp++)
                *(float4v*)(dst + 64 * pp) =
                    float4v{acc[pp][0][i], acc[pp][1][i], acc[pp][2][i], acc[pp][3][i]};
            if (r16 == 0) a.part_ml[pr] = float2{Mi[i], Li[i]};
        }
    }
}

// out[qh, r] = sum_p e^(m_p - M) O_p / sum_p e^(m_p - M) l_p (m in the log2 domain).
// grid (q heads, rows, D/64), 4 waves: lane = dim, wave w sums parts w, w+4, ...
// with every load issued before the first use (one memory round trip).
constexpr int kDlsaMaxParts = 128;

__global__ __launch_bounds__(256) void dlsa_merge_kernel(const float* __restrict__ part_o,
                                                         const float2* __restrict__ part_ml,
                                                         int parts, int D, int L, int hq,
                                                         f16* __restrict__ out) {
    const int qh = blockIdx.x, r = blockIdx.y, d = blockIdx.z * 64 + (threadIdx.x & 63);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t base = ((int64_t)r * hq + qh) * parts;
    constexpr int PER = kDlsaMaxParts / 4;
    float v[PER];
    float2 ml[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int p = wave + 4 * i;
        if (p < parts) {
            ml[i] = part_ml[base + p];
            v[i] = part_o[(base + p) * D + d];
        } else {
            ml[i] = float2{-INFINITY, 0.0f};
            v[i] = 0.0f;
        }
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; i++) m = fmaxf(m, ml[i].x);
    __shared__ float sm_m[4];
    __shared__ float sm[2][4][64];
    if (lane == 0) sm_m[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(sm_m[0], sm_m[1]), fmaxf(sm_m[2], sm_m[3]));
    float o = 0.0f, l = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const float f = ml[i].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml[i].x - m);
        o = __builtin_fmaf(f, v[i], o);
        l = __builtin_fmaf(f, ml[i].y, l);
    }
    sm[0][wave][lane] = o;
    sm[1][wave][lane] = l;
    __syncthreads();
    if (wave == 0) {
        const float O = (sm[0][0][lane] + sm[0][1][lane]) + (sm[0][2][lane] + sm[0][3][lane]);
        const float Ls = (sm[1][0][lane] + sm[1][1][lane]) + (sm[1][2][lane] + sm[1][3][lane]);
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
    return g_ws[{device, stream}].get(need, stream, out);
}

// Launch policy (the reference's auto_parts, mlx_cxx_dlsa_attention.cpp:379-400,
// re-derived for 256 CUs): one pass when rows x kv_heads alone fill the CUs,
// else split each list so that about one workgroup a CU runs (measured for one
// row, 4 KV heads, 4612 entries: 48 parts 14.2 us, 64 parts 14.3 us, 96 parts
// 15.3 us, 128 parts 16.3 us), keeping at least 16 entries (one tile) a part
// and at most 128 parts.
static int auto_parts(int units, int width) {
    if (units >= 256) return 1;
    int parts = (256 + units - 1) / units;
    parts = std::min(parts, std::max(1, width / 16));
    return std::max(1, std::min(parts, 128));
}

// scratch == nullptr: the split-K partials go to the stream's workspace
// (allocated or grown on demand); else to `scratch` (scratch_bytes), and an
// automatic part count is lowered until the partials fit it.
static int dlsa_sparse_attention_impl(const void* q, const void* k, const void* v, int64_t khs,
                                      int64_t krs, int64_t vhs, int64_t vrs,
                                      const int32_t* lists, const int32_t* lengths, int n_rows,
                                      int width, int n_q_heads, int n_kv_heads, int head_dim,
                                      int n_keys, float scale, int parts, int waves, void* out,
                                      hipStream_t stream, void* scratch, size_t scratch_bytes) {
    QW_REQUIRE(q && k && v && lists && lengths && out, QW_ERR_INVALID_ARGUMENT,
               "dlsa_sparse_attention: null pointer");
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
    // 16-byte row loads: row starts and strides must keep 8-element alignment.
    QW_REQUIRE(((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0 && khs % 8 == 0 &&
                   krs % 8 == 0 && vhs % 8 == 0 && vrs % 8 == 0 && ((uintptr_t)q % 16) == 0,
               QW_ERR_UNSUPPORTED,
               "dlsa_sparse_attention: K/V/q must be 16-byte aligned with strides % 8 == 0");
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
    a.k = (const f16*)k;
    a.v = (const f16*)v;
    a.khs = khs;
    a.krs = krs;
    a.vhs = vhs;
    a.vrs = vrs;
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
    dim3 grid(parts, n_rows, n_kv_heads);
#define QW_DLSA_LAUNCH(DD, GM) \
    hipLaunchKernelGGL((dlsa_kernel<DD, GM>), grid, dim3(256), 0, stream, a)
    if (head_dim == 256) {
        if (G <= 8) QW_DLSA_LAUNCH(256, 8); else QW_DLSA_LAUNCH(256, 16);
    } else if (head_dim == 128) {
        if (G <= 8) QW_DLSA_LAUNCH(128, 8); else QW_DLSA_LAUNCH(128, 16);
    } else {
        if (G <= 8) QW_DLSA_LAUNCH(64, 8); else QW_DLSA_LAUNCH(64, 16);
    }
#undef QW_DLSA_LAUNCH
    QW_HIP_CHECK(hipGetLastError());
    if (parts > 1) {
        hipLaunchKernelGGL(dlsa_merge_kernel, dim3(n_q_heads, n_rows, head_dim / 64), dim3(256), 0,
                           stream, a.part_o, a.part_ml, parts, head_dim, n_rows, n_q_heads,
                           (f16*)out);
        QW_HIP_CHECK(hipGetLastError());
    }
    (void)waves;  // one 4-wave workgroup shape; the knob is accepted for API parity
    return QW_OK;
}

int dlsa_sparse_attention(const void* q, const void* k, const void* v, int64_t khs, int64_t krs,
                          int64_t vhs, int64_t vrs, const int32_t* lists, const int32_t* lengths,
                          int n_rows, int width, int n_q_heads, int n_kv_heads, int head_dim,
                          int n_keys, float scale, int parts, int waves, void* out,
                          hipStream_t stream) {
    return dlsa_sparse_attention_impl(q, k, v, khs, krs, vhs, vrs, lists, lengths, n_rows, width,
                                      n_q_heads, n_kv_heads, head_dim, n_keys, scale, parts, waves,
                                      out, stream, nullptr, 0);
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
    return dlsa_sparse_attention_impl(q, k, v, khs, krs, vhs, vrs, lists, lengths, n_rows, width,
                                      n_q_heads, n_kv_heads, head_dim, n_keys, scale, parts, waves,
                                      out, stream, ws, kDlsaScratchBytes);
}

}  // namespace qw
