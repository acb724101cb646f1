// kv_cache.hip - KV cache lifecycle, quantize-on-append, dequantize and
// snapshot kernels for gfx950.
//
// Reference behaviour followed (cr0sh/qw):
//   KVCache::new_with_mode / update / update_and_fetch / trim / nbytes /
//   snapshot tensors: crates/mlxcel-core/src/cache.rs:526, :922-1157,
//   :2251-2300, :2709-2834, :3063, :570-626.
//   Affine codec (MLX `quantize` / `dequantize`, group 64):
//   crates/mlxcel-core/cpp/mlx_cxx_bridge.cpp:2991-3040, :6347-6393, at the
//   seam crates/mlxcel-core/src/cache/batch_quant.rs:109-158.
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>

#include "kv_cache.hpp"
#include "append.hpp"
#include "quant.hpp"
#include "rope.hpp"

namespace qw {

static thread_local std::string g_last_error;
void set_error(const std::string& msg) { g_last_error = msg; }
const char* last_error() { return g_last_error.c_str(); }

int GrowBuffer::get(size_t need, hipStream_t stream, void** out) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    QW_HIP_CHECK(hipStreamIsCapturing(stream, &cs));
    const bool capturing = cs != hipStreamCaptureStatusNone;
    if (need > bytes) {
        // HIP refuses allocation inside a global-mode capture, and the refused
        // call would invalidate the caller's capture: refuse here instead.
        QW_REQUIRE(!capturing, QW_ERR_STATE,
                   "split-K workspace: too small for this call and the stream is being captured; "
                   "run one call of this shape on this stream before capturing");
        if (ptr) {
            if (captured) {
                retired.push_back(ptr);  // a graph may still read it
            } else {
                if (stream_owned)
                    QW_HIP_CHECK(hipStreamSynchronize(stream));
                else
                    QW_HIP_CHECK(hipDeviceSynchronize());
                (void)hipFree(ptr);
            }
            ptr = nullptr;
            bytes = 0;
            captured = false;
        }
        const size_t nb = std::max(need + need / 4, (size_t)1 << 20);
        if (hipMalloc(&ptr, nb) != hipSuccess) {
            (void)hipGetLastError();
            ptr = nullptr;
            set_error("split-K workspace: hipMalloc failed");
            return QW_ERR_OUT_OF_MEMORY;
        }
        bytes = nb;
    }
    if (capturing) captured = true;
    *out = ptr;
    return QW_OK;
}

void GrowBuffer::release() {
    if (ptr) (void)hipFree(ptr);
    for (void* p : retired) (void)hipFree(p);
    retired.clear();
    ptr = nullptr;
    bytes = 0;
    captured = false;
}

// Dynamic-LDS limits already raised, per (kernel, device). The attribute is
// a property of the kernel on the current device, so it is recorded per
// device, and the mutex keeps two host threads from interleaving a check and
// a set (which could leave the limit below what the record says).
static std::mutex g_lds_mu;
static std::map<std::pair<const void*, int>, size_t> g_lds_set;

int ensure_dynamic_lds(const void* kernel, size_t bytes) {
    if (bytes <= 65536) return QW_OK;  // the default limit
    int dev = 0;
    QW_HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_lds_mu);
    size_t& cur = g_lds_set[{kernel, dev}];
    if (bytes <= cur) return QW_OK;
    QW_HIP_CHECK(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
    cur = bytes;
    return QW_OK;
}

// --------------------------------------------------------------- sizes

size_t KVCache::k_data_bytes(int c) const { return (size_t)hkv * c * D * bits / 8; }
size_t KVCache::k_param_bytes(int c) const {
    if (turbo4()) return (size_t)hkv * c * 4;
    return affine() ? (size_t)hkv * c * (D / kGroup) * 4 : 0;
}
size_t KVCache::v_data_bytes(int c) const { return (size_t)hkv * c * D * bits / 8; }
size_t KVCache::v_param_bytes(int c) const {
    if (turbo4()) return (size_t)hkv * (c / 8) * 32;
    return affine() ? (size_t)hkv * (c / 8) * (D / kGroup) * 32 : 0;
}

int64_t KVCache::nbytes() const {
    return (int64_t)(k_data_bytes(cap) + k_param_bytes(cap) + v_data_bytes(cap) +
                     v_param_bytes(cap));
}

static int round_cap(int capacity) {
    // The reference grows its buffers in steps of 256 tokens (cache.rs `step`).
    const int step = 256;
    return std::max(step, (capacity + step - 1) / step * step);
}

static int alloc_zero(void** p, size_t bytes) {
    *p = nullptr;
    if (bytes == 0) return QW_OK;
    if (hipMalloc(p, bytes) != hipSuccess) {
        (void)hipGetLastError();
        *p = nullptr;
        set_error("hipMalloc of " + std::to_string(bytes) + " bytes failed");
        return QW_ERR_OUT_OF_MEMORY;
    }
    // Zeroed so that rows past `offset` dequantize to finite zeros: masked keys
    // still pass through the P.V MFMA with weight 0.
    QW_HIP_CHECK(hipMemset(*p, 0, bytes));
    return QW_OK;
}

int KVCache::init(int mode_, int group_size, int n_kv_heads, int head_dim, int capacity,
                  int device_) {
    QW_REQUIRE(mode_ == QW_KV_FP16 || mode_ == QW_KV_AFFINE8 || mode_ == QW_KV_AFFINE4 ||
                   mode_ == QW_KV_INT8 || mode_ == QW_KV_TURBO4,
               QW_ERR_INVALID_ARGUMENT, "qw_kv_create: unknown mode");
    QW_REQUIRE(n_kv_heads > 0 && capacity >= 0 && head_dim > 0, QW_ERR_INVALID_ARGUMENT,
               "qw_kv_create: n_kv_heads, head_dim must be > 0 and capacity >= 0");
    if (mode_ == QW_KV_AFFINE8 || mode_ == QW_KV_AFFINE4) {
        QW_REQUIRE(group_size == kGroup, QW_ERR_UNSUPPORTED,
                   "qw_kv_create: affine modes use group_size 64");
        QW_REQUIRE(head_dim == 256 || head_dim == 128, QW_ERR_UNSUPPORTED,
                   "qw_kv_create: affine modes support head_dim 128 or 256");
    } else {
        // fp16, the per-token Int8 mode and Turbo4 have no group; group_size
        // is ignored
        QW_REQUIRE(head_dim == 256 || head_dim == 128, QW_ERR_UNSUPPORTED,
                   "qw_kv_create: fp16, int8 and turbo4 modes support head_dim 128 or 256");
    }
    mode = mode_;
    bits = (mode_ == QW_KV_AFFINE4 || mode_ == QW_KV_TURBO4) ? 4 : (mode_ == QW_KV_FP16 ? 16 : 8);
    D = head_dim;
    hkv = n_kv_heads;
    device = device_;
    offset = 0;
    cap = 0;
    DeviceGuard dg(device);
    QW_REQUIRE(dg.ok, QW_ERR_HIP, "qw_kv_create: hipSetDevice failed");
    if (hipMalloc(&fast_flag, 256) != hipSuccess) {
        (void)hipGetLastError();
        fast_flag = nullptr;
        set_error("qw_kv_create: hipMalloc failed");
        return QW_ERR_OUT_OF_MEMORY;
    }
    // Int8 codes always take the separately rounded dequant (offset 1152).
    const int fast0 = int8() ? 0 : 1;
    QW_HIP_CHECK(hipMemcpy(fast_flag, &fast0, sizeof(int), hipMemcpyHostToDevice));
    if (turbo4()) {
        int rc = turbo4_setup();
        if (rc) return rc;
    }
    return reserve(capacity, nullptr);
}

int KVCache::release() {
    DeviceGuard dg(device);
    (void)hipDeviceSynchronize();
    void* ptrs[6] = {k_data, (void*)k_params, v_data, (void*)v_params, (void*)fast_flag,
                     (void*)t4_tables};
    for (void* p : ptrs)
        if (p) (void)hipFree(p);
    ws.release();
    fetch_ws.release();
    ws_ptr = nullptr;
    fast_flag = nullptr;
    t4_tables = nullptr;
    k_data = v_data = nullptr;
    k_params = v_params = nullptr;
    cap = offset = 0;
    return QW_OK;
}

int KVCache::reserve(int capacity, hipStream_t stream) {
    const int nc = round_cap(capacity);
    if (nc <= cap) return QW_OK;
    DeviceGuard dg(device);
    void *nk = nullptr, *nkp = nullptr, *nv = nullptr, *nvp = nullptr;
    int rc;
    if ((rc = alloc_zero(&nk, k_data_bytes(nc))) || (rc = alloc_zero(&nkp, k_param_bytes(nc))) ||
        (rc = alloc_zero(&nv, v_data_bytes(nc))) || (rc = alloc_zero(&nvp, v_param_bytes(nc)))) {
        void* ps[4] = {nk, nkp, nv, nvp};
        for (void* p : ps)
            if (p) (void)hipFree(p);
        return rc;
    }
    if (cap > 0) {
        // Per head, the first `cap` rows (K, K params) or cap/8 blocks (V, V
        // params) move to the head's start in the new buffers.
        // (Turbo4: row-major packed V, cap/8 blocks of 8 rows are the same
        // bytes; one 4-byte side record a row.)
        const size_t kr = (size_t)D * bits / 8;
        const size_t kpr = turbo4() ? 4 : (affine() ? (size_t)(D / kGroup) * 4 : 0);
        const size_t vb = (size_t)D * bits;
        const size_t vpb = turbo4() ? 32 : (affine() ? (size_t)(D / kGroup) * 32 : 0);
        for (int h = 0; h < hkv; h++) {
            QW_HIP_CHECK(hipMemcpyAsync((char*)nk + h * (size_t)nc * kr,
                                        (char*)k_data + h * (size_t)cap * kr, cap * kr,
                                        hipMemcpyDeviceToDevice, stream));
            QW_HIP_CHECK(hipMemcpyAsync((char*)nv + h * (size_t)(nc / 8) * vb,
                                        (char*)v_data + h * (size_t)(cap / 8) * vb,
                                        (cap / 8) * vb, hipMemcpyDeviceToDevice, stream));
            if (kpr) {
                QW_HIP_CHECK(hipMemcpyAsync((char*)nkp + h * (size_t)nc * kpr,
                                            (char*)k_params + h * (size_t)cap * kpr, cap * kpr,
                                            hipMemcpyDeviceToDevice, stream));
                QW_HIP_CHECK(hipMemcpyAsync((char*)nvp + h * (size_t)(nc / 8) * vpb,
                                            (char*)v_params + h * (size_t)(cap / 8) * vpb,
                                            (cap / 8) * vpb, hipMemcpyDeviceToDevice, stream));
            }
        }
        QW_HIP_CHECK(hipStreamSynchronize(stream));
        void* old[4] = {k_data, (void*)k_params, v_data, (void*)v_params};
        for (void* p : old)
            if (p) (void)hipFree(p);
    }
    k_data = nk;
    k_params = (uint32_t*)nkp;
    v_data = nv;
    v_params = (uint32_t*)nvp;
    cap = nc;
    return QW_OK;
}

int KVCache::ensure_workspace(size_t bytes, hipStream_t stream) {
    DeviceGuard dg(device);
    return ws.get(bytes, stream, &ws_ptr);
}

int KVCache::demote(int target_mode, hipStream_t stream, int* demoted) {
    // cache.rs:3591 demote_fp16_to_turbo4: a populated fp16 cache is re-stored
    // in the quantized mode by quantize-appending its rows [0, offset) to an
    // empty cache of that mode; anything else is left alone (returns 0).
    *demoted = 0;
    QW_REQUIRE(target_mode == QW_KV_AFFINE4 || target_mode == QW_KV_AFFINE8 ||
                   target_mode == QW_KV_TURBO4,
               QW_ERR_INVALID_ARGUMENT, "demote: target mode must be an affine mode or turbo4");
    if (mode != QW_KV_FP16 || offset <= 0) return QW_OK;
    DeviceGuard dg(device);
    QW_REQUIRE(dg.ok, QW_ERR_HIP, "demote: hipSetDevice failed");
    const int n = offset;
    const size_t bytes = (size_t)hkv * n * D * sizeof(f16);
    void *tk = nullptr, *tv = nullptr;
    if (hipMalloc(&tk, bytes) != hipSuccess || hipMalloc(&tv, bytes) != hipSuccess) {
        (void)hipGetLastError();
        if (tk) (void)hipFree(tk);
        set_error("demote: hipMalloc of the fp16 staging rows failed");
        return QW_ERR_OUT_OF_MEMORY;
    }
    int rc = dequantize(0, n, tk, tv, stream);  // the fp16 rows, [hkv][n][D]
    if (rc == QW_OK) rc = hipStreamSynchronize(stream) == hipSuccess ? QW_OK : QW_ERR_HIP;
    if (rc) {
        (void)hipFree(tk);
        (void)hipFree(tv);
        return rc;
    }
    void* old[4] = {k_data, (void*)k_params, v_data, (void*)v_params};
    const int old_cap = cap;
    k_data = v_data = nullptr;
    k_params = v_params = nullptr;
    cap = 0;
    offset = 0;
    mode = target_mode;
    bits = target_mode == QW_KV_AFFINE8 ? 8 : 4;
    rc = turbo4() ? turbo4_setup() : QW_OK;
    if (rc == QW_OK) rc = reserve(old_cap, stream);
    if (rc == QW_OK) rc = update(tk, tv, n, stream);
    if (rc == QW_OK) rc = hipStreamSynchronize(stream) == hipSuccess ? QW_OK : QW_ERR_HIP;
    (void)hipFree(tk);
    (void)hipFree(tv);
    if (rc) return rc;  // the cache is left empty in the new mode
    for (void* p : old)
        if (p) (void)hipFree(p);
    *demoted = 1;
    return QW_OK;
}

int KVCache::trim(int n) {
    // cache.rs:2251: clamp to the cached length; buffers keep their rows, the
    // next append overwrites them.
    const int m = std::min(n, offset);
    if (m <= 0) return 0;
    offset -= m;
    return m;
}

// Quantize-on-append: one workgroup (4 waves) per (8-token V block touched by
// the append, KV head).
template <int D>
__global__ __launch_bounds__(256) void append_affine_kernel(
    RowSrc rs, int n_tokens, int t_old,
    int bits, int int8, int cap, uint32_t* __restrict__ k_codes, uint32_t* __restrict__ k_params,
    uint32_t* __restrict__ v_codes, f16* __restrict__ v_params, int* __restrict__ fast_flag) {
    __shared__ AppendScratch<D> sc;
    append_block<D>(rs, n_tokens, t_old, bits, int8 != 0, cap, k_codes, k_params, v_codes, v_params,
                    fast_flag, t_old / 8 + blockIdx.x, blockIdx.y, threadIdx.x, blockDim.x, sc);
}

// fp16 mode append: K rows copied, V scattered into 8-key blocks.
template <int D>
__global__ __launch_bounds__(256) void append_fp16_kernel(RowSrc rs, int n_tokens, int t_old,
                                                          int cap, f16* __restrict__ k_data,
                                                          f16* __restrict__ v_data) {
    const int h = blockIdx.y;
    const int64_t n = (int64_t)n_tokens * D;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / D), d = (int)(i % D);
        const int t = r + t_old;
        const int64_t src = (int64_t)r * rs.row_stride + (int64_t)h * rs.head_stride;
        const f16 kv = rs.rope_dims > 0 ? (f16)rope_elem(rs.k + src, d, rs.rope_dims, rs.traditional,
                                                       rs.log2_base, rs.scale, rs.position0 + r)
                                        : rs.k[src + d];
        const f16 vv = rs.v[src + d];
        k_data[((int64_t)h * cap + t) * D + d] = kv;
        v_data[(((int64_t)h * (cap / 8) + t / 8) * D + v_phys_dim(d, D, 16)) * 8 + (t & 7)] = vv;
    }
}

int KVCache::update(const void* k_new, const void* v_new, int n_tokens, hipStream_t stream) {
    QW_REQUIRE(n_tokens >= 0, QW_ERR_INVALID_ARGUMENT, "update: n_tokens must be >= 0");
    if (n_tokens == 0) return QW_OK;
    QW_REQUIRE(k_new && v_new, QW_ERR_INVALID_ARGUMENT, "update: null K/V pointer");
    RowSrc rs{};
    rs.k = (const f16*)k_new;
    rs.v = (const f16*)v_new;
    rs.row_stride = D;
    rs.head_stride = (int64_t)n_tokens * D;
    return update_rows(rs, n_tokens, stream);
}

int KVCache::update_rows(const RowSrc& rs, int n_tokens, hipStream_t stream) {
    if (n_tokens == 0) return QW_OK;
    DeviceGuard dg(device);
    QW_REQUIRE(dg.ok, QW_ERR_HIP, "update: hipSetDevice failed");
    const int need = offset + n_tokens;
    if (need > cap) {
        // Geometric growth keeps appends amortized O(1) per token.
        int rc = reserve(std::max(need, cap + cap / 2), stream);
        if (rc) return rc;
    }
    if (turbo4()) {
        int rc = turbo4_update(rs, n_tokens, stream);
        if (rc) return rc;
    } else if (affine()) {
        const int nblk = (offset + n_tokens - 1) / 8 - offset / 8 + 1;
        dim3 grid(nblk, hkv);
        if (D == 256)
            hipLaunchKernelGGL(append_affine_kernel<256>, grid, dim3(256), 0, stream,
                               rs, n_tokens, offset, bits,
                               int8() ? 1 : 0, cap, (uint32_t*)k_data, k_params,
                               (uint32_t*)v_data, (f16*)v_params, fast_flag);
        else
            hipLaunchKernelGGL(append_affine_kernel<128>, grid, dim3(256), 0, stream,
                               rs, n_tokens, offset, bits,
                               int8() ? 1 : 0, cap, (uint32_t*)k_data, k_params,
                               (uint32_t*)v_data, (f16*)v_params, fast_flag);
    } else {
        const int64_t n = (int64_t)n_tokens * D;
        dim3 grid((unsigned)std::min<int64_t>((n + 255) / 256, 1024), hkv);
        if (D == 256)
            hipLaunchKernelGGL(append_fp16_kernel<256>, grid, dim3(256), 0, stream,
                               rs, n_tokens, offset, cap,
                               (f16*)k_data, (f16*)v_data);
        else
            hipLaunchKernelGGL(append_fp16_kernel<128>, grid, dim3(256), 0, stream,
                               rs, n_tokens, offset, cap,
                               (f16*)k_data, (f16*)v_data);
    }
    QW_HIP_CHECK(hipGetLastError());
    offset += n_tokens;
    return QW_OK;
}

// ------------------------------------------------------------ dequantize
//
// MLX's composite dequantize: out = f16(f16(code * scale) + bias). code *
// scale is exact in fp32 (<= 8 x 11 significant bits), so the first cast is
// the fp16 product; the sum is formed in fp32 and cast once more, which is
// how MLX's CPU float16 type evaluates `a + b`.

// `off` is 128 for Int8 codes stored biased by 128 (bias 0: the result is
// f16(code * scale), the reference's Int8 dequantize, cache.rs:313-316).
__device__ inline f16 mlx_dequant(uint32_t c, int off, f16 s, f16 b) {
    const f16 prod = (f16)((float)((int)c - off) * (float)s);
    return (f16)((float)prod + (float)b);
}

// One thread per (head, row, 8 dims); writes 16 bytes of K and of V.
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ k_codes,
                                                      const uint32_t* __restrict__ k_params,
                                                      const uint32_t* __restrict__ v_codes,
                                                      const f16* __restrict__ v_params,
                                                      int bits, int code_off, int D, int cap,
                                                      int hkv, int start, int n,
                                                      f16* __restrict__ k_out,
                                                      f16* __restrict__ v_out) {
    const int64_t oct = D / 8;
    const int64_t total = (int64_t)hkv * n * oct;
    const int NG = D / kGroup;
    const int nw = D * bits / 32;
    const uint32_t m = (1u << bits) - 1u;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int h = (int)(i / (n * oct));
        const int r = (int)((i / oct) % n);
        const int d0 = (int)(i % oct) * 8;
        const int t = start + r;
        const int g = d0 / kGroup;
        const half2v ksb = __builtin_bit_cast(
            half2v, k_params[((int64_t)h * cap + t) * NG + k_param_slot(g, NG)]);
        const f16* vp = v_params + (((int64_t)h * (cap / 8) + t / 8) * NG + g) * 16;
        const f16 vs = vp[t & 7], vbias = vp[8 + (t & 7)];
        const uint32_t* krow = k_codes + ((int64_t)h * cap + t) * nw;
        const uint32_t* vblk = v_codes + ((int64_t)h * (cap / 8) + t / 8) * (D * bits / 4);
        half8 ko, vo;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int d = d0 + e;
            const int epw = 32 / bits;
            const uint32_t kcode = (krow[d / epw] >> ((d % epw) * bits)) & m;
            ko[e] = mlx_dequant(kcode, code_off, ksb.x, ksb.y);
            const int p = v_phys_dim(d, D, bits);
            const int k = t & 7;
            uint32_t vcode;
            if (bits == 4)
                vcode = (vblk[p] >> (4 * v4_nibble_pos(k))) & 0xFu;
            else
                vcode = (vblk[2 * p + (k >> 2)] >> (8 * (k & 3))) & 0xFFu;
            vo[e] = mlx_dequant(vcode, code_off, vs, vbias);
        }
        const int64_t o = ((int64_t)h * n + r) * D + d0;
        *(half8*)(k_out + o) = ko;
        *(half8*)(v_out + o) = vo;
    }
}

// fp16 mode: K rows copied; V gathered out of the 8-key blocks.
__global__ __launch_bounds__(256) void fetch_fp16_kernel(const f16* __restrict__ k_data,
                                                         const f16* __restrict__ v_data, int D,
                                                         int cap, int hkv, int start, int n,
                                                         f16* __restrict__ k_out,
                                                         f16* __restrict__ v_out) {
    const int64_t total = (int64_t)hkv * n * D;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int h = (int)(i / ((int64_t)n * D));
        const int r = (int)((i / D) % n);
        const int d = (int)(i % D);
        const int t = start + r;
        k_out[i] = k_data[((int64_t)h * cap + t) * D + d];
        v_out[i] =
            v_data[(((int64_t)h * (cap / 8) + t / 8) * D + v_phys_dim(d, D, 16)) * 8 + (t & 7)];
    }
}

int KVCache::dequantize(int start, int n, void* k_out, void* v_out, hipStream_t stream) const {
    QW_REQUIRE(start >= 0 && n >= 0 && start + n <= offset, QW_ERR_INVALID_ARGUMENT,
               "dequantize: window [start, start+n) outside the cached rows");
    if (n == 0) return QW_OK;
    QW_REQUIRE(k_out && v_out, QW_ERR_INVALID_ARGUMENT, "dequantize: null output");
    DeviceGuard dg(device);
    if (turbo4()) return turbo4_dequantize(start, n, k_out, v_out, stream);
    const int64_t work = affine() ? (int64_t)hkv * n * (D / 8) : (int64_t)hkv * n * D;
    const unsigned blocks = (unsigned)std::min<int64_t>((work + 255) / 256, 4096);
    if (affine())
        hipLaunchKernelGGL(dequant_kernel, dim3(blocks), dim3(256), 0, stream,
                           (const uint32_t*)k_data, k_params, (const uint32_t*)v_data,
                           (const f16*)v_params, bits, int8() ? 128 : 0, D, cap, hkv, start, n,
                           (f16*)k_out, (f16*)v_out);
    else
        hipLaunchKernelGGL(fetch_fp16_kernel, dim3(blocks), dim3(256), 0, stream,
                           (const f16*)k_data, (const f16*)v_data, D, cap, hkv, start, n,
                           (f16*)k_out, (f16*)v_out);
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

int KVCache::update_and_fetch(const void* k_new, const void* v_new, int n_tokens, void* k_out,
                              void* v_out, hipStream_t stream) {
    int rc = update(k_new, v_new, n_tokens, stream);
    if (rc) return rc;
    return dequantize(0, offset, k_out, v_out, stream);
}

// ------------------------------------------------------- snapshot tensors
//
// Export/import in the reference's layout: per head, rows [0, offset) of
// MLX-packed codes and separate fp16 scale and bias planes (cache.rs:570-626
// exports packed tensors as they are, without requantizing).

// V blocks <-> rows, plus the K param split/merge. dir = 0: export.
// Int8 mode: codes leave and enter as signed bytes (stored + 128, i.e. XOR
// 0x80 per byte) and one scale per row (the first group's; every group holds
// it, with bias 0).
__global__ __launch_bounds__(256) void snapshot_affine_kernel(
    int dir, int bits, int int8, int D, int cap, int hkv, int n, int* __restrict__ fast_flag,
    uint32_t* __restrict__ k_params,
    uint32_t* __restrict__ v_codes, f16* __restrict__ v_params, f16* __restrict__ ks_out,
    f16* __restrict__ kb_out, uint32_t* __restrict__ vc_rows, f16* __restrict__ vs_rows,
    f16* __restrict__ vb_rows) {
    const int NG = D / kGroup;
    const int nw = D * bits / 32;
    const int epw = 32 / bits;
    const uint32_t m = (1u << bits) - 1u;
    const int64_t total = (int64_t)hkv * n * nw;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int h = (int)(i / ((int64_t)n * nw));
        const int t = (int)((i / nw) % n);
        const int w = (int)(i % nw);
        const int k = t & 7;
        uint32_t* vblk = v_codes + ((int64_t)h * (cap / 8) + t / 8) * (D * bits / 4);
        const int64_t row = (int64_t)h * n + t;
        if (dir == 0) {
            uint32_t word = 0;
            for (int e = 0; e < epw; e++) {
                const int p = v_phys_dim(w * epw + e, D, bits);
                const uint32_t c = bits == 4 ? (vblk[p] >> (4 * v4_nibble_pos(k))) & m
                                             : (vblk[2 * p + (k >> 2)] >> (8 * (k & 3))) & m;
                word |= c << (e * bits);
            }
            vc_rows[row * nw + w] = int8 ? word ^ 0x80808080u : word;
        }
        if (w < NG) {
            const int g = w;
            const int64_t kp = ((int64_t)h * cap + t) * NG + k_param_slot(g, NG);
            f16* vp = v_params + (((int64_t)h * (cap / 8) + t / 8) * NG + g) * 16;
            if (int8) {
                if (dir == 0) {
                    if (g == 0) {
                        ks_out[row] = __builtin_bit_cast(half2v, k_params[kp]).x;
                        vs_rows[row] = vp[k];
                    }
                } else {
                    half2v sb;
                    sb.x = ks_out[row];
                    sb.y = (f16)0.0f;
                    k_params[kp] = __builtin_bit_cast(uint32_t, sb);
                    vp[k] = vs_rows[row];
                    vp[8 + k] = (f16)0.0f;
                }
            } else if (dir == 0) {
                const half2v sb = __builtin_bit_cast(half2v, k_params[kp]);
                ks_out[row * NG + g] = sb.x;
                kb_out[row * NG + g] = sb.y;
                vs_rows[row * NG + g] = vp[k];
                vb_rows[row * NG + g] = vp[8 + k];
            } else {
                half2v sb;
                sb.x = ks_out[row * NG + g];
                sb.y = kb_out[row * NG + g];
                k_params[kp] = __builtin_bit_cast(uint32_t, sb);
                vp[k] = vs_rows[row * NG + g];
                vp[8 + k] = vb_rows[row * NG + g];
                check_fast_scale(sb.x, bits, fast_flag);
                check_fast_scale(vp[k], bits, fast_flag);
            }
        }
    }
}

__global__ void set_flag_kernel(int* flag, int v) { *flag = v; }

// Import of V codes: one thread per (head, block, dim) builds the block word(s).
__global__ __launch_bounds__(256) void import_v_codes_kernel(int bits, int int8, int D, int cap,
                                                             int hkv, int n,
                                                             const uint32_t* __restrict__ rows,
                                                             uint32_t* __restrict__ v_codes) {
    const int nblk = (n + 7) / 8;
    const int nw = D * bits / 32;
    const int epw = 32 / bits;
    const uint32_t m = (1u << bits) - 1u;
    const int64_t total = (int64_t)hkv * nblk * D;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int h = (int)(i / ((int64_t)nblk * D));
        const int b = (int)((i / D) % nblk);
        const int d = (int)(i % D);
        uint32_t w0 = 0, w1 = 0;
        for (int k = 0; k < 8; k++) {
            const int t = b * 8 + k;
            if (t >= n) break;
            const uint32_t c = (rows[((int64_t)h * n + t) * nw + d / epw] >> ((d % epw) * bits)) & m;
            if (bits == 4)
                w0 |= c << (4 * v4_nibble_pos(k));
            else if (k < 4)
                w0 |= c << (8 * k);
            else
                w1 |= c << (8 * (k - 4));
        }
        if (int8) {
            // Int8: signed bytes in, biased bytes stored (slots past n stay 128 = code 0)
            w0 ^= 0x80808080u;
            w1 ^= 0x80808080u;
        }
        uint32_t* vblk = v_codes + ((int64_t)h * (cap / 8) + b) * (D * bits / 4);
        const int p = v_phys_dim(d, D, bits);
        if (bits == 4) {
            vblk[p] = w0;
        } else {
            vblk[2 * p] = w0;
            vblk[2 * p + 1] = w1;
        }
    }
}

// XOR 0x80 into every byte of rows [0, n) of each head's row-major K codes
// ([hkv][stride][nw] words): signed <-> biased Int8 codes.
__global__ __launch_bounds__(256) void flip_code_sign_kernel(uint32_t* __restrict__ words, int hkv,
                                                             int n, int nw, int stride) {
    const int64_t total = (int64_t)hkv * n * nw;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int h = (int)(i / ((int64_t)n * nw));
        const int64_t r = i % ((int64_t)n * nw);
        words[(int64_t)h * stride * nw + r] ^= 0x80808080u;
    }
}

int KVCache::export_tensors(void* k_codes, void* k_scales, void* k_biases, void* v_codes,
                            void* v_scales, void* v_biases, hipStream_t stream) const {
    QW_REQUIRE(!turbo4(), QW_ERR_STATE, "export: a Turbo4 cache exports with qw_kv_export_turbo4");
    QW_REQUIRE(k_codes && v_codes, QW_ERR_INVALID_ARGUMENT, "export: null code pointers");
    QW_REQUIRE(!affine() || (k_scales && v_scales && (int8() || (k_biases && v_biases))),
               QW_ERR_INVALID_ARGUMENT, "export: null scale/bias pointers");
    if (offset == 0) return QW_OK;
    DeviceGuard dg(device);
    const int n = offset;
    if (!affine()) {
        // Same as a full fetch in fp16 mode.
        return dequantize(0, n, k_codes, v_codes, stream);
    }
    const size_t kr = (size_t)D * bits / 8;
    for (int h = 0; h < hkv; h++)
        QW_HIP_CHECK(hipMemcpyAsync((char*)k_codes + h * (size_t)n * kr,
                                    (const char*)k_data + h * (size_t)cap * kr, n * kr,
                                    hipMemcpyDeviceToDevice, stream));
    const int64_t work = (int64_t)hkv * n * (D * bits / 32);
    const unsigned nb = (unsigned)std::min<int64_t>((work + 255) / 256, 4096);
    if (int8()) {
        hipLaunchKernelGGL(flip_code_sign_kernel, dim3(nb), dim3(256), 0, stream,
                           (uint32_t*)k_codes, hkv, n, D / 4, n);
        QW_HIP_CHECK(hipGetLastError());
    }
    hipLaunchKernelGGL(snapshot_affine_kernel, dim3(nb), dim3(256), 0, stream, 0, bits,
                       int8() ? 1 : 0, D, cap, hkv, n, fast_flag, k_params, (uint32_t*)v_data,
                       (f16*)v_params, (f16*)k_scales, (f16*)k_biases, (uint32_t*)v_codes,
                       (f16*)v_scales, (f16*)v_biases);
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

int KVCache::import_tensors(int n_tokens, const void* k_codes, const void* k_scales,
                            const void* k_biases, const void* v_codes, const void* v_scales,
                            const void* v_biases, hipStream_t stream) {
    QW_REQUIRE(!turbo4(), QW_ERR_STATE, "import: a Turbo4 cache imports with qw_kv_import_turbo4");
    QW_REQUIRE(n_tokens >= 0, QW_ERR_INVALID_ARGUMENT, "import: n_tokens must be >= 0");
    QW_REQUIRE(k_codes && v_codes, QW_ERR_INVALID_ARGUMENT, "import: null code pointers");
    QW_REQUIRE(!affine() || (k_scales && v_scales && (int8() || (k_biases && v_biases))),
               QW_ERR_INVALID_ARGUMENT, "import: null scale/bias pointers");
    DeviceGuard dg(device);
    offset = 0;
    if (n_tokens == 0) return QW_OK;
    if (!affine()) return update(k_codes, v_codes, n_tokens, stream);
    int rc = reserve(n_tokens, stream);
    if (rc) return rc;
    const int n = n_tokens;
    const size_t kr = (size_t)D * bits / 8;
    for (int h = 0; h < hkv; h++)
        QW_HIP_CHECK(hipMemcpyAsync((char*)k_data + h * (size_t)cap * kr,
                                    (const char*)k_codes + h * (size_t)n * kr, n * kr,
                                    hipMemcpyDeviceToDevice, stream));
    // The imported scales decide the fused kernels' dequant path afresh (Int8
    // always takes the separately rounded one).
    hipLaunchKernelGGL(set_flag_kernel, dim3(1), dim3(1), 0, stream, fast_flag, int8() ? 0 : 1);
    const int64_t work = (int64_t)hkv * n * (D * bits / 32);
    const unsigned nb = (unsigned)std::min<int64_t>((work + 255) / 256, 4096);
    if (int8()) {
        hipLaunchKernelGGL(flip_code_sign_kernel, dim3(nb), dim3(256), 0, stream,
                           (uint32_t*)k_data, hkv, n, D / 4, cap);
        QW_HIP_CHECK(hipGetLastError());
    }
    hipLaunchKernelGGL(snapshot_affine_kernel, dim3(nb), dim3(256), 0, stream, 1, bits,
                       int8() ? 1 : 0, D, cap, hkv, n, fast_flag, k_params, (uint32_t*)v_data,
                       (f16*)v_params, (f16*)k_scales, (f16*)k_biases, (uint32_t*)v_codes,
                       (f16*)v_scales, (f16*)v_biases);
    QW_HIP_CHECK(hipGetLastError());
    const int64_t vwork = (int64_t)hkv * ((n + 7) / 8) * D;
    hipLaunchKernelGGL(import_v_codes_kernel,
                       dim3((unsigned)std::min<int64_t>((vwork + 255) / 256, 4096)), dim3(256),
                       0, stream, bits, int8() ? 1 : 0, D, cap, hkv, n,
                       (const uint32_t*)v_codes, (uint32_t*)v_data);
    QW_HIP_CHECK(hipGetLastError());
    offset = n;
    return QW_OK;
}

}  // namespace qw
