// dlsa_select.hip - D-LSA K1: the fused top-p bucket select + expansion +
// window + sinks, gfx950.
//
// Reference: dlsa_select (crates/mlxcel-core/src/dlsa_kernels.rs:57-117,
// cpp/mlx_cxx_dlsa.cpp) whose lists, lengths and picked buckets equal the
// host select (crates/runtime/src/dlsa/select.rs:65-115) on the same scores.
// Row r (position p) ranks its first v = min(floor(p / window) * m,
// total_rows) score columns (clipped to the columns given: status bit 2):
// score descending, -0 == +0, a NaN below every number (status bit 1), ties
// to the lower bucket; keeps the best min(top_p, v); its list is the picked
// buckets' members in [sink, window_start) (pick order, members ascending,
// at most top_k), then the window [window_start, p], then the sinks
// [0, min(sink, window_start, p + 1)), -1 padded.
//
// One workgroup a row. The rank of column i is the 64-bit key
// (rank32(score) << 32) | i, unique, smaller = better. The top min(top_p, v)
// keys are found by a radix select on rank32 (4 passes of 8 bits over the
// row's scores, histograms in LDS); the keys strictly better than the
// threshold value are all kept, and of those equal to it the lowest indices
// (an index-ordered pass, run only when the threshold value is shared by more
// keys than remain to be taken). The kept keys (<= 2048) are sorted in LDS
// (bitonic), and a block prefix scan over the picked buckets' member counts
// places every member of the expansion without a serial walk.
#include "kv_cache.hpp"

namespace qw {

namespace {

constexpr int kSelectMax = 2048;  // most buckets a row may pick (top_p)

struct SelectArgs {
    const float* scores;      // [R][stride]
    int64_t stride;
    const int32_t* members;   // [n_member_rows][cap]
    int cap;
    const int32_t* positions; // [R]
    int total_rows;
    int window, sink, top_k, top_p, m;
    int32_t* lists;           // [R][top_k + window + sink]
    int32_t* lengths;         // [R]
    int32_t* picked;          // [R][top_p]
    int32_t* status;          // [R]
};

// Monotone key: smaller = better (score descending), -0 == +0, every NaN
// after every number.
__device__ __forceinline__ uint32_t rank32(float f) {
    if (f != f) return 0xFFFFFFFFu;
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7FFFFFFFu) == 0u) u = 0u;  // -0 -> +0
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);  // ascending in f
    return ~ord;
}

// Exclusive prefix sum of `x` over the workgroup's threads (any power-of-two
// size up to 1024); `tot` receives the total. Uses sm[0 .. 2*nthreads).
__device__ __forceinline__ int block_exclusive_scan(int x, int* sm, int& tot) {
    const int t = threadIdx.x, n = blockDim.x;
    int* a = sm;
    int* b = sm + n;
    a[t] = x;
    __syncthreads();
    for (int off = 1; off < n; off <<= 1) {
        b[t] = a[t] + (t >= off ? a[t - off] : 0);
        __syncthreads();
        int* c = a;
        a = b;
        b = c;
    }
    const int incl = a[t];
    tot = a[n - 1];
    __syncthreads();
    return incl - x;
}

__global__ __launch_bounds__(1024) void dlsa_select_kernel(SelectArgs a) {
    __shared__ uint64_t sel[kSelectMax];
    __shared__ int scan[2 * 1024];
    __shared__ int cnt[kSelectMax];
    __shared__ uint32_t hist[256];
    __shared__ int sh_int[4];
    const int r = blockIdx.x;
    const int t = threadIdx.x, T = blockDim.x;
    const int p = a.positions[r];
    int v = min((p / a.window) * a.m, a.total_rows);
    int st = 0;
    if ((int64_t)v > a.stride) {
        v = (int)a.stride;
        st |= 2;
    }
    const float* row = a.scores + (int64_t)r * a.stride;
    const int n_sel = min(a.top_p, v);

    // ---- threshold: the n_sel-th smallest rank32 (radix select, 8 bits a pass)
    uint32_t prefix = 0, pmask = 0;
    int k = n_sel;  // rank of the wanted key among those matching `prefix`
    int below = 0;  // keys with rank32 strictly below the final threshold
    if (t == 0) sh_int[0] = 0;
    __syncthreads();
    if (n_sel > 0 && n_sel < v) {
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int i = t; i < 256; i += T) hist[i] = 0;
            __syncthreads();
            bool nan = false;
            for (int i = t; i < v; i += T) {
                const float f = row[i];
                nan |= f != f;
                const uint32_t key = rank32(f);
                if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 0xFF], 1u);
            }
            if (nan) sh_int[0] = 1;
            __syncthreads();
            // the digit whose cumulative count reaches k (one wave scans)
            if (t < 64) {
                uint32_t c4[4], s = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    c4[j] = hist[4 * t + j];
                    s += c4[j];
                }
                uint32_t incl = s;
#pragma unroll
                for (int off = 1; off < 64; off <<= 1) {
                    const uint32_t o = __shfl_up(incl, off);
                    if (t >= off) incl += o;
                }
                uint32_t before = incl - s;
                // lane whose range [before, incl) holds the k-th (1-based) key
                if (before < (uint32_t)k && (uint32_t)k <= incl) {
                    int j = 0;
                    while (before + c4[j] < (uint32_t)k) before += c4[j++];
                    sh_int[1] = 4 * t + j;
                    sh_int[2] = (int)before;
                }
            }
            __syncthreads();
            const int digit = sh_int[1];
            k -= sh_int[2];
            below += sh_int[2];
            prefix |= (uint32_t)digit << shift;
            pmask |= 0xFFu << shift;
            __syncthreads();
        }
    } else if (n_sel > 0) {
        // every visible bucket is picked: just the NaN check
        bool nan = false;
        for (int i = t; i < v; i += T) nan |= row[i] != row[i];
        if (nan) sh_int[0] = 1;
    }
    __syncthreads();
    if (sh_int[0]) st |= 1;
    const uint32_t thr = prefix;
    const int need = k;  // keys equal to thr still to take (lowest indices first)

    // ---- compaction of the kept keys into sel[0 .. n_sel)
    if (t == 0) sh_int[3] = 0;
    __syncthreads();
    if (n_sel == v) {
        for (int i = t; i < v; i += T) sel[i] = ((uint64_t)rank32(row[i]) << 32) | (uint32_t)i;
    } else if (n_sel > 0) {
        int eq_local = 0;
        for (int i = t; i < v; i += T) {
            const uint32_t key = rank32(row[i]);
            if (key < thr) {
                sel[atomicAdd(&sh_int[3], 1)] = ((uint64_t)key << 32) | (uint32_t)i;
            } else if (key == thr) {
                eq_local++;
            }
        }
        int n_eq;
        (void)block_exclusive_scan(eq_local, scan, n_eq);
        if (n_eq == need) {
            for (int i = t; i < v; i += T)
                if (rank32(row[i]) == thr)
                    sel[atomicAdd(&sh_int[3], 1)] = ((uint64_t)thr << 32) | (uint32_t)i;
        } else {
            // ties across the threshold: the `need` lowest indices among them
            int taken = 0;
            for (int base = 0; base < v && taken < need; base += T) {
                const int i = base + t;
                const int eq = i < v && rank32(row[i]) == thr ? 1 : 0;
                int n_blk;
                const int pos = taken + block_exclusive_scan(eq, scan, n_blk);
                if (eq && pos < need) sel[below + pos] = ((uint64_t)thr << 32) | (uint32_t)i;
                taken += n_blk;
            }
        }
    }
    __syncthreads();

    // ---- sort the kept keys (bitonic over the next power of two)
    int n_pad = 1;
    while (n_pad < n_sel) n_pad <<= 1;
    if (n_sel > 0) {
        for (int i = n_sel + t; i < n_pad; i += T) sel[i] = ~0ull;
        __syncthreads();
        for (int size = 2; size <= n_pad; size <<= 1) {
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                for (int i = t; i < n_pad / 2; i += T) {
                    const int lo = 2 * i - (i & (stride - 1));
                    const int hi = lo + stride;
                    const bool up = (lo & size) == 0;
                    const uint64_t x = sel[lo], y = sel[hi];
                    if ((x > y) == up) {
                        sel[lo] = y;
                        sel[hi] = x;
                    }
                }
                __syncthreads();
            }
        }
    }

    // ---- picked buckets, best first
    int32_t* prow = a.picked + (int64_t)r * a.top_p;
    for (int i = t; i < a.top_p; i += T) prow[i] = i < n_sel ? (int32_t)(uint32_t)sel[i] : -1;

    // ---- expansion: members of the picked buckets in [sink, window_start)
    const int ws = max(0, p + 1 - a.window);
    const int lo = a.sink, hi = ws;
    const int width = a.top_k + a.window + a.sink;
    int32_t* lrow = a.lists + (int64_t)r * width;
    // counts per picked bucket, in pick order, then their exclusive prefix
    for (int i = t; i < n_sel; i += T) {
        const int32_t* mb = a.members + (int64_t)(uint32_t)sel[i] * a.cap;
        int c = 0;
        for (int j = 0; j < a.cap; j++) {
            const int x = mb[j];
            c += x >= lo && x < hi && x >= 0;
        }
        cnt[i] = c;
    }
    __syncthreads();
    // chunked scan: thread t owns picks [t*per, (t+1)*per)
    const int per = (n_sel + T - 1) / T;
    int chunk = 0;
    for (int i = t * per; i < min(n_sel, (t + 1) * per); i++) chunk += cnt[i];
    int total;
    int off = block_exclusive_scan(chunk, scan, total);
    for (int i = t * per; i < min(n_sel, (t + 1) * per); i++) {
        const int32_t* mb = a.members + (int64_t)(uint32_t)sel[i] * a.cap;
        for (int j = 0; j < a.cap; j++) {
            const int x = mb[j];
            if (x >= lo && x < hi && x >= 0) {
                if (off < a.top_k) lrow[off] = x;
                off++;
            }
        }
    }
    const int E = min(total, a.top_k);
    // ---- window, then sinks, then padding
    const int nw = p - ws + 1;
    const int ns = min(min(a.sink, ws), p + 1);
    for (int i = t; i < nw; i += T) lrow[E + i] = ws + i;
    for (int i = t; i < ns; i += T) lrow[E + nw + i] = i;
    for (int i = E + nw + ns + t; i < width; i += T) lrow[i] = -1;
    if (t == 0) {
        a.lengths[r] = E + nw + ns;
        a.status[r] = st;
    }
}

}  // namespace

int dlsa_select(const float* scores, int64_t stride, const int32_t* members, int n_member_rows,
                int bucket_cap, const int32_t* positions, int n_rows, int total_rows, int window,
                int sink, int top_k, int top_p, int buckets_per_block, int threads,
                int32_t* lists, int32_t* lengths, int32_t* picked, int32_t* status,
                hipStream_t stream) {
    QW_REQUIRE(n_rows >= 0 && stride >= 0 && n_member_rows >= 0, QW_ERR_INVALID_ARGUMENT,
               "dlsa_select: negative sizes");
    QW_REQUIRE(window > 0 && sink >= 0 && top_k >= 0 && top_p >= 0 && bucket_cap > 0 &&
                   buckets_per_block > 0,
               QW_ERR_INVALID_ARGUMENT, "dlsa_select: bad knobs");
    QW_REQUIRE(top_p <= kSelectMax, QW_ERR_INVALID_ARGUMENT,
               "dlsa_select: top_p exceeds 2048 (DLSA_TOP_P_MAX)");
    QW_REQUIRE(total_rows >= 0 && total_rows <= n_member_rows, QW_ERR_INVALID_ARGUMENT,
               "dlsa_select: total_rows exceeds the member table");
    QW_REQUIRE(threads == 0 || (threads >= 64 && threads <= 1024 && (threads & (threads - 1)) == 0),
               QW_ERR_INVALID_ARGUMENT,
               "dlsa_select: threads must be 0 or a power of two in [64, 1024]");
    if (n_rows == 0) return QW_OK;
    QW_REQUIRE(positions && lists && lengths && status && (picked || top_p == 0) &&
                   (scores || stride == 0) && (members || n_member_rows == 0),
               QW_ERR_INVALID_ARGUMENT, "dlsa_select: null pointer");
    SelectArgs a;
    a.scores = scores;
    a.stride = stride;
    a.members = members;
    a.cap = bucket_cap;
    a.positions = positions;
    a.total_rows = total_rows;
    a.window = window;
    a.sink = sink;
    a.top_k = top_k;
    a.top_p = top_p;
    a.m = buckets_per_block;
    a.lists = lists;
    a.lengths = lengths;
    a.picked = picked;
    a.status = status;
    const int T = threads ? threads : 256;
    hipLaunchKernelGGL(dlsa_select_kernel, dim3(n_rows), dim3(T), 0, stream, a);
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

}  // namespace qw
