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
// (rank32(score) << 32) | i, unique, smaller = better. The row's rank32 values
// are staged into LDS once (when they fit, rank_cap of them) so that every
// later pass reads LDS rather than global memory. The top min(top_p, v)
// keys are found by a radix select on rank32 (4 passes of 8 bits over the
// row, one LDS histogram a wave, summed per pass); the keys strictly better
// than the threshold value are all kept, and of those equal to it the lowest
// indices (an index-ordered pass, run only when the threshold value is shared
// by more keys than remain to be taken). The kept keys (<= 2048) are sorted
// bitonically: one key a thread in registers when they fit the workgroup
// (strides below 64 by wave shuffles, longer ones through LDS), else in LDS.
// A block prefix scan over the picked buckets' member counts places every
// member of the expansion without a serial walk; with one pick a thread and
// small, aligned member rows the members are read once into registers.
#include "kv_cache.hpp"

namespace qw {

namespace {

constexpr int kSelectMax = 2048;  // most buckets a row may pick (top_p)
constexpr int kKeysPerThread = 16;  // rank keys a thread keeps in registers

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
    int rank_cap;             // rank32 values the dynamic LDS holds (0: none)
    int vec_members;          // members 16-byte aligned, cap a multiple of 4, <= 16
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

// Ascending sort of a thread's N register values (bitonic network, N a power
// of two).
template <int N>
__device__ __forceinline__ void sort_regs(uint32_t (&x)[N]) {
#pragma unroll
    for (int k = 2; k <= N; k <<= 1)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1)
#pragma unroll
            for (int i = 0; i < N; i++) {
                const int l = i ^ j;
                if (l > i) {
                    const uint32_t lo = min(x[i], x[l]), hi = max(x[i], x[l]);
                    const bool up = (i & k) == 0;
                    x[i] = up ? lo : hi;
                    x[l] = up ? hi : lo;
                }
            }
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t x, int mask) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)x, mask);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(x >> 32), mask);
    return ((uint64_t)hi << 32) | lo;
}

__global__ __launch_bounds__(1024) void dlsa_select_kernel(SelectArgs a) {
    __shared__ uint64_t sel[kSelectMax];
    __shared__ __attribute__((aligned(16))) int scan[2 * 1024];
    __shared__ int cnt[kSelectMax];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t whist[16][256];  // one radix histogram a wave
    __shared__ int sh_int[4];
    extern __shared__ uint32_t rank_lds[];  // [rank_cap] rank32 of the row
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
    const int wave = t >> 6, n_waves = T >> 6;

    // ---- the row's rank32 values into LDS (one global pass), with the NaN
    // check; rows of up to kKeysPerThread * T also keep each thread's keys
    // (columns t, t + T, ...) in registers, so the radix passes and the
    // compaction load nothing.
    const bool cached = v <= a.rank_cap;
    const bool in_regs = v <= kKeysPerThread * T;
    uint32_t kr[kKeysPerThread];
    if (t == 0) sh_int[0] = 0;
    if (in_regs) {
        bool nan = false;
        float f[kKeysPerThread];
#pragma unroll
        for (int j = 0; j < kKeysPerThread; j++) f[j] = t + j * T < v ? row[t + j * T] : 0.0f;
#pragma unroll
        for (int j = 0; j < kKeysPerThread; j++) {
            nan |= f[j] != f[j];
            kr[j] = rank32(f[j]);
            if (t + j * T < v) rank_lds[t + j * T] = kr[j];
        }
        __syncthreads();
        if (nan && n_sel > 0) sh_int[0] = 1;  // (no pick, no NaN status, as below)
    } else if (cached) {
        bool nan = false;
        int i = t;
        for (; i + 3 * T < v; i += 4 * T) {
            float f[4];
#pragma unroll
            for (int j = 0; j < 4; j++) f[j] = row[i + j * T];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                nan |= f[j] != f[j];
                rank_lds[i + j * T] = rank32(f[j]);
            }
        }
        for (; i < v; i += T) {
            const float f = row[i];
            nan |= f != f;
            rank_lds[i] = rank32(f);
        }
        __syncthreads();
        if (nan && n_sel > 0) sh_int[0] = 1;  // (no pick, no NaN status, as below)
    }
    auto rank_at = [&](int i) -> uint32_t { return cached ? rank_lds[i] : rank32(row[i]); };

    // ---- threshold: the n_sel-th smallest rank32 (radix select, 8 bits a pass)
    uint32_t prefix = 0, pmask = 0;
    int k = n_sel;  // rank of the wanted key among those matching `prefix`
    int below = 0;  // keys with rank32 strictly below the final threshold
    __syncthreads();
    if (n_sel > 0 && n_sel < v) {
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int i = t; i < 16 * 256; i += T) (&whist[0][0])[i] = 0;
            __syncthreads();
            bool nan = false;
            if (in_regs && shift == 24) {
                // The first digit (sign and top exponent bits) takes few
                // values: the thread sorts its keys' digits and adds one count
                // a run, about 3x fewer atomics on the few busy bins.
                uint32_t d[kKeysPerThread];
#pragma unroll
                for (int j = 0; j < kKeysPerThread; j++) d[j] = t + j * T < v ? kr[j] >> 24 : 256u;
                sort_regs(d);
                uint32_t run = 1;
#pragma unroll
                for (int j = 0; j < kKeysPerThread; j++) {
                    if (j + 1 < kKeysPerThread && d[j] == d[j + 1]) {
                        run++;
                    } else {
                        if (d[j] < 256u) atomicAdd(&whist[wave][d[j]], run);
                        run = 1;
                    }
                }
            } else if (in_regs) {
#pragma unroll
                for (int j = 0; j < kKeysPerThread; j++)
                    if (t + j * T < v && (kr[j] & pmask) == prefix)
                        atomicAdd(&whist[wave][(kr[j] >> shift) & 0xFF], 1u);
            } else {
                for (int i = t; i < v; i += T) {
                    uint32_t key;
                    if (cached) {
                        key = rank_lds[i];
                    } else {
                        const float f = row[i];
                        nan |= f != f;
                        key = rank32(f);
                    }
                    if ((key & pmask) == prefix)
                        atomicAdd(&whist[wave][(key >> shift) & 0xFF], 1u);
                }
            }
            if (nan) sh_int[0] = 1;
            __syncthreads();
            for (int i = t; i < 256; i += T) {
                uint32_t sum = 0;
                for (int w = 0; w < n_waves; w++) sum += whist[w][i];
                hist[i] = sum;
            }
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
    } else if (n_sel > 0 && !cached) {
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
        for (int i = t; i < v; i += T) sel[i] = ((uint64_t)rank_at(i) << 32) | (uint32_t)i;
    } else if (n_sel > 0) {
        bool eq_placed;  // (workgroup-uniform)
        if (in_regs) {
            // keys below thr and equal to it, counted per thread and placed by
            // one block scan of both counts packed in an int (each <= 2^14)
            int c_lt = 0, c_eq = 0;
#pragma unroll
            for (int j = 0; j < kKeysPerThread; j++) {
                if (t + j * T < v) {
                    c_lt += kr[j] < thr;
                    c_eq += kr[j] == thr;
                }
            }
            int tot;
            const int ex = block_exclusive_scan(c_lt | (c_eq << 16), scan, tot);
            eq_placed = (tot >> 16) == need;
            int o_lt = ex & 0xFFFF, o_eq = below + (ex >> 16);
#pragma unroll
            for (int j = 0; j < kKeysPerThread; j++) {
                const int i = t + j * T;
                if (i < v) {
                    if (kr[j] < thr)
                        sel[o_lt++] = ((uint64_t)kr[j] << 32) | (uint32_t)i;
                    else if (eq_placed && kr[j] == thr)
                        sel[o_eq++] = ((uint64_t)thr << 32) | (uint32_t)i;
                }
            }
        } else {
            int eq_local = 0;
            for (int i = t; i < v; i += T) {
                const uint32_t key = rank_at(i);
                if (key < thr) sel[atomicAdd(&sh_int[3], 1)] = ((uint64_t)key << 32) | (uint32_t)i;
                eq_local += key == thr;
            }
            int n_eq;
            (void)block_exclusive_scan(eq_local, scan, n_eq);
            eq_placed = n_eq == need;
            if (eq_placed) {
                for (int i = t; i < v; i += T)
                    if (rank_at(i) == thr)
                        sel[atomicAdd(&sh_int[3], 1)] = ((uint64_t)thr << 32) | (uint32_t)i;
            }
        }
        if (!eq_placed) {
            // ties across the threshold: the `need` lowest indices among them
            int taken = 0;
            for (int base = 0; base < v && taken < need; base += T) {
                const int i = base + t;
                const int eq = i < v && rank_at(i) == thr ? 1 : 0;
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
    if (n_sel > 0 && n_pad <= T) {
        // One key a thread. Each wave sorts its 64 keys ascending (bitonic
        // by shuffles), then runs of 64, 128, ... merge pairwise: a key's
        // place in the merged run is its place in its own run plus the count
        // of the partner run's keys before it (a branch-free binary search in
        // LDS; keys are unique but for the padding, whose ties break left run
        // first). One barrier a merge round, none inside a wave's sort.
        const int lane = t & 63;
        uint64_t x = t < n_sel ? sel[t] : ~0ull;
        for (int size = 2; size <= 64; size <<= 1) {
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                const uint64_t y = shfl_xor_u64(x, stride);
                const bool keep_min = ((lane & stride) == 0) == ((lane & size) == 0);
                const uint64_t mn = x < y ? x : y, mx = x < y ? y : x;
                x = keep_min ? mn : mx;
            }
        }
        uint64_t* cur = sel;
        uint64_t* nxt = reinterpret_cast<uint64_t*>(scan);  // free during the sort
        if (t < n_pad) cur[t] = x;
        __syncthreads();
        for (int run = 64; run < n_pad; run <<= 1) {
            if (t < n_pad) {
                const int base = t & ~(2 * run - 1);
                const bool left = (t & run) == 0;
                const uint64_t* other = cur + base + (left ? run : 0);
                int c = 0;
                for (int step = run >> 1; step > 0; step >>= 1) {
                    const uint64_t o = other[c + step - 1];
                    if (left ? o < x : o <= x) c += step;
                }
                const uint64_t o = other[c];
                if (left ? o < x : o <= x) c += 1;
                nxt[base + (t & (run - 1)) + c] = x;
            }
            __syncthreads();
            if (t < n_pad) x = nxt[t];
            uint64_t* const tmp = cur;
            cur = nxt;
            nxt = tmp;
        }
        __syncthreads();
        if (t < n_pad) sel[t] = x;
        __syncthreads();
    } else if (n_sel > 0) {
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
    int total;
    if (a.vec_members && n_sel <= T) {
        // one pick a thread, its members read once (16-byte loads) and kept in
        // registers between the count and the write
        int32_t mem[16];
        int c = 0;
        if (t < n_sel) {
            const int4* mb4 = (const int4*)(a.members + (int64_t)(uint32_t)sel[t] * a.cap);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                if (4 * q < a.cap) {
                    const int4 w = mb4[q];
                    mem[4 * q] = w.x;
                    mem[4 * q + 1] = w.y;
                    mem[4 * q + 2] = w.z;
                    mem[4 * q + 3] = w.w;
                }
            }
#pragma unroll
            for (int j = 0; j < 16; j++)
                if (j < a.cap) c += mem[j] >= lo && mem[j] < hi && mem[j] >= 0;
        }
        int off = block_exclusive_scan(c, scan, total);
        if (t < n_sel) {
#pragma unroll
            for (int j = 0; j < 16; j++) {
                if (j < a.cap && mem[j] >= lo && mem[j] < hi && mem[j] >= 0) {
                    if (off < a.top_k) lrow[off] = mem[j];
                    off++;
                }
            }
        }
    } else {
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
    // Rows of up to kRankCap visible buckets keep their rank32 values in LDS
    // (96 KB beside the ~49 KB of static arrays); longer rows read global
    // memory in every pass.
    constexpr int kRankCap = 24576;
    a.rank_cap = kRankCap;
    a.vec_members = bucket_cap <= 16 && bucket_cap % 4 == 0 &&
                    ((uintptr_t)members & 15) == 0;
    const size_t shmem = (size_t)kRankCap * sizeof(uint32_t);
    int rc = ensure_dynamic_lds((const void*)dlsa_select_kernel, shmem);
    if (rc) return rc;
    const int T = threads ? threads : 1024;
    hipLaunchKernelGGL(dlsa_select_kernel, dim3(n_rows), dim3(T), shmem, stream, a);
    QW_HIP_CHECK(hipGetLastError());
    return QW_OK;
}

}  // namespace qw
