// Stable LSD radix sort of (key, value) pairs, digits of up to 8 bits,
// tiles of 1024 to 4096 keys (large sorts use 4096, so a tile's run of one
// digit averages at least 16 keys: 64-byte stores).
//
// Each pass is reduce-then-scan, with no inter-workgroup waiting:
//   1. upsweep   - every workgroup histograms the digit of its tile;
//   2. scan      - one workgroup per digit scans that digit's counts over the
//                  tiles (digit-major layout), leaving each tile's base;
//   3. downsweep - every workgroup ranks its keys stably (each wave ranks its
//                  own contiguous chunk with ballots against a wave-private
//                  LDS histogram; a prefix over the waves joins them), sorts
//                  the tile locally in LDS by digit, and writes each digit's
//                  run to its global slot so stores come out as contiguous
//                  runs.
// Stability holds because items are ranked in their input order (wave w,
// round r, lane l is item c w + 64 r + l of the tile, c the keys per wave),
// and tiles are ranked in tile order by the scan.
//
// Digits are taken from min(key, hi) - lo. With lo/hi the smallest and
// largest key that matters, this order-preserving shift lets a caller sort
// only the bits in which its keys differ (fewer passes); keys above hi tie
// with hi. The identity window is lo = 0, hi = all ones.
#include "mg_common.h"
#include "mg_sort.h"

namespace mg {

constexpr int kSortThreads = 256;
// Keys per thread: 4, 8 or 16 (tiles of 1024, 2048 or 4096 keys). Large
// sorts (from ~4M keys) take 4096-key tiles for long digit runs; mid-sized
// ones (from ~256k) 2048, small ones 1024 to spread over the CUs. Measured
// at config 4: the 1M-key depth sort is fastest at 2048 (67 vs 74 us at 1024
// and 80 at 4096), the 5M-pair tile sort at 4096 (102 vs 109 at 2048).
constexpr int kSortTileMin = kSortThreads * 4;
constexpr int kRadix = 256;

inline int sort_items_for(int64_t n) {
    if (n >= (int64_t)kSortThreads * 16 * 1024) return 16;
    if (n >= (int64_t)kSortThreads * 8 * 128) return 8;
    return 4;
}
constexpr int kSortWaves = kSortThreads / 64;

template <typename K>
struct KeyWin {
    K lo, hi;
};

template <typename K>
__device__ __forceinline__ uint32_t digit_of(K key, int shift, uint32_t mask, KeyWin<K> w) {
    return (uint32_t)(((key < w.hi ? key : w.hi) - w.lo) >> shift) & mask;
}

// The window a pass uses: the by-value one, or the device-resident one
// (dw != NULL), whose bit count also marks passes at or above it as plain
// copies (all their digits are 0, so a stable pass would not move a key).
template <typename K>
__device__ __forceinline__ KeyWin<K> pass_window(KeyWin<K> win, const DevWin<K> *dw, int shift,
                                                 bool &copy) {
    copy = false;
    if (dw == nullptr) return win;
    copy = shift >= dw->bits;
    return KeyWin<K>{dw->lo, dw->hi};
}

// The keys a pass sorts: n, or with a status (capacity-bounded tile lists,
// n being the capacity) the pairs kept, read on the device: none if
// status[1] flags an overflow, else min(status[0], n). Tiles past them
// count nothing and move nothing.
__device__ __forceinline__ int64_t sort_count(int64_t n, const int64_t *status) {
    return status ? (status[1] != 0 ? 0 : min(status[0], n)) : n;
}

template <typename K, int kSortItems>
__global__ __launch_bounds__(kSortThreads) void radix_upsweep_kernel(const K *keys, int64_t n,
                                                                     int shift, uint32_t mask,
                                                                     KeyWin<K> win0,
                                                                     const DevWin<K> *dw,
                                                                     uint32_t *hist,
                                                                     int64_t ntiles,
                                                                     const int64_t *status) {
    __shared__ uint32_t s_h[kSortWaves][kRadix];
    bool copy;
    const KeyWin<K> win = pass_window(win0, dw, shift, copy);
    if (copy) return;   // whole workgroup
    constexpr int kSortTile = kSortThreads * kSortItems;
    const int64_t base = (int64_t)blockIdx.x * kSortTile;
    n = sort_count(n, status);
    if (base >= n) {   // workgroup-uniform: a tile past the keys counts nothing
        for (int d = threadIdx.x; d < kRadix; d += kSortThreads)
            hist[(int64_t)d * ntiles + blockIdx.x] = 0u;
        return;
    }
    const int wave = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < kSortWaves * kRadix; i += kSortThreads) (&s_h[0][0])[i] = 0;
    __syncthreads();
    // Every key is requested before any is counted: loads at a clamped index
    // (n >= 1), and a count of 0 past n, so no load sits in a branch that
    // waits for it before the next.
    K kv[kSortItems];
#pragma unroll
    for (int r = 0; r < kSortItems; ++r)
        kv[r] = keys[min(base + (int64_t)r * kSortThreads + threadIdx.x, n - 1)];
#pragma unroll
    for (int r = 0; r < kSortItems; ++r) {
        const int64_t i = base + (int64_t)r * kSortThreads + threadIdx.x;
        atomicAdd(&s_h[wave][digit_of(kv[r], shift, mask, win)], i < n ? 1u : 0u);
    }
    __syncthreads();
    for (int d = threadIdx.x; d < kRadix; d += kSortThreads) {
        uint32_t s = 0;
#pragma unroll
        for (int w = 0; w < kSortWaves; ++w) s += s_h[w][d];
        hist[(int64_t)d * ntiles + blockIdx.x] = s;
    }
}

// One workgroup per digit: exclusive scan of hist[d][0..ntiles) in place,
// digit total to totals[d].
__global__ __launch_bounds__(kSortThreads) void radix_scan_kernel(uint32_t *hist, int64_t ntiles,
                                                                  uint32_t *totals, int shift,
                                                                  const int32_t *dbits) {
    __shared__ uint32_t s_w[kSortWaves];
    if (dbits && shift >= *dbits) return;   // a copy pass: nothing to scan
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t *row = hist + (int64_t)blockIdx.x * ntiles;
    uint32_t carry = 0;
    for (int64_t c0 = 0; c0 < ntiles; c0 += kSortThreads) {
        const int64_t i = c0 + threadIdx.x;
        const uint32_t v = i < ntiles ? row[i] : 0u;
        uint32_t incl = v;
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t t = __shfl_up(incl, o, 64);
            if (lane >= o) incl += t;
        }
        if (lane == 63) s_w[wave] = incl;
        __syncthreads();
        uint32_t before = 0, all = 0;
#pragma unroll
        for (int w = 0; w < kSortWaves; ++w) {
            if (w < wave) before += s_w[w];
            all += s_w[w];
        }
        __syncthreads();
        if (i < ntiles) row[i] = carry + before + incl - v;
        carry += all;
    }
    if (threadIdx.x == 0) totals[blockIdx.x] = carry;
}

// Downsweep: rank the tile's keys stably by digit, sort the tile in LDS,
// store each digit's run at its global slot.
//
// Wave w owns the contiguous chunk [c w, c w + c) of the tile (c = 64 x keys
// per thread), loaded in rounds of 64 consecutive keys. Within a round, lanes holding the same
// digit find each other with one ballot per live digit bit; the lowest such
// lane adds the group's size to the wave's own LDS digit histogram, which
// every lane of the group read first, so an item's rank within its wave is
// (earlier rounds' count of its digit) + (earlier lanes of its group). No
// workgroup barrier is needed while ranking. Afterwards each digit's wave
// counts become an exclusive prefix over the waves, and the tile's digit
// starts an exclusive scan over digits; position in the tile = digit start
// + wave prefix + rank in wave. Items are thus ranked in tile order (wave,
// round, lane), which makes every pass stable.
//
// The keys and then the values go through one LDS exchange buffer in turn
// (sized for the wider of the two), so a workgroup holds 37 KB of LDS rather
// than 53 KB and four fit on a CU instead of two. The store loop of the keys
// leaves each sorted position's digit in the thread's registers for the
// values' store loop.
template <typename K, typename V, int kSortItems>
__global__ __launch_bounds__(kSortThreads) void radix_downsweep_kernel(
    const K *keys_in, const V *vals_in, K *keys_out, V *vals_out, int64_t n,
    int shift, uint32_t mask, KeyWin<K> win0, const DevWin<K> *dw, const uint32_t *hist,
    int64_t ntiles, const uint32_t *totals, const int64_t *status) {
    constexpr int kSortTile = kSortThreads * kSortItems;
    constexpr int kChunk = kSortTile / kSortWaves;       // keys per wave
    constexpr int kItemBytes = sizeof(K) > sizeof(V) ? sizeof(K) : sizeof(V);
    __shared__ __align__(16) unsigned char s_x[kSortTile * kItemBytes];
    K *s_keys = reinterpret_cast<K *>(s_x);  // the exchange buffer, keys first
    V *s_vals = reinterpret_cast<V *>(s_x);  // then values
    __shared__ uint32_t s_base[kRadix];     // global slot of this tile's digit run
    __shared__ uint32_t s_loc[kRadix];      // start of each digit inside the tile
    __shared__ uint32_t s_wh[kSortWaves][kRadix];   // per-wave digit counts
    __shared__ uint32_t s_w[kSortWaves];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t base = (int64_t)blockIdx.x * kSortTile;
    n = sort_count(n, status);
    if (base >= n) return;   // workgroup-uniform: no key of this tile is sorted
    const int nitems = (int)min((int64_t)kSortTile, n - base);
    const int nbits = 32 - __builtin_clz(mask);          // live digit bits (mask = 2^b - 1)
    bool copy;
    const KeyWin<K> win = pass_window(win0, dw, shift, copy);
    if (copy) {
        // Every digit of this pass is 0: the stable order is the input order.
        // Only the values move; later passes are copies too, so the keys are
        // not read again (and are unspecified after a device-window sort).
        for (int i = tid; i < nitems; i += kSortThreads) vals_out[base + i] = vals_in[base + i];
        return;
    }

    // Global digit bases: exclusive scan of the digit totals (one digit per
    // thread), plus this tile's exclusive prefix within the digit.
    {
        const uint32_t v = tid < kRadix ? totals[tid] : 0u;
        uint32_t incl = v;
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t t = __shfl_up(incl, o, 64);
            if (lane >= o) incl += t;
        }
        if (lane == 63) s_w[wave] = incl;
        __syncthreads();
        uint32_t before = 0;
        for (int w = 0; w < wave; ++w) before += s_w[w];
        if (tid < kRadix)
            s_base[tid] = before + incl - v + hist[(int64_t)tid * ntiles + blockIdx.x];
    }
    for (int i = lane; i < kRadix; i += 64) s_wh[wave][i] = 0;

    K key[kSortItems];
    V val[kSortItems];
    uint32_t rank[kSortItems];
    const int c0 = wave * kChunk;
#pragma unroll
    for (int r = 0; r < kSortItems; ++r) {
        const int idx = c0 + r * 64 + lane;
        if (idx < nitems) {
            key[r] = keys_in[base + idx];
            val[r] = vals_in[base + idx];
        } else {
            key[r] = 0;
            val[r] = V{};
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    uint32_t *wh = s_wh[wave];
#pragma unroll
    for (int r = 0; r < kSortItems; ++r) {
        const bool ok = c0 + r * 64 + lane < nitems;
        const uint32_t d = digit_of(key[r], shift, mask, win);
        uint64_t peers = ballot(ok);
        for (int b = 0; b < nbits; ++b) {
            const bool bit = (d >> b) & 1u;
            const uint64_t m = ballot(bit);
            peers &= bit ? m : ~m;
        }
        const uint32_t wrank = (uint32_t)__popcll(peers & lt_mask);
        const uint32_t prior = ok ? wh[d] : 0u;
        rank[r] = prior + wrank;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (ok && wrank == 0) wh[d] = prior + (uint32_t)__popcll(peers);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    __syncthreads();

    // Per digit: wave counts -> exclusive prefix over the waves; the tile's
    // digit count, scanned over digits, gives the digit starts.
    {
        uint32_t cnt = 0;
        if (tid < kRadix) {
#pragma unroll
            for (int w = 0; w < kSortWaves; ++w) {
                const uint32_t t = s_wh[w][tid];
                s_wh[w][tid] = cnt;
                cnt += t;
            }
        }
        uint32_t incl = cnt;
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t t = __shfl_up(incl, o, 64);
            if (lane >= o) incl += t;
        }
        __syncthreads();                     // s_w is reused
        if (lane == 63) s_w[wave] = incl;
        __syncthreads();
        uint32_t before = 0;
        for (int w = 0; w < wave; ++w) before += s_w[w];
        if (tid < kRadix) s_loc[tid] = before + incl - cnt;
        __syncthreads();
    }
    // rank[r] becomes the item's position in the tile (kSortTile past the
    // keys: no item there).
#pragma unroll
    for (int r = 0; r < kSortItems; ++r) {
        uint32_t lp = (uint32_t)kSortTile;
        if (c0 + r * 64 + lane < nitems) {
            const uint32_t d = digit_of(key[r], shift, mask, win);
            lp = s_loc[d] + s_wh[wave][d] + rank[r];
        }
        rank[r] = lp;
        if (lp < (uint32_t)kSortTile) s_keys[lp] = key[r];
    }
    __syncthreads();
    // Sorted position tid + 256 j has digit byte j % 4 of dig[j / 4].
    uint32_t dig[kSortItems / 4];
#pragma unroll
    for (int j = 0; j < kSortItems / 4; ++j) dig[j] = 0u;
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int i = tid + j * kSortThreads;
        if (i < nitems) {
            const K k = s_keys[i];
            const uint32_t d = digit_of(k, shift, mask, win);
            dig[j >> 2] |= d << (8 * (j & 3));
            const uint32_t dst = s_base[d] + (uint32_t)i - s_loc[d];
            if ((int64_t)dst < n) keys_out[dst] = k;   // always, for a consistent histogram
        }
    }
    __syncthreads();   // every key is read before the values overwrite them
#pragma unroll
    for (int r = 0; r < kSortItems; ++r)
        if (rank[r] < (uint32_t)kSortTile) s_vals[rank[r]] = val[r];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int i = tid + j * kSortThreads;
        if (i < nitems) {
            const uint32_t d = (dig[j >> 2] >> (8 * (j & 3))) & 0xFFu;
            const uint32_t dst = s_base[d] + (uint32_t)i - s_loc[d];
            if ((int64_t)dst < n) vals_out[dst] = s_vals[i];
        }
    }
}

// Workspace: hist (kRadix * ntiles) + totals (kRadix), uint32, sized for the
// smallest tile.
int64_t sort_ws_bytes(int64_t n) {
    const int64_t ntiles = ceil_div(n > 0 ? n : 1, kSortTileMin);
    return (kRadix * ntiles + kRadix) * (int64_t)sizeof(uint32_t);
}

// Runs the passes; on return *res_k / *res_v point at whichever ping-pong
// buffer holds the sorted data (keys_out when the pass count is odd).
template <typename K, typename V>
int32_t radix_sort_passes(K *keys_in, V *vals_in, K *keys_out, V *vals_out,
                          int64_t n, int begin_bit, int end_bit, void *ws, int64_t ws_bytes,
                          hipStream_t s, const char *who, K **res_k, V **res_v, K lo,
                          K hi, const DevWin<K> *dw, const int64_t *status) {
    MG_REQUIRE(n >= 0 && n < (1LL << 31), "%s: n = %lld", who, (long long)n);
    MG_REQUIRE(begin_bit >= 0 && end_bit <= (int)(8 * sizeof(K)) && begin_bit <= end_bit,
               "%s: bit range [%d, %d)", who, begin_bit, end_bit);
    MG_REQUIRE(ws && ws_bytes >= sort_ws_bytes(n), "%s: workspace %lld bytes, need %lld", who,
               (long long)ws_bytes, (long long)sort_ws_bytes(n));
    *res_k = keys_in;
    *res_v = vals_in;
    if (n == 0) return MG_OK;
    MG_REQUIRE(keys_in && vals_in && keys_out && vals_out, "%s: null buffer", who);
    const int items = sort_items_for(n);
    const int64_t ntiles = ceil_div(n, (int64_t)kSortThreads * items);
    uint32_t *hist = static_cast<uint32_t *>(ws);
    uint32_t *totals = hist + kRadix * ntiles;
    K *src_k = keys_in, *dst_k = keys_out;
    V *src_v = vals_in, *dst_v = vals_out;
    MG_REQUIRE(lo <= hi, "%s: empty key window", who);
    const KeyWin<K> win{lo, hi};
    TimedScope ts(who, s);
    // Passes of at most 8 bits, the widths as even as the bit count allows
    // (13 bits: 7 + 6, not 8 + 5), so no pass has short digit runs.
    const int npass = (end_bit - begin_bit + 7) / 8;
    int pass = 0;
    for (int b = begin_bit; b < end_bit; ++pass) {
        const int width = (end_bit - begin_bit) / npass + (pass < (end_bit - begin_bit) % npass);
        const uint32_t mask = (1u << width) - 1u;
#define MG_SORT_PASS(IT)                                                                   \
    radix_upsweep_kernel<K, IT><<<(unsigned)ntiles, kSortThreads, 0, s>>>(                 \
        src_k, n, b, mask, win, dw, hist, ntiles, status);                                 \
    MG_LAUNCHED("radix_upsweep_kernel");                                                   \
    radix_scan_kernel<<<kRadix, kSortThreads, 0, s>>>(hist, ntiles, totals, b,             \
                                                      dw ? &dw->bits : nullptr);           \
    MG_LAUNCHED("radix_scan_kernel");                                                      \
    radix_downsweep_kernel<K, V, IT><<<(unsigned)ntiles, kSortThreads, 0, s>>>(            \
        src_k, src_v, dst_k, dst_v, n, b, mask, win, dw, hist, ntiles, totals, status);    \
    MG_LAUNCHED("radix_downsweep_kernel");
        if (items == 16) { MG_SORT_PASS(16) }
        else if (items == 8) { MG_SORT_PASS(8) }
        else { MG_SORT_PASS(4) }
#undef MG_SORT_PASS
        b += width;
        K *tk = src_k; src_k = dst_k; dst_k = tk;
        V *tv = src_v; src_v = dst_v; dst_v = tv;
    }
    *res_k = src_k;      // after the last swap src_* holds the sorted data
    *res_v = src_v;
    return MG_OK;
}

template <typename K>
int32_t radix_sort_pairs(K *keys_in, int32_t *vals_in, K *keys_out, int32_t *vals_out,
                         int64_t n, int begin_bit, int end_bit, void *ws, int64_t ws_bytes,
                         hipStream_t s, const char *who) {
    K *rk;
    int32_t *rv;
    int32_t rc = radix_sort_passes<K, int32_t>(keys_in, vals_in, keys_out, vals_out, n, begin_bit,
                                      end_bit, ws, ws_bytes, s, who, &rk, &rv, K(0), ~K(0),
                                      nullptr, nullptr);
    if (rc != MG_OK) return rc;
    if (n > 0 && rk != keys_out) {
        MG_HIP(hipMemcpyAsync(keys_out, rk, n * sizeof(K), hipMemcpyDeviceToDevice, s));
        MG_HIP(hipMemcpyAsync(vals_out, rv, n * sizeof(int32_t), hipMemcpyDeviceToDevice, s));
    }
    return MG_OK;
}

template int32_t radix_sort_pairs<uint32_t>(uint32_t *, int32_t *, uint32_t *, int32_t *, int64_t,
                                            int, int, void *, int64_t, hipStream_t, const char *);
template int32_t radix_sort_pairs<uint64_t>(uint64_t *, int32_t *, uint64_t *, int32_t *, int64_t,
                                            int, int, void *, int64_t, hipStream_t, const char *);
template int32_t radix_sort_passes<uint32_t, int32_t>(uint32_t *, int32_t *, uint32_t *,
                                                      int32_t *, int64_t, int, int, void *,
                                                      int64_t, hipStream_t, const char *,
                                                      uint32_t **, int32_t **, uint32_t, uint32_t,
                                                      const DevWin<uint32_t> *, const int64_t *);
template int32_t radix_sort_passes<uint32_t, uint2>(uint32_t *, uint2 *, uint32_t *, uint2 *,
                                                    int64_t, int, int, void *, int64_t,
                                                    hipStream_t, const char *, uint32_t **,
                                                    uint2 **, uint32_t, uint32_t,
                                                    const DevWin<uint32_t> *, const int64_t *);

}  // namespace mg

using namespace mg;

extern "C" {

int64_t mg_sort_workspace_bytes(int64_t n) { return sort_ws_bytes(n); }

int32_t mg_sort_pairs_u64(uint64_t *keys_in, int32_t *vals_in, uint64_t *keys_out,
                          int32_t *vals_out, int64_t n, int32_t begin_bit, int32_t end_bit,
                          void *workspace, int64_t workspace_bytes, mg_stream_t stream) {
    return radix_sort_pairs<uint64_t>(keys_in, vals_in, keys_out, vals_out, n, begin_bit,
                                      end_bit, workspace, workspace_bytes, as_stream(stream),
                                      "radix_sort");
}

}  // extern "C"
