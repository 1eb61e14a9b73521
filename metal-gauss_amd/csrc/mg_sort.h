// Host-side entry to the radix sort and scan, shared between translation
// units. Internal header.
#pragma once

#include "mg_common.h"

namespace mg {

// Workspace bytes for sorting n pairs.
int64_t sort_ws_bytes(int64_t n);

// A key window in device memory, for sorts queued before the host knows the
// key range: digits come from min(key, hi) - lo, and passes at or above
// `bits` only copy (their digits are all 0).
template <typename K>
struct DevWin {
    K lo, hi;
    int32_t bits;
};

// Stable LSD sort of (key, int32 value) pairs on key bits [begin_bit,
// end_bit), 8 bits per pass. Result in keys_out/vals_out; the inputs are
// clobbered (ping-pong). Instantiated for uint32_t and uint64_t keys.
template <typename K>
int32_t radix_sort_pairs(K *keys_in, int32_t *vals_in, K *keys_out, int32_t *vals_out,
                         int64_t n, int begin_bit, int end_bit, void *ws, int64_t ws_bytes,
                         hipStream_t s, const char *who);

// The passes only, for int32 or uint2 values (uint2: a tile key's
// {Gaussian id, depth bits}): the sorted data stays in whichever ping-pong buffer the
// last pass wrote (*res_k, *res_v), saving the final copy when the pass count
// is even. Digits come from min(key, hi) - lo, so keys known to lie in
// [lo, hi] sort on bits [0, bit_width(hi - lo)) alone. With dw (device) the
// window and live bit count are read on the device instead of lo/hi, and
// passes at or above dw->bits copy the values only: the sorted values are
// the result, the keys are left unspecified. With status (capacity-bounded
// tile lists: n is the capacity) only the pairs kept are sorted: none if
// status[1] != 0, else the first min(status[0], n). Instantiated for
// uint32_t keys.
template <typename K, typename V>
int32_t radix_sort_passes(K *keys_in, V *vals_in, K *keys_out, V *vals_out,
                          int64_t n, int begin_bit, int end_bit, void *ws, int64_t ws_bytes,
                          hipStream_t s, const char *who, K **res_k, V **res_v, K lo,
                          K hi, const DevWin<K> *dw, const int64_t *status = nullptr);

// Workspace bytes for an exclusive scan of n int32 values.
int64_t scan_ws_bytes(int64_t n);

// out[i] = sum_{j<i} in[idx ? idx[j] : j]; total to total_dev (device int64).
// With idx the values are gathered once (into out, which the second kernel
// then scans in place). idx_dev (device, may be null) supplies idx on the
// device instead, for an index buffer chosen by an earlier kernel.
int32_t exclusive_scan(const int32_t *in, const int32_t *idx, int64_t n, int32_t *out,
                       int64_t *total_dev, void *ws, int64_t ws_bytes, hipStream_t s,
                       const int32_t *const *idx_dev);

}  // namespace mg
