// Shared host + device helpers for libmgauss. Internal header.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mgauss.h"

namespace mg {

// ---------------------------------------------------------------- host side

// Records a printf-style message as the thread's last error.
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

// After a launch: maps hipGetLastError to MG_ERR_LAUNCH with the kernel name.
int32_t check_launch(const char *kernel);

// Device address, on the current device, of the static scratch array of the
// allocation-free loss entry point (looked up once per device).
int32_t static_scratch(float **out, const char *who);

// Event timing around one launch (active only while mg_timing_enable(1)).
struct TimedScope {
    TimedScope(const char *kernel, hipStream_t stream);
    ~TimedScope();
    const char *kernel_;
    hipStream_t stream_;
    int slot_;
};

// A pinned host word and an event of the current device, held (locked) for
// the life of the object: a host read that must not stall the stream copies
// its value into `slot`, records `ev`, queues further work, and only then
// waits on `ev`. ok() is false (with the error set) if allocation failed.
class HostReadback {
  public:
    HostReadback();
    ~HostReadback();
    HostReadback(const HostReadback &) = delete;
    HostReadback &operator=(const HostReadback &) = delete;
    bool ok() const { return slot != nullptr; }
    int64_t *slot = nullptr;
    hipEvent_t ev = nullptr;

  private:
    void *lock_;
};

inline hipStream_t as_stream(mg_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Workspace carving: every sub-buffer starts on a 256-byte boundary.
inline int64_t align256(int64_t b) { return (b + 255) & ~(int64_t)255; }

// Number of XCDs workgroups are spread over, round-robin by workgroup id.
constexpr int kXcds = 8;

// Work item of workgroup b out of nb such that each XCD runs one contiguous
// run of items (XCD k the k-th run, the first nb % 8 runs one item longer):
// neighbouring items then share an L2. A bijection of [0, nb).
__device__ __forceinline__ int64_t xcd_contiguous(int64_t b, int64_t nb) {
    const int64_t q = nb / kXcds, r = nb - q * kXcds;
    const int64_t xcd = b % kXcds, idx = b / kXcds;
    return xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
}

// One Adam element update, torch's formula with eps after the sqrt(bc2)
// divide (metal_gauss/csrc/adam.metal:34-41): step_size = lr / bc1 and
// inv_sqrt_bc2 = 1 / sqrt(bc2), formed in double by the caller. Shared by the
// optimizer kernels and the preprocess backward's optimizer epilogue so both
// round identically.
__device__ __forceinline__ void adam_update(float &p, float g, float &m, float &v, float b1,
                                            float b2, float omb1, float omb2, float eps,
                                            float step_size, float inv_sqrt_bc2,
                                            bool eps_inside) {
    m = fmaf(b1, m, omb1 * g);
    v = fmaf(b2, v, omb2 * g * g);
    const float sv = sqrtf(v);
    const float denom = eps_inside ? (sv + eps) : (sv * inv_sqrt_bc2 + eps);
    p = p - step_size * m / denom;
}

#define MG_REQUIRE(cond, ...)                                                  \
    do {                                                                       \
        if (!(cond)) {                                                         \
            ::mg::set_error(__VA_ARGS__);                                      \
            return MG_ERR_ARG;                                                 \
        }                                                                      \
    } while (0)

#define MG_HIP(call)                                                           \
    do {                                                                       \
        hipError_t e_ = (call);                                                \
        if (e_ != hipSuccess) {                                                \
            ::mg::set_error("%s failed: %s", #call, hipGetErrorString(e_));    \
            return MG_ERR_RUNTIME;                                             \
        }                                                                      \
    } while (0)

#define MG_LAUNCHED(name)                                                      \
    do {                                                                       \
        int32_t rc_ = ::mg::check_launch(name);                                \
        if (rc_ != MG_OK) return rc_;                                          \
    } while (0)

// -------------------------------------------------------------- device side

__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ uint64_t ballot(bool p) {
    return __builtin_amdgcn_ballot_w64(p);
}

// Lanes below this one that are set in `mask`.
__device__ __forceinline__ int rank_in(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
}

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                           ROW_MASK, 0xf, false));
}

// Sum over the 64 lanes of a wave; the total lands in lane 63.
// Rows of 16 are reduced with row_shr, then rows are combined with the GFX9
// row broadcasts (lane 15 -> rows 1,3; lane 31 -> rows 2,3).
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
    v += dpp_f<0x111>(v);        // row_shr:1
    v += dpp_f<0x112>(v);        // row_shr:2
    v += dpp_f<0x114>(v);        // row_shr:4
    v += dpp_f<0x118>(v);        // row_shr:8
    v += dpp_f<0x142, 0xa>(v);   // row_bcast:15
    v += dpp_f<0x143, 0xc>(v);   // row_bcast:31
    return v;
}

__device__ __forceinline__ float wave_min(float v) {
    for (int o = 32; o >= 1; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ int wave_max_i(int v) {
    for (int o = 32; o >= 1; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
    return v;
}

}  // namespace mg
