// Mip-Splatting's 3D filter size per Gaussian (metal_gauss/mipfilter.py:29-73).
//
//   dist  = min over the views that see the Gaussian of its camera depth
//   size  = dist / focal * sqrt(0.2),  focal = max over views of (fx, fy)
//
// A view sees a Gaussian when z > near and the projected centre lies inside
// the frame widened by `margin` on every side. A Gaussian no view sees gets
// the largest distance any seen Gaussian got; if none is seen, every distance
// is 1.
//
// Three launches: a one-thread reset of the running maximum, one thread per
// Gaussian over all views (views staged in LDS in chunks of kViewChunk; the
// seen maximum reduced per wave, then one integer atomic per wave on an
// order-preserving encoding of the float), and a finishing pass that fills
// the unseen and scales. The O(N V) pass reads each mean once.
#include "mg_common.h"

namespace mg {

constexpr int kMipThreads = 256;
constexpr int kViewChunk = 256;
// Per view: R (9, row-major), t (3), fx, fy, cx, cy, then the frame with its
// margin as four bounds u_lo, u_hi, v_lo, v_hi (-margin W, (1 + margin) W,
// -margin H, (1 + margin) H), formed on the host in double and rounded once,
// as the reference's comparisons against Python floats round them.
constexpr int kViewFloats = 20;

// Float -> int32 with the same order (negative floats flipped).
__device__ __forceinline__ int32_t f32_order(float f) {
    const int32_t i = __float_as_int(f);
    return i ^ ((i >> 31) & 0x7fffffff);
}
__device__ __forceinline__ float f32_unorder(int32_t i) {
    return __int_as_float(i ^ ((i >> 31) & 0x7fffffff));
}

constexpr int32_t kNoneSeen = INT32_MIN;

__global__ void mip_reset_kernel(int32_t *seen_max) { *seen_max = kNoneSeen; }

__global__ __launch_bounds__(kMipThreads) void mip_dist_kernel(
    const float *__restrict__ means, int64_t N, const float *__restrict__ views, int32_t V,
    float near_p, float *__restrict__ dist, int32_t *seen_max) {
    __shared__ float sv[kViewChunk * kViewFloats];
    const int64_t g = (int64_t)blockIdx.x * kMipThreads + threadIdx.x;
    const bool in = g < N;
    float mx = 0.f, my = 0.f, mz = 0.f;
    if (in) { mx = means[3 * g]; my = means[3 * g + 1]; mz = means[3 * g + 2]; }
    float d = __builtin_inff();
    for (int v0 = 0; v0 < V; v0 += kViewChunk) {
        const int nv = min(kViewChunk, V - v0);
        __syncthreads();
        for (int e = threadIdx.x; e < nv * kViewFloats; e += kMipThreads)
            sv[e] = views[(int64_t)v0 * kViewFloats + e];
        __syncthreads();
        for (int k = 0; k < nv; ++k) {
            const float *P = sv + k * kViewFloats;
            const float px = P[0] * mx + P[1] * my + P[2] * mz + P[9];
            const float py = P[3] * mx + P[4] * my + P[5] * mz + P[10];
            const float z = P[6] * mx + P[7] * my + P[8] * mz + P[11];
            const float zc = fmaxf(z, 1e-6f);
            const float u = P[12] * px / zc + P[14];
            const float w = P[13] * py / zc + P[15];
            const bool inview = (z > near_p) && (u > P[16]) && (u < P[17]) && (w > P[18]) &&
                                (w < P[19]);
            if (inview) d = fminf(d, z);
        }
    }
    const bool seen = in && d != __builtin_inff();
    if (in) dist[g] = d;
    // Wave maximum of the seen distances, one atomic per wave.
    int32_t m = seen ? f32_order(d) : kNoneSeen;
    for (int o = 32; o >= 1; o >>= 1) m = max(m, __shfl_xor(m, o, 64));
    if ((threadIdx.x & 63) == 0 && m != kNoneSeen) atomicMax(seen_max, m);
}

__global__ __launch_bounds__(kMipThreads) void mip_finish_kernel(float *dist, int64_t N,
                                                                 const int32_t *seen_max,
                                                                 float focal) {
    const int64_t g = (int64_t)blockIdx.x * kMipThreads + threadIdx.x;
    if (g >= N) return;
    const int32_t m = *seen_max;
    float d = dist[g];
    if (m == kNoneSeen) d = 1.0f;
    else if (d == __builtin_inff()) d = f32_unorder(m);
    // (dist / focal) * sqrt(0.2), rounded as mipfilter.py:73 rounds it.
    dist[g] = (d / focal) * 0.4472135954999579f;
}

}  // namespace mg

using namespace mg;

extern "C" {

int32_t mg_compute_3d_filter(int64_t N, const float *means, int32_t n_views, const float *views,
                             float focal, float near_plane, float *filter_3d, int32_t *scratch,
                             mg_stream_t stream) {
    MG_REQUIRE(N >= 0, "mg_compute_3d_filter: N = %lld", (long long)N);
    MG_REQUIRE(n_views >= 0, "mg_compute_3d_filter: %d views", n_views);
    if (N == 0) return MG_OK;
    MG_REQUIRE(means && filter_3d && scratch, "mg_compute_3d_filter: null pointer");
    MG_REQUIRE(n_views == 0 || views, "mg_compute_3d_filter: null views");
    // mipfilter.py:71-72: a non-positive focal length falls back to 1.
    const float f = focal > 0.0f ? focal : 1.0f;
    hipStream_t s = as_stream(stream);
    const unsigned blocks = (unsigned)ceil_div(N, kMipThreads);
    TimedScope ts("compute_3d_filter", s);
    mip_reset_kernel<<<1, 1, 0, s>>>(scratch);
    MG_LAUNCHED("mip_reset_kernel");
    mip_dist_kernel<<<blocks, kMipThreads, 0, s>>>(means, N, views, n_views, near_plane,
                                                   filter_3d, scratch);
    MG_LAUNCHED("mip_dist_kernel");
    mip_finish_kernel<<<blocks, kMipThreads, 0, s>>>(filter_3d, N, scratch, f);
    MG_LAUNCHED("mip_finish_kernel");
    return MG_OK;
}

}  // extern "C"
