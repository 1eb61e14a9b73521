// Fused Adam and selective (row-masked) Adam.
//
// Both are pure streaming kernels: 28 bytes of HBM traffic per parameter
// element (read p, g, m, v; write p, m, v) and a handful of flops, so the only
// design goals are full-width coalesced access, enough bytes in flight per CU,
// and one launch for every parameter group of a step.
//
// Formula (torch.optim.Adam, eps after the sqrt(bias_correction2) divide), as
// in metal_gauss/csrc/adam.metal:34-41 with bc1/sqrt(bc2) formed in double on
// the host (rasterize.mm:338-342):
//     m = b1 m + (1-b1) g
//     v = b2 v + (1-b2) g^2
//     p -= (lr / bc1) * m / (sqrt(v) / sqrt(bc2) + eps)
// The selective / dense-auxiliary variant of metal_gauss/selective_adam.py
// (lines 144-148, 182-186, 201-206) puts eps inside instead:
//     p -= lr * sqrt(bc2) / bc1 * m / (sqrt(v) + eps)
#include <algorithm>
#include <cmath>

#include "mg_common.h"

namespace mg {

constexpr int kAdamMaxTensors = 32;

// Every parameter byte is touched exactly once per step, so the vector path
// uses non-temporal loads and stores: they stream past the caches instead of
// evicting the rest of the step's working set (measured +5% bandwidth for
// this 4-read / 3-write mix).
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld_stream(const float *q) {
    const v4f v = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(q));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_stream(float *q, const float4 &a) {
    v4f v = {a.x, a.y, a.z, a.w};
    __builtin_nontemporal_store(v, reinterpret_cast<v4f *>(q));
}
constexpr int kAdamThreads = 256;
constexpr int kAdamVec = 4;                       // float4 per thread
constexpr int kAdamElemsPerBlock = kAdamThreads * kAdamVec * 2;  // 2048

struct AdamTensor {
    float *p;
    const float *g;
    float *m;
    float *v;
    int64_t n;
    int32_t block_begin;   // first workgroup of this tensor
    int32_t vec_ok;        // all four pointers 16-byte aligned
    float step_size;       // lr / bc1          (eps_inside: lr*sqrt(bc2)/bc1)
    float inv_sqrt_bc2;    // 1 / sqrt(bc2)     (eps_inside: 1)
};

struct AdamTable {
    AdamTensor t[kAdamMaxTensors];
    int32_t count;
    float b1, b2, omb1, omb2, eps;   // omb = 1 - beta, formed in double
    int32_t eps_inside;
    const int64_t *skip;             // NULL, or do nothing when skip[1] != 0
};

__device__ __forceinline__ void adam_elem(float &p, float g, float &m, float &v,
                                          const AdamTable &tab, float step_size,
                                          float inv_sqrt_bc2, bool eps_inside) {
    adam_update(p, g, m, v, tab.b1, tab.b2, tab.omb1, tab.omb2, tab.eps, step_size,
                inv_sqrt_bc2, eps_inside);
}

__global__ __launch_bounds__(kAdamThreads) void adam_multi_kernel(const AdamTable tab) {
    if (tab.skip && tab.skip[1] != 0) return;
    // Find this workgroup's tensor: a uniform linear scan over <= 32 entries.
    int k = 0;
    const int bid = blockIdx.x;
    while (k + 1 < tab.count && bid >= tab.t[k + 1].block_begin) ++k;
    const AdamTensor &T = tab.t[k];
    const int64_t base = (int64_t)(bid - T.block_begin) * kAdamElemsPerBlock;
    const bool ei = tab.eps_inside != 0;

    const int64_t e0 = base + (int64_t)threadIdx.x * kAdamVec;
    const int64_t e1 = e0 + (int64_t)kAdamThreads * kAdamVec;
    if (T.vec_ok && e1 + kAdamVec <= T.n) {
        // Both float4 of the thread (each instruction covering 4 KB
        // contiguous) are requested before any arithmetic or store: the
        // stores could alias later loads, so the compiler would not hoist
        // them itself, and eight loads in flight per thread instead of four
        // keep more of HBM busy.
        float4 p0 = ld_stream(T.p + e0), p1 = ld_stream(T.p + e1);
        const float4 g0 = ld_stream(T.g + e0), g1 = ld_stream(T.g + e1);
        float4 m0 = ld_stream(T.m + e0), m1 = ld_stream(T.m + e1);
        float4 v0 = ld_stream(T.v + e0), v1 = ld_stream(T.v + e1);
        const float ss = T.step_size, ib = T.inv_sqrt_bc2;
        adam_elem(p0.x, g0.x, m0.x, v0.x, tab, ss, ib, ei);
        adam_elem(p0.y, g0.y, m0.y, v0.y, tab, ss, ib, ei);
        adam_elem(p0.z, g0.z, m0.z, v0.z, tab, ss, ib, ei);
        adam_elem(p0.w, g0.w, m0.w, v0.w, tab, ss, ib, ei);
        adam_elem(p1.x, g1.x, m1.x, v1.x, tab, ss, ib, ei);
        adam_elem(p1.y, g1.y, m1.y, v1.y, tab, ss, ib, ei);
        adam_elem(p1.z, g1.z, m1.z, v1.z, tab, ss, ib, ei);
        adam_elem(p1.w, g1.w, m1.w, v1.w, tab, ss, ib, ei);
        st_stream(T.p + e0, p0);
        st_stream(T.p + e1, p1);
        st_stream(T.m + e0, m0);
        st_stream(T.m + e1, m1);
        st_stream(T.v + e0, v0);
        st_stream(T.v + e1, v1);
    } else if (T.vec_ok) {
        // The tensor's last workgroup.
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int64_t e = base + ((int64_t)r * kAdamThreads + threadIdx.x) * kAdamVec;
            if (e + kAdamVec <= T.n) {
                float4 p = ld_stream(T.p + e);
                const float4 g = ld_stream(T.g + e);
                float4 m = ld_stream(T.m + e);
                float4 v = ld_stream(T.v + e);
                adam_elem(p.x, g.x, m.x, v.x, tab, T.step_size, T.inv_sqrt_bc2, ei);
                adam_elem(p.y, g.y, m.y, v.y, tab, T.step_size, T.inv_sqrt_bc2, ei);
                adam_elem(p.z, g.z, m.z, v.z, tab, T.step_size, T.inv_sqrt_bc2, ei);
                adam_elem(p.w, g.w, m.w, v.w, tab, T.step_size, T.inv_sqrt_bc2, ei);
                st_stream(T.p + e, p);
                st_stream(T.m + e, m);
                st_stream(T.v + e, v);
            } else {
                for (int64_t i = e; i < T.n && i < e + kAdamVec; ++i) {
                    float p = T.p[i], m = T.m[i], v = T.v[i];
                    adam_elem(p, T.g[i], m, v, tab, T.step_size, T.inv_sqrt_bc2, ei);
                    T.p[i] = p; T.m[i] = m; T.v[i] = v;
                }
            }
        }
    } else {
        for (int r = 0; r < kAdamElemsPerBlock / kAdamThreads; ++r) {
            const int64_t i = base + (int64_t)r * kAdamThreads + threadIdx.x;
            if (i < T.n) {
                float p = T.p[i], m = T.m[i], v = T.v[i];
                adam_elem(p, T.g[i], m, v, tab, T.step_size, T.inv_sqrt_bc2, ei);
                T.p[i] = p; T.m[i] = m; T.v[i] = v;
            }
        }
    }
}

// ------------------------------------------------------------ selective Adam
// One workgroup owns a run of consecutive rows of one tensor (T.block_rows of
// them), so the per-row step count can be read, bumped and written back
// without any other workgroup touching it.
//
// Writes go to HBM in whole 64-byte chunks or not at all, because a partly
// written chunk costs the memory side a read-modify-write (measured at
// config 3: skipping per 32 or 16 bytes made the kernel 9% and 14% slower
// than per 64, for less data moved). With 16-byte aligned tensors:
//  * narrow tensors (fewer than 16 floats per row: means, scales, quats,
//    opacity, the DC band) hold one or more rows per chunk, so at any useful
//    visibility almost every chunk has a visible row. They are moved whole
//    as float4s (visible elements updated, the others stored back
//    unchanged), and their loads are issued before the step-count prologue,
//    whose latency they then overlap. A block holds at most 2048 floats (two
//    float4s per thread).
//  * wide tensors (16 floats or more per row, e.g. the 45-float SH rest) span
//    at most two rows per chunk; a chunk with no visible row is skipped, the
//    others are moved whole. Their blocks are short (64 rows: measured 30 us
//    faster than 256 at config 3, the long blocks' serial prologue and tail
//    no longer dominating), and the host puts the widest tensors first.
//  * the step counts (one float per row) are moved whole as well.
// Each visible element's arithmetic is the same on every path.
constexpr int kSelRowsMax = 1024;
constexpr int kSelRowsWide = 64;
constexpr int kSelWideMin = 16;            // floats per row of a wide tensor
constexpr int kSelDenseFloats = 2048;      // floats per narrow-tensor block

struct SelTensor {
    float *p;
    const float *g;
    float *m;
    float *v;
    float *steps;
    int64_t rows;
    int32_t width;
    int32_t block_begin;
    int32_t block_rows;   // rows per workgroup
    float lr;
    // ceil(2^32 / width) when 1 < width < 256 (1 when width is 1), else 0:
    // then an element index e < block_rows * width < 2^16 has row
    // __umulhi(e, wmagic) exactly (the round-up error times e stays below
    // 2^32).
    uint32_t wmagic;
    // 0: element by element; 1: narrow, moved whole; 2: wide, chunk-skipped.
    int32_t mode;
};

struct SelTable {
    SelTensor t[kAdamMaxTensors];
    int32_t count;
    float b1, b2, omb1, omb2, eps;   // omb = 1 - beta, formed in double
    const uint8_t *visible;
    int64_t n_visible;
    double l2b1, l2b2;               // log2 of the fp32 betas, in double
    const int64_t *skip;             // NULL, or do nothing when skip[1] != 0
};

// Rows a workgroup of a tensor of this width owns on each path.
inline int sel_block_rows(int width, int mode) {
    if (mode != 1) return kSelRowsWide;
    int r = kSelRowsMax;
    while (r * width > kSelDenseFloats) r >>= 1;
    return r;
}

__device__ __forceinline__ void sel_update(float &p, float g, float &m, float &v, float ss,
                                           float b1, float b2, float omb1, float omb2,
                                           float eps) {
    const float mn = m * b1 + g * omb1;
    const float vn = v * b2 + g * g * omb2;
    p = p - ss * mn / (sqrtf(vn) + eps);
    m = mn;
    v = vn;
}

// Element e of float4s of p, g, m, v.
__device__ __forceinline__ void sel_update4(v4f &p, const v4f &g, v4f &m, v4f &v, int e,
                                            float ss, float b1, float b2, float omb1,
                                            float omb2, float eps) {
    float pe = p[e], me = m[e], ve = v[e];
    sel_update(pe, g[e], me, ve, ss, b1, b2, omb1, omb2, eps);
    p[e] = pe;
    m[e] = me;
    v[e] = ve;
}

__global__ __launch_bounds__(kAdamThreads) void selective_adam_kernel(const SelTable tab) {
    __shared__ float s_step_size[kSelRowsMax];
    __shared__ uint8_t s_vis[kSelRowsMax];

    if (tab.skip && tab.skip[1] != 0) return;
    int k = 0;
    const int bid = blockIdx.x;
    while (k + 1 < tab.count && bid >= tab.t[k + 1].block_begin) ++k;
    const SelTensor &T = tab.t[k];
    const int R = T.block_rows;
    const int64_t r0 = (int64_t)(bid - T.block_begin) * R;
    const int nrows = (int)min((int64_t)R, T.rows - r0);
    const int64_t e0 = r0 * T.width;
    const int ne = nrows * T.width;
    const int n4 = ne >> 2;
    const float b1 = tab.b1, b2 = tab.b2, omb1 = tab.omb1, omb2 = tab.omb2, eps = tab.eps;
    const v4f *g4 = reinterpret_cast<const v4f *>(T.g + e0);
    v4f *m4 = reinterpret_cast<v4f *>(T.m + e0);
    v4f *v4 = reinterpret_cast<v4f *>(T.v + e0);
    v4f *p4 = reinterpret_cast<v4f *>(T.p + e0);
    auto row_of = [&](uint32_t le) {
        return T.width == 1 ? (int)le : (int)__umulhi(le, T.wmagic);
    };

    // Narrow tensors: every float4 of the block is loaded now (n4 <= kD * 256).
    constexpr int kD = kSelDenseFloats / 4 / kAdamThreads;
    v4f gq[kD], mq[kD], vq[kD], pq[kD];
    if (T.mode == 1) {
#pragma unroll
        for (int u = 0; u < kD; ++u) {
            const int q = (int)threadIdx.x + u * kAdamThreads;
            if (q < n4) {
                gq[u] = __builtin_nontemporal_load(g4 + q);
                mq[u] = __builtin_nontemporal_load(m4 + q);
                vq[u] = __builtin_nontemporal_load(v4 + q);
                pq[u] = __builtin_nontemporal_load(p4 + q);
            }
        }
    }

    for (int t = threadIdx.x; t < R; t += kAdamThreads) {
        const int64_t r = r0 + t;
        // On the whole-line paths the block's step counts are read (with
        // the mask, not after it) and written whole, an invisible row's
        // stored back unchanged.
        const bool whole = t < nrows && T.mode != 0;
        float k0 = whole ? T.steps[r] : 0.f;
        uint8_t vis = 0;
        if (t < nrows && r < tab.n_visible) vis = tab.visible[r] != 0;
        if (vis && !whole) k0 = T.steps[r];
        float ss = 0.f;
        if (vis) {
            // Per-row bias correction in fp32, as torch evaluates
            // 1 - b ** steps on a float32 tensor (b the fp32 beta). The
            // power is formed in double as exp2(k log2 b), with log2 b from
            // the host: relative error ~1e-14 for any step count, far below
            // fp32's, at a fraction of a double pow's cost.
            const float kf = k0 + 1.0f;
            const float pw1 = (float)exp2((double)kf * tab.l2b1);
            const float pw2 = (float)exp2((double)kf * tab.l2b2);
            const float bc1 = 1.0f - pw1;
            const float bc2 = 1.0f - pw2;
            ss = T.lr * (sqrtf(bc2) / bc1);
            T.steps[r] = kf;
        } else if (whole) {
            T.steps[r] = k0;
        }
        s_step_size[t] = ss;
        s_vis[t] = vis;
    }
    __syncthreads();

    if (T.mode == 1) {
#pragma unroll
        for (int u = 0; u < kD; ++u) {
            const int q = (int)threadIdx.x + u * kAdamThreads;
            if (q >= n4) continue;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = row_of(4u * (uint32_t)q + e);
                if (!s_vis[row]) continue;
                sel_update4(pq[u], gq[u], mq[u], vq[u], e, s_step_size[row], b1, b2, omb1,
                            omb2, eps);
            }
            __builtin_nontemporal_store(mq[u], m4 + q);
            __builtin_nontemporal_store(vq[u], v4 + q);
            __builtin_nontemporal_store(pq[u], p4 + q);
        }
    } else if (T.mode == 2) {
        // A chunk is 4 float4s; chunk c holds elements of rows row_of(16 c)
        // through row_of(16 c + 15), at most two rows as width >= 16.
        constexpr int kU = 2;
        for (int q0 = threadIdx.x; q0 < n4; q0 += kU * kAdamThreads) {
            v4f gw[kU], mw[kU], vw[kU], pw[kU];
            bool on[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const int q = q0 + u * kAdamThreads;
                const uint32_t first = (uint32_t)(q >> 2) * 16u;
                const uint32_t last = min(first + 15u, (uint32_t)ne - 1u);
                on[u] = q < n4 && (s_vis[min(row_of(first), R - 1)] |
                                   s_vis[min(row_of(last), R - 1)]);
                if (on[u]) {
                    gw[u] = __builtin_nontemporal_load(g4 + q);
                    mw[u] = __builtin_nontemporal_load(m4 + q);
                    vw[u] = __builtin_nontemporal_load(v4 + q);
                    pw[u] = __builtin_nontemporal_load(p4 + q);
                }
            }
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                if (!on[u]) continue;
                const int q = q0 + u * kAdamThreads;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int row = row_of(4u * (uint32_t)q + e);
                    if (!s_vis[row]) continue;
                    sel_update4(pw[u], gw[u], mw[u], vw[u], e, s_step_size[row], b1, b2,
                                omb1, omb2, eps);
                }
                __builtin_nontemporal_store(mw[u], m4 + q);
                __builtin_nontemporal_store(vw[u], v4 + q);
                __builtin_nontemporal_store(pw[u], p4 + q);
            }
        }
    }
    // Elements past the block's last float4 (whole-line paths), or all of
    // them (element path), one by one.
    for (int le = (T.mode != 0 ? 4 * n4 : 0) + (int)threadIdx.x; le < ne;
         le += kAdamThreads) {
        const int row = T.wmagic != 0 ? row_of((uint32_t)le) : le / T.width;
        if (!s_vis[row]) continue;
        const int64_t i = e0 + le;
        float pp = __builtin_nontemporal_load(T.p + i);
        float mm = __builtin_nontemporal_load(T.m + i);
        float vv = __builtin_nontemporal_load(T.v + i);
        sel_update(pp, __builtin_nontemporal_load(T.g + i), mm, vv, s_step_size[row], b1, b2,
                   omb1, omb2, eps);
        __builtin_nontemporal_store(mm, T.m + i);
        __builtin_nontemporal_store(vv, T.v + i);
        __builtin_nontemporal_store(pp, T.p + i);
    }
}

}  // namespace mg

using namespace mg;

extern "C" {

int32_t mg_adam_step_multi(int32_t count, float *const *p, const float *const *g,
                           float *const *m, float *const *v, const int64_t *n,
                           const double *lr, const int64_t *step, double beta1,
                           double beta2, double eps, int32_t eps_inside,
                           mg_stream_t stream) {
    return mg_adam_step_multi_guarded(count, p, g, m, v, n, lr, step, beta1, beta2, eps,
                                      eps_inside, nullptr, stream);
}

int32_t mg_adam_step_multi_guarded(int32_t count, float *const *p, const float *const *g,
                                   float *const *m, float *const *v, const int64_t *n,
                                   const double *lr, const int64_t *step, double beta1,
                                   double beta2, double eps, int32_t eps_inside,
                                   const int64_t *skip, mg_stream_t stream) {
    MG_REQUIRE(count >= 0 && count <= kAdamMaxTensors,
               "mg_adam_step_multi: %d tensors, at most %d per launch", count,
               kAdamMaxTensors);
    // The moments use fp32 betas (as the reference kernel, adam.metal:35-36);
    // the bias corrections and step size are formed in double from the exact
    // hyperparameters, as torch and rasterize.mm:338-342 do.
    AdamTable tab{};
    tab.b1 = (float)beta1;
    tab.b2 = (float)beta2;
    tab.omb1 = (float)(1.0 - beta1);   // torch's lerp weight / addcmul value
    tab.omb2 = (float)(1.0 - beta2);
    tab.eps = (float)eps;
    tab.eps_inside = eps_inside;
    tab.skip = skip;
    int64_t blocks = 0;
    int c = 0;
    for (int i = 0; i < count; ++i) {
        MG_REQUIRE(n[i] >= 0, "mg_adam_step_multi: tensor %d has negative size", i);
        if (n[i] == 0) continue;
        MG_REQUIRE(p[i] && g[i] && m[i] && v[i],
                   "mg_adam_step_multi: tensor %d has a null pointer", i);
        MG_REQUIRE(step[i] >= 1, "mg_adam_step_multi: tensor %d step %lld < 1", i,
                   (long long)step[i]);
        AdamTensor &T = tab.t[c++];
        T.p = p[i]; T.g = g[i]; T.m = m[i]; T.v = v[i]; T.n = n[i];
        T.block_begin = (int32_t)blocks;
        T.vec_ok = ((((uintptr_t)p[i]) | ((uintptr_t)g[i]) | ((uintptr_t)m[i]) |
                     ((uintptr_t)v[i])) & 15) == 0;
        const double bc1 = 1.0 - std::pow((double)beta1, (double)step[i]);
        const double bc2 = 1.0 - std::pow((double)beta2, (double)step[i]);
        if (eps_inside) {
            T.step_size = (float)(lr[i] * std::sqrt(bc2) / bc1);
            T.inv_sqrt_bc2 = 1.0f;
        } else {
            T.step_size = (float)(lr[i] / bc1);
            T.inv_sqrt_bc2 = (float)(1.0 / std::sqrt(bc2));
        }
        blocks += ceil_div(n[i], kAdamElemsPerBlock);
    }
    tab.count = c;
    if (c == 0) return MG_OK;
    MG_REQUIRE(blocks < (1LL << 31), "mg_adam_step_multi: too many elements");
    TimedScope ts("adam_step", as_stream(stream));
    adam_multi_kernel<<<(unsigned)blocks, kAdamThreads, 0, as_stream(stream)>>>(tab);
    MG_LAUNCHED("adam_multi_kernel");
    return MG_OK;
}

int32_t mg_adam_step(float *p, const float *g, float *m, float *v, int64_t n,
                     double lr, double beta1, double beta2, double eps, int64_t step,
                     mg_stream_t stream) {
    return mg_adam_step_multi(1, &p, &g, &m, &v, &n, &lr, &step, beta1, beta2,
                              eps, 0, stream);
}

int32_t mg_selective_adam_step(int32_t count, float *const *p,
                               const float *const *g, float *const *m,
                               float *const *v, float *const *steps,
                               const int64_t *rows, const int32_t *width,
                               const float *lr, const uint8_t *visible,
                               int64_t n_visible, double beta1, double beta2,
                               double eps, mg_stream_t stream) {
    return mg_selective_adam_step_guarded(count, p, g, m, v, steps, rows, width, lr, visible,
                                          n_visible, beta1, beta2, eps, nullptr, stream);
}

int32_t mg_selective_adam_step_guarded(int32_t count, float *const *p,
                                       const float *const *g, float *const *m,
                                       float *const *v, float *const *steps,
                                       const int64_t *rows, const int32_t *width,
                                       const float *lr, const uint8_t *visible,
                                       int64_t n_visible, double beta1, double beta2,
                                       double eps, const int64_t *skip, mg_stream_t stream) {
    MG_REQUIRE(count >= 0 && count <= kAdamMaxTensors,
               "mg_selective_adam_step: %d tensors, at most %d per launch", count,
               kAdamMaxTensors);
    MG_REQUIRE(n_visible >= 0 && (n_visible == 0 || visible),
               "mg_selective_adam_step: null visibility mask");
    SelTable tab{};
    tab.b1 = beta1;
    tab.b2 = beta2;
    tab.omb1 = (float)(1.0 - (double)beta1);
    tab.omb2 = (float)(1.0 - (double)beta2);
    tab.eps = eps;
    tab.visible = visible;
    tab.n_visible = n_visible;
    tab.l2b1 = std::log2((double)tab.b1);
    tab.l2b2 = std::log2((double)tab.b2);
    tab.skip = skip;
    // Widest tensors first: their workgroups are the longest, and the short
    // ones then fill the tail of the launch.
    int order[kAdamMaxTensors];
    for (int i = 0; i < count; ++i) order[i] = i;
    std::stable_sort(order, order + count,
                     [&](int a, int b) { return width[a] > width[b]; });
    int64_t blocks = 0;
    int c = 0;
    for (int oi = 0; oi < count; ++oi) {
        const int i = order[oi];
        MG_REQUIRE(rows[i] >= 0 && width[i] >= 1,
                   "mg_selective_adam_step: tensor %d has rows %lld width %d", i,
                   (long long)rows[i], width[i]);
        MG_REQUIRE(rows[i] >= n_visible,
                   "mg_selective_adam_step: tensor %d has %lld rows, fewer than the "
                   "%lld-entry visibility mask", i, (long long)rows[i],
                   (long long)n_visible);
        if (rows[i] == 0) continue;
        MG_REQUIRE(p[i] && g[i] && m[i] && v[i] && steps[i],
                   "mg_selective_adam_step: tensor %d has a null pointer", i);
        SelTensor &T = tab.t[c++];
        T.p = p[i]; T.g = g[i]; T.m = m[i]; T.v = v[i]; T.steps = steps[i];
        T.rows = rows[i];
        T.width = width[i];
        // (Width 1 needs no division; any non-zero marker selects the fast path.)
        T.wmagic = width[i] == 1 ? 1u : width[i] < 256
            ? (uint32_t)(((1ULL << 32) + (uint64_t)width[i] - 1) / (uint64_t)width[i]) : 0u;
        T.lr = lr[i];
        const bool aligned = (((uintptr_t)p[i] | (uintptr_t)g[i] | (uintptr_t)m[i] |
                               (uintptr_t)v[i] | (uintptr_t)steps[i]) & 15) == 0;
        T.mode = !aligned || T.wmagic == 0 ? 0 : width[i] < kSelWideMin ? 1 : 2;
        T.block_rows = sel_block_rows(width[i], T.mode);
        T.block_begin = (int32_t)blocks;
        blocks += ceil_div(rows[i], (int64_t)T.block_rows);
    }
    tab.count = c;
    if (c == 0) return MG_OK;
    MG_REQUIRE(blocks < (1LL << 31), "mg_selective_adam_step: too many rows");
    TimedScope ts("selective_adam_step", as_stream(stream));
    selective_adam_kernel<<<(unsigned)blocks, kAdamThreads, 0, as_stream(stream)>>>(tab);
    MG_LAUNCHED("selective_adam_kernel");
    return MG_OK;
}

}  // extern "C"
