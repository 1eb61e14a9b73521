// MCMC densification on the GPU (metal_gauss/mcmc.py, 3DGS-MCMC).
//
// add_noise (mcmc.py:164-192): per Gaussian, eps = z * exp(log_scales) with
//   z ~ N(0, I), rotated into the Gaussian's frame by its normalised
//   quaternion (v' = v + 2w (u x v) + 2 u x (u x v)), gated by
//   sigmoid(-100 (opacity - gate)) and scaled by lr * weight, added to the
//   mean. One pass: reads 44 bytes and writes 12 per Gaussian.
//
// relocate (mcmc.py:52-104) and grow (mcmc.py:124-161): sources are drawn
//   with replacement in proportion to a weight, then each source's opacity is
//   split N ways, o' = 1 - (1 - o)^(1/N), and its scale shrunk by
//   sqrt(clamp(o' / (N o'), 0.05, 1)) (eq. 9 of the MCMC paper). Copies land
//   at the destinations (dead rows, or rows active..target), the sources get
//   the same split, and the Adam moments (and SelectiveAdam's per-row step
//   counts) of every touched row are zeroed (mcmc.py:107-121).
//
// Sampling is by inverse CDF: a double-precision inclusive scan of the
// weights over the candidate rows (dead rows weigh 0, so they are never
// drawn), then one binary search per draw. Draw j's uniform comes from
// Philox4x64-10 (Salmon et al., SC'11) with counter (j, 0, 0, 0) and a key
// from the caller's seed, so a seed fixes every draw. Multiplicities are
// counted with integer atomics. Copies and source updates are separate
// launches: every copy reads its source before any source is rewritten.
//
// The per-row work runs one wave per touched row over the concatenated
// columns of all parameter and optimizer-state tensors (59 + 118 floats per
// row for a 3DGS parameter set), so each tensor row is a contiguous span.
#include "mg_common.h"

namespace mg {

// ------------------------------------------------------------- Philox4x64
struct U64x4 {
    uint64_t x[4];
};

__device__ __forceinline__ U64x4 philox4x64(uint64_t c0, uint64_t c1, uint64_t c2, uint64_t c3,
                                            uint64_t k0, uint64_t k1) {
    constexpr uint64_t kM0 = 0xD2E7470EE14C6C93ull, kM1 = 0xCA5A826395121157ull;
    constexpr uint64_t kW0 = 0x9E3779B97F4A7C15ull, kW1 = 0xBB67AE8584CAA73Bull;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        if (r) { k0 += kW0; k1 += kW1; }
        const uint64_t hi0 = __umul64hi(kM0, c0), lo0 = kM0 * c0;
        const uint64_t hi1 = __umul64hi(kM1, c2), lo1 = kM1 * c2;
        const uint64_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
        c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
    }
    return U64x4{{c0, c1, c2, c3}};
}

// 24-bit uniform in (0, 1), never 0: (top 24 bits + 1/2) / 2^24.
__device__ __forceinline__ float u01f(uint64_t x) {
    return ((float)(uint32_t)(x >> 40) + 0.5f) * 5.9604644775390625e-8f;
}
// 53-bit uniform in (0, 1), never 0.
__device__ __forceinline__ double u01d(uint64_t x) {
    return ((double)(x >> 11) + 0.5) * 1.1102230246251565e-16;
}

// Three standard normals for row i: Box-Muller on the block's four uniforms.
__device__ __forceinline__ void normals3(uint64_t i, uint64_t k0, uint64_t k1, float z[3]) {
    const U64x4 r = philox4x64(i, 0, 0, 0, k0, k1);
    const float r0 = sqrtf(-2.0f * logf(u01f(r.x[0])));
    const float t0 = 6.2831853071795864f * u01f(r.x[1]);
    const float r1 = sqrtf(-2.0f * logf(u01f(r.x[2])));
    const float t1 = 6.2831853071795864f * u01f(r.x[3]);
    z[0] = r0 * cosf(t0);
    z[1] = r0 * sinf(t0);
    z[2] = r1 * cosf(t1);
}

__device__ __forceinline__ float sigmoidf(float x) { return 1.0f / (1.0f + expf(-x)); }

// --------------------------------------------------------------- add_noise
struct NoiseArgs {
    float *means;
    const float *log_scales, *quats, *logit, *eps;   // eps (n,3) or null: Philox normals
    int64_t n;
    float lr, weight, gate;
    uint64_t k0, k1;
};

__global__ __launch_bounds__(256) void add_noise_kernel(const NoiseArgs A) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= A.n) return;
    const float op = sigmoidf(A.logit[i]);
    const float gate = sigmoidf(-100.0f * (op - A.gate));
    float z[3];
    if (A.eps) {
        z[0] = A.eps[3 * i]; z[1] = A.eps[3 * i + 1]; z[2] = A.eps[3 * i + 2];
    } else {
        normals3((uint64_t)i, A.k0, A.k1, z);
    }
    const float e0 = z[0] * expf(A.log_scales[3 * i]);
    const float e1 = z[1] * expf(A.log_scales[3 * i + 1]);
    const float e2 = z[2] * expf(A.log_scales[3 * i + 2]);
    float qw = A.quats[4 * i], qx = A.quats[4 * i + 1], qy = A.quats[4 * i + 2],
          qz = A.quats[4 * i + 3];
    const float inv = 1.0f / fmaxf(sqrtf(qw * qw + qx * qx + qy * qy + qz * qz), 1e-12f);
    qw *= inv; qx *= inv; qy *= inv; qz *= inv;
    // t = 2 u x eps; world = eps + w t + u x t
    const float t0 = 2.0f * (qy * e2 - qz * e1);
    const float t1 = 2.0f * (qz * e0 - qx * e2);
    const float t2 = 2.0f * (qx * e1 - qy * e0);
    const float w0 = e0 + qw * t0 + (qy * t2 - qz * t1);
    const float w1 = e1 + qw * t1 + (qz * t0 - qx * t2);
    const float w2 = e2 + qw * t2 + (qx * t1 - qy * t0);
    A.means[3 * i] += w0 * gate * A.lr * A.weight;
    A.means[3 * i + 1] += w1 * gate * A.lr * A.weight;
    A.means[3 * i + 2] += w2 * gate * A.lr * A.weight;
}

// ------------------------------------------------------- weights and scan
constexpr int kScanThreads = 256;
constexpr int kScanItems = 4;
constexpr int kScanBlock = kScanThreads * kScanItems;
constexpr int kMaxTensors = 32;

// Totals written by the scan's middle pass; read by the host once.
struct McmcTotals {
    double sum_w, sum_o;      // drawn candidate weights; the opacity fallback
    int64_t n_dead;           // rows below the threshold (relocate)
    int32_t nonfinite;        // some candidate weight is inf or nan
    int32_t has_pos;          // some candidate's weight (before grow's 1e-8 floor) is > 0
};

struct WeightArgs {
    const float *logit, *weights;   // weights may be null (use opacity)
    int64_t n;
    float thresh;                   // relocate: dead below; grow: <= 0 (all candidates)
    int32_t grow;                   // grow clamps the drawn weights at 1e-8
    int32_t use_opac;               // scan the opacity fallback instead of the weights
};

// Candidate weight of row i (0 for a dead row under relocate) and the
// opacity fallback's, as drawn; whether the row is dead; whether its weight
// is inf or nan (the reference's clamp_min(0) keeps a nan, fmaxf would not,
// so the raw value is tested); whether it is positive before grow's floor.
__device__ __forceinline__ void row_weights(const WeightArgs &W, int64_t i, double &w, double &o,
                                            bool &dead, bool &bad, bool &pos) {
    const float op = sigmoidf(W.logit[i]);
    dead = !W.grow && op < W.thresh;
    const float raw = W.weights ? W.weights[i] : op;
    float wf = fmaxf(raw, 0.0f);
    bad = !dead && (isnan(raw) || isinf(wf));
    pos = !dead && wf > 0.0f;
    float of = op;
    if (W.grow) { wf = fmaxf(wf, 1e-8f); of = fmaxf(of, 1e-8f); }
    w = dead || bad ? 0.0 : (double)wf;
    o = dead ? 0.0 : (double)of;
}

template <class T>
__device__ __forceinline__ T block_sum(T v, T *s_w) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) s_w[wave] = v;
    __syncthreads();
    T t = 0;
    for (int k = 0; k < kScanThreads / 64; ++k) t += s_w[k];
    return t;
}

// Pass 1: per block, the sums of both weight arrays, dead count, non-finite
// flag; also zeroes the multiplicity counts of the block's rows.
__global__ __launch_bounds__(kScanThreads) void mcmc_reduce_kernel(const WeightArgs W,
                                                                   double *blk_w, double *blk_o,
                                                                   int64_t *blk_dead,
                                                                   int32_t *blk_bad,
                                                                   int32_t *counts) {
    __shared__ double s_d[kScanThreads / 64];
    __shared__ int64_t s_i[kScanThreads / 64];
    const int64_t base = (int64_t)blockIdx.x * kScanBlock;
    double sw = 0.0, so = 0.0;
    int64_t nd = 0;
    int bad = 0, pos = 0;
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t i = base + (int64_t)k * kScanThreads + threadIdx.x;
        if (i < W.n) {
            double w, o;
            bool dead, b, ps;
            row_weights(W, i, w, o, dead, b, ps);
            sw += w; so += o; nd += dead ? 1 : 0; bad |= b ? 1 : 0; pos |= ps ? 1 : 0;
            counts[i] = 0;
        }
    }
    sw = block_sum(sw, s_d);
    so = block_sum(so, s_d);
    nd = block_sum(nd, s_i);
    const int anybad = __syncthreads_or(bad);
    const int anypos = __syncthreads_or(pos);
    if (threadIdx.x == 0) {
        blk_w[blockIdx.x] = sw;
        blk_o[blockIdx.x] = so;
        blk_dead[blockIdx.x] = nd;
        blk_bad[blockIdx.x] = anybad | (anypos << 1);
    }
}

// Pass 2 (one workgroup): exclusive scan of the block sums of both arrays in
// place, and the totals.
__global__ __launch_bounds__(1024) void mcmc_block_scan_kernel(double *blk_w, double *blk_o,
                                                               const int64_t *blk_dead,
                                                               const int32_t *blk_bad, int nblk,
                                                               McmcTotals *tot) {
    __shared__ double s_w[16], s_o[16];
    __shared__ double c_w, c_o;
    __shared__ int64_t s_dead;
    __shared__ int32_t s_bad, s_pos;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (threadIdx.x == 0) { c_w = 0.0; c_o = 0.0; s_dead = 0; s_bad = 0; s_pos = 0; }
    __syncthreads();
    for (int b0 = 0; b0 < nblk; b0 += 1024) {
        const int b = b0 + (int)threadIdx.x;
        const double vw = b < nblk ? blk_w[b] : 0.0, vo = b < nblk ? blk_o[b] : 0.0;
        double iw = vw, io = vo;
        for (int o = 1; o < 64; o <<= 1) {
            const double tw = __shfl_up(iw, o, 64), to = __shfl_up(io, o, 64);
            if (lane >= o) { iw += tw; io += to; }
        }
        if (lane == 63) { s_w[wave] = iw; s_o[wave] = io; }
        if (b < nblk) {
            atomicAdd((unsigned long long *)&s_dead, (unsigned long long)blk_dead[b]);
            if (blk_bad[b] & 1) s_bad = 1;
            if (blk_bad[b] & 2) s_pos = 1;
        }
        __syncthreads();
        double pw = c_w, po = c_o;
        for (int w = 0; w < wave; ++w) { pw += s_w[w]; po += s_o[w]; }
        if (b < nblk) { blk_w[b] = pw + iw - vw; blk_o[b] = po + io - vo; }
        __syncthreads();
        if (threadIdx.x == 1023) { c_w = pw + iw; c_o = po + io; }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        tot->sum_w = c_w;
        tot->sum_o = c_o;
        tot->n_dead = s_dead;
        tot->nonfinite = s_bad;
        tot->has_pos = s_pos;
    }
}

// Pass 3: inclusive CDF of the chosen weights (block offset + in-block scan,
// rows in the same order as pass 1).
__global__ __launch_bounds__(kScanThreads) void mcmc_cdf_kernel(const WeightArgs W,
                                                                const double *blk_off,
                                                                double *cdf) {
    __shared__ double s_w[kScanThreads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t base = (int64_t)blockIdx.x * kScanBlock;
    double carry = blk_off[blockIdx.x];
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t i = base + (int64_t)k * kScanThreads + threadIdx.x;
        double v = 0.0;
        if (i < W.n) {
            double w, o;
            bool dead, b, ps;
            row_weights(W, i, w, o, dead, b, ps);
            v = W.use_opac ? o : w;
        }
        double inc = v;
        for (int o = 1; o < 64; o <<= 1) {
            const double t = __shfl_up(inc, o, 64);
            if (lane >= o) inc += t;
        }
        __syncthreads();
        if (lane == 63) s_w[wave] = inc;
        __syncthreads();
        double pre = carry;
        for (int w = 0; w < wave; ++w) pre += s_w[w];
        if (i < W.n) cdf[i] = pre + inc;
        for (int w = wave; w < kScanThreads / 64; ++w) pre += s_w[w];
        carry = pre;   // carry + this round's total, the same in every thread
    }
}

// Weight row i carries in the CDF.
__device__ __forceinline__ double drawn_weight(const WeightArgs &W, int64_t i) {
    double w, o;
    bool dead, b, ps;
    row_weights(W, i, w, o, dead, b, ps);
    return W.use_opac ? o : w;
}

// First index whose CDF exceeds t. The block offsets and the in-block sums
// round in different orders, so the CDF may step back by a few ulps at a
// block boundary, and a draw landing there could name a row of weight 0;
// such a draw moves to the nearest row of positive weight (below, else
// above; the total is positive, so one exists). Its probability is of the
// order of the double rounding, ~1e-16 per draw.
__device__ __forceinline__ int64_t cdf_search(const WeightArgs &W, const double *cdf, int64_t n,
                                              double t) {
    int64_t lo = 0, hi = n - 1;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (cdf[mid] > t) hi = mid; else lo = mid + 1;
    }
    if (drawn_weight(W, lo) > 0.0) return lo;
    for (int64_t k = lo - 1; k >= 0; --k)
        if (drawn_weight(W, k) > 0.0) return k;
    for (int64_t k = lo + 1; k < n; ++k)
        if (drawn_weight(W, k) > 0.0) return k;
    return lo;
}

// Draws. Relocate: one per dead row i < n (counter i); the source is kept at
// the row itself, src[i], and rows that are not dead get -1. Grow: one per
// j < n_draw (counter j), for destination dst0 + j, source src[j].
struct DrawArgs {
    WeightArgs W;
    const double *cdf;
    int64_t n_draw;      // grow only
    uint64_t k0, k1;
    int32_t *src, *counts;
};

__global__ __launch_bounds__(256) void mcmc_draw_kernel(const DrawArgs D) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t n = D.W.n;
    const double last = D.cdf[n - 1];
    if (D.W.grow) {
        if (i >= D.n_draw) return;
    } else {
        if (i >= n) return;
        double w, o;
        bool dead, b, ps;
        row_weights(D.W, i, w, o, dead, b, ps);
        if (!dead) {
            D.src[i] = -1;
            return;
        }
    }
    const U64x4 r = philox4x64((uint64_t)i, 0, 0, 0, D.k0, D.k1);
    const int64_t s = cdf_search(D.W, D.cdf, n, u01d(r.x[0]) * last);
    D.src[i] = (int32_t)s;
    atomicAdd(&D.counts[s], 1);
}

// ------------------------------------------------------ per-row updates
struct RowTensors {
    float *p[kMaxTensors];
    int32_t width[kMaxTensors];   // floats per row
    int32_t kind[kMaxTensors];    // 0 copied param, 1 log-scales, 2 logit, 3 zeroed state
    int32_t col0[kMaxTensors];    // first column of each tensor in a row's concatenation
    int32_t cols;                 // columns of all tensors
    int32_t src_col0[kMaxTensors];   // the same over the tensors a source update touches
    int32_t src_cols;             // (kinds 1-3; copied tensors sit below column 0)
    int32_t count;
};

constexpr int kMaxMult = 51;      // mcmc.py:33

// The N-way split of opacity o: the new opacity, its logit and the log of
// the scale ratio (mcmc.py:43-49, 80-87).
__device__ __forceinline__ void split(float o, float n, float &logit_new, float &log_ratio) {
    const float o_new = 1.0f - powf(fmaxf(1.0f - o, 1e-6f), 1.0f / n);
    logit_new = logf(fminf(fmaxf(o_new, 1e-6f), 1.0f - 1e-6f) / fmaxf(1.0f - o_new, 1e-6f));
    const float denom = fmaxf(fmaxf(n, 1.0f) * fmaxf(o_new, 1e-6f), 1e-6f);
    const float ratio = sqrtf(fminf(fmaxf(o_new / denom, 0.05f), 1.0f));
    log_ratio = logf(ratio);
}

__device__ __forceinline__ float multiplicity(const int32_t *counts, int64_t s, int grow) {
    const int c = min(max(counts[s], 1), kMaxMult) + (grow ? 1 : 0);
    return (float)c;
}

enum RowMode { kRelocateCopies = 0, kGrowCopies = 1, kSources = 2 };

// One workgroup per `chunk` candidates (a power of two up to 256, chosen so
// that a workgroup holds about one selected row per wave): the selected ones
// (relocate: dead rows; grow: every draw; sources: rows drawn at least once)
// are compacted in LDS, then each wave takes one selected row at a time and
// spreads the row's columns, across every tensor, over its 64 lanes. The
// tensor table sits in LDS, where each lane finds its column's tensor.
//   copies:  destination <- source, logit <- split logit, log-scales <-
//            source's + log ratio, optimizer state <- 0;
//   sources: logit <- split logit, log-scales += log ratio, state <- 0.
template <int MODE>
__global__ __launch_bounds__(256) void mcmc_rows_kernel(const RowTensors R, const int32_t *src,
                                                        const int32_t *counts,
                                                        const float *logit, int64_t n_cand,
                                                        int64_t dst0, int grow, int chunk) {
    __shared__ float *s_p[kMaxTensors];
    __shared__ int32_t s_w[kMaxTensors], s_kind[kMaxTensors], s_col0[kMaxTensors];
    __shared__ int32_t s_list[256];
    __shared__ int32_t s_cnt;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < R.count) {
        s_p[tid] = R.p[tid];
        s_w[tid] = R.width[tid];
        s_kind[tid] = R.kind[tid];
        s_col0[tid] = MODE == kSources ? R.src_col0[tid] : R.col0[tid];
    }
    if (tid == 0) s_cnt = 0;
    __syncthreads();
    const int64_t c0 = (int64_t)blockIdx.x * chunk;
    bool sel = false;
    if (tid < chunk && c0 + tid < n_cand) {
        if (MODE == kRelocateCopies) sel = src[c0 + tid] >= 0;
        else if (MODE == kGrowCopies) sel = true;
        else sel = counts[c0 + tid] > 0;
    }
    const uint64_t m = ballot(sel);
    int base = 0;
    if (lane == 0 && m) base = atomicAdd(&s_cnt, __popcll(m));
    base = __shfl(base, 0, 64);
    if (sel) s_list[base + rank_in(m)] = tid;
    __syncthreads();
    const int cnt = s_cnt;
    const int cols = MODE == kSources ? R.src_cols : R.cols;
    const int count = R.count;
    for (int e = wave; e < cnt; e += 4) {
        const int64_t ci = c0 + s_list[e];
        int64_t d = 0, sr;
        if (MODE == kRelocateCopies) { d = ci; sr = src[ci]; }
        else if (MODE == kGrowCopies) { d = dst0 + ci; sr = src[ci]; }
        else sr = ci;
        float logit_new, log_ratio;
        split(sigmoidf(logit[sr]), multiplicity(counts, sr, grow), logit_new, log_ratio);
        int t = 0;
        for (int col = lane; col < cols; col += 64) {
            while (t + 1 < count && s_col0[t + 1] <= col) ++t;
            float *p = s_p[t];
            const int64_t w = s_w[t];
            const int k = col - s_col0[t], kind = s_kind[t];
            if (MODE == kSources) {
                if (kind == 3) p[sr * w + k] = 0.0f;
                else if (kind == 2) p[sr * w + k] = logit_new;
                else p[sr * w + k] += log_ratio;
            } else {
                float v;
                if (kind == 3) v = 0.0f;
                else if (kind == 2) v = logit_new;
                else if (kind == 1) v = p[sr * w + k] + log_ratio;
                else v = p[sr * w + k];
                p[d * w + k] = v;
            }
        }
    }
}

inline int64_t scan_blocks(int64_t n) { return ceil_div(n, kScanBlock); }

struct McmcWs {
    McmcTotals *tot;
    double *blk_w, *blk_o, *cdf;
    int64_t *blk_dead;
    int32_t *blk_bad, *counts, *src;
};

// src holds one source per row (relocate) or per draw (grow).
inline int64_t mcmc_ws_bytes(int64_t n, int64_t n_draw) {
    const int64_t nb = scan_blocks(n);
    return align256(sizeof(McmcTotals)) + 2 * align256(8 * nb) + align256(8 * nb) +
           align256(4 * nb) + align256(8 * n) + align256(4 * n) +
           align256(4 * (n > n_draw ? n : n_draw));
}

inline McmcWs mcmc_ws(void *ws, int64_t n, int64_t n_draw) {
    char *p = static_cast<char *>(ws);
    const int64_t nb = scan_blocks(n);
    McmcWs W;
    W.tot = (McmcTotals *)p; p += align256(sizeof(McmcTotals));
    W.blk_w = (double *)p; p += align256(8 * nb);
    W.blk_o = (double *)p; p += align256(8 * nb);
    W.blk_dead = (int64_t *)p; p += align256(8 * nb);
    W.blk_bad = (int32_t *)p; p += align256(4 * nb);
    W.cdf = (double *)p; p += align256(8 * n);
    W.counts = (int32_t *)p; p += align256(4 * n);
    W.src = (int32_t *)p;
    return W;
}

static int32_t row_tensors(RowTensors &R, int32_t n_tensors, float *const *tensors,
                           const int32_t *widths, const int32_t *kinds, const char *who) {
    MG_REQUIRE(n_tensors >= 1 && n_tensors <= kMaxTensors, "%s: %d tensors (1..%d)", who,
               n_tensors, kMaxTensors);
    MG_REQUIRE(tensors && widths && kinds, "%s: null tensor table", who);
    int n_logit = 0, n_scales = 0;
    for (int t = 0; t < n_tensors; ++t) {
        MG_REQUIRE(tensors[t] != nullptr, "%s: tensor %d is null", who, t);
        MG_REQUIRE(widths[t] >= 1, "%s: tensor %d has row width %d", who, t, widths[t]);
        MG_REQUIRE(kinds[t] >= 0 && kinds[t] <= 3, "%s: tensor %d kind %d", who, t, kinds[t]);
        MG_REQUIRE(kinds[t] != 2 || widths[t] == 1, "%s: the logit tensor has width %d", who,
                   widths[t]);
        R.p[t] = tensors[t];
        R.width[t] = widths[t];
        R.kind[t] = kinds[t];
        n_logit += kinds[t] == 2;
        n_scales += kinds[t] == 1;
    }
    MG_REQUIRE(n_logit == 1 && n_scales == 1,
               "%s: need exactly one logit-opacity and one log-scales tensor", who);
    // Copied tensors first for the source update's concatenation: order the
    // table so kinds 1-3 form a suffix, then give both column maps.
    RowTensors S{};
    int k = 0;
    for (int pass = 0; pass < 2; ++pass)
        for (int t = 0; t < n_tensors; ++t)
            if ((R.kind[t] == 0) == (pass == 0)) {
                S.p[k] = R.p[t]; S.width[k] = R.width[t]; S.kind[k] = R.kind[t]; ++k;
            }
    S.count = n_tensors;
    int cols = 0, src_cols = 0;
    for (int t = 0; t < n_tensors; ++t) {
        S.col0[t] = cols;
        cols += S.width[t];
        // Copied tensors take no source columns: they map below column 0.
        S.src_col0[t] = S.kind[t] == 0 ? -(1 << 30) : src_cols;
        if (S.kind[t] != 0) src_cols += S.width[t];
    }
    S.cols = cols;
    S.src_cols = src_cols;
    R = S;
    return MG_OK;
}

}  // namespace mg

using namespace mg;

extern "C" {

int32_t mg_add_noise(int64_t n, float *means, const float *log_scales, const float *quats,
                     const float *logit_opac, const float *eps, float lr_means, float weight,
                     float opacity_gate, uint64_t seed, mg_stream_t stream) {
    MG_REQUIRE(n >= 0, "mg_add_noise: n = %lld", (long long)n);
    if (n == 0) return MG_OK;
    MG_REQUIRE(means && log_scales && quats && logit_opac, "mg_add_noise: null pointer");
    NoiseArgs A{means, log_scales, quats, logit_opac, eps, n, lr_means, weight, opacity_gate,
                seed, 0x6e6f697365ull /* stream tag */};
    hipStream_t s = as_stream(stream);
    TimedScope ts("add_noise", s);
    add_noise_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, s>>>(A);
    MG_LAUNCHED("add_noise_kernel");
    return MG_OK;
}

int64_t mg_mcmc_workspace_bytes(int64_t n_rows, int64_t n_draw) {
    if (n_rows < 0 || n_draw < 0) return 0;
    return mcmc_ws_bytes(n_rows, n_draw);
}

int32_t mg_mcmc_weights(int64_t n, const float *logit_opac, const float *weights, float thresh,
                        int32_t grow, void *ws, int64_t ws_size, int64_t n_draw,
                        double *totals_host, mg_stream_t stream) {
    MG_REQUIRE(n >= 1, "mg_mcmc_weights: n = %lld", (long long)n);
    MG_REQUIRE(logit_opac && ws && totals_host, "mg_mcmc_weights: null pointer");
    MG_REQUIRE(ws_size >= mcmc_ws_bytes(n, n_draw),
               "mg_mcmc_weights: workspace %lld bytes, need %lld", (long long)ws_size,
               (long long)mcmc_ws_bytes(n, n_draw));
    McmcWs Wk = mcmc_ws(ws, n, n_draw);
    WeightArgs W{logit_opac, weights, n, thresh, grow, 0};
    hipStream_t s = as_stream(stream);
    const int64_t nb = scan_blocks(n);
    TimedScope ts("mcmc_weights", s);
    mcmc_reduce_kernel<<<(unsigned)nb, kScanThreads, 0, s>>>(W, Wk.blk_w, Wk.blk_o, Wk.blk_dead,
                                                             Wk.blk_bad, Wk.counts);
    MG_LAUNCHED("mcmc_reduce_kernel");
    mcmc_block_scan_kernel<<<1, 1024, 0, s>>>(Wk.blk_w, Wk.blk_o, Wk.blk_dead, Wk.blk_bad,
                                              (int)nb, Wk.tot);
    MG_LAUNCHED("mcmc_block_scan_kernel");
    McmcTotals t{};
    MG_HIP(hipMemcpyAsync(&t, Wk.tot, sizeof(t), hipMemcpyDeviceToHost, s));
    MG_HIP(hipStreamSynchronize(s));
    totals_host[0] = t.sum_w;
    totals_host[1] = t.sum_o;
    totals_host[2] = (double)t.n_dead;
    totals_host[3] = (double)t.nonfinite;
    totals_host[4] = (double)t.has_pos;
    return MG_OK;
}

int32_t mg_mcmc_apply(int64_t n, const float *logit_opac, const float *weights, float thresh,
                      int32_t grow, int32_t use_opacity, void *ws, int64_t ws_size,
                      int64_t n_draw, int64_t n_dest, int64_t dst0, uint64_t seed,
                      int32_t n_tensors, float *const *tensors, const int32_t *widths,
                      const int32_t *kinds, mg_stream_t stream) {
    MG_REQUIRE(n >= 1, "mg_mcmc_apply: n = %lld", (long long)n);
    MG_REQUIRE(logit_opac && ws, "mg_mcmc_apply: null pointer");
    MG_REQUIRE(ws_size >= mcmc_ws_bytes(n, n_draw),
               "mg_mcmc_apply: workspace %lld bytes, need %lld", (long long)ws_size,
               (long long)mcmc_ws_bytes(n, n_draw));
    MG_REQUIRE(n_dest >= 0 && n_dest <= n_draw, "mg_mcmc_apply: %lld copies for %lld draws",
               (long long)n_dest, (long long)n_draw);
    MG_REQUIRE(grow ? n_dest == n_draw : n_draw >= n,
               "mg_mcmc_apply: relocate needs a draw slot per row");
    RowTensors R{};
    int32_t rc = row_tensors(R, n_tensors, tensors, widths, kinds, "mg_mcmc_apply");
    if (rc != MG_OK) return rc;
    McmcWs Wk = mcmc_ws(ws, n, n_draw);
    WeightArgs W{logit_opac, weights, n, thresh, grow, use_opacity};
    hipStream_t s = as_stream(stream);
    const int64_t nb = scan_blocks(n);
    TimedScope ts("mcmc_apply", s);
    mcmc_cdf_kernel<<<(unsigned)nb, kScanThreads, 0, s>>>(
        W, use_opacity ? Wk.blk_o : Wk.blk_w, Wk.cdf);
    MG_LAUNCHED("mcmc_cdf_kernel");
    DrawArgs D{W, Wk.cdf, grow ? n_draw : 0, seed, 0x7069636bull /* stream tag */, Wk.src,
               Wk.counts};
    const int64_t n_cand = grow ? n_draw : n;
    mcmc_draw_kernel<<<(unsigned)ceil_div(n_cand, 256), 256, 0, s>>>(D);
    MG_LAUNCHED("mcmc_draw_kernel");
    if (n_dest > 0) {
        // About one selected row per wave: copies are n_dest of n_cand
        // candidates, sources at most n_dest of n rows.
        auto chunk_for = [](int64_t sel, int64_t cand) {
            int c = 4;
            while (c < 256 && (double)c * (double)sel < 4.0 * (double)cand) c *= 2;
            return c;
        };
        const int cc = chunk_for(n_dest, n_cand), cs = chunk_for(n_dest, n);
        // Every copy reads its source before the sources are rewritten.
        if (grow)
            mcmc_rows_kernel<kGrowCopies><<<(unsigned)ceil_div(n_cand, cc), 256, 0, s>>>(
                R, Wk.src, Wk.counts, logit_opac, n_cand, dst0, 1, cc);
        else
            mcmc_rows_kernel<kRelocateCopies><<<(unsigned)ceil_div(n_cand, cc), 256, 0, s>>>(
                R, Wk.src, Wk.counts, logit_opac, n_cand, 0, 0, cc);
        MG_LAUNCHED("mcmc_rows_kernel");
        mcmc_rows_kernel<kSources><<<(unsigned)ceil_div(n, cs), 256, 0, s>>>(
            R, Wk.src, Wk.counts, logit_opac, n, 0, grow, cs);
        MG_LAUNCHED("mcmc_rows_kernel");
    }
    return MG_OK;
}

}  // extern "C"
