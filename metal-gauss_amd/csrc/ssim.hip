// SSIM loss kernels: 11-tap separable Gaussian window (sigma 1.5), zero
// padding as F.conv2d, C1 = 0.01^2, C2 = 0.03^2.
//
// Two families:
//   * the five kernels of the reference's ABI (metal_gauss/csrc/ssim.metal:
//     23-188), same layouts: (H,W,3) images and (15,H,W) moment stacks;
//   * a fused pair. The forward loads an image tile with a 5-pixel halo into
//     LDS, forms the five moments, blurs them horizontally then vertically in
//     LDS, evaluates SSIM and writes the three adjoint maps the backward needs
//     (per colour: dS/dmx, dS/dE[xx], dS/dE[xy], unscaled); the backward blurs
//     those maps the same way (the window is symmetric, so the blur is its own
//     adjoint) and chains through the moments. 60 B/px of HBM traffic in the
//     forward and 48 B/px in the backward, against ~400 B/px for the five-pass
//     chain.
// Math: S = (2 mx my + C1)(2 sxy + C2) / ((mx^2 + my^2 + C1)(sxx + syy + C2))
// (metal_gauss/ssim.py:54-108).
#include <mutex>

#include "mg_common.h"

namespace mg {

constexpr float kSsimC1 = 0.01f * 0.01f;
constexpr float kSsimC2 = 0.03f * 0.03f;
constexpr int kR = 5;   // window radius

// ------------------------------------------------------------ compat kernels
__global__ void ssim_stack_blur_h_kernel(const float *x, const float *y, const float *w, int H,
                                         int W, float *out) {
    const int px = blockIdx.x * blockDim.x + threadIdx.x;
    const int py = blockIdx.y * blockDim.y + threadIdx.y;
    const int c = blockIdx.z;
    if (px >= W || py >= H) return;
    const int64_t N = (int64_t)W * H, row = (int64_t)py * W;
    float sx = 0, sy = 0, sxx = 0, syy = 0, sxy = 0;
    for (int k = -kR; k <= kR; ++k) {
        const int u = px + k;
        if (u < 0 || u >= W) continue;
        const float wk = w[k + kR];
        const float xv = x[(row + u) * 3 + c], yv = y[(row + u) * 3 + c];
        sx += wk * xv;
        sy += wk * yv;
        sxx += wk * xv * xv;
        syy += wk * yv * yv;
        sxy += wk * xv * yv;
    }
    const int64_t o = row + px;
    out[(0 + c) * N + o] = sx;
    out[(3 + c) * N + o] = sy;
    out[(6 + c) * N + o] = sxx;
    out[(9 + c) * N + o] = syy;
    out[(12 + c) * N + o] = sxy;
}

__global__ void ssim_blur15_kernel(const float *src, const float *w, int dir, int H, int W,
                                   float *dst) {
    const int px = blockIdx.x * blockDim.x + threadIdx.x;
    const int py = blockIdx.y * blockDim.y + threadIdx.y;
    const int ch = blockIdx.z;
    if (px >= W || py >= H) return;
    const int64_t N = (int64_t)W * H, base = (int64_t)ch * N;
    float s = 0;
    for (int k = -kR; k <= kR; ++k) {
        const int u = dir == 0 ? px + k : px, v = dir == 0 ? py : py + k;
        if (u < 0 || u >= W || v < 0 || v >= H) continue;
        s += w[k + kR] * src[base + (int64_t)v * W + u];
    }
    dst[base + (int64_t)py * W + px] = s;
}

__device__ __forceinline__ void ssim_terms(float mx, float my, float exx, float eyy, float exy,
                                           float &S, float &p_mx, float &p_xx, float &p_xy) {
    const float sxx = exx - mx * mx, syy = eyy - my * my, sxy = exy - mx * my;
    const float A = 2.0f * mx * my + kSsimC1;
    const float B = 2.0f * sxy + kSsimC2;
    const float C = mx * mx + my * my + kSsimC1;
    const float D = sxx + syy + kSsimC2;
    const float invCD = 1.0f / (C * D);
    S = A * B * invCD;
    const float dA = B * invCD, dB = A * invCD, dC = -S / C, dD = -S / D;
    p_xy = 2.0f * dB;
    p_xx = dD;
    p_mx = 2.0f * my * (dA - dB) + 2.0f * mx * (dC - dD);
}

__global__ void ssim_tail_fwd_kernel(const float *b, int64_t npix, float *out) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= 3 * npix) return;
    const int64_t c = gid / npix, i = gid - c * npix;
    const float mx = b[(0 + c) * npix + i], my = b[(3 + c) * npix + i];
    const float exx = b[(6 + c) * npix + i], eyy = b[(9 + c) * npix + i];
    const float exy = b[(12 + c) * npix + i];
    const float sxx = exx - mx * mx, syy = eyy - my * my, sxy = exy - mx * my;
    const float A = 2.0f * mx * my + kSsimC1, B = 2.0f * sxy + kSsimC2;
    const float C = mx * mx + my * my + kSsimC1, D = sxx + syy + kSsimC2;
    out[c * npix + i] = (A * B) / (C * D);
}

__global__ void ssim_tail_bwd_kernel(const float *b, const float *gout, int64_t npix, float *gb) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= 3 * npix) return;
    const int64_t c = gid / npix, i = gid - c * npix;
    const float mx = b[(0 + c) * npix + i], my = b[(3 + c) * npix + i];
    const float exx = b[(6 + c) * npix + i], eyy = b[(9 + c) * npix + i];
    const float exy = b[(12 + c) * npix + i];
    const float sxx = exx - mx * mx, syy = eyy - my * my, sxy = exy - mx * my;
    const float A = 2.0f * mx * my + kSsimC1, B = 2.0f * sxy + kSsimC2;
    const float C = mx * mx + my * my + kSsimC1, D = sxx + syy + kSsimC2;
    const float invCD = 1.0f / (C * D);
    const float S = A * B * invCD;
    const float g = gout[c * npix + i];
    const float dA = B * invCD, dB = A * invCD, dC = -S / C, dD = -S / D;
    gb[(6 + c) * npix + i] = g * dD;
    gb[(9 + c) * npix + i] = g * dD;
    gb[(12 + c) * npix + i] = g * (2.0f * dB);
    gb[(0 + c) * npix + i] = g * (2.0f * my * (dA - dB) + 2.0f * mx * (dC - dD));
    gb[(3 + c) * npix + i] = g * (2.0f * mx * (dA - dB) + 2.0f * my * (dC - dD));
}

__global__ void ssim_chain_bwd_kernel(const float *x, const float *y, const float *d, int H, int W,
                                      float *dx) {
    const int px = blockIdx.x * blockDim.x + threadIdx.x;
    const int py = blockIdx.y * blockDim.y + threadIdx.y;
    const int c = blockIdx.z;
    if (px >= W || py >= H) return;
    const int64_t N = (int64_t)W * H, o = (int64_t)py * W + px;
    const float xv = x[o * 3 + c], yv = y[o * 3 + c];
    dx[o * 3 + c] = d[(0 + c) * N + o] + 2.0f * xv * d[(6 + c) * N + o] + yv * d[(12 + c) * N + o];
}

// ------------------------------------------------------------- fused kernels
constexpr int kTW = 32, kTH = 16;                 // output tile
constexpr int kIW = kTW + 2 * kR, kIH = kTH + 2 * kR;   // 42 x 26 with halo
constexpr int kIWP = 44;                          // LDS row stride: 16-byte rows
constexpr int kSsimThreads = 256;
// Register blocking of the separable blur: a horizontal task makes kHRun
// neighbouring outputs of one row from one read of its kHRun + 2 kR inputs;
// a vertical task makes kVRun outputs of one column.
constexpr int kHRun = 4, kVRun = 2;
constexpr int kHTasks = kIH * (kTW / kHRun);      // 208
constexpr int kVTasks = (kTH / kVRun) * kTW;      // 256
static_assert(kHTasks <= kSsimThreads && kVTasks == kSsimThreads, "blur tasks per thread");
static_assert(kHRun + 2 * kR <= 16 && (kTW / kHRun - 1) * kHRun + 16 <= kIWP,
              "a horizontal task reads four float4s of its row");
// Halo elements per thread: all of a thread's loads are requested before any
// of them is stored to LDS (a rolled loop waits for each in turn).
constexpr int kLoadIters = (kIH * kIW + kSsimThreads - 1) / kSsimThreads;   // 5

// Work items of the fused kernels: (output tile, channel) pairs, item =
// 3 * tile + channel, tile = ty * tiles_x + tx. The items are dealt to the XCDs
// in contiguous runs, so the three channels of a tile (which read the same
// interleaved (H,W,3) lines) and its neighbours (which share the halo) run
// under one L2 and the lines come from HBM about once.
struct SsimItem {
    int tx, ty, c;
};
__device__ __forceinline__ SsimItem ssim_item(int tiles_x) {
    const int item = (int)xcd_contiguous(blockIdx.x, gridDim.x);
    const int tile = item / 3;
    return {tile % tiles_x, tile / tiles_x, item - 3 * tile};
}

// The horizontal task of thread t: row t / (kTW / kHRun), first output column
// kHRun * (t % (kTW / kHRun)); its inputs are 16 floats of that LDS row from
// the same column.
__device__ __forceinline__ void h_inputs(const float (*src)[kIWP], int t, int &row, int &c0,
                                         float (&v)[16]) {
    row = t / (kTW / kHRun);
    c0 = kHRun * (t % (kTW / kHRun));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 f = *reinterpret_cast<const float4 *>(&src[row][c0 + 4 * q]);
        v[4 * q] = f.x;
        v[4 * q + 1] = f.y;
        v[4 * q + 2] = f.z;
        v[4 * q + 3] = f.w;
    }
}

// block_sums[b] gets work item b's SSIM sum; with l1_sums, l1_sums[b] gets
// its sum of |x - y| over the same pixels and channel.
__global__ __launch_bounds__(kSsimThreads) void ssim_fused_fwd_kernel(
    const float *x, const float *y, const float *__restrict__ w, int H, int W, int tiles_x,
    float *partials, float *block_sums, float *l1_sums) {
    __shared__ __align__(16) float s_x[kIH][kIWP];
    __shared__ __align__(16) float s_y[kIH][kIWP];
    __shared__ __align__(16) float s_h[5][kIH][kTW];
    __shared__ float s_red[2][kSsimThreads / 64];
    const SsimItem it = ssim_item(tiles_x);
    const int c = it.c;
    const int x0 = it.tx * kTW - kR, y0 = it.ty * kTH - kR;
    const int tid = threadIdx.x;
    float wk[2 * kR + 1];
#pragma unroll
    for (int k = 0; k <= 2 * kR; ++k) wk[k] = w[k];
    {
        float xv[kLoadIters], yv[kLoadIters];
#pragma unroll
        for (int r = 0; r < kLoadIters; ++r) {
            const int i = tid + r * kSsimThreads;
            const int ly = i / kIW, lx = i - ly * kIW;
            const int gx = x0 + lx, gy = y0 + ly;
            xv[r] = 0.f;
            yv[r] = 0.f;
            if (i < kIH * kIW && gx >= 0 && gx < W && gy >= 0 && gy < H) {
                const int64_t o = ((int64_t)gy * W + gx) * 3 + c;
                xv[r] = x[o];
                yv[r] = y[o];
            }
        }
#pragma unroll
        for (int r = 0; r < kLoadIters; ++r) {
            const int i = tid + r * kSsimThreads;
            if (i < kIH * kIW) {
                const int ly = i / kIW, lx = i - ly * kIW;
                s_x[ly][lx] = xv[r];
                s_y[ly][lx] = yv[r];
            }
        }
    }
    // The pad columns are read by the last task of a row (weights beyond
    // its window are never applied to them, but they must be finite).
    for (int i = tid; i < kIH * (kIWP - kIW); i += kSsimThreads) {
        const int ly = i / (kIWP - kIW), lx = kIW + i % (kIWP - kIW);
        s_x[ly][lx] = 0.f;
        s_y[ly][lx] = 0.f;
    }
    __syncthreads();
    // Horizontal pass over the full halo height: each input's x, y, x^2,
    // y^2 and xy once, into the kHRun outputs whose window holds it.
    if (tid < kHTasks) {
        int row, c0;
        float xv[16], yv[16];
        h_inputs(s_x, tid, row, c0, xv);
        h_inputs(s_y, tid, row, c0, yv);
        float m[5][kHRun] = {};
#pragma unroll
        for (int j = 0; j < kHRun + 2 * kR; ++j) {
            const float a = xv[j], b = yv[j], aa = a * a, bb = b * b, ab = a * b;
#pragma unroll
            for (int o = 0; o < kHRun; ++o) {
                const int k = j - o;
                if (k < 0 || k > 2 * kR) continue;
                m[0][o] = fmaf(wk[k], a, m[0][o]);
                m[1][o] = fmaf(wk[k], b, m[1][o]);
                m[2][o] = fmaf(wk[k], aa, m[2][o]);
                m[3][o] = fmaf(wk[k], bb, m[3][o]);
                m[4][o] = fmaf(wk[k], ab, m[4][o]);
            }
        }
#pragma unroll
        for (int q = 0; q < 5; ++q)
            *reinterpret_cast<float4 *>(&s_h[q][row][c0]) =
                make_float4(m[q][0], m[q][1], m[q][2], m[q][3]);
    }
    __syncthreads();
    // Vertical pass and the SSIM tail: thread t makes rows kVRun * (t / kTW)
    // + [0, kVRun) of column t % kTW.
    const int64_t N = (int64_t)W * H;
    float local = 0.f, local_l1 = 0.f;
    {
        const int lx = tid % kTW, r0 = kVRun * (tid / kTW);
        float m[kVRun][5] = {};
#pragma unroll
        for (int j = 0; j < kVRun + 2 * kR; ++j) {
            float h[5];
#pragma unroll
            for (int q = 0; q < 5; ++q) h[q] = s_h[q][r0 + j][lx];
#pragma unroll
            for (int o = 0; o < kVRun; ++o) {
                const int k = j - o;
                if (k < 0 || k > 2 * kR) continue;
#pragma unroll
                for (int q = 0; q < 5; ++q) m[o][q] = fmaf(wk[k], h[q], m[o][q]);
            }
        }
        const int gx = it.tx * kTW + lx;
#pragma unroll
        for (int o = 0; o < kVRun; ++o) {
            const int ly = r0 + o, gy = it.ty * kTH + ly;
            if (gx >= W || gy >= H) continue;
            local_l1 += fabsf(s_x[ly + kR][lx + kR] - s_y[ly + kR][lx + kR]);
            float S, pm, pxx, pxy;
            ssim_terms(m[o][0], m[o][1], m[o][2], m[o][3], m[o][4], S, pm, pxx, pxy);
            local += S;
            const int64_t po = (int64_t)gy * W + gx;
            partials[(0 + c) * N + po] = pm;
            partials[(3 + c) * N + po] = pxx;
            partials[(6 + c) * N + po] = pxy;
        }
    }
    // Deterministic per-block sums (fixed reduction order).
    for (int off = 32; off >= 1; off >>= 1) {
        local += __shfl_xor(local, off, 64);
        local_l1 += __shfl_xor(local_l1, off, 64);
    }
    if ((tid & 63) == 0) {
        s_red[0][tid >> 6] = local;
        s_red[1][tid >> 6] = local_l1;
    }
    __syncthreads();
    if (tid == 0) {
        float s = 0.f, s1 = 0.f;
        for (int k = 0; k < kSsimThreads / 64; ++k) {
            s += s_red[0][k];
            s1 += s_red[1][k];
        }
        const int bid = 3 * (it.ty * tiles_x + it.tx) + c;
        block_sums[bid] = s;
        if (l1_sums) l1_sums[bid] = s1;
    }
}

// Sums of K arrays of block sums (nb >= 1) in double, for a one-workgroup
// reduction: each thread requests kSumPer values of every array at once per
// step (a rolled loop waits for each load in turn).
constexpr int kSumPer = 16;
template <int K>
__device__ __forceinline__ void sum_blocks(const float *const (&v)[K], int64_t nb, double (&s)[K]) {
#pragma unroll
    for (int k = 0; k < K; ++k) s[k] = 0.0;
    for (int64_t b = 0; b < nb; b += 256 * kSumPer) {
        float t[K][kSumPer];
        // Unconditional loads of a clamped index, then a select: a guarded
        // load becomes a branch that waits for it before the next.
#pragma unroll
        for (int j = 0; j < kSumPer; ++j) {
            const int64_t i = b + threadIdx.x + 256 * j;
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const float u = v[k][min(i, nb - 1)];
                t[k][j] = i < nb ? u : 0.0f;
            }
        }
#pragma unroll
        for (int j = 0; j < kSumPer; ++j)
#pragma unroll
            for (int k = 0; k < K; ++k) s[k] += (double)t[k][j];
    }
}

__global__ __launch_bounds__(256) void ssim_mean_kernel(const float *block_sums, int64_t nb,
                                                        int64_t count, float *mean_out) {
    __shared__ double s_red[4];
    double sv[1];
    sum_blocks<1>({block_sums}, nb, sv);
    double s = sv[0];
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) mean_out[0] = (float)((s_red[0] + s_red[1] + s_red[2] + s_red[3]) / (double)count);
}

// out[0] = (1 - lam) * mean|x - y| + lam * (1 - mean SSIM), out[1] = the L1
// mean, out[2] = the SSIM mean; sums in double.
__global__ __launch_bounds__(256) void photometric_loss_kernel(const float *ssim_sums,
                                                               const float *l1_sums, int64_t nb,
                                                               int64_t count, float lam,
                                                               float *out) {
    __shared__ double s_red[2][4];
    double sv[2];
    sum_blocks<2>({ssim_sums, l1_sums}, nb, sv);
    double s = sv[0], s1 = sv[1];
    for (int off = 32; off >= 1; off >>= 1) {
        s += __shfl_xor(s, off, 64);
        s1 += __shfl_xor(s1, off, 64);
    }
    if ((threadIdx.x & 63) == 0) {
        s_red[0][threadIdx.x >> 6] = s;
        s_red[1][threadIdx.x >> 6] = s1;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const double ss = (s_red[0][0] + s_red[0][1] + s_red[0][2] + s_red[0][3]) / (double)count;
        const double l1 = (s_red[1][0] + s_red[1][1] + s_red[1][2] + s_red[1][3]) / (double)count;
        const double l = (double)lam;
        out[0] = (float)((1.0 - l) * l1 + l * (1.0 - ss));
        out[1] = (float)l1;
        out[2] = (float)ss;
    }
}

// dx = g / (3N) * (a_ssim * dSSIM_sum/dx + a_l1 * sign(x - y)), g = scale_dev[0]:
// a_ssim = 1, a_l1 = 0 is the gradient of the SSIM mean; a_ssim = -lam,
// a_l1 = 1 - lam that of the photometric loss.
__global__ __launch_bounds__(kSsimThreads) void ssim_fused_bwd_kernel(
    const float *x, const float *y, const float *__restrict__ w, const float *partials,
    const float *scale_dev, int H, int W, int tiles_x, float a_ssim, float a_l1, float *dx) {
    __shared__ __align__(16) float s_p[3][kIH][kIWP];
    __shared__ __align__(16) float s_h[3][kIH][kTW];
    const SsimItem it = ssim_item(tiles_x);
    const int c = it.c;
    const int x0 = it.tx * kTW - kR, y0 = it.ty * kTH - kR;
    const int tid = threadIdx.x;
    const int64_t N = (int64_t)W * H;
    float wk[2 * kR + 1];
#pragma unroll
    for (int k = 0; k <= 2 * kR; ++k) wk[k] = w[k];
    {
        float pv[3][kLoadIters];
#pragma unroll
        for (int r = 0; r < kLoadIters; ++r) {
            const int i = tid + r * kSsimThreads;
            const int ly = i / kIW, lx = i - ly * kIW;
            const int gx = x0 + lx, gy = y0 + ly;
#pragma unroll
            for (int q = 0; q < 3; ++q) pv[q][r] = 0.f;
            if (i < kIH * kIW && gx >= 0 && gx < W && gy >= 0 && gy < H) {
                const int64_t o = (int64_t)gy * W + gx;
#pragma unroll
                for (int q = 0; q < 3; ++q) pv[q][r] = partials[(3 * q + c) * N + o];
            }
        }
#pragma unroll
        for (int r = 0; r < kLoadIters; ++r) {
            const int i = tid + r * kSsimThreads;
            if (i < kIH * kIW) {
                const int ly = i / kIW, lx = i - ly * kIW;
#pragma unroll
                for (int q = 0; q < 3; ++q) s_p[q][ly][lx] = pv[q][r];
            }
        }
    }
    for (int i = tid; i < kIH * (kIWP - kIW); i += kSsimThreads) {
        const int ly = i / (kIWP - kIW), lx = kIW + i % (kIWP - kIW);
        s_p[0][ly][lx] = 0.f;
        s_p[1][ly][lx] = 0.f;
        s_p[2][ly][lx] = 0.f;
    }
    __syncthreads();
    if (tid < kHTasks) {
        int row, c0;
        float v[3][16];
#pragma unroll
        for (int q = 0; q < 3; ++q) h_inputs(s_p[q], tid, row, c0, v[q]);
        float m[3][kHRun] = {};
#pragma unroll
        for (int j = 0; j < kHRun + 2 * kR; ++j) {
#pragma unroll
            for (int o = 0; o < kHRun; ++o) {
                const int k = j - o;
                if (k < 0 || k > 2 * kR) continue;
#pragma unroll
                for (int q = 0; q < 3; ++q) m[q][o] = fmaf(wk[k], v[q][j], m[q][o]);
            }
        }
#pragma unroll
        for (int q = 0; q < 3; ++q)
            *reinterpret_cast<float4 *>(&s_h[q][row][c0]) =
                make_float4(m[q][0], m[q][1], m[q][2], m[q][3]);
    }
    __syncthreads();
    const float scale = scale_dev[0] / (float)(3 * N);
    const int lx = tid % kTW, r0 = kVRun * (tid / kTW);
    float m[kVRun][3] = {};
#pragma unroll
    for (int j = 0; j < kVRun + 2 * kR; ++j) {
        float h[3];
#pragma unroll
        for (int q = 0; q < 3; ++q) h[q] = s_h[q][r0 + j][lx];
#pragma unroll
        for (int o = 0; o < kVRun; ++o) {
            const int k = j - o;
            if (k < 0 || k > 2 * kR) continue;
#pragma unroll
            for (int q = 0; q < 3; ++q) m[o][q] = fmaf(wk[k], h[q], m[o][q]);
        }
    }
    const int gx = it.tx * kTW + lx;
#pragma unroll
    for (int o = 0; o < kVRun; ++o) {
        const int gy = it.ty * kTH + r0 + o;
        if (gx >= W || gy >= H) continue;
        const int64_t po = ((int64_t)gy * W + gx) * 3 + c;
        const float xv = x[po], yv = y[po];
        float d = a_ssim * (m[o][0] + 2.0f * xv * m[o][1] + yv * m[o][2]);
        if (a_l1 != 0.0f) {
            // torch's abs backward: sign, with 0 at x == y.
            const float sg = xv > yv ? 1.0f : (xv < yv ? -1.0f : 0.0f);
            d += a_l1 * sg;
        }
        dx[po] = scale * d;
    }
}

// Work items (workgroups) of the fused kernels: one per (output tile, channel).
inline int64_t ssim_blocks(int H, int W) {
    return ceil_div(W, kTW) * ceil_div(H, kTH) * 3;
}

// ------------------------------------------------ allocation-free variant
// mg_photometric_loss_forward_noalloc keeps the loss forward's block sums in
// this file-scope device array instead of a caller workspace, for callers
// that cannot allocate device memory (graph capture, serving loops). Every
// GPU the library runs on holds its own copy until the process ends; calls
// that overlap on one GPU share it and race.
constexpr int64_t kStaticLossBlocks = int64_t(1) << 18;   // SSIM + L1 sums: 2 MiB
static __device__ __align__(256) float scratch[2 * kStaticLossBlocks];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static float *g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up once per
// device with that device current. Host code passes this address to kernels;
// the array's name is only a host-side stand-in.
int32_t static_scratch(float **out, const char *who) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        set_error("%s: hipGetDevice failed: %s", who, hipGetErrorString(e));
        return MG_ERR_RUNTIME;
    }
    MG_REQUIRE(dev >= 0 && dev < kMaxDevices, "%s: device %d beyond the %d supported", who, dev,
               kMaxDevices);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr) {
            set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who, dev,
                      hipGetErrorString(e));
            return MG_ERR_RUNTIME;
        }
        g_scratch_ptr[dev] = static_cast<float *>(ptr);
    }
    *out = g_scratch_ptr[dev];
    return MG_OK;
}

// The trainer's loss forward on `sums` (2 * ssim_blocks(H, W) floats): the
// fused SSIM pass writes every block's SSIM and L1 sums (each block its own
// entries, so nothing needs clearing), then one workgroup reduces them.
static int32_t photometric_forward(const float *x, const float *y, const float *w, int32_t H,
                                   int32_t W, float ssim_weight, float *partials, float *out,
                                   float *sums, mg_stream_t stream, const char *who) {
    MG_REQUIRE(ssim_weight >= 0.0f && ssim_weight <= 1.0f, "%s: ssim_weight %g outside [0, 1]",
               who, (double)ssim_weight);
    hipStream_t s = as_stream(stream);
    const int tiles_x = (int)ceil_div(W, kTW);
    const int64_t nb = ssim_blocks(H, W);
    const unsigned grid = (unsigned)nb;
    TimedScope ts("ssim_fused_forward", s);
    ssim_fused_fwd_kernel<<<grid, kSsimThreads, 0, s>>>(x, y, w, H, W, tiles_x, partials, sums,
                                                        sums + nb);
    MG_LAUNCHED("ssim_fused_fwd_kernel");
    photometric_loss_kernel<<<1, 256, 0, s>>>(sums, sums + nb, nb, 3LL * H * W, ssim_weight, out);
    MG_LAUNCHED("photometric_loss_kernel");
    return MG_OK;
}

}  // namespace mg

using namespace mg;

extern "C" {

int32_t mg_ssim_stack_blur_h(const float *x, const float *y, const float *w, int32_t H, int32_t W,
                             float *out, mg_stream_t stream) {
    MG_REQUIRE(H > 0 && W > 0 && x && y && w && out, "mg_ssim_stack_blur_h: bad arguments");
    dim3 blk(16, 16), grid((unsigned)ceil_div(W, 16), (unsigned)ceil_div(H, 16), 3);
    TimedScope ts("ssim_stack_blur_h", as_stream(stream));
    ssim_stack_blur_h_kernel<<<grid, blk, 0, as_stream(stream)>>>(x, y, w, H, W, out);
    MG_LAUNCHED("ssim_stack_blur_h_kernel");
    return MG_OK;
}

int32_t mg_ssim_blur15(const float *src, const float *w, int32_t dir, int32_t H, int32_t W,
                       float *out, mg_stream_t stream) {
    MG_REQUIRE(H > 0 && W > 0 && src && w && out && (dir == 0 || dir == 1),
               "mg_ssim_blur15: bad arguments");
    dim3 blk(16, 16), grid((unsigned)ceil_div(W, 16), (unsigned)ceil_div(H, 16), 15);
    TimedScope ts("ssim_blur15", as_stream(stream));
    ssim_blur15_kernel<<<grid, blk, 0, as_stream(stream)>>>(src, w, dir, H, W, out);
    MG_LAUNCHED("ssim_blur15_kernel");
    return MG_OK;
}

int32_t mg_ssim_tail_forward(const float *b, int32_t H, int32_t W, float *out, mg_stream_t stream) {
    MG_REQUIRE(H > 0 && W > 0 && b && out, "mg_ssim_tail_forward: bad arguments");
    const int64_t npix = (int64_t)H * W;
    TimedScope ts("ssim_tail_forward", as_stream(stream));
    ssim_tail_fwd_kernel<<<(unsigned)ceil_div(3 * npix, 256), 256, 0, as_stream(stream)>>>(b, npix,
                                                                                          out);
    MG_LAUNCHED("ssim_tail_fwd_kernel");
    return MG_OK;
}

int32_t mg_ssim_tail_backward(const float *b, const float *gout, int32_t H, int32_t W, float *gb,
                              mg_stream_t stream) {
    MG_REQUIRE(H > 0 && W > 0 && b && gout && gb, "mg_ssim_tail_backward: bad arguments");
    const int64_t npix = (int64_t)H * W;
    TimedScope ts("ssim_tail_backward", as_stream(stream));
    ssim_tail_bwd_kernel<<<(unsigned)ceil_div(3 * npix, 256), 256, 0, as_stream(stream)>>>(
        b, gout, npix, gb);
    MG_LAUNCHED("ssim_tail_bwd_kernel");
    return MG_OK;
}

int32_t mg_ssim_chain_backward(const float *x, const float *y, const float *d_stack, int32_t H,
                               int32_t W, float *d_x, mg_stream_t stream) {
    MG_REQUIRE(H > 0 && W > 0 && x && y && d_stack && d_x, "mg_ssim_chain_backward: bad arguments");
    dim3 blk(16, 16), grid((unsigned)ceil_div(W, 16), (unsigned)ceil_div(H, 16), 3);
    TimedScope ts("ssim_chain_backward", as_stream(stream));
    ssim_chain_bwd_kernel<<<grid, blk, 0, as_stream(stream)>>>(x, y, d_stack, H, W, d_x);
    MG_LAUNCHED("ssim_chain_bwd_kernel");
    return MG_OK;
}

int64_t mg_ssim_fused_workspace_bytes(int32_t H, int32_t W) {
    if (H <= 0 || W <= 0) return 0;
    return 2 * ssim_blocks(H, W) * (int64_t)sizeof(float);   // SSIM and L1 block sums
}

int32_t mg_ssim_fused_forward(const float *x, const float *y, const float *w, int32_t H, int32_t W,
                              float *partials, float *mean_out, void *workspace,
                              int64_t workspace_bytes, mg_stream_t stream) {
    MG_REQUIRE(H > 0 && W > 0 && x && y && w && partials && mean_out,
               "mg_ssim_fused_forward: bad arguments");
    MG_REQUIRE(workspace && workspace_bytes >= mg_ssim_fused_workspace_bytes(H, W),
               "mg_ssim_fused_forward: workspace %lld bytes, need %lld",
               (long long)workspace_bytes, (long long)mg_ssim_fused_workspace_bytes(H, W));
    hipStream_t s = as_stream(stream);
    const int tiles_x = (int)ceil_div(W, kTW);
    const unsigned grid = (unsigned)ssim_blocks(H, W);
    float *sums = static_cast<float *>(workspace);
    TimedScope ts("ssim_fused_forward", s);
    ssim_fused_fwd_kernel<<<grid, kSsimThreads, 0, s>>>(x, y, w, H, W, tiles_x, partials, sums,
                                                        nullptr);
    MG_LAUNCHED("ssim_fused_fwd_kernel");
    ssim_mean_kernel<<<1, 256, 0, s>>>(sums, (int64_t)grid, 3LL * H * W, mean_out);
    MG_LAUNCHED("ssim_mean_kernel");
    return MG_OK;
}

int32_t mg_ssim_fused_backward(const float *x, const float *y, const float *w,
                               const float *partials, const float *scale_dev, int32_t H,
                               int32_t W, float *d_x, mg_stream_t stream) {
    MG_REQUIRE(H > 0 && W > 0 && x && y && w && partials && scale_dev && d_x,
               "mg_ssim_fused_backward: bad arguments");
    hipStream_t s = as_stream(stream);
    const int tiles_x = (int)ceil_div(W, kTW);
    const unsigned grid = (unsigned)ssim_blocks(H, W);
    TimedScope ts("ssim_fused_backward", s);
    ssim_fused_bwd_kernel<<<grid, kSsimThreads, 0, s>>>(x, y, w, partials, scale_dev, H, W,
                                                        tiles_x, 1.0f, 0.0f, d_x);
    MG_LAUNCHED("ssim_fused_bwd_kernel");
    return MG_OK;
}

int32_t mg_photometric_loss_forward(const float *x, const float *y, const float *w, int32_t H,
                                    int32_t W, float ssim_weight, float *partials, float *out,
                                    void *workspace, int64_t workspace_bytes,
                                    mg_stream_t stream) {
    MG_REQUIRE(H > 0 && W > 0 && x && y && w && partials && out,
               "mg_photometric_loss_forward: bad arguments");
    MG_REQUIRE(workspace && workspace_bytes >= mg_ssim_fused_workspace_bytes(H, W),
               "mg_photometric_loss_forward: workspace %lld bytes, need %lld",
               (long long)workspace_bytes, (long long)mg_ssim_fused_workspace_bytes(H, W));
    return photometric_forward(x, y, w, H, W, ssim_weight, partials, out,
                               static_cast<float *>(workspace), stream,
                               "mg_photometric_loss_forward");
}

int32_t mg_photometric_loss_forward_noalloc(const float *x, const float *y, const float *w,
                                            int32_t H, int32_t W, float ssim_weight,
                                            float *partials, float *out, mg_stream_t stream) {
    const char *who = "mg_photometric_loss_forward_noalloc";
    MG_REQUIRE(H > 0 && W > 0 && x && y && w && partials && out, "%s: bad arguments", who);
    MG_REQUIRE(ssim_blocks(H, W) <= kStaticLossBlocks,
               "%s: a %dx%d image needs %lld block sums (3 per 32x16-pixel tile), more "
               "than the %lld the static scratch holds",
               who, H, W, (long long)ssim_blocks(H, W), (long long)kStaticLossBlocks);
    float *sums = nullptr;
    const int32_t rc = static_scratch(&sums, who);
    if (rc != MG_OK) return rc;
    return photometric_forward(x, y, w, H, W, ssim_weight, partials, out, sums, stream, who);
}

int32_t mg_photometric_loss_backward(const float *x, const float *y, const float *w,
                                     const float *partials, const float *grad_dev, int32_t H,
                                     int32_t W, float ssim_weight, float *d_x,
                                     mg_stream_t stream) {
    MG_REQUIRE(H > 0 && W > 0 && x && y && w && partials && grad_dev && d_x,
               "mg_photometric_loss_backward: bad arguments");
    MG_REQUIRE(ssim_weight >= 0.0f && ssim_weight <= 1.0f,
               "mg_photometric_loss_backward: ssim_weight %g outside [0, 1]",
               (double)ssim_weight);
    hipStream_t s = as_stream(stream);
    const int tiles_x = (int)ceil_div(W, kTW);
    const unsigned grid = (unsigned)ssim_blocks(H, W);
    TimedScope ts("ssim_fused_backward", s);
    ssim_fused_bwd_kernel<<<grid, kSsimThreads, 0, s>>>(x, y, w, partials, grad_dev, H, W, tiles_x,
                                                        -ssim_weight, 1.0f - ssim_weight, d_x);
    MG_LAUNCHED("ssim_fused_bwd_kernel");
    return MG_OK;
}

}  // extern "C"
