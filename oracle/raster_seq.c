/*
 * raster_seq.c -- the rasteriser's per-pixel contract on the CPU.
 * TEST INFRASTRUCTURE ONLY (built by oracle/build.py, used by tests/ and the
 * bench's CPU-baseline leg; never linked into the product).
 *
 * Restates metal_gauss/csrc/rasterize.metal:
 *   forward  (61-167): per pixel, walk the tile's depth-sorted list front to
 *     back; power = -0.5 (a dx^2 + 2 b dx dy + c dy^2), skip power > 0;
 *     alpha = min(0.999, op exp(power)), skip alpha < 1/255; accumulate
 *     colour and alpha with weight alpha T; T *= 1 - alpha; the stop index is
 *     the list index + 1 of the last blended Gaussian; stop once T < t_min.
 *   backward (173-340): per pixel, walk back to front from the stop index,
 *     recover T by dividing out (1 - alpha), keep colour and alpha suffix
 *     sums, and accumulate dL/dcolour, dL/duv, dL/dconic, dL/dopacity (none
 *     through the 0.999 clamp), plus sum |dL/duv| per pixel (absgrad).
 * fp32 arithmetic in the kernel's operation order (the exponent with the same
 * fused multiply-adds), so the only differences to the GPU are the exp
 * implementation and the order of the per-Gaussian gradient sums.
 *
 * Pinned by tests/test_oracle_adam_ssim_raster.py: against the torch restatement of
 * torch_ref (oracle/render_ref.py) on the same tile lists with t_min = 0, and
 * its backward against torch autograd of that restatement.
 *
 * Per pixel it also reports whether the result is ill-conditioned at fp32:
 * some evaluated alpha within a relative 1e-5 of the 1/255 cutoff, or the
 * stopping transmittance within a relative 1e-5 of t_min. There a last-bit
 * difference in exp flips a discrete decision and moves the pixel by up to
 * alpha * T * colour, so parity tests treat those pixels separately.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ALPHA_MAX 0.999f
#define ALPHA_MIN (1.0f / 255.0f)

static float splat_power(float dx, float dy, float a, float b, float c) {
    const float q = fmaf(a * dx, dx, fmaf(2.0f * b * dx, dy, c * dy * dy));
    return -0.5f * q;
}

static int near_rel(float x, float ref, float rel) {
    return fabsf(x - ref) <= rel * fabsf(ref);
}

/* Forward for one pixel; returns the stop index. */
static int shade(float fx, float fy, const float *uv, const float *conic, const float *op,
                 const float *color, const int32_t *ids, int start, int end, float t_min,
                 float out[4], float *T_out, uint8_t *amb) {
    float T = 1.0f, r = 0.f, g = 0.f, b = 0.f, acc = 0.f;
    int stop = start;
    for (int i = start; i < end; ++i) {
        const int k = ids[i];
        const float dx = fx - uv[2 * k], dy = fy - uv[2 * k + 1];
        const float power = splat_power(dx, dy, conic[3 * k], conic[3 * k + 1], conic[3 * k + 2]);
        if (power > 0.0f) continue;
        const float alpha = fminf(ALPHA_MAX, op[k] * expf(power));
        if (near_rel(alpha, ALPHA_MIN, 1e-5f)) *amb = 1;
        if (alpha < ALPHA_MIN) continue;
        const float w = alpha * T;
        r = fmaf(w, color[3 * k], r);
        g = fmaf(w, color[3 * k + 1], g);
        b = fmaf(w, color[3 * k + 2], b);
        acc += w;
        T = T * (1.0f - alpha);
        stop = i + 1;
        if (t_min > 0.0f && near_rel(T, t_min, 1e-5f)) *amb = 1;
        if (T < t_min) break;
    }
    out[0] = r; out[1] = g; out[2] = b; out[3] = acc;
    *T_out = T;
    return stop;
}

int raster_seq_forward(int64_t N, const float *uv, const float *conic, const float *op,
                       const float *color, const int32_t *ids, const int32_t *offsets,
                       int32_t W, int32_t H, int32_t tile, int32_t tiles_x, float t_min,
                       float *rgb, float *alpha, float *T, int32_t *stop, uint8_t *ambiguous) {
    (void)N;
    if (W <= 0 || H <= 0 || tile <= 0) return 1;
#pragma omp parallel for schedule(dynamic, 4)
    for (int64_t py = 0; py < H; ++py) {
        for (int px = 0; px < W; ++px) {
            const int t = (int)(py / tile) * tiles_x + px / tile;
            const int64_t o = py * W + px;
            float out[4], Tp;
            uint8_t amb = 0;
            stop[o] = shade((float)px + 0.5f, (float)py + 0.5f, uv, conic, op, color, ids,
                            offsets[t], offsets[t + 1], t_min, out, &Tp, &amb);
            rgb[3 * o] = out[0]; rgb[3 * o + 1] = out[1]; rgb[3 * o + 2] = out[2];
            alpha[o] = out[3];
            T[o] = Tp;
            if (ambiguous) ambiguous[o] = amb;
        }
    }
    return 0;
}

/* Gradient accumulators: 10 floats per Gaussian (col 3, uv 2, conic 3, op, abs). */
static void backward_pixel(float fx, float fy, const float *uv, const float *conic,
                           const float *op, const float *color, const int32_t *ids, int start,
                           int my_stop, float T, const float gc[3], float ga, float *acc) {
    float sr = 0.f, sg = 0.f, sb = 0.f, sa = 0.f;
    for (int i = my_stop - 1; i >= start; --i) {
        const int k = ids[i];
        const float dx = fx - uv[2 * k], dy = fy - uv[2 * k + 1];
        const float a = conic[3 * k], b = conic[3 * k + 1], c = conic[3 * k + 2];
        const float power = splat_power(dx, dy, a, b, c);
        if (power > 0.0f) continue;
        const float gauss = expf(power);
        const float alpha_raw = op[k] * gauss;
        const float alpha = fminf(ALPHA_MAX, alpha_raw);
        if (alpha < ALPHA_MIN) continue;
        const float om = fmaxf(1.0f - alpha, 1e-8f);
        T = T / om;
        const float iom = 1.0f / om;
        const float w = alpha * T;
        const float *col = color + 3 * k;
        float *d = acc + 10 * (int64_t)k;
        d[0] += w * gc[0];
        d[1] += w * gc[1];
        d[2] += w * gc[2];
        const float dal = gc[0] * (T * col[0] - sr * iom) + gc[1] * (T * col[1] - sg * iom) +
                          gc[2] * (T * col[2] - sb * iom) + ga * (T - sa * iom);
        sr = fmaf(w, col[0], sr);
        sg = fmaf(w, col[1], sg);
        sb = fmaf(w, col[2], sb);
        sa += w;
        if (alpha_raw <= ALPHA_MAX) {
            const float dpow = dal * op[k] * gauss;
            const float du = dpow * (a * dx + b * dy), dv = dpow * (b * dx + c * dy);
            d[3] += du;
            d[4] += dv;
            d[5] += -0.5f * dpow * dx * dx;
            d[6] += -dpow * dx * dy;
            d[7] += -0.5f * dpow * dy * dy;
            d[8] += dal * gauss;
            d[9] += sqrtf(du * du + dv * dv);
        }
    }
}

int raster_seq_backward(int64_t N, const float *uv, const float *conic, const float *op,
                        const float *color, const int32_t *ids, const int32_t *offsets,
                        const float *final_T, const int32_t *stop, const float *grad_rgb,
                        const float *grad_alpha, int32_t W, int32_t H, int32_t tile,
                        int32_t tiles_x, float *d_uv, float *d_conic, float *d_op,
                        float *d_col, float *d_abs) {
    if (W <= 0 || H <= 0 || tile <= 0) return 1;
    int nthreads = 1;
#ifdef _OPENMP
    nthreads = omp_get_max_threads();
#endif
    float *acc = (float *)calloc((size_t)nthreads * (size_t)N * 10 + 1, sizeof(float));
    if (!acc) return 2;
#pragma omp parallel
    {
        int tid = 0;
#ifdef _OPENMP
        tid = omp_get_thread_num();
#endif
        float *mine = acc + (size_t)tid * (size_t)N * 10;
#pragma omp for schedule(dynamic, 4)
        for (int64_t py = 0; py < H; ++py) {
            for (int px = 0; px < W; ++px) {
                const int t = (int)(py / tile) * tiles_x + px / tile;
                const int64_t o = py * W + px;
                const float gc[3] = {grad_rgb[3 * o], grad_rgb[3 * o + 1], grad_rgb[3 * o + 2]};
                backward_pixel((float)px + 0.5f, (float)py + 0.5f, uv, conic, op, color, ids,
                               offsets[t], stop[o], final_T[o], gc, grad_alpha[o], mine);
            }
        }
    }
    for (int64_t k = 0; k < N; ++k) {
        float s[10] = {0};
        for (int th = 0; th < nthreads; ++th)
            for (int j = 0; j < 10; ++j) s[j] += acc[(size_t)th * N * 10 + 10 * k + j];
        d_col[3 * k] = s[0]; d_col[3 * k + 1] = s[1]; d_col[3 * k + 2] = s[2];
        d_uv[2 * k] = s[3]; d_uv[2 * k + 1] = s[4];
        d_conic[3 * k] = s[5]; d_conic[3 * k + 1] = s[6]; d_conic[3 * k + 2] = s[7];
        d_op[k] = s[8];
        if (d_abs) d_abs[k] = s[9];
    }
    free(acc);
    return 0;
}
