// Tile rasteriser, forward and backward.
//
// One workgroup per tile, one thread per pixel, wave64. At tile sizes that are
// multiples of 8 each wave shades one 8x8 pixel block (compact, so the
// per-wave cull below rejects more); other tiles use row-major pixels.
//
// Per batch of up to 256 Gaussians from the tile's depth-sorted list:
//   1. every thread stages one Gaussian's record in LDS and tests it against
//      each wave's bounding box of pixel centres with the binning's own
//      min-over-rectangle test (plus a rounding margin), one bit per wave;
//   2. each wave compacts the indices of the Gaussians live for it with a
//      ballot, so dead entries cost nothing in the inner loop;
//   3. the wave walks its live list; every lane shades its own pixel.
//
// Forward (metal_gauss/csrc/rasterize.metal:61-167 contract): front to back,
//   alpha = min(0.999, op exp(power)), skip alpha < 1/255 or power > 0,
//   T *= 1 - alpha, stop index = list index + 1, pixel done at T < t_min;
//   a wave leaves the loop when all its pixels are done and the workgroup
//   when all its waves are.
// Backward (rasterize.metal:173-340 contract): back to front from the
//   largest stop index of the wave, T recovered by dividing out (1 - alpha),
//   colour/alpha suffix sums, gradients to colour, uv, conic and opacity.
//   The 9 (10 with absgrad) per-Gaussian sums are reduced across the 64
//   lanes with DPP and added into a per-batch LDS accumulator (LDS float
//   atomics: several waves may hold the same Gaussian); after the batch one
//   thread per Gaussian issues the global float atomics. Global atomics go
//   to a coherence point shared by all XCDs and cost HBM write traffic, so
//   there is one set per (Gaussian, tile) rather than per (Gaussian, wave).
#include "mg_common.h"

namespace mg {

constexpr int kBatch = 256;
constexpr int kMaxWaves = 16;        // tile 32 -> 1024 threads
constexpr float kAlphaMax = 0.999f;
constexpr float kAlphaMin = 1.0f / 255.0f;

struct RasterArgs {
    const float *uv, *conic, *opac, *color;
    const int32_t *ids, *offsets;
    int32_t W, H, tile, tiles_x, n_tiles;
    float t_min;
    // Optional background: rgb += max(1 - alpha, 0) * bg (has_bg != 0).
    int32_t has_bg;
    float bg[3];
};

__device__ __forceinline__ void tile_pixel(int tid, int tile, int &lx, int &ly, bool &inblk) {
    if ((tile & 7) == 0) {
        const int w = tid >> 6, l = tid & 63, bx = tile >> 3;
        lx = (w % bx) * 8 + (l & 7);
        ly = (w / bx) * 8 + (l >> 3);
        inblk = true;
    } else {
        lx = tid % tile;
        ly = tid / tile;
        inblk = tid < tile * tile;
    }
}

// The exponent of the splat at offset (dx, dy). Written with explicit fmas so
// the forward and the backward round identically: the backward divides the
// forward's (1 - alpha) back out and must see the same alpha bit for bit.
__device__ __forceinline__ float splat_power(float dx, float dy, float a, float b, float c) {
    const float q = fmaf(a * dx, dx, fmaf(2.0f * b * dx, dy, c * dy * dy));
    return -0.5f * q;
}

// Conservative per-wave cull: minimum of the quadratic form over the box of
// the wave's pixel centres, against 2 ln(255 op) widened by a rounding margin
// (the reference's own margin, rasterize.metal:150-151).
__device__ __forceinline__ float rect_min_q(float mux, float muy, float ca, float cb, float cc,
                                            float x0, float x1, float y0, float y1) {
    if (mux >= x0 && mux <= x1 && muy >= y0 && muy <= y1) return 0.0f;
    const float a = fmaxf(ca, 1e-12f), b = cb, c = fmaxf(cc, 1e-12f);
    float best = __builtin_inff();
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const float yc = e == 0 ? y0 : y1;
        const float xs = fminf(fmaxf(mux - b * (yc - muy) / a, x0), x1);
        const float ex = xs - mux, ey = yc - muy;
        best = fminf(best, a * ex * ex + 2.0f * b * ex * ey + c * ey * ey);
    }
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const float xc = e == 0 ? x0 : x1;
        const float ys = fminf(fmaxf(muy - b * (xc - mux) / c, y0), y1);
        const float ex = xc - mux, ey = ys - muy;
        best = fminf(best, a * ex * ex + 2.0f * b * ex * ey + c * ey * ey);
    }
    return best;
}

// LDS of one workgroup; MAXW bounds the waves per tile (4 up to 16x16).
template <int MAXW>
struct Stage {
    float4 geo[kBatch];       // u, v, opacity, unused
    float4 con[kBatch];       // conic a, b, c, unused
    float4 col[kBatch];       // r, g, b, unused
    int32_t id[kBatch];
    uint32_t live[kBatch];    // bit w: wave w may be touched
    uint16_t list[MAXW][kBatch];
    float4 rect[MAXW];        // x_lo, x_hi, y_lo, y_hi of pixel centres
    int32_t flag[MAXW];
};

constexpr int kGradSlots = 10;   // colour 3, uv 2, conic 3, opacity, |uv|

// Pairwise wave-wide sums by lane swaps. v_permlane32_swap a, b swaps lanes
// 32-63 of a with lanes 0-31 of b, leaving (a[0:32], b[0:32]) in a and
// (a[32:64], b[32:64]) in b, so a + b holds a's half-sums in lanes 0-31 and
// b's in lanes 32-63. v_permlane16_swap does the same between rows 0/1 and
// 2/3. Issued as inline assembly: this compiler folds the two results of the
// __builtin_amdgcn_permlane*_swap builtins into one register (r[0] + r[1]
// comes out as r[0] + r[0]). The s_nop gives the two wait states a swap
// needs after a VALU write of its operands.
__device__ __forceinline__ float swap32_sum(float a, float b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return a + b;
}
__device__ __forceinline__ float swap16_sum(float a, float b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return a + b;
}
// Sum over the 16 lanes of each row, in every lane of the row.
__device__ __forceinline__ float row_allsum(float x) {
    x += dpp_f<0x128>(x);   // row_ror:8
    x += dpp_f<0x124>(x);   // row_ror:4
    x += dpp_f<0x122>(x);   // row_ror:2
    x += dpp_f<0x121>(x);   // row_ror:1
    return x;
}
// Wave sums of ten values in 28 VALU operations instead of ten separate
// reductions: after the 32- and 16-lane swap stages each row of 16 lanes
// carries one value's partials, which a row reduction finishes. Rows of q0
// hold the sums of v0, v2, v1, v3; of q1 v4, v6, v5, v7; of q2 v8, -, v9, -.
__device__ __forceinline__ void reduce10_to_rows(const float v[10], float &q0, float &q1,
                                                 float &q2) {
    const float p0 = swap32_sum(v[0], v[1]);
    const float p1 = swap32_sum(v[2], v[3]);
    const float p2 = swap32_sum(v[4], v[5]);
    const float p3 = swap32_sum(v[6], v[7]);
    const float p4 = swap32_sum(v[8], v[9]);
    q0 = row_allsum(swap16_sum(p0, p1));
    q1 = row_allsum(swap16_sum(p2, p3));
    q2 = row_allsum(swap16_sum(p4, 0.0f));
}

template <int MAXW>
struct StageBwd : Stage<MAXW> {
    float grad[kGradSlots][kBatch];   // per batch entry, summed over waves
};

template <class S_>
__device__ __forceinline__ void stage_batch(S_ &S, const RasterArgs &A, int base, int n,
                                            int nwaves) {
    for (int t = threadIdx.x; t < n; t += blockDim.x) {
        const int g = A.ids[base + t];
        const float u = A.uv[2 * g], v = A.uv[2 * g + 1];
        const float op = A.opac[g];
        const float ca = A.conic[3 * g], cb = A.conic[3 * g + 1], cc = A.conic[3 * g + 2];
        S.geo[t] = make_float4(u, v, op, 0.f);
        S.con[t] = make_float4(ca, cb, cc, 0.f);
        S.col[t] = make_float4(A.color[3 * g], A.color[3 * g + 1], A.color[3 * g + 2], 0.f);
        S.id[t] = g;
        const float thr = 2.0f * __logf(fmaxf(255.0f * op, 1.0f));
        const float thr_m = thr * 1.0001f + 1e-4f;
        uint32_t m = 0;
        for (int w = 0; w < nwaves; ++w) {
            const float4 r = S.rect[w];
            if (r.x <= r.y && rect_min_q(u, v, ca, cb, cc, r.x, r.y, r.z, r.w) < thr_m) m |= 1u << w;
        }
        S.live[t] = m;
    }
}

__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Builds this wave's ordered list of batch entries j < lim that are live for
// it. Returns the count (wave-uniform).
template <class S_>
__device__ __forceinline__ int compact_live(S_ &S, int n, int lim, int wave, int lane) {
    int cnt = 0;
    for (int c = 0; c < n; c += 64) {
        const int j = c + lane;
        const bool bit = j < n && j < lim && ((S.live[j] >> wave) & 1u);
        const uint64_t m = ballot(bit);
        if (bit) S.list[wave][cnt + rank_in(m)] = (uint16_t)j;
        cnt += __popcll(m);
    }
    wave_sync_lds();
    return cnt;
}

template <class S_>
__device__ __forceinline__ void publish_rect(S_ &S, bool inimg, float fx, float fy, int wave,
                                             int lane) {
    const float inf = __builtin_inff();
    const float x0 = wave_min(inimg ? fx : inf), x1 = wave_max(inimg ? fx : -inf);
    const float y0 = wave_min(inimg ? fy : inf), y1 = wave_max(inimg ? fy : -inf);
    if (lane == 0) {
        S.rect[wave] = make_float4(x0, x1, y0, y1);
        S.flag[wave] = 0;
    }
}

template <int MAXW>
__global__ __launch_bounds__(MAXW * 64) void raster_fwd_kernel(const RasterArgs A, float *out_rgb,
                                                               float *out_alpha, float *out_T,
                                                               int32_t *out_stop) {
    __shared__ Stage<MAXW> S;
    const int tile_id = xcd_band(blockIdx.x, A.n_tiles);
    if (tile_id < 0) return;   // whole workgroup
    const int tx = tile_id % A.tiles_x, ty = tile_id / A.tiles_x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nwaves = blockDim.x >> 6;
    int lx, ly;
    bool inblk;
    tile_pixel(tid, A.tile, lx, ly, inblk);
    const int px = tx * A.tile + lx, py = ty * A.tile + ly;
    const bool inimg = inblk && lx < A.tile && ly < A.tile && px < A.W && py < A.H;
    const float fx = (float)px + 0.5f, fy = (float)py + 0.5f;
    publish_rect(S, inimg, fx, fy, wave, lane);

    const int start = A.offsets[tile_id], end = A.offsets[tile_id + 1];
    float T = 1.0f, cr = 0.f, cg = 0.f, cb = 0.f, acc = 0.f;
    int stop = start;
    bool done = !inimg;

    for (int base = start; base < end; base += kBatch) {
        __syncthreads();
        bool all_done = true;
        for (int w = 0; w < nwaves; ++w) all_done &= S.flag[w] != 0;
        if (all_done) break;                 // the whole tile is opaque
        const int n = min(kBatch, end - base);
        stage_batch(S, A, base, n, nwaves);
        __syncthreads();
        const int cnt = compact_live(S, n, n, wave, lane);
        if (ballot(!done) != 0) {
            for (int k = 0; k < cnt; ++k) {
                const int j = S.list[wave][k];
                if (!done) {
                    const float4 geo = S.geo[j];
                    const float4 con = S.con[j];
                    const float dx = fx - geo.x, dy = fy - geo.y;
                    const float power = splat_power(dx, dy, con.x, con.y, con.z);
                    if (power <= 0.0f) {
                        const float alpha = fminf(kAlphaMax, geo.z * __expf(power));
                        if (alpha >= kAlphaMin) {
                            const float4 col = S.col[j];
                            const float w = alpha * T;
                            cr = fmaf(w, col.x, cr);
                            cg = fmaf(w, col.y, cg);
                            cb = fmaf(w, col.z, cb);
                            acc += w;
                            T = T * (1.0f - alpha);
                            stop = base + j + 1;
                            if (T < A.t_min) done = true;
                        }
                    }
                }
                if (ballot(!done) == 0) break;
            }
        }
        const bool wave_done = ballot(!done) == 0;
        if (lane == 0) S.flag[wave] = wave_done ? 1 : 0;
    }
    if (!inimg) return;
    const int64_t o = (int64_t)py * A.W + px;
    if (A.has_bg) {
        // Rounded as the separate torch ops of metal_backend.py's blend
        // (rgb + (1 - alpha).clamp_min(0) * bg): no fused multiply-add.
        const float r = fmaxf(1.0f - acc, 0.0f);
        cr = __fadd_rn(cr, __fmul_rn(r, A.bg[0]));
        cg = __fadd_rn(cg, __fmul_rn(r, A.bg[1]));
        cb = __fadd_rn(cb, __fmul_rn(r, A.bg[2]));
    }
    out_rgb[3 * o] = cr;
    out_rgb[3 * o + 1] = cg;
    out_rgb[3 * o + 2] = cb;
    out_alpha[o] = acc;
    out_T[o] = T;
    out_stop[o] = stop;
}

struct RasterGrads {
    const float *final_T;
    const int32_t *stop;
    const float *grad_rgb, *grad_alpha;
    const float *alpha;   // the forward's alpha; read only with a background
    float *d_uv, *d_conic, *d_op, *d_col, *d_abs;
};

template <int MAXW>
__global__ __launch_bounds__(MAXW * 64) void raster_bwd_kernel(const RasterArgs A,
                                                               const RasterGrads G) {
    __shared__ StageBwd<MAXW> S;
    const int tile_id = xcd_band(blockIdx.x, A.n_tiles);
    if (tile_id < 0) return;
    const int tx = tile_id % A.tiles_x, ty = tile_id / A.tiles_x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nwaves = blockDim.x >> 6;
    int lx, ly;
    bool inblk;
    tile_pixel(tid, A.tile, lx, ly, inblk);
    const int px = tx * A.tile + lx, py = ty * A.tile + ly;
    const bool inimg = inblk && lx < A.tile && ly < A.tile && px < A.W && py < A.H;
    const float fx = (float)px + 0.5f, fy = (float)py + 0.5f;
    publish_rect(S, inimg, fx, fy, wave, lane);

    const int start = A.offsets[tile_id];
    const int64_t o = inimg ? (int64_t)py * A.W + px : 0;
    float T = inimg ? G.final_T[o] : 1.0f;
    const int my_stop = inimg ? G.stop[o] : start;
    const float gr = inimg ? G.grad_rgb[3 * o] : 0.f;
    const float gg = inimg ? G.grad_rgb[3 * o + 1] : 0.f;
    const float gb = inimg ? G.grad_rgb[3 * o + 2] : 0.f;
    float ga = inimg ? G.grad_alpha[o] : 0.f;
    // The background blend's share: d rgb_out / d alpha = -bg where
    // 1 - alpha >= 0 (torch's clamp_min passes the gradient at the bound).
    if (A.has_bg && inimg && 1.0f - G.alpha[o] >= 0.0f)
        ga -= gr * A.bg[0] + gg * A.bg[1] + gb * A.bg[2];
    const bool want_abs = G.d_abs != nullptr;

    // Nothing at or past a pixel's stop index contributed to it.
    const int wstop = wave_max_i(my_stop);
    if (lane == 0) S.flag[wave] = wstop;
    __syncthreads();
    int bstop = start;
    for (int w = 0; w < nwaves; ++w) bstop = max(bstop, S.flag[w]);

    float sr = 0.f, sg = 0.f, sb = 0.f, sa = 0.f;
    const int nbatch = (bstop - start + kBatch - 1) / kBatch;
    for (int bi = nbatch - 1; bi >= 0; --bi) {
        const int base = start + bi * kBatch;
        const int n = min(kBatch, bstop - base);
        __syncthreads();   // the previous batch's flush has read S.grad
        stage_batch(S, A, base, n, nwaves);
        for (int t = threadIdx.x; t < kGradSlots * kBatch; t += blockDim.x)
            (&S.grad[0][0])[t] = 0.f;
        __syncthreads();
        const int cnt = compact_live(S, n, wstop - base, wave, lane);
        for (int k = cnt - 1; k >= 0; --k) {
            const int j = S.list[wave][k];
            const int i = base + j;
            const float4 geo = S.geo[j];
            const float4 con = S.con[j];
            const float dx = fx - geo.x, dy = fy - geo.y;
            const float power = splat_power(dx, dy, con.x, con.y, con.z);
            const float gauss = __expf(power);
            const float op = geo.z;
            const float alpha_raw = op * gauss;
            const float alpha = fminf(kAlphaMax, alpha_raw);
            const bool active = inimg && i < my_stop && power <= 0.0f && alpha >= kAlphaMin;
            if (ballot(active) == 0) continue;
            float v[kGradSlots];
#pragma unroll
            for (int q = 0; q < kGradSlots; ++q) v[q] = 0.f;
            if (active) {
                const float4 col = S.col[j];
                const float om = fmaxf(1.0f - alpha, 1e-8f);
                T = T / om;
                const float iom = 1.0f / om;
                const float w = alpha * T;
                v[0] = w * gr;
                v[1] = w * gg;
                v[2] = w * gb;
                const float dal = gr * (T * col.x - sr * iom) + gg * (T * col.y - sg * iom) +
                                  gb * (T * col.z - sb * iom) + ga * (T - sa * iom);
                sr = fmaf(w, col.x, sr);
                sg = fmaf(w, col.y, sg);
                sb = fmaf(w, col.z, sb);
                sa += w;
                if (alpha_raw <= kAlphaMax) {
                    v[8] = dal * gauss;
                    const float dpow = dal * op * gauss;
                    v[3] = dpow * (con.x * dx + con.y * dy);
                    v[4] = dpow * (con.y * dx + con.z * dy);
                    v[5] = -0.5f * dpow * dx * dx;
                    v[6] = -dpow * dx * dy;
                    v[7] = -0.5f * dpow * dy * dy;
                    if (want_abs) v[9] = sqrtf(v[3] * v[3] + v[4] * v[4]);
                }
            }
            // Sums over the wave of v[0..9], deposited into S.grad[.][j]
            // with four lanes per LDS atomic (see reduce10_to_rows).
            float q0, q1, q2;
            reduce10_to_rows(v, q0, q1, q2);
            if ((lane & 15) == 0) {
                const int row = lane >> 4;
                // Row r of Q0 holds slot {0,2,1,3}[r], of Q1 {4,6,5,7}[r],
                // of Q2 {8,-,9,-}[r].
                const int s0 = (row & 1) * 2 + (row >> 1);
                if (q0 != 0.f) atomicAdd(&S.grad[s0][j], q0);
                if (q1 != 0.f) atomicAdd(&S.grad[4 + s0][j], q1);
                if ((row & 1) == 0 && q2 != 0.f && (row == 0 || want_abs))
                    atomicAdd(&S.grad[8 + (row >> 1)][j], q2);
            }
        }
        __syncthreads();
        // One thread per batch entry publishes the tile's sums.
        for (int t = threadIdx.x; t < n; t += blockDim.x) {
            const int g = S.id[t];
            float s[kGradSlots];
#pragma unroll
            for (int q = 0; q < kGradSlots; ++q) s[q] = S.grad[q][t];
            if (s[0] != 0.f) unsafeAtomicAdd(G.d_col + 3 * g, s[0]);
            if (s[1] != 0.f) unsafeAtomicAdd(G.d_col + 3 * g + 1, s[1]);
            if (s[2] != 0.f) unsafeAtomicAdd(G.d_col + 3 * g + 2, s[2]);
            if (s[3] != 0.f) unsafeAtomicAdd(G.d_uv + 2 * g, s[3]);
            if (s[4] != 0.f) unsafeAtomicAdd(G.d_uv + 2 * g + 1, s[4]);
            if (s[5] != 0.f) unsafeAtomicAdd(G.d_conic + 3 * g, s[5]);
            if (s[6] != 0.f) unsafeAtomicAdd(G.d_conic + 3 * g + 1, s[6]);
            if (s[7] != 0.f) unsafeAtomicAdd(G.d_conic + 3 * g + 2, s[7]);
            if (s[8] != 0.f) unsafeAtomicAdd(G.d_op + g, s[8]);
            if (want_abs && s[9] != 0.f) unsafeAtomicAdd(G.d_abs + g, s[9]);
        }
    }
}

// Zero-fills up to five float buffers in one launch (gradient accumulators).
struct ZeroSpans {
    float *p[5];
    int64_t n[5];
};

__global__ __launch_bounds__(256) void zero_spans_kernel(const ZeroSpans Z) {
    const int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * 256;
#pragma unroll
    for (int k = 0; k < 5; ++k) {
        if (!Z.p[k]) continue;
        for (int64_t i = i0; i < Z.n[k]; i += stride) Z.p[k][i] = 0.f;
    }
}

static int32_t check_raster(const char *who, int64_t N, const void *uv, const void *conic,
                            const void *opac, const void *color, const void *ids,
                            const void *offsets, int W, int H, int tile, int tiles_x) {
    MG_REQUIRE(W > 0 && H > 0, "%s: image %dx%d", who, W, H);
    MG_REQUIRE(tile >= 1, "%s: tile %d", who, tile);
    MG_REQUIRE(tile * tile <= 1024,
               "tile %d needs %d threads per threadgroup; %s allows at most 1024 on this GPU",
               tile, tile * tile, who);
    MG_REQUIRE(tiles_x == (W + tile - 1) / tile, "%s: tiles_x %d does not cover W %d at tile %d",
               who, tiles_x, W, tile);
    MG_REQUIRE(N >= 0 && N < (1LL << 31), "%s: N = %lld", who, (long long)N);
    MG_REQUIRE(offsets, "%s: null tile offsets", who);
    MG_REQUIRE(N == 0 || (uv && conic && opac && color), "%s: null tensor pointer", who);
    (void)ids;
    return MG_OK;
}

}  // namespace mg

using namespace mg;

extern "C" {

int32_t mg_rasterize_forward(int64_t N, const float *uv, const float *conic, const float *opacity,
                             const float *color, const int32_t *gauss_ids,
                             const int32_t *tile_offsets, int32_t W, int32_t H, int32_t tile,
                             int32_t tiles_x, float t_min, const float *background,
                             float *out_rgb, float *out_alpha, float *out_T, int32_t *out_stop,
                             mg_stream_t stream) {
    int32_t rc = check_raster("rasterize_forward", N, uv, conic, opacity, color, gauss_ids,
                              tile_offsets, W, H, tile, tiles_x);
    if (rc != MG_OK) return rc;
    MG_REQUIRE(out_rgb && out_alpha && out_T && out_stop, "rasterize_forward: null output");
    const int tiles_y = (H + tile - 1) / tile;
    RasterArgs A{uv, conic, opacity, color, gauss_ids, tile_offsets, W, H, tile, tiles_x,
                 tiles_x * tiles_y, t_min, background != nullptr,
                 {background ? background[0] : 0.f, background ? background[1] : 0.f,
                  background ? background[2] : 0.f}};
    const int threads = ((tile * tile + 63) / 64) * 64;
    const int grid = (int)ceil_div(A.n_tiles, kXcds) * kXcds;
    TimedScope ts("rasterize_forward", as_stream(stream));
    if (threads <= 4 * 64)
        raster_fwd_kernel<4><<<grid, threads, 0, as_stream(stream)>>>(A, out_rgb, out_alpha,
                                                                       out_T, out_stop);
    else
        raster_fwd_kernel<kMaxWaves><<<grid, threads, 0, as_stream(stream)>>>(
            A, out_rgb, out_alpha, out_T, out_stop);
    MG_LAUNCHED("raster_fwd_kernel");
    return MG_OK;
}

int32_t mg_rasterize_backward(int64_t N, const float *uv, const float *conic,
                              const float *opacity, const float *color,
                              const int32_t *gauss_ids, const int32_t *tile_offsets,
                              const float *final_T, const int32_t *stop, const float *grad_rgb,
                              const float *grad_alpha, const float *alpha,
                              const float *background, int32_t W, int32_t H, int32_t tile,
                              int32_t tiles_x, float *d_uv, float *d_conic, float *d_opacity,
                              float *d_color, float *d_absuv, mg_stream_t stream) {
    int32_t rc = check_raster("rasterize_backward", N, uv, conic, opacity, color, gauss_ids,
                              tile_offsets, W, H, tile, tiles_x);
    if (rc != MG_OK) return rc;
    MG_REQUIRE(final_T && stop && grad_rgb && grad_alpha, "rasterize_backward: null input");
    MG_REQUIRE(!background || alpha, "rasterize_backward: a background needs the forward's alpha");
    MG_REQUIRE(N == 0 || (d_uv && d_conic && d_opacity && d_color),
               "rasterize_backward: null gradient output");
    hipStream_t s = as_stream(stream);
    if (N > 0) {
        ZeroSpans Z{{d_uv, d_conic, d_opacity, d_color, d_absuv},
                    {2 * N, 3 * N, N, 3 * N, d_absuv ? N : 0}};
        const int64_t blocks = min(ceil_div(3 * N, 256), (int64_t)4096);
        zero_spans_kernel<<<(unsigned)blocks, 256, 0, s>>>(Z);
        MG_LAUNCHED("zero_spans_kernel");
    }
    const int tiles_y = (H + tile - 1) / tile;
    RasterArgs A{uv, conic, opacity, color, gauss_ids, tile_offsets, W, H, tile, tiles_x,
                 tiles_x * tiles_y, 0.0f, background != nullptr,
                 {background ? background[0] : 0.f, background ? background[1] : 0.f,
                  background ? background[2] : 0.f}};
    RasterGrads Gr{final_T, stop, grad_rgb, grad_alpha, alpha, d_uv, d_conic, d_opacity, d_color,
                   d_absuv};
    const int threads = ((tile * tile + 63) / 64) * 64;
    const int grid = (int)ceil_div(A.n_tiles, kXcds) * kXcds;
    TimedScope ts("rasterize_backward", s);
    if (threads <= 4 * 64)
        raster_bwd_kernel<4><<<grid, threads, 0, s>>>(A, Gr);
    else
        raster_bwd_kernel<kMaxWaves><<<grid, threads, 0, s>>>(A, Gr);
    MG_LAUNCHED("raster_bwd_kernel");
    return MG_OK;
}

}  // extern "C"
