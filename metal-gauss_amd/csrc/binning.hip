// Tile binning: per-Gaussian tile count, exclusive scan, (tile|depth) key
// emission and tile ranges over the sorted keys, plus the depth-first
// pipeline (mg_bin_lists_begin/finish) that builds the same lists with two
// cheaper sorts.
//
// Membership follows metal_gauss/csrc/binning.metal:25-90 and
// metal_backend.py:149-189: a Gaussian claims tile t when the minimum of its
// conic's quadratic form over the tile rectangle is below 2 ln(255 opacity),
// which is exactly the rasteriser's alpha >= 1/255 cutoff, so dropped pairs
// change no pixel. Keys and order are an integer contract that the CPU oracle
// reproduces bit for bit, so the float work here is written to be
// reproducible:
//   * FP contraction is off in the tile walk (no fused multiply-adds), so
//     every product and sum rounds exactly as a scalar fp32 CPU evaluation of
//     the same expression does;
//   * division is IEEE (hipcc's default correctly rounded fp32 divide);
//   * the threshold is 2 * log(255 op) taken in double and rounded once to
//     fp32, i.e. the correctly rounded value, rather than a fast fp32 log
//     whose last bit differs between libraries.
#include "mg_common.h"
#include "mg_sort.h"

namespace mg {

constexpr int kBinThreads = 256;

// 2 ln(255 op), correctly rounded to fp32; 0 when the Gaussian can never reach
// alpha 1/255 (it then claims no tiles).
__device__ __forceinline__ float level_threshold(float op, bool &live) {
    const float oa = 255.0f * op;
    live = oa > 1.0f;
    return live ? (float)(2.0 * log((double)oa)) : 0.0f;
}

struct BinArgs {
    int64_t N;
    const float *uv, *rxy, *conic, *opac, *depth;
    const int32_t *valid;
    int32_t W, H, tile, tiles_x, tiles_y;
};

// Everything the tile walk needs for one Gaussian, in one 32-byte sector:
// the centre, the conic with its diagonal clamped at 1e-12, the level
// threshold and the clamped tile rectangle (x0 | x1 << 16, y0 | y1 << 16).
// The count pass writes it in Gaussian order; the write pass gathers it in
// depth order, one sector per Gaussian instead of six scattered arrays.
struct __align__(16) BinRec {
    float ux, uy, a, b;
    float c, thr;
    uint32_t xs, ys;
};

// False when the Gaussian claims no tile (invalid, or alpha below 1/255 at
// every point); r is then filled from zeroed inputs and not used. Every input
// is requested before any is tested: a load whose value is needed only past
// a branch is issued there and waited for, one memory round trip per branch.
__device__ __forceinline__ bool make_rec(const BinArgs &A, int64_t g, BinRec &r) {
    const bool test = A.conic != nullptr;
    const bool vld = A.valid[g] != 0;
    float ux = A.uv[2 * g], uy = A.uv[2 * g + 1];
    float rx = A.rxy[2 * g], ry = A.rxy[2 * g + 1];
    float op = 0.0f, ca = 0.0f, cb = 0.0f, cc = 0.0f;
    if (test) {
        op = A.opac[g];
        ca = A.conic[3 * g];
        cb = A.conic[3 * g + 1];
        cc = A.conic[3 * g + 2];
    }
    // Invalid Gaussians may carry non-finite extents.
    ux = vld ? ux : 0.0f;
    uy = vld ? uy : 0.0f;
    rx = vld ? rx : 0.0f;
    ry = vld ? ry : 0.0f;
    const float tf = (float)A.tile;
    // For a power-of-two tile, x / tile and x * (1 / tile) are the same
    // correctly rounded value (1 / tile is exact), and the product is one
    // instruction instead of a division sequence.
    float e0 = ux - rx, e1 = ux + rx, f0 = uy - ry, f1 = uy + ry;
    if ((A.tile & (A.tile - 1)) == 0) {
        const float it = 1.0f / tf;
        e0 *= it; e1 *= it; f0 *= it; f1 *= it;
    } else {
        e0 /= tf; e1 /= tf; f0 /= tf; f1 /= tf;
    }
    int x0 = (int)floorf(e0), x1 = (int)floorf(e1);
    int y0 = (int)floorf(f0), y1 = (int)floorf(f1);
    x0 = min(max(x0, 0), A.tiles_x - 1);
    x1 = min(max(x1, 0), A.tiles_x - 1);
    y0 = min(max(y0, 0), A.tiles_y - 1);
    y1 = min(max(y1, 0), A.tiles_y - 1);
    r.ux = ux;
    r.uy = uy;
    r.xs = (uint32_t)x0 | ((uint32_t)x1 << 16);
    r.ys = (uint32_t)y0 | ((uint32_t)y1 << 16);
    // Without a conic (the circular-bounds caller of metal_backend.py:111-147)
    // every tile of the rectangle is claimed.
    bool live = true;
    r.thr = test ? level_threshold(op, live) : 0.0f;
    r.a = test ? fmaxf(ca, 1e-12f) : 0.0f;
    r.b = test ? cb : 0.0f;
    r.c = test ? fmaxf(cc, 1e-12f) : 0.0f;
    return vld && live;
}

// Walks the rectangle, rows outer and columns inner (binning.metal:74-77),
// calling emit(n, tile_id, loc) for the n-th claimed tile, loc being its
// row-major index in the rectangle; returns the count.
//
// A tile is claimed when the minimum over the tile rectangle of
// q(d) = a dx^2 + 2 b dx dy + c dy^2 is below the threshold. The minimum is 0
// when the centre lies inside; otherwise it lies on an edge. On a horizontal
// edge y = yc the unconstrained minimiser is x = ux - b (yc - uy) / a,
// clamped to the edge; on a vertical edge x = xc it is
// y = uy - b (xc - ux) / c. That minimiser depends on the edge line alone,
// so it is computed once per row boundary and once per column boundary and
// shared by the tiles on either side. Every value is the same fp32
// expression the oracle evaluates per tile, so each decision is bit-exact.
// FP contraction is off: every product and sum rounds separately.
template <typename Emit>
__device__ __forceinline__ int rec_walk(const BinRec &r, bool test, int tile, int W, int H,
                                        int tiles_x, Emit emit) {
#pragma clang fp contract(off)
    const int x0 = (int)(r.xs & 0xffffu), x1 = (int)(r.xs >> 16);
    const int y0 = (int)(r.ys & 0xffffu), y1 = (int)(r.ys >> 16);
    int n = 0, loc = 0;
    if (!test) {
        for (int ty = y0; ty <= y1; ++ty)
            for (int tx = x0; tx <= x1; ++tx, ++loc) emit(n++, (uint32_t)(ty * tiles_x + tx), loc);
        return n;
    }
    const float mux = r.ux, muy = r.uy, a = r.a, b = r.b, c = r.c;
    float ry0 = (float)(y0 * tile);
    float u0 = mux - b * (ry0 - muy) / a;
    for (int ty = y0; ty <= y1; ++ty) {
        const float ry1 = fminf((float)((ty + 1) * tile), (float)H);
        const float u1 = mux - b * (ry1 - muy) / a;
        const float ey0 = ry0 - muy, ey1 = ry1 - muy;
        const bool yin = muy >= ry0 && muy <= ry1;
        float rx0 = (float)(x0 * tile);
        float v0 = muy - b * (rx0 - mux) / c;
        for (int tx = x0; tx <= x1; ++tx) {
            const float rx1 = fminf((float)((tx + 1) * tile), (float)W);
            const float v1 = muy - b * (rx1 - mux) / c;
            bool claim = yin && mux >= rx0 && mux <= rx1;
            if (!claim) {
                float ex = fminf(fmaxf(u0, rx0), rx1) - mux;
                float best = a * ex * ex + 2.0f * b * ex * ey0 + c * ey0 * ey0;
                ex = fminf(fmaxf(u1, rx0), rx1) - mux;
                best = fminf(best, a * ex * ex + 2.0f * b * ex * ey1 + c * ey1 * ey1);
                float ey = fminf(fmaxf(v0, ry0), ry1) - muy;
                ex = rx0 - mux;
                best = fminf(best, a * ex * ex + 2.0f * b * ex * ey + c * ey * ey);
                ey = fminf(fmaxf(v1, ry0), ry1) - muy;
                ex = rx1 - mux;
                best = fminf(best, a * ex * ex + 2.0f * b * ex * ey + c * ey * ey);
                claim = best < r.thr;
            }
            if (claim) emit(n++, (uint32_t)(ty * tiles_x + tx), loc);
            ++loc;
            rx0 = rx1;      // equal to (tx + 1) * tile unless this is the last column
            v0 = v1;
        }
        ry0 = ry1;          // likewise for rows
        u0 = u1;
    }
    return n;
}

// One tile's decision, with exactly the expressions rec_walk evaluates for it
// (its shared edge minimisers are the same expressions of the same edge
// lines), so a wave that splits a rectangle over its lanes decides every
// tile as the walk does, bit for bit.
__device__ __forceinline__ bool tile_claim(const BinRec &r, bool test, int tx, int ty, int tile,
                                           int W, int H) {
#pragma clang fp contract(off)
    if (!test) return true;
    const float mux = r.ux, muy = r.uy, a = r.a, b = r.b, c = r.c;
    const float ry0 = (float)(ty * tile), ry1 = fminf((float)((ty + 1) * tile), (float)H);
    const float rx0 = (float)(tx * tile), rx1 = fminf((float)((tx + 1) * tile), (float)W);
    if (muy >= ry0 && muy <= ry1 && mux >= rx0 && mux <= rx1) return true;
    const float u0 = mux - b * (ry0 - muy) / a;
    const float u1 = mux - b * (ry1 - muy) / a;
    const float v0 = muy - b * (rx0 - mux) / c;
    const float v1 = muy - b * (rx1 - mux) / c;
    const float ey0 = ry0 - muy, ey1 = ry1 - muy;
    float ex = fminf(fmaxf(u0, rx0), rx1) - mux;
    float best = a * ex * ex + 2.0f * b * ex * ey0 + c * ey0 * ey0;
    ex = fminf(fmaxf(u1, rx0), rx1) - mux;
    best = fminf(best, a * ex * ex + 2.0f * b * ex * ey1 + c * ey1 * ey1);
    float ey = fminf(fmaxf(v0, ry0), ry1) - muy;
    ex = rx0 - mux;
    best = fminf(best, a * ex * ex + 2.0f * b * ex * ey + c * ey * ey);
    ey = fminf(fmaxf(v1, ry0), ry1) - muy;
    ex = rx1 - mux;
    best = fminf(best, a * ex * ex + 2.0f * b * ex * ey + c * ey * ey);
    return best < r.thr;
}

// Rectangles larger than this many tiles are walked by a whole wave instead
// of one thread: near-camera Gaussians can cover thousands of tiles, and one
// thread walking them holds up its workgroup.
constexpr int kWaveWalkArea = 32;

// A wave's walk of one large rectangle, lanes on fixed columns. The
// rectangle is cut into strips of s columns; a step covers R rows of a strip
// (lane = row group * s + column), with R and s chosen per rectangle for the
// fewest steps. A tile's four edge minima are then selects between values
// that depend on a row boundary, a column boundary or one corner:
//   * the top edge of row i, at x = clamp(u_i, X_j, X_j+1): the corner value
//     at X_j (u_i below the tile), at X_j+1 (above), else M_i, the minimum on
//     the row boundary line; likewise the bottom edge with boundary i + 1 and
//     the left / right edges with the column boundaries' v_j, v_j+1, N_j, N_j+1;
//   * a corner value (A_j + P_j ey_i) + C_i splits the walk's quadratic form
//     a ex^2 + 2 b ex ey + c ey^2 (evaluated left to right, no contraction)
//     into its column part A = a ex ex, P = 2 b ex and row part C = c ey ey.
// Every value is the walk's own fp32 expression on the same operands (the
// clamped coordinate equals the corner, or u / v itself), so each decision
// is bit for bit the walk's. The row boundaries {u, Y, C, M} are computed
// once per rectangle into the wave's LDS slice, the column boundaries once
// per strip into registers. Rectangles taller than the slice test each tile
// with tile_claim. The tiles are visited strip by strip, not in row-major
// order: a Gaussian's pairs go to distinct tiles, so their order within its
// run does not reach the sorted tile lists.
constexpr int kRowSlots = 128;
static_assert(kRowSlots * 16 == 64 * kWaveWalkArea, "the row slice aliases the small-claim bytes");

// The shape of a wave's walk over one large rectangle: ns strips of s
// columns, each nr steps of R rows; lane = row group rg * s + column cl.
// A function of the rectangle's size alone, so the count and write passes
// step through a rectangle identically.
struct StripPlan {
    int R, s, ns, nr, rg, cl;
    bool lane_ok;
};

// min(v, v of the lane the DPP control names); lanes with no such lane, or
// outside the row mask, keep v.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_min_u32(uint32_t v) {
    return min(v, (uint32_t)__builtin_amdgcn_update_dpp((int)0xFFFFFFFFu, (int)v, CTRL,
                                                        ROW_MASK, 0xf, false));
}

__device__ __forceinline__ StripPlan strip_plan(const BinRec &r, int lane) {
    const int w = (int)(r.xs >> 16) - (int)(r.xs & 0xffffu) + 1;
    const int h = (int)(r.ys >> 16) - (int)(r.ys & 0xffffu) + 1;
    // Lane l prices R = l + 1 rows a step (strips of min(w, 64 / R)
    // columns); the wave takes the fewest steps, the smallest R on ties.
    // The quotients of these small integers (w, h < 2^16, R <= 64) come from
    // correctly rounded float divisions, exact after floor / ceil; the step
    // count is held below 2^26 (beyond it any choice is as good), so the key
    // steps << 6 | lane fits 32 bits and the minimum takes DPP row shifts
    // and broadcasts rather than lane shuffles.
    uint32_t key;
    {
        const int R = lane + 1;
        const int s = min(w, (int)(64.0f / (float)R));
        const uint32_t ns = (uint32_t)ceilf((float)w / (float)s);
        const uint32_t nr = (uint32_t)ceilf((float)h / (float)R);
        const uint32_t steps = min(ns * nr, (1u << 26) - 1u);
        key = steps << 6 | (uint32_t)lane;
        key = dpp_min_u32<0x111>(key);        // row_shr:1
        key = dpp_min_u32<0x112>(key);        // row_shr:2
        key = dpp_min_u32<0x114>(key);        // row_shr:4
        key = dpp_min_u32<0x118>(key);        // row_shr:8
        key = dpp_min_u32<0x142, 0xa>(key);   // row_bcast:15
        key = dpp_min_u32<0x143, 0xc>(key);   // row_bcast:31
    }
    StripPlan P;
    P.R = (int)(__builtin_amdgcn_readlane(key, 63) & 63u) + 1;
    P.s = min(w, (int)(64.0f / (float)P.R));
    P.ns = (int)ceilf((float)w / (float)P.s);
    P.nr = (int)ceilf((float)h / (float)P.R);
    P.rg = (int)((float)lane / (float)P.s);
    P.cl = lane - P.rg * P.s;
    P.lane_ok = lane < P.R * P.s;
    return P;
}

template <class Step>
__device__ __forceinline__ void strip_walk(const BinRec &r, const StripPlan &P, bool test,
                                           int tile, int W, int H, float4 *rows, int lane,
                                           Step &&step) {
#pragma clang fp contract(off)
    // The rectangle is the wave's (read from LDS at one address): said so,
    // the compiler keeps its bounds in scalar registers and branches on
    // `fast` once instead of masking both step bodies every step.
    const uint32_t xs = __builtin_amdgcn_readfirstlane(r.xs);
    const uint32_t ys = __builtin_amdgcn_readfirstlane(r.ys);
    const int x0 = (int)(xs & 0xffffu), y0 = (int)(ys & 0xffffu);
    const int w = (int)(xs >> 16) - x0 + 1, h = (int)(ys >> 16) - y0 + 1;
    const int R = P.R, s = P.s, ns = P.ns, nr = P.nr, rg = P.rg, cl = P.cl;
    const bool lane_ok = P.lane_ok;
    const float mux = r.ux, muy = r.uy, a = r.a, b = r.b, c = r.c, thr = r.thr;
    const bool fast = test && h + 1 <= kRowSlots;
    if (fast) {
        for (int i = lane; i <= h; i += 64) {
            // Row boundary of row y0 + i: its top edge; the last is the
            // bottom of row y1, clamped to the image as the walk clamps it.
            const int ty = y0 + i;
            const float Y = i == 0 ? (float)(ty * tile) : fminf((float)(ty * tile), (float)H);
            const float u = mux - b * (Y - muy) / a;
            const float ey = Y - muy, ex = u - mux;
            const float C = c * ey * ey;
            rows[i] = make_float4(u, Y, C, a * ex * ex + 2.0f * b * ex * ey + C);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    for (int k = 0; k < ns; ++k) {
        const int j = k * s + cl;
        const bool col_ok = lane_ok && j < w;
        const int tx = x0 + min(j, w - 1);
        // Column boundaries j and j + 1 (the tile's left and right edges).
        const float Xl = (float)(tx * tile), Xr = fminf((float)((tx + 1) * tile), (float)W);
        const float vl = muy - b * (Xl - mux) / c, vr = muy - b * (Xr - mux) / c;
        const float exl = Xl - mux, exr = Xr - mux;
        const float Al = a * exl * exl, Pl = 2.0f * b * exl;
        const float Ar = a * exr * exr, Pr = 2.0f * b * exr;
        const float eyl = vl - muy, eyr = vr - muy;
        const float Nl = Al + Pl * eyl + c * eyl * eyl, Nr = Ar + Pr * eyr + c * eyr * eyr;
        const bool in_x = mux >= Xl && mux <= Xr;
        for (int t = 0; t < nr; ++t) {
            const int i = t * R + rg;
            const bool ok = col_ok && i < h;
            const int ty = y0 + min(i, h - 1);
            bool claim = ok;
            if (fast) {
                const float4 r0 = rows[min(i, h - 1)], r1 = rows[min(i, h - 1) + 1];
                const float ey0 = r0.y - muy, ey1 = r1.y - muy;
                const float F00 = Al + Pl * ey0 + r0.z, F01 = Ar + Pr * ey0 + r0.z;
                const float F10 = Al + Pl * ey1 + r1.z, F11 = Ar + Pr * ey1 + r1.z;
                const float top = r0.x >= Xl ? (r0.x > Xr ? F01 : r0.w) : F00;
                const float bot = r1.x >= Xl ? (r1.x > Xr ? F11 : r1.w) : F10;
                const float lft = vl >= r0.y ? (vl > r1.y ? F10 : Nl) : F00;
                const float rgt = vr >= r0.y ? (vr > r1.y ? F11 : Nr) : F01;
                float best = fminf(top, bot);
                best = fminf(best, lft);
                best = fminf(best, rgt);
                const bool in = in_x && muy >= r0.y && muy <= r1.y;
                claim = ok && (in || best < thr);
            } else if (test) {
                claim = ok && tile_claim(r, true, tx, ty, tile, W, H);
            }
            step(claim, tx, ty);
        }
    }
    // The slice is rewritten for the wave's next rectangle.
    __builtin_amdgcn_wave_barrier();
}

// The count pass keeps each large rectangle's claims, one 64-bit word per
// walk step (the wave's ballot of that step's claims), so the write pass
// replays the steps instead of testing every tile again. A count workgroup
// has kBlockWords words, taken by its rectangles as their walks start; a
// rectangle whose steps no longer fit is walked again by the write pass.
// Its mask word records where its words are: 1 + the first word's index,
// plus the step count from bit kWordSteps (0: not kept).
constexpr int kBlockWords = 1024;
constexpr int kWordSteps = 11;
static_assert(kBlockWords < (1 << kWordSteps), "the first word's index + 1 fits below the steps");

__device__ __forceinline__ uint32_t kept_mask(int first, int nst) {
    return (uint32_t)(first + 1) | ((uint32_t)nst << kWordSteps);
}
__device__ __forceinline__ int kept_first(uint32_t m) {
    return (int)(m & ((1u << kWordSteps) - 1u)) - 1;
}
__device__ __forceinline__ int kept_steps(uint32_t m) { return (int)(m >> kWordSteps); }

__device__ __forceinline__ int rec_area(const BinRec &r) {
    return ((int)(r.xs >> 16) - (int)(r.xs & 0xffffu) + 1) *
           ((int)(r.ys >> 16) - (int)(r.ys & 0xffffu) + 1);
}

// Tile t (row-major) of a rectangle of width w starting at (x0, y0).
__device__ __forceinline__ void rect_tile(const BinRec &r, int t, int &tx, int &ty) {
    const int x0 = (int)(r.xs & 0xffffu), y0 = (int)(r.ys & 0xffffu);
    const int w = (int)(r.xs >> 16) - x0 + 1;
    ty = y0 + t / w;
    tx = x0 + t % w;
}

__global__ __launch_bounds__(kBinThreads) void bin_count_kernel(const BinArgs A, int32_t *counts) {
    const int64_t g = (int64_t)blockIdx.x * kBinThreads + threadIdx.x;
    if (g >= A.N) return;
    BinRec r;
    int n = 0;
    if (make_rec(A, g, r))
        n = rec_walk(r, A.conic != nullptr, A.tile, A.W, A.H, A.tiles_x,
                     [](int, uint32_t, int) {});
    counts[g] = n;
}

__global__ __launch_bounds__(kBinThreads) void bin_write_kernel(const BinArgs A,
                                                                const int32_t *offsets,
                                                                uint64_t *keys, int32_t *ids) {
    const int64_t g = (int64_t)blockIdx.x * kBinThreads + threadIdx.x;
    if (g >= A.N) return;
    BinRec r;
    if (!make_rec(A, g, r)) return;
    const uint64_t dbits = (uint64_t)__float_as_uint(A.depth[g]);
    const int64_t at = offsets[g];
    rec_walk(r, A.conic != nullptr, A.tile, A.W, A.H, A.tiles_x, [&](int n, uint32_t t, int) {
        keys[at + n] = ((uint64_t)t << 32) | dbits;
        ids[at + n] = (int32_t)g;
    });
}

// ------------------------------------------------------------------- scan
// Three launches: per-chunk sums, a single-workgroup scan of those sums, and
// a downsweep that rescans each chunk and adds its prefix.
constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr int kScanChunk = kScanThreads * kScanItems;   // 2048

__device__ __forceinline__ int64_t wave_incl_scan(int64_t v, int lane) {
    for (int o = 1; o < 64; o <<= 1) {
        const int64_t t = __shfl_up(v, o, 64);
        if (lane >= o) v += t;
    }
    return v;
}

// Exclusive scan of one value per thread over a 256-thread workgroup; the
// workgroup total is returned through *total.
__device__ __forceinline__ int64_t block_excl_scan(int64_t v, int64_t *s_wave, int64_t *total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t incl = wave_incl_scan(v, lane);
    if (lane == 63) s_wave[wave] = incl;
    __syncthreads();
    int64_t before = 0, all = 0;
    for (int w = 0; w < kScanThreads / 64; ++w) {
        if (w < wave) before += s_wave[w];
        all += s_wave[w];
    }
    __syncthreads();
    *total = all;
    return before + incl - v;
}

// With idx (or *idx_dev, an index array chosen on the device), in[idx[i]] is
// gathered once and stored to gathered[i], which the downsweep then reads in
// order.
__global__ __launch_bounds__(kScanThreads) void scan_reduce_kernel(
    const int32_t *in, const int32_t *idx, const int32_t *const *idx_dev, int64_t n,
    int64_t *partials, int32_t *gathered) {
    __shared__ int64_t s_wave[kScanThreads / 64];
    if (idx_dev) idx = *idx_dev;
    const int64_t base = (int64_t)blockIdx.x * kScanChunk;
    int64_t s = 0;
#pragma unroll
    for (int r = 0; r < kScanItems; ++r) {
        const int64_t i = base + (int64_t)r * kScanThreads + threadIdx.x;
        if (i < n) {
            const int32_t v = in[idx ? idx[i] : i];
            if (idx) gathered[i] = v;
            s += v;
        }
    }
    int64_t total;
    block_excl_scan(s, s_wave, &total);
    if (threadIdx.x == 0) partials[blockIdx.x] = total;
}

__global__ __launch_bounds__(kScanThreads) void scan_partials_kernel(int64_t *partials,
                                                                     int64_t nparts,
                                                                     int64_t *total_out) {
    __shared__ int64_t s_wave[kScanThreads / 64];
    int64_t carry = 0;
    for (int64_t c0 = 0; c0 < nparts; c0 += kScanThreads) {
        const int64_t i = c0 + threadIdx.x;
        const int64_t v = i < nparts ? partials[i] : 0;
        int64_t tot;
        const int64_t ex = block_excl_scan(v, s_wave, &tot);
        if (i < nparts) partials[i] = carry + ex;
        carry += tot;
    }
    if (threadIdx.x == 0) *total_out = carry;
}

// May run in place (in == out): each thread reads its items before writing
// them and touches no other thread's.
__global__ __launch_bounds__(kScanThreads) void scan_down_kernel(const int32_t *in, int64_t n,
                                                                 const int64_t *partials,
                                                                 int32_t *out) {
    __shared__ int64_t s_wave[kScanThreads / 64];
    // Blocked arrangement: thread t owns items [t*8, t*8+8) of the chunk, so
    // one exclusive scan of the per-thread sums orders them correctly.
    const int64_t base = (int64_t)blockIdx.x * kScanChunk + (int64_t)threadIdx.x * kScanItems;
    int32_t v[kScanItems];
    int64_t s = 0;
#pragma unroll
    for (int r = 0; r < kScanItems; ++r) {
        v[r] = (base + r < n) ? in[base + r] : 0;
        s += v[r];
    }
    int64_t tot;
    int64_t run = block_excl_scan(s, s_wave, &tot) + partials[blockIdx.x];
#pragma unroll
    for (int r = 0; r < kScanItems; ++r) {
        if (base + r < n) out[base + r] = (int32_t)run;
        run += v[r];
    }
}

// -------------------------------------------------------------- tile ranges
// offsets[t] = first i with tile(keys[i]) >= t. Each boundary between
// consecutive keys fills the tiles it skips, so empty tiles get the index of
// the next non-empty one and offsets[n_tiles] = n.
__global__ __launch_bounds__(256) void tile_ranges_kernel(const uint64_t *keys, int64_t n,
                                                          int32_t n_tiles, int32_t *offsets) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i > n) return;
    const int64_t prev = i == 0 ? -1 : (int64_t)(keys[i - 1] >> 32);
    const int64_t cur = i == n ? (int64_t)n_tiles : (int64_t)(keys[i] >> 32);
    for (int64_t t = prev + 1; t <= cur && t <= n_tiles; ++t) offsets[t] = (int32_t)i;
}

int64_t scan_ws_bytes(int64_t n) {
    return (ceil_div(n > 0 ? n : 1, kScanChunk) + 1) * (int64_t)sizeof(int64_t);
}

int32_t exclusive_scan(const int32_t *in, const int32_t *idx, int64_t n, int32_t *out,
                       int64_t *total_dev, void *ws, int64_t ws_bytes, hipStream_t s,
                       const int32_t *const *idx_dev) {
    const bool gather = idx != nullptr || idx_dev != nullptr;
    MG_REQUIRE(ws && ws_bytes >= scan_ws_bytes(n), "exclusive scan: workspace %lld bytes, need %lld",
               (long long)ws_bytes, (long long)scan_ws_bytes(n));
    int64_t *partials = static_cast<int64_t *>(ws);
    const int64_t nparts = ceil_div(n > 0 ? n : 1, kScanChunk);
    TimedScope ts("exclusive_scan", s);
    // A zero-length input still runs one reduce block so the total is 0.
    scan_reduce_kernel<<<(unsigned)nparts, kScanThreads, 0, s>>>(in, idx, idx_dev, n, partials,
                                                                  gather ? out : nullptr);
    MG_LAUNCHED("scan_reduce_kernel");
    scan_partials_kernel<<<1, kScanThreads, 0, s>>>(partials, nparts, total_dev);
    MG_LAUNCHED("scan_partials_kernel");
    if (n > 0) {
        scan_down_kernel<<<(unsigned)nparts, kScanThreads, 0, s>>>(gather ? out : in, n,
                                                                    partials, out);
        MG_LAUNCHED("scan_down_kernel");
    }
    return MG_OK;
}

// ------------------------------------------------------ tile-major lists
// The (tile << 32 | depth) order is built without a global depth sort: the
// intersections are emitted Gaussian by Gaussian (ids ascending), grouped by
// tile id with a stable counting sort (ids stay ascending inside a tile),
// and each tile's list is then sorted stably by its depth bits alone, in LDS
// by one workgroup per tile. Inside a tile the order is thus (depth bits,
// Gaussian id): the same total order as one stable sort of the 64-bit keys.

struct BinStats {
    unsigned long long total;       // intersections
    unsigned long long scan_total;  // unused (kept zero)
};

// One per count workgroup, scanned by bin_offsets_kernel. (Same-address
// atomics from every wave would serialise at the memory side: the eight
// XCDs' L2s are not coherent with each other, so device-scope atomics are
// performed there.)
struct BinPart {
    unsigned long long total;
};

// Inclusive max over the wave of non-negative v, in lane order (DPP row
// shifts, then the row broadcasts).
__device__ __forceinline__ int wave_incl_max(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false));   // row_shr:1
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false));   // row_shr:2
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false));   // row_shr:4
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false));   // row_shr:8
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false));   // row_bcast:15
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false));   // row_bcast:31
    return v;
}

// The small rectangles' tile tests of one wave, one (Gaussian, tile)
// candidate per lane: a per-lane walk made every lane wait for the wave's
// largest rectangle. Lane l's rectangle has ar tiles (0 for none) and its
// candidates are [pre, pre + ar) of the wave's row; a candidate finds its
// rectangle as the last head mark at or before it (an inclusive max over the
// lanes), and its tile from its row-major index. Each tile's decision is
// tile_claim, the walk's own expressions, so the result is bit for bit the
// walk's. Returns this lane's claim mask (bit loc for tile loc).
__device__ __forceinline__ uint32_t wave_small_claims(const BinRec &r, int ar, bool test,
                                                      int tile, int W, int H, BinRec *w_rec,
                                                      int32_t *w_pre, uint32_t *w_msk,
                                                      uint8_t *w_own, int lane) {
    if (!test) return ar >= 32 ? 0xFFFFFFFFu : (1u << ar) - 1u;
    int incl = ar;
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o, 64);
        if (lane >= o) incl += t;
    }
    const int pre = incl - ar;
    const int total = __shfl(incl, 63, 64);
    if (total == 0) return 0u;   // wave-uniform
    w_rec[lane] = r;
    w_pre[lane] = pre;
    w_msk[lane] = 0u;
    for (int i = lane; i < (total + 3) / 4; i += 64) reinterpret_cast<uint32_t *>(w_own)[i] = 0u;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (ar > 0) w_own[pre] = (uint8_t)(lane + 1);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    int carry = 0;
    for (int c0 = 0; c0 < total; c0 += 64) {
        const int c = c0 + lane;
        const bool valid = c < total;
        const int h = valid ? (int)w_own[c] : 0;
        const int own = max(wave_incl_max(h), carry);   // owner lane + 1 (>= 1 when valid)
        carry = __shfl(own, 63, 64);
        const int ol = max(own - 1, 0);
        const BinRec q = w_rec[ol];
        const int loc = c - w_pre[ol];
        bool claim = false;
        if (valid) {
            const int x0 = (int)(q.xs & 0xffffu), y0 = (int)(q.ys & 0xffffu);
            const int w = (int)(q.xs >> 16) - x0 + 1;
            // loc < 32 and w <= 32: loc * ceil(2^16 / w) >> 16 is loc / w exactly.
            const int row = (int)(((uint32_t)loc * ((65535u + (uint32_t)w) / (uint32_t)w)) >> 16);
            const int col = loc - row * w;
            claim = tile_claim(q, true, x0 + col, y0 + row, tile, W, H);
        }
        // The candidates of one rectangle in this round are a run of lanes
        // starting at a head mark (or at lane 0); the run's first lane folds
        // the run's claims into the rectangle's mask.
        const uint64_t cm = ballot(claim);
        const uint64_t hm = ballot(valid && (h != 0 || lane == 0));
        if (valid && (h != 0 || lane == 0)) {
            const uint64_t above = lane == 63 ? 0ull : hm >> (lane + 1);
            const int len = above ? __builtin_ctzll(above) + 1 : min(64, total - c0) - lane;
            const uint32_t bits = (uint32_t)((cm >> lane) & ((len >= 64) ? ~0ull
                                                                          : ((1ull << len) - 1ull)));
            w_msk[ol] |= bits << loc;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    return w_msk[lane];
}

// Longest-processing-time-first orders, by one 1024-thread workgroup: a
// counting sort of the items over kBins bins of their estimated work,
// heaviest bin first (items of one bin in no fixed order). The bins are
// exact below 256, then 2^kOctBits an octave (to 2^31). Finer bins cost a
// longer scan; coarse ones crowd the items into a few bins, whose LDS
// atomics (one wave's lanes on one bin are served one after another) then
// dominate: the tile order past 4096 tiles took 12.1 us at config 5 with 32
// bins an octave and 7.5 with 128, the block order 10.8 with 32 and 12.2
// with 128.
constexpr int kOrdThreads = 1024;

template <int kOctBits>
__device__ __forceinline__ int fine_bin(int32_t w) {
    const uint32_t L = (uint32_t)max(w, 0);
    if (L < 256u) return (int)L;
    const int e = 31 - __builtin_clz(L);
    return 256 + (1 << kOctBits) * (e - 8) + (int)((L >> (e - kOctBits)) & ((1u << kOctBits) - 1u));
}
template <int kOctBits>
constexpr int fine_bins() { return 256 + (1 << kOctBits) * 24; }

// s_cnt's kBins counts become exclusive starts, the highest bin first:
// thread j owns bins kBins - 1 - kPer * j - k, k < kPer.
template <int kBins>
__device__ __forceinline__ void desc_bin_starts(uint32_t *s_cnt, uint32_t *s_wave) {
    constexpr int kPer = kBins / kOrdThreads;
    static_assert(kPer * kOrdThreads == kBins, "whole bins per thread");
    const int j = threadIdx.x, lane = j & 63, wave = j >> 6;
    uint32_t c[kPer], sum = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        c[k] = s_cnt[kBins - 1 - kPer * j - k];
        sum += c[k];
    }
    uint32_t incl = sum;
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t u = (uint32_t)__shfl_up((int)incl, o, 64);
        if (lane >= o) incl += u;
    }
    if (lane == 63) s_wave[wave] = incl;
    __syncthreads();
    uint32_t run = incl - sum;
    for (int v = 0; v < wave; ++v) run += s_wave[v];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        s_cnt[kBins - 1 - kPer * j - k] = run;
        run += c[k];
    }
    __syncthreads();
}

// The count and write passes' workgroup order, from a per-block work
// estimate (the tiles a block's rectangles cover, which the projection can
// emit): heaviest block first, so that the few blocks whose wave walks span
// thousands of tiles start at once instead of trailing the launch. Every
// block lands in order exactly once, whatever the estimates hold (a negative
// one counts as 0): they only reorder the blocks, and both passes index
// their outputs by block, not by workgroup.
constexpr int kBlkPer = 16, kBlkOctBits = 5, kBlkBins = 1024;
static_assert(fine_bins<kBlkOctBits>() <= kBlkBins, "block bins");

__global__ __launch_bounds__(kOrdThreads) void block_order_kernel(
    const int32_t *__restrict__ block_work, int64_t nparts, int32_t *__restrict__ order) {
    __shared__ uint32_t s_cnt[kBlkBins];
    __shared__ uint32_t s_wave[kOrdThreads / 64];
    const int j = threadIdx.x;
    constexpr int64_t kBatch = (int64_t)kOrdThreads * kBlkPer;
    for (int k = j; k < kBlkBins; k += kOrdThreads) s_cnt[k] = 0;   // nparts >= 1
    __syncthreads();
    // Each batch's loads are issued together, then binned.
    for (int64_t b0 = 0; b0 < nparts; b0 += kBatch) {
        int bin[kBlkPer];
#pragma unroll
        for (int r = 0; r < kBlkPer; ++r) {
            // Every load in range and its value always used (negative past
            // nparts), so no branch separates the batch's loads.
            const int64_t i = b0 + j + (int64_t)kOrdThreads * r;
            bin[r] = fine_bin<kBlkOctBits>(block_work[min(i, nparts - 1)]) -
                     (i < nparts ? 0 : 2 * kBlkBins);
        }
#pragma unroll
        for (int r = 0; r < kBlkPer; ++r)
            if (bin[r] >= 0) atomicAdd(&s_cnt[bin[r]], 1u);
    }
    __syncthreads();
    desc_bin_starts<kBlkBins>(s_cnt, s_wave);
    for (int64_t b0 = 0; b0 < nparts; b0 += kBatch) {
        int bin[kBlkPer];
#pragma unroll
        for (int r = 0; r < kBlkPer; ++r) {
            const int64_t i = b0 + j + (int64_t)kOrdThreads * r;
            bin[r] = fine_bin<kBlkOctBits>(block_work[min(i, nparts - 1)]) -
                     (i < nparts ? 0 : 2 * kBlkBins);
        }
#pragma unroll
        for (int r = 0; r < kBlkPer; ++r) {
            if (bin[r] >= 0)
                order[atomicAdd(&s_cnt[bin[r]], 1u)] =
                    (int32_t)(b0 + j + (int64_t)kOrdThreads * r);
        }
    }
}

// Count pass in Gaussian order (coalesced reads): the tile count and the
// walk record (with a small rectangle's claim mask, or a large one's kept
// step words); per workgroup the intersection total. At most 80 VGPRs, so
// six waves fit per SIMD.
__global__ __launch_bounds__(kBinThreads) __attribute__((amdgpu_waves_per_eu(6))) void
bin_count_rec_kernel(const BinArgs A, int32_t *counts, BinRec *recs, uint32_t *masks,
                     uint64_t *words, BinPart *parts, const int32_t *order) {
    __shared__ BinPart s_p[kBinThreads / 64];
    __shared__ BinRec s_rec[kBinThreads];
    __shared__ int32_t s_big[kBinThreads], s_cnt[kBinThreads];
    __shared__ int32_t s_nbig, s_used;
    __shared__ int32_t s_pre[kBinThreads];
    __shared__ uint32_t s_msk[kBinThreads];
    // Per wave: the small claims' owner marks, then the strip walk's row
    // boundaries.
    __shared__ float4 s_rows[kBinThreads / 64][kRowSlots];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // The block of 256 Gaussians this workgroup takes (see block_order_kernel).
    const int64_t blk = order ? order[blockIdx.x] : blockIdx.x;
    const int64_t g = blk * kBinThreads + tid;
    const bool test = A.conic != nullptr;
    if (tid == 0) {
        s_nbig = 0;
        s_used = 0;
    }
    __syncthreads();
    int n = 0;
    bool big = false;
    uint32_t mask = 0;
    BinRec r{};
    int ar = 0;
    if (g < A.N && make_rec(A, g, r)) {
        recs[g] = r;
        ar = rec_area(r);
        if (ar > kWaveWalkArea) {
            big = true;
            ar = 0;
        }
    }
    // The claimed tiles of a small rectangle, bit loc for its row-major tile
    // loc: the write pass emits from them without testing again.
    mask = wave_small_claims(r, ar, test, A.tile, A.W, A.H, s_rec + wave * 64,
                             s_pre + wave * 64, s_msk + wave * 64,
                             reinterpret_cast<uint8_t *>(s_rows[wave]), lane);
    n = __popc(mask);
    // s_rec's wave slice now holds the big rectangles' records (a lane's own
    // record, written by wave_small_claims or here).
    if (big) s_rec[tid] = r;
    // Large rectangles: compacted in LDS, one wave each.
    const uint64_t m = ballot(big);
    int at = 0;
    if (lane == 0 && m) at = atomicAdd(&s_nbig, __popcll(m));
    at = __shfl(at, 0, 64);
    if (big) s_big[at + rank_in(m)] = tid;
    __syncthreads();
    // Each walk's step ballots go to the workgroup's words while they fit
    // (kept_mask records where; s_pre holds it, the small claims being done
    // with their slices).
    for (int e = wave; e < s_nbig; e += kBinThreads / 64) {
        const int j = s_big[e];
        const BinRec r = s_rec[j];
        const StripPlan P = strip_plan(r, lane);
        const int nst = P.ns * P.nr;
        int first = 0;
        if (lane == 0) first = atomicAdd(&s_used, min(nst, kBlockWords + 1));
        first = __builtin_amdgcn_readfirstlane(first);
        const bool keep = first + nst <= kBlockWords;
        uint64_t *const wp = words + blk * kBlockWords + first;
        int cnt = 0, t = 0;
        strip_walk(r, P, test, A.tile, A.W, A.H, s_rows[wave], lane,
                   [&](bool claim, int, int) {
                       cnt += claim ? 1 : 0;
                       if (keep) {
                           const uint64_t cm = ballot(claim);
                           if (lane == 0) wp[t] = cm;
                       }
                       ++t;
                   });
        for (int o = 32; o >= 1; o >>= 1) cnt += __shfl_xor(cnt, o, 64);
        if (lane == 0) {
            s_cnt[j] = cnt;
            s_pre[j] = (int32_t)(keep ? kept_mask(first, nst) : 0u);
        }
    }
    __syncthreads();
    if (g < A.N) {
        if (big) n = s_cnt[tid];
        counts[g] = n;
        masks[g] = big ? (uint32_t)s_pre[tid] : mask;
    }
    unsigned long long tot = (unsigned long long)n;
    for (int o = 32; o >= 1; o >>= 1) tot += __shfl_xor(tot, o, 64);
    if ((threadIdx.x & 63) == 0) s_p[threadIdx.x >> 6] = BinPart{tot};
    __syncthreads();
    if (threadIdx.x == 0) {
        BinPart b = s_p[0];
        for (int w = 1; w < kBinThreads / 64; ++w) b.total += s_p[w].total;
        parts[blk] = b;
    }
}

// One workgroup scans the count pass's per-workgroup totals: part_off[i] is
// the first pair of count workgroup i's Gaussians, st->total the intersection
// total.
// With status (capacity-bounded lists) it also writes status[0] = the total
// and status[1] = 1 if the total exceeds capacity, else 0; with status_host
// (host memory the device can write) the same two words and then tag in
// status_host[2], ordered by a system-scope release, so the host can wait by
// polling for the tag instead of an event.
__global__ __launch_bounds__(kScanThreads) void bin_offsets_kernel(const BinPart *parts,
                                                                   int64_t nparts,
                                                                   int64_t *part_off,
                                                                   BinStats *st,
                                                                   int64_t capacity,
                                                                   int64_t *status,
                                                                   int64_t *status_host,
                                                                   int64_t tag) {
    // Blocked: thread t owns 16 consecutive totals of each 4096-entry step,
    // all requested at once; one block scan per step.
    constexpr int kPer = 16;
    __shared__ int64_t s_wave[kScanThreads / 64];
    int64_t carry = 0;
    for (int64_t c0 = 0; c0 < nparts; c0 += kScanThreads * kPer) {
        const int64_t i0 = c0 + (int64_t)threadIdx.x * kPer;
        int64_t v[kPer], sum = 0;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            v[j] = i0 + j < nparts ? (int64_t)parts[i0 + j].total : 0;
            sum += v[j];
        }
        int64_t tot;
        int64_t run = carry + block_excl_scan(sum, s_wave, &tot);
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            if (i0 + j < nparts) part_off[i0 + j] = run;
            run += v[j];
        }
        carry += tot;
    }
    if (threadIdx.x == 0) {
        st->total = (unsigned long long)carry;
        st->scan_total = 0;
        if (status) {
            status[0] = carry;
            status[1] = carry > capacity ? 1 : 0;
        }
        if (status_host) {
            __hip_atomic_store(status_host, carry, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(status_host + 1, (int64_t)(carry > capacity ? 1 : 0),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(status_host + 2, tag, __ATOMIC_RELEASE,
                               __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

// Pairs the capacity-bounded lists hold: the total, or none when it
// overflowed the capacity.
__device__ __forceinline__ int64_t lists_kept(const int64_t *status) {
    return status[1] != 0 ? 0 : status[0];
}

// Pairs staged in LDS per workgroup before the coalesced store.
constexpr int kBinStage = 2048;

// Exclusive sum and exclusive max of one value each per thread over a
// kBinThreads workgroup (max of non-negative values; 0 before thread 0).
// One barrier; sc holds 2 x (kBinThreads / 64) ints of its own.
__device__ __forceinline__ void block_excl_sum_max(int vs, int vm, int &ex_s, int &ex_m,
                                                   int *sc) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int is = vs, im = vm;
    for (int o = 1; o < 64; o <<= 1) {
        const int ts = __shfl_up(is, o, 64), tm = __shfl_up(im, o, 64);
        if (lane >= o) {
            is += ts;
            im = max(im, tm);
        }
    }
    if (lane == 63) {
        sc[wave] = is;
        sc[kBinThreads / 64 + wave] = im;
    }
    __syncthreads();
    int bs = 0, bm = 0;
    for (int w = 0; w < wave; ++w) {
        bs += sc[w];
        bm = max(bm, sc[kBinThreads / 64 + w]);
    }
    ex_s = bs + is - vs;
    // The inclusive max of the lanes before this one: shift by one lane.
    const int prev = __shfl_up(im, 1, 64);
    ex_m = max(bm, lane > 0 ? prev : 0);
}

// Thread k emits the pairs of Gaussian k (tile id key, Gaussian id) at its
// scanned offset; the workgroup's 256 Gaussians own one contiguous output
// range.
//   * Small rectangles (walked by their own thread) go through LDS: their
//     runs are numbered by a workgroup prefix scan of their counts (at most
//     256 x 32 pairs) and staged in windows of kBinStage slots, each slot
//     with its position in the range, then stored by consecutive lanes, so
//     adjacent runs land as coalesced stores.
//   * Large rectangles (more than kWaveWalkArea tiles) are replayed from the
//     step words the count pass kept. Those words are one run per rectangle
//     from the start of the workgroup's kBlockWords. The workgroup loads
//     them, finds each word's rectangle (the last run start at or before it,
//     an exclusive max scan), its step's first tile and the claims before it
//     in its rectangle (an exclusive sum scan of the words' bit counts), and
//     the four waves take the words in turn: a rectangle's steps are spread
//     over the waves however the rectangles' sizes fall. A step's claims
//     take consecutive positions by lane rank, stored directly, consecutive
//     lanes on consecutive addresses. Rectangles the count pass kept no words
//     for are walked again, a wave each (strip_walk, up to 64 tiles a step).
// With pairs (and depth) the value of a pair is {Gaussian id, its depth's
// float bits} in one 8-byte store instead of the id alone in ids.
// The workgroup's output range starts at part_off[blockIdx.x] (the count
// workgroup of the same 256 Gaussians, scanned); each Gaussian's offset in it
// is an exclusive scan of the counts, formed here.
__global__ __launch_bounds__(kBinThreads) void bin_write_rec_kernel(
    const BinRec *recs, const int32_t *counts, const uint32_t *masks, const uint64_t *words,
    const int64_t *part_off, int64_t N, int tile, int W, int H, int tiles_x, int test,
    uint32_t *tkeys, int32_t *ids, const float *depth, uint2 *pairs, const int64_t *status,
    const int32_t *order) {
    // Capacity-bounded lists that overflowed emit nothing.
    if (status && status[1] != 0) return;
    // The staging windows' arrays hold, until the small runs are staged:
    //   s_k: per kept word its step's first tile (s_tb), per rectangle the
    //        bit count before its first word (s_pf) and its walk plan
    //        (s_pl, s_pnr); then each wave's strip-walk row slice;
    //   s_i: the kept words;
    //   s_off: each Gaussian's offset in the range and count (s_at, s_cap),
    //        per kept word its rectangle + 1 (s_hown, 16 bits; run starts
    //        first) and the bit count before it (s_pw).
    __shared__ __align__(16) uint32_t s_k[kBinStage];
    __shared__ __align__(16) int32_t s_i[kBinStage];
    __shared__ __align__(16) int32_t s_off[kBinStage];
    static_assert(kBinStage * 4 >= (kBinThreads / 64) * kRowSlots * 16, "row slices fit s_k");
    static_assert(kBinStage == 2 * kBlockWords && kBinThreads * 4 == kBlockWords,
                  "the replay arrays fit the staging arrays");
    uint64_t *const s_words = reinterpret_cast<uint64_t *>(s_i);
    uint32_t *const s_tb = s_k;
    int32_t *const s_pf = reinterpret_cast<int32_t *>(s_k) + kBlockWords;
    uint32_t *const s_pl = s_k + kBlockWords + kBinThreads;
    int32_t *const s_pnr = reinterpret_cast<int32_t *>(s_k) + kBlockWords + 2 * kBinThreads;
    int32_t *const s_at = s_off, *const s_cap = s_off + kBinThreads;
    uint16_t *const s_hown = reinterpret_cast<uint16_t *>(s_off + 2 * kBinThreads);
    int32_t *const s_pw = s_off + kBlockWords;
    __shared__ BinRec s_rec[kBinThreads];
    __shared__ int32_t s_big[kBinThreads], s_g[kBinThreads];
    __shared__ uint32_t s_wm[kBinThreads];   // a large rectangle's kept_mask (or 0)
    __shared__ int32_t s_nbig, s_nfall, s_wext, s_wsum[kBinThreads / 64],
        s_csum[kBinThreads / 64], s_sc[2 * (kBinThreads / 64)];
    __shared__ uint32_t s_dk[kBinThreads];   // depth bits of the workgroup's Gaussians
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t blk = order ? order[blockIdx.x] : blockIdx.x;   // as in bin_count
    const int64_t k0 = blk * kBinThreads;
    const int64_t k = k0 + tid;
    const int64_t base = part_off[blk];
    if (pairs) s_dk[tid] = k < N ? __float_as_uint(depth[k]) : 0u;
    if (tid == 0) {
        s_nbig = 0;
        s_nfall = 0;
        s_wext = 0;
    }
    reinterpret_cast<uint32_t *>(s_hown)[2 * tid] = 0u;
    reinterpret_cast<uint32_t *>(s_hown)[2 * tid + 1] = 0u;
    __syncthreads();
    bool big = false;
    int small_cap = 0;        // pairs this thread stages (0 unless a small rectangle)
    int32_t g = 0;
    BinRec r{};
    uint32_t mask = 0;
    const int cap = k < N ? counts[k] : 0;
    {
        if (cap > 0) {
            g = (int32_t)k;
            r = recs[g];
            mask = masks[g];
            if (rec_area(r) > kWaveWalkArea) {
                big = true;
                s_rec[tid] = r;
                s_g[tid] = g;
                s_wm[tid] = mask;
                if (mask != 0) {
                    // Its run of words, marked at its start.
                    atomicMax(&s_wext, kept_first(mask) + kept_steps(mask));
                    s_hown[kept_first(mask)] = (uint16_t)(tid + 1);
                } else {
                    atomicAdd(&s_nfall, 1);
                }
            } else {
                small_cap = cap;
            }
        }
    }
    // Big rectangles, compacted; small runs, numbered (exclusive scan).
    const uint64_t m = ballot(big);
    int slot = 0;
    if (lane == 0 && m) slot = atomicAdd(&s_nbig, __popcll(m));
    slot = __shfl(slot, 0, 64);
    if (big) s_big[slot + rank_in(m)] = tid;
    int incl = small_cap, cincl = cap;
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o, 64), u = __shfl_up(cincl, o, 64);
        if (lane >= o) {
            incl += t;
            cincl += u;
        }
    }
    if (lane == 63) {
        s_wsum[wave] = incl;
        s_csum[wave] = cincl;
    }
    __syncthreads();
    int first = incl - small_cap, n_small = 0, off0 = cincl - cap;
    for (int w = 0; w < kBinThreads / 64; ++w) {
        if (w < wave) {
            first += s_wsum[w];
            off0 += s_csum[w];
        }
        n_small += s_wsum[w];
    }
    s_at[tid] = off0;
    s_cap[tid] = cap;
    const int wext = s_wext, nbig = s_nbig;
    if (wext > 0) {   // workgroup-uniform
        // The kept rectangles' walk plans, a wave each.
        for (int e = wave; e < nbig; e += kBinThreads / 64) {
            const int j = s_big[e];
            if (s_wm[j] == 0) continue;
            const StripPlan P = strip_plan(s_rec[j], lane);
            if (lane == 0) {
                // R and s up to 64, ceil(2^16 / s) up to 2^16.
                s_pl[j] = (uint32_t)P.R | (uint32_t)P.s << 7 |
                          ((65535u + (uint32_t)P.s) / (uint32_t)P.s) << 14;
                s_pnr[j] = P.nr;
            }
        }
        // Words 4 tid .. 4 tid + 3, all requested at once.
        const int i0 = 4 * tid;
        uint64_t v[4];
        int hp[4], pc[4], runmax = 0, psum = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = i0 + q;
            v[q] = i < wext ? words[blk * kBlockWords + i] : 0ull;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = i0 + q;
            // A run start marks its own position + 1; the max of those at
            // or before word i is its run's start + 1.
            runmax = max(runmax, (i < wext && s_hown[i] != 0) ? i + 1 : 0);
            hp[q] = runmax;
            pc[q] = psum;
            psum += __popcll(v[q]);
        }
        int ex_s, ex_m;
        block_excl_sum_max(psum, runmax, ex_s, ex_m, s_sc);   // orders the plans too
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = i0 + q;
            if (i >= wext) break;
            const int st = max(hp[q], ex_m) - 1;      // the run's first word
            const int j = (int)s_hown[st] - 1;
            const int t = i - st, nr = s_pnr[j];
            const int kk = t / nr, u = t - kk * nr;
            const uint32_t pl = s_pl[j];
            const BinRec rj = s_rec[j];
            s_words[i] = v[q];
            s_tb[i] = ((rj.xs & 0xffffu) + (uint32_t)kk * ((pl >> 7) & 127u)) |
                      (((rj.ys & 0xffffu) + (uint32_t)u * (pl & 127u)) << 16);
            s_pw[i] = ex_s + pc[q];
            if (st == i) s_pf[j] = ex_s + pc[q];
            // Every word's entry now names its rectangle (a run start's is
            // unchanged, and only those are read by other threads here).
            s_hown[i] = (uint16_t)(j + 1);
        }
    }
    __syncthreads();
    // A step's claims (cm, the walk's ballot): the lane's tile (tx, ty) at
    // position pos0 + its rank among them, within rectangle j's run.
    auto emit = [&](uint64_t cm, int j, int tx, int ty, int pos0) {
        const int pos = pos0 + rank_in(cm);
        if (((cm >> lane) & 1ull) && pos < s_cap[j]) {
            const int64_t at = base + s_at[j] + pos;
            tkeys[at] = (uint32_t)(ty * tiles_x + tx);
            if (pairs)
                pairs[at] = make_uint2((uint32_t)s_g[j], s_dk[j]);
            else
                ids[at] = s_g[j];
        }
    };
    // The kept words, the four waves in turn.
    for (int i = wave; i < wext; i += kBinThreads / 64) {
        const uint64_t cm = s_words[i];
        if (cm == 0) continue;
        const int j = (int)s_hown[i] - 1;
        const uint32_t tb = s_tb[i], pl = s_pl[j];
        // lane = rg * s + cl, rg = floor(lane / s) as lane * ceil(2^16 / s) >> 16
        // (exact for lane < 64 <= 2^16 / s).
        const int sw = (int)((pl >> 7) & 127u);
        const int rg = (int)(((uint32_t)lane * (pl >> 14)) >> 16), cl = lane - rg * sw;
        emit(cm, j, (int)(tb & 0xffffu) + cl, (int)(tb >> 16) + rg, s_pw[i] - s_pf[j]);
    }
    // Rectangles without kept words: walked again, a wave each, in the row
    // slices (s_k, once the replay is done with it).
    if (s_nfall > 0) {   // workgroup-uniform
        __syncthreads();
        for (int e = wave; e < nbig; e += kBinThreads / 64) {
            const int j = s_big[e];
            if (s_wm[j] != 0) continue;
            const BinRec rb = s_rec[j];
            const StripPlan P = strip_plan(rb, lane);
            int emitted = 0;
            strip_walk(rb, P, test != 0, tile, W, H,
                       reinterpret_cast<float4 *>(s_k) + wave * kRowSlots, lane,
                       [&](bool claim, int tx, int ty) {
                           const uint64_t cm = ballot(claim);
                           emit(cm, j, tx, ty, emitted);
                           emitted += __popcll(cm);
                       });
        }
    }
    __syncthreads();   // s_at / s_cap read; s_off becomes the staging window
    // Small rectangles: LDS windows over the numbered runs.
    for (int w0 = 0; w0 < n_small; w0 += kBinStage) {
        const int w1 = min(w0 + kBinStage, n_small);
        if (small_cap > 0 && first < w1 && first + small_cap > w0) {
            // The count pass's claimed tiles, in the walk's row-major order:
            // row = floor(loc / w) as (loc * ceil(2^16 / w)) >> 16, exact for
            // loc < 32 <= 2^16 / w.
            const int x0 = (int)(r.xs & 0xffffu), y0 = (int)(r.ys & 0xffffu);
            const int w = (int)(r.xs >> 16) - x0 + 1;
            const uint32_t inv = (65536u + (uint32_t)w - 1u) / (uint32_t)w;
            int n = 0;
            for (uint32_t mm = mask; mm != 0 && n < small_cap; mm &= mm - 1u, ++n) {
                const int sl = first + n;
                if (sl < w0 || sl >= w1) continue;
                const int loc = __builtin_ctz(mm);
                const int row = (int)(((uint32_t)loc * inv) >> 16);
                const int col = loc - row * w;
                s_k[sl - w0] = (uint32_t)((y0 + row) * tiles_x + x0 + col);
                s_i[sl - w0] = g;
                s_off[sl - w0] = off0 + n;
            }
        }
        __syncthreads();
        for (int i = tid; i < w1 - w0; i += kBinThreads) {
            const int64_t pos = base + s_off[i];
            tkeys[pos] = s_k[i];
            if (pairs)
                pairs[pos] = make_uint2((uint32_t)s_i[i], s_dk[s_i[i] - k0]);
            else
                ids[pos] = s_i[i];
        }
        __syncthreads();
    }
}

// Offsets of sorted tile keys: offsets[t] = the first i with tiles[i] >= t
// (n for t past the last key). A thread takes kRangePer consecutive keys,
// read as two 16-byte loads, and the key before them; at a change of key
// from a to b at position i it writes offsets[a + 1 .. b] = i. With status
// (capacity-bounded lists, n the capacity) n is the pairs kept.
constexpr int kRangePer = 8;
__global__ __launch_bounds__(256) void tile_ranges_u32_kernel(const uint32_t *tiles, int64_t n,
                                                              int32_t n_tiles, int32_t *offsets,
                                                              const int64_t *status) {
    if (status) n = min(lists_kept(status), n);
    const int64_t b = ((int64_t)blockIdx.x * 256 + threadIdx.x) * kRangePer;
    if (b > n) return;
    int64_t key[kRangePer + 1];   // key[j] is tiles[b + j - 1]; -1 before the first
    key[0] = b == 0 ? -1 : (int64_t)tiles[b - 1];
    if (b + kRangePer <= n && ((reinterpret_cast<uintptr_t>(tiles + b) & 15) == 0)) {
        const uint4 q0 = *reinterpret_cast<const uint4 *>(tiles + b);
        const uint4 q1 = *reinterpret_cast<const uint4 *>(tiles + b + 4);
        key[1] = q0.x; key[2] = q0.y; key[3] = q0.z; key[4] = q0.w;
        key[5] = q1.x; key[6] = q1.y; key[7] = q1.z; key[8] = q1.w;
    } else {
#pragma unroll
        for (int j = 0; j < kRangePer; ++j)
            key[j + 1] = b + j < n ? (int64_t)tiles[b + j] : (int64_t)n_tiles;
    }
#pragma unroll
    for (int j = 0; j < kRangePer; ++j) {
        const int64_t i = b + j;
        if (i > n) break;
        // Position n closes every tile after the last key.
        const int64_t cur = i == n ? (int64_t)n_tiles : key[j + 1];
        for (int64_t t = key[j] + 1; t <= cur && t <= n_tiles; ++t) offsets[t] = (int32_t)i;
    }
}

inline int tile_bits(int n_tiles) {
    int b = 1;
    while ((1LL << b) < n_tiles) ++b;
    return b;
}

// ------------------------------------------------------------ tile sort
// Stable counting sort of the (tile, id) pairs by tile, in one pass over the
// pairs, for up to kCsBuckets tiles (more take the radix sort). The pairs are
// cut into chunks of 256 * per consecutive pairs, one workgroup each, dealt
// to the XCDs in contiguous runs:
//   1. count_hist    - chunk c's count of each tile -> hist[c][t];
//   2. count_colscan - per tile, exclusive scan of its counts over the chunks
//                      (in place) and the tile's total;
//   3. count_scatter - each workgroup holds its chunk in registers, one
//                      contiguous part of 64 * per pairs per wave, counts
//                      each part into a wave-private LDS histogram, forms the
//                      tile starts (exclusive scan of the totals) and from
//                      them each wave's first slot per tile, then walks its
//                      part in input order, ranking pairs of one tile by
//                      ballots over the tile bits, and stores each id at its
//                      slot.
// A pair's slot is start(t) + the pairs of tile t in earlier chunks, in
// earlier waves' parts and earlier in its own part: the input order within
// each tile, i.e. the stable order. The tile starts double as the list
// offsets. Pairs with a tile >= n_tiles are dropped.
constexpr int kCsBuckets = 4096;
constexpr int kCsThreads = 256, kCsWaves = kCsThreads / 64;
constexpr int64_t kCsMaxChunks = 512;   // about two workgroups per CU
// Capacity-bounded lists plan for the capacity, which runs above the pairs
// actually sorted (by the caller's headroom, or more). With twice the limit
// the kept pairs get chunks no longer than the exact plan's as long as the
// capacity is at most twice their count; with the same limit a headroom that
// crossed it would lengthen the chunks a step and leave part of the GPU idle
// (measured: 94 -> 113 us at config 4).
constexpr int64_t kCsMaxChunksCapped = 2 * kCsMaxChunks;
constexpr int kColWaves = 16;           // waves of the column scan's workgroups

struct CsPlan {
    int per;        // pairs per lane (a chunk is 256 * per pairs)
    int64_t nchunks;
};

// The smallest chunk that needs no more than max_chunks workgroups.
inline CsPlan cs_plan(int64_t n, int64_t max_chunks = kCsMaxChunks) {
    static const int kPers[] = {8, 16, 24, 32, 48, 64};
    for (int p : kPers) {
        const int64_t nc = ceil_div(n, (int64_t)kCsThreads * p);
        if (nc <= max_chunks || p == 64) return {p, nc};
    }
    return {64, ceil_div(n, (int64_t)kCsThreads * 64)};
}

// Per-chunk counts, the tiles' totals, and the depth sort's tile order.
inline int64_t tile_sort_ws_bytes(int64_t n, int nb, int64_t max_chunks = kCsMaxChunks) {
    return align256(4 * (int64_t)nb * cs_plan(n, max_chunks).nchunks) +
           2 * align256(4 * (int64_t)nb);
}

// V is the value moved with each tile key: an int32 id, or a uint2
// {id, depth bits}.
template <typename V>
struct CsPass {
    const uint32_t *tiles;
    const V *ids;
    int64_t n;
    int nb, nbits;                  // tiles; bits that tell them apart
    V *out;
    int32_t *offsets;               // tile starts, nb + 1
    uint32_t *hist, *tot;           // hist[nchunks][nb], tot[nb]
    // Capacity-bounded lists: n is the capacity and the pairs to sort are
    // lists_kept(status), read on the device; NULL: n pairs.
    const int64_t *status;
    int64_t chunk;                  // pairs per chunk
    // Optional: the tiles longest list first, for the per-tile depth sort.
    int32_t *order;
};

template <typename V>
__device__ __forceinline__ int64_t cs_count(const CsPass<V> &P) {
    return P.status ? min(lists_kept(P.status), P.n) : P.n;
}

// Chunks holding pairs: all grid chunks, or for capacity-bounded lists the
// chunks of the kept pairs (at least one, chunk 0 writing the offsets).
// Workgroups past them do nothing; the others are dealt to the XCDs in
// contiguous runs over these chunks alone, so that every XCD gets a share of
// the work.
template <typename V>
__device__ __forceinline__ int64_t cs_active(const CsPass<V> &P, int64_t n, int64_t grid) {
    return P.status ? max((int64_t)1, (n + P.chunk - 1) / P.chunk) : grid;
}

// A chunk's tiles as kPer / 4 16-byte loads per thread, all in flight at once
// (chunk starts are multiples of 2048 pairs, so 16-byte aligned); ~0 past n.
template <int kPer>
__device__ __forceinline__ void load_chunk_tiles(const uint32_t *tiles, int64_t n, int64_t b,
                                                 uint32_t (&t)[kPer]) {
#pragma unroll
    for (int j = 0; j < kPer / 4; ++j) {
        const int64_t i = b + 4 * ((int64_t)threadIdx.x + (int64_t)kCsThreads * j);
        if (i + 4 <= n) {
            const uint4 q = *reinterpret_cast<const uint4 *>(tiles + i);
            t[4 * j] = q.x;
            t[4 * j + 1] = q.y;
            t[4 * j + 2] = q.z;
            t[4 * j + 3] = q.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) t[4 * j + e] = i + e < n ? tiles[i + e] : 0xFFFFFFFFu;
        }
    }
}

template <int kPer, typename V>
__global__ __launch_bounds__(kCsThreads) void count_hist_kernel(const CsPass<V> P) {
    __shared__ uint32_t s_h[kCsBuckets];
    const int64_t n = cs_count(P);
    const int64_t nact = cs_active(P, n, (int64_t)gridDim.x);
    if ((int64_t)blockIdx.x >= nact) return;
    const int64_t c = xcd_contiguous(blockIdx.x, nact);
    uint32_t t[kPer];
    load_chunk_tiles<kPer>(P.tiles, n, c * kCsThreads * kPer, t);
    for (int i = threadIdx.x; i < P.nb; i += kCsThreads) s_h[i] = 0;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kPer; ++r)
        if (t[r] < (uint32_t)P.nb) atomicAdd(&s_h[t[r]], 1u);
    __syncthreads();
    uint32_t *row = P.hist + c * P.nb;
    for (int i = threadIdx.x; i < P.nb; i += kCsThreads) row[i] = s_h[i];
}

// One workgroup per 64 tiles, lane = tile; each of its 16 waves scans a
// sixteenth of the chunks (coalesced rows), the waves' sums are joined
// through LDS, and each wave writes its running exclusive prefixes. Up to
// kColRows rows per wave (1024 chunks) all of a wave's rows are requested at
// once and parked in LDS as 16-bit counts (a chunk holds at most 16384
// pairs) for the prefix pass; walking the rows in batches instead makes a
// chain of dependent HBM round trips (12 us at config 4).
constexpr int kColRows = 64;
static_assert((int64_t)kCsThreads * 64 <= 65535, "per-chunk tile counts must fit 16 bits");

template <typename V>
__global__ __launch_bounds__(64 * kColWaves) void count_colscan_kernel(const CsPass<V> P,
                                                                       int64_t nchunks) {
    __shared__ uint32_t s_sum[kColWaves][64];
    __shared__ uint16_t s_val[kColWaves][kColRows][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int bkt = blockIdx.x * 64 + lane;
    const bool in = bkt < P.nb;
    if (P.status) nchunks = cs_active(P, cs_count(P), nchunks);
    const int64_t q = (nchunks + kColWaves - 1) / kColWaves;
    const int64_t c0 = wave * q, c1 = min(nchunks, c0 + q);
    if (q <= kColRows) {   // workgroup-uniform
        const uint32_t *row = P.hist + c0 * P.nb + bkt;
        uint32_t vals[kColRows];
#pragma unroll
        for (int i = 0; i < kColRows; ++i)
            vals[i] = in && c0 + i < c1 ? row[(int64_t)i * P.nb] : 0u;
        uint32_t sum = 0;
#pragma unroll
        for (int i = 0; i < kColRows; ++i) {
            s_val[wave][i][lane] = (uint16_t)vals[i];
            sum += vals[i];
        }
        s_sum[wave][lane] = sum;
        __syncthreads();
        uint32_t run = 0, all = 0;
#pragma unroll
        for (int w = 0; w < kColWaves; ++w) {
            const uint32_t v = s_sum[w][lane];
            run += w < wave ? v : 0u;
            all += v;
        }
        if (in) {
            for (int64_t c = c0; c < c1; ++c) {
                P.hist[c * P.nb + bkt] = run;
                run += s_val[wave][c - c0][lane];
            }
            if (wave == 0) P.tot[bkt] = all;
        }
        return;
    }
    uint32_t sum = 0;
#pragma unroll 8
    for (int64_t c = c0; c < c1; ++c) sum += in ? P.hist[c * P.nb + bkt] : 0u;
    s_sum[wave][lane] = sum;
    __syncthreads();
    uint32_t run = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kColWaves; ++w) {
        const uint32_t v = s_sum[w][lane];
        run += w < wave ? v : 0u;
        all += v;
    }
    if (in) {
#pragma unroll 8
        for (int64_t c = c0; c < c1; ++c) {
            uint32_t *h = P.hist + c * P.nb + bkt;
            const uint32_t v = *h;
            *h = run;
            run += v;
        }
        if (wave == 0) P.tot[bkt] = all;
    }
}

// Bin of a list length for the depth sort's order: exact below 64, then 16
// bins an octave (the four bits below the leading one), the last from 2^18
// entries up. A higher bin is a longer list.
__device__ __forceinline__ int len_bin(uint32_t L) {
    if (L < 64u) return (int)L;
    const int e = 31 - __builtin_clz(L);
    return min(255, 64 + 16 * (e - 6) + (int)((L >> (e - 4)) & 15u));
}

// The per-tile depth sort runs one workgroup per tile, each about as long as
// its list, in more rounds of workgroups than the GPU holds; taken longest
// list first, its last round holds the shortest lists (longest-processing-
// time first). The tile scatter launches one workgroup more than it has
// chunks, which writes that order from the tiles' totals (complete since the
// column scan) while the others scatter.
template <typename V>
__device__ __forceinline__ void cs_depth_order(const CsPass<V> &P, uint32_t *s_wh,
                                               uint32_t *s_part) {
    constexpr int kTPer = kCsBuckets / kCsThreads;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nb = P.nb, t0 = tid * kTPer;

    // A counting sort of the tiles over 256 list-length bins (tiles of one
    // bin in no fixed order), in the LDS of the scatter's wave counters.
    if (nb < kCsThreads / kCsWaves) {
        // Fewer words of wave counters than bins: the tiles in order.
        for (int i = tid; i < nb; i += kCsThreads) P.order[i] = i;
        return;
    }
    uint32_t *hb = s_wh;   // kCsThreads bins
    hb[tid] = 0;
    __syncthreads();
    int bin[kTPer];
    uint32_t slot[kTPer];
#pragma unroll
    for (int j = 0; j < kTPer; ++j) {
        const int tt = t0 + j;
        bin[j] = tt < nb ? len_bin(P.tot[tt]) : -1;
    }
#pragma unroll
    for (int j = 0; j < kTPer; ++j)
        if (bin[j] >= 0) slot[j] = atomicAdd(&hb[bin[j]], 1u);
    __syncthreads();
    // Exclusive starts, longest bin first: thread i scans bin 255 - i.
    const uint32_t cnt = hb[kCsThreads - 1 - tid];
    uint32_t incl = cnt;
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t u = __shfl_up(incl, o, 64);
        if (lane >= o) incl += u;
    }
    if (lane == 63) s_part[wave] = incl;
    __syncthreads();
    uint32_t before = incl - cnt;
    for (int w = 0; w < wave; ++w) before += s_part[w];
    hb[kCsThreads - 1 - tid] = before;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kTPer; ++j)
        if (bin[j] >= 0) P.order[hb[bin[j]] + slot[j]] = t0 + j;
}

template <int kPer, typename V>
__global__ __launch_bounds__(kCsThreads) void count_scatter_kernel(const CsPass<V> P) {
    constexpr int64_t kChunk = (int64_t)kCsThreads * kPer, kPart = 64 * kPer;
    constexpr int kTPer = kCsBuckets / kCsThreads;   // tiles owned per thread
    // Per wave and tile: the count, then the next slot; sized by the launch
    // to the tile count (kCsWaves * nb words), so that at config 4's 2500
    // tiles four workgroups share a CU and every chunk's workgroup is
    // resident at once (two with room for 4096 tiles).
    extern __shared__ uint32_t s_wh[];
    __shared__ uint32_t s_part[kCsWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (P.order && blockIdx.x == gridDim.x - 1) {   // the depth sort's order
        cs_depth_order(P, s_wh, s_part);
        return;
    }
    const int64_t n = cs_count(P);
    const int64_t nact = cs_active(P, n, (int64_t)gridDim.x - (P.order ? 1 : 0));
    if ((int64_t)blockIdx.x >= nact) return;
    const int64_t c = xcd_contiguous(blockIdx.x, nact);
    const int64_t pb = c * kChunk + wave * kPart;
    const int nb = P.nb;
    // The wave's part: pair pb + 64 r + lane is (tile t[r], id v[r]); a tile
    // of nb or more marks a dropped or absent pair.
    uint32_t t[kPer];
    V v[kPer];
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        const int64_t i = pb + 64 * r + lane;
        t[r] = i < n ? P.tiles[i] : 0xFFFFFFFFu;
        v[r] = i < n ? P.ids[i] : V{};
    }
    // Thread tid owns tiles [tid * kTPer, tid * kTPer + kTPer): their totals
    // and this chunk's prefix, requested with the pairs.
    const int t0 = tid * kTPer;
    uint32_t tv[kTPer], hv[kTPer];
#pragma unroll
    for (int j = 0; j < kTPer; ++j) {
        const bool in = t0 + j < nb;
        tv[j] = in ? P.tot[t0 + j] : 0u;
        hv[j] = in ? P.hist[c * nb + t0 + j] : 0u;
    }
    for (int i = tid; i < nb; i += kCsThreads) {
#pragma unroll
        for (int w = 0; w < kCsWaves; ++w) s_wh[w * nb + i] = 0;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kPer; ++r)
        if (t[r] < (uint32_t)nb) atomicAdd(&s_wh[wave * nb + t[r]], 1u);
    __syncthreads();
    uint32_t sum = 0;
#pragma unroll
    for (int j = 0; j < kTPer; ++j) sum += tv[j];
    uint32_t incl = sum;
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t u = __shfl_up(incl, o, 64);
        if (lane >= o) incl += u;
    }
    if (lane == 63) s_part[wave] = incl;
    __syncthreads();
    uint32_t start = incl - sum;
    for (int w = 0; w < wave; ++w) start += s_part[w];
#pragma unroll
    for (int j = 0; j < kTPer; ++j) {
        const int tt = t0 + j;
        if (tt < nb) {
            if (c == 0) P.offsets[tt] = (int32_t)start;
            uint32_t slot = start + hv[j];
#pragma unroll
            for (int w = 0; w < kCsWaves; ++w) {
                const uint32_t cnt = s_wh[w * nb + tt];
                s_wh[w * nb + tt] = slot;
                slot += cnt;
            }
        }
        start += tv[j];
    }
    // The last thread's running start has passed every tile: the total.
    if (c == 0 && tid == kCsThreads - 1) P.offsets[nb] = (int32_t)start;
    __syncthreads();
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    uint32_t *wh = s_wh + wave * nb;
    // Lanes whose pair is in the same tile (kept pairs only): one ballot per
    // tile bit, kept where the bit agrees; x is -1 where this lane's bit is 0.
    auto peers_of = [&](uint32_t tt) {
        uint64_t pm = ballot(tt < (uint32_t)nb);
        const int32_t nt = (int32_t)~tt;
        for (int b = 0; b < P.nbits; ++b) {
            const int32_t x = __builtin_amdgcn_sbfe(nt, b, 1);
            pm &= ballot(x == 0) ^ (uint64_t)(int64_t)x;
        }
        return pm;
    };
    uint64_t next = peers_of(t[0]);
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        const bool ok = t[r] < (uint32_t)nb;
        const uint64_t peers = next;
        const uint32_t wr = (uint32_t)__popcll(peers & lt);
        const uint32_t prior = ok ? wh[t[r]] : 0u;
        // The next round's ballots overlap this round's LDS read.
        if (r + 1 < kPer) next = peers_of(t[r + 1]);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (ok && wr == 0) wh[t[r]] = prior + (uint32_t)__popcll(peers);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const uint32_t pos = prior + wr;
        if (ok && (int64_t)pos < n) P.out[pos] = v[r];
    }
}

// Sorts n (tile, value) pairs stably by tile into out, and writes the list
// offsets (n_tiles + 1). Needs n_tiles <= kCsBuckets and n < 2^31.
template <typename V>
static int32_t tile_count_sort(const uint32_t *tiles, const V *ids, int64_t n, int n_tiles,
                               V *out, int32_t *tile_offsets, void *ws, int64_t ws_bytes,
                               hipStream_t s, const int64_t *status = nullptr,
                               int32_t **depth_order = nullptr) {
    MG_REQUIRE(n > 0 && n < (1LL << 31) && n_tiles >= 1 && n_tiles <= kCsBuckets,
               "tile sort: %lld pairs over %d tiles", (long long)n, n_tiles);
    const int64_t max_chunks = status ? kCsMaxChunksCapped : kCsMaxChunks;
    MG_REQUIRE(ws && ws_bytes >= tile_sort_ws_bytes(n, n_tiles, max_chunks),
               "tile sort: workspace %lld bytes, need %lld", (long long)ws_bytes,
               (long long)tile_sort_ws_bytes(n, n_tiles, max_chunks));
    const CsPlan plan = cs_plan(n, max_chunks);
    CsPass<V> P{};
    P.tiles = tiles;
    P.ids = ids;
    P.n = n;
    P.nb = n_tiles;
    P.nbits = tile_bits(n_tiles);
    P.out = out;
    P.offsets = tile_offsets;
    P.hist = static_cast<uint32_t *>(ws);
    P.tot = reinterpret_cast<uint32_t *>(static_cast<char *>(ws) +
                                         align256(4 * (int64_t)n_tiles * plan.nchunks));
    if (depth_order) {
        P.order = reinterpret_cast<int32_t *>(reinterpret_cast<char *>(P.tot) +
                                              align256(4 * (int64_t)n_tiles));
        *depth_order = P.order;
    }
    P.status = status;
    P.chunk = (int64_t)kCsThreads * plan.per;
    const unsigned grid = (unsigned)plan.nchunks;
    TimedScope ts("tile_sort", s);
#define MG_CS(PER)                                                                     \
    case PER:                                                                          \
        count_hist_kernel<PER, V><<<grid, kCsThreads, 0, s>>>(P);                      \
        MG_LAUNCHED("count_hist_kernel");                                              \
        count_colscan_kernel<V><<<(unsigned)ceil_div(n_tiles, 64), 64 * kColWaves, 0, s>>>( \
            P, plan.nchunks);                                                          \
        MG_LAUNCHED("count_colscan_kernel");                                           \
        count_scatter_kernel<PER, V><<<grid + (P.order ? 1 : 0), kCsThreads,             \
                                       4 * kCsWaves * n_tiles, s>>>(P);                   \
        MG_LAUNCHED("count_scatter_kernel");                                           \
        break;
    switch (plan.per) {
        MG_CS(8)
        MG_CS(16)
        MG_CS(24)
        MG_CS(32)
        MG_CS(48)
        MG_CS(64)
        default: MG_REQUIRE(false, "tile sort: %d pairs per lane", plan.per);
    }
#undef MG_CS
    return MG_OK;
}

// ------------------------------------------------------ per-tile depth sort
// One workgroup per tile sorts the tile's list [offsets[t], offsets[t+1]) of
// {id, depth bits} pairs stably by the depth's float bits (positive depths
// order as their bits), on only the bits in which the list's keys differ:
// LSD passes of 8 bits (9 where that takes fewer passes). The list
// arrives in ascending id, so ties keep id order. The ids are written to
// gauss_ids.
//   * Up to kTdCap entries whose keys span at most kTdKeyBits + 9 bits:
//     the keys live in registers, each wave holding one contiguous quarter
//     (rounded up to 64 entries); each pass ranks every wave's quarter
//     against a wave-private LDS histogram, joins the waves through a digit
//     scan, and exchanges the entries through LDS into their new order as
//     one word, the entry's index in the list (12 bits) over the key bits
//     still to sort (at most 20 after the first pass). After the last pass
//     the exchanged indices give each sorted position its entry, whose id is
//     read from the list (L2-resident) and stored coalesced. With one word
//     instead of a (key, id) pair the exchange buffer is 16 KB.
//   * Longer lists, or keys spanning more bits: the same pass over chunks of
//     kTdCap, in order, with the digit starts carried from chunk to chunk,
//     ping-ponging between the input pairs and scratch of the list's own
//     range.
// Lanes of a round holding the same digit find each other through a 64-bit
// LDS mask per digit: each ORs in its lane bit, then reads the mask back.
constexpr int kTdThreads = 256, kTdWaves = kTdThreads / 64, kTdPer = 16;
constexpr int kTdCap = kTdThreads * kTdPer;
constexpr int kTdBatch = 8;   // long lists: entries per thread per batch of loads
constexpr int kTdKeyBits = 20;   // key bits exchanged beside a 12-bit list index
constexpr uint32_t kTdKeyMask = (1u << kTdKeyBits) - 1u;
static_assert(kTdCap <= (1 << (32 - kTdKeyBits)), "a list index fits beside the key bits");

// The depth sort's tile order past kCsBuckets tiles (the radix route, which
// has no column scan to read the list lengths from): the tiles longest list
// first, by the order workgroup above, from the list offsets. Every tile
// lands in order once, whatever the offsets hold.
constexpr int kLenPer = 8, kLenOctBits = 7, kLenBins = 4096;
static_assert(fine_bins<kLenOctBits>() <= kLenBins, "list-length bins");

__global__ __launch_bounds__(kOrdThreads) void tile_len_order_kernel(
    const int32_t *__restrict__ offsets, int nb, int32_t *__restrict__ order) {
    __shared__ uint32_t s_cnt[kLenBins];
    __shared__ uint32_t s_wave[kOrdThreads / 64];
    const int j = threadIdx.x;
    constexpr int kBatch = kOrdThreads * kLenPer;
    for (int k = j; k < kLenBins; k += kOrdThreads) s_cnt[k] = 0;
    __syncthreads();
    // A tile's bin from its list length; its loads are issued with the
    // batch's (in range, values always used), and past nb it is negative.
    auto bins = [&](int b0, int (&bin)[kLenPer]) {
#pragma unroll
        for (int r = 0; r < kLenPer; ++r) {
            const int tt = b0 + j + kOrdThreads * r;
            const int tc = min(tt, nb - 1);
            bin[r] = fine_bin<kLenOctBits>(offsets[tc + 1] - offsets[tc]) -
                     (tt < nb ? 0 : 2 * kLenBins);
        }
    };
    for (int b0 = 0; b0 < nb; b0 += kBatch) {
        int bin[kLenPer];
        bins(b0, bin);
#pragma unroll
        for (int r = 0; r < kLenPer; ++r)
            if (bin[r] >= 0) atomicAdd(&s_cnt[bin[r]], 1u);
    }
    __syncthreads();
    desc_bin_starts<kLenBins>(s_cnt, s_wave);
    for (int b0 = 0; b0 < nb; b0 += kBatch) {
        int bin[kLenPer];
        bins(b0, bin);
#pragma unroll
        for (int r = 0; r < kLenPer; ++r)
            if (bin[r] >= 0) order[atomicAdd(&s_cnt[bin[r]], 1u)] = b0 + j + kOrdThreads * r;
    }
}

struct TdArgs {
    const int32_t *offsets;
    uint2 *pairs;                     // {id, depth bits}, grouped by tile (clobbered)
    uint2 *pairs_b;                   // scratch for lists longer than kTdCap
    int32_t *ids;                     // gauss_ids
    const int32_t *order;             // workgroup -> tile, longest list first (or NULL)
};

// Digits of the short-list passes: 8 bits, or 9 where that saves a pass,
// so that 25-27 bits take three passes instead of four (config 5's lists,
// whose depths run from the camera's near Gaussians to its far ones, span
// 25-27 bits; config 4's at most 24), and up to kTdKeyBits + 9 bits.
constexpr int kTdDigits = 512;

struct TdShared {
    // The exchange buffer and the per-digit lane masks are never live at
    // once, so they share storage (27.7 KB in all; 128 VGPRs hold the
    // workgroup to four per CU).
    union {
        uint32_t xk[kTdCap];   // exchange: list index << kTdKeyBits | key bits left
        unsigned long long mask[kTdWaves][kTdDigits];   // per wave: lanes of a round per digit
    } u;
    uint32_t wh[kTdWaves][kTdDigits];         // per wave: digit counts, then slots
    uint32_t run[256], tot[256];
    uint32_t red[2 * kTdWaves];
};

// Waits until this wave's outstanding LDS reads have returned. Needed before
// a barrier after which other waves overwrite what this wave has read: the
// barrier's own fence waits for LDS writes, not for reads whose values are
// first used after it.
__device__ __forceinline__ void lds_reads_done() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// Workgroup min and max of the keys.
__device__ __forceinline__ void td_minmax(uint32_t &kmin, uint32_t &kmax, uint32_t *red) {
    for (int o = 32; o >= 1; o >>= 1) {
        kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, o, 64));
        kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o, 64));
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) {
        red[wave] = kmin;
        red[kTdWaves + wave] = kmax;
    }
    __syncthreads();
    kmin = red[0];
    kmax = red[kTdWaves];
#pragma unroll
    for (int w = 1; w < kTdWaves; ++w) {
        kmin = min(kmin, red[w]);
        kmax = max(kmax, red[kTdWaves + w]);
    }
}

// Ranks the entries this lane holds in rounds [0, rounds) (bit r of valid
// marks a real entry) by digit d[r]: rank[r] = entries of digit d[r] before
// it in the wave's part. Counts accumulate in wh (zeroed by the caller); wm
// is zero on entry and on exit.
__device__ __forceinline__ void td_rank(const uint32_t (&d)[kTdPer], uint32_t valid, int rounds,
                                        uint32_t (&rank)[kTdPer], uint32_t *wh,
                                        unsigned long long *wm) {
    const int lane = threadIdx.x & 63;
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
    for (int r = 0; r < kTdPer; ++r) {
        if (r < rounds) {   // wave-uniform
            const bool ok = (valid >> r) & 1u;
            if (ok) atomicOr(&wm[d[r]], 1ull << lane);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const uint64_t pm = ok ? wm[d[r]] : 0ull;
            const uint32_t prior = ok ? wh[d[r]] : 0u;
            const uint32_t wr = (uint32_t)__popcll(pm & lt);
            rank[r] = prior + wr;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (ok && wr == 0) {
                wh[d[r]] = prior + (uint32_t)__popcll(pm);
                wm[d[r]] = 0ull;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }
}

// After td_rank: wh[w][dg] becomes the slot of wave w's first entry of digit
// dg: the digit's start plus the entries of that digit in earlier waves. The
// digit starts are an exclusive scan of the digit totals, or with base
// (chunked lists, 8-bit digits) base[dg], the running start carried from
// earlier chunks. tot (may be null) gets the digit totals. kPerT digits per
// thread, consecutive (256 or 512 digits).
template <int kPerT>
__device__ __forceinline__ void td_slots(TdShared &S, uint32_t *tot, const uint32_t *base) {
    static_assert(kPerT * kTdThreads <= kTdDigits, "digits fit the shared arrays");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t c[kPerT][kTdWaves], cnt[kPerT], sum = 0;
#pragma unroll
    for (int p = 0; p < kPerT; ++p) {
        cnt[p] = 0;
#pragma unroll
        for (int w = 0; w < kTdWaves; ++w) {
            c[p][w] = S.wh[w][kPerT * tid + p];
            cnt[p] += c[p][w];
        }
        sum += cnt[p];
    }
    uint32_t start;
    if (base) {
        start = base[kPerT * tid];
    } else {
        uint32_t incl = sum;
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t u = __shfl_up(incl, o, 64);
            if (lane >= o) incl += u;
        }
        if (lane == 63) S.red[wave] = incl;
        __syncthreads();
        start = incl - sum;
        for (int w = 0; w < wave; ++w) start += S.red[w];
    }
#pragma unroll
    for (int p = 0; p < kPerT; ++p) {
        if (base && p > 0) start = base[kPerT * tid + p];
#pragma unroll
        for (int w = 0; w < kTdWaves; ++w) {
            S.wh[w][kPerT * tid + p] = start;
            start += c[p][w];
        }
        if (tot) tot[kPerT * tid + p] = cnt[p];
    }
}

// Entries per wave part for a list (or chunk) of len: a quarter, rounded up
// to whole rounds of 64.
__device__ __forceinline__ int td_part(int len) { return ((len + 4 * 64 - 1) / (4 * 64)) * 64; }

// Clears every wave's lane masks. They share storage with the exchange
// buffer, which every wave may just have read: those reads must have
// returned before any wave clears the words (a barrier alone does not wait
// for LDS reads whose values are first used after it).
__device__ __forceinline__ void td_clear_masks(TdShared &S) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    lds_reads_done();
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kTdDigits / 64; ++j) S.u.mask[wave][lane + 64 * j] = 0ull;
}

// Sorts the len (2..kTdCap) entries at in by key, stably, in registers and
// LDS (see above), and writes their ids in sorted order to out. Returns
// false, having written nothing, when the keys span more than kTdKeyBits + 9
// bits. Workgroup-uniform. masks_clear: the lane masks are known zero (at
// the start of a workgroup, each wave having cleared its own), so the first
// pass need not clear them behind a barrier.
__device__ __forceinline__ bool td_fast(TdShared &S, const uint2 *in, int len, int32_t *out,
                                        bool masks_clear) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int part = td_part(len), rounds = part / 64;
    const int pb = wave * part + lane;   // entry of round r: pb + 64 r
    const uint32_t *in_key = reinterpret_cast<const uint32_t *>(in) + 1;
    uint32_t k[kTdPer], rank[kTdPer];
    uint32_t valid = 0, kmin = 0xFFFFFFFFu, kmax = 0u;
#pragma unroll
    for (int r = 0; r < kTdPer; ++r) {
        const int i = pb + 64 * r;
        const bool ok = r < rounds && i < len && 64 * r < part;
        const uint32_t ka = in_key[2 * min(i, len - 1)];
        k[r] = ok ? ka : 0u;
        valid |= ok ? 1u << r : 0u;
        kmin = min(kmin, ok ? ka : 0xFFFFFFFFu);
        kmax = max(kmax, k[r]);
    }
    td_minmax(kmin, kmax, S.red);
    const uint32_t span = kmax - kmin;
    const int bits = span == 0u ? 0 : 32 - __builtin_clz(span);
    // Digit bits (workgroup-uniform): 9 where that takes fewer passes (9,
    // 17-18 and 25-27 bits) or the keys need it (29 bits), else 8.
    const int db = ((bits + 8) / 9 < (bits + 7) / 8 || bits > kTdKeyBits + 8) ? 9 : 8;
    if (bits > kTdKeyBits + db) return false;   // workgroup-uniform
    // First pass: k is the key less kmin; later passes: k is the exchanged
    // word, the entry's list index over its key bits left.
#pragma unroll
    for (int r = 0; r < kTdPer; ++r) k[r] = ((valid >> r) & 1u) ? k[r] - kmin : 0u;
    const uint32_t dmask = (1u << db) - 1u;
    for (int shift = 0; shift < bits; shift += db) {
        if (shift > 0 || !masks_clear) td_clear_masks(S);
#pragma unroll
        for (int j = 0; j < kTdDigits / 64; ++j) S.wh[wave][lane + 64 * j] = 0;
        __syncthreads();
        uint32_t d[kTdPer];
#pragma unroll
        for (int r = 0; r < kTdPer; ++r) d[r] = k[r] & dmask;
        td_rank(d, valid, rounds, rank, S.wh[wave], S.u.mask[wave]);
        __syncthreads();
        if (db == 9) td_slots<2>(S, nullptr, nullptr);
        else td_slots<1>(S, nullptr, nullptr);
        __syncthreads();
        const bool last = shift + db >= bits;
#pragma unroll
        for (int r = 0; r < kTdPer; ++r) {
            if ((valid >> r) & 1u) {
                const uint32_t pos = S.wh[wave][d[r]] + rank[r];
                const uint32_t idx = shift == 0 ? (uint32_t)(pb + 64 * r) : k[r] >> kTdKeyBits;
                const uint32_t rest = (shift == 0 ? k[r] : k[r] & kTdKeyMask) >> db;
                // After the last pass only the index is needed.
                S.u.xk[pos] = last ? idx : (idx << kTdKeyBits) | rest;
            }
        }
        __syncthreads();
        if (last) break;
#pragma unroll
        for (int r = 0; r < kTdPer; ++r)
            if ((valid >> r) & 1u) k[r] = S.u.xk[pb + 64 * r];
    }
    if (bits == 0) {   // one key: the list order stands
        __syncthreads();
        for (int i = tid; i < len; i += kTdThreads) S.u.xk[i] = (uint32_t)i;
        __syncthreads();
    }
    // S.u.xk[i]: the list index of the entry at sorted position i. Past len
    // a lane rewrites the last position with its own value.
    uint32_t ix[kTdPer];
    int32_t id[kTdPer];
#pragma unroll
    for (int j = 0; j < kTdPer; ++j) ix[j] = S.u.xk[min(tid + kTdThreads * j, len - 1)];
#pragma unroll
    for (int j = 0; j < kTdPer; ++j) id[j] = (int32_t)in[ix[j]].x;
#pragma unroll
    for (int j = 0; j < kTdPer; ++j) out[min(tid + kTdThreads * j, len - 1)] = id[j];
    return true;
}

// Workgroup min and max of the len keys at in.
__device__ __forceinline__ void td_key_range(TdShared &S, const uint2 *in, int64_t len,
                                             uint32_t &kmin, uint32_t &kmax) {
    const int tid = threadIdx.x;
    kmin = 0xFFFFFFFFu;
    kmax = 0u;
    // The list is read kTdBatch entries per thread at a time, the loads
    // unconditional (clamped index) so that a batch is in flight at once.
    for (int64_t b = 0; b < len; b += (int64_t)kTdThreads * kTdBatch) {
        uint32_t kk[kTdBatch];
#pragma unroll
        for (int j = 0; j < kTdBatch; ++j)
            kk[j] = in[min(b + tid + (int64_t)kTdThreads * j, len - 1)].y;
#pragma unroll
        for (int j = 0; j < kTdBatch; ++j) {
            const bool ok = b + tid + (int64_t)kTdThreads * j < len;
            kmin = min(kmin, ok ? kk[j] : 0xFFFFFFFFu);
            kmax = max(kmax, ok ? kk[j] : 0u);
        }
    }
    td_minmax(kmin, kmax, S.red);
}

// Stable LSD passes of 8 bits over the len entries at pin, digits of
// (key - kmin) from bit shift0 up to bit end, in chunks of kTdCap through
// global memory: per pass the digit totals over the list, their scan into
// running starts (S.run), and the chunks in order, each ranked by its waves
// and scattered to the other buffer. With starts, the first pass's digit
// starts are also copied there (256 + 1 entries). Returns the buffer holding
// the result (pin or pout).
__device__ __forceinline__ uint2 *td_lsd_passes(TdShared &S, uint2 *pin, uint2 *pout,
                                                int64_t len, uint32_t kmin, int shift0,
                                                int end, uint32_t *starts) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int shift = shift0; shift < end; shift += 8) {
        td_clear_masks(S);
        S.tot[tid] = 0;
        __syncthreads();
        for (int64_t b = 0; b < len; b += (int64_t)kTdThreads * kTdBatch) {
            uint32_t kk[kTdBatch];
#pragma unroll
            for (int j = 0; j < kTdBatch; ++j)
                kk[j] = pin[min(b + tid + (int64_t)kTdThreads * j, len - 1)].y;
#pragma unroll
            for (int j = 0; j < kTdBatch; ++j) {
                const bool ok = b + tid + (int64_t)kTdThreads * j < len;
                atomicAdd(&S.tot[((kk[j] - kmin) >> shift) & 255u], ok ? 1u : 0u);
            }
        }
        __syncthreads();
        {
            const uint32_t cnt = S.tot[tid];
            uint32_t incl = cnt;
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t u = __shfl_up(incl, o, 64);
                if (lane >= o) incl += u;
            }
            if (lane == 63) S.red[wave] = incl;
            __syncthreads();
            uint32_t start = incl - cnt;
            for (int w = 0; w < wave; ++w) start += S.red[w];
            S.run[tid] = start;
            if (starts && shift == shift0) {
                starts[tid] = start;
                if (tid == kTdThreads - 1) starts[256] = start + cnt;
            }
        }
        for (int64_t c0 = 0; c0 < len; c0 += kTdCap) {
            const int cl = (int)min((int64_t)kTdCap, len - c0);
            const int part = td_part(cl), rounds = part / 64;
            const int pb = wave * part + lane;
            uint32_t k[kTdPer], d[kTdPer], rank[kTdPer];
            int32_t v[kTdPer];
            uint32_t valid = 0;
#pragma unroll
            for (int r = 0; r < kTdPer; ++r) {
                const int i = pb + 64 * r;
                const bool ok = r < rounds && i < cl && 64 * r < part;
                const uint2 q = pin[c0 + min(i, cl - 1)];   // loads issued together
                v[r] = ok ? (int32_t)q.x : 0;
                k[r] = ok ? q.y : 0u;
                valid |= ok ? 1u << r : 0u;
                d[r] = ((k[r] - kmin) >> shift) & 255u;
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) S.wh[wave][lane + 64 * j] = 0;
            __syncthreads();
            td_rank(d, valid, rounds, rank, S.wh[wave], S.u.mask[wave]);
            __syncthreads();
            td_slots<1>(S, S.tot, S.run);
            __syncthreads();
#pragma unroll
            for (int r = 0; r < kTdPer; ++r) {
                if ((valid >> r) & 1u) {
                    const uint32_t pos = S.wh[wave][d[r]] + rank[r];
                    pout[pos] = make_uint2((uint32_t)v[r], k[r]);
                }
            }
            S.run[tid] += S.tot[tid];   // this chunk's entries of digit tid
            __syncthreads();
        }
        // This pass's stores reach the next pass's loads: same workgroup,
        // ordered by the barrier's release and acquire.
        __syncthreads();
        uint2 *tp = pin;
        pin = pout;
        pout = tp;
    }
    return pin;
}

// The ids of the len entries at in, in order, to out.
__device__ __forceinline__ void td_write_ids(const uint2 *in, int64_t len, int32_t *out) {
    const int tid = threadIdx.x;
    // Past the end a lane rewrites the last entry with its own value.
    for (int64_t b = 0; b < len; b += (int64_t)kTdThreads * kTdBatch) {
        uint32_t id[kTdBatch];
#pragma unroll
        for (int j = 0; j < kTdBatch; ++j) id[j] = in[min(b + tid + (int64_t)kTdThreads * j, len - 1)].x;
#pragma unroll
        for (int j = 0; j < kTdBatch; ++j)
            out[min(b + tid + (int64_t)kTdThreads * j, len - 1)] = (int32_t)id[j];
    }
}

// Lists the fast path does not take: longer than kTdCap, or keys spanning
// more than kTdKeyBits + 9 bits. One LSD pass on the top 8 of the key bits
// (through global memory, into pairs_b) groups the list into up to 256
// buckets of consecutive key ranges, stably; runs of whole buckets of up to
// kTdCap entries are then sorted by the fast path, each its own segment of
// the ids (a bucket of more than kTdCap entries, or a run whose keys still
// span too many bits, takes the LSD passes on its own). Against LSD passes
// over the whole list this reads and writes the list through global memory
// once instead of once per 8 key bits. Not inlined: the kernel reaches it
// rarely, and inlined its registers made the fast path spill.
__device__ __noinline__ void td_long(TdShared &S, const TdArgs A, int64_t s0, int64_t len) {
    const int tid = threadIdx.x;
    __shared__ uint32_t s_starts[257];
    uint2 *in = A.pairs + s0, *tmp = A.pairs_b + s0;
    int32_t *out = A.ids + s0;
    uint32_t kmin, kmax;
    td_key_range(S, in, len, kmin, kmax);
    const uint32_t span = kmax - kmin;
    const int bits = span == 0u ? 0 : 32 - __builtin_clz(span);
    if (bits <= 8) {
        td_write_ids(td_lsd_passes(S, in, tmp, len, kmin, 0, bits, nullptr), len, out);
        return;
    }
    // in -> tmp, grouped by the digit of bits [bits - 8, bits).
    td_lsd_passes(S, in, tmp, len, kmin, bits - 8, bits, s_starts);
    __syncthreads();
    // Runs of whole buckets [b, e): every thread walks the same bucket
    // starts, so the loop is workgroup-uniform.
    int64_t b = 0;
    for (int dg = 0; dg <= 256; ++dg) {
        const int64_t e = s_starts[dg];   // end of bucket dg - 1
        const int64_t nxt = dg < 256 ? (int64_t)s_starts[dg + 1] : e;
        // Close the run before bucket dg if bucket dg would overfill it (or
        // at the end).
        if (dg == 256 || (nxt - b > kTdCap && e > b)) {
            const int64_t n = e - b;
            if (n == 1) {
                if (tid == 0) out[b] = (int32_t)tmp[b].x;
            } else if (n > 1) {
                if (n > kTdCap || !td_fast(S, tmp + b, (int)n, out + b, false)) {
                    // The run's own key range and LSD passes; the input region
                    // of the list is free scratch by now.
                    uint32_t rmin, rmax;
                    td_key_range(S, tmp + b, n, rmin, rmax);
                    const uint32_t rs = rmax - rmin;
                    const int rb = rs == 0u ? 0 : 32 - __builtin_clz(rs);
                    td_write_ids(td_lsd_passes(S, tmp + b, in + b, n, rmin, 0, rb, nullptr), n,
                                 out + b);
                }
            }
            __syncthreads();
            b = e;
        }
    }
}

// Four workgroups per CU: at most 128 VGPRs.
__global__ __launch_bounds__(kTdThreads) __attribute__((amdgpu_waves_per_eu(4))) void
tile_depth_sort_kernel(const TdArgs A) {
    __shared__ TdShared S;
    const int tid = threadIdx.x;
    const int t = A.order ? A.order[blockIdx.x] : (int)xcd_contiguous(blockIdx.x, gridDim.x);
    const int64_t s0 = A.offsets[t];
    const int64_t len = (int64_t)A.offsets[t + 1] - s0;
    if (len <= 0) return;   // workgroup-uniform
    const uint2 *in = A.pairs + s0;
    if (len == 1) {
        if (tid == 0) A.ids[s0] = (int32_t)in[0].x;
        return;
    }
    {
        const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
        for (int j = 0; j < kTdDigits / 64; ++j) S.u.mask[wave][lane + 64 * j] = 0ull;
    }
    if (len <= kTdCap && td_fast(S, in, (int)len, A.ids + s0, true)) return;
    td_long(S, A, s0, len);
}

// Carves the begin/finish workspace identically on both calls. After begin,
// counts holds each Gaussian's tile count, part_off the first pair of each
// 256-Gaussian workgroup, recs the walk records.
struct BeginWs {
    int32_t *counts;
    uint32_t *masks;
    BinRec *recs;
    uint64_t *words;    // kBlockWords per count workgroup
    BinPart *parts;
    int64_t *part_off;
    BinStats *stats;
    int32_t *order;     // the blocks' processing order (with a block work estimate)
    int64_t bytes;
    BeginWs(void *base, int64_t N) {
        char *p = static_cast<char *>(base);
        int64_t off = 0;
        auto take = [&](int64_t b) { char *q = p ? p + off : nullptr; off += align256(b); return q; };
        const int64_t nparts = ceil_div(N, kBinThreads);
        counts = (int32_t *)take(4 * N);
        masks = (uint32_t *)take(4 * N);
        recs = (BinRec *)take((int64_t)sizeof(BinRec) * N);
        words = (uint64_t *)take(8 * kBlockWords * nparts);
        parts = (BinPart *)take((int64_t)sizeof(BinPart) * nparts);
        part_off = (int64_t *)take(8 * nparts);
        stats = (BinStats *)take(sizeof(BinStats));
        order = (int32_t *)take(4 * nparts);
        bytes = off;
    }
};

static int32_t check_bin_args(const char *who, int64_t N, const void *uv, const void *rxy,
                              const void *conic, const void *opac, const void *valid, int W,
                              int H, int tile, int tiles_x, int tiles_y) {
    MG_REQUIRE(N >= 0 && N < (1LL << 31), "%s: N = %lld", who, (long long)N);
    MG_REQUIRE(W > 0 && H > 0 && tile > 0, "%s: image %dx%d tile %d", who, W, H, tile);
    MG_REQUIRE(tiles_x == (W + tile - 1) / tile && tiles_y == (H + tile - 1) / tile,
               "%s: tiles %dx%d do not cover %dx%d at tile %d", who, tiles_x, tiles_y, W, H,
               tile);
    MG_REQUIRE((int64_t)tiles_x * tiles_y < (1LL << 31) && tiles_x < 65536 && tiles_y < 65536,
               "%s: too many tiles (%d x %d)", who, tiles_x, tiles_y);
    MG_REQUIRE(N == 0 || (uv && rxy && valid), "%s: null tensor pointer", who);
    MG_REQUIRE((conic == nullptr) == (opac == nullptr),
               "%s: conic and opacity must be given together (or both omitted)", who);
    return MG_OK;
}

// Scratch of either tile sort: the radix passes' histograms, or the counting
// sort's per-chunk counts at its largest tile count.
static int64_t finish_sort_bytes(int64_t T, bool capped) {
    return align256(std::max(sort_ws_bytes(T),
                             tile_sort_ws_bytes(T, kCsBuckets,
                                                capped ? kCsMaxChunksCapped : kCsMaxChunks)));
}

// Pairs in Gaussian order, grouped by tile, then each tile's list sorted by
// depth, into gauss_ids and tile_offsets. n is the pair count (status NULL),
// or the capacity of capacity-bounded lists, whose kernels read the pairs to
// keep from status on the device (none after an overflow: every list empty).
// bin_write emits each pair's tile key and its {id, depth bits} value. Up to
// kCsBuckets tiles the one-pass counting sort carries the values by tile (and
// writes the offsets); otherwise radix passes on the tile bits carry them
// (the keys ping-pong through gauss_ids, which only the depth sort writes),
// and tile_ranges writes the offsets; for capacity-bounded lists both read
// the kept count from status and leave the slots past it alone.
static int32_t emit_and_sort(const BeginWs &ws, int64_t N, const float *conic,
                             const float *depth, int W, int H, int tile, int tiles_x,
                             int n_tiles, int64_t n, const int64_t *status, int32_t *gauss_ids,
                             int32_t *tile_offsets, void *finish_workspace, hipStream_t s,
                             const int32_t *block_order = nullptr) {
    const int64_t T = n > 0 ? n : 1;
    const int64_t T4 = align256(4 * T);
    char *f = static_cast<char *>(finish_workspace);
    uint2 *pairs_a = (uint2 *)f;                      // region A: 2 * T4 bytes
    uint2 *pairs_b = (uint2 *)(f + 2 * T4);           // region B: 2 * T4 bytes
    uint32_t *tk_a = (uint32_t *)(f + 4 * T4);
    void *sort_ws = f + 5 * T4;
    const int64_t sort_bytes = finish_sort_bytes(T, status != nullptr);
    uint32_t *res_tiles = tk_a;
    if (n == 0 || N == 0) {
        TimedScope ts("tile_ranges", s);
        tile_ranges_u32_kernel<<<1, 256, 0, s>>>(res_tiles, 0, n_tiles, tile_offsets, nullptr);
        MG_LAUNCHED("tile_ranges_u32_kernel");
        return MG_OK;
    }
    int32_t rc = MG_OK;
    const bool counting = n_tiles <= kCsBuckets;
    const int bits = tile_bits(n_tiles);
    {
        TimedScope ts("bin_write", s);
        bin_write_rec_kernel<<<(unsigned)ceil_div(N, kBinThreads), kBinThreads, 0, s>>>(
            ws.recs, ws.counts, ws.masks, ws.words, ws.part_off, N, tile, W, H, tiles_x,
            conic != nullptr ? 1 : 0, tk_a, nullptr, depth, pairs_a, status, block_order);
        MG_LAUNCHED("bin_write_rec_kernel");
    }
    // The tile-sorted pairs, and the other region (the long lists' scratch).
    uint2 *sorted = pairs_b, *scratch = pairs_a;
    int32_t *order = nullptr;
    if (counting) {
        rc = tile_count_sort<uint2>(tk_a, pairs_a, n, n_tiles, pairs_b, tile_offsets, sort_ws,
                                    sort_bytes, s, status, &order);
        if (rc != MG_OK) return rc;
    } else {
        rc = radix_sort_passes<uint32_t, uint2>(
            tk_a, pairs_a, reinterpret_cast<uint32_t *>(gauss_ids), pairs_b, n, 0, bits, sort_ws,
            sort_bytes, s, "tile_sort", &res_tiles, &sorted, 0u, 0xFFFFFFFFu, nullptr, status);
        if (rc != MG_OK) return rc;
        scratch = sorted == pairs_a ? pairs_b : pairs_a;
        {
            TimedScope ts("tile_ranges", s);
            tile_ranges_u32_kernel<<<(unsigned)ceil_div(n + 1, 256 * kRangePer), 256, 0, s>>>(
                res_tiles, n, n_tiles, tile_offsets, status);
            MG_LAUNCHED("tile_ranges_u32_kernel");
        }
        // The depth sort's longest-first order, in the keys region (free once
        // the tile ranges are read from whichever buffer holds the sorted
        // keys) when it holds a word per tile.
        if (n_tiles <= T) {
            order = reinterpret_cast<int32_t *>(tk_a);
            TimedScope ts("depth_order", s);
            tile_len_order_kernel<<<1, kOrdThreads, 0, s>>>(tile_offsets, n_tiles, order);
            MG_LAUNCHED("tile_len_order_kernel");
        }
    }
    TdArgs D{tile_offsets, sorted, scratch, gauss_ids, order};
    TimedScope ts("depth_sort", s);
    tile_depth_sort_kernel<<<(unsigned)n_tiles, kTdThreads, 0, s>>>(D);
    MG_LAUNCHED("tile_depth_sort_kernel");
    return MG_OK;
}

}  // namespace mg

using namespace mg;

extern "C" {

int32_t mg_bin_count(int64_t N, const float *uv, const float *rxy, const float *conic,
                     const float *opacity, const int32_t *valid, int32_t W, int32_t H,
                     int32_t tile, int32_t tiles_x, int32_t tiles_y, int32_t *counts,
                     mg_stream_t stream) {
    int32_t rc = check_bin_args("mg_bin_count", N, uv, rxy, conic, opacity, valid, W, H, tile,
                                tiles_x, tiles_y);
    if (rc != MG_OK) return rc;
    if (N == 0) return MG_OK;
    MG_REQUIRE(counts, "mg_bin_count: null counts");
    BinArgs A{N, uv, rxy, conic, opacity, nullptr, valid, W, H, tile, tiles_x, tiles_y};
    TimedScope ts("bin_count", as_stream(stream));
    bin_count_kernel<<<(unsigned)ceil_div(N, kBinThreads), kBinThreads, 0, as_stream(stream)>>>(
        A, counts);
    MG_LAUNCHED("bin_count_kernel");
    return MG_OK;
}

int64_t mg_scan_workspace_bytes(int64_t n) { return scan_ws_bytes(n); }

int32_t mg_exclusive_scan_i32(const int32_t *in, int64_t n, int32_t *out, int64_t *total_dev,
                              int64_t *total_host, void *workspace, int64_t workspace_bytes,
                              mg_stream_t stream) {
    MG_REQUIRE(n >= 0, "mg_exclusive_scan_i32: n = %lld", (long long)n);
    MG_REQUIRE(total_dev, "mg_exclusive_scan_i32: null total_dev");
    MG_REQUIRE(n == 0 || (in && out), "mg_exclusive_scan_i32: null input/output");
    hipStream_t s = as_stream(stream);
    int32_t rc =
        exclusive_scan(in, nullptr, n, out, total_dev, workspace, workspace_bytes, s, nullptr);
    if (rc != MG_OK) return rc;
    if (total_host) {
        MG_HIP(hipMemcpyAsync(total_host, total_dev, sizeof(int64_t), hipMemcpyDeviceToHost, s));
        MG_HIP(hipStreamSynchronize(s));
    }
    return MG_OK;
}

int32_t mg_bin_write(int64_t N, const float *uv, const float *rxy, const float *conic,
                     const float *opacity, const int32_t *valid, const float *depth,
                     const int32_t *offsets, int64_t total, int32_t W, int32_t H, int32_t tile,
                     int32_t tiles_x, int32_t tiles_y, uint64_t *keys, int32_t *ids,
                     mg_stream_t stream) {
    int32_t rc = check_bin_args("mg_bin_write", N, uv, rxy, conic, opacity, valid, W, H, tile,
                                tiles_x, tiles_y);
    if (rc != MG_OK) return rc;
    MG_REQUIRE(total >= 0 && total < (1LL << 31), "mg_bin_write: total %lld", (long long)total);
    if (N == 0 || total == 0) return MG_OK;
    MG_REQUIRE(depth && offsets && keys && ids, "mg_bin_write: null tensor pointer");
    BinArgs A{N, uv, rxy, conic, opacity, depth, valid, W, H, tile, tiles_x, tiles_y};
    TimedScope ts("bin_write", as_stream(stream));
    bin_write_kernel<<<(unsigned)ceil_div(N, kBinThreads), kBinThreads, 0, as_stream(stream)>>>(
        A, offsets, keys, ids);
    MG_LAUNCHED("bin_write_kernel");
    return MG_OK;
}

int32_t mg_tile_ranges(const uint64_t *sorted_keys, int64_t n, int32_t n_tiles,
                       int32_t *tile_offsets, mg_stream_t stream) {
    MG_REQUIRE(n >= 0 && n < (1LL << 31), "mg_tile_ranges: n = %lld", (long long)n);
    MG_REQUIRE(n_tiles >= 1 && tile_offsets, "mg_tile_ranges: n_tiles %d", n_tiles);
    MG_REQUIRE(n == 0 || sorted_keys, "mg_tile_ranges: null keys");
    TimedScope ts("tile_ranges", as_stream(stream));
    tile_ranges_kernel<<<(unsigned)ceil_div(n + 1, 256), 256, 0, as_stream(stream)>>>(
        sorted_keys, n, n_tiles, tile_offsets);
    MG_LAUNCHED("tile_ranges_kernel");
    return MG_OK;
}

int64_t mg_sort_pairs_by_tile_workspace_bytes(int64_t n, int32_t n_tiles) {
    if (n <= 0 || n_tiles < 1) return 0;
    return tile_sort_ws_bytes(n, n_tiles);
}

int32_t mg_sort_pairs_by_tile(int64_t n, const uint32_t *tiles, const int32_t *ids,
                              int32_t n_tiles, int32_t *ids_out, int32_t *tile_offsets,
                              void *workspace, int64_t workspace_bytes, mg_stream_t stream) {
    MG_REQUIRE(n > 0 && n < (1LL << 31), "mg_sort_pairs_by_tile: n = %lld", (long long)n);
    MG_REQUIRE(n_tiles >= 1 && n_tiles <= kCsBuckets, "mg_sort_pairs_by_tile: %d tiles (1..%d)",
               n_tiles, kCsBuckets);
    MG_REQUIRE(tiles && ids && ids_out && tile_offsets, "mg_sort_pairs_by_tile: null pointer");
    MG_REQUIRE(ids_out != ids, "mg_sort_pairs_by_tile: ids_out must not alias ids");
    MG_REQUIRE(((uintptr_t)tiles & 15) == 0, "mg_sort_pairs_by_tile: tiles not 16-byte aligned");
    return tile_count_sort(tiles, ids, n, n_tiles, ids_out, tile_offsets, workspace,
                           workspace_bytes, as_stream(stream));
}

int64_t mg_bin_lists_workspace_bytes(int64_t N) { return BeginWs(nullptr, N > 0 ? N : 1).bytes; }

// Two regions of 8 bytes per pair (the pairs' {id, depth bits} values, and
// the tile-sorted copy), the pairs' tile keys, then the sort scratch. The
// radix route (more than kCsBuckets tiles) ping-pongs the values between the
// two regions and the keys through the caller's gauss_ids.
int64_t mg_bin_lists_finish_workspace_bytes(int64_t total) {
    const int64_t T = total > 0 ? total : 1;
    return 5 * align256(4 * T) + finish_sort_bytes(T, false);
}

int32_t mg_bin_lists_begin(int64_t N, const float *uv, const float *rxy, const float *conic,
                           const float *opacity, const int32_t *valid, const float *depth,
                           int32_t W, int32_t H, int32_t tile, int32_t tiles_x, int32_t tiles_y,
                           void *workspace, int64_t workspace_bytes, int64_t *total_host,
                           mg_stream_t stream) {
    int32_t rc = check_bin_args("mg_bin_lists_begin", N, uv, rxy, conic, opacity, valid, W, H,
                                tile, tiles_x, tiles_y);
    if (rc != MG_OK) return rc;
    MG_REQUIRE(depth || N == 0, "mg_bin_lists_begin: null depth");
    BeginWs ws(workspace, N > 0 ? N : 1);
    MG_REQUIRE(workspace && workspace_bytes >= ws.bytes,
               "mg_bin_lists_begin: workspace %lld bytes, need %lld", (long long)workspace_bytes,
               (long long)ws.bytes);
    hipStream_t s = as_stream(stream);
    BinArgs A{N, uv, rxy, conic, opacity, depth, valid, W, H, tile, tiles_x, tiles_y};
    const int64_t nparts = N > 0 ? ceil_div(N, kBinThreads) : 0;
    if (N > 0) {
        TimedScope ts("bin_count", s);
        bin_count_rec_kernel<<<(unsigned)nparts, kBinThreads, 0, s>>>(
            A, ws.counts, ws.recs, ws.masks, ws.words, ws.parts, nullptr);
        MG_LAUNCHED("bin_count_rec_kernel");
    }
    {
        TimedScope ts("exclusive_scan", s);
        bin_offsets_kernel<<<1, kScanThreads, 0, s>>>(ws.parts, nparts, ws.part_off, ws.stats,
                                                       0, nullptr, nullptr, 0);
        MG_LAUNCHED("bin_offsets_kernel");
    }
    // The one host read: the total sizes the caller's id buffer. It is copied
    // into a pinned word behind an event.
    HostReadback rb;
    if (!rb.ok()) return MG_ERR_RUNTIME;
    MG_HIP(hipMemcpyAsync(rb.slot, &ws.stats->total, sizeof(int64_t), hipMemcpyDeviceToHost, s));
    MG_HIP(hipEventRecord(rb.ev, s));
    MG_HIP(hipEventSynchronize(rb.ev));
    const int64_t total = *rb.slot;
    MG_REQUIRE(total >= 0 && total < (1LL << 31),
               "mg_bin_lists_begin: %lld intersections exceed int32", (long long)total);
    if (total_host) *total_host = total;
    return MG_OK;
}

int32_t mg_bin_lists_finish(int64_t N, const float *uv, const float *rxy, const float *conic,
                            const float *opacity, const int32_t *valid, const float *depth,
                            int32_t W, int32_t H, int32_t tile, int32_t tiles_x, int32_t tiles_y,
                            const void *workspace, int64_t workspace_bytes, int64_t total,
                            int32_t *gauss_ids, int32_t *tile_offsets, void *finish_workspace,
                            int64_t finish_workspace_bytes, mg_stream_t stream) {
    int32_t rc = check_bin_args("mg_bin_lists_finish", N, uv, rxy, conic, opacity, valid, W, H,
                                tile, tiles_x, tiles_y);
    if (rc != MG_OK) return rc;
    MG_REQUIRE(total >= 0 && total < (1LL << 31), "mg_bin_lists_finish: total %lld",
               (long long)total);
    MG_REQUIRE(tile_offsets, "mg_bin_lists_finish: null tile_offsets");
    BeginWs ws(const_cast<void *>(workspace), N > 0 ? N : 1);
    MG_REQUIRE(workspace && workspace_bytes >= ws.bytes,
               "mg_bin_lists_finish: begin workspace %lld bytes, need %lld",
               (long long)workspace_bytes, (long long)ws.bytes);
    MG_REQUIRE(finish_workspace &&
                   finish_workspace_bytes >= mg_bin_lists_finish_workspace_bytes(total),
               "mg_bin_lists_finish: workspace %lld bytes, need %lld",
               (long long)finish_workspace_bytes,
               (long long)mg_bin_lists_finish_workspace_bytes(total));
    if (total > 0) {
        MG_REQUIRE(gauss_ids, "mg_bin_lists_finish: null gauss_ids");
        MG_REQUIRE(N > 0, "mg_bin_lists_finish: %lld intersections from no Gaussians",
                   (long long)total);
        MG_REQUIRE(depth, "mg_bin_lists_finish: null depth");
    }
    return emit_and_sort(ws, N, conic, depth, W, H, tile, tiles_x, tiles_x * tiles_y, total,
                         nullptr, gauss_ids, tile_offsets, finish_workspace, as_stream(stream));
}

int64_t mg_bin_lists_capped_workspace_bytes(int64_t N, int64_t capacity) {
    if (N < 0 || capacity < 0) return 0;
    const int64_t T = capacity > 0 ? capacity : 1;
    return BeginWs(nullptr, N > 0 ? N : 1).bytes + 5 * align256(4 * T) +
           finish_sort_bytes(T, true);
}

int32_t mg_bin_lists_capped(int64_t N, const float *uv, const float *rxy, const float *conic,
                            const float *opacity, const int32_t *valid, const float *depth,
                            int32_t W, int32_t H, int32_t tile, int32_t tiles_x, int32_t tiles_y,
                            int64_t capacity, int32_t *gauss_ids, int32_t *tile_offsets,
                            int64_t *status, int64_t *status_host, int64_t tag,
                            void *workspace, int64_t workspace_bytes,
                            const int32_t *block_work, mg_stream_t stream) {
    int32_t rc = check_bin_args("mg_bin_lists_capped", N, uv, rxy, conic, opacity, valid, W, H,
                                tile, tiles_x, tiles_y);
    if (rc != MG_OK) return rc;
    MG_REQUIRE(capacity >= 0 && capacity < (1LL << 31), "mg_bin_lists_capped: capacity %lld",
               (long long)capacity);
    MG_REQUIRE(tile_offsets && status, "mg_bin_lists_capped: null tile_offsets or status");
    MG_REQUIRE(capacity == 0 || gauss_ids, "mg_bin_lists_capped: null gauss_ids");
    MG_REQUIRE(depth || N == 0, "mg_bin_lists_capped: null depth");
    const int64_t need = mg_bin_lists_capped_workspace_bytes(N, capacity);
    MG_REQUIRE(workspace && workspace_bytes >= need,
               "mg_bin_lists_capped: workspace %lld bytes, need %lld",
               (long long)workspace_bytes, (long long)need);
    BeginWs ws(workspace, N > 0 ? N : 1);
    hipStream_t s = as_stream(stream);
    BinArgs A{N, uv, rxy, conic, opacity, depth, valid, W, H, tile, tiles_x, tiles_y};
    const int64_t nparts = N > 0 ? ceil_div(N, kBinThreads) : 0;
    const int32_t *order = (block_work && N > 0) ? ws.order : nullptr;
    if (N > 0) {
        TimedScope ts("bin_count", s);
        if (order) {
            block_order_kernel<<<1, kOrdThreads, 0, s>>>(block_work, nparts, ws.order);
            MG_LAUNCHED("block_order_kernel");
        }
        bin_count_rec_kernel<<<(unsigned)nparts, kBinThreads, 0, s>>>(
            A, ws.counts, ws.recs, ws.masks, ws.words, ws.parts, order);
        MG_LAUNCHED("bin_count_rec_kernel");
    }
    {
        TimedScope ts("exclusive_scan", s);
        bin_offsets_kernel<<<1, kScanThreads, 0, s>>>(ws.parts, nparts, ws.part_off, ws.stats,
                                                       capacity, status, status_host,
                                                       tag);
        MG_LAUNCHED("bin_offsets_kernel");
    }
    return emit_and_sort(ws, N, conic, depth, W, H, tile, tiles_x, tiles_x * tiles_y,
                         N > 0 ? capacity : 0, status, gauss_ids, tile_offsets,
                         static_cast<char *>(workspace) + ws.bytes, s, order);
}

}  // extern "C"
