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
//   Per pixel the backward keeps T and one running scalar, the suffix sum
//   of the output gradient dotted with the colour composited behind,
//   G = gr sr + gg sg + gb sb + ga sa, which is all that dL/dalpha needs:
//   dL/dalpha = (T (g . c + ga) - G) / (1 - alpha). The 9 (10 with absgrad)
//   per-Gaussian sums are the colour weights and the moments of
//   dg = dL/dgauss over the pixels (sum dg, dg dx, dg dy, dg dx^2, dg dx dy,
//   dg dy^2), reduced across the 64 lanes with lane swaps and DPP and added
//   into a per-batch LDS accumulator (LDS float atomics: several waves may
//   hold the same Gaussian). After the batch one thread per Gaussian turns
//   the moments into the uv, conic and opacity gradients with the
//   Gaussian's own opacity and conic, and the workgroup issues the global
//   float atomics into one 10-float gradient record per Gaussian, slot by
//   slot (consecutive lanes update consecutive slots of one record, so an
//   instruction touches a few records rather than 64 scattered lines: about
//   5x cheaper at the memory side, where device-scope atomics are performed
//   across MI355X's eight XCD L2s). There is one set per (Gaussian, tile)
//   rather than per (Gaussian, wave).
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
    // Forward only, optional: zero_n floats (16-byte aligned) cleared on the
    // way, a later backward's gradient records; each workgroup clears a slice.
    float *zero;
    int64_t zero_n;
    // Optional backward schedule: the forward writes each tile's walk length
    // (work, n_tiles); the backward's workgroup b takes tile order[b].
    int32_t *work;
    const int32_t *order;
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

// Workgroup -> tile. The dispatcher deals workgroup b to XCD b % 8, as that
// XCD's (b / 8)-th. Tiles are grouped into kSuper x kSuper super-tiles, and
// the super-tiles are dealt round-robin to the XCDs. Neighbouring tiles share
// many Gaussians, so each super-tile's 16 tiles run on one XCD and hit its
// L2. Every XCD gets super-tiles from all over the image, so the dense
// centre is spread over all eight. Slots outside the image get -1.
constexpr int kSuper = 4;

inline int raster_grid(int tiles_x, int tiles_y) {
    const int n_super = ((tiles_x + kSuper - 1) / kSuper) * ((tiles_y + kSuper - 1) / kSuper);
    return ((n_super + kXcds - 1) / kXcds) * kXcds * kSuper * kSuper;
}

__device__ __forceinline__ int tile_of_block(int bid, int tiles_x, int tiles_y) {
    const int xcd = bid % kXcds, k = bid / kXcds;
    const int per = kSuper * kSuper;
    const int sup = (k / per) * kXcds + xcd;
    const int sx = (tiles_x + kSuper - 1) / kSuper, sy = (tiles_y + kSuper - 1) / kSuper;
    if (sup >= sx * sy) return -1;
    const int local = k % per;
    const int tx = (sup % sx) * kSuper + local % kSuper;
    const int ty = (sup / sx) * kSuper + local / kSuper;
    return tx < tiles_x && ty < tiles_y ? ty * tiles_x + tx : -1;
}

// The conic as the walks keep it in LDS: (-a/2, -b, -c/2), so that the
// splat's exponent -(a dx^2 + 2 b dx dy + c dy^2) / 2 is one fma chain.
// Scaling by -1/2 and -1 is exact in floating point, so every product and
// sum rounds to exactly the negated half of what the unscaled expression
// fma(a dx, dx, fma(2 b dx, dy, c dy dy)) rounds to: the exponent is bit for
// bit the one of the per-pixel contract, with two instructions fewer per
// (entry, wave). Folding log2(e) in as well saves one more but rounds
// differently: on config 5's near-singular conics, whose terms cancel, that
// moved alphas across the 1/255 cutoff.
__device__ __forceinline__ float4 scale_conic(const float4 con) {
    return make_float4(-0.5f * con.x, -con.y, -0.5f * con.z, 0.f);
}

// The exponent of the splat at offset (dx, dy) from the staged conic.
// Written with explicit fmas so the forward and the backward round
// identically: the backward divides the forward's (1 - alpha) back out and
// must see the same alpha bit for bit.
__device__ __forceinline__ float splat_power(float dx, float dy, const float4 k) {
    return fmaf(k.x * dx, dx, fmaf(k.y * dx, dy, k.z * dy * dy));
}

// The raw conic (a, b, c) back from its staged form (exact).
__device__ __forceinline__ float3 raw_conic(const float4 k) {
    return make_float3(-2.0f * k.x, -k.y, -2.0f * k.z);
}

// Conservative per-wave cull: minimum of the quadratic form over the box of
// the wave's pixel centres, against 2 ln(255 op) widened by a rounding margin
// (the reference's own margin, rasterize.metal:150-151). The entry's 1/a and
// 1/c are formed once for all its wave boxes (a and c clamped at 1e-12).
__device__ __forceinline__ float rect_min_q(float mux, float muy, float a, float b, float c,
                                                float ia, float ic, float x0, float x1,
                                                float y0, float y1) {
    if (mux >= x0 && mux <= x1 && muy >= y0 && muy <= y1) return 0.0f;
    float best = __builtin_inff();
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const float yc = e == 0 ? y0 : y1;
        const float xs = fminf(fmaxf(mux - b * (yc - muy) * ia, x0), x1);
        const float ex = xs - mux, ey = yc - muy;
        best = fminf(best, a * ex * ex + 2.0f * b * ex * ey + c * ey * ey);
    }
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const float xc = e == 0 ? x0 : x1;
        const float ys = fminf(fmaxf(muy - b * (xc - mux) * ic, y0), y1);
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

constexpr int kGradSlots = 10;   // colour 3, moments 5, sum dg, |d uv|

// Wave sums of ten values by lane swaps. v_permlane32_swap a, b swaps lanes
// 32-63 of a with lanes 0-31 of b, leaving (a[0:32], b[0:32]) in a and
// (a[32:64], b[32:64]) in b, so a + b holds a's half-sums in lanes 0-31 and
// b's in lanes 32-63. v_permlane16_swap does the same between rows 0/1 and
// 2/3. After the two swap stages each row of 16 lanes carries one value's
// partials, which a row reduction finishes: rows of q0 hold the sums of v0,
// v2, v1, v3; of q1 v4, v6, v5, v7; of q2 v8, -, v9, -. 26 VALU operations
// for ten sums.
//
// The swaps are inline assembly: this compiler folds the two results of the
// __builtin_amdgcn_permlane*_swap builtins into one register (r[0] + r[1]
// comes out as r[0] + r[0]). A swap needs two wait states after a VALU write
// of its operands; each stage's swaps read only registers written before the
// stage and write disjoint pairs, so one s_nop 1 at the head of a stage
// covers all of them.
__device__ __forceinline__ float row_allsum(float x) {
    x += dpp_f<0x128>(x);   // row_ror:8
    x += dpp_f<0x124>(x);   // row_ror:4
    x += dpp_f<0x122>(x);   // row_ror:2
    x += dpp_f<0x121>(x);   // row_ror:1
    return x;
}
__device__ __forceinline__ void reduce10_to_rows(const float v[10], float &q0, float &q1,
                                                 float &q2) {
    float a0 = v[0], b0 = v[1], a1 = v[2], b1 = v[3], a2 = v[4], b2 = v[5];
    float a3 = v[6], b3 = v[7], a4 = v[8], b4 = v[9];
    asm volatile(
        "s_nop 1\n\t"
        "v_permlane32_swap_b32 %0, %1\n\t"
        "v_permlane32_swap_b32 %2, %3\n\t"
        "v_permlane32_swap_b32 %4, %5\n\t"
        "v_permlane32_swap_b32 %6, %7\n\t"
        "v_permlane32_swap_b32 %8, %9"
        : "+v"(a0), "+v"(b0), "+v"(a1), "+v"(b1), "+v"(a2), "+v"(b2), "+v"(a3), "+v"(b3),
          "+v"(a4), "+v"(b4));
    float p0 = a0 + b0, p1 = a1 + b1, p2 = a2 + b2, p3 = a3 + b3, p4 = a4 + b4;
    float z = 0.0f;
    asm volatile(
        "s_nop 1\n\t"
        "v_permlane16_swap_b32 %0, %1\n\t"
        "v_permlane16_swap_b32 %2, %3\n\t"
        "v_permlane16_swap_b32 %4, %5"
        : "+v"(p0), "+v"(p1), "+v"(p2), "+v"(p3), "+v"(p4), "+v"(z));
    q0 = row_allsum(p0 + p1);
    q1 = row_allsum(p2 + p3);
    q2 = row_allsum(p4 + z);
}

// Wave sums of two entries' nine values each (a: entry A, b: entry B), for
// one LDS atomic per sum. The two swap stages above leave, in lane bits 5 and
// 4, the entry and the parity of the value index; three transposing DPP
// stages then halve the values again per lane bit while summing (row_ror:8
// pairs lane bit 3, row_half_mirror pairs lanes l and 7 - l of an 8-lane
// group across bit 2, quad_perm l ^ 2 bit 1), and quad_perm l ^ 1 ends the
// sum. Lane l returns the full sum of value
//   4 b2 + 2 b3 + b4   when bit 1 is clear,
//   8                  when bit 1 is set and bits 2-4 are clear,
// of entry bit 5 (bits b_i of l); its pair partner l ^ 1 holds the same sum,
// and the other lanes with bit 1 set hold the zero padding. reduce18_slot
// names each lane's value, -1 for lanes that deposit nothing. 44 VALU
// operations for eighteen sums, against 2 x 26 plus twice the deposits.
__device__ __forceinline__ int reduce18_slot(int lane) {
    if (lane & 1) return -1;
    if (lane & 2) return (lane & 0x1C) == 0 ? 8 : -1;
    return 4 * ((lane >> 2) & 1) + 2 * ((lane >> 3) & 1) + ((lane >> 4) & 1);
}
__device__ __forceinline__ float reduce18(const float a[9], const float b[9], int lane) {
    float x0 = a[0], x1 = a[1], x2 = a[2], x3 = a[3], x4 = a[4], x5 = a[5], x6 = a[6];
    float x7 = a[7], x8 = a[8];
    float y0 = b[0], y1 = b[1], y2 = b[2], y3 = b[3], y4 = b[4], y5 = b[5], y6 = b[6];
    float y7 = b[7], y8 = b[8];
    asm volatile(
        "s_nop 1\n\t"
        "v_permlane32_swap_b32 %0, %1\n\t"
        "v_permlane32_swap_b32 %2, %3\n\t"
        "v_permlane32_swap_b32 %4, %5\n\t"
        "v_permlane32_swap_b32 %6, %7\n\t"
        "v_permlane32_swap_b32 %8, %9\n\t"
        "v_permlane32_swap_b32 %10, %11\n\t"
        "v_permlane32_swap_b32 %12, %13\n\t"
        "v_permlane32_swap_b32 %14, %15\n\t"
        "v_permlane32_swap_b32 %16, %17"
        : "+v"(x0), "+v"(y0), "+v"(x1), "+v"(y1), "+v"(x2), "+v"(y2), "+v"(x3), "+v"(y3),
          "+v"(x4), "+v"(y4), "+v"(x5), "+v"(y5), "+v"(x6), "+v"(y6), "+v"(x7), "+v"(y7),
          "+v"(x8), "+v"(y8));
    // Lanes 0-31: entry A's half sums of value i; lanes 32-63: entry B's.
    float p0 = x0 + y0, p1 = x1 + y1, p2 = x2 + y2, p3 = x3 + y3, p4 = x4 + y4;
    float p5 = x5 + y5, p6 = x6 + y6, p7 = x7 + y7, p8 = x8 + y8;
    float z = 0.0f;
    asm volatile(
        "s_nop 1\n\t"
        "v_permlane16_swap_b32 %0, %1\n\t"
        "v_permlane16_swap_b32 %2, %3\n\t"
        "v_permlane16_swap_b32 %4, %5\n\t"
        "v_permlane16_swap_b32 %6, %7\n\t"
        "v_permlane16_swap_b32 %8, %9"
        : "+v"(p0), "+v"(p1), "+v"(p2), "+v"(p3), "+v"(p4), "+v"(p5), "+v"(p6), "+v"(p7),
          "+v"(p8), "+v"(z));
    // Row (bit 4) r of q_m: value 2m + r (q4: value 8, padding).
    const float q0 = p0 + p1, q1 = p2 + p3, q2 = p4 + p5, q3 = p6 + p7, q4 = p8 + z;
    const bool b3 = lane & 8, b2 = lane & 4, b1 = lane & 2;
    const float r0 = (b3 ? q1 : q0) + dpp_f<0x128>(b3 ? q0 : q1);   // row_ror:8
    const float r1 = (b3 ? q3 : q2) + dpp_f<0x128>(b3 ? q2 : q3);
    const float r2 = q4 + dpp_f<0x128>(q4);
    const float s0 = (b2 ? r1 : r0) + dpp_f<0x141>(b2 ? r0 : r1);   // row_half_mirror
    const float s1 = r2 + dpp_f<0x141>(r2);
    const float t = (b1 ? s1 : s0) + dpp_f<0x4E>(b1 ? s0 : s1);     // quad_perm 2,3,0,1
    return t + dpp_f<0xB1>(t);                                       // quad_perm 1,0,3,2
}

// S.grad rows are padded by one float: the deposits and the flush touch the
// ten slots of one entry together, which then fall in distinct LDS banks.
constexpr int kGradStride = kBatch + 1;

template <int MAXW>
struct StageBwd : Stage<MAXW> {
    float grad[kGradSlots][kGradStride];   // per batch entry, summed over waves
};

// One list entry's record, gathered from the per-Gaussian arrays.
struct Rec {
    float4 geo;   // u, v, opacity
    float4 con;   // conic a, b, c
    float4 col;   // r, g, b
    int32_t id;
};

__device__ __forceinline__ Rec gather_rec(const RasterArgs &A, int g) {
    Rec r;
    r.id = g;
    r.geo = make_float4(A.uv[2 * g], A.uv[2 * g + 1], A.opac[g], 0.f);
    r.con = make_float4(A.conic[3 * g], A.conic[3 * g + 1], A.conic[3 * g + 2], 0.f);
    r.col = make_float4(A.color[3 * g], A.color[3 * g + 1], A.color[3 * g + 2], 0.f);
    return r;
}

// Writes entry t's record to LDS with its per-wave cull bits.
template <class S_>
__device__ __forceinline__ void put_rec(S_ &S, int t, const Rec &r, int nwaves) {
    S.geo[t] = r.geo;
    S.con[t] = scale_conic(r.con);
    S.col[t] = r.col;
    S.id[t] = r.id;
    const float thr = 2.0f * __logf(fmaxf(255.0f * r.geo.z, 1.0f));
    const float thr_m = thr * 1.0001f + 1e-4f;
    uint32_t m = 0;
    const float ca = fmaxf(r.con.x, 1e-12f), cc = fmaxf(r.con.z, 1e-12f);
    const float ia = __builtin_amdgcn_rcpf(ca), ic = __builtin_amdgcn_rcpf(cc);
    for (int w = 0; w < nwaves; ++w) {
        const float4 q = S.rect[w];
        if (q.x <= q.y &&
            rect_min_q(r.geo.x, r.geo.y, ca, r.con.y, cc, ia, ic, q.x, q.y, q.z, q.w) < thr_m)
            m |= 1u << w;
    }
    S.live[t] = m;
}

template <class S_>
__device__ __forceinline__ void stage_batch(S_ &S, const RasterArgs &A, int base, int n,
                                            int nwaves) {
    for (int t = threadIdx.x; t < n; t += blockDim.x)
        put_rec(S, t, gather_rec(A, A.ids[base + t]), nwaves);
}

// Forces the values to have arrived (the compiler waits for their loads
// here rather than at a first use inside a loop).
__device__ __forceinline__ void settle(float a, float b, float c, float d) {
    asm volatile("" ::"v"(a), "v"(b), "v"(c), "v"(d));
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

// ------------------------------------------------- chunked backward plan
// The backward walks a tile's list back to front, so a tile is one long
// dependent chain and the longest list bounds the whole kernel. With a chunk
// workspace the forward records, every kChunk list entries, each pixel's
// transmittance and accumulated colour (a checkpoint at the chunk's end), and
// the backward runs one workgroup per (tile, chunk): it starts from the
// chunk's end checkpoint, takes the colour behind it as final minus prefix,
// and walks only its kChunk entries. Each entry still belongs to exactly one
// workgroup, so the gradient atomics are unchanged.
constexpr int kChunk = 2 * kBatch;   // entries per backward unit

struct ChunkPlan {
    int32_t *base;        // n_tiles + 1: first unit of each tile; base[n_tiles] = units
    int32_t *unit_tile;   // unit -> tile
    float4 *ckpt;         // unit * tile^2 + pixel: (T, r, g, b) at the chunk's end
    int32_t cap;          // units the workspace holds
};

inline int64_t chunk_units_cap(int64_t n_isect, int n_tiles) {
    return (n_isect + kChunk - 1) / kChunk + n_tiles;
}

inline int64_t chunk_ws_bytes(int64_t n_isect, int n_tiles, int tile) {
    const int64_t cap = chunk_units_cap(n_isect, n_tiles);
    return align256(4 * ((int64_t)n_tiles + 1)) + align256(4 * cap) +
           cap * (int64_t)tile * tile * (int64_t)sizeof(float4);
}

inline ChunkPlan chunk_plan_of(void *ws, int64_t n_isect, int n_tiles) {
    char *p = static_cast<char *>(ws);
    const int64_t cap = chunk_units_cap(n_isect, n_tiles);
    ChunkPlan P;
    P.base = (int32_t *)p;
    P.unit_tile = (int32_t *)(p + align256(4 * ((int64_t)n_tiles + 1)));
    P.ckpt = (float4 *)(p + align256(4 * ((int64_t)n_tiles + 1)) + align256(4 * cap));
    P.cap = (int32_t)cap;
    return P;
}

// One workgroup: units per tile ceil(len / kChunk), their exclusive scan into
// base, and unit_tile.
__global__ __launch_bounds__(1024) void chunk_plan_kernel(const int32_t *offsets, int n_tiles,
                                                          ChunkPlan P) {
    __shared__ int32_t s_w[16];
    __shared__ int32_t s_carry;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (threadIdx.x == 0) s_carry = 0;
    __syncthreads();
    for (int t0 = 0; t0 < n_tiles; t0 += 1024) {
        const int t = t0 + (int)threadIdx.x;
        const int len = t < n_tiles ? offsets[t + 1] - offsets[t] : 0;
        const int nck = (len + kChunk - 1) / kChunk;
        int incl = nck;
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o, 64);
            if (lane >= o) incl += v;
        }
        if (lane == 63) s_w[wave] = incl;
        __syncthreads();
        int before = s_carry;
        for (int w = 0; w < wave; ++w) before += s_w[w];
        const int b = before + incl - nck;
        if (t < n_tiles) {
            P.base[t] = b;
            for (int k = 0; k < nck; ++k) P.unit_tile[b + k] = t;
        }
        __syncthreads();
        if (threadIdx.x == 1023) s_carry = b + nck;
        __syncthreads();
    }
    if (threadIdx.x == 0) P.base[n_tiles] = s_carry;
}

// ------------------------------------------------- backward tile schedule
// A backward workgroup lives about as long as its tile's walk, which runs
// from the tile's largest stop index back to its first entry, and it runs no
// faster when the CU empties around it: per-workgroup wall-clock stamps at
// config 4 showed lives of 71 us on average (p90 96, longest 140-220 us),
// and walks that started late with long tiles left the GPU draining, less
// than fully occupied, for the last 90 us of a 212-262 us kernel. So the
// forward records each tile's walk length (work) and, before the backward,
// one workgroup per XCD orders the tiles that tile_of_block deals that XCD,
// longest walk first; the backward's workgroup b takes the (b / kXcds)-th
// tile of XCD b % kXcds's list. Each XCD runs the same tiles as without the
// schedule (and keeps their L2 reuse); only the order changes, as in
// longest-processing-time-first scheduling.
//
// The buffer holds 2 * grid ints: the forward's workgroup b writes its
// tile's walk length at [b] (-1 without a tile), the backward's order kernel
// the tile for workgroup b at [grid + b] (-1: none).
constexpr int kOrderThreads = 1024;   // most tiles an XCD's list may hold
constexpr int kOrderBins = 1024;

inline int64_t sched_ints(int grid) { return 2 * (int64_t)grid; }
inline bool sched_fits(int grid) { return (grid + kXcds - 1) / kXcds <= kOrderThreads; }

// Counting-sort bin of a walk length: exact below 768 entries, 32 entries a
// bin above, the last bin from 8928 up. A higher bin is a longer walk.
__device__ __forceinline__ int order_bin(int w) {
    return w < 768 ? w : min(kOrderBins - 1, 768 + ((w - 768) >> 5));
}

// One workgroup per XCD: a counting sort of its list by bin, longest first.
// Tiles of one bin are placed in the order their LDS atomics land.
__global__ __launch_bounds__(kOrderThreads) void tile_order_kernel(const int32_t *work,
                                                                   int32_t *order, int grid,
                                                                   int tiles_x, int tiles_y) {
    __shared__ uint32_t s_cnt[kOrderBins];
    __shared__ uint32_t s_wave[kOrderThreads / 64];
    const int x = blockIdx.x, j = threadIdx.x, lane = j & 63, wave = j >> 6;
    const int K = (grid - x + kXcds - 1) / kXcds;   // blocks x, x + kXcds, ... below grid
    // Which slots hold a tile comes from the dealing itself, so a buffer the
    // forward did not fill can only reorder the tiles, never drop one.
    const int tb = j < K ? tile_of_block(x + kXcds * j, tiles_x, tiles_y) : -1;
    const int w = tb >= 0 ? max(work[x + kXcds * j], 0) : -1;
    for (int i = j; i < kOrderBins; i += kOrderThreads) s_cnt[i] = 0;
    __syncthreads();
    const int q = w >= 0 ? order_bin(w) : 0;
    uint32_t in_bin = 0;
    if (w >= 0) in_bin = atomicAdd(&s_cnt[q], 1u);
    __syncthreads();
    // Thread i scans bin kOrderBins - 1 - i: exclusive starts, longest first.
    const uint32_t c = s_cnt[kOrderBins - 1 - j];
    uint32_t incl = c;
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t u = (uint32_t)__shfl_up((int)incl, o, 64);
        if (lane >= o) incl += u;
    }
    if (lane == 63) s_wave[wave] = incl;
    __syncthreads();
    uint32_t before = 0, total = 0;
    for (int v = 0; v < kOrderThreads / 64; ++v) {
        const uint32_t s = s_wave[v];
        if (v < wave) before += s;
        total += s;
    }
    s_cnt[kOrderBins - 1 - j] = before + incl - c;
    __syncthreads();
    if (w >= 0) order[x + kXcds * (int)(s_cnt[q] + in_bin)] = tb;
    if (j < K && (uint32_t)j >= total) order[x + kXcds * j] = -1;
}

// Eight waves per SIMD (at most 64 VGPRs; 62 without spills): eight
// workgroups share a CU (LDS allows nine), so config 4's 2500 tiles take
// 1.22 rounds of workgroups instead of 1.63 at 73 VGPRs (step -2.5 us).
template <int MAXW>
__global__ __launch_bounds__(MAXW * 64) __attribute__((amdgpu_waves_per_eu(8))) void raster_fwd_kernel(const RasterArgs A, float *out_rgb,
                                                               float *out_alpha, float *out_T,
                                                               int32_t *out_stop,
                                                               const ChunkPlan P) {
    __shared__ Stage<MAXW> S;
    // The gradient records' clearing goes out last: on this GPU a load's
    // wait also waits for every earlier store of the wave.
    auto zero_fill = [&]() {
        if (!A.zero) return;
        // Slices of a multiple of 4 floats: float4 stores, a scalar tail.
        const int64_t per = (((A.zero_n + gridDim.x - 1) / gridDim.x) + 3) & ~(int64_t)3;
        const int64_t b = (int64_t)blockIdx.x * per, e = min(A.zero_n, b + per);
        for (int64_t i = b + 4 * (int64_t)threadIdx.x; i < e; i += 4 * (int64_t)blockDim.x) {
            if (i + 4 <= e)
                *reinterpret_cast<float4 *>(A.zero + i) = make_float4(0.f, 0.f, 0.f, 0.f);
            else
                for (int64_t j = i; j < e; ++j) A.zero[j] = 0.f;
        }
    };
    const int tile_id = tile_of_block(blockIdx.x, A.tiles_x, A.n_tiles / A.tiles_x);
    if (tile_id < 0) {   // whole workgroup
        if (A.work && threadIdx.x == 0) A.work[blockIdx.x] = -1;
        zero_fill();
        return;
    }
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
    // Checkpoints: pixel slot inside the tile, next unit to record.
    const int tile2 = A.tile * A.tile;
    const int pslot = ly * A.tile + lx;
    int unit = P.ckpt ? P.base[tile_id] : 0;
    const int unit_end = P.ckpt ? unit + (end - start + kChunk - 1) / kChunk : 0;

    for (int base = start; base < end; base += kBatch) {
        __syncthreads();
        bool all_done = true;
        for (int w = 0; w < nwaves; ++w) all_done &= S.flag[w] != 0;
        if (all_done) break;                 // the whole tile is opaque
        const int n = min(kBatch, end - base);
        stage_batch(S, A, base, n, nwaves);
        __syncthreads();
        const int cnt = compact_live(S, n, n, wave, lane);
        // Branch-free walk, U entries per round: the records of the round
        // are requested together, each entry updates the pixel with selects
        // (a lane that is done, or outside the splat, adds w = 0 and keeps T:
        // bit for bit what branches give), and the wave checks once per round
        // whether all its pixels are done. The list is read 64 indices at a
        // time into a register and each index taken with a lane read. With a
        // branch per entry the walk issued about as many scalar instructions
        // (exec-mask updates) as vector ones, and the CU's one scalar unit,
        // shared by its four SIMDs, set the pace: 171 us against 117 us here
        // at config 4 (U = 2: 126 us, U = 8: 134 us).
        constexpr int U = 4;
        if (cnt > 0 && ballot(!done) != 0) {
            int lreg = S.list[wave][lane];
            for (int k = 0; k < cnt; k += U) {
                if ((k & 63) == 0 && k) lreg = S.list[wave][k + lane];
                int jj[U];
                float4 gg[U], kk[U], cc[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    // Past the end, the round's last real entry again (masked
                    // below); a scalar min keeps the lane index in scalar registers.
                    const int ku = min(k + u, cnt - 1);
                    jj[u] = __builtin_amdgcn_readlane(lreg, ku & 63);
                    gg[u] = S.geo[jj[u]];
                    kk[u] = S.con[jj[u]];
                    cc[u] = S.col[jj[u]];
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const float dx = fx - gg[u].x, dy = fy - gg[u].y;
                    const float power = splat_power(dx, dy, kk[u]);
                    const float alpha = fminf(kAlphaMax,
                                              gg[u].z * __expf(power));
                    const bool live = (u == 0 || k + u < cnt) && !done && power <= 0.0f &&
                                      alpha >= kAlphaMin;
                    const float w = live ? alpha * T : 0.0f;
                    cr = fmaf(w, cc[u].x, cr);
                    cg = fmaf(w, cc[u].y, cg);
                    cb = fmaf(w, cc[u].z, cb);
                    acc += w;
                    const float Tn = T * (1.0f - alpha);
                    T = live ? Tn : T;
                    stop = live ? base + jj[u] + 1 : stop;
                    done = done || (live && Tn < A.t_min);
                }
                if (ballot(!done) == 0) break;
            }
        }
        const bool wave_done = ballot(!done) == 0;
        if (lane == 0) S.flag[wave] = wave_done ? 1 : 0;
        const int bend = min(base + kBatch, end);
        if (unit < unit_end && ((bend - start) % kChunk == 0 || bend == end)) {
            if (inimg) P.ckpt[(int64_t)unit * tile2 + pslot] = make_float4(T, cr, cg, cb);
            ++unit;
        }
    }
    if (A.work) {
        // The backward's walk over this tile starts at its largest stop
        // index (pixels outside the image keep stop = start).
        __shared__ int32_t s_wmax[MAXW];
        const int wm = wave_max_i(stop);
        if (lane == 0) s_wmax[wave] = wm;
        __syncthreads();
        if (threadIdx.x == 0) {
            int m = start;
            for (int w = 0; w < nwaves; ++w) m = max(m, s_wmax[w]);
            A.work[blockIdx.x] = m - start;
        }
    }
    // A tile that turned opaque early: its later chunks end in the final state.
    for (; unit < unit_end; ++unit)
        if (inimg) P.ckpt[(int64_t)unit * tile2 + pslot] = make_float4(T, cr, cg, cb);
    zero_fill();
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

// Per-Gaussian gradient record written by the backward (kRecFloats floats):
// d_u, d_v, d_conic (a, b, c), d_opacity, d_colour (r, g, b), and the sum
// over pixels of |d_uv| (absgrad).
constexpr int kRecFloats = 10;

struct RasterGrads {
    const float *final_T;
    const int32_t *stop;
    const float *grad_rgb, *grad_alpha;
    const float *alpha;   // the forward's alpha; read only with a background
    float *rec;           // N x kRecFloats
};

template <int MAXW, bool ABS, bool PIPE>
__global__ __launch_bounds__(MAXW * 64) void raster_bwd_kernel(const RasterArgs A,
                                                               const RasterGrads G,
                                                               const ChunkPlan P) {
    __shared__ StageBwd<MAXW> S;
    // Without a plan a workgroup takes a whole tile; with one, one chunk.
    int tile_id, chunk = 0, tile_start, tile_end;
    if (P.ckpt) {
        // Range checks keep a workspace that did not come from the forward
        // from indexing outside it (the whole workgroup returns).
        const int u = (int)blockIdx.x;
        if (u >= min(P.base[A.n_tiles], P.cap)) return;
        tile_id = P.unit_tile[u];
        if (tile_id < 0 || tile_id >= A.n_tiles) return;
        chunk = u - P.base[tile_id];
        tile_start = A.offsets[tile_id];
        tile_end = A.offsets[tile_id + 1];
        const int nck = (tile_end - tile_start + kChunk - 1) / kChunk;
        if (chunk < 0 || chunk >= nck || P.base[tile_id] + nck > P.cap) return;
    } else {
        tile_id = A.order ? A.order[blockIdx.x]
                          : tile_of_block(blockIdx.x, A.tiles_x, A.n_tiles / A.tiles_x);
        if (tile_id < 0 || tile_id >= A.n_tiles) return;
        tile_start = A.offsets[tile_id];
        tile_end = A.offsets[tile_id + 1];
    }
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

    const int start = tile_start + chunk * kChunk;   // this workgroup's entries
    const int cend = P.ckpt ? min(start + kChunk, tile_end) : tile_end;
    const int64_t o = inimg ? (int64_t)py * A.W + px : 0;
    // The pixel's inputs are loaded unconditionally (o is 0 outside the
    // image; an absent optional input reads final_T instead) and selected
    // after: a load in a conditional arm becomes a branch that waits for it
    // before the next load is issued.
    const int stop_o = G.stop[o];
    const float gr_o = G.grad_rgb[3 * o], gg_o = G.grad_rgb[3 * o + 1];
    const float gb_o = G.grad_rgb[3 * o + 2];
    const float ga_o = (G.grad_alpha ? G.grad_alpha : G.final_T)[o];
    const float alpha_o = (A.has_bg ? G.alpha : G.final_T)[o];
    const float T_o = G.final_T[o];
    const int my_stop = inimg ? min(stop_o, cend) : start;
    const float gr = inimg ? gr_o : 0.f;
    const float gg = inimg ? gg_o : 0.f;
    const float gb = inimg ? gb_o : 0.f;
    float ga = inimg && G.grad_alpha ? ga_o : 0.f;
    // The background blend's share: d rgb_out / d alpha = -bg where
    // 1 - alpha >= 0 (torch's clamp_min passes the gradient at the bound).
    if (A.has_bg && inimg && 1.0f - alpha_o >= 0.0f)
        ga -= gr * A.bg[0] + gg * A.bg[1] + gb * A.bg[2];
    float T = inimg ? T_o : 1.0f;
    // Gs = gr sr + gg sg + gb sb + ga sa over the colour (sr, sg, sb) and
    // coverage sa composited behind the current entry. With a chunk plan the
    // walk starts at the chunk's end: colour behind = final - prefix there,
    // coverage behind = T_end - T_final.
    float Gs = 0.f;
    if (P.ckpt && inimg) {
        const int tile2 = A.tile * A.tile, pslot = ly * A.tile + lx;
        const int u0 = P.base[tile_id];
        const int nck = (tile_end - tile_start + kChunk - 1) / kChunk;
        const float4 e = P.ckpt[(int64_t)(u0 + chunk) * tile2 + pslot];
        const float4 f = P.ckpt[(int64_t)(u0 + nck - 1) * tile2 + pslot];
        T = e.x;
        Gs = gr * (f.y - e.y) + gg * (f.z - e.z) + gb * (f.w - e.w) + ga * (e.x - f.x);
    }

    // Nothing at or past a pixel's stop index contributed to it.
    const int wstop = wave_max_i(my_stop);
    if (lane == 0) S.flag[wave] = wstop;
    __syncthreads();
    int bstop = start;
    for (int w = 0; w < nwaves; ++w) bstop = max(bstop, S.flag[w]);

    // One list entry's update of the pixel; v gets the pixel's share of the
    // entry's sums (zeros where it is not active). Returns whether it is.
    auto update = [&](const int i, const float4 geo, const float4 con, const float4 col,
                      float v[kGradSlots]) {
        const float dx = fx - geo.x, dy = fy - geo.y;
        const float power = splat_power(dx, dy, con);
        const float gauss = __expf(power);
        const float op = geo.z;
        const float alpha_raw = op * gauss;
        const float alpha = fminf(kAlphaMax, alpha_raw);
        const bool active = inimg && i < my_stop && power <= 0.0f && alpha >= kAlphaMin;
        // Branchless: inactive lanes compute on finite values and select
        // zeros (never multiply by 0, which would keep an inf as NaN); T and
        // Gs keep their values. T before this entry is recovered as
        // T / (1 - alpha) with a 1-ulp reciprocal; the forward's rounding of
        // T (1 - alpha) already makes the recovery approximate.
        // alpha <= 0.999 (fminf returns 0.999 for a NaN product too), so
        // 1 - alpha >= 0.001 needs no lower clamp.
        const float om = 1.0f - alpha;
        const float iom = __builtin_amdgcn_rcpf(om);
        const float gc = fmaf(gb, col.z, fmaf(gg, col.y, fmaf(gr, col.x, ga)));
        const float dal = (T * gc - Gs) * iom;
        const float Tn = T * iom;
        const float w = active ? alpha * Tn : 0.0f;
        T = active ? Tn : T;
        Gs = fmaf(w, gc, Gs);
        // Past the 0.999 clamp alpha no longer depends on the splat.
        const float dg = active && alpha_raw <= kAlphaMax ? dal * gauss : 0.0f;
        v[0] = w * gr;
        v[1] = w * gg;
        v[2] = w * gb;
        const float mx = dg * dx, my = dg * dy;
        v[3] = mx;
        v[4] = my;
        v[5] = mx * dx;
        v[6] = mx * dy;
        v[7] = my * dy;
        v[8] = dg;
        if (ABS) {
            // |d uv| of this pixel over op: |dg| |(a dx + b dy, b dx + c dy)|.
            const float3 kc = raw_conic(con);
            const float ex = fmaf(kc.x, dx, kc.y * dy), ey = fmaf(kc.y, dx, kc.z * dy);
            v[9] = fabsf(dg) * __builtin_amdgcn_sqrtf(fmaf(ex, ex, ey * ey));
        } else {
            v[9] = 0.0f;
        }
        return active;
    };

    // One list entry: the pixel's update and the wave's sums into S.grad.
    auto entry = [&](const int j, const int i, const float4 geo, const float4 con,
                     const float4 col) {
        float v[kGradSlots];
        // With no lane active the update leaves T and Gs as they were.
        if (ballot(update(i, geo, con, col, v)) == 0) return;
        // Sums over the wave of v[0..9], deposited into S.grad[.][j] with
        // four lanes per LDS atomic (see reduce10_to_rows).
        float q0, q1, q2;
        reduce10_to_rows(v, q0, q1, q2);
        if ((lane & 15) == 0) {
            const int row = lane >> 4;
            // Row r of q0 holds slot {0,2,1,3}[r], of q1 {4,6,5,7}[r], of
            // q2 {8,0,9,0}[r]: rows 1 and 3 of q2 are sums of zeros and add
            // nothing, so all four lanes deposit it (to slots 8, 8, 9, 9; a
            // lane-dependent address, which the compiler does not turn into
            // a wave-aggregation loop as it does a single lane's).
            const int s0 = (row & 1) * 2 + (row >> 1);
            atomicAdd(&S.grad[s0][j], q0);
            atomicAdd(&S.grad[4 + s0][j], q1);
            atomicAdd(&S.grad[8 + (row >> 1)][j], q2);
        }
    };

    // Two consecutive entries (back to front: a, then b), their eighteen
    // sums in one reduction and one LDS atomic per sum (without |d uv|).
    const int slot18 = reduce18_slot(lane);
    auto entry2 = [&](const int ja, const float4 geo_a, const float4 con_a, const float4 col_a,
                      const int jb, const float4 geo_b, const float4 con_b,
                      const float4 col_b, const int base) {
        float va[kGradSlots], vb[kGradSlots];
        const bool act_a = update(base + ja, geo_a, con_a, col_a, va);
        const bool act_b = update(base + jb, geo_b, con_b, col_b, vb);
        if (ballot(act_a || act_b) == 0) return;
        const float sum = reduce18(va, vb, lane);
        if (slot18 >= 0) atomicAdd(&S.grad[slot18][(lane & 32) ? jb : ja], sum);
    };

    // After a batch's walk, entry e's sums become its gradient record slots,
    // in place in S.grad: d_uv = op (a Sx + b Sy, b Sx + c Sy), d_conic =
    // -op (Sxx / 2, Sxy, Syy / 2), d_op = S1, d_col, and |d_uv| = op Sabs.
    auto take = [&](const int e) {
        float s[kGradSlots];
#pragma unroll
        for (int q = 0; q < kGradSlots; ++q) s[q] = S.grad[q][e];
        const float op = S.geo[e].z;
        const float3 con = raw_conic(S.con[e]);
        S.grad[0][e] = op * fmaf(con.x, s[3], con.y * s[4]);
        S.grad[1][e] = op * fmaf(con.y, s[3], con.z * s[4]);
        S.grad[2][e] = -0.5f * op * s[5];
        S.grad[3][e] = -op * s[6];
        S.grad[4][e] = -0.5f * op * s[7];
        S.grad[5][e] = s[8];
        S.grad[6][e] = s[0];
        S.grad[7][e] = s[1];
        S.grad[8][e] = s[2];
        S.grad[9][e] = op * s[9];
    };
    // The workgroup's atomics, (entry, slot)-major: consecutive lanes hit
    // consecutive slots of one record.
    auto flush = [&](const int n) {
        constexpr int V = ABS ? 10 : 9;
        for (int idx = (int)threadIdx.x; idx < V * n; idx += (int)blockDim.x) {
            const int e = idx / V, v = idx - V * e;
            const float val = S.grad[v][e];
            if (val != 0.f) unsafeAtomicAdd(G.rec + (int64_t)kRecFloats * S.id[e] + v, val);
        }
    };

    // PIPE (one batch entry per thread): while a batch is walked, the next
    // batch's records are gathered and the ids of the one after are loaded.
    const int t = threadIdx.x;
    Rec rec{};
    int nid = 0;
    const int nbatch = (bstop - start + kBatch - 1) / kBatch;
    if (PIPE && nbatch > 0) {
        const int b0 = start + (nbatch - 1) * kBatch;
        if (t < bstop - b0) rec = gather_rec(A, A.ids[b0 + t]);
        if (nbatch > 1 && t < kBatch) nid = A.ids[b0 - kBatch + t];
    }
    // The pixel's own inputs have arrived before the first walk.
    settle(gr, gg, gb, ga);
    settle(T, Gs, __int_as_float(my_stop), fx);
    for (int bi = nbatch - 1; bi >= 0; --bi) {
        const int base = start + bi * kBatch;
        const int n = min(kBatch, bstop - base);
        __syncthreads();   // the previous batch's flush has read S.grad and S.id
        if (PIPE) {
            if (t < n) put_rec(S, t, rec, nwaves);
        } else {
            stage_batch(S, A, base, n, nwaves);
        }
        for (int q = t; q < kGradSlots * kGradStride; q += blockDim.x) (&S.grad[0][0])[q] = 0.f;
        __syncthreads();
        if (PIPE) {
            // Batches below the first are full.
            if (bi > 0 && t < kBatch) rec = gather_rec(A, nid);
            if (bi > 1 && t < kBatch) nid = A.ids[base - 2 * kBatch + t];
        }
        const int cnt = compact_live(S, n, wstop - base, wave, lane);
        // Walk the wave's list back to front, two entries per iteration with
        // the records of the next entry read before this one's math. The
        // list is read 64 indices at a time into a register and the entry's
        // index taken from it with a lane read, so it is wave-uniform.
        if (cnt > 0 && !ABS) {
            // Entries k and k - 1 share one reduction; entry k - 2's records
            // are read before their math. Two pairs per iteration, so the
            // read-ahead record alternates between the a and c registers.
            int k = cnt - 1;
            int lreg = S.list[wave][(k & ~63) + lane];
            int ja = __builtin_amdgcn_readlane(lreg, k & 63), jc;
            float4 geo_a = S.geo[ja], con_a = S.con[ja], col_a = S.col[ja];
            float4 geo_c, con_c, col_c;
            // Entry k - 1 into (jx, x) and entry max(k - 2, 0) into (jy, y).
            auto read2 = [&](int &jx, float4 &gx, float4 &kx, float4 &cx, int &jy, float4 &gy,
                             float4 &ky, float4 &cy) {
                const int kb = k - 1;
                if ((kb & 63) == 63) lreg = S.list[wave][(kb & ~63) + lane];
                jx = __builtin_amdgcn_readlane(lreg, kb & 63);
                gx = S.geo[jx];
                kx = S.con[jx];
                cx = S.col[jx];
                const int kc = max(k - 2, 0);
                if ((kc & 63) == 63) lreg = S.list[wave][(kc & ~63) + lane];
                jy = __builtin_amdgcn_readlane(lreg, kc & 63);
                gy = S.geo[jy];
                ky = S.con[jy];
                cy = S.col[jy];
            };
            for (;;) {
                if (k == 0) {
                    entry(ja, base + ja, geo_a, con_a, col_a);
                    break;
                }
                {
                    int jb;
                    float4 geo_b, con_b, col_b;
                    read2(jb, geo_b, con_b, col_b, jc, geo_c, con_c, col_c);
                    entry2(ja, geo_a, con_a, col_a, jb, geo_b, con_b, col_b, base);
                }
                k -= 2;
                if (k < 0) break;
                if (k == 0) {
                    entry(jc, base + jc, geo_c, con_c, col_c);
                    break;
                }
                {
                    int jd;
                    float4 geo_d, con_d, col_d;
                    read2(jd, geo_d, con_d, col_d, ja, geo_a, con_a, col_a);
                    entry2(jc, geo_c, con_c, col_c, jd, geo_d, con_d, col_d, base);
                }
                k -= 2;
                if (k < 0) break;
            }
        } else if (cnt > 0) {
            int k = cnt - 1;
            int lreg = S.list[wave][(k & ~63) + lane];
            int ja = __builtin_amdgcn_readlane(lreg, k & 63);
            float4 geo_a = S.geo[ja], con_a = S.con[ja], col_a = S.col[ja];
            for (;;) {
                // Entry k - 1 (or k again at the end) into the b registers.
                const int kb = max(k - 1, 0);
                if ((kb & 63) == 63) lreg = S.list[wave][(kb & ~63) + lane];
                const int jb = __builtin_amdgcn_readlane(lreg, kb & 63);
                const float4 geo_b = S.geo[jb], con_b = S.con[jb], col_b = S.col[jb];
                entry(ja, base + ja, geo_a, con_a, col_a);
                if (--k < 0) break;
                const int kc = max(k - 1, 0);
                if ((kc & 63) == 63) lreg = S.list[wave][(kc & ~63) + lane];
                ja = __builtin_amdgcn_readlane(lreg, kc & 63);
                geo_a = S.geo[ja];
                con_a = S.con[ja];
                col_a = S.col[ja];
                entry(jb, base + jb, geo_b, con_b, col_b);
                if (--k < 0) break;
            }
        }
        __syncthreads();
        for (int e = t; e < n; e += blockDim.x) take(e);
        __syncthreads();
        flush(n);
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

int64_t mg_rasterize_chunk_workspace_bytes(int64_t n_isect, int32_t n_tiles, int32_t tile) {
    if (n_isect < 0 || n_tiles < 1 || tile < 1) return 0;
    return chunk_ws_bytes(n_isect, n_tiles, tile);
}

int64_t mg_rasterize_sched_ints(int32_t W, int32_t H, int32_t tile) {
    if (W < 1 || H < 1 || tile < 1) return 0;
    const int tiles_x = (W + tile - 1) / tile, tiles_y = (H + tile - 1) / tile;
    return sched_ints(raster_grid(tiles_x, tiles_y));
}

int32_t mg_rasterize_forward(int64_t N, const float *uv, const float *conic, const float *opacity,
                             const float *color, const int32_t *gauss_ids,
                             const int32_t *tile_offsets, int32_t W, int32_t H, int32_t tile,
                             int32_t tiles_x, float t_min, const float *background,
                             int64_t n_isect, void *chunk_ws, int64_t chunk_ws_size,
                             float *out_rgb, float *out_alpha, float *out_T, int32_t *out_stop,
                             float *zero_grads, int32_t *sched, mg_stream_t stream) {
    int32_t rc = check_raster("rasterize_forward", N, uv, conic, opacity, color, gauss_ids,
                              tile_offsets, W, H, tile, tiles_x);
    if (rc != MG_OK) return rc;
    MG_REQUIRE(out_rgb && out_alpha && out_T && out_stop, "rasterize_forward: null output");
    MG_REQUIRE(zero_grads == nullptr || ((uintptr_t)zero_grads & 15) == 0,
               "rasterize_forward: zero_grads not 16-byte aligned");
    const int tiles_y = (H + tile - 1) / tile;
    RasterArgs A{uv, conic, opacity, color, gauss_ids, tile_offsets, W, H, tile, tiles_x,
                 tiles_x * tiles_y, t_min, background != nullptr,
                 {background ? background[0] : 0.f, background ? background[1] : 0.f,
                  background ? background[2] : 0.f}};
    A.zero = N > 0 ? zero_grads : nullptr;
    A.zero_n = (int64_t)kRecFloats * N;
    A.work = sched;
    hipStream_t s = as_stream(stream);
    ChunkPlan P{nullptr, nullptr, nullptr, 0};
    if (chunk_ws) {
        MG_REQUIRE(n_isect >= 0 && chunk_ws_size >= chunk_ws_bytes(n_isect, A.n_tiles, tile),
                   "rasterize_forward: chunk workspace %lld bytes, need %lld for %lld "
                   "intersections", (long long)chunk_ws_size,
                   (long long)chunk_ws_bytes(n_isect, A.n_tiles, tile), (long long)n_isect);
        P = chunk_plan_of(chunk_ws, n_isect, A.n_tiles);
        chunk_plan_kernel<<<1, 1024, 0, s>>>(tile_offsets, A.n_tiles, P);
        MG_LAUNCHED("chunk_plan_kernel");
    }
    const int threads = ((tile * tile + 63) / 64) * 64;
    const int grid = raster_grid(tiles_x, tiles_y);
    TimedScope ts("rasterize_forward", s);
    if (threads <= 4 * 64)
        raster_fwd_kernel<4><<<grid, threads, 0, s>>>(A, out_rgb, out_alpha, out_T, out_stop, P);
    else
        raster_fwd_kernel<kMaxWaves><<<grid, threads, 0, s>>>(A, out_rgb, out_alpha, out_T,
                                                              out_stop, P);
    MG_LAUNCHED("raster_fwd_kernel");
    return MG_OK;
}

int32_t mg_rasterize_backward(int64_t N, const float *uv, const float *conic,
                              const float *opacity, const float *color,
                              const int32_t *gauss_ids, const int32_t *tile_offsets,
                              const float *final_T, const int32_t *stop, const float *grad_rgb,
                              const float *grad_alpha, const float *alpha,
                              const float *background, int64_t n_isect, const void *chunk_ws,
                              int64_t chunk_ws_size, int32_t W, int32_t H, int32_t tile,
                              int32_t tiles_x, float *d_grads, int32_t absgrad,
                              int32_t grads_zeroed, int32_t *sched, mg_stream_t stream) {
    int32_t rc = check_raster("rasterize_backward", N, uv, conic, opacity, color, gauss_ids,
                              tile_offsets, W, H, tile, tiles_x);
    if (rc != MG_OK) return rc;
    MG_REQUIRE(final_T && stop && grad_rgb, "rasterize_backward: null input");
    MG_REQUIRE(!background || alpha, "rasterize_backward: a background needs the forward's alpha");
    MG_REQUIRE(N == 0 || d_grads, "rasterize_backward: null gradient output");
    hipStream_t s = as_stream(stream);
    if (N > 0 && !grads_zeroed) {
        ZeroSpans Z{{d_grads, nullptr, nullptr, nullptr, nullptr},
                    {kRecFloats * N, 0, 0, 0, 0}};
        const int64_t blocks = min(ceil_div(kRecFloats * N, 256), (int64_t)4096);
        zero_spans_kernel<<<(unsigned)blocks, 256, 0, s>>>(Z);
        MG_LAUNCHED("zero_spans_kernel");
    }
    const int tiles_y = (H + tile - 1) / tile;
    RasterArgs A{uv, conic, opacity, color, gauss_ids, tile_offsets, W, H, tile, tiles_x,
                 tiles_x * tiles_y, 0.0f, background != nullptr,
                 {background ? background[0] : 0.f, background ? background[1] : 0.f,
                  background ? background[2] : 0.f}};
    RasterGrads Gr{final_T, stop, grad_rgb, grad_alpha, alpha, d_grads};
    ChunkPlan P{nullptr, nullptr, nullptr, 0};
    int grid = raster_grid(tiles_x, tiles_y);
    if (chunk_ws) {
        // The plan and checkpoints the forward wrote into this workspace.
        MG_REQUIRE(n_isect >= 0 && chunk_ws_size >= chunk_ws_bytes(n_isect, A.n_tiles, tile),
                   "rasterize_backward: chunk workspace %lld bytes, need %lld for %lld "
                   "intersections", (long long)chunk_ws_size,
                   (long long)chunk_ws_bytes(n_isect, A.n_tiles, tile), (long long)n_isect);
        P = chunk_plan_of(const_cast<void *>(chunk_ws), n_isect, A.n_tiles);
        grid = P.cap;
    }
    const int threads = ((tile * tile + 63) / 64) * 64;
    TimedScope ts("rasterize_backward", s);
    if (grid > 0 && sched && !chunk_ws && sched_fits(grid)) {
        int32_t *order = sched + grid;
        tile_order_kernel<<<kXcds, kOrderThreads, 0, s>>>(sched, order, grid, tiles_x, tiles_y);
        MG_LAUNCHED("tile_order_kernel");
        A.order = order;
    }
    if (grid > 0) {
        // One batch entry per thread (tile 16 and up) takes the pipelined
        // batch loop.
        const bool abs = absgrad != 0, pipe = threads >= kBatch;
        if (threads <= 4 * 64) {
            if (pipe) {
                if (abs) raster_bwd_kernel<4, true, true><<<grid, threads, 0, s>>>(A, Gr, P);
                else raster_bwd_kernel<4, false, true><<<grid, threads, 0, s>>>(A, Gr, P);
            } else {
                if (abs) raster_bwd_kernel<4, true, false><<<grid, threads, 0, s>>>(A, Gr, P);
                else raster_bwd_kernel<4, false, false><<<grid, threads, 0, s>>>(A, Gr, P);
            }
        } else {
            if (abs) raster_bwd_kernel<kMaxWaves, true, true><<<grid, threads, 0, s>>>(A, Gr, P);
            else raster_bwd_kernel<kMaxWaves, false, true><<<grid, threads, 0, s>>>(A, Gr, P);
        }
        MG_LAUNCHED("raster_bwd_kernel");
    }
    return MG_OK;
}

}  // extern "C"
