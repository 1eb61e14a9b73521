// Fused projection + EWA 2D covariance + SnugBox extents + SH colour, forward
// and analytic backward. One thread per Gaussian, no atomics.
//
// Follows metal_gauss/torch_ref.py:31-144 (projection, blur 0.3, Jacobian
// clamp at 1.3x the half field of view, 3-sigma radius), sh.py:24-62 (real SH
// basis, degree 0..3, +0.5 and clamp at 0) and preprocess.metal:180-195
// (SnugBox half-extents and the validity test that feeds binning).
//
// Memory: the per-Gaussian inputs are AoS rows (12/16/12/4 bytes plus a 192
// byte SH row). Each kernel runs in two phases over a wave's 64 Gaussians:
//   * projection: one lane per Gaussian; the small rows are contiguous spans
//     of 64 x 12-16 bytes per load instruction;
//   * SH colour: four lanes per Gaussian (a quad), in four rounds of 16
//     Gaussians. Lane q of a quad owns bases 4q..4q+3, i.e. 48 contiguous
//     bytes of the row, so a round reads (and the backward writes) 16 whole
//     rows as 16-byte accesses with no LDS. Partial sums are combined with
//     quad DPP swizzles; per-Gaussian values cross between the phases by wave
//     shuffles. Quads of Gaussians that are not visible skip their row.
// No LDS is used, so occupancy is limited by registers alone.
#include "mg_common.h"

namespace mg {

constexpr int kPreThreads = 256;

// Activations taken inside the projection (train.py:221-222 takes them in
// torch before render): the scales argument holds log scales (exp), the
// opacity argument logits (sigmoid). The effective-opacity kernels only.
constexpr int32_t kActLogScale = 1, kActLogitOpac = 2;

__device__ __forceinline__ float act_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

struct Cam {
    float R[9];      // world->camera rotation, row-major
    float t[3];
    float fx, fy, cx, cy;
    float near_p, far_p, blur, max_r;
    float cc[3];     // camera centre in world space
    int32_t W, H, deg;
};

// Real SH constants (sh.py:11-17), the textbook normalisations.
constexpr float kC0 = 0.28209479177387814f;
constexpr float kC1 = 0.4886025119029199f;
constexpr float kC2[5] = {1.0925484305920792f, -1.0925484305920792f, 0.31539156525252005f,
                          -1.0925484305920792f, 0.5462742152960396f};
constexpr float kC3[7] = {-0.5900435899266435f, 2.890611442640554f, -0.4570457994644658f,
                          0.3731763325901154f, -0.4570457994644658f, 1.445305721320277f,
                          -0.5900435899266435f};

// Basis values for a unit direction (16 entries; only the first (deg+1)^2 are
// meaningful).
__device__ __forceinline__ void sh_basis(int deg, float x, float y, float z, float B[16]) {
    B[0] = kC0;
    if (deg < 1) return;
    B[1] = -kC1 * y;
    B[2] = kC1 * z;
    B[3] = -kC1 * x;
    if (deg < 2) return;
    const float xx = x * x, yy = y * y, zz = z * z;
    B[4] = kC2[0] * x * y;
    B[5] = kC2[1] * y * z;
    B[6] = kC2[2] * (2.0f * zz - xx - yy);
    B[7] = kC2[3] * x * z;
    B[8] = kC2[4] * (xx - yy);
    if (deg < 3) return;
    B[9] = kC3[0] * y * (3.0f * xx - yy);
    B[10] = kC3[1] * x * y * z;
    B[11] = kC3[2] * y * (4.0f * zz - xx - yy);
    B[12] = kC3[3] * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
    B[13] = kC3[4] * x * (4.0f * zz - xx - yy);
    B[14] = kC3[5] * z * (xx - yy);
    B[15] = kC3[6] * x * (xx - 3.0f * yy);
}

// Accumulates sum_b w_b * dB_b/d(x,y,z) into g (the gradient of a weighted sum
// of basis values with respect to the unnormalised-then-normalised direction).
__device__ __forceinline__ void sh_basis_vjp(int deg, float x, float y, float z,
                                             const float w[16], float g[3]) {
    g[0] = g[1] = g[2] = 0.f;
    if (deg < 1) return;
    g[1] += -kC1 * w[1];
    g[2] += kC1 * w[2];
    g[0] += -kC1 * w[3];
    if (deg < 2) return;
    const float xx = x * x, yy = y * y, zz = z * z;
    // B4 = c xy ; B5 = c yz ; B6 = c (2zz - xx - yy) ; B7 = c xz ; B8 = c (xx - yy)
    g[0] += kC2[0] * y * w[4];
    g[1] += kC2[0] * x * w[4];
    g[1] += kC2[1] * z * w[5];
    g[2] += kC2[1] * y * w[5];
    g[0] += kC2[2] * (-2.0f * x) * w[6];
    g[1] += kC2[2] * (-2.0f * y) * w[6];
    g[2] += kC2[2] * (4.0f * z) * w[6];
    g[0] += kC2[3] * z * w[7];
    g[2] += kC2[3] * x * w[7];
    g[0] += kC2[4] * (2.0f * x) * w[8];
    g[1] += kC2[4] * (-2.0f * y) * w[8];
    if (deg < 3) return;
    // B9 = c y (3xx - yy)
    g[0] += kC3[0] * (6.0f * x * y) * w[9];
    g[1] += kC3[0] * (3.0f * xx - 3.0f * yy) * w[9];
    // B10 = c xyz
    g[0] += kC3[1] * (y * z) * w[10];
    g[1] += kC3[1] * (x * z) * w[10];
    g[2] += kC3[1] * (x * y) * w[10];
    // B11 = c y (4zz - xx - yy)
    g[0] += kC3[2] * (-2.0f * x * y) * w[11];
    g[1] += kC3[2] * (4.0f * zz - xx - 3.0f * yy) * w[11];
    g[2] += kC3[2] * (8.0f * y * z) * w[11];
    // B12 = c z (2zz - 3xx - 3yy)
    g[0] += kC3[3] * (-6.0f * x * z) * w[12];
    g[1] += kC3[3] * (-6.0f * y * z) * w[12];
    g[2] += kC3[3] * (6.0f * zz - 3.0f * xx - 3.0f * yy) * w[12];
    // B13 = c x (4zz - xx - yy)
    g[0] += kC3[4] * (4.0f * zz - 3.0f * xx - yy) * w[13];
    g[1] += kC3[4] * (-2.0f * x * y) * w[13];
    g[2] += kC3[4] * (8.0f * x * z) * w[13];
    // B14 = c z (xx - yy)
    g[0] += kC3[5] * (2.0f * x * z) * w[14];
    g[1] += kC3[5] * (-2.0f * y * z) * w[14];
    g[2] += kC3[5] * (xx - yy) * w[14];
    // B15 = c x (xx - 3yy)
    g[0] += kC3[6] * (3.0f * xx - 3.0f * yy) * w[15];
    g[1] += kC3[6] * (-6.0f * x * y) * w[15];
}

// Everything the forward derives from one Gaussian, kept so the backward can
// re-derive it identically.
struct Proj {
    float p[3];          // camera-space centre
    float zc, izc;
    bool clx, cly;       // Jacobian evaluation point clamped in x / y
    float tx, ty;        // clamped evaluation point
    float qn;            // |q|
    float q[4];          // normalised wxyz
    float R[9];          // rotation of the Gaussian, row-major
    float s[3];
    float M[9];          // R diag(s)
    float S[6];          // Sigma = M M^T: xx xy xz yy yz zz
    float T0[3], T1[3];  // rows of J * Rw
    float a0, c0;        // diagonal of the undilated 2D covariance
    float a, b, c;       // dilated 2D covariance
};

__device__ __forceinline__ void project(const Cam &C, float mx, float my, float mz,
                                        const float qin[4], const float sin_[3], Proj &P) {
    P.p[0] = C.R[0] * mx + C.R[1] * my + C.R[2] * mz + C.t[0];
    P.p[1] = C.R[3] * mx + C.R[4] * my + C.R[5] * mz + C.t[1];
    P.p[2] = C.R[6] * mx + C.R[7] * my + C.R[8] * mz + C.t[2];
    P.zc = fmaxf(P.p[2], C.near_p);
    P.izc = 1.0f / P.zc;

    const float lim_x = 1.3f * (0.5f * (float)C.W / C.fx);
    const float lim_y = 1.3f * (0.5f * (float)C.H / C.fy);
    const float txn = P.p[0] / P.zc, tyn = P.p[1] / P.zc;
    P.clx = (txn < -lim_x) || (txn > lim_x);
    P.cly = (tyn < -lim_y) || (tyn > lim_y);
    P.tx = fminf(fmaxf(txn, -lim_x), lim_x) * P.zc;
    P.ty = fminf(fmaxf(tyn, -lim_y), lim_y) * P.zc;

    const float qn = sqrtf(qin[0] * qin[0] + qin[1] * qin[1] + qin[2] * qin[2] + qin[3] * qin[3]);
    P.qn = qn;
    const float iq = 1.0f / fmaxf(qn, 1e-12f);
    const float w = qin[0] * iq, x = qin[1] * iq, y = qin[2] * iq, z = qin[3] * iq;
    P.q[0] = w; P.q[1] = x; P.q[2] = y; P.q[3] = z;
    P.R[0] = 1.f - 2.f * (y * y + z * z); P.R[1] = 2.f * (x * y - w * z); P.R[2] = 2.f * (x * z + w * y);
    P.R[3] = 2.f * (x * y + w * z); P.R[4] = 1.f - 2.f * (x * x + z * z); P.R[5] = 2.f * (y * z - w * x);
    P.R[6] = 2.f * (x * z - w * y); P.R[7] = 2.f * (y * z + w * x); P.R[8] = 1.f - 2.f * (x * x + y * y);
    P.s[0] = sin_[0]; P.s[1] = sin_[1]; P.s[2] = sin_[2];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) P.M[3 * i + j] = P.R[3 * i + j] * P.s[j];
    const float *M = P.M;
    P.S[0] = M[0] * M[0] + M[1] * M[1] + M[2] * M[2];
    P.S[1] = M[0] * M[3] + M[1] * M[4] + M[2] * M[5];
    P.S[2] = M[0] * M[6] + M[1] * M[7] + M[2] * M[8];
    P.S[3] = M[3] * M[3] + M[4] * M[4] + M[5] * M[5];
    P.S[4] = M[3] * M[6] + M[4] * M[7] + M[5] * M[8];
    P.S[5] = M[6] * M[6] + M[7] * M[7] + M[8] * M[8];

    // J rows: (fx/zc, 0, -fx tx/zc^2) and (0, fy/zc, -fy ty/zc^2); T = J Rw.
    const float izc2 = P.izc * P.izc;
    const float j0x = C.fx * P.izc, j0z = -C.fx * P.tx * izc2;
    const float j1y = C.fy * P.izc, j1z = -C.fy * P.ty * izc2;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        P.T0[k] = j0x * C.R[k] + j0z * C.R[6 + k];
        P.T1[k] = j1y * C.R[3 + k] + j1z * C.R[6 + k];
    }
    const float *S = P.S;
    const float s00 = S[0], s01 = S[1], s02 = S[2], s11 = S[3], s12 = S[4], s22 = S[5];
    const float ST0x = s00 * P.T0[0] + s01 * P.T0[1] + s02 * P.T0[2];
    const float ST0y = s01 * P.T0[0] + s11 * P.T0[1] + s12 * P.T0[2];
    const float ST0z = s02 * P.T0[0] + s12 * P.T0[1] + s22 * P.T0[2];
    const float ST1x = s00 * P.T1[0] + s01 * P.T1[1] + s02 * P.T1[2];
    const float ST1y = s01 * P.T1[0] + s11 * P.T1[1] + s12 * P.T1[2];
    const float ST1z = s02 * P.T1[0] + s12 * P.T1[1] + s22 * P.T1[2];
    P.a0 = P.T0[0] * ST0x + P.T0[1] * ST0y + P.T0[2] * ST0z;
    P.b = P.T0[0] * ST1x + P.T0[1] * ST1y + P.T0[2] * ST1z;
    P.c0 = P.T1[0] * ST1x + P.T1[1] * ST1y + P.T1[2] * ST1z;
    P.a = P.a0 + C.blur;
    P.c = P.c0 + C.blur;
}

// ------------------------------------------------------------ mip filters
// Mip-Splatting's two low-pass filters, folded into the projection.
//
// 3D (mipfilter.py:76-93): per-Gaussian filter size f widens every axis,
// s' = sqrt(s^2 + f^2), and dims the Gaussian by
// coef3 = sqrt(clamp(prod s^2 / prod s'^2, 0, 1)) so the total density is
// kept. The covariance is built from s'.
// 2D (torch_ref.py:100-124, metal_backend.py:367-393): the blur added to the
// projected covariance is compensated by coef2 = sqrt(clamp(max(det0, 0) /
// max(det, 1e-12), 0, 1)), det0 and det the determinants before and after the
// blur. The SnugBox extents and the validity test see the opacity after the
// 3D filter and before the 2D one, as the reference's kernel does (it is
// handed the filtered opacity and the antialias factor is applied after it,
// metal_backend.py:498-511); binning and compositing see both.
struct Mip3 {
    float s2[3], s2f[3];   // s^2 and s^2 + f^2
    float coef;            // 1 without a filter
};

__device__ __forceinline__ void mip3_apply(float f, float s[3], Mip3 &M) {
    const float f2 = f * f;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        M.s2[i] = s[i] * s[i];
        M.s2f[i] = M.s2[i] + f2;
        s[i] = sqrtf(M.s2f[i]);
    }
    const float r = (M.s2[0] * M.s2[1] * M.s2[2]) / (M.s2f[0] * M.s2f[1] * M.s2f[2]);
    M.coef = sqrtf(fminf(fmaxf(r, 0.0f), 1.0f));
}

__device__ __forceinline__ float mip2_coef(const Proj &P) {
    const float det0 = P.a0 * P.c0 - P.b * P.b;
    const float det = P.a * P.c - P.b * P.b;
    const float r = fmaxf(det0, 0.0f) / fmaxf(det, 1e-12f);
    return sqrtf(fminf(fmaxf(r, 0.0f), 1.0f));
}

// ------------------------------------------------------------ quad SH phase
// In round r lane L works on the wave's Gaussian 16 r + L / 4, bases
// 4 (L % 4) .. 4 (L % 4) + 3.

// Orders a wave's LDS writes before its following LDS reads (lanes read what
// other lanes of the same wave wrote).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Sum over the four lanes of a quad, in every lane of it.
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    return v;
}

struct ShRows {
    const float *sh, *rest;   // fused (N,16,3) in sh, or DC (N,1,3) + rest (N,15,3)
    int fused, vec4;          // vec4: degree 3 (and, when fused, 16-byte aligned)
};

// 16- and 12-byte accesses that need only 4-byte alignment (gfx9 global
// memory accepts dword-aligned multi-dword accesses): the split layout's
// 180-byte rest rows start on any dword.
typedef float v4u __attribute__((ext_vector_type(4), aligned(4)));
typedef float v3u __attribute__((ext_vector_type(3), aligned(4)));

// Loads coefficients c[k][ch] of bases 4q+k (k < 4) of Gaussian G; bases at
// or past nb read as 0.
__device__ __forceinline__ void load_bases(const ShRows &R, int64_t G, int q, int nb,
                                           float c[4][3]) {
    if (R.vec4 && R.fused) {
        const float4 *src = reinterpret_cast<const float4 *>(R.sh + G * 48 + 12 * q);
        const float4 a = src[0], b = src[1], d = src[2];
        c[0][0] = a.x; c[0][1] = a.y; c[0][2] = a.z;
        c[1][0] = a.w; c[1][1] = b.x; c[1][2] = b.y;
        c[2][0] = b.z; c[2][1] = b.w; c[2][2] = d.x;
        c[3][0] = d.y; c[3][1] = d.z; c[3][2] = d.w;
        return;
    }
    if (R.vec4) {   // split layout, degree 3: the quad reads the 180-byte rest row
        float f[12];
        if (q == 0) {
            const v3u d = *reinterpret_cast<const v3u *>(R.sh + G * 3);
            const float *r = R.rest + G * 45;
            const v4u a = *reinterpret_cast<const v4u *>(r);
            const v4u b = *reinterpret_cast<const v4u *>(r + 4);
            f[0] = d.x; f[1] = d.y; f[2] = d.z;
            f[3] = a.x; f[4] = a.y; f[5] = a.z; f[6] = a.w;
            f[7] = b.x; f[8] = b.y; f[9] = b.z; f[10] = b.w; f[11] = r[8];
        } else {
            const float *r = R.rest + G * 45 + 12 * q - 3;
            const v4u a = *reinterpret_cast<const v4u *>(r);
            const v4u b = *reinterpret_cast<const v4u *>(r + 4);
            const v4u d = *reinterpret_cast<const v4u *>(r + 8);
            f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
            f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
            f[8] = d.x; f[9] = d.y; f[10] = d.z; f[11] = d.w;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int ch = 0; ch < 3; ++ch) c[k][ch] = f[3 * k + ch];
        return;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = 4 * q + k;
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) {
            float v = 0.f;
            if (i < nb) {
                if (R.fused) v = R.sh[G * 48 + 3 * i + ch];
                else v = i == 0 ? R.sh[G * 3 + ch] : R.rest[G * 45 + 3 * (i - 1) + ch];
            }
            c[k][ch] = v;
        }
    }
}

// ------------------------------------------------ SH rows staged through LDS
// A round's 16 consecutive Gaussians G0..G0+15 (G0 a multiple of 16) own one
// contiguous block per SH tensor: 16 x 48 floats fused, or 16 x 3 (DC) plus
// 16 x 45 (rest) split, 768 floats either way, 16-byte aligned when the
// tensors are. Lane l moves float4s l, l + 64, l + 128 of the block (DC
// first when split) between global memory and a 3 KB LDS slice of its wave:
// aligned, fully coalesced 16-byte accesses instead of the quad lanes' own
// dword-aligned 48-byte pieces of the 180-byte rest rows. The quads then read
// and write their bases in the slice.
constexpr int kStageF4 = 192;

// The backward stages both ways; the forward, which only reads the rows,
// measured faster with its own dword-aligned loads (57 vs 60 us at config 4:
// the slice costs it occupancy).
// Row (Gaussian of the round) of float f of the block.
__device__ __forceinline__ int stage_row(int fused, int f) {
    return fused ? f / 48 : (f < 48 ? f / 3 : (f - 48) / 45);
}

// Whether the staged path applies: degree 3 and 16-byte aligned tensors.
__device__ __host__ __forceinline__ bool stage_aligned(const float *a, const float *b, int fused) {
    return ((uintptr_t)a & 15) == 0 && (fused || ((uintptr_t)b & 15) == 0);
}

__device__ __forceinline__ const float *stage_src(const float *sh, const float *rest, int fused,
                                                 int64_t G0, int f) {
    if (fused) return sh + G0 * 48 + f;
    return f < 48 ? sh + G0 * 3 + f : rest + G0 * 45 + (f - 48);
}

__device__ __forceinline__ float *stage_dst(float *sh, float *rest, int fused, int64_t G0,
                                           int f) {
    if (fused) return sh + G0 * 48 + f;
    return f < 48 ? sh + G0 * 3 + f : rest + G0 * 45 + (f - 48);
}

// This lane's three float4s of the round at G0 (ng of its 16 Gaussians exist;
// bit i of need set: Gaussian G0 + i is read). Unread floats are 0.
__device__ __forceinline__ void stage_load(const ShRows &R, int64_t G0, int ng, uint32_t need,
                                           float4 (&pf)[3]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int f = 4 * (lane + 64 * i);
        const int r0 = stage_row(R.fused, f), r3 = stage_row(R.fused, f + 3);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        const bool want = ((need >> r0) & 1u) || (r3 < 16 && ((need >> r3) & 1u));
        if (want && r3 < ng) {
            // The four floats lie in one tensor: block boundaries (48 and the
            // 3- and 45-float rows) never split an aligned float4 across the
            // DC and rest blocks, since 48 is a multiple of 4.
            v = *reinterpret_cast<const float4 *>(stage_src(R.sh, R.rest, R.fused, G0, f));
        } else if (want && r0 < ng) {
            float e[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (stage_row(R.fused, f + k) < ng) e[k] = *stage_src(R.sh, R.rest, R.fused, G0, f + k);
            v = make_float4(e[0], e[1], e[2], e[3]);
        }
        pf[i] = v;
    }
}

__device__ __forceinline__ void stage_put(float4 *sb, const float4 (&pf)[3]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 3; ++i) sb[lane + 64 * i] = pf[i];
}

// Float offset in the slice of base b (0..15), channel 0, of round Gaussian gl.
__device__ __forceinline__ int stage_off(int fused, int gl, int b) {
    if (fused) return gl * 48 + 3 * b;
    return b == 0 ? gl * 3 : 48 + gl * 45 + 3 * (b - 1);
}

// The quad lane's coefficients c[k][ch] of bases 4q+k of round Gaussian gl.
__device__ __forceinline__ void stage_read(const float *sb, int fused, int gl, int q,
                                           float c[4][3]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int o = stage_off(fused, gl, 4 * q + k);
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) c[k][ch] = sb[o + ch];
    }
}

__device__ __forceinline__ void stage_write(float *sb, int fused, int gl, int q,
                                            const float d[4][3]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int o = stage_off(fused, gl, 4 * q + k);
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) sb[o + ch] = d[k][ch];
    }
}

// Stores the slice (the round's d_sh) to the gradient tensors; only the ng
// existing Gaussians' floats are written.
__device__ __forceinline__ void stage_store(const float4 *sb, float *dsh, float *drest, int fused,
                                            int64_t G0, int ng) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int f = 4 * (lane + 64 * i);
        const float4 v = sb[lane + 64 * i];
        if (stage_row(fused, f + 3) < ng) {
            *reinterpret_cast<float4 *>(stage_dst(dsh, drest, fused, G0, f)) = v;
        } else {
            const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (stage_row(fused, f + k) < ng) *stage_dst(dsh, drest, fused, G0, f + k) = e[k];
        }
    }
}

// Stores d[k][ch] as the gradient of bases 4q+k of Gaussian G (all 16 bases
// are written; the caller passes zeros past the degree).
__device__ __forceinline__ void store_bases(float *dsh, float *drest, int fused, int vec4,
                                            int64_t G, int q, const float d[4][3]) {
    if (vec4 && fused) {
        float4 *dst = reinterpret_cast<float4 *>(dsh + G * 48 + 12 * q);
        dst[0] = make_float4(d[0][0], d[0][1], d[0][2], d[1][0]);
        dst[1] = make_float4(d[1][1], d[1][2], d[2][0], d[2][1]);
        dst[2] = make_float4(d[2][2], d[3][0], d[3][1], d[3][2]);
        return;
    }
    if (vec4) {     // split layout (the fused case returned above)
        float f[12];
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int ch = 0; ch < 3; ++ch) f[3 * k + ch] = d[k][ch];
        if (q == 0) {
            *reinterpret_cast<v3u *>(dsh + G * 3) = v3u{f[0], f[1], f[2]};
            float *r = drest + G * 45;
            *reinterpret_cast<v4u *>(r) = v4u{f[3], f[4], f[5], f[6]};
            *reinterpret_cast<v4u *>(r + 4) = v4u{f[7], f[8], f[9], f[10]};
            r[8] = f[11];
        } else {
            float *r = drest + G * 45 + 12 * q - 3;
            *reinterpret_cast<v4u *>(r) = v4u{f[0], f[1], f[2], f[3]};
            *reinterpret_cast<v4u *>(r + 4) = v4u{f[4], f[5], f[6], f[7]};
            *reinterpret_cast<v4u *>(r + 8) = v4u{f[8], f[9], f[10], f[11]};
        }
        return;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = 4 * q + k;
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) {
            if (fused) dsh[G * 48 + 3 * i + ch] = d[k][ch];
            else if (i == 0) dsh[G * 3 + ch] = d[k][ch];
            else drest[G * 45 + 3 * (i - 1) + ch] = d[k][ch];
        }
    }
}

struct PreFwdArgs {
    Cam C;
    int64_t N;
    const float *means, *quats, *scales, *sh, *rest, *opac;
    int32_t fused, vec4;
    float *uv, *conic, *depth, *rxy, *color;
    int32_t *valid;
    uint8_t *valid_mask;   // optional: the same flag as one byte (a torch bool mask)
    // Mip filters (MIP kernels only): per-Gaussian 3D filter size or null,
    // the 2D compensation flag, and the opacity binning and compositing use.
    const float *filt;
    int32_t aa;
    float *op_eff;
    int32_t act;   // kActLogScale | kActLogitOpac (effective-opacity kernel only)
    // Optional: per block of kPreThreads Gaussians, an estimate of the
    // binning's work over tiles of `tile` pixels (see block_work_of).
    int32_t *block_work;
    int32_t tile;
};

// The binning's count and write passes take a workgroup per block of 256
// Gaussians, and a block's time grows with the tiles its rectangles cover: a
// wave walks each rectangle over 32 tiles, which near the camera can span
// thousands. Each visible Gaussian counts the tiles of its clamped
// rectangle (as the binning forms it, rounded the same way for tiles of a
// power of two), or 4 for a rectangle the count pass tests lane-parallel.
__device__ __forceinline__ int block_work_of(bool ok, float u, float v, float rx, float ry,
                                             int tile, int W, int H) {
    if (!ok) return 0;
    const int tx = (W + tile - 1) / tile, ty = (H + tile - 1) / tile;
    const float it = 1.0f / (float)tile;
    const int x0 = min(max((int)floorf((u - rx) * it), 0), tx - 1);
    const int x1 = min(max((int)floorf((u + rx) * it), 0), tx - 1);
    const int y0 = min(max((int)floorf((v - ry) * it), 0), ty - 1);
    const int y1 = min(max((int)floorf((v + ry) * it), 0), ty - 1);
    // Capped so that a block's sum stays well inside int32.
    const int64_t area = (int64_t)(x1 - x0 + 1) * (y1 - y0 + 1);
    return area > 32 ? (int)min(area, (int64_t)1 << 22) : 4;
}

template <bool MIP>
__global__ __launch_bounds__(kPreThreads) void preprocess_fwd_kernel(const PreFwdArgs A) {
    const Cam &C = A.C;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // Blocks take the Gaussians from the last block to the first. In a
    // training step this kernel follows the optimizer update, which walks
    // them first to last, so the first blocks dispatched read the parameters
    // written last, which are still in the memory-side cache, before the
    // rest of this kernel's reads evict them (config 4: 62.5-63.5 -> 58-59 us,
    // step -4 us).
    const int64_t g0 = (int64_t)(gridDim.x - 1 - blockIdx.x) * kPreThreads + wave * 64;
    const int64_t g = g0 + lane;
    const bool in = g < A.N;

    // ------------------------------------------ projection: lane = Gaussian
    bool ok = false;
    int bwork = 0;
    float mx = 0.f, my = 0.f, mz = 0.f;
    if (in) {
        mx = A.means[3 * g]; my = A.means[3 * g + 1]; mz = A.means[3 * g + 2];
        const float qv[4] = {A.quats[4 * g], A.quats[4 * g + 1], A.quats[4 * g + 2], A.quats[4 * g + 3]};
        float sv[3] = {A.scales[3 * g], A.scales[3 * g + 1], A.scales[3 * g + 2]};
        float op = A.opac[g];
        if (MIP && (A.act & kActLogScale)) {
            sv[0] = expf(sv[0]);
            sv[1] = expf(sv[1]);
            sv[2] = expf(sv[2]);
        }
        if (MIP && (A.act & kActLogitOpac)) op = act_sigmoid(op);
        if (MIP && A.filt) {
            Mip3 M3;
            mip3_apply(A.filt[g], sv, M3);
            op *= M3.coef;
        }
        Proj P;
        project(C, mx, my, mz, qv, sv, P);
        const float z = P.p[2];
        const float u = C.fx * P.p[0] / P.zc + C.cx;
        const float v = C.fy * P.p[1] / P.zc + C.cy;
        const float det = P.a * P.c - P.b * P.b;
        const float dets = fmaxf(det, 1e-12f);
        const float mid = 0.5f * (P.a + P.c);
        const float disc = sqrtf(fmaxf(mid * mid - dets, 0.0f));
        const float lam = fmaxf(mid + disc, 1e-12f);
        const float radius = 3.0f * sqrtf(lam);
        // SnugBox: the alpha = 1/255 level set has per-axis half-extent
        // sqrt(2 ln(255 op)) * sqrt(cov_axis), never more than the 3-sigma
        // circle (preprocess.metal:180-190).
        const float two_l = 2.0f * logf(fmaxf(255.0f * op, 1.0f));
        const float rs = sqrtf(two_l);
        const float rx = fminf(rs * sqrtf(fmaxf(P.a, 0.0f)), radius);
        const float ry = fminf(rs * sqrtf(fmaxf(P.c, 0.0f)), radius);
        ok = (z > C.near_p) && (z < C.far_p) && (det > 1e-12f) && (radius < C.max_r) &&
             (rx > 0.0f) && (ry > 0.0f) && (u + rx > 0.0f) && (u - rx < (float)C.W) &&
             (v + ry > 0.0f) && (v - ry < (float)C.H);
        A.uv[2 * g] = u;
        A.uv[2 * g + 1] = v;
        A.conic[3 * g] = P.c / dets;
        A.conic[3 * g + 1] = -P.b / dets;
        A.conic[3 * g + 2] = P.a / dets;
        A.depth[g] = z;
        A.rxy[2 * g] = rx;
        A.rxy[2 * g + 1] = ry;
        A.valid[g] = ok ? 1 : 0;
        if (A.valid_mask) A.valid_mask[g] = ok ? 1 : 0;
        if (MIP) A.op_eff[g] = A.aa ? op * mip2_coef(P) : op;
        if (A.block_work) bwork = block_work_of(ok, u, v, rx, ry, A.tile, C.W, C.H);
    }
    if (A.block_work) {   // workgroup-uniform
        __shared__ int32_t s_work[kPreThreads / 64];
        for (int o = 32; o >= 1; o >>= 1) bwork += __shfl_xor(bwork, o, 64);
        if (lane == 0) s_work[wave] = bwork;
        __syncthreads();
        if (threadIdx.x == 0) {
            int sum = 0;
            for (int w = 0; w < kPreThreads / 64; ++w) sum += s_work[w];
            A.block_work[gridDim.x - 1 - blockIdx.x] = sum;
        }
    }

    if (A.sh == nullptr) return;   // explicit-colour callers: no SH, no colour
    // Colour is evaluated only where the rasteriser can look (sh.py at the
    // visible Gaussians); the rest get 0.
    if (ballot(ok) == 0) {
        if (in) { A.color[3 * g] = 0.f; A.color[3 * g + 1] = 0.f; A.color[3 * g + 2] = 0.f; }
        return;
    }
    // Basis values once per Gaussian (lane = Gaussian), parked in LDS for
    // the quads.
    __shared__ float s_b[kPreThreads / 64][64 * 16];
    float *bw = s_b[wave];
    {
        float B[16] = {};
        if (ok) {
            const float dx = mx - C.cc[0], dy = my - C.cc[1], dz = mz - C.cc[2];
            const float inv = 1.0f / fmaxf(sqrtf(dx * dx + dy * dy + dz * dz), 1e-12f);
            sh_basis(C.deg, dx * inv, dy * inv, dz * inv, B);
        }
        float4 *dst = reinterpret_cast<float4 *>(bw + 16 * lane);
#pragma unroll
        for (int k = 0; k < 4; ++k)
            dst[k] = make_float4(B[4 * k], B[4 * k + 1], B[4 * k + 2], B[4 * k + 3]);
    }
    wave_lds_sync();

    // ---------------------------------------------- SH colour: quad = Gaussian
    // Four rounds of 16 Gaussians; each round requests the next one's
    // coefficients before its own arithmetic.
    const int nb = (C.deg + 1) * (C.deg + 1);
    const ShRows R{A.sh, A.rest, A.fused, A.vec4};
    const int q = lane & 3;
    float c[4][3] = {};
    bool okq = __shfl((int)ok, lane >> 2, 64) != 0;     // false past the end
    if (okq) load_bases(R, g0 + (lane >> 2), q, nb, c);
#pragma unroll 1
    for (int r = 0; r < 4; ++r) {
        const int gl = 16 * r + (lane >> 2);
        const int64_t G = g0 + gl;
        float cn[4][3] = {};
        bool okn = false;
        if (r < 3) {
            okn = __shfl((int)ok, gl + 16, 64) != 0;
            if (okn) load_bases(R, G + 16, q, nb, cn);
        }
        const float4 bq = *reinterpret_cast<const float4 *>(bw + 16 * gl + 4 * q);
        const float b[4] = {bq.x, bq.y, bq.z, bq.w};
        float part[3] = {0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int ch = 0; ch < 3; ++ch) part[ch] += b[k] * c[k][ch];
        const float s0 = quad_sum(part[0]), s1 = quad_sum(part[1]), s2 = quad_sum(part[2]);
        if (G < A.N && q < 3) {
            const float sv = q == 0 ? s0 : (q == 1 ? s1 : s2);
            A.color[3 * G + q] = okq ? fmaxf(sv + 0.5f, 0.0f) : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int ch = 0; ch < 3; ++ch) c[k][ch] = cn[k][ch];
        okq = okn;
    }
}

// Adam applied in place by the backward instead of writing the gradients of
// its six parameter tensors: means 0, quats 1, scales 2, opacities 3, sh (DC
// or fused) 4, sh_rest 5.
struct AdamEpi {
    float *p[6], *m[6], *v[6];
    float step_size[6], inv_sqrt_bc2[6];
    float b1, b2, omb1, omb2, eps;
    const int64_t *skip;   // NULL, or the launch does nothing when skip[1] != 0
};

// Cache policy of the epilogue's traffic. The SH rows' moments (48 of the 59
// floats per Gaussian, moved as whole float4 lines) are loaded and stored
// non-temporally, so the 470 MB of moment traffic streams past the caches
// and the parameters the next projection forward reads stay resident: at
// config 4 that forward took 82 us after this kernel with ordinary moment
// accesses and 64 us with these, and the step 1.080 -> 1.060 ms, this
// kernel unchanged. The 11 non-SH moments of a Gaussian are stored as
// 4-byte pieces of 12- and 16-byte rows; non-temporal, those stores leave
// lines partly written and slowed this kernel by 25 us, so they stay
// ordinary, as do the parameter accesses; their loads are non-temporal
// (1.061 -> 1.059 ms). Bits: 0 non-SH moment loads, 1 non-SH moment stores,
// 2 parameter stores non-temporal.
constexpr int kEpiNt = 1;
constexpr bool kNtLoad = kEpiNt & 1, kNtMom = kEpiNt & 2, kNtPar = kEpiNt & 4;
constexpr bool kShNtMom = true;   // SH rows' moment loads and stores

typedef float v4a __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ float ld_nt(const float *q) {
    return NT ? __builtin_nontemporal_load(q) : *q;
}
template <bool NT>
__device__ __forceinline__ void st_nt(float *q, float x) {
    if (NT) __builtin_nontemporal_store(x, q);
    else *q = x;
}
template <bool NT>
__device__ __forceinline__ float4 ld_nt4(const float *q) {
    const v4a v = NT ? __builtin_nontemporal_load(reinterpret_cast<const v4a *>(q))
                     : *reinterpret_cast<const v4a *>(q);
    return make_float4(v.x, v.y, v.z, v.w);
}
template <bool NT>
__device__ __forceinline__ void st_nt4(float *q, const float4 &a) {
    v4a v = {a.x, a.y, a.z, a.w};
    if (NT) __builtin_nontemporal_store(v, reinterpret_cast<v4a *>(q));
    else *reinterpret_cast<v4a *>(q) = v;
}

// The moments could alias the parameters as far as the compiler knows, so it
// keeps every load after every earlier store: each helper below therefore
// requests all of its moments before it stores anything, one memory round
// trip instead of one per element.

// The Gaussian's 11 non-SH elements: means (3), quats (4), scales (3),
// opacity (1), with their gradients.
__device__ __forceinline__ void epi_rows(const AdamEpi &E, int64_t g, const float (&pm)[3],
                                         const float (&pq)[4], const float (&ps)[3],
                                         const float (&gm)[3], const float (&gq)[4],
                                         const float (&gs)[3], float gop) {
    float mm[3], vm[3], mq[4], vq[4], msc[3], vsc[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        mm[j] = ld_nt<kNtLoad>(E.m[0] + 3 * g + j);
        vm[j] = ld_nt<kNtLoad>(E.v[0] + 3 * g + j);
        msc[j] = ld_nt<kNtLoad>(E.m[2] + 3 * g + j);
        vsc[j] = ld_nt<kNtLoad>(E.v[2] + 3 * g + j);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        mq[j] = ld_nt<kNtLoad>(E.m[1] + 4 * g + j);
        vq[j] = ld_nt<kNtLoad>(E.v[1] + 4 * g + j);
    }
    float po = E.p[3][g];
    float mo = ld_nt<kNtLoad>(E.m[3] + g), vo = ld_nt<kNtLoad>(E.v[3] + g);
    float qm[3] = {pm[0], pm[1], pm[2]}, qq[4] = {pq[0], pq[1], pq[2], pq[3]};
    float qs[3] = {ps[0], ps[1], ps[2]};
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        adam_update(qm[j], gm[j], mm[j], vm[j], E.b1, E.b2, E.omb1, E.omb2, E.eps,
                    E.step_size[0], E.inv_sqrt_bc2[0], false);
        adam_update(qs[j], gs[j], msc[j], vsc[j], E.b1, E.b2, E.omb1, E.omb2, E.eps,
                    E.step_size[2], E.inv_sqrt_bc2[2], false);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
        adam_update(qq[j], gq[j], mq[j], vq[j], E.b1, E.b2, E.omb1, E.omb2, E.eps,
                    E.step_size[1], E.inv_sqrt_bc2[1], false);
    adam_update(po, gop, mo, vo, E.b1, E.b2, E.omb1, E.omb2, E.eps, E.step_size[3],
                E.inv_sqrt_bc2[3], false);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        st_nt<kNtPar>(E.p[0] + 3 * g + j, qm[j]);
        st_nt<kNtMom>(E.m[0] + 3 * g + j, mm[j]);
        st_nt<kNtMom>(E.v[0] + 3 * g + j, vm[j]);
        st_nt<kNtPar>(E.p[2] + 3 * g + j, qs[j]);
        st_nt<kNtMom>(E.m[2] + 3 * g + j, msc[j]);
        st_nt<kNtMom>(E.v[2] + 3 * g + j, vsc[j]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        st_nt<kNtPar>(E.p[1] + 4 * g + j, qq[j]);
        st_nt<kNtMom>(E.m[1] + 4 * g + j, mq[j]);
        st_nt<kNtMom>(E.v[1] + 4 * g + j, vq[j]);
    }
    st_nt<kNtPar>(E.p[3] + g, po);
    st_nt<kNtMom>(E.m[3] + g, mo);
    st_nt<kNtMom>(E.v[3] + g, vo);
}

// The staged round's Adam: the slice sb holds the round's d_sh and cb its
// parameters (the same block positions; each lane reads back the float4s it
// put there itself); moments are read and written at those positions of their
// tensors. A float4 that runs past the round's ng Gaussians is handled per
// element.
//
// A lane's tensor (t = 4, the SH or its DC rows, or 5, the rest rows) varies
// across the wave, so its pointers and step constants are selected from the
// two constant-index entries (held in scalar registers) rather than indexed
// by t: an index into the argument's tables is a vector load of the pointer,
// and every moment access waited for one.
struct EpiRow {
    float *p, *m, *v;
    float step_size, inv_sqrt_bc2;
};
__device__ __forceinline__ EpiRow epi_row(const AdamEpi &E, bool dc) {
    return {dc ? E.p[4] : E.p[5], dc ? E.m[4] : E.m[5], dc ? E.v[4] : E.v[5],
            dc ? E.step_size[4] : E.step_size[5], dc ? E.inv_sqrt_bc2[4] : E.inv_sqrt_bc2[5]};
}

__device__ __forceinline__ void stage_adam(const float4 *sb, const float4 *cb,
                                           const AdamEpi &E, int fused, int64_t G0, int ng) {
    const int lane = threadIdx.x & 63;
    float4 m4[3], v4[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int f = 4 * (lane + 64 * i);
        const EpiRow R = epi_row(E, fused || f < 48);
        const int64_t off = fused ? G0 * 48 + f : (f < 48 ? G0 * 3 + f : G0 * 45 + (f - 48));
        if (stage_row(fused, f + 3) < ng) {
            m4[i] = ld_nt4<kShNtMom>(R.m + off);
            v4[i] = ld_nt4<kShNtMom>(R.v + off);
        } else {
            float e[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (stage_row(fused, f + k) < ng) {
                    e[k] = ld_nt<kShNtMom>(R.m + off + k);
                    e[4 + k] = ld_nt<kShNtMom>(R.v + off + k);
                }
            }
            m4[i] = make_float4(e[0], e[1], e[2], e[3]);
            v4[i] = make_float4(e[4], e[5], e[6], e[7]);
        }
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int f = 4 * (lane + 64 * i);
        const EpiRow R = epi_row(E, fused || f < 48);
        const int64_t off = fused ? G0 * 48 + f : (f < 48 ? G0 * 3 + f : G0 * 45 + (f - 48));
        const float4 g4 = sb[lane + 64 * i];
        float gs[4] = {g4.x, g4.y, g4.z, g4.w};
        const float4 c4 = cb[lane + 64 * i];
        float po[4] = {c4.x, c4.y, c4.z, c4.w};
        float ms[4] = {m4[i].x, m4[i].y, m4[i].z, m4[i].w};
        float vs[4] = {v4[i].x, v4[i].y, v4[i].z, v4[i].w};
#pragma unroll
        for (int k = 0; k < 4; ++k)
            adam_update(po[k], gs[k], ms[k], vs[k], E.b1, E.b2, E.omb1, E.omb2, E.eps,
                        R.step_size, R.inv_sqrt_bc2, false);
        if (stage_row(fused, f + 3) < ng) {
            st_nt4<kNtPar>(R.p + off, make_float4(po[0], po[1], po[2], po[3]));
            st_nt4<kShNtMom>(R.m + off, make_float4(ms[0], ms[1], ms[2], ms[3]));
            st_nt4<kShNtMom>(R.v + off, make_float4(vs[0], vs[1], vs[2], vs[3]));
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (stage_row(fused, f + k) < ng) {
                    st_nt<kNtPar>(R.p + off + k, po[k]);
                    st_nt<kShNtMom>(R.m + off + k, ms[k]);
                    st_nt<kShNtMom>(R.v + off + k, vs[k]);
                }
            }
        }
    }
}

struct PreBwdArgs {
    Cam C;
    int64_t N;
    const float *means, *quats, *scales, *sh, *rest;
    int32_t fused, vec4, st_vec4;
    const float *d_uv, *d_conic, *d_color;
    // Floats per Gaussian between consecutive d_uv, d_conic, d_color and d_oe
    // entries: 2, 3, 3, 1 for separate arrays, one record stride otherwise.
    int32_t su, sk, sc, so;
    const int32_t *valid;
    float *d_means, *d_quats, *d_scales, *d_sh, *d_rest;
    // Mip filters (MIP kernels only): the unfiltered opacity, the 3D filter
    // size or null, the 2D flag, the gradient of the effective opacity, and
    // the opacity gradient written back.
    const float *opac, *filt, *d_oe;
    int32_t aa;
    float *d_op;
    int32_t act;   // kActLogScale | kActLogitOpac (effective-opacity kernel only)
    int32_t stage; // SH rows and their gradients staged through LDS
    // Regularisers (effective-opacity kernel only): the gradient of
    // reg_op * sum(opacity) + reg_sc * sum(scale) over every element of the
    // activated opacities and scales, added to every row (0: none).
    float reg_op, reg_sc;
    AdamEpi E;     // the optimizer epilogue (EPI kernels)
};

// Gaussians per wave of the epilogue kernel: two SH rounds. At 3 waves per
// SIMD the GPU holds 3072 of its waves; with 64 Gaussians each, config 4's
// 15625 waves filled those slots 5.09 times, and the last, nearly empty
// round of waves ran at a fraction of the bandwidth (per-wave timestamps:
// 47 us per wave, 35 of them in the SH rounds at about 6.4 TB/s overall).
// 32 per wave: 1.006 -> 0.994 ms per step (48: 0.996; 16: 1.014).
constexpr int kEpiGaussians = 32;

// EPI: the optimizer epilogue replaces the six gradient outputs (needs MIP,
// STAGE and d_color). A wave takes kGpw consecutive Gaussians (a multiple of
// the 16 of an SH round), one per lane; lanes past kGpw have none.
template <bool MIP, bool STAGE, bool EPI>
__device__ __forceinline__ void preprocess_bwd_body(const PreBwdArgs &A) {
    const Cam &C = A.C;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int kGpw = EPI ? kEpiGaussians : 64;
    static_assert(kGpw % 16 == 0 && kGpw <= 64, "whole SH rounds per wave");
    const int64_t g0 = ((int64_t)blockIdx.x * (kPreThreads / 64) + wave) * kGpw;
    const int64_t g = g0 + lane;
    const bool in = lane < kGpw && g < A.N;
    // With the epilogue every row of the wave's first SH round is read
    // whatever the gradients, so that round's rows are requested first and
    // arrive during the prologue's dependent loads and the basis evaluation
    // (config 4: 275-276 -> 272 us).
    float4 pf0[3];
    if (EPI) {
        const ShRows R0{A.sh, A.rest, A.fused, A.vec4};
        const int nw0 = (int)max((int64_t)0, min((int64_t)kGpw, A.N - g0));
        stage_load(R0, g0, min(16, nw0), 0xFFFFu, pf0);
    }

    float mx = 0.f, my = 0.f, mz = 0.f;
    int vld = 0;
    if (in) {
        mx = A.means[3 * g]; my = A.means[3 * g + 1]; mz = A.means[3 * g + 2];
        vld = A.valid[g];
    }
    float dmean[3] = {0.f, 0.f, 0.f};
    // The projection's inputs, requested now so they arrive during the SH
    // phase.
    float qv[4] = {0.f, 0.f, 0.f, 0.f}, sraw[3] = {0.f, 0.f, 0.f};
    float k0 = 0.f, k1 = 0.f, k2 = 0.f, du = 0.f, dv = 0.f;
    if (in) {
        qv[0] = A.quats[4 * g]; qv[1] = A.quats[4 * g + 1];
        qv[2] = A.quats[4 * g + 2]; qv[3] = A.quats[4 * g + 3];
        sraw[0] = A.scales[3 * g]; sraw[1] = A.scales[3 * g + 1]; sraw[2] = A.scales[3 * g + 2];
        const float *kc = A.d_conic + (int64_t)A.sk * g, *ku = A.d_uv + (int64_t)A.su * g;
        k0 = kc[0]; k1 = kc[1]; k2 = kc[2];
        du = ku[0]; dv = ku[1];
    }

    // --------------------------------------------------------------- SH
    // A (lane = Gaussian): view direction and the 16 basis values, parked in
    //   LDS. B (quad = Gaussian, four rounds of 16, the next round's
    //   coefficients loaded during this one): the quad's four bases and
    //   coefficients give the colour for the ReLU gate, d_sh, and the four
    //   per-basis weights w_b = c_b . dcolour, which overwrite those bases in
    //   LDS. C (lane = Gaussian): one VJP of the 16 bases with those weights
    //   gives the direction gradient. The basis values and the VJP are thus
    //   evaluated once per Gaussian rather than once per quad lane.
    __shared__ float s_bw[kPreThreads / 64][64 * 16];
    if (A.d_color != nullptr) {
        float dcol[3] = {0.f, 0.f, 0.f};
        if (in) {
            const float *kd = A.d_color + (int64_t)A.sc * g;
            dcol[0] = kd[0]; dcol[1] = kd[1]; dcol[2] = kd[2];
        }
        // The colour of a Gaussian that is not visible is the constant 0, so
        // its coefficients get no gradient.
        const bool need = vld != 0 && (dcol[0] != 0.f || dcol[1] != 0.f || dcol[2] != 0.f);
        const int ng = (int)max((int64_t)0, min((int64_t)kGpw, A.N - g0));
        if (!EPI && ballot(need) == 0) {
            // Coalesced zero fill of the wave's rows.
            if (A.fused) {
                for (int e = lane; e < ng * 48; e += 64) A.d_sh[g0 * 48 + e] = 0.f;
            } else {
                for (int e = lane; e < ng * 3; e += 64) A.d_sh[g0 * 3 + e] = 0.f;
                for (int e = lane; e < ng * 45; e += 64) A.d_rest[g0 * 45 + e] = 0.f;
            }
        } else {
            float *bw = s_bw[wave];
            float ux = 0.f, uy = 0.f, uz = 0.f, un = 1.f;
            {
                float B[16] = {};
                if (need) {
                    const float vx = mx - C.cc[0], vy = my - C.cc[1], vz = mz - C.cc[2];
                    un = fmaxf(sqrtf(vx * vx + vy * vy + vz * vz), 1e-12f);
                    ux = vx / un; uy = vy / un; uz = vz / un;
                    sh_basis(C.deg, ux, uy, uz, B);
                }
                float4 *dst = reinterpret_cast<float4 *>(bw + 16 * lane);
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    dst[k] = make_float4(B[4 * k], B[4 * k + 1], B[4 * k + 2], B[4 * k + 3]);
            }
            wave_lds_sync();
            const int nb = (C.deg + 1) * (C.deg + 1);
            const ShRows R{A.sh, A.rest, A.fused, A.vec4};
            const int q = lane & 3;
            // One round's arithmetic for the quad's Gaussian gl: d_sh of its
            // four bases (0 unless needed) and the per-basis weights into LDS.
            auto round_math = [&](int gl, bool nq, const float (&c)[4][3], float (&dsh)[4][3]) {
                const float d0 = __shfl(dcol[0], gl, 64), d1 = __shfl(dcol[1], gl, 64);
                const float d2 = __shfl(dcol[2], gl, 64);
                const float4 bq = *reinterpret_cast<const float4 *>(bw + 16 * gl + 4 * q);
                const float b[4] = {bq.x, bq.y, bq.z, bq.w};
                float pre[3] = {0.f, 0.f, 0.f};
#pragma unroll
                for (int k = 0; k < 4; ++k)
#pragma unroll
                    for (int ch = 0; ch < 3; ++ch) pre[ch] += b[k] * c[k][ch];
                const float p0 = quad_sum(pre[0]) + 0.5f, p1 = quad_sum(pre[1]) + 0.5f;
                const float p2 = quad_sum(pre[2]) + 0.5f;
                // ReLU gate of colour = max(pre, 0) (torch_ref.py:331).
                const float dp0 = p0 > 0.f ? d0 : 0.f, dp1 = p1 > 0.f ? d1 : 0.f;
                const float dp2 = p2 > 0.f ? d2 : 0.f;
                float wk[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    dsh[k][0] = nq ? b[k] * dp0 : 0.f;
                    dsh[k][1] = nq ? b[k] * dp1 : 0.f;
                    dsh[k][2] = nq ? b[k] * dp2 : 0.f;
                    wk[k] = nq ? c[k][0] * dp0 + c[k][1] * dp1 + c[k][2] * dp2 : 0.f;
                }
                *reinterpret_cast<float4 *>(bw + 16 * gl + 4 * q) =
                    make_float4(wk[0], wk[1], wk[2], wk[3]);
            };
            if (STAGE) {
                // Rounds staged through the wave's LDS slice: coefficients in
                // (the next round's requested first), d_sh out, both as
                // aligned coalesced float4s.
                __shared__ float4 s_st[kPreThreads / 64][kStageF4];
                float4 *sb = s_st[wave];
                float *sf = reinterpret_cast<float *>(sb);
                const uint64_t nm = ballot(need);
                const int nw = (int)max((int64_t)0, min((int64_t)kGpw, A.N - g0));
                // With the epilogue every row's parameters are read (all are
                // updated) and a second slice keeps the round's own for it.
                __shared__ float4 s_cur[EPI ? kPreThreads / 64 : 1][EPI ? kStageF4 : 1];
                float4 *cb = s_cur[EPI ? wave : 0];
                float4 pf[3];
                const uint64_t lm = EPI ? ~0ull : nm;
                if (EPI) {
                    pf[0] = pf0[0]; pf[1] = pf0[1]; pf[2] = pf0[2];
                } else {
                    stage_load(R, g0, min(16, nw), (uint32_t)(lm & 0xFFFFu), pf);
                }
#pragma unroll 1
                for (int r = 0; r < 4; ++r) {
                    const int ngr = min(16, max(0, nw - 16 * r));
                    if (ngr == 0) break;   // wave-uniform: no Gaussian left
                    stage_put(sb, pf);
                    if (EPI) stage_put(cb, pf);
                    wave_lds_sync();
                    const int ngn = min(16, max(0, nw - 16 * (r + 1)));
                    if (r < 3 && ngn > 0)
                        stage_load(R, g0 + 16 * (r + 1), ngn,
                                   (uint32_t)((lm >> (16 * (r + 1))) & 0xFFFFu), pf);
                    const int gl = 16 * r + (lane >> 2);
                    float c[4][3], dsh[4][3];
                    stage_read(sf, A.fused, lane >> 2, q, c);
                    round_math(gl, (nm >> gl) & 1u, c, dsh);
                    wave_lds_sync();   // every coefficient read before d_sh replaces it
                    stage_write(sf, A.fused, lane >> 2, q, dsh);
                    wave_lds_sync();
                    if (ngr > 0) {
                        if (EPI) stage_adam(sb, cb, A.E, A.fused, g0 + 16 * r, ngr);
                        else stage_store(sb, A.d_sh, A.d_rest, A.fused, g0 + 16 * r, ngr);
                    }
                    wave_lds_sync();   // the slice is rewritten next round
                }
            } else {
                // Round 0's coefficients; each round then requests the next one's.
                float c[4][3] = {};
                bool nq = __shfl((int)need, lane >> 2, 64) != 0;
                if (nq) load_bases(R, g0 + (lane >> 2), q, nb, c);
#pragma unroll 1
                for (int r = 0; r < 4; ++r) {
                    const int gl = 16 * r + (lane >> 2);
                    const int64_t G = g0 + gl;
                    float cn[4][3] = {};
                    bool nqn = false;
                    if (r < 3) {
                        nqn = __shfl((int)need, gl + 16, 64) != 0;
                        if (nqn) load_bases(R, G + 16, q, nb, cn);
                    }
                    float dsh[4][3];
                    round_math(gl, nq, c, dsh);
                    if (G < A.N) store_bases(A.d_sh, A.d_rest, A.fused, A.st_vec4, G, q, dsh);
#pragma unroll
                    for (int k = 0; k < 4; ++k)
#pragma unroll
                        for (int ch = 0; ch < 3; ++ch) c[k][ch] = cn[k][ch];
                    nq = nqn;
                }
            }
            wave_lds_sync();
            if (need) {
                float w16[16];
                const float4 *src = reinterpret_cast<const float4 *>(bw + 16 * lane);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float4 v = src[k];
                    w16[4 * k] = v.x; w16[4 * k + 1] = v.y; w16[4 * k + 2] = v.z; w16[4 * k + 3] = v.w;
                }
                float gp[3];
                sh_basis_vjp(C.deg, ux, uy, uz, w16, gp);
                // dir = v/|v|: d v = (I - dir dir^T) d dir / |v|
                const float dd = ux * gp[0] + uy * gp[1] + uz * gp[2];
                dmean[0] += (gp[0] - ux * dd) / un;
                dmean[1] += (gp[1] - uy * dd) / un;
                dmean[2] += (gp[2] - uz * dd) / un;
            }
        }
    }
    if (!in) return;

    // ------------------------------------------ projection: lane = Gaussian
    // The gradients of the quats, scales and opacity (zero for a row that is
    // not visible, before the regularisers).
    float gq[4] = {0.f, 0.f, 0.f, 0.f}, gsc[3] = {0.f, 0.f, 0.f}, gop = 0.f;
    if (vld != 0) {
        // s0: the activated scales before the 3D filter; op0: the activated
        // opacity.
        float s0[3] = {sraw[0], sraw[1], sraw[2]};
        float op0 = 0.0f;
        if (MIP) {
            if (A.act & kActLogScale) {
                s0[0] = expf(s0[0]);
                s0[1] = expf(s0[1]);
                s0[2] = expf(s0[2]);
            }
            op0 = A.opac[g];
            if (A.act & kActLogitOpac) op0 = act_sigmoid(op0);
        }
        float sv[3] = {s0[0], s0[1], s0[2]};
        Mip3 M3;
        M3.coef = 1.0f;
        float f3 = 0.0f;
        if (MIP && A.filt) {
            f3 = A.filt[g];
            mip3_apply(f3, sv, M3);
        }
        Proj P;
        project(C, mx, my, mz, qv, sv, P);
        const float a = P.a, b = P.b, c = P.c;
        const float det = a * c - b * b;
        const float id = 1.0f / fmaxf(det, 1e-12f);

        // conic = (c, -b, a) / det
        const float ddet = -(k0 * c - k1 * b + k2 * a) * id * id;
        float da = k2 * id + ddet * c;
        float db = -k1 * id - 2.0f * ddet * b;
        float dc = k0 * id + ddet * a;
        if (det <= 1e-12f) da = db = dc = 0.f;

        // Effective opacity oe = op coef3 coef2: its gradient reaches the
        // opacity, the 2D covariance (through coef2) and the scales (through
        // coef3, below).
        float d_op1 = 0.0f;
        if (MIP) {
            const float d_oe = A.d_oe[(int64_t)A.so * g];
            d_op1 = d_oe;
            if (A.aa) {
                const float op1 = op0 * M3.coef;
                const float det0 = P.a0 * P.c0 - b * b;
                const float r = fmaxf(det0, 0.0f) / fmaxf(det, 1e-12f);
                const float coef2 = sqrtf(fminf(fmaxf(r, 0.0f), 1.0f));
                d_op1 = d_oe * coef2;
                // coef2 = sqrt(det0 / det) where 0 < r <= 1 (the clamps pass
                // the gradient there; sqrt has none to give at r = 0).
                if (r > 0.0f && r <= 1.0f && det > 1e-12f) {
                    const float dr = 0.5f * d_oe * op1 / coef2;
                    const float ddet0 = dr / det;
                    const float ddet = -dr * r / det;
                    da += ddet0 * P.c0 + ddet * c;
                    dc += ddet0 * P.a0 + ddet * a;
                    db += -2.0f * b * (ddet0 + ddet);
                }
            }
        }

        // a = T0 S T0, b = T0 S T1, c = T1 S T1 (S symmetric).
        const float *S = P.S;
        const float s00 = S[0], s01 = S[1], s02 = S[2], s11 = S[3], s12 = S[4], s22 = S[5];
        const float *T0 = P.T0, *T1 = P.T1;
        float ST0[3], ST1[3];
        ST0[0] = s00 * T0[0] + s01 * T0[1] + s02 * T0[2];
        ST0[1] = s01 * T0[0] + s11 * T0[1] + s12 * T0[2];
        ST0[2] = s02 * T0[0] + s12 * T0[1] + s22 * T0[2];
        ST1[0] = s00 * T1[0] + s01 * T1[1] + s02 * T1[2];
        ST1[1] = s01 * T1[0] + s11 * T1[1] + s12 * T1[2];
        ST1[2] = s02 * T1[0] + s12 * T1[1] + s22 * T1[2];
        float dT0[3], dT1[3];
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            dT0[k] = 2.0f * da * ST0[k] + db * ST1[k];
            dT1[k] = 2.0f * dc * ST1[k] + db * ST0[k];
        }
        // Symmetric dSigma = da T0T0' + db (T0T1' + T1T0')/2 + dc T1T1'.
        float dS[9];
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j)
                dS[3 * i + j] = da * T0[i] * T0[j] + 0.5f * db * (T0[i] * T1[j] + T1[i] * T0[j]) +
                                dc * T1[i] * T1[j];

        // T0 = j0x Rw0 + j0z Rw2 ; T1 = j1y Rw1 + j1z Rw2.
        const float dj0x = dT0[0] * C.R[0] + dT0[1] * C.R[1] + dT0[2] * C.R[2];
        const float dj0z = dT0[0] * C.R[6] + dT0[1] * C.R[7] + dT0[2] * C.R[8];
        const float dj1y = dT1[0] * C.R[3] + dT1[1] * C.R[4] + dT1[2] * C.R[5];
        const float dj1z = dT1[0] * C.R[6] + dT1[1] * C.R[7] + dT1[2] * C.R[8];
        const float izc = P.izc, izc2 = izc * izc, izc3 = izc2 * izc;
        // j0x = fx/zc, j0z = -fx tx/zc^2, j1y = fy/zc, j1z = -fy ty/zc^2
        const float dtx = -C.fx * izc2 * dj0z;
        const float dty = -C.fy * izc2 * dj1z;
        float dzc = -C.fx * izc2 * dj0x - C.fy * izc2 * dj1y +
                    2.0f * C.fx * P.tx * izc3 * dj0z + 2.0f * C.fy * P.ty * izc3 * dj1z;
        // u = fx px/zc + cx, v = fy py/zc + cy
        float dpx = C.fx * izc * du;
        float dpy = C.fy * izc * dv;
        dzc += -C.fx * P.p[0] * izc2 * du - C.fy * P.p[1] * izc2 * dv;
        // tx = clamp(px/zc) zc: unclamped -> tx == px; clamped -> +-lim zc.
        if (!P.clx) dpx += dtx; else dzc += dtx * (P.tx * izc);
        if (!P.cly) dpy += dty; else dzc += dty * (P.ty * izc);
        const float dpz = (P.p[2] > C.near_p) ? dzc : 0.0f;
        // p = Rw m + t
        dmean[0] += C.R[0] * dpx + C.R[3] * dpy + C.R[6] * dpz;
        dmean[1] += C.R[1] * dpx + C.R[4] * dpy + C.R[7] * dpz;
        dmean[2] += C.R[2] * dpx + C.R[5] * dpy + C.R[8] * dpz;

        // Sigma = M M^T: dM = 2 dS M.
        float dM[9];
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j)
                dM[3 * i + j] = 2.0f * (dS[3 * i] * P.M[j] + dS[3 * i + 1] * P.M[3 + j] +
                                        dS[3 * i + 2] * P.M[6 + j]);
        // M = R diag(s)
        float dsc[3], G[9];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            dsc[j] = dM[j] * P.R[j] + dM[3 + j] * P.R[3 + j] + dM[6 + j] * P.R[6 + j];
            G[j] = dM[j] * P.s[j];
            G[3 + j] = dM[3 + j] * P.s[j];
            G[6 + j] = dM[6 + j] * P.s[j];
        }
        if (MIP) {
            if (A.filt) {
                // s' = sqrt(s^2 + f^2): ds = ds' s / s'. coef3^2 = prod s^2 /
                // prod (s^2 + f^2): d coef3 / d s_j = coef3 f^2 / (s_j (s_j^2 + f^2)).
                const float dcoef3 = d_op1 * op0;
                const float f2 = f3 * f3;
#pragma unroll
                for (int j = 0; j < 3; ++j) {
                    const float chain = sv[j] > 0.0f ? dsc[j] * s0[j] / sv[j] : 0.0f;
                    const float dimm = s0[j] > 0.0f
                        ? dcoef3 * M3.coef * f2 / (s0[j] * M3.s2f[j]) : 0.0f;
                    dsc[j] = chain + dimm;
                }
            }
            float dop = d_op1 * M3.coef;
            // Through the activations, as torch's backward of exp (grad *
            // result) and of sigmoid (grad * (1 - y) * y).
            if (A.act & kActLogitOpac) dop = dop * (1.0f - op0) * op0;
            gop = dop;
            if (A.act & kActLogScale) {
                dsc[0] = dsc[0] * s0[0];
                dsc[1] = dsc[1] * s0[1];
                dsc[2] = dsc[2] * s0[2];
            }
        }
#pragma unroll
        for (int j = 0; j < 3; ++j) gsc[j] = dsc[j];
        // R(q) for unit q = (w,x,y,z): d/dq of sum G_ij R_ij.
        const float w = P.q[0], x = P.q[1], y = P.q[2], z = P.q[3];
        const float G00 = G[0], G01 = G[1], G02 = G[2], G10 = G[3], G11 = G[4], G12 = G[5],
                    G20 = G[6], G21 = G[7], G22 = G[8];
        const float dw = 2.0f * (x * (G21 - G12) + y * (G02 - G20) + z * (G10 - G01));
        const float dxq = 2.0f * (w * (G21 - G12) + y * (G01 + G10) + z * (G02 + G20) - 2.0f * x * (G11 + G22));
        const float dyq = 2.0f * (w * (G02 - G20) + x * (G01 + G10) + z * (G12 + G21) - 2.0f * y * (G00 + G22));
        const float dzq = 2.0f * (w * (G10 - G01) + x * (G02 + G20) + y * (G12 + G21) - 2.0f * z * (G00 + G11));
        // through q/|q|
        const float dotq = w * dw + x * dxq + y * dyq + z * dzq;
        const float iq = 1.0f / fmaxf(P.qn, 1e-12f);
        const float dq[4] = {(dw - w * dotq) * iq, (dxq - x * dotq) * iq,
                             (dyq - y * dotq) * iq, (dzq - z * dotq) * iq};
#pragma unroll
        for (int j = 0; j < 4; ++j) gq[j] = dq[j];
    }
    // A row that is not visible keeps zero photometric gradients; with the
    // epilogue Adam still decays its moments and steps it.
    if (MIP && (A.reg_op != 0.0f || A.reg_sc != 0.0f)) {
        // The regularisers' share, on every row: d/dx of reg_op * sigmoid(x)
        // is reg_op * (1 - y) * y and of reg_sc * exp(x) is reg_sc * exp(x),
        // as torch's sigmoid and exp backward form them; without the
        // activations the opacities and scales are the regularised values.
        float ro = A.reg_op;
        if (A.act & kActLogitOpac) {
            const float y = act_sigmoid(A.opac[g]);
            ro = ro * (1.0f - y) * y;
        }
        gop += ro;
#pragma unroll
        for (int j = 0; j < 3; ++j)
            gsc[j] += (A.act & kActLogScale) ? A.reg_sc * expf(sraw[j]) : A.reg_sc;
    }
    if (EPI) {
        const float pm[3] = {mx, my, mz};
        epi_rows(A.E, g, pm, qv, sraw, dmean, gq, gsc, gop);
    } else {
        if (MIP) A.d_op[g] = gop;
        A.d_scales[3 * g] = gsc[0];
        A.d_scales[3 * g + 1] = gsc[1];
        A.d_scales[3 * g + 2] = gsc[2];
        A.d_quats[4 * g] = gq[0];
        A.d_quats[4 * g + 1] = gq[1];
        A.d_quats[4 * g + 2] = gq[2];
        A.d_quats[4 * g + 3] = gq[3];
        A.d_means[3 * g] = dmean[0];
        A.d_means[3 * g + 1] = dmean[1];
        A.d_means[3 * g + 2] = dmean[2];
    }
}

template <bool MIP, bool STAGE>
__global__ __launch_bounds__(kPreThreads) __attribute__((amdgpu_waves_per_eu(4)))
void preprocess_bwd_kernel(const PreBwdArgs A) {
    preprocess_bwd_body<MIP, STAGE, false>(A);
}

// The backward with the optimizer epilogue: 153 VGPRs, 3 waves/SIMD, a wave
// per kEpiGaussians Gaussians.
__global__ __launch_bounds__(kPreThreads) __attribute__((amdgpu_waves_per_eu(3)))
void preprocess_bwd_adam_kernel(const PreBwdArgs A) {
    if (A.E.skip && A.E.skip[1] != 0) return;
    preprocess_bwd_body<true, true, true>(A);
}

static int32_t make_cam(Cam &C, const float *viewmat, float fx, float fy, float cx, float cy,
                        int32_t W, int32_t H, float near_p, float far_p, float blur,
                        float max_r, const float *cam_center, int32_t deg, const char *who) {
    MG_REQUIRE(viewmat != nullptr, "%s: viewmat (host, 16 floats) is null", who);
    MG_REQUIRE(cam_center != nullptr, "%s: cam_center (host, 3 floats) is null", who);
    MG_REQUIRE(W > 0 && H > 0, "%s: image %dx%d", who, W, H);
    MG_REQUIRE(deg >= 0 && deg <= 3, "%s: sh_degree %d not in 0..3", who, deg);
    for (int i = 0; i < 3; ++i) {
        for (int j = 0; j < 3; ++j) C.R[3 * i + j] = viewmat[4 * i + j];
        C.t[i] = viewmat[4 * i + 3];
        C.cc[i] = cam_center[i];
    }
    C.fx = fx; C.fy = fy; C.cx = cx; C.cy = cy;
    C.near_p = near_p; C.far_p = far_p; C.blur = blur; C.max_r = max_r;
    C.W = W; C.H = H; C.deg = deg;
    return MG_OK;
}

static int32_t preprocess_fwd(int64_t N, const float *means, const float *quats,
                              const float *scales, const float *sh, const float *sh_rest,
                              int32_t sh_fused, const float *opacities, const float *viewmat,
                              float fx, float fy, float cx, float cy, int32_t W, int32_t H,
                              float near_plane, float far_plane, float blur, float max_radius,
                              const float *cam_center, int32_t sh_degree, bool mip,
                              const float *filter_3d, int32_t antialias, int32_t activations,
                              float *uv, float *conic, float *depth, float *rxy,
                              int32_t *valid, uint8_t *valid_mask, float *color,
                              float *opacity_eff, mg_stream_t stream, const char *who,
                              int32_t tile = 0, int32_t *block_work = nullptr) {
    PreFwdArgs A{};
    int32_t rc = make_cam(A.C, viewmat, fx, fy, cx, cy, W, H, near_plane, far_plane, blur,
                          max_radius, cam_center, sh_degree, who);
    if (rc != MG_OK) return rc;
    MG_REQUIRE(N >= 0, "%s: N = %lld", who, (long long)N);
    if (N == 0) return MG_OK;
    MG_REQUIRE(means && quats && scales && opacities && uv && conic && depth && rxy && valid,
               "%s: null tensor pointer", who);
    MG_REQUIRE(sh == nullptr || color != nullptr, "%s: SH given but no colour output", who);
    MG_REQUIRE(sh == nullptr || sh_fused || sh_rest != nullptr,
               "SH must be either one (N,16,3) tensor or (N,1,3)+(N,15,3)");
    MG_REQUIRE(!mip || opacity_eff != nullptr, "%s: null effective-opacity output", who);
    MG_REQUIRE((activations & ~(kActLogScale | kActLogitOpac)) == 0 && (mip || activations == 0),
               "%s: activations %d (bit 0: log scales, bit 1: logit opacities)", who,
               activations);
    A.N = N;
    A.means = means; A.quats = quats; A.scales = scales; A.sh = sh;
    A.rest = sh_rest; A.opac = opacities; A.fused = sh_fused;
    A.uv = uv; A.conic = conic; A.depth = depth; A.rxy = rxy; A.valid = valid; A.color = color;
    A.valid_mask = valid_mask;
    A.filt = filter_3d; A.aa = antialias; A.op_eff = opacity_eff; A.act = activations;
    A.vec4 = sh && sh_degree == 3 && (!sh_fused || ((uintptr_t)sh & 15) == 0);
    MG_REQUIRE(block_work == nullptr || tile >= 1, "%s: block_work needs a tile size, got %d",
               who, tile);
    A.block_work = block_work;
    A.tile = tile;
    const int64_t blocks = ceil_div(N, kPreThreads);
    TimedScope ts("preprocess_forward", as_stream(stream));
    if (mip)
        preprocess_fwd_kernel<true><<<(unsigned)blocks, kPreThreads, 0, as_stream(stream)>>>(A);
    else
        preprocess_fwd_kernel<false><<<(unsigned)blocks, kPreThreads, 0, as_stream(stream)>>>(A);
    MG_LAUNCHED("preprocess_fwd_kernel");
    return MG_OK;
}

static int32_t preprocess_bwd(int64_t N, const float *means, const float *quats,
                              const float *scales, const float *sh, const float *sh_rest,
                              int32_t sh_fused, const float *d_uv, const float *d_conic,
                              const float *d_color, int32_t grad_stride, const int32_t *valid,
                              const float *viewmat, float fx, float fy, float cx, float cy,
                              int32_t W, int32_t H, float near_plane, float far_plane,
                              float blur, float max_radius, const float *cam_center,
                              int32_t sh_degree, bool mip,
                              const float *opacities, const float *filter_3d, int32_t antialias,
                              int32_t activations, float reg_opacity, float reg_scale,
                              const float *d_opacity_eff, float *d_means, float *d_quats,
                              float *d_scales, float *d_sh, float *d_sh_rest,
                              float *d_opacities, const mg_adam_epilogue *adam,
                              mg_stream_t stream, const char *who) {
    PreBwdArgs A{};
    int32_t rc = make_cam(A.C, viewmat, fx, fy, cx, cy, W, H, near_plane, far_plane, blur,
                          max_radius, cam_center, sh_degree, who);
    if (rc != MG_OK) return rc;
    MG_REQUIRE(N >= 0, "%s: N = %lld", who, (long long)N);
    if (N == 0) return MG_OK;
    MG_REQUIRE(means && quats && scales && d_uv && d_conic && valid &&
                   (adam || (d_means && d_quats && d_scales)), "%s: null tensor pointer", who);
    if (d_color) {
        MG_REQUIRE(sh && (adam || d_sh) && (sh_fused || (sh_rest && (adam || d_sh_rest))),
                   "SH must be either one (N,16,3) tensor or (N,1,3)+(N,15,3)");
    }
    MG_REQUIRE(!mip || (opacities && d_opacity_eff && (adam || d_opacities)),
               "%s: null opacity pointer", who);
    MG_REQUIRE(grad_stride == 0 || grad_stride >= 3, "%s: gradient record stride %d", who,
               grad_stride);
    MG_REQUIRE((activations & ~(kActLogScale | kActLogitOpac)) == 0 && (mip || activations == 0),
               "%s: activations %d (bit 0: log scales, bit 1: logit opacities)", who,
               activations);
    MG_REQUIRE(mip || (reg_opacity == 0.0f && reg_scale == 0.0f),
               "%s: regularisers need the effective-opacity kernel", who);
    MG_REQUIRE(std::isfinite(reg_opacity) && std::isfinite(reg_scale),
               "%s: regulariser weights must be finite", who);
    A.reg_op = reg_opacity;
    A.reg_sc = reg_scale;
    A.su = grad_stride ? grad_stride : 2;
    A.sk = grad_stride ? grad_stride : 3;
    A.sc = grad_stride ? grad_stride : 3;
    A.so = grad_stride ? grad_stride : 1;
    A.N = N;
    A.means = means; A.quats = quats; A.scales = scales; A.sh = sh; A.rest = sh_rest;
    A.fused = sh_fused; A.d_uv = d_uv; A.d_conic = d_conic; A.d_color = d_color; A.valid = valid;
    A.d_means = d_means; A.d_quats = d_quats; A.d_scales = d_scales; A.d_sh = d_sh;
    A.d_rest = d_sh_rest;
    A.opac = opacities; A.filt = filter_3d; A.aa = antialias; A.d_oe = d_opacity_eff;
    A.d_op = d_opacities; A.act = activations;
    A.vec4 = sh && sh_degree == 3 && (!sh_fused || ((uintptr_t)sh & 15) == 0);
    A.st_vec4 = d_sh && sh_degree == 3 && (!sh_fused || ((uintptr_t)d_sh & 15) == 0);
    A.stage = A.vec4 && A.st_vec4 && stage_aligned(sh, sh_rest, sh_fused) &&
              stage_aligned(d_sh, d_sh_rest, sh_fused);
    if (adam) {
        // The epilogue reads the parameters the kernel already holds and
        // writes them back, so its tensors must be the kernel's inputs.
        const float *in[6] = {means, quats, scales, opacities, sh, sh_fused ? nullptr : sh_rest};
        for (int t = 0; t < 6; ++t) {
            MG_REQUIRE(adam->p[t] == in[t] && (in[t] == nullptr || (adam->m[t] && adam->v[t])),
                       "%s: optimizer epilogue tensor %d is not the kernel's input", who, t);
            MG_REQUIRE(in[t] == nullptr || adam->step[t] >= 1,
                       "%s: optimizer epilogue step %lld < 1", who, (long long)adam->step[t]);
        }
        MG_REQUIRE(mip && d_color && sh_degree == 3 && A.vec4 &&
                       stage_aligned(sh, sh_rest, sh_fused) &&
                       stage_aligned(adam->m[4], adam->m[5], sh_fused) &&
                       stage_aligned(adam->v[4], adam->v[5], sh_fused),
                   "%s: the optimizer epilogue needs the effective-opacity kernel, d_color, "
                   "SH degree 3 and 16-byte aligned SH tensors and moments", who);
        A.stage = 1;
        AdamEpi &E = A.E;
        E.b1 = (float)adam->beta1;
        E.b2 = (float)adam->beta2;
        E.omb1 = (float)(1.0 - adam->beta1);
        E.omb2 = (float)(1.0 - adam->beta2);
        E.eps = (float)adam->eps;
        E.skip = adam->skip;
        for (int t = 0; t < 6; ++t) {
            E.p[t] = adam->p[t];
            E.m[t] = adam->m[t];
            E.v[t] = adam->v[t];
            if (in[t] == nullptr) continue;
            // Formed in double from the exact hyperparameters, as FusedAdam.
            const double bc1 = 1.0 - std::pow(adam->beta1, (double)adam->step[t]);
            const double bc2 = 1.0 - std::pow(adam->beta2, (double)adam->step[t]);
            E.step_size[t] = (float)(adam->lr[t] / bc1);
            E.inv_sqrt_bc2[t] = (float)(1.0 / std::sqrt(bc2));
        }
    }
    const int64_t blocks = ceil_div(N, kPreThreads);
    hipStream_t st = as_stream(stream);
    if (adam) {
        TimedScope ts("preprocess_backward_adam", st);
        preprocess_bwd_adam_kernel<<<(unsigned)ceil_div(N, (kPreThreads / 64) * kEpiGaussians),
                                     kPreThreads, 0, st>>>(A);
        MG_LAUNCHED("preprocess_bwd_adam_kernel");
        return MG_OK;
    }
    TimedScope ts("preprocess_backward", st);
    if (mip && A.stage)
        preprocess_bwd_kernel<true, true><<<(unsigned)blocks, kPreThreads, 0, st>>>(A);
    else if (mip)
        preprocess_bwd_kernel<true, false><<<(unsigned)blocks, kPreThreads, 0, st>>>(A);
    else if (A.stage)
        preprocess_bwd_kernel<false, true><<<(unsigned)blocks, kPreThreads, 0, st>>>(A);
    else
        preprocess_bwd_kernel<false, false><<<(unsigned)blocks, kPreThreads, 0, st>>>(A);
    MG_LAUNCHED("preprocess_bwd_kernel");
    return MG_OK;
}

}  // namespace mg

using namespace mg;

extern "C" {

int32_t mg_preprocess_forward(int64_t N, const float *means, const float *quats,
                              const float *scales, const float *sh, const float *sh_rest,
                              int32_t sh_fused, const float *opacities, const float *viewmat,
                              float fx, float fy, float cx, float cy, int32_t W, int32_t H,
                              float near_plane, float far_plane, float blur, float max_radius,
                              const float *cam_center, int32_t sh_degree, float *uv,
                              float *conic, float *depth, float *rxy, int32_t *valid,
                              uint8_t *valid_mask, float *color, mg_stream_t stream) {
    return preprocess_fwd(N, means, quats, scales, sh, sh_rest, sh_fused, opacities, viewmat,
                          fx, fy, cx, cy, W, H, near_plane, far_plane, blur, max_radius,
                          cam_center, sh_degree, false, nullptr, 0, 0, uv, conic, depth, rxy,
                          valid, valid_mask, color, nullptr, stream, "mg_preprocess_forward");
}

int32_t mg_preprocess_forward_mip(int64_t N, const float *means, const float *quats,
                                  const float *scales, const float *sh, const float *sh_rest,
                                  int32_t sh_fused, const float *opacities,
                                  const float *viewmat, float fx, float fy, float cx, float cy,
                                  int32_t W, int32_t H, float near_plane, float far_plane,
                                  float blur, float max_radius, const float *cam_center,
                                  int32_t sh_degree, const float *filter_3d, int32_t antialias,
                                  int32_t activations, float *uv, float *conic, float *depth,
                                  float *rxy,
                                  int32_t *valid, uint8_t *valid_mask, float *color,
                                  float *opacity_eff, int32_t tile, int32_t *block_work,
                                  mg_stream_t stream) {
    return preprocess_fwd(N, means, quats, scales, sh, sh_rest, sh_fused, opacities, viewmat,
                          fx, fy, cx, cy, W, H, near_plane, far_plane, blur, max_radius,
                          cam_center, sh_degree, true, filter_3d, antialias, activations, uv,
                          conic, depth, rxy, valid, valid_mask, color, opacity_eff, stream,
                          "mg_preprocess_forward_mip", tile, block_work);
}

int32_t mg_preprocess_backward(int64_t N, const float *means, const float *quats,
                               const float *scales, const float *sh, const float *sh_rest,
                               int32_t sh_fused, const float *d_uv, const float *d_conic,
                               const float *d_color, int32_t grad_stride, const int32_t *valid,
                               const float *viewmat,
                               float fx, float fy, float cx, float cy, int32_t W, int32_t H,
                               float near_plane, float far_plane, float blur, float max_radius,
                               const float *cam_center, int32_t sh_degree, float *d_means,
                               float *d_quats, float *d_scales, float *d_sh, float *d_sh_rest,
                               mg_stream_t stream) {
    return preprocess_bwd(N, means, quats, scales, sh, sh_rest, sh_fused, d_uv, d_conic,
                          d_color, grad_stride, valid, viewmat, fx, fy, cx, cy, W, H, near_plane,
                          far_plane, blur, max_radius, cam_center, sh_degree, false, nullptr,
                          nullptr, 0, 0, 0.0f, 0.0f,
                          nullptr, d_means, d_quats, d_scales, d_sh, d_sh_rest, nullptr, nullptr,
                          stream, "mg_preprocess_backward");
}

int32_t mg_preprocess_backward_mip(int64_t N, const float *means, const float *quats,
                                   const float *scales, const float *sh, const float *sh_rest,
                                   int32_t sh_fused, const float *d_uv, const float *d_conic,
                                   const float *d_color, int32_t grad_stride,
                                   const int32_t *valid, const float *viewmat, float fx, float fy,
                                   float cx, float cy,
                                   int32_t W, int32_t H, float near_plane, float far_plane,
                                   float blur, float max_radius, const float *cam_center,
                                   int32_t sh_degree, const float *opacities,
                                   const float *filter_3d, int32_t antialias,
                                   int32_t activations, float reg_opacity, float reg_scale,
                                   const float *d_opacity_eff, float *d_means, float *d_quats,
                                   float *d_scales, float *d_sh, float *d_sh_rest,
                                   float *d_opacities, const mg_adam_epilogue *adam,
                                   mg_stream_t stream) {
    return preprocess_bwd(N, means, quats, scales, sh, sh_rest, sh_fused, d_uv, d_conic,
                          d_color, grad_stride, valid, viewmat, fx, fy, cx, cy, W, H,
                          near_plane, far_plane, blur, max_radius, cam_center, sh_degree, true,
                          opacities, filter_3d, antialias, activations, reg_opacity,
                          reg_scale, d_opacity_eff,
                          d_means, d_quats, d_scales, d_sh, d_sh_rest, d_opacities, adam,
                          stream, "mg_preprocess_backward_mip");
}

}  // extern "C"
