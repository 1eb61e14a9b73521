// The INRIA 3DGS .ply record <-> the renderer's tensors, on the GPU
// (metal_gauss/io.py:45-123, train.py:582-624).
//
// A 3DGS .ply body is an array of fixed-size float32 records, one per
// Gaussian, holding *parameterised* values: position, f_dc_{0,1,2},
// f_rest_{0..3*P-1} stored channel-major (f_rest_[c*P + b-1]), a logit
// opacity, log scales and an unnormalised wxyz quaternion. After one upload
// of the raw records, the decode kernel writes the activated tensors the
// renderer takes (sigmoid, exp, normalised quaternion, SH as (N, 1+P, 3));
// the encode kernel is the reverse for export, from the trainer's own
// parameters, optionally with Mip-Splatting's 3D filter baked in.
//
// Records are addressed by column index (the file's property order is free),
// one thread per (Gaussian, output value): consecutive threads write
// consecutive outputs, and their reads stay inside a few records.
#include "mg_common.h"

namespace mg {

// Column of each field in a record (in floats).
struct PlyCols {
    int32_t stride;          // floats per record
    int32_t xyz[3], rot[4], scale[3], opacity, dc[3];
    int32_t rest0;           // column of f_rest_0; f_rest_i is rest0 + i
    int32_t per_channel;     // P: higher bases per channel (0..15)
    // Whether f_rest_i sits at rest0 + i for every i (else rest_col holds them).
    int32_t rest_contig;
    int32_t rest_col[45];
    // The inverse map for encoding: what column c of a record holds. 0-2 xyz,
    // 3-6 rot, 7-9 scale, 10 opacity, 11-13 f_dc, 14 + i f_rest_i, -1 none.
    int8_t field_of[64];
};

// Values per Gaussian in the decoded layout: means 3, quats 4, scales 3,
// opacity 1, sh 3 (1 + P).
__device__ __forceinline__ int decoded_width(int P) { return 11 + 3 * (1 + P); }

__device__ __forceinline__ int rest_column(const PlyCols &C, int i) {
    return C.rest_contig ? C.rest0 + i : C.rest_col[i];
}

__global__ __launch_bounds__(256) void ply_decode_kernel(const float *__restrict__ rec, int64_t n,
                                                         const PlyCols C, float *means,
                                                         float *quats, float *scales,
                                                         float *opac, float *sh) {
    const int w = decoded_width(C.per_channel);
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= n * w) return;
    const int64_t g = t / w;
    const int k = (int)(t - g * w);
    const float *r = rec + g * C.stride;
    if (k < 3) {
        means[3 * g + k] = r[C.xyz[k]];
    } else if (k < 7) {
        // io.py:118: q / max(|q|, 1e-12), the norm in double as numpy forms it.
        const double q0 = r[C.rot[0]], q1 = r[C.rot[1]], q2 = r[C.rot[2]], q3 = r[C.rot[3]];
        const double nq = fmax(sqrt(q0 * q0 + q1 * q1 + q2 * q2 + q3 * q3), 1e-12);
        quats[4 * g + (k - 3)] = (float)((double)r[C.rot[k - 3]] / nq);
    } else if (k < 10) {
        scales[3 * g + (k - 7)] = (float)exp((double)r[C.scale[k - 7]]);
    } else if (k == 10) {
        opac[g] = (float)(1.0 / (1.0 + exp(-(double)r[C.opacity])));
    } else {
        // sh[g, b, c]: b = 0 from f_dc_c, b >= 1 from f_rest_[c P + b - 1].
        const int j = k - 11, b = j / 3, c = j - 3 * b;
        const int col = b == 0 ? C.dc[c] : rest_column(C, c * C.per_channel + b - 1);
        sh[g * 3 * (1 + C.per_channel) + j] = r[col];
    }
}

// Encode: trainer parameters -> INRIA records in the column order of C.
struct PlyEncodeSrc {
    const float *means, *quats, *log_scales, *logit, *sh_dc, *sh_rest, *sh;
    const float *filter_3d;   // optional: bake Mip-Splatting's 3D filter
    int32_t sh_bases;         // bases stored per Gaussian in sh / sh_rest (+1)
};

__global__ __launch_bounds__(256) void ply_encode_kernel(const PlyEncodeSrc S, int64_t n,
                                                         const PlyCols C, float *rec) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= n * C.stride) return;
    const int64_t g = t / C.stride;
    const int col = (int)(t - g * C.stride);
    const int P = C.per_channel;
    float v = 0.0f;
    const int field = C.field_of[col];
    if (field >= 0 && field < 3) {
        v = S.means[3 * g + field];
    } else if (field >= 3 && field < 7) {
        v = S.quats[4 * g + field - 3];
    } else if (field >= 7 && field <= 10) {
        // Log scales and logit opacity, with the 3D filter folded in when
        // given (train.py:603-615): s' = sqrt(s^2 + f^2), op' = op *
        // sqrt(clamp(prod s^2 / prod s'^2, 0, 1)), back to log / logit space
        // with the clamps of train.py:612-614.
        const int which = field < 10 ? field - 7 : -1;
        {
            if (S.filter_3d == nullptr) {
                v = which >= 0 ? S.log_scales[3 * g + which] : S.logit[g];
            } else {
                const float f = S.filter_3d[g], f2 = f * f;
                float s2[3], s2f[3];
#pragma unroll
                for (int i = 0; i < 3; ++i) {
                    const float sc = expf(S.log_scales[3 * g + i]);
                    s2[i] = sc * sc;
                    s2f[i] = s2[i] + f2;
                }
                if (which >= 0) {
                    v = logf(fmaxf(sqrtf(s2f[which]), 1e-12f));
                } else {
                    const float coef = sqrtf(fminf(fmaxf((s2[0] * s2[1] * s2[2]) /
                                                          (s2f[0] * s2f[1] * s2f[2]), 0.0f), 1.0f));
                    float op = (1.0f / (1.0f + expf(-S.logit[g]))) * coef;
                    op = fminf(fmaxf(op, 1e-6f), 1.0f - 1e-6f);
                    v = logf(op / (1.0f - op));
                }
            }
        }
    } else if (field >= 11 && field < 14) {
        const int c = field - 11;
        v = S.sh ? S.sh[g * 3 * S.sh_bases + c] : S.sh_dc[3 * g + c];
    } else if (field >= 14 && P > 0) {
        const int i = field - 14, c = i / P, b = i - c * P + 1;
        v = S.sh ? S.sh[g * 3 * S.sh_bases + 3 * b + c]
                 : S.sh_rest[g * 3 * (S.sh_bases - 1) + 3 * (b - 1) + c];
    }
    rec[t] = v;
}

static int32_t check_cols(const PlyCols &C, const char *who) {
    MG_REQUIRE(C.stride >= 14 && C.per_channel >= 0 && C.per_channel <= 15,
               "%s: record of %d floats with %d bases per channel", who, C.stride,
               C.per_channel);
    auto ok = [&](int c) { return c >= 0 && c < C.stride; };
    for (int i = 0; i < 3; ++i)
        MG_REQUIRE(ok(C.xyz[i]) && ok(C.scale[i]) && ok(C.dc[i]), "%s: column out of range", who);
    for (int i = 0; i < 4; ++i) MG_REQUIRE(ok(C.rot[i]), "%s: column out of range", who);
    MG_REQUIRE(ok(C.opacity), "%s: column out of range", who);
    for (int i = 0; i < 3 * C.per_channel; ++i)
        MG_REQUIRE(ok(C.rest_contig ? C.rest0 + i : C.rest_col[i]), "%s: f_rest column", who);
    return MG_OK;
}

static PlyCols make_cols(int32_t stride, const int32_t *cols, int32_t per_channel) {
    // cols: x y z rot0..3 scale0..2 opacity dc0..2, then 3P f_rest columns.
    PlyCols C{};
    C.stride = stride;
    for (int i = 0; i < 3; ++i) C.xyz[i] = cols[i];
    for (int i = 0; i < 4; ++i) C.rot[i] = cols[3 + i];
    for (int i = 0; i < 3; ++i) C.scale[i] = cols[7 + i];
    C.opacity = cols[10];
    for (int i = 0; i < 3; ++i) C.dc[i] = cols[11 + i];
    C.per_channel = per_channel;
    C.rest0 = per_channel > 0 ? cols[14] : 0;
    C.rest_contig = 1;
    for (int i = 0; i < 3 * per_channel && i < 45; ++i) {
        C.rest_col[i] = cols[14 + i];
        if (cols[14 + i] != C.rest0 + i) C.rest_contig = 0;
    }
    for (int c = 0; c < 64; ++c) C.field_of[c] = -1;
    for (int f = 0; f < 14 + 3 * per_channel && f < 59; ++f)
        if (cols[f] >= 0 && cols[f] < 64) C.field_of[cols[f]] = (int8_t)f;
    return C;
}

}  // namespace mg

using namespace mg;

extern "C" {

int32_t mg_ply_decode(int64_t n, const float *records, int32_t stride, const int32_t *columns,
                      int32_t per_channel, float *means, float *quats, float *scales,
                      float *opacities, float *sh, mg_stream_t stream) {
    MG_REQUIRE(n >= 0, "mg_ply_decode: n = %lld", (long long)n);
    MG_REQUIRE(columns, "mg_ply_decode: null column table");
    MG_REQUIRE(per_channel >= 0 && per_channel <= 15, "mg_ply_decode: %d bases per channel",
               per_channel);
    const PlyCols C = make_cols(stride, columns, per_channel);
    int32_t rc = check_cols(C, "mg_ply_decode");
    if (rc != MG_OK) return rc;
    if (n == 0) return MG_OK;
    MG_REQUIRE(records && means && quats && scales && opacities && sh,
               "mg_ply_decode: null pointer");
    const int64_t total = n * (11 + 3 * (1 + per_channel));
    hipStream_t s = as_stream(stream);
    TimedScope ts("ply_decode", s);
    ply_decode_kernel<<<(unsigned)ceil_div(total, 256), 256, 0, s>>>(records, n, C, means, quats,
                                                                     scales, opacities, sh);
    MG_LAUNCHED("ply_decode_kernel");
    return MG_OK;
}

int32_t mg_ply_encode(int64_t n, const float *means, const float *quats,
                      const float *log_scales, const float *logit_opac, const float *sh_dc,
                      const float *sh_rest, const float *sh, int32_t sh_bases,
                      const float *filter_3d, int32_t stride, const int32_t *columns,
                      int32_t per_channel, float *records, mg_stream_t stream) {
    MG_REQUIRE(n >= 0, "mg_ply_encode: n = %lld", (long long)n);
    MG_REQUIRE(columns, "mg_ply_encode: null column table");
    MG_REQUIRE(per_channel >= 0 && per_channel <= 15 && sh_bases >= 1 + per_channel,
               "mg_ply_encode: %d bases per channel from %d stored", per_channel, sh_bases);
    MG_REQUIRE(stride <= 64, "mg_ply_encode: records of %d floats (at most 64)", stride);
    const PlyCols C = make_cols(stride, columns, per_channel);
    int32_t rc = check_cols(C, "mg_ply_encode");
    if (rc != MG_OK) return rc;
    if (n == 0) return MG_OK;
    MG_REQUIRE(means && quats && log_scales && logit_opac && records, "mg_ply_encode: null pointer");
    MG_REQUIRE(sh || (sh_dc && (per_channel == 0 || sh_rest)),
               "SH must be either one (N,16,3) tensor or (N,1,3)+(N,15,3)");
    const PlyEncodeSrc S{means, quats, log_scales, logit_opac, sh_dc, sh_rest, sh, filter_3d,
                         sh_bases};
    hipStream_t s = as_stream(stream);
    TimedScope ts("ply_encode", s);
    ply_encode_kernel<<<(unsigned)ceil_div(n * stride, 256), 256, 0, s>>>(S, n, C, records);
    MG_LAUNCHED("ply_encode_kernel");
    return MG_OK;
}

}  // extern "C"
