/*
 * mgauss.h -- C ABI of the gfx950 splatting library (libmgauss.so).
 *
 * Every entry point takes raw device pointers, element counts, scalars and a
 * HIP stream, launches its kernels on that stream, and returns an MG_* status
 * code. Nothing here allocates device memory: callers pass every output and
 * every scratch buffer. On failure, mg_last_error() returns a message that
 * names the entry point and the offending argument (thread-local, valid until
 * the next failing call on the same thread).
 *
 * Each declaration cites the interface of nandometzger/metal-gauss it
 * replaces, as file:line under that repository. The reference binds these
 * through a pybind11 module (metal_gauss/csrc/rasterize.mm:518-533); this
 * library is bound through ctypes by metal-gauss_amd/_lib.py.
 *
 * Layout conventions (all fp32 unless stated, all row-major, contiguous):
 *   means (N,3)  quats (N,4) wxyz  scales (N,3) linear  opacities (N,) in [0,1]
 *   sh: fused (N,16,3), or split DC (N,1,3) + rest (N,15,3)
 *   uv (N,2)  conic (N,3) = (c,-b,a)/det of the dilated 2D covariance
 *   depth (N,)  rxy (N,2)  valid (N,) int32  color (N,3)
 *   images: rgb (H,W,3), alpha/T (H,W), stop index (H,W) int32
 */
#ifndef MGAUSS_H
#define MGAUSS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A hipStream_t. NULL selects the null stream. */
typedef void *mg_stream_t;

enum {
    MG_OK = 0,
    MG_ERR_ARG = 1,      /* bad argument: shape, size, pointer, tile */
    MG_ERR_LAUNCH = 2,   /* a kernel launch failed (hipGetLastError) */
    MG_ERR_RUNTIME = 3,  /* another HIP runtime call failed */
    MG_ERR_CAPACITY = 4  /* a caller buffer is smaller than the work needs */
};

/* ---------------------------------------------------------------- runtime */

/* Message for the last failing call on this thread ("" if none). */
const char *mg_last_error(void);

/* Library version, major*10000 + minor*100 + patch. */
int32_t mg_version(void);

/* Replaces init(src) (metal_gauss/csrc/rasterize.mm:196, 19-41). The reference
 * compiles Metal source at run time; here the gfx950 code objects are built
 * ahead of time, so init only checks that a HIP device is present and that
 * the code object loads on it. Idempotent. */
int32_t mg_init(void);

/* Largest tile edge the rasteriser accepts (one workgroup per tile, one
 * thread per pixel): 32, i.e. 1024 threads. The reference's equivalent check
 * is rasterize.mm:66-73. */
int32_t mg_max_tile(void);

/* Kernel timing with HIP events on each launch's own stream, for the bench
 * harness. No counterpart in the reference (it times phases from Python,
 * bench/step_profile.py:39-41). While enabled every launch records a pair of
 * events; mg_timing_query synchronises them and reports the summed duration
 * and launch count of one kernel by name since the last reset. */
int32_t mg_timing_enable(int32_t on);
int32_t mg_timing_reset(void);
int32_t mg_timing_query(const char *kernel, double *total_ms, int64_t *count);

/* STREAM "Copy" of `bytes` (a multiple of 16, 16-byte aligned buffers) from
 * src to dst, a hand-written float4 kernel: the achievable HBM bandwidth the
 * bench reports beside its roofline fractions. No counterpart in the
 * reference (its benchmark notes cite a STREAM-style copy). */
int32_t mg_stream_copy(const void *src, void *dst, int64_t bytes, mg_stream_t stream);

/* ------------------------------------------------------------- preprocess */

/* Fused projection + EWA covariance + SnugBox extents + validity + SH colour.
 * Replaces preprocess_forward (metal_gauss/csrc/rasterize.mm:244-284; kernel
 * preprocess.metal:114-221). viewmat (16 floats, row-major world->camera) and
 * cam_center (3 floats) are HOST pointers, read at call time, as the reference
 * reads them on the host (rasterize.mm:226-242). sh_fused != 0 means `sh` is
 * (N,16,3) and `sh_rest` is ignored; otherwise sh is (N,1,3) and sh_rest is
 * (N,15,3). sh_degree in 0..3. */
int32_t mg_preprocess_forward(
    int64_t N, const float *means, const float *quats, const float *scales,
    const float *sh, const float *sh_rest, int32_t sh_fused,
    const float *opacities, const float *viewmat, float fx, float fy,
    float cx, float cy, int32_t W, int32_t H, float near_plane,
    float far_plane, float blur, float max_radius, const float *cam_center,
    int32_t sh_degree, float *uv, float *conic, float *depth, float *rxy,
    int32_t *valid, uint8_t *valid_mask, float *color, mg_stream_t stream);

/* Analytic backward of mg_preprocess_forward. Replaces preprocess_backward
 * (metal_gauss/csrc/rasterize.mm:286-327; kernel preprocess.metal:223-411).
 * d_color may be NULL (explicit-colour callers): the SH branch is skipped and
 * d_sh / d_sh_rest are not written. In fused mode d_sh is (N,16,3) and
 * d_sh_rest is ignored (the reference aliases the two, rasterize.mm:300-302).
 * grad_stride 0: d_uv (N,2), d_conic (N,3), d_color (N,3) are separate
 * arrays; otherwise all three (and d_opacity_eff below) are read at
 * pointer + i * grad_stride floats for Gaussian i, e.g. slots 0, 2, 6 (and 5)
 * of mg_rasterize_backward's gradient records with grad_stride 10. */
int32_t mg_preprocess_backward(
    int64_t N, const float *means, const float *quats, const float *scales,
    const float *sh, const float *sh_rest, int32_t sh_fused,
    const float *d_uv, const float *d_conic, const float *d_color,
    int32_t grad_stride, const int32_t *valid, const float *viewmat, float fx, float fy, float cx,
    float cy, int32_t W, int32_t H, float near_plane, float far_plane,
    float blur, float max_radius, const float *cam_center, int32_t sh_degree,
    float *d_means, float *d_quats, float *d_scales, float *d_sh,
    float *d_sh_rest, mg_stream_t stream);

/* Mip-Splatting's filters folded into the projection: the same work as
 * mg_preprocess_forward, plus
 *   - filter_3d (N,) or NULL: the 3D low-pass of apply_3d_filter
 *     (metal_gauss/mipfilter.py:76-93), scales' = sqrt(scales^2 + f^2) and
 *     opacity * sqrt(prod scales^2 / prod scales'^2), which the reference's
 *     trainer applies in torch before render (train.py:223-227);
 *   - antialias != 0: the 2D compensation opacity * sqrt(det0 / det) of the
 *     blurred covariance, which the reference recomputes from the conic in
 *     torch (antialias_scale, metal_gauss/metal_backend.py:367-393, applied
 *     at 506-511; torch_ref.py:100-124).
 *   - activations: bit 0 set, scales holds log scales and the kernel takes
 *     their exp; bit 1 set, opacities holds logits and the kernel takes their
 *     sigmoid 1 / (1 + exp(-x)). These are the torch.exp and torch.sigmoid
 *     the reference's trainer applies before render (train.py:221-222); 0
 *     takes scales and opacities as given.
 * opacity_eff (N,) receives the opacity binning and compositing use. rxy and
 * valid see the opacity after the 3D filter and before the 2D one, as in the
 * reference.
 * block_work (device, ceil(N/256) int32, or NULL; needs tile >= 1) receives
 * per 256 Gaussians an estimate of mg_bin_lists_capped's work over tiles of
 * `tile` pixels, for its block_work argument. No counterpart in the
 * reference. */
int32_t mg_preprocess_forward_mip(
    int64_t N, const float *means, const float *quats, const float *scales,
    const float *sh, const float *sh_rest, int32_t sh_fused,
    const float *opacities, const float *viewmat, float fx, float fy,
    float cx, float cy, int32_t W, int32_t H, float near_plane,
    float far_plane, float blur, float max_radius, const float *cam_center,
    int32_t sh_degree, const float *filter_3d, int32_t antialias,
    int32_t activations, float *uv, float *conic, float *depth, float *rxy,
    int32_t *valid, uint8_t *valid_mask, float *color, float *opacity_eff,
    int32_t tile, int32_t *block_work, mg_stream_t stream);

/* Optional optimizer epilogue of mg_preprocess_backward_mip. The reference's
 * trainer runs FusedAdam after the backward (train.py:400-402, adam.metal);
 * with an epilogue the backward applies that Adam step itself to the six
 * parameter tensors, in the order means, quats, scales, opacities, sh (the
 * DC band, or the fused (N,16,3) tensor) and sh_rest (NULL when fused),
 * instead of writing their gradients: p, m (exp_avg) and v (exp_avg_sq) per
 * tensor, its learning rate and its step count after this step (>= 1), and
 * the shared betas and eps. The update is FusedAdam's (eps after the
 * sqrt(bc2) divide, bc1 and bc2 from the step count in double); every row is
 * updated, rows without gradient with g = 0. Needs sh_degree 3, d_color, and
 * 16-byte aligned SH tensors and moments. */
typedef struct mg_adam_epilogue {
    float *p[6];
    float *m[6];
    float *v[6];
    double lr[6];
    int64_t step[6];
    double beta1, beta2, eps;
    /* NULL, or the status words of the render's capacity-bounded tile lists
     * (mg_bin_lists_capped, device): when skip[1] != 0 (the lists
     * overflowed) the launch does nothing at all, so the step can be run
     * again with larger lists. */
    const int64_t *skip;
} mg_adam_epilogue;

/* Analytic backward of mg_preprocess_forward_mip. d_opacity_eff is the
 * gradient of opacity_eff; d_opacities (N,) receives the gradient of the
 * unfiltered opacities, and the filters' share of the scale and covariance
 * gradients is folded into d_scales, d_quats and d_means. With activations
 * (the forward's), d_scales and d_opacities are the gradients of the log
 * scales and the logits: times exp(log scale), and times (1 - y) y for
 * y = sigmoid(logit), as torch's backward of exp and sigmoid. The reference
 * gets these from torch autograd of the same expressions.
 * reg_opacity and reg_scale (0 for none) add, on every row visible or not,
 * the gradient of reg_opacity * sum(opacity) + reg_scale * sum(scale) over
 * all elements of the activated opacities (N,) and scales (N,3): the
 * trainer's regularisers opac_reg * mean(sigmoid(logit)) + scale_reg *
 * mean(exp(log_scales)) (metal_gauss/train.py:396-398) are
 * reg_opacity = opac_reg / N and reg_scale = scale_reg / (3 N). With adam
 * non-NULL the six gradients are not written (d_means .. d_opacities may be
 * NULL): the epilogue above applies them to the parameters in place. */
int32_t mg_preprocess_backward_mip(
    int64_t N, const float *means, const float *quats, const float *scales,
    const float *sh, const float *sh_rest, int32_t sh_fused,
    const float *d_uv, const float *d_conic, const float *d_color,
    int32_t grad_stride, const int32_t *valid, const float *viewmat, float fx, float fy, float cx,
    float cy, int32_t W, int32_t H, float near_plane, float far_plane,
    float blur, float max_radius, const float *cam_center, int32_t sh_degree,
    const float *opacities, const float *filter_3d, int32_t antialias,
    int32_t activations, float reg_opacity, float reg_scale,
    const float *d_opacity_eff, float *d_means, float *d_quats,
    float *d_scales, float *d_sh, float *d_sh_rest, float *d_opacities,
    const mg_adam_epilogue *adam, mg_stream_t stream);

/* Per-Gaussian 3D filter size. Replaces compute_3d_filter
 * (metal_gauss/mipfilter.py:29-73). views: (n_views, 20) device floats per
 * view: world->camera R (9, row-major), t (3), fx, fy, cx, cy, and the
 * frame's bounds with the margin, -margin*W, (1+margin)*W, -margin*H,
 * (1+margin)*H. focal is the largest fx or fy over the views (<= 0 means 1).
 * scratch: one device int32. filter_3d (N,) receives
 * (min seen depth / focal) * sqrt(0.2); unseen Gaussians take the largest
 * seen depth, and with none seen every depth is 1. */
int32_t mg_compute_3d_filter(int64_t N, const float *means, int32_t n_views,
                             const float *views, float focal,
                             float near_plane, float *filter_3d,
                             int32_t *scratch, mg_stream_t stream);

/* ------------------------------------------------------------------- MCMC */

/* SGLD exploration of the means of near-transparent Gaussians. Replaces
 * add_noise (metal_gauss/mcmc.py:164-192): means[i] += R(q_i) (z_i *
 * exp(log_scales_i)) * sigmoid(-100 (sigmoid(logit_i) - opacity_gate)) *
 * lr_means * weight for rows i < n. z are standard normals: eps (n,3) when
 * given, else drawn in the kernel (Philox4x64-10 keyed by `seed`, counter =
 * row, Box-Muller), so a seed fixes the draw. */
int32_t mg_add_noise(int64_t n, float *means, const float *log_scales,
                     const float *quats, const float *logit_opac,
                     const float *eps, float lr_means, float weight,
                     float opacity_gate, uint64_t seed, mg_stream_t stream);

/* Bytes of scratch relocate / grow need over n_rows candidate rows with
 * n_draw draw slots (relocate: n_draw = n_rows). */
int64_t mg_mcmc_workspace_bytes(int64_t n_rows, int64_t n_draw);

/* First half of relocate (metal_gauss/mcmc.py:52-104) or grow (124-161):
 * candidate weights over rows < n (weights (n,) or NULL for the opacity
 * sigmoid(logit); relocate: rows with opacity < thresh are dead and weigh 0;
 * grow != 0: every row is a candidate and drawn weights are floored at
 * 1e-8), their block sums, and the multiplicity counters cleared. Copies
 * five totals to totals_host after synchronising the stream (the
 * reference's nonzero / multinomial syncs too): [sum of weights, sum of the
 * opacity fallback, dead rows, any weight inf or nan, any weight > 0]. */
int32_t mg_mcmc_weights(int64_t n, const float *logit_opac, const float *weights,
                        float thresh, int32_t grow, void *ws, int64_t ws_size,
                        int64_t n_draw, double *totals_host, mg_stream_t stream);

/* Second half: draws with replacement in proportion to the weights (or the
 * opacity when use_opacity != 0, the reference's fallback), by inverse CDF
 * with Philox uniforms keyed by `seed`; relocate: one draw per dead row,
 * which becomes its destination; grow: n_draw draws with destinations
 * dst0 .. dst0 + n_draw - 1. Every destination gets its source's row of each
 * tensor, with the source's opacity split N ways (N = clamp(draws of the
 * source, 1, 51), plus 1 for grow) and its log-scales shrunk to match; every
 * drawn source gets the same split; both have their optimizer-state rows
 * zeroed (mcmc.py:107-121). tensors: n_tensors device pointers, each with
 * `widths[t]` floats per row and kinds[t] 0 = copied parameter, 1 =
 * log-scales, 2 = logit opacity (width 1), 3 = optimizer state (zeroed).
 * n_dest = dead rows (relocate) or n_draw (grow), from mg_mcmc_weights. */
int32_t mg_mcmc_apply(int64_t n, const float *logit_opac, const float *weights,
                      float thresh, int32_t grow, int32_t use_opacity, void *ws,
                      int64_t ws_size, int64_t n_draw, int64_t n_dest, int64_t dst0,
                      uint64_t seed, int32_t n_tensors, float *const *tensors,
                      const int32_t *widths, const int32_t *kinds,
                      mg_stream_t stream);

/* -------------------------------------------------------------------- PLY */

/* De-parameterise INRIA 3DGS .ply records on the device. Replaces the
 * arithmetic of load_ply (metal_gauss/io.py:89-123; the reference parses the
 * file with plyfile and computes in numpy). records: (n, stride) float32 as
 * they lie in the file. columns: 14 + 3*per_channel column indices, in the
 * order x y z rot_0..3 scale_0..2 opacity f_dc_0..2 f_rest_0..3P-1.
 * Writes means (n,3), quats (n,4) normalised, scales (n,3) = exp, opacities
 * (n,) = sigmoid, sh (n, 1+P, 3) (f_rest channel-major: f_rest_[c*P + b-1]
 * is sh[:, b, c]). */
int32_t mg_ply_decode(int64_t n, const float *records, int32_t stride,
                      const int32_t *columns, int32_t per_channel, float *means,
                      float *quats, float *scales, float *opacities, float *sh,
                      mg_stream_t stream);

/* Build INRIA records from the trainer's parameters. Replaces the arithmetic
 * of export_ply (metal_gauss/train.py:582-624): pre-activation values as
 * they are; SH from `sh` (n, sh_bases, 3) or from sh_dc (n,1,3) + sh_rest
 * (n, sh_bases-1, 3); with filter_3d (n,) the Mip 3D filter baked into the
 * log-scales and logit opacity. columns and per_channel as in
 * mg_ply_decode; records: (n, stride) float32. */
int32_t mg_ply_encode(int64_t n, const float *means, const float *quats,
                      const float *log_scales, const float *logit_opac,
                      const float *sh_dc, const float *sh_rest, const float *sh,
                      int32_t sh_bases, const float *filter_3d, int32_t stride,
                      const int32_t *columns, int32_t per_channel, float *records,
                      mg_stream_t stream);

/* ---------------------------------------------------------------- binning */

/* Per-Gaussian count of tiles that pass the exact ellipse-vs-tile test
 * (conic and opacity NULL: every tile of the uv +- rxy rectangle counts, the
 * circular-bounds contract of build_tile_lists, metal_backend.py:111-147).
 * Replaces bin_count (metal_gauss/csrc/rasterize.mm:485-497; kernel
 * binning.metal:92-104). counts: (N,) int32. */
int32_t mg_bin_count(int64_t N, const float *uv, const float *rxy,
                     const float *conic, const float *opacity,
                     const int32_t *valid, int32_t W, int32_t H, int32_t tile,
                     int32_t tiles_x, int32_t tiles_y, int32_t *counts,
                     mg_stream_t stream);

/* Bytes of scratch mg_exclusive_scan_i32 needs for n elements. */
int64_t mg_scan_workspace_bytes(int64_t n);

/* Exclusive prefix sum of int32 counts into int32 offsets, plus the int64
 * total written to total_dev (device) and, if total_host is not NULL, copied
 * to that host address and synchronised. Replaces the torch.cumsum and the
 * .item() of metal_backend.py:246-248. */
int32_t mg_exclusive_scan_i32(const int32_t *in, int64_t n, int32_t *out,
                              int64_t *total_dev, int64_t *total_host,
                              void *workspace, int64_t workspace_bytes,
                              mg_stream_t stream);

/* Emits one (key, id) pair per surviving (Gaussian, tile), Gaussian-major,
 * rows then columns, at offsets[g]: key = (tile_id << 32) | bits(depth).
 * Replaces bin_write (metal_gauss/csrc/rasterize.mm:499-516; kernel
 * binning.metal:106-120). keys: (total,) uint64, ids: (total,) int32. */
int32_t mg_bin_write(int64_t N, const float *uv, const float *rxy,
                     const float *conic, const float *opacity,
                     const int32_t *valid, const float *depth,
                     const int32_t *offsets, int64_t total, int32_t W,
                     int32_t H, int32_t tile, int32_t tiles_x,
                     int32_t tiles_y, uint64_t *keys, int32_t *ids,
                     mg_stream_t stream);

/* Bytes of scratch mg_sort_pairs_u64 needs for n pairs. */
int64_t mg_sort_workspace_bytes(int64_t n);

/* Stable LSD radix sort of (uint64 key, int32 value) pairs on bits
 * [begin_bit, end_bit) of the key, 8 bits per pass. Equal keys keep their
 * input order. Output goes to keys_out/vals_out; keys_in/vals_in are used as
 * ping-pong buffers and are clobbered. Replaces torch.argsort(keys) plus the
 * gather of ids (metal_backend.py:256-258). */
int32_t mg_sort_pairs_u64(uint64_t *keys_in, int32_t *vals_in,
                          uint64_t *keys_out, int32_t *vals_out, int64_t n,
                          int32_t begin_bit, int32_t end_bit, void *workspace,
                          int64_t workspace_bytes, mg_stream_t stream);

/* Bytes of scratch mg_sort_pairs_by_tile needs for n pairs over n_tiles. */
int64_t mg_sort_pairs_by_tile_workspace_bytes(int64_t n, int32_t n_tiles);

/* Stable counting sort of n (tile, id) pairs by tile, 0 < n < 2^31,
 * 1 <= n_tiles <= 4096: ids_out gets the ids in (tile, input position) order
 * and tile_offsets (n_tiles + 1,) the start of each tile's run, the last
 * entry the count of pairs with tile < n_tiles (pairs with a larger tile are
 * dropped). tiles must be 16-byte aligned. One pass over the pairs; the
 * tile-id sort of mg_bin_lists_finish.
 * With pairs emitted in depth order it replaces the argsort of the 64-bit
 * (tile << 32 | depth) keys and the searchsorted of the tile ranges
 * (metal_backend.py:256-260). */
int32_t mg_sort_pairs_by_tile(int64_t n, const uint32_t *tiles,
                              const int32_t *ids, int32_t n_tiles,
                              int32_t *ids_out, int32_t *tile_offsets,
                              void *workspace, int64_t workspace_bytes,
                              mg_stream_t stream);

/* tile_offsets[t] = first index i with (keys[i] >> 32) >= t, for
 * t = 0..n_tiles; keys sorted. Replaces keys >> 32 plus torch.searchsorted
 * (metal_backend.py:257-260). tile_offsets: (n_tiles + 1,) int32. */
int32_t mg_tile_ranges(const uint64_t *sorted_keys, int64_t n,
                       int32_t n_tiles, int32_t *tile_offsets,
                       mg_stream_t stream);

/* Tile lists: the whole of build_tile_lists_metal (metal_backend.py:217-285)
 * in two calls around the one host read of the intersection total.
 *
 * begin: per-Gaussian tile counts (the exact ellipse test, as mg_bin_count)
 * and their exclusive scan, then one synchronous host read of the
 * intersection total, which goes to total_host (host) when not NULL; the
 * stream is always synchronised once. The workspace
 * (mg_bin_lists_workspace_bytes(N), about 72 bytes per Gaussian: its count,
 * walk record, claimed tiles, and the claims of rectangles over 32 tiles as
 * one 64-bit word per walk step) carries state to finish and must not be
 * touched in between.
 *
 * finish: emits each Gaussian's (tile id, Gaussian id) pairs, Gaussian by
 * Gaussian, sorts them stably by tile id (up to 4096 tiles a one-pass
 * counting sort, as mg_sort_pairs_by_tile; beyond, radix passes on
 * ceil(log2(tiles_x*tiles_y)) bits), then sorts every tile's list stably by
 * the depth's float bits, and writes gauss_ids (total,) and tile_offsets
 * (tiles_x*tiles_y + 1,). The result equals a stable sort of the
 * (tile << 32 | depth bits) keys of mg_bin_write by mg_sort_pairs_u64: order
 * (tile, depth, Gaussian id). Same arguments as begin, plus its workspace,
 * the total, and a scratch of mg_bin_lists_finish_workspace_bytes(total). */
int64_t mg_bin_lists_workspace_bytes(int64_t N);
int64_t mg_bin_lists_finish_workspace_bytes(int64_t total);
int32_t mg_bin_lists_begin(int64_t N, const float *uv, const float *rxy,
                           const float *conic, const float *opacity,
                           const int32_t *valid, const float *depth, int32_t W,
                           int32_t H, int32_t tile, int32_t tiles_x,
                           int32_t tiles_y, void *workspace,
                           int64_t workspace_bytes, int64_t *total_host,
                           mg_stream_t stream);
int32_t mg_bin_lists_finish(int64_t N, const float *uv, const float *rxy,
                            const float *conic, const float *opacity,
                            const int32_t *valid, const float *depth, int32_t W,
                            int32_t H, int32_t tile, int32_t tiles_x,
                            int32_t tiles_y, const void *workspace,
                            int64_t workspace_bytes, int64_t total,
                            int32_t *gauss_ids, int32_t *tile_offsets,
                            void *finish_workspace,
                            int64_t finish_workspace_bytes, mg_stream_t stream);

/* Tile lists with no host read: the lists of mg_bin_lists_begin + _finish,
 * built in one call into buffers sized by the caller's capacity, so that a
 * render (or a training step) can be enqueued, or captured, whole. The
 * intersection total stays on the device: status (device, 2 int64) receives
 * status[0] = the total and status[1] = 1 if it exceeds capacity, else 0.
 * Within capacity, gauss_ids[0 .. total) and tile_offsets equal the two-call
 * result; past it every list is empty (tile_offsets all 0) and the caller
 * renders again with capacity >= status[0]. Entries of gauss_ids past the
 * kept pairs (all of them after an overflow) are unspecified (past 4096
 * tiles the sort uses the buffer as scratch). gauss_ids: (capacity,), may
 * be NULL when capacity is 0; tile_offsets: (tiles_x*tiles_y + 1,); one
 * workspace of mg_bin_lists_capped_workspace_bytes(N, capacity) bytes.
 * status_host (NULL, or 3 int64 of host memory the device can write, e.g.
 * from hipHostMalloc) receives the same two words and then tag in
 * status_host[2] with a system-scope release, so the host can wait for the
 * words by polling for the tag, with no copy or event on the stream.
 * block_work (device, ceil(N/256) int32, or NULL) orders the count and write
 * passes' blocks of 256 Gaussians heaviest first (mg_preprocess_forward_mip
 * writes it); any contents give the same lists, they only reorder the work.
 * Replaces the .item() read that sizes the reference's pair buffers
 * (metal_gauss/metal_backend.py:246-248) with a device-side check. */
int64_t mg_bin_lists_capped_workspace_bytes(int64_t N, int64_t capacity);
int32_t mg_bin_lists_capped(int64_t N, const float *uv, const float *rxy,
                            const float *conic, const float *opacity,
                            const int32_t *valid, const float *depth, int32_t W,
                            int32_t H, int32_t tile, int32_t tiles_x,
                            int32_t tiles_y, int64_t capacity,
                            int32_t *gauss_ids, int32_t *tile_offsets,
                            int64_t *status, int64_t *status_host,
                            int64_t tag, void *workspace,
                            int64_t workspace_bytes, const int32_t *block_work,
                            mg_stream_t stream);

/* -------------------------------------------------------------- rasteriser */

/* Front-to-back compositing, one workgroup per tile, one thread per pixel.
 * Replaces rasterize_forward (metal_gauss/csrc/rasterize.mm:79-113; kernel
 * rasterize.metal:61-167). t_min is the per-pixel stop transmittance (the
 * reference hard-codes 1e-4, rasterize.metal:149); 0 disables early stop.
 * out_stop holds the stop INDEX into gauss_ids (the reference's n_contrib).
 * background (host, 3 floats, or NULL) blends the colour in the kernel:
 * rgb += max(1 - alpha, 0) * background, the torch glue of
 * metal_backend.py:539-541 (out_alpha stays the coverage).
 *
 * chunk_ws (device, or NULL) enables the chunked backward: the forward plans
 * one backward work unit per 512 list entries of each tile and records each
 * pixel's state at every unit's end, so mg_rasterize_backward can run the
 * units in parallel instead of one long chain per tile. Size it with
 * mg_rasterize_chunk_workspace_bytes(n_isect, tiles, tile), where n_isect
 * is the length of gauss_ids, and pass it unchanged to the backward.
 *
 * zero_grads (device, 16-byte aligned, or NULL): the (N,10) gradient record
 * buffer a later mg_rasterize_backward will fill, cleared by this launch's
 * workgroups on the way (then pass grads_zeroed = 1 to the backward, which
 * skips its own fill).
 *
 * sched (device int32, mg_rasterize_sched_ints(W, H, tile) of them, or NULL)
 * is a backward schedule: the forward records in its first half, per
 * workgroup, the tile's walk length (its largest stop index minus its first
 * entry; -1 for a workgroup without a tile), and a backward given the same
 * buffer runs its tiles longest walk first (see mg_rasterize_backward). It
 * changes no result of the forward. */
int64_t mg_rasterize_chunk_workspace_bytes(int64_t n_isect, int32_t n_tiles,
                                           int32_t tile);
int64_t mg_rasterize_sched_ints(int32_t W, int32_t H, int32_t tile);
int32_t mg_rasterize_forward(
    int64_t N, const float *uv, const float *conic, const float *opacity,
    const float *color, const int32_t *gauss_ids, const int32_t *tile_offsets,
    int32_t W, int32_t H, int32_t tile, int32_t tiles_x, float t_min,
    const float *background, int64_t n_isect, void *chunk_ws,
    int64_t chunk_ws_bytes, float *out_rgb, float *out_alpha, float *out_T,
    int32_t *out_stop, float *zero_grads, int32_t *sched, mg_stream_t stream);

/* Back-to-front replay of mg_rasterize_forward. Replaces rasterize_backward
 * (metal_gauss/csrc/rasterize.mm:147-194; kernel rasterize.metal:173-340),
 * whose five gradient tensors come back here as one record of 10 floats per
 * Gaussian in d_grads (N,10), overwritten: d_uv (slots 0-1), d_conic (2-4),
 * d_opacity (5), d_color (6-8) and, when absgrad != 0, the per-pixel sum of
 * |d_uv| (9; the reference's absgrad statistic; 0 otherwise). The record
 * layout lets the kernel's cross-tile float atomics update one record with
 * consecutive lanes; strided views give the five tensors (see
 * mg_preprocess_backward's grad_stride). grad_alpha may be NULL
 * (a zero gradient, when the coverage is not used). With the forward's
 * background (host, or NULL), grad_rgb is the gradient of the blended colour
 * and alpha (the forward's out_alpha, device) adds the blend's share to
 * grad_alpha. n_isect / chunk_ws / chunk_ws_bytes are the forward's (chunk_ws
 * NULL: one workgroup per tile). grads_zeroed != 0: d_grads was cleared by the
 * forward (its zero_grads), so the backward does not fill it first; 0: the
 * backward zero-fills d_grads itself. sched (or NULL) is the buffer the
 * forward recorded the walk lengths in: the backward first orders each XCD's
 * tiles by them, longest first (a counting sort on the length, exact below
 * 768 entries, in bins of 32 above; tiles of one bin in no fixed order), into
 * the buffer's second half, and its workgroups take the tiles in that order,
 * which shortens the kernel's tail. No effect with chunk_ws, or past 8192
 * workgroups (1024 per XCD). The gradients are the same up to the order of
 * the float atomics, whatever the buffer holds (contents the forward did not
 * write only change the order). */
int32_t mg_rasterize_backward(
    int64_t N, const float *uv, const float *conic, const float *opacity,
    const float *color, const int32_t *gauss_ids, const int32_t *tile_offsets,
    const float *final_T, const int32_t *stop, const float *grad_rgb,
    const float *grad_alpha, const float *alpha, const float *background,
    int64_t n_isect, const void *chunk_ws, int64_t chunk_ws_bytes, int32_t W,
    int32_t H, int32_t tile, int32_t tiles_x, float *d_grads, int32_t absgrad,
    int32_t grads_zeroed, int32_t *sched, mg_stream_t stream);

/* ------------------------------------------------------------------- Adam */

/* One Adam step on one flat tensor, torch's formula with eps after the
 * sqrt(bias_correction2) divide. Replaces adam_step
 * (metal_gauss/csrc/rasterize.mm:329-360; kernel adam.metal:25-42). */
int32_t mg_adam_step(float *p, const float *g, float *m, float *v, int64_t n,
                     double lr, double beta1, double beta2, double eps,
                     int64_t step, mg_stream_t stream);

/* One Adam step on up to 32 flat tensors in ONE launch. Host arrays of length
 * count: p/g/m/v pointers, element counts, lr, and each tensor's step count
 * after this update. Hyperparameters are doubles: the bias corrections and
 * step sizes are formed in double on the host (rasterize.mm:338-342); the
 * moment updates use fp32 betas. eps_inside != 0 selects the
 * p -= lr*sqrt(bc2)/bc1 * m/(sqrt(v)+eps) placement used by
 * selective_adam.py:206 for dense groups. Replaces the per-tensor loop of
 * FusedAdam.step (fused_adam.py:31-54). */
int32_t mg_adam_step_multi(int32_t count, float *const *p,
                           const float *const *g, float *const *m,
                           float *const *v, const int64_t *n,
                           const double *lr, const int64_t *step, double beta1,
                           double beta2, double eps, int32_t eps_inside,
                           mg_stream_t stream);

/* mg_adam_step_multi that does nothing when skip[1] != 0, skip (device, 2
 * int64) being the status of capacity-bounded tile lists
 * (mg_bin_lists_capped): the step of a render whose lists overflowed leaves
 * every parameter and moment as it was, to be run again. No counterpart in
 * the reference, whose tile lists are sized by a host read. */
int32_t mg_adam_step_multi_guarded(int32_t count, float *const *p,
                                   const float *const *g, float *const *m,
                                   float *const *v, const int64_t *n,
                                   const double *lr, const int64_t *step,
                                   double beta1, double beta2, double eps,
                                   int32_t eps_inside, const int64_t *skip,
                                   mg_stream_t stream);

/* Row-masked Adam with a per-row float step count, over up to 32 tensors in
 * one launch. Tensor k has rows[k] rows of width[k] floats; rows r with
 * r < n_visible and visible[r] != 0 get steps[r] += 1 and
 * p -= lr * sqrt(1-b2^k)/(1-b1^k) * m/(sqrt(v)+eps); other rows keep their
 * values. visible: (n_visible,) uint8 (torch.bool). When p, g, m, v and
 * steps are 16-byte aligned, rows that keep their values may be stored back
 * unchanged (whole-line writes), so no two tensors may share p, m, v or
 * steps, and nothing else may write them during the call. The reference has no
 * kernel for this; it replaces SelectiveAdam._step_indexed / _step_masked
 * (selective_adam.py:116-187). */
int32_t mg_selective_adam_step(int32_t count, float *const *p,
                               const float *const *g, float *const *m,
                               float *const *v, float *const *steps,
                               const int64_t *rows, const int32_t *width,
                               const float *lr, const uint8_t *visible,
                               int64_t n_visible, double beta1, double beta2,
                               double eps, mg_stream_t stream);

/* mg_selective_adam_step that does nothing (step counts included) when
 * skip[1] != 0, skip (device, 2 int64) being the status of capacity-bounded
 * tile lists (mg_bin_lists_capped). No counterpart in the reference. */
int32_t mg_selective_adam_step_guarded(int32_t count, float *const *p,
                                       const float *const *g, float *const *m,
                                       float *const *v, float *const *steps,
                                       const int64_t *rows, const int32_t *width,
                                       const float *lr, const uint8_t *visible,
                                       int64_t n_visible, double beta1,
                                       double beta2, double eps,
                                       const int64_t *skip, mg_stream_t stream);

/* ------------------------------------------------------------------- SSIM */

/* The five SSIM entry points of the reference, same math and layouts
 * (metal_gauss/csrc/rasterize.mm:383-461; kernels ssim.metal:23-188). x, y
 * are (H,W,3); stacks are (15,H,W) with channels x,y,xx,yy,xy (x3 colours);
 * w is the 11-tap window (device, 11 floats). */
int32_t mg_ssim_stack_blur_h(const float *x, const float *y, const float *w,
                             int32_t H, int32_t W, float *out,
                             mg_stream_t stream);
int32_t mg_ssim_blur15(const float *src, const float *w, int32_t dir,
                       int32_t H, int32_t W, float *out, mg_stream_t stream);
int32_t mg_ssim_tail_forward(const float *b, int32_t H, int32_t W,
                             float *out, mg_stream_t stream);
int32_t mg_ssim_tail_backward(const float *b, const float *gout, int32_t H,
                              int32_t W, float *gb, mg_stream_t stream);
int32_t mg_ssim_chain_backward(const float *x, const float *y,
                               const float *d_stack, int32_t H, int32_t W,
                               float *d_x, mg_stream_t stream);

/* Fused SSIM: one pass builds the five moments, blurs both ways in LDS and
 * evaluates SSIM; it writes the mean SSIM to mean_out (device, 1 float) and
 * the three unscaled adjoint maps (9,H,W) the backward needs to partials.
 * No counterpart in the reference, which runs the five kernels above
 * (train.py:86-105). Scratch: mg_ssim_fused_workspace_bytes(H, W). */
int64_t mg_ssim_fused_workspace_bytes(int32_t H, int32_t W);
int32_t mg_ssim_fused_forward(const float *x, const float *y, const float *w,
                              int32_t H, int32_t W, float *partials,
                              float *mean_out, void *workspace,
                              int64_t workspace_bytes, mg_stream_t stream);
/* d_x = scale * (blur(partials) chained through the moments), scale read
 * from the device scalar scale_dev (the upstream gradient of the mean). */
int32_t mg_ssim_fused_backward(const float *x, const float *y, const float *w,
                               const float *partials, const float *scale_dev,
                               int32_t H, int32_t W, float *d_x,
                               mg_stream_t stream);

/* The trainer's photometric loss in the fused SSIM pass: replaces
 * l1 = (rgb - gt).abs().mean(); loss = 0.8 * l1 + 0.2 * (1 - ssim(rgb, gt))
 * (metal_gauss/train.py:389-390), with ssim_weight the 0.2. The forward
 * writes out[0] = loss, out[1] = the L1 mean, out[2] = the SSIM mean (device,
 * 3 floats) and the same partials as mg_ssim_fused_forward; its workspace is
 * mg_ssim_fused_workspace_bytes(H, W). The backward writes d_x = grad_dev[0] *
 * d loss / d x, with the L1 term's derivative sign(x - y) taken as 0 where
 * x == y (torch's abs). */
int32_t mg_photometric_loss_forward(const float *x, const float *y,
                                    const float *w, int32_t H, int32_t W,
                                    float ssim_weight, float *partials,
                                    float *out, void *workspace,
                                    int64_t workspace_bytes,
                                    mg_stream_t stream);
/* mg_photometric_loss_forward without a workspace argument: the block sums
 * live in a static device array of the library (2 MiB per GPU, held until
 * the process ends), so the call allocates nothing and takes no scratch from
 * the caller. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops). Limit: 2^18 blocks of 32x16 pixels and one colour, e.g. an image
 * of 8192x5440; larger ones are refused with MG_ERR_ARG. The array keeps
 * the last call's contents; calls that overlap on one GPU race on it. */
int32_t mg_photometric_loss_forward_noalloc(const float *x, const float *y,
                                            const float *w, int32_t H, int32_t W,
                                            float ssim_weight, float *partials,
                                            float *out, mg_stream_t stream);
int32_t mg_photometric_loss_backward(const float *x, const float *y,
                                     const float *w, const float *partials,
                                     const float *grad_dev, int32_t H,
                                     int32_t W, float ssim_weight, float *d_x,
                                     mg_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MGAUSS_H */
