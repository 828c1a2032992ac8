/* gsraster.h — C ABI of the MI355X (gfx950) differentiable Gaussian-splatting
 * rasterizer, libgsraster.so.
 *
 * Plain pointers and sizes only.  Every tensor argument is a DEVICE pointer
 * to contiguous fp32 / int32 data in the layouts of the reference's
 * custom_rasterizer_cuda extension (kmurungi/custom-3dgs-cuda):
 *   mu [N,3], q [N,4] (w,x,y,z; 16-byte aligned), s [N,3] log-scales,
 *   rot [3,3] row-major world-to-camera rows, trans [3],
 *   mean2d [N,2], cov2d [N,3] = (a, b, c) of [[a, b], [b, c]], depth [N],
 *   albedo [N,3], k_j [N,15,3], colors [N,3], alpha [N] post-sigmoid,
 *   img [H,W,3], final_T [H,W], n_contrib [H,W] int32,
 *   sorted_ids [M] int32, tile_ranges [T,2] int32, T = ceil(W/16)*ceil(H/16).
 * `stream` is a hipStream_t (NULL = the null stream); all work is enqueued
 * on it.  Only gsr_rasterize_bin (for the pair count) and gsr_rasterize_status
 * wait on it.
 *
 * Every entry point returns GSR_OK or an error code; gsr_last_error() gives
 * the calling thread's message for the last failure.  Outputs are fully
 * written by the call (no zero-initialisation by the caller is needed).
 *
 * Device errors.  A kernel that reaches its bounded look-back wait, or finds
 * counts that disagree with the binning, exits normally and ORs a bit into
 * its device's status word (its outputs are then invalid).  Calls do not
 * synchronize to look at it: gsr_rasterize_bin reads and clears it with the
 * pair count it waits for anyway, so it reports GSR_ERR_DEVICE for every
 * kernel queued on the device before it (an earlier frame's sorts, binning or
 * backward); gsr_rasterize_status synchronizes and reports the rest.
 */
#ifndef GSRASTER_H
#define GSRASTER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GSR_OK 0
#define GSR_ERR_INVALID_ARGUMENT 1 /* null pointer, bad size, misaligned q */
#define GSR_ERR_HIP 2              /* a HIP runtime call or launch failed */
#define GSR_ERR_WORKSPACE 3        /* workspace smaller than the size query */
#define GSR_ERR_TOO_MANY_PAIRS 4   /* M > 2^31 - 2^16 (the int32 sorted_ids limit, less headroom) */
#define GSR_ERR_DEVICE 5           /* a kernel reported an error (spin bound, bad counts) */

const char* gsr_last_error(void);
const char* gsr_version(void);
/* Build identification, no counterpart in the reference: "file=hash;..." with
 * the first 16 hex digits of the sha256 of each source file the library was
 * built from (empty when the build recorded none).  Measurements record it so a
 * later run can tell whether the kernels it measured have changed. */
const char* gsr_build_sources(void);

/* Replaces project_gaussians_to_2d (csrc/forward/projection.h:5,
 * launcher csrc/forward/projection.cu:109-153; bound as `project` at
 * csrc/bindings.cpp:12-29,142).  Culled Gaussians (camera z <= 0.2) get zero
 * mean, covariance and depth. */
int gsr_project(int n, const float* mu, const float* q, const float* s, const float* rot,
                const float* trans, float fx, float fy, float cx, float cy, float* mean2d,
                float* cov2d, float* depth, void* stream);

/* The autograd glue's approximate screen radii for densification
 * (gaussian_splatting/rasterizer/rasterize.py:49-53, torch ops there): one
 * kernel with the same fp32 operations in the same order. */
int gsr_screen_radii(int n, const float* cov2d, float* radii, void* stream);

/* The glue's camera position -R^T t (rasterize.py:43-44, a torch matmul there),
 * from device pointers to R [3,3] row-major and t [3]. */
int gsr_camera_position(const float* rot, const float* trans, float* cam_pos, void* stream);

/* Replaces launch_spherical_harmonics_kernel (csrc/forward/SH.h:4,
 * csrc/forward/SH.cu:95-131; bound as `SH` at csrc/bindings.cpp:32-46,143).
 * cam_pos is a device pointer to 3 floats (the reference copies it to the
 * host first).  k_j [N,15,3] must be 16-byte aligned. */
int gsr_sh(int n, const float* cam_pos, const float* mu, const float* albedo, const float* k_j,
           float* colors, void* stream);

/* No counterpart in the reference: its autograd glue's forward head
 * (gaussian_splatting/rasterizer/rasterize.py:42-54: camera position, project,
 * the screen radii, SH) in one kernel, for callers that run the whole
 * pipeline.  Every output is bit for bit what gsr_camera_position,
 * gsr_project, gsr_screen_radii and gsr_sh give: mean2d [N,2], cov2d [N,3],
 * depth [N], radii [N], colors [N,3] and cam_pos [3] (device pointers).
 * alpha_logits (may be NULL): opacity logits [N]; opacity [N] then receives
 * the glue's t.sigmoid(alpha) (rasterize.py:149), as torch computes it in
 * fp32 (1 / (1 + exp(-x)) with the device expf).  q and k_j must be 16-byte
 * aligned. */
int gsr_project_sh(int n, const float* mu, const float* q, const float* s, const float* rot,
                   const float* trans, float fx, float fy, float cx, float cy,
                   const float* albedo, const float* k_j, float* mean2d, float* cov2d,
                   float* depth, float* radii, float* colors, float* cam_pos,
                   const float* alpha_logits, float* opacity, void* stream);

/* Replaces launch_rasterization (csrc/forward/rasterize.h:11,
 * csrc/forward/rasterize.cu:284-487; bound as `rasterize` at
 * csrc/bindings.cpp:50-70,144), split where the reference itself reads the
 * pair count back to the host (rasterize.cu:382-390):
 *   1. gsr_rasterize_bin: per-Gaussian tile rectangles and counts, the depth
 *      order; writes M to *num_pairs (waits for the pair count on `stream`;
 *      the depth sort may still be running on the stream when it returns).
 *   2. gsr_rasterize_render: tile binning (sorted ids, tile ranges), blend.
 * bin_ws (gsr_bin_workspace_bytes) must stay untouched between the calls;
 * sort_ws is sized by gsr_sort_workspace_bytes(M, ...).  sorted_keys
 * (optional, may be NULL) receives the reference's 64-bit sort keys
 * (tile << 32 | float bits of depth) in sorted order. */
size_t gsr_bin_workspace_bytes(int n, int height, int width);
int gsr_rasterize_bin(int n, const float* depth, const float* mean2d, const float* cov2d,
                      int height, int width, void* bin_ws, size_t bin_ws_bytes,
                      int64_t* num_pairs, void* stream);
size_t gsr_sort_workspace_bytes(int64_t num_pairs, int n, int height, int width);
int gsr_rasterize_render(int n, const float* depth, const float* mean2d, const float* cov2d,
                         const float* colors, const float* alpha, int height, int width,
                         void* bin_ws, size_t bin_ws_bytes, int64_t num_pairs, void* sort_ws,
                         size_t sort_ws_bytes, int32_t* sorted_ids, int32_t* tile_ranges,
                         float* img, float* final_T, int32_t* n_contrib, uint64_t* sorted_keys,
                         void* stream);

/* No counterpart in the reference (its int32 lists cap a frame's pairs; the
 * screen-band path renders larger frames band by band).  For callers that
 * rasterize several screen bands of one frame:
 *   gsr_depth_order writes order[0 .. n) = every Gaussian, visible or not,
 *   stably sorted by the float bits of depth[i] (as unsigned); a band's
 *   visible Gaussians then appear in it in the order the reference's
 *   (tile << 32 | depth bits) sort gives them (rasterize.cu:423-435), ties by
 *   index.  ws is sized by gsr_depth_order_workspace_bytes(n).
 *   gsr_rasterize_bin_ordered is gsr_rasterize_bin with that order given
 *   instead of computed (no depth keys, no depth sort); `order` must be a
 *   permutation of [0, n) and stays read-only.  gsr_rasterize_render follows
 *   as usual. */
size_t gsr_depth_order_workspace_bytes(int n);
int gsr_depth_order(int n, const float* depth, void* ws, size_t ws_bytes, int32_t* order,
                    void* stream);
int gsr_rasterize_bin_ordered(int n, const int32_t* order, const float* mean2d,
                              const float* cov2d, int height, int width, void* bin_ws,
                              size_t bin_ws_bytes, int64_t* num_pairs, void* stream);

/* No counterpart in the reference (depth-prefix rendering of screen bands):
 * gsr_rasterize_render with tile_skip (device, one byte per tile of the
 * height x width screen, row-major): the lists of tiles marked nonzero may be
 * left empty (their ranges (0, 0), their pixels then blend nothing); every
 * other tile's list, range offsets aside, and its image, final_T and n_contrib
 * are gsr_rasterize_render's.  The block binning leaves them empty, so the
 * lists hold fewer than num_pairs entries (sorted_ids keeps its num_pairs
 * room); the tile-sort binning (screens beyond 8192 8x8-tile blocks) builds
 * them as usual. */
int gsr_rasterize_render_skip(int n, const float* depth, const float* mean2d, const float* cov2d,
                              const float* colors, const float* alpha, int height, int width,
                              void* bin_ws, size_t bin_ws_bytes, int64_t num_pairs,
                              void* sort_ws, size_t sort_ws_bytes, const uint8_t* tile_skip,
                              int32_t* sorted_ids, int32_t* tile_ranges, float* img,
                              float* final_T, int32_t* n_contrib, void* stream);
/* Synchronizes `stream`, then reads and clears the current device's status
 * word: GSR_ERR_DEVICE if a kernel queued on the device since the status was
 * last read hit its look-back spin bound or found inconsistent counts.
 * bin_ws is not read (it may be NULL); the status is per device. */
int gsr_rasterize_status(void* bin_ws, size_t bin_ws_bytes, void* stream);

/* Test hook (no counterpart in the reference): ORs `bits` (> 0) into the
 * current device's status word from a one-thread kernel on `stream`, as a
 * kernel that hit its spin bound would, so that callers can test their
 * handling of GSR_ERR_DEVICE. */
int gsr_debug_raise_status(int bits, void* stream);

/* Measurement support (no counterpart in the reference): launches one VALU
 * issue-rate calibration kernel on `stream`.  kind: 0 v_add_f32, 1 v_fma_f32,
 * 2 v_exp_f32, 3 v_permlane32/16_swap, 4 v_add_f32 with a DPP row rotate;
 * every lane runs 8 independent chains of `iters` (1..65536) steps, and the
 * grid is gsr_calibrate_valu_out_floats() / 256 work-groups of 256 threads,
 * each thread storing one float to `out`.  rocprofv3 issue counters of these
 * kernels give the practical VALU ceiling that bench.py reads the blends
 * against. */
size_t gsr_calibrate_valu_out_floats(void);
int gsr_calibrate_valu(int kind, int iters, float* out, void* stream);

/* No counterpart in the reference (whose frames are limited to int32 pair
 * lists): the (Gaussian, tile) pairs of each tile row of a height x width
 * frame, rows[r] for r < ceil(height / 16), counted from each Gaussian's tile
 * rectangle exactly as gsr_rasterize_bin counts them; for planning screen
 * bands of at most a given number of pairs.  `rows` (device) needs
 * ceil(height / 16) + 1 entries of room; height <= 65535. */
int gsr_tile_row_pairs(int n, const float* mean2d, const float* cov2d, int height, int width,
                       uint64_t* rows, void* stream);

/* No counterpart in the reference (screen-band support, like
 * gsr_tile_row_pairs): flags[i] = 1 when Gaussian i's tile rectangle, formed
 * as gsr_rasterize_bin forms it on the height x width frame and widened by one
 * tile row above and below, holds a marked tile, else 0.  `sat` (device) is
 * the summed-area table of the marked tiles: (ceil(height / 16) + 1) x
 * (ceil(width / 16) + 1) int32, row-major, its first row and column zero.  The
 * widening makes the flagged set cover every Gaussian that a render of a band
 * of whole tile rows (means moved up by the band's first row) bins into a
 * marked tile. */
int gsr_tiles_touch(int n, const float* mean2d, const float* cov2d, int height, int width,
                    const int32_t* sat, uint8_t* flags, void* stream);

/* Replaces launch_backward_rasterization (csrc/backward/rasterize_backward.h:5,
 * csrc/backward/rasterize_backward.cu:239-309; bound as
 * `backwards_rasterization` at csrc/bindings.cpp:72-100,147).  num_pairs is
 * the length of sorted_ids (tile ranges are clamped to it); ids outside
 * [0, n) are skipped as in the reference.  Outputs: d_mean2d [N,2],
 * d_cov2d [N,3] (dL/d(a,b,c)), d_colors [N,3], d_alpha [N].  The workspace
 * (about 36 B per pair plus 68 B per Gaussian) holds the blend records, the
 * per-tile schedule and one gradient slot per (Gaussian, tile) pair: the
 * per-tile sums are written to their slots and summed per Gaussian, with no
 * float atomics, so the result does not depend on scheduling. */
size_t gsr_backward_workspace_bytes(int n, int64_t num_pairs, int height, int width);
int gsr_rasterize_backward(int n, int height, int width, const float* grad_img,
                           const float* mean2d, const float* cov2d, const float* colors,
                           const float* alpha, const int32_t* sorted_ids, int64_t num_pairs,
                           const int32_t* tile_ranges, const float* final_T,
                           const int32_t* n_contrib, void* ws, size_t ws_bytes, float* d_mean2d,
                           float* d_cov2d, float* d_colors, float* d_alpha, void* stream);

/* No counterpart in the reference (its binding requires a contiguous
 * grad_output, and its glue copies one with .contiguous(),
 * rasterize.py:85-86): gsr_rasterize_backward with dL/dimage given as a
 * strided view, pixel (y, x) channel c at grad_img[y * grad_stride_h +
 * x * grad_stride_w + c * grad_stride_c] (element strides, any sign; all zero
 * for the broadcast gradient of image.sum()), so no contiguous copy is made.
 * Results are bit for bit those of gsr_rasterize_backward on the same values. */
int gsr_rasterize_backward_strided(int n, int height, int width, const float* grad_img,
                                   int64_t grad_stride_h, int64_t grad_stride_w,
                                   int64_t grad_stride_c, const float* mean2d,
                                   const float* cov2d, const float* colors, const float* alpha,
                                   const int32_t* sorted_ids, int64_t num_pairs,
                                   const int32_t* tile_ranges, const float* final_T,
                                   const int32_t* n_contrib, void* ws, size_t ws_bytes,
                                   float* d_mean2d, float* d_cov2d, float* d_colors,
                                   float* d_alpha, void* stream);

/* No counterpart in the reference (whose frames are limited to int32 pair
 * lists): gsr_rasterize_backward_strided that adds its gradients to what
 * d_mean2d, d_cov2d, d_colors and d_alpha hold instead of overwriting them,
 * for frames rendered as screen bands (one call per band into one set of
 * outputs).  Each Gaussian's band total is added once, so the result is bit
 * for bit the sum of the separate calls' outputs, added band by band, unless
 * list entries without a gradient slot (pairs outside the Gaussian's tile
 * rectangle, repeated ids) fall back to float atomics. */
int gsr_rasterize_backward_accumulate(int n, int height, int width, const float* grad_img,
                                      int64_t grad_stride_h, int64_t grad_stride_w,
                                      int64_t grad_stride_c, const float* mean2d,
                                      const float* cov2d, const float* colors,
                                      const float* alpha, const int32_t* sorted_ids,
                                      int64_t num_pairs, const int32_t* tile_ranges,
                                      const float* final_T, const int32_t* n_contrib, void* ws,
                                      size_t ws_bytes, float* d_mean2d, float* d_cov2d,
                                      float* d_colors, float* d_alpha, void* stream);

/* No counterpart in the reference: gsr_rasterize_backward for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  It takes no workspace: its
 * kernels use a fixed array of GSR_NOALLOC_SCRATCH_BYTES in the library's
 * device memory, one per GPU, held until the process ends.  A frame whose
 * workspace (gsr_backward_workspace_bytes: about 36 B per pair plus 68 B per
 * Gaussian) exceeds it is rejected with GSR_ERR_WORKSPACE.  The call
 * allocates nothing.  Every call on one GPU shares that GPU's array, so calls
 * that overlap on one GPU (other streams, other threads) race; calls queued
 * in order on one stream do not.  Results are bit for bit those of
 * gsr_rasterize_backward. */
#define GSR_NOALLOC_SCRATCH_BYTES (256u << 20)
int gsr_rasterize_backward_noalloc(int n, int height, int width, const float* grad_img,
                                   const float* mean2d, const float* cov2d, const float* colors,
                                   const float* alpha, const int32_t* sorted_ids,
                                   int64_t num_pairs, const int32_t* tile_ranges,
                                   const float* final_T, const int32_t* n_contrib,
                                   float* d_mean2d, float* d_cov2d, float* d_colors,
                                   float* d_alpha, void* stream);

/* Replaces launch_backward_SH (csrc/backward/delight_backward.h:5,
 * csrc/backward/delight_backward.cu:176-218; bound as `backwards_SH` at
 * csrc/bindings.cpp:102-116,148).  cam_pos is a device pointer; k_j and d_k_j
 * must be 16-byte aligned. */
int gsr_sh_backward(int n, const float* colors_grad, const float* mu, const float* albedo,
                    const float* k_j, const float* cam_pos, float* d_albedo, float* d_k_j,
                    float* d_mu, void* stream);

/* Replaces launch_backward_projection (csrc/backward/projection_backward.h:5,
 * csrc/backward/projection_backward.cu:142-187; bound as
 * `backwards_projection` at csrc/bindings.cpp:118-138,149).  cx, cy are
 * accepted and unused, as in the reference.  The quaternion gradient is the
 * derivative of the rotation the forward builds; with the environment
 * variable GSR_REFERENCE_QUAT_GRAD=1 (read on every call) d_q is the
 * reference's literal formula instead (projection_backward.cu:116-127, whose
 * w-multiplied terms carry the opposite sign), bit for bit; d_mu and d_s do
 * not depend on the setting. */
int gsr_project_backward(int n, const float* d_mean2d, const float* d_cov2d, const float* mu,
                         const float* q, const float* s, const float* rot, const float* trans,
                         float fx, float fy, float cx, float cy, float* d_mu, float* d_q,
                         float* d_s, void* stream);

/* No counterpart in the reference: its glue's backward tail
 * (rasterize.py:100-117: backwards_SH, backwards_projection and the sum of
 * their dL/dmu) in one kernel.  d_colors is dL/dcolors (the SH input
 * gradient); d_mu = the projection's dL/dmu + the SH's, in one fp32 addition
 * as the glue does; every output is bit for bit what gsr_sh_backward and
 * gsr_project_backward give (GSR_REFERENCE_QUAT_GRAD applies here too).
 * d_opacity (may be NULL): dL/dopacity [N] and the forward's opacity [N];
 * d_alpha_logits [N] then receives the sigmoid's backward, (d_opacity
 * (1 - opacity)) opacity, as torch's fp32 sigmoid backward.  q, d_q, k_j and
 * d_k_j must be 16-byte aligned. */
int gsr_project_sh_backward(int n, const float* d_mean2d, const float* d_cov2d,
                            const float* d_colors, const float* mu, const float* q,
                            const float* s, const float* rot, const float* trans, float fx,
                            float fy, const float* albedo, const float* k_j,
                            const float* cam_pos, float* d_mu, float* d_q, float* d_s,
                            float* d_albedo, float* d_k_j, const float* d_opacity,
                            const float* opacity, float* d_alpha_logits, void* stream);

/* Replaces the trainer's loss, calculate_loss (gaussian_splatting/utils/
 * loss.py:12-33): (1 - lambda_dssim) mean|gt - rendered| + lambda_dssim
 * (1 - SSIM(clamp(rendered, 0, 1), clamp(gt, 0, 1))), with torchmetrics'
 * SSIM (loss.py:2, the reference's torchmetrics >= 1.0: 11 x 11 Gaussian
 * window, sigma 1.5, K1 0.01, K2 0.03, data range 1, the windows that lie
 * inside the image).  rendered and gt are [H,W,3] fp32, H and W >= 11 (the
 * window).  gsr_l1_dssim writes out[0] = loss, out[1] = SSIM, out[2] = the L1
 * mean (device floats) and keeps in ws what gsr_l1_dssim_backward needs;
 * the backward writes d_rendered [H,W,3] = *grad_loss * dloss/drendered
 * (grad_loss a device float, NULL for 1), zero through the clamp outside
 * [0, 1] as torch's clamp backward.  ws (gsr_loss_workspace_bytes: 36 B per
 * pixel) must stay untouched between the two calls.  gsr_ssim gives the SSIM
 * alone (out[0] = 1 - SSIM, out[1] = SSIM, out[2] = mean|a - b|; the
 * reference's scripts/eval.py:60). */
size_t gsr_loss_workspace_bytes(int height, int width);
int gsr_l1_dssim(int height, int width, const float* rendered, const float* gt,
                 float lambda_dssim, void* ws, size_t ws_bytes, float* out, void* stream);
int gsr_l1_dssim_backward(int height, int width, const float* rendered, const float* gt,
                          float lambda_dssim, const void* ws, size_t ws_bytes,
                          const float* grad_loss, float* d_rendered, void* stream);
int gsr_ssim(int height, int width, const float* a, const float* b, void* ws, size_t ws_bytes,
             float* out, void* stream);

/* Replaces the trainer's optimizer step and its clamps: torch.optim.Adam
 * (gaussian_splatting/utils/optim.py:12-31: six parameter groups, eps 1e-15,
 * default betas) followed by the clamps of the updated parameters
 * (scripts/train.py:171-176, opacity logits; utils/adc.py:90-93,
 * log-scales), in one pass per element: 16 B read and 12 B written.  Each
 * tensor is fp32 and contiguous on the device; exp_avg / exp_avg_sq are its
 * Adam moments (updated in place), `step` the step number after this update
 * (1 for the first), lr its group's learning rate; clamp_min / clamp_max bound
 * the updated parameter (-INFINITY / INFINITY for none; NaN stays NaN).
 * The arithmetic is torch's single-tensor Adam's for fp32 tensors: the moments
 * come out bit for bit, the parameter within a few ulps of its operands. */
typedef struct gsr_adam_tensor {
    float* param;
    const float* grad;
    float* exp_avg;
    float* exp_avg_sq;
    int64_t numel;
    double lr;
    int64_t step;
    float clamp_min;
    float clamp_max;
} gsr_adam_tensor;
int gsr_adam_step(int count, const gsr_adam_tensor* tensors, double beta1, double beta2,
                  double eps, void* stream);

/* Replaces the record assembly of the reference's PLY export, save_ply
 * (scripts/run.py:66-165, the official Inria 3DGS point_cloud.ply layout):
 * records [N, 17 + 3K] fp32 on the device, one per Gaussian: x y z, nx ny nz
 * (0), f_dc_0..2 (albedo), f_rest_0..3K-1 channel-major (f_rest[c K + k] =
 * k_j[n][k][c], run.py:98-108), opacity, scale_0..2 (the log-scales), rot_0..3
 * (q / max(|q|, 1e-8), w x y z).  opacity is the stored logit, or with
 * opacity_from_probability log(a / (1 - a)) of a clamped to [1e-6, 1 - 1e-6]
 * (run.py:110-118, a legacy checkpoint holding probabilities).  k_j is
 * [N,K,3], 1 <= K <= 63; q must be 16-byte aligned. */
int gsr_ply_pack(int n, int rest_coeffs, const float* mu, const float* q, const float* s,
                 const float* alpha, const float* albedo, const float* k_j,
                 int opacity_from_probability, float* records, void* stream);

/* Replaces the reference's densification statistics
 * (gaussian_splatting/utils/adc.py:58-87, accumulate_densification_stats and
 * update_max_radii2d): with mean2d_grad [N,2] (may be NULL), its norm, scaled
 * by (width / 2, height / 2) when both are positive, is added to
 * grad_accum [N] and 1 to denom [N] where it is above 0; with radii [N] (may be
 * NULL), max_radii2d = max(max_radii2d, radii), NaN propagating. */
int gsr_adc_stats(int n, const float* mean2d_grad, int width, int height, const float* radii,
                  float* grad_accum, float* denom, float* max_radii2d, void* stream);

/* Replaces the reference's densify / prune pass (utils/adc.py:316-393 with
 * :209-294 and :122-165).  params: the six arrays mu [N,3], q [N,4], s [N,3],
 * alpha [N,1], A [N,3], k_j [N,15,3]; moments: exp_avg of each, then exp_avg_sq
 * of each (NULL entries: no optimizer state yet).  gsr_adc_plan decides every
 * Gaussian's fate and synchronizes to return counts[5]: kept originals, kept
 * clones, kept split sources (two copies each), all split sources, all clone
 * sources; the new cloud holds counts[0] + counts[1] + 2 counts[2] Gaussians.
 * gsr_adc_apply writes it to out_params / out_moments in the reference's order
 * (kept originals, kept clones, kept first split copies, kept second split
 * copies).  split_noise holds 2 counts[3] rows of 3 N(0, 1) values, the draws
 * of the reference's torch.normal (row k counts[3] + j: copy k of the j-th
 * split source).  ws (gsr_adc_workspace_bytes) must stay untouched between the
 * two calls.  Thresholds are rounded to fp32 as torch compares an fp32 tensor
 * with a Python float. */
typedef struct gsr_adc_config {
    double grad_threshold;   /* 0.00005 */
    double percent_dense;    /* 0.01 */
    double scene_extent;
    double min_opacity;      /* 0.01 */
    double max_screen_size;  /* used when has_max_screen_size */
    int has_max_screen_size;
    int densify;             /* allow_densify and N < max_gaussians */
    int prune;               /* allow_densify */
    int reset_opacity;       /* reset_opacity and allow_densify */
} gsr_adc_config;
size_t gsr_adc_workspace_bytes(int n);
int gsr_adc_plan(int n, float* const params[6], const float* grad_accum, const float* denom,
                 const float* max_radii2d, const gsr_adc_config* cfg, void* ws, size_t ws_bytes,
                 int64_t counts[5], void* stream);
int gsr_adc_apply(int n, float* const params[6], float* const moments[12],
                  const float* split_noise, const gsr_adc_config* cfg, const void* ws,
                  size_t ws_bytes, float* const out_params[6], float* const out_moments[12],
                  void* stream);

/* Stage timing (no counterpart in the reference; for benchmarks).  While
 * enabled, each entry point records a pair of HIP events on its stream around
 * its stage's kernels: "project", "sh", "project_sh", "bin_count",
 * "depth_sort", "scan", "records", "tile_binning", "tile_sort", "ranges",
 * "fwd_schedule", "blend_fwd", "bwd_records" (records and slot offsets),
 * "bwd_schedule",
 * "blend_bwd", "grad_reduce", "sh_bwd", "project_bwd", "project_sh_bwd",
 * "loss", "loss_bwd", "adam", "ply_pack", "adc_stats", "adc_plan", "adc_apply".
 * gsr_profile_collect waits for the recorded events
 * and adds their durations to per-stage totals read by gsr_profile_get;
 * gsr_profile_stage(i) names the i-th stage with a total (NULL past the end). */
void gsr_profile_enable(int on);
int gsr_profile_collect(void);
int gsr_profile_get(const char* stage, int64_t* count, double* total_ms);
const char* gsr_profile_stage(int index);
void gsr_profile_reset(void);

#ifdef __cplusplus
}
#endif

#endif /* GSRASTER_H */
