/*
 * gs_raster.h -- C ABI of the MI355X (gfx950) tiled Gaussian-splatting rasterizer.
 *
 * Every entry point takes plain device pointers, sizes and scalars, launches on the
 * HIP stream it is given (a hipStream_t passed as void*, NULL = default stream),
 * performs no host synchronisation and no device allocation, and returns GS_OK or an
 * error code; gs_last_error() then holds a message for the calling thread.
 *
 * Array layouts are the ones the reference's Python functions take and return
 * (row-major, float32 unless stated):
 *   means[N,3]  scales[N,3] (log)  quaternions[N,4] (w,x,y,z, unnormalised)
 *   opacities[N,1] (logit)  sh_coeffs[N,K,3] (coefficient-major, channel-minor)
 *   w2c[4,4] (device)  background[3] (device)  image[H,W,3]
 * The reference is ghif/jax-gs (pure JAX; it has no FFI of its own).  Each entry
 * point below names the reference function whose behaviour it reproduces; a jax.ffi
 * custom call or the ctypes host module in this repository binds to them.
 */
#ifndef GS_RASTER_H
#define GS_RASTER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GS_OK 0
#define GS_ERR_INVALID 1  /* bad shape / size / argument */
#define GS_ERR_HIP 2      /* a HIP runtime call or kernel launch failed */

/* Constants of the reference rasterizer (jax_gs/renderer/rasterizer.py:6-10). */
#define GS_TILE_SIZE 16
#define GS_OFFSET_SIZE 16
#define GS_BLOCK_SIZE 512
#define GS_MAX_TILE_CHUNKS 8
#define GS_MAX_TILE_INTERACTIONS 4096

/* Per-Gaussian compositing record: 12 floats, L = log2(e)
 *   [0]=mean2d.x [1]=mean2d.y [2]=-0.5*ic00*L [3]=-ic01*L [4]=-0.5*ic11*L
 *   [5]=log2(op) [6..8]=colour rgb [9]=op [10]=log2(op) - 10*L [11]=no_cap
 * where op = sigmoid(opacity) and ic = inverse of cov2D with det clamped to 1e-6
 * (rasterizer.py:147-156), so that alpha = exp2([2]dx^2 + [3]dx dy + [4]dy^2 + [5])
 * and the gate power > -10 is exponent > [10]; no_cap = 1.0 when no point that passes the
 * gate can reach the 0.99 alpha cap, the exponent's float32 rounding included (the conic
 * is positive definite and log2(op) plus a bound of that rounding, which grows with the
 * conic's tr^2/det, stays below log2(0.99)), else 0.0.  gs_composite_bwd skips its
 * per-wave cap test only for records holding exactly 1.0 there; any other value is safe.
 * The gradient record produced by gs_composite_bwd holds, with dP = dL/dpower of one
 * (pixel, entry) pair, dx = pixel.x - mean2d.x, dy = pixel.y - mean2d.y, summed over
 * the Gaussian's pairs:
 *   [0]=sum dP dx [1]=sum dP dy [2]=sum dP dx^2 [3]=sum dP dx dy [4]=sum dP dy^2
 *   [5]=sum dP (= op * dL/dop) [6..8]=dL/dcolour [9..11]=0
 * (gs_preprocess_bwd turns these into dL/dmean2d, dL/dic and dL/dopacity). */
#define GS_REC_STRIDE 12

/* Layout of the int32 stats[] array filled by gs_bin (renderer.py:63-90 extras). */
#define GS_STAT_N_INTERACTIONS 0
#define GS_STAT_MAX_PER_TILE 1
#define GS_STAT_OVERFLOW_TILES 2
#define GS_STAT_OVERFLOW_INTERACTIONS 3
#define GS_STAT_TRUNCATED_TILES 4
#define GS_STAT_TRUNCATED_INTERACTIONS 5
#define GS_STAT_RADIUS_CAP_VIOLATIONS 6
#define GS_STAT_NEGATIVE_DEPTH 7   /* Gaussians whose depth has its sign bit set */
#define GS_STAT_CAPACITY_EXCEEDED 8 /* 1 when n_interactions > capacity */
#define GS_STAT_MEAN_PER_TILE 9     /* float32 bits of float(n_interactions) / num_tiles */
#define GS_STAT_TILE_ENTRIES 10     /* entries of tiles 0..T-1 (= ranges[T]); n_interactions also
                                       counts valid slots of negative-depth Gaussians (tile -1) */
#define GS_STAT_WINDOW_CLAMPED 11   /* 1 when a tile's 512-entry chunk starts within 512 slots of the
                                       end of the reference's max(256 n, 512)-slot arrays, i.e. when
                                       its default path (rasterizer.py:184-190) reads other entries */
#define GS_STAT_ENTRIES_DEFERRED 12 /* 1 when gs_bin_deferred left the entry list to
                                       gs_composite_fwd_deferred (0 from every other binning) */
#define GS_NUM_STATS 16

const char* gs_last_error(void);
/* 2: gs_composite_fwd/bwd take the tile order; gs_mse_loss, gs_l1_ssim, gs_adam_step,
 * gs_densify_and_prune, gs_reset_opacities, gs_ply_pack/unpack, gs_preprocess_bwd_adam,
 * gs_l1_ssim_terms.  3: gs_l1_loss_bwd, gs_mse_loss_bwd.  4: gs_composite_fwd takes
 * clear_records, gs_composite_bwd accumulate.  5: gs_composite_fwd takes window_rule.
 * 6: gs_composite_fwd/bwd take a gs_window_t in place of window_rule; gs_window_from_list,
 * gs_window_from_bins; GS_STAT_WINDOW_CLAMPED.  7: gs_preprocess_bwd_w2c, gs_eval_sh,
 * gs_eval_sh_bwd.  8: gs_l1_ssim_window, gs_l1_ssim_window_bwd.  9: compositing records carry
 * a cap flag in slot 11.  10: that flag is no_cap (1.0 = proven below the cap, rounding
 * included; 0.0 = not proven), read by gs_composite_bwd; gs_composite_prep_bwd,
 * gs_project_bwd.  11: gs_bin_deferred, gs_composite_fwd_deferred.  12: the L1 loss fused
 * into compositing: gs_composite_l1_out_size, gs_composite_fwd_deferred_l1,
 * gs_composite_bwd_l1.  13: gs_bin and gs_bin_deferred take the chunk window (the binning
 * builds it; gs_window_from_bins stays for lists binned without it).  14: gs_composite_bwd
 * and gs_composite_bwd_l1 take a gs_clear_list_t; gs_preprocess_bwd and
 * gs_preprocess_bwd_w2c take zeroed. */
int gs_abi_version(void);

/* Projection + covariance + SH colour for every Gaussian.
 * Replaces jax_gs/renderer/projection.py:6-79 (project_gaussians),
 * jax_gs/core/gaussians.py:58-92 (get_covariance_3d), jax_gs/renderer/renderer.py:40-49
 * with jax_gs/renderer/sh.py:25-74 (view directions, eval_sh, +0.5, clip) and the
 * conic/sigmoid preparation of jax_gs/renderer/rasterizer.py:147-156.
 * mask may be NULL (all active).
 * Outputs: means2d[N,2] cov2d[N,2,2] radii[N] valid[N] (0/1) depths[N] colors[N,3]
 * records[N,GS_REC_STRIDE].  records may be NULL; when it is not, cov2d and colors may be
 * NULL (not written: the records carry the conic and colour that compositing reads).  With
 * colors NULL, the SH rows of masked-out Gaussians are not read and their records' colour
 * is that of zero coefficients (0.5): such a Gaussian is never an entry, so no compositing
 * reads it. */
int gs_preprocess_fwd(void* stream, int64_t n, int sh_k, int sh_degree,
                      const float* means, const float* scales, const float* quats,
                      const float* opacities, const float* sh_coeffs, const uint8_t* mask,
                      const float* w2c, int width, int height, float fx, float fy, float cx,
                      float cy, float* means2d, float* cov2d, float* radii, uint8_t* valid,
                      float* depths, float* colors, float* records);

/* Builds compositing records from projected quantities.
 * Replaces the prologue of jax_gs/renderer/rasterizer.py:119-156 (render_tiles):
 * det clamp, inverse covariance, sigmoid(opacity). */
int gs_composite_prep(void* stream, int64_t n, const float* means2d, const float* cov2d,
                      const float* opacities, const float* colors, float* records);

/* The 512 ids a clamped chunk of the reference's default compositing path reads.
 * rasterizer.py:184-190 slices chunk c of tile t at min(start + 512 c, L - 512) of its
 * L-slot arrays, L = max(256 n, 512) (get_tile_interactions, rasterizer.py:84-114); a
 * chunk starting past L - 512 reads the arrays' last 512 slots, which may hold other
 * tiles' entries, the empty slots of the Gaussians (tile T, in (depth quantum, id) order)
 * or the slots of negative-depth Gaussians.  thr is L - 512 in the coordinates of the
 * entry list the compositing launch is given; ids are the arrays' slots L-512..L-1. */
typedef struct {
  int64_t thr;
  int32_t reserved[2];
  int32_t ids[512];
} gs_window_t;

/* Float arrays a compositing backward launch sets to zero on the side, while its
 * arithmetic-bound waves run (16-byte non-temporal stores): up to GS_CLEAR_MAX arrays,
 * ptr[i] with count[i] floats; entries with a NULL ptr or a count of 0 are skipped.  The
 * five gradient arrays of a later gs_preprocess_bwd(..., zeroed = 1) are the intended use:
 * the VJP then writes only the rows of the Gaussians some pixel reached. */
#define GS_CLEAR_MAX 8
typedef struct {
  float* ptr[GS_CLEAR_MAX];
  int64_t count[GS_CLEAR_MAX];
} gs_clear_list_t;

/* Workspace bytes gs_bin needs for n Gaussians, a width x height image and an
 * interaction capacity (capacity <= 0 means the static bound 256*n). */
size_t gs_bin_workspace_size(int64_t n, int width, int height, int64_t capacity);

/* Tile binning: per-Gaussian tile rectangles, quantised 13-bit depth, stable sort
 * by (tile, depth bucket, Gaussian id), tile ranges and the renderer's health stats.
 * Replaces jax_gs/renderer/rasterizer.py:12-116 (get_tile_interactions) and the
 * searchsorted tile ranges + extras of jax_gs/renderer/renderer.py:57-90.
 * Outputs cover only the n_interactions valid entries, in the reference's order:
 *   sorted_gids[capacity]   Gaussian id of entry i
 *   sorted_tiles[capacity]  tile id of entry i (may be NULL)
 *   ranges[T+1]             first entry of tile t (searchsorted-left), ranges[T]=n
 *   stats[GS_NUM_STATS]     see GS_STAT_*
 * With k Gaussians whose depth has its sign bit set, the reference's arrays carry
 * 256*k extra entries in front (tile -1), so its boundaries equal ranges + 256*k.
 * capacity <= 0 selects the static bound 256*n.
 * window (may be NULL) receives the default path's chunk window of this list, what
 * gs_window_from_bins writes, built by the binning's last launch (its threshold, and when
 * GS_STAT_WINDOW_CLAMPED is set, the ids rebuilt from the inputs and the written list). */
int gs_bin(void* stream, int64_t n, const float* means2d, const float* radii,
           const uint8_t* valid, const float* depths, int width, int height,
           int64_t capacity, void* workspace, size_t workspace_bytes, int32_t* sorted_gids,
           int32_t* sorted_tiles, int32_t* ranges, int32_t* stats, gs_window_t* window);

/* Workspace bytes of gs_bin_deferred (gs_bin's and the count sweep's tile masks, 2 KiB
 * per chunk of 256 superblock words). */
size_t gs_bin_deferred_workspace_size(int64_t n, int width, int height, int64_t capacity);

/* gs_bin for the render path, with the entry list deferred to the compositing forward.
 * Same inputs and outputs as gs_bin without sorted_tiles (capacity > 0; the workspace of
 * gs_bin_deferred_workspace_size), except that sorted_gids is written here only when the
 * entries exceed the capacity or the stats set GS_STAT_WINDOW_CLAMPED.  Otherwise
 * gs_composite_fwd_deferred, given this workspace untouched, writes each tile's entries up
 * to those its walk meets, which cover every entry gs_composite_bwd reads (below the
 * tile's largest n_contrib); the rest of the list stays unwritten.  At full size the
 * compositing meets 2-10 % of the entries (tiles turn opaque early), and writing them all
 * was the binning's costliest step.  Same reference interface as gs_bin
 * (rasterizer.py:12-116, renderer.py:57-90). */
int gs_bin_deferred(void* stream, int64_t n, const float* means2d, const float* radii,
                    const uint8_t* valid, const float* depths, int width, int height,
                    int64_t capacity, void* workspace, size_t workspace_bytes, int32_t* sorted_gids,
                    int32_t* ranges, int32_t* stats, gs_window_t* window);

/* gs_bin without a workspace argument and without any allocation: the workspace is a
 * library-owned device array of GS_BIN_STATIC_SCRATCH_BYTES (128 MiB) that every GPU
 * the library runs on holds until the process ends.  No counterpart in the reference
 * (its sort allocates through XLA): it is for callers that cannot allocate, such as
 * code under HIP graph capture or serving loops that forbid hipMalloc.
 * Arguments and outputs as gs_bin; returns GS_ERR_INVALID when
 * gs_bin_workspace_size(n, width, height, capacity) exceeds the array (1080p: about
 * 1.09M Gaussians).  Calls share their GPU's array: calls that overlap on one GPU
 * (other streams or threads) race; calls in stream order do not. */
#define GS_BIN_STATIC_SCRATCH_BYTES ((size_t)128 << 20)
int gs_bin_static(void* stream, int64_t n, const float* means2d, const float* radii,
                  const uint8_t* valid, const float* depths, int width, int height,
                  int64_t capacity, int32_t* sorted_gids, int32_t* sorted_tiles, int32_t* ranges,
                  int32_t* stats);

/* Workspace bytes gs_bin_reference needs. */
size_t gs_bin_reference_workspace_size(int64_t n, int width, int height);

/* The reference's own output arrays of get_tile_interactions, all L = max(256 n, 512)
 * slots in the order of its stable sort of every slot's key (tile << 13) | depth
 * quantum (jax_gs/renderer/rasterizer.py:56-116): the 256 slots of each Gaussian whose
 * depth has its sign bit set (tile -1), then gs_bin's entries, then the remaining
 * 256 - count slots of every other Gaussian (tile T), both runs with Gaussians in
 * (quantum, id) order, then padding (tile T, id 0).  ranges[T+1] are the searchsorted-left
 * boundaries of these arrays (renderer.py:57-61); stats as gs_bin's (n_interactions is the
 * reference's n, which also counts valid slots of negative-depth Gaussians).
 * n < 2^23 (256 n slots indexed with int32). */
int gs_bin_reference(void* stream, int64_t n, const float* means2d, const float* radii,
                     const uint8_t* valid, const float* depths, int width, int height, void* workspace,
                     size_t workspace_bytes, int32_t* sorted_tiles, int32_t* sorted_gids, int32_t* ranges,
                     int32_t* stats);

/* Tile boundaries of an arbitrary sorted tile-id array (length L, entries in
 * [-1, T]): ranges[t] = first index with tile >= t for t in 0..T.
 * Replaces the searchsorted of jax_gs/renderer/renderer.py:57-61 and
 * jax_gs/renderer/rasterizer.py:159-160 for callers that hold sorted ids. */
int gs_tile_ranges(void* stream, const int32_t* sorted_tiles, int64_t length, int num_tiles,
                   int32_t* ranges);


/* Window of a caller list in the reference's layout (sorted_gids of L = n_entries
 * slots, e.g. from get_tile_interactions or gs_bin_reference): thr = L - 512 and the last
 * 512 ids (L < 512, which the reference cannot slice: thr = INT64_MAX, no clamp).
 * Replaces the clip of rasterizer.py:187 for gs_composite_fwd/bwd. */
int gs_window_from_list(void* stream, const int32_t* sorted_gids, int64_t n_entries, gs_window_t* window);

/* Window of gs_bin's compact list, from the same inputs and the stats of the same gs_bin
 * call: thr = L - 512 - 256 (negative-depth Gaussians); when GS_STAT_WINDOW_CLAMPED is
 * set, ids = slots L-512..L-1 of the reference's arrays rebuilt from the inputs (one
 * workgroup; otherwise no chunk reads them and only thr is written).  sorted_gids holds
 * capacity ids, as given to gs_bin. */
int gs_window_from_bins(void* stream, int64_t n, const float* means2d, const float* radii, const uint8_t* valid,
                        const float* depths, int width, int height, const int32_t* sorted_gids, int64_t capacity,
                        const int32_t* stats, gs_window_t* window);

/* Front-to-back compositing of every 16x16 tile.
 * Replaces jax_gs/renderer/rasterizer.py:157-248 (render_tiles body; its equivalent
 * jax_gs/renderer/rasterizer_tpu.py:13-135).  sorted_gids has n_entries elements and
 * ranges[T+1] indexes into it (out-of-range ids clamp to [0, n-1] as XLA's gather
 * does).  Per pixel it also writes the final
 * transmittance final_T[H,W] and n_contrib[H,W] = number of leading entries blended
 * while T > 1e-4, and tile_order[T] = the tiles sorted by decreasing walk length, the
 * launch order of gs_composite_bwd (residuals for gs_composite_bwd; each may be NULL).
 * clear_records (may be NULL): an [n, GS_REC_STRIDE] array the launch sets to zero on
 * the side (its waves are arithmetic-bound, so the stores cost nothing), for a later
 * gs_composite_bwd with accumulate = 1.
 * window (may be NULL) selects which ids entry k = 512 c + i of a tile reads:
 *   NULL  its own entries, sorted_gids[ranges[t] + k] (rasterizer_tpu.py:90-97);
 *   else  a gs_window_t in device memory, built by gs_window_from_list or
 *         gs_window_from_bins: the chunk reads window->ids[i] when its start
 *         ranges[t] + 512 c exceeds window->thr, else its own entries -- the default
 *         path's chunk windows (rasterizer.py:184-190), which slice 512 ids at
 *         min(start, L - 512) of the reference's L-slot arrays.
 * gs_composite_bwd takes the same window. */
int gs_composite_fwd(void* stream, int64_t n, const float* records, const int32_t* sorted_gids,
                     int64_t n_entries, const int32_t* ranges, int width, int height, const float* background,
                     float* image, float* final_T, int32_t* n_contrib, int32_t* tile_order, float* clear_records,
                     const gs_window_t* window);

/* gs_composite_fwd after gs_bin_deferred (the same n, width, height and capacity; its
 * workspace, sorted_gids, ranges and stats).  When the binning deferred the entry list,
 * each tile's walk reads its 8x8-tile superblock's list from the workspace (the words
 * whose bit is set in the tile's step masks, in the list's order, are the tile's entries)
 * and writes the entries it meets into sorted_gids; otherwise it reads sorted_gids as
 * gs_composite_fwd does.  Outputs are those of gs_composite_fwd on gs_bin's full list,
 * bit for bit; gs_composite_bwd then takes sorted_gids as usual.  Replaces the same
 * reference code as gs_composite_fwd (rasterizer.py:157-248). */
int gs_composite_fwd_deferred(void* stream, int64_t n, const float* records, int32_t* sorted_gids,
                              int64_t capacity, const int32_t* ranges, const int32_t* stats,
                              const void* bin_workspace, size_t bin_workspace_bytes, int width, int height,
                              const float* background, float* image, float* final_T, int32_t* n_contrib,
                              int32_t* tile_order, float* clear_records, const gs_window_t* window);

/* The L1 photometric loss fused into compositing: jax_gs/training/losses.py:4-8
 * (l1_loss(image, target) = mean |image - target|) applied to the rendered image, as
 * jax_gs/training/trainer.py differentiates l1_loss(render(...)).  The forward adds each
 * pixel's |image - target| over its channels as it writes the image (one partial sum per
 * workgroup) and the launch that orders the tiles sums the partials in a fixed order; the
 * backward forms the image cotangent sign(image - target) * dL/dloss / (3 H W) per pixel
 * where it reads it, so no separate loss launch, clear or image-gradient array is needed.
 *
 * gs_composite_l1_out_size: floats of l1_out (the loss, then the partial sums).
 * gs_composite_fwd_deferred_l1: gs_composite_fwd_deferred, plus l1_target[H,W,3] and
 *   l1_out, whose element 0 receives the loss. */
int64_t gs_composite_l1_out_size(int width, int height);
int gs_composite_fwd_deferred_l1(void* stream, int64_t n, const float* records, int32_t* sorted_gids,
                                 int64_t capacity, const int32_t* ranges, const int32_t* stats,
                                 const void* bin_workspace, size_t bin_workspace_bytes, int width, int height,
                                 const float* background, float* image, float* final_T, int32_t* n_contrib,
                                 int32_t* tile_order, float* clear_records, const gs_window_t* window,
                                 const float* l1_target, float* l1_out);

/* Vector-Jacobian product of gs_composite_fwd (JAX autodiff of render_tiles).
 * tile_order is the forward's (NULL: a fixed order; results agree up to the order of
 * floating-point additions).  grad_records[N,GS_REC_STRIDE] receives the gradient
 * record (layout above): overwritten when accumulate = 0, added to what it holds when
 * accumulate = 1 (records cleared by gs_composite_fwd's clear_records, or gradients of
 * several views summed in one buffer); grad_background[3] (may be NULL) is overwritten
 * with dL/d(background).  window: the forward's (entry ids read by the same rule).
 * clear (host pointer, may be NULL): arrays the launch sets to zero (gs_clear_list_t). */
int gs_composite_bwd(void* stream, int64_t n, const float* records, const int32_t* sorted_gids,
                     int64_t n_entries, const int32_t* ranges, int width, int height, const float* background,
                     const float* grad_image, const float* final_T, const int32_t* n_contrib,
                     const int32_t* tile_order, float* grad_records, float* grad_background, int accumulate,
                     const gs_window_t* window, const gs_clear_list_t* clear);

/* gs_composite_bwd of a render whose L1 loss was fused (gs_composite_fwd_deferred_l1): the
 * image cotangent of each pixel is sign(image - l1_target) * l1_cot[0] / (3 H W) (the VJP of
 * losses.py:4-8, sign(0) = 0, l1_cot = dL/dloss on the device), plus grad_image when it is
 * not NULL (the image also used elsewhere).  image is the forward's. */
int gs_composite_bwd_l1(void* stream, int64_t n, const float* records, const int32_t* sorted_gids,
                        int64_t n_entries, const int32_t* ranges, int width, int height, const float* background,
                        const float* grad_image, const float* image, const float* l1_target, const float* l1_cot,
                        const float* final_T, const int32_t* n_contrib, const int32_t* tile_order,
                        float* grad_records, float* grad_background, int accumulate, const gs_window_t* window,
                        const gs_clear_list_t* clear);

/* Vector-Jacobian product of gs_preprocess_fwd's compositing records with respect to
 * the five Gaussian parameter arrays (JAX autodiff of project_gaussians, eval_sh,
 * get_covariance_3d and the conic/sigmoid prologue).  Outputs are overwritten:
 * grad_means[N,3] grad_scales[N,3] grad_quats[N,4] grad_opacities[N,1]
 * grad_sh[N,K,3] (coefficients >= (sh_degree+1)^2 get 0).  A Gaussian whose gradient
 * record is all zero (no pixel reached it) has zero cotangents; zeroed = 1 promises that
 * the five arrays hold zeros on entry (gs_composite_bwd's clear list), and only the rows
 * of the other Gaussians are written; zeroed = 0 writes every row. */
int gs_preprocess_bwd(void* stream, int64_t n, int sh_k, int sh_degree, const float* means,
                      const float* scales, const float* quats, const float* opacities,
                      const float* sh_coeffs, const float* w2c, int width, int height,
                      float fx, float fy, float cx, float cy, const float* grad_records,
                      float* grad_means, float* grad_scales, float* grad_quats,
                      float* grad_opacities, float* grad_sh, int zeroed);

/* Workspace bytes gs_preprocess_bwd_w2c needs (16 floats per 64 Gaussians). */
size_t gs_preprocess_bwd_w2c_workspace_size(int64_t n);

/* gs_preprocess_bwd plus the camera cotangent grad_w2c[4,4] (JAX autodiff with respect to
 * Camera.W2C: through the camera-space means and W_rot of projection.py:26-57 and the view
 * directions of renderer.py:40-41 with camera.center = -R^T t, camera.py:15-21; row 3,
 * which never enters, is 0).  The per-Gaussian shares are summed per wave into workspace
 * and then in a fixed order by one workgroup. */
int gs_preprocess_bwd_w2c(void* stream, int64_t n, int sh_k, int sh_degree, const float* means,
                          const float* scales, const float* quats, const float* opacities,
                          const float* sh_coeffs, const float* w2c, int width, int height,
                          float fx, float fy, float cx, float cy, const float* grad_records,
                          float* grad_means, float* grad_scales, float* grad_quats,
                          float* grad_opacities, float* grad_sh, float* grad_w2c, void* workspace,
                          size_t workspace_bytes, int zeroed);

/* Vector-Jacobian product of gs_composite_prep on its own (JAX autodiff of the prologue of
 * jax_gs/renderer/rasterizer.py:119-156, render_tiles: det clamp, inverse covariance,
 * sigmoid): from the gradient records of gs_composite_bwd to the cotangents of
 * render_tiles' inputs, grad_means2d[N,2], grad_cov2d[N,2,2] ([1,0] is 0: render_tiles
 * reads cov2D[0,1] only), grad_opacities[N,1] (logits) and grad_colors[N,3]. */
int gs_composite_prep_bwd(void* stream, int64_t n, const float* cov2d, const float* opacities,
                          const float* grad_records, float* grad_means2d, float* grad_cov2d,
                          float* grad_opacities, float* grad_colors);

/* Vector-Jacobian product of jax_gs/renderer/projection.py:6-79 (project_gaussians, with
 * jax_gs/core/gaussians.py:58-92) on its own: from the cotangents of its outputs means2D
 * [N,2], cov2D [N,2,2] (all four entries) and z [N] (grad_depths, may be NULL = zero) to
 * those of means, scales and quaternions; radii and valid_mask carry none.  grad_w2c[4,4]
 * (may be NULL) receives dL/dW2C through the camera-space means and W_rot (row 3 is 0),
 * with a workspace of gs_preprocess_bwd_w2c_workspace_size(n) bytes (unused when NULL). */
int gs_project_bwd(void* stream, int64_t n, const float* means, const float* scales, const float* quats,
                   const float* w2c, float fx, float fy, const float* grad_means2d, const float* grad_cov2d,
                   const float* grad_depths, float* grad_means, float* grad_scales, float* grad_quats,
                   float* grad_w2c, void* workspace, size_t workspace_bytes);

/* jax_gs/renderer/sh.py:25-74 eval_sh: colors[N,3] = the real SH expansion of degree
 * sh_degree (0..3) of sh_coeffs[N,K,3] (K >= (sh_degree+1)^2) in the directions
 * view_dirs[N,3] (used as given), in the reference's association order; no +0.5 and no
 * clip (renderer.py:44-49 adds them). */
int gs_eval_sh(void* stream, int64_t n, int sh_k, int sh_degree, const float* sh_coeffs,
               const float* view_dirs, float* colors);

/* Vector-Jacobian product of gs_eval_sh: grad_sh[N,K,3] (coefficients >= (sh_degree+1)^2
 * get 0) and grad_dirs[N,3] (may be NULL), overwritten. */
int gs_eval_sh_bwd(void* stream, int64_t n, int sh_k, int sh_degree, const float* sh_coeffs,
                   const float* view_dirs, const float* grad_colors, float* grad_sh, float* grad_dirs);

/* The training step's tail in one pass: gs_preprocess_bwd's gradients, the
 * densification statistics of gs_densify_accumulate (from the means before the update;
 * skipped when grad_accum is NULL) and gs_adam_step's masked update of the five arrays,
 * in place; no parameter gradient is written.  Replaces trainer.py:137-159 after the
 * rasterizer's VJP, with optax.adam of train.py:127-155.  moments: host array of 10 device
 * pointers (first moments of means, scales, quaternions, opacities, sh_coeffs, then the
 * second moments), lrs[5] the learning rates, step the optimizer count after the update. */
int gs_preprocess_bwd_adam(void* stream, int64_t n, int sh_k, int sh_degree, float* means,
                           float* scales, float* quats, float* opacities, float* sh_coeffs,
                           const float* w2c, int width, int height, float fx, float fy, float cx,
                           float cy, const float* grad_records, float* const* moments,
                           const double* lrs, int step, double b1, double b2, double eps,
                           const uint8_t* active, const uint8_t* valid, const float* radii,
                           float focal, float pixel_scale, float* grad_accum, int32_t* denom,
                           float* max_radii);

/* mean(|pred - target|) into loss[0] and, when grad is not NULL, its gradient
 * sign(pred - target) / count.  Replaces jax_gs/training/losses.py:4-8 (l1_loss)
 * and its autodiff seed. */
int gs_l1_loss(void* stream, int64_t count, const float* pred, const float* target,
               float* loss, float* grad);

/* mean((pred - target)^2) into loss[0] and, when grad is not NULL, its gradient
 * 2 (pred - target) / count.  Replaces jax_gs/training/losses.py:10-14 (mse_loss). */
int gs_mse_loss(void* stream, int64_t count, const float* pred, const float* target,
                float* loss, float* grad);

/* VJP of gs_l1_loss / gs_mse_loss for a loss cotangent grad_out[0] on the device
 * (losses.py:4-14 under jax.grad): grad = sign(pred - target) * (g / count), or
 * 2 (pred - target) * (g / count).  One pass, no reduction. */
int gs_l1_loss_bwd(void* stream, int64_t count, const float* pred, const float* target, const float* grad_out,
                   float* grad);
int gs_mse_loss_bwd(void* stream, int64_t count, const float* pred, const float* target, const float* grad_out,
                    float* grad);

/* Workspace bytes of gs_l1_ssim / gs_l1_ssim_bwd for an image of height x width x
 * channels (0 for a bad shape). */
size_t gs_l1_ssim_workspace_size(int height, int width, int channels);

/* L1 and SSIM of pred against target [H,W,C] in one pass: out[0] = mean |pred - target|,
 * out[1] = mean SSIM.  Replaces jax_gs/training/losses.py:4-8 (l1_loss) and :16-68
 * (ssim: 11-tap Gaussian window, sigma 1.5, 'SAME' zero padding, C1 = 0.01^2,
 * C2 = 0.03^2, map clipped to [-1, 1]), the two terms of trainer.py:18-26.  With
 * with_grad != 0 the workspace also keeps what gs_l1_ssim_bwd needs. */
int gs_l1_ssim(void* stream, int height, int width, int channels, const float* pred,
               const float* target, float* out, int with_grad, void* workspace,
               size_t workspace_bytes);

/* grad_pred = grad_out[0] * d out[0] / d pred + grad_out[1] * d out[1] / d pred, with
 * grad_out[2] on the device (JAX autodiff of l1_loss and ssim; ties of max and clip pass
 * half).  Needs the workspace of a gs_l1_ssim call with_grad on the same images. */
int gs_l1_ssim_bwd(void* stream, int height, int width, int channels, const float* pred,
                   const float* target, const float* grad_out, const void* workspace,
                   size_t workspace_bytes, float* grad_pred);

/* gs_l1_ssim / gs_l1_ssim_bwd for any window size in [1, 63] and any channel count
 * (losses.py:16 ssim(..., window_size)): taps exp(-(j - L/2)^2 / 4.5) / sum for j < L and
 * XLA's 'SAME' correlation, which pads (L-1)/2 before and L/2 after (even L: the window is
 * off centre).  Workspace: gs_l1_ssim_window_workspace_size bytes (32 B per value); the
 * backward reads the gradient maps of a forward run with with_grad = 1 on the same
 * workspace and overwrites the rest of it. */
size_t gs_l1_ssim_window_workspace_size(int height, int width, int channels, int window_size);
int gs_l1_ssim_window(void* stream, int height, int width, int channels, int window_size, const float* pred,
                      const float* target, float* out, int with_grad, void* workspace, size_t workspace_bytes);
int gs_l1_ssim_window_bwd(void* stream, int height, int width, int channels, int window_size, const float* pred,
                          const float* target, const float* grad_out, void* workspace, size_t workspace_bytes,
                          float* grad_pred);

/* The trainer's loss from gs_l1_ssim's out[2] (trainer.py:18-26): terms[0] = d_ssim =
 * max(0, (1 - ssim) / 2) (losses.py:70-75), terms[1] = (1 - lambda) l1 + lambda d_ssim,
 * terms[2..3] = the cotangents of (l1, ssim) for a unit cotangent of terms[1] (the
 * grad_out of gs_l1_ssim_bwd; max passes half at a tie), terms[4] = 1 - 2 d_ssim (the
 * reported SSIM, trainer.py:30).  Device arrays, one launch. */
int gs_l1_ssim_terms(void* stream, const float* l1_ssim, double lambda_ssim, float* terms);

/* One Adam step, in place, of num_arrays (<= 8) float32 parameter arrays, each with
 * its gradient and first/second moments (same sizes), counts[i] elements laid out as
 * rows x row_lens[i] (row_lens[i] <= 64).  Replaces optax.adam (b1, b2, eps, eps_root 0)
 * in the optax.multi_transform of train.py:127-155, the trainer's row mask
 * (trainer.py:44-53: rows with active[row] == 0 get no update; active may be NULL) and
 * optax.apply_updates.  step = the optimizer's count after this update (>= 1); lrs[i]
 * is array i's learning rate at the count before it (schedules are evaluated by the
 * caller).  All pointer arrays are host arrays of device pointers. */
int gs_adam_step(void* stream, int num_arrays, float* const* params, const float* const* grads,
                 float* const* mus, float* const* nus, const int64_t* counts, const int* row_lens,
                 const double* lrs, const uint8_t* active, int64_t rows, int step, double b1,
                 double b2, double eps);

/* Workspace bytes of gs_densify_and_prune for a capacity of M Gaussians. */
size_t gs_densify_workspace_size(int64_t capacity);

/* Densify and prune the static-capacity arrays in place.  Replaces
 * jax_gs/training/density.py:98-211 (densify_and_prune) with :63-67
 * (_reset_accumulators): prunes active Gaussians with sigmoid(opacity) < min_opacity,
 * max exp(scale) > 0.1 extent or max_radii > max_screen_size; clones (max exp(scale)
 * <= 0.01 extent) or splits the remaining ones whose grad_accum / denom >=
 * grad_threshold into the empty slots (in index order; nothing is added when
 * densify_enabled is 0 or the new ones do not fit), splits taking scale - log(1.6) and
 * mean + noise * exp(new scale) on both copies; updates active, clears grad_accum and
 * denom.  The num_moments (0, 5 or 10) arrays of moments (host array of device
 * pointers, in the order means, scales, quaternions, opacities, sh_coeffs, repeated)
 * move with their Gaussians.  noise[M,3] holds standard normal draws (the reference's
 * jax.random.normal).  counts (may be NULL; device int32[5]) receives clones, splits,
 * pruned, available slots, densified (0/1). */
int gs_densify_and_prune(void* stream, int64_t capacity, int sh_k, float* means, float* scales,
                         float* quats, float* opacities, float* sh_coeffs, int num_moments,
                         float* const* moments, uint8_t* active, float* grad_accum, int32_t* denom,
                         const float* max_radii, const float* noise, int densify_enabled,
                         double grad_threshold, double min_opacity, double extent,
                         double max_screen_size, void* workspace, size_t workspace_bytes,
                         int32_t* counts);

/* opacities[i] = log(reset_value / (1 - reset_value)) where active[i] (in place).
 * Replaces jax_gs/training/density.py:69-93 (reset_opacities). */
int gs_reset_opacities(void* stream, int64_t capacity, const uint8_t* active, double reset_value,
                       float* opacities);

/* PLY vertex records [N, 62] float32 (x y z, nx ny nz = 0, f_dc_0..2, f_rest_0..44 with
 * f_rest_i = sh[1 + i/3][i%3], opacity, scale_0..2, rot_0..3) from the five arrays, and
 * back (normals ignored).  sh_k must be 16.  Replaces the record assembly of
 * jax_gs/io/ply.py:6-123 (save_ply / load_ply); the host writes the header. */
int gs_ply_pack(void* stream, int64_t n, int sh_k, const float* means, const float* scales,
                const float* quats, const float* opacities, const float* sh_coeffs, float* records);
int gs_ply_unpack(void* stream, int64_t n, int sh_k, const float* records, float* means,
                  float* scales, float* quats, float* opacities, float* sh_coeffs);

/* Densification statistics of one training step, updated in place.
 * Replaces jax_gs/training/trainer.py:143-159 (train_step, after value_and_grad):
 *   grad_accum += (|grad_means| * (max(z_cam,0.01) / focal)) * pixel_scale
 *   denom      += valid & active
 *   max_radii   = valid ? max(max_radii, radii) : max_radii
 * focal = float32((fx+fy)/2) and pixel_scale = float32(W*H*3), both formed in double
 * precision by the caller exactly as the reference's Python does.
 * active may be NULL (all active). */
int gs_densify_accumulate(void* stream, int64_t n, const float* grad_means, const float* means,
                          const float* w2c, float focal, float pixel_scale,
                          const uint8_t* valid, const uint8_t* active, const float* radii,
                          float* grad_accum, int32_t* denom, float* max_radii);

#ifdef __cplusplus
}
#endif
#endif /* GS_RASTER_H */
