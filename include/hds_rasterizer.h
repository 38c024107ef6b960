/*
 * C ABI of the MI355X-native high-dimensional splatting rasterizer (libhds_rasterizer.so).
 *
 * These entry points replace the ten functions of the reference's torch extension
 * "gaussian_rasterizer" (gaussian_splatting/rasterizer/bindings.cpp:4-42, api.h:4-119). They take
 * plain device pointers, sizes and a HIP stream, and hold no torch types, so any host language can
 * bind them (the Python mirror of the reference's autograd API does so with ctypes).
 *
 * Conventions
 *   - Every pointer is device memory on the current HIP device unless stated, fp32 or int32,
 *     contiguous, in the reference's layouts: means2D [N,2], conics [N,3] as (xx, xy, yy),
 *     colors [N,3], opacities [N] (the reference's [N,1]), images [H,W,3], feature images
 *     [H,W,C], tile_ranges [T,2] with T = ceil(W/16) * ceil(H/16).
 *   - conic4 [N,4] = (a, b, c, opacity) and color_opacity4 [N,4] = (r, g, b, opacity) are the
 *     packed per-gaussian records the binning call writes and every render call reads; they play
 *     the role of the reference's `conic` / `color_opacity` tuple members (forward.cu:274-276).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL is the default stream). Only
 *     hds_bin_count blocks the host: it reads the pair count P back once, as forward.cu:321-325.
 *     hds_bin_count_async + hds_bin_emit_capped are the same binning without that wait: the
 *     count reaches the host by an asynchronous copy and the emit runs on capacity-sized buffers.
 *   - Returns HDS_OK (0) or an error status; hds_last_error() then holds a message for the
 *     calling thread. Invalid arguments are rejected before anything is enqueued.
 *   - The library never allocates device memory: scratch comes in as caller-owned workspaces
 *     whose sizes the *_workspace_bytes queries give, except for hds_bin_static, whose workspaces
 *     are a static device array of the library (for callers that cannot allocate at all).
 *   - Gradient outputs of the backward calls are zeroed by the library before accumulation.
 */
#ifndef HDS_RASTERIZER_H
#define HDS_RASTERIZER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HDS_ABI_VERSION 1

#if defined(__GNUC__)
#define HDS_API __attribute__((visibility("default")))
#else
#define HDS_API
#endif

typedef void* hds_stream_t; /* hipStream_t */

/* Status codes. */
#define HDS_STATUS_OK 0
#define HDS_STATUS_INVALID_ARGUMENT 1
#define HDS_STATUS_RUNTIME_ERROR 2

/* Message of the last failed call on this thread (never NULL). */
HDS_API const char* hds_last_error(void);

/* HDS_ABI_VERSION of the loaded library. */
HDS_API int hds_abi_version(void);

/* ---- projection: replaces project_gaussians / project_gaussians_backward ------------------- */

/* projection.cu:210-231 (project_gaussians). world_to_camera is a device [4,4] row-major matrix.
 * Outputs means2D [N,2], depths [N], radii [N] (0 for culled), conics [N,3]. */
HDS_API int hds_project_gaussians(int64_t n, const float* means, const float* scales, const float* quats,
						  const float* opacities, const float* world_to_camera, float fx, float fy,
						  float cx, float cy, int width, int height, float near_plane,
						  float low_pass, float fov_scale, float* means2D, float* depths,
						  float* radii, float* conics, hds_stream_t stream);

/* projection.cu:234-253 (project_gaussians_backward). */
HDS_API int hds_project_gaussians_backward(int64_t n, const float* grad_means2D, const float* grad_conics,
								   const float* means, const float* scales, const float* quats,
								   const float* world_to_camera, float fx, float fy, float cx,
								   float cy, int width, int height, float near_plane,
								   float low_pass, float fov_scale, float* grad_means,
								   float* grad_scales, float* grad_quats, hds_stream_t stream);

/* ---- spherical harmonics: replaces eval_sh / eval_sh_backward_adam ------------------------- */

/* sh.cu:157-168 (eval_sh). sh_dc [N,1,3], sh_rest [N,15,3], dirs [N,3], radii [N] -> rgb [N,3]. */
HDS_API int hds_eval_sh(int64_t n, int degree, const float* sh_dc, const float* sh_rest, const float* dirs,
				const float* radii, float* rgb, hds_stream_t stream);

/* sh.cu:171-190 (eval_sh_backward_adam_host). Steps sh_dc, sh_rest and their Adam moments in
 * place with the device step counters step_dc / step_rest (0-d fp32, already incremented);
 * writes grad_dirs [N,3]. */
HDS_API int hds_eval_sh_backward_adam(int64_t n, int degree, const float* grad_rgb, float* sh_dc,
							  float* sh_rest, const float* dirs, const float* radii, float* m_dc,
							  float* v_dc, float* m_rest, float* v_rest, const float* step_dc,
							  const float* step_rest, double lr_dc, double lr_rest, double beta1,
							  double beta2, double eps, float* grad_dirs, hds_stream_t stream);

/* ---- binning: replaces the binning half of rasterize (forward.cu:239-405) ------------------ */

/* Bytes of the per-gaussian workspace hds_bin_count / hds_bin_tile_order_async fill and the emits
 * read. It includes the tile-order binning's count matrix (4 bytes per tile and chunk of 4096
 * gaussians) when that stays within 2^24 words; width = height = 0 leaves the matrix out (enough
 * for the depth-order binning). */
HDS_API size_t hds_bin_workspace_bytes(int64_t n, int width, int height);

/* forward.cu:284-326: culls, packs conic4 / color_opacity4 (colors may be NULL), counts the
 * tiles of each gaussian, orders the gaussians by depth and prefix-sums their counts. Writes the
 * total pair count P to *num_pairs (host memory) after the one blocking device-to-host read. */
HDS_API int hds_bin_count(int64_t n, const float* means2D, const float* depths, const float* radii,
				  const float* conics, const float* colors, const float* opacities, int width,
				  int height, float* conic4, float* color_opacity4, void* workspace,
				  size_t workspace_bytes, int64_t* num_pairs, hds_stream_t stream);

/* hds_bin_count without the blocking read (forward.cu:311-326 with the host read deferred):
 * enqueues the same work, then an asynchronous copy of 16 bytes to count_host, which must be
 * pinned host memory (hipHostMalloc): uint64 P, uint32 look-back error flag (nonzero = the
 * counts are invalid), uint32 tile-sort flag (zero here; hds_bin_status reads it after the emit).
 * The words are valid once the stream has passed this call; the caller checks them before
 * trusting what hds_bin_emit_capped produced. */
HDS_API int hds_bin_count_async(int64_t n, const float* means2D, const float* depths, const float* radii,
						const float* conics, const float* colors, const float* opacities, int width,
						int height, float* conic4, float* color_opacity4, void* workspace,
						size_t workspace_bytes, void* count_host, hds_stream_t stream);

/* Bytes of the per-pair workspace hds_bin_emit needs for P pairs. */
HDS_API size_t hds_pairs_workspace_bytes(int64_t num_pairs, int width, int height);

/* forward.cu:340-404: emits the (tile, gaussian) pairs, orders them by (tile, depth) keeping
 * index order on ties, and builds the per-tile [start, end) ranges, (0, 0) when untouched.
 * values_sorted [P] int32, tile_ranges [T,2] int32. If a look-back of the tile sort gives up
 * (bounded wait, see hds_set_lookback_limit), every tile range is left (0, 0), so nothing reads
 * the unsorted list, and the flag is raised in `workspace` for hds_bin_status. `workspace` must be
 * the one hds_bin_count(_async) last filled (the emits read what that count left in it); a workspace
 * hds_bin_tile_order_async filled, or one no count of this process filled, is rejected (status 1)
 * before anything is enqueued. The same holds for hds_bin_emit_capped, and the other way round for
 * hds_bin_emit_tile_order. */
HDS_API int hds_bin_emit(int64_t n, int64_t num_pairs, int width, int height, void* workspace,
				 void* pairs_workspace, size_t pairs_workspace_bytes, int32_t* values_sorted,
				 int32_t* tile_ranges, hds_stream_t stream);

/* hds_bin_emit (forward.cu:340-404) for a pair count the host has not read yet: values_sorted
 * and the pairs workspace are sized for `capacity` pairs, and the kernels take P from the
 * workspace hds_bin_count_async filled. When P <= capacity the result equals hds_bin_emit's for
 * P (values_sorted[0, P) and tile_ranges). When P > capacity only the first `capacity` pairs of
 * the depth order are sorted: tile_ranges stay consistent with what was written (every range
 * lies in [0, capacity)) but the binning is incomplete, and the caller runs hds_bin_emit again
 * with buffers for P. With the error flag set nothing is emitted (all ranges (0, 0)). */
HDS_API int hds_bin_emit_capped(int64_t n, int64_t capacity, int width, int height, void* workspace,
						void* pairs_workspace, size_t pairs_workspace_bytes, int32_t* values_sorted,
						int32_t* tile_ranges, hds_stream_t stream);

/* The whole binning (forward.cu:284-404) in one call for a pair count the host has not read yet,
 * with the depth order built per tile: no global depth sort. Each chunk of 4096 gaussians counts
 * its pairs per tile, one exclusive scan over (tile, chunk) places every chunk's run of every tile,
 * the pairs are scattered into their runs (counting scatter), and each tile's list is then sorted
 * by (depth bits, index) in one work-group, which gives the reference's (tile, depth bits, index)
 * order. When the count matrix (chunks x tiles) exceeds 2^24 words, the tile counts are scanned, the
 * pairs emitted in gaussian-index order and sorted by tile alone instead, before the same per-tile
 * sort. values_sorted, tile_ranges, conic4 and color_opacity4 equal hds_bin_count + hds_bin_emit's
 * bit for bit, under hds_bin_emit_capped's capacity contract (values_sorted sized for `capacity`
 * pairs; when P > capacity, tile_ranges are cut at `capacity` and everything inside them is
 * written, but the binning is incomplete). The pairs workspace (hds_pairs_workspace_bytes(capacity))
 * is used only when the count matrix is too large; it may be NULL otherwise. The call ends
 * with an asynchronous copy of the 16 status bytes of hds_bin_status to status_host (pinned host
 * memory), valid once the stream has passed the call. It takes tile lists of up to 4096 pairs: a
 * longer one is left in index order and flagged (bit 1 of the tile-sort word), and the caller bins
 * the frame again with hds_bin_count + hds_bin_emit. When P > capacity, hds_bin_emit_tile_order
 * emits again with buffers for P from the same workspace (then read the flags with
 * hds_bin_status). No counterpart in the reference. */
HDS_API int hds_bin_tile_order_async(int64_t n, const float* means2D, const float* depths, const float* radii,
							 const float* conics, const float* colors, const float* opacities, int width,
							 int height, float* conic4, float* color_opacity4, void* workspace,
							 size_t workspace_bytes, int64_t capacity, void* pairs_workspace,
							 size_t pairs_workspace_bytes, int32_t* values_sorted, int32_t* tile_ranges,
							 void* status_host, hds_stream_t stream);
HDS_API int hds_bin_emit_tile_order(int64_t n, int64_t num_pairs, int width, int height, void* workspace,
							void* pairs_workspace, size_t pairs_workspace_bytes, int32_t* values_sorted,
							int32_t* tile_ranges, hds_stream_t stream);

/* No counterpart in the reference (CUB's sort reports nothing): enqueues an asynchronous copy of
 * the binning's 16 status bytes from `workspace` (the one hds_bin_count(_async) filled for n
 * gaussians) to pinned host memory status_host: uint64 pair count P, uint32 flag of the depth sort
 * and count scan, uint32 word of the tile sort of the last emit (hds_bin_emit(_capped / _tile_order)):
 * a nonzero flag, or bit 0 of the word, means a look-back gave up and the binning must not be used;
 * bit 1 means a tile-order binning met a tile of more than 4096 pairs. Valid once the stream has
 * passed this call. */
HDS_API int hds_bin_status(int64_t n, const void* workspace, void* status_host, hds_stream_t stream);

/* No counterpart in the reference; for tests of the failure path. Polls a look-back of the
 * binning's sorts and scan makes on a silent predecessor before it gives up and raises its flag
 * (HDS_LOOKBACK_LIMIT_DEFAULT, seconds of waiting). 0 makes every look-back give up before its
 * first poll, so the failure is certain while every kernel still runs to its end. Applies to
 * launches made after the call, on every thread. */
#define HDS_LOOKBACK_LIMIT_DEFAULT 4194304u
HDS_API int hds_set_lookback_limit(uint32_t polls);

/* No counterpart in the reference; for tests of the tile-order binning's two paths. The largest
 * count matrix (chunks x tiles words) hds_bin_tile_order_async takes the counting scatter for; 0
 * restores the default, 2^24, which is also the most a workspace reserves room for. Applies to
 * calls made after it, on every thread; hds_bin_emit_tile_order follows the path its workspace's
 * count took. */
HDS_API int hds_set_tile_scatter_limit(uint64_t words);

/* No counterpart in the reference. For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): hds_bin_count_async
 * followed by hds_bin_emit_capped in one call, with both workspaces in a static device array of
 * HDS_BIN_STATIC_SCRATCH_MIB MiB inside the library (one per GPU, held until the process ends)
 * instead of caller-supplied ones; no allocation of any kind, and no host wait. The caller passes
 * the inputs and outputs of those two calls: conic4 / color_opacity4 [N,4], values_sorted sized for
 * `capacity` pairs, tile_ranges [T,2], and `status`, 16 bytes of pinned host or device memory
 * that receive uint64 P, uint32 depth-sort / scan flag, uint32 tile-sort flag once the stream has
 * passed this call. As with hds_bin_emit_capped, the binning is complete when P <= capacity and
 * both flags are zero; otherwise call again with a larger capacity. Rejects (status 1) a gaussian
 * count and capacity whose workspaces exceed the scratch: hds_bin_workspace_bytes(n, 0, 0) +
 * hds_pairs_workspace_bytes(capacity, 0, 0) must fit, which holds for 1.5M gaussians with 4M pairs.
 * Every call on a GPU shares that GPU's scratch: calls that overlap on one GPU (other streams,
 * other host threads) race and must be serialised by the caller. */
#define HDS_BIN_STATIC_SCRATCH_MIB 112
HDS_API int hds_bin_static(int64_t n, const float* means2D, const float* depths, const float* radii,
					   const float* conics, const float* colors, const float* opacities, int width,
					   int height, float* conic4, float* color_opacity4, int64_t capacity,
					   int32_t* values_sorted, int32_t* tile_ranges, void* status, hds_stream_t stream);

/* ---- blend forward: replaces render_gaussians (forward.cu:406-434) and rasterize_features
 *      (features.cu:299-346) with one tile walk ------------------------------------------------ */

/* Front-to-back blend of RGB (when image != NULL; background [3] required then) and of C
 * feature channels (when features != NULL; C in {32, 64, 128, 256, 512}) with the same weights.
 * final_T [H,W] and n_contrib [H,W] are always written. */
HDS_API int hds_render(int64_t n, int width, int height, int channels, const int32_t* tile_ranges,
			   const int32_t* values_sorted, int64_t num_pairs, const float* means2D,
			   const float* conic4, const float* color_opacity4, const float* background,
			   const float* features, float* image, float* final_T, int32_t* n_contrib,
			   float* feature_image, hds_stream_t stream);

/* hds_render that also zeroes `clear_count` floats at `clear` (16-byte aligned, a multiple of 4;
 * 0 clears nothing), each tile's work-group one share before its walk: the zero-initialised
 * gradient buffers of a following hds_render_backward_accumulate, cleared in the bandwidth the
 * walk leaves unused instead of by a fill of their own. The same results as hds_render followed by
 * hds_zero_async over the range; the range must not overlap the render's inputs or outputs. No
 * counterpart in the reference, which allocates its gradient
 * outputs with torch::zeros in the backward (backward.cu:166-226, features.cu:561-616). */
HDS_API int hds_render_clear(int64_t n, int width, int height, int channels, const int32_t* tile_ranges,
				 const int32_t* values_sorted, int64_t num_pairs, const float* means2D,
				 const float* conic4, const float* color_opacity4, const float* background,
				 const float* features, float* image, float* final_T, int32_t* n_contrib,
				 float* feature_image, float* clear, int64_t clear_count, hds_stream_t stream);

/* ---- blend backward: replaces rasterize_backward (backward.cu:166-226) and
 *      rasterize_features_backward (features.cu:561-616) with one back-to-front walk ----------- */

/* grad_image [H,W,3] (NULL: no RGB term; grad_colors may then be NULL) and, when features !=
 * NULL, grad_feature_image [H,W,C] with slice_width in {32, 64, 128} dividing C (the channels one
 * work-group owns). grad_features may be NULL (frozen features still shape the geometry
 * gradients). Outputs grad_means2D [N,2], grad_conics [N,3], grad_colors [N,3],
 * grad_opacities [N], grad_features [N,C]; all zeroed here first. */
HDS_API int hds_render_backward(int64_t n, int width, int height, int channels, int slice_width,
						const int32_t* tile_ranges, const int32_t* values_sorted, int64_t num_pairs,
						const float* means2D, const float* conic4, const float* color_opacity4,
						const float* background, const float* final_T, const int32_t* n_contrib,
						const float* grad_image, const float* features,
						const float* grad_feature_image, float* grad_means2D, float* grad_conics,
						float* grad_colors, float* grad_opacities, float* grad_features,
						hds_stream_t stream);

/* As hds_render_backward, but adds into the gradient outputs instead of zeroing them first: the
 * caller supplies zero-initialised buffers, or accumulates over several views. */
HDS_API int hds_render_backward_accumulate(
	int64_t n, int width, int height, int channels, int slice_width, const int32_t* tile_ranges,
	const int32_t* values_sorted, int64_t num_pairs, const float* means2D, const float* conic4,
	const float* color_opacity4, const float* background, const float* final_T, const int32_t* n_contrib,
	const float* grad_image, const float* features, const float* grad_feature_image, float* grad_means2D,
	float* grad_conics, float* grad_colors, float* grad_opacities, float* grad_features, hds_stream_t stream);

/* Zeroes `count` floats at p (16-byte aligned, count a multiple of 4) on `stream` with at most
 * `max_workgroups` work-groups of 256 threads (0: as many as fill the device), so that a large fill
 * enqueued beside latency-bound kernels takes only part of the CUs. The zero-initialised buffers of
 * hds_render_backward_accumulate; the reference zeroes its gradient outputs where it allocates them
 * (torch::zeros in backward.cu:166-226, features.cu:561-616). */
HDS_API int hds_zero_async(float* p, int64_t count, int max_workgroups, hds_stream_t stream);

/* ---- SSIM: replaces ssim_forward / ssim_backward ------------------------------------------- */

/* ssim.cu:116-148. rendered, gt [H,W,3] -> ssim_map, d_mu, d_aa, d_ab [H,W,3]. */
HDS_API int hds_ssim_forward(int height, int width, const float* rendered, const float* gt,
					 float* ssim_map, float* d_mu, float* d_aa, float* d_ab, hds_stream_t stream);

/* ssim.cu:151-177. grad_mean is a device scalar; writes grad_rendered [H,W,3]. */
HDS_API int hds_ssim_backward(int height, int width, const float* grad_mean, const float* rendered,
					  const float* gt, const float* d_mu, const float* d_aa, const float* d_ab,
					  float* grad_rendered, hds_stream_t stream);

/* ---- densification statistics: replaces GaussianModel.add_densification_stats -------------- */

/* utils/gaussian.py:143-160 for one view, in place, without the host synchronisation of the
 * reference's boolean indexing: for every gaussian with radii > 0, max_radii2D = max(max_radii2D,
 * radius), grad_accum += |grad_means2D * (width / 2, height / 2)|, denom += 1. grad_means2D [N,2]
 * (dL/dmeans2D, the gradient the rasterizer backward produced), radii [N], max_radii2D [N],
 * grad_accum [N] (the reference's [N,1]), denom [N] ([N,1]). */
HDS_API int hds_densification_stats(int64_t n, const float* grad_means2D, const float* radii, int width,
							int height, float* max_radii2D, float* grad_accum, float* denom,
							hds_stream_t stream);

/* ---- kernel timing (no counterpart in the reference; for benchmarks) ------------------------ */

/* Starts recording: from now on every hot-path kernel launch (projection, blend forward, the two
 * blend-backward kernels) is bracketed by HIP events on its own stream. Clears earlier records. */
HDS_API int hds_profile_begin(void);

/* hds_profile_begin restricted to the kernels named in `kernels`, a comma-separated list of kernel
 * names as hds_profile_record reports them (NULL or "" records every kernel). Each recorded launch
 * adds two timed events to its stream, a few microseconds each, so a benchmark that times a whole
 * step records only the kernels whose durations it needs. */
HDS_API int hds_profile_begin_only(const char* kernels);

/* Stops recording, waits for the recorded events and returns how many launches were recorded
 * (negative on error). */
HDS_API int64_t hds_profile_end(void);

/* Kernel name and duration in ms of record i (0 <= i < the count hds_profile_end returned). */
HDS_API int hds_profile_record(int64_t i, const char** name, float* ms);

/* Kernel name, start and end in ms of record i, relative to the start of record 0. */
HDS_API int hds_profile_timeline(int64_t i, const char** name, float* start_ms, float* end_ms);

#ifdef __cplusplus
}
#endif

#endif /* HDS_RASTERIZER_H */
