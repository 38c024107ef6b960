// Densification statistics of one training view (utils/gaussian.py:143-160), one pass.
//
// For every gaussian the view rendered (radii > 0): max_radii2D = max(max_radii2D, radius),
// grad_accum += |dL/dmeans2D * (W/2, H/2)| (the pixel-space gradient in normalised device units),
// denom += 1. The reference does this with about ten torch operations per step, including boolean
// indexing that waits for the device to count the visible gaussians; here it is one streaming kernel
// (20 B read, 12 B read-modify-written per visible gaussian) with no host synchronisation.
#include "hds_internal.h"
#include "hds_rasterizer.h"

namespace {

__global__ __launch_bounds__(256) void densification_stats_kernel(int64_t n, const float2* __restrict__ grad_means2D,
																   const float* __restrict__ radii, float half_w,
																   float half_h, float* __restrict__ max_radii2D,
																   float* __restrict__ grad_accum,
																   float* __restrict__ denom) {
	const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
	if (i >= n) return;
	const float r = radii[i];
	if (!(r > 0.0f)) return;  // culled (and NaN radii) leave the statistics alone
	max_radii2D[i] = fmaxf(max_radii2D[i], r);
	const float2 g = grad_means2D[i];
	const float gx = g.x * half_w, gy = g.y * half_h;
	grad_accum[i] += sqrtf(gx * gx + gy * gy);
	denom[i] += 1.0f;
}

}  // namespace

extern "C" int hds_densification_stats(int64_t n, const float* grad_means2D, const float* radii, int width, int height,
									   float* max_radii2D, float* grad_accum, float* denom, hds_stream_t stream) {
	HDS_REQUIRE(n >= 0, "densification_stats: negative gaussian count");
	HDS_REQUIRE(width > 0 && height > 0, "densification_stats: image size %dx%d must be positive", width, height);
	if (n == 0) return HDS_OK;
	HDS_REQUIRE(grad_means2D && radii && max_radii2D && grad_accum && denom,
				"densification_stats: null pointer argument");
	HDS_REQUIRE((reinterpret_cast<uintptr_t>(grad_means2D) & 7u) == 0, "densification_stats: misaligned grad_means2D");
	hipStream_t s = (hipStream_t)stream;
	densification_stats_kernel<<<hds_blocks(n, 256), 256, 0, s>>>(n, reinterpret_cast<const float2*>(grad_means2D), radii,
																 0.5f * (float)width, 0.5f * (float)height,
																 max_radii2D, grad_accum, denom);
	return hds_check_launch("densification_stats", s);
}
