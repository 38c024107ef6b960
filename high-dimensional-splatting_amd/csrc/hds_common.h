/*
 * Constants and reproducible scalar arithmetic shared by the HIP kernels and the CPU oracle.
 *
 * Everything here compiles both as HIP device code and as plain C (gcc), and uses only IEEE
 * operations that both sides round identically: +, -, *, correctly rounded / and sqrt, fmaf and
 * exact bit manipulation. Both sides are compiled with -ffp-contract=off, so a function below
 * returns the same bits on the CPU and on gfx950. That is what lets the tile counts, sorted pair
 * lists and tile ranges of the GPU binning match the oracle bit for bit.
 *
 * Constants follow the reference rasterizer:
 *   TILE_SIZE 16, MIN_TRANSMITTANCE 1e-4, MIN_ALPHA 1/255, MAX_ALPHA 0.99
 *   (gaussian_splatting/rasterizer/common.cuh:8-16; tests/oracle.py:4-6).
 */
#ifndef HDS_COMMON_H
#define HDS_COMMON_H

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define HDS_HD __host__ __device__ static inline
#else
#include <math.h>
#define HDS_HD static inline
#endif

#define HDS_TILE 16
#define HDS_MIN_ALPHA (1.0f / 255.0f)
#define HDS_MAX_ALPHA 0.99f
#define HDS_MIN_TRANSMITTANCE 1e-4f

/* Projection constants, projection.py:3-5. */
#define HDS_NEAR_PLANE 0.2f
#define HDS_LOW_PASS 0.3f
#define HDS_JACOBIAN_FOV_SCALE 1.3f

HDS_HD uint32_t hds_f2u(float x) {
	uint32_t u;
	memcpy(&u, &x, sizeof(u));
	return u;
}

HDS_HD float hds_u2f(uint32_t u) {
	float x;
	memcpy(&x, &u, sizeof(x));
	return x;
}

/*
 * Natural logarithm, written from the textbook reduction
 *   x = m * 2^e with m in [sqrt(1/2), sqrt(2)),  log x = e*ln2 + 2*atanh(s),  s = (m-1)/(m+1),
 * with 2*atanh(s) = 2s + 2s^3/3 + 2s^5/5 + ... truncated after s^13 (|s| <= 0.1716, so the first
 * dropped term is below 2^-40 relative) and ln2 split Cody-Waite style into a 16-bit head, which
 * makes e*ln2_hi exact, and a float tail. Accurate to a couple of float ULPs; identical on every
 * IEEE machine because it uses only correctly rounded operations.
 */
HDS_HD float hds_logf(float x) {
	if (!(x > 0.0f)) return x == 0.0f ? -HUGE_VALF : (x - x) / (x - x);
	if (x > 3.40282347e+38f) return x;
	uint32_t u = hds_f2u(x);
	int e = (int)(u >> 23) - 127;
	if ((u >> 23) == 0) {
		/* Subnormal: scale by 2^23, which is exact. */
		u = hds_f2u(x * 8388608.0f);
		e = (int)(u >> 23) - 127 - 23;
	}
	float m = hds_u2f((u & 0x007fffffu) | 0x3f800000u);
	if (m > 1.41421356f) {
		m *= 0.5f;
		e += 1;
	}
	const float s = (m - 1.0f) / (m + 1.0f);
	const float z = s * s;
	float p = 2.0f / 13.0f;
	p = fmaf(p, z, 2.0f / 11.0f);
	p = fmaf(p, z, 2.0f / 9.0f);
	p = fmaf(p, z, 2.0f / 7.0f);
	p = fmaf(p, z, 2.0f / 5.0f);
	p = fmaf(p, z, 2.0f / 3.0f);
	const float log_m = fmaf(s * z, p, 2.0f * s);
	const float ef = (float)e;
	const float ln2_hi = 0.693145751953125f;      /* 0x3f317200 */
	const float ln2_lo = 1.428606765330187e-06f;  /* ln2 - ln2_hi, rounded */
	return fmaf(ef, ln2_hi, fmaf(ef, ln2_lo, log_m));
}

/*
 * 2^x, written from the textbook reduction 2^x = 2^n * 2^f with n = rint(x) and f = x - n in
 * [-1/2, 1/2] (exact), and a degree-6 polynomial for 2^f: the interpolant of 2^f at the seven
 * Chebyshev nodes of [-1/2, 1/2] (computed in double, coefficients rounded to float), by Horner's
 * rule in fmaf; 2^n is applied exactly by ldexpf. Measured against 2^x in double over [-24, 0]:
 * at most 0.96 ulp. x is clamped to [-150, 128] first, so n fits an int (below -149 the result is
 * 0 either way). Only correctly rounded operations, so the bits are the same on the CPU and on
 * gfx950.
 */
HDS_HD float hds_exp2f(float x) {
	x = fminf(fmaxf(x, -150.0f), 128.0f);
	const float n = rintf(x);
	const float f = x - n;
	float p = 0x1.444000p-13f;
	p = fmaf(p, f, 0x1.5f48c0p-10f);
	p = fmaf(p, f, 0x1.3b2a1cp-7f);
	p = fmaf(p, f, 0x1.c6aeccp-5f);
	p = fmaf(p, f, 0x1.ebfbe0p-3f);
	p = fmaf(p, f, 0x1.62e430p-1f);
	p = fmaf(p, f, 1.0f);
	return ldexpf(p, (int)n);
}

/*
 * Alpha of a gaussian at a pixel centre (forward.cu:197-208): opacity * exp(-m / 2) with
 * m = d^T Q d, d = (dx, dy) = pixel centre - mean and Q = [[a, b], [b, c]] the conic, computed as
 * hds_exp2f(m * (-log2(e) / 2)). The quadratic form is spelled out in fmaf, so no compiler
 * contraction can change it. Stores G = exp(-m / 2). The blend kernels and the oracle both
 * evaluate alpha here, so they take every alpha >= 1/255 and T >= 1e-4 decision identically.
 */
HDS_HD float hds_gauss_alpha(float dx, float dy, float a, float b, float c, float opacity, float* G) {
	const float m = fmaf(dx, fmaf(a, dx, b * dy), dy * fmaf(b, dx, c * dy));
	*G = hds_exp2f(m * -0x1.715476p-1f);
	return opacity * *G;
}

/*
 * floor() then conversion to int, saturating: NaN maps to 0 and out-of-range values clamp to the
 * int range. This pins down what a bare (int)floorf(x) leaves to the hardware (the reference's
 * pixel_to_tile, common.cuh:19-21, runs on a GPU whose conversion saturates and maps NaN to 0),
 * so the CPU and the GPU agree for degenerate conics too.
 */
HDS_HD int hds_floor_to_int(float x) {
	if (x != x) return 0;
	const float f = floorf(x);
	if (f >= 2147483648.0f) return 2147483647;
	if (f < -2147483648.0f) return (int)(-2147483647 - 1);
	return (int)f;
}

/*
 * Half extents (x, y) of the box where a gaussian of this conic and opacity can reach MIN_ALPHA:
 * op * exp(-m/2) >= 1/255  <=>  m <= k^2 with k = sqrt(2 ln(255 op)), and the ellipse d^T Q d <= k^2
 * has half widths k*sqrt(Sigma_xx), k*sqrt(Sigma_yy), where Sigma = Q^-1 gives
 * Sigma_xx = c/det, Sigma_yy = a/det. Follows alpha_extent, common.cuh:49-53.
 */
HDS_HD void hds_alpha_extent(float a, float b, float c, float opacity, float* ex, float* ey) {
	const float k = sqrtf(2.0f * hds_logf(opacity / HDS_MIN_ALPHA));
	const float det = a * c - b * b;
	*ex = k * sqrtf(c / det);
	*ey = k * sqrtf(a / det);
}

/*
 * Tile rectangle a gaussian can touch, clamped to the grid: tile_rect, common.cuh:55-65.
 * Returns 1 and fills (x0, y0, w, h) when the rectangle is non-empty, else 0. The opacity test is
 * written !(op > MIN_ALPHA) so a NaN opacity is culled.
 */
HDS_HD int hds_tile_rect(float ux, float uy, float a, float b, float c, float opacity, int tiles_x,
						 int tiles_y, int* x0, int* y0, int* w, int* h) {
	if (!(opacity > HDS_MIN_ALPHA)) return 0;
	float ex, ey;
	hds_alpha_extent(a, b, c, opacity, &ex, &ey);
	const int lo_x = hds_floor_to_int((ux - ex) / (float)HDS_TILE);
	const int lo_y = hds_floor_to_int((uy - ey) / (float)HDS_TILE);
	const int hi_x = hds_floor_to_int((ux + ex) / (float)HDS_TILE);
	const int hi_y = hds_floor_to_int((uy + ey) / (float)HDS_TILE);
	const int64_t min_x = lo_x > 0 ? lo_x : 0;
	const int64_t min_y = lo_y > 0 ? lo_y : 0;
	const int64_t max_x = hi_x < tiles_x - 1 ? hi_x : tiles_x - 1;
	const int64_t max_y = hi_y < tiles_y - 1 ? hi_y : tiles_y - 1;
	const int64_t sx = max_x - min_x + 1;
	const int64_t sy = max_y - min_y + 1;
	if (sx <= 0 || sy <= 0) return 0;
	*x0 = (int)min_x;
	*y0 = (int)min_y;
	*w = (int)sx;
	*h = (int)sy;
	return 1;
}

#endif /* HDS_COMMON_H */
