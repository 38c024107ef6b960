/*
 * CPU oracle for the high-dimensional splatting rasterizer path. TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, on the CPU in float32, the reference's algorithm for every stage of the hot
 * path: projection (+backward), spherical harmonics (+backward fused with Adam), tile binning
 * (cull, tile rectangles, stable (tile, depth) ordering, tile ranges), the front-to-back RGB +
 * C-channel blend and its back-to-front replay backward, and the SSIM loss kernels. Each function
 * cites the reference file:line it follows (paths relative to the reference repository root,
 * gaussian_splatting/rasterizer/ unless stated).
 *
 * It is the checker, never the product: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. The product path is the HIP library, which has no CPU fallback.
 *
 * Differences from the reference, all deliberate:
 *   - The blend takes alpha from hds_gauss_alpha (hds_common.h: the quadratic form in fmaf and an
 *     exp2 of its own, shared with the HIP kernels) where the reference uses __expf, accumulates
 *     RGB and the background term with fmaf as the HIP forward does, and uses plain float products
 *     where the reference's feature kernel rounds weights and features to TF32
 *     (features.cu:50-58). So alpha, T, n_contrib and the RGB image come out bit for bit as on the
 *     GPU; the feature channels are the float32 semantics of tests/oracle.py.
 *   - The natural log inside tile_rect is hds_logf (hds_common.h), shared with the HIP kernels,
 *     so integer binning results can be compared bit for bit.
 *
 * Pinning (how this oracle is itself checked; see tests/test_oracle_pinning.py):
 *   projection fwd: closed form of an isotropic gaussian on the axis, near-plane and off-screen
 *     culling, an independent float64 torch matrix formulation, rigid motion of scene and camera;
 *   projection bwd: torch autograd of that float64 matrix formulation, including the clamped
 *     field-of-view and near-plane branches;
 *   SH fwd: orthonormality of the basis on the sphere, rgb_to_sh inverse, hand values at the poles;
 *   SH bwd + Adam: torch autograd of the closed form and torch.optim.Adam(fused=False);
 *   binning: brute-force enumeration of every (tile, gaussian) with the alpha test in float64;
 *   blend fwd: dense float64 cumprod formulation (tests/oracle.py semantics) + hand-solved pixels;
 *   blend bwd: torch autograd through that dense float64 formulation;
 *   SSIM: torch conv2d in float64 and ssim(x, x) = 1.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "hds_common.h"
#include "hds_ewa.h"

#define ORC_EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------------------------- */
/* Shared-arithmetic probes, so tests can pin hds_logf and hds_tile_rect directly.              */
/* ------------------------------------------------------------------------------------------- */

ORC_EXPORT float orc_logf(float x) { return hds_logf(x); }

/* hds_exp2f over an array (pinned by tests/test_oracle_pinning.py against 2^x in double). */
ORC_EXPORT void orc_exp2f(int64_t n, const float* x, float* y) {
	for (int64_t i = 0; i < n; i++) y[i] = hds_exp2f(x[i]);
}

ORC_EXPORT int orc_tile_rect(float ux, float uy, float a, float b, float c, float op, int tiles_x,
							 int tiles_y, int* rect4) {
	return hds_tile_rect(ux, uy, a, b, c, op, tiles_x, tiles_y, &rect4[0], &rect4[1], &rect4[2],
						 &rect4[3]);
}

/* ------------------------------------------------------------------------------------------- */
/* Projection: project_gaussians, projection.cu:36-111 (forward) and 114-197 (backward),         */
/* constants projection.py:3-5. The per-gaussian arithmetic is hds_ewa.h, shared with the HIP     */
/* kernels (the same bits on both sides); tests/test_oracle_pinning.py pins it against an         */
/* independent float64 matrix formulation and its autograd, closed forms and rigid motion.        */
/* ------------------------------------------------------------------------------------------- */

ORC_EXPORT void orc_project_forward(int64_t n, const float* means, const float* scales,
									const float* quats, const float* opacities, const float* w2c,
									float fx, float fy, float cx, float cy, int width, int height,
									float near_plane, float low_pass, float fov_scale,
									float* means2D, float* depths, float* radii, float* conics) {
	const hds_camera cam = {fx, fy, cx, cy, width, height, near_plane, low_pass, fov_scale};
#pragma omp parallel for schedule(static)
	for (int64_t i = 0; i < n; i++) {
		hds_ewa g;
		hds_ewa_project(&cam, w2c, means + i * 3, scales + i * 3, quats + i * 4, &g);
		hds_ewa_screen(&cam, &g, opacities[i], means2D + i * 2, depths + i, conics + i * 3, radii + i);
	}
}

ORC_EXPORT void orc_project_backward(int64_t n, const float* grad_means2D, const float* grad_conics,
									 const float* means, const float* scales, const float* quats,
									 const float* w2c, float fx, float fy, float cx, float cy,
									 int width, int height, float near_plane, float low_pass,
									 float fov_scale, float* grad_means, float* grad_scales,
									 float* grad_quats) {
	const hds_camera cam = {fx, fy, cx, cy, width, height, near_plane, low_pass, fov_scale};
#pragma omp parallel for schedule(static)
	for (int64_t i = 0; i < n; i++) {
		hds_ewa g;
		hds_ewa_project(&cam, w2c, means + i * 3, scales + i * 3, quats + i * 4, &g);
		hds_ewa_backward(&cam, w2c, scales + i * 3, quats + i * 4, &g, grad_means2D + i * 2, grad_conics + i * 3,
						 grad_means + i * 3, grad_scales + i * 3, grad_quats + i * 4);
	}
}

/* ------------------------------------------------------------------------------------------- */
/* Spherical harmonics: basis sh.cu:9-31, gradients sh.cu:34-55, forward sh.cu:62-83,           */
/* backward + Adam sh.cu:85-154, utils/sh.py:62-109.                                            */
/* ------------------------------------------------------------------------------------------- */

/* Real SH constants of degrees 0-3 in the 3DGS sign convention (sh.cu:9-15, test_sh.py:27-47). */
static const float ORC_SH_C[16] = {
	0.28209479177387814f,  -0.4886025119029199f, 0.4886025119029199f,  -0.4886025119029199f,
	1.0925484305920792f,   -1.0925484305920792f, 0.31539156525252005f, -1.0925484305920792f,
	0.5462742152960396f,   -0.5900435899266435f, 2.890611442640554f,   -0.4570457994644658f,
	0.3731763325901154f,   -0.4570457994644658f, 1.445305721320277f,   -0.5900435899266435f,
};

static void orc_sh_basis(float x, float y, float z, int k, float* b) {
	const float xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
	const float* C = ORC_SH_C;
	b[0] = C[0];
	if (k <= 1) return;
	b[1] = C[1] * y;
	b[2] = C[2] * z;
	b[3] = C[3] * x;
	if (k <= 4) return;
	b[4] = C[4] * xy;
	b[5] = C[5] * yz;
	b[6] = C[6] * (2 * zz - xx - yy);
	b[7] = C[7] * xz;
	b[8] = C[8] * (xx - yy);
	if (k <= 9) return;
	b[9] = C[9] * y * (3 * xx - yy);
	b[10] = C[10] * xy * z;
	b[11] = C[11] * y * (4 * zz - xx - yy);
	b[12] = C[12] * z * (2 * zz - 3 * xx - 3 * yy);
	b[13] = C[13] * x * (4 * zz - xx - yy);
	b[14] = C[14] * z * (xx - yy);
	b[15] = C[15] * x * (xx - 3 * yy);
}

static void orc_sh_basis_grad(float x, float y, float z, int k, float* bx, float* by, float* bz) {
	const float xx = x * x, yy = y * y, zz = z * z;
	const float* C = ORC_SH_C;
	for (int j = 0; j < 16; j++) bx[j] = by[j] = bz[j] = 0.0f;
	if (k <= 1) return;
	by[1] = C[1];
	bz[2] = C[2];
	bx[3] = C[3];
	if (k <= 4) return;
	bx[4] = C[4] * y;
	by[4] = C[4] * x;
	by[5] = C[5] * z;
	bz[5] = C[5] * y;
	bx[6] = C[6] * (-2 * x);
	by[6] = C[6] * (-2 * y);
	bz[6] = C[6] * (4 * z);
	bx[7] = C[7] * z;
	bz[7] = C[7] * x;
	bx[8] = C[8] * (2 * x);
	by[8] = C[8] * (-2 * y);
	if (k <= 9) return;
	bx[9] = C[9] * (6 * x * y);
	by[9] = C[9] * (3 * xx - 3 * yy);
	bx[10] = C[10] * y * z;
	by[10] = C[10] * x * z;
	bz[10] = C[10] * x * y;
	bx[11] = C[11] * (-2 * x * y);
	by[11] = C[11] * (4 * zz - xx - 3 * yy);
	bz[11] = C[11] * (8 * y * z);
	bx[12] = C[12] * (-6 * x * z);
	by[12] = C[12] * (-6 * y * z);
	bz[12] = C[12] * (6 * zz - 3 * xx - 3 * yy);
	bx[13] = C[13] * (4 * zz - 3 * xx - yy);
	by[13] = C[13] * (-2 * x * y);
	bz[13] = C[13] * (8 * x * z);
	bx[14] = C[14] * (2 * x * z);
	by[14] = C[14] * (-2 * y * z);
	bz[14] = C[14] * (xx - yy);
	bx[15] = C[15] * (3 * xx - 3 * yy);
	by[15] = C[15] * (-6 * x * y);
}

static float orc_sh_weight(const float* dc, const float* rest, int j, int c) {
	return j == 0 ? dc[c] : rest[(j - 1) * 3 + c];
}

/* eval_sh_forward: sh.cu:62-83. rgb = max(0.5 + sum_j b_j w_j, 0); culled -> 0. */
ORC_EXPORT void orc_eval_sh(int64_t n, int degree, const float* sh_dc, const float* sh_rest,
							const float* dirs, const float* radii, float* rgb) {
	const int k = (degree + 1) * (degree + 1);
#pragma omp parallel for schedule(static)
	for (int64_t i = 0; i < n; i++) {
		if (!(radii[i] > 0.0f)) {
			rgb[i * 3 + 0] = rgb[i * 3 + 1] = rgb[i * 3 + 2] = 0.0f;
			continue;
		}
		float b[16];
		orc_sh_basis(dirs[i * 3 + 0], dirs[i * 3 + 1], dirs[i * 3 + 2], k, b);
		const float* dc = sh_dc + i * 3;
		const float* rest = sh_rest + i * 45;
		for (int c = 0; c < 3; c++) {
			float value = 0.5f;
			for (int j = 0; j < k; j++) value += b[j] * orc_sh_weight(dc, rest, j, c);
			rgb[i * 3 + c] = fmaxf(value, 0.0f);
		}
	}
}

/*
 * eval_sh_backward_adam: sh.cu:104-154 with the host-side parameters of sh.cu:171-190. SH
 * gradients b_j g_c (zero where the colour clamped or the gaussian is culled), grad_dirs from the
 * basis gradients, then one Adam step on sh_dc and sh_rest in place:
 *   m += (1-b1)(g-m); v = b2 v + (1-b2) g^2; p -= lr/(1-b1^t) * m / (sqrt(v)/sqrt(1-b2^t) + eps),
 * with 1-b formed in double as the reference host does (sh.cu:85, 179-180).
 */
ORC_EXPORT void orc_eval_sh_backward_adam(int64_t n, int degree, const float* grad_rgb, float* sh_dc,
										  float* sh_rest, const float* dirs, const float* radii,
										  float* m_dc, float* v_dc, float* m_rest, float* v_rest,
										  float step_dc, float step_rest, double lr_dc,
										  double lr_rest, double beta1, double beta2, double eps,
										  float* grad_dirs) {
	const int k = (degree + 1) * (degree + 1);
	const float b1 = (float)beta1, b2 = (float)beta2;
	const float omb1 = (float)(1.0 - beta1), omb2 = (float)(1.0 - beta2);
	const float feps = (float)eps;
	const float ss_dc = (float)lr_dc / (1.0f - powf(b1, step_dc));
	const float bc2_dc = sqrtf(1.0f - powf(b2, step_dc));
	const float ss_rest = (float)lr_rest / (1.0f - powf(b1, step_rest));
	const float bc2_rest = sqrtf(1.0f - powf(b2, step_rest));
#pragma omp parallel for schedule(static)
	for (int64_t i = 0; i < n; i++) {
		float gsh[48];
		float dd[3] = {0.0f, 0.0f, 0.0f};
		for (int j = 0; j < 48; j++) gsh[j] = 0.0f;
		if (radii[i] > 0.0f) {
			float b[16], bx[16], by[16], bz[16];
			const float x = dirs[i * 3 + 0], y = dirs[i * 3 + 1], z = dirs[i * 3 + 2];
			orc_sh_basis(x, y, z, k, b);
			orc_sh_basis_grad(x, y, z, k, bx, by, bz);
			const float* dc = sh_dc + i * 3;
			const float* rest = sh_rest + i * 45;
			float g[3];
			for (int c = 0; c < 3; c++) {
				float value = 0.5f;
				for (int j = 0; j < k; j++) value += b[j] * orc_sh_weight(dc, rest, j, c);
				g[c] = value > 0.0f ? grad_rgb[i * 3 + c] : 0.0f;
			}
			for (int j = 0; j < k; j++) {
				float t = 0.0f;
				for (int c = 0; c < 3; c++) {
					gsh[j * 3 + c] = b[j] * g[c];
					t += orc_sh_weight(dc, rest, j, c) * g[c];
				}
				dd[0] += t * bx[j];
				dd[1] += t * by[j];
				dd[2] += t * bz[j];
			}
		}
		for (int c = 0; c < 3; c++) grad_dirs[i * 3 + c] = dd[c];
		for (int j = 0; j < 48; j++) {
			float* p = j < 3 ? &sh_dc[i * 3 + j] : &sh_rest[i * 45 + (j - 3)];
			float* m = j < 3 ? &m_dc[i * 3 + j] : &m_rest[i * 45 + (j - 3)];
			float* v = j < 3 ? &v_dc[i * 3 + j] : &v_rest[i * 45 + (j - 3)];
			const float ss = j < 3 ? ss_dc : ss_rest;
			const float bc2 = j < 3 ? bc2_dc : bc2_rest;
			const float grad = gsh[j];
			const float mt = *m + omb1 * (grad - *m);
			const float vt = b2 * *v + omb2 * grad * grad;
			*m = mt;
			*v = vt;
			*p -= ss * mt / (sqrtf(vt) / bc2 + feps);
		}
	}
}

/* ------------------------------------------------------------------------------------------- */
/* Binning: prepare_gaussians forward.cu:13-61, scan + pair count forward.cu:311-325,            */
/* duplicate_gaussians forward.cu:82-113, stable radix sort on (tile<<32 | depth bits)           */
/* forward.cu:363-394, identify_tile_ranges forward.cu:115-139.                                 */
/* ------------------------------------------------------------------------------------------- */

/* Tiles each gaussian touches (0 when culled), and the total pair count P. */
ORC_EXPORT int64_t orc_bin_count(int64_t n, const float* means2D, const float* radii,
								 const float* conics, const float* opacities, int width, int height,
								 int32_t* counts, int32_t* rects) {
	const int tiles_x = (width + HDS_TILE - 1) / HDS_TILE;
	const int tiles_y = (height + HDS_TILE - 1) / HDS_TILE;
	int64_t total = 0;
#pragma omp parallel for schedule(static) reduction(+ : total)
	for (int64_t i = 0; i < n; i++) {
		int x0 = 0, y0 = 0, w = 0, h = 0;
		int ok = radii[i] > 0.0f &&
				 hds_tile_rect(means2D[i * 2], means2D[i * 2 + 1], conics[i * 3], conics[i * 3 + 1],
							   conics[i * 3 + 2], opacities[i], tiles_x, tiles_y, &x0, &y0, &w, &h);
		counts[i] = ok ? w * h : 0;
		if (rects) {
			rects[i * 4 + 0] = x0;
			rects[i * 4 + 1] = y0;
			rects[i * 4 + 2] = ok ? w : 0;
			rects[i * 4 + 3] = ok ? h : 0;
		}
		total += counts[i];
	}
	return total;
}

typedef struct {
	uint64_t key;
	int32_t gid;
} orc_pair;

static int orc_pair_cmp(const void* pa, const void* pb) {
	const orc_pair* a = (const orc_pair*)pa;
	const orc_pair* b = (const orc_pair*)pb;
	if (a->key != b->key) return a->key < b->key ? -1 : 1;
	/* Equal keys come from different gaussians: keep index order, as a stable sort would. */
	return (a->gid > b->gid) - (a->gid < b->gid);
}

/* Pairs that fall in the tiles with tile_mask[tile] != 0 (tile_mask [T] bytes, row-major). */
ORC_EXPORT int64_t orc_bin_count_masked(int64_t n, const int32_t* rects, const uint8_t* tile_mask, int width) {
	const int tiles_x = (width + HDS_TILE - 1) / HDS_TILE;
	int64_t total = 0;
#pragma omp parallel for schedule(static) reduction(+ : total)
	for (int64_t i = 0; i < n; i++) {
		const int x0 = rects[i * 4], y0 = rects[i * 4 + 1], w = rects[i * 4 + 2], h = rects[i * 4 + 3];
		for (int y = y0; y < y0 + h; y++)
			for (int x = x0; x < x0 + w; x++) total += tile_mask[y * tiles_x + x] != 0;
	}
	return total;
}

/*
 * Emits every (tile, gaussian) pair, sorts by (tile, float bits of depth) keeping index order on
 * ties, and builds [start, end) per tile, zero for untouched tiles. Outputs values_sorted[P] and
 * tile_ranges[T][2] exactly as the reference rasterize returns them (forward.cu:434).
 *
 * With tile_mask != NULL only the pairs of the tiles whose mask byte is set are emitted: their
 * lists are exactly the full binning's lists for those tiles (the order inside a tile depends only
 * on the tile's own pairs), and every other tile is empty. Tiles are independent in the blend, so
 * rendering such a binning reproduces the full frame on the masked tiles, and the backward with an
 * upstream gradient that is zero outside them reproduces the full backward.
 */
ORC_EXPORT void orc_bin_fill(int64_t n, const float* depths, const int32_t* counts,
							 const int32_t* rects, int width, int height, int64_t num_pairs,
							 const uint8_t* tile_mask, int32_t* values_sorted, int32_t* tile_ranges) {
	const int tiles_x = (width + HDS_TILE - 1) / HDS_TILE;
	const int tiles_y = (height + HDS_TILE - 1) / HDS_TILE;
	orc_pair* pairs = (orc_pair*)malloc(sizeof(orc_pair) * (size_t)(num_pairs > 0 ? num_pairs : 1));
	int64_t o = 0;
	for (int64_t i = 0; i < n; i++) {
		if (counts[i] == 0) continue;
		uint32_t depth_bits = hds_f2u(depths[i]);
		const int x0 = rects[i * 4], y0 = rects[i * 4 + 1], w = rects[i * 4 + 2], h = rects[i * 4 + 3];
		for (int y = y0; y < y0 + h; y++)
			for (int x = x0; x < x0 + w; x++) {
				if (tile_mask && !tile_mask[y * tiles_x + x]) continue;
				pairs[o].key = ((uint64_t)(uint32_t)(y * tiles_x + x) << 32) | depth_bits;
				pairs[o].gid = (int32_t)i;
				o++;
			}
	}
	qsort(pairs, (size_t)o, sizeof(orc_pair), orc_pair_cmp);
	memset(tile_ranges, 0, sizeof(int32_t) * 2 * (size_t)tiles_x * (size_t)tiles_y);
	for (int64_t p = 0; p < o; p++) {
		values_sorted[p] = pairs[p].gid;
		const uint32_t tile = (uint32_t)(pairs[p].key >> 32);
		if (p == 0 || (uint32_t)(pairs[p - 1].key >> 32) != tile) tile_ranges[tile * 2 + 0] = (int32_t)p;
		if (p == o - 1 || (uint32_t)(pairs[p + 1].key >> 32) != tile) tile_ranges[tile * 2 + 1] = (int32_t)(p + 1);
	}
	free(pairs);
}

/* ------------------------------------------------------------------------------------------- */
/* Blend forward: render_gaussians forward.cu:141-237 (RGB, background), render_features       */
/* features.cu:116-282 (same weights, zero background, last = index + 1).                        */
/* ------------------------------------------------------------------------------------------- */

/* alpha of gaussian (mean, conic, opacity) at a pixel centre: forward.cu:197-208. */
static inline float orc_alpha(float px, float py, const float* mean, const float* conic, float opacity,
							  float* gauss, float* dx_out, float* dy_out) {
	const float dx = px - mean[0];
	const float dy = py - mean[1];
	*dx_out = dx;
	*dy_out = dy;
	return hds_gauss_alpha(dx, dy, conic[0], conic[1], conic[2], opacity, gauss);
}

/*
 * RGB (when colors != NULL) and C feature channels (when features != NULL), front to back per
 * pixel over its tile's sorted list. Pixel centres are at +0.5. A gaussian with alpha < 1/255 is
 * skipped but still counted in the list index; one that would leave T < 1e-4 ends the pixel
 * without blending. n_contrib is the 1-based list index of the last blended gaussian.
 */
/*
 * near_cut (optional, [H, W] bytes) marks the pixels whose walk passed a decision within rounding
 * distance of its cut, where an implementation that rounds differently (another exp, other fused
 * multiply-adds; the HIP kernels share this file's alpha arithmetic and decide identically) could
 * decide the other way:
 *   - a raw alpha against 1/255: alpha = op exp(-m / 2) is uncertain by a relative
 *     eps_a = u (2 (|a dx^2| + 2 |b dx dy| + |c dy^2|) + m / 2 + 4), u = 2^-24: a few roundings of
 *     the quadratic form's terms (which can cancel) carried through exp, the rounding of exp's
 *     argument and a few ulps of exp itself;
 *   - T (1 - alpha) against the 1e-4 floor, T carrying the sum of its factors' uncertainties
 *     (alpha's, scaled by alpha / (1 - alpha), plus u per step).
 * A decision counts as near when the value is within twice its uncertainty of the cut.
 */
#define ORC_U 5.9604645e-08f

ORC_EXPORT void orc_render_forward(int width, int height, const int32_t* tile_ranges,
								   const int32_t* values_sorted, const float* means2D,
								   const float* conics, const float* opacities, const float* colors,
								   const float* background, const float* features, int channels,
								   float* image, float* final_T, int32_t* n_contrib,
								   float* feature_image, uint8_t* near_cut) {
	const int tiles_x = (width + HDS_TILE - 1) / HDS_TILE;
	const int tiles_y = (height + HDS_TILE - 1) / HDS_TILE;
	const int64_t num_tiles = (int64_t)tiles_x * tiles_y;
#pragma omp parallel
	{
		float* acc = (float*)malloc(sizeof(float) * (size_t)(channels > 0 ? channels : 1));
#pragma omp for schedule(dynamic, 1)
		for (int64_t tile = 0; tile < num_tiles; tile++) {
			const int tx = (int)(tile % tiles_x), ty = (int)(tile / tiles_x);
			const int start = tile_ranges[tile * 2], end = tile_ranges[tile * 2 + 1];
			for (int ly = 0; ly < HDS_TILE; ly++)
				for (int lx = 0; lx < HDS_TILE; lx++) {
					const int x = tx * HDS_TILE + lx, y = ty * HDS_TILE + ly;
					if (x >= width || y >= height) continue;
					const float px = (float)x + 0.5f, py = (float)y + 0.5f;
					float T = 1.0f, r = 0.0f, g = 0.0f, b = 0.0f;
					int last = 0, near = 0;
					float eps_T = 0.0f;
					for (int c = 0; c < channels; c++) acc[c] = 0.0f;
					for (int j = start; j < end; j++) {
						const int gid = values_sorted[j];
						float G, dx, dy;
						const float raw = orc_alpha(px, py, means2D + gid * 2, conics + gid * 3,
													opacities[gid], &G, &dx, &dy);
						const float alpha = fminf(HDS_MAX_ALPHA, raw);
						const float* q = conics + gid * 3;
						const float terms = fabsf(q[0] * dx * dx) + 2.0f * fabsf(q[1] * dx * dy) + fabsf(q[2] * dy * dy);
						const float m = -2.0f * logf(G > 0.0f ? G : 1e-30f);
						const float eps_a = ORC_U * (2.0f * terms + 0.5f * m + 4.0f);
						near |= fabsf(raw - HDS_MIN_ALPHA) <= 2.0f * eps_a * raw;
						if (alpha < HDS_MIN_ALPHA) continue;
						const float test_T = T * (1.0f - alpha);
						eps_T += ORC_U + eps_a * alpha / (1.0f - alpha);
						near |= fabsf(test_T - HDS_MIN_TRANSMITTANCE) <= 2.0f * eps_T * test_T;
						if (test_T < HDS_MIN_TRANSMITTANCE) break;
						const float w = alpha * T;
						if (colors) {
							r = fmaf(w, colors[gid * 3 + 0], r);
							g = fmaf(w, colors[gid * 3 + 1], g);
							b = fmaf(w, colors[gid * 3 + 2], b);
						}
						const float* f = features ? features + (int64_t)gid * channels : NULL;
						for (int c = 0; c < channels && f; c++) acc[c] += w * f[c];
						T = test_T;
						last = j - start + 1;
					}
					const int64_t pix = (int64_t)y * width + x;
					if (image) {
						image[pix * 3 + 0] = fmaf(T, background[0], r);
						image[pix * 3 + 1] = fmaf(T, background[1], g);
						image[pix * 3 + 2] = fmaf(T, background[2], b);
					}
					if (final_T) final_T[pix] = T;
					if (n_contrib) n_contrib[pix] = last;
					if (near_cut) near_cut[pix] = (uint8_t)near;
					for (int c = 0; c < channels && feature_image; c++) feature_image[pix * channels + c] = acc[c];
				}
		}
		free(acc);
	}
}

/* ------------------------------------------------------------------------------------------- */
/* Blend backward: render_gaussians_backward backward.cu:7-164 (RGB with background term) and    */
/* render_features_backward features.cu:350-542 (dot / behind_dot recurrence). Both are summed  */
/* into one dL/dalpha before the geometry gradients, which is what the reference's torch add of */
/* the two kernels' outputs computes (rasterizer/__init__.py:160-162).                          */
/* ------------------------------------------------------------------------------------------- */

ORC_EXPORT void orc_render_backward(int width, int height, int64_t n, int64_t num_pairs,
									const int32_t* tile_ranges, const int32_t* values_sorted,
									const float* means2D, const float* conics,
									const float* opacities, const float* colors,
									const float* background, const float* final_T,
									const int32_t* n_contrib, const float* grad_image,
									const float* features, const float* grad_feature_image,
									int channels, float* grad_means2D, float* grad_conics,
									float* grad_colors, float* grad_opacities,
									float* grad_features) {
	const int tiles_x = (width + HDS_TILE - 1) / HDS_TILE;
	const int tiles_y = (height + HDS_TILE - 1) / HDS_TILE;
	const int64_t num_tiles = (int64_t)tiles_x * tiles_y;
	const int C = features ? channels : 0;
	const int K = 9 + C; /* per pair: opacity, mean x/y, conic a/b/c, colour r/g/b, features */
	float* partial = (float*)calloc((size_t)(num_pairs > 0 ? num_pairs : 1) * (size_t)K, sizeof(float));
	const int rgb = grad_image != NULL;
#pragma omp parallel for schedule(dynamic, 1)
		for (int64_t tile = 0; tile < num_tiles; tile++) {
			const int tx = (int)(tile % tiles_x), ty = (int)(tile / tiles_x);
			const int start = tile_ranges[tile * 2];
			for (int ly = 0; ly < HDS_TILE; ly++)
				for (int lx = 0; lx < HDS_TILE; lx++) {
					const int x = tx * HDS_TILE + lx, y = ty * HDS_TILE + ly;
					if (x >= width || y >= height) continue;
					const int64_t pix = (int64_t)y * width + x;
					const float px = (float)x + 0.5f, py = (float)y + 0.5f;
					const int last = n_contrib[pix];
					const float T_final = final_T[pix];
					float T = T_final;
					float gr = 0, gg = 0, gb = 0, dL_dT_final = 0;
					if (rgb) {
						gr = grad_image[pix * 3 + 0];
						gg = grad_image[pix * 3 + 1];
						gb = grad_image[pix * 3 + 2];
						dL_dT_final = background[0] * gr + background[1] * gg + background[2] * gb;
					}
					const float* gf = C ? grad_feature_image + pix * C : NULL;
					float rec_r = 0, rec_g = 0, rec_b = 0, last_alpha = 0;
					float last_r = 0, last_g = 0, last_b = 0, behind_dot = 0;
					for (int j = last - 1; j >= 0; j--) {
						const int gid = values_sorted[start + j];
						float G, dx, dy;
						const float* conic = conics + gid * 3;
						const float op = opacities[gid];
						const float raw = orc_alpha(px, py, means2D + gid * 2, conic, op, &G, &dx, &dy);
						const float alpha = fminf(HDS_MAX_ALPHA, raw);
						if (alpha < HDS_MIN_ALPHA) continue;
						const float inv_1ma = 1.0f / (1.0f - alpha);
						T = T * inv_1ma;
						float* out = partial + (size_t)(start + j) * (size_t)K;
						float dL_dalpha = 0.0f;
						const float weight = alpha * T;
						if (rgb) {
							const float cr = colors[gid * 3], cg = colors[gid * 3 + 1], cb = colors[gid * 3 + 2];
							rec_r = last_alpha * last_r + (1.0f - last_alpha) * rec_r;
							rec_g = last_alpha * last_g + (1.0f - last_alpha) * rec_g;
							rec_b = last_alpha * last_b + (1.0f - last_alpha) * rec_b;
							last_r = cr;
							last_g = cg;
							last_b = cb;
							last_alpha = alpha;
							dL_dalpha = ((cr - rec_r) * gr + (cg - rec_g) * gg + (cb - rec_b) * gb) * T -
										T_final * inv_1ma * dL_dT_final;
							out[6] += weight * gr;
							out[7] += weight * gg;
							out[8] += weight * gb;
						}
						if (C) {
							const float* f = features + (int64_t)gid * C;
							float dot = 0.0f;
							for (int c = 0; c < C; c++) dot += f[c] * gf[c];
							dL_dalpha += T * (dot - behind_dot);
							behind_dot = alpha * dot + (1.0f - alpha) * behind_dot;
							for (int c = 0; c < C; c++) out[9 + c] += weight * gf[c];
						}
						/* A clamped alpha no longer depends on the gaussian: backward.cu:126-135. */
						if (raw <= HDS_MAX_ALPHA) {
							const float dL_dG = op * dL_dalpha;
							out[0] += G * dL_dalpha;
							out[1] += dL_dG * G * (conic[0] * dx + conic[1] * dy);
							out[2] += dL_dG * G * (conic[1] * dx + conic[2] * dy);
							out[3] += dL_dG * G * -0.5f * dx * dx;
							out[4] += dL_dG * G * -dx * dy;
							out[5] += dL_dG * G * -0.5f * dy * dy;
						}
					}
				}
		}
	/* Deterministic reduction, in sorted pair order, of the per-pair partials into gaussians. */
	if (grad_means2D) memset(grad_means2D, 0, sizeof(float) * 2 * (size_t)n);
	if (grad_conics) memset(grad_conics, 0, sizeof(float) * 3 * (size_t)n);
	if (grad_colors) memset(grad_colors, 0, sizeof(float) * 3 * (size_t)n);
	if (grad_opacities) memset(grad_opacities, 0, sizeof(float) * (size_t)n);
	if (grad_features && C) memset(grad_features, 0, sizeof(float) * (size_t)C * (size_t)n);
	for (int64_t p = 0; p < num_pairs; p++) {
		const int gid = values_sorted[p];
		const float* in = partial + (size_t)p * (size_t)K;
		if (grad_opacities) grad_opacities[gid] += in[0];
		if (grad_means2D) {
			grad_means2D[gid * 2 + 0] += in[1];
			grad_means2D[gid * 2 + 1] += in[2];
		}
		if (grad_conics) {
			grad_conics[gid * 3 + 0] += in[3];
			grad_conics[gid * 3 + 1] += in[4];
			grad_conics[gid * 3 + 2] += in[5];
		}
		if (grad_colors && rgb) {
			grad_colors[gid * 3 + 0] += in[6];
			grad_colors[gid * 3 + 1] += in[7];
			grad_colors[gid * 3 + 2] += in[8];
		}
		if (grad_features && C)
			for (int c = 0; c < C; c++) grad_features[(int64_t)gid * C + c] += in[9 + c];
	}
	free(partial);
}

/* ------------------------------------------------------------------------------------------- */
/* SSIM: ssim.cu:18-113 (separable zero-padded 11-tap blur, sigma 1.5), utils/loss.py:8-9, 74.  */
/* ------------------------------------------------------------------------------------------- */

static void orc_ssim_window(float* g) {
	double w[11], s = 0.0;
	for (int i = 0; i < 11; i++) {
		const double x = (double)(i - 5);
		w[i] = exp(-x * x / (2.0 * 1.5 * 1.5));
		s += w[i];
	}
	for (int i = 0; i < 11; i++) g[i] = (float)(w[i] / s);
}

/* Horizontal then vertical blur of five moments, SSIM map and its partials: ssim.cu:18-72. */
ORC_EXPORT void orc_ssim_forward(int height, int width, const float* a, const float* b,
								 float* ssim_map, float* d_mu, float* d_aa, float* d_ab) {
	const float C1 = 0.01f * 0.01f, C2 = 0.03f * 0.03f;
	float G[11];
	orc_ssim_window(G);
	const int64_t n = (int64_t)height * width * 3;
	float* h = (float*)malloc(sizeof(float) * 5 * (size_t)n);
#pragma omp parallel for schedule(static)
	for (int64_t i = 0; i < n; i++) {
		const int x = (int)((i / 3) % width);
		float sa = 0, sb = 0, saa = 0, sbb = 0, sab = 0;
		for (int k = -5; k <= 5; k++) {
			if (x + k < 0 || x + k >= width) continue;
			const float w = G[k + 5], va = a[i + 3 * k], vb = b[i + 3 * k];
			sa += w * va;
			sb += w * vb;
			saa += w * va * va;
			sbb += w * vb * vb;
			sab += w * va * vb;
		}
		h[i] = sa;
		h[n + i] = sb;
		h[2 * n + i] = saa;
		h[3 * n + i] = sbb;
		h[4 * n + i] = sab;
	}
	const int64_t row = 3 * (int64_t)width;
#pragma omp parallel for schedule(static)
	for (int64_t i = 0; i < n; i++) {
		const int y = (int)(i / row);
		float mu_a = 0, mu_b = 0, e_aa = 0, e_bb = 0, e_ab = 0;
		for (int k = -5; k <= 5; k++) {
			if (y + k < 0 || y + k >= height) continue;
			const float w = G[k + 5];
			const int64_t j = i + k * row;
			mu_a += w * h[j];
			mu_b += w * h[n + j];
			e_aa += w * h[2 * n + j];
			e_bb += w * h[3 * n + j];
			e_ab += w * h[4 * n + j];
		}
		const float a1 = 2.0f * mu_a * mu_b + C1;
		const float a2 = 2.0f * (e_ab - mu_a * mu_b) + C2;
		const float b1 = mu_a * mu_a + mu_b * mu_b + C1;
		const float b2 = (e_aa - mu_a * mu_a) + (e_bb - mu_b * mu_b) + C2;
		const float inv_b = 1.0f / (b1 * b2);
		const float s = a1 * a2 * inv_b;
		ssim_map[i] = s;
		d_mu[i] = (2.0f * mu_b * (a2 - a1) - 2.0f * mu_a * s * (b2 - b1)) * inv_b;
		d_aa[i] = -s / b2;
		d_ab[i] = 2.0f * a1 * inv_b;
	}
	free(h);
}

/* grad = dL/dmean / n * (blur(d_mu) + 2a blur(d_aa) + b blur(d_ab)): ssim.cu:74-113. */
ORC_EXPORT void orc_ssim_backward(int height, int width, float grad_mean, const float* a,
								  const float* b, const float* d_mu, const float* d_aa,
								  const float* d_ab, float* grad) {
	float G[11];
	orc_ssim_window(G);
	const int64_t n = (int64_t)height * width * 3;
	float* h = (float*)malloc(sizeof(float) * 3 * (size_t)n);
#pragma omp parallel for schedule(static)
	for (int64_t i = 0; i < n; i++) {
		const int x = (int)((i / 3) % width);
		float s_mu = 0, s_aa = 0, s_ab = 0;
		for (int k = -5; k <= 5; k++) {
			if (x + k < 0 || x + k >= width) continue;
			const float w = G[k + 5];
			s_mu += w * d_mu[i + 3 * k];
			s_aa += w * d_aa[i + 3 * k];
			s_ab += w * d_ab[i + 3 * k];
		}
		h[i] = s_mu;
		h[n + i] = s_aa;
		h[2 * n + i] = s_ab;
	}
	const int64_t row = 3 * (int64_t)width;
	const float scale = grad_mean / (float)n;
#pragma omp parallel for schedule(static)
	for (int64_t i = 0; i < n; i++) {
		const int y = (int)(i / row);
		float s_mu = 0, s_aa = 0, s_ab = 0;
		for (int k = -5; k <= 5; k++) {
			if (y + k < 0 || y + k >= height) continue;
			const float w = G[k + 5];
			const int64_t j = i + k * row;
			s_mu += w * h[j];
			s_aa += w * h[n + j];
			s_ab += w * h[2 * n + j];
		}
		grad[i] = scale * (s_mu + 2.0f * a[i] * s_aa + b[i] * s_ab);
	}
	free(h);
}
