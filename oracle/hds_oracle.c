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
 *   - The blend uses libm expf where the reference uses __expf, and plain float products where the
 *     reference's feature kernel rounds weights and features to TF32 (features.cu:50-58). So this
 *     is the float32 semantics of tests/oracle.py, not the L4's rounding.
 *   - The natural log inside tile_rect is hds_logf (hds_common.h), shared with the HIP kernels,
 *     so integer binning results can be compared bit for bit.
 *
 * Pinning (how this oracle is itself checked; see tests/test_oracle_*.py):
 *   projection fwd: closed-form special cases and rigid-motion / mirror invariance;
 *   projection bwd: central finite differences of the forward, in float64 on the restated math;
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

#define ORC_EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------------------------- */
/* Shared-arithmetic probes, so tests can pin hds_logf and hds_tile_rect directly.              */
/* ------------------------------------------------------------------------------------------- */

ORC_EXPORT float orc_logf(float x) { return hds_logf(x); }

ORC_EXPORT int orc_tile_rect(float ux, float uy, float a, float b, float c, float op, int tiles_x,
							 int tiles_y, int* rect4) {
	return hds_tile_rect(ux, uy, a, b, c, op, tiles_x, tiles_y, &rect4[0], &rect4[1], &rect4[2],
						 &rect4[3]);
}

/* ------------------------------------------------------------------------------------------- */
/* Projection: projection.cu:36-111 (forward), 114-197 (backward); constants projection.py:3-5. */
/* ------------------------------------------------------------------------------------------- */

typedef struct {
	float fx, fy, cx, cy;
	int width, height;
	float near_plane, low_pass, fov_scale;
} orc_camera;

typedef struct {
	float R[3][3], t[3], p[3];
	float z, z_inv, jx, jy;
	int clamped_x, clamped_y, behind;
	float jw[2][3], M[3][3], T[2][3];
	float a, b, c, det;
} orc_projected;

/* Rotation of a unit quaternion (w, x, y, z): projection.cu:15-20, projection.py:8-22. */
static void orc_quat_to_rotmat(const float* q, float r[3][3]) {
	const float w = q[0], x = q[1], y = q[2], z = q[3];
	r[0][0] = 1 - 2 * (y * y + z * z);
	r[0][1] = 2 * (x * y - w * z);
	r[0][2] = 2 * (x * z + w * y);
	r[1][0] = 2 * (x * y + w * z);
	r[1][1] = 1 - 2 * (x * x + z * z);
	r[1][2] = 2 * (y * z - w * x);
	r[2][0] = 2 * (x * z - w * y);
	r[2][1] = 2 * (y * z + w * x);
	r[2][2] = 1 - 2 * (x * x + y * y);
}

/* EWA projection with the clamped Jacobian and the low-pass term: projection.cu:36-77. */
static void orc_project_one(const orc_camera* cam, const float* w2c, const float* mean,
							const float* scale, const float* quat, orc_projected* g) {
	for (int i = 0; i < 3; i++) {
		for (int j = 0; j < 3; j++) g->R[i][j] = w2c[i * 4 + j];
		g->t[i] = w2c[i * 4 + 3];
		g->p[i] = g->R[i][0] * mean[0] + g->R[i][1] * mean[1] + g->R[i][2] * mean[2] + g->t[i];
	}
	g->behind = g->p[2] <= cam->near_plane;
	g->z = fmaxf(g->p[2], cam->near_plane);
	g->z_inv = 1.0f / (g->z + 1e-6f);

	const float limit_x = cam->fov_scale * (0.5f * (float)cam->width / cam->fx);
	const float limit_y = cam->fov_scale * (0.5f * (float)cam->height / cam->fy);
	const float rx = g->p[0] * g->z_inv, ry = g->p[1] * g->z_inv;
	g->clamped_x = fabsf(rx) > limit_x;
	g->clamped_y = fabsf(ry) > limit_y;
	g->jx = fminf(fmaxf(rx, -limit_x), limit_x) * g->z;
	g->jy = fminf(fmaxf(ry, -limit_y), limit_y) * g->z;

	const float zz_inv = g->z_inv * g->z_inv;
	for (int j = 0; j < 3; j++) {
		g->jw[0][j] = cam->fx * g->z_inv * g->R[0][j] - cam->fx * g->jx * zz_inv * g->R[2][j];
		g->jw[1][j] = cam->fy * g->z_inv * g->R[1][j] - cam->fy * g->jy * zz_inv * g->R[2][j];
	}
	float rot[3][3];
	orc_quat_to_rotmat(quat, rot);
	for (int j = 0; j < 3; j++)
		for (int k = 0; k < 3; k++) g->M[j][k] = rot[j][k] * scale[k];
	for (int r = 0; r < 2; r++)
		for (int k = 0; k < 3; k++)
			g->T[r][k] = g->jw[r][0] * g->M[0][k] + g->jw[r][1] * g->M[1][k] + g->jw[r][2] * g->M[2][k];
	g->a = g->T[0][0] * g->T[0][0] + g->T[0][1] * g->T[0][1] + g->T[0][2] * g->T[0][2] + cam->low_pass;
	g->b = g->T[0][0] * g->T[1][0] + g->T[0][1] * g->T[1][1] + g->T[0][2] * g->T[1][2];
	g->c = g->T[1][0] * g->T[1][0] + g->T[1][1] * g->T[1][1] + g->T[1][2] * g->T[1][2] + cam->low_pass;
	g->det = g->a * g->c - g->b * g->b;
}

/* project_forward: projection.cu:80-111. */
ORC_EXPORT void orc_project_forward(int64_t n, const float* means, const float* scales,
									const float* quats, const float* opacities, const float* w2c,
									float fx, float fy, float cx, float cy, int width, int height,
									float near_plane, float low_pass, float fov_scale,
									float* means2D, float* depths, float* radii, float* conics) {
	const orc_camera cam = {fx, fy, cx, cy, width, height, near_plane, low_pass, fov_scale};
	const int tiles_x = (width + HDS_TILE - 1) / HDS_TILE;
	const int tiles_y = (height + HDS_TILE - 1) / HDS_TILE;
#pragma omp parallel for schedule(static)
	for (int64_t i = 0; i < n; i++) {
		orc_projected g;
		orc_project_one(&cam, w2c, means + i * 3, scales + i * 3, quats + i * 4, &g);
		const float u = cam.fx * g.p[0] / g.z + cam.cx;
		const float v = cam.fy * g.p[1] / g.z + cam.cy;
		means2D[i * 2 + 0] = u;
		means2D[i * 2 + 1] = v;
		depths[i] = g.p[2];
		const float scale_inv = g.det > 0.0f ? 1.0f / g.det : 1.0f;
		const float a_conic = g.c * scale_inv;
		const float b_conic = -g.b * scale_inv;
		const float c_conic = g.a * scale_inv;
		conics[i * 3 + 0] = a_conic;
		conics[i * 3 + 1] = b_conic;
		conics[i * 3 + 2] = c_conic;
		const float trace = g.a + g.c;
		const float radius = 3.0f * sqrtf(0.5f * (trace + sqrtf(fmaxf(trace * trace - 4.0f * g.det, 0.0f))));
		int x0, y0, w, h;
		const int visible = !g.behind && g.det > 0.0f &&
							hds_tile_rect(u, v, a_conic, b_conic, c_conic, opacities[i], tiles_x,
										  tiles_y, &x0, &y0, &w, &h);
		radii[i] = visible ? radius : 0.0f;
	}
}

/* project_backward: projection.cu:114-197. */
ORC_EXPORT void orc_project_backward(int64_t n, const float* grad_means2D, const float* grad_conics,
									 const float* means, const float* scales, const float* quats,
									 const float* w2c, float fx, float fy, float cx, float cy,
									 int width, int height, float near_plane, float low_pass,
									 float fov_scale, float* grad_means, float* grad_scales,
									 float* grad_quats) {
	const orc_camera cam = {fx, fy, cx, cy, width, height, near_plane, low_pass, fov_scale};
#pragma omp parallel for schedule(static)
	for (int64_t i = 0; i < n; i++) {
		const float* scale = scales + i * 3;
		const float* quat = quats + i * 4;
		orc_projected g;
		orc_project_one(&cam, w2c, means + i * 3, scale, quat, &g);

		const float g0 = grad_conics[i * 3 + 0], g1 = grad_conics[i * 3 + 1], g2 = grad_conics[i * 3 + 2];
		float da, db, dc;
		if (g.det > 0.0f) {
			/* conic = (c, -b, a) / det, differentiated through det = a c - b^2. */
			const float inv = 1.0f / g.det, inv2 = inv * inv;
			da = inv2 * (-g0 * g.c * g.c + g1 * g.b * g.c - g2 * g.b * g.b);
			db = inv2 * (2.0f * g0 * g.b * g.c + 2.0f * g2 * g.a * g.b) - g1 * (inv + 2.0f * g.b * g.b * inv2);
			dc = inv2 * (-g0 * g.b * g.b + g1 * g.a * g.b - g2 * g.a * g.a);
		} else {
			da = g2;
			db = -g1;
			dc = g0;
		}
		float dT[2][3];
		for (int k = 0; k < 3; k++) {
			dT[0][k] = 2.0f * da * g.T[0][k] + db * g.T[1][k];
			dT[1][k] = 2.0f * dc * g.T[1][k] + db * g.T[0][k];
		}
		float rot[3][3];
		orc_quat_to_rotmat(quat, rot);
		float djw[2][3], drot[3][3], dscale[3] = {0.0f, 0.0f, 0.0f};
		for (int j = 0; j < 3; j++) {
			djw[0][j] = dT[0][0] * g.M[j][0] + dT[0][1] * g.M[j][1] + dT[0][2] * g.M[j][2];
			djw[1][j] = dT[1][0] * g.M[j][0] + dT[1][1] * g.M[j][1] + dT[1][2] * g.M[j][2];
			for (int k = 0; k < 3; k++) {
				const float dM = g.jw[0][j] * dT[0][k] + g.jw[1][j] * dT[1][k];
				dscale[k] += dM * rot[j][k];
				drot[j][k] = dM * scale[k];
			}
		}
		const float w = quat[0], x = quat[1], y = quat[2], z = quat[3];
		grad_quats[i * 4 + 0] = 2.0f * (-drot[0][1] * z + drot[0][2] * y + drot[1][0] * z - drot[1][2] * x -
										drot[2][0] * y + drot[2][1] * x);
		grad_quats[i * 4 + 1] = 2.0f * (drot[0][1] * y + drot[0][2] * z + drot[1][0] * y - 2.0f * drot[1][1] * x -
										drot[1][2] * w + drot[2][0] * z + drot[2][1] * w - 2.0f * drot[2][2] * x);
		grad_quats[i * 4 + 2] = 2.0f * (-2.0f * drot[0][0] * y + drot[0][1] * x + drot[0][2] * w + drot[1][0] * x +
										drot[1][2] * z - drot[2][0] * w + drot[2][1] * z - 2.0f * drot[2][2] * y);
		grad_quats[i * 4 + 3] = 2.0f * (-2.0f * drot[0][0] * z - drot[0][1] * w + drot[0][2] * x + drot[1][0] * w -
										2.0f * drot[1][1] * z + drot[1][2] * y + drot[2][0] * x + drot[2][1] * y);
		for (int k = 0; k < 3; k++) grad_scales[i * 3 + k] = dscale[k];

		const float zz_inv = g.z_inv * g.z_inv;
		float dz_inv = 0.0f, djx = 0.0f, djy = 0.0f;
		for (int j = 0; j < 3; j++) {
			dz_inv += djw[0][j] * (cam.fx * g.R[0][j] - 2.0f * cam.fx * g.jx * g.z_inv * g.R[2][j]);
			dz_inv += djw[1][j] * (cam.fy * g.R[1][j] - 2.0f * cam.fy * g.jy * g.z_inv * g.R[2][j]);
			djx += djw[0][j] * (-cam.fx * zz_inv * g.R[2][j]);
			djy += djw[1][j] * (-cam.fy * zz_inv * g.R[2][j]);
		}
		float dp[3] = {0.0f, 0.0f, 0.0f};
		float dz = 0.0f;
		/* jx = clamp(p.x / z) * z: the ratio only carries gradient inside the clamp. */
		const float rx = g.jx / g.z, ry = g.jy / g.z;
		dz += djx * rx + djy * ry;
		if (!g.clamped_x) {
			dp[0] += djx * g.z * g.z_inv;
			dz_inv += djx * g.z * g.p[0];
		}
		if (!g.clamped_y) {
			dp[1] += djy * g.z * g.z_inv;
			dz_inv += djy * g.z * g.p[1];
		}
		const float gu = grad_means2D[i * 2 + 0], gv = grad_means2D[i * 2 + 1];
		dp[0] += gu * cam.fx / g.z;
		dp[1] += gv * cam.fy / g.z;
		dz += -(gu * cam.fx * g.p[0] + gv * cam.fy * g.p[1]) / (g.z * g.z);
		dz += dz_inv * (-zz_inv);
		if (!g.behind) dp[2] += dz;
		for (int k = 0; k < 3; k++)
			grad_means[i * 3 + k] = g.R[0][k] * dp[0] + g.R[1][k] * dp[1] + g.R[2][k] * dp[2];
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

/*
 * Emits every (tile, gaussian) pair, sorts by (tile, float bits of depth) keeping index order on
 * ties, and builds [start, end) per tile, zero for untouched tiles. Outputs values_sorted[P] and
 * tile_ranges[T][2] exactly as the reference rasterize returns them (forward.cu:434).
 */
ORC_EXPORT void orc_bin_fill(int64_t n, const float* depths, const int32_t* counts,
							 const int32_t* rects, int width, int height, int64_t num_pairs,
							 int32_t* values_sorted, int32_t* tile_ranges) {
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
	const float m = dx * (conic[0] * dx + conic[1] * dy) + dy * (conic[1] * dx + conic[2] * dy);
	const float G = expf(-0.5f * m);
	*gauss = G;
	*dx_out = dx;
	*dy_out = dy;
	return opacity * G;
}

/*
 * RGB (when colors != NULL) and C feature channels (when features != NULL), front to back per
 * pixel over its tile's sorted list. Pixel centres are at +0.5. A gaussian with alpha < 1/255 is
 * skipped but still counted in the list index; one that would leave T < 1e-4 ends the pixel
 * without blending. n_contrib is the 1-based list index of the last blended gaussian.
 */
ORC_EXPORT void orc_render_forward(int width, int height, const int32_t* tile_ranges,
								   const int32_t* values_sorted, const float* means2D,
								   const float* conics, const float* opacities, const float* colors,
								   const float* background, const float* features, int channels,
								   float* image, float* final_T, int32_t* n_contrib,
								   float* feature_image) {
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
					int last = 0;
					for (int c = 0; c < channels; c++) acc[c] = 0.0f;
					for (int j = start; j < end; j++) {
						const int gid = values_sorted[j];
						float G, dx, dy;
						const float raw = orc_alpha(px, py, means2D + gid * 2, conics + gid * 3,
													opacities[gid], &G, &dx, &dy);
						const float alpha = fminf(HDS_MAX_ALPHA, raw);
						if (alpha < HDS_MIN_ALPHA) continue;
						const float test_T = T * (1.0f - alpha);
						if (test_T < HDS_MIN_TRANSMITTANCE) break;
						const float w = alpha * T;
						if (colors) {
							r += w * colors[gid * 3 + 0];
							g += w * colors[gid * 3 + 1];
							b += w * colors[gid * 3 + 2];
						}
						const float* f = features ? features + (int64_t)gid * channels : NULL;
						for (int c = 0; c < channels && f; c++) acc[c] += w * f[c];
						T = test_T;
						last = j - start + 1;
					}
					const int64_t pix = (int64_t)y * width + x;
					if (image) {
						image[pix * 3 + 0] = r + T * background[0];
						image[pix * 3 + 1] = g + T * background[1];
						image[pix * 3 + 2] = b + T * background[2];
					}
					if (final_T) final_T[pix] = T;
					if (n_contrib) n_contrib[pix] = last;
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
