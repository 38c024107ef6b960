/*
 * EWA projection of one 3D gaussian to a screen-space conic, forward and backward, as scalar code
 * shared by the HIP projection kernels and the CPU oracle (compiled on both sides with
 * -ffp-contract=off and only correctly rounded operations, so both give the same bits).
 *
 * The function is the reference's project_gaussians (gaussian_splatting/rasterizer/projection.cu:
 * 36-111 forward, 114-197 backward; constants projection.py:3-5): camera-space centre p = R m + t,
 * near clamp z = max(p_z, near) with zeta = 1 / (z + 1e-6), the perspective Jacobian whose x / z and
 * y / z are clamped to fov_scale times the half field of view, 2D covariance J R M M^T R^T J^T plus
 * a low-pass of 0.3 px^2, pixel centre (fx p_x / z + cx, fy p_y / z + cy), conic = inverse
 * covariance, radius = 3 sqrt(largest eigenvalue), visible when in front of the near plane, with a
 * positive determinant and a non-empty tile rectangle.
 *
 * It is organised around the gaussian's principal axes. Axis k of the 3D gaussian is s_k r_k (r_k
 * the k-th column of the rotation of q); in camera space it is a_k = R s_k r_k, and the perspective
 * maps it to the screen vector e_k = J a_k = (fx zeta (a_kx - rho_x a_kz), fy zeta (a_ky - rho_y a_kz)),
 * rho = j zeta being the (clamped) slope of the line of sight. The 2D covariance is the sum of the
 * three screen axes' outer products, sum_k e_k e_k^T + low_pass I. The backward walks the same
 * chain: the conic's gradient to the covariance's as the 2x2 matrix identity dL/dSigma = -Q G Q
 * (Q = Sigma^-1, G the conic gradient as a symmetric matrix), then to each screen axis
 * (dL/de_k = 2 (dL/dSigma) e_k), camera axis, world axis, scale and rotation column, and the
 * rotation columns' gradient to the quaternion in vector form (see hds_ewa_backward).
 */
#ifndef HDS_EWA_H
#define HDS_EWA_H

#include "hds_common.h"

typedef struct {
	float fx, fy, cx, cy;
	int width, height;
	float near_plane, low_pass, fov_scale;
} hds_camera;

/* Forward state of one gaussian, everything the backward reuses. */
typedef struct {
	float p[3];             /* camera-space centre */
	float z, zeta;          /* near-clamped depth and 1 / (z + 1e-6) */
	float tx, ty;           /* line-of-sight slopes p_x zeta, p_y zeta clamped to the field of view */
	float rho_x, rho_y;     /* tx z zeta, ty z zeta: the slopes the Jacobian uses */
	int clamped_x, clamped_y, behind;
	float r[3][3];          /* r[k]: column k of the rotation of q */
	float axis[3][3];       /* axis[k] = R s_k r[k]: principal axis k in camera space */
	float screen[3][2];     /* screen[k] = J axis[k] */
	float a, b, c, det;     /* 2D covariance (a b; b c) with the low-pass, and its determinant */
} hds_ewa;

/* Columns of the rotation of the unit quaternion q = (w, x, y, z): r[k] is where the k-th basis
 * vector goes (the matrix of projection.py:8-22, read by columns). */
HDS_HD void hds_quat_columns(const float q[4], float r[3][3]) {
	const float w = q[0], x = q[1], y = q[2], z = q[3];
	r[0][0] = 1.0f - 2.0f * (y * y + z * z);
	r[0][1] = 2.0f * (x * y + w * z);
	r[0][2] = 2.0f * (x * z - w * y);
	r[1][0] = 2.0f * (x * y - w * z);
	r[1][1] = 1.0f - 2.0f * (x * x + z * z);
	r[1][2] = 2.0f * (y * z + w * x);
	r[2][0] = 2.0f * (x * z + w * y);
	r[2][1] = 2.0f * (y * z - w * x);
	r[2][2] = 1.0f - 2.0f * (x * x + y * y);
}

/* Forward state of the gaussian (m, s, q) seen by a camera with row-major world_to_camera w2c. */
HDS_HD void hds_ewa_project(const hds_camera* cam, const float w2c[16], const float m[3], const float s[3],
							const float q[4], hds_ewa* g) {
	for (int i = 0; i < 3; i++) g->p[i] = w2c[4 * i] * m[0] + w2c[4 * i + 1] * m[1] + w2c[4 * i + 2] * m[2] + w2c[4 * i + 3];
	g->behind = g->p[2] <= cam->near_plane;
	g->z = fmaxf(g->p[2], cam->near_plane);
	g->zeta = 1.0f / (g->z + 1e-6f);
	const float lim_x = cam->fov_scale * (0.5f * (float)cam->width / cam->fx);
	const float lim_y = cam->fov_scale * (0.5f * (float)cam->height / cam->fy);
	const float sx = g->p[0] * g->zeta, sy = g->p[1] * g->zeta;
	g->clamped_x = fabsf(sx) > lim_x;
	g->clamped_y = fabsf(sy) > lim_y;
	g->tx = fminf(fmaxf(sx, -lim_x), lim_x);
	g->ty = fminf(fmaxf(sy, -lim_y), lim_y);
	g->rho_x = g->tx * g->z * g->zeta;
	g->rho_y = g->ty * g->z * g->zeta;
	hds_quat_columns(q, g->r);
	const float kx = cam->fx * g->zeta, ky = cam->fy * g->zeta;
	float a = cam->low_pass, b = 0.0f, c = cam->low_pass;
	for (int k = 0; k < 3; k++) {
		const float wx = s[k] * g->r[k][0], wy = s[k] * g->r[k][1], wz = s[k] * g->r[k][2];
		for (int i = 0; i < 3; i++) g->axis[k][i] = w2c[4 * i] * wx + w2c[4 * i + 1] * wy + w2c[4 * i + 2] * wz;
		const float ex = kx * (g->axis[k][0] - g->rho_x * g->axis[k][2]);
		const float ey = ky * (g->axis[k][1] - g->rho_y * g->axis[k][2]);
		g->screen[k][0] = ex;
		g->screen[k][1] = ey;
		a += ex * ex;
		b += ex * ey;
		c += ey * ey;
	}
	g->a = a;
	g->b = b;
	g->c = c;
	g->det = a * c - b * b;
}

/* Screen-space outputs: pixel centre, depth, conic (c, -b, a) / det (unnormalised when det <= 0,
 * as the reference leaves it), radius 3 sqrt(lambda_max) and the visibility of
 * projection.cu:106-110. lambda_max = (a + c) / 2 + sqrt(((a - c) / 2)^2 + b^2) has no cancellation
 * under the root. Returns 1 when the gaussian is visible (radius > 0). */
HDS_HD int hds_ewa_screen(const hds_camera* cam, const hds_ewa* g, float opacity, float mean2d[2], float* depth,
						  float conic[3], float* radius) {
	mean2d[0] = cam->fx * g->p[0] / g->z + cam->cx;
	mean2d[1] = cam->fy * g->p[1] / g->z + cam->cy;
	*depth = g->p[2];
	const float inv = g->det > 0.0f ? 1.0f / g->det : 1.0f;
	conic[0] = g->c * inv;
	conic[1] = -g->b * inv;
	conic[2] = g->a * inv;
	const float half_gap = 0.5f * (g->a - g->c);
	const float lambda_max = 0.5f * (g->a + g->c) + sqrtf(half_gap * half_gap + g->b * g->b);
	const int tiles_x = (cam->width + HDS_TILE - 1) / HDS_TILE, tiles_y = (cam->height + HDS_TILE - 1) / HDS_TILE;
	int x0, y0, w, h;
	const int visible = !g->behind && g->det > 0.0f &&
						hds_tile_rect(mean2d[0], mean2d[1], conic[0], conic[1], conic[2], opacity, tiles_x, tiles_y, &x0,
									  &y0, &w, &h);
	*radius = visible ? 3.0f * sqrtf(lambda_max) : 0.0f;
	return visible;
}

/*
 * Gradients of the mean, scale and quaternion from those of the pixel centre (dmean2d) and the
 * conic (dconic), for the state g that hds_ewa_project computed from (m, s, q). Depth and radius
 * carry no gradient (projection.py:65, 71-72 of the reference).
 *
 * Steps, each the transpose of a forward step:
 *   conic -> covariance: with Q the conic as a matrix and G = (g0, g1/2; g1/2, g2) its gradient,
 *     dL/dSigma = -Q G Q; a and c take its diagonal, b (one entry filling both off-diagonal slots)
 *     twice its off-diagonal. An unnormalised conic (det <= 0) is a plain permutation.
 *   covariance -> screen axes: dL/de_k = (2 da e_kx + db e_ky, 2 dc e_ky + db e_kx).
 *   screen axes -> camera axes, zeta and the slopes rho (e = k (a_xy - rho a_z), k = f zeta).
 *   camera axes -> world axes (R^T), scales (s_k: the world axis along r_k) and rotation columns.
 *   rotation columns -> quaternion: with D the gradient of the rotation matrix (D[k] = dL/dr_k),
 *     v = its axial part (D - D^T)^v and S = D + D^T, dL/dw = 2 q_v . v and
 *     dL/dq_v = 2 (w v + S q_v - 2 tr(D) q_v).
 *   slopes -> line of sight: rho = t z zeta with t = clamp(p zeta); t only passes gradient inside
 *     the clamp.
 *   pixel centre and zeta -> depth and camera-space centre, which takes no depth gradient when the
 *     near clamp is active; then dL/dm = R^T dL/dp.
 */
HDS_HD void hds_ewa_backward(const hds_camera* cam, const float w2c[16], const float s[3], const float q[4],
							 const hds_ewa* g, const float dmean2d[2], const float dconic[3], float dm[3], float ds[3],
							 float dq[4]) {
	float da, db, dc;
	if (g->det > 0.0f) {
		const float inv = 1.0f / g->det;
		const float qa = g->c * inv, qb = -g->b * inv, qc = g->a * inv;
		const float h = 0.5f * dconic[1];
		/* (QG) rows, then the needed entries of (QG)Q */
		const float m00 = qa * dconic[0] + qb * h, m01 = qa * h + qb * dconic[2];
		const float m10 = qb * dconic[0] + qc * h, m11 = qb * h + qc * dconic[2];
		da = -(m00 * qa + m01 * qb);
		db = -2.0f * (m00 * qb + m01 * qc);
		dc = -(m10 * qb + m11 * qc);
	} else {
		da = dconic[2];
		db = -dconic[1];
		dc = dconic[0];
	}

	const float kx = cam->fx * g->zeta, ky = cam->fy * g->zeta;
	float dzeta = 0.0f, drho_x = 0.0f, drho_y = 0.0f;
	float D[3][3];
	for (int k = 0; k < 3; k++) {
		const float ex = g->screen[k][0], ey = g->screen[k][1];
		const float gx = 2.0f * da * ex + db * ey;
		const float gy = 2.0f * dc * ey + db * ex;
		const float ux = g->axis[k][0] - g->rho_x * g->axis[k][2];
		const float uy = g->axis[k][1] - g->rho_y * g->axis[k][2];
		dzeta += gx * cam->fx * ux + gy * cam->fy * uy;
		const float dax = kx * gx, day = ky * gy;
		const float daz = -(g->rho_x * dax + g->rho_y * day);
		drho_x -= dax * g->axis[k][2];
		drho_y -= day * g->axis[k][2];
		float wsum = 0.0f;
		for (int i = 0; i < 3; i++) {
			const float dw = w2c[i] * dax + w2c[4 + i] * day + w2c[8 + i] * daz; /* (R^T da)_i */
			wsum += g->r[k][i] * dw;
			D[k][i] = s[k] * dw;
		}
		ds[k] = wsum;
	}

	const float w = q[0], qv[3] = {q[1], q[2], q[3]};
	const float v[3] = {D[1][2] - D[2][1], D[2][0] - D[0][2], D[0][1] - D[1][0]};
	const float tr = D[0][0] + D[1][1] + D[2][2];
	dq[0] = 2.0f * (qv[0] * v[0] + qv[1] * v[1] + qv[2] * v[2]);
	for (int i = 0; i < 3; i++) {
		float sq = 0.0f;
		for (int j = 0; j < 3; j++) sq += (D[i][j] + D[j][i]) * qv[j];
		dq[1 + i] = 2.0f * (w * v[i] + sq - 2.0f * tr * qv[i]);
	}

	/* rho = t z zeta */
	float dp[3] = {0.0f, 0.0f, 0.0f};
	float dz = drho_x * g->tx * g->zeta + drho_y * g->ty * g->zeta;
	dzeta += drho_x * g->tx * g->z + drho_y * g->ty * g->z;
	const float dtx = drho_x * g->z * g->zeta, dty = drho_y * g->z * g->zeta;
	if (!g->clamped_x) {
		dp[0] += dtx * g->zeta;
		dzeta += dtx * g->p[0];
	}
	if (!g->clamped_y) {
		dp[1] += dty * g->zeta;
		dzeta += dty * g->p[1];
	}
	/* pixel centre (fx p_x / z + cx, fy p_y / z + cy) */
	dp[0] += dmean2d[0] * cam->fx / g->z;
	dp[1] += dmean2d[1] * cam->fy / g->z;
	dz -= (dmean2d[0] * cam->fx * g->p[0] + dmean2d[1] * cam->fy * g->p[1]) / (g->z * g->z);
	/* zeta = 1 / (z + 1e-6), z = max(p_z, near) */
	dz -= dzeta * g->zeta * g->zeta;
	if (!g->behind) dp[2] += dz;
	for (int i = 0; i < 3; i++) dm[i] = w2c[i] * dp[0] + w2c[4 + i] * dp[1] + w2c[8 + i] * dp[2];
}

#endif /* HDS_EWA_H */
