// EWA projection of 3D gaussians to screen-space conics, forward and backward.
//
// One thread per gaussian; both kernels are a single streaming pass (44 B read / 28 B written per
// gaussian forward, ~100 B backward), so they are HBM-bound and need nothing beyond coalesced
// per-gaussian loads. The arithmetic follows project(), project_forward and project_backward
// (projection.cu:36-197) operation for operation, compiled without contraction, so means2D,
// depths, conics and the radii > 0 visibility bit equal the CPU oracle's bit for bit.
#include "hds_internal.h"
#include "hds_rasterizer.h"

namespace {

struct Camera {
	float fx, fy, cx, cy;
	int width, height;
	float near_plane, low_pass, fov_scale;
};

struct Projected {
	float R[3][3], t[3], p[3];
	float z, z_inv, jx, jy;
	bool clamped_x, clamped_y, behind;
	float jw[2][3], M[3][3], T[2][3];
	float a, b, c, det;
};

// Rotation of a unit quaternion (w, x, y, z): projection.py:8-22.
__device__ inline void quat_to_rotmat(float w, float x, float y, float z, float r[3][3]) {
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

// World -> camera, near clamp, Jacobian with its x/z, y/z clamped to 1.3x the half field of view,
// T = J W R S and the 2D covariance T T^T + 0.3 I (projection.cu:36-77).
__device__ inline void project_one(const Camera& cam, const float* w2c, const float* mean, const float* scale,
								   const float* quat, Projected& g) {
	for (int i = 0; i < 3; i++) {
		for (int j = 0; j < 3; j++) g.R[i][j] = w2c[i * 4 + j];
		g.t[i] = w2c[i * 4 + 3];
		g.p[i] = g.R[i][0] * mean[0] + g.R[i][1] * mean[1] + g.R[i][2] * mean[2] + g.t[i];
	}
	g.behind = g.p[2] <= cam.near_plane;
	g.z = fmaxf(g.p[2], cam.near_plane);
	g.z_inv = 1.0f / (g.z + 1e-6f);

	const float limit_x = cam.fov_scale * (0.5f * (float)cam.width / cam.fx);
	const float limit_y = cam.fov_scale * (0.5f * (float)cam.height / cam.fy);
	const float rx = g.p[0] * g.z_inv, ry = g.p[1] * g.z_inv;
	g.clamped_x = fabsf(rx) > limit_x;
	g.clamped_y = fabsf(ry) > limit_y;
	g.jx = fminf(fmaxf(rx, -limit_x), limit_x) * g.z;
	g.jy = fminf(fmaxf(ry, -limit_y), limit_y) * g.z;

	const float zz_inv = g.z_inv * g.z_inv;
	for (int j = 0; j < 3; j++) {
		g.jw[0][j] = cam.fx * g.z_inv * g.R[0][j] - cam.fx * g.jx * zz_inv * g.R[2][j];
		g.jw[1][j] = cam.fy * g.z_inv * g.R[1][j] - cam.fy * g.jy * zz_inv * g.R[2][j];
	}
	float rot[3][3];
	quat_to_rotmat(quat[0], quat[1], quat[2], quat[3], rot);
	for (int j = 0; j < 3; j++)
		for (int k = 0; k < 3; k++) g.M[j][k] = rot[j][k] * scale[k];
	for (int r = 0; r < 2; r++)
		for (int k = 0; k < 3; k++)
			g.T[r][k] = g.jw[r][0] * g.M[0][k] + g.jw[r][1] * g.M[1][k] + g.jw[r][2] * g.M[2][k];
	g.a = g.T[0][0] * g.T[0][0] + g.T[0][1] * g.T[0][1] + g.T[0][2] * g.T[0][2] + cam.low_pass;
	g.b = g.T[0][0] * g.T[1][0] + g.T[0][1] * g.T[1][1] + g.T[0][2] * g.T[1][2];
	g.c = g.T[1][0] * g.T[1][0] + g.T[1][1] * g.T[1][1] + g.T[1][2] * g.T[1][2] + cam.low_pass;
	g.det = g.a * g.c - g.b * g.b;
}

__global__ __launch_bounds__(256) void project_forward_kernel(int64_t n, Camera cam, const float* __restrict__ w2c,
															  const float* __restrict__ means,
															  const float* __restrict__ scales,
															  const float* __restrict__ quats,
															  const float* __restrict__ opacities,
															  float* __restrict__ means2D, float* __restrict__ depths,
															  float* __restrict__ radii, float* __restrict__ conics) {
	const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
	if (i >= n) return;
	float mean[3] = {means[i * 3], means[i * 3 + 1], means[i * 3 + 2]};
	float scale[3] = {scales[i * 3], scales[i * 3 + 1], scales[i * 3 + 2]};
	float quat[4] = {quats[i * 4], quats[i * 4 + 1], quats[i * 4 + 2], quats[i * 4 + 3]};
	Projected g;
	project_one(cam, w2c, mean, scale, quat, g);

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
	const int tiles_x = (cam.width + HDS_TILE - 1) / HDS_TILE;
	const int tiles_y = (cam.height + HDS_TILE - 1) / HDS_TILE;
	int x0, y0, w, h;
	const bool visible = !g.behind && g.det > 0.0f &&
						 hds_tile_rect(u, v, a_conic, b_conic, c_conic, opacities[i], tiles_x, tiles_y, &x0, &y0, &w, &h);
	radii[i] = visible ? radius : 0.0f;
}

__global__ __launch_bounds__(256) void project_backward_kernel(
	int64_t n, Camera cam, const float* __restrict__ w2c, const float* __restrict__ means,
	const float* __restrict__ scales, const float* __restrict__ quats, const float* __restrict__ grad_means2D,
	const float* __restrict__ grad_conics, float* __restrict__ grad_means, float* __restrict__ grad_scales,
	float* __restrict__ grad_quats) {
	const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
	if (i >= n) return;
	float mean[3] = {means[i * 3], means[i * 3 + 1], means[i * 3 + 2]};
	float scale[3] = {scales[i * 3], scales[i * 3 + 1], scales[i * 3 + 2]};
	float quat[4] = {quats[i * 4], quats[i * 4 + 1], quats[i * 4 + 2], quats[i * 4 + 3]};
	Projected g;
	project_one(cam, w2c, mean, scale, quat, g);

	// conic = (c, -b, a) / det differentiated through det = a c - b^2 (projection.cu:127-136).
	const float g0 = grad_conics[i * 3 + 0], g1 = grad_conics[i * 3 + 1], g2 = grad_conics[i * 3 + 2];
	float da, db, dc;
	if (g.det > 0.0f) {
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
	quat_to_rotmat(quat[0], quat[1], quat[2], quat[3], rot);
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
	// d(rotation)/d(quaternion) of quat_to_rotmat (projection.cu:157-165).
	const float w = quat[0], x = quat[1], y = quat[2], z = quat[3];
	float dq[4];
	dq[0] = 2.0f * (-drot[0][1] * z + drot[0][2] * y + drot[1][0] * z - drot[1][2] * x - drot[2][0] * y + drot[2][1] * x);
	dq[1] = 2.0f * (drot[0][1] * y + drot[0][2] * z + drot[1][0] * y - 2.0f * drot[1][1] * x - drot[1][2] * w +
				   drot[2][0] * z + drot[2][1] * w - 2.0f * drot[2][2] * x);
	dq[2] = 2.0f * (-2.0f * drot[0][0] * y + drot[0][1] * x + drot[0][2] * w + drot[1][0] * x + drot[1][2] * z -
				   drot[2][0] * w + drot[2][1] * z - 2.0f * drot[2][2] * y);
	dq[3] = 2.0f * (-2.0f * drot[0][0] * z - drot[0][1] * w + drot[0][2] * x + drot[1][0] * w - 2.0f * drot[1][1] * z +
				   drot[1][2] * y + drot[2][0] * x + drot[2][1] * y);
	for (int k = 0; k < 4; k++) grad_quats[i * 4 + k] = dq[k];
	for (int k = 0; k < 3; k++) grad_scales[i * 3 + k] = dscale[k];

	// jw depends on z_inv, jx, jy; unwind them to the camera-space point (projection.cu:169-192).
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
	for (int k = 0; k < 3; k++) grad_means[i * 3 + k] = g.R[0][k] * dp[0] + g.R[1][k] * dp[1] + g.R[2][k] * dp[2];
}

Camera make_camera(float fx, float fy, float cx, float cy, int width, int height, float near_plane, float low_pass,
				   float fov_scale) {
	Camera cam;
	cam.fx = fx;
	cam.fy = fy;
	cam.cx = cx;
	cam.cy = cy;
	cam.width = width;
	cam.height = height;
	cam.near_plane = near_plane;
	cam.low_pass = low_pass;
	cam.fov_scale = fov_scale;
	return cam;
}

}  // namespace

extern "C" int hds_project_gaussians(int64_t n, const float* means, const float* scales, const float* quats,
									 const float* opacities, const float* world_to_camera, float fx, float fy,
									 float cx, float cy, int width, int height, float near_plane, float low_pass,
									 float fov_scale, float* means2D, float* depths, float* radii, float* conics,
									 hds_stream_t stream) {
	HDS_REQUIRE(n >= 0, "project_gaussians: negative gaussian count %lld", (long long)n);
	HDS_REQUIRE(width > 0 && height > 0, "project_gaussians: image size %dx%d must be positive", width, height);
	if (n == 0) return HDS_OK;
	HDS_REQUIRE(means && scales && quats && opacities && world_to_camera && means2D && depths && radii && conics,
				"project_gaussians: null pointer argument");
	hipStream_t s = (hipStream_t)stream;
	const Camera cam = make_camera(fx, fy, cx, cy, width, height, near_plane, low_pass, fov_scale);
	HdsKernelTimer timer1("project_forward_kernel", s);
	project_forward_kernel<<<hds_blocks(n, 256), 256, 0, s>>>(n, cam, world_to_camera, means, scales, quats,
															  opacities, means2D, depths, radii, conics);
	timer1.stop();
	HDS_LAUNCH_CHECK("project_forward", s);
	return HDS_OK;
}

extern "C" int hds_project_gaussians_backward(int64_t n, const float* grad_means2D, const float* grad_conics,
											  const float* means, const float* scales, const float* quats,
											  const float* world_to_camera, float fx, float fy, float cx, float cy,
											  int width, int height, float near_plane, float low_pass,
											  float fov_scale, float* grad_means, float* grad_scales,
											  float* grad_quats, hds_stream_t stream) {
	HDS_REQUIRE(n >= 0, "project_gaussians_backward: negative gaussian count %lld", (long long)n);
	if (n == 0) return HDS_OK;
	HDS_REQUIRE(grad_means2D && grad_conics && means && scales && quats && world_to_camera && grad_means &&
					grad_scales && grad_quats,
				"project_gaussians_backward: null pointer argument");
	hipStream_t s = (hipStream_t)stream;
	const Camera cam = make_camera(fx, fy, cx, cy, width, height, near_plane, low_pass, fov_scale);
	HdsKernelTimer timer2("project_backward_kernel", s);
	project_backward_kernel<<<hds_blocks(n, 256), 256, 0, s>>>(n, cam, world_to_camera, means, scales, quats,
															   grad_means2D, grad_conics, grad_means, grad_scales,
															   grad_quats);
	timer2.stop();
	HDS_LAUNCH_CHECK("project_backward", s);
	return HDS_OK;
}
