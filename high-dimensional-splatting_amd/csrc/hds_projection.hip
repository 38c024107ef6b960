// EWA projection of 3D gaussians to screen-space conics, forward and backward (hds_ewa.h).
//
// One thread per gaussian, a single streaming pass each way: 44 B read and 28 B written per
// gaussian forward, 60 B read and 40 B written backward, all of it coalesced across the wave
// (quaternions as one 16-byte load, the camera pose as wave-uniform scalar loads). Nothing is
// reused between gaussians, so there is nothing to stage through LDS: the kernels are bound by HBM
// and by the latency of their few loads, and 256-thread blocks over N / 256 work-groups give every
// CU several waves in flight. The per-gaussian arithmetic is hds_ewa.h, which the CPU oracle
// compiles too, so means2D, depths, radii, conics and all three gradients equal the oracle's bit
// for bit.
#include "hds_internal.h"
#include "hds_ewa.h"
#include "hds_rasterizer.h"

namespace {

struct GaussianIn {
	float m[3], s[3], q[4];
};

__device__ inline GaussianIn load_gaussian(int64_t i, const float* __restrict__ means, const float* __restrict__ scales,
										   const float* __restrict__ quats, bool quats16) {
	GaussianIn g;
#pragma unroll
	for (int k = 0; k < 3; k++) {
		g.m[k] = means[i * 3 + k];
		g.s[k] = scales[i * 3 + k];
	}
	if (quats16) {
		const float4 q = reinterpret_cast<const float4*>(quats)[i];
		g.q[0] = q.x;
		g.q[1] = q.y;
		g.q[2] = q.z;
		g.q[3] = q.w;
	} else {
#pragma unroll
		for (int k = 0; k < 4; k++) g.q[k] = quats[i * 4 + k];
	}
	return g;
}

// The three rows of the world-to-camera transform (the fourth is never read).
__device__ inline void load_pose(const float* __restrict__ w2c, float pose[16]) {
#pragma unroll
	for (int k = 0; k < 12; k++) pose[k] = w2c[k];
#pragma unroll
	for (int k = 12; k < 16; k++) pose[k] = 0.0f;
}

__global__ __launch_bounds__(256) void project_forward_kernel(int64_t n, hds_camera cam, const float* __restrict__ w2c,
															  const float* __restrict__ means,
															  const float* __restrict__ scales,
															  const float* __restrict__ quats, bool quats16,
															  const float* __restrict__ opacities,
															  float* __restrict__ means2D, float* __restrict__ depths,
															  float* __restrict__ radii, float* __restrict__ conics) {
	const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
	if (i >= n) return;
	float pose[16];
	load_pose(w2c, pose);
	const GaussianIn in = load_gaussian(i, means, scales, quats, quats16);
	hds_ewa g;
	hds_ewa_project(&cam, pose, in.m, in.s, in.q, &g);
	float mean2d[2], conic[3], depth, radius;
	hds_ewa_screen(&cam, &g, opacities[i], mean2d, &depth, conic, &radius);
	means2D[i * 2 + 0] = mean2d[0];
	means2D[i * 2 + 1] = mean2d[1];
	depths[i] = depth;
	radii[i] = radius;
#pragma unroll
	for (int k = 0; k < 3; k++) conics[i * 3 + k] = conic[k];
}

__global__ __launch_bounds__(256) void project_backward_kernel(
	int64_t n, hds_camera cam, const float* __restrict__ w2c, const float* __restrict__ means,
	const float* __restrict__ scales, const float* __restrict__ quats, bool quats16,
	const float* __restrict__ grad_means2D, const float* __restrict__ grad_conics, float* __restrict__ grad_means,
	float* __restrict__ grad_scales, float* __restrict__ grad_quats) {
	const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
	if (i >= n) return;
	float pose[16];
	load_pose(w2c, pose);
	const GaussianIn in = load_gaussian(i, means, scales, quats, quats16);
	const float dmean2d[2] = {grad_means2D[i * 2], grad_means2D[i * 2 + 1]};
	const float dconic[3] = {grad_conics[i * 3], grad_conics[i * 3 + 1], grad_conics[i * 3 + 2]};
	hds_ewa g;
	hds_ewa_project(&cam, pose, in.m, in.s, in.q, &g);
	float dm[3], ds[3], dq[4];
	hds_ewa_backward(&cam, pose, in.s, in.q, &g, dmean2d, dconic, dm, ds, dq);
#pragma unroll
	for (int k = 0; k < 3; k++) {
		grad_means[i * 3 + k] = dm[k];
		grad_scales[i * 3 + k] = ds[k];
	}
	if (quats16) {
		reinterpret_cast<float4*>(grad_quats)[i] = make_float4(dq[0], dq[1], dq[2], dq[3]);
	} else {
#pragma unroll
		for (int k = 0; k < 4; k++) grad_quats[i * 4 + k] = dq[k];
	}
}

hds_camera make_camera(float fx, float fy, float cx, float cy, int width, int height, float near_plane, float low_pass,
					   float fov_scale) {
	hds_camera cam;
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

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

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
	const hds_camera cam = make_camera(fx, fy, cx, cy, width, height, near_plane, low_pass, fov_scale);
	HdsKernelTimer timer1("project_forward_kernel", s);
	project_forward_kernel<<<hds_blocks(n, 256), 256, 0, s>>>(n, cam, world_to_camera, means, scales, quats,
															  aligned16(quats), opacities, means2D, depths, radii,
															  conics);
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
	const hds_camera cam = make_camera(fx, fy, cx, cy, width, height, near_plane, low_pass, fov_scale);
	HdsKernelTimer timer2("project_backward_kernel", s);
	project_backward_kernel<<<hds_blocks(n, 256), 256, 0, s>>>(
		n, cam, world_to_camera, means, scales, quats, aligned16(quats) && aligned16(grad_quats), grad_means2D,
		grad_conics, grad_means, grad_scales, grad_quats);
	timer2.stop();
	HDS_LAUNCH_CHECK("project_backward", s);
	return HDS_OK;
}
