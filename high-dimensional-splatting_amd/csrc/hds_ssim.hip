// SSIM loss kernels: forward (map + the three per-pixel partials the backward needs) and backward.
//
// Zero-padded separable 11-tap Gaussian window, sigma 1.5, C1 = 0.01^2, C2 = 0.03^2, on
// interleaved [H, W, 3] images (ssim.cu:6-113, utils/loss.py:8-9, 39-54). Each work-group owns a
// 32 x 8 pixel tile (x 3 channels): the tile plus a 5-pixel halo is read once into LDS, blurred
// horizontally into LDS, then vertically, so one launch replaces the reference's two and the
// intermediate moments never touch HBM.
#include "hds_internal.h"
#include "hds_rasterizer.h"

namespace {

constexpr int kR = 5;                      // window radius
constexpr int kTx = 32, kTy = 8;           // output pixels per work-group
constexpr int kHx = kTx + 2 * kR, kHy = kTy + 2 * kR;
constexpr float kC1 = 0.01f * 0.01f, kC2 = 0.03f * 0.03f;

// Normalised 11-tap Gaussian, sigma 1.5, filled once from the host (double, then rounded).
__constant__ float kWin[2 * kR + 1];

// Forward: moments a, b, aa, bb, ab blurred -> ssim, d_mu, d_aa, d_ab (ssim.cu:39-72).
__global__ __launch_bounds__(256) void ssim_forward_kernel(int height, int width, const float* __restrict__ img_a,
														   const float* __restrict__ img_b, float* __restrict__ ssim_map,
														   float* __restrict__ d_mu, float* __restrict__ d_aa,
														   float* __restrict__ d_ab) {
	__shared__ float s_a[kHy][kHx * 3], s_b[kHy][kHx * 3];
	__shared__ float s_h[5][kHy][kTx * 3];
	const int x0 = blockIdx.x * kTx - kR, y0 = blockIdx.y * kTy - kR;
	for (int i = threadIdx.x; i < kHy * kHx * 3; i += blockDim.x) {
		const int row = i / (kHx * 3), e = i - row * (kHx * 3);
		const int x = x0 + e / 3, y = y0 + row;
		const bool in = x >= 0 && x < width && y >= 0 && y < height;
		const int64_t g = ((int64_t)y * width + x) * 3 + e % 3;
		s_a[row][e] = in ? img_a[g] : 0.0f;
		s_b[row][e] = in ? img_b[g] : 0.0f;
	}
	__syncthreads();
	// Horizontal pass over every halo row, for the tile's columns.
	for (int i = threadIdx.x; i < kHy * kTx * 3; i += blockDim.x) {
		const int row = i / (kTx * 3), e = i - row * (kTx * 3);
		const int x = x0 + kR + e / 3;
		float sa = 0.0f, sb = 0.0f, saa = 0.0f, sbb = 0.0f, sab = 0.0f;
#pragma unroll
		for (int k = -kR; k <= kR; k++) {
			if (x + k < 0 || x + k >= width) continue;
			const float w = kWin[k + kR];
			const float va = s_a[row][e + 3 * (kR + k)], vb = s_b[row][e + 3 * (kR + k)];
			sa += w * va;
			sb += w * vb;
			saa += w * va * va;
			sbb += w * vb * vb;
			sab += w * va * vb;
		}
		s_h[0][row][e] = sa;
		s_h[1][row][e] = sb;
		s_h[2][row][e] = saa;
		s_h[3][row][e] = sbb;
		s_h[4][row][e] = sab;
	}
	__syncthreads();
	for (int i = threadIdx.x; i < kTy * kTx * 3; i += blockDim.x) {
		const int row = i / (kTx * 3), e = i - row * (kTx * 3);
		const int x = x0 + kR + e / 3, y = y0 + kR + row;
		if (x >= width || y >= height) continue;
		float mu_a = 0.0f, mu_b = 0.0f, e_aa = 0.0f, e_bb = 0.0f, e_ab = 0.0f;
#pragma unroll
		for (int k = -kR; k <= kR; k++) {
			if (y + k < 0 || y + k >= height) continue;
			const float w = kWin[k + kR];
			const int r = row + kR + k;
			mu_a += w * s_h[0][r][e];
			mu_b += w * s_h[1][r][e];
			e_aa += w * s_h[2][r][e];
			e_bb += w * s_h[3][r][e];
			e_ab += w * s_h[4][r][e];
		}
		const float a1 = 2.0f * mu_a * mu_b + kC1;
		const float a2 = 2.0f * (e_ab - mu_a * mu_b) + kC2;
		const float b1 = mu_a * mu_a + mu_b * mu_b + kC1;
		const float b2 = (e_aa - mu_a * mu_a) + (e_bb - mu_b * mu_b) + kC2;
		const float inv_b = 1.0f / (b1 * b2);
		const float s = a1 * a2 * inv_b;
		const int64_t g = ((int64_t)y * width + x) * 3 + e % 3;
		ssim_map[g] = s;
		d_mu[g] = (2.0f * mu_b * (a2 - a1) - 2.0f * mu_a * s * (b2 - b1)) * inv_b;
		d_aa[g] = -s / b2;
		d_ab[g] = 2.0f * a1 * inv_b;
	}
}

// Backward: grad = dL/dmean / n * (blur(d_mu) + 2 a blur(d_aa) + b blur(d_ab)) (ssim.cu:74-113).
__global__ __launch_bounds__(256) void ssim_backward_kernel(int height, int width, const float* __restrict__ grad_mean,
															const float* __restrict__ img_a,
															const float* __restrict__ img_b,
															const float* __restrict__ p_mu, const float* __restrict__ p_aa,
															const float* __restrict__ p_ab,
															float* __restrict__ grad) {
	__shared__ float s_p[3][kHy][kHx * 3];
	__shared__ float s_h[3][kHy][kTx * 3];
	const int x0 = blockIdx.x * kTx - kR, y0 = blockIdx.y * kTy - kR;
	for (int i = threadIdx.x; i < kHy * kHx * 3; i += blockDim.x) {
		const int row = i / (kHx * 3), e = i - row * (kHx * 3);
		const int x = x0 + e / 3, y = y0 + row;
		const bool in = x >= 0 && x < width && y >= 0 && y < height;
		const int64_t g = ((int64_t)y * width + x) * 3 + e % 3;
		s_p[0][row][e] = in ? p_mu[g] : 0.0f;
		s_p[1][row][e] = in ? p_aa[g] : 0.0f;
		s_p[2][row][e] = in ? p_ab[g] : 0.0f;
	}
	__syncthreads();
	for (int i = threadIdx.x; i < kHy * kTx * 3; i += blockDim.x) {
		const int row = i / (kTx * 3), e = i - row * (kTx * 3);
		const int x = x0 + kR + e / 3;
		float s_mu = 0.0f, s_aa = 0.0f, s_ab = 0.0f;
#pragma unroll
		for (int k = -kR; k <= kR; k++) {
			if (x + k < 0 || x + k >= width) continue;
			const float w = kWin[k + kR];
			const int c = e + 3 * (kR + k);
			s_mu += w * s_p[0][row][c];
			s_aa += w * s_p[1][row][c];
			s_ab += w * s_p[2][row][c];
		}
		s_h[0][row][e] = s_mu;
		s_h[1][row][e] = s_aa;
		s_h[2][row][e] = s_ab;
	}
	__syncthreads();
	const int64_t n = (int64_t)height * width * 3;
	const float scale = grad_mean[0] / (float)n;
	for (int i = threadIdx.x; i < kTy * kTx * 3; i += blockDim.x) {
		const int row = i / (kTx * 3), e = i - row * (kTx * 3);
		const int x = x0 + kR + e / 3, y = y0 + kR + row;
		if (x >= width || y >= height) continue;
		float s_mu = 0.0f, s_aa = 0.0f, s_ab = 0.0f;
#pragma unroll
		for (int k = -kR; k <= kR; k++) {
			if (y + k < 0 || y + k >= height) continue;
			const float w = kWin[k + kR];
			const int r = row + kR + k;
			s_mu += w * s_h[0][r][e];
			s_aa += w * s_h[1][r][e];
			s_ab += w * s_h[2][r][e];
		}
		const int64_t g = ((int64_t)y * width + x) * 3 + e % 3;
		grad[g] = scale * (s_mu + 2.0f * img_a[g] * s_aa + img_b[g] * s_ab);
	}
}

int upload_window() {
	static int status = -1;
	if (status >= 0) return status;
	double w[2 * kR + 1], sum = 0.0;
	for (int i = 0; i < 2 * kR + 1; i++) {
		const double x = (double)(i - kR);
		w[i] = exp(-x * x / (2.0 * 1.5 * 1.5));
		sum += w[i];
	}
	float wf[2 * kR + 1];
	for (int i = 0; i < 2 * kR + 1; i++) wf[i] = (float)(w[i] / sum);
	const hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(kWin), wf, sizeof(wf));
	status = e == hipSuccess ? HDS_OK : hds_set_error(HDS_ERR_RUNTIME, "ssim window upload: %s", hipGetErrorString(e));
	return status;
}

}  // namespace

extern "C" int hds_ssim_forward(int height, int width, const float* rendered, const float* gt, float* ssim_map,
								float* d_mu, float* d_aa, float* d_ab, hds_stream_t stream) {
	HDS_REQUIRE(height > 0 && width > 0, "ssim inputs must both be [H, W, 3] with H, W > 0");
	HDS_REQUIRE(rendered && gt && ssim_map && d_mu && d_aa && d_ab, "ssim_forward: null pointer argument");
	int st = upload_window();
	if (st != HDS_OK) return st;
	hipStream_t s = (hipStream_t)stream;
	const dim3 grid((unsigned)((width + kTx - 1) / kTx), (unsigned)((height + kTy - 1) / kTy));
	HdsKernelTimer timer1("ssim_forward_kernel", s);
	ssim_forward_kernel<<<grid, 256, 0, s>>>(height, width, rendered, gt, ssim_map, d_mu, d_aa, d_ab);
	timer1.stop();
	HDS_LAUNCH_CHECK("ssim_forward", s);
	return HDS_OK;
}

extern "C" int hds_ssim_backward(int height, int width, const float* grad_mean, const float* rendered, const float* gt,
								 const float* d_mu, const float* d_aa, const float* d_ab, float* grad_rendered,
								 hds_stream_t stream) {
	HDS_REQUIRE(height > 0 && width > 0, "ssim inputs must both be [H, W, 3] with H, W > 0");
	HDS_REQUIRE(grad_mean && rendered && gt && d_mu && d_aa && d_ab && grad_rendered, "ssim_backward: null pointer argument");
	int st = upload_window();
	if (st != HDS_OK) return st;
	hipStream_t s = (hipStream_t)stream;
	const dim3 grid((unsigned)((width + kTx - 1) / kTx), (unsigned)((height + kTy - 1) / kTy));
	HdsKernelTimer timer2("ssim_backward_kernel", s);
	ssim_backward_kernel<<<grid, 256, 0, s>>>(height, width, grad_mean, rendered, gt, d_mu, d_aa, d_ab, grad_rendered);
	timer2.stop();
	HDS_LAUNCH_CHECK("ssim_backward", s);
	return HDS_OK;
}
