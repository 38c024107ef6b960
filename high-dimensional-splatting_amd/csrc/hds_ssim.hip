// SSIM loss kernels: forward (map + the three per-pixel partials the backward needs) and backward.
//
// Zero-padded separable 11-tap Gaussian window, sigma 1.5, C1 = 0.01^2, C2 = 0.03^2, on
// interleaved [H, W, 3] images (ssim.cu:6-113, utils/loss.py:8-9, 39-54). Forward: a work-group owns
// a strip 32 pixels wide (96 channel elements, one per thread) and 16 rows high. It reads the strip's input
// rows plus a 5-pixel halo on every side into LDS in one go (every load in flight at once), then
// walks down the rows: each input row is blurred horizontally from LDS, the last 11 blurred rows sit
// in a ring of registers, and each output row is their vertical blur. Nothing intermediate goes to
// HBM and the halo costs 1.6x the strip's reads; the row loop is unrolled by 11 so that the ring's
// slots are static registers. Out-of-image taps read zeros, which add +0 exactly where the
// reference skips them.
#include "hds_internal.h"
#include "hds_rasterizer.h"

namespace {

constexpr int kR = 5;                        // window radius
constexpr int kTaps = 2 * kR + 1;
constexpr int kSx = 32;                      // output pixels per strip
constexpr int kE = 3 * kSx;                  // output elements per row (one per computing thread)
constexpr int kEin = 3 * (kSx + 2 * kR);     // input elements per row, with the halo
constexpr int kRy = 16;                      // output rows per work-group
constexpr int kRows = kRy + 2 * kR;          // input rows per work-group
constexpr int kThreads = 128;
constexpr float kC1 = 0.01f * 0.01f, kC2 = 0.03f * 0.03f;

// exp(-x^2 / (2 * 1.5^2)) / sum over x = -5..5, evaluated in double and rounded to float.
__device__ constexpr float kWin[kTaps] = {0x1.0d956cp-10f, 0x1.f1fe02p-8f, 0x1.26eb18p-5f, 0x1.bff0fep-4f,
										  0x1.b43c40p-3f,  0x1.106560p-2f, 0x1.b43c40p-3f, 0x1.bff0fep-4f,
										  0x1.26eb18p-5f,  0x1.f1fe02p-8f, 0x1.0d956cp-10f};

// Reads kM arrays of the strip (input rows y0 - kR .., columns x0 - kR .., zeros outside the image)
// into s[m][row][element].
template <int kM>
__device__ inline void load_strip(float (*s)[kRows][kEin], const float* const (&src)[kM], int height, int width,
								  int x0, int y0) {
	for (int i = threadIdx.x; i < kRows * kEin; i += kThreads) {
		const int row = i / kEin, e = i - row * kEin;
		const int x = x0 - kR + e / 3, y = y0 - kR + row;
		const bool in = x >= 0 && x < width && y >= 0 && y < height;
		const int64_t g = ((int64_t)y * width + x) * 3 + e % 3;
#pragma unroll
		for (int m = 0; m < kM; m++) s[m][row][e] = in ? src[m][g] : 0.0f;
	}
}

// Forward: moments a, b, aa, bb, ab blurred -> ssim, d_mu, d_aa, d_ab (ssim.cu:39-72).
__global__ __launch_bounds__(kThreads) void ssim_forward_kernel(int height, int width, const float* __restrict__ img_a,
																const float* __restrict__ img_b, float* __restrict__ ssim_map,
																float* __restrict__ d_mu, float* __restrict__ d_aa,
																float* __restrict__ d_ab) {
	__shared__ float s_in[2][kRows][kEin];
	const int x0 = blockIdx.x * kSx, y0 = blockIdx.y * kRy;
	const float* const src[2] = {img_a, img_b};
	load_strip<2>(s_in, src, height, width, x0, y0);
	__syncthreads();
	const int t = threadIdx.x;
	if (t >= kE) return;
	const bool col_out = x0 + t / 3 < width;
	float ring[kTaps][5];  // horizontal blurs of a, b, aa, bb, ab for the last 11 input rows
#pragma unroll 1
	for (int r0 = 0; r0 < kRows; r0 += kTaps) {
#pragma unroll
		for (int j = 0; j < kTaps; j++) {
			const int r = r0 + j;  // input row; its ring slot is r % 11 = j
			if (r >= kRows) break;
			float sa = 0.0f, sb = 0.0f, saa = 0.0f, sbb = 0.0f, sab = 0.0f;
#pragma unroll
			for (int k = 0; k < kTaps; k++) {
				const float w = kWin[k];
				const float va = s_in[0][r][t + 3 * k], vb = s_in[1][r][t + 3 * k];
				sa += w * va;
				sb += w * vb;
				saa += w * va * va;
				sbb += w * vb * vb;
				sab += w * va * vb;
			}
			ring[j][0] = sa;
			ring[j][1] = sb;
			ring[j][2] = saa;
			ring[j][3] = sbb;
			ring[j][4] = sab;
			const int y = y0 + r - 2 * kR;  // output row whose window ends at input row r
			if (r < 2 * kR || !col_out || y >= height) continue;
			float mu_a = 0.0f, mu_b = 0.0f, e_aa = 0.0f, e_bb = 0.0f, e_ab = 0.0f;
#pragma unroll
			for (int k = 0; k < kTaps; k++) {
				const int slot = (j + 1 + k) % kTaps;  // input row r - 10 + k
				const float w = kWin[k];
				mu_a += w * ring[slot][0];
				mu_b += w * ring[slot][1];
				e_aa += w * ring[slot][2];
				e_bb += w * ring[slot][3];
				e_ab += w * ring[slot][4];
			}
			const float a1 = 2.0f * mu_a * mu_b + kC1;
			const float a2 = 2.0f * (e_ab - mu_a * mu_b) + kC2;
			const float b1 = mu_a * mu_a + mu_b * mu_b + kC1;
			const float b2 = (e_aa - mu_a * mu_a) + (e_bb - mu_b * mu_b) + kC2;
			const float inv_b = 1.0f / (b1 * b2);
			const float sv = a1 * a2 * inv_b;
			const int64_t g = ((int64_t)y * width + x0) * 3 + t;
			ssim_map[g] = sv;
			d_mu[g] = (2.0f * mu_b * (a2 - a1) - 2.0f * mu_a * sv * (b2 - b1)) * inv_b;
			d_aa[g] = -sv / b2;
			d_ab[g] = 2.0f * a1 * inv_b;
		}
	}
}

// Backward: the three partials are blurred with the window (whose transpose is itself) and combined
// per pixel. It stays a tiled kernel: a work-group owns 32 x 8 output pixels, reads their partials
// plus a 5-pixel halo into LDS once, blurs horizontally into LDS, then vertically. (The strip walk
// of the forward, which keeps 3 arrays in LDS here, ran 1.3-1.5x slower at 979x546 and 1920x1080.)
constexpr int kBx = 32, kBy = 8;
constexpr int kBhx = kBx + 2 * kR, kBhy = kBy + 2 * kR;
constexpr int kTiledThreads = 256;

// Backward: grad = dL/dmean / n * (blur(d_mu) + 2 a blur(d_aa) + b blur(d_ab)) (ssim.cu:74-113).
__global__ __launch_bounds__(kTiledThreads) void ssim_backward_kernel(int height, int width, const float* __restrict__ grad_mean,
															const float* __restrict__ img_a,
															const float* __restrict__ img_b,
															const float* __restrict__ p_mu, const float* __restrict__ p_aa,
															const float* __restrict__ p_ab,
															float* __restrict__ grad) {
	__shared__ float s_p[3][kBhy][kBhx * 3];
	__shared__ float s_h[3][kBhy][kBx * 3];
	const int x0 = blockIdx.x * kBx - kR, y0 = blockIdx.y * kBy - kR;
	for (int i = threadIdx.x; i < kBhy * kBhx * 3; i += blockDim.x) {
		const int row = i / (kBhx * 3), e = i - row * (kBhx * 3);
		const int x = x0 + e / 3, y = y0 + row;
		const bool in = x >= 0 && x < width && y >= 0 && y < height;
		const int64_t g = ((int64_t)y * width + x) * 3 + e % 3;
		s_p[0][row][e] = in ? p_mu[g] : 0.0f;
		s_p[1][row][e] = in ? p_aa[g] : 0.0f;
		s_p[2][row][e] = in ? p_ab[g] : 0.0f;
	}
	__syncthreads();
	for (int i = threadIdx.x; i < kBhy * kBx * 3; i += blockDim.x) {
		const int row = i / (kBx * 3), e = i - row * (kBx * 3);
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
	for (int i = threadIdx.x; i < kBy * kBx * 3; i += blockDim.x) {
		const int row = i / (kBx * 3), e = i - row * (kBx * 3);
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

}  // namespace

extern "C" int hds_ssim_forward(int height, int width, const float* rendered, const float* gt, float* ssim_map,
								float* d_mu, float* d_aa, float* d_ab, hds_stream_t stream) {
	HDS_REQUIRE(height > 0 && width > 0, "ssim inputs must both be [H, W, 3] with H, W > 0");
	HDS_REQUIRE(rendered && gt && ssim_map && d_mu && d_aa && d_ab, "ssim_forward: null pointer argument");
	hipStream_t s = (hipStream_t)stream;
	const dim3 grid((unsigned)((width + kSx - 1) / kSx), (unsigned)((height + kRy - 1) / kRy));
	HdsKernelTimer timer1("ssim_forward_kernel", s);
	ssim_forward_kernel<<<grid, kThreads, 0, s>>>(height, width, rendered, gt, ssim_map, d_mu, d_aa, d_ab);
	timer1.stop();
	HDS_LAUNCH_CHECK("ssim_forward", s);
	return HDS_OK;
}

extern "C" int hds_ssim_backward(int height, int width, const float* grad_mean, const float* rendered, const float* gt,
								 const float* d_mu, const float* d_aa, const float* d_ab, float* grad_rendered,
								 hds_stream_t stream) {
	HDS_REQUIRE(height > 0 && width > 0, "ssim inputs must both be [H, W, 3] with H, W > 0");
	HDS_REQUIRE(grad_mean && rendered && gt && d_mu && d_aa && d_ab && grad_rendered, "ssim_backward: null pointer argument");
	hipStream_t s = (hipStream_t)stream;
	const dim3 grid((unsigned)((width + kBx - 1) / kBx), (unsigned)((height + kBy - 1) / kBy));
	HdsKernelTimer timer2("ssim_backward_kernel", s);
	ssim_backward_kernel<<<grid, kTiledThreads, 0, s>>>(height, width, grad_mean, rendered, gt, d_mu, d_aa, d_ab, grad_rendered);
	timer2.stop();
	HDS_LAUNCH_CHECK("ssim_backward", s);
	return HDS_OK;
}
