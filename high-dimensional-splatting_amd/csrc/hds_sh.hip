// Spherical-harmonic colours (degrees 0-3) and the fused SH backward + Adam step.
//
// eval_sh: one thread per gaussian, rgb = max(0.5 + sum_j b_j(dir) w_j, 0), culled -> 0
// (sh.cu:62-83). The backward computes the 48 SH gradients of each gaussian into LDS, writes
// grad_dirs, then the work-group steps Adam over its contiguous block of sh_dc / sh_rest with
// coalesced loads, so SH gradients never reach HBM (sh.cu:104-154, docs/rasterizer.md:56-100).
// The basis constants are the real SH of the 3DGS convention, sh.cu:9-15 / test_sh.py:27-47.
#include "hds_internal.h"
#include "hds_rasterizer.h"

namespace {

__constant__ float kShC[16] = {
	0.28209479177387814f,  -0.4886025119029199f, 0.4886025119029199f,  -0.4886025119029199f,
	1.0925484305920792f,   -1.0925484305920792f, 0.31539156525252005f, -1.0925484305920792f,
	0.5462742152960396f,   -0.5900435899266435f, 2.890611442640554f,   -0.4570457994644658f,
	0.3731763325901154f,   -0.4570457994644658f, 1.445305721320277f,   -0.5900435899266435f,
};

__device__ inline void sh_basis(float x, float y, float z, int k, float* b) {
	const float xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
	b[0] = kShC[0];
	if (k <= 1) return;
	b[1] = kShC[1] * y;
	b[2] = kShC[2] * z;
	b[3] = kShC[3] * x;
	if (k <= 4) return;
	b[4] = kShC[4] * xy;
	b[5] = kShC[5] * yz;
	b[6] = kShC[6] * (2 * zz - xx - yy);
	b[7] = kShC[7] * xz;
	b[8] = kShC[8] * (xx - yy);
	if (k <= 9) return;
	b[9] = kShC[9] * y * (3 * xx - yy);
	b[10] = kShC[10] * xy * z;
	b[11] = kShC[11] * y * (4 * zz - xx - yy);
	b[12] = kShC[12] * z * (2 * zz - 3 * xx - 3 * yy);
	b[13] = kShC[13] * x * (4 * zz - xx - yy);
	b[14] = kShC[14] * z * (xx - yy);
	b[15] = kShC[15] * x * (xx - 3 * yy);
}

// Gradient of each basis function with respect to the direction (sh.cu:34-55 semantics).
__device__ inline void sh_basis_grad(float x, float y, float z, int k, float* bx, float* by, float* bz) {
	const float xx = x * x, yy = y * y, zz = z * z;
#pragma unroll
	for (int j = 0; j < 16; j++) bx[j] = by[j] = bz[j] = 0.0f;
	if (k <= 1) return;
	by[1] = kShC[1];
	bz[2] = kShC[2];
	bx[3] = kShC[3];
	if (k <= 4) return;
	bx[4] = kShC[4] * y;
	by[4] = kShC[4] * x;
	by[5] = kShC[5] * z;
	bz[5] = kShC[5] * y;
	bx[6] = kShC[6] * (-2 * x);
	by[6] = kShC[6] * (-2 * y);
	bz[6] = kShC[6] * (4 * z);
	bx[7] = kShC[7] * z;
	bz[7] = kShC[7] * x;
	bx[8] = kShC[8] * (2 * x);
	by[8] = kShC[8] * (-2 * y);
	if (k <= 9) return;
	bx[9] = kShC[9] * (6 * x * y);
	by[9] = kShC[9] * (3 * xx - 3 * yy);
	bx[10] = kShC[10] * y * z;
	by[10] = kShC[10] * x * z;
	bz[10] = kShC[10] * x * y;
	bx[11] = kShC[11] * (-2 * x * y);
	by[11] = kShC[11] * (4 * zz - xx - 3 * yy);
	bz[11] = kShC[11] * (8 * y * z);
	bx[12] = kShC[12] * (-6 * x * z);
	by[12] = kShC[12] * (-6 * y * z);
	bz[12] = kShC[12] * (6 * zz - 3 * xx - 3 * yy);
	bx[13] = kShC[13] * (4 * zz - 3 * xx - yy);
	by[13] = kShC[13] * (-2 * x * y);
	bz[13] = kShC[13] * (8 * x * z);
	bx[14] = kShC[14] * (2 * x * z);
	by[14] = kShC[14] * (-2 * y * z);
	bz[14] = kShC[14] * (xx - yy);
	bx[15] = kShC[15] * (3 * xx - 3 * yy);
	by[15] = kShC[15] * (-6 * x * y);
}

__device__ inline float sh_weight(const float* dc, const float* rest, int j, int c) {
	return j == 0 ? dc[c] : rest[(j - 1) * 3 + c];
}

constexpr int kShEvalBlock = 256;

__global__ __launch_bounds__(kShEvalBlock) void eval_sh_kernel(int64_t n, int k, const float* __restrict__ sh_dc,
													  const float* __restrict__ sh_rest, const float* __restrict__ dirs,
													  const float* __restrict__ radii, float* __restrict__ rgb) {
	// The block's higher-order rows are one contiguous run of count * 45 floats: read it coalesced
	// into LDS (a thread's own row, read directly, puts 64 cache lines under every load). Row
	// stride 45 is odd, so the per-thread LDS reads hit 64 different banks.
	__shared__ float s_rest[kShEvalBlock * 45];
	const int64_t first = (int64_t)blockIdx.x * kShEvalBlock;
	const int64_t i = first + threadIdx.x;
	if (k > 1) {
		const int count = (int)(n - first < kShEvalBlock ? n - first : kShEvalBlock);
		const float* src = sh_rest + first * 45;
		for (int e = threadIdx.x; e < count * 45; e += kShEvalBlock) s_rest[e] = src[e];
		__syncthreads();
	}
	if (i >= n) return;
	if (!(radii[i] > 0.0f)) {
		rgb[i * 3 + 0] = rgb[i * 3 + 1] = rgb[i * 3 + 2] = 0.0f;
		return;
	}
	float b[16];
	sh_basis(dirs[i * 3], dirs[i * 3 + 1], dirs[i * 3 + 2], k, b);
	const float* dc = sh_dc + i * 3;
	const float* rest = s_rest + threadIdx.x * 45;
	for (int c = 0; c < 3; c++) {
		float value = 0.5f;
		for (int j = 0; j < k; j++) value += b[j] * sh_weight(dc, rest, j, c);
		rgb[i * 3 + c] = fmaxf(value, 0.0f);
	}
}

struct AdamArgs {
	float lr_dc, lr_rest, beta1, beta2, one_minus_beta1, one_minus_beta2, eps;
};

constexpr int kShAdamBlock = 256;

// One Adam step over `len` contiguous parameters whose gradients sit in LDS.
__device__ inline void adam_block(float* p, float* m, float* v, const float* g, int len, float step, float lr,
								  const AdamArgs& a) {
	const float step_size = lr / (1.0f - powf(a.beta1, step));
	const float bc2_sqrt = sqrtf(1.0f - powf(a.beta2, step));
	for (int t = threadIdx.x; t < len; t += blockDim.x) {
		const float grad = g[t];
		const float mt = m[t] + a.one_minus_beta1 * (grad - m[t]);
		const float vt = a.beta2 * v[t] + a.one_minus_beta2 * grad * grad;
		m[t] = mt;
		v[t] = vt;
		p[t] -= step_size * mt / (sqrtf(vt) / bc2_sqrt + a.eps);
	}
}

__global__ __launch_bounds__(kShAdamBlock) void eval_sh_backward_adam_kernel(
	int64_t n, int k, const float* __restrict__ grad_rgb, float* __restrict__ sh_dc, float* __restrict__ sh_rest,
	const float* __restrict__ dirs, const float* __restrict__ radii, float* __restrict__ m_dc,
	float* __restrict__ v_dc, float* __restrict__ m_rest, float* __restrict__ v_rest,
	const float* __restrict__ step_dc, const float* __restrict__ step_rest, AdamArgs a,
	float* __restrict__ grad_dirs) {
	__shared__ float s_dc[kShAdamBlock * 3];
	__shared__ float s_rest[kShAdamBlock * 45];
	const int64_t first = (int64_t)blockIdx.x * kShAdamBlock;
	const int64_t i = first + threadIdx.x;
	float* gdc = s_dc + threadIdx.x * 3;
	float* grest = s_rest + threadIdx.x * 45;
	if (k > 1) {
		// The block's coefficient rows, read coalesced into the gradient rows; a thread only
		// touches its own row, reading each weight before its gradient replaces it.
		const int rows = (int)min((int64_t)kShAdamBlock, n - first);
		const float* src = sh_rest + first * 45;
		for (int e = threadIdx.x; e < rows * 45; e += kShAdamBlock) s_rest[e] = src[e];
		__syncthreads();
	}
	if (i < n) {
		float dd[3] = {0.0f, 0.0f, 0.0f};
		if (radii[i] > 0.0f) {
			float b[16], bx[16], by[16], bz[16];
			const float x = dirs[i * 3], y = dirs[i * 3 + 1], z = dirs[i * 3 + 2];
			sh_basis(x, y, z, k, b);
			sh_basis_grad(x, y, z, k, bx, by, bz);
			const float* dc = sh_dc + i * 3;
			const float* rest = grest;
			// The colour clamp passes no gradient where it clipped; recomputed, not stored.
			float g[3];
			for (int c = 0; c < 3; c++) {
				float value = 0.5f;
				for (int j = 0; j < k; j++) value += b[j] * sh_weight(dc, rest, j, c);
				g[c] = value > 0.0f ? grad_rgb[i * 3 + c] : 0.0f;
			}
			for (int j = 0; j < 16; j++) {
				float t = 0.0f;
				for (int c = 0; c < 3; c++) {
					const float weight = j < k ? sh_weight(dc, rest, j, c) : 0.0f;
					const float grad = j < k ? b[j] * g[c] : 0.0f;
					if (j == 0)
						gdc[c] = grad;
					else
						grest[(j - 1) * 3 + c] = grad;
					if (j < k) t += weight * g[c];
				}
				if (j < k) {
					dd[0] += t * bx[j];
					dd[1] += t * by[j];
					dd[2] += t * bz[j];
				}
			}
		} else {
			for (int c = 0; c < 3; c++) gdc[c] = 0.0f;
			for (int j = 0; j < 45; j++) grest[j] = 0.0f;
		}
		for (int c = 0; c < 3; c++) grad_dirs[i * 3 + c] = dd[c];
	}
	__syncthreads();
	const int count = (int)min((int64_t)kShAdamBlock, n - first);
	adam_block(sh_dc + first * 3, m_dc + first * 3, v_dc + first * 3, s_dc, count * 3, *step_dc, a.lr_dc, a);
	adam_block(sh_rest + first * 45, m_rest + first * 45, v_rest + first * 45, s_rest, count * 45, *step_rest,
			   a.lr_rest, a);
}

}  // namespace

extern "C" int hds_eval_sh(int64_t n, int degree, const float* sh_dc, const float* sh_rest, const float* dirs,
						   const float* radii, float* rgb, hds_stream_t stream) {
	HDS_REQUIRE(degree >= 0 && degree <= 3, "eval_sh: degree %d outside 0..3", degree);
	HDS_REQUIRE(n >= 0, "eval_sh: negative gaussian count");
	if (n == 0) return HDS_OK;
	HDS_REQUIRE(sh_dc && sh_rest && dirs && radii && rgb, "eval_sh: null pointer argument");
	hipStream_t s = (hipStream_t)stream;
	HdsKernelTimer timer1("eval_sh_kernel", s);
	eval_sh_kernel<<<hds_blocks(n, kShEvalBlock), kShEvalBlock, 0, s>>>(n, (degree + 1) * (degree + 1), sh_dc, sh_rest, dirs, radii, rgb);
	timer1.stop();
	HDS_LAUNCH_CHECK("eval_sh_forward", s);
	return HDS_OK;
}

extern "C" int hds_eval_sh_backward_adam(int64_t n, int degree, const float* grad_rgb, float* sh_dc, float* sh_rest,
										 const float* dirs, const float* radii, float* m_dc, float* v_dc,
										 float* m_rest, float* v_rest, const float* step_dc,
										 const float* step_rest, double lr_dc, double lr_rest, double beta1,
										 double beta2, double eps, float* grad_dirs, hds_stream_t stream) {
	HDS_REQUIRE(degree >= 0 && degree <= 3, "eval_sh_backward_adam: degree %d outside 0..3", degree);
	HDS_REQUIRE(n >= 0, "eval_sh_backward_adam: negative gaussian count");
	if (n == 0) return HDS_OK;
	HDS_REQUIRE(grad_rgb && sh_dc && sh_rest && dirs && radii && m_dc && v_dc && m_rest && v_rest && step_dc &&
					step_rest && grad_dirs,
				"eval_sh_backward_adam: null pointer argument");
	hipStream_t s = (hipStream_t)stream;
	// 1 - beta is formed in double, as torch does (sh.cu:85, 179-180).
	AdamArgs a{(float)lr_dc, (float)lr_rest, (float)beta1, (float)beta2, (float)(1.0 - beta1), (float)(1.0 - beta2),
			   (float)eps};
	HdsKernelTimer timer2("eval_sh_backward_adam_kernel", s);
	eval_sh_backward_adam_kernel<<<hds_blocks(n, kShAdamBlock), kShAdamBlock, 0, s>>>(
		n, (degree + 1) * (degree + 1), grad_rgb, sh_dc, sh_rest, dirs, radii, m_dc, v_dc, m_rest, v_rest, step_dc,
		step_rest, a, grad_dirs);
	timer2.stop();
	HDS_LAUNCH_CHECK("eval_sh_backward_adam", s);
	return HDS_OK;
}
