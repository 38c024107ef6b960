// Spherical-harmonic colours (degrees 0-3) and the SH backward fused with the Adam step.
//
// eval_sh: one thread per gaussian, rgb = max(0.5 + sum_j b_j(dir) w_j, 0), culled -> 0
// (sh.cu:62-83). The backward (sh.cu:104-154, utils/sh.py:26-109; the fusion is
// docs/rasterizer.md:56-100) never materialises the 48 SH gradients of a gaussian: they are the
// outer product b_j(dir) g_c of its basis and its masked colour gradient, so a work-group keeps only
// those 19 numbers per gaussian and steps the parameters one thread per coefficient, forming each
// gradient where Adam consumes it (eval_sh_backward_adam_kernel). The basis constants are the real
// SH of the 3DGS convention, sh.cu:9-15 / test_sh.py:27-47.
#include "hds_internal.h"
#include "hds_stage.h"
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

__device__ inline float sh_weight(const float* dc, const float* rest, int j, int c) {
	return j == 0 ? dc[c] : rest[(j - 1) * 3 + c];
}

constexpr int kShEvalBlock = 256;
constexpr int kShRestRow = 45;  // floats of sh_rest per gaussian (15 coefficients x 3 channels)

// Copies the run of count consecutive 45-float sh_rest rows that starts at src into LDS and waits
// for it (and for every earlier vector-memory read of the calling wave); the caller's barrier then
// publishes it. When src is 16-byte aligned (a work-group's run is count * 180 bytes, so a
// 256-gaussian run starts aligned when the tensor does) the run goes HBM -> LDS by
// global_load_lds_dwordx4, one contiguous 1 KB block per wave instruction and all of them in flight
// at once with no registers held; the last len % 4 floats, or the whole run when src is not
// aligned, are copied with 4-byte loads.
__device__ inline void stage_rest_rows(float* dst, const float* src, int count, bool vec) {
	const int len = count * kShRestRow;
	int done = 0;
	if (vec) {
		constexpr int kWaves = kShEvalBlock / 64;
		constexpr int kOpsMax = (kShEvalBlock * kShRestRow / 4 + 63) / 64;  // 1 KB blocks of a full run: 45
		const int len4 = len / 4;
		const int ops = (len4 + 63) / 64;
		const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
		for (int j = 0; j < (kOpsMax + kWaves - 1) / kWaves; j++) {
			const int op = wave + j * kWaves;
			const int e4 = op * 64 + lane;
			if (op < ops && e4 < len4)
				__builtin_amdgcn_global_load_lds(src + 4 * e4, (hds_lds_void*)(dst + op * 256), 16, 0, 0);
		}
		done = 4 * len4;
	}
	for (int e = done + (int)threadIdx.x; e < len; e += kShEvalBlock) dst[e] = src[e];
	hds_wait_vmem();
}

__global__ __launch_bounds__(kShEvalBlock) void eval_sh_kernel(int64_t n, int k, const float* __restrict__ sh_dc,
													  const float* __restrict__ sh_rest, const float* __restrict__ dirs,
													  const float* __restrict__ radii, float* __restrict__ rgb,
													  bool vec) {
	// The block's higher-order rows are one contiguous run of count * 45 floats: read it coalesced
	// into LDS (a thread's own row, read directly, puts 64 cache lines under every load). Row
	// stride 45 is odd, so the per-thread LDS reads hit 64 different banks.
	__shared__ __attribute__((aligned(16))) float s_rest[kShEvalBlock * kShRestRow];
	const int64_t first = (int64_t)blockIdx.x * kShEvalBlock;
	const int64_t i = first + threadIdx.x;
	if (k > 1) {
		const int count = (int)(n - first < kShEvalBlock ? n - first : kShEvalBlock);
		stage_rest_rows(s_rest, sh_rest + first * kShRestRow, count, vec);
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
	const float* rest = s_rest + threadIdx.x * kShRestRow;
	for (int c = 0; c < 3; c++) {
		float value = 0.5f;
		for (int j = 0; j < k; j++) value += b[j] * sh_weight(dc, rest, j, c);
		rgb[i * 3 + c] = fmaxf(value, 0.0f);
	}
}

// Direction gradient of the colour polynomial P(d) = sum_j t_j b_j(d), with t_j = sum_c w_jc g_c the
// weight of basis function j in the loss: the partial derivatives of the degree-1..3 terms of the
// basis above, collected per axis (degree 0 is constant).
__device__ inline void sh_poly_grad(float x, float y, float z, int k, const float* t, float& gx, float& gy,
									float& gz) {
	gx = gy = gz = 0.0f;
	if (k <= 1) return;
	gx = t[3] * kShC[3];
	gy = t[1] * kShC[1];
	gz = t[2] * kShC[2];
	if (k <= 4) return;
	const float c4 = t[4] * kShC[4], c5 = t[5] * kShC[5], c6 = t[6] * kShC[6], c7 = t[7] * kShC[7],
				c8 = t[8] * kShC[8];
	gx += c4 * y - 2.0f * c6 * x + c7 * z + 2.0f * c8 * x;
	gy += c4 * x + c5 * z - 2.0f * c6 * y - 2.0f * c8 * y;
	gz += c5 * y + 4.0f * c6 * z + c7 * x;
	if (k <= 9) return;
	const float xx = x * x, yy = y * y, zz = z * z;
	const float c9 = t[9] * kShC[9], c10 = t[10] * kShC[10], c11 = t[11] * kShC[11], c12 = t[12] * kShC[12],
				c13 = t[13] * kShC[13], c14 = t[14] * kShC[14], c15 = t[15] * kShC[15];
	gx += 6.0f * c9 * x * y + c10 * y * z - 2.0f * c11 * x * y - 6.0f * c12 * x * z + c13 * (4.0f * zz - 3.0f * xx - yy) +
		  2.0f * c14 * x * z + 3.0f * c15 * (xx - yy);
	gy += 3.0f * c9 * (xx - yy) + c10 * x * z + c11 * (4.0f * zz - xx - 3.0f * yy) - 6.0f * c12 * y * z -
		  2.0f * c13 * x * y - 2.0f * c14 * y * z - 6.0f * c15 * x * y;
	gz += c10 * x * y + 8.0f * c11 * y * z + c12 * (6.0f * zz - 3.0f * xx - 3.0f * yy) + 8.0f * c13 * x * z +
		  c14 * (xx - yy);
}

// Adam as torch.optim.Adam defines it (exp_avg.lerp_(g, 1 - beta1), exp_avg_sq = beta2 v + (1 - beta2)
// g^2, p -= lr / (1 - beta1^t) * m / (sqrt(v) / sqrt(1 - beta2^t) + eps)), with the 1 - beta terms
// formed in double on the host as torch does.
struct AdamStep {
	float step_size, bias2_sqrt, beta2, one_minus_beta1, one_minus_beta2, eps;
};

__device__ inline AdamStep adam_step(float lr, float step, float beta1, float beta2, float omb1, float omb2, float eps) {
	AdamStep a;
	a.step_size = lr / (1.0f - powf(beta1, step));
	a.bias2_sqrt = sqrtf(1.0f - powf(beta2, step));
	a.beta2 = beta2;
	a.one_minus_beta1 = omb1;
	a.one_minus_beta2 = omb2;
	a.eps = eps;
	return a;
}

__device__ inline float adam_update(float p, float& m, float& v, float g, const AdamStep& a) {
	m = m + a.one_minus_beta1 * (g - m);
	v = a.beta2 * v + a.one_minus_beta2 * g * g;
	return p - a.step_size * m / (sqrtf(v) / a.bias2_sqrt + a.eps);
}

struct AdamArgs {
	float lr_dc, lr_rest, beta1, beta2, one_minus_beta1, one_minus_beta2, eps;
};

constexpr int kShAdamBlock = kShEvalBlock;  // gaussians (and threads) per work-group
constexpr int kBRow = 17;                    // basis values per gaussian (16, odd stride)

// One work-group owns kShAdamBlock consecutive gaussians, i.e. one contiguous run of 3 * count sh_dc
// and 45 * count sh_rest parameters and of their moments.
//  1. The run's weights are read into LDS (sh_rest as 16-byte loads, all in flight at once).
//  2. Thread = gaussian: basis of its direction, colour per channel, the clamp mask (max(., 0) passes
//     no gradient where it clipped), g_c = masked dL/drgb_c, the direction gradient from the colour
//     polynomial, and (b_j, g_c) into LDS. Culled gaussians get b = g = 0.
//  3. Thread = parameter: the whole run is stepped with 16-byte moment reads and writes, all of a
//     thread's reads issued before its first update, each coefficient's gradient formed on the fly
//     as b_j g_c of its gaussian and channel (no gradient array is ever materialised) and its
//     current value taken from the LDS copy. Culled gaussians and coefficients above the degree get
//     a zero gradient and are still stepped, as an optimizer step over the whole tensors does.
__global__ __launch_bounds__(kShAdamBlock) void eval_sh_backward_adam_kernel(
	int64_t n, int k, const float* __restrict__ grad_rgb, float* __restrict__ sh_dc, float* __restrict__ sh_rest,
	const float* __restrict__ dirs, const float* __restrict__ radii, float* __restrict__ m_dc,
	float* __restrict__ v_dc, float* __restrict__ m_rest, float* __restrict__ v_rest,
	const float* __restrict__ step_dc, const float* __restrict__ step_rest, AdamArgs args,
	float* __restrict__ grad_dirs, bool vec) {
	__shared__ __attribute__((aligned(16))) float s_rest[kShAdamBlock * kShRestRow];
	__shared__ float s_dc[kShAdamBlock * 3];
	__shared__ float s_b[kShAdamBlock * kBRow];
	__shared__ float s_g[kShAdamBlock * 4];
	const int64_t first = (int64_t)blockIdx.x * kShAdamBlock;
	const int count = (int)min((int64_t)kShAdamBlock, n - first);
	const int tid = threadIdx.x;

	float* const dc_run = sh_dc + first * 3;
	float* const rest_run = sh_rest + first * kShRestRow;
	float* const mr = m_rest + first * kShRestRow;
	float* const vr = v_rest + first * kShRestRow;
	const int len = count * kShRestRow;
	const int len4 = len / 4;
	// The sh_rest moments are read first, four consecutive elements per thread and step, so that
	// they are in flight with the weights and stay in registers through the gradient phase
	// (clamped indices: every lane loads, only the updates are guarded).
	constexpr int kIters = (kShAdamBlock * kShRestRow / 4 + kShAdamBlock - 1) / kShAdamBlock;
	float4 m4[kIters], v4[kIters];
	if (vec) {
#pragma unroll
		for (int r = 0; r < kIters; r++) {
			const int e4 = min(tid + r * kShAdamBlock, len4 - 1);
			m4[r] = reinterpret_cast<const float4*>(mr)[e4];
			v4[r] = reinterpret_cast<const float4*>(vr)[e4];
		}
	}
	for (int e = tid; e < count * 3; e += kShAdamBlock) s_dc[e] = dc_run[e];
	stage_rest_rows(s_rest, rest_run, count, vec);
	__syncthreads();

	if (tid < count) {
		const int64_t i = first + tid;
		// w(j, c): coefficient j of channel c of this thread's gaussian.
		auto w = [&](int j, int c) { return j == 0 ? s_dc[tid * 3 + c] : s_rest[tid * kShRestRow + 3 * (j - 1) + c]; };
		float b[16];
		float g[3] = {0.0f, 0.0f, 0.0f};
		float gd[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
		for (int j = 0; j < 16; j++) b[j] = 0.0f;
		if (radii[i] > 0.0f) {
			const float x = dirs[i * 3], y = dirs[i * 3 + 1], z = dirs[i * 3 + 2];
			sh_basis(x, y, z, k, b);
#pragma unroll
			for (int c = 0; c < 3; c++) {
				float value = 0.5f;
				for (int j = 0; j < k; j++) value += b[j] * w(j, c);
				g[c] = value > 0.0f ? grad_rgb[i * 3 + c] : 0.0f;
			}
			float t[16];
#pragma unroll
			for (int j = 0; j < 16; j++) t[j] = j < k ? w(j, 0) * g[0] + w(j, 1) * g[1] + w(j, 2) * g[2] : 0.0f;
			sh_poly_grad(x, y, z, k, t, gd[0], gd[1], gd[2]);
#pragma unroll
			for (int j = 0; j < 16; j++)
				if (j >= k) b[j] = 0.0f;
		}
#pragma unroll
		for (int c = 0; c < 3; c++) grad_dirs[i * 3 + c] = gd[c];
#pragma unroll
		for (int j = 0; j < 16; j++) s_b[tid * kBRow + j] = b[j];
#pragma unroll
		for (int c = 0; c < 3; c++) s_g[tid * 4 + c] = g[c];
	}
	__syncthreads();

	const AdamStep a_dc = adam_step(args.lr_dc, *step_dc, args.beta1, args.beta2, args.one_minus_beta1,
									args.one_minus_beta2, args.eps);
	const AdamStep a_rest = adam_step(args.lr_rest, *step_rest, args.beta1, args.beta2, args.one_minus_beta1,
									  args.one_minus_beta2, args.eps);
	// sh_dc: coefficient j = 0 of gaussian e / 3, channel e % 3.
	for (int e = tid; e < count * 3; e += kShAdamBlock) {
		const int r = e / 3, c = e % 3;
		const float grad = s_b[r * kBRow] * s_g[r * 4 + c];
		float m = m_dc[first * 3 + e], v = v_dc[first * 3 + e];
		dc_run[e] = adam_update(s_dc[e], m, v, grad, a_dc);
		m_dc[first * 3 + e] = m;
		v_dc[first * 3 + e] = v;
	}
	// sh_rest: element e of the run is coefficient 1 + (e % 45) / 3 of gaussian e / 45, channel e % 3.
	auto rest_grad = [&](int e) {
		const int r = e / kShRestRow, q = e - r * kShRestRow;
		return s_b[r * kBRow + 1 + q / 3] * s_g[r * 4 + q % 3];
	};
	int done = 0;
	if (vec) {
#pragma unroll
		for (int r = 0; r < kIters; r++) {
			const int e4 = tid + r * kShAdamBlock;
			if (e4 < len4) {
				float m[4] = {m4[r].x, m4[r].y, m4[r].z, m4[r].w}, v[4] = {v4[r].x, v4[r].y, v4[r].z, v4[r].w}, p[4];
#pragma unroll
				for (int u = 0; u < 4; u++) p[u] = adam_update(s_rest[4 * e4 + u], m[u], v[u], rest_grad(4 * e4 + u), a_rest);
				reinterpret_cast<float4*>(rest_run)[e4] = make_float4(p[0], p[1], p[2], p[3]);
				reinterpret_cast<float4*>(mr)[e4] = make_float4(m[0], m[1], m[2], m[3]);
				reinterpret_cast<float4*>(vr)[e4] = make_float4(v[0], v[1], v[2], v[3]);
			}
		}
		done = 4 * len4;
	}
	for (int e = done + tid; e < len; e += kShAdamBlock) {
		float m = mr[e], v = vr[e];
		rest_run[e] = adam_update(s_rest[e], m, v, rest_grad(e), a_rest);
		mr[e] = m;
		vr[e] = v;
	}
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
	const bool vec = (reinterpret_cast<uintptr_t>(sh_rest) & 15u) == 0;
	eval_sh_kernel<<<hds_blocks(n, kShEvalBlock), kShEvalBlock, 0, s>>>(n, (degree + 1) * (degree + 1), sh_dc, sh_rest, dirs,
																	   radii, rgb, vec);
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
	// 16-byte accesses to the sh_rest run and its moments (each work-group's run starts 16-byte aligned
	// when the tensors do).
	const bool vec = ((reinterpret_cast<uintptr_t>(sh_rest) | reinterpret_cast<uintptr_t>(m_rest) |
					   reinterpret_cast<uintptr_t>(v_rest)) & 15u) == 0;
	eval_sh_backward_adam_kernel<<<hds_blocks(n, kShAdamBlock), kShAdamBlock, 0, s>>>(
		n, (degree + 1) * (degree + 1), grad_rgb, sh_dc, sh_rest, dirs, radii, m_dc, v_dc, m_rest, v_rest, step_dc,
		step_rest, a, grad_dirs, vec);
	timer2.stop();
	HDS_LAUNCH_CHECK("eval_sh_backward_adam", s);
	return HDS_OK;
}
