// Back-to-front replay of the blend: RGB and feature gradients in one walk.
//
// Layout as in the forward: work-group = tile x slice of S channels, wave = 8x8 pixel block,
// lane = pixel. Each lane restarts from its final T and n_contrib and walks its tile's list back
// to front (backward.cu:53-163, features.cu:419-541):
//   T <- T / (1 - alpha);  RGB: accum_rec recurrence, dL/dalpha = (c - rec).g T - T_f/(1-a) bg.g;
//   features: dL/dalpha += T (dot - behind_dot), behind_dot <- a dot + (1 - a) behind_dot,
//   with dot = f . dL/dF[pixel];  geometry gradients only where the raw alpha <= 0.99.
// RGB and feature terms are summed into one dL/dalpha per pixel, then opacity, mean and conic
// gradients follow once (the reference sums two kernels' outputs, rasterizer/__init__.py:160-162).
//
// Every reduction over the wave's 64 pixels runs on MFMA in split-bf16, once per group of 16
// gaussians the wave walks next:
//   dot[px][g]  = sum_c dL/dF[px][c] F[g][c]     (A = dL/dF held in VGPRs, K = channels)
//   dF[g][c]   += sum_px w[px][g] dL/dF[px][c]   (B = dL/dF held in VGPRs, K = pixels, w = alpha T)
//   mom[g][j]   = sum_px s[px][g] P[px][j]       (s = G dL/dalpha, P = 1, x, y, x^2, xy, y^2)
//   rgb[g][c]   = sum_px w[px][g] dL/dRGB[px][c]
// dL/dF of the wave's 64 pixels lives in registers in both operand layouts for the whole walk, so
// the feature gradient of a gaussian needs no cross-lane reduction: the MFMA sums over pixels.
// The six geometry gradients are polynomials in the pixel offsets d = px - mean, so they follow
// from the six pixel moments of s about the block centre: dopac = sum s, dmean = op Q sum s d,
// dconic = -op (sum s dx^2 / 2, sum s dx dy, sum s dy^2 / 2). One lane per gaussian then turns
// moments into gradients and issues the atomics. Slices add their partial dot terms linearly
// through the same atomics (features.cu:348-349).
#include "hds_internal.h"
#include "hds_rasterizer.h"

namespace {

constexpr int kBatch = 64;
constexpr int kGroup = 16;       // gaussians per contraction group (N of the dot MFMA, M of dF)
constexpr int kRowStride = 68;   // words per [group position][pixel] row, 16-byte aligned
constexpr int kIlp = 4;          // positions whose alpha is evaluated together

struct BackwardArgs {
	int width, height, tiles_x, channels;
	const int2* ranges;
	const int* values;
	const float2* means2D;
	const float4* conic4;
	const float4* color_op4;
	const float* background;
	const float* final_T;
	const int* n_contrib;
	const float* grad_image;
	const float* features;
	const float* grad_feature_image;
	float* grad_means2D;
	float* grad_conics;
	float* grad_colors;
	float* grad_opacities;
	float* grad_features;
};

template <int S>
struct Slice {
	static constexpr int kKc = S / 32;      // K steps over channels (dot)
	static constexpr int kNcb = S / 16;     // 16-channel blocks (dF)
	static constexpr int kStride = S + 4;   // words per staged feature row
};

template <int S, bool RGB>
__global__ __launch_bounds__(256) void render_backward_kernel(const BackwardArgs a) {
	constexpr int kKc = S > 0 ? Slice<S>::kKc : 1;
	constexpr int kNcb = S > 0 ? Slice<S>::kNcb : 1;
	constexpr int kStride = S > 0 ? Slice<S>::kStride : 1;

	__shared__ int s_gid[kBatch];
	__shared__ float2 s_mean[kBatch];
	__shared__ float4 s_conic[kBatch];
	__shared__ float4 s_color[RGB ? kBatch : 1];
	__shared__ float4 s_box[kBatch];
	__shared__ __attribute__((aligned(16))) uint32_t s_feat[S > 0 ? (kBatch + 1) * kStride : 1];
	__shared__ __attribute__((aligned(16))) float s_dot[S > 0 ? 4 * kGroup * kRowStride : 1];
	__shared__ __attribute__((aligned(16))) uint32_t s_w[4 * kGroup * kRowStride];
	__shared__ __attribute__((aligned(16))) uint32_t s_s[4 * kGroup * kRowStride];
	__shared__ __attribute__((aligned(16))) float s_mom[4 * kGroup * 16];
	__shared__ int s_slot[4 * kGroup];
	__shared__ int s_max_last;

	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const int tile = blockIdx.x, slice = blockIdx.y;
	const int tx0 = (tile % a.tiles_x) * HDS_TILE, ty0 = (tile / a.tiles_x) * HDS_TILE;
	const int wx0 = tx0 + (wave & 1) * 8, wy0 = ty0 + (wave >> 1) * 8;
	const int px = wx0 + (lane & 7), py = wy0 + (lane >> 3);
	const bool inside = px < a.width && py < a.height;
	const int64_t pix = (int64_t)py * a.width + px;
	const float fx = (float)px + 0.5f, fy = (float)py + 0.5f;
	const float rx0 = (float)wx0 + 0.5f, rx1 = (float)wx0 + 7.5f;
	const float ry0 = (float)wy0 + 0.5f, ry1 = (float)wy0 + 7.5f;
	const float centre_x = (float)wx0 + 4.0f, centre_y = (float)wy0 + 4.0f;
	const int c0 = slice * S;
	const bool do_rgb = RGB && slice == 0;
	const bool want_dF = S > 0 && a.grad_features != nullptr;

	const float T_final = inside ? a.final_T[pix] : 0.0f;
	const int last = inside ? a.n_contrib[pix] : 0;
	float T = T_final;
	float gr = 0.0f, gg = 0.0f, gb = 0.0f, dL_dTf = 0.0f;
	if (do_rgb && inside) {
		gr = a.grad_image[pix * 3 + 0];
		gg = a.grad_image[pix * 3 + 1];
		gb = a.grad_image[pix * 3 + 2];
		dL_dTf = a.background[0] * gr + a.background[1] * gg + a.background[2] * gb;
	}
	float rec_r = 0.0f, rec_g = 0.0f, rec_b = 0.0f, last_alpha = 0.0f;
	float last_r = 0.0f, last_g = 0.0f, last_b = 0.0f, behind_dot = 0.0f;

	// P, the B operand of the moment MFMAs: lane = (pixels 32pk + 8(lane >> 4) + 0..7, column
	// lane & 15) with columns 1, x, y, x^2, xy, y^2 about the block centre (exact in bf16), then the
	// pixel's dL/dRGB (split) for the colour gradients, then zeros.
	hds_bf16x8 p_hi[2], p_lo[2];
	{
		const int colj = lane & 15;
#pragma unroll
		for (int pk = 0; pk < 2; pk++) {
			uint32_t d[8];
#pragma unroll
			for (int j = 0; j < 8; j++) {
				const int p = 32 * pk + 8 * (lane >> 4) + j;
				const float xl = (float)(p & 7) - 3.5f, yl = (float)(p >> 3) - 3.5f;
				float v = 0.0f;
				if (colj == 0) v = 1.0f;
				else if (colj == 1) v = xl;
				else if (colj == 2) v = yl;
				else if (colj == 3) v = xl * xl;
				else if (colj == 4) v = xl * yl;
				else if (colj == 5) v = yl * yl;
				else if (colj < 9 && do_rgb) {
					const int x = wx0 + (p & 7), y = wy0 + (p >> 3);
					if (x < a.width && y < a.height) v = a.grad_image[((int64_t)y * a.width + x) * 3 + (colj - 6)];
				}
				d[j] = hds_split_pack(v);
			}
			hds_unpack8(d, p_hi[pk], p_lo[pk]);
		}
	}

	// dL/dF of the wave's 64 pixels in both MFMA operand layouts.
	//   ga: A of dot, lane = (pixel 16m + (lane & 15), channels 32kk + 8(lane >> 4) + 0..7)
	//   gb: B of dF,  lane = (pixels 32pk + 8(lane >> 4) + 0..7, channel 16n + (lane & 15))
	hds_bf16x8 ga_hi[4][kKc], ga_lo[4][kKc], gb_hi[2][kNcb], gb_lo[2][kNcb];
	if constexpr (S > 0) {
#pragma unroll
		for (int m = 0; m < 4; m++) {
			const int p = 16 * m + (lane & 15);
			const int x = wx0 + (p & 7), y = wy0 + (p >> 3);
			const bool in = x < a.width && y < a.height;
			const float* src = a.grad_feature_image + ((int64_t)y * a.width + x) * a.channels + c0 + 8 * (lane >> 4);
#pragma unroll
			for (int kk = 0; kk < kKc; kk++) {
				float4 v0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), v1 = v0;
				if (in) {
					v0 = *reinterpret_cast<const float4*>(src + 32 * kk);
					v1 = *reinterpret_cast<const float4*>(src + 32 * kk + 4);
				}
				const uint32_t d[8] = {hds_split_pack(v0.x), hds_split_pack(v0.y), hds_split_pack(v0.z), hds_split_pack(v0.w),
									   hds_split_pack(v1.x), hds_split_pack(v1.y), hds_split_pack(v1.z), hds_split_pack(v1.w)};
				hds_unpack8(d, ga_hi[m][kk], ga_lo[m][kk]);
			}
		}
#pragma unroll
		for (int pk = 0; pk < 2; pk++) {
#pragma unroll
			for (int n = 0; n < kNcb; n++) {
				uint32_t d[8];
#pragma unroll
				for (int j = 0; j < 8; j++) {
					const int p = 32 * pk + 8 * (lane >> 4) + j;
					const int x = wx0 + (p & 7), y = wy0 + (p >> 3);
					float v = 0.0f;
					if (x < a.width && y < a.height)
						v = a.grad_feature_image[((int64_t)y * a.width + x) * a.channels + c0 + 16 * n + (lane & 15)];
					d[j] = hds_split_pack(v);
				}
				hds_unpack8(d, gb_hi[pk][n], gb_lo[pk][n]);
			}
		}
		for (int i = tid; i < kStride; i += blockDim.x) s_feat[kBatch * kStride + i] = 0u;
	}

	// Nothing past the deepest contributor of the tile can matter (backward.cu:53-60).
	if (tid == 0) s_max_last = 0;
	__syncthreads();
	if (last > 0) atomicMax(&s_max_last, last);
	__syncthreads();
	const int2 range = a.ranges[tile];
	const int num = min(range.y - range.x, s_max_last);
	const int wave_last = hds_wave_max(last);

	int* slots = s_slot + wave * kGroup;
	float* dot_rows = s_dot + wave * kGroup * kRowStride;
	uint32_t* w_rows = s_w + wave * kGroup * kRowStride;
	uint32_t* s_rows = s_s + wave * kGroup * kRowStride;
	float* mom = s_mom + wave * kGroup * 16;

	for (int batch_end = num; batch_end > 0; batch_end -= kBatch) {
		const int cnt = min(kBatch, batch_end);
		const int batch_start = batch_end - cnt;
		__syncthreads();
		if (tid < cnt) {
			const int gid = a.values[range.x + batch_start + tid];
			const float2 m = a.means2D[gid];
			const float4 co = a.conic4[gid];
			s_gid[tid] = gid;
			s_mean[tid] = m;
			s_conic[tid] = co;
			if constexpr (RGB) s_color[tid] = a.color_op4[gid];
			s_box[tid] = hds_cull_box(m, co);
		}
		if constexpr (S > 0) {
			// Feature rows of the batch, each read once for the whole tile; thread groups of S / 4 share
			// a row, so the gaussian id is one broadcast load.
			constexpr int kVec = S / 4;
			for (int i = tid; i < cnt * kVec; i += blockDim.x) {
				const int row = i / kVec, q = i - row * kVec;
				const int gid = a.values[range.x + batch_start + row];
				const float4 f = *reinterpret_cast<const float4*>(a.features + (size_t)gid * a.channels + c0 + 4 * q);
				*reinterpret_cast<uint4*>(&s_feat[row * kStride + 4 * q]) =
					make_uint4(hds_split_pack(f.x), hds_split_pack(f.y), hds_split_pack(f.z), hds_split_pack(f.w));
			}
		}
		__syncthreads();

		uint64_t hits = hds_ballot(lane < cnt && batch_start + lane < wave_last &&
								   hds_box_hits(s_box[lane < cnt ? lane : 0], rx0, rx1, ry0, ry1));
		while (hits) {
			// Next group: up to 16 candidates, deepest first.
			int count = 0;
			while (hits && count < kGroup) {
				const int slot = 63 - __builtin_clzll(hits);
				hits &= ~(1ull << slot);
				if (lane == 0) slots[count] = slot;
				count++;
			}
			if (lane >= count && lane < kGroup) slots[lane] = kBatch;
			hds_wave_fence();

			if constexpr (S > 0) {
				// dot[px][g]: B = F^T, lane = (channels 32kk + 8(lane >> 4) + 0..7, position lane & 15).
				const uint32_t* frow = s_feat + slots[lane & 15] * kStride + 8 * (lane >> 4);
				hds_bf16x8 fb_hi[kKc], fb_lo[kKc];
#pragma unroll
				for (int kk = 0; kk < kKc; kk++) {
					const uint4 d0 = *reinterpret_cast<const uint4*>(frow + 32 * kk);
					const uint4 d1 = *reinterpret_cast<const uint4*>(frow + 32 * kk + 4);
					const uint32_t d[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
					hds_unpack8(d, fb_hi[kk], fb_lo[kk]);
				}
#pragma unroll
				for (int m = 0; m < 4; m++) {
					hds_f32x4 dacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
					for (int kk = 0; kk < kKc; kk++)
						dacc = hds_mfma_split(ga_hi[m][kk], ga_lo[m][kk], fb_hi[kk], fb_lo[kk], dacc);
					// D: rows = pixels 16m + 4(lane >> 4) + i, column = position lane & 15.
					*reinterpret_cast<float4*>(&dot_rows[(lane & 15) * kRowStride + 16 * m + 4 * (lane >> 4)]) =
						make_float4(dacc[0], dacc[1], dacc[2], dacc[3]);
				}
				hds_wave_fence();
			}

			// Back-to-front replay of the group, kIlp positions at a time: their alphas are
			// independent, only T and the behind-sums chain through them.
			uint32_t active = 0;
			for (int q0 = 0; q0 < count; q0 += kIlp) {
				int slot[kIlp];
				float raw[kIlp], G[kIlp], dot[kIlp];
#pragma unroll
				for (int u = 0; u < kIlp; u++) {
					slot[u] = slots[min(q0 + u, kGroup - 1)];
					const int sl = min(slot[u], kBatch - 1);
					float dx, dy;
					raw[u] = hds_raw_alpha(fx, fy, s_mean[sl], s_conic[sl], G[u], dx, dy);
					dot[u] = 0.0f;
					if constexpr (S > 0) dot[u] = dot_rows[min(q0 + u, kGroup - 1) * kRowStride + lane];
				}
#pragma unroll
				for (int u = 0; u < kIlp; u++) {
					const int q = q0 + u;
					if (q >= count) break;
					const float alpha = fminf(HDS_MAX_ALPHA, raw[u]);
					const bool contributes = inside && batch_start + slot[u] < last && alpha >= HDS_MIN_ALPHA;
					float dL_dalpha = 0.0f, w = 0.0f;
					if (contributes) {
						const float inv_1ma = __builtin_amdgcn_rcpf(1.0f - alpha);
						T *= inv_1ma;
						w = alpha * T;
						if (do_rgb) {
							const float4 col = s_color[slot[u]];
							rec_r = last_alpha * last_r + (1.0f - last_alpha) * rec_r;
							rec_g = last_alpha * last_g + (1.0f - last_alpha) * rec_g;
							rec_b = last_alpha * last_b + (1.0f - last_alpha) * rec_b;
							last_r = col.x;
							last_g = col.y;
							last_b = col.z;
							last_alpha = alpha;
							dL_dalpha = ((col.x - rec_r) * gr + (col.y - rec_g) * gg + (col.z - rec_b) * gb) * T -
										T_final * inv_1ma * dL_dTf;
						}
						if constexpr (S > 0) {
							dL_dalpha += T * (dot[u] - behind_dot);
							behind_dot = alpha * dot[u] + (1.0f - alpha) * behind_dot;
						}
					}
					// A clamped alpha no longer depends on the gaussian (backward.cu:126-135).
					const float sg = (contributes && raw[u] <= HDS_MAX_ALPHA) ? G[u] * dL_dalpha : 0.0f;
					s_rows[q * kRowStride + lane] = hds_split_pack(sg);
					w_rows[q * kRowStride + lane] = hds_split_pack(w);
					if (hds_ballot(contributes)) active |= 1u << q;
				}
			}
			if (!active) continue;
			for (int q = count; q < kGroup; q++) {
				s_rows[q * kRowStride + lane] = 0u;
				w_rows[q * kRowStride + lane] = 0u;
			}
			hds_wave_fence();

			// A operands over the 16 positions: lane = (position lane & 15, pixels 32pk + 8(lane >> 4) + 0..7).
			hds_bf16x8 wa_hi[2], wa_lo[2], sa_hi[2], sa_lo[2];
#pragma unroll
			for (int pk = 0; pk < 2; pk++) {
				const int off = (lane & 15) * kRowStride + 32 * pk + 8 * (lane >> 4);
				{
					const uint4 d0 = *reinterpret_cast<const uint4*>(w_rows + off);
					const uint4 d1 = *reinterpret_cast<const uint4*>(w_rows + off + 4);
					const uint32_t d[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
					hds_unpack8(d, wa_hi[pk], wa_lo[pk]);
				}
				{
					const uint4 d0 = *reinterpret_cast<const uint4*>(s_rows + off);
					const uint4 d1 = *reinterpret_cast<const uint4*>(s_rows + off + 4);
					const uint32_t d[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
					hds_unpack8(d, sa_hi[pk], sa_lo[pk]);
				}
			}
			// Pixel moments of s (columns 0-5) and colour sums of w (columns 6-8).
			{
				hds_f32x4 ms = {0.0f, 0.0f, 0.0f, 0.0f}, mw = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
				for (int pk = 0; pk < 2; pk++) {
					ms = hds_mfma_split(sa_hi[pk], sa_lo[pk], p_hi[pk], p_lo[pk], ms);
					if (do_rgb) mw = hds_mfma_split(wa_hi[pk], wa_lo[pk], p_hi[pk], p_lo[pk], mw);
				}
				const int colj = lane & 15;
#pragma unroll
				for (int i = 0; i < 4; i++) {
					const int q = 4 * (lane >> 4) + i;
					if (colj < 6) mom[q * 16 + colj] = ms[i];
					else if (colj < 9) mom[q * 16 + colj] = mw[i];
				}
			}
			if constexpr (S > 0) {
				if (want_dF) {
					// D rows = positions 4(lane >> 4) + i, column = channel 16n + (lane & 15).
					int gid4[4];
#pragma unroll
					for (int i = 0; i < 4; i++) {
						const int q = 4 * (lane >> 4) + i;
						gid4[i] = ((active >> q) & 1u) ? s_gid[min(slots[q], kBatch - 1)] : -1;
					}
#pragma unroll
					for (int n = 0; n < kNcb; n++) {
						hds_f32x4 gacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
						for (int pk = 0; pk < 2; pk++) gacc = hds_mfma_split(wa_hi[pk], wa_lo[pk], gb_hi[pk][n], gb_lo[pk][n], gacc);
						const int c = c0 + 16 * n + (lane & 15);
#pragma unroll
						for (int i = 0; i < 4; i++)
							if (gid4[i] >= 0) atomicAdd(&a.grad_features[(int64_t)gid4[i] * a.channels + c], gacc[i]);
					}
				}
			}
			hds_wave_fence();
			// One lane per gaussian: moments about the block centre -> gradients, then the atomics.
			if (lane < count && ((active >> lane) & 1u)) {
				const int sl = slots[lane];
				const int gid = s_gid[sl];
				const float2 mn = s_mean[sl];
				const float4 co = s_conic[sl];
				const float* mq = mom + lane * 16;
				const float m00 = mq[0], m10 = mq[1], m01 = mq[2], m20 = mq[3], m11 = mq[4], m02 = mq[5];
				const float mx = mn.x - centre_x, my = mn.y - centre_y;
				const float sx = m10 - mx * m00, sy = m01 - my * m00;
				const float sxx = m20 - 2.0f * mx * m10 + mx * mx * m00;
				const float sxy = m11 - mx * m01 - my * m10 + mx * my * m00;
				const float syy = m02 - 2.0f * my * m01 + my * my * m00;
				atomicAdd(&a.grad_opacities[gid], m00);
				atomicAdd(&a.grad_means2D[gid * 2 + 0], co.w * (co.x * sx + co.y * sy));
				atomicAdd(&a.grad_means2D[gid * 2 + 1], co.w * (co.y * sx + co.z * sy));
				atomicAdd(&a.grad_conics[gid * 3 + 0], -0.5f * co.w * sxx);
				atomicAdd(&a.grad_conics[gid * 3 + 1], -co.w * sxy);
				atomicAdd(&a.grad_conics[gid * 3 + 2], -0.5f * co.w * syy);
				if (do_rgb) {
					atomicAdd(&a.grad_colors[gid * 3 + 0], mq[6]);
					atomicAdd(&a.grad_colors[gid * 3 + 1], mq[7]);
					atomicAdd(&a.grad_colors[gid * 3 + 2], mq[8]);
				}
			}
			hds_wave_fence();
		}
	}
}

template <int S, bool RGB>
int launch(const BackwardArgs& a, int num_tiles, int slices, hipStream_t s) {
	render_backward_kernel<S, RGB><<<dim3((unsigned)num_tiles, (unsigned)slices), 256, 0, s>>>(a);
	return hds_check_launch(RGB ? (S > 0 ? "render_backward_rgb_features" : "render_backward_rgb")
								: "render_backward_features",
							s);
}

__global__ __launch_bounds__(256) void zero_kernel(float* __restrict__ p, int64_t count) {
	const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
	if (i < count) p[i] = 0.0f;
}

int zero(float* p, int64_t count, hipStream_t s) {
	if (!p || count == 0) return HDS_OK;
	zero_kernel<<<hds_blocks(count, 256), 256, 0, s>>>(p, count);
	return hds_check_launch("zero_gradients", s);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int render_backward(bool zero_outputs, int64_t n, int width, int height, int channels, int slice_width,
								   const int32_t* tile_ranges, const int32_t* values_sorted, int64_t num_pairs,
								   const float* means2D, const float* conic4, const float* color_opacity4,
								   const float* background, const float* final_T, const int32_t* n_contrib,
								   const float* grad_image, const float* features, const float* grad_feature_image,
								   float* grad_means2D, float* grad_conics, float* grad_colors, float* grad_opacities,
								   float* grad_features, hds_stream_t stream) {
	HDS_REQUIRE(width > 0 && height > 0, "render_backward: image size %dx%d must be positive", width, height);
	HDS_REQUIRE(n >= 0, "render_backward: negative gaussian count");
	HDS_REQUIRE(tile_ranges && final_T && n_contrib && (n == 0 || (grad_means2D && grad_conics && grad_opacities)),
				"render_backward: null pointer argument");
	const bool rgb = grad_image != nullptr;
	const bool feats = features != nullptr;
	HDS_REQUIRE(rgb || feats, "render_backward: neither grad_image nor features given");
	HDS_REQUIRE(!rgb || n == 0 || (grad_colors && background && color_opacity4), "render_backward: RGB term needs colors / background");
	if (feats) {
		HDS_REQUIRE(channels == 32 || channels == 64 || channels == 128 || channels == 256 || channels == 512,
					"features must have 32, 64, 128, 256 or 512 channels, got %d", channels);
		HDS_REQUIRE(grad_feature_image, "render_backward: features given without grad_feature_image");
		HDS_REQUIRE((slice_width == 32 || slice_width == 64 || slice_width == 128) && slice_width <= channels &&
						channels % slice_width == 0,
					"no feature backward for %d channels in slices of %d", channels, slice_width);
		HDS_REQUIRE(aligned16(features) && aligned16(grad_feature_image), "render_backward: features must be 16-byte aligned");
	}
	HDS_REQUIRE(aligned16(conic4) && (!color_opacity4 || aligned16(color_opacity4)), "render_backward: misaligned conic4");
	hipStream_t s = (hipStream_t)stream;
	if (zero_outputs) {
		int st;
		if ((st = zero(grad_means2D, 2 * n, s)) != HDS_OK) return st;
		if ((st = zero(grad_conics, 3 * n, s)) != HDS_OK) return st;
		if ((st = zero(grad_opacities, n, s)) != HDS_OK) return st;
		if (grad_colors && (st = zero(grad_colors, 3 * n, s)) != HDS_OK) return st;
		if (feats && grad_features && (st = zero(grad_features, (int64_t)channels * n, s)) != HDS_OK) return st;
	}
	if (n == 0 || num_pairs == 0) return HDS_OK;

	const int tiles_x = (width + HDS_TILE - 1) / HDS_TILE, tiles_y = (height + HDS_TILE - 1) / HDS_TILE;
	const int num_tiles = tiles_x * tiles_y;
	BackwardArgs a{width,
				   height,
				   tiles_x,
				   feats ? channels : 0,
				   reinterpret_cast<const int2*>(tile_ranges),
				   values_sorted,
				   reinterpret_cast<const float2*>(means2D),
				   reinterpret_cast<const float4*>(conic4),
				   reinterpret_cast<const float4*>(color_opacity4),
				   background,
				   final_T,
				   n_contrib,
				   grad_image,
				   features,
				   grad_feature_image,
				   grad_means2D,
				   grad_conics,
				   grad_colors,
				   grad_opacities,
				   feats ? grad_features : nullptr};
	if (!feats) return launch<0, true>(a, num_tiles, 1, s);
	const int slices = channels / slice_width;
	switch (slice_width) {
		case 32: return rgb ? launch<32, true>(a, num_tiles, slices, s) : launch<32, false>(a, num_tiles, slices, s);
		case 64: return rgb ? launch<64, true>(a, num_tiles, slices, s) : launch<64, false>(a, num_tiles, slices, s);
		default: return rgb ? launch<128, true>(a, num_tiles, slices, s) : launch<128, false>(a, num_tiles, slices, s);
	}
}

}  // namespace

#define HDS_BACKWARD_ARGS                                                                                     \
	int64_t n, int width, int height, int channels, int slice_width, const int32_t *tile_ranges,               \
		const int32_t *values_sorted, int64_t num_pairs, const float *means2D, const float *conic4,             \
		const float *color_opacity4, const float *background, const float *final_T, const int32_t *n_contrib,   \
		const float *grad_image, const float *features, const float *grad_feature_image, float *grad_means2D,   \
		float *grad_conics, float *grad_colors, float *grad_opacities, float *grad_features, hds_stream_t stream
#define HDS_BACKWARD_PASS                                                                                      \
	n, width, height, channels, slice_width, tile_ranges, values_sorted, num_pairs, means2D, conic4,            \
		color_opacity4, background, final_T, n_contrib, grad_image, features, grad_feature_image, grad_means2D, \
		grad_conics, grad_colors, grad_opacities, grad_features, stream

extern "C" int hds_render_backward(HDS_BACKWARD_ARGS) { return render_backward(true, HDS_BACKWARD_PASS); }

extern "C" int hds_render_backward_accumulate(HDS_BACKWARD_ARGS) { return render_backward(false, HDS_BACKWARD_PASS); }
