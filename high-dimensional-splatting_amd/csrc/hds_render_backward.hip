// Replay of the blend for the gradients: two kernels over the same tile lists.
//
// Layout as in the forward: work-group = tile x slice of S channels, wave = 8x8 pixel block,
// lane = pixel, and a wave only visits the gaussians whose culling box reaches its block.
//
// backward_geometry_kernel walks each tile's list back to front from every pixel's final T and
// n_contrib (backward.cu:53-163, features.cu:419-541):
//   T <- T / (1 - alpha);  RGB: accum_rec recurrence, dL/dalpha = (c - rec).g T - T_f/(1-a) bg.g;
//   features: dL/dalpha += T (dot - behind_dot), behind_dot <- a dot + (1 - a) behind_dot,
//   with dot = f . dL/dF[pixel];  geometry gradients only where the raw alpha <= 0.99.
// RGB and feature terms go into one dL/dalpha per pixel (the reference sums two kernels' outputs,
// rasterizer/__init__.py:160-162). Slices add their partial dot terms linearly through the same
// atomics (features.cu:348-349). Per group of up to 16 gaussians the wave does, in split-bf16:
//   dot[g][px]  = sum_c F[g][c] dL/dF[px][c]   (16x16x32 MFMA, dL/dF^T held in VGPRs; a 4x4
//                                                 lane-group transpose leaves each lane its pixel)
//   mom[j][g]   = sum_px P[px][j] s[px][g]      (s = G dL/dalpha, P = 1, x, y, x^2, xy, y^2)
//   rgb[c][g]   = sum_px dL/dRGB[px][c] w[px][g] (w = alpha T)
// The six geometry gradients are polynomials in the pixel offsets d = px - mean, so they follow
// from the six pixel moments of s about the block centre: dopac = sum s, dmean = op Q sum s d,
// dconic = -op (sum s dx^2 / 2, sum s dx dy, sum s dy^2 / 2). One lane per gaussian issues them.
//
// backward_features_kernel replays the blend front to back with the forward's own arithmetic, so
// its weights w = alpha T equal the forward's bit for bit, and contracts them with dL/dF over the
// block's pixels, dF[g][c] += sum_px w[px][g] dL/dF[px][c] (features.cu:486-513), on 32x32x16 MFMA
// in groups of 32 gaussians that run across batches. dL/dF (K = pixels) stays in VGPRs; the weights
// are written once to LDS as rows per gaussian and read back as the A operand. The result of each
// lane is 32 consecutive channels of one gaussian, so the atomics are whole cache lines and a
// gaussian's gradient row sees one atomic per 8x8 block it touches.
#include <algorithm>

#include "hds_internal.h"
#include "hds_rasterizer.h"
#include "hds_stage.h"

namespace {

constexpr int kBatch = 64;
constexpr int kIlp = 4;         // positions whose alpha is evaluated together
constexpr int kGeoGroup = 16;   // gaussians per geometry group
constexpr int kFeatGroup = 32;  // gaussians per feature-gradient group
constexpr int kRowStride = 68;  // words per [position][pixel] row, 16-byte aligned

struct BackwardArgs {
	int width, height, tiles_x, channels, num_tiles;
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

__device__ inline float hds_swap16_from_odd(float v) {
	// Lanes of even 16-lane rows receive v of the row above them.
	const uint32_t u = hds_swap_operand(v);
	const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
	return __builtin_bit_cast(float, (uint32_t)r[1]);
}

// Tile-wide maximum of n_contrib: nothing past the deepest contributor can matter (backward.cu:53-60).
__device__ inline int tile_max_last(int last, int* s_max_last) {
	if (threadIdx.x == 0) *s_max_last = 0;
	__syncthreads();
	if (last > 0) atomicMax(s_max_last, last);
	__syncthreads();
	return *s_max_last;
}

template <int S, bool RGB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void backward_geometry_kernel(const BackwardArgs a) {
	constexpr int kKc = S > 0 ? S / 32 : 1;       // K steps of the dot over channels
	// Per gaussian slot: the six pixel moments of s of each wave's block, then the colour gradient.
	constexpr int kAccStride = 4 * 6 + 3;
	// Gaussians per batch: 32 at S >= 64 so that two work-groups fit a CU's LDS; positions whose
	// alphas are evaluated together: 2 at S = 128, where dL/dF takes half the registers.
	constexpr int kGB = S >= 64 ? 32 : kBatch;
	constexpr int kGeoIlp = S >= 128 ? 2 : kIlp;
	constexpr int kRows = S > 0 ? (kGB + 1) * S : 1;

	// Gaussian ids of batches b, b+1, b+2 (slot b % 3); records and feature rows of the batch being
	// walked and of the next one (the pipeline of render_forward_kernel). Feature rows are raw fp32
	// with their 16-byte chunks XOR-swizzled by row; row kGB stays zero (positions past the end of a
	// partial group point at it).
	__shared__ int s_gid[3][kGB];
	__shared__ HdsHeaderSlot<kGB, RGB> s_hdr0, s_hdr1;
	// Sums of batch b (slot b & 1) per gaussian: for each wave, the moments sum s {1, x, y, x^2, xy,
	// y^2} about its block centre, then sum w dL/dRGB. One lane per gaussian turns them into
	// gradients and adds those to HBM once per tile.
	__shared__ float s_acc[2][kGB * kAccStride];
	__shared__ __attribute__((aligned(16))) float s_feat0[kRows];
	__shared__ __attribute__((aligned(16))) float s_feat1[kRows];
	__shared__ int s_slot[4][kGeoGroup];
	__shared__ int s_max_last;
	// Per wave: s and w of the group as rows per position (the B operands of the moment MFMAs).
	__shared__ __attribute__((aligned(16))) float s_tr[4][2][kGeoGroup * kRowStride];

	const int tile = hds_xcd_tile(blockIdx.x, a.tiles_x, a.num_tiles);
	if (tile < 0) return;
	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const int slice = blockIdx.y;
	const int tx0 = (tile % a.tiles_x) * HDS_TILE, ty0 = (tile / a.tiles_x) * HDS_TILE;
	const int wx0 = tx0 + (wave & 1) * 8, wy0 = ty0 + (wave >> 1) * 8;
	const int px = wx0 + (lane & 7), py = wy0 + (lane >> 3);
	const bool inside = px < a.width && py < a.height;
	const int64_t pix = (int64_t)py * a.width + px;
	const float fx = (float)px + 0.5f, fy = (float)py + 0.5f;
	const float rx0 = (float)wx0 + 0.5f, rx1 = (float)wx0 + 7.5f;
	const float ry0 = (float)wy0 + 0.5f, ry1 = (float)wy0 + 7.5f;
	const int c0 = slice * S;
	const bool do_rgb = RGB && slice == 0;

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
	// One recurrence serves RGB and features: with dot = f . dL/dF + c . dL/dRGB, the reference's
	// RGB term (c - rec) . g T (rec = colour blended behind, backward.cu:113-122) is
	// T (c . g - rec . g), and rec . g obeys the same recurrence as the features' behind_dot.
	float behind_dot = 0.0f;

	// P^T, the A operand of the moment MFMAs: row lane % 16 = column j of P, k = pixels
	// 32kk + 8(lane / 16) + 0..7. Rows 0-5: 1, x, y, x^2, xy, y^2 about the block centre (exact in
	// bf16); rows 8-10: the pixel's dL/dRGB (split); other rows zero.
	hds_bf16x8 pt_hi[2], pt_lo[2];
	{
		const int row = lane & 15;
		// The 16 dL/dRGB values this lane contributes, loaded together (index 0 where unused).
		float g[2][8];
#pragma unroll
		for (int kk = 0; kk < 2; kk++)
#pragma unroll
			for (int j = 0; j < 8; j++) g[kk][j] = 0.0f;
		if (do_rgb) {
#pragma unroll
			for (int kk = 0; kk < 2; kk++)
#pragma unroll
				for (int j = 0; j < 8; j++) {
					const int p = 32 * kk + 8 * (lane >> 4) + j;
					const int x = wx0 + (p & 7), y = wy0 + (p >> 3);
					const bool use = row >= 8 && row < 11 && x < a.width && y < a.height;
					const float v = a.grad_image[use ? ((int64_t)y * a.width + x) * 3 + (row - 8) : 0];
					g[kk][j] = use ? v : 0.0f;
				}
		}
#pragma unroll
		for (int kk = 0; kk < 2; kk++) {
			float v[8];
#pragma unroll
			for (int j = 0; j < 8; j++) {
				const int p = 32 * kk + 8 * (lane >> 4) + j;
				const float xl = (float)(p & 7) - 3.5f, yl = (float)(p >> 3) - 3.5f;
				v[j] = row == 0 ? 1.0f : row == 1 ? xl : row == 2 ? yl : row == 3 ? xl * xl : row == 4 ? xl * yl
					 : row == 5 ? yl * yl : g[kk][j];
			}
			hds_split8(v, pt_hi[kk], pt_lo[kk]);
		}
	}

	// dL/dF^T, the B operand of the dot MFMAs, for pixel blocks n = 0..3:
	// B[k = 8(lane / 16) + j][col = lane % 16] = dL/dF[pixel 16n + lane % 16][channel c0 + 32kk + 8(lane / 16) + j].
	hds_bf16x8 gb_hi[4][kKc], gb_lo[4][kKc];
	if constexpr (S > 0) {
#pragma unroll
		for (int n = 0; n < 4; n++) {
			const int p = 16 * n + (lane & 15);
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
				uint32_t h[4], l[4];
				hds_split_pair(v0.x, v0.y, h[0], l[0]);
				hds_split_pair(v0.z, v0.w, h[1], l[1]);
				hds_split_pair(v1.x, v1.y, h[2], l[2]);
				hds_split_pair(v1.z, v1.w, h[3], l[3]);
				gb_hi[n][kk] = __builtin_bit_cast(hds_bf16x8, hds_u32x4{h[0], h[1], h[2], h[3]});
				gb_lo[n][kk] = __builtin_bit_cast(hds_bf16x8, hds_u32x4{l[0], l[1], l[2], l[3]});
			}
		}
		for (int i = tid; i < S; i += blockDim.x) s_feat0[kGB * S + i] = s_feat1[kGB * S + i] = 0.0f;
	}

	const int2 range = a.ranges[tile];
	const int num = min(range.y - range.x, tile_max_last(last, &s_max_last));
	const int wave_last = hds_wave_max(last);
	float* tr_s = s_tr[wave][0];
	float* tr_w = s_tr[wave][1];
	int* slots = s_slot[wave];

	// Batches run back to front: batch b holds list entries [start(b), start(b) + count(b)).
	const int num_batches = (num + kGB - 1) / kGB;
	auto batch_count = [&](int b) { return b < num_batches ? min(kGB, num - b * kGB) : 0; };
	auto batch_start_of = [&](int b) { return num - b * kGB - batch_count(b); };
	if (num_batches == 0) return;
	{
		// Prologue: gids of batches 0 and 1, then batch 0 staged synchronously.
		const int cnt0 = batch_count(0), cnt1 = batch_count(1);
		if (tid < cnt0) s_gid[0][tid] = a.values[range.x + batch_start_of(0) + tid];
		if (tid < cnt1) s_gid[1][tid] = a.values[range.x + batch_start_of(1) + tid];
		for (int i = tid; i < 2 * kGB * kAccStride; i += blockDim.x) (&s_acc[0][0])[i] = 0.0f;
		__syncthreads();
		hds_stage_headers_async<kGB, RGB>(s_hdr0, a.means2D, a.conic4, a.color_op4, s_gid[0], cnt0, tid);
		if constexpr (S > 0) hds_stage_rows_async<S, true, kGB>(s_feat0, a.features, a.channels, c0, s_gid[0], cnt0, tid);
		hds_wait_vmem();
		__syncthreads();
	}

	// Turns batch b's sums into gradients and adds them to HBM, one lane per gaussian, and clears the
	// slot for b + 2 (backward.cu:136-160 in moment form: with d = pixel - mean, dopacity = sum s,
	// dmean = op Q sum s d, dconic = -op (sum s dx^2 / 2, sum s dx dy, sum s dy^2 / 2), each wave's
	// moments shifted from its block centre to the mean). Runs at the end of the step that follows
	// batch b (after the barrier that closed b, before the gids of b + 3 replace those of b in slot
	// b % 3); mean and conic come from HBM, loaded at the start of that step (prefetch_geometry).
	// The work is spread over the whole work-group: thread t takes gaussian slot t / 4 and the
	// moments of wave t % 4, and the four partial gradients of a slot are summed across adjacent
	// lanes. Mean and conic come from HBM, loaded at the start of that step (prefetch_geometry).
	const int f_slot = tid >> 2, f_wave = tid & 3;
	// The gaussian id is read here too: the flush runs beside the stores of the gids of b + 3
	// into the same slot by other threads.
	int pf_gid = 0;
	float2 pf_mean = make_float2(0.0f, 0.0f);
	float4 pf_conic = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
	auto prefetch_geometry = [&](int b) {
		if (f_slot < batch_count(b)) {
			pf_gid = s_gid[b % 3][f_slot];
			pf_mean = a.means2D[pf_gid];
			pf_conic = a.conic4[pf_gid];
		}
	};
	auto flush_gradients = [&](int b) {
		const int cnt = batch_count(b);
		if (f_slot >= ((cnt + 15) & ~15)) return;  // whole 16-slot (64-lane) groups stay converged
		const bool valid = f_slot < cnt;
		float* g = s_acc[b & 1] + f_slot * kAccStride;
		float m[6];
#pragma unroll
		for (int k = 0; k < 6; k++) {
			m[k] = valid ? g[6 * f_wave + k] : 0.0f;
			if (valid) g[6 * f_wave + k] = 0.0f;
		}
		float rgb = 0.0f;
		if (valid && f_wave < 3) {
			rgb = g[24 + f_wave];
			g[24 + f_wave] = 0.0f;
		}
		const float4 co = pf_conic;
		const float mx = pf_mean.x - ((float)(tx0 + (f_wave & 1) * 8) + 4.0f);
		const float my = pf_mean.y - ((float)(ty0 + (f_wave >> 1) * 8) + 4.0f);
		const float sx = m[1] - mx * m[0], sy = m[2] - my * m[0];
		const float sxx = m[3] - 2.0f * mx * m[1] + mx * mx * m[0];
		const float sxy = m[4] - mx * m[2] - my * m[1] + mx * my * m[0];
		const float syy = m[5] - 2.0f * my * m[2] + my * my * m[0];
		float d[6] = {m[0], co.w * (co.x * sx + co.y * sy), co.w * (co.y * sx + co.z * sy), -0.5f * co.w * sxx,
					  -co.w * sxy, -0.5f * co.w * syy};
#pragma unroll
		for (int k = 0; k < 6; k++) {
			d[k] += hds_shfl_xor(d[k], 1);
			d[k] += hds_shfl_xor(d[k], 2);
		}
		if (!valid) return;
		const int gid = pf_gid;
		if (f_wave == 0 && (d[0] != 0.0f || d[1] != 0.0f || d[2] != 0.0f || d[3] != 0.0f || d[4] != 0.0f || d[5] != 0.0f)) {
			atomicAdd(&a.grad_opacities[gid], d[0]);
			atomicAdd(&a.grad_means2D[gid * 2 + 0], d[1]);
			atomicAdd(&a.grad_means2D[gid * 2 + 1], d[2]);
			atomicAdd(&a.grad_conics[gid * 3 + 0], d[3]);
			atomicAdd(&a.grad_conics[gid * 3 + 1], d[4]);
			atomicAdd(&a.grad_conics[gid * 3 + 2], d[5]);
		}
		if (do_rgb && f_wave < 3 && rgb != 0.0f) atomicAdd(&a.grad_colors[gid * 3 + f_wave], rgb);
	};

	// One batch: stage b+1, read the gids of b+2, walk b.
	auto step = [&](int b, const HdsHeaderSlot<kGB, RGB>& h, const float* feat, HdsHeaderSlot<kGB, RGB>& h_next,
					float* feat_next) {
		const int cnt = batch_count(b), cnt1 = batch_count(b + 1), cnt2 = batch_count(b + 2);
		const int batch_start = batch_start_of(b);
		float* acc = s_acc[b & 1];
		if (b > 0) prefetch_geometry(b - 1);
		int g2 = 0;
		if (tid < cnt2) g2 = a.values[range.x + batch_start_of(b + 2) + tid];
		const int* gid_next = s_gid[(b + 1) % 3];
		if (cnt1 > 0) {
			hds_stage_headers_async<kGB, RGB>(h_next, a.means2D, a.conic4, a.color_op4, gid_next, cnt1, tid);
			if constexpr (S > 0)
				hds_stage_rows_async<S, true, kGB>(feat_next, a.features, a.channels, c0, gid_next, cnt1, tid);
		}

		if (batch_start < wave_last) {
			bool box_hit = false;
			if (lane < cnt && batch_start + lane < wave_last) {
				box_hit = hds_block_reach(make_float2(h.mx[lane], h.my[lane]), h.conic[lane], rx0, rx1, ry0, ry1);
			}
			uint64_t hits = hds_ballot(box_hit);
			while (hits) {
				// Next group: the (up to) 16 deepest hits. Hit bit b is position (number of hits above b).
				const int count = min(kGeoGroup, __builtin_popcountll(hits));
				{
					const bool set = (hits >> lane) & 1ull;
					const int rank = __builtin_popcountll((hits >> lane) >> 1);
					const bool take = set && rank < kGeoGroup;
					if (take) slots[rank] = lane;
					if (lane >= count && lane < kGeoGroup) slots[lane] = kGB;
					hits &= ~hds_ballot(take);
				}
				hds_wave_fence();

				// dot[position 4h + i][own pixel] = dot[h][i] (zero without features).
				float dot[4][4];
	#pragma unroll
				for (int h = 0; h < 4; h++)
	#pragma unroll
					for (int i = 0; i < 4; i++) dot[h][i] = 0.0f;
				if constexpr (S > 0) {
					// A = F: row lane % 16 = position, k = channels 32kk + 8(lane / 16) + 0..7.
					const int frow_idx = slots[lane & 15];
					const float* frow = feat + frow_idx * S;
					hds_f32x4 X[4];
	#pragma unroll
					for (int n = 0; n < 4; n++) X[n] = hds_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
	#pragma unroll
					for (int kk = 0; kk < kKc; kk++) {
						// Logical chunks 8kk + 2(lane / 16) and the next one of the (swizzled) row.
						const int lc = 8 * kk + 2 * (lane >> 4);
						const float4 f0 = *reinterpret_cast<const float4*>(frow + 4 * hds_stage_chunk<true, S / 4>(lc, frow_idx));
						const float4 f1 = *reinterpret_cast<const float4*>(frow + 4 * hds_stage_chunk<true, S / 4>(lc + 1, frow_idx));
						const float v[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
						hds_bf16x8 f_hi, f_lo;
						hds_split8(v, f_hi, f_lo);
	#pragma unroll
						for (int n = 0; n < 4; n++) X[n] = hds_mfma_split(f_hi, f_lo, gb_hi[n][kk], gb_lo[n][kk], X[n]);
					}
					// X[n] of lane group h holds positions 4h + 0..3 of pixel 16n + lane % 16: transpose the
					// 4x4 (group, block) arrangement, first across halves, then across neighbouring rows.
					uint32_t t[4][4];
	#pragma unroll
					for (int n = 0; n < 4; n++)
	#pragma unroll
						for (int i = 0; i < 4; i++) t[n][i] = hds_swap_operand(X[n][i]);
	#pragma unroll
					for (int i = 0; i < 4; i++) {
	#pragma unroll
						for (int n = 0; n < 2; n++) {
							const auto r = __builtin_amdgcn_permlane32_swap(t[n][i], t[n + 2][i], false, false);
							t[n][i] = r[0];
							t[n + 2][i] = r[1];
						}
	#pragma unroll
						for (int n = 0; n < 4; n += 2) {
							const auto r = __builtin_amdgcn_permlane16_swap(t[n][i], t[n + 1][i], false, false);
							t[n][i] = r[0];
							t[n + 1][i] = r[1];
						}
					}
	#pragma unroll
					for (int h = 0; h < 4; h++)
	#pragma unroll
						for (int i = 0; i < 4; i++) dot[h][i] = __builtin_bit_cast(float, t[h][i]);
				}

				// Back-to-front replay of the group, kIlp positions at a time: their alphas are
				// independent, only T and the behind-sums chain through them.
				uint32_t active = 0;
	#pragma unroll
				for (int q0 = 0; q0 < kGeoGroup; q0 += kGeoIlp) {
					// Unrolled with no early exit, so every dot[][] index stays static.
					if (q0 < count) {
						int slot[kGeoIlp];
						float raw[kGeoIlp], G[kGeoIlp];
						float4 col[kGeoIlp];
		#pragma unroll
						for (int u = 0; u < kGeoIlp; u++) {
							slot[u] = slots[q0 + u];
							const int sl = min(slot[u], kGB - 1);
							float dx, dy;
							raw[u] = hds_raw_alpha(fx, fy, make_float2(h.mx[sl], h.my[sl]), h.conic[sl], G[u], dx, dy);
							// Read with the geometry: a read under the replay branch would stall on LDS latency.
							if constexpr (RGB) col[u] = h.color[sl];
						}
		#pragma unroll
						for (int u = 0; u < kGeoIlp; u++) {
							const int q = q0 + u;
							const float alpha = fminf(HDS_MAX_ALPHA, raw[u]);
							const bool contributes = q < count && batch_start + slot[u] < last && alpha >= HDS_MIN_ALPHA;
							float dL_dalpha = 0.0f, w = 0.0f;
							if (contributes) {
								float d = 0.0f;
								if constexpr (S > 0) d = dot[q >> 2][q & 3];
								if (do_rgb) d += col[u].x * gr + col[u].y * gg + col[u].z * gb;
								const float inv_1ma = __builtin_amdgcn_rcpf(1.0f - alpha);
								T *= inv_1ma;
								w = alpha * T;
								dL_dalpha = T * (d - behind_dot);
								if (do_rgb) dL_dalpha -= T_final * inv_1ma * dL_dTf;
								behind_dot = alpha * d + (1.0f - alpha) * behind_dot;
							}
							// A clamped alpha no longer depends on the gaussian (backward.cu:126-135).
							tr_s[q * kRowStride + lane] = (contributes && raw[u] <= HDS_MAX_ALPHA) ? G[u] * dL_dalpha : 0.0f;
							if (do_rgb) tr_w[q * kRowStride + lane] = w;
							if (hds_ballot(contributes)) active |= 1u << q;
						}
					}
				}
				if (!active) continue;
				// Rows of positions past count are stale: they only reach their own output columns,
				// which nobody reads.
				hds_wave_fence();

				// mom[j][position] = sum_px P^T[j][px] s[px][position]; B lane = (pixels 32kk + 8(lane / 16)
				// + 0..7, position lane % 16). D: row 4(lane / 16) + i = j, column lane % 16 = position.
				hds_f32x4 ms = {0.0f, 0.0f, 0.0f, 0.0f}, mw = {0.0f, 0.0f, 0.0f, 0.0f};
	#pragma unroll
				for (int kk = 0; kk < 2; kk++) {
					const int off = (lane & 15) * kRowStride + 32 * kk + 8 * (lane >> 4);
					{
						const hds_u32x4 d0 = hds_lds_read128(reinterpret_cast<const uint32_t*>(tr_s + off));
						const hds_u32x4 d1 = hds_lds_read128(reinterpret_cast<const uint32_t*>(tr_s + off + 4));
						const float v[8] = {hds_u2f(d0.x), hds_u2f(d0.y), hds_u2f(d0.z), hds_u2f(d0.w),
											hds_u2f(d1.x), hds_u2f(d1.y), hds_u2f(d1.z), hds_u2f(d1.w)};
						hds_bf16x8 b_hi, b_lo;
						hds_split8(v, b_hi, b_lo);
						// Only rows 0-5 of ms are read, and P is exact in bf16 there (pt_lo = 0): the
						// lo x hi product adds exact zeros, so two MFMAs give the same bits as three.
						ms = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pt_hi[kk], b_lo, ms, 0, 0, 0);
						ms = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pt_hi[kk], b_hi, ms, 0, 0, 0);
					}
					if (do_rgb) {
						const hds_u32x4 d0 = hds_lds_read128(reinterpret_cast<const uint32_t*>(tr_w + off));
						const hds_u32x4 d1 = hds_lds_read128(reinterpret_cast<const uint32_t*>(tr_w + off + 4));
						const float v[8] = {hds_u2f(d0.x), hds_u2f(d0.y), hds_u2f(d0.z), hds_u2f(d0.w),
											hds_u2f(d1.x), hds_u2f(d1.y), hds_u2f(d1.z), hds_u2f(d1.w)};
						hds_bf16x8 b_hi, b_lo;
						hds_split8(v, b_hi, b_lo);
						mw = hds_mfma_split(pt_hi[kk], pt_lo[kk], b_hi, b_lo, mw);
					}
				}
				// Rows 4, 5 (xy, y^2) live in lane group 1; bring them to group 0 beside rows 0-3.
				const float m11 = hds_swap16_from_odd(ms[0]);
				const float m02 = hds_swap16_from_odd(ms[1]);
				const int q = lane & 15;
				const bool mine = q < count && ((active >> q) & 1u);
				if (lane < 16 && mine) {
					// This wave's moments about its block centre, summed per gaussian in LDS (the
					// flush turns them into gradients).
					float* g = acc + slots[q] * kAccStride + 6 * wave;
					atomicAdd(&g[0], ms[0]);
					atomicAdd(&g[1], ms[1]);
					atomicAdd(&g[2], ms[2]);
					atomicAdd(&g[3], ms[3]);
					atomicAdd(&g[4], m11);
					atomicAdd(&g[5], m02);
				}
				if (do_rgb && lane >= 32 && lane < 48 && mine) {
					// Rows 8-10: the colour gradients sum_px w dL/dRGB (backward.cu:112-118).
					float* g = acc + slots[q] * kAccStride + 24;
					atomicAdd(&g[0], mw[0]);
					atomicAdd(&g[1], mw[1]);
					atomicAdd(&g[2], mw[2]);
				}
				hds_wave_fence();
			}
		}

		if (b > 0) flush_gradients(b - 1);
		if (tid < cnt2) s_gid[(b + 2) % 3][tid] = g2;
		hds_wait_vmem();
		__syncthreads();
	};
	for (int b = 0; b < num_batches; b += 2) {
		step(b, s_hdr0, s_feat0, s_hdr1, s_feat1);
		if (b + 1 < num_batches) step(b + 1, s_hdr1, s_feat1, s_hdr0, s_feat0);
	}
	prefetch_geometry(num_batches - 1);
	flush_gradients(num_batches - 1);
}

// dF[position][c] += sum_px W[position][px] dL/dF[px][c] for one group of up to 32 positions, then
// one atomic per (position, channel). rows: W as [position][pixel] split-packed; gids: the gaussian
// of each of the wave's `used` rows (rows from `used` on are stale and skipped).
template <int S>
__device__ inline void flush_features(const hds_bf16x8 (&gb_hi)[4][S / 32], const hds_bf16x8 (&gb_lo)[4][S / 32],
									  const uint32_t* rows, const int* gids, int used, float* grad_features,
									  int channels_log2, int c0, int lane) {
	hds_wave_fence();
	// A = W: row lane % 32 = position, k = pixels 16kp + 8(lane / 32) + 0..7.
	hds_bf16x8 a_hi[4], a_lo[4];
#pragma unroll
	for (int kp = 0; kp < 4; kp++) {
		const uint32_t* r = rows + (lane & 31) * kRowStride + 16 * kp + 8 * (lane >> 5);
		const hds_u32x4 d0 = hds_lds_read128(r);
		const hds_u32x4 d1 = hds_lds_read128(r + 4);
		const uint32_t d[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
		hds_unpack8(d, a_hi[kp], a_lo[kp]);
	}
	// D rows = positions 8(i / 4) + 4(lane / 32) + i % 4: their gaussians, read once for all channel
	// blocks (a row's address is formed once; channel block cb is the atomic's constant offset).
	int gid[16];
#pragma unroll
	for (int g = 0; g < 4; g++) {
		const int r = 8 * g + 4 * (lane >> 5);
		const int4 v = *reinterpret_cast<const int4*>(gids + r);
		gid[4 * g + 0] = r + 0 < used ? v.x : -1;
		gid[4 * g + 1] = r + 1 < used ? v.y : -1;
		gid[4 * g + 2] = r + 2 < used ? v.z : -1;
		gid[4 * g + 3] = r + 3 < used ? v.w : -1;
	}
	float* const base = grad_features + c0 + (lane & 31);
#pragma unroll
	for (int cb = 0; cb < S / 32; cb++) {
		hds_f32x16 acc = {};
#pragma unroll
		for (int kp = 0; kp < 4; kp++) acc = hds_mfma32_split(a_hi[kp], a_lo[kp], gb_hi[kp][cb], gb_lo[kp][cb], acc);
#pragma unroll
		for (int i = 0; i < 16; i++)
			if (gid[i] >= 0) atomicAdd(base + ((uint64_t)(uint32_t)gid[i] << channels_log2) + 32 * cb, acc[i]);
	}
	hds_wave_fence();
}

template <int S>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(S >= 128 ? 2 : 3))) void backward_features_kernel(
	const BackwardArgs a) {
	constexpr int kNcb = S / 32;

	// Gaussian ids of batches b, b+1, b+2 (slot b % 3) and the records of the batch being walked and of
	// the next one (the pipeline of render_forward_kernel).
	__shared__ int s_gid[3][kBatch];
	__shared__ HdsHeaderSlot<kBatch, false> s_hdr0, s_hdr1;
	__shared__ __attribute__((aligned(16))) uint32_t s_w[4][kFeatGroup * kRowStride];
	__shared__ __attribute__((aligned(16))) int s_ggid[4][kFeatGroup];
	__shared__ int s_max_last;

	const int tile = hds_xcd_tile(blockIdx.x, a.tiles_x, a.num_tiles);
	if (tile < 0) return;
	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const int slice = blockIdx.y;
	const int tx0 = (tile % a.tiles_x) * HDS_TILE, ty0 = (tile / a.tiles_x) * HDS_TILE;
	const int wx0 = tx0 + (wave & 1) * 8, wy0 = ty0 + (wave >> 1) * 8;
	const int px = wx0 + (lane & 7), py = wy0 + (lane >> 3);
	const bool inside = px < a.width && py < a.height;
	const float fx = (float)px + 0.5f, fy = (float)py + 0.5f;
	const float rx0 = (float)wx0 + 0.5f, rx1 = (float)wx0 + 7.5f;
	const float ry0 = (float)wy0 + 0.5f, ry1 = (float)wy0 + 7.5f;
	const int c0 = slice * S;
	const int channels_log2 = 31 - __builtin_clz((unsigned)a.channels);  // a power of two (32-512)
	const int last = inside ? a.n_contrib[(int64_t)py * a.width + px] : 0;

	// dL/dF, the B operand with K = pixels, for pixel steps kp = 0..3:
	// B[k = 8(lane / 32) + j][col = lane % 32] = dL/dF[pixel 16kp + 8(lane / 32) + j][channel c0 + 32cb + lane % 32].
	hds_bf16x8 gb_hi[4][kNcb], gb_lo[4][kNcb];
#pragma unroll
	for (int kp = 0; kp < 4; kp++) {
		// The 8 pixels of this step: row 2 kp + lane / 32 of the block (zero outside the image).
		const int y = wy0 + 2 * kp + (lane >> 5);
		const float* src = a.grad_feature_image + (((int64_t)y * a.width + wx0) << channels_log2) + c0 + (lane & 31);
#pragma unroll
		for (int cb = 0; cb < kNcb; cb++) {
			float v[8];
#pragma unroll
			for (int j = 0; j < 8; j++) {
				v[j] = 0.0f;
				if (wx0 + j < a.width && y < a.height) v[j] = src[((int64_t)j << channels_log2) + 32 * cb];
			}
			uint32_t h[4], l[4];
#pragma unroll
			for (int i = 0; i < 4; i++) hds_split_pair(v[2 * i], v[2 * i + 1], h[i], l[i]);
			gb_hi[kp][cb] = __builtin_bit_cast(hds_bf16x8, hds_u32x4{h[0], h[1], h[2], h[3]});
			gb_lo[kp][cb] = __builtin_bit_cast(hds_bf16x8, hds_u32x4{l[0], l[1], l[2], l[3]});
		}
	}

	const int2 range = a.ranges[tile];
	const int num = min(range.y - range.x, tile_max_last(last, &s_max_last));
	const int wave_last = hds_wave_max(last);
	uint32_t* rows = s_w[wave];
	int* gids = s_ggid[wave];

	float T = 1.0f;
	int q = 0;  // filled positions of the wave's current group (wave-uniform)
	const int num_batches = (num + kBatch - 1) / kBatch;
	auto batch_count = [&](int b) { return b < num_batches ? min(kBatch, num - b * kBatch) : 0; };
	if (num_batches > 0) {
		// Prologue: gids of batches 0 and 1, then the records of batch 0.
		const int cnt0 = batch_count(0), cnt1 = batch_count(1);
		if (tid < cnt0) s_gid[0][tid] = a.values[range.x + tid];
		if (tid < cnt1) s_gid[1][tid] = a.values[range.x + kBatch + tid];
		__syncthreads();
		hds_stage_headers_async<kBatch, false>(s_hdr0, a.means2D, a.conic4, nullptr, s_gid[0], cnt0, tid);
		hds_wait_vmem();
		__syncthreads();
	}
	auto flush = [&]() {
		flush_features<S>(gb_hi, gb_lo, rows, gids, q, a.grad_features, channels_log2, c0, lane);
		q = 0;
	};
	// One batch: stage b+1, read the gids of b+2, walk b.
	auto step = [&](int b, const HdsHeaderSlot<kBatch, false>& h, HdsHeaderSlot<kBatch, false>& h_next) {
		const int cnt = batch_count(b), cnt1 = batch_count(b + 1), cnt2 = batch_count(b + 2);
		const int batch = b * kBatch;
		const int* bgid = s_gid[b % 3];
		int g2 = 0;
		if (tid < cnt2) g2 = a.values[range.x + (b + 2) * kBatch + tid];
		if (cnt1 > 0) hds_stage_headers_async<kBatch, false>(h_next, a.means2D, a.conic4, nullptr, s_gid[(b + 1) % 3], cnt1, tid);

		if (batch < wave_last) {
			bool box_hit = false;
			if (lane < cnt && batch + lane < wave_last) {
				box_hit = hds_block_reach(make_float2(h.mx[lane], h.my[lane]), h.conic[lane], rx0, rx1, ry0, ry1);
			}
			// Lane i holds the gaussian of batch slot i (read by the row bookkeeping below).
			const int slot_gid = lane < cnt ? bgid[lane] : -1;
			uint64_t hits = hds_ballot(box_hit);
			while (hits) {
				// Room for kIlp more rows; the group is flushed a little early rather than split.
				if (q > kFeatGroup - kIlp) flush();
				// The next (up to) kIlp hits in list order. All bookkeeping here is wave-uniform.
				int slot[kIlp];
				float alpha[kIlp];
				int take = 0;
#pragma unroll
				for (int u = 0; u < kIlp; u++) {
					slot[u] = kBatch - 1;
					if (hits) {
						slot[u] = __builtin_amdgcn_readfirstlane(__builtin_ctzll(hits));
						hits &= hits - 1;
						take = u + 1;
					}
					float G, dx, dy;
					alpha[u] = fminf(HDS_MAX_ALPHA, hds_raw_alpha(fx, fy, make_float2(h.mx[slot[u]], h.my[slot[u]]),
																  h.conic[slot[u]], G, dx, dy));
				}
#pragma unroll
				for (int u = 0; u < kIlp; u++) {
					// The forward's test, with its termination read from n_contrib.
					const bool contributes = u < take && batch + slot[u] < last && alpha[u] >= HDS_MIN_ALPHA;
					float w = 0.0f;
					if (contributes) {
						const float test_T = T * (1.0f - alpha[u]);
						w = alpha[u] * T;
						T = test_T;
					}
					// A gaussian no pixel of the block takes gets no row (and no atomics). Every lane
					// writes the row's gaussian id to the same word.
					if (hds_ballot(contributes) != 0) {
						rows[q * kRowStride + lane] = hds_split_pack(w);
						gids[q] = __builtin_amdgcn_readlane(slot_gid, slot[u]);
						q++;
					}
				}
			}
		}

		if (tid < cnt2) s_gid[(b + 2) % 3][tid] = g2;
		hds_wait_vmem();
		__syncthreads();
	};
	for (int b = 0; b < num_batches; b += 2) {
		step(b, s_hdr0, s_hdr1);
		if (b + 1 < num_batches) step(b + 1, s_hdr1, s_hdr0);
	}
	if (q > 0) {
		for (int r = q; r < kFeatGroup; r++) rows[r * kRowStride + lane] = 0u;
		flush();
	}
}

template <int S, bool RGB>
int launch_geometry(const BackwardArgs& a, int slices, hipStream_t s) {
	HdsKernelTimer timer1("backward_geometry_kernel", s);
	backward_geometry_kernel<S, RGB><<<dim3(hds_xcd_grid(a.tiles_x, a.num_tiles), (unsigned)slices), 256, 0, s>>>(a);
	timer1.stop();
	return hds_check_launch(RGB ? (S > 0 ? "backward_geometry_rgb_features" : "backward_geometry_rgb")
								: "backward_geometry_features",
							s);
}

template <int S>
int launch_features(const BackwardArgs& a, int slices, hipStream_t s) {
	HdsKernelTimer timer2("backward_features_kernel", s);
	backward_features_kernel<S><<<dim3(hds_xcd_grid(a.tiles_x, a.num_tiles), (unsigned)slices), 256, 0, s>>>(a);
	timer2.stop();
	return hds_check_launch("backward_features", s);
}

// Zeroes up to four float ranges in one launch.
struct ZeroList {
	float* p[4];
	int64_t end[4];  // running sums of the range lengths
};

__global__ __launch_bounds__(256) void zero_kernel(const ZeroList z) {
	const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
	int64_t begin = 0;
#pragma unroll
	for (int k = 0; k < 4; k++) {
		if (i >= begin && i < z.end[k]) z.p[k][i - begin] = 0.0f;
		begin = z.end[k];
	}
}

int zero_small(hipStream_t s, float* p0, int64_t n0, float* p1 = nullptr, int64_t n1 = 0, float* p2 = nullptr,
			   int64_t n2 = 0, float* p3 = nullptr, int64_t n3 = 0);

// Zeroes a large 16-byte aligned range with one 16-byte store per thread and step.
__global__ __launch_bounds__(256) void zero4_kernel(float4* __restrict__ p, int64_t count4) {
	const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
	for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count4; i += (int64_t)gridDim.x * blockDim.x)
		p[i] = z;
}

int zero_large(hipStream_t s, float* p, int64_t count) {
	if (!p || count == 0) return HDS_OK;
	if ((reinterpret_cast<uintptr_t>(p) & 15u) != 0 || count % 4 != 0) return zero_small(s, p, count);
	const int64_t count4 = count / 4;
	const int64_t blocks = std::min<int64_t>(hds_blocks(count4, 256), 8192);
	HdsKernelTimer timer4("zero4_kernel", s);
	zero4_kernel<<<(unsigned)blocks, 256, 0, s>>>(reinterpret_cast<float4*>(p), count4);
	timer4.stop();
	return hds_check_launch("zero_feature_gradients", s);
}

int zero_small(hipStream_t s, float* p0, int64_t n0, float* p1, int64_t n1, float* p2, int64_t n2, float* p3,
			   int64_t n3) {
	ZeroList z{};
	float* ps[4] = {p0, p1, p2, p3};
	const int64_t ns[4] = {p0 ? n0 : 0, p1 ? n1 : 0, p2 ? n2 : 0, p3 ? n3 : 0};
	int64_t total = 0;
	for (int k = 0; k < 4; k++) {
		z.p[k] = ps[k];
		total += ns[k];
		z.end[k] = total;
	}
	if (total == 0) return HDS_OK;
	HdsKernelTimer timer3("zero_kernel", s);
	zero_kernel<<<hds_blocks(total, 256), 256, 0, s>>>(z);
	timer3.stop();
	return hds_check_launch("zero_gradients", s);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Work on the device's side stream that starts after everything queued on `main` so far
// (begin) and that `main` waits for before its later work (end). The events are released on
// every path.
struct Fork {
	hipStream_t main = nullptr, side = nullptr;
	hipEvent_t forked = nullptr, joined = nullptr;
	int begin(hipStream_t s) {
		main = s;
		int st = hds_side_stream(&side);
		if (st != HDS_OK) return st;
		HDS_HIP(hipEventCreateWithFlags(&forked, hipEventDisableTiming));
		HDS_HIP(hipEventCreateWithFlags(&joined, hipEventDisableTiming));
		HDS_HIP(hipEventRecord(forked, main));
		HDS_HIP(hipStreamWaitEvent(side, forked, 0));
		return HDS_OK;
	}
	int end() {
		HDS_HIP(hipEventRecord(joined, side));
		HDS_HIP(hipStreamWaitEvent(main, joined, 0));
		return HDS_OK;
	}
	~Fork() {
		if (forked) (void)hipEventDestroy(forked);
		if (joined) (void)hipEventDestroy(joined);
	}
};

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
	// The gradients are accumulated with atomics; the zeroing variant clears them first.
	const bool run = n > 0 && num_pairs > 0;
	if (zero_outputs) {
		int st = zero_small(s, grad_means2D, 2 * n, grad_conics, 3 * n, grad_opacities, n, grad_colors, 3 * n);
		if (st != HDS_OK) return st;
		// Before the fork: zeroing beside the running geometry kernel starves the fill of CUs.
		if (feats && grad_features && (st = zero_large(s, grad_features, (int64_t)channels * n)) != HDS_OK) return st;
	}
	if (!run) return HDS_OK;

	const int tiles_x = (width + HDS_TILE - 1) / HDS_TILE, tiles_y = (height + HDS_TILE - 1) / HDS_TILE;
	const int num_tiles = tiles_x * tiles_y;
	BackwardArgs a{width,
				   height,
				   tiles_x,
				   feats ? channels : 0,
				   num_tiles,
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
	if (!feats) return launch_geometry<0, true>(a, 1, s);
	const int slices = channels / slice_width;
	// The feature-gradient kernel runs beside the geometry kernel, on a second stream forked from
	// and joined back into the caller's: much of its time goes to HBM-bound gradient atomics, while
	// the geometry kernel is bound by VALU issue and LDS latency, so the two overlap well.
	Fork fork;
	if (grad_features) {
		int st = fork.begin(s);
		if (st != HDS_OK) return st;
		switch (slice_width) {
			case 32: st = launch_features<32>(a, slices, fork.side); break;
			case 64: st = launch_features<64>(a, slices, fork.side); break;
			default: st = launch_features<128>(a, slices, fork.side); break;
		}
		if (st != HDS_OK) return st;
	}
	int st;
	switch (slice_width) {
		case 32: st = rgb ? launch_geometry<32, true>(a, slices, s) : launch_geometry<32, false>(a, slices, s); break;
		case 64: st = rgb ? launch_geometry<64, true>(a, slices, s) : launch_geometry<64, false>(a, slices, s); break;
		default: st = rgb ? launch_geometry<128, true>(a, slices, s) : launch_geometry<128, false>(a, slices, s); break;
	}
	const int joined = grad_features ? fork.end() : HDS_OK;
	return st != HDS_OK ? st : joined;
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

extern "C" int hds_zero_async(float* p, int64_t count, int max_workgroups, hds_stream_t stream) {
	HDS_REQUIRE(count >= 0 && max_workgroups >= 0, "zero_async: negative count or work-group limit");
	if (count == 0) return HDS_OK;
	HDS_REQUIRE(p && aligned16(p) && count % 4 == 0, "zero_async: needs a 16-byte aligned range of a multiple of 4 floats");
	const int64_t count4 = count / 4;
	int64_t blocks = std::min<int64_t>(hds_blocks(count4, 256), 8192);
	if (max_workgroups > 0) blocks = std::min<int64_t>(blocks, max_workgroups);
	hipStream_t s = (hipStream_t)stream;
	HdsKernelTimer timer("zero4_kernel", s);
	zero4_kernel<<<(unsigned)blocks, 256, 0, s>>>(reinterpret_cast<float4*>(p), count4);
	timer.stop();
	return hds_check_launch("zero_async", s);
}
