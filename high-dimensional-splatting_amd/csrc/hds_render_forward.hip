// Front-to-back blend of RGB and C feature channels in one tile walk.
//
// Work-group = one 16x16 tile (and one slice of S <= 128 channels); wave w owns the 8x8 block
// ((w & 1) * 8, (w >> 1) * 8) and lane l the pixel (l & 7, l >> 3) of it. Gaussians of the tile's
// sorted list are staged 64 at a time in LDS (geometry, culling box and the slice's feature rows as
// raw fp32, split into bf16 operands when read); each wave ballots which of the 64 box-hit its block
// and walks only those, in order, updating T, RGB and n_contrib per lane exactly as render_gaussians does
// (forward.cu:181-225): alpha = min(0.99, op * exp(-m/2)), skip below 1/255, stop before T would
// drop below 1e-4, n_contrib = 1-based list index of the last blended gaussian.
//
// Features: the wave's box-hits are taken 16 at a time, in list order, as the K dimension of
//   out[c][px] += sum_k F[k][c] * W[k][px],
// one v_mfma_f32_32x32x16_bf16 per 32 channels x 32 pixels, both operands in split-bf16 (3 MFMAs
// per tile, ~2^-16 relative error; CDNA4 has no TF32). Each lane keeps its own pixel's 16 weights
// w = alpha * T (0 where it did not blend) in registers as packed bf16 pairs; one
// v_permlane32_swap per register pair then forms the B operands of the two 32-pixel halves, so the
// weights never touch LDS. The 16-hit groups depend on geometry only and the batch size is fixed,
// so each output channel sees the same operation sequence whatever C or the slicing is: channels
// are bitwise independent and RGB is bitwise equal with or without features (the properties the
// reference's tests/test_properties.py pins). The accumulators take S registers per lane (ordinary
// VGPRs: the compiler assigns no AGPRs here); with the walk's registers the 128-channel slice needs
// about 240 and runs two waves per SIMD, the 64-channel slice three, the 32-channel slice three with
// RGB (four would cap it at 128 registers, which spills) and four without.
#include <cstdlib>

#include "hds_internal.h"
#include "hds_rasterizer.h"
#include "hds_stage.h"

namespace {

constexpr int kBatch = 64;  // gaussians staged per LDS batch = one ballot per wave
constexpr int kGroup = 16;  // K of one MFMA: box-hits per group
constexpr int kIlp = 4;     // hits whose alpha is evaluated together

struct RenderArgs {
	int width, height, tiles_x, channels, num_tiles;
	const int2* ranges;
	const int* values;
	const float2* means2D;
	const float4* conic4;
	const float4* color_op4;
	const float* background;
	const float* features;
	float* image;
	float* final_T;
	int* n_contrib;
	float* feature_image;
	float4* clear;   // hds_render_clear's range (clear4 16-byte words), or null
	int64_t clear4;
};

// acc[m][cb] += F^T W for one group. w_hi / w_lo hold this lane's pixel's packed weights for
// positions (2i, 2i+1); after the swaps, words 0-3 are the B operand of pixels 0-31 and words 4-7
// that of pixels 32-63. A = features: lane = (channel lane % 32, positions 8 (lane / 32) + 0..7),
// read as raw fp32 from the staged rows (S floats each) and split here.
template <int S>
__device__ inline void flush_group(hds_f32x16 (&acc)[2][S / 32], uint32_t (&w_hi)[8], uint32_t (&w_lo)[8],
								   const int (&slot)[kGroup], const float* feat, int lane) {
#pragma unroll
	for (int i = 0; i < 4; i++) {
		const auto h = __builtin_amdgcn_permlane32_swap(w_hi[i], w_hi[4 + i], false, false);
		w_hi[i] = h[0];
		w_hi[4 + i] = h[1];
		const auto l = __builtin_amdgcn_permlane32_swap(w_lo[i], w_lo[4 + i], false, false);
		w_lo[i] = l[0];
		w_lo[4 + i] = l[1];
	}
	hds_bf16x8 b_hi[2], b_lo[2];
#pragma unroll
	for (int m = 0; m < 2; m++) {
		b_hi[m] = __builtin_bit_cast(hds_bf16x8, hds_u32x4{w_hi[4 * m], w_hi[4 * m + 1], w_hi[4 * m + 2], w_hi[4 * m + 3]});
		b_lo[m] = __builtin_bit_cast(hds_bf16x8, hds_u32x4{w_lo[4 * m], w_lo[4 * m + 1], w_lo[4 * m + 2], w_lo[4 * m + 3]});
	}
	const bool upper = lane >= 32;
	const int col = lane & 31;
	int row[8];
#pragma unroll
	for (int j = 0; j < 8; j++) {
		// Select the values, not the array half: an indexed pointer select would put slot in scratch.
		const int lo = slot[j], hi = slot[8 + j];
		row[j] = (upper ? hi : lo) * S + col;
	}
#pragma unroll
	for (int cb = 0; cb < S / 32; cb++) {
		float v[8];
#pragma unroll
		for (int j = 0; j < 8; j++) v[j] = feat[row[j] + 32 * cb];
		hds_bf16x8 a_hi, a_lo;
		hds_split8(v, a_hi, a_lo);
#pragma unroll
		for (int m = 0; m < 2; m++) acc[m][cb] = hds_mfma32_split(a_hi, a_lo, b_hi[m], b_lo[m], acc[m][cb]);
	}
}

// Per-lane state of the walk.
struct Pixel {
	float T;
	bool done;
	int last;
	float r, g, b;
};

// Occupancy: S accumulators per lane plus the walk's registers, two waves per SIMD with features.
//
// Pipeline per batch b: the records and feature rows of batch b+1 are copied into the other slot by
// LDS DMA while b is walked, and the gids of b+2 are read; one barrier, after each wave has waited
// for its copies, hands the next batch over.
template <int S, bool RGB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(S >= 128 ? 2 : (S == 64 || RGB) ? 3 : 4))) void render_forward_kernel(
	const RenderArgs a) {
	constexpr int kNcb = S > 0 ? S / 32 : 1;
	constexpr int kRows = S > 0 ? (kBatch + 1) * S : 1;

	// Gaussian ids of batches b, b+1, b+2 (slot b % 3).
	__shared__ int s_gid[3][kBatch];
	// Records and feature rows of the batch being walked and of the next one; feature row kBatch
	// stays zero (positions past the end of a partial group point at it).
	__shared__ HdsHeaderSlot<kBatch, RGB> s_hdr0, s_hdr1;
	__shared__ __attribute__((aligned(16))) float s_feat0[kRows];
	__shared__ __attribute__((aligned(16))) float s_feat1[kRows];
	// Per wave: the batch slots of its box-hits in list order, then kBatch (the zero row) as padding.
	__shared__ __attribute__((aligned(16))) int s_hit[4][kBatch + kGroup];

	const int tile = hds_xcd_tile(blockIdx.x, a.tiles_x, a.num_tiles);
	if (tile < 0) return;
	// hds_render_clear: every (tile, slice) work-group zeroes one contiguous share of the caller's
	// range before its walk. The walk leaves most of the HBM bandwidth unused, so the 16-byte stores
	// drain beside it instead of in a fill launch of their own; non-temporal, so the zeros do not
	// push the walk's feature rows out of L2 (render 1.68 -> 1.61 ms at 4M gaussians, C = 256).
	if (a.clear4 > 0) {
		typedef float f32x4v __attribute__((ext_vector_type(4)));
		const int64_t parts = (int64_t)a.num_tiles * gridDim.y;
		const int64_t per = (a.clear4 + parts - 1) / parts;
		const int64_t begin = ((int64_t)tile * gridDim.y + blockIdx.y) * per;
		const int64_t end = min(a.clear4, begin + per);
		f32x4v* const clear = reinterpret_cast<f32x4v*>(a.clear);
		for (int64_t e = begin + threadIdx.x; e < end; e += blockDim.x)
			__builtin_nontemporal_store((f32x4v){0.0f, 0.0f, 0.0f, 0.0f}, clear + e);
	}
	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const int slice = blockIdx.y;
	const int tx0 = (tile % a.tiles_x) * HDS_TILE, ty0 = (tile / a.tiles_x) * HDS_TILE;
	const int wx0 = tx0 + (wave & 1) * 8, wy0 = ty0 + (wave >> 1) * 8;
	const int px = wx0 + (lane & 7), py = wy0 + (lane >> 3);
	const bool inside = px < a.width && py < a.height;
	const float fx = (float)px + 0.5f, fy = (float)py + 0.5f;
	const float rx0 = (float)wx0 + 0.5f, rx1 = (float)wx0 + 7.5f;
	const float ry0 = (float)wy0 + 0.5f, ry1 = (float)wy0 + 7.5f;
	const int2 range = a.ranges[tile];
	const int num = range.y - range.x;
	const int num_batches = (num + kBatch - 1) / kBatch;
	const int c0 = slice * S;
	auto batch_count = [&](int b) { return b < num_batches ? min(kBatch, num - b * kBatch) : 0; };

	Pixel st{1.0f, !inside, 0, 0.0f, 0.0f, 0.0f};
	hds_f32x16 acc[2][kNcb];
#pragma unroll
	for (int m = 0; m < 2; m++)
#pragma unroll
		for (int c = 0; c < kNcb; c++) acc[m][c] = hds_f32x16{};

	if (num_batches == 0) goto write_out;
	{
		// Prologue: gids of batches 0 and 1, then batch 0 staged synchronously.
		if constexpr (S > 0)
			for (int i = tid; i < S; i += blockDim.x) s_feat0[kBatch * S + i] = s_feat1[kBatch * S + i] = 0.0f;
		const int cnt0 = batch_count(0), cnt1 = batch_count(1);
		if (tid < cnt0) s_gid[0][tid] = a.values[range.x + tid];
		if (tid < cnt1) s_gid[1][tid] = a.values[range.x + kBatch + tid];
		__syncthreads();
		hds_stage_headers_async<kBatch, RGB>(s_hdr0, a.means2D, a.conic4, a.color_op4, s_gid[0], cnt0, tid);
		if constexpr (S > 0)
			hds_stage_rows_async<S, false, kBatch>(s_feat0, a.features, a.channels, c0, s_gid[0], cnt0, tid);
		hds_wait_vmem();
		__syncthreads();
	}

	{
		// One batch: stage b+1, read the gids of b+2, walk b. Returns true when every pixel is done.
		auto step = [&](int b, const HdsHeaderSlot<kBatch, RGB>& h, const float* feat,
						HdsHeaderSlot<kBatch, RGB>& h_next, float* feat_next) -> bool {
			const int cnt = batch_count(b), cnt1 = batch_count(b + 1), cnt2 = batch_count(b + 2);
			int g2 = 0;
			if (tid < cnt2) g2 = a.values[range.x + (b + 2) * kBatch + tid];
			const int* gid_next = s_gid[(b + 1) % 3];
			if (cnt1 > 0) {
				hds_stage_headers_async<kBatch, RGB>(h_next, a.means2D, a.conic4, a.color_op4, gid_next, cnt1, tid);
				if constexpr (S > 0)
					hds_stage_rows_async<S, false, kBatch>(feat_next, a.features, a.channels, c0, gid_next, cnt1, tid);
			}

			if (hds_ballot(!st.done) != 0) {
				const int batch = b * kBatch;
				bool box_hit = false;
				if (lane < cnt) {
					box_hit = hds_block_reach(make_float2(h.mx[lane], h.my[lane]), h.conic[lane], rx0, rx1, ry0, ry1);
				}
				const uint64_t hits = hds_ballot(box_hit);
				const int total = __builtin_popcountll(hits);
				// List the hits once per batch: hit j goes to position rank(j); positions up to the
				// next multiple of kGroup past the last hit point at the zero row.
				int* hit_slot = s_hit[wave];
				if (box_hit) hit_slot[hds_rank_below(hits)] = lane;
				if (lane >= total && lane < ((total + kGroup - 1) & ~(kGroup - 1))) hit_slot[lane] = kBatch;
				hds_wave_fence();
				for (int g0 = 0; g0 < total; g0 += kGroup) {
					// The next group: up to 16 box-hits in list order; missing positions use the zero row.
					const int count = min(kGroup, total - g0);
					int slot[kGroup];
#pragma unroll
					for (int q4 = 0; q4 < kGroup; q4 += 4) {
						const int4 v = *reinterpret_cast<const int4*>(hit_slot + g0 + q4);
						slot[q4] = v.x;
						slot[q4 + 1] = v.y;
						slot[q4 + 2] = v.z;
						slot[q4 + 3] = v.w;
					}
					float w[kGroup];
#pragma unroll
					for (int q0 = 0; q0 < kGroup; q0 += kIlp) {
						if (q0 >= count) {
							// Past the group's last hit (wave-uniform): nothing to evaluate.
#pragma unroll
							for (int u = 0; u < kIlp; u++) w[q0 + u] = 0.0f;
							continue;
						}
						float alpha[kIlp];
						float4 col[kIlp];
#pragma unroll
						for (int u = 0; u < kIlp; u++) {
							const int sl = min(slot[q0 + u], kBatch - 1);
							float G, dx, dy;
							alpha[u] = fminf(HDS_MAX_ALPHA, hds_raw_alpha(fx, fy, make_float2(h.mx[sl], h.my[sl]),
																		  h.conic[sl], G, dx, dy));
							// Read with the geometry: a read under the blend branch would stall on LDS latency.
							if constexpr (RGB) col[u] = h.color[sl];
						}
#pragma unroll
						for (int u = 0; u < kIlp; u++) {
							const int q = q0 + u;
							w[q] = 0.0f;
							if (q < count && !st.done && alpha[u] >= HDS_MIN_ALPHA) {
								const float test_T = st.T * (1.0f - alpha[u]);
								if (test_T < HDS_MIN_TRANSMITTANCE) {
									st.done = true;
								} else {
									w[q] = alpha[u] * st.T;
									if constexpr (RGB) {
										// fmaf as the oracle does: the RGB image is bit-exact.
										st.r = fmaf(w[q], col[u].x, st.r);
										st.g = fmaf(w[q], col[u].y, st.g);
										st.b = fmaf(w[q], col[u].z, st.b);
									}
									st.T = test_T;
									st.last = batch + slot[q] + 1;
								}
							}
						}
					}
					if constexpr (S > 0) {
						uint32_t w_hi[8], w_lo[8];
#pragma unroll
						for (int i = 0; i < 8; i++) hds_split_pair(w[2 * i], w[2 * i + 1], w_hi[i], w_lo[i]);
						flush_group<S>(acc, w_hi, w_lo, slot, feat, lane);
					}
					if (hds_ballot(!st.done) == 0) break;
				}
			}

			if (tid < cnt2) s_gid[(b + 2) % 3][tid] = g2;
			hds_wait_vmem();
			return __syncthreads_count(st.done) == (int)blockDim.x;
		};
		for (int b = 0; b < num_batches; b += 2) {
			if (step(b, s_hdr0, s_feat0, s_hdr1, s_feat1) || b + 1 >= num_batches) break;
			if (step(b + 1, s_hdr1, s_feat1, s_hdr0, s_feat0)) break;
		}
	}

write_out:
	if (inside && slice == 0) {
		const int64_t pix = (int64_t)py * a.width + px;
		if constexpr (RGB) {
			a.image[pix * 3 + 0] = fmaf(st.T, a.background[0], st.r);
			a.image[pix * 3 + 1] = fmaf(st.T, a.background[1], st.g);
			a.image[pix * 3 + 2] = fmaf(st.T, a.background[2], st.b);
		}
		a.final_T[pix] = st.T;
		a.n_contrib[pix] = st.last;
	}
	if constexpr (S > 0) {
		// D of a 32x32 tile: lane holds pixel 32m + lane % 32 and, for each group g of four
		// accumulators, channels 8g + 4 (lane / 32) + 0..3.
#pragma unroll
		for (int m = 0; m < 2; m++) {
			const int p = 32 * m + (lane & 31);
			const int x = wx0 + (p & 7), y = wy0 + (p >> 3);
			if (x >= a.width || y >= a.height) continue;
			float* dst = a.feature_image + ((int64_t)y * a.width + x) * a.channels + c0 + 4 * (lane >> 5);
#pragma unroll
			for (int c = 0; c < kNcb; c++)
#pragma unroll
				for (int g = 0; g < 4; g++) {
					const hds_f32x16 v = acc[m][c];
					*reinterpret_cast<float4*>(dst + 32 * c + 8 * g) = make_float4(v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]);
				}
		}
	}
}

template <int S, bool RGB>
int launch(const RenderArgs& a, int num_tiles, int slices, hipStream_t s) {
	HdsKernelTimer timer1("render_forward_kernel", s);
	render_forward_kernel<S, RGB><<<dim3(hds_xcd_grid(a.tiles_x, num_tiles), (unsigned)slices), 256, 0, s>>>(a);
	timer1.stop();
	return hds_check_launch(RGB ? (S > 0 ? "render_rgb_features" : "render_rgb") : "render_features", s);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int render(int width, int height, int channels, const int32_t* tile_ranges, const int32_t* values_sorted,
		   int64_t num_pairs, const float* means2D, const float* conic4, const float* color_opacity4,
		   const float* background, const float* features, float* image, float* final_T, int32_t* n_contrib,
		   float* feature_image, float* clear, int64_t clear_count, hds_stream_t stream) {
	HDS_REQUIRE(clear_count >= 0, "render_clear: negative clear count");
	HDS_REQUIRE(clear_count == 0 || (clear && aligned16(clear) && clear_count % 4 == 0),
				"render_clear: needs a 16-byte aligned range of a multiple of 4 floats");
	HDS_REQUIRE(width > 0 && height > 0, "render: image size %dx%d must be positive", width, height);
	HDS_REQUIRE(tile_ranges && final_T && n_contrib, "render: null tile_ranges / final_T / n_contrib");
	const bool rgb = image != nullptr;
	const bool feats = features != nullptr;
	if (feats)
		HDS_REQUIRE(channels == 32 || channels == 64 || channels == 128 || channels == 256 || channels == 512,
					"features must have 32, 64, 128, 256 or 512 channels, got %d", channels);
	HDS_REQUIRE(!feats || feature_image, "render: features given without feature_image");
	HDS_REQUIRE(!rgb || (background && (color_opacity4 || num_pairs == 0)), "render: image requested without background / colors");
	HDS_REQUIRE(num_pairs == 0 || (values_sorted && means2D && conic4), "render: null gaussian arguments");
	HDS_REQUIRE(aligned16(conic4) && (!color_opacity4 || aligned16(color_opacity4)) && (!features || aligned16(features)) &&
					(!feature_image || aligned16(feature_image)) && (reinterpret_cast<uintptr_t>(means2D) & 7u) == 0 &&
					(reinterpret_cast<uintptr_t>(tile_ranges) & 7u) == 0,
				"render: misaligned buffer (conic4, color_opacity4, features, feature_image need 16 bytes)");
	const int tiles_x = (width + HDS_TILE - 1) / HDS_TILE, tiles_y = (height + HDS_TILE - 1) / HDS_TILE;
	const int num_tiles = tiles_x * tiles_y;
	RenderArgs a{width,
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
				 features,
				 image,
				 final_T,
				 n_contrib,
				 feature_image,
				 reinterpret_cast<float4*>(clear),
				 clear_count / 4};
	hipStream_t s = (hipStream_t)stream;
	if (!feats) {
		HDS_REQUIRE(rgb, "render: nothing to render (no image and no features)");
		return launch<0, true>(a, num_tiles, 1, s);
	}
	// Channels per work-group: 128 unless HDS_FORWARD_SLICE_WIDTH (32, 64 or 128) asks for less. The
	// result does not depend on it: every channel runs the same operation sequence.
	int width_slice = channels < 128 ? channels : 128;
	if (const char* env = std::getenv("HDS_FORWARD_SLICE_WIDTH")) {
		const int w = std::atoi(env);
		if ((w == 32 || w == 64 || w == 128) && w <= channels) width_slice = w;
	}
	const int slices = channels / width_slice;
	switch (width_slice) {
		case 32: return rgb ? launch<32, true>(a, num_tiles, slices, s) : launch<32, false>(a, num_tiles, slices, s);
		case 64: return rgb ? launch<64, true>(a, num_tiles, slices, s) : launch<64, false>(a, num_tiles, slices, s);
		default: return rgb ? launch<128, true>(a, num_tiles, slices, s) : launch<128, false>(a, num_tiles, slices, s);
	}
}

}  // namespace

extern "C" int hds_render(int64_t n, int width, int height, int channels, const int32_t* tile_ranges,
						  const int32_t* values_sorted, int64_t num_pairs, const float* means2D, const float* conic4,
						  const float* color_opacity4, const float* background, const float* features, float* image,
						  float* final_T, int32_t* n_contrib, float* feature_image, hds_stream_t stream) {
	(void)n;
	return render(width, height, channels, tile_ranges, values_sorted, num_pairs, means2D, conic4, color_opacity4,
				  background, features, image, final_T, n_contrib, feature_image, nullptr, 0, stream);
}

extern "C" int hds_render_clear(int64_t n, int width, int height, int channels, const int32_t* tile_ranges,
								const int32_t* values_sorted, int64_t num_pairs, const float* means2D,
								const float* conic4, const float* color_opacity4, const float* background,
								const float* features, float* image, float* final_T, int32_t* n_contrib,
								float* feature_image, float* clear, int64_t clear_count, hds_stream_t stream) {
	(void)n;
	return render(width, height, channels, tile_ranges, values_sorted, num_pairs, means2D, conic4, color_opacity4,
				  background, features, image, final_T, n_contrib, feature_image, clear, clear_count, stream);
}
