// Front-to-back blend of RGB and C feature channels in one tile walk.
//
// Work-group = one 16x16 tile (and one slice of S <= 128 channels); wave w owns the 8x8 block
// ((w & 1) * 8, (w >> 1) * 8) and lane l the pixel (l & 7, l >> 3) of it. Gaussians of the tile's
// sorted list are staged 64 at a time in LDS (geometry, culling box and the slice's features as
// split-bf16 words); each wave ballots which of the 64 box-hit its block and walks only those, in
// order, updating T, RGB and n_contrib per lane exactly as render_gaussians does
// (forward.cu:181-225): alpha = min(0.99, op * exp(-m/2)), skip below 1/255, stop before T would
// drop below 1e-4, n_contrib = 1-based list index of the last blended gaussian.
//
// Features: every gaussian some lane blended becomes one position of the wave's current group;
// its per-pixel weights w = alpha * T go to LDS. A full group of 32 is one contraction
//   out[c][px] += sum_k F[k][c] * W[k][px],
// 16 channels x 16 pixels per v_mfma_f32_16x16x32_bf16 tile, with both operands in split-bf16
// (3 MFMAs per tile, ~2^-16 relative error; CDNA4 has no TF32). Groups depend on geometry only
// and the batch size is fixed, so each output channel sees the same operation sequence whatever
// C or the slicing is: channels are bitwise independent and RGB is bitwise equal with or without
// features (the properties tests/test_properties.py pins for the reference).
#include <cstdlib>

#include "hds_internal.h"
#include "hds_rasterizer.h"

namespace {

constexpr int kBatch = 64;      // gaussians staged per LDS batch = one ballot per wave
constexpr int kGroup = 32;      // K of one MFMA: group positions per flush
constexpr int kWStride = 66;    // words per weight row: 64 pixels + 2 keeps the 4 lane groups on distinct banks
constexpr int kIlp = 4;         // hits evaluated together

struct RenderArgs {
	int width, height, tiles_x, channels;
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
};

template <int S>
struct FeatTraits {
	static constexpr int kNcb = S / 16;          // 16-channel MFMA row blocks
	static constexpr int kStride = S + 4;        // words per staged feature row (16-byte aligned)
};

// acc[m][cb] += F^T W for the wave's group: A = features (rows = 16 channels, K = 32 positions),
// B = weights (K = 32 positions, cols = 16 pixels of block m).
template <int S>
__device__ inline void flush_group(hds_f32x4 (&acc)[4][FeatTraits<S>::kNcb], const uint32_t* w_rows, const int* slots,
								   const uint32_t* s_feat, int lane) {
	constexpr int kNcb = FeatTraits<S>::kNcb;
	constexpr int kStride = FeatTraits<S>::kStride;
	hds_wave_fence();
	const int kq = lane >> 4, col = lane & 15;
	// B (weights) for the four 16-pixel blocks stays in registers for the whole flush; A (features)
	// is fetched one 16-channel block ahead of its MFMAs. The scheduling barriers bound how far the
	// compiler hoists those fetches, which keeps the C=128 flush inside two waves' register budget.
	hds_bf16x8 b_hi[4], b_lo[4];
#pragma unroll
	for (int m = 0; m < 4; m++) {
		uint32_t e[8];
#pragma unroll
		for (int j = 0; j < 8; j++) e[j] = w_rows[(8 * kq + j) * kWStride + 16 * m + col];
		hds_unpack8(e, b_hi[m], b_lo[m]);
	}
	int row[8];
#pragma unroll
	for (int j = 0; j < 8; j++) row[j] = slots[8 * kq + j] * kStride + col;
	uint32_t d[8];
#pragma unroll
	for (int j = 0; j < 8; j++) d[j] = s_feat[row[j]];
#pragma unroll
	for (int cb = 0; cb < kNcb; cb++) {
		hds_bf16x8 a_hi, a_lo;
		hds_unpack8(d, a_hi, a_lo);
		if (cb + 1 < kNcb) {
#pragma unroll
			for (int j = 0; j < 8; j++) d[j] = s_feat[row[j] + 16 * (cb + 1)];
		}
#pragma unroll
		for (int m = 0; m < 4; m++) acc[m][cb] = hds_mfma_split(a_hi, a_lo, b_hi[m], b_lo[m], acc[m][cb]);
		__builtin_amdgcn_sched_barrier(0);
	}
	hds_wave_fence();
}

// Occupancy targets: the 128-channel slice keeps its 128 accumulators in AGPRs at one wave per
// SIMD; narrower slices fit two or more.
template <int S, bool RGB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(S == 128 ? 1 : (S > 0 ? 2 : 4)))) void render_forward_kernel(
	const RenderArgs a) {
	constexpr int kNcb = S > 0 ? FeatTraits<S>::kNcb : 1;
	constexpr int kStride = S > 0 ? FeatTraits<S>::kStride : 1;

	__shared__ int s_gid[kBatch];
	__shared__ float2 s_mean[kBatch];
	__shared__ float4 s_conic[kBatch];
	__shared__ float4 s_color[RGB ? kBatch : 1];
	__shared__ float4 s_box[kBatch];
	// Row kBatch stays zero: padding positions of a partial group point at it.
	__shared__ __attribute__((aligned(16))) uint32_t s_feat[S > 0 ? (kBatch + 1) * kStride : 1];
	__shared__ uint32_t s_w[S > 0 ? 4 * kGroup * kWStride : 1];
	__shared__ int s_slot[S > 0 ? 4 * kGroup : 1];

	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const int tile = blockIdx.x, slice = blockIdx.y;
	const int tx0 = (tile % a.tiles_x) * HDS_TILE, ty0 = (tile / a.tiles_x) * HDS_TILE;
	const int wx0 = tx0 + (wave & 1) * 8, wy0 = ty0 + (wave >> 1) * 8;
	const int px = wx0 + (lane & 7), py = wy0 + (lane >> 3);
	const bool inside = px < a.width && py < a.height;
	const float fx = (float)px + 0.5f, fy = (float)py + 0.5f;
	const float rx0 = (float)wx0 + 0.5f, rx1 = (float)wx0 + 7.5f;
	const float ry0 = (float)wy0 + 0.5f, ry1 = (float)wy0 + 7.5f;
	const int2 range = a.ranges[tile];
	const int num = range.y - range.x;
	const int c0 = slice * S;

	float T = 1.0f;
	bool done = !inside;
	int last = 0;
	float cr = 0.0f, cg = 0.0f, cb_ = 0.0f;
	hds_f32x4 acc[4][kNcb];
#pragma unroll
	for (int m = 0; m < 4; m++)
#pragma unroll
		for (int c = 0; c < kNcb; c++) acc[m][c] = hds_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
	int k = 0;
	uint32_t* w_rows = s_w + wave * kGroup * kWStride;
	int* slots = s_slot + wave * kGroup;

	if constexpr (S > 0)
		for (int i = tid; i < kStride; i += blockDim.x) s_feat[kBatch * kStride + i] = 0u;

	for (int batch = 0; batch < num; batch += kBatch) {
		// Also the barrier between the last batch's LDS reads and this batch's writes.
		if (__syncthreads_count(done) == (int)blockDim.x) break;
		const int cnt = min(kBatch, num - batch);
		if (tid < cnt) {
			const int gid = a.values[range.x + batch + tid];
			const float2 m = a.means2D[gid];
			const float4 co = a.conic4[gid];
			s_gid[tid] = gid;
			s_mean[tid] = m;
			s_conic[tid] = co;
			if constexpr (RGB) s_color[tid] = a.color_op4[gid];
			s_box[tid] = hds_cull_box(m, co);
		}
		if constexpr (S > 0) {
			__syncthreads();
			constexpr int kVec = S / 4;
			for (int i = tid; i < cnt * kVec; i += blockDim.x) {
				const int row = i / kVec, q = i - row * kVec;
				const float4 f = *reinterpret_cast<const float4*>(a.features + (size_t)s_gid[row] * a.channels + c0 + 4 * q);
				uint4 packed = make_uint4(hds_split_pack(f.x), hds_split_pack(f.y), hds_split_pack(f.z), hds_split_pack(f.w));
				*reinterpret_cast<uint4*>(&s_feat[row * kStride + 4 * q]) = packed;
			}
		}
		__syncthreads();
		if (hds_ballot(!done) == 0) continue;

		uint64_t hits = hds_ballot(lane < cnt && hds_box_hits(s_box[lane < cnt ? lane : 0], rx0, rx1, ry0, ry1));
		// Hits go four at a time: their alphas are independent (only T chains through them), which
		// gives each wave enough independent work to cover LDS and transcendental latency.
		while (hits) {
			int slot[kIlp];
			int nq = 0;
#pragma unroll
			for (int q = 0; q < kIlp; q++) {
				slot[q] = nq > 0 ? slot[0] : 0;
				if (hits) {
					slot[q] = __builtin_ctzll(hits);
					hits &= hits - 1;
					nq = q + 1;
				}
			}
			float alpha[kIlp];
#pragma unroll
			for (int q = 0; q < kIlp; q++) {
				float G, dx, dy;
				alpha[q] = fminf(HDS_MAX_ALPHA, hds_raw_alpha(fx, fy, s_mean[slot[q]], s_conic[slot[q]], G, dx, dy));
			}
#pragma unroll
			for (int q = 0; q < kIlp; q++) {
				if (q >= nq) break;
				float w = 0.0f;
				if (!done && alpha[q] >= HDS_MIN_ALPHA) {
					const float test_T = T * (1.0f - alpha[q]);
					if (test_T < HDS_MIN_TRANSMITTANCE) {
						done = true;
					} else {
						w = alpha[q] * T;
						if constexpr (RGB) {
							const float4 col = s_color[slot[q]];
							cr += w * col.x;
							cg += w * col.y;
							cb_ += w * col.z;
						}
						T = test_T;
						last = batch + slot[q] + 1;
					}
				}
				if constexpr (S > 0) {
					if (hds_ballot(w > 0.0f)) {
						w_rows[k * kWStride + lane] = hds_split_pack(w);
						if (lane == 0) slots[k] = slot[q];
						k++;
						if (k == kGroup) {
							flush_group<S>(acc, w_rows, slots, s_feat, lane);
							k = 0;
						}
					}
				}
			}
			if (hds_ballot(!done) == 0) break;
		}
		if constexpr (S > 0) {
			// The next batch overwrites the staged features: flush the partial group now, its
			// free positions carrying zero weights and the zero feature row.
			if (k > 0) {
				for (int q = k; q < kGroup; q++) w_rows[q * kWStride + lane] = 0u;
				if (lane < kGroup - k) slots[k + lane] = kBatch;
				flush_group<S>(acc, w_rows, slots, s_feat, lane);
				k = 0;
			}
		}
	}

	if (inside && slice == 0) {
		const int64_t pix = (int64_t)py * a.width + px;
		if constexpr (RGB) {
			a.image[pix * 3 + 0] = cr + T * a.background[0];
			a.image[pix * 3 + 1] = cg + T * a.background[1];
			a.image[pix * 3 + 2] = cb_ + T * a.background[2];
		}
		a.final_T[pix] = T;
		a.n_contrib[pix] = last;
	}
	if constexpr (S > 0) {
		// D layout of the 16x16 tile: lane holds channels 4*(lane>>4)+0..3 of pixel lane & 15.
#pragma unroll
		for (int m = 0; m < 4; m++) {
			const int p = 16 * m + (lane & 15);
			const int x = wx0 + (p & 7), y = wy0 + (p >> 3);
			if (x >= a.width || y >= a.height) continue;
			float* dst = a.feature_image + ((int64_t)y * a.width + x) * a.channels + c0 + 4 * (lane >> 4);
#pragma unroll
			for (int c = 0; c < kNcb; c++) {
				const hds_f32x4 v = acc[m][c];
				*reinterpret_cast<float4*>(dst + 16 * c) = make_float4(v[0], v[1], v[2], v[3]);
			}
		}
	}
}

template <int S, bool RGB>
int launch(const RenderArgs& a, int num_tiles, int slices, hipStream_t s) {
	render_forward_kernel<S, RGB><<<dim3((unsigned)num_tiles, (unsigned)slices), 256, 0, s>>>(a);
	return hds_check_launch(RGB ? (S > 0 ? "render_rgb_features" : "render_rgb") : "render_features", s);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int hds_render(int64_t n, int width, int height, int channels, const int32_t* tile_ranges,
						  const int32_t* values_sorted, int64_t num_pairs, const float* means2D, const float* conic4,
						  const float* color_opacity4, const float* background, const float* features, float* image,
						  float* final_T, int32_t* n_contrib, float* feature_image, hds_stream_t stream) {
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
	(void)n;
	const int tiles_x = (width + HDS_TILE - 1) / HDS_TILE, tiles_y = (height + HDS_TILE - 1) / HDS_TILE;
	const int num_tiles = tiles_x * tiles_y;
	RenderArgs a{width,
				 height,
				 tiles_x,
				 feats ? channels : 0,
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
				 feature_image};
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
