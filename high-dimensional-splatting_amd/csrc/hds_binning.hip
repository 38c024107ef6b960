// Tile binning: cull + tile rectangles, depth order, pair emission, (tile, depth) order, ranges.
//
// The reference emits P (tile, gaussian) pairs with 64-bit keys (tile << 32 | depth bits) and
// radix-sorts all of them on 32 + ceil(log2 T) bits (forward.cu:82-113, 363-394). Here the same
// order is built in two cheaper steps:
//   1. stable radix sort of the N gaussians by the 32-bit depth key (ties keep index order),
//   2. pairs emitted in that depth order, then stable radix sort of the P pairs by tile id alone
//      (ceil(log2 T) bits: 12 at 979x546, so 2 passes of 8 bits instead of 6).
// Stability of both sorts gives exactly the reference's (tile, depth bits, index) order, so
// values_sorted and tile_ranges equal the CPU oracle's bit for bit, and the pair sort moves
// 8 B per pair and pass instead of 12. Everything is integer work; the only floating point is the
// shared tile rectangle of hds_common.h.
//
// Scans and sorts are written for wave64: ranks inside a wave come from ballot-based digit
// matching (no shuffles, no LDS atomics on a hot bin), and blocks own 4096 consecutive items.
#include "hds_internal.h"
#include "hds_rasterizer.h"

namespace {

constexpr int kThreads = 256;
constexpr int kItemsPerThread = 16;
constexpr int kTileItems = kThreads * kItemsPerThread;  // items one block owns
constexpr int kRadixBits = 8;
constexpr int kRadix = 1 << kRadixBits;
constexpr int kWaves = kThreads / HDS_WAVE;

static_assert(kRadix == kThreads, "one thread per radix bin");

inline int64_t tiles_of(int64_t n) { return (n + kTileItems - 1) / kTileItems; }

// ---------------------------------------------------------------------------------------------
// Exclusive prefix sum of uint32 values, optionally gathered through an index array
// (out[i] = sum_{j<i} in[idx[j]]), in three launches: block sums, one-block scan of the sums,
// block-local scans plus the block offset. The grand total goes to *total as uint64.
// ---------------------------------------------------------------------------------------------

__device__ inline uint32_t scan_load(const uint32_t* __restrict__ in, const uint32_t* __restrict__ idx, int64_t i) {
	return in[idx ? idx[i] : i];
}

// Exclusive scan across the block of one value per thread; also returns the block total.
__device__ inline uint32_t block_exclusive_scan(uint32_t v, uint32_t* s_wave, uint32_t& total) {
	const int lane = threadIdx.x & (HDS_WAVE - 1), wave = threadIdx.x / HDS_WAVE;
	uint32_t x = v;
#pragma unroll
	for (int off = 1; off < HDS_WAVE; off <<= 1) {
		const uint32_t y = __shfl_up(x, off, HDS_WAVE);
		if (lane >= off) x += y;
	}
	if (lane == HDS_WAVE - 1) s_wave[wave] = x;
	__syncthreads();
	uint32_t before = 0, sum = 0;
#pragma unroll
	for (int w = 0; w < kWaves; w++) {
		const uint32_t t = s_wave[w];
		if (w < wave) before += t;
		sum += t;
	}
	__syncthreads();
	total = sum;
	return before + x - v;
}

__global__ __launch_bounds__(kThreads) void scan_reduce_kernel(const uint32_t* __restrict__ in,
																const uint32_t* __restrict__ idx, int64_t n,
																uint32_t* __restrict__ sums) {
	__shared__ uint32_t s_wave[kWaves];
	const int64_t base = (int64_t)blockIdx.x * kTileItems;
	uint32_t v = 0;
#pragma unroll 4
	for (int r = 0; r < kItemsPerThread; r++) {
		const int64_t i = base + r * kThreads + threadIdx.x;
		if (i < n) v += scan_load(in, idx, i);
	}
	uint32_t total;
	block_exclusive_scan(v, s_wave, total);
	if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// Single work-group exclusive scan of the block sums, in place; total as uint64.
__global__ __launch_bounds__(1024) void scan_top_kernel(uint32_t* __restrict__ sums, int64_t count,
														uint64_t* __restrict__ total) {
	__shared__ uint32_t s_wave[1024 / HDS_WAVE];
	__shared__ uint64_t s_carry;
	const int lane = threadIdx.x & (HDS_WAVE - 1), wave = threadIdx.x / HDS_WAVE;
	if (threadIdx.x == 0) s_carry = 0;
	__syncthreads();
	for (int64_t base = 0; base < count; base += 1024) {
		const int64_t i = base + threadIdx.x;
		const uint32_t v = i < count ? sums[i] : 0u;
		uint32_t x = v;
#pragma unroll
		for (int off = 1; off < HDS_WAVE; off <<= 1) {
			const uint32_t y = __shfl_up(x, off, HDS_WAVE);
			if (lane >= off) x += y;
		}
		if (lane == HDS_WAVE - 1) s_wave[wave] = x;
		__syncthreads();
		uint64_t before = 0, sum = 0;
		for (int w = 0; w < 1024 / HDS_WAVE; w++) {
			if (w < wave) before += s_wave[w];
			sum += s_wave[w];
		}
		const uint64_t carry = s_carry;
		if (i < count) sums[i] = (uint32_t)(carry + before + x - v);
		__syncthreads();
		if (threadIdx.x == 0) s_carry = carry + sum;
		__syncthreads();
	}
	if (threadIdx.x == 0 && total) *total = s_carry;
}

__global__ __launch_bounds__(kThreads) void scan_apply_kernel(const uint32_t* __restrict__ in,
															   const uint32_t* __restrict__ idx, int64_t n,
															   const uint32_t* __restrict__ sums,
															   uint32_t* __restrict__ out) {
	// Items go through LDS so that global loads and stores stay coalesced while each thread
	// scans 16 consecutive items; a pad word every 16 keeps the strided LDS reads conflict-free.
	__shared__ uint32_t s_items[kTileItems + kTileItems / 16];
	__shared__ uint32_t s_wave[kWaves];
	const int64_t base = (int64_t)blockIdx.x * kTileItems;
#pragma unroll 4
	for (int r = 0; r < kItemsPerThread; r++) {
		const int j = r * kThreads + threadIdx.x;
		const int64_t i = base + j;
		s_items[j + j / 16] = i < n ? scan_load(in, idx, i) : 0u;
	}
	__syncthreads();
	uint32_t local[kItemsPerThread];
	uint32_t sum = 0;
	const int first = threadIdx.x * kItemsPerThread;
#pragma unroll
	for (int k = 0; k < kItemsPerThread; k++) {
		local[k] = sum;
		sum += s_items[first + k + (first + k) / 16];
	}
	uint32_t total;
	const uint32_t before = block_exclusive_scan(sum, s_wave, total) + sums[blockIdx.x];
#pragma unroll
	for (int k = 0; k < kItemsPerThread; k++) s_items[first + k + (first + k) / 16] = local[k] + before;
	__syncthreads();
#pragma unroll 4
	for (int r = 0; r < kItemsPerThread; r++) {
		const int j = r * kThreads + threadIdx.x;
		const int64_t i = base + j;
		if (i < n) out[i] = s_items[j + j / 16];
	}
}

int exclusive_scan(const uint32_t* in, const uint32_t* idx, int64_t n, uint32_t* out, uint32_t* sums,
				   uint64_t* total, hipStream_t s) {
	const int64_t blocks = tiles_of(n);
	HdsKernelTimer timer1("scan_reduce_kernel", s);
	scan_reduce_kernel<<<(unsigned)blocks, kThreads, 0, s>>>(in, idx, n, sums);
	timer1.stop();
	HDS_LAUNCH_CHECK("scan_reduce", s);
	HdsKernelTimer timer2("scan_top_kernel", s);
	scan_top_kernel<<<1, 1024, 0, s>>>(sums, blocks, total);
	timer2.stop();
	HDS_LAUNCH_CHECK("scan_top", s);
	HdsKernelTimer timer3("scan_apply_kernel", s);
	scan_apply_kernel<<<(unsigned)blocks, kThreads, 0, s>>>(in, idx, n, sums, out);
	timer3.stop();
	HDS_LAUNCH_CHECK("scan_apply", s);
	return HDS_OK;
}

// ---------------------------------------------------------------------------------------------
// Stable LSD radix sort of (uint32 key, uint32 value) pairs, 8 bits per pass.
// Pass = per-block digit histograms (digit-major) -> exclusive scan -> stable scatter.
// ---------------------------------------------------------------------------------------------

// Lanes of this wave (among `active`) whose digit equals ours.
__device__ inline uint64_t match_digit(uint32_t d, uint64_t active) {
	uint64_t peers = active;
#pragma unroll
	for (int b = 0; b < kRadixBits; b++) {
		const bool bit = (d >> b) & 1u;
		const uint64_t m = hds_ballot(bit);
		peers &= bit ? m : ~m;
	}
	return peers;
}

__global__ __launch_bounds__(kThreads) void radix_hist_kernel(const uint32_t* __restrict__ keys, int64_t n, int shift,
															   uint32_t num_blocks, uint32_t* __restrict__ hist) {
	__shared__ uint32_t s_hist[kRadix];
	s_hist[threadIdx.x] = 0;
	__syncthreads();
	const int64_t base = (int64_t)blockIdx.x * kTileItems;
	for (int r = 0; r < kItemsPerThread; r++) {
		const int64_t row = base + (int64_t)r * kThreads;
		if (row >= n) break;
		const int64_t i = row + threadIdx.x;
		const bool valid = i < n;
		const uint32_t d = valid ? (keys[i] >> shift) & (kRadix - 1) : 0u;
		const uint64_t peers = match_digit(d, hds_ballot(valid));
		if (valid && hds_rank_below(peers) == 0) atomicAdd(&s_hist[d], (uint32_t)__popcll(peers));
	}
	__syncthreads();
	hist[(int64_t)threadIdx.x * num_blocks + blockIdx.x] = s_hist[threadIdx.x];
}

__global__ __launch_bounds__(kThreads) void radix_scatter_kernel(const uint32_t* __restrict__ keys_in,
																  const uint32_t* __restrict__ vals_in,
																  uint32_t* __restrict__ keys_out,
																  uint32_t* __restrict__ vals_out, int64_t n,
																  int shift, uint32_t num_blocks,
																  const uint32_t* __restrict__ offsets) {
	__shared__ uint32_t s_running[kRadix];
	__shared__ uint32_t s_wave_count[kWaves][kRadix];
	const int wave = threadIdx.x / HDS_WAVE;
	s_running[threadIdx.x] = offsets[(int64_t)threadIdx.x * num_blocks + blockIdx.x];
#pragma unroll
	for (int w = 0; w < kWaves; w++) s_wave_count[w][threadIdx.x] = 0;
	__syncthreads();
	const int64_t base = (int64_t)blockIdx.x * kTileItems;
	for (int r = 0; r < kItemsPerThread; r++) {
		const int64_t row = base + (int64_t)r * kThreads;
		if (row >= n) break;
		const int64_t i = row + threadIdx.x;
		const bool valid = i < n;
		const uint32_t key = valid ? keys_in[i] : 0u;
		const uint32_t val = valid ? vals_in[i] : 0u;
		const uint32_t d = (key >> shift) & (kRadix - 1);
		const uint64_t peers = match_digit(d, hds_ballot(valid));
		const int rank = hds_rank_below(peers);
		if (valid && rank == 0) s_wave_count[wave][d] = (uint32_t)__popcll(peers);
		__syncthreads();
		if (valid) {
			uint32_t pos = s_running[d] + (uint32_t)rank;
			for (int w = 0; w < wave; w++) pos += s_wave_count[w][d];
			if (keys_out) keys_out[pos] = key;
			vals_out[pos] = val;
		}
		__syncthreads();
		uint32_t add = 0;
#pragma unroll
		for (int w = 0; w < kWaves; w++) {
			add += s_wave_count[w][threadIdx.x];
			s_wave_count[w][threadIdx.x] = 0;
		}
		s_running[threadIdx.x] += add;
		__syncthreads();
	}
}

// Sorts (keys, vals) on bits [0, bits) through the buffers a (input) and b; returns in *out_a
// whether the result ended in a (even pass count) or b. keys_final_needed=false lets the last
// pass skip writing keys.
int radix_sort(uint32_t* keys_a, uint32_t* vals_a, uint32_t* keys_b, uint32_t* vals_b, int64_t n, int bits,
			   uint32_t* hist, uint32_t* sums, bool keys_final_needed, hipStream_t s) {
	const int64_t blocks = tiles_of(n);
	const int passes = (bits + kRadixBits - 1) / kRadixBits;
	uint32_t *kin = keys_a, *vin = vals_a, *kout = keys_b, *vout = vals_b;
	for (int p = 0; p < passes; p++) {
		HdsKernelTimer timer4("radix_hist_kernel", s);
		radix_hist_kernel<<<(unsigned)blocks, kThreads, 0, s>>>(kin, n, p * kRadixBits, (uint32_t)blocks, hist);
		timer4.stop();
		HDS_LAUNCH_CHECK("radix_hist", s);
		int st = exclusive_scan(hist, nullptr, (int64_t)kRadix * blocks, hist, sums, nullptr, s);
		if (st != HDS_OK) return st;
		const bool last = p == passes - 1;
		HdsKernelTimer timer5("radix_scatter_kernel", s);
		radix_scatter_kernel<<<(unsigned)blocks, kThreads, 0, s>>>(kin, vin, (last && !keys_final_needed) ? nullptr : kout,
																   vout, n, p * kRadixBits, (uint32_t)blocks, hist);
		timer5.stop();
		HDS_LAUNCH_CHECK("radix_scatter", s);
		uint32_t* t;
		t = kin; kin = kout; kout = t;
		t = vin; vin = vout; vout = t;
	}
	return HDS_OK;
}

// ---------------------------------------------------------------------------------------------
// Binning kernels.
// ---------------------------------------------------------------------------------------------

// Cull, tile rectangle, packed records, tile count and depth key per gaussian (forward.cu:13-61).
__global__ __launch_bounds__(kThreads) void prepare_kernel(
	int64_t n, const float* __restrict__ means2D, const float* __restrict__ depths, const float* __restrict__ radii,
	const float* __restrict__ conics, const float* __restrict__ colors, const float* __restrict__ opacities,
	int tiles_x, int tiles_y, float4* __restrict__ conic4, float4* __restrict__ color_opacity4,
	uint32_t* __restrict__ counts, uint2* __restrict__ rects, uint32_t* __restrict__ depth_keys,
	uint32_t* __restrict__ order) {
	const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
	if (i >= n) return;
	const float radius = radii[i];
	const float op = opacities[i];
	const float a = conics[i * 3], b = conics[i * 3 + 1], c = conics[i * 3 + 2];
	const float ux = means2D[i * 2], uy = means2D[i * 2 + 1];
	conic4[i] = make_float4(a, b, c, op);
	if (colors) color_opacity4[i] = make_float4(colors[i * 3], colors[i * 3 + 1], colors[i * 3 + 2], op);
	int x0 = 0, y0 = 0, w = 0, h = 0;
	// !(radius > 0) culls NaN radii too (forward.cu:31-37).
	const bool ok = radius > 0.0f && hds_tile_rect(ux, uy, a, b, c, op, tiles_x, tiles_y, &x0, &y0, &w, &h);
	counts[i] = ok ? (uint32_t)(w * h) : 0u;
	rects[i] = ok ? make_uint2((uint32_t)x0 | ((uint32_t)y0 << 16), (uint32_t)w | ((uint32_t)h << 16)) : make_uint2(0u, 0u);
	depth_keys[i] = hds_f2u(depths[i]);
	order[i] = (uint32_t)i;
}

// One thread per output pair: the owning gaussian is the last depth-ordered entry whose offset is
// <= the pair index (gaussians with no tiles share their successor's offset and are skipped);
// tiles are enumerated row-major inside the rectangle (forward.cu:63-113).
__global__ __launch_bounds__(kThreads) void emit_kernel(int64_t n, int64_t num_pairs, const uint32_t* __restrict__ offsets,
														 const uint32_t* __restrict__ order,
														 const uint2* __restrict__ rects, int tiles_x,
														 uint32_t* __restrict__ tile_keys, uint32_t* __restrict__ gids) {
	const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
	if (p >= num_pairs) return;
	const uint32_t target = (uint32_t)p;
	int64_t lo = 0, hi = n - 1;
	while (lo < hi) {
		const int64_t mid = (lo + hi + 1) >> 1;
		if (offsets[mid] <= target)
			lo = mid;
		else
			hi = mid - 1;
	}
	const uint32_t gid = order[lo];
	const uint2 r = rects[gid];
	const uint32_t x0 = r.x & 0xffffu, y0 = r.x >> 16, w = r.y & 0xffffu;
	const uint32_t local = target - offsets[lo];
	const uint32_t ty = y0 + local / w, tx = x0 + local % w;
	tile_keys[p] = ty * (uint32_t)tiles_x + tx;
	gids[p] = gid;
}

__global__ __launch_bounds__(kThreads) void fill_kernel(uint32_t* __restrict__ out, int64_t count, uint32_t value) {
	const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
	if (i < count) out[i] = value;
}

// [start, end) of each tile in the sorted pair list (forward.cu:115-139).
__global__ __launch_bounds__(kThreads) void ranges_kernel(int64_t num_pairs, const uint32_t* __restrict__ tile_keys,
														   int2* __restrict__ ranges) {
	const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
	if (p >= num_pairs) return;
	const uint32_t t = tile_keys[p];
	if (p == 0 || tile_keys[p - 1] != t) ranges[t].x = (int)p;
	if (p == num_pairs - 1 || tile_keys[p + 1] != t) ranges[t].y = (int)(p + 1);
}

// ---------------------------------------------------------------------------------------------
// Workspace layouts. Every region is 256-byte aligned.
// ---------------------------------------------------------------------------------------------

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct GaussianSpace {
	size_t counts, rects, keys_a, vals_a, keys_b, vals_b, offsets, hist, sums, total, bytes;
};

GaussianSpace gaussian_space(int64_t n) {
	GaussianSpace g;
	const size_t items = (size_t)(n > 0 ? n : 1);
	const int64_t blocks = tiles_of(items);
	const int64_t scan_items = std::max<int64_t>((int64_t)items, (int64_t)kRadix * blocks);
	size_t o = 0;
	g.counts = o; o = align256(o + 4 * items);
	g.rects = o; o = align256(o + 8 * items);
	g.keys_a = o; o = align256(o + 4 * items);
	g.vals_a = o; o = align256(o + 4 * items);
	g.keys_b = o; o = align256(o + 4 * items);
	g.vals_b = o; o = align256(o + 4 * items);
	g.offsets = o; o = align256(o + 4 * items);
	g.hist = o; o = align256(o + 4 * (size_t)kRadix * blocks);
	g.sums = o; o = align256(o + 4 * (size_t)tiles_of(scan_items));
	g.total = o; o = align256(o + 8);
	g.bytes = o;
	return g;
}

struct PairSpace {
	size_t keys_a, keys_b, vals_tmp, hist, sums, bytes;
};

PairSpace pair_space(int64_t num_pairs) {
	PairSpace p;
	const size_t items = (size_t)(num_pairs > 0 ? num_pairs : 1);
	const int64_t blocks = tiles_of(items);
	const int64_t scan_items = std::max<int64_t>((int64_t)items, (int64_t)kRadix * blocks);
	size_t o = 0;
	p.keys_a = o; o = align256(o + 4 * items);
	p.keys_b = o; o = align256(o + 4 * items);
	p.vals_tmp = o; o = align256(o + 4 * items);
	p.hist = o; o = align256(o + 4 * (size_t)kRadix * blocks);
	p.sums = o; o = align256(o + 4 * (size_t)tiles_of(scan_items));
	p.bytes = o;
	return p;
}

template <typename T>
T* at(void* base, size_t offset) {
	return reinterpret_cast<T*>(static_cast<char*>(base) + offset);
}

int tile_bits(int64_t num_tiles) {
	int bits = 0;
	while ((int64_t(1) << bits) < num_tiles) bits++;
	return bits;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" size_t hds_bin_workspace_bytes(int64_t n, int width, int height) {
	(void)width;
	(void)height;
	return gaussian_space(n).bytes;
}

extern "C" size_t hds_pairs_workspace_bytes(int64_t num_pairs, int width, int height) {
	(void)width;
	(void)height;
	return pair_space(num_pairs).bytes;
}

extern "C" int hds_bin_count(int64_t n, const float* means2D, const float* depths, const float* radii,
							 const float* conics, const float* colors, const float* opacities, int width, int height,
							 float* conic4, float* color_opacity4, void* workspace, size_t workspace_bytes,
							 int64_t* num_pairs, hds_stream_t stream) {
	HDS_REQUIRE(num_pairs, "bin_count: num_pairs must not be NULL");
	*num_pairs = 0;
	HDS_REQUIRE(n >= 0 && n < INT32_MAX, "bin_count: gaussian count %lld outside [0, 2^31)", (long long)n);
	HDS_REQUIRE(width > 0 && height > 0, "bin_count: image size %dx%d must be positive", width, height);
	const int tiles_x = (width + HDS_TILE - 1) / HDS_TILE, tiles_y = (height + HDS_TILE - 1) / HDS_TILE;
	HDS_REQUIRE(tiles_x < 65536 && tiles_y < 65536, "bin_count: image %dx%d has too many tiles", width, height);
	if (n == 0) return HDS_OK;
	const GaussianSpace g = gaussian_space(n);
	HDS_REQUIRE(workspace && workspace_bytes >= g.bytes, "bin_count: workspace of %zu bytes, need %zu",
				workspace_bytes, g.bytes);
	HDS_REQUIRE(means2D && depths && radii && conics && opacities && conic4, "bin_count: null pointer argument");
	HDS_REQUIRE(colors == nullptr || color_opacity4 != nullptr, "bin_count: colors given without color_opacity4");
	HDS_REQUIRE(aligned16(conic4) && (!color_opacity4 || aligned16(color_opacity4)),
				"bin_count: conic4 / color_opacity4 must be 16-byte aligned");
	hipStream_t s = (hipStream_t)stream;

	uint32_t* counts = at<uint32_t>(workspace, g.counts);
	uint2* rects = at<uint2>(workspace, g.rects);
	uint32_t* keys_a = at<uint32_t>(workspace, g.keys_a);
	uint32_t* vals_a = at<uint32_t>(workspace, g.vals_a);
	uint32_t* keys_b = at<uint32_t>(workspace, g.keys_b);
	uint32_t* vals_b = at<uint32_t>(workspace, g.vals_b);
	uint32_t* offsets = at<uint32_t>(workspace, g.offsets);
	uint32_t* hist = at<uint32_t>(workspace, g.hist);
	uint32_t* sums = at<uint32_t>(workspace, g.sums);
	uint64_t* total = at<uint64_t>(workspace, g.total);

	HdsKernelTimer timer6("prepare_kernel", s);
	prepare_kernel<<<hds_blocks(n, kThreads), kThreads, 0, s>>>(
		n, means2D, depths, radii, conics, colors, opacities, tiles_x, tiles_y, reinterpret_cast<float4*>(conic4),
		reinterpret_cast<float4*>(color_opacity4), counts, rects, keys_a, vals_a);
	timer6.stop();
	HDS_LAUNCH_CHECK("prepare_gaussians", s);
	// 4 passes: the depth order ends back in (keys_a, vals_a).
	int st = radix_sort(keys_a, vals_a, keys_b, vals_b, n, 32, hist, sums, false, s);
	if (st != HDS_OK) return st;
	st = exclusive_scan(counts, vals_a, n, offsets, sums, total, s);
	if (st != HDS_OK) return st;
	uint64_t host_total = 0;
	HDS_HIP(hipMemcpyAsync(&host_total, total, sizeof(host_total), hipMemcpyDeviceToHost, s));
	HDS_HIP(hipStreamSynchronize(s));
	HDS_REQUIRE(host_total < (uint64_t)INT32_MAX, "bin_count: %llu tile-gaussian pairs overflow int32 indices",
				(unsigned long long)host_total);
	*num_pairs = (int64_t)host_total;
	return HDS_OK;
}

extern "C" int hds_bin_emit(int64_t n, int64_t num_pairs, int width, int height, const void* workspace,
							void* pairs_workspace, size_t pairs_workspace_bytes, int32_t* values_sorted,
							int32_t* tile_ranges, hds_stream_t stream) {
	HDS_REQUIRE(width > 0 && height > 0, "bin_emit: image size %dx%d must be positive", width, height);
	HDS_REQUIRE(num_pairs >= 0 && num_pairs < INT32_MAX, "bin_emit: pair count %lld outside [0, 2^31)",
				(long long)num_pairs);
	HDS_REQUIRE(tile_ranges, "bin_emit: tile_ranges must not be NULL");
	const int tiles_x = (width + HDS_TILE - 1) / HDS_TILE, tiles_y = (height + HDS_TILE - 1) / HDS_TILE;
	const int64_t num_tiles = (int64_t)tiles_x * tiles_y;
	hipStream_t s = (hipStream_t)stream;
	HdsKernelTimer timer7("fill_kernel", s);
	fill_kernel<<<hds_blocks(2 * num_tiles, kThreads), kThreads, 0, s>>>(reinterpret_cast<uint32_t*>(tile_ranges),
																		  2 * num_tiles, 0u);
	timer7.stop();
	HDS_LAUNCH_CHECK("fill_tile_ranges", s);
	if (num_pairs == 0) return HDS_OK;
	const PairSpace p = pair_space(num_pairs);
	HDS_REQUIRE(pairs_workspace && pairs_workspace_bytes >= p.bytes, "bin_emit: pairs workspace of %zu bytes, need %zu",
				pairs_workspace_bytes, p.bytes);
	HDS_REQUIRE(workspace && values_sorted && n > 0, "bin_emit: null pointer argument");
	const GaussianSpace g = gaussian_space(n);
	void* ws = const_cast<void*>(workspace);
	const uint32_t* offsets = at<uint32_t>(ws, g.offsets);
	const uint32_t* order = at<uint32_t>(ws, g.vals_a);
	const uint2* rects = at<uint2>(ws, g.rects);

	uint32_t* keys_a = at<uint32_t>(pairs_workspace, p.keys_a);
	uint32_t* keys_b = at<uint32_t>(pairs_workspace, p.keys_b);
	uint32_t* vals_tmp = at<uint32_t>(pairs_workspace, p.vals_tmp);
	uint32_t* hist = at<uint32_t>(pairs_workspace, p.hist);
	uint32_t* sums = at<uint32_t>(pairs_workspace, p.sums);
	uint32_t* out = reinterpret_cast<uint32_t*>(values_sorted);

	// Pick the ping-pong buffers so the last pass lands in values_sorted.
	const int bits = tile_bits(num_tiles);
	const int passes = (bits + kRadixBits - 1) / kRadixBits;
	uint32_t* vals_a = (passes % 2 == 0) ? out : vals_tmp;
	uint32_t* vals_b = (passes % 2 == 0) ? vals_tmp : out;

	HdsKernelTimer timer8("emit_kernel", s);
	emit_kernel<<<hds_blocks(num_pairs, kThreads), kThreads, 0, s>>>(n, num_pairs, offsets, order, rects, tiles_x,
																	  keys_a, vals_a);
	timer8.stop();
	HDS_LAUNCH_CHECK("emit_pairs", s);
	int st = radix_sort(keys_a, vals_a, keys_b, vals_b, num_pairs, bits, hist, sums, true, s);
	if (st != HDS_OK) return st;
	const uint32_t* keys_sorted = (passes % 2 == 0) ? keys_a : keys_b;
	HdsKernelTimer timer9("ranges_kernel", s);
	ranges_kernel<<<hds_blocks(num_pairs, kThreads), kThreads, 0, s>>>(num_pairs, keys_sorted,
																		reinterpret_cast<int2*>(tile_ranges));
	timer9.stop();
	HDS_LAUNCH_CHECK("identify_tile_ranges", s);
	return HDS_OK;
}
