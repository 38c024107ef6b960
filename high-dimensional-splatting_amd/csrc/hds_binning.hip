// Tile binning: cull + tile rectangles, depth order, pair emission, (tile, depth) order, ranges.
//
// The reference emits P (tile, gaussian) pairs with 64-bit keys (tile << 32 | depth bits) and
// radix-sorts all of them on 32 + ceil(log2 T) bits (forward.cu:82-113, 363-394). Here the same
// order is built in two cheaper steps:
//   1. stable radix sort of the N gaussians by the 32-bit depth key (ties keep index order),
//   2. pairs emitted in that depth order, then stable radix sort of the P pairs by tile id alone
//      (ceil(log2 T) bits: 12 at 979x546, so 2 passes of 6 bits instead of 6 passes of 8).
// Stability of both sorts gives exactly the reference's (tile, depth bits, index) order, so
// values_sorted and tile_ranges equal the CPU oracle's bit for bit, and the pair sort moves
// 8 B per pair and pass instead of 12. The tile-order variant (the autograd path) skips step 1
// and needs no pair sort at all: each chunk of 4096 gaussians counts its pairs per tile in LDS
// (one column of a tile-major count matrix), one exclusive scan of that matrix gives every
// (tile, chunk) run its place in the tile-major pair list and tile_ranges, and each chunk then
// scatters its pairs into its runs (counting scatter); each tile's list is finally sorted by
// (depth bits, index) in one work-group (tile_sort_kernel), the same order again. Frames whose
// count matrix would exceed 2^24 words take the emit + pair sort by tile instead. Everything is
// integer work; the only floating point is the shared tile rectangle of hds_common.h.
//
// Sorts and scans are single-pass: every radix pass is ONE launch in which each work-group ranks
// its 4096-item partition in registers and LDS, publishes its per-digit counts, and reads the
// counts of the partitions before it from a status array (decoupled look-back), so no separate
// histogram / scan launches sit between passes. Partitions are handed out in launch order by an
// atomic ticket, which is what makes the look-back safe: a work-group only ever waits for
// partitions whose owners are already running and never wait themselves before publishing. The
// digit histograms every pass needs up front come from the kernel that produces the keys
// (prepare for depths, emit for tile ids). The whole binning is 11 launches.
#include <atomic>
#include <mutex>
#include <vector>

#include "hds_internal.h"
#include "hds_rasterizer.h"

namespace {

constexpr int kThreads = 256;
constexpr int kItemsPerThread = 16;
constexpr int kTileItems = kThreads * kItemsPerThread;  // items one partition / work-group owns
constexpr int kWaves = kThreads / HDS_WAVE;
constexpr int kRadixBits = 8;
constexpr int kRadix = 1 << kRadixBits;
constexpr int kMaxPasses = 4;                           // 32-bit keys
// Copies of each global digit histogram: producers add into copy (block mod kHistCopies), so that
// no histogram word takes more than ~1/16 of the producers' atomics; passes sum the copies.
constexpr int kHistCopies = 16;
constexpr int kHistWords = kHistCopies * kRadix;        // one pass's histogram copies
// Polls of a silent predecessor before a look-back gives up and raises the error flag (seconds of
// waiting; reached only if a launch is broken, never by a slow but running predecessor). Tests of
// the failure path set it from the host (hds_set_lookback_limit): 0 makes every look-back give up
// before its first poll, so the failure is certain while every kernel still runs to its end.
constexpr uint32_t kSpinLimit = HDS_LOOKBACK_LIMIT_DEFAULT;
std::atomic<uint32_t> g_spin_limit{kSpinLimit};
// Counting scatter of the tile-order binning: one work-group of kScatterThreads threads per chunk of
// kChunk gaussians, with an LDS histogram of up to kHistBins tiles at a time. Workspaces reserve the
// count matrix (chunks x tiles words) when it stays within kScatterWords; a test hook can only
// lower the limit the path choice uses (hds_set_tile_scatter_limit), so a workspace always holds
// what the chosen path needs.
constexpr int kScatterThreads = 1024;
constexpr int kScatterWaves = kScatterThreads / HDS_WAVE;
constexpr int kChunk = 4 * kScatterThreads;
constexpr int kHistBins = 8192;
constexpr uint64_t kScatterWords = uint64_t(1) << 24;
std::atomic<uint64_t> g_scatter_words{kScatterWords};

static_assert(kRadix == kThreads, "one thread per radix bin");

__host__ __device__ inline int64_t parts_of(int64_t n) { return (n + kTileItems - 1) / kTileItems; }

// Item count of a launch sized on the host for `cap` items whose actual count sits in device
// memory: min(*total, cap), or 0 when the error word that follows *total is set (a failed
// look-back upstream leaves nothing trustworthy to emit). A null total means cap is exact.
__device__ inline int64_t device_count(const uint64_t* total, int64_t cap) {
	if (!total) return cap;
	if (reinterpret_cast<const uint32_t*>(total + 1)[0] != 0u) return 0;
	const uint64_t t = *total;
	return t < (uint64_t)cap ? (int64_t)t : cap;
}

// ---------------------------------------------------------------------------------------------
// Decoupled look-back. A status word is (flag << 56 | value): flag 2e+1 = the partition's own
// count (aggregate) of epoch e, 2e+2 = inclusive prefix through that partition; anything lower is
// "not yet". Epochs let one zeroed array serve all radix passes of a sort in turn.
// ---------------------------------------------------------------------------------------------

constexpr uint64_t kValueMask = (uint64_t(1) << 56) - 1;

__device__ inline uint64_t status_word(uint32_t flag, uint64_t value) { return ((uint64_t)flag << 56) | value; }

__device__ inline uint64_t status_load(uint64_t* p) {
	return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline void status_store(uint64_t* p, uint64_t v) {
	__hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sum of the values that partitions [0, part) published in one column (status + p * stride):
// walks back from part - 1 adding aggregates until an inclusive prefix ends the walk. W words are
// loaded at a time, so a walk over many aggregates costs one memory latency per W partitions.
template <int W>
__device__ inline uint64_t lookback(uint64_t* status, int64_t stride, int64_t part, uint32_t epoch,
									uint32_t* error, uint32_t spin_limit) {
	const uint32_t agg = 2 * epoch + 1, inc = 2 * epoch + 2;
	uint64_t sum = 0;
	uint32_t spins = 0;
	int64_t p = part - 1;
	if (spin_limit == 0u) {
		// Failure-path test mode (set from the host): give up before the first poll.
		atomicOr(error, 1u);
		return 0;
	}
	while (p >= 0) {
		uint64_t v[W];
#pragma unroll
		for (int k = 0; k < W; k++) v[k] = p - k >= 0 ? status_load(status + (p - k) * stride) : status_word(inc, 0);
		int k = 0;
		for (; k < W; k++) {
			const uint32_t flag = (uint32_t)(v[k] >> 56);
			if (flag == inc) return sum + (v[k] & kValueMask);
			if (flag != agg) break;
			sum += v[k] & kValueMask;
		}
		p -= k;
		if (k > 0) {
			spins = 0;
			continue;
		}
		if (++spins > spin_limit) {
			atomicOr(error, 1u);
			return sum;
		}
		__builtin_amdgcn_s_sleep(2);
	}
	return sum;
}

// Single-column look-back walked by a whole wave (every lane of the wave calls it with the same
// arguments and gets the sum): each step loads the words of the 64 partitions before p at once, so
// the walk advances up to 64 partitions per memory latency. Status words written by work-groups on
// other XCDs are read at agent scope, which costs a trip past the L2, so the number of dependent
// steps is what a look-back's time is made of.
__device__ inline uint64_t wave_sum64(uint64_t v) {
#pragma unroll
	for (int off = 1; off < HDS_WAVE; off <<= 1)
		v += ((uint64_t)hds_lane_xor((uint32_t)(v >> 32), off) << 32) | hds_lane_xor((uint32_t)v, off);
	return v;
}

__device__ inline uint64_t lookback_wave(uint64_t* status, int64_t part, uint32_t epoch, uint32_t* error,
										 uint32_t spin_limit) {
	const uint32_t agg = 2 * epoch + 1, inc = 2 * epoch + 2;
	const int lane = threadIdx.x & (HDS_WAVE - 1);
	if (spin_limit == 0u) {
		// Failure-path test mode (set from the host): give up before the first poll.
		if (lane == 0) atomicOr(error, 1u);
		return 0;
	}
	uint64_t sum = 0;
	uint32_t spins = 0;
	int64_t p = part - 1;
	while (p >= 0) {
		// Lane l reads partition p - l; below partition 0 reads as an inclusive prefix of 0.
		const int64_t q = p - lane;
		const uint64_t v = q >= 0 ? status_load(status + q) : status_word(inc, 0);
		const uint32_t flag = (uint32_t)(v >> 56);
		const uint64_t inc_lanes = hds_ballot(flag == inc);
		const uint64_t unready_lanes = hds_ballot(flag != inc && flag != agg);
		const int first_inc = inc_lanes ? (int)__builtin_ctzll(inc_lanes) : HDS_WAVE;
		const int first_unready = unready_lanes ? (int)__builtin_ctzll(unready_lanes) : HDS_WAVE;
		if (first_inc < first_unready) return sum + wave_sum64(lane <= first_inc ? (v & kValueMask) : 0);
		// Lanes below the first unpublished word hold aggregates.
		sum += wave_sum64(lane < first_unready ? (v & kValueMask) : 0);
		p -= first_unready;
		if (first_unready > 0) {
			spins = 0;
			continue;
		}
		if (++spins > spin_limit) {
			if (lane == 0) atomicOr(error, 1u);
			return sum;
		}
		__builtin_amdgcn_s_sleep(2);
	}
	return sum;
}

// Partition index in launch order (the look-back's progress guarantee), broadcast through LDS.
__device__ inline int64_t take_ticket(uint32_t* ticket, int64_t* s_part) {
	if (threadIdx.x == 0) *s_part = (int64_t)atomicAdd(ticket, 1u);
	__syncthreads();
	return *s_part;
}

// ---------------------------------------------------------------------------------------------
// Block primitives.
// ---------------------------------------------------------------------------------------------

// Exclusive scan across the block of one value per thread; also returns the block total.
__device__ inline uint32_t block_exclusive_scan(uint32_t v, uint32_t* s_wave, uint32_t& total) {
	const int lane = threadIdx.x & (HDS_WAVE - 1), wave = threadIdx.x / HDS_WAVE;
	const uint32_t x = hds_wave_inclusive_scan(v);
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

// Lanes of this wave (among `active`) whose digit equals ours. Digits narrower than 8 bits have
// zero high bits in every lane, whose ballots then change nothing.
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

// Adds a valid key to the work-group's LDS digit histograms, one per pass: one LDS atomic per lane
// and pass. Lanes that share a digit serialise in the LDS, which still costs less than grouping them
// with ballots first (measured on the depth keys and on the tile keys of the stress scene).
__device__ inline void count_digits(uint32_t key, bool valid, int passes, int bits, uint32_t (*s_hist)[kRadix]) {
	if (!valid) return;
	const uint32_t mask = (1u << bits) - 1u;
	for (int p = 0; p < passes; p++) atomicAdd(&s_hist[p][(key >> (p * bits)) & mask], 1u);
}

// hist = [pass][kHistCopies][kRadix]; this work-group adds into copy blockIdx.x % kHistCopies.
__device__ inline void flush_digits(int passes, uint32_t (*s_hist)[kRadix], uint32_t* __restrict__ hist) {
	__syncthreads();
	uint32_t* copy = hist + (blockIdx.x % kHistCopies) * kRadix + threadIdx.x;
	for (int p = 0; p < passes; p++) {
		const uint32_t c = s_hist[p][threadIdx.x];
		if (c) atomicAdd(copy + p * kHistWords, c);
	}
}

// ---------------------------------------------------------------------------------------------
// One stable LSD radix pass over a digit of at most 8 bits, single launch.
// ---------------------------------------------------------------------------------------------

// digit_hist = this pass's kHistCopies digit histograms; status = [partitions][kRadix] look-back
// words. Item order inside a partition is (wave, row, lane): wave w owns items [w*1024, w*1024 +
// 1024). With kGather, the value is an index and the pass also writes gathered[pos] = table[value]
// (the depth sort's last pass carries each gaussian's tile rectangle into depth order this way).
template <bool kKeysOut, bool kGather, int kIPT>
__global__ __launch_bounds__(kThreads) void onesweep_kernel(const uint32_t* __restrict__ keys_in,
															 const uint32_t* __restrict__ vals_in,
															 uint32_t* __restrict__ keys_out,
															 uint32_t* __restrict__ vals_out, int64_t n,
															 const uint64_t* __restrict__ n_total, int pass, int bits,
															 const uint32_t* __restrict__ digit_hist,
															 uint64_t* status, uint32_t* ticket, uint32_t* error,
															 uint32_t spin_limit, const uint2* __restrict__ table,
															 uint2* __restrict__ gathered) {
	constexpr int kPartItems = kThreads * kIPT;         // items of one partition
	constexpr int kPartWaveItems = kPartItems / kWaves;  // a wave ranks kIPT rows of 64 consecutive items
	__shared__ uint32_t s_keys[kPartItems];
	__shared__ uint32_t s_vals[kPartItems];
	__shared__ uint32_t s_cnt[kWaves][kRadix];  // per-wave running counts, then per-wave offsets
	__shared__ uint32_t s_local[kRadix];        // first slot of each digit in the partition
	__shared__ uint32_t s_adj[kRadix];          // output index of slot j of digit d = s_adj[d] + j
	__shared__ uint32_t s_wave[kWaves];
	__shared__ int64_t s_part;
	const int t = threadIdx.x, lane = t & (HDS_WAVE - 1), wave = t / HDS_WAVE;
	// Digit p of a key is bits [p * bits, (p + 1) * bits): every pass of a sort has the same width,
	// at most 8 bits; digits above 2^bits never occur.
	const int shift = pass * bits;
	const uint32_t mask = (1u << bits) - 1u;
#pragma unroll
	for (int w = 0; w < kWaves; w++) s_cnt[w][t] = 0;
	const int64_t part = take_ticket(ticket, &s_part);
	// Launched for n items; with n_total the count is read here, and tickets past its last
	// partition leave at once (every partition the look-back waits for has a lower ticket).
	n = device_count(n_total, n);
	if (part >= (n + kPartItems - 1) / kPartItems) return;
	const int64_t base = part * kPartItems;
	const int64_t wbase = base + (int64_t)wave * kPartWaveItems;

	uint32_t key[kIPT], val[kIPT];
#pragma unroll
	for (int r = 0; r < kIPT; r++) {
		const int64_t i = wbase + r * HDS_WAVE + lane;
		key[r] = i < n ? keys_in[i] : 0u;
		val[r] = i < n ? vals_in[i] : 0u;
	}
	// Rank inside the wave: earlier rows' count of the digit (s_cnt, kept by each digit group's
	// first lane) plus the lanes below with the same digit. A wave's LDS accesses run in order, so
	// the read of row r + 1 sees the update of row r.
	uint32_t rank[kIPT];
#pragma unroll
	for (int r = 0; r < kIPT; r++) {
		const bool valid = wbase + r * HDS_WAVE + lane < n;
		const uint32_t d = (key[r] >> shift) & mask;
		const uint64_t peers = match_digit(d, hds_ballot(valid));
		const uint32_t below = (uint32_t)hds_rank_below(peers);
		const uint32_t before = s_cnt[wave][d];
		rank[r] = before + below;
		if (valid && below == 0) s_cnt[wave][d] = before + (uint32_t)__popcll(peers);
	}
	__syncthreads();

	// Thread t owns digit t: per-wave offsets, the partition's count, publication and look-back.
	uint32_t count = 0;
#pragma unroll
	for (int w = 0; w < kWaves; w++) {
		const uint32_t c = s_cnt[w][t];
		s_cnt[w][t] = count;
		count += c;
	}
	// Digits that cannot occur (t > mask) have no count to publish and no predecessors to wait for.
	const bool digit_used = (uint32_t)t <= mask;
	uint64_t* mine = status + part * kRadix + t;
	if (digit_used) status_store(mine, status_word(part == 0 ? 2 * pass + 2 : 2 * pass + 1, count));
	uint32_t digit_total = 0;
#pragma unroll
	for (int c = 0; c < kHistCopies; c++) digit_total += digit_hist[c * kRadix + t];
	uint32_t unused;
	const uint32_t digit_start = block_exclusive_scan(digit_total, s_wave, unused);
	const uint32_t local_start = block_exclusive_scan(count, s_wave, unused);
	uint64_t before = 0;
	if (part > 0 && digit_used) {
		before = lookback<8>(status + t, kRadix, part, (uint32_t)pass, error, spin_limit);
		status_store(mine, status_word(2 * pass + 2, before + count));
	}
	s_local[t] = local_start;
	s_adj[t] = digit_start + (uint32_t)before - local_start;
	__syncthreads();

	// Reorder the partition by digit in LDS, then write it out: consecutive threads write
	// consecutive output positions inside each digit's run.
#pragma unroll
	for (int r = 0; r < kIPT; r++) {
		if (wbase + r * HDS_WAVE + lane < n) {
			const uint32_t d = (key[r] >> shift) & mask;
			const uint32_t slot = s_local[d] + s_cnt[wave][d] + rank[r];
			s_keys[slot] = key[r];
			s_vals[slot] = val[r];
		}
	}
	__syncthreads();
	const int64_t items = n - base < kPartItems ? n - base : kPartItems;
#pragma unroll
	for (int r = 0; r < kIPT; r++) {
		const int j = r * kThreads + t;
		if (j < items) {
			const uint32_t k = s_keys[j];
			const uint32_t pos = s_adj[(k >> shift) & mask] + (uint32_t)j;
			// Always in range when the digit counts are right; the test keeps a failed look-back
			// (error flag raised) from writing outside the buffers.
			if (pos < n) {
				const uint32_t v = s_vals[j];
				if (kKeysOut) keys_out[pos] = k;
				vals_out[pos] = v;
				// A value is an index below n unless an earlier pass failed and left this slot
				// unwritten (stale memory): the table is read only inside its n entries.
				if (kGather) gathered[pos] = v < (uint64_t)n ? table[v] : make_uint2(0u, 0u);
			}
		}
	}
}

// Sorts (keys, vals) on `passes` digits of `bits` bits through the buffers a (input) and b; the result
// ends in a for an even pass count, else in b. n items, or device_count(n_total, n) with n_total. hist holds every pass's digit histograms (filled by
// the producer of the keys); status/tickets are zeroed. Keys of the last pass are written only
// if keys_final_needed; with table, the last pass also writes gathered[i] = table[vals[i]].
int onesweep_sort(uint32_t* keys_a, uint32_t* vals_a, uint32_t* keys_b, uint32_t* vals_b, int64_t n,
				  const uint64_t* n_total, int passes, int bits, const uint32_t* hist, uint64_t* status, uint32_t* tickets, uint32_t* error, bool keys_final_needed,
				  const uint2* table, uint2* gathered, hipStream_t s) {
	// Passes over more than 16M items take 8192-item partitions: half the tickets and look-back
	// steps (both are paid per partition); smaller ones keep 4096 so that the grid fills the chip.
	const bool large = n > (int64_t(1) << 24);
	const unsigned parts = (unsigned)(large ? (n + 2 * kTileItems - 1) / (2 * kTileItems) : parts_of(n));
	uint32_t *kin = keys_a, *vin = vals_a, *kout = keys_b, *vout = vals_b;
	for (int p = 0; p < passes; p++) {
		const bool last = p == passes - 1;
		const bool keys_out = !last || keys_final_needed;
		const uint32_t* h = hist + p * kHistWords;
		HdsKernelTimer timer("onesweep_kernel", s);
		if (last && table && large)
			onesweep_kernel<false, true, 2 * kItemsPerThread><<<parts, kThreads, 0, s>>>(kin, vin, nullptr, vout, n, n_total, p, bits, h,
																						  status, tickets + p, error, g_spin_limit.load(std::memory_order_relaxed), table, gathered);
		else if (last && table)
			onesweep_kernel<false, true, kItemsPerThread><<<parts, kThreads, 0, s>>>(kin, vin, nullptr, vout, n, n_total, p, bits, h, status,
																					  tickets + p, error, g_spin_limit.load(std::memory_order_relaxed), table, gathered);
		else if (keys_out && large)
			onesweep_kernel<true, false, 2 * kItemsPerThread><<<parts, kThreads, 0, s>>>(kin, vin, kout, vout, n, n_total, p, bits, h,
																						  status, tickets + p, error, g_spin_limit.load(std::memory_order_relaxed), nullptr, nullptr);
		else if (keys_out)
			onesweep_kernel<true, false, kItemsPerThread><<<parts, kThreads, 0, s>>>(kin, vin, kout, vout, n, n_total, p, bits, h, status,
																					  tickets + p, error, g_spin_limit.load(std::memory_order_relaxed), nullptr, nullptr);
		else if (large)
			onesweep_kernel<false, false, 2 * kItemsPerThread><<<parts, kThreads, 0, s>>>(kin, vin, nullptr, vout, n, n_total, p, bits, h,
																						   status, tickets + p, error, g_spin_limit.load(std::memory_order_relaxed), nullptr, nullptr);
		else
			onesweep_kernel<false, false, kItemsPerThread><<<parts, kThreads, 0, s>>>(kin, vin, nullptr, vout, n, n_total, p, bits, h, status,
																					   tickets + p, error, g_spin_limit.load(std::memory_order_relaxed), nullptr, nullptr);
		timer.stop();
		HDS_LAUNCH_CHECK("onesweep_radix_pass", s);
		uint32_t* t;
		t = kin; kin = kout; kout = t;
		t = vin; vin = vout; vout = t;
	}
	return HDS_OK;
}

// ---------------------------------------------------------------------------------------------
// Single-pass exclusive scan of the tile counts (w * h of each rectangle, in depth order):
// out[i] = sum_{j<i} count[j]; the grand total goes to *total.
// ---------------------------------------------------------------------------------------------

// kRects: the counts are the w * h of rectangles (in = uint2 rects); else plain words (in =
// uint32 counts, which may be `out` itself: a partition reads all its items before writing any).
template <bool kRects>
__global__ __launch_bounds__(kThreads) void scan_kernel(const void* in, int64_t n, uint32_t* out, uint64_t* status,
														 uint32_t* ticket, uint32_t* error, uint32_t spin_limit,
														 uint64_t* __restrict__ total) {
	// Items go through LDS so that global loads and stores stay coalesced while each thread
	// scans 16 consecutive items; a pad word every 16 keeps the strided LDS reads conflict-free.
	__shared__ uint32_t s_items[kTileItems + kTileItems / 16];
	__shared__ uint32_t s_wave[kWaves];
	__shared__ uint64_t s_before;
	__shared__ int64_t s_part;
	const int64_t part = take_ticket(ticket, &s_part);
	const int64_t base = part * kTileItems;
#pragma unroll 4
	for (int r = 0; r < kItemsPerThread; r++) {
		const int j = r * kThreads + threadIdx.x;
		const int64_t i = base + j;
		if constexpr (kRects) {
			const uint32_t wh = i < n ? static_cast<const uint2*>(in)[i].y : 0u;
			s_items[j + j / 16] = (wh & 0xffffu) * (wh >> 16);
		} else {
			s_items[j + j / 16] = i < n ? static_cast<const uint32_t*>(in)[i] : 0u;
		}
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
	uint32_t block_total;
	const uint32_t before_thread = block_exclusive_scan(sum, s_wave, block_total);
	if (threadIdx.x < HDS_WAVE) {
		// Wave 0 publishes the partition's total and walks the look-back together.
		const bool lead = threadIdx.x == 0;
		uint64_t before = 0;
		if (part == 0) {
			if (lead) status_store(status, status_word(2, block_total));
		} else {
			if (lead) status_store(status + part, status_word(1, block_total));
			before = lookback_wave(status, part, 0, error, spin_limit);
			if (lead) status_store(status + part, status_word(2, before + block_total));
		}
		if (lead) {
			if (base + kTileItems >= n) *total = before + block_total;
			s_before = before;
		}
	}
	__syncthreads();
	const uint32_t offset = (uint32_t)s_before + before_thread;
#pragma unroll
	for (int k = 0; k < kItemsPerThread; k++) s_items[first + k + (first + k) / 16] = local[k] + offset;
	__syncthreads();
#pragma unroll 4
	for (int r = 0; r < kItemsPerThread; r++) {
		const int j = r * kThreads + threadIdx.x;
		const int64_t i = base + j;
		if (i < n) out[i] = s_items[j + j / 16];
	}
}

// ---------------------------------------------------------------------------------------------
// Binning kernels.
// ---------------------------------------------------------------------------------------------

// Cull, tile rectangle (its w * h is the tile count), packed records and depth key per gaussian
// (forward.cu:13-61), plus the depth keys' four digit histograms for the sort.
// Word ranges a kernel clears on the side (grid-stride over its whole grid), so that zeroing the
// control blocks of a binning costs no launch of its own.
struct ZeroRanges {
	uint32_t* p[3];
	int64_t n[3];
};

__device__ inline void zero_ranges(const ZeroRanges& z) {
	const int64_t stride = (int64_t)gridDim.x * blockDim.x;
#pragma unroll
	for (int k = 0; k < 3; k++)
		for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < z.n[k]; i += stride) z.p[k][i] = 0u;
}

// The per-gaussian records of both binnings: the conic (and colour) packed with the opacity, the
// tile rectangle ((x0 | y0 << 16), (w | h << 16)), zero for a culled gaussian, and the depth key.
struct GaussianInputs {
	const float* means2D;
	const float* depths;
	const float* radii;
	const float* conics;
	const float* colors;
	const float* opacities;
	int tiles_x, tiles_y;
	float4* conic4;
	float4* color_opacity4;
	uint2* rects;
	uint32_t* depth_keys;
};

// Writes gaussian i's records and returns its rectangle and depth key.
__device__ inline uint2 prepare_gaussian(const GaussianInputs& in, int64_t i, uint32_t* key) {
	const float radius = in.radii[i];
	const float op = in.opacities[i];
	const float a = in.conics[i * 3], b = in.conics[i * 3 + 1], c = in.conics[i * 3 + 2];
	const float ux = in.means2D[i * 2], uy = in.means2D[i * 2 + 1];
	in.conic4[i] = make_float4(a, b, c, op);
	if (in.colors)
		in.color_opacity4[i] = make_float4(in.colors[i * 3], in.colors[i * 3 + 1], in.colors[i * 3 + 2], op);
	int x0 = 0, y0 = 0, w = 0, h = 0;
	// !(radius > 0) culls NaN radii too (forward.cu:31-37).
	const bool ok = radius > 0.0f && hds_tile_rect(ux, uy, a, b, c, op, in.tiles_x, in.tiles_y, &x0, &y0, &w, &h);
	const uint2 rect = ok ? make_uint2((uint32_t)x0 | ((uint32_t)y0 << 16), (uint32_t)w | ((uint32_t)h << 16))
						  : make_uint2(0u, 0u);
	in.rects[i] = rect;
	*key = hds_f2u(in.depths[i]);
	in.depth_keys[i] = *key;
	return rect;
}

__global__ __launch_bounds__(kThreads) void prepare_kernel(int64_t n, const GaussianInputs in,
														   uint32_t* __restrict__ order, int passes,
														   uint32_t* __restrict__ hist, ZeroRanges zero) {
	__shared__ uint32_t s_hist[kMaxPasses][kRadix];
	// Control words the later kernels of this binning need cleared (none of them is touched here:
	// with passes > 0 the histograms were cleared by a launch before this one).
	zero_ranges(zero);
#pragma unroll
	for (int p = 0; p < kMaxPasses; p++) s_hist[p][threadIdx.x] = 0;
	__syncthreads();
	// 4 gaussians per thread keep the work-group count (and the histogram atomics) low while
	// leaving several waves per SIMD to hide the gathers.
	constexpr int kPer = 4;
#pragma unroll
	for (int r = 0; r < kPer; r++) {
		const int64_t i = ((int64_t)blockIdx.x * kPer + r) * kThreads + threadIdx.x;
		const bool valid = i < n;
		uint32_t key = 0;
		if (valid) {
			prepare_gaussian(in, i, &key);
			order[i] = (uint32_t)i;
		}
		count_digits(key, valid, passes, kRadixBits, s_hist);
	}
	flush_digits(passes, s_hist, hist);
}

// q = a / b, r = a % b: a float quotient estimate, within one of a / b for a < 2^22, corrected
// once (exact); larger a (rectangles of over 4M tiles) take the integer division.
__device__ inline void divmod_small(uint32_t a, uint32_t b, uint32_t& q, uint32_t& r) {
	if (a >= (1u << 22)) {
		q = a / b;
		r = a % b;
		return;
	}
	int qi = (int)((float)a * __builtin_amdgcn_rcpf((float)b));
	int ri = (int)a - (int)__umul24((uint32_t)qi, b);
	if (ri < 0) {
		qi -= 1;
		ri += (int)b;
	} else if (ri >= (int)b) {
		qi += 1;
		ri -= (int)b;
	}
	q = (uint32_t)qi;
	r = (uint32_t)ri;
}

// Pair emission (forward.cu:63-113): the pairs of gaussian g are [offsets[g], offsets[g] + w * h),
// tile (x0 + local % w, y0 + local / w) for local = 0 .. w * h - 1, in depth order. A wave takes 64
// consecutive depth-ordered gaussians, whose pairs are one contiguous run of the output; lane l
// writes pairs run_start + l, + 64, ... (coalesced), finding each pair's gaussian as the last of
// the wave's 64 whose offset is <= the pair index (gaussians with no tiles share their successor's
// offset, so they never own a pair) by binary search over the offsets in LDS, and reading that
// gaussian's record from its lane. Also counts the tile keys' digits for the pair sort. order /
// rects_sorted: gaussian id and tile rectangle of each depth-ordered entry. With pairs_total the
// pair count is read on the device and pairs past it are not written.
__global__ __launch_bounds__(kThreads) void emit_kernel(int64_t n, int64_t num_pairs, const uint64_t* __restrict__ pairs_total,
														 const uint32_t* __restrict__ offsets,
														 const uint32_t* __restrict__ order,
														 const uint2* __restrict__ rects_sorted, int tiles_x,
														 int passes, int bits, uint32_t* __restrict__ tile_keys,
														 uint32_t* __restrict__ gids, uint32_t* __restrict__ hist) {
	__shared__ uint32_t s_off[kWaves][HDS_WAVE];
	__shared__ uint32_t s_hist[kMaxPasses][kRadix];
	const int t = threadIdx.x, lane = t & (HDS_WAVE - 1), wave = t / HDS_WAVE;
	num_pairs = device_count(pairs_total, num_pairs);
#pragma unroll
	for (int p = 0; p < kMaxPasses; p++) s_hist[p][t] = 0;
	__syncthreads();

	const int64_t first = ((int64_t)blockIdx.x * kWaves + wave) * HDS_WAVE;
	const int64_t g = first + lane;
	const bool real = g < n;
	uint32_t off = 0, cnt = 0, gid = 0;
	uint2 rc = make_uint2(0u, 0u);
	if (real) {
		off = offsets[g];
		rc = rects_sorted[g];
		cnt = (rc.y & 0xffffu) * (rc.y >> 16);
		gid = order[g];
	}
	// The wave's run [run_start, run_end): from its first gaussian's offset to its last one's end,
	// cut at the pair count (which also bounds the loop when a failed count scan left the offsets
	// meaningless: device_count then gives 0 pairs).
	const int valid = first < n ? (int)min((int64_t)HDS_WAVE, n - first) : 0;
	const uint32_t run_start = __shfl(off, 0, HDS_WAVE);
	uint32_t run_end = valid > 0 ? __shfl(off + cnt, valid - 1, HDS_WAVE) : run_start;
	if ((int64_t)run_end > num_pairs) run_end = (uint32_t)num_pairs;
	s_off[wave][lane] = real ? off : 0xffffffffu;  // padding lanes never own a pair
	hds_wave_fence();

	for (uint32_t base = run_start; base < run_end; base += HDS_WAVE) {
		const uint32_t p = base + (uint32_t)lane;
		const bool in_run = p < run_end;
		// Last lane j of the wave with s_off[j] <= p (6 halvings over 64 entries).
		int j = 0;
#pragma unroll
		for (int step = HDS_WAVE / 2; step > 0; step >>= 1)
			if (s_off[wave][j + step] <= p) j += step;
		const uint32_t jx = (uint32_t)__shfl((int)rc.x, j, HDS_WAVE);
		const uint32_t jy = (uint32_t)__shfl((int)rc.y, j, HDS_WAVE);
		const uint32_t jgid = (uint32_t)__shfl((int)gid, j, HDS_WAVE);
		const uint32_t joff = s_off[wave][j];
		const bool valid_pair = in_run && (int64_t)p < num_pairs;
		uint32_t key = 0;
		if (valid_pair) {
			const uint32_t x0 = jx & 0xffffu, y0 = jx >> 16, w = jy & 0xffffu;
			uint32_t row, col;
			divmod_small(p - joff, w, row, col);
			key = (y0 + row) * (uint32_t)tiles_x + x0 + col;
			tile_keys[p] = key;
			gids[p] = jgid;
		}
		count_digits(key, valid_pair, passes, bits, s_hist);
	}
	flush_digits(passes, s_hist, hist);
}

// Zeroes two word ranges (control words of the sorts, tile ranges) in one launch.
__global__ __launch_bounds__(kThreads) void zero_kernel(uint32_t* __restrict__ a, int64_t na, uint32_t* __restrict__ b,
														 int64_t nb) {
	const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
	if (i < na)
		a[i] = 0u;
	else if (i < na + nb)
		b[i - na] = 0u;
}

// [start, end) of each tile in the sorted pair list (forward.cu:115-139): a pair starts its tile's
// range where the key before it differs and ends it where the key after it differs. A thread takes
// kRangeItems consecutive pairs with two 16-byte loads (keys are 256-byte aligned), plus the keys
// on either side.
// When the pair sort's look-back gave up (*sort_error set), the sorted list cannot be trusted and
// some of its slots may never have been written: no range is written (the ranges were zeroed
// before the emit, so every tile is empty and nothing indexes the list) and the failure is copied
// to *report, the word hds_bin_status hands to the host.
constexpr int kRangeItems = 8;
__global__ __launch_bounds__(kThreads) void ranges_kernel(int64_t num_pairs, const uint64_t* __restrict__ pairs_total,
														   const uint32_t* __restrict__ tile_keys, int64_t num_tiles,
														   const uint32_t* __restrict__ sort_error, uint32_t* __restrict__ report,
														   int2* __restrict__ ranges) {
	const int64_t p0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * kRangeItems;
	if (*sort_error != 0u) {
		if (blockIdx.x == 0 && threadIdx.x == 0) *report = 1u;
		return;
	}
	num_pairs = device_count(pairs_total, num_pairs);
	if (p0 >= num_pairs) return;
	// k[j] = key of pair p0 - 1 + j; outside [0, num_pairs) a value no tile has.
	constexpr uint32_t kNone = 0xffffffffu;
	uint32_t k[kRangeItems + 2];
	k[0] = p0 > 0 ? tile_keys[p0 - 1] : kNone;
	if (p0 + kRangeItems <= num_pairs && (reinterpret_cast<uintptr_t>(tile_keys) & 15u) == 0) {
		const uint4 a = *reinterpret_cast<const uint4*>(tile_keys + p0);
		const uint4 b = *reinterpret_cast<const uint4*>(tile_keys + p0 + 4);
		k[1] = a.x; k[2] = a.y; k[3] = a.z; k[4] = a.w;
		k[5] = b.x; k[6] = b.y; k[7] = b.z; k[8] = b.w;
	} else {
#pragma unroll
		for (int i = 0; i < kRangeItems; i++) k[i + 1] = p0 + i < num_pairs ? tile_keys[p0 + i] : kNone;
	}
	k[kRangeItems + 1] = p0 + kRangeItems < num_pairs ? tile_keys[p0 + kRangeItems] : kNone;
#pragma unroll
	for (int i = 0; i < kRangeItems; i++) {
		const uint32_t t = k[i + 1];
		if (t >= num_tiles) continue;  // also every position past num_pairs
		if (k[i] != t) ranges[t].x = (int)(p0 + i);
		if (k[i + 2] != t) ranges[t].y = (int)(p0 + i + 1);
	}
}

// ---------------------------------------------------------------------------------------------
// Depth order inside each tile (the tile-order binning). Every tile's list holds the right gaussians
// (placed by the counting scatter in an order the atomics chose, or, on the emit + pair sort path, in
// index order); one work-group per tile sorts it by the key (depth bits << 32 | gaussian id), which
// is the reference's (tile, depth bits, index) order restricted to the tile. Lists of up to 2048
// pairs are sorted in registers with E = 256..2048 / 256 keys per thread (tile_sort_registers: a
// 32-bit first pass, then the full keys); lists of up to kTileSortMax pairs take the 64-bit network
// entirely in LDS; longer ones are left unsorted and flagged (bit 1 of *overflow), and the caller
// bins the frame again with the global depth sort.
// ---------------------------------------------------------------------------------------------

constexpr int kTileSortRegMax = 2048;
constexpr int kTileSortMax = 4096;

__device__ inline uint64_t tile_sort_key(const int* vals, int i, int n, const uint32_t* __restrict__ depth_keys,
										 int64_t n_gaussians) {
	if (i >= n) return ~0ull;  // padding sorts last
	const uint32_t g = (uint32_t)vals[i];
	const uint32_t d = g < (uint64_t)n_gaussians ? depth_keys[g] : 0xffffffffu;
	return ((uint64_t)d << 32) | g;
}

// One side of a bitonic compare-exchange: the element keeps the smaller of (v, partner p) when
// keep_min (the pair's lower index in an ascending block, or its upper index in a descending one),
// else the larger: it takes p exactly when (v > p) == keep_min. One compare and one select per
// 32 bits.
template <typename K>
__device__ inline K bitonic_keep(K v, K p, bool keep_min) {
	return (v > p) == keep_min ? p : v;
}

__device__ __attribute__((always_inline)) inline uint32_t shfl_xor_key(uint32_t v, int mask) { return hds_lane_xor(v, mask); }
__device__ __attribute__((always_inline)) inline uint64_t shfl_xor_key(uint64_t v, int mask) {
	return ((uint64_t)hds_lane_xor((uint32_t)(v >> 32), mask) << 32) | hds_lane_xor((uint32_t)v, mask);
}

// Ascending bitonic sort of 256 * E keys held blocked (thread t: keys t * E .. t * E + E - 1):
// strides inside a thread's E keys are register swaps, strides inside a wave lane exchanges, and
// only the strides that cross waves go through LDS (s_x, 256 * E keys). Fully unrolled, so every
// stride and every keep-the-smaller bit of a stage is a constant.
template <int E, typename K>
__device__ void bitonic_blocked(K (&v)[E], K* s_x) {
	constexpr int M = kThreads * E;
	const int t = threadIdx.x;
#pragma unroll
	for (int k = 2; k <= M; k <<= 1) {
#pragma unroll
		for (int j = k >> 1; j >= E; j >>= 1) {
			// j >= E and k > j: bits j and k of t * E + e do not depend on e.
			const bool keep_min = ((t * E & j) == 0) == ((t * E & k) == 0);
			if (j >= HDS_WAVE * E) {
				// The partner sits in another wave.
				__syncthreads();
#pragma unroll
				for (int e = 0; e < E; e++) s_x[t * E + e] = v[e];
				__syncthreads();
#pragma unroll
				for (int e = 0; e < E; e++) v[e] = bitonic_keep(v[e], s_x[(t * E + e) ^ j], keep_min);
			} else {
				// Same slot e of lane t ^ (j / E).
#pragma unroll
				for (int e = 0; e < E; e++) v[e] = bitonic_keep(v[e], shfl_xor_key(v[e], j / E), keep_min);
			}
		}
		// Strides below E: both keys in this thread's registers (compile-time indices).
#pragma unroll
		for (int jj = E / 2; jj > 0; jj >>= 1) {
			if (jj < k) {
#pragma unroll
				for (int e = 0; e < E; e++) {
					if ((e & jj) == 0) {
						const bool ascending = ((t * E + e) & k) == 0;
						const K a = v[e], b = v[e | jj];
						const bool swap = (a > b) == ascending;
						v[e] = swap ? b : a;
						v[e | jj] = swap ? a : b;
					}
				}
			}
		}
	}
}

// Block-wide minimum and maximum of one value per thread (s_red: 2 * kWaves words).
__device__ inline void block_min_max(uint32_t lo, uint32_t hi, uint32_t* s_red, uint32_t& mn, uint32_t& mx) {
#pragma unroll
	for (int off = HDS_WAVE / 2; off > 0; off >>= 1) {
		lo = min(lo, hds_lane_xor(lo, off));
		hi = max(hi, hds_lane_xor(hi, off));
	}
	const int wave = threadIdx.x / HDS_WAVE;
	if ((threadIdx.x & (HDS_WAVE - 1)) == 0) {
		s_red[wave] = lo;
		s_red[kWaves + wave] = hi;
	}
	__syncthreads();
	mn = s_red[0];
	mx = s_red[kWaves];
#pragma unroll
	for (int w = 1; w < kWaves; w++) {
		mn = min(mn, s_red[w]);
		mx = max(mx, s_red[kWaves + w]);
	}
}

// Lists of n <= 256 * E pairs. The order wanted is that of the 64-bit key (depth bits << 32 | id).
// First pass: a network on unique 32-bit keys, the depth bits relative to the list's smallest,
// shifted right just enough to leave the low ib bits to the list index i (n < 2^ib): (coarse
// depth, i). That order already is the wanted one except among entries of equal coarse depth, so a
// check of adjacent full keys follows, with odd-even transposition rounds when it finds an
// inversion and, beyond kFixRounds rounds (many equal depths), the 64-bit network itself.
constexpr int kFixRounds = 8;

template <int E>
__device__ __attribute__((always_inline)) void tile_sort_registers(uint64_t* s_keys, uint32_t* s_red, int* vals, int n,
									const uint32_t* __restrict__ depth_keys, int64_t n_gaussians) {
	const int t = threadIdx.x;
	uint64_t* const s_full = s_keys;                                              // [n]: full key of entry i
	uint32_t* const s_x = reinterpret_cast<uint32_t*>(s_keys + kTileSortRegMax);  // 32-bit exchange area
	uint64_t full[E];
	uint32_t lo = 0xffffffffu, hi = 0u;
#pragma unroll
	for (int e = 0; e < E; e++) {
		const int i = t * E + e;
		full[e] = tile_sort_key(vals, i, n, depth_keys, n_gaussians);
		if (i < n) {
			s_full[i] = full[e];
			lo = min(lo, (uint32_t)(full[e] >> 32));
			hi = max(hi, (uint32_t)(full[e] >> 32));
		}
	}
	uint32_t dmin, dmax;
	block_min_max(lo, hi, s_red, dmin, dmax);  // also orders the s_full stores before the gathers below
	const int ib = 32 - __builtin_clz((unsigned)n);  // n < 2^ib
	const uint32_t range = dmax - dmin;
	const int span = range ? 32 - __builtin_clz(range) : 0;
	const int shift = span + ib > 32 ? span + ib - 32 : 0;
	uint32_t v[E];
#pragma unroll
	for (int e = 0; e < E; e++) {
		const int i = t * E + e;
		// Padding sorts last: a real key is at most (2^(32 - ib) - 1) << ib | (n - 1) < 2^32 - 1.
		v[e] = i < n ? ((((uint32_t)(full[e] >> 32) - dmin) >> shift) << ib) | (uint32_t)i : 0xffffffffu;
	}
	bitonic_blocked<E, uint32_t>(v, s_x);
	const uint32_t imask = (1u << ib) - 1u;
#pragma unroll
	for (int e = 0; e < E; e++) full[e] = t * E + e < n ? s_full[v[e] & imask] : ~0ull;
	__syncthreads();
	uint64_t* const s_sorted = s_keys;
#pragma unroll
	for (int e = 0; e < E; e++)
		if (t * E + e < n) s_sorted[t * E + e] = full[e];
	__syncthreads();
	// Odd-even transposition on the full keys: a round that swaps nothing after one that swapped
	// nothing (or the first two rounds) leaves no adjacent inversion, i.e. sorted.
	int clean = 0;
	int round = 0;
	for (; round < kFixRounds && clean < 2; round++) {
		bool swapped = false;
		for (int q = t; 2 * q + (round & 1) + 1 < n; q += kThreads) {
			const int p = 2 * q + (round & 1);
			const uint64_t a = s_sorted[p], b = s_sorted[p + 1];
			if (a > b) {
				s_sorted[p] = b;
				s_sorted[p + 1] = a;
				swapped = true;
			}
		}
		clean = __syncthreads_or(swapped) ? 0 : clean + 1;
	}
	if (clean < 2) {
		// Many entries of equal coarse depth: the 64-bit network over what the rounds left.
#pragma unroll
		for (int e = 0; e < E; e++) full[e] = t * E + e < n ? s_sorted[t * E + e] : ~0ull;
		__syncthreads();
		bitonic_blocked<E, uint64_t>(full, s_keys);
		__syncthreads();
#pragma unroll
		for (int e = 0; e < E; e++)
			if (t * E + e < n) s_sorted[t * E + e] = full[e];
		__syncthreads();
	}
	for (int p = t; p < n; p += kThreads) vals[p] = (int)(uint32_t)s_sorted[p];
}

// n <= kTileSortMax: the network over the next power of two, all in LDS.
__device__ void tile_sort_lds(uint64_t* s_keys, int* vals, int n, const uint32_t* __restrict__ depth_keys,
							  int64_t n_gaussians) {
	int m = kThreads;
	while (m < n) m <<= 1;
	for (int i = threadIdx.x; i < m; i += kThreads) s_keys[i] = tile_sort_key(vals, i, n, depth_keys, n_gaussians);
	__syncthreads();
	for (int k = 2; k <= m; k <<= 1) {
		for (int j = k >> 1; j > 0; j >>= 1) {
			for (int q = threadIdx.x; q < (m >> 1); q += kThreads) {
				const int i = 2 * j * (q / j) + (q % j);  // lower index of the pair (bit j clear)
				const uint64_t a = s_keys[i], b = s_keys[i + j];
				const bool swap = (a > b) == ((i & k) == 0);
				if (swap) {
					s_keys[i] = b;
					s_keys[i + j] = a;
				}
			}
			__syncthreads();
		}
	}
	for (int i = threadIdx.x; i < n; i += kThreads) vals[i] = (int)(uint32_t)s_keys[i];
}

// With pairs_total (the counting scatter), nothing is sorted when the binning outgrew its pair
// buffers (P > cap) or its scan failed: the caller bins that frame again.
__global__ __launch_bounds__(kThreads) void tile_sort_kernel(const int2* __restrict__ ranges, int* __restrict__ values,
															 const uint32_t* __restrict__ depth_keys, int64_t n_gaussians,
															 int64_t num_tiles, uint32_t* __restrict__ overflow,
															 const uint64_t* __restrict__ pairs_total, int64_t cap) {
	__shared__ uint64_t s_keys[kTileSortMax];
	__shared__ uint32_t s_red[2 * kWaves];
	const int64_t tile = blockIdx.x;
	if (tile >= num_tiles) return;
	if (pairs_total && (reinterpret_cast<const uint32_t*>(pairs_total + 1)[0] != 0u || *pairs_total > (uint64_t)cap))
		return;
	const int2 r = ranges[tile];
	const int n = r.y - r.x;
	if (n <= 1) return;
	if (n > kTileSortMax) {
		if (threadIdx.x == 0) atomicOr(overflow, 2u);
		return;
	}
	int* vals = values + r.x;
	if (n <= 256) tile_sort_registers<1>(s_keys, s_red, vals, n, depth_keys, n_gaussians);
	else if (n <= 512) tile_sort_registers<2>(s_keys, s_red, vals, n, depth_keys, n_gaussians);
	else if (n <= 1024) tile_sort_registers<4>(s_keys, s_red, vals, n, depth_keys, n_gaussians);
	else if (n <= kTileSortRegMax) tile_sort_registers<8>(s_keys, s_red, vals, n, depth_keys, n_gaussians);
	else tile_sort_lds(s_keys, vals, n, depth_keys, n_gaussians);
}

// ---------------------------------------------------------------------------------------------
// Counting scatter (tile-order binning): prepare_tiles_kernel, scan_kernel<false> over the
// tile-major count matrix, scatter_kernel, then tile_sort_kernel.
// ---------------------------------------------------------------------------------------------

// Calls f(tile, gaussian) for every pair of a wave's 64 consecutive gaussians (lane l holds
// gaussian first + l and its rectangle rc, zero when culled or past n). The wave's pairs form one
// run, which its lanes take 64 at a time; each lane finds its pair's gaussian as the last lane
// whose exclusive offset (in the wave's 64 LDS words s_off) is <= the pair index, so gaussians
// without tiles, which share their successor's offset, never own a pair (the emit kernel's search).
template <typename F>
__device__ inline void for_each_pair(uint2 rc, uint32_t first, int tiles_x, uint32_t* s_off, F&& f) {
	const int lane = threadIdx.x & (HDS_WAVE - 1);
	const uint32_t cnt = (rc.y & 0xffffu) * (rc.y >> 16);
	const uint32_t x = hds_wave_inclusive_scan(cnt);
	const uint32_t run = (uint32_t)__builtin_amdgcn_readlane((int)x, HDS_WAVE - 1);
	s_off[lane] = x - cnt;
	hds_wave_fence();
	for (uint32_t base = 0; base < run; base += HDS_WAVE) {
		const uint32_t p = base + (uint32_t)lane;
		int j = 0;
#pragma unroll
		for (int step = HDS_WAVE / 2; step > 0; step >>= 1)
			if (s_off[j + step] <= p) j += step;
		const uint32_t jx = (uint32_t)__shfl((int)rc.x, j, HDS_WAVE);
		const uint32_t jy = (uint32_t)__shfl((int)rc.y, j, HDS_WAVE);
		if (p < run) {
			uint32_t row, col;
			divmod_small(p - s_off[j], jy & 0xffffu, row, col);
			f(((jx >> 16) + row) * (uint32_t)tiles_x + (jx & 0xffffu) + col, first + (uint32_t)j);
		}
	}
	// The next call rewrites s_off: every lane's reads above come first in the wave's LDS order.
	hds_wave_fence();
}

// Gaussian i of thread t in round r of chunk c: c * kChunk + r * kScatterThreads + t, so that wave w
// holds 64 consecutive gaussians in every round.
__device__ inline int64_t chunk_gaussian(int64_t chunk, int r) {
	return chunk * kChunk + (int64_t)r * kScatterThreads + threadIdx.x;
}

// Step 1: the records of one chunk (prepare_kernel's, without the index order) and the chunk's
// pair count per tile, one LDS histogram of up to kHistBins tiles at a time, stored to column
// `chunk` of the tile-major count matrix: counts[tile * chunks + chunk]. Also clears `zero` (the
// control block and the status words the scan uses, tile_ranges) for the later launches.
__global__ __launch_bounds__(kScatterThreads) void prepare_tiles_kernel(int64_t n, const GaussianInputs in,
																		int64_t num_tiles, int64_t chunks,
																		uint32_t* __restrict__ counts, ZeroRanges zero) {
	__shared__ uint32_t s_bins[kHistBins];
	__shared__ uint32_t s_off[kScatterWaves][HDS_WAVE];
	zero_ranges(zero);
	const int64_t chunk = blockIdx.x;
	const int wave = threadIdx.x / HDS_WAVE;
	uint2 rc[4];
#pragma unroll
	for (int r = 0; r < 4; r++) {
		const int64_t i = chunk_gaussian(chunk, r);
		uint32_t key;
		rc[r] = i < n ? prepare_gaussian(in, i, &key) : make_uint2(0u, 0u);
	}
	for (int64_t w0 = 0; w0 < num_tiles; w0 += kHistBins) {
		const int nb = (int)min((int64_t)kHistBins, num_tiles - w0);
		for (int i = threadIdx.x; i < nb; i += kScatterThreads) s_bins[i] = 0u;
		__syncthreads();
#pragma unroll
		for (int r = 0; r < 4; r++) {
			const uint32_t first = (uint32_t)(chunk_gaussian(chunk, r) - (threadIdx.x & (HDS_WAVE - 1)));
			for_each_pair(rc[r], first, in.tiles_x, s_off[wave], [&](uint32_t tile, uint32_t) {
				const uint32_t b = tile - (uint32_t)w0;
				if (b < (uint32_t)nb) atomicAdd(&s_bins[b], 1u);
			});
		}
		__syncthreads();
		for (int i = threadIdx.x; i < nb; i += kScatterThreads) counts[(w0 + i) * chunks + chunk] = s_bins[i];
		__syncthreads();
	}
}

// Step 3, after the exclusive scan of the count matrix (entry (tile, chunk) = where the chunk's run
// of that tile starts in the tile-major pair list): the chunk's pairs go to their runs, the LDS copy
// of the chunk's run starts serving as write cursors (one LDS atomic per pair; the order inside a
// run is whatever the atomics make it, and tile_sort_kernel replaces it by (depth bits, index)).
// Every work-group also writes a share of tile_ranges: [run start of (tile, chunk 0), run start of
// (tile + 1, chunk 0)), (0, 0) when empty. Nothing at or past limit = min(P, cap) is written and the
// ranges are cut there, so a binning whose pair buffers were too small still leaves only written
// entries inside its ranges (the caller bins it again with exact buffers); a failed scan, or P beyond
// int32 indices, writes nothing (tile_ranges were cleared by prepare_tiles_kernel). With pairs_total
// null, cap is the exact pair count.
__global__ __launch_bounds__(kScatterThreads) void scatter_kernel(int64_t n, const uint2* __restrict__ rects,
																  int tiles_x, int64_t num_tiles, int64_t chunks,
																  const uint32_t* __restrict__ starts,
																  const uint64_t* __restrict__ pairs_total, int64_t cap,
																  int32_t* __restrict__ values, int2* __restrict__ ranges) {
	__shared__ uint32_t s_cursor[kHistBins];
	__shared__ uint32_t s_off[kScatterWaves][HDS_WAVE];
	int64_t total = cap;
	if (pairs_total) {
		if (reinterpret_cast<const uint32_t*>(pairs_total + 1)[0] != 0u) return;
		total = (int64_t)min(*pairs_total, (uint64_t)INT32_MAX);
	}
	if (total >= INT32_MAX) return;
	const int64_t limit = min(total, cap);
	const int64_t chunk = blockIdx.x;
	const int wave = threadIdx.x / HDS_WAVE;
	for (int64_t t = chunk * kScatterThreads + threadIdx.x; t < num_tiles; t += chunks * kScatterThreads) {
		const int64_t start = min((int64_t)starts[t * chunks], limit);
		const int64_t end = min(t + 1 < num_tiles ? (int64_t)starts[(t + 1) * chunks] : total, limit);
		// An empty range is (0, 0), as for a tile no pair touches (forward.cu:115-139).
		ranges[t] = end > start ? make_int2((int)start, (int)end) : make_int2(0, 0);
	}
	uint2 rc[4];
#pragma unroll
	for (int r = 0; r < 4; r++) {
		const int64_t i = chunk_gaussian(chunk, r);
		rc[r] = i < n ? rects[i] : make_uint2(0u, 0u);
	}
	for (int64_t w0 = 0; w0 < num_tiles; w0 += kHistBins) {
		const int nb = (int)min((int64_t)kHistBins, num_tiles - w0);
		for (int i = threadIdx.x; i < nb; i += kScatterThreads) s_cursor[i] = starts[(w0 + i) * chunks + chunk];
		__syncthreads();
#pragma unroll
		for (int r = 0; r < 4; r++) {
			const uint32_t first = (uint32_t)(chunk_gaussian(chunk, r) - (threadIdx.x & (HDS_WAVE - 1)));
			for_each_pair(rc[r], first, tiles_x, s_off[wave], [&](uint32_t tile, uint32_t g) {
				const uint32_t b = tile - (uint32_t)w0;
				if (b < (uint32_t)nb) {
					const uint32_t pos = atomicAdd(&s_cursor[b], 1u);
					if ((int64_t)pos < limit) values[pos] = (int32_t)g;
				}
			});
		}
		__syncthreads();
	}
}

// ---------------------------------------------------------------------------------------------
// Workspace layouts. Every region is 256-byte aligned; what a binning reads before writing (the
// control block, the look-back status words) is zeroed before use.
// ---------------------------------------------------------------------------------------------

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Control block at the start of the zeroed region: the total of the counts scan and the error
// flag sit together so that hds_bin_count reads both back in one 16-byte copy.
struct Control {
	uint64_t total;
	uint32_t error;       // a look-back of the depth sort or the scan gave up
	uint32_t pair_error;  // (gaussian workspace) bit 0: a look-back of the pair sort gave up;
						  // bit 1: a tile-order binning met a tile beyond kTileSortMax pairs
	uint32_t tickets[kMaxPasses + 1];  // one per radix pass, then the scan's
	uint32_t hist[kMaxPasses * kHistWords];
};

// Chunks of the counting scatter and the words of its count matrix (chunks x tiles); words = 0 when
// the matrix would exceed `limit` words (the frame then takes the emit + pair sort).
struct ScatterShape {
	int64_t chunks;
	uint64_t words;
};

ScatterShape scatter_shape(int64_t n, int64_t num_tiles, uint64_t limit) {
	const int64_t chunks = n > 0 ? (n + kChunk - 1) / kChunk : 0;
	const uint64_t words = (uint64_t)chunks * (uint64_t)(num_tiles > 0 ? num_tiles : 0);
	return {chunks, words <= limit ? words : 0};
}

// [ctrl, zero_end) is cleared before use; the count matrix after it is written whole by
// prepare_tiles_kernel. num_tiles = 0 leaves out the matrix (the depth-order binning never uses it).
struct GaussianSpace {
	size_t rects, rects_sorted, keys_a, vals_a, keys_b, vals_b, offsets, ctrl, status, scan_status, counts_status,
		zero_end, counts, bytes;
};

GaussianSpace gaussian_space(int64_t n, int64_t num_tiles = 0) {
	GaussianSpace g;
	const size_t items = (size_t)(n > 0 ? n : 1);
	const size_t parts = (size_t)parts_of((int64_t)items);
	const uint64_t words = scatter_shape(n, num_tiles, kScatterWords).words;
	size_t o = 0;
	g.rects = o; o = align256(o + 8 * items);
	g.rects_sorted = o; o = align256(o + 8 * items);
	g.keys_a = o; o = align256(o + 4 * items);
	g.vals_a = o; o = align256(o + 4 * items);
	g.keys_b = o; o = align256(o + 4 * items);
	g.vals_b = o; o = align256(o + 4 * items);
	g.offsets = o; o = align256(o + 4 * items);
	g.ctrl = o; o = align256(o + sizeof(Control));
	g.status = o; o = align256(o + 8 * parts * kRadix);
	g.scan_status = o; o = align256(o + 8 * parts);
	g.counts_status = o; o = align256(o + 8 * (size_t)parts_of((int64_t)(words > 0 ? words : 1)));
	g.zero_end = o;
	g.counts = o; o = align256(o + 4 * words);
	g.bytes = o;
	return g;
}

struct PairSpace {
	size_t keys_a, keys_b, vals_tmp, ctrl, status, bytes;
};

PairSpace pair_space(int64_t num_pairs) {
	PairSpace p;
	const size_t items = (size_t)(num_pairs > 0 ? num_pairs : 1);
	const size_t parts = (size_t)parts_of((int64_t)items);
	size_t o = 0;
	p.keys_a = o; o = align256(o + 4 * items);
	p.keys_b = o; o = align256(o + 4 * items);
	p.vals_tmp = o; o = align256(o + 4 * items);
	p.ctrl = o; o = align256(o + sizeof(Control));
	p.status = o; o = align256(o + 8 * parts * kRadix);
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
	const int64_t tiles_x = width > 0 ? (width + HDS_TILE - 1) / HDS_TILE : 0;
	const int64_t tiles_y = height > 0 ? (height + HDS_TILE - 1) / HDS_TILE : 0;
	return gaussian_space(n, tiles_x * tiles_y).bytes;
}

extern "C" size_t hds_pairs_workspace_bytes(int64_t num_pairs, int width, int height) {
	(void)width;
	(void)height;
	return pair_space(num_pairs).bytes;
}

namespace {

// Which count last filled each gaussian workspace: depth-sorted (hds_bin_count(_async)) or index
// order (hds_bin_tile_order_async, by the emit + pair sort or by the counting scatter). They leave
// different things in it (offsets scanned over the depth order or over the index order, or the
// scanned count matrix), so an emit checks the record and rejects a workspace another count
// filled, or one no count of this process filled, before it enqueues anything; the tile-order emit
// follows the recorded path. Keyed by address; the most recent kModeRecords workspaces are
// remembered.
enum CountMode { kModeDepth = 0, kModeTileEmit = 1, kModeTileScatter = 2 };
constexpr size_t kModeRecords = 256;
std::mutex g_mode_mutex;
std::vector<std::pair<const void*, int>> g_mode_records;  // (workspace, CountMode), newest last

void record_count_mode(const void* workspace, int mode) {
	std::lock_guard<std::mutex> lock(g_mode_mutex);
	for (size_t i = 0; i < g_mode_records.size(); i++)
		if (g_mode_records[i].first == workspace) {
			g_mode_records.erase(g_mode_records.begin() + (ptrdiff_t)i);
			break;
		}
	if (g_mode_records.size() == kModeRecords) g_mode_records.erase(g_mode_records.begin());
	g_mode_records.emplace_back(workspace, mode);
}

// HDS_OK when the workspace was last filled in the depth order (depth_sort) or in tile order (not
// depth_sort); *mode, when given, receives the recorded CountMode.
int check_count_mode(const void* workspace, bool depth_sort, const char* entry, int* mode = nullptr) {
	std::lock_guard<std::mutex> lock(g_mode_mutex);
	for (const auto& r : g_mode_records)
		if (r.first == workspace) {
			const bool depth = r.second == kModeDepth;
			if (mode) *mode = r.second;
			if (depth == depth_sort) return HDS_OK;
			return hds_set_error(HDS_ERR_INVALID, "%s: the workspace was filled by %s, this emit needs %s", entry,
								 depth ? "hds_bin_count (depth order)" : "hds_bin_tile_order_async (tile order)",
								 depth_sort ? "hds_bin_count's depth order" : "hds_bin_tile_order_async's tile order");
		}
	return hds_set_error(HDS_ERR_INVALID, "%s: the workspace was not filled by a count of this process (%s)", entry,
						 depth_sort ? "hds_bin_count" : "hds_bin_tile_order_async");
}

// Enqueues the counting half of the binning (cull, records, depth order, scan of the tile counts);
// the pair count and the look-back error flag end in the workspace's control block. *launched is
// false when there was nothing to enqueue (n == 0).
int bin_count_launch(int64_t n, const float* means2D, const float* depths, const float* radii, const float* conics,
					 const float* colors, const float* opacities, int width, int height, float* conic4,
					 float* color_opacity4, void* workspace, size_t workspace_bytes, bool depth_sort,
					 const ZeroRanges* fused_zero, hipStream_t s, bool* launched) {
	*launched = false;
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

	uint2* rects = at<uint2>(workspace, g.rects);
	uint2* rects_sorted = at<uint2>(workspace, g.rects_sorted);
	uint32_t* keys_a = at<uint32_t>(workspace, g.keys_a);
	uint32_t* vals_a = at<uint32_t>(workspace, g.vals_a);
	uint32_t* keys_b = at<uint32_t>(workspace, g.keys_b);
	uint32_t* vals_b = at<uint32_t>(workspace, g.vals_b);
	uint32_t* offsets = at<uint32_t>(workspace, g.offsets);
	Control* ctrl = at<Control>(workspace, g.ctrl);
	uint64_t* status = at<uint64_t>(workspace, g.status);
	uint64_t* scan_status = at<uint64_t>(workspace, g.scan_status);

	const int64_t zero_words = (int64_t)(g.zero_end - g.ctrl) / 4;
	ZeroRanges zero{};
	if (fused_zero) {
		// Without the depth sort prepare keeps no histograms, so it clears the control blocks itself.
		HDS_REQUIRE(!depth_sort, "bin_count: fused zeroing needs the tile order");
		zero = *fused_zero;
		zero.p[0] = at<uint32_t>(workspace, g.ctrl);
		zero.n[0] = zero_words;
	} else {
		HdsKernelTimer timer1("zero_kernel", s);
		zero_kernel<<<hds_blocks(zero_words, kThreads), kThreads, 0, s>>>(at<uint32_t>(workspace, g.ctrl), zero_words,
																		   nullptr, 0);
		timer1.stop();
		HDS_LAUNCH_CHECK("zero_sort_control", s);
	}
	HdsKernelTimer timer2("prepare_kernel", s);
	const GaussianInputs in{means2D, depths, radii, conics, colors, opacities, tiles_x, tiles_y,
							reinterpret_cast<float4*>(conic4), reinterpret_cast<float4*>(color_opacity4), rects, keys_a};
	prepare_kernel<<<hds_blocks(n, 4 * kThreads), kThreads, 0, s>>>(n, in, vals_a, depth_sort ? kMaxPasses : 0,
																	 ctrl->hist, zero);
	timer2.stop();
	HDS_LAUNCH_CHECK("prepare_gaussians", s);
	if (depth_sort) {
		// 4 passes: the depth order ends back in (keys_a, vals_a); the last one also writes each
		// entry's tile rectangle to rects_sorted.
		int st = onesweep_sort(keys_a, vals_a, keys_b, vals_b, n, nullptr, kMaxPasses, kRadixBits, ctrl->hist, status,
							   ctrl->tickets, &ctrl->error, false, rects, rects_sorted, s);
		if (st != HDS_OK) return st;
	}
	// Without the depth sort (tile order) the entries stay in index order: vals_a = identity,
	// keys_a = each gaussian's depth key, and the scan and the emit read the rectangles as prepared.
	HdsKernelTimer timer3("scan_kernel", s);
	scan_kernel<true><<<(unsigned)parts_of(n), kThreads, 0, s>>>(depth_sort ? rects_sorted : rects, n, offsets, scan_status,
															ctrl->tickets + kMaxPasses, &ctrl->error,
															g_spin_limit.load(std::memory_order_relaxed), &ctrl->total);
	timer3.stop();
	HDS_LAUNCH_CHECK("scan_tile_counts", s);
	record_count_mode(workspace, depth_sort ? kModeDepth : kModeTileEmit);
	*launched = true;
	return HDS_OK;
}

// The (pair count, error flags) words hds_bin_count_async and hds_bin_status copy out: the first
// three fields of the gaussian workspace's Control block.
struct CountWords {
	uint64_t total;
	uint32_t error, pair_error;
};

const CountWords* count_words(const void* workspace, int64_t n) {
	return at<CountWords>(const_cast<void*>(workspace), gaussian_space(n).ctrl);
}

// Enqueues the emitting half. With exact, num_pairs is the pair count; otherwise it is the
// capacity the buffers were sized for and the kernels take min(count in the workspace, capacity).
int bin_emit_launch(int64_t n, int64_t num_pairs, bool exact, bool tile_order, int width, int height, void* workspace,
					void* pairs_workspace, size_t pairs_workspace_bytes, int32_t* values_sorted, int32_t* tile_ranges,
					hipStream_t s, bool control_zeroed = false) {
	HDS_REQUIRE(width > 0 && height > 0, "bin_emit: image size %dx%d must be positive", width, height);
	HDS_REQUIRE(num_pairs >= 0 && num_pairs < INT32_MAX, "bin_emit: pair count %lld outside [0, 2^31)",
				(long long)num_pairs);
	HDS_REQUIRE(tile_ranges, "bin_emit: tile_ranges must not be NULL");
	const int tiles_x = (width + HDS_TILE - 1) / HDS_TILE, tiles_y = (height + HDS_TILE - 1) / HDS_TILE;
	const int64_t num_tiles = (int64_t)tiles_x * tiles_y;
	uint32_t* ranges_words = reinterpret_cast<uint32_t*>(tile_ranges);
	if (num_pairs == 0 || n == 0) {
		HdsKernelTimer timer1("zero_kernel", s);
		zero_kernel<<<hds_blocks(2 * num_tiles, kThreads), kThreads, 0, s>>>(ranges_words, 2 * num_tiles, nullptr, 0);
		timer1.stop();
		HDS_LAUNCH_CHECK("zero_tile_ranges", s);
		return HDS_OK;
	}
	const PairSpace p = pair_space(num_pairs);
	HDS_REQUIRE(pairs_workspace && pairs_workspace_bytes >= p.bytes, "bin_emit: pairs workspace of %zu bytes, need %zu",
				pairs_workspace_bytes, p.bytes);
	HDS_REQUIRE(workspace && values_sorted, "bin_emit: null pointer argument");
	const GaussianSpace g = gaussian_space(n);
	void* ws = workspace;
	const uint64_t* total = exact ? nullptr : &count_words(workspace, n)->total;
	const uint32_t* offsets = at<uint32_t>(ws, g.offsets);
	const uint32_t* order = at<uint32_t>(ws, g.vals_a);
	const uint2* rects_sorted = at<uint2>(ws, tile_order ? g.rects : g.rects_sorted);

	uint32_t* keys_a = at<uint32_t>(pairs_workspace, p.keys_a);
	uint32_t* keys_b = at<uint32_t>(pairs_workspace, p.keys_b);
	uint32_t* vals_tmp = at<uint32_t>(pairs_workspace, p.vals_tmp);
	Control* ctrl = at<Control>(pairs_workspace, p.ctrl);
	uint64_t* status = at<uint64_t>(pairs_workspace, p.status);
	uint32_t* out = reinterpret_cast<uint32_t*>(values_sorted);

	// Pick the ping-pong buffers so the last pass lands in values_sorted. The tile id's bits are
	// split evenly over the passes (12 bits at 979x546: two 6-bit digits, not 8 + 4), so each
	// digit's run in a partition's output is longer and its stores more coalesced.
	const int key_bits = tile_bits(num_tiles);
	const int passes = (key_bits + kRadixBits - 1) / kRadixBits;
	const int bits = passes > 0 ? (key_bits + passes - 1) / passes : kRadixBits;
	uint32_t* vals_a = (passes % 2 == 0) ? out : vals_tmp;
	uint32_t* vals_b = (passes % 2 == 0) ? vals_tmp : out;

	const int64_t ctrl_words = (int64_t)(p.bytes - p.ctrl) / 4;
	if (!control_zeroed) {
		HdsKernelTimer timer1("zero_kernel", s);
		zero_kernel<<<hds_blocks(ctrl_words + 2 * num_tiles, kThreads), kThreads, 0, s>>>(
			at<uint32_t>(pairs_workspace, p.ctrl), ctrl_words, ranges_words, 2 * num_tiles);
		timer1.stop();
		HDS_LAUNCH_CHECK("zero_sort_control", s);
	}
	HdsKernelTimer timer2("emit_kernel", s);
	emit_kernel<<<hds_blocks(n, kThreads), kThreads, 0, s>>>(n, num_pairs, total, offsets, order, rects_sorted,
																	tiles_x, passes, bits, keys_a, vals_a, ctrl->hist);
	timer2.stop();
	HDS_LAUNCH_CHECK("emit_pairs", s);
	int st = onesweep_sort(keys_a, vals_a, keys_b, vals_b, num_pairs, total, passes, bits, ctrl->hist, status,
						   ctrl->tickets, &ctrl->error, true, nullptr, nullptr, s);
	if (st != HDS_OK) return st;
	const uint32_t* keys_sorted = (passes % 2 == 0) ? keys_a : keys_b;
	HdsKernelTimer timer3("ranges_kernel", s);
	ranges_kernel<<<hds_blocks((num_pairs + kRangeItems - 1) / kRangeItems, kThreads), kThreads, 0, s>>>(
		num_pairs, total, keys_sorted, num_tiles, &ctrl->error, &at<Control>(ws, g.ctrl)->pair_error,
		reinterpret_cast<int2*>(tile_ranges));
	timer3.stop();
	HDS_LAUNCH_CHECK("identify_tile_ranges", s);
	if (tile_order) {
		HdsKernelTimer timer4("tile_sort_kernel", s);
		tile_sort_kernel<<<(unsigned)num_tiles, kThreads, 0, s>>>(
			reinterpret_cast<const int2*>(tile_ranges), values_sorted, at<uint32_t>(ws, g.keys_a), n, num_tiles,
			&at<Control>(ws, g.ctrl)->pair_error, nullptr, 0);
		timer4.stop();
		HDS_LAUNCH_CHECK("tile_depth_order", s);
	}
	return HDS_OK;
}

// The counting scatter's second half: the pairs into their runs and tile_ranges (scatter_kernel),
// then each tile's depth order. With exact, cap is the pair count; otherwise it is the capacity of
// values_sorted and the kernels read P (and the scan's error flag) from the workspace.
int scatter_emit_launch(int64_t n, int64_t cap, bool exact, int width, int height, void* workspace,
						int32_t* values_sorted, int32_t* tile_ranges, hipStream_t s) {
	const int tiles_x = (width + HDS_TILE - 1) / HDS_TILE, tiles_y = (height + HDS_TILE - 1) / HDS_TILE;
	const int64_t num_tiles = (int64_t)tiles_x * tiles_y;
	const GaussianSpace g = gaussian_space(n, num_tiles);
	const ScatterShape sh = scatter_shape(n, num_tiles, kScatterWords);
	Control* ctrl = at<Control>(workspace, g.ctrl);
	const uint64_t* total = exact ? nullptr : &ctrl->total;
	HdsKernelTimer timer1("scatter_kernel", s);
	scatter_kernel<<<(unsigned)sh.chunks, kScatterThreads, 0, s>>>(
		n, at<uint2>(workspace, g.rects), tiles_x, num_tiles, sh.chunks, at<uint32_t>(workspace, g.counts), total, cap,
		values_sorted, reinterpret_cast<int2*>(tile_ranges));
	timer1.stop();
	HDS_LAUNCH_CHECK("scatter_pairs", s);
	HdsKernelTimer timer2("tile_sort_kernel", s);
	tile_sort_kernel<<<(unsigned)num_tiles, kThreads, 0, s>>>(reinterpret_cast<const int2*>(tile_ranges),
															 values_sorted, at<uint32_t>(workspace, g.keys_a), n,
															 num_tiles, &ctrl->pair_error, total, cap);
	timer2.stop();
	HDS_LAUNCH_CHECK("tile_depth_order", s);
	return HDS_OK;
}

// The whole tile-order binning by counting scatter (n > 0, the matrix within the path's limit):
// prepare_tiles_kernel (records, per-chunk tile counts, clearing the control block and tile_ranges
// on the side), the exclusive scan of the count matrix (run starts; P and the look-back flag into
// the control block), then scatter_emit_launch.
int bin_tile_scatter_launch(int64_t n, const float* means2D, const float* depths, const float* radii,
							const float* conics, const float* colors, const float* opacities, int width, int height,
							float* conic4, float* color_opacity4, void* workspace, size_t workspace_bytes,
							int64_t capacity, int32_t* values_sorted, int32_t* tile_ranges, hipStream_t s) {
	HDS_REQUIRE(n > 0 && n < INT32_MAX, "bin_tile_order: gaussian count %lld outside [1, 2^31)", (long long)n);
	const int tiles_x = (width + HDS_TILE - 1) / HDS_TILE, tiles_y = (height + HDS_TILE - 1) / HDS_TILE;
	HDS_REQUIRE(tiles_x < 65536 && tiles_y < 65536, "bin_tile_order: image %dx%d has too many tiles", width, height);
	const int64_t num_tiles = (int64_t)tiles_x * tiles_y;
	const GaussianSpace g = gaussian_space(n, num_tiles);
	const ScatterShape sh = scatter_shape(n, num_tiles, kScatterWords);
	HDS_REQUIRE(workspace && workspace_bytes >= g.bytes, "bin_tile_order: workspace of %zu bytes, need %zu",
				workspace_bytes, g.bytes);
	HDS_REQUIRE(means2D && depths && radii && conics && opacities && conic4, "bin_tile_order: null pointer argument");
	HDS_REQUIRE(colors == nullptr || color_opacity4 != nullptr,
				"bin_tile_order: colors given without color_opacity4");
	HDS_REQUIRE(aligned16(conic4) && (!color_opacity4 || aligned16(color_opacity4)),
				"bin_tile_order: conic4 / color_opacity4 must be 16-byte aligned");
	Control* ctrl = at<Control>(workspace, g.ctrl);
	uint32_t* counts = at<uint32_t>(workspace, g.counts);
	// Cleared on the side: the control block (P, flags, the scan's ticket), the scan's status words
	// and tile_ranges (left empty if the scan fails).
	ZeroRanges zero{};
	zero.p[0] = at<uint32_t>(workspace, g.ctrl);
	zero.n[0] = (int64_t)sizeof(Control) / 4;
	zero.p[1] = at<uint32_t>(workspace, g.counts_status);
	zero.n[1] = (int64_t)(g.zero_end - g.counts_status) / 4;
	zero.p[2] = reinterpret_cast<uint32_t*>(tile_ranges);
	zero.n[2] = 2 * num_tiles;
	const GaussianInputs in{means2D, depths, radii, conics, colors, opacities, tiles_x, tiles_y,
							reinterpret_cast<float4*>(conic4), reinterpret_cast<float4*>(color_opacity4),
							at<uint2>(workspace, g.rects), at<uint32_t>(workspace, g.keys_a)};
	HdsKernelTimer timer1("prepare_tiles_kernel", s);
	prepare_tiles_kernel<<<(unsigned)sh.chunks, kScatterThreads, 0, s>>>(n, in, num_tiles, sh.chunks, counts, zero);
	timer1.stop();
	HDS_LAUNCH_CHECK("prepare_tile_counts", s);
	HdsKernelTimer timer2("scan_kernel", s);
	scan_kernel<false><<<(unsigned)parts_of((int64_t)sh.words), kThreads, 0, s>>>(
		counts, (int64_t)sh.words, counts, at<uint64_t>(workspace, g.counts_status), ctrl->tickets + kMaxPasses,
		&ctrl->error, g_spin_limit.load(std::memory_order_relaxed), &ctrl->total);
	timer2.stop();
	HDS_LAUNCH_CHECK("scan_tile_counts", s);
	record_count_mode(workspace, kModeTileScatter);
	return scatter_emit_launch(n, capacity, false, width, height, workspace, values_sorted, tile_ranges, s);
}

}  // namespace

extern "C" int hds_bin_count(int64_t n, const float* means2D, const float* depths, const float* radii,
							 const float* conics, const float* colors, const float* opacities, int width, int height,
							 float* conic4, float* color_opacity4, void* workspace, size_t workspace_bytes,
							 int64_t* num_pairs, hds_stream_t stream) {
	HDS_REQUIRE(num_pairs, "bin_count: num_pairs must not be NULL");
	*num_pairs = 0;
	hipStream_t s = (hipStream_t)stream;
	bool launched = false;
	int st = bin_count_launch(n, means2D, depths, radii, conics, colors, opacities, width, height, conic4,
							  color_opacity4, workspace, workspace_bytes, true, nullptr, s, &launched);
	if (st != HDS_OK || !launched) return st;
	CountWords host = {0, 0, 0};
	HDS_HIP(hipMemcpyAsync(&host, count_words(workspace, n), sizeof(host), hipMemcpyDeviceToHost, s));
	HDS_HIP(hipStreamSynchronize(s));
	if (host.error)
		return hds_set_error(HDS_ERR_RUNTIME, "bin_count: a sort or scan look-back did not complete");
	HDS_REQUIRE(host.total < (uint64_t)INT32_MAX, "bin_count: %llu tile-gaussian pairs overflow int32 indices",
				(unsigned long long)host.total);
	*num_pairs = (int64_t)host.total;
	return HDS_OK;
}

extern "C" int hds_bin_count_async(int64_t n, const float* means2D, const float* depths, const float* radii,
								   const float* conics, const float* colors, const float* opacities, int width,
								   int height, float* conic4, float* color_opacity4, void* workspace,
								   size_t workspace_bytes, void* count_host, hds_stream_t stream) {
	HDS_REQUIRE(count_host, "bin_count_async: count_host must not be NULL");
	hipStream_t s = (hipStream_t)stream;
	bool launched = false;
	int st = bin_count_launch(n, means2D, depths, radii, conics, colors, opacities, width, height, conic4,
							  color_opacity4, workspace, workspace_bytes, true, nullptr, s, &launched);
	if (st != HDS_OK) return st;
	if (!launched) {
		// Nothing enqueued: the count is known now.
		*static_cast<CountWords*>(count_host) = CountWords{0, 0, 0};
		return HDS_OK;
	}
	HDS_HIP(hipMemcpyAsync(count_host, count_words(workspace, n), sizeof(CountWords), hipMemcpyDeviceToHost, s));
	return HDS_OK;
}

extern "C" int hds_bin_status(int64_t n, const void* workspace, void* status_host, hds_stream_t stream) {
	HDS_REQUIRE(status_host, "bin_status: status_host must not be NULL");
	if (n <= 0) {
		*static_cast<CountWords*>(status_host) = CountWords{0, 0, 0};
		return HDS_OK;
	}
	HDS_REQUIRE(workspace, "bin_status: workspace must not be NULL");
	HDS_HIP(hipMemcpyAsync(status_host, count_words(workspace, n), sizeof(CountWords), hipMemcpyDeviceToHost,
						   (hipStream_t)stream));
	return HDS_OK;
}

extern "C" int hds_set_lookback_limit(uint32_t polls) {
	g_spin_limit.store(polls, std::memory_order_relaxed);
	return HDS_OK;
}

extern "C" int hds_set_tile_scatter_limit(uint64_t words) {
	g_scatter_words.store(words == 0 || words > kScatterWords ? kScatterWords : words, std::memory_order_relaxed);
	return HDS_OK;
}

extern "C" int hds_bin_emit(int64_t n, int64_t num_pairs, int width, int height, void* workspace,
							void* pairs_workspace, size_t pairs_workspace_bytes, int32_t* values_sorted,
							int32_t* tile_ranges, hds_stream_t stream) {
	if (n > 0 && num_pairs > 0) {
		const int st = check_count_mode(workspace, true, "bin_emit");
		if (st != HDS_OK) return st;
	}
	return bin_emit_launch(n, num_pairs, true, false, width, height, workspace, pairs_workspace, pairs_workspace_bytes,
						   values_sorted, tile_ranges, (hipStream_t)stream);
}

extern "C" int hds_bin_emit_capped(int64_t n, int64_t capacity, int width, int height, void* workspace,
								   void* pairs_workspace, size_t pairs_workspace_bytes, int32_t* values_sorted,
								   int32_t* tile_ranges, hds_stream_t stream) {
	if (n > 0 && capacity > 0) {
		const int st = check_count_mode(workspace, true, "bin_emit_capped");
		if (st != HDS_OK) return st;
	}
	return bin_emit_launch(n, capacity, false, false, width, height, workspace, pairs_workspace, pairs_workspace_bytes,
						   values_sorted, tile_ranges, (hipStream_t)stream);
}

extern "C" int hds_bin_emit_tile_order(int64_t n, int64_t num_pairs, int width, int height, void* workspace,
									   void* pairs_workspace, size_t pairs_workspace_bytes, int32_t* values_sorted,
									   int32_t* tile_ranges, hds_stream_t stream) {
	int mode = kModeTileEmit;
	if (n > 0 && num_pairs > 0) {
		const int st = check_count_mode(workspace, false, "bin_emit_tile_order", &mode);
		if (st != HDS_OK) return st;
	}
	if (mode == kModeTileScatter) {
		HDS_REQUIRE(width > 0 && height > 0, "bin_emit: image size %dx%d must be positive", width, height);
		HDS_REQUIRE(num_pairs < INT32_MAX, "bin_emit: pair count %lld outside [0, 2^31)", (long long)num_pairs);
		HDS_REQUIRE(tile_ranges && values_sorted, "bin_emit: null values_sorted / tile_ranges");
		return scatter_emit_launch(n, num_pairs, true, width, height, workspace, values_sorted, tile_ranges,
								   (hipStream_t)stream);
	}
	return bin_emit_launch(n, num_pairs, true, true, width, height, workspace, pairs_workspace, pairs_workspace_bytes,
						   values_sorted, tile_ranges, (hipStream_t)stream);
}

extern "C" int hds_bin_tile_order_async(int64_t n, const float* means2D, const float* depths, const float* radii,
										const float* conics, const float* colors, const float* opacities, int width,
										int height, float* conic4, float* color_opacity4, void* workspace,
										size_t workspace_bytes, int64_t capacity, void* pairs_workspace,
										size_t pairs_workspace_bytes, int32_t* values_sorted, int32_t* tile_ranges,
										void* status_host, hds_stream_t stream) {
	HDS_REQUIRE(status_host && tile_ranges, "bin_tile_order: null status_host / tile_ranges");
	HDS_REQUIRE(capacity >= 0 && capacity < INT32_MAX, "bin_tile_order: capacity %lld outside [0, 2^31)",
				(long long)capacity);
	HDS_REQUIRE(width > 0 && height > 0, "bin_tile_order: image size %dx%d must be positive", width, height);
	hipStream_t s = (hipStream_t)stream;
	const int tiles_x = (width + HDS_TILE - 1) / HDS_TILE, tiles_y = (height + HDS_TILE - 1) / HDS_TILE;
	const int64_t num_tiles = (int64_t)tiles_x * tiles_y;
	if (n == 0) {
		*static_cast<CountWords*>(status_host) = CountWords{0, 0, 0};
		return bin_emit_launch(0, 0, false, true, width, height, workspace, pairs_workspace, pairs_workspace_bytes,
							   values_sorted, tile_ranges, s);
	}
	HDS_REQUIRE(capacity == 0 || values_sorted, "bin_tile_order: null values_sorted");
	if (scatter_shape(n, num_tiles, g_scatter_words.load(std::memory_order_relaxed)).words > 0) {
		// Counting scatter: no pair workspace is used.
		int st = bin_tile_scatter_launch(n, means2D, depths, radii, conics, colors, opacities, width, height, conic4,
										 color_opacity4, workspace, workspace_bytes, capacity, values_sorted,
										 tile_ranges, s);
		if (st != HDS_OK) return st;
		HDS_HIP(hipMemcpyAsync(status_host, count_words(workspace, n), sizeof(CountWords), hipMemcpyDeviceToHost, s));
		return HDS_OK;
	}
	const PairSpace p = pair_space(capacity);
	HDS_REQUIRE(pairs_workspace && pairs_workspace_bytes >= p.bytes,
				"bin_tile_order: pairs workspace of %zu bytes, need %zu", pairs_workspace_bytes, p.bytes);
	// prepare clears the gaussian control block (slot 0, filled in by bin_count_launch), the pair
	// control block and the tile ranges, so neither half launches a zeroing kernel of its own.
	ZeroRanges zero{};
	zero.p[1] = at<uint32_t>(pairs_workspace, p.ctrl);
	zero.n[1] = (int64_t)(p.bytes - p.ctrl) / 4;
	zero.p[2] = reinterpret_cast<uint32_t*>(tile_ranges);
	zero.n[2] = 2 * num_tiles;
	bool launched = false;
	int st = bin_count_launch(n, means2D, depths, radii, conics, colors, opacities, width, height, conic4,
							  color_opacity4, workspace, workspace_bytes, false, &zero, s, &launched);
	if (st != HDS_OK) return st;
	st = bin_emit_launch(n, capacity, false, true, width, height, workspace, pairs_workspace, pairs_workspace_bytes,
						 values_sorted, tile_ranges, s, true);
	if (st != HDS_OK) return st;
	HDS_HIP(hipMemcpyAsync(status_host, count_words(workspace, n), sizeof(CountWords), hipMemcpyDeviceToHost, s));
	return HDS_OK;
}

// ---------------------------------------------------------------------------------------------
// Binning with the library's own scratch, for callers that cannot allocate device memory.
// ---------------------------------------------------------------------------------------------

namespace {

// Both workspaces of one binning (the per-gaussian one, then the per-pair one, each 256-byte
// aligned) live in this array. Every GPU the library runs on holds its own copy until the process
// ends. On the host the name is only a stand-in for the device address: host code uses the
// per-device address hipGetSymbolAddress returns (static_scratch_ptr), never the name.
constexpr size_t kStaticScratchBytes = size_t(HDS_BIN_STATIC_SCRATCH_MIB) << 20;
__device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

// The device address of `scratch` on the current device, looked up once per device.
int static_scratch_ptr(void** out) {
	static std::mutex mutex;
	static std::vector<void*> ptrs;
	int device = 0;
	HDS_HIP(hipGetDevice(&device));
	std::lock_guard<std::mutex> lock(mutex);
	if ((int)ptrs.size() <= device) ptrs.resize(device + 1, nullptr);
	if (!ptrs[device]) {
		void* ptr = nullptr;
		HDS_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
		HDS_REQUIRE(ptr != nullptr, "bin_static: no device address for the static scratch");
		ptrs[device] = ptr;
	}
	*out = ptrs[device];
	return HDS_OK;
}

}  // namespace

extern "C" int hds_bin_static(int64_t n, const float* means2D, const float* depths, const float* radii,
							  const float* conics, const float* colors, const float* opacities, int width, int height,
							  float* conic4, float* color_opacity4, int64_t capacity, int32_t* values_sorted,
							  int32_t* tile_ranges, void* status, hds_stream_t stream) {
	HDS_REQUIRE(n >= 0 && capacity >= 0, "bin_static: negative gaussian count or capacity");
	HDS_REQUIRE(status && tile_ranges, "bin_static: null pointer argument");
	HDS_REQUIRE(n == 0 || capacity == 0 || values_sorted, "bin_static: null values_sorted");
	const size_t gaussian_bytes = gaussian_space(n).bytes;
	const size_t pair_bytes = pair_space(capacity).bytes;
	HDS_REQUIRE(gaussian_bytes + pair_bytes <= kStaticScratchBytes,
				"bin_static: %lld gaussians and %lld pairs need %zu bytes of scratch, more than its %d MiB",
				(long long)n, (long long)capacity, gaussian_bytes + pair_bytes, HDS_BIN_STATIC_SCRATCH_MIB);
	void* ptr = nullptr;
	int st = static_scratch_ptr(&ptr);
	if (st != HDS_OK) return st;
	hipStream_t s = (hipStream_t)stream;
	void* ws = ptr;
	void* pws = static_cast<char*>(ptr) + align256(gaussian_bytes);
	bool launched = false;
	st = bin_count_launch(n, means2D, depths, radii, conics, colors, opacities, width, height, conic4, color_opacity4,
						  ws, gaussian_bytes, true, nullptr, s, &launched);
	if (st != HDS_OK) return st;
	if (!launched) {
		// No gaussians: empty tile ranges and zero status words, from a zeroed control block.
		const GaussianSpace g = gaussian_space(0);
		zero_kernel<<<1, kThreads, 0, s>>>(at<uint32_t>(ws, g.ctrl), sizeof(CountWords) / 4, nullptr, 0);
		HDS_LAUNCH_CHECK("zero_static_status", s);
		st = bin_emit_launch(0, 0, false, false, width, height, ws, pws, pair_bytes, values_sorted, tile_ranges, s);
		if (st != HDS_OK) return st;
		HDS_HIP(hipMemcpyAsync(status, count_words(ws, 0), sizeof(CountWords), hipMemcpyDefault, s));
		return HDS_OK;
	}
	st = bin_emit_launch(n, capacity, false, false, width, height, ws, pws, pair_bytes, values_sorted, tile_ranges, s);
	if (st != HDS_OK) return st;
	HDS_HIP(hipMemcpyAsync(status, count_words(ws, n), sizeof(CountWords), hipMemcpyDefault, s));
	return HDS_OK;
}
