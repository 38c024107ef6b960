/*
 * Asynchronous staging of a tile's gaussian batches for the blend kernels.
 *
 * The walks read each batch of 64 gaussians of a tile list from LDS. Staging the next batch while
 * the current one is processed hides the gather latency (feature rows are 64 scattered 128-512 byte
 * rows per batch): the feature rows go straight from HBM to LDS with gfx950's
 * global_load_lds_dwordx4 (no registers, no wait until the batch is needed), into one of two
 * buffers that are separate __shared__ arrays so the compiler's wait insertion can tell the buffer
 * being filled from the one being read. Rows are stored as raw fp32, S floats per row, and split
 * into bf16 hi/lo MFMA operands when they are read.
 */
#ifndef HDS_STAGE_H
#define HDS_STAGE_H

#include "hds_internal.h"

typedef __attribute__((address_space(3))) void hds_lds_void;

/* Waits for this wave's outstanding vector-memory operations, including LDS DMA. Before a barrier it
 * makes every wave's staged rows visible to the whole work-group. */
__device__ static inline void hds_wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

/* Physical 16-byte chunk of logical chunk c in staged row r of kChunks chunks. With kSwizzle the
 * chunks of a row are XOR-permuted by the row's low four bits (three for 8-chunk rows), so 16 lanes
 * reading the same logical chunk of rows with distinct r mod 16 hit 16 different bank groups of the
 * 64 banks (rows are whole multiples of 64 words apart for S >= 64). */
template <bool kSwizzle, int kChunks>
__device__ static inline int hds_stage_chunk(int c, int r) {
	static_assert(kChunks >= 8 && (kChunks & (kChunks - 1)) == 0, "rows of 8, 16 or 32 chunks");
	return kSwizzle ? (c ^ (r & (kChunks >= 16 ? 15 : 7))) : c;
}

/* Issues the copy of rows 0..cnt-1 (S channels from c0 of features[gids[row]]) into buf, one
 * 1 KB block of rows per wave instruction; cnt <= kRowsMax, the work-group has 256 threads. The
 * caller waits with hds_wait_vmem() and a barrier before reading. */
template <int S, bool kSwizzle, int kRowsMax>
__device__ inline void hds_stage_rows_async(float* buf, const float* features, int channels, int c0,
											const int* gids, int cnt, int tid) {
	constexpr int kChunks = S / 4;              // 16-byte chunks per row
	constexpr int kRowsPerOp = 64 / kChunks;    // rows per 1 KB wave instruction
	constexpr int kOps = kRowsMax / kRowsPerOp; // instructions per batch
	static_assert(kRowsMax % kRowsPerOp == 0, "batch must be whole 1 KB blocks");
	const int lane = tid & 63, wave = tid >> 6;
	const int chunk = lane % kChunks;
	// Not unrolled: one row address live at a time keeps this off the walk's register budget.
#pragma unroll 1
	for (int op = wave; op < kOps; op += 4) {
		const int row = op * kRowsPerOp + lane / kChunks;
		if (row < cnt) {
			const float* src = features + (size_t)gids[row] * channels + c0 + 4 * hds_stage_chunk<kSwizzle, kChunks>(chunk, row);
			__builtin_amdgcn_global_load_lds(src, (hds_lds_void*)(buf + op * 256), 16, 0, 0);
		}
	}
}

/* Gaussian records of one pipeline slot, filled by LDS DMA: mean x / y, conic4 = (a, b, c, opacity)
 * and, for the RGB walks, color_opacity4. Each slot is its own __shared__ object. */
template <int kB, bool kColor>
struct HdsHeaderSlot {
	float mx[kB];
	float my[kB];
	float4 conic[kB];
	float4 color[kColor ? kB : 1];
};

/* Issues the copy of the records of rows 0..cnt-1 (gaussians gids[row]) into h: one DMA
 * instruction per array, spread over the four waves. */
template <int kB, bool kColor>
__device__ inline void hds_stage_headers_async(HdsHeaderSlot<kB, kColor>& h, const float2* means2D,
											   const float4* conic4, const float4* color4,
											   const int* gids, int cnt, int tid) {
	static_assert(kB <= 64, "one row per lane");
	const int lane = tid & 63, wave = tid >> 6;
	if (lane >= cnt) return;
	const int gid = gids[lane];
	if (wave == 0) {
		__builtin_amdgcn_global_load_lds(conic4 + gid, (hds_lds_void*)h.conic, 16, 0, 0);
	} else if (wave == 1) {
		if constexpr (kColor) __builtin_amdgcn_global_load_lds(color4 + gid, (hds_lds_void*)h.color, 16, 0, 0);
	} else if (wave == 2) {
		__builtin_amdgcn_global_load_lds(&means2D[gid].x, (hds_lds_void*)h.mx, 4, 0, 0);
	} else {
		__builtin_amdgcn_global_load_lds(&means2D[gid].y, (hds_lds_void*)h.my, 4, 0, 0);
	}
}

/* One 16-byte LDS read kept as a single vector load. Left alone, the compiler splits a vector
 * load whose elements are used separately into scalar loads and merges them back into
 * ds_read_b128 late, and the merged access has lost the alias information that tells it apart from
 * the LDS DMA in flight: the wait-count pass then waits for all outstanding DMA before it. */
__device__ static inline hds_u32x4 hds_lds_read128(const uint32_t* p) {
	hds_u32x4 v = *reinterpret_cast<const hds_u32x4*>(p);
	asm volatile("" : "+v"(v));
	return v;
}

/* Eight fp32 values -> the split-bf16 hi and lo operands of one MFMA. */
__device__ static inline void hds_split8(const float (&v)[8], hds_bf16x8& hi, hds_bf16x8& lo) {
	uint32_t h[4], l[4];
#pragma unroll
	for (int i = 0; i < 4; i++) hds_split_pair(v[2 * i], v[2 * i + 1], h[i], l[i]);
	hi = __builtin_bit_cast(hds_bf16x8, hds_u32x4{h[0], h[1], h[2], h[3]});
	lo = __builtin_bit_cast(hds_bf16x8, hds_u32x4{l[0], l[1], l[2], l[3]});
}

#endif /* HDS_STAGE_H */
