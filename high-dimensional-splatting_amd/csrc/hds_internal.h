/*
 * Internal helpers of the HIP library: error reporting behind the C ABI, launch checks, wave64
 * primitives and the split-bf16 MFMA building blocks. Not part of the public interface
 * (include/hds_rasterizer.h is).
 */
#ifndef HDS_INTERNAL_H
#define HDS_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hds_common.h"

/* ------------------------------------------------------------------------------------------- */
/* Error reporting: every entry point returns an HDS_* status and leaves a thread-local message.  */
/* ------------------------------------------------------------------------------------------- */

#define HDS_OK 0
#define HDS_ERR_INVALID 1
#define HDS_ERR_RUNTIME 2

int hds_set_error(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
bool hds_debug_sync_enabled();

/* Checks the last launch; with HDS_DEBUG set, also synchronises the stream and checks execution. */
int hds_check_launch(const char* kernel, hipStream_t stream);

#define HDS_LAUNCH_CHECK(name, stream)                         \
	do {                                                       \
		int _st = hds_check_launch((name), (stream));          \
		if (_st != HDS_OK) return _st;                         \
	} while (0)

#define HDS_REQUIRE(cond, ...)                                 \
	do {                                                       \
		if (!(cond)) return hds_set_error(HDS_ERR_INVALID, __VA_ARGS__); \
	} while (0)

#define HDS_HIP(call)                                                                              \
	do {                                                                                           \
		hipError_t _e = (call);                                                                    \
		if (_e != hipSuccess)                                                                      \
			return hds_set_error(HDS_ERR_RUNTIME, "%s failed: %s", #call, hipGetErrorString(_e)); \
	} while (0)

/* Brackets one kernel launch with HIP events while hds_profile_begin() recording is on (no-op
 * otherwise): construct it right before the launch and call stop() right after it. */
class HdsKernelTimer {
   public:
	HdsKernelTimer(const char* name, hipStream_t stream);
	void stop();
	HdsKernelTimer(const HdsKernelTimer&) = delete;
	HdsKernelTimer& operator=(const HdsKernelTimer&) = delete;

   private:
	int64_t slot_;
	hipStream_t stream_;
};

/* Sets *out to this device's side stream (see hds_runtime.hip). */
int hds_side_stream(hipStream_t* out);

static inline unsigned hds_blocks(int64_t n, int threads) { return (unsigned)((n + threads - 1) / threads); }

/* ------------------------------------------------------------------------------------------- */
/* Wave64 primitives.                                                                            */
/* ------------------------------------------------------------------------------------------- */

#define HDS_WAVE 64

__device__ static inline int hds_lane() { return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

/* Number of set bits of mask in lanes below this one. */
__device__ static inline int hds_rank_below(uint64_t mask) {
	return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ static inline uint64_t hds_ballot(bool pred) { return __builtin_amdgcn_ballot_w64(pred); }

/* Keeps the compiler from moving the LDS accesses of one wave across this point. A wave's LDS
 * instructions execute in order, so lanes then see each other's earlier LDS writes. It is not a
 * memory fence: a fence would also wait for the wave's outstanding global loads, including the
 * asynchronous LDS DMA of the next batch. */
__device__ static inline void hds_wave_fence() {
	asm volatile("" ::: "memory");
	__builtin_amdgcn_wave_barrier();
	asm volatile("" ::: "memory");
}

/* Pins a value in a VGPR of its own. This compiler (ROCm 7.2 clang) folds v_permlane16/32_swap
 * calls whose operands are different elements of one MFMA result vector into a single swap, so
 * every element after the first silently receives the first one's result; passing each element
 * through this opaque move first keeps the swaps apart. */
__device__ static inline uint32_t hds_opaque(uint32_t v) {
	asm volatile("" : "+v"(v));
	return v;
}

/* The value of lane (this lane ^ m), m a power of two below 64 that is a constant at the call
 * (after unrolling), by the cheapest exchange for each stride instead of a ds_bpermute: DPP quad
 * permutes for 1 and 2 (VALU), ds_swizzle for 4 and 8, and the row swaps for 16 and 32
 * (v_permlane16/32_swap exchange the odd rows of their first operand with the even rows of their
 * second; with the same value in both, r[1] holds what the lower row of each pair needs and r[0]
 * what the upper one needs). Each value passes through hds_opaque first, which keeps the compiler
 * from merging the swaps of different values into one. */
__device__ __attribute__((always_inline)) static inline uint32_t hds_lane_xor(uint32_t v, int m) {
	const uint32_t u = hds_opaque(v);
	if (m == 1) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
	if (m == 2) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x4E, 0xF, 0xF, false);  // quad_perm 2,3,0,1
	if (m == 4) return (uint32_t)__builtin_amdgcn_ds_swizzle((int)u, 0x1F | (4 << 10));           // and 31, xor 4
	if (m == 8) return (uint32_t)__builtin_amdgcn_ds_swizzle((int)u, 0x1F | (8 << 10));           // and 31, xor 8
	const int lane = (int)(threadIdx.x & (HDS_WAVE - 1));
	if (m == 16) {
		const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
		return (lane & 16) ? (uint32_t)r[0] : (uint32_t)r[1];
	}
	const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
	return (lane & 32) ? (uint32_t)r[0] : (uint32_t)r[1];
}

/* Inclusive prefix sum over the 64 lanes (lane l gets v_0 + ... + v_l) by DPP moves instead of a
 * chain of ds_bpermutes: row shifts by 1, 2, 4 and 8 inside each 16-lane row (lanes shifted in from
 * outside the row read 0), then lane 15 of rows 0 and 2 added to rows 1 and 3 (row_bcast:15) and
 * lane 31 to rows 2 and 3 (row_bcast:31); rows the row mask leaves out keep the old value 0. */
__device__ __attribute__((always_inline)) static inline uint32_t hds_wave_inclusive_scan(uint32_t v) {
	uint32_t x = v;
	x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xF, 0xF, true);   // row_shr:1
	x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xF, 0xF, true);   // row_shr:2
	x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xF, 0xF, true);   // row_shr:4
	x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xF, 0xF, true);   // row_shr:8
	x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xA, 0xF, false);  // row_bcast:15
	x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xC, 0xF, false);  // row_bcast:31
	return x;
}

/* hds_lane_xor of a float (same conditions on the mask). */
__device__ __attribute__((always_inline)) static inline float hds_shfl_xor(float v, int mask) {
	return __builtin_bit_cast(float, hds_lane_xor(__builtin_bit_cast(uint32_t, v), mask));
}

/* Sum over all 64 lanes, result in every lane. */
__device__ static inline float hds_wave_sum(float v) {
#pragma unroll
	for (int off = 32; off > 0; off >>= 1) v += hds_shfl_xor(v, off);
	return v;
}

__device__ static inline int hds_wave_max(int v) {
#pragma unroll
	for (int off = 32; off > 0; off >>= 1) v = max(v, (int)hds_lane_xor((uint32_t)v, off));
	return v;
}

/*
 * Reduce-scatter of 8 values over the wave: afterwards every lane of the octet q = (lane >> 3) & 7
 * holds the wave-wide sum of v[q]. 10 shuffles instead of the 48 of eight full reductions.
 */
__device__ static inline float hds_wave_reduce_scatter8(float v[8], int lane) {
	{
		const bool hi = lane & 32;
#pragma unroll
		for (int i = 0; i < 4; i++) {
			const float send = hi ? v[i] : v[i + 4];
			const float keep = hi ? v[i + 4] : v[i];
			v[i] = keep + hds_shfl_xor(send, 32);
		}
	}
	{
		const bool hi = lane & 16;
#pragma unroll
		for (int i = 0; i < 2; i++) {
			const float send = hi ? v[i] : v[i + 2];
			const float keep = hi ? v[i + 2] : v[i];
			v[i] = keep + hds_shfl_xor(send, 16);
		}
	}
	{
		const bool hi = lane & 8;
		const float send = hi ? v[0] : v[1];
		const float keep = hi ? v[1] : v[0];
		v[0] = keep + hds_shfl_xor(send, 8);
	}
	v[0] += hds_shfl_xor(v[0], 4);
	v[0] += hds_shfl_xor(v[0], 2);
	v[0] += hds_shfl_xor(v[0], 1);
	return v[0];
}

/* ------------------------------------------------------------------------------------------- */
/* Split-bf16 MFMA. CDNA4 has no TF32 matrix path, so an fp32 operand x is carried as           */
/* hi = bf16(x) and lo = bf16(x - hi) (both round-to-nearest-even) and a product as             */
/* hi*hi + hi*lo + lo*hi: three v_mfma_f32_16x16x32_bf16 with fp32 accumulation, relative error */
/* about 2^-16 per product, against TF32's 2^-11. One packed dword per element holds             */
/* hi (bits 0-15) and lo (bits 16-31), so LDS stores one word per operand element.              */
/* ------------------------------------------------------------------------------------------- */

typedef __bf16 hds_bf16x8 __attribute__((ext_vector_type(8)));
typedef float hds_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t hds_u32x4 __attribute__((ext_vector_type(4)));

__device__ static inline uint32_t hds_bf16_bits(__bf16 h) { return (uint32_t)__builtin_bit_cast(unsigned short, h); }

/* x -> hi (bits 0-15) | lo (bits 16-31). The second packed conversion rounds x again, to the same hi,
 * beside the residual, so the pair is packed by the conversion itself (4 instructions). */
__device__ static inline uint32_t hds_split_pack(float x) {
	typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
	typedef float f32x2 __attribute__((ext_vector_type(2)));
	const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x, 0.0f}, bf16x2));
	const float hi = __builtin_bit_cast(float, h << 16);
	return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x, x - hi}, bf16x2));
}

/* Eight packed words -> the hi and lo bf16x8 operands of one MFMA. */
__device__ static inline void hds_unpack8(const uint32_t d[8], hds_bf16x8& hi, hds_bf16x8& lo) {
	hds_u32x4 h, l;
#pragma unroll
	for (int i = 0; i < 4; i++) {
		/* bytes 0,1 of d[2i] and d[2i+1] -> hi pair; bytes 2,3 -> lo pair */
		h[i] = __builtin_amdgcn_perm(d[2 * i + 1], d[2 * i], 0x05040100u);
		l[i] = __builtin_amdgcn_perm(d[2 * i + 1], d[2 * i], 0x07060302u);
	}
	hi = __builtin_bit_cast(hds_bf16x8, h);
	lo = __builtin_bit_cast(hds_bf16x8, l);
}

typedef float hds_f32x16 __attribute__((ext_vector_type(16)));

/* acc += A * B on 32x32x16 tiles, split-bf16 operands. Lane layouts (gfx950, checked on hardware):
 * A[row = lane % 32][k = 8 (lane / 32) + j], B[k = 8 (lane / 32) + j][col = lane % 32],
 * D[row = 8 (i / 4) + 4 (lane / 32) + i % 4][col = lane % 32] for the 16 accumulators i. */
__device__ static inline hds_f32x16 hds_mfma32_split(const hds_bf16x8& a_hi, const hds_bf16x8& a_lo,
													 const hds_bf16x8& b_hi, const hds_bf16x8& b_lo,
													 hds_f32x16 acc) {
	acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_lo, b_hi, acc, 0, 0, 0);
	acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_hi, b_lo, acc, 0, 0, 0);
	acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_hi, b_hi, acc, 0, 0, 0);
	return acc;
}

/* Two floats -> packed bf16 hi pair and bf16 lo (residual) pair, round-to-nearest-even. */
__device__ static inline void hds_split_pair(float x0, float x1, uint32_t& hi, uint32_t& lo) {
	typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
	const bf16x2 h = __builtin_convertvector((float __attribute__((ext_vector_type(2)))){x0, x1}, bf16x2);
	hi = __builtin_bit_cast(uint32_t, h);
	const float r0 = x0 - hds_u2f(hi << 16), r1 = x1 - hds_u2f(hi & 0xffff0000u);
	const bf16x2 l = __builtin_convertvector((float __attribute__((ext_vector_type(2)))){r0, r1}, bf16x2);
	lo = __builtin_bit_cast(uint32_t, l);
}

/* One MFMA result element as an independent 32-bit operand for a lane swap. */
__device__ static inline uint32_t hds_swap_operand(float v) { return hds_opaque(__builtin_bit_cast(uint32_t, v)); }

/* Tile of a work-group. Work-groups are dispatched round-robin over the 8 XCDs, so work-group b
 * runs on XCD b % 8. The image is cut into 2x2 super-blocks of tiles, dealt to the XCDs round-robin,
 * and an XCD's consecutive work-groups render the four tiles of one super-block: neighbouring tiles,
 * which share gaussians, then stage those gaussians through the same L2, while every XCD still gets
 * an even share of the dense centre (contiguous bands of tiles per XCD left the busiest XCD with 1.33x
 * the mean work at the headline scene; 4x2 and 4x4 super-blocks were measured slower than 2x2, which
 * took the blend forward from 0.62 to 0.58 ms). Padding work-groups get -1. */
#define HDS_XCDS 8
#define HDS_SUPER 2  // super-block edge in tiles
static inline unsigned hds_xcd_grid(int tiles_x, int num_tiles) {
	const int tiles_y = num_tiles / tiles_x;
	const int supers = ((tiles_x + HDS_SUPER - 1) / HDS_SUPER) * ((tiles_y + HDS_SUPER - 1) / HDS_SUPER);
	return (unsigned)(((supers + HDS_XCDS - 1) / HDS_XCDS) * HDS_XCDS * HDS_SUPER * HDS_SUPER);
}
__device__ static inline int hds_xcd_tile(int block, int tiles_x, int num_tiles) {
	const int tiles_y = num_tiles / tiles_x;
	const int sx = (tiles_x + HDS_SUPER - 1) / HDS_SUPER, sy = (tiles_y + HDS_SUPER - 1) / HDS_SUPER;
	const int xcd = block % HDS_XCDS, r = block / HDS_XCDS;
	const int k = r % (HDS_SUPER * HDS_SUPER), super = (r / (HDS_SUPER * HDS_SUPER)) * HDS_XCDS + xcd;
	if (super >= sx * sy) return -1;
	const int tx = (super % sx) * HDS_SUPER + k % HDS_SUPER, ty = (super / sx) * HDS_SUPER + k / HDS_SUPER;
	return tx < tiles_x && ty < tiles_y ? ty * tiles_x + tx : -1;
}

/* acc += A * B with A, B given as split-bf16 pairs (small terms first). */
__device__ static inline hds_f32x4 hds_mfma_split(const hds_bf16x8& a_hi, const hds_bf16x8& a_lo,
												  const hds_bf16x8& b_hi, const hds_bf16x8& b_lo,
												  hds_f32x4 acc) {
	acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_lo, b_hi, acc, 0, 0, 0);
	acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_hi, b_lo, acc, 0, 0, 0);
	acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_hi, b_hi, acc, 0, 0, 0);
	return acc;
}

/* ------------------------------------------------------------------------------------------- */
/* Blend helpers shared by the forward and backward tile walks.                                 */
/* ------------------------------------------------------------------------------------------- */

/* Can the gaussian reach alpha >= 1/255 anywhere in the rectangle [x0, x1] x [y0, y1] of pixel
 * centres? A conservative cull: it only drops gaussians whose alpha is below 1/255 at every pixel
 * of the rectangle, which the per-pixel test (forward.cu:207-208) would skip anyway, so no pixel's
 * result changes (features.cu:8-22 culls with the looser bounding box of the same ellipse).
 *
 * alpha = op exp(-q / 2) >= 1/255 needs q <= 2 ln(255 op), with q(d) = a dx^2 + 2 b dx dy + c dy^2
 * and d = pixel - mean. q is convex (a > 0, ac - b^2 > 0), so over the rectangle it is 0 when the
 * mean lies inside and otherwise smallest on one of the four edges, where it is a quadratic in one
 * variable, minimised at the clamped stationary point. On an edge dx = e it is evaluated as
 * c (dy + b e / c)^2 + (det / c) e^2, a sum of non-negative terms with no cancellation.
 *
 * The margin covers the rounding of the per-pixel q, whose terms can cancel for elongated
 * gaussians: 1e-5 of the largest term magnitude over the rectangle (the fp32 error of the
 * per-pixel form is below 1e-6 of it), plus 0.1% of the threshold and 0.01 for the exp and log.
 * Degenerate or NaN input keeps the gaussian. */
__device__ static inline bool hds_block_reach(float2 mean, float4 conic_op, float x0, float x1, float y0, float y1) {
	const float a = conic_op.x, b = conic_op.y, c = conic_op.z;
	const float det = a * c - b * b;
	const float thr = (2.0f * 0.693147182f) * __builtin_amdgcn_logf(255.0f * conic_op.w);
	const float lx = x0 - mean.x, hx = x1 - mean.x, ly = y0 - mean.y, hy = y1 - mean.y;
	if (!(a > 0.0f && c > 0.0f && det > 0.0f)) return true;
	if (lx <= 0.0f && hx >= 0.0f && ly <= 0.0f && hy >= 0.0f) return true;
	const float ia = __builtin_amdgcn_rcpf(a), ic = __builtin_amdgcn_rcpf(c);
	float qmin = 3.0e38f;
	// Vertical edges dx = e: dy* = -b e / c clamped to [ly, hy].
#pragma unroll
	for (int k = 0; k < 2; k++) {
		const float e = k ? hx : lx;
		const float dy = fminf(fmaxf(-b * e * ic, ly), hy);
		const float t = dy + b * e * ic;
		qmin = fminf(qmin, c * t * t + det * ic * e * e);
	}
	// Horizontal edges dy = e: dx* = -b e / a clamped to [lx, hx].
#pragma unroll
	for (int k = 0; k < 2; k++) {
		const float e = k ? hy : ly;
		const float dx = fminf(fmaxf(-b * e * ia, lx), hx);
		const float t = dx + b * e * ia;
		qmin = fminf(qmin, a * t * t + det * ia * e * e);
	}
	const float mx2 = fmaxf(lx * lx, hx * hx), my2 = fmaxf(ly * ly, hy * hy);
	const float margin = 1e-5f * ((a + fabsf(b)) * mx2 + (c + fabsf(b)) * my2) + 1e-3f * fabsf(thr) + 0.01f;
	return !(qmin > thr + margin);
}

/* Raw alpha of a gaussian at a pixel centre, forward.cu:197-208; G and the offsets are returned
 * for the backward. */
__device__ static inline float hds_raw_alpha(float px, float py, float2 mean, float4 conic_op, float& G,
											 float& dx, float& dy) {
	dx = px - mean.x;
	dy = py - mean.y;
	// The oracle's arithmetic (hds_common.h), bit for bit.
	return hds_gauss_alpha(dx, dy, conic_op.x, conic_op.y, conic_op.z, conic_op.w, &G);
}

#endif /* HDS_INTERNAL_H */
