// gemm_direct.hpp - operands of the 16x16x4 MFMA loaded straight from memory into its lane layout, with no LDS
// staging and no barrier: shared by the pieces kernel (gemm_pieces.hip) and the whole-depth chain kernel
// (gemm_chain.hip). Internal to libnnh.
//
// Mfma<kMf16x4>'s step covers four depth indices: lane l supplies op(A)[row l % 16][4 s + l / 16] and
// op(B)[4 s + l / 16][column l % 16]. A group is 16 consecutive depth indices, four steps; group h of a chunk holds
// the operands of steps 4 h .. 4 h + 3 in a[h][0..3] and b[h][0..3].
#pragma once

#include <hip/hip_runtime.h>

#include "gemm_tile.hpp"

namespace nnh {

// Loads through buffer resources: an element outside the matrix gets an offset past the resource's end,
// which the hardware answers with 0 and no memory access. No branches around the loads, so the compiler keeps
// several slabs of them in flight and waits for each by count.
constexpr int kOob = 0x7fffffff;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const float* base) {
	return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, kOob, 0x00020000);
}

// v[e] of lane group g (lanes 16 g .. 16 g + 15) becomes what v[g] of lane group e held: a 4 x 4 transpose of the
// lane groups' four registers, by two v_permlane32_swap (lane groups 2, 3 of one register with 0, 1 of another) and
// two v_permlane16_swap (odd groups of one with even groups of another), each after the two wait states a VALU
// result needs before a lane swap reads it. Written as assembly: the compiler's builtins for these swaps return the
// first register's result for both at -O3 (hipcc of ROCm 7.2). The registers are taken from a whole-vector bit
// cast: a bit cast of one element of a float vector read element 0 for all four in the same compiler.
__device__ __forceinline__ void transpose4(f32x4& v) {
	typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
	const u32x4 u = __builtin_bit_cast(u32x4, v);
	unsigned x0 = u.x, x1 = u.y, x2 = u.z, x3 = u.w;
	asm volatile(
	    "s_nop 1\n\t"
	    "v_permlane32_swap_b32 %0, %2\n\t"
	    "v_permlane32_swap_b32 %1, %3\n\t"
	    "s_nop 1\n\t"
	    "v_permlane16_swap_b32 %0, %1\n\t"
	    "v_permlane16_swap_b32 %2, %3\n\t"
	    "s_nop 1"
	    : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3));
	v = __builtin_bit_cast(f32x4, u32x4{x0, x1, x2, x3});
}

// G groups of depth indices kc .. kc + 16 G - 1 of the 16 x 16 tile at (m0, n0): kv depth indices are left in the
// chain from kc (PART: fewer than 16). A k-contiguous operand (A not transposed, B transposed) takes, with VA / VB,
// one 16-byte load per group (lane group g: depths 16 h + 4 g .. + 3 of its row), transposed across the lane
// groups by mma_groups; otherwise one element per lane and step. Rows and columns outside the matrix, and with PART
// depths past the chain's end, load +0 without touching memory. A group's offsets stay below 16 rows of a leading
// dimension, which the caller keeps below 2^24.
template <bool TA, bool TB, bool VA, bool VB, bool PART, int G>
__device__ __forceinline__ void load_groups(const float* A, int lda, const float* B, int ldb, int m0, int n0, int kc,
                                            int kv, int r, int j, bool row_in, bool col_in, f32x4* a, f32x4* b) {
#pragma unroll
	for (int h = 0; h < G; ++h) {
		const int k0 = kc + 16 * h;
		const __amdgpu_buffer_rsrc_t ares = rsrc(TA ? A + (int64_t)k0 * lda + m0 : A + (int64_t)m0 * lda + k0);
		const __amdgpu_buffer_rsrc_t bres = rsrc(TB ? B + (int64_t)n0 * ldb + k0 : B + (int64_t)k0 * ldb + n0);
		if (VA) a[h] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ares, row_in ? (r * lda + 4 * j) * 4 : kOob, 0, 0));
		if (VB) b[h] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(bres, col_in ? (r * ldb + 4 * j) * 4 : kOob, 0, 0));
#pragma unroll
		for (int e = 0; e < 4; ++e) {
			const int d = 4 * e + j;
			const bool din = !PART || d < kv;
			if (!VA) {
				const int aoff = row_in && din ? (TA ? d * lda + r : r * lda + d) * 4 : kOob;
				a[h][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ares, aoff, 0, 0));
			}
			if (!VB) {
				const int boff = col_in && din ? (TB ? r * ldb + d : d * ldb + r) * 4 : kOob;
				b[h][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(bres, boff, 0, 0));
			}
		}
	}
}

// The MFMA steps of G loaded groups, in depth order, into acc. PART: steps past the chain's end (depth offset kv
// and beyond) multiply A's +0 by B's fill turned into -0, which leaves every sum as it was, -0 included.
template <bool VA, bool VB, bool PART, int G>
__device__ __forceinline__ void mma_groups(f32x4* a, f32x4* b, int kv, int j, f32x4& acc) {
#pragma unroll
	for (int h = 0; h < G; ++h) {
		if (VA) transpose4(a[h]);
		if (VB) transpose4(b[h]);
#pragma unroll
		for (int e = 0; e < 4; ++e) {
			float bv = b[h][e];
			if (PART) bv = __builtin_bit_cast(float, __builtin_bit_cast(unsigned, bv) | (4 * e + j < kv ? 0u : 0x80000000u));
			acc = Mfma<kMf16x4>::mma(a[h][e], bv, acc);
		}
	}
}

}  // namespace nnh
