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

// G groups of depth indices kc .. kc + 16 G - 1 of the 16 x 16 tile at (m0, n0): kv depth indices are left in the
// chain from kc (PART: fewer than 16). A k-contiguous operand (A not transposed, B transposed) takes, with VA / VB,
// one 16-byte load per group (lane group g: depths 16 h + 4 g .. + 3 of its row), reordered through LDS by
// mma_groups; otherwise one element per lane and step. Rows and columns outside the matrix, and with PART
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

// Per-wave LDS staging of a k-contiguous operand's groups, in place of a transpose across lane groups (lane swaps
// are VALU instructions, and VALU work of a wave between its dependent MFMAs lengthens every chain step: measured
// 33 cycles per dependent 16x16x4 step alone, 53-56 with one four-swap transpose per four steps). A slot holds one
// group, 16 rows of 16 depths at a pitch of 20 floats; depth 4 t + e of a row sits at 4 e + t, so that lane group g's
// four depths of its row (4 s + g for the group's four steps s) are one 16-byte read. Lane (r, g) writes its 16-byte
// load (depths 4 g .. 4 g + 3) as four 4-byte stores; the pitch puts the 64 lanes of each store on 64 banks.
constexpr int kKPitch = 20;
constexpr int kKSlot = 16 * kKPitch;  // floats of one slot

__device__ __forceinline__ void kperm_write(float* slot, const f32x4& v, int r, int j) {
#pragma unroll
	for (int e = 0; e < 4; ++e) slot[r * kKPitch + 4 * e + j] = v[e];
}

__device__ __forceinline__ f32x4 kperm_read(const float* slot, int r, int j) {
	return *reinterpret_cast<const f32x4*>(slot + r * kKPitch + 4 * j);
}

// Orders a wave's LDS accesses for the compiler (the LDS runs one wave's accesses in issue order).
__device__ __forceinline__ void wave_lds_fence() {
	__builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
	__builtin_amdgcn_wave_barrier();
	__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The MFMA steps of G loaded groups, in depth order, into acc. VA / VB: that operand came as 16-byte loads and goes
// through the wave's two LDS slots (la, lb: 2 kKSlot floats each), group h + 1's round trip issued before group h's
// MFMAs. PART: steps past the chain's end (depth offset kv and beyond) multiply A's +0 by B's fill turned into -0,
// which leaves every sum as it was, -0 included.
template <bool VA, bool VB, bool PART, int G>
__device__ __forceinline__ void mma_groups(f32x4* a, f32x4* b, int kv, int r, int j, f32x4& acc, float* la,
                                           float* lb) {
	f32x4 ca = a[0], cb = b[0];
	if (VA || VB) {
		if (VA) kperm_write(la, a[0], r, j);
		if (VB) kperm_write(lb, b[0], r, j);
		wave_lds_fence();
		if (VA) ca = kperm_read(la, r, j);
		if (VB) cb = kperm_read(lb, r, j);
	}
#pragma unroll
	for (int h = 0; h < G; ++h) {
		f32x4 na = ca, nb = cb;
		if ((VA || VB) && h + 1 < G) {
			float* sa = la + ((h + 1) & 1) * kKSlot;
			float* sb = lb + ((h + 1) & 1) * kKSlot;
			if (VA) kperm_write(sa, a[h + 1], r, j);
			if (VB) kperm_write(sb, b[h + 1], r, j);
			wave_lds_fence();
			if (VA) na = kperm_read(sa, r, j);
			if (VB) nb = kperm_read(sb, r, j);
		}
		const f32x4 av = VA ? ca : a[h], bw = VB ? cb : b[h];
#pragma unroll
		for (int e = 0; e < 4; ++e) {
			float bv = bw[e];
			if (PART) bv = __builtin_bit_cast(float, __builtin_bit_cast(unsigned, bv) | (4 * e + j < kv ? 0u : 0x80000000u));
			acc = Mfma<kMf16x4>::mma(av[e], bv, acc);
		}
		if (VA) ca = na;
		if (VB) cb = nb;
	}
}

}  // namespace nnh
