// gemm_direct.hpp - operands of the 16x16x4 MFMA loaded straight from memory into its lane layout, with no LDS
// staging and no barrier: shared by the pieces kernel (gemm_pieces.hip) and the whole-depth chain kernel
// (gemm_chain.hip). Internal to libnnh.
//
// Mfma<kMf16x4>'s step covers four depth indices: lane l supplies op(A)[row l % 16][4 s + l / 16] and
// op(B)[4 s + l / 16][column l % 16]. A group is 16 consecutive depth indices, four steps; group h of a chunk holds
// the operands of steps 4 h .. 4 h + 3 in a[h][0..3] and b[h][0..3].
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "gelu_math.hpp"
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

// One 32 x 32 tile of a whole-depth product (the chain kernel, gemm_chain.hip; also the first product of the chain +
// pieces pair launch, gemm_pieces.hip): waves 0-3 of the workgroup each own a 16 x 16 quarter, block is the tile's
// index among the product's workgroups. Every output is one chain over the whole depth in order, four depth steps
// per instruction; the wave streams the depth in chunks of kChainChunkGroups groups, the next chunk's loads issued
// before the current chunk's MFMAs. Accumulate follows the reference's order (kAccAfter): old C joins the chain
// after the first 256 steps, or is added at the end of a shorter one. No barrier: only the wave's own LDS slots.
constexpr int kChainChunkGroups = 8;  // 128 depth indices

template <bool TA, bool TB, bool VEC>
__device__ __forceinline__ void chain4_tile(const GemmArgs& p, int block, int wave, int lane) {
	constexpr int kChunkGroups = kChainChunkGroups;
	constexpr bool KA = VEC && !TA, KB = VEC && TB;
	const int tiles = p.tiles_m * p.tiles_n;
	const int lid = xcd_remap(block, tiles * p.batch_count);
	const int t = lid % tiles, bi = lid / tiles;
	const int m0 = (t / p.tiles_n) * 32 + 16 * (wave >> 1), n0 = (t % p.tiles_n) * 32 + 16 * (wave & 1);
	int64_t oa = 0, ob = 0, oc = 0;
	if (p.batch.ndim > 0) batch_offsets(p.batch, bi, oa, ob, oc);
	const float* __restrict__ A = p.a + oa;
	const float* __restrict__ B = p.b + ob;
	float* __restrict__ Cp = p.c + oc;
	const int lda = (int)p.lda, ldb = (int)p.ldb;
	const int r = lane & 15, j = lane >> 4;
	const bool row_in = m0 + r < p.m, col_in = n0 + r < p.n;
	const int K = p.k;
	// the wave's LDS slots for its k-contiguous operands (two groups each)
	__shared__ __align__(16) float kst[(KA || KB) ? 4 * 2 * 2 * kKSlot : 1];
	float* const la = kst + (KA || KB ? wave * 4 * kKSlot : 0);
	float* const lb = la + 2 * kKSlot;
	f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
	// register e of lane l holds row 4 (l / 16) + e, column l % 16 of the quarter
	const int col = n0 + r;
	auto add_old = [&]() {
#pragma unroll
		for (int e = 0; e < 4; ++e) {
			const int row = m0 + 4 * j + e;
			if (row < p.m && col < p.n) acc[e] = Cp[(int64_t)row * p.ldc + col] + acc[e];
		}
	};
	using G4 = std::integral_constant<int, 4>;
	using G2 = std::integral_constant<int, 2>;
	using G1 = std::integral_constant<int, 1>;
	auto load8 = [&](int kc, f32x4 (&a)[kChunkGroups], f32x4 (&b)[kChunkGroups]) {
		load_groups<TA, TB, KA, KB, false, kChunkGroups>(A, lda, B, ldb, m0, n0, kc, K - kc, r, j, row_in, col_in, a, b);
	};
	auto run8 = [&](f32x4 (&a)[kChunkGroups], f32x4 (&b)[kChunkGroups]) {
		mma_groups<KA, KB, false, kChunkGroups>(a, b, 0, r, j, acc, la, lb);
	};
	// whole chunks, two register sets: chunk c + 1's loads in flight while chunk c's MFMAs run
	const int n128 = K / 128;
	const bool acc_mid = p.accumulate && K > kAccAfter;  // then n128 >= 2: old C joins after chunk 1
	f32x4 a0[kChunkGroups], b0[kChunkGroups], a1[kChunkGroups], b1[kChunkGroups];
	if (n128 > 0) load8(0, a0, b0);
	int c = 0;
	for (; c + 2 <= n128; c += 2) {
		load8(128 * (c + 1), a1, b1);
		__builtin_amdgcn_sched_barrier(0);
		run8(a0, b0);
		__builtin_amdgcn_sched_barrier(0);
		// unconditional (the last pair reloads its second chunk, unused): no branch, so the waits stay counted
		load8(128 * min(c + 2, n128 - 1), a0, b0);
		__builtin_amdgcn_sched_barrier(0);
		run8(a1, b1);
		__builtin_amdgcn_sched_barrier(0);
		if (c == 0 && acc_mid) add_old();
	}
	if (c < n128) run8(a0, b0);
	// the rest of the depth: 64, 32, 16 indices, then fewer than 16
	int kc = 128 * n128;
	auto part = [&](auto groups_tag, auto part_tag) {
		constexpr int G = decltype(groups_tag)::value;
		constexpr bool PART = decltype(part_tag)::value;
		f32x4 a[G], b[G];
		load_groups<TA, TB, KA && !PART, KB && !PART, PART, G>(A, lda, B, ldb, m0, n0, kc, K - kc, r, j, row_in, col_in,
		                                                       a, b);
		__builtin_amdgcn_sched_barrier(0);
		mma_groups<KA && !PART, KB && !PART, PART, G>(a, b, K - kc, r, j, acc, la, lb);
		__builtin_amdgcn_sched_barrier(0);
	};
	if (K - kc >= 64) {
		part(G4{}, std::false_type{});
		kc += 64;
	}
	if (K - kc >= 32) {
		part(G2{}, std::false_type{});
		kc += 32;
	}
	if (K - kc >= 16) {
		part(G1{}, std::false_type{});
		kc += 16;
	}
	if (kc < K) part(G1{}, std::true_type{});
	// the store (gemm.cpp:176-187, 245-252) and the op's bias and ReLU (src/autograd/ops.cpp:726-730, 1396-1409)
	const bool add_old_at_end = p.accumulate && K <= kAccAfter;
	unsigned char* alive = p.ep.alive ? p.ep.alive + oc : nullptr;
#pragma unroll
	for (int e = 0; e < 4; ++e) {
		const int row = m0 + 4 * j + e;
		if (row >= p.m || col >= p.n) continue;
		const int64_t off = (int64_t)row * p.ldc + col;
		float v = acc[e];
		if (add_old_at_end) v = K > 0 ? Cp[off] + v : Cp[off];
		if (p.ep.bias_mode == kBiasCol) v = v + p.ep.bias[col];
		else if (p.ep.bias_mode == kBiasRow) v = v + p.ep.bias[row];
		if (p.ep.res) v = p.ep.res[oc + off] + v;
		if (p.ep.gelu_y) {
			float t;
			p.ep.gelu_y[oc + off] = gelu_math::gelu_one(v, t);
			p.ep.gelu_t[oc + off] = t;
		}
		if (p.ep.relu) {
			const bool on = v > 0.0f;
			if (alive) alive[off] = on ? 1 : 0;
			v = on ? v : 0.0f;
		}
		Cp[off] = v;
	}
}

}  // namespace nnh
