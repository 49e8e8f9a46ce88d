// gemm_chain.hip - whole-depth products on the 16x16x4 MFMA with operands loaded straight into registers
// (gemm_direct.hpp): no LDS staging and no barrier in the depth loop.
//
// Every output is one chain over the whole depth in order, four depth steps per instruction (Mfma<kMf16x4>), the
// same bits as the tile kernels. A workgroup owns a 32 x 32 tile of C, a wave a 16 x 16 quarter of it; the two
// waves of a tile row read the same rows of op(A), which the CU's cache serves once. A wave streams the depth in
// chunks of 128 indices (all 16 or 64 loads of a chunk in flight), the next chunk's loads issued before the current
// chunk's MFMAs, so a chain waits on memory once instead of once per LDS stage; a k-contiguous operand is reordered
// for the MFMA through the wave's own LDS slots (gemm_direct.hpp), with no barrier. Accumulate follows the reference's
// order (kAccAfter): old C joins the chain after the first 256 steps, or is added at the end of a shorter one.
#include <algorithm>
#include <type_traits>

#include "gemm.hpp"
#include "gemm_direct.hpp"
#include "gemm_tile.hpp"

namespace nnh {

namespace {

constexpr int kChunkGroups = 8;  // 128 depth indices

template <bool TA, bool TB, bool VEC>
__global__ void __launch_bounds__(256) sgemm_chain4_kernel(const GemmArgs p) {
	constexpr bool KA = VEC && !TA, KB = VEC && TB;
	const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
	const int tiles = p.tiles_m * p.tiles_n;
	const int lid = xcd_remap((int)blockIdx.x, tiles * p.batch_count);
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
		if (p.ep.relu) {
			const bool on = v > 0.0f;
			if (alive) alive[off] = on ? 1 : 0;
			v = on ? v : 0.0f;
		}
		Cp[off] = v;
	}
}

using ChainFn = void (*)(const GemmArgs);

constexpr int64_t kMaxLd = int64_t(1) << 24;

bool chain4_vec(const GemmCall& g) {
	bool vec = true;
	if (!g.ta) {
		vec = vec && g.lda % 4 == 0 && reinterpret_cast<uintptr_t>(g.a) % 16 == 0;
		for (int d = 0; d < g.batch.ndim; ++d) vec = vec && g.batch.sa[d] % 4 == 0;
	}
	if (g.tb) {
		vec = vec && g.ldb % 4 == 0 && reinterpret_cast<uintptr_t>(g.b) % 16 == 0;
		for (int d = 0; d < g.batch.ndim; ++d) vec = vec && g.batch.sb[d] % 4 == 0;
	}
	return vec;
}

}  // namespace

bool chain4_ok(const GemmCall& g) {
	return !g.gather && !g.rowsum && g.k > 0 && !depth_cut(g.m, g.n, g.k) && g.m < kMaxLd && g.n < kMaxLd &&
	       g.k < kMaxLd && g.lda < kMaxLd && g.ldb < kMaxLd && g.batch_count < (int64_t(1) << 31);
}

bool chain4_takes(const GemmCall& g) {
	// Measured against the route before (device time on one MI355X; the tile, VALU and pieces kernels): short
	// depths, where every load of the chain is in flight at once, 256 x 256 x 10 NN 3.2 against 4.9 us, 128 x 784 x 32
	// TN 3.1 against 4.2, 1024 x 64 x 32 NT 3.3 against 3.4, 32 x 10 x 128 NT 3.8 against 5.2, 32 x 784 x 128 NN 4.1
	// against 5.2; 512 x 784 x 256 TN 7.6 against 8.3. Slower: 1024 x 64 x 64 NT 3.7 against 3.4, 1024 x 64 x 256 NT
	// 7.4 against 4.4, 256 x 10 x 256 NT 6.0 against 4.3 (a chain of whole 128-deep chunks waits on memory once a
	// chunk), and every large output (2048 x 2048 x 32 14.8 against 9.6).
	if (!chain4_ok(g) || g.m * g.n * g.batch_count > (int64_t(1) << 20)) return false;
	const int64_t mn = g.m * g.n * g.batch_count;
	if (g.k <= 32) return mn <= (int64_t(1) << 18);
	if (g.k <= 128) return std::min(g.m, g.n) <= 64 && (!g.tb || g.ta || g.m <= 64);
	return g.ta && !g.tb && g.k <= 256 && mn >= (int64_t(1) << 18);
}

hipError_t gemm_chain4_launch(const GemmCall& g, hipStream_t s) {
	static const ChainFn fns[2][4] = {
	    {sgemm_chain4_kernel<false, false, false>, sgemm_chain4_kernel<false, true, false>,
	     sgemm_chain4_kernel<true, false, false>, sgemm_chain4_kernel<true, true, false>},
	    {sgemm_chain4_kernel<false, false, true>, sgemm_chain4_kernel<false, true, true>,
	     sgemm_chain4_kernel<true, false, true>, sgemm_chain4_kernel<true, true, true>}};
	if (!chain4_ok(g)) return hipErrorInvalidValue;
	GemmArgs p{};
	p.a = g.a;
	p.b = g.b;
	p.c = g.c;
	p.lda = g.lda;
	p.ldb = g.ldb;
	p.ldc = g.ldc;
	p.m = (int)g.m;
	p.n = (int)g.n;
	p.k = (int)g.k;
	p.accumulate = g.accumulate;
	p.tiles_m = (int)((g.m + 31) / 32);
	p.tiles_n = (int)((g.n + 31) / 32);
	p.batch_count = (int)g.batch_count;
	p.batch = g.batch;
	p.ep = g.ep;
	p.pieces = 1;
	p.piece_k = (int)g.k;
	const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n * p.batch_count;
	if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
	const int f = (g.ta ? 2 : 0) + (g.tb ? 1 : 0);
	hipLaunchKernelGGL(fns[chain4_vec(g) ? 1 : 0][f], dim3((unsigned)blocks), dim3(256), 0, s, p);
	return hipGetLastError();
}

}  // namespace nnh
