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

template <bool TA, bool TB, bool VEC>
__global__ void __launch_bounds__(256) sgemm_chain4_kernel(const GemmArgs p) {
	chain4_tile<TA, TB, VEC>(p, (int)blockIdx.x, __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6),
	                         (int)threadIdx.x & 63);
}

// Two whole-depth products in one launch (a matmul's two operand gradients): workgroups below blocks0 take the first
// product's tiles, the others the second's, each with the chains of its own launch.
template <bool TA0, bool TB0, bool VEC0, bool TA1, bool TB1, bool VEC1>
__global__ void __launch_bounds__(256) sgemm_chain4_pair_kernel(const GemmArgs p0, const GemmArgs p1, int blocks0) {
	const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), lane = (int)threadIdx.x & 63;
	if ((int)blockIdx.x < blocks0) chain4_tile<TA0, TB0, VEC0>(p0, (int)blockIdx.x, wave, lane);
	else chain4_tile<TA1, TB1, VEC1>(p1, (int)blockIdx.x - blocks0, wave, lane);
}

// Up to kChainGroupMax whole-depth products of one layout in one launch (several linear layers over one input):
// product i takes the workgroups from start[i] on. The switch keeps each product's arguments a compile-time slot
// of the kernel's argument block.
struct ChainGroup {
	GemmArgs p[kChainGroupMax];
	int start[kChainGroupMax + 1];
	int count;
};

template <bool TA, bool TB, bool VEC>
__global__ void __launch_bounds__(256) sgemm_chain4_group_kernel(const ChainGroup g) {
	const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), lane = (int)threadIdx.x & 63;
	const int b = (int)blockIdx.x;
	if (b < g.start[1]) chain4_tile<TA, TB, VEC>(g.p[0], b, wave, lane);
	else if (g.count < 3 || b < g.start[2]) chain4_tile<TA, TB, VEC>(g.p[1], b - g.start[1], wave, lane);
	else chain4_tile<TA, TB, VEC>(g.p[2], b - g.start[2], wave, lane);
}

using ChainFn = void (*)(const GemmArgs);

constexpr int64_t kMaxLd = int64_t(1) << 24;

}  // namespace

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
	const GemmArgs p = chain4_args(g);
	const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n * p.batch_count;
	if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
	const int f = (g.ta ? 2 : 0) + (g.tb ? 1 : 0);
	hipLaunchKernelGGL(fns[chain4_vec(g) ? 1 : 0][f], dim3((unsigned)blocks), dim3(256), 0, s, p);
	return hipGetLastError();
}

GemmArgs chain4_args(const GemmCall& g) {
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
	return p;
}

bool chain4_pair_takes(const GemmCall& g0, const GemmCall& g1) {
	// the layouts of a matmul's gradients: dA = G B (NN) or G B^T (NT) beside dB = A^T G or G^T A (TN)
	if (g0.ta || !g1.ta || g1.tb || !chain4_takes(g0) || !chain4_takes(g1)) return false;
	const int64_t b0 = ((g0.m + 31) / 32) * ((g0.n + 31) / 32) * g0.batch_count;
	const int64_t b1 = ((g1.m + 31) / 32) * ((g1.n + 31) / 32) * g1.batch_count;
	return b0 > 0 && b1 > 0 && b0 + b1 <= 0x7fffffff;
}

hipError_t gemm_chain4_pair_launch(const GemmCall& g0, const GemmCall& g1, hipStream_t s) {
	using PairFn = void (*)(const GemmArgs, const GemmArgs, int);
	// [g0 transposes B][g0 16-byte loads]; g1 (A^T B) reads no k-contiguous operand, so its loads are the same either way
	static const PairFn fns[2][2] = {
	    {sgemm_chain4_pair_kernel<false, false, false, true, false, true>,
	     sgemm_chain4_pair_kernel<false, false, true, true, false, true>},
	    {sgemm_chain4_pair_kernel<false, true, false, true, false, true>,
	     sgemm_chain4_pair_kernel<false, true, true, true, false, true>}};
	if (!chain4_pair_takes(g0, g1)) return hipErrorInvalidValue;
	const GemmArgs p0 = chain4_args(g0), p1 = chain4_args(g1);
	const int b0 = p0.tiles_m * p0.tiles_n * p0.batch_count, b1 = p1.tiles_m * p1.tiles_n * p1.batch_count;
	hipLaunchKernelGGL(fns[g0.tb ? 1 : 0][chain4_vec(g0) ? 1 : 0], dim3((unsigned)(b0 + b1)), dim3(256), 0, s, p0, p1,
	                   b0);
	return hipGetLastError();
}

bool chain4_group_takes(const GemmCall* g, int count) {
	if (count < 2 || count > kChainGroupMax) return false;
	int64_t blocks = 0;
	for (int i = 0; i < count; ++i) {
		if (!chain4_ok(g[i]) || g[i].ta != g[0].ta || g[i].tb != g[0].tb || g[i].m <= 0 || g[i].n <= 0 ||
		    g[i].m * g[i].n * g[i].batch_count > (int64_t(1) << 20) || g[i].k > 256)
			return false;
		blocks += ((g[i].m + 31) / 32) * ((g[i].n + 31) / 32) * g[i].batch_count;
	}
	return blocks <= 0x7fffffff;
}

hipError_t gemm_chain4_group_launch(const GemmCall* g, int count, hipStream_t s) {
	using GroupFn = void (*)(const ChainGroup);
	static const GroupFn fns[2][4] = {
	    {sgemm_chain4_group_kernel<false, false, false>, sgemm_chain4_group_kernel<false, true, false>,
	     sgemm_chain4_group_kernel<true, false, false>, sgemm_chain4_group_kernel<true, true, false>},
	    {sgemm_chain4_group_kernel<false, false, true>, sgemm_chain4_group_kernel<false, true, true>,
	     sgemm_chain4_group_kernel<true, false, true>, sgemm_chain4_group_kernel<true, true, true>}};
	if (!chain4_group_takes(g, count)) return hipErrorInvalidValue;
	ChainGroup grp{};
	grp.count = count;
	bool vec = true;
	int start = 0;
	for (int i = 0; i < count; ++i) {
		grp.p[i] = chain4_args(g[i]);
		grp.start[i] = start;
		start += grp.p[i].tiles_m * grp.p[i].tiles_n * grp.p[i].batch_count;
		vec = vec && chain4_vec(g[i]);
	}
	for (int i = count; i <= kChainGroupMax; ++i) grp.start[i] = start;
	const int f = (g[0].ta ? 2 : 0) + (g[0].tb ? 1 : 0);
	hipLaunchKernelGGL(fns[vec ? 1 : 0][f], dim3((unsigned)start), dim3(256), 0, s, grp);
	return hipGetLastError();
}

}  // namespace nnh
