// gemm_config.hpp - one compiled tile configuration of the MFMA GEMM: its 8 kernels (4 operand layouts x
// interior/edge) and their LDS sizes. Each configuration is instantiated in its own gemm_cfg_*.hip.
#pragma once

#include "gemm_tile.hpp"

namespace nnh {

using KernelFn = void (*)(const GemmArgs);
using PairFn = void (*)(const GemmArgs, const GemmArgs, int);

struct Config {
	const char* name;
	int bm, bn, bk;
	int lds_bytes[4];   // per operand layout (ta * 2 + tb)
	KernelFn fn[4][2];  // [ta * 2 + tb][edge]
	KernelFn gather_fn[2];  // B gathered as im2col columns (ColGather), A not transposed: [tb]
	KernelFn rowsum_fn[2];  // transposed A, plain B, with row sums of op(A) (GemmArgs::rowsum): [edge]
	// A B and A^T B (with row sums or not) in one launch, compiled for the small-tile configurations only (null
	// otherwise): [edge of the first][edge of the second][row sums]
	PairFn pair_fn[2][2][2];
};

template <int BM, int BN, int BK, int WM, int WN, int WPE, int MF = kMf32, bool PAIR = false>
Config make_config(const char* name) {
	Config c{};
	c.name = name;
	c.bm = BM;
	c.bn = BN;
	c.bk = BK;
#define NNH_SET(TA, TB)                                                                                  \
	c.lds_bytes[TA * 2 + TB] = TileShape<BM, BN, BK, WM, WN, MF, TA, TB>::kLdsFloats * (int)sizeof(float); \
	c.fn[TA * 2 + TB][0] = sgemm_tile_kernel<BM, BN, BK, WM, WN, WPE, MF, TA, TB, false>;                     \
	c.fn[TA * 2 + TB][1] = sgemm_tile_kernel<BM, BN, BK, WM, WN, WPE, MF, TA, TB, true>;
	NNH_SET(false, false)
	NNH_SET(false, true)
	NNH_SET(true, false)
	NNH_SET(true, true)
#undef NNH_SET
	c.gather_fn[0] = sgemm_tile_kernel<BM, BN, BK, WM, WN, WPE, MF, false, false, true, true>;
	c.gather_fn[1] = sgemm_tile_kernel<BM, BN, BK, WM, WN, WPE, MF, false, true, true, true>;
	c.rowsum_fn[0] = sgemm_tile_kernel<BM, BN, BK, WM, WN, WPE, MF, true, false, false, false, true>;
	c.rowsum_fn[1] = sgemm_tile_kernel<BM, BN, BK, WM, WN, WPE, MF, true, false, true, false, true>;
	if constexpr (PAIR) {
#define NNH_PAIR(E0, E1, R) c.pair_fn[E0][E1][R] = sgemm_pair_kernel<BM, BN, BK, WM, WN, WPE, MF, E0, E1, R>;
		NNH_PAIR(false, false, false)
		NNH_PAIR(false, false, true)
		NNH_PAIR(false, true, false)
		NNH_PAIR(false, true, true)
		NNH_PAIR(true, false, false)
		NNH_PAIR(true, false, true)
		NNH_PAIR(true, true, false)
		NNH_PAIR(true, true, true)
#undef NNH_PAIR
	}
	return c;
}

Config config_64x128x32();
Config config_128x128x32();
Config config_64x256x32();
Config config_128x64x32();
Config config_128x256x16();
Config config_256x128x16();
Config config_64x128x64();
Config config_128x128x16();
// short-latency MFMAs (4x4x1, 16x16x1) for products too small or too skinny to fill the GPU with 32x32 units
Config config_32x32x32_mf4();
Config config_64x64x32_mf4();
Config config_64x64x32_mf16();
Config config_128x64x32_mf16();
// 16x16x4 MFMAs: four depth indices of every chain per instruction (the same fma chain)
Config config_32x32x32_mfk4();
Config config_64x64x32_mfk4();
Config config_128x64x32_mfk4();
Config config_128x128x32_mfk4();
Config config_32x32x64_mfk4();
Config config_32x32x128_mfk4();

}  // namespace nnh
