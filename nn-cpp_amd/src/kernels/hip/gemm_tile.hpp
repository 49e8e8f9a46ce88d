// gemm_tile.hpp - the fp32 MFMA tile GEMM for gfx950 (CDNA4), shared by every GEMM-shaped op.
//
// Numerical contract (what makes the results identical to nn-cpp's NN_NATIVE sgemm):
//   nn::kernels::sgemm's AVX2 microkernel computes each C element as a sequential fused
//   multiply-add chain over the depth, starting at +0 (src/kernels/gemm.cpp:232-244); depth
//   blocks of 256 store and reload the running sum unchanged (gemm.cpp:225-231, 371).
//   On gfx950 the k = 1 fp32 MFMAs compute exactly fma(a, b, c) per output element (single
//   rounding, denormals kept; see below). This kernel issues one MFMA per depth index k, in
//   increasing k, starting from +0,
//   so every element is the same fma chain. The k order never depends on the tile shape,
//   the grid, ld, alignment, batch or stream: results are a pure function of the inputs.
//   With accumulate, the old C is added after the first min(K, 256) steps (Store::kAdd then
//   Store::kContinue, gemm.cpp:245-252), exactly as the reference does.
//
// The three k = 1 fp32 MFMAs of gfx950 all compute exactly fma(a, b, c) per element (measured against fmaf on
// 1-8 million outputs each, special values included); they differ in latency per chain step, which bounds
// products whose grid cannot fill the GPU (each element is a K-long dependent chain):
//   32x32x1_2b: 2048 fmas, 16 passes; 16x16x1_4b: 1024 fmas, 8 passes; 4x4x1_16b: 256 fmas, 2 passes.
// Large products use 32x32x1 (the most reuse per LDS read); small and skinny ones use the shorter ones.
//
// Tiling: 256 threads = 4 waves. A workgroup owns a BM x BN tile of C; wave w owns a WM x WN
// sub-tile made of MFMA units (Mfma<MF>::UM x UN each):
//   32x32x1_2b: unit 64 x 32 (two 32x32 blocks: A lanes 0-31 and 32-63 carry 64 distinct rows,
//               B lanes 32-63 repeat lanes 0-31's 32 columns);
//   16x16x1_4b: unit 64 x 16 (four 16x16 blocks stacked along M, sharing their 16 columns);
//   4x4x1_16b:  unit 16 x 16 (sixteen 4x4 blocks as a 4 x 4 grid).
// Operands go global -> registers -> LDS (double buffered, one barrier per depth tile).
// LDS layouts follow the global layout so that every global load and LDS store is 16 bytes:
//   K-contiguous operands (A when !TA, B when TB) are stored [row][BK+4] and read as one
//   ds_read_b128 giving 4 consecutive k; M/N-contiguous operands are stored [BK][rows] and read
//   as 4 ds_read_b32 (one per k).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fastdiv.hpp"

namespace nnh {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x32 __attribute__((ext_vector_type(32)));

enum MfmaKind : int { kMf32 = 0, kMf16 = 1, kMf4 = 2, kMf16x4 = 3 };

// Per MFMA kind: the unit tile, which row of A (column of B) lane l supplies, and where accumulator
// register r of lane l sits in the unit (lane layouts measured on gfx950).
template <int MF>
struct Mfma;

template <>
struct Mfma<kMf32> {
	static constexpr int UM = 64, UN = 32, NV = 32, DEPTH = 1;
	using Acc = f32x32;
	__device__ static int arow(int l) { return l; }
	__device__ static int bcol(int l) { return l & 31; }
	__host__ __device__ static constexpr int crow(int r, int l) { return 32 * (r >> 4) + 8 * ((r & 15) >> 2) + 4 * (l >> 5) + (r & 3); }
	__device__ static int ccol(int l) { return l & 31; }
	__device__ static Acc mma(float a, float b, const Acc& c) { return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c, 0, 0, 0); }
};

template <>
struct Mfma<kMf16> {
	static constexpr int UM = 64, UN = 16, NV = 16, DEPTH = 1;
	using Acc = f32x16;
	__device__ static int arow(int l) { return l; }
	__device__ static int bcol(int l) { return l & 15; }
	__host__ __device__ static constexpr int crow(int r, int l) { return 16 * (r >> 2) + 4 * (l >> 4) + (r & 3); }
	__device__ static int ccol(int l) { return l & 15; }
	__device__ static Acc mma(float a, float b, const Acc& c) { return __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, c, 0, 0, 0); }
};

template <>
struct Mfma<kMf4> {
	static constexpr int UM = 16, UN = 16, NV = 4, DEPTH = 1;
	using Acc = f32x4;
	__device__ static int arow(int l) { return 4 * (l >> 4) + (l & 3); }
	__device__ static int bcol(int l) { return 4 * ((l >> 2) & 3) + (l & 3); }
	__host__ __device__ static constexpr int crow(int r, int l) { return 4 * (l >> 4) + r; }
	__device__ static int ccol(int l) { return 4 * ((l >> 2) & 3) + (l & 3); }
	__device__ static Acc mma(float a, float b, const Acc& c) { return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0); }
};

// 16x16x4: one 16 x 16 block over four depth indices per instruction. Lane l supplies A[l % 16][k0 + l / 16] and
// B[k0 + l / 16][l % 16], and each output becomes fma(a3, b3, fma(a2, b2, fma(a1, b1, fma(a0, b0, c)))), the depth
// indices in increasing order: measured on gfx950 bit-identical to four fmaf in sequence (on the same GPU's vector
// ALUs) on 5 million outputs, zeros of both signs, infinities, NaN payloads and subnormals included. So one
// instruction advances every chain of its block four steps of the reference's chain, in 44 cycles where the k = 1
// MFMAs take 44 for one.
template <>
struct Mfma<kMf16x4> {
	static constexpr int UM = 16, UN = 16, NV = 4, DEPTH = 4;
	using Acc = f32x4;
	__device__ static int arow(int l) { return l & 15; }
	__device__ static int bcol(int l) { return l & 15; }
	__host__ __device__ static constexpr int crow(int r, int l) { return 4 * (l >> 4) + r; }
	__device__ static int ccol(int l) { return l & 15; }
	__device__ static Acc mma(float a, float b, const Acc& c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }
};

constexpr int kMaxBatchDims = 4;
constexpr int kAccAfter = 256;  // nn-cpp's kKC (gemm.hpp:33): where an accumulating product adds old C

// Batch addressing: up to 4 batch dims, element strides per dim for A, B, C (0 = broadcast).
struct BatchDesc {
	int ndim;
	int64_t shape[kMaxBatchDims];
	int64_t sa[kMaxBatchDims], sb[kMaxBatchDims], sc[kMaxBatchDims];
};

enum BiasMode : int { kBiasNone = 0, kBiasCol = 1, kBiasRow = 2 };

// Applied to each finished element v (after any accumulate): v = v + bias; then, with relu,
// alive = v > 0, v = alive ? v : 0 (src/autograd/ops.cpp:726-730, 1396-1409).
struct Epilogue {
	int bias_mode;
	int relu;
	const float* bias;
	unsigned char* alive;  // optional, addressed like C
	// optional, addressed like C: added after the bias as res + v, the reference's add(residual, linear(...))
	const float* res;
	// optional, addressed like C, the chain kernel only (gemm_direct.hpp): GELU of the stored value (ops.cpp:461-466)
	// into gelu_y and its tanh into gelu_t, the reference's gelu(linear(...)) with C its input
	float* gelu_y;
	float* gelu_t;
};

// Implicit im2col (src/autograd/ops.cpp:188-212): B is a sample's column matrix col[k][p] of a convolution,
// read straight from its input x instead of a materialised buffer. Row k = (c, ph, pw) = (c * kh + ph) * kw + pw,
// column p = (oh, ow) = oh * wo + ow; the entry is x[c][oh * stride + ph - pad][ow * stride + pw - pad], or 0 in
// the padding. The batch's B stride steps from one sample's x to the next.
struct ColGather {
	int cin, h, w, kh, kw, stride, pad, ho, wo;
	FastDiv khkw, kw_div, wo_div;
};

struct GemmArgs {
	const float* a;
	const float* b;
	float* c;
	int64_t lda, ldb, ldc;
	int m, n, k;
	int accumulate;
	int tiles_m, tiles_n;
	int batch_count;
	int pieces;        // > 1: depth cut, each piece writes partial[(batch*pieces + piece)][m][n]
	int piece_k;       // depth of one piece
	int vec_ok;        // lda, ldb, strides multiples of 4 and a, b 16-byte aligned
	float* partial;
	BatchDesc batch;
	Epilogue ep;
	ColGather col;     // used by the GB (gather) kernels only
	// optional: rowsum[i] = the sum of row i of op(A) over k, in k order from +0 (Tensor::sum(0) of A's
	// transpose, tensor.cpp:422-456), computed by the first column tile; transposed A, single matrix, no depth cut.
	// combine: 0 store s, 1 store s + 0.0f, 2 rowsum[i] += s
	float* rowsum;
	int rowsum_combine;
	// > 0 (the 16x16x4 pieces kernel only): rowsum[i] is two ordered sums instead, as Tensor::sum(0) applied twice
	// to op(A)'s row i viewed as [rowsum_outer][k / rowsum_outer]: first over the outer index for each inner one,
	// each from +0, then over the inner index from +0; combined as above
	int rowsum_outer;
};

__device__ __forceinline__ void batch_offsets(const BatchDesc& d, int64_t bi, int64_t& oa, int64_t& ob,
                                              int64_t& oc) {
	oa = ob = oc = 0;
	for (int i = d.ndim - 1; i >= 0; --i) {
		const int64_t idx = bi % d.shape[i];
		bi /= d.shape[i];
		oa += idx * d.sa[i];
		ob += idx * d.sb[i];
		oc += idx * d.sc[i];
	}
}

// Loads an R x CC row-major tile (CC % 4 == 0) starting at g: 16-byte loads, `fill` outside
// rows_valid x cols_valid when EDGE. The B operand is filled with -0: a depth step past k then multiplies
// +0 (A's fill) by -0, and adding that -0 product leaves every sum as it was, -0 included (adding +0 would turn a
// chain that ended at -0 into +0).
template <int R, int CC, bool EDGE>
__device__ __forceinline__ void load_tile(const float* __restrict__ g, int64_t ld, int rows_valid,
                                          int cols_valid, bool vec_ok, f32x4* out, int tid, float fill = 0.0f) {
	constexpr int kVecPerRow = CC / 4;
	constexpr int kPer = R * CC / 4 / 256;
	static_assert(kPer * 256 * 4 == R * CC, "tile must split evenly over 256 threads");
#pragma unroll
	for (int i = 0; i < kPer; ++i) {
		const int idx = tid + 256 * i;
		const int r = idx / kVecPerRow;
		const int c = (idx % kVecPerRow) * 4;
		if (!EDGE) {
			out[i] = *reinterpret_cast<const f32x4*>(g + r * ld + c);
		} else {
			const bool row_in = r < rows_valid;
			if (row_in && c + 3 < cols_valid && vec_ok) {
				out[i] = *reinterpret_cast<const f32x4*>(g + r * ld + c);
			} else {
				f32x4 v;
#pragma unroll
				for (int e = 0; e < 4; ++e) v[e] = (row_in && c + e < cols_valid) ? g[r * ld + c + e] : fill;
				out[i] = v;
			}
		}
	}
}

// KPERM (a k-contiguous tile for the 16x16x4 MFMA): inside every 16 columns, column 4 t + e is stored at 4 e + t,
// so that lane group e's operands of four consecutive MFMAs (depth 4 t + e, t = 0..3) are one 16-byte read.
template <int R, int CC, int S, bool KPERM = false>
__device__ __forceinline__ void store_tile(float* lds, const f32x4* v, int tid) {
	constexpr int kVecPerRow = CC / 4;
	constexpr int kPer = R * CC / 4 / 256;
	static_assert(!KPERM || CC % 16 == 0, "the permutation works on 16 columns at a time");
#pragma unroll
	for (int i = 0; i < kPer; ++i) {
		const int idx = tid + 256 * i;
		const int r = idx / kVecPerRow;
		const int c = (idx % kVecPerRow) * 4;
		if constexpr (KPERM) {
			const int base = r * S + (c & ~15) + ((c >> 2) & 3);
#pragma unroll
			for (int e = 0; e < 4; ++e) lds[base + 4 * e] = v[i][e];
		} else {
			*reinterpret_cast<f32x4*>(lds + r * S + c) = v[i];
		}
	}
}

// Loads of a sample's column matrix (rows kk, columns p; zeros outside the matrix or in the convolution's
// padding) from its input x, in the register layout of load_tile for an R x CC tile: thread tid's slot i covers
// row (tid + 256 i) / (CC / 4) and the four columns from 4 ((tid + 256 i) % (CC / 4)). Because 256 is a
// multiple of CC / 4, a thread's columns are the same in every slot and every tile. ColCols holds their
// (oh, ow) geometry and ColRow a row's (c, ph, pw): the caller computes whichever side of the tile stays
// fixed over the depth loop once, and the other per tile.
constexpr int kColPast = -(1 << 30);  // ColCols::ihb of a column past the matrix
struct ColCols {
	int ihb[4], iwb[4];  // oh * stride - pad, ow * stride - pad; ihb = kColPast marks a column past the matrix
};
struct ColRow {
	int64_t xoff;  // c * h * w; -1 marks a row past the matrix
	int ph, pw;
};

__device__ __forceinline__ ColCols col_cols(const ColGather& cg, int p0, int cols_valid) {
	ColCols cc;
#pragma unroll
	for (int e = 0; e < 4; ++e) {
		const unsigned pp = (unsigned)(p0 + e);
		const unsigned oh = fdiv(pp, cg.wo_div);
		const int ow = (int)(pp - oh * cg.wo_div.d);
		const bool ok = e < cols_valid;
		cc.ihb[e] = ok ? (int)oh * cg.stride - cg.pad : kColPast;
		cc.iwb[e] = ow * cg.stride - cg.pad;
	}
	return cc;
}

__device__ __forceinline__ ColRow col_row(const ColGather& cg, int kk, bool valid) {
	const unsigned ci = fdiv((unsigned)kk, cg.khkw);
	const unsigned rem = (unsigned)kk - ci * cg.khkw.d;
	const unsigned ph = fdiv(rem, cg.kw_div);
	return ColRow{valid ? (int64_t)ci * cg.h * cg.w : (int64_t)-1, (int)ph, (int)(rem - ph * cg.kw_div.d)};
}

// Every load is issued, at an index clamped into the channel image (so the code has no branches and the loads
// of a tile are in flight together); the convolution's padding is then replaced by 0 (a real tap of the
// reference's chain, fma(w, 0, acc)) and entries past the matrix by -0 (B's fill, see load_tile).
__device__ __forceinline__ f32x4 col_values(const float* __restrict__ x, const ColGather& cg, const ColRow& r,
                                            const ColCols& cc) {
	f32x4 v;
	const float* xc = x + (r.xoff >= 0 ? r.xoff : 0);
#pragma unroll
	for (int e = 0; e < 4; ++e) {
		const int ih = cc.ihb[e] + r.ph, iw = cc.iwb[e] + r.pw;
		const bool past = r.xoff < 0 || cc.ihb[e] == kColPast;
		const bool in = !past && ih >= 0 && ih < cg.h && iw >= 0 && iw < cg.w;
		const float t = xc[min(max(ih, 0), cg.h - 1) * cg.w + min(max(iw, 0), cg.w - 1)];
		v[e] = in ? t : (past ? -0.0f : 0.0f);
	}
	return v;
}

// Whether every accumulator register r of an MFMA unit stays, for all 64 lanes, inside the pass of RP rows that
// lane 0 puts it in (the interior epilogue stages one pass at a time).
template <int MF>
__host__ __device__ constexpr bool passes_split_evenly(int rp) {
	for (int r = 0; r < Mfma<MF>::NV; ++r)
		for (int l = 0; l < 64; ++l)
			if (Mfma<MF>::crow(r, l) / rp != Mfma<MF>::crow(r, 0) / rp) return false;
	return Mfma<MF>::UM % rp == 0;
}

template <int BM, int BN, int BK, int WM, int WN, int MF, bool TA, bool TB>
struct TileShape {
	static constexpr int kWavesN = BN / WN;
	static_assert((BM / WM) * (BN / WN) == 4, "4 waves per workgroup");
	static_assert(WM % Mfma<MF>::UM == 0 && WN % Mfma<MF>::UN == 0, "wave tile must be whole MFMA units");
	static constexpr int D = Mfma<MF>::DEPTH;
	static_assert(kAccAfter % BK == 0 && BK % (4 * D) == 0, "depth tile must divide 256 and hold whole fragment groups");
	static constexpr int I = WM / Mfma<MF>::UM, J = WN / Mfma<MF>::UN;
	// LDS strides (floats). K-major tiles get 4 floats of padding so that 64 lanes reading 16 bytes
	// from 64 consecutive rows spread over the banks. With the 16x16x4 MFMA an M/N-major tile's rows get 16 floats
	// more, so that the four lane groups (four depth rows, 16 consecutive columns each) read distinct banks.
	static constexpr int kPadMN = D == 4 ? 16 : 0;
	static constexpr int SA = TA ? BM + kPadMN : BK + 4;
	static constexpr int SB = TB ? BK + 4 : BN + kPadMN;
	static constexpr int kASize = TA ? BK * SA : BM * SA;
	static constexpr int kBSize = TB ? BN * SB : BK * SB;
	static constexpr int kStage = kASize + kBSize;
	static constexpr int kLdsFloats = 2 * kStage;
	static constexpr int LA = BM * BK / 4 / 256;
	static constexpr int LB = BN * BK / 4 / 256;
	// Depth tiles whose global loads are in flight ahead of the one in LDS (a ring of register sets). Small tiles
	// do little MFMA work per depth tile, less than a load's latency, so they keep up to 4 tiles in flight; the
	// large tiles keep one (their registers are spent on accumulators).
	static constexpr int kPF = BM * BN <= 32 * 32 ? (LA + LB <= 2 ? 4 : (LA + LB <= 4 ? 2 : 1))
	                                              : (MF == kMf16x4 && BM * BN <= 64 * 64 ? 2 : 1);
	static_assert((kAccAfter / BK) % kPF == 0, "the accumulate split must fall on a ring boundary");
};

// Maps the hardware workgroup id to a logical tile id so that consecutive logical ids (which share
// A rows and B columns) run on the same XCD and therefore share its L2. Workgroups are dispatched to
// the 8 XCDs round-robin by id.
__device__ __forceinline__ int xcd_remap(int bid, int total) {
	const int per = total / 8;
	if (bid < per * 8) return (bid % 8) * per + bid / 8;
	return bid;
}

// One workgroup's tile of a product; block is the workgroup's index among the product's workgroups.
template <int BM, int BN, int BK, int WM, int WN, int MF, bool TA, bool TB, bool EDGE, bool GB = false, bool RS = false>
__device__ __forceinline__ void sgemm_tile_body(const GemmArgs& p, int block) {
	static_assert(!GB || (!TA && EDGE), "the implicit im2col operand is B, loaded with bounds checks");
	static_assert(!RS || (TA && !TB && !GB), "row sums are compiled for the weight-gradient layout only");
	static_assert(!RS || (BM & (BM - 1)) == 0, "row sums index rows as tid % BM");
	using S = TileShape<BM, BN, BK, WM, WN, MF, TA, TB>;
	using U = Mfma<MF>;
	constexpr int I = S::I, J = S::J;
	extern __shared__ __align__(16) float lds[];

	const int tid = threadIdx.x;
	const int lane = tid & 63;
	const int wave = tid >> 6;
	const int wm0 = (wave / S::kWavesN) * WM;
	const int wn0 = (wave % S::kWavesN) * WN;

	// ---- which tile, piece and batch matrix ----
	const int tiles = p.tiles_m * p.tiles_n;
	const int total = tiles * p.pieces * p.batch_count;
	const int lid = xcd_remap(block, total);
	const int t = lid % tiles;
	const int rest = lid / tiles;
	const int piece = rest % p.pieces;
	const int bi = rest / p.pieces;
	// grouped order: 8 tile-rows at a time, column-major inside the group
	constexpr int G = 8;
	const int group = t / (G * p.tiles_n);
	const int first_m = group * G;
	const int gsize = min(G, p.tiles_m - first_m);
	const int in_group = t % (G * p.tiles_n);
	const int tm = first_m + in_group % gsize;
	const int tn = in_group / gsize;
	const int m0 = tm * BM, n0 = tn * BN;

	int64_t oa = 0, ob = 0, oc = 0;
	if (p.batch.ndim > 0) batch_offsets(p.batch, bi, oa, ob, oc);
	const float* __restrict__ A = p.a + oa;
	const float* __restrict__ B = p.b + ob;

	const int k_lo = piece * p.piece_k;
	const int k_hi = min(p.k, k_lo + p.piece_k);
	const int kr = k_hi - k_lo;
	const int nkt = (kr + BK - 1) / BK;
	// accumulate: old C joins the chain after the first min(K, 256) steps (whole product only)
	const bool acc_mode = p.accumulate && p.pieces == 1;
	const int acc_tile = (p.k > kAccAfter) ? kAccAfter / BK - 1 : -1;

	typename U::Acc acc[I][J];
#pragma unroll
	for (int i = 0; i < I; ++i)
#pragma unroll
		for (int j = 0; j < J; ++j)
#pragma unroll
			for (int r = 0; r < U::NV; ++r) acc[i][j][r] = 0.0f;

	const bool vec_ok = p.vec_ok != 0;
	constexpr int PF = RS ? 1 : S::kPF;  // the row sums' registers leave no room for a ring
	f32x4 ra[PF][S::LA], rb[PF][S::LB];
	// implicit im2col: the side of each thread's B slots that is fixed over the depth loop (NN: its columns p,
	// NT: its rows kk), computed once
	constexpr int kGV = TB ? BK / 4 : BN / 4;  // 16-byte groups per row of the B tile
	ColCols gcols{};
	ColRow grows[S::LB];
	if constexpr (GB) {
		const int c = (tid % kGV) * 4;
		if constexpr (!TB) {
			gcols = col_cols(p.col, n0 + c, p.n - n0 - c);
		} else {
#pragma unroll
			for (int i = 0; i < S::LB; ++i) {
				const int r = (tid + 256 * i) / kGV;
				grows[i] = col_row(p.col, n0 + r, r < p.n - n0);
			}
		}
	}
	auto load = [&](int kt, f32x4* ra, f32x4* rb) {
		const int k0 = k_lo + kt * BK;
		if (!TA)  // A stored m x k: tile BM rows x BK
			load_tile<BM, BK, EDGE>(A + (int64_t)m0 * p.lda + k0, p.lda, p.m - m0, k_hi - k0, vec_ok, ra, tid);
		else      // A stored k x m: tile BK rows x BM
			load_tile<BK, BM, EDGE>(A + (int64_t)k0 * p.lda + m0, p.lda, k_hi - k0, p.m - m0, vec_ok, ra, tid);
		if constexpr (GB) {  // B = a sample's im2col columns, gathered from x
			const int c = (tid % kGV) * 4;
			if constexpr (TB) {  // rows kk fixed, columns p = depth
				const ColCols cc = col_cols(p.col, k0 + c, k_hi - k0 - c);
#pragma unroll
				for (int i = 0; i < S::LB; ++i) rb[i] = col_values(B, p.col, grows[i], cc);
			} else {  // rows kk = depth, columns p fixed
#pragma unroll
				for (int i = 0; i < S::LB; ++i) {
					const int r = (tid + 256 * i) / kGV;
					rb[i] = col_values(B, p.col, col_row(p.col, k0 + r, r < k_hi - k0), gcols);
				}
			}
		} else if constexpr (TB) {  // B stored n x k
			load_tile<BN, BK, EDGE>(B + (int64_t)n0 * p.ldb + k0, p.ldb, p.n - n0, k_hi - k0, vec_ok, rb, tid, -0.0f);
		} else {  // B stored k x n
			load_tile<BK, BN, EDGE>(B + (int64_t)k0 * p.ldb + n0, p.ldb, k_hi - k0, p.n - n0, vec_ok, rb, tid, -0.0f);
		}
	};
	constexpr bool kPerm = U::DEPTH == 4;  // k-contiguous tiles stored permuted for the 16x16x4 fragments
	auto store = [&](int buf, const f32x4* ra, const f32x4* rb) {
		float* As = lds + buf * S::kStage;
		float* Bs = As + S::kASize;
		if (!TA) store_tile<BM, BK, S::SA, kPerm>(As, ra, tid);
		else store_tile<BK, BM, S::SA>(As, ra, tid);
		if (TB) store_tile<BN, BK, S::SB, kPerm>(Bs, rb, tid);
		else store_tile<BK, BN, S::SB>(Bs, rb, tid);
	};

	// C element (i, j, r) of this lane: row and column inside the workgroup tile
	auto c_row = [&](int i, int r, int ln) { return wm0 + U::UM * i + U::crow(r, ln); };
	auto c_col = [&](int j, int ln) { return wn0 + U::UN * j + U::ccol(ln); };

	// One depth tile from LDS buffer buf: fragments for depth group kk+KG are read while the MFMAs of
	// group kk run (two register sets), and each element's chain advances one k per MFMA (four with 16x16x4), in
	// order. A group is 4 depth indices (k = 1 MFMAs: element e of a fragment is depth kk + e) or 16 (16x16x4:
	// element t of lane group g's fragment is depth kk + 4 t + g).
	constexpr int KG = 4 * U::DEPTH;
	auto read_frags = [&](const float* As, const float* Bs, int kk, f32x4* af, f32x4* bf) {
		if constexpr (U::DEPTH == 4) {
			const int g = lane >> 4;
#pragma unroll
			for (int i = 0; i < I; ++i) {
				const int row = wm0 + U::UM * i + U::arow(lane);
				if (!TA) {
					af[i] = *reinterpret_cast<const f32x4*>(As + row * S::SA + kk + 4 * g);
				} else {
#pragma unroll
					for (int t = 0; t < 4; ++t) af[i][t] = As[(kk + 4 * t + g) * S::SA + row];
				}
			}
#pragma unroll
			for (int j = 0; j < J; ++j) {
				const int col = wn0 + U::UN * j + U::bcol(lane);
				if (TB) {
					bf[j] = *reinterpret_cast<const f32x4*>(Bs + col * S::SB + kk + 4 * g);
				} else {
#pragma unroll
					for (int t = 0; t < 4; ++t) bf[j][t] = Bs[(kk + 4 * t + g) * S::SB + col];
				}
			}
			return;
		}
#pragma unroll
		for (int i = 0; i < I; ++i) {
			const int row = wm0 + U::UM * i + U::arow(lane);
			if (!TA) {
				af[i] = *reinterpret_cast<const f32x4*>(As + row * S::SA + kk);
			} else {
#pragma unroll
				for (int e = 0; e < 4; ++e) af[i][e] = As[(kk + e) * S::SA + row];
			}
		}
#pragma unroll
		for (int j = 0; j < J; ++j) {
			const int col = wn0 + U::UN * j + U::bcol(lane);
			if (TB) {
				bf[j] = *reinterpret_cast<const f32x4*>(Bs + col * S::SB + kk);
			} else {
#pragma unroll
				for (int e = 0; e < 4; ++e) bf[j][e] = Bs[(kk + e) * S::SB + col];
			}
		}
	};
	// Row sums of op(A) (see GemmArgs::rowsum; RS kernels, the weight-gradient layout): every thread folds row
	// tid % BM of each depth tile in k order, four values per MFMA group, read with that group's fragments, with
	// no branch; the first column tile's threads tid < BM store them. Depth past k is zero-filled by the edge
	// loader, and adding +0 leaves the sum unchanged (it starts at +0, so it is never -0).
	float rsum = 0.0f;
	auto read_rowsum = [&](const float* As, int kk, f32x4* v) {  // the group's KG depth values of the row
#pragma unroll
		for (int d = 0; d < U::DEPTH; ++d)
#pragma unroll
			for (int e = 0; e < 4; ++e) v[d][e] = As[(kk + 4 * d + e) * S::SA + (tid & (BM - 1))];
	};
	auto mma_tile = [&](int buf) {
		const float* As = lds + buf * S::kStage;
		const float* Bs = As + S::kASize;
		f32x4 af[2][I], bf[2][J];
		// row-sum values: read a group ahead with the fragments (k = 1 MFMAs: 4 per group), or, with 16x16x4 (16 per
		// group), for the current group only, so that they do not cost the registers of a second set
		constexpr int RSB = U::DEPTH == 4 ? 1 : 2;
		[[maybe_unused]] f32x4 rs[RSB][U::DEPTH];
		read_frags(As, Bs, 0, af[0], bf[0]);
		if constexpr (RS && RSB == 2) read_rowsum(As, 0, rs[0]);
#pragma unroll
		for (int kk = 0; kk < BK; kk += KG) {
			const int cur = (kk / KG) & 1;
			// issue the next group's LDS reads before this group's MFMAs, so their latency is hidden;
			// the scheduling fences stop the compiler from sinking them back next to their uses
			if (kk + KG < BK) {
				read_frags(As, Bs, kk + KG, af[cur ^ 1], bf[cur ^ 1]);
				if constexpr (RS && RSB == 2) read_rowsum(As, kk + KG, rs[cur ^ 1]);
			}
			if constexpr (RS && RSB == 1) read_rowsum(As, kk, rs[0]);
			__builtin_amdgcn_sched_barrier(0);
#pragma unroll
			for (int e = 0; e < 4; ++e)
#pragma unroll
				for (int i = 0; i < I; ++i)
#pragma unroll
					for (int j = 0; j < J; ++j)
						acc[i][j] = U::mma(af[cur][i][e], bf[cur][j][e], acc[i][j]);
			if constexpr (RS) {
#pragma unroll
				for (int d = 0; d < U::DEPTH; ++d)
#pragma unroll
					for (int e = 0; e < 4; ++e) rsum = rsum + rs[RSB == 2 ? cur : 0][d][e];
			}
			__builtin_amdgcn_sched_barrier(0);
		}
	};
	// Step kt, with u = kt % PF known at compile time: register set u held tile kt (already in LDS) and now loads
	// tile kt + PF (clamped to the last tile: a redundant load instead of a branch around it, so the compiler
	// waits for each set by count); the MFMAs run on LDS buffer kt & 1; set (u + 1) % PF, tile kt + 1, goes to the
	// other buffer.
	auto step = [&](int kt, int u) {
		if (PF > 1 || kt + 1 < nkt) load(min(kt + PF, nkt - 1), ra[u], rb[u]);
		mma_tile(kt & 1);
		if (kt + 1 < nkt) store((kt + 1) & 1, ra[(u + 1) % PF], rb[(u + 1) % PF]);
		__syncthreads();
	};
	// The same step with no branch at all (the ring's loads are then waited for by count: a branch anywhere in the
	// loop makes the compiler wait for every load at the merge): past the last tile the store writes a redundant
	// tile into the buffer no MFMA reads any more (the epilogue reuses LDS only after the loop's last barrier).
	auto step_full = [&](int kt, int u) {
		load(min(kt + PF, nkt - 1), ra[u], rb[u]);
		mma_tile(kt & 1);
		store((kt + 1) & 1, ra[(u + 1) % PF], rb[(u + 1) % PF]);
		__syncthreads();
	};
	// steps k0 .. k1 - 1 (k0 a multiple of PF): whole rounds of PF steps, then the rest
	auto run = [&](int k0, int k1) {
		int kt = k0;
		if constexpr (PF > 1) {
			for (; kt + PF <= k1; kt += PF) {
#pragma unroll
				for (int u = 0; u < PF; ++u) step_full(kt + u, u);
			}
		}
		for (; kt < k1; kt += PF) {
#pragma unroll
			for (int u = 0; u < PF; ++u)
				if (kt + u < k1) step(kt + u, u);
		}
	};

	if (nkt > 0) {
#pragma unroll
		for (int u = 0; u < PF; ++u) load(min(u, nkt - 1), ra[u], rb[u]);
		store(0, ra[0], rb[0]);
		__syncthreads();
	}
	// With accumulate, old C joins the chain after the first 256 steps; the loop is split there so the
	// accumulators never leave the matrix-core registers inside a loop.
	const bool add_mid = acc_mode && acc_tile >= 0;
	const int n1 = add_mid ? acc_tile + 1 : nkt;
	run(0, n1);
	if (add_mid) {
		int lane_m = lane;
		asm volatile("" : "+v"(lane_m));
#pragma unroll
		for (int i = 0; i < I; ++i)
#pragma unroll
			for (int j = 0; j < J; ++j)
#pragma unroll
				for (int r = 0; r < U::NV; ++r) {
					const int row = m0 + c_row(i, r, lane_m), col = n0 + c_col(j, lane_m);
					if (!EDGE || (row < p.m && col < p.n))
						acc[i][j][r] = p.c[oc + (int64_t)row * p.ldc + col] + acc[i][j][r];
				}
	}
	run(n1, nkt);
	if (RS && p.rowsum != nullptr && tn == 0 && p.pieces == 1 && tid < BM && m0 + tid < p.m) {
		float* d = p.rowsum + m0 + tid;
		*d = p.rowsum_combine == 0 ? rsum : (p.rowsum_combine == 1 ? rsum + 0.0f : *d + rsum);
	}

	// ---- epilogue ---- (the fenced lane keeps the store addresses from being computed before the loop)
	int lane_e = lane;
	asm volatile("" : "+v"(lane_e));
	if (p.pieces > 1) {
		float* part = p.partial + ((int64_t)bi * p.pieces + piece) * (int64_t)p.m * p.n;
#pragma unroll
		for (int i = 0; i < I; ++i)
#pragma unroll
			for (int j = 0; j < J; ++j)
#pragma unroll
				for (int r = 0; r < U::NV; ++r) {
					const int row = m0 + c_row(i, r, lane_e), col = n0 + c_col(j, lane_e);
					if (!EDGE || (row < p.m && col < p.n)) part[(int64_t)row * p.n + col] = acc[i][j][r];
				}
		return;
	}
	const bool add_old_at_end = acc_mode && p.k <= kAccAfter;
	float* __restrict__ Cp = p.c + oc;
	unsigned char* alive = p.ep.alive ? p.ep.alive + oc : nullptr;
	if constexpr (!EDGE) {
		// Interior tiles (C 16-byte aligned, ldc a multiple of 4): each wave passes its accumulators through its own
		// slice of the operand LDS (free after the depth loop's last barrier), RP rows of one MFMA row-block at a
		// time, and writes C as 16-byte stores of 4 consecutive columns; the epilogue is applied per element.
		constexpr int kPerWave = S::kLdsFloats / 4;
		constexpr int LS = WN + 4;
		constexpr int RP = (MF == kMf4 || MF == kMf16x4) ? 16 : (U::UM * LS <= kPerWave ? U::UM : (U::UM / 2 * LS <= kPerWave ? U::UM / 2 : 16));
		static_assert(RP * LS <= kPerWave, "an epilogue pass must fit in the wave's LDS slice");
		static_assert(passes_split_evenly<MF>(RP), "a register's pass must not depend on the lane");
		constexpr int kChunks = RP * WN / 4;        // 4-column groups in one pass
		constexpr int kRowChunks = WN / 4;
		float* st = lds + wave * kPerWave;
		const bool plain = !add_old_at_end && p.ep.bias_mode == kBiasNone && !p.ep.relu && !p.ep.res;
#pragma unroll
		for (int i = 0; i < I; ++i)
#pragma unroll
			for (int pass = 0; pass < U::UM / RP; ++pass) {
				// a register's pass does not depend on the lane: every lane-dependent row offset stays inside it
#pragma unroll
				for (int j = 0; j < J; ++j)
#pragma unroll
					for (int r = 0; r < U::NV; ++r) {
						if (U::crow(r, 0) / RP != pass) continue;
						st[(U::crow(r, lane_e) - pass * RP) * LS + U::UN * j + U::ccol(lane_e)] = acc[i][j][r];
					}
				static_assert(kChunks % 64 == 0, "a pass is a whole number of 16-byte stores per lane");
				if (plain) {
#pragma unroll
					for (int t = 0; t < kChunks / 64; ++t) {
						const int ch = lane_e + 64 * t;
						const int lr = ch / kRowChunks, c4 = (ch % kRowChunks) * 4;
						const int row = m0 + wm0 + U::UM * i + pass * RP + lr, col = n0 + wn0 + c4;
						*reinterpret_cast<f32x4*>(Cp + (int64_t)row * p.ldc + col) =
							*reinterpret_cast<const f32x4*>(st + lr * LS + c4);
					}
					continue;
				}
#pragma unroll
				for (int t = 0; t < kChunks / 64; ++t) {
					const int ch = lane_e + 64 * t;
					const int lr = ch / kRowChunks, c4 = (ch % kRowChunks) * 4;
					f32x4 v = *reinterpret_cast<const f32x4*>(st + lr * LS + c4);
					const int row = m0 + wm0 + U::UM * i + pass * RP + lr, col = n0 + wn0 + c4;
					const int64_t off = (int64_t)row * p.ldc + col;
					if (add_old_at_end) {
						const f32x4 old = *reinterpret_cast<const f32x4*>(Cp + off);
#pragma unroll
						for (int e = 0; e < 4; ++e) v[e] = (p.k > 0) ? old[e] + v[e] : old[e];
					}
#pragma unroll
					for (int e = 0; e < 4; ++e) {
						if (p.ep.bias_mode == kBiasCol) v[e] = v[e] + p.ep.bias[col + e];
						else if (p.ep.bias_mode == kBiasRow) v[e] = v[e] + p.ep.bias[row];
						if (p.ep.res) v[e] = p.ep.res[oc + off + e] + v[e];
						if (p.ep.relu) {
							const bool on = v[e] > 0.0f;
							if (alive) alive[off + e] = on ? 1 : 0;
							v[e] = on ? v[e] : 0.0f;
						}
					}
					*reinterpret_cast<f32x4*>(Cp + off) = v;
				}
			}
		return;
	}
#pragma unroll
	for (int i = 0; i < I; ++i)
#pragma unroll
		for (int j = 0; j < J; ++j) {
			// one MFMA unit at a time: bounds the registers the epilogue keeps live
			__builtin_amdgcn_sched_barrier(0);
			const int col = n0 + c_col(j, lane_e);
#pragma unroll
			for (int r = 0; r < U::NV; ++r) {
				const int row = m0 + c_row(i, r, lane_e);
				if (EDGE && (row >= p.m || col >= p.n)) continue;
				const int64_t off = (int64_t)row * p.ldc + col;
				float v = acc[i][j][r];
				if (add_old_at_end) v = (p.k > 0) ? Cp[off] + v : Cp[off];
				if (p.ep.bias_mode == kBiasCol) v = v + p.ep.bias[col];
				else if (p.ep.bias_mode == kBiasRow) v = v + p.ep.bias[row];
				if (p.ep.res) v = p.ep.res[oc + off] + v;
				if (p.ep.relu) {
					const bool on = v > 0.0f;
					if (alive) alive[off] = on ? 1 : 0;
					v = on ? v : 0.0f;
				}
				Cp[off] = v;
			}
		}
}

template <int BM, int BN, int BK, int WM, int WN, int WPE, int MF, bool TA, bool TB, bool EDGE, bool GB = false,
          bool RS = false>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE, WPE))) sgemm_tile_kernel(const GemmArgs p) {
	sgemm_tile_body<BM, BN, BK, WM, WN, MF, TA, TB, EDGE, GB, RS>(p, (int)blockIdx.x);
}

// Two independent products in one launch: A B (p0, workgroups below blocks0) and A^T B, with or without row sums
// (p1, the rest). A Linear backward's dX and dW are such a pair; when both are small, their tiles then run side by
// side instead of one product after the other. Each product's elements are computed exactly as in its own launch.
template <int BM, int BN, int BK, int WM, int WN, int WPE, int MF, bool EDGE0, bool EDGE1, bool RS1>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
sgemm_pair_kernel(const GemmArgs p0, const GemmArgs p1, int blocks0) {
	const int b = (int)blockIdx.x;
	if (b < blocks0) sgemm_tile_body<BM, BN, BK, WM, WN, MF, false, false, EDGE0>(p0, b);
	else sgemm_tile_body<BM, BN, BK, WM, WN, MF, true, false, EDGE1, false, RS1>(p1, b - blocks0);
}

}  // namespace nnh
