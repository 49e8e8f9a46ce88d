// gemm_valu.hip - the fp32 GEMM on the vector ALUs, for products too small to fill the GPU with MFMA tiles.
//
// Under nn-cpp's contract every element of C is one fma chain over the depth (gemm.cpp:232-244), so a product that
// cannot keep the matrix cores busy with independent chains runs at the latency of a dependent k = 1 MFMA, 44
// cycles per step. A dependent v_fma_f32 takes about 6 cycles, and a wave's lanes each run their own chains: here
// every lane owns an RM x RN block of C and runs its RM * RN chains interleaved, so the VALU issues back to back.
//   * A workgroup (4 waves as 2 x 2, each 8 x 8 lanes) owns a (16 RM) x (16 RN) tile. The depth is staged in LDS
//     in chunks of 256, both operands k-contiguous (op(A) rows, op(B) columns; the transposes happen on the way in),
//     row pitch 260 floats: a wave's 16-byte reads of 8 distinct rows land on distinct banks. A chunk's fmas take
//     longer than the next chunk's global loads, which are in registers meanwhile (one wait per chunk).
//   * Per four depth steps a lane reads RM + RN 16-byte words and issues 4 RM RN fmas, in depth order per chain,
//     the next group's reads in flight.
//   * The accumulate rule, the epilogue and the edges are the MFMA kernel's: old C joins after the first 256 steps
//     (Store::kAdd, gemm.cpp:245-252), then bias, ReLU and the alive flags; only the m x n window is written.
// Every chain has exactly k steps (a partial last chunk runs element by element), so -0 results stay -0.
// A second kernel below (sgemm_valu_bc_kernel) feeds op(A) through registers and DPP row broadcasts instead of LDS.
// The caller sends here only products without a depth cut.
#include "gemm_valu.hpp"

#include <utility>

namespace nnh {

namespace {

// VC: depth per LDS chunk (the chunk's fmas outlast the next chunk's global loads); row pitch VC + 4 floats, 4 mod 64:
// 16-byte reads of rows 4 floats apart hit distinct banks.
template <int RM, int RN, int VC>
struct VShape {
	static constexpr int BM = 16 * RM, BN = 16 * RN;
	static constexpr int kVp = VC + 4;
	static constexpr int kBuf = (BM + BN) * kVp;   // floats of one chunk buffer
	static_assert((BM * VC) % 1024 == 0 && (BN * VC) % 1024 == 0, "tiles split evenly over 256 threads");
};

// One chunk of op(X) (X = A with rows m, or B with columns n) into registers. R is the tile's row count (BM or BN),
// rows are the m (or n) index, the depth index runs along the LDS row. KCONTIG: element (r, p) at X[r * ld + p]
// (A untransposed, B transposed); otherwise at X[p * ld + r]. Branch-free: every address is clamped into the
// matrix, so nothing outside it is read and every load is in flight at once; the values read for rows past the
// matrix feed chains that are never stored, those for depth indices past k are never used (a partial chunk runs
// exactly its k steps). VEC (16-byte loads) needs ld a multiple of 4, a 16-byte aligned base, and the contiguous
// extent (k, or the rows) a multiple of 4.
template <int R, bool KCONTIG, bool VEC, int kVc>
struct ChunkLoader {
	static constexpr int kVp = kVc + 4;
	static constexpr int kPer = R * kVc / 4 / 256;
	__device__ __forceinline__ static void load(const float* __restrict__ x, int64_t ld, int r0, int rows, int k0,
	                                            int kdim, f32x4 (&v)[kPer], int tid) {
#pragma unroll
		for (int u = 0; u < kPer; ++u) {
			const int idx = tid + 256 * u;
			int r, p;
			if (KCONTIG) {
				r = idx / (kVc / 4);
				p = 4 * (idx % (kVc / 4));
			} else {
				p = idx / (R / 4);
				r = 4 * (idx % (R / 4));
			}
			const int gr = r0 + r, gp = k0 + p;
			if (KCONTIG) {
				const float* src = x + (int64_t)min(gr, rows - 1) * ld;
				if (VEC) {
					v[u] = *reinterpret_cast<const f32x4*>(src + min(gp, kdim - 4));
				} else {
#pragma unroll
					for (int e = 0; e < 4; ++e) v[u][e] = src[min(gp + e, kdim - 1)];
				}
			} else {
				const float* src = x + (int64_t)min(gp, kdim - 1) * ld;
				if (VEC) {
					v[u] = *reinterpret_cast<const f32x4*>(src + min(gr, rows - 4));
				} else {
#pragma unroll
					for (int e = 0; e < 4; ++e) v[u][e] = src[min(gr + e, rows - 1)];
				}
			}
		}
	}
	// into the LDS tile dst[r][p] (pitch kVp)
	__device__ __forceinline__ static void store(float* dst, const f32x4 (&v)[kPer], int tid) {
#pragma unroll
		for (int u = 0; u < kPer; ++u) {
			const int idx = tid + 256 * u;
			if (KCONTIG) {
				const int r = idx / (kVc / 4), p = 4 * (idx % (kVc / 4));
				*reinterpret_cast<f32x4*>(dst + r * kVp + p) = v[u];
			} else {
				const int p = idx / (R / 4), r = 4 * (idx % (R / 4));
#pragma unroll
				for (int e = 0; e < 4; ++e) dst[(r + e) * kVp + p] = v[u][e];
			}
		}
	}
};

template <bool TA, bool TB, int RM, int RN, bool VEC, int kVc>
__global__ void __launch_bounds__(256) sgemm_valu_kernel(const GemmArgs p) {
	using S = VShape<RM, RN, kVc>;
	using LA = ChunkLoader<S::BM, !TA, VEC, kVc>;
	using LB = ChunkLoader<S::BN, TB, VEC, kVc>;
	constexpr int kVp = S::kVp;
	extern __shared__ __align__(16) float lds[];  // 2 * S::kBuf floats
	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const int tiles = p.tiles_m * p.tiles_n;
	const int t = blockIdx.x % tiles, bi = blockIdx.x / tiles;
	const int tm = t / p.tiles_n, tn = t - tm * p.tiles_n;
	const int m0 = tm * S::BM, n0 = tn * S::BN;
	int64_t oa = 0, ob = 0, oc = 0;
	if (p.batch.ndim > 0) batch_offsets(p.batch, bi, oa, ob, oc);
	const float* __restrict__ A = p.a + oa;
	const float* __restrict__ B = p.b + ob;
	// this lane's block: rows lr0 .. lr0 + RM - 1, columns lc0 .. lc0 + RN - 1 of the tile
	const int lr0 = (wave >> 1) * 8 * RM + (lane >> 3) * RM;
	const int lc0 = (wave & 1) * 8 * RN + (lane & 7) * RN;

	float acc[RM][RN];
#pragma unroll
	for (int i = 0; i < RM; ++i)
#pragma unroll
		for (int j = 0; j < RN; ++j) acc[i][j] = 0.0f;

	const int nch = (p.k + kVc - 1) / kVc;
	// the next chunk's global loads are in registers while the current chunk runs from LDS
	f32x4 ra[LA::kPer], rb[LB::kPer];
	auto gload = [&](int ch) {
		const int k0 = ch * kVc;
		LA::load(A, p.lda, m0, p.m, k0, p.k, ra, tid);
		LB::load(B, p.ldb, n0, p.n, k0, p.k, rb, tid);
	};
	auto lstore = [&](int buf) {
		float* base = lds + buf * S::kBuf;
		LA::store(base, ra, tid);
		LB::store(base + S::BM * kVp, rb, tid);
	};
	// the old C joins the chain after the first 256 steps (kAccAfter: the end of chunk kAccAfter / VC - 1), or at
	// the end of a shorter one
	static_assert(kAccAfter % kVc == 0, "the accumulate point is a chunk boundary");
	const bool acc_mode = p.accumulate != 0;
	auto add_old = [&]() {
#pragma unroll
		for (int i = 0; i < RM; ++i)
#pragma unroll
			for (int j = 0; j < RN; ++j) {
				const int row = m0 + lr0 + i, col = n0 + lc0 + j;
				if (row < p.m && col < p.n) acc[i][j] = p.c[oc + (int64_t)row * p.ldc + col] + acc[i][j];
			}
	};
	auto compute = [&](int ch) {
		const float* As = lds + (ch & 1) * S::kBuf + lr0 * kVp;
		const float* Bs = lds + (ch & 1) * S::kBuf + S::BM * kVp + lc0 * kVp;
		const int kc = min(kVc, p.k - ch * kVc);
		auto rd = [&](f32x4 (&a)[RM], f32x4 (&b)[RN], int q) {
#pragma unroll
			for (int i = 0; i < RM; ++i) a[i] = *reinterpret_cast<const f32x4*>(As + i * kVp + 4 * q);
#pragma unroll
			for (int j = 0; j < RN; ++j) b[j] = *reinterpret_cast<const f32x4*>(Bs + j * kVp + 4 * q);
		};
		auto fm = [&](const f32x4 (&a)[RM], const f32x4 (&b)[RN], int steps) {
#pragma unroll
			for (int u = 0; u < 4; ++u)
				if (u < steps)
#pragma unroll
					for (int i = 0; i < RM; ++i)
#pragma unroll
						for (int j = 0; j < RN; ++j) acc[i][j] = __builtin_fmaf(a[i][u], b[j][u], acc[i][j]);
		};
		// runs of 16 groups of 4 depth steps; inside a run the next group's 16-byte reads are issued before this
		// group's fmas
		const int q_full = kc / 4;
		int q0 = 0;
		for (; q0 + 16 <= q_full; q0 += 16) {
			f32x4 a0[RM], b0[RN], a1[RM], b1[RN];
			rd(a0, b0, q0);
#pragma unroll
			for (int q = 0; q < 16; q += 2) {
				rd(a1, b1, q0 + q + 1);
				fm(a0, b0, 4);
				if (q + 2 < 16) rd(a0, b0, q0 + q + 2);
				fm(a1, b1, 4);
			}
		}
		for (; q0 < q_full; ++q0) {
			f32x4 a0[RM], b0[RN];
			rd(a0, b0, q0);
			fm(a0, b0, 4);
		}
		if (kc % 4) {  // the last 1-3 steps of the depth
			f32x4 a0[RM], b0[RN];
			rd(a0, b0, q_full);
			fm(a0, b0, kc % 4);
		}
	};

	gload(0);
	lstore(0);
	__syncthreads();
	for (int ch = 0; ch < nch; ++ch) {
		if (ch + 1 < nch) gload(ch + 1);
		compute(ch);
		if (ch == kAccAfter / kVc - 1 && acc_mode && p.k > kAccAfter) add_old();
		if (ch + 1 < nch) lstore((ch + 1) & 1);
		__syncthreads();
	}

	// epilogue
	const bool add_old_at_end = acc_mode && p.k <= kAccAfter;
	float* __restrict__ Cp = p.c + oc;
	unsigned char* alive = p.ep.alive ? p.ep.alive + oc : nullptr;
#pragma unroll
	for (int i = 0; i < RM; ++i) {
		const int row = m0 + lr0 + i;
		if (row >= p.m) continue;
#pragma unroll
		for (int j = 0; j < RN; ++j) {
			const int col = n0 + lc0 + j;
			if (col >= p.n) continue;
			const int64_t off = (int64_t)row * p.ldc + col;
			float v = acc[i][j];
			if (add_old_at_end) v = Cp[off] + v;
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

// ---- the row-broadcast variant: op(A) through registers and DPP, only op(B) through LDS ----
//
// The kernel above reads RM + RN LDS words per lane for RM * RN fmas, and the LDS is what binds it. Here a lane
// (q, c) = (lane >> 4, lane & 15) of wave w owns RM chains: rows m0 + 4 RM w + 4 i + q (i < RM) of op(A) and column
// n0 + c. op(A) never enters LDS: for each block of 16 depth steps, lane (q, j) holds op(A)[row(q, i)][k0 + j] in
// register a[i] (one dword load per lane and chain), and the fma of step j takes it from lane j of the lane's
// 16-lane row by a DPP row broadcast inside the instruction (v_fmac_f32_dpp ... row_newbcast:j). op(B)'s 16 columns
// of a 256-deep chunk sit in LDS, shared by the four waves; a lane reads its column's 16 values of a block as four
// 16-byte words, so a depth step costs one 4-byte LDS word per lane against RM fmas. A DPP read of a register
// written by a VALU instruction less than two cycles before is a hazard, so the first broadcast fma of each chain
// in a block is preceded by s_nop 1 in the same asm statement (the registers are loaded from memory, or at most
// copied between chunks). The last partial block (k not a multiple of 16) takes its values by ds_bpermute
// (__shfl) instead. Every chain runs exactly k steps, in depth order, from +0.

template <int J, bool FIRST>
__device__ __forceinline__ void fmac_bcast(float& acc, float a, float b) {
	if (FIRST)
		asm("s_nop 1\n\tv_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
		    : "+v"(acc)
		    : "v"(a), "v"(b), "i"(J));
	else
		asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(a), "v"(b), "i"(J));
}

template <int RM, int... J>
__device__ __forceinline__ void bcast_block(float (&acc)[RM], const float (&a)[RM], const float (&b)[16],
                                            std::integer_sequence<int, J...>) {
	(
	    [&] {
#pragma unroll
		    for (int i = 0; i < RM; ++i) fmac_bcast<J, J == 0>(acc[i], a[i], b[J]);
	    }(),
	    ...);
}

constexpr int kBcVc = 256;           // depth per LDS chunk
constexpr int kBcVp = kBcVc + 4;     // pitch: 16-byte reads of the 16 columns hit distinct banks

template <bool TA, bool TB, int RM, bool VEC>
__global__ void __launch_bounds__(256) sgemm_valu_bc_kernel(const GemmArgs p) {
	constexpr int BN = 16, kBlocks = kBcVc / 16;
	using LB = ChunkLoader<BN, TB, VEC, kBcVc>;
	__shared__ __align__(16) float lds[2 * BN * kBcVp];
	const int tid = threadIdx.x, lane = tid & 63;
	const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
	const int q = lane >> 4, c = lane & 15;
	const int tiles = p.tiles_m * p.tiles_n;
	const int t = blockIdx.x % tiles, bi = blockIdx.x / tiles;
	const int tm = t / p.tiles_n, tn = t - tm * p.tiles_n;
	const int m0 = tm * 16 * RM, n0 = tn * BN;
	int64_t oa = 0, ob = 0, oc = 0;
	if (p.batch.ndim > 0) batch_offsets(p.batch, bi, oa, ob, oc);
	const float* __restrict__ A = p.a + oa;
	const float* __restrict__ B = p.b + ob;
	const int rbase = m0 + wave * 4 * RM;
	const int K = p.k;

	float acc[RM];
#pragma unroll
	for (int i = 0; i < RM; ++i) acc[i] = 0.0f;

	// op(A) of one chunk: a[b][i] = op(A)[row(q, i)][chunk k0 + 16 b + c], addresses clamped into the matrix
	auto aload = [&](int ch, float (&a)[kBlocks][RM]) {
#pragma unroll
		for (int b = 0; b < kBlocks; ++b)
#pragma unroll
			for (int i = 0; i < RM; ++i) {
				const int64_t row = min(rbase + 4 * i + q, p.m - 1);
				const int64_t kk = min(ch * kBcVc + 16 * b + c, K - 1);
				a[b][i] = TA ? A[kk * p.lda + row] : A[row * p.lda + kk];
			}
	};
	f32x4 rb[LB::kPer];
	float ac[kBlocks][RM], an[kBlocks][RM];
	const int nch = (K + kBcVc - 1) / kBcVc;
	const bool acc_mode = p.accumulate != 0;
	auto add_old = [&]() {
		const int col = n0 + c;
#pragma unroll
		for (int i = 0; i < RM; ++i) {
			const int row = rbase + 4 * i + q;
			if (row < p.m && col < p.n) acc[i] = p.c[oc + (int64_t)row * p.ldc + col] + acc[i];
		}
	};

	aload(0, ac);
	LB::load(B, p.ldb, n0, p.n, 0, K, rb, tid);
	LB::store(lds, rb, tid);
	__syncthreads();
	for (int ch = 0; ch < nch; ++ch) {
		if (ch + 1 < nch) {
			aload(ch + 1, an);
			LB::load(B, p.ldb, n0, p.n, (ch + 1) * kBcVc, K, rb, tid);
		}
		const float* Bs = lds + (ch & 1) * BN * kBcVp + c * kBcVp;
		const int kc = __builtin_amdgcn_readfirstlane(min(kBcVc, K - ch * kBcVc));
		auto bread = [&](int b, float (&bv)[16]) {
#pragma unroll
			for (int u = 0; u < 4; ++u) {
				const f32x4 w = *reinterpret_cast<const f32x4*>(Bs + 16 * b + 4 * u);
				bv[4 * u] = w[0];
				bv[4 * u + 1] = w[1];
				bv[4 * u + 2] = w[2];
				bv[4 * u + 3] = w[3];
			}
		};
		if (kc == kBcVc) {
			// a whole chunk, straight-line: the next block's LDS words are in flight during this block's fmas
			float bv0[16], bv1[16];
			bread(0, bv0);
#pragma unroll
			for (int b = 0; b < kBlocks; b += 2) {
				bread(b + 1, bv1);
				bcast_block<RM>(acc, ac[b], bv0, std::make_integer_sequence<int, 16>{});
				if (b + 2 < kBlocks) bread(b + 2, bv0);
				bcast_block<RM>(acc, ac[b + 1], bv1, std::make_integer_sequence<int, 16>{});
			}
		} else {
			const int nb = kc / 16, rem = kc % 16;
#pragma unroll
			for (int b = 0; b < kBlocks; ++b) {
				if (b < nb) {
					float bv[16];
					bread(b, bv);
					bcast_block<RM>(acc, ac[b], bv, std::make_integer_sequence<int, 16>{});
				} else if (b == nb && rem) {
					for (int j = 0; j < rem; ++j) {
						const float bj = Bs[16 * b + j];
#pragma unroll
						for (int i = 0; i < RM; ++i)
							acc[i] = __builtin_fmaf(__shfl(ac[b][i], (lane & 48) | j), bj, acc[i]);
					}
				}
			}
		}
		if (ch == kAccAfter / kBcVc - 1 && acc_mode && K > kAccAfter) add_old();
		if (ch + 1 < nch) LB::store(lds + ((ch + 1) & 1) * BN * kBcVp, rb, tid);
		__syncthreads();
		if (ch + 1 < nch) {
#pragma unroll
			for (int b = 0; b < kBlocks; ++b)
#pragma unroll
				for (int i = 0; i < RM; ++i) ac[b][i] = an[b][i];
		}
	}

	const bool add_old_at_end = acc_mode && K <= kAccAfter;
	float* __restrict__ Cp = p.c + oc;
	unsigned char* alive = p.ep.alive ? p.ep.alive + oc : nullptr;
	const int col = n0 + c;
	if (col >= p.n) return;
#pragma unroll
	for (int i = 0; i < RM; ++i) {
		const int row = rbase + 4 * i + q;
		if (row >= p.m) continue;
		const int64_t off = (int64_t)row * p.ldc + col;
		float v = acc[i];
		if (add_old_at_end) v = Cp[off] + v;
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

// ---- cut products on the VALU: all pieces of an output in one lane ----
//
// A product with a depth cut is, per element, pieces of piece_k depth steps, each a chain from +0, added in piece
// order, then the old C (gemm.cpp:453-485). Cut products are small (at most 2^16 outputs in nn-cpp's rule), and
// their pieces are independent chains: a lane runs all NP of its output's pieces interleaved, so the latency of a
// DPP-fed fma (about 17 cycles) hides behind the other chains. A workgroup owns 16 x 16 outputs (wave w, lane
// (q, c): row m0 + 4 w + q, column n0 + c). op(A) comes by DPP row broadcasts as in the kernel above (one dword per
// lane, piece and 16-step block, all loaded up front); op(B)'s 16 columns stay in LDS for the whole depth
// (k-contiguous, pitch 4 mod 64 floats), staged once with every load in flight before the stores. A chain slot past
// the last piece runs piece 0's addresses and is dropped; the last piece runs exactly its own (possibly shorter)
// depth. The pieces are then added in order, the old C, bias and ReLU applied.

constexpr int kPcMaxBlocks = 8;     // piece depth <= 128
constexpr int kPcMaxK = 2048;       // op(B)'s 16 columns of the whole depth in LDS: <= 131 KB
constexpr int kPcMaxPieces = 8;   // forced (a configuration index); the shape rule sends at most 4
constexpr int kPcMaxOutputs = 1 << 16;

inline int pc_pitch(int k) { return ((k + 63) / 64) * 64 + 4; }

// four depth steps J0 .. J0 + 3 of a 16-step block, for every chain
template <int NP, int J0, int... J>
__device__ __forceinline__ void bcast_quad(float (&acc)[NP], const float (&a)[NP], const f32x4 (&b)[NP],
                                           std::integer_sequence<int, J...>) {
	(
	    [&] {
#pragma unroll
		    for (int u = 0; u < NP; ++u) fmac_bcast<J0 + J, J0 + J == 0>(acc[u], a[u], b[u][J]);
	    }(),
	    ...);
}

// SPLIT (more than four pieces): the workgroup owns 4 x 16 outputs instead (lane (q, c): row m0 + q) and wave w runs
// pieces w, w + 4 (NP = 2 chains per lane), so a small product spreads over four times the workgroups; the waves'
// results meet in LDS and the first wave adds them in piece order.
template <bool TA, bool TB, int NP, bool VEC, bool SPLIT>
__global__ void __launch_bounds__(256) sgemm_valu_pieces_kernel(const GemmArgs p) {
	extern __shared__ __align__(16) float lds[];  // [16][pitch]: lds[cc * pitch + kk] = op(B)[kk][n0 + cc]
	const int tid = threadIdx.x, lane = tid & 63;
	const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
	const int q = lane >> 4, c = lane & 15;
	const int tiles = p.tiles_m * p.tiles_n;
	const int t = blockIdx.x % tiles, bi = blockIdx.x / tiles;
	const int tm = t / p.tiles_n, tn = t - tm * p.tiles_n;
	const int m0 = tm * (SPLIT ? 4 : 16), n0 = tn * 16;
	int64_t oa = 0, ob = 0, oc = 0;
	if (p.batch.ndim > 0) batch_offsets(p.batch, bi, oa, ob, oc);
	const float* __restrict__ A = p.a + oa;
	const float* __restrict__ B = p.b + ob;
	const int K = p.k, P = p.pieces, pk = p.piece_k;
	const int pitch = ((K + 63) / 64) * 64 + 4;
	const int row = SPLIT ? m0 + q : m0 + 4 * wave + q, col = n0 + c;
	const int64_t rowc = min(row, p.m - 1);

	int pce[NP], len[NP];  // the piece each chain slot runs (piece 0 for an empty slot) and its depth
#pragma unroll
	for (int u = 0; u < NP; ++u) {
		const int pc = SPLIT ? wave + 4 * u : u;
		pce[u] = pc < P ? pc : 0;
		len[u] = pc < P ? min(pk, K - pc * pk) : pk;
	}
	float a[NP][kPcMaxBlocks];
#pragma unroll
	for (int u = 0; u < NP; ++u)
#pragma unroll
		for (int b = 0; b < kPcMaxBlocks; ++b) {
			const int64_t kk = min(pce[u] * pk + 16 * b + c, K - 1);
			a[u][b] = TA ? A[kk * p.lda + rowc] : A[rowc * p.lda + kk];
		}

	// op(B) into LDS, sixteen loads in flight per thread before their stores
	if (VEC) {  // K (TB) or n (!TB) a multiple of 4, 16-byte rows
		const int total = TB ? 16 * (K / 4) : K * 4;
		for (int e0 = 0; e0 < total; e0 += 16 * 256) {
			f32x4 v[16];
#pragma unroll
			for (int u = 0; u < 16; ++u) {
				const int e = min(e0 + tid + 256 * u, total - 1);
				if (TB) {
					const int cc = e / (K / 4), k4 = 4 * (e - cc * (K / 4));
					v[u] = *reinterpret_cast<const f32x4*>(B + (int64_t)min(n0 + cc, p.n - 1) * p.ldb + k4);
				} else {
					const int kk = e >> 2, c4 = 4 * (e & 3);
					v[u] = *reinterpret_cast<const f32x4*>(B + (int64_t)kk * p.ldb + min(n0 + c4, p.n - 4));
				}
			}
#pragma unroll
			for (int u = 0; u < 16; ++u) {
				const int e = e0 + tid + 256 * u;
				if (e >= total) continue;
				if (TB) {
					const int cc = e / (K / 4), k4 = 4 * (e - cc * (K / 4));
					*reinterpret_cast<f32x4*>(lds + cc * pitch + k4) = v[u];
				} else {
					const int kk = e >> 2, c4 = 4 * (e & 3);
					// columns n0 + c4 .. + 3 came from min(n0 + c4, n - 4): shift back when clamped
					const int sh = n0 + c4 - min(n0 + c4, p.n - 4);
#pragma unroll
					for (int x = 0; x < 4; ++x) lds[(c4 + x) * pitch + kk] = v[u][min(x + sh, 3)];
				}
			}
		}
	} else {
		const int total = 16 * K;
		for (int e0 = 0; e0 < total; e0 += 8 * 256) {
			float v[8];
#pragma unroll
			for (int u = 0; u < 8; ++u) {
				const int e = min(e0 + tid + 256 * u, total - 1);
				int cc, kk;
				if (TB) {
					cc = e / K;
					kk = e - cc * K;
				} else {
					kk = e >> 4;
					cc = e & 15;
				}
				const int64_t gc = min(n0 + cc, p.n - 1);
				v[u] = TB ? B[gc * p.ldb + kk] : B[(int64_t)kk * p.ldb + gc];
			}
#pragma unroll
			for (int u = 0; u < 8; ++u) {
				const int e = e0 + tid + 256 * u;
				if (e >= total) continue;
				const int cc = TB ? e / K : (e & 15), kk = TB ? e - (e / K) * K : (e >> 4);
				lds[cc * pitch + kk] = v[u];
			}
		}
	}
	__syncthreads();

	float acc[NP];
#pragma unroll
	for (int u = 0; u < NP; ++u) acc[u] = 0.0f;
	const float* Bc = lds + c * pitch;
#pragma unroll
	for (int b = 0; b < kPcMaxBlocks; ++b) {
		if (16 * b >= pk) break;
		bool all_full = true;
#pragma unroll
		for (int u = 0; u < NP; ++u) all_full = all_full && 16 * (b + 1) <= len[u];
		float av[NP];
#pragma unroll
		for (int u = 0; u < NP; ++u) av[u] = a[u][b];
		if (all_full) {
			f32x4 b0[NP], b1[NP];
#pragma unroll
			for (int u = 0; u < NP; ++u) b0[u] = *reinterpret_cast<const f32x4*>(Bc + pce[u] * pk + 16 * b);
#pragma unroll
			for (int u = 0; u < NP; ++u) b1[u] = *reinterpret_cast<const f32x4*>(Bc + pce[u] * pk + 16 * b + 4);
			bcast_quad<NP, 0>(acc, av, b0, std::make_integer_sequence<int, 4>{});
#pragma unroll
			for (int u = 0; u < NP; ++u) b0[u] = *reinterpret_cast<const f32x4*>(Bc + pce[u] * pk + 16 * b + 8);
			bcast_quad<NP, 4>(acc, av, b1, std::make_integer_sequence<int, 4>{});
#pragma unroll
			for (int u = 0; u < NP; ++u) b1[u] = *reinterpret_cast<const f32x4*>(Bc + pce[u] * pk + 16 * b + 12);
			bcast_quad<NP, 8>(acc, av, b0, std::make_integer_sequence<int, 4>{});
			bcast_quad<NP, 12>(acc, av, b1, std::make_integer_sequence<int, 4>{});
		} else {
			// the last piece ends inside this block or earlier: every chain on its own, by ds_bpermute
#pragma unroll
			for (int u = 0; u < NP; ++u) {
				const int steps = min(16, len[u] - 16 * b);
				const float* bp = Bc + pce[u] * pk + 16 * b;
				for (int j = 0; j < steps; ++j) acc[u] = __builtin_fmaf(__shfl(av[u], (lane & 48) | j), bp[j], acc[u]);
			}
		}
	}
	float v;
	if (SPLIT) {
		float* part = lds + 16 * pitch;  // [P][64]
#pragma unroll
		for (int u = 0; u < NP; ++u)
			if (wave + 4 * u < P) part[(wave + 4 * u) * 64 + lane] = acc[u];
		__syncthreads();
		if (wave != 0) return;
		v = part[lane];
		for (int pc = 1; pc < P; ++pc) v = v + part[pc * 64 + lane];
	} else {
		v = acc[0];
#pragma unroll
		for (int u = 1; u < NP; ++u)
			if (u < P) v = v + acc[u];
	}
	if (row >= p.m || col >= p.n) return;
	float* __restrict__ Cp = p.c + oc;
	const int64_t off = (int64_t)row * p.ldc + col;
	if (p.accumulate) v = Cp[off] + v;
	if (p.ep.bias_mode == kBiasCol) v = v + p.ep.bias[col];
	else if (p.ep.bias_mode == kBiasRow) v = v + p.ep.bias[row];
	if (p.ep.res) v = p.ep.res[oc + off] + v;
	if (p.ep.relu) {
		const bool on = v > 0.0f;
		if (p.ep.alive) p.ep.alive[oc + off] = on ? 1 : 0;
		v = on ? v : 0.0f;
	}
	Cp[off] = v;
}

typedef void (*ValuFn)(const GemmArgs);

template <int RM, int RN, bool VEC, int VC>
ValuFn valu_fn(int ta, int tb) {
	if (!ta && !tb) return sgemm_valu_kernel<false, false, RM, RN, VEC, VC>;
	if (!ta && tb) return sgemm_valu_kernel<false, true, RM, RN, VEC, VC>;
	if (ta && !tb) return sgemm_valu_kernel<true, false, RM, RN, VEC, VC>;
	return sgemm_valu_kernel<true, true, RM, RN, VEC, VC>;
}

template <int RM, bool VEC>
ValuFn valu_bc_fn(int ta, int tb) {
	if (!ta && !tb) return sgemm_valu_bc_kernel<false, false, RM, VEC>;
	if (!ta && tb) return sgemm_valu_bc_kernel<false, true, RM, VEC>;
	if (ta && !tb) return sgemm_valu_bc_kernel<true, false, RM, VEC>;
	return sgemm_valu_bc_kernel<true, true, RM, VEC>;
}

struct ValuShape {
	int rm, rn, vc;  // rn 0: the row-broadcast kernel (tile 16 rm x 16)
};
// kValu2x2, kValu1x2, kValu2x4, kValu1x4, kValuBc1, kValuBc2
constexpr ValuShape kShapes[kValuShapes] = {{2, 2, 256}, {1, 2, 256}, {2, 4, 128}, {1, 4, 128}, {1, 0, kBcVc},
                                            {2, 0, kBcVc}};

template <bool VEC>
ValuFn valu_pick(int shape, int ta, int tb) {
	switch (shape) {
	case kValu2x2: return valu_fn<2, 2, VEC, 256>(ta, tb);
	case kValu1x2: return valu_fn<1, 2, VEC, 256>(ta, tb);
	case kValu2x4: return valu_fn<2, 4, VEC, 128>(ta, tb);
	case kValu1x4: return valu_fn<1, 4, VEC, 128>(ta, tb);
	case kValuBc1: return valu_bc_fn<1, VEC>(ta, tb);
	default: return valu_bc_fn<2, VEC>(ta, tb);
	}
}

}  // namespace

int valu_shape(const GemmCall& g) {
	if (g.ta) return kValu1x2;
	const double outputs = (double)g.m * (double)g.n * (double)g.batch_count;
	return outputs <= 131072.0 ? kValuBc1 : kValuBc2;
}

bool valu_takes(const GemmCall& g) {
	if (g.gather || g.rowsum || g.k <= 0 || g.m <= 0 || g.n <= 0) return false;
	if (depth_cut(g.m, g.n, g.k)) return false;
	if (g.m >= (1 << 30) || g.n >= (1 << 30) || g.k >= (1 << 30)) return false;
	// Measured against the MFMA tiles (device time, one MI355X, every configuration forced):
	// * op(A) untransposed, the row-broadcast kernel: one chain per lane up to 2^17 outputs (256 x 512 x 784 NT 9.8
	//   against 11.2 us for the 1 x 2 lane block and 14.3 for the best MFMA tile; 256 x 10 x 256 4.4 against 5.3;
	//   256 x 512 x 256 NN 4.7 against 5.4), two chains per lane up to 2^18 outputs at depths up to 512 with op(B)
	//   untransposed (512^3 NN 9.75 against 10.3, 256 x 784 x 512 NN 9.1 against 11.9; 512^3 NT 9.8 against the
	//   MFMA tiles' 9.3); at 2^18 outputs and deeper it ties with the MFMA tiles (64 x 4096 x 4096: 58.6 against
	//   59.8; 256 x 1024 x 1024 NT: 15.7 against 15.2), and from 2^20 they win (1024^3: 27 against 47).
	// * op(A) transposed (its dword loads are strided), the 1 x 2 lane block, up to 2^17 outputs: slower than the
	//   MFMA tiles from 2^18 (512^3 TN: 15.0 against 10.9), where they have enough chains to overlap their 44-cycle
	//   steps and this kernel's LDS reads bind it.
	// Against the 16x16x4 tiles (four depth indices per chain step): the row-broadcast kernel keeps products up to 2^17
	// outputs (256 x 512 x 784 NT 10.5 against 12.4 us, 256 x 10 x 256 4.3 against 6.4, 256 x 512 x 256 NN 4.8
	// against 5.0); at 2^18 the tiles win (512^3 NN 7.1 against 9.9, 256 x 784 x 512 NN 9.4 against 9.6). With op(A)
	// transposed the tiles win from 2^17 outputs (256 x 512 x 256 TN 4.7 against 5.5), the 1 x 2 lane block keeps the
	// smaller ones (10 x 256 x 256 TN 6.8 against 7.5).
	const double outputs = (double)g.m * (double)g.n * (double)g.batch_count;
	if (g.k < 256) return false;
	if (g.ta) return outputs <= 65536.0;
	return outputs <= 131072.0;
}

hipError_t gemm_valu_launch(const GemmCall& g, int shape, hipStream_t s) {
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
	p.batch_count = (int)g.batch_count;
	p.batch = g.batch;
	p.ep = g.ep;
	p.pieces = 1;
	// 16-byte loads: leading dimensions, batch strides and bases 16-byte aligned, and each operand's contiguous
	// extent (k for a k-contiguous one, else m or n) a multiple of 4
	bool vec_ok = (g.lda % 4 == 0) && (g.ldb % 4 == 0) && reinterpret_cast<uintptr_t>(g.a) % 16 == 0 &&
	              reinterpret_cast<uintptr_t>(g.b) % 16 == 0 && (g.ta ? g.m : g.k) % 4 == 0 &&
	              (g.tb ? g.k : g.n) % 4 == 0;
	for (int d = 0; d < g.batch.ndim; ++d) vec_ok = vec_ok && g.batch.sa[d] % 4 == 0 && g.batch.sb[d] % 4 == 0;
	p.vec_ok = vec_ok ? 1 : 0;
	if (shape < 0 || shape >= kValuShapes) return hipErrorInvalidValue;
	const int rm = kShapes[shape].rm, rn = kShapes[shape].rn, vc = kShapes[shape].vc;
	const bool bc = rn == 0;
	const int tile_m = 16 * rm, tile_n = bc ? 16 : 16 * rn;
	p.tiles_m = (int)((g.m + tile_m - 1) / tile_m);
	p.tiles_n = (int)((g.n + tile_n - 1) / tile_n);
	const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n * g.batch_count;
	if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
	const ValuFn fn = vec_ok ? valu_pick<true>(shape, g.ta, g.tb) : valu_pick<false>(shape, g.ta, g.tb);
	if (bc) {  // static LDS
		hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(256), 0, s, p);
		return hipGetLastError();
	}
	const size_t lds = (size_t)2 * (16 * rm + 16 * rn) * (vc + 4) * sizeof(float);
	hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
	                                   (int)lds);
	if (e != hipSuccess) return e;
	hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(256), lds, s, p);
	return hipGetLastError();
}

bool valu_pieces_ok(const GemmCall& g) {
	if (g.gather || g.rowsum || g.m <= 0 || g.n <= 0 || g.k <= 0) return false;
	if (g.m >= (1 << 30) || g.n >= (1 << 30) || g.k > kPcMaxK) return false;
	const CutPlan plan = cut_plan(g.m, g.n, g.k);
	if (plan.pieces < 2 || plan.pieces > kPcMaxPieces || plan.piece_k % 16 != 0 || plan.piece_k > 16 * kPcMaxBlocks)
		return false;
	return (double)g.m * (double)g.n * (double)g.batch_count <= (double)kPcMaxOutputs;
}

bool valu_pieces_takes(const GemmCall& g) {
	// Measured against the MFMA pieces kernel (device time, one MI355X, the kernel forced as configuration 18):
	// * four pieces in a lane: config 2's 256 x 256 x 512 NT layer 1 us faster (the MLP forward 23.6 -> 22.5 us);
	// * five to eight pieces split over the waves: transformer_tiny's weight gradients 64 x 64 x 1024 TN 8.4 against
	//   9.0 us, 256 x 64 x 1024 and 64 x 256 x 1024 TN 8.6 against 9.2, 64 x 64 x 1024 NN 7.1 against 8.9,
	//   128 x 128 x 768 TN 7.9 against 8.9 (eight pieces in one lane had been slower: 16.3 us);
	// * up to four pieces with op(A) transposed (strided dword loads) stay on the MFMA kernel.
	if (!valu_pieces_ok(g)) return false;
	const int64_t pieces = cut_plan(g.m, g.n, g.k).pieces;
	return pieces > 4 || !g.ta;
}

template <int NP, bool VEC, bool SPLIT>
ValuFn valu_pieces_fn(int ta, int tb) {
	if (!ta && !tb) return sgemm_valu_pieces_kernel<false, false, NP, VEC, SPLIT>;
	if (!ta && tb) return sgemm_valu_pieces_kernel<false, true, NP, VEC, SPLIT>;
	if (ta && !tb) return sgemm_valu_pieces_kernel<true, false, NP, VEC, SPLIT>;
	return sgemm_valu_pieces_kernel<true, true, NP, VEC, SPLIT>;
}

// up to four pieces in one lane; five to eight split over the waves, two per lane
template <bool VEC>
ValuFn valu_pieces_pick(int pieces, int ta, int tb) {
	return pieces <= 4 ? valu_pieces_fn<4, VEC, false>(ta, tb) : valu_pieces_fn<2, VEC, true>(ta, tb);
}

hipError_t gemm_valu_pieces_launch(const GemmCall& g, hipStream_t s) {
	if (!valu_pieces_ok(g)) return hipErrorInvalidValue;
	const CutPlan plan = cut_plan(g.m, g.n, g.k);
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
	p.batch_count = (int)g.batch_count;
	p.batch = g.batch;
	p.ep = g.ep;
	p.pieces = (int)plan.pieces;
	p.piece_k = (int)plan.piece_k;
	const bool split = p.pieces > 4;
	p.tiles_m = (int)((g.m + (split ? 3 : 15)) / (split ? 4 : 16));
	p.tiles_n = (int)((g.n + 15) / 16);
	const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n * g.batch_count;
	if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
	// 16-byte staging of op(B): its contiguous extent (k for a transposed B, else n) a multiple of 4, ldb, the base
	// and the batch strides 16-byte aligned
	bool vec = g.ldb % 4 == 0 && reinterpret_cast<uintptr_t>(g.b) % 16 == 0 && (g.tb ? g.k : g.n) % 4 == 0;
	for (int d = 0; d < g.batch.ndim; ++d) vec = vec && g.batch.sb[d] % 4 == 0;
	const ValuFn fn =
	    vec ? valu_pieces_pick<true>(p.pieces, g.ta, g.tb) : valu_pieces_pick<false>(p.pieces, g.ta, g.tb);
	const size_t lds = ((size_t)16 * pc_pitch(p.k) + (split ? (size_t)p.pieces * 64 : 0)) * sizeof(float);
	hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
	                                   (int)lds);
	if (e != hipSuccess) return e;
	hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(256), lds, s, p);
	return hipGetLastError();
}

}  // namespace nnh
