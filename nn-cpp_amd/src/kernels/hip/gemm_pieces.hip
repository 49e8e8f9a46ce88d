// gemm_pieces.hip - products that take a depth cut (cut_plan in gemm.hpp; nn-cpp's blocked(),
// src/kernels/gemm.cpp:453-485, for nn-cpp's own rule) in one launch, without partial sums in HBM.
//
// A cut product's depth is split into `pieces` slices of piece_k depth indices; each piece is a chain from +0,
// the pieces are added in order (acc = piece 0, acc += piece 1, ...) and acc is stored, or added to C.
//
// One workgroup owns a 32 x 32 tile of C (of one batch matrix) and one wave per piece (at most 16, so a SIMD
// holds up to four independent chains). A piece is one 16x16x1 MFMA chain whose 4 blocks are the tile's four
// 16 x 16 quarters, one MFMA per depth index in order. Operands stream through 32-deep slabs (a slab row is one
// whole 128-byte line of a k-contiguous operand): the next slab's loads are in flight while the current one is
// consumed from the wave's own LDS staging, and no load is issued past a piece's last slab (the CU's address unit
// is shared by all 16 waves). Past a piece's end A is +0 and B is -0: fma(+0, -0, acc) = acc + (-0) = acc exactly,
// -0 included (a chain from +0 ends at -0 when its products round to -0). A finished piece goes to an LDS slot;
// after a barrier each thread adds the pieces in
// piece order for its outputs, and the store applies accumulate, bias and ReLU as the reference's does.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "gemm.hpp"
#include "gemm_direct.hpp"
#include "gemm_tile.hpp"

namespace nnh {

namespace {

constexpr int kT = 32;             // output tile side
constexpr int kMaxPieces = 16;     // = waves per workgroup at most
constexpr int kKC = 32;            // depth of one slab
constexpr int kSlab = kT * kKC;    // floats of one operand's slab
constexpr int kPerWave = 2 * kSlab;  // staging of A and B; then the finished piece
using U = Mfma<kMf16>;
static_assert(kT * kT <= kPerWave, "a finished piece fits in the staging");

// A slab of a k-contiguous operand is 32 rows of 8 16-byte chunks (depth 4 c .. 4 c + 3); chunk c of row r is
// stored at 16-byte slot 8 r + (c ^ ((r / 2) % 8)), so that 16 lanes reading one chunk of rows 0..15, and 16 lanes
// writing the 8 chunks of two rows, touch 16 distinct 4-bank groups. An m- or n-contiguous slab is [k][32], read
// one float per lane (consecutive lanes, consecutive banks).
__device__ __forceinline__ int kslot(int r, int c) { return 8 * r + (c ^ ((r >> 1) & 7)); }


// Four elements of a row-major matrix whose element (0, 0) is the resource's base: row r, columns c .. c + 3,
// 0 outside rows_valid x cols_valid (-0 with NEG: the B operand's fill, so that a step past a piece's end
// multiplies +0 by -0 and adding that -0 product leaves every sum as it was, a piece that ended at -0 included).
// VEC: the caller guarantees that c < cols_valid implies c + 3 < cols_valid and 16-byte alignment, so one
// 16-byte load serves.
template <bool VEC, bool NEG>
__device__ __forceinline__ f32x4 load4(__amdgpu_buffer_rsrc_t res, int ld, int r, int c, int rows_valid, int cols_valid) {
	constexpr unsigned kSign = NEG ? 0x80000000u : 0u;
	if (VEC) {
		const bool in = r < rows_valid && c < cols_valid;
		const int off = in ? (r * ld + c) * 4 : kOob;
		f32x4 v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(res, off, 0, 0));
		if (NEG) {
#pragma unroll
			for (int e = 0; e < 4; ++e) v[e] = in ? v[e] : __builtin_bit_cast(float, kSign);
		}
		return v;
	}
	f32x4 v;
#pragma unroll
	for (int e = 0; e < 4; ++e) {
		const bool in = r < rows_valid && c + e < cols_valid;
		const int off = in ? (r * ld + c + e) * 4 : kOob;
		v[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(res, off, 0, 0));
		if (NEG) v[e] = in ? v[e] : __builtin_bit_cast(float, kSign);
	}
	return v;
}

// Makes the wave's LDS writes visible to all its lanes before the reads that follow, and keeps the compiler from
// moving LDS accesses across it. Staging is private to a wave until the final barrier.
__device__ __forceinline__ void wave_lds_sync() {
	__builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
	__builtin_amdgcn_wave_barrier();
	__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The store of one finished output (gemm.cpp:481-484) and the op's bias and ReLU (src/autograd/ops.cpp:726-730,
// 1396-1409): v is the sum of the pieces; accumulate adds it to the old C.
__device__ __forceinline__ void put_output(const GemmArgs& p, float* __restrict__ Cp, unsigned char* alive, int row,
                                           int col, float v) {
	const int64_t off = (int64_t)row * p.ldc + col;
	float y = p.accumulate ? Cp[off] + v : v;
	if (p.ep.bias_mode == kBiasCol) y = y + p.ep.bias[col];
	else if (p.ep.bias_mode == kBiasRow) y = y + p.ep.bias[row];
	if (p.ep.res) y = p.ep.res[(Cp - p.c) + off] + y;
	if (p.ep.relu) {
		const bool on = y > 0.0f;
		if (alive) alive[off] = on ? 1 : 0;
		y = on ? y : 0.0f;
	}
	Cp[off] = y;
}

template <bool TA, bool TB, bool VEC>
__global__ void __launch_bounds__(kMaxPieces * 64) sgemm_pieces_kernel(const GemmArgs p) {
	extern __shared__ __align__(16) float lds[];
	// the wave index is uniform across the wave: said so, the resources built from it stay in scalar registers
	const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
	const int nthreads = blockDim.x;
	const int tiles = p.tiles_m * p.tiles_n;
	const int lid = xcd_remap((int)blockIdx.x, tiles * p.batch_count);
	const int t = lid % tiles, bi = lid / tiles;
	const int m0 = (t / p.tiles_n) * kT, n0 = (t % p.tiles_n) * kT;
	int64_t oa = 0, ob = 0, oc = 0;
	if (p.batch.ndim > 0) batch_offsets(p.batch, bi, oa, ob, oc);
	const float* __restrict__ A = p.a + oa;
	const float* __restrict__ B = p.b + ob;
	const int mv = p.m - m0, nv = p.n - n0;
	const int lda = (int)p.lda, ldb = (int)p.ldb;
	float* const As = lds + wave * kPerWave;
	float* const Bs = As + kSlab;

	// this wave's piece: depth indices [k_lo, k_hi) in nslab slabs
	const int k_lo = wave * p.piece_k, k_hi = min(p.k, k_lo + p.piece_k);
	const int nslab = (k_hi - k_lo + kKC - 1) / kKC;

	// slab s's operands into registers: A 32 x 32 and B 32 x 32, four 16-byte slots each per lane; a slab past the
	// piece's end loads zeros without touching memory
	f32x4 ra[4], rb[4];
	auto load = [&](int s, f32x4 (&a)[4], f32x4 (&b)[4]) {
		const int k0 = s < nslab ? k_lo + s * kKC : 0;
		const int kv = s < nslab ? k_hi - k0 : 0;
		const __amdgpu_buffer_rsrc_t ares = rsrc(TA ? A + (int64_t)k0 * lda + m0 : A + (int64_t)m0 * lda + k0);
		const __amdgpu_buffer_rsrc_t bres = rsrc(TB ? B + (int64_t)n0 * ldb + k0 : B + (int64_t)k0 * ldb + n0);
#pragma unroll
		for (int i = 0; i < 4; ++i) {
			const int idx = lane + 64 * i;  // row idx / 8, columns 4 (idx % 8) .. + 3 of the 32 x 32 slab
			if (!TA) a[i] = load4<VEC, false>(ares, lda, idx >> 3, (idx & 7) * 4, mv, kv);
			else a[i] = load4<VEC, false>(ares, lda, idx >> 3, (idx & 7) * 4, kv, mv);
			if (TB) b[i] = load4<VEC, true>(bres, ldb, idx >> 3, (idx & 7) * 4, nv, kv);
			else b[i] = load4<VEC, true>(bres, ldb, idx >> 3, (idx & 7) * 4, kv, nv);
		}
	};
	auto store = [&](const f32x4 (&a)[4], const f32x4 (&b)[4]) {
#pragma unroll
		for (int i = 0; i < 4; ++i) {
			const int idx = lane + 64 * i;
			const int sk = kslot(idx >> 3, idx & 7);
			*reinterpret_cast<f32x4*>(As + 4 * (TA ? idx : sk)) = a[i];
			*reinterpret_cast<f32x4*>(Bs + 4 * (TB ? sk : idx)) = b[i];
		}
	};
	// lane group g = lane / 16 runs block g of the MFMA: A rows 16 (g / 2) + lane % 16, B columns 16 (g % 2) + lane % 16
	const int arow = 16 * ((lane >> 4) >> 1) + (lane & 15), bcol = 16 * ((lane >> 4) & 1) + (lane & 15);
	auto frag = [&](int g, f32x4& a, f32x4& b) {
		if (!TA) {
			a = *reinterpret_cast<const f32x4*>(As + 4 * kslot(arow, g));
		} else {
#pragma unroll
			for (int e = 0; e < 4; ++e) a[e] = As[(4 * g + e) * kT + arow];
		}
		if (TB) {
			b = *reinterpret_cast<const f32x4*>(Bs + 4 * kslot(bcol, g));
		} else {
#pragma unroll
			for (int e = 0; e < 4; ++e) b[e] = Bs[(4 * g + e) * kT + bcol];
		}
	};
	U::Acc acc;
#pragma unroll
	for (int r = 0; r < U::NV; ++r) acc[r] = 0.0f;
	auto mma = [&]() {
		f32x4 af[2], bf[2];
		frag(0, af[0], bf[0]);
#pragma unroll
		for (int g = 0; g < kKC / 4; ++g) {
			// the next group's operands are read while this group's four MFMAs run
			if (g + 1 < kKC / 4) frag(g + 1, af[(g + 1) & 1], bf[(g + 1) & 1]);
			__builtin_amdgcn_sched_barrier(0);
#pragma unroll
			for (int e = 0; e < 4; ++e) acc = U::mma(af[g & 1][e], bf[g & 1][e], acc);
			__builtin_amdgcn_sched_barrier(0);
		}
	};

	load(0, ra, rb);
	for (int s = 0; s < nslab; ++s) {
		store(ra, rb);
		// slab s + 1 into the registers while slab s is consumed from LDS
		if (s + 1 < nslab) load(s + 1, ra, rb);
		wave_lds_sync();
		mma();
		wave_lds_sync();
	}
	// the finished piece into the staging: 16-byte slot j holds registers 4 (j / 64) .. + 3 of lane j % 64
#pragma unroll
	for (int q = 0; q < U::NV / 4; ++q)
		*reinterpret_cast<f32x4*>(As + (q * 64 + lane) * 4) = f32x4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
	__syncthreads();

	// piece order (gemm.cpp:475-480): piece 0 is the sum, each later piece is added to it; then the store
	// (gemm.cpp:481-484) and the op's bias and ReLU (src/autograd/ops.cpp:726-730, 1396-1409)
	float* __restrict__ Cp = p.c + oc;
	unsigned char* alive = p.ep.alive ? p.ep.alive + oc : nullptr;
	for (int j = tid; j < kT * kT / 4; j += nthreads) {
		// every piece's four values read first, then added in order
		f32x4 x[kMaxPieces];
#pragma unroll
		for (int q = 0; q < kMaxPieces; ++q)
			if (q < p.pieces) x[q] = *reinterpret_cast<const f32x4*>(lds + q * kPerWave + j * 4);
		f32x4 v = x[0];
#pragma unroll
		for (int q = 1; q < kMaxPieces; ++q)
			if (q < p.pieces)
#pragma unroll
				for (int e = 0; e < 4; ++e) v[e] = v[e] + x[q][e];
		const int blk = j >> 6, l = j & 63;
		const int col = n0 + 16 * (blk & 1) + (l & 15);
		if (col >= p.n) continue;
#pragma unroll
		for (int e = 0; e < 4; ++e) {
			const int row = m0 + 16 * (blk >> 1) + 4 * (l >> 4) + e;
			if (row < p.m) put_output(p, Cp, alive, row, col, v[e]);
		}
	}
}

constexpr int kRsMaxInner = 256;  // inner indices of the two-stage row sums (stage-one results held in LDS)
constexpr int kRsSteps = 16;      // outer indices whose loads are in flight together
constexpr int kRsWaves = 2;       // row-sum waves
constexpr int kRsMaxPieces = 10;  // pieces beside them: at most 12 waves, three a SIMD, room for the loads

// The pieces of a 16 x 16 tile, parked in LDS by piece (done[q][row][column]), added in piece order and stored.
__device__ __forceinline__ void finish_tile(const GemmArgs& p, int64_t oc, int m0, int n0, int tid, int nthreads,
                                            const float* done) {
	constexpr int kU = 16;
	float* __restrict__ Cp = p.c + oc;
	unsigned char* alive = p.ep.alive ? p.ep.alive + oc : nullptr;
	for (int o = tid; o < kU * kU; o += nthreads) {
		float v = done[o];
		for (int q = 1; q < p.pieces; ++q) v = v + done[q * kU * kU + o];
		const int row = m0 + o / kU, col = n0 + o % kU;
		if (row < p.m && col < p.n) put_output(p, Cp, alive, row, col, v);
	}
}

// Two-stage row sums of op(A) = A^T for rows m0 .. m0 + 15 (columns of A, k x m with leading dimension lda), by
// kRsWaves waves: A's row index is o * r1 + i (outer o < r0, inner i < r1 = k / r0).
// Stage one (Tensor::sum(0) over the outer axis, tensor.cpp:422-456): for each inner i, s1[i] = +0 + A[i] +
// A[r1 + i] + ... in outer order, parked in LDS as part[i][16]. Lane l of row-sum wave w sums four columns
// 4 (l % 4) .. + 3 (one 16-byte load per step) for inner indices i = ib + l / 4 + 16 (2 w + u), u < 2, with
// kRsSteps outer steps of loads in flight.
// Stage two (the second sum(0)), after the workgroup's barrier: rowsum = +0 + s1[0] + s1[1] + ... in inner order,
// lane c of the first row-sum wave for row m0 + c; then the combine of GemmArgs::rowsum_combine.
// The caller guarantees m and lda multiples of 4, A 16-byte aligned, r1 <= kRsMaxInner and k lda < 2^29 (every
// byte offset into A below 2^31).
__device__ __forceinline__ void rowsums_stage1(const GemmArgs& p, const float* __restrict__ A, int m0, int lane, int w,
                                               float* part) {
	const int r0 = p.rowsum_outer, r1 = p.k / p.rowsum_outer;
	const int cq = lane & 3, il = lane >> 2;
	// a column quad past m loads the last quad instead and is never summed in stage two
	const int col = min(m0 + 4 * cq, p.m - 4);
	const __amdgpu_buffer_rsrc_t res = rsrc(A);
	for (int ib = 0; ib < r1; ib += 16 * 2 * kRsWaves) {
		// byte offsets: the inner index and column per lane, the outer index in a scalar register
		int voff[2];
#pragma unroll
		for (int u = 0; u < 2; ++u) voff[u] = (min(ib + il + 16 * (2 * w + u), r1 - 1) * (int)p.lda + col) * 4;
		f32x4 acc[2];
#pragma unroll
		for (int u = 0; u < 2; ++u) acc[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
		for (int o0 = 0; o0 < r0; o0 += kRsSteps) {
			f32x4 v[kRsSteps][2];
#pragma unroll
			for (int st = 0; st < kRsSteps; ++st) {
				const int soff = min(o0 + st, r0 - 1) * r1 * (int)p.lda * 4;
#pragma unroll
				for (int u = 0; u < 2; ++u)
					v[st][u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(res, voff[u], soff, 0));
			}
#pragma unroll
			for (int st = 0; st < kRsSteps; ++st)
				if (o0 + st < r0)
#pragma unroll
					for (int u = 0; u < 2; ++u)
#pragma unroll
						for (int e = 0; e < 4; ++e) acc[u][e] = acc[u][e] + v[st][u][e];
		}
#pragma unroll
		for (int u = 0; u < 2; ++u) {
			const int i = ib + il + 16 * (2 * w + u);
			if (i < r1) *reinterpret_cast<f32x4*>(part + i * 16 + 4 * cq) = acc[u];
		}
	}
}

__device__ __forceinline__ void rowsums_stage2(const GemmArgs& p, int m0, int lane, const float* part) {
	const int r1 = p.k / p.rowsum_outer;
	if (lane >= 16 || m0 + lane >= p.m) return;
	float s = 0.0f;
	for (int i0 = 0; i0 < r1; i0 += 16) {
		float v[16];
#pragma unroll
		for (int e = 0; e < 16; ++e) v[e] = part[min(i0 + e, r1 - 1) * 16 + lane];
#pragma unroll
		for (int e = 0; e < 16; ++e)
			if (i0 + e < r1) s = s + v[e];
	}
	float* dst = p.rowsum + m0 + lane;
	if (p.rowsum_combine == 0) *dst = s;
	else if (p.rowsum_combine == 1) *dst = s + 0.0f;
	else *dst = *dst + s;
}

// The same cut on the 16x16x4 MFMA (Mfma<kMf16x4>: one instruction advances each chain of a 16 x 16 block four
// depth steps, bit-identical to four fmaf in order). One workgroup owns a 16 x 16 tile of C and one wave per piece,
// so a product with few outputs still spreads over many CUs (a 64 x 64 output is 16 workgroups). A wave loads its
// operands straight into the instruction's lane layout, 128 depth indices at a time with all 64 loads in flight
// (lane l supplies row or column l % 16 at depth 4 s + l / 16 of step s), with no LDS staging; past the piece's end
// A is +0 and B is -0 as above. The finished pieces meet in LDS and are added in piece order.
//
// RS (A transposed, B not: a linear layer's weight gradient G^T X): two more waves in the workgroups of the first
// column tile fold the two-stage row sums of op(A) = G^T for the tile's 16 rows, the bias gradient of a
// three-dimensional G (GemmArgs::rowsum_outer), while the MFMA waves run: 16-byte loads of four columns, chains
// over the outer index per inner index parked in LDS, then, after the barrier, one chain over the inner index per
// row.

//
// One workgroup's tile (block: its index among the product's workgroups) with nthreads threads: waves 0 .. pieces - 1
// run the pieces, with RS the next kRsWaves waves the row sums, and any further waves only take part in the barrier
// and the final sums.
template <bool TA, bool TB, bool RS, bool VEC>
__device__ __forceinline__ void pieces4_tile(const GemmArgs& p, int block, int tid, int nthreads) {
	static_assert(!RS || (TA && !TB), "row sums are compiled for the weight-gradient layout only");
	constexpr int kU = 16;      // tile side
	__shared__ float done[kMaxPieces * kU * kU];
	__shared__ float part[RS ? kRsMaxInner * kU : 1];
	const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
	const int tiles = p.tiles_m * p.tiles_n;
	const int lid = xcd_remap(block, tiles * p.batch_count);
	const int t = lid % tiles, bi = lid / tiles;
	const int m0 = (t / p.tiles_n) * kU, n0 = (t % p.tiles_n) * kU;
	int64_t oa = 0, ob = 0, oc = 0;
	if (p.batch.ndim > 0) batch_offsets(p.batch, bi, oa, ob, oc);
	const float* __restrict__ A = p.a + oa;
	const float* __restrict__ B = p.b + ob;
	const int lda = (int)p.lda, ldb = (int)p.ldb;
	const int r = lane & 15, j = lane >> 4;
	if (wave >= p.pieces) {
		if (RS && n0 == 0 && wave - p.pieces < kRsWaves) rowsums_stage1(p, A, m0, lane, wave - p.pieces, part);
		__syncthreads();
		if (RS && n0 == 0 && wave == p.pieces) rowsums_stage2(p, m0, lane, part);
		finish_tile(p, oc, m0, n0, tid, nthreads, done);
		return;
	}
	const bool row_in = m0 + r < p.m, col_in = n0 + r < p.n;
	const int k_lo = wave * p.piece_k, k_hi = min(p.k, k_lo + p.piece_k);
	f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
	// one chunk of G groups of 16 depth indices: every load issued before the first MFMA. Group h holds the operands
	// of steps 4 h .. 4 h + 3. A k-contiguous operand (A not transposed, B transposed) takes, with VEC, one 16-byte
	// load per group (lane group g: depths 16 h + 4 g .. + 3 of its row), reordered through the wave's LDS slots
	// (gemm_direct.hpp); otherwise one element per lane and step. PART (fewer than 16 indices left in
	// the piece) loads element by element, masks the depth and turns B's +0 fill past the end into -0 at the MFMA.
	constexpr bool KA = VEC && !TA, KB = VEC && TB;
	// the wave's LDS slots for its k-contiguous operands (two groups each)
	__shared__ __align__(16) float kst[(KA || KB) ? kMaxPieces * 2 * 2 * kKSlot : 1];
	float* const la = kst + (KA || KB ? wave * 4 * kKSlot : 0);
	float* const lb = la + 2 * kKSlot;
	auto chunk = [&](int kc, auto groups_tag, auto part_tag) {
		constexpr int G = decltype(groups_tag)::value;
		constexpr bool PART = decltype(part_tag)::value;
		f32x4 a[G], b[G];
		load_groups<TA, TB, KA && !PART, KB && !PART, PART, G>(A, lda, B, ldb, m0, n0, kc, k_hi - kc, r, j, row_in,
		                                                       col_in, a, b);
		__builtin_amdgcn_sched_barrier(0);
		mma_groups<KA && !PART, KB && !PART, PART, G>(a, b, k_hi - kc, r, j, acc, la, lb);
		__builtin_amdgcn_sched_barrier(0);
	};
	using I1 = std::integral_constant<int, 1>;
	using I2 = std::integral_constant<int, 2>;
	using I4 = std::integral_constant<int, 4>;
	using I8 = std::integral_constant<int, 8>;
	int kc = k_lo;
	for (; k_hi - kc >= 128; kc += 128) chunk(kc, I8{}, std::false_type{});
	if (k_hi - kc >= 64) {
		chunk(kc, I4{}, std::false_type{});
		kc += 64;
	}
	if (k_hi - kc >= 32) {
		chunk(kc, I2{}, std::false_type{});
		kc += 32;
	}
	if (k_hi - kc >= 16) {
		chunk(kc, I1{}, std::false_type{});
		kc += 16;
	}
	if (kc < k_hi) chunk(kc, I1{}, std::true_type{});
	// register e of lane l holds row 4 (l / 16) + e, column l % 16 of the tile
	float* const mine = done + wave * kU * kU;
#pragma unroll
	for (int e = 0; e < 4; ++e) mine[(4 * j + e) * kU + r] = acc[e];
	__syncthreads();
	finish_tile(p, oc, m0, n0, tid, nthreads, done);
}

template <bool TA, bool TB, bool RS, bool VEC>
__global__ void __launch_bounds__(RS ? (kRsMaxPieces + kRsWaves) * 64 : kMaxPieces * 64) sgemm_pieces4_kernel(const GemmArgs p) {
	pieces4_tile<TA, TB, RS, VEC>(p, (int)blockIdx.x, (int)threadIdx.x, (int)blockDim.x);
}

// A linear layer's two backward products in one launch (nnh_linear_backward's dX = G W and dW = G^T X, with or
// without dW's two-stage row sums, db): workgroups below blocks0 take dX's 32 x 32 tiles on their first four waves
// (chain4_tile: a whole-depth product, A and B not transposed), the others dW's 16 x 16 tiles (pieces4_tile: a cut
// product, A transposed). Each output gets the chain it gets from its own kernel, so the bits are those of the two
// launches; the caller guarantees that neither product writes what the other reads or writes. The workgroup has
// max(256, pieces-tile threads) threads, at most kPairThreads.
constexpr int kPairThreads = (kRsMaxPieces + kRsWaves) * 64;

template <bool VEC0, bool RS1>
__global__ void __launch_bounds__(kPairThreads) sgemm_chain_pieces_kernel(const GemmArgs p0, const GemmArgs p1,
                                                                         int blocks0) {
	const int tid = threadIdx.x;
	if ((int)blockIdx.x < blocks0) {
		const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
		if (wave < 4) chain4_tile<false, false, VEC0>(p0, (int)blockIdx.x, wave, tid & 63);
		return;
	}
	pieces4_tile<true, false, RS1, !RS1>(p1, (int)blockIdx.x - blocks0, tid, (int)blockDim.x);
}

using PiecesFn = void (*)(const GemmArgs);

constexpr int kPerWaveBytes = kPerWave * (int)sizeof(float);

// Leading dimensions (and the dimensions that are leading dimensions of contiguous operands) the kernel's 32-bit
// offsets cover: a slab's offsets stay below 32 rows of the larger leading dimension.
constexpr int64_t kMaxLd = int64_t(1) << 24;

}  // namespace

bool pieces_kernel_takes(int64_t m, int64_t n, int64_t k, int64_t batch_count, bool gather_or_rowsum) {
	(void)batch_count;
	if (gather_or_rowsum || m >= kMaxLd || n >= kMaxLd || k >= kMaxLd) return false;
	const CutPlan c = cut_plan(m, n, k);
	return c.pieces > 1 && c.pieces <= kMaxPieces;
}

bool pieces_kernel_takes(const GemmCall& g) {
	return pieces_kernel_takes(g.m, g.n, g.k, g.batch_count, g.gather || g.rowsum) && g.lda < kMaxLd && g.ldb < kMaxLd;
}

hipError_t gemm_pieces_launch(const GemmCall& g, hipStream_t s) {
	static const PiecesFn fns[2][4] = {
	    {sgemm_pieces_kernel<false, false, false>, sgemm_pieces_kernel<false, true, false>,
	     sgemm_pieces_kernel<true, false, false>, sgemm_pieces_kernel<true, true, false>},
	    {sgemm_pieces_kernel<false, false, true>, sgemm_pieces_kernel<false, true, true>,
	     sgemm_pieces_kernel<true, false, true>, sgemm_pieces_kernel<true, true, true>}};
	constexpr int kMaxDevices = 64;
	static std::mutex mu;
	static bool ready[kMaxDevices] = {};
	int dev = 0;
	hipError_t e = hipGetDevice(&dev);
	if (e != hipSuccess) return e;
	if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
	{
		std::lock_guard<std::mutex> lock(mu);
		if (!ready[dev]) {
			for (int v = 0; v < 2; ++v)
				for (int f = 0; f < 4; ++f) {
					e = hipFuncSetAttribute(reinterpret_cast<const void*>(fns[v][f]),
					                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxPieces * kPerWaveBytes);
					if (e != hipSuccess) return e;
				}
			ready[dev] = true;
		}
	}
	if (!pieces_kernel_takes(g)) return hipErrorInvalidValue;
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
	p.tiles_m = (int)((g.m + kT - 1) / kT);
	p.tiles_n = (int)((g.n + kT - 1) / kT);
	p.batch_count = (int)g.batch_count;
	p.batch = g.batch;
	p.ep = g.ep;
	p.pieces = (int)plan.pieces;
	p.piece_k = (int)plan.piece_k;
	bool vec_ok = (g.lda % 4 == 0) && (reinterpret_cast<uintptr_t>(g.a) % 16 == 0) && (g.ldb % 4 == 0) &&
	              (reinterpret_cast<uintptr_t>(g.b) % 16 == 0);
	for (int d = 0; d < g.batch.ndim; ++d) vec_ok = vec_ok && g.batch.sa[d] % 4 == 0 && g.batch.sb[d] % 4 == 0;
	p.vec_ok = vec_ok ? 1 : 0;
	// 16-byte loads need every 4-element group of a slab row wholly inside or wholly outside the matrix: the
	// depth (the rows of a k-contiguous operand) and, for an m- or n-contiguous operand, its width a multiple of 4
	const bool vec = vec_ok && g.k % 4 == 0 && (!g.ta || g.m % 4 == 0) && (g.tb || g.n % 4 == 0);
	const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n * p.batch_count;
	if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
	const int f = (g.ta ? 2 : 0) + (g.tb ? 1 : 0);
	hipLaunchKernelGGL(fns[vec ? 1 : 0][f], dim3((unsigned)blocks), dim3(p.pieces * 64), p.pieces * kPerWaveBytes, s, p);
	return hipGetLastError();
}

// 16-byte loads of a k-contiguous operand (A not transposed, B transposed): its leading dimension and batch
// strides multiples of 4 and its base 16-byte aligned (every chunk starts at a depth that is a multiple of 4).
bool pieces4_vec(const GemmCall& g) {
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

bool pieces4_takes(const GemmCall& g) {
	// Measured (device time on one MI355X, nn-cpp's cut, against the VALU pieces kernel that took these before):
	// A transposed and B not (the weight gradient's layout) 64 x 64 x 1024 4.3 against 8.4 us, 256 x 64 x 1024 4.4
	// against 8.8, 128 x 128 x 768 4.3 against 8.1; with 16-byte loads of k-contiguous operands 256 x 256 x 512 NT
	// (config 2's second layer) 5.1 against 7.3, NN 4.5 against 7.4, 64 x 64 x 1024 NN 5.5 against 7.1, NT 6.7
	// against 6.6, 64 x 64 x 1200 TT 6.2 against 10.6, 33 x 70 x 2048 NN 10.0 against 25.9. A k-contiguous operand
	// without them (one element per lane and load) is slower than the other kernels (64 x 64 x 1024 NN 10.4, NT 16.9).
	// At most 512 tiles of 16 x 16 (every product nn-cpp cuts has at most 256): beyond, a wave per piece and tile
	// re-reads the operands too often (NUMERICS_SPLIT_DEPTH's 512 x 512 x 512 in 32-deep pieces 10.4 us, 64 x 4096 x
	// 4096 in 256-deep pieces 59 us, against 7.0 and 33 us on the kernels below).
	if (g.gather || !pieces_kernel_takes(g.m, g.n, g.k, g.batch_count, false) || g.lda >= kMaxLd || g.ldb >= kMaxLd)
		return false;
	if (((g.m + 15) / 16) * ((g.n + 15) / 16) * g.batch_count > 512) return false;
	if ((!g.ta || g.tb) && !pieces4_vec(g)) return false;
	if (!g.rowsum) return true;
	// two-stage row sums: one matrix, the row-sum waves beside at most kRsMaxPieces piece waves, 16-byte loads of A
	const CutPlan plan = cut_plan(g.m, g.n, g.k);
	return g.rowsum_outer > 0 && g.k % g.rowsum_outer == 0 && g.k / g.rowsum_outer <= kRsMaxInner &&
	       g.batch_count == 1 && plan.pieces <= kRsMaxPieces && g.m % 4 == 0 && g.lda % 4 == 0 &&
	       g.k * g.lda < (int64_t(1) << 29) &&
	       reinterpret_cast<uintptr_t>(g.a) % 16 == 0;
}

namespace {

GemmArgs pieces4_args(const GemmCall& g) {
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
	p.tiles_m = (int)((g.m + 15) / 16);
	p.tiles_n = (int)((g.n + 15) / 16);
	p.batch_count = (int)g.batch_count;
	p.batch = g.batch;
	p.ep = g.ep;
	p.pieces = (int)plan.pieces;
	p.piece_k = (int)plan.piece_k;
	p.rowsum = g.rowsum;
	p.rowsum_combine = g.rowsum_combine;
	p.rowsum_outer = (int)g.rowsum_outer;
	return p;
}

}  // namespace

hipError_t gemm_pieces4_launch(const GemmCall& g, hipStream_t s) {
	static const PiecesFn fns[2][5] = {
	    {sgemm_pieces4_kernel<false, false, false, false>, sgemm_pieces4_kernel<false, true, false, false>,
	     sgemm_pieces4_kernel<true, false, false, false>, sgemm_pieces4_kernel<true, true, false, false>,
	     sgemm_pieces4_kernel<true, false, true, false>},
	    {sgemm_pieces4_kernel<false, false, false, true>, sgemm_pieces4_kernel<false, true, false, true>,
	     sgemm_pieces4_kernel<true, false, false, true>, sgemm_pieces4_kernel<true, true, false, true>,
	     sgemm_pieces4_kernel<true, false, true, false>}};
	if (g.rowsum ? !pieces4_takes(g) : !pieces_kernel_takes(g)) return hipErrorInvalidValue;
	const GemmArgs p = pieces4_args(g);
	const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n * p.batch_count;
	if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
	const bool vec = pieces4_vec(g);
	const int f = g.rowsum ? 4 : (g.ta ? 2 : 0) + (g.tb ? 1 : 0);
	hipLaunchKernelGGL(fns[vec ? 1 : 0][f], dim3((unsigned)blocks), dim3((p.pieces + (g.rowsum ? kRsWaves : 0)) * 64), 0,
	                   s, p);
	return hipGetLastError();
}

bool chain_pieces_pair_takes(const GemmCall& g0, const GemmCall& g1) {
	if (g0.ta || g0.tb || !g1.ta || g1.tb || g0.batch_count != 1 || g1.batch_count != 1 || g0.batch.ndim != 0 ||
	    g1.batch.ndim != 0 || g0.m <= 0 || g0.n <= 0 || g1.m <= 0 || g1.n <= 0)
		return false;
	// dW on the kernel its own launch takes; dX on the chain kernel where that is its own route, or where its chains
	// are at most 256 deep (the pair runs about as long as its slower half)
	if (!depth_cut(g1.m, g1.n, g1.k) || !pieces4_takes(g1)) return false;
	if (!chain4_takes(g0) && !(chain4_ok(g0) && g0.k <= 256 && g0.m * g0.n <= (int64_t(1) << 20))) return false;
	const int threads = (int)(cut_plan(g1.m, g1.n, g1.k).pieces + (g1.rowsum ? kRsWaves : 0)) * 64;
	return threads <= kPairThreads && (int64_t)((g0.m + 31) / 32) * ((g0.n + 31) / 32) +
	                                      ((g1.m + 15) / 16) * ((g1.n + 15) / 16) <= 0x7fffffff;
}

hipError_t gemm_chain_pieces_pair_launch(const GemmCall& g0, const GemmCall& g1, hipStream_t s) {
	using PairFn = void (*)(const GemmArgs, const GemmArgs, int);
	static const PairFn fns[2][2] = {{sgemm_chain_pieces_kernel<false, false>, sgemm_chain_pieces_kernel<false, true>},
	                                 {sgemm_chain_pieces_kernel<true, false>, sgemm_chain_pieces_kernel<true, true>}};
	if (!chain_pieces_pair_takes(g0, g1)) return hipErrorInvalidValue;
	const GemmArgs p0 = chain4_args(g0), p1 = pieces4_args(g1);
	const int b0 = p0.tiles_m * p0.tiles_n, b1 = p1.tiles_m * p1.tiles_n;
	const int threads = std::max(256, (p1.pieces + (g1.rowsum ? kRsWaves : 0)) * 64);
	hipLaunchKernelGGL(fns[chain4_vec(g0) ? 1 : 0][g1.rowsum ? 1 : 0], dim3((unsigned)(b0 + b1)), dim3(threads), 0, s,
	                   p0, p1, b0);
	return hipGetLastError();
}

}  // namespace nnh
