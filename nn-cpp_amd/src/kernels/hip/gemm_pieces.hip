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
#include <mutex>

#include "gemm.hpp"
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

// Operand loads through buffer resources: an element outside the matrix gets an offset past the resource's end,
// which the hardware answers with 0 and no memory access. No branches around the loads, so the compiler keeps
// several slabs of them in flight and waits for each by count.
constexpr int kOob = 0x7fffffff;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const float* base) {
	return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, kOob, 0x00020000);
}

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
			if (row >= p.m) continue;
			const int64_t off = (int64_t)row * p.ldc + col;
			float y = p.accumulate ? Cp[off] + v[e] : v[e];
			if (p.ep.bias_mode == kBiasCol) y = y + p.ep.bias[col];
			else if (p.ep.bias_mode == kBiasRow) y = y + p.ep.bias[row];
			if (p.ep.relu) {
				const bool on = y > 0.0f;
				if (alive) alive[off] = on ? 1 : 0;
				y = on ? y : 0.0f;
			}
			Cp[off] = y;
		}
	}
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

}  // namespace nnh
