// softmax.hip - the attention row softmax and its backward, with nn-cpp's exact operation order.
//
// masked_softmax_row (src/autograd/ops.cpp:1183-1204), per row i of length Tk:
//   v_j = s_j * scale; padded key -> -1e9; causal j > i -> -2e9
//   m = v_0, then m = (m < v_j) ? v_j : m       (std::max)
//   p_j = exp(v_j - m) for j < live (live = i + 1 when causal), exactly 0 beyond
//   sum = ((0 + p_0) + p_1) + ...  in j order;  p_j = p_j / sum
// The elementwise steps run on every lane; the two order-sensitive steps (the max scan and the sum) run
// one thread per row over the row held in LDS, so the bits match the reference's serial loops.
#include "softmax.hpp"

#include <math.h>

namespace nnh {

// The correctly rounded e^x for the softmax's arguments (x <= 0 or NaN): exp in double, rounded once to float.
// An exhaustive scan of every float in [-104.5, 0] (tests/golden/exp_scan.c, quad precision) finds exactly
// four inputs whose e^x lies within 8 double ulps of a float rounding midpoint, where the last bits of a
// double exp could decide the rounding; their correctly rounded results are given directly. Every other
// input lies farther than 8 ulps from a midpoint, so any double exp accurate to a few ulps rounds right.
// (nn-cpp's std::exp is glibc's expf, which is within 0.502 ulp and differs from this on 97052 of those
// 1.12e9 inputs, always by one ulp; that is the only arithmetic difference of the attention path.)
__device__ __forceinline__ float exp_ref(float x) {
	switch (__float_as_uint(x)) {
		case 0xb3000000u: return __uint_as_float(0x3f800000u);  // -0x1p-25       -> 1
		case 0xbae0e25cu: return __uint_as_float(0x3f7f8fa7u);  // -0x1.c1c4b8p-10 -> 0x1.ff1f4ep-1
		case 0xbbf0edf1u: return __uint_as_float(0x3f7e1fe9u);  // -0x1.e1dbe2p-8  -> 0x1.fc3fd2p-1
		case 0xc16912cdu: return __uint_as_float(0x34fd331bu);  // -0x1.d2259ap+3  -> 0x1.fa6636p-22
		default: return (float)exp((double)x);
	}
}

namespace {

constexpr int kThreads = 256;

struct RowGeom {
	int64_t rows;     // total rows
	int tk;           // row length
	int tq;           // rows per (sample, head): row r has query index i = r % tq
	int heads;        // sample of row r: n = r / (heads * tq)
	float scale;
	const float* pad; // {N, Tk} key padding mask (0 marks a padded key) or null
	int causal;
};

__device__ __forceinline__ float masked_value(float s, const RowGeom& g, const float* ph, int64_t i, int j) {
	float v = s * g.scale;
	if (ph && ph[j] == 0.0f) v = -1e9f;
	if (g.causal && j > i) v = -2e9f;
	return v;
}

// rb rows per block (dynamic), row stride tk + 1 in LDS (odd: a thread walking its own row and its
// neighbours walking theirs hit different banks).
__global__ void __launch_bounds__(kThreads) softmax_rows_kernel(const float* in, float* out, RowGeom g, int rb) {
	extern __shared__ float sm[];
	const int tid = threadIdx.x;
	const int64_t r0 = (int64_t)blockIdx.x * rb;
	const int nr = (int)min<int64_t>(rb, g.rows - r0);
	const int ld = g.tk + 1;
	float* rowmax = sm + rb * ld;
	float* rowsum = rowmax + rb;
	// A: load, scale and mask
	for (int e = tid; e < nr * g.tk; e += kThreads) {
		const int r = e / g.tk, j = e % g.tk;
		const int64_t row = r0 + r;
		const int64_t i = row % g.tq;
		const float* ph = g.pad ? g.pad + (row / ((int64_t)g.heads * g.tq)) * g.tk : nullptr;
		sm[r * ld + j] = masked_value(in[row * g.tk + j], g, ph, i, j);
	}
	__syncthreads();
	// B: the max scan, one thread per row
	if (tid < nr) {
		const float* o = sm + tid * ld;
		float m = o[0];
		for (int j = 1; j < g.tk; ++j) {
			const float v = o[j];
			m = (m < v) ? v : m;
		}
		rowmax[tid] = m;
	}
	__syncthreads();
	// C: exponentials (exact zeros past the causal limit)
	for (int e = tid; e < nr * g.tk; e += kThreads) {
		const int r = e / g.tk, j = e % g.tk;
		const int64_t i = (r0 + r) % g.tq;
		const int live = g.causal ? (int)min<int64_t>(g.tk, i + 1) : g.tk;
		float* p = sm + r * ld + j;
		*p = (j < live) ? exp_ref(*p - rowmax[r]) : 0.0f;
	}
	__syncthreads();
	// D: the sum in j order, one thread per row
	if (tid < nr) {
		const float* o = sm + tid * ld;
		const int64_t i = (r0 + tid) % g.tq;
		const int live = g.causal ? (int)min<int64_t>(g.tk, i + 1) : g.tk;
		float s = 0.0f;
		for (int j = 0; j < live; ++j) s += o[j];
		rowsum[tid] = s;
	}
	__syncthreads();
	// E: normalise and store
	for (int e = tid; e < nr * g.tk; e += kThreads) {
		const int r = e / g.tk, j = e % g.tk;
		out[(r0 + r) * g.tk + j] = sm[r * ld + j] / rowsum[r];
	}
}

// Backward of the row softmax (ops.cpp:1216-1224 in attention, 1323-1342 standalone):
//   dot = sum_j g_j * y_j (product rounded, then added, in j order)
//   term_j = scale * (y_j * (g_j - dot))
// mode 0 (attention): out_j = masked ? 0 : term_j + 0.0f
// mode 1 (standalone, fresh gradient): same as mode 0
// mode 2 (standalone, accumulate): out_j += term_j where not masked
__global__ void __launch_bounds__(kThreads) softmax_backward_rows_kernel(const float* y, const float* gin, float* out,
                                                                         RowGeom g, int rb, int mode) {
	extern __shared__ float sm[];
	const int tid = threadIdx.x;
	const int64_t r0 = (int64_t)blockIdx.x * rb;
	const int nr = (int)min<int64_t>(rb, g.rows - r0);
	const int ld = g.tk + 1;
	float* sy = sm;
	float* sg = sm + rb * ld;
	float* dot = sg + rb * ld;
	for (int e = tid; e < nr * g.tk; e += kThreads) {
		const int r = e / g.tk, j = e % g.tk;
		sy[r * ld + j] = y[(r0 + r) * g.tk + j];
		sg[r * ld + j] = gin[(r0 + r) * g.tk + j];
	}
	__syncthreads();
	if (tid < nr) {
		float d = 0.0f;
		for (int j = 0; j < g.tk; ++j) {
			const float t = sg[tid * ld + j] * sy[tid * ld + j];
			d = d + t;
		}
		dot[tid] = d;
	}
	__syncthreads();
	for (int e = tid; e < nr * g.tk; e += kThreads) {
		const int r = e / g.tk, j = e % g.tk;
		const int64_t row = r0 + r;
		const int64_t i = row % g.tq;
		const float* ph = g.pad ? g.pad + (row / ((int64_t)g.heads * g.tq)) * g.tk : nullptr;
		const bool masked = (ph && ph[j] == 0.0f) || (g.causal && j > i);
		const float term = g.scale * (sy[r * ld + j] * (sg[r * ld + j] - dot[r]));
		float* o = out + row * g.tk + j;
		if (mode == 2) {
			if (!masked) *o = *o + term;
		} else {
			*o = masked ? 0.0f : term + 0.0f;
		}
	}
}

constexpr int kMaxLdsBytes = 160 * 1024;

int rows_per_block(int tk, int arrays) {
	// arrays row buffers of (tk + 1) floats plus 2 per-row scalars, within the CU's LDS
	const int per_row = (arrays * (tk + 1) + 2) * 4;
	int rb = 64;
	while (rb > 1 && rb * per_row > kMaxLdsBytes / 2) rb /= 2;  // leave room for two blocks per CU
	if (rb * per_row > kMaxLdsBytes) return 0;
	return rb;
}

hipError_t set_lds_limit(const void* fn, int bytes) {
	return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

}  // namespace

hipError_t softmax_rows(const float* in, float* out, int64_t rows, int tk, int tq, int heads, float scale,
                        const float* pad, int causal, hipStream_t s) {
	if (rows == 0 || tk == 0) return hipSuccess;
	const int rb = rows_per_block(tk, 1);
	if (rb == 0) return hipErrorInvalidValue;
	RowGeom g{rows, tk, tq, heads, scale, pad, causal};
	const int lds = (rb * (tk + 1) + 2 * rb) * 4;
	hipError_t e = set_lds_limit(reinterpret_cast<const void*>(softmax_rows_kernel), lds);
	if (e != hipSuccess) return e;
	hipLaunchKernelGGL(softmax_rows_kernel, dim3((unsigned)((rows + rb - 1) / rb)), dim3(kThreads), lds, s, in, out,
	                   g, rb);
	return hipGetLastError();
}

hipError_t softmax_backward_rows(const float* y, const float* g_in, float* out, int64_t rows, int tk, int tq,
                                 int heads, float scale, const float* pad, int causal, int mode, hipStream_t s) {
	if (rows == 0 || tk == 0) return hipSuccess;
	const int rb = rows_per_block(tk, 2);
	if (rb == 0) return hipErrorInvalidValue;
	RowGeom g{rows, tk, tq, heads, scale, pad, causal};
	const int lds = (2 * rb * (tk + 1) + rb) * 4;
	hipError_t e = set_lds_limit(reinterpret_cast<const void*>(softmax_backward_rows_kernel), lds);
	if (e != hipSuccess) return e;
	hipLaunchKernelGGL(softmax_backward_rows_kernel, dim3((unsigned)((rows + rb - 1) / rb)), dim3(kThreads), lds, s, y,
	                   g_in, out, g, rb, mode);
	return hipGetLastError();
}

int softmax_max_row_length() {
	int tk = 1;
	while (rows_per_block(tk * 2, 2) > 0) tk *= 2;
	int lo = tk, hi = tk * 2;
	while (hi - lo > 1) {
		const int mid = (lo + hi) / 2;
		if (rows_per_block(mid, 2) > 0) lo = mid;
		else hi = mid;
	}
	return lo;
}

}  // namespace nnh
