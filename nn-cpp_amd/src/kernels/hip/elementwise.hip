// elementwise.hip - the transformer's element-wise ops around the GEMMs: add with a broadcast right operand, mul
// (Dropout's mask), GELU (tanh form) forward and backward, embedding lookup and its gradient
// (src/autograd/ops.cpp:331-357, 451-481, 1991-2015).
//
// GELU's tanh is nn-cpp's own (gelu_math.hpp), each element with the reference's bits (its 8-lane AVX2 form gives
// the scalar form's bits per lane).
#include "elementwise.hpp"
#include "gelu_math.hpp"

#include <cmath>

namespace nnh {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
using namespace gelu_math;

__global__ void __launch_bounds__(256) add_bcast_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                        int64_t total, int64_t inner, float* __restrict__ y) {
	const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (i >= total) return;
	y[i] = a[i] + b[i % inner];
}

__global__ void __launch_bounds__(256) add_bcast4_kernel(const f32x4* __restrict__ a, const f32x4* __restrict__ b,
                                                         int64_t total4, int64_t inner4, f32x4* __restrict__ y) {
	const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (i >= total4) return;
	const f32x4 u = a[i], v = b[i % inner4];
	y[i] = f32x4{u[0] + v[0], u[1] + v[1], u[2] + v[2], u[3] + v[3]};
}

// ops.cpp:461-466: th = k (x + c x x x), tanh in place, y = 0.5 x (1 + th); th is kept for the backward pass.
__global__ void __launch_bounds__(256) gelu_forward_kernel(const float* __restrict__ x, int64_t count,
                                                           float* __restrict__ y, float* __restrict__ th) {
	const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (i >= count) return;
	float t;
	y[i] = gelu_one(x[i], t);
	th[i] = t;
}

// ops.cpp:467-480: dx (first: term + 0, else +=) with term = g (0.5 (1 + t) + 0.5 v (1 - t t) k (1 + 3 c v v)).
__global__ void __launch_bounds__(256) gelu_backward_kernel(const float* __restrict__ x, const float* __restrict__ th,
                                                            const float* __restrict__ g, int64_t count,
                                                            float* __restrict__ dx, int first) {
	const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (i >= count) return;
	const float v = x[i], t = th[i];
	const float term = g[i] * (0.5f * (1.0f + t) + 0.5f * v * (1.0f - t * t) * kGeluK * (1.0f + 3.0f * kGeluC * v * v));
	dx[i] = first ? term + 0.0f : dx[i] + term;
}

// ops.cpp:2006-2007: out row i = weight row rows[i] (rows clamped into the table; the caller validates them).
// add (optional): add(embedding, addend) with the addend's rows broadcast over the ids (ops.cpp:333-336), row i
// taking addend row i % add_rows: out = w[row] + addend, the add's bits.
__global__ void __launch_bounds__(256) embedding_forward_kernel(const float* __restrict__ w, int64_t V, int64_t D,
                                                                const int* __restrict__ rows, int64_t count,
                                                                float* __restrict__ out, const float* __restrict__ add,
                                                                int64_t add_rows) {
	const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (e >= count * D) return;
	const int64_t i = e / D, d = e - i * D;
	const int64_t r = min<int64_t>(max(rows[i], 0), V - 1);
	const float v = w[r * D + d];
	out[e] = add ? v + add[(i % add_rows) * D + d] : v;
}

// ops.cpp:2008-2014: the gradient table (first: zeros) gets, for i in order, the output gradient's row i added to
// row rows[i]. Gather form, no atomics: a wave owns one table row and 64 of its columns (a lane per column). The
// workgroup stages 1024 ids at a time in LDS; a wave finds its row's tokens among them (16 ballots) and lists them in
// token order in its own LDS list, then walks the list sixteen tokens at a time: sixteen independent loads of the
// gradient rows, then sixteen ordered adds, so the usual handful of tokens a row costs one load latency.
constexpr int kEmbIds = 1024, kEmbBatch = 16;

__global__ void __launch_bounds__(256) embedding_backward_kernel(const float* __restrict__ g, const int* __restrict__ rows,
                                                                 int64_t count, int64_t V, int64_t D,
                                                                 float* __restrict__ dw, int first) {
	__shared__ int ids[kEmbIds];
	__shared__ int list[4][kEmbIds];
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int64_t dchunks = (D + 63) / 64;
	const int64_t item = (int64_t)blockIdx.x * 4 + wave;  // (row, 64-column chunk)
	const bool here = item < V * dchunks;                  // wave-uniform
	const int64_t v = here ? item / dchunks : 0;
	const int64_t d = (here ? item - v * dchunks : 0) * 64 + lane;
	const bool on = here && d < D;
	float acc = (first || !on) ? 0.0f : dw[v * D + d];
	int* const mine = list[wave];
	for (int64_t i0 = 0; i0 < count; i0 += kEmbIds) {
		const int n = (int)min<int64_t>(kEmbIds, count - i0);
		__syncthreads();
		for (int t = threadIdx.x; t < n; t += 256) ids[t] = rows[i0 + t];
		__syncthreads();
		if (!here) continue;
		// this row's tokens of the chunk, in order
		int nm = 0;
		for (int w0 = 0; w0 < n; w0 += 64) {
			const int t = w0 + lane;
			const bool hit = t < n && ids[t] == (int)v;
			const uint64_t mk = __ballot(hit);
			if (hit) mine[nm + __builtin_amdgcn_mbcnt_hi((unsigned)(mk >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)mk, 0))] = t;
			nm += __builtin_popcountll(mk);
		}
		__builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
		__builtin_amdgcn_wave_barrier();
		__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
		for (int b0 = 0; b0 < nm; b0 += kEmbBatch) {
			float x[kEmbBatch];
#pragma unroll
			for (int j = 0; j < kEmbBatch; ++j) {  // a clamped address for empty slots and idle lanes: no branch
				const int tk = mine[min(b0 + j, nm - 1)];
				x[j] = g[on ? (i0 + tk) * D + d : 0];
			}
#pragma unroll
			for (int j = 0; j < kEmbBatch; ++j) acc = b0 + j < nm ? acc + x[j] : acc;
		}
	}
	if (on) dw[v * D + d] = acc;
}

// nn::mul (tensor.cpp:551-553): y = a * b, element by element
__global__ void __launch_bounds__(256) mul_kernel(const float* __restrict__ a, const float* __restrict__ b, int64_t count,
                                                  float* __restrict__ y) {
	const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (i < count) y[i] = a[i] * b[i];
}

// mul's backward term for one operand (ops.cpp:347-357 through accumulate_grad): t = g * other, stored as t + 0 into a
// fresh gradient, else added
__global__ void __launch_bounds__(256) mul_grad_kernel(const float* __restrict__ g, const float* __restrict__ other,
                                                       int64_t count, float* __restrict__ d, int first) {
	const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (i >= count) return;
	const float t = g[i] * other[i];
	d[i] = first ? t + 0.0f : d[i] + t;
}

inline unsigned blocks_of(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

hipError_t add_bcast(const float* a, const float* b, int64_t outer, int64_t inner, float* y, hipStream_t s) {
	const int64_t total = outer * inner;
	if (total == 0) return hipSuccess;
	if (inner % 4 == 0 && reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0 &&
	    reinterpret_cast<uintptr_t>(y) % 16 == 0)
		hipLaunchKernelGGL(add_bcast4_kernel, dim3(blocks_of(total / 4)), dim3(256), 0, s,
		                   reinterpret_cast<const f32x4*>(a), reinterpret_cast<const f32x4*>(b), total / 4, inner / 4,
		                   reinterpret_cast<f32x4*>(y));
	else
		hipLaunchKernelGGL(add_bcast_kernel, dim3(blocks_of(total)), dim3(256), 0, s, a, b, total, inner, y);
	return hipGetLastError();
}

hipError_t mul(const float* a, const float* b, int64_t count, float* y, hipStream_t s) {
	if (count == 0) return hipSuccess;
	hipLaunchKernelGGL(mul_kernel, dim3(blocks_of(count)), dim3(256), 0, s, a, b, count, y);
	return hipGetLastError();
}

hipError_t mul_grad(const float* g, const float* other, int64_t count, float* d, int first, hipStream_t s) {
	if (count == 0) return hipSuccess;
	hipLaunchKernelGGL(mul_grad_kernel, dim3(blocks_of(count)), dim3(256), 0, s, g, other, count, d, first);
	return hipGetLastError();
}

hipError_t gelu_forward(const float* x, int64_t count, float* y, float* th, hipStream_t s) {
	if (count == 0) return hipSuccess;
	hipLaunchKernelGGL(gelu_forward_kernel, dim3(blocks_of(count)), dim3(256), 0, s, x, count, y, th);
	return hipGetLastError();
}

hipError_t gelu_backward(const float* x, const float* th, const float* g, int64_t count, float* dx, int first,
                         hipStream_t s) {
	if (count == 0) return hipSuccess;
	hipLaunchKernelGGL(gelu_backward_kernel, dim3(blocks_of(count)), dim3(256), 0, s, x, th, g, count, dx, first);
	return hipGetLastError();
}

hipError_t embedding_forward(const float* w, int64_t V, int64_t D, const int* rows, int64_t count, float* out,
                             hipStream_t s, const float* add, int64_t add_rows) {
	if (count * D == 0) return hipSuccess;
	hipLaunchKernelGGL(embedding_forward_kernel, dim3(blocks_of(count * D)), dim3(256), 0, s, w, V, D, rows, count, out,
	                   add, add_rows);
	return hipGetLastError();
}

hipError_t embedding_backward(const float* g, const int* rows, int64_t count, int64_t V, int64_t D, float* dw, int first,
                              hipStream_t s) {
	if (V * D == 0) return hipSuccess;
	const int64_t waves = V * ((D + 63) / 64);
	hipLaunchKernelGGL(embedding_backward_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, g, rows, count, V,
	                   D, dw, first);
	return hipGetLastError();
}

}  // namespace nnh
