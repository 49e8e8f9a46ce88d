// reduce.hip - memory-bound kernels around the GEMMs: column sums in the reference's fixed order
// (bias gradients), the ReLU node, and gradient stores with nn-cpp's first-write rule.
#include "reduce.hpp"

namespace nnh {

namespace {

// Tensor::sum(0) of a {rows, inner} tensor (src/tensor.cpp:422-456): a zero-filled output, then the
// rows added in order. One thread per column: consecutive threads read consecutive addresses.
// combine: 0 store s, 1 store s + 0.0f (first gradient write, ops.cpp:64-73), 2 dst += s.
__global__ void __launch_bounds__(256) sum_rows_kernel(const float* __restrict__ src, int64_t rows, int64_t inner,
                                                       float* __restrict__ dst, int combine) {
	const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (j >= inner) return;
	float s = 0.0f;
	const float* p = src + j;
	int64_t a = 0;
	// four independent loads in flight; the additions stay in row order
	for (; a + 4 <= rows; a += 4) {
		const float v0 = p[(a + 0) * inner], v1 = p[(a + 1) * inner], v2 = p[(a + 2) * inner], v3 = p[(a + 3) * inner];
		s = s + v0;
		s = s + v1;
		s = s + v2;
		s = s + v3;
	}
	for (; a < rows; ++a) s = s + p[a * inner];
	if (combine == 0) dst[j] = s;
	else if (combine == 1) dst[j] = s + 0.0f;
	else dst[j] = dst[j] + s;
}

// relu forward (ops.cpp:775-782): y = x > 0 ? x : 0
__global__ void __launch_bounds__(256) relu_forward_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                           int64_t count) {
	const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (i < count) {
		const float v = x[i];
		y[i] = v > 0.0f ? v : 0.0f;
	}
}

// relu backward (ops.cpp:783-792): term = x > 0 ? g : 0; first: dst = term + 0, else dst += term.
// x may be the forward output: y > 0 exactly where x > 0.
__global__ void __launch_bounds__(256) relu_backward_kernel(const float* __restrict__ x, const float* __restrict__ g,
                                                            float* __restrict__ dst, int64_t count, int first) {
	const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (i < count) {
		const float term = x[i] > 0.0f ? g[i] : 0.0f;
		dst[i] = first ? term + 0.0f : dst[i] + term;
	}
}

inline unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

hipError_t sum_rows(const float* src, int64_t rows, int64_t inner, float* dst, int combine, hipStream_t s) {
	if (inner == 0) return hipSuccess;
	hipLaunchKernelGGL(sum_rows_kernel, dim3(blocks_for(inner)), dim3(256), 0, s, src, rows, inner, dst, combine);
	return hipGetLastError();
}

hipError_t relu_forward(const float* x, float* y, int64_t count, hipStream_t s) {
	if (count == 0) return hipSuccess;
	hipLaunchKernelGGL(relu_forward_kernel, dim3(blocks_for(count)), dim3(256), 0, s, x, y, count);
	return hipGetLastError();
}

hipError_t relu_backward(const float* x, const float* g, float* dst, int64_t count, int first, hipStream_t s) {
	if (count == 0) return hipSuccess;
	hipLaunchKernelGGL(relu_backward_kernel, dim3(blocks_for(count)), dim3(256), 0, s, x, g, dst, count, first);
	return hipGetLastError();
}

}  // namespace nnh
