// reduce.hip - memory-bound kernels around the GEMMs: column sums in the reference's fixed order
// (bias gradients), the ReLU node, and gradient stores with nn-cpp's first-write rule.
#include "reduce.hpp"

namespace nnh {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

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

// The same sum, staged through LDS: a block owns kSumCols columns; all 256 threads load a chunk of up to
// kSumChunk rows at once (16-byte loads when the rows allow), then kSumCols lanes of the first wave add the chunk's
// rows in order onto their running sums, while the next chunk's loads are already in flight. Narrow blocks give
// many blocks (one column's chain is serial, so the parallelism is the number of columns). Same bits as
// sum_rows_kernel.
constexpr int kSumCols = 32, kSumChunk = 128;
constexpr int kSumQuads = kSumCols / 4;  // 16-byte groups per row of a block
constexpr int kSumPer = kSumCols * kSumChunk / 256;  // floats each thread loads per chunk

__device__ __forceinline__ void sum_chunk_load(const float* __restrict__ src, int rows, int inner, int c0, int ncol,
                                               int r0, int vec, float (&v)[kSumPer]) {
	const int tid = threadIdx.x;
	if (vec) {  // inner % 4 == 0 and 16-byte aligned: kSumQuads threads per row, 16 bytes each
#pragma unroll
		for (int u = 0; u < kSumPer / 4; ++u) {
			const int idx = tid + 256 * u, r = min(r0 + idx / kSumQuads, rows - 1), q = 4 * (idx % kSumQuads);
			const f32x4 x = *reinterpret_cast<const f32x4*>(src + (int64_t)r * inner + c0 + min(q, ncol - 4));
#pragma unroll
			for (int c = 0; c < 4; ++c) v[4 * u + c] = x[c];
		}
	} else {
#pragma unroll
		for (int u = 0; u < kSumPer; ++u) {
			const int idx = tid + 256 * u, r = min(r0 + idx / kSumCols, rows - 1), c = min(idx % kSumCols, ncol - 1);
			v[u] = src[(int64_t)r * inner + c0 + c];
		}
	}
}

__device__ __forceinline__ void sum_chunk_store(float (*tile)[kSumCols], int vec, const float (&v)[kSumPer]) {
	const int tid = threadIdx.x;
	if (vec) {
#pragma unroll
		for (int u = 0; u < kSumPer / 4; ++u) {
			const int idx = tid + 256 * u;
			*reinterpret_cast<f32x4*>(&tile[idx / kSumQuads][4 * (idx % kSumQuads)]) = f32x4{v[4 * u], v[4 * u + 1], v[4 * u + 2], v[4 * u + 3]};
		}
	} else {
#pragma unroll
		for (int u = 0; u < kSumPer; ++u) {
			const int idx = tid + 256 * u;
			tile[idx / kSumCols][idx % kSumCols] = v[u];
		}
	}
}

// One column sum: the source {rows, inner}, the destination and its combine rule, and whether 16-byte loads apply.
struct SumJob {
	const float* src;
	float* dst;
	int rows, inner, combine, vec;
};

// The columns block * kSumCols .. + kSumCols - 1 of one job.
__device__ __forceinline__ void sum_rows_block(const SumJob& job, int block) {
	__shared__ __align__(16) float tile[2][kSumChunk][kSumCols];
	const float* __restrict__ src = job.src;
	float* __restrict__ dst = job.dst;
	const int rows = job.rows, inner = job.inner, combine = job.combine, vec = job.vec;
	const int tid = threadIdx.x;
	const int c0 = block * kSumCols;
	const int ncol = min(kSumCols, inner - c0);
	// 16-byte loads need whole quads of columns in this block (the clamp above keeps them in the row)
	const int vec_here = vec && ncol % 4 == 0;
	float s = 0.0f;
	float v[kSumPer];
	if (rows > 0) {
		sum_chunk_load(src, rows, inner, c0, ncol, 0, vec_here, v);
		sum_chunk_store(tile[0], vec_here, v);
	}
	__syncthreads();
	for (int r0 = 0, b = 0; r0 < rows; r0 += kSumChunk, b ^= 1) {
		const bool next = r0 + kSumChunk < rows;
		if (next) sum_chunk_load(src, rows, inner, c0, ncol, r0 + kSumChunk, vec_here, v);  // in flight meanwhile
		if (tid < ncol) {
			const int nr = min(kSumChunk, rows - r0);
			int r = 0;
			for (; r + 16 <= nr; r += 16) {  // sixteen LDS reads ahead of the dependent additions
				float x[16];
#pragma unroll
				for (int u = 0; u < 16; ++u) x[u] = tile[b][r + u][tid];
#pragma unroll
				for (int u = 0; u < 16; ++u) s = s + x[u];
			}
			for (; r < nr; ++r) s = s + tile[b][r][tid];
		}
		if (next) sum_chunk_store(tile[b ^ 1], vec_here, v);
		__syncthreads();
	}
	if (tid < ncol) {
		float* d = dst + c0 + tid;
		if (combine == 0) *d = s;
		else if (combine == 1) *d = s + 0.0f;
		else *d = *d + s;
	}
}

__global__ void __launch_bounds__(256) sum_rows_lds_kernel(const SumJob job) { sum_rows_block(job, blockIdx.x); }

// Two independent column sums in one launch: blocks below blocks0 take the first job, the rest the second.
__global__ void __launch_bounds__(256) sum_rows_pair_kernel(const SumJob job0, const SumJob job1, int blocks0) {
	const int b = blockIdx.x;
	if (b < blocks0) sum_rows_block(job0, b);
	else sum_rows_block(job1, b - blocks0);
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

namespace {

bool lds_sum_fits(int64_t rows, int64_t inner) { return rows < ((int64_t)1 << 31) && inner < ((int64_t)1 << 31); }

SumJob sum_job(const float* src, int64_t rows, int64_t inner, float* dst, int combine) {
	const int vec = (inner % 4 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0) ? 1 : 0;
	return SumJob{src, dst, (int)rows, (int)inner, combine, vec};
}

unsigned sum_blocks(int64_t inner) { return (unsigned)((inner + kSumCols - 1) / kSumCols); }

// Tensor::sum(axis) of a tensor viewed as {pre, d, post} (src/tensor.cpp:421-456): each output [pre][post] is
// the sum over a = 0..d-1 in order from +0. One thread per output element; combine as sum_rows_kernel.
__global__ void __launch_bounds__(256) sum_axis_kernel(const float* __restrict__ src, int64_t pre, int64_t d,
                                                       int64_t post, float* __restrict__ dst, int combine) {
	const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (idx >= pre * post) return;
	const int64_t p = idx / post, j = idx - p * post;
	const float* q = src + p * d * post + j;
	float s = 0.0f;
	for (int64_t a = 0; a < d; ++a) s = s + q[a * post];
	dst[idx] = combine == 0 ? s : combine == 1 ? s + 0.0f : dst[idx] + s;
}

// add_to_grad (ops.cpp:55-82): a fresh gradient stores src + 0.0f, an existing one adds src.
__global__ void __launch_bounds__(256) add_to_grad_kernel(float* __restrict__ dst, const float* __restrict__ src,
                                                          int64_t count, int first) {
	const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (i >= count) return;
	dst[i] = first ? src[i] + 0.0f : dst[i] + src[i];
}

// The same rule into two gradients of one source (an add node's two operands, in one launch): dst0, then dst1.
__global__ void __launch_bounds__(256) add_to_grad2_kernel(float* __restrict__ dst0, int first0, float* __restrict__ dst1,
                                                           int first1, const float* __restrict__ src, int64_t count) {
	const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (i >= count) return;
	const float v = src[i];
	dst0[i] = first0 ? v + 0.0f : dst0[i] + v;
	dst1[i] = first1 ? v + 0.0f : dst1[i] + v;
}

}  // namespace

hipError_t sum_axis(const float* src, int64_t pre, int64_t d, int64_t post, float* dst, int combine, hipStream_t s) {
	const int64_t total = pre * post;
	if (total == 0) return hipSuccess;
	hipLaunchKernelGGL(sum_axis_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, src, pre, d, post, dst,
	                   combine);
	return hipGetLastError();
}

hipError_t add_to_grad(float* dst, const float* src, int64_t count, int first, hipStream_t s) {
	if (count == 0) return hipSuccess;
	hipLaunchKernelGGL(add_to_grad_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, dst, src, count,
	                   first);
	return hipGetLastError();
}

hipError_t add_to_grad2(float* dst0, int first0, float* dst1, int first1, const float* src, int64_t count, hipStream_t s) {
	if (count == 0) return hipSuccess;
	hipLaunchKernelGGL(add_to_grad2_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, dst0, first0, dst1,
	                   first1, src, count);
	return hipGetLastError();
}

// Two leading axes summed one after the other (sum_to_shape on a {r0, r1, inner} gradient, ops.cpp:35-53, two
// Tensor::sum(0) calls): t[b][j] = the sum over a of src[a][b][j], then s_j = the sum over b of t[b][j], each in
// order from +0, then combined into dst as sum_rows does. One launch instead of two: a workgroup owns 16 columns;
// its 256 threads (16 columns x 16 rows of b) run the first-stage chains, eight of them per thread at a time with
// the loads of eight depth steps of all eight in flight, park them in LDS, and 16 lanes run the second stage.
constexpr int kS2Cols = 16, kS2Rows = 16, kS2Chains = 8, kS2Steps = 8;

__global__ void __launch_bounds__(256) sum_rows2_kernel(const float* __restrict__ src, int r0, int r1, int inner,
                                                        float* __restrict__ dst, int combine) {
	__shared__ float part[kSum2MaxR1 * (kS2Cols + 1)];
	const int jj = threadIdx.x & (kS2Cols - 1), br = threadIdx.x / kS2Cols;
	const int j = min((int)blockIdx.x * kS2Cols + jj, inner - 1);
	const int64_t sa = (int64_t)r1 * inner;
	for (int bp = 0; bp < r1; bp += kS2Rows * kS2Chains) {
		float acc[kS2Chains];
#pragma unroll
		for (int c = 0; c < kS2Chains; ++c) acc[c] = 0.0f;
		for (int a0 = 0; a0 < r0; a0 += kS2Steps) {
			float v[kS2Chains][kS2Steps];
#pragma unroll
			for (int c = 0; c < kS2Chains; ++c)
#pragma unroll
				for (int u = 0; u < kS2Steps; ++u) {
					const int b = min(bp + br + kS2Rows * c, r1 - 1), a = min(a0 + u, r0 - 1);
					v[c][u] = src[a * sa + (int64_t)b * inner + j];
				}
#pragma unroll
			for (int u = 0; u < kS2Steps; ++u)
				if (a0 + u < r0)
#pragma unroll
					for (int c = 0; c < kS2Chains; ++c) acc[c] = acc[c] + v[c][u];
		}
#pragma unroll
		for (int c = 0; c < kS2Chains; ++c) {
			const int b = bp + br + kS2Rows * c;
			if (b < r1) part[b * (kS2Cols + 1) + jj] = acc[c];
		}
	}
	__syncthreads();
	if (threadIdx.x >= kS2Cols || (int)blockIdx.x * kS2Cols + jj >= inner) return;
	float s = 0.0f;
	for (int b = 0; b < r1; ++b) s = s + part[b * (kS2Cols + 1) + jj];
	if (combine == 0) dst[j] = s;
	else if (combine == 1) dst[j] = s + 0.0f;
	else dst[j] = dst[j] + s;
}

bool sum_rows2_fits(int64_t r0, int64_t r1, int64_t inner) {
	return r0 > 0 && r1 > 0 && r1 <= kSum2MaxR1 && inner > 0 && r0 < (1 << 30) && inner < (1 << 30) &&
	       r0 * r1 * inner < ((int64_t)1 << 62) / 4;
}

hipError_t sum_rows2(const float* src, int64_t r0, int64_t r1, int64_t inner, float* dst, int combine, hipStream_t s) {
	if (!sum_rows2_fits(r0, r1, inner)) return hipErrorInvalidValue;
	hipLaunchKernelGGL(sum_rows2_kernel, dim3((unsigned)((inner + kS2Cols - 1) / kS2Cols)), dim3(256), 0, s, src, (int)r0,
	                   (int)r1, (int)inner, dst, combine);
	return hipGetLastError();
}

// +0 into several buffers in one launch: job i covers elements start[i] .. start[i + 1] - 1 of the concatenation.
__global__ void __launch_bounds__(256) zero_many_kernel(const ZeroJobs jobs) {
	const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (e >= jobs.start[jobs.n]) return;
	// the job whose range holds e: the last i with start[i] <= e (a binary search over the starts)
	int lo = 0, hi = jobs.n - 1;
	while (lo < hi) {
		const int mid = (lo + hi + 1) >> 1;
		if (jobs.start[mid] <= e) lo = mid;
		else hi = mid - 1;
	}
	jobs.p[lo][e - jobs.start[lo]] = 0.0f;
}

hipError_t zero_many(const ZeroJobs& jobs, hipStream_t s) {
	const int64_t total = jobs.start[jobs.n];
	if (total == 0) return hipSuccess;
	if ((total + 255) / 256 > 0x7fffffff) return hipErrorInvalidConfiguration;
	hipLaunchKernelGGL(zero_many_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, jobs);
	return hipGetLastError();
}

hipError_t sum_rows(const float* src, int64_t rows, int64_t inner, float* dst, int combine, hipStream_t s) {
	if (inner == 0) return hipSuccess;
	if (lds_sum_fits(rows, inner)) {
		hipLaunchKernelGGL(sum_rows_lds_kernel, dim3(sum_blocks(inner)), dim3(256), 0, s,
		                   sum_job(src, rows, inner, dst, combine));
	} else {
		hipLaunchKernelGGL(sum_rows_kernel, dim3(blocks_for(inner)), dim3(256), 0, s, src, rows, inner, dst, combine);
	}
	return hipGetLastError();
}

hipError_t sum_rows_pair(const float* src0, int64_t rows0, int64_t inner0, float* dst0, int combine0,
                         const float* src1, int64_t rows1, int64_t inner1, float* dst1, int combine1, hipStream_t s) {
	const int64_t blocks = (int64_t)sum_blocks(inner0) + sum_blocks(inner1);
	if (inner0 == 0 || inner1 == 0 || !lds_sum_fits(rows0, inner0) || !lds_sum_fits(rows1, inner1) ||
	    blocks > 0x7fffffff) {
		const hipError_t e = sum_rows(src0, rows0, inner0, dst0, combine0, s);
		return e != hipSuccess ? e : sum_rows(src1, rows1, inner1, dst1, combine1, s);
	}
	hipLaunchKernelGGL(sum_rows_pair_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
	                   sum_job(src0, rows0, inner0, dst0, combine0), sum_job(src1, rows1, inner1, dst1, combine1),
	                   (int)sum_blocks(inner0));
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
