// reduce.hpp - launchers of the memory-bound kernels in reduce.hip (internal to libnnh).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nnh {

// dst[j] (combine 0: =, 1: = s + 0.0f, 2: +=) s_j = sum over rows a, in order from +0, of src[a * inner + j].
hipError_t sum_rows(const float* src, int64_t rows, int64_t inner, float* dst, int combine, hipStream_t s);
// Two independent sum_rows in one launch (the same bits as two calls).
hipError_t sum_rows_pair(const float* src0, int64_t rows0, int64_t inner0, float* dst0, int combine0,
                         const float* src1, int64_t rows1, int64_t inner1, float* dst1, int combine1, hipStream_t s);
// sum_rows over the first axis of a {r0, r1, inner} tensor, then over the second (two Tensor::sum(0) in turn, the
// same bits as two calls), in one launch, when r1 <= kSum2MaxR1; combine as sum_rows.
constexpr int kSum2MaxR1 = 512;
bool sum_rows2_fits(int64_t r0, int64_t r1, int64_t inner);
hipError_t sum_rows2(const float* src, int64_t r0, int64_t r1, int64_t inner, float* dst, int combine, hipStream_t s);
// Tensor::sum(axis) over {pre, d, post} into {pre, post} (combine as sum_rows).
hipError_t sum_axis(const float* src, int64_t pre, int64_t d, int64_t post, float* dst, int combine, hipStream_t s);
// Up to kZeroJobs buffers filled with +0 in one launch (start[0] = 0, start[i + 1] - start[i] = buffer i's length).
constexpr int kZeroJobs = 64;
struct ZeroJobs {
	float* p[kZeroJobs];
	int64_t start[kZeroJobs + 1];
	int n;
};
hipError_t zero_many(const ZeroJobs& jobs, hipStream_t s);
// dst = src + 0.0f (first) or dst += src, element by element (add_to_grad, ops.cpp:55-82).
hipError_t add_to_grad(float* dst, const float* src, int64_t count, int first, hipStream_t s);
// The same into two gradients that do not overlap each other or src: dst0's rule, then dst1's, in one launch.
hipError_t add_to_grad2(float* dst0, int first0, float* dst1, int first1, const float* src, int64_t count, hipStream_t s);
hipError_t relu_forward(const float* x, float* y, int64_t count, hipStream_t s);
hipError_t relu_backward(const float* x, const float* g, float* dst, int64_t count, int first, hipStream_t s);

}  // namespace nnh
