// elementwise.hpp - launchers of the element-wise kernels in elementwise.hip (internal to libnnh).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nnh {

// y[o][j] = a[o][j] + b[j] over outer x inner (nn::add with b broadcast along a's leading axes, tensor.cpp:543-545).
hipError_t add_bcast(const float* a, const float* b, int64_t outer, int64_t inner, float* y, hipStream_t s);
// nn::mul (tensor.cpp:551-553) of two same-shaped tensors, and one operand's backward term (ops.cpp:347-357):
// d = g * other, stored as term + 0 when first, else added.
hipError_t mul(const float* a, const float* b, int64_t count, float* y, hipStream_t s);
hipError_t mul_grad(const float* g, const float* other, int64_t count, float* d, int first, hipStream_t s);
// nn::gelu (ops.cpp:451-466): y, and th = tanh(k (x + c x^3)) kept for the backward pass.
hipError_t gelu_forward(const float* x, int64_t count, float* y, float* th, hipStream_t s);
// Its backward rule (ops.cpp:467-480); first: the gradient is fresh (term + 0 stored).
hipError_t gelu_backward(const float* x, const float* th, const float* g, int64_t count, float* dx, int first,
                         hipStream_t s);
// nn::embedding (ops.cpp:1991-2015) with validated rows (0 <= rows[i] < V).
// add (optional): the addend {add_rows, D} broadcast over the ids and added after the lookup.
hipError_t embedding_forward(const float* w, int64_t V, int64_t D, const int* rows, int64_t count, float* out,
                             hipStream_t s, const float* add = nullptr, int64_t add_rows = 1);
hipError_t embedding_backward(const float* g, const int* rows, int64_t count, int64_t V, int64_t D, float* dw, int first,
                              hipStream_t s);

}  // namespace nnh
