// gelu_math.hpp - nn-cpp's GELU (tanh form) for one element, shared by the element-wise kernels (elementwise.hip) and
// the GEMM epilogue that applies it to a linear layer's output (gemm_direct.hpp). Internal to libnnh.
//
// The tanh is nn-cpp's own (src/kernels/vmath.cpp:24-105): Cephes expf with the reference's constants and operation
// order (x = n ln2 + r, ln2 split in two, a degree-5 polynomial in r, 2^n by building the exponent bits),
// tanh(z) = (e^(2z) - 1) / (e^(2z) + 1) with z clamped to +-9. Every operation rounds on its own (every file that
// includes this is built with -ffp-contract=off), the division is correctly rounded, rintf rounds half to even as
// nearbyint and _MM_FROUND_TO_NEAREST_INT do, so each element gets the reference's bits.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>

namespace nnh {
namespace gelu_math {

constexpr float kExpLo = -87.3f, kExpHi = 88.3f;
constexpr float kLog2e = 1.44269504088896341f;
constexpr float kLn2Hi = 0.693359375f, kLn2Lo = -2.12194440e-4f;
constexpr float kP0 = 1.9875691500e-4f, kP1 = 1.3981999507e-3f, kP2 = 8.3334519073e-3f;
constexpr float kP3 = 4.1665795894e-2f, kP4 = 1.6666665459e-1f, kP5 = 5.0000001201e-1f;
constexpr float kTanhMax = 9.0f;
constexpr float kGeluK = 0.7978845608f;  // sqrt(2 / pi), ops.cpp:452
constexpr float kGeluC = 0.044715f;

__device__ __forceinline__ float exp_one(float x) {
	if (x != x) return x;
	if (x < kExpLo) return 0.0f;
	if (x > kExpHi) return INFINITY;
	const float n = rintf(x * kLog2e);
	float r = x - n * kLn2Hi;
	r = r - n * kLn2Lo;
	float p = kP0;
	p = p * r + kP1;
	p = p * r + kP2;
	p = p * r + kP3;
	p = p * r + kP4;
	p = p * r + kP5;
	const float e = (p * (r * r) + r) + 1.0f;
	const float pow2 = __int_as_float((int)(((unsigned)((int)n + 127)) << 23));
	return e * pow2;
}

__device__ __forceinline__ float tanh_one(float x) {
	if (x != x) return x;
	float z = x < -kTanhMax ? -kTanhMax : x;
	z = kTanhMax < z ? kTanhMax : z;
	const float e = exp_one(z + z);
	return (e - 1.0f) / (e + 1.0f);
}

// ops.cpp:461-466: t = tanh(k (v + c v v v)) (kept for the backward rule), y = 0.5 v (1 + t).
__device__ __forceinline__ float gelu_one(float v, float& t) {
	t = tanh_one(kGeluK * (v + kGeluC * v * v * v));
	return 0.5f * v * (1.0f + t);
}

}  // namespace gelu_math
}  // namespace nnh
