// softmax_row.hpp - device arithmetic of nn-cpp's masked_softmax_row (src/autograd/ops.cpp:1183-1204) shared by
// the row softmax kernels (softmax.hip) and the fused attention forward (attention.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace nnh {

// std::exp(float) in nn-cpp is glibc's expf (ops.cpp:1199). glibc (2.28 and later) implements it with the
// published algorithm of ARM's optimized-routines (expf by Szabolcs Nagy): e^x = 2^(k/32) 2^(r/32) with
// k = round(x 32/ln2) and |r| <= 1/2, 2^(k/32) from a 32-entry table, 2^(r/32) from a cubic, all in double, then
// rounded once to float. x86-64 glibc runs the build of it compiled with FMA, which fuses the reduction steps.
// This restatement of that algorithm (same constants, same fused steps, same special cases) returns glibc's
// expf bit for bit on every one of the 2^32 float inputs (tests/golden/expf_glibc_check.c), so the attention
// path has no arithmetic difference from the reference.
// kExp2Table[i] = bits of 2^(i/32) rounded to the nearest double, minus i << 47 (tests/golden/expf_table.py).
static __constant__ unsigned long long kExp2Table[32] = {  // copied into LDS by each block
	0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
	0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
	0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
	0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
	0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
	0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
	0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
	0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// The main path of expf_glibc, for |x| < 88 (for other x its value is discarded by expf_special; the table index
// is always in range). No branches, so the table reads of several calls overlap.
__device__ __forceinline__ float expf_main(float x, const unsigned long long* table) {
	constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32, kShift = 0x1.8p+52;
	constexpr double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
	                 kC2 = 0x1.62e42ff0c52d6p-1 / 32;
	const double xd = x;
	double kd = __builtin_fma(kInvLn2N, xd, kShift);  // k + kShift, rounded to an integer by the addition
	const unsigned long long ki = (unsigned long long)__double_as_longlong(kd);
	kd -= kShift;
	const double r = __builtin_fma(kInvLn2N, xd, -kd);
	const double s = __longlong_as_double((long long)(table[ki & 31] + (ki << 47)));
	const double z = __builtin_fma(kC0, r, kC1), r2 = r * r;
	double y = __builtin_fma(kC2, r, 1.0);
	y = __builtin_fma(z, r2, y);
	return (float)(y * s);
}

// Whether x takes glibc's special-case branch: |x| >= 88, infinity or NaN.
__device__ __forceinline__ bool expf_is_special(float x) { return ((__float_as_uint(x) >> 20) & 0x7ffu) >= 0x42bu; }

// glibc's special cases, in its order, for x with expf_is_special(x); main is expf_main(x) (used when x is in
// neither the overflow nor the underflow range).
__device__ __forceinline__ float expf_special(float x, float main) {
	const unsigned ux = __float_as_uint(x), abstop = (ux >> 20) & 0x7ffu;
	float r = main;
	r = x < -0x1.9fe368p6f ? 0.0f : r;             // e^x below half the smallest subnormal
	r = x > 0x1.62e42ep6f ? __builtin_inff() : r;  // e^x overflows
	r = abstop >= 0x7f8u ? x + x : r;              // infinity or NaN
	r = ux == 0xff800000u ? 0.0f : r;              // -infinity
	return r;
}

__device__ __forceinline__ float expf_glibc(float x, const unsigned long long* table) {
	const float m = expf_main(x, table);
	return expf_is_special(x) ? expf_special(x, m) : m;
}

// expf_glibc over N values with the special cases behind one test, which a wave skips when none of its lanes
// has one (the common case in a softmax, where x = v - max lies in (-88, 0]).
template <int N>
__device__ __forceinline__ void expf_glibc_n(float (&v)[N], const unsigned long long* table) {
	float x[N];
	bool special = false;
#pragma unroll
	for (int i = 0; i < N; ++i) {
		x[i] = v[i];
		v[i] = expf_main(x[i], table);
		special |= expf_is_special(x[i]);
	}
	if (special) {
#pragma unroll
		for (int i = 0; i < N; ++i) v[i] = expf_is_special(x[i]) ? expf_special(x[i], v[i]) : v[i];
	}
}

// p / s rounded once to float, for the quotients of a softmax row: p is one of the row's exponentials and s their
// sum, so 0 <= p <= s <= Tk unless one of them is NaN. With rinv = 1 / (double)s (one rounding), q = (double)p *
// rinv is within 2^-52 (relative) of p / s. A quotient of two floats in the normal range is a float or lies at
// least 2^-49 (relative) away from every midpoint between two floats (p = s m for such a midpoint m would give p
// an odd significand of 25 or more bits), so rounding q to float gives the correctly rounded p / s, i.e. the
// reference's division. Positive quotients below 2^-125 (where subnormal midpoints can be hit exactly) take the
// IEEE division instead. p = 0 gives +0 (or NaN for s = 0) and NaN stays NaN, as with the division. Checked
// against float division on adversarial and random operands (tests/test_softmax_division.py).
__device__ __forceinline__ bool row_quotient_tiny(double q) { return q > 0.0 && q < 0x1p-125; }

__device__ __forceinline__ float div_by_row_sum(float p, float s, double rinv) {
	const double q = (double)p * rinv;
	if (row_quotient_tiny(q)) return p / s;
	return (float)q;
}

// div_by_row_sum over N values of one row, without a branch per value: the products first, then the IEEE
// division only for the values that need it, behind one test that a wave skips when none of its lanes does.
template <int N>
__device__ __forceinline__ void div_n_by_row_sum(float (&v)[N], float s, double rinv) {
	bool tiny = false;
	float p[N];
#pragma unroll
	for (int i = 0; i < N; ++i) {
		p[i] = v[i];
		const double q = (double)p[i] * rinv;
		tiny |= row_quotient_tiny(q);
		v[i] = (float)q;
	}
	if (tiny) {
#pragma unroll
		for (int i = 0; i < N; ++i)
			if (row_quotient_tiny((double)p[i] * rinv)) v[i] = p[i] / s;
	}
}

}  // namespace nnh
