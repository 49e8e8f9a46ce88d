// fastdiv.hpp - unsigned division by a runtime constant as a multiply and a shift (round-up method), exact for
// every numerator below 2^31. Used by index arithmetic in the memory-bound kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace nnh {

struct FastDiv {
	unsigned d, m, s;
};

inline FastDiv make_fastdiv(unsigned d) {
	unsigned s = 0;
	while ((1ull << s) < d) ++s;
	const unsigned m = (unsigned)((((1ull << s) - d) << 32) / d + 1);
	return FastDiv{d, m, s};
}

__device__ __forceinline__ unsigned fdiv(unsigned q, const FastDiv& f) { return (__umulhi(q, f.m) + q) >> f.s; }

}  // namespace nnh
