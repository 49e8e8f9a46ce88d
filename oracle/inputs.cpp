// inputs.cpp - the reference's seeded input streams, for pinning the product's host-side generator.
// TEST INFRASTRUCTURE ONLY (see oracle.h).
// apps/bench/runner.cpp:80-86 and tests/test_kernels.cpp:75-83 fill operands in row-major order from
// std::mt19937(seed) through std::uniform_real_distribution<float>(lo, hi).
#include <cstddef>
#include <random>

extern "C" void oracle_mt19937_uniform(unsigned seed, float lo, float hi, float* out, size_t count) {
	std::mt19937 gen(seed);
	std::uniform_real_distribution<float> dist(lo, hi);
	for (size_t i = 0; i < count; ++i) out[i] = dist(gen);
}
