/*
 * expf_glibc_check.c - checks the restatement of glibc's expf that the GPU softmax uses (expf_glibc in
 * nn-cpp_amd/src/kernels/hip/softmax_row.hpp) against the C library's own expf, which is what nn-cpp's
 * std::exp(float) calls (src/autograd/ops.cpp:1199).
 *
 * The algorithm is ARM optimized-routines' expf (Szabolcs Nagy), which glibc 2.28+ ships: k = round(x 32/ln2)
 * by adding 1.5 * 2^52, r = x 32/ln2 - k, e^x = T[k mod 32] 2^(k div 32) (1 + C2 r + C1 r^2 + C0 r^3) in
 * double, rounded once to float; x86-64 glibc runs its FMA build, whose reduction steps are fused (kd and r
 * below). The unfused variant differs from glibc on 2 inputs, the fused one on none.
 *
 * Usage: expf_glibc_check [stride]   checks every stride-th 32-bit pattern (default 1: all 2^32), 8 processes;
 * prints the number of inputs whose result differs from the C library's (NaN results compare equal).
 * Result on this image (glibc 2.35, x86-64 with FMA), stride 1: 4294967296 inputs, 0 differ.
 * Build: gcc -O2 -ffp-contract=off expf_glibc_check.c -o expf_glibc_check -lm
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/wait.h>
#include <unistd.h>

/* entry i: bits of 2^(i/32) rounded to the nearest double, minus i << 47 (expf_table.py) */
static const uint64_t T[32] = {
0x3ff0000000000000ULL,
0x3fefd9b0d3158574ULL,
0x3fefb5586cf9890fULL,
0x3fef9301d0125b51ULL,
0x3fef72b83c7d517bULL,
0x3fef54873168b9aaULL,
0x3fef387a6e756238ULL,
0x3fef1e9df51fdee1ULL,
0x3fef06fe0a31b715ULL,
0x3feef1a7373aa9cbULL,
0x3feedea64c123422ULL,
0x3feece086061892dULL,
0x3feebfdad5362a27ULL,
0x3feeb42b569d4f82ULL,
0x3feeab07dd485429ULL,
0x3feea47eb03a5585ULL,
0x3feea09e667f3bcdULL,
0x3fee9f75e8ec5f74ULL,
0x3feea11473eb0187ULL,
0x3feea589994cce13ULL,
0x3feeace5422aa0dbULL,
0x3feeb737b0cdc5e5ULL,
0x3feec49182a3f090ULL,
0x3feed503b23e255dULL,
0x3feee89f995ad3adULL,
0x3feeff76f2fb5e47ULL,
0x3fef199bdd85529cULL,
0x3fef3720dcef9069ULL,
0x3fef5818dcfba487ULL,
0x3fef7c97337b9b5fULL,
0x3fefa4afa2a490daULL,
0x3fefd0765b6e4540ULL
};

static uint64_t u64(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static double f64(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }
static uint32_t u32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float expf_restated(float x) {
	const uint32_t abstop = (u32(x) >> 20) & 0x7ff;
	if (abstop >= 0x42b) {
		if (u32(x) == 0xff800000u) return 0.0f;
		if (abstop >= 0x7f8) return x + x;
		if (x > 0x1.62e42ep6f) return INFINITY;
		if (x < -0x1.9fe368p6f) return 0.0f;
	}
	const double InvLn2N = 0x1.71547652b82fep+0 * 32, Shift = 0x1.8p+52;
	const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
	             C2 = 0x1.62e42ff0c52d6p-1 / 32;
	const double xd = x;
	double kd = fma(InvLn2N, xd, Shift);
	const uint64_t ki = u64(kd);
	kd -= Shift;
	const double r = fma(InvLn2N, xd, -kd);
	const double s = f64(T[ki % 32] + (ki << 47));
	const double z = fma(C0, r, C1), r2 = r * r;
	double y = fma(C2, r, 1.0);
	y = fma(z, r2, y);
	return (float)(y * s);
}

int main(int argc, char** argv) {
	const uint64_t stride = argc > 1 ? strtoull(argv[1], NULL, 10) : 1;
	const int P = 8;
	int fds[8][2];
	for (int p = 0; p < P; ++p) {
		if (pipe(fds[p]) != 0) return 2;
		if (fork() == 0) {
			uint64_t counts[2] = {0, 0};
			for (uint64_t b = (uint64_t)p * stride; b < (1ull << 32); b += (uint64_t)P * stride) {
				const uint32_t bits = (uint32_t)b;
				float x;
				memcpy(&x, &bits, 4);
				const float g = expf(x), c = expf_restated(x);
				++counts[0];
				if (!(isnan(g) && isnan(c)) && memcmp(&g, &c, 4) != 0) {
					if (counts[1] < 3) fprintf(stderr, "x=%a glibc=%a restated=%a\n", x, g, c);
					++counts[1];
				}
			}
			if (write(fds[p][1], counts, sizeof counts) != sizeof counts) _exit(3);
			_exit(0);
		}
	}
	uint64_t n = 0, bad = 0;
	for (int p = 0; p < P; ++p) {
		uint64_t counts[2];
		if (read(fds[p][0], counts, sizeof counts) != sizeof counts) return 2;
		n += counts[0];
		bad += counts[1];
	}
	for (int p = 0; p < P; ++p) wait(NULL);
	printf("%llu inputs, %llu differ\n", (unsigned long long)n, (unsigned long long)bad);
	return bad != 0;
}
