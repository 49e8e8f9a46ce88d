// conv.hip - convolution kernels around the GEMM, each reproducing nn-cpp's operation order
// (src/autograd/ops.cpp:119-243 geometry and im2col, 1345-1472 conv2d_impl).
#include "conv.hpp"

namespace nnh {

namespace {

inline unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

// im2col (ops.cpp:188-212): col[n][(c*kh + ph)*kw + pw][oh*wo + ow] = x[n][c][oh*s + ph - p][ow*s + pw - p],
// 0 where the tap falls in the padding. One thread per column element, consecutive threads along ow:
// coalesced writes, cached reads.
__global__ void __launch_bounds__(256) im2col_kernel(const float* __restrict__ x, float* __restrict__ col, ConvGeom g,
                                                     int64_t total) {
	const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (e >= total) return;
	const int64_t hw = (int64_t)g.ho * g.wo;
	const int64_t K = (int64_t)g.cin * g.kh * g.kw;
	const int64_t p = e % hw;
	const int64_t kk = (e / hw) % K;
	const int64_t n = e / (hw * K);
	const int pw = (int)(kk % g.kw), ph = (int)((kk / g.kw) % g.kh), c = (int)(kk / ((int64_t)g.kh * g.kw));
	const int oh = (int)(p / g.wo), ow = (int)(p % g.wo);
	const int ih = oh * g.stride + ph - g.pad, iw = ow * g.stride + pw - g.pad;
	float v = 0.0f;
	if (ih >= 0 && ih < g.h && iw >= 0 && iw < g.w) v = x[((n * g.cin + c) * g.h + ih) * g.w + iw];
	col[e] = v;
}

// col2im_sample_add (ops.cpp:224-243) in gather form: each input element sums the column entries of its
// taps in (ph, pw) order, which is the order the reference's scatter loop adds them in. init: 0 when the
// gradient is fresh (the reference zero-fills it first), else its current value.
__global__ void __launch_bounds__(256) col2im_kernel(const float* __restrict__ col, float* __restrict__ dx, ConvGeom g,
                                                     int64_t total, int first) {
	const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (e >= total) return;
	const int iw = (int)(e % g.w), ih = (int)((e / g.w) % g.h);
	const int64_t c = (e / ((int64_t)g.w * g.h)) % g.cin;
	const int64_t n = e / ((int64_t)g.w * g.h * g.cin);
	const int64_t hw = (int64_t)g.ho * g.wo;
	const int64_t K = (int64_t)g.cin * g.kh * g.kw;
	const float* cn = col + n * K * hw;
	float acc = first ? 0.0f : dx[e];
	for (int ph = 0; ph < g.kh; ++ph) {
		const int th = ih + g.pad - ph;
		if (th < 0 || th % g.stride != 0) continue;
		const int oh = th / g.stride;
		if (oh >= g.ho) continue;
		for (int pw = 0; pw < g.kw; ++pw) {
			const int tw = iw + g.pad - pw;
			if (tw < 0 || tw % g.stride != 0) continue;
			const int ow = tw / g.stride;
			if (ow >= g.wo) continue;
			acc = acc + cn[((c * g.kh + ph) * g.kw + pw) * hw + (int64_t)oh * g.wo + ow];
		}
	}
	dx[e] = acc;
}

// Direct convolution for a short depth K = cin*kh*kw (the first layer of a CNN), fused with bias, ReLU and
// the alive flags (ops.cpp:1395-1409). Each thread owns one output pixel and CG output channels; every
// output is the reference's chain acc = fma(w[c][k], col[k][p], acc) over k in order from +0, taps in the
// padding included as fma(w, 0, acc), then v = acc + b[c]; relu: alive = v > 0, y = alive ? v : 0.
template <int CG>
__global__ void __launch_bounds__(256) conv_direct_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                          const float* __restrict__ bias, float* __restrict__ y,
                                                          unsigned char* __restrict__ alive, ConvGeom g, int cout,
                                                          int relu, int64_t pixels) {
	const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
	const int c0 = blockIdx.y * CG;
	if (e >= pixels) return;
	const int64_t hw = (int64_t)g.ho * g.wo;
	const int64_t n = e / hw, p = e % hw;
	const int oh = (int)(p / g.wo), ow = (int)(p % g.wo);
	const int K = g.cin * g.kh * g.kw;
	float acc[CG];
#pragma unroll
	for (int c = 0; c < CG; ++c) acc[c] = 0.0f;
	const float* xn = x + n * g.cin * (int64_t)g.h * g.w;
	for (int kk = 0; kk < K; ++kk) {
		const int pw = kk % g.kw, ph = (kk / g.kw) % g.kh, ci = kk / (g.kh * g.kw);
		const int ih = oh * g.stride + ph - g.pad, iw = ow * g.stride + pw - g.pad;
		const float xv = (ih >= 0 && ih < g.h && iw >= 0 && iw < g.w) ? xn[((int64_t)ci * g.h + ih) * g.w + iw] : 0.0f;
#pragma unroll
		for (int c = 0; c < CG; ++c) {
			const int cc = min(c0 + c, cout - 1);  // uniform across the wave: scalar loads
			acc[c] = __builtin_fmaf(w[(int64_t)cc * K + kk], xv, acc[c]);
		}
	}
#pragma unroll
	for (int c = 0; c < CG; ++c) {
		if (c0 + c >= cout) break;
		const int64_t o = (n * cout + c0 + c) * hw + p;
		float v = acc[c] + bias[c0 + c];
		if (relu) {
			const bool on = v > 0.0f;
			if (alive) alive[o] = on ? 1 : 0;
			v = on ? v : 0.0f;
		}
		y[o] = v;
	}
}

// The ReLU's gradient mask (ops.cpp:1439-1443): out = alive ? g : 0.
__global__ void __launch_bounds__(256) mask_kernel(const float* __restrict__ g, const unsigned char* __restrict__ alive,
                                                   float* __restrict__ out, int64_t total) {
	const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (e < total) out[e] = alive[e] ? g[e] : 0.0f;
}

// lane_sum (ops.cpp:804-812) of each of `rows` rows of length n: 8 partial sums in order, combined as
// ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7)), then the tail. One thread per row.
__global__ void __launch_bounds__(256) lane_sum_kernel(const float* __restrict__ src, int64_t rows, int64_t n,
                                                       float* __restrict__ dst) {
	const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (r >= rows) return;
	const float* p = src + r * n;
	float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
	int64_t i = 0;
	for (; i + 8 <= n; i += 8)
#pragma unroll
		for (int k = 0; k < 8; ++k) a[k] = a[k] + p[i + k];
	float t = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
	for (; i < n; ++i) t = t + p[i];
	dst[r] = t;
}

}  // namespace

hipError_t im2col(const float* x, float* col, const ConvGeom& g, int64_t samples, hipStream_t s) {
	const int64_t total = samples * g.cin * g.kh * g.kw * (int64_t)g.ho * g.wo;
	if (total == 0) return hipSuccess;
	hipLaunchKernelGGL(im2col_kernel, dim3(blocks_for(total)), dim3(256), 0, s, x, col, g, total);
	return hipGetLastError();
}

hipError_t col2im(const float* col, float* dx, const ConvGeom& g, int64_t samples, int first, hipStream_t s) {
	const int64_t total = samples * g.cin * (int64_t)g.h * g.w;
	if (total == 0) return hipSuccess;
	hipLaunchKernelGGL(col2im_kernel, dim3(blocks_for(total)), dim3(256), 0, s, col, dx, g, total, first);
	return hipGetLastError();
}

hipError_t conv_direct(const float* x, const float* w, const float* bias, float* y, unsigned char* alive,
                       const ConvGeom& g, int64_t samples, int cout, int relu, hipStream_t s) {
	const int64_t pixels = samples * (int64_t)g.ho * g.wo;
	if (pixels == 0 || cout == 0) return hipSuccess;
	constexpr int CG = 32;
	dim3 grid(blocks_for(pixels), (unsigned)((cout + CG - 1) / CG));
	hipLaunchKernelGGL(conv_direct_kernel<CG>, grid, dim3(256), 0, s, x, w, bias, y, alive, g, cout, relu, pixels);
	return hipGetLastError();
}

hipError_t mask_grad(const float* g, const unsigned char* alive, float* out, int64_t total, hipStream_t s) {
	if (total == 0) return hipSuccess;
	hipLaunchKernelGGL(mask_kernel, dim3(blocks_for(total)), dim3(256), 0, s, g, alive, out, total);
	return hipGetLastError();
}

hipError_t lane_sums(const float* src, int64_t rows, int64_t n, float* dst, hipStream_t s) {
	if (rows == 0) return hipSuccess;
	hipLaunchKernelGGL(lane_sum_kernel, dim3(blocks_for(rows)), dim3(256), 0, s, src, rows, n, dst);
	return hipGetLastError();
}

}  // namespace nnh
