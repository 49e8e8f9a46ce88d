// conv.hip - convolution kernels around the GEMM, each reproducing nn-cpp's operation order
// (src/autograd/ops.cpp:119-243 geometry and im2col, 1345-1472 conv2d_impl).
#include "conv.hpp"
#include "fastdiv.hpp"

namespace nnh {

namespace {

inline unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

typedef float f32x4 __attribute__((ext_vector_type(4)));

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

// Direct convolution for the common first-layer shape: stride 1, "same" width (kw = 2*PAD + 1, so wo == w),
// w % 4 == 0, ROWS = cin * kh input rows per output row. Each lane owns 4 consecutive output pixels of one row
// (a quad) and CG output channels, so every global access is 16 bytes: one aligned float4 of each input row it
// touches, one float4 of y and one 4-byte word of alive flags per channel. All ROWS row loads are issued
// before any arithmetic, so a wave waits for memory once. The PAD columns left and right of a quad's float4
// are the neighbouring lanes' float4 elements (lanes l-1 and l+1 own the quads before and after it in the same
// row), taken with lane shuffles; the first and last lane of a wave load them directly, and the row ends are
// zero padding. Each output is the same chain as conv_direct_kernel: fma over k = (c, ph, pw) in order from
// +0, padding taps included as fma(w, 0, acc), then v = acc + b[c] and the ReLU/alive rule.
template <int CG, int PAD, int ROWS>
__global__ void __launch_bounds__(256) conv_same_quad_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                             const float* __restrict__ bias, float* __restrict__ y,
                                                             unsigned char* __restrict__ alive, ConvGeom g, FastDiv qpr,
                                                             FastDiv ho, FastDiv kh, int cout, int relu,
                                                             int total_quads) {
	constexpr int KW = 2 * PAD + 1;
	constexpr int K = ROWS * KW;
	const int tid = threadIdx.x;
	const int lane = tid & 63;
	const int q = blockIdx.x * 256 + tid;
	const bool active = q < total_quads;
	const unsigned qc = active ? q : total_quads - 1;  // inactive lanes still take part in the shuffles
	const unsigned rest = fdiv(qc, qpr);
	const int ow0 = (int)(qc - rest * qpr.d) * 4;
	const unsigned n = fdiv(rest, ho);
	const int oh = (int)(rest - n * ho.d);
	const int c0 = blockIdx.y * CG;
	const bool has_left = ow0 > 0, has_right = ow0 + 4 < g.w;
	const float* __restrict__ xn = x + (int64_t)n * g.cin * g.h * g.w;

	// input row r = (ci, ph) with ci = r / kh, ph = r % kh; every load is issued before the arithmetic
	f32x4 v[ROWS];
	int off[ROWS];
	bool ok[ROWS];
#pragma unroll
	for (int r = 0; r < ROWS; ++r) {
		const int ci = (int)fdiv(r, kh);
		const int ih = oh + (r - ci * (int)kh.d) - PAD;
		ok[r] = ih >= 0 && ih < g.h;
		off[r] = (ci * g.h + (ok[r] ? ih : 0)) * g.w;
		v[r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
		if (ok[r]) v[r] = *reinterpret_cast<const f32x4*>(xn + off[r] + ow0);
	}

	float acc[CG][4];
#pragma unroll
	for (int c = 0; c < CG; ++c)
#pragma unroll
		for (int i = 0; i < 4; ++i) acc[c][i] = 0.0f;
#pragma unroll
	for (int r = 0; r < ROWS; ++r) {
		float seg[4 + 2 * PAD];
#pragma unroll
		for (int i = 0; i < 4; ++i) seg[PAD + i] = v[r][i];
#pragma unroll
		for (int e = 0; e < PAD; ++e) {
			float l = __shfl_up(v[r][4 - PAD + e], 1);
			float rr = __shfl_down(v[r][e], 1);
			if (lane == 0 && has_left) l = ok[r] ? xn[off[r] + ow0 - PAD + e] : 0.0f;
			if (lane == 63 && has_right) rr = ok[r] ? xn[off[r] + ow0 + 4 + e] : 0.0f;
			seg[e] = has_left ? l : 0.0f;
			seg[PAD + 4 + e] = has_right ? rr : 0.0f;
		}
#pragma unroll
		for (int pw = 0; pw < KW; ++pw) {
#pragma unroll
			for (int c = 0; c < CG; ++c) {
				const float wv = w[min(c0 + c, cout - 1) * K + r * KW + pw];
#pragma unroll
				for (int i = 0; i < 4; ++i) acc[c][i] = __builtin_fmaf(wv, seg[i + pw], acc[c][i]);
			}
		}
	}
	if (!active) return;
	const int64_t hw = (int64_t)g.ho * g.wo;
	const int64_t p0 = (int64_t)oh * g.wo + ow0;
#pragma unroll
	for (int c = 0; c < CG; ++c) {
		if (c0 + c >= cout) break;
		const int64_t o = ((int64_t)n * cout + c0 + c) * hw + p0;
		const float b = bias[c0 + c];
		f32x4 out;
		unsigned flags = 0;
#pragma unroll
		for (int i = 0; i < 4; ++i) {
			float val = acc[c][i] + b;
			if (relu) {
				const bool on = val > 0.0f;
				flags |= (on ? 1u : 0u) << (8 * i);
				val = on ? val : 0.0f;
			}
			out[i] = val;
		}
		*reinterpret_cast<f32x4*>(y + o) = out;
		if (alive) *reinterpret_cast<unsigned*>(alive + o) = flags;
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

namespace {

constexpr int kQuadMaxRows = 8;

template <int CG, int PAD, int ROWS>
hipError_t launch_quad_rows(const float* x, const float* w, const float* bias, float* y, unsigned char* alive,
                            const ConvGeom& g, int total_quads, int cout, int relu, hipStream_t s) {
	if constexpr (ROWS * (2 * PAD + 1) > 32) {
		return hipErrorInvalidValue;
	} else {
		dim3 grid(blocks_for(total_quads), (unsigned)((cout + CG - 1) / CG));
		hipLaunchKernelGGL((conv_same_quad_kernel<CG, PAD, ROWS>), grid, dim3(256), 0, s, x, w, bias, y, alive, g,
		                   make_fastdiv((unsigned)(g.wo / 4)), make_fastdiv((unsigned)g.ho), make_fastdiv((unsigned)g.kh),
		                   cout, relu, total_quads);
		return hipGetLastError();
	}
}

template <int CG, int PAD>
hipError_t launch_quad_pad(const float* x, const float* w, const float* bias, float* y, unsigned char* alive,
                           const ConvGeom& g, int total_quads, int cout, int relu, hipStream_t s) {
	switch (g.cin * g.kh) {
		case 1: return launch_quad_rows<CG, PAD, 1>(x, w, bias, y, alive, g, total_quads, cout, relu, s);
		case 2: return launch_quad_rows<CG, PAD, 2>(x, w, bias, y, alive, g, total_quads, cout, relu, s);
		case 3: return launch_quad_rows<CG, PAD, 3>(x, w, bias, y, alive, g, total_quads, cout, relu, s);
		case 4: return launch_quad_rows<CG, PAD, 4>(x, w, bias, y, alive, g, total_quads, cout, relu, s);
		case 5: return launch_quad_rows<CG, PAD, 5>(x, w, bias, y, alive, g, total_quads, cout, relu, s);
		case 6: return launch_quad_rows<CG, PAD, 6>(x, w, bias, y, alive, g, total_quads, cout, relu, s);
		case 7: return launch_quad_rows<CG, PAD, 7>(x, w, bias, y, alive, g, total_quads, cout, relu, s);
		case 8: return launch_quad_rows<CG, PAD, 8>(x, w, bias, y, alive, g, total_quads, cout, relu, s);
		default: return hipErrorInvalidValue;
	}
}

template <int CG>
hipError_t launch_same_quad(const float* x, const float* w, const float* bias, float* y, unsigned char* alive,
                            const ConvGeom& g, int total_quads, int cout, int relu, hipStream_t s) {
	switch (g.pad) {
		case 0: return launch_quad_pad<CG, 0>(x, w, bias, y, alive, g, total_quads, cout, relu, s);
		case 1: return launch_quad_pad<CG, 1>(x, w, bias, y, alive, g, total_quads, cout, relu, s);
		case 2: return launch_quad_pad<CG, 2>(x, w, bias, y, alive, g, total_quads, cout, relu, s);
		case 3: return launch_quad_pad<CG, 3>(x, w, bias, y, alive, g, total_quads, cout, relu, s);
		case 4: return launch_quad_pad<CG, 4>(x, w, bias, y, alive, g, total_quads, cout, relu, s);
		default: return hipErrorInvalidValue;
	}
}

}  // namespace

bool conv_same_quad_ok(const float* x, const float* y, const unsigned char* alive, const ConvGeom& g, int64_t samples) {
	return g.stride == 1 && g.kw == 2 * g.pad + 1 && g.pad <= 4 && g.w % 4 == 0 && g.wo == g.w &&
	       g.cin * g.kh <= kQuadMaxRows && g.cin * g.kh * g.kw <= 32 &&
	       samples * g.ho * (int64_t)(g.wo / 4) < (int64_t)1 << 30 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
	       reinterpret_cast<uintptr_t>(y) % 16 == 0 && reinterpret_cast<uintptr_t>(alive) % 4 == 0;
}

hipError_t conv_same_quad(const float* x, const float* w, const float* bias, float* y, unsigned char* alive,
                          const ConvGeom& g, int64_t samples, int cout, int relu, int cg, hipStream_t s) {
	const int total_quads = (int)(samples * g.ho * (int64_t)(g.wo / 4));
	if (total_quads == 0 || cout == 0) return hipSuccess;
	switch (cg) {
		case 4: return launch_same_quad<4>(x, w, bias, y, alive, g, total_quads, cout, relu, s);
		case 8: return launch_same_quad<8>(x, w, bias, y, alive, g, total_quads, cout, relu, s);
		default: return hipErrorInvalidValue;
	}
}

hipError_t conv_direct(const float* x, const float* w, const float* bias, float* y, unsigned char* alive,
                       const ConvGeom& g, int64_t samples, int cout, int relu, hipStream_t s) {
	const int64_t pixels = samples * (int64_t)g.ho * g.wo;
	if (pixels == 0 || cout == 0) return hipSuccess;
	if (conv_same_quad_ok(x, y, alive, g, samples)) return conv_same_quad(x, w, bias, y, alive, g, samples, cout, relu, 4, s);
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
