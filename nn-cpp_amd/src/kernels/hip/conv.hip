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
                                                             unsigned char* __restrict__ alive,
                                                             unsigned char* __restrict__ bits, ConvGeom g, FastDiv qpr,
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
	const int64_t hw = (int64_t)g.ho * g.wo;
	const int64_t p0 = (int64_t)oh * g.wo + ow0;
#pragma unroll
	for (int c = 0; c < CG; ++c) {
		if (c0 + c >= cout) break;  // uniform
		const int64_t o = ((int64_t)n * cout + c0 + c) * hw + p0;
		const float b = bias[c0 + c];
		f32x4 out;
		unsigned flags = 0, nib = 0;
#pragma unroll
		for (int i = 0; i < 4; ++i) {
			float val = acc[c][i] + b;
			if (relu) {
				const bool on = val > 0.0f;
				flags |= (on ? 1u : 0u) << (8 * i);
				nib |= (on ? 1u : 0u) << i;
				val = on ? val : 0.0f;
			}
			out[i] = val;
		}
		if (active) *reinterpret_cast<f32x4*>(y + o) = out;
		if (active && alive) *reinterpret_cast<unsigned*>(alive + o) = flags;
		if (bits) {
			// one bit per output in y's order (bit o at byte o / 8): with Ho Wo a multiple of 8, quads 2 t and 2 t + 1
			// (lanes of one wave) share a byte, which the even one writes
			const unsigned partner = __shfl_down(nib, 1);
			if (active && (q & 1) == 0) bits[o >> 3] = (unsigned char)(nib | (partner << 4));
		}
	}
}

// Index arithmetic of the fast im2col / col2im kernels: 32-bit division by the geometry as multiply-shifts.
struct ConvDiv {
	FastDiv hw4;   // quads per column row (hw / 4)
	FastDiv k;     // rows of a sample's columns (cin * kh * kw)
	FastDiv khkw;  // kh * kw
	FastDiv kw, wo, w, h, cin, stride;
};

// im2col with four consecutive column entries per thread (hw % 4 == 0): one 16-byte store, four cached loads.
// Same values as im2col_kernel.
__global__ void __launch_bounds__(256) im2col_quad_kernel(const float* __restrict__ x, float* __restrict__ col,
                                                          ConvGeom g, ConvDiv d, unsigned total4) {
	const unsigned e = blockIdx.x * 256 + threadIdx.x;
	if (e >= total4) return;
	const unsigned row = fdiv(e, d.hw4);  // n * K + kk
	const unsigned p0 = (e - row * d.hw4.d) * 4;
	const unsigned n = fdiv(row, d.k);
	const unsigned kk = row - n * d.k.d;
	const unsigned c = fdiv(kk, d.khkw);
	const unsigned rem = kk - c * d.khkw.d;
	const unsigned ph = fdiv(rem, d.kw);
	const int pw = (int)(rem - ph * d.kw.d);
	const float* xp = x + ((int64_t)n * g.cin + c) * g.h * g.w;
	f32x4 v;
#pragma unroll
	for (int i = 0; i < 4; ++i) {
		const unsigned p = p0 + i;
		const unsigned oh = fdiv(p, d.wo);
		const int ow = (int)(p - oh * d.wo.d);
		const int ih = (int)oh * g.stride + (int)ph - g.pad, iw = ow * g.stride + pw - g.pad;
		v[i] = (ih >= 0 && ih < g.h && iw >= 0 && iw < g.w) ? xp[ih * g.w + iw] : 0.0f;
	}
	*reinterpret_cast<f32x4*>(col + (int64_t)e * 4) = v;
}

// col2im_kernel with 32-bit index arithmetic (total < 2^31): the same gather in (ph, pw) order.
__global__ void __launch_bounds__(256) col2im_fast_kernel(const float* __restrict__ col, float* __restrict__ dx,
                                                          ConvGeom g, ConvDiv d, unsigned total, int first) {
	const unsigned e = blockIdx.x * 256 + threadIdx.x;
	if (e >= total) return;
	const unsigned t0 = fdiv(e, d.w);
	const int iw = (int)(e - t0 * d.w.d);
	const unsigned t1 = fdiv(t0, d.h);
	const int ih = (int)(t0 - t1 * d.h.d);
	const unsigned n = fdiv(t1, d.cin);
	const int c = (int)(t1 - n * d.cin.d);
	const int hw = g.ho * g.wo;
	const float* cn = col + (int64_t)n * d.k.d * hw;
	float acc = first ? 0.0f : dx[e];
	for (int ph = 0; ph < g.kh; ++ph) {
		const int th = ih + g.pad - ph;
		if (th < 0) continue;
		const unsigned qh = fdiv((unsigned)th, d.stride);
		if ((int)(qh * d.stride.d) != th || (int)qh >= g.ho) continue;
		for (int pw = 0; pw < g.kw; ++pw) {
			const int tw = iw + g.pad - pw;
			if (tw < 0) continue;
			const unsigned qw = fdiv((unsigned)tw, d.stride);
			if ((int)(qw * d.stride.d) != tw || (int)qw >= g.wo) continue;
			acc = acc + cn[((c * g.kh + ph) * g.kw + pw) * hw + (int)qh * g.wo + (int)qw];
		}
	}
	dx[e] = acc;
}

// The ReLU's gradient mask on four elements per thread (count % 4 == 0, 16-byte aligned g and out).
__global__ void __launch_bounds__(256) mask4_kernel(const float* __restrict__ g, const unsigned* __restrict__ alive,
                                                    float* __restrict__ out, unsigned total4) {
	const unsigned e = blockIdx.x * 256 + threadIdx.x;
	if (e >= total4) return;
	const f32x4 v = reinterpret_cast<const f32x4*>(g)[e];
	const unsigned a = alive[e];
	f32x4 o;
#pragma unroll
	for (int i = 0; i < 4; ++i) o[i] = ((a >> (8 * i)) & 0xffu) ? v[i] : 0.0f;
	reinterpret_cast<f32x4*>(out)[e] = o;
}

// lane_sum (ops.cpp:804-812) with eight lanes per row: lane k of a row's group computes the reference's partial
// sum a[k] (elements k, k+8, ... of the full groups of eight, in order, from +0); the group's first lane
// combines them as ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7)) and adds the tail in order.
__global__ void __launch_bounds__(256) lane_sum8_kernel(const float* __restrict__ src, unsigned rows, int n,
                                                        float* __restrict__ dst) {
	const unsigned gid = blockIdx.x * 256 + threadIdx.x;
	const unsigned row = gid >> 3;
	const int k = (int)(gid & 7);
	const bool valid = row < rows;
	const float* p = src + (int64_t)(valid ? row : 0) * n;
	const int full = n & ~7;
	float a = 0.0f;
	if (valid) {
		// eight loads in flight ahead of the dependent additions
		int i = k;
		for (; i + 56 < full; i += 64) {
			float v[8];
#pragma unroll
			for (int u = 0; u < 8; ++u) v[u] = p[i + 8 * u];
#pragma unroll
			for (int u = 0; u < 8; ++u) a = a + v[u];
		}
		for (; i < full; i += 8) a = a + p[i];
	}
	const int base = (int)(threadIdx.x & 63) & ~7;
	float part[8];
#pragma unroll
	for (int j = 0; j < 8; ++j) part[j] = __shfl(a, base + j);
	if (valid && k == 0) {
		float t = ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
		for (int i = full; i < n; ++i) t = t + p[i];
		dst[row] = t;
	}
}

// The ReLU's gradient mask and lane_sum of each masked row in one pass (ops.cpp:1439-1445): out = alive ? g : 0,
// and dst[row] = lane_sum(out row), with lane_sum8_kernel's arrangement (eight lanes per row, lane k the
// reference's partial a[k]).
__global__ void __launch_bounds__(256) mask_lane_sum8_kernel(const float* __restrict__ g,
                                                             const unsigned char* __restrict__ alive,
                                                             float* __restrict__ out, unsigned rows, int n,
                                                             float* __restrict__ dst) {
	const unsigned gid = blockIdx.x * 256 + threadIdx.x;
	const unsigned row = gid >> 3;
	const int k = (int)(gid & 7);
	const bool valid = row < rows;
	const int64_t off = (int64_t)(valid ? row : 0) * n;
	const float* p = g + off;
	const unsigned char* al = alive + off;
	float* o = out + off;
	const int full = n & ~7;
	float a = 0.0f;
	if (valid) {
		int i = k;
		for (; i + 56 < full; i += 64) {  // eight elements in flight ahead of the dependent additions
			float v[8];
			unsigned char f[8];
#pragma unroll
			for (int u = 0; u < 8; ++u) {
				v[u] = p[i + 8 * u];
				f[u] = al[i + 8 * u];
			}
#pragma unroll
			for (int u = 0; u < 8; ++u) {
				const float m = f[u] ? v[u] : 0.0f;
				o[i + 8 * u] = m;
				a = a + m;
			}
		}
		for (; i < full; i += 8) {
			const float m = al[i] ? p[i] : 0.0f;
			o[i] = m;
			a = a + m;
		}
	}
	const int base = (int)(threadIdx.x & 63) & ~7;
	float part[8];
#pragma unroll
	for (int j = 0; j < 8; ++j) part[j] = __shfl(a, base + j);
	if (valid && k == 0) {
		float t = ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
		for (int i = full; i < n; ++i) {
			const float m = al[i] ? p[i] : 0.0f;
			o[i] = m;
			t = t + m;
		}
		dst[row] = t;
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

namespace {

ConvDiv conv_div(const ConvGeom& g) {
	const unsigned hw = (unsigned)(g.ho * g.wo);
	ConvDiv d;
	d.hw4 = make_fastdiv(hw / 4 > 0 ? hw / 4 : 1);
	d.k = make_fastdiv((unsigned)(g.cin * g.kh * g.kw));
	d.khkw = make_fastdiv((unsigned)(g.kh * g.kw));
	d.kw = make_fastdiv((unsigned)g.kw);
	d.wo = make_fastdiv((unsigned)g.wo);
	d.w = make_fastdiv((unsigned)g.w);
	d.h = make_fastdiv((unsigned)g.h);
	d.cin = make_fastdiv((unsigned)g.cin);
	d.stride = make_fastdiv((unsigned)g.stride);
	return d;
}

constexpr int64_t kFast = (int64_t)1 << 31;  // the 32-bit index kernels take fewer elements than this

}  // namespace

hipError_t im2col(const float* x, float* col, const ConvGeom& g, int64_t samples, hipStream_t s) {
	const int64_t hw = (int64_t)g.ho * g.wo;
	const int64_t total = samples * g.cin * g.kh * g.kw * hw;
	if (total == 0) return hipSuccess;
	if (hw % 4 == 0 && total < kFast && reinterpret_cast<uintptr_t>(col) % 16 == 0) {
		const unsigned total4 = (unsigned)(total / 4);
		hipLaunchKernelGGL(im2col_quad_kernel, dim3(blocks_for(total4)), dim3(256), 0, s, x, col, g, conv_div(g), total4);
	} else {
		hipLaunchKernelGGL(im2col_kernel, dim3(blocks_for(total)), dim3(256), 0, s, x, col, g, total);
	}
	return hipGetLastError();
}

hipError_t col2im(const float* col, float* dx, const ConvGeom& g, int64_t samples, int first, hipStream_t s) {
	const int64_t total = samples * g.cin * (int64_t)g.h * g.w;
	if (total == 0) return hipSuccess;
	if (total < kFast && samples * g.cin * g.kh * g.kw * (int64_t)g.ho * g.wo < kFast)
		hipLaunchKernelGGL(col2im_fast_kernel, dim3(blocks_for(total)), dim3(256), 0, s, col, dx, g, conv_div(g),
		                   (unsigned)total, first);
	else
		hipLaunchKernelGGL(col2im_kernel, dim3(blocks_for(total)), dim3(256), 0, s, col, dx, g, total, first);
	return hipGetLastError();
}

namespace {

constexpr int kQuadMaxRows = 8;

template <int CG, int PAD, int ROWS>
hipError_t launch_quad_rows(const float* x, const float* w, const float* bias, float* y, unsigned char* alive,
                            unsigned char* bits, const ConvGeom& g, int total_quads, int cout, int relu, hipStream_t s) {
	if constexpr (ROWS * (2 * PAD + 1) > 32) {
		return hipErrorInvalidValue;
	} else {
		dim3 grid(blocks_for(total_quads), (unsigned)((cout + CG - 1) / CG));
		hipLaunchKernelGGL((conv_same_quad_kernel<CG, PAD, ROWS>), grid, dim3(256), 0, s, x, w, bias, y, alive, bits, g,
		                   make_fastdiv((unsigned)(g.wo / 4)), make_fastdiv((unsigned)g.ho), make_fastdiv((unsigned)g.kh),
		                   cout, relu, total_quads);
		return hipGetLastError();
	}
}

template <int CG, int PAD>
hipError_t launch_quad_pad(const float* x, const float* w, const float* bias, float* y, unsigned char* alive,
                           unsigned char* bits, const ConvGeom& g, int total_quads, int cout, int relu, hipStream_t s) {
	switch (g.cin * g.kh) {
		case 1: return launch_quad_rows<CG, PAD, 1>(x, w, bias, y, alive, bits, g, total_quads, cout, relu, s);
		case 2: return launch_quad_rows<CG, PAD, 2>(x, w, bias, y, alive, bits, g, total_quads, cout, relu, s);
		case 3: return launch_quad_rows<CG, PAD, 3>(x, w, bias, y, alive, bits, g, total_quads, cout, relu, s);
		case 4: return launch_quad_rows<CG, PAD, 4>(x, w, bias, y, alive, bits, g, total_quads, cout, relu, s);
		case 5: return launch_quad_rows<CG, PAD, 5>(x, w, bias, y, alive, bits, g, total_quads, cout, relu, s);
		case 6: return launch_quad_rows<CG, PAD, 6>(x, w, bias, y, alive, bits, g, total_quads, cout, relu, s);
		case 7: return launch_quad_rows<CG, PAD, 7>(x, w, bias, y, alive, bits, g, total_quads, cout, relu, s);
		case 8: return launch_quad_rows<CG, PAD, 8>(x, w, bias, y, alive, bits, g, total_quads, cout, relu, s);
		default: return hipErrorInvalidValue;
	}
}

template <int CG>
hipError_t launch_same_quad(const float* x, const float* w, const float* bias, float* y, unsigned char* alive,
                            unsigned char* bits, const ConvGeom& g, int total_quads, int cout, int relu, hipStream_t s) {
	switch (g.pad) {
		case 0: return launch_quad_pad<CG, 0>(x, w, bias, y, alive, bits, g, total_quads, cout, relu, s);
		case 1: return launch_quad_pad<CG, 1>(x, w, bias, y, alive, bits, g, total_quads, cout, relu, s);
		case 2: return launch_quad_pad<CG, 2>(x, w, bias, y, alive, bits, g, total_quads, cout, relu, s);
		case 3: return launch_quad_pad<CG, 3>(x, w, bias, y, alive, bits, g, total_quads, cout, relu, s);
		case 4: return launch_quad_pad<CG, 4>(x, w, bias, y, alive, bits, g, total_quads, cout, relu, s);
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
                          const ConvGeom& g, int64_t samples, int cout, int relu, int cg, hipStream_t s,
                          unsigned char* bits) {
	const int total_quads = (int)(samples * g.ho * (int64_t)(g.wo / 4));
	if (total_quads == 0 || cout == 0) return hipSuccess;
	if (bits && (!relu || ((int64_t)g.ho * g.wo) % 8 != 0)) return hipErrorInvalidValue;
	switch (cg) {
		case 4: return launch_same_quad<4>(x, w, bias, y, alive, bits, g, total_quads, cout, relu, s);
		case 8: return launch_same_quad<8>(x, w, bias, y, alive, bits, g, total_quads, cout, relu, s);
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
	if (total % 4 == 0 && total < kFast && reinterpret_cast<uintptr_t>(g) % 16 == 0 &&
	    reinterpret_cast<uintptr_t>(out) % 16 == 0 && reinterpret_cast<uintptr_t>(alive) % 4 == 0) {
		const unsigned total4 = (unsigned)(total / 4);
		hipLaunchKernelGGL(mask4_kernel, dim3(blocks_for(total4)), dim3(256), 0, s, g,
		                   reinterpret_cast<const unsigned*>(alive), out, total4);
	} else {
		hipLaunchKernelGGL(mask_kernel, dim3(blocks_for(total)), dim3(256), 0, s, g, alive, out, total);
	}
	return hipGetLastError();
}

hipError_t masked_lane_sums(const float* g, const unsigned char* alive, float* out, int64_t rows, int64_t n, float* dst,
                            hipStream_t s) {
	if (rows == 0) return hipSuccess;
	if (rows * 8 >= kFast || n >= kFast || rows * n >= kFast) {  // the two passes, with 64-bit indexing
		hipError_t e = mask_grad(g, alive, out, rows * n, s);
		return e != hipSuccess ? e : lane_sums(out, rows, n, dst, s);
	}
	hipLaunchKernelGGL(mask_lane_sum8_kernel, dim3(blocks_for(rows * 8)), dim3(256), 0, s, g, alive, out, (unsigned)rows,
	                   (int)n, dst);
	return hipGetLastError();
}

hipError_t lane_sums(const float* src, int64_t rows, int64_t n, float* dst, hipStream_t s) {
	if (rows == 0) return hipSuccess;
	if (rows * 8 < kFast && n < kFast)
		hipLaunchKernelGGL(lane_sum8_kernel, dim3(blocks_for(rows * 8)), dim3(256), 0, s, src, (unsigned)rows, (int)n, dst);
	else
		hipLaunchKernelGGL(lane_sum_kernel, dim3(blocks_for(rows)), dim3(256), 0, s, src, rows, n, dst);
	return hipGetLastError();
}

}  // namespace nnh
