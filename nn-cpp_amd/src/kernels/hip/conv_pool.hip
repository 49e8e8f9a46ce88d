// conv_pool.hip - conv2d_relu followed by maxpool2d(2, 2) (src/autograd/ops.cpp:1396-1416, 1609-1684) in one pass
// for a network's first layer: stride 1, "same" geometry (kh = kw = 2 pad + 1, so Ho = H and Wo = W), W a multiple
// of 4, H even, Cin (kh + 1) <= 8 input rows per output row pair.
//
// Each lane owns a quad of columns (ow0 .. ow0 + 3) of two output rows (2 pr and 2 pr + 1) and CG output channels.
// It loads the Cin (kh + 1) input rows the two output rows need, 16 bytes each (all issued before any arithmetic),
// takes the pad columns either side of its quad from the neighbouring lanes (lanes l - 1 and l + 1 own the quads
// before and after it in the same row pair; the first and last lane of a wave load them), and runs each output's
// chain of the reference: fma over k = (ci, ph, pw) in order from +0, padding taps included as fma(w, 0, acc), then
// v = acc + b and the ReLU with its alive flag. It stores y and the flags as the conv does, and from the same
// registers the two 2 x 2 windows of the quad's row pair: the maxpool's four comparisons in the reference's order
// (first maximum wins, from -inf, offset 0 kept when nothing beats it), the maximum and its offset in the (n, c)
// plane. Every value is the bits the two ops give one after the other.
#include <cmath>

#include "conv.hpp"
#include "fastdiv.hpp"

namespace nnh {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Packed outputs (bits and amax2 non-null, alive and argmax null): the flags as one bit per output in y's order
// (bit i of the flattened {N, Cout, H, W} index at byte i / 8, bit i % 8), and each window's maximum as its 2-bit
// position in the window (0 row 0 left, 1 row 0 right, 2 row 1 left, 3 row 1 right) at bits 2 (wc % 4) of byte
// (plane ph2 + pr) rb + wc / 4, a pooled row taking rb = ceil(W / 8) whole bytes. A window's maximum is always one of
// its own elements here (ReLU outputs are never NaN or -inf), so two bits hold the offset. Each byte is written by
// one lane from its own and its neighbours' flags; a wave then holds whole row pairs (lpw lanes, the rest idle), so
// that no byte's parts lie in two waves.
template <int CG, int PAD, int CIN>
__global__ void __launch_bounds__(256) conv_relu_pool2_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                              const float* __restrict__ bias, float* __restrict__ y,
                                                              unsigned char* __restrict__ alive, float* __restrict__ pooled,
                                                              uint32_t* __restrict__ argmax, unsigned char* __restrict__ bits,
                                                              unsigned char* __restrict__ amax2, ConvGeom g, FastDiv qpr,
                                                              FastDiv pairs, int cout, int total, int lpw) {
	constexpr int K = 2 * PAD + 1;  // kh = kw
	constexpr int R = K + 1;        // input rows per channel for two output rows
	constexpr int KK = CIN * K * K;
	const int tid = threadIdx.x;
	const int lane = tid & 63;
	const int q = (blockIdx.x * 4 + (tid >> 6)) * lpw + lane;
	const bool active = lane < lpw && q < total;
	const unsigned qc = active ? q : total - 1;  // inactive lanes still take part in the shuffles
	const unsigned rest = fdiv(qc, qpr);
	const int ow0 = (int)(qc - rest * qpr.d) * 4;
	const unsigned n = fdiv(rest, pairs);
	const int pr = (int)(rest - n * pairs.d);
	const int oh0 = 2 * pr;
	const int c0 = blockIdx.y * CG;
	const bool has_left = ow0 > 0, has_right = ow0 + 4 < g.w;
	const float* __restrict__ xn = x + (int64_t)n * CIN * g.h * g.w;

	f32x4 v[CIN][R];
	int off[CIN][R];
	bool ok[CIN][R];
#pragma unroll
	for (int ci = 0; ci < CIN; ++ci)
#pragma unroll
		for (int r = 0; r < R; ++r) {
			const int ih = oh0 + r - PAD;
			ok[ci][r] = ih >= 0 && ih < g.h;
			off[ci][r] = (ci * g.h + (ok[ci][r] ? ih : 0)) * g.w;
			v[ci][r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
			if (ok[ci][r]) v[ci][r] = *reinterpret_cast<const f32x4*>(xn + off[ci][r] + ow0);
		}

	float acc[2][CG][4];
#pragma unroll
	for (int t = 0; t < 2; ++t)
#pragma unroll
		for (int c = 0; c < CG; ++c)
#pragma unroll
			for (int i = 0; i < 4; ++i) acc[t][c][i] = 0.0f;
#pragma unroll
	for (int ci = 0; ci < CIN; ++ci) {
		// the quad of each input row with its pad columns either side
		float seg[R][4 + 2 * PAD];
#pragma unroll
		for (int r = 0; r < R; ++r) {
#pragma unroll
			for (int i = 0; i < 4; ++i) seg[r][PAD + i] = v[ci][r][i];
#pragma unroll
			for (int e = 0; e < PAD; ++e) {
				float l = __shfl_up(v[ci][r][4 - PAD + e], 1);
				float rr = __shfl_down(v[ci][r][e], 1);
				if (lane == 0 && has_left) l = ok[ci][r] ? xn[off[ci][r] + ow0 - PAD + e] : 0.0f;
				if (lane == lpw - 1 && has_right) rr = ok[ci][r] ? xn[off[ci][r] + ow0 + 4 + e] : 0.0f;
				seg[r][e] = has_left ? l : 0.0f;
				seg[r][PAD + 4 + e] = has_right ? rr : 0.0f;
			}
		}
#pragma unroll
		for (int ph = 0; ph < K; ++ph)
#pragma unroll
			for (int pw = 0; pw < K; ++pw)
#pragma unroll
				for (int c = 0; c < CG; ++c) {
					const float wv = w[min(c0 + c, cout - 1) * KK + (ci * K + ph) * K + pw];
#pragma unroll
					for (int t = 0; t < 2; ++t)
#pragma unroll
						for (int i = 0; i < 4; ++i) acc[t][c][i] = __builtin_fmaf(wv, seg[t + ph][i + pw], acc[t][c][i]);
				}
	}
	const int64_t hw = (int64_t)g.h * g.w;
	const int ph2 = g.h >> 1, pw2 = g.w >> 1;
	const uint32_t base = (uint32_t)(oh0 * g.w + ow0);  // window offsets inside the (n, c) plane
	const int x4 = ow0 >> 2, nq = (int)qpr.d;            // the quad's place in its row, quads per row
#pragma unroll
	for (int c = 0; c < CG; ++c) {
		if (c0 + c >= cout) break;  // uniform: every lane of the wave takes the same channels
		const int64_t plane = (int64_t)n * cout + c0 + c;
		const float b = bias[c0 + c];
		f32x4 out[2];
		unsigned nib[2];
#pragma unroll
		for (int t = 0; t < 2; ++t) {
			unsigned flags = 0;
			nib[t] = 0;
#pragma unroll
			for (int i = 0; i < 4; ++i) {
				float val = acc[t][c][i] + b;
				const bool on = val > 0.0f;
				flags |= (on ? 1u : 0u) << (8 * i);
				nib[t] |= (on ? 1u : 0u) << i;
				out[t][i] = on ? val : 0.0f;
			}
			const int64_t o = plane * hw + (int64_t)(oh0 + t) * g.w + ow0;
			if (active) *reinterpret_cast<f32x4*>(y + o) = out[t];
			if (active && alive) *reinterpret_cast<unsigned*>(alive + o) = flags;
		}
		// the two 2 x 2 windows (pool.hip's order: row 0 left, row 0 right, row 1 left, row 1 right)
		const f32x4 u = out[0], d = out[1];
		float b0 = -INFINITY, b1 = -INFINITY;
		uint32_t t0 = 0, t1 = 0, s0 = 0, s1 = 0;
		if (u[0] > b0) { b0 = u[0]; t0 = base; s0 = 0; }
		if (u[1] > b0) { b0 = u[1]; t0 = base + 1; s0 = 1; }
		if (d[0] > b0) { b0 = d[0]; t0 = base + g.w; s0 = 2; }
		if (d[1] > b0) { b0 = d[1]; t0 = base + g.w + 1; s0 = 3; }
		if (u[2] > b1) { b1 = u[2]; t1 = base + 2; s1 = 0; }
		if (u[3] > b1) { b1 = u[3]; t1 = base + 3; s1 = 1; }
		if (d[2] > b1) { b1 = d[2]; t1 = base + g.w + 2; s1 = 2; }
		if (d[3] > b1) { b1 = d[3]; t1 = base + g.w + 3; s1 = 3; }
		const int64_t po = plane * ph2 * pw2 + (int64_t)pr * pw2 + (ow0 >> 1);
		if (active) *reinterpret_cast<float2*>(pooled + po) = make_float2(b0, b1);
		if (active && argmax) *reinterpret_cast<uint2*>(argmax + po) = make_uint2(t0, t1);
		if (bits) {
			// flag nibbles N0 = (2 pr) nq + x4 (row 0) and N1 = N0 + nq (row 1), plane-relative; the even one of a
			// pair holds the byte. Its partner is the next quad of the row, or for row 0's last quad row 1's first:
			// lanes of the same row pair, so of the same wave
			const unsigned a = __shfl(nib[0], lane + 1);
			const unsigned bsrc = __shfl(nib[1], x4 + 1 < nq ? lane + 1 : lane - (nq - 1));
			const int64_t nb0 = plane * (hw >> 2) + (int64_t)(2 * pr) * nq + x4, nb1 = nb0 + nq;
			if (active && (nb0 & 1) == 0)
				bits[nb0 >> 1] = (unsigned char)(nib[0] | ((x4 + 1 < nq ? a : bsrc) << 4));
			if (active && (nb1 & 1) == 0) bits[nb1 >> 1] = (unsigned char)(nib[1] | (bsrc << 4));
			// window slots: the quad's two windows are a nibble; lanes x4 and x4 + 1 (even x4) share a byte
			const unsigned sn = s0 | (s1 << 2);
			const unsigned sp = __shfl(sn, lane + 1);
			const int rb = (g.w + 7) >> 3;
			if (active && (x4 & 1) == 0)
				amax2[(plane * ph2 + pr) * rb + (x4 >> 1)] = (unsigned char)(sn | (x4 + 1 < nq ? sp << 4 : 0u));
		}
	}
}

constexpr int kCG = 4;

template <int PAD, int CIN>
hipError_t launch(const float* x, const float* w, const float* bias, float* y, unsigned char* alive, float* pooled,
                  uint32_t* argmax, unsigned char* bits, unsigned char* amax2, const ConvGeom& g, int total, int cout,
                  hipStream_t s) {
	// packed outputs: whole row pairs per wave
	const int qpr = g.w / 4, lpw = bits ? (64 / qpr) * qpr : 64;
	const int64_t waves = (total + lpw - 1) / lpw;
	dim3 grid((unsigned)((waves + 3) / 4), (unsigned)((cout + kCG - 1) / kCG));
	hipLaunchKernelGGL((conv_relu_pool2_kernel<kCG, PAD, CIN>), grid, dim3(256), 0, s, x, w, bias, y, alive, pooled,
	                   argmax, bits, amax2, g, make_fastdiv((unsigned)qpr), make_fastdiv((unsigned)(g.h / 2)), cout, total,
	                   lpw);
	return hipGetLastError();
}

}  // namespace

bool conv_relu_pool2_ok(const float* x, const float* y, const unsigned char* alive, const float* pooled,
                        const uint32_t* argmax, const ConvGeom& g, int64_t samples) {
	const bool geom = g.stride == 1 && g.kh == g.kw && g.kw == 2 * g.pad + 1 && (g.pad == 1 || g.pad == 2) &&
	                  g.cin >= 1 && g.cin * (g.kh + 1) <= 8 && g.ho == g.h && g.wo == g.w && g.w % 4 == 0 &&
	                  g.h % 2 == 0 && g.h >= 2;
	const bool aligned = reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0 &&
	                     reinterpret_cast<uintptr_t>(alive) % 4 == 0 && reinterpret_cast<uintptr_t>(pooled) % 8 == 0 &&
	                     reinterpret_cast<uintptr_t>(argmax) % 8 == 0;
	return geom && aligned && samples * (g.h / 2) * (int64_t)(g.w / 4) < (int64_t)1 << 30;
}

hipError_t conv_relu_pool2(const float* x, const float* w, const float* bias, float* y, unsigned char* alive,
                           float* pooled, uint32_t* argmax, const ConvGeom& g, int64_t samples, int cout, hipStream_t s,
                           unsigned char* bits, unsigned char* amax2) {
	const int total = (int)(samples * (g.h / 2) * (int64_t)(g.w / 4));
	if (total == 0 || cout == 0) return hipSuccess;
	if ((bits != nullptr) != (amax2 != nullptr) || (bits && (alive || argmax || g.w > 256))) return hipErrorInvalidValue;
	if (g.pad == 1 && g.cin == 1) return launch<1, 1>(x, w, bias, y, alive, pooled, argmax, bits, amax2, g, total, cout, s);
	if (g.pad == 1 && g.cin == 2) return launch<1, 2>(x, w, bias, y, alive, pooled, argmax, bits, amax2, g, total, cout, s);
	if (g.pad == 2 && g.cin == 1) return launch<2, 1>(x, w, bias, y, alive, pooled, argmax, bits, amax2, g, total, cout, s);
	return hipErrorInvalidValue;
}

}  // namespace nnh
