// conv_dwp.hip - per-sample bias and weight gradients of a convolution with a short column depth (K = Cin*kh*kw
// <= 16: a network's first layer, one input channel and 3 x 3 taps) on planes of up to 1024 output positions
// (ops.cpp:1436-1449).
//
// The reference computes, per sample n: the masked gradient g' = alive ? g : 0 (1439-1443), db_n[c] = lane_sum of
// row c of g' (1445), and dW_n = g' col_n^T through sgemm(F, T, Cout, K, hw) (1448-1449): each element the fma chain
// over the hw output positions in order from +0 (no depth cut at these sizes; the caller checks). With K this short
// the product is a few hundred chains of ~800 steps per sample, so an MFMA tile would spend its time waiting on its
// own 44-cycle chain steps; here each chain is one lane's v_fma_f32 sequence over LDS:
//   * a workgroup owns one sample and 8 output channels: it stages the channels' masked gradient rows (16-byte
//     coalesced loads of g and 4-byte loads of the flags), the sample's input and, from it, the sample's K im2col
//     columns (zeros in the padding) in LDS;
//   * waves 0-1: lane c*K + k runs dW_n[c][k]'s chain, reading g'[c][p] and col[k][p] sixteen positions at a time,
//     the next 48 in flight while it multiplies and adds the current ones (the chain is otherwise bound by the LDS
//     read latency, not by the fma's);
//   * wave 2: two lanes per channel c run lane_sum's eight partial chains over g'[c] (four each, from 16-byte
//     reads), combine them as ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)) and add the tail.
// Row pitches keep the lanes of one LDS read on distinct banks: g' rows 8 mod 64 apart (8 channels), column rows
// 4 mod 64 apart (up to 16 taps). The per-sample results go to the workspace; the caller adds them over the
// samples in order, as the reference does (1461-1462). The masked gradient is not written out: the dx kernel masks
// on the fly.
#include "conv.hpp"

#include "fastdiv.hpp"
#include "gemm.hpp"

namespace nnh {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kPwThreads = 256;
constexpr int kPwCg = 8;          // output channels per workgroup
constexpr int kPwMaxK = 16;       // K <= 16: kPwCg * K <= 128 dW chains (waves 0-1)
constexpr int kPwMaxHw = 1024;
constexpr int kPwMaxLds = 96 * 1024;

inline int pw_gpitch(int hw) { return (hw + 63) / 64 * 64 + 8; }
inline int pw_cpitch(int hw) { return (hw + 63) / 64 * 64 + 4; }
inline size_t pw_lds_bytes(int hw, int K, int64_t x_plane) {
	// at least one float for the plane: the column build reads element 0 of an empty plane (and discards it)
	return ((size_t)kPwCg * pw_gpitch(hw) + (size_t)K * pw_cpitch(hw) + (size_t)(x_plane > 0 ? x_plane : 1)) *
	       sizeof(float);
}

struct PwArgs {
	const float* g;
	const unsigned char* alive;  // null: no folded ReLU
	const float* x;
	float* gb;                   // [N][Cout] per-sample bias sums, or null
	float* gw;                   // [N][Cout][K] per-sample weight gradients
	ConvGeom geo;
	int cout, groups, K, hw, gpitch, cpitch, vec;
	FastDiv hw_div, hw4_div, khkw_div, kw_div, ho_div;
};

__global__ void __launch_bounds__(kPwThreads) conv_dwp_kernel(const PwArgs a) {
	extern __shared__ __align__(16) float sm[];
	const int tid = threadIdx.x;
	const ConvGeom& G = a.geo;
	const int n = blockIdx.x / a.groups, grp = blockIdx.x - n * a.groups;
	const int c0 = grp * kPwCg, nc = min(kPwCg, a.cout - c0);
	const int hw = a.hw, K = a.K;
	float* gs = sm;                       // [kPwCg][gpitch]: masked gradient rows
	float* cs = sm + kPwCg * a.gpitch;    // [K][cpitch]: the sample's im2col columns

	// 0. the first batch of the sample's input x_n, loaded now so that its loads and the gradient rows' are in flight
	// together (stored to LDS in step 2)
	const float* xs = a.x + (int64_t)n * G.cin * G.h * G.w;
	const int xtot = G.cin * G.h * G.w;
	float xv[8];
	if (xtot > 0) {  // an empty plane (H or W = 0, outputs from the padding alone) has no x to read
#pragma unroll
		for (int u = 0; u < 8; ++u) xv[u] = xs[min(tid + kPwThreads * u, xtot - 1)];
	}

	// 1. masked gradient rows c0 .. c0 + nc - 1 of sample n: one contiguous block of nc * hw
	const int64_t row0 = (int64_t)n * a.cout + c0;
	const float* gsrc = a.g + row0 * hw;
	const unsigned char* asrc = a.alive ? a.alive + row0 * hw : nullptr;
	const int tot = nc * hw;
	if (a.vec) {
		const int q4 = hw >> 2, t4 = tot >> 2;
		for (int b = 0; b < t4; b += kPwThreads * 8) {
			f32x4 v[8];
			unsigned f[8];
#pragma unroll
			for (int u = 0; u < 8; ++u) {
				const int q = min(b + tid + kPwThreads * u, t4 - 1);
				v[u] = *reinterpret_cast<const f32x4*>(gsrc + 4 * q);
				f[u] = asrc ? *reinterpret_cast<const unsigned*>(asrc + 4 * q) : 0x01010101u;
			}
#pragma unroll
			for (int u = 0; u < 8; ++u) {
				const int q = b + tid + kPwThreads * u;
				if (q < t4) {
					const int r = (int)fdiv((unsigned)q, a.hw4_div), p = 4 * (q - r * q4);
#pragma unroll
					for (int i = 0; i < 4; ++i) gs[r * a.gpitch + p + i] = ((f[u] >> (8 * i)) & 0xffu) ? v[u][i] : 0.0f;
				}
			}
		}
	} else {
		for (int e = tid; e < tot; e += kPwThreads) {
			const int r = (int)fdiv((unsigned)e, a.hw_div), p = e - r * hw;
			const float v = gsrc[e];
			gs[r * a.gpitch + p] = (!asrc || asrc[e]) ? v : 0.0f;
		}
	}
	// 2. the sample's input x_n into LDS (the first batch loaded in step 0; every load of a batch issued before its
	// stores)
	float* xl = cs + K * a.cpitch;  // [cin][h][w]
	{
		for (int b = 0; b < xtot; b += kPwThreads * 8) {
			if (b > 0) {
#pragma unroll
				for (int u = 0; u < 8; ++u) xv[u] = xs[min(b + tid + kPwThreads * u, xtot - 1)];
			}
#pragma unroll
			for (int u = 0; u < 8; ++u)
				if (b + tid + kPwThreads * u < xtot) xl[b + tid + kPwThreads * u] = xv[u];
		}
	}
	__syncthreads();
	// 3. the sample's im2col columns (ops.cpp:188-212) from it: col[k][p], k = (ci, ph, pw), p = (oh, ow), 0 in the
	// padding
	{
		// a thread per (k, oh): one output row of column k, its reads batched eight at a time
		const int pairs = K * G.ho, khkw = G.kh * G.kw;
		for (int pr = tid; pr < pairs; pr += kPwThreads) {
			const int k = (int)fdiv((unsigned)pr, a.ho_div), oh = pr - k * G.ho;
			const int ci = (int)fdiv((unsigned)k, a.khkw_div), t = k - ci * khkw;
			const int ph = (int)fdiv((unsigned)t, a.kw_div), pw = t - ph * G.kw;
			const int ih = oh * G.stride - G.pad + ph;
			const bool row_in = ih >= 0 && ih < G.h;
			const float* xrow = xl + ci * G.h * G.w + (row_in ? ih * G.w : 0);
			float* dst = cs + k * a.cpitch + oh * G.wo;
			for (int ow0 = 0; ow0 < G.wo; ow0 += 8) {
				float v[8];
				bool in[8];
#pragma unroll
				for (int u = 0; u < 8; ++u) {
					const int iw = (ow0 + u) * G.stride - G.pad + pw;
					in[u] = row_in && iw >= 0 && iw < G.w;
					v[u] = xrow[in[u] ? iw : 0];
				}
#pragma unroll
				for (int u = 0; u < 8; ++u)
					if (ow0 + u < G.wo) dst[ow0 + u] = in[u] ? v[u] : 0.0f;
			}
		}
	}
	__syncthreads();

	const int nb = hw >> 4;  // whole batches of 16 positions
	if (tid < 2 * 64) {
		// 3. dW_n[c][k] = sum over p of g'[c][p] col[k][p], one fma chain per lane from +0
		const int c = tid / K, k = tid - c * K;
		if (c < nc) {
			const float* gr = gs + c * a.gpitch;
			const float* cr = cs + k * a.cpitch;
			float acc = 0.0f;
			// a ring of four batches of 16 positions: three batches' LDS reads are in flight while one batch's fmas
			// run (every read unconditional, at a batch index clamped into range; the remainder after the last
			// whole group of four is already in the ring)
			float g0[16], c0v[16], g1[16], c1v[16], g2[16], c2v[16], g3[16], c3v[16];
			auto load = [&](float (&gx)[16], float (&cx)[16], int b) {  // 16-byte LDS reads (rows 16-byte aligned)
#pragma unroll
				for (int q = 0; q < 4; ++q) {
					const f32x4 gv = *reinterpret_cast<const f32x4*>(gr + 16 * b + 4 * q);
					const f32x4 cv = *reinterpret_cast<const f32x4*>(cr + 16 * b + 4 * q);
#pragma unroll
					for (int i = 0; i < 4; ++i) {
						gx[4 * q + i] = gv[i];
						cx[4 * q + i] = cv[i];
					}
				}
			};
			auto fmas = [&](const float (&gx)[16], const float (&cx)[16]) {
#pragma unroll
				for (int u = 0; u < 16; ++u) acc = __builtin_fmaf(gx[u], cx[u], acc);
			};
			if (nb > 0) {
				load(g0, c0v, 0);
				load(g1, c1v, min(1, nb - 1));
				load(g2, c2v, min(2, nb - 1));
				int b = 0;
				for (; b + 4 <= nb; b += 4) {
					load(g3, c3v, min(b + 3, nb - 1));
					fmas(g0, c0v);
					load(g0, c0v, min(b + 4, nb - 1));
					fmas(g1, c1v);
					load(g1, c1v, min(b + 5, nb - 1));
					fmas(g2, c2v);
					load(g2, c2v, min(b + 6, nb - 1));
					fmas(g3, c3v);
				}
				if (b < nb) fmas(g0, c0v);
				if (b + 1 < nb) fmas(g1, c1v);
				if (b + 2 < nb) fmas(g2, c2v);
			}
			for (int p = 16 * nb; p < hw; ++p) acc = __builtin_fmaf(gr[p], cr[p], acc);
			a.gw[(row0 + c) * K + k] = acc;
		}
	} else if (tid < 2 * 64 + 2 * kPwCg && a.gb) {
		// 4. db_n[c] = lane_sum(g'[c]) (ops.cpp:804-812): lanes 2c and 2c + 1 of wave 2 hold the reference's
		// partials a[0..3] and a[4..7] of channel c (elements 8i + 4h + q), read 16 bytes at a time; lane 2c combines
		// them as ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)) and adds the tail
		const int l = tid - 2 * 64, c = l >> 1, h = l & 1;
		const int full = hw & ~7;
		const float* gr = gs + c * a.gpitch + 4 * h;
		float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f;
		int i = 0;
		for (; i + 8 * 7 < full; i += 8 * 8) {
			f32x4 v[8];
#pragma unroll
			for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const f32x4*>(gr + i + 8 * u);
#pragma unroll
			for (int u = 0; u < 8; ++u) {
				p0 = p0 + v[u][0];
				p1 = p1 + v[u][1];
				p2 = p2 + v[u][2];
				p3 = p3 + v[u][3];
			}
		}
		for (; i < full; i += 8) {
			const f32x4 v = *reinterpret_cast<const f32x4*>(gr + i);
			p0 = p0 + v[0];
			p1 = p1 + v[1];
			p2 = p2 + v[2];
			p3 = p3 + v[3];
		}
		const int other = (l | 1);
		const float q0 = __shfl(p0, other), q1 = __shfl(p1, other), q2 = __shfl(p2, other), q3 = __shfl(p3, other);
		if (h == 0 && c < nc) {
			float t = ((p0 + p1) + (p2 + p3)) + ((q0 + q1) + (q2 + q3));
			for (int p = full; p < hw; ++p) t = t + gr[p];
			a.gb[row0 + c] = t;
		}
	}
}

}  // namespace

bool conv_dwp_ok(const ConvGeom& g, int64_t samples, int cout) {
	const int64_t hw = (int64_t)g.ho * g.wo, K = (int64_t)g.cin * g.kh * g.kw;
	if (cout < 1 || hw < 1 || hw > kPwMaxHw || K < 1 || K > kPwMaxK) return false;
	if (pw_lds_bytes((int)hw, (int)K, (int64_t)g.cin * g.h * g.w) > (size_t)kPwMaxLds) return false;
	const int64_t groups = (cout + kPwCg - 1) / kPwCg;
	if (samples * groups >= ((int64_t)1 << 31)) return false;
	// the reference's dW_n product sgemm(F, T, Cout, K, hw) (ops.cpp:1449) is one chain per element only without
	// a depth cut (in either numerics mode)
	return !depth_cut(cout, K, hw);
}

hipError_t conv_dwp(const float* g, const unsigned char* alive, const float* x, float* gb, float* gw,
                    const ConvGeom& geo, int64_t samples, int cout, hipStream_t s) {
	if (!conv_dwp_ok(geo, samples, cout)) return hipErrorInvalidValue;
	PwArgs a;
	a.g = g;
	a.alive = alive;
	a.x = x;
	a.gb = gb;
	a.gw = gw;
	a.geo = geo;
	a.cout = cout;
	a.groups = (cout + kPwCg - 1) / kPwCg;
	a.hw = geo.ho * geo.wo;
	a.K = geo.cin * geo.kh * geo.kw;
	a.gpitch = pw_gpitch(a.hw);
	a.cpitch = pw_cpitch(a.hw);
	a.vec = a.hw % 4 == 0 && reinterpret_cast<uintptr_t>(g) % 16 == 0 &&
	        (!alive || reinterpret_cast<uintptr_t>(alive) % 4 == 0);
	a.hw_div = make_fastdiv((unsigned)a.hw);
	a.hw4_div = make_fastdiv((unsigned)(a.hw / 4 > 0 ? a.hw / 4 : 1));
	a.khkw_div = make_fastdiv((unsigned)(geo.kh * geo.kw));
	a.kw_div = make_fastdiv((unsigned)geo.kw);
	a.ho_div = make_fastdiv((unsigned)geo.ho);
	const size_t lds = pw_lds_bytes(a.hw, a.K, (int64_t)geo.cin * geo.h * geo.w);
	hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(conv_dwp_kernel),
	                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
	if (e != hipSuccess) return e;
	hipLaunchKernelGGL(conv_dwp_kernel, dim3((unsigned)(samples * a.groups)), dim3(kPwThreads), lds, s, a);
	return hipGetLastError();
}

}  // namespace nnh
