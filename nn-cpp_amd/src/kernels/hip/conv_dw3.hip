// conv_dw3.hip - the per-sample weight gradients of nn::conv2d for 3x3 kernels, stride 1, padding 1, on planes of
// up to 14 x 14 (src/autograd/ops.cpp:1448-1449), as MFMA chains over operands held in LDS.
//
// The reference computes, per sample, dW_n = g_n col_n^T (sgemm F,T): each element dW_n[co][k] is the fma chain
// over the output positions p = 0..hw-1 in order from +0 of g_n[co][p] * col_n[k][p], with k = (c, ph, pw) and
// col_n[k][p] = x_n[c][oh + ph - 1][ow + pw - 1], or 0 in the padding. The caller then sums dW_n over the samples
// in order. One workgroup here owns one sample, 64 output channels (a last group of 16, 32 or 48 when Cout is not a
// multiple of 64: zero rows past Cout, nothing written for them) and half of the 16-wide groups of k:
//   * the sample's (masked) gradient rows, [64][197], and its zero-padded input, [Cin][16][19], go to LDS;
//   * the 64 channels are the A operand of 16x16x1 MFMA units (lane l: channel l), one unit per 16 values of k
//     (lane l: k = 16 u + (l & 15), whose window offset c*304 + ph*19 + pw is fixed per lane), at most three units
//     per wave;
//   * step p = (oh, ow) reads g at [l][p] and the input at window offset + oh*19 + ow: output rows run as a loop,
//     the row's columns unrolled, so every LDS read has an immediate offset from a per-row base.
// Same bits as the batched GEMM with gathered columns; the result goes to the same per-sample buffer. The kernel
// also applies the forward's ReLU mask to the gradient as it stages it (writing the masked gradient out once, for
// the input gradient) and takes the per-sample bias gradients from the masked rows in LDS, so the backward needs
// no separate pass over the gradient for them.
#include "conv.hpp"

#include <algorithm>
#include <mutex>

#include "gemm.hpp"
#include "gemm_tile.hpp"

namespace nnh {

namespace {

constexpr int kD3Pad = 16;                 // padded plane width and height
constexpr int kD3Row = 19;                 // LDS row stride of the padded plane
constexpr int kD3Plane = kD3Pad * kD3Row;  // LDS plane stride: 16 x 19 (see below)
// The 16 lanes of a k group read taps (ph, pw) of one to three channels: with rows of 19 floats and planes of 304
// their addresses fall in 16 different banks for every depth (checked for K = 9 ... 378), where rows of 16 and
// planes of 256 gave four-way conflicts.
constexpr int kD3Co = 64;                  // output channels per workgroup (the MFMA A operand)
constexpr int kD3GLd = 197;                // LDS row stride of the gradient rows (odd: conflict-free column reads)
constexpr int kD3MaxW = 14;
constexpr int kD3Units = 3;                // 16-wide k groups per wave
constexpr int kD3MaxLds = 160 * 1024;
constexpr int kD3GQ = 13;                  // 16-byte groups of a gradient row per thread: 4 * 13 * 4 >= 196

using M16 = Mfma<kMf16>;

struct D3Args {
	const float* g;                // output gradient {N, Cout, hw}
	const unsigned char* alive;    // the forward's ReLU mask {N, Cout, hw}, or null: no mask
	float* gmo;                    // the masked gradient, written when alive is given
	float* gb;                     // per-sample bias gradients {N, Cout} (lane sums of the masked rows), or null
	const float* x;                // {N, Cin, H, W}
	float* gw;                     // per-sample weight gradients {N, Cout, K}
	int cin, height, width, cout, cogroups, khalf;  // khalf: 16-wide k groups per workgroup
	int pairs;            // (sample, channel group) pairs = workgroups / 2
};

// Workgroup id -> (half, pair): ids are taken in groups of 16, whose first 8 are half 0 and last 8 half 1 of the
// same 8 pairs, so the two halves of a pair share id modulo 8 (the XCD). A last, partial group of 2r ids holds r
// pairs the same way.
__device__ __forceinline__ void d3_unmap(int b, int pairs, int& half, int& pair) {
	const int grp = b >> 4, in = b & 15;
	const int full = pairs >> 3;  // complete groups of 8 pairs
	if (grp < full) {
		half = in >> 3;
		pair = grp * 8 + (in & 7);
	} else {
		const int r = pairs - full * 8;  // pairs in the partial group
		half = in >= r ? 1 : 0;
		pair = full * 8 + (in - half * r);
	}
}

template <int CX, int WC>  // most input channels; the plane width
__global__ void __launch_bounds__(256) conv_dw3_kernel(const D3Args a) {
	extern __shared__ __align__(16) float sm[];
	const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
	const int K = a.cin * 9, hw = a.height * a.width;
	// blocks b and b + 8 are the two halves of one (sample, channel group): workgroups are dispatched to the 8
	// XCDs by id modulo 8, so both read the sample's rows through one XCD's L2 (d3_unmap)
	int half, rest;
	d3_unmap(blockIdx.x, a.pairs, half, rest);
	const int n = rest / a.cogroups, co0 = (rest - n * a.cogroups) * kD3Co;
	float* gs = sm;                      // [64][kD3GLd]
	float* xs = sm + kD3Co * kD3GLd;     // [cin][16][19], zero outside the image
	const float* xn = a.x + (int64_t)n * a.cin * hw;

	// staging: every load issued (indices clamped into range) before the stores.
	//   padded input: slot u of thread t is channel u at padded row t >> 4, column t & 15 (fixed per thread, so
	//   its source offset and whether it lies in the image are computed once);
	//   gradient rows: thread t covers channel t >> 2 and its 16-byte groups (t & 3) + 4 j (hw % 4 == 0), masked
	//   here by the ReLU's alive bytes (ops.cpp:1439-1443); the half that owns the channel also writes the masked
	//   row out for the input gradient.
	// a last group of fewer than 64 channels (Cout a multiple of 16) stages zero rows past Cout, from clamped
	// addresses, and writes nothing for them
	const int gco = tid >> 2, ngq = hw >> 2;
	const bool glive = co0 + gco < a.cout;
	const int64_t grow = ((int64_t)n * a.cout + co0 + min(gco, a.cout - 1 - co0)) * hw;  // this thread's gradient row
	{
		const int r = tid >> 4, q = tid & 15, ih = r - 1, iw = q - 1;
		const bool in = ih >= 0 && ih < a.height && iw >= 0 && iw < a.width;
		const int src = min(max(ih, 0), a.height - 1) * a.width + min(max(iw, 0), a.width - 1);
		float xv[CX];
		f32x4 gv[kD3GQ];
		unsigned al[kD3GQ];
#pragma unroll
		for (int u = 0; u < CX; ++u) xv[u] = xn[min(u, a.cin - 1) * hw + src];
#pragma unroll
		for (int j = 0; j < kD3GQ; ++j)
			gv[j] = *reinterpret_cast<const f32x4*>(a.g + grow + 4 * min((tid & 3) + 4 * j, ngq - 1));
		if (a.alive) {
#pragma unroll
			for (int j = 0; j < kD3GQ; ++j)
				al[j] = *reinterpret_cast<const unsigned*>(a.alive + grow + 4 * min((tid & 3) + 4 * j, ngq - 1));
#pragma unroll
			for (int j = 0; j < kD3GQ; ++j)
#pragma unroll
				for (int e = 0; e < 4; ++e) gv[j][e] = ((al[j] >> (8 * e)) & 0xffu) ? gv[j][e] : 0.0f;
		}
		if (!glive) {
#pragma unroll
			for (int j = 0; j < kD3GQ; ++j) gv[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
		}
#pragma unroll
		for (int u = 0; u < CX; ++u)
			if (u < a.cin) xs[u * kD3Plane + r * kD3Row + q] = in ? xv[u] : 0.0f;
		const bool out = a.alive && (gco >> 5) == half && glive;  // uniform per wave (Cout is a multiple of 16)
#pragma unroll
		for (int j = 0; j < kD3GQ; ++j) {
			const int gq = (tid & 3) + 4 * j;
			if (gq < ngq) {
#pragma unroll
				for (int e = 0; e < 4; ++e) gs[gco * kD3GLd + 4 * gq + e] = gv[j][e];
				if (out) *reinterpret_cast<f32x4*>(a.gmo + grow + 4 * gq) = gv[j];
			}
		}
	}
	__syncthreads();

	// this wave's k groups: u_w = wave + 4 i (i < kD3Units) among the workgroup's khalf groups. Every wave runs
	// kD3Units chains (the unused ones on clamped, valid addresses, never stored), so the loop has no branch; the
	// waves with the most groups set the time either way.
	const int g0 = half * a.khalf;
	const int nunits_w = min(kD3Units, max(0, (a.khalf - wave + 3) / 4));
	// the per-sample bias gradients of this half's 32 channels, lane_sum (ops.cpp:804-812, 1445) of the masked
	// rows in LDS with eight lanes per row: lane k folds elements k, k + 8, ... of the full groups of eight in
	// order from +0; the row's first lane combines the eight as ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7))
	// and adds the tail in order
	auto bias_sums = [&]() {
		if (!a.gb) return;
		const int row = 32 * half + (tid >> 3), k = tid & 7;
		const float* pr = gs + row * kD3GLd;
		const int full = hw & ~7;
		float t = 0.0f;
#pragma unroll 8
		for (int i = k; i < full; i += 8) t = t + pr[i];
		float part[8];
#pragma unroll
		for (int j = 0; j < 8; ++j) part[j] = __shfl(t, (lane & ~7) + j);
		if (k == 0 && co0 + row < a.cout) {
			float v = ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
			for (int i = full; i < hw; ++i) v = v + pr[i];
			a.gb[(int64_t)n * a.cout + co0 + row] = v;
		}
	};
	if (nunits_w == 0) {  // uniform
		bias_sums();
		return;
	}
	int xoff[kD3Units];
#pragma unroll
	for (int i = 0; i < kD3Units; ++i) {
		const int k = min((g0 + wave + 4 * i) * 16 + M16::bcol(lane), K - 1);
		const int c = k / 9, t = k - c * 9;
		xoff[i] = c * kD3Plane + (t / 3) * kD3Row + (t % 3);
	}
	const float* gl = gs + M16::arow(lane) * kD3GLd;
	M16::Acc acc[kD3Units];
#pragma unroll
	for (int i = 0; i < kD3Units; ++i)
#pragma unroll
		for (int r = 0; r < M16::NV; ++r) acc[i][r] = 0.0f;

	// the chain over p = (oh, ow) in order. A row's operands are read a row ahead, each position's reads issued
	// right after the MFMAs of the same position of the row before, so the LDS reads interleave with the MFMAs
	// (a wait only covers reads issued some positions earlier).
	float av[2][WC], bv[2][WC][kD3Units];
	auto read_at = [&](int oh, int ow, int sl) {
		av[sl][ow] = gl[oh * WC + ow];
#pragma unroll
		for (int i = 0; i < kD3Units; ++i) bv[sl][ow][i] = xs[xoff[i] + oh * kD3Row + ow];
	};
	auto mma_at = [&](int ow, int sl) {
#pragma unroll
		for (int i = 0; i < kD3Units; ++i) acc[i] = M16::mma(av[sl][ow], bv[sl][ow][i], acc[i]);
	};
	// the MFMAs of row slot sl with the reads of row next into the other slot
	auto step_row = [&](int sl, int next) {
#pragma unroll
		for (int ow = 0; ow < WC; ++ow) {
			mma_at(ow, sl);
			read_at(next, ow, sl ^ 1);
		}
#pragma unroll
		for (int ow = 0; ow < WC; ++ow) {
			__builtin_amdgcn_sched_group_barrier(0x008, kD3Units, 0);      // MFMA
			__builtin_amdgcn_sched_group_barrier(0x100, 1 + kD3Units, 0);  // LDS read
		}
		__builtin_amdgcn_sched_barrier(0);
	};
#pragma unroll
	for (int ow = 0; ow < WC; ++ow) read_at(0, ow, 0);
	int oh = 0;
	for (; oh + 2 <= a.height; oh += 2) {
		step_row(0, oh + 1);
		step_row(1, min(oh + 2, a.height - 1));  // past the last row: a valid row, not used
	}
	if (oh < a.height) {
#pragma unroll
		for (int ow = 0; ow < WC; ++ow) mma_at(ow, 0);
	}

	// dW_n[co][k]: co = crow(r, lane), k = 16 u + ccol(lane)
	float* gwn = a.gw + ((int64_t)n * a.cout + co0) * K;
#pragma unroll
	for (int i = 0; i < kD3Units; ++i) {
		if (i >= nunits_w) continue;
		const int k = (g0 + wave + 4 * i) * 16 + M16::ccol(lane);
		if (k >= K) continue;
#pragma unroll
		for (int r = 0; r < M16::NV; ++r)
			if (co0 + M16::crow(r, lane) < a.cout) gwn[(int64_t)M16::crow(r, lane) * K + k] = acc[i][r];
	}
	bias_sums();
}

using KernelFnD3 = void (*)(const D3Args);

size_t d3_lds_bytes(int cin) { return (size_t)(kD3Co * kD3GLd + cin * kD3Plane) * sizeof(float); }

}  // namespace

bool conv_dw3_ok(const ConvGeom& g, int64_t samples, int cout, const float* gr, const unsigned char* alive,
                 const float* gmo) {
	if (g.kh != 3 || g.kw != 3 || g.stride != 1 || g.pad != 1 || g.h > 14 || g.w > kD3MaxW || g.ho != g.h ||
	    g.wo != g.w)
		return false;
	const int64_t hw = (int64_t)g.h * g.w, K = (int64_t)g.cin * 9;
	if (cout % 16 != 0 || K > 2 * 4 * kD3Units * 16 || samples * ((cout + kD3Co - 1) / kD3Co) * 2 > 0x7fffffff)
		return false;
	// the gradient rows are staged (and the masked rows written) in 16-byte groups, with 4-byte groups of the mask
	if (hw % 4 != 0 || reinterpret_cast<uintptr_t>(gr) % 16 != 0) return false;
	if (alive && (reinterpret_cast<uintptr_t>(alive) % 4 != 0 || !gmo || reinterpret_cast<uintptr_t>(gmo) % 16 != 0))
		return false;
	if (depth_cut(cout, K, hw)) return false;  // the reference splits such products into 128-deep pieces
	return d3_lds_bytes(g.cin) <= (size_t)kD3MaxLds;
}

hipError_t conv_dw3(const float* gr, const unsigned char* alive, float* gmo, float* gb, const float* x, float* gw,
                    const ConvGeom& g, int64_t samples, int cout, hipStream_t s) {
	static std::mutex mu;
	static bool raised[64] = {};
	int dev = 0;
	hipError_t e = hipGetDevice(&dev);
	if (e != hipSuccess) return e;
	if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
	// one kernel per plane width (the row of positions is unrolled) and bound on the input channels
#define NNH_D3(C) {conv_dw3_kernel<C, 1>, conv_dw3_kernel<C, 2>, conv_dw3_kernel<C, 3>, conv_dw3_kernel<C, 4>, \
	conv_dw3_kernel<C, 5>, conv_dw3_kernel<C, 6>, conv_dw3_kernel<C, 7>, conv_dw3_kernel<C, 8>, conv_dw3_kernel<C, 9>, \
	conv_dw3_kernel<C, 10>, conv_dw3_kernel<C, 11>, conv_dw3_kernel<C, 12>, conv_dw3_kernel<C, 13>, conv_dw3_kernel<C, 14>}
	static const KernelFnD3 kernels[2][kD3MaxW] = {NNH_D3(32), NNH_D3(48)};
#undef NNH_D3
	{
		std::lock_guard<std::mutex> lock(mu);
		if (!raised[dev]) {
			for (const auto& row : kernels)
			for (KernelFnD3 fn : row) {
				e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
				                        kD3MaxLds);
				if (e != hipSuccess) return e;
			}
			raised[dev] = true;
		}
	}
	const int K = g.cin * 9;
	const int units = (K + 15) / 16;
	const int cogroups = (cout + kD3Co - 1) / kD3Co;
	const int pairs = (int)(samples * cogroups);
	D3Args a{gr, alive, alive ? gmo : nullptr, gb, x, gw, g.cin, g.h, g.w, cout, cogroups, (units + 1) / 2, pairs};
	static_assert(kD3GQ * 4 * 4 >= 14 * 14, "a thread's groups cover a gradient row of a 14 x 14 plane");
	static_assert(2 * 4 * kD3Units * 16 / 9 <= 48, "every accepted depth has at most 48 input channels");
	hipLaunchKernelGGL(kernels[g.cin <= 32 ? 0 : 1][g.w - 1], dim3((unsigned)(samples * a.cogroups * 2)), dim3(256),
	                   d3_lds_bytes(g.cin), s, a);
	return hipGetLastError();
}

}  // namespace nnh
