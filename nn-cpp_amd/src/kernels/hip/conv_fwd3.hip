// conv_fwd3.hip - nn::conv2d / conv2d_relu forward for 3x3 kernels, stride 1, padding 1, on planes of up to
// 14 x 14 (src/autograd/ops.cpp:1345-1410), as MFMA chains over an input held in LDS.
//
// The reference computes, per sample, Y = W col + bias: sgemm F,F over k = Cin*9, each element the fma chain over
// k = (c, ph, pw) in order from +0 with col[k][p] = x[c][oh + ph - 1][ow + pw - 1], or 0 in the padding; then
// Y += bias and, for conv2d_relu, alive = Y > 0, Y = alive ? Y : 0. One workgroup here owns one sample and 32
// output channels:
//   * the sample, zero-padded to [Cin][16][16], and the transposed W rows of its channels, [K][33], go to LDS
//     (every global load of the staging is issued before the first LDS store);
//   * wave w owns output positions 64w..64w+63, the A operand of two 16x16x1 MFMA units (lane l: position
//     64w + l, clamped into the plane); the units' B operands are channels 0-15 and 16-31;
//   * step k = (c, ph, pw) reads the padded input at the lane's window origin + c*256 + ph*16 + pw and W^T[k][ch]:
//     the nine taps are unrolled, so both offsets are immediates and only the channel loop runs; a channel's 27
//     operands are read while the previous channel's MFMAs run;
//   * the epilogue adds the bias, applies the ReLU and writes y and the alive flags four positions per store.
// Each output is the reference's chain, padding taps included as fma(w, 0, acc): the same bits as the
// implicit-im2col GEMM. Taken when the product takes no depth cut and the buffers suit 16-byte stores.
#include "conv.hpp"

#include <algorithm>
#include <mutex>

#include "gemm.hpp"
#include "gemm_tile.hpp"

namespace nnh {

namespace {

constexpr int kF3Pad = 16;               // padded plane width and height
constexpr int kF3Plane = kF3Pad * kF3Pad;
constexpr int kF3Co = 32;                // output channels per workgroup
constexpr int kF3WLd = kF3Co + 1;        // LDS row stride of W^T (odd: conflict-free transposing stores)
constexpr int kF3MaxLds = 160 * 1024;

using M16 = Mfma<kMf16>;

struct F3Args {
	const float* x;        // {N, Cin, H, W}
	const float* w;        // {Cout, Cin*9}
	const float* bias;     // {Cout}
	float* y;              // {N, Cout, H, W}
	unsigned char* alive;  // like y, or null
	int cin, height, width, cout, groups, relu;
	FastDiv spandiv[2];    // division by 9 * (channels in the first half), 9 * (channels in the second half)
};

template <int CH>  // most input channels in one staging half
__global__ void __launch_bounds__(256) conv_fwd3_kernel(const F3Args a) {
	extern __shared__ __align__(16) float sm[];
	const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
	const int n = blockIdx.x / a.groups, co0 = (blockIdx.x - n * a.groups) * kF3Co;
	const int K = a.cin * 9, hw = a.height * a.width;
	float* xs = sm;                       // [cin][16][16], zero outside the image
	float* ws = sm + a.cin * kF3Plane;    // [K][kF3WLd]: ws[k][j] = W[co0 + j][k]
	const float* xn = a.x + (int64_t)n * a.cin * hw;

	// Staging in two halves of the input channels, [0, c1) and [c1, cin): the first half's input values and W rows
	// are loaded and stored, then the second half's loads are issued before the first half's MFMAs and stored
	// after them. Loads use indices clamped into range; input values outside the image become 0.
	const int c1 = (a.cin + 1) / 2;
	const float* wg = a.w + (int64_t)co0 * K;  // the workgroup's W rows, one contiguous block: e = j * K + k
	constexpr int kX = CH, kW = (CH * 9 * kF3Co + 255) / 256;  // per thread and half: input values, W values
	float xv[kX], wv[kW];
	auto load_half = [&](int cb, int ce) {
		const int x0 = cb * kF3Plane, nx = (ce - cb) * kF3Plane;
		const int nw = (ce - cb) * 9 * kF3Co;
#pragma unroll
		for (int u = 0; u < kX; ++u) {
			const int e = x0 + min(tid + 256 * u, nx - 1);
			const int c = e >> 8, ih = ((e >> 4) & 15) - 1, iw = (e & 15) - 1;
			const bool in = ih >= 0 && ih < a.height && iw >= 0 && iw < a.width;
			const float t = xn[(c * a.height + min(max(ih, 0), a.height - 1)) * a.width + min(max(iw, 0), a.width - 1)];
			xv[u] = in ? t : 0.0f;
		}
		// W^T rows k of channels [cb, ce): element (j, k) sits at j * K + k; thread slot e covers j = e / (span),
		// k = cb * 9 + e % span with span = (ce - cb) * 9
#pragma unroll
		for (int u = 0; u < kW; ++u) {
			const int e = min(tid + 256 * u, nw - 1);
			const int j = (int)fdiv((unsigned)e, a.spandiv[cb == 0 ? 0 : 1]), kk = e - j * (ce - cb) * 9;
			wv[u] = wg[j * K + cb * 9 + kk];
		}
	};
	auto store_half = [&](int cb, int ce) {
		const int x0 = cb * kF3Plane, nx = (ce - cb) * kF3Plane;
		const int nw = (ce - cb) * 9 * kF3Co;
		// nx is a multiple of 256, so slot u is in range for every thread exactly when 256 u < nx (uniform); for W
		// the test is uniform whenever the whole round is in range
#pragma unroll
		for (int u = 0; u < kX; ++u)
			if (256 * u < nx) xs[x0 + tid + 256 * u] = xv[u];
#pragma unroll
		for (int u = 0; u < kW; ++u) {
			const int e = tid + 256 * u;
			const int j = (int)fdiv((unsigned)e, a.spandiv[cb == 0 ? 0 : 1]), kk = e - j * (ce - cb) * 9;
			if (256 * (u + 1) <= nw) ws[(cb * 9 + kk) * kF3WLd + j] = wv[u];
			else if (e < nw) ws[(cb * 9 + kk) * kF3WLd + j] = wv[u];
		}
	};
	load_half(0, c1);
	store_half(0, c1);
	__syncthreads();
	if (c1 < a.cin) load_half(c1, a.cin);
	const bool active = 64 * wave < hw;  // waves past the plane compute nothing but still stage (uniform)

	// this lane's position (A operand row) and its window origin in the padded plane
	const int p = min(64 * wave + M16::arow(lane), hw - 1);
	const int oh = p / a.width, ow = p - oh * a.width;
	const float* xl = xs + oh * kF3Pad + ow;
	const float* wl = ws + M16::bcol(lane);
	M16::Acc acc0, acc1;
#pragma unroll
	for (int r = 0; r < M16::NV; ++r) acc0[r] = acc1[r] = 0.0f;

	// a channel's 9 input values and 2 x 9 W values, read one channel ahead of their MFMAs
	float xa[2][9], wa[2][9], wb[2][9];
	auto read_channel = [&](int c, int s) {
		const float* xc = xl + c * kF3Plane;
		const float* wc = wl + c * 9 * kF3WLd;
#pragma unroll
		for (int t = 0; t < 9; ++t) {
			xa[s][t] = xc[(t / 3) * kF3Pad + (t % 3)];
			wa[s][t] = wc[t * kF3WLd];
			wb[s][t] = wc[t * kF3WLd + 16];
		}
	};
	auto run_channel = [&](int s) {
#pragma unroll
		for (int t = 0; t < 9; ++t) {
			acc0 = M16::mma(xa[s][t], wa[s][t], acc0);
			acc1 = M16::mma(xa[s][t], wb[s][t], acc1);
		}
	};
	// channels [cb, ce) in order, two at a time, each channel's operands read while the previous one runs
	auto run_channels = [&](int cb, int ce) {
		read_channel(cb, 0);
		int c = cb;
		for (; c + 2 <= ce; c += 2) {
			read_channel(c + 1, 1);
			__builtin_amdgcn_sched_barrier(0);
			run_channel(0);
			__builtin_amdgcn_sched_barrier(0);
			if (c + 2 < ce) read_channel(c + 2, 0);
			__builtin_amdgcn_sched_barrier(0);
			run_channel(1);
			__builtin_amdgcn_sched_barrier(0);
		}
		if (c < ce) run_channel(0);
	};
	if (active) run_channels(0, c1);
	if (c1 < a.cin) {
		store_half(c1, a.cin);
		__syncthreads();
		if (active) run_channels(c1, a.cin);
	}
	if (!active) return;

	// epilogue (ops.cpp:1396-1409): v = acc + b, then alive = v > 0 and y = alive ? v : 0 with the ReLU
	float* yn = a.y + (int64_t)n * a.cout * hw;
	unsigned char* an = a.alive ? a.alive + (int64_t)n * a.cout * hw : nullptr;
#pragma unroll
	for (int u = 0; u < 2; ++u) {
		const M16::Acc& acc = u == 0 ? acc0 : acc1;
		const int co = co0 + 16 * u + M16::ccol(lane);
		if (co >= a.cout) continue;
		const float bv = a.bias[co];
#pragma unroll
		for (int t = 0; t < M16::NV / 4; ++t) {
			const int p0 = 64 * wave + M16::crow(4 * t, lane);  // four consecutive positions
			if (p0 >= hw) continue;
			f32x4 v;
			unsigned flags = 0;
#pragma unroll
			for (int e = 0; e < 4; ++e) {
				float z = acc[4 * t + e] + bv;
				if (a.relu) {
					const bool on = z > 0.0f;
					flags |= (on ? 1u : 0u) << (8 * e);
					z = on ? z : 0.0f;
				}
				v[e] = z;
			}
			*reinterpret_cast<f32x4*>(yn + (int64_t)co * hw + p0) = v;  // hw % 4 == 0
			if (an) *reinterpret_cast<unsigned*>(an + (int64_t)co * hw + p0) = flags;
		}
	}
}

size_t f3_lds_bytes(int cin) { return (size_t)(cin * kF3Plane + cin * 9 * kF3WLd) * sizeof(float); }

}  // namespace

bool conv_fwd3_ok(const ConvGeom& g, int64_t samples, int cout, const float* y, const unsigned char* alive) {
	if (g.kh != 3 || g.kw != 3 || g.stride != 1 || g.pad != 1 || g.h > 14 || g.w > 14 || g.ho != g.h || g.wo != g.w)
		return false;
	const int64_t hw = (int64_t)g.h * g.w, K = (int64_t)g.cin * 9;
	if (hw % 4 != 0 || cout % kF3Co != 0 || samples * (cout / kF3Co) > 0x7fffffff) return false;
	if (depth_cut(cout, hw, K)) return false;  // the reference splits such products into 128-deep pieces
	if (f3_lds_bytes(g.cin) > (size_t)kF3MaxLds || g.cin > 80) return false;  // a half stages <= 40 channels
	if (reinterpret_cast<uintptr_t>(y) % 16 != 0 || (alive && reinterpret_cast<uintptr_t>(alive) % 4 != 0)) return false;
	return true;
}

hipError_t conv_fwd3(const float* x, const float* w, const float* bias, float* y, unsigned char* alive,
                     const ConvGeom& g, int64_t samples, int cout, int relu, hipStream_t s) {
	const size_t lds = f3_lds_bytes(g.cin);
	static std::mutex mu;
	static bool raised[64] = {};
	int dev = 0;
	hipError_t e = hipGetDevice(&dev);
	if (e != hipSuccess) return e;
	if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
	{
		std::lock_guard<std::mutex> lock(mu);
		if (!raised[dev]) {
			for (const void* fn : {reinterpret_cast<const void*>(conv_fwd3_kernel<16>),
			                       reinterpret_cast<const void*>(conv_fwd3_kernel<40>)}) {
				e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kF3MaxLds);
				if (e != hipSuccess) return e;
			}
			raised[dev] = true;
		}
	}
	const int c1 = (g.cin + 1) / 2;
	F3Args a{x, w, bias, y, alive, g.cin, g.h, g.w, cout, cout / kF3Co, relu,
	         {make_fastdiv((unsigned)(c1 * 9)), make_fastdiv((unsigned)(std::max(g.cin - c1, 1) * 9))}};
	if (c1 <= 16) hipLaunchKernelGGL(conv_fwd3_kernel<16>, dim3((unsigned)(samples * a.groups)), dim3(256), lds, s, a);
	else hipLaunchKernelGGL(conv_fwd3_kernel<40>, dim3((unsigned)(samples * a.groups)), dim3(256), lds, s, a);
	return hipGetLastError();
}

}  // namespace nnh
