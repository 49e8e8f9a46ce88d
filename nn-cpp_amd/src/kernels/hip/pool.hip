// pool.hip - nn::maxpool2d forward and backward (src/autograd/ops.cpp:1609-1705) on NCHW planes.
//
// Forward: each output scans its kernel x kernel window row by row from best = -inf, at = 0, taking a value only
// when it is greater than best (the first maximum wins, NaN never does, and a window with nothing above -inf keeps
// offset 0 of the plane). The argmax is that offset inside the (n, c) plane, as the reference keeps it for backward.
// Backward: the reference zero-fills a fresh plane and adds g[i] at argmax[i] for i in output order. Here each
// input element gathers instead, visiting the windows that contain it in output order (no atomics, one writer per
// element). Offset 0 of a plane also receives the windows that kept offset 0 without containing it; when a plane
// has such windows its thread walks every output of the plane in order. 2 x 2 windows at stride 2 on even planes
// (one window per element) take a kernel of their own, a wave per plane.
#include "pool.hpp"

#include <cmath>

#include "fastdiv.hpp"

namespace nnh {

namespace {

struct PoolArgs {
	const float* x;
	float* y;
	uint32_t* arg;
	int64_t total;          // outputs
	int h, w, ho, wo, k, s;
	FastDiv plane_out, wo_div;
};

// One output per thread: the general window.
__global__ void __launch_bounds__(256) maxpool_forward_kernel(const PoolArgs a) {
	const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (idx >= a.total) return;
	const int64_t p = idx / (a.ho * a.wo);
	const int o = (int)(idx - p * (a.ho * a.wo));
	const int oh = (int)fdiv((unsigned)o, a.wo_div), ow = o - oh * a.wo;
	const float* plane = a.x + p * a.h * a.w;
	float best = -INFINITY;
	uint32_t at = 0;
	for (int ph = 0; ph < a.k; ++ph) {
		const int r = oh * a.s + ph;
		const float* row = plane + (int64_t)r * a.w + ow * a.s;
		for (int pw = 0; pw < a.k; ++pw) {
			const float v = row[pw];
			if (v > best) {
				best = v;
				at = (uint32_t)(r * a.w + ow * a.s + pw);
			}
		}
	}
	a.y[idx] = best;
	if (a.arg) a.arg[idx] = at;
}

// 2 x 2 windows, stride 2, W a multiple of 4 and 16-byte aligned planes: two outputs per thread from one 16-byte
// load of each of the window's two rows; the same four comparisons in the same order per output.
__global__ void __launch_bounds__(256) maxpool2x2_forward_kernel(const PoolArgs a) {
	const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // output pair
	const int pairs = a.wo >> 1;
	const int64_t per_plane = (int64_t)a.ho * pairs;
	if (idx >= a.total / 2) return;
	const int64_t p = idx / per_plane;
	const int q = (int)(idx - p * per_plane);
	const int oh = q / pairs, j = q - oh * pairs;
	const float* r0 = a.x + p * a.h * a.w + (int64_t)(2 * oh) * a.w + 4 * j;
	const float4 u = *reinterpret_cast<const float4*>(r0);
	const float4 v = *reinterpret_cast<const float4*>(r0 + a.w);
	const uint32_t base = (uint32_t)(2 * oh * a.w + 4 * j);
	float b0 = -INFINITY, b1 = -INFINITY;
	uint32_t t0 = 0, t1 = 0;
	if (u.x > b0) { b0 = u.x; t0 = base; }
	if (u.y > b0) { b0 = u.y; t0 = base + 1; }
	if (v.x > b0) { b0 = v.x; t0 = base + a.w; }
	if (v.y > b0) { b0 = v.y; t0 = base + a.w + 1; }
	if (u.z > b1) { b1 = u.z; t1 = base + 2; }
	if (u.w > b1) { b1 = u.w; t1 = base + 3; }
	if (v.z > b1) { b1 = v.z; t1 = base + a.w + 2; }
	if (v.w > b1) { b1 = v.w; t1 = base + a.w + 3; }
	const int64_t o = p * a.ho * a.wo + (int64_t)oh * a.wo + 2 * j;
	*reinterpret_cast<float2*>(a.y + o) = make_float2(b0, b1);
	if (a.arg) *reinterpret_cast<uint2*>(a.arg + o) = make_uint2(t0, t1);
}

struct PoolBwdArgs {
	const float* g;
	const uint32_t* arg;
	float* dx;
	int h, w, ho, wo, k, s, first;
	FastDiv w_div, s_div, wo_div;
};

// One (n, c) plane per workgroup (ops.cpp:1686-1704). Only the first window contains offset 0, so a later window
// whose argmax is 0 is one where nothing beat -inf; the threads look for such windows together first. Each input
// element then adds, in output order, g of the windows that contain it and picked it; offset 0 walks every output
// of the plane in order when such windows exist.
__global__ void __launch_bounds__(256) maxpool_backward_kernel(const PoolBwdArgs a) {
	__shared__ int empty_windows;
	const int tid = threadIdx.x;
	const int64_t p = blockIdx.x;
	const int hw = a.h * a.w, out_plane = a.ho * a.wo;
	const float* g = a.g + p * out_plane;
	const uint32_t* arg = a.arg + p * out_plane;
	float* dx = a.dx + p * hw;
	if (tid == 0) empty_windows = 0;
	__syncthreads();
	bool found = false;
	for (int i = tid + 1; i < out_plane; i += 256) found = found || arg[i] == 0u;
	if (found) empty_windows = 1;  // every writer stores the same value
	__syncthreads();
	const bool scan0 = empty_windows != 0;
	for (int e = tid; e < hw; e += 256) {
		float v = a.first ? 0.0f : dx[e];
		if (e == 0 && scan0) {
			for (int i = 0; i < out_plane; ++i)
				if (arg[i] == 0u) v = v + g[i];
		} else {
			const int ih = (int)fdiv((unsigned)e, a.w_div), iw = e - ih * a.w;
			// windows oh with oh*s <= ih <= oh*s + k - 1, oh < ho (and the same across)
			const int oh_lo = ih >= a.k ? (int)fdiv((unsigned)(ih - a.k), a.s_div) + 1 : 0;
			const int oh_hi = min((int)fdiv((unsigned)ih, a.s_div), a.ho - 1);
			const int ow_lo = iw >= a.k ? (int)fdiv((unsigned)(iw - a.k), a.s_div) + 1 : 0;
			const int ow_hi = min((int)fdiv((unsigned)iw, a.s_div), a.wo - 1);
			for (int oh = oh_lo; oh <= oh_hi; ++oh)
				for (int ow = ow_lo; ow <= ow_hi; ++ow) {
					const int i = oh * a.wo + ow;
					if (arg[i] == (uint32_t)e) v = v + g[i];
				}
		}
		dx[e] = v;
	}
}

// 2 x 2 windows at stride 2 on planes of even height and width: every element lies in exactly one window, so it gets
// that window's g when the window picked it, and offset 0 also gets the later windows that kept offset 0 (nothing in
// them beat -inf). A wave owns a plane and its lanes take kPool2Per windows each per pass, with every load of the
// pass (argmax, g, the four old values) issued before the first use; the first pass looks for windows that kept
// offset 0 with a ballot, and when a plane has any, lane 0 walks the plane's windows in order for offset 0.
constexpr int kPool2Per = 4;

__global__ void __launch_bounds__(256) maxpool2x2_backward_kernel(const PoolBwdArgs a, const int64_t planes) {
	const int lane = threadIdx.x & 63;
	const int64_t p = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
	if (p >= planes) return;
	const int out = a.ho * a.wo;
	const float* g = a.g + p * out;
	const uint32_t* arg = a.arg + p * out;
	float* dx = a.dx + p * a.h * a.w;
	bool walk0 = false;
	for (int i0 = 0; i0 < out; i0 += 64 * kPool2Per) {
		uint32_t at[kPool2Per];
		float gv[kPool2Per];
		int base[kPool2Per];
		float2 o0[kPool2Per], o1[kPool2Per];
#pragma unroll
		for (int j = 0; j < kPool2Per; ++j) {
			const int i = min(i0 + 64 * j + lane, out - 1);  // a repeated window is computed, stored once
			at[j] = arg[i];
			gv[j] = g[i];
			const int oh = (int)fdiv((unsigned)i, a.wo_div);
			base[j] = 2 * oh * a.w + 2 * (i - oh * a.wo);
			o0[j] = a.first ? make_float2(0.0f, 0.0f) : *reinterpret_cast<const float2*>(dx + base[j]);
			o1[j] = a.first ? make_float2(0.0f, 0.0f) : *reinterpret_cast<const float2*>(dx + base[j] + a.w);
		}
		if (i0 == 0) {
			bool kept0 = false;
#pragma unroll
			for (int j = 0; j < kPool2Per; ++j) {
				const int i = 64 * j + lane;
				kept0 = kept0 || (i > 0 && i < out && at[j] == 0u);
			}
			for (int i = 64 * kPool2Per + lane; i < out; i += 64) kept0 = kept0 || arg[i] == 0u;
			walk0 = __ballot(kept0) != 0;
		}
#pragma unroll
		for (int j = 0; j < kPool2Per; ++j) {
			const uint32_t e = (uint32_t)base[j];
			if (at[j] == e) o0[j].x = o0[j].x + gv[j];
			if (at[j] == e + 1) o0[j].y = o0[j].y + gv[j];
			if (at[j] == e + a.w) o1[j].x = o1[j].x + gv[j];
			if (at[j] == e + a.w + 1) o1[j].y = o1[j].y + gv[j];
		}
		if (i0 == 0 && lane == 0 && walk0) {  // window 0 is lane 0's first: its offset 0 takes every kept-0 window
			float v = a.first ? 0.0f : dx[0];
			for (int i = 0; i < out; ++i)
				if (arg[i] == 0u) v = v + g[i];
			o0[0].x = v;
		}
#pragma unroll
		for (int j = 0; j < kPool2Per; ++j)
			if (i0 + 64 * j + lane < out) {
				*reinterpret_cast<float2*>(dx + base[j]) = o0[j];
				*reinterpret_cast<float2*>(dx + base[j] + a.w) = o1[j];
			}
	}
}

// The same backward from 2-bit window positions (the packed form the fused conv2d_relu + 2 x 2 pool writes: window
// (pr, wc) of plane p at bits 2 (wc % 4) of byte (p ho + pr) rb + wc / 4, rb = ceil(w / 8)): every element gets its
// window's g when the window picked it (from 0 when first, else added to its old value); a window's maximum is
// always one of its own four elements there, so no window keeps the plane's offset 0. A thread per window.
__global__ void __launch_bounds__(256) maxpool2x2_backward_slots_kernel(const float* __restrict__ g,
                                                                        const unsigned char* __restrict__ slots,
                                                                        float* __restrict__ dx, int h, int w, int first,
                                                                        FastDiv wo_div, FastDiv out_div, int64_t total) {
	const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (t >= total) return;
	const int wo = (int)wo_div.d, out = (int)out_div.d;
	const int64_t p = t / out;
	const int i = (int)(t - p * out);
	const int pr = (int)fdiv((unsigned)i, wo_div), wc = i - pr * wo;
	const int rb = (w + 7) >> 3;
	const unsigned sl = (slots[(p * (h >> 1) + pr) * rb + (wc >> 2)] >> (2 * (wc & 3))) & 3u;
	const float gv = g[t];
	float* d = dx + p * h * w + (int64_t)(2 * pr) * w + 2 * wc;
	float2 r0 = first ? make_float2(0.0f, 0.0f) : *reinterpret_cast<const float2*>(d);
	float2 r1 = first ? make_float2(0.0f, 0.0f) : *reinterpret_cast<const float2*>(d + w);
	if (sl == 0) r0.x = r0.x + gv;
	if (sl == 1) r0.y = r0.y + gv;
	if (sl == 2) r1.x = r1.x + gv;
	if (sl == 3) r1.y = r1.y + gv;
	*reinterpret_cast<float2*>(d) = r0;
	*reinterpret_cast<float2*>(d + w) = r1;
}

}  // namespace

hipError_t maxpool2x2_backward_slots(const float* g, const unsigned char* slots, float* dx, int64_t planes, int h, int w,
                                     int first, hipStream_t st) {
	if (planes == 0 || h == 0 || w == 0) return hipSuccess;
	if (h % 2 != 0 || w % 2 != 0 || reinterpret_cast<uintptr_t>(dx) % 8 != 0) return hipErrorInvalidValue;
	const int ho = h / 2, wo = w / 2;
	const int64_t total = planes * ho * wo;
	if ((total + 255) / 256 > 0x7fffffff) return hipErrorInvalidConfiguration;
	hipLaunchKernelGGL(maxpool2x2_backward_slots_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, g, slots,
	                   dx, h, w, first, make_fastdiv((unsigned)wo), make_fastdiv((unsigned)(ho * wo)), total);
	return hipGetLastError();
}

hipError_t maxpool2d_forward(const float* x, float* y, uint32_t* arg, int64_t planes, int h, int w, int k, int s,
                             hipStream_t st) {
	PoolArgs a;
	a.x = x;
	a.y = y;
	a.arg = arg;
	a.h = h;
	a.w = w;
	a.k = k;
	a.s = s;
	a.ho = (h - k) / s + 1;
	a.wo = (w - k) / s + 1;
	a.total = planes * a.ho * a.wo;
	a.wo_div = make_fastdiv((unsigned)a.wo);
	if (a.total == 0) return hipSuccess;
	const bool quad = k == 2 && s == 2 && w % 4 == 0 && h % 2 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
	                  reinterpret_cast<uintptr_t>(y) % 8 == 0 && reinterpret_cast<uintptr_t>(arg) % 8 == 0;
	if (quad) {
		const int64_t threads = a.total / 2;
		hipLaunchKernelGGL(maxpool2x2_forward_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, a);
	} else {
		hipLaunchKernelGGL(maxpool_forward_kernel, dim3((unsigned)((a.total + 255) / 256)), dim3(256), 0, st, a);
	}
	return hipGetLastError();
}

hipError_t maxpool2d_backward(const float* g, const uint32_t* arg, float* dx, int64_t planes, int h, int w, int k, int s,
                              int first, hipStream_t st) {
	PoolBwdArgs a;
	a.g = g;
	a.arg = arg;
	a.dx = dx;
	a.h = h;
	a.w = w;
	a.k = k;
	a.s = s;
	a.first = first;
	a.ho = (h - k) / s + 1;
	a.wo = (w - k) / s + 1;
	a.w_div = make_fastdiv((unsigned)w);
	a.s_div = make_fastdiv((unsigned)s);
	a.wo_div = make_fastdiv((unsigned)a.wo);
	if (planes == 0 || (int64_t)h * w == 0) return hipSuccess;
	if (planes > 0x7fffffff) return hipErrorInvalidConfiguration;
	if (k == 2 && s == 2 && h % 2 == 0 && w % 2 == 0 && reinterpret_cast<uintptr_t>(dx) % 8 == 0)
		hipLaunchKernelGGL(maxpool2x2_backward_kernel, dim3((unsigned)((planes + 3) / 4)), dim3(256), 0, st, a, planes);
	else
		hipLaunchKernelGGL(maxpool_backward_kernel, dim3((unsigned)planes), dim3(256), 0, st, a);
	return hipGetLastError();
}

}  // namespace nnh
