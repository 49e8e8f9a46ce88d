// conv_dx.hip - the input gradient of nn::conv2d without the column matrix in HBM (ops.cpp:1452-1455).
//
// The reference computes, per sample, dcol = W^T g (sgemm T,F: each element the fma chain over the output
// channels co = 0..Cout-1 from +0) and then col2im: each dx element, starting from 0 (a fresh gradient) or its old
// value, adds its taps in (ph, pw) order. One workgroup here owns one sample and a group of CG input channels:
//   1. dcol rows k = (c, ph, pw) of its channels for every output position, as 16x16x1 MFMA chains over co:
//      wave w owns positions 64w..64w+63 (the MFMA's A operand: the masked gradient g[co][p], read from global
//      memory one row per step), against up to 80 rows k in five 16-wide units (B operand: W[co][k], staged in LDS
//      a chunk of 64 output channels at a time); the chains never leave the accumulators across chunks.
//   2. The dcol tile goes to LDS, and each dx element of the group gathers its taps from there, in (ph, pw) order.
// Same bits as the batched GEMM + col2im path, with no dcol in HBM. Three shapes of workgroup: 4 waves and up to 80
// dcol rows (Ho*Wo <= 256, a deeper layer); for a first layer (Ho*Wo <= 1024 and kh*kw <= 16, such as 28 x 28 with
// Cin = 1, where one row of W^T per tap is all a sample needs), 4 waves and up to 16 rows on a band of dx rows when
// the stride is 1 (the band's output rows, halo included, in 256 positions: a 28 x 28 plane is four bands of seven
// rows, four workgroups a sample), else 16 waves and up to 16 rows on the whole plane. Otherwise the caller uses the
// batched GEMM + col2im path.
#include "conv.hpp"

#include <algorithm>

#include "gemm.hpp"
#include "gemm_tile.hpp"

namespace nnh {

namespace {

constexpr int kDxCo = 64;        // output channels of W staged per chunk
constexpr int kDxWLd = kDxCo + 4;
constexpr int kDxLdsBytes = 80 * 1024;
constexpr int kDxACh = 16;       // gradient rows each lane keeps in flight

// The two workgroup shapes: NW waves (one output position per lane, 64 NW positions) and ROWS dcol rows (16-wide
// MFMA units).
struct DxShape {
	int nw, rows;
};
constexpr DxShape kDxDeep{4, 80};
constexpr DxShape kDxFirst{16, 16};
constexpr DxShape kDxBand{4, 16};  // kDxFirst's rows on a band of a stride-1 plane's rows

constexpr bool same_shape(const DxShape& a, const DxShape& b) { return a.nw == b.nw && a.rows == b.rows; }

using M16 = Mfma<kMf16>;

struct DxArgs {
	const float* g;   // output gradient {N, Cout, hw}, masked unless alive is given
	const unsigned char* alive;  // the folded ReLU's flags: g is masked here (alive ? g : 0), or null
	const float* w;   // {Cout, K}
	float* dx;        // {N, Cin, H, W}
	ConvGeom geo;
	int cout, cg, groups, total, first;
	int bands, band_rows;  // stride 1 only: a workgroup takes band_rows rows of dx (bands per sample), else 1 and H
	int hwp;          // LDS row stride of the dcol tile (a multiple of 4, > the positions a workgroup computes)
	FastDiv plane, width, stride;  // division by band_rows*W, W and the stride
};

// The taps of a 3x3, stride-1 convolution, unrolled: the same order and the same additions as gather_taps. The
// nine reads are unconditional (positions clamped into the row) so that all are in flight at once; a tap outside
// the output plane is dropped by a select, which leaves the sum exactly as skipping it would.
__device__ __forceinline__ float gather_taps_3x3(const float* tile, const DxArgs& a, int q0, int q1, int c, int ih, int iw,
                                                 float v) {
	const ConvGeom& G = a.geo;
	float x[9];
	bool ok[9];
#pragma unroll
	for (int ph = 0; ph < 3; ++ph) {
		const int qh = ih + G.pad - ph;
		const bool row_ok = qh >= 0 && qh < G.ho;
		const float* trow = tile + (c * 9 + ph * 3) * a.hwp + (min(max(qh, q0), q1 - 1) - q0) * G.wo;
#pragma unroll
		for (int pw = 0; pw < 3; ++pw) {
			const int qw = iw + G.pad - pw;
			ok[ph * 3 + pw] = row_ok && qw >= 0 && qw < G.wo;
			x[ph * 3 + pw] = trow[pw * a.hwp + min(max(qw, 0), G.wo - 1)];
		}
	}
#pragma unroll
	for (int t = 0; t < 9; ++t) v = ok[t] ? v + x[t] : v;
	return v;
}

// The taps of dx element (ih, iw) of channel c from the dcol tile, in (ph, pw) order (col2im_fast_kernel's gather);
// the tile's first row is output row q0
template <bool STRIDE1>
__device__ __forceinline__ float gather_taps(const float* tile, const DxArgs& a, int q0, int c, int ih, int iw, float v) {
	const ConvGeom& G = a.geo;
	for (int ph = 0; ph < G.kh; ++ph) {
		const int th = ih + G.pad - ph;
		int qh = th;
		if (th < 0) continue;
		if (!STRIDE1) {
			qh = (int)fdiv((unsigned)th, a.stride);
			if (qh * G.stride != th) continue;
		}
		if (qh >= G.ho) continue;
		const float* trow = tile + (c * G.kh + ph) * G.kw * a.hwp + (qh - q0) * G.wo;
		for (int pw = 0; pw < G.kw; ++pw) {
			const int tw = iw + G.pad - pw;
			int qw = tw;
			if (tw < 0) continue;
			if (!STRIDE1) {
				qw = (int)fdiv((unsigned)tw, a.stride);
				if (qw * G.stride != tw) continue;
			}
			if (qw >= G.wo) continue;
			v = v + trow[pw * a.hwp + qw];
		}
	}
	return v;
}

template <int NW, int kDxRows>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2))) conv_dx_fused_kernel(const DxArgs a) {
	constexpr int kThreads = NW * 64;
	extern __shared__ __align__(16) float sm[];
	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const ConvGeom& G = a.geo;
	const int khkw = G.kh * G.kw, hw = G.ho * G.wo, K = G.cin * khkw;
	const int lid = xcd_remap(blockIdx.x, a.total);  // the channel groups and bands of one sample share an XCD's L2
	const int gb = lid / a.bands, band = lid - gb * a.bands;
	const int n = gb / a.groups, grp = gb - n * a.groups;
	const int c0 = grp * a.cg, cg = min(a.cg, G.cin - c0), rows = cg * khkw, k0 = c0 * khkw;
	// dx rows r0 .. r0 + band_rows - 1 take taps from output rows q0 .. q1 - 1 (stride 1: qh = ih + pad - ph)
	const int r0 = band * a.band_rows;
	const int q0 = a.bands > 1 ? max(0, r0 + G.pad - G.kh + 1) : 0;
	const int q1 = a.bands > 1 ? min(G.ho, r0 + a.band_rows + G.pad) : G.ho;
	const int p_lo = q0 * G.wo, np = (q1 - q0) * G.wo;  // the positions this workgroup computes
	float* wl = sm;                          // [kDxRows][kDxWLd]: W^T for a chunk of output channels
	float* tile = sm + kDxRows * kDxWLd;     // [cg * khkw][hwp]: the group's dcol rows
	const float* gn = a.g + (int64_t)n * a.cout * hw;
	const unsigned char* an = a.alive ? a.alive + (int64_t)n * a.cout * hw : nullptr;

	// 1. the chains
	M16::Acc acc[kDxRows / 16];
#pragma unroll
	for (int u = 0; u < kDxRows / 16; ++u)
#pragma unroll
		for (int r = 0; r < M16::NV; ++r) acc[u][r] = 0.0f;
	const int pos = p_lo + min(64 * wave + M16::arow(lane), np - 1);  // positions past np compute values never stored
	const bool pos_here = 64 * wave < np;
	// gradient rows co .. co+kDxACh-1 at this lane's position (rows clamped into range, never used past cout)
	auto load_g = [&](float (&dst)[kDxACh], int co) {
		if (an) {  // ops.cpp:1439-1443's mask, applied as the rows are read
			unsigned char f[kDxACh];
#pragma unroll
			for (int u = 0; u < kDxACh; ++u) {
				const int64_t off = (int64_t)min(co + u, a.cout - 1) * hw + pos;
				dst[u] = gn[off];
				f[u] = an[off];
			}
#pragma unroll
			for (int u = 0; u < kDxACh; ++u) dst[u] = f[u] ? dst[u] : 0.0f;
		} else {
#pragma unroll
			for (int u = 0; u < kDxACh; ++u) dst[u] = gn[(int64_t)min(co + u, a.cout - 1) * hw + pos];
		}
	};
	for (int cc = 0; cc < a.cout; cc += kDxCo) {
		const int nco = min(kDxCo, a.cout - cc);
		// W[cc + j][k0 + k] into wl[k][j] (rows past the group and channels past cout read as 0); every load is
		// issued (at an index clamped into range) before the first store
		{
			constexpr int kPer = kDxRows * kDxCo / kThreads;
			static_assert(kPer * kThreads == kDxRows * kDxCo, "the W chunk splits evenly over the threads");
			float wv[kPer];
#pragma unroll
			for (int u = 0; u < kPer; ++u) {
				const int idx = tid + kThreads * u, j = idx / kDxRows, k = idx - j * kDxRows;
				wv[u] = a.w[(int64_t)(cc + min(j, nco - 1)) * K + k0 + min(k, rows - 1)];
			}
#pragma unroll
			for (int u = 0; u < kPer; ++u) {
				const int idx = tid + kThreads * u, j = idx / kDxRows, k = idx - j * kDxRows;
				wl[k * kDxWLd + j] = (k < rows && j < nco) ? wv[u] : 0.0f;
			}
		}
		__syncthreads();
		if (pos_here) {
			float g0[kDxACh], g1[kDxACh];
			load_g(g0, cc);
			load_g(g1, cc + kDxACh);
			auto steps = [&](const float (&gv)[kDxACh], int j0) {
#pragma unroll
				for (int q = 0; q < kDxACh / 4; ++q) {
					const int j = j0 + 4 * q;
					if (j < nco) {  // whole quads of channels, then single steps for a ragged end
						f32x4 b[kDxRows / 16];
#pragma unroll
						for (int u = 0; u < kDxRows / 16; ++u)
							b[u] = *reinterpret_cast<const f32x4*>(wl + (16 * u + M16::bcol(lane)) * kDxWLd + j);
#pragma unroll
						for (int e = 0; e < 4; ++e)
							if (j + e < nco)
#pragma unroll
								for (int u = 0; u < kDxRows / 16; ++u)
									acc[u] = M16::mma(gv[4 * q + e], b[u][e], acc[u]);
					}
				}
			};
			for (int j0 = 0; j0 < nco; j0 += 2 * kDxACh) {  // two chunks of gradient rows in flight
				steps(g0, j0);
				load_g(g0, cc + j0 + 2 * kDxACh);
				steps(g1, j0 + kDxACh);
				load_g(g1, cc + j0 + 3 * kDxACh);
			}
		}
		__syncthreads();  // wl is rewritten by the next chunk
	}

	// 2a. the dcol rows into LDS: registers 4t .. 4t+3 of unit u hold row 16u + (l & 15) at four consecutive
	// positions
	if (pos_here) {
#pragma unroll
		for (int u = 0; u < kDxRows / 16; ++u) {
			const int k = 16 * u + M16::ccol(lane);
#pragma unroll
			for (int t = 0; t < M16::NV / 4; ++t) {
				const int p0 = 64 * wave + M16::crow(4 * t, lane);
				if (k < rows && p0 < np)
					*reinterpret_cast<f32x4*>(tile + k * a.hwp + p0) =
					    f32x4{acc[u][4 * t], acc[u][4 * t + 1], acc[u][4 * t + 2], acc[u][4 * t + 3]};
			}
		}
	}
	__syncthreads();

	// 2b. col2im for the group's channels: every dx element adds its taps in (ph, pw) order
	// elements e = (c, ih - r0, iw) over the group's channels and the band's rows; rows past H (a short last band)
	// are computed at row H - 1 and not stored
	const int plane = G.h * G.w, bplane = a.band_rows * G.w, total = cg * bplane;
	float* dxn = a.dx + ((int64_t)n * G.cin + c0) * plane + r0 * G.w;
	if (G.stride == 1 && G.kh == 3 && G.kw == 3) {  // uniform: two elements per thread at a time
		for (int e0 = tid; e0 < total; e0 += 2 * kThreads) {
			int c[2], ih[2], iw[2], at[2];
			bool keep[2];
			float v[2];
#pragma unroll
			for (int h = 0; h < 2; ++h) {
				const int e = min(e0 + kThreads * h, total - 1);  // a repeated element is computed, stored once
				c[h] = (int)fdiv((unsigned)e, a.plane);
				const int rem = e - c[h] * bplane, rr = (int)fdiv((unsigned)rem, a.width);
				iw[h] = rem - rr * G.w;
				ih[h] = min(r0 + rr, G.h - 1);
				keep[h] = e0 + kThreads * h < total && r0 + rr < G.h;
				at[h] = c[h] * plane + (ih[h] - r0) * G.w + iw[h];
				v[h] = a.first ? 0.0f : dxn[at[h]];
			}
#pragma unroll
			for (int h = 0; h < 2; ++h) v[h] = gather_taps_3x3(tile, a, q0, q1, c[h], ih[h], iw[h], v[h]);
#pragma unroll
			for (int h = 0; h < 2; ++h)
				if (keep[h]) dxn[at[h]] = v[h];
		}
	} else {
		for (int e = tid; e < total; e += kThreads) {
			const int c = (int)fdiv((unsigned)e, a.plane), rem = e - c * bplane;
			const int rr = (int)fdiv((unsigned)rem, a.width), iw = rem - rr * G.w, ih = r0 + rr;
			if (ih >= G.h) continue;
			const int at = c * plane + rr * G.w + iw;
			const float v0 = a.first ? 0.0f : dxn[at];
			dxn[at] = G.stride != 1 ? gather_taps<false>(tile, a, q0, c, ih, iw, v0)
			                        : gather_taps<true>(tile, a, q0, c, ih, iw, v0);
		}
	}
}

// Rows of dx per band for kDxBand, balanced over the bands, with a band's output rows (band rows + kh - 1 at most,
// stride 1) within the workgroup's 64 * nw positions; 0 when not even one row fits
int dx_band_rows(const ConvGeom& g) {
	if (g.stride != 1 || g.h < 1 || g.wo < 1) return 0;
	const int most = 64 * kDxBand.nw / g.wo - (g.kh - 1);
	if (most < 1) return 0;
	const int bands = (g.h + most - 1) / most;
	return (g.h + bands - 1) / bands;
}

int dx_hwp(const ConvGeom& g, const DxShape& sh) {
	const int positions = same_shape(sh, kDxBand) ? (dx_band_rows(g) + g.kh - 1) * g.wo : g.ho * g.wo;
	return (positions + 3) / 4 * 4 + 4;
}

int dx_lds_bytes(const ConvGeom& g, const DxShape& sh, int cg) {
	return (sh.rows * kDxWLd + cg * g.kh * g.kw * dx_hwp(g, sh)) * 4;
}

// Input channels per workgroup: as many as the shape's MFMA rows hold, fewer if the dcol tile would not fit LDS
int dx_group(const ConvGeom& g, const DxShape& sh) {
	int cg = std::min(sh.rows / (g.kh * g.kw), g.cin);
	while (cg > 0 && dx_lds_bytes(g, sh, cg) > kDxLdsBytes) --cg;
	return cg;
}

// The workgroup shape that takes the geometry (nw 0: neither)
DxShape dx_shape(const ConvGeom& g) {
	const int64_t hw = (int64_t)g.ho * g.wo;
	if (hw >= 1 && hw <= 64 * kDxDeep.nw && g.kh * g.kw <= kDxDeep.rows && dx_group(g, kDxDeep) >= 1) return kDxDeep;
	// a first layer's plane in bands of rows: more workgroups than samples, each of four waves
	if (hw >= 1 && hw <= 64 * kDxFirst.nw && g.kh * g.kw <= kDxBand.rows && dx_band_rows(g) >= 1 &&
	    dx_group(g, kDxBand) >= 1)
		return kDxBand;
	if (hw >= 1 && hw <= 64 * kDxFirst.nw && g.kh * g.kw <= kDxFirst.rows && dx_group(g, kDxFirst) >= 1) return kDxFirst;
	return DxShape{0, 0};
}

}  // namespace

bool conv_dx_fused_ok(const ConvGeom& g, int64_t samples, int cout) {
	if (cout < 1) return false;
	const DxShape sh = dx_shape(g);
	if (sh.nw == 0) return false;
	// the reference's dcol product sgemm(T, F, K, hw, Cout) (ops.cpp:1452) splits into pieces over the output
	// channels when it takes the depth cut; this kernel runs one chain over all of them
	if (depth_cut((int64_t)g.cin * g.kh * g.kw, (int64_t)g.ho * g.wo, cout)) return false;
	const int64_t groups = (g.cin + dx_group(g, sh) - 1) / dx_group(g, sh);
	const int64_t bands = same_shape(sh, kDxBand) ? (g.h + dx_band_rows(g) - 1) / dx_band_rows(g) : 1;
	return samples * groups * bands < ((int64_t)1 << 31) && samples * cout * (int64_t)g.ho * g.wo < ((int64_t)1 << 40);
}

hipError_t conv_dx_fused(const float* gm, const unsigned char* alive, const float* w, float* dx, const ConvGeom& g,
                         int64_t samples, int cout, int first, hipStream_t s) {
	if (!conv_dx_fused_ok(g, samples, cout)) return hipErrorInvalidValue;
	const DxShape sh = dx_shape(g);
	DxArgs a;
	a.g = gm;
	a.alive = alive;
	a.w = w;
	a.dx = dx;
	a.geo = g;
	a.cout = cout;
	a.cg = dx_group(g, sh);
	a.groups = (g.cin + a.cg - 1) / a.cg;
	const bool band = same_shape(sh, kDxBand);
	a.band_rows = band ? dx_band_rows(g) : g.h;
	a.bands = (g.h + a.band_rows - 1) / a.band_rows;
	a.total = (int)(samples * a.groups * a.bands);
	a.first = first;
	a.hwp = dx_hwp(g, sh);
	a.plane = make_fastdiv((unsigned)(a.band_rows * g.w));
	a.width = make_fastdiv((unsigned)g.w);
	a.stride = make_fastdiv((unsigned)g.stride);
	const int lds = dx_lds_bytes(g, sh, a.cg);
	void (*fn)(DxArgs) = same_shape(sh, kDxDeep)  ? conv_dx_fused_kernel<kDxDeep.nw, kDxDeep.rows>
	                     : same_shape(sh, kDxBand) ? conv_dx_fused_kernel<kDxBand.nw, kDxBand.rows>
	                                               : conv_dx_fused_kernel<kDxFirst.nw, kDxFirst.rows>;
	hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
	if (e != hipSuccess) return e;
	hipLaunchKernelGGL(fn, dim3((unsigned)a.total), dim3(64 * sh.nw), lds, s, a);
	return hipGetLastError();
}

}  // namespace nnh
