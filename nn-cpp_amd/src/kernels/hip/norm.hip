// norm.hip - nn::batchnorm (training mode, optionally with its folded ReLU) and nn::layernorm, forward and backward
// (src/autograd/ops.cpp:900-1078), with the reference's summation orders.
//
// Batch norm. The reference gives each channel to one thread: for n = 0..N-1 in order it adds, in double, the
// lane_sum of row (n, c) (eight float partial sums over the row, combined as ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)),
// then the tail), divides by N*S, and does the same with lane_sq around the mean. Here:
//   * bn_rows_kernel computes the per-row float sums (lane_sum, lane_sq, or the backward's masked lane_sum and
//     lane_dot): a workgroup owns eight rows of one channel; all its threads stage row chunks in LDS with wide
//     coalesced loads, and wave 0 runs the reference's eight lane chains per row over LDS (lane 8r + k is partial
//     a[k] of row r), combines them and adds the tail in order.
//   * The channel-level double sums over n run in order in one thread of every workgroup that needs them (the
//     rows' sums are staged in LDS first), so the channel's statistics come with each workgroup's own prologue
//     instead of a launch of their own.
//   * bn_norm_kernel (forward) and bn_dx_kernel (backward) are elementwise over a channel's N*S elements in 4096-
//     element chunks, 16-byte loads and stores where the rows allow.
// Layer norm. Each row's sums are single float chains (ops.cpp:1017-1026), so one thread owns a row; the
// gamma/beta gradient sums run down columns in row order, one thread per column (ops.cpp:1063-1075).
#include "norm.hpp"

#include <algorithm>

#include "fastdiv.hpp"

namespace nnh {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kRows = 8;  // rows per workgroup in bn_rows_kernel: one 8-lane group each, all in wave 0

enum BnRowMode { kSum = 0, kSq = 1, kBwd = 2 };

// Elements of each row staged per step. The LDS row pitch is the chunk plus 8 floats: lane 8r + k reads element
// k + 8i of row r, bank (8r + k + 8i) mod 64 for a pitch of 8 mod 64, so the 64 lanes hit 64 banks.
template <int MODE>
struct RowChunk {
	static constexpr int kChunk = MODE == kBwd ? 768 : 1024;
	static constexpr int kPitch = kChunk + 8;
};

struct BnRowArgs {
	const float* x;
	const float* g;               // kBwd: the upstream gradient
	const unsigned char* alive;   // kBwd: the folded ReLU's flags, or null
	const float* rowsum;          // kSq: the rows' lane sums, source of the channel mean
	const float* mean;            // kBwd: the forward's channel means
	float* out0;                  // per row (n * C + c): kSum lane_sum, kSq lane_sq, kBwd lane_sum of masked g
	float* out1;                  // kBwd: lane_dot of masked g with x - mean
	float* mean_out;              // kSq: the channel mean, written by the channel's first workgroup
	int64_t N, C, S;
	int groups;                   // workgroups per channel: ceil(N / kRows)
	double dm;
	int vec;                      // S % 4 == 0 and the row starts are 16-byte (flags 4-byte) aligned
};

// Sums in double of v0[n * C + c] (and v1's) for n = 0..N-1 in order, as the reference adds a channel's row sums
// (ops.cpp:927-929, 973-978): the values are staged 256 at a time in LDS and one thread adds them. Every thread
// of the block receives the sums.
template <int NSUM>
__device__ void channel_dsums(const float* v0, const float* v1, int64_t N, int64_t C, int64_t c, float (*buf)[256],
                              double* out, double* res) {
	const int tid = threadIdx.x;
	double s0 = 0.0, s1 = 0.0;
	for (int64_t n0 = 0; n0 < N; n0 += 256) {
		const int64_t n = n0 + tid;
		if (n < N) {
			buf[0][tid] = v0[n * C + c];
			if (NSUM == 2) buf[1][tid] = v1[n * C + c];
		}
		__syncthreads();
		if (tid == 0) {
			const int cnt = (int)(N - n0 < 256 ? N - n0 : 256);
			for (int i = 0; i < cnt; ++i) {
				s0 += (double)buf[0][i];
				if (NSUM == 2) s1 += (double)buf[1][i];
			}
		}
		__syncthreads();
	}
	if (tid == 0) {
		out[0] = s0;
		out[1] = s1;
	}
	__syncthreads();
	res[0] = out[0];
	res[1] = out[1];
}

// Stages elements [s0, s0 + len) of rows n0 .. n0 + nrows - 1 of channel c from src into dst[r * PITCH + l].
// Loads are clamped to valid addresses and all issued before the LDS stores.
template <int CHUNK, int PITCH>
__device__ __forceinline__ void stage_rows(const float* __restrict__ src, int64_t row0, int64_t row_step, int64_t S,
                                           int64_t s0, int nrows, int len, int vec, float* dst) {
	const int tid = threadIdx.x;
	if (vec) {
		constexpr int kPer = kRows * CHUNK / 4 / 256;
		const int q4 = len >> 2, tot = nrows * q4;
		if (tot == 0) return;
		f32x4 v[kPer];
#pragma unroll
		for (int u = 0; u < kPer; ++u) {
			const int ii = min(tid + 256 * u, tot - 1);
			const int r = ii / q4, q = ii - r * q4;
			v[u] = *reinterpret_cast<const f32x4*>(src + (row0 + r * row_step) * S + s0 + 4 * q);
		}
#pragma unroll
		for (int u = 0; u < kPer; ++u) {
			const int idx = tid + 256 * u;
			if (idx < tot) {
				const int r = idx / q4, q = idx - r * q4;
				*reinterpret_cast<f32x4*>(dst + r * PITCH + 4 * q) = v[u];
			}
		}
	} else {
		constexpr int kPer = kRows * CHUNK / 256;
		const int tot = nrows * len;
		if (tot == 0) return;
		for (int b = 0; b < kPer; b += 16) {
			float v[16];
#pragma unroll
			for (int u = 0; u < 16; ++u) {
				const int ii = min(tid + 256 * (b + u), tot - 1);
				const int r = ii / len, l = ii - r * len;
				v[u] = src[(row0 + r * row_step) * S + s0 + l];
			}
#pragma unroll
			for (int u = 0; u < 16; ++u) {
				const int idx = tid + 256 * (b + u);
				if (idx < tot) {
					const int r = idx / len, l = idx - r * len;
					dst[r * PITCH + l] = v[u];
				}
			}
		}
	}
}

__device__ __forceinline__ void stage_flags(const unsigned char* __restrict__ src, int64_t row0, int64_t row_step,
                                            int64_t S, int64_t s0, int nrows, int len, int vec, unsigned char* dst,
                                            int pitch) {
	const int tid = threadIdx.x;
	if (vec) {
		const int q4 = len >> 2, tot = nrows * q4;
		for (int idx = tid; idx < tot; idx += 256) {
			const int r = idx / q4, q = idx - r * q4;
			*reinterpret_cast<unsigned*>(dst + r * pitch + 4 * q) =
			    *reinterpret_cast<const unsigned*>(src + (row0 + r * row_step) * S + s0 + 4 * q);
		}
	} else {
		const int tot = nrows * len;
		for (int idx = tid; idx < tot; idx += 256) {
			const int r = idx / len, l = idx - r * len;
			dst[r * pitch + l] = src[(row0 + r * row_step) * S + s0 + l];
		}
	}
}

// lane_sum (ops.cpp:804-812), lane_sq (824-834), and the backward's lane_sum / lane_sum_masked with lane_dot /
// lane_dot_masked (848-897) of eight rows (n0 .. n0 + 7) of channel c per workgroup.
template <int MODE>
__global__ void __launch_bounds__(256) bn_rows_kernel(const BnRowArgs a) {
	constexpr int kChunk = RowChunk<MODE>::kChunk, kPitch = RowChunk<MODE>::kPitch;
	__shared__ __align__(16) float xs[kRows * kPitch];
	__shared__ __align__(16) float gs[MODE == kBwd ? kRows * kPitch : 1];
	__shared__ __align__(16) unsigned char fs[MODE == kBwd ? kRows * kPitch : 4];
	__shared__ float buf[2][256];
	__shared__ double bcast[2];
	const int tid = threadIdx.x;
	const int64_t c = blockIdx.x / a.groups;
	const int j = (int)(blockIdx.x - c * a.groups);
	const int64_t n0 = (int64_t)j * kRows;
	const int nrows = (int)(a.N - n0 < kRows ? a.N - n0 : kRows);
	float mu = 0.0f;
	if (MODE == kSq) {
		double s[2];
		channel_dsums<1>(a.rowsum, nullptr, a.N, a.C, c, buf, bcast, s);
		mu = (float)(s[0] / a.dm);
		if (j == 0 && tid == 0) a.mean_out[c] = mu;
	} else if (MODE == kBwd) {
		mu = a.mean[c];
	}
	const bool masked = MODE == kBwd && a.alive != nullptr;
	const int r = tid >> 3, k = tid & 7;
	const int64_t full = a.S & ~(int64_t)7;
	const int64_t row0 = n0 * a.C + c;  // row index of (n0, c); rows of one channel are C apart
	float acc0 = 0.0f, acc1 = 0.0f;
	int64_t s0 = 0;
	do {
		const int len = (int)(a.S - s0 < kChunk ? a.S - s0 : kChunk);
		stage_rows<kChunk, kPitch>(MODE == kBwd ? a.g : a.x, row0, a.C, a.S, s0, nrows, len, a.vec,
		                           MODE == kBwd ? gs : xs);
		if (MODE == kBwd) {
			stage_rows<kChunk, kPitch>(a.x, row0, a.C, a.S, s0, nrows, len, a.vec, xs);
			if (masked) stage_flags(a.alive, row0, a.C, a.S, s0, nrows, len, a.vec, fs, kPitch);
		}
		__syncthreads();
		if (tid < 64) {
			const int lfull = (int)(full - s0 < len ? (full - s0 > 0 ? full - s0 : 0) : len);
			if (r < nrows) {
				const float* xr = xs + r * kPitch;
				const float* gr = gs + r * kPitch;
				const unsigned char* fr = fs + r * kPitch;
				// 16 steps of the lane's chain per batch: the batch's LDS reads are all issued before its adds
				int l = k;
				for (; l + 8 * 15 < lfull; l += 8 * 16) {
					float xv[16], gv[16];
					unsigned char fv[16];
#pragma unroll
					for (int u = 0; u < 16; ++u) {
						xv[u] = xr[l + 8 * u];
						if (MODE == kBwd) {
							gv[u] = gr[l + 8 * u];
							if (masked) fv[u] = fr[l + 8 * u];
						}
					}
#pragma unroll
					for (int u = 0; u < 16; ++u) {
						if (MODE == kSum) {
							acc0 = acc0 + xv[u];
						} else if (MODE == kSq) {
							const float d = xv[u] - mu;
							acc0 = acc0 + d * d;
						} else {
							const float gm = masked ? (fv[u] ? gv[u] : 0.0f) : gv[u];
							acc0 = acc0 + gm;
							acc1 = acc1 + gm * (xv[u] - mu);
						}
					}
				}
				for (; l < lfull; l += 8) {
					if (MODE == kSum) {
						acc0 = acc0 + xr[l];
					} else if (MODE == kSq) {
						const float d = xr[l] - mu;
						acc0 = acc0 + d * d;
					} else {
						const float gm = masked ? (fr[l] ? gr[l] : 0.0f) : gr[l];
						acc0 = acc0 + gm;
						acc1 = acc1 + gm * (xr[l] - mu);
					}
				}
			}
			if (s0 + len >= a.S) {  // last chunk: combine the eight partials of each row, then the tail in order
				const int base = (tid & 63) & ~7;
				float p0[8], p1[8];
#pragma unroll
				for (int u = 0; u < 8; ++u) {
					p0[u] = __shfl(acc0, base + u);
					if (MODE == kBwd) p1[u] = __shfl(acc1, base + u);
				}
				if (k == 0 && r < nrows) {
					float t0 = ((p0[0] + p0[1]) + (p0[2] + p0[3])) + ((p0[4] + p0[5]) + (p0[6] + p0[7]));
					float t1 = 0.0f;
					if (MODE == kBwd) t1 = ((p1[0] + p1[1]) + (p1[2] + p1[3])) + ((p1[4] + p1[5]) + (p1[6] + p1[7]));
					const float* xr = xs + r * kPitch;
					for (int l = lfull; l < len; ++l) {
						if (MODE == kSum) {
							t0 = t0 + xr[l];
						} else if (MODE == kSq) {
							t0 = t0 + (xr[l] - mu) * (xr[l] - mu);
						} else {
							const float gv =
							    masked ? (fs[r * kPitch + l] ? gs[r * kPitch + l] : 0.0f) : gs[r * kPitch + l];
							t0 = t0 + gv;
							t1 = t1 + gv * (xr[l] - mu);
						}
					}
					const int64_t row = row0 + r * a.C;
					a.out0[row] = t0;
					if (MODE == kBwd) a.out1[row] = t1;
				}
			}
		}
		__syncthreads();
		s0 += kChunk;
	} while (s0 < a.S);
}

constexpr int kElemChunk = 4096;  // channel elements per workgroup in the elementwise kernels (16 per thread)

struct BnElemArgs {
	const float* x;
	const float* g;               // backward: upstream gradient
	const unsigned char* alive_in;  // backward: the folded ReLU's flags, or null
	const float* w;
	const float* b;
	const float* rowv0;           // forward: rows' lane_sq; backward: rows' lane sums of masked g
	const float* rowv1;           // backward: rows' lane_dot
	const float* mean;
	const float* inv_in;          // backward: inv_std from the forward
	float* y;                     // forward output / backward dx
	unsigned char* alive;         // forward: flags out (relu), may be null
	float* var_out;
	float* inv_out;
	float* dw;
	float* db;
	int64_t N, C, S;
	int64_t chunks;               // workgroups per channel
	double dm;
	float fm, eps;
	int relu, vec, first, dw_first, db_first;
	FastDiv sdiv;                 // S, when N * S < 2^31
};

// Channel element e (0 <= e < N*S) -> its offset (n * C + c) * S + s.
template <bool FAST>
__device__ __forceinline__ int64_t channel_offset(int64_t e, const BnElemArgs& a, int64_t c) {
	int64_t n;
	if (FAST) n = (int64_t)fdiv((unsigned)e, a.sdiv);
	else n = e / a.S;
	return (n * a.C + c) * a.S + (e - n * a.S);
}

// y = (x - mean) * (weight * inv_std) + bias (ops.cpp:931-957), alive and clipping with relu. The prologue turns the
// rows' lane_sq into the channel's variance and inv_std; the channel's first workgroup stores them.
template <bool FAST>
__global__ void __launch_bounds__(256) bn_norm_kernel(const BnElemArgs a) {
	__shared__ float buf[2][256];
	__shared__ double bcast[2];
	const int tid = threadIdx.x;
	const int64_t c = blockIdx.x / a.chunks;
	const int64_t j = blockIdx.x - c * a.chunks;
	double s[2];
	channel_dsums<1>(a.rowv0, nullptr, a.N, a.C, c, buf, bcast, s);
	const float mu = a.mean[c];
	const float v = (float)(s[0] / a.dm);
	const float inv = 1.0f / sqrtf(v + a.eps);
	if (j == 0 && tid == 0) {
		if (a.var_out) a.var_out[c] = v;
		a.inv_out[c] = inv;
	}
	const float scale = a.w[c] * inv, bc = a.b[c];
	const int64_t total = a.N * a.S;
	const int64_t e0 = j * kElemChunk;
	if (a.vec) {
#pragma unroll
		for (int u = 0; u < kElemChunk / 1024; ++u) {
			const int64_t e = e0 + 4 * (tid + 256 * u);
			if (e >= total) break;
			const int64_t off = channel_offset<FAST>(e, a, c);
			const f32x4 xv = *reinterpret_cast<const f32x4*>(a.x + off);
			f32x4 o;
			unsigned fl = 0;
#pragma unroll
			for (int i = 0; i < 4; ++i) {
				const float t = (xv[i] - mu) * scale + bc;
				if (a.relu) {
					fl |= (t > 0.0f ? 1u : 0u) << (8 * i);
					o[i] = t > 0.0f ? t : 0.0f;
				} else {
					o[i] = t;
				}
			}
			*reinterpret_cast<f32x4*>(a.y + off) = o;
			if (a.relu && a.alive) *reinterpret_cast<unsigned*>(a.alive + off) = fl;
		}
	} else {
		for (int u = 0; u < kElemChunk / 256; ++u) {
			const int64_t e = e0 + tid + 256 * u;
			if (e >= total) break;
			const int64_t off = channel_offset<FAST>(e, a, c);
			const float t = (a.x[off] - mu) * scale + bc;
			if (a.relu) {
				if (a.alive) a.alive[off] = t > 0.0f;
				a.y[off] = t > 0.0f ? t : 0.0f;
			} else {
				a.y[off] = t;
			}
		}
	}
}

// The backward rule's per-channel part (ops.cpp:970-999): the prologue adds the rows' sums in double, the
// channel's first workgroup adds sdy into db and sdg * inv_std into dw, and every workgroup writes its chunk of
// dx = k * (M * g' - a - ((x - mean) * inv_std) * b) with k = weight * inv_std / M, g' masked by alive.
template <bool FAST>
__global__ void __launch_bounds__(256) bn_dx_kernel(const BnElemArgs a) {
	__shared__ float buf[2][256];
	__shared__ double bcast[2];
	const int tid = threadIdx.x;
	const int64_t c = blockIdx.x / a.chunks;
	const int64_t j = blockIdx.x - c * a.chunks;
	double s[2];
	channel_dsums<2>(a.rowv0, a.rowv1, a.N, a.C, c, buf, bcast, s);
	const float mu = a.mean[c], inv = a.inv_in[c];
	const double sdy = s[0], sdyx = s[1] * (double)inv;
	if (j == 0 && tid == 0) {
		if (a.db) a.db[c] = a.db_first ? 0.0f + (float)sdy : a.db[c] + (float)sdy;
		if (a.dw) a.dw[c] = a.dw_first ? 0.0f + (float)sdyx : a.dw[c] + (float)sdyx;
	}
	if (!a.y) return;
	const float kk = a.w[c] * inv / a.fm, fm = a.fm, av = (float)sdy, bb = (float)sdyx;
	const int64_t total = a.N * a.S;
	const int64_t e0 = j * kElemChunk;
	const bool masked = a.alive_in != nullptr;
	if (a.vec) {
#pragma unroll
		for (int u = 0; u < kElemChunk / 1024; ++u) {
			const int64_t e = e0 + 4 * (tid + 256 * u);
			if (e >= total) break;
			const int64_t off = channel_offset<FAST>(e, a, c);
			const f32x4 gv = *reinterpret_cast<const f32x4*>(a.g + off);
			const f32x4 xv = *reinterpret_cast<const f32x4*>(a.x + off);
			const unsigned fl = masked ? *reinterpret_cast<const unsigned*>(a.alive_in + off) : 0x01010101u;
			f32x4 old = a.first ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : *reinterpret_cast<const f32x4*>(a.y + off);
			f32x4 o;
#pragma unroll
			for (int i = 0; i < 4; ++i) {
				const float gm = masked ? (((fl >> (8 * i)) & 0xffu) ? gv[i] : 0.0f) : gv[i];
				const float term = kk * (fm * gm - av - ((xv[i] - mu) * inv) * bb);
				o[i] = a.first ? term + 0.0f : old[i] + term;
			}
			*reinterpret_cast<f32x4*>(a.y + off) = o;
		}
	} else {
		for (int u = 0; u < kElemChunk / 256; ++u) {
			const int64_t e = e0 + tid + 256 * u;
			if (e >= total) break;
			const int64_t off = channel_offset<FAST>(e, a, c);
			const float gm = masked ? (a.alive_in[off] ? a.g[off] : 0.0f) : a.g[off];
			const float term = kk * (fm * gm - av - ((a.x[off] - mu) * inv) * bb);
			a.y[off] = a.first ? term + 0.0f : a.y[off] + term;
		}
	}
}

// layernorm forward, one thread per row (ops.cpp:1017-1030): the row's sum and its sum of squared deviations are
// single float chains in column order.
__global__ void __launch_bounds__(256) ln_forward_kernel(const float* __restrict__ x, const float* __restrict__ gm,
                                                         const float* __restrict__ bt, int64_t R, int D, float fd,
                                                         float eps, float* __restrict__ y, float* __restrict__ mean,
                                                         float* __restrict__ inv_std, int vec) {
	const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (r >= R) return;
	const float* row = x + r * D;
	float* out = y + r * D;
	float sum = 0.0f;
	if (vec) {
		for (int j = 0; j < D; j += 4) {
			const f32x4 v = *reinterpret_cast<const f32x4*>(row + j);
			sum = sum + v[0];
			sum = sum + v[1];
			sum = sum + v[2];
			sum = sum + v[3];
		}
	} else {
		for (int j = 0; j < D; ++j) sum = sum + row[j];
	}
	const float mu = sum / fd;
	float sq = 0.0f;
	if (vec) {
		for (int j = 0; j < D; j += 4) {
			const f32x4 v = *reinterpret_cast<const f32x4*>(row + j);
#pragma unroll
			for (int i = 0; i < 4; ++i) sq = sq + (v[i] - mu) * (v[i] - mu);
		}
	} else {
		for (int j = 0; j < D; ++j) sq = sq + (row[j] - mu) * (row[j] - mu);
	}
	const float inv = 1.0f / sqrtf(sq / fd + eps);
	mean[r] = mu;
	inv_std[r] = inv;
	if (vec) {
		for (int j = 0; j < D; j += 4) {
			const f32x4 v = *reinterpret_cast<const f32x4*>(row + j);
			const f32x4 g = *reinterpret_cast<const f32x4*>(gm + j);
			const f32x4 b = *reinterpret_cast<const f32x4*>(bt + j);
			f32x4 o;
#pragma unroll
			for (int i = 0; i < 4; ++i) o[i] = (v[i] - mu) * inv * g[i] + b[i];
			*reinterpret_cast<f32x4*>(out + j) = o;
		}
	} else {
		for (int j = 0; j < D; ++j) out[j] = (row[j] - mu) * inv * gm[j] + bt[j];
	}
}

struct LnBwdArgs {
	const float* g;
	const float* x;
	const float* gm;
	const float* mean;
	const float* inv;
	float* dx;
	float* dgamma;
	float* dbeta;
	int64_t R;
	int D;
	float fd;
	int dx_first, dg_first, db_first;
	unsigned row_blocks;  // blocks [0, row_blocks) own rows (dx), the rest own columns (dgamma, dbeta)
};

// layernorm backward: blocks below row_blocks give each thread a row of dx (ops.cpp:1043-1060), the others each
// thread a column of dgamma and dbeta, summed over the rows in order (ops.cpp:1061-1076).
__global__ void __launch_bounds__(256) ln_backward_kernel(const LnBwdArgs a) {
	if (blockIdx.x < a.row_blocks) {
		const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
		if (r >= a.R) return;
		const float* gr = a.g + r * a.D;
		const float* xr = a.x + r * a.D;
		float* dr = a.dx + r * a.D;
		const float mu = a.mean[r], inv = a.inv[r];
		float sa = 0.0f, sb = 0.0f;
		for (int j = 0; j < a.D; ++j) {
			const float dxhat = gr[j] * a.gm[j];
			sa = sa + dxhat;
			sb = sb + dxhat * ((xr[j] - mu) * inv);
		}
		const float k = inv / a.fd, fd = a.fd;
		for (int j = 0; j < a.D; ++j) {
			const float dxhat = gr[j] * a.gm[j];
			const float term = k * (fd * dxhat - sa - ((xr[j] - mu) * inv) * sb);
			dr[j] = a.dx_first ? term + 0.0f : dr[j] + term;
		}
		return;
	}
	const int64_t col = (int64_t)(blockIdx.x - a.row_blocks) * 256 + threadIdx.x;
	if (col >= a.D) return;
	float sg = 0.0f, sb = 0.0f;
	int64_t r = 0;
	for (; r + 8 <= a.R; r += 8) {
		float gv[8], xv[8], mv[8], iv[8];
#pragma unroll
		for (int u = 0; u < 8; ++u) {
			gv[u] = a.g[(r + u) * a.D + col];
			xv[u] = a.x[(r + u) * a.D + col];
			mv[u] = a.mean[r + u];
			iv[u] = a.inv[r + u];
		}
#pragma unroll
		for (int u = 0; u < 8; ++u) {
			sg = sg + gv[u] * ((xv[u] - mv[u]) * iv[u]);
			sb = sb + gv[u];
		}
	}
	for (; r < a.R; ++r) {
		const float gv = a.g[r * a.D + col];
		sg = sg + gv * ((a.x[r * a.D + col] - a.mean[r]) * a.inv[r]);
		sb = sb + gv;
	}
	if (a.dgamma) a.dgamma[col] = a.dg_first ? 0.0f + sg : a.dgamma[col] + sg;
	if (a.dbeta) a.dbeta[col] = a.db_first ? 0.0f + sb : a.dbeta[col] + sb;
}

// ---- layernorm with its rows staged in LDS ----
// A workgroup owns `rw` consecutive rows (a contiguous block of rw * D floats): its 256 threads copy the block into
// LDS with 16-byte coalesced loads, all issued before the first LDS store (row pitch D + 1, so lane r walking row r
// hits bank (r + j) mod 64), lane r of wave 0 runs row r's chains over LDS and writes its outputs back into its LDS
// row, and the 256 threads copy the block out with coalesced stores. The LDS budget is 64 KB of floats (16384):
// rw = min(64, 16384 / (D + 1)) rows for the forward, about half of that for the backward (g and x), and no more
// than R / 256 rows when that leaves about 256 workgroups on a small input.

constexpr int kLnLdsFloats = 16384;
constexpr int kLnLoadPer = kLnLdsFloats / 4 / 256;  // float4 loads per thread for a full block (16)

__device__ __forceinline__ void ln_block_load(const float* __restrict__ src, int nr, int D, int pitch, int vec,
                                              const FastDiv& dq, float* dst) {
	const int tid = threadIdx.x;
	const int total = nr * D;
	if (vec) {
		const int q4 = D >> 2, tot = total >> 2;
		if (tot == 0) return;
		f32x4 v[kLnLoadPer];
#pragma unroll
		for (int u = 0; u < kLnLoadPer; ++u) {
			const int q = min(tid + 256 * u, tot - 1);
			v[u] = *reinterpret_cast<const f32x4*>(src + 4 * q);
		}
#pragma unroll
		for (int u = 0; u < kLnLoadPer; ++u) {
			const int q = tid + 256 * u;
			if (q < tot) {
				const int r = (int)fdiv((unsigned)q, dq), c = 4 * (q - r * q4);
#pragma unroll
				for (int i = 0; i < 4; ++i) dst[r * pitch + c + i] = v[u][i];
			}
		}
	} else {
		for (int b = 0; b < total; b += 256 * 16) {
			float v[16];
#pragma unroll
			for (int u = 0; u < 16; ++u) v[u] = src[min(b + tid + 256 * u, total - 1)];
#pragma unroll
			for (int u = 0; u < 16; ++u) {
				const int e = b + tid + 256 * u;
				if (e < total) {
					const int r = (int)fdiv((unsigned)e, dq);
					dst[r * pitch + e - r * D] = v[u];
				}
			}
		}
	}
}

// dst (global) = block in LDS; with add, dst = old + block (the backward's accumulate).
__device__ __forceinline__ void ln_block_store(float* __restrict__ dst, int nr, int D, int pitch, int vec,
                                               const FastDiv& dq, const float* src, bool add) {
	const int tid = threadIdx.x;
	const int total = nr * D;
	if (vec) {
		const int q4 = D >> 2, tot = total >> 2;
		for (int q = tid; q < tot; q += 256) {
			const int r = (int)fdiv((unsigned)q, dq), c = 4 * (q - r * q4);
			f32x4 v;
#pragma unroll
			for (int i = 0; i < 4; ++i) v[i] = src[r * pitch + c + i];
			if (add) {
				const f32x4 o = *reinterpret_cast<const f32x4*>(dst + 4 * q);
#pragma unroll
				for (int i = 0; i < 4; ++i) v[i] = o[i] + v[i];
			}
			*reinterpret_cast<f32x4*>(dst + 4 * q) = v;
		}
	} else {
		for (int e = tid; e < total; e += 256) {
			const int r = (int)fdiv((unsigned)e, dq);
			const float v = src[r * pitch + e - r * D];
			dst[e] = add ? dst[e] + v : v;
		}
	}
}

struct LnArgs {
	const float* x;
	const float* g;       // backward: upstream gradient
	const float* gm;
	const float* bt;
	const float* mean_in;  // backward
	const float* inv_in;   // backward
	float* y;              // forward: y; backward: dx
	float* mean;           // forward
	float* inv;            // forward
	int64_t R;
	int D, rw, vec, first;
	float fd, eps;
	FastDiv dq;            // D / 4 (vec) or D
	FastDiv dd;            // D
};

// layernorm forward (ops.cpp:1017-1030) on rw rows per workgroup.
__global__ void __launch_bounds__(256) ln_forward_lds_kernel(const LnArgs a) {
	extern __shared__ __align__(16) float lds[];
	const int pitch = a.D + 1;
	const int64_t r0 = (int64_t)blockIdx.x * a.rw;
	const int nr = (int)(a.R - r0 < a.rw ? a.R - r0 : a.rw);
	ln_block_load(a.x + r0 * a.D, nr, a.D, pitch, a.vec, a.dq, lds);
	__syncthreads();
	const int r = threadIdx.x;
	if (r < nr) {
		float* row = lds + r * pitch;
		const int D16 = a.D & ~15;
		float sum = 0.0f;
		for (int j = 0; j < D16; j += 16) {  // 16 LDS reads issued, then the 16 dependent adds
			float v[16];
#pragma unroll
			for (int u = 0; u < 16; ++u) v[u] = row[j + u];
#pragma unroll
			for (int u = 0; u < 16; ++u) sum = sum + v[u];
		}
		for (int j = D16; j < a.D; ++j) sum = sum + row[j];
		const float mu = sum / a.fd;
		float sq = 0.0f;
		for (int j = 0; j < D16; j += 16) {
			float v[16];
#pragma unroll
			for (int u = 0; u < 16; ++u) v[u] = row[j + u];
#pragma unroll
			for (int u = 0; u < 16; ++u) sq = sq + (v[u] - mu) * (v[u] - mu);
		}
		for (int j = D16; j < a.D; ++j) sq = sq + (row[j] - mu) * (row[j] - mu);
		const float inv = 1.0f / sqrtf(sq / a.fd + a.eps);
		a.mean[r0 + r] = mu;
		a.inv[r0 + r] = inv;
		for (int j = 0; j < D16; j += 16) {
			float v[16];
#pragma unroll
			for (int u = 0; u < 16; ++u) v[u] = row[j + u];
#pragma unroll
			for (int u = 0; u < 16; ++u) row[j + u] = (v[u] - mu) * inv * a.gm[j + u] + a.bt[j + u];
		}
		for (int j = D16; j < a.D; ++j) row[j] = (row[j] - mu) * inv * a.gm[j] + a.bt[j];
	}
	__syncthreads();
	ln_block_store(a.y + r0 * a.D, nr, a.D, pitch, a.vec, a.dq, lds, false);
}

// layernorm backward's dx (ops.cpp:1043-1060) on rw rows per workgroup. g and x are staged in LDS; all 256 threads
// form the products dxhat * ((x - mean) * inv_std) of the second sum elementwise, so the lane that owns a row only
// runs its two addition chains (sa over g * gamma, sb over the products, both in column order); then all threads
// write dx = k * (D * dxhat - sa - xhat * sb) elementwise, straight to HBM.
__device__ __forceinline__ void ln_dx_body(const LnArgs& a, int block, float* lds) {
	const int pitch = a.D + 1;
	float* gs = lds;
	float* xs = gs + a.rw * pitch;
	float* gms = xs + a.rw * pitch;
	float* st = gms + a.D;  // per row: mean, inv_std, sa, sb
	const int tid = threadIdx.x;
	const int64_t r0 = (int64_t)block * a.rw;
	const int nr = (int)(a.R - r0 < a.rw ? a.R - r0 : a.rw);
	ln_block_load(a.g + r0 * a.D, nr, a.D, pitch, a.vec, a.dq, gs);
	ln_block_load(a.x + r0 * a.D, nr, a.D, pitch, a.vec, a.dq, xs);
	for (int j = tid; j < a.D; j += 256) gms[j] = a.gm[j];
	if (tid < nr) {
		st[4 * tid] = a.mean_in[r0 + tid];
		st[4 * tid + 1] = a.inv_in[r0 + tid];
	}
	__syncthreads();
	if (tid < nr) {
		// the row's two chains (ops.cpp:1040-1047): sa += g gamma, sb += (g gamma) ((x - mean) inv_std), each
		// product formed as the reference forms it, 16 steps' LDS reads issued before their arithmetic
		const float* gr = gs + tid * pitch;
		const float* xr = xs + tid * pitch;
		const float mu = st[4 * tid], iv = st[4 * tid + 1];
		const int D16 = a.D & ~15;
		float sa = 0.0f, sb = 0.0f;
		for (int j = 0; j < D16; j += 16) {
			float gv[16], mv[16], xv[16];
#pragma unroll
			for (int u = 0; u < 16; ++u) {
				gv[u] = gr[j + u];
				mv[u] = gms[j + u];
				xv[u] = xr[j + u];
			}
#pragma unroll
			for (int u = 0; u < 16; ++u) {
				const float dxhat = gv[u] * mv[u];
				sa = sa + dxhat;
				sb = sb + dxhat * ((xv[u] - mu) * iv);
			}
		}
		for (int j = D16; j < a.D; ++j) {
			const float dxhat = gr[j] * gms[j];
			sa = sa + dxhat;
			sb = sb + dxhat * ((xr[j] - mu) * iv);
		}
		st[4 * tid + 2] = sa;
		st[4 * tid + 3] = sb;
	}
	__syncthreads();
	const float fd = a.fd;
	float* dst = a.y + r0 * a.D;
	const int total = nr * a.D;
	for (int e = tid; e < total; e += 256) {
		const int r = (int)fdiv((unsigned)e, a.dd), j = e - r * a.D;
		const float mu = st[4 * r], inv = st[4 * r + 1], sa = st[4 * r + 2], sb = st[4 * r + 3];
		const float k = inv / fd;
		const float dxhat = gs[r * pitch + j] * gms[j];
		const float term = k * (fd * dxhat - sa - ((xs[r * pitch + j] - mu) * inv) * sb);
		dst[e] = a.first ? term + 0.0f : dst[e] + term;
	}
}

__global__ void __launch_bounds__(256) ln_dx_lds_kernel(const LnArgs a) {
	extern __shared__ __align__(16) float lds[];
	ln_dx_body(a, (int)blockIdx.x, lds);
}

// layernorm backward's dgamma and dbeta (ops.cpp:1061-1076): each is a chain down a column in row order, so the
// columns are the only parallelism. A workgroup owns 32 columns and streams the rows in chunks of 120. Waves 1-15
// produce: each thread loads four rows of its column (or, VEC, one row's four columns with 16-byte loads) with the
// rows' mean and inv_std, four chunks ahead in a register ring, and writes g * ((x - mean) * inv_std), formed
// exactly as the reference forms it, and g into the chunk's LDS buffer (a row of 64 floats: the products, then g,
// so wave 0 reads 64 consecutive words). Wave 0 consumes one chunk behind: lanes 0-31 add the products down their
// column (dgamma), lanes 32-63 add g (dbeta), 24 rows' LDS reads in flight while they add eight. One barrier per
// chunk; two buffers. Measured at [32, 256, 512]: 53 us (the chains of 8192 rows bound it near 23 us; 8-column
// blocks, 4x the workgroups, and a raised wave priority for the chains measured no faster).
constexpr int kLnCols = 32, kLnProducers = 960, kLnThreads = 64 + kLnProducers, kLnAhead = 4, kLnPer = 4;
constexpr int kLnRowStride = kLnProducers / kLnCols;  // 30: a scalar producer's rows are rr + 30 u
constexpr int kLnChunk = kLnRowStride * kLnPer;       // 120 rows
constexpr int kLnVecPerRow = kLnCols / 4;             // 8 16-byte loads cover a row's columns

template <bool VEC>
__global__ void __launch_bounds__(kLnThreads) ln_dgamma_kernel(const float* __restrict__ g,
                                                               const float* __restrict__ x,
                                                               const float* __restrict__ mean,
                                                               const float* __restrict__ inv, int64_t R, int D,
                                                               float* dgamma, int dg_first, float* dbeta,
                                                               int db_first) {
	__shared__ __align__(16) float buf[2][kLnChunk][2 * kLnCols];
	const int tid = threadIdx.x;
	const int c0 = blockIdx.x * kLnCols;
	const int64_t chunks = (R + kLnChunk - 1) / kLnChunk;
	const bool producer = tid >= 64;
	const bool consumer = !producer;
	const int pt = tid - 64;
	// scalar: column c of rows rr + 30 u; VEC: columns 4 q4 .. 4 q4 + 3 of row vr
	const int c = pt % kLnCols, rr = pt / kLnCols;
	const int q4 = pt % kLnVecPerRow, vr = pt / kLnVecPerRow;
	constexpr int kVecRows = kLnProducers / kLnVecPerRow;  // 120: one row per producer thread and chunk
	static_assert(kVecRows == kLnChunk, "a VEC producer owns one row of a chunk");
	const int col = min(c0 + c, D - 1);
	const int col4 = min(c0 + 4 * q4, D - 4);
	float gv[kLnAhead][kLnPer], xv[kLnAhead][kLnPer], mv[kLnAhead][kLnPer], iv[kLnAhead][kLnPer];
	auto load = [&](int64_t ch, int slot) {
		if (VEC) {
			const int64_t r = min(ch * kLnChunk + vr, R - 1);
			const f32x4 g4 = *reinterpret_cast<const f32x4*>(g + r * D + col4);
			const f32x4 x4 = *reinterpret_cast<const f32x4*>(x + r * D + col4);
			const float m = mean[r], iv0 = inv[r];
#pragma unroll
			for (int u = 0; u < 4; ++u) {
				gv[slot][u] = g4[u];
				xv[slot][u] = x4[u];
				mv[slot][u] = m;
				iv[slot][u] = iv0;
			}
			return;
		}
#pragma unroll
		for (int u = 0; u < kLnPer; ++u) {
			const int64_t r = min(ch * kLnChunk + rr + kLnRowStride * u, R - 1);
			gv[slot][u] = g[r * D + col];
			xv[slot][u] = x[r * D + col];
			mv[slot][u] = mean[r];
			iv[slot][u] = inv[r];
		}
	};
	// the consumer's chain over n rows of buffer b: batches of eight rows in a ring of four, three batches' LDS reads
	// in flight while one batch's eight dependent adds run
	auto chain = [&](float& acc, int b, int n) {
		const float* v = &buf[b][0][tid];
		if (n == kLnChunk) {
			constexpr int kB = kLnChunk / 8;
			float t[4][8];
#pragma unroll
			for (int q = 0; q < 3; ++q)
#pragma unroll
				for (int u = 0; u < 8; ++u) t[q][u] = v[(8 * q + u) * 2 * kLnCols];
#pragma unroll
			for (int q = 0; q < kB; ++q) {
				if (q + 3 < kB) {
#pragma unroll
					for (int u = 0; u < 8; ++u) t[(q + 3) & 3][u] = v[(8 * (q + 3) + u) * 2 * kLnCols];
				}
#pragma unroll
				for (int u = 0; u < 8; ++u) acc = acc + t[q & 3][u];
			}
		} else {
			for (int i = 0; i < n; ++i) acc = acc + v[i * 2 * kLnCols];
		}
	};
	static_assert(kLnChunk % 8 == 0 && kLnChunk >= 24, "the chain reads batches of eight rows, three ahead");
	if (producer) {
#pragma unroll
		for (int k = 0; k < kLnAhead; ++k)
			if (k < chunks) load(k, k);
	}
	float acc = 0.0f;
	for (int64_t base = 0; base < chunks; base += kLnAhead) {
#pragma unroll
		for (int k = 0; k < kLnAhead; ++k) {
			const int64_t ch = base + k;
			if (ch >= chunks) break;
			const int b = (int)(ch & 1);
			if (producer) {
				if (VEC) {
					// columns past D read a clamped address: their values are never used
					f32x4 pr, gg;
#pragma unroll
					for (int u = 0; u < 4; ++u) {
						pr[u] = gv[k][u] * ((xv[k][u] - mv[k][u]) * iv[k][u]);
						gg[u] = gv[k][u];
					}
					*reinterpret_cast<f32x4*>(&buf[b][vr][4 * q4]) = pr;
					*reinterpret_cast<f32x4*>(&buf[b][vr][kLnCols + 4 * q4]) = gg;
				} else {
#pragma unroll
					for (int u = 0; u < kLnPer; ++u) {
						const int row = rr + kLnRowStride * u;
						buf[b][row][c] = gv[k][u] * ((xv[k][u] - mv[k][u]) * iv[k][u]);
						buf[b][row][kLnCols + c] = gv[k][u];
					}
				}
				if (ch + kLnAhead < chunks) load(ch + kLnAhead, k);
			} else if (consumer && ch > 0) {
				chain(acc, b ^ 1, kLnChunk);  // chunk ch - 1 is whole
			}
			__syncthreads();
		}
	}
	if (consumer && chunks > 0) {
		const int64_t last = chunks - 1;
		chain(acc, (int)(last & 1), (int)(R - last * kLnChunk));
	}
	if (consumer && c0 + (tid % kLnCols) < D) {
		const int j = c0 + tid % kLnCols;
		if (tid < kLnCols) {
			if (dgamma) dgamma[j] = dg_first ? 0.0f + acc : dgamma[j] + acc;
		} else {
			if (dbeta) dbeta[j] = db_first ? 0.0f + acc : dbeta[j] + acc;
		}
	}
}

// dgamma and dbeta for at most 1024 rows (transformer_tiny's 16 x 64 tokens): the same chains, one pass. A
// workgroup owns a few columns (four with 1024 threads alone, one with 256 threads beside dx, so that the loads
// spread over many CUs); every thread loads its share of a column's rows (g, x, the rows' mean and inv_std, all in
// flight at once) and parks g * ((x - mean) * inv_std) and g in LDS, column by column; then one lane per column adds
// the products down it in row order (dgamma) and one the gradients (dbeta), four rows per 16-byte LDS read. Rows
// past R are parked as +0: a chain from +0 never holds -0 (x + (-x) rounds to +0, and no sum of finite floats
// underflows to zero), so adding +0 leaves it unchanged.
constexpr int kLnSmallRows = 1024, kLnSmallThreads = 1024;
constexpr int kLnSmallCols = 4;     // columns of a workgroup of the standalone kernel
constexpr int kLnMergedCols = 1;    // columns of a 256-thread workgroup beside dx
constexpr int kLnSmallPitch = kLnSmallRows + 4;  // a column's rows, padded against bank conflicts of the stores
constexpr size_t kLnMergedLds = 2 * kLnMergedCols * kLnSmallPitch * sizeof(float);

struct LnSmallArgs {
	const float* g;
	const float* x;
	const float* mean;
	const float* inv;
	int R, D;
	float* dgamma;
	int dg_first;
	float* dbeta;
	int db_first;
	int blocks;  // workgroups of the column chains
};

// block: the workgroup's index among the chains' workgroups; THREADS its size, COLS its columns; buf:
// 2 COLS kLnSmallPitch floats of LDS.
template <int THREADS, int COLS>
__device__ __forceinline__ void ln_dgamma_small_body(const LnSmallArgs& d, int block, float* buf) {
	constexpr int kRowStep = THREADS / COLS;
	constexpr int kPer = kLnSmallRows / kRowStep;
	const int R = d.R, D = d.D;
	const int tid = threadIdx.x;
	const int c = tid % COLS, r0 = tid / COLS;  // rows r0 + kRowStep u
	const int c0 = block * COLS;
	const int col = min(c0 + c, D - 1);
	float gv[kPer], xv[kPer], mv[kPer], iv[kPer];
#pragma unroll
	for (int u = 0; u < kPer; ++u) {
		const int64_t r = min(r0 + kRowStep * u, R - 1);
		gv[u] = d.g[r * D + col];
		xv[u] = d.x[r * D + col];
		mv[u] = d.mean[r];
		iv[u] = d.inv[r];
	}
	// the chains read whole blocks of 32 rows
	const int rpad = (R + 31) & ~31;
#pragma unroll
	for (int u = 0; u < kPer; ++u) {
		const int r = r0 + kRowStep * u;
		if (r < rpad) {
			const bool in = r < R;
			buf[c * kLnSmallPitch + r] = in ? gv[u] * ((xv[u] - mv[u]) * iv[u]) : 0.0f;
			buf[(COLS + c) * kLnSmallPitch + r] = in ? gv[u] : 0.0f;
		}
	}
	__syncthreads();
	if (tid >= 2 * COLS) return;
	// lane c: column c's products (dgamma); lane COLS + c: its gradients (dbeta). Rows in order, 32 at a time; the
	// reads of the next two blocks are in flight while one is added (a dependent add takes about six cycles).
	const f32x4* v = reinterpret_cast<const f32x4*>(buf + tid * kLnSmallPitch);
	const int nb = rpad / 32;
	float acc = 0.0f;
	f32x4 t[3][8];
#pragma unroll
	for (int e = 0; e < 8; ++e) t[0][e] = v[e];
	if (nb > 1) {
#pragma unroll
		for (int e = 0; e < 8; ++e) t[1][e] = v[8 + e];
	}
	for (int b = 0; b < nb; b += 3) {
#pragma unroll
		for (int k = 0; k < 3; ++k) {
			if (b + k >= nb) break;
			if (b + k + 2 < nb) {
#pragma unroll
				for (int e = 0; e < 8; ++e) t[(k + 2) % 3][e] = v[8 * (b + k + 2) + e];
			}
#pragma unroll
			for (int e = 0; e < 8; ++e)
#pragma unroll
				for (int q = 0; q < 4; ++q) acc = acc + t[k][e][q];
		}
	}
	if (c0 + c >= D) return;
	const int j = c0 + c;
	if (tid < COLS) {
		if (d.dgamma) d.dgamma[j] = d.dg_first ? 0.0f + acc : d.dgamma[j] + acc;
	} else {
		if (d.dbeta) d.dbeta[j] = d.db_first ? 0.0f + acc : d.dbeta[j] + acc;
	}
}

__global__ void __launch_bounds__(kLnSmallThreads) ln_dgamma_small_kernel(const LnSmallArgs d) {
	__shared__ __align__(16) float buf[2 * kLnSmallCols * kLnSmallPitch];
	ln_dgamma_small_body<kLnSmallThreads, kLnSmallCols>(d, (int)blockIdx.x, buf);
}

// dx and the column chains of one layernorm backward in one launch (up to 1024 rows): a workgroup per column for
// the chains, first, so that the longest work starts first, then the dx row blocks beside them on the other CUs.
__global__ void __launch_bounds__(256) ln_backward_small_kernel(const LnArgs a, const LnSmallArgs d) {
	extern __shared__ __align__(16) float lds[];
	if ((int)blockIdx.x < d.blocks) ln_dgamma_small_body<256, kLnMergedCols>(d, (int)blockIdx.x, lds);
	else ln_dx_body(a, (int)blockIdx.x - d.blocks, lds);
}

inline bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

template <int MODE>
hipError_t launch_rows(BnRowArgs& a, hipStream_t s) {
	a.groups = (int)((a.N + kRows - 1) / kRows);
	const int64_t blocks = a.C * (a.groups > 0 ? a.groups : 1);
	if (a.groups == 0) a.groups = 1;
	hipLaunchKernelGGL(bn_rows_kernel<MODE>, dim3((unsigned)blocks), dim3(256), 0, s, a);
	return hipGetLastError();
}

hipError_t launch_elem(bool fwd, BnElemArgs& a, hipStream_t s) {
	const int64_t total = a.N * a.S;
	a.chunks = total > 0 ? (total + kElemChunk - 1) / kElemChunk : 1;
	const bool fast = total < ((int64_t)1 << 31) && a.S > 0 && a.S < ((int64_t)1 << 31);
	if (fast) a.sdiv = make_fastdiv((unsigned)a.S);
	const dim3 grid((unsigned)(a.C * a.chunks));
	if (fwd) {
		if (fast) hipLaunchKernelGGL(bn_norm_kernel<true>, grid, dim3(256), 0, s, a);
		else hipLaunchKernelGGL(bn_norm_kernel<false>, grid, dim3(256), 0, s, a);
	} else {
		if (fast) hipLaunchKernelGGL(bn_dx_kernel<true>, grid, dim3(256), 0, s, a);
		else hipLaunchKernelGGL(bn_dx_kernel<false>, grid, dim3(256), 0, s, a);
	}
	return hipGetLastError();
}

}  // namespace

hipError_t batchnorm_forward(const float* x, const float* w, const float* b, const BnGeom& g, float eps, int relu,
                             float* y, unsigned char* alive, float* mean, float* var, float* inv_std, float* scratch,
                             hipStream_t s) {
	if (g.C == 0) return hipSuccess;
	const bool vec = g.S % 4 == 0 && aligned16(x) && aligned16(y) && (!alive || reinterpret_cast<uintptr_t>(alive) % 4 == 0);
	float* rowsum = scratch;
	float* rowsq = scratch + g.N * g.C;
	BnRowArgs r{};
	r.x = x;
	r.out0 = rowsum;
	r.N = g.N;
	r.C = g.C;
	r.S = g.S;
	r.dm = g.dm;
	r.vec = g.S % 4 == 0 && aligned16(x);
	hipError_t e = hipSuccess;
	if (g.N > 0) {
		e = launch_rows<kSum>(r, s);
		if (e != hipSuccess) return e;
	}
	r.rowsum = rowsum;
	r.out0 = rowsq;
	r.mean_out = mean;
	e = launch_rows<kSq>(r, s);  // also writes the channel means (a workgroup per channel when N is 0)
	if (e != hipSuccess) return e;
	BnElemArgs a{};
	a.x = x;
	a.w = w;
	a.b = b;
	a.rowv0 = rowsq;
	a.mean = mean;
	a.y = y;
	a.alive = alive;
	a.var_out = var;
	a.inv_out = inv_std;
	a.N = g.N;
	a.C = g.C;
	a.S = g.S;
	a.dm = g.dm;
	a.fm = g.fm;
	a.eps = eps;
	a.relu = relu;
	a.vec = vec;
	return launch_elem(true, a, s);
}

hipError_t batchnorm_backward(const float* gy, const float* x, const unsigned char* alive, const float* w,
                              const float* mean, const float* inv_std, const BnGeom& g, float* dx, int dx_first,
                              float* dw, int dw_first, float* db, int db_first, float* scratch, hipStream_t s) {
	if (g.C == 0 || (!dx && !dw && !db)) return hipSuccess;
	float* rowdy = scratch;
	float* rowdg = scratch + g.N * g.C;
	if (g.N > 0) {
		BnRowArgs r{};
		r.x = x;
		r.g = gy;
		r.alive = alive;
		r.mean = mean;
		r.out0 = rowdy;
		r.out1 = rowdg;
		r.N = g.N;
		r.C = g.C;
		r.S = g.S;
		r.dm = g.dm;
		r.vec = g.S % 4 == 0 && aligned16(x) && aligned16(gy) && (!alive || reinterpret_cast<uintptr_t>(alive) % 4 == 0);
		const hipError_t e = launch_rows<kBwd>(r, s);
		if (e != hipSuccess) return e;
	}
	BnElemArgs a{};
	a.x = x;
	a.g = gy;
	a.alive_in = alive;
	a.w = w;
	a.rowv0 = rowdy;
	a.rowv1 = rowdg;
	a.mean = mean;
	a.inv_in = inv_std;
	a.y = dx;
	a.dw = dw;
	a.db = db;
	a.N = g.N;
	a.C = g.C;
	a.S = g.S;
	a.dm = g.dm;
	a.fm = g.fm;
	a.first = dx_first;
	a.dw_first = dw_first;
	a.db_first = db_first;
	a.vec = g.S % 4 == 0 && aligned16(x) && aligned16(gy) && aligned16(dx) &&
	        (!alive || reinterpret_cast<uintptr_t>(alive) % 4 == 0);
	return launch_elem(false, a, s);
}

hipError_t layernorm_forward(const float* x, const float* gamma, const float* beta, int64_t R, int D, float fd,
                             float eps, float* y, float* mean, float* inv_std, hipStream_t s) {
	if (R == 0) return hipSuccess;
	// as many rows per workgroup as LDS holds, but few enough for about 256 workgroups when the rows are few
	const int rw = (int)std::min<int64_t>(std::min<int64_t>(std::min(64, kLnLdsFloats / (D + 1)), R), std::max<int64_t>(1, (R + 255) / 256));
	if (rw >= 1 && R / rw < ((int64_t)1 << 31) && (int64_t)rw * D < ((int64_t)1 << 31)) {
		LnArgs a{};
		a.x = x;
		a.gm = gamma;
		a.bt = beta;
		a.y = y;
		a.mean = mean;
		a.inv = inv_std;
		a.R = R;
		a.D = D;
		a.rw = rw;
		a.fd = fd;
		a.eps = eps;
		a.vec = D % 4 == 0 && aligned16(x) && aligned16(y);
		a.dq = make_fastdiv((unsigned)(a.vec ? D / 4 : D));
		hipLaunchKernelGGL(ln_forward_lds_kernel, dim3((unsigned)((R + rw - 1) / rw)), dim3(256),
		                   (size_t)rw * (D + 1) * sizeof(float), s, a);
		return hipGetLastError();
	}
	const int vec = D % 4 == 0 && aligned16(x) && aligned16(y) && aligned16(gamma) && aligned16(beta);
	hipLaunchKernelGGL(ln_forward_kernel, dim3((unsigned)((R + 255) / 256)), dim3(256), 0, s, x, gamma, beta, R, D, fd,
	                   eps, y, mean, inv_std, vec);
	return hipGetLastError();
}

hipError_t layernorm_backward(const float* gy, const float* x, const float* gamma, const float* mean,
                              const float* inv_std, int64_t R, int D, float fd, float* dx, int dx_first,
                              float* dgamma, int dgamma_first, float* dbeta, int dbeta_first, hipStream_t s) {
	if (R == 0 && !dgamma && !dbeta) return hipSuccess;
	const int rw = (int)std::min<int64_t>(std::min<int64_t>(std::min(64, (kLnLdsFloats - D) / (2 * (D + 1) + 4)),
	                                                        std::max<int64_t>(R, 1)),
	                                      std::max<int64_t>(1, (R + 255) / 256));
	if (rw >= 1 && R / rw < ((int64_t)1 << 31) && (int64_t)rw * D < ((int64_t)1 << 31)) {
		LnArgs a{};
		a.g = gy;
		a.x = x;
		a.gm = gamma;
		a.mean_in = mean;
		a.inv_in = inv_std;
		a.y = dx;
		a.R = R;
		a.D = D;
		a.rw = rw;
		a.fd = fd;
		a.first = dx_first;
		a.vec = D % 4 == 0 && aligned16(x) && aligned16(gy) && aligned16(dx);
		a.dq = make_fastdiv((unsigned)(a.vec ? D / 4 : D));
		a.dd = make_fastdiv((unsigned)D);
		const size_t dx_lds = ((size_t)2 * rw * (D + 1) + D + 4 * rw) * sizeof(float);
		const int64_t dx_blocks = (R + rw - 1) / rw;
		const bool small = (dgamma || dbeta) && R > 0 && R <= kLnSmallRows;
		LnSmallArgs d{gy, x, mean, inv_std, (int)R, D, dgamma, dgamma_first, dbeta, dbeta_first,
		              (D + kLnMergedCols - 1) / kLnMergedCols};
		if (dx && R > 0 && small && dx_blocks + d.blocks < ((int64_t)1 << 31)) {
			hipLaunchKernelGGL(ln_backward_small_kernel, dim3((unsigned)(d.blocks + dx_blocks)), dim3(256),
			                   std::max(dx_lds, kLnMergedLds), s, a, d);
			return hipGetLastError();
		}
		d.blocks = (D + kLnSmallCols - 1) / kLnSmallCols;
		if (dx && R > 0) {
			hipLaunchKernelGGL(ln_dx_lds_kernel, dim3((unsigned)dx_blocks), dim3(256), dx_lds, s, a);
			const hipError_t e = hipGetLastError();
			if (e != hipSuccess) return e;
		}
		if (small)
			hipLaunchKernelGGL(ln_dgamma_small_kernel, dim3((unsigned)d.blocks), dim3(kLnSmallThreads), 0, s, d);
		else if ((dgamma || dbeta) && D % 4 == 0 && aligned16(gy) && aligned16(x))
			hipLaunchKernelGGL(ln_dgamma_kernel<true>, dim3((unsigned)((D + kLnCols - 1) / kLnCols)), dim3(kLnThreads), 0, s,
			                   gy, x, mean, inv_std, R, D, dgamma, dgamma_first, dbeta, dbeta_first);
		else if (dgamma || dbeta)
			hipLaunchKernelGGL(ln_dgamma_kernel<false>, dim3((unsigned)((D + kLnCols - 1) / kLnCols)), dim3(kLnThreads), 0, s,
			                   gy, x, mean, inv_std, R, D, dgamma, dgamma_first, dbeta, dbeta_first);
		return hipGetLastError();
	}
	LnBwdArgs a{};
	a.g = gy;
	a.x = x;
	a.gm = gamma;
	a.mean = mean;
	a.inv = inv_std;
	a.dx = dx;
	a.dgamma = dgamma;
	a.dbeta = dbeta;
	a.R = R;
	a.D = D;
	a.fd = fd;
	a.dx_first = dx_first;
	a.dg_first = dgamma_first;
	a.db_first = dbeta_first;
	a.row_blocks = dx ? (unsigned)((R + 255) / 256) : 0u;
	const unsigned col_blocks = (dgamma || dbeta) ? (unsigned)((D + 255) / 256) : 0u;
	if (a.row_blocks + col_blocks == 0) return hipSuccess;
	hipLaunchKernelGGL(ln_backward_kernel, dim3(a.row_blocks + col_blocks), dim3(256), 0, s, a);
	return hipGetLastError();
}

}  // namespace nnh
