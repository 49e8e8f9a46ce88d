// softmax.hip - the attention row softmax and its backward, with nn-cpp's exact operation order.
//
// masked_softmax_row (src/autograd/ops.cpp:1183-1204), per row i of length Tk:
//   v_j = s_j * scale; padded key -> -1e9; causal j > i -> -2e9
//   m = v_0, then m = (m < v_j) ? v_j : m       (std::max)
//   p_j = exp(v_j - m) for j < live (live = i + 1 when causal), exactly 0 beyond
//   sum = ((0 + p_0) + p_1) + ...  in j order;  p_j = p_j / sum  (as div_by_row_sum: the same rounding)
// A block holds up to 64 rows in LDS. Loads and stores are batched 16-byte accesses; the elementwise steps
// run on every lane. The max is a wave reduction that reproduces std::max's scan exactly (see row_max); the
// sum, whose rounding depends on its order, runs one lane per row in j order, as the reference's loop does.
#include "softmax.hpp"
#include "softmax_row.hpp"
#include "fastdiv.hpp"

#include <math.h>

namespace nnh {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kUnroll = 8;  // 16-byte loads each thread keeps in flight

struct RowGeom {
	int64_t rows;     // total rows
	int tk;           // row length
	int tq;           // rows per (sample, head): row r has query index i = r % tq
	int heads;        // sample of row r: n = r / (heads * tq)
	float scale;
	const float* pad; // {N, Tk} key padding mask (0 marks a padded key) or null
	int causal;
	FastDiv fq, fhq;  // division by tq and by heads * tq (rows < 2^31)
};

__device__ __forceinline__ int query_index(const RowGeom& g, int64_t row) {
	return (int)((unsigned)row - fdiv((unsigned)row, g.fq) * (unsigned)g.tq);
}

__device__ __forceinline__ const float* pad_row(const RowGeom& g, int64_t row) {
	return g.pad ? g.pad + (int64_t)fdiv((unsigned)row, g.fhq) * g.tk : nullptr;
}

__device__ __forceinline__ float masked_value(float s, const RowGeom& g, int64_t row, int j) {
	float v = s * g.scale;
	if (g.pad && pad_row(g, row)[j] == 0.0f) v = -1e9f;
	if (g.causal && j > query_index(g, row)) v = -2e9f;
	return v;
}

__device__ __forceinline__ int live_keys(const RowGeom& g, int64_t row) {
	return g.causal ? min(g.tk, query_index(g, row) + 1) : g.tk;
}

// Copies rows r0 .. r0+nr-1 of src (row length tk) into LDS rows of stride ld, applying f(value, row, j).
// 16-byte loads when vec (tk % 4 == 0, src 16-byte aligned), kUnroll of them in flight per thread.
template <typename F>
__device__ __forceinline__ void load_rows(const float* src, float* sm, int64_t r0, int nr, int tk, int ld,
                                          bool vec, FastDiv per_row, F f) {
	const int tid = threadIdx.x;
	if (vec) {
		const unsigned total = (unsigned)(nr * (tk / 4));
		const f32x4* s4 = reinterpret_cast<const f32x4*>(src + r0 * tk);
		for (unsigned base = tid; base < total; base += kThreads * kUnroll) {
			f32x4 v[kUnroll];
#pragma unroll
			for (int u = 0; u < kUnroll; ++u) {
				const unsigned e = base + u * kThreads;
				if (e < total) v[u] = s4[e];
			}
#pragma unroll
			for (int u = 0; u < kUnroll; ++u) {
				const unsigned e = base + u * kThreads;
				if (e < total) {
					const unsigned r = fdiv(e, per_row);
					const int j = (int)(e - r * per_row.d) * 4;
#pragma unroll
					for (int c = 0; c < 4; ++c) sm[r * ld + j + c] = f(v[u][c], r0 + r, j + c);
				}
			}
		}
	} else {
		const unsigned total = (unsigned)(nr * tk);
		const float* s1 = src + r0 * tk;
		for (unsigned base = tid; base < total; base += kThreads * kUnroll) {
			float v[kUnroll];
#pragma unroll
			for (int u = 0; u < kUnroll; ++u) {
				const unsigned e = base + u * kThreads;
				if (e < total) v[u] = s1[e];
			}
#pragma unroll
			for (int u = 0; u < kUnroll; ++u) {
				const unsigned e = base + u * kThreads;
				if (e < total) {
					const unsigned r = fdiv(e, per_row);
					const int j = (int)(e - r * per_row.d);
					sm[r * ld + j] = f(v[u], r0 + r, j);
				}
			}
		}
	}
}

// std::max scan of the reference (m = o_0, then m = (m < o_j) ? o_j : m) over a row: the scan returns NaN when
// o_0 is NaN (no comparison with NaN is true, so m stays), otherwise the largest non-NaN value (a NaN o_j never
// replaces m). fmaxf ignores NaN operands, so fmaxf over the row in any order gives that largest value; the
// kernel keeps four independent chains per lane. The sign of a zero maximum does not matter (v - m and exp see
// the same value for m = +0 or -0).

// The row softmax, rb rows per block. VEC (tk % 4 == 0, 16-byte aligned rows): LDS rows of stride tk + 4 and
// 16-byte accesses everywhere (the stride puts the 16-byte reads of lanes walking different rows on different
// banks); otherwise stride tk + 1 and 4-byte accesses.
template <bool VEC>
__global__ void __launch_bounds__(kThreads) softmax_rows_kernel(const float* in, float* out, RowGeom g, int rb,
                                                                FastDiv per_row) {
	extern __shared__ float sm[];
	__shared__ unsigned long long table[32];
	__shared__ double rowinv[64];
	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const int64_t r0 = (int64_t)blockIdx.x * rb;
	const int nr = (int)min<int64_t>(rb, g.rows - r0);
	const int ld = VEC ? g.tk + 4 : g.tk + 1;
	float* rowsum = sm + rb * ld;
	float* rowmax = rowsum + rb;
	if (tid < 32) table[tid] = kExp2Table[tid];
	// A: load (every load issued before the first use), scale and mask
	if (VEC) {
		const unsigned total = (unsigned)(nr * (g.tk / 4));
		const f32x4* s4 = reinterpret_cast<const f32x4*>(in + r0 * g.tk);
		for (unsigned base = tid; base < total; base += kThreads * 2 * kUnroll) {
			f32x4 v[2 * kUnroll];
#pragma unroll
			for (int u = 0; u < 2 * kUnroll; ++u) {
				const unsigned e = base + u * kThreads;
				if (e < total) v[u] = s4[e];
			}
#pragma unroll
			for (int u = 0; u < 2 * kUnroll; ++u) {
				const unsigned e = base + u * kThreads;
				if (e < total) {
					const unsigned r = fdiv(e, per_row);
					const int j = (int)(e - r * per_row.d) * 4;
					f32x4 w;
#pragma unroll
					for (int c = 0; c < 4; ++c) w[c] = masked_value(v[u][c], g, r0 + r, j + c);
					*reinterpret_cast<f32x4*>(sm + r * ld + j) = w;
				}
			}
		}
	} else {
		load_rows(in, sm, r0, nr, g.tk, ld, false, per_row,
		          [&](float s, int64_t row, int j) { return masked_value(s, g, row, j); });
	}
	__syncthreads();
	// B: the max of each row, one lane per row (rows spread over the four waves)
	{
		const int r = lane * 4 + wave;
		if (r < nr) {
			const float* o = sm + r * ld;
			float m0 = __builtin_nanf(""), m1 = m0, m2 = m0, m3 = m0;
			int j = 0;
			if (VEC) {
				for (; j + 16 <= g.tk; j += 16) {  // four 16-byte reads in flight
					f32x4 v[4];
#pragma unroll
					for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const f32x4*>(o + j + 4 * u);
#pragma unroll
					for (int u = 0; u < 4; ++u) {
						m0 = fmaxf(m0, v[u][0]);
						m1 = fmaxf(m1, v[u][1]);
						m2 = fmaxf(m2, v[u][2]);
						m3 = fmaxf(m3, v[u][3]);
					}
				}
				for (; j + 4 <= g.tk; j += 4) {
					const f32x4 v = *reinterpret_cast<const f32x4*>(o + j);
					m0 = fmaxf(m0, v[0]);
					m1 = fmaxf(m1, v[1]);
					m2 = fmaxf(m2, v[2]);
					m3 = fmaxf(m3, v[3]);
				}
			}
			for (; j < g.tk; ++j) m0 = fmaxf(m0, o[j]);
			const float m = fmaxf(fmaxf(m0, m1), fmaxf(m2, m3));
			const float first = o[0];
			rowmax[r] = (first != first) ? first : m;  // std::max's scan: see row_max
		}
	}
	__syncthreads();
	// B': the exponentials, a row per wave at a time (exact zeros past the causal limit; those keys take exp(0) in
	// place of exp(-2e9 - m), whose result is discarded, so that waves stay out of exp's special-case path)
	for (int r = wave; r < nr; r += kThreads / 64) {
		float* o = sm + r * ld;
		const float m = rowmax[r];
		const int live = live_keys(g, r0 + r);
		if (VEC) {
			for (int j = 4 * lane; j < g.tk; j += 256) {
				f32x4 v = *reinterpret_cast<const f32x4*>(o + j);
				float e[4];
#pragma unroll
				for (int c = 0; c < 4; ++c) e[c] = j + c < live ? v[c] - m : 0.0f;
				expf_glibc_n(e, table);
#pragma unroll
				for (int c = 0; c < 4; ++c) v[c] = j + c < live ? e[c] : 0.0f;
				*reinterpret_cast<f32x4*>(o + j) = v;
			}
		} else {
			for (int j = lane; j < g.tk; j += 64) {
				const float e = expf_glibc(j < live ? o[j] - m : 0.0f, table);
				o[j] = j < live ? e : 0.0f;
			}
		}
	}
	__syncthreads();
	// C: the sum in j order, one lane per row
	{
		const int r = lane * 4 + wave;
		if (r < nr) {
			const float* o = sm + r * ld;
			const int live = live_keys(g, r0 + r);
			float s = 0.0f;
			int j = 0;
			if (VEC) {
				for (; j + 16 <= live; j += 16) {  // four 16-byte reads in flight, additions in order
					f32x4 v[4];
#pragma unroll
					for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const f32x4*>(o + j + 4 * u);
#pragma unroll
					for (int u = 0; u < 4; ++u) {
						s += v[u][0];
						s += v[u][1];
						s += v[u][2];
						s += v[u][3];
					}
				}
				for (; j + 4 <= live; j += 4) {
					const f32x4 v = *reinterpret_cast<const f32x4*>(o + j);
					s += v[0];
					s += v[1];
					s += v[2];
					s += v[3];
				}
			}
			for (; j < live; ++j) s += o[j];
			rowsum[r] = s;
			rowinv[r] = 1.0 / (double)s;
		}
	}
	__syncthreads();
	// D: normalise and store
	if (VEC) {
		const unsigned total = (unsigned)(nr * (g.tk / 4));
		f32x4* o4 = reinterpret_cast<f32x4*>(out + r0 * g.tk);
		for (unsigned e = tid; e < total; e += kThreads) {
			const unsigned r = fdiv(e, per_row);
			const int j = (int)(e - r * per_row.d) * 4;
			const f32x4 v = *reinterpret_cast<const f32x4*>(sm + r * ld + j);
			const float s = rowsum[r];
			const double ri = rowinv[r];
			float q[4] = {v[0], v[1], v[2], v[3]};
			div_n_by_row_sum(q, s, ri);
			o4[e] = f32x4{q[0], q[1], q[2], q[3]};
		}
	} else {
		const unsigned total = (unsigned)(nr * g.tk);
		for (unsigned e = tid; e < total; e += kThreads) {
			const unsigned r = fdiv(e, per_row);
			const int j = (int)(e - r * per_row.d);
			out[r0 * g.tk + e] = div_by_row_sum(sm[r * ld + j], rowsum[r], rowinv[r]);
		}
	}
}

// Backward of the row softmax (ops.cpp:1216-1224 in attention, 1323-1342 standalone):
//   dot = sum_j g_j * y_j (product rounded, then added, in j order)
//   term_j = scale * (y_j * (g_j - dot))
// mode 0 (attention): out_j = masked ? 0 : term_j + 0.0f
// mode 1 (standalone, fresh gradient): same as mode 0
// mode 2 (standalone, accumulate): out_j += term_j where not masked
template <bool VEC>
__global__ void __launch_bounds__(kThreads) softmax_backward_rows_kernel(const float* y, const float* gin, float* out,
                                                                         RowGeom g, int rb, int mode, FastDiv per_row) {
	extern __shared__ float sm[];
	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const int64_t r0 = (int64_t)blockIdx.x * rb;
	const int nr = (int)min<int64_t>(rb, g.rows - r0);
	const int ld = VEC ? g.tk + 4 : g.tk + 1;
	float* sy = sm;
	float* sg = sm + rb * ld;
	float* dot = sg + rb * ld;
	// A: both rows into LDS, every load issued before the first use
	if (VEC) {
		const unsigned total = (unsigned)(nr * (g.tk / 4));
		const f32x4* y4 = reinterpret_cast<const f32x4*>(y + r0 * g.tk);
		const f32x4* g4 = reinterpret_cast<const f32x4*>(gin + r0 * g.tk);
		for (unsigned base = tid; base < total; base += kThreads * kUnroll) {
			f32x4 vy[kUnroll], vg[kUnroll];
#pragma unroll
			for (int u = 0; u < kUnroll; ++u) {
				const unsigned e = base + u * kThreads;
				if (e < total) {
					vy[u] = y4[e];
					vg[u] = g4[e];
				}
			}
#pragma unroll
			for (int u = 0; u < kUnroll; ++u) {
				const unsigned e = base + u * kThreads;
				if (e < total) {
					const unsigned r = fdiv(e, per_row);
					const int j = (int)(e - r * per_row.d) * 4;
					*reinterpret_cast<f32x4*>(sy + r * ld + j) = vy[u];
					*reinterpret_cast<f32x4*>(sg + r * ld + j) = vg[u];
				}
			}
		}
	} else {
		load_rows(y, sy, r0, nr, g.tk, ld, false, per_row, [](float v, int64_t, int) { return v; });
		load_rows(gin, sg, r0, nr, g.tk, ld, false, per_row, [](float v, int64_t, int) { return v; });
	}
	__syncthreads();
	// the dot product in j order (product rounded, then added), one lane per row
	{
		const int r = lane * 4 + wave;
		if (r < nr) {
			const float* a = sy + r * ld;
			const float* b = sg + r * ld;
			float d = 0.0f;
			int j = 0;
			if (VEC) {
				for (; j + 16 <= g.tk; j += 16) {  // eight 16-byte reads in flight, additions in order
					f32x4 va[4], vb[4];
#pragma unroll
					for (int u = 0; u < 4; ++u) {
						va[u] = *reinterpret_cast<const f32x4*>(a + j + 4 * u);
						vb[u] = *reinterpret_cast<const f32x4*>(b + j + 4 * u);
					}
#pragma unroll
					for (int u = 0; u < 4; ++u)
#pragma unroll
						for (int c = 0; c < 4; ++c) {
							const float t = vb[u][c] * va[u][c];
							d = d + t;
						}
				}
				for (; j + 4 <= g.tk; j += 4) {
					const f32x4 va = *reinterpret_cast<const f32x4*>(a + j);
					const f32x4 vb = *reinterpret_cast<const f32x4*>(b + j);
#pragma unroll
					for (int c = 0; c < 4; ++c) {
						const float t = vb[c] * va[c];
						d = d + t;
					}
				}
			}
			for (; j < g.tk; ++j) {
				const float t = b[j] * a[j];
				d = d + t;
			}
			dot[r] = d;
		}
	}
	__syncthreads();
	// the terms, a row per wave at a time
	for (int r = wave; r < nr; r += kThreads / 64) {
		const int64_t row = r0 + r;
		const float* ph = g.pad ? pad_row(g, row) : nullptr;
		const int i = g.causal ? query_index(g, row) : 0;
		const float dr = dot[r];
		float* o = out + row * g.tk;
		auto term = [&](int j, float yv, float gv, float old) {
			const bool masked = (ph && ph[j] == 0.0f) || (g.causal && j > i);
			const float t = g.scale * (yv * (gv - dr));
			if (mode == 2) return masked ? old : old + t;
			return masked ? 0.0f : t + 0.0f;
		};
		if (VEC) {
			for (int j = 4 * lane; j < g.tk; j += 256) {
				const f32x4 vy = *reinterpret_cast<const f32x4*>(sy + r * ld + j);
				const f32x4 vg = *reinterpret_cast<const f32x4*>(sg + r * ld + j);
				f32x4 old = {0.0f, 0.0f, 0.0f, 0.0f};
				if (mode == 2) old = *reinterpret_cast<const f32x4*>(o + j);
				f32x4 res;
#pragma unroll
				for (int c = 0; c < 4; ++c) res[c] = term(j + c, vy[c], vg[c], old[c]);
				*reinterpret_cast<f32x4*>(o + j) = res;
			}
		} else {
			for (int j = lane; j < g.tk; j += 64)
				o[j] = term(j, sy[r * ld + j], sg[r * ld + j], mode == 2 ? o[j] : 0.0f);
		}
	}
}

constexpr int kMaxLdsBytes = 160 * 1024;

int rows_per_block(int tk, int arrays) {
	// arrays row buffers of (tk + 4) floats plus 2 per-row scalars, within the CU's LDS (less the exp table)
	const int per_row = (arrays * (tk + 4) + 2) * 4;
	int rb = 64;
	while (rb > 1 && rb * per_row > kMaxLdsBytes / 2) rb /= 2;  // leave room for two blocks per CU
	if (rb * per_row > kMaxLdsBytes - 1024) return 0;
	return rb;
}

hipError_t set_lds_limit(const void* fn, int bytes) {
	return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

RowGeom row_geom(int64_t rows, int tk, int tq, int heads, float scale, const float* pad, int causal) {
	const unsigned q = tq > 0 ? (unsigned)tq : 1u, hq = q * (heads > 0 ? (unsigned)heads : 1u);
	return RowGeom{rows, tk, tq, heads, scale, pad, causal, make_fastdiv(q), make_fastdiv(hq)};
}

bool vec_ok(int tk, const void* a, const void* b) {
	return tk % 4 == 0 && reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0;
}

}  // namespace

hipError_t softmax_rows(const float* in, float* out, int64_t rows, int tk, int tq, int heads, float scale,
                        const float* pad, int causal, hipStream_t s) {
	if (rows == 0 || tk == 0) return hipSuccess;
	int rb = min(32, rows_per_block(tk, 1));  // 32 rows (33 KB at tk = 256): four blocks share a CU
	if (rb == 0) return hipErrorInvalidValue;
	// fewer rows a block while that leaves CUs idle (2048 rows of 64 keys: 8.9 -> us with 4 rows a block)
	while (rb > 4 && (rows + rb - 1) / rb < 512) rb /= 2;
	if (rows >= ((int64_t)1 << 31) || (int64_t)rb * tk >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
	const RowGeom g = row_geom(rows, tk, tq, heads, scale, pad, causal);
	const bool vec = vec_ok(tk, in, out);
	const int lds = (rb * (tk + (vec ? 4 : 1)) + 2 * rb) * 4;
	const void* fn = vec ? reinterpret_cast<const void*>(softmax_rows_kernel<true>)
	                     : reinterpret_cast<const void*>(softmax_rows_kernel<false>);
	hipError_t e = set_lds_limit(fn, lds);
	if (e != hipSuccess) return e;
	const dim3 grid((unsigned)((rows + rb - 1) / rb));
	if (vec)
		hipLaunchKernelGGL(softmax_rows_kernel<true>, grid, dim3(kThreads), lds, s, in, out, g, rb,
		                   make_fastdiv((unsigned)(tk / 4)));
	else
		hipLaunchKernelGGL(softmax_rows_kernel<false>, grid, dim3(kThreads), lds, s, in, out, g, rb,
		                   make_fastdiv((unsigned)tk));
	return hipGetLastError();
}

hipError_t softmax_backward_rows(const float* y, const float* g_in, float* out, int64_t rows, int tk, int tq,
                                 int heads, float scale, const float* pad, int causal, int mode, hipStream_t s) {
	if (rows == 0 || tk == 0) return hipSuccess;
	int rb = min(16, rows_per_block(tk, 2));  // 16 rows (33 KB at tk = 256): four blocks share a CU
	if (rb == 0) return hipErrorInvalidValue;
	while (rb > 4 && (rows + rb - 1) / rb < 512) rb /= 2;  // fewer rows a block while that leaves CUs idle
	if (rows >= ((int64_t)1 << 31) || (int64_t)rb * tk >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
	const RowGeom g = row_geom(rows, tk, tq, heads, scale, pad, causal);
	const bool vec = vec_ok(tk, y, g_in) && reinterpret_cast<uintptr_t>(out) % 16 == 0;
	const int lds = (2 * rb * (tk + (vec ? 4 : 1)) + rb) * 4;
	const void* fn = vec ? reinterpret_cast<const void*>(softmax_backward_rows_kernel<true>)
	                     : reinterpret_cast<const void*>(softmax_backward_rows_kernel<false>);
	hipError_t e = set_lds_limit(fn, lds);
	if (e != hipSuccess) return e;
	const dim3 grid((unsigned)((rows + rb - 1) / rb));
	if (vec)
		hipLaunchKernelGGL(softmax_backward_rows_kernel<true>, grid, dim3(kThreads), lds, s, y, g_in, out, g, rb, mode,
		                   make_fastdiv((unsigned)(tk / 4)));
	else
		hipLaunchKernelGGL(softmax_backward_rows_kernel<false>, grid, dim3(kThreads), lds, s, y, g_in, out, g, rb, mode,
		                   make_fastdiv((unsigned)tk));
	return hipGetLastError();
}

int softmax_max_row_length() {
	int tk = 1;
	while (rows_per_block(tk * 2, 2) > 0) tk *= 2;
	int lo = tk, hi = tk * 2;
	while (hi - lo > 1) {
		const int mid = (lo + hi) / 2;
		if (rows_per_block(mid, 2) > 0) lo = mid;
		else hi = mid;
	}
	return lo;
}

}  // namespace nnh
