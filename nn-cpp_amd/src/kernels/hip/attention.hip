// attention.hip - nn::attention's forward (src/autograd/ops.cpp:1226-1261) as one kernel for head width 64.
//
// A workgroup owns 64 query rows of one (sample, head) pair and runs the reference's three steps for them
// with the score rows resident in LDS:
//   1. S = Q_h K_h^T: each element the fma chain over d = 0..63 from +0 (sgemm F,T, ops.cpp:1256). Wave w
//      takes keys 64w..64w+63 against the 64 queries as two 32x32x1 MFMA chains computing S^T (the product
//      fma(k, q, acc) is the reference's fma(q, k, acc)); lane l holds key row 64w + l in registers (the
//      MFMA's A operand), the queries come from LDS.
//   2. masked_softmax_row (ops.cpp:1183-1204) over the 64 rows: scale and mask, std::max's scan, glibc's
//      expf, the sum over live keys in key order, the division; the probabilities go to `probs` (kept for the
//      backward pass) and stay in LDS.
//   3. O_h = P V_h: each element the fma chain over the keys j = 0..Tk-1 from +0 (sgemm F,F, ops.cpp:1259),
//      every key included (a zero probability still meets its V entry). Wave w takes output columns
//      16w..16w+15 as one 16x16x1 MFMA chain over the 64 rows; P comes from LDS, V from global memory a
//      chunk of keys ahead.
// Same bits as the three-launch path (batched GEMM, row softmax, batched GEMM): both sgemm shapes are below
// nn-cpp's depth cut (k = 64 and k = Tk <= 256), so every element is a single chain.
// Two workgroups share a CU (about 67 KB of LDS each at Tk = 256), so one's MFMA phases can overlap the other's
// VALU phases.
#include "attention.hpp"
#include "gemm.hpp"

#include "gemm_tile.hpp"
#include "softmax_row.hpp"

namespace nnh {

namespace {

constexpr int kRows = 64;          // query rows per workgroup
constexpr int kDh = 64;            // head width
constexpr int kKLd = kDh + 4;      // LDS row stride of the queries (16-byte reads of 16 lanes hit distinct banks)
constexpr int kMaxKeys = 256;     // four waves of 64 keys
constexpr int kVChunk = 16;        // keys of V each lane keeps in flight

struct FusedArgs {
	const float* q;
	const float* k;
	const float* v;
	float* out;
	float* probs;
	const float* pad;  // {N, Tk}, 0 marks a padded key; or null
	int heads, tq, tk, d;
	int qblocks, total;
	int causal;
	float scale;
	FastDiv quads;     // division by tk / 4
};

inline int lds_floats_p(int tk) { return kRows * (tk + 4); }

using M32 = Mfma<kMf32>;
using M16 = Mfma<kMf16>;

// Phases 0 and 1, shared by the forward and the backward: (R K^T)^T for the 64 rows of R (row stride d, nr of
// them valid) against the keys of K (row stride d, tk valid). Wave w takes keys 64w + l (lane l holds key row
// 64w + l in registers: the MFMA's A operand) against rows 32u + (l & 31), u = 0, 1 (staged in LDS with
// coalesced loads, read as the B operand), each element the fma chain over d = 0..63 from +0. Ends with a
// barrier after which the LDS is free.
__device__ __forceinline__ void rows_times_keys(const float* rp, int nr, const float* kp, int tk, int d, float* sm,
                                                M32::Acc& s0, M32::Acc& s1) {
	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const bool keys_here = 64 * wave < tk;
	// loads are unconditional (indices clamped into range) so that all are in flight before the first wait;
	// values past the end are never used
	f32x4 kv[kDh / 4];
	if (keys_here) {
		const float* kr = kp + (int64_t)min(64 * wave + lane, tk - 1) * d;
#pragma unroll
		for (int u = 0; u < kDh / 4; ++u) kv[u] = *reinterpret_cast<const f32x4*>(kr + 4 * u);
	}
	{
		f32x4 rs[kRows * kDh / 4 / 256];
#pragma unroll
		for (int u = 0; u < kRows * kDh / 4 / 256; ++u) {
			const int row = (tid >> 4) + 16 * u;
			rs[u] = *reinterpret_cast<const f32x4*>(rp + (int64_t)min(row, nr - 1) * d + 4 * (tid & 15));
		}
#pragma unroll
		for (int u = 0; u < kRows * kDh / 4 / 256; ++u)
			*reinterpret_cast<f32x4*>(sm + ((tid >> 4) + 16 * u) * kKLd + 4 * (tid & 15)) = rs[u];
	}
	__syncthreads();
#pragma unroll
	for (int r = 0; r < M32::NV; ++r) s0[r] = s1[r] = 0.0f;
	if (keys_here) {
		const float* rb0 = sm + (lane & 31) * kKLd;
		const float* rb1 = rb0 + 32 * kKLd;
#pragma unroll
		for (int d4 = 0; d4 < kDh / 4; ++d4) {
			const f32x4 b0 = *reinterpret_cast<const f32x4*>(rb0 + 4 * d4);
			const f32x4 b1 = *reinterpret_cast<const f32x4*>(rb1 + 4 * d4);
#pragma unroll
			for (int c = 0; c < 4; ++c) {
				s0 = M32::mma(kv[d4][c], b0[c], s0);
				s1 = M32::mma(kv[d4][c], b1[c], s1);
			}
		}
	}
	__syncthreads();  // the staged rows are dead
}

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) attention_fused_kernel(const FusedArgs a) {
	extern __shared__ __align__(16) float sm[];
	__shared__ unsigned long long table[32];
	__shared__ float rowmax[kRows], rowsum[kRows];
	__shared__ double rowinv[kRows];
	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const int lid = xcd_remap(blockIdx.x, a.total);  // the query blocks of one head share an XCD's L2
	const int nh = lid / a.qblocks, qb = lid - nh * a.qblocks;
	const int n = nh / a.heads, h = nh - n * a.heads;
	const int i0 = qb * kRows, nq = min(kRows, a.tq - i0);
	const int tk = a.tk, ldp = tk + 4;
	const float* qp = a.q + ((int64_t)n * a.tq + i0) * a.d + h * kDh;
	const float* kp = a.k + (int64_t)n * tk * a.d + h * kDh;
	const float* vp = a.v + (int64_t)n * tk * a.d + h * kDh;
	const float* padrow = a.pad ? a.pad + (int64_t)n * tk : nullptr;
	if (tid < 32) table[tid] = kExp2Table[tid];
	const bool pv4 = tk % 16 == 0;  // O = P V on the 16x16x4 MFMA (P kept in LDS in its permuted layout)

	// 0, 1. S^T for keys 64w + l against queries 32u + (l & 31), u = 0, 1 (fma(k, q, acc) is the reference's
	// fma(q, k, acc))
	const bool keys_here = 64 * wave < tk;
	M32::Acc s0, s1;
	rows_times_keys(qp, nq, kp, tk, a.d, sm, s0, s1);

	// 2a. scaled and masked scores into LDS rows of stride tk + 4 (ops.cpp:1186-1191). Accumulator registers
	// 4t .. 4t+3 hold four consecutive keys of one query: one 16-byte store each.
	f32x4* sm4 = reinterpret_cast<f32x4*>(sm);
	const int ldp4 = ldp / 4;
	if (keys_here) {
		const bool masked = padrow != nullptr || a.causal;
#pragma unroll
		for (int t = 0; t < M32::NV / 4; ++t) {
			const int j = 64 * wave + M32::crow(4 * t, lane);
#pragma unroll
			for (int u = 0; u < 2; ++u) {
				const int row = 32 * u + M32::ccol(lane);
				f32x4 val;
#pragma unroll
				for (int c = 0; c < 4; ++c) val[c] = (u ? s1[4 * t + c] : s0[4 * t + c]) * a.scale;
				if (masked) {  // uniform
					const f32x4 pd = padrow ? *reinterpret_cast<const f32x4*>(padrow + min(j, tk - 4)) : f32x4{1, 1, 1, 1};
#pragma unroll
					for (int c = 0; c < 4; ++c) {
						val[c] = pd[c] == 0.0f ? -1e9f : val[c];
						val[c] = a.causal && j + c > i0 + row ? -2e9f : val[c];
					}
				}
				if (row < nq && j < tk) sm4[row * ldp4 + j / 4] = val;  // tk % 4 == 0: the quad is whole
			}
		}
	}
	__syncthreads();

	// 2b. the row maxima: std::max's scan is v_0 when v_0 is NaN, else the largest non-NaN value, which fmaxf
	// gives in any order (a zero maximum's sign cannot change v - m or its exp). Four lanes per row.
	{
		const int row = 16 * wave + (lane >> 2), q = lane & 3;
		float m = __builtin_nanf("");
		if (row < nq) {
			const float* o = sm + row * ldp;
			for (int j = 4 * q; j < tk; j += 16) {
				const f32x4 x = *reinterpret_cast<const f32x4*>(o + j);
				m = fmaxf(m, fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
			}
		}
		m = fmaxf(m, __shfl_xor(m, 1));
		m = fmaxf(m, __shfl_xor(m, 2));
		if (row < nq && q == 0) {
			const float first = sm[row * ldp];
			rowmax[row] = first != first ? first : m;
		}
	}
	__syncthreads();

	// 2c. p_j = exp(v_j - m) for the live keys, exact zeros past the causal limit (ops.cpp:1197-1201). Lane l takes
	// row l, wave w the quads of keys w, w + 4, ..., kExpQuads of them at a time so that their table reads and
	// double-precision chains overlap. Keys past a row's causal limit take exp(0) in place of exp(-2e9 - m), whose
	// result is replaced by an exact zero, which keeps waves out of exp's special-case path (padded keys stay live
	// and go through exp). Quads past the block's last live key are zero for every row: a wave stores them without
	// computing anything.
	{
		constexpr int kExpQuads = 4;
		const int row = lane, nq4 = tk / 4;
		const float m = rowmax[min(row, nq - 1)];
		const int live = a.causal ? min(tk, i0 + row + 1) : tk;
		const int block_live = a.causal ? min(tk, i0 + nq) : tk;  // keys any row of the block reaches
		f32x4* orow = sm4 + row * ldp4;
		for (int q0 = wave; q0 < nq4; q0 += 4 * kExpQuads) {
			if (4 * q0 >= block_live) {  // uniform: this and every later quad of the wave is dead for all rows
				if (row < nq) {
#pragma unroll
					for (int h2 = 0; h2 < kExpQuads; ++h2)
						if (q0 + 4 * h2 < nq4) orow[q0 + 4 * h2] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
				}
				continue;
			}
			f32x4 x[kExpQuads];
#pragma unroll
			for (int h2 = 0; h2 < kExpQuads; ++h2) x[h2] = orow[min(q0 + 4 * h2, nq4 - 1)];
			float ex[4 * kExpQuads];
#pragma unroll
			for (int h2 = 0; h2 < kExpQuads; ++h2)
#pragma unroll
				for (int c = 0; c < 4; ++c) ex[4 * h2 + c] = 4 * (q0 + 4 * h2) + c < live ? x[h2][c] - m : 0.0f;
			expf_glibc_n(ex, table);
			if (row < nq) {
#pragma unroll
				for (int h2 = 0; h2 < kExpQuads; ++h2) {
					const int q = q0 + 4 * h2;
#pragma unroll
					for (int c = 0; c < 4; ++c) x[h2][c] = 4 * q + c < live ? ex[4 * h2 + c] : 0.0f;
					if (q < nq4) orow[q] = x[h2];
				}
			}
		}
	}
	__syncthreads();

	// 2d. the sum over the live keys in key order from +0, one lane per row (ops.cpp:1198-1200)
	{
		const int row = 16 * wave + lane;
		if (lane < 16 && row < nq) {
			const float* o = sm + row * ldp;
			const int live = a.causal ? min(tk, i0 + row + 1) : tk;
			float s = 0.0f;
			int j = 0;
			for (; j + 16 <= live; j += 16) {
				f32x4 x[4];
#pragma unroll
				for (int u = 0; u < 4; ++u) x[u] = *reinterpret_cast<const f32x4*>(o + j + 4 * u);
#pragma unroll
				for (int u = 0; u < 4; ++u) {
					s += x[u][0];
					s += x[u][1];
					s += x[u][2];
					s += x[u][3];
				}
			}
			for (; j < live; ++j) s += o[j];
			rowsum[row] = s;
			rowinv[row] = 1.0 / (double)s;
		}
	}
	__syncthreads();

	// 2e. p_j / sum into probs and back into LDS (ops.cpp:1203)
	{
		float* pr = a.probs + ((int64_t)nh * a.tq + i0) * tk;
		const unsigned quads = (unsigned)(nq * (tk / 4));
		if (pv4) {
			// the 16x16x4 product below reads each row permuted, key j at j % 4 (Tk / 4) + j / 4: every quad is read
			// and divided first, then, after a barrier, written back in that order (at most kRows Tk / 1024 quads a
			// thread)
			constexpr int kPer = kRows * kMaxKeys / 4 / 256;
			f32x4 yv[kPer];
#pragma unroll
			for (int u = 0; u < kPer; ++u) {
				const unsigned e = tid + 256 * u;
				if (e < quads) {
					const unsigned row = fdiv(e, a.quads);
					const int j = (int)(e - row * a.quads.d) * 4;
					const f32x4 x = *reinterpret_cast<const f32x4*>(sm + row * ldp + j);
					float y[4] = {x[0], x[1], x[2], x[3]};
					div_n_by_row_sum(y, rowsum[row], rowinv[row]);
					yv[u] = f32x4{y[0], y[1], y[2], y[3]};
					*reinterpret_cast<f32x4*>(pr + (int64_t)row * tk + j) = yv[u];
				}
			}
			__syncthreads();
#pragma unroll
			for (int u = 0; u < kPer; ++u) {
				const unsigned e = tid + 256 * u;
				if (e < quads) {
					const unsigned row = fdiv(e, a.quads);
					const int jq = (int)(e - row * a.quads.d);
#pragma unroll
					for (int c = 0; c < 4; ++c) sm[row * ldp + c * (tk >> 2) + jq] = yv[u][c];
				}
			}
		} else {
			for (unsigned e = tid; e < quads; e += 256) {
				const unsigned row = fdiv(e, a.quads);
				const int j = (int)(e - row * a.quads.d) * 4;
				float* o = sm + row * ldp + j;
				const f32x4 x = *reinterpret_cast<const f32x4*>(o);
				float y[4] = {x[0], x[1], x[2], x[3]};
				div_n_by_row_sum(y, rowsum[row], rowinv[row]);
				const f32x4 y4 = {y[0], y[1], y[2], y[3]};
				*reinterpret_cast<f32x4*>(o) = y4;
				*reinterpret_cast<f32x4*>(pr + (int64_t)row * tk + j) = y4;
			}
		}
	}
	__syncthreads();

	if (pv4) {
		// 3. O columns 16w .. 16w+15 for the 64 rows on the 16x16x4 MFMA (Mfma<kMf16x4>: four keys per instruction,
		// bit for bit four fmas in key order): four 16-row tiles, four independent chains over every key. At step s
		// lane (g, i) supplies P[16 t + i][4 s + g], read four steps at a time from the permuted rows (positions
		// g Tk / 4 + s), and V[4 s + g][16 w + i], loaded 16 steps ahead.
		using M4 = Mfma<kMf16x4>;
		const int g = lane >> 4, il = lane & 15, q4 = tk >> 2;
		M4::Acc acc4[4];
#pragma unroll
		for (int t = 0; t < 4; ++t) acc4[t] = M4::Acc{0.0f, 0.0f, 0.0f, 0.0f};
		const float* vcol = vp + 16 * wave + il;
		const float* pbase = sm + il * ldp + g * q4;
		auto load_v = [&](float (&dst)[16], int s0) {  // steps s0 .. s0 + 15 (clamped rows are loaded, never used)
#pragma unroll
			for (int u = 0; u < 16; ++u) dst[u] = vcol[(int64_t)min(4 * (s0 + u) + g, tk - 1) * a.d];
		};
		auto load_p = [&](f32x4 (&dst)[4], int s0) {  // steps s0 .. s0 + 3 of the four tiles
#pragma unroll
			for (int t = 0; t < 4; ++t) dst[t] = *reinterpret_cast<const f32x4*>(pbase + 16 * t * ldp + min(s0, q4 - 4));
		};
		float v0[16], v1[16];
		f32x4 pa[4], pb[4];
		auto chunk = [&](const float (&v)[16], int s0) {  // 16 steps from s0, P one group of four steps ahead
			load_p(pa, s0);
#pragma unroll
			for (int h4 = 0; h4 < 4; ++h4) {
				f32x4 (&cur)[4] = (h4 & 1) ? pb : pa;
				f32x4 (&nxt)[4] = (h4 & 1) ? pa : pb;
				if (h4 < 3) load_p(nxt, s0 + 4 * (h4 + 1));
#pragma unroll
				for (int e = 0; e < 4; ++e)
#pragma unroll
					for (int t = 0; t < 4; ++t) acc4[t] = M4::mma(cur[t][e], v[4 * h4 + e], acc4[t]);
			}
		};
		// tk % 16 == 0: q4 is a multiple of 4, whole groups of four steps; chunks of 16 steps, V two chunks ahead
		load_v(v0, 0);
		load_v(v1, 16);
		int s0 = 0;
		for (; s0 + 32 <= q4; s0 += 32) {
			chunk(v0, s0);
			load_v(v0, s0 + 32);
			chunk(v1, s0 + 16);
			load_v(v1, s0 + 48);
		}
		// the rest: fewer than 32 steps, in groups of four
		for (; s0 < q4; s0 += 4) {
			float vv[16];
			f32x4 pp[4];
			load_p(pp, s0);
#pragma unroll
			for (int e = 0; e < 4; ++e) vv[e] = vcol[(int64_t)(4 * (s0 + e) + g) * a.d];
#pragma unroll
			for (int e = 0; e < 4; ++e)
#pragma unroll
				for (int t = 0; t < 4; ++t) acc4[t] = M4::mma(pp[t][e], vv[e], acc4[t]);
		}
		float* op = a.out + ((int64_t)n * a.tq + i0) * a.d + h * kDh + 16 * wave + il;
#pragma unroll
		for (int t = 0; t < 4; ++t)
#pragma unroll
			for (int r = 0; r < 4; ++r) {
				const int row = 16 * t + 4 * g + r;
				if (row < nq) op[(int64_t)row * a.d] = acc4[t][r];
			}
		return;
	}

	// 3. O columns 16w .. 16w+15 for the 64 rows: the chain over every key in order
	M16::Acc o;
#pragma unroll
	for (int r = 0; r < M16::NV; ++r) o[r] = 0.0f;
	{
		const f32x4* prow4 = sm4 + M16::arow(lane) * ldp4;  // rows past nq hold stale values, never stored
		const int vlane = 16 * wave + M16::bcol(lane);
		// V entries of keys j0 .. j0+kVChunk-1 for this lane's column; rows past tk are clamped to the last key
		// (loaded, never used), so every load is issued unconditionally with a uniform row address.
		auto load_v = [&](float (&dst)[kVChunk], int j0) {
#pragma unroll
			for (int u = 0; u < kVChunk; ++u) dst[u] = (vp + (int64_t)min(j0 + u, tk - 1) * a.d)[vlane];
		};
		// P quads of keys j0 .. j0+kVChunk-1 (quads past tk, in a partial chunk, read a stale in-row value)
		auto load_p = [&](f32x4 (&dst)[kVChunk / 4], int j0) {
#pragma unroll
			for (int u4 = 0; u4 < kVChunk / 4; ++u4) dst[u4] = prow4[min(j0 + 4 * u4, tk - 4) / 4];
		};
		auto steps = [&](const f32x4 (&p)[kVChunk / 4], const float (&src)[kVChunk], int j0, bool whole) {
#pragma unroll
			for (int u4 = 0; u4 < kVChunk / 4; ++u4) {
				if (whole || j0 + 4 * u4 < tk) {  // tk % 4 == 0: whole quads only, no step past the last key
#pragma unroll
					for (int c = 0; c < 4; ++c) o = M16::mma(p[u4][c], src[4 * u4 + c], o);
				}
			}
		};
		float v0[kVChunk], v1[kVChunk];
		f32x4 p0[kVChunk / 4], p1[kVChunk / 4];
		load_v(v0, 0);
		load_v(v1, kVChunk);
		load_p(p0, 0);
		int j0 = 0;
		for (; j0 + 2 * kVChunk <= tk; j0 += 2 * kVChunk) {  // V two chunks ahead, P one chunk ahead
			load_p(p1, j0 + kVChunk);
			steps(p0, v0, j0, true);
			load_v(v0, j0 + 2 * kVChunk);
			load_p(p0, j0 + 2 * kVChunk);
			steps(p1, v1, j0 + kVChunk, true);
			load_v(v1, j0 + 3 * kVChunk);
		}
		if (j0 < tk) {
			load_p(p1, j0 + kVChunk);
			steps(p0, v0, j0, false);
			if (j0 + kVChunk < tk) steps(p1, v1, j0 + kVChunk, false);
		}
	}
	float* op = a.out + ((int64_t)n * a.tq + i0) * a.d + h * kDh + 16 * wave + M16::ccol(lane);
#pragma unroll
	for (int r = 0; r < M16::NV; ++r) {
		const int row = M16::crow(r, lane);
		if (row < nq) op[(int64_t)row * a.d] = o[r];
	}
}


struct DScoresArgs {
	const float* g;      // upstream gradient {N, Tq, D}
	const float* v;
	const float* probs;  // the forward's {N, heads, Tq, Tk}
	float* ds;           // {N, heads, Tq, Tk}
	const float* pad;
	int heads, tq, tk, d;
	int qblocks, total;
	int causal;
	float scale;
};

// The first half of nn::attention's backward for 64 query rows of one (sample, head) pair (ops.cpp:1286-1290):
//   dP = G_h V_h^T                     each element the fma chain over d = 0..63 from +0 (sgemm F,T)
//   dot_i = sum_j dP_ij * y_ij         the products rounded, then added in key order from +0
//   dS_ij = masked ? 0 : scale * (y_ij * (dP_ij - dot_i)) + 0     (masked_softmax_row_backward, ops.cpp:1216-1224)
// dP stays in the MFMA accumulators (wave w holds keys 64w..64w+63 of the 64 rows, four consecutive keys per
// four registers); y is loaded in the same layout; only the products dP y go through LDS, where one lane per
// row adds them in key order. dS is written to HBM for the dQ and dK products.
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) attention_dscores_kernel(const DScoresArgs a) {
	extern __shared__ __align__(16) float sm[];
	__shared__ float rowdot[kRows];
	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const int lid = xcd_remap(blockIdx.x, a.total);
	const int nh = lid / a.qblocks, qb = lid - nh * a.qblocks;
	const int n = nh / a.heads, h = nh - n * a.heads;
	const int i0 = qb * kRows, nq = min(kRows, a.tq - i0);
	const int tk = a.tk, ldp4 = (tk + 4) / 4;
	const float* gp = a.g + ((int64_t)n * a.tq + i0) * a.d + h * kDh;
	const float* vp = a.v + (int64_t)n * tk * a.d + h * kDh;
	const float* yp = a.probs + ((int64_t)nh * a.tq + i0) * tk;
	float* dsp = a.ds + ((int64_t)nh * a.tq + i0) * tk;
	const float* padrow = a.pad ? a.pad + (int64_t)n * tk : nullptr;
	f32x4* sm4 = reinterpret_cast<f32x4*>(sm);

	// dP^T for keys 64w + l against rows 32u + (l & 31)
	const bool keys_here = 64 * wave < tk;
	M32::Acc s0, s1;
	rows_times_keys(gp, nq, vp, tk, a.d, sm, s0, s1);

	// y in the accumulator layout: quad t of unit u is y[32u + ccol][64w + crow(4t) .. +3] (rows and keys clamped
	// into range; values outside are never used)
	constexpr int kQ = M32::NV / 4;
	f32x4 y[2][kQ];
	if (keys_here) {
#pragma unroll
		for (int u = 0; u < 2; ++u) {
			const int row = min(32 * u + M32::ccol(lane), nq - 1);
#pragma unroll
			for (int t = 0; t < kQ; ++t) {
				const int j = min(64 * wave + M32::crow(4 * t, lane), tk - 4);
				y[u][t] = *reinterpret_cast<const f32x4*>(yp + (int64_t)row * tk + j);
			}
		}
		// the products dP y, rounded, into LDS rows of stride tk + 4 (tk % 4 == 0: every quad is whole)
#pragma unroll
		for (int u = 0; u < 2; ++u) {
			const int row = 32 * u + M32::ccol(lane);
#pragma unroll
			for (int t = 0; t < kQ; ++t) {
				const int j = 64 * wave + M32::crow(4 * t, lane);
				f32x4 prod;
#pragma unroll
				for (int c = 0; c < 4; ++c) prod[c] = (u ? s1[4 * t + c] : s0[4 * t + c]) * y[u][t][c];
				if (row < nq && j < tk) sm4[row * ldp4 + j / 4] = prod;
			}
		}
	}
	__syncthreads();

	// dot_i: one lane per row, every key in order from +0
	{
		const int row = 16 * wave + lane;
		if (lane < 16 && row < nq) {
			const f32x4* o = sm4 + row * ldp4;
			float dot = 0.0f;
			int q = 0;
			for (; q + 4 <= tk / 4; q += 4) {
				f32x4 x[4];
#pragma unroll
				for (int u = 0; u < 4; ++u) x[u] = o[q + u];
#pragma unroll
				for (int u = 0; u < 4; ++u) {
					dot += x[u][0];
					dot += x[u][1];
					dot += x[u][2];
					dot += x[u][3];
				}
			}
			for (; q < tk / 4; ++q) {
				const f32x4 x = o[q];
				dot += x[0];
				dot += x[1];
				dot += x[2];
				dot += x[3];
			}
			rowdot[row] = dot;
		}
	}
	__syncthreads();

	// dS from the registers
	if (keys_here) {
		const bool masked = padrow != nullptr || a.causal;
#pragma unroll
		for (int u = 0; u < 2; ++u) {
			const int row = 32 * u + M32::ccol(lane);
			const float dot = rowdot[min(row, nq - 1)];
#pragma unroll
			for (int t = 0; t < kQ; ++t) {
				const int j = 64 * wave + M32::crow(4 * t, lane);
				f32x4 r;
#pragma unroll
				for (int c = 0; c < 4; ++c) {
					const float dp = u ? s1[4 * t + c] : s0[4 * t + c];
					r[c] = a.scale * (y[u][t][c] * (dp - dot)) + 0.0f;
				}
				if (masked) {  // uniform
					const f32x4 pd = padrow ? *reinterpret_cast<const f32x4*>(padrow + min(j, tk - 4)) : f32x4{1, 1, 1, 1};
#pragma unroll
					for (int c = 0; c < 4; ++c)
						r[c] = pd[c] == 0.0f || (a.causal && j + c > i0 + row) ? 0.0f : r[c];
				}
				if (row < nq && j < tk) *reinterpret_cast<f32x4*>(dsp + (int64_t)row * tk + j) = r;
			}
		}
	}
}

}  // namespace

bool attention_fused_ok(int64_t tq, int64_t tk, int64_t dh, int64_t d, const void* q, const void* k, const void* v,
                        const void* out, const void* probs, const void* pad) {
	auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
	// the kernel runs S = Q K^T and O = P V as whole-depth chains: products that take the depth cut go elsewhere
	if (depth_cut(tq, tk, dh) || depth_cut(tq, dh, tk)) return false;
	return dh == kDh && tk >= 1 && tk <= kMaxKeys && tk % 4 == 0 && d % 4 == 0 && tq >= 1 && tq < (1 << 24) &&
	       al(q) && al(k) && al(v) && al(out) && al(probs) && (pad == nullptr || al(pad));
}

hipError_t attention_fused_forward(const float* q, const float* k, const float* v, int64_t n, int64_t tq, int64_t tk,
                                   int64_t d, int64_t heads, const float* pad, int causal, float scale, float* out,
                                   float* probs, hipStream_t s) {
	const int64_t qblocks = (tq + kRows - 1) / kRows, total = n * heads * qblocks;
	if (total == 0) return hipSuccess;
	if (total >= ((int64_t)1 << 31) || n * heads * tq * tk >= ((int64_t)1 << 62)) return hipErrorInvalidValue;
	FusedArgs a;
	a.q = q;
	a.k = k;
	a.v = v;
	a.out = out;
	a.probs = probs;
	a.pad = pad;
	a.heads = (int)heads;
	a.tq = (int)tq;
	a.tk = (int)tk;
	a.d = (int)d;
	a.qblocks = (int)qblocks;
	a.total = (int)total;
	a.causal = causal ? 1 : 0;
	a.scale = scale;
	a.quads = make_fastdiv((unsigned)(tk / 4));
	const int lds = 4 * max(kRows * kKLd, lds_floats_p((int)tk));
	hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(attention_fused_kernel),
	                                   hipFuncAttributeMaxDynamicSharedMemorySize, lds);
	if (e != hipSuccess) return e;
	hipLaunchKernelGGL(attention_fused_kernel, dim3((unsigned)total), dim3(256), lds, s, a);
	return hipGetLastError();
}

hipError_t attention_fused_dscores(const float* g, const float* v, const float* probs, int64_t n, int64_t tq, int64_t tk,
                                   int64_t d, int64_t heads, const float* pad, int causal, float scale, float* ds,
                                   hipStream_t s) {
	const int64_t qblocks = (tq + kRows - 1) / kRows, total = n * heads * qblocks;
	if (total == 0) return hipSuccess;
	if (total >= ((int64_t)1 << 31) || n * heads * tq * tk >= ((int64_t)1 << 62)) return hipErrorInvalidValue;
	DScoresArgs a;
	a.g = g;
	a.v = v;
	a.probs = probs;
	a.ds = ds;
	a.pad = pad;
	a.heads = (int)heads;
	a.tq = (int)tq;
	a.tk = (int)tk;
	a.d = (int)d;
	a.qblocks = (int)qblocks;
	a.total = (int)total;
	a.causal = causal ? 1 : 0;
	a.scale = scale;
	const int lds = 4 * max(kRows * kKLd, lds_floats_p((int)tk));
	hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(attention_dscores_kernel),
	                                   hipFuncAttributeMaxDynamicSharedMemorySize, lds);
	if (e != hipSuccess) return e;
	hipLaunchKernelGGL(attention_dscores_kernel, dim3((unsigned)total), dim3(256), lds, s, a);
	return hipGetLastError();
}

}  // namespace nnh
