/*
 * oracle.c - CPU restatement of nn-cpp's GEMM hot path (reference: MiguelMochizuki/nn-cpp v2.0.0).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg. The product library never links or calls it.
 *
 * Compiled with -ffp-contract=off, like the reference (CMakeLists.txt:61-65): every fused
 * multiply-add below is an explicit fmaf(), every other operation rounds on its own.
 *
 * What the reference computes (NN_NATIVE, AVX2/FMA host, src/kernels/gemm.cpp:14-20 selects micro_avx2):
 * each C element is a sequential fused multiply-add chain over the depth starting at +0
 * (gemm.cpp:232-244), cut into depth blocks of kKC = 256 (gemm.hpp:33) whose running sum is stored
 * to C and reloaded unchanged (Store::kContinue, gemm.cpp:225-231, 371). With accumulate the old C
 * is added once, after the first depth block (Store::kAdd, gemm.cpp:245-252). Small-output,
 * long-depth products are cut into 128-deep pieces summed in piece order (gemm.cpp:453-485).
 * No thread count changes any of this (gemm.cpp:404-406).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define KKC 256       /* gemm.hpp:33 kKC */
#define KPIECE 128    /* gemm.cpp:461 kPiece = kKC / 2 */

static inline float op_a(int ta, const float* a, size_t lda, size_t i, size_t p) {
	return ta ? a[p * lda + i] : a[i * lda + p];
}
static inline float op_b(int tb, const float* b, size_t ldb, size_t p, size_t j) {
	return tb ? b[j * ldb + p] : b[p * ldb + j];
}

/* blocked_flat + micro_avx2, element by element (gemm.cpp:342-437, 201-262). */
static void sgemm_flat(int ta, int tb, size_t m, size_t n, size_t k, const float* a, size_t lda,
		const float* b, size_t ldb, float* c, size_t ldc, int accumulate) {
	if (m == 0 || n == 0) return;                                   /* gemm.cpp:344 */
	if (k == 0) {                                                   /* gemm.cpp:345-350 */
		if (!accumulate)
			for (size_t i = 0; i < m; ++i)
				for (size_t j = 0; j < n; ++j) c[i * ldc + j] = 0.0f;
		return;
	}
	for (size_t i = 0; i < m; ++i) {
		for (size_t j = 0; j < n; ++j) {
			float run = 0.0f;
			for (size_t pc = 0; pc < k; pc += KKC) {
				const size_t kc = (k - pc < KKC) ? k - pc : KKC;
				float t = pc > 0 ? run : 0.0f;                  /* kContinue reloads the stored sum */
				for (size_t p = pc; p < pc + kc; ++p) t = fmaf(op_a(ta, a, lda, i, p), op_b(tb, b, ldb, p, j), t);
				if (pc == 0 && accumulate) t = c[i * ldc + j] + t;  /* kAdd: c + acc */
				run = t;
			}
			c[i * ldc + j] = run;
		}
	}
}

/* Numerics mode of the checked library: 0 nn-cpp's own depth cut (below), 1 the split-depth rule, under which
 * every oracle function follows the library's NNH_NUMERICS_SPLIT_DEPTH. */
static int g_split_depth = 0;
void oracle_set_numerics(int mode) { g_split_depth = mode == 1; }

/* Depth of one piece of a cut product, or 0 when the product is not cut (one chain over the whole depth).
 * nn-cpp (gemm.cpp:456-461): m n <= kDepthMaxOut = 2^16, k >= 4 kPiece and m n k >= kDepthMinWork = 2^20 cut
 * into kPiece = 128-deep pieces. Split mode: m n <= 2^18 and k >= 256, with T = ceil(m / 64) ceil(n / 16) and
 * s = min(16, max(2, 4096 / T)), pieces of ceil(k / s) rounded up to a multiple of 32. */
size_t oracle_piece_depth(size_t m, size_t n, size_t k) {
	if (m == 0 || n == 0 || k == 0) return 0;
	if (g_split_depth) {
		if (m * n > ((size_t)1 << 18) || k < 256) return 0;
		const size_t tiles = ((m + 63) / 64) * ((n + 15) / 16);
		size_t s = 4096 / tiles;
		s = s < 2 ? 2 : s > 16 ? 16 : s;
		return ((k + s - 1) / s + 31) / 32 * 32;
	}
	if (m * n > ((size_t)1 << 16) || k < 4 * KPIECE || m * n * k < ((size_t)1 << 20)) return 0;
	return KPIECE;
}

/* Whether the product is cut into more than one piece. */
int oracle_depth_cut(size_t m, size_t n, size_t k) {
	const size_t pk = oracle_piece_depth(m, n, k);
	return pk > 0 && pk < k;
}

/* nn::kernels::sgemm (gemm.cpp:546-556 -> blocked, 453-485). */
void oracle_sgemm(int ta, int tb, size_t m, size_t n, size_t k, const float* a, size_t lda, const float* b,
		size_t ldb, float* c, size_t ldc, int accumulate) {
	if (!oracle_depth_cut(m, n, k)) {
		sgemm_flat(ta, tb, m, n, k, a, lda, b, ldb, c, ldc, accumulate);
		return;
	}
	const size_t pk = oracle_piece_depth(m, n, k), pieces = (k + pk - 1) / pk;
	for (size_t i = 0; i < m; ++i) {
		for (size_t j = 0; j < n; ++j) {
			float acc = 0.0f;
			for (size_t p = 0; p < pieces; ++p) {
				const size_t pc = p * pk, kc = (k - pc < pk) ? k - pc : pk;
				float t = 0.0f;                                 /* each piece: its own overwrite product */
				for (size_t q = pc; q < pc + kc; ++q) t = fmaf(op_a(ta, a, lda, i, q), op_b(tb, b, ldb, q, j), t);
				acc = p == 0 ? t : acc + t;                     /* gemm.cpp:475-480, piece order */
			}
			c[i * ldc + j] = accumulate ? c[i * ldc + j] + acc : acc;  /* gemm.cpp:481-483 */
		}
	}
}

/* oracle_sgemm for selected elements only: out[t] = what sgemm leaves in C(rows[t], cols[t]), with
 * c_old[t] the element's value before an accumulating call. Lets full-size products be checked on a
 * sample of elements. */
void oracle_sgemm_at(int ta, int tb, size_t m, size_t n, size_t k, const float* a, size_t lda, const float* b,
		size_t ldb, int accumulate, const size_t* rows, const size_t* cols, const float* c_old, size_t count,
		float* out) {
	const int cut = oracle_depth_cut(m, n, k);
	for (size_t t = 0; t < count; ++t) {
		const size_t i = rows[t], j = cols[t];
		float v;
		if (k == 0) {
			v = accumulate ? c_old[t] : 0.0f;
		} else if (!cut) {
			float run = 0.0f;
			for (size_t pc = 0; pc < k; pc += KKC) {
				const size_t kc = (k - pc < KKC) ? k - pc : KKC;
				float x = pc > 0 ? run : 0.0f;
				for (size_t p = pc; p < pc + kc; ++p) x = fmaf(op_a(ta, a, lda, i, p), op_b(tb, b, ldb, p, j), x);
				if (pc == 0 && accumulate) x = c_old[t] + x;
				run = x;
			}
			v = run;
		} else {
			float acc = 0.0f;
			const size_t pk = oracle_piece_depth(m, n, k), pieces = (k + pk - 1) / pk;
			for (size_t p = 0; p < pieces; ++p) {
				const size_t pc = p * pk, kc = (k - pc < pk) ? k - pc : pk;
				float x = 0.0f;
				for (size_t q = pc; q < pc + kc; ++q) x = fmaf(op_a(ta, a, lda, i, q), op_b(tb, b, ldb, q, j), x);
				acc = p == 0 ? x : acc + x;
			}
			v = accumulate ? c_old[t] + acc : acc;
		}
		out[t] = v;
	}
}

/* tests/reference_gemm.hpp:31-45: the reference's own fp32 triple-loop ground truth (separate
 * multiply and add, -ffp-contract=off). */
void oracle_sgemm_naive(int ta, int tb, size_t m, size_t n, size_t k, const float* a, size_t lda,
		const float* b, size_t ldb, float* c, size_t ldc, int accumulate) {
	for (size_t i = 0; i < m; ++i)
		for (size_t j = 0; j < n; ++j) {
			float sum = 0.0f;
			for (size_t p = 0; p < k; ++p) sum += op_a(ta, a, lda, i, p) * op_b(tb, b, ldb, p, j);
			c[i * ldc + j] = accumulate ? c[i * ldc + j] + sum : sum;
		}
}

/* fp64 closed form: out = op(A) op(B) (+ C), mag = sum |a||b| (+ |C|); both dense m x n. */
void oracle_sgemm_f64(int ta, int tb, size_t m, size_t n, size_t k, const float* a, size_t lda,
		const float* b, size_t ldb, const float* c_in, size_t ldc, int accumulate, double* out, double* mag) {
	for (size_t i = 0; i < m; ++i)
		for (size_t j = 0; j < n; ++j) {
			double s = 0.0, g = 0.0;
			for (size_t p = 0; p < k; ++p) {
				const double t = (double)op_a(ta, a, lda, i, p) * (double)op_b(tb, b, ldb, p, j);
				s += t;
				g += fabs(t);
			}
			if (accumulate) {
				s += (double)c_in[i * ldc + j];
				g += fabs((double)c_in[i * ldc + j]);
			}
			out[i * n + j] = s;
			if (mag) mag[i * n + j] = g;
		}
}

/* Tensor::sum(0) of a {rows, inner} tensor (tensor.cpp:422-456): a zero-filled output, then the
 * rows added in order (the outer_size == 1 branch). */
void oracle_sum_axis0(const float* src, size_t rows, size_t inner, float* dst) {
	for (size_t j = 0; j < inner; ++j) dst[j] = 0.0f;
	for (size_t a = 0; a < rows; ++a)
		for (size_t j = 0; j < inner; ++j) dst[j] += src[a * inner + j];
}

/* lane_sum (ops.cpp:804-812): 8 partial sums, combined in a fixed tree, then the tail. */
float oracle_lane_sum(const float* p, size_t n) {
	float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
	size_t i = 0;
	for (; i + 8 <= n; i += 8)
		for (size_t k = 0; k < 8; ++k) a[k] += p[i + k];
	float t = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
	for (; i < n; ++i) t += p[i];
	return t;
}

/* linear forward (ops.cpp:714-730): Y = X W^T through sgemm(F,T), then Y[r][j] += b[j]. */
void oracle_linear_forward(const float* x, size_t M, size_t K, const float* w, size_t n, const float* bias,
		float* y) {
	oracle_sgemm(0, 1, M, n, K, x, K, w, K, y, n, 0);
	for (size_t r = 0; r < M; ++r)
		for (size_t j = 0; j < n; ++j) y[r * n + j] += bias[j];
}

/* linear backward (ops.cpp:731-744). dx = G W (F,F), dw = G^T X (T,F), each accumulating unless its
 * buffer is fresh (value.cpp:60-64). db follows accumulate_grad -> sum_to_shape: the gradient of shape
 * lead + {n} is reduced by Tensor::sum(0) once per leading axis (ops.cpp:35-53), then stored as
 * s + 0.0f when fresh or added (ops.cpp:64-73, 85-99). */
void oracle_linear_backward(const float* g, const float* x, const float* w, size_t M, size_t K, size_t n,
		const size_t* lead, int nlead, float* dx, int dx_first, float* dw, int dw_first, float* db,
		int db_first) {
	if (dx) oracle_sgemm(0, 0, M, K, n, g, n, w, K, dx, K, !dx_first);
	if (dw) oracle_sgemm(1, 0, n, K, M, g, n, x, K, dw, K, !dw_first);
	if (db) {
		size_t total = M;
		float* cur = (float*)malloc(sizeof(float) * (M * n > 0 ? M * n : 1));
		memcpy(cur, g, sizeof(float) * M * n);
		for (int d = 0; d < nlead; ++d) {
			const size_t rows = lead[d], inner = (total / (rows ? rows : 1)) * n;
			float* nxt = (float*)malloc(sizeof(float) * (inner > 0 ? inner : 1));
			if (rows == 0) {
				for (size_t j = 0; j < inner; ++j) nxt[j] = 0.0f;
			} else {
				oracle_sum_axis0(cur, rows, inner, nxt);
			}
			free(cur);
			cur = nxt;
			total = rows ? total / rows : 1;
		}
		for (size_t j = 0; j < n; ++j) db[j] = db_first ? cur[j] + 0.0f : db[j] + cur[j];
		free(cur);
	}
}

/* relu (ops.cpp:775-782). */
void oracle_relu(const float* x, float* y, size_t count) {
	for (size_t i = 0; i < count; ++i) y[i] = x[i] > 0.0f ? x[i] : 0.0f;
}

/* ---- normalisation ---- */

/* The eight-partial sums of ops.cpp:804-897 over one row, as one helper: mode 0 lane_sum(x), 1 lane_sq(x, mu),
 * 2 lane_sum of g masked by alive (alive NULL: g itself) with lane_dot of the same g against x - mu in *dot. */
static float lane_row(int mode, const float* x, const float* g, const unsigned char* alive, size_t n, float mu,
		float* dot) {
	float a[8] = {0, 0, 0, 0, 0, 0, 0, 0}, d[8] = {0, 0, 0, 0, 0, 0, 0, 0};
	size_t i = 0;
	for (; i + 8 <= n; i += 8)
		for (size_t k = 0; k < 8; ++k) {
			if (mode == 0) {
				a[k] += x[i + k];
			} else if (mode == 1) {
				const float t = x[i + k] - mu;
				a[k] += t * t;
			} else {
				const float gv = alive ? (alive[i + k] ? g[i + k] : 0.0f) : g[i + k];
				a[k] += gv;
				d[k] += gv * (x[i + k] - mu);
			}
		}
	float t = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
	float u = ((d[0] + d[1]) + (d[2] + d[3])) + ((d[4] + d[5]) + (d[6] + d[7]));
	for (; i < n; ++i) {
		if (mode == 0) {
			t += x[i];
		} else if (mode == 1) {
			t += (x[i] - mu) * (x[i] - mu);
		} else {
			const float gv = alive ? (alive[i] ? g[i] : 0.0f) : g[i];
			t += gv;
			u += gv * (x[i] - mu);
		}
	}
	if (dot) *dot = u;
	return t;
}

/* batchnorm forward in training mode (ops.cpp:900-958) on x {N, C, S}: per channel, in double over the samples in
 * order, the rows' lane sums, then lane_sq around the mean; y = (x - mu) * (w * inv) + b, alive and clipping with
 * relu. mean, var and inv_std receive C floats each (any may be NULL). */
void oracle_batchnorm_forward(const float* x, size_t N, size_t C, size_t S, const float* w, const float* b, float eps,
		int relu, float* y, unsigned char* alive, float* mean, float* var, float* inv_std) {
	const size_t M = N * S;
	for (size_t c = 0; c < C; ++c) {
		double sum = 0.0;
		for (size_t n = 0; n < N; ++n) sum += lane_row(0, x + (n * C + c) * S, NULL, NULL, S, 0.0f, NULL);
		const float mu = (float)(sum / (double)M);
		double sq = 0.0;
		for (size_t n = 0; n < N; ++n) sq += lane_row(1, x + (n * C + c) * S, NULL, NULL, S, mu, NULL);
		const float v = (float)(sq / (double)M);
		const float inv = 1.0f / sqrtf(v + eps);
		if (mean) mean[c] = mu;
		if (var) var[c] = v;
		if (inv_std) inv_std[c] = inv;
		const float scale = w[c] * inv;
		for (size_t n = 0; n < N; ++n)
			for (size_t s = 0; s < S; ++s) {
				const size_t i = (n * C + c) * S + s;
				const float t = (x[i] - mu) * scale + b[c];
				if (relu) {
					if (alive) alive[i] = t > 0.0f;
					y[i] = t > 0.0f ? t : 0.0f;
				} else {
					y[i] = t;
				}
			}
	}
}

/* batchnorm backward rule (ops.cpp:960-1000): per channel sdy = sum of lane_sum(g'), sdg = sum of lane_dot(g', x,
 * mu) in double over the samples in order (g' = g masked by alive), sdyx = sdg * inv; db += (float)sdy,
 * dw += (float)sdyx (first: 0 + value), dx = k * (M g' - sdy - ((x - mu) * inv) * sdyx), k = w * inv / M, stored
 * as term + 0 when first. */
void oracle_batchnorm_backward(const float* g, const float* x, const unsigned char* alive, const float* w,
		const float* mean, const float* inv_std, size_t N, size_t C, size_t S, float* dx, int dx_first, float* dw,
		int dw_first, float* db, int db_first) {
	const size_t M = N * S;
	for (size_t c = 0; c < C; ++c) {
		const float mu = mean[c], inv = inv_std[c];
		double sdy = 0.0, sdg = 0.0;
		for (size_t n = 0; n < N; ++n) {
			const size_t base = (n * C + c) * S;
			float dot = 0.0f;
			sdy += lane_row(2, x + base, g + base, alive ? alive + base : NULL, S, mu, &dot);
			sdg += dot;
		}
		const double sdyx = sdg * inv;
		if (db) db[c] = db_first ? 0.0f + (float)sdy : db[c] + (float)sdy;
		if (dw) dw[c] = dw_first ? 0.0f + (float)sdyx : dw[c] + (float)sdyx;
		if (dx) {
			const float k = w[c] * inv / (float)M;
			const float fm = (float)M, av = (float)sdy, bb = (float)sdyx;
			for (size_t n = 0; n < N; ++n)
				for (size_t s = 0; s < S; ++s) {
					const size_t i = (n * C + c) * S + s;
					const float gm = alive ? (alive[i] ? g[i] : 0.0f) : g[i];
					const float term = k * (fm * gm - av - ((x[i] - mu) * inv) * bb);
					dx[i] = dx_first ? term + 0.0f : dx[i] + term;
				}
		}
	}
}

/* layernorm forward (ops.cpp:1003-1034) over R rows of D: float sums in column order. mean, inv_std: R floats. */
void oracle_layernorm_forward(const float* x, size_t R, size_t D, const float* gm, const float* bt, float eps,
		float* y, float* mean, float* inv_std) {
	for (size_t r = 0; r < R; ++r) {
		const float* row = x + r * D;
		float sum = 0.0f;
		for (size_t j = 0; j < D; ++j) sum += row[j];
		const float mu = sum / (float)D;
		float sq = 0.0f;
		for (size_t j = 0; j < D; ++j) sq += (row[j] - mu) * (row[j] - mu);
		const float inv = 1.0f / sqrtf(sq / (float)D + eps);
		if (mean) mean[r] = mu;
		if (inv_std) inv_std[r] = inv;
		for (size_t j = 0; j < D; ++j) y[r * D + j] = (row[j] - mu) * inv * gm[j] + bt[j];
	}
}

/* layernorm backward rule (ops.cpp:1035-1077). */
void oracle_layernorm_backward(const float* g, const float* x, const float* gm, const float* mean,
		const float* inv_std, size_t R, size_t D, float* dx, int dx_first, float* dgamma, int dgamma_first,
		float* dbeta, int dbeta_first) {
	if (dx)
		for (size_t r = 0; r < R; ++r) {
			const float mu = mean[r], inv = inv_std[r];
			float a = 0.0f, b = 0.0f;
			for (size_t j = 0; j < D; ++j) {
				const float dxhat = g[r * D + j] * gm[j];
				a += dxhat;
				b += dxhat * ((x[r * D + j] - mu) * inv);
			}
			const float k = inv / (float)D, fd = (float)D;
			for (size_t j = 0; j < D; ++j) {
				const float dxhat = g[r * D + j] * gm[j];
				const float term = k * (fd * dxhat - a - ((x[r * D + j] - mu) * inv) * b);
				dx[r * D + j] = dx_first ? term + 0.0f : dx[r * D + j] + term;
			}
		}
	if (dgamma || dbeta)
		for (size_t j = 0; j < D; ++j) {
			float sg = 0.0f, sb = 0.0f;
			for (size_t r = 0; r < R; ++r) {
				const float gv = g[r * D + j];
				sg += gv * ((x[r * D + j] - mean[r]) * inv_std[r]);
				sb += gv;
			}
			if (dgamma) dgamma[j] = dgamma_first ? 0.0f + sg : dgamma[j] + sg;
			if (dbeta) dbeta[j] = dbeta_first ? 0.0f + sb : dbeta[j] + sb;
		}
}

/* fp64 closed forms: batchnorm's normalised output over the channel's N*S elements (biased variance), and
 * layernorm's over each row, without weights. */
void oracle_batchnorm_f64(const float* x, size_t N, size_t C, size_t S, double eps, double* xhat) {
	const size_t M = N * S;
	for (size_t c = 0; c < C; ++c) {
		double s = 0.0, q = 0.0;
		for (size_t n = 0; n < N; ++n)
			for (size_t t = 0; t < S; ++t) s += x[(n * C + c) * S + t];
		const double mu = s / (double)M;
		for (size_t n = 0; n < N; ++n)
			for (size_t t = 0; t < S; ++t) {
				const double d = x[(n * C + c) * S + t] - mu;
				q += d * d;
			}
		const double inv = 1.0 / sqrt(q / (double)M + eps);
		for (size_t n = 0; n < N; ++n)
			for (size_t t = 0; t < S; ++t) xhat[(n * C + c) * S + t] = (x[(n * C + c) * S + t] - mu) * inv;
	}
}

void oracle_layernorm_f64(const float* x, size_t R, size_t D, double eps, double* xhat) {
	for (size_t r = 0; r < R; ++r) {
		double s = 0.0, q = 0.0;
		for (size_t j = 0; j < D; ++j) s += x[r * D + j];
		const double mu = s / (double)D;
		for (size_t j = 0; j < D; ++j) q += (x[r * D + j] - mu) * (x[r * D + j] - mu);
		const double inv = 1.0 / sqrt(q / (double)D + eps);
		for (size_t j = 0; j < D; ++j) xhat[r * D + j] = (x[r * D + j] - mu) * inv;
	}
}

/* ---- element-wise: GELU and embedding ---- */

/* nn-cpp's exp_one and tanh_one (src/kernels/vmath.cpp:68-97): Cephes expf with the reference's constants; every
 * operation rounds on its own (-ffp-contract=off). */
static float vm_exp_one(float x) {
	if (x != x) return x;
	if (x < -87.3f) return 0.0f;
	if (x > 88.3f) return HUGE_VALF;
	const float n = nearbyintf(x * 1.44269504088896341f);
	float r = x - n * 0.693359375f;
	r = r - n * -2.12194440e-4f;
	float p = 1.9875691500e-4f;
	p = p * r + 1.3981999507e-3f;
	p = p * r + 8.3334519073e-3f;
	p = p * r + 4.1665795894e-2f;
	p = p * r + 1.6666665459e-1f;
	p = p * r + 5.0000001201e-1f;
	const float e = (p * (r * r) + r) + 1.0f;
	const uint32_t bits = (uint32_t)((int32_t)n + 127) << 23;
	float pow2;
	memcpy(&pow2, &bits, sizeof pow2);
	return e * pow2;
}

float oracle_tanh_one(float x) {
	if (x != x) return x;
	float z = x < -9.0f ? -9.0f : x;
	z = 9.0f < z ? 9.0f : z;
	const float e = vm_exp_one(z + z);
	return (e - 1.0f) / (e + 1.0f);
}

/* gelu forward (ops.cpp:451-466): th = tanh(k (x + c x x x)), y = 0.5 x (1 + th). */
void oracle_gelu_forward(const float* x, size_t count, float* y, float* th) {
	const float k = 0.7978845608f, c = 0.044715f;
	for (size_t i = 0; i < count; ++i) {
		const float t = oracle_tanh_one(k * (x[i] + c * x[i] * x[i] * x[i]));
		th[i] = t;
		y[i] = 0.5f * x[i] * (1.0f + t);
	}
}

/* gelu backward rule (ops.cpp:467-480). */
void oracle_gelu_backward(const float* x, const float* th, const float* g, size_t count, float* dx, int first) {
	const float k = 0.7978845608f, c = 0.044715f;
	for (size_t i = 0; i < count; ++i) {
		const float v = x[i], t = th[i];
		const float term = g[i] * (0.5f * (1.0f + t) + 0.5f * v * (1.0f - t * t) * k * (1.0f + 3.0f * c * v * v));
		dx[i] = first ? term + 0.0f : dx[i] + term;
	}
}

/* embedding backward rule (ops.cpp:2008-2014): a fresh table is zero-filled, then g row i is added to row rows[i]
 * for i in order. */
void oracle_embedding_backward(const float* g, const int32_t* rows, size_t count, size_t V, size_t D, float* dw,
		int first) {
	if (first)
		for (size_t e = 0; e < V * D; ++e) dw[e] = 0.0f;
	for (size_t i = 0; i < count; ++i)
		for (size_t d = 0; d < D; ++d) dw[(size_t)rows[i] * D + d] += g[i * D + d];
}

/* ---- max pooling ---- */

/* maxpool2d forward (ops.cpp:1609-1684): per window, best = -inf and at = 0, then row by row a value replaces
 * best only when greater; at is the winner's offset inside its (n, c) plane. */
void oracle_maxpool2d_forward(const float* x, size_t planes, size_t H, size_t W, size_t k, size_t s, float* y,
		uint32_t* argmax) {
	const size_t ho = (H - k) / s + 1, wo = (W - k) / s + 1;
	for (size_t p = 0; p < planes; ++p) {
		const float* plane = x + p * H * W;
		for (size_t oh = 0; oh < ho; ++oh)
			for (size_t ow = 0; ow < wo; ++ow) {
				float best = -INFINITY;
				uint32_t at = 0;
				for (size_t ph = 0; ph < k; ++ph)
					for (size_t pw = 0; pw < k; ++pw) {
						const size_t off = (oh * s + ph) * W + ow * s + pw;
						if (plane[off] > best) {
							best = plane[off];
							at = (uint32_t)off;
						}
					}
				y[(p * ho + oh) * wo + ow] = best;
				argmax[(p * ho + oh) * wo + ow] = at;
			}
	}
}

/* maxpool2d backward (ops.cpp:1686-1704): a fresh plane is zero-filled, then g[i] is added at argmax[i] for i in
 * output order. */
void oracle_maxpool2d_backward(const float* g, const uint32_t* argmax, size_t planes, size_t H, size_t W, size_t k,
		size_t s, float* dx, int first) {
	const size_t out_plane = ((H - k) / s + 1) * ((W - k) / s + 1);
	for (size_t p = 0; p < planes; ++p) {
		float* plane = dx + p * H * W;
		if (first)
			for (size_t i = 0; i < H * W; ++i) plane[i] = 0.0f;
		for (size_t i = p * out_plane; i < (p + 1) * out_plane; ++i) plane[argmax[i]] += g[i];
	}
}

/* ---- convolution ---- */

/* conv2d_output_size (ops.cpp:135-139). */
void oracle_conv2d_output_size(size_t h, size_t w, size_t kh, size_t kw, size_t stride, size_t padding,
		size_t* h_out, size_t* w_out) {
	*h_out = (h + 2 * padding - kh) / stride + 1;
	*w_out = (w + 2 * padding - kw) / stride + 1;
}

/* im2col_sample (ops.cpp:188-212), written from the definition: column row (c*kh + ph)*kw + pw,
 * column index oh*w_out + ow, zero where the tap falls in the padding. */
void oracle_im2col_sample(const float* x, float* col, size_t Cin, size_t H, size_t W, size_t kh, size_t kw,
		size_t stride, size_t padding) {
	size_t ho, wo;
	oracle_conv2d_output_size(H, W, kh, kw, stride, padding, &ho, &wo);
	const size_t hw = ho * wo;
	for (size_t c = 0; c < Cin; ++c)
		for (size_t ph = 0; ph < kh; ++ph)
			for (size_t pw = 0; pw < kw; ++pw) {
				float* row = col + ((c * kh + ph) * kw + pw) * hw;
				for (size_t oh = 0; oh < ho; ++oh)
					for (size_t ow = 0; ow < wo; ++ow) {
						const long ih = (long)(oh * stride + ph) - (long)padding;
						const long iw = (long)(ow * stride + pw) - (long)padding;
						row[oh * wo + ow] = (ih < 0 || iw < 0 || ih >= (long)H || iw >= (long)W)
							? 0.0f : x[(c * H + (size_t)ih) * W + (size_t)iw];
					}
			}
}

/* col2im_sample_add (ops.cpp:224-243): the transpose of im2col, adding taps in (c, ph, pw, oh, ow) order. */
void oracle_col2im_sample_add(const float* col, float* x, size_t Cin, size_t H, size_t W, size_t kh, size_t kw,
		size_t stride, size_t padding) {
	size_t ho, wo;
	oracle_conv2d_output_size(H, W, kh, kw, stride, padding, &ho, &wo);
	const size_t hw = ho * wo;
	for (size_t c = 0; c < Cin; ++c)
		for (size_t ph = 0; ph < kh; ++ph)
			for (size_t pw = 0; pw < kw; ++pw) {
				const float* row = col + ((c * kh + ph) * kw + pw) * hw;
				for (size_t oh = 0; oh < ho; ++oh)
					for (size_t ow = 0; ow < wo; ++ow) {
						const long ih = (long)(oh * stride + ph) - (long)padding;
						const long iw = (long)(ow * stride + pw) - (long)padding;
						if (ih < 0 || iw < 0 || ih >= (long)H || iw >= (long)W) continue;
						x[(c * H + (size_t)ih) * W + (size_t)iw] += row[oh * wo + ow];
					}
			}
}

/* conv2d_impl forward (ops.cpp:1345-1410): per sample, im2col, Y_n = W col (sgemm F,F), then
 * v = acc + b[c]; alive = v > 0; y = alive ? v : 0 (fused ReLU) or y = acc + b[c]. */
void oracle_conv2d_forward(const float* x, size_t N, size_t Cin, size_t H, size_t W, const float* w, size_t Cout,
		size_t kh, size_t kw, const float* bias, size_t stride, size_t padding, int fuse_relu, float* y,
		unsigned char* alive) {
	size_t ho, wo;
	oracle_conv2d_output_size(H, W, kh, kw, stride, padding, &ho, &wo);
	const size_t hw = ho * wo, K = Cin * kh * kw;
	float* col = (float*)malloc(sizeof(float) * (K * hw > 0 ? K * hw : 1));
	for (size_t n = 0; n < N; ++n) {
		oracle_im2col_sample(x + n * Cin * H * W, col, Cin, H, W, kh, kw, stride, padding);
		float* yn = y + n * Cout * hw;
		oracle_sgemm(0, 0, Cout, hw, K, w, K, col, hw, yn, hw, 0);
		for (size_t c = 0; c < Cout; ++c) {
			float* row = yn + c * hw;
			for (size_t i = 0; i < hw; ++i) {
				if (fuse_relu) {
					const float v = row[i] + bias[c];
					if (alive) alive[(n * Cout + c) * hw + i] = v > 0.0f;
					row[i] = v > 0.0f ? v : 0.0f;
				} else {
					row[i] += bias[c];
				}
			}
		}
	}
	free(col);
}

/* conv2d_impl backward (ops.cpp:1418-1463). g is masked by alive when given; db_n = lane_sum over each
 * channel's row; dW_n = g col^T (sgemm F,T); dcol = W^T g (sgemm T,F) scattered back by col2im into a
 * zero-filled (fresh) or existing dx; then the per-sample dW and db are summed in sample order by
 * Tensor::sum(0) and added to the gradients (bias.grad() += ..., weight.grad() += ...). Here dw and db
 * receive those sums (the caller adds them to an existing gradient if it has one). */
void oracle_conv2d_backward(const float* g, const float* x, const float* w, const unsigned char* alive, size_t N,
		size_t Cin, size_t H, size_t W, size_t Cout, size_t kh, size_t kw, size_t stride, size_t padding,
		float* dx, int dx_first, float* dw, float* db) {
	size_t ho, wo;
	oracle_conv2d_output_size(H, W, kh, kw, stride, padding, &ho, &wo);
	const size_t hw = ho * wo, K = Cin * kh * kw, xs = Cin * H * W;
	float* col = (float*)malloc(sizeof(float) * (K * hw > 0 ? K * hw : 1));
	float* masked = (float*)malloc(sizeof(float) * (Cout * hw > 0 ? Cout * hw : 1));
	float* gw = dw ? (float*)malloc(sizeof(float) * (N * Cout * K > 0 ? N * Cout * K : 1)) : NULL;
	float* gb = db ? (float*)malloc(sizeof(float) * (N * Cout > 0 ? N * Cout : 1)) : NULL;
	for (size_t n = 0; n < N; ++n) {
		const float* gn = g + n * Cout * hw;
		if (alive) {
			const unsigned char* f = alive + n * Cout * hw;
			for (size_t i = 0; i < Cout * hw; ++i) masked[i] = f[i] ? gn[i] : 0.0f;
			gn = masked;
		}
		if (gb)
			for (size_t c = 0; c < Cout; ++c) gb[n * Cout + c] = oracle_lane_sum(gn + c * hw, hw);
		if (gw) {
			oracle_im2col_sample(x + n * xs, col, Cin, H, W, kh, kw, stride, padding);
			oracle_sgemm(0, 1, Cout, K, hw, gn, hw, col, hw, gw + n * Cout * K, K, 0);
		}
		if (dx) {
			oracle_sgemm(1, 0, K, hw, Cout, w, K, gn, hw, col, hw, 0);
			float* dxn = dx + n * xs;
			if (dx_first)
				for (size_t i = 0; i < xs; ++i) dxn[i] = 0.0f;
			oracle_col2im_sample_add(col, dxn, Cin, H, W, kh, kw, stride, padding);
		}
	}
	if (db) oracle_sum_axis0(gb, N, Cout, db);
	if (dw) oracle_sum_axis0(gw, N, Cout * K, dw);
	free(col);
	free(masked);
	free(gw);
	free(gb);
}

/* Direct convolution in fp64 (the shape of test_autograd.cpp:420-440's reference_conv), with the
 * magnitude sum |x||w| + |b| for error bounds. */
void oracle_conv2d_f64(const float* x, size_t N, size_t Cin, size_t H, size_t W, const float* w, size_t Cout,
		size_t kh, size_t kw, const float* bias, size_t stride, size_t padding, double* y, double* mag) {
	size_t ho, wo;
	oracle_conv2d_output_size(H, W, kh, kw, stride, padding, &ho, &wo);
	for (size_t n = 0; n < N; ++n)
		for (size_t co = 0; co < Cout; ++co)
			for (size_t oh = 0; oh < ho; ++oh)
				for (size_t ow = 0; ow < wo; ++ow) {
					double s = bias[co], g = fabs((double)bias[co]);
					for (size_t c = 0; c < Cin; ++c)
						for (size_t i = 0; i < kh; ++i)
							for (size_t j = 0; j < kw; ++j) {
								const long ih = (long)(oh * stride + i) - (long)padding;
								const long iw = (long)(ow * stride + j) - (long)padding;
								if (ih < 0 || iw < 0 || ih >= (long)H || iw >= (long)W) continue;
								const double t = (double)x[((n * Cin + c) * H + (size_t)ih) * W + (size_t)iw] *
									(double)w[((co * Cin + c) * kh + i) * kw + j];
								s += t;
								g += fabs(t);
							}
					const size_t o = ((n * Cout + co) * ho + oh) * wo + ow;
					y[o] = s;
					if (mag) mag[o] = g;
				}
}

/* ---- attention ---- */

static inline float std_max(float a, float b) { return (a < b) ? b : a; }  /* std::max(a, b) */

/* exp of the softmax: the C library's expf, which is what the reference's std::exp(float) calls (ops.cpp:1199). */
static inline float softmax_exp(float x) { return expf(x); }

/* masked_softmax_row (ops.cpp:1183-1204). */
void oracle_masked_softmax_row(const float* row, float* o, size_t Tk, size_t i, const float* ph, int causal,
		float scale_by) {
	for (size_t j = 0; j < Tk; ++j) {
		float v = row[j] * scale_by;
		if (ph && ph[j] == 0.0f) v = -1e9f;
		if (causal && j > i) v = -2e9f;
		o[j] = v;
	}
	float m = o[0];
	for (size_t j = 1; j < Tk; ++j) m = std_max(m, o[j]);
	const size_t live = causal ? (Tk < i + 1 ? Tk : i + 1) : Tk;
	float sum = 0.0f;
	for (size_t j = 0; j < live; ++j) {
		o[j] = softmax_exp(o[j] - m);
		sum += o[j];
	}
	for (size_t j = live; j < Tk; ++j) o[j] = 0.0f;
	for (size_t j = 0; j < Tk; ++j) o[j] /= sum;
}

/* masked_softmax_row_backward (ops.cpp:1216-1224). */
void oracle_masked_softmax_row_backward(const float* y, float* g, size_t Tk, size_t i, const float* ph,
		int causal, float scale_by) {
	float dot = 0.0f;
	for (size_t j = 0; j < Tk; ++j) dot += g[j] * y[j];
	for (size_t j = 0; j < Tk; ++j) {
		const int masked = (ph && ph[j] == 0.0f) || (causal && j > i);
		g[j] = masked ? 0.0f : scale_by * (y[j] * (g[j] - dot)) + 0.0f;
	}
}

/* scaled_masked_softmax backward over {N, H, Tq, Tk} (ops.cpp:1318-1341): per row, dot = sum of g y in j order
 * (each product rounded, then added), term = scale (y (g - dot)); a fresh gradient stores term + 0.0f (0 where
 * masked), an existing one adds term where not masked. */
void oracle_scaled_masked_softmax_backward(const float* y, const float* g, size_t N, size_t H, size_t Tq, size_t Tk,
		float scale_by, const float* pad, int causal, float* dx, int first) {
	for (size_t r = 0; r < N * H * Tq; ++r) {
		const size_t i = r % Tq, n = r / (H * Tq);
		const float* ph = pad ? pad + n * Tk : NULL;
		float dot = 0.0f;
		for (size_t j = 0; j < Tk; ++j) dot += g[r * Tk + j] * y[r * Tk + j];
		for (size_t j = 0; j < Tk; ++j) {
			const int masked = (ph && ph[j] == 0.0f) || (causal && j > i);
			const float term = scale_by * (y[r * Tk + j] * (g[r * Tk + j] - dot));
			if (first) dx[r * Tk + j] = masked ? 0.0f : term + 0.0f;
			else if (!masked) dx[r * Tk + j] += term;
		}
	}
}

/* attention forward (ops.cpp:1226-1261): per (n, h), S = Q_h K_h^T (sgemm F,T with row stride D),
 * masked softmax row by row into probs, O_h = P V_h (sgemm F,F) into column block h*Dh. */
void oracle_attention_forward(const float* q, const float* k, const float* v, size_t N, size_t Tq, size_t Tk,
		size_t D, size_t heads, const float* pad, int causal, float* out, float* probs) {
	const size_t H = heads, Dh = D / H;
	const float scale_by = 1.0f / sqrtf((float)Dh);
	for (size_t nh = 0; nh < N * H; ++nh) {
		const size_t n = nh / H, h = nh % H;
		float* p = probs + nh * Tq * Tk;
		oracle_sgemm(0, 1, Tq, Tk, Dh, q + n * Tq * D + h * Dh, D, k + n * Tk * D + h * Dh, D, p, Tk, 0);
		for (size_t i = 0; i < Tq; ++i)
			oracle_masked_softmax_row(p + i * Tk, p + i * Tk, Tk, i, pad ? pad + n * Tk : NULL, causal, scale_by);
		oracle_sgemm(0, 0, Tq, Dh, Tk, p, Tk, v + n * Tk * D + h * Dh, D, out + n * Tq * D + h * Dh, D, 0);
	}
}

/* attention backward (ops.cpp:1263-1295), per (n, h) in order: dP = G_h V_h^T, dV += P^T G_h,
 * softmax backward row by row, dQ += dS K_h, dK += dS^T Q_h. */
void oracle_attention_backward(const float* g, const float* q, const float* k, const float* v,
		const float* probs, size_t N, size_t Tq, size_t Tk, size_t D, size_t heads, const float* pad, int causal,
		float* dq, int dq_first, float* dk, int dk_first, float* dv, int dv_first) {
	const size_t H = heads, Dh = D / H;
	const float scale_by = 1.0f / sqrtf((float)Dh);
	float* ds = (float*)malloc(sizeof(float) * (Tq * Tk > 0 ? Tq * Tk : 1));
	for (size_t nh = 0; nh < N * H; ++nh) {
		const size_t n = nh / H, h = nh % H;
		const float* p = probs + nh * Tq * Tk;
		const float* gh = g + n * Tq * D + h * Dh;
		oracle_sgemm(0, 1, Tq, Tk, Dh, gh, D, v + n * Tk * D + h * Dh, D, ds, Tk, 0);
		if (dv) oracle_sgemm(1, 0, Tk, Dh, Tq, p, Tk, gh, D, dv + n * Tk * D + h * Dh, D, !dv_first);
		if (!dq && !dk) continue;
		for (size_t i = 0; i < Tq; ++i)
			oracle_masked_softmax_row_backward(p + i * Tk, ds + i * Tk, Tk, i, pad ? pad + n * Tk : NULL, causal,
				scale_by);
		if (dq) oracle_sgemm(0, 0, Tq, Dh, Tk, ds, Tk, k + n * Tk * D + h * Dh, D, dq + n * Tq * D + h * Dh, D, !dq_first);
		if (dk) oracle_sgemm(1, 0, Tk, Dh, Tq, ds, Tk, q + n * Tq * D + h * Dh, D, dk + n * Tk * D + h * Dh, D, !dk_first);
	}
	free(ds);
}

/* scaled_masked_softmax forward (ops.cpp:1298-1322) over {N, H, Tq, Tk}. */
void oracle_scaled_masked_softmax(const float* x, size_t N, size_t H, size_t Tq, size_t Tk, float scale_by,
		const float* pad, int causal, float* y) {
	const size_t R = N * H * Tq;
	for (size_t r = 0; r < R; ++r) {
		const size_t i = r % Tq, n = r / (H * Tq);
		oracle_masked_softmax_row(x + r * Tk, y + r * Tk, Tk, i, pad ? pad + n * Tk : NULL, causal, scale_by);
	}
}

/* Attention in fp64: the per-head softmax(scale Q K^T + mask) V closed form. */
void oracle_attention_f64(const float* q, const float* k, const float* v, size_t N, size_t Tq, size_t Tk,
		size_t D, size_t heads, const float* pad, int causal, double* out, double* probs) {
	const size_t H = heads, Dh = D / H;
	const double scale_by = 1.0 / sqrt((double)Dh);
	double* s = (double*)malloc(sizeof(double) * (Tk > 0 ? Tk : 1));
	for (size_t n = 0; n < N; ++n)
		for (size_t h = 0; h < H; ++h)
			for (size_t i = 0; i < Tq; ++i) {
				double mx = -INFINITY;
				for (size_t j = 0; j < Tk; ++j) {
					double t = 0.0;
					for (size_t d = 0; d < Dh; ++d)
						t += (double)q[(n * Tq + i) * D + h * Dh + d] * (double)k[(n * Tk + j) * D + h * Dh + d];
					t *= scale_by;
					if (pad && pad[n * Tk + j] == 0.0f) t = -1e9;
					if (causal && j > i) t = -2e9;
					s[j] = t;
					if (t > mx) mx = t;
				}
				double z = 0.0;
				for (size_t j = 0; j < Tk; ++j) {
					s[j] = (causal && j > i) ? 0.0 : exp(s[j] - mx);
					z += s[j];
				}
				for (size_t j = 0; j < Tk; ++j) {
					s[j] /= z;
					if (probs) probs[((n * H + h) * Tq + i) * Tk + j] = s[j];
				}
				for (size_t d = 0; d < Dh; ++d) {
					double t = 0.0;
					for (size_t j = 0; j < Tk; ++j) t += s[j] * (double)v[(n * Tk + j) * D + h * Dh + d];
					out[(n * Tq + i) * D + h * Dh + d] = t;
				}
			}
	free(s);
}
