// ops_linear.hip - extern "C" entry points of nn::linear and the ReLU node (include/nnh.h).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "abi_common.hpp"
#include "kernels/hip/reduce.hpp"
#include "nnh.h"
#include "workspace.hpp"

using namespace nnh;

namespace {

bool product_fits(const size_t* dims, int n, size_t& out) {
	uint64_t p = 0;
	if (!count_ok(dims, n, p)) return false;
	out = (size_t)p;
	return true;
}

// Scratch of nnh_linear_backward: the depth-cut partials of dX and dW, or two buffers for a bias gradient
// reduced over several leading axes; they are taken one after the other, so the largest is what it needs.
size_t linear_backward_ws(const size_t* lead, int nlead, size_t M, size_t K, size_t n, bool dx, bool dw, bool db) {
	size_t bytes = 0;
	if (dx) bytes = std::max(bytes, gemm_workspace_bytes(M, K, n, 1));
	if (dw) bytes = std::max(bytes, gemm_workspace_bytes(n, K, M, 1));
	if (db && n > 0 && nlead > 1) {
		size_t row = n;
		for (int d = 1; d < nlead; ++d) row *= lead[d];
		WorkspacePlan plan;
		const size_t tmp_bytes = (row ? row : 1) * sizeof(float);
		plan.add(tmp_bytes);
		plan.add(tmp_bytes);
		bytes = std::max(bytes, plan.total);
	}
	return bytes;
}

}  // namespace

extern "C" {

int nnh_linear_forward_workspace_size(size_t M, size_t K, size_t n, size_t* bytes) {
	return query_both_modes(bytes, [&](size_t* bytes) {
		return put_bytes(bytes, gemm_workspace_bytes(M, n, K, 1));
	});
}

int nnh_linear_backward_workspace_size(const size_t* lead, int nlead, size_t K, size_t n, int want_dx, int want_dw,
                                       int want_db, size_t* bytes) {
	return query_both_modes(bytes, [&](size_t* bytes) {
		if (nlead > 0 && !lead) return fail(NNH_ERR_INVALID, "lead is null");
		if (nlead < 1) return fail(NNH_ERR_SHAPE, "linear input needs at least 2 dimensions");
		size_t M = 0;
		if (!product_fits(lead, nlead, M)) return fail(NNH_ERR_INVALID, "input size overflows");
		return put_bytes(bytes, linear_backward_ws(lead, nlead, M, K, n, want_dx, want_dw, want_db));
	});
}

int nnh_linear_forward(const float* x, size_t M, size_t K, const float* w, size_t n, const float* bias, int relu,
                       float* y, void* stream) {
	NumericsScope numerics_scope(stream);
	if (M > 0 && n > 0 && !bias) return fail(NNH_ERR_INVALID, "bias is null");
	nnh_epilogue ep{NNH_BIAS_COL, relu ? 1 : 0, bias, nullptr};
	GemmCall g;
	// Y = X W^T (ops.cpp:725): sgemm(F, T, M, n, K, x, K, w, K, y, n, false), then + bias (726-730)
	int rc = build_gemm(0, 1, M, n, K, x, K, w, K, y, n, 0, nullptr, &ep, g);
	if (rc != NNH_OK) return rc;
	return run_gemm(g, stream, -1);
}

int nnh_linear_forward_multi(const float* x, size_t M, size_t K, int count, const float* const* w, const size_t* n,
                             const float* const* bias, float* const* y, void* stream) {
	NumericsScope numerics_scope(stream);
	if (count < 1 || count > 8) return fail(NNH_ERR_INVALID, "linear multi: count must be 1 to 8");
	if (!w || !n || !bias || !y) return fail(NNH_ERR_INVALID, "linear multi: null array");
	GemmCall calls[8];
	for (int i = 0; i < count; ++i) {
		if (M > 0 && n[i] > 0 && !bias[i]) return fail(NNH_ERR_INVALID, "bias is null");
		nnh_epilogue ep{NNH_BIAS_COL, 0, bias[i], nullptr};
		const int rc = build_gemm(0, 1, M, n[i], K, x, K, w[i], K, y[i], n[i], 0, nullptr, &ep, calls[i]);
		if (rc != NNH_OK) return rc;
	}
	// no output may overlap another output or another layer's weight or bias (build_gemm checked x and its own)
	for (int i = 0; i < count; ++i)
		for (int j = 0; j < count; ++j) {
			if (i == j || M == 0 || n[i] == 0) continue;
			const uint64_t yb = (uint64_t)M * n[i] * 4;
			if ((j < i && n[j] > 0 && ranges_overlap(y[i], yb, y[j], (uint64_t)M * n[j] * 4)) ||
			    ranges_overlap(y[i], yb, w[j], (uint64_t)n[j] * K * 4) || ranges_overlap(y[i], yb, bias[j], n[j] * 4))
				return fail(NNH_ERR_ALIAS, "linear multi: an output overlaps another layer's output or parameters");
		}
	bool grouped = false;
	if (count >= 2) {
		const int rc = hip_status(gemm_launch_group(calls, count, reinterpret_cast<hipStream_t>(stream), grouped),
		                          "linear multi");
		if (rc != NNH_OK || grouped) return rc;
	}
	for (int i = 0; i < count; ++i) {
		const int rc = run_gemm(calls[i], stream, -1);
		if (rc != NNH_OK) return rc;
	}
	return NNH_OK;
}

int nnh_linear_gelu_forward(const float* x, size_t M, size_t K, const float* w, size_t n, const float* bias, float* h,
                            float* y, float* tanh_saved, void* stream) {
	NumericsScope numerics_scope(stream);
	if (M > 0 && n > 0 && (!bias || !y || !tanh_saved)) return fail(NNH_ERR_INVALID, "linear gelu: null pointer");
	const uint64_t bytes = (uint64_t)M * n * 4;
	if (M > 0 && n > 0 &&
	    (ranges_overlap(y, bytes, h, bytes) || ranges_overlap(tanh_saved, bytes, h, bytes) ||
	     ranges_overlap(tanh_saved, bytes, y, bytes) || ranges_overlap(y, bytes, x, (uint64_t)M * K * 4) ||
	     ranges_overlap(tanh_saved, bytes, x, (uint64_t)M * K * 4) || ranges_overlap(y, bytes, w, (uint64_t)n * K * 4) ||
	     ranges_overlap(tanh_saved, bytes, w, (uint64_t)n * K * 4)))
		return fail(NNH_ERR_ALIAS, "linear gelu: the outputs overlap each other or the inputs");
	nnh_epilogue ep{NNH_BIAS_COL, 0, bias, nullptr};
	GemmCall g;
	int rc = build_gemm(0, 1, M, n, K, x, K, w, K, h, n, 0, nullptr, &ep, g);
	if (rc != NNH_OK || M == 0 || n == 0) return rc;
	if (chain4_ok(g)) {  // the chain kernel applies the GELU in its epilogue
		g.ep.gelu_y = y;
		g.ep.gelu_t = tanh_saved;
		return hip_status(gemm_chain4_launch(g, reinterpret_cast<hipStream_t>(stream)), "linear gelu");
	}
	rc = run_gemm(g, stream, -1);
	if (rc != NNH_OK) return rc;
	return nnh_gelu_forward(h, M * n, y, tanh_saved, stream);
}

int nnh_linear_forward_add(const float* x, size_t M, size_t K, const float* w, size_t n, const float* bias,
                           const float* residual, float* y, void* stream) {
	NumericsScope numerics_scope(stream);
	if (M > 0 && n > 0 && (!bias || !residual)) return fail(NNH_ERR_INVALID, "bias or residual is null");
	if (M > 0 && n > 0 && residual != y && ranges_overlap(residual, (uint64_t)M * n * 4, y, (uint64_t)M * n * 4))
		return fail(NNH_ERR_ALIAS, "residual overlaps y other than in place");
	nnh_epilogue ep{NNH_BIAS_COL, 0, bias, nullptr};
	GemmCall g;
	int rc = build_gemm(0, 1, M, n, K, x, K, w, K, y, n, 0, nullptr, &ep, g);
	if (rc != NNH_OK) return rc;
	g.ep.res = residual;
	return run_gemm(g, stream, -1);
}

int nnh_linear_backward(const float* g, const float* x, const float* w, const size_t* lead, int nlead, size_t K,
                        size_t n, float* dx, int dx_first, float* dw, int dw_first, float* db, int db_first,
                        void* stream) {
	NumericsScope numerics_scope(stream);
	if (nlead > 0 && !lead) return fail(NNH_ERR_INVALID, "lead is null");
	if (nlead < 1) return fail(NNH_ERR_SHAPE, "linear input needs at least 2 dimensions");
	size_t M = 0;
	if (!product_fits(lead, nlead, M)) return fail(NNH_ERR_INVALID, "input size overflows");
	if (!count_ok({M, K}) || !count_ok({M, n}) || !count_ok({n, K}))
		return fail(NNH_ERR_INVALID, "linear: size out of range (above 2^60 elements)");
	hipStream_t s = reinterpret_cast<hipStream_t>(stream);
	// db of a 2-D gradient is one Tensor::sum(0): each column of G folded over the rows in order from +0, which is
	// the row sum of op(A) = G^T over k in the dW product, so that product computes it on the way
	const bool db_in_dw = dw && db && nlead == 1 && M > 0 && K > 0 && n > 0 && !depth_cut((int64_t)n, (int64_t)K, (int64_t)M) &&
	                      !ranges_overlap(db, n * 4, dw, (uint64_t)n * K * 4) && !ranges_overlap(db, n * 4, g, (uint64_t)M * n * 4) &&
	                      !ranges_overlap(db, n * 4, x, (uint64_t)M * K * 4);
	// every argument is checked before anything is enqueued
	GemmCall cx, cw;
	if (dx) {  // dX = G W (ops.cpp:737)
		const int rc = build_gemm(0, 0, M, K, n, g, n, w, K, dx, K, !dx_first, nullptr, nullptr, cx);
		if (rc != NNH_OK) return rc;
	}
	if (dw) {  // dW = G^T X (ops.cpp:741)
		const int rc = build_gemm(1, 0, n, K, M, g, n, x, K, dw, K, !dw_first, nullptr, nullptr, cw);
		if (rc != NNH_OK) return rc;
		if (db_in_dw) {
			cw.rowsum = db;
			cw.rowsum_combine = db_first ? 1 : 2;
		}
	}
	if (db && n > 0 && M > 0) {
		if (!g) return fail(NNH_ERR_INVALID, "G is null");
		if (ranges_overlap(db, n * 4, g, (uint64_t)M * n * 4)) return fail(NNH_ERR_ALIAS, "db overlaps G");
	}
	// db of a three-dimensional G is the two ordered sums of sum_to_shape (first over axis 0, then axis 1, each
	// from +0): folded into a cut dW product that runs on the 16x16x4 pieces kernel, which sums G's columns in one
	// more wave while the product runs
	bool db_in_pieces = false;
	if (dw && db && nlead == 2 && M > 0 && K > 0 && n > 0 && depth_cut((int64_t)n, (int64_t)K, (int64_t)M) &&
	    !ranges_overlap(db, n * 4, dw, (uint64_t)n * K * 4) && !ranges_overlap(db, n * 4, x, (uint64_t)M * K * 4)) {
		GemmCall t = cw;
		t.rowsum = db;
		t.rowsum_combine = db_first ? 1 : 2;
		t.rowsum_outer = (int64_t)lead[0];
		if (pieces4_takes(t)) {
			cw = t;
			db_in_pieces = true;
		}
	}
	{
		const int rc = check_workspace(stream, linear_backward_ws(lead, nlead, M, K, n, dx, dw, db));
		if (rc != NNH_OK) return rc;
	}
	// the two products in one launch when neither writes what the other reads or writes (the reference runs dX
	// first; with disjoint buffers the order cannot show)
	bool paired = false;
	if (dx && dw && M > 0 && K > 0 && n > 0) {
		const uint64_t bx = (uint64_t)M * K * 4, bw = (uint64_t)n * K * 4, bg = (uint64_t)M * n * 4;
		const bool apart = !ranges_overlap(dx, bx, g, bg) && !ranges_overlap(dx, bx, w, bw) &&
		                   !ranges_overlap(dx, bx, x, bx) && !ranges_overlap(dx, bx, dw, bw) &&
		                   !ranges_overlap(dw, bw, w, bw) &&
		                   (!(db_in_dw || db_in_pieces) ||
		                    (!ranges_overlap(db, n * 4, dx, bx) && !ranges_overlap(db, n * 4, w, bw)));
		if (apart) {
			const int rc = hip_status(gemm_launch_pair(cx, cw, s, paired), "linear backward");
			if (rc != NNH_OK) return rc;
		}
	}
	if (!paired) {
		if (dx) {
			const int rc = run_gemm(cx, stream, -1);
			if (rc != NNH_OK) return rc;
		}
		if (dw) {
			const int rc = run_gemm(cw, stream, -1);
			if (rc != NNH_OK) return rc;
		}
	}
	if (db && n > 0 && !db_in_dw && !db_in_pieces) {
		// accumulate_grad(bias, G): Tensor::sum(0) once per leading axis (ops.cpp:35-53), then stored as
		// s + 0.0f into a fresh gradient or added (ops.cpp:85-99)
		const int combine = db_first ? 1 : 2;
		if (nlead == 1) return hip_status(sum_rows(g, (int64_t)lead[0], (int64_t)n, db, combine, s), "bias gradient");
		if (nlead == 2 && sum_rows2_fits((int64_t)lead[0], (int64_t)lead[1], (int64_t)n))
			return hip_status(sum_rows2(g, (int64_t)lead[0], (int64_t)lead[1], (int64_t)n, db, combine, s), "bias gradient");
		// suffix[d] = n * prod(lead[d+1 ..]): the row length left after reducing axes 0..d
		std::vector<size_t> suffix(nlead);
		suffix[nlead - 1] = n;
		for (int d = nlead - 2; d >= 0; --d) suffix[d] = suffix[d + 1] * lead[d + 1];
		WorkspacePlan plan;
		const size_t tmp_bytes = (suffix[0] ? suffix[0] : 1) * sizeof(float);
		const size_t off[2] = {plan.add(tmp_bytes), plan.add(tmp_bytes)};
		StreamWorkspace ws(s, plan.total);
		hipError_t e = ws.error();
		const float* cur = g;
		for (int d = 0; d < nlead && e == hipSuccess; ++d) {
			if (d == nlead - 1) {
				e = sum_rows(cur, (int64_t)lead[d], (int64_t)n, db, combine, s);
				break;
			}
			float* out = ws.at<float>(off[d & 1]);
			e = sum_rows(cur, (int64_t)lead[d], (int64_t)suffix[d], out, 0, s);
			cur = out;
		}
		return hip_status(e, "bias gradient");
	}
	return NNH_OK;
}

int nnh_relu_forward(const float* x, float* y, size_t count, void* stream) {
	if (count == 0) return NNH_OK;
	if (!x || !y) return fail(NNH_ERR_INVALID, "null pointer");
	if (count > kMaxElems) return fail(NNH_ERR_INVALID, "count out of range (above 2^60)");
	if (partial_overlap(y, count * 4, x, count * 4)) return fail(NNH_ERR_ALIAS, "y overlaps x other than in place");
	return hip_status(relu_forward(x, y, (int64_t)count, reinterpret_cast<hipStream_t>(stream)), "relu forward");
}

int nnh_relu_backward(const float* x, const float* g, float* dx, int first, size_t count, void* stream) {
	if (count == 0) return NNH_OK;
	if (!x || !g || !dx) return fail(NNH_ERR_INVALID, "null pointer");
	if (count > kMaxElems) return fail(NNH_ERR_INVALID, "count out of range (above 2^60)");
	if (partial_overlap(dx, count * 4, g, count * 4) || partial_overlap(dx, count * 4, x, count * 4))
		return fail(NNH_ERR_ALIAS, "dx overlaps x or g other than in place");
	return hip_status(relu_backward(x, g, dx, (int64_t)count, first, reinterpret_cast<hipStream_t>(stream)),
	                  "relu backward");
}

int nnh_add_to_grad(float* dst, const float* src, size_t count, int first, void* stream) {
	if (count == 0) return NNH_OK;
	if (!dst || !src) return fail(NNH_ERR_INVALID, "null pointer");
	if (count > kMaxElems) return fail(NNH_ERR_INVALID, "count out of range (above 2^60)");
	if (dst != src && ranges_overlap(dst, count * 4, src, count * 4)) return fail(NNH_ERR_ALIAS, "dst overlaps src");
	return hip_status(add_to_grad(dst, src, (int64_t)count, first ? 1 : 0, reinterpret_cast<hipStream_t>(stream)),
	                  "add_to_grad");
}

int nnh_add_to_grad2(float* dst0, int first0, float* dst1, int first1, const float* src, size_t count, void* stream) {
	if (count == 0) return NNH_OK;
	if (!dst0 || !dst1 || !src) return fail(NNH_ERR_INVALID, "null pointer");
	if (count > kMaxElems) return fail(NNH_ERR_INVALID, "count out of range (above 2^60)");
	const uint64_t b = count * 4;
	if (ranges_overlap(dst0, b, dst1, b) || ranges_overlap(dst0, b, src, b) || ranges_overlap(dst1, b, src, b))
		return fail(NNH_ERR_ALIAS, "add_to_grad2: the gradients overlap each other or src");
	return hip_status(add_to_grad2(dst0, first0 ? 1 : 0, dst1, first1 ? 1 : 0, src, (int64_t)count,
	                               reinterpret_cast<hipStream_t>(stream)),
	                  "add_to_grad2");
}

int nnh_zero_many(float* const* buffers, const size_t* counts, size_t n, void* stream) {
	if (n == 0) return NNH_OK;
	if (!buffers || !counts) return fail(NNH_ERR_INVALID, "zero_many: null pointer");
	uint64_t total = 0;
	for (size_t i = 0; i < n; ++i) {
		if (counts[i] > 0 && !buffers[i]) return fail(NNH_ERR_INVALID, "zero_many: null buffer");
		if (counts[i] > ((uint64_t)1 << 60) || total + counts[i] > ((uint64_t)1 << 60))
			return fail(NNH_ERR_INVALID, "zero_many: size out of range (above 2^60 elements)");
		total += counts[i];
	}
	for (size_t i = 0; i < n; ++i)
		for (size_t j = i + 1; j < n; ++j)
			if (ranges_overlap(buffers[i], (uint64_t)counts[i] * 4, buffers[j], (uint64_t)counts[j] * 4))
				return fail(NNH_ERR_ALIAS, "zero_many: buffers overlap");
	hipStream_t s = reinterpret_cast<hipStream_t>(stream);
	for (size_t b = 0; b < n; b += kZeroJobs) {
		ZeroJobs jobs{};
		jobs.n = (int)std::min<size_t>(kZeroJobs, n - b);
		for (int i = 0; i < jobs.n; ++i) {
			jobs.p[i] = buffers[b + i];
			jobs.start[i + 1] = jobs.start[i] + (int64_t)counts[b + i];
		}
		const hipError_t e = zero_many(jobs, s);
		if (e != hipSuccess) return hip_status(e, "zero_many");
	}
	return NNH_OK;
}

int nnh_tensor_sum0(const float* src, size_t rows, size_t inner, float* dst, int combine, void* stream) {
	if (inner == 0) return NNH_OK;
	if (!dst || (rows > 0 && !src)) return fail(NNH_ERR_INVALID, "null pointer");
	if (combine < 0 || combine > 2) return fail(NNH_ERR_INVALID, "combine must be 0, 1 or 2");
	if (!count_ok({rows, inner})) return fail(NNH_ERR_INVALID, "size out of range (above 2^60 elements)");
	if (ranges_overlap(dst, inner * 4, src, (uint64_t)rows * inner * 4)) return fail(NNH_ERR_ALIAS, "dst overlaps src");
	return hip_status(sum_rows(src, (int64_t)rows, (int64_t)inner, dst, combine, reinterpret_cast<hipStream_t>(stream)),
	                  "sum0");
}

}  // extern "C"
