// abi.hip - the extern "C" boundary (include/nnh.h): argument validation, shape logic of the reference's
// op surface, and dispatch to the HIP kernels. Nothing throws across this boundary.
#include "nnh.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "abi_common.hpp"
#include "kernels/hip/gemm.hpp"
#include "workspace.hpp"

namespace nnh {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
	g_last_error = msg;
	return code;
}

int hip_status(hipError_t e, const char* what) {
	if (e == hipSuccess) return NNH_OK;
	return fail(NNH_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

bool ranges_overlap(const void* p0, uint64_t bytes0, const void* p1, uint64_t bytes1) {
	if (!p0 || !p1 || bytes0 == 0 || bytes1 == 0) return false;
	const uintptr_t a0 = reinterpret_cast<uintptr_t>(p0), a1 = reinterpret_cast<uintptr_t>(p1);
	return a0 < a1 + bytes1 && a1 < a0 + bytes0;
}

// Validates one (batched) GEMM in nn::kernels::sgemm's terms and fills g. Returns NNH_OK or an error.
int build_gemm(int ta, int tb, size_t m, size_t n, size_t k, const float* a, size_t lda, const float* b, size_t ldb,
               float* c, size_t ldc, int accumulate, const nnh_batch* batch, const nnh_epilogue* ep, GemmCall& g,
               const ColGather* gather) {
	g = GemmCall{};
	if (gather) {
		if (ta) return fail(NNH_ERR_INVALID, "a gathered B needs an untransposed A");
		g.gather = true;
		g.col = *gather;
	}
	const size_t kIntMax = INT_MAX;
	if (m > kIntMax || n > kIntMax || k > kIntMax) return fail(NNH_ERR_INVALID, "m, n and k must be below 2^31");
	if (lda > kMaxElems || ldb > kMaxElems || ldc > kMaxElems)
		return fail(NNH_ERR_INVALID, "leading dimension out of range (above 2^60)");
	g.ta = ta ? 1 : 0;
	g.tb = tb ? 1 : 0;
	g.m = (int64_t)m;
	g.n = (int64_t)n;
	g.k = (int64_t)k;
	g.a = a;
	g.b = b;
	g.c = c;
	g.lda = (int64_t)lda;
	g.ldb = (int64_t)ldb;
	g.ldc = (int64_t)ldc;
	g.accumulate = accumulate ? 1 : 0;
	// the batch's problem count and the largest offset of each operand's last problem, in elements
	uint64_t count = 1, max_oa = 0, max_ob = 0, max_oc = 0;
	if (batch) {
		if (batch->ndim < 0 || batch->ndim > NNH_MAX_BATCH_DIMS) return fail(NNH_ERR_INVALID, "batch ndim must be 0..4");
		g.batch.ndim = batch->ndim;
		for (int d = 0; d < batch->ndim; ++d) {
			if (batch->shape[d] > kIntMax) return fail(NNH_ERR_INVALID, "batch dimension too large");
			if (batch->stride_a[d] < 0 || batch->stride_b[d] < 0 || batch->stride_c[d] < 0)
				return fail(NNH_ERR_INVALID, "batch strides must be non-negative");
			const uint64_t span = batch->shape[d] > 0 ? batch->shape[d] - 1 : 0;
			if (!mad_ok(count, batch->shape[d], 0, count) || !mad_ok(span, (uint64_t)batch->stride_a[d], max_oa, max_oa) ||
			    !mad_ok(span, (uint64_t)batch->stride_b[d], max_ob, max_ob) ||
			    !mad_ok(span, (uint64_t)batch->stride_c[d], max_oc, max_oc))
				return fail(NNH_ERR_INVALID, "batch extent out of range (above 2^60 elements)");
			g.batch.shape[d] = (int64_t)batch->shape[d];
			g.batch.sa[d] = batch->stride_a[d];
			g.batch.sb[d] = batch->stride_b[d];
			g.batch.sc[d] = batch->stride_c[d];
		}
	}
	g.batch_count = (int64_t)count;
	if (ep) {
		if (ep->bias_mode < NNH_BIAS_NONE || ep->bias_mode > NNH_BIAS_ROW) return fail(NNH_ERR_INVALID, "bad bias mode");
		if (ep->bias_mode != NNH_BIAS_NONE && !ep->bias) return fail(NNH_ERR_INVALID, "bias is null");
		g.ep.bias_mode = ep->bias_mode;
		g.ep.relu = ep->relu ? 1 : 0;
		g.ep.bias = ep->bias;
		g.ep.alive = ep->relu ? ep->alive : nullptr;
	}
	if (m == 0 || n == 0 || count == 0) return NNH_OK;  // nothing is touched (gemm.cpp:344)
	if (!c) return fail(NNH_ERR_INVALID, "C is null");
	if (ldc < n) return fail(NNH_ERR_INVALID, "ldc < n");
	uint64_t c_elems = 0;
	if (!mad_ok(m - 1, ldc, max_oc + n, c_elems)) return fail(NNH_ERR_INVALID, "C's extent out of range");
	const uint64_t c_extent = c_elems * sizeof(float);
	if (k > 0) {
		if (!a || !b) return fail(NNH_ERR_INVALID, "A or B is null");
		const size_t a_rows = ta ? k : m, a_cols = ta ? m : k;
		const size_t b_rows = tb ? n : k, b_cols = tb ? k : n;
		if (lda < a_cols) return fail(NNH_ERR_INVALID, "lda smaller than the stored row length of A");
		if (!gather && ldb < b_cols) return fail(NNH_ERR_INVALID, "ldb smaller than the stored row length of B");
		uint64_t a_elems = 0, b_elems = 0;
		const bool b_ok = gather ? mad_ok((uint64_t)gather->cin * (uint64_t)gather->h, (uint64_t)gather->w, max_ob, b_elems)
		                         : mad_ok(b_rows - 1, ldb, max_ob + b_cols, b_elems);
		if (!mad_ok(a_rows - 1, lda, max_oa + a_cols, a_elems) || !b_ok)
			return fail(NNH_ERR_INVALID, "A's or B's extent out of range");
		if (ranges_overlap(c, c_extent, a, a_elems * 4) || ranges_overlap(c, c_extent, b, b_elems * 4))
			return fail(NNH_ERR_ALIAS, "C overlaps A or B");
	}
	if (g.ep.bias_mode != kBiasNone) {
		const uint64_t bias_bytes = (uint64_t)(g.ep.bias_mode == kBiasCol ? n : m) * 4;
		if (ranges_overlap(c, c_extent, g.ep.bias, bias_bytes)) return fail(NNH_ERR_ALIAS, "C overlaps the bias");
	}
	return NNH_OK;
}

int run_gemm(const GemmCall& g, void* stream, int config, float* workspace) {
	if (g.m == 0 || g.n == 0 || g.batch_count == 0) return NNH_OK;
	if (!workspace) {
		const int rc = check_workspace(stream, gemm_workspace_bytes(g));
		if (rc != NNH_OK) return rc;
	}
	return hip_status(gemm_launch(g, reinterpret_cast<hipStream_t>(stream), config, workspace), "sgemm launch");
}

int check_workspace(void* stream, size_t bytes) {
	if (bytes == 0) return NNH_OK;
	bool external = false;
	size_t have = 0;
	const int rc = hip_status(stream_workspace_external(reinterpret_cast<hipStream_t>(stream), external, have),
	                          "workspace lookup");
	if (rc != NNH_OK) return rc;
	if (external && have < bytes)
		return fail(NNH_ERR_WORKSPACE, "the stream's workspace holds " + std::to_string(have) + " bytes; this call needs " +
		                                   std::to_string(bytes));
	return NNH_OK;
}

int put_bytes(size_t* out, size_t bytes) {
	if (!out) return fail(NNH_ERR_INVALID, "bytes is null");
	*out = bytes;
	return NNH_OK;
}

}  // namespace nnh

using namespace nnh;

extern "C" {

const char* nnh_last_error(void) { return g_last_error.c_str(); }

const char* nnh_version(void) { return "nnh 0.1.0 (gfx950 fp32 MFMA, bit-exact with nn-cpp 2.0.0 NN_NATIVE)"; }

int nnh_sgemm(int trans_a, int trans_b, size_t m, size_t n, size_t k, const float* a, size_t lda, const float* b,
              size_t ldb, float* c, size_t ldc, int accumulate, void* stream) {
	NumericsScope numerics_scope(stream);
	GemmCall g;
	int rc = build_gemm(trans_a, trans_b, m, n, k, a, lda, b, ldb, c, ldc, accumulate, nullptr, nullptr, g);
	if (rc != NNH_OK) return rc;
	return run_gemm(g, stream, -1);
}

int nnh_sgemm_batched(int trans_a, int trans_b, size_t m, size_t n, size_t k, const float* a, size_t lda,
                      const float* b, size_t ldb, float* c, size_t ldc, int accumulate, const nnh_batch* batch,
                      const nnh_epilogue* epilogue, void* stream) {
	return nnh_sgemm_config(trans_a, trans_b, m, n, k, a, lda, b, ldb, c, ldc, accumulate, batch, epilogue, -1,
	                        stream);
}

int nnh_sgemm_config(int trans_a, int trans_b, size_t m, size_t n, size_t k, const float* a, size_t lda,
                     const float* b, size_t ldb, float* c, size_t ldc, int accumulate, const nnh_batch* batch,
                     const nnh_epilogue* epilogue, int config, void* stream) {
	NumericsScope numerics_scope(stream);
	GemmCall g;
	int rc = build_gemm(trans_a, trans_b, m, n, k, a, lda, b, ldb, c, ldc, accumulate, batch, epilogue, g);
	if (rc != NNH_OK) return rc;
	if (config < -1 || config >= gemm_config_count()) return fail(NNH_ERR_INVALID, "no such kernel configuration");
	return run_gemm(g, stream, config);
}

int nnh_set_workspace(void* stream, void* workspace, size_t bytes) {
	if (bytes > 0 && !workspace) return fail(NNH_ERR_INVALID, "workspace is null");
	return hip_status(set_stream_workspace(reinterpret_cast<hipStream_t>(stream), workspace, bytes), "set workspace");
}

int nnh_sgemm_workspace_size(size_t m, size_t n, size_t k, size_t batch_count, size_t* bytes) {
	return query_both_modes(bytes, [&](size_t* bytes) {
		return put_bytes(bytes, gemm_workspace_bytes(m, n, k, batch_count));
	});
}

int nnh_matmul_workspace_size(const size_t* a_shape, int a_ndim, const size_t* b_shape, int b_ndim, int trans_a,
                              int trans_b, size_t* bytes) {
	return query_both_modes(bytes, [&](size_t* bytes) {
		MatmulPlan plan;
		const int rc = plan_matmul(a_shape, a_ndim, b_shape, b_ndim, trans_a, trans_b, plan);
		if (rc != NNH_OK) return rc;
		size_t count = 1;
		for (int d = 0; d < plan.batch.ndim; ++d) count *= plan.batch.shape[d];
		return put_bytes(bytes, gemm_workspace_bytes(plan.m, plan.n, plan.k, count));
	});
}

int nnh_set_numerics(int mode) {
	if (mode != NNH_NUMERICS_NNCPP && mode != NNH_NUMERICS_SPLIT_DEPTH) return fail(NNH_ERR_INVALID, "no such numerics mode");
	set_numerics(mode);
	return NNH_OK;
}

int nnh_get_numerics(void) { return default_numerics(); }

int nnh_set_stream_numerics(void* stream, int mode) {
	if (mode != NNH_NUMERICS_DEFAULT && mode != NNH_NUMERICS_NNCPP && mode != NNH_NUMERICS_SPLIT_DEPTH)
		return fail(NNH_ERR_INVALID, "no such numerics mode");
	set_stream_numerics(stream, mode);
	return NNH_OK;
}

int nnh_get_stream_numerics(void* stream) { return stream_numerics(stream); }

int nnh_gemm_config_count(void) { return gemm_config_count(); }

const char* nnh_gemm_config_name(int config) { return gemm_config_name(config); }

int nnh_matmul_shape(const size_t* a_shape, int a_ndim, const size_t* b_shape, int b_ndim, int trans_a, int trans_b,
                     size_t* out_shape, int* out_ndim) {
	MatmulPlan plan;
	int rc = plan_matmul(a_shape, a_ndim, b_shape, b_ndim, trans_a, trans_b, plan);
	if (rc != NNH_OK) return rc;
	if (!out_shape || !out_ndim) return fail(NNH_ERR_INVALID, "out_shape or out_ndim is null");
	*out_ndim = (int)plan.out_shape.size();
	for (size_t i = 0; i < plan.out_shape.size(); ++i) out_shape[i] = plan.out_shape[i];
	return NNH_OK;
}

int nnh_matmul(const float* a, const size_t* a_shape, int a_ndim, const float* b, const size_t* b_shape, int b_ndim,
               int trans_a, int trans_b, float* out, void* stream) {
	NumericsScope numerics_scope(stream);
	MatmulPlan plan;
	int rc = plan_matmul(a_shape, a_ndim, b_shape, b_ndim, trans_a, trans_b, plan);
	if (rc != NNH_OK) return rc;
	GemmCall g;
	rc = build_gemm(plan.fold ? 0 : trans_a, trans_b, plan.m, plan.n, plan.k, a, plan.lda, b, plan.ldb, out, plan.n, 0,
	                plan.batch.ndim ? &plan.batch : nullptr, nullptr, g);
	if (rc != NNH_OK) return rc;
	return run_gemm(g, stream, -1);
}

}  // extern "C"
