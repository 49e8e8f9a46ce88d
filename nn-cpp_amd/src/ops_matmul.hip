// ops_matmul.hip - extern "C" backward of nn::matmul and nn::matmul_bt (src/autograd/ops.cpp:683-712, 747-773).
//
// Two paths, as in the reference:
//   * b a plain 2-D matrix: a's leading axes fold into M rows and each gradient is one sgemm straight into its
//     buffer with accumulate = !first (ops.cpp:688-701, 751-762).
//   * otherwise: the gradient is a batched Tensor matmul into scratch (grad_a = G B^T or G B, grad_b = A^T G or
//     G^T A), reduced over broadcast axes by sum_to_shape (Tensor::sum(0) while it has more axes than the operand,
//     then Tensor::sum(i) on each axis the operand has as 1; ops.cpp:35-53), and added with add_to_grad's rule
//     (a fresh gradient stores term + 0.0f, ops.cpp:55-99). A fresh gradient of the operand's own shape takes the
//     matmul directly: its fma chains start at +0 and never end at -0, so + 0.0f would leave every bit unchanged.
// dA is computed before dB (a and b may be one node; then the caller passes db_first = 0).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "abi_common.hpp"
#include "kernels/hip/reduce.hpp"
#include "nnh.h"
#include "workspace.hpp"

using namespace nnh;

namespace {

size_t numel(const std::vector<size_t>& s) {
	size_t n = 1;
	for (size_t d : s) n *= d;
	return n;
}

// One operand's gradient on the batched path: the matmul that produces it (ta/tb over the given shapes), the
// shape it has, and the reductions down to the operand's shape.
struct GradPlan {
	bool on = false;
	const float* left = nullptr;
	const float* right = nullptr;
	std::vector<size_t> left_shape, right_shape;
	int ta = 0, tb = 0;
	MatmulPlan mm;
	std::vector<size_t> target;
	bool direct = false;  // fresh gradient, no reduction: the matmul writes the gradient itself
};

struct Plan {
	bool fold = false;
	std::vector<size_t> out_shape;
	GradPlan ga, gb;
	size_t total = 0, off_tmp = 0, off_pp0 = 0, off_pp1 = 0, off_part = 0;
	size_t tmp_floats = 0, pp_floats = 0;
	int64_t part = 0;
};

// The reductions of sum_to_shape (ops.cpp:35-53) for a gradient of shape `from` and an operand of shape `to`:
// each step is (pre, d, post) of one Tensor::sum, applied in turn.
struct SumStep {
	size_t pre, d, post;
};
std::vector<SumStep> sum_steps(std::vector<size_t> cur, const std::vector<size_t>& to) {
	std::vector<SumStep> steps;
	while (cur.size() > to.size()) {
		steps.push_back({1, cur[0], numel(cur) / std::max<size_t>(cur[0], 1)});
		if (cur[0] == 0) steps.back().post = numel(std::vector<size_t>(cur.begin() + 1, cur.end()));
		cur.erase(cur.begin());
	}
	for (size_t i = 0; i < to.size(); ++i) {
		if (to[i] == 1 && cur[i] != 1) {
			size_t pre = 1, post = 1;
			for (size_t j = 0; j < i; ++j) pre *= cur[j];
			for (size_t j = i + 1; j < cur.size(); ++j) post *= cur[j];
			steps.push_back({pre, cur[i], post});
			cur[i] = 1;
		}
	}
	return steps;
}

int plan_backward(const float* g, const float* a, const size_t* as, int an, const float* b, const size_t* bs, int bn,
                  int bt, bool want_a, bool want_b, int a_first, int b_first, Plan& p) {
	MatmulPlan fwd;
	int rc = plan_matmul(as, an, bs, bn, 0, bt, fwd);  // the forward's shape rules (tensor.cpp:572-585)
	if (rc != NNH_OK) return rc;
	p = Plan{};
	p.out_shape = fwd.out_shape;
	const std::vector<size_t> ash(as, as + an), bsh(bs, bs + bn);
	p.fold = bn == 2;  // ops.cpp:688, 751 (a has at least 2 axes: matmul requires it)
	if (p.fold) return NNH_OK;
	auto grad = [&](GradPlan& gp, const float* l, std::vector<size_t> ls, const float* r, std::vector<size_t> rs, int ta,
	                int tb, const std::vector<size_t>& target, int first) -> int {
		gp.on = true;
		gp.left = l;
		gp.right = r;
		gp.left_shape = std::move(ls);
		gp.right_shape = std::move(rs);
		gp.ta = ta;
		gp.tb = tb;
		gp.target = target;
		int rc2 = plan_matmul(gp.left_shape.data(), (int)gp.left_shape.size(), gp.right_shape.data(),
		                      (int)gp.right_shape.size(), ta, tb, gp.mm);
		if (rc2 != NNH_OK) return rc2;
		gp.direct = first && gp.mm.out_shape == target;
		return NNH_OK;
	};
	if (want_a) {  // grad_a = matmul(G, b, F, T) for matmul, matmul(G, b) for matmul_bt (ops.cpp:703-706, 764-767)
		rc = bt ? grad(p.ga, g, p.out_shape, b, bsh, 0, 0, ash, a_first) : grad(p.ga, g, p.out_shape, b, bsh, 0, 1, ash, a_first);
		if (rc != NNH_OK) return rc;
	}
	if (want_b) {  // grad_b = matmul(a, G, T, F) for matmul, matmul(G, a, T, F) for matmul_bt (ops.cpp:707-710, 768-771)
		rc = bt ? grad(p.gb, g, p.out_shape, a, ash, 1, 0, bsh, b_first) : grad(p.gb, a, ash, g, p.out_shape, 1, 0, bsh, b_first);
		if (rc != NNH_OK) return rc;
	}
	for (const GradPlan* gp : {&p.ga, &p.gb}) {
		if (!gp->on) continue;
		size_t count = 1;
		for (int d = 0; d < gp->mm.batch.ndim; ++d) count *= gp->mm.batch.shape[d];
		p.part = std::max<int64_t>(p.part, gemm_workspace_floats((int64_t)gp->mm.m, (int64_t)gp->mm.n, (int64_t)gp->mm.k,
		                                                         (int64_t)count));
		if (gp->direct) continue;
		p.tmp_floats = std::max(p.tmp_floats, numel(gp->mm.out_shape));
		for (const SumStep& st : sum_steps(gp->mm.out_shape, gp->target))
			p.pp_floats = std::max(p.pp_floats, st.pre * st.post);
	}
	WorkspacePlan wp;
	p.off_tmp = p.tmp_floats ? wp.add(p.tmp_floats * 4) : 0;
	p.off_pp0 = p.pp_floats ? wp.add(p.pp_floats * 4) : 0;
	p.off_pp1 = p.pp_floats ? wp.add(p.pp_floats * 4) : 0;
	p.off_part = p.part ? wp.add((size_t)p.part * 4) : 0;
	p.total = wp.total;
	return NNH_OK;
}

// The product of one gradient into out (the gradient itself when direct, else the scratch it is reduced from).
int grad_call(const GradPlan& gp, float* out, GemmCall& call) {
	const MatmulPlan& m = gp.mm;
	return build_gemm(m.fold ? 0 : gp.ta, gp.tb, m.m, m.n, m.k, gp.left, m.lda, gp.right, m.ldb, out, m.n, 0,
	                  m.batch.ndim ? &m.batch : nullptr, nullptr, call);
}

// The two gradients in one launch (gemm_launch_pair) when both go straight into their buffers, those do not overlap,
// and the pair kernels take the products; launched tells whether it did (otherwise nothing was enqueued).
int run_pair(const GemmCall& ca, float* da, uint64_t da_bytes, const GemmCall& cb, float* db, uint64_t db_bytes,
             void* stream, bool& launched) {
	launched = false;
	if (ranges_overlap(da, da_bytes, db, db_bytes)) return NNH_OK;
	return hip_status(gemm_launch_pair(ca, cb, reinterpret_cast<hipStream_t>(stream), launched), "matmul backward");
}

int run_grad(const GradPlan& gp, float* dst, int first, float* tmp, float* pp0, float* pp1, float* part, void* stream) {
	hipStream_t s = reinterpret_cast<hipStream_t>(stream);
	GemmCall call;
	const MatmulPlan& m = gp.mm;
	int rc = grad_call(gp, gp.direct ? dst : tmp, call);
	if (rc != NNH_OK) return rc;
	rc = run_gemm(call, stream, -1, part);
	if (rc != NNH_OK || gp.direct) return rc;
	const float* cur = tmp;
	const std::vector<SumStep> steps = sum_steps(m.out_shape, gp.target);
	if (steps.empty()) return hip_status(add_to_grad(dst, cur, (int64_t)numel(gp.target), first, s), "matmul grad");
	for (size_t i = 0; i < steps.size(); ++i) {
		const SumStep& st = steps[i];
		const bool last = i + 1 == steps.size();
		float* o = last ? dst : (i % 2 == 0 ? pp0 : pp1);
		rc = hip_status(sum_axis(cur, (int64_t)st.pre, (int64_t)st.d, (int64_t)st.post, o, last ? (first ? 1 : 2) : 0, s),
		                "matmul grad reduction");
		if (rc != NNH_OK) return rc;
		cur = o;
	}
	return NNH_OK;
}

}  // namespace

extern "C" {

int nnh_matmul_backward_workspace_size(const size_t* a_shape, int a_ndim, const size_t* b_shape, int b_ndim,
                                       int b_transposed, int want_da, int want_db, size_t* bytes) {
	return query_both_modes(bytes, [&](size_t* bytes) {
		Plan p;
		const int rc = plan_backward(nullptr, nullptr, a_shape, a_ndim, nullptr, b_shape, b_ndim, b_transposed ? 1 : 0,
		                             want_da, want_db, 0, 0, p);
		if (rc != NNH_OK) return rc;
		if (p.fold) {
			const size_t K = b_transposed ? b_shape[1] : b_shape[0], n = b_transposed ? b_shape[0] : b_shape[1];
			size_t M = 1;
			for (int d = 0; d < a_ndim; ++d) M *= a_shape[d];
			M = K ? M / K : 0;
			return put_bytes(bytes, std::max(want_da ? gemm_workspace_bytes(M, K, n, 1) : 0,
			                                 want_db ? (b_transposed ? gemm_workspace_bytes(n, K, M, 1)
			                                                         : gemm_workspace_bytes(K, n, M, 1))
			                                         : 0));
		}
		return put_bytes(bytes, p.total);
	});
}

int nnh_matmul_backward(const float* g, const float* a, const size_t* a_shape, int a_ndim, const float* b,
                        const size_t* b_shape, int b_ndim, int b_transposed, float* da, int da_first, float* db,
                        int db_first, void* stream) {
	NumericsScope numerics_scope(stream);
	const int bt = b_transposed ? 1 : 0;
	Plan p;
	int rc = plan_backward(g, a, a_shape, a_ndim, b, b_shape, b_ndim, bt, da != nullptr, db != nullptr, da_first,
	                       db_first, p);
	if (rc != NNH_OK) return rc;
	if (!da && !db) return NNH_OK;
	{
		// da and db may be one buffer (a and b one node); neither may overlap an input
		const uint64_t ab = numel(std::vector<size_t>(a_shape, a_shape + a_ndim)) * 4;
		const uint64_t bb = numel(std::vector<size_t>(b_shape, b_shape + b_ndim)) * 4;
		const uint64_t gb = numel(p.out_shape) * 4;
		for (const float* o : {da, db}) {
			const uint64_t ob = o == da ? ab : bb;
			if (ranges_overlap(o, ob, g, gb) || ranges_overlap(o, ob, a, ab) || ranges_overlap(o, ob, b, bb))
				return fail(NNH_ERR_ALIAS, "matmul backward: a gradient overlaps an input");
		}
	}
	if (p.fold) {
		// ops.cpp:688-701 (matmul: b is {K, n}) and 751-762 (matmul_bt: b is {n, K}); M = a.size / K
		const size_t K = bt ? b_shape[1] : b_shape[0], n = bt ? b_shape[0] : b_shape[1];
		size_t asz = 1;
		for (int d = 0; d < a_ndim; ++d) asz *= a_shape[d];
		const size_t M = K ? asz / K : 0;
		size_t need = 0;
		nnh_matmul_backward_workspace_size(a_shape, a_ndim, b_shape, b_ndim, bt, da != nullptr, db != nullptr, &need);
		rc = check_workspace(stream, need);
		if (rc != NNH_OK) return rc;
		GemmCall ca, cb;  // both checked before either runs
		if (da) {
			rc = bt ? build_gemm(0, 0, M, K, n, g, n, b, K, da, K, !da_first, nullptr, nullptr, ca)
			        : build_gemm(0, 1, M, K, n, g, n, b, n, da, K, !da_first, nullptr, nullptr, ca);
			if (rc != NNH_OK) return rc;
		}
		if (db) {
			rc = bt ? build_gemm(1, 0, n, K, M, g, n, a, K, db, K, !db_first, nullptr, nullptr, cb)
			        : build_gemm(1, 0, K, n, M, a, K, g, n, db, n, !db_first, nullptr, nullptr, cb);
			if (rc != NNH_OK) return rc;
		}
		bool paired = false;
		if (da && db) {
			rc = run_pair(ca, da, (uint64_t)M * K * 4, cb, db, (uint64_t)K * n * 4, stream, paired);
			if (rc != NNH_OK || paired) return rc;
		}
		if (da) rc = run_gemm(ca, stream, -1);
		if (rc == NNH_OK && db) rc = run_gemm(cb, stream, -1);
		return rc;
	}
	rc = check_workspace(stream, p.total);
	if (rc != NNH_OK) return rc;
	if (p.total == 0) {  // fresh gradients of the operands' own shapes, no depth cut: straight into them
		if (da && db) {
			GemmCall ca, cb;
			rc = grad_call(p.ga, da, ca);
			if (rc == NNH_OK) rc = grad_call(p.gb, db, cb);
			if (rc != NNH_OK) return rc;
			const uint64_t ab = numel(std::vector<size_t>(a_shape, a_shape + a_ndim)) * 4;
			const uint64_t bb = numel(std::vector<size_t>(b_shape, b_shape + b_ndim)) * 4;
			bool paired = false;
			rc = run_pair(ca, da, ab, cb, db, bb, stream, paired);
			if (rc != NNH_OK || paired) return rc;
		}
		if (da) rc = run_grad(p.ga, da, da_first, nullptr, nullptr, nullptr, nullptr, stream);
		if (rc == NNH_OK && db) rc = run_grad(p.gb, db, db_first, nullptr, nullptr, nullptr, nullptr, stream);
		return rc;
	}
	StreamWorkspace ws(reinterpret_cast<hipStream_t>(stream), p.total);
	if (ws.error() != hipSuccess) return hip_status(ws.error(), "matmul backward workspace");
	float* tmp = p.tmp_floats ? ws.at<float>(p.off_tmp) : nullptr;
	float* pp0 = p.pp_floats ? ws.at<float>(p.off_pp0) : nullptr;
	float* pp1 = p.pp_floats ? ws.at<float>(p.off_pp1) : nullptr;
	float* part = p.part ? ws.at<float>(p.off_part) : nullptr;
	if (da) rc = run_grad(p.ga, da, da_first, tmp, pp0, pp1, part, stream);
	if (rc == NNH_OK && db) rc = run_grad(p.gb, db, db_first, tmp, pp0, pp1, part, stream);
	return rc;
}

}  // extern "C"
