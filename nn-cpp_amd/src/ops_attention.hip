// ops_attention.hip - extern "C" entry points of nn::attention and nn::scaled_masked_softmax (include/nnh.h).
//
// Forward (src/autograd/ops.cpp:1226-1261): for heads of width 64 and Tk <= 256, one fused kernel per 64 query
// rows (kernels/hip/attention.hip). Otherwise three launches over all (sample, head) pairs at once:
//   probs = Q_h K_h^T   (batched sgemm F,T with two-level batch addressing n*T*D + h*Dh, row stride D)
//   probs = masked_softmax_row(probs) per row
//   out_h = probs V_h   (batched sgemm F,F into column block h*Dh, row stride D)
// Backward (ops.cpp:1263-1295): dP = G_h V_h^T, dV (+)= P^T G_h, dS = softmax backward, dQ (+)= dS K_h,
// dK (+)= dS^T Q_h; for the fused forward's shapes dP and dS come from one kernel (dP never leaves the chip). Heads write disjoint column blocks, so batching the heads keeps, for every element, the
// reference's order of contributions (dV, then dQ, then dK, which matters when q, k and v are one node).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "abi_common.hpp"
#include "kernels/hip/attention.hpp"
#include "kernels/hip/gemm.hpp"
#include "kernels/hip/softmax.hpp"
#include "workspace.hpp"
#include "nnh.h"

using namespace nnh;

namespace {

struct AttnGeom {
	size_t N, Tq, Tk, D, H, Dh;
	float scale;
};

int check_attention(size_t N, size_t Tq, size_t Tk, size_t D, size_t heads, int causal, AttnGeom& a) {
	// ops.cpp:1228-1236
	if (heads == 0 || D % heads != 0 || Tq == 0 || Tk == 0 || (causal && Tq != Tk))
		return fail(NNH_ERR_SHAPE, "attention: heads must divide D, sequences non-empty, causal needs Tq == Tk");
	const size_t lim = (size_t)1 << 31;
	if (Tq >= lim || Tk >= lim || D >= lim || !count_ok({N, Tq, D}) || !count_ok({N, Tk, D}) ||
	    !count_ok({N, heads, Tq, Tk}))
		return fail(NNH_ERR_INVALID, "attention: size out of range");
	a = AttnGeom{N, Tq, Tk, D, heads, D / heads, 1.0f / std::sqrt(static_cast<float>(D / heads))};
	if ((int64_t)Tk > softmax_max_row_length())
		return fail(NNH_ERR_INVALID, "attention: key length beyond the row softmax's LDS capacity");
	return NNH_OK;
}

// (sample, head) batch over {N, T, D} operands: head h of sample n starts at n*T*D + h*Dh
nnh_batch head_batch(const AttnGeom& a, size_t ta_rows, size_t tb_rows, bool a_is_probs, bool c_is_probs,
                     size_t tc_rows) {
	nnh_batch b{};
	b.ndim = 2;
	b.shape[0] = a.N;
	b.shape[1] = a.H;
	const ptrdiff_t pp = (ptrdiff_t)(a.Tq * a.Tk);
	b.stride_a[0] = a_is_probs ? (ptrdiff_t)a.H * pp : (ptrdiff_t)(ta_rows * a.D);
	b.stride_a[1] = a_is_probs ? pp : (ptrdiff_t)a.Dh;
	b.stride_b[0] = (ptrdiff_t)(tb_rows * a.D);
	b.stride_b[1] = (ptrdiff_t)a.Dh;
	b.stride_c[0] = c_is_probs ? (ptrdiff_t)a.H * pp : (ptrdiff_t)(tc_rows * a.D);
	b.stride_c[1] = c_is_probs ? pp : (ptrdiff_t)a.Dh;
	return b;
}

int gemm(int ta, int tb, size_t m, size_t n, size_t k, const float* A, size_t lda, const float* B, size_t ldb,
         float* Cm, size_t ldc, int acc, const nnh_batch& batch, void* stream, float* partials = nullptr) {
	GemmCall g;
	int rc = build_gemm(ta, tb, m, n, k, A, lda, B, ldb, Cm, ldc, acc, &batch, nullptr, g);
	if (rc != NNH_OK) return rc;
	return run_gemm(g, stream, -1, partials);
}

// Two products that write apart from each other and from what the other reads, in one launch where the pair
// kernels take them (gemm_launch_pair), else in turn.
int gemm2(int ta0, int tb0, size_t m0, size_t n0, size_t k0, const float* A0, size_t lda0, const float* B0, size_t ldb0,
          float* C0, size_t ldc0, int acc0, const nnh_batch& batch0, int ta1, int tb1, size_t m1, size_t n1, size_t k1,
          const float* A1, size_t lda1, const float* B1, size_t ldb1, float* C1, size_t ldc1, int acc1,
          const nnh_batch& batch1, void* stream, float* partials) {
	GemmCall g0, g1;
	int rc = build_gemm(ta0, tb0, m0, n0, k0, A0, lda0, B0, ldb0, C0, ldc0, acc0, &batch0, nullptr, g0);
	if (rc == NNH_OK) rc = build_gemm(ta1, tb1, m1, n1, k1, A1, lda1, B1, ldb1, C1, ldc1, acc1, &batch1, nullptr, g1);
	if (rc != NNH_OK) return rc;
	bool paired = false;
	rc = hip_status(gemm_launch_pair(g0, g1, reinterpret_cast<hipStream_t>(stream), paired), "attention backward");
	if (rc != NNH_OK || paired) return rc;
	rc = run_gemm(g0, stream, -1, partials);
	if (rc == NNH_OK) rc = run_gemm(g1, stream, -1, partials);
	return rc;
}

// One workspace for nnh_attention_backward: dS, then the depth-cut partials the dV, dQ and dK products share
// (they run in turn).
struct BwdPlan {
	size_t total = 0, off_ds = 0, off_part = 0;
	int64_t part = 0;
};

BwdPlan attention_backward_plan(const AttnGeom& a) {
	BwdPlan p;
	if (a.N == 0) return p;
	WorkspacePlan plan;
	p.off_ds = plan.add(a.N * a.H * a.Tq * a.Tk * sizeof(float));
	const int64_t nb = (int64_t)(a.N * a.H);
	p.part = std::max({gemm_workspace_floats((int64_t)a.Tk, (int64_t)a.Dh, (int64_t)a.Tq, nb),
	                   gemm_workspace_floats((int64_t)a.Tq, (int64_t)a.Dh, (int64_t)a.Tk, nb),
	                   gemm_workspace_floats((int64_t)a.Tq, (int64_t)a.Tk, (int64_t)a.Dh, nb)});
	p.off_part = p.part ? plan.add((size_t)p.part * sizeof(float)) : 0;
	p.total = plan.total;
	return p;
}

// Scratch of nnh_attention_forward: the depth-cut partials of the S and O products where the three-launch path
// may run (the fused kernel needs none).
size_t attention_forward_ws(const AttnGeom& a) {
	if (a.N == 0) return 0;
	const size_t nb = a.N * a.H;
	return std::max(gemm_workspace_bytes(a.Tq, a.Tk, a.Dh, nb), gemm_workspace_bytes(a.Tq, a.Dh, a.Tk, nb));
}

}  // namespace

extern "C" {

int nnh_attention_forward_workspace_size(size_t N, size_t Tq, size_t Tk, size_t D, size_t heads, size_t* bytes) {
	return query_both_modes(bytes, [&](size_t* bytes) {
		AttnGeom a;
		const int rc = check_attention(N, Tq, Tk, D, heads, 0, a);
		if (rc != NNH_OK) return rc;
		return put_bytes(bytes, attention_forward_ws(a));
	});
}

int nnh_attention_backward_workspace_size(size_t N, size_t Tq, size_t Tk, size_t D, size_t heads, size_t* bytes) {
	return query_both_modes(bytes, [&](size_t* bytes) {
		AttnGeom a;
		const int rc = check_attention(N, Tq, Tk, D, heads, 0, a);
		if (rc != NNH_OK) return rc;
		return put_bytes(bytes, attention_backward_plan(a).total);
	});
}

int nnh_attention_forward(const float* q, const float* k, const float* v, size_t N, size_t Tq, size_t Tk, size_t D,
                          size_t heads, const float* key_padding_mask, int causal, float* out, float* probs,
                          void* stream) {
	NumericsScope numerics_scope(stream);
	AttnGeom a;
	int rc = check_attention(N, Tq, Tk, D, heads, causal, a);
	if (rc != NNH_OK) return rc;
	if (N == 0) return NNH_OK;
	if (!q || !k || !v || !out || !probs) return fail(NNH_ERR_INVALID, "attention: null pointer");
	{
		const uint64_t qb = (uint64_t)N * Tq * D * 4, kb = (uint64_t)N * Tk * D * 4, pb = (uint64_t)N * heads * Tq * Tk * 4;
		const uint64_t mb = (uint64_t)N * Tk * 4;
		const void* ins[4] = {q, k, v, key_padding_mask};
		const uint64_t in_bytes[4] = {qb, kb, kb, mb};
		for (int i = 0; i < 4; ++i)
			if (ranges_overlap(out, qb, ins[i], in_bytes[i]) || ranges_overlap(probs, pb, ins[i], in_bytes[i]))
				return fail(NNH_ERR_ALIAS, "attention: an output overlaps an input");
		if (ranges_overlap(out, qb, probs, pb)) return fail(NNH_ERR_ALIAS, "attention: out overlaps probs");
	}
	hipStream_t s = reinterpret_cast<hipStream_t>(stream);
	const bool fused_fwd = attention_fused_ok((int64_t)Tq, (int64_t)Tk, (int64_t)a.Dh, (int64_t)D, q, k, v, out, probs,
	                                          key_padding_mask);
	if (!fused_fwd) {
		rc = check_workspace(stream, attention_forward_ws(a));
		if (rc != NNH_OK) return rc;
	}
	if (attention_fused_ok((int64_t)Tq, (int64_t)Tk, (int64_t)a.Dh, (int64_t)D, q, k, v, out, probs, key_padding_mask))
		return hip_status(attention_fused_forward(q, k, v, (int64_t)N, (int64_t)Tq, (int64_t)Tk, (int64_t)D,
		                                          (int64_t)heads, key_padding_mask, causal, a.scale, out, probs, s),
		                  "attention forward");
	// S = Q_h K_h^T into probs (ops.cpp:1256)
	rc = gemm(0, 1, Tq, Tk, a.Dh, q, D, k, D, probs, Tk, 0, head_batch(a, Tq, Tk, false, true, 0), stream);
	if (rc != NNH_OK) return rc;
	rc = hip_status(softmax_rows(probs, probs, (int64_t)(N * heads * Tq), (int)Tk, (int)Tq, (int)heads, a.scale,
	                             key_padding_mask, causal, s),
	                "attention softmax");
	if (rc != NNH_OK) return rc;
	// O_h = P V_h into column block h (ops.cpp:1259)
	nnh_batch bo = head_batch(a, 0, Tk, true, false, Tq);
	return gemm(0, 0, Tq, a.Dh, Tk, probs, Tk, v, D, out, D, 0, bo, stream);
}

int nnh_attention_backward(const float* g, const float* q, const float* k, const float* v, const float* probs,
                           size_t N, size_t Tq, size_t Tk, size_t D, size_t heads, const float* key_padding_mask,
                           int causal, float* dq, int dq_first, float* dk, int dk_first, float* dv, int dv_first,
                           void* stream) {
	NumericsScope numerics_scope(stream);
	AttnGeom a;
	int rc = check_attention(N, Tq, Tk, D, heads, causal, a);
	if (rc != NNH_OK) return rc;
	if (N == 0 || (!dq && !dk && !dv)) return NNH_OK;
	if (!g || !q || !k || !v || !probs) return fail(NNH_ERR_INVALID, "attention backward: null pointer");
	{
		// dq, dk and dv may be one buffer (q, k and v one node); none may overlap an input
		const uint64_t qb = (uint64_t)N * Tq * D * 4, kb = (uint64_t)N * Tk * D * 4, pb = (uint64_t)N * heads * Tq * Tk * 4;
		const uint64_t mb = (uint64_t)N * Tk * 4;
		const void* ins[6] = {g, q, k, v, probs, key_padding_mask};
		const uint64_t in_bytes[6] = {qb, qb, kb, kb, pb, mb};
		const void* outs[3] = {dq, dk, dv};
		const uint64_t out_bytes[3] = {qb, kb, kb};
		for (int o = 0; o < 3; ++o)
			for (int i = 0; i < 6; ++i)
				if (ranges_overlap(outs[o], out_bytes[o], ins[i], in_bytes[i]))
					return fail(NNH_ERR_ALIAS, "attention backward: a gradient overlaps an input");
	}
	hipStream_t s = reinterpret_cast<hipStream_t>(stream);
	const BwdPlan plan = attention_backward_plan(a);
	rc = check_workspace(stream, plan.total);
	if (rc != NNH_OK) return rc;
	StreamWorkspace ws(s, plan.total);
	if (ws.error() != hipSuccess) return hip_status(ws.error(), "attention workspace");
	float* ds = ws.at<float>(plan.off_ds);
	float* partials = plan.part ? ws.at<float>(plan.off_part) : nullptr;
	const bool fused = (dq || dk) && attention_fused_ok((int64_t)Tq, (int64_t)Tk, (int64_t)a.Dh, (int64_t)D, g, v, v, ds,
	                                                    probs, key_padding_mask);
	const uint64_t qb = (uint64_t)N * Tq * D * 4, kb = (uint64_t)N * Tk * D * 4, sb = (uint64_t)N * heads * Tq * Tk * 4;
	if (!fused && (dq || dk) && dv && !ranges_overlap(dv, kb, ds, sb)) {
		// dP = G_h V_h^T (ops.cpp:1286) and dV (+)= P^T G_h (ops.cpp:1287), which reads P, not dP
		rc = gemm2(0, 1, Tq, Tk, a.Dh, g, D, v, D, ds, Tk, 0, head_batch(a, Tq, Tk, false, true, 0), 1, 0, Tk, a.Dh, Tq,
		           probs, Tk, g, D, dv, D, !dv_first, head_batch(a, 0, Tq, true, false, Tk), stream, partials);
	} else {
		if (fused)  // dP = G_h V_h^T and the softmax backward in one kernel (ops.cpp:1286, 1289-1290)
			rc = hip_status(attention_fused_dscores(g, v, probs, (int64_t)N, (int64_t)Tq, (int64_t)Tk, (int64_t)D,
			                                        (int64_t)heads, key_padding_mask, causal, a.scale, ds, s),
			                "attention backward");
		else if (dq || dk)  // dP = G_h V_h^T (ops.cpp:1286)
			rc = gemm(0, 1, Tq, Tk, a.Dh, g, D, v, D, ds, Tk, 0, head_batch(a, Tq, Tk, false, true, 0), stream, partials);
		// dV (+)= P^T G_h (ops.cpp:1287): A = probs stored Tq x Tk, read transposed
		if (rc == NNH_OK && dv) {
			nnh_batch b = head_batch(a, 0, Tq, true, false, Tk);
			rc = gemm(1, 0, Tk, a.Dh, Tq, probs, Tk, g, D, dv, D, !dv_first, b, stream, partials);
		}
	}
	if (rc == NNH_OK && (dq || dk) && !fused)
		rc = hip_status(softmax_backward_rows(probs, ds, ds, (int64_t)(N * heads * Tq), (int)Tk, (int)Tq, (int)heads,
		                                      a.scale, key_padding_mask, causal, 0, s),
		                "attention softmax backward");
	// dQ (+)= dS K_h (ops.cpp:1291) and dK (+)= dS^T Q_h (ops.cpp:1292) in one launch when they are apart
	if (rc == NNH_OK && dq && dk && !ranges_overlap(dq, qb, dk, kb))
		return gemm2(0, 0, Tq, a.Dh, Tk, ds, Tk, k, D, dq, D, !dq_first, head_batch(a, 0, Tk, true, false, Tq), 1, 0, Tk,
		             a.Dh, Tq, ds, Tk, q, D, dk, D, !dk_first, head_batch(a, 0, Tq, true, false, Tk), stream, partials);
	// dQ (+)= dS K_h (ops.cpp:1291)
	if (rc == NNH_OK && dq) {
		nnh_batch b = head_batch(a, 0, Tk, true, false, Tq);
		rc = gemm(0, 0, Tq, a.Dh, Tk, ds, Tk, k, D, dq, D, !dq_first, b, stream, partials);
	}
	// dK (+)= dS^T Q_h (ops.cpp:1292)
	if (rc == NNH_OK && dk) {
		nnh_batch b = head_batch(a, 0, Tq, true, false, Tk);
		rc = gemm(1, 0, Tk, a.Dh, Tq, ds, Tk, q, D, dk, D, !dk_first, b, stream, partials);
	}
	return rc;
}

int nnh_scaled_masked_softmax_forward(const float* x, size_t N, size_t H, size_t Tq, size_t Tk, float scale,
                                      const float* key_padding_mask, int causal, float* y, void* stream) {
	if (Tk == 0) return fail(NNH_ERR_SHAPE, "scaled_masked_softmax: empty rows");  // ops.cpp:1300
	if (N == 0 || H == 0 || Tq == 0) return NNH_OK;
	if (!x || !y) return fail(NNH_ERR_INVALID, "null pointer");
	if ((int64_t)Tk > softmax_max_row_length()) return fail(NNH_ERR_INVALID, "row too long for the row softmax");
	if (Tq >= ((size_t)1 << 31) || H >= ((size_t)1 << 31) || !count_ok({N, H, Tq, Tk}))
		return fail(NNH_ERR_INVALID, "scaled_masked_softmax: size out of range");
	{
		const uint64_t bytes = (uint64_t)N * H * Tq * Tk * 4;
		if (partial_overlap(y, bytes, x, bytes) || ranges_overlap(y, bytes, key_padding_mask, (uint64_t)N * Tk * 4))
			return fail(NNH_ERR_ALIAS, "scaled_masked_softmax: y overlaps x (other than in place) or the mask");
	}
	return hip_status(softmax_rows(x, y, (int64_t)(N * H * Tq), (int)Tk, (int)Tq, (int)H, scale, key_padding_mask,
	                               causal, reinterpret_cast<hipStream_t>(stream)),
	                  "scaled_masked_softmax");
}

int nnh_scaled_masked_softmax_backward(const float* y, const float* g, size_t N, size_t H, size_t Tq, size_t Tk,
                                       float scale, const float* key_padding_mask, int causal, float* dx, int first,
                                       void* stream) {
	if (Tk == 0) return fail(NNH_ERR_SHAPE, "scaled_masked_softmax: empty rows");
	if (N == 0 || H == 0 || Tq == 0) return NNH_OK;
	if (!y || !g || !dx) return fail(NNH_ERR_INVALID, "null pointer");
	if ((int64_t)Tk > softmax_max_row_length()) return fail(NNH_ERR_INVALID, "row too long for the row softmax");
	if (Tq >= ((size_t)1 << 31) || H >= ((size_t)1 << 31) || !count_ok({N, H, Tq, Tk}))
		return fail(NNH_ERR_INVALID, "scaled_masked_softmax backward: size out of range");
	{
		const uint64_t bytes = (uint64_t)N * H * Tq * Tk * 4;
		if (ranges_overlap(dx, bytes, y, bytes) || partial_overlap(dx, bytes, g, bytes) ||
		    ranges_overlap(dx, bytes, key_padding_mask, (uint64_t)N * Tk * 4))
			return fail(NNH_ERR_ALIAS, "scaled_masked_softmax backward: dx overlaps y, the mask or g (other than in place)");
	}
	return hip_status(softmax_backward_rows(y, g, dx, (int64_t)(N * H * Tq), (int)Tk, (int)Tq, (int)H, scale,
	                                        key_padding_mask, causal, first ? 1 : 2,
	                                        reinterpret_cast<hipStream_t>(stream)),
	                  "scaled_masked_softmax backward");
}

}  // extern "C"
