// abi_common.hpp - host-side helpers shared by the C ABI translation units: error reporting and the
// shape logic of nn::matmul.
#pragma once

#include <cstdint>
#include <initializer_list>
#include <string>
#include <vector>

#include "kernels/hip/gemm.hpp"
#include "nnh.h"

namespace nnh {

// Element counts, offsets and leading dimensions above 2^60 are refused at this boundary (NNH_ERR_INVALID): no
// device holds that many floats, and below the limit every byte count and signed offset computed from them fits
// in 64 bits.
constexpr uint64_t kMaxElems = (uint64_t)1 << 60;

// out = a * b + c, when that is at most kMaxElems.
inline bool mad_ok(uint64_t a, uint64_t b, uint64_t c, uint64_t& out) {
	const unsigned __int128 r = (unsigned __int128)a * b + c;
	if (r > kMaxElems) return false;
	out = (uint64_t)r;
	return true;
}

// The product of n sizes (1 for n = 0, 0 when one of them is 0), when the product of the nonzero ones is at most
// kMaxElems: then every partial product, strides included, is too.
inline bool count_ok(const size_t* dims, int n, uint64_t& out) {
	uint64_t p = 1;
	bool empty = false;
	for (int i = 0; i < n; ++i) {
		if (dims[i] == 0) empty = true;
		else if (!mad_ok(p, dims[i], 0, p)) return false;
	}
	out = empty ? 0 : p;
	return true;
}

inline bool count_ok(std::initializer_list<size_t> dims, uint64_t& out) {
	return count_ok(dims.begin(), (int)dims.size(), out);
}
inline bool count_ok(std::initializer_list<size_t> dims) {
	uint64_t c = 0;
	return count_ok(dims, c);
}

extern thread_local std::string g_last_error;
int fail(int code, const std::string& msg);
int hip_status(hipError_t e, const char* what);
bool ranges_overlap(const void* p0, uint64_t bytes0, const void* p1, uint64_t bytes1);
// Overlap other than the same range twice (an op that goes element by element may write in place).
inline bool partial_overlap(const void* p0, uint64_t bytes0, const void* p1, uint64_t bytes1) {
	return !(p0 == p1 && bytes0 == bytes1) && ranges_overlap(p0, bytes0, p1, bytes1);
}
// gather: B is each sample's im2col columns read from the convolution input b (then ldb is unused and B's
// extent is one sample's input per batch step); null for an ordinary B.
int build_gemm(int ta, int tb, size_t m, size_t n, size_t k, const float* a, size_t lda, const float* b, size_t ldb,
               float* c, size_t ldc, int accumulate, const nnh_batch* batch, const nnh_epilogue* ep, GemmCall& g,
               const ColGather* gather = nullptr);
// workspace: depth-cut partials (at least gemm_workspace_floats(g)), required when the caller holds the
// stream's StreamWorkspace; otherwise null (the partials then come from the stream's workspace, checked first).
int run_gemm(const GemmCall& g, void* stream, int config, float* workspace = nullptr);
// Bytes of stream workspace g's depth-cut partials take (0 without a depth cut).
inline size_t gemm_workspace_bytes(const GemmCall& g) { return (size_t)gemm_workspace_floats(g) * sizeof(float); }
inline size_t gemm_workspace_bytes(size_t m, size_t n, size_t k, size_t batch_count, bool gather = false) {
	return (size_t)gemm_workspace_floats((int64_t)m, (int64_t)n, (int64_t)k, (int64_t)batch_count, gather) * sizeof(float);
}
// NNH_ERR_WORKSPACE when the caller registered a workspace for the stream that holds fewer than `bytes`;
// called by every entry point before it launches anything.
int check_workspace(void* stream, size_t bytes);
// maxpool2d's checks of ops.cpp:1610-1627 on one (H, W) plane, and its output plane (ho, wo).
int maxpool_geometry(size_t H, size_t W, size_t kernel, size_t stride, size_t& ho, size_t& wo);
// Stores a workspace query's answer.
int put_bytes(size_t* out, size_t bytes);
// A workspace query answers for both numerics modes, the larger of the two: the stream a caller sizes a workspace
// for may run either mode. f(size_t* bytes) is the query in the current mode.
template <class F>
int query_both_modes(size_t* bytes, F&& f) {
	size_t b[2] = {0, 0};
	const int modes[2] = {kNumericsNnCpp, kNumericsSplitDepth};
	for (int i = 0; i < 2; ++i) {
		NumericsScope scope(modes[i], true);
		const int rc = f(&b[i]);
		if (rc != NNH_OK) return rc;
	}
	return put_bytes(bytes, b[0] > b[1] ? b[0] : b[1]);
}

// How nn::matmul(a, b, trans_a, trans_b) (src/tensor.cpp:571-641) maps onto one (batched) GEMM.
struct MatmulPlan {
	bool fold = false;              // 3-D+ a times 2-D b, a folded into M rows (tensor.cpp:587-596)
	size_t m = 0, n = 0, k = 0, lda = 0, ldb = 0;
	std::vector<size_t> out_shape;
	nnh_batch batch{};              // output batch dims (coalesced to at most NNH_MAX_BATCH_DIMS)
};

inline int plan_matmul(const size_t* as, int an, const size_t* bs, int bn, int ta, int tb, MatmulPlan& p) {
	p = MatmulPlan{};
	if (an < 0 || bn < 0 || (an > 0 && !as) || (bn > 0 && !bs)) return fail(NNH_ERR_INVALID, "bad shape arrays");
	if (an < 2 || bn < 2) return fail(NNH_ERR_SHAPE, "matmul needs operands of rank 2 or more");
	uint64_t a_count = 0, b_count = 0;
	if (!count_ok(as, an, a_count) || !count_ok(bs, bn, b_count))
		return fail(NNH_ERR_INVALID, "operand size out of range (above 2^60 elements)");
	const size_t a_rows = as[an - 2], a_cols = as[an - 1], b_rows = bs[bn - 2], b_cols = bs[bn - 1];
	const size_t m = ta ? a_cols : a_rows, k = ta ? a_rows : a_cols;
	const size_t k2 = tb ? b_cols : b_rows, n = tb ? b_rows : b_cols;
	if (k != k2) return fail(NNH_ERR_SHAPE, "matmul inner dimensions differ");
	p.n = n;
	p.k = k;
	p.lda = a_cols;
	p.ldb = b_cols;
	if (bn == 2 && !ta && an > 2) {
		p.fold = true;
		size_t rows = 1;
		for (int d = 0; d < an - 1; ++d) rows *= as[d];
		p.m = rows;
		p.out_shape.assign(as, as + an - 1);
		p.out_shape.push_back(n);
		return NNH_OK;
	}
	p.m = m;
	uint64_t out_count = 0;
	if (!mad_ok(m, n, 0, out_count)) return fail(NNH_ERR_INVALID, "output size out of range (above 2^60 elements)");
	// broadcast the leading axes (tensor.cpp:121-136), right-aligned
	const int ra = an - 2, rb = bn - 2, rank = ra > rb ? ra : rb;
	std::vector<size_t> shape(rank);
	std::vector<int64_t> sa(rank, 0), sb(rank, 0), sc(rank, 0);
	std::vector<int64_t> astr(an), bstr(bn);
	{
		int64_t s = 1;
		for (int d = an - 1; d >= 0; --d) { astr[d] = s; s *= (int64_t)as[d]; }
		s = 1;
		for (int d = bn - 1; d >= 0; --d) { bstr[d] = s; s *= (int64_t)bs[d]; }
	}
	for (int i = 0; i < rank; ++i) {
		const int ia = i - (rank - ra), ib = i - (rank - rb);
		const size_t ad = ia < 0 ? 1 : as[ia], bd = ib < 0 ? 1 : bs[ib];
		if (ad == bd || bd == 1) shape[i] = ad;
		else if (ad == 1) shape[i] = bd;
		else return fail(NNH_ERR_SHAPE, "matmul batch dimensions do not broadcast");
		// broadcast_offset (tensor.cpp:138-148): a source axis of size 1 contributes nothing
		sa[i] = (ia >= 0 && as[ia] != 1) ? astr[ia] : 0;
		sb[i] = (ib >= 0 && bs[ib] != 1) ? bstr[ib] : 0;
		if (shape[i] != 0 && !mad_ok(out_count, shape[i], 0, out_count))
			return fail(NNH_ERR_INVALID, "output size out of range (above 2^60 elements)");
	}
	{
		int64_t s = (int64_t)(m * n);
		for (int i = rank - 1; i >= 0; --i) { sc[i] = s; s *= (int64_t)shape[i]; }
	}
	p.out_shape = shape;
	p.out_shape.push_back(m);
	p.out_shape.push_back(n);
	// drop size-1 axes and merge axes that are contiguous for A, B and C alike
	std::vector<size_t> cs;
	std::vector<int64_t> ca, cb, cc;
	for (int i = 0; i < rank; ++i) {
		if (shape[i] == 1) continue;
		if (!cs.empty()) {
			const size_t last = cs.size() - 1;
			if (ca[last] == sa[i] * (int64_t)shape[i] && cb[last] == sb[i] * (int64_t)shape[i] &&
			    cc[last] == sc[i] * (int64_t)shape[i]) {
				cs[last] *= shape[i];
				ca[last] = sa[i];
				cb[last] = sb[i];
				cc[last] = sc[i];
				continue;
			}
		}
		cs.push_back(shape[i]);
		ca.push_back(sa[i]);
		cb.push_back(sb[i]);
		cc.push_back(sc[i]);
	}
	if (cs.size() > NNH_MAX_BATCH_DIMS) return fail(NNH_ERR_INVALID, "more than 4 non-mergeable batch axes");
	p.batch.ndim = (int)cs.size();
	for (size_t d = 0; d < cs.size(); ++d) {
		p.batch.shape[d] = cs[d];
		p.batch.stride_a[d] = ca[d];
		p.batch.stride_b[d] = cb[d];
		p.batch.stride_c[d] = cc[d];
	}
	// an empty batch axis means no matrices at all
	for (int i = 0; i < rank; ++i)
		if (shape[i] == 0) {
			p.batch.ndim = 1;
			p.batch.shape[0] = 0;
			p.batch.stride_a[0] = p.batch.stride_b[0] = p.batch.stride_c[0] = 0;
		}
	return NNH_OK;
}

}  // namespace nnh
