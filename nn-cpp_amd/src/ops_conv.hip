// ops_conv.hip - extern "C" entry points of nn::conv2d / nn::conv2d_relu, im2col and col2im (include/nnh.h).
//
// Forward (src/autograd/ops.cpp:1345-1410): a short depth (K = Cin*kh*kw <= kDirectMaxK, a network's first
// layer) runs as a direct convolution fused with bias/ReLU, memory-bound; 3x3, stride 1, padding 1 on small
// planes runs with the padded sample in LDS (conv_fwd3.hip); any other depth is one batched MFMA GEMM
// W[Cout x K] col_n[K x hw] over all samples with the bias/ReLU/alive epilogue, whose B tiles are gathered from x
// (implicit im2col: the column matrix is never stored). All give each output the reference's fma chain over
// k = (c, ph, pw) in order.
// Backward (ops.cpp:1418-1463): g masked by alive; db = per-sample lane_sum, then summed in sample order;
// dW_n = g_n col_n^T, summed in sample order; dcol_n = W^T g_n then col2im in gather form into a zero-filled
// (fresh) or existing dx. For 3x3, stride 1, padding 1 on small planes one kernel takes the mask, the
// per-sample db and dW_n with its operands in LDS (conv_dw3.hip); otherwise the mask and db take one pass and
// dW_n a batched sgemm F,T with col_n gathered from x. The two sample-order sums share a launch. dx is one
// kernel with dcol in LDS when a sample's output positions fit it (conv_dx.hip), else a batched sgemm T,F into
// the workspace and col2im.
// A fresh dW or db is stored as the sum s, where the reference adds s to a zero-filled gradient (0 + s): the
// two agree because every such sum starts at +0 (fma chains, lane sums and Tensor::sum(0) alike) and so is
// never -0.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "abi_common.hpp"
#include "kernels/hip/conv.hpp"
#include "kernels/hip/gemm.hpp"
#include "kernels/hip/reduce.hpp"
#include "workspace.hpp"
#include "nnh.h"

using namespace nnh;

namespace {

constexpr size_t kDirectMaxK = 32;

int conv_geometry(size_t N, size_t Cin, size_t H, size_t W, size_t Cout, size_t kh, size_t kw, int stride,
                  int padding, ConvGeom& g) {
	// ops.cpp:1350-1365 (the padded extent computed without wrapping)
	if (stride <= 0 || padding < 0) return fail(NNH_ERR_SHAPE, "conv2d: stride must be positive, padding >= 0");
	const unsigned __int128 pad2 = 2 * (unsigned __int128)padding;
	if (kh > H + pad2 || kw > W + pad2) return fail(NNH_ERR_SHAPE, "conv2d: kernel larger than the padded input");
	const size_t lim = 1u << 30;
	if (Cin > lim || H > lim || W > lim || kh > lim || kw > lim || (size_t)padding > lim || Cout >= ((size_t)1 << 31))
		return fail(NNH_ERR_INVALID, "conv2d: size too large");
	g.cin = (int)Cin;
	g.h = (int)H;
	g.w = (int)W;
	g.kh = (int)kh;
	g.kw = (int)kw;
	g.stride = stride;
	g.pad = padding;
	const size_t ho = (H + 2 * (size_t)padding - kh) / (size_t)stride + 1;  // ops.cpp:135-139
	const size_t wo = (W + 2 * (size_t)padding - kw) / (size_t)stride + 1;
	if (Cin * H * W >= ((size_t)1 << 31) || ho * wo >= ((size_t)1 << 31) || Cin * kh * kw >= ((size_t)1 << 31))
		return fail(NNH_ERR_INVALID, "conv2d: a sample is too large");
	g.ho = (int)ho;
	g.wo = (int)wo;
	if (!count_ok({N, Cin, H, W}) || !count_ok({N, Cout, ho, wo}) || !count_ok({Cout, Cin, kh, kw}))
		return fail(NNH_ERR_INVALID, "conv2d: size out of range (above 2^60 elements)");
	return NNH_OK;
}

ColGather col_gather(const ConvGeom& g) {
	ColGather c;
	c.cin = g.cin;
	c.h = g.h;
	c.w = g.w;
	c.kh = g.kh;
	c.kw = g.kw;
	c.stride = g.stride;
	c.pad = g.pad;
	c.ho = g.ho;
	c.wo = g.wo;
	c.khkw = make_fastdiv((unsigned)(g.kh * g.kw));
	c.kw_div = make_fastdiv((unsigned)g.kw);
	c.wo_div = make_fastdiv((unsigned)g.wo);
	return c;
}

// One workspace for nnh_conv2d_backward: the masked gradient, per-sample bias and weight gradients, dcol, and
// the depth-cut partials of the two GEMMs (which run one after the other and share them).
struct BwdPlan {
	size_t total = 0, off_m = 0, off_gb = 0, off_gw = 0, off_col = 0, off_part = 0;
	int64_t part = 0;
	bool dx_fused = false;
};

// packed: the flags are bits and the first-layer kernel runs the whole backward (it writes the per-sample weight
// gradients even when dW is not asked for, and needs no masked copy).
BwdPlan conv_backward_plan(const ConvGeom& geo, size_t N, size_t Cout, bool alive, bool dx, bool dw, bool db,
                           bool packed = false) {
	BwdPlan p;
	const size_t hw = (size_t)geo.ho * geo.wo, K = (size_t)geo.cin * geo.kh * geo.kw;
	if (N == 0 || (!dx && !dw && !db)) return p;
	WorkspacePlan plan;
	if (packed) {
		p.off_gb = db ? plan.add(N * Cout * 4) : 0;
		p.off_gw = plan.add(N * Cout * K * 4);
		p.total = plan.total;
		return p;
	}
	p.off_m = alive ? plan.add(N * Cout * hw * 4) : 0;
	p.off_gb = db ? plan.add(N * Cout * 4) : 0;
	p.off_gw = dw ? plan.add(N * Cout * K * 4) : 0;
	p.dx_fused = dx && conv_dx_fused_ok(geo, (int64_t)N, (int)Cout);
	p.off_col = dx && !p.dx_fused ? plan.add(N * K * hw * 4) : 0;
	p.part = std::max(dw ? gemm_workspace_floats((int64_t)Cout, (int64_t)K, (int64_t)hw, (int64_t)N, true) : 0,
	                  dx && !p.dx_fused ? gemm_workspace_floats((int64_t)K, (int64_t)hw, (int64_t)Cout, (int64_t)N) : 0);
	p.off_part = p.part ? plan.add((size_t)p.part * 4) : 0;
	p.total = plan.total;
	return p;
}

// Scratch of nnh_conv2d_forward: the depth-cut partials of the batched implicit GEMM, where that path may run
// (the direct and LDS kernels need none).
size_t conv_forward_ws(const ConvGeom& g, size_t N, size_t Cout) {
	const size_t hw = (size_t)g.ho * g.wo, K = (size_t)g.cin * g.kh * g.kw;
	if (N == 0 || Cout == 0 || hw == 0 || K <= kDirectMaxK) return 0;
	return gemm_workspace_bytes(Cout, hw, K, N, true);
}

// Whether the packed flag (and pooling-offset) forms take a geometry: the forward's quad kernel (or, with the 2 x 2
// pool, the fused kernel) writes them and the first-layer backward kernel reads them.
bool packed_geometry(const ConvGeom& g, size_t N, size_t Cout, bool pool) {
	const int64_t hw = (int64_t)g.ho * g.wo;
	if (N == 0 || Cout == 0 || hw == 0) return false;
	const bool fwd = pool ? conv_relu_pool2_ok(nullptr, nullptr, nullptr, nullptr, nullptr, g, (int64_t)N) && g.w <= 256
	                      : conv_same_quad_ok(nullptr, nullptr, nullptr, g, (int64_t)N) && hw % 8 == 0 &&
	                            (size_t)g.cin * g.kh * g.kw <= kDirectMaxK;
	return fwd && conv_first_bwd_ok(g, (int64_t)N, (int)Cout, true, nullptr, nullptr, true);
}

int conv_backward_impl(const float* g, const float* x, const float* w, const unsigned char* alive, bool packed, size_t N,
                       size_t Cin, size_t H, size_t W, size_t Cout, size_t kh, size_t kw, int stride, int padding,
                       float* dx, int dx_first, float* dw, int dw_first, float* db, int db_first, void* stream);

}  // namespace

extern "C" {

int nnh_conv2d_packed_supported(size_t N, size_t Cin, size_t H, size_t W, size_t Cout, size_t kh, size_t kw, int stride,
                                int padding, int with_pool) {
	ConvGeom g;
	const std::string saved = g_last_error;
	const bool ok = conv_geometry(N, Cin, H, W, Cout, kh, kw, stride, padding, g) == NNH_OK &&
	                packed_geometry(g, N, Cout, with_pool != 0);
	g_last_error = saved;
	return ok ? 1 : 0;
}

int nnh_conv2d_forward_workspace_size(size_t N, size_t Cin, size_t H, size_t W, size_t Cout, size_t kh, size_t kw,
                                      int stride, int padding, size_t* bytes) {
	return query_both_modes(bytes, [&](size_t* bytes) {
		ConvGeom g;
		const int rc = conv_geometry(N, Cin, H, W, Cout, kh, kw, stride, padding, g);
		if (rc != NNH_OK) return rc;
		return put_bytes(bytes, conv_forward_ws(g, N, Cout));
	});
}

int nnh_conv2d_backward_workspace_size(size_t N, size_t Cin, size_t H, size_t W, size_t Cout, size_t kh, size_t kw,
                                       int stride, int padding, int with_alive, int want_dx, int want_dw, int want_db,
                                       size_t* bytes) {
	return query_both_modes(bytes, [&](size_t* bytes) {
		ConvGeom g;
		const int rc = conv_geometry(N, Cin, H, W, Cout, kh, kw, stride, padding, g);
		if (rc != NNH_OK) return rc;
		size_t total = conv_backward_plan(g, N, Cout, with_alive, want_dx, want_dw, want_db).total;
		// with flags: also enough for nnh_conv2d_backward_packed where that takes the geometry
		if (with_alive && packed_geometry(g, N, Cout, false))
			total = std::max(total, conv_backward_plan(g, N, Cout, true, want_dx, want_dw, want_db, true).total);
		return put_bytes(bytes, total);
	});
}

int nnh_conv2d_forward(const float* x, size_t N, size_t Cin, size_t H, size_t W, const float* w, size_t Cout,
                       size_t kh, size_t kw, const float* bias, int stride, int padding, int fuse_relu, float* y,
                       unsigned char* alive, void* stream) {
	NumericsScope numerics_scope(stream);
	ConvGeom g;
	int rc = conv_geometry(N, Cin, H, W, Cout, kh, kw, stride, padding, g);
	if (rc != NNH_OK) return rc;
	const size_t hw = (size_t)g.ho * g.wo, K = Cin * kh * kw;
	if (N == 0 || Cout == 0 || hw == 0) return NNH_OK;
	if (!x || !w || !bias || !y) return fail(NNH_ERR_INVALID, "conv2d: null pointer");
	if (ranges_overlap(y, N * Cout * hw * 4, x, N * Cin * H * W * 4)) return fail(NNH_ERR_ALIAS, "conv2d: y overlaps x");
	hipStream_t s = reinterpret_cast<hipStream_t>(stream);
	unsigned char* al = fuse_relu ? alive : nullptr;
	if (K <= kDirectMaxK)
		return hip_status(conv_direct(x, w, bias, y, al, g, (int64_t)N, (int)Cout, fuse_relu ? 1 : 0, s), "conv2d direct");
	if (conv_fwd3_ok(g, (int64_t)N, (int)Cout, y, al))
		return hip_status(conv_fwd3(x, w, bias, y, al, g, (int64_t)N, (int)Cout, fuse_relu ? 1 : 0, s), "conv2d 3x3");
	// Y_n = W col_n (ops.cpp:1395), W shared by every sample, col_n gathered from x_n
	nnh_batch b{};
	b.ndim = 1;
	b.shape[0] = N;
	b.stride_a[0] = 0;
	b.stride_b[0] = (ptrdiff_t)(Cin * H * W);
	b.stride_c[0] = (ptrdiff_t)(Cout * hw);
	nnh_epilogue ep{NNH_BIAS_ROW, fuse_relu ? 1 : 0, bias, al};
	const ColGather cg = col_gather(g);
	GemmCall call;
	rc = build_gemm(0, 0, Cout, hw, K, w, K, x, hw, y, hw, 0, &b, &ep, call, &cg);
	if (rc != NNH_OK) return rc;
	return run_gemm(call, stream, -1);
}

int nnh_conv2d_relu_maxpool2d_forward(const float* x, size_t N, size_t Cin, size_t H, size_t W, const float* w,
                                      size_t Cout, size_t kh, size_t kw, const float* bias, int stride, int padding,
                                      size_t pool_kernel, size_t pool_stride, float* y, unsigned char* alive,
                                      float* pooled, unsigned int* argmax, void* stream) {
	NumericsScope numerics_scope(stream);
	ConvGeom g;
	int rc = conv_geometry(N, Cin, H, W, Cout, kh, kw, stride, padding, g);
	if (rc != NNH_OK) return rc;
	const size_t hw = (size_t)g.ho * g.wo;
	size_t pho = 0, pwo = 0;
	rc = maxpool_geometry((size_t)g.ho, (size_t)g.wo, pool_kernel, pool_stride, pho, pwo);
	if (rc != NNH_OK) return rc;
	if (N == 0 || Cout == 0 || hw == 0) return NNH_OK;
	if (!x || !w || !bias || !y || !pooled) return fail(NNH_ERR_INVALID, "conv2d_relu_maxpool2d: null pointer");
	const uint64_t xb = (uint64_t)N * Cin * H * W * 4, yb = (uint64_t)N * Cout * hw * 4;
	const uint64_t pb = (uint64_t)N * Cout * pho * pwo * 4, ab = yb / 4;
	if (ranges_overlap(y, yb, x, xb) || ranges_overlap(pooled, pb, x, xb) || ranges_overlap(pooled, pb, y, yb) ||
	    ranges_overlap(argmax, pb, x, xb) || ranges_overlap(argmax, pb, y, yb) || ranges_overlap(argmax, pb, pooled, pb) ||
	    ranges_overlap(alive, ab, pooled, pb) || ranges_overlap(alive, ab, argmax, pb) ||
	    ranges_overlap(alive, ab, y, yb) || ranges_overlap(alive, ab, x, xb))
		return fail(NNH_ERR_ALIAS, "conv2d_relu_maxpool2d: outputs overlap each other or the input");
	const bool fused = pool_kernel == 2 && pool_stride == 2 && conv_relu_pool2_ok(x, y, alive, pooled, argmax, g, (int64_t)N);
	if (!fused) {  // the two ops one after the other
		rc = nnh_conv2d_forward(x, N, Cin, H, W, w, Cout, kh, kw, bias, stride, padding, 1, y, alive, stream);
		if (rc != NNH_OK) return rc;
		return nnh_maxpool2d_forward(y, N, Cout, g.ho, g.wo, pool_kernel, pool_stride, pooled, argmax, stream);
	}
	return hip_status(conv_relu_pool2(x, w, bias, y, alive, pooled, argmax, g, (int64_t)N, (int)Cout,
	                                  reinterpret_cast<hipStream_t>(stream)),
	                  "conv2d_relu_maxpool2d");
}

int nnh_conv2d_backward(const float* g, const float* x, const float* w, const unsigned char* alive, size_t N,
                        size_t Cin, size_t H, size_t W, size_t Cout, size_t kh, size_t kw, int stride, int padding,
                        float* dx, int dx_first, float* dw, int dw_first, float* db, int db_first, void* stream) {
	return conv_backward_impl(g, x, w, alive, false, N, Cin, H, W, Cout, kh, kw, stride, padding, dx, dx_first, dw,
	                          dw_first, db, db_first, stream);
}

int nnh_conv2d_backward_packed(const float* g, const float* x, const float* w, const unsigned char* alive_bits,
                               size_t N, size_t Cin, size_t H, size_t W, size_t Cout, size_t kh, size_t kw, int stride,
                               int padding, float* dx, int dx_first, float* dw, int dw_first, float* db, int db_first,
                               void* stream) {
	if (N > 0 && (dx || dw || db) && !alive_bits) return fail(NNH_ERR_INVALID, "conv2d backward: null alive bits");
	return conv_backward_impl(g, x, w, alive_bits, true, N, Cin, H, W, Cout, kh, kw, stride, padding, dx, dx_first, dw,
	                          dw_first, db, db_first, stream);
}

int nnh_conv2d_relu_forward_packed(const float* x, size_t N, size_t Cin, size_t H, size_t W, const float* w,
                                   size_t Cout, size_t kh, size_t kw, const float* bias, int stride, int padding,
                                   float* y, unsigned char* alive_bits, void* stream) {
	NumericsScope numerics_scope(stream);
	ConvGeom g;
	int rc = conv_geometry(N, Cin, H, W, Cout, kh, kw, stride, padding, g);
	if (rc != NNH_OK) return rc;
	const size_t hw = (size_t)g.ho * g.wo;
	if (N == 0 || Cout == 0 || hw == 0) return NNH_OK;
	if (!x || !w || !bias || !y || !alive_bits) return fail(NNH_ERR_INVALID, "conv2d_relu packed: null pointer");
	if (!packed_geometry(g, N, Cout, false) || !conv_same_quad_ok(x, y, nullptr, g, (int64_t)N))
		return fail(NNH_ERR_INVALID, "conv2d_relu packed: geometry or alignment not taken (nnh_conv2d_packed_supported, "
		                             "16-byte aligned x and y)");
	const uint64_t xb = (uint64_t)N * Cin * H * W * 4, yb = (uint64_t)N * Cout * hw * 4, bb = yb / 32;
	if (ranges_overlap(y, yb, x, xb) || ranges_overlap(alive_bits, bb, x, xb) || ranges_overlap(alive_bits, bb, y, yb))
		return fail(NNH_ERR_ALIAS, "conv2d_relu packed: outputs overlap each other or the input");
	return hip_status(conv_same_quad(x, w, bias, y, nullptr, g, (int64_t)N, (int)Cout, 1, 4,
	                                 reinterpret_cast<hipStream_t>(stream), alive_bits),
	                  "conv2d_relu packed");
}

int nnh_conv2d_relu_maxpool2d_forward_packed(const float* x, size_t N, size_t Cin, size_t H, size_t W, const float* w,
                                             size_t Cout, size_t kh, size_t kw, const float* bias, int stride,
                                             int padding, float* y, unsigned char* alive_bits, float* pooled,
                                             unsigned char* argmax2, void* stream) {
	NumericsScope numerics_scope(stream);
	ConvGeom g;
	int rc = conv_geometry(N, Cin, H, W, Cout, kh, kw, stride, padding, g);
	if (rc != NNH_OK) return rc;
	const size_t hw = (size_t)g.ho * g.wo;
	if (N == 0 || Cout == 0 || hw == 0) return NNH_OK;
	if (!x || !w || !bias || !y || !alive_bits || !pooled || !argmax2)
		return fail(NNH_ERR_INVALID, "conv2d_relu_maxpool2d packed: null pointer");
	if (!packed_geometry(g, N, Cout, true) || !conv_relu_pool2_ok(x, y, nullptr, pooled, nullptr, g, (int64_t)N))
		return fail(NNH_ERR_INVALID, "conv2d_relu_maxpool2d packed: geometry or alignment not taken "
		                             "(nnh_conv2d_packed_supported, 16-byte aligned x and y, 8-byte aligned pooled)");
	const uint64_t xb = (uint64_t)N * Cin * H * W * 4, yb = (uint64_t)N * Cout * hw * 4, bb = yb / 32;
	const uint64_t pb = yb / 4, ab = (uint64_t)N * Cout * (g.h / 2) * ((g.w + 7) / 8);
	if (ranges_overlap(y, yb, x, xb) || ranges_overlap(pooled, pb, x, xb) || ranges_overlap(pooled, pb, y, yb) ||
	    ranges_overlap(argmax2, ab, x, xb) || ranges_overlap(argmax2, ab, y, yb) || ranges_overlap(argmax2, ab, pooled, pb) ||
	    ranges_overlap(alive_bits, bb, pooled, pb) || ranges_overlap(alive_bits, bb, argmax2, ab) ||
	    ranges_overlap(alive_bits, bb, y, yb) || ranges_overlap(alive_bits, bb, x, xb))
		return fail(NNH_ERR_ALIAS, "conv2d_relu_maxpool2d packed: outputs overlap each other or the input");
	return hip_status(conv_relu_pool2(x, w, bias, y, nullptr, pooled, nullptr, g, (int64_t)N, (int)Cout,
	                                  reinterpret_cast<hipStream_t>(stream), alive_bits, argmax2),
	                  "conv2d_relu_maxpool2d packed");
}

}  // extern "C"

namespace {

int conv_backward_impl(const float* g, const float* x, const float* w, const unsigned char* alive, bool packed, size_t N,
                       size_t Cin, size_t H, size_t W, size_t Cout, size_t kh, size_t kw, int stride, int padding,
                       float* dx, int dx_first, float* dw, int dw_first, float* db, int db_first, void* stream) {
	NumericsScope numerics_scope(stream);
	ConvGeom geo;
	int rc = conv_geometry(N, Cin, H, W, Cout, kh, kw, stride, padding, geo);
	if (rc != NNH_OK) return rc;
	const size_t hw = (size_t)geo.ho * geo.wo, K = Cin * kh * kw;
	hipStream_t s = reinterpret_cast<hipStream_t>(stream);
	if (!dx && !dw && !db) return NNH_OK;
	if (N == 0) {
		// no samples: dx is empty, and dW, db receive a sum over zero samples (zeros), stored or added
		if (dw) rc = hip_status(sum_rows(nullptr, 0, (int64_t)(Cout * K), dw, dw_first ? 0 : 2, s), "conv2d dw");
		if (rc == NNH_OK && db) rc = hip_status(sum_rows(nullptr, 0, (int64_t)Cout, db, db_first ? 0 : 2, s), "conv2d db");
		return rc;
	}
	if (!g || !x || !w) return fail(NNH_ERR_INVALID, "conv2d backward: null pointer");
	{
		const uint64_t gb_ = (uint64_t)N * Cout * hw * 4, xb = (uint64_t)N * Cin * H * W * 4, wb = (uint64_t)Cout * K * 4;
		const uint64_t ab = packed ? gb_ / 32 : gb_ / 4;
		const void* ins[4] = {g, x, w, alive};
		const uint64_t in_bytes[4] = {gb_, xb, wb, ab};
		const void* outs[3] = {dx, dw, db};
		const uint64_t out_bytes[3] = {xb, wb, (uint64_t)Cout * 4};
		for (int o = 0; o < 3; ++o) {
			for (int i = 0; i < 4; ++i)
				if (ranges_overlap(outs[o], out_bytes[o], ins[i], in_bytes[i]))
					return fail(NNH_ERR_ALIAS, "conv2d backward: a gradient overlaps an input");
			for (int p = 0; p < o; ++p)
				if (ranges_overlap(outs[o], out_bytes[o], outs[p], out_bytes[p]))
					return fail(NNH_ERR_ALIAS, "conv2d backward: gradients overlap each other");
		}
	}
	// packed flags: the first-layer kernel reads them (nnh_conv2d_packed_supported's backward half; g 16-byte aligned)
	if (packed && !conv_first_bwd_ok(geo, (int64_t)N, (int)Cout, dx != nullptr, g, nullptr, true))
		return fail(NNH_ERR_INVALID, "conv2d backward packed: geometry or alignment not taken "
		                             "(nnh_conv2d_packed_supported, 16-byte aligned g)");
	const BwdPlan plan =
	    conv_backward_plan(geo, N, Cout, alive != nullptr, dx != nullptr, dw != nullptr, db != nullptr, packed);
	rc = check_workspace(stream, plan.total);
	if (rc != NNH_OK) return rc;
	const bool dx_fused = plan.dx_fused;
	StreamWorkspace ws(s, plan.total);
	if (ws.error() != hipSuccess) return hip_status(ws.error(), "conv2d workspace");
	float* partials = plan.part ? ws.at<float>(plan.off_part) : nullptr;
	float* m = alive ? ws.at<float>(plan.off_m) : nullptr;
	float* gb = db ? ws.at<float>(plan.off_gb) : nullptr;
	float* gw = dw || packed ? ws.at<float>(plan.off_gw) : nullptr;
	const float* gm = alive ? m : g;
	// 3x3, stride 1, padding 1 on small planes: one kernel takes the mask (ops.cpp:1439-1443), the per-sample bias
	// sums (1445) and the per-sample weight gradients (1448-1449) with its operands in LDS
	const bool dw3 = !packed && dw && conv_dw3_ok(geo, (int64_t)N, (int)Cout, g, alive, m);
	// short column depth (a first layer): db and dW per sample from LDS, the mask applied as g is staged; the dx
	// kernel then masks g itself, so the masked gradient is never written
	// a first layer's whole backward (K <= 16, Cout <= 32) in one workgroup per sample (always with packed flags)
	const bool first =
	    packed || (dw && !dw3 && conv_first_bwd_ok(geo, (int64_t)N, (int)Cout, dx != nullptr, g, alive));
	const bool dwp = dw && !dw3 && !first && (!dx || dx_fused) && conv_dwp_ok(geo, (int64_t)N, (int)Cout);
	if (dw3) {
		rc = hip_status(conv_dw3(g, alive, m, gb, x, gw, geo, (int64_t)N, (int)Cout, s), "conv2d mask, db, dw 3x3");
	} else if (first) {
		rc = hip_status(conv_first_bwd(g, alive, x, w, gb, gw, dx, dx_first ? 1 : 0, geo, (int64_t)N, (int)Cout, s, packed),
		                "conv2d db, dw, dx");
	} else if (dwp) {
		rc = hip_status(conv_dwp(g, alive, x, gb, gw, geo, (int64_t)N, (int)Cout, s), "conv2d db, dw");
	} else if (alive) {  // ops.cpp:1439-1443, with the per-sample bias sums of ops.cpp:1445 in the same pass
		rc = db ? hip_status(masked_lane_sums(g, alive, m, (int64_t)(N * Cout), (int64_t)hw, gb, s), "conv2d mask, db")
		        : hip_status(mask_grad(g, alive, m, (int64_t)(N * Cout * hw), s), "conv2d mask");
	} else if (db) {  // ops.cpp:1445
		rc = hip_status(lane_sums(gm, (int64_t)(N * Cout), (int64_t)hw, gb, s), "conv2d db");
	}
	if (rc == NNH_OK && dw && !dw3 && !dwp && !first) {  // ops.cpp:1448-1449: dW_n = g_n col_n^T with col_n gathered from x_n
		nnh_batch b{};
		b.ndim = 1;
		b.shape[0] = N;
		b.stride_a[0] = (ptrdiff_t)(Cout * hw);
		b.stride_b[0] = (ptrdiff_t)(Cin * H * W);
		b.stride_c[0] = (ptrdiff_t)(Cout * K);
		const ColGather cg = col_gather(geo);
		GemmCall call;
		rc = build_gemm(0, 1, Cout, K, hw, gm, hw, x, hw, gw, K, 0, &b, nullptr, call, &cg);
		if (rc == NNH_OK) rc = run_gemm(call, stream, -1, partials);
	}
	// the sample-order sums (ops.cpp:1461-1462), in one launch when both are asked for
	if (rc == NNH_OK && db && dw)
		rc = hip_status(sum_rows_pair(gw, (int64_t)N, (int64_t)(Cout * K), dw, dw_first ? 0 : 2, gb, (int64_t)N,
		                              (int64_t)Cout, db, db_first ? 0 : 2, s),
		                "conv2d dw, db");
	else if (rc == NNH_OK && dw)
		rc = hip_status(sum_rows(gw, (int64_t)N, (int64_t)(Cout * K), dw, dw_first ? 0 : 2, s), "conv2d dw");
	else if (rc == NNH_OK && db)
		rc = hip_status(sum_rows(gb, (int64_t)N, (int64_t)Cout, db, db_first ? 0 : 2, s), "conv2d db");
	if (rc == NNH_OK && dx && first) {
		// computed with dW above
	} else if (rc == NNH_OK && dx && dx_fused) {  // ops.cpp:1452-1455, dcol kept on chip
		rc = hip_status(dwp ? conv_dx_fused(g, alive, w, dx, geo, (int64_t)N, (int)Cout, dx_first ? 1 : 0, s)
		                    : conv_dx_fused(gm, nullptr, w, dx, geo, (int64_t)N, (int)Cout, dx_first ? 1 : 0, s),
		                "conv2d dx");
	} else if (rc == NNH_OK && dx) {  // ops.cpp:1452-1455
		float* col = ws.at<float>(plan.off_col);
		nnh_batch b{};
		b.ndim = 1;
		b.shape[0] = N;
		b.stride_a[0] = 0;
		b.stride_b[0] = (ptrdiff_t)(Cout * hw);
		b.stride_c[0] = (ptrdiff_t)(K * hw);
		GemmCall call;
		rc = build_gemm(1, 0, K, hw, Cout, w, K, gm, hw, col, hw, 0, &b, nullptr, call);
		if (rc == NNH_OK) rc = run_gemm(call, stream, -1, partials);
		if (rc == NNH_OK) rc = hip_status(col2im(col, dx, geo, (int64_t)N, dx_first ? 1 : 0, s), "col2im");
	}
	return rc;
}

}  // namespace

extern "C" {

int nnh_im2col(const float* x, size_t N, size_t Cin, size_t H, size_t W, size_t kh, size_t kw, int stride, int padding,
               float* col, void* stream) {
	ConvGeom g;
	int rc = conv_geometry(N, Cin, H, W, 1, kh, kw, stride, padding, g);
	if (rc != NNH_OK) return rc;
	if (!count_ok({N, Cin * kh * kw, (size_t)g.ho * g.wo})) return fail(NNH_ERR_INVALID, "im2col: size out of range");
	const size_t total = N * Cin * kh * kw * (size_t)g.ho * g.wo;
	if (total == 0) return NNH_OK;
	if (!x || !col) return fail(NNH_ERR_INVALID, "im2col: null pointer");
	if (ranges_overlap(col, (uint64_t)total * 4, x, (uint64_t)N * Cin * H * W * 4))
		return fail(NNH_ERR_ALIAS, "im2col: col overlaps x");
	return hip_status(im2col(x, col, g, (int64_t)N, reinterpret_cast<hipStream_t>(stream)), "im2col");
}

int nnh_col2im_add(const float* col, size_t N, size_t Cin, size_t H, size_t W, size_t kh, size_t kw, int stride,
                   int padding, float* dx, int first, void* stream) {
	ConvGeom g;
	int rc = conv_geometry(N, Cin, H, W, 1, kh, kw, stride, padding, g);
	if (rc != NNH_OK) return rc;
	if (!count_ok({N, Cin * kh * kw, (size_t)g.ho * g.wo})) return fail(NNH_ERR_INVALID, "col2im: size out of range");
	if (N * Cin * H * W == 0) return NNH_OK;
	if (!col || !dx) return fail(NNH_ERR_INVALID, "col2im: null pointer");
	if (ranges_overlap(dx, (uint64_t)N * Cin * H * W * 4, col, (uint64_t)N * Cin * kh * kw * g.ho * g.wo * 4))
		return fail(NNH_ERR_ALIAS, "col2im: dx overlaps col");
	return hip_status(col2im(col, dx, g, (int64_t)N, first, reinterpret_cast<hipStream_t>(stream)), "col2im");
}

}  // extern "C"
