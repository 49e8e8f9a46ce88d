// abi_sanitize.cpp - TEST CODE: the argument validation and shape logic of every include/nnh.h entry point, run on
// the host against libnnh's C-ABI translation units built with -fsanitize=address,undefined on their host side
// (tests/cpp/Makefile's `sanitize` target links them with the kernel objects of the ordinary build). Meant for a
// machine without a GPU:
// calls whose arguments are valid reach the HIP runtime and must come back NNH_ERR_HIP; invalid ones must be
// refused with their code before any HIP call. Sizes at and past every limit (2^31 dimensions, leading dimensions
// and batch strides near 2^63, shape products that overflow 64 bits) check that the validation's own arithmetic
// stays defined. Exit status 0 when every call returned an expected code; 77 when a GPU is visible (the buffers
// here are host memory); the sanitizers abort on their first report. Run by tests/test_sanitize.py.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <initializer_list>
#include <vector>

#include "nnh.h"
#include "nnh_noalloc.h"

namespace {

int g_failures = 0;
int g_calls = 0;

void expect(const char* what, int got, std::initializer_list<int> allowed) {
	++g_calls;
	for (int a : allowed)
		if (got == a) return;
	std::fprintf(stderr, "FAILED: %s returned %d (%s)\n", what, got, nnh_last_error());
	++g_failures;
}

#define EXPECT(call, ...) expect(#call, (call), {__VA_ARGS__})

constexpr int OK = NNH_OK, INV = NNH_ERR_INVALID, SHAPE = NNH_ERR_SHAPE, ALIAS = NNH_ERR_ALIAS, HIP = NNH_ERR_HIP;
constexpr size_t kHuge = (size_t)1 << 62;
constexpr size_t kMax = SIZE_MAX;
constexpr size_t k31 = (size_t)1 << 31;

std::vector<float> buf(size_t n) { return std::vector<float>(n, 1.0f); }

void gemm() {
	auto a = buf(64), b = buf(64), c = buf(64);
	EXPECT(nnh_sgemm(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, c.data(), 4, 0, nullptr), HIP);
	EXPECT(nnh_sgemm(0, 0, 0, 4, 4, nullptr, 4, nullptr, 4, nullptr, 4, 0, nullptr), OK);
	EXPECT(nnh_sgemm(0, 0, 4, 4, 0, nullptr, 0, nullptr, 0, c.data(), 4, 0, nullptr), HIP);  // k = 0: C = 0 (or kept)
	EXPECT(nnh_sgemm(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, nullptr, 4, 0, nullptr), INV);
	EXPECT(nnh_sgemm(0, 0, 4, 4, 4, nullptr, 4, b.data(), 4, c.data(), 4, 0, nullptr), INV);
	EXPECT(nnh_sgemm(0, 0, 4, 4, 4, a.data(), 3, b.data(), 4, c.data(), 4, 0, nullptr), INV);
	EXPECT(nnh_sgemm(1, 1, 4, 4, 4, a.data(), 3, b.data(), 4, c.data(), 4, 0, nullptr), INV);
	EXPECT(nnh_sgemm(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, c.data(), 3, 0, nullptr), INV);
	EXPECT(nnh_sgemm(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, a.data() + 2, 4, 0, nullptr), ALIAS);
	EXPECT(nnh_sgemm(0, 0, 4, 4, 4, a.data(), 4, c.data() + 8, 4, c.data(), 4, 0, nullptr), ALIAS);
	for (size_t big : {k31, kMax, kHuge}) {
		EXPECT(nnh_sgemm(0, 0, big, 4, 4, a.data(), 4, b.data(), 4, c.data(), 4, 0, nullptr), INV);
		EXPECT(nnh_sgemm(0, 0, 4, big, 4, a.data(), 4, b.data(), big, c.data(), big, 0, nullptr), INV);
		EXPECT(nnh_sgemm(0, 0, 4, 4, big, a.data(), big, b.data(), 4, c.data(), 4, 0, nullptr), INV);
	}
	const size_t m31 = k31 - 1;
	EXPECT(nnh_sgemm(0, 0, m31, m31, m31, a.data(), m31, b.data(), m31, c.data(), m31, 0, nullptr), INV, HIP);
	// leading dimensions past the limit are refused; 2^40 passes, and then A's (or B's) extent reaches C
	for (size_t ld : {kHuge, kMax, kMax / 2}) {
		EXPECT(nnh_sgemm(0, 0, 4, 4, 4, a.data(), ld, b.data(), 4, c.data(), 4, 0, nullptr), INV);
		EXPECT(nnh_sgemm(1, 1, 4, 4, 4, a.data(), 4, b.data(), ld, c.data(), 4, 0, nullptr), INV);
		EXPECT(nnh_sgemm(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, c.data(), ld, 1, nullptr), INV);
	}
	const size_t ld40 = (size_t)1 << 40;
	EXPECT(nnh_sgemm(0, 0, 4, 4, 4, a.data(), ld40, b.data(), 4, c.data(), 4, 0, nullptr), ALIAS, HIP);
	EXPECT(nnh_sgemm(1, 1, 4, 4, 4, a.data(), 4, b.data(), ld40, c.data(), 4, 0, nullptr), ALIAS, HIP);
	EXPECT(nnh_sgemm(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, c.data(), ld40, 1, nullptr), ALIAS, HIP);
	nnh_batch bt{};
	bt.ndim = 2;
	bt.shape[0] = 3;
	bt.shape[1] = 2;
	bt.stride_a[0] = 16;
	bt.stride_b[0] = 0;
	bt.stride_c[0] = 32;
	bt.stride_c[1] = 16;
	auto cb = buf(256);
	EXPECT(nnh_sgemm_batched(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, cb.data(), 4, 0, &bt, nullptr, nullptr), HIP);
	bt.ndim = 5;
	EXPECT(nnh_sgemm_batched(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, cb.data(), 4, 0, &bt, nullptr, nullptr), INV);
	bt.ndim = -1;
	EXPECT(nnh_sgemm_batched(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, cb.data(), 4, 0, &bt, nullptr, nullptr), INV);
	bt.ndim = 2;
	bt.stride_a[1] = -1;
	EXPECT(nnh_sgemm_batched(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, cb.data(), 4, 0, &bt, nullptr, nullptr), INV);
	bt.stride_a[1] = INT64_MAX;
	EXPECT(nnh_sgemm_batched(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, cb.data(), 4, 0, &bt, nullptr, nullptr), INV, HIP);
	bt.stride_a[1] = 0;
	bt.shape[0] = kHuge;
	EXPECT(nnh_sgemm_batched(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, cb.data(), 4, 0, &bt, nullptr, nullptr), INV);
	bt.shape[0] = k31 - 1;
	bt.shape[1] = k31 - 1;
	bt.stride_c[0] = INT64_MAX / 4;
	EXPECT(nnh_sgemm_batched(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, cb.data(), 4, 0, &bt, nullptr, nullptr), INV, HIP);
	nnh_batch b4{};
	b4.ndim = 4;
	for (int d = 0; d < 4; ++d) {
		b4.shape[d] = k31 - 1;  // 2^124 problems
		b4.stride_c[d] = 1;
	}
	EXPECT(nnh_sgemm_batched(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, cb.data(), 4, 0, &b4, nullptr, nullptr), INV, HIP);
	nnh_epilogue ep{};
	ep.bias_mode = 7;
	EXPECT(nnh_sgemm_batched(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, c.data(), 4, 0, nullptr, &ep, nullptr), INV);
	ep.bias_mode = NNH_BIAS_COL;
	EXPECT(nnh_sgemm_batched(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, c.data(), 4, 0, nullptr, &ep, nullptr), INV);
	ep.bias = c.data() + 1;
	EXPECT(nnh_sgemm_batched(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, c.data(), 4, 0, nullptr, &ep, nullptr), ALIAS);
	ep.bias = b.data();
	ep.relu = 1;
	EXPECT(nnh_sgemm_batched(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, c.data(), 4, 0, nullptr, &ep, nullptr), HIP);
	EXPECT(nnh_sgemm_config(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, c.data(), 4, 0, nullptr, nullptr, 999, nullptr),
	       INV);
	EXPECT(nnh_sgemm_config(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, c.data(), 4, 0, nullptr, nullptr, -2, nullptr),
	       INV);
	EXPECT(nnh_gemm_config_count() > 0 ? OK : INV, OK);
	EXPECT(nnh_gemm_config_name(-5)[0] == '\0' ? OK : INV, OK);  // no such configuration: ""
	EXPECT(nnh_gemm_config_name(1 << 30)[0] == '\0' ? OK : INV, OK);
	EXPECT(nnh_gemm_config_name(0)[0] != '\0' ? OK : INV, OK);
	EXPECT(nnh_sgemm_noalloc(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, c.data(), 4, 0, nullptr), HIP);
	EXPECT(nnh_sgemm_noalloc(0, 0, 4, 4, 4, a.data(), 3, b.data(), 4, c.data(), 4, 0, nullptr), INV);
	EXPECT(nnh_sgemm_noalloc(0, 0, 4, 4, kHuge, a.data(), kHuge, b.data(), 4, c.data(), 4, 0, nullptr), INV);
	EXPECT(nnh_sgemm_noalloc(0, 0, 40, 48, 1u << 20, a.data(), 1u << 20, b.data(), 48, c.data(), 48, 0, nullptr), INV,
	       ALIAS, HIP);
}

void sizes() {
	size_t bytes = 0;
	EXPECT(nnh_sgemm_workspace_size(4, 4, 4, 1, nullptr), INV);
	EXPECT(nnh_sgemm_workspace_size(4, 4, 4, 1, &bytes), OK);
	EXPECT(nnh_sgemm_workspace_size(kMax, kMax, kMax, kMax, &bytes), OK, INV);
	EXPECT(nnh_sgemm_workspace_size(40, 48, kHuge, kHuge, &bytes), OK, INV);
	EXPECT(nnh_linear_forward_workspace_size(kMax, kMax, kMax, &bytes), OK, INV);
	const size_t lead[3] = {kHuge, kHuge, 3};
	EXPECT(nnh_linear_backward_workspace_size(lead, 3, 4, 4, 1, 1, 1, &bytes), OK, INV);
	EXPECT(nnh_linear_backward_workspace_size(nullptr, 2, 4, 4, 1, 1, 1, &bytes), INV);
	EXPECT(nnh_linear_backward_workspace_size(lead, -1, 4, 4, 1, 1, 1, &bytes), INV, SHAPE);
	EXPECT(nnh_conv2d_forward_workspace_size(kMax, kMax, kMax, kMax, kMax, 3, 3, 1, 1, &bytes), OK, INV, SHAPE);
	EXPECT(nnh_conv2d_forward_workspace_size(2, 3, 8, 8, 4, 3, 3, 0, 1, &bytes), INV, SHAPE);
	EXPECT(nnh_conv2d_forward_workspace_size(2, 3, 8, 8, 4, 3, 3, 1, -1, &bytes), INV, SHAPE);
	EXPECT(nnh_conv2d_forward_workspace_size(2, 3, 8, 8, 4, 30, 3, 1, 0, &bytes), INV, SHAPE);
	EXPECT(nnh_conv2d_backward_workspace_size(kHuge, kHuge, 8, 8, kHuge, 3, 3, 1, 1, 1, 1, 1, 1, &bytes), OK, INV,
	       SHAPE);
	EXPECT(nnh_conv2d_backward_workspace_size(2, 3, 8, 8, 4, 3, 3, INT32_MAX, INT32_MAX, 1, 1, 1, 1, &bytes), OK, INV,
	       SHAPE);
	EXPECT(nnh_attention_forward_workspace_size(kMax, kMax, kMax, kMax, kMax, &bytes), OK, INV, SHAPE);
	EXPECT(nnh_attention_forward_workspace_size(2, 4, 4, 8, 0, &bytes), INV, SHAPE);
	EXPECT(nnh_attention_forward_workspace_size(2, 4, 4, 8, 3, &bytes), INV, SHAPE);
	EXPECT(nnh_attention_backward_workspace_size(kHuge, kHuge, 4, 8, 2, &bytes), OK, INV, SHAPE);
	const size_t as[2] = {kHuge, kHuge}, bs[2] = {kHuge, kHuge};
	EXPECT(nnh_matmul_workspace_size(as, 2, bs, 2, 0, 0, &bytes), OK, INV);
	EXPECT(nnh_matmul_backward_workspace_size(as, 2, bs, 2, 0, 1, 1, &bytes), OK, INV);
}

void matmul() {
	auto a = buf(256), b = buf(256), c = buf(256);
	size_t out[8];
	int nd = 0;
	const size_t a2[2] = {4, 8}, b2[2] = {8, 4}, b2x[2] = {7, 4};
	EXPECT(nnh_matmul_shape(a2, 2, b2, 2, 0, 0, out, &nd), OK);
	EXPECT(nnh_matmul_shape(a2, 2, b2x, 2, 0, 0, out, &nd), SHAPE);
	EXPECT(nnh_matmul_shape(a2, 1, b2, 2, 0, 0, out, &nd), SHAPE);
	EXPECT(nnh_matmul_shape(a2, -3, b2, 2, 0, 0, out, &nd), INV);
	EXPECT(nnh_matmul_shape(nullptr, 2, b2, 2, 0, 0, out, &nd), INV);
	EXPECT(nnh_matmul_shape(a2, 2, b2, 2, 0, 0, nullptr, &nd), INV);
	EXPECT(nnh_matmul(a.data(), a2, 2, b.data(), b2, 2, 0, 0, c.data(), nullptr), HIP);
	EXPECT(nnh_matmul(a.data(), a2, 2, b.data(), b2, 2, 0, 0, a.data(), nullptr), ALIAS);
	const size_t a4[4] = {2, 3, 4, 8}, b3[3] = {3, 8, 4}, b3x[3] = {2, 8, 4};
	EXPECT(nnh_matmul(a.data(), a4, 4, b.data(), b3, 3, 0, 0, c.data(), nullptr), HIP);
	EXPECT(nnh_matmul(a.data(), a4, 4, b.data(), b3x, 3, 0, 0, c.data(), nullptr), SHAPE);
	EXPECT(nnh_matmul(a.data(), a4, 4, b.data(), b2, 2, 0, 0, c.data(), nullptr), HIP);  // folded
	// shape products past 64 bits, and 2^31 rows after folding
	const size_t ah[4] = {kHuge, kHuge, 4, 8}, bh[3] = {kHuge, 8, 4}, af[3] = {k31, 2, 8};
	EXPECT(nnh_matmul_shape(ah, 4, bh, 3, 0, 0, out, &nd), OK, INV);
	EXPECT(nnh_matmul(a.data(), ah, 4, b.data(), bh, 3, 0, 0, c.data(), nullptr), INV);
	EXPECT(nnh_matmul(a.data(), af, 3, b.data(), b2, 2, 0, 0, c.data(), nullptr), INV);
	const size_t many[9] = {2, 1, 2, 1, 2, 1, 2, 4, 8}, manyb[9] = {1, 2, 1, 2, 1, 2, 1, 8, 4};
	EXPECT(nnh_matmul(a.data(), many, 9, b.data(), manyb, 9, 0, 0, c.data(), nullptr), INV, HIP);
	auto g = buf(256), da = buf(256), db = buf(256);
	EXPECT(nnh_matmul_backward(g.data(), a.data(), a2, 2, b.data(), b2, 2, 0, da.data(), 1, db.data(), 1, nullptr), HIP);
	EXPECT(nnh_matmul_backward(g.data(), a.data(), a2, 2, b.data(), b2x, 2, 0, da.data(), 1, db.data(), 1, nullptr),
	       SHAPE);
	EXPECT(nnh_matmul_backward(g.data(), a.data(), a2, 2, b.data(), b2, 2, 0, nullptr, 1, nullptr, 1, nullptr), OK, HIP);
	EXPECT(nnh_matmul_backward(g.data(), a.data(), a2, 2, b.data(), b2, 2, 0, g.data(), 1, db.data(), 1, nullptr),
	       ALIAS, INV);
	EXPECT(nnh_matmul_backward(g.data(), a.data(), ah, 4, b.data(), bh, 3, 0, da.data(), 1, db.data(), 1, nullptr), INV);
}

void linear_relu() {
	auto x = buf(256), w = buf(256), bias = buf(16), y = buf(256);
	EXPECT(nnh_linear_forward(x.data(), 4, 8, w.data(), 4, bias.data(), 1, y.data(), nullptr), HIP);
	EXPECT(nnh_linear_forward(x.data(), 4, 8, w.data(), 4, nullptr, 0, y.data(), nullptr), INV);  // linear has a bias
	EXPECT(nnh_linear_forward(nullptr, 4, 8, w.data(), 4, bias.data(), 1, y.data(), nullptr), INV);
	EXPECT(nnh_linear_forward(x.data(), 4, 8, w.data(), 4, bias.data(), 1, x.data(), nullptr), ALIAS);
	EXPECT(nnh_linear_forward(x.data(), kHuge, kHuge, w.data(), 4, bias.data(), 1, y.data(), nullptr), INV);
	EXPECT(nnh_linear_forward(x.data(), 4, 8, w.data(), kMax, bias.data(), 1, y.data(), nullptr), INV);
	auto g = buf(256), dx = buf(256), dw = buf(256), db = buf(16);
	const size_t lead[2] = {2, 2}, huge_lead[3] = {kHuge, kHuge, 2};
	EXPECT(nnh_linear_backward(g.data(), x.data(), w.data(), lead, 2, 8, 4, dx.data(), 1, dw.data(), 1, db.data(), 1,
	                           nullptr),
	       HIP);
	EXPECT(nnh_linear_backward(g.data(), x.data(), w.data(), lead, 2, 8, 4, nullptr, 1, nullptr, 1, nullptr, 1, nullptr),
	       OK);
	EXPECT(nnh_linear_backward(g.data(), x.data(), w.data(), nullptr, 2, 8, 4, dx.data(), 1, dw.data(), 1, db.data(), 1,
	                           nullptr),
	       INV);
	EXPECT(nnh_linear_backward(g.data(), x.data(), w.data(), huge_lead, 3, 8, 4, dx.data(), 1, dw.data(), 1, db.data(),
	                           1, nullptr),
	       INV);
	EXPECT(nnh_linear_backward(g.data(), x.data(), w.data(), lead, 2, 8, 4, g.data(), 1, dw.data(), 1, db.data(), 1,
	                           nullptr),
	       ALIAS, INV);
	EXPECT(nnh_relu_forward(x.data(), y.data(), 16, nullptr), HIP);
	EXPECT(nnh_relu_forward(x.data(), y.data(), 0, nullptr), OK);
	EXPECT(nnh_relu_forward(nullptr, y.data(), 16, nullptr), INV);
	EXPECT(nnh_relu_forward(x.data(), y.data(), kMax, nullptr), INV);
	EXPECT(nnh_relu_backward(x.data(), g.data(), dx.data(), 1, 16, nullptr), HIP);
	EXPECT(nnh_relu_backward(x.data(), g.data(), dx.data(), 1, kHuge, nullptr), INV);
	EXPECT(nnh_add_to_grad(dx.data(), g.data(), 16, 0, nullptr), HIP);
	EXPECT(nnh_add_to_grad(dx.data(), g.data(), kMax, 0, nullptr), INV);
	EXPECT(nnh_add_to_grad(nullptr, g.data(), 16, 0, nullptr), INV);
	EXPECT(nnh_tensor_sum0(x.data(), 4, 4, y.data(), 0, nullptr), HIP);
	EXPECT(nnh_tensor_sum0(x.data(), kHuge, kHuge, y.data(), 0, nullptr), INV);
	EXPECT(nnh_tensor_sum0(x.data(), 4, 4, nullptr, 0, nullptr), INV);
}

void attention() {
	auto q = buf(4096), k = buf(4096), v = buf(4096), out = buf(4096), probs = buf(4096), mask = buf(64);
	// N = 2, Tq = Tk = 4, D = 8, 2 heads
	EXPECT(nnh_attention_forward(q.data(), k.data(), v.data(), 2, 4, 4, 8, 2, nullptr, 1, out.data(), probs.data(),
	                             nullptr),
	       HIP);
	EXPECT(nnh_attention_forward(q.data(), k.data(), v.data(), 2, 4, 4, 8, 3, nullptr, 1, out.data(), probs.data(),
	                             nullptr),
	       SHAPE, INV);
	EXPECT(nnh_attention_forward(q.data(), k.data(), v.data(), 2, 4, 4, 8, 0, nullptr, 1, out.data(), probs.data(),
	                             nullptr),
	       SHAPE, INV);
	EXPECT(nnh_attention_forward(nullptr, k.data(), v.data(), 2, 4, 4, 8, 2, nullptr, 1, out.data(), probs.data(),
	                             nullptr),
	       INV);
	EXPECT(nnh_attention_forward(q.data(), k.data(), v.data(), 2, 4, 4, 8, 2, mask.data(), 0, q.data(), probs.data(),
	                             nullptr),
	       ALIAS);
	EXPECT(nnh_attention_forward(q.data(), k.data(), v.data(), kHuge, kHuge, 4, 8, 2, nullptr, 1, out.data(),
	                             probs.data(), nullptr),
	       SHAPE);  // causal needs Tq == Tk
	EXPECT(nnh_attention_forward(q.data(), k.data(), v.data(), kHuge, kHuge, 4, 8, 2, nullptr, 0, out.data(),
	                             probs.data(), nullptr),
	       INV);
	EXPECT(nnh_attention_forward(q.data(), k.data(), v.data(), 2, 4, kMax, kMax, 1, nullptr, 0, out.data(),
	                             probs.data(), nullptr),
	       INV);
	auto g = buf(4096), dq = buf(4096), dk = buf(4096), dv = buf(4096);
	EXPECT(nnh_attention_backward(g.data(), q.data(), k.data(), v.data(), probs.data(), 2, 4, 4, 8, 2, nullptr, 1,
	                              dq.data(), 1, dk.data(), 1, dv.data(), 1, nullptr),
	       HIP);
	EXPECT(nnh_attention_backward(g.data(), q.data(), k.data(), v.data(), probs.data(), 2, 4, 4, 8, 2, nullptr, 1,
	                              nullptr, 1, nullptr, 1, nullptr, 1, nullptr),
	       OK, HIP);
	EXPECT(nnh_attention_backward(g.data(), q.data(), k.data(), v.data(), nullptr, 2, 4, 4, 8, 2, nullptr, 1,
	                              dq.data(), 1, dk.data(), 1, dv.data(), 1, nullptr),
	       INV);
	EXPECT(nnh_attention_backward(g.data(), q.data(), k.data(), v.data(), probs.data(), kHuge, 4, kHuge, 8, 2, nullptr,
	                              0, dq.data(), 1, dk.data(), 1, dv.data(), 1, nullptr),
	       INV);
	EXPECT(nnh_attention_backward(g.data(), q.data(), k.data(), v.data(), probs.data(), 2, 4, 4, 8, 2, nullptr, 0,
	                              dq.data(), 1, dq.data(), 0, dq.data(), 0, nullptr),
	       HIP);  // q, k and v one node: one gradient buffer
	EXPECT(nnh_attention_backward(g.data(), q.data(), k.data(), v.data(), probs.data(), 2, 4, 4, 8, 2, nullptr, 0,
	                              dq.data(), 1, dk.data(), 1, probs.data() + 8, 1, nullptr),
	       ALIAS);
	EXPECT(nnh_scaled_masked_softmax_forward(q.data(), 2, 2, 4, 4, 0.5f, mask.data(), 1, out.data(), nullptr), HIP);
	EXPECT(nnh_scaled_masked_softmax_forward(q.data(), 2, 2, 4, 4, 0.5f, mask.data(), 1, q.data(), nullptr), HIP);
	EXPECT(nnh_scaled_masked_softmax_forward(q.data(), 2, 2, 4, 4, 0.5f, mask.data(), 1, q.data() + 4, nullptr), ALIAS);
	EXPECT(nnh_scaled_masked_softmax_forward(q.data(), kHuge, kHuge, 4, 4, 0.5f, nullptr, 1, out.data(), nullptr), INV);
	EXPECT(nnh_scaled_masked_softmax_forward(nullptr, 2, 2, 4, 4, 0.5f, nullptr, 1, out.data(), nullptr), INV);
	EXPECT(nnh_scaled_masked_softmax_backward(probs.data(), g.data(), 2, 2, 4, 4, 0.5f, nullptr, 0, dq.data(), 1,
	                                          nullptr),
	       HIP);
	EXPECT(nnh_scaled_masked_softmax_backward(probs.data(), g.data(), 2, 2, kMax, kMax, 0.5f, nullptr, 0, dq.data(), 1,
	                                          nullptr),
	       INV);
}

void conv_pool() {
	auto x = buf(4096), w = buf(4096), bias = buf(64), y = buf(8192), col = buf(16384);
	std::vector<unsigned char> alive(8192);
	std::vector<unsigned int> am(8192);
	auto pooled = buf(4096);
	// N = 2, Cin = 3, 8 x 8, Cout = 4, 3 x 3, stride 1, pad 1
	EXPECT(nnh_conv2d_forward(x.data(), 2, 3, 8, 8, w.data(), 4, 3, 3, bias.data(), 1, 1, 1, y.data(), alive.data(),
	                          nullptr),
	       HIP);
	EXPECT(nnh_conv2d_forward(x.data(), 2, 3, 8, 8, w.data(), 4, 3, 3, bias.data(), 0, 1, 1, y.data(), nullptr, nullptr),
	       INV, SHAPE);
	EXPECT(nnh_conv2d_forward(x.data(), 2, 3, 8, 8, w.data(), 4, 3, 3, bias.data(), 1, -1, 1, y.data(), nullptr,
	                          nullptr),
	       INV, SHAPE);
	EXPECT(nnh_conv2d_forward(x.data(), 2, 3, 8, 8, w.data(), 4, 12, 3, bias.data(), 1, 0, 1, y.data(), nullptr,
	                          nullptr),
	       INV, SHAPE);
	EXPECT(nnh_conv2d_forward(x.data(), 2, 3, 8, 8, w.data(), 4, 3, 3, nullptr, 1, 1, 1, y.data(), nullptr, nullptr),
	       INV, HIP);
	EXPECT(nnh_conv2d_forward(x.data(), 2, 3, 8, 8, w.data(), 4, 3, 3, bias.data(), 1, 1, 1, x.data(), nullptr, nullptr),
	       ALIAS);
	EXPECT(nnh_conv2d_forward(x.data(), kHuge, kHuge, 8, 8, w.data(), 4, 3, 3, bias.data(), 1, 1, 1, y.data(), nullptr,
	                          nullptr),
	       INV);
	EXPECT(nnh_conv2d_forward(x.data(), 2, 3, kMax, kMax, w.data(), 4, 3, 3, bias.data(), 1, 1, 1, y.data(), nullptr,
	                          nullptr),
	       INV);
	EXPECT(nnh_conv2d_forward(x.data(), 2, 3, 8, 8, w.data(), 4, kMax, kMax, bias.data(), INT32_MAX, INT32_MAX, 1,
	                          y.data(), nullptr, nullptr),
	       INV, SHAPE);
	EXPECT(nnh_conv2d_relu_maxpool2d_forward(x.data(), 2, 1, 8, 8, w.data(), 4, 3, 3, bias.data(), 1, 1, 2, 2, y.data(),
	                                         alive.data(), pooled.data(), am.data(), nullptr),
	       HIP);
	EXPECT(nnh_conv2d_relu_maxpool2d_forward(x.data(), 2, 1, 8, 8, w.data(), 4, 3, 3, bias.data(), 1, 1, 0, 2, y.data(),
	                                         alive.data(), pooled.data(), am.data(), nullptr),
	       INV, SHAPE);
	EXPECT(nnh_conv2d_relu_maxpool2d_forward(x.data(), 2, 1, 8, 8, w.data(), 4, 3, 3, bias.data(), 1, 1, 2, 2, y.data(),
	                                         alive.data(), y.data() + 4, am.data(), nullptr),
	       ALIAS);
	EXPECT(nnh_conv2d_relu_maxpool2d_forward(x.data(), 2, 1, 8, 8, w.data(), 4, 3, 3, bias.data(), 1, 1, kMax, kMax,
	                                         y.data(), alive.data(), pooled.data(), am.data(), nullptr),
	       INV, SHAPE);
	auto g = buf(8192), dx = buf(4096), dw = buf(4096), db = buf(64);
	EXPECT(nnh_conv2d_backward(g.data(), x.data(), w.data(), alive.data(), 2, 3, 8, 8, 4, 3, 3, 1, 1, dx.data(), 1,
	                           dw.data(), 1, db.data(), 1, nullptr),
	       HIP);
	EXPECT(nnh_conv2d_backward(g.data(), x.data(), w.data(), nullptr, 2, 3, 8, 8, 4, 3, 3, 1, 1, nullptr, 1, nullptr, 1,
	                           nullptr, 1, nullptr),
	       OK, HIP);
	EXPECT(nnh_conv2d_backward(g.data(), x.data(), w.data(), alive.data(), kHuge, 3, 8, 8, kHuge, 3, 3, 1, 1, dx.data(),
	                           1, dw.data(), 1, db.data(), 1, nullptr),
	       INV);
	EXPECT(nnh_conv2d_backward(g.data(), x.data(), w.data(), alive.data(), 2, 3, 8, 8, 4, 3, 3, 1, 1, g.data(), 1,
	                           dw.data(), 1, db.data(), 1, nullptr),
	       ALIAS, INV);
	EXPECT(nnh_im2col(x.data(), 2, 3, 8, 8, 3, 3, 1, 1, col.data(), nullptr), HIP);
	EXPECT(nnh_im2col(x.data(), 2, 3, 8, 8, 3, 3, 0, 1, col.data(), nullptr), INV, SHAPE);
	EXPECT(nnh_im2col(x.data(), kHuge, kHuge, 8, 8, 3, 3, 1, 1, col.data(), nullptr), INV);
	EXPECT(nnh_im2col(x.data(), 2, 3, 8, 8, 3, 3, 1, 1, x.data(), nullptr), ALIAS);
	EXPECT(nnh_col2im_add(col.data(), 2, 3, 8, 8, 3, 3, 1, 1, dx.data(), 1, nullptr), HIP);
	EXPECT(nnh_col2im_add(col.data(), 2, 3, 8, 8, kMax, 3, 1, 1, dx.data(), 1, nullptr), INV, SHAPE);
	EXPECT(nnh_maxpool2d_forward(x.data(), 2, 3, 8, 8, 2, 2, y.data(), am.data(), nullptr), HIP);
	EXPECT(nnh_maxpool2d_forward(x.data(), 2, 3, 8, 8, 0, 2, y.data(), am.data(), nullptr), INV, SHAPE);
	EXPECT(nnh_maxpool2d_forward(x.data(), 2, 3, 8, 8, 2, 0, y.data(), am.data(), nullptr), INV, SHAPE);
	EXPECT(nnh_maxpool2d_forward(x.data(), 2, 3, 8, 8, 9, 2, y.data(), am.data(), nullptr), INV, SHAPE);
	EXPECT(nnh_maxpool2d_forward(x.data(), kHuge, kHuge, 8, 8, 2, 2, y.data(), am.data(), nullptr), INV);
	EXPECT(nnh_maxpool2d_forward(x.data(), 2, 3, kMax, kMax, kMax, kMax, y.data(), am.data(), nullptr), INV, SHAPE);
	EXPECT(nnh_maxpool2d_backward(g.data(), am.data(), 2, 3, 8, 8, 2, 2, dx.data(), 1, nullptr), HIP);
	EXPECT(nnh_maxpool2d_backward(g.data(), nullptr, 2, 3, 8, 8, 2, 2, dx.data(), 1, nullptr), INV);
	EXPECT(nnh_maxpool2d_backward(g.data(), am.data(), kHuge, kHuge, 8, 8, 2, 2, dx.data(), 1, nullptr), INV);
}

void norm() {
	auto x = buf(2 * 3 * 16), y = buf(2 * 3 * 16), g = buf(2 * 3 * 16), dx = buf(2 * 3 * 16), w = buf(16), b = buf(16);
	auto mean = buf(32), var = buf(32), inv = buf(32), dw = buf(16), db = buf(16);
	std::vector<unsigned char> alive(2 * 3 * 16);
	size_t bytes = 0;
	EXPECT(nnh_batchnorm_workspace_size(2, 3, 16, &bytes), OK);
	EXPECT(bytes >= 2 * 2 * 3 * sizeof(float) ? OK : INV, OK);
	EXPECT(nnh_batchnorm_workspace_size(kHuge, kHuge, 16, &bytes), INV);
	EXPECT(nnh_batchnorm_workspace_size(2, kMax, 1, &bytes), INV);
	EXPECT(nnh_batchnorm_forward(x.data(), 2, 3, 16, w.data(), b.data(), 1e-5f, 1, y.data(), alive.data(), mean.data(),
	                             var.data(), inv.data(), nullptr),
	       HIP);
	EXPECT(nnh_batchnorm_forward(x.data(), 2, 3, 16, w.data(), b.data(), 1e-5f, 0, y.data(), nullptr, nullptr,
	                             var.data(), inv.data(), nullptr),
	       INV);
	EXPECT(nnh_batchnorm_forward(x.data(), 2, 3, 16, w.data(), b.data(), 1e-5f, 0, x.data(), nullptr, mean.data(),
	                             var.data(), inv.data(), nullptr),
	       ALIAS);
	EXPECT(nnh_batchnorm_forward(x.data(), 2, 3, 16, w.data(), b.data(), 1e-5f, 0, y.data(), nullptr, mean.data(),
	                             mean.data(), inv.data(), nullptr),
	       ALIAS);
	EXPECT(nnh_batchnorm_forward(x.data(), kHuge, kHuge, kHuge, w.data(), b.data(), 1e-5f, 0, y.data(), nullptr,
	                             mean.data(), var.data(), inv.data(), nullptr),
	       INV);
	EXPECT(nnh_batchnorm_forward(nullptr, 2, 0, 16, nullptr, nullptr, 1e-5f, 0, nullptr, nullptr, nullptr, nullptr,
	                             nullptr, nullptr),
	       OK);
	EXPECT(nnh_batchnorm_backward(g.data(), x.data(), alive.data(), w.data(), mean.data(), inv.data(), 2, 3, 16,
	                              dx.data(), 1, dw.data(), 1, db.data(), 1, nullptr),
	       HIP);
	EXPECT(nnh_batchnorm_backward(g.data(), x.data(), nullptr, w.data(), mean.data(), inv.data(), 2, 3, 16, g.data(), 1,
	                              dw.data(), 1, db.data(), 1, nullptr),
	       ALIAS);
	EXPECT(nnh_batchnorm_backward(g.data(), x.data(), nullptr, w.data(), nullptr, inv.data(), 2, 3, 16, dx.data(), 1,
	                              nullptr, 1, nullptr, 1, nullptr),
	       INV);
	EXPECT(nnh_batchnorm_backward(g.data(), x.data(), nullptr, w.data(), mean.data(), inv.data(), 2, 3, 16, nullptr, 1,
	                              nullptr, 1, nullptr, 1, nullptr),
	       OK);
	EXPECT(nnh_layernorm_forward(x.data(), 6, 16, w.data(), b.data(), 1e-5f, y.data(), mean.data(), inv.data(), nullptr),
	       HIP);
	EXPECT(nnh_layernorm_forward(x.data(), 6, 0, w.data(), b.data(), 1e-5f, y.data(), mean.data(), inv.data(), nullptr),
	       INV);
	EXPECT(nnh_layernorm_forward(x.data(), kHuge, kHuge, w.data(), b.data(), 1e-5f, y.data(), mean.data(), inv.data(),
	                             nullptr),
	       INV);
	EXPECT(nnh_layernorm_forward(x.data(), 6, 16, w.data(), b.data(), 1e-5f, x.data(), mean.data(), inv.data(), nullptr),
	       ALIAS);
	EXPECT(nnh_layernorm_backward(g.data(), x.data(), w.data(), mean.data(), inv.data(), 6, 16, dx.data(), 1, dw.data(),
	                              1, db.data(), 1, nullptr),
	       HIP);
	EXPECT(nnh_layernorm_backward(g.data(), x.data(), w.data(), mean.data(), inv.data(), 6, 16, dx.data(), 1, dw.data(),
	                              1, dw.data(), 1, nullptr),
	       ALIAS);
	EXPECT(nnh_layernorm_backward(g.data(), x.data(), nullptr, mean.data(), inv.data(), 6, 16, dx.data(), 1, nullptr, 1,
	                              nullptr, 1, nullptr),
	       INV);
}

void misc() {
	EXPECT(nnh_set_numerics(5), INV);
	EXPECT(nnh_set_numerics(NNH_NUMERICS_SPLIT_DEPTH), OK);
	EXPECT(nnh_get_numerics() == NNH_NUMERICS_SPLIT_DEPTH ? OK : INV, OK);
	auto a = buf(64), b = buf(64), c = buf(64);
	EXPECT(nnh_sgemm(0, 0, 4, 4, 4, a.data(), 4, b.data(), 4, c.data(), 4, 0, nullptr), HIP);
	EXPECT(nnh_set_numerics(NNH_NUMERICS_NNCPP), OK);
	// a stream's own mode, beside the process default
	void* s1 = reinterpret_cast<void*>(uintptr_t(0x1000));
	void* s2 = reinterpret_cast<void*>(uintptr_t(0x2000));
	EXPECT(nnh_set_stream_numerics(s1, 7), INV);
	EXPECT(nnh_set_stream_numerics(s1, NNH_NUMERICS_SPLIT_DEPTH), OK);
	EXPECT(nnh_get_stream_numerics(s1) == NNH_NUMERICS_SPLIT_DEPTH ? OK : INV, OK);
	EXPECT(nnh_get_stream_numerics(s2) == NNH_NUMERICS_NNCPP ? OK : INV, OK);
	EXPECT(nnh_get_numerics() == NNH_NUMERICS_NNCPP ? OK : INV, OK);
	EXPECT(nnh_set_stream_numerics(s2, NNH_NUMERICS_NNCPP), OK);
	EXPECT(nnh_set_numerics(NNH_NUMERICS_SPLIT_DEPTH), OK);
	EXPECT(nnh_get_stream_numerics(s2) == NNH_NUMERICS_NNCPP ? OK : INV, OK);
	EXPECT(nnh_set_stream_numerics(s2, NNH_NUMERICS_DEFAULT), OK);
	EXPECT(nnh_get_stream_numerics(s2) == NNH_NUMERICS_SPLIT_DEPTH ? OK : INV, OK);
	EXPECT(nnh_set_stream_numerics(s1, NNH_NUMERICS_DEFAULT), OK);
	EXPECT(nnh_set_stream_numerics(s1, NNH_NUMERICS_DEFAULT), OK);
	EXPECT(nnh_set_numerics(NNH_NUMERICS_NNCPP), OK);
	// the queries answer for both modes whatever the default: 64 x 64 x 4096 takes 32 pieces of partials in nn-cpp's
	// mode, none in the split mode (16 pieces, one launch)
	size_t q0 = 0, q1 = 0;
	EXPECT(nnh_sgemm_workspace_size(64, 64, 4096, 1, &q0), OK);
	EXPECT(nnh_set_numerics(NNH_NUMERICS_SPLIT_DEPTH), OK);
	EXPECT(nnh_sgemm_workspace_size(64, 64, 4096, 1, &q1), OK);
	EXPECT(nnh_set_numerics(NNH_NUMERICS_NNCPP), OK);
	EXPECT(q0 == 32u * 64 * 64 * 4 && q1 == q0 ? OK : INV, OK);
	EXPECT(nnh_set_workspace(nullptr, nullptr, 64), INV);
	EXPECT(nnh_set_workspace(nullptr, c.data(), 64), HIP);
	EXPECT(nnh_version() ? OK : INV, OK);
}

void elem() {
	auto a = buf(64), b = buf(64), y = buf(64), th = buf(64);
	std::vector<int> rows(8, 0);
	EXPECT(nnh_add_forward(a.data(), b.data(), 4, 16, y.data(), nullptr), HIP);
	EXPECT(nnh_add_forward(a.data(), b.data(), 4, 16, a.data(), nullptr), HIP);
	EXPECT(nnh_add_forward(a.data(), b.data(), 4, 16, a.data() + 1, nullptr), ALIAS);
	EXPECT(nnh_add_forward(a.data(), b.data(), 4, 16, b.data(), nullptr), ALIAS);
	EXPECT(nnh_add_forward(a.data(), b.data(), kHuge, kHuge, y.data(), nullptr), INV);
	EXPECT(nnh_add_forward(nullptr, nullptr, 0, 16, nullptr, nullptr), OK);
	EXPECT(nnh_add_forward(a.data(), nullptr, 4, 16, y.data(), nullptr), INV);
	EXPECT(nnh_gelu_forward(a.data(), 64, y.data(), th.data(), nullptr), HIP);
	EXPECT(nnh_gelu_forward(a.data(), 64, y.data(), y.data(), nullptr), ALIAS);
	EXPECT(nnh_gelu_forward(a.data(), 64, a.data(), th.data(), nullptr), ALIAS);
	EXPECT(nnh_gelu_forward(a.data(), 64, y.data(), nullptr, nullptr), INV);
	EXPECT(nnh_gelu_forward(nullptr, 0, nullptr, nullptr, nullptr), OK);
	EXPECT(nnh_gelu_backward(a.data(), th.data(), b.data(), 64, y.data(), 1, nullptr), HIP);
	EXPECT(nnh_gelu_backward(a.data(), th.data(), b.data(), 64, b.data(), 1, nullptr), HIP);
	EXPECT(nnh_gelu_backward(a.data(), th.data(), b.data(), 64, th.data(), 1, nullptr), ALIAS);
	EXPECT(nnh_gelu_backward(a.data(), th.data(), b.data(), 64, b.data() + 2, 1, nullptr), ALIAS);
	EXPECT(nnh_gelu_backward(a.data(), th.data(), b.data(), kHuge, y.data(), 1, nullptr), INV);
	EXPECT(nnh_embedding_forward(a.data(), 8, 8, rows.data(), 8, y.data(), nullptr), HIP);
	EXPECT(nnh_embedding_forward(a.data(), 0, 8, rows.data(), 8, y.data(), nullptr), SHAPE);
	EXPECT(nnh_embedding_forward(a.data(), 8, 8, rows.data(), 8, a.data(), nullptr), ALIAS);
	EXPECT(nnh_embedding_forward(a.data(), 8, 8, nullptr, 8, y.data(), nullptr), INV);
	EXPECT(nnh_embedding_forward(a.data(), 8, 8, rows.data(), kHuge, y.data(), nullptr), INV);
	EXPECT(nnh_embedding_forward(a.data(), 8, 8, rows.data(), 0, y.data(), nullptr), OK);
	EXPECT(nnh_embedding_backward(b.data(), rows.data(), 8, 8, 8, y.data(), 1, nullptr), HIP);
	EXPECT(nnh_embedding_backward(b.data(), rows.data(), 8, 8, 8, b.data(), 1, nullptr), ALIAS);
	EXPECT(nnh_embedding_backward(b.data(), rows.data(), 8, 8, 8, nullptr, 1, nullptr), INV);
	EXPECT(nnh_embedding_backward(b.data(), rows.data(), 8, kHuge, kHuge, y.data(), 1, nullptr), INV);
	EXPECT(nnh_embedding_backward(nullptr, nullptr, 0, 8, 8, y.data(), 1, nullptr), HIP);
	float* bufs[3] = {a.data(), b.data(), y.data()};
	size_t counts[3] = {64, 64, 64};
	EXPECT(nnh_zero_many(bufs, counts, 3, nullptr), HIP);
	EXPECT(nnh_zero_many(nullptr, nullptr, 0, nullptr), OK);
	EXPECT(nnh_zero_many(nullptr, counts, 3, nullptr), INV);
	float* overlap[2] = {a.data(), a.data() + 10};
	EXPECT(nnh_zero_many(overlap, counts, 2, nullptr), ALIAS);
	float* withnull[2] = {a.data(), nullptr};
	EXPECT(nnh_zero_many(withnull, counts, 2, nullptr), INV);
	size_t huge[2] = {kHuge, 1};
	EXPECT(nnh_zero_many(bufs, huge, 2, nullptr), INV);
}

}  // namespace

int main() {
	int devices = 0;
	if (hipGetDeviceCount(&devices) == hipSuccess && devices > 0) {
		std::printf("skipped: a GPU is visible (this test passes host buffers where device pointers belong)\n");
		return 77;
	}
	gemm();
	norm();
	elem();
	sizes();
	matmul();
	linear_relu();
	attention();
	conv_pool();
	misc();
	if (g_failures) {
		std::fprintf(stderr, "%d of %d calls returned an unexpected code\n", g_failures, g_calls);
		return 1;
	}
	std::printf("abi validation: %d calls, every code as expected\n", g_calls);
	return 0;
}
