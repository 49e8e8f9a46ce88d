// ref_shim.cpp - a C ABI over nn-cpp's own C++ API, compiled together with the reference's
// unmodified sources (read in place under /root/reference by oracle/Makefile) into
// oracle/_ref/libnnref.so. TEST INFRASTRUCTURE ONLY: the checker and the CPU baseline.
//
// Every entry point copies host buffers into nn::Tensor / nn::Value, calls the reference op and
// copies the result back. Gradients are obtained with loss = sum(y * G) so that the op's backward
// rule receives exactly G (sum's backward gives ones, mul's gives 1 * G).
// Return codes: 0 ok, 2 TensorShapeError (or another shape/argument exception), 1 anything else.
#include "nn/autograd/ops.hpp"
#include "nn/autograd/value.hpp"
#include "nn/kernels/gemm.hpp"
#include "nn/kernels/parallel.hpp"
#include "nn/tensor.hpp"

#include <cstring>
#include <exception>
#include <stdexcept>
#include <vector>

using nn::Tensor;
using nn::Value;

namespace {

Tensor make(const float* p, std::vector<size_t> shape) {
	size_t n = 1;
	for (size_t d : shape) n *= d;
	std::vector<float> v(p, p + n);
	return Tensor(std::move(shape), std::move(v));
}

void put(const Tensor& t, float* out) {
	if (t.size()) std::memcpy(out, t.data().data(), t.size() * sizeof(float));
}

std::vector<size_t> shape_of(const size_t* s, int nd) { return std::vector<size_t>(s, s + nd); }

template <typename F>
int guard(F f) {
	try {
		f();
		return 0;
	} catch (const nn::TensorShapeError&) {
		return 2;
	} catch (const std::invalid_argument&) {
		return 2;
	} catch (...) {
		return 1;
	}
}

// loss = sum(y * G): the backward of y's producer receives G
Value probe_loss(const Value& y, const float* g) {
	Value gv = Value::leaf(make(g, y.data().shape()), false);
	return nn::sum(nn::mul(y, gv));
}

}  // namespace

extern "C" {

void nnref_set_threads(size_t n) { nn::kernels::set_num_threads(n); }
size_t nnref_num_threads(void) { return nn::kernels::num_threads(); }
int nnref_uses_avx2(void) { return nn::kernels::sgemm_uses_avx2() ? 1 : 0; }

void nnref_sgemm(int ta, int tb, size_t m, size_t n, size_t k, const float* a, size_t lda, const float* b,
		size_t ldb, float* c, size_t ldc, int accumulate) {
	nn::kernels::sgemm(ta != 0, tb != 0, m, n, k, a, lda, b, ldb, c, ldc, accumulate != 0);
}

// nn::matmul(a, b, ta, tb) (src/tensor.cpp:571-641). out must hold the result; its shape is returned.
int nnref_matmul(const float* a, const size_t* as, int an, const float* b, const size_t* bs, int bn, int ta,
		int tb, float* out, size_t out_cap, size_t* out_shape, int* out_ndim) {
	return guard([&] {
		Tensor r = nn::matmul(make(a, shape_of(as, an)), make(b, shape_of(bs, bn)), ta != 0, tb != 0);
		if (r.size() > out_cap) throw std::runtime_error("capacity");
		*out_ndim = static_cast<int>(r.ndim());
		for (size_t i = 0; i < r.ndim(); ++i) out_shape[i] = r.shape()[i];
		put(r, out);
	});
}

// nn::linear forward (src/autograd/ops.cpp:714-730); x has shape xs (last dim K).
int nnref_linear_forward(const float* x, const size_t* xs, int xn, const float* w, size_t n, const float* bias,
		float* y) {
	return guard([&] {
		const size_t K = xs[xn - 1];
		nn::NoGradGuard ng;
		Value r = nn::linear(Value::leaf(make(x, shape_of(xs, xn))), Value::leaf(make(w, {n, K})),
			Value::leaf(make(bias, {n})));
		put(r.data(), y);
	});
}

// nn::linear backward with upstream gradient g (ops.cpp:731-744). Leaves start with zero gradients,
// exactly as in a training step after zero_grad().
int nnref_linear_backward(const float* x, const size_t* xs, int xn, const float* w, size_t n, const float* bias,
		const float* g, float* dx, float* dw, float* db) {
	return guard([&] {
		const size_t K = xs[xn - 1];
		Value xv = Value::leaf(make(x, shape_of(xs, xn)), true);
		Value wv = Value::leaf(make(w, {n, K}), true);
		Value bv = Value::leaf(make(bias, {n}), true);
		probe_loss(nn::linear(xv, wv, bv), g).backward();
		put(xv.grad(), dx);
		put(wv.grad(), dw);
		put(bv.grad(), db);
	});
}

// nn::conv2d_relu / nn::conv2d forward (ops.cpp:1345-1472).
int nnref_conv2d_forward(const float* x, size_t N, size_t Cin, size_t H, size_t W, const float* w, size_t Cout,
		size_t kh, size_t kw, const float* bias, int stride, int padding, int fuse_relu, float* y) {
	return guard([&] {
		nn::NoGradGuard ng;
		Value xv = Value::leaf(make(x, {N, Cin, H, W})), wv = Value::leaf(make(w, {Cout, Cin, kh, kw}));
		Value bv = Value::leaf(make(bias, {Cout}));
		Value r = fuse_relu ? nn::conv2d_relu(xv, wv, bv, stride, padding) : nn::conv2d(xv, wv, bv, stride, padding);
		put(r.data(), y);
	});
}

int nnref_conv2d_backward(const float* x, size_t N, size_t Cin, size_t H, size_t W, const float* w, size_t Cout,
		size_t kh, size_t kw, const float* bias, int stride, int padding, int fuse_relu, const float* g, float* dx,
		float* dw, float* db) {
	return guard([&] {
		Value xv = Value::leaf(make(x, {N, Cin, H, W}), true), wv = Value::leaf(make(w, {Cout, Cin, kh, kw}), true);
		Value bv = Value::leaf(make(bias, {Cout}), true);
		Value r = fuse_relu ? nn::conv2d_relu(xv, wv, bv, stride, padding) : nn::conv2d(xv, wv, bv, stride, padding);
		probe_loss(r, g).backward();
		put(xv.grad(), dx);
		put(wv.grad(), dw);
		put(bv.grad(), db);
	});
}

// nn::attention forward (ops.cpp:1226-1261); pad may be null (no key padding mask).
int nnref_attention_forward(const float* q, const float* k, const float* v, size_t N, size_t Tq, size_t Tk,
		size_t D, size_t heads, const float* pad, int causal, float* out) {
	return guard([&] {
		nn::NoGradGuard ng;
		Tensor mask = pad ? make(pad, {N, Tk}) : Tensor::empty({0});
		Value r = nn::attention(Value::leaf(make(q, {N, Tq, D})), Value::leaf(make(k, {N, Tk, D})),
			Value::leaf(make(v, {N, Tk, D})), heads, mask, causal != 0);
		put(r.data(), out);
	});
}

// nn::scaled_masked_softmax forward (ops.cpp:1298-1322) over {N, H, Tq, Tk}.
int nnref_scaled_masked_softmax(const float* x, size_t N, size_t H, size_t Tq, size_t Tk, float scale_by,
		const float* pad, int causal, float* y) {
	return guard([&] {
		nn::NoGradGuard ng;
		Tensor mask = pad ? make(pad, {N, Tk}) : Tensor::empty({0});
		Value r = nn::scaled_masked_softmax(Value::leaf(make(x, {N, H, Tq, Tk})), scale_by, mask, causal != 0);
		put(r.data(), y);
	});
}

int nnref_attention_backward(const float* q, const float* k, const float* v, size_t N, size_t Tq, size_t Tk,
		size_t D, size_t heads, const float* pad, int causal, const float* g, float* dq, float* dk, float* dv) {
	return guard([&] {
		Tensor mask = pad ? make(pad, {N, Tk}) : Tensor::empty({0});
		Value qv = Value::leaf(make(q, {N, Tq, D}), true), kv = Value::leaf(make(k, {N, Tk, D}), true);
		Value vv = Value::leaf(make(v, {N, Tk, D}), true);
		probe_loss(nn::attention(qv, kv, vv, heads, mask, causal != 0), g).backward();
		put(qv.grad(), dq);
		put(kv.grad(), dk);
		put(vv.grad(), dv);
	});
}

}  // extern "C"
