// ref_shim.cpp - a C ABI over nn-cpp's own C++ API, compiled together with the reference's
// unmodified sources (read in place under /root/reference by oracle/Makefile) into
// oracle/_ref/libnnref.so. TEST INFRASTRUCTURE ONLY: the checker and the CPU baseline.
//
// Every entry point copies host buffers into nn::Tensor / nn::Value, calls the reference op and
// copies the result back. Gradients come either from loss = sum(y * G), so that the op's backward rule receives
// exactly G (sum's backward gives ones, mul's gives 1 * G), or from the op's backward rule called directly with G
// on fresh leaf gradients (run_backward_rule, what Value::backward runs for that node); the nnref_time_* entry
// points time the forward and that backward rule separately, as the reference's runner times a step.
// Return codes: 0 ok, 2 TensorShapeError (or another shape/argument exception), 1 anything else.
#include "nn/autograd/ops.hpp"
#include "nn/autograd/value.hpp"
#include "nn/kernels/gemm.hpp"
#include "nn/nn/activation.hpp"
#include "nn/nn/attention.hpp"
#include "nn/nn/conv2d.hpp"
#include "nn/nn/dropout.hpp"
#include "nn/nn/flatten.hpp"
#include "nn/nn/linear.hpp"
#include "nn/nn/pool2d.hpp"
#include "nn/nn/sequential.hpp"
#include "nn/nn/transformer.hpp"
#include "nn/random.hpp"
#include "nn/kernels/parallel.hpp"
#include "nn/tensor.hpp"

#include <chrono>
#include <cstring>
#include <exception>
#include <memory>
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

using Clock = std::chrono::steady_clock;

// apps/bench/runner.cpp's method: `warmup` untimed calls, then timed calls (steady_clock, milliseconds) until
// max_runs of them or budget_s seconds of them, at least one. Returns the number of timed runs.
template <typename F>
int time_runs(F fn, int warmup, int max_runs, double budget_s, double* times) {
	for (int i = 0; i < warmup; ++i) fn();
	int n = 0;
	const auto start = Clock::now();
	while (n < max_runs) {
		const auto t0 = Clock::now();
		fn();
		const auto t1 = Clock::now();
		times[n++] = std::chrono::duration<double, std::milli>(t1 - t0).count();
		if (std::chrono::duration<double>(t1 - start).count() >= budget_s) break;
	}
	return n;
}

// The backward rule of node y alone (what Value::backward runs for it), with every leaf's gradient fresh, as a
// call with *_first set on the GPU side: the rule overwrites instead of adding.
void run_backward_rule(const Value& y, const Tensor& g, std::initializer_list<const Value*> leaves) {
	for (const Value* v : leaves) v->impl()->grad_fresh = true;
	y.impl()->backward_fn(g);
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

// The alternate kernels of include/nn/kernels/gemm.hpp:61-94 (in libnnref_hip.so they are the GPU drop-in's).
void nnref_sgemm_portable(int ta, int tb, size_t m, size_t n, size_t k, const float* a, size_t lda, const float* b,
		size_t ldb, float* c, size_t ldc, int accumulate) {
	nn::kernels::sgemm_portable(ta != 0, tb != 0, m, n, k, a, lda, b, ldb, c, ldc, accumulate != 0);
}
void nnref_sgemm_unpacked(int ta, int tb, size_t m, size_t n, size_t k, const float* a, size_t lda, const float* b,
		size_t ldb, float* c, size_t ldc, int accumulate) {
	nn::kernels::sgemm_unpacked(ta != 0, tb != 0, m, n, k, a, lda, b, ldb, c, ldc, accumulate != 0);
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

// nn::maxpool2d (ops.cpp:1609-1705) on {N, C, H, W}: the forward output, then (when g is not null) the input
// gradient for upstream gradient g, through the op's own backward rule with a fresh gradient.
int nnref_maxpool2d(const float* x, size_t N, size_t C, size_t H, size_t W, size_t kernel, size_t stride, float* y,
		const float* g, float* dx) {
	return guard([&] {
		const Value xv = Value::leaf(make(x, {N, C, H, W}), true);
		const Value r = nn::maxpool2d(xv, kernel, stride);
		put(r.data(), y);
		if (g) {
			run_backward_rule(r, make(g, r.data().shape()), {&xv});
			put(xv.grad(), dx);
		}
	});
}

// The backward rule of nn::matmul(a, b) (bt = 0) or nn::matmul_bt(a, b) (bt = 1) for upstream gradient g, applied
// `repeats` times: first into fresh gradients, then added (ops.cpp:683-712, 747-773). da, db receive the gradients.
int nnref_matmul_backward(const float* a, const size_t* as, int an, const float* b, const size_t* bs, int bn, int bt,
		const float* g, int repeats, float* da, float* db) {
	return guard([&] {
		// b null: the second operand is a itself (one node, both gradients into one buffer, written to da)
		const Value av = Value::leaf(make(a, shape_of(as, an)), true);
		const Value bv = b ? Value::leaf(make(b, shape_of(bs, bn)), true) : av;
		const Value r = bt ? nn::matmul_bt(av, bv) : nn::matmul(av, bv);
		const Tensor gt = make(g, r.data().shape());
		run_backward_rule(r, gt, {&av, &bv});
		for (int i = 1; i < repeats; ++i) r.impl()->backward_fn(gt);
		put(av.grad(), da);
		if (b) put(bv.grad(), db);
	});
}

// ---- graphs composed from nn-cpp's ops: the counterparts of tests/cpp/nn_hip_harness.cpp, on the CPU ----
// Leaves start with zero gradients (Value::leaf allocates them zeroed), the backward pass is seeded with g through
// probe_loss, exactly as the harness seeds its Value::backward.

Value leaf_of(const float* p, std::vector<size_t> shape) { return Value::leaf(make(p, std::move(shape)), true); }

int nnref_cnn_step(const float* x, size_t N, size_t c0, size_t side, size_t c1, size_t c2, size_t hidden,
		size_t classes, const float* w1, const float* b1, const float* w2, const float* b2, const float* w3,
		const float* b3, const float* w4, const float* b4, const float* g, float* logits, float* dx, float* dw1,
		float* db1, float* dw2, float* db2, float* dw3, float* db3, float* dw4, float* db4) {
	return guard([&] {
		const size_t flat = c2 * (side / 4) * (side / 4);
		const Value xv = leaf_of(x, {N, c0, side, side});
		const Value W1 = leaf_of(w1, {c1, c0, 3, 3}), B1 = leaf_of(b1, {c1}), W2 = leaf_of(w2, {c2, c1, 3, 3});
		const Value B2 = leaf_of(b2, {c2}), W3 = leaf_of(w3, {hidden, flat}), B3 = leaf_of(b3, {hidden});
		const Value W4 = leaf_of(w4, {classes, hidden}), B4 = leaf_of(b4, {classes});
		Value h = nn::maxpool2d(nn::conv2d_relu(xv, W1, B1, 1, 1), 2, 2);
		h = nn::maxpool2d(nn::conv2d_relu(h, W2, B2, 1, 1), 2, 2);
		h = nn::reshape(h, {N, flat});
		const Value y = nn::linear(nn::relu(nn::linear(h, W3, B3)), W4, B4);
		probe_loss(y, g).backward();
		put(y.data(), logits);
		put(xv.grad(), dx);
		put(W1.grad(), dw1);
		put(B1.grad(), db1);
		put(W2.grad(), dw2);
		put(B2.grad(), db2);
		put(W3.grad(), dw3);
		put(B3.grad(), db3);
		put(W4.grad(), dw4);
		put(B4.grad(), db4);
	});
}

int nnref_mlp_step(const float* x, size_t M, const size_t* dims, int layers, const float* const* w,
		const float* const* b, const float* g, float* y, float* dx, float* const* dw, float* const* db) {
	return guard([&] {
		const Value xv = leaf_of(x, {M, dims[0]});
		std::vector<Value> W, B;
		Value h = xv;
		for (int i = 0; i < layers; ++i) {
			W.push_back(leaf_of(w[i], {dims[i + 1], dims[i]}));
			B.push_back(leaf_of(b[i], {dims[i + 1]}));
			h = nn::linear(h, W[i], B[i]);
			if (i + 1 < layers) h = nn::relu(h);
		}
		probe_loss(h, g).backward();
		put(h.data(), y);
		put(xv.grad(), dx);
		for (int i = 0; i < layers; ++i) {
			put(W[i].grad(), dw[i]);
			put(B[i].grad(), db[i]);
		}
	});
}

int nnref_matmul_chain(const float* a, const size_t* as, const float* b, const size_t* bs, const float* c,
		const size_t* cs, const float* g, float* y, float* da, float* db, float* dc) {
	return guard([&] {
		const Value A = leaf_of(a, {as[0], as[1], as[2]}), B = leaf_of(b, {bs[0], bs[1], bs[2]});
		const Value Cv = leaf_of(c, {cs[0], cs[1]});
		const Value r = nn::matmul_bt(nn::matmul(A, B), Cv);
		probe_loss(r, g).backward();
		put(r.data(), y);
		put(A.grad(), da);
		put(B.grad(), db);
		put(Cv.grad(), dc);
	});
}

int nnref_self_attention(const float* x, size_t N, size_t T, size_t D, size_t heads, int causal, const float* g,
		float* o, float* dx) {
	return guard([&] {
		const Value xv = leaf_of(x, {N, T, D});
		const Value r = nn::attention(xv, xv, xv, heads, Tensor::empty({0}), causal != 0);
		probe_loss(r, g).backward();
		put(r.data(), o);
		put(xv.grad(), dx);
	});
}

int nnref_softmax_step(const float* x, size_t N, size_t H, size_t Tq, size_t Tk, float scale, const float* pad,
		int causal, const float* g, float* y, float* dx) {
	return guard([&] {
		const Value xv = leaf_of(x, {N, H, Tq, Tk});
		const Tensor mask = pad ? make(pad, {N, Tk}) : Tensor::empty({0});
		const Value r = nn::scaled_masked_softmax(xv, scale, mask, causal != 0);
		probe_loss(r, g).backward();
		put(r.data(), y);
		put(xv.grad(), dx);
	});
}

// A Conv-BN-ReLU stack with a layer-normalised head (the ops of nn-cpp's cnn_fer and transformer models):
// conv2d(c0 -> c1, 3x3, pad 1) -> batchnorm + ReLU folded -> maxpool2d(2, 2) -> conv2d(c1 -> c2) -> batchnorm ->
// relu -> reshape {N, flat} -> layernorm -> linear(classes); then the backward pass from the output gradient g.
// p: w1, b1, bn1 weight, bn1 bias, w2, b2, bn2 weight, bn2 bias, ln gamma, ln beta, w3, b3; grads likewise, then dx.
int nnref_norm_step(const float* x, size_t N, size_t c0, size_t side, size_t c1, size_t c2, size_t classes,
		const float* const* p, const float* g, float* y, float* const* grads, float* dx) {
	return guard([&] {
		const size_t flat = c2 * (side / 2) * (side / 2);
		const Value xv = leaf_of(x, {N, c0, side, side});
		const std::vector<std::vector<size_t>> shapes = {{c1, c0, 3, 3}, {c1}, {c1}, {c1}, {c2, c1, 3, 3}, {c2}, {c2},
		                                                 {c2}, {flat}, {flat}, {classes, flat}, {classes}};
		std::vector<Value> v;
		for (size_t i = 0; i < shapes.size(); ++i) v.push_back(leaf_of(p[i], shapes[i]));
		Value h = nn::batchnorm(nn::conv2d(xv, v[0], v[1], 1, 1), v[2], v[3], 1e-5f, nullptr, nullptr, true);
		h = nn::maxpool2d(h, 2, 2);
		h = nn::relu(nn::batchnorm(nn::conv2d(h, v[4], v[5], 1, 1), v[6], v[7], 1e-5f));
		h = nn::layernorm(nn::reshape(h, {N, flat}), v[8], v[9], 1e-5f);
		const Value r = nn::linear(h, v[10], v[11]);
		probe_loss(r, g).backward();
		put(r.data(), y);
		for (size_t i = 0; i < v.size(); ++i) put(v[i].grad(), grads[i]);
		put(xv.grad(), dx);
	});
}

// ---- nn-cpp's modules, unchanged (src/nn/*.cpp): the callers of the path ----
// Builds model `which` after nn::manual_seed(seed) (so parameters come from the modules' own initialisation),
// runs forward on x, seeds the backward pass with g through probe_loss, and returns the output (out, n_out floats)
// and, concatenated in parameters() order followed by x's, every gradient (grads, n_grads floats).
//   0: nn-cpp's cnn_mnist (apps/bench/workloads.cpp:113-137): Sequential of Conv2d(1,8,3,1,1), ReLU, MaxPool2d(2,2),
//      Conv2d(8,16,3,1,1), ReLU, MaxPool2d(2,2), Flatten, Linear(784,128), ReLU, Linear(128,10); Sequential folds
//      each Conv2d + ReLU into conv2d_relu (src/nn/sequential.cpp:16-28).
//   1: MultiHeadAttention(64, 4 heads, causal), no dropout: the fused attention op (src/nn/attention.cpp:33-35).
//   2: MultiHeadAttention(64, 4 heads) with dropout 0.1 in training mode: the composed path through matmul_bt,
//      scaled_masked_softmax, dropout and a batched matmul (attention.cpp:36-47).
//   3: Sequential of Linear(20,30), ReLU, Linear(30,5) on a 3-D input (Linear is not folded with ReLU).
//   4: Transformer{vocab 11, dim 16, heads 2, layers 2, max_len 12, mlp_ratio 2, dropout 0, causal, learned
//      positions} on float ids x (x's gradient stays zero: ids are not differentiated).
//   5: Sequential of Linear(20,30), Dropout(0.25) in training mode, ReLU, Linear(30,5).
//   6: Transformer{vocab 13, dim 24, heads 3, layers 1, max_len 9, mlp_ratio 4, dropout 0.1, non-causal, sinusoidal
//      positions} in evaluation mode.
int nnref_module_run(int which, unsigned seed, const float* x, const size_t* xs, int xn, const float* g, float* out,
		size_t out_cap, float* grads, size_t grads_cap, size_t* n_out, size_t* n_grads) {
	return guard([&] {
		nn::manual_seed(seed);
		std::unique_ptr<nn::Module> m;
		if (which == 0) {
			auto s = std::make_unique<nn::Sequential>();
			s->add(std::make_unique<nn::Conv2d>(1, 8, 3, 1, 1));
			s->add(std::make_unique<nn::ReLU>());
			s->add(std::make_unique<nn::MaxPool2d>(2, 2));
			s->add(std::make_unique<nn::Conv2d>(8, 16, 3, 1, 1));
			s->add(std::make_unique<nn::ReLU>());
			s->add(std::make_unique<nn::MaxPool2d>(2, 2));
			s->add(std::make_unique<nn::Flatten>());
			s->add(std::make_unique<nn::Linear>(784, 128));
			s->add(std::make_unique<nn::ReLU>());
			s->add(std::make_unique<nn::Linear>(128, 10));
			m = std::move(s);
		} else if (which == 1) {
			m = std::make_unique<nn::MultiHeadAttention>(64, 4, true);
		} else if (which == 2) {
			m = std::make_unique<nn::MultiHeadAttention>(64, 4, false, 0.1f);
			m->train(true);
		} else if (which == 3) {
			auto s = std::make_unique<nn::Sequential>();
			s->add(std::make_unique<nn::Linear>(20, 30));
			s->add(std::make_unique<nn::ReLU>());
			s->add(std::make_unique<nn::Linear>(30, 5));
			m = std::move(s);
		} else if (which == 4) {
			m = std::make_unique<nn::Transformer>(nn::TransformerConfig{11, 16, 2, 2, 12, 2, 0.0f, true, true});
		} else if (which == 5) {
			auto s = std::make_unique<nn::Sequential>();
			s->add(std::make_unique<nn::Linear>(20, 30));
			s->add(std::make_unique<nn::Dropout>(0.25f));
			s->add(std::make_unique<nn::ReLU>());
			s->add(std::make_unique<nn::Linear>(30, 5));
			m = std::move(s);
			m->train(true);
		} else {
			m = std::make_unique<nn::Transformer>(nn::TransformerConfig{13, 24, 3, 1, 9, 4, 0.1f, false, false});
			m->eval();
		}
		const Value xv = Value::leaf(make(x, shape_of(xs, xn)), true);
		const Value y = m->forward(xv);
		probe_loss(y, g).backward();
		if (y.data().size() > out_cap) throw std::runtime_error("capacity");
		put(y.data(), out);
		*n_out = y.data().size();
		size_t off = 0;
		std::vector<Value> ps = m->parameters();
		ps.push_back(xv);
		for (const Value& p : ps) {
			if (off + p.grad().size() > grads_cap) throw std::runtime_error("capacity");
			put(p.grad(), grads + off);
			off += p.grad().size();
		}
		*n_grads = off;
	});
}

// n draws of nn::derive_generator(stream) after nn::manual_seed(seed), the k-th generator of the stream for k = 0 ..
// gens - 1 in turn (n / gens draws each): the seeding the module layer's initial values come from.
int nnref_random_draws(unsigned long long seed, const char* stream, int gens, size_t n, unsigned* out) {
	return guard([&] {
		nn::manual_seed(seed);
		size_t o = 0;
		for (int k = 0; k < gens; ++k) {
			std::mt19937 gen = nn::derive_generator(stream);
			for (size_t i = 0; i < n / gens; ++i) out[o++] = static_cast<unsigned>(gen());
		}
	});
}

// ---- timing (the CPU baseline): each returns the number of timed runs, or -1 on an exception ----

// nn::matmul(a, b, ta, tb) (src/tensor.cpp:571-641) on Tensors built once, as run_matmul (runner.cpp:80-96);
// out receives the last result.
int nnref_time_matmul(const float* a, const size_t* as, int an, const float* b, const size_t* bs, int bn, int ta,
		int tb, int warmup, int max_runs, double budget_s, double* times, float* out) {
	int runs = -1;
	guard([&] {
		const Tensor A = make(a, shape_of(as, an)), B = make(b, shape_of(bs, bn));
		Tensor r = Tensor::empty({0});
		runs = time_runs([&] { r = nn::matmul(A, B, ta != 0, tb != 0); }, warmup, max_runs, budget_s, times);
		put(r, out);
	});
	return runs;
}

// A chain of `layers` nn::linear + nn::relu (ops.cpp:714-793) without a graph, x {M, dims[0]}, w[i] {dims[i+1],
// dims[i]}, b[i] {dims[i+1]}; outs[i] receives layer i's activation.
int nnref_time_linear_relu_chain(const float* x, size_t M, const size_t* dims, int layers, const float* const* w,
		const float* const* b, int warmup, int max_runs, double budget_s, double* times, float* const* outs) {
	int runs = -1;
	guard([&] {
		nn::NoGradGuard ng;
		const Value xv = Value::leaf(make(x, {M, dims[0]}));
		std::vector<Value> wv, bv, hs(layers, Value::leaf(Tensor::empty({0})));
		for (int i = 0; i < layers; ++i) {
			wv.push_back(Value::leaf(make(w[i], {dims[i + 1], dims[i]})));
			bv.push_back(Value::leaf(make(b[i], {dims[i + 1]})));
		}
		runs = time_runs([&] {
			Value h = xv;
			for (int i = 0; i < layers; ++i) hs[i] = h = nn::relu(nn::linear(h, wv[i], bv[i]));
		}, warmup, max_runs, budget_s, times);
		for (int i = 0; i < layers; ++i) put(hs[i].data(), outs[i]);
	});
	return runs;
}

// The backward rules of `layers` independent nn::linear nodes (ops.cpp:731-744): layer i has input x[i] {M, dims[i]},
// weight w[i] {dims[i+1], dims[i]}, bias b[i] and upstream gradient g[i] {M, dims[i+1]}; fresh leaf gradients.
// dx[i], dw[i], db[i] receive the last run's gradients.
int nnref_time_linear_backward_layers(const float* const* x, size_t M, const size_t* dims, int layers,
		const float* const* w, const float* const* b, const float* const* g, int warmup, int max_runs,
		double budget_s, double* times, float* const* dx, float* const* dw, float* const* db) {
	int runs = -1;
	guard([&] {
		std::vector<Value> xv, wv, bv, ys;
		std::vector<Tensor> gs;
		for (int i = 0; i < layers; ++i) {
			xv.push_back(Value::leaf(make(x[i], {M, dims[i]}), true));
			wv.push_back(Value::leaf(make(w[i], {dims[i + 1], dims[i]}), true));
			bv.push_back(Value::leaf(make(b[i], {dims[i + 1]}), true));
			ys.push_back(nn::linear(xv[i], wv[i], bv[i]));
			gs.push_back(make(g[i], {M, dims[i + 1]}));
		}
		runs = time_runs([&] {
			for (int i = 0; i < layers; ++i) run_backward_rule(ys[i], gs[i], {&xv[i], &wv[i], &bv[i]});
		}, warmup, max_runs, budget_s, times);
		for (int i = 0; i < layers; ++i) {
			put(xv[i].grad(), dx[i]);
			put(wv[i].grad(), dw[i]);
			put(bv[i].grad(), db[i]);
		}
	});
	return runs;
}

// nn::conv2d_relu / nn::conv2d (ops.cpp:1345-1472): the forward without a graph (times_fwd, y), then the node's
// backward rule for upstream gradient g with fresh leaf gradients (times_bwd, dx, dw, db).
int nnref_time_conv2d(const float* x, size_t N, size_t Cin, size_t H, size_t W, const float* w, size_t Cout,
		size_t kh, size_t kw, const float* bias, int stride, int padding, int fuse_relu, const float* g, int warmup,
		int max_runs, double budget_s, double* times_fwd, int* runs_fwd, double* times_bwd, float* y, float* dx,
		float* dw, float* db) {
	int runs = -1;
	guard([&] {
		const Value xv = Value::leaf(make(x, {N, Cin, H, W}), true), wv = Value::leaf(make(w, {Cout, Cin, kh, kw}), true);
		const Value bv = Value::leaf(make(bias, {Cout}), true);
		auto op = [&] { return fuse_relu ? nn::conv2d_relu(xv, wv, bv, stride, padding) : nn::conv2d(xv, wv, bv, stride, padding); };
		{
			nn::NoGradGuard ng;
			Value r = Value::leaf(Tensor::empty({0}));
			*runs_fwd = time_runs([&] { r = op(); }, warmup, max_runs, budget_s, times_fwd);
			put(r.data(), y);
		}
		if (!g) {
			runs = 0;
			return;
		}
		const Value r = op();
		const Tensor gt = make(g, r.data().shape());
		runs = time_runs([&] { run_backward_rule(r, gt, {&xv, &wv, &bv}); }, warmup, max_runs, budget_s, times_bwd);
		put(xv.grad(), dx);
		put(wv.grad(), dw);
		put(bv.grad(), db);
	});
	return runs;
}

// nn::attention (ops.cpp:1226-1296) without a key padding mask: the forward without a graph, then the node's
// backward rule for g (when g is not null), as nnref_time_conv2d.
int nnref_time_attention(const float* q, const float* k, const float* v, size_t N, size_t T, size_t D, size_t heads,
		int causal, const float* g, int warmup, int max_runs, double budget_s, double* times_fwd, int* runs_fwd,
		double* times_bwd, float* out, float* dq, float* dk, float* dv) {
	int runs = -1;
	guard([&] {
		const Value qv = Value::leaf(make(q, {N, T, D}), true), kv = Value::leaf(make(k, {N, T, D}), true);
		const Value vv = Value::leaf(make(v, {N, T, D}), true);
		const Tensor none = Tensor::empty({0});
		{
			nn::NoGradGuard ng;
			Value r = Value::leaf(Tensor::empty({0}));
			*runs_fwd = time_runs([&] { r = nn::attention(qv, kv, vv, heads, none, causal != 0); }, warmup, max_runs,
				budget_s, times_fwd);
			put(r.data(), out);
		}
		if (!g) {
			runs = 0;
			return;
		}
		const Value r = nn::attention(qv, kv, vv, heads, none, causal != 0);
		const Tensor gt = make(g, {N, T, D});
		runs = time_runs([&] { run_backward_rule(r, gt, {&qv, &kv, &vv}); }, warmup, max_runs, budget_s, times_bwd);
		put(qv.grad(), dq);
		put(kv.grad(), dk);
		put(vv.grad(), dv);
	});
	return runs;
}

// nn::maxpool2d (ops.cpp:1609-1705): the forward without a graph, then the node's backward rule for g.
int nnref_time_maxpool2d(const float* x, size_t N, size_t C, size_t H, size_t W, size_t kernel, size_t stride,
		const float* g, int warmup, int max_runs, double budget_s, double* times_fwd, int* runs_fwd, double* times_bwd,
		float* y, float* dx) {
	int runs = -1;
	guard([&] {
		const Value xv = Value::leaf(make(x, {N, C, H, W}), true);
		{
			nn::NoGradGuard ng;
			Value r = Value::leaf(Tensor::empty({0}));
			*runs_fwd = time_runs([&] { r = nn::maxpool2d(xv, kernel, stride); }, warmup, max_runs, budget_s, times_fwd);
			put(r.data(), y);
		}
		const Value r = nn::maxpool2d(xv, kernel, stride);
		const Tensor gt = make(g, r.data().shape());
		runs = time_runs([&] { run_backward_rule(r, gt, {&xv}); }, warmup, max_runs, budget_s, times_bwd);
		put(xv.grad(), dx);
	});
	return runs;
}

// nn::batchnorm in training mode (ops.cpp:900-1001) on x {N, C, S}: y, and mean and var when not null; then, when
// g is not null, the node's backward rule `repeats` times (first into fresh gradients, then added), the gradients
// of x, weight and bias into dx, dw, db (each may be null: that input then needs no gradient).
int nnref_batchnorm(const float* x, size_t N, size_t C, size_t S, const float* w, const float* b, float eps, int relu,
		float* y, float* mean, float* var, const float* g, int repeats, float* dx, float* dw, float* db) {
	return guard([&] {
		const Value xv = Value::leaf(make(x, {N, C, S}), dx != nullptr);
		const Value wv = Value::leaf(make(w, {C}), dw != nullptr);
		const Value bv = Value::leaf(make(b, {C}), db != nullptr);
		Tensor mu({C}), va({C});
		const Value r = nn::batchnorm(xv, wv, bv, eps, &mu, &va, relu != 0);
		put(r.data(), y);
		if (mean) put(mu, mean);
		if (var) put(va, var);
		if (g) {
			const Tensor gt = make(g, r.data().shape());
			run_backward_rule(r, gt, {&xv, &wv, &bv});
			for (int i = 1; i < repeats; ++i) r.impl()->backward_fn(gt);
			if (dx) put(xv.grad(), dx);
			if (dw) put(wv.grad(), dw);
			if (db) put(bv.grad(), db);
		}
	});
}

// nn::gelu (ops.cpp:451-481) on count elements: y, then (g not null) the backward rule `repeats` times into dx.
int nnref_gelu(const float* x, size_t count, float* y, const float* g, int repeats, float* dx) {
	return guard([&] {
		const Value xv = Value::leaf(make(x, {count}), true);
		const Value r = nn::gelu(xv);
		put(r.data(), y);
		if (g) {
			const Tensor gt = make(g, {count});
			run_backward_rule(r, gt, {&xv});
			for (int i = 1; i < repeats; ++i) r.impl()->backward_fn(gt);
			put(xv.grad(), dx);
		}
	});
}

// nn::embedding (ops.cpp:1991-2015): weight {V, D}, ids (floats, as nn-cpp takes them) {count}; y, then (g not null)
// the weight gradient through the backward rule `repeats` times. Returns 2 where nn-cpp throws TensorShapeError.
int nnref_embedding(const float* w, size_t V, size_t D, const float* ids, size_t count, float* y, const float* g,
		int repeats, float* dw) {
	return guard([&] {
		const Value wv = Value::leaf(make(w, {V, D}), true);
		const Value r = nn::embedding(wv, make(ids, {count}));
		put(r.data(), y);
		if (g) {
			const Tensor gt = make(g, {count, D});
			run_backward_rule(r, gt, {&wv});
			for (int i = 1; i < repeats; ++i) r.impl()->backward_fn(gt);
			put(wv.grad(), dw);
		}
	});
}

// nn::layernorm (ops.cpp:1003-1078) over R rows of D, then its backward rule as nnref_batchnorm's.
int nnref_layernorm(const float* x, size_t R, size_t D, const float* gm, const float* bt, float eps, float* y,
		const float* g, int repeats, float* dx, float* dgamma, float* dbeta) {
	return guard([&] {
		const Value xv = Value::leaf(make(x, {R, D}), dx != nullptr);
		const Value gv = Value::leaf(make(gm, {D}), dgamma != nullptr);
		const Value bv = Value::leaf(make(bt, {D}), dbeta != nullptr);
		const Value r = nn::layernorm(xv, gv, bv, eps);
		put(r.data(), y);
		if (g) {
			const Tensor gt = make(g, r.data().shape());
			run_backward_rule(r, gt, {&xv, &gv, &bv});
			for (int i = 1; i < repeats; ++i) r.impl()->backward_fn(gt);
			if (dx) put(xv.grad(), dx);
			if (dgamma) put(gv.grad(), dgamma);
			if (dbeta) put(bv.grad(), dbeta);
		}
	});
}

// Timing of nn::batchnorm (relu folded or not) and of its backward rule, as nnref_time_maxpool2d.
int nnref_time_batchnorm(const float* x, size_t N, size_t C, size_t S, const float* w, const float* b, float eps,
		int relu, const float* g, int warmup, int max_runs, double budget_s, double* times_fwd, int* runs_fwd,
		double* times_bwd, float* y, float* dx) {
	int runs = -1;
	guard([&] {
		const Value xv = Value::leaf(make(x, {N, C, S}), true);
		const Value wv = Value::leaf(make(w, {C}), true);
		const Value bv = Value::leaf(make(b, {C}), true);
		{
			nn::NoGradGuard ng;
			Value r = Value::leaf(Tensor::empty({0}));
			*runs_fwd = time_runs([&] { r = nn::batchnorm(xv, wv, bv, eps, nullptr, nullptr, relu != 0); }, warmup,
			                      max_runs, budget_s, times_fwd);
			put(r.data(), y);
		}
		const Value r = nn::batchnorm(xv, wv, bv, eps, nullptr, nullptr, relu != 0);
		const Tensor gt = make(g, r.data().shape());
		runs = time_runs([&] { run_backward_rule(r, gt, {&xv, &wv, &bv}); }, warmup, max_runs, budget_s, times_bwd);
		put(xv.grad(), dx);
	});
	return runs;
}

// Timing of nn::layernorm and of its backward rule.
int nnref_time_layernorm(const float* x, size_t R, size_t D, const float* gm, const float* bt, float eps,
		const float* g, int warmup, int max_runs, double budget_s, double* times_fwd, int* runs_fwd,
		double* times_bwd, float* y, float* dx) {
	int runs = -1;
	guard([&] {
		const Value xv = Value::leaf(make(x, {R, D}), true);
		const Value gv = Value::leaf(make(gm, {D}), true);
		const Value bv = Value::leaf(make(bt, {D}), true);
		{
			nn::NoGradGuard ng;
			Value r = Value::leaf(Tensor::empty({0}));
			*runs_fwd = time_runs([&] { r = nn::layernorm(xv, gv, bv, eps); }, warmup, max_runs, budget_s, times_fwd);
			put(r.data(), y);
		}
		const Value r = nn::layernorm(xv, gv, bv, eps);
		const Tensor gt = make(g, r.data().shape());
		runs = time_runs([&] { run_backward_rule(r, gt, {&xv, &gv, &bv}); }, warmup, max_runs, budget_s, times_bwd);
		put(xv.grad(), dx);
	});
	return runs;
}

// transformer_tiny's parameters as nn-cpp's Transformer{64, 64, 4, 2, 64} holds them, in parameters() order: for
// each, its rank, its dimensions, and 1 when it starts at all ones (else 0). Writes at most cap values; *count
// receives the number of parameters.
int nnref_transformer_tiny_layout(size_t* out, size_t cap, size_t* count) {
	return guard([&] {
		nn::Transformer tf(nn::TransformerConfig{64, 64, 4, 2, 64});
		const std::vector<Value> ps = tf.parameters();
		*count = ps.size();
		size_t n = 0;
		auto push = [&](size_t v) {
			if (n < cap) out[n] = v;
			++n;
		};
		for (const Value& p : ps) {
			const nn::Tensor& t = p.data();
			push(t.ndim());
			for (size_t d : t.shape()) push(d);
			bool ones = true;
			for (float v : t.data()) ones = ones && v == 1.0f;
			push(ones ? 1 : 0);
		}
		if (n > cap) throw std::invalid_argument("layout buffer too small");
	});
}

// nn-cpp's side of the bench models' training step (the counterpart of nn-cpp_amd/src/bench/workloads.cpp, with
// apps/bench/runner.cpp:33-45's clock points): the forward pass, then zero_grad and the backward pass from the
// logits' gradient g; no loss, no optimizer step. Model 2 is transformer_tiny: nn-cpp's own Transformer module
// (apps/bench/workloads.cpp:80-92) with the given parameters copied in, its {N, T, V} logits flattened as
// FlatTransformer does. grads (optional) receives each parameter's gradient of the last step.
int nnref_time_workload_step(int model, const float* x, size_t N, const float* const* params, const float* g,
		int warmup, int runs, double* fwd_ms, double* bwd_ms, float* logits, float* const* grads) {
	return guard([&] {
		static const std::vector<std::vector<size_t>> mlp = {{1024, 784}, {1024}, {1024, 1024}, {1024}, {10, 1024}, {10}};
		static const std::vector<std::vector<size_t>> cnn = {{8, 1, 3, 3}, {8}, {16, 8, 3, 3}, {16}, {128, 784}, {128},
			{10, 128}, {10}};
		std::vector<Value> p;
		std::unique_ptr<nn::Transformer> tf;
		if (model == 2) {
			tf = std::make_unique<nn::Transformer>(nn::TransformerConfig{64, 64, 4, 2, 64});
			p = tf->parameters();
			for (size_t i = 0; i < p.size(); ++i) {
				nn::Tensor& t = p[i].data();
				std::memcpy(t.data().data(), params[i], t.size() * sizeof(float));
			}
		} else {
			const auto& shapes = model == 0 ? mlp : cnn;
			for (size_t i = 0; i < shapes.size(); ++i) p.push_back(Value::leaf(make(params[i], shapes[i]), true));
		}
		const std::vector<size_t> xs = model == 0 ? std::vector<size_t>{N, 784}
			: model == 2 ? std::vector<size_t>{N, 64} : std::vector<size_t>{N, 1, 28, 28};
		const Value xv = Value::leaf(make(x, xs));
		for (int i = 0; i < warmup + runs; ++i) {
			const auto t0 = Clock::now();
			Value y = Value::leaf(Tensor::empty({0}));
			if (model == 0) {
				Value h = nn::relu(nn::linear(xv, p[0], p[1]));
				h = nn::relu(nn::linear(h, p[2], p[3]));
				y = nn::linear(h, p[4], p[5]);
			} else if (model == 2) {
				const Value o = tf->forward(xv);
				const std::vector<size_t>& os = o.data().shape();
				y = nn::reshape(o, {os[0] * os[1], os[2]});
			} else {
				Value h = nn::maxpool2d(nn::conv2d_relu(xv, p[0], p[1], 1, 1), 2, 2);
				h = nn::maxpool2d(nn::conv2d_relu(h, p[2], p[3], 1, 1), 2, 2);
				h = nn::reshape(h, {N, 784});
				y = nn::linear(nn::relu(nn::linear(h, p[4], p[5])), p[6], p[7]);
			}
			const auto t1 = Clock::now();
			for (const Value& v : p) v.zero_grad();
			probe_loss(y, g).backward();
			const auto t2 = Clock::now();
			if (i >= warmup) {
				fwd_ms[i - warmup] = std::chrono::duration<double, std::milli>(t1 - t0).count();
				bwd_ms[i - warmup] = std::chrono::duration<double, std::milli>(t2 - t1).count();
			}
			if (i + 1 == warmup + runs) {
				if (logits) put(y.data(), logits);
				if (grads)
					for (size_t j = 0; j < p.size(); ++j)
						if (grads[j]) put(p[j].grad(), grads[j]);
			}
		}
	});
}

}  // extern "C"
