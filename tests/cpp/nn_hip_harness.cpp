// nn_hip_harness.cpp - TEST CODE: a C entry for each graph the tests run through include/nn_hip.hpp (nn-cpp's op
// surface on device-resident tensors), so pytest can compare them with nn-cpp's CPU build on the same host buffers
// (oracle/ref_shim.cpp composes the same graphs from nn-cpp's own ops). Inputs are copied to the device once;
// every op in between reads and writes HBM; outputs and gradients are copied back at the end.
// Return codes: 0 ok, 2 nn::hip::TensorShapeError, 1 any other exception.
#include <cstring>
#include <string>
#include <memory>
#include <stdexcept>
#include <vector>

#include "nn_hip.hpp"
#include "nn_hip_modules.hpp"

using nn::hip::Tensor;
using nn::hip::Value;

namespace {

std::string g_last_error;

template <typename F>
int guard(F f) {
	try {
		f();
		return 0;
	} catch (const nn::hip::TensorShapeError& e) {
		g_last_error = e.what();
		return 2;
	} catch (const std::exception& e) {
		g_last_error = e.what();
		return 1;
	} catch (...) {
		g_last_error = "unknown exception";
		return 1;
	}
}

Value param(const float* p, std::vector<size_t> shape) { return Value::leaf(Tensor::from_host(std::move(shape), p), true); }

void out(const Tensor& t, float* dst) {
	if (dst) t.to_host(dst);
}

}  // namespace

extern "C" {

// The message of the last exception a harness entry caught.
const char* h_last_error(void) { return g_last_error.c_str(); }

// nn-cpp's cnn_mnist model (apps/bench/workloads.cpp:113-137 with Sequential's Conv2d + ReLU folding,
// src/nn/sequential.cpp:16-28): conv2d_relu(c0 -> c1, 3x3, pad 1) -> maxpool2d(2, 2) -> conv2d_relu(c1 -> c2) ->
// maxpool2d(2, 2) -> reshape {N, c2 * (side/4)^2} -> linear(hidden) -> relu -> linear(classes); then the backward
// pass from the logits' gradient g.
static int cnn_step(bool fused, const float* x, size_t N, size_t c0, size_t side, size_t c1, size_t c2, size_t hidden,
                    size_t classes, const float* w1, const float* b1, const float* w2, const float* b2, const float* w3,
                    const float* b3, const float* w4, const float* b4, const float* g, float* logits, float* dx,
                    float* dw1, float* db1, float* dw2, float* db2, float* dw3, float* db3, float* dw4, float* db4) {
	return guard([&] {
		const size_t flat = c2 * (side / 4) * (side / 4);
		Value xv = param(x, {N, c0, side, side});
		Value W1 = param(w1, {c1, c0, 3, 3}), B1 = param(b1, {c1}), W2 = param(w2, {c2, c1, 3, 3}), B2 = param(b2, {c2});
		Value W3 = param(w3, {hidden, flat}), B3 = param(b3, {hidden}), W4 = param(w4, {classes, hidden});
		Value B4 = param(b4, {classes});
		Value h = fused ? nn::hip::conv2d_relu_maxpool2d(xv, W1, B1, 1, 1, 2, 2)
		                : nn::hip::maxpool2d(nn::hip::conv2d_relu(xv, W1, B1, 1, 1), 2, 2);
		h = fused ? nn::hip::conv2d_relu_maxpool2d(h, W2, B2, 1, 1, 2, 2)
		          : nn::hip::maxpool2d(nn::hip::conv2d_relu(h, W2, B2, 1, 1), 2, 2);
		h = nn::hip::reshape(h, {N, flat});
		Value y = nn::hip::linear(nn::hip::relu(nn::hip::linear(h, W3, B3)), W4, B4);
		y.backward(Tensor::from_host({N, classes}, g));
		out(y.data(), logits);
		out(xv.grad(), dx);
		out(W1.grad(), dw1);
		out(B1.grad(), db1);
		out(W2.grad(), dw2);
		out(B2.grad(), db2);
		out(W3.grad(), dw3);
		out(B3.grad(), db3);
		out(W4.grad(), dw4);
		out(B4.grad(), db4);
	});
}

int h_cnn_step(const float* x, size_t N, size_t c0, size_t side, size_t c1, size_t c2, size_t hidden, size_t classes,
               const float* w1, const float* b1, const float* w2, const float* b2, const float* w3, const float* b3,
               const float* w4, const float* b4, const float* g, float* logits, float* dx, float* dw1, float* db1,
               float* dw2, float* db2, float* dw3, float* db3, float* dw4, float* db4) {
	return cnn_step(false, x, N, c0, side, c1, c2, hidden, classes, w1, b1, w2, b2, w3, b3, w4, b4, g, logits, dx, dw1,
	                db1, dw2, db2, dw3, db3, dw4, db4);
}

// The same step with each conv2d_relu -> maxpool2d pair as nn::hip::conv2d_relu_maxpool2d (one pass where fusable).
int h_cnn_step_fused(const float* x, size_t N, size_t c0, size_t side, size_t c1, size_t c2, size_t hidden,
                     size_t classes, const float* w1, const float* b1, const float* w2, const float* b2, const float* w3,
                     const float* b3, const float* w4, const float* b4, const float* g, float* logits, float* dx,
                     float* dw1, float* db1, float* dw2, float* db2, float* dw3, float* db3, float* dw4, float* db4) {
	return cnn_step(true, x, N, c0, side, c1, c2, hidden, classes, w1, b1, w2, b2, w3, b3, w4, b4, g, logits, dx, dw1,
	                db1, dw2, db2, dw3, db3, dw4, db4);
}

// linear -> relu -> ... -> linear (the MLPs of apps/bench/workloads.cpp:100-107), backward from g.
int h_mlp_step(const float* x, size_t M, const size_t* dims, int layers, const float* const* w, const float* const* b,
               const float* g, float* y, float* dx, float* const* dw, float* const* db) {
	return guard([&] {
		Value xv = param(x, {M, dims[0]});
		std::vector<Value> W, B;
		Value h = xv;
		for (int i = 0; i < layers; ++i) {
			W.push_back(param(w[i], {dims[i + 1], dims[i]}));
			B.push_back(param(b[i], {dims[i + 1]}));
			h = nn::hip::linear(h, W[i], B[i]);
			if (i + 1 < layers) h = nn::hip::relu(h);
		}
		h.backward(Tensor::from_host({M, dims[layers]}, g));
		out(h.data(), y);
		out(xv.grad(), dx);
		for (int i = 0; i < layers; ++i) {
			out(W[i].grad(), dw[i]);
			out(B[i].grad(), db[i]);
		}
	});
}

// y = matmul_bt(matmul(a, b), c) for a {B, M, K}, b {B, K, N}, c {P, N}: the batched Value matmul and the folded
// matmul_bt, forward and backward from g {B, M, P}.
int h_matmul_chain(const float* a, const size_t* as, const float* b, const size_t* bs, const float* c, const size_t* cs,
                   const float* g, float* y, float* da, float* db, float* dc) {
	return guard([&] {
		Value A = param(a, {as[0], as[1], as[2]}), Bv = param(b, {bs[0], bs[1], bs[2]}), Cv = param(c, {cs[0], cs[1]});
		Value r = nn::hip::matmul_bt(nn::hip::matmul(A, Bv), Cv);
		r.backward(Tensor::from_host(r.data().shape(), g));
		out(r.data(), y);
		out(A.grad(), da);
		out(Bv.grad(), db);
		out(Cv.grad(), dc);
	});
}

// attention(x, x, x): one node as q, k and v, so its gradient is stored by dV and added to by dQ, then dK.
int h_self_attention(const float* x, size_t N, size_t T, size_t D, size_t heads, int causal, const float* g,
                     float* o, float* dx) {
	return guard([&] {
		Value xv = param(x, {N, T, D});
		Value r = nn::hip::attention(xv, xv, xv, heads, Tensor(), causal != 0);
		r.backward(Tensor::from_host({N, T, D}, g));
		out(r.data(), o);
		out(xv.grad(), dx);
	});
}

// scaled_masked_softmax forward and backward on {N, H, Tq, Tk} with a key padding mask (may be null).
int h_softmax(const float* x, size_t N, size_t H, size_t Tq, size_t Tk, float scale, const float* pad, int causal,
              const float* g, float* y, float* dx) {
	return guard([&] {
		Value xv = param(x, {N, H, Tq, Tk});
		const Tensor mask = pad ? Tensor::from_host({N, Tk}, pad) : Tensor();
		Value r = nn::hip::scaled_masked_softmax(xv, scale, mask, causal != 0);
		r.backward(Tensor::from_host({N, H, Tq, Tk}, g));
		out(r.data(), y);
		out(xv.grad(), dx);
	});
}

// The Conv-BN-ReLU stack with a layer-normalised head of oracle/ref_shim.cpp's nnref_norm_step, through nn::hip.
int h_norm_step(const float* x, size_t N, size_t c0, size_t side, size_t c1, size_t c2, size_t classes,
                const float* const* p, const float* g, float* y, float* const* grads, float* dx) {
	return guard([&] {
		const size_t flat = c2 * (side / 2) * (side / 2);
		Value xv = param(x, {N, c0, side, side});
		const std::vector<std::vector<size_t>> shapes = {{c1, c0, 3, 3}, {c1}, {c1}, {c1}, {c2, c1, 3, 3}, {c2}, {c2},
		                                                 {c2}, {flat}, {flat}, {classes, flat}, {classes}};
		std::vector<Value> v;
		for (size_t i = 0; i < shapes.size(); ++i) v.push_back(param(p[i], shapes[i]));
		Value h = nn::hip::batchnorm(nn::hip::conv2d(xv, v[0], v[1], 1, 1), v[2], v[3], 1e-5f, nullptr, nullptr, true);
		h = nn::hip::maxpool2d(h, 2, 2);
		h = nn::hip::relu(nn::hip::batchnorm(nn::hip::conv2d(h, v[4], v[5], 1, 1), v[6], v[7], 1e-5f));
		h = nn::hip::layernorm(nn::hip::reshape(h, {N, flat}), v[8], v[9], 1e-5f);
		Value r = nn::hip::linear(h, v[10], v[11]);
		r.backward(Tensor::from_host({N, classes}, g));
		out(r.data(), y);
		for (size_t i = 0; i < v.size(); ++i) out(v[i].grad(), grads[i]);
		out(xv.grad(), dx);
	});
}

// The shape errors nn-cpp throws: bit i of the result is set when case i threw nn::hip::TensorShapeError.
int h_shape_errors(void) {
	int bits = 0;
	auto expect = [&](int i, auto f) {
		try {
			f();
		} catch (const nn::hip::TensorShapeError&) {
			bits |= 1 << i;
		} catch (...) {
		}
	};
	expect(0, [] { nn::hip::matmul(Tensor({2, 3}), Tensor({4, 5})); });
	expect(1, [] { nn::hip::matmul(Tensor({2, 3, 4}), Tensor({3, 4, 5})); });  // batch 2 against 3
	expect(2, [] { nn::hip::linear(Value::leaf(Tensor({4, 5})), Value::leaf(Tensor({3, 6})), Value::leaf(Tensor({3}))); });
	expect(3, [] { nn::hip::linear(Value::leaf(Tensor({4, 5})), Value::leaf(Tensor({3, 5})), Value::leaf(Tensor({4}))); });
	expect(4, [] { nn::hip::conv2d(Value::leaf(Tensor({1, 2, 5, 5})), Value::leaf(Tensor({3, 1, 3, 3})),
	                               Value::leaf(Tensor({3})), 1, 1); });
	expect(5, [] { nn::hip::maxpool2d(Value::leaf(Tensor({1, 1, 3, 3})), 4, 1); });
	expect(6, [] { nn::hip::attention(Value::leaf(Tensor({1, 4, 6})), Value::leaf(Tensor({1, 4, 6})),
	                                  Value::leaf(Tensor({1, 4, 6})), 4, Tensor(), false); });  // 4 heads do not divide 6
	expect(7, [] { Value::leaf(Tensor({2, 2})).backward(); });                               // not one element
	expect(8, [] { nn::hip::batchnorm(Value::leaf(Tensor({4})), Value::leaf(Tensor({4})), Value::leaf(Tensor({4})),
	                                  1e-5f); });                                          // no channel axis
	expect(9, [] { nn::hip::batchnorm(Value::leaf(Tensor({2, 3, 4})), Value::leaf(Tensor({4})),
	                                  Value::leaf(Tensor({3})), 1e-5f); });                // weight of the wrong size
	expect(10, [] { nn::hip::layernorm(Value::leaf(Tensor({2, 5})), Value::leaf(Tensor({4})), Value::leaf(Tensor({5})),
	                                   1e-5f); });                                         // gamma of the wrong size
	return bits;
}

// nn::hip::mul forward and backward on count elements: y = a * b, then the gradients of a and b from g; same = 1
// passes a as both operands (its gradient stored by the first term, added to by the second).
int h_mul_step(const float* a, const float* b, size_t count, int same, const float* g, float* y, float* da, float* db) {
	return guard([&] {
		Value av = param(a, {count});
		Value bv = same ? av : param(b, {count});
		Value r = nn::hip::mul(av, bv);
		r.backward(Tensor::from_host({count}, g));
		out(r.data(), y);
		out(av.grad(), da);
		if (!same) out(bv.grad(), db);
	});
}

// n draws of nn::hip::derive_generator(stream) after nn::hip::manual_seed(seed), generators k = 0 .. gens - 1 of the
// stream in turn (n / gens draws each); host only, no device work.
int h_random_draws(unsigned long long seed, const char* stream, int gens, size_t n, unsigned* outp) {
	return guard([&] {
		nn::hip::manual_seed(seed);
		size_t o = 0;
		for (int k = 0; k < gens; ++k) {
			std::mt19937 gen = nn::hip::derive_generator(stream);
			for (size_t i = 0; i < n / gens; ++i) outp[o++] = static_cast<unsigned>(gen());
		}
	});
}

// The module layer (include/nn_hip_modules.hpp): the models of oracle/ref_shim.cpp's nnref_module_run, built with
// nn::hip's modules after nn::hip::manual_seed(seed), the same input x (shape xs) and the output gradient g; out
// receives the output and grads every parameter's gradient in parameters() order, then x's. *n_out and *n_grads
// receive the counts; capacities are checked.
int h_module_run(int which, unsigned seed, const float* x, const size_t* xs, int xn, const float* g, float* outp,
                 size_t out_cap, float* grads, size_t grads_cap, size_t* n_out, size_t* n_grads) {
	return guard([&] {
		namespace H = nn::hip;
		H::manual_seed(seed);
		std::unique_ptr<H::Module> m;
		if (which == 0) {
			auto s = std::make_unique<H::Sequential>();
			s->add(std::make_unique<H::Conv2d>(1, 8, 3, 1, 1));
			s->add(std::make_unique<H::ReLU>());
			s->add(std::make_unique<H::MaxPool2d>(2, 2));
			s->add(std::make_unique<H::Conv2d>(8, 16, 3, 1, 1));
			s->add(std::make_unique<H::ReLU>());
			s->add(std::make_unique<H::MaxPool2d>(2, 2));
			s->add(std::make_unique<H::Flatten>());
			s->add(std::make_unique<H::Linear>(784, 128));
			s->add(std::make_unique<H::ReLU>());
			s->add(std::make_unique<H::Linear>(128, 10));
			m = std::move(s);
		} else if (which == 1) {
			m = std::make_unique<H::MultiHeadAttention>(64, 4, true);
		} else if (which == 3) {
			auto s = std::make_unique<H::Sequential>();
			s->add(std::make_unique<H::Linear>(20, 30));
			s->add(std::make_unique<H::ReLU>());
			s->add(std::make_unique<H::Linear>(30, 5));
			m = std::move(s);
		} else if (which == 4) {
			m = std::make_unique<H::Transformer>(H::TransformerConfig{11, 16, 2, 2, 12, 2, 0.0f, true, true});
		} else if (which == 5) {
			auto s = std::make_unique<H::Sequential>();
			s->add(std::make_unique<H::Linear>(20, 30));
			s->add(std::make_unique<H::Dropout>(0.25f));
			s->add(std::make_unique<H::ReLU>());
			s->add(std::make_unique<H::Linear>(30, 5));
			m = std::move(s);
			m->train(true);
		} else if (which == 6) {
			m = std::make_unique<H::Transformer>(H::TransformerConfig{13, 24, 3, 1, 9, 4, 0.1f, false, false});
			m->eval();
		} else {
			throw std::invalid_argument("h_module_run: unknown model");
		}
		const Value xv = param(x, std::vector<size_t>(xs, xs + xn));
		const Value y = m->forward(xv);
		y.backward(Tensor::from_host(y.data().shape(), g));
		if (y.data().size() > out_cap) throw std::runtime_error("capacity");
		out(y.data(), outp);
		*n_out = y.data().size();
		std::vector<Value> ps = m->parameters();
		ps.push_back(xv);
		size_t off = 0;
		for (const Value& p : ps) {
			if (off + p.grad().size() > grads_cap) throw std::runtime_error("capacity");
			out(p.grad(), grads + off);
			off += p.grad().size();
		}
		*n_grads = off;
	});
}

}  // extern "C"
