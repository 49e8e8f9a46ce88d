// workloads.cpp - measurement helper for bench.py (lib/libnnh_workloads.so, not part of the ABI): a training step
// of nn-cpp's bench models (apps/bench/workloads.cpp:100-137) run through include/nn_hip.hpp, timed the way
// apps/bench/runner.cpp:33-45 times time_train_step: the forward pass, then zero_grad and the backward pass, each
// between two points where the device has finished. The loss and the optimizer step (elementwise work outside the
// GEMM path) are not part of it: the backward pass starts from a given gradient of the logits.
//   model 0, mlp_wide: Linear(784,1024) ReLU Linear(1024,1024) ReLU Linear(1024,10); params W1 b1 W2 b2 W3 b3.
//   model 1, cnn_mnist: Conv2d(1,8,3,1,1) ReLU MaxPool2d(2,2) Conv2d(8,16,3,1,1) ReLU MaxPool2d(2,2) Flatten
//            Linear(784,128) ReLU Linear(128,10), with Sequential's Conv2d + ReLU folding (src/nn/sequential.cpp:16-28)
//            and each Conv2d + ReLU + MaxPool2d run as nn::hip::conv2d_relu_maxpool2d (the same values and
//            gradients); params conv1 w b, conv2 w b, fc1 w b, fc2 w b.
//   model 2, transformer_tiny (apps/bench/workloads.cpp:80-92): Transformer{vocab 64, dim 64, heads 4, layers 2,
//            max_len 64} (src/nn/transformer.cpp:59-69), logits flattened to {N*T, 64}; params in named_parameters
//            order: embed.weight, per block ln1 gamma beta, attn q k v o (weight, bias each), ln2 gamma beta, fc1 w b,
//            fc2 w b; then ln_f gamma beta, head w b. x holds {N, 64} float token ids.
#include <chrono>
#include <vector>

#include "nn_hip.hpp"

using nn::hip::Tensor;
using nn::hip::Value;

namespace {

using Clock = std::chrono::steady_clock;

double ms_between(Clock::time_point a, Clock::time_point b) {
	return std::chrono::duration<double, std::milli>(b - a).count();
}

constexpr size_t kVocab = 64, kDim = 64, kHeads = 4, kLayers = 2, kMaxLen = 64, kHidden = 4 * kDim;

std::vector<std::vector<size_t>> transformer_shapes() {
	std::vector<std::vector<size_t>> s = {{kVocab, kDim}};
	for (size_t l = 0; l < kLayers; ++l) {
		s.insert(s.end(), {{kDim}, {kDim}});
		for (int i = 0; i < 4; ++i) s.insert(s.end(), {{kDim, kDim}, {kDim}});
		s.insert(s.end(), {{kDim}, {kDim}, {kHidden, kDim}, {kHidden}, {kDim, kHidden}, {kDim}});
	}
	s.insert(s.end(), {{kDim}, {kDim}, {kVocab, kDim}, {kVocab}});
	return s;
}

const std::vector<std::vector<size_t>>& param_shapes(int model) {
	static const std::vector<std::vector<size_t>> mlp = {{1024, 784}, {1024}, {1024, 1024}, {1024}, {10, 1024}, {10}};
	static const std::vector<std::vector<size_t>> cnn = {{8, 1, 3, 3}, {8}, {16, 8, 3, 3}, {16}, {128, 784}, {128},
	                                                     {10, 128}, {10}};
	static const std::vector<std::vector<size_t>> tf = transformer_shapes();
	return model == 0 ? mlp : model == 1 ? cnn : tf;
}

// Transformer::forward (transformer.cpp:59-63) with its blocks (transformer.cpp:37-40), attention without dropout
// (attention.cpp:31-35) and LayerNorm's default eps 1e-5; dropout 0 leaves every Dropout the identity.
Value transformer_forward(const std::vector<float>& ids, size_t N, const std::vector<Value>& p, const Value& pe) {
	const Tensor no_mask;
	// add(embedding(...), pe) with the positions added in the lookup's kernel (the same nodes and bits)
	Value h = nn::hip::embedding_add(p[0], ids, {N, kMaxLen}, pe);
	size_t i = 1;
	for (size_t l = 0; l < kLayers; ++l, i += 16) {
		const Value a = nn::hip::layernorm(h, p[i], p[i + 1], 1e-5f);
		// the q, k and v projections in one launch (the nodes and bits of three linear calls)
		const std::vector<Value> qkv =
		    nn::hip::linear_many(a, {{p[i + 2], p[i + 3]}, {p[i + 4], p[i + 5]}, {p[i + 6], p[i + 7]}});
		const Value att = nn::hip::attention(qkv[0], qkv[1], qkv[2], kHeads, no_mask, true);
		// add(h, linear(...)) with the add in the linear's epilogue: the same nodes and bits
		h = nn::hip::linear_add(att, p[i + 8], p[i + 9], h);
		// gelu(linear(...)) with the GELU in the linear's epilogue (the same nodes and bits)
		const Value m = nn::hip::linear_gelu(nn::hip::layernorm(h, p[i + 10], p[i + 11], 1e-5f), p[i + 12], p[i + 13]);
		h = nn::hip::linear_add(m, p[i + 14], p[i + 15], h);
	}
	const Value o = nn::hip::linear(nn::hip::layernorm(h, p[i], p[i + 1], 1e-5f), p[i + 2], p[i + 3]);
	return nn::hip::reshape(o, {N * kMaxLen, kVocab});
}

Value forward(int model, const Value& x, const std::vector<Value>& p) {
	if (model == 0) {
		Value h = nn::hip::linear_relu(x, p[0], p[1]);
		h = nn::hip::linear_relu(h, p[2], p[3]);
		return nn::hip::linear(h, p[4], p[5]);
	}
	const size_t N = x.data().shape()[0];
	// each conv2d_relu -> maxpool2d pair in one call: the first layer's in one pass, the second's in turn
	Value h = nn::hip::conv2d_relu_maxpool2d(x, p[0], p[1], 1, 1, 2, 2);
	h = nn::hip::conv2d_relu_maxpool2d(h, p[2], p[3], 1, 1, 2, 2);
	h = nn::hip::reshape(h, {N, 784});
	return nn::hip::linear(nn::hip::linear_relu(h, p[4], p[5]), p[6], p[7]);
}

}  // namespace

extern "C" {

// warmup untimed steps, then `runs` timed ones: fwd_ms[i], bwd_ms[i]; logits ({N, 10}, transformer_tiny {N*64, 64})
// and, when grads is given, each parameter's gradient (in parameter order) of the last step.
// Returns 0, or 1 when an exception was thrown.
int nnh_bench_workload_step(int model, const float* x, size_t N, const float* const* params, const float* g, int warmup,
                            int runs, double* fwd_ms, double* bwd_ms, float* logits, float* const* grads) {
	try {
		const auto& shapes = param_shapes(model);
		std::vector<Value> p;
		for (size_t i = 0; i < shapes.size(); ++i) p.push_back(Value::leaf(Tensor::from_host(shapes[i], params[i]), true));
		const bool tf = model == 2;
		const std::vector<size_t> xs = model == 0 ? std::vector<size_t>{N, 784}
		                               : tf      ? std::vector<size_t>{N, kMaxLen}
		                                         : std::vector<size_t>{N, 1, 28, 28};
		const Value xv = Value::leaf(Tensor::from_host(xs, x), false);
		const std::vector<float> ids = tf ? std::vector<float>(x, x + N * kMaxLen) : std::vector<float>();
		// PositionalEncoding's fixed table; slice(pe, 0, 0, T) at T = max_len is all of it
		const Value pe = Value::leaf(tf ? nn::hip::sinusoidal_table(kMaxLen, kDim) : Tensor(), false);
		const Tensor seed = Tensor::from_host(tf ? std::vector<size_t>{N * kMaxLen, kVocab} : std::vector<size_t>{N, 10}, g);
		nn::hip::synchronize();
		for (int i = 0; i < warmup + runs; ++i) {
			const auto t0 = Clock::now();
			Value y = tf ? transformer_forward(ids, N, p, pe) : forward(model, xv, p);
			nn::hip::synchronize();
			const auto t1 = Clock::now();
			nn::hip::zero_grad(p);  // Optimizer::zero_grad: marks every parameter's gradient fresh (no launch)
			y.backward(seed);
			nn::hip::synchronize();
			const auto t2 = Clock::now();
			if (i >= warmup) {
				fwd_ms[i - warmup] = ms_between(t0, t1);
				bwd_ms[i - warmup] = ms_between(t1, t2);
			}
			if (i + 1 == warmup + runs) {
				if (logits) y.data().to_host(logits);
				if (grads)
					for (size_t j = 0; j < p.size(); ++j)
						if (grads[j]) p[j].grad().to_host(grads[j]);
			}
		}
		return 0;
	} catch (...) {
		return 1;
	}
}

}  // extern "C"
