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

const std::vector<std::vector<size_t>>& param_shapes(int model) {
	static const std::vector<std::vector<size_t>> mlp = {{1024, 784}, {1024}, {1024, 1024}, {1024}, {10, 1024}, {10}};
	static const std::vector<std::vector<size_t>> cnn = {{8, 1, 3, 3}, {8}, {16, 8, 3, 3}, {16}, {128, 784}, {128},
	                                                     {10, 128}, {10}};
	return model == 0 ? mlp : cnn;
}

Value forward(int model, const Value& x, const std::vector<Value>& p) {
	if (model == 0) {
		Value h = nn::hip::relu(nn::hip::linear(x, p[0], p[1]));
		h = nn::hip::relu(nn::hip::linear(h, p[2], p[3]));
		return nn::hip::linear(h, p[4], p[5]);
	}
	const size_t N = x.data().shape()[0];
	// each conv2d_relu -> maxpool2d pair in one call: the first layer's in one pass, the second's in turn
	Value h = nn::hip::conv2d_relu_maxpool2d(x, p[0], p[1], 1, 1, 2, 2);
	h = nn::hip::conv2d_relu_maxpool2d(h, p[2], p[3], 1, 1, 2, 2);
	h = nn::hip::reshape(h, {N, 784});
	return nn::hip::linear(nn::hip::relu(nn::hip::linear(h, p[4], p[5])), p[6], p[7]);
}

}  // namespace

extern "C" {

// warmup untimed steps, then `runs` timed ones: fwd_ms[i], bwd_ms[i]; logits (N x 10) of the last step.
// Returns 0, or 1 when an exception was thrown.
int nnh_bench_workload_step(int model, const float* x, size_t N, const float* const* params, const float* g, int warmup,
                            int runs, double* fwd_ms, double* bwd_ms, float* logits) {
	try {
		const auto& shapes = param_shapes(model);
		std::vector<Value> p;
		for (size_t i = 0; i < shapes.size(); ++i) p.push_back(Value::leaf(Tensor::from_host(shapes[i], params[i]), true));
		const std::vector<size_t> xs = model == 0 ? std::vector<size_t>{N, 784} : std::vector<size_t>{N, 1, 28, 28};
		const Value xv = Value::leaf(Tensor::from_host(xs, x), false);
		const Tensor seed = Tensor::from_host({N, 10}, g);
		nn::hip::synchronize();
		for (int i = 0; i < warmup + runs; ++i) {
			const auto t0 = Clock::now();
			Value y = forward(model, xv, p);
			nn::hip::synchronize();
			const auto t1 = Clock::now();
			for (const Value& v : p) v.zero_grad();
			y.backward(seed);
			nn::hip::synchronize();
			const auto t2 = Clock::now();
			if (i >= warmup) {
				fwd_ms[i - warmup] = ms_between(t0, t1);
				bwd_ms[i - warmup] = ms_between(t1, t2);
			}
			if (i + 1 == warmup + runs && logits) y.data().to_host(logits);
		}
		return 0;
	} catch (...) {
		return 1;
	}
}

}  // extern "C"
