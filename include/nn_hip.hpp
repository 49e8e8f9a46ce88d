// nn_hip.hpp - nn-cpp's op surface on an MI355X, with device-resident tensors (C++17; lib/libnn_hip.so).
//
// The names, argument meanings, shape rules and exceptions follow nn-cpp 2.0.0's own API so that code written
// against it reads the same:
//   * Tensor and matmul(a, b, trans_a, trans_b)                  include/nn/tensor.hpp:47-510, 465-491
//   * Value, NoGradGuard, grad_accum and backward                include/nn/autograd/value.hpp:41-228
//   * matmul, linear, matmul_bt, relu, reshape, conv2d, conv2d_relu, maxpool2d, batchnorm, layernorm, attention,
//     scaled_masked_softmax (and conv2d_relu_maxpool2d, the two ops of a first layer in one call)
//                                                                include/nn/autograd/ops.hpp:22-523
// The difference is where the numbers live: a Tensor's storage is HBM, so a chain of ops (linear -> relu ->
// linear, conv -> pool -> conv) never leaves the device; data crosses PCIe only in from_host / to_host. Every op
// runs the C ABI of include/nnh.h and gives the bits nn-cpp's NN_NATIVE CPU build gives on the same inputs,
// gradients included (each backward rule takes its gradient buffers in the reference's order and passes the
// first-write flags of grad_accum).
//
// Work is enqueued on one stream (set_stream; default the null stream). Device memory comes from a caching
// allocator: a Tensor's storage returns to it when the last Tensor sharing it is destroyed and is reused by later
// work on the same stream, which stream order makes safe.
// Errors: TensorShapeError where nn-cpp throws it (nnh's NNH_ERR_SHAPE), std::invalid_argument for other
// invalid arguments, HipError for runtime failures.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

namespace nn {
namespace hip {

class TensorShapeError : public std::runtime_error {
public:
	TensorShapeError() : std::runtime_error("nn::hip: tensor shape mismatch") {}
	explicit TensorShapeError(const std::string& m) : std::runtime_error(m) {}
};

class HipError : public std::runtime_error {
public:
	explicit HipError(const std::string& m) : std::runtime_error(m) {}
};

// nn-cpp's library-wide seeding (include/nn/random.hpp, src/random.cpp): manual_seed restarts every named stream;
// derive_generator hands out the k-th generator of a stream, seeded from splitmix64(base ^ fnv1a(stream) ^
// k * golden) through std::seed_seq as the reference does, so that parameters initialised here (Tensor::random,
// Dropout's masks) equal the reference's after the same seed. Without a manual_seed the base comes from
// std::random_device once.
void manual_seed(uint64_t seed);
bool is_seeded();
uint64_t seed_epoch();
std::mt19937 derive_generator(const std::string& stream);

// The stream every op enqueues on (setting another first waits for the current one).
void set_stream(hipStream_t s);
hipStream_t current_stream();
void synchronize();
// Device bytes the allocator holds (in use and cached), and a release of the cached ones.
size_t allocator_bytes();
void empty_cache();

struct Block;  // a device allocation of the caching allocator

// A row-major, contiguous fp32 tensor in HBM (tensor.hpp:90-413, device storage).
class Tensor {
public:
	Tensor();                                                  // shape {0}
	explicit Tensor(std::vector<size_t> shape, float value = 0.0f);  // filled with value
	static Tensor empty(std::vector<size_t> shape);            // uninitialised (Tensor::empty, tensor.cpp:263)
	static Tensor from_host(std::vector<size_t> shape, const float* data);
	// Tensor::random (tensor.cpp:504-522): uniform in [lo, hi) from the "tensor.random" stream of manual_seed below,
	// drawn on the host (std::mt19937 and std::uniform_real_distribution<float>) and copied in: after the same
	// manual_seed and the same sequence of draws, the values nn-cpp's Tensor::random gives.
	static Tensor random(std::vector<size_t> shape, float lo, float hi);
	void to_host(float* out) const;
	std::vector<float> to_host() const;

	const std::vector<size_t>& shape() const { return shape_; }
	size_t ndim() const { return shape_.size(); }
	size_t size() const { return size_; }
	float* data() const;                                       // device pointer
	Tensor reshape(std::vector<size_t> new_shape) const;       // shares the storage
	void zero_();
	void fill_(float value);

private:
	std::shared_ptr<Block> storage_;
	std::vector<size_t> shape_;
	size_t size_ = 0;
};

// nn::matmul(a, b, trans_a, trans_b) (tensor.cpp:571-641): batched, broadcast, 2-D right operand folded.
Tensor matmul(const Tensor& a, const Tensor& b, bool trans_a = false, bool trans_b = false);

class Value;

// Graph node state (value.hpp:60-84).
struct NodeImpl {
	Tensor data;
	Tensor grad;
	bool grad_fresh = false;
	bool requires_grad = false;
	size_t consumers = 0;  // uses as a parent in the graph of the last backward() that reached this node
	std::vector<Value> parents;
	std::function<void(const Tensor&)> backward_fn;
};

// Reference-counted handle to a graph node (value.hpp:86-228).
class Value {
public:
	Value() = default;
	static Value leaf(Tensor data, bool requires_grad = false);
	static Value node(Tensor data, std::vector<Value> parents, std::function<void(const Tensor&)> backward_fn);
	Tensor& data() const;
	Tensor& grad() const;                     // a fresh gradient is zeroed on first read
	Tensor& grad_accum(bool& first) const;    // value.cpp:60-64: first = the buffer holds nothing yet
	bool requires_grad() const;
	// value.cpp's zero_grad: the gradient reads as zeros from here on; marked fresh rather than filled (no launch),
	// the next backward rule's first write giving the bits of an add to zeros
	void zero_grad() const;
	// Value::backward (value.cpp:80-132) for a one-element value; the overload seeds the output gradient with
	// `seed` (the output's shape) instead of ones, for a graph whose loss is formed elsewhere.
	void backward() const;
	void backward(const Tensor& seed) const;
	NodeImpl* impl() const { return impl_.get(); }

private:
	explicit Value(std::shared_ptr<NodeImpl> impl) : impl_(std::move(impl)) {}
	std::shared_ptr<NodeImpl> impl_;
};

// Value::zero_grad over a list (Optimizer::zero_grad, src/optim/sgd.cpp:19-21): the same gradients, no launch.
void zero_grad(const std::vector<Value>& values);

// Ops record no graph while one is alive on the thread (value.hpp:24-40).
class NoGradGuard {
public:
	NoGradGuard();
	~NoGradGuard();
	NoGradGuard(const NoGradGuard&) = delete;
	NoGradGuard& operator=(const NoGradGuard&) = delete;
	static bool grad_enabled();

private:
	bool previous_;
};

// ops.hpp:289 / 337: differentiable matmul and matmul against a transposed right operand.
Value matmul(const Value& a, const Value& b);
Value matmul_bt(const Value& a, const Value& b);
// ops.hpp:304: x W^T + b, x {..., K}, weight {N, K}, bias {N}.
Value linear(const Value& x, const Value& weight, const Value& bias);
// relu(linear(x, weight, bias)) with both forwards in one launch: the same two nodes, outputs and gradients. No
// counterpart in the reference, whose model code calls the two ops in turn.
Value linear_relu(const Value& x, const Value& weight, const Value& bias);
// add(residual, linear(x, weight, bias)) with the add in the linear's epilogue (one kernel): the same two nodes and
// bits. A residual of another shape runs the two ops.
Value linear_add(const Value& x, const Value& weight, const Value& bias, const Value& residual);
// gelu(linear(x, weight, bias)) with the GELU in the linear's epilogue: the same two nodes and bits.
Value linear_gelu(const Value& x, const Value& weight, const Value& bias);
// linear(x, w_i, b_i) for each (w_i, b_i) of layers (an attention layer's q, k and v projections): the nodes and bits
// of the separate calls, in one launch where the shapes allow.
std::vector<Value> linear_many(const Value& x, const std::vector<std::pair<Value, Value>>& layers);
Value relu(const Value& x);
// ops.cpp:672-681: same elements, new shape (the Flatten module's op).
Value reshape(const Value& x, std::vector<size_t> new_shape);
// ops.hpp:392 / 402: 2-D convolution (x {N, Cin, H, W}, weight {Cout, Cin, kH, kW}, bias {Cout}), and with ReLU.
Value conv2d(const Value& x, const Value& weight, const Value& bias, int stride, int padding);
Value conv2d_relu(const Value& x, const Value& weight, const Value& bias, int stride, int padding);
// ops.cpp:1609-1705: max pooling, kernel x kernel windows at `stride`.
Value maxpool2d(const Value& x, size_t kernel_size, size_t stride);
// maxpool2d(conv2d_relu(x, weight, bias, stride, padding), kernel_size, pool_stride): the same two graph nodes, the
// same values and gradients, with both forwards in one pass where nnh_conv2d_relu_maxpool2d_forward fuses them (a
// network's first layer). No counterpart in the reference, whose Sequential runs the two modules in turn.
Value conv2d_relu_maxpool2d(const Value& x, const Value& weight, const Value& bias, int stride, int padding,
                            size_t kernel_size, size_t pool_stride);
// ops.hpp:114-115: batch normalisation in training mode over every axis but axis 1 of x {N, C, ...}; mean_out and
// var_out (optional) receive the batch mean and biased variance {C}; fuse_relu clips the result at 0 in the same op.
Value batchnorm(const Value& x, const Value& weight, const Value& bias, float eps, Tensor* mean_out = nullptr,
                Tensor* var_out = nullptr, bool fuse_relu = false);
// ops.hpp:130: layer normalisation over the last axis of x {..., D}, gamma and beta {D}.
Value layernorm(const Value& x, const Value& gamma, const Value& beta, float eps);
// ops.hpp:324: multi-head attention core; key_padding_mask {N, Tk} (0 = padded) or empty.
Value attention(const Value& q, const Value& k, const Value& v, size_t heads, const Tensor& key_padding_mask,
                bool causal);
// ops.cpp:1298-1343: softmax over the last axis of {N, H, Tq, Tk} after scaling and masking.
Value scaled_masked_softmax(const Value& x, float scale_by, const Tensor& key_padding_mask, bool causal);
// ops.hpp:22 (ops.cpp:331-337): a + b, for b of a's shape or of a's trailing axes (broadcast along the leading
// ones, as PositionalEncoding adds its table); b's gradient is then summed one leading axis at a time
// (sum_to_shape, ops.cpp:35-53). Other broadcasts are refused with std::invalid_argument.
Value add(const Value& a, const Value& b);
// ops.hpp (ops.cpp:347-357): element-wise product of two tensors of one shape (other broadcasts are refused with
// std::invalid_argument); Dropout multiplies by its mask with it.
Value mul(const Value& a, const Value& b);
// ops.cpp:592-608: rows start .. end - 1 of axis 0 (other axes are refused with std::invalid_argument); the gradient
// adds into that band of x's (PositionalEncoding takes its first T rows with it).
Value slice(const Value& x, int axis, size_t start, size_t end);
// ops.hpp:195 (ops.cpp:451-481): GELU, tanh form.
Value gelu(const Value& x);
// ops.hpp:255 (ops.cpp:1991-2015): rows of weight {V, D} picked by float ids (whole numbers in [0, V), checked on the
// host: TensorShapeError otherwise); the result has ids' shape plus D. The device-tensor form reads the ids back.
Value embedding(const Value& weight, const std::vector<float>& ids, const std::vector<size_t>& ids_shape);
Value embedding(const Value& weight, const Tensor& ids);
// add(embedding(weight, ids), addend) with the addend (of the output's trailing axes: a transformer's positions)
// added in the lookup's kernel: the nodes and bits of the two ops.
Value embedding_add(const Value& weight, const std::vector<float>& ids, const std::vector<size_t>& ids_shape,
                    const Value& addend);
Value embedding_add(const Value& weight, const Tensor& ids, const Value& addend);
// positional.cpp:15-25: the fixed sinusoidal table {max_len, dim}, computed in double on the host and stored as fp32.
Tensor sinusoidal_table(size_t max_len, size_t dim);

}  // namespace hip
}  // namespace nn
