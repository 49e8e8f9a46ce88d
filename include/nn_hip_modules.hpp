// nn_hip_modules.hpp - nn-cpp's module layer over nn::hip's device-resident Values (C++17; lib/libnn_hip.so).
//
// The classes, constructor arguments, defaults, parameter names and orders, checks and exceptions follow nn-cpp
// 2.0.0's include/nn/nn/*.hpp, so that a model written against them reads the same with `nn::hip::` in front:
//   * Module (module.hpp:23-113) and Sequential with its Conv2d + ReLU folding (sequential.cpp:16-28)
//   * Linear, Conv2d, ReLU, GELU, Flatten, MaxPool2d, Dropout, LayerNorm, Embedding, PositionalEncoding
//     (linear.cpp, conv2d.cpp, activation.cpp, flatten.hpp, pool2d.cpp, dropout.cpp, layernorm.cpp, embedding.cpp,
//     positional.cpp)
//   * MultiHeadAttention (attention.cpp:22-48), TransformerBlock and Transformer (transformer.cpp)
// Parameters live in HBM from construction on. Their initial values come from Tensor::random's seeded stream, so
// after the same nn::hip::manual_seed a module holds the values nn-cpp's module holds after nn::manual_seed, and its
// forward and backward give the same bits.
//
// Differences, each stated where it applies: MultiHeadAttention refuses dropout on its attention weights in training
// mode (std::invalid_argument; the reference composes that path from ops this library does not have), and Sequential
// also runs a Conv2d, ReLU, MaxPool2d triple as nn::hip::conv2d_relu_maxpool2d and a Linear, ReLU pair as
// nn::hip::linear_relu (the same graph nodes and bits as the ops in turn, with the forwards in one pass).
#pragma once

#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "nn_hip.hpp"

namespace nn {
namespace hip {

// module.hpp:23-113: maps a Value to a Value and may own parameters.
class Module {
public:
	virtual ~Module() = default;
	virtual Value forward(const Value& input) = 0;
	// whether forward_relu can run this layer and a following ReLU as one op (Sequential folds the pair)
	virtual bool can_fuse_relu() const { return false; }
	virtual Value forward_relu(const Value& input) { return forward(input); }
	virtual std::vector<Value> parameters() const { return {}; }
	virtual std::vector<std::pair<std::string, Value>> named_parameters() const { return {}; }
	virtual std::vector<std::pair<std::string, Tensor*>> named_buffers() const { return {}; }
	virtual void train(bool mode = true) { training_ = mode; }
	void eval() { train(false); }
	bool is_training() const { return training_; }

protected:
	bool training_ = true;
};

// activation.cpp: relu / gelu of the input.
class ReLU : public Module {
public:
	Value forward(const Value& input) override { return relu(input); }
};

class GELU : public Module {
public:
	Value forward(const Value& input) override { return gelu(input); }
};

// flatten.hpp: {N, d1, d2, ...} -> {N, d1 d2 ...}.
class Flatten : public Module {
public:
	Value forward(const Value& input) override;
};

// linear.cpp: y = x W^T + b; W {out, in} uniform in +-1/sqrt(in), b zeros. A following ReLU folds into linear_relu
// (the reference's Sequential folds only Conv2d + ReLU; the nodes and bits are those of the two ops).
class Linear : public Module {
public:
	Linear(size_t in_features, size_t out_features);
	Value forward(const Value& input) override;
	bool can_fuse_relu() const override { return true; }
	Value forward_relu(const Value& input) override { return linear_relu(input, weight_, bias_); }
	// add(residual, forward(input)) in one kernel (linear_add)
	Value forward_add(const Value& input, const Value& residual) { return linear_add(input, weight_, bias_, residual); }
	// gelu(forward(input)) in one kernel (linear_gelu)
	Value forward_gelu(const Value& input) { return linear_gelu(input, weight_, bias_); }
	std::vector<Value> parameters() const override;
	std::vector<std::pair<std::string, Value>> named_parameters() const override;
	const Value& weight() const { return weight_; }
	const Value& bias() const { return bias_; }

private:
	Value weight_, bias_;
};

// conv2d.cpp: square kernels; W {out, in, k, k} uniform in +-1/sqrt(in k k), b zeros. A following ReLU folds into
// conv2d_relu.
class Conv2d : public Module {
public:
	Conv2d(size_t in_channels, size_t out_channels, size_t kernel_size, size_t stride = 1, size_t padding = 0);
	Value forward(const Value& input) override;
	bool can_fuse_relu() const override { return true; }
	Value forward_relu(const Value& input) override;
	std::vector<Value> parameters() const override;
	std::vector<std::pair<std::string, Value>> named_parameters() const override;
	size_t stride() const { return stride_; }
	size_t padding() const { return padding_; }
	const Value& weight() const { return weight_; }
	const Value& bias() const { return bias_; }

private:
	Value weight_, bias_;
	size_t stride_, padding_;
};

// pool2d.cpp: max over kernel x kernel windows at `stride`.
class MaxPool2d : public Module {
public:
	MaxPool2d(size_t kernel_size, size_t stride) : kernel_size_(kernel_size), stride_(stride) {}
	Value forward(const Value& input) override { return maxpool2d(input, kernel_size_, stride_); }
	size_t kernel_size() const { return kernel_size_; }
	size_t stride() const { return stride_; }

private:
	size_t kernel_size_, stride_;
};

// dropout.cpp: in training mode with p > 0 each element is kept (scaled by 1 / (1 - p)) or zeroed by a mask drawn
// on the host from this module's "dropout" stream, then multiplied in (nn::hip::mul); otherwise the input itself.
class Dropout : public Module {
public:
	explicit Dropout(float p = 0.5f);
	Value forward(const Value& input) override;
	bool active() const { return training_ && p_ > 0.0f; }

private:
	float p_;
	std::mt19937 gen_;
};

// layernorm.cpp: over the last axis, gamma ones and beta zeros {dim}.
class LayerNorm : public Module {
public:
	explicit LayerNorm(size_t dim, float eps = 1e-5f);
	Value forward(const Value& input) override;
	std::vector<Value> parameters() const override;
	std::vector<std::pair<std::string, Value>> named_parameters() const override;

private:
	size_t dim_;
	float eps_;
	Value gamma_, beta_;
};

// embedding.cpp: rows of weight {num_embeddings, dim} (uniform in +-1/sqrt(dim)) picked by float ids.
class Embedding : public Module {
public:
	Embedding(size_t num_embeddings, size_t dim);
	Value forward(const Value& ids) override;
	// add(forward(ids), addend) in one kernel (embedding_add)
	Value forward_add(const Value& ids, const Value& addend);
	std::vector<Value> parameters() const override;
	std::vector<std::pair<std::string, Value>> named_parameters() const override;

private:
	Value weight_;
};

// positional.cpp: x {N, T, dim} + the first T rows of a {max_len, dim} table, sinusoidal (fixed) or learned
// (uniform in +-0.02).
class PositionalEncoding : public Module {
public:
	PositionalEncoding(size_t max_len, size_t dim, bool learned = false);
	Value forward(const Value& input) override;
	// the addend forward adds to a {N, T, dim} input: the table's first T rows (the same node forward builds)
	Value rows(size_t T);
	std::vector<Value> parameters() const override;
	std::vector<std::pair<std::string, Value>> named_parameters() const override;

private:
	size_t max_len_, dim_;
	bool learned_;
	Value pe_;
};

// attention.cpp: q, k, v and output projections (dim x dim Linears) around the fused attention op.
class MultiHeadAttention : public Module {
public:
	MultiHeadAttention(size_t dim, size_t heads, bool causal = false, float dropout = 0.0f);
	Value forward(const Value& x) override;
	Value attend(const Value& query, const Value& context, const Tensor& key_padding_mask = Tensor({0}));
	// add(residual, forward(x)), the output projection's epilogue adding the residual (a transformer block's x +
	// attn(ln1(x)))
	Value forward_add(const Value& x, const Value& residual);
	std::vector<Value> parameters() const override;
	std::vector<std::pair<std::string, Value>> named_parameters() const override;
	void train(bool mode = true) override;

private:
	Value attend_impl(const Value& query, const Value& context, const Tensor& key_padding_mask, const Value* residual);
	size_t dim_, heads_;
	bool causal_;
	Linear q_, k_, v_, o_;
	Dropout drop_;
};

// sequential.cpp: layers in order; a layer that can fold a following ReLU runs both as one op.
class Sequential : public Module {
public:
	Sequential() = default;
	void add(std::unique_ptr<Module> layer);
	Value forward(const Value& input) override;
	std::vector<Value> parameters() const override;
	std::vector<std::pair<std::string, Value>> named_parameters() const override;
	std::vector<std::pair<std::string, Tensor*>> named_buffers() const override;
	void train(bool mode = true) override;
	size_t size() const { return layers_.size(); }

private:
	std::vector<std::unique_ptr<Module>> layers_;
};

// transformer.hpp:36-46.
struct TransformerConfig {
	size_t vocab_size;
	size_t dim;
	size_t heads;
	size_t layers;
	size_t max_len;
	size_t mlp_ratio = 4;
	float dropout = 0.0f;
	bool causal = true;
	bool learned_positions = false;
};

// transformer.cpp: pre-norm block x + attn(ln1(x)), then + drop(fc2(gelu(fc1(ln2(.))))).
class TransformerBlock : public Module {
public:
	TransformerBlock(size_t dim, size_t heads, size_t mlp_ratio, float dropout, bool causal);
	Value forward(const Value& x) override;
	std::vector<Value> parameters() const override;
	std::vector<std::pair<std::string, Value>> named_parameters() const override;
	void train(bool mode = true) override;

private:
	LayerNorm ln1_;
	MultiHeadAttention attn_;
	LayerNorm ln2_;
	Linear fc1_;
	GELU act_;
	Linear fc2_;
	Dropout drop_;
};

// transformer.cpp: embedding, positions, blocks, final layer norm and the vocabulary head; forward takes float ids
// {N, T} and gives logits {N, T, vocab_size}.
class Transformer : public Module {
public:
	explicit Transformer(const TransformerConfig& config);
	Value forward(const Value& ids) override;
	std::vector<Value> parameters() const override;
	std::vector<std::pair<std::string, Value>> named_parameters() const override;
	void train(bool mode = true) override;

private:
	Embedding embed_;
	PositionalEncoding pos_;
	std::vector<std::unique_ptr<TransformerBlock>> blocks_;
	LayerNorm ln_f_;
	Linear head_;
};

}  // namespace hip
}  // namespace nn
