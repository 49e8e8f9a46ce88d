// nn_hip_modules.cpp - nn-cpp's module layer over device-resident Values (include/nn_hip_modules.hpp), and the
// library-wide seeding its initial values come from (include/nn/random.hpp, src/random.cpp; src/tensor.cpp:504-522).
#include <cmath>
#include <cstdint>
#include <map>
#include <mutex>
#include <stdexcept>
#include <typeinfo>

#include "nn_hip_modules.hpp"

namespace nn {
namespace hip {

// ---- seeding (src/random.cpp): the stream derivation must match the reference's for the same initial values ----

namespace {

std::mutex g_seed_mutex;
bool g_seeded = false;
bool g_has_base = false;
uint64_t g_base = 0;
uint64_t g_epoch = 0;
std::map<std::string, uint64_t> g_counters;

// splitmix64 (Vigna's finaliser) and FNV-1a 64, the mixing steps src/random.cpp names
uint64_t mix64(uint64_t x) {
	x += 0x9e3779b97f4a7c15ULL;
	x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ULL;
	x = (x ^ (x >> 27)) * 0x94d049bb133111ebULL;
	return x ^ (x >> 31);
}

uint64_t fnv1a64(const std::string& s) {
	uint64_t h = 0xcbf29ce484222325ULL;
	for (unsigned char c : s) h = (h ^ c) * 0x100000001b3ULL;
	return h;
}

}  // namespace

void manual_seed(uint64_t seed) {
	std::lock_guard<std::mutex> lock(g_seed_mutex);
	g_seeded = true;
	g_has_base = true;
	g_base = seed;
	++g_epoch;
	g_counters.clear();
}

bool is_seeded() {
	std::lock_guard<std::mutex> lock(g_seed_mutex);
	return g_seeded;
}

uint64_t seed_epoch() {
	std::lock_guard<std::mutex> lock(g_seed_mutex);
	return g_epoch;
}

std::mt19937 derive_generator(const std::string& stream) {
	std::lock_guard<std::mutex> lock(g_seed_mutex);
	if (!g_has_base) {
		std::random_device rd;
		g_base = (static_cast<uint64_t>(rd()) << 32) ^ rd();
		g_has_base = true;
	}
	const uint64_t k = g_counters[stream]++;
	const uint64_t s = mix64(g_base ^ fnv1a64(stream) ^ (k * 0x9e3779b97f4a7c15ULL));
	std::seed_seq seq{static_cast<uint32_t>(s), static_cast<uint32_t>(s >> 32)};
	return std::mt19937(seq);
}

Tensor Tensor::random(std::vector<size_t> shape, float lo, float hi) {
	// one generator per seed epoch, continued by later calls (tensor.cpp:504-522); not for concurrent use, as there
	static std::mt19937 gen;
	static uint64_t epoch = 0;
	static bool init = false;
	if (!init || epoch != seed_epoch()) {
		epoch = seed_epoch();
		gen = derive_generator("tensor.random");
		init = true;
	}
	std::uniform_real_distribution<float> dist(lo, hi);
	size_t n = 1;
	for (size_t d : shape) n *= d;
	std::vector<float> host(n);
	for (float& v : host) v = dist(gen);
	Tensor out = Tensor::from_host(std::move(shape), host.data());
	synchronize();  // host is released on return
	return out;
}

// ---- modules ----

Value Flatten::forward(const Value& input) {
	const auto& s = input.data().shape();
	if (s.empty() || s[0] == 0) throw TensorShapeError("nn::hip: Flatten needs a non-empty leading axis");
	const size_t n = s[0];
	return reshape(input, {n, input.data().size() / n});
}

namespace {

float bound(size_t fan_in) { return 1.0f / std::sqrt(static_cast<float>(fan_in)); }

}  // namespace

Linear::Linear(size_t in_features, size_t out_features)
	: weight_(Value::leaf(Tensor::random({out_features, in_features}, -bound(in_features), bound(in_features)), true)),
	  bias_(Value::leaf(Tensor({out_features}), true)) {}

Value Linear::forward(const Value& input) { return linear(input, weight_, bias_); }
std::vector<Value> Linear::parameters() const { return {weight_, bias_}; }
std::vector<std::pair<std::string, Value>> Linear::named_parameters() const {
	return {{"weight", weight_}, {"bias", bias_}};
}

Conv2d::Conv2d(size_t in_channels, size_t out_channels, size_t kernel_size, size_t stride, size_t padding)
	: weight_(Value::leaf(Tensor::random({out_channels, in_channels, kernel_size, kernel_size},
	                                     -bound(in_channels * kernel_size * kernel_size),
	                                     bound(in_channels * kernel_size * kernel_size)),
	                      true)),
	  bias_(Value::leaf(Tensor({out_channels}), true)),
	  stride_(stride),
	  padding_(padding) {}

Value Conv2d::forward(const Value& input) {
	return conv2d(input, weight_, bias_, static_cast<int>(stride_), static_cast<int>(padding_));
}
Value Conv2d::forward_relu(const Value& input) {
	return conv2d_relu(input, weight_, bias_, static_cast<int>(stride_), static_cast<int>(padding_));
}
std::vector<Value> Conv2d::parameters() const { return {weight_, bias_}; }
std::vector<std::pair<std::string, Value>> Conv2d::named_parameters() const {
	return {{"weight", weight_}, {"bias", bias_}};
}

Dropout::Dropout(float p) : p_(p), gen_(derive_generator("dropout")) {
	if (!(p >= 0.0f && p <= 1.0f)) throw std::invalid_argument("Dropout: p must be in [0, 1]");
}

Value Dropout::forward(const Value& input) {
	if (!training_ || p_ == 0.0f) return input;
	std::vector<float> mask(input.data().size(), 0.0f);
	if (p_ < 1.0f) {  // p == 1 zeroes everything and draws nothing (dropout.cpp:24-25)
		const float keep_scale = 1.0f / (1.0f - p_);
		for (float& m : mask) {
			// the top 24 bits as a uniform in [0, 1) (dropout.cpp:27-30)
			const float u = static_cast<float>(gen_() >> 8) * (1.0f / 16777216.0f);
			m = u < p_ ? 0.0f : keep_scale;
		}
	}
	Tensor mt = Tensor::from_host(input.data().shape(), mask.data());
	synchronize();  // mask is released on return
	return mul(input, Value::leaf(std::move(mt)));
}

LayerNorm::LayerNorm(size_t dim, float eps)
	: dim_(dim), eps_(eps), gamma_(Value::leaf(Tensor({dim}, 1.0f), true)), beta_(Value::leaf(Tensor({dim}), true)) {}

Value LayerNorm::forward(const Value& input) {
	const auto& s = input.data().shape();
	if (s.empty() || s.back() != dim_) throw TensorShapeError("nn::hip: LayerNorm input's last axis differs from dim");
	return layernorm(input, gamma_, beta_, eps_);
}
std::vector<Value> LayerNorm::parameters() const { return {gamma_, beta_}; }
std::vector<std::pair<std::string, Value>> LayerNorm::named_parameters() const {
	return {{"gamma", gamma_}, {"beta", beta_}};
}

Embedding::Embedding(size_t num_embeddings, size_t dim)
	: weight_(Value::leaf(Tensor::random({num_embeddings, dim}, -bound(dim), bound(dim)), true)) {}

Value Embedding::forward(const Value& ids) { return embedding(weight_, ids.data()); }
Value Embedding::forward_add(const Value& ids, const Value& addend) { return embedding_add(weight_, ids.data(), addend); }
std::vector<Value> Embedding::parameters() const { return {weight_}; }
std::vector<std::pair<std::string, Value>> Embedding::named_parameters() const { return {{"weight", weight_}}; }

PositionalEncoding::PositionalEncoding(size_t max_len, size_t dim, bool learned)
	: max_len_(max_len),
	  dim_(dim),
	  learned_(learned),
	  pe_(learned ? Value::leaf(Tensor::random({max_len, dim}, -0.02f, 0.02f), true)
	              : Value::leaf(sinusoidal_table(max_len, dim), false)) {}

Value PositionalEncoding::forward(const Value& input) {
	const auto& s = input.data().shape();
	if (s.size() != 3 || s[1] > max_len_ || s[2] != dim_)
		throw TensorShapeError("nn::hip: PositionalEncoding takes {N, T <= max_len, dim}");
	return add(input, rows(s[1]));
}
Value PositionalEncoding::rows(size_t T) {
	if (T > max_len_) throw TensorShapeError("nn::hip: PositionalEncoding takes {N, T <= max_len, dim}");
	return slice(pe_, 0, 0, T);
}
std::vector<Value> PositionalEncoding::parameters() const {
	return learned_ ? std::vector<Value>{pe_} : std::vector<Value>{};
}
std::vector<std::pair<std::string, Value>> PositionalEncoding::named_parameters() const {
	return learned_ ? std::vector<std::pair<std::string, Value>>{{"pe", pe_}}
	                : std::vector<std::pair<std::string, Value>>{};
}

MultiHeadAttention::MultiHeadAttention(size_t dim, size_t heads, bool causal, float dropout)
	: dim_(dim), heads_(heads), causal_(causal), q_(dim, dim), k_(dim, dim), v_(dim, dim), o_(dim, dim), drop_(dropout) {
	if (heads == 0 || dim % heads != 0) throw std::invalid_argument("MultiHeadAttention: dim must be divisible by heads");
}

Value MultiHeadAttention::forward(const Value& x) { return attend(x, x); }

Value MultiHeadAttention::forward_add(const Value& x, const Value& residual) {
	return attend_impl(x, x, Tensor({0}), &residual);
}

Value MultiHeadAttention::attend(const Value& query, const Value& context, const Tensor& key_padding_mask) {
	return attend_impl(query, context, key_padding_mask, nullptr);
}

Value MultiHeadAttention::attend_impl(const Value& query, const Value& context, const Tensor& key_padding_mask,
                                      const Value* residual) {
	const auto& qs = query.data().shape();
	const auto& cs = context.data().shape();
	if (qs.size() != 3 || cs.size() != 3 || qs[2] != dim_ || cs[2] != dim_ || qs[0] != cs[0])
		throw TensorShapeError("nn::hip: MultiHeadAttention takes {N, T, dim} query and context");
	if (causal_ && qs[1] != cs[1]) throw TensorShapeError("nn::hip: causal attention needs Tq == Tk");
	if (key_padding_mask.size() != 0 && key_padding_mask.shape() != std::vector<size_t>{qs[0], cs[1]})
		throw TensorShapeError("nn::hip: key_padding_mask must be {N, Tk}");
	if (drop_.active())
		throw std::invalid_argument(
		    "nn::hip::MultiHeadAttention: dropout on the attention weights in training mode is not available");
	// one op reads each head in place (attention.cpp:33-35); self-attention's three projections in one launch
	Value a;
	if (query.impl() == context.impl()) {
		const std::vector<Value> qkv = linear_many(query, {{q_.weight(), q_.bias()}, {k_.weight(), k_.bias()},
		                                                   {v_.weight(), v_.bias()}});
		a = attention(qkv[0], qkv[1], qkv[2], heads_, key_padding_mask, causal_);
	} else {
		a = attention(q_.forward(query), k_.forward(context), v_.forward(context), heads_, key_padding_mask, causal_);
	}
	return residual ? o_.forward_add(a, *residual) : o_.forward(a);
}

std::vector<Value> MultiHeadAttention::parameters() const {
	std::vector<Value> out;
	for (const auto& p : named_parameters()) out.push_back(p.second);
	return out;
}

std::vector<std::pair<std::string, Value>> MultiHeadAttention::named_parameters() const {
	std::vector<std::pair<std::string, Value>> out;
	const std::pair<const char*, const Linear*> subs[] = {{"q.", &q_}, {"k.", &k_}, {"v.", &v_}, {"o.", &o_}};
	for (const auto& s : subs)
		for (const auto& p : s.second->named_parameters()) out.emplace_back(s.first + p.first, p.second);
	return out;
}

void MultiHeadAttention::train(bool mode) {
	drop_.train(mode);
	training_ = mode;
}

void Sequential::add(std::unique_ptr<Module> layer) { layers_.push_back(std::move(layer)); }

Value Sequential::forward(const Value& input) {
	Value cur = input;
	for (size_t i = 0; i < layers_.size(); ++i) {
		Module& m = *layers_[i];
		const Module* next = i + 1 < layers_.size() ? layers_[i + 1].get() : nullptr;
		const Module* after = i + 2 < layers_.size() ? layers_[i + 2].get() : nullptr;
		if (next && m.can_fuse_relu() && typeid(*next) == typeid(ReLU)) {
			// Conv2d, ReLU, MaxPool2d: conv2d_relu and maxpool2d with both forwards in one pass (same nodes, same bits)
			const auto* conv = typeid(m) == typeid(Conv2d) ? static_cast<const Conv2d*>(&m) : nullptr;
			const auto* pool = after && typeid(*after) == typeid(MaxPool2d) ? static_cast<const MaxPool2d*>(after) : nullptr;
			if (conv && pool) {
				cur = conv2d_relu_maxpool2d(cur, conv->weight(), conv->bias(), static_cast<int>(conv->stride()),
				                            static_cast<int>(conv->padding()), pool->kernel_size(), pool->stride());
				i += 2;
				continue;
			}
			cur = m.forward_relu(cur);  // sequential.cpp:20-24
			++i;
			continue;
		}
		cur = m.forward(cur);
	}
	return cur;
}

std::vector<Value> Sequential::parameters() const {
	std::vector<Value> all;
	for (const auto& l : layers_) {
		std::vector<Value> p = l->parameters();
		all.insert(all.end(), p.begin(), p.end());
	}
	return all;
}

std::vector<std::pair<std::string, Value>> Sequential::named_parameters() const {
	std::vector<std::pair<std::string, Value>> all;
	for (size_t i = 0; i < layers_.size(); ++i)
		for (auto& e : layers_[i]->named_parameters()) all.emplace_back(std::to_string(i) + "." + e.first, e.second);
	return all;
}

std::vector<std::pair<std::string, Tensor*>> Sequential::named_buffers() const {
	std::vector<std::pair<std::string, Tensor*>> all;
	for (size_t i = 0; i < layers_.size(); ++i)
		for (auto& e : layers_[i]->named_buffers()) all.emplace_back(std::to_string(i) + "." + e.first, e.second);
	return all;
}

void Sequential::train(bool mode) {
	for (auto& l : layers_) l->train(mode);
	training_ = mode;
}

namespace {

size_t checked_dim(size_t dim, size_t heads, size_t mlp_ratio) {
	if (dim == 0 || heads == 0 || mlp_ratio == 0) throw std::invalid_argument("Transformer: sizes must be non-zero");
	if (dim % heads != 0) throw std::invalid_argument("Transformer: dim must be divisible by heads");
	return dim;
}

size_t checked_vocab(const TransformerConfig& c) {
	checked_dim(c.dim, c.heads, c.mlp_ratio);
	if (c.vocab_size == 0 || c.layers == 0 || c.max_len == 0)
		throw std::invalid_argument("Transformer: sizes must be non-zero");
	return c.vocab_size;
}

void append(std::vector<std::pair<std::string, Value>>& out, const std::string& prefix, const Module& m) {
	for (const auto& p : m.named_parameters()) out.emplace_back(prefix + p.first, p.second);
}

}  // namespace

TransformerBlock::TransformerBlock(size_t dim, size_t heads, size_t mlp_ratio, float dropout, bool causal)
	: ln1_(checked_dim(dim, heads, mlp_ratio)),
	  attn_(dim, heads, causal, dropout),
	  ln2_(dim),
	  fc1_(dim, mlp_ratio * dim),
	  fc2_(mlp_ratio * dim, dim),
	  drop_(dropout) {}

Value TransformerBlock::forward(const Value& x) {
	// x + attn(ln1(x)) and h + drop(fc2(...)) with each add in the producing linear's epilogue (the same nodes and
	// bits); an active dropout between fc2 and the add keeps the ops apart
	const Value h = attn_.forward_add(ln1_.forward(x), x);
	const Value f = fc1_.forward_gelu(ln2_.forward(h));  // act_ is the GELU
	return drop_.active() ? add(h, drop_.forward(fc2_.forward(f))) : fc2_.forward_add(f, h);
}

std::vector<Value> TransformerBlock::parameters() const {
	std::vector<Value> out;
	for (const auto& p : named_parameters()) out.push_back(p.second);
	return out;
}

std::vector<std::pair<std::string, Value>> TransformerBlock::named_parameters() const {
	std::vector<std::pair<std::string, Value>> out;
	append(out, "ln1.", ln1_);
	append(out, "attn.", attn_);
	append(out, "ln2.", ln2_);
	append(out, "fc1.", fc1_);
	append(out, "fc2.", fc2_);
	return out;
}

void TransformerBlock::train(bool mode) {
	attn_.train(mode);
	drop_.train(mode);
	training_ = mode;
}

Transformer::Transformer(const TransformerConfig& c)
	: embed_(checked_vocab(c), c.dim), pos_(c.max_len, c.dim, c.learned_positions), ln_f_(c.dim), head_(c.dim, c.vocab_size) {
	for (size_t i = 0; i < c.layers; ++i)
		blocks_.push_back(std::make_unique<TransformerBlock>(c.dim, c.heads, c.mlp_ratio, c.dropout, c.causal));
}

Value Transformer::forward(const Value& ids) {
	// pos(embed(ids)) with the positions added in the lookup's kernel for {N, T} ids (the same nodes and bits)
	const auto& is = ids.data().shape();
	Value h = is.size() == 2 ? embed_.forward_add(ids, pos_.rows(is[1])) : pos_.forward(embed_.forward(ids));
	for (auto& b : blocks_) h = b->forward(h);
	return head_.forward(ln_f_.forward(h));
}

std::vector<Value> Transformer::parameters() const {
	std::vector<Value> out;
	for (const auto& p : named_parameters()) out.push_back(p.second);
	return out;
}

std::vector<std::pair<std::string, Value>> Transformer::named_parameters() const {
	std::vector<std::pair<std::string, Value>> out;
	append(out, "embed.", embed_);
	append(out, "pos.", pos_);
	for (size_t i = 0; i < blocks_.size(); ++i) append(out, "blocks." + std::to_string(i) + ".", *blocks_[i]);
	append(out, "ln_f.", ln_f_);
	append(out, "head.", head_);
	return out;
}

void Transformer::train(bool mode) {
	for (auto& b : blocks_) b->train(mode);
	training_ = mode;
}

}  // namespace hip
}  // namespace nn
