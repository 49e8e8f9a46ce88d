// nn_hip.cpp - include/nn_hip.hpp: nn-cpp's op surface over device-resident tensors, on the C ABI of include/nnh.h.
#include "nn_hip.hpp"

#include <algorithm>
#include <cmath>
#include <map>
#include <mutex>
#include <unordered_set>

#include "nnh.h"

namespace nn {
namespace hip {

namespace {

hipStream_t g_stream = nullptr;

void check(int rc) {
	if (rc == NNH_OK) return;
	const std::string msg = std::string("nn::hip: ") + nnh_last_error();
	if (rc == NNH_ERR_SHAPE) throw TensorShapeError(msg);
	if (rc == NNH_ERR_HIP) throw HipError(msg);
	throw std::invalid_argument(msg);
}

void check_hip(hipError_t e, const char* what) {
	if (e != hipSuccess) throw HipError(std::string("nn::hip: ") + what + ": " + hipGetErrorString(e));
}

size_t numel(const std::vector<size_t>& s) {
	size_t n = 1;
	for (size_t d : s) n *= d;
	return n;
}

// Caching allocator: free blocks kept by rounded size and handed out again (all work is on g_stream, so a block
// released after its last use was enqueued can be reused by work enqueued later).
class Cache {
public:
	void* get(size_t bytes, size_t& rounded) {
		rounded = round(bytes);
		std::lock_guard<std::mutex> lock(mu_);
		auto it = free_.find(rounded);
		if (it != free_.end()) {
			void* p = it->second;
			free_.erase(it);
			return p;
		}
		void* p = nullptr;
		check_hip(hipMalloc(&p, rounded), "device allocation");
		held_ += rounded;
		return p;
	}
	void put(void* p, size_t rounded) {
		std::lock_guard<std::mutex> lock(mu_);
		free_.emplace(rounded, p);
	}
	size_t held() {
		std::lock_guard<std::mutex> lock(mu_);
		return held_;
	}
	void release() {
		check_hip(hipStreamSynchronize(g_stream), "synchronize");
		std::lock_guard<std::mutex> lock(mu_);
		for (auto& e : free_) {
			(void)hipFree(e.second);
			held_ -= e.first;
		}
		free_.clear();
	}

private:
	static size_t round(size_t b) {
		if (b <= 256) return 256;
		if (b <= (size_t(1) << 20)) return (b + 511) & ~size_t(511);
		return (b + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1);
	}
	std::mutex mu_;
	std::multimap<size_t, void*> free_;
	size_t held_ = 0;
};

Cache& cache() {
	static Cache* c = new Cache;  // kept until the process ends (the HIP runtime may be gone at static teardown)
	return *c;
}

thread_local bool g_grad_enabled = true;

std::vector<size_t> to_vec(const size_t* p, size_t n) { return std::vector<size_t>(p, p + n); }

}  // namespace

struct Block {
	void* p = nullptr;
	size_t bytes = 0;
	explicit Block(size_t b) { p = cache().get(std::max<size_t>(b, 1), bytes); }
	~Block() { cache().put(p, bytes); }
	Block(const Block&) = delete;
	Block& operator=(const Block&) = delete;
};

void set_stream(hipStream_t s) {
	if (s == g_stream) return;
	check_hip(hipStreamSynchronize(g_stream), "synchronize");
	g_stream = s;
}
hipStream_t current_stream() { return g_stream; }
void synchronize() { check_hip(hipStreamSynchronize(g_stream), "synchronize"); }
size_t allocator_bytes() { return cache().held(); }
void empty_cache() { cache().release(); }

// ---- Tensor ----

Tensor::Tensor() : shape_{0}, size_(0) {}

Tensor::Tensor(std::vector<size_t> shape, float value) : Tensor(empty(std::move(shape))) { fill_(value); }

Tensor Tensor::empty(std::vector<size_t> shape) {
	Tensor t;
	t.shape_ = std::move(shape);
	t.size_ = numel(t.shape_);
	t.storage_ = std::make_shared<Block>(t.size_ * sizeof(float));
	return t;
}

Tensor Tensor::from_host(std::vector<size_t> shape, const float* data) {
	Tensor t = empty(std::move(shape));
	if (t.size_) check_hip(hipMemcpyAsync(t.data(), data, t.size_ * 4, hipMemcpyHostToDevice, g_stream), "copy in");
	return t;
}

void Tensor::to_host(float* out) const {
	if (size_) check_hip(hipMemcpyAsync(out, data(), size_ * 4, hipMemcpyDeviceToHost, g_stream), "copy out");
	synchronize();
}

std::vector<float> Tensor::to_host() const {
	std::vector<float> v(size_);
	to_host(v.data());
	return v;
}

float* Tensor::data() const { return storage_ ? static_cast<float*>(storage_->p) : nullptr; }

Tensor Tensor::reshape(std::vector<size_t> new_shape) const {
	if (numel(new_shape) != size_) throw TensorShapeError("nn::hip: reshape changes the element count");
	Tensor t = *this;
	t.shape_ = std::move(new_shape);
	return t;
}

void Tensor::zero_() { fill_(0.0f); }

void Tensor::fill_(float value) {
	if (!size_) return;
	if (value == 0.0f && !std::signbit(value)) {
		// Tensor::sum(0) over no rows stores +0 everywhere: a fill kernel (no memset node if the stream is captured)
		check(nnh_tensor_sum0(nullptr, 0, size_, data(), 0, g_stream));
		return;
	}
	std::vector<float> host(size_, value);
	check_hip(hipMemcpyAsync(data(), host.data(), size_ * 4, hipMemcpyHostToDevice, g_stream), "fill");
	synchronize();
}

Tensor matmul(const Tensor& a, const Tensor& b, bool trans_a, bool trans_b) {
	size_t out[16];
	int nd = 0;
	check(nnh_matmul_shape(a.shape().data(), (int)a.ndim(), b.shape().data(), (int)b.ndim(), trans_a, trans_b, out, &nd));
	Tensor r = Tensor::empty(to_vec(out, nd));
	check(nnh_matmul(a.data(), a.shape().data(), (int)a.ndim(), b.data(), b.shape().data(), (int)b.ndim(), trans_a,
	                 trans_b, r.data(), g_stream));
	return r;
}

// ---- Value ----

NoGradGuard::NoGradGuard() : previous_(g_grad_enabled) { g_grad_enabled = false; }
NoGradGuard::~NoGradGuard() { g_grad_enabled = previous_; }
bool NoGradGuard::grad_enabled() { return g_grad_enabled; }

Value Value::leaf(Tensor data, bool requires_grad) {
	auto n = std::make_shared<NodeImpl>();
	n->requires_grad = requires_grad;
	if (requires_grad) n->grad = Tensor(data.shape(), 0.0f);  // a leaf's gradient starts as zeros (value.cpp:18-21)
	n->data = std::move(data);
	return Value(n);
}

Value Value::node(Tensor data, std::vector<Value> parents, std::function<void(const Tensor&)> backward_fn) {
	if (!g_grad_enabled) return leaf(std::move(data), false);
	auto n = std::make_shared<NodeImpl>();
	n->data = std::move(data);
	n->requires_grad = true;
	n->parents = std::move(parents);
	n->backward_fn = std::move(backward_fn);
	return Value(n);
}

Tensor& Value::data() const { return impl_->data; }

Tensor& Value::grad() const {
	if (impl_->grad_fresh) {
		impl_->grad.zero_();
		impl_->grad_fresh = false;
	}
	return impl_->grad;
}

Tensor& Value::grad_accum(bool& first) const {
	first = impl_->grad_fresh;
	impl_->grad_fresh = false;
	return impl_->grad;
}

bool Value::requires_grad() const { return impl_->requires_grad; }

// zero_grad marks the gradient fresh instead of filling it with zeros: the next backward rule stores its
// contribution as nn-cpp adds it to zeros (every rule's first write is that sum: s + 0.0f, or a chain from +0, which
// is never -0), and grad() fills a gradient no rule wrote with zeros when it is read. No launch.
void Value::zero_grad() const {
	if (impl_->grad.shape() != impl_->data.shape()) impl_->grad = Tensor::empty(impl_->data.shape());
	impl_->grad_fresh = true;
}

void zero_grad(const std::vector<Value>& values) {
	for (const Value& v : values) v.zero_grad();
}

void Value::backward() const {
	if (impl_->data.size() != 1) throw TensorShapeError("nn::hip: backward() needs a one-element value");
	backward(Tensor(impl_->data.shape(), 1.0f));
}

void Value::backward(const Tensor& seed) const {
	if (seed.shape() != impl_->data.shape()) throw TensorShapeError("nn::hip: the seed must have the output's shape");
	// value.cpp:80-132: an iterative post-order walk, gradients sized (not zeroed) and marked fresh, the output's
	// set, then every backward rule in reverse topological order
	std::vector<Value> topo;
	std::unordered_set<NodeImpl*> expanded, done;
	std::vector<Value> stack{*this};
	while (!stack.empty()) {
		Value v = stack.back();
		if (done.count(v.impl())) {
			stack.pop_back();
			continue;
		}
		if (expanded.count(v.impl())) {
			stack.pop_back();
			done.insert(v.impl());
			topo.push_back(v);
			continue;
		}
		expanded.insert(v.impl());
		for (const Value& p : v.impl()->parents)
			if (!expanded.count(p.impl())) stack.push_back(p);
	}
	for (const Value& v : topo) {
		v.impl()->consumers = 0;
		if (v.impl()->backward_fn) {
			// a buffer of its own every walk: an earlier walk may have left it sharing storage (take_grad, the seed)
			v.impl()->grad = Tensor::empty(v.impl()->data.shape());
			v.impl()->grad_fresh = true;
		}
	}
	for (const Value& v : topo)
		for (const Value& p : v.impl()->parents) ++p.impl()->consumers;
	if (impl_->backward_fn) {
		// an intermediate output's gradient is the seed itself (shared storage, no copy): nothing writes it during the
		// walk (only single-use pass-through operands take a gradient's storage, and no contribution reaches them
		// later), and the next walk gives the node a buffer of its own again
		impl_->grad = seed;
	} else {
		if (impl_->grad.shape() != impl_->data.shape()) impl_->grad = Tensor::empty(impl_->data.shape());
		if (seed.size())
			check_hip(hipMemcpyAsync(impl_->grad.data(), seed.data(), seed.size() * 4, hipMemcpyDeviceToDevice, g_stream),
			          "seed");
	}
	impl_->grad_fresh = false;
	for (auto it = topo.rbegin(); it != topo.rend(); ++it)
		if (it->impl()->backward_fn) it->impl()->backward_fn(it->grad());
}

// ---- ops ----

namespace {

float* grad_if(const Value& v, bool& first) {
	first = false;
	return v.requires_grad() ? v.grad_accum(first).data() : nullptr;
}

// A pass-through rule (add, reshape) hands its gradient g to an operand that is an intermediate node, used only by
// this node and not yet written: the operand's gradient takes g's storage (the values a store of g would give,
// nothing is written to it later), instead of a copy. Returns whether it did.
bool take_grad(const Value& v, const Tensor& g) {
	NodeImpl* n = v.impl();
	if (!n->requires_grad || !n->backward_fn || !n->grad_fresh || n->consumers != 1) return false;
	n->grad = g.reshape(n->data.shape());
	n->grad_fresh = false;
	return true;
}

// A byte or uint32 side buffer an op keeps for its backward (conv's alive flags, pooling's argmax).
std::shared_ptr<Block> side_buffer(size_t bytes) { return std::make_shared<Block>(bytes); }

Value matmul_op(const Value& a, const Value& b, bool bt) {
	Tensor r = matmul(a.data(), b.data(), false, bt);
	return Value::node(std::move(r), {a, b}, [a, b, bt](const Tensor& g) {
		bool fa = false, fb = false;
		float* da = grad_if(a, fa);  // a first: one node passed as both operands is stored by dA, added to by dB
		float* db = grad_if(b, fb);
		if (!da && !db) return;
		const Tensor& A = a.data();
		const Tensor& B = b.data();
		check(nnh_matmul_backward(g.data(), A.data(), A.shape().data(), (int)A.ndim(), B.data(), B.shape().data(),
		                          (int)B.ndim(), bt, da, fa, db, fb, g_stream));
	});
}

struct ConvShape {
	size_t N, Cin, H, W, Cout, kh, kw, ho, wo;
};

ConvShape conv_shape(const Value& x, const Value& w, const Value& b, int stride, int padding) {
	const auto& xs = x.data().shape();
	const auto& ws = w.data().shape();
	// ops.cpp:1347-1365
	if (xs.size() != 4 || ws.size() != 4 || xs[1] != ws[1] || b.data().shape() != std::vector<size_t>{ws[0]})
		throw TensorShapeError("nn::hip: conv2d shapes");
	if (stride <= 0 || padding < 0 || ws[2] > xs[2] + 2 * (size_t)padding || ws[3] > xs[3] + 2 * (size_t)padding)
		throw TensorShapeError("nn::hip: conv2d geometry");
	ConvShape c{xs[0], xs[1], xs[2], xs[3], ws[0], ws[2], ws[3], 0, 0};
	c.ho = (c.H + 2 * padding - c.kh) / stride + 1;
	c.wo = (c.W + 2 * padding - c.kw) / stride + 1;
	return c;
}

// Whether a conv node keeps its ReLU's alive flags for the backward.
bool keeps_alive(const Value& x, const Value& w, const Value& b, bool fuse_relu) {
	return fuse_relu && NoGradGuard::grad_enabled() && (x.requires_grad() || w.requires_grad() || b.requires_grad());
}

// The conv node over its forward's outputs y and alive (packed: one bit per output, nnh.h's packed form).
Value conv_node(const Value& x, const Value& w, const Value& b, int stride, int padding, const ConvShape& c, Tensor y,
                std::shared_ptr<Block> alive, bool packed) {
	return Value::node(std::move(y), {x, w, b}, [=](const Tensor& g) {
		// ops.cpp:1418-1463: dx taken first (grad_accum), then db and dW (grad() +=, a fresh one zeroed first,
		// which gives the sum itself)
		bool fx = false, fb = false, fw = false;
		float* dx = grad_if(x, fx);
		float* db = grad_if(b, fb);
		float* dw = grad_if(w, fw);
		if (!dx && !dw && !db) return;
		const unsigned char* al = alive ? static_cast<const unsigned char*>(alive->p) : nullptr;
		if (packed)
			check(nnh_conv2d_backward_packed(g.data(), x.data().data(), w.data().data(), al, c.N, c.Cin, c.H, c.W, c.Cout,
			                                 c.kh, c.kw, stride, padding, dx, fx, dw, fw, db, fb, g_stream));
		else
			check(nnh_conv2d_backward(g.data(), x.data().data(), w.data().data(), al, c.N, c.Cin, c.H, c.W, c.Cout, c.kh,
			                          c.kw, stride, padding, dx, fx, dw, fw, db, fb, g_stream));
	});
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

Value conv_op(const Value& x, const Value& w, const Value& b, int stride, int padding, bool fuse_relu) {
	const ConvShape c = conv_shape(x, w, b, stride, padding);
	Tensor y = Tensor::empty({c.N, c.Cout, c.ho, c.wo});
	const bool keep = keeps_alive(x, w, b, fuse_relu);
	// a first layer keeps its flags as bits (its backward is their only reader)
	const bool packed = keep && aligned16(x.data().data()) && aligned16(y.data()) &&
	                    nnh_conv2d_packed_supported(c.N, c.Cin, c.H, c.W, c.Cout, c.kh, c.kw, stride, padding, 0);
	std::shared_ptr<Block> alive = keep ? side_buffer(packed ? (y.size() + 7) / 8 : y.size()) : nullptr;
	unsigned char* al = alive ? static_cast<unsigned char*>(alive->p) : nullptr;
	if (packed)
		check(nnh_conv2d_relu_forward_packed(x.data().data(), c.N, c.Cin, c.H, c.W, w.data().data(), c.Cout, c.kh, c.kw,
		                                     b.data().data(), stride, padding, y.data(), al, g_stream));
	else
		check(nnh_conv2d_forward(x.data().data(), c.N, c.Cin, c.H, c.W, w.data().data(), c.Cout, c.kh, c.kw,
		                         b.data().data(), stride, padding, fuse_relu, y.data(), al, g_stream));
	return conv_node(x, w, b, stride, padding, c, std::move(y), std::move(alive), packed);
}

// ops.cpp:1610-1617: the pooled shape, or TensorShapeError.
std::vector<size_t> pool_shape(const std::vector<size_t>& xs, size_t kernel_size, size_t stride) {
	if (xs.size() != 4) throw TensorShapeError("nn::hip: maxpool2d needs {N, C, H, W}");
	if (kernel_size == 0 || stride == 0 || kernel_size > xs[2] || kernel_size > xs[3])
		throw TensorShapeError("nn::hip: maxpool2d geometry");
	return {xs[0], xs[1], (xs[2] - kernel_size) / stride + 1, (xs[3] - kernel_size) / stride + 1};
}

// The pool node over its forward's output y and argmax (packed: 2-bit window positions of a 2 x 2, stride-2 pool).
Value pool_node(const Value& x, size_t kernel_size, size_t stride, Tensor y, std::shared_ptr<Block> arg,
                bool packed = false) {
	const auto& xs = x.data().shape();
	const size_t N = xs[0], C = xs[1], H = xs[2], W = xs[3];
	return Value::node(std::move(y), {x}, [=](const Tensor& g) {
		bool first = false;
		float* dx = grad_if(x, first);
		if (!dx) return;
		if (packed)
			check(nnh_maxpool2d_backward_packed(g.data(), static_cast<const unsigned char*>(arg->p), N, C, H, W, dx, first,
			                                    g_stream));
		else
			check(nnh_maxpool2d_backward(g.data(), static_cast<const unsigned int*>(arg->p), N, C, H, W, kernel_size,
			                             stride, dx, first, g_stream));
	});
}

}  // namespace

Value matmul(const Value& a, const Value& b) { return matmul_op(a, b, false); }
Value matmul_bt(const Value& a, const Value& b) { return matmul_op(a, b, true); }

namespace {

// nn::linear's node (ops.cpp:714-745); with relu, its forward also applies the ReLU that follows it in the same
// launch (the GEMM epilogue) and a relu node over it is returned: the same two nodes and bits as relu(linear(...)).
// The linear node's own data is then the ReLU's output: no backward rule reads it (linear's reads x and W, relu's
// masks with its output, y > 0 exactly where its input is), and the caller only holds the relu node.
// The linear node over its forward's output y (ops.cpp:733-745).
Value linear_node(const Value& x, const Value& weight, const Value& bias, const Tensor& y) {
	const size_t n = weight.data().shape()[0], K = weight.data().shape()[1];
	return Value::node(y, {x, weight, bias}, [x, weight, bias, n, K](const Tensor& g) {
		bool fx = false, fw = false, fb = false;
		float* dx = grad_if(x, fx);
		float* dw = grad_if(weight, fw);
		float* db = grad_if(bias, fb);
		if (!dx && !dw && !db) return;
		const auto& xs2 = x.data().shape();
		check(nnh_linear_backward(g.data(), x.data().data(), weight.data().data(), xs2.data(), (int)xs2.size() - 1, K, n,
		                          dx, fx, dw, fw, db, fb, g_stream));
	});
}

Value linear_op(const Value& x, const Value& weight, const Value& bias, bool relu) {
	const auto& xs = x.data().shape();
	const auto& ws = weight.data().shape();
	// ops.cpp:717-719
	if (xs.size() < 2 || ws.size() != 2 || xs.back() != ws[1] || bias.data().shape() != std::vector<size_t>{ws[0]})
		throw TensorShapeError("nn::hip: linear shapes");
	const size_t n = ws[0], K = ws[1], M = x.data().size() / std::max<size_t>(K, 1);
	std::vector<size_t> out(xs.begin(), xs.end() - 1);
	out.push_back(n);
	Tensor y = Tensor::empty(out);
	check(nnh_linear_forward(x.data().data(), K ? M : numel(std::vector<size_t>(xs.begin(), xs.end() - 1)), K,
	                         weight.data().data(), n, bias.data().data(), relu ? 1 : 0, y.data(), g_stream));
	Value h = linear_node(x, weight, bias, y);
	if (!relu) return h;
	// ops.cpp:775-793 on h, masked with the output
	return Value::node(y, {h}, [h, y](const Tensor& g) {
		bool first = false;
		float* dh = grad_if(h, first);
		if (dh) check(nnh_relu_backward(y.data(), g.data(), dh, first, g.size(), g_stream));
	});
}

}  // namespace

Value linear(const Value& x, const Value& weight, const Value& bias) { return linear_op(x, weight, bias, false); }

Value linear_relu(const Value& x, const Value& weight, const Value& bias) { return linear_op(x, weight, bias, true); }

Value relu(const Value& x) {
	Tensor y = Tensor::empty(x.data().shape());
	check(nnh_relu_forward(x.data().data(), y.data(), y.size(), g_stream));
	return Value::node(std::move(y), {x}, [x](const Tensor& g) {
		bool first = false;
		float* dx = grad_if(x, first);
		if (dx) check(nnh_relu_backward(x.data().data(), g.data(), dx, first, g.size(), g_stream));
	});
}

Value reshape(const Value& x, std::vector<size_t> new_shape) {
	Tensor y = x.data().reshape(std::move(new_shape));
	return Value::node(std::move(y), {x}, [x](const Tensor& g) {
		if (take_grad(x, g)) return;
		bool first = false;
		float* dx = grad_if(x, first);
		if (dx) check(nnh_add_to_grad(dx, g.data(), g.size(), first, g_stream));
	});
}

Value conv2d(const Value& x, const Value& weight, const Value& bias, int stride, int padding) {
	return conv_op(x, weight, bias, stride, padding, false);
}

Value conv2d_relu(const Value& x, const Value& weight, const Value& bias, int stride, int padding) {
	return conv_op(x, weight, bias, stride, padding, true);
}

Value maxpool2d(const Value& x, size_t kernel_size, size_t stride) {
	const auto& xs = x.data().shape();
	Tensor y = Tensor::empty(pool_shape(xs, kernel_size, stride));
	std::shared_ptr<Block> arg = side_buffer(y.size() * 4);
	check(nnh_maxpool2d_forward(x.data().data(), xs[0], xs[1], xs[2], xs[3], kernel_size, stride, y.data(),
	                            static_cast<unsigned int*>(arg->p), g_stream));
	return pool_node(x, kernel_size, stride, std::move(y), std::move(arg));
}

Value conv2d_relu_maxpool2d(const Value& x, const Value& weight, const Value& bias, int stride, int padding,
                            size_t kernel_size, size_t pool_stride) {
	const ConvShape c = conv_shape(x, weight, bias, stride, padding);
	const std::vector<size_t> ys{c.N, c.Cout, c.ho, c.wo};
	Tensor y = Tensor::empty(ys);
	Tensor p = Tensor::empty(pool_shape(ys, kernel_size, pool_stride));
	const bool keep = keeps_alive(x, weight, bias, true);
	// a first layer keeps its flags as bits and the window maxima as 2-bit positions (the backward is their only
	// reader)
	const bool packed = keep && kernel_size == 2 && pool_stride == 2 && aligned16(x.data().data()) &&
	                    aligned16(y.data()) &&
	                    nnh_conv2d_packed_supported(c.N, c.Cin, c.H, c.W, c.Cout, c.kh, c.kw, stride, padding, 1);
	if (packed) {
		std::shared_ptr<Block> alive = side_buffer((y.size() + 7) / 8);
		std::shared_ptr<Block> arg = side_buffer(c.N * c.Cout * (c.ho / 2) * ((c.wo + 7) / 8));
		check(nnh_conv2d_relu_maxpool2d_forward_packed(x.data().data(), c.N, c.Cin, c.H, c.W, weight.data().data(), c.Cout,
		                                               c.kh, c.kw, bias.data().data(), stride, padding, y.data(),
		                                               static_cast<unsigned char*>(alive->p), p.data(),
		                                               static_cast<unsigned char*>(arg->p), g_stream));
		Value conv = conv_node(x, weight, bias, stride, padding, c, std::move(y), std::move(alive), true);
		return pool_node(conv, kernel_size, pool_stride, std::move(p), std::move(arg), true);
	}
	std::shared_ptr<Block> alive = keep ? side_buffer(y.size()) : nullptr;
	std::shared_ptr<Block> arg = side_buffer(p.size() * 4);
	check(nnh_conv2d_relu_maxpool2d_forward(x.data().data(), c.N, c.Cin, c.H, c.W, weight.data().data(), c.Cout, c.kh,
	                                        c.kw, bias.data().data(), stride, padding, kernel_size, pool_stride,
	                                        y.data(), alive ? static_cast<unsigned char*>(alive->p) : nullptr, p.data(),
	                                        static_cast<unsigned int*>(arg->p), g_stream));
	Value conv = conv_node(x, weight, bias, stride, padding, c, std::move(y), std::move(alive), false);
	return pool_node(conv, kernel_size, pool_stride, std::move(p), std::move(arg));
}

Value batchnorm(const Value& x, const Value& weight, const Value& bias, float eps, Tensor* mean_out, Tensor* var_out,
                bool fuse_relu) {
	const auto& xs = x.data().shape();
	// ops.cpp:901-907
	if (xs.size() < 2) throw TensorShapeError("nn::hip: batchnorm needs a channel axis");
	const size_t N = xs[0], C = xs[1];
	size_t S = 1;
	for (size_t i = 2; i < xs.size(); ++i) S *= xs[i];
	if (weight.data().size() != C || bias.data().size() != C) throw TensorShapeError("nn::hip: batchnorm parameters");
	Tensor y = Tensor::empty(xs);
	Tensor mean = Tensor::empty({C}), var = Tensor::empty({C}), inv = Tensor::empty({C});
	const bool keep = fuse_relu && NoGradGuard::grad_enabled() &&
	                  (x.requires_grad() || weight.requires_grad() || bias.requires_grad());
	std::shared_ptr<Block> alive = keep ? side_buffer(y.size()) : nullptr;
	check(nnh_batchnorm_forward(x.data().data(), N, C, S, weight.data().data(), bias.data().data(), eps,
	                            fuse_relu ? 1 : 0, y.data(), alive ? static_cast<unsigned char*>(alive->p) : nullptr,
	                            mean.data(), var.data(), inv.data(), g_stream));
	if (mean_out) *mean_out = mean;
	if (var_out) *var_out = var;
	return Value::node(std::move(y), {x, weight, bias}, [x, weight, bias, mean, inv, alive, N, C, S](const Tensor& g) {
		// ops.cpp:960-1000: dx by grad_accum, then weight and bias (grad() +=, a fresh one zeroed first)
		bool fx = false, fw = false, fb = false;
		float* dx = grad_if(x, fx);
		float* dw = grad_if(weight, fw);
		float* db = grad_if(bias, fb);
		if (!dx && !dw && !db) return;
		check(nnh_batchnorm_backward(g.data(), x.data().data(),
		                             alive ? static_cast<const unsigned char*>(alive->p) : nullptr,
		                             weight.data().data(), mean.data(), inv.data(), N, C, S, dx, fx, dw, fw, db, fb,
		                             g_stream));
	});
}

Value layernorm(const Value& x, const Value& gamma, const Value& beta, float eps) {
	const auto& xs = x.data().shape();
	// ops.cpp:1004-1006
	if (xs.empty() || gamma.data().size() != xs.back() || beta.data().size() != xs.back())
		throw TensorShapeError("nn::hip: layernorm shapes");
	const size_t D = xs.back();
	if (D == 0) throw std::invalid_argument("nn::hip: layernorm over an empty axis");
	const size_t R = x.data().size() / D;
	Tensor y = Tensor::empty(xs);
	Tensor mean = Tensor::empty({R}), inv = Tensor::empty({R});
	check(nnh_layernorm_forward(x.data().data(), R, D, gamma.data().data(), beta.data().data(), eps, y.data(),
	                            mean.data(), inv.data(), g_stream));
	return Value::node(std::move(y), {x, gamma, beta}, [x, gamma, beta, mean, inv, R, D](const Tensor& g) {
		// ops.cpp:1035-1077: dx by grad_accum, then gamma and beta (grad() +=)
		bool fx = false, fg = false, fb = false;
		float* dx = grad_if(x, fx);
		float* dg = grad_if(gamma, fg);
		float* db = grad_if(beta, fb);
		if (!dx && !dg && !db) return;
		check(nnh_layernorm_backward(g.data(), x.data().data(), gamma.data().data(), mean.data(), inv.data(), R, D, dx,
		                             fx, dg, fg, db, fb, g_stream));
	});
}

Value attention(const Value& q, const Value& k, const Value& v, size_t heads, const Tensor& key_padding_mask,
                bool causal) {
	const auto& qs = q.data().shape();
	const auto& ks = k.data().shape();
	// ops.cpp:1228-1236
	if (qs.size() != 3 || ks.size() != 3 || v.data().shape() != ks || qs[0] != ks[0] || qs[2] != ks[2])
		throw TensorShapeError("nn::hip: attention shapes");
	const size_t N = qs[0], Tq = qs[1], D = qs[2], Tk = ks[1];
	const bool mask = key_padding_mask.size() != 0;
	if (mask && key_padding_mask.shape() != std::vector<size_t>{N, Tk})
		throw TensorShapeError("nn::hip: attention key padding mask shape");
	Tensor out = Tensor::empty({N, Tq, D});
	Tensor probs = Tensor::empty({N, heads ? heads : 1, Tq, Tk});
	const float* pm = mask ? key_padding_mask.data() : nullptr;
	check(nnh_attention_forward(q.data().data(), k.data().data(), v.data().data(), N, Tq, Tk, D, heads, pm, causal,
	                            out.data(), probs.data(), g_stream));
	const Tensor keep_mask = key_padding_mask;
	return Value::node(std::move(out), {q, k, v}, [=](const Tensor& g) {
		// ops.cpp:1274-1278: the gradients in the order they are written, v, q, k
		bool fv = false, fq = false, fk = false;
		float* dv = grad_if(v, fv);
		float* dq = grad_if(q, fq);
		float* dk = grad_if(k, fk);
		if (!dq && !dk && !dv) return;
		check(nnh_attention_backward(g.data(), q.data().data(), k.data().data(), v.data().data(), probs.data(), N, Tq,
		                             Tk, D, heads, mask ? keep_mask.data() : nullptr, causal, dq, fq, dk, fk, dv, fv,
		                             g_stream));
	});
}

Value scaled_masked_softmax(const Value& x, float scale_by, const Tensor& key_padding_mask, bool causal) {
	const auto& xs = x.data().shape();
	if (xs.size() != 4) throw TensorShapeError("nn::hip: scaled_masked_softmax needs {N, H, Tq, Tk}");
	const size_t N = xs[0], H = xs[1], Tq = xs[2], Tk = xs[3];
	const bool mask = key_padding_mask.size() != 0;
	if (mask && key_padding_mask.shape() != std::vector<size_t>{N, Tk})
		throw TensorShapeError("nn::hip: scaled_masked_softmax key padding mask shape");
	Tensor y = Tensor::empty(xs);
	check(nnh_scaled_masked_softmax_forward(x.data().data(), N, H, Tq, Tk, scale_by,
	                                        mask ? key_padding_mask.data() : nullptr, causal, y.data(), g_stream));
	const Tensor keep_mask = key_padding_mask;
	const Tensor yk = y;
	return Value::node(std::move(y), {x}, [=](const Tensor& g) {
		bool first = false;
		float* dx = grad_if(x, first);
		if (dx)
			check(nnh_scaled_masked_softmax_backward(yk.data(), g.data(), N, H, Tq, Tk, scale_by,
			                                         mask ? keep_mask.data() : nullptr, causal, dx, first, g_stream));
	});
}

namespace {

// The add node over its forward's output y = a + b.
Value add_node(const Value& a, const Value& b, Tensor y) {
	return Value::node(std::move(y), {a, b}, [a, b](const Tensor& g) {
		// ops.cpp:333-336 then accumulate_grad (ops.cpp:110-117): a, then b, each stored fresh or added to
		const auto& gs = g.shape();
		const size_t lead = gs.size() - b.data().ndim();
		bool first = false, first_b = false;
		// an operand used only here takes g's storage (a.impl() == b.impl() counts two uses)
		const bool took_a = take_grad(a, g);
		const bool took_b = lead == 0 && take_grad(b, g);
		if (took_a || took_b) {
			if (!took_a) {
				if (float* da = grad_if(a, first)) check(nnh_add_to_grad(da, g.data(), g.size(), first, g_stream));
			}
			if (took_b) return;
		}
		float* da = took_a ? nullptr : grad_if(a, first);
		if (lead == 0 && da && a.impl() != b.impl()) {
			// both operands of the output's shape: both gradients in one launch
			if (float* db = grad_if(b, first_b)) {
				check(nnh_add_to_grad2(da, first, db, first_b, g.data(), g.size(), g_stream));
				return;
			}
		}
		if (da) check(nnh_add_to_grad(da, g.data(), g.size(), first, g_stream));
		float* db = grad_if(b, first);
		if (!db) return;
		if (lead == 0) {
			check(nnh_add_to_grad(db, g.data(), g.size(), first, g_stream));
			return;
		}
		// sum_to_shape: Tensor::sum(0) once per leading axis, the last one straight into the gradient
		Tensor cur = g;
		for (size_t i = 0; i < lead; ++i) {
			const std::vector<size_t> rest(cur.shape().begin() + 1, cur.shape().end());
			if (i + 1 == lead) {
				check(nnh_tensor_sum0(cur.data(), cur.shape()[0], numel(rest), db, first ? 1 : 2, g_stream));
			} else {
				Tensor next = Tensor::empty(rest);
				check(nnh_tensor_sum0(cur.data(), cur.shape()[0], numel(rest), next.data(), 0, g_stream));
				cur = next;
			}
		}
	});
}

}  // namespace

Value add(const Value& a, const Value& b) {
	const auto& as = a.data().shape();
	const auto& bs = b.data().shape();
	if (bs.size() > as.size() || !std::equal(bs.begin(), bs.end(), as.end() - bs.size()))
		throw std::invalid_argument("nn::hip: add takes b of a's shape or of a's trailing axes");
	const size_t inner = b.data().size(), total = a.data().size();
	const size_t outer = inner ? total / inner : 0;
	Tensor y = Tensor::empty(as);
	check(nnh_add_forward(a.data().data(), b.data().data(), outer, inner, y.data(), g_stream));
	return add_node(a, b, std::move(y));
}

std::vector<Value> linear_many(const Value& x, const std::vector<std::pair<Value, Value>>& layers) {
	const auto& xs = x.data().shape();
	const size_t count = layers.size();
	if (count == 0) return {};
	if (count > 8) {
		std::vector<Value> out;
		for (const auto& l : layers) out.push_back(linear(x, l.first, l.second));
		return out;
	}
	std::vector<Tensor> ys;
	std::vector<const float*> w(count), b(count);
	std::vector<float*> y(count);
	std::vector<size_t> n(count);
	const size_t K = xs.empty() ? 0 : xs.back();
	for (size_t i = 0; i < count; ++i) {
		const auto& ws = layers[i].first.data().shape();
		// ops.cpp:717-719
		if (xs.size() < 2 || ws.size() != 2 || xs.back() != ws[1] ||
		    layers[i].second.data().shape() != std::vector<size_t>{ws[0]})
			throw TensorShapeError("nn::hip: linear shapes");
		std::vector<size_t> out(xs.begin(), xs.end() - 1);
		out.push_back(ws[0]);
		ys.push_back(Tensor::empty(out));
		w[i] = layers[i].first.data().data();
		b[i] = layers[i].second.data().data();
		y[i] = ys.back().data();
		n[i] = ws[0];
	}
	const size_t M = K ? x.data().size() / K : numel(std::vector<size_t>(xs.begin(), xs.end() - 1));
	check(nnh_linear_forward_multi(x.data().data(), M, K, (int)count, w.data(), n.data(), b.data(), y.data(), g_stream));
	std::vector<Value> out;
	for (size_t i = 0; i < count; ++i) out.push_back(linear_node(x, layers[i].first, layers[i].second, ys[i]));
	return out;
}

Value linear_add(const Value& x, const Value& weight, const Value& bias, const Value& residual) {
	const auto& xs = x.data().shape();
	const auto& ws = weight.data().shape();
	// ops.cpp:717-719
	if (xs.size() < 2 || ws.size() != 2 || xs.back() != ws[1] || bias.data().shape() != std::vector<size_t>{ws[0]})
		throw TensorShapeError("nn::hip: linear shapes");
	std::vector<size_t> out(xs.begin(), xs.end() - 1);
	out.push_back(ws[0]);
	if (residual.data().shape() != out) return add(residual, linear(x, weight, bias));
	const size_t n = ws[0], K = ws[1], M = numel(out) / std::max<size_t>(n, 1);
	Tensor y = Tensor::empty(out);
	check(nnh_linear_forward_add(x.data().data(), M, K, weight.data().data(), n, bias.data().data(),
	                             residual.data().data(), y.data(), g_stream));
	// the linear node (whose backward does not read its data) and the add node over it, as add(residual, linear(..))
	return add_node(residual, linear_node(x, weight, bias, y), y);
}

Value mul(const Value& a, const Value& b) {
	if (a.data().shape() != b.data().shape())
		throw std::invalid_argument("nn::hip: mul takes two tensors of one shape");
	Tensor y = Tensor::empty(a.data().shape());
	check(nnh_mul_forward(a.data().data(), b.data().data(), y.size(), y.data(), g_stream));
	return Value::node(std::move(y), {a, b}, [a, b](const Tensor& g) {
		// ops.cpp:349-356: a's term g * b, then b's term g * a, each through accumulate_grad
		bool first = false;
		if (float* da = grad_if(a, first)) check(nnh_mul_backward(g.data(), b.data().data(), g.size(), da, first, g_stream));
		if (float* db = grad_if(b, first)) check(nnh_mul_backward(g.data(), a.data().data(), g.size(), db, first, g_stream));
	});
}

Value slice(const Value& x, int axis, size_t start, size_t end) {
	const auto& xs = x.data().shape();
	if (axis != 0) throw std::invalid_argument("nn::hip: slice takes axis 0");
	if (xs.empty() || start >= end || end > xs[0]) throw TensorShapeError("nn::hip: slice out of range");
	const size_t inner = x.data().size() / xs[0];
	std::vector<size_t> ys = xs;
	ys[0] = end - start;
	Tensor y = Tensor::empty(ys);
	if (y.size())
		check_hip(hipMemcpyAsync(y.data(), x.data().data() + start * inner, y.size() * 4, hipMemcpyDeviceToDevice,
		                         g_stream),
		          "slice");
	return Value::node(std::move(y), {x}, [x, start, inner](const Tensor& g) {
		// ops.cpp:603-607: x.grad() (zeroed when fresh), then the band adds g
		if (!x.requires_grad()) return;
		float* dx = x.grad().data() + start * inner;
		check(nnh_add_to_grad(dx, g.data(), g.size(), 0, g_stream));
	});
}

namespace {

// The GELU node over its forward's output y and the tanh it keeps for the backward rule.
Value gelu_node(const Value& x, Tensor y, Tensor th) {
	return Value::node(std::move(y), {x}, [x, th](const Tensor& g) {
		bool first = false;
		float* dx = grad_if(x, first);
		if (dx) check(nnh_gelu_backward(x.data().data(), th.data(), g.data(), g.size(), dx, first, g_stream));
	});
}

}  // namespace

Value gelu(const Value& x) {
	Tensor y = Tensor::empty(x.data().shape());
	Tensor th = Tensor::empty(x.data().shape());  // tanh(k (x + c x^3)), kept for the backward rule
	check(nnh_gelu_forward(x.data().data(), y.size(), y.data(), th.data(), g_stream));
	return gelu_node(x, std::move(y), std::move(th));
}

Value linear_gelu(const Value& x, const Value& weight, const Value& bias) {
	const auto& xs = x.data().shape();
	const auto& ws = weight.data().shape();
	// ops.cpp:717-719
	if (xs.size() < 2 || ws.size() != 2 || xs.back() != ws[1] || bias.data().shape() != std::vector<size_t>{ws[0]})
		throw TensorShapeError("nn::hip: linear shapes");
	std::vector<size_t> out(xs.begin(), xs.end() - 1);
	out.push_back(ws[0]);
	const size_t n = ws[0], K = ws[1], M = numel(out) / std::max<size_t>(n, 1);
	Tensor h = Tensor::empty(out), y = Tensor::empty(out), th = Tensor::empty(out);
	check(nnh_linear_gelu_forward(x.data().data(), M, K, weight.data().data(), n, bias.data().data(), h.data(), y.data(),
	                              th.data(), g_stream));
	return gelu_node(linear_node(x, weight, bias, h), std::move(y), std::move(th));
}

namespace {

// embedding, or embedding_add with addend (its rows broadcast over the ids), as the nodes of the separate ops
Value embedding_op(const Value& weight, const std::vector<float>& ids, const std::vector<size_t>& ids_shape,
                   const Value* addend) {
	const auto& ws = weight.data().shape();
	// ops.cpp:1992-2001
	if (ws.size() != 2) throw TensorShapeError("nn::hip: embedding weight must be {V, D}");
	if (numel(ids_shape) != ids.size()) throw std::invalid_argument("nn::hip: embedding ids and their shape differ");
	const size_t V = ws[0], D = ws[1];
	if (ids.size() > (size_t)INT32_MAX || V > (size_t)INT32_MAX)
		throw std::invalid_argument("nn::hip: embedding takes at most 2^31 - 1 ids and table rows");
	std::vector<int> rows(ids.size());
	for (size_t i = 0; i < ids.size(); ++i) {
		const float f = ids[i];
		if (!(f >= 0.0f) || f != std::floor(f) || f >= static_cast<float>(V))
			throw TensorShapeError("nn::hip: embedding id out of range or not a whole number");
		rows[i] = static_cast<int>(f);
	}
	std::vector<size_t> out = ids_shape;
	out.push_back(D);
	Tensor y = Tensor::empty(out);
	std::shared_ptr<Block> rb = side_buffer(rows.size() * sizeof(int));
	if (!rows.empty()) {
		check_hip(hipMemcpyAsync(rb->p, rows.data(), rows.size() * sizeof(int), hipMemcpyHostToDevice, g_stream),
		          "copy in");
		synchronize();  // rows is released on return
	}
	const size_t count = rows.size();
	// the addend's shape must be trailing axes of the output's (add's rule), its rows dividing the ids' count
	const bool fuse = addend && addend->data().ndim() >= 1 && addend->data().ndim() <= out.size() &&
	                  std::equal(addend->data().shape().begin(), addend->data().shape().end(),
	                             out.end() - addend->data().ndim()) &&
	                  addend->data().size() > 0;
	if (fuse)
		check(nnh_embedding_add_forward(weight.data().data(), V, D, static_cast<const int*>(rb->p), count,
		                                addend->data().data(), addend->data().size() / std::max<size_t>(D, 1), y.data(),
		                                g_stream));
	else
		check(nnh_embedding_forward(weight.data().data(), V, D, static_cast<const int*>(rb->p), count, y.data(),
		                            g_stream));
	Value e = Value::node(y, {weight}, [weight, rb, count, V, D](const Tensor& g) {
		// ops.cpp:2008-2014: weight.grad() (zeroed when fresh) gets the rows added in token order
		bool first = false;
		float* dw = grad_if(weight, first);
		if (dw) check(nnh_embedding_backward(g.data(), static_cast<const int*>(rb->p), count, V, D, dw, first, g_stream));
	});
	if (!addend) return e;
	// the embedding node (whose backward does not read its data) and the add node over it
	return fuse ? add_node(e, *addend, y) : add(e, *addend);
}

}  // namespace

Value embedding(const Value& weight, const std::vector<float>& ids, const std::vector<size_t>& ids_shape) {
	return embedding_op(weight, ids, ids_shape, nullptr);
}

Value embedding_add(const Value& weight, const std::vector<float>& ids, const std::vector<size_t>& ids_shape,
                    const Value& addend) {
	return embedding_op(weight, ids, ids_shape, &addend);
}

Value embedding_add(const Value& weight, const Tensor& ids, const Value& addend) {
	return embedding_add(weight, ids.to_host(), ids.shape(), addend);
}

Value embedding(const Value& weight, const Tensor& ids) {
	return embedding(weight, ids.to_host(), ids.shape());
}

Tensor sinusoidal_table(size_t max_len, size_t dim) {
	// positional.cpp:15-25: angle = pos / 10000^((c - c % 2) / dim) in double; sin on even columns, cos on odd
	std::vector<float> t(max_len * dim);
	for (size_t pos = 0; pos < max_len; ++pos)
		for (size_t c = 0; c < dim; ++c) {
			const double angle = static_cast<double>(pos) /
			                     std::pow(10000.0, static_cast<double>(c - c % 2) / static_cast<double>(dim));
			t[pos * dim + c] = static_cast<float>(c % 2 == 0 ? std::sin(angle) : std::cos(angle));
		}
	Tensor out = Tensor::from_host({max_len, dim}, t.data());
	synchronize();  // t is released on return
	return out;
}

}  // namespace hip
}  // namespace nn
