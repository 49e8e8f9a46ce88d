// gemm.hip - instantiations, depth-cut reduction and launch logic of the fp32 MFMA GEMM.
#include "gemm.hpp"
#include "gemm_valu.hpp"

#include <optional>

#include "workspace.hpp"
#include "gemm_config.hpp"

#include <algorithm>
#include <atomic>
#include <mutex>

namespace nnh {

namespace {

__device__ __forceinline__ float finish(float v, int64_t row, int64_t col, int64_t off, const Epilogue& ep,
                                        unsigned char* alive, const float* res) {
	if (ep.bias_mode == kBiasCol) v = v + ep.bias[col];
	else if (ep.bias_mode == kBiasRow) v = v + ep.bias[row];
	if (res) v = res[off] + v;
	if (ep.relu) {
		const bool on = v > 0.0f;
		if (alive) alive[off] = on ? 1 : 0;
		v = on ? v : 0.0f;
	}
	return v;
}

// Depth-cut second pass (gemm.cpp:475-484): acc = piece 0, then += each later piece in order;
// C = acc, or C = C + acc when accumulating. One thread per element, no atomics.
__global__ void __launch_bounds__(256) reduce_pieces_kernel(const float* __restrict__ part, int pieces, int m, int n,
                                                            float* c, int64_t ldc, int accumulate, BatchDesc batch,
                                                            int64_t batch_count, Epilogue ep) {
	const int64_t mn = (int64_t)m * n;
	const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
	if (idx >= mn * batch_count) return;
	const int64_t bi = idx / mn, e = idx % mn;
	const int64_t row = e / n, col = e % n;
	const float* pp = part + bi * pieces * mn + e;
	float acc = pp[0];
	for (int q = 1; q < pieces; ++q) acc = acc + pp[q * mn];
	int64_t oa, ob, oc = 0;
	if (batch.ndim > 0) batch_offsets(batch, bi, oa, ob, oc);
	const int64_t off = row * ldc + col;
	float* cp = c + oc;
	float v = accumulate ? cp[off] + acc : acc;
	cp[off] = finish(v, row, col, off, ep, ep.alive ? ep.alive + oc : nullptr, ep.res ? ep.res + oc : nullptr);
}

const Config* configs() {
	static const Config table[] = {
		config_64x128x32(), config_128x128x32(), config_64x256x32(), config_128x64x32(),
		config_128x256x16(), config_256x128x16(), config_64x128x64(), config_128x128x16(),
		config_32x32x32_mf4(), config_64x64x32_mf4(), config_64x64x32_mf16(), config_128x64x32_mf16(),
		config_32x32x32_mfk4(), config_64x64x32_mfk4(), config_128x64x32_mfk4(), config_128x128x32_mfk4(),
		config_32x32x64_mfk4(), config_32x32x128_mfk4(),
	};
	return table;
}
constexpr int kNumConfigs = 18;

// Raises each kernel's dynamic LDS limit once per device (gfx950 has 160 KiB per CU).
hipError_t prepare_device() {
	static std::mutex mu;
	static bool done[64] = {};
	int dev = 0;
	hipError_t e = hipGetDevice(&dev);
	if (e != hipSuccess) return e;
	if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
	std::lock_guard<std::mutex> lock(mu);
	if (done[dev]) return hipSuccess;
	const Config* cfg = configs();
	for (int i = 0; i < kNumConfigs; ++i) {
		for (int f = 0; f < 4; ++f)
			for (int edge = 0; edge < 5; ++edge) {
				if (edge == 2 && f >= 2) continue;  // gather kernels: A not transposed
				if (edge >= 3 && f != 2) continue;  // row-sum kernels: transposed A, plain B
				const KernelFn fn = edge < 2 ? cfg[i].fn[f][edge] : edge == 2 ? cfg[i].gather_fn[f] : cfg[i].rowsum_fn[edge - 3];
				e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
				                        cfg[i].lds_bytes[f]);
				if (e != hipSuccess) return e;
			}
		for (int p = 0; p < 8; ++p) {
			const PairFn fn = cfg[i].pair_fn[p >> 2][(p >> 1) & 1][p & 1];
			if (!fn) continue;
			e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
			                        std::max(cfg[i].lds_bytes[0], cfg[i].lds_bytes[2]));
			if (e != hipSuccess) return e;
		}
	}
	done[dev] = true;
	return hipSuccess;
}

// Choice by measured device time on MI355X (every configuration on every BASELINE shape, and the MLP's). Each
// output element is a K-long chain of dependent MFMAs: a dependent step costs about 64 cycles with 32x32x1 and 44
// with 16x16x1 or 4x4x1, for one depth index, and 44 with 16x16x4 for four. Large products fill the GPU with
// 128 x 128 or 128 x 64 tiles of 32x32x1 units (16-deep stages for A B, 32-deep when an operand is transposed);
// from about 4 million outputs down to 2^20, 128 x 128 and then 64 x 64 workgroups of 16x16x4 units; smaller
// products use 32 x 32 workgroups of 16x16x4 units (one wave per 16 x 16 block, as many chains as possible), with
// 64-deep stages (128-deep with op(A) transposed and 512 or more deep, 32-deep up to 32). Measured (us, exact
// mode): 512^3 NN 9.9 -> 7.1, TN 9.8 -> 6.7, NT 8.4 -> 7.0; 64 x 4096 x 4096 59.6 -> 35.7; 2048^3 168 -> 158.
// Results never depend on the choice.
enum {
	kCfg128x128x32 = 1,
	kCfg128x64x32 = 3,
	kCfg128x128x16 = 7,
	kCfg64x64x32Mfk4 = 13,
	kCfg128x128x32Mfk4 = 15,
	kCfg32x32x64Mfk4 = 16,
	kCfg32x32x128Mfk4 = 17,
	kCfg32x32x32Mfk4 = 12,
};

int pick_config(const GemmCall& g) {
	const double outputs = (double)g.m * (double)g.n * (double)g.batch_count;
	// short depth (one or two 32-deep tiles): 128 x 64 tiles measured faster than 128 x 128 (4096 x 4096 x 64:
	// 28.2 against 30.0 us), while 16-deep products keep the 16-deep tiles their depth divides
	if (outputs >= 512.0 * 128 * 128 && !g.ta && !g.tb && g.k >= 32 && g.k <= 64 && g.k % 32 == 0) return kCfg128x64x32;
	if (outputs >= 512.0 * 128 * 128) return (!g.ta && !g.tb) ? kCfg128x128x16 : kCfg128x128x32;
	if (g.m >= 128 && g.n >= 128 && outputs >= 256.0 * 128 * 128) return kCfg128x128x32Mfk4;
	// narrower products of that size (attention's batched 256 x 64 per head) keep 128 x 64 tiles
	if (g.m >= 128 && outputs >= 512.0 * 128 * 64) return kCfg128x64x32;
	if (outputs >= 1024.0 * 1024) return kCfg64x64x32Mfk4;
	if (g.k <= 32) return kCfg32x32x32Mfk4;
	return (g.ta && g.k >= 512) ? kCfg32x32x128Mfk4 : kCfg32x32x64Mfk4;
}

// The kernel arguments of one product on configuration cf; cut: the product takes nn-cpp's depth cut (the
// caller supplies p.partial); interior: every tile is whole and 16-byte aligned (the kernels without bounds checks).
GemmArgs make_args(const GemmCall& g, const Config& cf, bool& cut, bool& interior) {
	GemmArgs p{};
	p.a = g.a;
	p.b = g.b;
	p.c = g.c;
	p.lda = g.lda;
	p.ldb = g.ldb;
	p.ldc = g.ldc;
	p.m = (int)g.m;
	p.n = (int)g.n;
	p.k = (int)g.k;
	p.accumulate = g.accumulate;
	p.tiles_m = (int)((g.m + cf.bm - 1) / cf.bm);
	p.tiles_n = (int)((g.n + cf.bn - 1) / cf.bn);
	p.batch_count = (int)g.batch_count;
	p.batch = g.batch;
	p.ep = g.ep;
	p.col = g.col;
	const CutPlan plan = cut_plan(g.m, g.n, g.k);
	cut = plan.pieces > 1;
	p.rowsum = g.rowsum;
	p.rowsum_combine = g.rowsum_combine;
	p.pieces = cut ? (int)plan.pieces : 1;
	p.piece_k = cut ? (int)plan.piece_k : (int)std::max<int64_t>(g.k, 1);
	// 16-byte operand loads need 16-byte rows and strides (a gathered B is read element by element)
	bool vec_ok = (g.lda % 4 == 0) && (reinterpret_cast<uintptr_t>(g.a) % 16 == 0) &&
	              (g.gather || ((g.ldb % 4 == 0) && (reinterpret_cast<uintptr_t>(g.b) % 16 == 0)));
	for (int d = 0; d < g.batch.ndim; ++d)
		vec_ok = vec_ok && g.batch.sa[d] % 4 == 0 && (g.gather || g.batch.sb[d] % 4 == 0);
	p.vec_ok = vec_ok ? 1 : 0;
	// interior kernels also write C with 16-byte stores
	bool c_vec = (g.ldc % 4 == 0) && (reinterpret_cast<uintptr_t>(g.c) % 16 == 0);
	for (int d = 0; d < g.batch.ndim; ++d) c_vec = c_vec && g.batch.sc[d] % 4 == 0;
	interior = vec_ok && c_vec && g.m % cf.bm == 0 && g.n % cf.bn == 0 && g.k % cf.bk == 0 && g.k > 0 &&
	           p.piece_k % cf.bk == 0;
	return p;
}

}  // namespace

namespace {
std::atomic<int> g_numerics{kNumericsNnCpp};  // the process default
std::mutex g_stream_modes_mu;
std::vector<std::pair<void*, int>> g_stream_modes;  // per-stream overrides (few streams: a short list)
thread_local int t_call_numerics = -1;              // the mode of the call being issued on this thread, or -1
}  // namespace

int set_numerics(int mode) { return g_numerics.exchange(mode); }
int default_numerics() { return g_numerics.load(std::memory_order_relaxed); }

int set_stream_numerics(void* stream, int mode) {
	std::lock_guard<std::mutex> lk(g_stream_modes_mu);
	int prev = -1;
	for (size_t i = 0; i < g_stream_modes.size(); ++i) {
		if (g_stream_modes[i].first != stream) continue;
		prev = g_stream_modes[i].second;
		if (mode < 0) g_stream_modes.erase(g_stream_modes.begin() + (ptrdiff_t)i);
		else g_stream_modes[i].second = mode;
		return prev;
	}
	if (mode >= 0) g_stream_modes.emplace_back(stream, mode);
	return prev;
}

int stream_numerics(void* stream) {
	{
		std::lock_guard<std::mutex> lk(g_stream_modes_mu);
		for (const auto& e : g_stream_modes)
			if (e.first == stream) return e.second;
	}
	return default_numerics();
}

int numerics() { return t_call_numerics >= 0 ? t_call_numerics : default_numerics(); }

NumericsScope::NumericsScope(void* stream) : prev_(t_call_numerics) {
	if (prev_ < 0) t_call_numerics = stream_numerics(stream);
}
NumericsScope::NumericsScope(int mode, bool) : prev_(t_call_numerics) { t_call_numerics = mode; }
NumericsScope::~NumericsScope() { t_call_numerics = prev_; }

CutPlan cut_plan(int64_t m, int64_t n, int64_t k) {
	CutPlan c;
	if (m <= 0 || n <= 0 || k <= 0) return c;
	if (numerics() == kNumericsSplitDepth) {
		if (m * n > (int64_t(1) << 18) || k < 256) return c;
		const int64_t tiles = ((m + 63) / 64) * ((n + 15) / 16);
		const int64_t s = std::min<int64_t>(16, std::max<int64_t>(2, 4096 / tiles));
		c.piece_k = ((k + s - 1) / s + 31) / 32 * 32;
	} else {
		if (m * n > (int64_t(1) << 16) || k < 4 * 128 || m * n * k < (int64_t(1) << 20)) return c;
		c.piece_k = 128;
	}
	c.pieces = (k + c.piece_k - 1) / c.piece_k;
	return c;
}

bool depth_cut(int64_t m, int64_t n, int64_t k) { return cut_plan(m, n, k).pieces > 1; }

int64_t gemm_workspace_floats(int64_t m, int64_t n, int64_t k, int64_t batch_count, bool gather) {
	if (!depth_cut(m, n, k) || pieces_kernel_takes(m, n, k, batch_count, gather)) return 0;
	return cut_plan(m, n, k).pieces * m * n * batch_count;
}

int64_t gemm_workspace_floats(const GemmCall& g) {
	if (!depth_cut(g.m, g.n, g.k) || pieces_kernel_takes(g) || pieces4_takes(g)) return 0;
	return cut_plan(g.m, g.n, g.k).pieces * g.m * g.n * g.batch_count;
}

// Configurations kNumConfigs .. kNumConfigs + kValuShapes - 1 are the VALU kernel's lane blocks (gemm_valu.hip).
// Configuration kNumConfigs + kValuShapes forces the VALU pieces kernel on a cut product it can take,
// kNumConfigs + kValuShapes + 1 the 16x16x4 MFMA pieces kernel, and kNumConfigs + kValuShapes + 2 the whole-depth
// 16x16x4 chain kernel on a product that is not cut.
int gemm_config_count() { return kNumConfigs + kValuShapes + 3; }
const char* gemm_config_name(int config) {
	if (config == kNumConfigs + kValu2x2) return "valu 32x32 (2x2 chains per lane)";
	if (config == kNumConfigs + kValu1x2) return "valu 16x32 (1x2 chains per lane)";
	if (config == kNumConfigs + kValu2x4) return "valu 32x64 (2x4 chains per lane)";
	if (config == kNumConfigs + kValu1x4) return "valu 16x64 (1x4 chains per lane)";
	if (config == kNumConfigs + kValuBc1) return "valu bcast 16x16 (1 chain per lane, A by DPP)";
	if (config == kNumConfigs + kValuBc2) return "valu bcast 32x16 (2 chains per lane, A by DPP)";
	if (config == kNumConfigs + kValuShapes) return "valu pieces 16x16 (every piece of a cut output in one lane)";
	if (config == kNumConfigs + kValuShapes + 1) return "mfma pieces 16x16x4 (a wave per piece, 16x16 tiles)";
	if (config == kNumConfigs + kValuShapes + 2) return "mfma chain 16x16x4 (32x32 tiles, no LDS)";

	return (config >= 0 && config < kNumConfigs) ? configs()[config].name : "";
}

hipError_t gemm_launch(const GemmCall& g, hipStream_t s, int config, float* workspace) {
	if (g.m == 0 || g.n == 0 || g.batch_count == 0) return hipSuccess;
	hipError_t e = prepare_device();
	if (e != hipSuccess) return e;
	const bool force_pieces = config == kNumConfigs + kValuShapes;
	const bool force_pieces4 = config == kNumConfigs + kValuShapes + 1;
	// the VALU kernel: forced, or chosen by shape, for a product it can take
	const bool valu_ok = !g.gather && !g.rowsum && g.k > 0 && !depth_cut(g.m, g.n, g.k) && g.m < (1 << 30) &&
	                     g.n < (1 << 30) && g.k < (1 << 30);
	if (valu_ok && config >= kNumConfigs && config < kNumConfigs + kValuShapes)
		return gemm_valu_launch(g, config - kNumConfigs, s);
	if (config == kNumConfigs + kValuShapes + 2 && chain4_ok(g)) return gemm_chain4_launch(g, s);
	if (config < 0 && chain4_takes(g)) return gemm_chain4_launch(g, s);
	if ((config < 0 || config >= kNumConfigs) && valu_ok && valu_takes(g)) return gemm_valu_launch(g, valu_shape(g), s);
	if (config < 0 || config >= kNumConfigs) config = pick_config(g);
	const Config& cf = configs()[config];

	if (g.gather && g.ta) return hipErrorInvalidValue;
	// the 16x16x4 pieces kernel: its own route, forced, or the only one for two-stage row sums (a forced VALU pieces
	// configuration keeps the VALU kernel where that can take the product)
	const bool p4 = g.rowsum ? pieces4_takes(g)
	                         : force_pieces4 ? pieces_kernel_takes(g) : !force_pieces && pieces4_takes(g);
	if (p4) return gemm_pieces4_launch(g, s);
	if (g.rowsum && (g.rowsum_outer > 0 || depth_cut(g.m, g.n, g.k) || g.batch_count != 1 || g.gather || !g.ta || g.tb))
		return hipErrorInvalidValue;
	if (force_pieces ? valu_pieces_ok(g) : valu_pieces_takes(g))
		return gemm_valu_pieces_launch(g, s);
	if (pieces_kernel_takes(g)) return gemm_pieces_launch(g, s);
	bool cut = false, interior = false;
	GemmArgs p = make_args(g, cf, cut, interior);

	float* part = nullptr;
	std::optional<StreamWorkspace> ws;
	if (cut) {
		if (workspace) {
			part = workspace;
		} else {
			ws.emplace(s, (size_t)gemm_workspace_floats(g) * sizeof(float));
			if (ws->error() != hipSuccess) return ws->error();
			part = ws->at<float>(0);
		}
		p.partial = part;
	}
	const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n * p.pieces * p.batch_count;
	if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
	const int f = (g.ta ? 2 : 0) + (g.tb ? 1 : 0);
	const KernelFn fn = g.gather ? cf.gather_fn[g.tb ? 1 : 0] : g.rowsum ? cf.rowsum_fn[interior ? 0 : 1] : cf.fn[f][interior ? 0 : 1];
	hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(256), cf.lds_bytes[f], s, p);
	e = hipGetLastError();
	if (e == hipSuccess && cut) {
		const int64_t total = g.m * g.n * g.batch_count;
		hipLaunchKernelGGL(reduce_pieces_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, part,
		                   p.pieces, p.m, p.n, g.c, g.ldc, g.accumulate, g.batch, g.batch_count, g.ep);
		e = hipGetLastError();
	}
	return e;
}

hipError_t gemm_launch_pair(const GemmCall& g0, const GemmCall& g1, hipStream_t s, bool& launched) {
	launched = false;
	// a whole-depth A B on the chain kernel beside a cut A^T B (with or without two-stage row sums) on the pieces
	// kernel: the kernels their own launches take, in one grid
	if (chain_pieces_pair_takes(g0, g1)) {
		hipError_t e = prepare_device();
		if (e != hipSuccess) return e;
		e = gemm_chain_pieces_pair_launch(g0, g1, s);
		launched = e == hipSuccess;
		return e;
	}
	// two products that each run on the chain kernel (a matmul's dA = G B or G B^T and dB = A^T G or G^T A)
	if (chain4_pair_takes(g0, g1)) {
		hipError_t e = prepare_device();
		if (e != hipSuccess) return e;
		e = gemm_chain4_pair_launch(g0, g1, s);
		launched = e == hipSuccess;
		return e;
	}
	// g0 = A B and g1 = A^T B (row sums allowed), single matrices, no depth cut, both on one configuration that
	// has the pair kernels
	if (g0.ta || g0.tb || g0.gather || g0.rowsum || !g1.ta || g1.tb || g1.gather || g1.rowsum_outer > 0) return hipSuccess;
	if (g0.batch_count != 1 || g1.batch_count != 1 || g0.batch.ndim != 0 || g1.batch.ndim != 0) return hipSuccess;
	if (g0.m == 0 || g0.n == 0 || g1.m == 0 || g1.n == 0) return hipSuccess;
	if (depth_cut(g0.m, g0.n, g0.k) || depth_cut(g1.m, g1.n, g1.k)) return hipSuccess;
	const int c0 = pick_config(g0), c1 = pick_config(g1);
	if (c0 != c1) return hipSuccess;
	const Config& cf = configs()[c0];
	bool cut0 = false, cut1 = false, in0 = false, in1 = false;
	const GemmArgs p0 = make_args(g0, cf, cut0, in0), p1 = make_args(g1, cf, cut1, in1);
	const PairFn fn = cf.pair_fn[in0 ? 0 : 1][in1 ? 0 : 1][g1.rowsum ? 1 : 0];
	if (!fn) return hipSuccess;
	const int64_t b0 = (int64_t)p0.tiles_m * p0.tiles_n, b1 = (int64_t)p1.tiles_m * p1.tiles_n;
	if (b0 + b1 > 0x7fffffff) return hipSuccess;
	hipError_t e = prepare_device();
	if (e != hipSuccess) return e;
	hipLaunchKernelGGL(fn, dim3((unsigned)(b0 + b1)), dim3(256), std::max(cf.lds_bytes[0], cf.lds_bytes[2]), s, p0, p1,
	                   (int)b0);
	e = hipGetLastError();
	launched = e == hipSuccess;
	return e;
}

hipError_t gemm_launch_group(const GemmCall* g, int count, hipStream_t s, bool& launched) {
	launched = false;
	if (!chain4_group_takes(g, count)) return hipSuccess;
	hipError_t e = prepare_device();
	if (e != hipSuccess) return e;
	e = gemm_chain4_group_launch(g, count, s);
	launched = e == hipSuccess;
	return e;
}

}  // namespace nnh
