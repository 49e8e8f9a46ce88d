// gemm.hpp - host-side launch API of the fp32 MFMA GEMM (internal to libnnh; the public C ABI is
// include/nnh.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemm_tile.hpp"

namespace nnh {

// One GEMM, or a batch of GEMMs sharing m, n, k and leading dimensions, in nn::kernels::sgemm's
// terms (include/nn/kernels/gemm.hpp:36-59): C = op(A) op(B) (+ C when accumulate), then the epilogue.
struct GemmCall {
	int ta = 0, tb = 0;
	int64_t m = 0, n = 0, k = 0;
	const float* a = nullptr;
	int64_t lda = 0;
	const float* b = nullptr;
	int64_t ldb = 0;
	float* c = nullptr;
	int64_t ldc = 0;
	int accumulate = 0;
	BatchDesc batch{};        // ndim 0: a single matrix
	int64_t batch_count = 1;
	Epilogue ep{};
	bool gather = false;      // B is each sample's im2col columns, read from the convolution input b (ColGather)
	ColGather col{};
	float* rowsum = nullptr;  // optional row sums of op(A) (GemmArgs::rowsum); A transposed, B not, one matrix, no depth cut
	int rowsum_combine = 0;
	// > 0: the row sums are two ordered sums instead (GemmArgs::rowsum_outer), on a cut product the 16x16x4 pieces
	// kernel takes (pieces4_takes)
	int64_t rowsum_outer = 0;
};

// Numerics modes (nnh_set_numerics). kNumericsNnCpp: nn-cpp's bits. kNumericsSplitDepth: every product with
// m n <= 2^18 and k >= 256 is cut into pieces whose depth is chosen so that the product fills the GPU (below).
constexpr int kNumericsNnCpp = 0;
constexpr int kNumericsSplitDepth = 1;
// The mode a call runs in is read once, where it enters the C ABI (NumericsScope): the stream's own mode
// (set_stream_numerics) if it has one, else the process default (set_numerics). numerics() returns that mode for
// the rest of the call on the calling thread, so every decision of one call (kernel choice, workspace size,
// partial layout) sees one mode whatever other threads set meanwhile; outside a call it is the process default.
int set_numerics(int mode);                      // process default; returns the previous one
int default_numerics();
int set_stream_numerics(void* stream, int mode); // mode < 0 clears the stream's own mode; returns the previous (-1: none)
int stream_numerics(void* stream);               // the stream's mode, else the process default
int numerics();
class NumericsScope {
public:
	explicit NumericsScope(void* stream);  // nested in another scope on this thread: keeps the outer call's mode
	NumericsScope(int mode, bool forced);  // a given mode (the workspace queries evaluate both)
	~NumericsScope();
	NumericsScope(const NumericsScope&) = delete;
	NumericsScope& operator=(const NumericsScope&) = delete;

private:
	int prev_;
};

// How a product's depth is cut: `pieces` contiguous slices of `piece_k` depth indices (the last one shorter),
// each a chain from +0, summed in piece order (acc = piece 0, acc += piece 1, ...), then stored or added to C.
// pieces <= 1: no cut, one chain over the whole depth. A pure function of (m, n, k) and the numerics mode, per
// matrix of a batch:
//   kNumericsNnCpp: nn-cpp's rule (src/kernels/gemm.cpp:453-461): m n <= 2^16, k >= 512 and m n k >= 2^20 cut
//     into 128-deep pieces.
//   kNumericsSplitDepth: m n <= 2^18 and k >= 256, with T = ceil(m / 64) ceil(n / 16) tiles of 64 x 16 and
//     s = min(16, max(2, 4096 / T)): piece_k = ceil(k / s) rounded up to a multiple of 32.
struct CutPlan {
	int64_t piece_k = 0;
	int64_t pieces = 1;
};
CutPlan cut_plan(int64_t m, int64_t n, int64_t k);
// cut_plan(m, n, k).pieces > 1. Every kernel that runs a whole-depth chain declines a product this is true for.
bool depth_cut(int64_t m, int64_t n, int64_t k);

// Whether a depth-cut product runs as one launch of the pieces kernel (gemm_pieces.hip): not gathered, no row sums,
// at most 16 pieces, dimensions below 2^24. Otherwise a cut product spreads its pieces over workgroups that write partial sums to the
// workspace, and a second kernel adds them in piece order.
bool pieces_kernel_takes(int64_t m, int64_t n, int64_t k, int64_t batch_count, bool gather_or_rowsum);
bool pieces_kernel_takes(const GemmCall& g);  // also: leading dimensions below 2^24
hipError_t gemm_pieces_launch(const GemmCall& g, hipStream_t s);
// The same products on the 16x16x4 MFMA: 16 x 16 tiles, a wave per piece, operands loaded into registers. It is
// the route of the cut products it takes (pieces4_takes: A transposed and B not, the weight gradient's layout, also
// with two-stage row sums; other layouts when their k-contiguous operands allow 16-byte loads); a forced
// configuration runs it on any product pieces_kernel_takes.
bool pieces4_takes(const GemmCall& g);
// Whole-depth products (no cut, no gather, no row sums) on the 16x16x4 MFMA without LDS (gemm_chain.hip).
bool chain4_ok(const GemmCall& g);
bool chain4_takes(const GemmCall& g);  // the shapes it is routed for (measured)
hipError_t gemm_chain4_launch(const GemmCall& g, hipStream_t s);
bool chain4_vec(const GemmCall& g);       // 16-byte loads of its k-contiguous operands
GemmArgs chain4_args(const GemmCall& g);  // the chain kernel's arguments (32 x 32 tiles)
hipError_t gemm_pieces4_launch(const GemmCall& g, hipStream_t s);
// A B on the chain kernel and A^T B (row sums allowed) on the pieces kernel in one launch (gemm_pieces.hip): single
// matrices, each taken by its own kernel's route (chain4_takes, a depth cut and pieces4_takes) and at most
// 768 threads for the pieces' workgroup. The caller guarantees that neither product writes what the other reads or
// writes.
bool chain_pieces_pair_takes(const GemmCall& g0, const GemmCall& g1);
// Two whole-depth products on the chain kernel in one launch (gemm_chain.hip): g0 = A B or A B^T and g1 = A^T B,
// each one the chain kernel's own route takes (chain4_takes). The caller guarantees that neither product writes what
// the other reads or writes.
bool chain4_pair_takes(const GemmCall& g0, const GemmCall& g1);
// Two or three whole-depth products of one layout on the chain kernel in one launch (gemm_chain.hip: several linear
// layers over one input), each at most 2^20 outputs and 256 deep. The caller guarantees that no product writes what
// another reads or writes.
constexpr int kChainGroupMax = 3;
bool chain4_group_takes(const GemmCall* g, int count);
hipError_t gemm_chain4_group_launch(const GemmCall* g, int count, hipStream_t s);
hipError_t gemm_chain4_pair_launch(const GemmCall& g0, const GemmCall& g1, hipStream_t s);
hipError_t gemm_chain_pieces_pair_launch(const GemmCall& g0, const GemmCall& g1, hipStream_t s);

// Floats of workspace a call needs: the partial sums of a depth cut the pieces kernel does not take, else 0. The
// shape-only overload (plans and workspace queries) assumes leading dimensions below 2^24, which every op's own
// products have (their leading dimensions are extents of tensors whose cut dimensions are below 2^24).
int64_t gemm_workspace_floats(const GemmCall& g);
int64_t gemm_workspace_floats(int64_t m, int64_t n, int64_t k, int64_t batch_count, bool gather = false);

// Launches on stream s. Kernel configuration: -1 picks one by shape; results never depend on it.
// Workspace for a depth cut comes from workspace (if non-null, at least gemm_workspace_floats) or else from
// the stream's StreamWorkspace (so a caller holding that one must pass workspace).
hipError_t gemm_launch(const GemmCall& g, hipStream_t s, int config = -1, float* workspace = nullptr);
// A B (g0) and A^T B (g1, row sums allowed) in one launch when both are single matrices without a depth cut and
// pick the same small-tile configuration; launched tells whether it did (otherwise nothing was launched and the
// caller runs them in turn). The caller guarantees that neither product writes what the other reads or writes.
hipError_t gemm_launch_pair(const GemmCall& g0, const GemmCall& g1, hipStream_t s, bool& launched);

// Two or three products in one launch where the chain kernel's group launch takes them (chain4_group_takes);
// launched tells whether it did (otherwise nothing was launched and the caller runs them in turn). The caller
// guarantees that no product writes what another reads or writes.
hipError_t gemm_launch_group(const GemmCall* g, int count, hipStream_t s, bool& launched);

int gemm_config_count();
const char* gemm_config_name(int config);

}  // namespace nnh
