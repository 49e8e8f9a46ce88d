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
};

// Numerics modes (nnh_set_numerics). kNumericsNnCpp: nn-cpp's bits. kNumericsSplitDepth: every product with
// m n <= 2^18 and k >= 256 also takes the depth cut below, so its chains are at most 128 deep.
constexpr int kNumericsNnCpp = 0;
constexpr int kNumericsSplitDepth = 1;
int set_numerics(int mode);  // returns the previous mode
int numerics();

// nn-cpp's depth-cut rule (src/kernels/gemm.cpp:453-458): small output, long depth -> 128-deep pieces
// summed in piece order (and, in kNumericsSplitDepth, the wider rule above). Applies per matrix; every kernel
// that runs a whole-depth chain declines a product this returns true for.
bool depth_cut(int64_t m, int64_t n, int64_t k);

// Floats of workspace a call needs (0 when it takes no depth cut).
int64_t gemm_workspace_floats(const GemmCall& g);
int64_t gemm_workspace_floats(int64_t m, int64_t n, int64_t k, int64_t batch_count);

// Launches on stream s. Kernel configuration: -1 picks one by shape; results never depend on it.
// Workspace for a depth cut comes from workspace (if non-null, at least gemm_workspace_floats) or else from
// the stream's StreamWorkspace (so a caller holding that one must pass workspace).
hipError_t gemm_launch(const GemmCall& g, hipStream_t s, int config = -1, float* workspace = nullptr);
// A B (g0) and A^T B (g1, row sums allowed) in one launch when both are single matrices without a depth cut and
// pick the same small-tile configuration; launched tells whether it did (otherwise nothing was launched and the
// caller runs them in turn). The caller guarantees that neither product writes what the other reads or writes.
hipError_t gemm_launch_pair(const GemmCall& g0, const GemmCall& g1, hipStream_t s, bool& launched);

int gemm_config_count();
const char* gemm_config_name(int config);

}  // namespace nnh
