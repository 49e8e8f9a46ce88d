// noalloc.hip - nnh_sgemm_noalloc: nnh_sgemm for callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc).
//
// nnh_sgemm's only scratch is the depth-cut partial sums (one m x n partial per 128-deep piece, summed in piece
// order by a second kernel), written by cut products whose pieces are spread over workgroups. Here they live in `scratch`, a file-scope device array of kScratchFloats floats that
// every GPU the library runs on holds until the process ends. In host code the name `scratch` is a host-side
// stand-in, not a device address: its address on a device comes from hipGetSymbolAddress, taken once per device
// (with that device current) on the first call there, and only that address is passed to kernels.
//
// Every call on one GPU shares that GPU's array. Calls on one stream run in order; calls that overlap on one GPU
// (different streams, no ordering between them) race on it. Each piece writes its whole partial before the
// reduction reads it, so nothing needs clearing between calls.
#include <hip/hip_runtime.h>

#include <mutex>

#include "abi_common.hpp"
#include "kernels/hip/gemm.hpp"
#include "nnh.h"
#include "nnh_noalloc.h"

namespace nnh {

namespace {

constexpr size_t kScratchFloats = size_t(1) << 22;  // 16 MiB: every depth cut up to k = 8192 (m n <= 2^16)
constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[kScratchFloats];

std::mutex scratch_mu;
float* scratch_ptr[kMaxDevices] = {};

// The device address of this GPU's `scratch` (dev is the device the call's stream belongs to).
int device_scratch(int dev, float** out) {
	if (dev < 0 || dev >= kMaxDevices) return fail(NNH_ERR_INVALID, "device index out of range");
	std::lock_guard<std::mutex> lock(scratch_mu);
	if (!scratch_ptr[dev]) {
		int cur = 0;
		int rc = hip_status(hipGetDevice(&cur), "hipGetDevice");
		if (rc != NNH_OK) return rc;
		if (cur != dev) {
			rc = hip_status(hipSetDevice(dev), "hipSetDevice");
			if (rc != NNH_OK) return rc;
		}
		void* p = nullptr;
		const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
		if (cur != dev) (void)hipSetDevice(cur);
		rc = hip_status(e, "hipGetSymbolAddress(scratch)");
		if (rc != NNH_OK) return rc;
		if (!p) return fail(NNH_ERR_HIP, "hipGetSymbolAddress(scratch) gave a null address");
		scratch_ptr[dev] = static_cast<float*>(p);
	}
	*out = scratch_ptr[dev];
	return NNH_OK;
}

}  // namespace

}  // namespace nnh

using namespace nnh;

extern "C" {

size_t nnh_sgemm_noalloc_max_workspace(void) { return kScratchFloats * sizeof(float); }

int nnh_sgemm_noalloc(int trans_a, int trans_b, size_t m, size_t n, size_t k, const float* a, size_t lda,
                      const float* b, size_t ldb, float* c, size_t ldc, int accumulate, void* stream) {
	NumericsScope numerics_scope(stream);
	GemmCall g;
	int rc = build_gemm(trans_a, trans_b, m, n, k, a, lda, b, ldb, c, ldc, accumulate, nullptr, nullptr, g);
	if (rc != NNH_OK) return rc;
	if (g.m == 0 || g.n == 0) return NNH_OK;
	const int64_t need = gemm_workspace_floats(g);
	if (need > (int64_t)kScratchFloats)
		return fail(NNH_ERR_INVALID, "nnh_sgemm_noalloc: the depth-cut partials (" + std::to_string(need * 4) +
		                                 " bytes) exceed the static scratch (" + std::to_string(kScratchFloats * 4) + " bytes)");
	float* part = nullptr;
	if (need > 0) {
		hipDevice_t dev = 0;
		rc = hip_status(hipStreamGetDevice(reinterpret_cast<hipStream_t>(stream), &dev), "hipStreamGetDevice");
		if (rc != NNH_OK) return rc;
		rc = device_scratch((int)dev, &part);
		if (rc != NNH_OK) return rc;
	}
	// with an explicit workspace the launch takes no stream workspace and allocates nothing
	return hip_status(gemm_launch(g, reinterpret_cast<hipStream_t>(stream), -1, part), "sgemm launch");
}

}  // extern "C"
