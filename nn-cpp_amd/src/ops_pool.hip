// ops_pool.hip - extern "C" entry points of nn::maxpool2d (include/nnh.h).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <limits>

#include "abi_common.hpp"
#include "kernels/hip/pool.hpp"
#include "nnh.h"

using namespace nnh;

namespace nnh {

// ops.cpp:1610-1627: 4-D input, kernel and stride positive, the window inside the plane, plane offsets in 32 bits.
int maxpool_geometry(size_t H, size_t W, size_t kernel, size_t stride, size_t& ho, size_t& wo) {
	if (kernel == 0 || stride == 0) return fail(NNH_ERR_SHAPE, "maxpool2d: kernel and stride must be positive");
	if (kernel > H || kernel > W) return fail(NNH_ERR_SHAPE, "maxpool2d: kernel larger than the input plane");
	if ((unsigned __int128)H * W > std::numeric_limits<uint32_t>::max())
		return fail(NNH_ERR_SHAPE, "maxpool2d: plane beyond 2^32 elements");
	if (H >= (1u << 30) || W >= (1u << 30) || H * W >= ((size_t)1 << 31))
		return fail(NNH_ERR_INVALID, "maxpool2d: plane too large");
	ho = (H - kernel) / stride + 1;  // conv2d_output_size with no padding (ops.cpp:135-139)
	wo = (W - kernel) / stride + 1;
	return NNH_OK;
}

}  // namespace nnh

extern "C" {

int nnh_maxpool2d_forward(const float* x, size_t N, size_t C, size_t H, size_t W, size_t kernel, size_t stride,
                          float* y, unsigned int* argmax, void* stream) {
	if (!count_ok({N, C, H, W})) return fail(NNH_ERR_INVALID, "maxpool2d: size out of range (above 2^60 elements)");
	size_t ho = 0, wo = 0;
	int rc = maxpool_geometry(H, W, kernel, stride, ho, wo);
	if (rc != NNH_OK) return rc;
	const size_t planes = N * C;
	if (planes == 0) return NNH_OK;
	if (!x || !y) return fail(NNH_ERR_INVALID, "maxpool2d: null pointer");
	const uint64_t xb = (uint64_t)planes * H * W * 4, yb = (uint64_t)planes * ho * wo * 4;
	if (ranges_overlap(y, yb, x, xb) || ranges_overlap(argmax, yb, x, xb) || ranges_overlap(argmax, yb, y, yb))
		return fail(NNH_ERR_ALIAS, "maxpool2d: outputs overlap each other or the input");
	return hip_status(maxpool2d_forward(x, y, argmax, (int64_t)planes, (int)H, (int)W, (int)kernel, (int)stride,
	                                    reinterpret_cast<hipStream_t>(stream)),
	                  "maxpool2d forward");
}

int nnh_maxpool2d_backward(const float* g, const unsigned int* argmax, size_t N, size_t C, size_t H, size_t W,
                           size_t kernel, size_t stride, float* dx, int first, void* stream) {
	if (!count_ok({N, C, H, W})) return fail(NNH_ERR_INVALID, "maxpool2d backward: size out of range (above 2^60 elements)");
	size_t ho = 0, wo = 0;
	int rc = maxpool_geometry(H, W, kernel, stride, ho, wo);
	if (rc != NNH_OK) return rc;
	const size_t planes = N * C;
	if (planes == 0) return NNH_OK;
	if (!g || !argmax || !dx) return fail(NNH_ERR_INVALID, "maxpool2d backward: null pointer");
	const uint64_t xb = (uint64_t)planes * H * W * 4, yb = (uint64_t)planes * ho * wo * 4;
	if (ranges_overlap(dx, xb, g, yb) || ranges_overlap(dx, xb, argmax, yb))
		return fail(NNH_ERR_ALIAS, "maxpool2d backward: dx overlaps g or argmax");
	return hip_status(maxpool2d_backward(g, argmax, dx, (int64_t)planes, (int)H, (int)W, (int)kernel, (int)stride,
	                                     first ? 1 : 0, reinterpret_cast<hipStream_t>(stream)),
	                  "maxpool2d backward");
}

int nnh_maxpool2d_backward_packed(const float* g, const unsigned char* argmax2, size_t N, size_t C, size_t H, size_t W,
                                  float* dx, int first, void* stream) {
	if (!count_ok({N, C, H, W})) return fail(NNH_ERR_INVALID, "maxpool2d backward packed: size out of range");
	size_t ho = 0, wo = 0;
	int rc = maxpool_geometry(H, W, 2, 2, ho, wo);
	if (rc != NNH_OK) return rc;
	const size_t planes = N * C;
	if (planes == 0) return NNH_OK;
	if (!g || !argmax2 || !dx) return fail(NNH_ERR_INVALID, "maxpool2d backward packed: null pointer");
	if (H % 2 != 0 || W % 2 != 0 || reinterpret_cast<uintptr_t>(dx) % 8 != 0)
		return fail(NNH_ERR_INVALID, "maxpool2d backward packed: H and W must be even and dx 8-byte aligned");
	const uint64_t xb = (uint64_t)planes * H * W * 4, yb = (uint64_t)planes * ho * wo * 4;
	const uint64_t ab = (uint64_t)planes * (H / 2) * ((W + 7) / 8);
	if (ranges_overlap(dx, xb, g, yb) || ranges_overlap(dx, xb, argmax2, ab))
		return fail(NNH_ERR_ALIAS, "maxpool2d backward packed: dx overlaps g or argmax2");
	return hip_status(maxpool2x2_backward_slots(g, argmax2, dx, (int64_t)planes, (int)H, (int)W, first ? 1 : 0,
	                                            reinterpret_cast<hipStream_t>(stream)),
	                  "maxpool2d backward packed");
}

}  // extern "C"
