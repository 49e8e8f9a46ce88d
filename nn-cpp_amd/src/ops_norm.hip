// ops_norm.hip - extern "C" entry points of nn::batchnorm and nn::layernorm (include/nnh.h).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "abi_common.hpp"
#include "kernels/hip/norm.hpp"
#include "nnh.h"
#include "workspace.hpp"

using namespace nnh;

namespace {

constexpr uint64_t kGridMax = ((uint64_t)1 << 31) - 1;

// ops.cpp:901-907: x needs a channel axis (the caller folds the axes after it into S); N, C and S describe it.
// Also the limits of the kernels' grids: C * ceil(N / 8) and C * ceil(N * S / 4096) workgroups.
int bn_geom(size_t N, size_t C, size_t S, BnGeom& g) {
	uint64_t count = 0;
	if (!count_ok({N, C, S}, count)) return fail(NNH_ERR_INVALID, "batchnorm: size out of range (above 2^60 elements)");
	const uint64_t M = (uint64_t)N * S;
	if (C > 0 && ((N + 7) / 8 > kGridMax / C || (M + 4095) / 4096 > kGridMax / C))
		return fail(NNH_ERR_INVALID, "batchnorm: too many channels for the grid");
	g.N = (int64_t)N;
	g.C = (int64_t)C;
	g.S = (int64_t)S;
	g.fm = static_cast<float>(static_cast<size_t>(M));   // static_cast<float>(M) (ops.cpp:982)
	g.dm = static_cast<double>(static_cast<size_t>(M));  // static_cast<double>(M) (ops.cpp:928)
	return NNH_OK;
}

size_t bn_ws(const BnGeom& g) {
	WorkspacePlan p;
	p.add((size_t)batchnorm_scratch_floats(g) * sizeof(float));
	return g.N * g.C == 0 ? 0 : p.total;
}

// ops.cpp:1004-1006: gamma and beta of the last axis' size; D = 0 divides by zero in the reference and is refused.
int ln_geom(size_t R, size_t D) {
	if (D == 0) return fail(NNH_ERR_INVALID, "layernorm: the last axis is empty");
	if (D >= ((size_t)1 << 31)) return fail(NNH_ERR_INVALID, "layernorm: rows longer than 2^31 elements");
	if (!count_ok({R, D})) return fail(NNH_ERR_INVALID, "layernorm: size out of range (above 2^60 elements)");
	if ((R + 255) / 256 + 1 > kGridMax) return fail(NNH_ERR_INVALID, "layernorm: too many rows for the grid");
	return NNH_OK;
}

}  // namespace

extern "C" {

int nnh_batchnorm_workspace_size(size_t N, size_t C, size_t S, size_t* bytes) {
	BnGeom g;
	const int rc = bn_geom(N, C, S, g);
	if (rc != NNH_OK) return rc;
	return put_bytes(bytes, bn_ws(g));
}

int nnh_batchnorm_forward(const float* x, size_t N, size_t C, size_t S, const float* weight, const float* bias,
                          float eps, int fuse_relu, float* y, unsigned char* alive, float* mean, float* var,
                          float* inv_std, void* stream) {
	BnGeom g;
	int rc = bn_geom(N, C, S, g);
	if (rc != NNH_OK) return rc;
	if (C == 0) return NNH_OK;
	const uint64_t xb = (uint64_t)N * C * S * 4, cb = (uint64_t)C * 4;
	if (!weight || !bias || !mean || !inv_std || (xb > 0 && (!x || !y)))
		return fail(NNH_ERR_INVALID, "batchnorm: null pointer");
	{
		const void* ins[3] = {x, weight, bias};
		const uint64_t in_bytes[3] = {xb, cb, cb};
		void* outs[5] = {y, alive, mean, var, inv_std};
		const uint64_t out_bytes[5] = {xb, fuse_relu ? xb / 4 : 0, cb, cb, cb};
		for (int o = 0; o < 5; ++o) {
			for (int i = 0; i < 3; ++i)
				if (ranges_overlap(outs[o], out_bytes[o], ins[i], in_bytes[i]))
					return fail(NNH_ERR_ALIAS, "batchnorm: an output overlaps an input");
			for (int p = o + 1; p < 5; ++p)
				if (ranges_overlap(outs[o], out_bytes[o], outs[p], out_bytes[p]))
					return fail(NNH_ERR_ALIAS, "batchnorm: outputs overlap each other");
		}
	}
	const size_t ws_bytes = bn_ws(g);
	rc = check_workspace(stream, ws_bytes);
	if (rc != NNH_OK) return rc;
	hipStream_t s = reinterpret_cast<hipStream_t>(stream);
	StreamWorkspace ws(s, ws_bytes);
	if (ws.error() != hipSuccess) return hip_status(ws.error(), "batchnorm workspace");
	return hip_status(batchnorm_forward(x, weight, bias, g, eps, fuse_relu ? 1 : 0, y, fuse_relu ? alive : nullptr, mean,
	                                    var, inv_std, ws_bytes ? ws.at<float>(0) : nullptr, s),
	                  "batchnorm forward");
}

int nnh_batchnorm_backward(const float* g, const float* x, const unsigned char* alive, const float* weight,
                           const float* mean, const float* inv_std, size_t N, size_t C, size_t S, float* dx,
                           int dx_first, float* dweight, int dweight_first, float* dbias, int dbias_first,
                           void* stream) {
	BnGeom geo;
	int rc = bn_geom(N, C, S, geo);
	if (rc != NNH_OK) return rc;
	if (C == 0 || (!dx && !dweight && !dbias)) return NNH_OK;
	const uint64_t xb = (uint64_t)N * C * S * 4, cb = (uint64_t)C * 4;
	if (!weight || !mean || !inv_std || (xb > 0 && (!g || !x))) return fail(NNH_ERR_INVALID, "batchnorm backward: null pointer");
	{
		const void* ins[6] = {g, x, alive, weight, mean, inv_std};
		const uint64_t in_bytes[6] = {xb, xb, xb / 4, cb, cb, cb};
		void* outs[3] = {dx, dweight, dbias};
		const uint64_t out_bytes[3] = {xb, cb, cb};
		for (int o = 0; o < 3; ++o) {
			for (int i = 0; i < 6; ++i)
				if (ranges_overlap(outs[o], out_bytes[o], ins[i], in_bytes[i]))
					return fail(NNH_ERR_ALIAS, "batchnorm backward: a gradient overlaps an input");
			for (int p = o + 1; p < 3; ++p)
				if (ranges_overlap(outs[o], out_bytes[o], outs[p], out_bytes[p]))
					return fail(NNH_ERR_ALIAS, "batchnorm backward: gradients overlap each other");
		}
	}
	const size_t ws_bytes = bn_ws(geo);
	rc = check_workspace(stream, ws_bytes);
	if (rc != NNH_OK) return rc;
	hipStream_t s = reinterpret_cast<hipStream_t>(stream);
	StreamWorkspace ws(s, ws_bytes);
	if (ws.error() != hipSuccess) return hip_status(ws.error(), "batchnorm workspace");
	return hip_status(batchnorm_backward(g, x, alive, weight, mean, inv_std, geo, xb ? dx : nullptr, dx_first ? 1 : 0,
	                                     dweight, dweight_first ? 1 : 0, dbias, dbias_first ? 1 : 0,
	                                     ws_bytes ? ws.at<float>(0) : nullptr, s),
	                  "batchnorm backward");
}

int nnh_layernorm_forward(const float* x, size_t R, size_t D, const float* gamma, const float* beta, float eps,
                          float* y, float* mean, float* inv_std, void* stream) {
	int rc = ln_geom(R, D);
	if (rc != NNH_OK) return rc;
	if (R == 0) return NNH_OK;
	if (!x || !gamma || !beta || !y || !mean || !inv_std) return fail(NNH_ERR_INVALID, "layernorm: null pointer");
	const uint64_t xb = (uint64_t)R * D * 4, db = (uint64_t)D * 4, rb = (uint64_t)R * 4;
	{
		const void* ins[3] = {x, gamma, beta};
		const uint64_t in_bytes[3] = {xb, db, db};
		void* outs[3] = {y, mean, inv_std};
		const uint64_t out_bytes[3] = {xb, rb, rb};
		for (int o = 0; o < 3; ++o) {
			for (int i = 0; i < 3; ++i)
				if (ranges_overlap(outs[o], out_bytes[o], ins[i], in_bytes[i]))
					return fail(NNH_ERR_ALIAS, "layernorm: an output overlaps an input");
			for (int p = o + 1; p < 3; ++p)
				if (ranges_overlap(outs[o], out_bytes[o], outs[p], out_bytes[p]))
					return fail(NNH_ERR_ALIAS, "layernorm: outputs overlap each other");
		}
	}
	return hip_status(layernorm_forward(x, gamma, beta, (int64_t)R, (int)D, static_cast<float>(D), eps, y, mean, inv_std,
	                                    reinterpret_cast<hipStream_t>(stream)),
	                  "layernorm forward");
}

int nnh_layernorm_backward(const float* g, const float* x, const float* gamma, const float* mean, const float* inv_std,
                           size_t R, size_t D, float* dx, int dx_first, float* dgamma, int dgamma_first, float* dbeta,
                           int dbeta_first, void* stream) {
	int rc = ln_geom(R, D);
	if (rc != NNH_OK) return rc;
	if (!dx && !dgamma && !dbeta) return NNH_OK;
	if (R == 0) dx = nullptr;  // nothing to write; dgamma and dbeta still receive their (empty) sums
	if (!gamma || (R > 0 && (!g || !x || !mean || !inv_std))) return fail(NNH_ERR_INVALID, "layernorm backward: null pointer");
	const uint64_t xb = (uint64_t)R * D * 4, db = (uint64_t)D * 4, rb = (uint64_t)R * 4;
	{
		const void* ins[5] = {g, x, gamma, mean, inv_std};
		const uint64_t in_bytes[5] = {xb, xb, db, rb, rb};
		void* outs[3] = {dx, dgamma, dbeta};
		const uint64_t out_bytes[3] = {xb, db, db};
		for (int o = 0; o < 3; ++o) {
			for (int i = 0; i < 5; ++i)
				if (ranges_overlap(outs[o], out_bytes[o], ins[i], in_bytes[i]))
					return fail(NNH_ERR_ALIAS, "layernorm backward: a gradient overlaps an input");
			for (int p = o + 1; p < 3; ++p)
				if (ranges_overlap(outs[o], out_bytes[o], outs[p], out_bytes[p]))
					return fail(NNH_ERR_ALIAS, "layernorm backward: gradients overlap each other");
		}
	}
	return hip_status(layernorm_backward(g, x, gamma, mean, inv_std, (int64_t)R, (int)D, static_cast<float>(D), dx,
	                                     dx_first ? 1 : 0, dgamma, dgamma_first ? 1 : 0, dbeta, dbeta_first ? 1 : 0,
	                                     reinterpret_cast<hipStream_t>(stream)),
	                  "layernorm backward");
}

}  // extern "C"
