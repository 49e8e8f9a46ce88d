// norm.hpp - launchers of the normalisation kernels in norm.hip (internal to libnnh): nn::batchnorm (with its
// folded ReLU) and nn::layernorm, forward and backward (src/autograd/ops.cpp:900-1078).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nnh {

// x {N, C, S}: S is the product of the axes after the channel axis (1 for a {N, C} input).
struct BnGeom {
	int64_t N = 0, C = 0, S = 0;
	float fm = 0.0f;   // static_cast<float>(N * S), converted on the host as the reference converts it
	double dm = 0.0;   // static_cast<double>(N * S)
};

// Scratch floats the forward and the backward take: two per (n, c) row.
inline int64_t batchnorm_scratch_floats(const BnGeom& g) { return 2 * g.N * g.C; }

// Training-mode forward (ops.cpp:900-958): per channel the mean and biased variance over N * S elements, then
// y = (x - mean) * (weight * inv_std) + bias, with relu: alive = y > 0 and y clipped at 0. mean and inv_std are
// required (the backward pass reads them), var optional.
hipError_t batchnorm_forward(const float* x, const float* w, const float* b, const BnGeom& g, float eps, int relu,
                             float* y, unsigned char* alive, float* mean, float* var, float* inv_std, float* scratch,
                             hipStream_t s);
// Its backward rule (ops.cpp:960-1000). alive null: no folded ReLU. dx, dw, db optional (null: not wanted);
// *_first: the buffer holds nothing yet (dx stores term + 0; dw and db store 0 + sum).
hipError_t batchnorm_backward(const float* gy, const float* x, const unsigned char* alive, const float* w,
                              const float* mean, const float* inv_std, const BnGeom& g, float* dx, int dx_first,
                              float* dw, int dw_first, float* db, int db_first, float* scratch, hipStream_t s);

// Forward over R rows of D (ops.cpp:1003-1034); fd = static_cast<float>(D). mean and inv_std per row, required.
hipError_t layernorm_forward(const float* x, const float* gamma, const float* beta, int64_t R, int D, float fd,
                             float eps, float* y, float* mean, float* inv_std, hipStream_t s);
// Its backward rule (ops.cpp:1035-1077). dx, dgamma, dbeta optional.
hipError_t layernorm_backward(const float* gy, const float* x, const float* gamma, const float* mean,
                              const float* inv_std, int64_t R, int D, float fd, float* dx, int dx_first,
                              float* dgamma, int dgamma_first, float* dbeta, int dbeta_first, hipStream_t s);

}  // namespace nnh
