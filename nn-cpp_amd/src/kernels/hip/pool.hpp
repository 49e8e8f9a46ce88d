// pool.hpp - launchers of the max-pooling kernels in pool.hip (internal to libnnh).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nnh {

// y[p][oh][ow] = max over the k x k window at (oh s, ow s) of plane p of x (planes of h x w), argmax (optional)
// its offset inside the plane, as nn::maxpool2d (ops.cpp:1609-1684).
hipError_t maxpool2d_forward(const float* x, float* y, uint32_t* arg, int64_t planes, int h, int w, int k, int s,
                             hipStream_t st);
// dx (first: from 0, else added to) += g at each output's argmax, in output order (ops.cpp:1686-1704).
hipError_t maxpool2d_backward(const float* g, const uint32_t* arg, float* dx, int64_t planes, int h, int w, int k, int s,
                              int first, hipStream_t st);
// Its 2 x 2, stride 2 form from 2-bit window positions (the fused conv2d_relu + pool's packed output; h and w even,
// dx 8-byte aligned).
hipError_t maxpool2x2_backward_slots(const float* g, const unsigned char* slots, float* dx, int64_t planes, int h, int w,
                                     int first, hipStream_t st);

}  // namespace nnh
