// softmax.hpp - launchers of the row softmax kernels (internal to libnnh).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nnh {

// masked_softmax_row over `rows` rows of length tk (src/autograd/ops.cpp:1183-1204); row r has query index
// r % tq and sample r / (heads * tq) (for the {N, Tk} padding mask). in may equal out.
hipError_t softmax_rows(const float* in, float* out, int64_t rows, int tk, int tq, int heads, float scale,
                        const float* pad, int causal, hipStream_t s);

// Its backward (ops.cpp:1216-1224; 1323-1342). mode 0/1: out = masked ? 0 : term + 0; mode 2: out += term where
// not masked. g_in may equal out.
hipError_t softmax_backward_rows(const float* y, const float* g_in, float* out, int64_t rows, int tk, int tq,
                                 int heads, float scale, const float* pad, int causal, int mode, hipStream_t s);

// Longest row the LDS-resident kernels take.
int softmax_max_row_length();

}  // namespace nnh
