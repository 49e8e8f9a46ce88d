// attention.hpp - launcher of the fused attention forward kernel (internal to libnnh).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nnh {

// Whether the fused kernel takes this attention: head width 64, Tk <= 256 and a multiple of 4, 16-byte aligned
// operands (pad may be null). Other shapes run as batched GEMM, row softmax, batched GEMM.
bool attention_fused_ok(int64_t tq, int64_t tk, int64_t dh, int64_t d, const void* q, const void* k, const void* v,
                        const void* out, const void* probs, const void* pad);

// nn::attention forward (src/autograd/ops.cpp:1226-1261) for q {n, tq, d}, k and v {n, tk, d}, heads of width 64:
// probs {n, heads, tq, tk} and out {n, tq, d}, bit for bit the reference's.
hipError_t attention_fused_forward(const float* q, const float* k, const float* v, int64_t n, int64_t tq, int64_t tk,
                                   int64_t d, int64_t heads, const float* pad, int causal, float scale, float* out,
                                   float* probs, hipStream_t s);

// The first half of nn::attention's backward (ops.cpp:1286-1290) for the same shapes: dP = G_h V_h^T and the
// softmax backward, ds {n, heads, tq, tk} = dL/d(scores), bit for bit the reference's.
hipError_t attention_fused_dscores(const float* g, const float* v, const float* probs, int64_t n, int64_t tq, int64_t tk,
                                   int64_t d, int64_t heads, const float* pad, int causal, float scale, float* ds,
                                   hipStream_t s);

}  // namespace nnh
