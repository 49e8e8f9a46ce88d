// conv.hpp - launchers of the convolution kernels (internal to libnnh).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nnh {

// One convolution's geometry (ConvGeometry, src/autograd/ops.cpp:164-176): input cin x h x w, kernel kh x kw,
// stride, zero padding, output ho x wo.
struct ConvGeom {
	int cin, h, w, kh, kw, stride, pad, ho, wo;
};

hipError_t im2col(const float* x, float* col, const ConvGeom& g, int64_t samples, hipStream_t s);
hipError_t col2im(const float* col, float* dx, const ConvGeom& g, int64_t samples, int first, hipStream_t s);
// 3x3, stride 1, padding 1 convolutions of planes up to 14 x 14 as MFMA chains over the input held in LDS
// (conv_fwd3.hip): whether it takes this forward (no depth cut, Cout a multiple of 32, 16-byte aligned y), and
// the launch.
bool conv_fwd3_ok(const ConvGeom& g, int64_t samples, int cout, const float* y, const unsigned char* alive);
hipError_t conv_fwd3(const float* x, const float* w, const float* bias, float* y, unsigned char* alive,
                     const ConvGeom& g, int64_t samples, int cout, int relu, hipStream_t s);
// The per-sample weight gradients dW_n = g_n col_n^T of the same convolutions (conv_dw3.hip; Cout a multiple of
// 64, K = Cin*9 <= 384, hw % 4 == 0, 16-byte aligned gradient), into gw {N, Cout, K}: whether it takes them, and
// the launch. With alive (4-byte aligned), the gradient is masked as it is read and the masked gradient is written
// to gmo (16-byte aligned); with gb, gb {N, Cout} receives the per-sample bias gradients (lane sums of the masked
// rows).
bool conv_dw3_ok(const ConvGeom& g, int64_t samples, int cout, const float* gr, const unsigned char* alive,
                 const float* gmo);
hipError_t conv_dw3(const float* gr, const unsigned char* alive, float* gmo, float* gb, const float* x, float* gw,
                    const ConvGeom& g, int64_t samples, int cout, hipStream_t s);
hipError_t conv_direct(const float* x, const float* w, const float* bias, float* y, unsigned char* alive,
                       const ConvGeom& g, int64_t samples, int cout, int relu, hipStream_t s);
// The direct kernel's vectorised form (stride 1, "same" width, w % 4 == 0, aligned buffers), with an explicit
// number of output channels per lane (4 or 8); conv_direct uses it whenever conv_same_quad_ok holds.
bool conv_same_quad_ok(const float* x, const float* y, const unsigned char* alive, const ConvGeom& g, int64_t samples);
// conv2d_relu then maxpool2d(2, 2) in one pass (conv_pool.hip): whether it takes the geometry and pointers, and the
// launch (alive and argmax may be null).
bool conv_relu_pool2_ok(const float* x, const float* y, const unsigned char* alive, const float* pooled,
                        const uint32_t* argmax, const ConvGeom& g, int64_t samples);
// bits / amax2 (both or neither, alive and argmax then null, W <= 256): the packed flags and window slots
// (conv_pool.hip states the layouts).
hipError_t conv_relu_pool2(const float* x, const float* w, const float* bias, float* y, unsigned char* alive,
                           float* pooled, uint32_t* argmax, const ConvGeom& g, int64_t samples, int cout, hipStream_t s,
                           unsigned char* bits = nullptr, unsigned char* amax2 = nullptr);
// bits: the ReLU's flags packed one bit per output in y's order (byte o / 8, bit o % 8; Ho Wo a multiple of 8).
hipError_t conv_same_quad(const float* x, const float* w, const float* bias, float* y, unsigned char* alive,
                          const ConvGeom& g, int64_t samples, int cout, int relu, int cg, hipStream_t s,
                          unsigned char* bits = nullptr);
hipError_t mask_grad(const float* g, const unsigned char* alive, float* out, int64_t total, hipStream_t s);
// mask_grad and lane_sums in one pass: out = alive ? g : 0 over rows x n, dst[row] = lane_sum of out's row.
// dx of nn::conv2d's backward from the masked output gradient gm {samples, cout, Ho*Wo} (ops.cpp:1452-1455): the
// per-sample dcol = W^T gm and col2im in one kernel, dcol kept in LDS (same bits). first: dx = 0 + taps, else
// dx += taps. conv_dx_fused_ok tells whether the geometry fits (Ho*Wo <= 256, or Ho*Wo <= 1024 with kh*kw <= 16).
bool conv_dx_fused_ok(const ConvGeom& g, int64_t samples, int cout);
// Per-sample bias sums and weight gradients of a convolution with K = Cin*kh*kw <= 16 on planes of up to 1024
// output positions (conv_dwp.hip): gb[n][c] = lane_sum of the masked gradient row, gw[n][c][k] = its product with
// column k of sample n, one fma chain per element; the masked gradient stays in LDS. Declines depth-cut products.
bool conv_dwp_ok(const ConvGeom& g, int64_t samples, int cout);
hipError_t conv_dwp(const float* g, const unsigned char* alive, const float* x, float* gb, float* gw,
                    const ConvGeom& geo, int64_t samples, int cout, hipStream_t s);
hipError_t conv_dx_fused(const float* gm, const unsigned char* alive, const float* w, float* dx, const ConvGeom& g,
                         int64_t samples, int cout, int first, hipStream_t s);
// The whole backward of a first layer (conv_first.hip: K = Cin*kh*kw <= 16, Cout <= 32, stride 1, Ho*Wo a multiple
// of 4 up to 65536, 16-byte aligned g, flags 4-byte aligned bytes or, alive_bits, one bit per output in y's order)
// in one launch, a workgroup per sample: the per-sample bias sums gb {N, Cout} (may be null) and weight gradients
// gw {N, Cout, K}, and dx (may be null; first: dx = 0 + taps, else dx += taps), g masked as it is read. Declines
// depth-cut products.
bool conv_first_bwd_ok(const ConvGeom& g, int64_t samples, int cout, bool dx, const float* gr,
                       const unsigned char* alive, bool alive_bits = false);
hipError_t conv_first_bwd(const float* g, const unsigned char* alive, const float* x, const float* w, float* gb,
                          float* gw, float* dx, int dx_first, const ConvGeom& geo, int64_t samples, int cout,
                          hipStream_t s, bool alive_bits = false);
hipError_t masked_lane_sums(const float* g, const unsigned char* alive, float* out, int64_t rows, int64_t n, float* dst,
                            hipStream_t s);
hipError_t lane_sums(const float* src, int64_t rows, int64_t n, float* dst, hipStream_t s);

}  // namespace nnh
