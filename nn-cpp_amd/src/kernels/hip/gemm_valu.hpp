// gemm_valu.hpp - the fp32 GEMM on the vector ALUs (gemm_valu.hip; internal to libnnh): one fma chain per C element
// as the MFMA kernel, for products whose outputs cannot fill the GPU with MFMA chains.
#pragma once

#include "gemm.hpp"

namespace nnh {

// Lane blocks: 2 x 2 chains (32 x 32 workgroup tiles), 1 x 2 (16 x 32), 2 x 4 (32 x 64), 1 x 4 (16 x 64).
constexpr int kValu2x2 = 0;
constexpr int kValu1x2 = 1;
constexpr int kValu2x4 = 2;
constexpr int kValu1x4 = 3;
// The row-broadcast kernel (op(A) by DPP row broadcasts, only op(B) in LDS): RM chains per lane, tile 16 RM x 16.
constexpr int kValuBc1 = 4;
constexpr int kValuBc2 = 5;
constexpr int kValuShapes = 6;

// Whether the shape-based choice sends this product to a VALU kernel (no gather, no row sums, no depth cut, a depth
// of 256 or more, at most 2^17 outputs, or 2^18 at depths up to 512 when neither operand is transposed), and which kernel
// and lane block it takes.
bool valu_takes(const GemmCall& g);
int valu_shape(const GemmCall& g);
// The launch (any product without gather, row sums or a depth cut; k > 0).
hipError_t gemm_valu_launch(const GemmCall& g, int shape, hipStream_t s);

// Cut products (nn-cpp's depth cut, or the split-depth mode's) of at most 8 pieces of at most 128 steps and at most
// 2^16 outputs, on the VALU: up to 4 pieces (op(A) untransposed) as chains in one lane, 5 to 8 split over the waves.
bool valu_pieces_takes(const GemmCall& g);
// Whether the kernel can take the product at all (any layout, up to 8 pieces): configuration kValuPiecesConfig.
bool valu_pieces_ok(const GemmCall& g);
hipError_t gemm_valu_pieces_launch(const GemmCall& g, hipStream_t s);

}  // namespace nnh
