// Tile configuration 64x64x32_w64x16_mf16 (workgroup 64 x 64 x 32, wave 64 x 16 of 16x16x1 MFMAs).
#include "gemm_config.hpp"

namespace nnh {
Config config_64x64x32_mf16() { return make_config<64, 64, 32, 64, 16, 4, kMf16, true>("64x64x32_w64x16_mf16"); }
}  // namespace nnh
