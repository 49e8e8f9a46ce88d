// Tile configuration 64x64x32_w32x32_mfk4 (workgroup 64 x 64 x 32, wave 32 x 32 of 16x16x4 MFMAs).
#include "gemm_config.hpp"

namespace nnh {
Config config_64x64x32_mfk4() { return make_config<64, 64, 32, 32, 32, 4, kMf16x4, true>("64x64x32_w32x32_mfk4"); }
}  // namespace nnh
