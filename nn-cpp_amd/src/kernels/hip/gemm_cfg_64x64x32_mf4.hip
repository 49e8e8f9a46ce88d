// Tile configuration 64x64x32_w32x32_mf4 (workgroup 64 x 64 x 32, wave 32 x 32 of 4x4x1 MFMAs).
#include "gemm_config.hpp"

namespace nnh {
Config config_64x64x32_mf4() { return make_config<64, 64, 32, 32, 32, 4, kMf4>("64x64x32_w32x32_mf4"); }
}  // namespace nnh
