// Tile configuration 32x32x32_w16x16_mf4 (workgroup 32 x 32 x 32, wave 16 x 16 of 4x4x1 MFMAs).
#include "gemm_config.hpp"

namespace nnh {
Config config_32x32x32_mf4() { return make_config<32, 32, 32, 16, 16, 4, kMf4, true>("32x32x32_w16x16_mf4"); }
}  // namespace nnh
