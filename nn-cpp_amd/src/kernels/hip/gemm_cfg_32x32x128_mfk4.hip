// Tile configuration 32x32x128_w16x16_mfk4 (workgroup 32 x 32 x 128, wave 16 x 16 of 16x16x4 MFMAs).
#include "gemm_config.hpp"

namespace nnh {
Config config_32x32x128_mfk4() { return make_config<32, 32, 128, 16, 16, 2, kMf16x4, true>("32x32x128_w16x16_mfk4"); }
}  // namespace nnh
