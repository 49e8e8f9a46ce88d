// Tile configuration 128x64x32_w64x32_mfk4 (workgroup 128 x 64 x 32, wave 64 x 32 of 16x16x4 MFMAs).
#include "gemm_config.hpp"

namespace nnh {
Config config_128x64x32_mfk4() { return make_config<128, 64, 32, 64, 32, 2, kMf16x4>("128x64x32_w64x32_mfk4"); }
}  // namespace nnh
