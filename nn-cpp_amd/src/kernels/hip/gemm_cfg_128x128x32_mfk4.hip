// Tile configuration 128x128x32_w64x64_mfk4 (workgroup 128 x 128 x 32, wave 64 x 64 of 16x16x4 MFMAs).
#include "gemm_config.hpp"

namespace nnh {
Config config_128x128x32_mfk4() { return make_config<128, 128, 32, 64, 64, 2, kMf16x4>("128x128x32_w64x64_mfk4"); }
}  // namespace nnh
