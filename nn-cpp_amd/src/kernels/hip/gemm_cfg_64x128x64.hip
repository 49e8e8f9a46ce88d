// Tile configuration 64x128x64 (workgroup 64 x 128 x 64, wave 64 x 32).
#include "gemm_config.hpp"

namespace nnh {
Config config_64x128x64() { return make_config<64, 128, 64, 64, 32, 3>("64x128x64_w64x32"); }
}  // namespace nnh
