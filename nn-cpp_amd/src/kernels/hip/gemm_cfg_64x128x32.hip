// Tile configuration 64x128x32 (workgroup 64 x 128 x 32, wave 64 x 32).
#include "gemm_config.hpp"

namespace nnh {
Config config_64x128x32() { return make_config<64, 128, 32, 64, 32, 3>("64x128x32_w64x32"); }
}  // namespace nnh
