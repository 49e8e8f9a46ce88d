// Tile configuration 128x64x32 (workgroup 128 x 64 x 32, wave 64 x 32).
#include "gemm_config.hpp"

namespace nnh {
Config config_128x64x32() { return make_config<128, 64, 32, 64, 32, 3>("128x64x32_w64x32"); }
}  // namespace nnh
