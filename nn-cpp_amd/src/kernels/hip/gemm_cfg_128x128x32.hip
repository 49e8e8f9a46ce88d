// Tile configuration 128x128x32 (workgroup 128 x 128 x 32, wave 64 x 64).
#include "gemm_config.hpp"

namespace nnh {
Config config_128x128x32() { return make_config<128, 128, 32, 64, 64, 2>("128x128x32_w64x64"); }
}  // namespace nnh
