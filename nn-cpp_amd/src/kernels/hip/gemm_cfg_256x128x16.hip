// Tile configuration 256x128x16 (workgroup 256 x 128 x 16, wave 128 x 64).
#include "gemm_config.hpp"

namespace nnh {
Config config_256x128x16() { return make_config<256, 128, 16, 128, 64, 1>("256x128x16_w128x64"); }
}  // namespace nnh
