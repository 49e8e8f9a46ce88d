// Tile configuration 128x256x16 (workgroup 128 x 256 x 16, wave 128 x 64).
#include "gemm_config.hpp"

namespace nnh {
Config config_128x256x16() { return make_config<128, 256, 16, 128, 64, 1>("128x256x16_w128x64"); }
}  // namespace nnh
