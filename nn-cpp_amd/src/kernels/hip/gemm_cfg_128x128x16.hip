// Tile configuration 128x128x16 (workgroup 128 x 128 x 16, wave 64 x 64).
#include "gemm_config.hpp"

namespace nnh {
Config config_128x128x16() { return make_config<128, 128, 16, 64, 64, 2>("128x128x16_w64x64"); }
}  // namespace nnh
