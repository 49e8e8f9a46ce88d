// Tile configuration 64x256x32 (workgroup 64 x 256 x 32, wave 64 x 64).
#include "gemm_config.hpp"

namespace nnh {
Config config_64x256x32() { return make_config<64, 256, 32, 64, 64, 2>("64x256x32_w64x64"); }
}  // namespace nnh
