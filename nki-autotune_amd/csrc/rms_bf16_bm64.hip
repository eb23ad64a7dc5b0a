// Instances of the fused rmsnorm_matmul kernel with block_m = 64, both
// normalisation placements (variant 0: 1/rms on the accumulator after the
// K loop; variant 1: 1/rms prologue, rows scaled while staged into LDS).
#include "mi_registry.hpp"

namespace mi {
MI_GRID_BK_W4_S(MI_RMS_INST, 64, 64, , 0)
MI_GRID_BK_W4_S(MI_RMS_INST, 64, 64, , 1)
MI_GRID_BK_W_S(MI_RMS_INST, 64, 128, , 0)
MI_GRID_BK_W_S(MI_RMS_INST, 64, 128, , 1)
MI_GRID_BK_W_S(MI_RMS_INST, 64, 256, , 0)
MI_GRID_BK_W_S(MI_RMS_INST, 64, 256, , 1)

const MiEntry* table_rms_bm64(int* n) {
  static const MiEntry t[] = {
      MI_GRID_BK_W4_S(MI_RMS_ROW, 64, 64, , 0)
      MI_GRID_BK_W4_S(MI_RMS_ROW, 64, 64, , 1)
      MI_GRID_BK_W_S(MI_RMS_ROW, 64, 128, , 0)
      MI_GRID_BK_W_S(MI_RMS_ROW, 64, 128, , 1)
      MI_GRID_BK_W_S(MI_RMS_ROW, 64, 256, , 0)
      MI_GRID_BK_W_S(MI_RMS_ROW, 64, 256, , 1)
  };
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
