// Instances of mm_lhsT_rhs_bf16 with block_m = 64 (rows of the 72-point search grid).
#include "mi_registry.hpp"

namespace mi {
MI_GRID_BK_W4_S(MI_MM_INST, 64, 64)
MI_GRID_BK_W_S(MI_MM_INST, 64, 128)
MI_GRID_BK_W_S(MI_MM_INST, 64, 256)
MI_MM_INST(64, 256, 128, 4, 2)

const MiEntry* table_mm_bm64(int* n) {
  static const MiEntry t[] = {
      MI_GRID_BK_W4_S(MI_MM_ROW, 64, 64)
      MI_GRID_BK_W_S(MI_MM_ROW, 64, 128)
      MI_GRID_BK_W_S(MI_MM_ROW, 64, 256)
      MI_MM_ROW(64, 256, 128, 4, 2)
  };
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
