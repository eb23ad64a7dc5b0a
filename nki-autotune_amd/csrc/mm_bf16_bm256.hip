// Instances of mm_lhsT_rhs_bf16 with block_m = 256 (rows of the 72-point search grid).
#include "mi_registry.hpp"

namespace mi {
MI_GRID_BK_W_S(MI_MM_INST, 256, 64)
MI_GRID_BK_W_S(MI_MM_INST, 256, 128)
MI_GRID_BK_W_S(MI_MM_INST, 256, 256)

const MiEntry* table_mm_bm256(int* n) {
  static const MiEntry t[] = {
      MI_GRID_BK_W_S(MI_MM_ROW, 256, 64)
      MI_GRID_BK_W_S(MI_MM_ROW, 256, 128)
      MI_GRID_BK_W_S(MI_MM_ROW, 256, 256)
  };
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
