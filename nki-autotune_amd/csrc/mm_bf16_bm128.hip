// Instances of mm_lhsT_rhs_bf16 with block_m = 128 (rows of the 72-point search grid).
#include "mi_registry.hpp"

namespace mi {
MI_GRID_BK_W_S(MI_MM_INST, 128, 64)
MI_GRID_BK_W_S(MI_MM_INST, 128, 128)
MI_GRID_BK_W_S(MI_MM_INST, 128, 256)

const MiEntry* table_mm_bm128(int* n) {
  static const MiEntry t[] = {
      MI_GRID_BK_W_S(MI_MM_ROW, 128, 64)
      MI_GRID_BK_W_S(MI_MM_ROW, 128, 128)
      MI_GRID_BK_W_S(MI_MM_ROW, 128, 256)
  };
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
