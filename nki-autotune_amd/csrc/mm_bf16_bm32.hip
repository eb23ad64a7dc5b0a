// Instances of mm_lhsT_rhs_bf16 with block_m = 32: the skinny, HBM-bound
// shapes (M <= 32 rows of output) stream rhs with deep K panels.
#include "mi_registry.hpp"

namespace mi {
MI_MM_INST(32, 128, 64, 4, 2)
MI_MM_INST(32, 128, 128, 4, 2)
MI_MM_INST(32, 256, 64, 4, 2)
MI_MM_INST(32, 256, 128, 4, 2)
MI_MM_INST(32, 256, 64, 8, 2)
MI_MM_INST(32, 256, 128, 8, 2)

const MiEntry* table_mm_bm32(int* n) {
  static const MiEntry t[] = {
      MI_MM_ROW(32, 128, 64, 4, 2)
      MI_MM_ROW(32, 128, 128, 4, 2)
      MI_MM_ROW(32, 256, 64, 4, 2)
      MI_MM_ROW(32, 256, 128, 4, 2)
      MI_MM_ROW(32, 256, 64, 8, 2)
      MI_MM_ROW(32, 256, 128, 8, 2)
  };
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
