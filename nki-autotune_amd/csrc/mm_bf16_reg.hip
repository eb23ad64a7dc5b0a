// Instances of the register-ring lhsT.rhs matmul (matmul variant 2) for the
// skinny HBM-bound shapes: small block_m, ring depth (lds_stages) 2..6.
#include "mi_registry.hpp"

#define MI_REG_CONFIGS(X) \
  X(128, 128, 64, 4, 4)   \
  X(128, 128, 64, 8, 4)   \
  X(128, 128, 64, 8, 6)   \
  X(128, 64, 64, 4, 4)    \
  X(128, 64, 64, 4, 6)    \
  X(64, 128, 64, 4, 4)    \
  X(64, 128, 64, 4, 6)    \
  X(64, 256, 64, 8, 4)    \
  X(32, 128, 64, 4, 4)    \
  X(32, 128, 64, 4, 8)    \
  X(32, 256, 64, 4, 4)    \
  X(32, 256, 64, 4, 6)

namespace mi {
MI_REG_CONFIGS(MI_MMR_INST)

const MiEntry* table_mm_reg(int* n) {
  static const MiEntry t[] = {MI_REG_CONFIGS(MI_MMR_ROW)};
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
