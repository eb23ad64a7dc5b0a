// Instances of the fused rmsnorm_matmul with the x operand loaded straight
// into MFMA registers (rmsnorm_matmul variants 6..9): variant = 6 + (D-2) +
// 2 * (wave grid transposed from the squarest one), D = x tiles in flight.
#include "mi_registry.hpp"

#define MI_RMS_DIRECT_CONFIGS(X)    \
  X(256, 256, 32, 8, 3, 0, 2, 6)    \
  X(256, 256, 32, 8, 2, 0, 2, 6)    \
  X(256, 256, 32, 8, 4, 0, 2, 6)    \
  X(256, 256, 32, 8, 3, 4, 2, 8)    \
  X(256, 256, 32, 8, 3, 4, 3, 9)    \
  X(256, 256, 32, 8, 2, 4, 3, 9)    \
  X(256, 256, 32, 4, 3, 0, 2, 6)    \
  X(256, 256, 32, 4, 3, 0, 3, 7)    \
  X(256, 128, 32, 8, 3, 0, 2, 6)    \
  X(256, 128, 32, 8, 3, 0, 3, 7)    \
  X(128, 256, 32, 8, 3, 0, 2, 6)    \
  X(128, 256, 32, 8, 3, 0, 3, 7)    \
  X(128, 128, 64, 4, 2, 0, 2, 6)

namespace mi {
MI_RMS_DIRECT_CONFIGS(MI_RMSD_INST)

const MiEntry* table_rms_direct(int* n) {
  static const MiEntry t[] = {MI_RMS_DIRECT_CONFIGS(MI_RMSD_ROW)};
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
