// Instances of the fused rmsnorm_matmul whose x loads fetch two K tiles
// (128-byte row segments) per instruction (rmsnorm_matmul variant 10).
#include "mi_registry.hpp"

#define MI_RMS_XPAIR_CONFIGS(X) \
  X(256, 256, 32, 8, 3)         \
  X(256, 128, 32, 8, 3)         \
  X(128, 256, 32, 4, 3)         \
  X(128, 256, 32, 8, 3)         \
  X(128, 128, 32, 4, 3)         \
  X(128, 512, 32, 8, 3)

namespace mi {
MI_RMS_XPAIR_CONFIGS(MI_RMSP_INST)

const MiEntry* table_rms_xpair(int* n) {
  static const MiEntry t[] = {MI_RMS_XPAIR_CONFIGS(MI_RMSP_ROW)};
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
