// Instances of the ring-pipelined fused rmsnorm_matmul: variant 2 (1/rms on
// the accumulators in the epilogue) and variant 3 (1/rms prologue, rows
// scaled before they reach LDS).
#include "mi_registry.hpp"

#define MI_RMS_RING_CONFIGS(X, PRE) \
  X(256, 256, 32, 4, PRE)           \
  X(256, 256, 32, 8, PRE)           \
  X(128, 256, 64, 4, PRE)           \
  X(128, 256, 64, 8, PRE)           \
  X(256, 128, 32, 4, PRE)           \
  X(256, 128, 32, 8, PRE)           \
  X(128, 256, 32, 8, PRE)           \
  X(128, 128, 64, 4, PRE)

namespace mi {
MI_RMS_RING_CONFIGS(MI_RMSR_INST, 0)
MI_RMS_RING_CONFIGS(MI_RMSR_INST, 1)

const MiEntry* table_rms_pipe(int* n) {
  static const MiEntry t[] = {MI_RMS_RING_CONFIGS(MI_RMSR_ROW, 0) MI_RMS_RING_CONFIGS(MI_RMSR_ROW, 1)};
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
