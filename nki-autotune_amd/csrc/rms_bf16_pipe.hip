// Instances of the software-pipelined fused rmsnorm_matmul: variant 2
// (1/rms on the accumulators in the epilogue) and variant 3 (1/rms prologue,
// rows scaled before they reach LDS).
#include "mi_registry.hpp"

#define MI_RMS_PIPE_CONFIGS(X, PRE) \
  X(256, 256, 64, 4, 2, PRE)        \
  X(256, 256, 32, 4, 3, PRE)        \
  X(256, 256, 64, 8, 2, PRE)        \
  X(256, 256, 32, 8, 3, PRE)        \
  X(256, 128, 64, 4, 2, PRE)        \
  X(128, 256, 64, 4, 2, PRE)        \
  X(256, 128, 64, 8, 2, PRE)        \
  X(128, 128, 64, 4, 2, PRE)        \
  X(128, 128, 64, 4, 3, PRE)

namespace mi {
MI_RMS_PIPE_CONFIGS(MI_RMSP_INST, 0)
MI_RMS_PIPE_CONFIGS(MI_RMSP_INST, 1)

const MiEntry* table_rms_pipe(int* n) {
  static const MiEntry t[] = {MI_RMS_PIPE_CONFIGS(MI_RMSP_ROW, 0) MI_RMS_PIPE_CONFIGS(MI_RMSP_ROW, 1)};
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
