// Instances of the fused rmsnorm_matmul with the x panel staged through
// registers on the pipelined matmul core (rmsnorm_matmul variants 4, 5:
// x register ring of 2 or 3 K tiles; 11, 12: the same with W read
// non-temporally).
#include "mi_registry.hpp"

#define MI_RMS_XREG_CONFIGS(X) \
  X(256, 256, 32, 8, 2, 2)     \
  X(256, 256, 32, 8, 3, 2)     \
  X(256, 256, 32, 8, 4, 2)     \
  X(256, 256, 32, 8, 2, 3)     \
  X(256, 256, 32, 8, 3, 3)     \
  X(256, 256, 32, 4, 3, 2)     \
  X(256, 256, 32, 4, 3, 3)     \
  X(256, 256, 64, 4, 2, 2)     \
  X(128, 256, 32, 4, 3, 3)     \
  X(128, 256, 64, 4, 2, 2)     \
  X(256, 128, 32, 8, 3, 3)     \
  X(256, 128, 64, 8, 2, 2)     \
  X(128, 128, 64, 4, 2, 2)     \
  X(128, 512, 32, 8, 3, 2)     \
  X(128, 512, 32, 8, 3, 3)     \
  X(128, 512, 32, 8, 2, 2)     \
  X(128, 512, 32, 4, 3, 3)

// W read non-temporally (variants 11 / 12), for skinny M where W is
// streamed once: block_n 128 for enough workgroups, small block_m.
#define MI_RMS_XREG_NT_CONFIGS(X) \
  X(32, 128, 64, 4, 2, 2)         \
  X(32, 128, 64, 4, 3, 2)         \
  X(32, 128, 64, 4, 4, 2)         \
  X(32, 128, 128, 4, 2, 2)        \
  X(32, 128, 128, 4, 3, 2)        \
  X(64, 128, 128, 4, 2, 2)        \
  X(64, 128, 64, 4, 2, 2)         \
  X(64, 128, 64, 4, 3, 2)         \
  X(128, 128, 64, 4, 3, 2)        \
  X(64, 128, 32, 4, 3, 2)         \
  X(128, 128, 64, 4, 2, 2)        \
  X(128, 128, 32, 4, 3, 2)        \
  X(128, 128, 32, 4, 3, 3)        \
  X(256, 128, 32, 8, 3, 3)

namespace mi {
MI_RMS_XREG_CONFIGS(MI_RMSX_INST)
MI_RMS_XREG_NT_CONFIGS(MI_RMSXN_INST)

const MiEntry* table_rms_xreg(int* n) {
  static const MiEntry t[] = {MI_RMS_XREG_CONFIGS(MI_RMSX_ROW) MI_RMS_XREG_NT_CONFIGS(MI_RMSXN_ROW)};
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
