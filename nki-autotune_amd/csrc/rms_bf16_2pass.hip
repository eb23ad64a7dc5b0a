// Instances of the two-pass fused rmsnorm_matmul (variant 13): the main
// pass is the pipelined lhsT.rhs core, so its configs are that kernel's
// square- and mid-shape configs.  Variant 15: the main pass on the
// paired-load K-contiguous core, at that core's configs
// (matmul_lhs_rhs variant 1).
#include "mi_registry.hpp"

#define MI_RMS_2PASS_CONFIGS(X) \
  X(256, 256, 64, 4, 2)         \
  X(256, 256, 32, 4, 2)         \
  X(256, 256, 32, 4, 3)         \
  X(256, 256, 32, 4, 4)         \
  X(256, 256, 32, 8, 3)         \
  X(128, 512, 32, 8, 3)         \
  X(256, 128, 64, 4, 3)         \
  X(128, 256, 64, 4, 3)         \
  X(128, 128, 64, 4, 2)         \
  X(128, 128, 64, 4, 3)         \
  X(64, 128, 64, 4, 4)          \
  X(64, 64, 64, 4, 4)

#define MI_RMS_2PASS_PAIR_CONFIGS(X) \
  X(256, 256, 32, 4, 3)              \
  X(256, 256, 32, 8, 3)              \
  X(128, 512, 32, 8, 3)              \
  X(256, 128, 32, 8, 3)              \
  X(128, 256, 32, 4, 3)              \
  X(128, 128, 32, 4, 4)

namespace mi {
MI_RMS_2PASS_CONFIGS(MI_RMS2_INST)
MI_RMS_2PASS_PAIR_CONFIGS(MI_RMS2P_INST)

const MiEntry* table_rms_2pass(int* n) {
  static const MiEntry t[] = {MI_RMS_2PASS_CONFIGS(MI_RMS2_ROW) MI_RMS_2PASS_PAIR_CONFIGS(MI_RMS2P_ROW)};
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
