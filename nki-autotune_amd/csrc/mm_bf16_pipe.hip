// Instances of the software-pipelined lhsT.rhs matmul (matmul variant 1):
// 4-wave blocks with 128x128 (or 128x64, 64x64) per wave at one wave per
// SIMD, and 8-wave blocks at two waves per SIMD; 2 to 4 LDS stages.  The
// small-block, deep-pipeline rows serve the skinny HBM-bound shapes, which
// need many loads in flight per CU rather than MFMA throughput.  Every config
// is also instantiated as variant 3, which loads rhs non-temporally.
#include "mi_registry.hpp"

#define MI_PIPE_CONFIGS(X)   \
  X(256, 256, 64, 4, 2)      \
  X(256, 256, 32, 4, 2)      \
  X(256, 256, 32, 4, 3)      \
  X(256, 256, 32, 4, 4)      \
  X(256, 256, 64, 8, 2)      \
  X(256, 256, 32, 8, 3)      \
  X(128, 512, 32, 8, 3)      \
  X(256, 128, 64, 4, 2)      \
  X(256, 128, 64, 4, 3)      \
  X(128, 256, 64, 4, 2)      \
  X(128, 256, 64, 4, 3)      \
  X(128, 256, 32, 4, 3)      \
  X(128, 256, 32, 4, 4)      \
  X(256, 128, 32, 4, 3)      \
  X(256, 128, 32, 4, 4)      \
  X(256, 128, 64, 8, 2)      \
  X(256, 128, 64, 8, 3)      \
  X(128, 128, 64, 4, 2)      \
  X(128, 128, 64, 4, 3)      \
  X(128, 128, 64, 4, 4)      \
  X(128, 128, 32, 4, 4)      \
  X(128, 64, 64, 4, 4)       \
  X(64, 128, 64, 4, 4)       \
  X(64, 256, 64, 4, 3)       \
  X(32, 256, 64, 4, 4)       \
  X(32, 128, 64, 4, 4)       \
  X(32, 128, 128, 4, 3)      \
  X(64, 64, 64, 4, 4)        \
  X(64, 128, 128, 4, 3)

namespace mi {
MI_PIPE_CONFIGS(MI_MMP_INST)
MI_PIPE_CONFIGS(MI_MMPN_INST)

const MiEntry* table_mm_pipe(int* n) {
  static const MiEntry t[] = {MI_PIPE_CONFIGS(MI_MMP_ROW) MI_PIPE_CONFIGS(MI_MMPN_ROW)};
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
