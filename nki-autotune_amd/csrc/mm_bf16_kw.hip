// Instances of the lhsT.rhs matmul with each K tile's 16-deep sub-steps
// split over the waves of a workgroup (matmul variant 4): every wave
// accumulates the whole block, so blocks are at most 128x128 (256 fp32
// accumulators per lane at one wave per SIMD).  They serve shapes with few
// output tiles and a long K, where a wave-grid split of a small block reads
// two to three times the LDS bytes per MFMA; 2-wave 128x128 blocks run two
// workgroups per CU.
#include "mi_registry.hpp"

#define MI_KW_CONFIGS(X)    \
  X(128, 128, 64, 4, 4)     \
  X(128, 128, 64, 4, 2)     \
  X(128, 128, 128, 4, 2)    \
  X(128, 128, 32, 2, 4)     \
  X(128, 128, 32, 2, 2)     \
  X(128, 128, 64, 2, 3)     \
  X(128, 128, 64, 2, 2)     \
  X(64, 128, 64, 4, 4)      \
  X(128, 64, 64, 4, 4)      \
  X(64, 128, 128, 4, 2)

namespace mi {
MI_KW_CONFIGS(MI_MMW_INST)

const MiEntry* table_mm_kw(int* n) {
  static const MiEntry t[] = {MI_KW_CONFIGS(MI_MMW_ROW)};
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
