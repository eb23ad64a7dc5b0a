// Instances of matmul_lhs_rhs (out = lhs[M,K] . rhs[K,N], lhs K-contiguous)
// on the software-pipelined core.  Variant 0: the same tile configs as the
// lhsT.rhs kernel, the A panel K-contiguous in LDS and read without a
// transpose.  Variant 1: A loaded two K tiles at a time (whole 128-byte
// lines) into pair buffers; B keeps its per-tile ring.  Variant 2: variant
// 0 with rhs read non-temporally, for skinny M where rhs is streamed once.
#include "mi_registry.hpp"

#define MI_LHS_CONFIGS(X)   \
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

#define MI_LHS_PAIR_CONFIGS(X) \
  X(256, 256, 32, 4, 3)        \
  X(256, 256, 32, 4, 4)        \
  X(256, 256, 32, 8, 3)        \
  X(256, 256, 32, 4, 2)        \
  X(256, 256, 32, 8, 2)        \
  X(128, 512, 32, 8, 3)        \
  X(256, 128, 32, 8, 3)        \
  X(128, 256, 32, 4, 3)        \
  X(128, 256, 64, 4, 2)        \
  X(128, 128, 64, 4, 3)        \
  X(128, 128, 32, 4, 4)

#define MI_LHS_SKINNY_CONFIGS(X) \
  X(32, 128, 128, 4, 3)          \
  X(32, 256, 64, 4, 4)           \
  X(64, 128, 64, 4, 4)           \
  X(64, 128, 128, 4, 3)          \
  X(128, 128, 64, 4, 3)          \
  X(256, 128, 64, 8, 3)

namespace mi {
MI_LHS_CONFIGS(MI_MMK_INST)
MI_LHS_PAIR_CONFIGS(MI_MMKP_INST)
MI_LHS_SKINNY_CONFIGS(MI_MMKN_INST)

const MiEntry* table_mm_lhs(int* n) {
  static const MiEntry t[] = {MI_LHS_CONFIGS(MI_MMK_ROW) MI_LHS_PAIR_CONFIGS(MI_MMKP_ROW)
                              MI_LHS_SKINNY_CONFIGS(MI_MMKN_ROW)};
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
