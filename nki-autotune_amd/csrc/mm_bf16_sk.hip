// Instances of the stream-K lhsT.rhs matmul: variant 5 (rhs cached) and
// variant 6 (rhs non-temporal).  One workgroup per CU takes an equal share
// of every tile's K loop, so shapes with fewer output tiles than CUs (the
// skinny decode shapes: 224 tiles of 128 columns at N = 28672; the short,
// wide C4a output with 128x128 blocks) keep every CU busy.  The configs are
// the pipelined core's skinny and 128x128 blocks (larger blocks spill
// registers in the combine).
#include "mi_registry.hpp"

#define MI_SK_CONFIGS(X) \
  X(32, 128, 128, 4, 3)  \
  X(32, 128, 64, 4, 4)   \
  X(32, 256, 64, 4, 4)   \
  X(64, 128, 64, 4, 4)   \
  X(64, 128, 128, 4, 3)  \
  X(64, 256, 64, 4, 3)   \
  X(128, 128, 64, 4, 3)  \
  X(128, 128, 64, 4, 4)

namespace mi {
MI_SK_CONFIGS(MI_MMS_INST)
MI_SK_CONFIGS(MI_MMSN_INST)

const MiEntry* table_mm_sk(int* n) {
  static const MiEntry t[] = {MI_SK_CONFIGS(MI_MMS_ROW) MI_SK_CONFIGS(MI_MMSN_ROW)};
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
