// Instances of rmsnorm_matmul variant 14: the fused kernel without gamma on
// the K-contiguous pipelined core, the rows' sums of squares taken from its
// A fragments (mi_gemm.hpp, rmsnorm_mm_bf16_sq_kernel).  The tile configs
// of matmul_lhs_rhs variant 0 that suit square and tall shapes; 256x256
// blocks take 8 waves (with 4, a wave's 128x128 block and its share of the
// squares spill registers).  Variant 16: the same on the paired-load core
// of matmul_lhs_rhs variant 1 (mi_mm_lhs_pair.hpp,
// rmsnorm_mm_bf16_sq_pair_kernel), at that variant's configs.
#include "mi_registry.hpp"

#define MI_RMSQ_CONFIGS(X) \
  X(256, 256, 64, 8, 2)     \
  X(256, 256, 32, 8, 3)     \
  X(128, 512, 32, 8, 3)     \
  X(256, 128, 64, 4, 2)     \
  X(256, 128, 64, 4, 3)     \
  X(128, 256, 64, 4, 2)     \
  X(128, 256, 64, 4, 3)     \
  X(256, 128, 64, 8, 3)     \
  X(128, 128, 64, 4, 2)     \
  X(128, 128, 64, 4, 3)     \
  X(128, 128, 64, 4, 4)     \
  X(64, 128, 64, 4, 4)      \
  X(64, 64, 64, 4, 4)

#define MI_RMSQP_CONFIGS(X) \
  X(256, 256, 32, 8, 3)      \
  X(256, 256, 32, 8, 2)      \
  X(128, 512, 32, 8, 3)      \
  X(256, 128, 32, 8, 3)      \
  X(128, 256, 32, 4, 3)      \
  X(128, 256, 64, 4, 2)      \
  X(128, 128, 64, 4, 3)      \
  X(128, 128, 32, 4, 4)

namespace mi {
MI_RMSQ_CONFIGS(MI_RMSQ_INST)
MI_RMSQP_CONFIGS(MI_RMSQP_INST)

const MiEntry* table_rms_sq(int* n) {
  static const MiEntry t[] = {MI_RMSQ_CONFIGS(MI_RMSQ_ROW) MI_RMSQP_CONFIGS(MI_RMSQP_ROW)};
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace mi
