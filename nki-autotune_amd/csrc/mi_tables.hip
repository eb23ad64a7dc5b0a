// mi_tables.hip -- the instance tables served by libmi_kernels.so: every
// prebuilt tile config of the four kernel families.
#include "mi_registry.hpp"

namespace mi {
const TableFn* table_list(int* n) {
  static const TableFn tables[] = {table_mm_bm32,   table_mm_bm64,  table_mm_bm128,  table_mm_bm256, table_mm_pipe,
                                   table_mm_sk,     table_mm_kw,    table_mm_reg,    table_mm_lhs,   table_rms_bm64,
                                   table_rms_bm128, table_rms_bm256, table_rms_xreg, table_rms_2pass, table_rms_sq,
                                   table_f32};
  *n = (int)(sizeof(tables) / sizeof(tables[0]));
  return tables;
}
}  // namespace mi
