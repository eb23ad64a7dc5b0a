// mi_capi_internal.hpp -- pieces of the C ABI implementation (mi_capi.hip)
// shared with the other translation units of libmi_kernels.so.
#pragma once
#include <stddef.h>

#include "mi_registry.hpp"

namespace mi {
namespace capi {

// Records the message of a failure for mi_last_error on this thread and
// returns `code`.
int fail(int code, const char* fmt, ...);

// The body of mi_matmul_lhsT_rhs_bf16.  fixed_ws == NULL: a call that needs
// device workspace takes it from the library's stream-ordered pool;
// otherwise fixed_ws (fixed_cap bytes, 256-byte aligned) is the workspace
// and a config needing more is rejected with MI_E_RANGE.
int matmul_lhsT_rhs_bf16(const void* lhsT, const void* rhs, void* out, int M, int N, int K, const mi_tile_cfg* cfg,
                         void* stream, char* fixed_ws, size_t fixed_cap);

}  // namespace capi
}  // namespace mi
