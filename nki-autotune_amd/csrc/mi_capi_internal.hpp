// mi_capi_internal.hpp -- pieces of the C ABI implementation (mi_capi.hip)
// shared with the other translation units of libmi_kernels.so.
#pragma once
#include <stddef.h>

#include "mi_registry.hpp"

namespace mi {
namespace capi {

// Limits of a call: split-K parts, and bytes of device workspace.
constexpr int kMaxSplit = 16;
constexpr unsigned long long kMaxWorkspace = 1ull << 31;

// Records the message of a failure for mi_last_error on this thread and
// returns `code`.
int fail(int code, const char* fmt, ...);

// The prebuilt instance of `kernel_id` for cfg's tile parameters and
// variant (split_k and group_m aside), or NULL.
const MiEntry* find(int kernel_id, const mi_tile_cfg& cfg);

// Compute units of the current device (the stream-K grid); kDefaultCus,
// MI355X's count, when no device is visible.
constexpr int kDefaultCus = 256;
int device_cus();

// Whether `variant` of `kernel_id` takes split_k > 1.
bool splittable(int kernel_id, int variant);

// The library default config at a shape (mi_default_config without its
// argument checks; mi_defaults.hip).
int pick_default(int kernel_id, int M, int N, int K, mi_tile_cfg* cfg);
// The fused kernel's default for a call without gamma (mi_defaults.hip).
int pick_default_no_gamma(int M, int N, int K, mi_tile_cfg* cfg);

// The body of mi_matmul_lhsT_rhs_bf16.  fixed_ws == NULL: a call that needs
// device workspace takes it from the library's stream-ordered pool;
// otherwise fixed_ws (fixed_cap bytes, 256-byte aligned) is the workspace
// and a config needing more is rejected with MI_E_RANGE.
int matmul_lhsT_rhs_bf16(const void* lhsT, const void* rhs, void* out, int M, int N, int K, const mi_tile_cfg* cfg,
                         void* stream, char* fixed_ws, size_t fixed_cap);

}  // namespace capi
}  // namespace mi
