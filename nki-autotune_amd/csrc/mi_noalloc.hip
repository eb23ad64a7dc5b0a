// mi_noalloc.hip -- mi_matmul_lhsT_rhs_bf16_noalloc: the lhsT.rhs product
// without any device allocation, for callers that cannot allocate (code
// under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).
//
// The only launches of that product that need memory beyond their inputs
// and output are the split-K ones (split_k > 1): their parts write fp32
// partial products [split_k][M][N] that a second kernel sums.  Here that
// workspace is `scratch`, a file-scope device array of kScratchBytes that
// every GPU the library runs on holds until the process ends.  Its device
// address on the current GPU is looked up once per device, on the first
// call there, and kept; host code passes that address, never the array's
// name (a host-side stand-in), to the kernels.
//
// The parts overwrite every element of their slices before the summing
// kernel reads them, so nothing in the scratch needs clearing between
// calls.  All calls on one GPU share its scratch: calls ordered on one
// stream are safe, calls that overlap on one GPU (different streams, no
// ordering between them) race.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>

#include "mi_capi_internal.hpp"

namespace {

constexpr size_t kScratchBytes = (size_t)MI_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kScratchBytes];

std::mutex g_scratch_mu;
std::map<int, char*> g_scratch_ptr;  // device ordinal -> device address of `scratch`

int scratch_address(char** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return mi::capi::fail(-(int)e, "hipGetDevice: %s", hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  auto it = g_scratch_ptr.find(dev);
  if (it == g_scratch_ptr.end()) {
    char* p = nullptr;
    e = hipGetSymbolAddress((void**)&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return mi::capi::fail(e != hipSuccess ? -(int)e : -(int)hipErrorInvalidSymbol,
                            "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    it = g_scratch_ptr.emplace(dev, p).first;
  }
  *out = it->second;
  return MI_OK;
}

}  // namespace

extern "C" int mi_matmul_lhsT_rhs_bf16_noalloc(const void* lhsT, const void* rhs, void* out, int M, int N, int K,
                                               const mi_tile_cfg* cfg, void* stream) {
  char* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != MI_OK) return rc;
  return mi::capi::matmul_lhsT_rhs_bf16(lhsT, rhs, out, M, N, K, cfg, stream, ws, kScratchBytes);
}
