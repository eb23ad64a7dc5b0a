// mi_capi.hip -- the C ABI declared in include/mi_kernels.h.
//
// Launchers over the instance table: look the config up, check its static
// legality for the shape, launch on the caller's stream.  The only state is
// the instance table and, for calls that need device workspace (split-K,
// the two-pass fused kernel), a memory pool per device from which each such
// call takes its workspace stream-ordered.  No entry point throws; failures
// are return codes plus a thread-local message (mi_last_error).
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "mi_capi_internal.hpp"

namespace mi {
namespace capi {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace capi
}  // namespace mi

namespace {

using mi::capi::fail;
using mi::capi::g_err;

int hip_fail(hipError_t e, const char* what) {
  snprintf(g_err, sizeof(g_err), "%s: %s", what, hipGetErrorString(e));
  return -(int)e;
}

const std::vector<mi::MiEntry>& registry() {
  static std::vector<mi::MiEntry> all;
  static std::once_flag once;
  std::call_once(once, [] {
    int ntables = 0;
    const mi::TableFn* tables = mi::table_list(&ntables);
    for (int i = 0; i < ntables; ++i) {
      int n = 0;
      const mi::MiEntry* t = tables[i](&n);
      all.insert(all.end(), t, t + n);
    }
  });
  return all;
}

bool same_instance(const mi_tile_cfg& a, const mi_tile_cfg& b) {
  return a.block_m == b.block_m && a.block_n == b.block_n && a.block_k == b.block_k && a.waves == b.waves &&
         a.lds_stages == b.lds_stages && a.variant == b.variant;
}

}  // namespace

namespace mi {
namespace capi {

const MiEntry* find(int kernel_id, const mi_tile_cfg& cfg) {
  for (const MiEntry& e : registry())
    if (e.kernel_id == kernel_id && same_instance(e.cfg, cfg)) return &e;
  return nullptr;
}

int device_cus() {
  static std::mutex mu;
  static std::map<int, int> cus;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();  // no device (a CPU-only host): leave no error behind for a later launch check
    return kDefaultCus;
  }
  std::lock_guard<std::mutex> lock(mu);
  auto it = cus.find(dev);
  if (it == cus.end()) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
      (void)hipGetLastError();
      n = kDefaultCus;
    }
    it = cus.emplace(dev, n).first;
  }
  return it->second;
}

bool splittable(int kernel_id, int variant) {
  return (kernel_id == MI_KERNEL_MATMUL_LHST_RHS_BF16 && (variant == 1 || variant == 3 || variant == 4)) ||
         (kernel_id == MI_KERNEL_MATMUL_LHS_RHS_BF16 && (variant == 0 || variant == 2)) ||
         (kernel_id == MI_KERNEL_RMSNORM_MATMUL_BF16 &&
          (variant == 4 || variant == 5 || variant == 11 || variant == 12 || variant == 13));
}

}  // namespace capi
}  // namespace mi

namespace {

using mi::capi::find;
using mi::capi::kMaxSplit;
using mi::capi::kMaxWorkspace;
using mi::capi::pick_default;
using mi::capi::splittable;

constexpr unsigned long long kMaxOffset = 0xFFFFFFFFull;        // 32-bit buffer offsets

// The template rules of the variant `c` names (mi_legal.hpp: the same
// predicates the kernel templates assert when they are instantiated).
mi::Legal template_legal(int kernel_id, const mi_tile_cfg& c) {
  const int bm = c.block_m, bn = c.block_n, bk = c.block_k, w = c.waves, s = c.lds_stages;
  switch (kernel_id) {
    case MI_KERNEL_MATMUL_LHST_RHS_BF16:
      if (c.variant == 0) return mi::legal_mm_plain(bm, bn, bk, w, s);
      if (c.variant == 1 || c.variant == 3) return mi::legal_mm_pipe(bm, bn, bk, w, s, false);
      if (c.variant == 2) return mi::legal_mm_reg(bm, bn, bk, w, s);
      if (c.variant == 4) return mi::legal_mm_kw(bm, bn, bk, w, s);
      if (c.variant == 5 || c.variant == 6) return mi::legal_mm_pipe(bm, bn, bk, w, s, false);
      break;
    case MI_KERNEL_MATMUL_LHS_RHS_BF16:
      if (c.variant == 0 || c.variant == 2) return mi::legal_mm_pipe(bm, bn, bk, w, s, true);
      if (c.variant == 1) return mi::legal_lhs_pair(bm, bn, bk, w, s);
      break;
    case MI_KERNEL_RMSNORM_MATMUL_BF16:
      if (c.variant == 0 || c.variant == 1) return mi::legal_rms_plain(bm, bn, bk, w, s);
      if (c.variant == 4 || c.variant == 5) return mi::legal_rms_xreg(bm, bn, bk, w, s, c.variant - 2);
      if (c.variant == 11 || c.variant == 12) return mi::legal_rms_xreg(bm, bn, bk, w, s, c.variant - 9);
      if (c.variant == 13) return mi::legal_rms2(bm, bn, bk, w, s);
      if (c.variant == 15) return mi::legal_rms2_pair(bm, bn, bk, w, s);
      if (c.variant == 14) return mi::legal_mm_pipe(bm, bn, bk, w, s, true);
      if (c.variant == 16) return mi::legal_lhs_pair(bm, bn, bk, w, s);
      break;
    case MI_KERNEL_MATMUL_LHST_RHS_F32:
      // 16 x 16 threads with 4 x 4 outputs each, K slices of 16 or 32.
      if (c.variant == 0) {
        if (bm != 64 || bn != 64 || (bk != 16 && bk != 32) || w != 4 || s != 1)
          return mi::bad(MI_E_TILE, "the fp32 kernel takes 64x64 blocks, block_k 16 or 32, 4 waves, 1 stage");
        return mi::ok();
      }
      if (c.variant == 1) {
        if ((bm != 64 && bm != 128) || bn != bm || bk != 16 || w != 4 || s != 1)
          return mi::bad(MI_E_TILE, "the fp32 MFMA kernel takes 64x64 or 128x128 blocks, block_k 16, 4 waves, 1 stage");
        return mi::ok();
      }
      break;
    default:
      break;
  }
  return mi::bad(MI_E_TILE, "no such variant of this kernel");
}

int check(int kernel_id, const mi_tile_cfg* cfg, int M, int N, int K, const mi::MiEntry** out) {
  if (kernel_id < 0 || kernel_id >= MI_NUM_KERNELS) return fail(MI_E_KERNEL, "unknown kernel id %d", kernel_id);
  if (!cfg) return fail(MI_E_ARGS, "null config");
  if (M < 0 || N < 0 || K < 0) return fail(MI_E_ARGS, "negative size M=%d N=%d K=%d", M, N, K);
  const mi_tile_cfg& c = *cfg;
  if (c.block_m <= 0 || c.block_n <= 0 || c.block_k <= 0 || c.waves <= 0 || c.lds_stages <= 0)
    return fail(MI_E_ARGS, "non-positive tile parameter");
  if (c.split_k < 1 || c.split_k > kMaxSplit)
    return fail(MI_E_SPLIT, "split_k=%d outside [1, %d]", c.split_k, kMaxSplit);
  if (c.split_k > 1) {
    if (!splittable(kernel_id, c.variant))
      return fail(MI_E_SPLIT,
                  "split_k=%d needs the pipelined matmul (lhsT.rhs variants 1, 3; lhs.rhs variants 0, 2) or a "
                  "register-staged or two-pass fused kernel (rmsnorm_matmul variants 4, 5, 11, 12, 13)",
                  c.split_k);
    // Every part must get at least one K tile.
    const long long kt = ((long long)K + c.block_k - 1) / c.block_k;
    const long long kts = (kt + c.split_k - 1) / c.split_k;
    if ((long long)(c.split_k - 1) * kts >= kt)
      return fail(MI_E_SPLIT, "split_k=%d leaves a K part empty at K=%d, block_k=%d", c.split_k, K, c.block_k);
  }
  if (c.group_m < 0) return fail(MI_E_ARGS, "group_m=%d negative", c.group_m);
  const mi::Legal lg = template_legal(kernel_id, c);
  if (lg.code != MI_OK)
    return fail(lg.code, "kernel %d variant %d bm=%d bn=%d bk=%d waves=%d stages=%d: %s", kernel_id, c.variant,
                c.block_m, c.block_n, c.block_k, c.waves, c.lds_stages, lg.why);
  if (mi::is_streamk(kernel_id, c.variant) && mi::grid_tiles(M, N, c.block_m, c.block_n) > mi::kSkMaxTiles)
    return fail(MI_E_RANGE, "stream-K takes at most %d output tiles (%d x %d blocks at M=%d N=%d)", mi::kSkMaxTiles,
                c.block_m, c.block_n, M, N);
  const size_t ws = mi::workspace_bytes(kernel_id, c, M, N, K, mi::capi::device_cus());
  if (ws > kMaxWorkspace) return fail(MI_E_RANGE, "device workspace of %zu bytes exceeds %llu", ws, kMaxWorkspace);
  const mi::MiEntry* e = find(kernel_id, c);
  if (!e)
    return fail(MI_E_NO_INSTANCE, "no compiled instance for kernel %d bm=%d bn=%d bk=%d waves=%d stages=%d variant=%d",
                kernel_id, c.block_m, c.block_n, c.block_k, c.waves, c.lds_stages, c.variant);
  if (e->lds_bytes > mi::kLdsBytesMax)
    return fail(MI_E_LDS, "instance LDS %d bytes > %d", e->lds_bytes, mi::kLdsBytesMax);
  if (kernel_id != MI_KERNEL_MATMUL_LHST_RHS_F32) {
    if (M % 8 || N % 8) return fail(MI_E_ALIGN, "M=%d and N=%d must be multiples of 8", M, N);
    const bool k_rows = kernel_id == MI_KERNEL_RMSNORM_MATMUL_BF16 || kernel_id == MI_KERNEL_MATMUL_LHS_RHS_BF16;
    if (k_rows && K % 8)
      return fail(MI_E_ALIGN, "K=%d must be a multiple of 8 (16-byte rows of the K-contiguous operand)", K);
    // Loads run up to one tile (the ring depth, for matmul variant 2) past K.
    const bool reg_ring = kernel_id == MI_KERNEL_MATMUL_LHST_RHS_BF16 && c.variant == 2;
    const unsigned long long kpad =
        (unsigned long long)K + (unsigned long long)c.block_k * (unsigned long long)(reg_ring ? c.lds_stages + 1 : 1);
    const unsigned long long mpad = (unsigned long long)M + (unsigned long long)c.block_m;
    // The A operand is MN-contiguous for lhsT.rhs and for the main pass of
    // the two-pass fused kernel (its packed xt[K][M]), K-contiguous
    // otherwise (x, lhs: loads run up to 8 tiles past K on the last rows).
    const bool a_mn = kernel_id == MI_KERNEL_MATMUL_LHST_RHS_BF16 ||
                      (kernel_id == MI_KERNEL_RMSNORM_MATMUL_BF16 && c.variant == 13);
    const unsigned long long a_span = a_mn ? kpad * (unsigned long long)M * 2ull
                                           : (mpad * (unsigned long long)K + 8ull * (unsigned long long)c.block_k) * 2ull;
    const unsigned long long b_span = kpad * (unsigned long long)N * 2ull;
    if (a_span > kMaxOffset || b_span > kMaxOffset)
      return fail(MI_E_RANGE, "operand spans exceed 32-bit buffer offsets (%llu, %llu bytes)", a_span, b_span);
    // The register-staged fused variants stage gamma in LDS (one K tile at a
    // time, K rounded up to it); with split_k > 1 each part stages the gamma
    // of its own K range: ceil(ceil(K/block_k)/split_k) tiles.  The limit
    // holds with or without gamma (legality is gamma-agnostic).
    if (e->gamma_kmax > 0) {
      const long long kt = ((long long)K + c.block_k - 1) / c.block_k;
      const long long need = (kt + c.split_k - 1) / c.split_k * c.block_k;
      if (need > e->gamma_kmax)
        return fail(MI_E_RANGE, "K=%d (%lld per part) exceeds the %d gamma entries variant %d stages in LDS", K,
                    need, e->gamma_kmax, c.variant);
    }
  }
  if (out) *out = e;
  g_err[0] = '\0';
  return MI_OK;
}

// An empty contraction (K = 0) leaves out = 0.  Written by a small kernel
// rather than hipMemsetAsync so that a caller may capture the call in a HIP
// graph (memset nodes have misbehaved on replay on this platform).
template <typename T>
__global__ void zero_fill_kernel(T* __restrict__ p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = T(0);
}

template <typename T>
int zero_output(void* out, size_t n, void* stream) {
  const size_t blocks = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
  hipLaunchKernelGGL(zero_fill_kernel<T>, dim3((unsigned)(blocks > 0 ? blocks : 1)), dim3(256), 0,
                     (hipStream_t)stream, (T*)out, n);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MI_OK : hip_fail(e, "zero fill");
}

// Device workspace (split-K partial products, the two-pass fused kernel's
// packed operand, stream-K partial tiles): from a memory pool the library
// keeps per device, stream-ordered (hipMallocFromPoolAsync / hipFreeAsync).
// Outside graph capture a workspace of at most kKeepBytes is a buffer kept
// per stream (run_kept below); otherwise each call allocates its own and
// frees it after its launches, and under HIP graph capture those become
// allocation and free nodes of the graph.  The runtime hands a freed
// buffer back to the pool at the pool's next allocation (measured: not at
// a synchronisation), and the pool's release threshold, kPoolKeepBytes,
// then returns what it holds beyond that to the device.
// mi_release_workspace returns all of it.
constexpr uint64_t kPoolKeepBytes = 256ull << 20;
std::mutex g_pool_mu;
std::map<int, hipMemPool_t> g_pools;

int workspace_pool(hipMemPool_t* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_pool_mu);
  auto it = g_pools.find(dev);
  if (it == g_pools.end()) {
    hipMemPoolProps props = {};
    props.allocType = hipMemAllocationTypePinned;
    props.handleTypes = hipMemHandleTypeNone;
    props.location.type = hipMemLocationTypeDevice;
    props.location.id = dev;
    hipMemPool_t pool = nullptr;
    if ((e = hipMemPoolCreate(&pool, &props)) != hipSuccess) return hip_fail(e, "workspace memory pool");
    uint64_t keep = kPoolKeepBytes;
    if ((e = hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep)) != hipSuccess)
      return hip_fail(e, "workspace memory pool threshold");
    it = g_pools.emplace(dev, pool).first;
  }
  *out = it->second;
  return MI_OK;
}

// Resolves the config (cfg == NULL: the library default) and checks it.
int resolve(int kernel_id, const mi_tile_cfg* cfg_in, const mi::MiArgs& a, mi_tile_cfg* cfg,
            const mi::MiEntry** e) {
  if (cfg_in) *cfg = *cfg_in;
  else pick_default(kernel_id, a.M, a.N, a.K, cfg);
  return check(kernel_id, cfg, a.M, a.N, a.K, e);
}

int launch(const mi::MiEntry* e, const mi_tile_cfg& cfg, const mi::MiArgs& args_in, char* ws, bool ws_zeroed,
           void* stream) {
  mi::MiArgs a = args_in;
  a.group_m = cfg.group_m > 0 ? cfg.group_m : 8;
  a.parts = cfg.split_k;
  a.ws = ws;
  a.ws_zeroed = ws_zeroed;
  const hipError_t err = e->launch(a, (hipStream_t)stream);
  return err == hipSuccess ? MI_OK : hip_fail(err, "kernel launch");
}

// A workspace of its own for one call, allocated and freed stream-ordered
// from the pool (under HIP graph capture these become allocation and free
// nodes of the graph).
int run_pooled(const mi::MiEntry* e, const mi_tile_cfg& cfg, const mi::MiArgs& a, size_t ws_bytes, hipMemPool_t pool,
               void* stream) {
  char* ws = nullptr;
  const hipError_t ae = hipMallocFromPoolAsync((void**)&ws, ws_bytes, pool, (hipStream_t)stream);
  if (ae != hipSuccess) return hip_fail(ae, "workspace alloc");
  const int lrc = launch(e, cfg, a, ws, false, stream);
  const hipError_t fe = hipFreeAsync(ws, (hipStream_t)stream);
  if (lrc != MI_OK) return lrc;
  if (fe != hipSuccess) return hip_fail(fe, "workspace free");
  return MI_OK;
}

// Kept workspaces: outside HIP graph capture, a call that needs at most
// kKeepBytes of workspace reuses a buffer the library keeps for its
// (device, stream), at most kKeepStreams streams per device; other
// streams' calls take a buffer of their own from the pool.  Calls on one
// stream run in stream order, so the buffer is free for the next call once
// the last one's kernels end, and a call that needs more frees it and
// allocates a larger one, both stream-ordered.  A stream that can be
// destroyed (any but the null and per-thread default streams) could leave
// kernels running on its buffer while a new stream gets the same handle,
// so its buffer carries an event recorded after each use, which the next
// call's stream waits for before touching the buffer (a wait costs nothing
// measurable; recording the event costs the GPU about 2.5 us per call).
// The default streams skip both.  This saves the pool allocation and free
// of every call (about 7 us of host time).  A kept buffer's stream-K
// counters (its first kSkCounterBytes) are zeroed by its first stream-K
// launch, and every stream-K launch leaves them 0, so later ones skip the
// zeroing.  Buffers stay with their stream until mi_release_workspace
// returns them all.
constexpr size_t kKeepBytes = 64ull << 20;
constexpr int kKeepStreams = 4;

struct KeptWs {
  int dev;
  hipStream_t stream;
  char* ptr;
  size_t bytes;
  hipEvent_t done;  // null for a default stream
  bool zeroed;
};
std::vector<KeptWs> g_kept;  // guarded by g_pool_mu

int run_kept(const mi::MiEntry* e, const mi_tile_cfg& cfg, const mi::MiArgs& a, size_t ws_bytes, int kernel_id,
             hipMemPool_t pool, int dev, void* stream_v) {
  hipStream_t stream = (hipStream_t)stream_v;
  std::unique_lock<std::mutex> lock(g_pool_mu);
  KeptWs* k = nullptr;
  int held = 0;
  for (KeptWs& x : g_kept) {
    if (x.dev != dev) continue;
    ++held;
    if (x.stream == stream) k = &x;
  }
  hipError_t err;
  if (!k) {
    if (held >= kKeepStreams) {
      lock.unlock();
      return run_pooled(e, cfg, a, ws_bytes, pool, stream);
    }
    hipEvent_t ev = nullptr;
    const bool permanent = stream == nullptr || stream == hipStreamPerThread;
    if (!permanent && (err = hipEventCreateWithFlags(&ev, hipEventDisableTiming)) != hipSuccess)
      return hip_fail(err, "workspace event");
    g_kept.push_back(KeptWs{dev, stream, nullptr, 0, ev, false});
    k = &g_kept.back();
  } else if (k->done && (err = hipStreamWaitEvent(stream, k->done, 0)) != hipSuccess) {
    return hip_fail(err, "workspace wait");
  }
  if (k->bytes < ws_bytes) {
    if (k->ptr && (err = hipFreeAsync(k->ptr, stream)) != hipSuccess) return hip_fail(err, "workspace free");
    k->ptr = nullptr;
    k->bytes = 0;
    // Round up (to 1 MiB, at least 1/4 more) so that growing shapes reallocate rarely.
    size_t want = ws_bytes + ws_bytes / 4;
    want = (want + (1u << 20) - 1) / (1u << 20) * (1u << 20);
    if (want > kKeepBytes) want = kKeepBytes;
    if ((err = hipMallocFromPoolAsync((void**)&k->ptr, want, pool, stream)) != hipSuccess) {
      k->ptr = nullptr;
      return hip_fail(err, "workspace alloc");
    }
    k->bytes = want;
    k->zeroed = false;
  }
  const int lrc = launch(e, cfg, a, k->ptr, k->zeroed, stream);
  if (lrc == MI_OK && mi::is_streamk(kernel_id, cfg.variant)) k->zeroed = true;
  if (k->done && (err = hipEventRecord(k->done, stream)) != hipSuccess && lrc == MI_OK)
    return hip_fail(err, "workspace event");
  return lrc;
}

// fixed_ws != NULL: the caller's device buffer of fixed_cap bytes serves as
// the workspace (nothing is allocated; a larger need is rejected); its
// stream-K counters must be 0 (a static array, zero when loaded; every
// stream-K launch leaves them 0).
int run(int kernel_id, const mi_tile_cfg* cfg_in, const mi::MiArgs& args_in, void* stream, char* fixed_ws = nullptr,
        size_t fixed_cap = 0) {
  mi_tile_cfg cfg;
  const mi::MiEntry* e = nullptr;
  int rc = resolve(kernel_id, cfg_in, args_in, &cfg, &e);
  if (rc != MI_OK) return rc;
  mi::MiArgs a = args_in;
  a.cus = mi::capi::device_cus();
  const size_t ws_bytes = mi::workspace_bytes(kernel_id, cfg, a.M, a.N, a.K, a.cus);
  if (ws_bytes == 0) return launch(e, cfg, a, nullptr, false, stream);
  if (fixed_ws) {
    if (ws_bytes > fixed_cap)
      return fail(MI_E_RANGE, "the config needs %zu bytes of workspace, over the %zu-byte static scratch", ws_bytes,
                  fixed_cap);
    return launch(e, cfg, a, fixed_ws, true, stream);
  }
  hipMemPool_t pool = nullptr;
  if ((rc = workspace_pool(&pool)) != MI_OK) return rc;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t err = hipStreamIsCapturing((hipStream_t)stream, &cap);
  if (err != hipSuccess) return hip_fail(err, "hipStreamIsCapturing");
  if (cap == hipStreamCaptureStatusNone && ws_bytes <= kKeepBytes) {
    int dev = 0;
    if ((err = hipGetDevice(&dev)) != hipSuccess) return hip_fail(err, "hipGetDevice");
    return run_kept(e, cfg, a, ws_bytes, kernel_id, pool, dev, stream);
  }
  // Under capture, or a large workspace: a buffer of its own.
  return run_pooled(e, cfg, a, ws_bytes, pool, stream);
}

// Device pointers are read and written in 16-byte vectors (bf16 kernels)
// or as fp32 elements (the fp32 kernel).
// [p, p + pb) and [q, q + qb) share a byte (null or empty ranges never do).
bool overlaps(const void* p, size_t pb, const void* q, size_t qb) {
  if (!p || !q || pb == 0 || qb == 0) return false;
  const uintptr_t a = (uintptr_t)p, b = (uintptr_t)q;
  return a < b + qb && b < a + pb;
}

bool misaligned(const void* p, uintptr_t align) { return p && ((uintptr_t)p & (align - 1)) != 0; }

}  // namespace

namespace mi {
namespace capi {

int matmul_lhsT_rhs_bf16(const void* lhsT, const void* rhs, void* out, int M, int N, int K, const mi_tile_cfg* cfg,
                         void* stream, char* fixed_ws, size_t fixed_cap) {
  if (M < 0 || N < 0 || K < 0) return fail(MI_E_ARGS, "negative size M=%d N=%d K=%d", M, N, K);
  if (M == 0 || N == 0) return MI_OK;
  if (!out) return fail(MI_E_ARGS, "null output pointer");
  if (K == 0) {
    return zero_output<uint16_t>(out, (size_t)M * N, stream);
  }
  if (!lhsT || !rhs) return fail(MI_E_ARGS, "null input pointer");
  if (misaligned(lhsT, 16) || misaligned(rhs, 16) || misaligned(out, 16))
    return fail(MI_E_ALIGN, "lhsT, rhs and out must be 16-byte aligned");
  const size_t ob = (size_t)M * N * 2;
  if (overlaps(out, ob, lhsT, (size_t)K * M * 2) || overlaps(out, ob, rhs, (size_t)K * N * 2))
    return fail(MI_E_ARGS, "out overlaps an input");
  mi::MiArgs a = {lhsT, rhs, nullptr, out, M, N, K, 0.0f, 0.0f, 8};
  return run(MI_KERNEL_MATMUL_LHST_RHS_BF16, cfg, a, stream, fixed_ws, fixed_cap);
}

}  // namespace capi
}  // namespace mi

extern "C" {

int mi_cfg_check(int kernel_id, const mi_tile_cfg* cfg, int M, int N, int K) {
  return check(kernel_id, cfg, M, N, K, nullptr);
}

int mi_num_configs(int kernel_id) {
  int n = 0;
  for (const mi::MiEntry& e : registry()) n += e.kernel_id == kernel_id;
  return n;
}

int mi_get_config(int kernel_id, int idx, mi_tile_cfg* cfg) {
  if (!cfg) return fail(MI_E_ARGS, "null config");
  int i = 0;
  for (const mi::MiEntry& e : registry()) {
    if (e.kernel_id != kernel_id) continue;
    if (i++ == idx) {
      *cfg = e.cfg;
      cfg->group_m = 8;
      return MI_OK;
    }
  }
  return fail(MI_E_ARGS, "config index %d out of range for kernel %d", idx, kernel_id);
}

int mi_default_config(int kernel_id, int M, int N, int K, mi_tile_cfg* cfg) {
  if (kernel_id < 0 || kernel_id >= MI_NUM_KERNELS) return fail(MI_E_KERNEL, "unknown kernel id %d", kernel_id);
  if (!cfg) return fail(MI_E_ARGS, "null config");
  if (M < 0 || N < 0 || K < 0) return fail(MI_E_ARGS, "negative size M=%d N=%d K=%d", M, N, K);
  return pick_default(kernel_id, M, N, K, cfg);
}

int mi_default_config_no_gamma(int M, int N, int K, mi_tile_cfg* cfg) {
  if (!cfg) return fail(MI_E_ARGS, "null config");
  if (M < 0 || N < 0 || K < 0) return fail(MI_E_ARGS, "negative size M=%d N=%d K=%d", M, N, K);
  return mi::capi::pick_default_no_gamma(M, N, K, cfg);
}

int mi_matmul_lhsT_rhs_bf16(const void* lhsT, const void* rhs, void* out, int M, int N, int K,
                            const mi_tile_cfg* cfg, void* stream) {
  return mi::capi::matmul_lhsT_rhs_bf16(lhsT, rhs, out, M, N, K, cfg, stream, nullptr, 0);
}

int mi_matmul_lhs_rhs_bf16(const void* lhs, const void* rhs, void* out, int M, int N, int K,
                           const mi_tile_cfg* cfg, void* stream) {
  if (M < 0 || N < 0 || K < 0) return fail(MI_E_ARGS, "negative size M=%d N=%d K=%d", M, N, K);
  if (M == 0 || N == 0) return MI_OK;
  if (!out) return fail(MI_E_ARGS, "null output pointer");
  if (K == 0) {
    return zero_output<uint16_t>(out, (size_t)M * N, stream);
  }
  if (!lhs || !rhs) return fail(MI_E_ARGS, "null input pointer");
  if (misaligned(lhs, 16) || misaligned(rhs, 16) || misaligned(out, 16))
    return fail(MI_E_ALIGN, "lhs, rhs and out must be 16-byte aligned");
  const size_t ob = (size_t)M * N * 2;
  if (overlaps(out, ob, lhs, (size_t)M * K * 2) || overlaps(out, ob, rhs, (size_t)K * N * 2))
    return fail(MI_E_ARGS, "out overlaps an input");
  mi::MiArgs a = {lhs, rhs, nullptr, out, M, N, K, 0.0f, 0.0f, 8};
  return run(MI_KERNEL_MATMUL_LHS_RHS_BF16, cfg, a, stream);
}

int mi_matmul_lhsT_rhs_f32(const float* lhsT, const float* rhs, float* out, int M, int N, int K,
                           const mi_tile_cfg* cfg, void* stream) {
  if (M < 0 || N < 0 || K < 0) return fail(MI_E_ARGS, "negative size M=%d N=%d K=%d", M, N, K);
  if (M == 0 || N == 0) return MI_OK;
  if (!out) return fail(MI_E_ARGS, "null output pointer");
  if (K == 0) {
    return zero_output<float>(out, (size_t)M * N, stream);
  }
  if (!lhsT || !rhs) return fail(MI_E_ARGS, "null input pointer");
  if (misaligned(lhsT, 4) || misaligned(rhs, 4) || misaligned(out, 4))
    return fail(MI_E_ALIGN, "lhsT, rhs and out must be 4-byte aligned");
  const size_t ob = (size_t)M * N * 4;
  if (overlaps(out, ob, lhsT, (size_t)K * M * 4) || overlaps(out, ob, rhs, (size_t)K * N * 4))
    return fail(MI_E_ARGS, "out overlaps an input");
  mi::MiArgs a = {lhsT, rhs, nullptr, out, M, N, K, 0.0f, 0.0f, 8};
  return run(MI_KERNEL_MATMUL_LHST_RHS_F32, cfg, a, stream);
}

int mi_rmsnorm_matmul_bf16(const void* x, const void* gamma, const void* W, void* out, int M, int N, int K,
                           float eps, const mi_tile_cfg* cfg, void* stream) {
  if (M < 0 || N < 0 || K <= 0) return fail(MI_E_ARGS, "bad size M=%d N=%d K=%d (K must be positive)", M, N, K);
  if (!(eps >= 0.0f) || eps > 3.0e38f) return fail(MI_E_ARGS, "eps must be finite and >= 0");
  if (M == 0 || N == 0) return MI_OK;
  if (!x || !W || !out) return fail(MI_E_ARGS, "null pointer");
  if (misaligned(x, 16) || misaligned(gamma, 16) || misaligned(W, 16) || misaligned(out, 16))
    return fail(MI_E_ALIGN, "x, gamma, W and out must be 16-byte aligned");
  const size_t ob = (size_t)M * N * 2;
  if (overlaps(out, ob, x, (size_t)M * K * 2) || overlaps(out, ob, W, (size_t)K * N * 2) ||
      overlaps(out, ob, gamma, (size_t)K * 2))
    return fail(MI_E_ARGS, "out overlaps an input");
  if (gamma && cfg && (cfg->variant == 14 || cfg->variant == 16))
    return fail(MI_E_TILE, "rmsnorm_matmul variants 14 and 16 compute the fused product without gamma; with gamma "
                           "use variant 0, 1, 4, 5, 11, 12, 13 or 15");
  mi_tile_cfg no_gamma_default;
  if (!cfg && !gamma) {
    mi::capi::pick_default_no_gamma(M, N, K, &no_gamma_default);
    cfg = &no_gamma_default;
  }
  mi::MiArgs a = {x, W, gamma, out, M, N, K, eps, 1.0f / (float)K, 8};
  return run(MI_KERNEL_RMSNORM_MATMUL_BF16, cfg, a, stream);
}

int mi_device_info(int* num_devices, char* arch, int arch_len, int* num_cus) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  if (num_devices) *num_devices = n;
  if (n > 0 && (arch || num_cus)) {
    hipDeviceProp_t p;
    e = hipGetDeviceProperties(&p, 0);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    if (arch && arch_len > 0) {
      strncpy(arch, p.gcnArchName, (size_t)arch_len - 1);
      arch[arch_len - 1] = '\0';
    }
    if (num_cus) *num_cus = p.multiProcessorCount;
  }
  return MI_OK;
}

int mi_release_workspace(void) {
  std::lock_guard<std::mutex> lock(g_pool_mu);
  if (g_pools.empty()) return MI_OK;  // no call has needed workspace yet
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  int rc = MI_OK;
  // The kept buffers first, once every stream's work on the device is done.
  for (KeptWs& k : g_kept) {
    if ((e = hipSetDevice(k.dev)) != hipSuccess || (e = hipDeviceSynchronize()) != hipSuccess ||
        (k.ptr && (e = hipFreeAsync(k.ptr, nullptr)) != hipSuccess) ||
        (k.done && (e = hipEventDestroy(k.done)) != hipSuccess)) {
      rc = hip_fail(e, "releasing a kept workspace");
      break;
    }
    k.ptr = nullptr;
  }
  if (rc != MI_OK) {
    (void)hipSetDevice(cur);
    return rc;
  }
  g_kept.clear();
  for (const auto& kv : g_pools) {
    // The runtime hands memory freed by hipFreeAsync back to its pool at the
    // pool's next allocation, not at a synchronisation: one small
    // allocation makes the earlier frees trimmable.  It may be carved out
    // of the block just freed, so it is freed with hipFree (synchronous,
    // at once) rather than hipFreeAsync (pending until the next allocation,
    // which would keep that whole block from the trim).
    void* p = nullptr;
    if ((e = hipSetDevice(kv.first)) != hipSuccess || (e = hipMallocFromPoolAsync(&p, 256, kv.second, nullptr)) != hipSuccess ||
        (e = hipStreamSynchronize(nullptr)) != hipSuccess || (e = hipFree(p)) != hipSuccess ||
        (e = hipMemPoolTrimTo(kv.second, 0)) != hipSuccess) {
      rc = hip_fail(e, "releasing the workspace pool");
      break;
    }
  }
  e = hipSetDevice(cur);
  if (rc == MI_OK && e != hipSuccess) rc = hip_fail(e, "hipSetDevice");
  return rc;
}

const char* mi_last_error(void) { return g_err; }

const char* mi_version(void) { return "mi_kernels 0.1 gfx950"; }

}  // extern "C"
