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

const mi::MiEntry* find(int kernel_id, const mi_tile_cfg& cfg) {
  for (const mi::MiEntry& e : registry())
    if (e.kernel_id == kernel_id && same_instance(e.cfg, cfg)) return &e;
  return nullptr;
}

constexpr unsigned long long kMaxOffset = 0xFFFFFFFFull;        // 32-bit buffer offsets
constexpr int kMaxSplit = 16;                                    // split-K parts
constexpr unsigned long long kMaxWorkspace = 1ull << 31;         // bytes of device workspace per call

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
      break;
    case MI_KERNEL_MATMUL_LHST_RHS_F32:
      // 16 x 16 threads with 4 x 4 outputs each, K slices of 16 or 32.
      if (c.variant == 0) {
        if (bm != 64 || bn != 64 || (bk != 16 && bk != 32) || w != 4 || s != 1)
          return mi::bad(MI_E_TILE, "the fp32 kernel takes 64x64 blocks, block_k 16 or 32, 4 waves, 1 stage");
        return mi::ok();
      }
      break;
    default:
      break;
  }
  return mi::bad(MI_E_TILE, "no such variant of this kernel");
}

bool splittable(int kernel_id, int variant) {
  return (kernel_id == MI_KERNEL_MATMUL_LHST_RHS_BF16 && (variant == 1 || variant == 3 || variant == 4)) ||
         (kernel_id == MI_KERNEL_MATMUL_LHS_RHS_BF16 && (variant == 0 || variant == 2)) ||
         (kernel_id == MI_KERNEL_RMSNORM_MATMUL_BF16 &&
          (variant == 4 || variant == 5 || variant == 11 || variant == 12 || variant == 13));
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
  const size_t ws = mi::workspace_bytes(kernel_id, c, M, N, K);
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

// Default configs.  A grid fills the chip with one workgroup per CU on 256
// CUs; 224 (28 per XCD) still counts as full.
constexpr long long kFillTiles = 224;
constexpr long long kCUs = 256;

long long tiles_of(int M, int N, int bm, int bn) {
  return (((long long)M + bm - 1) / bm) * (((long long)N + bn - 1) / bn);
}

// The most parts (a power of two, at most 16) that keep the grid within one
// workgroup per CU, every part at least 4 K tiles of block_k, and no part
// empty; 1 when no split qualifies.
int fill_parts(long long tiles, int K, int block_k) {
  const long long kt = ((long long)K + block_k - 1) / block_k;
  int parts = 1;
  for (int next = 2; next <= 16; next *= 2) {
    const long long kts = (kt + next - 1) / next;
    if (tiles * next > kCUs || kt < 4LL * next || (long long)(next - 1) * kts >= kt) break;
    parts = next;
  }
  return parts;
}

// A candidate block and its relative throughput per CU (output area per
// unit time at the same K, the 256 x 256 block = 1), measured with the
// autotuner at shapes that give every CU one tile.
struct Cand {
  mi_tile_cfg c;
  double rate;
};

// The candidate with the least estimated time: the rounds of tiles the
// busiest CU runs, times a tile's area over its rate.  Ties go to the
// earlier (larger) block.  Then, if its grid leaves CUs idle and K is long
// enough to split, K is split so the grid fills the chip.
mi_tile_cfg fastest_estimate(const Cand* cands, int n, int M, int N, int K, int kernel_id) {
  int best = 0;
  double best_t = 0.0;
  for (int i = 0; i < n; ++i) {
    const mi_tile_cfg& c = cands[i].c;
    const long long rounds = (tiles_of(M, N, c.block_m, c.block_n) + kCUs - 1) / kCUs;
    const double t = (double)rounds * c.block_m * c.block_n / cands[i].rate;
    if (i == 0 || t < best_t) {
      best = i;
      best_t = t;
    }
  }
  mi_tile_cfg c = cands[best].c;
  const long long tiles = tiles_of(M, N, c.block_m, c.block_n);
  if (tiles >= kFillTiles || fill_parts(tiles, K, c.block_k) == 1) return c;
  // The grid needs a split: the largest splittable block whose split grid
  // is as large as any (a bigger block moves fewer operand bytes per
  // multiply-add for the same workgroup count).
  long long most = 0;
  for (int i = 0; i < n; ++i) {
    const mi_tile_cfg& ci = cands[i].c;
    if (!splittable(kernel_id, ci.variant)) continue;
    const long long t = tiles_of(M, N, ci.block_m, ci.block_n);
    const long long wgs = t * fill_parts(t, K, ci.block_k);
    if (wgs > most) {
      most = wgs;
      c = ci;
    }
  }
  c.split_k = fill_parts(tiles_of(M, N, c.block_m, c.block_n), K, c.block_k);
  return c;
}

// As fastest_estimate, for the fused kernel (whose first candidate needs no
// workspace), but each candidate is first split by fill_parts when its grid
// leaves CUs idle, a candidate whose device workspace would pass the 2 GiB
// limit is skipped, and its estimated time (microseconds) adds the
// split's fp32 partial products, written once and read back once at about
// 5 TB/s, and for the two-pass fused kernel (variant 13) its pack pass (x
// read, x * gamma written: 4 bytes per x element at about 5 TB/s) and 3 us
// for the second launch.  R0 is the fused kernel's 128 x 512 rate per CU at
// 4096^3, in multiply-adds per second.
// The fewest parts, from c.split_k up by powers of two, that leave every K
// part within the gamma entries the fused instance stages in LDS and no part
// empty; 0 when none up to kMaxSplit does (or the instance is not built).
int gamma_fit_parts(const mi_tile_cfg& c, int K) {
  const mi::MiEntry* e = find(MI_KERNEL_RMSNORM_MATMUL_BF16, c);
  if (!e) return 0;
  const long long kt = ((long long)K + c.block_k - 1) / c.block_k;
  for (int p = c.split_k; p <= kMaxSplit; p *= 2) {
    const long long kts = (kt + p - 1) / p;
    if (p > 1 && (long long)(p - 1) * kts >= kt) return 0;
    if (e->gamma_kmax <= 0 || kts * c.block_k <= e->gamma_kmax) return p;
  }
  return 0;
}

mi_tile_cfg fastest_split_estimate(const Cand* cands, int n, int M, int N, int K, const mi_tile_cfg& fallback) {
  constexpr double R0 = 2.28e12, kSplitBytesPerUs = 5e6, kPackBytesPerUs = 5e6, kLaunchUs = 3.0;
  double best_t = 0.0;
  mi_tile_cfg best_c = fallback;
  bool found = false;
  for (int i = 0; i < n; ++i) {
    mi_tile_cfg c = cands[i].c;
    const long long tiles = tiles_of(M, N, c.block_m, c.block_n);
    c.split_k = tiles < kFillTiles ? fill_parts(tiles, K, c.block_k) : 1;
    // Past the gamma entries an instance stages, K splits further; a
    // candidate no split makes legal, or whose workspace the call could not
    // allocate, is out.
    c.split_k = gamma_fit_parts(c, K);
    if (c.split_k == 0) continue;
    if (mi::workspace_bytes(MI_KERNEL_RMSNORM_MATMUL_BF16, c, M, N, K) > kMaxWorkspace) continue;
    const long long wgs = tiles * c.split_k, rounds = (wgs + kCUs - 1) / kCUs;
    const double kp = (double)((K + c.split_k - 1) / c.split_k);
    double t = (double)rounds * c.block_m * c.block_n * kp / (cands[i].rate * R0) * 1e6;
    // The chip is power-limited under this load, so a single round that
    // leaves CUs idle runs each busy CU faster (its clock rises): by up to
    // 0.88 / (the busy fraction), at most 1.65 times (fitted to the fused
    // candidates timed at 23 shapes).
    if (rounds == 1) {
      const double busy = (double)wgs / kCUs, speed = 0.88 / busy;
      t /= speed > 1.65 ? 1.65 : speed < 1.0 ? 1.0 : speed;
    }
    if (c.split_k > 1) t += (double)c.split_k * M * N * 8.0 / kSplitBytesPerUs + kLaunchUs;
    if (c.variant == 13) t += (double)M * K * 4.0 / kPackBytesPerUs + kLaunchUs;
    if (!found || t < best_t) {
      found = true;
      best_t = t;
      best_c = c;
    }
  }
  return best_c;
}

// Skinny M (decode-like), either matmul: the weight is streamed once with
// the non-temporal variants (lhsT.rhs 3, lhs.rhs 2).
mi_tile_cfg skinny_matmul_default(bool lhs, int M, int N, int K) {
  const int v_nt = lhs ? 2 : 3;
  const mi_tile_cfg skinny = lhs ? mi_tile_cfg{128, 128, 64, 4, 3, 1, 8, v_nt}
                             : M <= 32 ? mi_tile_cfg{32, 128, 128, 4, 3, 1, 8, v_nt}
                             : M <= 64 ? mi_tile_cfg{64, 128, 64, 4, 4, 1, 8, v_nt}
                                       : mi_tile_cfg{128, 128, 64, 4, 3, 1, 8, v_nt};
  // A grid of the skinny block that fills the chip runs unsplit.
  if (tiles_of(M, N, skinny.block_m, skinny.block_n) >= kFillTiles) return skinny;
  mi_tile_cfg c = skinny;
  if (lhs) {
    // lhs.rhs: the non-temporal block with the fewest wasted rows (64 x 128
    // up to M = 64), split over K to up to one workgroup per CU.
    if (M <= 64) c = {64, 128, 64, 4, 4, 1, 8, v_nt};
    c.split_k = fill_parts(tiles_of(M, N, c.block_m, c.block_n), K, c.block_k);
    return c;
  }
  // lhsT.rhs with a long K (8192 or more): 256-wide column blocks (512-byte
  // weight row segments per workgroup) split over K, when that fills three
  // quarters of the CUs or more with at least 16 K steps per part.
  mi_tile_cfg wide = M <= 64 ? mi_tile_cfg{64, 256, 64, 4, 3, 1, 8, v_nt} : mi_tile_cfg{128, 256, 32, 4, 3, 1, 8, v_nt};
  const long long wide_tiles = tiles_of(M, N, wide.block_m, wide.block_n);
  wide.split_k = fill_parts(wide_tiles, K, wide.block_k);
  if (K >= 8192 && wide_tiles * wide.split_k >= 3 * kCUs / 4 && (long long)K / wide.split_k >= 16LL * wide.block_k)
    return wide;
  // Otherwise the block with the most tiles up to one per CU (ties to the
  // larger), split only when that grid still leaves CUs idle.
  const mi_tile_cfg cands[] = {skinny, mi_tile_cfg{64, 128, 64, 4, 4, 1, 8, v_nt},
                               mi_tile_cfg{64, 64, 64, 4, 4, 1, 8, v_nt}};
  long long most = 0;
  for (const mi_tile_cfg& ci : cands) {
    const long long t = tiles_of(M, N, ci.block_m, ci.block_n), capped = t < kCUs ? t : kCUs;
    if (capped > most) {
      most = capped;
      c = ci;
    }
  }
  if (most < kFillTiles) c.split_k = fill_parts(most, K, c.block_k);
  return c;
}

// Either matmul past skinny M: the block whose rounds of tiles take the
// least time (a block that leaves CUs idle can still beat a smaller one
// whose grid needs a second, partial round), K split when the chosen grid
// leaves CUs idle.  lhsT.rhs runs the pipelined variant 1; a 256-long block
// lies with its long side along the shorter output side (128 x 256 when
// M >= N), or along N at any shape when K <= 2048, and a 128-long one along
// N unless N is at least four times M, as the winners do.  lhs.rhs runs
// variant 0 and keeps block_m the short side (fewer rows of its
// K-contiguous operand per tile); its 256-long blocks take the paired-load
// variant 1 (block_k 32, the K-contiguous panel loaded as whole 128-byte
// lines).
mi_tile_cfg matmul_default(int kernel_id, bool lhs, int M, int N, int K) {
  const int v = lhs ? 0 : 1;
  const bool m_long = M >= N, n_much_longer = (long long)N >= 4LL * M;
  const Cand cands[] = {
      {lhs ? mi_tile_cfg{256, 256, 32, 8, 3, 1, 8, 1} : mi_tile_cfg{256, 256, 32, 4, 3, 1, 8, v}, 1.0},
      {lhs ? mi_tile_cfg{128, 256, 32, 4, 3, 1, 8, 1}
           : (m_long || K <= 2048 ? mi_tile_cfg{128, 256, 32, 4, 3, 1, 8, v} : mi_tile_cfg{256, 128, 32, 4, 3, 1, 8, v}),
       0.93},
      {mi_tile_cfg{128, 128, 64, 4, 3, 1, 8, v}, 0.62},
      {n_much_longer && !lhs ? mi_tile_cfg{128, 64, 64, 4, 4, 1, 8, v} : mi_tile_cfg{64, 128, 64, 4, 4, 1, 8, v}, 0.60},
      {mi_tile_cfg{64, 64, 64, 4, 4, 1, 8, v}, 0.35}};
  return fastest_estimate(cands, 5, M, N, K, kernel_id);
}

// rmsnorm_matmul.  The register-staged kernels keep gamma in LDS (8192
// entries here).
mi_tile_cfg fused_default(int M, int N, int K) {
  if (M <= 128 && K > 8192) {
    // Skinny M past K = 8192: the skinny variant 11 split into the fewest
    // parts whose gamma fits (1..16 parts, none empty); past that the
    // LDS-staged kernel (variant 0) takes any K.
    const long long kt = (K + 63) / 64;
    for (int p = 2; p <= 16; p *= 2) {
      const long long kts = (kt + p - 1) / p;
      const unsigned long long ws = (unsigned long long)p * ((unsigned long long)M * N + M) * 4ull;
      if (kts * 64 <= 8192 && (long long)(p - 1) * kts < kt && ws <= kMaxWorkspace)
        return {M <= 32 ? 32 : M <= 64 ? 64 : 128, 128, 64, 4, 3, p, 8, 11};
    }
    return {64, 128, 64, 4, 2, 1, 8, 0};
  }
  if (M <= 128) {
    // Weight streamed once (variant 11).  With a weight of 16 MiB or less
    // (re-read from the caches), 32-row blocks (more tiles) win at any M
    // (measured up to 16 MiB; at 32 MiB the 64-row block won); a larger one
    // takes the block that covers M, with 64-row blocks before a split when
    // 128-row ones leave CUs idle.  Below K = 4096 the summing launch of a
    // split costs more than the idle CUs do.
    const bool cached_w = (long long)K * N * 2 <= (16LL << 20);
    mi_tile_cfg c = {cached_w || M <= 32 ? 32 : M <= 64 ? 64 : 128, 128, 64, 4, 3, 1, 8, 11};
    if (c.block_m == 128 && tiles_of(M, N, 128, 128) < kFillTiles) c.block_m = 64;
    if (K >= 4096) c.split_k = fill_parts(tiles_of(M, N, c.block_m, c.block_n), K, c.block_k);
    return c;
  }
  // Each workgroup of the one-pass kernels scales its x rows once per column
  // tile, so narrow blocks pay that work many times over: per CU, 128 x 256
  // runs at 0.83 and 128 x 128 at 0.54 of the rate of 128 x 512.  The
  // two-pass kernel scales x once, in a pass of its own, and its main pass
  // runs the lhsT core (256 x 256 at 1.10 of that rate; past K = 8192 also
  // 256 x 128, its long side along the shorter output side, at 0.95).
  // Few-tile shapes split K, which the estimate charges for its fp32 partial
  // products and the launch of the summing kernel; past K = 8192 the
  // one-pass kernels split at least until each part's gamma fits.
  const Cand cands[] = {{mi_tile_cfg{128, 512, 32, 8, 3, 1, 8, 4}, 1.0},
                        {mi_tile_cfg{128, 256, 32, 4, 3, 1, 8, 5}, 0.83},
                        {mi_tile_cfg{128, 128, 64, 4, 2, 1, 8, 4}, 0.54},
                        {mi_tile_cfg{256, 256, 32, 4, 3, 1, 8, 13}, 1.10},
                        {mi_tile_cfg{128, 128, 64, 4, 3, 1, 8, 13}, 0.68},
                        {mi_tile_cfg{64, 128, 64, 4, 4, 1, 8, 13}, 0.57},
                        {M <= N ? mi_tile_cfg{256, 128, 64, 4, 3, 1, 8, 13} : mi_tile_cfg{128, 256, 64, 4, 3, 1, 8, 13},
                         0.95}};
  return fastest_split_estimate(cands, K > 8192 ? 7 : 6, M, N, K, mi_tile_cfg{128, 256, 64, 8, 2, 1, 8, 0});
}

// The library default, generalised from the autotune winners at the
// benchmark shapes and studies of 83 other shapes and 30 seeded random ones.
int pick_default(int kernel_id, int M, int N, int K, mi_tile_cfg* cfg) {
  const bool lhs = kernel_id == MI_KERNEL_MATMUL_LHS_RHS_BF16;
  switch (kernel_id) {
    case MI_KERNEL_MATMUL_LHST_RHS_F32:
      *cfg = {64, 64, 16, 4, 1, 1, 0, 0};
      break;
    case MI_KERNEL_MATMUL_LHST_RHS_BF16:
    case MI_KERNEL_MATMUL_LHS_RHS_BF16:
      *cfg = M <= 128 ? skinny_matmul_default(lhs, M, N, K) : matmul_default(kernel_id, lhs, M, N, K);
      break;
    case MI_KERNEL_RMSNORM_MATMUL_BF16:
      *cfg = fused_default(M, N, K);
      break;
    default:
      *cfg = {256, 256, 64, 8, 2, 1, 8, 0};
      break;
  }
  return MI_OK;
}

// Device workspace (split-K partial products, the two-pass fused kernel's
// packed operand): allocated per call, stream-ordered (hipMallocFromPoolAsync
// / hipFreeAsync), from a memory pool the library keeps per device.  The
// runtime hands a call's freed workspace back to the pool at the pool's
// next allocation (measured: not at a synchronisation), and the pool's
// release threshold, kPoolKeepBytes, then returns what it holds beyond that
// to the device.  So between calls the library holds up to the last
// workspace call's buffer plus kPoolKeepBytes; mi_release_workspace returns
// all of it.
// Each call has its own buffer (calls on different streams do not share
// one), and a call under HIP graph capture becomes allocation and free
// nodes of the graph.
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

int launch(const mi::MiEntry* e, const mi_tile_cfg& cfg, const mi::MiArgs& args_in, char* ws, void* stream) {
  mi::MiArgs a = args_in;
  a.group_m = cfg.group_m > 0 ? cfg.group_m : 8;
  a.parts = cfg.split_k;
  a.ws = ws;
  const hipError_t err = e->launch(a, (hipStream_t)stream);
  return err == hipSuccess ? MI_OK : hip_fail(err, "kernel launch");
}

// fixed_ws != NULL: the caller's device buffer of fixed_cap bytes serves as
// the workspace (nothing is allocated; a larger need is rejected).
int run(int kernel_id, const mi_tile_cfg* cfg_in, const mi::MiArgs& args_in, void* stream, char* fixed_ws = nullptr,
        size_t fixed_cap = 0) {
  mi_tile_cfg cfg;
  const mi::MiEntry* e = nullptr;
  const int rc = resolve(kernel_id, cfg_in, args_in, &cfg, &e);
  if (rc != MI_OK) return rc;
  const size_t ws_bytes = mi::workspace_bytes(kernel_id, cfg, args_in.M, args_in.N, args_in.K);
  if (ws_bytes == 0) return launch(e, cfg, args_in, nullptr, stream);
  if (fixed_ws) {
    if (ws_bytes > fixed_cap)
      return fail(MI_E_RANGE, "the config needs %zu bytes of workspace, over the %zu-byte static scratch", ws_bytes,
                  fixed_cap);
    return launch(e, cfg, args_in, fixed_ws, stream);
  }
  hipMemPool_t pool = nullptr;
  const int prc = workspace_pool(&pool);
  if (prc != MI_OK) return prc;
  char* ws = nullptr;
  const hipError_t ae = hipMallocFromPoolAsync((void**)&ws, ws_bytes, pool, (hipStream_t)stream);
  if (ae != hipSuccess) return hip_fail(ae, "workspace alloc");
  const int lrc = launch(e, cfg, args_in, ws, stream);
  const hipError_t fe = hipFreeAsync(ws, (hipStream_t)stream);
  if (lrc != MI_OK) return lrc;
  if (fe != hipSuccess) return hip_fail(fe, "workspace free");
  return MI_OK;
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
  for (const auto& kv : g_pools) {
    // The runtime hands memory freed by hipFreeAsync back to its pool at the
    // pool's next allocation, not at a synchronisation: one small
    // allocation and free, completed, makes the earlier frees trimmable.
    void* p = nullptr;
    if ((e = hipSetDevice(kv.first)) != hipSuccess || (e = hipMallocFromPoolAsync(&p, 256, kv.second, nullptr)) != hipSuccess ||
        (e = hipFreeAsync(p, nullptr)) != hipSuccess || (e = hipStreamSynchronize(nullptr)) != hipSuccess ||
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
