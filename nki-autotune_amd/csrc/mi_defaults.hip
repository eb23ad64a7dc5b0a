// mi_defaults.hip -- the library default config (mi_default_config): for a
// call with no config, the block whose estimated time at the shape is the
// least, generalised from the autotune winners at the benchmark shapes,
// campaigns that timed every candidate block and split at about 200 more
// shapes, and studies of 83 shapes and of seeded random ones.  Host code
// only.
#include "mi_capi_internal.hpp"

namespace mi {
namespace capi {
namespace {

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
    if (!splittable(MI_KERNEL_RMSNORM_MATMUL_BF16, c.variant)) c.split_k = 1;
    // Past the gamma entries an instance stages, K splits further; a
    // candidate no split makes legal, or whose workspace the call could not
    // allocate, is out.
    c.split_k = gamma_fit_parts(c, K);
    if (c.split_k == 0) continue;
    if (mi::workspace_bytes(MI_KERNEL_RMSNORM_MATMUL_BF16, c, M, N, K, kDefaultCus) > kMaxWorkspace) continue;
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
    // Variant 15's pack writes x's own layout, no transpose: 0.9 of the time.
    if (c.variant == 15) t += 0.9 * (double)M * K * 4.0 / kPackBytesPerUs + kLaunchUs;
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
  if (lhs) {
    // lhs.rhs: the non-temporal 128 x 128 block when its grid fills the
    // chip; otherwise the non-temporal block with the fewest wasted rows
    // (64 x 128 up to M = 64), split over K to up to one workgroup per CU.
    const mi_tile_cfg skinny = {128, 128, 64, 4, 3, 1, 8, v_nt};
    if (tiles_of(M, N, skinny.block_m, skinny.block_n) >= kFillTiles) return skinny;
    mi_tile_cfg c = M <= 64 ? mi_tile_cfg{64, 128, 64, 4, 4, 1, 8, v_nt} : skinny;
    c.split_k = fill_parts(tiles_of(M, N, c.block_m, c.block_n), K, c.block_k);
    // A 128-row split whose parts would keep under 1024 of K gives way to
    // the 64 x 128 block with block_k 128, itself split to fill the CUs
    // (128x9920x1600: unsplit, 17.9 us against 21.6 us for 128 x 128 in 2
    // parts of 800; 128x1856x14272: 8 parts, 26.0 us).
    if (c.block_m == 128 && c.split_k >= 2 && (K + c.split_k - 1) / c.split_k < 1024) {
      c = {64, 128, 128, 4, 3, 1, 8, v_nt};
      c.split_k = fill_parts(tiles_of(M, N, 64, 128), K, 128);
    }
    return c;
  }
  // lhsT.rhs: a skinny launch is bound by each workgroup's own loads (its
  // MFMA pipe is a quarter busy at most), so the estimate is the rounds of
  // workgroups times one workgroup's panel bytes, (block_m + block_n) x (its
  // K range + 256) x 2, at 70 GB/s per CU plus 3 us (the 256 rows of K
  // stand for the ring's fill, which a short part does not hide), and a
  // split pays its fp32 partial products, written and read back (8 bytes
  // per output element and part), at 5 TB/s plus 1 us for the summing
  // launch; splits stop at 8 parts, and every part keeps at least 512 of K.
  // Fitted to every block and split timed at 46 skinny shapes (M 8-128, K
  // 512-16384) with the weight flushed and the split workspace kept per
  // stream: the pick within 1.069 of the fastest at all of them (mean
  // 1.009), and within 1.034 at the third of the shapes held out of a fit
  // to the other two thirds.  Equal estimates go to the earlier block (32 x
  // 128 with block_k 64 and 4 stages measured faster than with block_k 128
  // and 3; 128 x 128 with block_k 32 and 4 stages than with 64 and 3).
  const mi_tile_cfg cands[] = {
      {32, 128, 64, 4, 4, 1, 8, v_nt},  {32, 128, 128, 4, 3, 1, 8, v_nt}, {32, 256, 64, 4, 4, 1, 8, v_nt},
      {64, 128, 64, 4, 4, 1, 8, v_nt},  {64, 64, 64, 4, 4, 1, 8, v_nt},   {64, 256, 64, 4, 3, 1, 8, v_nt},
      {128, 128, 32, 4, 4, 1, 8, v_nt}, {128, 128, 64, 4, 3, 1, 8, v_nt}, {128, 256, 32, 4, 3, 1, 8, v_nt},
      {128, 256, 32, 4, 4, 1, 8, v_nt}};
  // Blocks more than twice as tall as M are not considered; splits stop at
  // 320 workgroups.
  const int m_cap = 2 * (M > 32 ? M : 32);
  mi_tile_cfg c = cands[0];
  double best_t = 0.0;
  bool found = false;
  for (const mi_tile_cfg& ci : cands) {
    if (ci.block_m > m_cap) continue;
    const long long tiles = tiles_of(M, N, ci.block_m, ci.block_n), kt = ((long long)K + ci.block_k - 1) / ci.block_k;
    for (int p = 1; p <= 8; p *= 2) {
      const long long kts = (kt + p - 1) / p, wgs = tiles * p;
      const double kp = (double)((K + p - 1) / p);
      if (p > 1 && (wgs > 320 || (long long)(p - 1) * kts >= kt || kp < 512.0)) break;
      double t = (double)((wgs + kCUs - 1) / kCUs) * ((ci.block_m + ci.block_n) * (kp + 256.0) * 2.0 / 70e3 + 3.0);
      if (p > 1) t += (double)p * M * N * 8.0 / 5e6 + 1.0;
      if (!found || t < best_t) {
        found = true;
        best_t = t;
        c = ci;
        c.split_k = p;
      }
    }
  }
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
  // lhsT.rhs with M <= N also weighs a 64 x 256 block, at a rate just under
  // the 128 x 128 block's: it is taken only where it needs fewer rounds of
  // tiles.  Timed with every candidate and split at 40 shapes past skinny M,
  // it changed the pick at three (1088x3840x4096: 1.29 x the fastest to
  // 1.00; 1088x3712x8000: 1.26 to 1.00; 704x11648x1088: 1.08 to 1.01).
  Cand cands[7];
  int n = 0;
  cands[n++] = {lhs ? mi_tile_cfg{256, 256, 32, 8, 3, 1, 8, 1} : mi_tile_cfg{256, 256, 32, 4, 3, 1, 8, v}, 1.0};
  cands[n++] = {lhs ? mi_tile_cfg{128, 256, 32, 4, 3, 1, 8, 1}
                    : (m_long || K <= 2048 ? mi_tile_cfg{128, 256, 32, 4, 3, 1, 8, v} : mi_tile_cfg{256, 128, 32, 4, 3, 1, 8, v}),
                0.93};
  // lhsT.rhs also weighs the other orientation of the 256-long block, after
  // the preferred one: it wins only where it needs fewer rounds of tiles
  // (7616x2112x1280: 510 tiles of 256 x 128 in two rounds against 540 of
  // 128 x 256 in three, 39.3 against 49.0 us).
  if (!lhs) {
    const mi_tile_cfg pref = cands[1].c;
    cands[n++] = {mi_tile_cfg{pref.block_n, pref.block_m, 32, 4, 3, 1, 8, v}, 0.93};
  }
  cands[n++] = {mi_tile_cfg{128, 128, 64, 4, 3, 1, 8, v}, 0.62};
  if (!lhs && M <= N) cands[n++] = {mi_tile_cfg{64, 256, 64, 4, 3, 1, 8, v}, 0.60};
  cands[n++] = {n_much_longer && !lhs ? mi_tile_cfg{128, 64, 64, 4, 4, 1, 8, v} : mi_tile_cfg{64, 128, 64, 4, 4, 1, 8, v}, 0.60};
  cands[n++] = {mi_tile_cfg{64, 64, 64, 4, 4, 1, 8, v}, 0.35};
  mi_tile_cfg c = fastest_estimate(cands, n, M, N, K, kernel_id);
  const bool small = c.split_k == 1 && c.block_m * c.block_n <= 128 * 64;
  if (lhs) {
    // lhs.rhs: a small unsplit block over K >= 8192 becomes the 128 x 128
    // block split to fill the chip.  Timed with every candidate and split at
    // 8 such shapes (256-3200 rows, interleaved rounds, one box): within
    // 1.045 of the fastest at all of them, against 1.29 for the small block.
    if (small && K >= 8192) {
      const int parts = fill_parts(tiles_of(M, N, 128, 128), K, 64);
      if (parts >= 2) c = {128, 128, 64, 4, 3, parts, 8, 0};
    }
    // An unsplit 128 x 128 grid that leaves CUs idle, over K >= 12288 and a
    // whole number of 256-row blocks, takes 256 x 128 in 2 parts (the same
    // workgroup count, a quarter fewer operand bytes per multiply-add):
    // 256x12224x12288 94.4 against 116.9 us, 256x9216x16384 1.23 x and
    // 512x6144x16384 1.03 x faster; not at 384 rows (the 256-row blocks'
    // tail, 1.17 x slower), K = 10240 or 224 tiles (1.07-1.10 x slower).
    if (c.block_m == 128 && c.block_n == 128 && c.split_k == 1 && tiles_of(M, N, 128, 128) < kFillTiles &&
        M % 256 == 0 && K >= 12288 && 2 * tiles_of(M, N, 256, 128) <= kCUs)
      return {256, 128, 64, 8, 3, 2, 8, 0};
    // An unsplit 128 x 128 block runs on the paired-load variant 1 with
    // block_k 32 and 4 stages (whole 128-byte lines of the K-contiguous
    // operand, three K tiles in flight): 0.90-0.99 x variant 0's time with
    // block_k 64 at the 8 shapes above, and the sweep's winner at 2048^3,
    // 1536x1536x6144, 704x5376x13824 and 704x4800x11712, where variant 0
    // ran 1.04-1.06 x its time.
    if (c.block_m == 128 && c.block_n == 128 && c.split_k == 1 && c.variant == 0) c = {128, 128, 32, 4, 4, 1, 8, 1};
    return c;
  }
  // lhsT.rhs 128x128 blocks then run block_k 32 with 4 stages, the same
  // parts (each part keeps at least 8 K tiles of 32): three tiles in flight
  // instead of two.  Measured against block_k 64 with 3 stages at eleven
  // shapes this picker gives the 128x128 block (split or not), in
  // interleaved rounds on one box: median 0.958 x the time, 0.880-1.022 x,
  // bitwise equal outputs.  (The K-contiguous lhs.rhs variant 0 keeps
  // block_k 64, where 32 loads half lines: median 1.008 x, up to 1.079 x;
  // its unsplit 128x128 block moves to the paired-load variant 1 above.)
  if (c.block_m == 128 && c.block_n == 128 && c.block_k == 64) {
    c.block_k = 32;
    c.lds_stages = 4;
  }
  // Where the rounds estimate settles on a small unsplit block with a long K
  // (64 x 64 from K = 3072; 64 x 128 or 128 x 64 from K = 8192, or where
  // each part of the 128 x 128 split keeps 3072 of K), or splits a 256-long
  // block 8 ways or more (below), the 128 x 128 block split to fill the
  // chip is faster: it moves half the operand bytes per multiply-add of a 64 x 64
  // block, and each part's partial products cost less than the MFMA time
  // they save.  Timed with every candidate and split at 30 shapes past
  // skinny M (interleaved rounds, one box), this takes the pick from within
  // 1.74 of the fastest (mean 1.082) to within 1.21 (mean 1.011); it
  // applies at 9 of the shapes, and the rest keep their pick.  The per-part
  // bound adds 896x1472x7872 (37.1 us for 64 x 128 against 31.5 us in 2
  // parts of 128 x 128) and changes no pick at the 70 timed shapes.
  const int parts = fill_parts(tiles_of(M, N, 128, 128), K, 32);
  const bool long_parts = parts >= 2 && (K + parts - 1) / parts >= 3072;
  const bool long_k = K >= 8192 || long_parts || (c.block_m == 64 && c.block_n == 64 && K >= 3072);
  const bool thin_256 = (c.block_m == 256 || c.block_n == 256) && c.split_k >= 8;
  if (small && long_k && parts >= 2) return {128, 128, 32, 4, 4, parts, 8, v};
  if (thin_256) {
    // A 256-long block split 8 ways or more: the largest of 128 x 128, the
    // 64-wide block (oriented as above) and 64 x 64 whose split to fill the
    // chip keeps each part at least 1536 (128 x 128) or 1792 (64-wide) of K,
    // else 64 x 64: shorter parts pay more in partial products than the
    // larger block saves.  Timed with every candidate and split at 12 such
    // shapes (K 4096-16384), the pick is within 1.035 of the fastest
    // (mean 1.007), against 1.43 (mean 1.108) for 128 x 128 at any K.
    if (parts >= 2 && (K + parts - 1) / parts >= 1536) return {128, 128, 32, 4, 4, parts, 8, v};
    const int bm = n_much_longer ? 128 : 64, bn = n_much_longer ? 64 : 128;
    const int pw = fill_parts(tiles_of(M, N, bm, bn), K, 64);
    if (pw >= 2 && (K + pw - 1) / pw >= 1792) return {bm, bn, 64, 4, 4, pw, 8, v};
    return {64, 64, 64, 4, 4, fill_parts(tiles_of(M, N, 64, 64), K, 64), 8, v};
  }
  return c;
}

// rmsnorm_matmul.  The register-staged kernels keep gamma in LDS (8192
// entries here).
// The skinny fused kernel's 128-row block leaves CUs idle below 256 tiles;
// it then keeps 128 rows (the weight read once) where its split to fill the
// CUs leaves each part at least 1024 of K, and takes 64-row blocks (the
// weight read twice, fewer parts) otherwise.  Timed with every block and
// split: 128x5760x10944 ran 46.0 us in 4 parts of 128 rows against 57.8 us
// for 64 rows in 2, 128x7552x5952 35.4 against 38.4, 96x3584x10176 32.4
// against 34.8; 128x8192x3072 (768 of K per part) 1.064 x and 128x1792x11008
// (688) 1.137 x the 64-row block's time.
bool skinny_keeps_128_rows(int M, int N, int K) {
  const long long t128 = tiles_of(M, N, 128, 128);
  if (t128 >= kFillTiles) return true;
  const int p = fill_parts(t128, K, 64);
  return p >= 2 && (K + p - 1) / p >= 1024;
}

mi_tile_cfg fused_default(int M, int N, int K) {
  if (M <= 128 && K > 8192) {
    // Skinny M past K = 8192: the skinny variant 11 (64-row blocks when
    // 128-row ones leave CUs idle) split into the fewest parts whose gamma
    // fits (1..16 parts, none empty), or into more when that fills more CUs
    // (up to one workgroup per CU); past 16 parts the LDS-staged kernel
    // (variant 0) takes any K.
    int bm = M <= 32 ? 32 : M <= 64 ? 64 : 128;
    if (bm == 128 && !skinny_keeps_128_rows(M, N, K)) bm = 64;
    const long long kt = (K + 63) / 64;
    const int fill = fill_parts(tiles_of(M, N, bm, 128), K, 64);
    for (int p = 2; p <= 16; p *= 2) {
      const long long kts = (kt + p - 1) / p;
      const unsigned long long ws = (unsigned long long)p * ((unsigned long long)M * N + M) * 4ull;
      if (kts * 64 <= 8192 && (long long)(p - 1) * kts < kt && ws <= kMaxWorkspace) {
        int parts = p;
        // A larger split: still no empty part, and its workspace fits.
        for (int q = p * 2; q <= fill; q *= 2) {
          const long long qts = (kt + q - 1) / q;
          const unsigned long long qws = (unsigned long long)q * ((unsigned long long)M * N + M) * 4ull;
          if ((long long)(q - 1) * qts < kt && qws <= kMaxWorkspace) parts = q;
        }
        // 32-row blocks whose split leaves more than 16 CUs idle take block_k
        // 128 (twice the K panel in flight per workgroup), where its parts
        // still hold their gamma and none is empty: at 6 such shapes it ran
        // 0.89-0.96 x the time of block_k 64 (8x12864x16256, 32x9728x9984,
        // 16x9088x9536, 32x13504x13056, 32x12864x14144, 32x10752x11328).
        const long long kt128 = (K + 127) / 128, kts128 = (kt128 + parts - 1) / parts;
        if (bm == 32 && tiles_of(M, N, 32, 128) * parts < 240 && kts128 * 128 <= 8192 && (parts - 1) * kts128 < kt128)
          return {32, 128, 128, 4, 3, parts, 8, 11};
        return {bm, 128, 64, 4, 3, parts, 8, 11};
      }
    }
    return {64, 128, 64, 4, 2, 1, 8, 0};
  }
  if (M <= 128) {
    // Weight streamed once (variant 11).  With a weight of 16 MiB or less
    // (re-read from the caches), 32-row blocks (more tiles) win at any M
    // (measured up to 16 MiB; at 32 MiB the 64-row block won); a larger one
    // takes the block that covers M, with 64-row blocks before a split when
    // 128-row ones leave CUs idle.  From K = 1024 K is split to fill the
    // CUs.  Timed with every block, stage count and split at 20 skinny fused
    // shapes (weight flushed, split workspace kept per stream): within 1.078
    // of the fastest at all of them (mean 1.017), against 1.82 (mean 1.22)
    // when splits started at K = 4096 (8x4096x3072: 28.8 us unsplit, 15.8
    // us in 8 parts).
    const bool cached_w = (long long)K * N * 2 <= (16LL << 20);
    mi_tile_cfg c = {cached_w || M <= 32 ? 32 : M <= 64 ? 64 : 128, 128, 64, 4, 3, 1, 8, 11};
    if (c.block_m == 128 && !skinny_keeps_128_rows(M, N, K)) c.block_m = 64;
    if (K >= 1024) c.split_k = fill_parts(tiles_of(M, N, c.block_m, c.block_n), K, c.block_k);
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
  // one-pass kernels split at least until each part's gamma fits.  The
  // two-pass kernel on the paired-load core (variant 15, never split) adds
  // 128 x 256 at 0.95, and 128 x 128 at 0.80 where that grid keeps more
  // than half the CUs busy (with fewer, a split or a 64-row block won at
  // every shape timed).  Fitted to every candidate and split timed at 23
  // fused shapes with M > 128 (interleaved rounds, one box): the pick within
  // 1.012 of the fastest at all of them (mean 1.0005, against 1.17 and 1.040
  // without variant 15).  The rates alone, without the half-busy rule, were
  // within 1.064 at the third of the shapes held out of a fit to the other
  // two thirds.
  Cand cands[9];
  int n = 0;
  cands[n++] = {mi_tile_cfg{128, 512, 32, 8, 3, 1, 8, 4}, 1.0};
  cands[n++] = {mi_tile_cfg{128, 256, 32, 4, 3, 1, 8, 5}, 0.83};
  cands[n++] = {mi_tile_cfg{128, 128, 64, 4, 2, 1, 8, 4}, 0.54};
  cands[n++] = {mi_tile_cfg{256, 256, 32, 4, 3, 1, 8, 13}, 1.10};
  cands[n++] = {mi_tile_cfg{128, 128, 64, 4, 3, 1, 8, 13}, 0.68};
  cands[n++] = {mi_tile_cfg{64, 128, 64, 4, 4, 1, 8, 13}, 0.57};
  if (2 * tiles_of(M, N, 128, 128) > kCUs) cands[n++] = {mi_tile_cfg{128, 128, 32, 4, 4, 1, 8, 15}, 0.80};
  cands[n++] = {mi_tile_cfg{128, 256, 32, 4, 3, 1, 8, 15}, 0.95};
  if (K > 8192)
    cands[n++] = {M <= N ? mi_tile_cfg{256, 128, 64, 4, 3, 1, 8, 13} : mi_tile_cfg{128, 256, 64, 4, 3, 1, 8, 13}, 0.95};
  return fastest_split_estimate(cands, n, M, N, K, mi_tile_cfg{128, 256, 64, 8, 2, 1, 8, 0});
}

}  // namespace

// The library default: the estimates and rules above, fitted to timed
// campaigns and checked against full autotune sweeps.
int pick_default(int kernel_id, int M, int N, int K, mi_tile_cfg* cfg) {
  const bool lhs = kernel_id == MI_KERNEL_MATMUL_LHS_RHS_BF16;
  switch (kernel_id) {
    case MI_KERNEL_MATMUL_LHST_RHS_F32:
      // The fp32 MFMA kernel; variant 0 (sequential K order) stays selectable.
      *cfg = {64, 64, 16, 4, 1, 1, 0, 1};
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

// The fused kernel's default for a call without gamma: pick_default's
// choice, except that its 128x128, 64x128 and 64x64 blocks (shapes of one
// or two rounds of tiles, split or not) go to a gamma-free variant, unsplit:
// 64x128 and 64x64 to variant 14 with the same block, 128x128 as below.
// Variant 14 measured in interleaved rounds against
// the default (no gamma): 0.60 x its time at 1024^3 (against the 4-part
// split), 0.89 x at 2048^3, 0.90 x at 1024x4096x4096, 0.80 x at
// 512x4096x4096, 0.78 x at 256x8192x2048; variant 16 at 128x128, against
// variant 14's 128x128 block: 0.924-0.957 x (median 0.938) at twelve shapes
// from 256x512x2048 to 4096x512x1024, with bitwise equal outputs.  The
// larger blocks (128x512, 256x256 two-pass, 128x256) stay,
// variant 14 being 0-8 % slower there.  Skinny M keeps its non-temporal
// variants.
int pick_default_no_gamma(int M, int N, int K, mi_tile_cfg* cfg) {
  const int rc = pick_default(MI_KERNEL_RMSNORM_MATMUL_BF16, M, N, K, cfg);
  if (rc != MI_OK) return rc;
  const int v = cfg->variant, bm = cfg->block_m, bn = cfg->block_n;
  const bool one_pass_or_two = v == 4 || v == 5 || v == 13 || v == 15;
  const bool small_block = (bm == 128 && bn == 128) || (bm == 64 && bn == 128) || (bm == 64 && bn == 64);
  if (M > 128 && one_pass_or_two && small_block) {
    // A 128 x 128 pick takes the largest block whose grid keeps more than
    // half the CUs busy: variant 16 at 128 x 128, else variant 14 at 64 x 128,
    // else at 64 x 64.  Measured without gamma (us, 128 x 128 v16 / 64 x 128
    // v14 / 64 x 64 v14): 59.9 / 76.1 / 75.5 at 384x8192x8192 (192 tiles of
    // 128 x 128); 29.2 / 23.5 / 28.7 at 512x4096x4096 (128 tiles), 53.7 /
    // 42.8 / 54.6 at 512x4096x8192, 16.3 / 12.9 / 14.3 at 1024x2048x2048;
    // 10.1 / 7.9 / 6.4 at 1024^3 (64 tiles), 27.2 / 20.8 / 16.4 at
    // 1024x1024x4096, 15.7 / 11.2 / 8.2 at 256x512x2048.
    if (bm == 128) {
      const long long t128 = tiles_of(M, N, 128, 128);
      if (2 * t128 > kCUs)
        *cfg = {128, 128, 32, 4, 4, 1, cfg->group_m, 16};
      else if (4 * t128 > kCUs)
        *cfg = {64, 128, 64, 4, 4, 1, cfg->group_m, 14};
      else
        *cfg = {64, 64, 64, 4, 4, 1, cfg->group_m, 14};
    } else {
      *cfg = {bm, bn, 64, 4, 4, 1, cfg->group_m, 14};
    }
  }
  return MI_OK;
}

}  // namespace capi
}  // namespace mi
