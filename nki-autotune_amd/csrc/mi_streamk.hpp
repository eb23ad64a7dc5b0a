// mi_streamk.hpp -- work split and combine protocol of the stream-K kernels.
//
// A stream-K launch deals the K tiles of every output tile evenly over a
// fixed grid of G workgroups (one per CU), instead of one output tile per
// workgroup: with T output tiles of KT K tiles each, the T*KT "units" are
// numbered tile-major (unit u = t*KT + kt) and workgroup w takes units
// [begin(w), begin(w+1)), begin(w) = floor(w*T*KT / G).  A workgroup's range
// is at most one tile's tail (its first segment), then whole tiles, then
// one tile's head (its last segment).  When T < G (the skinny shapes: 224
// tiles of 128 columns for 256 CUs) every CU still gets the same share of
// the K loop, where one tile per workgroup would leave CUs idle.
//
// A workgroup runs its segments in reverse: the head of its last tile
// first (K tiles from 0), the tail of its first tile last.  With equal
// shares of L = T*KT/G units, a workgroup whose head has h units reads K
// tile tau at time tau for tau < h and K tile tau + (KT - L) after, so the
// whole grid streams the operands on two fronts KT - L tiles apart, close
// to the lockstep in which one-tile-per-workgroup kernels read them (and
// which keeps the HBM pages they read shared).  Unit order would scatter
// the workgroups over K and cost about a tenth of the bandwidth.
//
// The parts of a tile split between workgroups, in K order, are p_0 (held
// by first_wg(t), which holds K tile 0) .. p_n (n = later_parts(t); p_e by
// workgroup first_wg(t) + e).  p_n, which holds the last K tile, is the
// *checker*, run last by its workgroup; the others are *storers*, run
// early.  Exactly one part combines the tile, and nobody waits for anybody
// (the tile counter ctr[t] starts at 0):
//   storer: store its fp32 partial to its slot (p_0: the tile's first slot;
//     p_e: the later slot of its workgroup), then ctr += 1; if the checker's
//     partial was already stored (LAST_READY set) and this was the last
//     storer to arrive, combine (every part from the slots);
//   checker: ctr += LAST_ARRIVED; if every storer had arrived, combine
//     (its own part still in registers); else store its partial to its
//     later slot, then ctr += LAST_READY; if every storer has arrived by
//     then, combine.
// In every order of those atomic additions exactly one part combines, and
// it finds every other part's partial stored (tests/test_streamk_plan.py
// checks all interleavings).  Storers run first in their workgroups and the
// checker last, so normally the checker combines and never stores.  Either
// combiner adds ((p_0 + p_1) + ...) + p_n in that order, so the result does
// not depend on who combined or when; it resets ctr[t] to 0 for the next
// launch.
//
// Plain C++ (MI_HD functions), shared by the kernels and a CPU test.
#pragma once
#include <stdint.h>

#ifndef MI_HD
#define MI_HD __host__ __device__
#endif

namespace mi {

constexpr int kSkLastArrived = 1 << 16;
constexpr int kSkLastReady = 1 << 17;
constexpr int kSkStoredMask = kSkLastArrived - 1;
// The stream-K counters live in the first kSkCounterBytes of every device
// workspace (split-K and two-pass data start after them), so a workspace
// that is reused keeps them at 0: each stream-K launch leaves them 0.
constexpr int kSkCounterBytes = 16384;
constexpr int kSkMaxTiles = kSkCounterBytes / 4;

struct StreamKPlan {
  long long tiles, kt, grid, total;

  MI_HD StreamKPlan(long long tiles_, long long kt_, long long grid_)
      : tiles(tiles_), kt(kt_), grid(grid_), total(tiles_ * kt_) {}

  // First unit of workgroup w (w = grid gives total).
  MI_HD long long begin(long long w) const { return w * total / grid; }
  // The workgroup whose range holds unit u: the largest w with begin(w) <= u.
  MI_HD long long wg_of_unit(long long u) const { return ((u + 1) * grid - 1) / total; }
  // The workgroup holding K tile 0 of tile t (its part p_0).
  MI_HD long long first_wg(long long t) const { return wg_of_unit(t * kt); }
  // Parts of tile t after p_0: workgroups first_wg(t)+1 .. first_wg(t)+later_parts(t),
  // each starting inside the tile (every workgroup's range is non-empty
  // because grid <= total).
  MI_HD long long later_parts(long long t) const { return wg_of_unit(t * kt + kt - 1) - first_wg(t); }
};

// Grid of a stream-K launch: one workgroup per CU, at most one per unit.
MI_HD inline long long streamk_grid(long long cus, long long tiles, long long kt) {
  const long long total = tiles * kt;
  return cus < total ? cus : total;
}

}  // namespace mi
