// mi_legal.hpp -- static legality of every kernel template, as constexpr
// predicates shared by the device code and the host.
//
// Each kernel template asserts `legal_<template>(params).code == MI_OK` at
// instantiation, and mi_cfg_check evaluates the same function at run time
// on the requested config.  So a config the host accepts as legal (whether
// prebuilt or to be built just in time from its template) is one whose
// template instantiates, and the LDS size the host budgets is the one the
// template allocates (each kernel also asserts that equality).
//
// The predicates return MI_OK, or the MI_E_* code of the first rule broken
// (include/mi_kernels.h) with a sentence naming it.
#pragma once
#include "../../include/mi_kernels.h"

#define MI_HD __host__ __device__

namespace mi {

constexpr int kLdsBytesMax = 160 * 1024;

struct Legal {
  int code;
  const char* why;
};
MI_HD constexpr Legal ok() { return Legal{MI_OK, ""}; }
MI_HD constexpr Legal bad(int code, const char* why) { return Legal{code, why}; }

MI_HD constexpr bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }
MI_HD constexpr int cmax(int a, int b) { return a > b ? a : b; }

// Wave grid: WM x WN waves, each owning a (BM/WM) x (BN/WN) block that is a
// whole number of 32x32 MFMA tiles; the most square wave block wins (first
// found on ties).  wm = -1 when no split exists.
struct WaveSplit {
  int wm, wn, wtm, wtn;
};
MI_HD constexpr WaveSplit wave_split(int bm, int bn, int waves) {
  int best = -1, bestd = 1 << 30;
  for (int wm = 1; wm <= waves; wm *= 2) {
    const int wn = waves / wm;
    if (wm * wn != waves || bm % wm || bn % wn) continue;
    const int tm = bm / wm, tn = bn / wn;
    if (tm < 32 || tn < 32 || tm % 32 || tn % 32) continue;
    const int d = tm > tn ? tm - tn : tn - tm;
    if (d < bestd) {
      bestd = d;
      best = wm;
    }
  }
  if (best < 0) return WaveSplit{-1, 1, 32, 32};
  return WaveSplit{best, waves / best, bm / best, bn / (waves / best)};
}

// Epilogue staging: one 32-row slice per wave, row stride WTN*2+16 bytes.
MI_HD constexpr int epilogue_bytes(int bm, int bn, int waves) {
  return waves * 32 * (wave_split(bm, bn, waves).wtn * 2 + 16);
}

// LDS-direct loader of an MN-contiguous [bk][w] panel (PanelLoader): rows of
// at most 1 KiB, at least one 1 KiB chunk; `even` when every wave issues the
// same number of chunk loads.
MI_HD constexpr bool mn_panel_ok(int bk, int w) { return w >= 32 && is_pow2(w) && w * 2 <= 1024 && bk * w * 2 >= 1024; }
MI_HD constexpr int mn_panel_loads(int bk, int w, int waves) { return (bk * w * 2 / 1024 + waves - 1) / waves; }
MI_HD constexpr bool mn_panel_even(int bk, int w, int waves) { return (bk * w * 2 / 1024) % waves == 0; }

// LDS-direct loader of a K-contiguous [rows][bk] panel (KPanelLoader).
MI_HD constexpr bool k_panel_ok(int bk, int rows) {
  return bk >= 16 && bk <= 128 && is_pow2(bk) && rows * bk * 2 >= 1024;
}
MI_HD constexpr int k_panel_loads(int bk, int rows, int waves) { return (rows * bk * 2 / 1024 + waves - 1) / waves; }
MI_HD constexpr bool k_panel_even(int bk, int rows, int waves) { return (rows * bk * 2 / 1024) % waves == 0; }

// Block sizes every bf16 template takes: powers of two, 32..512 wide.
MI_HD constexpr bool block_mn_ok(int bm, int bn) {
  return is_pow2(bm) && is_pow2(bn) && bm >= 32 && bm <= 512 && bn >= 32 && bn <= 512;
}
MI_HD constexpr bool waves_ok(int waves) { return is_pow2(waves) && waves <= 16; }

// The waves split the block into whole 32x32 MFMA tiles, and each wave's
// fp32 accumulators fit its share of the SIMD's 512 registers with room for
// operands: 256 registers at one wave per SIMD (a 128x128 wave tile), 128 at
// two, ...
MI_HD constexpr Legal wave_rules(int bm, int bn, int waves) {
  if (!waves_ok(waves) || wave_split(bm, bn, waves).wm < 0)
    return bad(MI_E_WAVE_TILE, "the waves cannot split the block into whole 32x32 MFMA tiles");
  const WaveSplit w = wave_split(bm, bn, waves);
  const int per_simd = (waves + 3) / 4;
  if (w.wtm * w.wtn / 64 * per_simd > 256)
    return bad(MI_E_WAVE_TILE, "each wave's accumulators exceed its share of the 512 registers");
  return ok();
}

// ---- lhsT.rhs, plain double buffer (matmul variant 0) ---------------------
MI_HD constexpr int lds_mm_plain(int bm, int bn, int bk, int waves, int stages) {
  return cmax(stages * (bk * bm * 2 + bk * bn * 2), epilogue_bytes(bm, bn, waves));
}
MI_HD constexpr Legal legal_mm_plain(int bm, int bn, int bk, int waves, int stages) {
  if (!block_mn_ok(bm, bn) || !is_pow2(bk) || bk < 16 || bk > 128)
    return bad(MI_E_TILE, "block_m, block_n must be powers of two in [32, 512] and block_k in [16, 128]");
  if (wave_rules(bm, bn, waves).code != MI_OK) return wave_rules(bm, bn, waves);
  if (stages < 1 || stages > 2) return bad(MI_E_TILE, "this variant takes 1 or 2 LDS stages");
  if (!mn_panel_ok(bk, bm) || !mn_panel_ok(bk, bn)) return bad(MI_E_TILE, "a K panel is smaller than one 1 KiB wave load");
  if (lds_mm_plain(bm, bn, bk, waves, stages) > kLdsBytesMax) return bad(MI_E_LDS, "LDS over 160 KiB");
  return ok();
}

// ---- pipelined core: lhsT.rhs variants 1 / 3, lhs.rhs variants 0 / 2, and
// the main pass of the two-pass fused kernel (variant 13).  ak: the A panel
// is K-contiguous (lhs[M,K]).
MI_HD constexpr int lds_mm_pipe(int bm, int bn, int bk, int waves, int stages) {
  return cmax(stages * (bk * bm * 2 + bk * bn * 2), epilogue_bytes(bm, bn, waves));
}
MI_HD constexpr Legal legal_mm_pipe(int bm, int bn, int bk, int waves, int stages, bool ak) {
  if (!block_mn_ok(bm, bn) || !is_pow2(bk) || bk < 32 || bk > 128)
    return bad(MI_E_TILE, "block_m, block_n must be powers of two in [32, 512] and block_k in [32, 128]");
  if (wave_rules(bm, bn, waves).code != MI_OK) return wave_rules(bm, bn, waves);
  if (stages < 2 || stages > 4) return bad(MI_E_TILE, "this variant takes 2..4 LDS stages");
  const bool a_ok = ak ? k_panel_ok(bk, bm) : mn_panel_ok(bk, bm);
  if (!a_ok || !mn_panel_ok(bk, bn)) return bad(MI_E_TILE, "a K panel is smaller than one 1 KiB wave load");
  const bool a_even = ak ? k_panel_even(bk, bm, waves) : mn_panel_even(bk, bm, waves);
  // Deeper rings wait with vmcnt counts that assume equal load groups.
  if (stages > 2 && !(a_even && mn_panel_even(bk, bn, waves)))
    return bad(MI_E_TILE, "more than 2 stages need every wave to issue the same number of panel loads");
  const int lpt = (ak ? k_panel_loads(bk, bm, waves) : mn_panel_loads(bk, bm, waves)) + mn_panel_loads(bk, bn, waves);
  if ((stages - 1) * lpt >= 64) return bad(MI_E_TILE, "loads in flight exceed the 6-bit vmcnt");
  if (lds_mm_pipe(bm, bn, bk, waves, stages) > kLdsBytesMax) return bad(MI_E_LDS, "LDS over 160 KiB");
  return ok();
}

// ---- pipelined core with each K tile's 16-deep sub-steps split over the
// waves (lhsT.rhs variant 4): every wave accumulates the whole block over
// its own sub-steps, so it holds BM*BN/64 fp32 accumulators per lane, and
// the epilogue sums the waves' blocks through LDS one 32-row slice at a time
// (WAVES slots of 32 rows, row stride BN*4+16 bytes).
MI_HD constexpr int lds_mm_kw(int bm, int bn, int bk, int waves, int stages) {
  return cmax(stages * (bk * bm * 2 + bk * bn * 2), waves * 32 * (bn * 4 + 16));
}
MI_HD constexpr Legal legal_mm_kw(int bm, int bn, int bk, int waves, int stages) {
  if (!block_mn_ok(bm, bn) || !is_pow2(bk) || bk < 32 || bk > 128)
    return bad(MI_E_TILE, "block_m, block_n must be powers of two in [32, 512] and block_k in [32, 128]");
  if (!waves_ok(waves) || (bk / 16) % waves != 0)
    return bad(MI_E_WAVE_TILE, "the waves must split a K tile's block_k/16 sub-steps evenly");
  if (bm * bn / 64 * ((waves + 3) / 4) > 256)
    return bad(MI_E_WAVE_TILE, "each wave's accumulators (the whole block) exceed its share of the 512 registers");
  if (stages < 2 || stages > 4) return bad(MI_E_TILE, "this variant takes 2..4 LDS stages");
  // Operand registers alternate between two buffers across the ring.
  if ((stages * (bk / 16 / waves)) % 2 != 0)
    return bad(MI_E_TILE, "an odd number of sub-steps per wave needs an even number of LDS stages");
  if (!mn_panel_ok(bk, bm) || !mn_panel_ok(bk, bn)) return bad(MI_E_TILE, "a K panel is smaller than one 1 KiB wave load");
  if (stages > 2 && !(mn_panel_even(bk, bm, waves) && mn_panel_even(bk, bn, waves)))
    return bad(MI_E_TILE, "more than 2 stages need every wave to issue the same number of panel loads");
  if ((stages - 1) * (mn_panel_loads(bk, bm, waves) + mn_panel_loads(bk, bn, waves)) >= 64)
    return bad(MI_E_TILE, "loads in flight exceed the 6-bit vmcnt");
  if (lds_mm_kw(bm, bn, bk, waves, stages) > kLdsBytesMax) return bad(MI_E_LDS, "LDS over 160 KiB");
  return ok();
}

// ---- main pass of the two-pass fused kernel (rmsnorm_matmul variant 13):
// the pipelined lhsT.rhs core plus the block's BM row scales in LDS.
MI_HD constexpr int lds_rms2(int bm, int bn, int bk, int waves, int stages) {
  return lds_mm_pipe(bm, bn, bk, waves, stages) + bm * 4;
}
MI_HD constexpr Legal legal_rms2(int bm, int bn, int bk, int waves, int stages) {
  const Legal core = legal_mm_pipe(bm, bn, bk, waves, stages, false);
  if (core.code != MI_OK) return core;
  if (lds_rms2(bm, bn, bk, waves, stages) > kLdsBytesMax) return bad(MI_E_LDS, "LDS over 160 KiB");
  return ok();
}

// ---- lhsT.rhs with a register prefetch ring (matmul variant 2); `stages`
// is the ring depth, the LDS holds two stages.
MI_HD constexpr int lds_mm_reg(int bm, int bn, int bk, int waves) {
  return cmax(2 * (bk * bm * 2 + bk * bn * 2), epilogue_bytes(bm, bn, waves));
}
MI_HD constexpr Legal legal_mm_reg(int bm, int bn, int bk, int waves, int ring) {
  if (!block_mn_ok(bm, bn) || !is_pow2(bk) || bk < 32 || bk > 128)
    return bad(MI_E_TILE, "block_m, block_n must be powers of two in [32, 512] and block_k in [32, 128]");
  if (wave_rules(bm, bn, waves).code != MI_OK) return wave_rules(bm, bn, waves);
  if (ring < 1 || ring > 8) return bad(MI_E_TILE, "the register ring holds 1..8 K tiles (lds_stages)");
  const int nt = waves * 64;
  // Every thread owns the same number of 16-byte pieces of each panel.
  if ((bk * bm * 2 / 16) % nt || (bk * bn * 2 / 16) % nt || bk * bm * 2 / 16 < nt || bk * bn * 2 / 16 < nt)
    return bad(MI_E_TILE, "a K panel does not split evenly into 16-byte pieces per thread");
  if (lds_mm_reg(bm, bn, bk, waves) > kLdsBytesMax) return bad(MI_E_LDS, "LDS over 160 KiB");
  return ok();
}

// ---- lhs.rhs with the A panel loaded two K tiles at a time (lhs.rhs
// variant 1).
MI_HD constexpr int lds_lhs_pair(int bm, int bn, int bk, int waves, int stages) {
  return cmax(((stages + 2) / 2) * (bm * 2 * bk * 2) + stages * (bk * bn * 2), epilogue_bytes(bm, bn, waves));
}
MI_HD constexpr Legal legal_lhs_pair(int bm, int bn, int bk, int waves, int stages) {
  if (!block_mn_ok(bm, bn) || (bk != 32 && bk != 64))
    return bad(MI_E_TILE, "block_m, block_n must be powers of two in [32, 512] and block_k 32 or 64");
  if (wave_rules(bm, bn, waves).code != MI_OK) return wave_rules(bm, bn, waves);
  if (stages < 2 || stages > 4) return bad(MI_E_TILE, "this variant takes 2..4 LDS stages");
  if (!k_panel_ok(2 * bk, bm) || !mn_panel_ok(bk, bn)) return bad(MI_E_TILE, "a K panel is smaller than one 1 KiB wave load");
  if (!k_panel_even(2 * bk, bm, waves) || !mn_panel_even(bk, bn, waves))
    return bad(MI_E_TILE, "every wave must issue the same number of panel loads");
  if (lds_lhs_pair(bm, bn, bk, waves, stages) > kLdsBytesMax) return bad(MI_E_LDS, "LDS over 160 KiB");
  return ok();
}

// ---- main pass of the two-pass fused kernel on the paired-load core
// (rmsnorm_matmul variant 15): the matmul_lhs_rhs variant-1 core plus BM
// row scales in LDS.
MI_HD constexpr int lds_rms2_pair(int bm, int bn, int bk, int waves, int stages) {
  return lds_lhs_pair(bm, bn, bk, waves, stages) + bm * 4;
}
MI_HD constexpr Legal legal_rms2_pair(int bm, int bn, int bk, int waves, int stages) {
  const Legal core = legal_lhs_pair(bm, bn, bk, waves, stages);
  if (core.code != MI_OK) return core;
  if (lds_rms2_pair(bm, bn, bk, waves, stages) > kLdsBytesMax) return bad(MI_E_LDS, "LDS over 160 KiB");
  return ok();
}

// ---- fused kernel, x scaled while staged (rmsnorm_matmul variants 0 / 1):
// x rows are reduced over BK/8 lanes (4, 8 or 16).
MI_HD constexpr int lds_rms_plain(int bm, int bn, int bk, int waves, int stages) {
  return (cmax(stages * (bm * bk * 2 + bk * bn * 2), epilogue_bytes(bm, bn, waves)) + 15) / 16 * 16 + bm * 4;
}
MI_HD constexpr Legal legal_rms_plain(int bm, int bn, int bk, int waves, int stages) {
  if (!block_mn_ok(bm, bn) || (bk != 32 && bk != 64 && bk != 128))
    return bad(MI_E_TILE, "block_m, block_n must be powers of two in [32, 512] and block_k 32, 64 or 128");
  if (wave_rules(bm, bn, waves).code != MI_OK) return wave_rules(bm, bn, waves);
  if (stages < 1 || stages > 2) return bad(MI_E_TILE, "this variant takes 1 or 2 LDS stages");
  if (!mn_panel_ok(bk, bn)) return bad(MI_E_TILE, "the W panel is smaller than one 1 KiB wave load");
  if (lds_rms_plain(bm, bn, bk, waves, stages) > kLdsBytesMax) return bad(MI_E_LDS, "LDS over 160 KiB");
  return ok();
}

// ---- fused kernel, x through a register ring of xs tiles on the pipelined
// core (rmsnorm_matmul variants 4 / 5 / 11 / 12).  gamma is staged in LDS as
// fp32 in whatever room the panels leave, at most 8192 entries, in whole K
// tiles.
MI_HD constexpr int xreg_gamma_offset(int bm, int bn, int bk, int waves, int stages) {
  return (cmax(stages * (bm * bk * 2 + bk * bn * 2), epilogue_bytes(bm, bn, waves)) + 15) / 16 * 16 + bm * 4;
}
MI_HD constexpr int xreg_gamma_kmax(int bm, int bn, int bk, int waves, int stages) {
  const int fit = (kLdsBytesMax - xreg_gamma_offset(bm, bn, bk, waves, stages)) / 4 / bk * bk;
  return fit < 8192 ? fit : 8192;
}
MI_HD constexpr int lds_rms_xreg(int bm, int bn, int bk, int waves, int stages) {
  return xreg_gamma_offset(bm, bn, bk, waves, stages) + xreg_gamma_kmax(bm, bn, bk, waves, stages) * 4;
}
MI_HD constexpr Legal legal_rms_xreg(int bm, int bn, int bk, int waves, int stages, int xs) {
  if (!block_mn_ok(bm, bn) || (bk != 32 && bk != 64 && bk != 128))
    return bad(MI_E_TILE, "block_m, block_n must be powers of two in [32, 512] and block_k 32, 64 or 128");
  if (wave_rules(bm, bn, waves).code != MI_OK) return wave_rules(bm, bn, waves);
  if (stages < 2 || stages > 4 || (xs != 2 && xs != 3))
    return bad(MI_E_TILE, "this variant takes 2..4 LDS stages and a 2- or 3-tile x ring");
  const int nt = waves * 64, kc = bk / 8, chunks = bm * kc;
  if (chunks % nt || chunks < nt || nt % kc) return bad(MI_E_TILE, "x chunks do not split evenly over the threads");
  if (!mn_panel_ok(bk, bn) || !mn_panel_even(bk, bn, waves))
    return bad(MI_E_TILE, "every wave must issue the same number of W panel loads");
  const int nlb = mn_panel_loads(bk, bn, waves), nlx = chunks / nt;
  if ((xs - 1) * (nlb + nlx) >= 64 || nlx + (stages - 2) * (nlb + nlx) >= 64)
    return bad(MI_E_TILE, "loads in flight exceed the 6-bit vmcnt");
  if (xreg_gamma_offset(bm, bn, bk, waves, stages) > kLdsBytesMax) return bad(MI_E_LDS, "LDS over 160 KiB");
  if (xreg_gamma_kmax(bm, bn, bk, waves, stages) < bk) return bad(MI_E_LDS, "no LDS left for one K tile of gamma");
  return ok();
}

}  // namespace mi
