// mi_rms_direct.hpp -- fused rmsnorm_matmul with the x operand loaded
// straight into MFMA registers (rmsnorm_matmul variants 6..9).
//
//   out[M,N] = (x[M,K] * rsqrt(mean_k x^2 + eps) * gamma[K]) . W[K,N]
//
// x is K-contiguous, which is already the MFMA operand layout: lane l of a
// 32x32x16 fragment holds row l%32, K 8*(l/32) .. +8, i.e. 16 contiguous
// bytes of x.  So the x operand never touches LDS: every wave buffer-loads
// its own x fragments (a ring of D K tiles in registers), and LDS carries
// only the W panel (LDS-direct loads into a STAGES ring, read with the
// transposing ds_read_b64_tr_b16) and the gamma vector.  Per K tile and
// workgroup the LDS moves the W panel once in and WN*... out -- less than
// half of what the LDS-staged variants move, which is what bounds them.
//
// gamma multiplies the W fragments after they are read (the B operand of a
// wave is the smaller one), so x reaches the MFMA as loaded; the row sums
// of squares come from the same x registers, each x fragment summed by one
// of the WN waves that share it; 1/rms scales the fp32 accumulators in the
// epilogue (out row m = inv_rms[m] * (x . gamma*W)[m]).
//
// Loads are inline asm (the compiler inserts no vmcnt waits): at the end
// of tile t each thread issues its W loads of tile t+STAGES (at the tile
// barrier) and then its x loads of tile t+D, so with LB W loads and LA x
// loads per tile the number of younger loads that may still fly is
//   x(t+1), waited for at the end of tile t:    (D-1) * (LB + LA)
//   W(t+1), waited for at the barrier of tile t: LA + (STAGES-2) * (LB + LA)
// and after each wait the loaded registers pass through an empty asm so no
// use is scheduled before it.
#pragma once
#include <type_traits>

#include "mi_gemm.hpp"
#include "mi_rms_xreg.hpp"

namespace mi {

// Wave grid with a forced number of wave rows (WMX = 0: the squarest one).
template <int BM, int BN, int WAVES, int WMX>
struct WaveGridX {
  using Auto = WaveGrid<BM, BN, WAVES>;
  static constexpr int WM = WMX > 0 ? WMX : Auto::WM;
  static constexpr int WN = WAVES / WM;
  static constexpr bool ok = WM > 0 && WM * WN == WAVES && BM % (32 * WM) == 0 && BN % (32 * WN) == 0;
  static constexpr int WTM = BM / WM;
  static constexpr int WTN = BN / WN;
  static constexpr int TM = WTM / 32;
  static constexpr int TN = WTN / 32;
};

template <int BM, int BN, int BK, int WAVES, int STAGES, int WMX>
struct DirectCfg {
  using G = WaveGridX<BM, BN, WAVES, WMX>;
  static constexpr int B_BYTES = BK * BN * 2;        // W panel, N contiguous, mn_swz
  static constexpr int MAIN_BYTES = STAGES * B_BYTES;
  static constexpr int EPI_BYTES = WAVES * 32 * (G::WTN * 2 + 16);
  static constexpr int G_OFF = ((MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES) + 15) / 16 * 16;
  static constexpr int GK_MAX = 16384;               // gamma entries staged in LDS (K rounded up to D*BK)
  static constexpr int RMS_OFF = G_OFF + GK_MAX * 2;
  static constexpr int LDS_BYTES = RMS_OFF + BM * 4;
};

template <int BM, int BN, int BK, int WAVES, int STAGES, int WMX, int D, bool HG>
__global__ __launch_bounds__(WAVES * 64) void rmsnorm_mm_bf16_direct_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ out, int M, int N, int K, float inv_k, float eps, int group_m) {
  using C = DirectCfg<BM, BN, BK, WAVES, STAGES, WMX>;
  using G = typename C::G;
  static_assert(G::ok, "illegal wave grid");
  static_assert(BK % 32 == 0, "BK must be a multiple of 32 (even number of MFMA K steps)");
  static_assert(STAGES >= 2 && STAGES <= 4, "2..4 LDS stages");
  static_assert(D == 2 || D == 3, "2 or 3 x tiles in registers");
  constexpr int TM = G::TM, TN = G::TN, KS = BK / 16, WN = G::WN;
  using LB = PanelLoader<BK, BN, WAVES>;
  static_assert(LB::EVEN, "every wave issues the same number of W loads");
  constexpr int NLB = LB::LOADS_PER_TILE;
  constexpr int NLA = TM * KS;
  constexpr int A_WAIT = (D - 1) * (NLB + NLA);
  constexpr int B_WAIT = NLA + (STAGES - 2) * (NLB + NLA);
  static_assert(A_WAIT < 64 && B_WAIT < 64, "vmcnt is 6 bits");
  __shared__ __attribute__((aligned(1024))) char smem[HG ? C::LDS_BYTES : C::G_OFF + BM * 4];
  float* rms_lds = (float*)(smem + (HG ? C::RMS_OFF : C::G_OFF));

  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tmi, tni;
  tile_coords(tiles_m, tiles_n, group_m, tmi, tni);
  const int m0 = tmi * BM, n0 = tni * BN;
  const int wmi = wave / WN, wn = wave % WN;
  const int wm0 = wmi * G::WTM;
  const int wn0 = wn * G::WTN;

  const uint32_t x_bytes = (uint32_t)M * (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, x_bytes);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)K * (uint32_t)N * 2u);
  const int KT = (K + BK - 1) / BK;
  const int KTP = (KT + D - 1) / D * D;  // tiles walked: KT rounded up to D
  auto clamp = [&](int kt) { return kt < KT ? kt : KT - 1; };

  // gamma -> LDS (zeros past K, up to the last tile), with ordinary loads,
  // before any asynchronous load is issued.
  if constexpr (HG) {
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(gamma, (uint32_t)K * 2u);
    for (int c = tid; c < KTP * BK / 8; c += WAVES * 64)
      *(MI_LDS u32x4_t*)((MI_LDS char*)smem + C::G_OFF + 16 * c) =
          __builtin_amdgcn_raw_buffer_load_b128(rg, 16u * (uint32_t)c, 0, 0);
  }

  // ---- x fragments: fragment (i, kk) of lane l is row m0+wm0+32i+l%32,
  // K kt*BK + 16kk + 8(l/32) .. +8.  Chunks past K read zeros.
  const int khalf = 8 * (lane >> 5);
  uint32_t arow[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i)
    arow[i] = ((uint32_t)(m0 + wm0 + 32 * i + (lane & 31)) * (uint32_t)K + (uint32_t)khalf) * 2u;
  u32x4_t ar[D][TM][KS];
  auto issue_a = [&](int kt, auto slot_c) {
    constexpr int P = decltype(slot_c)::value;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int k = kt * BK + 16 * kk;
      const bool kin = k + khalf < K;
#pragma unroll
      for (int i = 0; i < TM; ++i) ar[P][i][kk] = vload16(rx, kin ? arow[i] + 2u * (uint32_t)k : x_bytes);
    }
  };
  auto a_ready = [&](auto slot_c) {
    constexpr int P = decltype(slot_c)::value;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) reg_ready(ar[P][i][kk]);
  };

  LB lb;
  lb.init(wave, lane, n0, N);
  const uint32_t kstep_b = (uint32_t)BK * (uint32_t)N * 2u;
  TrFrag<BN, TN> fb;
  fb.init(lane, wn0);
  bf16x8_t bf[2][TN];
  auto read_b = [&](int stage, int kk, int buf, int j) {
    const int bbase = stage * C::B_BYTES;
    bf[buf][j] =
        read_tr_frag(smem, bbase + (kk * 16) * (BN * 2) + fb.off[j], bbase + (kk * 16 + 4) * (BN * 2) + fb.off[j]);
  };
  auto read_bs = [&](int stage, int kk, int buf) {
#pragma unroll
    for (int j = 0; j < TN; ++j) read_b(stage, kk, buf, j);
  };

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16_t{};
  // Sums of squares: fragment row group i is summed by wave column i % WN.
  constexpr int SPW = (TM + WN - 1) / WN;
  float ssq[SPW];
#pragma unroll
  for (int s = 0; s < SPW; ++s) ssq[s] = 0.0f;

  // One MFMA K sub-step of tile kt: gamma-scale the W fragments, add the
  // squares of this wave's share of x, then MFMAs of rows [i0, i1).
  bf16x8_t bsc[TN];
  auto prep = [&](int kt, int kk, int buf, auto slot_c) {
    constexpr int P = decltype(slot_c)::value;
    if constexpr (HG) {
      const u32x4_t g =
          *(MI_LDS u32x4_t*)((MI_LDS char*)smem + C::G_OFF + 2 * (kt * BK + 16 * kk + khalf));
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const u32x4_t b = __builtin_bit_cast(u32x4_t, bf[buf][j]);
        u32x4_t o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(bf16lo(b[e]) * bf16lo(g[e]), bf16hi(b[e]) * bf16hi(g[e]));
        bsc[j] = __builtin_bit_cast(bf16x8_t, o);
      }
    } else {
#pragma unroll
      for (int j = 0; j < TN; ++j) bsc[j] = bf[buf][j];
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
      if (i % WN == wn) ssq[i / WN] = sum_sq_chunk(ar[P][i][kk], ssq[i / WN]);
  };
  auto mfma_rows = [&](int kk, auto slot_c, int i0, int i1) {
    constexpr int P = decltype(slot_c)::value;
#pragma unroll
    for (int i = i0; i < i1; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bsc[j], __builtin_bit_cast(bf16x8_t, ar[P][i][kk]),
                                                            acc[i][j], 0, 0, 0);
  };
  constexpr int VPS = (HG ? 20 * TN : 0) + 16 * SPW;  // VALU per sub-step
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2 % D>;
  auto issue_a_tile = [&](int j) {
    if (j % D == 0) issue_a(j, S0{});
    else if (j % D == 1) issue_a(j, S1{});
    else issue_a(j, S2{});
  };

  // ---- prologue: W(0 .. STAGES-1) and x(0 .. D-1), in the steady-state
  // group order (W(u+STAGES), x(u+D) for u = -max(STAGES, D) .. -1), all
  // drained before tile 0 (so the steady-state counts hold from there on),
  // and gamma is published by the barrier.
  constexpr int U0 = STAGES > D ? STAGES : D;
#pragma unroll
  for (int u = -U0; u <= -1; ++u) {
    const int wj = u + STAGES, xj = u + D;
    if (wj >= 0) lb.issue(rw, smem, wj * C::B_BYTES, kstep_b, clamp(wj));
    if (xj >= 0) issue_a_tile(xj);
  }
  wait_vmem();
  a_ready(S0{});
  __syncthreads();
  read_bs(0, 0, 0);

  int cur = 0;
  auto tile = [&](int t, auto slot_c, auto next_c) {
    const int nxt = cur + 1 == STAGES ? 0 : cur + 1;
#pragma unroll
    for (int kk = 0; kk + 1 < KS; ++kk) {
      read_bs(cur, kk + 1, (kk + 1) & 1);
      prep(t, kk, kk & 1, slot_c);
      mfma_rows(kk, slot_c, 0, TM);
      interleave_mfma_mix<TM * TN, 2 * TN + (HG ? 1 : 0), VPS, 0>();
    }
    prep(t, KS - 1, (KS - 1) & 1, slot_c);
    mfma_rows(KS - 1, slot_c, 0, TM / 2);
    interleave_mfma_mix<(TM / 2) * TN, HG ? 1 : 0, VPS, 0>();
    vm_wait<B_WAIT>();  // this wave's W(t+1) landed
    __syncthreads();    // everyone's W(t+1) landed, nobody reads stage cur any more
    const int kw = clamp(t + STAGES);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      read_b(nxt, 0, 0, j);
#pragma unroll
      for (int q = j * NLB / TN; q < (j + 1) * NLB / TN; ++q)
        lb.issue_one(q, rw, smem, cur * C::B_BYTES, kstep_b, kw);
    }
    mfma_rows(KS - 1, slot_c, TM / 2, TM);
    interleave_mfma_ds<(TM - TM / 2) * TN, 2 * TN>();
    // Every MFMA reading slot t%D is issued: refill it with x(t+D), then
    // wait for x(t+1).
    issue_a(t + D, slot_c);
    vm_wait<A_WAIT>();
    a_ready(next_c);
    cur = nxt;
  };
  // Last tile: no loads, no barrier.
  auto last = [&](int t, auto slot_c) {
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      if (kk + 1 < KS) read_bs(cur, kk + 1, (kk + 1) & 1);
      prep(t, kk, kk & 1, slot_c);
      mfma_rows(kk, slot_c, 0, TM);
      interleave_mfma_mix<TM * TN, 2 * TN + (HG ? 1 : 0), VPS, 0>();
    }
  };
  // Unrolled D times so that slot indices are compile-time constants: tile
  // t + s of a round reads slot s and waits for slot (s+1)%D.  The tile
  // count is padded to a multiple of D (padding tiles read x = 0 and add
  // nothing), so the last tile always reads slot D-1.
  int t = 0;
  if constexpr (D == 2) {
    for (; t + 2 < KTP; t += 2) {
      tile(t, S0{}, S1{});
      tile(t + 1, S1{}, S0{});
    }
    tile(t, S0{}, S1{});
    last(t + 1, S1{});
  } else {
    for (; t + 3 < KTP; t += 3) {
      tile(t, S0{}, S1{});
      tile(t + 1, S1{}, S2{});
      tile(t + 2, S2{}, S0{});
    }
    tile(t, S0{}, S1{});
    tile(t + 1, S1{}, S2{});
    last(t + 2, S2{});
  }
  wait_vmem();
  // x loads of tiles past the end were never consumed: keep their registers
  // allocated until the wait above has drained them.
  a_ready(S0{});
  a_ready(S1{});
  if constexpr (D == 3) a_ready(S2{});
  __syncthreads();  // the epilogue reuses the W buffers

  // Row sums: lanes l and l+32 hold the two K halves of row l%32.
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    if (i % WN == wn) {
      float r = ssq[i / WN];
      r += __shfl_xor(r, 32);
      if (lane < 32) rms_lds[wm0 + 32 * i + lane] = 1.0f / __builtin_sqrtf(r * inv_k + eps);
    }
  }
  __syncthreads();
  float scale[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) scale[i] = rms_lds[wm0 + 32 * i + (lane & 31)];
  store_tile<TM, TN, WAVES>(acc, scale, smem, wave, lane, out, M, N, m0 + wm0, n0 + wn0);
}

}  // namespace mi
