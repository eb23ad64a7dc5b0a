// mi_rms_xpair.hpp -- fused rmsnorm_matmul, x staged through registers two
// K tiles per load (rmsnorm_matmul variant 10).
//
//   out[M,N] = (x[M,K] * rsqrt(mean_k x^2 + eps) * gamma[K]) . W[K,N]
//
// Same pipeline as variants 4/5 (W panel by LDS-direct loads into a
// STAGES ring on the pipelined matmul core; x through registers, scaled by
// gamma into the K-contiguous A panel during the tile before its use), with
// the x loads reshaped for the memory system.  At BK = 32 an x row segment
// of one K tile is 64 bytes, half a 128-byte cache line, so loading x one
// tile at a time fetches every line twice.  Here one load instruction reads
// 8 rows x 128 bytes -- the x of K tiles 2u and 2u+1 ("pair" u) -- with
// lanes 0..31 on the first 64 bytes of each row and lanes 32..63 on the
// second.  One v_permlane32_swap per dword then regroups two such registers
// so that one holds tile 2u for 16 rows and the other tile 2u+1, and every
// lane scales a full chunk in both tiles.
//
//   pair u (x of tiles 2u, 2u+1) -> register slot u%2, issued at the barrier
//                                   that ends tile 2u-4
//   A(2u)   <- scaled from slot u%2 during tile 2u-1 (after the swap)
//   A(2u+1) <- scaled from slot u%2 during tile 2u
//   W(t)    -> stage t%STAGES, issued at the barrier that ends tile t-STAGES
//
// gamma is staged in LDS once, as fp32 (K up to 8192 after rounding).  1/rms scales
// the fp32 accumulators in the epilogue.  Loads are inline asm with explicit
// vmcnt waits: at barrier t each thread issues LB W loads, then (t even)
// LX x loads, so
//   pair u, waited for at the start of tile 2u-1:  2*LB + LX younger loads
//   W(t+1), waited for at barrier t:  (STAGES-2)*LB + floor((STAGES-1)/2)*LX
// (the second is exact for STAGES = 3; otherwise it may wait a little more
// than needed, never less).
#pragma once
#include <type_traits>

#include "mi_gemm.hpp"
#include "mi_rms_xreg.hpp"

namespace mi {

template <int BM, int BN, int BK, int WAVES, int STAGES>
struct XpairCfg {
  using G = WaveGrid<BM, BN, WAVES>;
  static constexpr int KC = BK / 8;                  // 16-byte chunks per x row per K tile
  static constexpr int CP = BM / (8 * WAVES);        // pair loads per wave (8 rows each)
  static constexpr int XD = (128 / BK) > 0 ? (128 / BK) : 1;
  static constexpr int A_BYTES = BM * BK * 2;        // scaled x panel, K contiguous, k_swz
  static constexpr int B_BYTES = BK * BN * 2;        // W panel, N contiguous, mn_swz
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int MAIN_BYTES = STAGES * STAGE_BYTES;
  static constexpr int EPI_BYTES = WAVES * 32 * (G::WTN * 2 + 16);
  static constexpr int G_OFF = ((MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES) + 15) / 16 * 16;
  static constexpr int GK_MAX = 8192;                // fp32 gamma entries staged in LDS (K rounded up to 4*BK)
  static constexpr int RMS_OFF = G_OFF + GK_MAX * 4;
  static constexpr int LDS_BYTES = RMS_OFF + BM * 4;
  static_assert(BK == 32, "pairs of 64-byte row segments fill 128-byte lines at BK = 32");
  static_assert(CP >= 2 && CP % 2 == 0, "pair loads are swapped two by two");
};

template <int BM, int BN, int BK, int WAVES, int STAGES, bool HG, int SSQ_PARTS = 4>
__global__ __launch_bounds__(WAVES * 64) void rmsnorm_mm_bf16_xpair_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ out, int M, int N, int K, float inv_k, float eps, int group_m) {
  using C = XpairCfg<BM, BN, BK, WAVES, STAGES>;
  using G = typename C::G;
  static_assert(G::ok, "illegal wave grid");
  static_assert(STAGES >= 3 && STAGES <= 4, "3..4 LDS stages");
  constexpr int TM = G::TM, TN = G::TN, KS = BK / 16, KC = C::KC, CP = C::CP, NH = CP / 2;
  using LB = PanelLoader<BK, BN, WAVES>;
  static_assert(LB::EVEN, "every wave issues the same number of W loads");
  constexpr int NLB = LB::LOADS_PER_TILE;
  constexpr int NLX = CP;
  constexpr int X_WAIT = 2 * NLB + NLX;
  constexpr int B_WAIT = (STAGES - 2) * NLB + ((STAGES - 1) / 2) * NLX;
  static_assert(X_WAIT < 64 && B_WAIT < 64, "vmcnt is 6 bits");
  __shared__ __attribute__((aligned(1024))) char smem[HG ? C::LDS_BYTES : C::G_OFF + BM * 4];
  float* rms_lds = (float*)(smem + (HG ? C::RMS_OFF : C::G_OFF));

  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tmi, tni;
  tile_coords(tiles_m, tiles_n, group_m, tmi, tni);
  const int m0 = tmi * BM, n0 = tni * BN;
  const int wm0 = (wave / G::WN) * G::WTM;
  const int wn0 = (wave % G::WN) * G::WTN;

  const uint32_t x_bytes = (uint32_t)M * (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, x_bytes);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)K * (uint32_t)N * 2u);
  const int KT = (K + BK - 1) / BK;
  const int KTP = (KT + 3) / 4 * 4;  // tiles walked: padding tiles read x = 0 and add nothing
  auto clamp = [&](int kt) { return kt < KT ? kt : KT - 1; };

  if constexpr (HG) {
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(gamma, (uint32_t)K * 2u);
    for (int c = tid; c < KTP * BK / 8; c += WAVES * 64) {
      const u32x4_t g = __builtin_amdgcn_raw_buffer_load_b128(rg, 16u * (uint32_t)c, 0, 0);
      MI_LDS float* d = (MI_LDS float*)((MI_LDS char*)smem + C::G_OFF) + 8 * c;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        d[2 * e] = bf16lo(g[e]);
        d[2 * e + 1] = bf16hi(g[e]);
      }
    }
  }

  // ---- x pair loads: load i of this wave covers rows 8*(wave*CP + i) .. +8;
  // lane l reads row +(l%32)/4, chunk l%4 of tile 2u (l < 32) or of 2u+1.
  const int kc = lane & 3;
  const int kpair = 8 * (kc + 4 * (lane >> 5));  // K offset inside the pair
  uint32_t xoff[CP];
#pragma unroll
  for (int i = 0; i < CP; ++i)
    xoff[i] = ((uint32_t)(m0 + 8 * (wave * CP + i) + ((lane & 31) >> 2)) * (uint32_t)K + (uint32_t)kpair) * 2u;
  // After the swap, register h of a tile (h < NH) holds, in every lane,
  // chunk kc of row xrow[h]: lanes 0..31 from load 2h, 32..63 from 2h+1.
  int xrow[NH], xlds[NH];
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    xrow[h] = 8 * (wave * CP + 2 * h + (lane >> 5)) + ((lane & 31) >> 2);
    xlds[h] = xrow[h] * (BK * 2) + 16 * (kc ^ k_swz<BK>(xrow[h]));
  }
  u32x4_t xr[2][CP];
  auto issue_x = [&](int q, int u, auto slot_c) {
    constexpr int P = decltype(slot_c)::value;
    const int k = u * 2 * BK + kpair;
    xr[P][q] = vload16(rx, k < K ? xoff[q] + 2u * (uint32_t)(u * 2 * BK) : x_bytes);
  };
  auto issue_pair = [&](int u, auto slot_c) {
#pragma unroll
    for (int q = 0; q < NLX; ++q) issue_x(q, u, slot_c);
  };
  auto x_ready = [&](auto slot_c) {
    constexpr int P = decltype(slot_c)::value;
#pragma unroll
    for (int q = 0; q < CP; ++q) reg_ready(xr[P][q]);
  };
  // Regroup: (load 2h, load 2h+1) -> (tile 2u rows, tile 2u+1 rows).
  auto swap_pair = [&](auto slot_c) {
    constexpr int P = decltype(slot_c)::value;
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const auto r = __builtin_amdgcn_permlane32_swap(xr[P][2 * h][e], xr[P][2 * h + 1][e], false, false);
        xr[P][2 * h][e] = r[0];
        xr[P][2 * h + 1][e] = r[1];
      }
  };

  LB lb;
  lb.init(wave, lane, n0, N);
  const uint32_t kstep_b = (uint32_t)BK * (uint32_t)N * 2u;
  auto issue_w = [&](int q, int kt, int stage) {
    lb.issue_one(q, rw, smem, stage * C::STAGE_BYTES + C::A_BYTES, kstep_b, kt);
  };
  TrFrag<BN, TN> fb;
  fb.init(lane, wn0);

  // ---- scaling: tile j (half H = j&1 of its pair, slot P) -> A panel of
  // `stage`; register h is scaled during MFMA sub-step h % KS.
  // Row sums of squares, NSA partial sums per owned chunk.
  constexpr int NSA = SSQ_PARTS;
  float ss[NH][NSA];
#pragma unroll
  for (int h = 0; h < NH; ++h)
#pragma unroll
    for (int a = 0; a < NSA; ++a) ss[h][a] = 0.0f;
  // gamma of tile j for this lane's K chunk (8 fp32): every register of a
  // tile shares it, so it is read once per tile.
  f32x4_t g0 = {}, g1 = {};
  auto gamma_of = [&](int j) {
    if constexpr (HG) {
      const MI_LDS f32x4_t* gp = (const MI_LDS f32x4_t*)((MI_LDS char*)smem + C::G_OFF + 4 * (j * BK + 8 * kc));
      g0 = gp[0];
      g1 = gp[1];
    }
  };
  auto scale_one = [&](int h, int H, auto slot_c, int stage) {
    constexpr int P = decltype(slot_c)::value;
    const u32x4_t o = scale_sumsq_chunk_f32g<NSA, HG>(xr[P][2 * h + H], g0, g1, ss[h]);
    *(MI_LDS u32x4_t*)((MI_LDS char*)smem + stage * C::STAGE_BYTES + xlds[h]) = o;
  };
  auto scale_step = [&](int s, int H, auto slot_c, int stage) {
#pragma unroll
    for (int h = s; h < NH; h += KS) scale_one(h, H, slot_c, stage);
  };
  constexpr int CPS = (NH + KS - 1) / KS;  // registers scaled per sub-step (at most)
  constexpr int VPC = HG ? 28 : 16;        // VALU per chunk (unpack, squares, scale, pack)

  // ---- MFMA operands (A: ds_read_b128 of 8 consecutive K of one row).
  const int xsl = ((lane & 31) / C::XD) & (KC - 1);
  const int arow = (wm0 + (lane & 31)) * (BK * 2);
  int akoff[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) akoff[kk] = 16 * ((2 * kk + (lane >> 5)) ^ xsl);
  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16_t{};
  bf16x8_t af[2][TM], bf[2][TN];
  constexpr int NF = TM + TN;
  auto read_frag = [&](int stage, int kk, int buf, int f) {
    const int abase = stage * C::STAGE_BYTES;
    const int bbase = abase + C::A_BYTES;
    if (f == 0 || f > TN) {
      const int t = f == 0 ? 0 : f - TN;
      af[buf][t] = __builtin_bit_cast(
          bf16x8_t, *(MI_LDS u32x4_t*)((MI_LDS char*)smem + abase + arow + t * 32 * (BK * 2) + akoff[kk]));
    } else {
      const int t = f - 1;
      bf[buf][t] = read_tr_frag(smem, bbase + (kk * 16) * (BN * 2) + fb.off[t],
                                bbase + (kk * 16 + 4) * (BN * 2) + fb.off[t]);
    }
  };
  auto read_frags = [&](int stage, int kk, int buf) {
#pragma unroll
    for (int f = 0; f < NF; ++f) read_frag(stage, kk, buf, f);
  };
  auto mfma_rows = [&](int buf, int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[buf][j], af[buf][i], acc[i][j], 0, 0, 0);
  };
  constexpr int ND = TM + 2 * TN;  // LDS reads per sub-step (a B fragment takes two)
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;

  // ---- prologue: barriers u = -4 .. -1 issue W(u+STAGES) (if >= 0) and,
  // at even u, pair u/2+2; all drained, then A(0) is scaled.
#pragma unroll
  for (int u = -4; u <= -1; ++u) {
    const int wj = u + STAGES;
    if (wj >= 0) {
#pragma unroll
      for (int q = 0; q < NLB; ++q) issue_w(q, clamp(wj), wj);
    }
    if (u == -4) issue_pair(0, S0{});
    if (u == -2) issue_pair(1, S1{});
  }
  wait_vmem();
  x_ready(S0{});
  x_ready(S1{});
  __syncthreads();  // gamma in LDS
  swap_pair(S0{});
  gamma_of(0);
#pragma unroll
  for (int s = 0; s < KS; ++s) scale_step(s, 0, S0{}, 0);
  __syncthreads();
  read_frags(0, 0, 0);

  // ---- steady state, four tiles per round (R = t % 4):
  //   R = 0: scale A(t+1) = second half of pair t/2 (slot 0); barrier issues pair t/2+2 -> slot 0
  //   R = 1: wait + swap pair (t+1)/2 (slot 1); scale A(t+1), first half
  //   R = 2: scale A(t+1), second half (slot 1); barrier issues pair t/2+2 -> slot 1
  //   R = 3: wait + swap pair (t+1)/2 (slot 0); scale A(t+1), first half
  int cur = 0;
  auto tile = [&](int t, auto r_c) {
    constexpr int R = decltype(r_c)::value;
    using SP = std::integral_constant<int, (R == 0 || R == 3) ? 0 : 1>;
    constexpr int H = (R == 0 || R == 2) ? 1 : 0;
    constexpr bool ISSUE = R == 0 || R == 2;
    const int nxt = cur + 1 == STAGES ? 0 : cur + 1;
    // The wait sits at the top of the tile so that the scaling VALU, the
    // operand reads and the MFMAs of each sub-step share one scheduling
    // region (an asm statement ends a region); the LDS writes are left
    // unplaced so that each follows its own VALU chain.
    if constexpr (H == 0) {
      vm_wait<X_WAIT>();
      x_ready(SP{});
    }
    gamma_of(t + 1);
#pragma unroll
    for (int kk = 0; kk + 1 < KS; ++kk) {
      read_frags(cur, kk + 1, (kk + 1) & 1);
      if (kk == 0 && H == 0) swap_pair(SP{});
      scale_step(kk, H, SP{}, nxt);
      mfma_rows(kk & 1, 0, TM);
      interleave_mfma_mix<TM * TN, ND + (HG ? 2 : 0), CPS * VPC + (H == 0 ? 4 * NH : 0), 0>();
    }
    scale_step(KS - 1, H, SP{}, nxt);
    mfma_rows((KS - 1) & 1, 0, TM / 2);
    interleave_mfma_mix<(TM / 2) * TN, 0, CPS * VPC, 0>();
    vm_wait<B_WAIT>();  // this wave's W(t+1) landed
    __syncthreads();    // every wave's W(t+1) and A(t+1) are in LDS
    const int kw = clamp(t + STAGES);
    constexpr int NI = NLB + (ISSUE ? NLX : 0);
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      read_frag(nxt, 0, 0, f);
#pragma unroll
      for (int q = f * NI / NF; q < (f + 1) * NI / NF; ++q) {
        if (q < NLB) issue_w(q, kw, cur);
        else if constexpr (ISSUE) issue_x(q - NLB, t / 2 + 2, SP{});
      }
    }
    mfma_rows((KS - 1) & 1, TM / 2, TM);
    interleave_mfma_ds<(TM - TM / 2) * TN, ND>();
    cur = nxt;
  };
  using R0 = std::integral_constant<int, 0>;
  using R1 = std::integral_constant<int, 1>;
  using R2 = std::integral_constant<int, 2>;
  using R3 = std::integral_constant<int, 3>;
  int t = 0;
  for (; t + 4 < KTP; t += 4) {
    tile(t, R0{});
    tile(t + 1, R1{});
    tile(t + 2, R2{});
    tile(t + 3, R3{});
  }
  tile(t, R0{});
  tile(t + 1, R1{});
  tile(t + 2, R2{});
  // Last tile (R = 3): nothing left to scale or load.
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    if (kk + 1 < KS) read_frags(cur, kk + 1, (kk + 1) & 1);
    mfma_rows(kk & 1, 0, TM);
    interleave_mfma_ds<TM * TN, ND>();
  }
  wait_vmem();
  // Pairs past the end were never consumed: keep their registers allocated
  // until the wait above has drained them.
  x_ready(S0{});
  x_ready(S1{});
  __syncthreads();  // the epilogue reuses the panel buffers

#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const float r = row_allreduce<KC>(sum_parts<NSA>(ss[h]));
    if (kc == 0) rms_lds[xrow[h]] = 1.0f / __builtin_sqrtf(r * inv_k + eps);
  }
  __syncthreads();
  float scale[TM];
#pragma unroll
  for (int mt = 0; mt < TM; ++mt) scale[mt] = rms_lds[wm0 + mt * 32 + (lane & 31)];
  store_tile<TM, TN, WAVES>(acc, scale, smem, wave, lane, out, M, N, m0 + wm0, n0 + wn0);
}

}  // namespace mi
