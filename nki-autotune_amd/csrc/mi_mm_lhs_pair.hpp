// mi_mm_lhs_pair.hpp -- matmul_lhs_rhs variant 1: the pipelined core with
// the K-contiguous A panel fetched two K tiles at a time.
//
//   out[M,N] = lhs[M,K] . rhs[K,N]   (lhs row-major, K contiguous)
//
// One K tile of a K-contiguous panel is BK*2 bytes of each of BM rows.  With
// BK = 32 that is half of a 128-byte line per row, and the vector L1 sends
// one request per half line, so the A side of a tile costs twice the L2
// requests of the same bytes in the lhsT layout (measured: +50 % L1->L2
// read requests and +12..19 % time for the per-tile variant 0).  Here each
// A load covers K tiles 2u and 2u+1 together -- whole lines, the same bytes
// -- into a pair buffer whose rows hold both tiles (row stride 4*BK bytes,
// 16-byte chunks XOR-swizzled by k_swz<2*BK>); B keeps its per-tile ring:
//
//   B(j)         -> stage j % STAGES, issued at the barrier that ends tile
//                   j - STAGES (with A(j, j+1) when j is even)
//   A(2u, 2u+1)  -> pair buffer u % NP
//
// Pair u's buffer is reused by pair u + NP, issued at the barrier ending
// tile 2u + 2*NP - STAGES; tile 2u+1 has been consumed by then when
// NP = (STAGES + 2) / 2.  At the barrier that ends tile t the wave waits for
// tile t+1: its B loads, and its A loads, which are issued in the same group
// (t+1 even, after the B loads) or one group earlier (t+1 odd).  The groups
// of barriers t+2-STAGES .. t-1 may still fly: (STAGES-2) B groups plus one
// A pair for every even tile among t+2 .. t+STAGES-1.  The loop is unrolled
// over lcm(STAGES, 2*NP) tiles, so stage, pair buffer, tile half and wait
// counts are compile-time constants in every tile body.
//
// SQ (rmsnorm_matmul variant 16, the fused product without gamma on this
// core, as variant 14 is on the per-tile core): x is the A operand, loaded
// unscaled, and each wave also sums its rows' squares from the A fragments
// its MFMAs consume (v_dot2c_f32_bf16: exact bf16 products, fp32 sums).
// Sub-step s = t*KS + kk of the K loop goes to wave column s % WN; a round
// holds a multiple of WN sub-steps, so inside the unrolled round the choice
// is a compile-time constant, and the K loop is compiled once per wave
// column.  The epilogue adds the wave columns' sums through LDS and scales
// output row m by 1/sqrt(sum_m / K + eps).
//
// RS (rmsnorm_matmul variant 15, the main pass of the two-pass fused kernel
// on this core, mi_rms_2pass.hpp): the A operand is the packed xg =
// bf16(x * gamma), and the rows' sums of squares come from the pack as
// partial sums ssq[p][m].  Each workgroup loads the first partial sums of
// its rows before the prologue's panel loads, adds them in part order after
// the prologue's wait, keeps 1/sqrt(sum / K + eps) per row in LDS past the
// panel buffers, and its epilogue scales output row m by it (the same steps
// as the lhsT core's row scale in mi_gemm.hpp).
#pragma once
#include <numeric>

#include "mi_gemm.hpp"

namespace mi {

template <int BM, int BN, int BK, int WAVES, int STAGES>
struct PairCfg {
  using G = WaveGrid<BM, BN, WAVES>;
  static constexpr int NP = (STAGES + 2) / 2;          // A pair buffers
  static constexpr int A_PAIR_BYTES = BM * 2 * BK * 2;
  static constexpr int B_BYTES = BK * BN * 2;
  static constexpr int B_OFF = NP * A_PAIR_BYTES;
  static constexpr int MAIN_BYTES = B_OFF + STAGES * B_BYTES;
  static constexpr int EPI_BYTES = WAVES * 32 * (G::WTN * 2 + 16);
  static constexpr int LDS_BYTES = MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES;
};

// Number of even j in [lo, hi].
constexpr int count_even(int lo, int hi) {
  int n = 0;
  for (int j = lo; j <= hi; ++j) n += (j % 2 == 0) ? 1 : 0;
  return n;
}

template <int BM, int BN, int BK, int WAVES, int STAGES, bool SQ, bool RS = false>
__device__ __forceinline__ void mm_lhs_pair_body(const uint16_t* __restrict__ lhs, const uint16_t* __restrict__ rhs,
                                                 uint16_t* __restrict__ out, int M, int N, int K, int group_m,
                                                 char* smem, const RowScale rsc) {
  using C = PairCfg<BM, BN, BK, WAVES, STAGES>;
  using G = typename C::G;
  static_assert(legal_lhs_pair(BM, BN, BK, WAVES, STAGES).code == MI_OK, "illegal tile config (mi_legal.hpp)");
  static_assert(C::LDS_BYTES == lds_lhs_pair(BM, BN, BK, WAVES, STAGES), "host LDS budget out of step");
  static_assert(G::ok, "illegal wave grid");
  static_assert(BK % 32 == 0 && BK <= 64, "BK of 32 or 64 (pairs of 64 or 128 columns)");
  static_assert(STAGES >= 2 && STAGES <= 4, "2..4 LDS stages for B");
  constexpr int TM = G::TM, TN = G::TN, KS = BK / 16, KC = BK / 8, NP = C::NP;
  using LA = KPanelLoader<2 * BK, BM, WAVES>;
  using LB = PanelLoader<BK, BN, WAVES>;
  constexpr int NLA = LA::LOADS_PER_TILE, NLB = LB::LOADS_PER_TILE;
  // vm_wait<n> counts assume every wave issues the same number of loads.
  static_assert(LA::EVEN && LB::EVEN, "every wave issues the same number of loads");
  static_assert(!SQ || G::WN * BM * 4 <= C::LDS_BYTES, "row sums of squares exchanged through LDS");
  static_assert(!(SQ && RS), "row sums from the A fragments or from the pack, not both");

  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tmi, tni;
  tile_coords(tiles_m, tiles_n, group_m, tmi, tni);
  const int m0 = tmi * BM, n0 = tni * BN;
  const int wm0 = (wave / G::WN) * G::WTM;
  const int wn0 = (wave % G::WN) * G::WTN;

  const uint32_t a_bytes = (uint32_t)K * (uint32_t)M * 2u;
  const uint32_t b_bytes = (uint32_t)K * (uint32_t)N * 2u;
  const int KT = (K + BK - 1) / BK;
  const int UT = (KT + 1) / 2;  // A pairs
  LA la;
  LB lb;
  la.init(wave, lane, m0, K, K - (UT - 1) * 2 * BK, a_bytes);
  lb.init(wave, lane, n0, N);
  const uint32_t kstep_pair = (uint32_t)(2 * BK) * 2u;
  const uint32_t kstep_b = (uint32_t)BK * (uint32_t)N * 2u;
  TrFrag<BN, TN> fb;
  fb.init(lane, wn0);
  // A operand: lane l reads row l%32 of a fragment, K chunk h*KC + 2*kk +
  // l/32 of the pair row (h: which tile of the pair), at its k_swz slot.
  const int arow = (wm0 + (lane & 31)) * (4 * BK);
  const int aswz = k_swz<2 * BK>(wm0 + (lane & 31));
  int akoff[2][KS];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) akoff[h][kk] = 16 * ((h * KC + 2 * kk + (lane >> 5)) ^ aswz);

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16_t{};
  bf16x8_t af[2][TM], bf[2][TN];
  constexpr int NF = TM + TN;
  // Operand f of sub-step kk of the tile in B stage `stage`, pair buffer
  // `pb`, half `h`: A0, B0 .. B(TN-1), A1 .. A(TM-1).
  auto read_frag = [&](int stage, int pb, int h, int kk, int buf, int f) {
    if (f == 0 || f > TN) {
      const int t = f == 0 ? 0 : f - TN;
      af[buf][t] = __builtin_bit_cast(
          bf16x8_t, *(MI_LDS u32x4_t*)((MI_LDS char*)smem + pb * C::A_PAIR_BYTES + arow + t * 32 * (4 * BK) +
                                        akoff[h][kk]));
    } else {
      const int t = f - 1;
      const int bbase = C::B_OFF + stage * C::B_BYTES;
      bf[buf][t] = read_tr_frag(smem, bbase + (kk * 16) * (BN * 2) + fb.off[t],
                                bbase + (kk * 16 + 4) * (BN * 2) + fb.off[t]);
    }
  };
  auto read_frags = [&](int stage, int pb, int h, int kk, int buf) {
#pragma unroll
    for (int f = 0; f < NF; ++f) read_frag(stage, pb, h, kk, buf, f);
  };
  auto mfmas = [&](int buf) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[buf][j], af[buf][i], acc[i][j], 0, 0, 0);
  };
  float sq[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) sq[i] = 0.0f;
  const int wcol = wave % G::WN;
  // SQ: the rows' squares of the A fragments in register set `buf`.  Pair d
  // of a fragment is taken as a shuffle with constant indices (a bf16x2
  // bit-cast from dword d of the fragment viewed as u32x4 is compiled as
  // dword 0 for every d by this hipcc).
  auto squares = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
      static_for<4>([&](auto d_c) __attribute__((always_inline)) {
        constexpr int d = decltype(d_c)::value;
        const bf16x2_t v = __builtin_shufflevector(af[buf][i], af[buf][i], 2 * d, 2 * d + 1);
        sq[i] = __builtin_amdgcn_fdot2_f32_bf16(v, v, sq[i], false);
      });
  };
  // The MFMAs of one sub-step, with this wave's squares when `mine`, and
  // their scheduling against the LDS reads (and the dot2 VALU work).
  auto step = [&](int buf, auto mine_c) __attribute__((always_inline)) {
    mfmas(buf);
    if constexpr (SQ && decltype(mine_c)::value) {
      squares(buf);
      interleave_mfma_mix<TM * TN, 2 * NF, 4 * TM, 0>();
    } else {
      interleave_mfma_ds<TM * TN, 2 * NF>();
    }
  };
  // Tiles and pairs past the end are clamped to the last one (re-read into
  // a buffer that is never consumed), so every group has a static size.
  auto clamp = [&](int kt) { return kt < KT ? kt : KT - 1; };
  auto clamp_pair = [&](int u) { return u < UT ? u : UT - 1; };
  // Load q of the group that brings tile j: the B loads of tile j, then
  // (j even) the A loads of pair j/2.
  auto issue_one = [&](int q, int j) {
    if (q < NLB) {
      lb.issue_at(q, make_rsrc_from(rhs, b_bytes, (uint32_t)clamp(j) * kstep_b), smem,
                  C::B_OFF + (j % STAGES) * C::B_BYTES);
    } else {
      const int u = clamp_pair(j / 2);
      la.issue_at(q - NLB, make_rsrc_from(lhs, a_bytes, (uint32_t)u * kstep_pair), smem,
                  ((j / 2) % NP) * C::A_PAIR_BYTES, u == UT - 1);
    }
  };

  // RS: the rows' partial sums of squares (BM floats past the panels;
  // each thread takes rows tid, tid + NTH, ...), the first RSB parts
  // loaded ahead of the prologue's panel loads.
  constexpr int NTH = WAVES * 64, RSB = 8, RPT = RS ? (BM + NTH - 1) / NTH : 1;
  float* rs_lds = (float*)(smem + C::LDS_BYTES);
  float rpart[RPT][RSB];
  auto load_parts = [&](int p0) {
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int r = tid + j * NTH, m = m0 + r;
#pragma unroll
      for (int q = 0; q < RSB; ++q)
        rpart[j][q] = (r < BM && m < M && p0 + q < rsc.parts) ? rsc.ssq[(size_t)(p0 + q) * (size_t)M + m] : 0.0f;
    }
  };
  if constexpr (RS) load_parts(0);

  // Prologue: the groups of tiles 0 .. STAGES-1, then wait for tile 0.
#pragma unroll
  for (int j = 0; j < STAGES; ++j) {
#pragma unroll
    for (int q = 0; q < NLB + (j % 2 == 0 ? NLA : 0); ++q) issue_one(q, j);
  }
  vm_wait<(STAGES - 1) * NLB + NLA * count_even(1, STAGES - 1)>();
  __syncthreads();
  if constexpr (RS) {
    // The compiler's wait for the partial sums drains the prologue's panel
    // loads too (they were issued after them); no load is in flight after.
    float rsum[RPT];
#pragma unroll
    for (int j = 0; j < RPT; ++j) rsum[j] = 0.0f;
    for (int p0 = 0;; p0 += RSB) {
#pragma unroll
      for (int j = 0; j < RPT; ++j)
#pragma unroll
        for (int q = 0; q < RSB; ++q) rsum[j] += rpart[j][q];
      if (p0 + RSB >= rsc.parts) break;
      load_parts(p0 + RSB);
    }
#pragma unroll
    for (int j = 0; j < RPT; ++j)
      if (tid + j * NTH < BM) rs_lds[tid + j * NTH] = 1.0f / __builtin_sqrtf(rsum[j] * rsc.inv_k + rsc.eps);
  }
  read_frags(0, 0, 0, 0, 0);

  // Tile t = t0 + I of a round (t0 a multiple of the round length, so even).
  constexpr int UR = std::lcm(STAGES, 2 * NP);
  static_assert((UR * KS) % G::WN == 0, "a round holds whole turns of the wave columns");
  // Whether sub-step kk of round tile I is squared by wave column WC.
  auto mine = [](auto i_c, auto kk_c, auto wc_c) {
    return std::integral_constant<bool, (decltype(i_c)::value * KS + decltype(kk_c)::value) % G::WN ==
                                            decltype(wc_c)::value>{};
  };
  auto tile = [&](int t, auto i_c, auto wc_c) __attribute__((always_inline)) {
    constexpr int I = decltype(i_c)::value;
    constexpr int cur = I % STAGES, pb = (I / 2) % NP, h = I % 2;
    constexpr int nxt = (I + 1) % STAGES, npb = ((I + 1) / 2) % NP, nh = (I + 1) % 2;
    constexpr int WAIT = (STAGES - 2) * NLB + NLA * count_even(I + 2, I + STAGES - 1);
    constexpr int NI = NLB + ((I + STAGES) % 2 == 0 ? NLA : 0);  // loads of the group issued here
    static_for<KS - 1>([&](auto kk_c) __attribute__((always_inline)) {
      constexpr int kk = decltype(kk_c)::value;
      read_frags(cur, pb, h, kk + 1, (kk + 1) & 1);
      step(kk & 1, mine(i_c, kk_c, wc_c));
    });
    vm_wait<WAIT>();
    __syncthreads();
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      read_frag(nxt, npb, nh, 0, 0, f);
#pragma unroll
      for (int q = f * NI / NF; q < (f + 1) * NI / NF; ++q) issue_one(q, t + STAGES);
    }
    step((KS - 1) & 1, mine(i_c, std::integral_constant<int, KS - 1>{}, wc_c));
  };
  // The K loop for wave column WC (SQ: one copy per column, each wave runs
  // its own; otherwise one copy).
  auto k_loop = [&](auto wc_c) __attribute__((always_inline)) {
    int t0 = 0;
    for (; t0 + UR < KT; t0 += UR)
      static_for<UR>([&](auto i_c) __attribute__((always_inline)) { tile(t0 + i_c(), i_c, wc_c); });
    static_while<UR>([&](auto i_c) __attribute__((always_inline)) {
      if (t0 + i_c() + 1 >= KT) return false;
      tile(t0 + i_c(), i_c, wc_c);
      return true;
    });
    // Last tile: no further loads.  It is tile I = tl - t0 of its round,
    // known only at run time, so its squares go by a wave-uniform test.
    const int tl = KT - 1;
    const int cur = tl % STAGES, pb = (tl / 2) % NP, h = tl % 2;
    static_for<KS>([&](auto kk_c) __attribute__((always_inline)) {
      constexpr int kk = decltype(kk_c)::value;
      if (kk + 1 < KS) read_frags(cur, pb, h, kk + 1, (kk + 1) & 1);
      mfmas(kk & 1);
      if constexpr (SQ) {
        if ((tl * KS + kk) % G::WN == decltype(wc_c)::value) squares(kk & 1);
      }
      interleave_mfma_ds<TM * TN, 2 * NF>();
    });
  };
  if constexpr (SQ && G::WN > 1) {
    static_for<G::WN>([&](auto wc_c) __attribute__((always_inline)) {
      if (wcol == decltype(wc_c)::value) k_loop(wc_c);
    });
  } else {
    k_loop(std::integral_constant<int, 0>{});
  }
  wait_vmem();
  __syncthreads();  // the epilogue reuses the panel buffers

  float scale[TM];
  if constexpr (SQ) {
    // Lanes l and l^32 hold the two K halves of one row's sum; the WN waves
    // of a wave row then add theirs through LDS [WN][BM], in column order.
    float* xs = (float*)smem;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const float t = sq[i] + __shfl_xor(sq[i], 32);
      if (lane < 32) xs[wcol * BM + wm0 + i * 32 + lane] = t;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = wm0 + i * 32 + (lane & 31);
      float t = xs[r];
#pragma unroll
      for (int c = 1; c < G::WN; ++c) t += xs[c * BM + r];
      scale[i] = 1.0f / __builtin_sqrtf(t * rsc.inv_k + rsc.eps);
    }
    __syncthreads();  // store_tile reuses the same LDS
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i) scale[i] = RS ? rs_lds[wm0 + i * 32 + (lane & 31)] : 1.0f;
  }
  store_tile<TM, TN, WAVES>(acc, scale, smem, wave, lane, out, M, N, m0 + wm0, n0 + wn0);
}

template <int BM, int BN, int BK, int WAVES, int STAGES>
__global__ __launch_bounds__(WAVES * 64) void mm_lhs_rhs_bf16_pair_kernel(const uint16_t* __restrict__ lhs,
                                                                         const uint16_t* __restrict__ rhs,
                                                                         uint16_t* __restrict__ out, int M, int N,
                                                                         int K, int group_m) {
  __shared__ __attribute__((aligned(1024))) char smem[PairCfg<BM, BN, BK, WAVES, STAGES>::LDS_BYTES];
  mm_lhs_pair_body<BM, BN, BK, WAVES, STAGES, false>(lhs, rhs, out, M, N, K, group_m, smem,
                                                     RowScale{nullptr, 0, 0.0f, 0.0f});
}

// Fused out[M,N] = (x[M,K] / sqrt(mean_k x^2 + eps)) . W[K,N] without gamma
// (rmsnorm_matmul variant 16): the paired-load core with the rows' squares
// (SQ above).
template <int BM, int BN, int BK, int WAVES, int STAGES>
__global__ __launch_bounds__(WAVES * 64) void rmsnorm_mm_bf16_sq_pair_kernel(const uint16_t* __restrict__ x,
                                                                            const uint16_t* __restrict__ w,
                                                                            uint16_t* __restrict__ out, int M,
                                                                            int N, int K, int group_m, float eps,
                                                                            float inv_k) {
  __shared__ __attribute__((aligned(1024))) char smem[PairCfg<BM, BN, BK, WAVES, STAGES>::LDS_BYTES];
  mm_lhs_pair_body<BM, BN, BK, WAVES, STAGES, true>(x, w, out, M, N, K, group_m, smem,
                                                    RowScale{nullptr, 0, inv_k, eps});
}

// Main pass of the two-pass fused kernel on this core (rmsnorm_matmul
// variant 15): out = diag(1/rms) . xg . W with xg = bf16(x * gamma) and the
// rows' partial sums of squares ssq[p][m] from the pack (RS above).
template <int BM, int BN, int BK, int WAVES, int STAGES>
__global__ __launch_bounds__(WAVES * 64) void rmsnorm_mm_bf16_2pass_pair_kernel(
    const uint16_t* __restrict__ xg, const uint16_t* __restrict__ w, uint16_t* __restrict__ out, int M, int N, int K,
    int group_m, const float* __restrict__ ssq, int ssq_parts, float inv_k, float eps) {
  static_assert(legal_rms2_pair(BM, BN, BK, WAVES, STAGES).code == MI_OK, "illegal tile config (mi_legal.hpp)");
  static_assert(lds_rms2_pair(BM, BN, BK, WAVES, STAGES) == PairCfg<BM, BN, BK, WAVES, STAGES>::LDS_BYTES + BM * 4,
                "host LDS budget out of step");
  __shared__ __attribute__((aligned(1024))) char smem[lds_rms2_pair(BM, BN, BK, WAVES, STAGES)];
  mm_lhs_pair_body<BM, BN, BK, WAVES, STAGES, false, true>(xg, w, out, M, N, K, group_m, smem,
                                                          RowScale{ssq, ssq_parts, inv_k, eps});
}

}  // namespace mi
