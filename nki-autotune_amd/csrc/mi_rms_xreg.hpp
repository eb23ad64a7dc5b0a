// mi_rms_xreg.hpp -- fused rmsnorm_matmul on the pipelined matmul core, with
// the x panel staged through registers (rmsnorm_matmul variants 4 and 5;
// 11 and 12 are the same with W read non-temporally).
//
//   out[M,N] = (x[M,K] * rsqrt(mean_k x^2 + eps) * gamma[K]) . W[K,N]
//
// The W panel takes the path of the pipelined matmul: LDS-direct loads into
// a STAGES-deep ring, one barrier per K tile, MFMAs interleaved with the
// operand reads.  The x panel (K contiguous) is fetched by buffer loads into
// an XS-slot register ring (XS = 2: variant 4, XS = 3: variant 5), so it
// crosses LDS once, already scaled:
//
//   tile j's x                  -> register slot j%XS, issued at the barrier
//                                 that ends tile j-1-XS
//   tile j's A panel            <- x * gamma (bf16), written by every thread
//                                 into stage j%STAGES during tile j-1, spread
//                                 over the MFMA sub-steps, while the row sums
//                                 of squares accumulate in fp32
//   tile j's W                  -> stage j%STAGES, issued at the barrier that
//                                 ends tile j-STAGES
//
// 1/rms is known only after the last tile, so it scales the fp32
// accumulators in the epilogue (out row m = inv_rms[m] * (x*gamma . W)[m]).
// gamma is staged in LDS once, as fp32 (K up to GK_MAX), so scaling needs
// no unpacking of gamma and no per-tile gamma load.
//
// Both loads are issued as inline asm, so the compiler inserts no vmcnt
// waits of its own: the kernel waits with exact counts (the memory system
// returns vector loads in issue order) and then passes the loaded registers
// through an empty asm so that nothing reads them before the wait.  At every
// barrier each thread issues the same group -- its LB W loads of tile
// t+STAGES, then its LX x loads of tile t+1+XS (tiles past the end re-read
// the last W tile, or read zeros) -- so the counts are compile-time
// constants (younger loads that may still fly):
//   x(j), needed during tile j-1:   (XS-1) * (LB + LX)
//   W(t+1), needed at barrier t:    LX + (STAGES-2) * (LB + LX)
#pragma once
#include <type_traits>

#include "mi_gemm.hpp"

namespace mi {

template <int BM, int BN, int BK, int WAVES, int STAGES>
struct XregCfg {
  using G = WaveGrid<BM, BN, WAVES>;
  static constexpr int NT = WAVES * 64;
  static constexpr int KC = BK / 8;                  // 16-byte chunks per x row per K tile
  static constexpr int CHUNKS = BM * KC;
  static constexpr int CPT = CHUNKS / NT;            // x chunks per thread per tile
  static constexpr int XD = (128 / BK) > 0 ? (128 / BK) : 1;
  static constexpr int A_BYTES = BM * BK * 2;        // scaled x panel, K contiguous, k_swz
  static constexpr int B_BYTES = BK * BN * 2;        // W panel, N contiguous, mn_swz
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int MAIN_BYTES = STAGES * STAGE_BYTES;
  static constexpr int EPI_BYTES = WAVES * 32 * (G::WTN * 2 + 16);
  static constexpr int RMS_OFF = ((MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES) + 15) / 16 * 16;
  static constexpr int G_OFF = RMS_OFF + BM * 4;     // fp32 gamma, GK_MAX entries
  // fp32 gamma entries (K rounded up to BK): 8192, or what the LDS left
  // beside the panels holds.
  static constexpr int GK_FIT = (160 * 1024 - G_OFF) / 4 / BK * BK;
  static constexpr int GK_MAX = GK_FIT < 8192 ? GK_FIT : 8192;
  static constexpr int LDS_BYTES = G_OFF + GK_MAX * 4;
  static_assert(CHUNKS % NT == 0 && CPT >= 1, "every thread owns the same number of x chunks");
  static_assert(GK_MAX % BK == 0, "gamma capacity in whole K tiles");
  static_assert(NT % KC == 0, "row lanes must not straddle threads");
};

// 16-byte buffer load into a VGPR quad, invisible to the compiler's waitcnt
// bookkeeping; the caller waits with vm_wait and then calls reg_ready.
__device__ __forceinline__ u32x4_t vload16(__amdgpu_buffer_rsrc_t rs, uint32_t voff) {
  u32x4_t r;
  asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(r) : "v"(voff), "s"(rs));
  return r;
}
// Orders every later use of r after the preceding vm_wait.
__device__ __forceinline__ void reg_ready(u32x4_t& r) { asm volatile("" : "+v"(r)); }

// NTW: W read non-temporally (variants 11 / 12: skinny M, where W is
// streamed once).  SPLIT: K split over `parts` workgroups per output tile;
// part p writes its unscaled fp32 products to ws[p][M][N] and its rows'
// sums of squares over its K range to ws[parts*M*N + p*M + m] (from the
// workgroups of the first column of tiles), and splitk_rms_sum_kernel forms
// out.  gamma then needs LDS room for one part's K range only.
template <int BM, int BN, int BK, int WAVES, int STAGES, int XS, bool HG, bool NTW = false, bool SPLIT = false,
          int SSQ_PARTS = 4>
__global__ __launch_bounds__(WAVES * 64) void rmsnorm_mm_bf16_xreg_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ out, int M, int N, int K, float inv_k, float eps, int group_m, int parts,
    float* __restrict__ ws) {
  using C = XregCfg<BM, BN, BK, WAVES, STAGES>;
  using G = typename C::G;
  static_assert(legal_rms_xreg(BM, BN, BK, WAVES, STAGES, XS).code == MI_OK, "illegal tile config (mi_legal.hpp)");
  static_assert(C::LDS_BYTES == lds_rms_xreg(BM, BN, BK, WAVES, STAGES), "host LDS budget out of step");
  static_assert(C::GK_MAX == xreg_gamma_kmax(BM, BN, BK, WAVES, STAGES), "host gamma capacity out of step");
  static_assert(G::ok, "illegal wave grid");
  static_assert(BK % 32 == 0, "BK must be a multiple of 32 (even number of MFMA K steps)");
  static_assert(STAGES >= 2 && STAGES <= 4, "2..4 LDS stages");
  static_assert(XS == 2 || XS == 3, "2 or 3 register slots");
  constexpr int TM = G::TM, TN = G::TN, KS = BK / 16, KC = C::KC, CPT = C::CPT, NT = C::NT;
  using LB = PanelLoader<BK, BN, WAVES>;
  static_assert(LB::EVEN, "every wave issues the same number of W loads");
  constexpr int NLB = LB::LOADS_PER_TILE;
  constexpr int NLX = CPT;
  constexpr int X_WAIT = (XS - 1) * (NLB + NLX);
  constexpr int B_WAIT = NLX + (STAGES - 2) * (NLB + NLX);
  static_assert(X_WAIT < 64 && B_WAIT < 64, "vmcnt is 6 bits");
  __shared__ __attribute__((aligned(1024))) char smem[HG ? C::LDS_BYTES : C::G_OFF];
  float* rms_lds = (float*)(smem + C::RMS_OFF);

  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tmi, tni, part = 0;
  if constexpr (SPLIT) tile_coords_split(tiles_m, tiles_n, group_m, parts, tmi, tni, part);
  else tile_coords(tiles_m, tiles_n, group_m, tmi, tni);
  const int m0 = tmi * BM, n0 = tni * BN;
  const int wm0 = (wave / G::WN) * G::WTM;
  const int wn0 = (wave % G::WN) * G::WTN;

  const int ldx = K;  // row stride of x: the whole K
  int k0 = 0;
  if constexpr (SPLIT) {
    // Part `part`: K indices [k0, k0 + K) -- columns of x, entries of gamma,
    // rows of W (the host guarantees every part a non-empty range).
    const int kts = ((K + BK - 1) / BK + parts - 1) / parts;
    k0 = part * kts * BK;
    x += k0;
    gamma += k0;
    w += (size_t)k0 * (size_t)N;
    K = K - k0 < kts * BK ? K - k0 : kts * BK;
  }
  // Bytes from the (part's) base to the end of x.
  const uint32_t x_bytes = ((uint32_t)M * (uint32_t)ldx - (uint32_t)k0) * 2u;
  const uint32_t w_bytes = (uint32_t)K * (uint32_t)N * 2u;
  const int KT = (K + BK - 1) / BK;
  auto clamp = [&](int kt) { return kt < KT ? kt : KT - 1; };

  // gamma -> LDS as fp32 (zeros past K, up to the last tile), with ordinary
  // loads before any asynchronous load is issued; published by the barrier
  // before the first scaling.
  if constexpr (HG) {
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(gamma, (uint32_t)K * 2u);
    for (int c = tid; c < KT * BK / 8; c += NT) {
      const u32x4_t g = __builtin_amdgcn_raw_buffer_load_b128(rg, 16u * (uint32_t)c, 0, 0);
      MI_LDS float* d = (MI_LDS float*)((MI_LDS char*)smem + C::G_OFF) + 8 * c;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        d[2 * e] = bf16lo(g[e]);
        d[2 * e + 1] = bf16hi(g[e]);
      }
    }
    __syncthreads();
  }

  // ---- x chunks of this thread: c = i*NT + tid -> row c/KC, K chunk tid%KC.
  // Chunks past K (and rows past M) fall outside the buffer and read zeros.
  const int kc = tid % KC;
  int xrow[CPT], xlds[CPT];
  uint32_t xoff[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = i * NT + tid;
    xrow[i] = c / KC;
    xoff[i] = ((uint32_t)(m0 + xrow[i]) * (uint32_t)ldx + (uint32_t)(8 * kc)) * 2u;
    xlds[i] = xrow[i] * (BK * 2) + 16 * (kc ^ k_swz<BK>(xrow[i]));
  }
  u32x4_t xr[XS][CPT];
  // x load q (< NLX) of tile kt into register slot P.
  auto issue_x = [&](int q, int kt, auto slot_c) __attribute__((always_inline)) {
    constexpr int P = decltype(slot_c)::value;
    // Tiles past the end take the last tile's descriptor (offset <= size)
    // and an offset past every descriptor's end.
    const bool kin = kt * BK + 8 * kc < K;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc_from(x, x_bytes, (uint32_t)clamp(kt) * (uint32_t)(BK * 2));
    xr[P][q] = vload16(rs, kin ? xoff[q] : x_bytes);
  };
  auto x_ready = [&](auto slot_c) __attribute__((always_inline)) {
    constexpr int P = decltype(slot_c)::value;
#pragma unroll
    for (int i = 0; i < CPT; ++i) reg_ready(xr[P][i]);
  };

  LB lb;
  lb.init(wave, lane, n0, N);
  const uint32_t kstep_b = (uint32_t)BK * (uint32_t)N * 2u;
  auto issue_w = [&](int q, int kt, int stage) {
    lb.template issue_at<NTW>(q, make_rsrc_from(w, w_bytes, (uint32_t)kt * kstep_b), smem,
                              stage * C::STAGE_BYTES + C::A_BYTES);
  };
  TrFrag<BN, TN> fb;
  fb.init(lane, wn0);

  // ---- scaling: chunk i of slot P -> A panel of `stage`, i = s, s+KS, ...
  // during MFMA sub-step s.
  // Row sums of squares, NSA partial sums per owned chunk.
  constexpr int NSA = SSQ_PARTS;
  float ss[CPT][NSA];
#pragma unroll
  for (int i = 0; i < CPT; ++i)
#pragma unroll
    for (int a = 0; a < NSA; ++a) ss[i][a] = 0.0f;
  // gamma of tile j for this thread's K chunk (8 fp32): every chunk of the
  // thread shares it (NT is a multiple of KC), so it is read once per tile.
  f32x4_t g0 = {}, g1 = {};
  auto gamma_of = [&](int j) {
    if constexpr (HG) {
      const MI_LDS f32x4_t* gp = (const MI_LDS f32x4_t*)((MI_LDS char*)smem + C::G_OFF + 4 * (j * BK + 8 * kc));
      g0 = gp[0];
      g1 = gp[1];
    }
  };
  auto scale_chunk = [&](int i, auto slot_c, int stage) {
    constexpr int P = decltype(slot_c)::value;
    const u32x4_t o = scale_sumsq_chunk_f32g<NSA, HG>(xr[P][i], g0, g1, ss[i]);
    *(MI_LDS u32x4_t*)((MI_LDS char*)smem + stage * C::STAGE_BYTES + xlds[i]) = o;
  };
  auto scale_step = [&](int s, auto slot_c, int stage) {
#pragma unroll
    for (int i = s; i < CPT; i += KS) scale_chunk(i, slot_c, stage);
  };
  constexpr int CPS = (CPT + KS - 1) / KS;    // chunks per sub-step (at most)
  constexpr int VPC = HG ? 28 : 16;           // VALU per chunk (unpack, squares, scale, pack)

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
  using S2 = std::integral_constant<int, 2 % XS>;

  // ---- prologue: the groups of the barriers before tile 0 (absent tiles
  // left out: no steady-state wait counts across them), then A(0) is
  // scaled and the last group is issued after the barrier.
  //   barrier u (u = -U0 .. -1) issues W(u+STAGES), x(u+1+XS)
  constexpr int U0 = STAGES > XS + 1 ? STAGES : XS + 1;
  auto issue_x_tile = [&](int j) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < NLX; ++q) {
      if (j % XS == 0) issue_x(q, j, S0{});
      else if (j % XS == 1) issue_x(q, j, S1{});
      else issue_x(q, j, S2{});
    }
  };
#pragma unroll
  for (int u = -U0; u <= -2; ++u) {
    const int wj = u + STAGES, xj = u + 1 + XS;
    if (wj >= 0) {
#pragma unroll
      for (int q = 0; q < NLB; ++q) issue_w(q, clamp(wj), wj % STAGES);
    }
    if (xj >= 0) issue_x_tile(xj);
  }
  wait_vmem();
  x_ready(S0{});
  gamma_of(0);
#pragma unroll
  for (int s = 0; s < KS; ++s) scale_step(s, S0{}, 0);
  __syncthreads();
#pragma unroll
  for (int q = 0; q < NLB; ++q) issue_w(q, clamp(STAGES - 1), STAGES - 1);
  issue_x_tile(XS);
  read_frags(0, 0, 0);

  // ---- steady state.  Tile t sits in LDS stage t%STAGES, consumes
  // register slot (t+1)%XS (x of tile t+1) and refills it with x of tile
  // t+1+XS at its closing barrier.
  auto tile = [&](int t, auto slot_c, auto stage_c) __attribute__((always_inline)) {
    constexpr int cur = decltype(stage_c)::value;
    constexpr int nxt = cur + 1 == STAGES ? 0 : cur + 1;
    // The wait sits at the top of the tile so that the scaling VALU, the
    // operand reads and the MFMAs of each sub-step share one scheduling
    // region (an asm statement ends a region); the LDS writes are left
    // unplaced so that each follows its own VALU chain.
    vm_wait<X_WAIT>();
    x_ready(slot_c);
    gamma_of(t + 1);
#pragma unroll
    for (int kk = 0; kk + 1 < KS; ++kk) {
      read_frags(cur, kk + 1, (kk + 1) & 1);
      scale_step(kk, slot_c, nxt);
      mfma_rows(kk & 1, 0, TM);
      interleave_mfma_mix<TM * TN, ND + (HG ? 2 : 0), CPS * VPC, 0>();
    }
    scale_step(KS - 1, slot_c, nxt);
    mfma_rows((KS - 1) & 1, 0, TM / 2);
    interleave_mfma_mix<(TM / 2) * TN, 0, CPS * VPC, 0>();
    // W(t+1) landed; every wave's A(t+1) writes are complete once the
    // barrier is passed.
    vm_wait<B_WAIT>();
    __syncthreads();
    const int kw = clamp(t + STAGES);
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      read_frag(nxt, 0, 0, f);
#pragma unroll
      for (int q = f * (NLX + NLB) / NF; q < (f + 1) * (NLX + NLB) / NF; ++q) {
        if (q < NLB) issue_w(q, kw, cur);
        else issue_x(q - NLB, t + 1 + XS, slot_c);
      }
    }
    mfma_rows((KS - 1) & 1, TM / 2, TM);
    interleave_mfma_ds<(TM - TM / 2) * TN, ND>();
  };
  // Unrolled lcm(XS, STAGES) times so that every slot and stage index is a
  // compile-time constant (LDS operands then take immediate offsets).
  constexpr int UR = std::lcm(XS, STAGES);
  auto round_tile = [&](int t, auto i_c) __attribute__((always_inline)) {
    constexpr int i = decltype(i_c)::value;
    tile(t, std::integral_constant<int, (i + 1) % XS>{}, std::integral_constant<int, i % STAGES>{});
  };
  int t0 = 0;
  for (; t0 + UR < KT; t0 += UR)
    static_for<UR>([&](auto i_c) __attribute__((always_inline)) { round_tile(t0 + i_c(), i_c); });
  static_while<UR>([&](auto i_c) __attribute__((always_inline)) {
    if (t0 + i_c() + 1 >= KT) return false;
    round_tile(t0 + i_c(), i_c);
    return true;
  });
  const int cur = (KT - 1) % STAGES;
  // Last tile: nothing left to scale or load.
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    if (kk + 1 < KS) read_frags(cur, kk + 1, (kk + 1) & 1);
    mfma_rows(kk & 1, 0, TM);
    interleave_mfma_ds<TM * TN, ND>();
  }
  wait_vmem();
  // The x loads of tiles past the end were never consumed: keep their
  // registers allocated until the wait above has drained them.
  x_ready(S0{});
  x_ready(S1{});
  if constexpr (XS == 3) x_ready(S2{});
  __syncthreads();  // the epilogue reuses the panel buffers

  if constexpr (SPLIT) {
    // This part's sums of squares (one column of tiles writes them) and its
    // unscaled products; the second pass sums the parts and scales.
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const float r = row_allreduce<KC>(sum_parts<NSA>(ss[i]));
      const int m = m0 + xrow[i];
      if (tni == 0 && kc == 0 && m < M) ws[(size_t)parts * M * N + (size_t)part * M + m] = r;
    }
    store_partial<TM, TN>(acc, ws + (size_t)part * M * N, lane, M, N, m0 + wm0, n0 + wn0);
    return;
  }
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const float r = row_allreduce<KC>(sum_parts<NSA>(ss[i]));
    if (kc == 0) rms_lds[xrow[i]] = 1.0f / __builtin_sqrtf(r * inv_k + eps);
  }
  __syncthreads();
  float scale[TM];
#pragma unroll
  for (int mt = 0; mt < TM; ++mt) scale[mt] = rms_lds[wm0 + mt * 32 + (lane & 31)];
  store_tile<TM, TN, WAVES>(acc, scale, smem, wave, lane, out, M, N, m0 + wm0, n0 + wn0);
}

// Split-K second pass of the fused kernel: for 8 consecutive elements of
// row m, out = bf16(rsqrt(sum_q ssq[q][m] * inv_k + eps) * sum_p ws[p][...]),
// both sums in part order (ws = [parts][M][N] products, ssq = [ssq_parts][M]
// partial sums of squares; N % 8 == 0, so 8 elements never straddle rows).
template <int UNUSED = 0>
__global__ __launch_bounds__(256) void splitk_rms_sum_kernel(const float* __restrict__ ws, uint16_t* __restrict__ out,
                                                             int M, int N, int parts, const float* __restrict__ ssq,
                                                             int ssq_parts, float inv_k, float eps) {
  const size_t n = (size_t)M * (size_t)N;
  const size_t stride = (size_t)gridDim.x * 256 * 8;
  for (size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 8; i < n; i += stride) {
    const size_t m = i / (size_t)N;
    float r = ssq[m];
    for (int q = 1; q < ssq_parts; ++q) r += ssq[(size_t)q * M + m];
    f32x4_t lo = *(const f32x4_t*)(ws + i), hi = *(const f32x4_t*)(ws + i + 4);
    for (int p = 1; p < parts; ++p) {
      lo += *(const f32x4_t*)(ws + (size_t)p * n + i);
      hi += *(const f32x4_t*)(ws + (size_t)p * n + i + 4);
    }
    const float sc = 1.0f / __builtin_sqrtf(r * inv_k + eps);
    u32x4_t o;
    o.x = pack_bf16x2(lo[0] * sc, lo[1] * sc);
    o.y = pack_bf16x2(lo[2] * sc, lo[3] * sc);
    o.z = pack_bf16x2(hi[0] * sc, hi[1] * sc);
    o.w = pack_bf16x2(hi[2] * sc, hi[3] * sc);
    *(u32x4_t*)(out + i) = o;
  }
}

}  // namespace mi
