// mi_mm_reg.hpp -- lhsT.rhs matmul with a register prefetch ring
// (matmul variant 2), for the skinny, HBM-bound shapes.
//
// A skinny product (M <= 128 against N = 28672, K = 8192) is a stream of
// the rhs panel: it is HBM-bound, and what limits it is how many bytes each
// CU keeps in flight.  LDS cannot hold a deep enough ring (the lhsT tile
// takes half of every stage), so this kernel keeps the ring in VGPRs: every
// thread holds its 16-byte pieces of the next PF K tiles of both operands
// (ordinary buffer loads, so the compiler's vmcnt waits are exact), writes
// the oldest tile to a double-buffered LDS stage with the same swizzled
// layout the LDS-direct loaders produce, and the MFMA core is the one of
// the pipelined matmul (transposing LDS reads, 32x32x16 bf16 MFMA).
//
// Step t:  ds_write tile t (registers -> LDS stage t%2);  load tile t+PF into
//          the registers just freed;  barrier;  MFMAs of tile t.
// Steps run in groups of PF (register slots are compile-time); steps past
// the last K tile load zeros (buffer bounds) and add nothing.
#pragma once
#include "mi_gemm.hpp"

namespace mi {

// 16-byte pieces of one [BK][W] MN-contiguous panel owned by one thread:
// piece i is LDS chunk position p = 16 * (i*NT + tid) of the panel, whose
// row is p / (2W) and whose global column is that of the swizzled slot.
template <int BK, int W, int NT>
struct RegPanel {
  static constexpr int ROWB = W * 2;
  static constexpr int PIECES = BK * W * 2 / 16;
  static constexpr int PPT = PIECES / NT;  // pieces per thread
  static_assert(PIECES % NT == 0, "every thread loads the same number of pieces");
  uint32_t goff[PPT];  // global byte offset at K tile 0
  int lds[PPT];        // LDS byte offset inside the panel
  __device__ __forceinline__ void init(int tid, int col0, int ld) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int p = 16 * (i * NT + tid);
      const int row = p / ROWB;
      const int slot = (p % ROWB) / 16;
      const int q = slot ^ mn_swz<ROWB>(row);
      goff[i] = ((uint32_t)row * (uint32_t)ld + (uint32_t)(col0 + 8 * q)) * 2u;
      lds[i] = p;
    }
  }
};

template <int BM, int BN, int BK, int WAVES, int PF>
__global__ __launch_bounds__(WAVES * 64) void mm_lhsT_rhs_bf16_reg_kernel(const uint16_t* __restrict__ lhsT,
                                                                         const uint16_t* __restrict__ rhs,
                                                                         uint16_t* __restrict__ out, int M, int N,
                                                                         int K, int group_m) {
  using G = WaveGrid<BM, BN, WAVES>;
  static_assert(legal_mm_reg(BM, BN, BK, WAVES, PF).code == MI_OK, "illegal tile config (mi_legal.hpp)");
  static_assert(G::ok, "illegal wave grid");
  static_assert(BK % 32 == 0, "BK must be a multiple of 32");
  static_assert(PF >= 1 && PF <= 8, "1..8 tiles in the register ring");
  constexpr int NT = WAVES * 64, TM = G::TM, TN = G::TN, KS = BK / 16;
  constexpr int A_BYTES = BK * BM * 2, B_BYTES = BK * BN * 2, STAGE = A_BYTES + B_BYTES;
  constexpr int EPI = WAVES * 32 * (G::WTN * 2 + 16);
  constexpr int LDS = 2 * STAGE > EPI ? 2 * STAGE : EPI;
  static_assert(LDS == lds_mm_reg(BM, BN, BK, WAVES), "host LDS budget out of step");
  using PA = RegPanel<BK, BM, NT>;
  using PB = RegPanel<BK, BN, NT>;
  __shared__ __attribute__((aligned(1024))) char smem[LDS];

  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tmi, tni;
  tile_coords(tiles_m, tiles_n, group_m, tmi, tni);
  const int m0 = tmi * BM, n0 = tni * BN;
  const int wm0 = (wave / G::WN) * G::WTM;
  const int wn0 = (wave % G::WN) * G::WTN;

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(lhsT, (uint32_t)K * (uint32_t)M * 2u);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(rhs, (uint32_t)K * (uint32_t)N * 2u);
  PA pa;
  PB pb;
  pa.init(tid, m0, M);
  pb.init(tid, n0, N);
  const uint32_t kstep_a = (uint32_t)BK * (uint32_t)M * 2u;
  const uint32_t kstep_b = (uint32_t)BK * (uint32_t)N * 2u;
  TrFrag<BM, TM> fa;
  TrFrag<BN, TN> fb;
  fa.init(lane, wm0);
  fb.init(lane, wn0);

  u32x4_t xa[PF][PA::PPT], xb[PF][PB::PPT];
  auto load = [&](int kt, u32x4_t (&va)[PA::PPT], u32x4_t (&vb)[PB::PPT]) {
    // Rows past K fall outside the buffers and read as zeros.
#pragma unroll
    for (int i = 0; i < PB::PPT; ++i)
      vb[i] = __builtin_amdgcn_raw_buffer_load_b128(rb, pb.goff[i] + (uint32_t)kt * kstep_b, 0, 0);
#pragma unroll
    for (int i = 0; i < PA::PPT; ++i)
      va[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, pa.goff[i] + (uint32_t)kt * kstep_a, 0, 0);
  };
  auto store = [&](int stage, const u32x4_t (&va)[PA::PPT], const u32x4_t (&vb)[PB::PPT]) {
#pragma unroll
    for (int i = 0; i < PA::PPT; ++i) *(MI_LDS u32x4_t*)((MI_LDS char*)smem + stage * STAGE + pa.lds[i]) = va[i];
#pragma unroll
    for (int i = 0; i < PB::PPT; ++i)
      *(MI_LDS u32x4_t*)((MI_LDS char*)smem + stage * STAGE + A_BYTES + pb.lds[i]) = vb[i];
  };

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16_t{};
  auto compute = [&](int stage) {
    const int abase = stage * STAGE, bbase = abase + A_BYTES;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      bf16x8_t af[TM], bf[TN];
#pragma unroll
      for (int t = 0; t < TM; ++t)
        af[t] = read_tr_frag(smem, abase + (kk * 16) * (BM * 2) + fa.off[t], abase + (kk * 16 + 4) * (BM * 2) + fa.off[t]);
#pragma unroll
      for (int t = 0; t < TN; ++t)
        bf[t] = read_tr_frag(smem, bbase + (kk * 16) * (BN * 2) + fb.off[t], bbase + (kk * 16 + 4) * (BN * 2) + fb.off[t]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[j], af[i], acc[i][j], 0, 0, 0);
    }
  };

  const int KT = (K + BK - 1) / BK;
#pragma unroll
  for (int s = 0; s < PF; ++s) load(s, xa[s], xb[s]);
  for (int t0 = 0; t0 < KT; t0 += PF) {
#pragma unroll
    for (int s = 0; s < PF; ++s) {
      const int t = t0 + s;
      const int stage = s & 1 ? (t0 & 1) ^ 1 : (t0 & 1);  // = t & 1
      store(stage, xa[s], xb[s]);
      load(t + PF, xa[s], xb[s]);
      __syncthreads();
      compute(stage);
    }
  }
  __syncthreads();  // the epilogue reuses the panel buffers

  float one[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) one[i] = 1.0f;
  store_tile<TM, TN, WAVES>(acc, one, smem, wave, lane, out, M, N, m0 + wm0, n0 + wn0);
}

}  // namespace mi
