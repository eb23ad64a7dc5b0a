// mi_rms_2pass.hpp -- fused rmsnorm_matmul in two passes (variants 13, 15).
//
//   out[M,N] = (x[M,K] * rsqrt(mean_k x^2 + eps) * gamma[K]) . W[K,N]
//
// The one-pass variants (4, 5, 11, 12) scale x inside the matmul: every
// workgroup of a row block loads its x rows (K contiguous, half cache lines
// per K tile), unpacks them, multiplies by gamma and writes the scaled
// panel to LDS -- once per column of output tiles, so 8 times over at
// 4096 x 4096 with 512-wide tiles.  Here that work is done once:
//
//   pass 1, rms_pack_kernel: xt[k][m] = bf16(x[m][k] * gamma[k]) -- the
//     lhsT layout -- and ssq[p][m] = sum of x[m][k]^2 over the columns
//     k of chunk p (RP_KCH columns per chunk), in fp32;
//   pass 2, the pipelined lhsT.rhs core on (xt, W); each workgroup sums its
//     rows' partial sums (part order) while its first K tiles load, keeps
//     1/sqrt(sum / K + eps) per row in LDS, and its epilogue multiplies the
//     fp32 accumulators of output row m by it.
//
// Variant 15 packs bf16(x * gamma) in x's own layout instead (xg[m][k], a
// pass with no transpose) and runs the paired-load K-contiguous core
// (mi_mm_lhs_pair.hpp) on (xg, W) with the same row scale.  Its MFMAs see
// the same operands in the same K order as variant 13's at the same tile
// config, and the row sums are added in the same order, so the two give the
// same bits.
//
// The arithmetic is that of the one-pass variants: x*gamma rounded once to
// bf16 (the operand the MFMAs see), fp32 accumulation over the whole K, and
// 1/rms applied to the fp32 sums before the single rounding of the output.
// Only the order in which each row's sum of squares is added differs.
//
// Pass 1 layout: lane l of a wave owns rows 8*(l/8) .. +7 of the block and
// columns 8*(l%8) .. +7 of a 64-column step.  It loads its 8 row segments
// (16 bytes each; the 8 lanes of a row block read one whole 128-byte line
// per row), scales and rounds them, and writes the 8 columns of the
// transposed block as 8 16-byte row segments of xt (the 8 lanes of a
// column chunk write one whole 128-byte line per xt row).  The transpose is
// in registers: packing the products of rows j and j+1 at column e into one
// dword forms xt's row e directly.  Row sums of squares are reduced across
// the 8 lanes of a row block with DPP and across the 4 waves in LDS.
#pragma once
#include "mi_gemm.hpp"

namespace mi {

constexpr int RP_ROWS = 64;    // x rows per workgroup of pass 1
constexpr int RP_KCH = 512;    // x columns per workgroup of pass 1 (one ssq part)
constexpr int RP_WAVES = 4;    // each wave takes a 64-column step of every 256 columns

__host__ __device__ constexpr int rms2_parts(int K) { return (K + RP_KCH - 1) / RP_KCH; }

// Requires M % 8 == 0 and K % 8 == 0 (every 8-row block and 8-column chunk
// is wholly inside or outside the matrix) and 16-byte aligned x, gamma, xt.
// KMAJOR: xt is written as xg[m][k] (x's layout; the 8 lanes of a row block
// write one whole 128-byte line per row) instead of xt[k][m].
template <int KMAJOR = 0>
__global__ __launch_bounds__(RP_WAVES * 64) void rms_pack_kernel(const uint16_t* __restrict__ x,
                                                                const uint16_t* __restrict__ gamma,
                                                                uint16_t* __restrict__ xt, float* __restrict__ ssq,
                                                                int M, int K) {
  constexpr int STEPS = RP_KCH / (RP_WAVES * 64);  // 64-column steps per wave
  __shared__ float part[RP_WAVES][RP_ROWS];
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int rb = lane >> 3, kc = lane & 7;
  const int m0 = (int)blockIdx.x * RP_ROWS + 8 * rb;
  const bool rows_in = m0 < M;
  float ss[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) ss[j] = 0.0f;

  u32x4_t v[STEPS][8];
  bool in[STEPS];
  int kcol[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    kcol[s] = (int)blockIdx.y * RP_KCH + (s * RP_WAVES + wave) * 64 + 8 * kc;
    in[s] = rows_in && kcol[s] < K;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      v[s][j] = in[s] ? *(const u32x4_t*)(x + (size_t)(m0 + j) * (size_t)K + kcol[s]) : u32x4_t{0, 0, 0, 0};
  }
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    if (!in[s]) continue;
    float g[8];
    if (gamma != nullptr) {
      const u32x4_t gw = *(const u32x4_t*)(gamma + kcol[s]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        g[2 * e] = bf16lo(gw[e]);
        g[2 * e + 1] = bf16hi(gw[e]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) g[e] = 1.0f;
    }
    float val[8][8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        val[j][2 * e] = bf16lo(v[s][j][e]);
        val[j][2 * e + 1] = bf16hi(v[s][j][e]);
      }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss[j] = __builtin_fmaf(val[j][e], val[j][e], ss[j]);
    if constexpr (KMAJOR) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        u32x4_t o;
        o.x = pack_bf16x2(val[j][0] * g[0], val[j][1] * g[1]);
        o.y = pack_bf16x2(val[j][2] * g[2], val[j][3] * g[3]);
        o.z = pack_bf16x2(val[j][4] * g[4], val[j][5] * g[5]);
        o.w = pack_bf16x2(val[j][6] * g[6], val[j][7] * g[7]);
        *(u32x4_t*)(xt + (size_t)(m0 + j) * (size_t)K + kcol[s]) = o;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        u32x4_t o;
        o.x = pack_bf16x2(val[0][e] * g[e], val[1][e] * g[e]);
        o.y = pack_bf16x2(val[2][e] * g[e], val[3][e] * g[e]);
        o.z = pack_bf16x2(val[4][e] * g[e], val[5][e] * g[e]);
        o.w = pack_bf16x2(val[6][e] * g[e], val[7][e] * g[e]);
        *(u32x4_t*)(xt + (size_t)(kcol[s] + e) * (size_t)M + m0) = o;
      }
    }
  }
  // Row sums: the 8 lanes of a row block (DPP), then the 4 waves (LDS).
#pragma unroll
  for (int j = 0; j < 8; ++j) ss[j] = row_allreduce<8>(ss[j]);
  if (kc == 0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) part[wave][8 * rb + j] = ss[j];
  }
  __syncthreads();
  if (tid < RP_ROWS) {
    const int m = (int)blockIdx.x * RP_ROWS + tid;
    float r = part[0][tid];
#pragma unroll
    for (int w = 1; w < RP_WAVES; ++w) r += part[w][tid];
    if (m < M) ssq[(size_t)blockIdx.y * (size_t)M + m] = r;
  }
}

// Pass 2: the pipelined lhsT.rhs core on (xt, W) with the rms row scale in
// the epilogue; SPLIT: fp32 partial products to ws, scaled by the second
// pass of split-K (splitk_rms_sum_kernel) instead.
template <int BM, int BN, int BK, int WAVES, int STAGES, bool SPLIT = false>
__global__ __launch_bounds__(WAVES * 64) void rmsnorm_mm_bf16_2pass_kernel(
    const uint16_t* __restrict__ xt, const uint16_t* __restrict__ w, uint16_t* __restrict__ out, int M, int N, int K,
    int group_m, int parts, float* __restrict__ ws, const float* __restrict__ ssq, int ssq_parts, float inv_k,
    float eps) {
  // The pipelined core's LDS, then the block's BM row scales.
  static_assert(lds_rms2(BM, BN, BK, WAVES, STAGES) == PipeCfg<BM, BN, BK, WAVES, STAGES>::LDS_BYTES + BM * 4,
                "host LDS budget out of step");
  __shared__ __attribute__((aligned(1024))) char smem[lds_rms2(BM, BN, BK, WAVES, STAGES)];
  mm_pipe_body<BM, BN, BK, WAVES, STAGES, false, false, SPLIT, true>(xt, w, out, M, N, K, group_m, smem,
                                                                     SplitK{parts, ws},
                                                                     RowScale{ssq, ssq_parts, inv_k, eps});
}

}  // namespace mi
