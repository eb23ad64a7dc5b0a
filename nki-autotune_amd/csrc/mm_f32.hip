// mm_f32.hip -- fp32 out[M,N] = lhsT[K,M]^T . rhs[K,N] (benchmark config C1).
//
// This is the fp32 semantics the reference checks every kernel against
// (simulate_fp32 rewrites all dtypes to fp32;
// reference nkigym/src/nkigym/synthesis/simulate_nki.py:24-48).  It is a
// parity path, not a throughput path: an LDS-tiled FMA kernel with the K
// sum in plain sequential order.  lhsT rows are M-contiguous, so a K slice
// of both operands is an outer product of two contiguous vectors and needs
// no transpose.  Variant 1 below is the throughput path on the fp32 MFMA.
#include "mi_registry.hpp"

namespace mi {

template <int BM, int BN, int BK>
__global__ __launch_bounds__(256) void mm_f32_kernel(const float* __restrict__ lhsT, const float* __restrict__ rhs,
                                                     float* __restrict__ out, int M, int N, int K) {
  static_assert(BM == 64 && BN == 64, "16x16 threads, 4x4 outputs each");
  __shared__ float As[BK][BM + 1];
  __shared__ float Bs[BK][BN + 1];
  const int tid = (int)threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const int tiles_n = (N + BN - 1) / BN;
  const int m0 = ((int)blockIdx.x / tiles_n) * BM;
  const int n0 = ((int)blockIdx.x % tiles_n) * BN;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;

  for (int k0 = 0; k0 < K; k0 += BK) {
    for (int i = tid; i < BK * BM; i += 256) {
      const int kk = i / BM, mm = i % BM;
      const int k = k0 + kk, m = m0 + mm;
      As[kk][mm] = (k < K && m < M) ? lhsT[(size_t)k * M + m] : 0.0f;
    }
    for (int i = tid; i < BK * BN; i += 256) {
      const int kk = i / BN, nn = i % BN;
      const int k = k0 + kk, n = n0 + nn;
      Bs[kk][nn] = (k < K && n < N) ? rhs[(size_t)k * N + n] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + ty + 16 * i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tx + 16 * j;
      if (n < N) out[(size_t)m * N + n] = acc[i][j];
    }
  }
}

// Variant 1: the same product on the fp32 MFMA (v_mfma_f32_32x32x2_f32).
// Four waves in a 2 x 2 grid, each a (BM/2) x (BN/2) block of 32x32 MFMA
// tiles.  An fp32 MFMA takes 2 K values per lane (lane l: K row l/32 of the
// step, column l%32), so its operands are read straight from the K-major
// inputs, each lane one 4-byte element and each half-wave one 128-byte row
// segment, with no LDS and no transpose: lhsT[k][m] is the second MFMA
// operand (output column m = lane%32), rhs[k][n] the first (output rows n),
// so a lane ends with 4 consecutive n of one output row per dword quad.
// Each loop step loads U K pairs for every fragment first, then runs their
// MFMAs.  The MFMA adds its two products and the accumulator in one step,
// so the K sum is in a different order from variant 0's sequential one
// (fp32 rounding differences only).  Any M, N, K: loads past an edge read
// 0, stores past an edge are skipped.
template <int BM, int BN>
__global__ __launch_bounds__(256) void mm_f32_mfma_kernel(const float* __restrict__ lhsT,
                                                          const float* __restrict__ rhs, float* __restrict__ out,
                                                          int M, int N, int K) {
  constexpr int TM = BM / 64, TN = BN / 64, U = 8;
  static_assert(BM % 64 == 0 && BN % 64 == 0, "2 x 2 waves of 32x32 MFMA tiles");
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int tiles_n = (N + BN - 1) / BN;
  const int m0 = ((int)blockIdx.x / tiles_n) * BM + (wave >> 1) * (BM / 2);
  const int n0 = ((int)blockIdx.x % tiles_n) * BN + (wave & 1) * (BN / 2);
  const int kr = lane >> 5, c = lane & 31;
  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16_t{};
  for (int k0 = 0; k0 < K; k0 += 2 * U) {
    float a[U][TM], b[U][TN];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = k0 + 2 * u + kr;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int m = m0 + 32 * i + c;
        a[u][i] = (k < K && m < M) ? lhsT[(size_t)k * M + m] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + 32 * j + c;
        b[u][j] = (k < K && n < N) ? rhs[(size_t)k * N + n] : 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(b[u][j], a[u][i], acc[i][j], 0, 0, 0);
  }
  // Lane l holds output row m = m0 + 32i + l%32 and, for quad q, columns
  // n0 + 32j + 8q + 4*(l/32) + 0..3 in acc[i][j][4q .. 4q+3].
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + 32 * i + c;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int n = n0 + 32 * j + 8 * q + 4 * kr + r;
          if (n < N) out[(size_t)m * N + n] = acc[i][j][4 * q + r];
        }
  }
}

template <int BM, int BN>
hipError_t launch_mm_f32_mfma(const MiArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((mm_f32_mfma_kernel<BM, BN>), dim3(grid_tiles(a.M, a.N, BM, BN)), dim3(256), 0, s,
                     (const float*)a.a, (const float*)a.b, (float*)a.out, a.M, a.N, a.K);
  return hipGetLastError();
}

template <int BM, int BN, int BK>
hipError_t launch_mm_f32(const MiArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((mm_f32_kernel<BM, BN, BK>), dim3(grid_tiles(a.M, a.N, BM, BN)), dim3(256), 0, s,
                     (const float*)a.a, (const float*)a.b, (float*)a.out, a.M, a.N, a.K);
  return hipGetLastError();
}

const MiEntry* table_f32(int* n) {
  static const MiEntry t[] = {
      {MI_KERNEL_MATMUL_LHST_RHS_F32, {64, 64, 16, 4, 1, 1, 0, 0}, (int)(16 * 65 * 4 * 2), &launch_mm_f32<64, 64, 16>},
      {MI_KERNEL_MATMUL_LHST_RHS_F32, {64, 64, 32, 4, 1, 1, 0, 0}, (int)(32 * 65 * 4 * 2), &launch_mm_f32<64, 64, 32>},
      {MI_KERNEL_MATMUL_LHST_RHS_F32, {64, 64, 16, 4, 1, 1, 0, 1}, 0, &launch_mm_f32_mfma<64, 64>},
      {MI_KERNEL_MATMUL_LHST_RHS_F32, {128, 128, 16, 4, 1, 1, 0, 1}, 0, &launch_mm_f32_mfma<128, 128>},
  };
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}

}  // namespace mi
