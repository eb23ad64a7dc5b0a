// mm_f32.hip -- fp32 out[M,N] = lhsT[K,M]^T . rhs[K,N] (benchmark config C1).
//
// This is the fp32 semantics the reference checks every kernel against
// (simulate_fp32 rewrites all dtypes to fp32;
// reference nkigym/src/nkigym/synthesis/simulate_nki.py:24-48).  It is a
// parity path, not a throughput path: an LDS-tiled FMA kernel with the K
// sum in plain sequential order.  lhsT rows are M-contiguous, so a K slice
// of both operands is an outer product of two contiguous vectors and needs
// no transpose.
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
  };
  *n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}

}  // namespace mi
