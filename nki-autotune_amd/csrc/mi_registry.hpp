// mi_registry.hpp -- table of compiled kernel instances and their launchers.
//
// Every tile config in the search space is a template instance compiled
// ahead of time into libmi_kernels.so; each translation unit contributes a
// table of MiEntry rows.  The C ABI (mi_capi.hip) looks a config up in the
// merged table, checks its static legality and calls its launcher.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mi_kernels.h"
#include "mi_gemm.hpp"
#include "mi_legal.hpp"
#include "mi_mm_lhs_pair.hpp"
#include "mi_mm_reg.hpp"
#include "mi_rms_2pass.hpp"
#include "mi_rms_xreg.hpp"

namespace mi {

struct MiArgs {
  const void* a;      // lhsT / lhs / x
  const void* b;      // rhs / W
  const void* g;      // gamma (fused kernel, may be null)
  void* out;
  int M, N, K;
  float eps, inv_k;
  int group_m;
  int parts = 1;          // split-K parts
  char* ws = nullptr;     // workspace of workspace_bytes() bytes (256-byte aligned), or null if none is needed
  int cus = 256;          // compute units of the device (the stream-K grid)
  bool ws_zeroed = false; // the workspace's stream-K counters are known to be 0 (a reused workspace)
};

// Every workspace starts with the stream-K tile counters (kSkCounterBytes,
// mi_streamk.hpp), which only the stream-K kernels touch and which each of
// their launches leaves at 0; the data of the other kernels follows.
inline char* ws_data(const MiArgs& a) { return a.ws + kSkCounterBytes; }

// Stream-K variants (lhsT.rhs 5 and 6).
inline bool is_streamk(int kernel_id, int variant) {
  return kernel_id == MI_KERNEL_MATMUL_LHST_RHS_BF16 && (variant == 5 || variant == 6);
}

typedef hipError_t (*LaunchFn)(const MiArgs&, hipStream_t);

struct MiEntry {
  int kernel_id;
  mi_tile_cfg cfg;
  int lds_bytes;  // static LDS of the instance
  LaunchFn launch;
  int gamma_kmax;  // K (rounded up to the kernel's K step) whose gamma fits in LDS; 0 = no limit
};

inline int grid_tiles(int M, int N, int BM, int BN) { return ((M + BM - 1) / BM) * ((N + BN - 1) / BN); }

inline size_t align256(size_t v) { return (v + 255) / 256 * 256; }

// Device workspace a launch needs, in bytes (0: none): the stream-K
// counters (kSkCounterBytes), then
//   split-K matmul:                 fp32 products [parts][M][N]
//   split-K fused (variants 4..12): products, then row sums of squares [parts][M]
//   two-pass fused (variants 13, 15): xt [K][M] (15: xg [M][K]) bf16,
//                                   ssq [ceil(K/512)][M] fp32,
//                                   then (split) products [parts][M][N]
//   stream-K (lhsT.rhs 5, 6):       fp32 partial tiles: one early slot per
//                                   workgroup of the grid, one owner slot per
//                                   output tile, BM*BN each (the counters
//                                   themselves are the reserved region)
inline size_t workspace_bytes(int kernel_id, const mi_tile_cfg& c, int M, int N, int K, int cus) {
  const size_t m = (size_t)M, n = (size_t)N, k = (size_t)K, p = (size_t)(c.split_k > 1 ? c.split_k : 0);
  size_t data = 0;
  if (kernel_id == MI_KERNEL_RMSNORM_MATMUL_BF16 && (c.variant == 13 || c.variant == 15))
    data = align256(k * m * 2) + align256((size_t)rms2_parts(K) * m * 4) + p * m * n * 4;
  else if (is_streamk(kernel_id, c.variant)) {
    const long long tiles = grid_tiles(M, N, c.block_m, c.block_n);
    const long long kt = (K + c.block_k - 1) / c.block_k;
    const size_t grid = (size_t)streamk_grid(cus, tiles, kt);
    data = (grid + (size_t)tiles) * (size_t)c.block_m * (size_t)c.block_n * 4;
  } else if (p == 0)
    return 0;
  else if (kernel_id == MI_KERNEL_RMSNORM_MATMUL_BF16)
    data = p * (m * n + m) * 4;
  else
    data = p * m * n * 4;
  return (size_t)kSkCounterBytes + data;
}

template <int BM, int BN, int BK, int W, int S>
hipError_t launch_mm_bf16(const MiArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((mm_lhsT_rhs_bf16_kernel<BM, BN, BK, W, S>), dim3(grid_tiles(a.M, a.N, BM, BN)), dim3(W * 64),
                     0, s, (const uint16_t*)a.a, (const uint16_t*)a.b, (uint16_t*)a.out, a.M, a.N, a.K, a.group_m);
  return hipGetLastError();
}

// Split-K second pass: out = bf16(sum over the parts of ws), in part order.
inline void launch_splitk_sum(const float* ws, uint16_t* out, size_t n, int parts, hipStream_t s) {
  const size_t blocks = (n / 8 + 255) / 256;
  hipLaunchKernelGGL(splitk_sum_kernel<0>, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, s, ws, out,
                     n, parts);
}

// Split-K second pass of the fused kernels: products and sums of squares in
// part order, then 1/rms and the bf16 rounding.
inline void launch_splitk_rms_sum(const float* prod, int parts, const float* ssq, int ssq_parts, const MiArgs& a,
                                  hipStream_t s) {
  const size_t blocks = ((size_t)a.M * (size_t)a.N / 8 + 255) / 256;
  hipLaunchKernelGGL(splitk_rms_sum_kernel<0>, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, s,
                     prod, (uint16_t*)a.out, a.M, a.N, parts, ssq, ssq_parts, a.inv_k, a.eps);
}

template <int BM, int BN, int BK, int W, int S, bool NTB = false>
hipError_t launch_mm_pipe(const MiArgs& a, hipStream_t s) {
  if (a.parts > 1) {
    // Split-K: the parts' fp32 products into ws, then their sum into out.
    hipLaunchKernelGGL((mm_lhsT_rhs_bf16_pipe_kernel<BM, BN, BK, W, S, NTB, true>),
                       dim3(grid_tiles(a.M, a.N, BM, BN) * a.parts), dim3(W * 64), 0, s, (const uint16_t*)a.a,
                       (const uint16_t*)a.b, (uint16_t*)a.out, a.M, a.N, a.K, a.group_m, a.parts, (float*)ws_data(a));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_splitk_sum((const float*)ws_data(a), (uint16_t*)a.out, (size_t)a.M * (size_t)a.N, a.parts, s);
  } else {
    hipLaunchKernelGGL((mm_lhsT_rhs_bf16_pipe_kernel<BM, BN, BK, W, S, NTB, false>),
                       dim3(grid_tiles(a.M, a.N, BM, BN)), dim3(W * 64), 0, s, (const uint16_t*)a.a,
                       (const uint16_t*)a.b, (uint16_t*)a.out, a.M, a.N, a.K, a.group_m, 1, nullptr);
  }
  return hipGetLastError();
}

// Zeroes the stream-K tile counters of a fresh workspace (a small kernel,
// not hipMemsetAsync, so that a caller may capture the call in a HIP graph).
template <int UNUSED = 0>
__global__ __launch_bounds__(256) void sk_zero_kernel(int* __restrict__ p, int n) {
  for (int i = (int)(blockIdx.x * 256 + threadIdx.x); i < n; i += (int)(gridDim.x * 256)) p[i] = 0;
}

// Stream-K (variants 5 and 6): one workgroup per CU; the counters are
// zeroed first unless the workspace is known to hold zeros.
template <int BM, int BN, int BK, int W, int S, bool NTB>
hipError_t launch_mm_sk(const MiArgs& a, hipStream_t s) {
  const int tiles = grid_tiles(a.M, a.N, BM, BN);
  const int kt = (a.K + BK - 1) / BK;
  const long long grid = streamk_grid(a.cus, tiles, kt);
  if (!a.ws_zeroed) {
    hipLaunchKernelGGL(sk_zero_kernel<0>, dim3((unsigned)((tiles + 255) / 256)), dim3(256), 0, s, (int*)a.ws, tiles);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((mm_lhsT_rhs_bf16_sk_kernel<BM, BN, BK, W, S, NTB>), dim3((unsigned)grid), dim3(W * 64), 0, s,
                     (const uint16_t*)a.a, (const uint16_t*)a.b, (uint16_t*)a.out, a.M, a.N, a.K, a.group_m, a.ws);
  return hipGetLastError();
}

// K split over the waves of a workgroup (variant 4), unsplit or split-K.
template <int BM, int BN, int BK, int W, int S>
hipError_t launch_mm_kw(const MiArgs& a, hipStream_t s) {
  if (a.parts > 1) {
    hipLaunchKernelGGL((mm_lhsT_rhs_bf16_kw_kernel<BM, BN, BK, W, S, true>),
                       dim3(grid_tiles(a.M, a.N, BM, BN) * a.parts), dim3(W * 64), 0, s, (const uint16_t*)a.a,
                       (const uint16_t*)a.b, (uint16_t*)a.out, a.M, a.N, a.K, a.group_m, a.parts, (float*)ws_data(a));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_splitk_sum((const float*)ws_data(a), (uint16_t*)a.out, (size_t)a.M * (size_t)a.N, a.parts, s);
  } else {
    hipLaunchKernelGGL((mm_lhsT_rhs_bf16_kw_kernel<BM, BN, BK, W, S, false>), dim3(grid_tiles(a.M, a.N, BM, BN)),
                       dim3(W * 64), 0, s, (const uint16_t*)a.a, (const uint16_t*)a.b, (uint16_t*)a.out, a.M, a.N,
                       a.K, a.group_m, 1, nullptr);
  }
  return hipGetLastError();
}

template <int BM, int BN, int BK, int W, int S, bool NTB = false>
hipError_t launch_mm_lhs(const MiArgs& a, hipStream_t s) {
  if (a.parts > 1) {
    hipLaunchKernelGGL((mm_lhs_rhs_bf16_pipe_kernel<BM, BN, BK, W, S, NTB, true>),
                       dim3(grid_tiles(a.M, a.N, BM, BN) * a.parts), dim3(W * 64), 0, s, (const uint16_t*)a.a,
                       (const uint16_t*)a.b, (uint16_t*)a.out, a.M, a.N, a.K, a.group_m, a.parts, (float*)ws_data(a));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_splitk_sum((const float*)ws_data(a), (uint16_t*)a.out, (size_t)a.M * (size_t)a.N, a.parts, s);
  } else {
    hipLaunchKernelGGL((mm_lhs_rhs_bf16_pipe_kernel<BM, BN, BK, W, S, NTB, false>),
                       dim3(grid_tiles(a.M, a.N, BM, BN)), dim3(W * 64), 0, s, (const uint16_t*)a.a,
                       (const uint16_t*)a.b, (uint16_t*)a.out, a.M, a.N, a.K, a.group_m, 1, nullptr);
  }
  return hipGetLastError();
}

template <int BM, int BN, int BK, int W, int S>
hipError_t launch_mm_lhs_pair(const MiArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((mm_lhs_rhs_bf16_pair_kernel<BM, BN, BK, W, S>), dim3(grid_tiles(a.M, a.N, BM, BN)),
                     dim3(W * 64), 0, s, (const uint16_t*)a.a, (const uint16_t*)a.b, (uint16_t*)a.out, a.M, a.N, a.K,
                     a.group_m);
  return hipGetLastError();
}

template <int BM, int BN, int BK, int W, int S, bool PRE>
hipError_t launch_rms_bf16(const MiArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((rmsnorm_mm_bf16_kernel<BM, BN, BK, W, S, PRE>), dim3(grid_tiles(a.M, a.N, BM, BN)),
                     dim3(W * 64), 0, s, (const uint16_t*)a.a, (const uint16_t*)a.g, (const uint16_t*)a.b,
                     (uint16_t*)a.out, a.M, a.N, a.K, a.inv_k, a.eps, a.group_m);
  return hipGetLastError();
}

template <int BM, int BN, int BK, int W, int PF>
hipError_t launch_mm_reg(const MiArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((mm_lhsT_rhs_bf16_reg_kernel<BM, BN, BK, W, PF>), dim3(grid_tiles(a.M, a.N, BM, BN)),
                     dim3(W * 64), 0, s, (const uint16_t*)a.a, (const uint16_t*)a.b, (uint16_t*)a.out, a.M, a.N, a.K,
                     a.group_m);
  return hipGetLastError();
}

template <int BM, int BN, int BK, int W, int S, int XS, bool HG, bool NTW, bool SPLIT>
void launch_rms_xreg_one(const MiArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((rmsnorm_mm_bf16_xreg_kernel<BM, BN, BK, W, S, XS, HG, NTW, SPLIT>),
                     dim3(grid_tiles(a.M, a.N, BM, BN) * (SPLIT ? a.parts : 1)), dim3(W * 64), 0, s,
                     (const uint16_t*)a.a, (const uint16_t*)a.g, (const uint16_t*)a.b, (uint16_t*)a.out, a.M, a.N,
                     a.K, a.inv_k, a.eps, a.group_m, SPLIT ? a.parts : 1, SPLIT ? (float*)ws_data(a) : nullptr);
}

template <int BM, int BN, int BK, int W, int S, int XS, bool NTW = false>
hipError_t launch_rms_xreg(const MiArgs& a, hipStream_t s) {
  if (a.parts > 1) {
    // Split-K: the parts' products and sums of squares into ws, then out.
    if (a.g) launch_rms_xreg_one<BM, BN, BK, W, S, XS, true, NTW, true>(a, s);
    else launch_rms_xreg_one<BM, BN, BK, W, S, XS, false, NTW, true>(a, s);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const float* prod = (const float*)ws_data(a);
    launch_splitk_rms_sum(prod, a.parts, prod + (size_t)a.parts * (size_t)a.M * (size_t)a.N, a.parts, a, s);
  } else if (a.g) {
    launch_rms_xreg_one<BM, BN, BK, W, S, XS, true, NTW, false>(a, s);
  } else {
    launch_rms_xreg_one<BM, BN, BK, W, S, XS, false, NTW, false>(a, s);
  }
  return hipGetLastError();
}

// Two-pass fused kernel (variant 13): pass 1 packs x*gamma into the lhsT
// layout and the row sums of squares into the workspace, pass 2 is the
// pipelined lhsT.rhs core with the rms row scale (split: into the
// products, then the fused second pass of split-K).
template <int BM, int BN, int BK, int W, int S>
hipError_t launch_rms_2pass(const MiArgs& a, hipStream_t s) {
  const size_t m = (size_t)a.M, k = (size_t)a.K;
  const int sparts = rms2_parts(a.K);
  char* data = ws_data(a);
  uint16_t* xt = (uint16_t*)data;
  float* ssq = (float*)(data + align256(k * m * 2));
  float* prod = (float*)(data + align256(k * m * 2) + align256((size_t)sparts * m * 4));
  hipLaunchKernelGGL(rms_pack_kernel<0>, dim3((unsigned)((a.M + RP_ROWS - 1) / RP_ROWS), (unsigned)sparts),
                     dim3(RP_WAVES * 64), 0, s, (const uint16_t*)a.a, (const uint16_t*)a.g, xt, ssq, a.M, a.K);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (a.parts > 1) {
    hipLaunchKernelGGL((rmsnorm_mm_bf16_2pass_kernel<BM, BN, BK, W, S, true>),
                       dim3(grid_tiles(a.M, a.N, BM, BN) * a.parts), dim3(W * 64), 0, s, xt, (const uint16_t*)a.b,
                       (uint16_t*)a.out, a.M, a.N, a.K, a.group_m, a.parts, prod, ssq, sparts, a.inv_k, a.eps);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    launch_splitk_rms_sum(prod, a.parts, ssq, sparts, a, s);
  } else {
    hipLaunchKernelGGL((rmsnorm_mm_bf16_2pass_kernel<BM, BN, BK, W, S, false>), dim3(grid_tiles(a.M, a.N, BM, BN)),
                       dim3(W * 64), 0, s, xt, (const uint16_t*)a.b, (uint16_t*)a.out, a.M, a.N, a.K, a.group_m, 1,
                       nullptr, ssq, sparts, a.inv_k, a.eps);
  }
  return hipGetLastError();
}

// Two-pass fused kernel on the paired-load core (variant 15): pass 1 packs
// x*gamma in x's own layout (xg[M][K]) and the row sums of squares, pass 2
// is the paired-load K-contiguous core with the rms row scale.  Unsplit.
template <int BM, int BN, int BK, int W, int S>
hipError_t launch_rms_2pass_pair(const MiArgs& a, hipStream_t s) {
  const size_t m = (size_t)a.M, k = (size_t)a.K;
  const int sparts = rms2_parts(a.K);
  char* data = ws_data(a);
  uint16_t* xg = (uint16_t*)data;
  float* ssq = (float*)(data + align256(k * m * 2));
  hipLaunchKernelGGL(rms_pack_kernel<1>, dim3((unsigned)((a.M + RP_ROWS - 1) / RP_ROWS), (unsigned)sparts),
                     dim3(RP_WAVES * 64), 0, s, (const uint16_t*)a.a, (const uint16_t*)a.g, xg, ssq, a.M, a.K);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((rmsnorm_mm_bf16_2pass_pair_kernel<BM, BN, BK, W, S>), dim3(grid_tiles(a.M, a.N, BM, BN)),
                     dim3(W * 64), 0, s, xg, (const uint16_t*)a.b, (uint16_t*)a.out, a.M, a.N, a.K, a.group_m, ssq,
                     sparts, a.inv_k, a.eps);
  return hipGetLastError();
}

// Fused kernel without gamma (variant 14): one launch of the K-contiguous
// pipelined core that takes the rows' sums of squares from its A operand.
// The C ABI rejects it with gamma.
template <int BM, int BN, int BK, int W, int S>
hipError_t launch_rms_sq(const MiArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((rmsnorm_mm_bf16_sq_kernel<BM, BN, BK, W, S>), dim3(grid_tiles(a.M, a.N, BM, BN)), dim3(W * 64),
                     0, s, (const uint16_t*)a.a, (const uint16_t*)a.b, (uint16_t*)a.out, a.M, a.N, a.K, a.group_m,
                     a.eps, a.inv_k);
  return hipGetLastError();
}

// Fused kernel without gamma on the paired-load K-contiguous core (variant
// 16): one launch, as variant 14.
template <int BM, int BN, int BK, int W, int S>
hipError_t launch_rms_sq_pair(const MiArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((rmsnorm_mm_bf16_sq_pair_kernel<BM, BN, BK, W, S>), dim3(grid_tiles(a.M, a.N, BM, BN)),
                     dim3(W * 64), 0, s, (const uint16_t*)a.a, (const uint16_t*)a.b, (uint16_t*)a.out, a.M, a.N, a.K,
                     a.group_m, a.eps, a.inv_k);
  return hipGetLastError();
}

// Explicit instantiation of one config's kernel (namespace scope); every
// table row needs its kernel instantiated in the same translation unit so
// the host launch stub is emitted there.
#define MI_MM_INST(BM, BN, BK, W, S)                                                                      \
  template __global__ void mm_lhsT_rhs_bf16_kernel<BM, BN, BK, W, S>(const uint16_t*, const uint16_t*, \
                                                                      uint16_t*, int, int, int, int);
// Pipelined lhsT matmul (variant 1; MI_MMPN: variant 3, rhs non-temporal),
// unsplit and split-K instances.
#define MI_MMP_INST(BM, BN, BK, W, S)                                                     \
  template __global__ void mm_lhsT_rhs_bf16_pipe_kernel<BM, BN, BK, W, S, false, false>( \
      const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, int, float*);     \
  template __global__ void mm_lhsT_rhs_bf16_pipe_kernel<BM, BN, BK, W, S, false, true>(  \
      const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, int, float*);
#define MI_MMPN_INST(BM, BN, BK, W, S)                                                   \
  template __global__ void mm_lhsT_rhs_bf16_pipe_kernel<BM, BN, BK, W, S, true, false>( \
      const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, int, float*);    \
  template __global__ void mm_lhsT_rhs_bf16_pipe_kernel<BM, BN, BK, W, S, true, true>(  \
      const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, int, float*);
// Stream-K lhsT matmul (variant 5; MI_MMSN: variant 6, rhs non-temporal).
#define MI_MMS_INST(BM, BN, BK, W, S)                                                 \
  template __global__ void mm_lhsT_rhs_bf16_sk_kernel<BM, BN, BK, W, S, false>(      \
      const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, char*);
#define MI_MMSN_INST(BM, BN, BK, W, S)                                                \
  template __global__ void mm_lhsT_rhs_bf16_sk_kernel<BM, BN, BK, W, S, true>(       \
      const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, char*);
// K split over the waves (variant 4), unsplit and split-K instances.
#define MI_MMW_INST(BM, BN, BK, W, S)                                                  \
  template __global__ void mm_lhsT_rhs_bf16_kw_kernel<BM, BN, BK, W, S, false>(       \
      const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, int, float*);  \
  template __global__ void mm_lhsT_rhs_bf16_kw_kernel<BM, BN, BK, W, S, true>(        \
      const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, int, float*);
#define MI_MMK_INST(BM, BN, BK, W, S)                                                    \
  template __global__ void mm_lhs_rhs_bf16_pipe_kernel<BM, BN, BK, W, S, false, false>( \
      const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, int, float*);    \
  template __global__ void mm_lhs_rhs_bf16_pipe_kernel<BM, BN, BK, W, S, false, true>(  \
      const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, int, float*);
#define MI_MMKN_INST(BM, BN, BK, W, S)                                                  \
  template __global__ void mm_lhs_rhs_bf16_pipe_kernel<BM, BN, BK, W, S, true, false>( \
      const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, int, float*);   \
  template __global__ void mm_lhs_rhs_bf16_pipe_kernel<BM, BN, BK, W, S, true, true>(  \
      const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, int, float*);
#define MI_MMKP_INST(BM, BN, BK, W, S)                                                                     \
  template __global__ void mm_lhs_rhs_bf16_pair_kernel<BM, BN, BK, W, S>(const uint16_t*, const uint16_t*, \
                                                                          uint16_t*, int, int, int, int);
#define MI_RMS_INST(BM, BN, BK, W, S, PRE)                                        \
  template __global__ void rmsnorm_mm_bf16_kernel<BM, BN, BK, W, S, (PRE != 0)>( \
      const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, int, int, int, float, float, int);
#define MI_MMR_INST(BM, BN, BK, W, PF)                                                                       \
  template __global__ void mm_lhsT_rhs_bf16_reg_kernel<BM, BN, BK, W, PF>(const uint16_t*, const uint16_t*, \
                                                                           uint16_t*, int, int, int, int);

// Variant 4 stages x through a 2-slot register ring, variant 5 a 3-slot one.
// Each with and without gamma, unsplit and split-K.
#define MI_RMSX_ONE(BM, BN, BK, W, S, XS, HG, NTW, SPLIT)                                                  \
  template __global__ void rmsnorm_mm_bf16_xreg_kernel<BM, BN, BK, W, S, XS, HG, NTW, SPLIT>(              \
      const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, int, int, int, float, float, int, int, \
      float*);
#define MI_RMSX_INST(BM, BN, BK, W, S, XS)              \
  MI_RMSX_ONE(BM, BN, BK, W, S, XS, true, false, false)  \
  MI_RMSX_ONE(BM, BN, BK, W, S, XS, false, false, false) \
  MI_RMSX_ONE(BM, BN, BK, W, S, XS, true, false, true)   \
  MI_RMSX_ONE(BM, BN, BK, W, S, XS, false, false, true)

// Variants 11 / 12: 4 / 5 with W read non-temporally (skinny M).
#define MI_RMSXN_INST(BM, BN, BK, W, S, XS)           \
  MI_RMSX_ONE(BM, BN, BK, W, S, XS, true, true, false)  \
  MI_RMSX_ONE(BM, BN, BK, W, S, XS, false, true, false) \
  MI_RMSX_ONE(BM, BN, BK, W, S, XS, true, true, true)   \
  MI_RMSX_ONE(BM, BN, BK, W, S, XS, false, true, true)

// Variant 13: the main pass of the two-pass fused kernel, unsplit and split.
#define MI_RMS2_INST(BM, BN, BK, W, S)                                                                       \
  template __global__ void rmsnorm_mm_bf16_2pass_kernel<BM, BN, BK, W, S, false>(                           \
      const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, int, float*, const float*, int, float, \
      float);                                                                                                \
  template __global__ void rmsnorm_mm_bf16_2pass_kernel<BM, BN, BK, W, S, true>(                            \
      const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, int, float*, const float*, int, float, \
      float);

// Variant 15: the main pass of the two-pass fused kernel on the paired-load core.
#define MI_RMS2P_INST(BM, BN, BK, W, S)                                                                         \
  template __global__ void rmsnorm_mm_bf16_2pass_pair_kernel<BM, BN, BK, W, S>(                                \
      const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, const float*, int, float, float);

// Variant 14: the fused kernel without gamma.
#define MI_RMSQ_INST(BM, BN, BK, W, S)                                                                     \
  template __global__ void rmsnorm_mm_bf16_sq_kernel<BM, BN, BK, W, S>(const uint16_t*, const uint16_t*, \
                                                                       uint16_t*, int, int, int, int, float, float);
// Variant 16: the fused kernel without gamma on the paired-load core.
#define MI_RMSQP_INST(BM, BN, BK, W, S)                                                                       \
  template __global__ void rmsnorm_mm_bf16_sq_pair_kernel<BM, BN, BK, W, S>(const uint16_t*, const uint16_t*, \
                                                                            uint16_t*, int, int, int, int,     \
                                                                            float, float);

// Table rows.
#define MI_MM_ROW(BM, BN, BK, W, S)                                                                  \
  {MI_KERNEL_MATMUL_LHST_RHS_BF16, {BM, BN, BK, W, S, 1, 0, 0}, MatmulCfg<BM, BN, BK, W, S>::LDS_BYTES, \
   &launch_mm_bf16<BM, BN, BK, W, S>},
#define MI_MMP_ROW(BM, BN, BK, W, S)                                                               \
  {MI_KERNEL_MATMUL_LHST_RHS_BF16, {BM, BN, BK, W, S, 1, 0, 1}, PipeCfg<BM, BN, BK, W, S>::LDS_BYTES, \
   &launch_mm_pipe<BM, BN, BK, W, S>},
// Pipelined matmul with rhs streamed non-temporally: variant 3.
#define MI_MMPN_ROW(BM, BN, BK, W, S)                                                              \
  {MI_KERNEL_MATMUL_LHST_RHS_BF16, {BM, BN, BK, W, S, 1, 0, 3}, PipeCfg<BM, BN, BK, W, S>::LDS_BYTES, \
   &launch_mm_pipe<BM, BN, BK, W, S, true>},
// Stream-K pipelined matmul: variant 5 (rhs cached), variant 6 (rhs non-temporal).
#define MI_MMS_ROW(BM, BN, BK, W, S)                                                               \
  {MI_KERNEL_MATMUL_LHST_RHS_BF16, {BM, BN, BK, W, S, 1, 0, 5}, PipeCfg<BM, BN, BK, W, S>::LDS_BYTES, \
   &launch_mm_sk<BM, BN, BK, W, S, false>},
#define MI_MMSN_ROW(BM, BN, BK, W, S)                                                              \
  {MI_KERNEL_MATMUL_LHST_RHS_BF16, {BM, BN, BK, W, S, 1, 0, 6}, PipeCfg<BM, BN, BK, W, S>::LDS_BYTES, \
   &launch_mm_sk<BM, BN, BK, W, S, true>},
// Pipelined matmul with each K tile's sub-steps split over the waves: variant 4.
#define MI_MMW_ROW(BM, BN, BK, W, S)                                                               \
  {MI_KERNEL_MATMUL_LHST_RHS_BF16, {BM, BN, BK, W, S, 1, 0, 4}, lds_mm_kw(BM, BN, BK, W, S), \
   &launch_mm_kw<BM, BN, BK, W, S>},
// matmul_lhs_rhs (K-contiguous lhs) on the pipelined core: variant 0.
#define MI_MMK_ROW(BM, BN, BK, W, S)                                                                \
  {MI_KERNEL_MATMUL_LHS_RHS_BF16, {BM, BN, BK, W, S, 1, 0, 0}, PipeCfg<BM, BN, BK, W, S>::LDS_BYTES, \
   &launch_mm_lhs<BM, BN, BK, W, S>},
// matmul_lhs_rhs with rhs read non-temporally: variant 2.
#define MI_MMKN_ROW(BM, BN, BK, W, S)                                                              \
  {MI_KERNEL_MATMUL_LHS_RHS_BF16, {BM, BN, BK, W, S, 1, 0, 2}, PipeCfg<BM, BN, BK, W, S>::LDS_BYTES, \
   &launch_mm_lhs<BM, BN, BK, W, S, true>},
// matmul_lhs_rhs with A loaded two K tiles at a time: variant 1.
#define MI_MMKP_ROW(BM, BN, BK, W, S)                                                               \
  {MI_KERNEL_MATMUL_LHS_RHS_BF16, {BM, BN, BK, W, S, 1, 0, 1}, PairCfg<BM, BN, BK, W, S>::LDS_BYTES, \
   &launch_mm_lhs_pair<BM, BN, BK, W, S>},
#define MI_RMS_ROW(BM, BN, BK, W, S, PRE)                                                            \
  {MI_KERNEL_RMSNORM_MATMUL_BF16, {BM, BN, BK, W, S, 1, 0, PRE}, RmsCfg<BM, BN, BK, W, S>::LDS_BYTES,   \
   &launch_rms_bf16<BM, BN, BK, W, S, (PRE != 0)>},

// Register-ring matmul (variant 2): lds_stages carries the prefetch depth PF
// (its LDS is always two stages).
#define MI_MMR_ROW(BM, BN, BK, W, PF)                                                         \
  {MI_KERNEL_MATMUL_LHST_RHS_BF16, {BM, BN, BK, W, PF, 1, 0, 2}, lds_mm_reg(BM, BN, BK, W), \
   &launch_mm_reg<BM, BN, BK, W, PF>},

#define MI_RMSX_ROW(BM, BN, BK, W, S, XS)                                                                   \
  {MI_KERNEL_RMSNORM_MATMUL_BF16, {BM, BN, BK, W, S, 1, 0, 2 + XS}, XregCfg<BM, BN, BK, W, S>::LDS_BYTES, \
   &launch_rms_xreg<BM, BN, BK, W, S, XS>, XregCfg<BM, BN, BK, W, S>::GK_MAX},

#define MI_RMSXN_ROW(BM, BN, BK, W, S, XS)                                                                  \
  {MI_KERNEL_RMSNORM_MATMUL_BF16, {BM, BN, BK, W, S, 1, 0, 9 + XS}, XregCfg<BM, BN, BK, W, S>::LDS_BYTES, \
   &launch_rms_xreg<BM, BN, BK, W, S, XS, true>, XregCfg<BM, BN, BK, W, S>::GK_MAX},

#define MI_RMSQ_ROW(BM, BN, BK, W, S)                                                                  \
  {MI_KERNEL_RMSNORM_MATMUL_BF16, {BM, BN, BK, W, S, 1, 0, 14}, PipeCfg<BM, BN, BK, W, S>::LDS_BYTES, \
   &launch_rms_sq<BM, BN, BK, W, S>},
#define MI_RMSQP_ROW(BM, BN, BK, W, S)                                                                 \
  {MI_KERNEL_RMSNORM_MATMUL_BF16, {BM, BN, BK, W, S, 1, 0, 16}, PairCfg<BM, BN, BK, W, S>::LDS_BYTES, \
   &launch_rms_sq_pair<BM, BN, BK, W, S>},

#define MI_RMS2_ROW(BM, BN, BK, W, S)                                                               \
  {MI_KERNEL_RMSNORM_MATMUL_BF16, {BM, BN, BK, W, S, 1, 0, 13}, lds_rms2(BM, BN, BK, W, S),         \
   &launch_rms_2pass<BM, BN, BK, W, S>},
#define MI_RMS2P_ROW(BM, BN, BK, W, S)                                                              \
  {MI_KERNEL_RMSNORM_MATMUL_BF16, {BM, BN, BK, W, S, 1, 0, 15}, lds_rms2_pair(BM, BN, BK, W, S),    \
   &launch_rms_2pass_pair<BM, BN, BK, W, S>},

// The 72-point search grid for one (BM, BN): BK in {32,64} x waves in {4,8} x
// stages in {1,2}.  X is a row macro taking (BM, BN, BK, W, S, ...).
#define MI_GRID_BK_W_S(X, BM, BN, ...) \
  X(BM, BN, 32, 4, 1 __VA_ARGS__)      \
  X(BM, BN, 32, 4, 2 __VA_ARGS__)      \
  X(BM, BN, 64, 4, 1 __VA_ARGS__)      \
  X(BM, BN, 64, 4, 2 __VA_ARGS__)      \
  X(BM, BN, 32, 8, 1 __VA_ARGS__)      \
  X(BM, BN, 32, 8, 2 __VA_ARGS__)      \
  X(BM, BN, 64, 8, 1 __VA_ARGS__)      \
  X(BM, BN, 64, 8, 2 __VA_ARGS__)
#define MI_GRID_BK_W4_S(X, BM, BN, ...) \
  X(BM, BN, 32, 4, 1 __VA_ARGS__)       \
  X(BM, BN, 32, 4, 2 __VA_ARGS__)       \
  X(BM, BN, 64, 4, 1 __VA_ARGS__)       \
  X(BM, BN, 64, 4, 2 __VA_ARGS__)

typedef const MiEntry* (*TableFn)(int*);

// The list of instance tables the C ABI serves.  libmi_kernels.so defines it
// in mi_tables.hip (every prebuilt table); a just-in-time autotune library
// defines it in its one generated translation unit (one instance).
const TableFn* table_list(int* n);

// Per-translation-unit tables (defined in mm_bf16_*.hip, rms_bf16_*.hip,
// mm_f32.hip).
const MiEntry* table_mm_bm32(int* n);
const MiEntry* table_mm_bm64(int* n);
const MiEntry* table_mm_bm128(int* n);
const MiEntry* table_mm_bm256(int* n);
const MiEntry* table_mm_pipe(int* n);
const MiEntry* table_mm_sk(int* n);
const MiEntry* table_mm_kw(int* n);
const MiEntry* table_mm_reg(int* n);
const MiEntry* table_mm_lhs(int* n);
const MiEntry* table_rms_xreg(int* n);
const MiEntry* table_rms_2pass(int* n);
const MiEntry* table_rms_sq(int* n);
const MiEntry* table_rms_bm64(int* n);
const MiEntry* table_rms_bm128(int* n);
const MiEntry* table_rms_bm256(int* n);
const MiEntry* table_f32(int* n);

}  // namespace mi
