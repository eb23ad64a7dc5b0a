// mi_probe.hip -- measurement probes for bench.py, built as libmi_probe.so.
// Not part of the kernel_library C ABI (include/mi_kernels.h): nothing on the
// kernel path calls them.
//
// mi_probe_clocked_lhsT_rhs: the pipelined lhsT.rhs kernel (matmul variant 1,
//   the body the benchmark ships) with each workgroup recording, around its
//   whole run, its engine cycles (s_memtime) and its real time
//   (s_memrealtime, a 100 MHz counter).  Summed over workgroups,
//   cycles / (ticks / 100 MHz) is the engine clock the kernel ran at.  The
//   two counter reads are the only difference from the product kernel.
//
// mi_probe_mfma: the MFMA work of one 128x128 wave tile -- per 16-wide K
//   step, 4 x 4 v_mfma_f32_32x32x16_bf16 -- on every SIMD of the GPU
//   (256 workgroups of 4 waves), with no global memory traffic:
//     mode 0: operands from registers, 4 rotating sets loaded once from
//             `src` (each MFMA sees different bits from the one before);
//     mode 1: operands read from two 64 x 256 bf16 LDS panels filled from
//             `src`, with the transposing reads (ds_read_b64_tr_b16) and the
//             read/MFMA interleave of the pipelined kernel.
//   On data drawn like the benchmark's, these are the rates of the MFMA
//   pipe alone, and with its operand reads, under the chip's power limit:
//   ceilings for any kernel that has to run those instructions.
//
// mi_probe_panel_stream: the kernels' K-panel loads alone -- LDS-direct
//   buffer_load_dwordx4 ... lds, one 1 KiB chunk (64 lanes x 16 bytes) per
//   wave instruction -- with no LDS reads and no MFMA.  One workgroup per
//   CU (its static LDS keeps a second one off the CU), every wave streaming
//   consecutive chunks of a `region`-byte buffer with INFLIGHT loads in
//   flight.  A region that fits in one XCD's L2 gives the L2 -> LDS rate a
//   CU's panel loads can reach; larger ones the MALL and HBM paths.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../mi_gemm.hpp"

namespace mi {
namespace probe {

template <int BM, int BN, int BK, int W, int S>
__global__ __launch_bounds__(W * 64) void clocked_lhsT_rhs_kernel(const uint16_t* __restrict__ a,
                                                                  const uint16_t* __restrict__ b,
                                                                  uint16_t* __restrict__ out, int M, int N, int K,
                                                                  int group_m, unsigned long long* __restrict__ clk) {
  __shared__ __attribute__((aligned(1024))) char smem[PipeCfg<BM, BN, BK, W, S>::LDS_BYTES];
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  mm_pipe_body<BM, BN, BK, W, S, false>(a, b, out, M, N, K, group_m, smem);
  const unsigned long long c1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) {
    clk[2 * blockIdx.x] = c1 - c0;
    clk[2 * blockIdx.x + 1] = r1 - r0;
  }
}

constexpr int PTM = 4, PTN = 4, PSETS = 4, PWG = 256;

__global__ __launch_bounds__(256) void mfma_regs_kernel(const bf16x8_t* __restrict__ src, long long chunks,
                                                        float* __restrict__ out, int iters,
                                                        unsigned long long* __restrict__ clk) {
  const int lane = threadIdx.x & 63;
  const long long gw = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  bf16x8_t a[PSETS][PTM], b[PSETS][PTN];
#pragma unroll
  for (int s = 0; s < PSETS; ++s) {
#pragma unroll
    for (int i = 0; i < PTM; ++i) a[s][i] = src[(((gw * PSETS + s) * (PTM + PTN) + i) * 64 + lane) % chunks];
#pragma unroll
    for (int j = 0; j < PTN; ++j) b[s][j] = src[(((gw * PSETS + s) * (PTM + PTN) + PTM + j) * 64 + lane) % chunks];
  }
  f32x16_t acc[PTM][PTN];
#pragma unroll
  for (int i = 0; i < PTM; ++i)
#pragma unroll
    for (int j = 0; j < PTN; ++j) acc[i][j] = f32x16_t{};
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int s = 0; s < PSETS; ++s)
#pragma unroll
      for (int i = 0; i < PTM; ++i)
#pragma unroll
        for (int j = 0; j < PTN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[s][j], a[s][i], acc[i][j], 0, 0, 0);
  }
  const unsigned long long c1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < PTM; ++i)
#pragma unroll
    for (int j = 0; j < PTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) sum += acc[i][j][r];
  out[gw * 64 + lane] = sum;
  if (threadIdx.x == 0) {
    clk[2 * blockIdx.x] = c1 - c0;
    clk[2 * blockIdx.x + 1] = r1 - r0;
  }
}

// Two panels of 64 K rows x 256 columns (the 256x256 tile's A and B panels
// at four 16-wide K steps); waves in a 2x2 grid of 128x128 wave tiles.
__global__ __launch_bounds__(256) void mfma_lds_kernel(const uint16_t* __restrict__ src, long long elems,
                                                       float* __restrict__ out, int iters,
                                                       unsigned long long* __restrict__ clk) {
  constexpr int ROWB = 256 * 2, PANEL = 64 * ROWB;
  __shared__ __attribute__((aligned(1024))) char smem[2 * PANEL];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < 2 * PANEL / 2; i += 256)
    ((uint16_t*)smem)[i] = src[((long long)blockIdx.x * (2 * PANEL / 2) + i) % elems];
  __syncthreads();
  TrFrag<256, PTM> fa;
  TrFrag<256, PTN> fb;
  fa.init(lane, (wave / 2) * 128);
  fb.init(lane, (wave % 2) * 128);
  f32x16_t acc[PTM][PTN];
#pragma unroll
  for (int i = 0; i < PTM; ++i)
#pragma unroll
    for (int j = 0; j < PTN; ++j) acc[i][j] = f32x16_t{};
  bf16x8_t af[2][PTM], bf[2][PTN];
  auto rd = [&](int kk, int buf) {
#pragma unroll
    for (int t = 0; t < PTM; ++t)
      af[buf][t] = read_tr_frag(smem, (kk * 16) * ROWB + fa.off[t], (kk * 16 + 4) * ROWB + fa.off[t]);
#pragma unroll
    for (int t = 0; t < PTN; ++t)
      bf[buf][t] = read_tr_frag(smem, PANEL + (kk * 16) * ROWB + fb.off[t], PANEL + (kk * 16 + 4) * ROWB + fb.off[t]);
  };
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  rd(0, 0);
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      rd((kk + 1) & 3, (kk + 1) & 1);
#pragma unroll
      for (int i = 0; i < PTM; ++i)
#pragma unroll
        for (int j = 0; j < PTN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[kk & 1][j], af[kk & 1][i], acc[i][j], 0, 0, 0);
      interleave_mfma_ds<PTM * PTN, 2 * (PTM + PTN)>();
    }
  }
  const unsigned long long c1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < PTM; ++i)
#pragma unroll
    for (int j = 0; j < PTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) sum += acc[i][j][r];
  out[(long long)blockIdx.x * 256 + threadIdx.x] = sum;
  if (threadIdx.x == 0) {
    clk[2 * blockIdx.x] = c1 - c0;
    clk[2 * blockIdx.x + 1] = r1 - r0;
  }
}

constexpr int kStreamLds = 128 * 1024;

template <int W, int INF>
__global__ __launch_bounds__(W * 64) void panel_stream_kernel(const char* __restrict__ src, uint32_t region,
                                                             int row_bytes, uint32_t pitch, int rounds,
                                                             unsigned long long* __restrict__ clk) {
  static_assert(W * INF * 1024 <= kStreamLds && INF < 64, "ring of INF 1 KiB slots per wave");
  __shared__ __attribute__((aligned(1024))) char smem[kStreamLds];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(src, region);
  // The buffer is a row-major matrix of `pitch`-byte rows; a panel is
  // `row_bytes` of each row (the K rows of an MN-contiguous operand panel).
  // A 1 KiB load covers 1024 / row_bytes consecutive rows of one panel:
  // lane l takes row l*16 / row_bytes, bytes (l*16) % row_bytes.  Each wave
  // walks its panel's rows from a spread-out start; panels of different
  // waves sit at different column offsets.
  const uint32_t rows = region / pitch, rpc = 1024u / (uint32_t)row_bytes;
  const uint32_t panels = pitch / (uint32_t)row_bytes;
  const unsigned long long gw = (unsigned long long)blockIdx.x * W + (unsigned)wave;
  const uint32_t col0 = (uint32_t)(gw % panels) * (uint32_t)row_bytes;
  const uint32_t lrow = (uint32_t)lane * 16u / (uint32_t)row_bytes, lcol = (uint32_t)lane * 16u % (uint32_t)row_bytes;
  uint32_t r0 = (uint32_t)(gw * 977ull % (rows / rpc)) * rpc;
  char* ring = smem + wave * INF * 1024;
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  for (int r = 0; r < rounds; ++r)
    static_for<INF>([&](auto s_c) __attribute__((always_inline)) {
      vm_wait<INF - 1>();  // the load that last filled this slot has landed
      lds_dma16(rs, ring + decltype(s_c)::value * 1024, (r0 + lrow) * pitch + col0 + lcol);
      r0 = r0 + rpc >= rows ? 0 : r0 + rpc;
    });
  wait_vmem();
  const unsigned long long c1 = __builtin_amdgcn_s_memtime();
  const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) {
    clk[2 * blockIdx.x] = c1 - c0;
    clk[2 * blockIdx.x + 1] = t1 - t0;
  }
}

#define MI_STREAM_CONFIGS(X) X(4, 2) X(4, 4) X(4, 8) X(4, 16) X(4, 32) X(8, 4) X(8, 8) X(8, 16)

typedef void (*StreamFn)(const char*, uint32_t, int, uint32_t, int, int, unsigned long long*, hipStream_t);
template <int W, int INF>
void launch_stream(const char* src, uint32_t region, int row_bytes, uint32_t pitch, int rounds, int wgs,
                   unsigned long long* clk, hipStream_t s) {
  hipLaunchKernelGGL((panel_stream_kernel<W, INF>), dim3(wgs), dim3(W * 64), 0, s, src, region, row_bytes, pitch,
                     rounds, clk);
}
struct StreamEntry {
  int w, inf;
  StreamFn fn;
};
#define MI_STREAM_ROW(W, INF) {W, INF, &launch_stream<W, INF>},
const StreamEntry kStream[] = {MI_STREAM_CONFIGS(MI_STREAM_ROW)};

// The configs of the clocked twin: the pipelined configs the benchmark's
// 8192^3 sweep ships.
#define MI_PROBE_CONFIGS(X) \
  X(256, 256, 32, 4, 2)     \
  X(256, 256, 32, 4, 3)     \
  X(256, 256, 32, 4, 4)     \
  X(256, 256, 64, 4, 2)     \
  X(256, 256, 32, 8, 3)     \
  X(256, 256, 64, 8, 2)     \
  X(128, 512, 32, 8, 3)     \
  X(128, 256, 32, 4, 3)     \
  X(128, 128, 64, 4, 3)     \
  X(64, 128, 64, 4, 4)

typedef void (*ClockedFn)(const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, unsigned long long*,
                          hipStream_t);

template <int BM, int BN, int BK, int W, int S>
void launch_clocked(const uint16_t* a, const uint16_t* b, uint16_t* out, int M, int N, int K, int group_m,
                    unsigned long long* clk, hipStream_t s) {
  const int grid = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  hipLaunchKernelGGL((clocked_lhsT_rhs_kernel<BM, BN, BK, W, S>), dim3(grid), dim3(W * 64), 0, s, a, b, out, M, N, K,
                     group_m, clk);
}

struct ClockedEntry {
  int bm, bn, bk, w, s;
  ClockedFn fn;
};

#define MI_PROBE_ROW(BM, BN, BK, W, S) {BM, BN, BK, W, S, &launch_clocked<BM, BN, BK, W, S>},
const ClockedEntry kClocked[] = {MI_PROBE_CONFIGS(MI_PROBE_ROW)};

}  // namespace probe
}  // namespace mi

extern "C" {

// Clocked twin of the pipelined lhsT.rhs kernel (variant 1) at `cfg` (one
// of MI_PROBE_CONFIGS, split_k 1).  clk receives 2 uint64 per workgroup
// (engine cycles, 100 MHz ticks), ceil(M/bm) * ceil(N/bn) workgroups.
// Returns 0, MI_E_NO_INSTANCE for a config without a twin, MI_E_ARGS /
// MI_E_ALIGN for bad arguments, or -hipError_t.
int mi_probe_clocked_lhsT_rhs(const void* lhsT, const void* rhs, void* out, int M, int N, int K,
                              const mi_tile_cfg* cfg, unsigned long long* clk, void* stream) {
  if (!lhsT || !rhs || !out || !clk || !cfg || M <= 0 || N <= 0 || K <= 0) return MI_E_ARGS;
  if (M % 8 || N % 8 || ((uintptr_t)lhsT | (uintptr_t)rhs | (uintptr_t)out) & 15) return MI_E_ALIGN;
  if (cfg->variant != 1 || cfg->split_k != 1) return MI_E_NO_INSTANCE;
  if (2ull * (unsigned long long)(K + cfg->block_k) * (unsigned long long)M > 0xFFFFFFFFull ||
      2ull * (unsigned long long)(K + cfg->block_k) * (unsigned long long)N > 0xFFFFFFFFull)
    return MI_E_RANGE;
  for (const mi::probe::ClockedEntry& e : mi::probe::kClocked) {
    if (e.bm == cfg->block_m && e.bn == cfg->block_n && e.bk == cfg->block_k && e.w == cfg->waves &&
        e.s == cfg->lds_stages) {
      e.fn((const uint16_t*)lhsT, (const uint16_t*)rhs, (uint16_t*)out, M, N, K,
           cfg->group_m > 0 ? cfg->group_m : 8, clk, (hipStream_t)stream);
      const hipError_t err = hipGetLastError();
      return err == hipSuccess ? MI_OK : -(int)err;
    }
  }
  return MI_E_NO_INSTANCE;
}

// The MFMA ceiling probe: 256 workgroups x 4 waves, each wave running
// iters * 64 MFMAs (32x32x16 bf16) on operands drawn from src (bf16,
// src_elems >= 65536 elements): mode 0 from registers, mode 1 through LDS.
// out receives 65536 floats (keeps the work live), clk 2 uint64 per
// workgroup.  Returns 0, MI_E_ARGS or -hipError_t.
int mi_probe_mfma(const void* src, long long src_elems, float* out, unsigned long long* clk, int iters, int mode,
                  void* stream) {
  if (!src || !out || !clk || src_elems < 65536 || iters <= 0 || (mode != 0 && mode != 1) ||
      ((uintptr_t)src & 15))
    return MI_E_ARGS;
  if (mode == 0)
    hipLaunchKernelGGL(mi::probe::mfma_regs_kernel, dim3(mi::probe::PWG), dim3(256), 0, (hipStream_t)stream,
                       (const mi::bf16x8_t*)src, src_elems / 8, out, iters, clk);
  else
    hipLaunchKernelGGL(mi::probe::mfma_lds_kernel, dim3(mi::probe::PWG), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)src, src_elems, out, iters, clk);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? MI_OK : -(int)err;
}

// The panel-load stream probe: `wgs` workgroups of `waves` waves, each wave
// issuing rounds * inflight LDS-direct 1 KiB loads with `inflight` in
// flight (waves/inflight one of MI_STREAM_CONFIGS), reading `row_bytes`
// of each `pitch`-byte row of src[0, region): the panel loads of an
// operand whose rows are `pitch` bytes long.  row_bytes: a power of two in
// [16, 1024]; pitch: a multiple of row_bytes; region: a multiple of
// pitch * 1024 / row_bytes, below 4 GiB.  clk receives 2 uint64 per
// workgroup.  Returns 0, MI_E_ARGS, MI_E_NO_INSTANCE or -hipError_t.
int mi_probe_panel_stream(const void* src, unsigned long long region, int row_bytes, unsigned long long pitch,
                          int waves, int inflight, int wgs, int rounds, unsigned long long* clk, void* stream) {
  if (!src || !clk || row_bytes < 16 || row_bytes > 1024 || (row_bytes & (row_bytes - 1)) || pitch < 16 ||
      pitch % row_bytes || region >= (1ull << 32) || region < pitch * (1024 / row_bytes) ||
      region % (pitch * (1024 / row_bytes)) || wgs <= 0 || rounds <= 0 || ((uintptr_t)src & 15))
    return MI_E_ARGS;
  for (const mi::probe::StreamEntry& e : mi::probe::kStream) {
    if (e.w == waves && e.inf == inflight) {
      e.fn((const char*)src, (uint32_t)region, row_bytes, (uint32_t)pitch, rounds, wgs, clk, (hipStream_t)stream);
      const hipError_t err = hipGetLastError();
      return err == hipSuccess ? MI_OK : -(int)err;
    }
  }
  return MI_E_NO_INSTANCE;
}

}  // extern "C"
