// mi_gemm.hpp -- gfx950 (CDNA4) kernels of the kernel_library hot path.
//
// Two templated kernels share one MFMA core:
//   mm_lhsT_rhs_bf16<BM,BN,BK,WAVES,STAGES>    out = lhsT^T . rhs
//   rmsnorm_mm_bf16<BM,BN,BK,WAVES,STAGES,PRE> out = rmsnorm(x) * gamma . W
//
// Both reference kernels keep the contraction axis K as the row index of
// every operand (lhsT[K,M], rhs[K,N]; reference
// kernel_library/matmul/lhsT_rhs/kernel_hand_90.92mfu.py:101-105), so a
// 16-byte global load brings 8 consecutive M (or N) values of one K row.
// The MFMA wants 8 consecutive K values per lane.  The transpose happens in
// the LDS read: panels are copied HBM->LDS unchanged by buffer_load ... lds
// (no VGPR staging), and each MFMA operand is assembled by two
// ds_read_b64_tr_b16, which read a 4x16 block of 16-bit elements across a
// 16-lane group and hand lane j the 4 values of column j.
//
// MFMA v_mfma_f32_32x32x16_bf16 lane layout (gfx950, checked on hardware):
//   A (32x16): lane l holds A[l%32][8*(l/32) + 0..7]
//   B (16x32): lane l holds B[8*(l/32) + 0..7][l%32]
//   D (32x32): lane l, reg r holds D[8*(r/4) + 4*(l/32) + r%4][l%32]
// The kernels issue mfma(Bfrag, Afrag), i.e. they compute out^T per 32x32
// tile, so each lane ends with 4 consecutive N values of one output row.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <numeric>
#include <type_traits>
#include <utility>

#include "mi_legal.hpp"
#include "mi_streamk.hpp"

namespace mi {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

#define MI_LDS __attribute__((address_space(3)))

// gfx9 buffer descriptor word 3 (raw buffer, 32-bit element format).
constexpr int kRsrcWord3 = 0x00020000;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kRsrcWord3);
}
// f(std::integral_constant<int, i>{}) for i = 0 .. N-1, unrolled: loop
// bodies whose LDS stage is a compile-time constant address their operands
// with immediate offsets.
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}
// f(integral_constant<I>) for I = 0, 1, ... while it returns true (at most
// N calls).  The calls nest, so no control-flow path runs call i+1 after
// skipping call i (wait counts that assume every earlier call hold on
// every path).
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_while(F&& f) {
  if constexpr (I < N) {
    if (f(std::integral_constant<int, I>{})) static_while<N, I + 1>(f);
  }
}

// Descriptor of bytes [off, bytes) of p (off <= bytes, wave-uniform).  A
// K tile's offset rides in the scalar base address, so the per-lane offsets
// stay the same for every tile and a load needs no vector add; loads past
// the end still read zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_from(const void* p, uint32_t bytes, uint32_t off) {
  off = __builtin_amdgcn_readfirstlane(off);  // keeps the descriptor in SGPRs
  return make_rsrc((const char*)p + off, bytes - off);
}

// s_waitcnt vmcnt(0): every outstanding vector-memory load (including the
// LDS-direct loads) has landed.  expcnt/lgkmcnt fields are left at max.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// s_waitcnt vmcnt(N): at most N vector-memory loads of this wave still in
// flight (gfx9 encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14).
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// One LDS-direct load: 16 bytes per lane from the buffer at byte `voff` to
// LDS at `lds` + 16 * lane (buffer_load_dwordx4 ... lds, base address in M0).
// Issued as inline assembly so that the compiler does not treat it as a
// store that every later LDS read must wait for: the kernels order these
// loads against LDS reads themselves (vm_wait / wait_vmem, then a barrier).
// NT sets the non-temporal cache policy: data read once (a streamed
// operand) then does not displace reused data in L2 and the MALL, which
// nearly doubles the read bandwidth of a large streamed operand.
template <bool NT = false>
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rs, char* lds, uint32_t voff) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(MI_LDS char*)lds;
  if constexpr (NT)
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen nt lds" ::"v"(voff), "s"(rs), "{m0}"(m0) : "memory");
  else
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rs), "{m0}"(m0) : "memory");
}

// Wave grid: WM x WN waves, each owning a (BM/WM) x (BN/WN) block that is
// a whole number of 32x32 MFMA tiles.  The most square wave block wins.
template <int BM, int BN, int WAVES>
struct WaveGrid {
  static constexpr int pick() {
    int best = -1, bestd = 1 << 30;
    for (int wm = 1; wm <= WAVES; wm *= 2) {
      const int wn = WAVES / wm;
      if (wm * wn != WAVES || BM % wm || BN % wn) continue;
      const int tm = BM / wm, tn = BN / wn;
      if (tm < 32 || tn < 32 || tm % 32 || tn % 32) continue;
      const int d = tm > tn ? tm - tn : tn - tm;
      if (d < bestd) { bestd = d; best = wm; }
    }
    return best;
  }
  static constexpr int WM = pick();
  static constexpr bool ok = WM > 0;
  static constexpr int WN = ok ? WAVES / WM : 1;
  static constexpr int WTM = ok ? BM / WM : 32;
  static constexpr int WTN = ok ? BN / WN : 32;
  static constexpr int TM = WTM / 32;
  static constexpr int TN = WTN / 32;
};

// Logical tile of this workgroup.  The dispatcher hands workgroup i to XCD
// i % 8; renumbering makes each XCD own a contiguous run of logical tiles,
// and the grouped raster (group_m tile-rows per group, column-major inside
// a group) makes the tiles that run together on one XCD share A and B
// panels in that XCD's L2.
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int group_m, int& tm, int& tn) {
  const int nwg = (int)gridDim.x;
  int wg = (int)blockIdx.x;
  const int per = nwg >> 3, rem = nwg & 7, xcd = wg & 7;
  wg = xcd * per + (xcd < rem ? xcd : rem) + (wg >> 3);
  const int width = group_m * tiles_n;
  const int group = wg / width;
  const int first_m = group * group_m;
  const int gm = (tiles_m - first_m) < group_m ? (tiles_m - first_m) : group_m;
  const int in_group = wg - group * width;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

// Split-K: the grid holds `parts` copies of the tile grid, copy p computing
// K tiles [p*KTS, (p+1)*KTS) of every output tile (KTS = ceil(KT/parts)).
// Logical workgroup index = p * tiles + tile, so after the XCD renumbering
// each XCD works on neighbouring tiles of one K range.
struct SplitK {
  int parts;          // 1: no split
  float* ws;          // fp32 partial products, [parts][M][N]
};

// One segment of a stream-K workgroup (mi_streamk.hpp): K tiles
// [kt0, kt0 + kts) of output tile (tm, tn).
struct SegK {
  int tm, tn, kt0, kts;
};

// Epilogue row scale of the two-pass fused kernel: output row m is
// multiplied by 1/sqrt(sum_p ssq[p][m] * inv_k + eps), the partial sums of
// squares taken in part order.
struct RowScale {
  const float* ssq;   // [parts][M]
  int parts;
  float inv_k, eps;
};

__device__ __forceinline__ void tile_coords_split(int tiles_m, int tiles_n, int group_m, int parts, int& tm, int& tn,
                                                  int& part) {
  const int nwg = (int)gridDim.x;
  int wg = (int)blockIdx.x;
  const int per = nwg >> 3, rem = nwg & 7, xcd = wg & 7;
  wg = xcd * per + (xcd < rem ? xcd : rem) + (wg >> 3);
  const int tiles = tiles_m * tiles_n;
  part = parts > 1 ? wg / tiles : 0;
  wg -= part * tiles;
  const int width = group_m * tiles_n;
  const int group = wg / width;
  const int first_m = group * group_m;
  const int gm = (tiles_m - first_m) < group_m ? (tiles_m - first_m) : group_m;
  const int in_group = wg - group * width;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

// XOR swizzle of 16-byte chunks inside one K row of an MN-contiguous panel
// (row = one K index, ROWB/16 chunks).  gfx950's LDS has 64 banks of 4 bytes
// (a 256-byte bank window).  One ds_read_b64_tr_b16 reads, per 32 lanes,
// K rows k0..k0+3 x 64 bytes (k0 a multiple of 4), and lanes 32..63 read
// rows k0+8..k0+11.  The swizzle puts the four rows of one read in four
// different 64-byte quarters of the bank window, and rows k and k+8 in
// different 32-byte halves of a quarter, whatever the row pitch:
//   pitch >= 256 B: every row starts at bank 0, XOR the quarter by k&3;
//   pitch == 128 B: rows alternate window halves, XOR the quarter by bit 1;
//   pitch ==  64 B: consecutive rows already sit in consecutive quarters.
template <int ROWB>
__device__ __forceinline__ int mn_swz(int k) {
  const int half = 2 * ((k >> 3) & 1);
  if constexpr (ROWB >= 256) return 4 * (k & 3) ^ half;
  else if constexpr (ROWB == 128) return 4 * ((k >> 1) & 1) ^ half;
  else return half & (ROWB / 16 - 1);
}

// LDS-direct loader of one [BK][W] MN-contiguous panel (W = BM or BN):
// the panel is CH = BK*W*2/1024 chunks of 1 KiB; one wave instruction fills
// one chunk, lane l writing bytes [16l, 16l+16).  The lane fetches the
// global 16 bytes that the swizzle maps to that LDS position.
template <int BK, int W, int WAVES>
struct PanelLoader {
  static constexpr int ROWB = W * 2;
  static constexpr int CH = BK * W * 2 / 1024;
  static constexpr int PER_WAVE = (CH + WAVES - 1) / WAVES;
  static constexpr int LANES_PER_ROW = W / 8;  // 16-byte slots per K row
  static constexpr int ROWS_PER_CH = 1024 / ROWB;
  static constexpr bool EVEN = CH % WAVES == 0;  // every wave issues PER_WAVE loads
  static_assert(W >= 32 && (W & (W - 1)) == 0, "panel width must be a power of two >= 32");
  static_assert(CH >= 1, "panel smaller than one wave load");
  static_assert(ROWB <= 1024, "panel row wider than one wave load");
  uint32_t voff[PER_WAVE];  // per-lane byte offset at K tile 0
  int lds_off[PER_WAVE];    // wave-uniform LDS byte offset of the chunk
  bool active[PER_WAVE];

  __device__ __forceinline__ void init(int wave, int lane, int col0, int ld) {
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int c = wave + j * WAVES;
      active[j] = c < CH;
      const int row = c * ROWS_PER_CH + lane / LANES_PER_ROW;
      const int slot = lane % LANES_PER_ROW;
      const int q = slot ^ mn_swz<ROWB>(row);
      voff[j] = ((uint32_t)row * (uint32_t)ld + (uint32_t)(col0 + 8 * q)) * 2u;
      lds_off[j] = c * 1024;
    }
  }
  // Issue the loads of K tile `kt` into the panel at LDS byte `base`.
  // Completion is tracked by vmcnt only: every reader waits with
  // wait_vmem() (or vm_wait<n>) and a workgroup barrier first.
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t rs, char* smem, int base, uint32_t kstep_bytes,
                                        int kt) const {
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      if (EVEN || active[j]) lds_dma16(rs, smem + base + lds_off[j], voff[j] + (uint32_t)kt * kstep_bytes);
    }
  }
  // Load j (< PER_WAVE) of K tile `kt` alone, for schedules that spread a
  // tile's loads between other instructions.
  __device__ __forceinline__ void issue_one(int j, __amdgpu_buffer_rsrc_t rs, char* smem, int base,
                                            uint32_t kstep_bytes, int kt) const {
    if (EVEN || active[j]) lds_dma16(rs, smem + base + lds_off[j], voff[j] + (uint32_t)kt * kstep_bytes);
  }
  // Load j of the K tile that the descriptor `rs_kt` starts at
  // (make_rsrc_from with the tile's byte offset).
  template <bool NT = false>
  __device__ __forceinline__ void issue_at(int j, __amdgpu_buffer_rsrc_t rs_kt, char* smem, int base) const {
    if (EVEN || active[j]) lds_dma16<NT>(rs_kt, smem + base + lds_off[j], voff[j]);
  }
  // Number of LDS-direct loads one wave issues per K tile.
  static constexpr int LOADS_PER_TILE = PER_WAVE;
};

// Swizzle of the 16-byte K chunks of one row in a K-contiguous panel:
// the 16 lanes of one ds_read_b128 phase (16 rows, same K chunk) hit 16
// different 16-byte bank groups.
template <int BK>
__device__ __forceinline__ int k_swz(int row) {
  constexpr int XD = (128 / BK) > 0 ? (128 / BK) : 1;
  return (row / XD) & (BK / 8 - 1);
}

// LDS-direct loader of a K-contiguous panel: rows row0 .. row0+ROWS-1 of a
// row-major [rows][ld] bf16 matrix, BK columns per K tile, into an LDS panel
// [ROWS][BK] (row stride BK*2 bytes) whose 16-byte chunks are XOR-swizzled
// by k_swz: LDS slot s of row r holds K chunk s ^ k_swz(r).  Lane l of a
// 1 KiB wave load lands at byte 16*l of its chunk, so each lane fetches the
// global chunk that its LDS slot must hold.  The K tile offset rides in the
// buffer descriptor (make_rsrc_from).  In the last K tile, chunks past K
// read zeros (voff_tail).
template <int BK, int ROWS, int WAVES>
struct KPanelLoader {
  static constexpr int ROWB = BK * 2;
  static constexpr int CH = ROWS * ROWB / 1024;
  static constexpr int PER_WAVE = (CH + WAVES - 1) / WAVES;
  static constexpr int LANES_PER_ROW = BK / 8;
  static constexpr int ROWS_PER_CH = 1024 / ROWB;
  static constexpr bool EVEN = CH % WAVES == 0;
  static_assert(BK >= 16 && BK <= 128 && (BK & (BK - 1)) == 0, "K tile of 16..128 columns");
  static_assert(CH >= 1, "panel smaller than one wave load");
  uint32_t voff[PER_WAVE];       // per-lane byte offset inside a K tile
  uint32_t voff_tail[PER_WAVE];  // the same for the last K tile (past K: out of range)
  int lds_off[PER_WAVE];
  bool active[PER_WAVE];

  // oob: any offset at or past the end of the whole buffer.
  __device__ __forceinline__ void init(int wave, int lane, int row0, int ld, int k_last, uint32_t oob) {
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int c = wave + j * WAVES;
      active[j] = c < CH;
      const int row = c * ROWS_PER_CH + lane / LANES_PER_ROW;
      const int q = (lane % LANES_PER_ROW) ^ k_swz<BK>(row);
      voff[j] = ((uint32_t)(row0 + row) * (uint32_t)ld + (uint32_t)(8 * q)) * 2u;
      voff_tail[j] = 8 * q < k_last ? voff[j] : oob;
      lds_off[j] = c * 1024;
    }
  }
  __device__ __forceinline__ void issue_at(int j, __amdgpu_buffer_rsrc_t rs_kt, char* smem, int base,
                                           bool tail) const {
    // One load either way, its offset selected without a branch: a branch
    // per load splits the main loop into blocks, and code the compiler
    // moves between blocks (sinking a chain of VALU work into the last
    // block of the loop body) escapes the scheduling hints of its sub-step.
    if (EVEN || active[j]) lds_dma16(rs_kt, smem + base + lds_off[j], tail ? voff_tail[j] : voff[j]);
  }
  static constexpr int LOADS_PER_TILE = PER_WAVE;
};

// Per-lane LDS byte offsets of the MFMA operand fragments read with
// ds_read_b64_tr_b16 from an MN-contiguous [BK][W] panel.  For fragment t
// (32 columns starting at w0 + 32t) and K sub-step kk, half h, the address
// is panel + (kk*16 + 4h) * ROWB + off[t].
template <int W, int T>
struct TrFrag {
  static constexpr int ROWB = W * 2;
  int off[T];
  __device__ __forceinline__ void init(int lane, int w0) {
    const int g = lane >> 4, i = lane & 15, r = i >> 2, c = i & 3;
    const int krow = 8 * (g >> 1) + r;  // K row inside the 16-row sub-step
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int col = w0 + 32 * t + 16 * (g & 1) + 4 * c;
      off[t] = krow * ROWB + 16 * ((col >> 3) ^ mn_swz<ROWB>(krow)) + (col & 7) * 2;
    }
  }
};

__device__ __forceinline__ bf16x8_t read_tr_frag(const char* smem, int addr0, int addr1) {
  const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((MI_LDS s16x4_t*)(smem + addr0));
  const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((MI_LDS s16x4_t*)(smem + addr1));
  typedef short s16x8_t __attribute__((ext_vector_type(8)));
  const s16x8_t v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ float bf16lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xFFFF0000u); }

// Epilogue: each wave stages one 32-row slice of its accumulator block as
// bf16 in LDS (row stride WTN*2+16 bytes), reads it back as 16-byte row
// chunks and stores whole rows.  `scale[mt]` multiplies every value of the
// lane's output row in slice mt (1/rms for the fused kernel, 1 otherwise).
template <int TM, int TN, int WAVES>
__device__ __forceinline__ void store_tile(f32x16_t (&acc)[TM][TN], const float (&scale)[TM], char* smem, int wave,
                                           int lane, uint16_t* __restrict__ out, int M, int N, int row0, int col0) {
  constexpr int WTN = TN * 32;
  constexpr int SROW = WTN * 2 + 16;
  constexpr int CPR = WTN / 8;       // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;      // rows per read instruction
  char* ep = smem + wave * (32 * SROW);
#pragma unroll
  for (int mt = 0; mt < TM; ++mt) {
    const float s = scale[mt];
#pragma unroll
    for (int nt = 0; nt < TN; ++nt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int nl = nt * 32 + 8 * j + 4 * (lane >> 5);
        const int ml = lane & 31;
        u32x2_t v;
        v.x = pack_bf16x2(acc[mt][nt][4 * j + 0] * s, acc[mt][nt][4 * j + 1] * s);
        v.y = pack_bf16x2(acc[mt][nt][4 * j + 2] * s, acc[mt][nt][4 * j + 3] * s);
        *(MI_LDS u32x2_t*)((MI_LDS char*)ep + ml * SROW + nl * 2) = v;
      }
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 32 / RPI; ++it) {
      const int rl = it * RPI + lane / CPR;
      const int cl = lane % CPR;
      const u32x4_t v = *(MI_LDS u32x4_t*)((MI_LDS char*)ep + rl * SROW + cl * 16);
      const int m = row0 + mt * 32 + rl;
      const int n = col0 + cl * 8;
      if (m < M && n < N) *(u32x4_t*)(out + (size_t)m * N + n) = v;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// out[M,N] = lhsT[K,M]^T . rhs[K,N]
// ---------------------------------------------------------------------------
template <int BM, int BN, int BK, int WAVES, int STAGES>
struct MatmulCfg {
  using G = WaveGrid<BM, BN, WAVES>;
  static constexpr int A_BYTES = BK * BM * 2;
  static constexpr int B_BYTES = BK * BN * 2;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int EPI_BYTES = WAVES * 32 * (G::WTN * 2 + 16);
  static constexpr int MAIN_BYTES = STAGES * STAGE_BYTES;
  static constexpr int LDS_BYTES = MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES;
};

template <int BM, int BN, int BK, int WAVES, int STAGES>
__global__ __launch_bounds__(WAVES * 64) void mm_lhsT_rhs_bf16_kernel(const uint16_t* __restrict__ lhsT,
                                                                     const uint16_t* __restrict__ rhs,
                                                                     uint16_t* __restrict__ out, int M, int N,
                                                                     int K, int group_m) {
  using C = MatmulCfg<BM, BN, BK, WAVES, STAGES>;
  using G = typename C::G;
  static_assert(legal_mm_plain(BM, BN, BK, WAVES, STAGES).code == MI_OK, "illegal tile config (mi_legal.hpp)");
  static_assert(C::LDS_BYTES == lds_mm_plain(BM, BN, BK, WAVES, STAGES), "host LDS budget out of step");
  static_assert(G::ok, "illegal wave grid");
  static_assert(BK % 16 == 0, "BK must be a multiple of 16");
  constexpr int TM = G::TM, TN = G::TN;
  __shared__ __attribute__((aligned(1024))) char smem[C::LDS_BYTES];

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

  PanelLoader<BK, BM, WAVES> la;
  PanelLoader<BK, BN, WAVES> lb;
  la.init(wave, lane, m0, M);
  lb.init(wave, lane, n0, N);
  const uint32_t kstep_a = (uint32_t)BK * (uint32_t)M * 2u;
  const uint32_t kstep_b = (uint32_t)BK * (uint32_t)N * 2u;

  TrFrag<BM, TM> fa;
  TrFrag<BN, TN> fb;
  fa.init(lane, wm0);
  fb.init(lane, wn0);

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16_t{};

  auto compute = [&](int stage) {
    const int abase = stage * C::STAGE_BYTES;
    const int bbase = abase + C::A_BYTES;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      bf16x8_t af[TM], bf[TN];
#pragma unroll
      for (int t = 0; t < TM; ++t)
        af[t] = read_tr_frag(smem, abase + (kk * 16) * (BM * 2) + fa.off[t],
                             abase + (kk * 16 + 4) * (BM * 2) + fa.off[t]);
#pragma unroll
      for (int t = 0; t < TN; ++t)
        bf[t] = read_tr_frag(smem, bbase + (kk * 16) * (BN * 2) + fb.off[t],
                             bbase + (kk * 16 + 4) * (BN * 2) + fb.off[t]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[j], af[i], acc[i][j], 0, 0, 0);
    }
  };

  const int KT = (K + BK - 1) / BK;
  if constexpr (STAGES == 1) {
    for (int t = 0; t < KT; ++t) {
      la.issue(ra, smem, 0, kstep_a, t);
      lb.issue(rb, smem, C::A_BYTES, kstep_b, t);
      wait_vmem();
      __syncthreads();
      compute(0);
      __syncthreads();
    }
  } else {
    la.issue(ra, smem, 0, kstep_a, 0);
    lb.issue(rb, smem, C::A_BYTES, kstep_b, 0);
    wait_vmem();
    __syncthreads();
    for (int t = 0; t < KT; ++t) {
      const int cur = t & 1;
      if (t + 1 < KT) {
        const int nb = (cur ^ 1) * C::STAGE_BYTES;
        la.issue(ra, smem, nb, kstep_a, t + 1);
        lb.issue(rb, smem, nb + C::A_BYTES, kstep_b, t + 1);
      }
      compute(cur);
      wait_vmem();
      __syncthreads();
    }
  }

  float one[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) one[i] = 1.0f;
  store_tile<TM, TN, WAVES>(acc, one, smem, wave, lane, out, M, N, m0 + wm0, n0 + wn0);
}

// Scheduling hint for one MFMA K sub-step: NM MFMAs with ND LDS reads spread
// between them (a wave issues in order, so an MFMA stuck behind a run of LDS
// reads -- or reads stuck behind a run of MFMAs -- idles the matrix core).
// Masks: 0x008 MFMA, 0x100 DS read; the trailing sched_barrier closes the
// region so the next sub-step gets its own pattern.
// General form: per MFMA also a share of NV VALU instructions and NW LDS
// writes (masks 0x002 VALU, 0x200 DS write).
template <int NM, int NR, int NV, int NW, int M = 0>
__device__ __forceinline__ void interleave_mfma_mix() {
  if constexpr (M < NM) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    constexpr int r = NR / NM + (M < NR % NM ? 1 : 0);
    constexpr int v = NV / NM + (M < NV % NM ? 1 : 0);
    constexpr int w = NW / NM + (M < NW % NM ? 1 : 0);
    if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);
    if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(0x002, v, 0);
    if constexpr (w > 0) __builtin_amdgcn_sched_group_barrier(0x200, w, 0);
    interleave_mfma_mix<NM, NR, NV, NW, M + 1>();
  } else {
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int NM, int ND, int M = 0>
__device__ __forceinline__ void interleave_mfma_ds() {
  if constexpr (M < NM) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    constexpr int n = ND / NM + (M < ND % NM ? 1 : 0);
    if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x100, n, 0);
    interleave_mfma_ds<NM, ND, M + 1>();
  } else {
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ---------------------------------------------------------------------------
// out[M,N] = lhsT[K,M]^T . rhs[K,N], software-pipelined (matmul variant 1).
//
// STAGES LDS buffers hold K tiles t .. t+STAGES-1.  Inside a K tile the
// MFMA operands of sub-step kk+1 are read from LDS while the MFMAs of kk
// run (two register sets).  At the last sub-step of tile t each wave waits
// for its own loads of tile t+1, the workgroup meets at one barrier (after
// which tile t+1 is visible and nobody reads tile t's buffer any more), the
// first operands of tile t+1 are read, and the loads of tile t+STAGES are
// issued into the buffer tile t just vacated -- so one barrier per K tile,
// and global loads run STAGES-1 tiles ahead of the MFMAs.
// ---------------------------------------------------------------------------
template <int BM, int BN, int BK, int WAVES, int STAGES>
struct PipeCfg {
  using G = WaveGrid<BM, BN, WAVES>;
  static constexpr int A_BYTES = BK * BM * 2;
  static constexpr int B_BYTES = BK * BN * 2;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int EPI_BYTES = WAVES * 32 * (G::WTN * 2 + 16);
  static constexpr int MAIN_BYTES = STAGES * STAGE_BYTES;
  static constexpr int LDS_BYTES = MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES;
};

// The pipelined body, for two layouts of the A operand: AK = false takes
// lhsT[K,M] (M contiguous; MN-swizzled panel, transposing operand reads),
// AK = true takes lhs[M,K] (K contiguous; K-swizzled panel, one
// ds_read_b128 per operand fragment, no transpose).
// Split-K epilogue: part p stores its fp32 accumulators to ws[p][M][N]
// straight from registers (lane l holds row l%32 of each 32x32 fragment,
// four consecutive columns per dword quad; N % 8 == 0, so a quad is in
// bounds whenever its first column is).  A second kernel sums the parts.
template <int TM, int TN>
__device__ __forceinline__ void store_partial(const f32x16_t (&acc)[TM][TN], float* __restrict__ ws, int lane,
                                              int M, int N, int row0, int col0) {
#pragma unroll
  for (int mt = 0; mt < TM; ++mt) {
    const int m = row0 + mt * 32 + (lane & 31);
#pragma unroll
    for (int nt = 0; nt < TN; ++nt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = col0 + nt * 32 + 8 * j + 4 * (lane >> 5);
        if (m < M && n < N) {
          const f32x4_t v = {acc[mt][nt][4 * j], acc[mt][nt][4 * j + 1], acc[mt][nt][4 * j + 2],
                             acc[mt][nt][4 * j + 3]};
          *(f32x4_t*)(ws + (size_t)m * N + n) = v;
        }
      }
  }
}

// Epilogue of the K-split-over-waves core: every wave holds the whole
// block's fp32 sums over its own K sub-steps.  One 32-row slice at a time,
// each wave writes its slice to its LDS slot (32 rows, stride BN*4+16
// bytes: the 16 lanes of a ds_write_b128 phase hit 16 different bank
// quads), then every thread takes 8-column items of the slice, sums the
// waves' values in wave order (so the result does not depend on timing),
// and stores 8 bf16 to out -- or, split-K, the 8 fp32 to its part's ws.
template <int BN, int WAVES, int TM, int TN, bool SPLIT>
__device__ __forceinline__ void kw_reduce_store(const f32x16_t (&acc)[TM][TN], char* smem, int wave, int lane,
                                                int tid, uint16_t* __restrict__ out, float* __restrict__ ws, int M,
                                                int N, int m0, int n0) {
  constexpr int RSB = BN * 4 + 16, SLOT = 32 * RSB, NTH = WAVES * 64, ITEMS = 32 * (BN / 8);
  MI_LDS char* lds = (MI_LDS char*)smem;
  const int r = lane & 31;
#pragma unroll
  for (int mt = 0; mt < TM; ++mt) {
#pragma unroll
    for (int nt = 0; nt < TN; ++nt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = nt * 32 + 8 * j + 4 * (lane >> 5);
        const f32x4_t v = {acc[mt][nt][4 * j], acc[mt][nt][4 * j + 1], acc[mt][nt][4 * j + 2],
                           acc[mt][nt][4 * j + 3]};
        *(MI_LDS f32x4_t*)(lds + wave * SLOT + r * RSB + c * 4) = v;
      }
    __syncthreads();
    for (int it = tid; it < ITEMS; it += NTH) {
      const int rr = it / (BN / 8), c8 = (it % (BN / 8)) * 8;
      const int off = rr * RSB + c8 * 4;
      f32x4_t lo = *(MI_LDS f32x4_t*)(lds + off), hi = *(MI_LDS f32x4_t*)(lds + off + 16);
#pragma unroll
      for (int w = 1; w < WAVES; ++w) {
        lo += *(MI_LDS f32x4_t*)(lds + w * SLOT + off);
        hi += *(MI_LDS f32x4_t*)(lds + w * SLOT + off + 16);
      }
      const int m = m0 + mt * 32 + rr, n = n0 + c8;
      if (m < M && n < N) {
        if constexpr (SPLIT) {
          *(f32x4_t*)(ws + (size_t)m * N + n) = lo;
          *(f32x4_t*)(ws + (size_t)m * N + n + 4) = hi;
        } else {
          u32x4_t o;
          o.x = pack_bf16x2(lo[0], lo[1]);
          o.y = pack_bf16x2(lo[2], lo[3]);
          o.z = pack_bf16x2(hi[0], hi[1]);
          o.w = pack_bf16x2(hi[2], hi[3]);
          *(u32x4_t*)(out + (size_t)m * N + n) = o;
        }
      }
    }
    __syncthreads();
  }
}

// out[i] = bf16(sum over p = 0 .. parts-1 of ws[p][i]), summed in part order
// (so the result does not depend on the order the parts ran in); 8
// elements per thread (n = M*N, a multiple of 8).  A template so that every
// translation unit may instantiate it.
template <int UNUSED = 0>
__global__ __launch_bounds__(256) void splitk_sum_kernel(const float* __restrict__ ws, uint16_t* __restrict__ out,
                                                         size_t n, int parts) {
  const size_t stride = (size_t)gridDim.x * 256 * 8;
  for (size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 8; i < n; i += stride) {
    f32x4_t lo = *(const f32x4_t*)(ws + i), hi = *(const f32x4_t*)(ws + i + 4);
    for (int p = 1; p < parts; ++p) {
      lo += *(const f32x4_t*)(ws + (size_t)p * n + i);
      hi += *(const f32x4_t*)(ws + (size_t)p * n + i + 4);
    }
    u32x4_t o;
    o.x = pack_bf16x2(lo[0], lo[1]);
    o.y = pack_bf16x2(lo[2], lo[3]);
    o.z = pack_bf16x2(hi[0], hi[1]);
    o.w = pack_bf16x2(hi[2], hi[3]);
    *(u32x4_t*)(out + i) = o;
  }
}

struct NoEpi {};

// SK (stream-K): the tile and its K range come from `seg`, and instead of an
// epilogue of its own the body hands its accumulators to
// epi(acc, row0, col0) (row0, col0: this wave's first output row and
// column), after the main loop's final barrier.
// SQ (the fused kernel without gamma, rmsnorm_matmul variant 14): the
// K-contiguous A operand is x itself, so every x value of the block passes
// through the A fragments the MFMAs consume, each sub-step once.  Lane l
// holds row l%32 of each 32-row fragment and K chunk 2*kk + l/32 of
// sub-step kk; it sums the squares of its chunks' 8 values with bf16 dot2
// (v_dot2c_f32_bf16: exact bf16 products, fp32 sums), four per fragment,
// in K order.  The waves that share rows (one wave row of the grid) take
// the sub-steps in turns, the two half-waves' sums are added, the wave
// row's parts are added through LDS in a fixed order, and the epilogue
// scales output row m by 1/sqrt(ssq[m] * inv_k + eps) (rsc.inv_k,
// rsc.eps).  K chunks past K read zeros and add nothing.
template <int BM, int BN, int BK, int WAVES, int STAGES, bool AK, bool NTB = false, bool SPLIT = false,
          bool RS = false, bool KW = false, bool SK = false, class Epi = NoEpi, bool SQ = false>
__device__ __forceinline__ void mm_pipe_body(const uint16_t* __restrict__ a, const uint16_t* __restrict__ rhs,
                                             uint16_t* __restrict__ out, int M, int N, int K, int group_m,
                                             char* smem, const SplitK sk = SplitK{1, nullptr},
                                             const RowScale rsc = RowScale{nullptr, 0, 0.0f, 0.0f},
                                             const SegK seg = SegK{0, 0, 0, 0}, Epi&& epi = Epi{}) {
  using C = PipeCfg<BM, BN, BK, WAVES, STAGES>;
  using G = typename C::G;
  static_assert(KW ? legal_mm_kw(BM, BN, BK, WAVES, STAGES).code == MI_OK
                   : legal_mm_pipe(BM, BN, BK, WAVES, STAGES, AK).code == MI_OK,
                "illegal tile config (mi_legal.hpp)");
  static_assert(C::LDS_BYTES == lds_mm_pipe(BM, BN, BK, WAVES, STAGES), "host LDS budget out of step");
  static_assert(KW || G::ok, "illegal wave grid");
  static_assert(!KW || (!AK && !RS), "K split over the waves: lhsT operand, no row scale");
  static_assert(!SK || (!KW && !RS && !SPLIT), "stream-K: the plain wave-grid core");
  static_assert(!SQ || (AK && !KW && !RS && !SPLIT && !SK), "row sums of squares: the K-contiguous unsplit core");
  static_assert(!SQ || G::WN * BM * 4 <= C::LDS_BYTES, "row sums of squares exchanged through LDS");
  static_assert(BK % 32 == 0, "BK must be a multiple of 32 (even number of MFMA K steps)");
  static_assert(STAGES >= 2 && STAGES <= 4, "2..4 LDS stages");
  // KW: every wave covers the whole block (TM x TN MFMA tiles) over its own
  // KSW consecutive 16-deep sub-steps of each K tile; otherwise each wave
  // covers its wave-grid block over all KS sub-steps.
  constexpr int TM = KW ? BM / 32 : G::TM, TN = KW ? BN / 32 : G::TN, KS = BK / 16;
  constexpr int KSW = KW ? KS / WAVES : KS;
  using LA = std::conditional_t<AK, KPanelLoader<BK, BM, WAVES>, PanelLoader<BK, BM, WAVES>>;
  using LB = PanelLoader<BK, BN, WAVES>;
  // Loads of one K tile by this wave; vm_wait<n> with n > 0 needs every wave
  // to issue the same number.
  constexpr int LPT = LA::LOADS_PER_TILE + LB::LOADS_PER_TILE;
  static_assert(STAGES == 2 || (LA::EVEN && LB::EVEN), "deeper pipelines need an even panel split");

  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tmi, tni, part = 0;
  if constexpr (SK) {
    tmi = seg.tm;
    tni = seg.tn;
  } else if constexpr (SPLIT) {
    tile_coords_split(tiles_m, tiles_n, group_m, sk.parts, tmi, tni, part);
  } else {
    tile_coords(tiles_m, tiles_n, group_m, tmi, tni);
  }
  const int m0 = tmi * BM, n0 = tni * BN;
  const int wm0 = KW ? 0 : (wave / G::WN) * G::WTM;
  const int wn0 = KW ? 0 : (wave % G::WN) * G::WTN;
  const int lda = K;  // row stride of the K-contiguous lhs: the whole K
  int k0 = 0;
  if constexpr (SPLIT) {
    // Split-K part `part`: K indices [k0, k0 + K) of both operands (the host
    // guarantees every part a non-empty range): rows of lhsT and rhs,
    // columns of a K-contiguous lhs (whose rows keep their stride).
    const int kts = ((K + BK - 1) / BK + sk.parts - 1) / sk.parts;
    k0 = part * kts * BK;
    a += AK ? (size_t)k0 : (size_t)k0 * (size_t)M;
    rhs += (size_t)k0 * (size_t)N;
    K = K - k0 < kts * BK ? K - k0 : kts * BK;
  } else if constexpr (SK) {
    // The segment's K tiles (the host grid keeps every segment non-empty).
    k0 = seg.kt0 * BK;
    a += AK ? (size_t)k0 : (size_t)k0 * (size_t)M;
    rhs += (size_t)k0 * (size_t)N;
    K = K - k0 < seg.kts * BK ? K - k0 : seg.kts * BK;
  }

  // Bytes from the (part's) base to the end of the A buffer.
  const uint32_t a_bytes = AK ? ((uint32_t)M * (uint32_t)lda - (uint32_t)k0) * 2u : (uint32_t)K * (uint32_t)M * 2u;
  const uint32_t b_bytes = (uint32_t)K * (uint32_t)N * 2u;
  const int KT = (K + BK - 1) / BK;
  LA la;
  LB lb;
  if constexpr (AK) la.init(wave, lane, m0, lda, K - (KT - 1) * BK, a_bytes);
  else la.init(wave, lane, m0, M);
  lb.init(wave, lane, n0, N);
  const uint32_t kstep_a = AK ? (uint32_t)BK * 2u : (uint32_t)BK * (uint32_t)M * 2u;
  const uint32_t kstep_b = (uint32_t)BK * (uint32_t)N * 2u;
  TrFrag<BM, TM> fa;
  TrFrag<BN, TN> fb;
  if constexpr (!AK) fa.init(lane, wm0);
  fb.init(lane, wn0);
  if constexpr (KW) {
    // This wave's sub-steps start KSW * wave rows into each K tile (the
    // operand swizzle repeats every 16 rows, so a row offset is enough).
    const int kb = wave * KSW * 16;
#pragma unroll
    for (int t = 0; t < TM; ++t) fa.off[t] += kb * (BM * 2);
#pragma unroll
    for (int t = 0; t < TN; ++t) fb.off[t] += kb * (BN * 2);
  }
  // K-contiguous A operand: lane l reads row l%32 of the fragment, K chunk
  // 2*kk + l/32 of the sub-step, at its k_swz slot (the same for every
  // 32-row fragment of the wave).
  const int arow = (wm0 + (lane & 31)) * (BK * 2);
  int akoff[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) akoff[kk] = 16 * ((2 * kk + (lane >> 5)) ^ k_swz<BK>(wm0 + (lane & 31)));

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16_t{};

  bf16x8_t af[2][TM], bf[2][TN];
  // Operand f of a K sub-step, in the order the MFMAs (row-major over
  // (i, j)) consume them: A0, B0 .. B(TN-1), A1 .. A(TM-1).
  constexpr int NF = TM + TN;
  auto read_frag = [&](int stage, int kk, int buf, int f) {
    const int abase = stage * C::STAGE_BYTES;
    const int bbase = abase + C::A_BYTES;
    if (f == 0 || f > TN) {
      const int t = f == 0 ? 0 : f - TN;
      if constexpr (AK)
        af[buf][t] = __builtin_bit_cast(
            bf16x8_t, *(MI_LDS u32x4_t*)((MI_LDS char*)smem + abase + arow + t * 32 * (BK * 2) + akoff[kk]));
      else
        af[buf][t] = read_tr_frag(smem, abase + (kk * 16) * (BM * 2) + fa.off[t],
                                  abase + (kk * 16 + 4) * (BM * 2) + fa.off[t]);
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
  float sq[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) sq[i] = 0.0f;
  // SQ: the G::WN waves that share rows take turns, sub-step kk going to
  // the wave in column kk % WN, and add their sums at the end.
  const int wcol = KW ? 0 : wave % G::WN;
  auto mfmas = [&](int buf, int kk, auto wc_c) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[buf][j], af[buf][i], acc[i][j], 0, 0, 0);
    if constexpr (SQ) {
      if (G::WN > 1 && kk % G::WN != decltype(wc_c)::value) return;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        // Pair d of the fragment as a shuffle with constant indices.  (A
        // bf16x2 bit-cast from dword d of the fragment viewed as u32x4 is
        // compiled as dword 0 for every d by this hipcc; the shuffle and an
        // element-wise build are not.)
        static_for<4>([&](auto d_c) __attribute__((always_inline)) {
          constexpr int d = decltype(d_c)::value;
          const bf16x2_t v = __builtin_shufflevector(af[buf][i], af[buf][i], 2 * d, 2 * d + 1);
          sq[i] = __builtin_amdgcn_fdot2_f32_bf16(v, v, sq[i], false);
        });
      }
    }
  };
  // Scheduling of one sub-step: its MFMAs with the LDS reads (and, SQ, the
  // dot2 VALU work) spread between them.
  auto sched = [&]() __attribute__((always_inline)) {
    if constexpr (SQ) interleave_mfma_mix<TM * TN, 2 * NF, 4 * TM, 0>();
    else interleave_mfma_ds<TM * TN, 2 * NF>();
  };
  // Load q (< LPT) of K tile kt into `stage`: the A loads, then the B loads.
  auto issue_one = [&](int q, int kt, int stage) {
    if (q < LA::LOADS_PER_TILE) {
      if constexpr (AK)
        la.issue_at(q, make_rsrc_from(a, a_bytes, (uint32_t)kt * kstep_a), smem, stage * C::STAGE_BYTES,
                    kt == KT - 1);
      else
        la.issue_at(q, make_rsrc_from(a, a_bytes, (uint32_t)kt * kstep_a), smem, stage * C::STAGE_BYTES);
    } else
      lb.template issue_at<NTB>(q - LA::LOADS_PER_TILE, make_rsrc_from(rhs, b_bytes, (uint32_t)kt * kstep_b), smem,
                  stage * C::STAGE_BYTES + C::A_BYTES);
  };

  // Tiles past the end are clamped to the last one: the loads stay in
  // bounds, every tile issues the same number of loads (so vmcnt counts are
  // static) and the loop needs no branch.  Re-reading the last tile into a
  // buffer that is never read again costs STAGES-1 tiles of bandwidth.
  auto clamp = [&](int kt) { return kt < KT ? kt : KT - 1; };

  // Row scale (two-pass fused kernel): 1/sqrt(sum_p ssq[p][m] * inv_k + eps)
  // for each row m of the block, p in order, into LDS past the panels
  // (rs_lds, BM floats; the caller allocates them).  Each thread takes
  // rows tid, tid + NT, ...; the first RSB partial sums of its rows are
  // loaded before the prologue's panel loads, so they arrive with the first
  // tiles, and summed after the prologue's wait.
  constexpr int NTH = WAVES * 64, RSB = 8, RPT = RS && !SPLIT ? (BM + NTH - 1) / NTH : 1;
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
  if constexpr (RS && !SPLIT) load_parts(0);

  // Prologue: tiles 0 .. STAGES-1 in flight, wait for tile 0.
#pragma unroll
  for (int s = 0; s < STAGES; ++s)
#pragma unroll
    for (int q = 0; q < LPT; ++q) issue_one(q, clamp(s), s);
  vm_wait<(STAGES - 1) * LPT>();
  __syncthreads();
  if constexpr (RS && !SPLIT) {
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
  read_frags(0, 0, 0);

  // Steady state: every tile but the last.  At the last sub-step the wave
  // waits for tile t+1 (tiles t+2 .. t+STAGES-1 may still fly), meets the
  // workgroup, then reads tile t+1's first operands and issues tile
  // t+STAGES into the buffer tile t vacated, both between the MFMAs of the
  // sub-step.
  // Tile t sits in stage t % STAGES; the loop is unrolled STAGES times so
  // that the stage is a compile-time constant in every body.
  // Operand buffer of sub-step kk of the tile held in `stage`: sub-steps
  // alternate between the two buffers across tile boundaries, so the next
  // tile's first operands never overwrite the ones the last MFMAs of this
  // tile still read.  With an even sub-step count per tile this is kk & 1;
  // with an odd one (KW with one sub-step per wave) it needs STAGES * KSW
  // even, so the ring's wrap keeps the alternation.
  static_assert((STAGES * KSW) % 2 == 0, "operand buffers need an even sub-step count per ring turn");
  auto bufof = [](int stage, int kk) { return (stage * KSW + kk) & 1; };
  // wc_c: the wave column as a compile-time constant (SQ, below), so that
  // each sub-step's share of the sums of squares is decided at compile time.
  auto tile = [&](int t, auto cur_c, auto wc_c) __attribute__((always_inline)) {
    constexpr int cur = decltype(cur_c)::value;
    constexpr int nxt = cur + 1 == STAGES ? 0 : cur + 1;
#pragma unroll
    for (int kk = 0; kk + 1 < KSW; ++kk) {
      read_frags(cur, kk + 1, bufof(cur, kk + 1));
      mfmas(bufof(cur, kk), kk, wc_c);
      sched();
    }
    vm_wait<(STAGES - 2) * LPT>();
    __syncthreads();
    const int kt_new = clamp(t + STAGES);
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      read_frag(nxt, 0, bufof(nxt, 0), f);
#pragma unroll
      for (int q = f * LPT / NF; q < (f + 1) * LPT / NF; ++q) issue_one(q, kt_new, cur);
    }
    mfmas(bufof(cur, KSW - 1), KSW - 1, wc_c);
    sched();
  };
  // Last tile: no further loads.
  auto last_tile = [&](int cur, auto wc_c) __attribute__((always_inline)) {
#pragma unroll
    for (int kk = 0; kk < KSW; ++kk) {
      if (kk + 1 < KSW) read_frags(cur, kk + 1, (kk + 1) & 1);
      mfmas(kk & 1, kk, wc_c);
      sched();
    }
  };
  auto k_loop = [&](auto wc_c) __attribute__((always_inline)) {
    int t0 = 0;
    for (; t0 + STAGES < KT; t0 += STAGES)
      static_for<STAGES>([&](auto s_c) __attribute__((always_inline)) { tile(t0 + s_c(), s_c, wc_c); });
    if constexpr (KSW % 2 == 1) {
      // The buffer parity depends on the stage, which is a compile-time
      // constant only inside tile(): the last tile runs through tile() too.
      // Its extra barrier reads the next stage (a clamped re-read of the
      // last K tile) into the unused buffer and issues one more clamped
      // load group, which the drain below retires.
      static_while<STAGES>([&](auto s_c) __attribute__((always_inline)) {
        if (t0 + s_c() >= KT) return false;
        tile(t0 + s_c(), s_c, wc_c);
        return true;
      });
    } else {
      static_while<STAGES>([&](auto s_c) __attribute__((always_inline)) {
        if (t0 + s_c() + 1 >= KT) return false;
        tile(t0 + s_c(), s_c, wc_c);
        return true;
      });
      last_tile((KT - 1) % STAGES, wc_c);
    }
  };
  if constexpr (SQ && G::WN > 1) {
    // One copy of the K loop per wave column; each wave runs its own.
    static_for<G::WN>([&](auto wc_c) __attribute__((always_inline)) {
      if (wcol == decltype(wc_c)::value) k_loop(wc_c);
    });
  } else {
    k_loop(std::integral_constant<int, 0>{});
  }
  wait_vmem();
  __syncthreads();  // the epilogue reuses the panel buffers

  if constexpr (KW) {
    kw_reduce_store<BN, WAVES, TM, TN, SPLIT>(acc, smem, wave, lane, tid, out,
                                             SPLIT ? sk.ws + (size_t)part * (size_t)M * (size_t)N : nullptr, M, N,
                                             m0, n0);
    return;
  }
  if constexpr (SPLIT) {
    store_partial<TM, TN>(acc, sk.ws + (size_t)part * (size_t)M * (size_t)N, lane, M, N, m0 + wm0, n0 + wn0);
    return;
  }
  if constexpr (SK) {
    epi(acc, m0 + wm0, n0 + wn0);
    return;
  }
  float scale[TM];
  if constexpr (SQ) {
    // Lanes l and l^32 hold the two K halves of one row (a + b == b + a,
    // so both get the same bits); the WN waves of a wave row then add
    // their sums through LDS [WN][BM], in wave-column order.
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

// NTB: rhs loaded with the non-temporal cache policy (matmul variant 3, for
// shapes where rhs is streamed once: skinny M).  SPLIT: K split over
// `parts` workgroups per output tile, each writing fp32 partial products to
// ws (splitk_sum_kernel then forms out); a separate instance, so that the
// unsplit kernel is unchanged.
template <int BM, int BN, int BK, int WAVES, int STAGES, bool NTB = false, bool SPLIT = false>
__global__ __launch_bounds__(WAVES * 64) void mm_lhsT_rhs_bf16_pipe_kernel(const uint16_t* __restrict__ lhsT,
                                                                          const uint16_t* __restrict__ rhs,
                                                                          uint16_t* __restrict__ out, int M, int N,
                                                                          int K, int group_m, int parts,
                                                                          float* __restrict__ ws) {
  __shared__ __attribute__((aligned(1024))) char smem[PipeCfg<BM, BN, BK, WAVES, STAGES>::LDS_BYTES];
  mm_pipe_body<BM, BN, BK, WAVES, STAGES, false, NTB, SPLIT>(lhsT, rhs, out, M, N, K, group_m, smem,
                                                             SplitK{parts, ws});
}

// ---------------------------------------------------------------------------
// Stream-K lhsT.rhs (matmul variants 5 and 6): the pipelined core over a
// grid of one workgroup per CU, each taking an equal share of all tiles' K
// tiles (mi_streamk.hpp has the split and the combine protocol).
// ---------------------------------------------------------------------------

// Cache policy of the buffer intrinsics on gfx950: SC0 = 1, NT = 2, SC1 = 16.
// sc0 sc1 is system scope: a store is written through to memory before it
// is acknowledged, and a load misses every cache on the way, so a partial
// sum stored by one workgroup and loaded by another after the tile
// counter's atomic shows the stored values whichever CU or XCD each ran on.
constexpr int kCpolSystem = 1 | 16;

// Workspace of a stream-K launch: the tile counters at its start
// (kSkCounterBytes), then `grid` later slots (one per workgroup, for its one
// segment that is not a tile's p_0) and `tiles` first slots (p_0 of each
// tile), BM*BN fp32 each.
struct StreamKWs {
  int* ctr;
  float* later;
  float* first;
};

// A slot holds one workgroup's accumulators in its own register order:
// wave v, fragment (i, j), quad q of the 16 fp32 values, lane l at byte
// ((((v * TM + i) * TN + j) * 4 + q) * 64 + l) * 16, so each wave store is
// one contiguous 1 KiB.
template <int TM, int TN>
__device__ __forceinline__ uint32_t sk_slot_off(int wave, int i, int j, int q, int lane) {
  return (uint32_t)((((wave * TM + i) * TN + j) * 4 + q) * 64 + lane) * 16u;
}

template <int BM, int BN, int TM, int TN>
__device__ __forceinline__ void sk_store_slot(const f32x16_t (&acc)[TM][TN], float* slot, int wave, int lane) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(slot, (uint32_t)BM * BN * 4u);
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4_t v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r,
                                               sk_slot_off<TM, TN>(wave, i, j, q, lane), 0, kCpolSystem);
      }
}

__device__ __forceinline__ f32x4_t sk_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCpolSystem));
}

// s[i][j] (+)= slot.
template <int TM, int TN, bool ADD>
__device__ __forceinline__ void sk_take_slot(f32x16_t (&s)[TM][TN], const float* slot, size_t slot_floats, int wave,
                                             int lane) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(slot, (uint32_t)slot_floats * 4u);
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4_t v = sk_load4(r, sk_slot_off<TM, TN>(wave, i, j, q, lane));
#pragma unroll
        for (int x = 0; x < 4; ++x) s[i][j][4 * q + x] = ADD ? s[i][j][4 * q + x] + v[x] : v[x];
      }
}

// The combine of tile t: acc = ((p_0 + p_1) + ...) + p_n, where p_0 is in
// the tile's first slot and p_e (e = 1 .. n) in later slot `base + e`.  The
// checker (last_in_regs) holds p_n in acc and the storers' parts come from
// their slots; a storer that combines takes every part from the slots, its
// own included (stored, and drained, before its counter update).  Both add
// in the same order, so the bits are the same.  One 16-byte quad at a time:
// no second copy of the accumulators.
template <int BM, int BN, int TM, int TN>
__device__ __forceinline__ void sk_combine(f32x16_t (&acc)[TM][TN], const StreamKWs& ws, int t, int base, int n,
                                           bool last_in_regs, int wave, int lane) {
  const size_t slot = (size_t)BM * BN;
  const __amdgpu_buffer_rsrc_t r0 = make_rsrc(ws.first + (size_t)t * slot, (uint32_t)slot * 4u);
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t off = sk_slot_off<TM, TN>(wave, i, j, q, lane);
        f32x4_t v = sk_load4(r0, off);
        for (int e = 1; e < n; ++e)
          v += sk_load4(make_rsrc(ws.later + (size_t)(base + e) * slot, (uint32_t)slot * 4u), off);
        f32x4_t last;
        if (last_in_regs) {
          last = f32x4_t{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        } else {
          last = sk_load4(make_rsrc(ws.later + (size_t)(base + n) * slot, (uint32_t)slot * 4u), off);
        }
        v = v + last;
#pragma unroll
        for (int x = 0; x < 4; ++x) acc[i][j][4 * q + x] = v[x];
      }
}

// s_waitcnt vmcnt(0) that the compiler may not move memory operations across.
__device__ __forceinline__ void sk_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// The protocol of mi_streamk.hpp for one part of tile t split into n + 1
// parts: `mine` is the part's slot (the tile's first slot for p_0, a later
// slot otherwise), later slot base + e holds p_e, and `is_last` marks the
// checker p_n.  The part that combines stores the tile.  `bcast` is an LDS
// word for thread 0's atomic results.
template <int BM, int BN, int WAVES, int TM, int TN>
__device__ __forceinline__ void sk_part_epilogue(f32x16_t (&acc)[TM][TN], const StreamKWs& ws, int t, float* mine,
                                                 int base, int n, bool is_last, char* smem, int* bcast, int wave,
                                                 int lane, uint16_t* __restrict__ out, int M, int N, int row0,
                                                 int col0) {
  const int tid = wave * 64 + lane;
  bool combine;
  if (!is_last) {
    // A storer.
    sk_store_slot<BM, BN, TM, TN>(acc, mine, wave, lane);
    sk_drain();
    __syncthreads();
    if (tid == 0) *bcast = __hip_atomic_fetch_add(ws.ctr + t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __syncthreads();
    const int old = *bcast;
    combine = (old & kSkLastReady) != 0 && (old & kSkStoredMask) == n - 1;
  } else {
    // The checker.
    if (tid == 0)
      *bcast = __hip_atomic_fetch_add(ws.ctr + t, kSkLastArrived, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __syncthreads();
    int old = *bcast;
    combine = (old & kSkStoredMask) == n;
    if (!combine) {
      __syncthreads();  // every thread has read bcast before thread 0 writes it again
      sk_store_slot<BM, BN, TM, TN>(acc, mine, wave, lane);
      sk_drain();
      __syncthreads();
      if (tid == 0)
        *bcast = __hip_atomic_fetch_add(ws.ctr + t, kSkLastReady, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      __syncthreads();
      old = *bcast;
      combine = (old & kSkStoredMask) == n;
    }
  }
  if (!combine) return;
  // Every part has arrived: reset the counter for the next launch.
  if (tid == 0) __hip_atomic_store(ws.ctr + t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  sk_combine<BM, BN, TM, TN>(acc, ws, t, base, n, is_last, wave, lane);
  float one[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) one[i] = 1.0f;
  store_tile<TM, TN, WAVES>(acc, one, smem, wave, lane, out, M, N, row0, col0);
}

// Epilogue of one stream-K segment: K tiles [kb, ke) of tile t, computed by
// workgroup w.  A whole tile is stored; a part runs the protocol (its later
// slot is workgroup w's own, p_e's is that of workgroup first_wg(t) + e).
template <int BM, int BN, int WAVES, int TM, int TN>
__device__ __forceinline__ void sk_epilogue(f32x16_t (&acc)[TM][TN], const StreamKPlan& plan, const StreamKWs& ws,
                                            int w, int t, int kb, int ke, char* smem, int* bcast, int wave,
                                            int lane, uint16_t* __restrict__ out, int M, int N, int row0,
                                            int col0) {
  if (kb == 0 && ke == plan.kt) {
    float one[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) one[i] = 1.0f;
    store_tile<TM, TN, WAVES>(acc, one, smem, wave, lane, out, M, N, row0, col0);
    return;
  }
  const size_t slot = (size_t)BM * BN;
  float* mine = kb == 0 ? ws.first + (size_t)t * slot : ws.later + (size_t)w * slot;
  sk_part_epilogue<BM, BN, WAVES>(acc, ws, t, mine, (int)plan.first_wg(t), (int)plan.later_parts(t), ke == plan.kt,
                                  smem, bcast, wave, lane, out, M, N, row0, col0);
}

// The stream-K kernel: gridDim.x workgroups (the host launches
// streamk_grid(CUs, tiles, K tiles)); `ws` is the workspace, its counters
// zero.  NTB: rhs read non-temporally (variant 6, skinny M).
template <int BM, int BN, int BK, int WAVES, int STAGES, bool NTB>
__global__ __launch_bounds__(WAVES * 64) void mm_lhsT_rhs_bf16_sk_kernel(const uint16_t* __restrict__ lhsT,
                                                                        const uint16_t* __restrict__ rhs,
                                                                        uint16_t* __restrict__ out, int M, int N,
                                                                        int K, int group_m, char* __restrict__ ws) {
  using C = PipeCfg<BM, BN, BK, WAVES, STAGES>;
  __shared__ __attribute__((aligned(1024))) char smem[C::LDS_BYTES];
  __shared__ int bcast;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int KT = (K + BK - 1) / BK;
  const int grid = (int)gridDim.x;
  const StreamKPlan plan((long long)tiles_m * tiles_n, KT, grid);
  const StreamKWs sw{(int*)ws, (float*)(ws + kSkCounterBytes),
                     (float*)(ws + kSkCounterBytes) + (size_t)grid * BM * BN};
  // Logical workgroup id: the dispatcher deals workgroups round-robin to the
  // 8 XCDs, so renumbering gives each XCD a run of consecutive ranges (the
  // workgroups that share a tile mostly run on one XCD).  The protocol
  // itself does not depend on where they run.
  int w = (int)blockIdx.x;
  {
    const int per = grid >> 3, rem = grid & 7, xcd = w & 7;
    w = xcd * per + (xcd < rem ? xcd : rem) + (w >> 3);
  }
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Segments in reverse unit order: the head of the last tile first, the
  // tail of the first tile last (mi_streamk.hpp).
  const long long ubeg = plan.begin(w);
  long long u = plan.begin(w + 1);
  while (u > ubeg) {
    const int t = (int)((u - 1) / KT);
    const long long tstart = (long long)t * KT;
    const int kb = (int)((tstart > ubeg ? tstart : ubeg) - tstart);
    const int ke = (int)(u - tstart);
    const int tm = t % tiles_m, tn = t / tiles_m;
    mm_pipe_body<BM, BN, BK, WAVES, STAGES, false, NTB, false, false, false, true>(
        lhsT, rhs, out, M, N, K, group_m, smem, SplitK{1, nullptr}, RowScale{nullptr, 0, 0.0f, 0.0f},
        SegK{tm, tn, kb, ke - kb}, [&](auto& acc, int row0, int col0) __attribute__((always_inline)) {
          sk_epilogue<BM, BN, WAVES>(acc, plan, sw, w, t, kb, ke, smem, &bcast, wave, lane, out, M, N, row0, col0);
        });
    u = tstart + kb;
  }
}

// lhsT.rhs matmul variant 4: the pipelined core with each K tile's
// sub-steps split over the waves (every wave accumulates the whole block;
// the epilogue sums the waves' blocks).  Half or less of the LDS operand
// bytes per MFMA of a wave-grid split for blocks up to 128x128, at the
// cost of a different fp32 summation order.  SPLIT: split-K as for variant 1.
template <int BM, int BN, int BK, int WAVES, int STAGES, bool SPLIT = false>
__global__ __launch_bounds__(WAVES * 64) void mm_lhsT_rhs_bf16_kw_kernel(const uint16_t* __restrict__ lhsT,
                                                                        const uint16_t* __restrict__ rhs,
                                                                        uint16_t* __restrict__ out, int M, int N,
                                                                        int K, int group_m, int parts,
                                                                        float* __restrict__ ws) {
  __shared__ __attribute__((aligned(1024))) char smem[lds_mm_kw(BM, BN, BK, WAVES, STAGES)];
  mm_pipe_body<BM, BN, BK, WAVES, STAGES, false, false, SPLIT, false, true>(lhsT, rhs, out, M, N, K, group_m, smem,
                                                                           SplitK{parts, ws});
}

// out[M,N] = lhs[M,K] . rhs[K,N] with lhs K-contiguous (matmul_lhs_rhs);
// NTB: rhs read non-temporally (variant 2, skinny M); SPLIT: split-K as for
// the lhsT kernel.
template <int BM, int BN, int BK, int WAVES, int STAGES, bool NTB = false, bool SPLIT = false>
__global__ __launch_bounds__(WAVES * 64) void mm_lhs_rhs_bf16_pipe_kernel(const uint16_t* __restrict__ lhs,
                                                                         const uint16_t* __restrict__ rhs,
                                                                         uint16_t* __restrict__ out, int M, int N,
                                                                         int K, int group_m, int parts,
                                                                         float* __restrict__ ws) {
  __shared__ __attribute__((aligned(1024))) char smem[PipeCfg<BM, BN, BK, WAVES, STAGES>::LDS_BYTES];
  mm_pipe_body<BM, BN, BK, WAVES, STAGES, true, NTB, SPLIT>(lhs, rhs, out, M, N, K, group_m, smem,
                                                            SplitK{parts, ws});
}

// Fused out[M,N] = (x[M,K] * rsqrt(mean_k x^2 + eps)) . W[K,N] without gamma
// (rmsnorm_matmul variant 14): the pipelined K-contiguous core with the
// rows' sums of squares taken from its A fragments (SQ above), so x is read
// once, by LDS-direct loads, and never scaled: 1/rms scales the fp32
// accumulators in the epilogue.
template <int BM, int BN, int BK, int WAVES, int STAGES>
__global__ __launch_bounds__(WAVES * 64) void rmsnorm_mm_bf16_sq_kernel(const uint16_t* __restrict__ x,
                                                                       const uint16_t* __restrict__ w,
                                                                       uint16_t* __restrict__ out, int M, int N,
                                                                       int K, int group_m, float eps, float inv_k) {
  __shared__ __attribute__((aligned(1024))) char smem[PipeCfg<BM, BN, BK, WAVES, STAGES>::LDS_BYTES];
  mm_pipe_body<BM, BN, BK, WAVES, STAGES, true, false, false, false, false, false, NoEpi, true>(
      x, w, out, M, N, K, group_m, smem, SplitK{1, nullptr}, RowScale{nullptr, 0, inv_k, eps});
}

// ---------------------------------------------------------------------------
// Fused out[M,N] = (x[M,K] * rsqrt(mean_k x^2 + eps) * gamma[K]) . W[K,N]
// ---------------------------------------------------------------------------

// acc + the sum of squares of the 8 bf16 values of one 16-byte chunk, in
// fp32 FMAs (each square of a bf16 value is exact in fp32).
__device__ __forceinline__ float sum_sq_chunk(const u32x4_t& w, float acc) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lo = bf16lo(w[e]), hi = bf16hi(w[e]);
    acc = __builtin_fmaf(lo, lo, acc);
    acc = __builtin_fmaf(hi, hi, acc);
  }
  return acc;
}

// Row sums of squares (NA partial sums) and x * gamma (HG) of the 8 bf16
// values of one chunk, in plain fp32 VALU: unpack, FMA, multiply, round.
// (v_dot2c_f32_bf16 does a product pair per instruction, but it issues far
// slower than FMA/multiply next to the MFMAs, so it loses overall.)
template <int NA, bool HG>
__device__ __forceinline__ u32x4_t scale_sumsq_chunk(const u32x4_t& x, const u32x4_t& g, float (&acc)[NA]) {
  u32x4_t o = x;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lo = bf16lo(x[e]), hi = bf16hi(x[e]);
    acc[e % NA] = __builtin_fmaf(lo, lo, acc[e % NA]);
    acc[e % NA] = __builtin_fmaf(hi, hi, acc[e % NA]);
    if constexpr (HG) o[e] = pack_bf16x2(lo * bf16lo(g[e]), hi * bf16hi(g[e]));
  }
  return o;
}
// The same with gamma already unpacked to fp32 (g0: values 0..3, g1: 4..7).
template <int NA, bool HG>
__device__ __forceinline__ u32x4_t scale_sumsq_chunk_f32g(const u32x4_t& x, const f32x4_t& g0, const f32x4_t& g1,
                                                          float (&acc)[NA]) {
  u32x4_t o = x;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lo = bf16lo(x[e]), hi = bf16hi(x[e]);
    acc[e % NA] = __builtin_fmaf(lo, lo, acc[e % NA]);
    acc[e % NA] = __builtin_fmaf(hi, hi, acc[e % NA]);
    if constexpr (HG) {
      const float glo = e < 2 ? g0[2 * e] : g1[2 * e - 4];
      const float ghi = e < 2 ? g0[2 * e + 1] : g1[2 * e - 3];
      o[e] = pack_bf16x2(lo * glo, hi * ghi);
    }
  }
  return o;
}

template <int NA>
__device__ __forceinline__ float sum_parts(const float (&acc)[NA]) {
  if constexpr (NA == 4) return (acc[0] + acc[1]) + (acc[2] + acc[3]);
  else if constexpr (NA == 2) return acc[0] + acc[1];
  else return acc[0];
}

// Sum of v over the KC consecutive lanes that share one x row (KC = 4, 8 or
// 16), broadcast to all of them: a DPP butterfly inside the wavefront.
template <int KC>
__device__ __forceinline__ float row_allreduce(float v) {
  static_assert(KC == 4 || KC == 8 || KC == 16, "row lanes");
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  if constexpr (KC >= 8)
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  if constexpr (KC >= 16)
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  return v;
}

template <int BM, int BN, int BK, int WAVES, int STAGES>
struct RmsCfg {
  using G = WaveGrid<BM, BN, WAVES>;
  static constexpr int NT = WAVES * 64;
  static constexpr int KC = BK / 8;                 // 16-byte chunks per x row per K tile
  static constexpr int CHUNKS = BM * KC;
  static constexpr int CPT = (CHUNKS + NT - 1) / NT;  // chunks per thread
  static constexpr int XD = (128 / BK) > 0 ? (128 / BK) : 1;
  static constexpr int A_BYTES = BM * BK * 2;       // x panel [BM][BK], K contiguous
  static constexpr int B_BYTES = BK * BN * 2;       // W panel [BK][BN], N contiguous
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int MAIN_BYTES = STAGES * STAGE_BYTES;
  static constexpr int EPI_BYTES = WAVES * 32 * (G::WTN * 2 + 16);
  static constexpr int RMS_OFF = ((MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES) + 15) / 16 * 16;
  static constexpr int LDS_BYTES = RMS_OFF + BM * 4;
  static_assert(NT % KC == 0, "row lanes must not straddle threads");
};


template <int BM, int BN, int BK, int WAVES, int STAGES, bool PRE>
__global__ __launch_bounds__(WAVES * 64) void rmsnorm_mm_bf16_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ out, int M, int N, int K, float inv_k, float eps, int group_m) {
  using C = RmsCfg<BM, BN, BK, WAVES, STAGES>;
  using G = typename C::G;
  static_assert(legal_rms_plain(BM, BN, BK, WAVES, STAGES).code == MI_OK, "illegal tile config (mi_legal.hpp)");
  static_assert(C::LDS_BYTES == lds_rms_plain(BM, BN, BK, WAVES, STAGES), "host LDS budget out of step");
  static_assert(G::ok, "illegal wave grid");
  static_assert(BK % 16 == 0, "BK must be a multiple of 16");
  constexpr int TM = G::TM, TN = G::TN, KC = C::KC, CPT = C::CPT, NT = C::NT;
  __shared__ __attribute__((aligned(1024))) char smem[C::LDS_BYTES];
  float* rms_lds = (float*)(smem + C::RMS_OFF);

  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tmi, tni;
  tile_coords(tiles_m, tiles_n, group_m, tmi, tni);
  const int m0 = tmi * BM, n0 = tni * BN;
  const int wm0 = (wave / G::WN) * G::WTM;
  const int wn0 = (wave % G::WN) * G::WTN;
  const bool has_gamma = gamma != nullptr;

  const uint32_t x_bytes = (uint32_t)M * (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, x_bytes);
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(has_gamma ? (const void*)gamma : (const void*)x, (uint32_t)K * 2u);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)K * (uint32_t)N * 2u);

  // x chunks of this thread: chunk c = i*NT + tid -> row c/KC, K chunk tid%KC.
  const int kc = tid % KC;
  int xrow[CPT];
  bool xact[CPT];
  uint32_t xoff[CPT];
  int xlds[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = i * NT + tid;
    xact[i] = c < C::CHUNKS;
    xrow[i] = c / KC;
    xoff[i] = ((uint32_t)(m0 + xrow[i]) * (uint32_t)K + (uint32_t)(8 * kc)) * 2u;
    xlds[i] = xrow[i] * (BK * 2) + 16 * (kc ^ k_swz<BK>(xrow[i]));
  }
  auto load_x = [&](int kt, u32x4_t (&raw)[CPT], u32x4_t& g) {
    const int k = kt * BK + 8 * kc;
    const bool kin = k < K;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const uint32_t off = kin ? xoff[i] + (uint32_t)kt * (uint32_t)(BK * 2) : x_bytes;
      raw[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
    }
    if (has_gamma) g = __builtin_amdgcn_raw_buffer_load_b128(rg, kin ? (uint32_t)k * 2u : (uint32_t)K * 2u, 0, 0);
  };

  PanelLoader<BK, BN, WAVES> lb;
  lb.init(wave, lane, n0, N);
  const uint32_t kstep_b = (uint32_t)BK * (uint32_t)N * 2u;
  TrFrag<BN, TN> fb;
  fb.init(lane, wn0);

  // A fragments: ds_read_b128 of 8 consecutive K of row wm0 + 32*mt + lane%32.
  const int xsl = ((lane & 31) / C::XD) & (KC - 1);
  const int arow = (wm0 + (lane & 31)) * (BK * 2);
  int akoff[BK / 16];
#pragma unroll
  for (int kk = 0; kk < BK / 16; ++kk) akoff[kk] = 16 * ((2 * kk + (lane >> 5)) ^ xsl);

  float ss[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) ss[i] = 0.0f;
  const int KT = (K + BK - 1) / BK;

  float rs[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) rs[i] = 1.0f;
  if constexpr (PRE) {
    // Prologue: full-K sum of squares of this block's rows, 1/rms to LDS.
    for (int kt = 0; kt < KT; ++kt) {
      u32x4_t raw[CPT], g;
      load_x(kt, raw, g);
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = bf16lo(raw[i][e]), hi = bf16hi(raw[i][e]);
          ss[i] = __builtin_fmaf(lo, lo, ss[i]);
          ss[i] = __builtin_fmaf(hi, hi, ss[i]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const float t = row_allreduce<KC>(ss[i]);
      if (xact[i] && kc == 0) rms_lds[xrow[i]] = 1.0f / __builtin_sqrtf(t * inv_k + eps);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < CPT; ++i) rs[i] = xact[i] ? rms_lds[xrow[i]] : 0.0f;
  }

  // Scale the raw x chunks (gamma, and 1/rms in the prologue variant),
  // accumulate the sum of squares (epilogue variant) and write them to LDS.
  auto stage_x = [&](const u32x4_t (&raw)[CPT], const u32x4_t& g, int abase) {
    float gv[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      gv[2 * e] = has_gamma ? bf16lo(g[e]) : 1.0f;
      gv[2 * e + 1] = has_gamma ? bf16hi(g[e]) : 1.0f;
    }
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      if (!xact[i]) continue;
      u32x4_t o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = bf16lo(raw[i][e]), hi = bf16hi(raw[i][e]);
        if constexpr (!PRE) {
          ss[i] = __builtin_fmaf(lo, lo, ss[i]);
          ss[i] = __builtin_fmaf(hi, hi, ss[i]);
        }
        o[e] = pack_bf16x2(lo * gv[2 * e] * rs[i], hi * gv[2 * e + 1] * rs[i]);
      }
      *(MI_LDS u32x4_t*)((MI_LDS char*)smem + abase + xlds[i]) = o;
    }
  };

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16_t{};

  auto compute = [&](int stage) {
    const int abase = stage * C::STAGE_BYTES;
    const int bbase = abase + C::A_BYTES;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      bf16x8_t af[TM], bf[TN];
#pragma unroll
      for (int t = 0; t < TM; ++t)
        af[t] = __builtin_bit_cast(
            bf16x8_t, *(MI_LDS u32x4_t*)((MI_LDS char*)smem + abase + arow + t * 32 * (BK * 2) + akoff[kk]));
#pragma unroll
      for (int t = 0; t < TN; ++t)
        bf[t] = read_tr_frag(smem, bbase + (kk * 16) * (BN * 2) + fb.off[t],
                             bbase + (kk * 16 + 4) * (BN * 2) + fb.off[t]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[j], af[i], acc[i][j], 0, 0, 0);
    }
  };

  if constexpr (STAGES == 1) {
    for (int t = 0; t < KT; ++t) {
      u32x4_t raw[CPT], g;
      lb.issue(rw, smem, C::A_BYTES, kstep_b, t);
      load_x(t, raw, g);
      stage_x(raw, g, 0);
      wait_vmem();
      __syncthreads();
      compute(0);
      __syncthreads();
    }
  } else {
    {
      u32x4_t raw[CPT], g;
      lb.issue(rw, smem, C::A_BYTES, kstep_b, 0);
      load_x(0, raw, g);
      stage_x(raw, g, 0);
      wait_vmem();
      __syncthreads();
    }
    for (int t = 0; t < KT; ++t) {
      const int cur = t & 1;
      const bool more = t + 1 < KT;
      u32x4_t raw[CPT], g;
      if (more) {
        const int nb = (cur ^ 1) * C::STAGE_BYTES;
        lb.issue(rw, smem, nb + C::A_BYTES, kstep_b, t + 1);
        load_x(t + 1, raw, g);
      }
      compute(cur);
      if (more) stage_x(raw, g, (cur ^ 1) * C::STAGE_BYTES);
      wait_vmem();
      __syncthreads();
    }
  }

  float scale[TM];
  if constexpr (!PRE) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const float t = row_allreduce<KC>(ss[i]);
      if (xact[i] && kc == 0) rms_lds[xrow[i]] = 1.0f / __builtin_sqrtf(t * inv_k + eps);
    }
    __syncthreads();
#pragma unroll
    for (int mt = 0; mt < TM; ++mt) scale[mt] = rms_lds[wm0 + mt * 32 + (lane & 31)];
  } else {
#pragma unroll
    for (int mt = 0; mt < TM; ++mt) scale[mt] = 1.0f;
  }
  store_tile<TM, TN, WAVES>(acc, scale, smem, wave, lane, out, M, N, m0 + wm0, n0 + wn0);
}

}  // namespace mi
