/*
 * mi_kernels.h -- C ABI of the MI355X (gfx950) kernel_library hot path.
 *
 * The reference (awslabs/nki-autotune) has no native boundary: its kernels
 * are @nki.jit Python functions that take HBM tensors positionally and
 * allocate and return their output, and its profiler reaches them through
 * KernelJob source text.  Each entry point below replaces one reference
 * interface; the citation names it.  All pointers are device pointers owned
 * by the caller; tensors are row-major and contiguous.  bf16 tensors are
 * passed as raw 16-bit storage; bf16 operands must be 16-byte aligned
 * (fp32 ones 4-byte aligned), and the output must not overlap an input
 * (MI_E_ARGS).  Launches are asynchronous on `stream` (a
 * hipStream_t, NULL = default stream).  No entry point throws, and only a
 * call that needs device workspace allocates: a split-K config (split_k >
 * 1) and the two-pass fused kernel (rmsnorm_matmul variant 13) take it
 * stream-ordered from a library-owned pool (see split_k below).
 *
 * Return value: 0 on success; a positive MI_E_* legality code when the
 * request is rejected before launch; a negative value (-hipError_t) when the
 * HIP runtime reports an error.  mi_last_error() holds the message of the
 * last failure on the calling thread.
 */
#ifndef MI_KERNELS_H
#define MI_KERNELS_H

#ifdef __cplusplus
extern "C" {
#endif

/* Kernel identifiers (one per hot-path kernel family). */
enum {
  MI_KERNEL_MATMUL_LHST_RHS_BF16 = 0, /* lhsT[K,M]^T . rhs[K,N], bf16 in/out, fp32 accumulate */
  MI_KERNEL_MATMUL_LHST_RHS_F32 = 1,  /* same product in fp32 (benchmark config C1)            */
  MI_KERNEL_RMSNORM_MATMUL_BF16 = 2,  /* rmsnorm(x[M,K]) * gamma[K] . W[K,N], bf16 in/out     */
  MI_KERNEL_MATMUL_LHS_RHS_BF16 = 3,  /* lhs[M,K] . rhs[K,N], lhs K-contiguous, bf16 in/out   */
  MI_NUM_KERNELS = 4
};

/* Legality / rejection codes (positive return values). */
enum {
  MI_OK = 0,
  MI_E_NO_INSTANCE = 1,    /* the tile config was not compiled into this library     */
  MI_E_LDS = 2,            /* LDS bytes of the config exceed 160 KiB                 */
  MI_E_WAVE_TILE = 3,      /* a wave's share of the block is smaller than one MFMA   */
  MI_E_ALIGN = 4,          /* M or N (or K of a K-contiguous operand) not a multiple of 8,
                              or a pointer not 16-byte aligned (4-byte for fp32)     */
  MI_E_RANGE = 5,          /* an operand is 4 GiB or larger (32-bit buffer offsets)  */
  MI_E_ARGS = 6,           /* null pointer, non-positive size, bad eps, or an output
                              that overlaps an input                                 */
  MI_E_KERNEL = 7,         /* unknown kernel id                                      */
  MI_E_SPLIT = 8,          /* split_k unsupported for this kernel / shape            */
  MI_E_TILE = 9            /* tile parameters the variant's template does not take, or
                              no such variant                                        */
};

/*
 * Tile meta-parameters: the CDNA4 search space that replaces the NKI block
 * knobs (tbm/tbn/tbk, dim_order, multi-buffer counts;
 * reference kernel_library/README.md:12-13,
 * kernel_library/matmul/lhsT_rhs/kernel_hand_90.92mfu.py:107-112).
 *   block_m, block_n, block_k : workgroup tile (output rows, cols, K panel)
 *   waves                     : wavefronts (64 lanes) per workgroup
 *   lds_stages                : LDS ring depth for K panels (1..4); for matmul
 *                               variant 2 the depth of its register ring
 *   split_k                   : K split over this many workgroups per output
 *                               tile (1..16; > 1 only for the pipelined matmul
 *                               body: lhsT variants 1, 3 and 4, matmul_lhs_rhs
 *                               variants 0 and 2, and the fused kernels on it:
 *                               rmsnorm_matmul variants 4, 5, 11, 12 -- whose
 *                               gamma limit then applies per part -- and 13;
 *                               every part must get at least one K tile).  The
 *                               parts write fp32 partial products (and, fused,
 *                               their rows' sums of squares) to a workspace
 *                               (split_k * (M * N + M) * 4 bytes) that the
 *                               call allocates stream-ordered from a
 *                               library-owned memory pool and frees after the
 *                               launch; a second kernel sums them in part
 *                               order into out (and applies 1/rms, fused).
 *                               Every workspace also starts with 16 KiB of
 *                               stream-K tile counters.  A call's workspace
 *                               is at most 2 GiB.  Outside graph capture a
 *                               workspace of at most 64 MiB is a buffer the
 *                               library keeps per stream (up to 4 streams
 *                               per device; it grows when a call needs
 *                               more), so back-to-back calls allocate
 *                               nothing; a larger one, or any under HIP
 *                               graph capture, is allocated and freed
 *                               around the call (under capture: allocation
 *                               and free nodes of the graph).  The pool
 *                               keeps at most 256 MiB of freed workspace
 *                               cached per device; mi_release_workspace
 *                               returns all of it.
 *   group_m                   : L2 raster group height in tiles (0 = default 8)
 *   variant                   : kernel-specific pipeline (every variant computes
 *                               the same function):
 *     matmul         0 plain double buffer; 1 software-pipelined LDS-direct
 *                    loads; 2 register prefetch ring (skinny shapes); 3 as 1
 *                    with rhs read non-temporally (streamed once: skinny M);
 *                    4 as 1 with each K tile's 16-deep sub-steps split over
 *                    the waves, every wave accumulating the whole block (at
 *                    most 128x128) and the epilogue adding the waves' sums
 *                    in wave order (few output tiles, long K).  Variant 4
 *                    adds in another fp32 order than 0..3, so its result
 *                    may differ from theirs in the last bit; 5 stream-K: a
 *                    grid of one workgroup per CU (at most 4096 output
 *                    tiles), each taking an equal share of all tiles' K
 *                    loops on the pipelined core; a tile computed in parts
 *                    is summed by the part that finishes it, in K order,
 *                    from fp32 partials in the workspace ((CUs + tiles) *
 *                    block_m * block_n * 4 bytes after the counters); 6 as
 *                    5 with rhs read non-temporally (skinny M)
 *     matmul_lhs_rhs 0 the software-pipelined core (block_k >= 32, 2..4 stages);
 *                    1 the same with the K-contiguous A panel loaded two K
 *                    tiles per load (block_k 32 or 64); 2 as 0 with rhs read
 *                    non-temporally (skinny M)
 *     rmsnorm_matmul 0 / 1 x scaled while staged (1/rms on the accumulators /
 *                    from a prologue pass); 4 / 5 x through a 2 / 3 tile
 *                    register ring on the pipelined matmul core (gamma staged
 *                    in LDS: K up to 8192 per part); 11 / 12 as 4 / 5 with W
 *                    read non-temporally (skinny M); 13 two passes: a pack
 *                    kernel writes bf16(x * gamma) in the lhsT layout and
 *                    the rows' sums of squares to the workspace (K * M * 2 +
 *                    ceil(K / 512) * M * 4 bytes), then the pipelined lhsT
 *                    core applies 1/rms to its fp32 accumulators; 15 as 13
 *                    with the pack in x's own layout (K * M * 2 bytes as
 *                    well) and the paired-load K-contiguous core of
 *                    matmul_lhs_rhs variant 1 (bitwise equal to 13); 14
 *                    without gamma only (gamma != NULL: MI_E_TILE): the
 *                    matmul_lhs_rhs core reads x once, LDS-direct, sums its
 *                    rows' squares from the MFMA A fragments (bf16 dot2)
 *                    and applies 1/rms to its fp32 accumulators; 16 as 14
 *                    on the paired-load core of matmul_lhs_rhs variant 1
 *                    (block_k 32 or 64; without gamma only).  Variants
 *                    2, 3 and 6..10 do not exist (MI_E_TILE).
 */
typedef struct {
  int block_m, block_n, block_k, waves, lds_stages, split_k, group_m, variant;
} mi_tile_cfg;

/* Static legality of `cfg` for kernel `kernel_id` at M,N,K (no launch).
 * Replaces the compile-time rejection of an NKI candidate
 * (reference autotune/src/autotune/runner/compile.py:197-244, which turns a
 * failed neuronx-cc compile into an error string). */
int mi_cfg_check(int kernel_id, const mi_tile_cfg* cfg, int M, int N, int K);

/* Enumerate the configs compiled into the library for `kernel_id`.
 * mi_num_configs returns the count; mi_get_config fills cfg for idx. */
int mi_num_configs(int kernel_id);
int mi_get_config(int kernel_id, int idx, mi_tile_cfg* cfg);

/* The library's default config for a kernel at a shape: always prebuilt and
 * legal there.  Generalised from the autotune winners: the block whose
 * rounds of tiles take the least estimated time (rounds on the busiest CU
 * times the block's area over its measured rate per CU), split-K when that
 * grid leaves CUs idle (or where a small block faces a long K), non-temporal
 * variants for skinny M sized by an estimate of each workgroup's panel
 * bytes; for the fused kernel, the one-pass and two-pass kernels weighed by
 * the same estimate with their split and pack passes charged, past the K
 * its gamma staging holds split until each part's gamma fits.
 * A negative size is MI_E_ARGS. */
int mi_default_config(int kernel_id, int M, int N, int K, mi_tile_cfg* cfg);

/* The default of rmsnorm_matmul for a call without gamma (what
 * mi_rmsnorm_matmul_bf16 takes when cfg and gamma are both NULL):
 * mi_default_config's pick, except that its 64x128 and 64x64 blocks go to
 * the gamma-free variant 14 with the same block, and its 128x128 blocks to
 * the largest gamma-free block whose grid keeps more than half the CUs busy
 * (variant 16 at 128x128 with block_k 32 and 4 stages, else variant 14 at
 * 64x128, else at 64x64), all unsplit.
 * No counterpart in the reference, whose kernel has no gamma at all; for
 * callers of its contract (rmsnorm_matmul_online).  A negative size is
 * MI_E_ARGS. */
int mi_default_config_no_gamma(int M, int N, int K, mi_tile_cfg* cfg);

/* out[M,N] = lhsT[K,M]^T . rhs[K,N]; bf16 storage, fp32 accumulation over
 * the whole K (over each K part, then across parts in part order, when
 * cfg->split_k > 1), one round-to-nearest-even store.
 * Replaces matmul_lhsT_rhs_nkigym(lhs_T, rhs)
 * (reference kernel_library/matmul/lhsT_rhs/kernel_hand_90.92mfu.py:101-131).
 * cfg == NULL selects mi_default_config. */
int mi_matmul_lhsT_rhs_bf16(const void* lhsT, const void* rhs, void* out, int M, int N, int K,
                            const mi_tile_cfg* cfg, void* stream);

/* out[M,N] = lhs[M,K] . rhs[K,N] with lhs row-major (K contiguous); bf16
 * storage, fp32 accumulation over the whole K.  K must be a multiple of 8.
 * Replaces matmul_lhs_rhs_nkigym(lhs, rhs)
 * (reference kernel_library/matmul/lhs_rhs/kernel_handtuned_89.26mfu.py:226-287).
 * cfg == NULL selects mi_default_config; the pipelined core is variant 0. */
int mi_matmul_lhs_rhs_bf16(const void* lhs, const void* rhs, void* out, int M, int N, int K,
                           const mi_tile_cfg* cfg, void* stream);

/* fp32 variant of the lhsT product (the fp32 CPU-simulation semantics of
 * reference nkigym/src/nkigym/synthesis/simulate_nki.py:24-48).  Variant 0:
 * LDS-tiled FMAs, K summed in sequential order (64x64 blocks, block_k 16 or
 * 32); variant 1: the fp32 MFMA (v_mfma_f32_32x32x2_f32), K summed two at a
 * time (64x64 or 128x128 blocks, block_k 16).  Any M, N, K; 4-byte aligned
 * pointers; cfg == NULL selects mi_default_config. */
int mi_matmul_lhsT_rhs_f32(const float* lhsT, const float* rhs, float* out, int M, int N, int K,
                           const mi_tile_cfg* cfg, void* stream);

/* out[M,N] = (x[M,K] / sqrt(mean_k x^2 + eps) * gamma[K]) . W[K,N];
 * bf16 storage, fp32 accumulation and fp32 row statistics.
 * gamma == NULL means gamma = 1, which is exactly the reference kernel
 * rmsnorm_matmul_online(lhs, rhs) with EPS = 1e-6
 * (reference kernel_library/rmsnorm_matmul/kernel_hand_online.py:195-353).
 * cfg == NULL selects mi_default_config, or mi_default_config_no_gamma
 * when gamma is NULL too; variant 14 or 16 with gamma is MI_E_TILE. */
int mi_rmsnorm_matmul_bf16(const void* x, const void* gamma, const void* W, void* out, int M, int N,
                           int K, float eps, const mi_tile_cfg* cfg, void* stream);

/* mi_matmul_lhsT_rhs_bf16 without any device allocation.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, result and errors as mi_matmul_lhsT_rhs_bf16;
 * the workspace of a split-K or stream-K config (16 KiB of stream-K
 * counters, then split_k * M * N * 4 bytes of fp32 partial products, or the
 * stream-K partial tiles) is a static device array of MI_NOALLOC_SCRATCH_BYTES
 * that each GPU holds from the first call there until the process ends, and
 * a config needing more returns MI_E_RANGE (cfg == NULL never does: the
 * default splits at most 256 blocks of 256 x 256).  Calls on one GPU share that
 * array: calls ordered on one stream are safe, calls that overlap on one GPU
 * race. */
#define MI_NOALLOC_SCRATCH_BYTES (64ull * 1024ull * 1024ull)
int mi_matmul_lhsT_rhs_bf16_noalloc(const void* lhsT, const void* rhs, void* out, int M, int N, int K,
                                    const mi_tile_cfg* cfg, void* stream);

/* Device discovery: number of visible HIP devices and the gfx arch name of
 * device 0 (written to arch, at most arch_len bytes).  Returns 0 or -error.
 * Replaces detect_neuron_cores()
 * (reference autotune/src/autotune/runner/detect.py:7-20). */
int mi_device_info(int* num_devices, char* arch, int arch_len, int* num_cus);

/* Returns the device memory the library holds for split-K, stream-K and
 * two-pass workspace to the device, on every device the library has used:
 * the buffers kept per stream (after a device synchronisation) and what
 * earlier calls freed into the library's pool.  Without it, the runtime
 * hands a call's freed workspace back to the library's pool only at the
 * pool's next allocation (the next call that needs workspace), which then
 * keeps at most 256 MiB cached: between calls the library holds its kept
 * buffers (at most 64 MiB for each of up to 4 streams per device) plus up
 * to the last larger call's workspace and 256 MiB.  Not under graph
 * capture.  No counterpart in the reference (its kernels allocate nothing
 * beyond their output).  Returns 0 or -error. */
int mi_release_workspace(void);

/* Message of the last failure on the calling thread ("" if none). */
const char* mi_last_error(void);

/* Library version string. */
const char* mi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* MI_KERNELS_H */
