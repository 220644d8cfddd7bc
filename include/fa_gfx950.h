/*
 * fa_gfx950.h -- C ABI of libfa_gfx950.so, the MI355X (gfx950 / CDNA4) FlashAttention-forward
 * and fp16 GEMM library.
 *
 * Every entry point is plain C: pointers, fixed-width integers and floats, no HIP or torch types.
 * Device pointers come from the caller (PyTorch allocates every buffer, including the split-KV
 * workspace); the library never allocates or frees device memory. `stream` is a hipStream_t
 * passed as void* (the caller's current stream); no entry point synchronises the host.
 *
 * Return value of every int-returning entry point: FA_OK (0) or one of the FA_E* codes below;
 * fa_last_error() then gives a thread-local message.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   fa_fwd(variant=FA_VARIANT_BASIC)   <- _flash_attn_fwd_kernel_basic[grid](...)          flash_atten.py:14-50
 *   fa_fwd(variant=FA_VARIANT_OPT)     <- _flash_attn_fwd_kernel_optimize_shared_mem[...]   flash_atten.py:136-172
 *   fa_fwd(variant=FA_VARIANT_SLICED)  <- _flash_attn_fwd_kernel_block_d_nomask_contiguous  flash_atten.py:261-275
 *                                         (re-defined as split-KV partials + LSE merge)
 *   gemm_f16                           <- _matmul_contiguous_kernel[grid](a,b,c,M,N,K,...)  mma.py:8-21
 *   fa_device_limits                   <- get_sm_resource_limits()                         exceptions.py:760-775
 *   fa_kernel_resources                <- Triton compile metadata (shared, n_regs)          tuner.py:341-376
 *   fa_kernel_symbol                   <- the compiled kernel that metadata belongs to      tuner.py:356-357
 *   fa_fwd_noalloc                     (no counterpart: fa_fwd for callers that cannot allocate)
 */
#ifndef FA_GFX950_H
#define FA_GFX950_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_ABI_VERSION 4

enum {
  FA_OK = 0,
  FA_EINVAL = 1,      /* bad shape, stride, pointer or argument combination          */
  FA_ENOTSUP = 2,     /* head dim / dtype / tile configuration not built              */
  FA_EHIP = 3,        /* a HIP runtime call failed (message carries hipGetErrorString) */
  FA_EWORKSPACE = 4,  /* split-KV workspace missing or too small                      */
};

enum { FA_DTYPE_F16 = 0, FA_DTYPE_BF16 = 1 };

/* The three reference kernels (flash_atten.py:364-368). */
enum { FA_VARIANT_BASIC = 0, FA_VARIANT_OPT = 1, FA_VARIANT_SLICED = 2 };

/* One attention tile configuration. block_m = waves * rows_per_wave (rows_per_wave in {32, 64});
 * block_n = KV rows per LDS tile; splits = KV splits of the sliced variant (1 = no split, no merge
 * pass). stages selects the K/V pipeline of the optimized and sliced variants (basic always runs
 * stages 1):
 *   1  one K/V LDS buffer, staged through registers;
 *   2  double-buffered K/V LDS tiles, staged through registers;
 *   3  software-pipelined kernel: K/V reach a ring of LDS tiles by LDS-DMA, and the QK^T MFMAs of
 *      tile u+1 run beside the softmax of tile u;
 *   4  two-tile-ahead pipeline on the same rings: the QK^T MFMAs of tile u+2 alternate with the PV
 *      MFMAs of tile u while the softmax of tile u+1 runs;
 *   5  one tile per step on a 2-slot LDS-DMA ring, lean enough in registers for two waves per
 *      SIMD (D = 256: O and Q in VGPRs);
 *   6  the stages=5 pipeline with 16x16x32 MFMA tiles (less accumulator traffic per flop) instead
 *      of 32x32x16 ones; 32 query rows per wave;
 *   7  the stages=3 pipeline with 16x16x32 MFMA tiles (D <= 128);
 *   8  ping-pong (block_m 256, 8 waves, block_n 64, D <= 128): two groups of four waves, one phase
 *      apart, alternate a matrix phase (QK^T of the next tile, PV of this one) and a softmax phase,
 *      so that on every SIMD one wave issues MFMAs while the other issues the exp/pack work;
 *   9  the stages=8 ping-pong in a persistent grid (one workgroup per CU walks a fixed sequence of
 *      query blocks; the last steps of a block fetch the next block's Q, K and V, so blocks start
 *      without waiting on memory). Launches whose query heads fa_fwd_pack_group would pack, or
 *      whose Q rows (M * q_stride[2] * 2 bytes) reach 2^32, run the stages=8 kernel instead.
 *   The LDS-DMA kernels (3-9) need (N + block_n) * max(k_stride[2], v_stride[2]) * 2 < 2^32
 *   bytes and row strides >= D; when a launch breaks either rule, fa_fwd runs the stages=2 kernel
 *   of the same block_m and waves instead (same block_n where built, else 64). fa_fwd_supported()
 *   reports such a tile as built only when that fallback is built too. */
typedef struct {
  int32_t block_m;
  int32_t block_n;
  int32_t waves;
  int32_t stages;
  int32_t splits;
} fa_tile;

/* Arguments of one attention forward. Tensors are [batch, heads, seq, head_dim] with element
 * strides (the 16 stride arguments of flash_atten.py:20-39); the head_dim stride must be 1.
 * H_kv divides H (grouped-query attention: query head h reads kv head h / (H / H_kv)).
 * lse (nullable) is fp32 [B, H, M] with strides lse_stride: natural-log sum-exp of the scaled
 * logits, as flash_atten.py:130-133. workspace is required when variant == SLICED and
 * tile.splits > 1; its size is fa_fwd_workspace_bytes(). causal is top-left (row i sees keys
 * j <= i), as flash_atten.py:103-105. */
typedef struct {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  void* workspace;
  int64_t workspace_bytes;
  int64_t q_stride[4];
  int64_t k_stride[4];
  int64_t v_stride[4];
  int64_t o_stride[4];
  int64_t lse_stride[3];
  int32_t B, H, H_kv, M, N, D;
  float sm_scale;
  int32_t dtype;
  int32_t causal;
  int32_t variant;
  fa_tile tile;
} fa_fwd_args;

/* GEMM tile configuration: block_m x block_n macro tile, block_k deep, waves per workgroup,
 * group_m rows of tiles per L2 group (mma.py:22-30 GROUP_M). The 128x128x32 and 64x64x32 tiles
 * with 8 waves and the 128x64x32 tile with 8 or 16 waves split each tile's K loop over 2 or 4
 * groups of 4 waves (partial sums added through LDS inside the workgroup). */
typedef struct {
  int32_t block_m;
  int32_t block_n;
  int32_t block_k;
  int32_t waves;
  int32_t group_m;
} gemm_tile;

/* Per-kernel resources. vgprs, agprs, sgprs, scratch_bytes and occupancy come from a table that
 * the build generates from the compiler's resource-usage report for each gfx950 kernel and links
 * into the library; lds_bytes and max_threads are read from the loaded kernel at run time
 * (hipFuncGetAttributes). */
typedef struct {
  int32_t vgprs;          /* architectural VGPRs per lane                          */
  int32_t agprs;          /* accumulation VGPRs per lane                           */
  int32_t sgprs;          /* scalar registers per wave                             */
  int32_t lds_bytes;      /* static LDS per workgroup                              */
  int32_t scratch_bytes;  /* private (spill) bytes per lane                        */
  int32_t threads;        /* threads per workgroup                                 */
  int32_t max_threads;    /* largest workgroup the kernel accepts                  */
  int32_t occupancy;      /* waves per SIMD the register and LDS budgets allow     */
} fa_resources;

/* Device limits (the keys of exceptions.py:766-774, in gfx950 terms). */
typedef struct {
  int32_t lds_bytes_per_cu;
  int32_t registers_per_simd;       /* 512 VGPR+AGPR lanes-registers x 64 lanes              */
  int32_t register_file_bytes_per_simd;
  int32_t wavefront_size;
  int32_t max_threads_per_block;
  int32_t cu_count;
  int32_t clock_khz;
  int32_t gcn_arch;                 /* e.g. 950                                              */
} fa_device_limits_t;

int fa_abi_version(void);

/* Thread-local text of the last error returned on this thread ("" if none). */
const char* fa_last_error(void);

/* Attention forward; launches on `stream`. */
int fa_fwd(const fa_fwd_args* args, void* stream);

/* fa_fwd without a workspace argument, for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc). The split-KV partials go to a
 * static device array of FA_NOALLOC_SCRATCH_BYTES that each GPU holds until the process ends;
 * args->workspace must be NULL and args->workspace_bytes 0. A launch whose partials
 * (fa_fwd_workspace_bytes) exceed the array fails with FA_EWORKSPACE before anything runs.
 * Calls on one GPU share its array: calls that overlap (other streams, other threads) race, so
 * the caller orders them. Launches without splits use no scratch and behave as fa_fwd. The first
 * call on a device looks up that device's array address (hipGetSymbolAddress), so make one call
 * on each device before capturing fa_fwd_noalloc into a HIP graph. No counterpart in the reference
 * (for callers that cannot allocate). */
#define FA_NOALLOC_SCRATCH_BYTES (64LL << 20)
int fa_fwd_noalloc(const fa_fwd_args* args, void* stream);

/* Bytes of split-KV workspace fa_fwd needs for these sizes (0 when splits <= 1). */
int64_t fa_fwd_workspace_bytes(int32_t B, int32_t H, int32_t M, int32_t D, int32_t splits);

/* Query heads that fa_fwd packs into one tile's rows (1 = none): decode-shaped split-KV launches
 * (splits > 1, non-causal, H > H_kv, M * H / H_kv <= block_m) give each workgroup all query heads
 * of one kv head, so K/V are read once per kv head; the grid then runs over (batch, kv head).
 * Callers sizing `splits` for a target grid use it to count workgroups. Part of the behaviour of
 * the sliced path (flash_atten.py:261-361 re-defined as split-KV), no separate reference entry. */
int32_t fa_fwd_pack_group(int32_t H, int32_t H_kv, int32_t M, int32_t causal, int32_t block_m, int32_t splits);

/* Is this (variant, dtype, D, tile) built? Returns FA_OK or FA_ENOTSUP. */
int fa_fwd_supported(int32_t variant, int32_t dtype, int32_t D, const fa_tile* tile);

/* C[M,N] (fp16, row stride ldc) = A[M,K] (fp16, lda) x B[K,N] (fp16, ldb), fp32 accumulation;
 * launches on `stream`. Partial tiles are masked: any M, with K % 8 == 0 and N % 4 == 0 (16-byte
 * loads, 8-byte stores); lda and ldb multiples of 8, ldc of 4. (The reference needs multiples of
 * the tile, mma.py:63-81; its selector, mma._select_2d_contiguous_config, keeps that rule.)
 * When K spans at most 8 slabs (K <= 8 * block_k) the tile's shallow-ring kernel runs (two LDS
 * slabs, more workgroups per CU), where one is built; fa_kernel_resources reports the default
 * (deep-ring) kernel of the tile. */
int gemm_f16(const void* a, const void* b, void* c, int32_t M, int32_t N, int32_t K,
             int64_t lda, int64_t ldb, int64_t ldc, const gemm_tile* tile, void* stream);

int gemm_f16_supported(const gemm_tile* tile);

/* Resources of one built kernel: op 0 = attention (variant, dtype, D, tile; the kernel that tile
 * resolves to, before any stages=3 fallback), op 1 = GEMM (gtile; the default deep-ring kernel).
 * Needs a device (hipFuncGetAttributes). */
int fa_kernel_resources(int32_t op, int32_t variant, int32_t dtype, int32_t D, const fa_tile* tile,
                        const gemm_tile* gtile, fa_resources* out);

/* Mangled symbol of the kernel fa_kernel_resources describes for the same arguments (the name
 * under which the compiler's resource report and profiler traces list it), NUL-terminated into
 * buf[0..buf_bytes). The tuner uses it to match its candidates to those rows (the reference's
 * tuner reads the compiled kernel's registers and shared memory, tuner.py:341-376).
 * Needs no device. FA_EINVAL when the buffer is too small. */
int fa_kernel_symbol(int32_t op, int32_t variant, int32_t dtype, int32_t D, const fa_tile* tile,
                     const gemm_tile* gtile, char* buf, int32_t buf_bytes);

int fa_device_limits(int32_t device, fa_device_limits_t* out);

#ifdef __cplusplus
}
#endif

#endif /* FA_GFX950_H */
