// Host-visible kernel parameter blocks and registries shared between the kernel translation units
// and the C ABI (fa_abi.hip).
#pragma once

#include <stdint.h>

namespace fa {

// One attention-forward launch. Pointers are device pointers; strides are in elements.
struct FwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;     // nullable: fp32 [B,H,M] natural-log sum-exp of the scaled logits
  float* ws_o;    // split partials [splits][B*H][M][D] fp32 (SPLIT kernels only)
  float* ws_lse;  // split partial lse [splits][B*H][M] fp32 (SPLIT kernels only)
  int64_t sq0, sq1, sq2;
  int64_t sk0, sk1, sk2;
  int64_t sv0, sv1, sv2;
  int64_t so0, so1, so2;
  int64_t sl0, sl1, sl2;
  int32_t B, H, Hkv, M, N;
  int32_t group;            // H / Hkv
  int32_t pack;             // 1, or group: the query heads of a kv head share one row space
                            // (row r = head offset r / M, position r % M); grid over (b, kv head)
  float c;                  // sm_scale * log2(e): exp(x*sm_scale) == exp2(x*c)
  float sm_scale;
  int32_t causal;
  int32_t splits;           // KV splits (1 when not splitting)
  int32_t tiles_per_split;  // KV tiles (of block_n rows) per split
  int32_t m_blocks;         // ceil(M / block_m)
  int32_t total_blocks;     // m_blocks * B * H * splits
};

struct MergeParams {
  const float* ws_o;
  const float* ws_lse;
  uint16_t* o;
  float* lse;
  int64_t so0, so1, so2;
  int64_t sl0, sl1, sl2;
  int32_t B, H, M, splits;
  int32_t waves_per_row;  // 1, 2 or 4: the waves of a workgroup that share one row's splits
};

typedef void (*FwdKernelFn)(FwdParams);
typedef void (*MergeKernelFn)(MergeParams);

struct FaKernelEntry {
  int32_t stages;  // 1 = single-buffered K/V LDS (basic), 2 = double-buffered (optimized)
  int32_t dtype;   // FA_DTYPE_*
  int32_t D;
  int32_t waves;
  int32_t rows_per_wave;
  int32_t block_n;
  int32_t split;   // writes fp32 partials for the LSE merge
  const void* fn;
};

struct FaMergeEntry {
  int32_t dtype;
  int32_t D;
  const void* fn;
};

const FaKernelEntry* fa_fwd_registry(int* count);
const FaMergeEntry* fa_merge_registry(int* count);

struct GemmParams {
  const uint16_t* a;
  const uint16_t* b;
  uint16_t* c;
  int32_t M, N, K;
  int64_t lda, ldb, ldc;
  int32_t group_m;
  int32_t tiles_m, tiles_n;
  int32_t region_m;  // 0: flat grouped order; else XCD regions in region_m rows x (8 / region_m) columns
};

struct GemmKernelEntry {
  int32_t block_m, block_n, block_k, waves;
  const void* fn;          // default slab ring (as deep as fits in 128 KiB, up to 4)
  const void* fn_shallow;  // shallow ring for short K (nullptr when it would be the same)
};

// K slabs up to which a tile's shallow-ring kernel is launched (more workgroups per CU beat a
// deeper prefetch when the whole K loop is this short).
constexpr int kGemmShallowMaxSlabs = 8;

const GemmKernelEntry* gemm_registry(int* count);

}  // namespace fa
