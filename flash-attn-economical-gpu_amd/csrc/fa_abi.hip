// C ABI of libfa_gfx950.so (declared in include/fa_gfx950.h): argument validation, kernel
// selection from the registries of built instantiations, and launches on the caller's stream.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <atomic>
#include <string>

#include "fa_kernels.h"
#include "../../include/fa_gfx950.h"

// Split-KV partials of fa_fwd_noalloc (no allocation on that path). Each GPU holds its own copy
// of this array for the life of the process; its address on a device comes from
// hipGetSymbolAddress with that device current, once, and only that address is handed to kernels
// (the array's name in host code is a host-side stand-in, not a device address). Nothing in it
// needs to start at zero: every split writes all of its partial rows before the merge reads them.
constexpr int64_t kScratchBytes = FA_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return FA_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

const fa::FaKernelEntry* find_fwd(int stages, int dtype, int D, int waves, int rows_per_wave, int block_n,
                                  int split) {
  // stages 1-5: fa_fwd.hip (32x32x16 MFMAs); stages 6-9: fa_fwd16.hip (16x16x32 MFMAs)
  int n = 0;
  const fa::FaKernelEntry* e = stages >= 6 ? fa::fa_fwd16_registry(&n) : fa::fa_fwd_registry(&n);
  for (int i = 0; i < n; ++i)
    if (e[i].stages == stages && e[i].dtype == dtype && e[i].D == D && e[i].waves == waves &&
        e[i].rows_per_wave == rows_per_wave && e[i].block_n == block_n && e[i].split == split)
      return &e[i];
  return nullptr;
}

const fa::FaMergeEntry* find_merge(int dtype, int D) {
  int n = 0;
  const fa::FaMergeEntry* e = fa::fa_merge_registry(&n);
  for (int i = 0; i < n; ++i)
    if (e[i].dtype == dtype && e[i].D == D) return &e[i];
  return nullptr;
}

const fa::GemmKernelEntry* find_gemm(const gemm_tile* t) {
  int n = 0;
  const fa::GemmKernelEntry* e = fa::gemm_registry(&n);
  for (int i = 0; i < n; ++i)
    if (e[i].block_m == t->block_m && e[i].block_n == t->block_n && e[i].block_k == t->block_k &&
        e[i].waves == t->waves)
      return &e[i];
  return nullptr;
}

// Pipeline of a launch: basic keeps one K/V buffer (1); optimized and sliced double-buffer K/V (2),
// or, when the tile asks for stages 3-9, run that LDS-DMA kernel (3-5: 32x32x16 MFMA tiles, 6-9:
// 16x16x32 ones; the stages doc of fa_tile in the header lists them).
int stages_of(int variant, const fa_tile* t) {
  if (variant == FA_VARIANT_BASIC) return 1;
  return (t != nullptr && t->stages >= 3 && t->stages <= 9) ? t->stages : 2;
}

// Compute units of the current device (the persistent kernel's grid), looked up once per device.
int current_device_cus(int* cus) {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return fail(FA_EHIP, "hipGetDevice failed: %s", hipGetErrorString(err));
  if (dev >= 0 && dev < kMaxDevices) {
    const int known = cache[dev].load(std::memory_order_relaxed);
    if (known > 0) {
      *cus = known;
      return FA_OK;
    }
  }
  int n = 0;
  err = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
  if (err != hipSuccess || n <= 0) return fail(FA_EHIP, "hipDeviceGetAttribute(CU count) failed: %s", hipGetErrorString(err));
  if (dev >= 0 && dev < kMaxDevices) cache[dev].store(n, std::memory_order_relaxed);
  *cus = n;
  return FA_OK;
}

// Resolve (variant, tile) to the main kernel; nullptr + message when not built.
const fa::FaKernelEntry* resolve_fwd(int variant, int dtype, int D, const fa_tile* t, bool* split_out,
                                     int* code) {
  *code = FA_OK;
  if (variant < FA_VARIANT_BASIC || variant > FA_VARIANT_SLICED) {
    *code = fail(FA_EINVAL, "unknown attention variant %d", variant);
    return nullptr;
  }
  if (dtype != FA_DTYPE_F16 && dtype != FA_DTYPE_BF16) {
    *code = fail(FA_ENOTSUP, "unsupported dtype code %d (fp16=0, bf16=1)", dtype);
    return nullptr;
  }
  if (D != 64 && D != 128 && D != 256) {
    *code = fail(FA_ENOTSUP, "head dim D=%d is not built (64, 128, 256)", D);
    return nullptr;
  }
  if (t == nullptr || t->waves <= 0 || t->block_m <= 0 || t->block_m % t->waves != 0) {
    *code = fail(FA_EINVAL, "invalid attention tile");
    return nullptr;
  }
  const int splits = t->splits < 1 ? 1 : t->splits;
  if (variant != FA_VARIANT_SLICED && splits != 1) {
    *code = fail(FA_EINVAL, "splits=%d requires the sliced variant", splits);
    return nullptr;
  }
  const bool split = splits > 1;
  *split_out = split;
  const fa::FaKernelEntry* e =
      find_fwd(stages_of(variant, t), dtype, D, t->waves, t->block_m / t->waves, t->block_n, split ? 1 : 0);
  if (e == nullptr)
    *code = fail(FA_ENOTSUP,
                 "attention tile block_m=%d block_n=%d waves=%d stages=%d split=%d is not built for "
                 "dtype=%d D=%d",
                 t->block_m, t->block_n, t->waves, stages_of(variant, t), split ? 1 : 0, dtype, D);
  return e;
}

// Does the pipelined (stages=3 or 4) kernels' addressing hold for this launch? It reads one (batch,
// kv-head) row range [0, N + block_n) of K and V with 32-bit byte offsets, and its tail check needs
// whole rows (row stride >= D).
bool pipelined_fits(const fa_fwd_args* a, int block_n) {
  const int64_t stride = a->k_stride[2] > a->v_stride[2] ? a->k_stride[2] : a->v_stride[2];
  const int64_t span = ((int64_t)a->N + block_n) * 2 * stride;
  return span <= 0xffffffffLL && a->k_stride[2] >= a->D && a->v_stride[2] >= a->D;
}

// The double-buffered kernel that replaces a pipelined one when pipelined_fits() fails: same
// dtype, D, waves, rows per wave and split, the same block_n if built, else 64 keys.
const fa::FaKernelEntry* double_buffered_fallback(const fa::FaKernelEntry* e) {
  const fa::FaKernelEntry* fb = find_fwd(2, e->dtype, e->D, e->waves, e->rows_per_wave, e->block_n, e->split);
  if (fb == nullptr) fb = find_fwd(2, e->dtype, e->D, e->waves, e->rows_per_wave, 64, e->split);
  return fb;
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return fail(FA_EHIP, "hipGetDevice failed: %s", hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxDevices) return fail(FA_EINVAL, "device index %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr)
      return fail(FA_EHIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(err));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return FA_OK;
}

const fa::KernelResourceRow* find_resource_row(const char* symbol) {
  for (int i = 0; i < fa::kKernelResourceRowCount; ++i)
    if (std::strcmp(fa::kKernelResourceRows[i].symbol, symbol) == 0) return &fa::kKernelResourceRows[i];
  return nullptr;
}

// GEMM tile regions per XCD: the split of the tile grid into region_m x (8 / region_m) equal
// rectangles whose A + B panel footprint (rows * block_m + columns * block_n) is smallest, or 0
// (flat grouped order) when no split divides the grid.
int gemm_region_rows(int tiles_m, int tiles_n, int block_m, int block_n) {
  constexpr int kXcds = 8;
  int best = 0;
  int64_t best_cost = 0;
  for (int rm = 1; rm <= kXcds; rm *= 2) {
    const int rn = kXcds / rm;
    if (tiles_m % rm != 0 || tiles_n % rn != 0) continue;
    const int64_t cost = (int64_t)(tiles_m / rm) * block_m + (int64_t)(tiles_n / rn) * block_n;
    if (best == 0 || cost < best_cost) {
      best = rm;
      best_cost = cost;
    }
  }
  return best;
}

}  // namespace

extern "C" {

int fa_abi_version(void) { return FA_ABI_VERSION; }

const char* fa_last_error(void) { return g_last_error.c_str(); }

int64_t fa_fwd_workspace_bytes(int32_t B, int32_t H, int32_t M, int32_t D, int32_t splits) {
  if (splits <= 1 || B <= 0 || H <= 0 || M <= 0 || D <= 0) return 0;
  const int64_t rows = (int64_t)splits * B * H * M;
  const int64_t o_bytes = rows * D * 4;
  const int64_t lse_off = (o_bytes + 255) & ~(int64_t)255;
  return lse_off + rows * 4;
}

int32_t fa_fwd_pack_group(int32_t H, int32_t H_kv, int32_t M, int32_t causal, int32_t block_m, int32_t splits) {
  if (H <= 0 || H_kv <= 0 || H % H_kv != 0 || M <= 0 || block_m <= 0) return 1;
  const int32_t group = H / H_kv;
  if (splits <= 1 || causal || group <= 1 || (int64_t)M * group > block_m) return 1;
  return group;
}

int fa_fwd_supported(int32_t variant, int32_t dtype, int32_t D, const fa_tile* tile) {
  bool split = false;
  int code = FA_OK;
  const fa::FaKernelEntry* e = resolve_fwd(variant, dtype, D, tile, &split, &code);
  if (e == nullptr) return code;
  if (split && find_merge(dtype, D) == nullptr) return fail(FA_ENOTSUP, "no merge kernel for D=%d", D);
  if (e->stages >= 3 && double_buffered_fallback(e) == nullptr)
    return fail(FA_ENOTSUP, "pipelined tile without a double-buffered fallback for D=%d", D);
  return ok();
}

// The body of fa_fwd and fa_fwd_noalloc: the split-KV workspace comes in as (ws, ws_bytes).
static int launch_fwd(const fa_fwd_args* a, void* ws, int64_t ws_bytes, void* stream) {
  bool split = false;
  int code = FA_OK;
  const fa::FaKernelEntry* e = resolve_fwd(a->variant, a->dtype, a->D, &a->tile, &split, &code);
  if (e == nullptr) return code;
  if (a->B < 0 || a->H <= 0 || a->H_kv <= 0 || a->M < 0 || a->N < 0)
    return fail(FA_EINVAL, "invalid sizes B=%d H=%d H_kv=%d M=%d N=%d", a->B, a->H, a->H_kv, a->M, a->N);
  if (a->H % a->H_kv != 0)
    return fail(FA_EINVAL, "query heads H=%d must be a multiple of kv heads H_kv=%d", a->H, a->H_kv);
  if (a->B == 0 || a->M == 0) return ok();  // nothing to compute
  if (!a->q || !a->k || !a->v || !a->o) return fail(FA_EINVAL, "null q/k/v/o pointer");
  if (a->q_stride[3] != 1 || a->k_stride[3] != 1 || a->v_stride[3] != 1 || a->o_stride[3] != 1)
    return fail(FA_EINVAL, "head-dim stride must be 1 for q, k, v and o");
  if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->o))
    return fail(FA_EINVAL, "q, k, v and o must be 16-byte aligned");
  for (int i = 0; i < 3; ++i)
    if (a->q_stride[i] % 8 || a->k_stride[i] % 8 || a->v_stride[i] % 8 || a->o_stride[i] % 4)
      return fail(FA_EINVAL, "row strides must keep 16-byte alignment (q/k/v multiple of 8, o of 4 elements)");
  if (!std::isfinite(a->sm_scale) || a->sm_scale <= 0.f)
    return fail(FA_EINVAL, "sm_scale must be positive and finite, got %g", (double)a->sm_scale);

  if (e->stages >= 3 && !pipelined_fits(a, e->block_n)) {
    // The pipelined kernel addresses one (batch, kv-head) row range [0, N + block_n) of K and V
    // with 32-bit byte offsets and relies on whole rows for its tail check: run the
    // double-buffered kernel of the same rows per workgroup instead (same block_n where it is
    // built, else the 64-key tile: the D = 256 pipelined tile has 32 keys).
    const fa::FaKernelEntry* fb = double_buffered_fallback(e);
    if (fb == nullptr) return fail(FA_ENOTSUP, "no double-buffered fallback for the pipelined attention tile");
    e = fb;
  }
  const int bm = a->tile.block_m, bn = e->block_n;
  const int splits = a->tile.splits < 1 ? 1 : a->tile.splits;
  // Decode shapes: when every query row of a GQA group fits in one tile (non-causal), the group's
  // query heads share the tile's rows, so each workgroup reads its kv head's K/V once for all of
  // them instead of once per query head.
  const int group = a->H / a->H_kv;
  const int pack = fa_fwd_pack_group(a->H, a->H_kv, a->M, a->causal, bm, splits);
  if (e->stages == 9 && (pack > 1 || (int64_t)a->M * a->q_stride[2] * 2 > 0xffffffffLL || a->q_stride[2] < a->D)) {
    // The persistent kernel fetches Q rows of one (batch, head) by LDS-DMA (32-bit offsets, whole
    // rows) and does not pack query heads: the per-workgroup ping-pong kernel runs these launches.
    e = find_fwd(8, e->dtype, e->D, e->waves, e->rows_per_wave, e->block_n, e->split);
    if (e == nullptr) return fail(FA_ENOTSUP, "no stages=8 kernel behind the persistent attention tile");
  }
  const int64_t m_blocks = ((int64_t)a->M * pack + bm - 1) / bm;
  const int64_t n_tiles = a->N > 0 ? (a->N + bn - 1) / bn : 1;
  const int64_t tiles_per_split = (n_tiles + splits - 1) / splits;
  const int64_t total = m_blocks * a->B * (pack > 1 ? a->H_kv : a->H) * splits;
  if (total > 0x7fffffffLL) return fail(FA_EINVAL, "grid too large (%lld workgroups)", (long long)total);

  fa::FwdParams p;
  std::memset(&p, 0, sizeof(p));
  p.q = static_cast<const uint16_t*>(a->q);
  p.k = static_cast<const uint16_t*>(a->k);
  p.v = static_cast<const uint16_t*>(a->v);
  p.o = static_cast<uint16_t*>(a->o);
  p.lse = a->lse;
  p.sq0 = a->q_stride[0]; p.sq1 = a->q_stride[1]; p.sq2 = a->q_stride[2];
  p.sk0 = a->k_stride[0]; p.sk1 = a->k_stride[1]; p.sk2 = a->k_stride[2];
  p.sv0 = a->v_stride[0]; p.sv1 = a->v_stride[1]; p.sv2 = a->v_stride[2];
  p.so0 = a->o_stride[0]; p.so1 = a->o_stride[1]; p.so2 = a->o_stride[2];
  p.sl0 = a->lse_stride[0]; p.sl1 = a->lse_stride[1]; p.sl2 = a->lse_stride[2];
  p.B = a->B; p.H = a->H; p.Hkv = a->H_kv; p.M = a->M; p.N = a->N;
  p.group = group;
  p.pack = pack;
  p.sm_scale = a->sm_scale;
  p.c = a->sm_scale * 1.4426950408889634f;
  p.causal = a->causal ? 1 : 0;
  p.splits = splits;
  p.tiles_per_split = (int32_t)tiles_per_split;
  p.m_blocks = (int32_t)m_blocks;
  p.total_blocks = (int32_t)total;

  const fa::FaMergeEntry* me = nullptr;
  if (split) {
    me = find_merge(a->dtype, a->D);
    if (me == nullptr) return fail(FA_ENOTSUP, "no merge kernel for D=%d", a->D);
    const int64_t need = fa_fwd_workspace_bytes(a->B, a->H, a->M, a->D, splits);
    if (ws == nullptr || ws_bytes < need)
      return fail(FA_EWORKSPACE, "split-KV workspace of %lld bytes needed, got %lld", (long long)need,
                  (long long)ws_bytes);
    if (!aligned16(ws)) return fail(FA_EINVAL, "workspace must be 16-byte aligned");
    const int64_t rows = (int64_t)splits * a->B * a->H * a->M;
    p.ws_o = static_cast<float*>(ws);
    p.ws_lse = reinterpret_cast<float*>(static_cast<char*>(ws) + ((rows * a->D * 4 + 255) & ~(int64_t)255));
  }

  hipStream_t s = static_cast<hipStream_t>(stream);
  void* kargs[] = {&p};
  int64_t grid = total;
  if (e->stages == 9) {  // persistent: one workgroup per CU (fewer when there are fewer blocks)
    int cus = 0;
    const int code = current_device_cus(&cus);
    if (code != FA_OK) return code;
    if (grid > cus) grid = cus;
  }
  p.grid = (int32_t)grid;
  hipError_t err = hipLaunchKernel(e->fn, dim3((unsigned)grid), dim3(e->waves * 64), kargs, 0, s);
  if (err != hipSuccess) return fail(FA_EHIP, "attention launch failed: %s", hipGetErrorString(err));

  if (split) {
    fa::MergeParams mp;
    mp.ws_o = p.ws_o;
    mp.ws_lse = p.ws_lse;
    mp.o = p.o;
    mp.lse = a->lse;
    mp.so0 = p.so0; mp.so1 = p.so1; mp.so2 = p.so2;
    mp.sl0 = p.sl0; mp.sl1 = p.sl1; mp.sl2 = p.sl2;
    mp.B = a->B; mp.H = a->H; mp.M = a->M; mp.splits = splits;
    // up to 16 splits per wave: decode rows (few rows, many splits) get 2 or 4 waves each
    mp.waves_per_row = splits > 32 ? 4 : (splits > 16 ? 2 : 1);
    const int64_t rows = (int64_t)a->B * a->H * a->M;
    const int64_t rows_per_block = 4 / mp.waves_per_row;
    const int64_t blocks = (rows + rows_per_block - 1) / rows_per_block;
    if (blocks > 0x7fffffffLL) return fail(FA_EINVAL, "merge grid too large");
    void* margs[] = {&mp};
    err = hipLaunchKernel(me->fn, dim3((unsigned)blocks), dim3(256), margs, 0, s);
    if (err != hipSuccess) return fail(FA_EHIP, "merge launch failed: %s", hipGetErrorString(err));
  }
  return ok();
}

int fa_fwd(const fa_fwd_args* a, void* stream) {
  if (a == nullptr) return fail(FA_EINVAL, "null argument block");
  return launch_fwd(a, a->workspace, a->workspace_bytes, stream);
}

int fa_fwd_noalloc(const fa_fwd_args* a, void* stream) {
  if (a == nullptr) return fail(FA_EINVAL, "null argument block");
  if (a->workspace != nullptr || a->workspace_bytes != 0)
    return fail(FA_EINVAL, "fa_fwd_noalloc takes no workspace (workspace must be NULL, workspace_bytes 0)");
  const int splits = a->tile.splits < 1 ? 1 : a->tile.splits;
  if (a->variant != FA_VARIANT_SLICED || splits == 1) return launch_fwd(a, nullptr, 0, stream);
  const int64_t need = fa_fwd_workspace_bytes(a->B, a->H, a->M, a->D, splits);
  if (need > kScratchBytes)
    return fail(FA_EWORKSPACE,
                "fa_fwd_noalloc: split-KV partials of %lld bytes exceed its static scratch of %lld bytes "
                "(B=%d H=%d M=%d D=%d splits=%d); use fa_fwd with a workspace, or fewer splits",
                (long long)need, (long long)kScratchBytes, a->B, a->H, a->M, a->D, splits);
  void* ptr = nullptr;
  const int code = scratch_of_current_device(&ptr);
  if (code != FA_OK) return code;
  return launch_fwd(a, ptr, kScratchBytes, stream);
}

int gemm_f16_supported(const gemm_tile* tile) {
  if (tile == nullptr) return fail(FA_EINVAL, "null gemm tile");
  if (find_gemm(tile) == nullptr)
    return fail(FA_ENOTSUP, "gemm tile %dx%dx%d with %d waves is not built", tile->block_m, tile->block_n,
                tile->block_k, tile->waves);
  return ok();
}

int gemm_f16(const void* a, const void* b, void* c, int32_t M, int32_t N, int32_t K, int64_t lda, int64_t ldb,
             int64_t ldc, const gemm_tile* tile, void* stream) {
  if (tile == nullptr) return fail(FA_EINVAL, "null gemm tile");
  const fa::GemmKernelEntry* e = find_gemm(tile);
  if (e == nullptr)
    return fail(FA_ENOTSUP, "gemm tile %dx%dx%d with %d waves is not built", tile->block_m, tile->block_n,
                tile->block_k, tile->waves);
  if (M < 0 || N < 0 || K < 0) return fail(FA_EINVAL, "negative GEMM size");
  if (M == 0 || N == 0) return ok();
  if (K == 0) return fail(FA_EINVAL, "K=0 is not supported (the reference requires K %% 32 == 0, K > 0)");
  // Any M; N and K need only whole 8-byte output groups and 16-byte K chunks (the reference's
  // divisibility rule, mma.py:76-81, is kept by the drop-in selector, not here).
  if (K % 8 || N % 4)
    return fail(FA_EINVAL, "K=%d must be a multiple of 8 and N=%d a multiple of 4", K, N);
  if (!a || !b || !c) return fail(FA_EINVAL, "null GEMM pointer");
  if (!aligned16(a) || !aligned16(b) || (reinterpret_cast<uintptr_t>(c) & 7u))
    return fail(FA_EINVAL, "A and B must be 16-byte aligned, C 8-byte aligned");
  if (lda < K || ldb < N || ldc < N || lda % 8 || ldb % 8 || ldc % 4)
    return fail(FA_EINVAL, "leading dimensions lda=%lld ldb=%lld ldc=%lld invalid", (long long)lda,
                (long long)ldb, (long long)ldc);
  if (tile->group_m < 1) return fail(FA_EINVAL, "group_m must be >= 1");
  // The kernel addresses a tile's A rows and B columns (all of K) as raw buffers with 32-bit byte
  // offsets, and uses 2^31 as its out-of-range offset.
  if ((int64_t)e->block_m * lda * 2 > 0x7fffffffLL || ((int64_t)(K - 1) * ldb + N) * 2 > 0x7fffffffLL)
    return fail(FA_ENOTSUP, "GEMM operand spans beyond 2 GiB per tile (lda=%lld ldb=%lld K=%d)", (long long)lda,
                (long long)ldb, K);
  fa::GemmParams p;
  p.a = static_cast<const uint16_t*>(a);
  p.b = static_cast<const uint16_t*>(b);
  p.c = static_cast<uint16_t*>(c);
  p.M = M; p.N = N; p.K = K;
  p.lda = lda; p.ldb = ldb; p.ldc = ldc;
  p.group_m = tile->group_m;
  p.tiles_m = (M + e->block_m - 1) / e->block_m;
  p.tiles_n = (N + e->block_n - 1) / e->block_n;
  const int64_t total = (int64_t)p.tiles_m * p.tiles_n;
  if (total > 0x7fffffffLL) return fail(FA_EINVAL, "grid too large");
  p.region_m = gemm_region_rows(p.tiles_m, p.tiles_n, e->block_m, e->block_n);
  // Short K loops run the tile's shallow-ring kernel where one is built (more workgroups per CU),
  // or its persistent kernel (one workgroup per CU overlapping each tile's C write with the next
  // tile) when the shape is whole tiles and C takes 16-byte stores.
  const int slabs = (K + e->block_k - 1) / e->block_k;
  const void* fn = (e->fn_shallow && slabs <= fa::kGemmShallowMaxSlabs) ? e->fn_shallow : e->fn;
  unsigned grid = (unsigned)total, threads = (unsigned)e->waves * 64;
  if (e->fn_persist && M % e->block_m == 0 && N % e->block_n == 0 && K % e->block_k == 0 &&
      slabs >= fa::kGemmPersistMinSlabs && slabs <= fa::kGemmPersistMaxSlabs && total % 8 == 0 &&
      aligned16(c) && ldc % 8 == 0 && (int64_t)e->block_m * ldc * 2 <= 0x7fffffffLL) {
    int cus = 0;
    if (current_device_cus(&cus) == FA_OK && cus >= 8) {
      const int64_t g = (total < cus ? total : cus) / 8 * 8;  // whole XCD rows of workgroups
      fn = e->fn_persist;
      grid = (unsigned)g;
      threads = (unsigned)(e->waves + fa::kGemmPersistStoreWaves) * 64;
    }
  }
  p.grid = (int32_t)grid;
  void* kargs[] = {&p};
  hipError_t err = hipLaunchKernel(fn, dim3(grid), dim3(threads), kargs, 0, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(FA_EHIP, "gemm launch failed: %s", hipGetErrorString(err));
  return ok();
}

// The built kernel an (op, variant, dtype, D, tile) or GEMM tile resolves to: its function, mangled
// symbol and workgroup size (shared by fa_kernel_resources and fa_kernel_symbol).
static int resolve_kernel(int32_t op, int32_t variant, int32_t dtype, int32_t D, const fa_tile* tile,
                          const gemm_tile* gtile, const void** fn, const char** symbol, int* threads) {
  if (op == 0) {
    bool split = false;
    int code = FA_OK;
    const fa::FaKernelEntry* e = resolve_fwd(variant, dtype, D, tile, &split, &code);
    if (e == nullptr) return code;
    *fn = e->fn;
    *symbol = e->symbol;
    *threads = e->waves * 64;
  } else if (op == 1) {
    if (gtile == nullptr) return fail(FA_EINVAL, "null gemm tile");
    const fa::GemmKernelEntry* e = find_gemm(gtile);
    if (e == nullptr) return fail(FA_ENOTSUP, "gemm tile not built");
    *fn = e->fn;
    *symbol = e->symbol;
    *threads = e->waves * 64;
  } else {
    return fail(FA_EINVAL, "unknown op %d", op);
  }
  return FA_OK;
}

int fa_kernel_symbol(int32_t op, int32_t variant, int32_t dtype, int32_t D, const fa_tile* tile,
                     const gemm_tile* gtile, char* buf, int32_t buf_bytes) {
  if (buf == nullptr || buf_bytes <= 0) return fail(FA_EINVAL, "null or empty output buffer");
  const void* fn = nullptr;
  const char* symbol = nullptr;
  int threads = 0;
  const int code = resolve_kernel(op, variant, dtype, D, tile, gtile, &fn, &symbol, &threads);
  if (code != FA_OK) return code;
  const size_t n = std::strlen(symbol);
  if ((int64_t)n + 1 > (int64_t)buf_bytes)
    return fail(FA_EINVAL, "a %d-byte buffer cannot hold the %zu-byte symbol", buf_bytes, n + 1);
  std::memcpy(buf, symbol, n + 1);
  return ok();
}

int fa_kernel_resources(int32_t op, int32_t variant, int32_t dtype, int32_t D, const fa_tile* tile,
                        const gemm_tile* gtile, fa_resources* out) {
  if (out == nullptr) return fail(FA_EINVAL, "null output");
  const void* fn = nullptr;
  const char* symbol = nullptr;
  int threads = 0;
  const int code = resolve_kernel(op, variant, dtype, D, tile, gtile, &fn, &symbol, &threads);
  if (code != FA_OK) return code;
  const fa::KernelResourceRow* row = find_resource_row(symbol);
  if (row == nullptr) return fail(FA_ENOTSUP, "no compiler resource row for %s (stale build)", symbol);
  hipFuncAttributes attr;
  std::memset(&attr, 0, sizeof(attr));
  hipError_t err = hipFuncGetAttributes(&attr, fn);
  if (err != hipSuccess) return fail(FA_EHIP, "hipFuncGetAttributes failed: %s", hipGetErrorString(err));
  out->vgprs = row->vgprs;
  out->agprs = row->agprs;
  out->sgprs = row->sgprs;
  out->lds_bytes = (int32_t)attr.sharedSizeBytes;
  out->scratch_bytes = row->scratch_bytes;
  out->threads = threads;
  out->max_threads = attr.maxThreadsPerBlock;
  out->occupancy = row->occupancy;
  return ok();
}

int fa_device_limits(int32_t device, fa_device_limits_t* out) {
  if (out == nullptr) return fail(FA_EINVAL, "null output");
  hipDeviceProp_t prop;
  hipError_t err = hipGetDeviceProperties(&prop, device);
  if (err != hipSuccess) return fail(FA_EHIP, "hipGetDeviceProperties failed: %s", hipGetErrorString(err));
  out->lds_bytes_per_cu = (int32_t)prop.maxSharedMemoryPerMultiProcessor;
  out->registers_per_simd = 512 * 64;
  out->register_file_bytes_per_simd = 512 * 64 * 4;
  out->wavefront_size = prop.warpSize;
  out->max_threads_per_block = prop.maxThreadsPerBlock;
  out->cu_count = prop.multiProcessorCount;
  out->clock_khz = prop.clockRate;
  int arch = 0;
  if (std::sscanf(prop.gcnArchName, "gfx%d", &arch) != 1) arch = 0;
  out->gcn_arch = arch;
  return ok();
}

}  // extern "C"
