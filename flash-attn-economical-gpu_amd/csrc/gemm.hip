// fp16 GEMM C[M,N] = A[M,K] B[K,N] (row-major, fp32 accumulation, fp16 output) for gfx950.
//
// Replaces the reference's Triton `_matmul_contiguous_kernel` (mma.py:8-52): grouped tile order
// with GROUP_M rows of tiles per group (mma.py:22-30), fp32 accumulate over K (mma.py:39-49),
// fp16 store (mma.py:51-52), no masks (M, N, K multiples of the tile).
//
// gfx950 design: v_mfma_f32_32x32x16_f16 computes C^T = B^T A^T per 32x32 tile, so the
// accumulator gives every lane four consecutive output columns of one row (8-byte stores).
// A tiles are staged in LDS as [m][k]; B tiles are transposed on the way into LDS ([n][k]) with
// 4x8 register blocks (v_perm-style half-word shuffles), so both MFMA operands are one 16-byte LDS
// read per lane. The next K slab is prefetched from HBM into registers while the current one is
// multiplied, and the two LDS buffers alternate so one barrier per slab suffices. Workgroup ids
// are remapped so each XCD (own L2) walks a contiguous range of GROUP_M-grouped tiles.
#include "fa_common.h"
#include "fa_kernels.h"

namespace fa {

template <int BM, int BN, int BK, int WM, int WN>
struct GemmKernel {
  static constexpr int THREADS = WM * WN * 64;
  static constexpr int TM = BM / WM / 32;  // 32-row tiles per wave along M
  static constexpr int TN = BN / WN / 32;  // 32-col tiles per wave along N
  static constexpr int ASTR = BK + 8;      // LDS row stride (elements), +16 B pad
  static constexpr int BSTR = BK + 8;
  static constexpr int A_ELEMS = BM * ASTR;
  static constexpr int B_ELEMS = BN * BSTR;
  static constexpr int STAGE_ELEMS = A_ELEMS + B_ELEMS;
  static constexpr int A_CHUNKS = BM * BK / 8;  // 16-byte chunks of an A slab
  static constexpr int A_ITERS = (A_CHUNKS + THREADS - 1) / THREADS;
  static constexpr int B_QUADS = BK * BN / 32;  // 4(k) x 8(n) blocks of a B slab
  static constexpr int B_ITERS = (B_QUADS + THREADS - 1) / THREADS;
  static constexpr bool A_EVEN = A_CHUNKS % THREADS == 0;
  static constexpr bool B_EVEN = B_QUADS % THREADS == 0;
  static_assert(TM >= 1 && TN >= 1 && BK % 16 == 0, "tile shape");

  struct Prefetch {
    u32x4 a[A_ITERS];
    u32x4 b[B_ITERS][4];
  };

  __device__ static inline void load(Prefetch& pf, const uint16_t* a, const uint16_t* b, int64_t lda,
                                     int64_t ldb, int k0, int tid) {
#pragma unroll
    for (int i = 0; i < A_ITERS; ++i) {
      const int id = tid + i * THREADS;
      const int row = id / (BK / 8), c8 = id % (BK / 8);
      if (A_EVEN || id < A_CHUNKS) pf.a[i] = *reinterpret_cast<const u32x4*>(a + (int64_t)row * lda + k0 + c8 * 8);
    }
#pragma unroll
    for (int i = 0; i < B_ITERS; ++i) {
      const int id = tid + i * THREADS;
      const int kq = id / (BN / 8), n8 = id % (BN / 8);
      if (B_EVEN || id < B_QUADS) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          pf.b[i][r] = *reinterpret_cast<const u32x4*>(b + (int64_t)(k0 + kq * 4 + r) * ldb + n8 * 8);
      }
    }
  }

  __device__ static inline void store(const Prefetch& pf, uint16_t* as, uint16_t* bs, int tid) {
#pragma unroll
    for (int i = 0; i < A_ITERS; ++i) {
      const int id = tid + i * THREADS;
      const int row = id / (BK / 8), c8 = id % (BK / 8);
      if (A_EVEN || id < A_CHUNKS) *reinterpret_cast<u32x4*>(as + row * ASTR + c8 * 8) = pf.a[i];
    }
#pragma unroll
    for (int i = 0; i < B_ITERS; ++i) {
      const int id = tid + i * THREADS;
      const int kq = id / (BN / 8), n8 = id % (BN / 8);
      if (!(B_EVEN || id < B_QUADS)) continue;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int w = e >> 1;
        const int sh = (e & 1) * 16;
        const uint32_t a0 = (pf.b[i][0][w] >> sh) & 0xffffu, a1 = (pf.b[i][1][w] >> sh) & 0xffffu;
        const uint32_t a2 = (pf.b[i][2][w] >> sh) & 0xffffu, a3 = (pf.b[i][3][w] >> sh) & 0xffffu;
        u32x2 out = {a0 | (a1 << 16), a2 | (a3 << 16)};
        *reinterpret_cast<u32x2*>(bs + (n8 * 8 + e) * BSTR + kq * 4) = out;
      }
    }
  }

  __device__ static void run(const GemmParams& p) {
    __shared__ __attribute__((aligned(16))) uint16_t smem[2 * STAGE_ELEMS];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, col = lane & 31, hh = lane >> 5;
    const int wm = wave / WN, wn = wave % WN;

    const int total = p.tiles_m * p.tiles_n;
    const int pid = xcd_remap(blockIdx.x, total);
    const int in_group = p.group_m * p.tiles_n;
    const int group_id = pid / in_group;
    const int first_m = group_id * p.group_m;
    const int gsz = min(p.tiles_m - first_m, p.group_m);
    const int pid_m = first_m + (pid % in_group) % gsz;
    const int pid_n = (pid % in_group) / gsz;
    const int m0 = pid_m * BM, n0 = pid_n * BN;

    const uint16_t* a = p.a + (int64_t)m0 * p.lda;
    const uint16_t* b = p.b + n0;

    floatx16 acc[TN][TM];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[tn][tm][r] = 0.f;

    Prefetch pf;
    load(pf, a, b, p.lda, p.ldb, 0, tid);
    store(pf, smem, smem + A_ELEMS, tid);
    __syncthreads();

    const int ksteps = p.K / BK;
    for (int ks = 0; ks < ksteps; ++ks) {
      const uint16_t* as = smem + (ks & 1) * STAGE_ELEMS;
      const uint16_t* bs = as + A_ELEMS;
      if (ks + 1 < ksteps) load(pf, a, b, p.lda, p.ldb, (ks + 1) * BK, tid);
#pragma unroll
      for (int c = 0; c < BK / 16; ++c) {
        u32x4 af[TM], bf[TN];
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
          af[tm] = *reinterpret_cast<const u32x4*>(as + ((wm * TM + tm) * 32 + col) * ASTR + c * 16 + hh * 8);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
          bf[tn] = *reinterpret_cast<const u32x4*>(bs + ((wn * TN + tn) * 32 + col) * BSTR + c * 16 + hh * 8);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
          for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = DT<f16_t>::mfma32(bf[tn], af[tm], acc[tn][tm]);
      }
      if (ks + 1 < ksteps) {
        uint16_t* an = smem + ((ks + 1) & 1) * STAGE_ELEMS;
        store(pf, an, an + A_ELEMS, tid);
      }
      __syncthreads();
    }

    // C^T tile: lane holds row m = ...+col, columns n = 8*g + 4*hh + 0..3 of each 32-col tile.
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int m = m0 + (wm * TM + tm) * 32 + col;
      uint16_t* crow = p.c + (int64_t)m * p.ldc + n0;
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = (wn * TN + tn) * 32 + 8 * g + 4 * hh;
          u32x2 val = {DT<f16_t>::pack2(acc[tn][tm][4 * g], acc[tn][tm][4 * g + 1]),
                       DT<f16_t>::pack2(acc[tn][tm][4 * g + 2], acc[tn][tm][4 * g + 3])};
          *reinterpret_cast<u32x2*>(crow + n) = val;
        }
    }
  }
};

template <int BM, int BN, int BK, int WM, int WN>
__global__ __launch_bounds__(WM * WN * 64) void gemm_f16_kernel(GemmParams p) {
  GemmKernel<BM, BN, BK, WM, WN>::run(p);
}

#define GEMM_ENTRY(BM, BN, BK, WM, WN) \
  {BM, BN, BK, WM * WN, (const void*)&gemm_f16_kernel<BM, BN, BK, WM, WN>}

static const GemmKernelEntry kGemmEntries[] = {
    GEMM_ENTRY(256, 256, 64, 2, 2),
    GEMM_ENTRY(256, 256, 32, 2, 2),
    GEMM_ENTRY(128, 128, 64, 2, 2),
    GEMM_ENTRY(128, 256, 64, 2, 2),
    GEMM_ENTRY(256, 128, 64, 2, 2),
    GEMM_ENTRY(128, 128, 32, 2, 2),
    GEMM_ENTRY(128, 64, 32, 2, 2),
    GEMM_ENTRY(64, 256, 32, 2, 2),
};

const GemmKernelEntry* gemm_registry(int* count) {
  *count = (int)(sizeof(kGemmEntries) / sizeof(kGemmEntries[0]));
  return kGemmEntries;
}

}  // namespace fa
