// fp16 GEMM C[M,N] = A[M,K] B[K,N] (row-major, fp32 accumulation, fp16 output) for gfx950.
//
// Replaces the reference's Triton `_matmul_contiguous_kernel` (mma.py:8-52): grouped tile order
// with GROUP_M rows of tiles per group (mma.py:22-30), fp32 accumulate over K (mma.py:39-49),
// fp16 store (mma.py:51-52), no masks (M, N, K multiples of the tile).
//
// gfx950 design:
//  * v_mfma_f32_32x32x16_f16 computes C^T = B^T A^T per 32x32 tile, so the accumulator gives each
//    lane four consecutive output columns of one row (8-byte stores).
//  * A slabs are staged in LDS as [m][k] (16-byte skewed rows): the MFMA B operand (A^T columns) is
//    one ds_read_b128 per lane.
//  * B slabs are staged untransposed, [k][n] (64-byte skewed rows). The MFMA A operand (B^T rows,
//    8 consecutive k per lane) comes from two ds_read_b64_tr_b16 transposing reads: in each 16-lane
//    group, lane L addresses row k0 + (L >> 2) at columns n0 + 4 (L & 3), and result lane i then
//    holds B[k0 + c][n0 + i] for c = 0..3. No register shuffles.
//  * Each slab is loaded HBM -> registers while the previous one is multiplied; LDS is double
//    buffered with one barrier per slab; LDS fragment reads for the next 16-deep chunk are issued
//    while the current chunk's MFMAs run (scheduling-group hints).
//  * Workgroup ids are remapped so each XCD (own L2) walks a contiguous range of GROUP_M-grouped
//    tiles.
#include "fa_common.h"
#include "fa_kernels.h"

namespace fa {

typedef short g_s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) g_s16x4 g_lds_s16x4;

__device__ inline u32x2 gemm_lds_read_tr16(const uint16_t* p) {
  g_s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((g_lds_s16x4*)(p));
  return __builtin_bit_cast(u32x2, r);
}

template <int BM, int BN, int BK, int WM, int WN>
struct GemmKernel {
  static constexpr int THREADS = WM * WN * 64;
  static constexpr int TM = BM / WM / 32;  // 32-row tiles per wave along M
  static constexpr int TN = BN / WN / 32;  // 32-col tiles per wave along N
  static constexpr int ASTR = BK + 8;      // A LDS row stride (elements): 16-byte skew
  static constexpr int BSTR = BN + 32;     // B LDS row stride (elements): 64-byte skew
  static constexpr int A_ELEMS = BM * ASTR;
  static constexpr int B_ELEMS = BK * BSTR;
  static constexpr int STAGE_ELEMS = A_ELEMS + B_ELEMS;
  static constexpr int A_CPR = BK / 8;     // 16-byte chunks per A row
  static constexpr int B_CPR = BN / 8;     // 16-byte chunks per B row
  static constexpr int A_RSTEP = THREADS / A_CPR;
  static constexpr int B_RSTEP = THREADS / B_CPR;
  static constexpr int A_PASSES = (BM + A_RSTEP - 1) / A_RSTEP;
  static constexpr int B_PASSES = (BK + B_RSTEP - 1) / B_RSTEP;
  static constexpr int KCH = BK / 16;      // 16-deep MFMA chunks per slab
  static constexpr int READS = TM + 2 * TN;  // LDS reads per chunk
  static_assert(THREADS % A_CPR == 0 && THREADS % B_CPR == 0, "threads must cover whole rows");
  static_assert(TM >= 1 && TN >= 1 && BK % 16 == 0, "tile shape");

  struct Prefetch {
    u32x4 a[A_PASSES];
    u32x4 b[B_PASSES];
  };

  struct Ctx {
    const uint16_t* ap;        // this thread's A chunk (row a_r0, column a_c8) of slab 0
    const uint16_t* bp;        // this thread's B chunk (row b_r0, column b_c8) of slab 0
    int64_t a_rstep, b_rstep;  // pointer step between passes
    int64_t b_slab;            // pointer step between slabs for B (BK rows)
    int a_r0, a_c8, b_r0, b_c8;
  };

  __device__ static inline void load(Prefetch& pf, const Ctx& cx, int ks) {
    const uint16_t* a = cx.ap + ks * BK;
    const uint16_t* b = cx.bp + ks * cx.b_slab;
#pragma unroll
    for (int i = 0; i < A_PASSES; ++i)
      if (BM % A_RSTEP == 0 || cx.a_r0 + i * A_RSTEP < BM)
        pf.a[i] = *reinterpret_cast<const u32x4*>(a + i * cx.a_rstep);
#pragma unroll
    for (int i = 0; i < B_PASSES; ++i)
      if (BK % B_RSTEP == 0 || cx.b_r0 + i * B_RSTEP < BK)
        pf.b[i] = *reinterpret_cast<const u32x4*>(b + i * cx.b_rstep);
  }

  __device__ static inline void store(const Prefetch& pf, uint16_t* as, uint16_t* bs, const Ctx& cx) {
#pragma unroll
    for (int i = 0; i < A_PASSES; ++i) {
      const int row = cx.a_r0 + i * A_RSTEP;
      if (BM % A_RSTEP == 0 || row < BM) *reinterpret_cast<u32x4*>(as + row * ASTR + cx.a_c8 * 8) = pf.a[i];
    }
#pragma unroll
    for (int i = 0; i < B_PASSES; ++i) {
      const int row = cx.b_r0 + i * B_RSTEP;
      if (BK % B_RSTEP == 0 || row < BK) *reinterpret_cast<u32x4*>(bs + row * BSTR + cx.b_c8 * 8) = pf.b[i];
    }
  }

  __device__ static inline void compute(floatx16 (&acc)[TN][TM], const uint16_t* as, const uint16_t* bs,
                                        int a_off, int b_off) {
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      u32x4 af[TM], bf[TN];
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        af[tm] = *reinterpret_cast<const u32x4*>(as + a_off + tm * 32 * ASTR + c * 16);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const uint16_t* base = bs + b_off + c * 16 * BSTR + tn * 32;
        const u32x2 lo = gemm_lds_read_tr16(base);
        const u32x2 hi = gemm_lds_read_tr16(base + 4 * BSTR);
        bf[tn] = (u32x4){lo[0], lo[1], hi[0], hi[1]};
      }
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = DT<f16_t>::mfma32(bf[tn], af[tm], acc[tn][tm]);
    }
    // The reads of chunk c+1 are issued while chunk c's MFMAs run.
    __builtin_amdgcn_sched_group_barrier(0x100, READS, 0);
#pragma unroll
    for (int i = 0; i < KCH * TM * TN; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, (READS + TM * TN - 1) / (TM * TN), 0);
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

    Ctx cx;
    cx.a_r0 = tid / A_CPR;
    cx.a_c8 = tid % A_CPR;
    cx.b_r0 = tid / B_CPR;
    cx.b_c8 = tid % B_CPR;
    cx.ap = p.a + (int64_t)(m0 + cx.a_r0) * p.lda + cx.a_c8 * 8;
    cx.bp = p.b + (int64_t)cx.b_r0 * p.ldb + n0 + cx.b_c8 * 8;
    cx.a_rstep = (int64_t)A_RSTEP * p.lda;
    cx.b_rstep = (int64_t)B_RSTEP * p.ldb;
    cx.b_slab = (int64_t)BK * p.ldb;

    // Per-lane LDS fragment offsets.
    const int a_off = ((wm * TM) * 32 + col) * ASTR + hh * 8;
    const int g = lane & 15;
    const int b_off = (8 * hh + (g >> 2)) * BSTR + wn * TN * 32 + 16 * ((lane >> 4) & 1) + 4 * (g & 3);

    floatx16 acc[TN][TM];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[tn][tm][r] = 0.f;

    Prefetch pf;
    load(pf, cx, 0);
    store(pf, smem, smem + A_ELEMS, cx);
    __syncthreads();

    const int ksteps = p.K / BK;
    for (int ks = 0; ks < ksteps; ++ks) {
      const uint16_t* as = smem + (ks & 1) * STAGE_ELEMS;
      if (ks + 1 < ksteps) load(pf, cx, ks + 1);
      compute(acc, as, as + A_ELEMS, a_off, b_off);
      if (ks + 1 < ksteps) {
        uint16_t* an = smem + ((ks + 1) & 1) * STAGE_ELEMS;
        store(pf, an, an + A_ELEMS, cx);
      }
      __syncthreads();
    }

    // C^T tile: lane holds row m = ...+col, columns n = 8*gq + 4*hh + 0..3 of each 32-col tile.
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int m = m0 + (wm * TM + tm) * 32 + col;
      uint16_t* crow = p.c + (int64_t)m * p.ldc + n0;
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int n = (wn * TN + tn) * 32 + 8 * gq + 4 * hh;
          u32x2 val = {DT<f16_t>::pack2(acc[tn][tm][4 * gq], acc[tn][tm][4 * gq + 1]),
                       DT<f16_t>::pack2(acc[tn][tm][4 * gq + 2], acc[tn][tm][4 * gq + 3])};
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
    GEMM_ENTRY(256, 256, 64, 2, 4),
    GEMM_ENTRY(256, 256, 32, 2, 4),
    GEMM_ENTRY(256, 128, 64, 2, 4),
    GEMM_ENTRY(128, 256, 64, 2, 4),
    GEMM_ENTRY(256, 256, 64, 2, 2),
    GEMM_ENTRY(128, 128, 64, 2, 2),
    GEMM_ENTRY(128, 128, 32, 2, 2),
    GEMM_ENTRY(128, 64, 32, 2, 2),
    GEMM_ENTRY(64, 256, 32, 2, 2),
};

const GemmKernelEntry* gemm_registry(int* count) {
  *count = (int)(sizeof(kGemmEntries) / sizeof(kGemmEntries[0]));
  return kGemmEntries;
}

}  // namespace fa
