// fp16 GEMM C[M,N] = A[M,K] B[K,N] (row-major, fp32 accumulation, fp16 output) for gfx950.
//
// Replaces the reference's Triton `_matmul_contiguous_kernel` (mma.py:8-52): grouped tile order
// with GROUP_M rows of tiles per group (mma.py:22-30), fp32 accumulate over K (mma.py:39-49),
// fp16 store (mma.py:51-52). The reference needs M, N, K to be multiples of the tile; here partial
// tiles are masked (loads past M, N or K read zeros, stores outside [M, N) are skipped), so any M
// with K % 8 == 0 and N % 4 == 0 runs.
//
// gfx950 design:
//  * v_mfma_f32_32x32x16_f16 computes C^T = B^T A^T per 32x32 tile, so the accumulator gives each
//    lane four consecutive output columns of one row (8-byte stores).
//  * K slabs (BK deep) reach LDS by LDS-DMA (buffer_load_dwordx4 ... lds), no staging registers,
//    into a ring of RING slabs: slab s is requested RING-1 slabs before it is multiplied, and the
//    barrier ending a slab waits only for the next slab's loads (vmcnt), not for the newer ones.
//  * LDS slabs keep HBM's row-major order, so one DMA instruction (1 KiB, 16 bytes per lane) reads
//    whole rows: 1024 / (2 BK) rows of A or 1024 / (2 BN) rows of B. Reads are made conflict-free by
//    XOR-swizzling the 16-byte chunks of each row (the DMA lane that fills slot s fetches logical
//    chunk s ^ f(row); a lane reading logical chunk c looks at slot c ^ f(row)):
//      A (row pitch 2 BK = 64 or 128 bytes): f(r) = (r / rows-per-256-bytes) & (chunks - 1), so the
//        16 rows one ds_read_b128 cycle touches land on 16 distinct 16-byte bank groups;
//      B (row pitch 2 BN >= 128 bytes): f(k) = 4 ((k / rows-per-256-bytes) & (QB - 1)), so the 4 rows
//        x 64 bytes of a ds_read_b64_tr_b16 cycle land on distinct bank groups.
//    Per lane the swizzled addresses reduce to a few registers (one per 16-deep chunk for A, one per
//    32-column tile for B) plus immediate offsets.
//  * The MFMA B operand (A^T columns) is one ds_read_b128 per lane; the MFMA A operand (B^T rows, 8
//    consecutive k per lane) comes from two transposing reads ds_read_b64_tr_b16 of B kept as [k][n]:
//    in each 16-lane group, lane L addresses row k0 + (L >> 2) at columns n0 + 4 (L & 3), and result
//    lane i then holds B[k0 + e][n0 + i] for e = 0..3. No register shuffles.
//  * LDS fragment reads for the next 16-deep chunk are issued while the current chunk's MFMAs run
//    (scheduling-group hints).
//  * Each XCD (own L2) walks one rectangle of the tile grid in GROUP_M-grouped order (the split with
//    the smallest A + B panel footprint, chosen by the host), or, when the grid does not split into
//    8 equal rectangles, a contiguous range of the flat grouped order.
#include "fa_common.h"
#include "fa_kernels.h"

namespace fa {

typedef short g_s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) g_s16x4 g_lds_s16x4;

__device__ inline u32x2 gemm_lds_read_tr16(const char* p) {
  g_s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((g_lds_s16x4*)(p));
  return __builtin_bit_cast(u32x2, r);
}

template <int BM, int BN, int BK, int WM, int WN, bool SHALLOW = false>
struct GemmKernel {
  static constexpr int WAVES = WM * WN;
  static constexpr int TM = BM / WM / 32;  // 32-row tiles per wave along M
  static constexpr int TN = BN / WN / 32;  // 32-col tiles per wave along N
  static constexpr int KCH = BK / 16;      // 16-deep MFMA chunks per slab
  static constexpr int AP = BK * 2;        // A row pitch in LDS (bytes)
  static constexpr int BP = BN * 2;        // B row pitch in LDS (bytes)
  static constexpr int SA = BK / 8;        // 16-byte chunks per A row
  static constexpr int RA = 256 / AP;      // A rows per 256-byte bank line
  static constexpr int SB = BN / 8;        // 16-byte chunks per B row
  static constexpr int RB = BP >= 256 ? 1 : 256 / BP;  // B rows per 256-byte bank line
  static constexpr int QB = SB / 4 < 4 ? SB / 4 : 4;   // distinct 64-byte XOR offsets for B rows
  static constexpr int A_BYTES = BM * AP;
  static constexpr int B_BYTES = BK * BP;
  static constexpr int SLAB_BYTES = A_BYTES + B_BYTES;
  // Slabs resident in LDS: as many as fit in 128 KiB, 2..4. The SHALLOW variant keeps the fewest
  // that still hold the staged C tile (at least 2): less LDS per workgroup, so more workgroups
  // share a CU, which pays when K is only a few slabs deep (their latency is then the cost).
  static constexpr int RING_FIT = 131072 / SLAB_BYTES;
  static constexpr int RING_DEEP = RING_FIT > 4 ? 4 : (RING_FIT < 2 ? 2 : RING_FIT);
  static constexpr int RING_C = (BM * BN * 2 + SLAB_BYTES - 1) / SLAB_BYTES;
  static constexpr int RING = SHALLOW ? (RING_C > 2 ? RING_C : 2) : RING_DEEP;
  static constexpr int A_PER_WAVE = A_BYTES / 1024 / WAVES;  // DMA instructions per wave per slab
  static constexpr int B_PER_WAVE = B_BYTES / 1024 / WAVES;
  static constexpr int DMA_PER_SLAB = A_PER_WAVE + B_PER_WAVE;
  static constexpr int READS = TM + 2 * TN;  // LDS reads per chunk
  static_assert(TM >= 1 && TN >= 1 && BK % 16 == 0, "tile shape");
  static_assert(AP == 64 || AP == 128, "A swizzle assumes 64- or 128-byte rows");
  static_assert(BP >= 128 && QB >= 2, "B swizzle assumes rows of at least 128 bytes");
  static_assert(A_BYTES % (1024 * WAVES) == 0 && B_BYTES % (1024 * WAVES) == 0, "slab must split evenly");
  static_assert(RING * SLAB_BYTES <= 160 * 1024, "LDS");
  static constexpr int CP = BN * 2;                      // C tile row pitch in LDS (bytes)
  static constexpr int CHS = CP / 16 < 16 ? CP / 16 : 16;  // swizzled 16-byte chunks per C row
  static_assert(BM * CP <= RING * SLAB_BYTES, "the C tile is staged in the slab ring");

  __device__ static inline void compute(floatx16 (&acc)[TN][TM], const char* slab, const uint32_t (&aaddr)[KCH],
                                        const uint32_t (&baddr)[TN], int wm) {
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      u32x4 af[TM], bf[TN];
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        af[tm] = *reinterpret_cast<const u32x4*>(slab + aaddr[c] + (wm * TM + tm) * 32 * AP);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const char* base = slab + A_BYTES + baddr[tn] + c * 16 * BP;
        const u32x2 lo = gemm_lds_read_tr16(base);
        const u32x2 hi = gemm_lds_read_tr16(base + 4 * BP);
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
    __shared__ __attribute__((aligned(16))) char smem[RING * SLAB_BYTES];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, hh = lane >> 5;
    const int wm = wave / WN, wn = wave % WN;

    int pid_m, pid_n;
    if (p.region_m > 0) {
      // XCD x (workgroups are dispatched round-robin: blockIdx % 8) owns one rectangle of tiles,
      // region (x / rn, x % rn) of a region_m x rn split, and walks it in GROUP_M-grouped order:
      // each XCD's L2 then sees tiles_m / region_m A panels and tiles_n / rn B panels instead of
      // every B panel.
      constexpr int kXcds = 8;
      const int rn = kXcds / p.region_m;
      const int xcd = blockIdx.x % kXcds, slot = blockIdx.x / kXcds;
      const int rt_m = p.tiles_m / p.region_m, rt_n = p.tiles_n / rn;
      const int in_group = p.group_m * rt_n;
      const int first_m = (slot / in_group) * p.group_m;
      const int gsz = min(rt_m - first_m, p.group_m);
      pid_m = (xcd / rn) * rt_m + first_m + (slot % in_group) % gsz;
      pid_n = (xcd % rn) * rt_n + (slot % in_group) / gsz;
    } else {
      const int total = p.tiles_m * p.tiles_n;
      const int pid = xcd_remap(blockIdx.x, total);
      const int in_group = p.group_m * p.tiles_n;
      const int first_m = (pid / in_group) * p.group_m;
      const int gsz = min(p.tiles_m - first_m, p.group_m);
      pid_m = first_m + (pid % in_group) % gsz;
      pid_n = (pid % in_group) / gsz;
    }
    const int m0 = pid_m * BM, n0 = pid_n * BN;

    // Buffer resources over this tile's A rows [m0, min(m0 + BM, M)) and B columns [n0, n0 + BN)
    // of rows [0, K) (byte spans below 2^31: the host checks). Loads past the ranges return zeros:
    // rows of A past M and rows of B past K need no branch. Columns of B past N read neighbouring
    // data of the same rows (finite) and only reach output columns that are not stored.
    const int m_rows = min(BM, p.M - m0);
    const u32x4 ars = make_rsrc(p.a + (int64_t)m0 * p.lda, (uint32_t)((int64_t)m_rows * p.lda * 2));
    const u32x4 brs = make_rsrc(p.b + n0, (uint32_t)(((int64_t)(p.K - 1) * p.ldb + (p.N - n0)) * 2));

    // DMA: the lane filling slab byte `byte` of its block fetches the logical chunk stored there.
    uint32_t aoffs[A_PER_WAVE], boffs[B_PER_WAVE];
    int ak0[A_PER_WAVE];  // first k of the A chunk this lane moves (within a slab)
#pragma unroll
    for (int j = 0; j < A_PER_WAVE; ++j) {
      const int byte = (wave * A_PER_WAVE + j) * 1024 + lane * 16;
      const int r = byte / AP, s = (byte % AP) / 16;
      const int c = s ^ ((r / RA) & (SA - 1));
      aoffs[j] = ((uint32_t)r * (uint32_t)p.lda + c * 8) * 2u;
      ak0[j] = c * 8;
    }
#pragma unroll
    for (int j = 0; j < B_PER_WAVE; ++j) {
      const int byte = (wave * B_PER_WAVE + j) * 1024 + lane * 16;
      const int k = byte / BP, s = (byte % BP) / 16;
      const int c = s ^ (4 * ((k / RB) & (QB - 1)));
      boffs[j] = ((uint32_t)k * (uint32_t)p.ldb + c * 8) * 2u;
    }

    // Read addresses within a slab. A: lane reads row `col` of each 32-row tile at logical chunk
    // 2c + hh, i.e. slot (2c + hh) ^ x = (2c) ^ (hh ^ x) with x = (col / RA) & (SA - 1): the
    // address is (col*AP + 16 (hh ^ x)) ^ 32 c; the tile's 32*AP row offset does not change x.
    // B: lane L reads row k = 8 (L >> 5) + ((L & 15) >> 2) (+16 per chunk, +4 for the second read,
    // neither of which changes k's swizzle term w) at logical chunk 4 jt + sb, byte 8 (L & 1) of it;
    // slot = 4 (jt ^ w) + sb.
    uint32_t aaddr[KCH], baddr[TN];
    {
      const int x = (col / RA) & (SA - 1);
#pragma unroll
      for (int c = 0; c < KCH; ++c) aaddr[c] = (uint32_t)((col * AP + 16 * (hh ^ x)) ^ (32 * c));
      const int kr = 8 * (lane >> 5) + ((lane & 15) >> 2);
      const int sb = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
      const int w = (kr / RB) & (QB - 1);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const int jt = wn * TN + tn;
        baddr[tn] = (uint32_t)(kr * BP + 64 * (jt ^ w) + 16 * sb + 8 * (lane & 1));
      }
    }

    const uint32_t a_slab_bytes = (uint32_t)BK * 2u;                    // next K slab of A
    const uint32_t b_slab_bytes = (uint32_t)BK * (uint32_t)p.ldb * 2u;  // next K slab of B
    const int ksteps = (p.K + BK - 1) / BK;
    const bool k_ragged = (p.K % BK) != 0;  // last slab runs past K: A chunks there read zeros
    const uint32_t smem_lds = lds_address(smem);
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);  // scalar DMA destinations
    auto issue = [&](int ks) {
      if (ks >= ksteps) return;
      const uint32_t slot = smem_lds + (uint32_t)(ks % RING) * SLAB_BYTES;
      const bool tail = k_ragged && ks == ksteps - 1;
#pragma unroll
      for (int j = 0; j < A_PER_WAVE; ++j) {
        // past-K chunks of the ragged slab get an offset beyond the range (zeros): A's rows may hold
        // anything there, and 0 * NaN would reach valid outputs. 2^31 is past every range (the host
        // keeps spans below 2 GiB) and far from 32-bit wrap-around.
        const uint32_t off = (tail && ks * BK + ak0[j] >= p.K) ? 0x80000000u : aoffs[j] + (uint32_t)ks * a_slab_bytes;
        buffer_load16_to_lds(ars, off, slot + (wave_u * A_PER_WAVE + j) * 1024);
      }
#pragma unroll
      for (int j = 0; j < B_PER_WAVE; ++j)
        buffer_load16_to_lds(brs, boffs[j] + (uint32_t)ks * b_slab_bytes,
                             slot + A_BYTES + (wave_u * B_PER_WAVE + j) * 1024);
    };

    floatx16 acc[TN][TM];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[tn][tm][r] = 0.f;

#pragma unroll
    for (int s = 0; s + 1 < RING; ++s) issue(s);
    wait_vm_lds_barrier<0>();

    for (int ks = 0; ks < ksteps; ++ks) {
      issue(ks + RING - 1);  // into the slot slab ks-1 left (read in step ks-1)
      compute(acc, smem + (ks % RING) * SLAB_BYTES, aaddr, baddr, wm);
      // Step ks+1 reads slab ks+1; the RING-2 newer slabs may stay in flight.
      if (RING > 2 && ks + RING - 1 < ksteps)
        wait_vm_lds_barrier<(RING > 2 ? (RING - 2) * DMA_PER_SLAB : 0)>();
      else
        wait_vm_lds_barrier<0>();
    }

    // C goes out through LDS (the ring is free after the last step's barrier): each lane holds 4
    // consecutive columns of one row per 32x32 tile (C^T layout), which as direct 8-byte stores
    // left C lines written in pieces; staged in LDS, each lane stores 16 contiguous bytes and 8
    // lanes a full 128-byte line. LDS rows are XOR-swizzled in 16-byte chunks
    // (chunk ^ (row & (CHS - 1))), so the 32 rows one write instruction touches spread over the banks.
    char* ctile = smem;
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int r = (wm * TM + tm) * 32 + col;
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int cb = ((wn * TN + tn) * 32 + 8 * gq + 4 * hh) * 2;  // byte column in the tile row
          const int phys = r * CP + ((((cb >> 4) ^ (r & (CHS - 1)))) << 4) + (cb & 15);
          *reinterpret_cast<u32x2*>(ctile + phys) =
              (u32x2){DT<f16_t>::pack2(acc[tn][tm][4 * gq], acc[tn][tm][4 * gq + 1]),
                      DT<f16_t>::pack2(acc[tn][tm][4 * gq + 2], acc[tn][tm][4 * gq + 3])};
        }
    }
    __syncthreads();
    // 16-byte global stores need C and its row stride 16-byte aligned (the ABI guarantees 8).
    const bool c16 = ((reinterpret_cast<uintptr_t>(p.c) & 15) == 0) && ((p.ldc & 7) == 0);
    constexpr int CHUNKS = BM * CP / 16;  // 16-byte chunks of the C tile
    static_assert(CHUNKS % (WAVES * 64) == 0, "C tile chunks split evenly over the threads");
#pragma unroll 4
    for (int i = tid; i < CHUNKS; i += WAVES * 64) {
      const int r = i / (CP / 16), c = i % (CP / 16);
      const int m = m0 + r, n = n0 + c * 8;
      if (m >= p.M || n >= p.N) continue;
      const u32x4 v = *reinterpret_cast<const u32x4*>(ctile + r * CP + ((c ^ (r & (CHS - 1))) << 4));
      uint16_t* dst = p.c + (int64_t)m * p.ldc + n;
      if (c16 && n + 8 <= p.N) {
        *reinterpret_cast<u32x4*>(dst) = v;
      } else {
        // N % 4 == 0: the chunk's first 4 columns are in range, its last 4 only when n + 8 <= N
        *reinterpret_cast<u32x2*>(dst) = (u32x2){v[0], v[1]};
        if (n + 8 <= p.N) *reinterpret_cast<u32x2*>(dst + 4) = (u32x2){v[2], v[3]};
      }
    }
  }
};

template <int BM, int BN, int BK, int WM, int WN>
__global__ __launch_bounds__(WM * WN * 64) void gemm_f16_kernel(GemmParams p) {
  GemmKernel<BM, BN, BK, WM, WN>::run(p);
}

template <int BM, int BN, int BK, int WM, int WN>
__global__ __launch_bounds__(WM * WN * 64) void gemm_f16_shallow_kernel(GemmParams p) {
  GemmKernel<BM, BN, BK, WM, WN, true>::run(p);
}

// The shallow-ring kernel of a tile, or nullptr when its ring would be as deep as the default one.
template <int BM, int BN, int BK, int WM, int WN>
const void* gemm_shallow_fn() {
  if constexpr (GemmKernel<BM, BN, BK, WM, WN, true>::RING < GemmKernel<BM, BN, BK, WM, WN>::RING)
    return (const void*)&gemm_f16_shallow_kernel<BM, BN, BK, WM, WN>;
  else
    return nullptr;
}

#define GEMM_ENTRY(BM, BN, BK, WM, WN)                                                  \
  {BM, BN, BK, WM * WN, (const void*)&gemm_f16_kernel<BM, BN, BK, WM, WN>,             \
   gemm_shallow_fn<BM, BN, BK, WM, WN>(),                                               \
   "_ZN2fa15gemm_f16_kernelILi" #BM "ELi" #BN "ELi" #BK "ELi" #WM "ELi" #WN "EEEvNS_10GemmParamsE"}

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
