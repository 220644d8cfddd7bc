// fp16 GEMM C[M,N] = A[M,K] B[K,N] (row-major, fp32 accumulation, fp16 output) for gfx950.
//
// Replaces the reference's Triton `_matmul_contiguous_kernel` (mma.py:8-52): grouped tile order
// with GROUP_M rows of tiles per group (mma.py:22-30), fp32 accumulate over K (mma.py:39-49),
// fp16 store (mma.py:51-52). The reference needs M, N, K to be multiples of the tile; here partial
// tiles are masked (loads past M, N or K read zeros, stores outside [M, N) are skipped), so any M
// with K % 8 == 0 and N % 4 == 0 runs.
//
// gfx950 design:
//  * C^T = B^T A^T per MFMA tile, so the accumulator gives each lane four consecutive output
//    columns of one row (8-byte stores). Two MFMA shapes, chosen per tile in the registry:
//    v_mfma_f32_32x32x16_f16 and v_mfma_f32_16x16x32_f16. The 16x16x32 form moves half the
//    accumulator registers per flop; on MI355X it draws less power per flop, so the power-capped
//    8-wave tiles run at a higher clock with it (about 1.8 instead of 1.5-1.6 GHz at the same MFMA
//    occupancy, measured with GRBM_GUI_ACTIVE / SQ_VALU_MFMA_BUSY_CYCLES).
//  * K slabs (BK deep) reach LDS by LDS-DMA (buffer_load_dwordx4 ... lds), no staging registers,
//    into a ring of RING slabs: slab s is requested RING-1 slabs before it is multiplied, and the
//    barrier ending a slab waits only for the next slab's loads (vmcnt), not for the newer ones.
//  * LDS slabs keep HBM's row-major order, so one DMA instruction (1 KiB, 16 bytes per lane) reads
//    whole rows: 1024 / (2 BK) rows of A or 1024 / (2 BN) rows of B. Reads are made conflict-free by
//    XOR-swizzling the 16-byte chunks of each row (the DMA lane that fills slot s fetches logical
//    chunk s ^ f(row); a lane reading logical chunk c looks at slot c ^ f(row)):
//      A (row pitch 2 BK = 64 or 128 bytes): f(r) = (r / rows-per-256-bytes) & (chunks - 1);
//      B, 32x32 layout (row pitch 2 BN >= 128 bytes): f(k) = 4 ((k / rows-per-256-bytes) & (QB - 1)),
//        so the 4 rows x 64 bytes of a ds_read_b64_tr_b16 half-wave land on distinct bank groups;
//      B, 16x16 layout (row pitch >= 256 bytes): 32-byte chunks XORed with
//        h(k) = (k & 3) | ((k >> 3) & 1) << 2, so the 8 rows x 32 bytes of a half-wave do.
//    Measured with the LDS bank-conflict counters: every combination in use is conflict-free except
//    A with 64-byte rows in the 16x16 layout (BK = 32), which conflicts on a sixth of its cycles; the
//    16x16 tiles that matter use BK = 64.
//  * The MFMA B operand (A^T columns, 8 consecutive k per lane) is one ds_read_b128 per lane; the
//    MFMA A operand (B^T rows) comes from two transposing reads ds_read_b64_tr_b16 of B kept as
//    [k][n]: in each 16-lane group, lane L addresses row k0 + (L >> 2) at columns n0 + 4 (L & 3),
//    and result lane i then holds B[k0 + e][n0 + i] for e = 0..3. No register shuffles.
//  * Two schedules (SCHED). 0: one fragment buffer per chunk, the compiler interleaving the next
//    chunk's reads with the current MFMAs (scheduling-group hints). 1: fragments double-buffered in
//    registers across chunks and slabs; in a slab's last chunk the barrier comes first, then the
//    refill of the slot just freed is spread one LDS-DMA instruction per group of MFMAs (a burst of
//    DMA issue would leave the MFMA pipe idle with one or two waves per SIMD) together with the next
//    slab's first reads. The DMA is branch-free (past the last slab it reads zeros), so every slab
//    takes the same step and no tail code keeps fragments live into the epilogue.
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

template <int MI>
struct GemmAcc {
  typedef floatx16 type;  // v_mfma_f32_32x32x16_f16: 16 accumulators per lane
};
template <>
struct GemmAcc<16> {
  typedef floatx4 type;  // v_mfma_f32_16x16x32_f16: 4 accumulators per lane
};

// MI: MFMA shape (32: v_mfma_f32_32x32x16_f16, 16: v_mfma_f32_16x16x32_f16). SCHED: 0 = one fragment
// buffer per chunk, scheduled by the compiler; 1 = fragments double-buffered across chunks and
// slabs, LDS-DMA spread over the last chunk's MFMAs. KSG: K groups -- the workgroup holds KSG groups
// of WM x WN waves, group g multiplying its own contiguous run of the K slabs through its own LDS
// ring; the partial sums of groups 1.. are added into group 0's through LDS before the epilogue
// (a short serial K loop and more waves per CU for shapes with few tiles).
template <int BM, int BN, int BK, int WM, int WN, bool SHALLOW, int MI, int SCHED, int KSG = 1>
struct GemmKernel {
  static constexpr int WAVES = WM * WN;  // waves of one K group
  static constexpr int KD = MI == 32 ? 16 : 32;  // k depth of one MFMA
  static constexpr int TM = BM / WM / MI;        // MI-row tiles per wave along M
  static constexpr int TN = BN / WN / MI;        // MI-col tiles per wave along N
  static constexpr int KCH = BK / KD;            // MFMA-deep chunks per slab
  typedef typename GemmAcc<MI>::type Acc;
  // Accumulators of the wave's TN x TM MFMA tiles. 16x16 tiles are stored four to a floatx16 (tile
  // tm in elements 4 (tm % 4) .. 4 (tm % 4) + 3 of vector tm / 4), so the register allocator works
  // with 16-register tuples as for the 32x32 tiles.
  static constexpr int AG = (MI == 16 && TM % 4 == 0) ? 4 : 1;
  struct AccTiles {
    floatx16 v[TN][AG == 4 ? TM / 4 : (MI == 32 ? TM : 1)];
    Acc t[TN][AG == 4 || MI == 32 ? 1 : TM];
  };
  __device__ __attribute__((always_inline)) static inline void mma(AccTiles& acc, int tn, int tm, const u32x4& b,
                                                                   const u32x4& a) {
    if constexpr (MI == 32) {
      acc.v[tn][tm] = DT<f16_t>::mfma32(b, a, acc.v[tn][tm]);
    } else if constexpr (AG == 4) {
      floatx16& g = acc.v[tn][tm / 4];
      const int q = 4 * (tm % 4);
      floatx4 c = {g[q], g[q + 1], g[q + 2], g[q + 3]};
      c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, b), __builtin_bit_cast(half8, a), c, 0, 0, 0);
      g[q] = c[0];
      g[q + 1] = c[1];
      g[q + 2] = c[2];
      g[q + 3] = c[3];
    } else {
      acc.t[tn][tm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, b), __builtin_bit_cast(half8, a),
                                                             acc.t[tn][tm], 0, 0, 0);
    }
  }
  __device__ __attribute__((always_inline)) static inline float acc_at(const AccTiles& acc, int tn, int tm, int r) {
    if constexpr (MI == 32)
      return acc.v[tn][tm][r];
    else if constexpr (AG == 4)
      return acc.v[tn][tm / 4][4 * (tm % 4) + r];
    else
      return acc.t[tn][tm][r];
  }
  static constexpr int ACC = MI == 32 ? 16 : 4;
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
  // Slabs resident in LDS: as many as fit in 128 KiB, 2..4 (with K groups, as many as fit in each
  // group's share of 160 KiB). The SHALLOW variant keeps the fewest
  // that still hold the staged C tile (at least 2): less LDS per workgroup, so more workgroups
  // share a CU, which pays when K is only a few slabs deep (their latency is then the cost).
  static constexpr int RING_FIT = KSG == 1 ? 131072 / SLAB_BYTES : 163840 / KSG / SLAB_BYTES;
  static constexpr int RING_DEEP = RING_FIT > 4 ? 4 : (RING_FIT < 2 ? 2 : RING_FIT);
  static constexpr int RING_C = (BM * BN * 2 + SLAB_BYTES - 1) / SLAB_BYTES;
  static constexpr int RING = SHALLOW ? (RING_C > 2 ? RING_C : 2) : RING_DEEP;
  static constexpr int A_PER_WAVE = A_BYTES / 1024 / WAVES;  // DMA instructions per wave per slab
  static constexpr int B_PER_WAVE = B_BYTES / 1024 / WAVES;
  static constexpr int DMA_PER_SLAB = A_PER_WAVE + B_PER_WAVE;
  static constexpr int READS = TM + 2 * TN;  // LDS reads per chunk
  static constexpr bool kPipe = SCHED == 1;
  static_assert(MI == 32 || MI == 16, "MFMA shape");
  static_assert(SCHED == 0 || SCHED == 1, "schedule");
  static_assert(TM >= 1 && TN >= 1 && BK % KD == 0, "tile shape");
  static_assert(MI == 32 || BP >= 256, "16x16 B swizzle assumes rows of at least 256 bytes");
  static_assert(AP == 64 || AP == 128, "A swizzle assumes 64- or 128-byte rows");
  static_assert(BP >= 128 && QB >= 2, "B swizzle assumes rows of at least 128 bytes");
  static_assert(A_BYTES % (1024 * WAVES) == 0 && B_BYTES % (1024 * WAVES) == 0, "slab must split evenly");
  static_assert(RING * SLAB_BYTES <= 160 * 1024, "LDS");
  static constexpr int CP = BN * 2;                      // C tile row pitch in LDS (bytes)
  static constexpr int CHS = CP / 16 < 16 ? CP / 16 : 16;  // swizzled 16-byte chunks per C row
  static_assert(KSG > 1 || BM * CP <= RING * SLAB_BYTES, "the C tile is staged in the slab ring");
  // K groups: after the K loop the LDS holds the staged C tile and, behind it, the partial sums of
  // groups 1 .. KSG-1 (each wave's accumulators as NQ lane-major 16-byte pieces).
  static constexpr int NV = AG == 4 ? TM / 4 : (MI == 32 ? TM : 1);  // floatx16 tuples per B block
  static constexpr int NQ = TN * ((MI == 32 || AG == 4) ? NV * 4 : TM);  // accumulator float4s per lane
  static constexpr int CT_BYTES = BM * CP;
  static constexpr int PART_BYTES = (KSG - 1) * WAVES * NQ * 1024;
  static constexpr int RING_BYTES = KSG * RING * SLAB_BYTES;
  static constexpr int SMEM_BYTES = RING_BYTES > CT_BYTES + PART_BYTES ? RING_BYTES : CT_BYTES + PART_BYTES;
  static_assert(KSG == 1 || (kPipe && !SHALLOW), "K groups: the pipelined per-tile kernel only");
  static_assert(KSG >= 1 && SMEM_BYTES <= 160 * 1024, "LDS");
  static_assert(NQ == TM * TN * MI * MI / 256, "accumulator pieces cover the wave's tile");

  // The accumulators as NQ pieces of 4 consecutive floats: f(q, tuple, offset) for piece q, which is
  // elements offset .. offset + 3 of `tuple` (a floatx16 or floatx4 register tuple, by reference).
  template <class F>
  __device__ __attribute__((always_inline)) static inline void acc_quads(AccTiles& acc, F&& f) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      if constexpr (MI == 32 || AG == 4) {
#pragma unroll
        for (int i = 0; i < NV; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) f((tn * NV + i) * 4 + r, acc.v[tn][i], 4 * r);
      } else {
#pragma unroll
        for (int i = 0; i < TM; ++i) f(tn * TM + i, acc.t[tn][i], 0);
      }
    }
  }

  // Fragments of one KD-deep chunk: TM A^T column blocks (ds_read_b128) and TN B^T row blocks (two
  // transposing reads each).
  struct Frag {
    u32x4 a[TM];
    u32x4 b[TN];
  };

  template <int C>
  __device__ __attribute__((always_inline)) static inline void read_frag(Frag& f, const char* slab, const uint32_t (&aaddr)[KCH],
                                          const uint32_t (&baddr)[TN], int wm) {
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
      f.a[tm] = *reinterpret_cast<const u32x4*>(slab + aaddr[C] + (wm * TM + tm) * MI * AP);
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const char* base = slab + A_BYTES + baddr[tn] + C * KD * BP;
      const u32x2 lo = gemm_lds_read_tr16(base);
      const u32x2 hi = gemm_lds_read_tr16(base + 4 * BP);
      f.b[tn] = (u32x4){lo[0], lo[1], hi[0], hi[1]};
    }
  }

  __device__ __attribute__((always_inline)) static inline void mfma_frag(AccTiles& acc, const Frag& f) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) mma(acc, tn, tm, f.b[tn], f.a[tm]);
  }



  // Read R of a chunk's fragments (0..TM-1: A blocks; then B block (R - TM) / 2, low or high half).
  template <int C, int R>
  __device__ __attribute__((always_inline)) static inline void read_one(Frag& f, const char* slab, const uint32_t (&aaddr)[KCH],
                                         const uint32_t (&baddr)[TN], int wm) {
    if constexpr (R < TM) {
      f.a[R] = *reinterpret_cast<const u32x4*>(slab + aaddr[C] + (wm * TM + R) * MI * AP);
    } else {
      constexpr int tn = (R - TM) / 2, hi = (R - TM) & 1;
      const u32x2 v = gemm_lds_read_tr16(slab + A_BYTES + baddr[tn] + C * KD * BP + hi * 4 * BP);
      f.b[tn][2 * hi] = v[0];
      f.b[tn][2 * hi + 1] = v[1];
    }
  }

  template <int C, int R0, int R1>
  __device__ __attribute__((always_inline)) static inline void read_range(Frag& f, const char* slab, const uint32_t (&aaddr)[KCH],
                                           const uint32_t (&baddr)[TN], int wm) {
    if constexpr (R0 < R1) {
      read_one<C, R0>(f, slab, aaddr, baddr, wm);
      read_range<C, R0 + 1, R1>(f, slab, aaddr, baddr, wm);
    }
  }

  // MFMAs M0..M1-1 of a chunk (MFMA m: B block m / TM, A block m % TM).
  template <int M0, int M1>
  __device__ __attribute__((always_inline)) static inline void mfma_range(AccTiles& acc, const Frag& f) {
    if constexpr (M0 < M1) {
      mma(acc, M0 / TM, M0 % TM, f.b[M0 / TM], f.a[M0 % TM]);
      mfma_range<M0 + 1, M1>(acc, f);
    }
  }


  // NM MFMAs, each followed by its share of NR LDS reads.
  template <int NM, int NR, int I = 0, int LEFT = NR>
  __device__ __attribute__((always_inline)) static inline void interleave_n() {
    constexpr int kPer = NM > 0 ? (NR + NM - 1) / NM : 0;
    if constexpr (I < NM) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      constexpr int kReads = LEFT < kPer ? LEFT : kPer;
      if constexpr (kReads > 0) __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);
      interleave_n<NM, NR, I + 1, LEFT - kReads>();
    }
  }

  // The last chunk of a slab with a successor, in DMA_PER_SLAB groups: group G issues LDS-DMA
  // instruction G of slab ks + RING (into the slot every wave finished at the barrier), its share of
  // the next slab's first-chunk reads and its share of this chunk's MFMAs, so the DMA issue is
  // spread over the MFMA stream instead of stalling it in one burst.
  template <int G, class Dma>
  __device__ __attribute__((always_inline)) static inline void last_chunk_groups(
      AccTiles& acc, const Frag& cur, Frag& nxt, const char* next, const uint32_t (&aaddr)[KCH],
      const uint32_t (&baddr)[TN], int wm, Dma& dma) {
    constexpr int NG = DMA_PER_SLAB, MF = TM * TN;
    if constexpr (G < NG) {
      constexpr int R0 = G * READS / NG, R1 = (G + 1) * READS / NG;
      constexpr int M0 = G * MF / NG, M1 = (G + 1) * MF / NG;
      dma(std::integral_constant<int, G>{});
      read_range<0, R0, R1>(nxt, next, aaddr, baddr, wm);
      mfma_range<M0, M1>(acc, cur);
      interleave_n<M1 - M0, R1 - R0>();
      __builtin_amdgcn_sched_barrier(0);
      last_chunk_groups<G + 1>(acc, cur, nxt, next, aaddr, baddr, wm, dma);
    }
  }

  // Chunks C.. of a slab with one fragment buffer per chunk (the compiler allocates and schedules
  // them): the reads of chunk c+1 are issued while chunk c's MFMAs run.
  template <int C = 0>
  __device__ static inline void compute(AccTiles& acc, const char* slab, const uint32_t (&aaddr)[KCH],
                                        const uint32_t (&baddr)[TN], int wm) {
    if constexpr (C < KCH) {
      Frag f;
      read_frag<C>(f, slab, aaddr, baddr, wm);
      mfma_frag(acc, f);
      compute<C + 1>(acc, slab, aaddr, baddr, wm);
    } else {
      __builtin_amdgcn_sched_group_barrier(0x100, READS, 0);
#pragma unroll
      for (int i = 0; i < KCH * TM * TN; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, (READS + TM * TN - 1) / (TM * TN), 0);
      }
    }
  }

  // Chunk C of a slab in the double-buffered loop; the slab's chunk 0 uses fragment buffer BUF0
  // and chunk C buffer (BUF0 + C) & 1. Before a slab's last chunk `wait` synchronises the workgroup
  // and returns the next slab, `dma(J)` issues LDS-DMA instruction J of the slab that refills the
  // ring, and the next slab's first chunk is read into the buffer that follows.
  template <int BUF0, int C, class Wait, class Dma>
  __device__ __attribute__((always_inline)) static inline void chunk_step(
      AccTiles& acc, Frag (&f)[2], const char* slab, const uint32_t (&aaddr)[KCH], const uint32_t (&baddr)[TN],
      int wm, Wait& wait, Dma& dma) {
    constexpr int kCur = (BUF0 + C) & 1, kNext = (BUF0 + C + 1) & 1;
    if constexpr (C + 1 < KCH) {
      read_frag<C + 1>(f[kNext], slab, aaddr, baddr, wm);
      mfma_frag(acc, f[kCur]);
      interleave_n<TM * TN, READS>();
      __builtin_amdgcn_sched_barrier(0);
      chunk_step<BUF0, C + 1>(acc, f, slab, aaddr, baddr, wm, wait, dma);
    } else {
      const char* next = wait();
      last_chunk_groups<0>(acc, f[kCur], f[kNext], next, aaddr, baddr, wm, dma);
    }
  }

  template <int J, class Dma>
  __device__ __attribute__((always_inline)) static inline void dma_all(Dma& dma) {
    if constexpr (J < DMA_PER_SLAB) {
      dma(std::integral_constant<int, J>{});
      dma_all<J + 1>(dma);
    }
  }

  __device__ static void run(const GemmParams& p) {
    __shared__ __attribute__((aligned(16))) char smem[SMEM_BYTES];
    const int tid = (int)__builtin_amdgcn_workitem_id_x();
    const int lane = tid & 63;
    // K group kg of the workgroup, wave wl of it (without K groups: 0 and the wave)
    const int kg = KSG == 1 ? 0 : __builtin_amdgcn_readfirstlane((tid >> 6) / WAVES);
    const int wave = KSG == 1 ? tid >> 6 : (tid >> 6) % WAVES;
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
      const int xcd = (int)__builtin_amdgcn_workgroup_id_x() % kXcds, slot = (int)__builtin_amdgcn_workgroup_id_x() / kXcds;
      const int rt_m = p.tiles_m / p.region_m, rt_n = p.tiles_n / rn;
      const int in_group = p.group_m * rt_n;
      const int first_m = (slot / in_group) * p.group_m;
      const int gsz = min(rt_m - first_m, p.group_m);
      pid_m = (xcd / rn) * rt_m + first_m + (slot % in_group) % gsz;
      pid_n = (xcd % rn) * rt_n + (slot % in_group) / gsz;
    } else {
      const int total = p.tiles_m * p.tiles_n;
      const int pid = xcd_remap((int)__builtin_amdgcn_workgroup_id_x(), total);
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
      const int c = MI == 32 ? s ^ (4 * ((k / RB) & (QB - 1))) : s ^ (2 * ((k & 3) | (((k >> 3) & 1) << 2)));
      boffs[j] = ((uint32_t)k * (uint32_t)p.ldb + c * 8) * 2u;
    }

    // Read addresses within a slab. A: lane reads row `col` of each 32-row tile at logical chunk
    // 2c + hh, i.e. slot (2c + hh) ^ x = (2c) ^ (hh ^ x) with x = (col / RA) & (SA - 1): the
    // address is (col*AP + 16 (hh ^ x)) ^ 32 c; the tile's 32*AP row offset does not change x.
    // B: lane L reads row k = 8 (L >> 5) + ((L & 15) >> 2) (+16 per chunk, +4 for the second read,
    // neither of which changes k's swizzle term w) at logical chunk 4 jt + sb, byte 8 (L & 1) of it;
    // slot = 4 (jt ^ w) + sb.
    uint32_t aaddr[KCH], baddr[TN];
    if constexpr (MI == 16) {
      // A: lane reads row r16 = lane & 15 of each 16-row tile at logical chunk 4c + g (g = lane >> 4),
      // slot (4c + g) ^ x = 4c ^ (g ^ x), x = (r16 / RA) & (SA - 1): address (r16*AP + 16 (g ^ x)) ^ 64 c.
      // B: lane reads row k = 8 g + (r16 >> 2) (+32 per chunk, +4 for the second read) at byte
      // 8 (r16 & 3) of logical 32-byte chunk jt (16-column tile), stored at 32-byte slot jt ^ h with
      // h = (k & 3) | ((k >> 3) & 1) << 2 = (r16 >> 2) | (g & 1) << 2: the 8 rows one half-wave reads
      // land on the 8 distinct 32-byte bank groups of a 256-byte line.
      const int r16 = lane & 15, g = lane >> 4;
      const int x = (r16 / RA) & (SA - 1);
#pragma unroll
      for (int c = 0; c < KCH; ++c) aaddr[c] = (uint32_t)((r16 * AP + 16 * (g ^ x)) ^ (64 * c));
      const int kr = 8 * g + (r16 >> 2);
      const int h = (r16 >> 2) | ((g & 1) << 2);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const int jt = wn * TN + tn;
        baddr[tn] = (uint32_t)(kr * BP + 32 * (jt ^ h) + 8 * (r16 & 3));
      }
    } else {
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
    // DMA instruction j (A blocks first, then B blocks) of slab ks; nothing past the last slab.
    auto issue_one = [&](int ks, int j) {
      if (ks >= ksteps) return;
      const uint32_t slot = smem_lds + (uint32_t)(ks % RING) * SLAB_BYTES;
      if (j < A_PER_WAVE) {
        // past-K chunks of the ragged slab get an offset beyond the range (zeros): A's rows may hold
        // anything there, and 0 * NaN would reach valid outputs. 2^31 is past every range (the host
        // keeps spans below 2 GiB) and far from 32-bit wrap-around.
        const bool tail = k_ragged && ks == ksteps - 1;
        const uint32_t off = (tail && ks * BK + ak0[j] >= p.K) ? 0x80000000u : aoffs[j] + (uint32_t)ks * a_slab_bytes;
        buffer_load16_to_lds(ars, off, slot + (wave_u * A_PER_WAVE + j) * 1024);
      } else {
        const int jb = j - A_PER_WAVE;
        buffer_load16_to_lds(brs, boffs[jb] + (uint32_t)ks * b_slab_bytes,
                             slot + A_BYTES + (wave_u * B_PER_WAVE + jb) * 1024);
      }
    };
    auto issue = [&](int ks) {
#pragma unroll
      for (int j = 0; j < DMA_PER_SLAB; ++j) issue_one(ks, j);
    };

    AccTiles acc;
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
#pragma unroll
      for (int i = 0; i < (int)(sizeof(acc.v[0]) / sizeof(floatx16)); ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc.v[tn][i][r] = 0.f;
#pragma unroll
      for (int i = 0; i < (int)(sizeof(acc.t[0]) / sizeof(Acc)); ++i)
#pragma unroll
        for (int r = 0; r < ACC; ++r) acc.t[tn][i][r] = 0.f;
    }

    if constexpr (kPipe) {
      // Fragments double-buffered in registers across chunks and slabs: chunk c's MFMAs run while
      // chunk c+1's fragments are read; in a slab's last chunk the barrier comes first (slab ks+1
      // landed, every wave done reading slab ks), then the DMA into slab ks's slot and the reads of
      // slab ks+1's first chunk, interleaved with the last chunk's MFMAs.
      // DMA instruction J of slab ks, branch-free: past the last slab it reads an offset beyond the
      // range, so the slot holds zeros, and exactly RING - 2 slabs are always in flight behind the
      // one a barrier waits for.
      // K group kg multiplies slabs kbase .. kbase + per - 1 (its step ks is slab kbase + ks) in its
      // own ring; all groups take the same steps and barriers, a group's steps past its run or past
      // K multiplying zeros.
      const int per = KSG == 1 ? ksteps : (ksteps + KSG - 1) / KSG;
      const int kbase = kg * per;
      const uint32_t ring_lds = smem_lds + (uint32_t)(kg * RING * SLAB_BYTES);
      const char* const ring = smem + kg * RING * SLAB_BYTES;
      auto dma_slab = [&](int ks, auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
        const uint32_t slot = ring_lds + (uint32_t)(ks % RING) * SLAB_BYTES;
        const int gk = kbase + ks;
        const bool live = (ks < per) & (gk < ksteps);
        // 16x16 tiles: the slab's offset moves the buffer resource (base + offset, range - offset,
        // range 0 past the last slab), so each lane's offset is the same on every step and the
        // DMA takes no vector op; a lane reads zeros exactly where it did with the offset added to
        // its own. Only the last slab of a K that is not a multiple of BK checks its columns per
        // lane, in a uniform branch, with an offset of 2^31, past every range (operand spans stay
        // below 2 GiB: the host checks). The 4-wave 32x32 tiles, at 256 VGPRs, add the slab
        // offset (2^31 past the last slab) to the lane's and keep one select per lane for A.
        if constexpr (j < A_PER_WAVE && MI == 16) {
          uint32_t off = aoffs[j];
          if (__builtin_expect(k_ragged && gk == ksteps - 1, 0)) {
            if (gk * BK + ak0[j] >= p.K) off = 0x80000000u;
          }
          buffer_load16_to_lds(slab_rsrc(ars, (uint32_t)gk * a_slab_bytes, live), off,
                               slot + (wave_u * A_PER_WAVE + j) * 1024);
        } else if constexpr (j < A_PER_WAVE) {
          // bitwise, not short-circuit: the scalar and per-lane parts stay one select
          const bool zero = !live | (k_ragged & (gk == ksteps - 1) & (gk * BK + ak0[j] >= p.K));
          const uint32_t off = zero ? 0x80000000u : aoffs[j] + (uint32_t)gk * a_slab_bytes;
          buffer_load16_to_lds(ars, off, slot + (wave_u * A_PER_WAVE + j) * 1024);
        } else if constexpr (MI == 16) {
          constexpr int jb = j - A_PER_WAVE;
          buffer_load16_to_lds(slab_rsrc(brs, (uint32_t)gk * b_slab_bytes, live), boffs[jb],
                               slot + A_BYTES + (wave_u * B_PER_WAVE + jb) * 1024);
        } else {
          constexpr int jb = j - A_PER_WAVE;
          const uint32_t off = boffs[jb] + (live ? (uint32_t)gk * b_slab_bytes : 0x80000000u);
          buffer_load16_to_lds(brs, off, slot + A_BYTES + (wave_u * B_PER_WAVE + jb) * 1024);
        }
      };
      // Prologue: slabs 0 .. RING-1 (zeros past the last one: the loop below may multiply one slab
      // past it); slab 0 must have landed in every wave's part before its first reads.
#pragma unroll
      for (int s0 = 0; s0 < RING; ++s0) {
        auto d = [&](auto jc) __attribute__((always_inline)) { dma_slab(s0, jc); };
        dma_all<0>(d);
      }
      wait_vm_lds_barrier<(RING - 1) * DMA_PER_SLAB>();
      Frag f[2];
      read_frag<0>(f[0], ring, aaddr, baddr, wm);
      // Every slab takes the same step (barrier, refill, next slab's first reads): the last one
      // reads a slab that is never multiplied. Slab ks's chunk 0 uses buffer (ks * KCH) & 1, so with an
      // odd chunk count slabs go in pairs and an odd slab count gets one more slab, which the
      // branch-free DMA fills with zeros (its products add exactly 0). No tail code: the epilogue
      // starts with only the accumulators live.
      auto slab_step = [&](int ks, auto par_c) __attribute__((always_inline)) {
        const char* slab = ring + (ks % RING) * SLAB_BYTES;
        // Slab ks+1 must have landed; the RING - 2 slabs after it stay in flight.
        auto wait = [&]() __attribute__((always_inline)) {
          wait_vm_lds_barrier<(RING - 2) * DMA_PER_SLAB>();
          __builtin_amdgcn_sched_barrier(0);
          return ring + ((ks + 1) % RING) * SLAB_BYTES;
        };
        // Slab ks + RING goes into slab ks's slot: every wave passed the barrier.
        auto dma = [&](auto jc) __attribute__((always_inline)) { dma_slab(ks + RING, jc); };
        chunk_step<(decltype(par_c)::value * KCH) & 1, 0>(acc, f, slab, aaddr, baddr, wm, wait, dma);
      };
      if constexpr (KCH % 2 == 0) {
        for (int ks = 0; ks < per; ++ks) slab_step(ks, std::integral_constant<int, 0>{});
      } else {
        for (int ks = 0; ks < per; ks += 2) {
          slab_step(ks, std::integral_constant<int, 0>{});
          slab_step(ks + 1, std::integral_constant<int, 1>{});
        }
      }
      wait_vm_lds_barrier<0>();  // every wave done with the ring before it holds the C tile
    } else {
#pragma unroll
      for (int s0 = 0; s0 + 1 < RING; ++s0) issue(s0);
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
    }

    if constexpr (KSG > 1) {
      // Partial sums of groups 1 .. KSG-1 into group 0's accumulators, through LDS behind the C
      // staging area (the ring is free: every wave passed the last step's barrier with its DMA and
      // LDS reads done). Each wave's piece q sits at q * 1 KiB + lane * 16 of its own block, so
      // every write and read instruction covers 1 KiB contiguously.
      char* const part = smem + CT_BYTES;
      if (kg > 0) {
        char* const mine = part + ((kg - 1) * WAVES + wave) * NQ * 1024 + lane * 16;
        acc_quads(acc, [&](int q, auto& t, int o) __attribute__((always_inline)) {
          *reinterpret_cast<floatx4*>(mine + q * 1024) = (floatx4){t[o], t[o + 1], t[o + 2], t[o + 3]};
        });
      }
      __syncthreads();
      if (kg == 0) {
#pragma unroll
        for (int g = 1; g < KSG; ++g) {
          const char* const src = part + ((g - 1) * WAVES + wave) * NQ * 1024 + lane * 16;
          acc_quads(acc, [&](int q, auto& t, int o) __attribute__((always_inline)) {
            const floatx4 x = *reinterpret_cast<const floatx4*>(src + q * 1024);
            t[o] += x[0];
            t[o + 1] += x[1];
            t[o + 2] += x[2];
            t[o + 3] += x[3];
          });
        }
      }
    }

    // C goes out through LDS (the ring is free after the last step's barrier): each lane holds 4
    // consecutive columns of one row per 32x32 tile (C^T layout), which as direct 8-byte stores
    // left C lines written in pieces; staged in LDS, each lane stores 16 contiguous bytes and 8
    // lanes a full 128-byte line. LDS rows are XOR-swizzled in 16-byte chunks
    // (chunk ^ (row & (CHS - 1))), so the 32 rows one write instruction touches spread over the banks.
    // With K groups, group 0 (holding the sums) stages the tile and every wave stores it.
    char* ctile = smem;
    if (KSG == 1 || kg == 0) {
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) {
        // 32x32: lane holds row col, columns 8 gq + 4 hh + 0..3; 16x16: row lane & 15, columns
        // 4 (lane >> 4) + 0..3.
        const int r = (wm * TM + tm) * MI + (MI == 32 ? col : (lane & 15));
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
          for (int gq = 0; gq < ACC / 4; ++gq) {
            const int cb = MI == 32 ? ((wn * TN + tn) * 32 + 8 * gq + 4 * hh) * 2   // byte column in the tile row
                                    : ((wn * TN + tn) * 16 + 4 * (lane >> 4)) * 2;
            const int phys = r * CP + ((((cb >> 4) ^ (r & (CHS - 1)))) << 4) + (cb & 15);
            *reinterpret_cast<u32x2*>(ctile + phys) =
                (u32x2){DT<f16_t>::pack2(acc_at(acc, tn, tm, 4 * gq), acc_at(acc, tn, tm, 4 * gq + 1)),
                        DT<f16_t>::pack2(acc_at(acc, tn, tm, 4 * gq + 2), acc_at(acc, tn, tm, 4 * gq + 3))};
          }
      }
    }
    __syncthreads();
    // 16-byte global stores need C and its row stride 16-byte aligned (the ABI guarantees 8).
    const bool c16 = ((reinterpret_cast<uintptr_t>(p.c) & 15) == 0) && ((p.ldc & 7) == 0);
    constexpr int CHUNKS = BM * CP / 16;  // 16-byte chunks of the C tile
    static_assert(CHUNKS % (WAVES * KSG * 64) == 0, "C tile chunks split evenly over the threads");
#pragma unroll 4
    for (int i = tid; i < CHUNKS; i += WAVES * KSG * 64) {
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

  // ---- persistent short-K kernel ----------------------------------------------------------------
  // With a short K loop a tile's C write takes as long as its MFMAs, and a workgroup per tile
  // issues the two in turn. Here one workgroup per CU walks its tiles (XCD x = w % 8 takes a
  // contiguous range of the grouped tile order, its workgroups striding through it) in one
  // continuous slab loop: the DMA for slabs past a tile's last fetches the next tile's first slabs,
  // and the next tile's first chunk is read during the last chunk's MFMAs. A finished tile's C
  // goes to LDS, and kGemmPersistStoreWaves more waves of the workgroup (one per SIMD) copy it to
  // HBM during the next tile's first kStoreSteps slab steps. The store waves issue no loads and
  // wait for nothing but the workgroup barriers, and the compute waves issue no stores, so their
  // waits (vmcnt retires in order, loads and stores alike) see only their own slab DMA: C's write
  // overlaps the next tile's loads and MFMAs instead of following them. (Stores issued by the
  // compute waves after a step's DMA stalled the wait two steps later.)
  // Shapes: whole tiles (M % BM, N % BN, K % BK zero), kGemmPersistMinSlabs.. K slabs, a grid that
  // is a multiple of 8 and a tile count that is too (the host checks).
  static constexpr int kStoreWaves = kGemmPersistStoreWaves;
  // C rows leave after the barriers of slab steps 0 .. kStoreSteps - 1 of the next tile, so at
  // least one barrier (step kStoreSteps <= ksteps - 1) separates the store waves' last LDS reads
  // from the compute waves' next write of the tile after its last step. Three steps rather than
  // two: the smoother write stream measured 5-9% faster at 8192x8192x256 and x512.
  static constexpr int kStoreSteps = 3;
  static_assert(kStoreSteps + 1 <= kGemmPersistMinSlabs, "a barrier between the last C read and the next C write");
  static constexpr int kHeldLds = BM * BN * 2;      // the C tile, row-major, 16-byte chunks swizzled
  static constexpr int kRowChunks = BN / 8;         // 16-byte chunks per C row
  static constexpr int kRowsPerStore = 64 / kRowChunks;  // rows one store-wave instruction writes
  static constexpr int kWaveRows = BM / kStoreWaves;  // C rows per store wave
  // rows per store wave per step (whole store instructions; the last step takes what is left)
  static constexpr int kStoreRows = ((kWaveRows + kStoreSteps - 1) / kStoreSteps + kRowsPerStore - 1) / kRowsPerStore * kRowsPerStore;

  // Byte offset of 16-byte chunk c of row r in the LDS C tile: chunks XORed with the row's low bits,
  // so the 16 rows one compute-wave write touches, and the row one store-wave read touches, spread
  // over all banks.
  __device__ static inline int c_lds_off(int r, int c) { return r * (BN * 2) + ((c ^ (r & (kRowChunks - 1))) << 4); }

  // The compute wave's C values, rounded, into the LDS tile. MFMA tile tn gives lane row g (lanes
  // 16 g .. 16 g + 15) columns 4 g .. 4 g + 3; one v_permlane16_swap per dword of tiles 2 pp and
  // 2 pp + 1 (it swaps the odd 16-lane rows of one operand with the even rows of the other) leaves
  // lane row g holding columns 32 pp + 8 ((g & 1) << 1 | g >> 1) .. +7 of the pair: 16 bytes per
  // lane. Cross-lane: all lanes active.
  __device__ static inline void c_to_lds(const AccTiles& acc, char* ctile, int wm, int wn, int lane) {
    const int r16 = lane & 15, g = lane >> 4;
    const int cw = 8 * (((g & 1) << 1) | (g >> 1));
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int pp = 0; pp < TN / 2; ++pp) {
        const auto lo = __builtin_amdgcn_permlane16_swap(
            DT<f16_t>::pack2(acc_at(acc, 2 * pp, tm, 0), acc_at(acc, 2 * pp, tm, 1)),
            DT<f16_t>::pack2(acc_at(acc, 2 * pp + 1, tm, 0), acc_at(acc, 2 * pp + 1, tm, 1)), false, false);
        const auto hi = __builtin_amdgcn_permlane16_swap(
            DT<f16_t>::pack2(acc_at(acc, 2 * pp, tm, 2), acc_at(acc, 2 * pp, tm, 3)),
            DT<f16_t>::pack2(acc_at(acc, 2 * pp + 1, tm, 2), acc_at(acc, 2 * pp + 1, tm, 3)), false, false);
        const int r = (wm * TM + tm) * MI + r16;
        const int col = wn * (BN / WN) + 32 * pp + cw;
        *reinterpret_cast<u32x4*>(ctile + c_lds_off(r, col / 8)) = (u32x4){lo[0], hi[0], lo[1], hi[1]};
      }
  }
  // Rows r0 .. r0 + nrows - 1 (a multiple of kRowsPerStore) of the LDS C tile to C (`rsrc` over the
  // tile's rows): each instruction writes kRowsPerStore whole tile rows, 16 bytes per lane.
  __device__ static inline void c_rows_out(const char* ctile, const u32x4& rsrc, uint32_t ldc, int r0, int lane, int nrows) {
    const int rr = lane / kRowChunks, c = lane % kRowChunks;
#pragma unroll 2
    for (int q = 0; q < nrows / kRowsPerStore; ++q) {
      const int r = r0 + q * kRowsPerStore + rr;
      const u32x4 v = *reinterpret_cast<const u32x4*>(ctile + c_lds_off(r, c));
      const uint32_t off = ((uint32_t)r * ldc + (uint32_t)(c * 8)) * 2u;
      // The s_nop covers the gfx9 hazard of a VALU write to the data VGPRs of a just-issued store of
      // more than 8 bytes (one wait state), which the compiler does not see through inline asm.
      // Non-temporal: C is written once and never read here, so its lines should not displace the
      // A and B slabs in L2 (4096^2 x 256 -6%, 8192^2 x 1024 -3%, 16384^2 x 256 -8%; 8192^2 x 256
      // within 1%).
      asm volatile("buffer_store_dwordx4 %0, %1, %2, 0 offen nt\n\ts_nop 1" : : "v"(v), "v"(off), "s"(rsrc) : "memory");
    }
  }

  __device__ static void run_persistent(const GemmParams& p) {
    static_assert(MI == 16 && SCHED == 1 && TN % 2 == 0 && KCH % 2 == 0, "persistent kernel: pipelined 16x16 tiles");
    static_assert(RING == 2, "persistent kernel waits assume a 2-slab ring");
    static_assert(64 % kRowChunks == 0 && kWaveRows % kRowsPerStore == 0 && kStoreRows * (kStoreSteps - 1) < kWaveRows,
                  "C rows split into whole store instructions, every step some");
    static_assert(RING * SLAB_BYTES + kHeldLds <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(16))) char smem[RING * SLAB_BYTES + kHeldLds];
    char* const ctile = smem + RING * SLAB_BYTES;
    const int tid = (int)__builtin_amdgcn_workitem_id_x();
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // This workgroup's tiles: i-th is entry slot + i * S of XCD x's range of the grouped order.
    const int G = p.grid, w = (int)__builtin_amdgcn_workgroup_id_x();
    const int per = (p.tiles_m * p.tiles_n) / 8, S = G / 8, x = w % 8, slot = w / 8;
    const int n_my = slot < per ? (per - 1 - slot) / S + 1 : 0;
    if (n_my == 0) return;  // workgroup-uniform
    auto tile_origin = [&](int i, int& m0, int& n0) {
      const int pid = x * per + slot + i * S;
      const int in_group = p.group_m * p.tiles_n;
      const int first_m = (pid / in_group) * p.group_m;
      const int gsz = min(p.tiles_m - first_m, p.group_m);
      m0 = (first_m + (pid % in_group) % gsz) * BM;
      n0 = ((pid % in_group) / gsz) * BN;
    };
    auto c_rsrc = [&](int m0, int n0) {
      return make_rsrc(p.c + (int64_t)m0 * p.ldc + n0, (uint32_t)BM * (uint32_t)p.ldc * 2u);
    };
    const int ksteps = p.K / BK;

    if (wave >= WAVES) {
      // Store wave: the same barriers as the compute waves (one before the first tile, one per
      // slab step, one after the last tile). After the barrier of step ks < kStoreSteps of tile
      // i >= 1 it writes its rows of tile i - 1's C, which the compute waves put in LDS after tile
      // i - 1's last barrier and overwrite only after tile i's last one; after the final barrier,
      // its rows of the last tile.
      const int r_base = (wave - WAVES) * kWaveRows;
      __builtin_amdgcn_s_barrier();
      int pm0 = 0, pn0 = 0;
      for (int i = 0; i < n_my; ++i) {
        for (int ks = 0; ks < ksteps; ++ks) {
          __builtin_amdgcn_s_barrier();
          if (i > 0 && ks < kStoreSteps)
            c_rows_out(ctile, c_rsrc(pm0, pn0), (uint32_t)p.ldc, r_base + ks * kStoreRows, lane,
                       min(kStoreRows, kWaveRows - ks * kStoreRows));
        }
        tile_origin(i, pm0, pn0);
      }
      __builtin_amdgcn_s_barrier();
      c_rows_out(ctile, c_rsrc(pm0, pn0), (uint32_t)p.ldc, r_base, lane, kWaveRows);
      return;
    }

    const int wm = wave / WN, wn = wave % WN;
    const int r16 = lane & 15, g = lane >> 4;
    auto a_rsrc = [&](int m0) { return make_rsrc(p.a + (int64_t)m0 * p.lda, (uint32_t)BM * (uint32_t)p.lda * 2u); };
    auto b_rsrc = [&](int n0) {
      return make_rsrc(p.b + n0, (uint32_t)(((int64_t)(p.K - 1) * p.ldb + (p.N - n0)) * 2));
    };

    // DMA and read addresses as run() (16x16 layout, K whole slabs).
    uint32_t aoffs[A_PER_WAVE], boffs[B_PER_WAVE];
#pragma unroll
    for (int j = 0; j < A_PER_WAVE; ++j) {
      const int byte = (wave * A_PER_WAVE + j) * 1024 + lane * 16;
      const int r = byte / AP, s = (byte % AP) / 16;
      const int c = s ^ ((r / RA) & (SA - 1));
      aoffs[j] = ((uint32_t)r * (uint32_t)p.lda + c * 8) * 2u;
    }
#pragma unroll
    for (int j = 0; j < B_PER_WAVE; ++j) {
      const int byte = (wave * B_PER_WAVE + j) * 1024 + lane * 16;
      const int k = byte / BP, s = (byte % BP) / 16;
      const int c = s ^ (2 * ((k & 3) | (((k >> 3) & 1) << 2)));
      boffs[j] = ((uint32_t)k * (uint32_t)p.ldb + c * 8) * 2u;
    }
    uint32_t aaddr[KCH], baddr[TN];
    {
      const int xs = (r16 / RA) & (SA - 1);
#pragma unroll
      for (int c = 0; c < KCH; ++c) aaddr[c] = (uint32_t)((r16 * AP + 16 * (g ^ xs)) ^ (64 * c));
      const int kr = 8 * g + (r16 >> 2);
      const int h = (r16 >> 2) | ((g & 1) << 2);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const int jt = wn * TN + tn;
        baddr[tn] = (uint32_t)(kr * BP + 32 * (jt ^ h) + 8 * (r16 & 3));
      }
    }

    const uint32_t a_slab_bytes = (uint32_t)BK * 2u;
    const uint32_t b_slab_bytes = (uint32_t)BK * (uint32_t)p.ldb * 2u;
    const uint32_t smem_lds = lds_address(smem);

    int m0c, n0c, m0n = 0, n0n = 0;
    tile_origin(0, m0c, n0c);
    bool has_next = n_my > 1;
    if (has_next) tile_origin(1, m0n, n0n);
    int gs0 = 0;  // global index of the current tile's slab 0 (its ring slot is (gs0 + ks) % RING)
    // DMA instruction J of the current tile's slab ks_t; ks_t >= ksteps is the next tile's slab
    // ks_t - ksteps, or zeros (an offset past the range) when there is none.
    auto dma_slab = [&](int ks_t, auto jc) __attribute__((always_inline)) {
      constexpr int j = decltype(jc)::value;
      const uint32_t slotb = smem_lds + (uint32_t)((gs0 + ks_t) % RING) * SLAB_BYTES;
      const bool nxt = ks_t >= ksteps;
      const uint32_t ks = (uint32_t)(nxt ? ks_t - ksteps : ks_t);
      const bool live = !nxt | has_next;
      // the slab offset moves the resource (range 0 when there is no slab): lane offsets stay fixed
      if constexpr (j < A_PER_WAVE) {
        buffer_load16_to_lds(slab_rsrc(a_rsrc(nxt ? m0n : m0c), ks * a_slab_bytes, live), aoffs[j],
                             slotb + (wave * A_PER_WAVE + j) * 1024);
      } else {
        constexpr int jb = j - A_PER_WAVE;
        buffer_load16_to_lds(slab_rsrc(b_rsrc(nxt ? n0n : n0c), ks * b_slab_bytes, live), boffs[jb],
                             slotb + A_BYTES + (wave * B_PER_WAVE + jb) * 1024);
      }
    };

    // Prologue: the first tile's slabs 0 .. RING - 1 (ksteps >= kStoreSteps >= RING).
#pragma unroll
    for (int s0 = 0; s0 < RING; ++s0) {
      auto d = [&](auto jc) __attribute__((always_inline)) { dma_slab(s0, jc); };
      dma_all<0>(d);
    }
    wait_vm_lds_barrier<(RING - 1) * DMA_PER_SLAB>();
    Frag f[2];
    read_frag<0>(f[0], smem, aaddr, baddr, wm);

    for (int i = 0; i < n_my; ++i) {
      AccTiles acc;
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
#pragma unroll
        for (int q = 0; q < (int)(sizeof(acc.v[0]) / sizeof(floatx16)); ++q)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc.v[tn][q][r] = 0.f;
#pragma unroll
        for (int q = 0; q < (int)(sizeof(acc.t[0]) / sizeof(Acc)); ++q)
#pragma unroll
          for (int r = 0; r < ACC; ++r) acc.t[tn][q][r] = 0.f;
      }
      for (int ks = 0; ks < ksteps; ++ks) {
        const char* slab = smem + ((gs0 + ks) % RING) * SLAB_BYTES;
        auto wait = [&]() __attribute__((always_inline)) {
          wait_vm_lds_barrier<0>();  // slab ks + 1 landed (only slab DMA is in flight)
          __builtin_amdgcn_sched_barrier(0);
          return smem + ((gs0 + ks + 1) % RING) * SLAB_BYTES;
        };
        auto dma = [&](auto jc) __attribute__((always_inline)) { dma_slab(ks + RING, jc); };
        chunk_step<0, 0>(acc, f, slab, aaddr, baddr, wm, wait, dma);
      }
      // C to LDS for the store waves (they finished reading the previous tile's before this
      // tile's barrier of step kStoreSteps); the next tile's first slabs and first chunk are
      // already in flight / read
      c_to_lds(acc, ctile, wm, wn, lane);
      if (i + 1 < n_my) {
        gs0 += ksteps;
        m0c = m0n;
        n0c = n0n;
        has_next = i + 2 < n_my;
        if (has_next) tile_origin(i + 2, m0n, n0n);
      } else {
        wait_vm_lds_barrier<0>();  // the last tile's C is in LDS for the store waves
      }
    }
  }
};

template <int BM, int BN, int BK, int WM, int WN, int MI, int SCHED>
__global__ __launch_bounds__(WM * WN * 64) void gemm_f16_kernel(GemmParams p) {
  GemmKernel<BM, BN, BK, WM, WN, false, MI, SCHED>::run(p);
}

template <int BM, int BN, int BK, int WM, int WN, int MI, int SCHED>
__global__ __launch_bounds__(WM * WN * 64) void gemm_f16_shallow_kernel(GemmParams p) {
  GemmKernel<BM, BN, BK, WM, WN, true, MI, SCHED>::run(p);
}

template <int BM, int BN, int BK, int WM, int WN, int MI, int SCHED>
__global__ __launch_bounds__((WM * WN + kGemmPersistStoreWaves) * 64) void gemm_f16_persist_kernel(GemmParams p) {
  GemmKernel<BM, BN, BK, WM, WN, false, MI, SCHED>::run_persistent(p);
}

template <int BM, int BN, int BK, int WM, int WN, int MI, int KSG>
__global__ __launch_bounds__(WM * WN * KSG * 64) void gemm_f16_ksplit_kernel(GemmParams p) {
  GemmKernel<BM, BN, BK, WM, WN, false, MI, 1, KSG>::run(p);
}

// The shallow-ring kernel of a tile, or nullptr when its ring would be as deep as the default one.
template <int BM, int BN, int BK, int WM, int WN, int MI, int SCHED>
const void* gemm_shallow_fn() {
  if constexpr (GemmKernel<BM, BN, BK, WM, WN, true, MI, SCHED>::RING < GemmKernel<BM, BN, BK, WM, WN, false, MI, SCHED>::RING)
    return (const void*)&gemm_f16_shallow_kernel<BM, BN, BK, WM, WN, MI, SCHED>;
  else
    return nullptr;
}

#define GEMM_ENTRY(BM, BN, BK, WM, WN, MI, SCHED)                                                         \
  {BM, BN, BK, WM * WN, (const void*)&gemm_f16_kernel<BM, BN, BK, WM, WN, MI, SCHED>,                    \
   gemm_shallow_fn<BM, BN, BK, WM, WN, MI, SCHED>(),                                                      \
   "_ZN2fa15gemm_f16_kernelILi" #BM "ELi" #BN "ELi" #BK "ELi" #WM "ELi" #WN "ELi" #MI "ELi" #SCHED \
   "EEEvNS_10GemmParamsE", nullptr}
// A tile that also has the persistent short-K kernel.
#define GEMM_ENTRY_PERSIST(BM, BN, BK, WM, WN, MI, SCHED)                                                 \
  {BM, BN, BK, WM * WN, (const void*)&gemm_f16_kernel<BM, BN, BK, WM, WN, MI, SCHED>,                    \
   gemm_shallow_fn<BM, BN, BK, WM, WN, MI, SCHED>(),                                                      \
   "_ZN2fa15gemm_f16_kernelILi" #BM "ELi" #BN "ELi" #BK "ELi" #WM "ELi" #WN "ELi" #MI "ELi" #SCHED \
   "EEEvNS_10GemmParamsE",                                                                                \
   (const void*)&gemm_f16_persist_kernel<BM, BN, BK, WM, WN, MI, SCHED>}
// A tile of KSG K groups of WM x WN waves (pipelined schedule; no shallow or persistent kernel).
#define GEMM_ENTRY_KSPLIT(BM, BN, BK, WM, WN, MI, KSG)                                                    \
  {BM, BN, BK, WM * WN * KSG, (const void*)&gemm_f16_ksplit_kernel<BM, BN, BK, WM, WN, MI, KSG>, nullptr, \
   "_ZN2fa22gemm_f16_ksplit_kernelILi" #BM "ELi" #BN "ELi" #BK "ELi" #WM "ELi" #WN "ELi" #MI "ELi" #KSG \
   "EEEvNS_10GemmParamsE", nullptr}

// One kernel per tile: the MFMA shape and schedule measured fastest for it on MI355X (16x16x32
// MFMAs draw less power per flop, which raises the clock of the 8-wave tiles; the pipelined
// schedule pays where one or two waves per SIMD would otherwise wait on LDS and barriers).
static const GemmKernelEntry kGemmEntries[] = {
    GEMM_ENTRY(256, 256, 64, 2, 4, 16, 1),
    GEMM_ENTRY(256, 256, 32, 2, 4, 16, 1),
    GEMM_ENTRY_PERSIST(256, 128, 64, 4, 2, 16, 1),
    GEMM_ENTRY(128, 256, 64, 2, 4, 16, 1),
    GEMM_ENTRY(256, 256, 64, 2, 2, 32, 1),
    GEMM_ENTRY(256, 256, 32, 2, 2, 32, 1),
    GEMM_ENTRY(128, 128, 64, 2, 2, 32, 1),
    GEMM_ENTRY(128, 128, 32, 2, 2, 32, 1),
    GEMM_ENTRY(128, 64, 32, 2, 2, 32, 0),
    GEMM_ENTRY(64, 256, 32, 2, 2, 16, 1),
    GEMM_ENTRY_KSPLIT(128, 128, 32, 2, 2, 32, 2),
    GEMM_ENTRY_KSPLIT(128, 64, 32, 2, 2, 32, 2),
    GEMM_ENTRY_KSPLIT(128, 64, 32, 2, 2, 32, 4),
    GEMM_ENTRY_KSPLIT(64, 64, 32, 2, 2, 32, 2),
};

const GemmKernelEntry* gemm_registry(int* count) {
  *count = (int)(sizeof(kGemmEntries) / sizeof(kGemmEntries[0]));
  return kGemmEntries;
}

}  // namespace fa
