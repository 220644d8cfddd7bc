// FlashAttention forward for gfx950 (MI355X, CDNA4): basic, optimized and split-KV ("sliced").
//
// Follows the online-softmax algorithm of the reference kernels (flash_atten.py:76-133): per KV
// tile, S = Q K^T * scale, running row max m, P = exp(S - m), rescale alpha = exp(m_old - m),
// acc = acc*alpha + P V with P rounded to the input dtype, l = l*alpha + rowsum(P); finally
// O = acc / l and LSE = m + ln l. The design is gfx950-first:
//
//  * Each wave owns 32*RT query rows. S is computed transposed, S^T = K Q^T, with
//    v_mfma_f32_32x32x16: the accumulator then gives every lane ONE query row (lane & 31) and 16
//    keys per 32x32 tile, so the row max / sum / rescale factor are per-lane scalars and the only
//    cross-lane step is one exchange between the two half-waves.
//  * Q^T is the B operand and stays in registers for the whole kernel (loaded once; AGPRs in the
//    kernels with one wave per SIMD).
//  * P^T is fed to O^T = V^T P^T directly from the S^T accumulator registers (the B-operand k-slots
//    of a 16-key chunk are exactly 8 accumulator rows the lane already holds), so P never goes
//    through LDS. V^T is the A operand, read from V stored naturally ([key][d]) in LDS with the
//    gfx950 transposing read ds_read_b64_tr_b16: in a 16-lane group, result lane i element c is
//    element (i & 3) of the 8-byte chunk addressed by group lane 4c + (i >> 2). Each lane of group
//    lane L addresses key J + (L >> 2), columns d0 + 4 (L & 3); lane i then holds V[J + c][d0 + i].
//  * stages=1 (basic) and stages=2: K and V tiles are staged HBM -> registers -> LDS with
//    precomputed per-thread addresses (padded rows), the next tile's global loads issued before the
//    current tile is computed; stages=1 keeps one LDS buffer (two barriers per tile), stages=2
//    double-buffers K/V (one barrier per tile).
//    stages=3: software pipeline inside each wave (QK MFMAs of tile u+1 interleaved with the
//    softmax VALU work of tile u, PV of tile u with the row max of tile u+1), K/V brought into a
//    ring of fragment-major LDS tiles by LDS-DMA loads (see the stages=3 branch of run()).
//    LDS fragment reads are issued a few MFMAs ahead of use (scheduling-group hints).
//  * Softmax in the exp2 domain with scale*log2(e) folded into one FMA per score; the O rescale is
//    lazy: the exponent offset only moves when a row max grows by more than 8 (log2 units), so
//    P <= 256 and the 4*D accumulator multiplies run on a handful of tiles per row. For fp16 the
//    row sum is accumulated from the rounded P (v_dot2 with (1, 1)), i.e. the same P the PV
//    product uses; for bf16 from the fp32 values.
//  * Causal (top-left, row i sees keys j <= i as flash_atten.py:103-105) skips KV tiles past the
//    diagonal (stages 1/2 also skip waves whose rows all precede a tile), masks only diagonal
//    tiles, and walks query blocks heaviest-first.
//  * GQA: query head h reads KV head h / (H / H_kv); no K/V expansion.
//  * Split-KV: the SPLIT instantiation writes fp32 normalised partial O and partial LSE per KV
//    split; fa_merge_kernel combines them: lse = ln sum_j exp(lse_j), O = sum_j exp(lse_j - lse) O_j.
#include <type_traits>

#include "fa_common.h"
#include "fa_kernels.h"
#include "../../include/fa_gfx950.h"

namespace fa {

template <typename Tag, int D, int WAVES, int RT, int BN, int STAGES, bool SPLIT>
struct FwdKernel {
  static constexpr int THREADS = WAVES * 64;
  static constexpr int ROWS = 32 * RT;          // query rows per wave
  static constexpr int BM = WAVES * ROWS;       // query rows per workgroup
  static constexpr int DC = D / 16;             // 16-wide d chunks of Q K^T
  static constexpr int DTL = D / 32;            // 32-row d tiles of O^T
  static constexpr int JT = BN / 32;            // 32-key tiles of S^T
  static constexpr int KC = BN / 16;            // 16-key chunks of P V
  static constexpr int KSTR = D + 8;            // K LDS row stride (elements): 16-byte skew
  static constexpr int VSTR = D + 32;           // V LDS row stride (elements): 64-byte skew
  static constexpr int KTILE = BN * KSTR;
  static constexpr int VTILE = BN * VSTR;
  static constexpr int CPR = D / 8;             // 16-byte chunks per K/V row
  static constexpr int RSTEP = THREADS / CPR;   // rows covered by one pass of the workgroup
  static constexpr int PASSES = (BN + RSTEP - 1) / RSTEP;
  static constexpr float THRESH = 8.0f;         // lazy-rescale threshold (log2 units)
  static constexpr bool kSumRounded = __is_same(Tag, f16_t);  // row sum from the rounded P
  static_assert(D % 32 == 0 && BN % 32 == 0, "tile shape");
  static_assert(THREADS % CPR == 0, "threads must cover whole rows");
  static_assert(BM % BN == 0, "causal tile bound assumes block_m % block_n == 0");

  typedef DT<Tag> T;
  typedef floatx16 STile[JT][RT];

  struct Ctx {
    const uint16_t* kp;  // this thread's first K chunk (row r0, column c8) of tile 0
    const uint16_t* vp;
    int64_t sk2, sv2;    // row strides
    int r0, c8;
    int N;
  };

  __device__ static inline void load_rows(u32x4 (&dst)[PASSES], const uint16_t* base, int64_t stride, int n0,
                                          const Ctx& cx) {
    const uint16_t* p = base + (int64_t)n0 * stride;
    const bool full = n0 + BN <= cx.N;
#pragma unroll
    for (int i = 0; i < PASSES; ++i) {
      const int row = cx.r0 + i * RSTEP;
      u32x4 val = {0u, 0u, 0u, 0u};
      if ((BN % RSTEP == 0 || row < BN) && (full || n0 + row < cx.N))
        val = *reinterpret_cast<const u32x4*>(p + (int64_t)(i * RSTEP) * stride);
      dst[i] = val;
    }
  }

  template <int STR>
  __device__ static inline void store_rows(const u32x4 (&src)[PASSES], uint16_t* buf, const Ctx& cx) {
#pragma unroll
    for (int i = 0; i < PASSES; ++i) {
      const int row = cx.r0 + i * RSTEP;
      if (BN % RSTEP == 0 || row < BN) *reinterpret_cast<u32x4*>(buf + row * STR + cx.c8 * 8) = src[i];
    }
  }

  // S^T tiles for one KV tile: s[jt][rt] = K[jt*32 + ., :] Q^T[:, rt*32 + .]
  __device__ static inline void qk(STile& s, const u32x4 (&qf)[RT][DC], const uint16_t* ks, int lane_k_off) {
#pragma unroll
    for (int jt = 0; jt < JT; ++jt)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[jt][rt][r] = 0.f;
#pragma unroll
    for (int cc = 0; cc < DC; ++cc) {
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) {
        const u32x4 kf = *reinterpret_cast<const u32x4*>(ks + lane_k_off + jt * 32 * KSTR + cc * 16);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) s[jt][rt] = T::mfma32(kf, qf[rt][cc], s[jt][rt]);
      }
    }
  }

  // Keys past N, and (causal) keys after the query row, get score -inf. Wave-uniform test first:
  // only tiles at the sequence end or on the diagonal need the per-element masks.
  __device__ static inline bool tile_needs_mask(int n0, int wrow0, const FwdParams& p) {
    return (n0 + BN > p.N) || (p.causal && n0 + BN - 1 > wrow0);
  }
  __device__ static inline void mask_tile(STile& s, int n0, int wrow0, int col, int hh, const FwdParams& p) {
#pragma unroll
    for (int jt = 0; jt < JT; ++jt)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int i = wrow0 + rt * 32 + col;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = n0 + jt * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (j >= p.N || (p.causal && j > i)) s[jt][rt][r] = FA_NEG_INF;
        }
      }
  }

  // Row max of a score tile (each lane's row, both half-waves).
  __device__ static inline void tile_max(const STile& s, float (&mx)[RT]) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float m = FA_NEG_INF;
#pragma unroll
      for (int jt = 0; jt < JT; ++jt)
#pragma unroll
        for (int r = 0; r < 16; r += 2) m = fmaxf(m, fmaxf(s[jt][rt][r], s[jt][rt][r + 1]));
      mx[rt] = xhalf_max(m);
    }
  }

  // Kernels with one wave per SIMD keep O in AGPRs (the MFMAs accumulate there directly). The rare
  // rescale needs O in VGPRs; pinning O to AGPRs on both sides of it keeps the AGPR <-> VGPR copies
  // inside the rescale branch. Without the pins the compiler hoisted them to the loop header, where
  // 144 v_accvgpr_read ran on every step of the D = 256 kernel (~15% of its time).
  // more than 256 registers per lane (the stages=5 kernel is built to fit 256: O and Q in VGPRs)
  static constexpr bool kAccInAgpr = (RT > 1 || D > 128) && STAGES != 5;
  // Workgroups per CU the launch bounds ask for: four-wave workgroups with RT = 1 and D <= 128 (and
  // the lean stages=5 kernels) fit two per CU; the lean kernel with 32-key D <= 128 tiles fits three.
  static constexpr int kBlocksPerCu =
      (WAVES == 4 && RT == 1 && STAGES == 5 && D <= 128 && BN == 32) ? 3
      : (WAVES == 4 && RT == 1 && (D <= 128 || STAGES == 5))          ? 2
                                                                       : 1;
  __device__ static inline void pin_acc_agpr(floatx16 (&acc)[DTL][RT], int rt) {
    if constexpr (kAccInAgpr) {
#pragma unroll
      for (int dt = 0; dt < DTL; ++dt) asm volatile("" : "+a"(acc[dt][rt]));
    }
  }

  // Lazy rescale: move the exponent offset m_use (and rescale O and l) only when some row of the
  // wave sees a max more than THRESH (log2 units) above it.
  __device__ static inline void rescale(const float (&mx)[RT], floatx16 (&acc)[DTL][RT], float (&m_use)[RT],
                                        float (&l_i)[RT], float c) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const bool need = mx[rt] > m_use[rt] + THRESH / c;
      if (__builtin_amdgcn_ballot_w64(need) != 0) {
        const float m_new = fmaxf(m_use[rt], mx[rt]);
        const float alpha = (m_use[rt] == FA_NEG_INF) ? 0.f : fast_exp2((m_use[rt] - m_new) * c);
        m_use[rt] = m_new;
        l_i[rt] *= alpha;
        pin_acc_agpr(acc, rt);
#pragma unroll
        for (int dt = 0; dt < DTL; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[dt][rt][r] *= alpha;
        pin_acc_agpr(acc, rt);
      }
    }
  }

  // Masks (only on tiles that need them), online softmax with lazy rescale, P packing. Leaves
  // packed P in pk.
  __device__ static inline void softmax(STile& s, u32x4 (&pk)[KC][RT], floatx16 (&acc)[DTL][RT], float (&m_use)[RT],
                                        float (&l_i)[RT], int n0, int wrow0, int col, int hh, const FwdParams& p) {
    if (tile_needs_mask(n0, wrow0, p)) mask_tile(s, n0, wrow0, col, hh, p);
    float mx[RT];
    tile_max(s, mx);
    rescale(mx, acc, m_use, l_i, p.c);
    exp_pack(s, pk, m_use, l_i, p.c);
  }

  // P = exp2(S c - m_use c) rounded to the input dtype and packed as the B operand of P V; the
  // row sum l accumulates the same P.
  __device__ static inline void exp_pack(const STile& s, u32x4 (&pk)[KC][RT], const float (&m_use)[RT],
                                         float (&l_i)[RT], float c) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const float mc = (m_use[rt] == FA_NEG_INF) ? 0.f : m_use[rt] * c;
      float l0 = 0.f, l1 = 0.f;
#pragma unroll
      for (int jt = 0; jt < JT; ++jt)
#pragma unroll
        for (int half = 0; half < 2; ++half)
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const int r = half * 8 + 2 * w;
            const float e0 = fast_exp2(__builtin_fmaf(s[jt][rt][r], c, -mc));
            const float e1 = fast_exp2(__builtin_fmaf(s[jt][rt][r + 1], c, -mc));
            const uint32_t pw = T::pack2(e0, e1);
            pk[jt * 2 + half][rt][w] = pw;
            if (kSumRounded) {
              // binary16 P (11-bit significand): summing the rounded pair moves l by <= 2^-12 relative
              if (w & 1) l1 = dot2_sum<Tag>(pw, l1);
              else l0 = dot2_sum<Tag>(pw, l0);
            } else {
              // bfloat16 P (8-bit significand) is too coarse for l: sum the fp32 values
              if (w & 1) l1 += e0 + e1;
              else l0 += e0 + e1;
            }
          }
      l_i[rt] += l0 + l1;
    }
  }

  // Scheduling hints (apply to the basic block they are emitted in): issue the LDS fragment reads
  // a few MFMAs ahead of their use instead of waiting on each read right before its MFMA.
  static constexpr int kReadAheadK = 4;  // K fragments (one ds_read_b128 each)
  // V fragments (two ds_read_b64_tr_b16 each); one wave per SIMD (D = 256) has no second wave to
  // hide LDS latency and, with Q and O in AGPRs, the VGPRs to read further ahead
  static constexpr int kReadAheadV = kAccInAgpr ? 4 : 2;
  __device__ static inline void qk_schedule() {
    __builtin_amdgcn_sched_group_barrier(0x100, kReadAheadK, 0);  // DS read
#pragma unroll
    for (int i = 0; i < DC * JT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, RT, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
    }
  }
  __device__ static inline void pv_schedule() {
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kReadAheadV, 1);
#pragma unroll
    for (int i = 0; i < KC * DTL; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, RT, 1);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
    }
  }

  // Software-pipelined step (stages=3), first half: the QK MFMAs of the next tile interleaved
  // with the exp / pack / row-sum VALU work of the current tile, a few VALU ops per MFMA, so the
  // matrix core and the VALU run at the same time inside one wave.
  static constexpr int kExpValu = JT * RT * (16 * 2 + 8 * 2);  // FMA + exp per score, pack + sum per pair
  static constexpr int kXValuPerMfma = (kExpValu + DC * JT - 1) / (DC * JT);  // per group of RT MFMAs
  __device__ static inline void x_schedule() {
    __builtin_amdgcn_sched_group_barrier(0x100, kReadAheadK, 2);
#pragma unroll
    for (int i = 0; i < DC * JT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, RT, 2);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 2);
      __builtin_amdgcn_sched_group_barrier(0x002, kXValuPerMfma, 2);
    }
  }
  // Second half: the PV MFMAs of the current tile interleaved with the row max of the next one.
  __device__ static inline void y_schedule() {
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kReadAheadV, 2);
#pragma unroll
    for (int i = 0; i < KC * DTL; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, RT, 2);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 2);
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 2);
    }
  }

  // ---- stages=3: fragment-major LDS tiles filled by LDS-DMA ----
  // K tile: NKB blocks of 1 KiB, block (jt, cc) = jt * DC + cc holds, at byte 16 l, the 16 bytes
  // lane l feeds to the QK MFMA: K[jt*32 + (l & 31)][cc*16 + 8*(l >> 5) .. +7].
  // V tile: NVB blocks of 1 KiB, block (kc, dt) = kc * DTL + dt holds the two transposing reads
  // (rows kc*16 + 0..7, then + 8..15) of that (key chunk, d tile), lane L's 8 bytes at 8 L.
  // Every LDS read instruction thus reads one contiguous block (no bank conflicts, no per-lane
  // address arithmetic), and every DMA instruction writes one block.
  static constexpr int NKB = JT * DC;
  static constexpr int NVB = KC * DTL;
  static constexpr int KT_ELEMS = NKB * 512;  // 16-bit elements per K tile
  static constexpr int VT_ELEMS = NVB * 512;
  // Tiles of K (and of V) resident in LDS: 3 when one workgroup owns the CU, 2 when two
  // four-wave workgroups share it (RT = 1: two waves per SIMD). The stages=4 D = 256 kernel holds
  // one workgroup per CU (one wave per SIMD) and keeps 3.
  static constexpr int RING = (STAGES == 5) ? 2 : (WAVES >= 8 || RT >= 2 || (STAGES == 4 && D > 128)) ? 3 : 2;
  static constexpr int NKW = NKB / WAVES;            // DMA blocks per wave per K tile
  static constexpr int NVW = NVB / WAVES;
  static_assert(STAGES < 3 || (NKB % WAVES == 0 && NVB % WAVES == 0), "tile blocks must split evenly over waves");
  static_assert(STAGES != 4 || RING <= 3, "the stages=4 waits assume a ring of at most 3 tiles");

  __device__ static inline void qk_fm(STile& s, const u32x4 (&qf)[RT][DC], const uint16_t* kslot_lane) {
    if constexpr (JT * RT == 1 && STAGES != 5) {
      // A single score tile (D = 256 with 32-key tiles) would be one chain of DC dependent MFMAs:
      // run the even and odd d chunks as two independent chains and add them (+1.5% at D = 256).
      // The stages=5 kernel has no registers for the second chain; its second wave per SIMD
      // covers the chain's latency instead.
      floatx16 s0 = {}, s1 = {};
#pragma unroll
      for (int cc = 0; cc < DC; cc += 2) {
        const u32x4 k0 = *reinterpret_cast<const u32x4*>(kslot_lane + cc * 512);
        const u32x4 k1 = *reinterpret_cast<const u32x4*>(kslot_lane + (cc + 1) * 512);
        s0 = T::mfma32(k0, qf[0][cc], s0);
        s1 = T::mfma32(k1, qf[0][cc + 1], s1);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) s[0][0][r] = s0[r] + s1[r];
      return;
    }
#pragma unroll
    for (int jt = 0; jt < JT; ++jt)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[jt][rt][r] = 0.f;
#pragma unroll
    for (int cc = 0; cc < DC; ++cc) {
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) {
        const u32x4 kf = *reinterpret_cast<const u32x4*>(kslot_lane + (jt * DC + cc) * 512);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) s[jt][rt] = T::mfma32(kf, qf[rt][cc], s[jt][rt]);
      }
    }
  }

  __device__ static inline void pv_fm(floatx16 (&acc)[DTL][RT], const u32x4 (&pk)[KC][RT], const uint16_t* vslot_lane) {
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
      for (int dt = 0; dt < DTL; ++dt) {
        const uint16_t* base = vslot_lane + (kc * DTL + dt) * 512;
        const u32x2 lo = lds_read_tr16(base);
        const u32x2 hi = lds_read_tr16(base + 256);
        const u32x4 vf = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) acc[dt][rt] = T::mfma32(vf, pk[kc][rt], acc[dt][rt]);
      }
    }
  }

  // ---- stages=4: two-tile-ahead pipeline ----
  // One step's matrix work: the QK MFMAs of tile u+2 (S^T into `nxt`) and the PV MFMAs of tile u
  // (O^T += V^T P^T with `pk`), one for one. Both counts are BN * D / 512 per row tile. QK pairs
  // run score-tile-major, so the second 32-key score tile's accumulators come to life only halfway
  // through the step (registers: the step also holds S_{u+1}, P_u and P_{u+1}); a QK MFMA then
  // depends on the QK two MFMAs back, with an independent PV MFMA between them. PV pairs run
  // key-chunk-major, so P_u's registers die chunk by chunk.
  static constexpr int NQ = JT * DC;
  static_assert(NQ == KC * DTL, "QK and PV MFMA counts per tile are equal");
  __device__ static inline void qk_pv_fm(STile& nxt, const u32x4 (&qf)[RT][DC], const uint16_t* kslot_lane,
                                         floatx16 (&acc)[DTL][RT], const u32x4 (&pk)[KC][RT],
                                         const uint16_t* vslot_lane) {
#pragma unroll
    for (int jt = 0; jt < JT; ++jt)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int r = 0; r < 16; ++r) nxt[jt][rt][r] = 0.f;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int jt = i / DC, cc = i % DC;
      const int kc = i / DTL, dt = i % DTL;
      const u32x4 kf = *reinterpret_cast<const u32x4*>(kslot_lane + (jt * DC + cc) * 512);
      const uint16_t* vb = vslot_lane + (kc * DTL + dt) * 512;
      const u32x2 lo = lds_read_tr16(vb);
      const u32x2 hi = lds_read_tr16(vb + 256);
      const u32x4 vf = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        nxt[jt][rt] = T::mfma32(kf, qf[rt][cc], nxt[jt][rt]);
        acc[dt][rt] = T::mfma32(vf, pk[kc][rt], acc[dt][rt]);
      }
    }
  }

  // Online softmax of one (already masked) score tile without a branch: a row whose max grew by
  // more than THRESH (log2 units) over its exponent offset moves the offset to that max, and its
  // alpha = exp2((m_old - m_new) c) rescales l now and O once this step's PV is done
  // (rescale_acc); other rows keep alpha = 1. P and the row sum use the updated offset.
  __device__ static inline void softmax_nb(const STile& s, u32x4 (&pk)[KC][RT], float (&m_use)[RT],
                                           float (&l_i)[RT], float (&alpha)[RT], float c, float thr) {
    float mx[RT];
    tile_max(s, mx);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const bool up = mx[rt] > m_use[rt] + thr;  // false while the row has seen no key (mx = -inf)
      const float m_new = up ? mx[rt] : m_use[rt];
      // one unconditional exp of a selected argument (a conditional exp becomes a divergent branch
      // that splits the step's block): exp2(0) = 1 for rows that keep their offset, exp2(-inf) = 0
      // for a row's first finite max
      alpha[rt] = fast_exp2(up ? (m_use[rt] - m_new) * c : 0.f);
      l_i[rt] *= alpha[rt];
      m_use[rt] = m_new;
    }
    exp_pack(s, pk, m_use, l_i, c);
  }

  // O *= alpha per row, when any row of the wave moved its offset (rare).
  __device__ static inline void rescale_acc(floatx16 (&acc)[DTL][RT], const float (&alpha)[RT]) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      if (__builtin_amdgcn_ballot_w64(alpha[rt] != 1.f) != 0) {
        pin_acc_agpr(acc, rt);
#pragma unroll
        for (int dt = 0; dt < DTL; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[dt][rt][r] *= alpha[rt];
        pin_acc_agpr(acc, rt);
      }
    }
  }

  // Scheduling of a stages=4 step block: LDS reads a few fragments ahead, then per MFMA one or two
  // LDS reads and an even share of the softmax VALU work.
  static constexpr int kSoftValu = JT * RT * (16 * 2 + 8 * 2) + 12 * RT;
  template <bool WITH_QK>
  __device__ static inline void step_schedule() {
    constexpr int mfma = (WITH_QK ? 2 : 1) * NQ;  // groups of RT MFMAs
    constexpr int valu = (kSoftValu + mfma - 1) / mfma;
    // QK and PV alternate: 1 K read, then 2 V reads per pair of MFMAs
    __builtin_amdgcn_sched_group_barrier(0x100, WITH_QK ? 3 : 2 * kReadAheadV, 3);
#pragma unroll
    for (int i = 0; i < mfma / 2; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, RT, 3);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 3);
      __builtin_amdgcn_sched_group_barrier(0x002, valu, 3);
      __builtin_amdgcn_sched_group_barrier(0x008, RT, 3);
      __builtin_amdgcn_sched_group_barrier(0x100, WITH_QK ? 1 : 2, 3);
      __builtin_amdgcn_sched_group_barrier(0x002, valu, 3);
    }
  }

  // O^T += V^T P^T
  __device__ static inline void pv(floatx16 (&acc)[DTL][RT], const u32x4 (&pk)[KC][RT], const uint16_t* vs,
                                   int lane_v_off) {
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
      for (int dt = 0; dt < DTL; ++dt) {
        const uint16_t* base = vs + lane_v_off + kc * 16 * VSTR + dt * 32;
        const u32x2 lo = lds_read_tr16(base);
        const u32x2 hi = lds_read_tr16(base + 8 * VSTR);
        const u32x4 vf = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) acc[dt][rt] = T::mfma32(vf, pk[kc][rt], acc[dt][rt]);
      }
    }
  }

  __device__ static void run(const FwdParams& p) {
    constexpr int SMEM = (STAGES == 1)   ? (KTILE + VTILE)
                         : (STAGES == 2) ? 2 * (KTILE + VTILE)
                                         : RING * (KT_ELEMS + VT_ELEMS);
    __shared__ __attribute__((aligned(16))) uint16_t smem[SMEM];

    const int tid = threadIdx.x;
    // wave index in a scalar register: wave-uniform row bounds and mask tests stay scalar
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), col = lane & 31, hh = lane >> 5;

    // Logical block id: XCD-local, then (bh, split, m-block) with the m-block fastest. bh is
    // (batch, query head), or (batch, kv head) when the query heads of a GQA group are packed
    // into the rows (pack > 1, decode shapes): row r is then query head h + r / M, position r % M.
    const int pid = xcd_remap(blockIdx.x, p.total_blocks);
    int mb = pid % p.m_blocks;
    const int rest = pid / p.m_blocks;
    const int split = rest % p.splits;
    const int bh = rest / p.splits;
    if (p.causal) mb = p.m_blocks - 1 - mb;  // heaviest query blocks first
    int b, h, hk;
    if (p.pack > 1) {
      b = bh / p.Hkv;
      hk = bh % p.Hkv;
      h = hk * p.group;
    } else {
      b = bh / p.H;
      h = bh % p.H;
      hk = h / p.group;
    }
    const int rows = p.M * p.pack;       // query rows of this workgroup's row space
    const int m0 = mb * BM;
    const int wrow0 = m0 + wave * ROWS;  // first query row of this wave
    const bool wave_has_rows = wrow0 < rows;
    auto row_head = [&](int r) { return p.pack > 1 ? h + r / p.M : h; };
    auto row_pos = [&](int r) { return p.pack > 1 ? r % p.M : r; };

    Ctx cx;
    cx.r0 = tid / CPR;
    cx.c8 = tid % CPR;
    cx.sk2 = p.sk2;
    cx.sv2 = p.sv2;
    cx.N = p.N;
    cx.kp = p.k + (int64_t)b * p.sk0 + (int64_t)hk * p.sk1 + (int64_t)cx.r0 * p.sk2 + cx.c8 * 8;
    cx.vp = p.v + (int64_t)b * p.sv0 + (int64_t)hk * p.sv1 + (int64_t)cx.r0 * p.sv2 + cx.c8 * 8;

    // Q^T fragments (B operand): lane holds row wrow0 + 32*rt + col, d = 16c + 8hh .. +7.
    u32x4 qf[RT][DC];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int row = wrow0 + rt * 32 + col;
      const uint16_t* qrow =
          p.q + (int64_t)b * p.sq0 + (int64_t)row_head(row) * p.sq1 + (int64_t)row_pos(row) * p.sq2;
#pragma unroll
      for (int cc = 0; cc < DC; ++cc) {
        u32x4 val = {0u, 0u, 0u, 0u};
        if (row < rows) val = *reinterpret_cast<const u32x4*>(qrow + cc * 16 + hh * 8);
        qf[rt][cc] = val;
      }
    }
    if constexpr (STAGES == 4) {
      // Retire the Q loads here, on every path, before any LDS-DMA is in flight. The compiler does
      // not see the DMAs (inline asm); where it cannot prove the Q loads were waited for on every
      // path into the loop it puts a vmcnt(0) before the step's first MFMA, which at run time
      // waits for the step's own K/V prefetch as well.
      __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (15 << 8) | (0 << 14));
    }
    if constexpr (kAccInAgpr) {
      // Q is only ever an MFMA operand, which may sit in AGPRs: this leaves VGPRs for fragment
      // read-ahead in the one-wave-per-SIMD kernels.
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int cc = 0; cc < DC; ++cc) asm volatile("" : "+a"(qf[rt][cc]));
    }

    // KV tiles of this split, clipped by the causal diagonal.
    const int t_begin = split * p.tiles_per_split;
    int n_end = (t_begin + p.tiles_per_split) * BN;
    if (n_end > p.N) n_end = p.N;
    if (p.causal && n_end > m0 + BM) n_end = m0 + BM;
    const int t_end = (n_end + BN - 1) / BN;
    const int ntiles = t_end > t_begin ? t_end - t_begin : 0;

    floatx16 acc[DTL][RT];
    float m_use[RT], l_i[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      m_use[rt] = FA_NEG_INF;
      l_i[rt] = 0.f;
#pragma unroll
      for (int dt = 0; dt < DTL; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[dt][rt][r] = 0.f;
    }

    // Per-lane LDS fragment offsets.
    const int lane_k_off = col * KSTR + hh * 8;
    const int g = lane & 15;
    const int lane_v_off = (4 * hh + (g >> 2)) * VSTR + 16 * ((lane >> 4) & 1) + 4 * (g & 3);

    // Waves skip tiles they have no work in: rows past the row space (packed decode tiles), or
    // (causal) rows that all precede the tile.
    auto active = [&](int t) { return wave_has_rows && !(p.causal && t * BN > wrow0 + ROWS - 1); };

    if constexpr (STAGES == 1) {
      uint16_t* ks = smem;
      uint16_t* vs = smem + KTILE;
      u32x4 pkr[PASSES], pvr[PASSES];
      if (ntiles > 0) {
        load_rows(pkr, cx.kp, cx.sk2, t_begin * BN, cx);
        load_rows(pvr, cx.vp, cx.sv2, t_begin * BN, cx);
      }
      for (int u = 0; u < ntiles; ++u) {
        const int n0 = (t_begin + u) * BN;
        __syncthreads();
        store_rows<KSTR>(pkr, ks, cx);
        store_rows<VSTR>(pvr, vs, cx);
        __syncthreads();
        if (u + 1 < ntiles) {
          load_rows(pkr, cx.kp, cx.sk2, n0 + BN, cx);
          load_rows(pvr, cx.vp, cx.sv2, n0 + BN, cx);
        }
        if (active(t_begin + u)) {
          STile s;
          u32x4 pk[KC][RT];
          qk(s, qf, ks, lane_k_off);
          qk_schedule();
          softmax(s, pk, acc, m_use, l_i, n0, wrow0, col, hh, p);
          pv(acc, pk, vs, lane_v_off);
          pv_schedule();
        }
      }
    } else if constexpr (STAGES >= 3) {
      // stages=3: software pipeline across KV tiles inside each wave. Step u starts with S_u = K_u Q^T and
      // its row max already computed, then
      //   (rare branch) lazy rescale for tile u
      //   X: P_u = exp(S_u)      interleaved with  S_{u+1} = K_{u+1} Q^T      (VALU | MFMA)
      //   Y: O += P_u V_u        interleaved with  rowmax(S_{u+1})             (MFMA | VALU)
      // K runs one tile ahead of V: step u reads K_{u+1} and V_u. Tiles reach LDS by LDS-DMA
      // (buffer_load ... lds, no registers) into rings of RING K slots and RING V slots: step u
      // issues K_{u+RING} into the slot K_u left and V_{u+RING-1} into the slot V_{u-1} left, so
      // with RING = 3 a tile has two steps to arrive; the barrier at the end of a step waits only
      // for the loads the next step reads. The buffer range is the (b, kv-head) rows [0, N): rows
      // past N read as zero without a branch (the host keeps (N + block_n) * row stride * 2 bytes
      // below 2^32). The step is unrolled by two so the two score tiles alternate without copies.
      uint16_t* kring = smem;
      uint16_t* vring = smem + RING * KT_ELEMS;
      const auto krs = make_rsrc(p.k + (int64_t)b * p.sk0 + (int64_t)hk * p.sk1, (uint32_t)p.N * (uint32_t)p.sk2 * 2u);
      const auto vrs = make_rsrc(p.v + (int64_t)b * p.sv0 + (int64_t)hk * p.sv1, (uint32_t)p.N * (uint32_t)p.sv2 * 2u);
      // Byte offset (within a tile) of the 16 bytes this lane moves for the first block of this
      // wave. A wave's blocks are consecutive d chunks of one 32-key tile (K: +16 columns = +32
      // bytes per block) or consecutive d tiles of one 16-key chunk (V: +32 columns = +64 bytes),
      // so the other blocks differ by an immediate offset.
      static_assert(DC % NKW == 0 && DTL % NVW == 0, "a wave's DMA blocks stay in one key group");
      uint32_t koff, voff;
      {
        const int blk = wave * NKW, jt = blk / DC, cc = blk % DC;
        const uint32_t row = jt * 32 + (lane & 31), c0 = cc * 16 + 8 * (lane >> 5);
        koff = (row * (uint32_t)p.sk2 + c0) * 2u;
      }
      {
        const int blk = wave * NVW, kc = blk / DTL, dt = blk % DTL;
        const int m = lane & 31, half = lane >> 5;  // the lane pair (2m, 2m+1) of read `half`
        const uint32_t row = kc * 16 + 8 * half + 4 * (m >> 4) + ((m & 7) >> 1);
        const uint32_t c0 = dt * 32 + 16 * ((m >> 3) & 1) + 8 * (m & 1);
        voff = (row * (uint32_t)p.sv2 + c0) * 2u;
      }
      // DMA destinations as LDS byte addresses from the (scalar) wave index: M0 is computed with
      // scalar instructions only.
      const uint32_t kring_lds = lds_address(smem), vring_lds = kring_lds + RING * KT_ELEMS * 2;
      auto issue_k = [&](int u) {
        if (u >= ntiles) return;
        const uint32_t toff = (uint32_t)((t_begin + u) * BN) * (uint32_t)p.sk2 * 2u;
        const uint32_t slot = kring_lds + (uint32_t)(u % RING) * (KT_ELEMS * 2);
        buffer_load16_to_lds_blocks<NKW, 32, 0, true>(krs, koff + toff, slot + wave * NKW * 1024);
      };
      auto issue_v = [&](int u) {
        if (u >= ntiles) return;
        const uint32_t toff = (uint32_t)((t_begin + u) * BN) * (uint32_t)p.sv2 * 2u;
        const uint32_t slot = vring_lds + (uint32_t)(u % RING) * (VT_ELEMS * 2);
        buffer_load16_to_lds_blocks<NVW, 64, 0, true>(vrs, voff + toff, slot + wave * NVW * 1024);
      };
      const uint16_t* klane = kring + lane * 8;  // this lane's 16 bytes in every K block
      const uint16_t* vlane = vring + lane * 4;  // this lane's 8 bytes in every V half-block
      if constexpr (STAGES == 3) {
      STile sa, sb;
      float mxa[RT], mxb[RT];
      if (ntiles > 0) {
#pragma unroll
        for (int i = 0; i < RING; ++i) {
          issue_k(i);
          if (i + 1 < RING) issue_v(i);
        }
        wait_vm_lds_barrier<0>();
        if (wave_has_rows) {
          qk_fm(sa, qf, klane);
          qk_schedule();
          tile_max(sa, mxa);         // masks, if tile 0 needs them, come in step 0
        }
        wait_vm_lds_barrier<0>();    // every wave is done with K slot 0 before step 0 refills it
      }
      // Masks for tile u (rare: sequence end, causal diagonal) and the row max they change. The
      // steady-state step computes the max of the next tile unmasked, inside the same basic block
      // as its MFMAs; tiles that need masks redo it here.
      auto fix_masked = [&](STile& cur, float (&mx_cur)[RT], int u) {
        const int n0 = (t_begin + u) * BN;
        if (tile_needs_mask(n0, wrow0, p)) {
          mask_tile(cur, n0, wrow0, col, hh, p);
          tile_max(cur, mx_cur);
        }
      };
      // Step u of a tile that has a successor (u + 1 < ntiles).
      auto step = [&](STile& cur, float (&mx_cur)[RT], STile& nxt, float (&mx_nxt)[RT], int u) {
        issue_k(u + RING);      // into K_u's slot (read in step u-1)
        issue_v(u + RING - 1);  // into V_{u-1}'s slot (read in step u-1)
        if (wave_has_rows) {    // waves without rows still move their share of K/V
          fix_masked(cur, mx_cur, u);
          rescale(mx_cur, acc, m_use, l_i, p.c);
          u32x4 pk[KC][RT];
          exp_pack(cur, pk, m_use, l_i, p.c);
          qk_fm(nxt, qf, klane + ((u + 1) % RING) * KT_ELEMS);
          x_schedule();
          pv_fm(acc, pk, vlane + (u % RING) * VT_ELEMS);
          tile_max(nxt, mx_nxt);
          y_schedule();
        }
        // Step u+1 reads K_{u+2} and V_{u+1}. With RING = 3 they were issued in step u-1 (or
        // before the loop), and this step's loads may stay in flight.
        if (RING > 2 && u + RING < ntiles)
          wait_vm_lds_barrier<NKW + NVW>();
        else
          wait_vm_lds_barrier<0>();
      };
      // The last tile: no successor to overlap with.
      auto last = [&](STile& cur, float (&mx_cur)[RT], int u) {
        if (!wave_has_rows) return;
        fix_masked(cur, mx_cur, u);
        rescale(mx_cur, acc, m_use, l_i, p.c);
        u32x4 pk[KC][RT];
        exp_pack(cur, pk, m_use, l_i, p.c);
        pv_fm(acc, pk, vlane + (u % RING) * VT_ELEMS);
        pv_schedule();
      };
      if (ntiles > 0) {
        int u = 0;
        for (; u + 2 < ntiles; u += 2) {
          step(sa, mxa, sb, mxb, u);
          step(sb, mxb, sa, mxa, u + 1);
        }
        if (u + 1 < ntiles) {
          step(sa, mxa, sb, mxb, u);
          last(sb, mxb, u + 1);
        } else {
          last(sa, mxa, u);
        }
      }
      } else if constexpr (STAGES == 4) {
      // stages=4: two-tile-ahead pipeline. Before step u the wave holds P_u (packed) and S_{u+1}
      // (scores); step u is one block of
      //   MFMA: S_{u+2} = K_{u+2} Q^T  one for one with  O += P_u V_u
      //   VALU: masks (rare branch before the block), row max, offset update and P_{u+1} = exp(S_{u+1})
      // so the softmax VALU work spreads evenly over all of the step's MFMAs, none of which waits
      // on an MFMA of the same step except every other QK of a single score tile. A row whose
      // offset moved has O rescaled after the block (rare). K runs two tiles ahead of V: step u
      // reads K_{u+2} and V_u. Rings of RING slots: after the prologue (which reads K_0 and K_1)
      // K_{RING} and K_{RING+1} refill their slots; step u >= 1 issues K_{u+RING+1} into K_{u+1}'s
      // slot and V_{u+RING-1} into V_{u-1}'s (both read in step u-1). With RING = 3 those loads
      // stay in flight across the barrier ending step u (they are read in step u+2 or later).
      STile s0, s1;                    // scores of even / odd tiles
      u32x4 p0[KC][RT], p1[KC][RT];    // packed P of even / odd tiles
      float alpha[RT];
      const float thr = THRESH / p.c;
      auto fix_masked4 = [&](STile& cur, int u) {
        const int n0 = (t_begin + u) * BN;
        if (tile_needs_mask(n0, wrow0, p)) mask_tile(cur, n0, wrow0, col, hh, p);
      };
      if (ntiles > 0) {
#pragma unroll
        for (int i = 0; i < RING; ++i) {
          issue_k(i);
          issue_v(i);
        }
        wait_vm_lds_barrier<0>();
        if (wave_has_rows) {
          qk_fm(s0, qf, klane);
          if (ntiles > 1) qk_fm(s1, qf, klane + KT_ELEMS);
        }
        wait_vm_lds_barrier<0>();  // every wave is done with K slots 0 and 1
        issue_k(RING);
        issue_k(RING + 1);
        if (wave_has_rows) {
          fix_masked4(s0, 0);
          softmax_nb(s0, p0, m_use, l_i, alpha, p.c, thr);  // O is zero: alpha needs no rescale
        }
        // Step 0 reads K_2: with RING = 2 it was just issued (into K_0's slot), so wait for it (K_3,
        // when issued after it, may stay in flight); with RING = 3 it arrived before the prologue.
        if constexpr (RING == 2) {
          if (RING + 1 < ntiles)
            wait_vm_lds_barrier<NKW>();
          else
            wait_vm_lds_barrier<0>();
        }
      }
      // WITH_QK: tile u+2 exists. s_a: S_{u+1} (becomes P_{u+1} in p_n); s_b: receives S_{u+2};
      // p_c: P_u.
      auto step4 = [&](auto with_qk, STile& s_a, STile& s_b, u32x4 (&p_c)[KC][RT], u32x4 (&p_n)[KC][RT],
                       int u) {
        constexpr bool WITH_QK = decltype(with_qk)::value;
        const bool full_issue = u >= 1 && u + RING + 1 < ntiles;
        if (u >= 1) {
          issue_k(u + RING + 1);  // into K_{u+1}'s slot
          issue_v(u + RING - 1);  // into V_{u-1}'s slot
        }
        if (wave_has_rows) {      // waves without rows still move their share of K/V
          fix_masked4(s_a, u + 1);
          if constexpr (WITH_QK)
            qk_pv_fm(s_b, qf, klane + ((u + 2) % RING) * KT_ELEMS, acc, p_c, vlane + (u % RING) * VT_ELEMS);
          else
            pv_fm(acc, p_c, vlane + (u % RING) * VT_ELEMS);
          softmax_nb(s_a, p_n, m_use, l_i, alpha, p.c, thr);
          if constexpr (D <= 128) step_schedule<WITH_QK>();
          // P_{u+1} and l are complete here: without this the compiler sinks their VALU work past
          // the rescale branch below, out of the MFMA block it is meant to overlap.
#pragma unroll
          for (int kc = 0; kc < KC; ++kc)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) asm volatile("" : "+v"(p_n[kc][rt]));
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) asm volatile("" : "+v"(l_i[rt]));
          rescale_acc(acc, alpha);
        }
        // Step u+1 reads K_{u+3} and V_{u+1}: with RING = 3 both were issued before this step.
        if (RING > 2 && full_issue)
          wait_vm_lds_barrier<NKW + NVW>();
        else
          wait_vm_lds_barrier<0>();
      };
      auto last4 = [&](u32x4 (&p_c)[KC][RT], int u) {
        if (!wave_has_rows) return;
        pv_fm(acc, p_c, vlane + (u % RING) * VT_ELEMS);
        pv_schedule();
      };
      // Every step runs its QK MFMAs, also when tile u+2 does not exist (the second-to-last step):
      // that score tile is never used, and it costs one step's QK work per workgroup. A final step
      // without QK, or the last tile handled inside the loop, raised the kernel's register peak
      // past the file and made the compiler spill inside the steady-state loop.
      using QK = std::integral_constant<bool, true>;
      if (ntiles > 0) {
        int u = 0;  // even at the top: P_u in p0, S_{u+1} in s1
        for (; u + 2 < ntiles; u += 2) {
          step4(QK{}, s1, s0, p0, p1, u);
          step4(QK{}, s0, s1, p1, p0, u + 1);
        }
        if (u + 1 < ntiles) {
          step4(QK{}, s1, s0, p0, p1, u);
          last4(p1, u + 1);
        } else {
          last4(p0, u);
        }
      }
      } else {
      // stages=5: one KV tile per step, no cross-tile pipeline inside the wave. The wave holds one
      // score tile and reads fragments only a little ahead, so O and Q fit in its 256 registers
      // beside them (D = 256: 128 + 64) and two workgroups share a CU: the other workgroup's wave
      // on the same SIMD runs its MFMAs while this one does its softmax or waits at its barrier.
      // Tiles reach LDS by LDS-DMA into a 2-slot ring: step u issues tile u+1 into the slot tile
      // u-1 left (read in step u-1) and waits for it at the end of the step.
      static_assert(RING == 2, "stages=5 alternates two ring slots");
      if (ntiles > 0) {
        issue_k(0);
        issue_v(0);
        wait_vm_lds_barrier<0>();
      }
      for (int u = 0; u < ntiles; ++u) {
        issue_k(u + 1);
        issue_v(u + 1);
        if (wave_has_rows) {  // waves without rows still move their share of K/V
          STile s;
          u32x4 pk[KC][RT];
          qk_fm(s, qf, klane + (u & 1) * KT_ELEMS);
          qk_schedule();
          softmax(s, pk, acc, m_use, l_i, (t_begin + u) * BN, wrow0, col, hh, p);
          pv_fm(acc, pk, vlane + (u & 1) * VT_ELEMS);
          pv_schedule();
        }
        wait_vm_lds_barrier<0>();
      }
      }
    } else {
      // Double-buffered K/V tiles: tile u is computed from buffer u & 1 while tile u+1 travels
      // HBM -> registers; the registers go to the other buffer after the compute, and one barrier
      // per tile both publishes them and retires the buffer just read.
      auto kb = [&](int i) { return smem + (i & 1) * (KTILE + VTILE); };
      u32x4 pkr[PASSES], pvr[PASSES];
      if (ntiles > 0) {
        load_rows(pkr, cx.kp, cx.sk2, t_begin * BN, cx);
        load_rows(pvr, cx.vp, cx.sv2, t_begin * BN, cx);
        store_rows<KSTR>(pkr, kb(0), cx);
        store_rows<VSTR>(pvr, kb(0) + KTILE, cx);
        __syncthreads();
      }
      for (int u = 0; u < ntiles; ++u) {
        const int t = t_begin + u;
        const int n0 = t * BN;
        if (u + 1 < ntiles) {
          load_rows(pkr, cx.kp, cx.sk2, n0 + BN, cx);
          load_rows(pvr, cx.vp, cx.sv2, n0 + BN, cx);
        }
        if (active(t)) {
          STile s;
          u32x4 pk[KC][RT];
          qk(s, qf, kb(u), lane_k_off);
          qk_schedule();
          softmax(s, pk, acc, m_use, l_i, n0, wrow0, col, hh, p);
          pv(acc, pk, kb(u) + KTILE, lane_v_off);
          pv_schedule();
        }
        if (u + 1 < ntiles) {
          store_rows<KSTR>(pkr, kb(u + 1), cx);
          store_rows<VSTR>(pvr, kb(u + 1) + KTILE, cx);
        }
        __syncthreads();
      }
    }

    // Epilogue: l over both half-waves, O = acc / l.
    constexpr float kLn2 = 0.69314718055994530942f;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const float l = xhalf_sum(l_i[rt]);
      const int i = wrow0 + rt * 32 + col;
      const float inv = (l > 0.f) ? 1.f / l : 0.f;
      const float lse_val = (l > 0.f) ? (m_use[rt] * p.c + __builtin_amdgcn_logf(l)) * kLn2 : FA_NEG_INF;
      if (i < rows) {
        const int hr = row_head(i), mr = row_pos(i);
        if (SPLIT) {
          const int64_t wrow = (int64_t)(split * p.B + b) * p.H + hr;  // [split][b][h][m] rows
          float* wo = p.ws_o + (wrow * p.M + mr) * D;
#pragma unroll
          for (int dt = 0; dt < DTL; ++dt)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
              floatx4 val = {acc[dt][rt][4 * gq] * inv, acc[dt][rt][4 * gq + 1] * inv,
                             acc[dt][rt][4 * gq + 2] * inv, acc[dt][rt][4 * gq + 3] * inv};
              *reinterpret_cast<floatx4*>(wo + dt * 32 + 8 * gq + 4 * hh) = val;
            }
          if (hh == 0) p.ws_lse[wrow * p.M + mr] = lse_val;
        } else {
          uint16_t* orow = p.o + (int64_t)b * p.so0 + (int64_t)hr * p.so1 + (int64_t)mr * p.so2;
#pragma unroll
          for (int dt = 0; dt < DTL; ++dt)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
              u32x2 val = {T::pack2(acc[dt][rt][4 * gq] * inv, acc[dt][rt][4 * gq + 1] * inv),
                           T::pack2(acc[dt][rt][4 * gq + 2] * inv, acc[dt][rt][4 * gq + 3] * inv)};
              *reinterpret_cast<u32x2*>(orow + dt * 32 + 8 * gq + 4 * hh) = val;
            }
          if (p.lse != nullptr && hh == 0)
            p.lse[(int64_t)b * p.sl0 + (int64_t)hr * p.sl1 + (int64_t)mr * p.sl2] = lse_val;
        }
      }
    }
  }
};

template <typename Tag, int D, int WAVES, int RT, int BN, int STAGES, bool SPLIT>
// Workgroups per CU from kBlocksPerCu: independent workgroups sharing a CU align only their own
// waves at their barriers.
__global__ __launch_bounds__(WAVES * 64, (FwdKernel<Tag, D, WAVES, RT, BN, STAGES, SPLIT>::kBlocksPerCu)) void fa_fwd_kernel(
    FwdParams p) {
  FwdKernel<Tag, D, WAVES, RT, BN, STAGES, SPLIT>::run(p);
}

// Merge of split-KV partials. A query row's splits are shared by waves_per_row waves of the
// workgroup (1, 2 or 4; decode rows merge tens of splits, and a wave waiting on one load per split
// was latency-bound). Each wave computes the weights of its splits 64 at a time (lane s holds split
// c + s), then takes its splits in batches of 16: one readlane of the weight and one vector load of
// the partial row per split (lane l owns d = PL l .. PL l + PL - 1), all 16 loads in flight
// together. The waves of a row add their partial sums through LDS.
template <int PL>
struct MergeVec;
template <>
struct MergeVec<1> { typedef float type; };
template <>
struct MergeVec<2> { typedef float type __attribute__((ext_vector_type(2))); };
template <>
struct MergeVec<4> { typedef floatx4 type; };

template <typename Tag, int D>
__global__ __launch_bounds__(256) void fa_merge_kernel(MergeParams p) {
  typedef DT<Tag> T;
  constexpr int PL = D / 64;
  static_assert(D == 64 * PL && (PL == 1 || PL == 2 || PL == 4), "merge layout");
  typedef typename MergeVec<PL>::type fvec;
  constexpr int kBatch = 16;
  __shared__ float part_acc[4][D];
  __shared__ float part_sum[4];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wpr = p.waves_per_row;
  const int64_t rows = (int64_t)p.B * p.H * p.M;
  const int64_t row = (int64_t)blockIdx.x * (4 / wpr) + wave / wpr;
  const int part = wave % wpr;
  const bool live = row < rows;  // no early return: the waves of a row meet at a barrier
  const int64_t split_stride = rows;  // rows per split

  constexpr float kLog2e = 1.44269504088896340736f, kLn2 = 0.69314718055994530942f;
  float mx = FA_NEG_INF;
  if (live)
    for (int s = lane; s < p.splits; s += 64) mx = fmaxf(mx, p.ws_lse[s * split_stride + row]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));

  float acc[PL];
#pragma unroll
  for (int e = 0; e < PL; ++e) acc[e] = 0.f;
  float wsum = 0.f;  // this lane's splits; summed over the wave below
  const int per = (p.splits + wpr - 1) / wpr;
  const int s_begin = min(part * per, p.splits), s_end = min(s_begin + per, p.splits);
  if (live && mx != FA_NEG_INF) {
    const float* src = p.ws_o + row * D + lane * PL;
    for (int c = s_begin; c < s_end; c += 64) {
      const int s_lane = c + lane;
      const float ls = (s_lane < s_end) ? p.ws_lse[s_lane * split_stride + row] : FA_NEG_INF;
      const float w_lane = fast_exp2((ls - mx) * kLog2e);  // 0 for empty or absent splits (ls = -inf)
      wsum += w_lane;
      const int cnt = min(64, s_end - c);
      for (int j0 = 0; j0 < cnt; j0 += kBatch) {
        // indices past cnt re-read the last split (a valid address) with weight 0
        fvec o[kBatch];
        float w[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          const int j = min(j0 + u, cnt - 1);
          w[u] = (j0 + u < cnt)
                     ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w_lane), j))
                     : 0.f;
          o[u] = *reinterpret_cast<const fvec*>(src + (int64_t)(c + j) * split_stride * D);
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          if constexpr (PL == 1) {
            acc[0] += w[u] * o[u];
          } else {
#pragma unroll
            for (int e = 0; e < PL; ++e) acc[e] += w[u] * o[u][e];
          }
        }
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) wsum += __shfl_xor(wsum, off, 64);
  if (wpr > 1) {
#pragma unroll
    for (int e = 0; e < PL; ++e) part_acc[wave][lane * PL + e] = acc[e];
    if (lane == 0) part_sum[wave] = wsum;
    __syncthreads();
    if (part != 0 || !live) return;
    for (int k = 1; k < wpr; ++k) {
#pragma unroll
      for (int e = 0; e < PL; ++e) acc[e] += part_acc[wave + k][lane * PL + e];
      wsum += part_sum[wave + k];
    }
  } else if (!live) {
    return;
  }
  const int64_t bh = row / p.M;
  const int i = (int)(row % p.M);
  const float inv = (wsum > 0.f) ? 1.f / wsum : 0.f;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  uint16_t* orow = p.o + (int64_t)b * p.so0 + (int64_t)h * p.so1 + (int64_t)i * p.so2 + lane * PL;
  if constexpr (PL == 1) {
    orow[0] = T::from_float(acc[0] * inv);
  } else {
#pragma unroll
    for (int e = 0; e < PL; e += 2)
      *reinterpret_cast<uint32_t*>(orow + e) = T::pack2(acc[e] * inv, acc[e + 1] * inv);
  }
  if (p.lse != nullptr && lane == 0)
    p.lse[(int64_t)b * p.sl0 + (int64_t)h * p.sl1 + (int64_t)i * p.sl2] =
        (wsum > 0.f) ? mx + __builtin_amdgcn_logf(wsum) * kLn2 : FA_NEG_INF;
}

// ---------------------------------------------------------------------------------------------
// Registry of built instantiations.

// Itanium-mangled names of the instantiations (arguments are literal tokens, so # spells them).
#define FA_SYM_TAG_f16_t "5f16_t"
#define FA_SYM_TAG_bf16_t "6bf16_t"
#define FA_SYMBOL(TAG, D, W, RT, BN, ST, SP)                                                          \
  "_ZN2fa13fa_fwd_kernelINS_" FA_SYM_TAG_##TAG "ELi" #D "ELi" #W "ELi" #RT "ELi" #BN "ELi" #ST "ELb" #SP \
  "EEEvNS_9FwdParamsE"

#define FA_ENTRY(TAG, DTYPE, D, W, RT, BN, ST, SP)                                         \
  {ST, DTYPE, D, W, 32 * RT, BN, SP, (const void*)&fa_fwd_kernel<TAG, D, W, RT, BN, ST, (SP != 0)>, \
   FA_SYMBOL(TAG, D, W, RT, BN, ST, SP)}

#define FA_ENTRIES_D(TAG, DTYPE, D)                         \
  FA_ENTRY(TAG, DTYPE, D, 4, 1, 64, 1, 0),                  \
  FA_ENTRY(TAG, DTYPE, D, 4, 1, 64, 2, 0),                  \
  FA_ENTRY(TAG, DTYPE, D, 4, 1, 64, 2, 1)

#define FA_ENTRIES_D_WIDE(TAG, DTYPE, D)                    \
  FA_ENTRY(TAG, DTYPE, D, 4, 2, 64, 1, 0),                  \
  FA_ENTRY(TAG, DTYPE, D, 8, 1, 64, 1, 0),                  \
  FA_ENTRY(TAG, DTYPE, D, 4, 2, 64, 2, 0),                  \
  FA_ENTRY(TAG, DTYPE, D, 4, 2, 64, 2, 1),                  \
  FA_ENTRY(TAG, DTYPE, D, 8, 1, 64, 2, 0),                  \
  FA_ENTRY(TAG, DTYPE, D, 8, 1, 64, 2, 1),                  \
  FA_ENTRY(TAG, DTYPE, D, 8, 1, 128, 1, 0),                 \
  FA_ENTRY(TAG, DTYPE, D, 4, 1, 128, 1, 0),                 \
  FA_ENTRY(TAG, DTYPE, D, 8, 1, 128, 2, 0),                 \
  FA_ENTRY(TAG, DTYPE, D, 8, 1, 128, 2, 1),                 \
  FA_ENTRY(TAG, DTYPE, D, 8, 1, 64, 3, 0),                  \
  FA_ENTRY(TAG, DTYPE, D, 8, 1, 64, 3, 1),                  \
  FA_ENTRY(TAG, DTYPE, D, 4, 1, 64, 3, 0),                  \
  FA_ENTRY(TAG, DTYPE, D, 4, 1, 64, 3, 1)

// Two-tile-ahead pipelined kernels (stages=4; the 8-wave version never beat the 4-wave tiles in
// the timed sweep and is not built).
#define FA_ENTRIES_PIPE4(TAG, DTYPE, D)                     \
  FA_ENTRY(TAG, DTYPE, D, 4, 1, 64, 4, 0),                  \
  FA_ENTRY(TAG, DTYPE, D, 4, 1, 64, 4, 1)

// Lean one-tile-per-step kernels (stages=5): 64-key tiles at two workgroups per CU, 32-key tiles at
// three (D = 128) or more (D = 64).
#define FA_ENTRIES_LEAN(TAG, DTYPE, D)                      \
  FA_ENTRY(TAG, DTYPE, D, 4, 1, 64, 5, 0),                  \
  FA_ENTRY(TAG, DTYPE, D, 4, 1, 64, 5, 1),                  \
  FA_ENTRY(TAG, DTYPE, D, 4, 1, 32, 5, 0),                  \
  FA_ENTRY(TAG, DTYPE, D, 4, 1, 32, 5, 1)

// D = 256, pipelined with 32-key tiles: Q (64 registers) and O (128) leave room for two 32-key
// score tiles; a step then has the MFMA count and LDS bytes of a 64-key D = 128 step with half
// its softmax work per MFMA.
#define FA_ENTRIES_D256_PIPE(TAG, DTYPE)                    \
  FA_ENTRY(TAG, DTYPE, 256, 4, 1, 32, 3, 0),                \
  FA_ENTRY(TAG, DTYPE, 256, 4, 1, 32, 3, 1),                \
  FA_ENTRY(TAG, DTYPE, 256, 4, 1, 32, 4, 0),                \
  FA_ENTRY(TAG, DTYPE, 256, 4, 1, 32, 4, 1),                \
  FA_ENTRY(TAG, DTYPE, 256, 4, 1, 32, 5, 0),                \
  FA_ENTRY(TAG, DTYPE, 256, 4, 1, 32, 5, 1)

static const FaKernelEntry kFwdEntries[] = {
    FA_ENTRIES_D(f16_t, FA_DTYPE_F16, 64),    FA_ENTRIES_D(f16_t, FA_DTYPE_F16, 128),
    FA_ENTRIES_D(f16_t, FA_DTYPE_F16, 256),   FA_ENTRIES_D(bf16_t, FA_DTYPE_BF16, 64),
    FA_ENTRIES_D(bf16_t, FA_DTYPE_BF16, 128), FA_ENTRIES_D(bf16_t, FA_DTYPE_BF16, 256),
    FA_ENTRIES_D_WIDE(f16_t, FA_DTYPE_F16, 64), FA_ENTRIES_D_WIDE(f16_t, FA_DTYPE_F16, 128),
    FA_ENTRIES_D_WIDE(bf16_t, FA_DTYPE_BF16, 64), FA_ENTRIES_D_WIDE(bf16_t, FA_DTYPE_BF16, 128),
    FA_ENTRIES_D256_PIPE(f16_t, FA_DTYPE_F16), FA_ENTRIES_D256_PIPE(bf16_t, FA_DTYPE_BF16),
    FA_ENTRIES_PIPE4(f16_t, FA_DTYPE_F16, 64),  FA_ENTRIES_PIPE4(f16_t, FA_DTYPE_F16, 128),
    FA_ENTRIES_PIPE4(bf16_t, FA_DTYPE_BF16, 64), FA_ENTRIES_PIPE4(bf16_t, FA_DTYPE_BF16, 128),
    FA_ENTRIES_LEAN(f16_t, FA_DTYPE_F16, 64),   FA_ENTRIES_LEAN(f16_t, FA_DTYPE_F16, 128),
    FA_ENTRIES_LEAN(bf16_t, FA_DTYPE_BF16, 64), FA_ENTRIES_LEAN(bf16_t, FA_DTYPE_BF16, 128),
};

static const FaMergeEntry kMergeEntries[] = {
    {FA_DTYPE_F16, 64, (const void*)&fa_merge_kernel<f16_t, 64>},
    {FA_DTYPE_F16, 128, (const void*)&fa_merge_kernel<f16_t, 128>},
    {FA_DTYPE_F16, 256, (const void*)&fa_merge_kernel<f16_t, 256>},
    {FA_DTYPE_BF16, 64, (const void*)&fa_merge_kernel<bf16_t, 64>},
    {FA_DTYPE_BF16, 128, (const void*)&fa_merge_kernel<bf16_t, 128>},
    {FA_DTYPE_BF16, 256, (const void*)&fa_merge_kernel<bf16_t, 256>},
};

const FaKernelEntry* fa_fwd_registry(int* count) {
  *count = (int)(sizeof(kFwdEntries) / sizeof(kFwdEntries[0]));
  return kFwdEntries;
}

const FaMergeEntry* fa_merge_registry(int* count) {
  *count = (int)(sizeof(kMergeEntries) / sizeof(kMergeEntries[0]));
  return kMergeEntries;
}

}  // namespace fa
