// Attention forward with v_mfma_f32_16x16x32 tiles (stages=6): the lean one-KV-tile-per-step
// pipeline (stages=5) rebuilt around 16x16 MFMA tiles.
//
// Same algorithm as fa_fwd.hip (reference flash_atten.py:14-50 / 136-172 / 261-275: online
// softmax over KV tiles in the exp2 domain with a lazily moved row offset, P rounded to the input
// dtype before P V, O normalised by the row sum at the end; causal top-left; GQA by head index;
// split-KV partials + LSE merge for the sliced variant). What changes is the matrix-core shape:
//  * 16x16x32 MFMAs move half the accumulator registers per flop of 32x32x16 ones. The attention
//    kernels run at the chip's power cap (MFMA busy ~0.6 at 1.5-1.7 GHz); in the GEMM the same
//    switch raised the clock of the power-capped 8-wave tiles from ~1.5 to ~1.8 GHz.
//  * Scores are S^T = K Q^T per 16-key x 16-query tile: lane l holds query (l & 15) and keys
//    4 (l >> 4) + 0..3, so a query's row max / sum spans the four 16-lane rows of the wave (two
//    permlane swaps). Each wave owns 32 query rows as two 16-query tiles.
//  * P feeds P V straight from the score registers. For 32 keys (score tiles 2c, 2c+1) a lane holds
//    keys {4g .. 4g+3} and {16+4g .. 16+4g+3} (g = l >> 4) of its query: those 8 values are its B
//    operand (MFMA k index 8g + e), and the V^T A operand is built to match: two transposing reads
//    whose 16-lane group g addresses rows 4g.. and 16+4g.. of the 32-key chunk.
//  * The pipelined binary16 kernels take the row sum l from P V itself: one more MFMA per 32-key
//    chunk and query tile, with an all-ones A operand, leaves every lane its query's sum.
//  * K and V tiles reach LDS by LDS-DMA in fragment-major order (every 1 KiB block is exactly what
//    one read instruction of the wave reads), into a 2-slot ring, as in stages=5.
#include <type_traits>

#include "fa_common.h"
#include "fa_kernels.h"
#include "../../include/fa_gfx950.h"

namespace fa {

// PIPE 0 (stages=6): one KV tile per step. PIPE 1 (stages=7): the stages=3 software pipeline --
// the QK MFMAs of tile u+1 beside the exp / pack VALU work of tile u, then the PV MFMAs of tile u
// beside the row max of tile u+1.
template <typename Tag, int D, int WAVES, int BN, int PIPE, bool SPLIT>
struct Fwd16 {
  static constexpr int THREADS = WAVES * 64;
  static constexpr int QT = 2;            // 16-query tiles per wave
  static constexpr int ROWS = 16 * QT;    // query rows per wave
  static constexpr int BM = WAVES * ROWS;
  static constexpr int DC = D / 32;       // 32-deep d chunks of Q K^T
  static constexpr int DTL = D / 16;      // 16-row d tiles of O^T
  static constexpr int JT = BN / 16;      // 16-key score tiles
  static constexpr int KC = BN / 32;      // 32-key chunks of P V
  static constexpr int NKB = JT * DC;     // 1 KiB K blocks per tile
  static constexpr int NVB = KC * DTL;    // 1 KiB V blocks per tile
  static constexpr int KT_ELEMS = NKB * 512;
  static constexpr int VT_ELEMS = NVB * 512;
  static constexpr int NKW = NKB / WAVES;  // DMA blocks per wave per tile
  static constexpr int NVW = NVB / WAVES;
  static constexpr float THRESH = 8.0f;    // lazy-rescale threshold (log2 units)
  static constexpr bool kSumRounded = __is_same(Tag, f16_t);
  // Pipelined binary16 kernels: the row sum l comes from one more MFMA per (32-key chunk, query
  // tile) whose A operand is all ones, so every lane ends with its query's full sum of the rounded
  // P (the same sum the VALU dot2 path forms) and the step's VALU work loses 16 ops. bfloat16 keeps
  // the fp32 sum of the unrounded P.
  static constexpr bool kSumMfma = PIPE && __is_same(Tag, f16_t);
  static_assert(D % 32 == 0 && BN % 32 == 0, "tile shape");
  static_assert(NKB % WAVES == 0 && NVB % WAVES == 0, "tile blocks must split evenly over waves");
  static_assert(DC % NKW == 0 && DTL % NVW == 0, "a wave's DMA blocks stay in one key group");
  static_assert(BM % BN == 0, "causal tile bound assumes block_m % block_n == 0");
  // Workgroups per CU the launch bounds ask for: the one-tile-per-step kernel with 32-key tiles at
  // D <= 128 fits three (LDS and registers), the others two (the pipelined kernel holds two score
  // tiles).
  static constexpr int kBlocksPerCu = PIPE >= 2 ? 1 : (!PIPE && BN == 32 && D <= 128) ? 3 : 2;
  static_assert(PIPE < 2 || WAVES == 8, "the ping-pong kernels run two groups of four waves");
  // Q fragments of the workgroup's rows in LDS (persistent kernel): block (wave, qt, cc) of 1 KiB
  // holds, at byte 16 l, Q[row wave*ROWS + 16 qt + (l & 15)][32 cc + 8 (l >> 4) .. +7] -- lane l's qf.
  static constexpr int QB_ELEMS = PIPE == 3 ? WAVES * QT * DC * 512 : 0;
  static constexpr int kQChunks = 4;  // steps over which the persistent kernel prefetches the next Q
  // O leaves in 64-byte row pieces (pack_o_wide) except from the kernels held to three workgroups
  // per CU, whose register cap the extra swap registers would exceed (they spilled).
  static constexpr bool kWideO = !SPLIT && kBlocksPerCu < 3;
  static constexpr bool kScalarIds = BN == 64 && PIPE != 1;

  typedef DT<Tag> T;
  typedef floatx4 STile[JT][QT];
  typedef floatx4 OAcc[DTL][QT];

  // S^T tiles of one KV tile from its fragment-major K slot: block (jt, cc) holds, at byte 16 l,
  // K[jt*16 + (l & 15)][cc*32 + 8 (l >> 4) .. +7] (the MFMA A operand of lane l).
  __device__ static inline void qk(STile& s, const u32x4 (&qf)[QT][DC], const uint16_t* kslot_lane) {
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < DC; ++cc) {
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) {
        const u32x4 kf = *reinterpret_cast<const u32x4*>(kslot_lane + (jt * DC + cc) * 512);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) s[jt][qt] = T::mfma16(kf, qf[qt][cc], cc == 0 ? zero : s[jt][qt]);
      }
    }
  }

  // O^T += V^T P^T from the fragment-major V slot: block (kc, dt) holds the two transposing reads of
  // that (32-key chunk, 16-column d tile); in read `half` lane L's 8 bytes (at 8 L) are
  // V[kc*32 + 16 half + 4 (L >> 4) + ((L & 15) >> 2)][dt*16 + 4 (L & 3) .. +3].
  __device__ static inline void pv(OAcc& acc, const u32x4 (&pk)[KC][QT], const uint16_t* vslot_lane,
                                   floatx4 (&lsum)[QT]) {
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      if constexpr (kSumMfma) {
        constexpr uint32_t one2 = __is_same(Tag, f16_t) ? 0x3c003c00u : 0x3f803f80u;
        const u32x4 ones = {one2, one2, one2, one2};
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) lsum[qt] = T::mfma16(ones, pk[kc][qt], lsum[qt]);
      }
#pragma unroll
      for (int dt = 0; dt < DTL; ++dt) {
        const uint16_t* base = vslot_lane + (kc * DTL + dt) * 512;
        const u32x2 lo = lds_read_tr16(base);
        const u32x2 hi = lds_read_tr16(base + 256);
        const u32x4 vf = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) acc[dt][qt] = T::mfma16(vf, pk[kc][qt], acc[dt][qt]);
      }
    }
  }

  // Keys past N, and (causal) keys after the query row, get score -inf. Wave-uniform test first.
  __device__ static inline bool tile_needs_mask(int n0, int wrow0, const FwdParams& p) {
    return (n0 + BN > p.N) || (p.causal && n0 + BN - 1 > wrow0);
  }
  // Key j of query i is kept when j < lim_i = N (or min(N, i + 1) causal). Each element takes a
  // sign-bit mask and a bitfield select -- vector ALU only: per-element compares would each hold a
  // scalar register pair, and the scheduler hoists all 32 of them.
  __device__ static inline void mask_tile(STile& s, int n0, int wrow0, int q16, int g, const FwdParams& p) {
    const uint32_t ninf = __float_as_uint(FA_NEG_INF);
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int i = wrow0 + qt * 16 + q16;
      const int lim = p.causal ? min(p.N, i + 1) : p.N;
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) {
        const int rel = lim - (n0 + jt * 16 + 4 * g);  // keys r < rel of this lane are kept
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t keep = (uint32_t)((r - rel) >> 31);  // all ones when r < rel
          s[jt][qt][r] = __uint_as_float((__float_as_uint(s[jt][qt][r]) & keep) | (ninf & ~keep));
        }
      }
    }
  }

  // Max of a score tile over this lane's keys of each query (a quarter of the row: the row's max
  // over the four lane rows is formed only when the offset moves, in rescale). A chain that takes
  // two scores per step (v_max3_f32): 4·JT/2 ops per query tile, where a tree per key tile costs more.
  __device__ static inline void tile_max(const STile& s, float (&mx)[QT]) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float m = fmaxf(s[0][qt][0], s[0][qt][1]);
      m = fmaxf(fmaxf(m, s[0][qt][2]), s[0][qt][3]);
#pragma unroll
      for (int jt = 1; jt < JT; ++jt) {
        m = fmaxf(fmaxf(m, s[jt][qt][0]), s[jt][qt][1]);
        m = fmaxf(fmaxf(m, s[jt][qt][2]), s[jt][qt][3]);
      }
      mx[qt] = m;
    }
  }

  // O and l of query tile qt times alpha.
  __device__ static inline void scale_row(int qt, float alpha, OAcc& acc, float (&l_i)[QT], floatx4 (&lsum)[QT]) {
    if constexpr (kSumMfma) {
#pragma unroll
      for (int r = 0; r < 4; ++r) lsum[qt][r] *= alpha;
    } else {
      l_i[qt] *= alpha;
    }
#pragma unroll
    for (int dt = 0; dt < DTL; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[dt][qt][r] *= alpha;
  }
  // Exponent offsets of a wave's QT query tiles: m in score units (-inf before the first tile),
  // and two values derived from it: mc(c) = m c (0 while m is -inf), the offset every score's FMA
  // subtracts, and thr(c) = m + THRESH / c, the bound of the rescale test. The ping-pong kernels,
  // whose softmax phase is VALU-bound, keep both and update them only when the offset moves
  // (rare; measured 0.4-0.7% faster non-causal); the others take them per step (the 256-dimension
  // kernel at its register cap ran 4.5% slower keeping them).
  static constexpr bool kCachedOff = PIPE >= 2;
  struct RowOff {
    float m[QT], mc_[kCachedOff ? QT : 1], thr_[kCachedOff ? QT : 1];
    __device__ inline void reset() {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        m[qt] = FA_NEG_INF;
        if constexpr (kCachedOff) {
          mc_[qt] = 0.f;
          thr_[qt] = FA_NEG_INF;
        }
      }
    }
    __device__ inline void set(int qt, float m_new, float c) {
      m[qt] = m_new;
      if constexpr (kCachedOff) {
        mc_[qt] = (m_new == FA_NEG_INF) ? 0.f : m_new * c;
        thr_[qt] = m_new + THRESH / c;
      }
    }
    __device__ inline float mc(int qt, float c) const {
      if constexpr (kCachedOff) return mc_[qt];
      else return (m[qt] == FA_NEG_INF) ? 0.f : m[qt] * c;
    }
    __device__ inline float thr(int qt, float c) const {
      if constexpr (kCachedOff) return thr_[qt];
      else return m[qt] + THRESH / c;
    }
  };

  // Lazy rescale: move the exponent offset (and rescale O and l) only when some lane of the wave
  // sees a score more than THRESH (log2 units) above it; the moved offset is the row max over the
  // four lane rows, so the lanes of a query keep one offset. One ballot over all query tiles guards
  // the per-tile tests, so a step that moves no offset (the common case) takes a single branch.
  __device__ static inline void rescale(const float (&mx)[QT], OAcc& acc, RowOff& ro, float (&l_i)[QT],
                                        floatx4 (&lsum)[QT], float c) {
    bool need[QT], any = false;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      need[qt] = mx[qt] > ro.thr(qt, c);
      any |= need[qt];
    }
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(any) == 0, 1)) return;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      if (__builtin_amdgcn_ballot_w64(need[qt]) != 0) {
        const float m_new = fmaxf(ro.m[qt], xquad_max(mx[qt]));
        const float alpha = (ro.m[qt] == FA_NEG_INF) ? 0.f : fast_exp2((ro.m[qt] - m_new) * c);
        ro.set(qt, m_new, c);
        scale_row(qt, alpha, acc, l_i, lsum);
      }
    }
  }

  // Online softmax of one score tile: masks where needed, row max, lazy rescale, then P.
  __device__ static inline void softmax(STile& s, u32x4 (&pk)[KC][QT], OAcc& acc, RowOff& ro,
                                        float (&l_i)[QT], floatx4 (&lsum)[QT], int n0, int wrow0, int q16, int g,
                                        const FwdParams& p) {
    if (tile_needs_mask(n0, wrow0, p)) mask_tile(s, n0, wrow0, q16, g, p);
    float mx[QT];
    tile_max(s, mx);
    rescale(mx, acc, ro, l_i, lsum, p.c);
    exp_pack(s, pk, ro, l_i, p.c);
  }

  // P = exp2(S c - m c) rounded to the input dtype and packed as the B operand of P V; the row
  // sum l accumulates the same P.
  __device__ static inline void exp_pack(const STile& s, u32x4 (&pk)[KC][QT], const RowOff& ro,
                                         float (&l_i)[QT], float c) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const float mc = ro.mc(qt, c);
      float l0 = 0.f, l1 = 0.f;
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int half = 0; half < 2; ++half)
#pragma unroll
          for (int w = 0; w < 2; ++w) {
            const floatx4& t = s[2 * kc + half][qt];
            const float e0 = fast_exp2(__builtin_fmaf(t[2 * w], c, -mc));
            const float e1 = fast_exp2(__builtin_fmaf(t[2 * w + 1], c, -mc));
            const uint32_t pw = T::pack2(e0, e1);
            pk[kc][qt][2 * half + w] = pw;
            if (kSumMfma) {
              // l comes from the ones-row MFMA in pv
            } else if (kSumRounded) {
              // binary16 P: summing the rounded pair moves l by <= 2^-12 relative
              if (w) l1 = dot2_sum<Tag>(pw, l1);
              else l0 = dot2_sum<Tag>(pw, l0);
            } else {
              // bfloat16 P is too coarse for l: sum the fp32 values
              if (w) l1 += e0 + e1;
              else l0 += e0 + e1;
            }
          }
      if (!kSumMfma) l_i[qt] += l0 + l1;
    }
  }

  // Scheduling hints: LDS fragment reads a few MFMAs ahead of their use.
  __device__ static inline void qk_schedule() {
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // DS read
#pragma unroll
    for (int i = 0; i < DC * JT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, QT, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
    }
  }
  __device__ static inline void pv_schedule() {
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
#pragma unroll
    for (int i = 0; i < KC * DTL; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, QT, 1);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
    }
  }
  // Ping-pong matrix block (QK of the next tile, then PV of this one, one scheduling region): AHEAD
  // LDS reads first, then the remaining K and V fragment reads spread evenly over the MFMA groups.
  template <int I, int G, int NR>
  __device__ static inline void m_schedule_groups() {
    if constexpr (I < G) {
      __builtin_amdgcn_sched_group_barrier(0x008, QT, 3);
      constexpr int r = (NR * (I + 1)) / G - (NR * I) / G;
      if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 3);
      m_schedule_groups<I + 1, G, NR>();
    }
  }
  template <int AHEAD>
  __device__ static inline void m_schedule() {
    constexpr int reads = DC * JT + 2 * KC * DTL;
    __builtin_amdgcn_sched_group_barrier(0x100, AHEAD, 3);
    m_schedule_groups<0, DC * JT + KC * DTL, reads - AHEAD>();
  }
  // Pipelined step, first half: the next tile's QK MFMAs with this tile's exp / pack / sum VALU work
  // (FMA + exp per score, pack + sum per pair), a few VALU ops per group of QT MFMAs.
  static constexpr int kExpValu = QT * JT * (4 * 2 + 2 * (kSumMfma ? 1 : 2));
  static constexpr int kXValuPerMfma = (kExpValu + DC * JT - 1) / (DC * JT);
  __device__ static inline void x_schedule() {
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 2);
#pragma unroll
    for (int i = 0; i < DC * JT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, QT, 2);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 2);
      __builtin_amdgcn_sched_group_barrier(0x002, kXValuPerMfma, 2);
    }
  }
  // Second half: this tile's PV MFMAs with the next tile's row max.
  __device__ static inline void y_schedule() {
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 2);
#pragma unroll
    for (int i = 0; i < KC * DTL; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, QT, 2);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 2);
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 2);
    }
  }

  // Epilogue of one work item of the persistent kernel (the same code as the end of run(), which
  // keeps its copy inline: called there, even always-inlined, it pushed the 32-key one-tile-per-step
  // kernel past its 168-VGPR cap into scratch). l over the four lane rows, O = acc / l; lane holds
  // d = 16 dt + 4 g .. +3. The output parameters are read from the kernel-argument segment (scalar
  // loads at the point of use); fa_fwd16_kernel takes FwdParams as its only argument (checked there).
  __device__ __attribute__((always_inline)) static inline void store_out(const OAcc& acc, const RowOff& ro, const float (&l_i)[QT],
                                          const floatx4 (&lsum)[QT], int wrow0, int q16, int g, int rows, int b, int h,
                                          int split_u) {
    const auto pe = kernarg_params<FwdParams>();
    constexpr float kLn2 = 0.69314718055994530942f;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const float l = kSumMfma ? lsum[qt][0] : xquad_sum(l_i[qt]);
      const int i = wrow0 + qt * 16 + q16;
      const float inv = (l > 0.f) ? 1.f / l : 0.f;
      const float lse_val = (l > 0.f) ? (ro.m[qt] * pe->c + __builtin_amdgcn_logf(l)) * kLn2 : FA_NEG_INF;
      u32x4 wide[DTL / 2];
      if constexpr (kWideO) pack_o_wide(acc, qt, inv, wide);  // cross-lane: before the row test
      if (i < rows) {
        const int hr = pe->pack > 1 ? h + i / pe->M : h;
        const int mr = pe->pack > 1 ? i % pe->M : i;
        if (SPLIT) {
          const int64_t wrow = (int64_t)(split_u * pe->B + b) * pe->H + hr;  // [split][b][h][m] rows
          float* wo = pe->ws_o + (wrow * pe->M + mr) * D;
#pragma unroll
          for (int dt = 0; dt < DTL; ++dt) {
            floatx4 val = {acc[dt][qt][0] * inv, acc[dt][qt][1] * inv, acc[dt][qt][2] * inv, acc[dt][qt][3] * inv};
            *reinterpret_cast<floatx4*>(wo + dt * 16 + 4 * g) = val;
          }
          if (g == 0) pe->ws_lse[wrow * pe->M + mr] = lse_val;
        } else {
          uint16_t* orow = pe->o + (int64_t)b * pe->so0 + (int64_t)hr * pe->so1 + (int64_t)mr * pe->so2;
          if constexpr (kWideO) {
#pragma unroll
            for (int pp = 0; pp < DTL / 2; ++pp)
              *reinterpret_cast<u32x4*>(orow + 32 * pp + wide_col(g)) = wide[pp];
          } else {
#pragma unroll
            for (int dt = 0; dt < DTL; ++dt) {
              u32x2 val = {T::pack2(acc[dt][qt][0] * inv, acc[dt][qt][1] * inv),
                           T::pack2(acc[dt][qt][2] * inv, acc[dt][qt][3] * inv)};
              *reinterpret_cast<u32x2*>(orow + dt * 16 + 4 * g) = val;
            }
          }
          float* lse = pe->lse;
          if (lse != nullptr && g == 0)
            lse[(int64_t)b * pe->sl0 + (int64_t)hr * pe->sl1 + (int64_t)mr * pe->sl2] = lse_val;
        }
      }
    }
  }

  // O of query tile qt (times inv), rounded, as 16-byte lane chunks. The accumulator gives lane row g
  // (lanes 16 g .. 16 g + 15) columns d = 16 dt + 4 g .. +3 of each d tile, so a store per tile
  // writes 32 bytes of each of 16 rows, and every such half line is an L2 request of its own. One
  // v_permlane16_swap per dword of tiles 2 pp and 2 pp + 1 (it swaps the odd 16-lane rows of one
  // operand with the even rows of the other) leaves lane row g holding 8 consecutive columns of the
  // pair, starting at 32 pp + wide_col(g): each store then writes 64 contiguous bytes of each row,
  // half the store instructions and L2 requests. Cross-lane: call with every lane active.
  __device__ static inline void pack_o_wide(const OAcc& acc, int qt, float inv, u32x4 (&wide)[DTL / 2]) {
    static_assert(DTL % 2 == 0, "d tiles pair up");
#pragma unroll
    for (int pp = 0; pp < DTL / 2; ++pp) {
      const floatx4& a = acc[2 * pp][qt];
      const floatx4& b = acc[2 * pp + 1][qt];
      const auto lo = __builtin_amdgcn_permlane16_swap(T::pack2(a[0] * inv, a[1] * inv), T::pack2(b[0] * inv, b[1] * inv),
                                                       false, false);
      const auto hi = __builtin_amdgcn_permlane16_swap(T::pack2(a[2] * inv, a[3] * inv), T::pack2(b[2] * inv, b[3] * inv),
                                                       false, false);
      wide[pp] = (u32x4){lo[0], hi[0], lo[1], hi[1]};
    }
  }
  // First column, within a pair of d tiles, of lane row g's chunk: rows 0..3 hold tile 2 pp's
  // columns 0..7, tile 2 pp + 1's 0..7, tile 2 pp's 8..15, tile 2 pp + 1's 8..15.
  __device__ static inline int wide_col(int g) { return 8 * (((g & 1) << 1) | (g >> 1)); }

  // ---- persistent ping-pong (stages=9) ----------------------------------------------------------
  // One workgroup per CU walks a fixed sequence of work items (the logical blocks of run()). The
  // sequence is a snake over the XCD's slots: item k of XCD x goes to slot k % S in round k / S,
  // slots reversed in odd rounds, so that with heaviest-first causal blocks each slot's rounds pair
  // a heavy block with a light one. Within an item the schedule is run()'s ping-pong; across items
  // the K/V rings keep running: the last two steps of an item fetch the next item's K_0, K_1 and
  // V_0 into the slots the ring frees, and its first steps fetch the next item's Q into an LDS
  // buffer (each wave's own fragments, in kQChunks pieces), so an item starts without waiting on
  // memory.
  // A work item: its logical block (decoded to batch, head and split where needed: few scalar
  // registers stay live across the KV loop), first query row and KV tile range.
  struct Item {
    int pid, m0, t_begin, ntiles;
  };
  struct Ids {
    int b, h, hk, split;
  };
  template <class P>
  __device__ static inline Ids decode(int pid, const P& p) {
    const int rest = pid / p.m_blocks;
    const int bh = rest / p.splits;
    Ids ids;
    ids.split = __builtin_amdgcn_readfirstlane(rest % p.splits);
    ids.b = __builtin_amdgcn_readfirstlane(bh / p.H);
    ids.h = __builtin_amdgcn_readfirstlane(bh % p.H);
    ids.hk = __builtin_amdgcn_readfirstlane(ids.h / p.group);
    return ids;
  }
  // Buffer descriptors of an item's K and V rows (its (batch, kv head)) and Q rows (batch, head).
  template <class P>
  __device__ static inline u32x4 k_rsrc(const Ids& d, const P& p) {
    return make_rsrc(p.k + (int64_t)d.b * p.sk0 + (int64_t)d.hk * p.sk1, (uint32_t)p.N * (uint32_t)p.sk2 * 2u);
  }
  template <class P>
  __device__ static inline u32x4 v_rsrc(const Ids& d, const P& p) {
    return make_rsrc(p.v + (int64_t)d.b * p.sv0 + (int64_t)d.hk * p.sv1, (uint32_t)p.N * (uint32_t)p.sv2 * 2u);
  }
  template <class P>
  __device__ static inline u32x4 q_rsrc(const Ids& d, const P& p) {
    return make_rsrc(p.q + (int64_t)d.b * p.sq0 + (int64_t)d.h * p.sq1, (uint32_t)p.M * (uint32_t)p.sq2 * 2u);
  }
  // Logical block of round r for workgroup w of G, or -1 past the end of its sequence.
  __device__ static inline int item_pid(int r, int w, int G, int total) {
    int x = 0, slot = w, S = G, per = total;
    if ((total & 7) == 0 && (G & 7) == 0) {  // XCD x = w % 8 walks logical blocks [x per, (x+1) per)
      x = w & 7;
      slot = w >> 3;
      S = G >> 3;
      per = total >> 3;
    }
    const int k = r * S + ((r & 1) ? S - 1 - slot : slot);
    return k < per ? x * per + k : -1;
  }
  template <class P>
  __device__ static inline Item make_item(int pid, const P& p) {
    Item it;
    it.pid = pid;
    int mb = pid % p.m_blocks;
    if (p.causal) mb = p.m_blocks - 1 - mb;  // heaviest query blocks first, as run()
    it.m0 = __builtin_amdgcn_readfirstlane(mb) * BM;
    const int split = (pid / p.m_blocks) % p.splits;
    it.t_begin = __builtin_amdgcn_readfirstlane(split * p.tiles_per_split);
    int n_end = (it.t_begin + p.tiles_per_split) * BN;
    if (n_end > p.N) n_end = p.N;
    if (p.causal && n_end > it.m0 + BM) n_end = it.m0 + BM;
    const int t_end = (n_end + BN - 1) / BN;
    it.ntiles = __builtin_amdgcn_readfirstlane(t_end > it.t_begin ? t_end - it.t_begin : 0);
    return it;
  }

  template <int GRP>
  __device__ static void persistent_group(const FwdParams& p, uint16_t* smem, int lane, int wave, int first_pid) {
    // lane-derived values are computed inside each group's copy of the loop: shared ones, hoisted
    // above the group branch, stayed live across group 0's loop and spilled
    asm volatile("" : "+v"(lane));
    const int q16 = lane & 15, g = lane >> 4;
    // workgroup id and count from the builtin and the host (blockIdx / gridDim go through library
    // calls that this build does not inline, whose results the compiler cannot prove uniform)
    const int G = p.grid, w = (int)__builtin_amdgcn_workgroup_id_x();
    // per-lane DMA offsets (item-independent): K, V as run(); Q rows of this wave within an item
    uint32_t koff, voff;
    {
      const int blk = wave * NKW, jt = blk / DC, cc = blk % DC;
      const uint32_t row = jt * 16 + (lane & 15), c0 = cc * 32 + 8 * (lane >> 4);
      koff = (row * (uint32_t)p.sk2 + c0) * 2u;
    }
    {
      const int blk = wave * NVW, kc = blk / DTL, dt = blk % DTL;
      const int m = lane;
      const uint32_t row = kc * 32 + 16 * (m >> 5) + 4 * ((m & 31) >> 3) + ((m & 7) >> 1);
      const uint32_t c0 = dt * 16 + 8 * (m & 1);
      voff = (row * (uint32_t)p.sv2 + c0) * 2u;
    }
    uint32_t qoff[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
      qoff[qt] = ((uint32_t)(wave * ROWS + qt * 16 + q16) * (uint32_t)p.sq2 + 8 * g) * 2u;
    uint16_t* kring = smem;
    uint16_t* vring = smem + 2 * KT_ELEMS;
    const uint16_t* qbuf = smem + 2 * (KT_ELEMS + VT_ELEMS);
    const uint32_t kring_lds = lds_address(smem), vring_lds = kring_lds + 2 * KT_ELEMS * 2;
    const uint32_t qbuf_lds = kring_lds + 2 * (KT_ELEMS + VT_ELEMS) * 2;
    const uint16_t* klane = kring + lane * 8;
    const uint16_t* vlane = vring + lane * 4;
    const uint16_t* qlane = qbuf + (wave * QT * DC) * 512 + lane * 8;

    // bytes between consecutive KV tiles of K and of V (the host keeps them below 2^32); a tile's
    // offset moves the buffer resource (slab_rsrc), so the lanes' offsets koff / voff stay fixed
    const uint32_t kstep = (uint32_t)BN * (uint32_t)p.sk2 * 2u, vstep = (uint32_t)BN * (uint32_t)p.sv2 * 2u;
    // Item-level parameters (pointers, strides, grid shape) are read through a fresh kernel-
    // argument pointer at each item boundary rather than held in scalar registers across the KV
    // loop: held there, they pushed the loop's own scalars out, and the compiler re-read strides
    // with scalar loads inside the loop, whose waits (lgkmcnt, shared with LDS reads) then
    // serialised every LDS fragment read.
    Item cur = make_item(first_pid, *kernarg_params<FwdParams>());
    int par = 0;              // ring slot of the current item's tile 0
    bool prefetched = false;  // its Q, K_0, K_1, V_0 were fetched by the previous item
    for (int r = 0;; ++r) {
      const auto pi = kernarg_params<FwdParams>();
      const int pid_n = item_pid(r + 1, w, pi->grid, pi->total_blocks);
      Item nxt;
      if (pid_n >= 0) {
        nxt = make_item(pid_n, *pi);
      } else {
        nxt = cur;
        nxt.ntiles = 0;
      }
      const int ntiles = cur.ntiles;
      const u32x4 krs = k_rsrc(decode(cur.pid, *pi), *pi), vrs = v_rsrc(decode(cur.pid, *pi), *pi);
      const int wrow0 = cur.m0 + wave * ROWS;
      const bool wave_has_rows = wrow0 < p.M;
      // Tile u of the current item, or tile u - ntiles of the next one (K up to the next item's
      // tile 1, V up to its tile 0), into ring slot (par + u) & 1.
      // (The next item's branch builds its descriptors there, in the two steps per item that take
      // it; the empty asm keeps the compiler from merging the two branches' loads into one, which
      // would build those descriptors on every step.)
      auto issue_k = [&](int u) {
        const uint32_t slot = kring_lds + (uint32_t)((par + u) & 1) * (KT_ELEMS * 2) + wave * NKW * 1024;
        if (__builtin_expect(u < ntiles, 1)) {
          buffer_load16_to_lds_blocks<NKW, 64>(slab_rsrc(krs, (uint32_t)(cur.t_begin + u) * kstep, true), koff, slot);
        } else if (u - ntiles < nxt.ntiles) {
          asm volatile("");
          const uint32_t toff = (uint32_t)(nxt.t_begin + u - ntiles) * kstep;
          const auto pn = kernarg_params<FwdParams>();
          buffer_load16_to_lds_blocks<NKW, 64>(slab_rsrc(k_rsrc(decode(nxt.pid, *pn), *pn), toff, true), koff, slot);
        }
      };
      auto issue_v = [&](int u) {
        const uint32_t slot = vring_lds + (uint32_t)((par + u) & 1) * (VT_ELEMS * 2) + wave * NVW * 1024;
        if (__builtin_expect(u < ntiles, 1)) {
          buffer_load16_to_lds_blocks<NVW, 32>(slab_rsrc(vrs, (uint32_t)(cur.t_begin + u) * vstep, true), voff, slot);
        } else if (u - ntiles < nxt.ntiles) {
          asm volatile("");
          const uint32_t toff = (uint32_t)(nxt.t_begin + u - ntiles) * vstep;
          const auto pn = kernarg_params<FwdParams>();
          buffer_load16_to_lds_blocks<NVW, 32>(slab_rsrc(v_rsrc(decode(nxt.pid, *pn), *pn), toff, true), voff, slot);
        }
      };
      auto issue_q = [&](const Item& it) {
        const auto pq = kernarg_params<FwdParams>();
        const uint32_t moff = (uint32_t)it.m0 * (uint32_t)pq->sq2 * 2u;
        const u32x4 qrs = q_rsrc(decode(it.pid, *pq), *pq);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
          buffer_load16_to_lds_blocks<DC, 64>(qrs, qoff[qt] + moff, qbuf_lds + ((wave * QT + qt) * DC) * 1024);
      };
      // Chunk c (of kQChunks) of this wave's QT * DC Q blocks of item `it`. Every workgroup starts
      // its items at about the same time, so the whole chip's next-item Q fetch issued in one step
      // (64 KiB per workgroup) made that step wait on HBM; in chunks over the item's first steps
      // it hides behind their K/V traffic (measured 1-4% faster; 8 chunks were slower than 4).
      auto issue_q_chunk = [&](const Item& it, int c) {
        const auto pq = kernarg_params<FwdParams>();
        const uint32_t moff = (uint32_t)it.m0 * (uint32_t)pq->sq2 * 2u;
        const u32x4 qrs = q_rsrc(decode(it.pid, *pq), *pq);
#pragma unroll
        for (int bq = 0; bq < QT * DC; ++bq) {
          if (bq * kQChunks / (QT * DC) == c) {
            const int qt = bq / DC, cc = bq % DC;
            buffer_load16_to_lds(qrs, qoff[qt] + moff + cc * 64, qbuf_lds + ((wave * QT + qt) * DC + cc) * 1024);
          }
        }
      };
      auto kslot = [&](int u) { return klane + ((par + u) & 1) * KT_ELEMS; };
      auto vslot = [&](int u) { return vlane + ((par + u) & 1) * VT_ELEMS; };

      OAcc acc;
      RowOff ro;
      ro.reset();
      float l_i[QT];
      floatx4 lsum[QT];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        l_i[qt] = 0.f;
        lsum[qt] = (floatx4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dt = 0; dt < DTL; ++dt) acc[dt][qt] = (floatx4){0.f, 0.f, 0.f, 0.f};
      }
      if (ntiles > 0) {
        // DMA over an item of T tiles: K 0..T+1 and V 0..T (tiles past T - 1 are the next item's).
        // The previous item fetched this one's K_0, V_0 and, when T >= 2, K_1; with T == 1 this
        // item's K_1 is the next item's K_0, fetched here.
        if (!prefetched) {
          issue_q(cur);
          issue_k(0);
          wait_vm_lds_barrier<0>();
          issue_k(1);  // K_1 (or the next item's K_0) and V_0 land by the end of phase 2
          issue_v(0);
        } else if (ntiles == 1) {
          issue_k(1);
        }
        u32x4 qf[QT][DC];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
#pragma unroll
          for (int cc = 0; cc < DC; ++cc) qf[qt][cc] = *reinterpret_cast<const u32x4*>(qlane + (qt * DC + cc) * 512);
        STile s;
        u32x4 pk[KC][QT];
        auto mma_block = [&](int u) {  // S = Q K_{u+1}^T, O += P_u V_u
          // in the last step the QK reads the slot holding the next item's K_0 (landed one step
          // earlier; the step's DMA fills the other slot) and its S is never used: one
          // straight-line block, as in run()
          __builtin_amdgcn_s_setprio(1);
          qk(s, qf, kslot(u + 1));
          pv(acc, pk, vslot(u), lsum);
          m_schedule<8>();
          __builtin_amdgcn_s_setprio(0);
        };
        auto softmax_block = [&](int t) {
          if (t < ntiles) softmax(s, pk, acc, ro, l_i, lsum, (cur.t_begin + t) * BN, wrow0, q16, g, p);
        };
        if (GRP == 0 && wave_has_rows) {
          qk(s, qf, kslot(0));
          qk_schedule();
        }
        wait_vm_lds_barrier<63>();
        if (wave_has_rows) {
          if (GRP == 0) {
            softmax_block(0);
          } else {
            qk(s, qf, kslot(0));
            qk_schedule();
          }
        }
        // A prefetched item's Q, K_0, K_1 and V_0 landed by the previous item's last wait; what is
        // still in flight here is that item's O stores and (T == 1) the next item's K_0, which
        // only step 1's discarded QK reads before step 1's own wait. So the barrier need not
        // wait for memory (the O stores then drain during step 1).
        if (prefetched) wait_vm_lds_barrier<63>();
        else wait_vm_lds_barrier<0>();
        // Steps that take chunks of the next item's Q: 1 .. min(kQChunks, T) (none without a next
        // item). The step loop tests this once and the tile ownership of K_{j+1} and V_j once: the
        // per-chunk and per-operand tests it replaced, each a branch in every step, had made a step
        // ~1-2% longer than the per-workgroup kernel's (same instructions otherwise).
        const int q_last = __builtin_amdgcn_readfirstlane(nxt.ntiles > 0 ? min(kQChunks, ntiles) : 0);
        for (int j = 1; j <= ntiles; ++j) {
          if (__builtin_expect(j + 1 < ntiles, 1)) {  // K_{j+1} and V_j of this item
            const uint32_t ks = kring_lds + (uint32_t)((par + j + 1) & 1) * (KT_ELEMS * 2) + wave * NKW * 1024;
            buffer_load16_to_lds_blocks<NKW, 64>(slab_rsrc(krs, (uint32_t)(cur.t_begin + j + 1) * kstep, true), koff, ks);
            const uint32_t vs = vring_lds + (uint32_t)((par + j) & 1) * (VT_ELEMS * 2) + wave * NVW * 1024;
            buffer_load16_to_lds_blocks<NVW, 32>(slab_rsrc(vrs, (uint32_t)(cur.t_begin + j) * vstep, true), voff, vs);
          } else {
            issue_k(j + 1);
            issue_v(j);
          }
          // every wave read its Q fragments before the barriers above: the buffer takes the next
          // item's Q, chunk c at step min(c + 1, T), so all of it has landed by the item's last wait
          if (__builtin_expect(j <= q_last, 0)) {
#pragma unroll
            for (int c = 0; c < kQChunks; ++c)
              if (j == min(c + 1, ntiles)) issue_q_chunk(nxt, c);
          }
          if (wave_has_rows) {
            if (GRP == 0) mma_block(j - 1);
            else softmax_block(j - 1);
          }
          wait_vm_lds_barrier<63>();
          if (wave_has_rows) {
            if (GRP == 0) softmax_block(j);
            else mma_block(j - 1);
          }
          wait_vm_lds_barrier<0>();
        }
      }
      {
        const auto pe = kernarg_params<FwdParams>();
        const Ids ids = decode(cur.pid, *pe);
        store_out(acc, ro, l_i, lsum, wrow0, q16, g, pe->M, ids.b, ids.h, ids.split);
      }
      if (pid_n < 0) break;
      prefetched = ntiles > 0 && nxt.ntiles > 0;
      par = (par + ntiles) & 1;
      cur = nxt;
    }
  }

  __device__ static void run_persistent(const FwdParams& p) {
    __shared__ __attribute__((aligned(16))) uint16_t smem[2 * (KT_ELEMS + VT_ELEMS) + QB_ELEMS];
    const int tid = (int)__builtin_amdgcn_workitem_id_x();
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pid0 = item_pid(0, (int)__builtin_amdgcn_workgroup_id_x(), p.grid, p.total_blocks);
    if (pid0 < 0) return;  // workgroup-uniform: more workgroups than blocks
    if (wave < 4) persistent_group<0>(p, smem, lane, wave, pid0);
    else persistent_group<1>(p, smem, lane, wave, pid0);
  }

  __device__ static void run(const FwdParams& p) {
    __shared__ __attribute__((aligned(16))) uint16_t smem[2 * (KT_ELEMS + VT_ELEMS)];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q16 = lane & 15, g = lane >> 4;

    // Logical block id: XCD-local, then (bh, split, m-block), m-block fastest; packed GQA rows for
    // decode shapes (row r = query head h + r / M, position r % M), as in fa_fwd.hip.
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
    // The integer divisions above run on the vector ALU, though their results are workgroup-
    // uniform. Declaring them uniform puts the tile bounds, and the loop's branches on them, in
    // scalar registers: measured 1-3% faster for the 64-key kernels; the 32-key ones lose (their
    // register allocation grows by 30-60 VGPRs), so they keep vector copies.
    if constexpr (kScalarIds) {
      mb = __builtin_amdgcn_readfirstlane(mb);
      b = __builtin_amdgcn_readfirstlane(b);
      h = __builtin_amdgcn_readfirstlane(h);
      hk = __builtin_amdgcn_readfirstlane(hk);
    }
    const int split_u = kScalarIds ? __builtin_amdgcn_readfirstlane(split) : split;
    const int rows = p.M * p.pack;
    const int m0 = mb * BM;
    const int wrow0 = m0 + wave * ROWS;
    const bool wave_has_rows = wrow0 < rows;
    auto row_head = [&](int r) { return p.pack > 1 ? h + r / p.M : h; };
    auto row_pos = [&](int r) { return p.pack > 1 ? r % p.M : r; };

    // Q^T fragments (B operand of Q K^T): lane holds query row wrow0 + 16 qt + q16 at
    // d = 32 cc + 8 g .. +7.
    u32x4 qf[QT][DC];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int row = wrow0 + qt * 16 + q16;
      const uint16_t* qrow =
          p.q + (int64_t)b * p.sq0 + (int64_t)row_head(row) * p.sq1 + (int64_t)row_pos(row) * p.sq2;
#pragma unroll
      for (int cc = 0; cc < DC; ++cc) {
        u32x4 val = {0u, 0u, 0u, 0u};
        if (row < rows) val = *reinterpret_cast<const u32x4*>(qrow + cc * 32 + g * 8);
        qf[qt][cc] = val;
      }
    }

    // KV tiles of this split, clipped by the causal diagonal.
    const int t_begin = split_u * p.tiles_per_split;
    int n_end = (t_begin + p.tiles_per_split) * BN;
    if (n_end > p.N) n_end = p.N;
    if (p.causal && n_end > m0 + BM) n_end = m0 + BM;
    const int t_end = (n_end + BN - 1) / BN;
    const int ntiles = t_end > t_begin ? t_end - t_begin : 0;

    OAcc acc;
    RowOff ro;
    ro.reset();
    float l_i[QT];
    floatx4 lsum[QT];  // row sums of the ones-row MFMA (kSumMfma)
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      l_i[qt] = 0.f;
      lsum[qt] = (floatx4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int dt = 0; dt < DTL; ++dt) acc[dt][qt] = (floatx4){0.f, 0.f, 0.f, 0.f};
    }

    // LDS-DMA sources: the buffer range is the (b, kv-head) rows [0, N) of K and of V, so rows past
    // N read as zero (the host keeps (N + block_n) * row stride * 2 bytes below 2^32). Lane m of a
    // K block (jt, cc) moves K[jt*16 + (m & 15)][cc*32 + 8 (m >> 4) .. +7]; a wave's next block is
    // the next d chunk (+64 bytes). Lane m of a V block (kc, dt) moves the 16 bytes of transposing-
    // read lanes L = 2 (m & 31), L + 1 of read m >> 5: V[kc*32 + 16 (m >> 5) + 4 ((m & 31) >> 3)
    // + ((m & 7) >> 1)][dt*16 + 8 (m & 1) .. +7]; a wave's next block is the next d tile (+32 bytes).
    const auto krs = make_rsrc(p.k + (int64_t)b * p.sk0 + (int64_t)hk * p.sk1, (uint32_t)p.N * (uint32_t)p.sk2 * 2u);
    const auto vrs = make_rsrc(p.v + (int64_t)b * p.sv0 + (int64_t)hk * p.sv1, (uint32_t)p.N * (uint32_t)p.sv2 * 2u);
    uint32_t koff, voff;
    {
      const int blk = wave * NKW, jt = blk / DC, cc = blk % DC;
      const uint32_t row = jt * 16 + (lane & 15), c0 = cc * 32 + 8 * (lane >> 4);
      koff = (row * (uint32_t)p.sk2 + c0) * 2u;
    }
    {
      const int blk = wave * NVW, kc = blk / DTL, dt = blk % DTL;
      const int m = lane;
      const uint32_t row = kc * 32 + 16 * (m >> 5) + 4 * ((m & 31) >> 3) + ((m & 7) >> 1);
      const uint32_t c0 = dt * 16 + 8 * (m & 1);
      voff = (row * (uint32_t)p.sv2 + c0) * 2u;
    }
    uint16_t* kring = smem;
    uint16_t* vring = smem + 2 * KT_ELEMS;
    const uint32_t kring_lds = lds_address(smem), vring_lds = kring_lds + 2 * KT_ELEMS * 2;
    auto issue_k = [&](int u) {
      if (u >= ntiles) return;
      const uint32_t toff = (uint32_t)((t_begin + u) * BN) * (uint32_t)p.sk2 * 2u;
      const uint32_t slot = kring_lds + (uint32_t)(u & 1) * (KT_ELEMS * 2);
      // uniform tile offset (64-key kernels): it moves the resource, the lanes' offsets stay fixed
      if constexpr (kScalarIds)
        buffer_load16_to_lds_blocks<NKW, 64>(slab_rsrc(krs, toff, true), koff, slot + wave * NKW * 1024);
      else
        buffer_load16_to_lds_blocks<NKW, 64>(krs, koff + toff, slot + wave * NKW * 1024);
    };
    auto issue_v = [&](int u) {
      if (u >= ntiles) return;
      const uint32_t toff = (uint32_t)((t_begin + u) * BN) * (uint32_t)p.sv2 * 2u;
      const uint32_t slot = vring_lds + (uint32_t)(u & 1) * (VT_ELEMS * 2);
      if constexpr (kScalarIds)
        buffer_load16_to_lds_blocks<NVW, 32>(slab_rsrc(vrs, toff, true), voff, slot + wave * NVW * 1024);
      else
        buffer_load16_to_lds_blocks<NVW, 32>(vrs, voff + toff, slot + wave * NVW * 1024);
    };
    const uint16_t* klane = kring + lane * 8;  // this lane's 16 bytes in every K block
    const uint16_t* vlane = vring + lane * 4;  // this lane's 8 bytes in every V half-block

    if constexpr (PIPE == 2) {
      // Ping-pong: waves 0-3 (group 0) and 4-7 (group 1) run the same sequence of blocks, group 1
      // one phase behind, with a workgroup barrier between phases. Blocks alternate between matrix
      // work and softmax work -- block 0: S = Q K_0^T; block 2u+1: softmax of tile u (mask, row
      // max, rescale, P_u); block 2u+2: S = Q K_{u+1}^T (u+1 < n) and O += P_u V_u -- so in every
      // phase one group issues MFMAs while the other, on the same SIMDs, issues the exp/pack VALU
      // work, and the two streams overlap instead of taking turns inside one wave.
      // K_t and V_t live in slot t & 1 of two-slot rings. K_t is read in phases 2t (group 0) and
      // 2t+1 (group 1), V_t in phases 2t+2 and 2t+3; phase 2s (s >= 1) refills with K_{s+1} and
      // V_s (their slots' previous tiles were last read in phase 2s-1) and every wave waits for its
      // own refills before the barrier that ends phase 2s+1, two phases before their first reader.
      STile s;
      u32x4 pk[KC][QT];
      auto mma_block = [&](int u) {  // S = Q K_{u+1}^T, O += P_u V_u
        // past the last tile the QK reads a stale K slot and its S is never used: one straight-line
        // block lets the V reads start during the QK MFMAs
        // the matrix group issues first: its MFMAs then wait for no VALU op of the softmax group
        __builtin_amdgcn_s_setprio(1);
        qk(s, qf, klane + ((u + 1) & 1) * KT_ELEMS);
        pv(acc, pk, vlane + (u & 1) * VT_ELEMS, lsum);
        m_schedule<8>();
        __builtin_amdgcn_s_setprio(0);
      };
      auto softmax_block = [&](int t) {
        if (t < ntiles) softmax(s, pk, acc, ro, l_i, lsum, (t_begin + t) * BN, wrow0, q16, g, p);
      };
      // Group G's sequence; phases 2j and 2j+1 form iteration j. The branches on G and on
      // wave_has_rows are wave-uniform, and every wave runs the same barriers.
      auto run_group = [&](auto G) {
        constexpr int grp = decltype(G)::value;
        issue_k(0);
        wait_vm_lds_barrier<0>();
        issue_k(1);  // K_1 and V_0 land by the end of phase 1
        issue_v(0);
        if (grp == 0 && wave_has_rows) {
          qk(s, qf, klane);
          qk_schedule();
        }
        wait_vm_lds_barrier<63>();
        if (wave_has_rows) {
          if (grp == 0) {
            softmax_block(0);
          } else {
            qk(s, qf, klane);
            qk_schedule();
          }
        }
        wait_vm_lds_barrier<0>();
        for (int j = 1; j <= ntiles; ++j) {
          issue_k(j + 1);
          issue_v(j);
          if (wave_has_rows) {
            if (grp == 0) mma_block(j - 1);
            else softmax_block(j - 1);
          }
          wait_vm_lds_barrier<63>();
          if (wave_has_rows) {
            if (grp == 0) softmax_block(j);
            else mma_block(j - 1);
          }
          wait_vm_lds_barrier<0>();
        }
      };
      if (ntiles > 0) {
        if (wave < 4) run_group(std::integral_constant<int, 0>{});
        else run_group(std::integral_constant<int, 1>{});
      }
    } else if constexpr (PIPE) {
      // Step u reads K_{u+1} and V_u: K runs one tile ahead of V. 2-slot rings: step u issues
      // K_{u+2} into K_u's slot and V_{u+1} into V_{u-1}'s (both read in step u-1) and waits for
      // them at the end of the step. Before step u the wave holds S_u and its unmasked row max.
      STile sa, sb;
      float mxa[QT], mxb[QT];
      if (ntiles > 0) {
        issue_k(0);
        issue_v(0);
        issue_k(1);
        wait_vm_lds_barrier<0>();
        if (wave_has_rows) {
          qk(sa, qf, klane);
          qk_schedule();
          tile_max(sa, mxa);
        }
        wait_vm_lds_barrier<0>();  // every wave is done with K slot 0 before step 0 refills it
      }
      // Masks for tile u (rare: sequence end, causal diagonal) and the row max they change.
      auto fix_masked = [&](STile& cur, float (&mx_cur)[QT], int u) {
        const int n0 = (t_begin + u) * BN;
        if (tile_needs_mask(n0, wrow0, p)) {
          mask_tile(cur, n0, wrow0, q16, g, p);
          tile_max(cur, mx_cur);
        }
      };
      auto step = [&](STile& cur, float (&mx_cur)[QT], STile& nxt, float (&mx_nxt)[QT], int u) {
        issue_k(u + 2);
        issue_v(u + 1);
        if (wave_has_rows) {  // waves without rows still move their share of K/V
          fix_masked(cur, mx_cur, u);
          rescale(mx_cur, acc, ro, l_i, lsum, p.c);
          u32x4 pk[KC][QT];
          exp_pack(cur, pk, ro, l_i, p.c);
          qk(nxt, qf, klane + ((u + 1) & 1) * KT_ELEMS);
          x_schedule();
          pv(acc, pk, vlane + (u & 1) * VT_ELEMS, lsum);
          tile_max(nxt, mx_nxt);
          y_schedule();
        }
        wait_vm_lds_barrier<0>();
      };
      auto last = [&](STile& cur, float (&mx_cur)[QT], int u) {
        if (!wave_has_rows) return;
        fix_masked(cur, mx_cur, u);
        rescale(mx_cur, acc, ro, l_i, lsum, p.c);
        u32x4 pk[KC][QT];
        exp_pack(cur, pk, ro, l_i, p.c);
        pv(acc, pk, vlane + (u & 1) * VT_ELEMS, lsum);
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
    } else {
    // One KV tile per step: step u issues tile u+1 into the slot tile u-1 left (read in step u-1)
    // and waits for it at the end of the step.
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
        u32x4 pk[KC][QT];
        qk(s, qf, klane + (u & 1) * KT_ELEMS);
        qk_schedule();
        softmax(s, pk, acc, ro, l_i, lsum, (t_begin + u) * BN, wrow0, q16, g, p);
        pv(acc, pk, vlane + (u & 1) * VT_ELEMS, lsum);
        pv_schedule();
      }
      wait_vm_lds_barrier<0>();
    }
    }

    // Epilogue: l over the four lane rows, O = acc / l; lane holds d = 16 dt + 4 g .. +3. The
    // output parameters are read again from the kernel-argument segment (scalar loads) rather than
    // kept in scalar registers across the loop, where they would crowd out its own; fa_fwd16_kernel
    // takes FwdParams as its only argument (checked there), so the segment starts with it.
    const auto pe = kernarg_params<FwdParams>();
    constexpr float kLn2 = 0.69314718055994530942f;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const float l = kSumMfma ? lsum[qt][0] : xquad_sum(l_i[qt]);
      const int i = wrow0 + qt * 16 + q16;
      const float inv = (l > 0.f) ? 1.f / l : 0.f;
      const float lse_val = (l > 0.f) ? (ro.m[qt] * pe->c + __builtin_amdgcn_logf(l)) * kLn2 : FA_NEG_INF;
      u32x4 wide[DTL / 2];
      if constexpr (kWideO) pack_o_wide(acc, qt, inv, wide);  // cross-lane: before the row test
      if (i < rows) {
        const int hr = pe->pack > 1 ? h + i / pe->M : h;
        const int mr = pe->pack > 1 ? i % pe->M : i;
        if (SPLIT) {
          const int64_t wrow = (int64_t)(split_u * pe->B + b) * pe->H + hr;  // [split][b][h][m] rows
          float* wo = pe->ws_o + (wrow * pe->M + mr) * D;
#pragma unroll
          for (int dt = 0; dt < DTL; ++dt) {
            floatx4 val = {acc[dt][qt][0] * inv, acc[dt][qt][1] * inv, acc[dt][qt][2] * inv, acc[dt][qt][3] * inv};
            *reinterpret_cast<floatx4*>(wo + dt * 16 + 4 * g) = val;
          }
          if (g == 0) pe->ws_lse[wrow * pe->M + mr] = lse_val;
        } else {
          uint16_t* orow = pe->o + (int64_t)b * pe->so0 + (int64_t)hr * pe->so1 + (int64_t)mr * pe->so2;
          if constexpr (kWideO) {
#pragma unroll
            for (int pp = 0; pp < DTL / 2; ++pp)
              *reinterpret_cast<u32x4*>(orow + 32 * pp + wide_col(g)) = wide[pp];
          } else {
#pragma unroll
            for (int dt = 0; dt < DTL; ++dt) {
              u32x2 val = {T::pack2(acc[dt][qt][0] * inv, acc[dt][qt][1] * inv),
                           T::pack2(acc[dt][qt][2] * inv, acc[dt][qt][3] * inv)};
              *reinterpret_cast<u32x2*>(orow + dt * 16 + 4 * g) = val;
            }
          }
          float* lse = pe->lse;
          if (lse != nullptr && g == 0)
            lse[(int64_t)b * pe->sl0 + (int64_t)hr * pe->sl1 + (int64_t)mr * pe->sl2] = lse_val;
        }
      }
    }
  }

};

template <typename Tag, int D, int WAVES, int BN, int PIPE, bool SPLIT>
__global__ __launch_bounds__(WAVES * 64, (Fwd16<Tag, D, WAVES, BN, PIPE, SPLIT>::kBlocksPerCu)) void fa_fwd16_kernel(
    FwdParams p) {
  static_assert(kernel_has_sole_arg<FwdParams>(&fa_fwd16_kernel<Tag, D, WAVES, BN, PIPE, SPLIT>),
                "the epilogues read FwdParams from kernel-argument offset 0: it must stay the only argument");
  if constexpr (PIPE == 3)
    Fwd16<Tag, D, WAVES, BN, PIPE, SPLIT>::run_persistent(p);
  else
    Fwd16<Tag, D, WAVES, BN, PIPE, SPLIT>::run(p);
}

// Registry (stages=6: PIPE 0, stages=7: PIPE 1, stages=8: PIPE 2 and stages=9: PIPE 3 with 8 waves;
// 32 query rows per wave).
#define FA16_SYM_TAG_f16_t "5f16_t"
#define FA16_SYM_TAG_bf16_t "6bf16_t"
#define FA16_SYMBOL(TAG, D, W, BN, PI, SP)                                                                    \
  "_ZN2fa15fa_fwd16_kernelINS_" FA16_SYM_TAG_##TAG "ELi" #D "ELi" #W "ELi" #BN "ELi" #PI "ELb" #SP \
  "EEEvNS_9FwdParamsE"
#define FA16_ENTRY(TAG, DTYPE, D, W, BN, PI, SP)                                                         \
  {6 + PI, DTYPE, D, W, 32, BN, SP, (const void*)&fa_fwd16_kernel<TAG, D, W, BN, PI, (SP != 0)>, \
   FA16_SYMBOL(TAG, D, W, BN, PI, SP)}
#define FA16_PAIR(TAG, DTYPE, D, BN, PI) FA16_ENTRY(TAG, DTYPE, D, 4, BN, PI, 0), FA16_ENTRY(TAG, DTYPE, D, 4, BN, PI, 1)
#define FA16_PAIR8(TAG, DTYPE, D, BN, PI) FA16_ENTRY(TAG, DTYPE, D, 8, BN, PI, 0), FA16_ENTRY(TAG, DTYPE, D, 8, BN, PI, 1)
#define FA16_ENTRIES(TAG, DTYPE, D)                                                             \
  FA16_PAIR(TAG, DTYPE, D, 64, 0), FA16_PAIR(TAG, DTYPE, D, 32, 0), FA16_PAIR(TAG, DTYPE, D, 64, 1), \
      FA16_PAIR(TAG, DTYPE, D, 32, 1), FA16_PAIR8(TAG, DTYPE, D, 64, 2), FA16_PAIR8(TAG, DTYPE, D, 64, 3)

static const FaKernelEntry kFwd16Entries[] = {
    FA16_ENTRIES(f16_t, FA_DTYPE_F16, 64),        FA16_ENTRIES(f16_t, FA_DTYPE_F16, 128),
    FA16_ENTRIES(bf16_t, FA_DTYPE_BF16, 64),      FA16_ENTRIES(bf16_t, FA_DTYPE_BF16, 128),
    // D = 256: one tile per step only (the pipelined kernel's two score tiles do not fit beside O
    // and Q in 256 registers)
    FA16_PAIR(f16_t, FA_DTYPE_F16, 256, 32, 0),   FA16_PAIR(bf16_t, FA_DTYPE_BF16, 256, 32, 0),
};

const FaKernelEntry* fa_fwd16_registry(int* count) {
  *count = (int)(sizeof(kFwd16Entries) / sizeof(kFwd16Entries[0]));
  return kFwd16Entries;
}

}  // namespace fa
