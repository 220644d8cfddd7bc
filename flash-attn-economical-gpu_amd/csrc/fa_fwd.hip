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
//  * Q^T is the B operand and stays in VGPRs for the whole kernel (loaded once).
//  * P^T is fed to the PV product O^T = V^T P^T directly from the S^T accumulator registers (the
//    B-operand k-slots of a 16-key chunk are exactly the accumulator rows the lane already holds),
//    so P never goes through LDS. V^T is the A operand, read from an LDS copy of V that is stored
//    transposed ([d][key]) with keys permuted inside each 16-key chunk (bits 2 and 3 swapped) so
//    that one 16-byte LDS read yields the 8 keys a lane needs.
//  * K (natural [key][d]) and V^T tiles go through LDS; stages=1 single-buffers them (basic),
//    stages=2 double-buffers them with one barrier per tile (optimized). Both prefetch the next
//    tile from HBM into registers while the current tile is computed.
//  * Softmax uses exp2 with scale*log2(e) folded into one FMA per score.
//  * Causal (top-left, row i sees keys j <= i as flash_atten.py:103-105) skips KV tiles past the
//    diagonal, masks only diagonal tiles, and walks query blocks heaviest-first.
//  * GQA: query head h reads KV head h / (H / H_kv); no K/V expansion.
//  * Split-KV: the SPLIT instantiation writes fp32 normalised partial O and partial LSE per KV
//    split; fa_merge_kernel combines them: lse = ln sum_j exp(lse_j), O = sum_j exp(lse_j - lse) O_j.
#include "fa_common.h"
#include "fa_kernels.h"
#include "../../include/fa_gfx950.h"

namespace fa {

#define FA_NEG_INF (-__builtin_inff())

// Position of key j (0 <= j < block_n) inside a V^T LDS row: bits 2 and 3 of j swapped, so that
// the lane of half-wave `h` finds the 8 keys {16c + 4h + 0..3, 16c + 8 + 4h + 0..3} of chunk c
// in one contiguous 16-byte run at slot 16c + 8h.
__device__ inline int vt_slot(int j) { return (j & ~12) | ((j & 4) << 1) | ((j & 8) >> 1); }

template <typename Tag, int D, int WAVES, int RT, int BN, int STAGES, bool SPLIT>
struct FwdKernel {
  static constexpr int THREADS = WAVES * 64;
  static constexpr int ROWS = 32 * RT;          // query rows per wave
  static constexpr int BM = WAVES * ROWS;       // query rows per workgroup
  static constexpr int DC = D / 16;             // 16-wide d chunks of Q K^T
  static constexpr int DTL = D / 32;            // 32-row d tiles of O^T
  static constexpr int JT = BN / 32;            // 32-key tiles of S^T
  static constexpr int KC = BN / 16;            // 16-key chunks of P V
  static constexpr int KSTR = D + 8;            // K LDS row stride (elements), +16 B pad
  static constexpr int VSTR = BN + 8;           // V^T LDS row stride (elements), +16 B pad
  static constexpr int KTILE = BN * KSTR;
  static constexpr int VTILE = D * VSTR;
  static constexpr int STAGE_ELEMS = KTILE + VTILE;
  static constexpr int K_CHUNKS = BN * D / 8;   // 16-byte chunks per K tile
  static constexpr int K_ITERS = (K_CHUNKS + THREADS - 1) / THREADS;
  static constexpr int V_QUADS = BN * D / 32;   // 4-key x 8-d blocks per V tile
  static constexpr int V_ITERS = (V_QUADS + THREADS - 1) / THREADS;
  static_assert(D % 32 == 0 && BN % 32 == 0, "tile shape");
  static_assert(BM % BN == 0, "causal tile bound assumes block_m % block_n == 0");

  typedef DT<Tag> T;

  struct Prefetch {
    u32x4 k[K_ITERS];
    u32x4 v[V_ITERS][4];
  };

  __device__ static inline void load_tile(Prefetch& pf, const uint16_t* kbase, const uint16_t* vbase,
                                          int64_t sk2, int64_t sv2, int n0, int N, int tid) {
#pragma unroll
    for (int i = 0; i < K_ITERS; ++i) {
      const int id = tid + i * THREADS;
      const int row = id / (D / 8), c8 = id % (D / 8);
      u32x4 val = {0u, 0u, 0u, 0u};
      if ((K_CHUNKS % THREADS == 0 || id < K_CHUNKS) && n0 + row < N)
        val = *reinterpret_cast<const u32x4*>(kbase + (int64_t)(n0 + row) * sk2 + c8 * 8);
      pf.k[i] = val;
    }
#pragma unroll
    for (int i = 0; i < V_ITERS; ++i) {
      const int id = tid + i * THREADS;
      const int jq = id / (D / 8), d8 = id % (D / 8);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = n0 + jq * 4 + r;
        u32x4 val = {0u, 0u, 0u, 0u};
        if ((V_QUADS % THREADS == 0 || id < V_QUADS) && j < N)
          val = *reinterpret_cast<const u32x4*>(vbase + (int64_t)j * sv2 + d8 * 8);
        pf.v[i][r] = val;
      }
    }
  }

  __device__ static inline void store_tile(const Prefetch& pf, uint16_t* ks, uint16_t* vs, int tid) {
#pragma unroll
    for (int i = 0; i < K_ITERS; ++i) {
      const int id = tid + i * THREADS;
      if (K_CHUNKS % THREADS == 0 || id < K_CHUNKS) {
        const int row = id / (D / 8), c8 = id % (D / 8);
        *reinterpret_cast<u32x4*>(ks + row * KSTR + c8 * 8) = pf.k[i];
      }
    }
#pragma unroll
    for (int i = 0; i < V_ITERS; ++i) {
      const int id = tid + i * THREADS;
      if (V_QUADS % THREADS == 0 || id < V_QUADS) {
        const int jq = id / (D / 8), d8 = id % (D / 8);
        const int slot = vt_slot(jq * 4);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int w = e >> 1;
          const int sh = (e & 1) * 16;
          const uint32_t a0 = (pf.v[i][0][w] >> sh) & 0xffffu, a1 = (pf.v[i][1][w] >> sh) & 0xffffu;
          const uint32_t a2 = (pf.v[i][2][w] >> sh) & 0xffffu, a3 = (pf.v[i][3][w] >> sh) & 0xffffu;
          u32x2 out = {a0 | (a1 << 16), a2 | (a3 << 16)};
          *reinterpret_cast<u32x2*>(vs + (d8 * 8 + e) * VSTR + slot) = out;
        }
      }
    }
  }

  __device__ static void run(const FwdParams& p) {
    __shared__ __attribute__((aligned(16))) uint16_t smem[STAGES * STAGE_ELEMS];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, col = lane & 31, hh = lane >> 5;

    // Logical block id: XCD-local, then (bh, split, m-block) with the m-block fastest.
    const int pid = xcd_remap(blockIdx.x, p.total_blocks);
    int mb = pid % p.m_blocks;
    const int rest = pid / p.m_blocks;
    const int split = rest % p.splits;
    const int bh = rest / p.splits;
    if (p.causal) mb = p.m_blocks - 1 - mb;  // heaviest query blocks first
    const int b = bh / p.H, h = bh % p.H;
    const int hk = h / p.group;
    const int m0 = mb * BM;
    const int wrow0 = m0 + wave * ROWS;  // first query row of this wave

    const uint16_t* qbase = p.q + (int64_t)b * p.sq0 + (int64_t)h * p.sq1;
    const uint16_t* kbase = p.k + (int64_t)b * p.sk0 + (int64_t)hk * p.sk1;
    const uint16_t* vbase = p.v + (int64_t)b * p.sv0 + (int64_t)hk * p.sv1;

    // Q^T fragments (B operand): lane holds row wrow0 + 32*rt + col, d = 16c + 8hh .. +7.
    u32x4 qf[RT][DC];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int row = wrow0 + rt * 32 + col;
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        u32x4 val = {0u, 0u, 0u, 0u};
        if (row < p.M) val = *reinterpret_cast<const u32x4*>(qbase + (int64_t)row * p.sq2 + c * 16 + hh * 8);
        qf[rt][c] = val;
      }
    }

    // KV tiles of this split, clipped by the causal diagonal.
    const int t_begin = split * p.tiles_per_split;
    int n_end = (t_begin + p.tiles_per_split) * BN;
    if (n_end > p.N) n_end = p.N;
    if (p.causal && n_end > m0 + BM) n_end = m0 + BM;
    const int t_end = (n_end + BN - 1) / BN;

    floatx16 acc[DTL][RT];
    float m_i[RT], l_i[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      m_i[rt] = FA_NEG_INF;
      l_i[rt] = 0.f;
#pragma unroll
      for (int dt = 0; dt < DTL; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[dt][rt][r] = 0.f;
    }

    const float c = p.c;
    Prefetch pf;
    if (t_begin < t_end) {
      load_tile(pf, kbase, vbase, p.sk2, p.sv2, t_begin * BN, p.N, tid);
      if (STAGES == 2) {
        store_tile(pf, smem, smem + KTILE, tid);
        __syncthreads();
      }
    }

    for (int t = t_begin; t < t_end; ++t) {
      const int n0 = t * BN;
      uint16_t* ks;
      uint16_t* vs;
      if (STAGES == 1) {
        __syncthreads();  // every wave finished reading the previous tile
        store_tile(pf, smem, smem + KTILE, tid);
        __syncthreads();
        ks = smem;
        vs = smem + KTILE;
        if (t + 1 < t_end) load_tile(pf, kbase, vbase, p.sk2, p.sv2, n0 + BN, p.N, tid);
      } else {
        const int cur = (t - t_begin) & 1;
        ks = smem + cur * STAGE_ELEMS;
        vs = ks + KTILE;
        if (t + 1 < t_end) load_tile(pf, kbase, vbase, p.sk2, p.sv2, n0 + BN, p.N, tid);
      }

      // A wave whose rows all precede this tile (causal) has nothing to add from it.
      const bool wave_active = !(p.causal && n0 > wrow0 + ROWS - 1);
      if (wave_active) {
        // S^T = K Q^T for JT x RT 32x32 tiles.
        floatx16 s[JT][RT];
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
            const u32x4 kf = *reinterpret_cast<const u32x4*>(ks + (jt * 32 + col) * KSTR + cc * 16 + hh * 8);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) s[jt][rt] = T::mfma32(kf, qf[rt][cc], s[jt][rt]);
          }
        }

        // Key-range and causal masks, only on tiles that need them.
        const bool need_mask = (n0 + BN > p.N) || (p.causal && n0 + BN - 1 > wrow0);
        if (need_mask) {
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

        // Online softmax (per-lane row statistics).
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          float mx = FA_NEG_INF;
#pragma unroll
          for (int jt = 0; jt < JT; ++jt)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[jt][rt][r]);
          mx = fmaxf(mx, xhalf(mx));
          const float m_new = fmaxf(m_i[rt], mx);
          const float m_use = (m_new == FA_NEG_INF) ? 0.f : m_new;
          const float alpha = fast_exp2((m_i[rt] - m_use) * c);
          m_i[rt] = m_new;
          const float mc = m_use * c;
          float rs = 0.f;
#pragma unroll
          for (int jt = 0; jt < JT; ++jt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float e = fast_exp2(__builtin_fmaf(s[jt][rt][r], c, -mc));
              s[jt][rt][r] = e;
              rs += e;
            }
          l_i[rt] = l_i[rt] * alpha + rs;
#pragma unroll
          for (int dt = 0; dt < DTL; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[dt][rt][r] *= alpha;
        }

        // O^T += V^T P^T.
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
          const int jt = kc >> 1, rb = (kc & 1) * 8;
          u32x4 pb[RT];
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            pb[rt][0] = T::pack2(s[jt][rt][rb + 0], s[jt][rt][rb + 1]);
            pb[rt][1] = T::pack2(s[jt][rt][rb + 2], s[jt][rt][rb + 3]);
            pb[rt][2] = T::pack2(s[jt][rt][rb + 4], s[jt][rt][rb + 5]);
            pb[rt][3] = T::pack2(s[jt][rt][rb + 6], s[jt][rt][rb + 7]);
          }
#pragma unroll
          for (int dt = 0; dt < DTL; ++dt) {
            const u32x4 vf = *reinterpret_cast<const u32x4*>(vs + (dt * 32 + col) * VSTR + kc * 16 + hh * 8);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) acc[dt][rt] = T::mfma32(vf, pb[rt], acc[dt][rt]);
          }
        }
      }

      if (STAGES == 2) {
        if (t + 1 < t_end) {
          const int nxt = (t + 1 - t_begin) & 1;
          uint16_t* kn = smem + nxt * STAGE_ELEMS;
          store_tile(pf, kn, kn + KTILE, tid);
        }
        __syncthreads();
      }
    }

    // Epilogue: l over both half-waves, O = acc / l.
    constexpr float kLn2 = 0.69314718055994530942f;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const float l = l_i[rt] + xhalf(l_i[rt]);
      const int i = wrow0 + rt * 32 + col;
      const float inv = (l > 0.f) ? 1.f / l : 0.f;
      const float lse_val = (l > 0.f) ? (m_i[rt] * c + __builtin_amdgcn_logf(l)) * kLn2 : FA_NEG_INF;
      if (i < p.M) {
        if (SPLIT) {
          float* wo = p.ws_o + ((int64_t)(split * p.B * p.H + bh) * p.M + i) * D;
#pragma unroll
          for (int dt = 0; dt < DTL; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              floatx4 val = {acc[dt][rt][4 * g] * inv, acc[dt][rt][4 * g + 1] * inv,
                             acc[dt][rt][4 * g + 2] * inv, acc[dt][rt][4 * g + 3] * inv};
              *reinterpret_cast<floatx4*>(wo + dt * 32 + 8 * g + 4 * hh) = val;
            }
          if (hh == 0) p.ws_lse[(int64_t)(split * p.B * p.H + bh) * p.M + i] = lse_val;
        } else {
          uint16_t* orow = p.o + (int64_t)b * p.so0 + (int64_t)h * p.so1 + (int64_t)i * p.so2;
#pragma unroll
          for (int dt = 0; dt < DTL; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              u32x2 val = {T::pack2(acc[dt][rt][4 * g] * inv, acc[dt][rt][4 * g + 1] * inv),
                           T::pack2(acc[dt][rt][4 * g + 2] * inv, acc[dt][rt][4 * g + 3] * inv)};
              *reinterpret_cast<u32x2*>(orow + dt * 32 + 8 * g + 4 * hh) = val;
            }
          if (p.lse != nullptr && hh == 0)
            p.lse[(int64_t)b * p.sl0 + (int64_t)h * p.sl1 + (int64_t)i * p.sl2] = lse_val;
        }
      }
    }
  }
};

template <typename Tag, int D, int WAVES, int RT, int BN, int STAGES, bool SPLIT>
__global__ __launch_bounds__(WAVES * 64) void fa_fwd_kernel(FwdParams p) {
  FwdKernel<Tag, D, WAVES, RT, BN, STAGES, SPLIT>::run(p);
}

// Merge of split-KV partials: one wave per query row.
template <typename Tag, int D>
__global__ __launch_bounds__(256) void fa_merge_kernel(MergeParams p) {
  typedef DT<Tag> T;
  constexpr int PER_LANE = D / 64 > 0 ? D / 64 : 1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t rows = (int64_t)p.B * p.H * p.M;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= rows) return;
  const int64_t bh = row / p.M;
  const int i = (int)(row % p.M);
  const int64_t split_stride = rows;  // rows per split

  constexpr float kLog2e = 1.44269504088896340736f, kLn2 = 0.69314718055994530942f;
  float mx = FA_NEG_INF;
  for (int s = lane; s < p.splits; s += 64) mx = fmaxf(mx, p.ws_lse[s * split_stride + row]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));

  float acc[PER_LANE];
#pragma unroll
  for (int e = 0; e < PER_LANE; ++e) acc[e] = 0.f;
  float wsum = 0.f;
  if (mx != FA_NEG_INF) {
    for (int s = 0; s < p.splits; ++s) {
      const float ls = p.ws_lse[s * split_stride + row];
      const float w = fast_exp2((ls - mx) * kLog2e);  // 0 for an empty split (ls = -inf)
      wsum += w;
      const float* src = p.ws_o + (s * split_stride + row) * D;
#pragma unroll
      for (int e = 0; e < PER_LANE; ++e) {
        const int d = lane + 64 * e;
        if (d < D) acc[e] += w * src[d];
      }
    }
  }
  const float inv = (wsum > 0.f) ? 1.f / wsum : 0.f;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  uint16_t* orow = p.o + (int64_t)b * p.so0 + (int64_t)h * p.so1 + (int64_t)i * p.so2;
#pragma unroll
  for (int e = 0; e < PER_LANE; ++e) {
    const int d = lane + 64 * e;
    if (d < D) orow[d] = T::from_float(acc[e] * inv);
  }
  if (p.lse != nullptr && lane == 0)
    p.lse[(int64_t)b * p.sl0 + (int64_t)h * p.sl1 + (int64_t)i * p.sl2] =
        (wsum > 0.f) ? mx + __builtin_amdgcn_logf(wsum) * kLn2 : FA_NEG_INF;
}

// ---------------------------------------------------------------------------------------------
// Registry of built instantiations.

#define FA_ENTRY(TAG, DTYPE, D, W, RT, BN, ST, SP) \
  {ST, DTYPE, D, W, 32 * RT, BN, SP, (const void*)&fa_fwd_kernel<TAG, D, W, RT, BN, ST, (SP != 0)>}

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
  FA_ENTRY(TAG, DTYPE, D, 8, 1, 64, 2, 1)

static const FaKernelEntry kFwdEntries[] = {
    FA_ENTRIES_D(f16_t, FA_DTYPE_F16, 64),    FA_ENTRIES_D(f16_t, FA_DTYPE_F16, 128),
    FA_ENTRIES_D(f16_t, FA_DTYPE_F16, 256),   FA_ENTRIES_D(bf16_t, FA_DTYPE_BF16, 64),
    FA_ENTRIES_D(bf16_t, FA_DTYPE_BF16, 128), FA_ENTRIES_D(bf16_t, FA_DTYPE_BF16, 256),
    FA_ENTRIES_D_WIDE(f16_t, FA_DTYPE_F16, 64), FA_ENTRIES_D_WIDE(f16_t, FA_DTYPE_F16, 128),
    FA_ENTRIES_D_WIDE(bf16_t, FA_DTYPE_BF16, 64), FA_ENTRIES_D_WIDE(bf16_t, FA_DTYPE_BF16, 128),
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
