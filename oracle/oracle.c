/*
 * oracle.c -- CPU restatement of the reference's hot-path arithmetic. TEST INFRASTRUCTURE ONLY:
 * imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker; the
 * product (libfa_gfx950.so and the Python modules beside it) never links or calls it.
 *
 * Reference citations are relative to the reference repository.
 *
 *  oracle_attention        exact softmax(Q K^T * scale) V in double precision, with top-left causal
 *                          mask, GQA head mapping and LSE. This is the mathematics every reference
 *                          kernel computes (flash_atten.py:14-133, 136-258, 261-361) and what the
 *                          reference tests check against (CPU fp32 SDPA, test_flash_atten.py:459-461,
 *                          498-499). GQA mapping h -> h / (H / H_kv) matches repeat_interleave
 *                          (ttft.py:203-209). LSE = m + ln(l) over scaled logits (flash_atten.py:130-133).
 *  oracle_attention_rows   the same for a list of (b, h, m) query rows (full-size spot checks).
 *  oracle_attention_online the reference kernel's own blocked algorithm in fp32
 *                          (flash_atten.py:76-133): per BLOCK_N keys, m_ij = max(m_i, rowmax),
 *                          p = exp(qk - m_ij), alpha = exp(m_i - m_ij), acc = acc*alpha + round(p) V,
 *                          l = l*alpha + sum(p), with p rounded to the input dtype before PV
 *                          (flash_atten.py:113).
 *  oracle_lse_merge        merge of split-KV partials: lse = ln sum_j exp(lse_j),
 *                          O = sum_j exp(lse_j - lse) O_j (no reference function; north-star "sliced").
 *  oracle_gemm             C = A B with double accumulation (mma.py:39-52 computes it in fp32).
 *  oracle_gemm_entries     selected entries C[i][j] of the same product.
 *  oracle_round_f16/bf16   IEEE round-to-nearest-even to binary16 / bfloat16 (the `.to(dtype)` casts).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- rounding to 16-bit formats (IEEE 754 round-to-nearest-even) ------------------------- */

static uint16_t f32_to_f16_bits(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (ax < 0x38800000u) { /* below 2^-14: binary16 subnormal, unit 2^-24 */
    float af;
    memcpy(&af, &ax, 4);
    const uint32_t m = (uint32_t)nearbyintf(af * 16777216.0f); /* exact scaling, RNE */
    return (uint16_t)(sign | m);
  }
  const uint32_t mant = ax & 0x7fffffu;
  const uint32_t exp = (ax >> 23) - 127u + 15u;
  uint32_t h = (exp << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* carry may reach infinity */
  if (h >= 0x7c00u) h = 0x7c00u;
  return (uint16_t)(sign | h);
}

static float f16_bits_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
  const uint32_t mant = (uint32_t)h & 0x3ffu;
  float out;
  if (exp == 0) {
    out = ldexpf((float)mant, -24);
    if (sign) out = -out;
    return out;
  }
  uint32_t x;
  if (exp == 31) x = sign | 0x7f800000u | (mant << 13);
  else x = sign | ((exp - 15u + 127u) << 23) | (mant << 13);
  memcpy(&out, &x, 4);
  return out;
}

static float round_bf16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) x = (x | 0x00400000u) & 0xffff0000u;
  else x = (x + 0x7fffu + ((x >> 16) & 1u)) & 0xffff0000u;
  float out;
  memcpy(&out, &x, 4);
  return out;
}

float oracle_round_f16(float f) { return f16_bits_to_f32(f32_to_f16_bits(f)); }
float oracle_round_bf16(float f) { return round_bf16(f); }

void oracle_round_array(const float* in, float* out, int64_t n, int dtype) {
  for (int64_t i = 0; i < n; ++i) out[i] = dtype == 1 ? round_bf16(in[i]) : oracle_round_f16(in[i]);
}

/* ---- attention ------------------------------------------------------------------------------ */

/* One query row: o[D], returns lse. q row, k/v head base pointers, N keys. Keys j with
 * causal && j > m are masked (top-left causal, flash_atten.py:103-105). */
static double attention_row(const float* qr, const float* kh, const float* vh, float* orow, int64_t m, int N,
                            int D, double scale, int causal, double* work) {
  int n_eff = N;
  if (causal && m + 1 < (int64_t)n_eff) n_eff = (int)(m + 1);
  double mx = -INFINITY;
  for (int j = 0; j < n_eff; ++j) {
    const float* kr = kh + (int64_t)j * D;
    double s = 0.0;
    for (int d = 0; d < D; ++d) s += (double)qr[d] * (double)kr[d];
    s *= scale;
    work[j] = s;
    if (s > mx) mx = s;
  }
  double l = 0.0;
  for (int j = 0; j < n_eff; ++j) {
    work[j] = exp(work[j] - mx);
    l += work[j];
  }
  for (int d = 0; d < D; ++d) {
    double acc = 0.0;
    for (int j = 0; j < n_eff; ++j) acc += work[j] * (double)vh[(int64_t)j * D + d];
    orow[d] = (n_eff > 0) ? (float)(acc / l) : NAN;
  }
  return (n_eff > 0) ? mx + log(l) : -INFINITY;
}

/* q [B,H,M,D], k/v [B,Hkv,N,D], o [B,H,M,D], lse [B,H,M] (nullable); all contiguous fp32. */
int oracle_attention(const float* q, const float* k, const float* v, float* o, float* lse, int B, int H, int Hkv,
                     int M, int N, int D, double scale, int causal) {
  if (H % Hkv != 0) return 1;
  double* work = (double*)malloc(sizeof(double) * (size_t)(N > 0 ? N : 1));
  if (!work) return 2;
  const int group = H / Hkv;
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      const int hk = h / group;
      const float* kh = k + ((int64_t)b * Hkv + hk) * N * D;
      const float* vh = v + ((int64_t)b * Hkv + hk) * N * D;
      for (int m = 0; m < M; ++m) {
        const int64_t row = ((int64_t)b * H + h) * M + m;
        const double l = attention_row(q + row * D, kh, vh, o + row * D, m, N, D, scale, causal, work);
        if (lse) lse[row] = (float)l;
      }
    }
  free(work);
  return 0;
}

/* rows[i] = flattened (b*H + h)*M + m; o_rows [nrows, D]; lse_rows [nrows] (nullable). */
int oracle_attention_rows(const float* q, const float* k, const float* v, const int64_t* rows, int64_t nrows,
                          float* o_rows, float* lse_rows, int B, int H, int Hkv, int M, int N, int D, double scale,
                          int causal) {
  if (H % Hkv != 0) return 1;
  double* work = (double*)malloc(sizeof(double) * (size_t)(N > 0 ? N : 1));
  if (!work) return 2;
  const int group = H / Hkv;
  for (int64_t i = 0; i < nrows; ++i) {
    const int64_t row = rows[i];
    if (row < 0 || row >= (int64_t)B * H * M) {
      free(work);
      return 3;
    }
    const int64_t m = row % M;
    const int64_t bh = row / M;
    const int b = (int)(bh / H), h = (int)(bh % H), hk = h / group;
    const float* kh = k + ((int64_t)b * Hkv + hk) * N * D;
    const float* vh = v + ((int64_t)b * Hkv + hk) * N * D;
    const double l = attention_row(q + row * D, kh, vh, o_rows + i * D, m, N, D, scale, causal, work);
    if (lse_rows) lse_rows[i] = (float)l;
  }
  free(work);
  return 0;
}

/* The reference kernel's blocked online softmax in fp32 (flash_atten.py:76-133), BLOCK_N keys per
 * step, p rounded to `dtype` (0 fp16, 1 bf16) before the PV product; output rounded to dtype. */
int oracle_attention_online(const float* q, const float* k, const float* v, float* o, float* lse, int B, int H,
                            int Hkv, int M, int N, int D, float sm_scale, int causal, int block_n, int dtype) {
  if (H % Hkv != 0 || block_n <= 0) return 1;
  const int group = H / Hkv;
  float* qk = (float*)malloc(sizeof(float) * (size_t)block_n);
  float* acc = (float*)malloc(sizeof(float) * (size_t)D);
  if (!qk || !acc) {
    free(qk);
    free(acc);
    return 2;
  }
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      const int hk = h / group;
      const float* kh = k + ((int64_t)b * Hkv + hk) * N * D;
      const float* vh = v + ((int64_t)b * Hkv + hk) * N * D;
      for (int m = 0; m < M; ++m) {
        const int64_t row = ((int64_t)b * H + h) * M + m;
        const float* qr = q + row * D;
        float m_i = -INFINITY, l_i = 0.f;
        for (int d = 0; d < D; ++d) acc[d] = 0.f;
        for (int n0 = 0; n0 < N; n0 += block_n) {
          float rowmax = -INFINITY;
          for (int jj = 0; jj < block_n; ++jj) {
            const int j = n0 + jj;
            float s = -INFINITY;
            if (j < N && !(causal && m < j)) {
              float dot = 0.f;
              for (int d = 0; d < D; ++d) dot += qr[d] * kh[(int64_t)j * D + d];
              s = dot * sm_scale;
            }
            qk[jj] = s;
            if (s > rowmax) rowmax = s;
          }
          const float m_ij = m_i > rowmax ? m_i : rowmax;
          const float alpha = expf(m_i - m_ij);
          float l_ij = 0.f;
          for (int d = 0; d < D; ++d) acc[d] *= alpha;
          for (int jj = 0; jj < block_n; ++jj) {
            const float p = expf(qk[jj] - m_ij);
            l_ij += p;
            const float pr = dtype == 1 ? round_bf16(p) : oracle_round_f16(p);
            const int j = n0 + jj;
            if (pr != 0.f && j < N)
              for (int d = 0; d < D; ++d) acc[d] += pr * vh[(int64_t)j * D + d];
          }
          l_i = l_i * alpha + l_ij;
          m_i = m_ij;
        }
        for (int d = 0; d < D; ++d) {
          const float out = acc[d] / l_i;
          o[row * D + d] = dtype == 1 ? round_bf16(out) : oracle_round_f16(out);
        }
        if (lse) lse[row] = m_i + logf(l_i);
      }
    }
  free(qk);
  free(acc);
  return 0;
}

/* o_parts [splits][rows][D], lse_parts [splits][rows] -> o [rows][D], lse [rows]. */
int oracle_lse_merge(const float* o_parts, const float* lse_parts, int splits, int64_t rows, int D, float* o,
                     float* lse) {
  for (int64_t r = 0; r < rows; ++r) {
    double mx = -INFINITY;
    for (int s = 0; s < splits; ++s)
      if (lse_parts[s * rows + r] > mx) mx = lse_parts[s * rows + r];
    double wsum = 0.0;
    for (int d = 0; d < D; ++d) o[r * D + d] = 0.f;
    if (mx == -INFINITY) {
      lse[r] = -INFINITY;
      continue;
    }
    double* acc = (double*)calloc((size_t)D, sizeof(double));
    if (!acc) return 2;
    for (int s = 0; s < splits; ++s) {
      const double w = exp((double)lse_parts[s * rows + r] - mx);
      wsum += w;
      for (int d = 0; d < D; ++d) acc[d] += w * (double)o_parts[((int64_t)s * rows + r) * D + d];
    }
    for (int d = 0; d < D; ++d) o[r * D + d] = (float)(acc[d] / wsum);
    lse[r] = (float)(mx + log(wsum));
    free(acc);
  }
  return 0;
}

/* ---- GEMM ------------------------------------------------------------------------------------ */

/* a [M,K], b [K,N], c [M,N] row-major fp32, double accumulation. */
int oracle_gemm(const float* a, const float* b, float* c, int M, int N, int K) {
  double* row = (double*)malloc(sizeof(double) * (size_t)(N > 0 ? N : 1));
  if (!row) return 2;
  for (int i = 0; i < M; ++i) {
    for (int j = 0; j < N; ++j) row[j] = 0.0;
    for (int kk = 0; kk < K; ++kk) {
      const double av = a[(int64_t)i * K + kk];
      const float* br = b + (int64_t)kk * N;
      for (int j = 0; j < N; ++j) row[j] += av * (double)br[j];
    }
    for (int j = 0; j < N; ++j) c[(int64_t)i * N + j] = (float)row[j];
  }
  free(row);
  return 0;
}

/* out[t] = sum_k a[ii[t]][k] * b[k][jj[t]] in double (returned as double). */
int oracle_gemm_entries(const float* a, const float* b, const int64_t* ii, const int64_t* jj, int64_t n, double* out,
                        int M, int N, int K) {
  for (int64_t t = 0; t < n; ++t) {
    if (ii[t] < 0 || ii[t] >= M || jj[t] < 0 || jj[t] >= N) return 3;
    double s = 0.0;
    for (int kk = 0; kk < K; ++kk) s += (double)a[ii[t] * K + kk] * (double)b[(int64_t)kk * N + jj[t]];
    out[t] = s;
  }
  return 0;
}
