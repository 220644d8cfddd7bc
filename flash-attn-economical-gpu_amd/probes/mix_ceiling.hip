// Instruction-mix ceiling probe for the attention kernel on MI355X (gfx950).
//
// MI355X is power-limited under dense MFMA work: the clock falls well below 2.4 GHz, so the dense
// fp16 peak (2516.6 TFLOP/s) is not reachable by any real kernel, and every non-MFMA instruction
// spends power the MFMAs could have used. This probe measures the throughput of dependency-free
// loops whose per-MFMA mix matches the attention kernel's, step by step:
//
//   mode 0  MFMA only (v_mfma_f32_32x32x16, random fp16 operands rotating over 8 register sets)
//   mode 1  + the A operand read from LDS, 1 KiB per MFMA (one K or V fragment per MFMA, as a wave
//            owning 32 query rows reads them)
//   mode 2  + softmax-like VALU per MFMA (exp2, fma, max, mul: the kernel's ~1 exp + 3 VALU)
//   mode 3  + one workgroup barrier per 32 MFMAs (one per KV tile step)
//   mode 4  + LDS-DMA (buffer_load ... lds) of 256 B per MFMA from L2: the K/V tile traffic of a
//            128-row workgroup. This is the attention kernel's mix.
//   mode 5  as 4 with 128 B/MFMA of DMA (256-row workgroups)
//   mode 6  as 5 with 0.5 KiB of LDS reads per MFMA (64 query rows per wave)
//
// Two four-wave workgroups per CU (two waves per SIMD), as the attention kernel runs. Nothing in the
// loops depends on a previous result except the MFMA accumulators, so the figures are upper bounds
// for kernels with these mixes. Build: python build_lib.py (writes probes/mix_ceiling next to this
// file); run: probes/mix_ceiling on a GPU box.
#include <hip/hip_runtime.h>

#include <stdio.h>
#include <stdlib.h>

#include "../csrc/fa_common.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bhalf8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));

#define PROBE_CHECK(x)                                                                  \
  do {                                                                                  \
    hipError_t e_ = (x);                                                                \
    if (e_ != hipSuccess) {                                                             \
      fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);    \
      exit(1);                                                                          \
    }                                                                                   \
  } while (0)

constexpr int kThreads = 256;       // four waves
constexpr int kFrags = 32;          // LDS fragments of 1 KiB (32 KiB)
constexpr int kSrcChunks = 65536;   // 16-byte chunks of the global source (1 MiB, L2-resident)
constexpr int kMfmaPerIter = 32;    // one KV tile step of a 32-row wave (16 QK + 16 PV)

template <bool BF16>
__device__ inline floatx16 mfma(const u32x4v& a, const u32x4v& b, const floatx16& c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bhalf8, a), __builtin_bit_cast(bhalf8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0,
                                                  0, 0);
}

template <int MODE, bool BF16>
__global__ __launch_bounds__(kThreads, 2) void mix_kernel(const u32x4v* src, float* out, int iters) {
  __shared__ u32x4v frags[kFrags * 64];  // read by the MFMAs (modes >= 1)
  __shared__ u32x4v dma_area[kThreads / 64 * 8 * 64];  // DMA target: 8 KiB per wave, never read
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  for (int i = threadIdx.x; i < kFrags * 64; i += kThreads) frags[i] = src[(blockIdx.x * 2048 + i) % kSrcChunks];
  __syncthreads();
  const auto rsrc = fa::make_rsrc(src, kSrcChunks * 16u);
  const uint32_t dma_lds = fa::lds_address(dma_area) + (uint32_t)wave * 8192u;
  constexpr int lds_every = (MODE == 6) ? 2 : 1;                     // MFMAs per LDS fragment read
  constexpr int dma_every = (MODE == 4) ? 4 : (MODE >= 5 ? 8 : 0);   // MFMAs per 1 KiB DMA per wave

  u32x4v q[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) q[j] = src[(threadIdx.x * 8 + j + blockIdx.x * 3) % kSrcChunks];
  floatx16 c0 = {}, c1 = {};
  float e0 = 0.01f * lane, e1 = 0.02f, e2 = -1.f, e3 = -1.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int f = 0; f < kMfmaPerIter; f += 2) {
      u32x4v a0, a1;
      if (MODE == 0) {
        a0 = q[(f + 3) & 7];
        a1 = q[(f + 6) & 7];
      } else {
        const int fb = (f + 2 * it) & (kFrags - 1);  // varies with it: the reads stay in the loop
        a0 = frags[fb * 64 + lane];
        a1 = (lds_every == 2) ? a0 : frags[(fb ^ 1) * 64 + lane];
      }
      c0 = mfma<BF16>(a0, q[f & 7], c0);
      c1 = mfma<BF16>(a1, q[(f + 1) & 7], c1);
      if (dma_every != 0 && f % dma_every == 0) {
        const uint32_t chunk = ((blockIdx.x * 97u + it * 8u + f / dma_every) * 64u + lane) % kSrcChunks;
        fa::buffer_load16_to_lds(rsrc, chunk * 16u, dma_lds + (uint32_t)(f / dma_every) * 1024u);
      }
      if (MODE >= 2) {
        e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(e0, 0.5f, -0.25f)) * 0.9f;
        e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(e1, 0.5f, -0.25f)) * 0.9f;
        e2 = __builtin_fmaxf(e2, e0) * 0.99f;
        e3 = __builtin_fmaxf(e3, e1) * 0.99f;
      }
    }
    if (MODE >= 3) fa::wait_vm_lds_barrier<0>();
  }
  float s = e0 + e1 + e2 + e3;
#pragma unroll
  for (int r = 0; r < 16; ++r) s += c0[r] + c1[r];
  out[blockIdx.x * kThreads + threadIdx.x] = s;
}

constexpr int kBlocks = 256 * 2 * 8;  // 8 rounds of two workgroups per CU

template <int MODE, bool BF16>
double run(const char* name, const u32x4v* src, float* out, int iters, double ref_tf) {
  // src holds the operands in the MFMA's input type
  hipEvent_t s, e;
  PROBE_CHECK(hipEventCreate(&s));
  PROBE_CHECK(hipEventCreate(&e));
  hipLaunchKernelGGL((mix_kernel<MODE, BF16>), dim3(kBlocks), dim3(kThreads), 0, 0, src, out, iters);
  PROBE_CHECK(hipGetLastError());
  PROBE_CHECK(hipDeviceSynchronize());
  constexpr int reps = 5;
  PROBE_CHECK(hipEventRecord(s));
  for (int r = 0; r < reps; ++r)
    hipLaunchKernelGGL((mix_kernel<MODE, BF16>), dim3(kBlocks), dim3(kThreads), 0, 0, src, out, iters);
  PROBE_CHECK(hipEventRecord(e));
  PROBE_CHECK(hipEventSynchronize(e));
  float ms = 0.f;
  PROBE_CHECK(hipEventElapsedTime(&ms, s, e));
  ms /= reps;
  const double flops = (double)kBlocks * (kThreads / 64) * iters * kMfmaPerIter * 32768.0;
  const double tf = flops / ms / 1e9;
  printf("mode %d %-5s %-58s %8.3f ms %7.1f TFLOP/s %5.1f%% of 2516.6", MODE, BF16 ? "bf16" : "fp16", name, ms, tf,
         100.0 * tf / 2516.6);
  if (ref_tf > 0) printf("  (%.1f%% of mode 0)", 100.0 * tf / ref_tf);
  printf("\n");
  fflush(stdout);
  PROBE_CHECK(hipEventDestroy(s));
  PROBE_CHECK(hipEventDestroy(e));
  return tf;
}

}  // namespace

int main() {
  u32x4v* src = nullptr;     // fp16 operands
  u32x4v* src_bf = nullptr;  // the same values as bf16
  float* out = nullptr;
  PROBE_CHECK(hipMalloc(&src, kSrcChunks * sizeof(u32x4v)));
  PROBE_CHECK(hipMalloc(&src_bf, kSrcChunks * sizeof(u32x4v)));
  PROBE_CHECK(hipMalloc(&out, (size_t)kBlocks * kThreads * sizeof(float)));
  // uniform [-1, 1) operands; the bf16 runs read the same values rounded to bf16
  unsigned short* h = (unsigned short*)malloc(kSrcChunks * 16);
  unsigned short* hb = (unsigned short*)malloc(kSrcChunks * 16);
  unsigned long long x = 0x9E3779B97F4A7C15ull;
  for (int i = 0; i < kSrcChunks * 8; ++i) {
    x = x * 6364136223846793005ull + 1442695040888963407ull;
    const float v = (float)((x >> 40) & 0xFFFFFF) / 16777216.0f * 2.f - 1.f;
    h[i] = __builtin_bit_cast(unsigned short, (_Float16)v);
    hb[i] = __builtin_bit_cast(unsigned short, (__bf16)v);
  }
  PROBE_CHECK(hipMemcpy(src, h, kSrcChunks * 16, hipMemcpyHostToDevice));
  PROBE_CHECK(hipMemcpy(src_bf, hb, kSrcChunks * 16, hipMemcpyHostToDevice));
  free(h);
  free(hb);
  const int iters = 400;
  for (int rep = 0; rep < 2; ++rep) {
    printf("-- pass %d\n", rep + 1);
    const double m0 = run<0, false>("MFMA only", src, out, iters, 0);
    run<1, false>("+ A operand from LDS, 1 KiB/MFMA", src, out, iters, m0);
    run<2, false>("+ exp/fma/max VALU per MFMA", src, out, iters, m0);
    run<3, false>("+ barrier per 32 MFMAs", src, out, iters, m0);
    run<4, false>("+ LDS-DMA 256 B/MFMA (attention kernel's mix)", src, out, iters, m0);
    run<5, false>("  DMA 128 B/MFMA (256-row workgroups)", src, out, iters, m0);
    run<6, false>("  DMA 128 B + LDS 0.5 KiB per MFMA (64-row waves)", src, out, iters, m0);
    const double b0 = run<0, true>("MFMA only", src_bf, out, iters, 0);
    run<4, true>("attention kernel's mix", src_bf, out, iters, b0);
  }
  PROBE_CHECK(hipFree(src));
  PROBE_CHECK(hipFree(src_bf));
  PROBE_CHECK(hipFree(out));
  return 0;
}
