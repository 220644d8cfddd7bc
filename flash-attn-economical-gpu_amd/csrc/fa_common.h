// Device-side helpers shared by the attention and GEMM kernels (gfx950 / CDNA4 only).
//
// MFMA fragment conventions used throughout (v_mfma_f32_32x32x16_{f16,bf16}, wave64):
//   lane l, col = l & 31, half = l >> 5
//   A operand (32 x 16): lane holds row `col`, k-slots 8*half .. 8*half+7   (8 x 16-bit)
//   B operand (16 x 32): lane holds column `col`, k-slots 8*half .. 8*half+7 (8 x 16-bit)
//   C/D (32 x 32 fp32): lane holds column `col`, register r holds row 8*(r/4) + 4*half + (r%4)
// The hardware pairs A's and B's k-slots identically, so any permutation of the 16 k values that
// is applied to both operands leaves the product unchanged; the kernels rely on that.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct f16_t {};   // tag: IEEE binary16 storage
struct bf16_t {};  // tag: bfloat16 storage

template <typename Tag>
struct DT;

template <>
struct DT<f16_t> {
  typedef half8 vec8;
  __device__ static inline floatx16 mfma32(const u32x4& a, const u32x4& b, const floatx16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a),
                                                  __builtin_bit_cast(half8, b), c, 0, 0, 0);
  }
  __device__ static inline floatx4 mfma16(const u32x4& a, const u32x4& b, const floatx4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a),
                                                  __builtin_bit_cast(half8, b), c, 0, 0, 0);
  }
  // Two fp32 -> packed pair of binary16 (round to nearest even), low half = x.
  __device__ static inline uint32_t pack2(float x, float y) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    h2 v;
    v[0] = (_Float16)x;
    v[1] = (_Float16)y;
    return __builtin_bit_cast(uint32_t, v);
  }
  __device__ static inline float to_float(uint16_t bits) {
    return (float)__builtin_bit_cast(_Float16, bits);
  }
  __device__ static inline uint16_t from_float(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  }
};

template <>
struct DT<bf16_t> {
  typedef bf16x8 vec8;
  __device__ static inline floatx16 mfma32(const u32x4& a, const u32x4& b, const floatx16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static inline floatx4 mfma16(const u32x4& a, const u32x4& b, const floatx4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack2(float x, float y) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    b2 v;
    v[0] = (__bf16)x;
    v[1] = (__bf16)y;
    return __builtin_bit_cast(uint32_t, v);
  }
  __device__ static inline float to_float(uint16_t bits) {
    return __uint_as_float(((uint32_t)bits) << 16);
  }
  __device__ static inline uint16_t from_float(float x) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
  }
};

// Value of x in lane (l ^ 32), through the LDS crossbar (ds_bpermute).
__device__ inline float xhalf(float x) {
  return __shfl_xor(x, 32, 64);
}

// max(x[l], x[l ^ 32]) in every lane with one v_permlane32_swap (a VALU op, no LDS round trip):
// swapping lanes 32..63 of a copy with lanes 0..31 of another copy leaves, in each lane, its own
// value in one result and its partner's value in the other.
__device__ inline float xhalf_max(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ inline float xhalf_sum(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// max / sum over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (the 16-lane rows of a wave that hold
// one column of a 16x16 MFMA tile): v_permlane32_swap, then v_permlane16_swap, which swaps the odd
// 16-lane rows of one copy with the even rows of another.
__device__ inline float xquad_max(float x) {
  const float h = xhalf_max(x);
  const uint32_t u = __float_as_uint(h);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ inline float xquad_sum(float x) {
  const float h = xhalf_sum(x);
  const uint32_t u = __float_as_uint(h);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

#define FA_NEG_INF (-__builtin_inff())

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// 4 x 16-bit transposing LDS read (ds_read_b64_tr_b16), returned as two dwords: in each 16-lane
// group, lane L addresses 4 elements of row L >> 2 at columns 4 (L & 3) .. +3 of a 4 x 16 block,
// and result lane i holds column i of the 4 rows.
__device__ inline u32x2 lds_read_tr16(const uint16_t* p) {
  s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(u32x2, r);
}

// acc + the two 16-bit values of `packed` (v_dot2 with (1, 1)).
template <typename Tag>
__device__ inline float dot2_sum(uint32_t packed, float acc);
template <>
__device__ inline float dot2_sum<f16_t>(uint32_t packed, float acc) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, packed), (h2){(_Float16)1.0f, (_Float16)1.0f}, acc, false);
}
template <>
__device__ inline float dot2_sum<bf16_t>(uint32_t packed, float acc) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, packed), (b2){(__bf16)1.0f, (__bf16)1.0f}, acc,
                                         false);
}

// Raw buffer resource (the four descriptor words) over [base, base + bytes): buffer loads address
// it with a 32-bit per-lane byte offset and return zeros for offsets at or past `bytes` (the
// hardware range check), so tiles that run past the end of a sequence need no branch. Word 1
// carries stride 0 (raw buffer); 0x00020000 is the gfx9-family word 3 for untyped 32-bit data.
// Callers pass wave-uniform values; readfirstlane puts them in scalar registers.
__device__ inline u32x4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  u32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) & 0xffffu;
  r[2] = __builtin_amdgcn_readfirstlane(bytes);
  r[3] = 0x00020000u;
  return r;
}

// The resource of make_rsrc moved `shift` bytes on (shift <= its range: the range shrinks by as
// much, so a load at offset o of the result reads zeros exactly where o + shift did in `r`), or
// with range 0 (every load reads zeros) when !live. Scalar arithmetic only: r, shift and live are
// uniform.
__device__ inline u32x4 slab_rsrc(const u32x4& r, uint32_t shift, bool live) {
  const uint64_t a = (((uint64_t)r[1] << 32) | r[0]) + shift;  // base < 2^48: no carry into the stride
  u32x4 s;
  s[0] = (uint32_t)a;
  s[1] = (uint32_t)(a >> 32);
  s[2] = live ? r[2] - shift : 0u;
  s[3] = r[3];
  return s;
}

// 16 bytes per lane from the buffer straight into LDS (buffer_load_dwordx4 ... lds): lane i writes
// lds_block[16 i .. 16 i + 15], so one wave instruction fills one contiguous 1 KiB block (M0 holds
// the wave-uniform block address). Completion is tracked by vmcnt. The instruction is issued from
// inline asm so that the compiler, which cannot tell the ring slots apart, does not wait for every
// LDS-DMA in flight before each LDS read; the kernel waits explicitly (wait_vm_lds_barrier).
// vmcnt retires in order, so the compiler's own vmcnt waits stay correct (they can only wait
// longer when these loads are outstanding).
// `lds_block` is the block's LDS byte address (lds_address of the __shared__ array plus a
// wave-uniform offset), so M0 is computed with scalar instructions. IMM is the instruction's 12-bit
// offset field: the hardware adds it to the memory offset (byte_off) AND to the LDS address
// (M0 + IMM + 16 * lane), so M0 is set to lds_block - IMM.
// GUARD: 5 wait states before the load. On gfx9 a vector-memory instruction must not read an SGPR
// (here the descriptor) within 5 wait states of a VALU write to it (v_readfirstlane, or v_readlane
// restoring an SGPR the compiler spilled to a VGPR lane); the compiler inserts those for its own
// memory instructions but cannot see into inline asm. Kernels whose build shows such a write
// before this asm take the guard (build_lib.py checks every kernel's assembly for it).
template <int IMM = 0, bool GUARD = false>
__device__ inline void buffer_load16_to_lds(const u32x4& rsrc, uint32_t byte_off, uint32_t lds_block) {
  static_assert(IMM >= 0 && IMM < 4096, "12-bit immediate offset");
  const uint32_t lds = __builtin_amdgcn_readfirstlane(lds_block - (uint32_t)IMM);
  if constexpr (GUARD) {
    asm volatile("s_nop 4\n\ts_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen offset:%3 lds"
                 :
                 : "v"(byte_off), "s"(lds), "s"(rsrc), "n"(IMM)
                 : "memory", "m0");
  } else {
    asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen offset:%3 lds"
                 :
                 : "v"(byte_off), "s"(lds), "s"(rsrc), "n"(IMM)
                 : "memory", "m0");
  }
}

// N consecutive 1 KiB blocks whose per-lane sources are STEP bytes apart: one offset register, the
// steps in the immediate field.
template <int N, int STEP, int J = 0, bool GUARD = false>
__device__ inline void buffer_load16_to_lds_blocks(const u32x4& rsrc, uint32_t byte_off, uint32_t lds_block) {
  if constexpr (J < N) {
    buffer_load16_to_lds<J * STEP, GUARD>(rsrc, byte_off, lds_block + J * 1024u);
    buffer_load16_to_lds_blocks<N, STEP, J + 1, GUARD>(rsrc, byte_off, lds_block);
  }
}

// LDS byte address of a __shared__ array (the generic -> LDS cast of the array itself folds to a
// constant; casting a computed generic pointer would add a null check).
__device__ inline uint32_t lds_address(const void* shared_array) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)shared_array;
}

// Wait until at most N vector-memory operations of this wave are outstanding and all its LDS
// operations are done, then barrier. Unlike __syncthreads() this does not wait for every
// outstanding load: LDS-DMA loads issued for later steps stay in flight across the barrier.
// (gfx9 s_waitcnt encoding: vmcnt [3:0] and [15:14], expcnt [6:4] (7 = no wait), lgkmcnt [11:8].)
template <int N>
__device__ inline void wait_vm_lds_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The kernel's parameter struct read straight from the kernel-argument segment (scalar loads at
// the point of use, instead of scalar registers held across a loop). Valid only for a kernel whose
// one and only argument is a `P` passed by value: it then sits at offset 0 of the segment. Kernels
// that call this pin their signature with kernel_has_sole_arg<P>(&kernel) (a compile-time check).
template <typename P>
__device__ inline const __attribute__((address_space(4))) P* kernarg_params() {
  typedef const __attribute__((address_space(4))) P* Ptr;
  Ptr ptr = (Ptr)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(ptr));
  return ptr;
}
template <typename P>
constexpr bool kernel_has_sole_arg(void (*)(P)) { return true; }
template <typename P, typename... Other>
constexpr bool kernel_has_sole_arg(void (*)(Other...)) { return false; }

// Workgroup id remapped so that consecutive logical ids land on the same XCD. Workgroups are
// dispatched round-robin over the 8 XCDs of MI355X; logical id L = xcd * per + slot keeps
// neighbouring tiles (which share K/V or A/B panels) inside one XCD's L2.
__device__ inline int xcd_remap(int pid, int total) {
  constexpr int kXcds = 8;
  if (total % kXcds != 0) return pid;
  const int per = total / kXcds;
  return (pid % kXcds) * per + (pid / kXcds);
}

}  // namespace fa
