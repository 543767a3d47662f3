// mfma_common.h -- gfx950 MFMA operand helpers shared by the quantized
// matmul and attention kernels.
//
// v_mfma_f32_16x16x32_{bf16,f16} operand layout (wave64):
//   A[16 x 32]: lane l supplies row l%16, k = 8*(l/16) + e (e = 0..7)
//   B[32 x 16]: lane l supplies col l%16, k = 8*(l/16) + e
//   D[16 x 16]: lane l holds rows 4*(l/16) + i (i = 0..3), col l%16
// Only the pairing of A's and B's k slots matters for the product, so the
// kernels are free to permute k inside a lane's 8 slots as long as both
// operands use the same permutation.
//
// Packed codes become exact MFMA operands without a per-element convert:
// OR-ing a code c < 128 into the mantissa of bf16 128.0 (0x4300) gives the
// bf16 value 128 + c exactly; the same trick on f16 1024.0 (0x6400) gives
// 1024 + c for c < 1024.  The offset is removed after the contraction with
// the sum of the other operand (sum_k x_k (c_k + off) = sum x c + off * sum x).
#pragma once

#include "mlxq_internal.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// (x & mask) | (y & ~mask): one v_bfi_b32 when y is not a compile-time
// constant (see opaque()).
__device__ __forceinline__ uint32_t bfi32(uint32_t mask, uint32_t x, uint32_t y) { return (x & mask) | (y & ~mask); }

// Hide a constant from the optimiser so it lives in a register and bit
// selects against it lower to v_bfi_b32 instead of and + or.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

template <typename T>
struct Mma;

template <>
struct Mma<BF16> {
  static constexpr uint32_t MAGIC = 0x43004300u;  // bf16 pair (128, 128)
  static constexpr float MAGIC_VAL = 128.0f;
  static constexpr uint32_t ONES = 0x3f803f80u;   // bf16 pair (1, 1)
  __device__ static __forceinline__ f32x4_t mma(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  }
  // two floats -> packed pair of T (round to nearest even, v_cvt_pk_bf16_f32)
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
  }
  // acc + lo + hi of a packed pair (v_dot2c_f32_bf16 against (1, 1))
  __device__ static __forceinline__ float sum2(uint32_t pair, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pair), __builtin_bit_cast(bf16x2_t, ONES), acc,
                                           false);
  }
};

template <>
struct Mma<F16> {
  static constexpr uint32_t MAGIC = 0x64006400u;  // f16 pair (1024, 1024)
  static constexpr float MAGIC_VAL = 1024.0f;
  static constexpr uint32_t ONES = 0x3c003c00u;   // f16 pair (1, 1)
  __device__ static __forceinline__ f32x4_t mma(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {  // v_cvt_pk_f16_f32
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, f16x2_t));
  }
  __device__ static __forceinline__ float sum2(uint32_t pair, float acc) {  // v_dot2c_f32_f16
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, pair), __builtin_bit_cast(f16x2_t, ONES), acc, false);
  }
};

// Raw buffer resource over `bytes` bytes from `base` (gfx9 descriptor word 3
// = 0x00020000): loads past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// Cache policy of a buffer load (the instruction's aux bits): 0 = default,
// LOAD_STREAM = nt, for data a launch reads exactly once in whole lines
// (KV codes and scales in decode).  A 37.7 MB streaming read with nt loads
// runs at 5.57 TB/s on MI355X against 5.0-5.2 TB/s without; qmv, whose
// loads take half of a 128-byte line each, runs 10 % slower with them.
constexpr int LOAD_STREAM = 2;

template <int AUX = 0>
__device__ __forceinline__ uint32_t buf_load32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, AUX);
}
template <int AUX = 0>
__device__ __forceinline__ u32x4_t buf_load128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, AUX));
}
template <int AUX = 0>
__device__ __forceinline__ uint32_t buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, AUX);
}

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt left at their maxima): the
// kernels that load straight into LDS wait on their own counts (the compiler
// does not track those loads' data)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

typedef __attribute__((address_space(3))) uint8_t lds_u8;  // LDS byte (32-bit addresses)

// Workgroup barrier that orders LDS only.  __syncthreads() also orders
// global memory, which compiles to s_waitcnt vmcnt(0) before s_barrier: every
// wave would wait for all of its outstanding global loads, draining any
// register prefetch carried across the barrier.  Here only LDS accesses
// (lgkmcnt) are completed first.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// v_mfma_f32_32x32x16_{bf16,f16}: A [32 x 16] lane l = row l % 32, k slots
// 8 (l / 32) .. + 8; B likewise by column; D [32 x 32] lane l = column
// l % 32, rows 8 (v / 4) + 4 (l / 32) + v % 4 for v = 0..15.
template <typename T>
__device__ __forceinline__ f32x16_t mma32(u32x4_t a, u32x4_t b, f32x16_t c) {
  if constexpr (std::is_same<T, BF16>::value)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0,
                                                  0, 0);
}

__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// 4 x 4 dword transpose across the lane quarters (lanes l, l+16, l+32, l+48):
// on entry quarter q holds a_q[0..3]; on exit word k of quarter q is a_k[q].
__device__ __forceinline__ void quarter_transpose(uint32_t (&w)[4]) {
  auto s02 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
  auto s13 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
  auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
  auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
  w[0] = s01[0];
  w[1] = s01[1];
  w[2] = s23[0];
  w[3] = s23[1];
}

// ---- code -> operand conversion --------------------------------------------
//
// The 8 k slots of one operand come from 8 consecutive codes of a row.  The
// slot order each conversion produces (SlotOrder) must be applied to the
// other operand (see permute8 below).
//   4-bit (bf16 or f16): slots [c0,c4,c1,c5,c2,c6,c3,c7], value off + c
//   8-bit bf16:          slots [c0..c7] natural, value c (exact), off = 0
//   8-bit f16:           slots [c0,c2,c1,c3,c4,c6,c5,c7], value 1024 + c
enum SlotOrder { ORDER_NIBBLE = 0, ORDER_NATURAL = 1, ORDER_BYTEPAIR = 2 };

template <typename T, int BITS>
struct CodeOps;

template <typename T>
struct CodeOps<T, 4> {
  static constexpr int ORDER = ORDER_NIBBLE;
  static constexpr float OFFSET = Mma<T>::MAGIC_VAL;
  // w holds codes c0..c7 (c_j at bits 4j..4j+3)
  __device__ static __forceinline__ u32x4_t operand(uint32_t w) {
    u32x4_t r;
    r.x = (w & 0x000f000fu) | Mma<T>::MAGIC;
    r.y = ((w >> 4) & 0x000f000fu) | Mma<T>::MAGIC;
    r.z = ((w >> 8) & 0x000f000fu) | Mma<T>::MAGIC;
    r.w = ((w >> 12) & 0x000f000fu) | Mma<T>::MAGIC;
    return r;
  }
  // same slots, with `magic` = opaque(Mma<T>::MAGIC): 3 shifts + 4 v_bfi_b32
  __device__ static __forceinline__ u32x4_t operand(uint32_t w, uint32_t magic) {
    u32x4_t r;
    r.x = bfi32(0x000f000fu, w, magic);
    r.y = bfi32(0x000f000fu, w >> 4, magic);
    r.z = bfi32(0x000f000fu, w >> 8, magic);
    r.w = bfi32(0x000f000fu, w >> 12, magic);
    return r;
  }
};

template <>
struct CodeOps<BF16, 8> {
  static constexpr int ORDER = ORDER_NATURAL;
  static constexpr float OFFSET = 0.0f;
  // w0 = c0..c3, w1 = c4..c7 (bytes); integers <= 255 are exact in bf16 and
  // the bf16 of an exact small float is its upper half.
  __device__ static __forceinline__ uint32_t two(uint32_t w, int lo_byte) {
    float a = (float)((w >> (8 * lo_byte)) & 0xffu);
    float b = (float)((w >> (8 * lo_byte + 8)) & 0xffu);
    return perm_b32(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
  }
  __device__ static __forceinline__ u32x4_t operand(uint32_t w0, uint32_t w1) {
    u32x4_t r;
    r.x = two(w0, 0);
    r.y = two(w0, 2);
    r.z = two(w1, 0);
    r.w = two(w1, 2);
    return r;
  }
};

template <>
struct CodeOps<F16, 8> {
  static constexpr int ORDER = ORDER_BYTEPAIR;
  static constexpr float OFFSET = 1024.0f;
  __device__ static __forceinline__ u32x4_t operand(uint32_t w0, uint32_t w1) {
    u32x4_t r;
    r.x = (w0 & 0x00ff00ffu) | 0x64006400u;
    r.y = ((w0 >> 8) & 0x00ff00ffu) | 0x64006400u;
    r.z = (w1 & 0x00ff00ffu) | 0x64006400u;
    r.w = ((w1 >> 8) & 0x00ff00ffu) | 0x64006400u;
    return r;
  }
};

// Reorder 8 consecutive 16-bit values (4 dwords, natural order) into the
// slot order a code conversion produces.
template <int ORDER>
__device__ __forceinline__ u32x4_t permute8(u32x4_t d) {
  if (ORDER == ORDER_NIBBLE) {  // [0,4,1,5,2,6,3,7]
    u32x4_t r;
    r.x = perm_b32(d.z, d.x, 0x05040100u);
    r.y = perm_b32(d.z, d.x, 0x07060302u);
    r.z = perm_b32(d.w, d.y, 0x05040100u);
    r.w = perm_b32(d.w, d.y, 0x07060302u);
    return r;
  } else if (ORDER == ORDER_BYTEPAIR) {  // [0,2,1,3,4,6,5,7]
    u32x4_t r;
    r.x = perm_b32(d.y, d.x, 0x05040100u);
    r.y = perm_b32(d.y, d.x, 0x07060302u);
    r.z = perm_b32(d.w, d.z, 0x05040100u);
    r.w = perm_b32(d.w, d.z, 0x07060302u);
    return r;
  } else {
    return d;
  }
}
