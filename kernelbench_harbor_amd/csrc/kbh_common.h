// Shared device/host helpers for the gfx950 (CDNA4) quantized-GEMM kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kbh_qgemm.h"

typedef _Float16 kbh_f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 kbh_bf16x8 __attribute__((ext_vector_type(8)));
typedef float kbh_f32x4 __attribute__((ext_vector_type(4)));
typedef float kbh_f32x16 __attribute__((ext_vector_type(16)));
typedef int kbh_i32x4 __attribute__((ext_vector_type(4)));
typedef int kbh_i32x8 __attribute__((ext_vector_type(8)));
typedef int kbh_i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t kbh_u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t kbh_u32x4 __attribute__((ext_vector_type(4)));

namespace kbh {

// Records the HIP error of the last failed launch (read back through kbh_last_hip_error).
void set_last_hip_error(int e);

// Translates hipGetLastError() after a launch into a kbh_status.
int launch_status();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// ---- device helpers -------------------------------------------------------------------

// Workgroups of one launch are dealt to the 8 XCDs round-robin (linear id % 8). Remapping the
// linear id so that each XCD receives one contiguous range of logical ids keeps the tiles that
// share cache lines, or that reduce into the same output tile, inside one XCD's L2.
__device__ inline int xcd_remap(int bid, int nblocks) {
  if ((nblocks & 7) != 0) return bid;
  return (bid & 7) * (nblocks >> 3) + (bid >> 3);
}

// Buffer resource over [p, p + bytes) (bytes clamped to 4 GiB - 1) for raw buffer loads: offsets
// at or past the end read as zero. Word 3 is the gfx9 raw-buffer format (32-bit data, no swizzle).
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* p, size_t bytes) {
  const int n = bytes >= 0xffffffffu ? -1 : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, n, 0x00020000);
}
// Cache policy of streaming loads (read once): the nt bit.
constexpr int kBufNT = 2;

// 16x16x32 MFMA, fp16 or bf16 operands (8 values per lane, packed in 4 dwords), fp32 accumulate.
// Lane l holds A[row l%16][k 8(l/16)..+8] and B[k 8(l/16)..+8][col l%16]; C lane l holds
// C[4(l/16)+i][l%16], i = 0..3.
template <bool BF16>
__device__ inline kbh_f32x4 mfma16x16x32(kbh_u32x4 a, kbh_u32x4 b, kbh_f32x4 c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(kbh_bf16x8, a),
                                                   __builtin_bit_cast(kbh_bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(kbh_f16x8, a),
                                                  __builtin_bit_cast(kbh_f16x8, b), c, 0, 0, 0);
  }
}

// 32x32x16 MFMA (fp16/bf16). Lane l holds A[row l%32][k 8(l/32)..+8], B[k 8(l/32)..+8][col l%32];
// C lane l holds C[8(i/4) + 4(l/32) + i%4][l%32], i = 0..15.
template <bool BF16>
__device__ inline kbh_f32x16 mfma32x32x16(kbh_u32x4 a, kbh_u32x4 b, kbh_f32x16 c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(kbh_bf16x8, a),
                                                   __builtin_bit_cast(kbh_bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(kbh_f16x8, a),
                                                  __builtin_bit_cast(kbh_f16x8, b), c, 0, 0, 0);
  }
}

// fp16 / bf16 bit patterns <-> fp32.
__device__ inline float f16_bits_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ inline float bf16_bits_to_f32(uint16_t h) { return __builtin_bit_cast(float, (uint32_t)h << 16); }
template <bool BF16>
__device__ inline float half_bits_to_f32(uint16_t h) {
  if constexpr (BF16) return bf16_bits_to_f32(h); else return f16_bits_to_f32(h);
}

// 16-bit element i (0..7) of a 16-byte vector.
__device__ inline uint16_t half_of(kbh_u32x4 v, int i) {
  return (uint16_t)((i & 1) ? (v[i >> 1] >> 16) : (v[i >> 1] & 0xffffu));
}

// Materialises v as an fp32 register value. Used where the reference rounds an intermediate to
// fp32 before a narrower conversion: without it the compiler may fuse a multiply with the
// conversion (v_fma_mix*), which rounds once and can differ from the reference in a tie.
__device__ inline float keep_f32(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

// fp32 -> fp16 / bf16 with round-to-nearest-even (NaN is kept quiet); both are hardware
// conversions on gfx950 (v_cvt_f16_f32, v_cvt_pk_bf16_f32; two neighbouring bf16 conversions
// become one packed instruction).
__device__ inline uint16_t f32_to_f16_bits(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ inline uint16_t f32_to_bf16_bits(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
// Two fp32 values to one dword of bf16 (lo in bits 0-15), one v_cvt_pk_bf16_f32.
__device__ inline uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{lo, hi}, b2));
}
template <bool BF16>
__device__ inline uint16_t f32_to_half_bits(float f) {
  if constexpr (BF16) return f32_to_bf16_bits(f); else return f32_to_f16_bits(f);
}

// Output policy: fp16/bf16 output of fp32 sums (emit: one element; emit4: four consecutive
// elements of a row, n % 4 == 0).
template <bool BF16>
struct HalfOut {
  static constexpr bool kPaired = false;
  uint16_t* y;
  int N;
  __device__ void emit(int r, int n, float v) const {
    y[(size_t)r * N + n] = f32_to_half_bits<BF16>(v);
  }
  __device__ void emit4(int r, int n, kbh_f32x4 v) const {
    kbh_u32x2 o;
    o[0] = (uint32_t)f32_to_half_bits<BF16>(v[0]) | ((uint32_t)f32_to_half_bits<BF16>(v[1]) << 16);
    o[1] = (uint32_t)f32_to_half_bits<BF16>(v[2]) | ((uint32_t)f32_to_half_bits<BF16>(v[3]) << 16);
    *reinterpret_cast<kbh_u32x2*>(y + (size_t)r * N + n) = o;
  }
};

// p[0] + p[stride] + ... + p[(n-1)*stride], added in slice order (n >= 1). The slices were just
// written by another kernel, so every load is a full memory round trip: the loads of up to 16
// slices are issued together before their adds.
template <int C, class V>
__device__ inline void sum_chunk(V& v, const V* p, size_t stride, int s) {
  V t[C];
#pragma unroll
  for (int j = 0; j < C; ++j) t[j] = __builtin_nontemporal_load(p + (size_t)(s + j) * stride);
#pragma unroll
  for (int j = 0; j < C; ++j) v += t[j];
}
template <class V>
__device__ inline V sum_slices(const V* p, size_t stride, int n) {
  V v = __builtin_nontemporal_load(p);
  int s = 1;
  for (; s + 16 <= n; s += 16) sum_chunk<16>(v, p, stride, s);
  if (s + 8 <= n) { sum_chunk<8>(v, p, stride, s); s += 8; }
  if (s + 4 <= n) { sum_chunk<4>(v, p, stride, s); s += 4; }
  if (s + 2 <= n) { sum_chunk<2>(v, p, stride, s); s += 2; }
  if (s < n) v += __builtin_nontemporal_load(p + (size_t)s * stride);
  return v;
}

}  // namespace kbh
