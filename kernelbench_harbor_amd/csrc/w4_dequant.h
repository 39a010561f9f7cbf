// W4 (packed-asymmetric int4) dequantisation helpers shared by the dense and grouped GEMMs.
#pragma once

#include "kbh_common.h"
#include "tiled_f16.h"

namespace kbh {

constexpr uint32_t kMagicF16 = 0x64006400u;   // fp16 1024.0 in both halves
constexpr uint32_t kMagicBF16 = 0x43004300u;  // bf16 128.0 in both halves
constexpr uint32_t kOneF16 = 0x3c003c00u;
constexpr uint32_t kOneBF16 = 0x3f803f80u;

// Byte J of word wa (row k) to bits 0..7 and byte J of word wb (row k+1) to bits 16..23; the
// other bytes are zero. v_perm_b32 numbers the bytes of {src0, src1} as src1 = 0..3, src0 = 4..7
// and selector value 0x0c yields 0x00.
template <int J>
__device__ inline uint32_t pair_bytes(uint32_t wa, uint32_t wb) {
  constexpr uint32_t sel = 0x0c000c00u | ((4u + J) << 16) | (uint32_t)J;
  return __builtin_amdgcn_perm(wb, wa, sel);
}
__device__ inline uint32_t pair_bytes_rt(uint32_t wa, uint32_t wb, int j) {
  switch (j) {
    case 0: return pair_bytes<0>(wa, wb);
    case 1: return pair_bytes<1>(wa, wb);
    case 2: return pair_bytes<2>(wa, wb);
    default: return pair_bytes<3>(wa, wb);
  }
}

// Dequantizes one thread's 2 rows (k, k+1) x 8 columns: result column c is the dword holding
// the two 16-bit values (k, k+1). The arithmetic is the reference's: (q - z) in the input dtype
// (exact: small integers), times s with one rounding.
template <bool BF16>
__device__ inline void dequant_2x8(uint32_t w0, uint32_t w1, kbh_u32x4 sv, kbh_u32x4 zv,
                                   uint32_t out[8]) {
  constexpr uint32_t MAGIC = BF16 ? kMagicBF16 : kMagicF16;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t P = pair_bytes_rt(w0, w1, j);
    const uint32_t hl = (P & 0x000F000Fu) | MAGIC;          // column 2j   at rows (k, k+1)
    const uint32_t hh = ((P >> 4) & 0x000F000Fu) | MAGIC;   // column 2j+1 at rows (k, k+1)
#pragma unroll
    for (int hsel = 0; hsel < 2; ++hsel) {
      const int col = 2 * j + hsel;
      const uint32_t h = hsel ? hh : hl;
      const uint16_t sb = (uint16_t)((col & 1) ? (sv[col >> 1] >> 16) : (sv[col >> 1] & 0xffffu));
      const uint16_t zb = (uint16_t)((col & 1) ? (zv[col >> 1] >> 16) : (zv[col >> 1] & 0xffffu));
      if constexpr (BF16) {
        // (128+q) - (128+z) is exact in fp32, times s is exact in fp32; one rounding to bf16.
        const float s = bf16_bits_to_f32(sb);
        const float bz = 128.0f + bf16_bits_to_f32(zb);
        const float lo = (bf16_bits_to_f32((uint16_t)(h & 0xffffu)) - bz) * s;
        const float hi = (bf16_bits_to_f32((uint16_t)(h >> 16)) - bz) * s;
        out[col] = (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
      } else {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        const _Float16 sc = __builtin_bit_cast(_Float16, sb);
        const _Float16 bz = (_Float16)1024.0f + __builtin_bit_cast(_Float16, zb);
        const h2 d = __builtin_bit_cast(h2, h) - h2{bz, bz};  // q - z, exact
        out[col] = __builtin_bit_cast(uint32_t, d * h2{sc, sc});
      }
    }
  }
}

// Weight-slab producer for tiled_f16_gemm: thread t dequantizes rows 2*(t%16), +1 of the slab
// for the 8 columns of packed word column t/16 and stores them k-major per column.
template <bool BF16>
struct W4SlabPolicy {
  const uint32_t* qw;
  const uint16_t* scales;
  const uint16_t* zeros;
  int N, group;
  size_t q_stride, s_stride;  // elements between experts (grouped GEMMs); 0 for one matrix
  __device__ W4SlabPolicy at_expert(int e) const {
    W4SlabPolicy p = *this;
    p.qw += (size_t)e * q_stride;
    p.scales += (size_t)e * s_stride;
    p.zeros += (size_t)e * s_stride;
    return p;
  }
  struct Regs {
    uint32_t b[2];
    kbh_u32x4 s, z;
  };
  __device__ void load(Regs& r, int k0, int n0, int t) const {
    const int kp = t & 15, wc = t >> 4;
    const int NP = N >> 3;
    const uint32_t* q = qw + (size_t)(k0 + 2 * kp) * NP + (n0 >> 3) + wc;
    r.b[0] = __builtin_nontemporal_load(q);
    r.b[1] = __builtin_nontemporal_load(q + NP);
    const size_t off = (size_t)(k0 / group) * N + n0 + 8 * wc;
    r.s = *reinterpret_cast<const kbh_u32x4*>(scales + off);
    r.z = *reinterpret_cast<const kbh_u32x4*>(zeros + off);
  }
  __device__ void store(const Regs& r, uint16_t* Bs, int t) const {
    const int kp = t & 15, wc = t >> 4;
    uint32_t dq[8];
    dequant_2x8<BF16>(r.b[0], r.b[1], r.s, r.z, dq);
#pragma unroll
    for (int c = 0; c < 8; ++c) *reinterpret_cast<uint32_t*>(&Bs[(wc * 8 + c) * TLD + 2 * kp]) = dq[c];
  }
};

}  // namespace kbh
