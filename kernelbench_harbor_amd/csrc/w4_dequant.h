// W4 (packed-asymmetric int4) dequantisation helpers shared by the dense and grouped GEMMs.
#pragma once

#include "kbh_common.h"
#include "tiled_f16.h"
#include "tiled_wide.h"

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
// the two 16-bit values (k, k+1). The arithmetic is the reference's: (q - z) rounded to the
// input dtype (exact for integer zero points), times s rounded to the input dtype.
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
        // q - z is exact in fp32 and rounds once to bf16; times s is exact in fp32 and rounds.
        const float s = bf16_bits_to_f32(sb);
        const float z = bf16_bits_to_f32(zb);
        const uint32_t d =
            f32x2_to_bf16x2_bits((bf16_bits_to_f32((uint16_t)(h & 0xffffu)) - 128.0f) - z,
                                 (bf16_bits_to_f32((uint16_t)(h >> 16)) - 128.0f) - z);
        out[col] = f32x2_to_bf16x2_bits(__builtin_bit_cast(float, d << 16) * s,
                                        __builtin_bit_cast(float, d & 0xffff0000u) * s);
      } else {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        const _Float16 sc = __builtin_bit_cast(_Float16, sb);
        const _Float16 zc = __builtin_bit_cast(_Float16, zb);
        const h2 magic = {(_Float16)1024.0f, (_Float16)1024.0f};
        const h2 q = __builtin_bit_cast(h2, h) - magic;  // exact
        out[col] = __builtin_bit_cast(uint32_t, (q - h2{zc, zc}) * h2{sc, sc});
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
    r.b[0] = q[0];
    r.b[1] = q[NP];
    const size_t off = (size_t)(k0 / group) * N + n0 + 8 * wc;
    r.s = *reinterpret_cast<const kbh_u32x4*>(scales + off);
    r.z = *reinterpret_cast<const kbh_u32x4*>(zeros + off);
  }
  __device__ void store(const Regs& r, uint16_t* Bs, int t) const {
    const int kp = t & 15, wc = t >> 4;
    uint32_t dq[8];
    dequant_2x8<BF16>(r.b[0], r.b[1], r.s, r.z, dq);
#pragma unroll
    for (int c = 0; c < 8; ++c) *reinterpret_cast<uint32_t*>(&Bs[tld_row(wc * 8 + c) * TLD + 2 * kp]) = dq[c];
  }
};

// Weight-slab producer for tiled_wide_gemm (32 rows x TN columns per slab, TN = 128 or 256).
// Thread t owns packed word column w (8 output columns) and kRows consecutive rows of the slab
// (word_of, rows_of); its LDS writes are bank-conflict free. The arithmetic is the reference's,
// exactly: (q - z) rounded to the input dtype, times s rounded to the input dtype.
template <bool BF16, int TN>
struct W4WidePolicy {
  static constexpr int kTN = TN;
  static constexpr int kRows = TN / 64;  // rows per thread: 4 (TN = 256) or 2 (TN = 128)
  static constexpr int kParts = 8;       // store_part(p) writes column p of the thread's word
  const uint32_t* qw;
  const uint16_t* scales;
  const uint16_t* zeros;
  int N, group;
  size_t q_stride, s_stride;  // elements between experts (grouped GEMMs); 0 for one matrix
  uint32_t mask;              // 0x000F000F, as a kernel argument so it lives in an SGPR
  __device__ W4WidePolicy at_expert(int e) const {
    W4WidePolicy p = *this;
    p.qw += (size_t)e * q_stride;
    p.scales += (size_t)e * s_stride;
    p.zeros += (size_t)e * s_stride;
    return p;
  }
  struct Raw {
    uint32_t w[kRows];
  };
  // s, z: the group's scales and zero points of the thread's 8 columns (two per dword); on the
  // one-step fp16 path (FAST below) prepare_group replaces z by 1024 + z.
  struct Grp {
    kbh_u32x4 s, z;
  };
  static constexpr bool kHasFast = !BF16;
  // TN = 256: t = [w bits 0-2][h bit 0][w bits 3-4][h bits 1-2], rows 4h..4h+3.
  // TN = 128: t = [h bits 0-1][w bits 0-2][w bit 3][h bits 2-3], rows 2h, 2h+1.
  // Either way the lanes of one LDS write pass cover distinct banks.
  __device__ static int word_of(int t) {
    if constexpr (TN == 256) return (t & 7) | (((t >> 4) & 3) << 3);
    else return ((t >> 2) & 7) | (((t >> 5) & 1) << 3);
  }
  __device__ static int rows_of(int t) {  // index h of the thread's row block
    if constexpr (TN == 256) return ((t >> 3) & 1) | ((t >> 6) << 1);
    else return (t & 3) | ((t >> 6) << 2);
  }

  __device__ void load(Raw& r, int k0, int n0, int t) const { load_from(r, qw, k0, n0, t); }
  // load / load_group from another matrix of the same shape (paired producers select the
  // matrix per lane by pointer)
  __device__ void load_from(Raw& r, const uint32_t* qw_, int k0, int n0, int t) const {
    const int w = word_of(t), h = rows_of(t);
    const int NP = N >> 3;
    const uint32_t* q = qw_ + (size_t)(k0 + kRows * h) * NP + (n0 >> 3) + w;
    // Plain (cached) loads: the row blocks of one K range run on one XCD and share these
    // words through its L2 (the non-temporal hint measured 2-7% slower at M=64..2048).
#pragma unroll
    for (int i = 0; i < kRows; ++i) r.w[i] = q[(size_t)i * NP];
  }
  __device__ void load_group(Grp& g, int k0, int n0, int t) const {
    load_group_from(g, scales, zeros, k0, n0, t);
  }
  __device__ void load_group_from(Grp& g, const uint16_t* scales_, const uint16_t* zeros_, int k0,
                                  int n0, int t) const {
    const size_t off = (size_t)(k0 / group) * N + n0 + 8 * word_of(t);
    g.s = *reinterpret_cast<const kbh_u32x4*>(scales_ + off);
    g.z = *reinterpret_cast<const kbh_u32x4*>(zeros_ + off);
  }
  // FAST (fp16 only): every zero point of the workgroup's K range and columns is an integer of
  // magnitude below 960, as the reference's uint4 zero points are. Then 1024 + z is exact, and
  // q - z is one exact subtraction from the magic number 1024 + q (low nibble), or an fma and an
  // add from 1024 + 16q (high nibble), instead of removing the magic number first: the same
  // values with fewer instructions. scan_cols reports whether this thread's share of the
  // zero points [k_begin, k_end) x [n0, n0 + cols) allows it; the kernel ANDs the workgroup.
  __device__ bool scan_cols(int k_begin, int k_end, int n0, int cols, int t) const {
    return scan_from(k_begin, k_end, n0, cols, t, 0);
  }
  __device__ bool scan_fast(int k_begin, int k_end, int n0, int t) const {
    return scan_cols(k_begin, k_end, n0, TN, t);
  }
  // The same test in two steps: scan_load issues this thread's first kScanPre chunk loads (the
  // warp-specialised kernel calls it before the weights' first slabs, so that the zero points
  // are the first data to come back instead of the last), scan_check tests them and any further
  // chunks.
  static constexpr int kScanPre = 4;
  struct ScanPre {
    kbh_u32x4 z[kScanPre];
  };
  __device__ void scan_load_cols(ScanPre& sp, int k_begin, int k_end, int n0, int cols, int t) const {
    const int g0 = k_begin / group, chunks = cols / 8;
    const int total = ((k_end - 1) / group - g0 + 1) * chunks;
#pragma unroll
    for (int j = 0; j < kScanPre; ++j) {
      const int i = t + 256 * j;
      sp.z[j] = i < total ? *reinterpret_cast<const kbh_u32x4*>(zeros + (size_t)(g0 + i / chunks) * N +
                                                               n0 + 8 * (i % chunks))
                          : kbh_u32x4{0u, 0u, 0u, 0u};  // zero points 0: allowed
    }
  }
  __device__ bool scan_check_cols(const ScanPre& sp, int k_begin, int k_end, int n0, int cols,
                                  int t) const {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < kScanPre; ++j) ok &= zeros_fast(sp.z[j]);
    return ok & scan_from(k_begin, k_end, n0, cols, t, kScanPre);
  }
  __device__ void scan_load(ScanPre& sp, int k_begin, int k_end, int n0, int t) const {
    scan_load_cols(sp, k_begin, k_end, n0, TN, t);
  }
  __device__ bool scan_check(const ScanPre& sp, int k_begin, int k_end, int n0, int t) const {
    return scan_check_cols(sp, k_begin, k_end, n0, TN, t);
  }
  // Whether the 8 fp16 zero points of one chunk allow FAST (always false for bf16).
  __device__ static bool zeros_fast(kbh_u32x4 zv) {
    if constexpr (BF16) {
      return false;
    } else {
      typedef _Float16 h8 __attribute__((ext_vector_type(8)));
      const h8 z = __builtin_bit_cast(h8, zv);
      // z + 1024 rounds to an integer below 2048: the round trip is exact iff z is an integer
      // in (-1024, 1024); |z| < 960 keeps (64 + q) - (1024 + z) + 960 in range too
      const h8 bm = (z + (_Float16)1024.0f) - (_Float16)1024.0f;
      bool ok = true;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        ok &= (bm[e] == z[e]) & ((float)z[e] < 960.0f) & ((float)z[e] > -960.0f);
      return ok;
    }
  }
  // Chunks t + 256 (first + j), j >= 0, of the zero points [k_begin, k_end) x [n0, n0 + cols).
  __device__ bool scan_from(int k_begin, int k_end, int n0, int cols, int t, int first) const {
    if constexpr (BF16) {
      return false;
    } else {
      const int g0 = k_begin / group, chunks = cols / 8;
      const int total = ((k_end - 1) / group - g0 + 1) * chunks;
      // Branch-free and unrolled, so that the loads of several chunks are in flight together
      // (with short-circuit tests each load waited for the previous chunk's verdict).
      bool ok = true;
#pragma unroll 4
      for (int i = t + 256 * first; i < total; i += 256)
        ok &= zeros_fast(*reinterpret_cast<const kbh_u32x4*>(zeros + (size_t)(g0 + i / chunks) * N +
                                                             n0 + 8 * (i % chunks)));
      return ok;
    }
  }
  // Derived constants of a loaded group, once before its first slab (the loads have landed).
  template <bool FAST>
  __device__ void prepare_group(Grp& g) const {
    if constexpr (FAST) {
      typedef _Float16 h8 __attribute__((ext_vector_type(8)));
      g.z = __builtin_bit_cast(kbh_u32x4, __builtin_bit_cast(h8, g.z) + (_Float16)1024.0f);
    }
  }

  // Rows (2i, 2i+1) of column C of the thread's word, dequantized: one dword (two values), from
  // P = pair_bytes<C / 2> of the two raw rows.
  template <int C>
  __device__ uint32_t value(uint32_t P, const Grp& g) const {
    const uint32_t m = (C & 1) ? ((P >> 4) & mask) : (P & mask);
    const uint32_t zw = g.z[C >> 1], sw = g.s[C >> 1];
    const uint16_t zb = (uint16_t)((C & 1) ? (zw >> 16) : (zw & 0xffffu));
    const uint16_t sb = (uint16_t)((C & 1) ? (sw >> 16) : (sw & 0xffffu));
    if constexpr (BF16) {
      // q - z is exact in fp32 and rounds once to bf16; times s is exact in fp32 and rounds once.
      const float z = bf16_bits_to_f32(zb), s = bf16_bits_to_f32(sb);
      const uint32_t d = f32x2_to_bf16x2_bits((float)(m & 0xffu) - z, (float)(m >> 16) - z);
      return f32x2_to_bf16x2_bits(__builtin_bit_cast(float, d << 16) * s,
                                  __builtin_bit_cast(float, d & 0xffff0000u) * s);
    } else {
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      const _Float16 z = __builtin_bit_cast(_Float16, zb), sc = __builtin_bit_cast(_Float16, sb);
      const h2 magic = {(_Float16)1024.0f, (_Float16)1024.0f};
      const h2 q = __builtin_bit_cast(h2, m | kMagicF16) - magic;  // exact
      return __builtin_bit_cast(uint32_t, (q - h2{z, z}) * h2{sc, sc});
    }
  }
  // The same value as value<C> under FAST (fp16): (q - z) exactly in one step, then * s.
  template <int C>
  __device__ uint32_t value_fast(uint32_t P, const Grp& g) const {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const uint32_t sw = g.s[C >> 1];
    const _Float16 sc = __builtin_bit_cast(_Float16, (uint16_t)((C & 1) ? (sw >> 16) : (sw & 0xffffu)));
    const uint32_t zw = g.z[C >> 1];  // 1024 + z (prepare_group<true>)
    const _Float16 zm = __builtin_bit_cast(_Float16, (uint16_t)((C & 1) ? (zw >> 16) : (zw & 0xffffu)));
    uint32_t magic = kMagicF16;
    asm("" : "+v"(magic));  // a VGPR: v_and_or_b32 takes the mask from an SGPR
    h2 d;
    if constexpr ((C & 1) == 0) {
      d = __builtin_bit_cast(h2, (P & mask) | magic) - h2{zm, zm};  // (1024 + q) - (1024 + z)
    } else {
      // (1024 + 16q) / 16 - (1024 + z) = q - z - 960 and + 960: integers below 2048, exact
      uint32_t mask_hi = 0x00F000F0u, sixteenth = 0x2C002C00u;  // fp16 {1/16, 1/16}
      asm("" : "+s"(mask_hi), "+s"(sixteenth));  // SGPR operands (one per VOP3)
      const h2 k960 = {(_Float16)960.0f, (_Float16)960.0f};
      d = __builtin_elementwise_fma(__builtin_bit_cast(h2, (P & mask_hi) | magic),
                                    __builtin_bit_cast(h2, sixteenth), -h2{zm, zm}) + k960;
    }
    return __builtin_bit_cast(uint32_t, d * h2{sc, sc});
  }
  template <int C>
  __device__ uint32_t pair(const Raw& r, const Grp& g, int i) const {
    return value<C>(pair_bytes<(C >> 1)>(r.w[2 * i], r.w[2 * i + 1]), g);
  }
  template <int C>
  __device__ uint32_t pair_fast(const Raw& r, const Grp& g, int i) const {
    return value_fast<C>(pair_bytes<(C >> 1)>(r.w[2 * i], r.w[2 * i + 1]), g);
  }
  template <bool FAST, int C>
  __device__ void put(const Raw& r, const Grp& g, uint8_t* base, int fw) const {
    uint8_t* p = base + ((C ^ fw) << 4);
    if constexpr (FAST && !BF16) {
      if constexpr (kRows == 4)
        *reinterpret_cast<kbh_u32x2*>(p) = kbh_u32x2{pair_fast<C>(r, g, 0), pair_fast<C>(r, g, 1)};
      else *reinterpret_cast<uint32_t*>(p) = pair_fast<C>(r, g, 0);
    } else if constexpr (kRows == 4) {
      *reinterpret_cast<kbh_u32x2*>(p) = kbh_u32x2{pair<C>(r, g, 0), pair<C>(r, g, 1)};
    } else {
      *reinterpret_cast<uint32_t*>(p) = pair<C>(r, g, 0);
    }
  }
  template <bool FAST>
  __device__ void store_part(const Raw& r, const Grp& g, uint8_t* Bs, int t, int p) const {
    const int w = word_of(t), h = rows_of(t);
    // Rows kRows*h.. are bytes 2*kRows*h.. of the column's K run:
    // wide_b_offset<TN>(2 kRows h, 8w + c) = base + 16 * (c ^ f(w)).
    uint8_t* base = Bs + wide_b_offset<TN>(2 * kRows * h, 8 * w) - wide_slot(8 * w) * 16 + w * 128;
    const int fw = (w ^ (w >> 3)) & 7;
    switch (p) {
      case 0: put<FAST, 0>(r, g, base, fw); break;
      case 1: put<FAST, 1>(r, g, base, fw); break;
      case 2: put<FAST, 2>(r, g, base, fw); break;
      case 3: put<FAST, 3>(r, g, base, fw); break;
      case 4: put<FAST, 4>(r, g, base, fw); break;
      case 5: put<FAST, 5>(r, g, base, fw); break;
      case 6: put<FAST, 6>(r, g, base, fw); break;
      default: put<FAST, 7>(r, g, base, fw); break;
    }
  }
  // Every part of the thread's slab share at once, the same LDS bytes as store_part(p) for
  // p < kParts, computed stage by stage across all columns and row pairs (8 perms, then 16
  // independent chains side by side) instead of one column's dependent chain after another, whose
  // latency (~9.5 cycles per dependent VALU instruction against ~5 with 4-8 chains in flight)
  // bounds a wave that only dequantizes.
  template <bool FAST>
  __device__ void store_all(const Raw& r, const Grp& g, uint8_t* Bs, int t) const {
    store_cols<FAST, 0, 8>(r, g, Bs, t);
  }
  // Two producer sets (TN = 256): set `half` of thread t loads and dequantizes rows
  // 4h + 2 half, +1 of the thread's 4 (one row pair) and writes their dword of each column.
  struct RawHalf {
    uint32_t w[2];
  };
  __device__ void load_half(RawHalf& r, int k0, int n0, int t, int half) const {
    static_assert(kRows == 4, "row pairs of 4-row threads");
    const int w = word_of(t), h = rows_of(t);
    const int NP = N >> 3;
    const uint32_t* q = qw + (size_t)(k0 + kRows * h + 2 * half) * NP + (n0 >> 3) + w;
    r.w[0] = q[0];
    r.w[1] = q[NP];
  }
  template <bool FAST>
  __device__ void store_half(const RawHalf& r, const Grp& g, uint8_t* Bs, int t, int half) const {
    const Raw full{{r.w[0], r.w[1], 0u, 0u}};
    store_cols<FAST, 0, 8, 1>(full, g, Bs + 4 * half, t);
  }
  // Columns C0..C0+NC-1 (C0, NC even) of the thread's word, as store_part(p) for those p, for
  // the first NIP row pairs of r (a single pair is stored as one dword per column at Bs + the
  // pair-0 offset).
  template <bool FAST, int C0, int NC, int NIP = kRows / 2>
  __device__ void store_cols(const Raw& r, const Grp& g, uint8_t* Bs, int t) const {
    static_assert(C0 % 2 == 0 && NC % 2 == 0 && C0 + NC <= 8, "whole byte pairs");
    static_assert(NIP >= 1 && NIP <= kRows / 2, "row pairs");
    constexpr int NI = NIP;  // row pairs
    const int w = word_of(t), h = rows_of(t);
    uint8_t* base = Bs + wide_b_offset<TN>(2 * kRows * h, 8 * w) - wide_slot(8 * w) * 16 + w * 128;
    const int fw = (w ^ (w >> 3)) & 7;
    uint32_t P[4][NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      if constexpr (C0 <= 0 && 0 < C0 + NC) P[0][i] = pair_bytes<0>(r.w[2 * i], r.w[2 * i + 1]);
      if constexpr (C0 <= 2 && 2 < C0 + NC) P[1][i] = pair_bytes<1>(r.w[2 * i], r.w[2 * i + 1]);
      if constexpr (C0 <= 4 && 4 < C0 + NC) P[2][i] = pair_bytes<2>(r.w[2 * i], r.w[2 * i + 1]);
      if constexpr (C0 <= 6 && 6 < C0 + NC) P[3][i] = pair_bytes<3>(r.w[2 * i], r.w[2 * i + 1]);
    }
    uint32_t v[8][NI];
    if constexpr (FAST && !BF16) {
      // The steps of value_fast, one stage at a time over all NC x NI values (scheduling
      // barriers keep the stages apart: left alone, the scheduler reuses one temporary register
      // per value and the chains run back to back).
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      uint32_t magic = kMagicF16, mask_hi = 0x00F000F0u, sixteenth = 0x2C002C00u;
      asm("" : "+v"(magic));
      asm("" : "+s"(mask_hi), "+s"(sixteenth));
      const h2 k960 = {(_Float16)960.0f, (_Float16)960.0f};
      h2 zm[8], sc[8];
#pragma unroll
      for (int c = C0; c < C0 + NC; ++c) {
        const uint32_t zw = g.z[c >> 1], sw = g.s[c >> 1];
        const _Float16 z1 = __builtin_bit_cast(_Float16, (uint16_t)((c & 1) ? (zw >> 16) : (zw & 0xffffu)));
        const _Float16 s1 = __builtin_bit_cast(_Float16, (uint16_t)((c & 1) ? (sw >> 16) : (sw & 0xffffu)));
        zm[c] = h2{z1, z1};
        sc[c] = h2{s1, s1};
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int c = C0; c < C0 + NC; ++c)
          v[c][i] = (c & 1) ? ((P[c >> 1][i] & mask_hi) | magic) : ((P[c >> 1][i] & mask) | magic);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int c = C0; c < C0 + NC; ++c) {
          const h2 m = __builtin_bit_cast(h2, v[c][i]);
          v[c][i] = __builtin_bit_cast(
              uint32_t, (c & 1) ? __builtin_elementwise_fma(m, __builtin_bit_cast(h2, sixteenth), -zm[c])
                                : m - zm[c]);
        }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int c = C0 + 1; c < C0 + NC; c += 2) v[c][i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v[c][i]) + k960);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int c = C0; c < C0 + NC; ++c) v[c][i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v[c][i]) * sc[c]);
      __builtin_amdgcn_sched_barrier(0);
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        if constexpr (C0 <= 0 && 0 < C0 + NC) { v[0][i] = value<0>(P[0][i], g); v[1][i] = value<1>(P[0][i], g); }
        if constexpr (C0 <= 2 && 2 < C0 + NC) { v[2][i] = value<2>(P[1][i], g); v[3][i] = value<3>(P[1][i], g); }
        if constexpr (C0 <= 4 && 4 < C0 + NC) { v[4][i] = value<4>(P[2][i], g); v[5][i] = value<5>(P[2][i], g); }
        if constexpr (C0 <= 6 && 6 < C0 + NC) { v[6][i] = value<6>(P[3][i], g); v[7][i] = value<7>(P[3][i], g); }
      }
    }
#pragma unroll
    for (int c = C0; c < C0 + NC; ++c) {
      uint8_t* p = base + ((c ^ fw) << 4);
      if constexpr (NI == 2) *reinterpret_cast<kbh_u32x2*>(p) = kbh_u32x2{v[c][0], v[c][1]};
      else *reinterpret_cast<uint32_t*>(p) = v[c][0];
    }
  }
};

}  // namespace kbh
