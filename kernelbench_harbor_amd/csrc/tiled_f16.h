// LDS-tiled fp16/bf16 MFMA GEMM with a pluggable weight-slab producer (larger-M kernels).
//
// y[M, N] = x[M, K] @ W[K, N], x and y in fp16 or bf16, W produced 32 rows at a time by a policy
// from its packed/quantized storage. One 256-thread workgroup computes a 256x128 tile:
//  * K advances in 32-row slabs. Each thread holds TDEPTH slabs of raw global data in registers
//    (a ring), so global loads are issued TDEPTH slabs ahead of their use; the steady-state loop
//    is branch-free (K is a multiple of 32*TDEPTH and loads past the end re-read the last slab),
//    which keeps the compiler's wait counts per slab instead of draining all loads.
//  * Two LDS buffers. Per slab: the MFMAs of slab kt run while the wave copies x and the
//    policy's dequantized weights of slab kt+1 into the other buffer; one barrier per slab.
//  * LDS rows are 40 elements (80 bytes): 16-byte fragment reads of 32 consecutive rows hit
//    distinct banks. The weight slab is stored k-major per output column ([128][40]), column n
//    at row tld_row(n).
//  * 2x2 waves, each 128x64 with 32x32x16 MFMAs (4x2 accumulator tiles).
//  * Workgroup ids are remapped so that each XCD receives consecutive tiles of the same rows of
//    x (its L2 then serves the shared x slabs).
//
// Policy interface (BP):
//   struct Regs;                                          per-thread raw data of one slab
//   void load(Regs&, int k0, int n0, int t) const;        issue global loads of slab [k0, k0+32)
//   void store(const Regs&, uint16_t* Bs, int t) const;   write Bs[tld_row(n) * TLD + k] for the slab
#pragma once

#include "kbh_common.h"

namespace kbh {

constexpr int TBM = 256, TBN = 128, TBK = 32;
constexpr int TLD = TBK + 8;  // LDS row stride in 16-bit elements
constexpr int TDEPTH = 4;     // K slabs in flight in registers ahead of the MFMAs

// LDS row of output column n in a [column][TLD] weight slab. The low three bits of n are permuted
// within each 8-column block, l -> l ^ (((n >> 2) & 6) | (l >> 2)) (a bijection of 0..7 for every
// block): the producers' 8-byte stores of columns 4c + j (c = 0..7, one j) then land in 8
// distinct 16-byte bank groups instead of 2 (an 80-byte row stride puts columns 8 apart on the
// same banks), while 8 consecutive columns, one fragment read, stay in distinct bank groups.
// Bits 3 and up are kept, so tld_row(n + 32 i) = tld_row(n) + 32 i.
__device__ inline int tld_row(int n) {
  const int l = n & 7;
  return (n & ~7) | (l ^ (((n >> 2) & 6) | (l >> 2)));
}

template <bool BF16, class BP>
__global__ __launch_bounds__(256) void tiled_f16_gemm(const uint16_t* __restrict__ x, BP bp,
                                                      uint16_t* __restrict__ y, int M, int N,
                                                      int K) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][TBM * TLD];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][TBN * TLD];

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int ntn = N / TBN;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int mb = id / ntn, nb = id - mb * ntn;
  const int m0 = mb * TBM, n0 = nb * TBN;
  const int KT = K / TBK;

  // x: rows t/4 + 64i (i < 4), 16-byte chunk t%4 of the slab.
  const int a_ch = t & 3, a_row = t >> 2;
  const uint16_t* xrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = m0 + a_row + 64 * i;
    xrow[i] = x + (size_t)(r < M ? r : M - 1) * K + a_ch * 8;  // rows >= M are never stored
  }
  struct Slab {
    kbh_u32x4 a[4];
    typename BP::Regs b;
  };
  auto load = [&](Slab& sl, int kt) {
    const int k0 = kt * TBK;
#pragma unroll
    for (int i = 0; i < 4; ++i) sl.a[i] = *reinterpret_cast<const kbh_u32x4*>(xrow[i] + k0);
    bp.load(sl.b, k0, n0, t);
  };
  auto store_a = [&](const Slab& sl, int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<kbh_u32x4*>(&As[buf][(a_row + 64 * i) * TLD + a_ch * 8]) = sl.a[i];
  };

  kbh_f32x16 accv[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) accv[i][j][e] = 0.f;

  const int fr = lane & 31, fk = (lane >> 5) * 8;
  // One 16-deep K step of the wave's 128x64 tile: 6 LDS fragment reads, 8 MFMAs.
  auto mma_k16 = [&](int buf, int kk) {
    const uint16_t* Ab = &As[buf][(wm * 128 + fr) * TLD + fk + kk * 16];
    const uint16_t* Bb = &Bs[buf][tld_row(wn * 64 + fr) * TLD + fk + kk * 16];
    kbh_u32x4 a[4], b[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const kbh_u32x4*>(Ab + i * 32 * TLD);
#pragma unroll
    for (int j = 0; j < 2; ++j) b[j] = *reinterpret_cast<const kbh_u32x4*>(Bb + j * 32 * TLD);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) accv[i][j] = mfma32x32x16<BF16>(a[i], b[j], accv[i][j]);
  };

  Slab ring[TDEPTH];
#pragma unroll
  for (int d = 0; d < TDEPTH; ++d) load(ring[d], min(d, KT - 1));
  store_a(ring[0], 0);
  bp.store(ring[0].b, Bs[0], t);
  load(ring[0], min(TDEPTH, KT - 1));
  __syncthreads();

  for (int kt0 = 0; kt0 < KT; kt0 += TDEPTH) {
#pragma unroll
    for (int d = 0; d < TDEPTH; ++d) {
      const int kt = kt0 + d;
      const int nxt = (d + 1) % TDEPTH;  // ring stage of slab kt+1
      // After the last slab the other buffer is written but never read.
      // Scheduling fences keep each slab's phases in this order: unfenced, the scheduler
      // hoists the stores (and the weight producer's VALU) of all TDEPTH unrolled slabs to the
      // top of the loop, which waits for the most recent loads and drains the prefetch ring.
      mma_k16(kt & 1, 0);
      __builtin_amdgcn_sched_barrier(0);
      store_a(ring[nxt], (kt + 1) & 1);
      __builtin_amdgcn_sched_barrier(0);
      mma_k16(kt & 1, 1);
      __builtin_amdgcn_sched_barrier(0);
      bp.store(ring[nxt].b, Bs[(kt + 1) & 1], t);
      __builtin_amdgcn_sched_barrier(0);
      load(ring[nxt], min(kt + 1 + TDEPTH, KT - 1));
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Accumulator element e of tile (i, j): row 8(e/4) + 4(l/32) + e%4, column l%32.
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = m0 + wm * 128 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int n = n0 + wn * 64 + j * 32 + (lane & 31);
        if (r < M) y[(size_t)r * N + n] = f32_to_half_bits<BF16>(accv[i][j][e]);
      }
}

// Grid of the tiled kernel: one workgroup per 256x128 tile.
inline dim3 tiled_f16_grid(int M, int N) { return dim3(((M + TBM - 1) / TBM) * (N / TBN)); }

}  // namespace kbh
