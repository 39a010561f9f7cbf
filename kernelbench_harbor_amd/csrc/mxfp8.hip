// MXFP8 block-scaled GEMM on gfx950 scaled MFMA (the benchmark's MXFP8 configuration; no reference module:
// the nearest reference math is generate_tasks.py:337-342 (absmax / 448, cast to e4m3fn) and
// tasks/fp8_microscale/*/environment/reference.py:11 (fp8 decode times scale)).
//
//   a [M, K] e4m3fn codes, a_scale [M, K/32] e8m0      (1x32 blocks along K)
//   b [N, K] e4m3fn codes, b_scale [N, K/32] e8m0
//   y[m, n] = sum_blocks 2^(ea-127) 2^(eb-127) sum_{k in block} a[m,k] b[n,k]   (fp32 accumulate)
//
// v_mfma_scale_f32_32x32x64_f8f6f4 operand layout (measured on gfx950): lane l = 32g + r holds
// row r of the operand, bytes 0-15 = k [16g, 16g+16) and bytes 16-31 = k [32+16g, 32+16g+16) of
// the 64-deep step; its scale operand is the e8m0 of row r, 32-block g of the step. The decode of
// the e8m0 exponents happens inside the MFMA.
//
// Kernel: 256 threads (2x2 waves), tile 128 x (64*WNT), K in 128-deep slabs (4 scale blocks)
// held in a two-slab register ring, two LDS buffers with 144-byte rows (conflict-free 16-byte
// fragment reads). Each wave computes 64 x (32*WNT) with 2 x WNT MFMA tiles; per slab the LDS
// stores of the next slab, the fragment reads of the next K step and the global loads are
// interleaved with the MFMAs (one barrier per slab). From 1024 rows mxfp8_dma_kernel takes
// 256 x 256 tiles instead (below). When the tiles fill fewer than 256 workgroups the K range is
// split over gridDim.z; each split stores its partial tile into its own fp32 workspace slice and
// splitk_sum_half (splitk.h) adds the slices in split order and converts.
#include "kbh_common.h"
#include "splitk.h"

#include <type_traits>

namespace kbh {
namespace {

constexpr int XBM = 128, XBK = 128;  // rows per tile, k (bytes) per slab
constexpr int XLD = XBK + 16;        // LDS row stride in bytes
constexpr int XDEPTH = 2;

__device__ inline kbh_f32x16 mfma_mx32(kbh_u32x4 a0, kbh_u32x4 a1, kbh_u32x4 b0, kbh_u32x4 b1,
                                       kbh_f32x16 c, int sa, int sb) {
  const kbh_i32x8 a = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3],
                       (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
  const kbh_i32x8 b = {(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3],
                       (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
  // format codes 0 = fp8 e4m3 for both operands; opsel 0 = low byte of the scale registers
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, sa, 0, sb);
}

template <int WNT, bool BF16>
__global__ __launch_bounds__(256) void mxfp8_kernel(
    const uint8_t* __restrict__ a, const uint8_t* __restrict__ as, const uint8_t* __restrict__ b,
    const uint8_t* __restrict__ bs, uint16_t* __restrict__ y, float* __restrict__ acc, int M,
    int N, int K, int slabs_per_split) {
  constexpr int XBN = 64 * WNT;
  __shared__ __attribute__((aligned(16))) uint8_t Al[2][XBM * XLD];
  __shared__ __attribute__((aligned(16))) uint8_t Bl[2][XBN * XLD];
  // e8m0 scale dwords of the slab (4 blocks of 32 along K per row): A rows, then B rows (and
  // 128 unused dwords that waves 2-3 write so the store needs no branch).
  __shared__ uint32_t Sl[2][XBM + XBN + XBM];

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int ntn = N / XBN;
  // Tile order: groups of up to 8 row blocks, rows fastest within a group, so the 32 tiles an
  // XCD runs (consecutive ids after xcd_remap) form an 8 x 4 block that shares A rows and B
  // columns in its L2 (row-major order would give each XCD 2 x 16 tiles and make every XCD
  // stream all of B).
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int nmb = gridDim.x / ntn;
  const int gm0 = nmb < 8 ? nmb : 8;
  const int grp = id / (gm0 * ntn), first_m = grp * gm0;
  const int gm = nmb - first_m < gm0 ? nmb - first_m : gm0;
  const int r_in = id - grp * gm0 * ntn;
  const int mb = first_m + r_in % gm, nb = r_in / gm;
  const int m0 = mb * XBM, n0 = nb * XBN;
  const int splits = gridDim.z, split = blockIdx.z;
  const int KS = K / 32;  // scale columns
  const int kt_begin = split * slabs_per_split;
  const int KT = slabs_per_split;

  // global -> register mapping: 16-byte chunk t%8 of rows t/8 + 32i. Buffer loads: one VGPR
  // offset per matrix plus the uniform row/k offset in an SGPR; A rows past M (offsets past
  // the end of a) read as zero and are never stored.
  const int ch = t & 7, rr = t >> 3;
  const int fr = lane & 31, fg = lane >> 5;
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(a, (size_t)M * K);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(b, (size_t)N * K);
  // Scale rows of the slab: waves 0-1 (t < 128) load A row t and B row 128 + t (read only for
  // 256-row B tiles), waves 2-3 load B row t - 128 (and an unused dword). The choice of matrix
  // is uniform per wave, so it selects the buffer resource and the loop body has no branch.
  const bool sa_wave = __builtin_amdgcn_readfirstlane(t) < XBM;
  const __amdgpu_buffer_rsrc_t rs0 =
      make_rsrc(sa_wave ? (const void*)as : (const void*)bs, (size_t)(sa_wave ? M : N) * KS);
  const __amdgpu_buffer_rsrc_t rsb = make_rsrc(bs, (size_t)N * KS);  // rows past N read as 0
  const uint32_t va = (uint32_t)((m0 + rr) * K + ch * 16);
  const uint32_t vb = (uint32_t)((n0 + rr) * K + ch * 16);
  const uint32_t vs0 = sa_wave ? (uint32_t)((m0 + t) * KS) : (uint32_t)((n0 + t - XBM) * KS);
  const uint32_t vs1 = (uint32_t)((n0 + XBM + t) * KS);

  struct Slab {
    kbh_u32x4 a[4];
    kbh_u32x4 b[2 * WNT];
    uint32_t s[2];
  };
  struct Scales {
    uint32_t sa[2];
    uint32_t sb[WNT];
  };
  struct Frags {
    kbh_u32x4 a0[2], a1[2], b0[WNT], b1[WNT];
  };
  auto load = [&](Slab& sl, int kt) {
    const int k0 = (kt_begin + kt) * XBK;
    // the scale dwords first: the oldest loads of the group, so waiting for them does not wait
    // for the A/B data issued after them
    sl.s[0] = __builtin_amdgcn_raw_buffer_load_b32(rs0, vs0, k0 / 32, 0);
    if constexpr (XBN > XBM) sl.s[1] = __builtin_amdgcn_raw_buffer_load_b32(rsb, vs1, k0 / 32, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      sl.a[i] = __builtin_bit_cast(kbh_u32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, va, 32 * i * K + k0, 0));
#pragma unroll
    for (int i = 0; i < 2 * WNT; ++i)
      sl.b[i] = __builtin_bit_cast(kbh_u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, vb, 32 * i * K + k0, kBufNT));
  };
  // LDS stores of a slab in 4 parts (A chunks, then B chunks), interleaved with MFMAs.
  constexpr int NCH = 4 + 2 * WNT;  // 16-byte chunks per thread
  auto store_part = [&](const Slab& sl, int buf, int p) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (c * 4 / NCH != p) continue;
      if (c < 4)
        *reinterpret_cast<kbh_u32x4*>(&Al[buf][(rr + 32 * c) * XLD + ch * 16]) = sl.a[c];
      else
        *reinterpret_cast<kbh_u32x4*>(&Bl[buf][(rr + 32 * (c - 4)) * XLD + ch * 16]) = sl.b[c - 4];
    }
    if (p == 3) {
      Sl[buf][t] = sl.s[0];  // A row t, or B row t - 128 at index 128 + (t - 128)
      if constexpr (XBN > XBM) Sl[buf][2 * XBM + t] = sl.s[1];  // B row 128 + t (t < 128)
    }
  };
  // This wave's scale dwords of the slab in LDS buffer buf.
  auto read_scales = [&](Scales& sc, int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) sc.sa[i] = Sl[buf][wm * 64 + i * 32 + fr];
#pragma unroll
    for (int j = 0; j < WNT; ++j) sc.sb[j] = Sl[buf][XBM + wn * 32 * WNT + j * 32 + fr];
  };

  kbh_f32x16 accv[2][WNT];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < WNT; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) accv[i][j][e] = 0.f;

  // Fragments of one 64-deep K step (kk = 0, 1 within the slab) from LDS buffer buf.
  auto read_frags = [&](Frags& f, int buf, int kk) {
    const uint8_t* Ab = &Al[buf][(wm * 64 + fr) * XLD + kk * 64 + 16 * fg];
    const uint8_t* Bb = &Bl[buf][(wn * 32 * WNT + fr) * XLD + kk * 64 + 16 * fg];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      f.a0[i] = *reinterpret_cast<const kbh_u32x4*>(Ab + i * 32 * XLD);
      f.a1[i] = *reinterpret_cast<const kbh_u32x4*>(Ab + i * 32 * XLD + 32);
    }
#pragma unroll
    for (int j = 0; j < WNT; ++j) {
      f.b0[j] = *reinterpret_cast<const kbh_u32x4*>(Bb + j * 32 * XLD);
      f.b1[j] = *reinterpret_cast<const kbh_u32x4*>(Bb + j * 32 * XLD + 32);
    }
  };
  // MFMAs q in [lo, hi) of step kk (q = i * WNT + j); scale byte 2*kk + g of the slab's dword.
  auto mma_range = [&](const Frags& f, int kk, const Scales& sc, int lo, int hi) {
    const int sh = 8 * (2 * kk + fg);
#pragma unroll
    for (int q = 0; q < 2 * WNT; ++q) {
      if (q < lo || q >= hi) continue;
      const int i = q / WNT, j = q % WNT;
      const int sa = (int)((sc.sa[i] >> sh) & 0xffu);
      const int sb = (int)((sc.sb[j] >> sh) & 0xffu);
      accv[i][j] = mfma_mx32(f.a0[i], f.a1[i], f.b0[j], f.b1[j], accv[i][j], sa, sb);
    }
  };

  // Ring of XDEPTH slabs in registers (slab s is loaded two iterations before it is stored to
  // LDS); LDS buffer s & 1 holds slab s. Per slab: step-1 fragments are read, the step-0 MFMAs
  // run interleaved with the LDS stores of slab s+1, one barrier, then the step-0 fragments of
  // slab s+1 are read while the step-1 MFMAs run interleaved with the global loads of slab s+3.
  Slab ring[XDEPTH];
  Frags f0, f1;
#pragma unroll
  for (int d = 0; d < XDEPTH; ++d) load(ring[d], min(d, KT - 1));
#pragma unroll
  for (int p = 0; p < 4; ++p) store_part(ring[0], 0, p);
  load(ring[0], min(XDEPTH, KT - 1));
  __syncthreads();
  Scales scur;
  read_scales(scur, 0);
  read_frags(f0, 0, 0);
  constexpr int NMF = 2 * WNT;  // MFMAs per step
  for (int kt0 = 0; kt0 < KT; kt0 += XDEPTH) {
#pragma unroll
    for (int d = 0; d < XDEPTH; ++d) {
      // KT is a multiple of XDEPTH: no branch here (see tiled_f16.h on wait counts).
      const int kt = kt0 + d;
      const int cur = kt & 1;
      const int nxt = (d + 1) % XDEPTH;
      read_frags(f1, cur, 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        mma_range(f0, 0, scur, p * NMF / 4, (p + 1) * NMF / 4);
        __builtin_amdgcn_sched_barrier(0);
        store_part(ring[nxt], 1 - cur, p);  // slab kt+1 (after the last: unused buffer)
        __builtin_amdgcn_sched_barrier(0);
      }
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
      Scales snext;
      read_scales(snext, 1 - cur);  // slab kt+1
      read_frags(f0, 1 - cur, 0);   // step 0 of slab kt+1
      mma_range(f1, 1, scur, 0, NMF);
      load(ring[nxt], min(kt + 1 + XDEPTH, KT - 1));
#pragma unroll
      for (int q = 0; q < NMF; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x020, 2, 1);  // two VMEM reads
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);  // two LDS reads
      }
      __builtin_amdgcn_sched_barrier(0);
      scur = snext;
    }
  }

  // Accumulator element e of tile (i, j): row 8(e/4) + 4(l/32) + e%4, column l%32.
  auto for_each = [&](auto&& f) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < WNT; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * fg + (e & 3);
          const int n = n0 + wn * 32 * WNT + j * 32 + fr;
          if (r < M) f(i, j, e, (size_t)r * N + n);
        }
  };
  if (splits == 1) {
    for_each([&](int i, int j, int e, size_t o) { y[o] = f32_to_half_bits<BF16>(accv[i][j][e]); });
    return;
  }
  float* slice = acc + (size_t)split * M * N;
  for_each([&](int i, int j, int e, size_t o) { slice[o] = accv[i][j][e]; });
}


// ---------------------------------------------------------------------------------------------
// 256 x 256 tiles for large M (mxfp8_dma_kernel). The operands go from global memory straight
// into LDS with the buffer loads' LDS mode (lane i of a 16-byte load lands at M0 + 16 i, of a
// 4-byte load at M0 + 4 i; measured on gfx950), so no register ring stages them and each of the
// 4 waves holds a 128 x 128 accumulator (4 x 4 MFMA tiles). Per 128-deep slab a workgroup loads
// 64 KB for 2x the MFMA work of the 128 x 256 tile's 48 KB.
//
// LDS per buffer: A and B slabs of 256 rows x 128 bytes without padding, 16-byte chunk c of row
// r at r * 128 + 16 (c ^ ((r >> 1) & 7)) (the 16 rows one fragment read covers hit 16 different
// 16-byte bank groups), then the 256 + 256 scale dwords. A load instruction fills one 1 KB
// block (8 rows): lane i takes row 8 blk + i / 8 and the chunk that the swizzle puts at
// position i % 8. Two buffers; slab s + 2 is loaded into buffer s & 1 during the second half of
// slab s, after the barrier that ends every wave's reads of slab s.
constexpr int DBM = 256;          // tile rows = tile columns
constexpr int DSLAB = DBM * XBK;  // bytes of one operand slab

template <bool BF16>
__global__ __launch_bounds__(256) void mxfp8_dma_kernel(
    const uint8_t* __restrict__ a, const uint8_t* __restrict__ as, const uint8_t* __restrict__ b,
    const uint8_t* __restrict__ bs, uint16_t* __restrict__ y, float* __restrict__ acc, int M,
    int N, int K, int slabs_per_split) {
  // One object per buffer and operand, so that the compiler can tell the LDS writes of the
  // loads in flight from the fragment reads of the other buffer.
  __shared__ __attribute__((aligned(16))) uint8_t La0[DSLAB], La1[DSLAB], Lb0[DSLAB], Lb1[DSLAB];
  __shared__ __attribute__((aligned(16))) uint32_t Ls0[2 * DBM], Ls1[2 * DBM];

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wu = __builtin_amdgcn_readfirstlane(wave);
  const int wm = wave >> 1, wn = wave & 1;
  const int ntn = N / DBM;
  // Tile order as in mxfp8_kernel: groups of up to 8 row blocks, rows fastest in a group.
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int nmb = gridDim.x / ntn;
  const int gm0 = nmb < 8 ? nmb : 8;
  const int grp = id / (gm0 * ntn), first_m = grp * gm0;
  const int gm = nmb - first_m < gm0 ? nmb - first_m : gm0;
  const int r_in = id - grp * gm0 * ntn;
  const int mb = first_m + r_in % gm, nb = r_in / gm;
  const int m0 = mb * DBM, n0 = nb * DBM;
  const int splits = gridDim.z, split = blockIdx.z;
  const int KS = K / 32;
  const int kt_begin = split * slabs_per_split;
  const int KT = slabs_per_split;

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(a, (size_t)M * K);  // rows past M read as zero
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(b, (size_t)N * K);
  const __amdgpu_buffer_rsrc_t rsa = make_rsrc(as, (size_t)M * KS);
  const __amdgpu_buffer_rsrc_t rsb = make_rsrc(bs, (size_t)N * KS);
  // Load-side lane offsets: row 8 blk + lane / 8 of the tile, chunk (lane % 8) ^ ((row >> 1) & 7);
  // (row >> 1) & 7 = 4 (blk & 1) + lane / 16, so even and odd blocks need one offset each and
  // the block's 8 blk * K goes into the uniform soffset.
  const int lr = lane >> 3;
  const uint32_t ce = (uint32_t)(16 * ((lane & 7) ^ (lane >> 4)));
  const uint32_t co = (uint32_t)(16 * ((lane & 7) ^ (4 + (lane >> 4))));
  const uint32_t va_e = (uint32_t)((m0 + lr) * K) + ce, va_o = (uint32_t)((m0 + lr) * K) + co;
  const uint32_t vb_e = (uint32_t)((n0 + lr) * K) + ce, vb_o = (uint32_t)((n0 + lr) * K) + co;
  const uint32_t vsa = (uint32_t)((m0 + 64 * wave + lane) * KS);
  const uint32_t vsb = (uint32_t)((n0 + 64 * wave + lane) * KS);

  typedef __attribute__((address_space(3))) void* lds_t;
  // Wave w loads A and B blocks 8w .. 8w + 7 and the scale dwords of rows 64w .. 64w + 63.
  auto issue = [&](uint8_t* LA, uint8_t* LB, uint32_t* LS, int kt) {
    const int k0 = (kt_begin + kt) * XBK;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_t)(LS + 64 * wu), 4, vsa, k0 / 32, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, (lds_t)(LS + DBM + 64 * wu), 4, vsb, k0 / 32, 0, 0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int blk = 8 * wu + j;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_t)(LA + 1024 * blk), 16, (j & 1) ? va_o : va_e,
                                               8 * blk * K + k0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_t)(LB + 1024 * blk), 16, (j & 1) ? vb_o : vb_e,
                                               8 * blk * K + k0, 0, kBufNT);
    }
  };

  // Read-side lane offsets: fragment row r = base + fr (base a multiple of 32), so the swizzle
  // term is (fr >> 1) & 7; chunk 4 kk + fg (+ 2 for the second 16 bytes).
  const int fr = lane & 31, fg = lane >> 5;
  const int sw = (fr >> 1) & 7;
  int oa[2][2], ob[2][2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = 16 * ((4 * kk + fg + 2 * h) ^ sw);
      oa[kk][h] = (wm * 128 + fr) * XBK + c;
      ob[kk][h] = (wn * 128 + fr) * XBK + c;
    }
  struct Frags {
    kbh_u32x4 a0[4], a1[4], b0[4], b1[4];
  };
  struct Scales {
    uint32_t sa[4], sb[4];
  };
  auto read_frags = [&](Frags& f, const uint8_t* LA, const uint8_t* LB, int kk) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f.a0[i] = *reinterpret_cast<const kbh_u32x4*>(LA + oa[kk][0] + i * 32 * XBK);
      f.a1[i] = *reinterpret_cast<const kbh_u32x4*>(LA + oa[kk][1] + i * 32 * XBK);
      f.b0[i] = *reinterpret_cast<const kbh_u32x4*>(LB + ob[kk][0] + i * 32 * XBK);
      f.b1[i] = *reinterpret_cast<const kbh_u32x4*>(LB + ob[kk][1] + i * 32 * XBK);
    }
  };
  auto read_scales = [&](Scales& sc, const uint32_t* LS) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc.sa[i] = LS[wm * 128 + i * 32 + fr];
      sc.sb[i] = LS[DBM + wn * 128 + i * 32 + fr];
    }
  };
  kbh_f32x16 accv[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) accv[i][j][e] = 0.f;
  auto mma = [&](const Frags& f, int kk, const Scales& sc) {
    const int sh = 8 * (2 * kk + fg);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        accv[i][j] = mfma_mx32(f.a0[i], f.a1[i], f.b0[j], f.b1[j], accv[i][j],
                               (int)((sc.sa[i] >> sh) & 0xffu), (int)((sc.sb[j] >> sh) & 0xffu));
  };

  // vmcnt(0) with the other counters left alone (gfx9 s_waitcnt encoding).
  constexpr int kWaitVm0 = 0x0F70;
  Frags f0, f1;
  Scales scur, snext;
  issue(La0, Lb0, Ls0, 0);
  issue(La1, Lb1, Ls1, min(1, KT - 1));
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  __syncthreads();
  read_scales(scur, Ls0);
  read_frags(f0, La0, Lb0, 0);
  // Slab kt in buffer P = kt & 1 (Q = the other): read its step-1 fragments, run its step-0
  // MFMAs, wait for this wave's loads of slab kt + 1 (buffer Q), barrier (every wave is done
  // with buffer P and slab kt + 1 is complete), read slab kt + 1's scales and step-0 fragments,
  // start slab kt + 2's loads into buffer P, run step 1.
  auto slab = [&](auto par, int kt) {
    constexpr int P = decltype(par)::value;
    uint8_t* const LAp = P ? La1 : La0;
    uint8_t* const LBp = P ? Lb1 : Lb0;
    uint32_t* const LSp = P ? Ls1 : Ls0;
    const uint8_t* const LAq = P ? La0 : La1;
    const uint8_t* const LBq = P ? Lb0 : Lb1;
    const uint32_t* const LSq = P ? Ls0 : Ls1;
    read_frags(f1, LAp, LBp, 1);
    mma(f0, 0, scur);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    read_scales(snext, LSq);
    read_frags(f0, LAq, LBq, 0);
    issue(LAp, LBp, LSp, min(kt + 2, KT - 1));
    mma(f1, 1, scur);
    // The slab's fragment and scale reads first, then the 18 loads of slab kt + 2 one per MFMA
    // (three with the first) rather than in one burst after the barrier: 2-3% faster at
    // M=1024-4096.
    __builtin_amdgcn_sched_group_barrier(0x100, 24, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x020, 3, 0);
#pragma unroll
    for (int q = 1; q < 16; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    scur = snext;
  };
  for (int kt0 = 0; kt0 < KT; kt0 += 2) {
    slab(std::integral_constant<int, 0>{}, kt0);
    slab(std::integral_constant<int, 1>{}, kt0 + 1);
  }

  // Accumulator element e of tile (i, j): row 8(e/4) + 4(l/32) + e%4, column l%32.
  const bool full = m0 + DBM <= M;  // no row of the tile lies past M
  auto for_each = [&](auto&& f) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = m0 + wm * 128 + i * 32 + 8 * (e >> 2) + 4 * fg + (e & 3);
          const int n = n0 + wn * 128 + j * 32 + fr;
          if (full || r < M) f(i, j, e, (size_t)r * N + n);
        }
  };
  if (splits == 1) {
    for_each([&](int i, int j, int e, size_t o) { y[o] = f32_to_half_bits<BF16>(accv[i][j][e]); });
    return;
  }
  float* slice = acc + (size_t)split * M * N;
  for_each([&](int i, int j, int e, size_t o) { slice[o] = accv[i][j][e]; });
}

#ifndef KBH_MX_DMA_MIN_M
#define KBH_MX_DMA_MIN_M 1024
#endif

struct MXPlan {
  bool dma;  // 256 x 256 tiles (mxfp8_dma_kernel)
  int wnt, tiles, splits, slabs_per_split;
};

MXPlan plan_mx(int M, int N, int K) {
  MXPlan p;
  p.dma = M >= KBH_MX_DMA_MIN_M && N % DBM == 0;
  const int mblocks = (M + XBM - 1) / XBM;
  p.wnt = (mblocks * (N / 256) >= 128 && N % 256 == 0) ? 4 : 1;
  p.tiles = p.dma ? ((M + DBM - 1) / DBM) * (N / DBM) : mblocks * (N / (64 * p.wnt));
  const int slabs = K / XBK;
  // Split K only while the grid is below one workgroup per CU; every split keeps a multiple of
  // XDEPTH slabs (branch-free ring) and at least 4 slabs.
  int splits = 1;
  while (p.tiles * splits < 256 && slabs % (splits * 2) == 0 &&
         (slabs / (splits * 2)) % XDEPTH == 0 && slabs / (splits * 2) >= 4)
    splits *= 2;
  p.splits = splits;
  p.slabs_per_split = slabs / splits;
  return p;
}

template <bool BF16>
int mx_launch(const MXPlan& p, const void* a, const void* as, const void* b, const void* bs,
              void* y, float* acc, int M, int N, int K, hipStream_t st) {
  const dim3 grid(p.tiles, 1, p.splits);
  if (p.dma)
    hipLaunchKernelGGL((mxfp8_dma_kernel<BF16>), grid, dim3(256), 0, st, (const uint8_t*)a,
                       (const uint8_t*)as, (const uint8_t*)b, (const uint8_t*)bs, (uint16_t*)y,
                       acc, M, N, K, p.slabs_per_split);
  else if (p.wnt == 4)
    hipLaunchKernelGGL((mxfp8_kernel<4, BF16>), grid, dim3(256), 0, st, (const uint8_t*)a,
                       (const uint8_t*)as, (const uint8_t*)b, (const uint8_t*)bs, (uint16_t*)y,
                       acc, M, N, K, p.slabs_per_split);
  else
    hipLaunchKernelGGL((mxfp8_kernel<1, BF16>), grid, dim3(256), 0, st, (const uint8_t*)a,
                       (const uint8_t*)as, (const uint8_t*)b, (const uint8_t*)bs, (uint16_t*)y,
                       acc, M, N, K, p.slabs_per_split);
  if (p.splits > 1)
    hipLaunchKernelGGL((splitk_sum_half<BF16>), dim3(splitk_sum_blocks(M, N)), dim3(256), 0, st,
                       acc, (uint16_t*)y, (size_t)M * N / 4, p.splits);
  return launch_status();
}

}  // namespace
}  // namespace kbh

extern "C" size_t kbh_mxfp8_workspace_bytes(int M, int N, int K) {
  using namespace kbh;
  if (M <= 0 || N < 64 || K < XBK) return 0;
  const MXPlan p = plan_mx(M, N, K);
  return splitk_workspace_bytes(M, N, p.splits);
}

extern "C" int kbh_mxfp8_gemm(const uint8_t* a, const uint8_t* a_scale, const uint8_t* b,
                              const uint8_t* b_scale, void* y, void* workspace,
                              size_t workspace_bytes, int M, int N, int K, int out_dtype,
                              void* stream) {
  using namespace kbh;
  if (!a || !a_scale || !b || !b_scale || !y) return KBH_ERR_NULL;
  if (out_dtype != KBH_F16 && out_dtype != KBH_BF16) return KBH_ERR_DTYPE;
  if (M < 1 || N < 64 || (N % 64) != 0 || K < XBK * XDEPTH || (K % (XBK * XDEPTH)) != 0)
    return KBH_ERR_SHAPE;
  // The kernel addresses a and b with 32-bit buffer offsets.
  if ((size_t)M * K >= 0x80000000u || (size_t)N * K >= 0x80000000u) return KBH_ERR_SHAPE;
  if (!aligned16(a) || !aligned16(b) || !aligned16(y) || (reinterpret_cast<uintptr_t>(a_scale) & 3) ||
      (reinterpret_cast<uintptr_t>(b_scale) & 3))
    return KBH_ERR_ALIGN;
  const MXPlan p = plan_mx(M, N, K);
  float* acc = nullptr;
  if (p.splits > 1) {
    if (!workspace || workspace_bytes < splitk_workspace_bytes(M, N, p.splits))
      return KBH_ERR_WORKSPACE;
    if (!aligned16(workspace)) return KBH_ERR_ALIGN;
    acc = (float*)workspace;
  }
  hipStream_t st = (hipStream_t)stream;
  if (out_dtype == KBH_BF16) return mx_launch<true>(p, a, a_scale, b, b_scale, y, acc, M, N, K, st);
  return mx_launch<false>(p, a, a_scale, b, b_scale, y, acc, M, N, K, st);
}
