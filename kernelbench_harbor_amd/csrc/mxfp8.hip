// MXFP8 block-scaled GEMM on gfx950 scaled MFMA (no reference module:
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
// fragment reads). Each wave computes 64 x (32*WNT) with 2 x WNT MFMA tiles. For small M the K
// range is split over gridDim.z; each split stores its partial tile into its own fp32 workspace
// slice and splitk_sum_half (splitk.h) adds the slices in split order and converts.
#include "kbh_common.h"
#include "splitk.h"

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

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int ntn = N / XBN;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int mb = id / ntn, nb = id - mb * ntn;
  const int m0 = mb * XBM, n0 = nb * XBN;
  const int splits = gridDim.z, split = blockIdx.z;
  const int KS = K / 32;  // scale columns
  const int kt_begin = split * slabs_per_split;
  const int KT = slabs_per_split;

  // global -> register mapping: 16-byte chunk t%8 of rows t/8 + 32i
  const int ch = t & 7, rr = t >> 3;
  const uint8_t* arow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = m0 + rr + 32 * i;
    arow[i] = a + (size_t)(r < M ? r : M - 1) * K + ch * 16;  // rows >= M are never stored
  }
  const uint8_t* brow[WNT * 2];
#pragma unroll
  for (int i = 0; i < 2 * WNT; ++i) brow[i] = b + (size_t)(n0 + rr + 32 * i) * K + ch * 16;
  // scale rows of this lane: A row tiles i < 2, B column tiles j < WNT
  const int fr = lane & 31, fg = lane >> 5;
  const uint8_t* asrow[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = m0 + wm * 64 + i * 32 + fr;
    asrow[i] = as + (size_t)(r < M ? r : M - 1) * KS;
  }
  const uint8_t* bsrow[WNT];
#pragma unroll
  for (int j = 0; j < WNT; ++j) bsrow[j] = bs + (size_t)(n0 + wn * 32 * WNT + j * 32 + fr) * KS;

  struct Slab {
    kbh_u32x4 a[4];
    kbh_u32x4 b[2 * WNT];
    uint32_t sa[2];
    uint32_t sb[WNT];
  };
  auto load = [&](Slab& sl, int kt) {
    const int k0 = (kt_begin + kt) * XBK;
#pragma unroll
    for (int i = 0; i < 4; ++i) sl.a[i] = *reinterpret_cast<const kbh_u32x4*>(arow[i] + k0);
#pragma unroll
    for (int i = 0; i < 2 * WNT; ++i)
      sl.b[i] = __builtin_nontemporal_load(reinterpret_cast<const kbh_u32x4*>(brow[i] + k0));
#pragma unroll
    for (int i = 0; i < 2; ++i) sl.sa[i] = *reinterpret_cast<const uint32_t*>(asrow[i] + k0 / 32);
#pragma unroll
    for (int j = 0; j < WNT; ++j) sl.sb[j] = *reinterpret_cast<const uint32_t*>(bsrow[j] + k0 / 32);
  };
  auto store = [&](const Slab& sl, int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<kbh_u32x4*>(&Al[buf][(rr + 32 * i) * XLD + ch * 16]) = sl.a[i];
#pragma unroll
    for (int i = 0; i < 2 * WNT; ++i)
      *reinterpret_cast<kbh_u32x4*>(&Bl[buf][(rr + 32 * i) * XLD + ch * 16]) = sl.b[i];
  };

  kbh_f32x16 accv[2][WNT];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < WNT; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) accv[i][j][e] = 0.f;

  // One 64-deep K step (kk = 0, 1 within the slab). Scale byte 2*kk + g of the slab's dword.
  auto mma_k64 = [&](int buf, int kk, const Slab& sl) {
    const uint8_t* Ab = &Al[buf][(wm * 64 + fr) * XLD + kk * 64 + 16 * fg];
    const uint8_t* Bb = &Bl[buf][(wn * 32 * WNT + fr) * XLD + kk * 64 + 16 * fg];
    kbh_u32x4 a0[2], a1[2], b0[WNT], b1[WNT];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      a0[i] = *reinterpret_cast<const kbh_u32x4*>(Ab + i * 32 * XLD);
      a1[i] = *reinterpret_cast<const kbh_u32x4*>(Ab + i * 32 * XLD + 32);
    }
#pragma unroll
    for (int j = 0; j < WNT; ++j) {
      b0[j] = *reinterpret_cast<const kbh_u32x4*>(Bb + j * 32 * XLD);
      b1[j] = *reinterpret_cast<const kbh_u32x4*>(Bb + j * 32 * XLD + 32);
    }
    const int sh = 8 * (2 * kk + fg);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int sa = (int)((sl.sa[i] >> sh) & 0xffu);
#pragma unroll
      for (int j = 0; j < WNT; ++j) {
        const int sb = (int)((sl.sb[j] >> sh) & 0xffu);
        accv[i][j] = mfma_mx32(a0[i], a1[i], b0[j], b1[j], accv[i][j], sa, sb);
      }
    }
  };

  // Ring of XDEPTH slabs; the scales of slab kt stay in `cur` while its data sits in LDS.
  Slab ring[XDEPTH];
  Slab cur;
#pragma unroll
  for (int d = 0; d < XDEPTH; ++d) load(ring[d], min(d, KT - 1));
  store(ring[0], 0);
  cur = ring[0];
  load(ring[0], min(XDEPTH, KT - 1));
  __syncthreads();
  for (int kt0 = 0; kt0 < KT; kt0 += XDEPTH) {
#pragma unroll
    for (int d = 0; d < XDEPTH; ++d) {
      // KT is a multiple of XDEPTH: no branch here (see tiled_f16.h on wait counts).
      const int kt = kt0 + d;
      const int nxt = (d + 1) % XDEPTH;
      mma_k64(kt & 1, 0, cur);
      store(ring[nxt], (kt + 1) & 1);  // after the last slab: unused buffer
      mma_k64(kt & 1, 1, cur);
      cur.sa[0] = ring[nxt].sa[0];
      cur.sa[1] = ring[nxt].sa[1];
#pragma unroll
      for (int j = 0; j < WNT; ++j) cur.sb[j] = ring[nxt].sb[j];
      load(ring[nxt], min(kt + 1 + XDEPTH, KT - 1));
      __syncthreads();
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

struct MXPlan {
  int wnt, tiles, splits, slabs_per_split;
};

MXPlan plan_mx(int M, int N, int K) {
  MXPlan p;
  const int mblocks = (M + XBM - 1) / XBM;
  p.wnt = (mblocks * (N / 256) >= 128 && N % 256 == 0) ? 4 : 1;
  p.tiles = mblocks * (N / (64 * p.wnt));
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
  if (p.wnt == 4)
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
