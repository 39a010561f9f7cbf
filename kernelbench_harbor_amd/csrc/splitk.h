// Split-K reduction shared by the decode kernels.
//
// Every decode kernel leaves each wavefront with a 16-row x (16*NCS)-column partial tile in the
// 16x16 MFMA accumulator layout: lane l holds, for column set cs < NCS, rows 4*(l/16)+i (i < 4)
// of output column n0 + (l%16)*NCS + cs. splitk_reduce() sums the waves of the workgroup through
// private LDS slices (one 16-byte write per column set and lane; the reads of the summing pass
// are 16-byte and bank-conflict free; lanes whose rows are all beyond M skip the write), then:
//  * splits == 1: the workgroup emits its tile directly;
//  * otherwise it stores its tile, with plain coalesced stores, into slice `split` of the
//    workspace (acc[split][M][ld]) and ends. A summing kernel launched after it on the same
//    stream adds the slices in split order and applies the epilogue, so the result does not
//    depend on workgroup timing and the workspace needs no clearing. (Device-scope atomics
//    instead cost several microseconds at 16 rows, and an in-kernel last-arriver protocol three
//    serialised memory round trips; the launch boundary orders the two kernels for free.)
#pragma once

#include "kbh_common.h"

namespace kbh {

constexpr int kSplitKMaxWaves = 8;
constexpr int kSplitKCsStride = 260;  // LDS elements per column set per wave (4*64 + pad)

template <int NCS, typename T>
struct SplitKSmem {
  __attribute__((aligned(16))) T red[kSplitKMaxWaves * NCS * kSplitKCsStride];
};

// V is the 4-element vector of T held per column set (kbh_f32x4 / kbh_i32x4).
// emit(r, n, v): row r (< rows) of the tile, column n (< 16*NCS), reduced value v (splits == 1).
// M: rows of one workspace slice; ld: its row stride (the output's N).
template <int NCS, typename T, typename V, typename Emit>
__device__ inline void splitk_reduce(const V (&tot)[NCS], SplitKSmem<NCS, T>& sm, T* acc,
                                     int split, int splits, int rows, int M, int ld, int m0,
                                     int n0, Emit emit) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
  if (4 * (lane >> 4) < rows) {
    T* slice = sm.red + wave * NCS * kSplitKCsStride;
#pragma unroll
    for (int cs = 0; cs < NCS; ++cs)
      *reinterpret_cast<V*>(&slice[cs * kSplitKCsStride + lane * 4]) = tot[cs];
  }
  __syncthreads();
  // Position p = (lane l, column set cs), cs fastest: consecutive threads read consecutive
  // 16-byte chunks (the slice stride is 16 bytes mod 256) and own consecutive output columns.
  const int npos = NCS * 16 * ((rows + 3) >> 2);
  for (int p = threadIdx.x; p < npos; p += blockDim.x) {
    const int cs = p % NCS, l = p / NCS;
    const T* src = &sm.red[cs * kSplitKCsStride + l * 4];
    V v = *reinterpret_cast<const V*>(src);
    for (int wv = 1; wv < waves; ++wv)
      v += *reinterpret_cast<const V*>(src + wv * NCS * kSplitKCsStride);
    const int n = (l & 15) * NCS + cs;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * (l >> 4) + i;
      if (r >= rows) continue;
      if (splits == 1)
        emit(r, n, v[i]);
      else
        acc[((size_t)split * M + m0 + r) * ld + n0 + n] = v[i];
    }
  }
}

// Sums the fp32 split-K slices acc[splits][M*N] in split order and converts the sums to
// fp16/bf16 y. n4 = M*N/4.
template <bool BF16>
__global__ __launch_bounds__(256) void splitk_sum_half(const float* __restrict__ acc,
                                                       uint16_t* __restrict__ y, size_t n4,
                                                       int splits) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  const kbh_f32x4 v = sum_slices(reinterpret_cast<const kbh_f32x4*>(acc) + i, n4, splits);
  kbh_u32x2 o;
  o[0] = (uint32_t)f32_to_half_bits<BF16>(v[0]) | ((uint32_t)f32_to_half_bits<BF16>(v[1]) << 16);
  o[1] = (uint32_t)f32_to_half_bits<BF16>(v[2]) | ((uint32_t)f32_to_half_bits<BF16>(v[3]) << 16);
  *reinterpret_cast<kbh_u32x2*>(y + 4 * i) = o;
}

inline unsigned splitk_sum_blocks(int M, int N) {
  return (unsigned)(((size_t)M * N / 4 + 255) / 256);
}

// Slice sum placed on the XCDs that wrote the slices. A decode launch of ntiles x splits
// workgroups (grid.x, logical id = tile * splits + split after xcd_remap) runs logical ids
// [x P, (x + 1) P), P = grid.x / 8, on XCD x: the splits of tiles [t_lo(x), t_lo(x + 1)),
// t_lo(x) = ceil(x P / splits). Workgroup b of this kernel runs on XCD b % 8 and sums (in split
// order) outputs of those tiles only, so its loads hit the L2 that holds the freshly written
// slices instead of crossing to another XCD's writes through the Infinity Cache (measured on a
// 16 x 16 split M=16 decode: 5.4 -> 2.6 us per sum). Any dispatch order gives the same result;
// only the speed depends on it. xcd == 0: plain indexing (thread i sums outputs 4i..4i+3).
// One thread per 4 consecutive outputs of a row; ep.emit4(r, n, V) writes them.
template <class V, class EP>
__global__ __launch_bounds__(256) void splitk_sum_kernel(const V* __restrict__ acc, EP ep, int M,
                                                         int N, int ntiles, int tn, int splits,
                                                         int xcd, int per_xcd) {
  const size_t n4 = (size_t)M * N / 4;
  if (!xcd) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const V v = sum_slices(acc + i, n4, splits);
    const int r = (int)(4 * i / (size_t)N);
    ep.emit4(r, (int)(4 * i - (size_t)r * N), v);
    return;
  }
  const int x = blockIdx.x & 7, j = blockIdx.x >> 3;
  const int P = ntiles * splits / 8;
  const int t_lo = (x * P + splits - 1) / splits;
  const int t_hi = min(ntiles, ((x + 1) * P + splits - 1) / splits);
  const int c4 = (t_hi - t_lo) * tn / 4;  // 4-output groups per row on this XCD
  const int total = M * c4;
  for (int q = j * 256 + threadIdx.x; q < total; q += per_xcd * 256) {
    const int r = q / c4, n = t_lo * tn + 4 * (q - r * c4);
    const size_t i = ((size_t)r * N + n) / 4;
    ep.emit4(r, n, sum_slices(acc + i, n4, splits));
  }
}

// Launches splitk_sum_kernel for a decode grid of ntiles x splits workgroups of tn columns.
template <class V, class EP>
void launch_splitk_sum(const V* acc, EP ep, int M, int N, int ntiles, int tn, int splits,
                       hipStream_t st) {
  const int nb = ntiles * splits;
  if (nb % 8 != 0) {
    hipLaunchKernelGGL((splitk_sum_kernel<V, EP>), dim3(splitk_sum_blocks(M, N)), dim3(256), 0, st,
                       acc, ep, M, N, ntiles, tn, splits, 0, 0);
    return;
  }
  const int P = nb / 8;
  int most = 0;  // 4-output groups of the busiest XCD
  for (int x = 0; x < 8; ++x) {
    const int lo = (x * P + splits - 1) / splits;
    const int hi = ((x + 1) * P + splits - 1) / splits;
    most = hi - lo > most ? hi - lo : most;
  }
  const int per_xcd = (int)(((size_t)M * most * tn / 4 + 255) / 256);
  hipLaunchKernelGGL((splitk_sum_kernel<V, EP>), dim3(8 * per_xcd), dim3(256), 0, st, acc, ep, M, N,
                     ntiles, tn, splits, 1, per_xcd);
}

// Workspace of a split-K call: `splits` slices of fp32/int32 partial sums [M, N] (none
// unsplit). No content requirement between calls.
inline size_t splitk_workspace_bytes(int M, int N, int splits) {
  if (M <= 0 || N <= 0 || splits <= 1) return 0;
  return round_up((size_t)splits * M * (size_t)N * 4u, 256);
}

// Picks waves per workgroup (<= kSplitKMaxWaves) so that `units` wave-sized K ranges per column
// tile split evenly and the grid is close to one or two workgroups per CU. Returns the number of
// waves (0 if none divides) and sets *splits.
inline int splitk_pick_waves(int units, int tiles_per_split, int* splits) {
  int best_w = 0, best_score = 1 << 30;
  for (int w = kSplitKMaxWaves; w >= 1; --w) {
    if (units % w) continue;
    const int grid = tiles_per_split * (units / w);
    const int score = grid < 256 ? (256 - grid) * 4 : (grid > 512 ? grid - 512 : 0) + (8 - w);
    if (score < best_score) { best_score = score; best_w = w; }
  }
  if (best_w) *splits = units / best_w;
  return best_w;
}

}  // namespace kbh
