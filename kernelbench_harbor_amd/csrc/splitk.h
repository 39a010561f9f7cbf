// Split-K reduction shared by the decode kernels.
//
// Every decode kernel leaves each wavefront with a 16-row x (16*NCS)-column partial tile in the
// 16x16 MFMA accumulator layout: lane l holds, for column set cs < NCS, rows 4*(l/16)+i (i < 4)
// of output column n0 + (l%16)*NCS + cs. splitk_finish() sums the waves of the workgroup through
// private LDS slices (no LDS atomics: waves adding into one slice serialise), then sums the
// K-split workgroups of the tile:
//  * splits == 1: the workgroup emits its tile directly;
//  * otherwise each workgroup adds its tile into the workspace with agent-scope atomics, waits
//    until its atomics are acknowledged (s_waitcnt 0), and counts its arrival on the tile's
//    counter; the workgroup that arrives last reads the complete sums with agent-scope atomic
//    loads, emits them and clears the workspace tile and the counter for the next call.
// Agent-scope atomics are performed at the device coherence point, so partial sums from
// workgroups on different XCDs meet there.
#pragma once

#include "kbh_common.h"

namespace kbh {

constexpr int kSplitKMaxWaves = 8;
constexpr int kSplitKCsStride = 260;  // LDS elements per column set per wave (4*64 + pad)

template <int NCS, typename T>
struct SplitKSmem {
  T red[kSplitKMaxWaves * NCS * kSplitKCsStride];
  int last;
};

// emit(r, n, v): row r (< rows) of the tile, column n (< 16*NCS), reduced value v.
template <int NCS, typename T, typename V, typename Emit>
__device__ inline void splitk_finish(const V (&tot)[NCS], SplitKSmem<NCS, T>& sm, T* acc,
                                     int* counter, int splits, int rows, int ld, int m0, int n0,
                                     Emit emit) {
  constexpr int NWG = 16 * NCS;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
  {
    T* slice = sm.red + wave * NCS * kSplitKCsStride;
#pragma unroll
    for (int cs = 0; cs < NCS; ++cs)
#pragma unroll
      for (int i = 0; i < 4; ++i) slice[cs * kSplitKCsStride + i * 64 + lane] = tot[cs][i];
  }
  __syncthreads();
  auto lds_sum = [&](int r, int n) {
    const int cc = n / NCS, cs = n - cc * NCS;
    const int off = cs * kSplitKCsStride + (r & 3) * 64 + (r >> 2) * 16 + cc;
    T v = 0;
    for (int wv = 0; wv < waves; ++wv) v += sm.red[wv * NCS * kSplitKCsStride + off];
    return v;
  };
  if (splits == 1) {
    for (int e = threadIdx.x; e < rows * NWG; e += blockDim.x) {
      const int r = e / NWG, n = e - r * NWG;
      emit(r, n, lds_sum(r, n));
    }
    return;
  }
  for (int e = threadIdx.x; e < rows * NWG; e += blockDim.x) {
    const int r = e / NWG, n = e - r * NWG;
    __hip_atomic_fetch_add(&acc[(size_t)(m0 + r) * ld + n0 + n], lds_sum(r, n), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sm.last = (prev == splits - 1);
  }
  __syncthreads();
  if (!sm.last) return;
  for (int e = threadIdx.x; e < rows * NWG; e += blockDim.x) {
    const int r = e / NWG, n = e - r * NWG;
    T* p = &acc[(size_t)(m0 + r) * ld + n0 + n];
    const T v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p, (T)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    emit(r, n, v);
  }
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workspace layout of a split-K call: fp32/int32 accumulators [M, N], then one arrival counter
// per (16-row block, 128-column tile).
inline size_t splitk_workspace_bytes(int M, int N) {
  if (M <= 0 || N <= 0) return 0;
  return round_up((size_t)M * (size_t)N * 4u, 256) +
         round_up((size_t)((M + 15) / 16) * (size_t)(N / 128 + 1) * 4u, 256);
}
inline int* splitk_counters(void* workspace, int M, int N) {
  return (int*)((char*)workspace + round_up((size_t)M * (size_t)N * 4u, 256));
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
