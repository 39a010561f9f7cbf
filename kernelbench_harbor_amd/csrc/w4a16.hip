// W4A16 packed-asymmetric group-quantized GEMM for gfx950.
//
// Semantics (reference tasks/quant_w4a16_pa/*/environment/reference.py:10-17):
//   w[k, n] = (((qweight[k, n/8] >> 4*(n%8)) & 0xF) - zeros[k/G, n]) * scales[k/G, n]
//   y       = x @ w
//
// Two kernels:
//
// w4a16_decode_kernel (M <= 16 per 16-row block; HBM-bound decode shapes)
//  * A wavefront owns 128*NW output columns and SPW consecutive 32-row K steps; every load of
//    the wavefront (SPW*8 rows of NW packed words per lane, plus its x fragments) is issued
//    before any arithmetic so that the whole chip's weight stream is in flight at once.
//    Lane l reads qweight[k0 + 8(l/16) + i][n0/8 + (l%16)*NW + w], i = 0..7.
//  * Nibbles become fp16/bf16 MFMA B-fragments with no per-weight arithmetic: one v_perm_b32
//    places byte j of the words of rows k, k+1 into the two 16-bit halves and one v_and_or_b32
//    with a magic exponent turns nibble q into the value B+q (fp16: 1024+q, or 1024+16q for the
//    high nibble; bf16: 128+q). Each (word, nibble) pair feeds one 16x16x32 MFMA whose 16 output
//    columns lie 8*NW apart in n.
//  * Zero points and scales are applied once per quantization group on the fp32 accumulators:
//      sum_k x_k (q_k - z) s = s * (sum_k x_k (B + f q_k) / f - (B/f + z) * sum_k x_k)
//    with sum_k x_k from one extra MFMA against a ones fragment.
//  * The waves of a workgroup (consecutive K ranges of one column tile) reduce through private
//    LDS slices; each workgroup (K split) stores its tile into its own workspace slice, and
//    splitk_sum_kernel, run on the XCDs that wrote them, adds the slices in split order and
//    converts to the output dtype (splitk.h). Workgroup ids are remapped so that all K splits
//    of a column tile run on one XCD.
//
// Larger M (M > 32): tiled_wide_gemm (tiled_wide.h) with W4WidePolicy, which dequantizes each
// packed 32 x TN weight slab once per workgroup into LDS with the exact reference arithmetic
// ((q - z) rounded to the input dtype, times s rounded), in MFMA fragment order; x goes from
// global memory straight into MFMA registers. Split-K partial sums use the caller's scratch.
// Shapes it does not cover fall back to tiled_f16_gemm (256 x 128 LDS-staged tiles) or to the
// decode kernel.
#include "kbh_common.h"
#include "splitk.h"
#include "tiled_f16.h"
#include "tiled_wide.h"
#include "tiled_ws.h"
#include "tiled_ws256.h"
#include "w4_dequant.h"

namespace kbh {
namespace {

// ======================================================================================
// Decode kernel
// ======================================================================================

// SPG = K steps per quantization group when a group is shorter than a wave's K range
// (SPG < SPW), otherwise SPG == SPW (each wave lies inside one group). The fold schedule is thus
// static, and the scales/zeros of every group a wave touches are loaded with its weights.
template <int NW, int SPW, int SPG, bool BF16>
__global__ __launch_bounds__(kSplitKMaxWaves * 64) void w4a16_decode_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ qw,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    uint16_t* __restrict__ y, float* __restrict__ acc, int M, int N, int K, int group,
    int splits) {
  constexpr int NWG = 128 * NW;  // output columns of one workgroup
  constexpr int NCS = 8 * NW;    // MFMA column sets per wave
  constexpr uint32_t MAGIC = BF16 ? kMagicBF16 : kMagicF16;
  __shared__ SplitKSmem<NCS, float> sm;

  const int waves = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: SGPR addressing
  const int c = lane & 15;
  const int g = lane >> 4;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = id / splits;
  const int split = id - tile * splits;
  const int n0 = tile * NWG;
  const int m0 = blockIdx.y * 16;
  const int st0 = (split * waves + wave) * SPW;  // first 32-row K step of this wave
  const int NP = N >> 3;

  // ---- every load of this wave, up front ----------------------------------------------
  // x fragments and group constants first: loads complete in issue order, so the MFMAs of
  // step u can start as soon as step u's weights arrive, while later steps are still in flight.
  kbh_u32x4 af[SPW];
  const bool xok = m0 + c < M;
  const uint16_t* xb = x + (size_t)(xok ? m0 + c : 0) * K + st0 * 32 + 8 * g;
#pragma unroll
  for (int u = 0; u < SPW; ++u) af[u] = *reinterpret_cast<const kbh_u32x4*>(xb + u * 32);
  constexpr int NG = SPW / SPG;  // quantization groups touched by this wave
  kbh_u32x4 sv[NG][NW], zv[NG][NW];
#pragma unroll
  for (int gq = 0; gq < NG; ++gq) {
    const int gi = ((st0 + gq * SPG) << 5) / group;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const size_t off = (size_t)gi * N + n0 + 8 * (c * NW + w);
      sv[gq][w] = *reinterpret_cast<const kbh_u32x4*>(scales + off);
      zv[gq][w] = *reinterpret_cast<const kbh_u32x4*>(zeros + off);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // keeps the group constants ahead of the weight stream
  uint32_t wd[SPW][8][NW];
  // Buffer loads from the wave's first row: the row offset is an SGPR (soffset) and the lane
  // offset one VGPR, so no load needs per-lane 64-bit address arithmetic (global loads got a
  // v_lshl_add_u64 chain). Reads past the matrix would return zero (range-checked resource).
  const size_t qbase = (size_t)st0 * 32 * NP + (n0 >> 3);
  const __amdgpu_buffer_rsrc_t qres = make_rsrc(qw + qbase, ((size_t)K * NP - qbase) * 4);
  const uint32_t qlane = (uint32_t)(8 * g * NP + c * NW) * 4u;
#pragma unroll
  for (int u = 0; u < SPW; ++u) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int soff = (u * 32 + i) * NP * 4;
      if constexpr (NW == 2) {
        const kbh_u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(qres, qlane, soff, kBufNT);
        wd[u][i][0] = v[0];
        wd[u][i][1] = v[1];
      } else {
        wd[u][i][0] = __builtin_amdgcn_raw_buffer_load_b32(qres, qlane, soff, kBufNT);
      }
    }
  }
  // Nothing may use a loaded value before the last load is issued: a consumer scheduled between
  // the loads makes the wave wait one memory latency with part of its stream not yet requested.
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < SPW; ++u)
    if (!xok) af[u] = kbh_u32x4{0u, 0u, 0u, 0u};  // rows past M contribute zero

  const uint32_t one = BF16 ? kOneBF16 : kOneF16;
  const kbh_u32x4 ones = {one, one, one, one};
  // The nibble masks in SGPRs and the magic exponent in a VGPR: (P & mask) | magic is then one
  // v_and_or_b32 (a VOP3 here takes no literal and reads at most one SGPR); with literals the
  // compiler emits a v_and_b32 and a v_or_b32 per B dword.
  uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u, magic = MAGIC;
  asm volatile("" : "+s"(mlo), "+s"(mhi));
  asm volatile("" : "+v"(magic));
  kbh_f32x4 tot[NCS], part[NCS], xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int cs = 0; cs < NCS; ++cs) {
    tot[cs] = kbh_f32x4{0.f, 0.f, 0.f, 0.f};
    part[cs] = tot[cs];
  }
#pragma unroll
  for (int u = 0; u < SPW; ++u) {
    xs = mfma16x16x32<BF16>(af[u], ones, xs);
#pragma unroll
    for (int w = 0; w < NW; ++w) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        kbh_u32x4 blo, bhi;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const uint32_t P = pair_bytes_rt(wd[u][2 * p][w], wd[u][2 * p + 1][w], j);
          blo[p] = (P & mlo) | magic;
          bhi[p] = BF16 ? (((P >> 4) & mlo) | magic) : ((P & mhi) | magic);
        }
        part[w * 8 + 2 * j] = mfma16x16x32<BF16>(af[u], blo, part[w * 8 + 2 * j]);
        part[w * 8 + 2 * j + 1] = mfma16x16x32<BF16>(af[u], bhi, part[w * 8 + 2 * j + 1]);
      }
    }
    // Fold at the end of each quantization group (static schedule).
    if ((u + 1) % SPG == 0) {
      const int gq = u / SPG;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
#pragma unroll
        for (int nib = 0; nib < 8; ++nib) {
          const uint32_t sw = sv[gq][w][nib >> 1], zw = zv[gq][w][nib >> 1];
          const uint16_t sh = (uint16_t)((nib & 1) ? (sw >> 16) : (sw & 0xffffu));
          const uint16_t zh = (uint16_t)((nib & 1) ? (zw >> 16) : (zw & 0xffffu));
          const float s = half_bits_to_f32<BF16>(sh);
          const float z = half_bits_to_f32<BF16>(zh);
          const float a = (!BF16 && (nib & 1)) ? 0.0625f : 1.0f;
          const float bz = (BF16 ? 128.0f : ((nib & 1) ? 64.0f : 1024.0f)) + z;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float t = fmaf(-bz, xs[i], part[w * 8 + nib][i] * a);
            tot[w * 8 + nib][i] = fmaf(s, t, tot[w * 8 + nib][i]);
          }
          part[w * 8 + nib] = kbh_f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
      xs = kbh_f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  // The fold's only use is inside splitk_reduce's row-guarded branch; without this the compiler
  // sinks the fold, and the group-constant loads with it, behind that branch and the last weight.
#pragma unroll
  for (int cs = 0; cs < NCS; ++cs) asm volatile("" : "+v"(tot[cs]));
  const int rows = min(16, M - m0);
  splitk_reduce<NCS, float>(tot, sm, acc, split, splits, rows, M, N, m0, n0, [&](int r, int n, float v) {
    y[(size_t)(m0 + r) * N + n0 + n] = f32_to_half_bits<BF16>(v);
  });
}

struct DecodePlan {
  int nw, spw, spg, waves, ntiles, splits, mblocks;
};

// The (NW, SPW, SPG) instantiations of w4a16_decode_kernel; plan_decode picks only from these.
// NW = 2 takes at most two quantization groups per wave (SPW / SPG <= 2): more groups' constants
// on top of 256 columns' accumulators spill. SPW = 8 exists only with NW = 2 (NW = 1 was measured
// slower with it on every shape swept).
#define KBH_DECODE_VARIANTS(X)                                                                   \
  X(2, 8, 8) X(2, 8, 4) X(2, 4, 4) X(2, 4, 2) X(2, 2, 2) X(2, 2, 1) X(2, 1, 1) X(1, 4, 4)         \
  X(1, 4, 2) X(1, 4, 1) X(1, 2, 2) X(1, 2, 1) X(1, 1, 1)

bool decode_variant_built(int nw, int spw, int spg) {
#define KBH_DEC_IS(NW_, SPW_, SPG_) if (nw == NW_ && spw == SPW_ && spg == SPG_) return true;
  KBH_DECODE_VARIANTS(KBH_DEC_IS)
#undef KBH_DEC_IS
  return false;
}

// Estimated duration (µs, up to a constant) of a decode launch plus its split-K sum. Every load
// of a workgroup is in flight at once, so a CU's time is set by the weight bytes of the
// workgroups it runs one after another (KB = 2 per K step per 128 columns) plus a fixed cost per
// workgroup (halved when two fit on a CU: NW = 1 needs half the LDS), and fewer waves issue
// those bytes more slowly; the split-K slices add a write and a read of splits x M x N fp32.
// The constants are a least-squares fit to a sweep of every (NW, SPW, waves) plan on MI355X
// over the shapes K x N = 4096 x 14336, 14336 x 4096, 8192 x 28672, 28672 x 8192,
// 3584 x 18944, 18944 x 3584, 8192 x 29568 and 29568 x 8192 at M = 1 and 16 (group 128): the
// plan it picks is within 2% of the sweep's fastest NW = 2 plan on all 16, where the former
// "grid closest to one workgroup per CU" rule lost up to 28%.
float decode_cost(int M, int N, int nw, int spw, int waves, int splits, int grid) {
  const float kb = 2.0f * spw * waves * nw;
  const float slowdown = 1.0f + 0.53f * (8 - waves) / 8.0f;
  const int per_cu = (grid + 255) / 256;
  float t = per_cu * ((nw == 1 ? 0.9f : 1.8f) + kb * slowdown / 23.3f);
  if (splits > 1) t += (float)splits * M * N * 8.0f / 1024.0f / 2540.0f;
  return t;
}

// Chooses column width (NW: 128*NW columns per workgroup), K steps per wave (SPW) and waves per
// workgroup (the K steps divide evenly) by decode_cost. NW = 2 whenever N allows it (NW = 1 plans
// that the cost prefers there were measured slower on most shapes: half-width rows per load),
// except with 32-row groups, where NW = 2 holds at most SPW = 2 and NW = 1 with SPW = 4
// measured 4-11% faster.
bool plan_decode(int M, int N, int K, int group_steps_, DecodePlan* p) {
  const int nsteps = K / 32;
  const int gsteps = group_steps_;  // 1, 2, 4 or 8 (group 32..256); divides nsteps
  const int nw = (N % 256 == 0 && gsteps > 1) ? 2 : 1;
  const int ntiles = N / (128 * nw);
  const int mblocks = (M + 15) / 16;
  float best = 0.0f;
  p->waves = 0;
  for (int spw = 8; spw >= 1; spw >>= 1) {
    if (nsteps % spw != 0) continue;
    // Wave ranges start at multiples of SPW steps, so they stay inside one group when the group
    // spans a multiple of SPW steps; otherwise the group (1, 2 or 4 steps) divides SPW.
    const int spg = (gsteps % spw == 0) ? spw : gsteps;
    if (!decode_variant_built(nw, spw, spg)) continue;
    const int units = nsteps / spw;
    for (int w = kSplitKMaxWaves; w >= 1; --w) {
      if (units % w != 0) continue;
      const int splits = units / w;
      const float c = decode_cost(M, N, nw, spw, w, splits, ntiles * splits * mblocks);
      if (p->waves == 0 || c < best) {
        best = c;
        *p = DecodePlan{nw, spw, spg, w, ntiles, splits, mblocks};
      }
    }
  }
  return p->waves > 0;
}

template <int NW, int SPW, int SPG, bool BF16>
void launch_decode(const DecodePlan& p, const void* x, const int32_t* qw, const void* s,
                   const void* z, void* y, float* acc, int M, int N, int K, int group,
                   hipStream_t stream) {
  dim3 grid(p.ntiles * p.splits, p.mblocks);
  hipLaunchKernelGGL((w4a16_decode_kernel<NW, SPW, SPG, BF16>), grid, dim3(p.waves * 64), 0, stream,
                     (const uint16_t*)x, (const uint32_t*)qw, (const uint16_t*)s,
                     (const uint16_t*)z, (uint16_t*)y, acc, M, N, K, group, p.splits);
  if (p.splits > 1)
    launch_splitk_sum(reinterpret_cast<const kbh_f32x4*>(acc), HalfOut<BF16>{(uint16_t*)y, N}, M, N,
                      p.ntiles, 128 * NW, p.splits, stream);
}

template <bool BF16>
void dispatch_decode(const DecodePlan& p, const void* x, const int32_t* qw, const void* s,
                     const void* z, void* y, float* acc, int M, int N, int K, int group,
                     hipStream_t st) {
#define KBH_DEC(NW_, SPW_, SPG_)                                                                 \
  if (p.nw == NW_ && p.spw == SPW_ && p.spg == SPG_)                                             \
    return launch_decode<NW_, SPW_, SPG_, BF16>(p, x, qw, s, z, y, acc, M, N, K, group, st);
  KBH_DECODE_VARIANTS(KBH_DEC)
#undef KBH_DEC
}

// ======================================================================================
// Large-M kernels
// ======================================================================================
// Above kWideMinM rows the wide-tile kernel (tiled_wide.h) takes over from the split-K decode
// kernel: up to 64 rows, 64 x 256 tiles; up to 256 rows, 128 x 256 tiles with one workgroup per
// CU (128 x 128 tiles, two per CU, up to 128 rows when N is not a multiple of 256); 256 x 256
// tiles above unless the planner's estimate prefers 128-row tiles. The 256-column tiles run
// with a 4-slab prefetch ring; those of 64 and 128 rows on the warp-specialised kernel
// (tiled_ws.h: 4 dequantizing and 4 MFMA waves per workgroup), those of 256 rows on its 12-wave
// form (tiled_ws256.h: 4 waves stage weights and x, 8 MFMA waves; K=14336 N=4096 M=1024
// 153.0 -> 131.7 us, M=2048 282.7 -> 245.9 us against the 4-wave kernel). The older 256 x 128
// LDS-staged kernel remains for shapes the wide kernel does not cover.
constexpr int kWideMinM = 33;
constexpr int kTiledMinM = 128;

struct W4Wide {
  WidePlan plan;
  int tn;
  int spg;  // K slabs (32 rows) per quantization group
};

// Prefetch depth of a wide W4 launch with tn-column tiles.
constexpr int w4_wide_pd(int tn) { return tn == 256 ? 4 : 2; }

bool plan_w4_wide(int M, int N, int K, int group, W4Wide* w) {
  if (M < kWideMinM) return false;
  w->spg = group / 32;
  const bool small = M <= 128;
  w->tn = (N % 256 == 0) ? 256 : 128;
  if (!small && w->tn != 256) return false;
  const int pd = w4_wide_pd(w->tn);
  const int unroll = 2 * w->spg > pd ? 2 * w->spg : pd;  // the kernel's slabs per iteration
  // Up to 64 rows with 256-column tiles: 64 x 256 tiles (2 x 2 waves of 32 x 128); a 128-row
  // tile would spend half its MFMAs and A loads on padding. The split count is planned for one
  // workgroup per CU: more splits (two per CU) measured slower, their fp32 slices outweighing
  // the extra parallelism (K=14336 N=4096 M=64: 14 splits 31.2 us, 28 splits 34.4 us).
  // 128-row tiles (one warp-specialised workgroup per CU) up to 256 rows: fewer K splits, so
  // fewer fp32 slices to write and sum, than 256-row tiles (K=14336 N=4096, M=256: 50.5 against
  // 53.7 us); above, 256-row tiles on the 12-wave kernel unless the estimate prefers 128 rows
  // (M=320 68.9 against 75.2 us, M=384 71.4 / 77.3, M=512 80.5 / 84.7).
  const bool rows64 = M <= 64 && w->tn == 256;
  return plan_wide(M, N, K, w->tn, 32, unroll, w->tn == 128 ? 512 : 256, &w->plan,
                   rows64 ? 64 : 128, w->tn == 256, w->tn == 256 ? 256 : 128);
}

template <bool BF16, int TM, int TN, int SPG>
void launch_w4_wide(const W4Wide& w, const void* x, const int32_t* qw, const void* s, const void* z,
                    void* y, float* scratch, int M, int N, int K, int group, hipStream_t st) {
  using E = WideHalf<BF16>;
  using BP = W4WidePolicy<BF16, TN>;
  using EP = HalfOut<BF16>;
  // MFMA waves along M: 2 x 2 waves for 64- and 128-row tiles (128-row tiles: 64 x 128 per wave,
  // each B fragment read by 2 waves instead of 4; K=14336 N=4096 M=128 35.6 -> 34.9 us, M=256
  // 50.9 -> 49.8 against 4 x 1 waves of 32 x 256), 4 x 1 for the 4-wave kernel's 256-row tiles.
  constexpr int WM = TM == 256 ? 4 : 2;
  const BP bp{(const uint32_t*)qw, (const uint16_t*)s, (const uint16_t*)z, N, group, 0, 0,
              0x000F000Fu};
  const EP ep{(uint16_t*)y, N};
  // Producer sets of the warp-specialised kernel: two for 64-row tiles, whose MFMA waves need
  // only 64 accumulator registers, so that 12 waves fit (K=14336 N=4096: M=33 24.2 -> 23.5 us,
  // M=48 25.4 -> 24.7, M=64 26.7 -> 26.4; an 8-slab raw ring on top measured no faster).
  constexpr int PS = TM == 64 ? 2 : 1;
  if constexpr (TM <= 128 && TN == 256) {
    // 128-row tiles stage x through LDS too (XD) while x is under 2 GiB.
    if (TM == 128 && (size_t)M * K * 2 < ((size_t)1 << 31))
      hipLaunchKernelGGL((tiled_ws_gemm<E, TM, WM, SPG, BP, EP, DenseRows, w4_wide_pd(TN), PS,
                                        TM == 128>),
                         dim3(w.plan.grid), dim3(256 * (1 + PS)), 0, st,
                         x, bp, ep, scratch, M, N, K, w.plan.splits, w.plan.slabs_per_split,
                         DenseRows{M});
    else
      hipLaunchKernelGGL((tiled_ws_gemm<E, TM, WM, SPG, BP, EP, DenseRows, w4_wide_pd(TN), PS>),
                         dim3(w.plan.grid), dim3(256 * (1 + PS)), 0, st,
                         x, bp, ep, scratch, M, N, K, w.plan.splits, w.plan.slabs_per_split,
                         DenseRows{M});
  } else {
    // 256 x 256 tiles: the 12-wave kernel while x is under 2 GiB (its buffer offsets are
    // 32-bit), else the 4-wave one.
    bool done = false;
    if constexpr (TM == 256 && TN == 256) {
      if ((size_t)(M + TM) * K * 2 < ((size_t)1 << 31)) {
        hipLaunchKernelGGL((tiled_ws256_gemm<E, SPG, BP, EP, w4_wide_pd(TN)>), dim3(w.plan.grid),
                           dim3(768), 0, st, x, bp, ep, scratch, M, N, K, w.plan.splits,
                           w.plan.slabs_per_split);
        done = true;
      }
    }
    if (!done)
      hipLaunchKernelGGL((tiled_wide_gemm<E, TM, WM, SPG, BP, EP, DenseRows, 0, w4_wide_pd(TN)>),
                         dim3(w.plan.grid), dim3(256), 0, st,
                         x, bp, ep, scratch, M, N, K, w.plan.splits, w.plan.slabs_per_split,
                         DenseRows{M});
  }
  if (w.plan.splits > 1) {
    const size_t n4 = (size_t)M * N / 4;
    hipLaunchKernelGGL((wide_reduce_kernel<E, EP>), dim3((unsigned)((n4 + 255) / 256)), dim3(256),
                       0, st, scratch, ep, N, n4, w.plan.splits);
  }
}

template <bool BF16, int TM, int TN>
void dispatch_w4_wide_spg(const W4Wide& w, const void* x, const int32_t* qw, const void* s,
                          const void* z, void* y, float* scratch, int M, int N, int K, int group,
                          hipStream_t st) {
  switch (w.spg) {
    case 1: return launch_w4_wide<BF16, TM, TN, 1>(w, x, qw, s, z, y, scratch, M, N, K, group, st);
    case 2: return launch_w4_wide<BF16, TM, TN, 2>(w, x, qw, s, z, y, scratch, M, N, K, group, st);
    case 4: return launch_w4_wide<BF16, TM, TN, 4>(w, x, qw, s, z, y, scratch, M, N, K, group, st);
    default: return launch_w4_wide<BF16, TM, TN, 8>(w, x, qw, s, z, y, scratch, M, N, K, group, st);
  }
}

template <bool BF16>
void dispatch_w4_wide(const W4Wide& w, const void* x, const int32_t* qw, const void* s,
                      const void* z, void* y, float* scratch, int M, int N, int K, int group,
                      hipStream_t st) {
  if (w.plan.tm == 256)
    dispatch_w4_wide_spg<BF16, 256, 256>(w, x, qw, s, z, y, scratch, M, N, K, group, st);
  else if (w.plan.tm == 64)
    dispatch_w4_wide_spg<BF16, 64, 256>(w, x, qw, s, z, y, scratch, M, N, K, group, st);
  else if (w.tn == 256)
    dispatch_w4_wide_spg<BF16, 128, 256>(w, x, qw, s, z, y, scratch, M, N, K, group, st);
  else
    dispatch_w4_wide_spg<BF16, 128, 128>(w, x, qw, s, z, y, scratch, M, N, K, group, st);
}

}  // namespace

// Bytes of device memory the path a call takes needs beyond its inputs and outputs: the wide
// kernel's split-K scratch, nothing for the LDS-staged kernel, or the decode kernel's split-K
// workspace (the dispatch order of kbh_w4a16_gemm).
size_t w4a16_path_bytes(int M, int N, int K, int group) {
  W4Wide w;
  if (plan_w4_wide(M, N, K, group, &w)) return wide_workspace_bytes(M, N, w.plan.splits);
  if (M >= kTiledMinM && K % (TBK * TDEPTH) == 0) return 0;
  DecodePlan p;
  if (!plan_decode(M, N, K, group / 32, &p)) return 0;
  return splitk_workspace_bytes(M, N, p.splits);
}

}  // namespace kbh

extern "C" size_t kbh_w4a16_workspace_bytes(int M, int N, int K, int group) {
  kbh::DecodePlan p;
  if (M < 1 || N < 128 || K < 32 || group < 32 || !kbh::plan_decode(M, N, K, group / 32, &p))
    return 0;
  return kbh::splitk_workspace_bytes(M, N, p.splits);
}

extern "C" size_t kbh_w4a16_scratch_bytes(int M, int N, int K, int group) {
  kbh::W4Wide w;
  if (M < 1 || N < 128 || K < 32 || group < 32 || !kbh::plan_w4_wide(M, N, K, group, &w)) return 0;
  return kbh::wide_workspace_bytes(M, N, w.plan.splits);
}

extern "C" int kbh_w4a16_gemm(const void* x, const int32_t* qweight, const void* scales,
                              const void* zeros, void* y, void* workspace, size_t workspace_bytes,
                              void* scratch, size_t scratch_bytes, int M, int N, int K, int group,
                              int dtype, void* stream) {
  using namespace kbh;
  if (!x || !qweight || !scales || !zeros || !y) return KBH_ERR_NULL;
  if (dtype != KBH_F16 && dtype != KBH_BF16) return KBH_ERR_DTYPE;
  if (M < 1 || N < 128 || K < 32 || (N % 128) != 0 || (K % 32) != 0) return KBH_ERR_SHAPE;
  if (group != 32 && group != 64 && group != 128 && group != 256) return KBH_ERR_SHAPE;
  if (K % group != 0) return KBH_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(qweight) || !aligned16(scales) || !aligned16(zeros) ||
      !aligned16(y))
    return KBH_ERR_ALIGN;
  const bool bf = dtype == KBH_BF16;
  hipStream_t st = (hipStream_t)stream;

  W4Wide wide;
  if (plan_w4_wide(M, N, K, group, &wide)) {
    const size_t need = wide_workspace_bytes(M, N, wide.plan.splits);
    if (need > 0 && (!scratch || scratch_bytes < need)) return KBH_ERR_WORKSPACE;
    if (need > 0 && !aligned16(scratch)) return KBH_ERR_ALIGN;
    if (bf) dispatch_w4_wide<true>(wide, x, qweight, scales, zeros, y, (float*)scratch, M, N, K, group, st);
    else dispatch_w4_wide<false>(wide, x, qweight, scales, zeros, y, (float*)scratch, M, N, K, group, st);
    return launch_status();
  }

  if (M >= kTiledMinM && K % (TBK * TDEPTH) == 0) {
    if (bf) {
      const W4SlabPolicy<true> bp{(const uint32_t*)qweight, (const uint16_t*)scales,
                                  (const uint16_t*)zeros, N, group, 0, 0};
      hipLaunchKernelGGL((tiled_f16_gemm<true, W4SlabPolicy<true>>), tiled_f16_grid(M, N),
                         dim3(256), 0, st, (const uint16_t*)x, bp, (uint16_t*)y, M, N, K);
    } else {
      const W4SlabPolicy<false> bp{(const uint32_t*)qweight, (const uint16_t*)scales,
                                   (const uint16_t*)zeros, N, group, 0, 0};
      hipLaunchKernelGGL((tiled_f16_gemm<false, W4SlabPolicy<false>>), tiled_f16_grid(M, N),
                         dim3(256), 0, st, (const uint16_t*)x, bp, (uint16_t*)y, M, N, K);
    }
    return launch_status();
  }

  DecodePlan p;
  if (!plan_decode(M, N, K, group / 32, &p)) return KBH_ERR_SHAPE;
  const size_t need = splitk_workspace_bytes(M, N, p.splits);
  if (need > 0 && (!workspace || workspace_bytes < need)) return KBH_ERR_WORKSPACE;
  if (need > 0 && !aligned16(workspace)) return KBH_ERR_ALIGN;
  float* acc = (float*)workspace;
  if (bf) dispatch_decode<true>(p, x, qweight, scales, zeros, y, acc, M, N, K, group, st);
  else dispatch_decode<false>(p, x, qweight, scales, zeros, y, acc, M, N, K, group, st);
  return launch_status();
}
