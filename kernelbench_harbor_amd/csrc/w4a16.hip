// W4A16 packed-asymmetric group-quantized GEMM for gfx950.
//
// Semantics (reference tasks/quant_w4a16_pa/*/environment/reference.py:10-17):
//   w[k, n] = ((qweight[k, n/8] >> 4*(n%8)) & 0xF - zeros[k/G, n]) * scales[k/G, n]
//   y       = x @ w
//
// Kernel design (split-K, all M; tuned for the HBM-bound decode shapes M <= 32):
//  * One wavefront owns 128*NW output columns. Lane l reads, per 32-row K step, the packed words
//    qweight[k0 + 8(l/16) + i][n0/8 + (l%16)*NW + w], i = 0..7, w < NW (NW consecutive words per
//    row, so 16 lanes cover 64*NW contiguous bytes of a row).
//  * The nibbles are turned into fp16/bf16 MFMA B-fragments without any per-weight arithmetic:
//    one v_perm_b32 places byte j of two words of rows k, k+1 into the two 16-bit halves, and one
//    v_and_or_b32 with a magic exponent turns a nibble q into the value B+q (fp16: 1024+q, or
//    1024+16q for the high nibble; bf16: 128+q). Each (word, nibble) pair is one 16x16x32 MFMA
//    whose 16 columns are 8*NW apart in n; the epilogue undoes that permutation.
//  * Zero points and scales are applied once per quantization group on the fp32 accumulators:
//      sum_k x_k (q_k - z) s = s * (sum_k x_k (B + f q_k) / f - (B/f + z) * sum_k x_k)
//    with sum_k x_k from one extra MFMA against a ones fragment.
//  * Workgroups split K; partial tiles are reduced in LDS across the waves of a workgroup, then
//    with fp32 atomics into a workspace; the last workgroup of a tile (atomic counter) converts
//    the tile to the output dtype and clears the workspace. Workgroup ids are remapped so that
//    all K-splits of a column tile run on the same XCD.
#include "kbh_common.h"

namespace kbh {
namespace {

constexpr uint32_t kMagicF16 = 0x64006400u;   // fp16 1024.0 in both halves
constexpr uint32_t kMagicBF16 = 0x43004300u;  // bf16 128.0 in both halves
constexpr uint32_t kOneF16 = 0x3c003c00u;
constexpr uint32_t kOneBF16 = 0x3f803f80u;

// Byte j of word wa (row k) to bits 0..7 and byte j of word wb (row k+1) to bits 16..23; the
// other bytes are zero. v_perm_b32 numbers the bytes of {src0, src1} as src1 = 0..3, src0 = 4..7
// and selector value 0x0c yields 0x00.
template <int J>
__device__ inline uint32_t pair_bytes(uint32_t wa, uint32_t wb) {
  constexpr uint32_t sel = 0x0c000c00u | ((4u + J) << 16) | (uint32_t)J;
  return __builtin_amdgcn_perm(wb, wa, sel);
}

template <int NW, int MT, int WAVES, int U, bool BF16>
__global__ __launch_bounds__(WAVES * 64) void w4a16_splitk_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ qw,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    uint16_t* __restrict__ y, float* __restrict__ acc, int* __restrict__ counters,
    int M, int N, int K, int group, int splits, int steps_per_split) {
  constexpr int NWG = 128 * NW;  // output columns of one workgroup
  constexpr int NCS = 8 * NW;    // MFMA column sets per 16-row tile
  constexpr int LDS_STRIDE = NWG + 4;
  constexpr uint32_t MAGIC = BF16 ? kMagicBF16 : kMagicF16;
  __shared__ float red[MT * 16 * LDS_STRIDE];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane & 15;
  const int g = lane >> 4;

  const int ntiles = N / NWG;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = id / splits;
  const int split = id - tile * splits;
  const int n0 = tile * NWG;
  const int m0 = blockIdx.y * (16 * MT);

  const int nsteps = K >> 5;
  const int sb = split * steps_per_split;
  const int se = min(sb + steps_per_split, nsteps);
  const int per_wave = (se - sb + WAVES - 1) / WAVES;
  const int wb = min(sb + wave * per_wave, se);
  const int we = min(wb + per_wave, se);

  const int NP = N >> 3;
  const uint32_t* qbase = qw + (n0 >> 3) + c * NW;
  const int steps_per_group = group >> 5;

  kbh_f32x4 tot[MT][NCS], part[MT][NCS], xs[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    xs[mt] = kbh_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cs = 0; cs < NCS; ++cs) {
      tot[mt][cs] = kbh_f32x4{0.f, 0.f, 0.f, 0.f};
      part[mt][cs] = kbh_f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  const uint16_t* xrow[MT];
  bool xok[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = m0 + mt * 16 + c;
    xok[mt] = r < M;
    xrow[mt] = x + (size_t)(xok[mt] ? r : 0) * K + 8 * g;
  }
  const uint32_t one = BF16 ? kOneBF16 : kOneF16;
  const kbh_u32x4 ones = {one, one, one, one};

  for (int s0 = wb; s0 < we; s0 += U) {
    uint32_t wd[U][8][NW];
    kbh_u32x4 af[U][MT];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int st = s0 + u;
      if (st < we) {
        const int kb = st << 5;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t* p = qbase + (size_t)(kb + 8 * g + i) * NP;
          if constexpr (NW == 2) {
            kbh_u32x2 v = *reinterpret_cast<const kbh_u32x2*>(p);
            wd[u][i][0] = v[0];
            wd[u][i][1] = v[1];
          } else {
#pragma unroll
            for (int w = 0; w < NW; ++w) wd[u][i][w] = p[w];
          }
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          af[u][mt] = xok[mt] ? *reinterpret_cast<const kbh_u32x4*>(xrow[mt] + kb)
                              : kbh_u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int st = s0 + u;
      if (st < we) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) xs[mt] = mfma16x16x32<BF16>(af[u][mt], ones, xs[mt]);
#pragma unroll
        for (int w = 0; w < NW; ++w) {
#define KBH_W4_BYTE(J)                                                                    \
  {                                                                                       \
    kbh_u32x4 blo, bhi;                                                                   \
    _Pragma("unroll") for (int p = 0; p < 4; ++p) {                                       \
      const uint32_t P = pair_bytes<J>(wd[u][2 * p][w], wd[u][2 * p + 1][w]);             \
      blo[p] = (P & 0x000F000Fu) | MAGIC;                                                 \
      bhi[p] = BF16 ? (((P >> 4) & 0x000F000Fu) | MAGIC) : ((P & 0x00F000F0u) | MAGIC);   \
    }                                                                                     \
    _Pragma("unroll") for (int mt = 0; mt < MT; ++mt) {                                   \
      part[mt][w * 8 + 2 * J] = mfma16x16x32<BF16>(af[u][mt], blo, part[mt][w * 8 + 2 * J]); \
      part[mt][w * 8 + 2 * J + 1] =                                                       \
          mfma16x16x32<BF16>(af[u][mt], bhi, part[mt][w * 8 + 2 * J + 1]);                \
    }                                                                                     \
  }
          KBH_W4_BYTE(0)
          KBH_W4_BYTE(1)
          KBH_W4_BYTE(2)
          KBH_W4_BYTE(3)
#undef KBH_W4_BYTE
        }
        // Fold the group's partial sums at the end of a quantization group or of this wave's range.
        if (((st + 1) % steps_per_group) == 0 || st + 1 == we) {
          const int gi = (st << 5) / group;
#pragma unroll
          for (int w = 0; w < NW; ++w) {
            const size_t off = (size_t)gi * N + n0 + 8 * (c * NW + w);
            const kbh_u32x4 sv = *reinterpret_cast<const kbh_u32x4*>(scales + off);
            const kbh_u32x4 zv = *reinterpret_cast<const kbh_u32x4*>(zeros + off);
#pragma unroll
            for (int nib = 0; nib < 8; ++nib) {
              const uint16_t sh = (uint16_t)((nib & 1) ? (sv[nib >> 1] >> 16) : (sv[nib >> 1] & 0xffffu));
              const uint16_t zh = (uint16_t)((nib & 1) ? (zv[nib >> 1] >> 16) : (zv[nib >> 1] & 0xffffu));
              const float s = half_bits_to_f32<BF16>(sh);
              const float z = half_bits_to_f32<BF16>(zh);
              const float a = (!BF16 && (nib & 1)) ? 0.0625f : 1.0f;
              const float bz = (BF16 ? 128.0f : ((nib & 1) ? 64.0f : 1024.0f)) + z;
#pragma unroll
              for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                  const float t = fmaf(-bz, xs[mt][i], part[mt][w * 8 + nib][i] * a);
                  tot[mt][w * 8 + nib][i] = fmaf(s, t, tot[mt][w * 8 + nib][i]);
                }
                part[mt][w * 8 + nib] = kbh_f32x4{0.f, 0.f, 0.f, 0.f};
              }
            }
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) xs[mt] = kbh_f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
  }

  // ---- reduce the waves of this workgroup in LDS -------------------------------------------
  // LDS tile element (row r, column n) with n = 8*(c*NW + w) + nib lives at
  // r*LDS_STRIDE + (w*8 + nib)*16 + c (lane-contiguous writes, conflict free).
  for (int e = threadIdx.x; e < MT * 16 * LDS_STRIDE; e += WAVES * 64) red[e] = 0.f;
  __syncthreads();
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int cs = 0; cs < NCS; ++cs)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = mt * 16 + 4 * g + i;
        atomicAdd(&red[r * LDS_STRIDE + cs * 16 + c], tot[mt][cs][i]);
      }
  __syncthreads();

  const int rows = min(16 * MT, M - m0);
  if (splits == 1) {
    for (int e = threadIdx.x; e < rows * NWG; e += WAVES * 64) {
      const int r = e / NWG, n = e - r * NWG;
      const int cc = n / (8 * NW), w = (n >> 3) % NW, nib = n & 7;
      const float v = red[r * LDS_STRIDE + (w * 8 + nib) * 16 + cc];
      y[(size_t)(m0 + r) * N + n0 + n] = f32_to_half_bits<BF16>(v);
    }
    return;
  }
  for (int e = threadIdx.x; e < rows * NWG; e += WAVES * 64) {
    const int r = e / NWG, n = e - r * NWG;
    const int cc = n / (8 * NW), w = (n >> 3) % NW, nib = n & 7;
    const float v = red[r * LDS_STRIDE + (w * 8 + nib) * 16 + cc];
    unsafeAtomicAdd(&acc[(size_t)(m0 + r) * N + n0 + n], v);
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = atomicAdd(&counters[blockIdx.y * ntiles + tile], 1);
    s_last = (prev == splits - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  for (int e = threadIdx.x; e < rows * NWG; e += WAVES * 64) {
    const int r = e / NWG, n = e - r * NWG;
    float* p = &acc[(size_t)(m0 + r) * N + n0 + n];
    const float v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p, 0.f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    y[(size_t)(m0 + r) * N + n0 + n] = f32_to_half_bits<BF16>(v);
  }
  if (threadIdx.x == 0) {
    __hip_atomic_store(&counters[blockIdx.y * ntiles + tile], 0, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
}

struct SplitKPlan {
  int nw, mt, ntiles, mblocks, splits, steps_per_split;
};

SplitKPlan plan_splitk(int M, int N, int K) {
  SplitKPlan p;
  // Two 16-row tiles with 256 columns per wave exceed the register file, so M > 16 uses
  // 128-column waves.
  p.mt = (M <= 16) ? 1 : 2;
  p.nw = (N % 256 == 0 && p.mt == 1) ? 2 : 1;
  p.ntiles = N / (128 * p.nw);
  p.mblocks = (M + 16 * p.mt - 1) / (16 * p.mt);
  const int nsteps = K / 32;
  const int base = p.ntiles * p.mblocks;
  int splits = (256 + base - 1) / base;
  if (splits < 1) splits = 1;
  if (splits > nsteps) splits = nsteps;
  p.steps_per_split = (nsteps + splits - 1) / splits;
  p.splits = (nsteps + p.steps_per_split - 1) / p.steps_per_split;
  return p;
}

template <int NW, int MT, bool BF16>
void launch_splitk(const SplitKPlan& p, const void* x, const int32_t* qw, const void* s,
                   const void* z, void* y, float* acc, int* counters, int M, int N, int K, int group,
                   hipStream_t stream) {
  constexpr int WAVES = 4;
  constexpr int U = 4;
  dim3 grid(p.ntiles * p.splits, p.mblocks);
  hipLaunchKernelGGL((w4a16_splitk_kernel<NW, MT, WAVES, U, BF16>), grid, dim3(WAVES * 64), 0,
                     stream, (const uint16_t*)x, (const uint32_t*)qw, (const uint16_t*)s,
                     (const uint16_t*)z, (uint16_t*)y, acc, counters, M, N, K, group, p.splits,
                     p.steps_per_split);
}

}  // namespace
}  // namespace kbh

extern "C" size_t kbh_w4a16_workspace_bytes(int M, int N, int K, int group) {
  (void)K;
  (void)group;
  if (M <= 0 || N <= 0) return 0;
  const size_t acc = kbh::round_up((size_t)M * (size_t)N * 4u, 256);
  const size_t cnt = kbh::round_up((size_t)((M + 15) / 16) * (size_t)(N / 128 + 1) * 4u, 256);
  return acc + cnt;
}

extern "C" int kbh_w4a16_gemm(const void* x, const int32_t* qweight, const void* scales,
                              const void* zeros, void* y, void* workspace, size_t workspace_bytes,
                              int M, int N, int K, int group, int dtype, void* stream) {
  using namespace kbh;
  if (!x || !qweight || !scales || !zeros || !y) return KBH_ERR_NULL;
  if (dtype != KBH_F16 && dtype != KBH_BF16) return KBH_ERR_DTYPE;
  if (M < 1 || N < 128 || K < 32 || (N % 128) != 0) return KBH_ERR_SHAPE;
  if (group != 32 && group != 64 && group != 128 && group != 256) return KBH_ERR_SHAPE;
  if (K % group != 0) return KBH_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(qweight) || !aligned16(scales) || !aligned16(zeros) ||
      !aligned16(y))
    return KBH_ERR_ALIGN;
  const size_t need = kbh_w4a16_workspace_bytes(M, N, K, group);
  if (!workspace || workspace_bytes < need) return KBH_ERR_WORKSPACE;
  float* acc = (float*)workspace;
  int* counters = (int*)((char*)workspace + round_up((size_t)M * (size_t)N * 4u, 256));
  hipStream_t st = (hipStream_t)stream;

  const SplitKPlan p = plan_splitk(M, N, K);
  const bool bf = dtype == KBH_BF16;
#define KBH_W4_LAUNCH(NW, MT)                                                                    \
  if (p.nw == NW && p.mt == MT) {                                                                \
    if (bf) launch_splitk<NW, MT, true>(p, x, qweight, scales, zeros, y, acc, counters, M, N, K, \
                                        group, st);                                              \
    else launch_splitk<NW, MT, false>(p, x, qweight, scales, zeros, y, acc, counters, M, N, K,   \
                                      group, st);                                                \
    return launch_status();                                                                      \
  }
  KBH_W4_LAUNCH(2, 1)
  KBH_W4_LAUNCH(1, 1)
  KBH_W4_LAUNCH(1, 2)
#undef KBH_W4_LAUNCH
  return KBH_ERR_SHAPE;
}
