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
//    LDS slices; workgroups (K splits) reduce with fp32 atomics into a workspace tile, and the
//    last workgroup of a tile (per-tile arrival counter) converts it to the output dtype and
//    clears the workspace. Workgroup ids are remapped so that all K splits of a column tile run
//    on one XCD.
//
// w4a16_tiled_kernel (larger M; MFMA-bound)
//  * 256x128 output tile per 256-thread workgroup, K in 32-row slabs held in a register ring
//    three slabs ahead of the MFMAs, two LDS stages, one barrier per slab. x rows are staged in
//    LDS as is; packed weights are dequantized on the way into LDS with the exact
//    reference arithmetic ((q - z) in the input dtype, times s, one rounding), stored k-major
//    per column so that both MFMA operands are 16-byte LDS reads. 2x2 waves, each 128x64 with
//    32x32x16 MFMAs. XCD remapping gives each XCD whole rows of tiles (shared x rows in L2).
#include "kbh_common.h"

namespace kbh {
namespace {

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

// ======================================================================================
// Decode kernel
// ======================================================================================
constexpr int kDecodeMaxWaves = 8;
constexpr int kCsStride = 260;  // LDS floats per MFMA column set per wave (4*64 + pad)

// SPG = K steps per quantization group when a group is shorter than a wave's K range
// (SPG < SPW), otherwise SPG == SPW (each wave lies inside one group). The fold schedule is thus
// static, and the scales/zeros of every group a wave touches are loaded with its weights.
template <int NW, int SPW, int SPG, bool BF16>
__global__ __launch_bounds__(kDecodeMaxWaves * 64) void w4a16_decode_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ qw,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    uint16_t* __restrict__ y, float* __restrict__ acc, int* __restrict__ counters,
    int M, int N, int K, int group, int splits) {
  constexpr int NWG = 128 * NW;  // output columns of one workgroup
  constexpr int NCS = 8 * NW;    // MFMA column sets per wave
  constexpr uint32_t MAGIC = BF16 ? kMagicBF16 : kMagicF16;
  __shared__ float red[kDecodeMaxWaves * NCS * kCsStride];
  __shared__ int s_last;

  const int waves = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane & 15;
  const int g = lane >> 4;
  const int ntiles = N / NWG;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = id / splits;
  const int split = id - tile * splits;
  const int n0 = tile * NWG;
  const int m0 = blockIdx.y * 16;
  const int st0 = (split * waves + wave) * SPW;  // first 32-row K step of this wave
  const int NP = N >> 3;

  // ---- every load of this wave, up front -----------------------------------------------
  uint32_t wd[SPW][8][NW];
  kbh_u32x4 af[SPW];
  const uint32_t* qb = qw + (size_t)(st0 * 32 + 8 * g) * NP + (n0 >> 3) + c * NW;
#pragma unroll
  for (int u = 0; u < SPW; ++u) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t* p = qb + (size_t)(u * 32 + i) * NP;
      if constexpr (NW == 2) {
        const kbh_u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const kbh_u32x2*>(p));
        wd[u][i][0] = v[0];
        wd[u][i][1] = v[1];
      } else {
        wd[u][i][0] = __builtin_nontemporal_load(p);
      }
    }
  }
  const bool xok = m0 + c < M;
  const uint16_t* xb = x + (size_t)(xok ? m0 + c : 0) * K + st0 * 32 + 8 * g;
#pragma unroll
  for (int u = 0; u < SPW; ++u) {
    const kbh_u32x4 v = *reinterpret_cast<const kbh_u32x4*>(xb + u * 32);
    af[u] = xok ? v : kbh_u32x4{0u, 0u, 0u, 0u};
  }
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

  const uint32_t one = BF16 ? kOneBF16 : kOneF16;
  const kbh_u32x4 ones = {one, one, one, one};
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
          blo[p] = (P & 0x000F000Fu) | MAGIC;
          bhi[p] = BF16 ? (((P >> 4) & 0x000F000Fu) | MAGIC) : ((P & 0x00F000F0u) | MAGIC);
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

  // ---- reduce the waves of the workgroup through private LDS slices -----------------------
  // Slice element (column set cs, row 4*(l/16)+i, lane column l%16) at cs*kCsStride + i*64 + l.
  {
    float* slice = red + wave * NCS * kCsStride;
#pragma unroll
    for (int cs = 0; cs < NCS; ++cs)
#pragma unroll
      for (int i = 0; i < 4; ++i) slice[cs * kCsStride + i * 64 + lane] = tot[cs][i];
  }
  __syncthreads();
  // Output element (r, n), n = 8*(cc*NW + w) + nib, is the sum over waves of slice entry
  // (cs = w*8 + nib, i = r%4, lane = (r/4)*16 + cc).
  auto lds_sum = [&](int r, int n) {
    const int cc = n / (8 * NW), w = (n >> 3) % NW, nib = n & 7;
    const int off = (w * 8 + nib) * kCsStride + (r & 3) * 64 + (r >> 2) * 16 + cc;
    float v = 0.f;
    for (int wv = 0; wv < waves; ++wv) v += red[wv * NCS * kCsStride + off];
    return v;
  };
  const int rows = min(16, M - m0);
  if (splits == 1) {
    for (int e = threadIdx.x; e < rows * NWG; e += blockDim.x) {
      const int r = e / NWG, n = e - r * NWG;
      y[(size_t)(m0 + r) * N + n0 + n] = f32_to_half_bits<BF16>(lds_sum(r, n));
    }
    return;
  }
  // ---- cross-workgroup reduction --------------------------------------------------------
  // All cross-workgroup traffic uses agent-scope atomics, which are performed at the device
  // coherence point. Each thread waits until its atomics are acknowledged (s_waitcnt 0) before
  // the workgroup's arrival is counted, so the workgroup that sees count == splits-1 reads
  // complete sums with agent-scope atomic loads.
  for (int e = threadIdx.x; e < rows * NWG; e += blockDim.x) {
    const int r = e / NWG, n = e - r * NWG;
    __hip_atomic_fetch_add(&acc[(size_t)(m0 + r) * N + n0 + n], lds_sum(r, n), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int* counter = &counters[blockIdx.y * ntiles + tile];
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == splits - 1);
  }
  __syncthreads();
  if (!s_last) return;
  for (int e = threadIdx.x; e < rows * NWG; e += blockDim.x) {
    const int r = e / NWG, n = e - r * NWG;
    float* p = &acc[(size_t)(m0 + r) * N + n0 + n];
    const float v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p, 0.f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    y[(size_t)(m0 + r) * N + n0 + n] = f32_to_half_bits<BF16>(v);
  }
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct DecodePlan {
  int nw, spw, spg, waves, ntiles, splits, mblocks;
};

// Chooses column width (NW), K steps per wave (SPW) and waves per workgroup so that the K steps
// divide evenly and the grid is close to one workgroup per CU (256).
bool plan_decode(int M, int N, int K, int group_steps_, DecodePlan* p) {
  const int nsteps = K / 32;
  p->nw = (N % 256 == 0) ? 2 : 1;
  p->ntiles = N / (128 * p->nw);
  p->mblocks = (M + 15) / 16;
  p->spw = (nsteps % 4 == 0) ? 4 : (nsteps % 2 == 0 ? 2 : 1);
  // Wave ranges start at multiples of SPW steps, so they stay inside one group when the group
  // spans a multiple of SPW steps; otherwise the group (1 or 2 steps) divides SPW.
  const int gsteps = group_steps_;
  p->spg = (gsteps % p->spw == 0) ? p->spw : gsteps;
  const int units = nsteps / p->spw;  // wave-sized K units per column tile
  int best_w = -1, best_score = 1 << 30;
  for (int w = kDecodeMaxWaves; w >= 1; --w) {
    if (units % w) continue;
    const int grid = p->ntiles * (units / w) * p->mblocks;
    // Prefer grids of 256..512 workgroups; penalise tiny or huge grids.
    const int score = grid < 256 ? (256 - grid) * 4 : (grid > 512 ? grid - 512 : 0) + (8 - w);
    if (score < best_score) { best_score = score; best_w = w; }
  }
  if (best_w < 0) return false;
  p->waves = best_w;
  p->splits = units / best_w;
  return true;
}

template <int NW, int SPW, int SPG, bool BF16>
void launch_decode(const DecodePlan& p, const void* x, const int32_t* qw, const void* s,
                   const void* z, void* y, float* acc, int* counters, int M, int N, int K,
                   int group, hipStream_t stream) {
  dim3 grid(p.ntiles * p.splits, p.mblocks);
  hipLaunchKernelGGL((w4a16_decode_kernel<NW, SPW, SPG, BF16>), grid, dim3(p.waves * 64), 0, stream,
                     (const uint16_t*)x, (const uint32_t*)qw, (const uint16_t*)s,
                     (const uint16_t*)z, (uint16_t*)y, acc, counters, M, N, K, group, p.splits);
}

template <bool BF16>
void dispatch_decode(const DecodePlan& p, const void* x, const int32_t* qw, const void* s,
                     const void* z, void* y, float* acc, int* counters, int M, int N, int K,
                     int group, hipStream_t st) {
#define KBH_DEC(NW_, SPW_, SPG_)                                                                 \
  if (p.nw == NW_ && p.spw == SPW_ && p.spg == SPG_)                                             \
    return launch_decode<NW_, SPW_, SPG_, BF16>(p, x, qw, s, z, y, acc, counters, M, N, K, group, st);
  KBH_DEC(2, 4, 4) KBH_DEC(2, 4, 2) KBH_DEC(2, 4, 1) KBH_DEC(2, 2, 2) KBH_DEC(2, 2, 1)
  KBH_DEC(2, 1, 1) KBH_DEC(1, 4, 4) KBH_DEC(1, 4, 2) KBH_DEC(1, 4, 1) KBH_DEC(1, 2, 2)
  KBH_DEC(1, 2, 1) KBH_DEC(1, 1, 1)
#undef KBH_DEC
}

// ======================================================================================
// Tiled kernel
// ======================================================================================
constexpr int TBM = 256, TBN = 128, TBK = 32;
constexpr int TLD = TBK + 8;  // LDS row stride in 16-bit elements (80 B: conflict-free b128)
constexpr int TDEPTH = 4;     // K slabs in flight in registers ahead of the MFMAs

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

// One K slab of one thread, held in registers between its global load and its LDS store.
struct TiledSlab {
  kbh_u32x4 a[4];   // x: rows t/4 + 64i, 16-byte chunk t%4 of the slab
  uint32_t b[2];    // qweight rows 2*(t%16), +1 of the slab, word column t/16
  kbh_u32x4 s, z;   // scales / zeros of columns 8*(t/16) .. +7 for the slab's group
};

template <bool BF16>
__global__ __launch_bounds__(256) void w4a16_tiled_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ qw,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    uint16_t* __restrict__ y, int M, int N, int K, int group) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][TBM * TLD];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][TBN * TLD];

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int ntn = N / TBN;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int mb = id / ntn, nb = id - mb * ntn;
  const int m0 = mb * TBM, n0 = nb * TBN;
  const int NP = N >> 3;
  const int KT = K / TBK;

  const int a_ch = t & 3, a_row = t >> 2;
  const int b_kp = t & 15, b_wc = t >> 4;
  const uint16_t* xrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = m0 + a_row + 64 * i;
    xrow[i] = x + (size_t)(r < M ? r : M - 1) * K + a_ch * 8;  // rows >= M are never stored
  }
  const uint32_t* qcol = qw + (size_t)(2 * b_kp) * NP + (n0 >> 3) + b_wc;
  const size_t scol = (size_t)n0 + 8 * b_wc;

  auto load = [&](TiledSlab& sl, int kt) {
    const int k0 = kt * TBK;
#pragma unroll
    for (int i = 0; i < 4; ++i) sl.a[i] = *reinterpret_cast<const kbh_u32x4*>(xrow[i] + k0);
    const uint32_t* q = qcol + (size_t)k0 * NP;
    sl.b[0] = __builtin_nontemporal_load(q);
    sl.b[1] = __builtin_nontemporal_load(q + NP);
    const size_t off = (size_t)(k0 / group) * N + scol;
    sl.s = *reinterpret_cast<const kbh_u32x4*>(scales + off);
    sl.z = *reinterpret_cast<const kbh_u32x4*>(zeros + off);
  };
  auto store_a = [&](const TiledSlab& sl, int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<kbh_u32x4*>(&As[buf][(a_row + 64 * i) * TLD + a_ch * 8]) = sl.a[i];
  };
  auto store_b = [&](const TiledSlab& sl, int buf) {
    uint32_t dq[8];
    dequant_2x8<BF16>(sl.b[0], sl.b[1], sl.s, sl.z, dq);
#pragma unroll
    for (int c = 0; c < 8; ++c)
      *reinterpret_cast<uint32_t*>(&Bs[buf][(b_wc * 8 + c) * TLD + 2 * b_kp]) = dq[c];
  };
  auto store = [&](const TiledSlab& sl, int buf) {
    store_a(sl, buf);
    store_b(sl, buf);
  };

  kbh_f32x16 accv[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) accv[i][j][e] = 0.f;

  const int fr = lane & 31, fk = (lane >> 5) * 8;
  // One 16-wide K step of the wave's 128x64 tile: 6 LDS fragment reads, 8 MFMAs.
  auto mma_k16 = [&](int buf, int kk) {
    const uint16_t* Ab = &As[buf][(wm * 128 + fr) * TLD + fk + kk * 16];
    const uint16_t* Bb = &Bs[buf][(wn * 64 + fr) * TLD + fk + kk * 16];
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

  // Register ring: slab j lives in stage j % TDEPTH from its load until its LDS store. KT is a
  // multiple of TDEPTH and loads past the last slab re-read it, so the steady-state loop has no
  // branches (a conditional load would make the compiler wait for every load in flight).
  TiledSlab ring[TDEPTH];
#pragma unroll
  for (int d = 0; d < TDEPTH; ++d) load(ring[d], d);
  store(ring[0], 0);
  load(ring[0], min(TDEPTH, KT - 1));
  __syncthreads();

  for (int kt0 = 0; kt0 < KT; kt0 += TDEPTH) {
#pragma unroll
    for (int d = 0; d < TDEPTH; ++d) {
      const int kt = kt0 + d;
      const int nxt = (d + 1) % TDEPTH;      // stage of slab kt+1
      // The MFMAs of slab kt run asynchronously while the wave stages slab kt+1 (x copy,
      // dequantization) into the other LDS buffer; after the last slab that buffer is unused.
      mma_k16(kt & 1, 0);
      store_a(ring[nxt], (kt + 1) & 1);
      mma_k16(kt & 1, 1);
      store_b(ring[nxt], (kt + 1) & 1);
      load(ring[nxt], min(kt + 1 + TDEPTH, KT - 1));
      __syncthreads();
    }
  }

  // epilogue: accumulator element e of tile (i, j) is row 8(e/4) + 4(l/32) + e%4, column l%32
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

// The tiled kernel beats the split-K decode kernel once the 256-row tiles are reasonably full.
constexpr int kTiledMinM = 128;

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
  if (M < 1 || N < 128 || K < 32 || (N % 128) != 0 || (K % 32) != 0) return KBH_ERR_SHAPE;
  if (group != 32 && group != 64 && group != 128 && group != 256) return KBH_ERR_SHAPE;
  if (K % group != 0) return KBH_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(qweight) || !aligned16(scales) || !aligned16(zeros) ||
      !aligned16(y))
    return KBH_ERR_ALIGN;
  const bool bf = dtype == KBH_BF16;
  hipStream_t st = (hipStream_t)stream;

  if (M >= kTiledMinM && K % (TBK * TDEPTH) == 0) {
    const int tiles = ((M + TBM - 1) / TBM) * (N / TBN);
    if (bf)
      hipLaunchKernelGGL(w4a16_tiled_kernel<true>, dim3(tiles), dim3(256), 0, st,
                         (const uint16_t*)x, (const uint32_t*)qweight, (const uint16_t*)scales,
                         (const uint16_t*)zeros, (uint16_t*)y, M, N, K, group);
    else
      hipLaunchKernelGGL(w4a16_tiled_kernel<false>, dim3(tiles), dim3(256), 0, st,
                         (const uint16_t*)x, (const uint32_t*)qweight, (const uint16_t*)scales,
                         (const uint16_t*)zeros, (uint16_t*)y, M, N, K, group);
    return launch_status();
  }

  const size_t need = kbh_w4a16_workspace_bytes(M, N, K, group);
  if (!workspace || workspace_bytes < need) return KBH_ERR_WORKSPACE;
  float* acc = (float*)workspace;
  int* counters = (int*)((char*)workspace + round_up((size_t)M * (size_t)N * 4u, 256));
  DecodePlan p;
  if (!plan_decode(M, N, K, group / 32, &p)) return KBH_ERR_SHAPE;
  if (bf) dispatch_decode<true>(p, x, qweight, scales, zeros, y, acc, counters, M, N, K, group, st);
  else dispatch_decode<false>(p, x, qweight, scales, zeros, y, acc, counters, M, N, K, group, st);
  return launch_status();
}
