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
//  * 256x128 output tile per 256-thread workgroup, K in 64-row slabs, two LDS stages. x rows are
//    staged in LDS as is; packed weights are dequantized on the way into LDS with the exact
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

template <int NW, int SPW, bool BF16>
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

  const uint32_t one = BF16 ? kOneBF16 : kOneF16;
  const kbh_u32x4 ones = {one, one, one, one};
  kbh_f32x4 tot[NCS], part[NCS], xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int cs = 0; cs < NCS; ++cs) {
    tot[cs] = kbh_f32x4{0.f, 0.f, 0.f, 0.f};
    part[cs] = tot[cs];
  }
  const int spg = group >> 5;
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
    const int st = st0 + u;
    // Fold at the end of a quantization group or of this wave's K range.
    if (((st + 1) % spg) == 0 || u == SPW - 1) {
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
  int nw, spw, waves, ntiles, splits, mblocks;
};

// Chooses column width (NW), K steps per wave (SPW) and waves per workgroup so that the K steps
// divide evenly and the grid is close to one workgroup per CU (256).
bool plan_decode(int M, int N, int K, DecodePlan* p) {
  const int nsteps = K / 32;
  p->nw = (N % 256 == 0) ? 2 : 1;
  p->ntiles = N / (128 * p->nw);
  p->mblocks = (M + 15) / 16;
  p->spw = (nsteps % 4 == 0) ? 4 : (nsteps % 2 == 0 ? 2 : 1);
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

template <int NW, int SPW, bool BF16>
void launch_decode(const DecodePlan& p, const void* x, const int32_t* qw, const void* s,
                   const void* z, void* y, float* acc, int* counters, int M, int N, int K,
                   int group, hipStream_t stream) {
  dim3 grid(p.ntiles * p.splits, p.mblocks);
  hipLaunchKernelGGL((w4a16_decode_kernel<NW, SPW, BF16>), grid, dim3(p.waves * 64), 0, stream,
                     (const uint16_t*)x, (const uint32_t*)qw, (const uint16_t*)s,
                     (const uint16_t*)z, (uint16_t*)y, acc, counters, M, N, K, group, p.splits);
}

template <bool BF16>
void dispatch_decode(const DecodePlan& p, const void* x, const int32_t* qw, const void* s,
                     const void* z, void* y, float* acc, int* counters, int M, int N, int K,
                     int group, hipStream_t st) {
#define KBH_DEC(NW_, SPW_)                                                                       \
  if (p.nw == NW_ && p.spw == SPW_)                                                              \
    return launch_decode<NW_, SPW_, BF16>(p, x, qw, s, z, y, acc, counters, M, N, K, group, st);
  KBH_DEC(2, 4) KBH_DEC(2, 2) KBH_DEC(2, 1) KBH_DEC(1, 4) KBH_DEC(1, 2) KBH_DEC(1, 1)
#undef KBH_DEC
}

// ======================================================================================
// Tiled kernel
// ======================================================================================
constexpr int TBM = 256, TBN = 128, TBK = 64;
constexpr int TLD = TBK + 8;  // LDS row stride in 16-bit elements (144 B: conflict-free b128)

// Dequantizes one thread's 4 rows x 8 columns and stores them k-major per column.
// w[4] are the packed words of rows k..k+3 (same word column); result column c (0..7) gets
// halves for k..k+3 as two dwords.
template <bool BF16>
__device__ inline void dequant_4x8(const uint32_t w[4], kbh_u32x4 sv, kbh_u32x4 zv,
                                   uint32_t out[8][2]) {
  constexpr uint32_t MAGIC = BF16 ? kMagicBF16 : kMagicF16;
#pragma unroll
  for (int pr = 0; pr < 2; ++pr) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t P = pair_bytes_rt(w[2 * pr], w[2 * pr + 1], j);
      const uint32_t hl = (P & 0x000F000Fu) | MAGIC;          // column 2j   at rows (k, k+1)
      const uint32_t hh = ((P >> 4) & 0x000F000Fu) | MAGIC;   // column 2j+1 at rows (k, k+1)
#pragma unroll
      for (int hsel = 0; hsel < 2; ++hsel) {
        const int col = 2 * j + hsel;
        const uint32_t h = hsel ? hh : hl;
        const uint16_t sb = (uint16_t)((col & 1) ? (sv[col >> 1] >> 16) : (sv[col >> 1] & 0xffffu));
        const uint16_t zb = (uint16_t)((col & 1) ? (zv[col >> 1] >> 16) : (zv[col >> 1] & 0xffffu));
        uint32_t r;
        if constexpr (BF16) {
          // (B+q) - (B+z) is exact in fp32; times s is exact in fp32 (8+5 bit significands);
          // one rounding to bf16.
          const float s = bf16_bits_to_f32(sb);
          const float bz = 128.0f + bf16_bits_to_f32(zb);
          const float lo = (bf16_bits_to_f32((uint16_t)(h & 0xffffu)) - bz) * s;
          const float hi = (bf16_bits_to_f32((uint16_t)(h >> 16)) - bz) * s;
          r = (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
        } else {
          typedef _Float16 h2 __attribute__((ext_vector_type(2)));
          const _Float16 s = __builtin_bit_cast(_Float16, sb);
          const _Float16 bz = (_Float16)1024.0f + __builtin_bit_cast(_Float16, zb);
          const h2 hv = __builtin_bit_cast(h2, h);
          const h2 d = hv - h2{bz, bz};  // q - z, exact
          const h2 wv = d * h2{s, s};     // one rounding, as the reference's fp16 multiply
          r = __builtin_bit_cast(uint32_t, wv);
        }
        out[col][pr] = r;
      }
    }
  }
}

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

  // global -> register mapping
  // A: rows t/8 + 32i (i < 8), 16-byte chunk t%8 of the 64-column slab.
  const int a_row = t >> 3, a_ch = t & 7;
  // B: rows 4*(t%16) .. +3 of the slab, packed word column t/16 (columns 8*(t/16) .. +7).
  const int b_kq = t & 15, b_wc = t >> 4;

  kbh_u32x4 ar[8];
  uint32_t br[4];
  kbh_u32x4 sv, zv;

  auto load_tile = [&](int kt) {
    const int k0 = kt * TBK;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = m0 + a_row + 32 * i;
      const bool ok = r < M;
      const kbh_u32x4 v = *reinterpret_cast<const kbh_u32x4*>(x + (size_t)(ok ? r : 0) * K + k0 + a_ch * 8);
      ar[i] = ok ? v : kbh_u32x4{0u, 0u, 0u, 0u};
    }
    const uint32_t* qp = qw + (size_t)(k0 + 4 * b_kq) * NP + (n0 >> 3) + b_wc;
#pragma unroll
    for (int r = 0; r < 4; ++r) br[r] = qp[(size_t)r * NP];
    const int gi = (k0 + 4 * b_kq) / group;
    const size_t off = (size_t)gi * N + n0 + 8 * b_wc;
    sv = *reinterpret_cast<const kbh_u32x4*>(scales + off);
    zv = *reinterpret_cast<const kbh_u32x4*>(zeros + off);
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      *reinterpret_cast<kbh_u32x4*>(&As[buf][(a_row + 32 * i) * TLD + a_ch * 8]) = ar[i];
    uint32_t dq[8][2];
    dequant_4x8<BF16>(br, sv, zv, dq);
#pragma unroll
    for (int c = 0; c < 8; ++c)
      *reinterpret_cast<kbh_u32x2*>(&Bs[buf][(b_wc * 8 + c) * TLD + 4 * b_kq]) = kbh_u32x2{dq[c][0], dq[c][1]};
  };

  kbh_f32x16 accv[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) accv[i][j][e] = 0.f;

  const int KT = K / TBK;
  load_tile(0);
  store_tile(0);
  __syncthreads();
  const int fr = lane & 31, fk = (lane >> 5) * 8;
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) load_tile(kt + 1);
    const uint16_t* Ab = &As[buf][(wm * 128 + fr) * TLD + fk];
    const uint16_t* Bb = &Bs[buf][(wn * 64 + fr) * TLD + fk];
#pragma unroll
    for (int kk = 0; kk < TBK / 16; ++kk) {
      kbh_u32x4 a[4], b[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const kbh_u32x4*>(Ab + i * 32 * TLD + kk * 16);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = *reinterpret_cast<const kbh_u32x4*>(Bb + j * 32 * TLD + kk * 16);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) accv[i][j] = mfma32x32x16<BF16>(a[i], b[j], accv[i][j]);
    }
    if (kt + 1 < KT) store_tile(buf ^ 1);
    __syncthreads();
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

  if (M >= kTiledMinM && K % TBK == 0) {
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
  if (!plan_decode(M, N, K, &p)) return KBH_ERR_SHAPE;
  if (bf) dispatch_decode<true>(p, x, qweight, scales, zeros, y, acc, counters, M, N, K, group, st);
  else dispatch_decode<false>(p, x, qweight, scales, zeros, y, acc, counters, M, N, K, group, st);
  return launch_status();
}
