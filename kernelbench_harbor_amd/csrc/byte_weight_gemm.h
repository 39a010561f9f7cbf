// Byte-weight GEMM for gfx950: y = x @ W with W[k, n] = dtype(decode(w[k, n]) * scales[k/B, n]),
// w one byte per element, [K, N] with N contiguous, one scale per B consecutive k of a column.
// Decoders (DEC): kDecE4M3 — OCP e4m3fn codes with fp16 scales (tasks/fp8_microscale/
// fp8_microscale__llama3_8b_down__b128__fp16/environment/reference.py:9-12); kDecInt8 — int8
// values (int4 stored one per byte) with scales in the activation dtype (tasks/multi_lora_qgemm/
// multi_lora_qgemm__llama3_8b_r16__fp16/environment/reference.py:12). Either way every weight
// is rounded once, as in the references: the decoded value is exact in fp16/bf16 and fp32, and
// the product with the scale is rounded once (v_pk_mul_f16, or an exact fp32 product rounded to
// bf16).
//
// Both kernels transpose 4x4 byte blocks in registers so that each lane holds consecutive k of
// one column, as the MFMA B operand needs.
//  * byte_decode_kernel (small M): a wave owns 128 columns (8 per lane, dwordx2 loads) and SPW
//    steps of 32 k for MB blocks of 16 rows (each dequantised weight fragment feeds MB MFMAs, so
//    the weights are streamed once per 16 MB rows); all loads up front; 16x16x32 fp16/bf16
//    MFMAs; split-K epilogue of splitk.h, once per row block.
//  * larger M: tiled_f16_gemm (tiled_f16.h) with ByteSlabPolicy.
#pragma once

#include "kbh_common.h"
#include "splitk.h"
#include "tiled_f16.h"

namespace kbh {
namespace {

constexpr int kDecE4M3 = 0;
constexpr int kDecInt8 = 1;

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f2_t __attribute__((ext_vector_type(2)));

// 4x4 byte transpose: r[i] holds bytes (row i, columns 0..3); c[j] receives (rows 0..3, column j).
__device__ inline void transpose4x4_b(const uint32_t r[4], uint32_t c[4]) {
  const uint32_t t0 = __builtin_amdgcn_perm(r[1], r[0], 0x05010400u);
  const uint32_t t1 = __builtin_amdgcn_perm(r[1], r[0], 0x07030602u);
  const uint32_t t2 = __builtin_amdgcn_perm(r[3], r[2], 0x05010400u);
  const uint32_t t3 = __builtin_amdgcn_perm(r[3], r[2], 0x07030602u);
  c[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
  c[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
  c[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
  c[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

// Four codes (bytes of v, k order) times scale s -> four dtype values in two dwords, each
// rounded once. e4m3: s holds fp16 bits; int8: s holds bits of the activation dtype.
template <bool BF16, int DEC>
__device__ inline kbh_u32x2 byte4_dequant(uint32_t v, uint16_t s) {
  if constexpr (DEC == kDecInt8) {
    if constexpr (BF16) {
      const float sf = bf16_bits_to_f32(s);
      const float q0 = (float)(int8_t)(v & 0xffu), q1 = (float)(int8_t)((v >> 8) & 0xffu);
      const float q2 = (float)(int8_t)((v >> 16) & 0xffu), q3 = (float)(int8_t)(v >> 24);
      return kbh_u32x2{f32x2_to_bf16x2_bits(keep_f32(q0 * sf), keep_f32(q1 * sf)),
                       f32x2_to_bf16x2_bits(keep_f32(q2 * sf), keep_f32(q3 * sf))};
    } else {
      // (byte ^ 0x80) | 0x6400 is the fp16 1024 + (q + 128); minus 1152 gives q exactly
      const _Float16 sh = __builtin_bit_cast(_Float16, s);
      const _Float16 bias = (_Float16)1152.0f;
      const uint32_t p0 = (__builtin_amdgcn_perm(0u, v, 0x0c010c00u) ^ 0x00800080u) | 0x64006400u;
      const uint32_t p1 = (__builtin_amdgcn_perm(0u, v, 0x0c030c02u) ^ 0x00800080u) | 0x64006400u;
      const h2_t lo = (__builtin_bit_cast(h2_t, p0) - h2_t{bias, bias}) * h2_t{sh, sh};
      const h2_t hi = (__builtin_bit_cast(h2_t, p1) - h2_t{bias, bias}) * h2_t{sh, sh};
      return kbh_u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
    }
  } else if constexpr (BF16) {
    const float sf = f16_bits_to_f32(s);
    const f2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(v, false);
    const f2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8(v, true);
    return kbh_u32x2{f32x2_to_bf16x2_bits(keep_f32(lo[0] * sf), keep_f32(lo[1] * sf)),
                     f32x2_to_bf16x2_bits(keep_f32(hi[0] * sf), keep_f32(hi[1] * sf))};
  } else {
    const _Float16 sh = __builtin_bit_cast(_Float16, s);
    const h2_t lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v, 1.0f, false) * h2_t{sh, sh};
    const h2_t hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v, 1.0f, true) * h2_t{sh, sh};
    return kbh_u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
  }
}

template <int SPW, bool BF16, int DEC, int MB>
__global__ __launch_bounds__(kSplitKMaxWaves * 64) void byte_decode_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ w,
    const uint16_t* __restrict__ scales, uint16_t* __restrict__ y, float* __restrict__ acc,
    int M, int N, int K, int block, int splits) {
  constexpr int NCS = 8;  // lane column c owns output columns n0 + 8c .. +7
  constexpr int NWG = 128;
  __shared__ SplitKSmem<NCS, float> sm;
  const int waves = blockDim.x >> 6;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = id / splits, split = id - tile * splits;
  const int n0 = tile * NWG;
  const int m0 = blockIdx.y * 16 * MB;
  const int st0 = (split * waves + wave) * SPW;  // first 32-deep K step of this wave

  // lane (c, g): rows k0 + 8g + i (i < 8), bytes n0 + 8c .. +7
  kbh_u32x2 wd[SPW][8];
  const uint8_t* wb = w + (size_t)(st0 * 32 + 8 * g) * N + n0 + 8 * c;
#pragma unroll
  for (int u = 0; u < SPW; ++u)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      wd[u][i] = __builtin_nontemporal_load(reinterpret_cast<const kbh_u32x2*>(wb + (size_t)(u * 32 + i) * N));
  kbh_u32x4 af[SPW][MB], sv[SPW];
  bool xok[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    xok[mb] = m0 + 16 * mb + c < M;
    const uint16_t* xb = x + (size_t)(xok[mb] ? m0 + 16 * mb + c : 0) * K + st0 * 32 + 8 * g;
#pragma unroll
    for (int u = 0; u < SPW; ++u) af[u][mb] = *reinterpret_cast<const kbh_u32x4*>(xb + u * 32);
  }
#pragma unroll
  for (int u = 0; u < SPW; ++u)
    sv[u] = *reinterpret_cast<const kbh_u32x4*>(scales + (size_t)(((st0 + u) * 32) / block) * N + n0 + 8 * c);
  // All loads are issued before any use (a consumer between them stalls the stream).
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < SPW; ++u)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      if (!xok[mb]) af[u][mb] = kbh_u32x4{0u, 0u, 0u, 0u};  // rows past M contribute zero

  kbh_f32x4 part[MB][NCS];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int cs = 0; cs < NCS; ++cs) part[mb][cs] = kbh_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < SPW; ++u) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // dword h: columns 4h .. 4h+3
      uint32_t col[4][2];          // col[j][b]: column 4h+j, rows 4b .. 4b+3
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const uint32_t r[4] = {wd[u][4 * b][h], wd[u][4 * b + 1][h], wd[u][4 * b + 2][h],
                               wd[u][4 * b + 3][h]};
        uint32_t t4[4];
        transpose4x4_b(r, t4);
#pragma unroll
        for (int j = 0; j < 4; ++j) col[j][b] = t4[j];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int cs = 4 * h + j;
        const uint16_t s = half_of(sv[u], cs);
        const kbh_u32x2 lo = byte4_dequant<BF16, DEC>(col[j][0], s);
        const kbh_u32x2 hi = byte4_dequant<BF16, DEC>(col[j][1], s);
        const kbh_u32x4 bf = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) part[mb][cs] = mfma16x16x32<BF16>(af[u][mb], bf, part[mb][cs]);
      }
    }
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int mr = m0 + 16 * mb;
    const int rows = min(16, M - mr);
    if (rows <= 0) break;      // uniform across the workgroup
    if (mb) __syncthreads();   // the previous block's LDS reads are done
    splitk_reduce<NCS, float>(part[mb], sm, acc, split, splits, rows, M, N, mr, n0, [&](int r, int n, float v) {
      y[(size_t)(mr + r) * N + n0 + n] = f32_to_half_bits<BF16>(v);
    });
  }
}

// Weight-slab producer for tiled_f16_gemm: thread t loads rows 4*(t/32) .. +3 of the slab for
// columns 4*(t%32) .. +3, transposes, dequantizes and stores them k-major per column.
template <bool BF16, int DEC>
struct ByteSlabPolicy {
  const uint8_t* w;
  const uint16_t* scales;
  int N, block;
  struct Regs {
    uint32_t b[4];
    kbh_u32x2 s;
  };
  __device__ void load(Regs& r, int k0, int n0, int t) const {
    const int cq = t & 31, rq = t >> 5;
    const uint8_t* p = w + (size_t)(k0 + 4 * rq) * N + n0 + 4 * cq;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      r.b[i] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p + (size_t)i * N));
    r.s = *reinterpret_cast<const kbh_u32x2*>(scales + (size_t)(k0 / block) * N + n0 + 4 * cq);
  }
  __device__ void store(const Regs& r, uint16_t* Bs, int t) const {
    const int cq = t & 31, rq = t >> 5;
    uint32_t cols[4];
    transpose4x4_b(r.b, cols);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint16_t s = (uint16_t)((j & 1) ? (r.s[j >> 1] >> 16) : (r.s[j >> 1] & 0xffffu));
      *reinterpret_cast<kbh_u32x2*>(&Bs[tld_row(4 * cq + j) * TLD + 4 * rq]) = byte4_dequant<BF16, DEC>(cols[j], s);
    }
  }
};

constexpr int kByteTiledMinM = 128;

struct BytePlan {
  int spw, waves, ntiles, mb, mblocks, splits;
};

// Row blocks per wave (MB: 1 up to 16 rows, 2 up to 32, 4 up to 64, then 16-row blocks of 4),
// 4-step (128-deep) wave K ranges when they divide K (2 at MB = 4, for registers), waves per
// workgroup and K splits as for the W4 decode kernel.
bool plan_byte_decode(int M, int N, int K, BytePlan* p) {
  const int nsteps = K / 32;
  const int m16 = (M + 15) / 16;
  p->mb = m16 <= 1 ? 1 : (m16 <= 2 ? 2 : 4);
  const int smax = p->mb == 4 ? 2 : 4;
  p->spw = (nsteps % smax == 0) ? smax : (nsteps % 2 == 0 ? 2 : 1);
  p->ntiles = N / 128;
  p->mblocks = (m16 + p->mb - 1) / p->mb;
  p->splits = 0;
  p->waves = splitk_pick_waves(nsteps / p->spw, p->ntiles * p->mblocks, &p->splits);
  return p->waves > 0;
}

// Runs the GEMM; with `defer_sum` and a split K the slices are left in the workspace
// (acc[splits][M][N] fp32) for the caller to sum, and *splits_out tells how many (1: y written).
template <bool BF16, int DEC>
int byte_gemm_run(const void* x, const void* w, const void* scales, void* y, void* workspace,
                  size_t workspace_bytes, int M, int N, int K, int block, hipStream_t st,
                  bool defer_sum = false, int* splits_out = nullptr) {
  if (splits_out) *splits_out = 1;
  if (M >= kByteTiledMinM && K % (TBK * TDEPTH) == 0) {
    const ByteSlabPolicy<BF16, DEC> bp{(const uint8_t*)w, (const uint16_t*)scales, N, block};
    hipLaunchKernelGGL((tiled_f16_gemm<BF16, ByteSlabPolicy<BF16, DEC>>), tiled_f16_grid(M, N),
                       dim3(256), 0, st, (const uint16_t*)x, bp, (uint16_t*)y, M, N, K);
    return launch_status();
  }
  BytePlan pl;
  if (!plan_byte_decode(M, N, K, &pl)) return KBH_ERR_SHAPE;
  const int spw = pl.spw, waves = pl.waves, splits = pl.splits;
  const size_t need = splitk_workspace_bytes(M, N, splits);
  if (need > 0 && (!workspace || workspace_bytes < need)) return KBH_ERR_WORKSPACE;
  if (need > 0 && !aligned16(workspace)) return KBH_ERR_ALIGN;
  dim3 grid(pl.ntiles * splits, pl.mblocks);
  float* acc = (float*)workspace;
#define KBH_BYTE_DEC(SPW_, MB_)                                                                  \
  if (spw == SPW_ && pl.mb == MB_)                                                               \
    hipLaunchKernelGGL((byte_decode_kernel<SPW_, BF16, DEC, MB_>), grid, dim3(waves * 64), 0, st, \
                       (const uint16_t*)x, (const uint8_t*)w, (const uint16_t*)scales,           \
                       (uint16_t*)y, acc, M, N, K, block, splits);
  KBH_BYTE_DEC(4, 1) else KBH_BYTE_DEC(2, 1) else KBH_BYTE_DEC(1, 1)
  else KBH_BYTE_DEC(4, 2) else KBH_BYTE_DEC(2, 2) else KBH_BYTE_DEC(1, 2)
  else KBH_BYTE_DEC(2, 4) else KBH_BYTE_DEC(1, 4)
#undef KBH_BYTE_DEC
  if (splits_out) *splits_out = splits;
  if (splits > 1 && !defer_sum)
    launch_splitk_sum(reinterpret_cast<const kbh_f32x4*>(acc), HalfOut<BF16>{(uint16_t*)y, N}, M, N,
                      pl.ntiles, 128, splits, st);
  return launch_status();
}

// Workspace bytes of byte_gemm_run for this shape (0 when K is not split).
size_t byte_gemm_workspace_bytes(int M, int N, int K) {
  BytePlan p;
  if (M < 1 || N < 128 || K < 32) return 0;
  if (M >= kByteTiledMinM && K % (TBK * TDEPTH) == 0) return 0;  // tiled path: no split
  if (!plan_byte_decode(M, N, K, &p)) return 0;
  return splitk_workspace_bytes(M, N, p.splits);
}

}  // namespace
}  // namespace kbh
