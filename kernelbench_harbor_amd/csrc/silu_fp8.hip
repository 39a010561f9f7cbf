// Fused SiLU-and-multiply with per-group dynamic e4m3 quantisation: the activation stage of an
// MoE expert between its gate/up GEMM and an FP8 down GEMM.
//
// Restates tasks/fused_silu_fp8/<task>/environment/reference.py:13-23 (template
// generate_tasks.py:321-348): y [T, 2H] = concat(gate, up) in fp16/bf16,
//   act   = fp32(silu(fp32(gate)) * fp32(up))
//   scale = max(amax_group(|act|) / 448, 1e-12)            one per GROUP consecutive columns
//   q     = e4m3fn_rne(clamp(act / scale, -448, 448))
//   out   = fp32(q) * scale                                 [T, H] fp32 (the reference's output)
// plus, when asked for, the e4m3 codes [T, H] and the fp32 scales [T, H/GROUP] that an FP8 GEMM
// would consume.
//
// One pass over HBM: every element is read once (two 16-byte loads per lane: 8 gate and 8 up
// values) and written once. LPG lanes share one group (8 elements each); the group's absmax is
// reduced across them with lane shuffles, so no LDS and no barrier. GPS groups per lane are in
// flight together to cover HBM latency on large launches.
//
// Arithmetic per element is kept to ~16 VALU operations so that the kernel stays HBM bound
// (a correctly rounded fp32 division alone is ~10): SiLU uses the hardware exp2 and reciprocal
// (a few ulp from torch's expf and division, within the tolerance), and act / scale is exact:
// with r = RN(1 / scale) (one true division per group), q0 = RN(act r), rem = act - q0 scale
// (exact, one fma), RN(q0 + rem r) is the correctly rounded quotient (Markstein's theorem; no
// overflow here since |act / scale| <= ~448; subnormal quotients round to code 0 either way).
// Infinite or NaN scales take true divisions.
#include "kbh_common.h"

namespace kbh {
namespace {

typedef float kbh_f32x2 __attribute__((ext_vector_type(2)));

constexpr float kFp8Max = 448.0f;
constexpr float kLog2e = 1.44269504088896341f;
constexpr int kSiluThreads = 256;

template <bool BF16>
__device__ inline void unpack8(kbh_u32x4 w, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = half_bits_to_f32<BF16>((uint16_t)(w[i] & 0xffffu));
    f[2 * i + 1] = half_bits_to_f32<BF16>((uint16_t)(w[i] >> 16));
  }
}

// clamp(v, -448, 448) (v_med3_f32). A NaN group is handled by its caller: its scale is NaN, so
// every dequantised output is NaN, and its codes are set to the NaN code.
__device__ inline float clamp448(float v) { return __builtin_amdgcn_fmed3f(v, -kFp8Max, kFp8Max); }

// Grid: T x CB blocks, CB = ceil(G / (SEGS GPS)) blocks per row (row = block / CB, a scalar
// division); segment s of round i of a block handles group (chunk GPS + i) SEGS + s of its row.
template <bool BF16, int LPG, int GPS>
__global__ __launch_bounds__(kSiluThreads) void silu_fp8_kernel(
    const uint16_t* __restrict__ y, float* __restrict__ out, uint8_t* __restrict__ codes,
    float* __restrict__ scales, int H, int G, int CB) {
  constexpr int SEGS = kSiluThreads / LPG;  // groups per block and round
  const int seg = threadIdx.x / LPG, l = threadIdx.x % LPG;
  const int row = blockIdx.x / CB, chunk = blockIdx.x - row * CB;
  const uint16_t* yrow = y + (size_t)row * 2 * H;
  kbh_u32x4 gw[GPS], uw[GPS];
  int g[GPS], col[GPS];
#pragma unroll
  for (int i = 0; i < GPS; ++i) {
    g[i] = (chunk * GPS + i) * SEGS + seg;
    const int gi = g[i] < G ? g[i] : G - 1;  // loads stay in range; the store is skipped
    col[i] = gi * (LPG * 8) + l * 8;
    gw[i] = __builtin_nontemporal_load(reinterpret_cast<const kbh_u32x4*>(yrow + col[i]));
    uw[i] = __builtin_nontemporal_load(reinterpret_cast<const kbh_u32x4*>(yrow + H + col[i]));
  }
#pragma unroll
  for (int i = 0; i < GPS; ++i) {
    float a[8], u[8];
    unpack8<BF16>(gw[i], a);
    unpack8<BF16>(uw[i], u);
    float m = 0.0f;
    bool nan = false;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // F.silu in fp32: x / (1 + e^-x); e^-x = 2^(-x log2 e) -> inf for x < -88, giving -0
      const float e = __builtin_amdgcn_exp2f(-a[j] * kLog2e);
      const float s = keep_f32(a[j] * __builtin_amdgcn_rcpf(1.0f + e));
      a[j] = s * u[j];
      nan |= a[j] != a[j];
      m = fmaxf(m, fabsf(a[j]));
    }
#pragma unroll
    for (int o = 1; o < LPG; o <<= 1) {
      m = fmaxf(m, __shfl_xor(m, o, 64));
      nan |= __shfl_xor((int)nan, o, 64) != 0;
    }
    const float scale = nan ? __builtin_nanf("") : fmaxf(m / kFp8Max, 1e-12f);
    float q[8];
    if (scale < __builtin_inff()) {
      const float r = 1.0f / scale;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float q0 = a[j] * r;
        q[j] = __builtin_fmaf(__builtin_fmaf(-q0, scale, a[j]), r, q0);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) q[j] = a[j] / scale;
    }
    kbh_u32x2 c;
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      int v = __builtin_amdgcn_cvt_pk_fp8_f32(clamp448(q[4 * w]), clamp448(q[4 * w + 1]), 0, false);
      v = __builtin_amdgcn_cvt_pk_fp8_f32(clamp448(q[4 * w + 2]), clamp448(q[4 * w + 3]), v, true);
      c[w] = (uint32_t)v;
    }
    if (nan) c = kbh_u32x2{0x7f7f7f7fu, 0x7f7f7f7fu};  // e4m3fn NaN codes
    if (g[i] >= G) continue;
    const size_t obase = (size_t)row * H + col[i];
    kbh_f32x4 d[2];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const kbh_f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)c[w], false);
      const kbh_f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)c[w], true);
      d[w] = kbh_f32x4{lo[0] * scale, lo[1] * scale, hi[0] * scale, hi[1] * scale};
    }
    kbh_f32x4* po = reinterpret_cast<kbh_f32x4*>(out + obase);
    __builtin_nontemporal_store(d[0], po);
    __builtin_nontemporal_store(d[1], po + 1);
    if (codes) __builtin_nontemporal_store(c, reinterpret_cast<kbh_u32x2*>(codes + obase));
    if (scales && l == 0) scales[(size_t)row * G + g[i]] = scale;
  }
}

template <bool BF16, int LPG>
void launch_silu_fp8(const uint16_t* y, float* out, uint8_t* codes, float* scales, int T, int H,
                     hipStream_t st) {
  constexpr int SEGS = kSiluThreads / LPG;
  const int G = H / (LPG * 8);
  // Two groups per lane when they tile the row exactly and the launch still has four blocks
  // per CU; otherwise one (more blocks, fewer idle lanes on ragged rows).
  if (G % (2 * SEGS) == 0 && (long)T * (G / (2 * SEGS)) >= 4L * 256) {
    const int CB = G / (2 * SEGS);
    hipLaunchKernelGGL((silu_fp8_kernel<BF16, LPG, 2>), dim3((unsigned)(T * CB)),
                       dim3(kSiluThreads), 0, st, y, out, codes, scales, H, G, CB);
  } else {
    const int CB = (G + SEGS - 1) / SEGS;
    hipLaunchKernelGGL((silu_fp8_kernel<BF16, LPG, 1>), dim3((unsigned)(T * CB)),
                       dim3(kSiluThreads), 0, st, y, out, codes, scales, H, G, CB);
  }
}

template <bool BF16>
void silu_fp8_run(const uint16_t* y, float* out, uint8_t* codes, float* scales, int T, int H,
                  int group, hipStream_t st) {
  switch (group) {
    case 32: launch_silu_fp8<BF16, 4>(y, out, codes, scales, T, H, st); break;
    case 64: launch_silu_fp8<BF16, 8>(y, out, codes, scales, T, H, st); break;
    default: launch_silu_fp8<BF16, 16>(y, out, codes, scales, T, H, st); break;
  }
}

}  // namespace
}  // namespace kbh

extern "C" int kbh_silu_fp8_quant(const void* y, float* out, uint8_t* q_codes, float* q_scales,
                                  int T, int H, int group, int dtype, void* stream) {
  using namespace kbh;
  if (!y || !out) return KBH_ERR_NULL;
  if (dtype != KBH_F16 && dtype != KBH_BF16) return KBH_ERR_DTYPE;
  if (group != 32 && group != 64 && group != 128) return KBH_ERR_SHAPE;
  if (T < 0 || H < group || H % group != 0) return KBH_ERR_SHAPE;
  // one block per (row, chunk of >= 8 groups) in a 32-bit grid
  if ((long)T * ((H / group + 7) / 8) >= (1L << 31)) return KBH_ERR_SHAPE;
  if (!aligned16(y) || !aligned16(out)) return KBH_ERR_ALIGN;
  if ((reinterpret_cast<uintptr_t>(q_codes) & 7u) || (reinterpret_cast<uintptr_t>(q_scales) & 3u))
    return KBH_ERR_ALIGN;
  if (T == 0) return KBH_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == KBH_BF16)
    silu_fp8_run<true>((const uint16_t*)y, out, q_codes, q_scales, T, H, group, st);
  else
    silu_fp8_run<false>((const uint16_t*)y, out, q_codes, q_scales, T, H, group, st);
  return launch_status();
}
