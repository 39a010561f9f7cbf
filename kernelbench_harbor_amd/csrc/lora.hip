// Multi-LoRA quantized linear for gfx950: an int4 base weight (stored one value per int8) with
// per-token low-rank adapters.
//
// Reference tasks/multi_lora_qgemm/multi_lora_qgemm__llama3_8b_r16__fp16/environment/
// reference.py:10-17 (template generate_tasks.py:396-420), in the activation dtype:
//   W    = dtype(dtype(qweight) * dtype(scales[d / GROUP]))          [D, N]      (:12)
//   base = dtype(x @ W)                                              [T, N]      (:13)
//   lo   = dtype(x[t] @ A[id_t])                                     [T, r]      (:14-15)
//   y    = dtype(base + dtype(lo[t] @ B[id_t]))                      [T, N]      (:16-17)
// Three launches: the base GEMM is the byte-weight GEMM of byte_weight_gemm.h with the int8
// decoder (its split-K slices left in the workspace, or base written into y when K is not
// split); lora_shrink_kernel computes fp32 partial sums of x[t] @ A[id] over DS ranges of D
// (T x DS workgroups, so that a few tokens still fill the chip); lora_expand_add_kernel sums
// the DS partials in order and rounds lo to dtype, sums the GEMM's slices in split order (or
// reads base from y) and rounds base, and writes dtype(base + dtype(lo @ B)) (four columns per
// thread). Adapter ids index as torch does (reference.py:14-16, A[lora_ids]): an id in [-L, 0)
// selects adapter id + L. An id outside [-L, L), for which torch raises, makes its output row
// NaN (the adapter reads stay in bounds on adapter 0 or L - 1): no plausible wrong values.
#include "byte_weight_gemm.h"

namespace kbh {
namespace {

constexpr int kLoraMaxRank = 64;
constexpr int kLoraThreads = 256;
constexpr int kLoraMaxSplits = 16;  // D ranges of the shrink

__device__ inline bool lora_id_valid(const int64_t* ids, int t, int L) {
  const int64_t v = ids[t];
  return v >= -(int64_t)L && v < (int64_t)L;
}
__device__ inline int lora_id(const int64_t* ids, int t, int L) {
  int64_t v = ids[t];
  if (v < 0 && v >= -(int64_t)L) v += L;
  return v < 0 ? 0 : (v >= L ? L - 1 : (int)v);
}

// part[ds][t][j] = sum over d in range ds of x[t][d] A[id][d][j], fp32. Lane (row rr, column
// group c4) of a wave reads 8 bytes (columns 4c4..4c4+3) of row d of A; a wave covers 256 / r
// rows per step, the four waves interleave their rows; partial sums meet by lane shuffles, then
// across waves in LDS.
template <bool BF16>
__global__ __launch_bounds__(kLoraThreads) void lora_shrink_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ A, const int64_t* __restrict__ ids,
    float* __restrict__ out, int T, int D, int r, int L, int dchunk) {
  __shared__ float part[kLoraThreads / 64][kLoraMaxRank];
  const int t = blockIdx.x;
  const int d0 = blockIdx.y * dchunk, d1 = min(D, d0 + dchunk);
  const int l = lora_id(ids, t, L);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lpr = r >> 2;          // lanes per row of A
  const int rps = 64 / lpr;        // rows per wave and step
  const int c4 = lane % lpr, rr = lane / lpr;
  const uint16_t* xr = x + (size_t)t * D;
  const uint16_t* Al = A + (size_t)l * D * r + 4 * c4;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  const int step = 4 * rps;
  int d = d0 + wave * rps + rr;
  for (; d + 3 * step < d1; d += 4 * step) {  // four rows in flight
    kbh_u32x2 a[4];
    float xv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      a[u] = *reinterpret_cast<const kbh_u32x2*>(Al + (size_t)(d + u * step) * r);
      xv[u] = half_bits_to_f32<BF16>(xr[d + u * step]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        acc[c] += xv[u] * half_bits_to_f32<BF16>((uint16_t)(a[u][c >> 1] >> (16 * (c & 1))));
  }
  for (; d < d1; d += step) {
    const kbh_u32x2 a = *reinterpret_cast<const kbh_u32x2*>(Al + (size_t)d * r);
    const float xv = half_bits_to_f32<BF16>(xr[d]);
#pragma unroll
    for (int c = 0; c < 4; ++c)
      acc[c] += xv * half_bits_to_f32<BF16>((uint16_t)(a[c >> 1] >> (16 * (c & 1))));
  }
  for (int o = lpr; o < 64; o <<= 1)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] += __shfl_xor(acc[c], o, 64);
  if (rr == 0)
#pragma unroll
    for (int c = 0; c < 4; ++c) part[wave][4 * c4 + c] = acc[c];
  __syncthreads();
  if (threadIdx.x < r) {
    const int j = threadIdx.x;
    out[((size_t)blockIdx.y * T + t) * r + j] = part[0][j] + part[1][j] + part[2][j] + part[3][j];
  }
}

// lo[t][j] = dtype(sum over ds in order of part[ds][t][j]);
// base[t][n] = dtype(sum over s in order of slices[s][t][n]) (splits > 1), else y[t][n];
// y[t][n] = dtype(fp32(base) + fp32(dtype(sum_j lo[t][j] B[id][j][n]))).
template <bool BF16>
__global__ __launch_bounds__(kLoraThreads) void lora_expand_add_kernel(
    const float* __restrict__ part, const uint16_t* __restrict__ B, const int64_t* __restrict__ ids,
    const float* __restrict__ slices, int splits, uint16_t* __restrict__ y, int T, int N, int r,
    int L, int ds) {
  __shared__ float los[kLoraMaxRank];
  const int t = blockIdx.y;
  const int l = lora_id(ids, t, L);
  if (threadIdx.x < r) {
    float pv[kLoraMaxSplits];  // all partials requested before the first add
#pragma unroll
    for (int s = 0; s < kLoraMaxSplits; ++s)
      pv[s] = s < ds ? part[((size_t)s * T + t) * r + threadIdx.x] : 0.f;
    float v = pv[0];
#pragma unroll
    for (int s = 1; s < kLoraMaxSplits; ++s)
      if (s < ds) v += pv[s];
    los[threadIdx.x] = half_bits_to_f32<BF16>(f32_to_half_bits<BF16>(v));
  }
  __syncthreads();
  const int n = (blockIdx.x * kLoraThreads + threadIdx.x) * 4;
  if (n >= N) return;
  const uint16_t* Bl = B + (size_t)l * r * N + n;
  uint16_t* yr = y + (size_t)t * N + n;
  float bs[4];
  if (splits > 1) {  // the base GEMM's split-K slices, added in split order
    const size_t stride = (size_t)T * N;
    const kbh_f32x4 v = sum_slices(reinterpret_cast<const kbh_f32x4*>(slices + (size_t)t * N + n),
                                   stride / 4, splits);
#pragma unroll
    for (int c = 0; c < 4; ++c) bs[c] = half_bits_to_f32<BF16>(f32_to_half_bits<BF16>(v[c]));
  } else {
    const kbh_u32x2 base = *reinterpret_cast<const kbh_u32x2*>(yr);
#pragma unroll
    for (int c = 0; c < 4; ++c) bs[c] = half_bits_to_f32<BF16>((uint16_t)(base[c >> 1] >> (16 * (c & 1))));
  }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < r; j += 4) {  // r % 4 == 0: four rows of B in flight
    kbh_u32x2 b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) b[u] = *reinterpret_cast<const kbh_u32x2*>(Bl + (size_t)(j + u) * N);
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        acc[c] += los[j + u] * half_bits_to_f32<BF16>((uint16_t)(b[u][c >> 1] >> (16 * (c & 1))));
  }
  const bool valid = lora_id_valid(ids, t, L);
  kbh_u32x2 out;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float v[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const float e = half_bits_to_f32<BF16>(f32_to_half_bits<BF16>(acc[2 * h + c]));
      v[c] = valid ? keep_f32(bs[2 * h + c] + e) : __builtin_nanf("");  // select: keeps -0.0
    }
    out[h] = (uint32_t)f32_to_half_bits<BF16>(v[0]) | ((uint32_t)f32_to_half_bits<BF16>(v[1]) << 16);
  }
  *reinterpret_cast<kbh_u32x2*>(yr) = out;
}

struct LoraLayout {
  size_t part, total;
  int ds, dchunk;
};

// DS ranges of D for the shrink: enough workgroups (T x DS >= 1024, DS <= 16) while each keeps
// at least four steps of 1024 / r rows (one round of four loads in flight per lane).
LoraLayout lora_layout(int T, int D, int N, int r) {
  LoraLayout L;
  const int step = 1024 / r;
  const int ds_max = max(1, min(kLoraMaxSplits, D / (4 * step)));
  L.ds = max(1, min((1024 + T - 1) / T, ds_max));
  L.dchunk = (D + L.ds - 1) / L.ds;
  L.part = round_up(byte_gemm_workspace_bytes(T, N, D), 256);
  L.total = L.part + round_up((size_t)L.ds * T * r * 4, 256);
  return L;
}

template <bool BF16>
int lora_run(const void* x, const int8_t* qweight, const void* scales, const void* A,
             const void* B, const int64_t* ids, void* y, void* ws, size_t ws_bytes, int T, int D,
             int N, int r, int L, int group, hipStream_t st) {
  const LoraLayout lay = lora_layout(T, D, N, r);
  float* part = (float*)((char*)ws + lay.part);
  int splits = 1;
  const int s = byte_gemm_run<BF16, kDecInt8>(x, qweight, scales, y, ws, lay.part, T, N, D, group,
                                              st, true, &splits);
  if (s != KBH_OK) return s;
  hipLaunchKernelGGL(lora_shrink_kernel<BF16>, dim3(T, lay.ds), dim3(kLoraThreads), 0, st,
                     (const uint16_t*)x, (const uint16_t*)A, ids, part, T, D, r, L, lay.dchunk);
  const dim3 grid((N / 4 + kLoraThreads - 1) / kLoraThreads, T);
  hipLaunchKernelGGL(lora_expand_add_kernel<BF16>, grid, dim3(kLoraThreads), 0, st,
                     (const float*)part, (const uint16_t*)B, ids, (const float*)ws, splits,
                     (uint16_t*)y, T, N, r, L, lay.ds);
  return launch_status();
}

}  // namespace
}  // namespace kbh

extern "C" size_t kbh_lora_qgemm_workspace_bytes(int T, int D, int N, int r) {
  if (T < 1 || D < 32 || N < 128 || r < 1) return 0;
  return kbh::lora_layout(T, D, N, r).total;
}

extern "C" int kbh_lora_qgemm(const void* x, const int8_t* qweight, const void* scales,
                              const void* A, const void* B, const int64_t* lora_ids, void* y,
                              void* workspace, size_t workspace_bytes, int T, int D, int N, int r,
                              int L, int group, int dtype, void* stream) {
  using namespace kbh;
  if (!x || !qweight || !scales || !A || !B || !lora_ids || !y || !workspace) return KBH_ERR_NULL;
  if (dtype != KBH_F16 && dtype != KBH_BF16) return KBH_ERR_DTYPE;
  if (T < 1 || L < 1 || N < 128 || N % 128 != 0 || D < 32 || D % 32 != 0) return KBH_ERR_SHAPE;
  if (group != 32 && group != 64 && group != 128 && group != 256) return KBH_ERR_SHAPE;
  if (D % group != 0) return KBH_ERR_SHAPE;
  if (r != 4 && r != 8 && r != 16 && r != 32 && r != 64) return KBH_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(qweight) || !aligned16(scales) || !aligned16(y) ||
      !aligned16(workspace))
    return KBH_ERR_ALIGN;
  if ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) & 7u) return KBH_ERR_ALIGN;
  if (workspace_bytes < lora_layout(T, D, N, r).total) return KBH_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == KBH_BF16)
    return lora_run<true>(x, qweight, scales, A, B, lora_ids, y, workspace, workspace_bytes, T, D,
                          N, r, L, group, st);
  return lora_run<false>(x, qweight, scales, A, B, lora_ids, y, workspace, workspace_bytes, T, D,
                         N, r, L, group, st);
}
