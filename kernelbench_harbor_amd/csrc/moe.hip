// Top-2 quantized mixture-of-experts on gfx950.
//
// Reference op (tasks/fused_qmoe/fused_qmoe__mixtral__fp16/environment/reference.py:11-21):
//   probs = softmax(fp32(router_logits)); topv, topi = top2(probs); w = dtype(topv / sum(topv))
//   W_e   = dtype(dtype(qweight[e]) * dtype(scales[e, d/G]))          (int4 values stored int8)
//   y[t]  = sum_k dtype(dtype(x[t] @ W_{topi[t,k]}) * w[t,k])          (the gather of all_out)
// SiLU FFN (the benchmark's SiLU FFN configuration; no reference module, same routing and combine):
//   h = dtype(silu(x @ Wg_e) * (x @ Wu_e)),  o = dtype(h @ Wd_e),  y[t] = sum_k dtype(o_k w_k)
// with W4A16 g128 gate/up/down weights (packed along their output dimension).
//
// Kernels:
//  * moe_topk_select_kernel + moe_route_build_kernel (with k = 2): softmax + top-2 per token
//    (one wave per token), then per-expert counts (LDS atomics), prefix sums, the slot
//    permutation perm[slot] = 2t + k (slots grouped by expert) and a tile table of (expert,
//    first slot, rows) with BM rows per tile; unused table entries get rows = 0. Only the
//    routed (token, expert) pairs are computed downstream — the reference computes all experts
//    densely (reference.py:19).
//  * moe_gemm_kernel: expert-grouped GEMM. A workgroup takes one tile of one expert and 128
//    output columns; x rows are gathered through perm, the expert's weights come from a slab
//    policy (int8-stored int4 or packed int4, dequantized exactly into LDS), the K loop is the
//    register-ring / two-LDS-buffer pipeline of tiled_f16.h, and the epilogue writes rows either
//    per slot (the FFN intermediate h) or per (token, k) pair. GATED fuses two weight streams
//    (gate and up) and applies silu(g) * u before rounding.
//  * moe_combine_kernel: y[t] = dtype(o[2t] w[2t] + o[2t+1] w[2t+1]) with the reference's
//    roundings (each product rounded to dtype, fp32 sum of the two, one rounding).
#include <type_traits>

#include "kbh_common.h"
#include "tiled_f16.h"
#include "tiled_wide.h"
#include "tiled_ws.h"
#include "w4_dequant.h"

namespace kbh {
namespace {

constexpr int kMoeMaxExperts = 256;

template <int LDT>  // logits dtype: 0 fp16, 1 bf16, 2 fp32
__device__ inline float logit_at(const void* p, size_t i) {
  if constexpr (LDT == 0) return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  else if constexpr (LDT == 1) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  else return reinterpret_cast<const float*>(p)[i];
}

struct MoeBuffers {
  int* topi;        // [2T]
  uint16_t* topw;   // [2T] routing weights in the activation dtype (fp32 when wmode == 2)
  int* slot_of;     // [2T] position of (t, k) inside its expert's slot range
  int* perm;        // [2T] slot -> 2t + k
  int* tiles;       // [max_tiles][3] = expert, first slot, rows
  float* topw32;    // [2T] the same weights unrounded (fp32), when not null
};

// Top-k routing (k <= kMoeMaxTopk, E <= kMoeMaxExperts) for every MoE op here
// (tasks/fused_qmoe/<task>/environment/reference.py:14-16, tasks/moe/<task>/environment/
// reference.py:11-13: probs = softmax(fp32 logits); topv, topi = probs.topk(k)), in two kernels:
//  * moe_topk_select_kernel: one wave per token, lanes across experts (up to 4 each). The
//    softmax max and sum are wave reductions. The ids and their order are those torch.topk
//    returns on the GPU, in its two steps: the k picks are k rounds of a wave argmax on (logit
//    descending, index ascending), which selects every value above the k-th largest and, on a
//    tie at the boundary, the lowest indices; they are then laid out in torch's slot order
//    (values above the k-th ascending by index, then the k-th value's ties ascending by index)
//    and put through the 32-slot descending bitonic network of torch's small sort (lane = slot,
//    invalid slots sink), whose compare-exchange keeps or swaps equal keys by slot position:
//    e.g. two equal top values come out higher index first. Logits order like the
//    probabilities (softmax is monotonic; fp16/bf16 logits that differ never round to equal
//    fp32 probabilities). NaN logits rank as -inf (every id is a distinct expert in range).
//    Weights p_j / sum_j p_j (summed in output order) are written in the activation dtype
//    (wmode 0 fp16, 1 bf16) or fp32 (wmode 2), and unrounded to topw32 when it is set.
//  * moe_route_build_kernel (one workgroup): per-expert slot counts (LDS atomics), offsets,
//    the permutation perm[slot] = k t + j and the tile table (unused entries: rows = 0).
constexpr int kMoeMaxTopk = 8;
constexpr int kTopkWaves = 4;  // tokens per workgroup of the select kernel
constexpr int kTopkSlots = 32;  // slots of torch's small bitonic sort

template <int LDT, int K>
__global__ __launch_bounds__(kTopkWaves * 64) void moe_topk_select_kernel(
    const void* __restrict__ logits, int T, int E, int wmode, MoeBuffers mb) {
  static_assert(K >= 1 && K <= kMoeMaxTopk, "top-k");
  constexpr int EPL = kMoeMaxExperts / 64;
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * kTopkWaves + (threadIdx.x >> 6);
  if (t >= T) return;  // whole waves
  const size_t row = (size_t)t * E;
  float v[EPL];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? logit_at<LDT>(logits, row + e) : -INFINITY;
    mx = fmaxf(mx, v[i]);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i)
    if (lane + 64 * i < E) sum += expf(v[i] - mx);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, 64);
  // Selection: k rounds of a wave argmax; every lane ends with all picks (lv, li).
  unsigned taken = 0;
  float lv[K];
  int li[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    float bv = -INFINITY;
    int be = kMoeMaxExperts;  // sentinel above every index
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane + 64 * i;
      const float w = v[i] != v[i] ? -INFINITY : v[i];
      if (e < E && !((taken >> i) & 1u) && (w > bv || (w == bv && e < be))) { bv = w; be = e; }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oe = __shfl_xor(be, o, 64);
      if (ov > bv || (ov == bv && oe < be)) { bv = ov; be = oe; }
    }
    if ((be & 63) == lane) taken |= 1u << (be >> 6);
    li[j] = be;
    lv[j] = bv;
  }
  // Slot order of torch's gather step: the picks above the k-th value by ascending index, then
  // the k-th value's ties by ascending index. Lane s (< K) takes the pick of rank s.
  const int slot = lane & (kTopkSlots - 1);
  const float vk = lv[K - 1];
  float sv = -INFINITY;
  int si = 0, ok = 0;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const int kj = (lv[j] > vk ? 0 : kMoeMaxExperts) + li[j];
    int rank = 0;
#pragma unroll
    for (int i = 0; i < K; ++i)
      if ((lv[i] > vk ? 0 : kMoeMaxExperts) + li[i] < kj) ++rank;
    if (rank == slot) { sv = lv[j]; si = li[j]; ok = 1; }
  }
  // torch's small sort: slots a < b = a ^ stride exchange when
  // ((key[a] > key[b] && a valid) || b invalid) == dir, dir = (a & size) != 0 while building
  // bitonic sequences, false in the final merge. Both lanes of a pair evaluate it alike.
  auto cx = [&](int size, int stride) {
    const float ov = __shfl_xor(sv, stride, 64);
    const int oi = __shfl_xor(si, stride, 64);
    const int ook = __shfl_xor(ok, stride, 64);
    const bool lo = (slot & stride) == 0;
    const float va = lo ? sv : ov, vb = lo ? ov : sv;
    const int oka = lo ? ok : ook, okb = lo ? ook : ok;
    const bool dir = size < kTopkSlots && (((lo ? slot : slot ^ stride) & size) != 0);
    if ((((va > vb) && oka) || !okb) == dir) { sv = ov; si = oi; ok = ook; }
  };
  if constexpr (K > 1) {
#pragma unroll
    for (int size = 2; size <= kTopkSlots; size *= 2)
#pragma unroll
      for (int stride = size / 2; stride > 0; stride /= 2) cx(size, stride);
  }
  // Weights in output order: p_s = exp(l_s - max) / sum, renormalised by their sum (slot order).
  const float pk = keep_f32(expf(sv - mx) / sum);
  float ps = 0.f;
#pragma unroll
  for (int j = 0; j < K; ++j) ps = keep_f32(ps + __shfl(pk, j, 64));
  if (lane < K) {
    const float w = keep_f32(pk / ps);
    mb.topi[K * t + lane] = si;
    if (wmode == 2) reinterpret_cast<float*>(mb.topw)[K * t + lane] = w;
    else mb.topw[K * t + lane] = wmode ? f32_to_bf16_bits(w) : f32_to_f16_bits(w);
    if (mb.topw32) mb.topw32[K * t + lane] = w;
  }
}

__global__ __launch_bounds__(1024) void moe_route_build_kernel(int T, int E, int K, MoeBuffers mb,
                                                               int max_tiles, int bm) {
  __shared__ int cnt[kMoeMaxExperts];
  __shared__ int off[kMoeMaxExperts];
  __shared__ int tbase[kMoeMaxExperts + 1];
  const int S = K * T;
  for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < S; i += blockDim.x) mb.slot_of[i] = atomicAdd(&cnt[mb.topi[i]], 1);
  __syncthreads();
  if (threadIdx.x == 0) {
    int o = 0, tb = 0;
    for (int e = 0; e < E; ++e) {
      off[e] = o;
      tbase[e] = tb;
      o += cnt[e];
      tb += (cnt[e] + bm - 1) / bm;
    }
    tbase[E] = tb;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < S; i += blockDim.x) mb.perm[off[mb.topi[i]] + mb.slot_of[i]] = i;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    for (int j = 0; j < tbase[e + 1] - tbase[e]; ++j) {
      int* tl = &mb.tiles[3 * (tbase[e] + j)];
      tl[0] = e;
      tl[1] = off[e] + j * bm;
      tl[2] = min(bm, cnt[e] - j * bm);
    }
  }
  for (int i = tbase[E] + threadIdx.x; i < max_tiles; i += blockDim.x) {
    mb.tiles[3 * i] = 0;
    mb.tiles[3 * i + 1] = 0;
    mb.tiles[3 * i + 2] = 0;
  }
}

// Slab producer for fp16/bf16 weights [E][K][N] (N contiguous), used as they are and stored
// as they lie in memory: LDS rows of kBnPitch halves per k (128 columns + 32 of padding), each
// thread copying 16 bytes of rows t / 16 and t / 16 + 16. The GEMM reads its B fragments with
// the transposing LDS read (kNMajor; see moe_gemm_kernel), so no transpose happens here.
constexpr int kBnPitch = 160;  // 320-byte rows: the 4 rows x 64 bytes of one 32-lane read fill
                               // 64 distinct banks
struct F16SlabPolicy {
  static constexpr bool kNMajor = true;
  const uint16_t* w;
  int N;
  size_t w_stride;
  __device__ F16SlabPolicy at_expert(int e) const {
    F16SlabPolicy p = *this;
    p.w += (size_t)e * w_stride;
    return p;
  }
  struct Regs {
    kbh_u32x4 r[2];
  };
  __device__ void load(Regs& r, int k0, int n0, int t) const {
    const int c = t & 15, k = t >> 4;
    const uint16_t* p = w + (size_t)(k0 + k) * N + n0 + 8 * c;
    r.r[0] = __builtin_nontemporal_load(reinterpret_cast<const kbh_u32x4*>(p));
    r.r[1] = __builtin_nontemporal_load(reinterpret_cast<const kbh_u32x4*>(p + (size_t)16 * N));
  }
  __device__ void store(const Regs& r, uint16_t* Bs, int t) const {
    const int c = t & 15, k = t >> 4;
    *reinterpret_cast<kbh_u32x4*>(&Bs[k * kBnPitch + 8 * c]) = r.r[0];
    *reinterpret_cast<kbh_u32x4*>(&Bs[(k + 16) * kBnPitch + 8 * c]) = r.r[1];
  }
};
static_assert(32 * kBnPitch == 128 * TLD, "an N-major slab uses the buffer of a k-major one");

// Weight producer of the warp-specialised kernel (tiled_ws.h) for fp16/bf16 weights [E][K][N]
// (N contiguous): thread t loads 4 rows (K) x 8 columns (16 bytes per row) of a 32 x 256 slab
// and writes each column's 4 values as one 8-byte piece of the K-contiguous operand layout
// (wide_b_offset), pairing the 16-bit halves of two rows with one v_perm_b32 per dword; the
// thread map (column block cb, row block rb) is the int8 producer's.
struct F16WidePolicy {
  static constexpr int kTN = 256;
  static constexpr bool kHasFast = false;
  const uint16_t* w;
  int N;
  size_t w_stride;
  struct Raw {
    kbh_u32x4 r[4];
  };
  struct Grp {};
  struct ScanPre {};
  __device__ F16WidePolicy at_expert(int e) const {
    F16WidePolicy p = *this;
    p.w += (size_t)e * w_stride;
    return p;
  }
  __device__ static int cb_of(int t) { return (t & 7) | (((t >> 4) & 3) << 3); }
  __device__ static int rb_of(int t) { return ((t >> 3) & 1) | ((t >> 6) << 1); }
  __device__ void load(Raw& r, int k0, int n0, int t) const {
    const uint16_t* p = w + (size_t)(k0 + 4 * rb_of(t)) * N + n0 + 8 * cb_of(t);
#pragma unroll
    for (int i = 0; i < 4; ++i) r.r[i] = *reinterpret_cast<const kbh_u32x4*>(p + (size_t)i * N);
  }
  __device__ void load_group(Grp&, int, int, int) const {}
  template <bool FAST>
  __device__ void prepare_group(Grp&) const {}
  template <bool FAST>
  __device__ void store_all(const Raw& r, const Grp&, uint8_t* Bs, int t) const {
    const int cb = cb_of(t), rb = rb_of(t);
    // wide_b_offset<256>(8 rb, 8 cb + c) = base + 16 (c ^ fw)
    uint8_t* base = Bs + wide_b_offset<256>(8 * rb, 8 * cb) - wide_slot(8 * cb) * 16 + cb * 128;
    const int fw = (cb ^ (cb >> 3)) & 7;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;  // high or low halves
      const uint32_t d0 = __builtin_amdgcn_perm(r.r[1][c >> 1], r.r[0][c >> 1], sel);
      const uint32_t d1 = __builtin_amdgcn_perm(r.r[3][c >> 1], r.r[2][c >> 1], sel);
      *reinterpret_cast<kbh_u32x2*>(base + ((c ^ fw) << 4)) = kbh_u32x2{d0, d1};
    }
  }
};

// Policies without kNMajor store k-major slabs (Bs[tld_row(n) * TLD + k]).
template <class BP, class = void>
struct NMajor {
  static constexpr bool value = false;
};
template <class BP>
struct NMajor<BP, std::void_t<decltype(BP::kNMajor)>> {
  static constexpr bool value = BP::kNMajor;
};

typedef short kbh_i16x4 __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16 (measured lane layout): within each 16-lane group, output lane i element j
// is element i % 4 of the 8 bytes addressed by lane 4j + i / 4. With lane 4j + q addressing row
// k0 + j, columns n0 + 4q .. +3 of an N-major slab, lane i receives rows k0 .. k0 + 3 of column
// n0 + i.
__device__ inline kbh_i16x4 lds_read_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) kbh_i16x4*)(const_cast<uint16_t*>(p)));
}

// Slab producer for int8-stored weights [E][K][N] (N contiguous) without their scales: the
// integers q themselves in the activation dtype (every int8 value is exact in fp16 and bf16).
// The reference qMoE op applies the scales per quantization group to the fp32 accumulators
// instead (moe_gemm_kernel with GS > 0), so each expert's weights enter the products exactly,
// as in the grader's fp32 ground truth (q * s is exact in fp32). Stored N-major (read with the
// transposing LDS read): thread t converts 16 consecutive columns (16 bytes) of row t / 8 and
// writes them as two 16-byte stores.
// fp32 value of the signed byte B (0..3) of v: v_cvt_f32_i32 with a sign-extended SDWA byte
// select (exact).
template <int B>
__device__ inline float sbyte_to_f32(uint32_t v) {
  float r;
  asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_%2"
      : "=v"(r) : "v"(v), "n"(B));
  return r;
}

template <bool BF16>
struct I8QSlabPolicy {
  static constexpr bool kNMajor = true;
  const int8_t* w;
  int N;
  size_t w_stride;
  __device__ I8QSlabPolicy at_expert(int e) const {
    I8QSlabPolicy p = *this;
    p.w += (size_t)e * w_stride;
    return p;
  }
  struct Regs {
    kbh_u32x4 q;
  };
  __device__ void load(Regs& r, int k0, int n0, int t) const {
    const int c = t & 7, k = t >> 3;
    r.q = __builtin_nontemporal_load(
        reinterpret_cast<const kbh_u32x4*>(w + (size_t)(k0 + k) * N + n0 + 16 * c));
  }
  __device__ void store(const Regs& r, uint16_t* Bs, int t) const {
    const int c = t & 7, k = t >> 3;
    kbh_u32x4 out[2];
#pragma unroll
    for (int d = 0; d < 4; ++d) {  // dword d of the 16 bytes: columns 4d .. 4d + 3
      const uint32_t v = r.q[d];
#pragma unroll
      for (int h = 0; h < 2; ++h) {  // columns 4d + 2h, 4d + 2h + 1
        if constexpr (BF16) {
          // An int8 value has at most 8 significant bits, so its fp32 image ends in 16 zero bits
          // and its upper half is the exact bf16. One SDWA conversion per byte, one v_perm_b32
          // per pair (the compiler's own code took a shift, a v_bfe_i32 and a conversion).
          const float lo = h ? sbyte_to_f32<2>(v) : sbyte_to_f32<0>(v);
          const float hi = h ? sbyte_to_f32<3>(v) : sbyte_to_f32<1>(v);
          out[d >> 1][2 * (d & 1) + h] = __builtin_amdgcn_perm(
              __builtin_bit_cast(uint32_t, hi), __builtin_bit_cast(uint32_t, lo), 0x07060302u);
        } else {
          // fp16 magic: (byte ^ 0x80) | 0x6400 is 1024 + (q + 128); minus 1152 gives q exactly.
          typedef _Float16 h2 __attribute__((ext_vector_type(2)));
          const _Float16 bias = (_Float16)1152.0f;
          const uint32_t P = __builtin_amdgcn_perm(0u, v, h ? 0x0c030c02u : 0x0c010c00u);
          const h2 q = __builtin_bit_cast(h2, (P ^ 0x00800080u) | 0x64006400u) - h2{bias, bias};
          out[d >> 1][2 * (d & 1) + h] = __builtin_bit_cast(uint32_t, q);
        }
      }
    }
    *reinterpret_cast<kbh_u32x4*>(&Bs[k * kBnPitch + 16 * c]) = out[0];
    *reinterpret_cast<kbh_u32x4*>(&Bs[k * kBnPitch + 16 * c + 8]) = out[1];
  }
};

__device__ inline float silu(float v) { return v / (1.0f + expf(-v)); }
// The same with the hardware exponential and reciprocal (v_exp_f32 of -v log2(e), v_rcp_f32;
// ~1e-6 relative error, against ~35 VALU instructions per value for expf and the IEEE
// division): the FFN's gate/up epilogue evaluates 128 x 128 of them per tile.
__device__ inline float silu_fast(float v) {
  return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v));
}

// Expert-grouped GEMM. BM = 64 (1x4 waves, 64x32 each) or 128 (2x2 waves, 64x64 each).
// GS > 0 (the reference qMoE op): the producer delivers unscaled integer weights and every GS
// slabs (one quantization group) the group's fp32 sums are scaled by the group's scales
// (fscales [E][K/(GS*TBK)][N], x.dtype) into fp32 totals, which are written as fp32 to `out`.
template <bool BF16, int BM, class BP, bool GATHER, bool GATED, bool OUT_PERM, int GS = 0>
__global__ __launch_bounds__(256, GS > 0 ? 2 : 1) void moe_gemm_kernel(const uint16_t* __restrict__ A, int lda,
                                                       const int* __restrict__ perm,
                                                       const int* __restrict__ tiles, BP bp,
                                                       BP bp2, uint16_t* __restrict__ out,
                                                       int ldo, int N, int K, int topk,
                                                       const uint16_t* __restrict__ fscales = nullptr,
                                                       size_t fs_stride = 0) {
  constexpr int BN = 128;
  constexpr int WM = BM / 64, WN = 4 / WM;  // waves along M and N
  constexpr int WNT = BN / WN / 32;         // 32-column MFMA tiles per wave
  constexpr int NB = GATED ? 2 : 1;
  constexpr int AL = BM / 64;               // 16-byte x chunks per thread per slab
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * TLD];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[NB][2][BN * TLD];

  const int* tl = &tiles[3 * blockIdx.y];
  const int e = tl[0], s0 = tl[1], rows = tl[2];
  if (rows == 0) return;  // unused tile-table entry (uniform across the workgroup)
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int n0 = blockIdx.x * BN;
  const BP bpe = bp.at_expert(e);
  const BP bpe2 = bp2.at_expert(e);
  const int KT = K / TBK;

  const int a_ch = t & 3, a_row = t >> 2;
  const uint16_t* arow[AL];
#pragma unroll
  for (int i = 0; i < AL; ++i) {
    const int r = min(a_row + 64 * i, rows - 1);  // rows past the tile repeat the last one
    const int s = s0 + r;
    const int src = GATHER ? (perm[s] / topk) : s;  // perm[s] = topk * token + k
    arow[i] = A + (size_t)src * lda + a_ch * 8;
  }
  struct Slab {
    kbh_u32x4 a[AL];
    typename BP::Regs b[NB];
  };
  auto load = [&](Slab& sl, int kt) {
    const int k0 = kt * TBK;
#pragma unroll
    for (int i = 0; i < AL; ++i) sl.a[i] = *reinterpret_cast<const kbh_u32x4*>(arow[i] + k0);
    bpe.load(sl.b[0], k0, n0, t);
    if constexpr (GATED) bpe2.load(sl.b[1], k0, n0, t);
  };
  auto store = [&](const Slab& sl, int buf) {
#pragma unroll
    for (int i = 0; i < AL; ++i)
      *reinterpret_cast<kbh_u32x4*>(&As[buf][(a_row + 64 * i) * TLD + a_ch * 8]) = sl.a[i];
    bpe.store(sl.b[0], Bs[0][buf], t);
    if constexpr (GATED) bpe2.store(sl.b[1], Bs[1][buf], t);
  };

  kbh_f32x16 accv[NB][2][WNT];
#pragma unroll
  for (int q = 0; q < NB; ++q)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < WNT; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) accv[q][i][j][v] = 0.f;

  const int fr = lane & 31, fk = (lane >> 5) * 8;
  auto mma = [&](int buf) {
#pragma unroll
    for (int kk = 0; kk < TBK / 16; ++kk) {
      kbh_u32x4 a[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const kbh_u32x4*>(&As[buf][(wm * 64 + i * 32 + fr) * TLD + fk + kk * 16]);
#pragma unroll
      for (int q = 0; q < NB; ++q)
#pragma unroll
        for (int j = 0; j < WNT; ++j) {
          kbh_u32x4 b;
          if constexpr (NMajor<BP>::value) {
            // 32x32x16 B operand: lane l takes k 8(l / 32) .. +7 of column l % 32; 16-lane group
            // g = l / 16 covers columns 16(g & 1) .. +15 at k 8(g >> 1), in two 4-row reads.
            const int g16 = lane >> 4, s16 = lane & 15;
            const uint16_t* p = &Bs[q][buf][(kk * 16 + 8 * (g16 >> 1) + (s16 >> 2)) * kBnPitch +
                                            wn * 32 * WNT + j * 32 + 16 * (g16 & 1) + 4 * (s16 & 3)];
            const kbh_i16x4 lo = lds_read_tr16(p), hi = lds_read_tr16(p + 4 * kBnPitch);
            b = kbh_u32x4{__builtin_bit_cast(kbh_u32x2, lo)[0], __builtin_bit_cast(kbh_u32x2, lo)[1],
                          __builtin_bit_cast(kbh_u32x2, hi)[0], __builtin_bit_cast(kbh_u32x2, hi)[1]};
          } else {
            b = *reinterpret_cast<const kbh_u32x4*>(
                &Bs[q][buf][tld_row(wn * 32 * WNT + j * 32 + fr) * TLD + fk + kk * 16]);
          }
#pragma unroll
          for (int i = 0; i < 2; ++i) accv[q][i][j] = mfma32x32x16<BF16>(a[i], b, accv[q][i][j]);
        }
    }
  };

  // Fold (GS > 0): totals, and the scales of this lane's columns for the current group (loaded
  // one group ahead of their use).
  constexpr bool FOLD = GS > 0;
  constexpr int U = (GS > TDEPTH) ? GS : TDEPTH;  // slabs per loop iteration
  kbh_f32x16 tot[FOLD ? 2 : 1][FOLD ? WNT : 1];
  float sc[WNT];
  const uint16_t* fsc = fscales + (FOLD ? (size_t)e * fs_stride : 0);
  auto load_scales = [&](int g) {
#pragma unroll
    for (int j = 0; j < WNT; ++j)
      sc[j] = half_bits_to_f32<BF16>(fsc[(size_t)g * N + n0 + wn * 32 * WNT + j * 32 + fr]);
  };
  if constexpr (FOLD) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < WNT; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) tot[i][j][v] = 0.f;
    load_scales(0);
  }
  auto fold = [&](int g_next) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < WNT; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          tot[i][j][v] = fmaf(sc[j], accv[0][i][j][v], tot[i][j][v]);
          accv[0][i][j][v] = 0.f;
        }
    load_scales(g_next);
  };

  Slab ring[TDEPTH];
#pragma unroll
  for (int d = 0; d < TDEPTH; ++d) load(ring[d], min(d, KT - 1));
  store(ring[0], 0);
  load(ring[0], min(TDEPTH, KT - 1));
  __syncthreads();
  for (int kt0 = 0; kt0 < KT; kt0 += U) {
#pragma unroll
    for (int d = 0; d < U; ++d) {
      const int kt = kt0 + d;
      const int nxt = (d + 1) % TDEPTH;
      mma(kt & 1);
      if constexpr (FOLD) {
        if ((d + 1) % GS == 0) fold(min((kt + 1) / GS, KT / GS - 1));  // a group ends here
      }
      __builtin_amdgcn_sched_barrier(0);  // phases in order (see tiled_f16.h)
      store(ring[nxt], (kt + 1) & 1);     // after the last slab: unused buffer
      __builtin_amdgcn_sched_barrier(0);
      load(ring[nxt], min(kt + 1 + TDEPTH, KT - 1));
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Accumulator element v of tile (i, j): row 8(v/4) + 4(l/32) + v%4, column l%32.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < WNT; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = wm * 64 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (r < rows) {
          const int s = s0 + r;
          const int orow = OUT_PERM ? perm[s] : s;
          const int n = n0 + wn * 32 * WNT + j * 32 + fr;
          if constexpr (FOLD) {
            reinterpret_cast<float*>(out)[(size_t)orow * ldo + n] = tot[i][j][v];
            continue;
          }
          float val = accv[0][i][j][v];
          if constexpr (GATED) val = keep_f32(silu(val)) * accv[1][i][j][v];
          out[(size_t)orow * ldo + n] = f32_to_half_bits<BF16>(val);
        }
      }
}

// y[t][n] = dtype(fp32(dtype(o0 * w0)) + fp32(dtype(o1 * w1))), o_k = o[2t+k][n].
template <bool BF16>
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t* __restrict__ o,
                                                          const uint16_t* __restrict__ topw,
                                                          uint16_t* __restrict__ y, int T, int N) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)T * N) return;
  const size_t t = i / N, n = i - t * N;
  const float p0 = half_bits_to_f32<BF16>(f32_to_half_bits<BF16>(
      keep_f32(half_bits_to_f32<BF16>(o[(2 * t) * N + n]) * half_bits_to_f32<BF16>(topw[2 * t]))));
  const float p1 = half_bits_to_f32<BF16>(f32_to_half_bits<BF16>(keep_f32(
      half_bits_to_f32<BF16>(o[(2 * t + 1) * N + n]) * half_bits_to_f32<BF16>(topw[2 * t + 1]))));
  y[i] = f32_to_half_bits<BF16>(keep_f32(p0 + p1));
}

// y[t][n] = dtype(fp32(o[2t][n] w[2t]) + fp32(o[2t+1][n] w[2t+1])) with fp32 expert outputs
// and fp32 routing weights: the reference's (sel * topv).sum(dim=1) (reference.py:20-21)
// evaluated as in the grader's fp32 ground truth, rounded once. Four columns per thread.
template <bool BF16>
__global__ __launch_bounds__(256) void moe_combine_f32_kernel(const float* __restrict__ o,
                                                              const float* __restrict__ w,
                                                              uint16_t* __restrict__ y, int T,
                                                              int N) {
  const size_t i4 = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i4 >= (size_t)T * N) return;
  const size_t t = i4 / N, n = i4 - t * N;
  const kbh_f32x4 a = *reinterpret_cast<const kbh_f32x4*>(o + (2 * t) * N + n);
  const kbh_f32x4 b = *reinterpret_cast<const kbh_f32x4*>(o + (2 * t + 1) * N + n);
  const float w0 = w[2 * t], w1 = w[2 * t + 1];
  uint16_t r[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    r[c] = f32_to_half_bits<BF16>(keep_f32(keep_f32(a[c] * w0) + keep_f32(b[c] * w1)));
  kbh_u32x2 out;
  out[0] = (uint32_t)r[0] | ((uint32_t)r[1] << 16);
  out[1] = (uint32_t)r[2] | ((uint32_t)r[3] << 16);
  *reinterpret_cast<kbh_u32x2*>(y + i4) = out;
}

// y[t][n] = dtype(sum_j fp32(dtype(o[k t + j][n] * w[k t + j]))), j = 0..k-1 in order: the
// reference's (sel * topv).sum(dim=1) in the activation dtype (tasks/moe/<task>/environment/
// reference.py:16-17). Four columns per thread.
template <bool BF16>
__global__ __launch_bounds__(256) void moe_combine_k_kernel(const uint16_t* __restrict__ o,
                                                            const uint16_t* __restrict__ topw,
                                                            uint16_t* __restrict__ y, int T, int N,
                                                            int K) {
  const size_t i4 = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i4 >= (size_t)T * N) return;
  const size_t t = i4 / N, n = i4 - t * N;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < K; ++j) {
    const size_t r = (size_t)K * t + j;
    const float w = half_bits_to_f32<BF16>(topw[r]);
    const kbh_u32x2 v = *reinterpret_cast<const kbh_u32x2*>(o + r * N + n);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint16_t h = (uint16_t)(v[c >> 1] >> (16 * (c & 1)));
      acc[c] = keep_f32(acc[c] + half_bits_to_f32<BF16>(
                                     f32_to_half_bits<BF16>(keep_f32(half_bits_to_f32<BF16>(h) * w))));
    }
  }
  kbh_u32x2 out;
  out[0] = (uint32_t)f32_to_half_bits<BF16>(acc[0]) | ((uint32_t)f32_to_half_bits<BF16>(acc[1]) << 16);
  out[1] = (uint32_t)f32_to_half_bits<BF16>(acc[2]) | ((uint32_t)f32_to_half_bits<BF16>(acc[3]) << 16);
  *reinterpret_cast<kbh_u32x2*>(y + i4) = out;
}

// ---- SiLU FFN on the wide-tile kernel -------------------------------------------------------

// Gate and up weights as one virtual TN-column slab: in each 16-word chunk c of the tile, packed
// words 0..7 come from the gate matrix and words 8..15 from the up matrix, both at real output
// columns n0/2 + 64c + 8(w % 8) .. +7, so each lane ends with matching gate and up accumulators
// (virtual columns 128c + v and 128c + 64 + v).
template <bool BF16, int TN>
struct W4PairPolicy {
  using Half = W4WidePolicy<BF16, TN>;
  static constexpr int kTN = TN;
  static constexpr int kParts = Half::kParts;
  using Raw = typename Half::Raw;
  using Grp = typename Half::Grp;
  Half g, u;  // N = real output columns (F)
  __device__ W4PairPolicy at_expert(int e) const {
    return W4PairPolicy{g.at_expert(e), u.at_expert(e)};
  }
  // Word w of the tile: chunk c = w / 16, matrix (w / 8) % 2, real column n0/2 + 64c + 8(w % 8).
  // Half::load reads word w at column n0' + 8w, so n0' = n0/2 - 64c - 64 * matrix.
  __device__ static int shift(int w) { return 4 * (w & 16) + 8 * (w & 8); }
  // The matrix of lane t's word is selected per lane by pointer (a uniform instruction stream).
  __device__ void load(Raw& r, int k0, int n0, int t) const {
    const int w = Half::word_of(t);
    g.load_from(r, (w & 8) ? u.qw : g.qw, k0, n0 / 2 - shift(w), t);
  }
  __device__ void load_group(Grp& gr, int k0, int n0, int t) const {
    const int w = Half::word_of(t);
    const bool up = (w & 8) != 0;
    g.load_group_from(gr, up ? u.scales : g.scales, up ? u.zeros : g.zeros, k0, n0 / 2 - shift(w), t);
  }
  static constexpr bool kHasFast = Half::kHasFast;
  // Tile columns n0 .. n0 + TN are real columns n0/2 .. n0/2 + TN/2 of both matrices.
  __device__ bool scan_fast(int k_begin, int k_end, int n0, int t) const {
    return g.scan_cols(k_begin, k_end, n0 / 2, TN / 2, t) &&
           u.scan_cols(k_begin, k_end, n0 / 2, TN / 2, t);
  }
  struct ScanPre {
    typename Half::ScanPre g, u;
  };
  __device__ void scan_load(ScanPre& sp, int k_begin, int k_end, int n0, int t) const {
    g.scan_load_cols(sp.g, k_begin, k_end, n0 / 2, TN / 2, t);
    u.scan_load_cols(sp.u, k_begin, k_end, n0 / 2, TN / 2, t);
  }
  __device__ bool scan_check(const ScanPre& sp, int k_begin, int k_end, int n0, int t) const {
    // both checks run (no short circuit), so both matrices' scan loads are consumed together
    return (int)g.scan_check_cols(sp.g, k_begin, k_end, n0 / 2, TN / 2, t) &
           (int)u.scan_check_cols(sp.u, k_begin, k_end, n0 / 2, TN / 2, t);
  }
  template <bool FAST>
  __device__ void prepare_group(Grp& gr) const { g.template prepare_group<FAST>(gr); }
  template <bool FAST>
  __device__ void store_part(const Raw& r, const Grp& gr, uint8_t* Bs, int t, int p) const {
    // dequantisation and LDS layout do not depend on the matrix
    g.template store_part<FAST>(r, gr, Bs, t, p);
  }
  template <bool FAST>
  __device__ void store_all(const Raw& r, const Grp& gr, uint8_t* Bs, int t) const {
    g.template store_all<FAST>(r, gr, Bs, t);
  }
};

// h[slot][n] = dtype(silu(gate) * up) from the paired accumulators (fp32 math, one rounding).
template <bool BF16>
struct SiluPairOut {
  static constexpr bool kPaired = true;
  uint16_t* h;
  int ldh;
  // The 16-bit output of one (gate, up) accumulator pair.
  __device__ uint16_t pair_bits(float g, float u) const {
    return f32_to_half_bits<BF16>(keep_f32(silu_fast(g)) * u);
  }
  __device__ void emit_pair(int r, int n, float g, float u) const {
    h[(size_t)r * ldh + n] = pair_bits(g, u);
  }
  // Outputs n .. n + 7 of row r (n % 8 == 0), two per word.
  __device__ void store8(int r, int n, kbh_u32x4 v) const {
    *reinterpret_cast<kbh_u32x4*>(h + (size_t)r * ldh + n) = v;
  }
};

// Split-K down projection: the partial slices hold rows 2t + k; y[t] combines the two rows
// after summing the slices in split order and rounding each expert output to dtype, exactly as
// moe_combine_kernel does with unsplit outputs. One thread per 4 columns of one token.
template <bool BF16>
__global__ __launch_bounds__(256) void moe_reduce_combine_kernel(
    const float* __restrict__ part, int splits, const uint16_t* __restrict__ topw,
    uint16_t* __restrict__ y, int T, int N) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t n4 = (size_t)T * N / 4;
  if (i >= n4) return;
  const size_t e = 4 * i;
  const int t = (int)(e / (size_t)N), n = (int)(e - (size_t)t * N);
  const size_t slice4 = (size_t)2 * T * N / 4;  // one split's slice, in 4-float units
  const kbh_f32x4* p0 = reinterpret_cast<const kbh_f32x4*>(part + (size_t)(2 * t) * N + n);
  const kbh_f32x4* p1 = reinterpret_cast<const kbh_f32x4*>(part + (size_t)(2 * t + 1) * N + n);
  const kbh_f32x4 a = sum_slices(p0, slice4, splits), b = sum_slices(p1, slice4, splits);
  const float w0 = half_bits_to_f32<BF16>(topw[2 * t]), w1 = half_bits_to_f32<BF16>(topw[2 * t + 1]);
  uint16_t r[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float o0 = half_bits_to_f32<BF16>(f32_to_half_bits<BF16>(a[q]));
    const float o1 = half_bits_to_f32<BF16>(f32_to_half_bits<BF16>(b[q]));
    const float q0 = half_bits_to_f32<BF16>(f32_to_half_bits<BF16>(keep_f32(o0 * w0)));
    const float q1 = half_bits_to_f32<BF16>(f32_to_half_bits<BF16>(keep_f32(o1 * w1)));
    r[q] = f32_to_half_bits<BF16>(keep_f32(q0 + q1));
  }
  kbh_u32x2 o;
  o[0] = (uint32_t)r[0] | ((uint32_t)r[1] << 16);
  o[1] = (uint32_t)r[2] | ((uint32_t)r[3] << 16);
  *reinterpret_cast<kbh_u32x2*>(y + e) = o;
}

// FFN plan: TM x 256 expert tiles (TM = 256 rows when experts average at least 192 routed rows,
// else 128: at ~128 rows per expert, 256-row tiles measured 20% slower despite fewer tiles), one
// workgroup per CU with a 4-slab prefetch ring; gate/up unsplit (about
// 2T/TM x 2F/256 workgroups), down split over K until the estimated 2T/TM x D/256 tiles fill
// the CUs.
constexpr int kFfnPD = 4;
struct FfnPlan {
  int spg, tm;
  WidePlan down;
};
bool plan_ffn(int T, int E, int D, int F, int group, FfnPlan* p) {
  p->spg = group / 32;
  p->tm = (2 * T) / (E > 0 ? E : 1) >= 192 ? 256 : 128;
  const int unroll = 2 * p->spg > kFfnPD ? 2 * p->spg : kFfnPD;  // the kernel's slabs per iteration
  if (F % 128 != 0 || D % 256 != 0 || D % (unroll * 32) != 0 || F % (unroll * 32) != 0) return false;
  return plan_wide(2 * T, D, F, 256, 32, unroll, 256, &p->down, p->tm == 256 ? 256 : 128);
}

// ---- host side ------------------------------------------------------------------------------
struct MoeLayout {
  size_t topi, topw, slot_of, perm, tiles, h, o, part, topw32, total;
  int bm, max_tiles, topk;
};

// Slots: topk per token (slot order grouped by expert). bm: rows per tile-table entry (0: 128
// when an expert averages more than 48 rows, else 64). f32_out: expert outputs o in fp32 and
// fp32 routing weights (the reference qMoE op), else in the activation dtype.
MoeLayout moe_layout(int T, int E, int hidden, int out_cols, int bm = 0, size_t part_bytes = 0,
                     int topk = 2, bool f32_out = false) {
  MoeLayout L;
  const size_t S = (size_t)topk * T;
  L.topk = topk;
  L.bm = bm ? bm : ((int)S / (E > 0 ? E : 1) > 48 ? 128 : 64);
  L.max_tiles = (int)((S + L.bm - 1) / L.bm) + E;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += round_up(bytes, 256);
    return at;
  };
  L.topi = take(S * 4);
  L.topw = take(S * 2);
  L.slot_of = take(S * 4);
  L.perm = take(S * 4);
  L.tiles = take((size_t)L.max_tiles * 3 * 4);
  L.h = take(S * hidden * 2);
  L.o = take(S * out_cols * (f32_out ? 4 : 2));
  L.part = take(part_bytes);
  L.topw32 = f32_out ? take(S * 4) : 0;
  L.total = o;
  return L;
}

MoeBuffers moe_buffers(void* ws, const MoeLayout& L) {
  char* b = (char*)ws;
  return MoeBuffers{(int*)(b + L.topi), (uint16_t*)(b + L.topw), (int*)(b + L.slot_of),
                    (int*)(b + L.perm), (int*)(b + L.tiles),
                    L.topw32 ? (float*)(b + L.topw32) : nullptr};
}

// wmode: routing weights written to mb.topw as 0 fp16, 1 bf16, 2 fp32.
void launch_route_topk(const void* logits, int logits_dtype, int T, int E, int wmode,
                       const MoeBuffers& mb, const MoeLayout& L, hipStream_t st) {
  const dim3 g((T + kTopkWaves - 1) / kTopkWaves), b(kTopkWaves * 64);
  const int K = L.topk;
  auto sel = [&](auto ldt) {
    constexpr int LDT = decltype(ldt)::value;
    switch (K) {
#define KBH_SEL(K_)                                                                          \
  case K_:                                                                                   \
    hipLaunchKernelGGL((moe_topk_select_kernel<LDT, K_>), g, b, 0, st, logits, T, E, wmode,  \
                       mb);                                                                  \
    return;
      KBH_SEL(1) KBH_SEL(2) KBH_SEL(3) KBH_SEL(4) KBH_SEL(5) KBH_SEL(6) KBH_SEL(7)
      default: KBH_SEL(8)
#undef KBH_SEL
    }
  };
  if (logits_dtype == 0) sel(std::integral_constant<int, 0>{});
  else if (logits_dtype == 1) sel(std::integral_constant<int, 1>{});
  else sel(std::integral_constant<int, 2>{});
  hipLaunchKernelGGL(moe_route_build_kernel, dim3(1), dim3(1024), 0, st, T, E, K, mb, L.max_tiles,
                     L.bm);
}

template <bool BF16, class BP, bool GATHER, bool GATED, bool OUT_PERM, int GS = 0>
void launch_moe_gemm(const MoeLayout& L, const void* A, int lda, const MoeBuffers& mb, const BP& bp,
                     const BP& bp2, void* out, int ldo, int N, int K, hipStream_t st,
                     const uint16_t* fscales = nullptr, size_t fs_stride = 0) {
  const dim3 grid(N / 128, L.max_tiles);
  if (L.bm == 64)
    hipLaunchKernelGGL((moe_gemm_kernel<BF16, 64, BP, GATHER, GATED, OUT_PERM, GS>), grid, dim3(256),
                       0, st, (const uint16_t*)A, lda, mb.perm, mb.tiles, bp, bp2, (uint16_t*)out,
                       ldo, N, K, L.topk, fscales, fs_stride);
  else
    hipLaunchKernelGGL((moe_gemm_kernel<BF16, 128, BP, GATHER, GATED, OUT_PERM, GS>), grid,
                       dim3(256), 0, st, (const uint16_t*)A, lda, mb.perm, mb.tiles, bp, bp2,
                       (uint16_t*)out, ldo, N, K, L.topk, fscales, fs_stride);
}

// The reference qMoE op's expert GEMM: exact integer weights, the scales folded per group
// (GS = group / TBK slabs), fp32 outputs per (token, k) row.
template <bool BF16>
void launch_qmoe_gemm(const MoeLayout& L, const void* x, const MoeBuffers& mb, const int8_t* q,
                      const void* scales, void* o, int D, int N, int group, hipStream_t st) {
  const I8QSlabPolicy<BF16> bp{q, N, (size_t)D * N};
  const uint16_t* sc = (const uint16_t*)scales;
  const size_t ss = (size_t)(D / group) * N;
  using BP = I8QSlabPolicy<BF16>;
  switch (group / TBK) {
    case 1: return launch_moe_gemm<BF16, BP, true, false, true, 1>(L, x, D, mb, bp, bp, o, N, N, D, st, sc, ss);
    case 2: return launch_moe_gemm<BF16, BP, true, false, true, 2>(L, x, D, mb, bp, bp, o, N, N, D, st, sc, ss);
    case 4: return launch_moe_gemm<BF16, BP, true, false, true, 4>(L, x, D, mb, bp, bp, o, N, N, D, st, sc, ss);
    default: return launch_moe_gemm<BF16, BP, true, false, true, 8>(L, x, D, mb, bp, bp, o, N, N, D, st, sc, ss);
  }
}

template <bool BF16>
void launch_combine(const void* o, const uint16_t* topw, void* y, int T, int N, hipStream_t st) {
  const size_t n = (size_t)T * N;
  hipLaunchKernelGGL(moe_combine_kernel<BF16>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     (const uint16_t*)o, topw, (uint16_t*)y, T, N);
}

template <bool BF16, int TM, int SPG>
void launch_ffn_wide_spg(const FfnPlan& fp, const MoeLayout& L, const MoeBuffers& mb,
                         const void* x, const W4WidePolicy<BF16, 256>& gp,
                         const W4WidePolicy<BF16, 256>& upp, const W4WidePolicy<BF16, 256>& dp,
                         void* h, void* o, float* part, void* y, int T, int D, int F,
                         hipStream_t st) {
  using E = WideHalf<BF16>;
  // gate/up: rows gathered from x through perm, h written in slot order
  {
    using RM = GroupedRows<true, false>;
    using BP = W4PairPolicy<BF16, 256>;
    const BP bp{gp, upp};
    const SiluPairOut<BF16> ep{(uint16_t*)h, F};
    const int grid = L.max_tiles * (2 * F / 256);
    // 128-row tiles: 2 x 2 MFMA waves of 64 x 128 (each wave one gate/up column pair chunk), x
    // staged through LDS (XD: 32-bit offsets; ffn_layout takes this path only while 2T rows of
    // x and of h stay under 2 GiB).
    if constexpr (TM == 128)
      hipLaunchKernelGGL((tiled_ws_gemm<E, TM, 2, SPG, BP, SiluPairOut<BF16>, RM, kFfnPD, 1, true>),
                         dim3(grid), dim3(512), 0, st, x, bp, ep, (float*)nullptr, 2 * T, 2 * F,
                         D, 1, D / 32, RM{mb.tiles, mb.perm});
    else
      hipLaunchKernelGGL((tiled_wide_gemm<E, TM, 4, SPG, BP, SiluPairOut<BF16>, RM, 1, kFfnPD>),
                         dim3(grid), dim3(256), 0, st, x, bp, ep, (float*)nullptr, 2 * T, 2 * F,
                         D, 1, D / 32, RM{mb.tiles, mb.perm});
  }
  // down: h rows in slot order, outputs (or split-K partials) in row 2t + k
  {
    using RM = GroupedRows<false, true>;
    using BP = W4WidePolicy<BF16, 256>;
    const HalfOut<BF16> ep{(uint16_t*)o, D};
    const int splits = fp.down.splits;
    const int grid = L.max_tiles * (D / 256) * splits;
    if constexpr (TM == 128)
      hipLaunchKernelGGL((tiled_ws_gemm<E, TM, 2, SPG, BP, HalfOut<BF16>, RM, kFfnPD, 1, true>),
                         dim3(grid), dim3(512), 0, st, h, dp, ep, part, 2 * T, D, F, splits,
                         fp.down.slabs_per_split, RM{mb.tiles, mb.perm});
    else
      hipLaunchKernelGGL((tiled_wide_gemm<E, TM, 4, SPG, BP, HalfOut<BF16>, RM, 1, kFfnPD>),
                         dim3(grid), dim3(256), 0, st, h, dp, ep, part, 2 * T, D, F, splits,
                         fp.down.slabs_per_split, RM{mb.tiles, mb.perm});
    if (splits > 1) {
      const size_t n4 = (size_t)T * D / 4;
      hipLaunchKernelGGL((moe_reduce_combine_kernel<BF16>), dim3((unsigned)((n4 + 255) / 256)),
                         dim3(256), 0, st, part, splits, mb.topw, (uint16_t*)y, T, D);
    } else {
      launch_combine<BF16>(o, mb.topw, y, T, D, st);
    }
  }
}

template <bool BF16>
void launch_ffn_wide(const FfnPlan& fp, const MoeLayout& L, const MoeBuffers& mb, const void* x,
                     const int32_t* gq_, const void* gs_, const void* gz_, const int32_t* uq_,
                     const void* us_, const void* uz_, const int32_t* dq_, const void* ds_,
                     const void* dz_, void* h, void* o, float* part, void* y, int T, int D, int F,
                     int group, size_t gq, size_t gs, size_t dq, size_t ds, hipStream_t st) {
  const W4WidePolicy<BF16, 256> gp{(const uint32_t*)gq_, (const uint16_t*)gs_,
                                   (const uint16_t*)gz_, F, group, gq, gs, 0x000F000Fu};
  const W4WidePolicy<BF16, 256> upp{(const uint32_t*)uq_, (const uint16_t*)us_,
                                    (const uint16_t*)uz_, F, group, gq, gs, 0x000F000Fu};
  const W4WidePolicy<BF16, 256> dp{(const uint32_t*)dq_, (const uint16_t*)ds_,
                                   (const uint16_t*)dz_, D, group, dq, ds, 0x000F000Fu};
#define KBH_FFN(TM_, SPG_) \
  return launch_ffn_wide_spg<BF16, TM_, SPG_>(fp, L, mb, x, gp, upp, dp, h, o, part, y, T, D, F, st)
  if (fp.tm == 256) {
    switch (fp.spg) {
      case 1: KBH_FFN(256, 1);
      case 2: KBH_FFN(256, 2);
      case 4: KBH_FFN(256, 4);
      default: KBH_FFN(256, 8);
    }
  }
  switch (fp.spg) {
    case 1: KBH_FFN(128, 1);
    case 2: KBH_FFN(128, 2);
    case 4: KBH_FFN(128, 4);
    default: KBH_FFN(128, 8);
  }
#undef KBH_FFN
}

// FFN layout: TM-row tiles (the plan's) and room for the down projection's split-K partials when the wide
// path applies (plan_ffn); otherwise the 256 x 128 grouped kernels run.
MoeLayout ffn_layout(int T, int E, int D, int F, int group, bool* wide, FfnPlan* fp) {
  // The wide path stages x (T x D) and h (2T x F) through LDS with 32-bit buffer offsets, so it
  // needs 2T rows of either under 2 GiB; beyond that the grouped kernels (64-bit addresses) run.
  const size_t act_bytes = (size_t)2 * T * (size_t)(D > F ? D : F) * 2;
  *wide = (group == 32 || group == 64 || group == 128 || group == 256) &&
          act_bytes < ((size_t)1 << 31) && plan_ffn(T, E, D, F, group, fp);
  if (!*wide) return moe_layout(T, E, F, D);
  const size_t part = fp->down.splits > 1 ? (size_t)fp->down.splits * 2 * T * D * 4 : 0;
  return moe_layout(T, E, F, D, fp->tm, part);
}

bool moe_shape_ok(int T, int E, int K, int N, int group) {
  return T >= 1 && E >= 2 && E <= kMoeMaxExperts && N >= 128 && N % 128 == 0 && K >= 128 &&
         K % (TBK * TDEPTH) == 0 && (group == 32 || group == 64 || group == 128 || group == 256) &&
         K % group == 0;
}

}  // namespace
}  // namespace kbh

extern "C" size_t kbh_qmoe_workspace_bytes(int T, int D, int N, int E) {
  (void)D;
  if (T <= 0 || E <= 0) return 0;
  return kbh::moe_layout(T, E, 0, N, 0, 0, 2, true).total;
}

extern "C" int kbh_moe_route_top2(const void* router_logits, int logits_dtype, int32_t* topi,
                                  void* topw, void* workspace, size_t workspace_bytes, int T,
                                  int E, int dtype, void* stream) {
  using namespace kbh;
  if (!router_logits || !topi || !topw || !workspace) return KBH_ERR_NULL;
  if (logits_dtype < 0 || logits_dtype > 2 ||
      (dtype != KBH_F16 && dtype != KBH_BF16 && dtype != KBH_F32))
    return KBH_ERR_DTYPE;
  if (T < 1 || E < 2 || E > kMoeMaxExperts) return KBH_ERR_SHAPE;
  const MoeLayout L = moe_layout(T, E, 0, 0);
  if (workspace_bytes < L.total) return KBH_ERR_WORKSPACE;
  MoeBuffers mb = moe_buffers(workspace, L);
  mb.topi = topi;
  mb.topw = (uint16_t*)topw;
  launch_route_topk(router_logits, logits_dtype, T, E, dtype, mb, L, (hipStream_t)stream);
  return launch_status();
}

extern "C" int kbh_qmoe(const void* x, const int8_t* qweight, const void* scales,
                        const void* router_logits, int logits_dtype, void* y, void* workspace,
                        size_t workspace_bytes, int T, int D, int N, int E, int group, int dtype,
                        void* stream) {
  using namespace kbh;
  if (!x || !qweight || !scales || !router_logits || !y || !workspace) return KBH_ERR_NULL;
  if (dtype != KBH_F16 && dtype != KBH_BF16) return KBH_ERR_DTYPE;
  if (logits_dtype < 0 || logits_dtype > 2) return KBH_ERR_DTYPE;
  if (!moe_shape_ok(T, E, D, N, group)) return KBH_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(qweight) || !aligned16(scales) || !aligned16(y)) return KBH_ERR_ALIGN;
  const MoeLayout L = moe_layout(T, E, 0, N, 0, 0, 2, true);
  if (workspace_bytes < L.total) return KBH_ERR_WORKSPACE;
  const MoeBuffers mb = moe_buffers(workspace, L);
  hipStream_t st = (hipStream_t)stream;
  void* o = (char*)workspace + L.o;
  const bool bf = dtype == KBH_BF16;
  launch_route_topk(router_logits, logits_dtype, T, E, dtype, mb, L, st);
  const size_t n = (size_t)T * N;
  const dim3 cgrid((unsigned)((n / 4 + 255) / 256));
  if (bf) {
    launch_qmoe_gemm<true>(L, x, mb, qweight, scales, o, D, N, group, st);
    hipLaunchKernelGGL(moe_combine_f32_kernel<true>, cgrid, dim3(256), 0, st, (const float*)o,
                       mb.topw32, (uint16_t*)y, T, N);
  } else {
    launch_qmoe_gemm<false>(L, x, mb, qweight, scales, o, D, N, group, st);
    hipLaunchKernelGGL(moe_combine_f32_kernel<false>, cgrid, dim3(256), 0, st, (const float*)o,
                       mb.topw32, (uint16_t*)y, T, N);
  }
  return launch_status();
}

extern "C" size_t kbh_qmoe_ffn_workspace_bytes(int T, int D, int F, int E) {
  if (T <= 0 || E <= 0) return 0;
  // The group size is not an argument here: size for the largest layout over the allowed
  // groups (the split count of the down projection, hence its partials, depends on it).
  size_t best = 0;
  for (int group : {32, 64, 128, 256}) {
    bool wide;
    kbh::FfnPlan fp;
    const size_t b = kbh::ffn_layout(T, E, D, F, group, &wide, &fp).total;
    best = b > best ? b : best;
  }
  return best;
}

extern "C" int kbh_qmoe_ffn(const void* x, const void* router_logits, int logits_dtype,
                            const int32_t* gate_qweight, const void* gate_scales,
                            const void* gate_zeros, const int32_t* up_qweight,
                            const void* up_scales, const void* up_zeros,
                            const int32_t* down_qweight, const void* down_scales,
                            const void* down_zeros, void* y, void* workspace,
                            size_t workspace_bytes, int T, int D, int F, int E, int group,
                            int dtype, void* stream) {
  using namespace kbh;
  if (!x || !router_logits || !gate_qweight || !gate_scales || !gate_zeros || !up_qweight ||
      !up_scales || !up_zeros || !down_qweight || !down_scales || !down_zeros || !y || !workspace)
    return KBH_ERR_NULL;
  if (dtype != KBH_F16 && dtype != KBH_BF16) return KBH_ERR_DTYPE;
  if (logits_dtype < 0 || logits_dtype > 2) return KBH_ERR_DTYPE;
  if (!moe_shape_ok(T, E, D, F, group) || !moe_shape_ok(T, E, F, D, group)) return KBH_ERR_SHAPE;
  const void* ptrs[] = {x, gate_qweight, gate_scales, gate_zeros, up_qweight, up_scales, up_zeros,
                        down_qweight, down_scales, down_zeros, y};
  for (const void* p : ptrs)
    if (!aligned16(p)) return KBH_ERR_ALIGN;
  bool wide;
  FfnPlan fp;
  const MoeLayout L = ffn_layout(T, E, D, F, group, &wide, &fp);
  if (workspace_bytes < L.total) return KBH_ERR_WORKSPACE;
  const MoeBuffers mb = moe_buffers(workspace, L);
  hipStream_t st = (hipStream_t)stream;
  void* h = (char*)workspace + L.h;
  void* o = (char*)workspace + L.o;
  const bool bf = dtype == KBH_BF16;
  launch_route_topk(router_logits, logits_dtype, T, E, dtype, mb, L, st);
  // gate/up: [D -> F] packed along F; down: [F -> D] packed along D
  const size_t gq = (size_t)D * (F / 8), gs = (size_t)(D / group) * F;
  const size_t dq = (size_t)F * (D / 8), ds = (size_t)(F / group) * D;
  if (wide) {
    float* part = (float*)((char*)workspace + L.part);
    if (bf)
      launch_ffn_wide<true>(fp, L, mb, x, gate_qweight, gate_scales, gate_zeros, up_qweight,
                            up_scales, up_zeros, down_qweight, down_scales, down_zeros, h, o, part,
                            y, T, D, F, group, gq, gs, dq, ds, st);
    else
      launch_ffn_wide<false>(fp, L, mb, x, gate_qweight, gate_scales, gate_zeros, up_qweight,
                             up_scales, up_zeros, down_qweight, down_scales, down_zeros, h, o,
                             part, y, T, D, F, group, gq, gs, dq, ds, st);
    return launch_status();
  }
#define KBH_FFN(BF)                                                                              \
  {                                                                                              \
    const W4SlabPolicy<BF> gp{(const uint32_t*)gate_qweight, (const uint16_t*)gate_scales,       \
                              (const uint16_t*)gate_zeros, F, group, gq, gs};                    \
    const W4SlabPolicy<BF> upp{(const uint32_t*)up_qweight, (const uint16_t*)up_scales,         \
                               (const uint16_t*)up_zeros, F, group, gq, gs};                     \
    const W4SlabPolicy<BF> dp{(const uint32_t*)down_qweight, (const uint16_t*)down_scales,       \
                              (const uint16_t*)down_zeros, D, group, dq, ds};                    \
    launch_moe_gemm<BF, W4SlabPolicy<BF>, true, true, false>(L, x, D, mb, gp, upp, h, F, F, D, st); \
    launch_moe_gemm<BF, W4SlabPolicy<BF>, false, false, true>(L, h, F, mb, dp, dp, o, D, D, F, st); \
    launch_combine<BF>(o, mb.topw, y, T, D, st);                                                  \
  }
  if (bf) KBH_FFN(true) else KBH_FFN(false)
#undef KBH_FFN
  return launch_status();
}

extern "C" size_t kbh_moe_workspace_bytes(int T, int D, int H, int E, int topk) {
  (void)D;
  if (T <= 0 || E <= 0 || topk < 1 || topk > kbh::kMoeMaxTopk) return 0;
  return kbh::moe_layout(T, E, 0, H, 0, 0, topk).total;
}

extern "C" int kbh_moe_route_topk(const void* router_logits, int logits_dtype, int32_t* topi,
                                  void* topw, void* workspace, size_t workspace_bytes, int T,
                                  int E, int topk, int dtype, void* stream) {
  using namespace kbh;
  if (!router_logits || !topi || !topw || !workspace) return KBH_ERR_NULL;
  if (logits_dtype < 0 || logits_dtype > 2 ||
      (dtype != KBH_F16 && dtype != KBH_BF16 && dtype != KBH_F32))
    return KBH_ERR_DTYPE;
  if (T < 1 || E < 2 || E > kMoeMaxExperts || topk < 1 || topk > kMoeMaxTopk || topk > E)
    return KBH_ERR_SHAPE;
  const MoeLayout L = moe_layout(T, E, 0, 0, 0, 0, topk);
  if (workspace_bytes < L.total) return KBH_ERR_WORKSPACE;
  MoeBuffers mb = moe_buffers(workspace, L);
  mb.topi = topi;
  mb.topw = (uint16_t*)topw;
  launch_route_topk(router_logits, logits_dtype, T, E, dtype, mb, L, (hipStream_t)stream);
  return launch_status();
}

extern "C" int kbh_moe(const void* x, const void* w, const void* router_logits, int logits_dtype,
                       void* y, void* workspace, size_t workspace_bytes, int T, int D, int H, int E,
                       int topk, int dtype, void* stream) {
  using namespace kbh;
  if (!x || !w || !router_logits || !y || !workspace) return KBH_ERR_NULL;
  if (dtype != KBH_F16 && dtype != KBH_BF16) return KBH_ERR_DTYPE;
  if (logits_dtype < 0 || logits_dtype > 2) return KBH_ERR_DTYPE;
  if (!moe_shape_ok(T, E, D, H, 128) || topk < 1 || topk > kMoeMaxTopk || topk > E)
    return KBH_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(w) || !aligned16(y)) return KBH_ERR_ALIGN;
  const MoeLayout L = moe_layout(T, E, 0, H, 0, 0, topk);
  if (workspace_bytes < L.total) return KBH_ERR_WORKSPACE;
  const MoeBuffers mb = moe_buffers(workspace, L);
  hipStream_t st = (hipStream_t)stream;
  void* o = (char*)workspace + L.o;
  const bool bf = dtype == KBH_BF16;
  launch_route_topk(router_logits, logits_dtype, T, E, dtype, mb, L, st);
  const F16SlabPolicy bp{(const uint16_t*)w, H, (size_t)D * H};
  const size_t n4 = (size_t)T * H / 4;
  const dim3 cgrid((unsigned)((n4 + 255) / 256));
  const size_t S = (size_t)T * topk;
  // Experts averaging 96 or more routed rows: 128-row expert tiles of 256 columns on the
  // warp-specialised kernel (x staged through LDS, 32-bit offsets; bit-identical to the grouped
  // kernel). Measured at T=512 (graph-replayed): grok1 295 -> 275 us, mixtral 411 -> 409; at 64
  // rows per expert (qwen2_57b top-8) 313 -> 324, so those stay on the grouped kernel.
  if (L.bm == 128 && S >= (size_t)96 * E && H % 256 == 0 && D % 128 == 0 &&
      S * D * 2 < ((size_t)1 << 31)) {
    const F16WidePolicy wp{(const uint16_t*)w, H, (size_t)D * H};
    using RM = GroupedRows<true, true>;
    const RM rm{mb.tiles, mb.perm, topk};
    const dim3 grid((unsigned)(L.max_tiles * (H / 256)));
    if (bf)
      hipLaunchKernelGGL((tiled_ws_gemm<WideHalf<true>, 128, 2, 1, F16WidePolicy, HalfOut<true>, RM,
                                        4, 1, true>),
                         grid, dim3(512), 0, st, x, wp, HalfOut<true>{(uint16_t*)o, H},
                         (float*)nullptr, (int)S, H, D, 1, D / 32, rm);
    else
      hipLaunchKernelGGL((tiled_ws_gemm<WideHalf<false>, 128, 2, 1, F16WidePolicy, HalfOut<false>,
                                        RM, 4, 1, true>),
                         grid, dim3(512), 0, st, x, wp, HalfOut<false>{(uint16_t*)o, H},
                         (float*)nullptr, (int)S, H, D, 1, D / 32, rm);
    if (bf)
      hipLaunchKernelGGL(moe_combine_k_kernel<true>, cgrid, dim3(256), 0, st, (const uint16_t*)o,
                         mb.topw, (uint16_t*)y, T, H, topk);
    else
      hipLaunchKernelGGL(moe_combine_k_kernel<false>, cgrid, dim3(256), 0, st, (const uint16_t*)o,
                         mb.topw, (uint16_t*)y, T, H, topk);
    return launch_status();
  }
  if (bf) {
    launch_moe_gemm<true, F16SlabPolicy, true, false, true>(L, x, D, mb, bp, bp, o, H, H, D, st);
    hipLaunchKernelGGL(moe_combine_k_kernel<true>, cgrid, dim3(256), 0, st, (const uint16_t*)o,
                       mb.topw, (uint16_t*)y, T, H, topk);
  } else {
    launch_moe_gemm<false, F16SlabPolicy, true, false, true>(L, x, D, mb, bp, bp, o, H, H, D, st);
    hipLaunchKernelGGL(moe_combine_k_kernel<false>, cgrid, dim3(256), 0, st, (const uint16_t*)o,
                       mb.topw, (uint16_t*)y, T, H, topk);
  }
  return launch_status();
}
