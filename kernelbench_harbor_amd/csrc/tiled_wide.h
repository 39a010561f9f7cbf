// Wide-tile MFMA GEMM for large M with a pluggable weight-slab producer and output policy.
//
// y[M, N] = x[M, K] @ W[K, N] with x and W in fp16/bf16 (E = WideHalf) or int8 (E = WideI8);
// a slab is 64 bytes of K per row (32 fp16 or 64 int8 elements), i.e. two 32x32 MFMA k-steps of
// 16 bytes per lane, and W is produced one 64-byte x TN slab at a time by a policy from its
// packed/quantized storage. The output policy (EP) turns fp32 or exact int32 sums into the
// output format. One 256-thread workgroup owns a TM x TN output tile
// and one K range (split-K); the tile is sized so that two workgroups fit on a CU (<= 128
// accumulator and <= 128 other VGPRs per lane), which lets one workgroup's MFMAs run while the
// other waits on memory or a barrier:
//  * x is not shared through LDS: each wave loads its own rows' MFMA A fragments straight from
//    global memory (16 bytes per lane per 32x16 fragment), PD slabs ahead of their use; int8
//    (WideI8) loads the same rows in a coalesced pattern and reorders them through a private
//    LDS buffer of the wave (XS in the kernel).
//  * The weight slab is dequantized once per workgroup into LDS in MFMA B-fragment order
//    (wide_b_offset), so a fragment read is one conflict-free ds_read_b128 per wave.
//  * WM x (4/WM) waves, each (TM/WM) x (TN*WM/4) with 32x32x16 MFMAs; accumulators in AGPRs.
//  * Per slab, one barrier: B fragments of k16 step 1 are read before the step-0 MFMAs, the next
//    slab's weights are dequantized and written in parts between the step-0 MFMAs, and the next
//    slab's step-0 fragments are read after the barrier while the step-1 MFMAs run, interleaved
//    with the next global loads.
//  * Per-group constants of the weight format (scales, zero points) are loaded once per
//    quantization group into one of two register sets; the loop is unrolled over two groups
//    (2*SPG slabs, SPG = slabs per group), so the set in use is known at compile time and no
//    register copies are needed.
//  * Split-K (splits > 1): partial tiles go to per-split slices of a workspace (plain stores of
//    E::Part: fp32, or int32 which sums exactly), summed in split order by wide_reduce_kernel.
//  * Workgroup ids are remapped so that each XCD runs consecutive ids, which are the column
//    tiles of consecutive row blocks in one K range: its L2 then serves both the x rows the
//    column tiles share and the weight slabs the row blocks share (the order (split, row block,
//    column block) measured 65 vs 71 us on W8A8 M=512 and 288 vs 299 us on W4A16 M=2048 against
//    (row block, split, column block), whose weight slabs each XCD fetched separately).
//
// Output policy (EP): void emit(int r, int n, E::Part v) const; one output element, and
//   void emit4(int r, int n, vec4 v) const; four consecutive outputs of one row (n % 4 == 0).
//   A paired policy (EP::kPaired, one wave column) instead receives emit_pair(r, n, a, b): each
//   128 virtual columns 128c.. of the tile hold 64 columns of a first matrix, then the same 64
//   columns of a second one (a paired weight policy fills them), and virtual columns
//   128c + v, 128c + 64 + v (v < 64) become output column n = n0/2 + 64c + v.
//
// Row map (RM): tile(mb) -> {first row, rows, expert}; a_row(tile, r) the x row feeding tile row
//   r; out_row(tile, r) the output row of tile row r. DenseRows is the plain GEMM; GroupedRows
//   walks an expert tile table (mixture of experts). A tile with rows == 0 does nothing.
//
// Policy interface (BP), for 256 threads and a (E::kSlabK) x TN slab:
//   struct Raw;  struct Grp;                            per-thread slab data / group constants
//   static constexpr int kTN, kParts;
//   void load(Raw&, int k0, int n0, int t) const;       issue the slab's global loads
//   void load_group(Grp&, int k0, int n0, int t) const; constants of the group holding row k0
//   void prepare_group(Grp&) const;                     once per group, before its first slab's
//                                                       store_part (its loads have arrived)
//   void store_part(const Raw&, const Grp&, uint8_t* Bs, int t, int p) const;
//                                                       part p < kParts of the slab into LDS
//   The LDS byte offset of byte kb (= k * element size) of column n of the slab is
//   wide_b_offset<kTN>(kb, n).
#pragma once

#include "kbh_common.h"

namespace kbh {

constexpr int WSLAB_BYTES = 64;  // bytes of K per row per slab

template <bool B>
struct WideFlag {
  static constexpr bool value = B;
};

// Element traits: MFMA and accumulator types of the two operand families.
template <bool BF16>
struct WideHalf {
  using Acc = kbh_f32x16;
  using Part = float;
  using Part4 = kbh_f32x4;
  static constexpr int kSlabK = 32;  // K elements per slab
  static constexpr bool kStageX = false;  // x fragments straight from global memory
  __device__ static Acc mma(kbh_u32x4 a, kbh_u32x4 b, Acc c) { return mfma32x32x16<BF16>(a, b, c); }
};
struct WideI8 {
  using Acc = kbh_i32x16;
  using Part = int;
  using Part4 = kbh_i32x4;
  static constexpr int kSlabK = 64;
  static constexpr bool kStageX = true;  // x through a per-wave LDS buffer (XS below)
  // 32x32x32 int8: lane l holds A[row l%32][k 16(l/32)..+16], B[k 16(l/32)..+16][col l%32].
  __device__ static Acc mma(kbh_u32x4 a, kbh_u32x4 b, Acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(kbh_i32x4, a),
                                                 __builtin_bit_cast(kbh_i32x4, b), c, 0, 0, 0);
  }
};

// Column slot within a slab: columns are permuted within groups of 8 (slot = 8q + ((n ^ f(q)) &
// 7), q = n/8, f(q) = q ^ (q >> 3)) so that producer writes, which step through packed words 8
// columns apart, spread over all LDS banks.
__device__ __host__ inline int wide_slot(int n) {
  const int q = n >> 3;
  return (n & ~7) | ((n ^ q ^ (q >> 3)) & 7);
}
// Byte offset of byte kb (< 64) of the K run of column n (< TN) in a slab buffer: [k-step (32
// bytes)][lane half (16 bytes)][column slot][16 bytes]. The 16 bytes of one column that a lane
// feeds to an MFMA are one chunk and the 32 lanes of a fragment read 512 contiguous bytes.
template <int TN>
__device__ __host__ inline int wide_b_offset(int kb, int n) {
  return (kb >> 5) * (TN * 32) + ((kb >> 4) & 1) * (TN * 16) + wide_slot(n) * 16 + (kb & 15);
}

struct DenseRows {
  int M;
  struct Tile {
    int m0, rows, expert;
  };
  __device__ Tile tile(int mb, int TM) const { return Tile{mb * TM, min(TM, M - mb * TM), 0}; }
  __device__ int a_row(const Tile& ti, int r) const { return ti.m0 + min(r, ti.rows - 1); }
  __device__ int out_row(const Tile& ti, int r) const { return ti.m0 + r; }
};

// Tile mb of the table {expert, first slot, rows}; slot s reads x row perm[s] / topk (GATHER;
// perm[s] = topk * token + k) or row s, and writes output row perm[s] (PERM_OUT) or row s.
template <bool GATHER, bool PERM_OUT>
struct GroupedRows {
  const int* tiles;
  const int* perm;
  int topk = 2;
  struct Tile {
    int s0, rows, expert;
  };
  __device__ Tile tile(int mb, int) const {
    const int* p = tiles + 3 * mb;
    return Tile{p[1], p[2], p[0]};
  }
  __device__ int a_row(const Tile& ti, int r) const {
    const int s = ti.s0 + min(r, ti.rows - 1);
    return GATHER ? (topk == 2 ? (perm[s] >> 1) : perm[s] / topk) : s;
  }
  __device__ int out_row(const Tile& ti, int r) const {
    const int s = ti.s0 + r;
    return PERM_OUT ? perm[s] : s;
  }
};

template <int TM, int TN, int WM>
struct WideShape {
  static constexpr int WN = 4 / WM;
  static constexpr int RB = TM / (32 * WM);  // 32-row MFMA blocks per wave
  static constexpr int CB = TN / (32 * WN);  // 32-column MFMA blocks per wave
  static_assert(RB >= 1 && CB >= 1 && WM * WN == 4, "tile shape");
  // Two workgroups per CU when the accumulators fit in 128 registers per lane.
  static constexpr int kMinBlocks = RB * CB <= 8 ? 2 : 1;
};

// A wave's accumulators ((TM/WM) x (TN*WM/4) of the tile at row block wm, column block wn)
// through the output policy (splits == 1, or a paired policy) or into this split's slice of the
// workspace (plain stores; wide_reduce_kernel sums the slices afterwards, ordered by the launch
// boundary, so no device-scope fences or atomics are needed and the sum order is fixed).
// Accumulator element e of tile (i, j): row 8(e/4) + 4(lane/32) + e%4, column lane%32.
template <class E, int TM, int WM, int TN, class EP, class RM, int RB, int CB>
__device__ inline void wide_store_tile(const typename E::Acc (&acc)[RB][CB], const EP& ep,
                                       const RM& rm, const typename RM::Tile& ti,
                                       typename E::Part* __restrict__ ws, int split, int splits,
                                       int M, int N, int n0, int wm, int wn, int lane) {
  constexpr int WN = 4 / WM;
  const int fr = lane & 31, fg = lane >> 5;
  const int rbase = wm * (TM / WM) + 4 * fg;
  const int cbase = n0 + wn * 32 * CB + fr;
  if constexpr (EP::kPaired) {
    static_assert(WN == 1 && CB % 4 == 0, "paired output needs whole 128-column chunks per wave");
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j) {
        if ((j & 3) >= 2) continue;  // second-matrix blocks pair with block j - 2
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
          if (r < ti.rows)
            ep.emit_pair(rm.out_row(ti, r), n0 / 2 + 64 * (j >> 2) + 32 * (j & 1) + fr,
                         acc[i][j][e], acc[i][j + 2][e]);
        }
      }
  } else if (splits == 1) {
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
          if (r < ti.rows) ep.emit(rm.out_row(ti, r), cbase + 32 * j, acc[i][j][e]);
        }
  } else {
    typename E::Part* part = ws + (size_t)split * M * N;
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = rbase + 32 * i + 8 * (e >> 2) + (e & 3);
          if (r < ti.rows) part[(size_t)rm.out_row(ti, r) * N + cbase + 32 * j] = acc[i][j][e];
        }
  }
}

// M: output rows (the size of a split-K slice); N: output columns of the weight producer (TN
// per tile; paired producers: twice the real output columns).
// MINB: workgroups per CU the register allocation must allow (0: the shape's default).
// PD: prefetch depth in slabs. x fragments and raw weights are requested PD slabs before their
//   use; loads complete in issue order, so PD is the latency budget of the whole stream.
template <class E, int TM, int WM, int SPG, class BP, class EP, class RM = DenseRows, int MINB = 0,
          int PD = 2>
__global__ __launch_bounds__(256, (MINB ? MINB : WideShape<TM, BP::kTN, WM>::kMinBlocks)) void
tiled_wide_gemm(
    const void* __restrict__ x, BP bp, EP ep, typename E::Part* __restrict__ ws, int M, int N,
    int K, int splits, int slabs_per_split, RM rm) {
  constexpr int TN = BP::kTN;
  constexpr int SK = E::kSlabK;
  constexpr int EB = WSLAB_BYTES / SK;  // bytes per element
  using Shape = WideShape<TM, TN, WM>;
  constexpr int RB = Shape::RB, CB = Shape::CB, WN = Shape::WN;
  constexpr int SLAB = TN * 64;  // LDS bytes per slab buffer
  // Slabs per loop iteration: two groups, and a multiple of the prefetch ring.
  constexpr int U = 2 * SPG > PD ? 2 * SPG : PD;
  static_assert(U % PD == 0 && U % (2 * SPG) == 0, "prefetch depth and group parity");
  __shared__ __attribute__((aligned(16))) uint8_t Bs[2][SLAB];

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int NB = N / TN;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int nb = id % NB;
  const int rest = id / NB;
  const int MB = gridDim.x / (NB * splits);  // row blocks (tile-table entries)
  const int mb = rest % MB;
  const int split = rest / MB;
  const int n0 = nb * TN;
  const int kt0 = split * slabs_per_split;
  const int KT = slabs_per_split;
  const typename RM::Tile ti = rm.tile(mb, TM);
  if (ti.rows <= 0) return;  // unused tile-table entry (uniform across the workgroup)
  bp = bp.at_expert(ti.expert);

  // A fragments: lane (r = lane%32, g = lane/32) of row block rb holds tile row
  // wm*TM/WM + 32rb + r, bytes 32*step + 16g .. +16 of the slab's 64-byte K run.
  const int fr = lane & 31, fg = lane >> 5;
  // XS (E::kStageX, one wave per row stripe): x reaches the fragments through a private LDS
  // double buffer of the wave. Its global loads cover 16 rows x 64 bytes each (four lanes per
  // row) instead of a fragment's 32 rows x 32 bytes, halving the cache lines per load; the wave
  // then writes the rows into its LDS slot and reads them back in fragment order. Row q of the
  // slot keeps 16-byte chunk c at q*64 + 16*(c ^ ((q >> 1) & 3)): the writes (4 lanes per row)
  // and the fragment reads (one chunk of 8 consecutive rows per 8 lanes) are both conflict free.
  // Measured: int8 W8A8 M=512 65 -> 60 us; fp16 W4A16 M=256..2048 and the MoE FFN 0-3% slower
  // (their 32-deep slabs carry half the x bytes per MFMA), so only WideI8 stages.
  constexpr bool XS = WN == 1 && E::kStageX;
  constexpr int XR = TM / WM;                  // rows of one wave's stripe
  constexpr int XSLOT = XR * WSLAB_BYTES;      // LDS bytes of one slab of the stripe
  __shared__ __attribute__((aligned(16))) uint8_t Xs[XS ? 4 * 2 * XSLOT : 16];
  uint8_t* const xw = Xs + (XS ? wave * 2 * XSLOT : 0);
  const uint8_t* xrow[2 * RB];
#pragma unroll
  for (int q = 0; q < 2 * RB; ++q) {
    if constexpr (XS) {
      if (q >= XR / 16) continue;
      const int r = wm * XR + 16 * q + (lane >> 2);  // rows past the tile re-read its last row
      xrow[q] = (const uint8_t*)x + (size_t)rm.a_row(ti, r) * K * EB + 16 * (lane & 3);
    } else {
      if (q >= RB) continue;
      const int r = wm * (TM / WM) + q * 32 + fr;
      xrow[q] = (const uint8_t*)x + (size_t)rm.a_row(ti, r) * K * EB + fg * 16;
    }
  }
  struct AStage {
    kbh_u32x4 a[RB][2];  // XS: a[rb][s] = 16-row load 2rb + s of the stripe
  };
  auto load_a_step = [&](AStage& st, int kt, int s) {
    if constexpr (XS) {
      const size_t b0 = (size_t)(kt0 + kt) * WSLAB_BYTES;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        st.a[rb][s] = *reinterpret_cast<const kbh_u32x4*>(xrow[2 * rb + s] + b0);
    } else {
      const size_t b0 = (size_t)(kt0 + kt) * WSLAB_BYTES + 32 * s;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        st.a[rb][s] = *reinterpret_cast<const kbh_u32x4*>(xrow[rb] + b0);
    }
  };
  auto xs_chunk = [](int q, int c) { return q * WSLAB_BYTES + 16 * (c ^ ((q >> 1) & 3)); };
  // XS: one slab of the stripe from the load ring into LDS slot `slot`.
  auto stage_a = [&](const AStage& st, int slot) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        *reinterpret_cast<kbh_u32x4*>(xw + slot * XSLOT + xs_chunk(16 * (2 * rb + h) + (lane >> 2), lane & 3)) = st.a[rb][h];
  };
  // Fragments of k16 step s of the slab in registers (no XS) or in LDS slot `slot` (XS).
  auto frag_a = [&](kbh_u32x4 (&af)[RB], const AStage& st, int slot, int s) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      if constexpr (XS)
        af[rb] = *reinterpret_cast<const kbh_u32x4*>(xw + slot * XSLOT + xs_chunk(32 * rb + fr, 2 * s + fg));
      else
        af[rb] = st.a[rb][s];
    }
  };
  auto load_b = [&](typename BP::Raw& r, int kt) { bp.load(r, (kt0 + kt) * SK, n0, t); };
  auto load_g = [&](typename BP::Grp& g, int kt) { bp.load_group(g, (kt0 + kt) * SK, n0, t); };

  // B fragment of step s, column block j of this wave: lane (c = lane%32, g) reads column
  // wn*32CB + 32j + c, bytes 32s + 16g .. +16.
  int boff[CB];
#pragma unroll
  for (int j = 0; j < CB; ++j) boff[j] = wide_b_offset<TN>(16 * fg, wn * 32 * CB + 32 * j + fr);
  auto read_b = [&](kbh_u32x4 (&bf)[CB], int buf, int s) {
#pragma unroll
    for (int j = 0; j < CB; ++j)
      bf[j] = *reinterpret_cast<const kbh_u32x4*>(&Bs[buf][boff[j] + s * (TN * 32)]);
  };

  typename E::Acc acc[RB][CB];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

  auto mma = [&](const kbh_u32x4 (&af)[RB], const kbh_u32x4 (&bf)[CB]) {
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j) acc[i][j] = E::mma(af[i], bf[j], acc[i][j]);
  };
  // MFMAs q in [lo, hi) of a k16 step (q = CB*i + j).
  auto mma_range = [&](const kbh_u32x4 (&af)[RB], const kbh_u32x4 (&bf)[CB], int lo, int hi) {
#pragma unroll
    for (int q = 0; q < RB * CB; ++q)
      if (q >= lo && q < hi)
        acc[q / CB][q % CB] = E::mma(af[q / CB], bf[q % CB], acc[q / CB][q % CB]);
  };

  // FAST: the policy's faster producer path, valid when every weight constant of this
  // workgroup's K range and columns allows it (one check before the loop, then a separate copy
  // of the loop, so the loop itself has no branch). The 64- and 128-row tiles take it: there
  // the producer is on the critical path (measured on 256-column tiles, which now run on
  // tiled_ws_gemm: W4A16 M=256 57 -> 55 us, MoE FFN 993 -> 974 us); with 256-row tiles the
  // second copy of the loop spilled registers and ran no faster.
  constexpr bool kFast = BP::kHasFast && (TM == 64 || TM == 128);
  bool fast = false;
  if constexpr (kFast) fast = __syncthreads_and(bp.scan_fast(kt0 * SK, (kt0 + KT) * SK, n0, t)) != 0;
  auto run = [&](auto fast_tag) {
    constexpr bool FAST = decltype(fast_tag)::value;
    // Prologue: slab 0 in LDS, step-0 fragments of slab 0 in registers, A of slabs 0..PD-1, raw
    // weights of slabs 1..PD and the constants of the second group in flight. Ring slot s % PD
    // holds the A fragments of slab s and the raw weights of slab s (consumed during slab s - 1).
    AStage A[PD];
    typename BP::Raw R[PD];
    typename BP::Grp G[2];  // constants of groups with even / odd index within the K range
    const int last = KT - 1;
    load_b(R[0], 0);
    load_g(G[0], 0);
#pragma unroll
    for (int i = 0; i < PD; ++i)
#pragma unroll
      for (int st = 0; st < 2; ++st) load_a_step(A[i], min(i, last), st);
    bp.template prepare_group<FAST>(G[0]);
#pragma unroll
    for (int p = 0; p < BP::kParts; ++p) bp.template store_part<FAST>(R[0], G[0], Bs[0], t, p);
#pragma unroll
    for (int i = 1; i <= PD; ++i) load_b(R[i % PD], min(i, last));
    load_g(G[1], min(SPG, last));
    constexpr int NP = BP::kParts;
    kbh_u32x4 a0[RB], a1[RB];  // A fragments of step 0 (of the slab after next's barrier) / 1
    if constexpr (XS) stage_a(A[0], 0);
    __syncthreads();
    kbh_u32x4 b0[CB], b1[CB];
    read_b(b0, 0, 0);
    frag_a(a0, A[0], 0, 0);

    // Steady state: KT is a multiple of U; loads past the end re-read the last slab or group
    // (never used), so the loop body is branch-free. Slab s+1, dequantized during slab s, belongs
    // to group (u+1)/SPG of the iteration (register set ((u+1)/SPG) & 1); when it starts a group,
    // the set of the group just finished is reloaded with the group after next. The order inside
    // a slab is fixed with scheduling barriers (the scheduler otherwise clusters the
    // dequantisation and moves MFMAs across s_barrier).
    constexpr int NMF = RB * CB;  // MFMAs per k16 step
    for (int kt = 0; kt < KT; kt += U) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int s = kt + u;  // slab in registers / LDS buffer u&1
        const int cur = u & 1;
        const int ra = u % PD, rr = (u + 1) % PD;  // ring slots of slab s (A) and s+1 (raw)
        const bool new_group = (u + 1) % SPG == 0;  // slab s+1 starts a group
        const int gsel = ((u + 1) / SPG) & 1;
        read_b(b1, cur, 1);
        frag_a(a1, A[ra], u & 1, 1);
        if (new_group) bp.template prepare_group<FAST>(G[gsel]);  // slab s+1 starts set gsel's group
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          mma_range(a0, b0, p * NMF / NP, (p + 1) * NMF / NP);
          __builtin_amdgcn_sched_barrier(0);
          bp.template store_part<FAST>(R[rr], G[gsel], Bs[1 - cur], t, p);  // slab s+1 (after last: unused)
          __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();  // s_barrier alone does not stop MFMAs moving across: fenced both sides
        __builtin_amdgcn_sched_barrier(0);
        read_b(b0, 1 - cur, 0);  // step 0 of slab s+1
        // XS: slab s+1 from its ring slot into the wave's other LDS slot (slab s-1's, read in the
        // previous iteration), then its step-0 fragments.
        if constexpr (XS) stage_a(A[(u + 1) % PD], (u + 1) & 1);
        frag_a(a0, A[(u + 1) % PD], (u + 1) & 1, 0);
        mma(a1, b1);
        load_a_step(A[ra], min(s + PD, last), 0);
        load_b(R[rr], min(s + 1 + PD, last));
        if (new_group) load_g(G[gsel ^ 1], min(s + 1 + SPG, last));
        load_a_step(A[ra], min(s + PD, last), 1);
        __builtin_amdgcn_sched_group_barrier(0x100, CB, 1);
#pragma unroll
        for (int i = 0; i < NMF; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 1);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  if constexpr (kFast) {
    if (fast) run(WideFlag<true>{});
    else run(WideFlag<false>{});
  } else {
    run(WideFlag<false>{});
  }

  wide_store_tile<E, TM, WM, TN>(acc, ep, rm, ti, ws, split, splits, M, N, n0, wm, wn, lane);
}

// Output = sum over splits of ws[split] (in split order), through the output policy. One thread
// per 4 consecutive outputs of a row (N % 4 == 0); n4 = M * N / 4.
template <class E, class EP>
__global__ __launch_bounds__(256) void wide_reduce_kernel(const typename E::Part* __restrict__ ws,
                                                          EP ep, int N, size_t n4, int splits) {
  using P4 = typename E::Part4;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  const P4 v = sum_slices(reinterpret_cast<const P4*>(ws) + i, n4, splits);
  const size_t e = 4 * i;
  const int r = (int)(e / (size_t)N);
  ep.emit4(r, (int)(e - (size_t)r * N), v);
}

// LDS-mode buffer loads issued as inline assembly (M0 = the LDS address), for kernels that wait
// for them with explicit vmcnt counts: the compiler does not track such loads, so it adds no
// waits for them (as a compiler builtin, every barrier after one became a wait for all of them).
// Lane i's 16 bytes land at LDS byte address lds + 16 i; the global offset is voff + soff within
// the buffer r (offsets are 32-bit; loads past the buffer's size read as zero).
typedef unsigned int kbh_rsrc4 __attribute__((ext_vector_type(4)));
__device__ inline kbh_rsrc4 raw_rsrc(const void* p, size_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  return kbh_rsrc4{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu,
                   bytes >= 0xffffffffu ? 0xffffffffu : (uint32_t)bytes, 0x00020000u};
}
__device__ inline uint32_t lds_addr(const void* p) {
  typedef __attribute__((address_space(3))) const void* lds_cptr;
  return (uint32_t)(uintptr_t)(lds_cptr)p;
}
// The m0 clobber is declared although clang reports m0 as reserved (-Winline-asm): the compiler
// sets m0 itself before each of its own m0 uses, and no kernel here keeps a value in m0 across
// these loads (every one of them sets m0 first).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ inline void lds_load16(uint32_t lds, uint32_t voff, kbh_rsrc4 r, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}
#pragma clang diagnostic pop

// Split-K plans keep their partial-sum slices within this many bytes (the writes and reads of
// more cost more than the extra splits gain, and it bounds the scratch a call needs).
constexpr size_t kWideMaxSliceBytes = (size_t)64 << 20;

// Launch geometry: grid = row blocks x column blocks x splits, ids ordered (split, row block,
// column block) so that consecutive ids, which share an XCD, share a K range.
struct WidePlan {
  int tm;               // 128 or 256
  int splits;           // K ranges
  int slabs_per_split;  // multiple of the loop unroll
  int grid;
};

// Picks the tile height and the split count. Up to small_upto rows (default 128) the tiles are
// tm_small rows high;
// above, 256 rows, or (choose_tm) tm_small rows when the cost estimate favours them, i.e. when
// 256-row tiles would leave CUs idle. `slots` is the number of workgroups the GPU runs at once
// (256 CUs x workgroups per CU). A split count is valid when it divides the K slabs into ranges
// of at least 8 slabs that are a multiple of `unroll`; among those, the plan minimises (waves of
// workgroups) x (slabs per workgroup), preferring fewer splits on a tie.
inline bool plan_wide(int M, int N, int K, int tn, int slab_k, int unroll, int slots,
                      WidePlan* p, int tm_small = 128, bool choose_tm = false,
                      int small_upto = 128) {
  if (N % tn != 0 || K % (unroll * slab_k) != 0 || M < 1) return false;
  const int KT = K / slab_k;
  // Plan for tile height tm; returns the estimated time in units of a third of a 128-row slab
  // (a 256-row slab measures about 4/3 of a 128-row one, ~1 us at the benchmark shapes), plus
  // the split-K slices: s slices of M x N 4-byte partial sums are written and read back, about
  // one unit per 2^18 of them (2 MiB of traffic at ~5 TB/s). Without that term the plan chose
  // 56 splits at M=384 (336 MiB of slices).
  auto plan_tm = [&](int tm, WidePlan* q) {
    q->tm = tm;
    const int tiles = ((M + tm - 1) / tm) * (N / tn);
    long best = -1;
    for (int s = 1; s <= KT / unroll; ++s) {
      if (KT % s != 0) continue;
      const int spp = KT / s;
      if (spp % unroll != 0 || (spp < 8 && s > 1)) continue;
      if (s > 1 && (size_t)s * M * N * 4u > kWideMaxSliceBytes) continue;
      const long waves = ((long)tiles * s + slots - 1) / slots;
      const long slices = s > 1 ? (long)s * M * N >> 18 : 0;
      const long cost = waves * spp * (tm == 256 ? 4 : 3) + slices;
      if (best < 0 || cost < best) {
        best = cost;
        q->splits = s;
        q->slabs_per_split = spp;
      }
    }
    q->grid = tiles * q->splits;
    return best;
  };
  if (M <= small_upto) {
    plan_tm(tm_small, p);
    return true;
  }
  const long c256 = plan_tm(256, p);
  if (choose_tm && tm_small != 256) {
    WidePlan q;
    if (plan_tm(tm_small, &q) < c256) *p = q;
  }
  return true;
}

// Workspace: `splits` slices of M x N 4-byte partial sums (none without split-K).
inline size_t wide_workspace_bytes(int M, int N, int splits) {
  return splits <= 1 ? 0 : round_up((size_t)splits * M * N * 4u, 256);
}

}  // namespace kbh
