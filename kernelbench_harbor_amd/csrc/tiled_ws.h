// Warp-specialised wide-tile GEMM for 64- and 128-row tiles (tiled_ws_gemm).
//
// The same computation, policies (weight producer BP, output EP, row map RM) and launch geometry
// as tiled_wide_gemm with fp16/bf16 operands, but a workgroup of 8 waves in two roles:
//  * waves 4..7 (256 threads, the policy's thread ids t = 0..255) only produce: they load the
//    packed weights PD slabs ahead, dequantize slab s + 2 into LDS buffer (s + 2) % 4 and load
//    the quantization groups' constants;
//  * waves 0..3 only consume: x fragments straight from global memory (PD slabs ahead; with XD,
//    128-row tiles, from an LDS x buffer the producers fill three slabs ahead), the B fragments
//    of slab s from LDS buffer s % 4 (and, before the slab's barrier, the step-0 fragments of
//    slab s + 1, which was completed one barrier earlier), and the MFMAs.
// One barrier per slab. Buffer (s + 3) % 4 is idle during slab s, so a producer write never
// meets a consumer read: in slab s the consumers read buffers s % 4 and (s + 1) % 4 and the
// producers write (s + 2) % 4. Each SIMD holds one wave of each role, so the dequantizing VALU
// work of one runs beside the MFMAs of the other, where the 4-wave kernel issued both from the
// same wave in turn. Both roles run their own loop of exactly KT barriers (plus the two of the
// set-up), so the barrier counts match by construction, and then meet again for the epilogue:
// split-K partial tiles go through the LDS ring, so that all 8 waves store whole rows.
// 64-row tiles run two producer sets (waves 4..7 and 8..11, PS below), each dequantizing one
// row pair of every thread's four rows.
// Measured against tiled_wide_gemm (same shapes, graph-replayed, bit-identical outputs): W4A16
// K=14336 N=4096 M=64 29.1 -> 27.3 us, M=128 38.0 -> 35.3, M=256 55.3 -> 50.4, M=384 84.8 ->
// 75.5, the Mixtral MoE SiLU FFN T=512 978 -> 864 us. Per-slab timestamps at M=256: the
// producers take ~1000-1200 cycles per slab against ~780 for the consumers' 16 MFMAs and reads
// (a dependent VALU instruction issues ~9.5 cycles after the one it waits for; see store_all).
#pragma once

#include "tiled_wide.h"

namespace kbh {

// Raw weights one producer thread holds per slab: the policy's whole share (one producer set) or
// its half (BP::RawHalf, two sets).
template <class BP, int PS>
struct WsRaw {
  using type = typename BP::Raw;
};
template <class BP>
struct WsRaw<BP, 2> {
  using type = typename BP::RawHalf;
};

// PS: producer sets. 1: waves 4..7 dequantize whole slabs. 2: waves 4..7 and 8..11 run the same
//   loop on the same thread ids and barriers, set p loading and dequantizing row pair p of each
//   thread's rows (BP::load_half / store_half), so two producer waves share each SIMD's VALU
//   with the MFMA wave (768 threads, at most 168 VGPRs per wave: 64-row tiles).
// XD: x through the LDS ring too (128-row tiles, one producer set): the producers stage each
//   slab's x rows with LDS-mode buffer loads three slabs ahead (as tiled_ws256_gemm does) and the
//   MFMA waves read their A fragments from LDS instead of holding a register ring of them. The
//   x offsets are 32-bit: the caller keeps M x K x 2 bytes under 2 GiB.
template <class E, int TM, int WM, int SPG, class BP, class EP, class RM = DenseRows, int PD = 4,
          int PS = 1, bool XD = false>
__global__ __launch_bounds__(256 * (1 + PS), 1) void tiled_ws_gemm(
    const void* __restrict__ x, BP bp, EP ep, typename E::Part* __restrict__ ws, int M, int N,
    int K, int splits, int slabs_per_split, RM rm) {
  constexpr int TN = BP::kTN;
  constexpr int SK = E::kSlabK;
  static_assert(!E::kStageX, "fp16/bf16 operands: x fragments straight from global memory");
  using Shape = WideShape<TM, TN, WM>;
  constexpr int RB = Shape::RB, CB = Shape::CB, WN = Shape::WN;
  constexpr int SLAB = TN * 64;  // LDS bytes per slab buffer
  constexpr int NBUF = 4;
  constexpr int U = 2 * SPG > PD ? 2 * SPG : PD;  // slabs per loop iteration
  static_assert(PD >= 2 && U % PD == 0 && U % (2 * SPG) == 0 && U % NBUF == 0, "unroll");
  static_assert(PS == 1 || PS == 2, "one or two producer sets");
  static_assert(!XD || (TM == 128 && PS == 1 && !E::kStageX), "LDS x: 128-row fp16 tiles");
  constexpr int NT = 256 * (1 + PS);  // threads
  __shared__ __attribute__((aligned(16))) uint8_t Bs[NBUF][SLAB];
  // XD: x of a slab, row r keeping its 16-byte chunk c at r * 64 + 16 (c ^ ((r >> 2) & 3)).
  __shared__ __attribute__((aligned(16))) uint8_t Xs[XD ? NBUF : 1][XD ? TM * 64 : 16];

  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
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
  const int last = KT - 1;
  const typename RM::Tile ti = rm.tile(mb, TM);
  if (ti.rows <= 0) return;  // unused tile-table entry (uniform across the workgroup)
  bp = bp.at_expert(ti.expert);

  typename E::Acc acc[RB][CB];  // the consumers' accumulators
  const bool producer = wave >= 4;
  // FAST: the policy's faster producer path when every weight constant of this workgroup's K
  // range and columns allows it. The producers scan and every wave takes part in the barrier
  // (one __syncthreads_and in each role's branch); both roles issue their set-up loads before
  // it, so that the scan's latency and theirs overlap.
  constexpr bool kFast = BP::kHasFast;
  const int fr = lane & 31, fg = lane >> 5;
  if (producer) {
    // ---- producers ----
    const int pset = PS == 1 ? 0 : (wave - 4) >> 2;            // producer set
    const int t = (int)threadIdx.x - 256 - 256 * pset;  // the policy's thread id
    using Raw = typename WsRaw<BP, PS>::type;
    auto load_b = [&](Raw& r, int s) {
      if constexpr (PS == 1) bp.load(r, (kt0 + min(s, last)) * SK, n0, t);
      else bp.load_half(r, (kt0 + min(s, last)) * SK, n0, t, pset);
    };
    auto load_g = [&](typename BP::Grp& g, int s) {
      bp.load_group(g, (kt0 + min(s, last)) * SK, n0, t);
    };
    // Ring slot s % PD holds the raw weights of slab s; constants of even / odd groups (index
    // within the K range) in G[0] / G[1], the next group's loaded one group ahead.
    // The zero points' first loads go out before the weights', so that they come back first
    // (measured at K=14336 N=4096: the scan's barrier passed 8.1k -> 6.9k cycles into the kernel
    // at M=64, 8.6k -> 6.8k at M=256; M=512 82.3 -> 81.3 us).
    typename BP::ScanPre sp;
    if constexpr (kFast) {
      if (pset == 0) bp.scan_load(sp, kt0 * SK, (kt0 + KT) * SK, n0, t);
    }
    Raw R[PD];
    typename BP::Grp G[2];
#pragma unroll
    for (int i = 0; i < PD; ++i) load_b(R[i], i);
    load_g(G[0], 0);
    load_g(G[1], SPG);
    // XD: producer wave p stages x blocks 2p and 2p + 1 (16 rows each) of every slab; lane l
    // takes row l / 4 of a block and the chunk the swizzle puts at position l % 4.
    uint32_t vxh[2] = {0u, 0u};
    kbh_rsrc4 rx = {0u, 0u, 0u, 0u};
    auto stage_x = [&](int s, int buf) {
      if constexpr (XD) {
        const uint32_t k0b = (uint32_t)((kt0 + min(s, last)) * WSLAB_BYTES);
#pragma unroll
        for (int h = 0; h < 2; ++h)
          lds_load16(lds_addr(&Xs[buf][1024 * (2 * (wave - 4) + h)]), vxh[h], rx, k0b);
      }
    };
    if constexpr (XD) {
      rx = raw_rsrc(x, (size_t)M * K * 2);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r = 16 * (2 * (wave - 4) + h) + (lane >> 2);
        vxh[h] = (uint32_t)((size_t)rm.a_row(ti, r) * K * 2) +
                 (uint32_t)(16 * ((lane & 3) ^ ((lane >> 4) & 3)));
      }
      stage_x(0, 0);
      stage_x(1, 1);
      stage_x(2, 2);
    }
    bool fast = false;
    if constexpr (kFast)
      fast = __syncthreads_and(pset == 0 ? (int)bp.scan_check(sp, kt0 * SK, (kt0 + KT) * SK, n0, t) : 1) != 0;
    auto produce = [&](auto fast_tag) {
      constexpr bool FAST = decltype(fast_tag)::value;
      auto put = [&](const Raw& r, const typename BP::Grp& g, uint8_t* b) {
        if constexpr (PS == 1) bp.template store_all<FAST>(r, g, b, t);
        else bp.template store_half<FAST>(r, g, b, t, pset);
      };
      bp.template prepare_group<FAST>(G[0]);
      put(R[0], G[0], Bs[0]);  // slab 0
      load_b(R[0], PD);
      if constexpr (SPG == 1) {  // slab 1 starts group 1; set 0 is reloaded with group 2
        bp.template prepare_group<FAST>(G[1]);
        load_g(G[0], 2);
        put(R[1], G[1], Bs[1]);
      } else {
        put(R[1], G[0], Bs[1]);
      }
      load_b(R[1 % PD], PD + 1);
      // XD: x of slabs 0 and 1 has landed (younger: slab 2's two x loads, the two raw-word
      // loads and at most one group load pair)
      if constexpr (XD) asm volatile("s_waitcnt vmcnt(10)" ::: "memory");
      __syncthreads();  // slabs 0 and 1 are in LDS
      // Slab kt + u + 2 during consumer slab kt + u. Slabs past the end re-produce the last one
      // into a buffer nobody reads, so the loop has no branch.
      for (int kt = 0; kt < KT; kt += U) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int pu = u + 2;
          const int set = (pu / SPG) & 1;
          if (pu % SPG == 0) {  // slab kt + pu starts a group: its set is ready, reload the other
            bp.template prepare_group<FAST>(G[set]);
            load_g(G[set ^ 1], kt + pu + SPG);
          }
          put(R[pu % PD], G[set], Bs[pu % NBUF]);
          stage_x(kt + u + 3, (u + 3) % NBUF);  // into the x buffer idle during slab kt + u
          load_b(R[pu % PD], kt + pu + PD);
          // XD: x of the next slab has landed (at least 16 loads are younger)
          if constexpr (XD) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
          __syncthreads();
        }
      }
    };
    if constexpr (kFast) {
      if (fast) produce(WideFlag<true>{});
      else produce(WideFlag<false>{});
    } else {
      produce(WideFlag<false>{});
    }
    if constexpr (XD) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // none past the loops
  } else {
    // ---- consumers ----
    const int wm = wave / WN, wn = wave % WN;
    // A fragments: lane (r = lane%32, g = lane/32) of row block rb holds tile row
    // wm*TM/WM + 32rb + r, bytes 32*step + 16g .. +16 of the slab's 64-byte K run.
    const uint8_t* xrow[RB];
#pragma unroll
    for (int q = 0; q < RB; ++q) {
      const int r = wm * (TM / WM) + q * 32 + fr;
      xrow[q] = (const uint8_t*)x + (size_t)rm.a_row(ti, r) * K * 2 + fg * 16;
    }
    struct AStage {
      kbh_u32x4 a[RB][2];
    };
    auto load_a = [&](AStage& st, int s) {
      if constexpr (!XD) {
        const size_t b0 = (size_t)(kt0 + min(s, last)) * WSLAB_BYTES;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            st.a[rb][h] = *reinterpret_cast<const kbh_u32x4*>(xrow[rb] + b0 + 32 * h);
      }
    };
    // XD: the fragment of k16 step h, chunk 2h + fg of row 32 wm + fr (RB = 1), from LDS
    int xoff[2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
      xoff[h] = (wm * (TM / WM) + fr) * 64 + 16 * ((2 * h + fg) ^ ((fr >> 2) & 3));
    auto read_a = [&](AStage& st, int buf) {
      if constexpr (XD) {
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            st.a[i][h] = *reinterpret_cast<const kbh_u32x4*>(&Xs[buf][xoff[h] + 2048 * i]);
      }
    };
    constexpr int PDA = XD ? 1 : PD;  // register ring of x fragments
    AStage A[PDA];  // slot s % PD holds the x fragments of slab s (XD: the current slab's)
#pragma unroll
    for (int i = 0; i < PDA; ++i) load_a(A[i], i);
    if constexpr (kFast) (void)__syncthreads_and(1);  // the producers' FAST barrier
    int boff[CB];
#pragma unroll
    for (int j = 0; j < CB; ++j) boff[j] = wide_b_offset<TN>(16 * fg, wn * 32 * CB + 32 * j + fr);
    auto read_b = [&](kbh_u32x4 (&bf)[CB], int buf, int s) {
#pragma unroll
      for (int j = 0; j < CB; ++j)
        bf[j] = *reinterpret_cast<const kbh_u32x4*>(&Bs[buf][boff[j] + s * (TN * 32)]);
    };

#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

    __syncthreads();  // slabs 0 and 1 are in LDS
    kbh_u32x4 b0[CB], b1[CB];
    read_b(b0, 0, 0);
    constexpr int NMF = RB * CB;  // MFMAs per k16 step
    for (int kt = 0; kt < KT; kt += U) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int cur = u % NBUF, nxt = (u + 1) % NBUF, ra = u % PDA;
        read_a(A[ra], cur);
        read_b(b1, cur, 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
          for (int j = 0; j < CB; ++j) acc[i][j] = E::mma(A[ra].a[i][0], b0[j], acc[i][j]);
        __builtin_amdgcn_sched_barrier(0);
        read_b(b0, nxt, 0);  // step 0 of slab kt + u + 1
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
          for (int j = 0; j < CB; ++j) acc[i][j] = E::mma(A[ra].a[i][1], b1[j], acc[i][j]);
        load_a(A[ra], kt + u + PD);
        // Step-1 MFMAs interleaved with the next slab's B reads and this slot's x loads.
#pragma unroll
        for (int i = 0; i < NMF; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (i < CB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          if (i < 2 * RB) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
      }
    }
  }

  if constexpr (!EP::kPaired) {
    // The tile leaves through the LDS ring (free after the loops' last barrier), RP rows at a
    // time: the consumers write their accumulators, then all 8 waves store 16-byte chunks of
    // whole rows (row-major, coalesced): fp32 partial sums into this split's slice of the
    // workspace (split-K) or four outputs at a time through the output policy. The consumers'
    // own stores of one accumulator element at a time (wide_store_tile) took 13.7 us of a
    // 44 us W4A16 M=128 call.
    constexpr int RP = NBUF * SLAB / (TN * 4);  // rows per pass
    constexpr int RW = TM / WM;                 // rows of one consumer wave
    static_assert(RP % RW == 0 || RW % RP == 0, "whole wave stripes or row blocks per pass");
    float* Ls = reinterpret_cast<float*>(&Bs[0][0]);
    typename E::Part* part = ws + (size_t)split * M * N;
#pragma unroll
    for (int p = 0; p < (TM + RP - 1) / RP; ++p) {
      __syncthreads();  // the ring (first pass) or the previous pass's rows have been read
      if (wave < 4) {
        const int wm = wave / WN, wn = wave % WN;
#pragma unroll
        for (int i = 0; i < RB; ++i) {
          const int r0 = wm * RW + 32 * i - p * RP;  // row block i's first row within the pass
          if (r0 < 0 || r0 >= RP) continue;
#pragma unroll
          for (int j = 0; j < CB; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
              Ls[(r0 + 8 * (e >> 2) + 4 * fg + (e & 3)) * TN + wn * 32 * CB + 32 * j + fr] =
                  acc[i][j][e];
        }
      }
      __syncthreads();
      for (int q = (int)threadIdx.x; q < RP * TN / 4; q += NT) {
        const int rl = q / (TN / 4), c = 4 * (q % (TN / 4));
        const int r = p * RP + rl;
        if (r >= ti.rows) continue;
        const kbh_f32x4 v = *reinterpret_cast<const kbh_f32x4*>(&Ls[rl * TN + c]);
        if (splits > 1)
          *reinterpret_cast<kbh_f32x4*>(part + (size_t)rm.out_row(ti, r) * N + n0 + c) = v;
        else
          ep.emit4(rm.out_row(ti, r), n0 + c, v);
      }
    }
    return;
  }
  if constexpr (EP::kPaired) {
    // Paired output (gate/up accumulator blocks j and j + 2 give one output block of TN / 2
    // columns): also through the ring. The consumers write each output's 16-bit result as one
    // 32-bit word (RQ rows per pass), then all waves store 16-byte chunks of 8 outputs. Measured
    // on the Mixtral SiLU FFN's gate/up launch: 16.3k -> 10.3k cycles per workgroup against the
    // consumers' own 2-byte stores (wide_store_tile); FFN 854 -> 826 us.
    static_assert(CB % 4 == 0, "paired output needs whole 128-column chunks per wave");
    constexpr int NO = TN / 2;                     // output columns of the tile
    constexpr int RQ = NBUF * SLAB / (NO * 4);     // rows per pass
    constexpr int RW = TM / WM;                    // rows of one consumer wave
    static_assert(RQ % RW == 0 || RW % RQ == 0, "whole wave stripes or row blocks per pass");
    uint32_t* Lw = reinterpret_cast<uint32_t*>(&Bs[0][0]);
#pragma unroll
    for (int p = 0; p < (TM + RQ - 1) / RQ; ++p) {
      __syncthreads();  // the ring (first pass) or the previous pass's rows have been read
      if (wave < 4) {
#pragma unroll
        for (int i = 0; i < RB; ++i) {
          const int r0 = (wave / WN) * RW + 32 * i - p * RQ;
          if (r0 < 0 || r0 >= RQ) continue;
#pragma unroll
          for (int j = 0; j < CB; ++j) {
            if ((j & 3) >= 2) continue;  // second-matrix blocks pair with block j - 2
            const int jg = (wave % WN) * CB + j;  // block index within the tile
#pragma unroll
            for (int e = 0; e < 16; ++e)
              Lw[(r0 + 8 * (e >> 2) + 4 * fg + (e & 3)) * NO + 64 * (jg >> 2) + 32 * (jg & 1) + fr] =
                  ep.pair_bits(acc[i][j][e], acc[i][j + 2][e]);
          }
        }
      }
      __syncthreads();
      for (int q = (int)threadIdx.x; q < RQ * NO / 8; q += NT) {
        const int rl = q / (NO / 8), c = 8 * (q % (NO / 8));
        const int r = p * RQ + rl;
        if (r >= ti.rows) continue;
        const kbh_u32x4 a = *reinterpret_cast<const kbh_u32x4*>(&Lw[rl * NO + c]);
        const kbh_u32x4 b = *reinterpret_cast<const kbh_u32x4*>(&Lw[rl * NO + c + 4]);
        ep.store8(rm.out_row(ti, r), n0 / 2 + c,
                  kbh_u32x4{a[0] | (a[1] << 16), a[2] | (a[3] << 16), b[0] | (b[1] << 16),
                            b[2] | (b[3] << 16)});
      }
    }
  }
}

}  // namespace kbh
