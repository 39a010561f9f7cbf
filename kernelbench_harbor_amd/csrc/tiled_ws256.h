// Warp-specialised 256 x 256 tiles (tiled_ws256_gemm) for dense rows: W4A16 (fp16/bf16) and
// W8A8 (int8) operands.
//
// The computation, weight policy BP, output policy EP and launch geometry of tiled_wide_gemm with
// 256 x 256 tiles, on 12 waves in two roles:
//  * waves 8..11 (the policy's thread ids t = 0..255) write the weights of every slab (64 bytes
//    of K: 32 fp16/bf16 or 64 int8 values) into a 4-buffer LDS ring in MFMA operand order
//    (BP::store_all: dequantized W4, or transposed int8), the raw words loaded PD slabs ahead,
//    and stage the slab's x rows (256 rows x 64 bytes) into the same ring with LDS-mode buffer
//    loads, three slabs ahead (into the buffer that is idle during the current slab);
//  * waves 0..7 only read fragments and issue MFMAs, 64 rows x 128 columns each (4 x 2 waves),
//    with the accumulators of a whole 256 x 256 tile between them.
// One barrier per slab, as in tiled_ws_gemm: in slab s the MFMA waves read buffer s % 4, the
// producers fill (s + 2) % 4, and buffers (s + 1) % 4 (filled a barrier earlier) and (s + 3) % 4
// are idle, so a write never meets a read (x for slab s + 3 goes into x buffer (s + 3) % 4).
// x goes through LDS because an MFMA wave holding 128 accumulator registers has no room
// for a register ring of x fragments (12 waves: at most 168 registers per wave); the LDS-mode
// loads need no registers at all. The x loads are inline assembly (M0 = the LDS block, then
// buffer_load_dwordx4 ... lds) and the producers wait for them with explicit vmcnt counts: as
// compiler builtins, every barrier waited for all of them (vmcnt(0)), including the ones just
// issued for two slabs later (M=2048 250 -> 296 us). The offsets are 32-bit: the caller keeps
// (M + 256) rows of x under 2 GiB. Rows past M read as zero (the buffer's size bound).
#pragma once

#include "tiled_ws.h"

namespace kbh {

template <class E, int SPG, class BP, class EP, int PD = 4>
__global__ __launch_bounds__(768, 1) void tiled_ws256_gemm(
    const void* __restrict__ x, BP bp, EP ep, typename E::Part* __restrict__ ws, int M, int N,
    int K, int splits, int slabs_per_split) {
  constexpr int TM = 256, TN = 256;
  static_assert(BP::kTN == TN, "256-column weight policy");
  constexpr int SK = E::kSlabK;        // K elements per slab (64 bytes of every row)
  constexpr int EB = WSLAB_BYTES / SK;  // bytes per element
  constexpr int SLAB = TN * 64;        // B bytes per buffer
  constexpr int ASLAB = TM * 64;       // A bytes per buffer: 256 rows x 64 bytes
  constexpr int NBUF = 4;
  constexpr int RING = NBUF * (SLAB + ASLAB);  // weight and x buffers (the epilogue's staging)
  constexpr int U = 2 * SPG > PD ? 2 * SPG : PD;  // slabs per loop iteration
  static_assert(PD >= 2 && U % PD == 0 && U % (2 * SPG) == 0 && U % NBUF == 0, "unroll");
  constexpr int RB = 2, CB = 4;  // 32 x 32 blocks of one MFMA wave
  constexpr int NT = 768;
  // The weight buffers, then the x buffers; the epilogue stages rows through all of it.
  __shared__ __attribute__((aligned(16))) uint8_t L[RING];
  auto bbuf = [&](int b) { return L + b * SLAB; };
  auto abuf = [&](int b) { return L + NBUF * SLAB + b * ASLAB; };

  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int NB = N / TN;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int nb = id % NB;
  const int rest = id / NB;
  const int MB = gridDim.x / (NB * splits);
  const int mb = rest % MB;
  const int split = rest / MB;
  const int n0 = nb * TN, m0 = mb * TM;
  const int rows = min(TM, M - m0);
  const int kt0 = split * slabs_per_split;
  const int KT = slabs_per_split;
  const int last = KT - 1;
  constexpr bool kFast = BP::kHasFast;
  const int fr = lane & 31, fg = lane >> 5;

  typename E::Acc acc[RB][CB];
  if (wave >= 8) {
    // ---- producers ----
    const int t = (int)threadIdx.x - 512;
    auto load_b = [&](typename BP::Raw& r, int s) { bp.load(r, (kt0 + min(s, last)) * SK, n0, t); };
    auto load_g = [&](typename BP::Grp& g, int s) {
      bp.load_group(g, (kt0 + min(s, last)) * SK, n0, t);
    };
    // x, straight from global memory into the ring with the buffer loads' LDS mode (lane i of a
    // 16-byte load lands at M0 + 16 i): a load fills one 1 KB block of 16 rows; lane l takes row
    // l / 4 of the block and the chunk the swizzle puts at position l % 4. Producer wave p
    // loads blocks 4p .. 4p + 3 of every slab.
    const uint32_t vx =
        (uint32_t)((m0 + (lane >> 2)) * K * EB + 16 * ((lane & 3) ^ ((lane >> 4) & 3)));
    const kbh_rsrc4 rxs = raw_rsrc(x, (size_t)M * K * EB);
    auto stage_x = [&](int s, int buf) {
      const int k0b = (kt0 + min(s, last)) * WSLAB_BYTES;
      const uint8_t* a = abuf(buf);
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int blk = 4 * (wave - 8) + h;
        lds_load16(lds_addr(a + 1024 * blk), vx, rxs, (uint32_t)(16 * blk * K * EB + k0b));
      }
    };
    typename BP::ScanPre sp;
    if constexpr (kFast) bp.scan_load(sp, kt0 * SK, (kt0 + KT) * SK, n0, t);
    typename BP::Raw R[PD];
    typename BP::Grp G[2];
#pragma unroll
    for (int i = 0; i < PD; ++i) load_b(R[i], i);
    load_g(G[0], 0);
    load_g(G[1], SPG);
    stage_x(0, 0);
    stage_x(1, 1);
    stage_x(2, 2);
    bool fast = false;
    if constexpr (kFast)
      fast = __syncthreads_and((int)bp.scan_check(sp, kt0 * SK, (kt0 + KT) * SK, n0, t)) != 0;
    auto produce = [&](auto fast_tag) {
      constexpr bool FAST = decltype(fast_tag)::value;
      auto put = [&](const typename BP::Raw& r, const typename BP::Grp& g, int b) {
        bp.template store_all<FAST>(r, g, bbuf(b), t);
      };
      bp.template prepare_group<FAST>(G[0]);
      put(R[0], G[0], 0);  // slab 0
      load_b(R[0], PD);
      if constexpr (SPG == 1) {  // slab 1 starts group 1; set 0 is reloaded with group 2
        bp.template prepare_group<FAST>(G[1]);
        load_g(G[0], 2);
        put(R[1], G[1], 1);
      } else {
        put(R[1], G[0], 1);
      }
      load_b(R[1 % PD], PD + 1);
      // x of slabs 0 and 1 has landed (younger: slab 2's 4 x loads, the two 4-word raw loads and
      // at most one group load pair)
      asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
      __syncthreads();  // slabs 0 and 1 are in LDS
      for (int kt = 0; kt < KT; kt += U) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int pu = u + 2;
          const int set = (pu / SPG) & 1;
          if (pu % SPG == 0) {
            bp.template prepare_group<FAST>(G[set]);
            load_g(G[set ^ 1], kt + pu + SPG);
          }
          put(R[pu % PD], G[set], pu % NBUF);
          // x of slab kt + u + 3 into the buffer that is idle during slab kt + u (read three
          // barriers later)
          stage_x(kt + u + 3, (u + 3) % NBUF);
          load_b(R[pu % PD], kt + pu + PD);
          // x of the next slab (issued two iterations ago) has landed: at least 20 loads are
          // younger (4 raw words of that iteration, 8-10 loads of each of the last two).
          asm volatile("s_waitcnt vmcnt(20)" ::: "memory");
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
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no x load in flight past the loops
  } else {
    // ---- MFMA waves: rows 64 wm .., columns 128 wn .. of the tile ----
    // x of a slab: row r keeps its 16-byte chunk c at r * 64 + 16 (c ^ ((r >> 2) & 3)) of the
    // buffer (staged by the producers), so the 16 rows a fragment read covers hit 16 different
    // bank groups.
    const int wm = wave >> 1, wn = wave & 1;
    if constexpr (kFast) (void)__syncthreads_and(1);  // the producers' FAST barrier
    // B fragment j: column 128 wn + 32 j + fr at wide_b_offset = bbase + 512 j + (bsw ^ 16 c_j):
    // the column slot's low 3 bits are s_0 ^ c_j with c_j = 4 (j & 1) ^ (j >> 1) (two registers
    // instead of four offsets)
    const int bsw = 16 * (wide_slot(128 * wn + fr) & 7);
    const int bbase = wide_b_offset<TN>(16 * fg, 128 * wn + fr) - bsw;
    // [k16 step]: chunk 2 step + fg of row 64 wm + fr (row block i adds 32 rows: the swizzle
    // term (r >> 2) & 3 = (fr >> 2) & 3 is the same for both)
    int aoff[2];
#pragma unroll
    for (int st = 0; st < 2; ++st)
      aoff[st] = (64 * wm + fr) * 64 + 16 * ((2 * st + fg) ^ ((fr >> 2) & 3));
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;
    __syncthreads();  // slabs 0 and 1 are in LDS
    for (int kt = 0; kt < KT; kt += U) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint8_t* bb = bbuf(u % NBUF);
        const uint8_t* ab = abuf(u % NBUF);
#pragma unroll
        for (int s = 0; s < 2; ++s) {  // k16 steps
          kbh_u32x4 af[RB], bf[CB];
#pragma unroll
          for (int i = 0; i < RB; ++i)
            af[i] = *reinterpret_cast<const kbh_u32x4*>(ab + aoff[s] + 32 * 64 * i);
#pragma unroll
          for (int j = 0; j < CB; ++j)
            bf[j] = *reinterpret_cast<const kbh_u32x4*>(
                bb + bbase + (bsw ^ (16 * ((4 * (j & 1)) ^ (j >> 1)))) + 512 * j + s * (TN * 32));
#pragma unroll
          for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int j = 0; j < CB; ++j) acc[i][j] = E::mma(af[i], bf[j], acc[i][j]);
        }
        __syncthreads();
      }
    }
  }

  // The tile leaves through the ring, RP rows at a time: the MFMA waves write their
  // accumulators, then all 12 waves store 16-byte chunks of whole rows (fp32 split-K slices, or
  // four outputs at a time through the output policy).
  constexpr int RP = 128;  // rows per pass: 128 x 256 x 4 bytes, the whole ring
  static_assert(RP * TN * 4 <= RING, "pass fits the ring");
  using Part = typename E::Part;
  using Part4 = typename E::Part4;
  Part* Ls = reinterpret_cast<Part*>(L);
  typename E::Part* part = ws + (size_t)split * M * N;
#pragma unroll
  for (int p = 0; p < TM / RP; ++p) {
    __syncthreads();  // the ring (first pass) or the previous pass's rows have been read
    if (wave < 8) {
      const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int r0 = 64 * wm + 32 * i - p * RP;
        if (r0 < 0 || r0 >= RP) continue;
#pragma unroll
        for (int j = 0; j < CB; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            Ls[(r0 + 8 * (e >> 2) + 4 * fg + (e & 3)) * TN + 128 * wn + 32 * j + fr] = acc[i][j][e];
      }
    }
    __syncthreads();
    for (int q = (int)threadIdx.x; q < RP * TN / 4; q += NT) {
      const int rl = q / (TN / 4), c = 4 * (q % (TN / 4));
      const int r = p * RP + rl;
      if (r >= rows) continue;
      const Part4 v = *reinterpret_cast<const Part4*>(&Ls[rl * TN + c]);
      if (splits > 1)
        *reinterpret_cast<Part4*>(part + (size_t)(m0 + r) * N + n0 + c) = v;
      else
        ep.emit4(m0 + r, n0 + c, v);
    }
  }
}

}  // namespace kbh
