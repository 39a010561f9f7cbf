// Warp-specialised 256 x 256 tiles (tiled_ws256_gemm) for dense W4A16 rows.
//
// The computation, weight policy BP, output policy EP and launch geometry of tiled_wide_gemm with
// 256 x 256 tiles and fp16/bf16 operands, on 12 waves in two roles:
//  * waves 8..11 (the policy's thread ids t = 0..255) produce both operands of every 32-deep
//    slab into a 4-buffer LDS ring: the dequantized weights (BP::store_all) and the slab's x
//    rows (256 rows x 64 bytes), each loaded PD slabs ahead;
//  * waves 0..7 only read fragments and issue MFMAs, 64 rows x 128 columns each (4 x 2 waves),
//    with the accumulators of a whole 256 x 256 tile between them.
// One barrier per slab, as in tiled_ws_gemm: in slab s the MFMA waves read buffer s % 4, the
// producers fill (s + 2) % 4, and buffers (s + 1) % 4 (filled a barrier earlier) and (s + 3) % 4
// are idle, so a write never meets a read. x goes through LDS because an MFMA wave holding 128
// accumulator registers has no room for a register ring of x fragments (12 waves: at most 168
// registers per wave).
#pragma once

#include "tiled_ws.h"

namespace kbh {

template <class E, int SPG, class BP, class EP, int PD = 4>
__global__ __launch_bounds__(768, 1) void tiled_ws256_gemm(
    const void* __restrict__ x, BP bp, EP ep, typename E::Part* __restrict__ ws, int M, int N,
    int K, int splits, int slabs_per_split) {
  constexpr int TM = 256, TN = 256;
  static_assert(BP::kTN == TN, "256-column weight policy");
  static_assert(!E::kStageX, "fp16/bf16 operands");
  constexpr int SK = E::kSlabK;        // 32 K elements per slab
  constexpr int SLAB = TN * 64;        // B bytes per buffer
  constexpr int ACH = TM * 16 + 64;    // A bytes per 16-byte chunk column (+64: bank skew)
  constexpr int ASLAB = 4 * ACH;       // A bytes per buffer: 4 chunks of every row
  constexpr int NBUF = 4;
  constexpr int RING = NBUF * (SLAB + ASLAB);
  constexpr int U = 2 * SPG > PD ? 2 * SPG : PD;  // slabs per loop iteration
  static_assert(PD >= 2 && U % PD == 0 && U % (2 * SPG) == 0 && U % NBUF == 0, "unroll");
  constexpr int RB = 2, CB = 4;  // 32 x 32 blocks of one MFMA wave
  constexpr int NT = 768;
  constexpr int PDX = 2;  // x prefetch depth (x rows are shared by the column tiles, mostly L2 hits)
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
    // x: producer wave pw stages rows 64 pw .. 64 pw + 63; lane l loads chunk l % 4 (16 bytes)
    // of rows 64 pw + 16 i + l / 4, i < 4, so one load covers 16 rows x 64 bytes.
    const int xc = lane & 3;
    int xr[4];
    const uint8_t* xp[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xr[i] = 64 * (wave - 8) + 16 * i + (lane >> 2);
      xp[i] = (const uint8_t*)x + (size_t)(m0 + min(xr[i], rows - 1)) * K * 2 + 16 * xc;
    }
    struct XStage {
      kbh_u32x4 c[4];
    };
    auto load_x = [&](XStage& st, int s) {
      const size_t b0 = (size_t)(kt0 + min(s, last)) * WSLAB_BYTES;
#pragma unroll
      for (int i = 0; i < 4; ++i) st.c[i] = *reinterpret_cast<const kbh_u32x4*>(xp[i] + b0);
    };
    auto put_x = [&](const XStage& st, uint8_t* a) {
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<kbh_u32x4*>(a + xc * ACH + xr[i] * 16) = st.c[i];
    };
    typename BP::ScanPre sp;
    if constexpr (kFast) bp.scan_load(sp, kt0 * SK, (kt0 + KT) * SK, n0, t);
    typename BP::Raw R[PD];
    XStage X[PDX];
    typename BP::Grp G[2];
#pragma unroll
    for (int i = 0; i < PD; ++i) load_b(R[i], i);
#pragma unroll
    for (int i = 0; i < PDX; ++i) load_x(X[i], i);
    load_g(G[0], 0);
    load_g(G[1], SPG);
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
      put_x(X[0], abuf(0));
      load_b(R[0], PD);
      load_x(X[0], PDX);
      if constexpr (SPG == 1) {  // slab 1 starts group 1; set 0 is reloaded with group 2
        bp.template prepare_group<FAST>(G[1]);
        load_g(G[0], 2);
        put(R[1], G[1], 1);
      } else {
        put(R[1], G[0], 1);
      }
      put_x(X[1], abuf(1));
      load_b(R[1 % PD], PD + 1);
      load_x(X[1 % PDX], PDX + 1);
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
          put_x(X[pu % PDX], abuf(pu % NBUF));
          load_b(R[pu % PD], kt + pu + PD);
          load_x(X[pu % PDX], kt + pu + PDX);
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
  } else {
    // ---- MFMA waves: rows 64 wm .., columns 128 wn .. of the tile ----
    const int wm = wave >> 1, wn = wave & 1;
    if constexpr (kFast) (void)__syncthreads_and(1);  // the producers' FAST barrier
    int boff[CB];
#pragma unroll
    for (int j = 0; j < CB; ++j) boff[j] = wide_b_offset<TN>(16 * fg, 128 * wn + 32 * j + fr);
    int aoff[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) aoff[i] = fg * ACH + (64 * wm + 32 * i + fr) * 16;
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
            af[i] = *reinterpret_cast<const kbh_u32x4*>(ab + aoff[i] + 2 * s * ACH);
#pragma unroll
          for (int j = 0; j < CB; ++j)
            bf[j] = *reinterpret_cast<const kbh_u32x4*>(bb + boff[j] + s * (TN * 32));
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
  constexpr int RP = 128;  // rows per pass: 128 x 256 x 4 bytes of the ring
  static_assert(RP * TN * 4 <= RING, "pass fits the ring");
  float* Ls = reinterpret_cast<float*>(L);
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
      const kbh_f32x4 v = *reinterpret_cast<const kbh_f32x4*>(&Ls[rl * TN + c]);
      if (splits > 1)
        *reinterpret_cast<kbh_f32x4*>(part + (size_t)(m0 + r) * N + n0 + c) = v;
      else
        ep.emit4(m0 + r, n0 + c, v);
    }
  }
}

}  // namespace kbh
