// Workgroup GEMM through LDS for gfx950: bf16 weight rows x activation rows,
// fp32 accumulation on MFMA 16x16x32.
#pragma once

#include "kve_common.h"

namespace kve {

// Weight and activation tiles are read from global memory as whole rows (a wave
// instruction covers 4 rows x 256 contiguous bytes at KC = 4, i.e. full cache
// lines): loading MFMA fragments straight from global memory (16 rows x 64
// bytes per instruction) moves the same bytes about 3.5x slower on gfx950. The
// tiles are staged in LDS (row stride padded by 16 bytes, so fragment reads are
// conflict-free) and double-buffered, with P chunks in flight in registers.
//
// Workgroup of NW waves, each owning WN 16-row weight tiles: BN = 16 WN NW
// weight rows (tile row r of wave w's tile j is 16 (WN w + j) + lane row),
// activation rows 0..M-1 (M <= 16 MT, row stride xstride elements), k-steps
// [ks0, ks1) of 32, KC k-steps per chunk. acc[j][mt] (lane: weight row
// 16 (WN w + j) + 4 (lane / 16) + i, activation row 16 mt + lane % 16).
template <int MT, int NW, int WN, int KC, int P>
struct LdsGemm {
  static constexpr int BN = 16 * WN * NW;
  static constexpr int NT = 64 * NW;
  static constexpr int UPR = KC * 4;            // 16-byte units per row per chunk
  static constexpr int LDR = KC * 32 + 8;       // LDS row stride (bf16 elements)
  static constexpr int XROWS = 16 * MT;
  static constexpr int BUF = (BN + XROWS) * LDR;  // elements per buffer
  static constexpr int WU = cdiv(BN * UPR, NT);  // weight units per thread per chunk
  static constexpr int XU = cdiv(XROWS * UPR, NT);
  static constexpr int U = WU + XU;
  static constexpr size_t LDS_BYTES = static_cast<size_t>(2) * BUF * 2;
  static_assert(P % 2 == 0, "P must be even");

  // wrow(r): weight row (of the [N, K] matrix w) behind tile row r < BN.
  // Chunk c is stored to LDS (waiting only for its own loads, the oldest), then
  // chunk c + P is requested and chunk c multiplied. Every unit is loaded, also
  // past ks1 (the k-step index is clamped), so each wait is for an exact count
  // of loads; k-steps past ks1 get a zero weight fragment and add nothing.
  template <typename WRow>
  __device__ __forceinline__ static void run(const uint16_t* w, WRow wrow, const uint16_t* x,
                                             int64_t xstride, int M, int K, int ks0, int ks1,
                                             uint16_t* lds, f32x4 (&acc)[WN][MT]) {
    const int tid = threadIdx.x;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l = tid & 63, lr = l & 15, lg = l >> 4;
    const uint16_t* src[U];
    int dst[U], uks[U];
#pragma unroll
    for (int i = 0; i < WU; ++i) {
      const int u = tid + NT * i, r = min(u / UPR, BN - 1), c = u % UPR;
      src[i] = w + static_cast<size_t>(wrow(r)) * K + 8 * (c & 3);
      uks[i] = c >> 2;
      dst[i] = u < BN * UPR ? r * LDR + 8 * c : -1;
    }
#pragma unroll
    for (int i = 0; i < XU; ++i) {
      // rows past M repeat row M - 1 (their sums are dropped); units past the
      // tile are loaded, not stored
      const int u = tid + NT * i, r = u / UPR, c = u % UPR;
      src[WU + i] = x + static_cast<int64_t>(min(r, M - 1)) * xstride + 8 * (c & 3);
      uks[WU + i] = c >> 2;
      dst[WU + i] = u < XROWS * UPR ? (BN + r) * LDR + 8 * c : -1;
    }
    u32x4 reg[P][U];
    auto gload = [&](u32x4 (&rg)[U], int c0) {
#pragma unroll
      for (int i = 0; i < U; ++i)
        rg[i] = *reinterpret_cast<const u32x4*>(src[i] + 32 * min(c0 + uks[i], ks1 - 1));
    };
    auto lstore = [&](uint16_t* buf, const u32x4 (&rg)[U]) {
#pragma unroll
      for (int i = 0; i < U; ++i)
        if (dst[i] >= 0) *reinterpret_cast<u32x4*>(buf + dst[i]) = rg[i];
    };
    auto compute = [&](const uint16_t* buf, int c0) {
#pragma unroll
      for (int kk = 0; kk < KC; ++kk) {
        u32x4 av[WN];
#pragma unroll
        for (int j = 0; j < WN; ++j) {
          const u32x4 ld =
              *reinterpret_cast<const u32x4*>(buf + (16 * (WN * wv + j) + lr) * LDR + 32 * kk + 8 * lg);
          av[j] = c0 + kk < ks1 ? ld : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const u32x4 bv =
              *reinterpret_cast<const u32x4*>(buf + (BN + 16 * mt + lr) * LDR + 32 * kk + 8 * lg);
#pragma unroll
          for (int j = 0; j < WN; ++j) acc[j][mt] = mfma16x16x32_bf16(av[j], bv, acc[j][mt]);
        }
      }
    };
    // Whole batches of P chunks, no branch inside a batch: the loads in flight
    // at the loop head are always the same P chunks in the same order. P is
    // even, so chunk q of a batch uses LDS buffer q & 1.
#pragma unroll
    for (int q = 0; q < P; ++q) gload(reg[q], ks0 + q * KC);
    for (int c0 = ks0; c0 < ks1; c0 += P * KC) {
#pragma unroll
      for (int q = 0; q < P; ++q) {
        const int cc = c0 + q * KC;
        uint16_t* buf = lds + (q & 1) * BUF;
        lstore(buf, reg[q]);
        __syncthreads();
        gload(reg[q], cc + P * KC);
        compute(buf, cc);
      }
    }
    __syncthreads();  // the caller may reuse the LDS once every wave is done
  }
};

}  // namespace kve
