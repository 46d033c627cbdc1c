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

// s_waitcnt immediate: at most n vector-memory operations and no LDS operation
// of this wave outstanding (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt
// bits 6:4 left at their maximum, lgkmcnt bits 11:8 = 0).
constexpr int waitcnt_vm_lgkm0(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }

// Workgroup barrier after this wave's loads of the current chunk have landed
// (at most n vector-memory operations outstanding) and its LDS reads are done.
// __syncthreads() would wait for every outstanding direct-to-LDS load (its
// release fence counts them as LDS writes); the "memory" clobbers keep the
// compiler from moving LDS accesses across the barrier.
template <int N>
__device__ __forceinline__ void barrier_after_vm() {
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(N));
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

// The same workgroup GEMM with the tiles copied global -> LDS by the gfx950
// direct loads (global_load_lds_dwordx4: each lane's 16 bytes land at
// LDS base + 16 * lane), so no registers hold tiles in flight and the prefetch
// depth is set by LDS: NBUF chunk buffers, NBUF - 1 chunks in flight.
//
// A chunk is ROWS = BN + 16 MT rows (weight rows, then activation rows) of KC
// k-steps (UPR = 4 KC 16-byte units per row), row-major in LDS without
// padding; unit c of row r sits at unit c ^ swz(r), which puts the 16 rows of
// a fragment read in 16 different 4-bank groups. One instruction fills 64
// consecutive units (1 KiB); instruction g of a chunk is issued by wave g % NW.
// Chunk c waits for its own loads only (vmcnt), then one barrier makes every
// wave's loads visible and frees the buffer of chunk c - 1 for chunk
// c + NBUF - 1. Same operands, k order and accumulator layout as LdsGemm.
template <int MT, int NW, int WN, int KC, int NBUF>
struct DmaGemm {
  static constexpr int BN = 16 * WN * NW;
  static constexpr int NT = 64 * NW;
  static constexpr int UPR = KC * 4;
  static constexpr int XROWS = 16 * MT;
  static constexpr int ROWS = BN + XROWS;
  static constexpr int CH_UNITS = ROWS * UPR;
  static constexpr int U = CH_UNITS / NT;  // units (instructions) per thread per chunk
  static constexpr size_t CH_BYTES = static_cast<size_t>(CH_UNITS) * 16;
  static constexpr size_t LDS_BYTES = NBUF * CH_BYTES;
  static_assert(CH_UNITS % NT == 0, "chunk must split evenly over the waves");
  static_assert(NBUF >= 2 && (NBUF - 2) * U <= 63, "vmcnt range");
  static constexpr int RPS = UPR >= 16 ? 1 : 16 / UPR;  // rows sharing a swizzle value
  static constexpr int SWM = UPR >= 16 ? 15 : UPR - 1;
  __device__ __forceinline__ static int swz(int r) { return (r / RPS) & SWM; }

  template <typename WRow>
  __device__ __forceinline__ static void run(const uint16_t* w, WRow wrow, const uint16_t* x,
                                             int64_t xstride, int M, int K, int ks0, int ks1,
                                             uint16_t* lds, f32x4 (&acc)[WN][MT]) {
    const int tid = threadIdx.x;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l = tid & 63, lr = l & 15, lg = l >> 4;
    const uint16_t* src[U];
    int uks[U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int u = 64 * (NW * i + wv) + l;  // LDS unit this lane fills
      const int r = u / UPR, pc = u % UPR, c = pc ^ swz(r);
      const uint16_t* row = r < BN ? w + static_cast<size_t>(wrow(r)) * K
                                   : x + static_cast<int64_t>(min(r - BN, M - 1)) * xstride;
      src[i] = row + 8 * (c & 3);
      uks[i] = c >> 2;
    }
    auto issue = [&](int c0, int b) {
      uint16_t* base = lds + static_cast<size_t>(b) * (CH_BYTES / 2);
#pragma unroll
      for (int i = 0; i < U; ++i)
        __builtin_amdgcn_global_load_lds(
            (__attribute__((address_space(1))) void*)(src[i] + 32 * min(c0 + uks[i], ks1 - 1)),
            (__attribute__((address_space(3))) void*)(base + 512 * (NW * i + wv)), 16, 0, 0);
    };
    auto compute = [&](const uint16_t* buf, int c0) {
#pragma unroll
      for (int kk = 0; kk < KC; ++kk) {
        u32x4 av[WN];
#pragma unroll
        for (int j = 0; j < WN; ++j) {
          const int r = 16 * (WN * wv + j) + lr;
          const u32x4 ld = *reinterpret_cast<const u32x4*>(buf + 8 * (r * UPR + ((4 * kk + lg) ^ swz(r))));
          av[j] = c0 + kk < ks1 ? ld : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int r = BN + 16 * mt + lr;
          const u32x4 bv = *reinterpret_cast<const u32x4*>(buf + 8 * (r * UPR + ((4 * kk + lg) ^ swz(r))));
#pragma unroll
          for (int j = 0; j < WN; ++j) acc[j][mt] = mfma16x16x32_bf16(av[j], bv, acc[j][mt]);
        }
      }
    };
    const int nch = (ks1 - ks0 + KC - 1) / KC;
#pragma unroll
    for (int q = 0; q < NBUF - 1; ++q)
      if (q < nch) issue(ks0 + q * KC, q);
    for (int c = 0; c < nch; ++c) {
      if (c + NBUF - 2 < nch) barrier_after_vm<(NBUF - 2) * U>();
      else barrier_after_vm<0>();
      if (c + NBUF - 1 < nch) issue(ks0 + (c + NBUF - 1) * KC, (c + NBUF - 1) % NBUF);
      compute(lds + static_cast<size_t>(c % NBUF) * (CH_BYTES / 2), ks0 + c * KC);
    }
    __syncthreads();  // the caller may reuse the LDS once every wave is done
  }
};

// DmaGemm with as many chunk buffers as fit in lds_budget bytes (and in the
// vmcnt range), at least two.
template <int MT, int NW, int WN, int KC, int LDS_BUDGET = 96 * 1024>
struct DmaCfg {
  static constexpr int ROWS = 16 * WN * NW + 16 * MT;
  static constexpr int CHB = ROWS * KC * 64;
  static constexpr int U = ROWS * KC * 4 / (64 * NW);
  static constexpr int BY_LDS = LDS_BUDGET / CHB;
  static constexpr int BY_VM = 63 / U + 2;
  static constexpr int NB0 = BY_LDS < BY_VM ? BY_LDS : BY_VM;
  static constexpr int NBUF = NB0 < 2 ? 2 : NB0;
  using G = DmaGemm<MT, NW, WN, KC, NBUF>;
};

}  // namespace kve
