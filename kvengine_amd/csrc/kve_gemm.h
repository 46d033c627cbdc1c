// Workgroup GEMM through LDS for gfx950: bf16 weight rows x activation rows,
// fp32 accumulation on MFMA 16x16x32.
#pragma once

#include "kve_common.h"

namespace kve {

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

// Workgroup of NW waves in NR row groups of NC = NW / NR: wave w (column
// wc = w % NC, row group wr = w / NC) owns WN 16-row weight tiles and MTW =
// MT / NR activation row tiles: BN = 16 WN NC weight rows (tile row r of
// tile j is 16 (WN wc + j) + lane row), activation rows 0..M-1 (M <= 16 MT,
// row stride xstride elements), k-steps [ks0, ks1) of 32, KC k-steps per
// chunk. acc[j][mt] (lane: weight row 16 (WN wc + j) + 4 (lane / 16) + i,
// activation row 16 (MTW wr + mt) + lane % 16). Row groups cut the LDS
// fragment reads: each wave reads WN + MTW fragments per k-step.
// Every output element sums its k-steps in order, one MFMA each, whatever the
// tiling, so a row's result does not depend on M, MT, NW, NR, WN, KC or NBUF.
//
// Weight and activation tiles are read from global memory as whole rows (an
// instruction covers 4-8 rows x 128-256 contiguous bytes), or, with BLK, from
// the blocked layout (kve_common.h blk_off), where an instruction reads two
// 512-byte runs: loading MFMA fragments straight from row-major global memory
// (16 rows x 64 bytes per instruction) moves the same bytes about 3.5x slower
// on gfx950, and the row-major chunk reads themselves run up to 1.5-2x slower
// than the blocked ones at 32-160 rows. The tiles are copied
// global -> LDS by the gfx950 direct loads (global_load_lds_dwordx4: each
// lane's 16 bytes land at LDS base + 16 * lane), so no registers hold tiles in
// flight and the prefetch depth is set by LDS: NBUF chunk buffers, NBUF - 1
// chunks in flight.
//
// A chunk is ROWS = BN + 16 MT rows (weight rows, then activation rows) of KC
// k-steps (UPR = 4 KC 16-byte units per row), row-major in LDS without
// padding; unit c of row r sits at unit c ^ swz(r), which puts the 16 rows of
// a fragment read in 16 different 4-bank groups. One instruction fills 64
// consecutive units (1 KiB); instruction g of a chunk is issued by wave g % NW.
// Chunk c waits for its own loads only (vmcnt), then one barrier makes every
// wave's loads visible and frees the buffer of chunk c - 1 for chunk
// c + NBUF - 1. Every load is issued (k-steps past ks1 are clamped to ks1 - 1
// and read, and their weight fragments zeroed), so the vmcnt counts are exact.
template <int MT, int NW, int WN, int KC, int NBUF, int NR = 1>
struct DmaGemm {
  static constexpr int NC = NW / NR;    // wave columns
  static constexpr int MTW = MT / NR;   // row tiles per wave
  static_assert(NC * NR == NW && MTW * NR == MT, "waves split evenly into row groups");
  static constexpr int BN = 16 * WN * NC;
  static constexpr int NT = 64 * NW;
  static constexpr int UPR = KC * 4;
  static constexpr int XROWS = 16 * MT;
  static constexpr int ROWS = BN + XROWS;
  // units per chunk, rounded up so that every wave issues the same number of
  // loads (the rows past ROWS re-read the last activation row into LDS that
  // nothing reads)
  static constexpr int CH_UNITS = (ROWS * UPR + NT - 1) / NT * NT;
  static constexpr int U = CH_UNITS / NT;  // units (instructions) per thread per chunk
  static constexpr size_t CH_BYTES = static_cast<size_t>(CH_UNITS) * 16;
  static constexpr size_t LDS_BYTES = NBUF * CH_BYTES;
  static_assert(NBUF >= 2 && (NBUF - 2) * U <= 63, "vmcnt range");
  static constexpr int RPS = UPR >= 16 ? 1 : 16 / UPR;  // rows sharing a swizzle value
  static constexpr int SWM = UPR >= 16 ? 15 : UPR - 1;
  __device__ __forceinline__ static int swz(int r) { return (r / RPS) & SWM; }

  struct NoStep {
    __device__ __forceinline__ void operator()(int) const {}
  };

  // after(ks) runs once every wave's MFMAs of k-step ks (< ks1) are issued, in
  // k-step order: a caller can fold or restart acc there (k-slice boundaries).
  // BLK: weight and activation matrices in the blocked layout (blk_off; the
  // activation rows padded to 16, xstride unused): a chunk's 16-row tile of a
  // k-step is one contiguous 1 KB block, so an instruction reads two 512-byte
  // runs where the row-major layout gives it eight 128-byte pieces of eight
  // rows. The loads and the LDS image are otherwise the same.
  template <bool BLK = false, typename WRow, typename After = NoStep>
  __device__ __forceinline__ static void run(const uint16_t* w, WRow wrow, const uint16_t* x,
                                             int64_t xstride, int M, int K, int ks0, int ks1,
                                             uint16_t* lds, f32x4 (&acc)[WN][MTW],
                                             After after = After{}) {
    const int tid = threadIdx.x;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wc = wv % NC, wr = wv / NC;
    const int l = tid & 63, lr = l & 15, lg = l >> 4;
    const uint16_t* src[U];
    int uks[U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int u = 64 * (NW * i + wv) + l;  // LDS unit this lane fills
      const int r = u / UPR, pc = u % UPR, c = pc ^ swz(r);
      if constexpr (BLK) {
        const int n = r < BN ? wrow(r) : min(r - BN, M - 1);
        src[i] = (r < BN ? w : x) + blk_off(n, 8 * (c & 3), K);
      } else {
        const uint16_t* row = r < BN ? w + static_cast<size_t>(wrow(r)) * K
                                     : x + static_cast<int64_t>(min(r - BN, M - 1)) * xstride;
        src[i] = row + 8 * (c & 3);
      }
      uks[i] = c >> 2;
    }
    constexpr int KSTEP = BLK ? 512 : 32;  // elements from one k-step to the next
    auto issue = [&](int c0, int b) {
      uint16_t* base = lds + static_cast<size_t>(b) * (CH_BYTES / 2);
#pragma unroll
      for (int i = 0; i < U; ++i)
        __builtin_amdgcn_global_load_lds(
            (__attribute__((address_space(1))) void*)(src[i] + KSTEP * min(c0 + uks[i], ks1 - 1)),
            (__attribute__((address_space(3))) void*)(base + 512 * (NW * i + wv)), 16, 0, 0);
    };
    // The fragments of k-step kk + 1 are read before the MFMAs of k-step kk
    // are issued (the scheduling barrier keeps them there): left to itself
    // the compiler interleaves each fragment read with a full LDS wait. The
    // MFMA sequence of every accumulator is unchanged.
    auto frag = [&](const uint16_t* buf, int r, int kk) {
      return *reinterpret_cast<const u32x4*>(buf + 8 * (r * UPR + ((4 * kk + lg) ^ swz(r))));
    };
    auto compute = [&](const uint16_t* buf, int c0) {
      u32x4 fa[2][WN], fb[2][MTW];
#pragma unroll
      for (int j = 0; j < WN; ++j) fa[0][j] = frag(buf, 16 * (WN * wc + j) + lr, 0);
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) fb[0][mt] = frag(buf, BN + 16 * (MTW * wr + mt) + lr, 0);
#pragma unroll
      for (int kk = 0; kk < KC; ++kk) {
        const int cur = kk & 1, nxt = cur ^ 1;
        if (kk + 1 < KC) {
#pragma unroll
          for (int j = 0; j < WN; ++j) fa[nxt][j] = frag(buf, 16 * (WN * wc + j) + lr, kk + 1);
#pragma unroll
          for (int mt = 0; mt < MTW; ++mt)
            fb[nxt][mt] = frag(buf, BN + 16 * (MTW * wr + mt) + lr, kk + 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        const bool live = c0 + kk < ks1;
        u32x4 av[WN];
#pragma unroll
        for (int j = 0; j < WN; ++j) av[j] = live ? fa[cur][j] : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
          for (int j = 0; j < WN; ++j) acc[j][mt] = mfma16x16x32_bf16(av[j], fb[cur][mt], acc[j][mt]);
        if (live) after(c0 + kk);
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
template <int MT, int NW, int WN, int KC, int LDS_BUDGET = 96 * 1024, int NR = 1>
struct DmaCfg {
  static constexpr int ROWS = 16 * WN * (NW / NR) + 16 * MT;
  static constexpr int U = (ROWS * KC * 4 + 64 * NW - 1) / (64 * NW);
  static constexpr int CHB = U * 64 * NW * 16;
  static constexpr int BY_LDS = LDS_BUDGET / CHB;
  static constexpr int BY_VM = 63 / U + 2;
  static constexpr int NB0 = BY_LDS < BY_VM ? BY_LDS : BY_VM;
  static constexpr int NBUF = NB0 < 2 ? 2 : NB0;
  using G = DmaGemm<MT, NW, WN, KC, NBUF, NR>;
};

}  // namespace kve
