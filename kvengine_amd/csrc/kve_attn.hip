// Paged GQA verify attention for CDNA4 (gfx950).
//
// One launch computes, for every sequence of a batch, softmax(q k^T * scale) v
// over that sequence's paged history, for the q_len newest positions with the
// causal rule "query t sees keys 0..start+t". It replaces the reference's
// gather (kvengine/paged.py:315-331) + repeat_kv (forward.py:72-82) + masked
// SDPA (forward.py:85-144), which materialise the history and the expanded
// heads before attending.
//
// Work decomposition. A work item is (sequence, kv head, row group, split):
//  * the G = Hq/Hkv query heads of one kv head times the q_len queries form
//    G*q_len "rows" (row r = t*G + j); a row group is up to 64 of them, one
//    16-row tile per wave, so all the query heads sharing a kv head read each
//    K/V tile from HBM once (the workgroup's waves share it through L2/L1);
//  * the visible history is cut into 16-token key tiles (one tile = one block
//    of 16 tokens of one kv head: 2 KB of K and 2 KB of V in bf16 at D=64), and
//    a split is `split_tiles` consecutive tiles.
// Every wave walks all tiles of its split for its own 16 rows, so waves never
// exchange data: no LDS, no barrier.
//
// Per burst a wave issues the K/V loads of NPRE tiles (block ids come from one
// vector read of the table, picked out with readlane) straight into MFMA
// operand registers, and only then does math, so a burst costs one memory round
// trip. Scores come from S^T = K Q^T (keys on the M side, rows on the N side):
// each lane owns one query row (lane % 16) and 4 keys of every tile. The
// softmax is taken over the whole burst at once: one row max (two permlane
// swaps), a rare rescale, then P^T goes straight back as the B operand of
// O^T = V^T P^T. V is stored channel-major inside a block ([D][16]) so the A
// operand (4 keys of one channel per lane per tile) is one 8-byte load; two
// tiles fill the 32-deep k side of one 16x16x32 MFMA. In bf16, P is split into
// hi + lo bf16 halves so the P.V product carries 16 significant bits of P.
//
// A work item with one split writes the output; otherwise each wave writes an
// unnormalised partial (O, max, sum) for its rows and verify_attn_combine_kernel,
// launched next on the same stream, merges them.

#include "kve_common.h"
#include "kve_gemm.h"

#include <algorithm>
#include <type_traits>

namespace kve {

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  const int32_t* tables;
  const int32_t* seq_rows;
  const int32_t* start_pos;
  const int32_t* q_lens;
  float* part_o;   // [items][max_splits][ROWS][D]
  float* part_ml;  // [items][max_splits][ROWS][2]: (max, sum) per row
  int num_seqs, Tq, Hq, Hkv, G, bs, max_blocks, num_rows, num_blocks, max_ctx;
  int split_tiles, max_splits, row_groups;
  int lds_kv_off;  // ints from the start of dynamic LDS to the K/V chunk buffers
  int direct;      // 1: unit v = item * max_splits + split, no work list
  float scale_log2;
  uint32_t g_magic;  // ceil(2^32 / G) for G >= 2: row -> (query, head) without a division
};

// r / G for 0 <= r < 2^16 (the host checks G * q_len < 2^16): with
// m = ceil(2^32 / G) = (2^32 + e) / G, 0 <= e < G, r*m / 2^32 exceeds r/G by
// r*e / (G*2^32) < 2^-16 <= 1/G, which never reaches the next integer.
__device__ __forceinline__ int div_g(int r, const AttnArgs& a) {
  return a.G == 1 ? r : static_cast<int>(__umulhi(static_cast<uint32_t>(r), a.g_magic));
}

// A block id outside the pool is never dereferenced (block 0 is read instead).
__device__ __forceinline__ int safe_block(int blk, int num_blocks) {
  return static_cast<unsigned>(blk) < static_cast<unsigned>(num_blocks) ? blk : 0;
}

constexpr int kMaxSplits = 128;
constexpr float kNegBig = -1.0e30f;

template <int D, bool BF16>
struct AttnFrag;

// bf16: K is 8 bf16 per 32-channel MFMA step, V is 4 bf16 (4 keys) per 16-channel tile.
template <int D>
struct AttnFrag<D, true> {
  static constexpr int KS = D / 32;
  u32x4 k[KS];
  u32x2 v[D / 16];
};

template <int D>
struct AttnFrag<D, false> {
  static constexpr int KS = D / 4;
  float k[KS];
  f32x4 v[D / 16];
};

template <int D, bool BF16>
__device__ __forceinline__ void zero_v(AttnFrag<D, BF16>& f) {
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) {
    if constexpr (BF16) f.v[dt] = u32x2{0, 0};
    else f.v[dt] = f32x4{0, 0, 0, 0};
  }
}

// Slots past the visible history hold stale data; zero V there so a masked
// (p = 0) slot can never contribute 0 * inf. Applied when the tile is used, so
// the loads of a burst are all in flight before any of them is waited for.
template <int D, bool BF16>
__device__ __forceinline__ void mask_v_tail(AttnFrag<D, BF16>& f, int kt, int Lk, int lg) {
  if ((kt + 1) * 16 <= Lk) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (kt * 16 + 4 * lg + i >= Lk) {
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
        if constexpr (BF16) f.v[dt][i >> 1] &= (i & 1) ? 0x0000ffffu : 0xffff0000u;
        else f.v[dt][i] = 0.0f;
      }
    }
  }
}

// Channel mapping shared by Q and K fragments: lane group g (= lane/16) owns the
// contiguous quarter [g*D/4, (g+1)*D/4) of the head dimension.

// One 16-token block (block size 16): K row lr, V channels dt*16+lr, keys 4*lg..+3.
template <int D, bool BF16>
__device__ __forceinline__ void load_tile16(AttnFrag<D, BF16>& f, const AttnArgs& a, int blk,
                                            int kvh, int lr, int lg) {
  using elem_t = std::conditional_t<BF16, uint16_t, float>;
  constexpr int DQ = D / 4;
  const size_t tile = (static_cast<size_t>(blk) * a.Hkv + kvh) * 16 * D;
  const elem_t* kp = static_cast<const elem_t*>(a.k) + tile + lr * D + lg * DQ;
  const elem_t* vp = static_cast<const elem_t*>(a.v) + tile + lr * 16 + 4 * lg;
  if constexpr (BF16) {
#pragma unroll
    for (int s = 0; s < D / 32; ++s) f.k[s] = reinterpret_cast<const u32x4*>(kp)[s];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) f.v[dt] = *reinterpret_cast<const u32x2*>(vp + dt * 256);
  } else {
#pragma unroll
    for (int s = 0; s < DQ / 4; ++s) {
      const f32x4 x = reinterpret_cast<const f32x4*>(kp)[s];
      f.k[4 * s + 0] = x[0];
      f.k[4 * s + 1] = x[1];
      f.k[4 * s + 2] = x[2];
      f.k[4 * s + 3] = x[3];
    }
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) f.v[dt] = *reinterpret_cast<const f32x4*>(vp + dt * 256);
  }
}

// Any block size: resolve each key's (block, offset) separately.
template <int D, bool BF16>
__device__ __forceinline__ void load_tile_any(AttnFrag<D, BF16>& f, const AttnArgs& a,
                                              const int32_t* table, int kvh, int kt, int Lk,
                                              int lr, int lg) {
  using elem_t = std::conditional_t<BF16, uint16_t, float>;
  constexpr int DQ = D / 4;
  const elem_t* kb = static_cast<const elem_t*>(a.k);
  const elem_t* vb = static_cast<const elem_t*>(a.v);
  const int bs = a.bs;
  const int key = kt * 16 + lr;
  if (key < Lk) {
    const int blk = safe_block(table[key / bs], a.num_blocks);
    const elem_t* kp = kb + ((static_cast<size_t>(blk) * a.Hkv + kvh) * bs + key % bs) * D + lg * DQ;
    if constexpr (BF16) {
#pragma unroll
      for (int s = 0; s < D / 32; ++s) f.k[s] = reinterpret_cast<const u32x4*>(kp)[s];
    } else {
#pragma unroll
      for (int s = 0; s < DQ; ++s) f.k[s] = kp[s];
    }
  } else {
#pragma unroll
    for (int s = 0; s < AttnFrag<D, BF16>::KS; ++s) {
      if constexpr (BF16) f.k[s] = u32x4{0, 0, 0, 0};
      else f.k[s] = 0.0f;
    }
  }
  zero_v(f);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int kk = kt * 16 + 4 * lg + i;
    if (kk >= Lk) continue;
    const int blk = safe_block(table[kk / bs], a.num_blocks);
    const elem_t* vp = vb + (static_cast<size_t>(blk) * a.Hkv + kvh) * D * bs + kk % bs;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
      const elem_t x = vp[static_cast<size_t>(dt * 16 + lr) * bs];
      if constexpr (BF16) f.v[dt][i >> 1] |= static_cast<uint32_t>(x) << ((i & 1) * 16);
      else f.v[dt][i] = x;
    }
  }
}

// Tiles per wave per burst (two bursts are in registers at once: the one being
// multiplied and the next one loading). Even in bf16 (tiles pair up on the
// MFMA k side). 8 KB of K/V per wave per burst at D=64, 16 KB at D=128.
template <int D, bool BF16>
constexpr int burst_tiles() {
  return BF16 ? (D == 64 ? 4 : 2) : (D == 64 ? 2 : 1);
}

// Direct-to-LDS K/V windows (bf16, 16-token blocks, several row tiles): a tile
// is K [16][D] then V [D][16] in LDS, 64 * D bytes; a window holds 64 KB.
template <int D>
constexpr int kDmaTileBytes() {
  return 64 * D;
}
constexpr int kDmaWindowBytes = 64 * 1024;

// V chunk swizzle: a channel's two 16-byte chunks trade places when bit 2 xor
// bit 3 of the channel is set.
__device__ __forceinline__ int vsw(int ch) { return ((ch >> 2) ^ (ch >> 3)) & 1; }

// Per-sequence state read once by every workgroup of the attention kernel.
struct SeqInfo {
  int row, start, T;  // T = 0: sequence skipped (bad row or length)
};

__device__ __forceinline__ SeqInfo read_seq(const AttnArgs& a, int b) {
  SeqInfo q{0, 0, 0};
  const int row = a.seq_rows ? a.seq_rows[b] : b;
  if (row < 0 || row >= a.num_rows) return q;
  const int start = a.start_pos[row];
  const int T = a.q_lens ? min(a.q_lens[b], a.Tq) : a.Tq;
  if (T <= 0 || start < 0 || start + T > a.max_ctx) return q;
  q.row = row;
  q.start = start;
  q.T = T;
  return q;
}

// 16-token tiles visible to row group rg of a sequence (0 if the group is past q_len).
__device__ __forceinline__ int group_tiles(const AttnArgs& a, const SeqInfo& q, int rg, int rows) {
  const int R = a.G * q.T;
  const int row0 = rg * rows;
  if (q.T == 0 || row0 >= R) return 0;
  return cdiv(q.start + div_g(min(R, row0 + rows) - 1, a) + 1, 16);
}

// The attention kernel is persistent: every workgroup reads the lengths of the
// whole batch, builds the list of (sequence, row group, split) units in LDS,
// and takes units blockIdx.x, blockIdx.x + gridDim.x, ... (times the kv heads),
// so no workgroup is launched for work that turns out not to exist.
//
// Within a unit, one wave = one 16-row tile (times KW key waves): the
// workgroup's waves share the (sequence, kv head, split). With several row
// tiles (bf16, 16-token blocks) the unit's K/V tiles are copied into LDS once
// and every wave reads its fragments there; with one row tile each key wave
// loads its own tiles into registers.
//
// Dynamic LDS: SeqInfo[num_seqs], the unit prefix int[items + 1], then
// (16-byte aligned) the K/V window, which the key-wave merge reuses.
template <int D, bool BF16, int NT, bool BS16, int KW>
__global__ __launch_bounds__(64 * NT * KW) void paged_verify_attn_kernel(AttnArgs a) {
  using elem_t = std::conditional_t<BF16, uint16_t, float>;
  constexpr int NPRE = burst_tiles<D, BF16>();
  constexpr int ROWS = 16 * NT;
  constexpr int DT = D / 16;
  constexpr int DQ = D / 4;
  constexpr int KS = AttnFrag<D, BF16>::KS;
  // bf16 with 16-token blocks and several row tiles: the K/V tiles of the
  // unit are copied into LDS once per workgroup (direct loads, no registers)
  // and every row tile's waves read them there; with one row tile each key
  // wave loads its own bursts into registers.
  constexpr bool DMAKV = BF16 && BS16 && NT >= 2;
  constexpr int KI = D / 32;                      // 1 KB pieces per K (or V) tile
  constexpr int TI = 2 * KI;                      // per tile
  constexpr int UT = kDmaWindowBytes / kDmaTileBytes<D>();  // tiles per window
  static_assert(!DMAKV || UT % (KW * NPRE) == 0, "a window holds whole rounds of bursts");
  extern __shared__ int sm_dyn[];
  SeqInfo* sm_seq = reinterpret_cast<SeqInfo*>(sm_dyn);
  int* sm_pre = sm_dyn + 3 * a.num_seqs;

  const int tid = threadIdx.x;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nt = wid / KW;       // this wave's row tile
  const int kw = wid - nt * KW;  // and its share of the unit's key tiles
  const int l = tid & 63, lr = l & 15, lg = l >> 4;
  const int RG = a.row_groups;
  const int items = a.num_seqs * RG;


  // ---- work list, built by wave 0: per (sequence, row group) item, its
  // number of splits, as an exclusive prefix in LDS. When the launch has a
  // workgroup for every (item, split) slot (or one split at most), units map
  // to slots directly instead: each workgroup reads only its own sequence's
  // length, its table and Q loads go out at once, and the slots a sequence
  // does not fill end there -- one memory round trip less on every unit. ----
  const int st = a.split_tiles;
  const bool direct = a.direct != 0;
  if (!direct && wid == 0) {
    for (int b = l; b < a.num_seqs; b += 64) sm_seq[b] = read_seq(a, b);
    __builtin_amdgcn_wave_barrier();  // LDS is in order within a wave: the entries are visible
    int carry = 0;
    for (int i0 = 0; i0 < items; i0 += 64) {
      const int i = i0 + l;
      int n = 0;
      if (i < items) {
        const int b = RG == 1 ? i : i / RG;
        const SeqInfo sq = sm_seq[b];
        n = cdiv(group_tiles(a, sq, i - b * RG, ROWS), st);
      }
      int incl = n;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int x = __shfl_up(incl, o);
        if (l >= o) incl += x;
      }
      if (i < items) sm_pre[i] = carry + incl - n;
      carry += __shfl(incl, 63);
    }
    if (l == 0) sm_pre[items] = carry;
  }
  int nunits = items * a.max_splits * a.Hkv;
  if (!direct) {
    __syncthreads();
    nunits = __builtin_amdgcn_readfirstlane(sm_pre[items]) * a.Hkv;
  }

  const elem_t* qb = static_cast<const elem_t*>(a.q);
  const float c = a.scale_log2;

  for (int u = blockIdx.x; u < nunits; u += gridDim.x) {
    // ---- decode the unit: kv head fastest, then (item, split) ----
    const int kvh = u % a.Hkv;
    const int v = u / a.Hkv;
    int lo = a.max_splits == 1 ? v : v / a.max_splits;
    if (!direct) {
      lo = 0;
      int hi = items;  // largest i with sm_pre[i] <= v (units of empty items are skipped)
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (sm_pre[mid] <= v) lo = mid;
        else hi = mid;
      }
    }
    // everything about the unit is wave-uniform: keep it in scalar registers
    const int item = __builtin_amdgcn_readfirstlane(lo);
    const int s = __builtin_amdgcn_readfirstlane(v - (direct ? item * a.max_splits : sm_pre[item]));
    const int b = RG == 1 ? item : item / RG;
    const int rg = item - b * RG;
    SeqInfo sq = direct ? read_seq(a, b) : sm_seq[b];
    sq.row = __builtin_amdgcn_readfirstlane(sq.row);
    sq.start = __builtin_amdgcn_readfirstlane(sq.start);
    sq.T = __builtin_amdgcn_readfirstlane(sq.T);
    const int row0 = rg * ROWS;
    const int R = a.G * sq.T;
    if (direct && row0 >= R) continue;  // an empty item (the listed path never has its unit)
    const int r = row0 + nt * 16 + lr;  // this lane's row
    // A row tile wholly past q_len has nothing to compute; with K/V staged in
    // LDS the wave still takes its share of the loads and barriers.
    const bool active = row0 + nt * 16 < R;
    if (!DMAKV && KW == 1 && !active) continue;  // (key waves still meet at the merge)
    const int row_end = min(R, row0 + ROWS);
    const int Lk = sq.start + div_g(row_end - 1, a) + 1;  // keys visible to this row group
    const int ntiles = cdiv(Lk, 16);
    const int nsplit = cdiv(ntiles, st);
    if (direct && s >= nsplit) continue;  // a slot past the sequence's splits
    const int kt0 = s * st;
    const int kt1 = min(ntiles, kt0 + st);
    // With KW waves per row tile, wave kw takes bursts kw, kw + KW, ... of the
    // unit (bursts at fixed tile offsets from the unit start, so which wave
    // sums which keys, and in what order, does not depend on the history
    // length; the merge then adds the waves in order).
    const int first = kt0 + kw * NPRE;  // this wave's first burst
    const int qlim = r < R ? sq.start + div_g(r, a) : -1;  // last key this row sees
    const int32_t* table = a.tables + static_cast<size_t>(sq.row) * a.max_blocks;

    u32x4 qf16[BF16 ? KS : 1];
    float qf32[BF16 ? 1 : KS];
    {
      const bool ok = r < R;
      const int t = ok ? div_g(r, a) : 0;
      const int h = kvh * a.G + (ok ? r - t * a.G : 0);
      const elem_t* qp = qb + ((static_cast<size_t>(b) * a.Tq + t) * a.Hq + h) * D + lg * DQ;
      if constexpr (BF16) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          qf16[ks] = ok ? reinterpret_cast<const u32x4*>(qp)[ks] : u32x4{0, 0, 0, 0};
      } else {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qf32[ks] = ok ? qp[ks] : 0.0f;
      }
    }

    float m_run = kNegBig, l_run = 0.0f;
    f32x4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0, 0, 0, 0};

    // Bursts of NPRE tiles, double-buffered: the K/V loads of burst b+1 are in
    // flight while burst b is multiplied. Block ids come 64 tiles at a time
    // from one vector read of the table (lane i: tile c0 + i), picked out with
    // readlane; every tile slot of a burst is loaded (tiles past the split read
    // a clamped, in-range entry and are dropped by the math), so the number of
    // loads per burst is fixed and the wait for burst b never waits for b+1.
    int tv = 0;
    int c0 = kt0;
    auto issue = [&](AttnFrag<D, BF16> (&f)[NPRE], int r0) {
      if constexpr (BS16) {
#pragma unroll
        for (int j = 0; j < NPRE; ++j) {
          const int lane = min(r0 - c0 + j, 63);
          const int blk = safe_block(__builtin_amdgcn_readlane(tv, lane), a.num_blocks);
          load_tile16<D, BF16>(f[j], a, blk, kvh, lr, lg);
        }
      } else {
#pragma unroll
        for (int j = 0; j < NPRE; ++j) {
          if (r0 + j < kt1) load_tile_any<D, BF16>(f[j], a, table, kvh, r0 + j, Lk, lr, lg);
          else zero_v(f[j]);
        }
      }
    };
    auto consume = [&](AttnFrag<D, BF16> (&fr)[NPRE], int r0) {
      // ---- scores S^T = K Q^T of the burst; lane holds keys 4*lg..+3 of each tile ----
      f32x4 sc[NPRE];
#pragma unroll
      for (int j = 0; j < NPRE; ++j) {
        f32x4 acc_s = {0, 0, 0, 0};
        if (r0 + j < kt1) {
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            if constexpr (BF16) acc_s = mfma16x16x32_bf16(fr[j].k[ks], qf16[ks], acc_s);
            else acc_s = mfma16x16x4_f32(fr[j].k[ks], qf32[ks], acc_s);
          }
        }
        sc[j] = acc_s;
      }
      if constexpr (BS16) {
#pragma unroll
        for (int j = 0; j < NPRE; ++j) {
          if (r0 + j < kt1) mask_v_tail(fr[j], r0 + j, Lk, lg);
          else zero_v(fr[j]);
        }
      }

      // ---- one online-softmax step over the burst ----
      // Scores stay unscaled until the exponent: p = 2^(s*c - m) with m kept in
      // the scaled log2 domain, one FMA per score. Only tiles that straddle the
      // causal edge pay for masking (a wave-uniform test). The reference max m
      // moves only when a row's max grows by more than 8 (p then stays below
      // 256, harmless in fp32 and for the hi/lo split), so the rescale of the
      // accumulators is rare; the first burst has nothing to rescale.
      float smax = -INFINITY;
#pragma unroll
      for (int j = 0; j < NPRE; ++j) {
        const int kt = r0 + j;
        if (kt >= kt1) break;
        if (kt * 16 + 15 > sq.start) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (kt * 16 + 4 * lg + i > qlim) sc[j][i] = -INFINITY;
        }
        smax = fmaxf(fmaxf(smax, sc[j][0]), sc[j][1]);
        smax = fmaxf(fmaxf(smax, sc[j][2]), sc[j][3]);
      }
      smax = max_across_groups(smax);
      const float m_new = fmaxf(m_run, smax * c);
      float m_use = m_new;
      if (r0 != first) {
        const bool grow = m_new > m_run + 8.0f;
        m_use = grow ? m_new : m_run;
        if (__any(grow)) {
          const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
          l_run *= alpha;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
        }
      }
      m_run = m_use;
#pragma unroll
      for (int j = 0; j < NPRE; ++j) {
        if (r0 + j >= kt1) {
          sc[j] = f32x4{0, 0, 0, 0};
          continue;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sc[j][i] = __builtin_amdgcn_exp2f(fmaf(sc[j][i], c, -m_use));
          l_run += sc[j][i];
        }
      }

      // ---- O^T += V^T P^T ----
      if constexpr (BF16) {
#pragma unroll
        for (int jp = 0; jp < NPRE / 2; ++jp) {
          const int j0 = 2 * jp, j1 = j0 + 1;
          if (r0 + j0 >= kt1) break;
          // P = hi + lo: hi is p truncated to its top 16 bits (a bf16, exactly),
          // lo = p - hi (exact in fp32) rounded to bf16.
          u32x4 ph, pl;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float pa = sc[q < 2 ? j0 : j1][2 * (q & 1)];
            const float pb = sc[q < 2 ? j0 : j1][2 * (q & 1) + 1];
            const uint32_t ua = __float_as_uint(pa), ub = __float_as_uint(pb);
            ph[q] = __builtin_amdgcn_perm(ub, ua, 0x07060302u);
            pl[q] = pack_bf16x2(pa - __uint_as_float(ua & 0xffff0000u),
                                pb - __uint_as_float(ub & 0xffff0000u));
          }
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            const u32x4 va = {fr[j0].v[dt][0], fr[j0].v[dt][1], fr[j1].v[dt][0], fr[j1].v[dt][1]};
            acc[dt] = mfma16x16x32_bf16(va, ph, acc[dt]);
            acc[dt] = mfma16x16x32_bf16(va, pl, acc[dt]);
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < NPRE; ++j) {
          if (r0 + j >= kt1) break;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[dt] = mfma16x16x4_f32(fr[j].v[dt][i], sc[j][i], acc[dt]);
          }
        }
      }
    };

    if constexpr (DMAKV) {
      // Windows of up to UT tiles: every (K or V) 1 KB piece of the window is
      // one global_load_lds (16 bytes per lane, straight into LDS, no
      // registers), spread over the workgroup's waves, all in flight at once;
      // then each wave reads its bursts' MFMA fragments from LDS. A K row's
      // 16-byte chunks are stored XOR-swizzled by the row (c ^ (row & 7)) and a
      // V channel's two chunks by vsw(channel), so the fragment reads of
      // neighbouring lanes fall in different banks.
      char* kvl = reinterpret_cast<char*>(sm_dyn + a.lds_kv_off);
      const char* kg = static_cast<const char*>(a.k);
      const char* vg = static_cast<const char*>(a.v);
      auto dread = [&](AttnFrag<D, BF16> (&f)[NPRE], int t0) {
#pragma unroll
        for (int j = 0; j < NPRE; ++j) {
          const char* tb = kvl + (t0 + j) * kDmaTileBytes<D>();
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            const int cch = lg * (DQ / 8) + ks;
            f[j].k[ks] = *reinterpret_cast<const u32x4*>(tb + lr * 2 * D + ((cch ^ (lr & 7)) << 4));
          }
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            const int ch = dt * 16 + lr;
            f[j].v[dt] = *reinterpret_cast<const u32x2*>(
                tb + 32 * D + ch * 32 + (((lg >> 1) ^ vsw(ch)) << 4) + ((lg & 1) << 3));
          }
        }
      };
      for (int w0 = kt0; w0 < kt1; w0 += UT) {
        const int wn = min(UT, kt1 - w0);
        tv = table[min(w0 + l, a.max_blocks - 1)];
        for (int g = wid; g < wn * TI; g += NT * KW) {
          const int t = g / TI, part = g - t * TI;
          const int blk = safe_block(__builtin_amdgcn_readlane(tv, t), a.num_blocks);
          const size_t tb = (static_cast<size_t>(blk) * a.Hkv + kvh) * 16 * D;
          const char* src;
          if (part < KI) {
            const int j = part * 64 + l, row = j / (D / 8), pc = j - row * (D / 8);
            src = kg + (tb + static_cast<size_t>(row) * D) * 2 + ((pc ^ (row & 7)) << 4);
          } else {
            const int j = (part - KI) * 64 + l, ch = j >> 1;
            src = vg + (tb + static_cast<size_t>(ch) * 16) * 2 + (((j & 1) ^ vsw(ch)) << 4);
          }
          __builtin_amdgcn_global_load_lds(
              (__attribute__((address_space(1))) void*)(src),
              (__attribute__((address_space(3))) void*)(kvl + t * kDmaTileBytes<D>() + part * 1024),
              16, 0, 0);
        }
        barrier_after_vm<0>();  // this wave's pieces landed; after the barrier, everyone's
        if (active) {
          // bursts of this wave at fixed offsets kw * NPRE + m * KW * NPRE from
          // the unit start (UT is a multiple of KW * NPRE); tiles past kt1 hold
          // stale LDS and are dropped by consume
          for (int r0 = w0 + kw * NPRE; r0 < w0 + wn; r0 += KW * NPRE) {
            AttnFrag<D, BF16> fr[NPRE];
            dread(fr, r0 - w0);
            consume(fr, r0);
          }
        }
        __syncthreads();  // the window's LDS is rewritten by the next window, merge or unit
      }
    } else {
    constexpr int BSTEP = KW * NPRE;  // tiles between this wave's bursts (divides 64)
    AttnFrag<D, BF16> fa[NPRE], fb[NPRE];
    if (!active) c0 = kt1;  // an inactive row tile's key waves only take part in the merge
    for (; c0 < kt1; c0 += 64) {
      const int c1 = min(kt1, c0 + 64);
      const int b0 = c0 + kw * NPRE;
      if (b0 >= c1) continue;
      if constexpr (BS16) tv = table[min(c0 + l, a.max_blocks - 1)];
      issue(fa, b0);
      for (int r0 = b0; r0 < c1; r0 += 2 * BSTEP) {
        if (r0 + BSTEP < c1) issue(fb, r0 + BSTEP);
        consume(fa, r0);
        if (r0 + BSTEP >= c1) break;
        if (r0 + 2 * BSTEP < c1) issue(fa, r0 + 2 * BSTEP);
        consume(fb, r0 + BSTEP);
      }
    }
    }

    // ---- results: lane (lr, lg) holds O^T[channel dt*16 + 4*lg + i][row lr] ----
    if (KW == 1 && !active) continue;
    float lt = sum_across_groups(l_run);
    if constexpr (KW > 1) {
      // merge the KW waves' (max, sum, O) through LDS, in wave order
      // per row tile nt: [KW][16][2] (max, sum), then [KW][DT][64] accumulators
      float* sm_ml = reinterpret_cast<float*>(sm_dyn + a.lds_kv_off) + nt * KW * (32 + DT * 256);
      f32x4* sm_o = reinterpret_cast<f32x4*>(sm_ml + KW * 32);
      if (lg == 0) {
        sm_ml[(kw * 16 + lr) * 2] = m_run;
        sm_ml[(kw * 16 + lr) * 2 + 1] = lt;
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) sm_o[(kw * DT + dt) * 64 + l] = acc[dt];
      __syncthreads();
      if (kw == 0) {
        float M = m_run;
#pragma unroll
        for (int w = 1; w < KW; ++w) M = fmaxf(M, sm_ml[(w * 16 + lr) * 2]);
        const float a0 = __builtin_amdgcn_exp2f(m_run - M);
        lt *= a0;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] *= a0;
#pragma unroll
        for (int w = 1; w < KW; ++w) {
          const float aw = __builtin_amdgcn_exp2f(sm_ml[(w * 16 + lr) * 2] - M);
          lt += sm_ml[(w * 16 + lr) * 2 + 1] * aw;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) acc[dt] += sm_o[(w * DT + dt) * 64 + l] * aw;
        }
        m_run = M;
      }
      __syncthreads();  // the next unit rewrites these
      if (kw != 0 || !active) continue;
    }
    if (r >= R) continue;
    if (nsplit == 1) {
      const float inv = 1.0f / lt;
      const int t = div_g(r, a), h = kvh * a.G + r - t * a.G;
      elem_t* op =
          static_cast<elem_t*>(a.out) + ((static_cast<size_t>(b) * a.Tq + t) * a.Hq + h) * D + 4 * lg;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const f32x4 x = acc[dt] * inv;
        if constexpr (BF16) {
          *reinterpret_cast<u32x2*>(op + dt * 16) = u32x2{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])};
        } else {
          *reinterpret_cast<f32x4*>(op + dt * 16) = x;
        }
      }
      continue;
    }
    // split: unnormalised partial of this row tile
    const size_t slot =
        (static_cast<size_t>(b * a.Hkv + kvh) * RG + rg) * a.max_splits + s;
    float* po = a.part_o + (slot * ROWS + nt * 16 + lr) * D + 4 * lg;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4*>(po + dt * 16) = acc[dt];
    if (lg == 0) {
      float* pml = a.part_ml + (slot * ROWS + nt * 16 + lr) * 2;
      pml[0] = m_run;
      pml[1] = lt;
    }
  }
}

// Merge the split partials of one (sequence, kv head, row group):
// O = sum_s exp2(m_s - M) * acc_s / sum_s exp2(m_s - M) * l_s.
// Grid (items, D/16); thread (row, 4 channels). One pass: SPL splits' (m, l, O)
// loads are issued together, then folded into a running (M, L, O), so a merge
// of n splits costs about 1 + (n - 2)/SPL memory round trips. Work items with a
// single split were finished by the attention kernel and exit here at once.
template <int D, bool BF16, int NT>
__global__ __launch_bounds__(64 * NT) void verify_attn_combine_kernel(AttnArgs a) {
  using elem_t = std::conditional_t<BF16, uint16_t, float>;
  constexpr int ROWS = 16 * NT;
  constexpr int SPL = 16;
  const int tid = threadIdx.x;
  const int item = blockIdx.x;
  const int rg = item % a.row_groups;
  const int bk = item / a.row_groups;
  const int b = bk / a.Hkv, kvh = bk % a.Hkv;
  const int rr = tid >> 2;  // < ROWS: the block has 4 * ROWS threads
  const int d = blockIdx.y * 16 + (tid & 3) * 4;
  const float* po = a.part_o + static_cast<size_t>(item) * a.max_splits * ROWS * D + rr * D + d;
  const float* pml = a.part_ml + static_cast<size_t>(item) * a.max_splits * ROWS * 2 + 2 * rr;

  // Fold n splits of (o, m, l) into the running (x, M, L).
  float M = kNegBig, L = 0.0f;
  f32x4 x = {0, 0, 0, 0};
  auto fold = [&](const f32x4* o, const float* m, const float* lv, int n) {
    float cm = M;
    for (int u = 0; u < n; ++u) cm = fmaxf(cm, m[u]);
    const float al = __builtin_amdgcn_exp2f(M - cm);
    x *= al;
    L *= al;
    for (int u = 0; u < n; ++u) {
      const float f = __builtin_amdgcn_exp2f(m[u] - cm);
      x += o[u] * f;
      L += lv[u] * f;
    }
    M = cm;
  };
  // The first splits are read before the length is known (they lie inside
  // this item's partial slots whatever it turns out to be; slots the item did
  // not fill hold stale values that are discarded). Two: reading more ahead
  // (16) measured no faster on the lognormal verify batch and fetched the
  // stale slots of every short item from HBM.
  constexpr int SP0 = 2;
  f32x4 o0[SP0];
  float m0[SP0], l0[SP0];
#pragma unroll
  for (int u = 0; u < SP0; ++u) {
    if (u < a.max_splits) {
      o0[u] = *reinterpret_cast<const f32x4*>(po + static_cast<size_t>(u) * ROWS * D);
      m0[u] = pml[static_cast<size_t>(u) * ROWS * 2];
      l0[u] = pml[static_cast<size_t>(u) * ROWS * 2 + 1];
    }
  }
  const int st = a.split_tiles;
  const SeqInfo sq = read_seq(a, b);
  const int R = a.G * sq.T;
  const int row0 = rg * ROWS;
  if (sq.T == 0 || row0 >= R) return;
  const int row_end = min(R, row0 + ROWS);
  const int Lk = sq.start + div_g(row_end - 1, a) + 1;
  const int nsplit = cdiv(cdiv(Lk, 16), st);
  if (nsplit <= 1 || rr >= row_end - row0) return;
#pragma unroll
  for (int u = 0; u < SP0; ++u) {
    if (u >= nsplit) {
      o0[u] = f32x4{0, 0, 0, 0};
      m0[u] = -INFINITY;
      l0[u] = 0.0f;
    }
  }
  fold(o0, m0, l0, SP0);
  for (int s0 = SP0; s0 < nsplit; s0 += SPL) {
    f32x4 o[SPL];
    float m[SPL], lv[SPL];
#pragma unroll
    for (int u = 0; u < SPL; ++u) {
      if (s0 + u < nsplit) {
        const size_t sp = static_cast<size_t>(s0 + u);
        o[u] = *reinterpret_cast<const f32x4*>(po + sp * ROWS * D);
        m[u] = pml[sp * ROWS * 2];
        lv[u] = pml[sp * ROWS * 2 + 1];
      } else {
        o[u] = f32x4{0, 0, 0, 0};
        m[u] = -INFINITY;
        lv[u] = 0.0f;
      }
    }
    fold(o, m, lv, SPL);
  }
  x *= 1.0f / L;
  const int r = row0 + rr;
  const int t = div_g(r, a), h = kvh * a.G + r - t * a.G;
  elem_t* op = static_cast<elem_t*>(a.out) + ((static_cast<size_t>(b) * a.Tq + t) * a.Hq + h) * D + d;
  if constexpr (BF16) {
    *reinterpret_cast<u32x2*>(op) = u32x2{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])};
  } else {
    *reinterpret_cast<f32x4*>(op) = x;
  }
}

// ---- host side ----------------------------------------------------------------

// Row tiles (waves) per workgroup: every row of a (sequence, kv head) in one
// workgroup up to 128 rows, so the sequence's K/V is read from HBM once.
// Instantiated for 1-4, 6 and 8 tiles; 5 and 7 round up (the extra wave skips).
static int attn_row_tiles(int tiles) {
  if (tiles <= 4) return std::max(tiles, 1);
  return tiles <= 6 ? 6 : 8;
}

struct AttnPlan {
  int NT, KW, rows, row_groups, split_tiles, max_splits, items, lds_kv_off;
  size_t off_ml, off_o, bytes, lds;
};

// Work list limits per launch (the list lives in LDS: 12 bytes per sequence,
// 4 per (sequence, row group) pair).
constexpr int kMaxLaunchSeqs = 2048;
constexpr int kMaxLaunchItems = 8192;

// Default split (tiles): four bursts per wave. Finer splits shorten the
// attention kernel but lengthen the merge by as much or more on the lognormal
// 32-sequence verify batch this was tuned on.
static int default_split_tiles(int, int dtype) { return dtype == KVE_DTYPE_BF16 ? 16 : 8; }
constexpr int kNoSplitTiles = 64;
// Key waves of a one-row-tile unit (512 threads): 0.5B draft forward at 32
// rows 1080 -> 1062 us against 4, batched 32-request workload +0.9 %.
constexpr int kKW1 = 8;

static inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

static AttnPlan plan_attn(int num_seqs, int q_len, int Hq, int Hkv, int D, int max_ctx,
                          int split_blocks, int block_size, int dtype) {
  AttnPlan p{};
  const int rows = (Hq / Hkv) * q_len;
  const int tiles = cdiv(max_ctx, 16);
  // Short histories (<= 64 tiles, not split by default): one row tile per
  // workgroup with kKW1 key waves, so the rows of a kv head are spread over
  // several workgroups that re-read its K/V from L2 -- more parallelism per
  // sequence (3B verify pass at 32 x 5 tokens: 4.54 -> 4.18 ms, at 1 x 5:
  // 2.62 -> 2.49 ms). Longer histories share each K/V tile between up to 8
  // row tiles of one workgroup (the verify microbench: 16.1 vs 18.3 us).
  const bool short_ctx = split_blocks <= 0 && tiles <= kNoSplitTiles;
  p.NT = short_ctx ? 1 : attn_row_tiles(cdiv(rows, 16));
  p.rows = 16 * p.NT;
  p.row_groups = cdiv(rows, p.rows);
  // Key waves per row tile: with one row tile kKW1 waves share it, each taking
  // bursts kw, kw + KW, ... of the unit's key tiles, and a unit (the default
  // split) is 4 times longer; with 2-4 row tiles and units of 16 tiles or more, 2 waves per tile
  // halve each wave's walk (shorter units gain less than the merge costs).
  int st = split_blocks > 0
               ? (block_size == 16 ? split_blocks : cdiv(split_blocks * block_size, 16))
               : default_split_tiles(D, dtype);
  // A history of at most 64 tiles is not split by default: one unit per
  // (sequence, kv head, row group), no merge launch (measured +0.7 % on the
  // batched 32-request workload, whose contexts stay under 600 tokens).
  if (split_blocks <= 0 && tiles <= kNoSplitTiles) st = std::max(st, tiles);
  p.KW = p.NT == 1 ? kKW1 : (p.NT <= 4 && st >= 16 ? 2 : 1);
  if (p.NT == 1 && split_blocks <= 0) st *= 4;  // 64-tile units for one row tile
  st = std::max({st, 1, cdiv(tiles, kMaxSplits)});
  p.split_tiles = st;
  p.max_splits = cdiv(tiles, st);
  const size_t items = static_cast<size_t>(num_seqs) * Hkv * p.row_groups;
  p.items = static_cast<int>(items);
  p.off_ml = 0;
  if (p.max_splits > 1) {
    p.off_o = p.off_ml + align256(items * p.max_splits * p.rows * 2 * sizeof(float));
    p.bytes = p.off_o + align256(items * p.max_splits * p.rows * D * sizeof(float));
  } else {
    p.off_o = 0;
    p.bytes = 0;
  }
  p.lds = static_cast<size_t>(num_seqs) * sizeof(SeqInfo) +
          (static_cast<size_t>(num_seqs) * p.row_groups + 1) * sizeof(int);
  p.lds_kv_off = 0;
  // After the work list, 16-byte aligned: the direct-load K/V window (bf16,
  // 16-token blocks, several row tiles) and the key waves' (max, sum,
  // accumulators) for the in-workgroup merge, which reuses the window's LDS
  // once the unit's last window is consumed.
  size_t region = 0;
  if (dtype == KVE_DTYPE_BF16 && block_size == 16 && p.NT >= 2) region = kDmaWindowBytes;
  if (p.KW > 1)
    region = std::max(region, static_cast<size_t>(p.NT) * p.KW *
                                  (16 * 2 * sizeof(float) + (D / 16) * 64 * 16));
  if (region) {
    const size_t off = (p.lds + 15) & ~static_cast<size_t>(15);
    p.lds_kv_off = static_cast<int>(off / sizeof(int));
    p.lds = off + region;
  }
  return p;
}

// Workgroups of the persistent attention kernel: what the chip holds at once
// (occupancy of this instantiation, asked once per device and kept in `cache`),
// or fewer when the launch cannot have that many units.
template <typename K>
static int resident_workgroups(K kernel, int threads, size_t lds, int (&cache)[16]) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) dev = 0;
  if (cache[dev] == 0) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds) != hipSuccess ||
        per_cu <= 0)
      per_cu = 1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cache[dev] = per_cu * cus;
  }
  return cache[dev];
}

template <int D, bool BF16, int NT, int KW>
static int launch_attn_t(const AttnArgs& a0, const AttnPlan& p, bool split, hipStream_t st,
                         bool bs16) {
  AttnArgs a = a0;
  // Resident workgroups per device, one table per block-size path. Computed
  // with the work list of the first launch; a larger list later only lowers
  // how many of the launched workgroups are resident at once.
  static int occ[2][16] = {};
  static size_t granted[2] = {0, 0};  // dynamic LDS each block-size path may use
  const long long max_units = static_cast<long long>(p.items) * p.max_splits;
  auto go = [&](auto kernel, int (&cache)[16]) {
    size_t& g = granted[bs16 ? 1 : 0];
    if (p.lds > g && p.lds > 64 * 1024) {
      if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(p.lds)) != hipSuccess) {
        set_error("kve_paged_verify_attn: %zu bytes of LDS refused", p.lds);
        return KVE_ELAUNCH;
      }
      g = p.lds;
    }
    int nwg = resident_workgroups(kernel, 64 * NT * KW, p.lds, cache);
    // one workgroup per (item, split) slot when the chip holds them all
    a.direct = p.max_splits == 1 || max_units <= nwg;
    nwg = static_cast<int>(std::max(1LL, std::min<long long>(nwg, max_units)));
    hipLaunchKernelGGL(kernel, dim3(nwg), dim3(64 * NT * KW), p.lds, st, a);
    return KVE_OK;
  };
  const int rc = bs16 ? go(paged_verify_attn_kernel<D, BF16, NT, true, KW>, occ[1])
                      : go(paged_verify_attn_kernel<D, BF16, NT, false, KW>, occ[0]);
  if (rc) return rc;
  if (split)
    hipLaunchKernelGGL((verify_attn_combine_kernel<D, BF16, NT>), dim3(p.items, D / 16),
                       dim3(64 * NT), 0, st, a);
  return KVE_OK;
}

template <int D, bool BF16>
static int launch_attn_nt(const AttnArgs& a, const AttnPlan& p, bool split, hipStream_t st,
                          bool bs16) {
  if (p.NT == 1) return launch_attn_t<D, BF16, 1, kKW1>(a, p, split, st, bs16);
  if (p.NT == 2) return p.KW == 2 ? launch_attn_t<D, BF16, 2, 2>(a, p, split, st, bs16)
                                  : launch_attn_t<D, BF16, 2, 1>(a, p, split, st, bs16);
  if (p.NT == 3) return p.KW == 2 ? launch_attn_t<D, BF16, 3, 2>(a, p, split, st, bs16)
                                  : launch_attn_t<D, BF16, 3, 1>(a, p, split, st, bs16);
  if (p.NT == 4) return p.KW == 2 ? launch_attn_t<D, BF16, 4, 2>(a, p, split, st, bs16)
                                  : launch_attn_t<D, BF16, 4, 1>(a, p, split, st, bs16);
  if (p.NT == 6) return launch_attn_t<D, BF16, 6, 1>(a, p, split, st, bs16);
  return launch_attn_t<D, BF16, 8, 1>(a, p, split, st, bs16);
}

}  // namespace kve

using namespace kve;

extern "C" size_t kve_attn_workspace_bytes(int num_seqs, int q_len, int num_q_heads,
                                           int num_kv_heads, int head_dim, int block_size,
                                           int max_ctx, int split_blocks, int dtype) {
  if (num_seqs <= 0 || q_len <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || max_ctx <= 0 ||
      block_size <= 0 || num_q_heads % num_kv_heads != 0)
    return 0;
  return plan_attn(num_seqs, q_len, num_q_heads, num_kv_heads, head_dim, max_ctx, split_blocks,
                   block_size, dtype)
      .bytes;
}

extern "C" int kve_paged_verify_attn(const void* q, const void* k_pool, const void* v_pool,
                                     const int32_t* block_tables, const int32_t* seq_rows,
                                     const int32_t* start_pos, const int32_t* q_lens, int num_seqs,
                                     int q_len, int num_q_heads, int num_kv_heads, int head_dim,
                                     int block_size, int max_blocks, int num_rows, int num_blocks,
                                     int max_ctx, int split_blocks, float scale, int dtype,
                                     void* out, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  clear_error();
  if (num_seqs == 0) return KVE_OK;
  KVE_REQUIRE(q && k_pool && v_pool && block_tables && start_pos && out,
              "kve_paged_verify_attn: null pointer argument");
  KVE_REQUIRE(((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out) |
                reinterpret_cast<uintptr_t>(k_pool) | reinterpret_cast<uintptr_t>(v_pool)) &
               15) == 0,
              "kve_paged_verify_attn: q, out, k_pool and v_pool must be 16-byte aligned");
  KVE_REQUIRE(num_seqs > 0 && q_len > 0, "kve_paged_verify_attn: num_seqs=%d q_len=%d", num_seqs,
              q_len);
  KVE_REQUIRE(num_kv_heads > 0 && num_q_heads > 0 && num_q_heads % num_kv_heads == 0,
              "kve_paged_verify_attn: %d q heads not a multiple of %d kv heads", num_q_heads,
              num_kv_heads);
  KVE_REQUIRE(head_dim == 64 || head_dim == 128,
              "kve_paged_verify_attn: head_dim %d unsupported (64 or 128)", head_dim);
  KVE_REQUIRE(dtype == KVE_DTYPE_BF16 || dtype == KVE_DTYPE_F32,
              "kve_paged_verify_attn: dtype %d unsupported", dtype);
  KVE_REQUIRE(block_size > 0 && max_ctx > 0 && max_blocks >= cdiv(max_ctx, block_size),
              "kve_paged_verify_attn: max_blocks %d cannot hold max_ctx %d at block_size %d",
              max_blocks, max_ctx, block_size);
  KVE_REQUIRE(split_blocks >= 0, "kve_paged_verify_attn: split_blocks %d < 0", split_blocks);
  KVE_REQUIRE(static_cast<long long>(num_q_heads) * q_len < 65536 &&
                  static_cast<long long>(num_seqs) * q_len * num_q_heads * head_dim < (1ll << 31),
              "kve_paged_verify_attn: q of %d x %d x %d heads too large for one launch", num_seqs,
              q_len, num_q_heads);
  KVE_REQUIRE(num_rows > 0 && num_blocks > 0, "kve_paged_verify_attn: num_rows=%d num_blocks=%d",
              num_rows, num_blocks);
  const AttnPlan p = plan_attn(num_seqs, q_len, num_q_heads, num_kv_heads, head_dim, max_ctx,
                               split_blocks, block_size, dtype);
  KVE_REQUIRE(num_seqs <= kMaxLaunchSeqs, "kve_paged_verify_attn: %d sequences exceed %d per launch",
              num_seqs, kMaxLaunchSeqs);
  KVE_REQUIRE(static_cast<long long>(num_seqs) * p.row_groups <= kMaxLaunchItems,
              "kve_paged_verify_attn: %d sequences x %d row groups exceed %d per launch", num_seqs,
              p.row_groups, kMaxLaunchItems);
  if (p.max_splits > 1) {
    KVE_REQUIRE(workspace != nullptr, "kve_paged_verify_attn: workspace required");
    if (workspace_bytes < p.bytes) {
      set_error("kve_paged_verify_attn: workspace %zu bytes, need %zu", workspace_bytes, p.bytes);
      return KVE_EWORKSPACE;
    }
    KVE_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15) == 0,
                "kve_paged_verify_attn: workspace must be 16-byte aligned");
  }
  AttnArgs a;
  a.q = q;
  a.k = k_pool;
  a.v = v_pool;
  a.out = out;
  a.tables = block_tables;
  a.seq_rows = seq_rows;
  a.start_pos = start_pos;
  a.q_lens = q_lens;
  const bool split = p.max_splits > 1;
  char* ws = static_cast<char*>(workspace);
  a.part_ml = split ? reinterpret_cast<float*>(ws + p.off_ml) : nullptr;
  a.part_o = split ? reinterpret_cast<float*>(ws + p.off_o) : nullptr;
  a.num_seqs = num_seqs;
  a.Tq = q_len;
  a.Hq = num_q_heads;
  a.Hkv = num_kv_heads;
  a.G = num_q_heads / num_kv_heads;
  a.bs = block_size;
  a.max_blocks = max_blocks;
  a.num_rows = num_rows;
  a.num_blocks = num_blocks;
  a.max_ctx = max_ctx;
  a.split_tiles = p.split_tiles;
  a.max_splits = p.max_splits;
  a.row_groups = p.row_groups;
  a.lds_kv_off = p.lds_kv_off;
  a.direct = 0;  // chosen per launch from the occupancy
  a.scale_log2 = scale * 1.4426950408889634f;
  a.g_magic = a.G >= 2 ? static_cast<uint32_t>(((1ull << 32) + a.G - 1) / a.G) : 0u;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool bs16 = block_size == 16;
  int rc;
  if (dtype == KVE_DTYPE_BF16) {
    rc = head_dim == 64 ? launch_attn_nt<64, true>(a, p, split, st, bs16)
                        : launch_attn_nt<128, true>(a, p, split, st, bs16);
  } else {
    rc = head_dim == 64 ? launch_attn_nt<64, false>(a, p, split, st, bs16)
                        : launch_attn_nt<128, false>(a, p, split, st, bs16);
  }
  if (rc) return rc;
  return check_launch("kve_paged_verify_attn");
}
