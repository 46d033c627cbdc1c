// Paged GQA verify attention for CDNA4 (gfx950).
//
// One launch computes, for every sequence of a batch, softmax(q k^T * scale) v
// over that sequence's paged history, for the q_len newest positions with the
// causal rule "query t sees keys 0..start+t". It replaces the reference's
// gather (kvengine/paged.py:315-331) + repeat_kv (forward.py:72-82) + masked
// SDPA (forward.py:85-144), which materialise the history and the expanded
// heads before attending.
//
// Work decomposition.
//  * Rows: the G = Hq/Hkv query heads of one kv head times the q_len queries
//    form G*q_len rows (row r = t*G + j); a row group is 16*NT of them, one
//    16-row tile per wave, so the heads sharing a kv head read each K/V tile
//    once per row group.
//  * Keys: the visible history is cut into 16-token tiles (one tile = one
//    block of 16 tokens of one kv head). An item (sequence, row group) is cut
//    into units of U tiles at fixed offsets (unit k = tiles [kU, kU + U)).
//  * Plan: a small kernel run once per forward pass (every layer has the same
//    lengths and tables) writes one 256-byte record per unit -- sequence, row
//    group, tile range, table row, lengths and the unit's block ids -- and one
//    record per item that has more than one unit. A layer's attention then
//    needs one dependent load (its record) before the K/V loads, and the merge
//    kernel runs over the split items only.
//  * A unit is one workgroup of NT row tiles x KW key waves (persistent: units
//    blockIdx.x, + gridDim.x, ... times the kv heads). Key wave kw takes the
//    unit's bursts of NPRE tiles at offsets kw*NPRE, kw*NPRE + KW*NPRE, ... from
//    the unit start. An item of one unit writes its output; the units of a
//    longer one write their states and a small merge kernel, launched next on
//    the same stream when max_ctx allows more than one unit, folds them.
//
// Summation order. Each wave keeps an online-softmax state (m, l, O) over its
// bursts; the unit's state is the fold of its waves' states in wave order, and
// a split item's result is the fold of its units' states in unit order, with
// the same fold (fold_state) in both places. Keys a row cannot see contribute
// exactly nothing (p = 0; a state with no visible key folds as the identity).
// So a row's result depends only on its query, its visible keys and (U, KW):
// not on q_len, on which other sequences or rows share the launch, or on how
// many units its item has. Callers that need results independent of the batch
// (the batched speculative engine's target model) fix U and KW.
//
// Per burst a wave issues the K/V loads of NPRE tiles straight into MFMA
// operand registers (one row tile), or the workgroup streams the unit's tiles
// through NBUF chunk buffers in LDS with direct loads (several row tiles: the
// loads of the next chunks are in flight while a chunk is multiplied). Scores
// come from S^T = K Q^T (keys on the M side, rows on the N side): each lane
// owns one query row (lane % 16) and 4 keys of every tile. The softmax is
// taken over the whole burst at once: one row max (two permlane swaps), a
// rare rescale, then P^T goes straight back as the B operand of
// O^T = V^T P^T. V is stored channel-major inside a block ([D][16]) so the A
// operand (4 keys of one channel per lane per tile) is one 8-byte load; two
// tiles fill the 32-deep k side of one 16x16x32 MFMA. In bf16, P is split into
// hi + lo bf16 halves so the P.V product carries 16 significant bits of P (a
// single bf16 P, as the reference's eager path rounds it, forward.py:141-144,
// measured 2.3-2.6e-3 relative RMS from exact attention on the verify
// microbench against 1.2e-3 with the split), and the row sums l are the
// product of a row of ones with the same hi and lo P^T on the matrix cores
// instead of VALU adds.

#include "kve_common.h"
#include "kve_gemm.h"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace kve {

// ---- plan layout (int32) --------------------------------------------------------
// [0, kPlanHead): header: units, split items, unit_tiles, row_groups, rows, max_units
// then max_units unit records of kRecInts ints:
//   [0] sequence  [1] row group  [2] first tile  [3] tiles
//   [4] state slot of this unit (-1: the item has one unit; else split item
//   index * max_item_units + unit index)  [5] table row  [6] start  [7] q_len
//   [8 + j] block id of tile first + j (16-token blocks; j < tiles)
// then max_split split-item records of kSplitInts ints:
//   [0] sequence  [1] row group  [2] units  [3] q_len
constexpr int kPlanHead = 16;
constexpr int kRecInts = 64;
constexpr int kRecHead = 8;
constexpr int kMaxUnitTiles = kRecInts - kRecHead;  // 56
constexpr int kSplitInts = 4;

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  const int32_t* tables;
  const int32_t* seq_rows;
  const int32_t* start_pos;
  const int32_t* q_lens;
  int32_t* plan;   // written by the plan kernel, read by the attention and merge kernels
  float* part_o;   // [slot][Hkv][ROWS][D]: unit states of split items
  float* part_ml;  // [slot][Hkv][ROWS][2]: (max, sum) per row
  int num_seqs, Tq, Hq, Hkv, G, bs, max_blocks, num_rows, num_blocks, max_ctx;
  int unit_tiles, row_groups, rows;  // rows per group = 16 * NT
  int max_units, max_split, max_item_units;
  int lds_kv_off;  // ints from the start of dynamic LDS to the K/V window / merge area
  int out_blocked;  // out in the 16 x 32 blocked layout of [Tq rows per sequence, Hq * D]
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

constexpr float kNegBig = -1.0e30f;

// The fold of two online-softmax states (m, l, O) -> (max m, l*2^(m-M) + ...).
// Used for the waves of a unit and for the units of an item, so both give the
// same bits for the same sequence of states. A state with no visible key
// (m = kNegBig, l = 0, O = 0) folds as the identity: M keeps its value, the
// old state is scaled by 2^0 = 1 and the new one by 2^(kNegBig - M) = 0.
template <int N>
__device__ __forceinline__ void fold_state(float& M, float& L, f32x4 (&O)[N], float m, float l,
                                           const f32x4 (&o)[N]) {
  const float Mn = fmaxf(M, m);
  const float al = __builtin_amdgcn_exp2f(M - Mn);
  const float be = __builtin_amdgcn_exp2f(m - Mn);
  L = fmaf(l, be, L * al);
#pragma unroll
  for (int i = 0; i < N; ++i) {
#pragma unroll
    for (int c = 0; c < 4; ++c) O[i][c] = fmaf(o[i][c], be, O[i][c] * al);
  }
  M = Mn;
}

// ---- fp32 operands (16x16x4 MFMA), one 16-token tile at a time -------------------
// K: lane (row lr, group lg) holds channels lg*D/4 .. of key row lr (one MFMA
// per channel); V: channel dt*16 + lr, keys 4*lg .. 4*lg + 3.
template <int D>
struct F32Frag {
  static constexpr int KS = D / 4;
  float k[KS];
  f32x4 v[D / 16];
};

template <int D>
__device__ __forceinline__ void zero_v(F32Frag<D>& f) {
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) f.v[dt] = f32x4{0, 0, 0, 0};
}

// Slots past the visible history hold stale data; zero V there so a masked
// (p = 0) slot can never contribute 0 * inf. Applied when the tile is used, so
// the loads of a burst are all in flight before any of them is waited for.
template <int D>
__device__ __forceinline__ void mask_v_tail(F32Frag<D>& f, int kt, int Lk, int lg) {
  if ((kt + 1) * 16 <= Lk) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (kt * 16 + 4 * lg + i >= Lk) {
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) f.v[dt][i] = 0.0f;
    }
  }
}

// One 16-token block (block size 16): K row lr, V channels dt*16+lr, keys 4*lg..+3.
template <int D>
__device__ __forceinline__ void load_tile16(F32Frag<D>& f, const AttnArgs& a, int blk, int kvh,
                                            int lr, int lg) {
  constexpr int DQ = D / 4;
  const size_t tile = (static_cast<size_t>(blk) * a.Hkv + kvh) * 16 * D;
  const float* kp = static_cast<const float*>(a.k) + tile + lr * D + lg * DQ;
  const float* vp = static_cast<const float*>(a.v) + tile + lr * 16 + 4 * lg;
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

// Any block size: resolve each key's (block, offset) separately; keys at or
// past Lk read as zero.
template <int D>
__device__ __forceinline__ void load_tile_any(F32Frag<D>& f, const AttnArgs& a,
                                              const int32_t* table, int kvh, int kt, int Lk,
                                              int lr, int lg) {
  constexpr int DQ = D / 4;
  const float* kb = static_cast<const float*>(a.k);
  const float* vb = static_cast<const float*>(a.v);
  const int bs = a.bs;
  const int key = kt * 16 + lr;
  if (key < Lk) {
    const int blk = safe_block(table[key / bs], a.num_blocks);
    const float* kp = kb + ((static_cast<size_t>(blk) * a.Hkv + kvh) * bs + key % bs) * D + lg * DQ;
#pragma unroll
    for (int s = 0; s < DQ; ++s) f.k[s] = kp[s];
  } else {
#pragma unroll
    for (int s = 0; s < DQ; ++s) f.k[s] = 0.0f;
  }
  zero_v(f);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int kk = kt * 16 + 4 * lg + i;
    if (kk >= Lk) continue;
    const int blk = safe_block(table[kk / bs], a.num_blocks);
    const float* vp = vb + (static_cast<size_t>(blk) * a.Hkv + kvh) * D * bs + kk % bs;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) f.v[dt][i] = vp[static_cast<size_t>(dt * 16 + lr) * bs];
  }
}

// ---- bf16 operands (16x16x32 MFMA), pairs of 16-token tiles ----------------------
// A pair is two consecutive tiles, 32 keys: pair key j < 16 is key j of the
// first tile, j >= 16 key j - 16 of the second. On the 32-deep k side of
// O^T = V^T P^T, lane group g (lane / 16) holds pair keys 8g .. 8g + 7, so its
// V operand is 8 consecutive keys of one channel (16 bytes of the
// channel-major [D][16] tile: one load, no register moves) and its P operand
// the same keys. The pair's two score MFMAs S^T = K Q^T (h = 0, 1) put pair
// key 8 (r / 4) + 4h + r % 4 on A row r, so value i of output lane (row lr,
// group g) is pair key 8g + 4h + i: the scores a lane ends with are exactly
// the P^T slots it feeds back. Channels: lane group g owns the contiguous
// quarter [g*D/4, (g+1)*D/4) of the head dimension in Q and K.
__device__ __forceinline__ int pair_key_of_row(int r, int h) {
  return 8 * (r >> 2) + 4 * h + (r & 3);
}

template <int D>
struct PairFrag {
  static constexpr int KS = D / 32;
  u32x4 k[2][KS];   // [h][k-step]: K row pair_key_of_row(lr, h), channels lg*D/4 + 8 ks ..
  u32x4 v[D / 16];  // [dt]: channel dt*16 + lr, pair keys 8 lg .. 8 lg + 7
};

// Any block size: each key's (block, offset) resolved separately; keys at or
// past `lim` read as zero (K and V).
template <int D>
__device__ __forceinline__ void load_pair_any(PairFrag<D>& f, const AttnArgs& a,
                                              const int32_t* table, int kvh, int kt, int lim,
                                              int lr, int lg) {
  constexpr int DQ = D / 4;
  const uint16_t* kb = static_cast<const uint16_t*>(a.k);
  const uint16_t* vb = static_cast<const uint16_t*>(a.v);
  const int bs = a.bs;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int key = kt * 16 + pair_key_of_row(lr, h);
    if (key < lim) {
      const int blk = safe_block(table[key / bs], a.num_blocks);
      const uint16_t* kp =
          kb + ((static_cast<size_t>(blk) * a.Hkv + kvh) * bs + key % bs) * D + lg * DQ;
#pragma unroll
      for (int ks = 0; ks < D / 32; ++ks) f.k[h][ks] = reinterpret_cast<const u32x4*>(kp)[ks];
    } else {
#pragma unroll
      for (int ks = 0; ks < D / 32; ++ks) f.k[h][ks] = u32x4{0, 0, 0, 0};
    }
  }
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) f.v[dt] = u32x4{0, 0, 0, 0};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int key = kt * 16 + 8 * lg + e;
    if (key >= lim) continue;
    const int blk = safe_block(table[key / bs], a.num_blocks);
    const uint16_t* vp = vb + (static_cast<size_t>(blk) * a.Hkv + kvh) * D * bs + key % bs;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
      f.v[dt][e >> 1] |= static_cast<uint32_t>(vp[static_cast<size_t>(dt * 16 + lr) * bs])
                         << ((e & 1) * 16);
  }
}


// Tiles per wave per burst (with one row tile two bursts are in registers at
// once: the one being multiplied and the next one loading). Even in bf16
// (tiles pair up on the MFMA k side).
constexpr int kBurstBf16D64 = 4;
constexpr int kBurstBf16D128 = 2;
template <int D, bool BF16>
__host__ __device__ constexpr int burst_tiles() {
  return BF16 ? (D == 64 ? kBurstBf16D64 : kBurstBf16D128) : (D == 64 ? 2 : 1);
}

// Direct-to-LDS K/V chunks (bf16, 16-token blocks, several row tiles): a tile
// is K [16][D] then V [D][16] in LDS, 64 * D bytes; a chunk is one round of
// bursts of the unit (KW * NPRE tiles).
template <int D>
__host__ __device__ constexpr int kDmaTileBytes() {
  return 64 * D;
}
// Chunk buffers of a workgroup: 64 KB when two workgroups share a CU (up to 6
// waves), 128 KB for one of 8-12 waves, between 2 and 8 chunks; NBUF - 1
// chunks load while one is multiplied. Measured on one box, runs repeated
// (per-workgroup timestamps and HIP-graph timings): at D = 64 with two key
// waves, 4-tile bursts (one 32 KB chunk loading while one is multiplied)
// beat 2-tile bursts with three 16 KB chunks in flight: verify microbench
// 14.4 vs 15.1 us, 32 x 4096 tokens 24.1 vs 27.5 us; 96 KB of buffers leaves
// one workgroup per CU (32 x 4096: 32.7 us).
template <int D>
__host__ __device__ constexpr int dma_nbuf(int NT, int KW) {
  const int bytes = NT * KW >= 8 ? 128 * 1024 : 64 * 1024;
  const int n = bytes / (KW * burst_tiles<D, true>() * kDmaTileBytes<D>());
  return n < 2 ? 2 : n > 8 ? 8 : n;
}

// V chunk swizzle: a channel's two 16-byte chunks trade places when bit 2 xor
// bit 3 of the channel is set.
__device__ __forceinline__ int vsw(int ch) { return ((ch >> 2) ^ (ch >> 3)) & 1; }

// K chunk swizzle: a K row's 16-byte chunk c of a tile sits at
// c ^ ksw(row, tile), so the 16 lanes of a fragment read (rows
// pair_key_of_row(lane, h) of a pair's two tiles, one 16-byte chunk each)
// cover the 16 distinct 16-byte bank groups of a 256-byte LDS line: at D = 64
// two rows share a line (the row's half and (row / 2) % 8 pick the group), at
// D = 128 a row is a line; the tile's parity moves the second tile's rows to
// the groups the first tile's leave free.
template <int D>
__device__ __forceinline__ int ksw(int row, int tile) {
  return D == 64 ? (((row >> 1) & 7) ^ ((tile & 1) << 1)) : ((row & 15) ^ ((tile & 1) << 2));
}


// This wave's vector-memory operations down to at most N outstanding (its
// direct-to-LDS loads older than those have landed and are visible to it),
// no LDS operation pending; the "memory" clobbers keep LDS reads after it.
template <int N>
__device__ __forceinline__ void wave_wait_vm() {
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(N));
  __asm__ volatile("" ::: "memory");
}

// Workgroup barrier once this wave has at most `ahead` chunks of LPW direct
// loads outstanding (0 <= ahead <= K; the count must be an immediate).
template <int LPW, int K>
__device__ __forceinline__ void barrier_after_chunks(int ahead) {
  if constexpr (K > 0) {
    if (ahead >= K) {
      barrier_after_vm<K * LPW>();
      return;
    }
    barrier_after_chunks<LPW, K - 1>(ahead);
  } else {
    barrier_after_vm<0>();
  }
}

// Per-sequence state of a launch.
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
__device__ __forceinline__ int group_tiles(const AttnArgs& a, const SeqInfo& q, int rg) {
  const int R = a.G * q.T;
  const int row0 = rg * a.rows;
  if (q.T == 0 || row0 >= R) return 0;
  return cdiv(q.start + div_g(min(R, row0 + a.rows) - 1, a) + 1, 16);
}

// ---- plan kernel -----------------------------------------------------------------
// Items are (sequence, row group). Every workgroup scans the items' unit counts
// (units and split items) in LDS -- a few hundred items, cheaper than a second
// launch -- then writes its share of the records: wave w of workgroup g takes
// records (g * 16 + w) + k * 16 * gridDim.x, lane j writing int j, so the table
// reads of many records are in flight at once. Workgroup 0 writes the header
// and the split-item records.
constexpr int kPlanThreads = 1024;

__global__ __launch_bounds__(kPlanThreads) void attn_plan_kernel(AttnArgs a) {
  extern __shared__ int sm_plan[];
  const int items = a.num_seqs * a.row_groups;
  int* sm_u = sm_plan;           // exclusive prefix of units, [items + 1]
  int* sm_s = sm_u + items + 1;  // exclusive prefix of split items, [items]
  int* sm_n = sm_s + items;      // tiles of the item, [items]
  SeqInfo* sm_q = reinterpret_cast<SeqInfo*>(sm_n + items);  // per sequence
  __shared__ int sm_wsum[2][kPlanThreads / 64];
  const int tid = threadIdx.x, l = tid & 63, w = tid >> 6;
  const int U = a.unit_tiles;
  int32_t* recs = a.plan + kPlanHead;
  int32_t* splits = recs + static_cast<size_t>(a.max_units) * kRecInts;
  for (int b = tid; b < a.num_seqs; b += kPlanThreads) sm_q[b] = read_seq(a, b);
  __syncthreads();
  int carry_u = 0, carry_s = 0;
  for (int i0 = 0; i0 < items; i0 += kPlanThreads) {
    const int i = i0 + tid;
    int n = 0, nu = 0;
    if (i < items) {
      const int b = i / a.row_groups;
      n = group_tiles(a, sm_q[b], i - b * a.row_groups);
      nu = cdiv(n, U);
      sm_n[i] = n;
    }
    const int ns = nu > 1 ? 1 : 0;
    int iu = nu, is = ns;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int xu = __shfl_up(iu, o), xs = __shfl_up(is, o);
      if (l >= o) {
        iu += xu;
        is += xs;
      }
    }
    if (l == 63) {
      sm_wsum[0][w] = iu;
      sm_wsum[1][w] = is;
    }
    __syncthreads();
    int wu = 0, ws = 0, tu = 0, ts = 0;
    for (int q = 0; q < kPlanThreads / 64; ++q) {
      if (q < w) {
        wu += sm_wsum[0][q];
        ws += sm_wsum[1][q];
      }
      tu += sm_wsum[0][q];
      ts += sm_wsum[1][q];
    }
    if (i < items) {
      sm_u[i] = carry_u + wu + iu - nu;
      sm_s[i] = carry_s + ws + is - ns;
    }
    carry_u += tu;
    carry_s += ts;
    __syncthreads();  // sm_wsum is rewritten by the next round
  }
  if (tid == 0) sm_u[items] = carry_u;
  __syncthreads();
  const int nunits = min(carry_u, a.max_units);
  if (blockIdx.x == 0) {
    if (tid == 0) {
      int32_t* h = a.plan;
      h[0] = nunits;
      h[1] = min(carry_s, a.max_split);
      h[2] = U;
      h[3] = a.row_groups;
      h[4] = a.rows;
      h[5] = a.max_units;
    }
    for (int i = tid; i < items; i += kPlanThreads) {
      const int nu = cdiv(sm_n[i], U);
      if (nu <= 1 || sm_s[i] >= a.max_split) continue;
      const int b = i / a.row_groups;
      int32_t* r = splits + static_cast<size_t>(sm_s[i]) * kSplitInts;
      r[0] = b;
      r[1] = i - b * a.row_groups;
      r[2] = nu;
      r[3] = sm_q[b].T;
    }
  }
  const int wstride = (kPlanThreads / 64) * gridDim.x;
  for (int u = blockIdx.x * (kPlanThreads / 64) + w; u < nunits; u += wstride) {
    int lo = 0, hi = items;  // largest i with sm_u[i] <= u
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (sm_u[mid] <= u) lo = mid;
      else hi = mid;
    }
    const int i = lo, k = u - sm_u[i];
    const int b = i / a.row_groups, rg = i - b * a.row_groups;
    const SeqInfo q = sm_q[b];
    const int n = sm_n[i];
    const int nu = cdiv(n, U);
    const int t0 = k * U, nt = min(U, n - t0);
    int val;
    if (l >= kRecHead) {
      // block id of tile t0 + j (the last one repeated past the unit, so every
      // lane of a burst reads an in-range entry)
      const int j = min(l - kRecHead, nt - 1);
      val = a.bs == 16 ? a.tables[static_cast<size_t>(q.row) * a.max_blocks + t0 + j] : 0;
    } else {
      const int slot = nu > 1 && sm_s[i] < a.max_split ? sm_s[i] * a.max_item_units + k : -1;
      const int hv[kRecHead] = {b, rg, t0, nt, slot, q.row, q.start, q.T};
      val = hv[0];
#pragma unroll
      for (int x = 1; x < kRecHead; ++x)
        if (l == x) val = hv[x];
    }
    recs[static_cast<size_t>(u) * kRecInts + l] = val;
  }
}

// What a wave knows of its unit: the record's fields (wave-uniform) and its
// own row r (lane % 16 of row tile nt) with the last key that row sees.
struct UnitInfo {
  int kvh, b, kt0, kt1, pslot, srow, start, R, r, Lk, qlim;
  bool active;  // the wave's row tile has rows below R
};

template <int NT>
__device__ __forceinline__ UnitInfo unit_info(const AttnArgs& a, int rec, int u, int nt, int lr) {
  UnitInfo x;
  x.kvh = u % a.Hkv;
  x.b = __builtin_amdgcn_readlane(rec, 0);
  const int rg = __builtin_amdgcn_readlane(rec, 1);
  x.kt0 = __builtin_amdgcn_readlane(rec, 2);
  x.kt1 = x.kt0 + __builtin_amdgcn_readlane(rec, 3);
  x.pslot = __builtin_amdgcn_readlane(rec, 4);
  x.srow = __builtin_amdgcn_readlane(rec, 5);
  x.start = __builtin_amdgcn_readlane(rec, 6);
  const int T = __builtin_amdgcn_readlane(rec, 7);
  const int row0 = rg * 16 * NT;
  x.R = a.G * T;
  x.r = row0 + nt * 16 + lr;
  x.active = row0 + nt * 16 < x.R;
  const int row_end = min(x.R, row0 + 16 * NT);
  x.Lk = x.start + div_g(row_end - 1, a) + 1;  // keys visible to the row group
  x.qlim = x.r < x.R ? x.start + div_g(x.r, a) : -1;
  return x;
}

// End of a unit: the KW key waves' states are folded in wave order through
// LDS (waves 1..KW-1 of row tile nt store (max, sum) [KW-1][16][2] and O
// [KW-1][DT][64], wave 0 folds them into its own), then wave 0 writes its
// rows: the normalised output for an item of one unit, else the unit's state
// for verify_attn_merge_kernel. Every wave of the workgroup calls it (KW > 1
// has barriers). Lane (lr, lg) holds O^T[channel dt*16 + 4*lg + i][row lr].
template <int D, bool BF16, int NT, int KW>
__device__ __forceinline__ void finish_unit(const AttnArgs& a, const UnitInfo& x, int* sm, int nt,
                                            int kw, int l, float m_run, float lt,
                                            f32x4 (&acc)[D / 16]) {
  using elem_t = std::conditional_t<BF16, uint16_t, float>;
  constexpr int DT = D / 16;
  constexpr int ROWS = 16 * NT;
  const int lr = l & 15, lg = l >> 4;
  if constexpr (KW > 1) {
    float* sm_ml = reinterpret_cast<float*>(sm + a.lds_kv_off) + nt * (KW - 1) * (32 + DT * 256);
    f32x4* sm_o = reinterpret_cast<f32x4*>(sm_ml + (KW - 1) * 32);
    if (kw > 0) {
      if (lg == 0) {
        sm_ml[((kw - 1) * 16 + lr) * 2] = m_run;
        sm_ml[((kw - 1) * 16 + lr) * 2 + 1] = lt;
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) sm_o[((kw - 1) * DT + dt) * 64 + l] = acc[dt];
    }
    __syncthreads();
    if (kw == 0) {
#pragma unroll
      for (int w = 1; w < KW; ++w) {
        f32x4 ow[DT];
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) ow[dt] = sm_o[((w - 1) * DT + dt) * 64 + l];
        fold_state(m_run, lt, acc, sm_ml[((w - 1) * 16 + lr) * 2],
                   sm_ml[((w - 1) * 16 + lr) * 2 + 1], ow);
      }
    }
    __syncthreads();  // the next unit rewrites these
  }
  if (kw != 0 || !x.active || x.r >= x.R) return;
  if (x.pslot < 0) {
    const int t_out = div_g(x.r, a);
    const int orow = x.b * a.Tq + t_out, ocol = (x.kvh * a.G + x.r - t_out * a.G) * D + 4 * lg;
    const float inv = 1.0f / lt;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const f32x4 y = acc[dt] * inv;
      elem_t* op = static_cast<elem_t*>(a.out) +
                   mat_off(orow, ocol + 16 * dt, a.Hq * D, a.Hq * D, a.out_blocked);
      if constexpr (BF16) {
        *reinterpret_cast<u32x2*>(op) = u32x2{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
      } else {
        *reinterpret_cast<f32x4*>(op) = y;
      }
    }
    return;
  }
  const size_t slot = static_cast<size_t>(x.pslot) * a.Hkv + x.kvh;
  float* po = a.part_o + (slot * ROWS + nt * 16 + lr) * D + 4 * lg;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4*>(po + dt * 16) = acc[dt];
  if (lg == 0) {
    float* pml = a.part_ml + (slot * ROWS + nt * 16 + lr) * 2;
    pml[0] = m_run;
    pml[1] = lt;
  }
}

// The attention kernels are persistent: workgroups take units blockIdx.x,
// blockIdx.x + gridDim.x, ... (times the kv heads) from the plan. Within a
// unit, one wave = one 16-row tile times KW key waves: the workgroup's waves
// share the (sequence, kv head, unit), and key wave kw takes the unit's
// bursts of NPRE tiles at offsets kw*NPRE, kw*NPRE + KW*NPRE, ... Dynamic LDS:
// the K/V chunk buffers (bf16 with several row tiles), which the key-wave
// fold reuses.

// fp32: each key wave loads its bursts into registers (two bursts in flight).
template <int D, int NT, bool BS16, int KW>
__global__ __launch_bounds__(64 * NT * KW) void verify_attn_f32_kernel(AttnArgs a) {
  constexpr int NPRE = burst_tiles<D, false>();
  constexpr int DT = D / 16;
  constexpr int DQ = D / 4;
  constexpr int KS = F32Frag<D>::KS;
  extern __shared__ int sm_dyn[];

  const int tid = threadIdx.x;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nt = wid / KW, kw = wid - nt * KW;
  const int l = tid & 63, lr = l & 15, lg = l >> 4;
  const int32_t* recs = a.plan + kPlanHead;
  const float* qb = static_cast<const float*>(a.q);
  const float c = a.scale_log2;

  // the unit count and the first record are loaded together (the record is
  // inside the plan whatever the count turns out to be)
  int nunits = a.plan[0];
  int rec = recs[static_cast<size_t>(blockIdx.x / a.Hkv) * kRecInts + l];
  nunits = __builtin_amdgcn_readfirstlane(min(nunits, a.max_units)) * a.Hkv;
  for (int u = blockIdx.x; u < nunits; u += gridDim.x) {
    if (u != static_cast<int>(blockIdx.x)) rec = recs[static_cast<size_t>(u / a.Hkv) * kRecInts + l];
    const UnitInfo x = unit_info<NT>(a, rec, u, nt, lr);
    if (KW == 1 && !x.active) continue;  // (key waves still meet at the fold)
    const int kt0 = x.kt0, kt1 = x.kt1, kvh = x.kvh, start = x.start, Lk = x.Lk, qlim = x.qlim;
    const int32_t* table = a.tables + static_cast<size_t>(x.srow) * a.max_blocks;

    float qf[KS];
    {
      const bool ok = x.r < x.R;
      const int t = ok ? div_g(x.r, a) : 0;
      const int h = kvh * a.G + (ok ? x.r - t * a.G : 0);
      const float* qp = qb + ((static_cast<size_t>(x.b) * a.Tq + t) * a.Hq + h) * D + lg * DQ;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qf[ks] = ok ? qp[ks] : 0.0f;
    }

    float m_run = kNegBig, l_run = 0.0f;
    f32x4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0, 0, 0, 0};
    const int first = kt0 + kw * NPRE;  // this wave's first burst

    // Block ids come from the unit's record (lane 8 + j: tile kt0 + j), picked
    // out with readlane; every tile slot of a burst is loaded (slots past the
    // unit read an in-range entry and are dropped by the math), so the wait
    // for burst b never waits for b+1.
    const int tv = rec;
    const int c0 = kt0 - kRecHead;
    auto issue = [&](F32Frag<D> (&f)[NPRE], int r0) {
#pragma unroll
      for (int j = 0; j < NPRE; ++j) {
        if constexpr (BS16) {
          const int lane = min(r0 - c0 + j, 63);
          load_tile16<D>(f[j], a, safe_block(__builtin_amdgcn_readlane(tv, lane), a.num_blocks),
                         kvh, lr, lg);
        } else {
          if (r0 + j < kt1) load_tile_any<D>(f[j], a, table, kvh, r0 + j, Lk, lr, lg);
          else zero_v(f[j]);
        }
      }
    };
    auto consume = [&](F32Frag<D> (&fr)[NPRE], int r0) {
      f32x4 sc[NPRE];
#pragma unroll
      for (int j = 0; j < NPRE; ++j) {
        f32x4 s = {0, 0, 0, 0};
        if (r0 + j < kt1) {
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) s = mfma16x16x4_f32(fr[j].k[ks], qf[ks], s);
        }
        sc[j] = s;
      }
      if constexpr (BS16) {
#pragma unroll
        for (int j = 0; j < NPRE; ++j) {
          if (r0 + j < kt1) mask_v_tail(fr[j], r0 + j, Lk, lg);
          else zero_v(fr[j]);
        }
      }
      // one online-softmax step over the burst (see verify_attn_bf16_kernel)
      float smax = -INFINITY;
#pragma unroll
      for (int j = 0; j < NPRE; ++j) {
        const int kt = r0 + j;
        if (kt >= kt1) break;
        if (kt * 16 + 15 > start) {
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
        if (r0 + j >= kt1) break;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = __builtin_amdgcn_exp2f(fmaf(sc[j][i], c, -m_use));
          l_run += p;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) acc[dt] = mfma16x16x4_f32(fr[j].v[dt][i], p, acc[dt]);
        }
      }
    };

    constexpr int BSTEP = KW * NPRE;  // tiles between this wave's bursts
    F32Frag<D> fa[NPRE], fb[NPRE];
    if (x.active && first < kt1) {
      issue(fa, first);
      for (int r0 = first; r0 < kt1; r0 += 2 * BSTEP) {
        if (r0 + BSTEP < kt1) issue(fb, r0 + BSTEP);
        consume(fa, r0);
        if (r0 + BSTEP >= kt1) break;
        if (r0 + 2 * BSTEP < kt1) issue(fa, r0 + 2 * BSTEP);
        consume(fb, r0 + BSTEP);
      }
    }
    finish_unit<D, false, NT, KW>(a, x, sm_dyn, nt, kw, l, m_run, sum_across_groups(l_run), acc);
  }
}

// bf16: bursts of NPRE tiles (NPRE / 2 pairs). With one row tile (or any
// block size) each key wave loads its bursts into registers, two bursts in
// flight; with several row tiles and 16-token blocks the unit's tiles stream
// through NBUF chunk buffers in LDS (one chunk = one round of bursts, KW*NPRE
// tiles) and every row tile's waves read their fragments there, so each K/V
// tile crosses L2 -> CU once per workgroup while the next chunks load.
// LDS-path workgroups (several row tiles) of up to 6 waves are held to 128
// registers: their waves land unevenly on the SIMDs (2, 2, 1, 1 for six), so
// two such workgroups share a CU only at four waves per SIMD (measured: at
// 151 registers the second one waited for the first to finish). The register
// path keeps two bursts in registers and takes what it needs.
template <int D, int NT, bool BS16, int KW>
__global__ __launch_bounds__(64 * NT * KW)
__attribute__((amdgpu_waves_per_eu(NT >= 2 && NT * KW <= 6 ? 4 : 1))) void verify_attn_bf16_kernel(AttnArgs a) {
  constexpr int NPRE = burst_tiles<D, true>();
  constexpr int NP = NPRE / 2;  // pairs per burst
  constexpr int DT = D / 16;
  constexpr int DQ = D / 4;
  constexpr int KS = D / 32;
  constexpr bool DMAKV = BS16 && NT >= 2;
  constexpr int KI = D / 32;                    // 1 KB pieces per K (or V) tile
  constexpr int TI = 2 * KI;                    // per tile
  constexpr int TB = kDmaTileBytes<D>();
  constexpr int NW = NT * KW;                   // waves
  constexpr int CT = KW * NPRE;                 // tiles per chunk
  constexpr int CPIECES = CT * TI;              // 1 KB pieces per chunk
  constexpr int LPW = (CPIECES + NW - 1) / NW;  // direct loads per wave per chunk
  constexpr int NBUF = dma_nbuf<D>(NT, KW);
  static_assert(!DMAKV || (NBUF - 2) * LPW <= 63, "vmcnt range");
  extern __shared__ int sm_dyn[];

  const int tid = threadIdx.x;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nt = wid / KW, kw = wid - nt * KW;
  const int l = tid & 63, lr = l & 15, lg = l >> 4;
  const int32_t* recs = a.plan + kPlanHead;
  const uint16_t* qb = static_cast<const uint16_t*>(a.q);
  const float c = a.scale_log2;
  const u32x4 ones = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};  // bf16 1.0 x 8

  int nunits = a.plan[0];
  int rec = recs[static_cast<size_t>(blockIdx.x / a.Hkv) * kRecInts + l];
  nunits = __builtin_amdgcn_readfirstlane(min(nunits, a.max_units)) * a.Hkv;
  for (int u = blockIdx.x; u < nunits; u += gridDim.x) {
    if (u != static_cast<int>(blockIdx.x)) rec = recs[static_cast<size_t>(u / a.Hkv) * kRecInts + l];
    const UnitInfo x = unit_info<NT>(a, rec, u, nt, lr);
    // A row tile wholly past q_len has nothing to compute; with K/V staged in
    // LDS the wave still takes its share of the loads and barriers.
    if (!DMAKV && KW == 1 && !x.active) continue;  // (key waves still meet at the fold)
    const int kt0 = x.kt0, kt1 = x.kt1, kvh = x.kvh;
    // keys a pair must mask: past this lane's row (causal) or past the unit
    const int klim = min(x.qlim, kt1 * 16 - 1);
    // a pair whose last key passes `edge` needs the mask (wave-uniform test;
    // every real row sees keys up to start)
    const int edge = min(x.start, kt1 * 16 - 1);
    // V keys from vlim on are zeroed: stale slots past the history, tiles past the unit
    const int vlim = min(x.Lk, kt1 * 16);
    const int32_t* table = a.tables + static_cast<size_t>(x.srow) * a.max_blocks;

    u32x4 qf[KS];
    {
      const bool ok = x.r < x.R;
      const int t = ok ? div_g(x.r, a) : 0;
      const int h = kvh * a.G + (ok ? x.r - t * a.G : 0);
      const uint16_t* qp = qb + ((static_cast<size_t>(x.b) * a.Tq + t) * a.Hq + h) * D + lg * DQ;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        qf[ks] = ok ? reinterpret_cast<const u32x4*>(qp)[ks] : u32x4{0, 0, 0, 0};
    }

    float m_run = kNegBig;
    f32x4 acc[DT], lsum = {0, 0, 0, 0};  // every lane of a row holds its row's sum
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0, 0, 0, 0};
    const int first = kt0 + kw * NPRE;  // this wave's first burst

    // One online-softmax step over a burst starting at tile r0 (< kt1).
    // Scores stay unscaled until the exponent: p = 2^(s*c - m) with m kept in
    // the scaled log2 domain, one FMA per score. Only pairs that reach the
    // causal edge or the unit's end pay for masking (a wave-uniform test);
    // pairs past the unit are masked whole. The reference max m moves only
    // when a row's max grows by more than 8 (p then stays below 256), so the
    // rescale of the accumulators is rare; the first burst has nothing to
    // rescale. P is split into bf16 hi + lo halves (16 significant bits of P
    // reach the product), which feed both O^T += V^T P^T and the row sums
    // l += 1^T P^T.
    // vget(p, dt): the V fragment dt of pair p (registers, or read from LDS
    // just before its product, which keeps the LDS path's register count down)
    auto consume = [&](PairFrag<D> (&fr)[NP], int r0, auto&& vget) {
      f32x4 sc[NP][2];
#pragma unroll
      for (int p = 0; p < NP; ++p) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          f32x4 s = {0, 0, 0, 0};
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) s = mfma16x16x32_bf16(fr[p].k[h][ks], qf[ks], s);
          sc[p][h] = s;
        }
      }
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int kt = r0 + 2 * p;
        if (kt * 16 + 31 > edge) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (kt * 16 + 8 * lg + 4 * h + i > klim) sc[p][h][i] = -INFINITY;
          }
        }
      }
      float smax = -INFINITY;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          smax = fmaxf(fmaxf(smax, sc[p][h][0]), sc[p][h][1]);
          smax = fmaxf(fmaxf(smax, sc[p][h][2]), sc[p][h][3]);
        }
      }
      smax = max_across_groups(smax);
      const float m_new = fmaxf(m_run, smax * c);
      float m_use = m_new;
      if (r0 != first) {
        const bool grow = m_new > m_run + 8.0f;
        m_use = grow ? m_new : m_run;
        if (__any(grow)) {
          const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
          lsum *= alpha;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
        }
      }
      m_run = m_use;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        f32x4 e[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int i = 0; i < 4; ++i) e[h][i] = __builtin_amdgcn_exp2f(fmaf(sc[p][h][i], c, -m_use));
        }
        // P = hi + lo: hi is p truncated to its top 16 bits (a bf16, exactly),
        // lo = p - hi (exact in fp32) rounded to bf16
        u32x4 ph, pl;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float pa = e[q >> 1][2 * (q & 1)], pb = e[q >> 1][2 * (q & 1) + 1];
          const uint32_t ua = __float_as_uint(pa), ub = __float_as_uint(pb);
          ph[q] = __builtin_amdgcn_perm(ub, ua, 0x07060302u);
          pl[q] = pack_bf16x2(pa - __uint_as_float(ua & 0xffff0000u),
                              pb - __uint_as_float(ub & 0xffff0000u));
        }
        // V keys at or past vlim are zeroed (stale slots past the history,
        // tiles past the unit), so a p = 0 slot never meets an inf or NaN
        const int k0 = (r0 + 2 * p) * 16 + 8 * lg;
        const bool vz = k0 - 8 * lg + 31 >= vlim;  // wave-uniform
        u32x4 keep = {~0u, ~0u, ~0u, ~0u};
        if (vz) {
#pragma unroll
          for (int w = 0; w < 4; ++w)
            keep[w] = (k0 + 2 * w < vlim ? 0x0000ffffu : 0u) | (k0 + 2 * w + 1 < vlim ? 0xffff0000u : 0u);
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          u32x4 v = vget(p, dt);
          if (vz) v &= keep;
          acc[dt] = mfma16x16x32_bf16(v, ph, acc[dt]);
          acc[dt] = mfma16x16x32_bf16(v, pl, acc[dt]);
        }
        lsum = mfma16x16x32_bf16(ones, ph, lsum);
        lsum = mfma16x16x32_bf16(ones, pl, lsum);
      }
    };

    const int tv = rec;  // block ids: lane kRecHead + j holds tile kt0 + j
    if constexpr (!DMAKV) {
      // Register path: bursts double-buffered, the K/V loads of burst b+1 in
      // flight while burst b is multiplied. Every pair of a burst is loaded
      // (pairs past the unit read an in-range block and are masked), so the
      // number of loads per burst is fixed.
      constexpr int BSTEP = KW * NPRE;
      PairFrag<D> fa[NP], fb[NP];
      if constexpr (BS16) {
        // 16-token blocks: V straight into registers (a V fragment is one
        // 16-byte load per lane, two 512-byte runs per instruction), K staged
        // per wave in LDS: each K tile of a burst is copied by 1 KB direct
        // loads (whole 128- or 256-byte rows per instruction, a K row's
        // 16-byte chunks XOR-swizzled as in the LDS path) into one of the
        // wave's two burst buffers, and its fragments are read back just
        // before the burst's product. Loading K fragments straight from global
        // memory (16 rows x 64 bytes per instruction) streams far slower per
        // CU. The values multiplied are the same either way. A burst waits
        // for its own loads only (vmcnt: the next burst's loads may stay in
        // flight); the buffers belong to one wave, so no barrier is needed
        // until the fold reuses the LDS.
        constexpr int KTB = 32 * D;          // bytes of a K tile: 16 rows x D x 2
        constexpr int KPT = KTB / 1024;      // 1 KB direct loads per K tile
        constexpr int BURST_OPS = NPRE * KPT + NP * DT;  // vector-memory ops of one burst
        static_assert(BURST_OPS <= 63, "vmcnt range");
        char* kst = reinterpret_cast<char*>(sm_dyn + a.lds_kv_off) + wid * (2 * NPRE * KTB);
        const char* kg = static_cast<const char*>(a.k);
        const uint16_t* vb = static_cast<const uint16_t*>(a.v);
        auto issue = [&](PairFrag<D> (&f)[NP], int r0, int buf) {
          char* kb_ = kst + buf * (NPRE * KTB);
          int blk[NPRE];
#pragma unroll
          for (int t = 0; t < NPRE; ++t)
            blk[t] = safe_block(__builtin_amdgcn_readlane(tv, min(kRecHead + r0 + t - kt0, 63)),
                                a.num_blocks);
#pragma unroll
          for (int t = 0; t < NPRE; ++t) {
            const size_t tb = (static_cast<size_t>(blk[t]) * a.Hkv + kvh) * 16 * D;
#pragma unroll
            for (int q = 0; q < KPT; ++q) {
              const int j = q * 64 + l, row = j / (D / 8), pc = j - row * (D / 8);
              const char* src =
                  kg + (tb + static_cast<size_t>(row) * D) * 2 + ((pc ^ ksw<D>(row, t)) << 4);
              __builtin_amdgcn_global_load_lds(
                  (__attribute__((address_space(1))) void*)(src),
                  (__attribute__((address_space(3))) void*)(kb_ + t * KTB + q * 1024), 16, 0, 0);
            }
          }
#pragma unroll
          for (int p = 0; p < NP; ++p) {
            const size_t t0 = (static_cast<size_t>(blk[2 * p]) * a.Hkv + kvh) * 16 * D;
            const size_t t1 = (static_cast<size_t>(blk[2 * p + 1]) * a.Hkv + kvh) * 16 * D;
            const uint16_t* vp = vb + (lg < 2 ? t0 : t1) + lr * 16 + 8 * (lg & 1);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) f[p].v[dt] = *reinterpret_cast<const u32x4*>(vp + dt * 256);
          }
        };
        // K fragments of burst buffer buf (the rows of pair p's two tiles)
        auto kread = [&](PairFrag<D> (&f)[NP], int buf) {
          const char* kb_ = kst + buf * (NPRE * KTB);
#pragma unroll
          for (int p = 0; p < NP; ++p) {
            const char* tk = kb_ + (2 * p + (lr >> 3)) * KTB;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int row = pair_key_of_row(lr, h) & 15;
#pragma unroll
              for (int ks = 0; ks < KS; ++ks) {
                const int cch = lg * (DQ / 8) + ks;
                f[p].k[h][ks] = *reinterpret_cast<const u32x4*>(
                    tk + row * 2 * D + ((cch ^ ksw<D>(row, lr >> 3)) << 4));
              }
            }
          }
        };
        if (x.active && first < kt1) {
          issue(fa, first, 0);
          // the Q fragment (loaded before the first burst) has landed: without
          // this wait the compiler loses track of it across the loop and waits
          // for every outstanding load (the next burst's too) before each
          // burst's first MFMA
          wave_wait_vm<BURST_OPS>();
          // The loop runs while both following bursts exist, so its issues
          // and waits are unconditional; the last one or two bursts are
          // consumed after it. (With the last-burst test inside the loop the
          // compiler split each if/else into two flagged branches, and on
          // the path it could not rule out, with neither wait taken, it
          // waited for every load, the next burst's too, before each product
          // with V.)
          int r0 = first;
          for (; r0 + 2 * BSTEP < kt1; r0 += 2 * BSTEP) {
            issue(fb, r0 + BSTEP, 1);
            wave_wait_vm<BURST_OPS>();
            kread(fa, 0);
            consume(fa, r0, [&](int p, int dt) { return fa[p].v[dt]; });
            issue(fa, r0 + 2 * BSTEP, 0);
            wave_wait_vm<BURST_OPS>();
            kread(fb, 1);
            consume(fb, r0 + BSTEP, [&](int p, int dt) { return fb[p].v[dt]; });
          }
          if (r0 + BSTEP < kt1) {
            issue(fb, r0 + BSTEP, 1);
            wave_wait_vm<BURST_OPS>();
            kread(fa, 0);
            consume(fa, r0, [&](int p, int dt) { return fa[p].v[dt]; });
            wave_wait_vm<0>();
            kread(fb, 1);
            consume(fb, r0 + BSTEP, [&](int p, int dt) { return fb[p].v[dt]; });
          } else {
            wave_wait_vm<0>();
            kread(fa, 0);
            consume(fa, r0, [&](int p, int dt) { return fa[p].v[dt]; });
          }
        }
        if constexpr (KW > 1) barrier_after_vm<0>();  // the fold reuses the waves' K buffers
      } else {
        auto issue = [&](PairFrag<D> (&f)[NP], int r0) {
#pragma unroll
          for (int p = 0; p < NP; ++p) load_pair_any<D>(f[p], a, table, kvh, r0 + 2 * p, vlim, lr, lg);
        };
        if (x.active && first < kt1) {
          issue(fa, first);
          for (int r0 = first; r0 < kt1; r0 += 2 * BSTEP) {
            if (r0 + BSTEP < kt1) issue(fb, r0 + BSTEP);
            consume(fa, r0, [&](int p, int dt) { return fa[p].v[dt]; });
            if (r0 + BSTEP >= kt1) break;
            if (r0 + 2 * BSTEP < kt1) issue(fa, r0 + 2 * BSTEP);
            consume(fb, r0 + BSTEP, [&](int p, int dt) { return fb[p].v[dt]; });
          }
        }
      }
    } else {
      // LDS path: chunks of CT tiles through NBUF buffers. Every 1 KB (K or V)
      // piece of a chunk is one global_load_lds (16 bytes per lane, straight
      // into LDS, no registers), LPW per wave, so each wave issues the same
      // number of loads per chunk (a wave short of pieces re-loads the chunk's
      // last piece onto itself) and chunk ch waits with one vmcnt for its own
      // loads only, then one barrier makes every wave's pieces visible and
      // frees the buffer of chunk ch - 1 for chunk ch + NBUF - 1. Tiles past
      // kt1 read an in-range block (the record repeats its last id) and are
      // masked. A K row's 16-byte chunks are stored XOR-swizzled by the row
      // and the tile's parity (ksw) and a V channel's two chunks by vsw, so a
      // fragment read's 16 lanes cover the 16 bank groups of a 256-byte line.
      char* kvl = reinterpret_cast<char*>(sm_dyn + a.lds_kv_off);
      const char* kg = static_cast<const char*>(a.k);
      const char* vg = static_cast<const char*>(a.v);
      const int nch = cdiv(kt1 - kt0, CT);
      auto issue_chunk = [&](int ch) {
        char* buf = kvl + (ch % NBUF) * (CT * TB);
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
          const int g = min(wid + i * NW, CPIECES - 1);
          const int t = g / TI, part = g - t * TI;
          const int lane = min(kRecHead + ch * CT + t, 63);
          const int blk = safe_block(__builtin_amdgcn_readlane(tv, lane), a.num_blocks);
          const size_t tb = (static_cast<size_t>(blk) * a.Hkv + kvh) * 16 * D;
          const char* src;
          if (part < KI) {
            const int j = part * 64 + l, row = j / (D / 8), pc = j - row * (D / 8);
            src = kg + (tb + static_cast<size_t>(row) * D) * 2 + ((pc ^ ksw<D>(row, t)) << 4);
          } else {
            const int j = (part - KI) * 64 + l, chn = j >> 1;
            src = vg + (tb + static_cast<size_t>(chn) * 16) * 2 + (((j & 1) ^ vsw(chn)) << 4);
          }
          __builtin_amdgcn_global_load_lds(
              (__attribute__((address_space(1))) void*)(src),
              (__attribute__((address_space(3))) void*)(buf + t * TB + part * 1024), 16, 0, 0);
        }
      };
      // K fragments of the burst whose first tile sits at tb0 (an even tile of the chunk)
      auto dread = [&](PairFrag<D> (&f)[NP], const char* tb0) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const char* tk = tb0 + (2 * p + (lr >> 3)) * TB;  // the tile of this lane's K row
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int row = pair_key_of_row(lr, h) & 15;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
              const int cch = lg * (DQ / 8) + ks;
              f[p].k[h][ks] = *reinterpret_cast<const u32x4*>(
                  tk + row * 2 * D + ((cch ^ ksw<D>(row, lr >> 3)) << 4));
            }
          }
        }
      };
      // V fragment dt of pair p of the burst at tb0: channel dt*16 + lr, the
      // lane's 8 keys of the tile (lg / 2)
      auto vread = [&](const char* tb0, int p, int dt) {
        const char* tvv = tb0 + (2 * p + (lg >> 1)) * TB + 32 * D;
        const int chn = dt * 16 + lr;
        return *reinterpret_cast<const u32x4*>(tvv + chn * 32 + (((lg & 1) ^ vsw(chn)) << 4));
      };
#pragma unroll
      for (int ch = 0; ch < NBUF - 1; ++ch)
        if (ch < nch) issue_chunk(ch);
      for (int ch = 0; ch < nch; ++ch) {
        // chunk ch has landed (this wave's loads, then everyone's), and every
        // wave is done with chunk ch - 1, whose buffer takes chunk ch + NBUF - 1
        barrier_after_chunks<LPW, NBUF - 2>(min(NBUF - 2, nch - 1 - ch));
        if (ch + NBUF - 1 < nch) issue_chunk(ch + NBUF - 1);
        const int r0 = kt0 + ch * CT + kw * NPRE;
        if (x.active && r0 < kt1) {
          PairFrag<D> fr[NP];
          const char* tb0 = kvl + ((ch % NBUF) * CT + kw * NPRE) * TB;
          dread(fr, tb0);
          consume(fr, r0, [&](int p, int dt) { return vread(tb0, p, dt); });
        }
      }
      barrier_after_vm<0>();  // the buffers are rewritten by the fold or the next unit
    }
    finish_unit<D, true, NT, KW>(a, x, sm_dyn, nt, kw, l, m_run, lsum[0], acc);
  }
}

// Merge the units of one split item (and kv head): the units' states folded
// in unit order with fold_state -- as the waves of a unit are -- then
// normalised. Grid (split-item bound, Hkv * D/16); thread (row, 4 channels).
// The first two units' states are read before the item's record arrives (its
// slots follow from its index), the next SPL together once it has, so an item
// of up to SPL + 2 units costs two round trips; an index past the plan's split
// items exits.
template <int D, bool BF16, int NT>
__global__ __launch_bounds__(64 * NT) void verify_attn_merge_kernel(AttnArgs a) {
  using elem_t = std::conditional_t<BF16, uint16_t, float>;
  constexpr int ROWS = 16 * NT;
  constexpr int SPL = 16;
  const int tid = threadIdx.x;
  const int j = blockIdx.x;
  const int kvh = blockIdx.y / (D / 16);
  const int d = (blockIdx.y - kvh * (D / 16)) * 16 + (tid & 3) * 4;
  const int rr = tid >> 2;  // < ROWS: the block has 4 * ROWS threads
  const size_t slot0 = static_cast<size_t>(j) * a.max_item_units;
  auto po = [&](int u) {
    return a.part_o + (((slot0 + u) * a.Hkv + kvh) * ROWS + rr) * D + d;
  };
  auto pml = [&](int u) { return a.part_ml + (((slot0 + u) * a.Hkv + kvh) * ROWS + rr) * 2; };
  const int32_t* sp = a.plan + kPlanHead + static_cast<size_t>(a.max_units) * kRecInts +
                      static_cast<size_t>(j) * kSplitInts;
  const int nsplit_items = a.plan[1];
  const int b = sp[0], rg = sp[1], nu = sp[2], T = sp[3];
  // units 0 and 1 exist for every split item (and lie in its slots if not)
  f32x4 x[1] = {*reinterpret_cast<const f32x4*>(po(0))};
  const f32x4 o1[1] = {*reinterpret_cast<const f32x4*>(po(1))};
  float M = pml(0)[0], L = pml(0)[1];
  const float m1 = pml(1)[0], l1 = pml(1)[1];
  if (j >= nsplit_items) return;
  const int R = a.G * T;
  const int row0 = rg * ROWS;
  if (row0 + rr >= R) return;
  fold_state(M, L, x, m1, l1, o1);
  // Units 2.. in batches of SPL: every load of a batch is issued (indices past
  // the item's last unit re-read it) and every fold computed, a fold past the
  // last unit discarded by a select. With a branch per unit the compiler sank
  // each unit's loads into it and waited for them one unit at a time.
  for (int u0 = 2; u0 < nu; u0 += SPL) {
    f32x4 o[SPL];
    float m[SPL], lv[SPL];
#pragma unroll
    for (int q = 0; q < SPL; ++q) {
      const int u = min(u0 + q, nu - 1);
      o[q] = *reinterpret_cast<const f32x4*>(po(u));
      m[q] = pml(u)[0];
      lv[q] = pml(u)[1];
    }
#pragma unroll
    for (int q = 0; q < SPL; ++q) {
      const bool live = u0 + q < nu;
      float M2 = M, L2 = L;
      f32x4 x2[1] = {x[0]};
      const f32x4 oq[1] = {o[q]};
      fold_state(M2, L2, x2, m[q], lv[q], oq);
      M = live ? M2 : M;
      L = live ? L2 : L;
      x[0] = live ? x2[0] : x[0];
    }
  }
  const float inv = 1.0f / L;
  const f32x4 y = x[0] * inv;
  const int r = row0 + rr;
  const int t = div_g(r, a), h = kvh * a.G + r - t * a.G;
  elem_t* op = static_cast<elem_t*>(a.out) +
               mat_off(b * a.Tq + t, h * D + d, a.Hq * D, a.Hq * D, a.out_blocked);
  if constexpr (BF16) {
    *reinterpret_cast<u32x2*>(op) = u32x2{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
  } else {
    *reinterpret_cast<f32x4*>(op) = y;
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

struct AttnCfg {
  int NT, KW, rows, row_groups, unit_tiles, max_units, max_split, max_item_units, lds_kv_off;
  size_t plan_bytes, part_ml_bytes, part_o_bytes, lds, plan_lds;
};

// Work list limits per launch (the plan kernel scans them in LDS).
constexpr int kMaxLaunchSeqs = 2048;
constexpr int kMaxLaunchItems = 8192;

// Automatic unit size (tiles) for histories longer than one record holds:
// four bursts per wave at D = 64 in bf16. Finer units shorten the attention
// but add unit states to merge.
// With at least kWideUnitsAt units of that size per launch (counted at
// max_ctx: sequences x units x kv heads) the chip is full either way and
// units twice as long halve the states to merge: 32 x 4096 tokens
// 31.7 -> 25.8 us, 16 x 8192 (D = 128) 72.4 -> 56.0 us; the verify
// microbench's mix of mostly short histories keeps 16 (13.6 vs 16.6 us).
constexpr long long kWideUnitsAt = 1024;
static int default_unit_tiles(int num_seqs, int tiles, int Hkv, int dtype) {
  if (dtype != KVE_DTYPE_BF16) return 8;
  const long long units = static_cast<long long>(num_seqs) * cdiv(tiles, 16) * Hkv;
  return units >= kWideUnitsAt ? 32 : 16;
}
// Key waves of a one-row-tile unit (512 threads): 0.5B draft forward at 32
// rows 1080 -> 1062 us against 4, batched 32-request workload +0.9 %.
constexpr int kKW1 = 8;

static inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// Unit size and key waves either fixed by the caller (unit_blocks, key_waves
// > 0: every launch with the same values sums a row's keys in the same order)
// or chosen from the launch's shape.
static AttnCfg attn_cfg(int num_seqs, int q_len, int Hq, int Hkv, int D, int max_ctx,
                        int unit_blocks, int key_waves, int block_size, int dtype) {
  AttnCfg p{};
  const int rows = (Hq / Hkv) * q_len;
  const int tiles = cdiv(max_ctx, 16);
  int U;
  if (unit_blocks > 0)
    U = block_size == 16 ? unit_blocks : cdiv(unit_blocks * block_size, 16);
  else
    U = tiles <= kMaxUnitTiles ? kMaxUnitTiles : default_unit_tiles(num_seqs, tiles, Hkv, dtype);
  U = std::min(std::max(U, 1), kMaxUnitTiles);
  const bool bf16_dma = dtype == KVE_DTYPE_BF16 && block_size == 16;
  // Short histories (one unit) spread the rows of a kv head over workgroups of
  // one row tile with kKW1 key waves (more parallelism per sequence; 3B verify
  // pass at 32 x 5 tokens: 4.54 -> 4.18 ms); longer ones share each K/V tile
  // between up to 8 row tiles of a workgroup (LDS chunks).
  // Waves per workgroup stay within what the kernels hold without spilling: up
  // to 12 with LDS chunks, 8 on the register path.
  auto nt_cap = [&](int kw) {
    if (bf16_dma) return kw >= 8 ? 1 : kw >= 4 ? 3 : kw == 2 ? 6 : 8;
    return kw >= 8 ? 1 : kw >= 4 ? 2 : kw == 2 ? 4 : 8;
  };
  int NT, KW;
  if (key_waves > 0) {
    KW = key_waves;
    NT = std::min(attn_row_tiles(cdiv(rows, 16)), nt_cap(KW));
  } else if (tiles <= U && unit_blocks <= 0) {
    NT = 1;
    KW = kKW1;
  } else {
    NT = attn_row_tiles(cdiv(rows, 16));
    // one row tile (decode rows of a long history): as many key waves as one
    // round of bursts covers the unit with, up to kKW1
    const int burst = dtype == KVE_DTYPE_BF16 ? (D == 64 ? 4 : 2) : (D == 64 ? 2 : 1);
    KW = NT == 1 ? std::min(kKW1, std::max(1, U / burst)) : NT <= 4 && U >= 16 ? 2 : 1;
    NT = std::min(NT, nt_cap(KW));
  }
  p.NT = NT;
  p.KW = KW;
  p.rows = 16 * NT;
  p.row_groups = cdiv(rows, p.rows);
  p.unit_tiles = U;
  p.max_item_units = cdiv(tiles, U);
  const long long items = static_cast<long long>(num_seqs) * p.row_groups;
  p.max_units = static_cast<int>(std::min<long long>(items * p.max_item_units, 1 << 30));
  p.max_split = p.max_item_units > 1 ? static_cast<int>(items) : 0;
  p.plan_bytes = align256((kPlanHead + static_cast<size_t>(p.max_units) * kRecInts +
                           static_cast<size_t>(p.max_split) * kSplitInts) * sizeof(int32_t));
  const size_t slots = static_cast<size_t>(p.max_split) * p.max_item_units * Hkv;
  p.part_ml_bytes = align256(slots * p.rows * 2 * sizeof(float));
  p.part_o_bytes = align256(slots * p.rows * D * sizeof(float));
  // dynamic LDS: the direct-load K/V chunk buffers (bf16, 16-token blocks,
  // several row tiles) and the key waves' states for the in-workgroup fold,
  // which reuses the buffers once the unit's last chunk is consumed
  size_t region = 0;
  const int npre = D == 64 ? burst_tiles<64, true>() : burst_tiles<128, true>();
  if (bf16_dma && NT >= 2) {
    const int nbuf = D == 64 ? dma_nbuf<64>(NT, KW) : dma_nbuf<128>(NT, KW);
    region = static_cast<size_t>(nbuf) * KW * npre * kDmaTileBytes<64>() * (D / 64);
  } else if (bf16_dma) {
    // one row tile: each key wave's two K burst buffers (16 x D bf16 per tile)
    region = static_cast<size_t>(KW) * 2 * npre * 32 * D;
  }
  if (KW > 1)
    region = std::max(region, static_cast<size_t>(NT) * (KW - 1) *
                                  (16 * 2 * sizeof(float) + (D / 16) * 64 * 16));
  p.lds_kv_off = 0;
  p.lds = region;
  p.plan_lds = (static_cast<size_t>(items) * 3 + 1) * sizeof(int) +
               static_cast<size_t>(num_seqs) * sizeof(SeqInfo);
  return p;
}

static size_t attn_ws_bytes(const AttnCfg& p, bool with_plan) {
  return (with_plan ? p.plan_bytes : 0) + p.part_ml_bytes + p.part_o_bytes;
}

// Workgroups of the persistent attention kernel: what the chip holds at once
// (occupancy of this instantiation at this LDS size, asked once per device
// and LDS size), or fewer when the launch cannot have that many units.
template <typename K>
static int resident_workgroups(K kernel, int threads, size_t lds) {
  struct Entry {
    const void* fn;
    size_t lds;
    int dev, n;
  };
  static Entry cache[64];
  static int used = 0;
  static std::mutex mu;
  std::lock_guard<std::mutex> lock(mu);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  for (int i = 0; i < used; ++i)
    if (cache[i].fn == reinterpret_cast<const void*>(kernel) && cache[i].lds == lds &&
        cache[i].dev == dev)
      return cache[i].n;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds) != hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  const int n = per_cu * cus;
  if (used < 64) cache[used++] = Entry{reinterpret_cast<const void*>(kernel), lds, dev, n};
  return n;
}

template <typename K>
static int grant_lds(K kernel, size_t bytes, const char* what) {
  if (bytes <= 64 * 1024) return KVE_OK;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(bytes)) != hipSuccess) {
    set_error("%s: %zu bytes of LDS refused", what, bytes);
    return KVE_ELAUNCH;
  }
  return KVE_OK;
}

static int launch_plan(const AttnArgs& a, const AttnCfg& p, hipStream_t st) {
  const int rc = grant_lds(attn_plan_kernel, p.plan_lds, "kve_attn_plan");
  if (rc) return rc;
  const int grid = std::max(1, std::min(64, cdiv(p.max_units, kPlanThreads / 64)));
  hipLaunchKernelGGL(attn_plan_kernel, dim3(grid), dim3(kPlanThreads), p.plan_lds, st, a);
  return KVE_OK;
}

template <int D, bool BF16, int NT, int KW>
static int launch_attn_t(const AttnArgs& a, const AttnCfg& p, hipStream_t st, bool bs16) {
  auto go = [&](auto kernel) {
    const int rc = grant_lds(kernel, p.lds, "kve_paged_verify_attn");
    if (rc) return rc;
    const int nwg = resident_workgroups(kernel, 64 * NT * KW, p.lds);
    const long long max_units = static_cast<long long>(p.max_units) * a.Hkv;
    const int grid = static_cast<int>(std::max(1LL, std::min<long long>(nwg, max_units)));
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(64 * NT * KW), p.lds, st, a);
    return KVE_OK;
  };
  int rc;
  if constexpr (BF16)
    rc = bs16 ? go(verify_attn_bf16_kernel<D, NT, true, KW>)
              : go(verify_attn_bf16_kernel<D, NT, false, KW>);
  else
    rc = bs16 ? go(verify_attn_f32_kernel<D, NT, true, KW>)
              : go(verify_attn_f32_kernel<D, NT, false, KW>);
  if (rc) return rc;
  // histories longer than one unit: merge their units' states (only launched
  // when max_ctx allows more than one unit per history)
  if (p.max_split > 0)
    hipLaunchKernelGGL((verify_attn_merge_kernel<D, BF16, NT>), dim3(p.max_split, a.Hkv * (D / 16)),
                       dim3(64 * NT), 0, st, a);
  return KVE_OK;
}

// Instantiated (row tiles, key waves): (1, 1), (1, 2), (1, 4), (1, 8), (2-4, 1),
// (2-4, 2), (2-3, 4), (6, 1), (6, 2), (8, 1).
template <int D, bool BF16>
static int launch_attn_nt(const AttnArgs& a, const AttnCfg& p, hipStream_t st, bool bs16) {
  const int NT = p.NT, KW = p.KW;
#define KVE_ATTN_CASE(nt, kw) \
  if (NT == nt && KW == kw) return launch_attn_t<D, BF16, nt, kw>(a, p, st, bs16);
  KVE_ATTN_CASE(1, 8)
  KVE_ATTN_CASE(1, 4)
  KVE_ATTN_CASE(1, 2)
  KVE_ATTN_CASE(1, 1)
  KVE_ATTN_CASE(2, 1)
  KVE_ATTN_CASE(2, 2)
  KVE_ATTN_CASE(2, 4)
  KVE_ATTN_CASE(3, 1)
  KVE_ATTN_CASE(3, 2)
  KVE_ATTN_CASE(3, 4)
  KVE_ATTN_CASE(4, 1)
  KVE_ATTN_CASE(4, 2)
  KVE_ATTN_CASE(6, 1)
  KVE_ATTN_CASE(6, 2)
  KVE_ATTN_CASE(8, 1)
#undef KVE_ATTN_CASE
  set_error("kve_paged_verify_attn: no kernel for %d row tiles x %d key waves", NT, KW);
  return KVE_EUNSUPPORTED;
}

// Shared argument checks and AttnArgs assembly for the plan and attention
// entry points.
static int attn_setup(AttnArgs& a, AttnCfg& p, const char* name, const int32_t* block_tables,
                      const int32_t* seq_rows, const int32_t* start_pos, const int32_t* q_lens,
                      int num_seqs, int q_len, int num_q_heads, int num_kv_heads, int head_dim,
                      int block_size, int max_blocks, int num_rows, int num_blocks, int max_ctx,
                      int unit_blocks, int key_waves, int dtype) {
  KVE_REQUIRE(block_tables && start_pos, "%s: null pointer argument", name);
  KVE_REQUIRE(num_seqs > 0 && q_len > 0, "%s: num_seqs=%d q_len=%d", name, num_seqs, q_len);
  KVE_REQUIRE(num_kv_heads > 0 && num_q_heads > 0 && num_q_heads % num_kv_heads == 0,
              "%s: %d q heads not a multiple of %d kv heads", name, num_q_heads, num_kv_heads);
  KVE_REQUIRE(head_dim == 64 || head_dim == 128, "%s: head_dim %d unsupported (64 or 128)", name,
              head_dim);
  KVE_REQUIRE(dtype == KVE_DTYPE_BF16 || dtype == KVE_DTYPE_F32, "%s: dtype %d unsupported", name,
              dtype);
  KVE_REQUIRE(block_size > 0 && max_ctx > 0 && max_blocks >= cdiv(max_ctx, block_size),
              "%s: max_blocks %d cannot hold max_ctx %d at block_size %d", name, max_blocks,
              max_ctx, block_size);
  KVE_REQUIRE(unit_blocks >= 0 && key_waves >= 0, "%s: unit_blocks %d, key_waves %d", name,
              unit_blocks, key_waves);
  KVE_REQUIRE(key_waves == 0 || key_waves == 1 || key_waves == 2 || key_waves == 4 || key_waves == 8,
              "%s: key_waves %d (0 = automatic, or 1, 2, 4, 8)", name, key_waves);
  KVE_REQUIRE(static_cast<long long>(num_q_heads) * q_len < 65536 &&
                  static_cast<long long>(num_seqs) * q_len * num_q_heads * head_dim < (1ll << 31),
              "%s: q of %d x %d x %d heads too large for one launch", name, num_seqs, q_len,
              num_q_heads);
  KVE_REQUIRE(num_rows > 0 && num_blocks > 0, "%s: num_rows=%d num_blocks=%d", name, num_rows,
              num_blocks);
  p = attn_cfg(num_seqs, q_len, num_q_heads, num_kv_heads, head_dim, max_ctx, unit_blocks,
               key_waves, block_size, dtype);
  KVE_REQUIRE(dtype == KVE_DTYPE_BF16 || p.KW != 8 || p.NT == 1,
              "%s: key waves %d with %d row tiles", name, p.KW, p.NT);
  KVE_REQUIRE(num_seqs <= kMaxLaunchSeqs, "%s: %d sequences exceed %d per launch", name, num_seqs,
              kMaxLaunchSeqs);
  KVE_REQUIRE(static_cast<long long>(num_seqs) * p.row_groups <= kMaxLaunchItems,
              "%s: %d sequences x %d row groups exceed %d per launch", name, num_seqs,
              p.row_groups, kMaxLaunchItems);
  a = AttnArgs{};
  a.tables = block_tables;
  a.seq_rows = seq_rows;
  a.start_pos = start_pos;
  a.q_lens = q_lens;
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
  a.unit_tiles = p.unit_tiles;
  a.row_groups = p.row_groups;
  a.rows = p.rows;
  a.max_units = p.max_units;
  a.max_split = p.max_split;
  a.max_item_units = p.max_item_units;
  a.lds_kv_off = p.lds_kv_off;
  a.g_magic = a.G >= 2 ? static_cast<uint32_t>(((1ull << 32) + a.G - 1) / a.G) : 0u;
  return KVE_OK;
}

}  // namespace kve

using namespace kve;

extern "C" size_t kve_attn_plan_bytes(int num_seqs, int q_len, int num_q_heads, int num_kv_heads,
                                      int head_dim, int block_size, int max_ctx, int unit_blocks,
                                      int key_waves, int dtype) {
  if (num_seqs <= 0 || q_len <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || max_ctx <= 0 ||
      block_size <= 0 || num_q_heads % num_kv_heads != 0)
    return 0;
  return attn_cfg(num_seqs, q_len, num_q_heads, num_kv_heads, head_dim, max_ctx, unit_blocks,
                  key_waves, block_size, dtype)
      .plan_bytes;
}

extern "C" size_t kve_attn_workspace_bytes(int num_seqs, int q_len, int num_q_heads,
                                           int num_kv_heads, int head_dim, int block_size,
                                           int max_ctx, int unit_blocks, int key_waves, int dtype) {
  if (num_seqs <= 0 || q_len <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || max_ctx <= 0 ||
      block_size <= 0 || num_q_heads % num_kv_heads != 0)
    return 0;
  return attn_ws_bytes(attn_cfg(num_seqs, q_len, num_q_heads, num_kv_heads, head_dim, max_ctx,
                                unit_blocks, key_waves, block_size, dtype),
                       true);
}

extern "C" int kve_attn_plan(const int32_t* block_tables, const int32_t* seq_rows,
                             const int32_t* start_pos, const int32_t* q_lens, int num_seqs,
                             int q_len, int num_q_heads, int num_kv_heads, int head_dim,
                             int block_size, int max_blocks, int num_rows, int num_blocks,
                             int max_ctx, int unit_blocks, int key_waves, int dtype, void* plan,
                             size_t plan_bytes, void* stream) {
  clear_error();
  if (num_seqs == 0) return KVE_OK;
  AttnArgs a{};
  AttnCfg p;
  int rc = attn_setup(a, p, "kve_attn_plan", block_tables, seq_rows, start_pos, q_lens, num_seqs,
                      q_len, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks, num_rows,
                      num_blocks, max_ctx, unit_blocks, key_waves, dtype);
  if (rc) return rc;
  KVE_REQUIRE(plan && (reinterpret_cast<uintptr_t>(plan) & 15) == 0,
              "kve_attn_plan: plan must be a 16-byte aligned buffer");
  if (plan_bytes < p.plan_bytes) {
    set_error("kve_attn_plan: plan buffer %zu bytes, need %zu", plan_bytes, p.plan_bytes);
    return KVE_EWORKSPACE;
  }
  a.plan = static_cast<int32_t*>(plan);
  rc = launch_plan(a, p, static_cast<hipStream_t>(stream));
  if (rc) return rc;
  return check_launch("kve_attn_plan");
}

extern "C" int kve_paged_verify_attn(const void* q, const void* k_pool, const void* v_pool,
                                     const int32_t* block_tables, const int32_t* seq_rows,
                                     const int32_t* start_pos, const int32_t* q_lens, int num_seqs,
                                     int q_len, int num_q_heads, int num_kv_heads, int head_dim,
                                     int block_size, int max_blocks, int num_rows, int num_blocks,
                                     int max_ctx, int unit_blocks, int key_waves, float scale,
                                     int dtype, const void* plan, void* out, void* workspace,
                                     size_t workspace_bytes, int layout, void* stream) {
  clear_error();
  if (num_seqs == 0) return KVE_OK;
  KVE_REQUIRE(q && k_pool && v_pool && out, "kve_paged_verify_attn: null pointer argument");
  KVE_REQUIRE(((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out) |
                reinterpret_cast<uintptr_t>(k_pool) | reinterpret_cast<uintptr_t>(v_pool)) &
               15) == 0,
              "kve_paged_verify_attn: q, out, k_pool and v_pool must be 16-byte aligned");
  AttnArgs a{};
  AttnCfg p;
  int rc = attn_setup(a, p, "kve_paged_verify_attn", block_tables, seq_rows, start_pos, q_lens,
                      num_seqs, q_len, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks,
                      num_rows, num_blocks, max_ctx, unit_blocks, key_waves, dtype);
  if (rc) return rc;
  const size_t need = attn_ws_bytes(p, plan == nullptr);
  if (need) {
    KVE_REQUIRE(workspace != nullptr && (reinterpret_cast<uintptr_t>(workspace) & 255) == 0,
                "kve_paged_verify_attn: workspace required (256-byte aligned)");
    if (workspace_bytes < need) {
      set_error("kve_paged_verify_attn: workspace %zu bytes, need %zu", workspace_bytes, need);
      return KVE_EWORKSPACE;
    }
  }
  char* ws = static_cast<char*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (plan == nullptr) {
    a.plan = reinterpret_cast<int32_t*>(ws);
    ws += p.plan_bytes;
    rc = launch_plan(a, p, st);
    if (rc) return rc;
  } else {
    KVE_REQUIRE((reinterpret_cast<uintptr_t>(plan) & 15) == 0,
                "kve_paged_verify_attn: plan must be 16-byte aligned");
    a.plan = static_cast<int32_t*>(const_cast<void*>(plan));
  }
  a.part_ml = p.max_split ? reinterpret_cast<float*>(ws) : nullptr;
  a.part_o = p.max_split ? reinterpret_cast<float*>(ws + p.part_ml_bytes) : nullptr;
  a.q = q;
  a.k = k_pool;
  a.v = v_pool;
  KVE_REQUIRE(layout == KVE_LAYOUT_ROWS ||
                  (layout == KVE_LAYOUT_BLOCKED && dtype == KVE_DTYPE_BF16 &&
                   (num_q_heads * head_dim) % 32 == 0),
              "kve_paged_verify_attn: layout %d with dtype %d", layout, dtype);
  a.out = out;
  a.out_blocked = layout == KVE_LAYOUT_BLOCKED ? 1 : 0;
  a.scale_log2 = scale * 1.4426950408889634f;
  const bool bs16 = block_size == 16;
  if (dtype == KVE_DTYPE_BF16) {
    rc = head_dim == 64 ? launch_attn_nt<64, true>(a, p, st, bs16)
                        : launch_attn_nt<128, true>(a, p, st, bs16);
  } else {
    rc = head_dim == 64 ? launch_attn_nt<64, false>(a, p, st, bs16)
                        : launch_attn_nt<128, false>(a, p, st, bs16);
  }
  if (rc) return rc;
  return check_launch("kve_paged_verify_attn");
}
