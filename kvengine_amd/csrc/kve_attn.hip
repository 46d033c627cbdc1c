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
//    G*q_len "rows" (row r = t*G + j); a row group is 16*NT of them, so all the
//    query heads sharing a kv head read each K/V tile once;
//  * the visible history is cut into 16-token key tiles, and a split is
//    `split_tiles` consecutive tiles; the 4 waves of a workgroup take every
//    4th tile of the split.
// Per key tile a wave computes S^T = K Q^T with MFMA (keys on the M side,
// rows on the N side), so each lane ends up owning one query row (lane % 16)
// and 4 keys; the row max/sum need only two cross-group shuffles. P^T is fed
// straight back as the B operand of O^T = V^T P^T, which is why V is stored
// channel-major inside a block ([D][16]): the A operand wants 4 consecutive
// keys of one channel per lane, a single 8-byte (bf16) or 16-byte (f32) load.
// Waves merge their (max, sum, O) in LDS; splits write unnormalised partials
// and the last workgroup of a (sequence, kv head, row group) to finish merges
// them, so the whole operation is one kernel.

#include "kve_common.h"

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
  float* part_o;
  float* part_ml;
  int Tq, Hq, Hkv, G, bs, max_blocks, num_rows, num_blocks, max_ctx;
  int split_tiles, max_splits, row_groups;
  float scale_log2;
};

// A block id outside the pool is never dereferenced (block 0 is read instead).
__device__ __forceinline__ int safe_block(int blk, int num_blocks) {
  return static_cast<unsigned>(blk) < static_cast<unsigned>(num_blocks) ? blk : 0;
}

constexpr int kMaxSplits = 128;
constexpr float kNegBig = -1.0e30f;

template <int D, bool BF16>
struct AttnFrag;

// bf16: Q/K fragments are 8 bf16 per 32-channel step, V is 4 bf16 per d tile.
template <int D>
struct AttnFrag<D, true> {
  static constexpr int KS = D / 32;  // MFMA k-steps over the channels
  u32x4 k[KS];
  u32x2 v[D / 16];
};

template <int D>
struct AttnFrag<D, false> {
  static constexpr int KS = D / 4;
  float k[KS];
  f32x4 v[D / 16];
};

// Channel mapping shared by Q and K fragments: lane group g (= lane/16) owns the
// contiguous quarter [g*D/4, (g+1)*D/4) of the head dimension.

template <int D, bool BF16, bool BS16>
__device__ __forceinline__ void load_kv_tile(AttnFrag<D, BF16>& f, const AttnArgs& a,
                                             const int32_t* table, int kvh, int kt, int Lk,
                                             int lr, int lg) {
  using elem_t = std::conditional_t<BF16, uint16_t, float>;
  constexpr int DQ = D / 4;
  const elem_t* kb = static_cast<const elem_t*>(a.k);
  const elem_t* vb = static_cast<const elem_t*>(a.v);
  if constexpr (BS16) {
    const int blk = safe_block(table[kt], a.num_blocks);
    const size_t tile = (static_cast<size_t>(blk) * a.Hkv + kvh) * 16 * D;
    const elem_t* kp = kb + tile + lr * D + lg * DQ;
    if constexpr (BF16) {
#pragma unroll
      for (int s = 0; s < D / 32; ++s) f.k[s] = reinterpret_cast<const u32x4*>(kp)[s];
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt)
        f.v[dt] = *reinterpret_cast<const u32x2*>(vb + tile + (dt * 16 + lr) * 16 + 4 * lg);
    } else {
#pragma unroll
      for (int s = 0; s < DQ / 4; ++s) {
        f32x4 x = reinterpret_cast<const f32x4*>(kp)[s];
        f.k[4 * s + 0] = x[0];
        f.k[4 * s + 1] = x[1];
        f.k[4 * s + 2] = x[2];
        f.k[4 * s + 3] = x[3];
      }
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt)
        f.v[dt] = *reinterpret_cast<const f32x4*>(vb + tile + (dt * 16 + lr) * 16 + 4 * lg);
    }
    // Slots past the visible history hold stale data; zero V there so a masked
    // (p = 0) slot can never contribute 0 * inf.
    if ((kt + 1) * 16 > Lk) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (kt * 16 + 4 * lg + i >= Lk) {
#pragma unroll
          for (int dt = 0; dt < D / 16; ++dt) {
            if constexpr (BF16) {
              f.v[dt][i >> 1] &= (i & 1) ? 0x0000ffffu : 0xffff0000u;
            } else {
              f.v[dt][i] = 0.0f;
            }
          }
        }
      }
    }
  } else {
    // Any block size: resolve each key's (block, offset) separately.
    const int bs = a.bs;
    const int key = kt * 16 + lr;
    if (key < Lk) {
      const int blk = safe_block(table[key / bs], a.num_blocks);
      const elem_t* kp =
          kb + ((static_cast<size_t>(blk) * a.Hkv + kvh) * bs + key % bs) * D + lg * DQ;
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
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
      if constexpr (BF16) f.v[dt] = u32x2{0, 0};
      else f.v[dt] = f32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kk = kt * 16 + 4 * lg + i;
      if (kk >= Lk) continue;
      const int blk = safe_block(table[kk / bs], a.num_blocks);
      const elem_t* vp = vb + (static_cast<size_t>(blk) * a.Hkv + kvh) * D * bs + kk % bs;
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
        const elem_t x = vp[static_cast<size_t>(dt * 16 + lr) * bs];
        if constexpr (BF16) {
          f.v[dt][i >> 1] |= static_cast<uint32_t>(x) << ((i & 1) * 16);
        } else {
          f.v[dt][i] = x;
        }
      }
    }
  }
}

// Tiles each wave loads in one burst: what fits beside the accumulators.
template <int D, bool BF16>
constexpr int burst_tiles() {
  return BF16 ? (D == 64 ? 4 : 2) : (D == 64 ? 2 : 1);
}

template <int D, bool BF16, int NT, bool BS16>
__global__ __launch_bounds__(256) void paged_verify_attn_kernel(AttnArgs a) {
  using elem_t = std::conditional_t<BF16, uint16_t, float>;
  constexpr int NPRE = burst_tiles<D, BF16>();
  constexpr int ROWS = 16 * NT;
  constexpr int DT = D / 16;
  constexpr int DQ = D / 4;
  constexpr int KS = AttnFrag<D, BF16>::KS;
  constexpr int LDO = D + 1;  // padded row stride of the LDS accumulator
  __shared__ float sm_buf[ROWS * LDO];
  __shared__ float sm_m[4][ROWS];
  __shared__ float sm_l[4][ROWS];
  __shared__ float sm_rowM[ROWS];
  __shared__ float sm_rowL[ROWS];

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, lr = l & 15, lg = l >> 4;
  const int b = blockIdx.z / a.Hkv, kvh = blockIdx.z % a.Hkv;
  const int rg = blockIdx.y, s = blockIdx.x;
  const int row = a.seq_rows ? a.seq_rows[b] : b;
  if (row < 0 || row >= a.num_rows) return;
  const int start = a.start_pos[row];
  const int T = a.q_lens ? min(a.q_lens[b], a.Tq) : a.Tq;
  if (T <= 0 || start < 0 || start + T > a.max_ctx) return;
  const int R = a.G * T;
  const int row0 = rg * ROWS;
  if (row0 >= R) return;
  const int row_end = min(R, row0 + ROWS);
  const int Lk = start + (row_end - 1) / a.G + 1;  // keys visible to this row group
  const int ntiles = cdiv(Lk, 16);
  const int nsplit = cdiv(ntiles, a.split_tiles);
  if (s >= nsplit) return;
  const int kt0 = s * a.split_tiles;
  const int kt1 = min(ntiles, kt0 + a.split_tiles);
  const int32_t* table = a.tables + static_cast<size_t>(row) * a.max_blocks;

  // Query fragments of this lane's row in each row tile, and its causal limit.
  const elem_t* qb = static_cast<const elem_t*>(a.q);
  int qlim[NT];
  u32x4 qf16[BF16 ? NT : 1][BF16 ? KS : 1];
  float qf32[BF16 ? 1 : NT][BF16 ? 1 : KS];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int r = row0 + nt * 16 + lr;
    const bool ok = r < R;
    const int t = ok ? r / a.G : 0;
    const int h = kvh * a.G + (ok ? r % a.G : 0);
    qlim[nt] = ok ? start + t : -1;
    const elem_t* qp = qb + ((static_cast<size_t>(b) * a.Tq + t) * a.Hq + h) * D + lg * DQ;
    if constexpr (BF16) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        qf16[nt][ks] = ok ? reinterpret_cast<const u32x4*>(qp)[ks] : u32x4{0, 0, 0, 0};
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qf32[nt][ks] = ok ? qp[ks] : 0.0f;
    }
  }

  float m_run[NT], l_run[NT];
  f32x4 acc[NT][DT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    m_run[nt] = kNegBig;
    l_run[nt] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[nt][dt] = f32x4{0, 0, 0, 0};
  }

  // One memory round trip per work item: every wave issues the loads of all its
  // tiles of a round (NPRE of them, registers permitting) before any math, so
  // a split costs one HBM latency plus the MFMA work instead of one latency
  // per tile. Rounds repeat only when the caller asks for splits longer than
  // 4 * NPRE tiles.
  auto attend_tile = [&](const AttnFrag<D, BF16>& f, int kt) {
  #pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        f32x4 st = {0, 0, 0, 0};
  #pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          if constexpr (BF16) st = mfma16x16x32_bf16(f.k[ks], qf16[nt][ks], st);
          else st = mfma16x16x4_f32(f.k[ks], qf32[nt][ks], st);
        }
        float sv[4];
        float tmax = -INFINITY;
  #pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kt * 16 + 4 * lg + i;
          sv[i] = key <= qlim[nt] ? st[i] * a.scale_log2 : -INFINITY;
          tmax = fmaxf(tmax, sv[i]);
        }
        tmax = max_across_groups(tmax);
        const float m_new = fmaxf(m_run[nt], tmax);
        const float alpha = exp2f(m_run[nt] - m_new);
        float p[4];
  #pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = exp2f(sv[i] - m_new);
        l_run[nt] = l_run[nt] * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
        m_run[nt] = m_new;
  #pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[nt][dt] *= alpha;
        if constexpr (BF16) {
          // P = hi + lo with both halves in bf16 (16 significant bits): the PV
          // product then carries no rounding beyond the final output's.
          uint16_t hi[4], lo[4];
  #pragma unroll
          for (int i = 0; i < 4; ++i) {
            hi[i] = f32_to_bf16(p[i]);
            lo[i] = f32_to_bf16(p[i] - bf16_to_f32(hi[i]));
          }
          const u32x2 ph = {static_cast<uint32_t>(hi[0]) | (static_cast<uint32_t>(hi[1]) << 16),
                            static_cast<uint32_t>(hi[2]) | (static_cast<uint32_t>(hi[3]) << 16)};
          const u32x2 pl = {static_cast<uint32_t>(lo[0]) | (static_cast<uint32_t>(lo[1]) << 16),
                            static_cast<uint32_t>(lo[2]) | (static_cast<uint32_t>(lo[3]) << 16)};
  #pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            acc[nt][dt] = mfma16x16x16_bf16(f.v[dt], ph, acc[nt][dt]);
            acc[nt][dt] = mfma16x16x16_bf16(f.v[dt], pl, acc[nt][dt]);
          }
        } else {
  #pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
  #pragma unroll
            for (int i = 0; i < 4; ++i) acc[nt][dt] = mfma16x16x4_f32(f.v[dt][i], p[i], acc[nt][dt]);
          }
        }
      }
  };
  for (int r0 = kt0; r0 < kt1; r0 += 4 * NPRE) {
    AttnFrag<D, BF16> fr[NPRE];
#pragma unroll
    for (int j = 0; j < NPRE; ++j) {
      const int kt = r0 + w + 4 * j;
      if (kt < kt1) load_kv_tile<D, BF16, BS16>(fr[j], a, table, kvh, kt, Lk, lr, lg);
    }
#pragma unroll
    for (int j = 0; j < NPRE; ++j) {
      const int kt = r0 + w + 4 * j;
      if (kt < kt1) attend_tile(fr[j], kt);
    }
  }

  // ---- merge the four waves in LDS ----
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const float lt = sum_across_groups(l_run[nt]);
    if (lg == 0) {
      sm_m[w][nt * 16 + lr] = m_run[nt];
      sm_l[w][nt * 16 + lr] = lt;
    }
  }
  __syncthreads();
  float fscale[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int rr = nt * 16 + lr;
    const float M = fmaxf(fmaxf(sm_m[0][rr], sm_m[1][rr]), fmaxf(sm_m[2][rr], sm_m[3][rr]));
    fscale[nt] = exp2f(m_run[nt] - M);
  }
  if (tid < ROWS) {
    const float M = fmaxf(fmaxf(sm_m[0][tid], sm_m[1][tid]), fmaxf(sm_m[2][tid], sm_m[3][tid]));
    float L = 0.0f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) L += sm_l[ww][tid] * exp2f(sm_m[ww][tid] - M);
    sm_rowM[tid] = M;
    sm_rowL[tid] = L;
  }
  for (int ww = 0; ww < 4; ++ww) {
    if (w == ww) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float* dst = &sm_buf[(nt * 16 + lr) * LDO + dt * 16 + 4 * lg + i];
            const float x = acc[nt][dt][i] * fscale[nt];
            *dst = (ww == 0) ? x : *dst + x;
          }
        }
      }
    }
    __syncthreads();
  }

  elem_t* ob = static_cast<elem_t*>(a.out);
  if (nsplit == 1) {
    for (int idx = tid; idx < ROWS * D; idx += 256) {
      const int rr = idx / D, d = idx % D;
      const int r = row0 + rr;
      if (r >= R) continue;
      const int t = r / a.G, h = kvh * a.G + r % a.G;
      const float x = sm_buf[rr * LDO + d] / sm_rowL[rr];
      elem_t* op = ob + ((static_cast<size_t>(b) * a.Tq + t) * a.Hq + h) * D + d;
      if constexpr (BF16) *op = f32_to_bf16(x);
      else *op = x;
    }
    return;
  }

  // ---- split: publish the partial; kve_attn_combine merges after this kernel ----
  const int item = (b * a.Hkv + kvh) * a.row_groups + rg;
  float* po = a.part_o + (static_cast<size_t>(item) * a.max_splits + s) * ROWS * D;
  float* pml = a.part_ml + (static_cast<size_t>(item) * a.max_splits + s) * ROWS * 2;
  const int nrows = row_end - row0;
  for (int idx = tid; idx < nrows * D; idx += 256) po[idx] = sm_buf[(idx / D) * LDO + idx % D];
  if (tid < nrows) {
    pml[2 * tid] = sm_rowM[tid];
    pml[2 * tid + 1] = sm_rowL[tid];
  }
}

// Merge the split partials of one (sequence, kv head, row group):
// O = sum_s exp2(m_s - M) * acc_s / sum_s exp2(m_s - M) * l_s.
// Launched right after the attention kernel; work items with a single split
// were finished there and exit here at once.
template <int D, bool BF16, int NT>
__global__ __launch_bounds__(256) void verify_attn_combine_kernel(AttnArgs a) {
  using elem_t = std::conditional_t<BF16, uint16_t, float>;
  constexpr int ROWS = 16 * NT;
  __shared__ float sm_f[kMaxSplits * ROWS];
  __shared__ float sm_L[ROWS];
  const int tid = threadIdx.x;
  const int item = blockIdx.x;
  const int rg = item % a.row_groups;
  const int bk = item / a.row_groups;
  const int b = bk / a.Hkv, kvh = bk % a.Hkv;
  const int row = a.seq_rows ? a.seq_rows[b] : b;
  if (row < 0 || row >= a.num_rows) return;
  const int start = a.start_pos[row];
  const int T = a.q_lens ? min(a.q_lens[b], a.Tq) : a.Tq;
  if (T <= 0 || start < 0 || start + T > a.max_ctx) return;
  const int R = a.G * T;
  const int row0 = rg * ROWS;
  if (row0 >= R) return;
  const int row_end = min(R, row0 + ROWS);
  const int Lk = start + (row_end - 1) / a.G + 1;
  const int nsplit = cdiv(cdiv(Lk, 16), a.split_tiles);
  if (nsplit <= 1) return;
  const int nrows = row_end - row0;
  const float* po0 = a.part_o + static_cast<size_t>(item) * a.max_splits * ROWS * D;
  const float* pml0 = a.part_ml + static_cast<size_t>(item) * a.max_splits * ROWS * 2;
  if (tid < nrows) {
    float M = kNegBig;
    for (int ss = 0; ss < nsplit; ++ss) M = fmaxf(M, pml0[ss * ROWS * 2 + 2 * tid]);
    float L = 0.0f;
    for (int ss = 0; ss < nsplit; ++ss) {
      const float f = exp2f(pml0[ss * ROWS * 2 + 2 * tid] - M);
      sm_f[ss * ROWS + tid] = f;
      L += pml0[ss * ROWS * 2 + 2 * tid + 1] * f;
    }
    sm_L[tid] = L;
  }
  __syncthreads();
  elem_t* ob = static_cast<elem_t*>(a.out);
  // float4 per thread; the split loop issues 8 independent loads per step so
  // the merge costs a few memory round trips, not one per split.
  for (int idx = tid; idx < nrows * (D / 4); idx += 256) {
    const int rr = idx / (D / 4), d = (idx % (D / 4)) * 4;
    const float* src = po0 + rr * D + d;
    f32x4 x = {0, 0, 0, 0};
    int ss = 0;
    for (; ss + 8 <= nsplit; ss += 8) {
      f32x4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        v[u] = *reinterpret_cast<const f32x4*>(src + static_cast<size_t>(ss + u) * ROWS * D);
#pragma unroll
      for (int u = 0; u < 8; ++u) x += v[u] * sm_f[(ss + u) * ROWS + rr];
    }
    for (; ss < nsplit; ++ss)
      x += *reinterpret_cast<const f32x4*>(src + static_cast<size_t>(ss) * ROWS * D) *
           sm_f[ss * ROWS + rr];
    const float inv = 1.0f / sm_L[rr];
    const int r = row0 + rr;
    const int t = r / a.G, h = kvh * a.G + r % a.G;
    elem_t* op = ob + ((static_cast<size_t>(b) * a.Tq + t) * a.Hq + h) * D + d;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (BF16) op[e] = f32_to_bf16(x[e] * inv);
      else op[e] = x[e] * inv;
    }
  }
}

// ---- host side ----------------------------------------------------------------

struct AttnPlan {
  int NT, rows, row_groups, split_tiles, max_splits, items;
  size_t off_ml, off_o, bytes;
};

static int rows_per_group(int head_dim, int dtype) {
  if (dtype == KVE_DTYPE_BF16) return 3;
  return head_dim == 64 ? 2 : 1;
}

static inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

static AttnPlan plan_attn(int num_seqs, int q_len, int Hq, int Hkv, int D, int max_ctx,
                          int split_blocks, int block_size, int dtype) {
  AttnPlan p{};
  p.NT = rows_per_group(D, dtype);
  p.rows = 16 * p.NT;
  p.row_groups = cdiv((Hq / Hkv) * q_len, p.rows);
  const int tiles = cdiv(max_ctx, 16);
  int st;
  if (split_blocks > 0) {
    // Caller's split is in blocks; keep it in 16-token tiles, at least one.
    st = block_size == 16 ? split_blocks : cdiv(split_blocks * block_size, 16);
  } else {
    st = 4 * (dtype == KVE_DTYPE_BF16 ? (D == 64 ? 4 : 2) : (D == 64 ? 2 : 1));
  }
  st = max(st, cdiv(tiles, kMaxSplits));
  st = max(st, 1);
  p.split_tiles = st;
  p.max_splits = cdiv(tiles, st);
  const size_t items = static_cast<size_t>(num_seqs) * Hkv * p.row_groups;
  p.items = static_cast<int>(items);
  p.off_ml = 0;
  if (p.max_splits > 1) {
    p.off_o = align256(items * p.max_splits * p.rows * 2 * sizeof(float));
    p.bytes = p.off_o + align256(items * p.max_splits * p.rows * D * sizeof(float));
  } else {
    p.off_o = 0;
    p.bytes = 0;
  }
  return p;
}

template <int D, bool BF16, int NT>
static void launch_attn_t(const AttnArgs& a, dim3 grid, int items, bool split, hipStream_t st,
                          bool bs16) {
  if (bs16)
    hipLaunchKernelGGL((paged_verify_attn_kernel<D, BF16, NT, true>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((paged_verify_attn_kernel<D, BF16, NT, false>), grid, dim3(256), 0, st, a);
  if (split)
    hipLaunchKernelGGL((verify_attn_combine_kernel<D, BF16, NT>), dim3(items), dim3(256), 0, st, a);
}

}  // namespace kve

using namespace kve;

extern "C" size_t kve_attn_workspace_bytes(int num_seqs, int q_len, int num_q_heads,
                                           int num_kv_heads, int head_dim, int block_size,
                                           int max_ctx, int split_blocks, int dtype) {
  if (num_seqs <= 0 || q_len <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || max_ctx <= 0 ||
      block_size <= 0)
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
  KVE_REQUIRE(num_rows > 0 && num_blocks > 0, "kve_paged_verify_attn: num_rows=%d num_blocks=%d",
              num_rows, num_blocks);
  const AttnPlan p = plan_attn(num_seqs, q_len, num_q_heads, num_kv_heads, head_dim, max_ctx,
                               split_blocks, block_size, dtype);
  if (p.max_splits > 1) {
    KVE_REQUIRE(workspace != nullptr, "kve_paged_verify_attn: workspace required");
    if (workspace_bytes < p.bytes) {
      set_error("kve_paged_verify_attn: workspace %zu bytes, need %zu", workspace_bytes, p.bytes);
      return KVE_EWORKSPACE;
    }
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
  char* ws = static_cast<char*>(workspace);
  a.part_ml = ws ? reinterpret_cast<float*>(ws + p.off_ml) : nullptr;
  a.part_o = ws ? reinterpret_cast<float*>(ws + p.off_o) : nullptr;
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
  a.scale_log2 = scale * 1.4426950408889634f;
  const dim3 grid(p.max_splits, p.row_groups, num_seqs * num_kv_heads);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool bs16 = block_size == 16;
  const bool split = p.max_splits > 1;
  if (dtype == KVE_DTYPE_BF16) {
    if (head_dim == 64) launch_attn_t<64, true, 3>(a, grid, p.items, split, st, bs16);
    else launch_attn_t<128, true, 3>(a, grid, p.items, split, st, bs16);
  } else {
    if (head_dim == 64) launch_attn_t<64, false, 2>(a, grid, p.items, split, st, bs16);
    else launch_attn_t<128, false, 1>(a, grid, p.items, split, st, bs16);
  }
  return check_launch("kve_paged_verify_attn");
}
