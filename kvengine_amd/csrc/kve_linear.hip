// Skinny bf16 linear layers for decode-sized batches on gfx950, with the
// elementwise work around them in a Qwen2 layer fused in.
//
// In a speculative iteration the draft model runs its 24 layers once per
// drafted token over B rows (B <= 64), where each projection is a GEMV-like
// stream of the weight matrix and every separate elementwise op costs a
// launch. The reference runs, per layer (kvengine/forward.py:190-207 calling
// transformers' Qwen2 modules, models/qwen2/modeling_qwen2.py:35-48, 237-255):
// RMSNorm, q/k/v Linear (+bias), RoPE, cache write, attention, o_proj, residual
// add, RMSNorm, gate/up Linear, SiLU, mul, down Linear, residual add. Here:
//
//   kve_fused_qkv:       RMSNorm(residual) -> [q|k|v] Linear + bias -> RoPE ->
//                        q for the attention kernel, k/v into the paged pool
//   kve_linear_residual: residual += x W^T (o_proj, down_proj)
//   kve_fused_gate_up:   RMSNorm(residual) -> [gate|up] Linear -> SiLU(gate)*up
//
// Every value the reference materialises in bf16 is rounded to bf16 at the
// same point here (Linear outputs, the residual sums, RMSNorm's cast before the
// weight multiply, RoPE's products and sum, SiLU's result and the product).
//
// GEMM shape: Y[M, N] = X[M, K] W[N, K]^T with the weight row-major ([N, K], as
// torch keeps nn.Linear.weight). One wave's MFMA tile holds 16 weight rows and
// all M rows: MFMA 16x16x32 with the weight rows on the M side, so a lane ends
// up with 4 consecutive output columns of one X row (o/down_proj and q/k/v give
// a wave 4 to 8 distinct columns, repeated over the tile's 16 rows, to spread
// a projection over more workgroups). The weight rows
// are read straight from HBM in 16-byte pieces, up to 16 k-steps (16 KB per
// wave) issued ahead of the math; X is staged once per workgroup in LDS (normalised
// there when the op starts with RMSNorm), or, for long K, each wave reads its
// own K range of X and the four partial sums meet in LDS.

#include "kve_common.h"
#include "kve_gemm.h"

#include <algorithm>

#pragma clang fp contract(off)

namespace kve {

constexpr int kLinMaxRows = 64;
constexpr size_t kLinMaxLds = 159 * 1024;  // LDS of one gfx950 CU, less the static arrays

__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
// Two floats -> packed bf16 pair, round to nearest even (the same rounding as
// torch's float -> bfloat16 for every finite value).
__device__ __forceinline__ uint32_t bf_pack(float a, float b) { return pack_bf16x2(a, b); }
__device__ __forceinline__ float rbf(float x) { return round_bf16_hw(x); }

// acc[mt] += W[n0..n0+16, k range] . X[mt*16.., k range]^T for k-steps [ks0, ks1).
// W row n0 + lr, k = 32*ks + 8*lg..+7 per lane; X fragments come from `xfrag(mt, ks)`.
// The weight loads of PF k-steps (PF KB per wave) are issued before the math of
// the previous PF, so about 2*PF KB per wave are in flight.
template <int MT, int PF, typename XF>
__device__ __forceinline__ void wave_gemm(const uint16_t* w_row, int ks0, int ks1, XF xfrag,
                                          f32x4 (&acc)[MT], int lg) {
  const u32x4* wp = reinterpret_cast<const u32x4*>(w_row + 8 * lg);  // step ks at wp[4*ks]
  u32x4 wa[PF], wb[PF];
  // every slot is loaded (past ks1 it repeats the last step): a fixed number
  // of loads per chunk lets the compiler wait for exactly the chunk it needs
  auto load = [&](u32x4 (&dst)[PF], int c0) {
#pragma unroll
    for (int j = 0; j < PF; ++j) dst[j] = wp[4 * min(c0 + j, ks1 - 1)];
  };
  auto run = [&](const u32x4 (&src)[PF], int c0) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      if (c0 + j >= ks1) break;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma16x16x32_bf16(src[j], xfrag(mt, c0 + j), acc[mt]);
    }
  };
  // the loop runs while both following chunks exist, so every load in it is
  // unconditional: with `if (next exists) load(next)` before each chunk's
  // math the compiler, merging the paths with and without that load, waited
  // for every load (the next chunk's too) before the math
  load(wa, ks0);
  int c = ks0;
  for (; c + 2 * PF < ks1; c += 2 * PF) {
    load(wb, c + PF);
    run(wa, c);
    load(wa, c + 2 * PF);
    run(wb, c + PF);
  }
  if (c + PF < ks1) {
    load(wb, c + PF);
    run(wa, c);
    run(wb, c + PF);
  } else {
    run(wa, c);
  }
}

// Same with X read from global memory: the X fragments of a chunk are loaded
// together with its weights.
// kst: 16-byte vectors from one k-step of the weight to the next (4 row-major,
// 64 blocked: a 16-row tile's k-step is then one contiguous 1 KB block).
template <int MT, int PF>
__device__ __forceinline__ void wave_gemm_gx(const uint16_t* w_row, const uint16_t* x, int M, int K,
                                             int ks0, int ks1, f32x4 (&acc)[MT], int lr, int lg,
                                             int kst) {
  const u32x4* wp = reinterpret_cast<const u32x4*>(w_row + 8 * lg);
  const u32x4* xp[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + lr;  // rows past M read row 0 (in bounds); their sums are dropped
    xp[mt] = reinterpret_cast<const u32x4*>(x + static_cast<size_t>(m < M ? m : 0) * K + 8 * lg);
  }
  u32x4 wa[PF], wb[PF], xa[PF][MT], xb[PF][MT];
  auto load = [&](u32x4 (&dw)[PF], u32x4 (&dx)[PF][MT], int c0) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int ks = min(c0 + j, ks1 - 1);  // fixed load count (see wave_gemm)
      dw[j] = wp[kst * ks];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) dx[j][mt] = xp[mt][4 * ks];
    }
  };
  auto run = [&](const u32x4 (&sw)[PF], const u32x4 (&sx)[PF][MT], int c0) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      if (c0 + j >= ks1) break;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma16x16x32_bf16(sw[j], sx[j][mt], acc[mt]);
    }
  };
  load(wa, xa, ks0);
  int c = ks0;  // loop and tail as in wave_gemm
  for (; c + 2 * PF < ks1; c += 2 * PF) {
    load(wb, xb, c + PF);
    run(wa, xa, c);
    load(wa, xa, c + 2 * PF);
    run(wb, xb, c + PF);
  }
  if (c + PF < ks1) {
    load(wb, xb, c + PF);
    run(wa, xa, c);
    run(wb, xb, c + PF);
  } else {
    run(wa, xa, c);
  }
}

// The weight slice of a wave, loaded before anything else the kernel waits for:
// W row `w_row` (16 B per lane per k-step, k-steps kst vectors apart: 4
// row-major, 64 blocked), first min(PF, nks) k-steps.
template <int PF>
struct WPrefetch {
  u32x4 w[PF];
  const u32x4* wp;
  int nks, kst;
  __device__ __forceinline__ void issue(const uint16_t* w_row, int nks_, int lg, int kst_) {
    wp = reinterpret_cast<const u32x4*>(w_row + 8 * lg);
    nks = nks_;
    kst = kst_;
    // PF loads whatever nks is (clamped to the last step): later waits for
    // older loads (the rows to normalise) then never wait for these
#pragma unroll
    for (int j = 0; j < PF; ++j) w[j] = wp[kst * min(j, nks - 1)];
  }
  // acc[mt] += this slice . X^T; beyond PF k-steps the next PF are loaded once
  // the current ones are consumed.
  template <int MT, typename XF>
  __device__ __forceinline__ void run(XF xfrag, f32x4 (&acc)[MT]) {
    for (int c = 0; c < nks; c += PF) {
#pragma unroll
      for (int j = 0; j < PF; ++j) {
        if (c + j >= nks) break;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma16x16x32_bf16(w[j], xfrag(mt, c + j), acc[mt]);
      }
      if (c + PF < nks) {
#pragma unroll
        for (int j = 0; j < PF; ++j) w[j] = wp[kst * min(c + PF + j, nks - 1)];
      }
    }
  }
};

// RMSNorm of rows [0, M) of residual [M, H] into LDS (bf16, row stride ldx):
// x = w * cast(r * rsqrt(mean(r^2) + eps)), as the reference's Qwen2RMSNorm.
// One wave per row (rows w, w+4, ...: at most RW per wave); each lane owns
// 16-byte vectors l, l+64, ... of a row. `load` issues every read of the wave;
// `store` waits for them, so loads issued in between (the weights) stay in
// flight during the normalisation.
template <int NV, int RW>
struct NormStage {
  u32x4 wv[NV];
  u32x4 xv[RW][NV];
  __device__ __forceinline__ void load(const uint16_t* residual, const uint16_t* norm_w, int M,
                                       int H, int w, int l) {
    // Unconditional loads (rows past M and vectors past the row repeat the
    // last one; `store` skips them): a fixed count, so the wait in `store` is
    // for these loads only, not for the weight loads issued after them.
    const int nvec = H / 8;
#pragma unroll
    for (int k = 0; k < NV; ++k)
      wv[k] = reinterpret_cast<const u32x4*>(norm_w)[min(l + 64 * k, nvec - 1)];
#pragma unroll
    for (int rb = 0; rb < RW; ++rb) {
      const int m = min(w + 4 * rb, M - 1);
      const u32x4* rr = reinterpret_cast<const u32x4*>(residual + static_cast<size_t>(m) * H);
#pragma unroll
      for (int k = 0; k < NV; ++k) xv[rb][k] = rr[min(l + 64 * k, nvec - 1)];
    }
  }
  __device__ __forceinline__ void store(float eps, int M, int H, uint16_t* sx, int ldx, int w, int l) {
    const int nvec = H / 8;
    const float inv_h = 1.0f / static_cast<float>(H);
#pragma unroll
    for (int rb = 0; rb < RW; ++rb) {
      const int m = w + 4 * rb;
      if (m >= M) break;
      float ss = 0.0f;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        if (l + 64 * k >= nvec) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a = bf_lo(xv[rb][k][e]), b = bf_hi(xv[rb][k][e]);
          ss = __fadd_rn(ss, __fadd_rn(__fmul_rn(a, a), __fmul_rn(b, b)));
        }
      }
      ss = wave_sum(ss);
      const float inv = rsqrtf(__fadd_rn(__fmul_rn(ss, inv_h), eps));
      uint16_t* dst = sx + static_cast<size_t>(m) * ldx;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        if (l + 64 * k >= nvec) continue;
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a = rbf(__fmul_rn(bf_lo(xv[rb][k][e]), inv));
          const float b = rbf(__fmul_rn(bf_hi(xv[rb][k][e]), inv));
          o[e] = bf_pack(__fmul_rn(bf_lo(wv[k][e]), a), __fmul_rn(bf_hi(wv[k][e]), b));
        }
        *reinterpret_cast<u32x4*>(dst + 8 * (l + 64 * k)) = o;
      }
    }
  }
};

// X fragment of row tile mt, k-step ks from LDS rows of stride ldx.
struct LdsX {
  const uint16_t* sx;
  int ldx, lr, lg;
  __device__ __forceinline__ u32x4 operator()(int mt, int ks) const {
    return *reinterpret_cast<const u32x4*>(sx + (mt * 16 + lr) * ldx + 32 * ks + 8 * lg);
  }
};

// ---- [q|k|v] projection with RMSNorm, bias, RoPE and the KV write ------------
// A head slot of D columns (q head, k head or v head) is shared by kQkvSplit = 4
// workgroups: workgroup p owns the RoPE pairs j in [p*D/8, (p+1)*D/8) (columns j
// and j + D/2), its waves 0-1 the first columns of those pairs and waves 2-3
// the second, CW = D/16 columns per wave. A wave's MFMA tile has 16 weight
// rows, tile row r holding column r % CW. Each column is one wave's sum over
// every k-step in order, as with one workgroup per slot (0.5B, one row: 18
// workgroups -> 72, 7.0 -> 6.5 us).
struct QkvArgs {
  const uint16_t* residual;  // [M, H]
  const uint16_t* norm_w;    // [H]
  const uint16_t* w;         // [(Hq + 2 Hkv) D, H], row-major or blocked (w_blocked)
  const uint16_t* bias;      // [(Hq + 2 Hkv) D]
  const uint16_t* cos;       // [M, D]
  const uint16_t* sin;       // [M, D]
  uint16_t* q_out;           // [M, Hq, D]
  uint16_t* k_pool;          // [NB, Hkv, bs, D]
  uint16_t* v_pool;          // [NB, Hkv, D, bs]
  const int32_t* tables;
  const int32_t* seq_rows;
  const int32_t* start_pos;
  const int32_t* q_lens;
  int M, Tq, H, Hq, Hkv, bs, max_blocks, num_rows, num_blocks;
  int w_blocked;
  float eps;
};

constexpr int kQkvSplit = 4;

template <int MT, int D, int NV>
__global__ __launch_bounds__(256) void fused_qkv_kernel(QkvArgs a) {
  constexpr int DL = D / kQkvSplit;  // columns of the workgroup
  constexpr int hl = DL / 2;         // its RoPE pairs
  constexpr int CW = DL / 4;         // columns of each wave
  constexpr int PF = 32;             // k-steps of weights prefetched
  extern __shared__ __align__(16) uint16_t sm_lin[];
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63, lr = l & 15, lg = l >> 4;
  const int ldx = a.H + 8;
  uint16_t* sx = sm_lin;                                         // [16 MT][H + 8]
  float* sy = reinterpret_cast<float*>(sm_lin + 16 * MT * ldx);  // [16 MT][D + 1], DL used
  uint16_t* scs = reinterpret_cast<uint16_t*>(sy + 16 * MT * (D + 1));  // cos [M][D], sin [M][D]
  __shared__ int sm_slot[kLinMaxRows];  // pool slot (block * bs + offset) of each row, -1: none
  const int hs = blockIdx.x / kQkvSplit;  // head slot
  const int part = blockIdx.x - hs * kQkvSplit;
  const int n_base = hs * D;
  const bool is_q = hs < a.Hq, is_k = !is_q && hs < a.Hq + a.Hkv;
  const int nks = a.H / 32;
  // slot column of the workgroup's local column lc (pairs first halves, then second halves)
  auto col_of = [&](int lc) { return lc < hl ? part * hl + lc : D / 2 + part * hl + lc - hl; };
  const int c0 = (w < 2 ? 0 : hl) + (w & 1) * CW;  // first local column of this wave

  // 1. reads, oldest first so each wait covers only what it needs: the first
  //    step of the pool-slot lookup of k/v rows (the sequence's q_len and
  //    table row), the rows to normalise, this wave's weight rows, its bias,
  //    cos/sin (q and k slots). The lookup is a chain of dependent loads:
  //    its second step (start position) is issued once the rows to normalise
  //    have landed, its third (block table entry) after the GEMM, so one
  //    round trip, not four, follows the GEMM.
  const int crow = min(tid, a.M - 1), ci = crow / a.Tq, ct = crow - ci * a.Tq;
  int c_ql = a.Tq, c_row = ci;
  if (!is_q) {
    if (a.q_lens) c_ql = a.q_lens[ci];
    if (a.seq_rows) c_row = a.seq_rows[ci];
  }
  NormStage<NV, 4 * MT> ns;
  ns.load(a.residual, a.norm_w, a.M, a.H, w, l);
  WPrefetch<PF> wpf;
  wpf.issue(a.w + mat_off(n_base + col_of(c0 + lr % CW), 0, a.H, a.H, a.w_blocked), nks, lg,
            a.w_blocked ? 64 : 4);
  // lanes holding tile rows 0..CW-1 store the output; the others read the
  // first lanes' bias (in bounds) and drop it
  const uint32_t* bb =
      reinterpret_cast<const uint32_t*>(a.bias + n_base + col_of(c0 + (4 * lg < CW ? 4 * lg : 0)));
  const uint32_t b01 = bb[0], b23 = bb[1];
  // cos/sin into registers (stored to LDS once the GEMM is done)
  constexpr int CSV = cdiv(2 * 16 * MT * D / 8, 256);  // 16-byte vectors per thread
  const int ncs = (is_q || is_k) ? a.M * D / 8 : 0;        // vectors of one table
  u32x4 csr[CSV];
#pragma unroll
  for (int v = 0; v < CSV; ++v) {
    const int i = tid + 256 * v;
    if (i < 2 * ncs)
      csr[v] = reinterpret_cast<const u32x4*>(i < ncs ? a.cos : a.sin)[i < ncs ? i : i - ncs];
  }
  // 2. the slot lookup's second step, then the normalised rows
  const bool c_ok = !is_q && tid < a.M && ct < min(c_ql, a.Tq) && c_row >= 0 && c_row < a.num_rows;
  int c_start = 0;  // used as loaded (an add here would wait for it right away)
  if (c_ok) c_start = a.start_pos[c_row];
  ns.store(a.eps, a.M, a.H, sx, ldx, w, l);
  __syncthreads();

  const LdsX xf{sx, ldx, lr, lg};
  {
    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0, 0, 0, 0};
    wpf.template run<MT>(xf, acc);
    if (4 * lg < CW) {  // lanes holding tile rows 0..CW-1 (the rest repeat them)
      // Linear output with bias, rounded to bf16 (F.linear's output)
      const float b4[4] = {bf_lo(b01), bf_hi(b01), bf_lo(b23), bf_hi(b23)};
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + lr;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          sy[m * (D + 1) + c0 + 4 * lg + i] = rbf(__fadd_rn(acc[mt][i], b4[i]));
      }
    }
  }
  // 3. with every weight load consumed, the waits below hold up nothing else
#pragma unroll
  for (int v = 0; v < CSV; ++v) {
    const int i = tid + 256 * v;
    if (i < 2 * ncs) reinterpret_cast<u32x4*>(scs)[i] = csr[v];
  }
  if (!is_q && tid < a.M) {
    // pool slot of row tid = token ct of sequence ci, as kv_slots_kernel
    int slot = -1;
    const int c_pos = c_start + ct;
    if (c_ok && c_pos >= 0 && c_pos / a.bs < a.max_blocks) {
      const int b = a.tables[static_cast<size_t>(c_row) * a.max_blocks + c_pos / a.bs];
      if (b >= 0 && b < a.num_blocks) slot = b * a.bs + c_pos % a.bs;
    }
    sm_slot[tid] = slot;
  }
  __syncthreads();

  // ---- epilogue: rotate (q, k) and write q / K / V ----
  constexpr int half = D / 2;
  for (int idx = tid; idx < a.M * (is_q || is_k ? hl : DL); idx += 256) {
    const int m = is_q || is_k ? idx / hl : idx / DL;
    const int jl = is_q || is_k ? idx - m * hl : idx - m * DL;  // local column
    const int j = col_of(jl);                                    // slot column
    int blk = 0, off = 0;
    if (!is_q) {
      const int slot = sm_slot[m];
      if (slot < 0) continue;  // padding row, bad row or table
      blk = slot / a.bs;
      off = slot - blk * a.bs;
    }
    if (is_q || is_k) {
      const float x0 = sy[m * (D + 1) + jl], x1 = sy[m * (D + 1) + jl + hl];
      const uint16_t* cr = scs + m * D;
      const uint16_t* sr = scs + (a.M + m) * D;
      const float c_lo = bf16_to_f32(cr[j]), c_hi = bf16_to_f32(cr[j + half]);
      const float s_lo = bf16_to_f32(sr[j]), s_hi = bf16_to_f32(sr[j + half]);
      const float lo = rbf(__fadd_rn(rbf(__fmul_rn(x0, c_lo)), rbf(__fmul_rn(-x1, s_lo))));
      const float hi = rbf(__fadd_rn(rbf(__fmul_rn(x1, c_hi)), rbf(__fmul_rn(x0, s_hi))));
      uint16_t* dst = is_q ? a.q_out + (static_cast<size_t>(m) * a.Hq + hs) * D
                           : a.k_pool + ((static_cast<size_t>(blk) * a.Hkv + (hs - a.Hq)) * a.bs + off) * D;
      dst[j] = static_cast<uint16_t>(pack_bf16x2(lo, 0.0f));
      dst[j + half] = static_cast<uint16_t>(pack_bf16x2(hi, 0.0f));
    } else {
      const int kh = hs - a.Hq - a.Hkv;
      a.v_pool[((static_cast<size_t>(blk) * a.Hkv + kh) * D + j) * a.bs + off] =
          static_cast<uint16_t>(pack_bf16x2(sy[m * (D + 1) + jl], 0.0f));
    }
  }
}

// ---- o_proj / down_proj: residual += X W^T -----------------------------------
// Workgroup = kLrCols (4) output columns; the 4 waves split K, X is read from
// global memory by each wave for its own K range, partial sums meet in LDS. A
// wave's MFMA tile has 16 weight rows: tile row r holds column r % 4 (lanes
// 16-63 of the output repeat lanes 0-15), so a 896-column projection runs on
// 224 workgroups instead of the 56 a full tile per workgroup gives (0.5B, one
// row: 5.8 -> 5.5 us per projection; fused layer at 8 / 16 / 32 rows 860 / 970
// / 1275 -> 830 / 920 / 1180 us with the q/k/v split below). Each column is
// one wave's MFMA sum over the same k-steps either way.
constexpr int kLrCols = 4;

template <int MT>
__global__ __launch_bounds__(256) void linear_residual_kernel(const uint16_t* x, const uint16_t* w,
                                                              uint16_t* residual, int M, int N,
                                                              int K, int w_blocked) {
  __shared__ float sm_p[4][kLinMaxRows * kLrCols];
  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63, lr = l & 15, lg = l >> 4;
  const int n0 = blockIdx.x * kLrCols;
  // the residual this thread updates at the end: row tid (+256 ...), its 4 columns
  constexpr int RI = cdiv(kLinMaxRows, 256);
  u32x2 rv[RI];
#pragma unroll
  for (int it = 0; it < RI; ++it) {
    const int m = tid + 256 * it;
    if (m < M) rv[it] = *reinterpret_cast<const u32x2*>(residual + static_cast<size_t>(m) * N + n0);
  }
  const int nks = K / 32;
  const int per = cdiv(nks, 4);
  const int ks0 = min(nks, wv * per), ks1 = min(nks, ks0 + per);
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0, 0, 0, 0};
  wave_gemm_gx<MT, (MT <= 2 ? 8 : 4)>(w + mat_off(n0 + lr % kLrCols, 0, K, K, w_blocked), x, M, K,
                                      ks0, ks1, acc, lr, lg, w_blocked ? 64 : 4);
  if (lg == 0) {  // lanes holding tile rows 0-3
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      *reinterpret_cast<f32x4*>(&sm_p[wv][(mt * 16 + lr) * 4]) = acc[mt];
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < RI; ++it) {
    const int m = tid + 256 * it;
    if (m >= M) break;
    f32x4 s = *reinterpret_cast<const f32x4*>(&sm_p[0][m * 4]);
    s += *reinterpret_cast<const f32x4*>(&sm_p[1][m * 4]);
    s += *reinterpret_cast<const f32x4*>(&sm_p[2][m * 4]);
    s += *reinterpret_cast<const f32x4*>(&sm_p[3][m * 4]);
    const u32x2 r = rv[it];
    // out = residual + cast(linear), both in bf16 as the reference's residual add
    *reinterpret_cast<u32x2*>(residual + static_cast<size_t>(m) * N + n0) =
        u32x2{bf_pack(__fadd_rn(bf_lo(r[0]), rbf(s[0])), __fadd_rn(bf_hi(r[0]), rbf(s[1]))),
              bf_pack(__fadd_rn(bf_lo(r[1]), rbf(s[2])), __fadd_rn(bf_hi(r[1]), rbf(s[3])))};
  }
}

// ---- [gate|up] projection with RMSNorm and SiLU(gate) * up --------------------
// Workgroup = 32 output columns f0..f0+31 of the activation: waves 0-1 compute
// the gate columns, waves 2-3 the matching up columns (rows F + f of the fused
// weight), and the product is formed through LDS.
template <int MT, int NV>
__global__ __launch_bounds__(256) void fused_gate_up_kernel(const uint16_t* residual,
                                                            const uint16_t* norm_w, float eps,
                                                            const uint16_t* w, uint16_t* act, int M,
                                                            int H, int F, int w_blocked,
                                                            int act_blocked) {
  extern __shared__ __align__(16) uint16_t sm_lin[];
  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63, lr = l & 15, lg = l >> 4;
  const int ldx = H + 8;
  uint16_t* sx = sm_lin;                                         // [16 MT][H + 8]
  float* sy = reinterpret_cast<float*>(sm_lin + 16 * MT * ldx);  // [16 MT][64]: gate 0..31, up 32..63
  const int f0 = blockIdx.x * 32;
  const int c = (wv & 1) * 16;  // column within the 32
  const int wrow = (wv < 2 ? 0 : F) + f0 + c;
  NormStage<NV, 4 * MT> ns;
  ns.load(residual, norm_w, M, H, wv, l);
  WPrefetch<32> wpf;
  wpf.issue(w + mat_off(wrow + lr, 0, H, H, w_blocked), H / 32, lg, w_blocked ? 64 : 4);
  ns.store(eps, M, H, sx, ldx, wv, l);
  __syncthreads();
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0, 0, 0, 0};
  wpf.template run<MT>(LdsX{sx, ldx, lr, lg}, acc);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + lr;
#pragma unroll
    for (int i = 0; i < 4; ++i) sy[m * 64 + (wv < 2 ? 0 : 32) + c + 4 * lg + i] = rbf(acc[mt][i]);
  }
  __syncthreads();
  for (int idx = tid; idx < M * 16; idx += 256) {
    const int m = idx >> 4, cc = (idx & 15) * 2;
    float o[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float g = sy[m * 64 + cc + e], u = sy[m * 64 + 32 + cc + e];
      const float sg = rbf(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))));
      o[e] = __fmul_rn(sg, u);
    }
    *reinterpret_cast<uint32_t*>(act + mat_off(m, f0 + cc, F, F, act_blocked)) = bf_pack(o[0], o[1]);
  }
}

// ============================================================================
// Split-K decode layer. The kernels above give each workgroup whole output
// columns over all of K, so at 32 rows a workgroup streams its columns' whole
// weight rows and re-reads X for every few columns (0.5B at 32 rows: 1180 us
// per forward against 1023 here). Here every projection is cut into k-slices
// too, so hundreds of workgroups each read a few tens of KB:
//
//   kve_linear_splitk:   partials[s] = x[:, slice s] . W[:, slice s]^T (fp32)
//   kve_residual_norm:   residual += cast(sum_s partials[s]); xn = RMSNorm(residual)
//   kve_qkv_rope:        xn -> [q|k|v] + bias -> RoPE -> q, K/V into the pool
//   kve_gate_up_silu:    xn -> cast(silu(gate)) * up
//
// The wide layer (up to 160 rows: a verify pass over 32 sequences x 5 tokens)
// runs the QKV projection through kve_linear_splitk too, and
//   kve_qkv_part_rope:   sum_s partials[s] + bias -> RoPE -> q, K/V into the pool
// replaces kve_qkv_rope.
//
// The number of slices and their bounds depend only on the weight's shape
// (never on the row count), and every sum runs in a fixed order, so each row's
// result is the same whatever batch it is computed in.

// k-steps [a, b) of slice s out of S over nks steps (contiguous, sizes differ by <= 1)
__host__ __device__ __forceinline__ void split_range(int nks, int S, int s, int& a, int& b) {
  a = nks * s / S;
  b = nks * (s + 1) / S;
}

constexpr int kSplitMax = 16;
constexpr int kSplitMaxRows = 160;  // the 3B verify pass at 32 sequences x 5 tokens

// Slices for an [N, K] weight: 64 columns x one slice per workgroup, about 128
// workgroups below 1024 columns and 256 from there (measured best for the
// 896-wide 0.5B and 2048-wide 3B projections), at least 4 k-steps per slice,
// at most 8 slices: the reductions (kve_residual_norm, kve_qkv_part_rope) load
// 8 slices per memory round trip, and the partial sums cost 4 bytes per row
// and column per slice, written and read back.
constexpr int kSplitPick = 8;
__host__ __device__ inline int splitk_slices(int N, int K) {
  const int tiles = N / 64, nks = K / 32;
  if (tiles <= 0 || nks <= 0) return 1;
  const int wgs = N < 1024 ? 128 : 256;
  int S = (wgs + tiles / 2) / tiles;
  S = S < nks / 4 ? S : nks / 4;
  S = S < kSplitPick ? S : kSplitPick;
  return S < 1 ? 1 : S;
}

// Tiles of the split-K projection: 2 k-steps per chunk where the chunk splits
// evenly over the 4 waves (even MT), else 4. Up to 5 row tiles: LDS kept near
// 56 KB (one chunk in flight; deeper prefetch measured slower at 1-4 row
// tiles). 6-10 row tiles: three 28 KB chunk buffers (two in flight) and the
// waves as 2 x 2 (32 columns x half the rows each, 7 fragment reads per
// k-step instead of 11): the 3B down projection at 160 rows 27.8 -> 23.5 us.
constexpr int kProjLds = 56 * 1024;
// A projection tile: the DmaGemm, its thread count and the dynamic LDS of a
// launch (gate/up stages its [16 MT][BN] fp32 outputs there for the SiLU).
template <int MT_, int NW_, int WN_, int KC_, int LDS_, int NR_>
struct ProjTile {
  using G = typename DmaCfg<MT_, NW_, WN_, KC_, LDS_, NR_>::G;
  static constexpr int NT = 64 * NW_;
  static constexpr size_t STAGE = static_cast<size_t>(16) * MT_ * G::BN * 4;
  static constexpr size_t LDS = G::LDS_BYTES > STAGE ? G::LDS_BYTES : STAGE;
};
// One row tile: four chunk buffers (80 KB, still two workgroups per CU) with
// three chunks in flight: 3B down projection at 5-16 rows 13.3 -> 11.5 us
// (rows 17-64 measured no faster or slower with deeper prefetch).
// 8-10 row tiles: the same 64 columns on 8 waves as 4 x 2 (each wave one
// 16-column tile x half the rows), three 32 KB chunk buffers. With one
// workgroup per CU a chunk streams faster the more waves issue its loads
// (gfx950, 256 workgroups each streaming 1 MB of which 3/8 from HBM and the
// rest from one L2-resident 640 KB region: 36 GB/s per CU on 4 waves, 45 on
// 8, 45 on 16); 3B verify pass at 32 x 5 rows, with the 12-wave gate/up
// below: 3733 -> 3618 us (24 x 5: 3337 -> 3262). At 6 row tiles 8 waves
// measured 11 us slower per pass, so they keep 2 x 2.
template <int MT>
using SplitCfg = ProjTile<MT, (MT >= 8 ? 8 : 4), (MT == 6 ? 2 : 1), (MT % 2 == 0 ? 2 : 4),
                          (MT >= 8 ? 96 * 1024 : MT == 6 ? 84 * 1024 : MT == 1 ? 80 * 1024 : kProjLds),
                          (MT % 2 == 0 ? 2 : 1)>;

// Grid (N/BN) * S: workgroup L takes k-slice L % S of output columns
// [BN (L / S), BN (L / S + 1)) (BN = 32 at 2 and 4 row tiles: the waves split
// 2 x 2, twice the workgroups for the skinny draft projections, 0.5B forward at
// 32 rows 1068 -> 1041 us; 64 otherwise). Workgroups are dealt to the eight
// XCDs in turn (L % 8), so with S = 8 all column tiles of a slice share an XCD
// and its L2 fetches that slice of X once, where slice-major numbering had
// every XCD fetch all of X (3B down_proj at 160 rows: 3.5 MB of X read 8 times).
template <int MT, typename C = SplitCfg<MT>, bool BLK = false>
__global__ __launch_bounds__(C::NT) void linear_splitk_kernel(const uint16_t* x, const uint16_t* w,
                                                              float* part, int M, int N, int K,
                                                              int S) {
  using G = typename C::G;
  constexpr int WN = G::BN / (16 * G::NC), MTW = G::MTW;
  extern __shared__ __align__(16) uint16_t sm_lin[];
  const int s = blockIdx.x % S, n0 = (blockIdx.x / S) * G::BN;
  int a, b;
  split_range(K / 32, S, s, a, b);
  f32x4 acc[WN][MTW];
#pragma unroll
  for (int j = 0; j < WN; ++j)
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt) acc[j][mt] = f32x4{0, 0, 0, 0};
  G::template run<BLK>(w, [n0](int r) { return n0 + r; }, x, K, M, K, a, b, sm_lin, acc);
  const int l = threadIdx.x & 63, lr = l & 15, lg = l >> 4, wv = threadIdx.x >> 6;
  const int wc = wv % G::NC, wr = wv / G::NC;
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt) {
    const int m = 16 * (MTW * wr + mt) + lr;
    if (m < M) {
#pragma unroll
      for (int j = 0; j < WN; ++j)
        *reinterpret_cast<f32x4*>(part + (static_cast<size_t>(s) * M + m) * N + n0 +
                                  16 * (WN * wc + j) + 4 * lg) = acc[j][mt];
    }
  }
}

// One workgroup per row: residual = cast(residual + cast(sum_s part[s])) (the
// projection's bf16 output added to the bf16 residual), then xn =
// w * cast(r * rsqrt(mean(r^2) + eps)) as Qwen2RMSNorm. Thread t owns the
// 4-column groups t, t + 256 (H <= 2048), so each load instruction reads
// contiguous memory; the slices' loads go out eight at a time and are summed
// in order 0, 1, ..., S-1.
__global__ __launch_bounds__(256) void residual_norm_kernel(const float* part, int S,
                                                            uint16_t* residual,
                                                            const uint16_t* norm_w, float eps,
                                                            uint16_t* xn, int M, int H,
                                                            int xn_blocked) {
  constexpr int NG = 2;
  __shared__ float sm_ss[4];
  const int m = blockIdx.x;
  const int tid = threadIdx.x, l = tid & 63, wv = tid >> 6;
  const int ngr = H / 4;
  int g[NG];
  u32x2 rv[NG], wvv[NG];
  f32x4 acc[NG];
  uint16_t* rrow = residual + static_cast<size_t>(m) * H;
#pragma unroll
  for (int j = 0; j < NG; ++j) {
    g[j] = min(tid + 256 * j, ngr - 1);
    rv[j] = reinterpret_cast<const u32x2*>(rrow)[g[j]];
    wvv[j] = reinterpret_cast<const u32x2*>(norm_w)[g[j]];
  }
  for (int s0 = 0; s0 < S; s0 += 8) {
    f32x4 t[8][NG];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const f32x4* ps =
          reinterpret_cast<const f32x4*>(part + (static_cast<size_t>(min(s0 + i, S - 1)) * M + m) * H);
#pragma unroll
      for (int j = 0; j < NG; ++j) t[i][j] = ps[g[j]];
    }
    // Every loaded slice is consumed unconditionally (a slice past S keeps acc
    // by a select): with a branch here the compiler sank each slice's loads
    // into it and waited for them one slice at a time.
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool first = s0 + i == 0, live = s0 + i < S;
#pragma unroll
      for (int j = 0; j < NG; ++j) {
        const f32x4 sum = acc[j] + t[i][j];
        acc[j] = first ? t[i][j] : live ? sum : acc[j];
      }
    }
  }
  float ss = 0.0f;
  u32x2 rn[NG];
#pragma unroll
  for (int j = 0; j < NG; ++j) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float a = rbf(__fadd_rn(bf_lo(rv[j][e]), rbf(acc[j][2 * e])));
      const float b = rbf(__fadd_rn(bf_hi(rv[j][e]), rbf(acc[j][2 * e + 1])));
      rn[j][e] = bf_pack(a, b);
      if (tid + 256 * j < ngr) ss = __fadd_rn(ss, __fadd_rn(__fmul_rn(a, a), __fmul_rn(b, b)));
    }
  }
  ss = wave_sum(ss);
  if (l == 0) sm_ss[wv] = ss;
  __syncthreads();
  ss = __fadd_rn(__fadd_rn(sm_ss[0], sm_ss[1]), __fadd_rn(sm_ss[2], sm_ss[3]));
  const float inv = rsqrtf(__fadd_rn(__fmul_rn(ss, 1.0f / static_cast<float>(H)), eps));
#pragma unroll
  for (int j = 0; j < NG; ++j) {
    if (tid + 256 * j >= ngr) break;
    reinterpret_cast<u32x2*>(rrow)[g[j]] = rn[j];
    u32x2 o;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float a = rbf(__fmul_rn(bf_lo(rn[j][e]), inv));
      const float b = rbf(__fmul_rn(bf_hi(rn[j][e]), inv));
      o[e] = bf_pack(__fmul_rn(bf_lo(wvv[j][e]), a), __fmul_rn(bf_hi(wvv[j][e]), b));
    }
    *reinterpret_cast<u32x2*>(xn + mat_off(m, 4 * g[j], H, H, xn_blocked)) = o;
  }
}

// Pool slot (block * bs + offset) of every new token, -1 where nothing is
// written (token past q_len, bad row, position outside the table): resolved
// once per forward pass, shared by every layer's K/V write.
__global__ void kv_slots_kernel(const int32_t* tables, const int32_t* seq_rows,
                                const int32_t* start_pos, const int32_t* q_lens, int M, int Tq,
                                int bs, int max_blocks, int num_rows, int num_blocks,
                                int32_t* slots) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M) return;
  const int i = idx / Tq, t = idx - i * Tq;
  int slot = -1;
  const int T_i = q_lens ? min(q_lens[i], Tq) : Tq;
  if (t < T_i) {
    const int row = seq_rows ? seq_rows[i] : i;
    if (row >= 0 && row < num_rows) {
      const int pos = start_pos[row] + t;
      if (pos >= 0 && pos / bs < max_blocks) {
        const int b = tables[static_cast<size_t>(row) * max_blocks + pos / bs];
        if (b >= 0 && b < num_blocks) slot = b * bs + pos % bs;
      }
    }
  }
  slots[idx] = slot;
}

// Columns (and as many RoPE partners) per kve_qkv_rope workgroup: 4 at
// head_dim 64 (0.5B forward at 32 rows 1008 -> 984 us, at 64 rows 1149 ->
// 1101; 16 columns measured again with every load issued ahead of its
// waits: 928 -> 955 us at 32 rows, 824 -> 841 at 16), 16 at head_dim 128 (the
// 3B at one row took 2126 -> 2336 us with 4: its 2048-wide rows make the
// repeated tile rows' chunk loads cost more than the extra workgroups gain).
template <int D>
constexpr int qkv_rope_cols() { return D == 64 ? 4 : 16; }

struct QkvRopeArgs {
  const uint16_t* xn;    // [M, H], normalised
  const uint16_t* w;     // [(Hq + 2 Hkv) D, H]
  const uint16_t* bias;  // [(Hq + 2 Hkv) D]
  const uint16_t* cos;   // [M, D]
  const uint16_t* sin;   // [M, D]
  const int32_t* slots;  // [M]
  uint16_t* q_out;       // [M, Hq, D]
  uint16_t* k_pool;      // [NB, Hkv, bs, D]
  uint16_t* v_pool;      // [NB, Hkv, D, bs]
  int M, H, Hq, Hkv, bs;
};

// Grid (Hq + 2 Hkv, D / (2 NS)), 2 waves: wave 0 computes head columns
// [NS p, NS p + NS), wave 1 the RoPE partners [NS p + D/2, ...), so each
// rotation's two inputs are in one workgroup. NS = 16 fills a wave's MFMA
// tile; NS = 4 repeats the 4 columns over its 16 rows (tile row r holds column
// r % 4): the same sums on four times the workgroups.
template <int MT, int D, bool BLK = false, int NS = 16>
__global__ __launch_bounds__(128) void qkv_rope_kernel(QkvRopeArgs a) {
  static_assert(NS == 16 || NS == 4, "columns per wave");
  constexpr int half = D / 2;
  using G = typename DmaCfg<MT, 2, 1, 4>::G;
  extern __shared__ __align__(16) uint16_t sm_lin[];
  __shared__ int sm_slot[kLinMaxRows];
  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63, lr = l & 15, lg = l >> 4;
  const int hs = blockIdx.x, p = blockIdx.y;
  const bool is_q = hs < a.Hq, is_k = !is_q && hs < a.Hq + a.Hkv;
  const int base = hs * D + NS * p;  // weight row of tile row 0; tile rows 16.. are + half
  // oldest first: slots, bias and the epilogue's cos/sin (so the epilogue
  // waits for no memory), then the GEMM's own loads
  const int slot_m = a.slots[min(tid, a.M - 1)];
  const uint32_t* bb =
      reinterpret_cast<const uint32_t*>(a.bias + base + wv * half + (NS == 16 ? 4 * lg : 0));
  const uint32_t b01 = bb[0], b23 = bb[1];
  constexpr int NI = cdiv(16 * MT * NS, 128);  // epilogue items (row, column pair) per thread
  // cos/sin kept as loaded (bf16 bits) and widened in the epilogue, loaded
  // for v heads too (in bounds: row clamped to M - 1): widened here, or loaded
  // under a branch, they made the compiler wait for them before the GEMM's
  // first load
  uint16_t cs[NI][4];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int idx = tid + 128 * i;
    const int m = min(idx / NS, a.M - 1), jl = NS * p + idx % NS;
    cs[i][0] = a.cos[m * D + jl];
    cs[i][1] = a.cos[m * D + jl + half];
    cs[i][2] = a.sin[m * D + jl];
    cs[i][3] = a.sin[m * D + jl + half];
  }
  f32x4 acc2[1][MT];
  f32x4 (&acc)[MT] = acc2[0];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0, 0, 0, 0};
  G::template run<BLK>(a.w, [base](int r) {
    return base + (r < 16 ? r % NS : (r - 16) % NS + half);
  }, a.xn, a.H, a.M, a.H, 0, a.H / 32, sm_lin, acc2);
  if (tid < a.M) sm_slot[tid] = slot_m;
  float* sy = reinterpret_cast<float*>(sm_lin);  // [M][33], the GEMM buffers are free
  const float b4[4] = {bf_lo(b01), bf_hi(b01), bf_lo(b23), bf_hi(b23)};
  if (4 * lg < NS) {  // lanes holding tile rows 0..NS-1 (the rest repeat them)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + lr;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sy[m * 33 + wv * 16 + 4 * lg + i] = rbf(__fadd_rn(acc[mt][i], b4[i]));
    }
  }
  __syncthreads();
  // (row m, column j of the NS): j pairs with j + half
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int idx = tid + 128 * i;
    if (idx >= a.M * NS) break;
    const int m = idx / NS, j = idx % NS;
    const float x0 = sy[m * 33 + j], x1 = sy[m * 33 + 16 + j];
    const int jl = NS * p + j;  // column within the head (low half)
    if (is_q || is_k) {
      const float c_lo = bf16_to_f32(cs[i][0]), c_hi = bf16_to_f32(cs[i][1]);
      const float s_lo = bf16_to_f32(cs[i][2]), s_hi = bf16_to_f32(cs[i][3]);
      const float lo = rbf(__fadd_rn(rbf(__fmul_rn(x0, c_lo)), rbf(__fmul_rn(-x1, s_lo))));
      const float hi = rbf(__fadd_rn(rbf(__fmul_rn(x1, c_hi)), rbf(__fmul_rn(x0, s_hi))));
      uint16_t* dst;
      if (is_q) {
        dst = a.q_out + (static_cast<size_t>(m) * a.Hq + hs) * D;
      } else {
        const int slot = sm_slot[m];
        if (slot < 0) continue;
        const int blk = slot / a.bs, off = slot - blk * a.bs;
        dst = a.k_pool + ((static_cast<size_t>(blk) * a.Hkv + (hs - a.Hq)) * a.bs + off) * D;
      }
      dst[jl] = static_cast<uint16_t>(pack_bf16x2(lo, 0.0f));
      dst[jl + half] = static_cast<uint16_t>(pack_bf16x2(hi, 0.0f));
    } else {
      const int slot = sm_slot[m];
      if (slot < 0) continue;
      const int blk = slot / a.bs, off = slot - blk * a.bs;
      uint16_t* vb = a.v_pool + (static_cast<size_t>(blk) * a.Hkv + (hs - a.Hq - a.Hkv)) * D * a.bs + off;
      vb[static_cast<size_t>(jl) * a.bs] = static_cast<uint16_t>(pack_bf16x2(x0, 0.0f));
      vb[static_cast<size_t>(jl + half) * a.bs] = static_cast<uint16_t>(pack_bf16x2(x1, 0.0f));
    }
  }
}

struct QkvPartArgs {
  const float* part;     // [S, M, (Hq + 2 Hkv) D] k-slice partial products
  const uint16_t* bias;  // [(Hq + 2 Hkv) D]
  const uint16_t* cos;   // [M, D]
  const uint16_t* sin;   // [M, D]
  const int32_t* slots;  // [M]
  uint16_t* q_out;       // [M, Hq, D]
  uint16_t* k_pool;      // [NB, Hkv, bs, D]
  uint16_t* v_pool;      // [NB, Hkv, D, bs]
  int S, M, Hq, Hkv, bs;
};

// Epilogue of the split-K [q|k|v] projection: per row, each column's slices
// summed in order 0..S-1, + bias, rounded to bf16 (the projection's output),
// then RoPE for q and k heads (as qkv_rope_kernel) and q out / K and V into
// their pool slot. Thread: 4 columns of a head's low half and their RoPE
// partners in the high half; grid (rows, parts): a row's column groups are
// dealt 256 to a workgroup, so every thread makes one round trip for its
// partials (the 3B's 320 groups on one workgroup took two: 3B verify pass at
// 5 / 40 / 160 rows 2414 / 2735 / 3640 -> 2349 / 2677 / 3602 us).
template <int D>
__global__ __launch_bounds__(256) void qkv_part_rope_kernel(QkvPartArgs a) {
  constexpr int half = D / 2;
  constexpr int GPH = half / 4;  // 4-column groups per head half
  constexpr int SB = 8;          // slices loaded per batch
  const int m = blockIdx.x;
  const int N = (a.Hq + 2 * a.Hkv) * D;
  const int slot = a.slots[m];
  const int blk = slot >= 0 ? slot / a.bs : 0, off = slot >= 0 ? slot - blk * a.bs : 0;
  const size_t plane = static_cast<size_t>(a.M) * N;
  const int items = min((a.Hq + 2 * a.Hkv) * GPH, static_cast<int>(blockIdx.y + 1) * 256);
  for (int idx = blockIdx.y * 256 + threadIdx.x; idx < items; idx += 256) {
    const int h = idx / GPH, j = 4 * (idx - h * GPH);
    const int c_lo = h * D + j;
    const float* p_lo = a.part + static_cast<size_t>(m) * N + c_lo;
    // bias and cos/sin first, so they are in flight with the partials
    const uint32_t* bl = reinterpret_cast<const uint32_t*>(a.bias + c_lo);
    const uint32_t* bh = reinterpret_cast<const uint32_t*>(a.bias + c_lo + half);
    const uint32_t bl0 = bl[0], bl1 = bl[1], bh0 = bh[0], bh1 = bh[1];
    const bool rot = h < a.Hq + a.Hkv;
    const u32x2 c_l = rot ? *reinterpret_cast<const u32x2*>(a.cos + m * D + j) : u32x2{0, 0};
    const u32x2 c_h = rot ? *reinterpret_cast<const u32x2*>(a.cos + m * D + j + half) : u32x2{0, 0};
    const u32x2 s_l = rot ? *reinterpret_cast<const u32x2*>(a.sin + m * D + j) : u32x2{0, 0};
    const u32x2 s_h = rot ? *reinterpret_cast<const u32x2*>(a.sin + m * D + j + half) : u32x2{0, 0};
    f32x4 lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
    // A batch of SB slices, each consumed through a select (a slice past S
    // keeps the sums), and the first batch outside any loop: with a branch per
    // slice or a loop around the first batch the compiler waited for the
    // bias / cos / sin loads, or for one slice at a time, before the rest.
    auto batch = [&](int s0) {
      f32x4 vl[SB], vh[SB];
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const size_t sp = static_cast<size_t>(min(s0 + u, a.S - 1)) * plane;
        vl[u] = *reinterpret_cast<const f32x4*>(p_lo + sp);
        vh[u] = *reinterpret_cast<const f32x4*>(p_lo + sp + half);
      }
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const bool live = s0 + u < a.S;
        const f32x4 nl = lo + vl[u], nh = hi + vh[u];
        lo = live ? nl : lo;
        hi = live ? nh : hi;
      }
    };
    batch(0);
    for (int s0 = SB; s0 < a.S; s0 += SB) batch(s0);
    float x0[4] = {rbf(__fadd_rn(lo[0], bf_lo(bl0))), rbf(__fadd_rn(lo[1], bf_hi(bl0))),
                   rbf(__fadd_rn(lo[2], bf_lo(bl1))), rbf(__fadd_rn(lo[3], bf_hi(bl1)))};
    float x1[4] = {rbf(__fadd_rn(hi[0], bf_lo(bh0))), rbf(__fadd_rn(hi[1], bf_hi(bh0))),
                   rbf(__fadd_rn(hi[2], bf_lo(bh1))), rbf(__fadd_rn(hi[3], bf_hi(bh1)))};
    if (rot) {
      uint16_t* dst;
      if (h < a.Hq) {
        dst = a.q_out + (static_cast<size_t>(m) * a.Hq + h) * D;
      } else {
        if (slot < 0) continue;
        dst = a.k_pool + ((static_cast<size_t>(blk) * a.Hkv + (h - a.Hq)) * a.bs + off) * D;
      }
      const float cl[4] = {bf_lo(c_l[0]), bf_hi(c_l[0]), bf_lo(c_l[1]), bf_hi(c_l[1])};
      const float ch[4] = {bf_lo(c_h[0]), bf_hi(c_h[0]), bf_lo(c_h[1]), bf_hi(c_h[1])};
      const float sl[4] = {bf_lo(s_l[0]), bf_hi(s_l[0]), bf_lo(s_l[1]), bf_hi(s_l[1])};
      const float sh[4] = {bf_lo(s_h[0]), bf_hi(s_h[0]), bf_lo(s_h[1]), bf_hi(s_h[1])};
      float ro[4], rh[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ro[e] = rbf(__fadd_rn(rbf(__fmul_rn(x0[e], cl[e])), rbf(__fmul_rn(-x1[e], sl[e]))));
        rh[e] = rbf(__fadd_rn(rbf(__fmul_rn(x1[e], ch[e])), rbf(__fmul_rn(x0[e], sh[e]))));
      }
      *reinterpret_cast<u32x2*>(dst + j) = u32x2{pack_bf16x2(ro[0], ro[1]), pack_bf16x2(ro[2], ro[3])};
      *reinterpret_cast<u32x2*>(dst + j + half) =
          u32x2{pack_bf16x2(rh[0], rh[1]), pack_bf16x2(rh[2], rh[3])};
    } else {
      if (slot < 0) continue;
      uint16_t* vb = a.v_pool + (static_cast<size_t>(blk) * a.Hkv + (h - a.Hq - a.Hkv)) * D * a.bs + off;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vb[static_cast<size_t>(j + e) * a.bs] = static_cast<uint16_t>(pack_bf16x2(x0[e], 0.0f));
        vb[static_cast<size_t>(j + e + half) * a.bs] = static_cast<uint16_t>(pack_bf16x2(x1[e], 0.0f));
      }
    }
  }
}

// [gate|up] projection of normalised rows with SiLU(gate) * up: workgroup =
// HALF = BN / 2 activation columns f0.. (tile rows 0..HALF-1: gate rows, then
// the matching up rows F + f0..). 1-4 row tiles: 32 columns on 4 waves.
// (Workgroups of 16 + 16 columns at 2 row tiles measured slower: 0.5B forward at
// 32 rows 1045 -> 1073 us.)
template <int MT>
using GateUpCfg = ProjTile<MT, 4, 1, (MT % 2 == 0 ? 2 : 4), kProjLds, 1>;
// 6-10 row tiles of a projection whose width is not a multiple of 64: the
// waves split 2 x 2 (32 columns x half the rows each), as in the split-K
// projection (40.7 -> 39.8 us at 160 rows against 4 x 1).
template <int MT>
using GateUpCfg64 = ProjTile<MT, 4, 2, 2, kProjLds, 2>;
// 6-10 row tiles: 96 weight rows (48 gate/up column pairs) on 12 waves as 6
// column x 2 row groups (each wave one 16-row weight tile x half the rows),
// three 36 KB chunk buffers (one workgroup per CU, two chunks in flight). The
// 3B's 11008 columns make 230 workgroups (the last one 16 pairs wide). 3B
// verify pass (32 x 5 rows, 36 layers): 3811 -> 3769 us against 64 pairs on 8
// waves as 4 x 2 (172 workgroups), which in turn took gate/up at 81-96 rows
// 33 -> 27 us, 128 rows 36 -> 31 us, 160 rows 39 -> 35 us against 32 pairs on 4
// waves; four buffers, or chunks of 1 or 4 k-steps, no faster (3780-3840 us).
// 12 waves instead of 6 (3 x 2, each wave 2 weight tiles): more waves issue
// the chunk loads (as for the split-K tiles above), 32.0 -> 30.1 us per launch
// at 160 rows; 3-k-step chunks in 150 KB no faster.
template <int MT>
using GateUpCfg48 = ProjTile<MT, 12, 1, 2, 120 * 1024, 2>;
// 1-4 row tiles of a wide projection (ffn >= 8192, a multiple of 64): 48 pairs
// on 6 waves (one 16-row weight tile each), 4 k-steps per chunk, 3-4 chunk
// buffers, one workgroup per CU. The 32-pair tile makes 344 workgroups for the
// 3B's 11008 columns, two on 88 CUs, which set the pace; 230 workgroups of 48
// pairs are one per CU. 3B verify pass at 5 / 20 / 40 / 60 rows: 2455 -> 2413,
// 2600 -> 2537, 2851 -> 2740, 2927 -> 2822 us (12 waves at 2 row tiles the
// same). Narrow widths (the 0.5B's 4864) keep 32 pairs: 48 would leave 102
// workgroups.
template <int MT>
using GateUpCfgN48 = ProjTile<MT, 6, 1, 4, 128 * 1024, 1>;

template <int MT, typename C = GateUpCfg<MT>, bool BLK = false>
__global__ __launch_bounds__(C::NT) void gate_up_silu_kernel(const uint16_t* xn, const uint16_t* w,
                                                             uint16_t* act, int M, int H, int F) {
  using G = typename C::G;
  constexpr int WN = G::BN / (16 * G::NC), MTW = G::MTW;
  constexpr int HALF = G::BN / 2;  // activation columns per workgroup
  extern __shared__ __align__(16) uint16_t sm_lin[];
  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wc = wv % G::NC, wr = wv / G::NC;
  const int l = tid & 63, lr = l & 15, lg = l >> 4;
  const int f0 = blockIdx.x * HALF;
  f32x4 acc[WN][MTW];
#pragma unroll
  for (int j = 0; j < WN; ++j)
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt) acc[j][mt] = f32x4{0, 0, 0, 0};
  // columns past F (the last workgroup when HALF does not divide F) re-read
  // column F - 1 and are not stored
  G::template run<BLK>(w, [f0, F](int r) {
    return r < HALF ? min(f0 + r, F - 1) : F + min(f0 + r - HALF, F - 1);
  }, xn, H, M, H, 0, H / 32, sm_lin, acc);
  float* sy = reinterpret_cast<float*>(sm_lin);  // [16 MT][2 HALF]: gate, then up
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt) {
    const int m = (MTW * wr + mt) * 16 + lr;
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sy[m * 2 * HALF + 16 * (WN * wc + j) + 4 * lg + i] = rbf(acc[j][mt][i]);
  }
  __syncthreads();
  for (int idx = tid; idx < M * (HALF / 2); idx += C::NT) {
    const int m = idx / (HALF / 2), cc = (idx % (HALF / 2)) * 2;
    if (f0 + cc >= F) continue;
    float o[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float g = sy[m * 2 * HALF + cc + e], u = sy[m * 2 * HALF + HALF + cc + e];
      const float sg = rbf(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))));
      o[e] = __fmul_rn(sg, u);
    }
    *reinterpret_cast<uint32_t*>(act + mat_off(m, f0 + cc, F, F, BLK)) = bf_pack(o[0], o[1]);
  }
}

// ---- many-row projections with the split-K layer's sums -----------------------
// A prefill (hundreds to thousands of rows) must give every row the bits the
// split-K layer gives it in a verify pass, so that a token's K/V and hidden
// state do not depend on which pass computed them. linear_splitk_kernel
// computes, per output element, one MFMA chain per k-slice (from zero, k-steps
// in order) and its reductions add the slices in order; gate_up_silu_kernel
// runs one chain over all of K. Here a workgroup takes 128 weight rows x 128
// rows over the whole of K and keeps both sums in registers: acc is the
// current slice's chain, added to tot and restarted at every slice boundary.
// MODE 0: tot starts at -0, the additive identity, so it ends as
// t0 + t1 + ... (residual_norm_kernel's acc = t0, acc += t1, ...); MODE 1: at
// +0, as qkv_part_rope_kernel's 0 + t0 + t1 + ...; either is written as one
// fp32 slice for those reductions to finish with S = 1 (their sum 0 + tot or
// tot is tot again). MODE 2 (gate/up, one slice): tile rows interleave gate
// and up so that acc[j] and acc[j + 2] of a lane are the gate and up of the
// same column, and SiLU(gate) * up is applied as in gate_up_silu_kernel.
// The chains use the same MFMA with the same operands per lane (weight rows
// on the A side, 8 consecutive k of a k-step per lane group), so each slice
// sum is the split-K kernel's bit for bit.
template <int MT_, int NW_, int WN_, int KC_, int LDS_, int NR_>
struct RowsTile {
  using G = typename DmaCfg<MT_, NW_, WN_, KC_, LDS_, NR_>::G;
  static constexpr int NT = 64 * NW_;
};
// 16 waves (four per SIMD) as 4 column x 4 row groups, each 32 weight rows x
// 64 rows: a 128 x 256 tile, three 48 KB chunk buffers. Measured on the 3B layer
// at 5400 rows, 8 waves with 128 x 256 tiles against 4 waves with 128 x 128:
// 2.19 -> 1.24 ms; 16 waves against 8 (the same tile, more waves issuing the
// chunk loads) at 4096 rows: q/k/v 89.5 -> 80.4 us, o 52.4 -> 47.5, gate/up
// 529 -> 490, down 209 -> 195 (535 / 722 / 754 / 948 TFLOP/s); one-k-step
// chunks with five in flight measured slower on 8 and on 16 waves.
using RowsCfg = RowsTile<16, 16, 2, 2, 144 * 1024, 4>;

template <int MODE, bool SLICED, typename C, bool BLK = false>
__global__ __launch_bounds__(C::NT) void linear_rows_kernel(const uint16_t* x, const uint16_t* w,
                                                            void* out, int M, int N, int K, int S) {
  using G = typename C::G;
  constexpr int WN = G::BN / (16 * G::NC), MTW = G::MTW, BM = G::XROWS, HALF = WN / 2;
  static_assert(WN % 2 == 0, "gate and up tiles pair up");
  extern __shared__ __align__(16) uint16_t sm_lin[];
  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wc = wv % G::NC, wr = wv / G::NC;
  const int l = tid & 63, lr = l & 15, lg = l >> 4;
  const int m0 = blockIdx.y * BM;
  const int Mb = min(BM, M - m0);
  const int nks = K / 32;
  f32x4 acc[WN][MTW], tot[WN][MTW];
  const float t0 = MODE == 1 ? 0.0f : -0.0f;
#pragma unroll
  for (int j = 0; j < WN; ++j)
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt) {
      acc[j][mt] = f32x4{0, 0, 0, 0};
      tot[j][mt] = f32x4{t0, t0, t0, t0};
    }
  int s = 0, next = nks / S;  // end of slice 0 (split_range)
  auto fold = [&](int ks) {
    if (ks + 1 != next) return;
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) {
        tot[j][mt] += acc[j][mt];
        acc[j][mt] = f32x4{0, 0, 0, 0};
      }
    ++s;
    next = static_cast<int>(static_cast<int64_t>(nks) * (s + 1) / S);
  };
  const uint16_t* xb = x + static_cast<size_t>(m0) * K;  // row m0 in either layout (m0 % 16 == 0)
  if (MODE == 2) {
    const int f0 = blockIdx.x * (G::BN / 2), F = N;
    G::template run<BLK>(w,
           [f0, F](int r) {
             const int t = r >> 4, j = t % WN;
             const int c = f0 + 16 * (HALF * (t / WN) + j % HALF) + (r & 15);
             return j < HALF ? c : F + c;
           },
           xb, K, Mb, K, 0, nks, sm_lin, acc, fold);
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt) {
      const int m = 16 * (MTW * wr + mt) + lr;
      if (m >= Mb) continue;
#pragma unroll
      for (int j = 0; j < HALF; ++j) {
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float g = rbf(tot[j][mt][i]), u = rbf(tot[j + HALF][mt][i]);
          const float sg = rbf(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))));
          o[i] = __fmul_rn(sg, u);
        }
        const int c = f0 + 16 * (HALF * wc + j) + 4 * lg;
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(out) + mat_off(m0 + m, c, F, F, BLK)) =
            u32x2{bf_pack(o[0], o[1]), bf_pack(o[2], o[3])};
      }
    }
  } else if (SLICED) {
    // one slice per workgroup (blockIdx.z), written as linear_splitk_kernel writes it
    const int n0 = blockIdx.x * G::BN, sl = blockIdx.z;
    int a, b;
    split_range(nks, S, sl, a, b);
    G::template run<BLK>(w, [n0](int r) { return n0 + r; }, xb, K, Mb, K, a, b, sm_lin, acc);
    float* part = static_cast<float*>(out) + static_cast<size_t>(sl) * M * N;
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt) {
      const int m = 16 * (MTW * wr + mt) + lr;
      if (m >= Mb) continue;
#pragma unroll
      for (int j = 0; j < WN; ++j)
        *reinterpret_cast<f32x4*>(part + static_cast<size_t>(m0 + m) * N + n0 + 16 * (WN * wc + j) +
                                  4 * lg) = acc[j][mt];
    }
  } else {
    const int n0 = blockIdx.x * G::BN;
    G::template run<BLK>(w, [n0](int r) { return n0 + r; }, xb, K, Mb, K, 0, nks, sm_lin, acc, fold);
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt) {
      const int m = 16 * (MTW * wr + mt) + lr;
      if (m >= Mb) continue;
#pragma unroll
      for (int j = 0; j < WN; ++j)
        *reinterpret_cast<f32x4*>(static_cast<float*>(out) + static_cast<size_t>(m0 + m) * N + n0 +
                                  16 * (WN * wc + j) + 4 * lg) = tot[j][mt];
    }
  }
}


static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <typename K>
static int allow_lds(K kernel, size_t bytes) {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                             hipFuncAttributeMaxDynamicSharedMemorySize,
                             static_cast<int>(bytes)) == hipSuccess
             ? 0
             : -1;
}

// Launch `kernel` with `lds` bytes of dynamic LDS, raising the kernel's limit
// the first time (per instantiation: `granted` is a static of the caller).
template <typename K, typename... Args>
static int launch_lds(K kernel, size_t& granted, dim3 grid, dim3 block, size_t lds, hipStream_t st,
                      Args... args) {
  if (lds > granted) {
    if (allow_lds(kernel, lds)) {
      set_error("%zu bytes of LDS refused", lds);
      return KVE_ELAUNCH;
    }
    granted = lds;
  }
  hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
  return KVE_OK;
}

}  // namespace kve

using namespace kve;

extern "C" int kve_fused_qkv(const void* residual, const void* norm_weight, float eps,
                             const void* weight, const void* bias, const void* cos,
                             const void* sin, void* q_out, void* k_pool, void* v_pool,
                             const int32_t* block_tables, const int32_t* seq_rows,
                             const int32_t* start_pos, const int32_t* q_lens, int num_seqs,
                             int q_len, int hidden, int num_q_heads, int num_kv_heads,
                             int head_dim, int block_size, int max_blocks, int num_rows,
                             int num_blocks, int layout, void* stream) {
  clear_error();
  if (num_seqs == 0) return KVE_OK;
  const int M = num_seqs * q_len;
  KVE_REQUIRE(residual && norm_weight && weight && bias && cos && sin && q_out && k_pool && v_pool &&
                  block_tables && start_pos,
              "kve_fused_qkv: null pointer argument");
  KVE_REQUIRE(num_seqs > 0 && q_len > 0 && M <= kLinMaxRows, "kve_fused_qkv: %d rows (max %d)", M,
              kLinMaxRows);
  KVE_REQUIRE(head_dim == 64 || head_dim == 128, "kve_fused_qkv: head_dim %d", head_dim);
  KVE_REQUIRE(hidden % 32 == 0 && hidden <= 2048, "kve_fused_qkv: hidden %d (multiple of 32, <= 2048)",
              hidden);
  KVE_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && block_size > 0 && max_blocks > 0 &&
                  num_rows > 0 && num_blocks > 0,
              "kve_fused_qkv: bad sizes");
  KVE_REQUIRE(aligned16(residual) && aligned16(norm_weight) && aligned16(weight) && aligned16(bias),
              "kve_fused_qkv: buffers must be 16-byte aligned");
  KVE_REQUIRE(layout == KVE_LAYOUT_ROWS || layout == KVE_LAYOUT_BLOCKED, "kve_fused_qkv: layout %d",
              layout);
  QkvArgs a;
  a.w_blocked = layout == KVE_LAYOUT_BLOCKED ? 1 : 0;
  a.residual = static_cast<const uint16_t*>(residual);
  a.norm_w = static_cast<const uint16_t*>(norm_weight);
  a.w = static_cast<const uint16_t*>(weight);
  a.bias = static_cast<const uint16_t*>(bias);
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.q_out = static_cast<uint16_t*>(q_out);
  a.k_pool = static_cast<uint16_t*>(k_pool);
  a.v_pool = static_cast<uint16_t*>(v_pool);
  a.tables = block_tables;
  a.seq_rows = seq_rows;
  a.start_pos = start_pos;
  a.q_lens = q_lens;
  a.M = M;
  a.Tq = q_len;
  a.H = hidden;
  a.Hq = num_q_heads;
  a.Hkv = num_kv_heads;
  a.bs = block_size;
  a.max_blocks = max_blocks;
  a.num_rows = num_rows;
  a.num_blocks = num_blocks;
  a.eps = eps;
  const int MT = cdiv(M, 16);
  const size_t lds = static_cast<size_t>(16 * MT) * (hidden + 8) * 2 +
                     static_cast<size_t>(16 * MT) * (head_dim + 1) * 4 +
                     static_cast<size_t>(M) * head_dim * 2 * 2;
  KVE_REQUIRE(aligned16(cos) && aligned16(sin), "kve_fused_qkv: cos/sin must be 16-byte aligned");
  KVE_REQUIRE(lds <= kLinMaxLds, "kve_fused_qkv: %d rows x hidden %d need %zu bytes of LDS (max %zu)",
              M, hidden, lds, kLinMaxLds);
  const dim3 grid((num_q_heads + 2 * num_kv_heads) * kQkvSplit);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int NV = cdiv(hidden / 8, 64);
#define KVE_QKV(MT_, D_, NV_)                                                              \
  do {                                                                                     \
    auto k_ = fused_qkv_kernel<MT_, D_, NV_>;          \
    static size_t granted_ = 0; /* dynamic LDS this instantiation may use */ \
    if (lds > granted_) {                                                     \
      if (allow_lds(k_, lds)) {                                               \
        set_error("%s: %zu bytes of LDS refused", __func__, lds);            \
        return KVE_ELAUNCH;                                                   \
      }                                                                       \
      granted_ = lds;                                                         \
    }                                                                         \
    hipLaunchKernelGGL(k_, grid, dim3(256), lds, st, a);                                   \
  } while (0)
#define KVE_QKV_D(MT_, NV_)           \
  if (head_dim == 64) KVE_QKV(MT_, 64, NV_); \
  else KVE_QKV(MT_, 128, NV_)
#define KVE_QKV_NV(MT_)                       \
  if (NV <= 2) { KVE_QKV_D(MT_, 2); }         \
  else { KVE_QKV_D(MT_, 4); }
  if (MT == 1) { KVE_QKV_NV(1) }
  else if (MT == 2) { KVE_QKV_NV(2) }
  else if (MT == 3) { KVE_QKV_NV(3) }
  else { KVE_QKV_NV(4) }
#undef KVE_QKV_NV
#undef KVE_QKV_D
#undef KVE_QKV
  return check_launch("kve_fused_qkv");
}

extern "C" int kve_linear_residual(const void* x, const void* weight, void* residual, int rows,
                                   int out_features, int in_features, int layout, void* stream) {
  clear_error();
  if (rows == 0) return KVE_OK;
  KVE_REQUIRE(x && weight && residual, "kve_linear_residual: null pointer argument");
  KVE_REQUIRE(rows > 0 && rows <= kLinMaxRows, "kve_linear_residual: %d rows (max %d)", rows,
              kLinMaxRows);
  KVE_REQUIRE(out_features > 0 && out_features % 16 == 0 && in_features > 0 && in_features % 32 == 0,
              "kve_linear_residual: %d x %d (multiples of 16 and 32)", out_features, in_features);
  KVE_REQUIRE(aligned16(x) && aligned16(weight) && aligned16(residual),
              "kve_linear_residual: buffers must be 16-byte aligned");
  KVE_REQUIRE(layout == KVE_LAYOUT_ROWS || layout == KVE_LAYOUT_BLOCKED,
              "kve_linear_residual: layout %d", layout);
  const int wb = layout == KVE_LAYOUT_BLOCKED ? 1 : 0;
  const dim3 grid(out_features / kLrCols);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* wp = static_cast<const uint16_t*>(weight);
  uint16_t* rp = static_cast<uint16_t*>(residual);
  switch (cdiv(rows, 16)) {
    case 1: hipLaunchKernelGGL(linear_residual_kernel<1>, grid, dim3(256), 0, st, xp, wp, rp, rows, out_features, in_features, wb); break;
    case 2: hipLaunchKernelGGL(linear_residual_kernel<2>, grid, dim3(256), 0, st, xp, wp, rp, rows, out_features, in_features, wb); break;
    case 3: hipLaunchKernelGGL(linear_residual_kernel<3>, grid, dim3(256), 0, st, xp, wp, rp, rows, out_features, in_features, wb); break;
    default: hipLaunchKernelGGL(linear_residual_kernel<4>, grid, dim3(256), 0, st, xp, wp, rp, rows, out_features, in_features, wb); break;
  }
  return check_launch("kve_linear_residual");
}

extern "C" int kve_fused_gate_up(const void* residual, const void* norm_weight, float eps,
                                 const void* weight, void* act, int rows, int hidden, int ffn,
                                 int layout, int act_layout, void* stream) {
  clear_error();
  if (rows == 0) return KVE_OK;
  KVE_REQUIRE(residual && norm_weight && weight && act, "kve_fused_gate_up: null pointer argument");
  KVE_REQUIRE(layout == KVE_LAYOUT_ROWS || layout == KVE_LAYOUT_BLOCKED, "kve_fused_gate_up: layout %d",
              layout);
  KVE_REQUIRE(act_layout == KVE_LAYOUT_ROWS || act_layout == KVE_LAYOUT_BLOCKED,
              "kve_fused_gate_up: act_layout %d", act_layout);
  const int wb = layout == KVE_LAYOUT_BLOCKED ? 1 : 0;
  const int ab = act_layout == KVE_LAYOUT_BLOCKED ? 1 : 0;
  KVE_REQUIRE(rows > 0 && rows <= kLinMaxRows, "kve_fused_gate_up: %d rows (max %d)", rows,
              kLinMaxRows);
  KVE_REQUIRE(hidden % 32 == 0 && hidden <= 2048 && ffn % 32 == 0,
              "kve_fused_gate_up: hidden %d ffn %d", hidden, ffn);
  KVE_REQUIRE(aligned16(residual) && aligned16(norm_weight) && aligned16(weight) && aligned16(act),
              "kve_fused_gate_up: buffers must be 16-byte aligned");
  const int MT = cdiv(rows, 16);
  const size_t lds = static_cast<size_t>(16 * MT) * (hidden + 8) * 2 +
                     static_cast<size_t>(16 * MT) * 64 * 4;
  KVE_REQUIRE(lds <= kLinMaxLds, "kve_fused_gate_up: %d rows x hidden %d need %zu bytes of LDS (max %zu)",
              rows, hidden, lds, kLinMaxLds);
  const dim3 grid(ffn / 32);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int NV = cdiv(hidden / 8, 64);
  const uint16_t* rp = static_cast<const uint16_t*>(residual);
  const uint16_t* np = static_cast<const uint16_t*>(norm_weight);
  const uint16_t* wp = static_cast<const uint16_t*>(weight);
  uint16_t* ap = static_cast<uint16_t*>(act);
#define KVE_GU(MT_, NV_)                                                                  \
  do {                                                                                    \
    auto k_ = fused_gate_up_kernel<MT_, NV_>;          \
    static size_t granted_ = 0; /* dynamic LDS this instantiation may use */ \
    if (lds > granted_) {                                                     \
      if (allow_lds(k_, lds)) {                                               \
        set_error("%s: %zu bytes of LDS refused", __func__, lds);            \
        return KVE_ELAUNCH;                                                   \
      }                                                                       \
      granted_ = lds;                                                         \
    }                                                                         \
    hipLaunchKernelGGL(k_, grid, dim3(256), lds, st, rp, np, eps, wp, ap, rows, hidden, ffn, wb, \
                       ab);                                                               \
  } while (0)
#define KVE_GU_NV(MT_)              \
  if (NV <= 2) KVE_GU(MT_, 2);      \
  else KVE_GU(MT_, 4)
  if (MT == 1) { KVE_GU_NV(1); }
  else if (MT == 2) { KVE_GU_NV(2); }
  else if (MT == 3) { KVE_GU_NV(3); }
  else { KVE_GU_NV(4); }
#undef KVE_GU_NV
#undef KVE_GU
  return check_launch("kve_fused_gate_up");
}

// ---- split-K decode layer entry points ----------------------------------------

extern "C" int kve_splitk_slices(int out_features, int in_features) {
  if (out_features <= 0 || in_features <= 0) return 0;
  return splitk_slices(out_features, in_features);
}

extern "C" int kve_linear_splitk(const void* x, const void* weight, float* partials, int rows,
                                 int out_features, int in_features, int slices, int layout,
                                 void* stream) {
  clear_error();
  if (rows == 0) return KVE_OK;
  KVE_REQUIRE(x && weight && partials, "kve_linear_splitk: null pointer argument");
  KVE_REQUIRE(rows > 0 && rows <= kSplitMaxRows, "kve_linear_splitk: %d rows (max %d)", rows,
              kSplitMaxRows);
  KVE_REQUIRE(out_features > 0 && out_features % 64 == 0 && in_features > 0 && in_features % 32 == 0,
              "kve_linear_splitk: out %d (multiple of 64) in %d (multiple of 32)", out_features,
              in_features);
  KVE_REQUIRE(slices == splitk_slices(out_features, in_features),
              "kve_linear_splitk: %d slices, the [%d, %d] weight takes %d", slices, out_features,
              in_features, splitk_slices(out_features, in_features));
  KVE_REQUIRE(aligned16(x) && aligned16(weight) && aligned16(partials),
              "kve_linear_splitk: buffers must be 16-byte aligned");
  KVE_REQUIRE(layout == KVE_LAYOUT_ROWS || layout == KVE_LAYOUT_BLOCKED,
              "kve_linear_splitk: layout %d", layout);
  const bool blk = layout == KVE_LAYOUT_BLOCKED;
  dim3 grid(1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* wp = static_cast<const uint16_t*>(weight);
  int rc = KVE_OK;
#define KVE_SKC(MT_, C_)                                                                           \
  do {                                                                                             \
    static size_t granted_ = 0;                                                                    \
    grid.x = out_features / C_::G::BN * slices;                                                    \
    static size_t granted_b_ = 0;                                                                  \
    if (blk)                                                                                       \
      rc = launch_lds(linear_splitk_kernel<MT_, C_, true>, granted_b_, grid, dim3(C_::NT), C_::LDS, \
                      st, xp, wp, partials, rows, out_features, in_features, slices);              \
    else                                                                                           \
      rc = launch_lds(linear_splitk_kernel<MT_, C_>, granted_, grid, dim3(C_::NT), C_::LDS, st, xp, \
                      wp, partials, rows, out_features, in_features, slices);                      \
  } while (0)
#define KVE_SK(MT_) KVE_SKC(MT_, SplitCfg<MT_>)
  switch (cdiv(rows, 16)) {
    case 1: KVE_SK(1); break;
    case 2: KVE_SK(2); break;
    case 3: KVE_SK(3); break;
    case 4: KVE_SK(4); break;
    case 5:
    case 6: KVE_SK(6); break;
    case 7:
    case 8: KVE_SK(8); break;
    default: KVE_SK(10); break;
  }
#undef KVE_SK
#undef KVE_SKC
  if (rc) return rc;
  return check_launch("kve_linear_splitk");
}

extern "C" int kve_residual_norm(const float* partials, int slices, void* residual,
                                 const void* norm_weight, float eps, void* xn, int rows, int hidden,
                                 int layout, void* stream) {
  clear_error();
  if (rows == 0) return KVE_OK;
  KVE_REQUIRE(partials && residual && norm_weight && xn, "kve_residual_norm: null pointer argument");
  KVE_REQUIRE(rows > 0 && slices >= 1 && slices <= kSplitMax, "kve_residual_norm: rows %d slices %d",
              rows, slices);
  KVE_REQUIRE(hidden > 0 && hidden % 4 == 0 && hidden <= 2048,
              "kve_residual_norm: hidden %d (multiple of 4, at most 2048)", hidden);
  KVE_REQUIRE(aligned16(partials) && aligned16(residual) && aligned16(norm_weight) && aligned16(xn),
              "kve_residual_norm: buffers must be 16-byte aligned");
  KVE_REQUIRE(layout == KVE_LAYOUT_ROWS || (layout == KVE_LAYOUT_BLOCKED && hidden % 32 == 0),
              "kve_residual_norm: layout %d with hidden %d", layout, hidden);
  hipLaunchKernelGGL(residual_norm_kernel, dim3(rows), dim3(256), 0, static_cast<hipStream_t>(stream),
                     partials, slices, static_cast<uint16_t*>(residual),
                     static_cast<const uint16_t*>(norm_weight), eps, static_cast<uint16_t*>(xn), rows,
                     hidden, layout == KVE_LAYOUT_BLOCKED ? 1 : 0);
  return check_launch("kve_residual_norm");
}

extern "C" int kve_kv_slots(const int32_t* block_tables, const int32_t* seq_rows,
                            const int32_t* start_pos, const int32_t* q_lens, int num_seqs,
                            int q_len, int block_size, int max_blocks, int num_rows,
                            int num_blocks, int32_t* slots, void* stream) {
  clear_error();
  if (num_seqs == 0) return KVE_OK;
  KVE_REQUIRE(block_tables && start_pos && slots, "kve_kv_slots: null pointer argument");
  KVE_REQUIRE(num_seqs > 0 && q_len > 0 && block_size > 0 && max_blocks > 0 && num_rows > 0 &&
                  num_blocks > 0,
              "kve_kv_slots: bad sizes");
  const int M = num_seqs * q_len;
  hipLaunchKernelGGL(kv_slots_kernel, dim3(cdiv(M, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), block_tables, seq_rows, start_pos, q_lens, M,
                     q_len, block_size, max_blocks, num_rows, num_blocks, slots);
  return check_launch("kve_kv_slots");
}

extern "C" int kve_qkv_rope(const void* xn, const void* weight, const void* bias, const void* cos,
                            const void* sin, const int32_t* slots, void* q_out, void* k_pool,
                            void* v_pool, int rows, int hidden, int num_q_heads, int num_kv_heads,
                            int head_dim, int block_size, int layout, void* stream) {
  clear_error();
  if (rows == 0) return KVE_OK;
  KVE_REQUIRE(xn && weight && bias && cos && sin && slots && q_out && k_pool && v_pool,
              "kve_qkv_rope: null pointer argument");
  KVE_REQUIRE(rows > 0 && rows <= kLinMaxRows, "kve_qkv_rope: %d rows (max %d)", rows, kLinMaxRows);
  KVE_REQUIRE(head_dim == 64 || head_dim == 128, "kve_qkv_rope: head_dim %d", head_dim);
  KVE_REQUIRE(hidden > 0 && hidden % 32 == 0, "kve_qkv_rope: hidden %d (multiple of 32)", hidden);
  KVE_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && block_size > 0, "kve_qkv_rope: bad sizes");
  KVE_REQUIRE(aligned16(xn) && aligned16(weight) && aligned16(bias),
              "kve_qkv_rope: xn, weight and bias must be 16-byte aligned");
  KVE_REQUIRE(layout == KVE_LAYOUT_ROWS || layout == KVE_LAYOUT_BLOCKED, "kve_qkv_rope: layout %d",
              layout);
  const bool blk = layout == KVE_LAYOUT_BLOCKED;
  QkvRopeArgs a;
  a.xn = static_cast<const uint16_t*>(xn);
  a.w = static_cast<const uint16_t*>(weight);
  a.bias = static_cast<const uint16_t*>(bias);
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.slots = slots;
  a.q_out = static_cast<uint16_t*>(q_out);
  a.k_pool = static_cast<uint16_t*>(k_pool);
  a.v_pool = static_cast<uint16_t*>(v_pool);
  a.M = rows;
  a.H = hidden;
  a.Hq = num_q_heads;
  a.Hkv = num_kv_heads;
  a.bs = block_size;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int rc = KVE_OK;
#define KVE_QR1(MT_, D_)                                                                    \
  do {                                                                                      \
    static size_t granted_ = 0, granted_b_ = 0;                                             \
    constexpr int NS_ = qkv_rope_cols<D_>();                                                \
    const dim3 grid(num_q_heads + 2 * num_kv_heads, D_ / (2 * NS_));                        \
    if (blk)                                                                                \
      rc = launch_lds(qkv_rope_kernel<MT_, D_, true, NS_>, granted_b_, grid, dim3(128),     \
                      DmaCfg<MT_, 2, 1, 4>::G::LDS_BYTES, st, a);                           \
    else                                                                                    \
      rc = launch_lds(qkv_rope_kernel<MT_, D_, false, NS_>, granted_, grid, dim3(128),      \
                      DmaCfg<MT_, 2, 1, 4>::G::LDS_BYTES, st, a);                           \
  } while (0)
#define KVE_QR(MT_)                  \
  if (head_dim == 64) KVE_QR1(MT_, 64); \
  else KVE_QR1(MT_, 128)
  switch (cdiv(rows, 16)) {
    case 1: KVE_QR(1); break;
    case 2: KVE_QR(2); break;
    case 3: KVE_QR(3); break;
    default: KVE_QR(4); break;
  }
#undef KVE_QR
#undef KVE_QR1
  if (rc) return rc;
  return check_launch("kve_qkv_rope");
}

extern "C" int kve_qkv_part_rope(const float* partials, int slices, const void* bias,
                                 const void* cos, const void* sin, const int32_t* slots,
                                 void* q_out, void* k_pool, void* v_pool, int rows,
                                 int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                 void* stream) {
  clear_error();
  if (rows == 0) return KVE_OK;
  KVE_REQUIRE(partials && bias && cos && sin && slots && q_out && k_pool && v_pool,
              "kve_qkv_part_rope: null pointer argument");
  KVE_REQUIRE(rows > 0 && slices >= 1 && slices <= kSplitMax, "kve_qkv_part_rope: rows %d slices %d",
              rows, slices);
  KVE_REQUIRE(head_dim == 64 || head_dim == 128, "kve_qkv_part_rope: head_dim %d", head_dim);
  KVE_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && block_size > 0, "kve_qkv_part_rope: bad sizes");
  KVE_REQUIRE(aligned16(partials) && aligned16(bias) && aligned16(q_out),
              "kve_qkv_part_rope: partials, bias and q_out must be 16-byte aligned");
  KVE_REQUIRE(((reinterpret_cast<uintptr_t>(cos) | reinterpret_cast<uintptr_t>(sin)) & 7) == 0,
              "kve_qkv_part_rope: cos and sin must be 8-byte aligned");
  QkvPartArgs a;
  a.part = partials;
  a.bias = static_cast<const uint16_t*>(bias);
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.slots = slots;
  a.q_out = static_cast<uint16_t*>(q_out);
  a.k_pool = static_cast<uint16_t*>(k_pool);
  a.v_pool = static_cast<uint16_t*>(v_pool);
  a.S = slices;
  a.M = rows;
  a.Hq = num_q_heads;
  a.Hkv = num_kv_heads;
  a.bs = block_size;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(rows, cdiv((num_q_heads + 2 * num_kv_heads) * (head_dim / 8), 256));
  if (head_dim == 64) hipLaunchKernelGGL(qkv_part_rope_kernel<64>, grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL(qkv_part_rope_kernel<128>, grid, dim3(256), 0, st, a);
  return check_launch("kve_qkv_part_rope");
}

extern "C" int kve_gate_up_silu(const void* xn, const void* weight, void* act, int rows, int hidden,
                                int ffn, int layout, void* stream) {
  clear_error();
  if (rows == 0) return KVE_OK;
  KVE_REQUIRE(xn && weight && act, "kve_gate_up_silu: null pointer argument");
  KVE_REQUIRE(rows > 0 && rows <= kSplitMaxRows, "kve_gate_up_silu: %d rows (max %d)", rows,
              kSplitMaxRows);
  KVE_REQUIRE(hidden % 32 == 0 && hidden > 0 && ffn % 32 == 0 && ffn > 0,
              "kve_gate_up_silu: hidden %d ffn %d", hidden, ffn);
  KVE_REQUIRE(aligned16(xn) && aligned16(weight) && aligned16(act),
              "kve_gate_up_silu: buffers must be 16-byte aligned");
  KVE_REQUIRE(layout == KVE_LAYOUT_ROWS || layout == KVE_LAYOUT_BLOCKED,
              "kve_gate_up_silu: layout %d", layout);
  const bool blk = layout == KVE_LAYOUT_BLOCKED;
  dim3 grid(ffn / 32);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* xp = static_cast<const uint16_t*>(xn);
  const uint16_t* wp = static_cast<const uint16_t*>(weight);
  uint16_t* ap = static_cast<uint16_t*>(act);
  int rc = KVE_OK;
#define KVE_GUSC(MT_, C_)                                                                    \
  do {                                                                                      \
    static size_t granted_ = 0, granted_b_ = 0;                                             \
    grid.x = cdiv(ffn, C_::G::BN / 2);                                                      \
    if (blk)                                                                                \
      rc = launch_lds(gate_up_silu_kernel<MT_, C_, true>, granted_b_, grid, dim3(C_::NT),   \
                      C_::LDS, st, xp, wp, ap, rows, hidden, ffn);                          \
    else                                                                                    \
      rc = launch_lds(gate_up_silu_kernel<MT_, C_>, granted_, grid, dim3(C_::NT), C_::LDS,  \
                      st, xp, wp, ap, rows, hidden, ffn);                                   \
  } while (0)
#define KVE_GUS(MT_)                                                  \
  if (ffn >= 8192 && ffn % 64 == 0) KVE_GUSC(MT_, GateUpCfgN48<MT_>); \
  else KVE_GUSC(MT_, GateUpCfg<MT_>)
  // 6-10 row tiles: 48 column pairs per workgroup where the width is a
  // multiple of 64; other widths keep 64-row tiles of 4 waves (the same sums)
#define KVE_GUS_WIDE(MT_)                                        \
  if (ffn % 64 == 0) KVE_GUSC(MT_, GateUpCfg48<MT_>);            \
  else KVE_GUSC(MT_, GateUpCfg64<MT_>)
  switch (cdiv(rows, 16)) {
    case 1: KVE_GUS(1); break;
    case 2: KVE_GUS(2); break;
    case 3: KVE_GUS(3); break;
    case 4: KVE_GUS(4); break;
    case 5:
    case 6: KVE_GUS_WIDE(6); break;
    case 7:
    case 8: KVE_GUS_WIDE(8); break;
    default: KVE_GUS_WIDE(10); break;
  }
#undef KVE_GUS_WIDE
#undef KVE_GUS
#undef KVE_GUSC
  if (rc) return rc;
  return check_launch("kve_gate_up_silu");
}

// Compute units of the current device (cached per device).
static int resident_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// Slices kve_linear_rows writes: the whole sum (1) when the output tiles alone
// give the chip a workgroup per CU, else every k-slice (the reductions then sum
// them, as after kve_linear_splitk). Gate/up always writes its activation.
static int rows_slices(int rows, int N, int K, int mode) {
  if (mode == 2) return 1;
  const int tiles = (N / RowsCfg::G::BN) * cdiv(rows, RowsCfg::G::XROWS);
  return tiles >= resident_cus() ? 1 : splitk_slices(N, K);
}

extern "C" int kve_linear_rows_slices(int rows, int out_features, int in_features, int mode) {
  if (rows <= 0 || out_features <= 0 || in_features <= 0 || mode < 0 || mode > 2) return 0;
  return rows_slices(rows, out_features, in_features, mode);
}

extern "C" int kve_linear_rows(const void* x, const void* weight, void* out, int rows,
                               int out_features, int in_features, int mode, int layout,
                               void* stream) {
  clear_error();
  if (rows == 0) return KVE_OK;
  KVE_REQUIRE(x && weight && out, "kve_linear_rows: null pointer argument");
  KVE_REQUIRE(rows > 0 && mode >= 0 && mode <= 2, "kve_linear_rows: rows %d mode %d", rows, mode);
  KVE_REQUIRE(in_features > 0 && in_features % 64 == 0,
              "kve_linear_rows: in %d (multiple of 64)", in_features);
  using C = RowsCfg;
  const int unit = C::G::BN;
  KVE_REQUIRE(out_features > 0 && out_features % unit == 0,
              "kve_linear_rows: out %d (multiple of %d)", out_features, unit);
  KVE_REQUIRE(aligned16(x) && aligned16(weight) && aligned16(out),
              "kve_linear_rows: buffers must be 16-byte aligned");
  KVE_REQUIRE(layout == KVE_LAYOUT_ROWS || layout == KVE_LAYOUT_BLOCKED, "kve_linear_rows: layout %d",
              layout);
  const bool blk = layout == KVE_LAYOUT_BLOCKED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* wp = static_cast<const uint16_t*>(weight);
  const int F = out_features / 2;
  const int S = mode == 2 ? 1 : splitk_slices(out_features, in_features);
  const bool sliced = rows_slices(rows, out_features, in_features, mode) > 1;
  dim3 grid(mode == 2 ? F / (C::G::BN / 2) : out_features / C::G::BN, cdiv(rows, C::G::XROWS),
            sliced ? S : 1);
  const size_t lds = C::G::LDS_BYTES;
  int rc;
#define KVE_ROWS(MODE_, SL_, N_)                                                                \
  do {                                                                                         \
    static size_t granted_ = 0, granted_b_ = 0;                                                \
    if (blk)                                                                                   \
      rc = launch_lds(linear_rows_kernel<MODE_, SL_, C, true>, granted_b_, grid, dim3(C::NT), lds, \
                      st, xp, wp, out, rows, N_, in_features, S);                              \
    else                                                                                       \
      rc = launch_lds(linear_rows_kernel<MODE_, SL_, C>, granted_, grid, dim3(C::NT), lds, st, xp, \
                      wp, out, rows, N_, in_features, S);                                      \
  } while (0)
  if (mode == 2) KVE_ROWS(2, false, F);
  else if (mode == 1 && sliced) KVE_ROWS(1, true, out_features);
  else if (mode == 1) KVE_ROWS(1, false, out_features);
  else if (sliced) KVE_ROWS(0, true, out_features);
  else KVE_ROWS(0, false, out_features);
#undef KVE_ROWS
  if (rc) return rc;
  return check_launch("kve_linear_rows");
}
