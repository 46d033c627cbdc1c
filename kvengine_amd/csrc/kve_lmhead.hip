// LM head with fused row argmax for CDNA4 (gfx950).
//
// logits[m, v] = hidden[m, :] . E[v, :] over the tied embedding E [V, H], then
// for each row m the first index of the maximum of the logits rounded to the
// model dtype. This replaces model.lm_head(hidden) followed by torch.argmax
// (kvengine/forward.py:215, speculative.py:155,167): the reference materialises
// [rows, 151936] logits and scans them again; here the logits never leave
// registers.
//
// Each workgroup streams a slab of 64*WV embedding rows once from HBM (wave w
// owns WV 16-row tiles) against all M hidden rows (MT 16-row tiles at a time).
// Logit tiles come out of MFMA with the vocabulary on the M side, so each lane
// holds 4 vocabulary ids of one hidden row; (value, index) pairs are packed
// into one 64-bit key (order-preserving float bits, then the complemented
// index) so a plain integer max picks the largest logit and, among equal
// rounded logits, the lowest id. Workgroup maxima go to a 64-bit atomicMax on
// one of kKeySlots copies of the row's key (workgroup g uses copy g mod
// kKeySlots; with a single copy the ~2400 workgroups' atomics on the same few
// addresses queue in one L2 channel: 0.5B LM head at 32 rows 68 -> 58 us); a
// second small kernel (one wave per row) takes the max of the copies and
// clears them, so the workspace is zero again for the next launch.
//
// Runner-up (TOP2, when the caller asks for it): every lane, wave and
// workgroup keeps the two largest keys of what it saw. A workgroup's pair
// (a, b) enters a copy (k1, k2) as old = atomicMax(k1, a), then
// atomicMax(k2, max(min(old, a), b)): whatever k1 does not keep (the smaller
// of old and a) and b both reach k2, so k2 ends as the largest key other than
// k1's whatever the order of the atomics. The finalize merges the copies'
// pairs the same way.

#include "kve_common.h"
#include "kve_gemm.h"

#include <mutex>
#include <type_traits>

namespace kve {

constexpr int kKeySlots = 64;  // one per lane of the finalize wave

// A workgroup's (a, b) into key copy (k1, k2); see the header comment.
__device__ __forceinline__ void publish_top2(unsigned long long* k1, unsigned long long* k2,
                                             uint64_t a, uint64_t b) {
  const uint64_t old = atomicMax(k1, static_cast<unsigned long long>(a));
  const uint64_t lose = old < a ? old : a;
  atomicMax(k2, static_cast<unsigned long long>(umax64(lose, b)));
}

template <bool BF16, int WV, int MT, bool TOP2>
__global__ __launch_bounds__(256) void lmhead_argmax_kernel(
    const void* hidden, int64_t hstride, const void* weight, int M, int H, int V,
    unsigned long long* keys) {
  using elem_t = std::conditional_t<BF16, uint16_t, float>;
  constexpr int KSTEP = BF16 ? 32 : 16;  // channels consumed per loop step
  __shared__ unsigned long long sm_key[4][16 * MT];
  __shared__ unsigned long long sm_key2[TOP2 ? 4 : 1][TOP2 ? 16 * MT : 1];

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, lr = l & 15, lg = l >> 4;
  const int v_wave = blockIdx.x * (64 * WV) + w * (16 * WV);
  const elem_t* W = static_cast<const elem_t*>(weight);
  const elem_t* Hd = static_cast<const elem_t*>(hidden);

  const elem_t* wrow[WV];
#pragma unroll
  for (int vt = 0; vt < WV; ++vt) {
    const int v = min(v_wave + vt * 16 + lr, V - 1);
    wrow[vt] = W + static_cast<size_t>(v) * H;
  }

  for (int m0 = 0; m0 < M; m0 += 16 * MT) {
    f32x4 acc[WV][MT];
    const elem_t* hrow[MT];
    bool hok[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = m0 + mt * 16 + lr;
      hok[mt] = m < M;
      hrow[mt] = Hd + static_cast<size_t>(hok[mt] ? m : 0) * hstride;
#pragma unroll
      for (int vt = 0; vt < WV; ++vt) acc[vt][mt] = f32x4{0, 0, 0, 0};
    }
#pragma unroll 2
    for (int k0 = 0; k0 < H; k0 += KSTEP) {
      if constexpr (BF16) {
        const int kk = k0 + 8 * lg;
        u32x4 a[WV], bv[MT];
#pragma unroll
        for (int vt = 0; vt < WV; ++vt) a[vt] = *reinterpret_cast<const u32x4*>(wrow[vt] + kk);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          bv[mt] = hok[mt] ? *reinterpret_cast<const u32x4*>(hrow[mt] + kk) : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int vt = 0; vt < WV; ++vt)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[vt][mt] = mfma16x16x32_bf16(a[vt], bv[mt], acc[vt][mt]);
      } else {
        const int kk = k0 + 4 * lg;
        f32x4 a[WV], bv[MT];
#pragma unroll
        for (int vt = 0; vt < WV; ++vt) a[vt] = *reinterpret_cast<const f32x4*>(wrow[vt] + kk);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          bv[mt] = hok[mt] ? *reinterpret_cast<const f32x4*>(hrow[mt] + kk) : f32x4{0, 0, 0, 0};
#pragma unroll
        for (int vt = 0; vt < WV; ++vt)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[vt][mt] = mfma16x16x4_f32(a[vt][i], bv[mt][i], acc[vt][mt]);
      }
    }
    // lane holds logits of vocab ids v_wave + vt*16 + 4*lg + i for row m0 + mt*16 + lr
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      uint64_t best = 0, second = 0;
#pragma unroll
      for (int vt = 0; vt < WV; ++vt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int v = v_wave + vt * 16 + 4 * lg + i;
          if (v < V) {
            const float x = BF16 ? round_bf16(acc[vt][mt][i]) : acc[vt][mt][i];
            const uint64_t key = (static_cast<uint64_t>(order_key(x)) << 32) |
                                 static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(v));
            if constexpr (TOP2)
              top2_insert(best, second, key);
            else
              best = umax64(key, best);
          }
        }
      }
      if constexpr (TOP2) {
        top2_across_groups(best, second);
        if (lg == 0) sm_key2[w][mt * 16 + lr] = second;
      } else {
        best = max_across_groups_u64(best);
      }
      if (lg == 0) sm_key[w][mt * 16 + lr] = best;
    }
    __syncthreads();
    for (int r = tid; r < 16 * MT; r += 256) {
      if (m0 + r < M) {
        unsigned long long* k1 = &keys[static_cast<size_t>(blockIdx.x % kKeySlots) * M + m0 + r];
        if constexpr (TOP2) {
          uint64_t a = sm_key[0][r], b = sm_key2[0][r];
          for (int q = 1; q < 4; ++q) top2_merge(a, b, sm_key[q][r], sm_key2[q][r]);
          publish_top2(k1, k1 + static_cast<size_t>(kKeySlots) * M, a, b);
        } else {
          unsigned long long k = sm_key[0][r];
          k = sm_key[1][r] > k ? sm_key[1][r] : k;
          k = sm_key[2][r] > k ? sm_key[2][r] : k;
          k = sm_key[3][r] > k ? sm_key[3][r] : k;
          atomicMax(k1, k);
        }
      }
    }
    __syncthreads();
  }

}

// bf16 path through LDS (kve_gemm.h): workgroup = NW waves as NR row groups x
// NC = NW / NR wave columns; BN = 16 WN NC vocabulary rows x up to 16 MT
// hidden rows per pass (each wave WN vocabulary tiles x MT / NR row tiles).
// The hidden rows are staged once per workgroup and shared by its waves, and
// every tile is read from global memory as whole rows, by direct-to-LDS
// loads. The keys of the wave columns meet in the dynamic LDS after the GEMM.
// MINW: waves per SIMD the register allocation must leave room for (2 keeps
// two 4-wave workgroups on a CU, at most 256 registers per lane).
template <int MT_, int NW_, int WN_, int KC_, int LDS_, int NR_, int MINW_ = 1>
struct LmTile {
  using G = typename DmaCfg<MT_, NW_, WN_, KC_, LDS_, NR_>::G;
  static constexpr int MT = MT_, NW = NW_, WN = WN_, NR = NR_, NC = NW_ / NR_, NT = 64 * NW_;
  static constexpr int MINW = MINW_;
  static constexpr size_t KEY_BYTES = 2 * sizeof(unsigned long long) * NC * 16 * MT_;
  static constexpr size_t LDS = G::LDS_BYTES > KEY_BYTES ? G::LDS_BYTES : KEY_BYTES;
};

template <typename C, bool TOP2, bool BLK = false>
__global__ __launch_bounds__(C::NT, C::MINW) void lmhead_lds_kernel(const uint16_t* hidden, int64_t hstride,
                                                           const uint16_t* weight, int M, int H,
                                                           int V, unsigned long long* keys) {
  using G = typename C::G;
  constexpr int MT = C::MT, WN = C::WN, NC = C::NC, MTW = MT / C::NR, ROWS = 16 * MT;
  extern __shared__ __align__(16) uint16_t sm_lh[];
  unsigned long long* sk = reinterpret_cast<unsigned long long*>(sm_lh);  // [NC][ROWS]
  unsigned long long* sk2 = sk + NC * ROWS;                               // [NC][ROWS]
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wc = w % NC, wr = w / NC;
  const int l = tid & 63, lr = l & 15, lg = l >> 4;
  const int v0 = blockIdx.x * G::BN;
  for (int m0 = 0; m0 < M; m0 += ROWS) {
    f32x4 acc[WN][MTW];
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) acc[j][mt] = f32x4{0, 0, 0, 0};
    G::template run<BLK>(weight, [v0, V](int r) { return min(v0 + r, V - 1); }, hidden + m0 * hstride, hstride,
           min(M - m0, ROWS), H, 0, H / 32, sm_lh, acc);
    // lane holds logits of vocab ids v0 + 16 (WN wc + j) + 4 lg + i for row
    // m0 + 16 (MTW wr + mt) + lr
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt) {
      uint64_t best = 0, second = 0;
#pragma unroll
      for (int j = 0; j < WN; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int v = v0 + 16 * (WN * wc + j) + 4 * lg + i;
          if (v < V) {
            const float x = round_bf16(acc[j][mt][i]);
            const uint64_t key = (static_cast<uint64_t>(order_key(x)) << 32) |
                                 static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(v));
            if constexpr (TOP2)
              top2_insert(best, second, key);
            else
              best = umax64(key, best);
          }
        }
      }
      const int r = 16 * (MTW * wr + mt) + lr;
      if constexpr (TOP2) {
        top2_across_groups(best, second);
        if (lg == 0) sk2[wc * ROWS + r] = second;
      } else {
        best = max_across_groups_u64(best);
      }
      if (lg == 0) sk[wc * ROWS + r] = best;
    }
    __syncthreads();
    for (int r = tid; r < ROWS; r += C::NT) {
      if (m0 + r < M) {
        unsigned long long* k1 = &keys[static_cast<size_t>(blockIdx.x % kKeySlots) * M + m0 + r];
        if constexpr (TOP2) {
          uint64_t a = sk[r], b = sk2[r];
          for (int q = 1; q < NC; ++q) top2_merge(a, b, sk[q * ROWS + r], sk2[q * ROWS + r]);
          publish_top2(k1, k1 + static_cast<size_t>(kKeySlots) * M, a, b);
        } else {
          unsigned long long k = sk[r];
          for (int q = 1; q < NC; ++q) k = sk[q * ROWS + r] > k ? sk[q * ROWS + r] : k;
          atomicMax(k1, k);
        }
      }
    }
    __syncthreads();
  }
}

// Second launch: read each row's winning key (and runner-up), write the ids and
// values, and clear the keys for the next launch. Running after the GEMM kernel
// makes every workgroup's atomics visible without a device-scope fence in the
// hot kernel.
__device__ __forceinline__ int32_t key_id(uint64_t k) {
  return static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(k & 0xffffffffull));
}

template <bool TOP2>
__global__ __launch_bounds__(64) void lmhead_finalize_kernel(unsigned long long* keys, int M,
                                                              int32_t* argmax, float* maxval,
                                                              int32_t* second_id, float* second_val) {
  const int m = blockIdx.x, l = threadIdx.x;  // lane l: key copy l
  unsigned long long* p = keys + static_cast<size_t>(l) * M + m;
  uint64_t k = *p, k2 = 0;
  *p = 0ull;
  if constexpr (TOP2) {
    unsigned long long* p2 = p + static_cast<size_t>(kKeySlots) * M;
    k2 = *p2;
    *p2 = 0ull;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t x = __shfl_xor(static_cast<unsigned long long>(k), o);
      const uint64_t x2 = __shfl_xor(static_cast<unsigned long long>(k2), o);
      top2_merge(k, k2, x, x2);
    }
  } else {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const unsigned long long x = __shfl_xor(static_cast<unsigned long long>(k), o);
      k = x > k ? x : k;
    }
    k = max_across_groups_u64(k);
  }
  if (l != 0) return;
  argmax[m] = key_id(k);
  if (maxval) maxval[m] = unorder_key(static_cast<uint32_t>(k >> 32));
  if constexpr (TOP2) {
    if (second_id) second_id[m] = k2 ? key_id(k2) : -1;
    if (second_val) second_val[m] = k2 ? unorder_key(static_cast<uint32_t>(k2 >> 32)) : -INFINITY;
  }
}

// Everything a launch needs besides the GEMM shape.
struct LmOut {
  int32_t* argmax;
  float* maxval;
  int32_t* second_id;  // with second_val: NULL for top-1 only
  float* second_val;
  unsigned long long* keys;
  bool top2() const { return second_id || second_val; }
};

static void launch_finalize(int M, const LmOut& o, hipStream_t st) {
  if (o.top2())
    hipLaunchKernelGGL(lmhead_finalize_kernel<true>, dim3(M), dim3(64), 0, st, o.keys, M, o.argmax,
                       o.maxval, o.second_id, o.second_val);
  else
    hipLaunchKernelGGL(lmhead_finalize_kernel<false>, dim3(M), dim3(64), 0, st, o.keys, M, o.argmax,
                       o.maxval, nullptr, nullptr);
}

template <bool BF16, int MT>
static void launch_lmhead(const void* hidden, int64_t hs, const void* w, int M, int H, int V,
                          const LmOut& o, hipStream_t st) {
  constexpr int WV = 2;
  const dim3 grid(cdiv(V, 64 * WV));
  if (o.top2())
    hipLaunchKernelGGL((lmhead_argmax_kernel<BF16, WV, MT, true>), grid, dim3(256), 0, st, hidden,
                       hs, w, M, H, V, o.keys);
  else
    hipLaunchKernelGGL((lmhead_argmax_kernel<BF16, WV, MT, false>), grid, dim3(256), 0, st, hidden,
                       hs, w, M, H, V, o.keys);
  launch_finalize(M, o, st);
}

template <typename K>
static int allow_lds_lm(K kernel, size_t bytes) {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                             hipFuncAttributeMaxDynamicSharedMemorySize,
                             static_cast<int>(bytes)) == hipSuccess
             ? 0
             : -1;
}

template <typename C, bool TOP2, bool BLK>
static int launch_lmhead_lds_t(const void* hidden, int64_t hs, const void* w, int M, int H, int V,
                               const LmOut& o, hipStream_t st) {
  auto kernel = lmhead_lds_kernel<C, TOP2, BLK>;
  static size_t granted = 0;  // dynamic LDS this instantiation may use
  if (C::LDS > granted) {
    if (allow_lds_lm(kernel, C::LDS)) {
      set_error("kve_lmhead_argmax: %zu bytes of LDS refused", C::LDS);
      return KVE_ELAUNCH;
    }
    granted = C::LDS;
  }
  hipLaunchKernelGGL(kernel, dim3(cdiv(V, C::G::BN)), dim3(C::NT), C::LDS, st,
                     static_cast<const uint16_t*>(hidden), hs, static_cast<const uint16_t*>(w), M,
                     H, V, o.keys);
  launch_finalize(M, o, st);
  return KVE_OK;
}

template <typename C>
static int launch_lmhead_lds(const void* hidden, int64_t hs, const void* w, int M, int H, int V,
                             const LmOut& o, hipStream_t st, bool blk) {
  if (blk)
    return o.top2() ? launch_lmhead_lds_t<C, true, true>(hidden, hs, w, M, H, V, o, st)
                    : launch_lmhead_lds_t<C, false, true>(hidden, hs, w, M, H, V, o, st);
  return o.top2() ? launch_lmhead_lds_t<C, true, false>(hidden, hs, w, M, H, V, o, st)
                  : launch_lmhead_lds_t<C, false, false>(hidden, hs, w, M, H, V, o, st);
}

// bf16: the LDS-staged kernel (row tiles of 16, hidden rows in passes of up to
// 160); four waves and about 56 KB of LDS, so two workgroups share a CU.
// Measured against eight waves with 144 KB of chunk buffers (one workgroup
// per CU, two or three chunks in flight): no faster at any row count (160 x
// 2048 x 151936: 191.6 us against 201.7-225.3; 32 x 896: 45.5 against
// 52.4-75.4).
static int dispatch_lmhead_bf16(int M, const void* hidden, int64_t hs, const void* w, int H, int V,
                                const LmOut& o, hipStream_t st, bool blk) {
  const int tiles = cdiv(M, 16);
#define LM(...) return launch_lmhead_lds<LmTile<__VA_ARGS__>>(hidden, hs, w, M, H, V, o, st, blk)
  if (tiles <= 1) LM(1, 4, 1, 4, 56 * 1024, 1);
  if (tiles <= 2) LM(2, 4, 1, 2, 56 * 1024, 1);
  if (tiles <= 4) LM(4, 4, 1, 2, 56 * 1024, 1);
  if (tiles <= 6) LM(6, 4, 1, 2, 56 * 1024, 1);
  // 7-10 row tiles, blocked operands: 192 embedding rows on the waves as 2
  // column x 2 row groups (each wave 6 x 5 tiles) with one-k-step chunks, held
  // to 256 registers so two workgroups share a CU (240, no spills; without the
  // bound the compiler takes 294 and one runs per CU: 194 us). Each workgroup
  // re-reads the hidden rows for 192 embedding rows instead of 128, 19 % fewer
  // bytes per CU in all: 160 x 2048 x 151936 149.5-150.0 -> 144.3-147.5 us
  // (HIP graph 156-158 -> 148-150). Earlier: the 4 x 1 split of 128 rows below
  // takes 260 registers and runs one per CU, 2 x 2 of 128 rows 159 -> 152 us.
  // Measured no faster: 128- and 256-row tiles on 8 or 10 waves, one
  // workgroup per CU (163-216 us), three chunk buffers (194 us), 128 rows on 8
  // waves as 4 x 2 (two per CU: 148.4-148.9 against 149.8-150.3 us) or 10
  // waves as 2 x 5 (one per CU: 170 us), weight and activation chunks in
  // separate LDS rings loaded by separate waves (155-157 us).
  if (blk) LM(10, 4, 6, 1, 72 * 1024, 2, 2);
  LM(10, 4, 2, 2, 56 * 1024, 1);
#undef LM
}

template <bool BF16>
static void dispatch_lmhead(int M, const void* hidden, int64_t hs, const void* w, int H, int V,
                            const LmOut& o, hipStream_t st) {
  const int tiles = cdiv(M, 16);
  if (tiles <= 1) launch_lmhead<BF16, 1>(hidden, hs, w, M, H, V, o, st);
  else if (tiles <= 2) launch_lmhead<BF16, 2>(hidden, hs, w, M, H, V, o, st);
  else if (tiles <= 4) launch_lmhead<BF16, 4>(hidden, hs, w, M, H, V, o, st);
  else if (tiles <= 6) launch_lmhead<BF16, 6>(hidden, hs, w, M, H, V, o, st);
  else if (tiles <= 8) launch_lmhead<BF16, 8>(hidden, hs, w, M, H, V, o, st);
  else launch_lmhead<BF16, 10>(hidden, hs, w, M, H, V, o, st);
}

// Validates the arguments shared by both entry points and runs the two launches
// with the key buffer `keys` (kKeySlots * M keys, twice that for top-2).
static int lmhead_run(const void* hidden, int64_t hidden_row_stride, const void* weight, int M,
                      int H, int V, int dtype, int layout, const LmOut& o, hipStream_t st,
                      const char* name) {
  KVE_REQUIRE(hidden && weight && o.argmax, "%s: null pointer argument", name);
  KVE_REQUIRE(M > 0 && V > 0 && H > 0 && H % 32 == 0, "%s: M=%d H=%d V=%d", name, M, H, V);
  KVE_REQUIRE(dtype == KVE_DTYPE_BF16 || dtype == KVE_DTYPE_F32, "%s: dtype %d", name, dtype);
  KVE_REQUIRE(((reinterpret_cast<uintptr_t>(hidden) | reinterpret_cast<uintptr_t>(weight)) & 15) == 0,
              "%s: hidden and weight must be 16-byte aligned", name);
  const int vec = dtype == KVE_DTYPE_BF16 ? 8 : 4;
  KVE_REQUIRE(layout == KVE_LAYOUT_ROWS ||
                  (layout == KVE_LAYOUT_BLOCKED && dtype == KVE_DTYPE_BF16 && V % 16 == 0),
              "%s: layout %d with dtype %d, V=%d", name, layout, dtype, V);
  const bool blk = layout == KVE_LAYOUT_BLOCKED;
  if (blk) hidden_row_stride = H;  // row tiles of 16 sit H * 16 elements apart
  KVE_REQUIRE(hidden_row_stride >= H && hidden_row_stride % vec == 0, "%s: hidden_row_stride %lld",
              name, static_cast<long long>(hidden_row_stride));
  if (dtype == KVE_DTYPE_BF16) {
    const int rc = dispatch_lmhead_bf16(M, hidden, hidden_row_stride, weight, H, V, o, st, blk);
    if (rc) return rc;
  } else {
    dispatch_lmhead<false>(M, hidden, hidden_row_stride, weight, H, V, o, st);
  }
  return check_launch(name);
}

}  // namespace kve

using namespace kve;

extern "C" size_t kve_lmhead_workspace_bytes(int M) {
  if (M <= 0) return 0;
  return 256 + static_cast<size_t>(M) * 8 * kKeySlots * 2;
}

extern "C" int kve_lmhead_argmax(const void* hidden, int64_t hidden_row_stride, const void* weight,
                                 int M, int H, int V, int dtype, int32_t* argmax, float* maxval,
                                 int32_t* second_id, float* second_val, void* workspace,
                                 size_t workspace_bytes, int layout, void* stream) {
  clear_error();
  if (M == 0) return KVE_OK;
  KVE_REQUIRE(workspace, "kve_lmhead_argmax: null workspace");
  if (M > 0 && workspace_bytes < kve_lmhead_workspace_bytes(M)) {
    set_error("kve_lmhead_argmax: workspace %zu bytes, need %zu", workspace_bytes,
              kve_lmhead_workspace_bytes(M));
    return KVE_EWORKSPACE;
  }
  const LmOut o{argmax, maxval, second_id, second_val,
                reinterpret_cast<unsigned long long*>(static_cast<char*>(workspace) + 256)};
  return lmhead_run(hidden, hidden_row_stride, weight, M, H, V, dtype, layout, o,
                    static_cast<hipStream_t>(stream), "kve_lmhead_argmax");
}


// ---- no-allocation variant ---------------------------------------------------
// For callers that cannot allocate (code under graph capture, serving loops that
// forbid hipMalloc): the key copies live in a file-scope device array instead of
// a caller workspace. Each GPU holds its own copy of the array for the life of
// the process; host code never passes the array's name to a kernel (on the host
// it is only a stand-in for the symbol), it passes the device address that
// hipGetSymbolAddress returned for the current device.

constexpr int kNoAllocMaxRows = KVE_LMHEAD_NOALLOC_MAX_ROWS;
constexpr size_t kNoAllocKeys = static_cast<size_t>(kNoAllocMaxRows) * kKeySlots * 2;  // top-2

static __device__ __align__(256) unsigned long long scratch[kNoAllocKeys];

namespace {

constexpr int kMaxDevices = 64;

struct ScratchSlot {
  unsigned long long* ptr = nullptr;
  bool cleared = false;
};

std::mutex g_scratch_mu;
ScratchSlot g_scratch[kMaxDevices];

__global__ __launch_bounds__(256) void clear_keys_kernel(unsigned long long* keys, size_t n) {
  for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256)
    keys[i] = 0ull;
}

// The current device's scratch address, resolved once per device; the keys are
// cleared on the stream before the first use there (a launch error on the way
// marks them for clearing again).
int noalloc_keys(hipStream_t st, unsigned long long** out, ScratchSlot** slot) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("kve_lmhead_argmax_noalloc: no usable current device (%s)", hipGetErrorString(e));
    return KVE_ELAUNCH;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchSlot& s = g_scratch[dev];
  if (!s.ptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("kve_lmhead_argmax_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
      return KVE_ELAUNCH;
    }
    s.ptr = static_cast<unsigned long long*>(p);
  }
  if (!s.cleared) {
    hipLaunchKernelGGL(clear_keys_kernel, dim3(64), dim3(256), 0, st, s.ptr, kNoAllocKeys);
    const int rc = check_launch("kve_lmhead_argmax_noalloc");
    if (rc) return rc;
    s.cleared = true;
  }
  *out = s.ptr;
  *slot = &s;
  return KVE_OK;
}

}  // namespace

extern "C" int kve_lmhead_argmax_noalloc(const void* hidden, int64_t hidden_row_stride,
                                         const void* weight, int M, int H, int V, int dtype,
                                         int32_t* argmax, float* maxval, int32_t* second_id,
                                         float* second_val, void* stream) {
  clear_error();
  if (M == 0) return KVE_OK;
  KVE_REQUIRE(M > 0 && M <= kNoAllocMaxRows,
              "kve_lmhead_argmax_noalloc: M=%d rows, this entry point takes 1..%d", M,
              kNoAllocMaxRows);
  hipStream_t st = static_cast<hipStream_t>(stream);
  unsigned long long* keys = nullptr;
  ScratchSlot* slot = nullptr;
  int rc = noalloc_keys(st, &keys, &slot);
  if (rc) return rc;
  const LmOut o{argmax, maxval, second_id, second_val, keys};
  rc = lmhead_run(hidden, hidden_row_stride, weight, M, H, V, dtype, KVE_LAYOUT_ROWS, o, st,
                  "kve_lmhead_argmax_noalloc");
  if (rc == KVE_ELAUNCH) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    slot->cleared = false;  // a launch may have left keys behind
  }
  return rc;
}
