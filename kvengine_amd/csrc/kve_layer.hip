// Fused per-layer elementwise kernels for the Qwen2 forward pass on gfx950.
//
// In the reference every layer runs transformers' modules as separate torch
// ops (kvengine/forward.py:190-207): RMSNorm is eight kernels (cast, pow, mean,
// add, rsqrt, mul, cast, mul), RoPE about six per tensor (slice, neg, cat, two
// muls, add), the residual adds and SwiGLU's silu and mul one each. At decode
// batch sizes each of those is a few microseconds of launch for almost no
// bytes. These kernels do the same arithmetic with the same rounding points
// (every intermediate the reference materialises in the model dtype is rounded
// to it here too; products and sums use explicit round-to-nearest intrinsics
// so nothing is contracted into an FMA), one launch each:
//
//   kve_rmsnorm:        r = x (+ delta); y = w * cast(r * rsqrt(mean(r^2) + eps))
//   kve_rope_kv_write:  q' = q*cos + rotate_half(q)*sin (likewise k) from the
//                       fused QKV projection; k', v scattered into the paged
//                       pool; q' written for the attention kernel
//   kve_silu_mul:       silu(gate) * up from the fused gate/up projection

#include "kve_common.h"

#include <type_traits>

// hipcc contracts a*b + c*d into an FMA by default; these kernels must round
// each product and sum separately, as the torch ops they replace do.
#pragma clang fp contract(off)

namespace kve {

template <bool BF16>
struct Elem;
template <>
struct Elem<true> {
  using T = uint16_t;
  __device__ static float ld(const T* p, size_t i) { return bf16_to_f32(p[i]); }
  __device__ static T cvt(float x) { return f32_to_bf16(x); }
  // value as the model dtype would hold it
  __device__ static float rnd(float x) { return round_bf16(x); }
};
template <>
struct Elem<false> {
  using T = float;
  __device__ static float ld(const T* p, size_t i) { return p[i]; }
  __device__ static T cvt(float x) { return x; }
  __device__ static float rnd(float x) { return x; }
};

// Vector of VPT model-dtype values: 8 bf16 or 4 fp32 (16 bytes).
template <bool BF16>
struct Vec;
template <>
struct Vec<true> {
  static constexpr int N = 8;
  using raw = u32x4;
  __device__ static void unpack(const raw& r, float (&f)[N]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(r[i] << 16);
      f[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
    }
  }
  __device__ static raw pack(const float (&f)[N]) {
    raw r;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      r[i] = static_cast<uint32_t>(f32_to_bf16(f[2 * i])) |
             (static_cast<uint32_t>(f32_to_bf16(f[2 * i + 1])) << 16);
    return r;
  }
};
template <>
struct Vec<false> {
  static constexpr int N = 4;
  using raw = f32x4;
  __device__ static void unpack(const raw& r, float (&f)[N]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = r[i];
  }
  __device__ static raw pack(const float (&f)[N]) { return raw{f[0], f[1], f[2], f[3]}; }
};

// ---- RMSNorm (+ residual) ----------------------------------------------------
// One workgroup per row, NV 16-byte vectors per thread held in registers.
// torch's Qwen2RMSNorm: x.float(); var = x.pow(2).mean(); x * rsqrt(var + eps);
// cast to the input dtype; weight * x (in the dtype). The mean's float32 sum is
// taken in a different order than torch's, which can move the result by an ulp.
template <bool BF16, int NV>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const void* x, const void* delta,
                                                      void* residual_out, const void* weight,
                                                      void* out, int H, float eps, int out_blocked) {
  using E = Elem<BF16>;
  using V = Vec<BF16>;
  using raw = typename V::raw;
  constexpr int VN = V::N;
  __shared__ float sm_part[4];
  const int row = blockIdx.x;
  const size_t base = static_cast<size_t>(row) * H;
  const raw* xr = reinterpret_cast<const raw*>(static_cast<const typename E::T*>(x) + base);
  const raw* dr = delta ? reinterpret_cast<const raw*>(static_cast<const typename E::T*>(delta) + base) : nullptr;
  const raw* wr = reinterpret_cast<const raw*>(weight);
  const int nvec = H / VN;
  raw xv[NV], dv[NV], wv[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = threadIdx.x + k * 256;
    if (i < nvec) {
      xv[k] = xr[i];
      wv[k] = wr[i];
      if (dr) dv[k] = dr[i];
    }
  }
  float v[NV][VN];
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = threadIdx.x + k * 256;
    if (i >= nvec) continue;
    V::unpack(xv[k], v[k]);
    if (dr) {
      float d[VN];
      V::unpack(dv[k], d);
#pragma unroll
      for (int e = 0; e < VN; ++e) v[k][e] = E::rnd(__fadd_rn(v[k][e], d[e]));  // residual add in the dtype
      if (residual_out)
        reinterpret_cast<raw*>(static_cast<typename E::T*>(residual_out) + base)[i] = V::pack(v[k]);
    } else if (residual_out) {
      reinterpret_cast<raw*>(static_cast<typename E::T*>(residual_out) + base)[i] = xv[k];
    }
#pragma unroll
    for (int e = 0; e < VN; ++e) ss = __fadd_rn(ss, __fmul_rn(v[k][e], v[k][e]));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss = __fadd_rn(ss, __shfl_xor(ss, o));
  if ((threadIdx.x & 63) == 0) sm_part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = __fadd_rn(__fadd_rn(sm_part[0], sm_part[1]), __fadd_rn(sm_part[2], sm_part[3]));
  const float inv = rsqrtf(__fadd_rn(__fmul_rn(tot, 1.0f / static_cast<float>(H)), eps));
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = threadIdx.x + k * 256;
    if (i >= nvec) continue;
    float w[VN], o[VN];
    V::unpack(wv[k], w);
#pragma unroll
    for (int e = 0; e < VN; ++e) o[e] = __fmul_rn(w[e], E::rnd(__fmul_rn(v[k][e], inv)));
    *reinterpret_cast<raw*>(static_cast<typename E::T*>(out) +
                            mat_off(row, i * VN, H, H, out_blocked)) = V::pack(o);
  }
}

// ---- RoPE + KV write ---------------------------------------------------------
// One workgroup per token; a thread rotates 4 pairs (j..j+3, j+D/2..j+D/2+3)
// of one head. qkv row: [Hq*D | Hkv*D | Hkv*D] (bias already added by the
// projection). cos/sin rows [D] in the model dtype (transformers computes them
// in float32 and casts). rotate_half(x)[d] = -x[d + D/2] (d < D/2), x[d - D/2].
template <bool BF16, int D>
__global__ __launch_bounds__(256) void rope_kv_write_kernel(
    const void* qkv, const void* cos, const void* sin, void* q_out, void* k_pool, void* v_pool,
    const int32_t* tables, const int32_t* seq_rows, const int32_t* start_pos,
    const int32_t* q_lens, int Tq, int Hq, int Hkv, int bs, int max_blocks, int num_rows,
    int num_blocks) {
  using E = Elem<BF16>;
  using T = typename E::T;
  using raw4 = std::conditional_t<BF16, u32x2, f32x4>;  // 4 values
  constexpr int half = D / 2;
  constexpr int TPH = half / 4;  // threads per head
  const int tok = blockIdx.x;
  const int i = tok / Tq, t = tok - i * Tq;
  const int width = (Hq + 2 * Hkv) * D;
  const T* src = static_cast<const T*>(qkv) + static_cast<size_t>(tok) * width;
  const T* cr = static_cast<const T*>(cos) + static_cast<size_t>(tok) * D;
  const T* sr = static_cast<const T*>(sin) + static_cast<size_t>(tok) * D;
  // where this token's K/V go (or nowhere, for padding or a bad table)
  int blk = -1, off = 0;
  const int T_i = q_lens ? min(q_lens[i], Tq) : Tq;
  if (t < T_i) {
    const int row = seq_rows ? seq_rows[i] : i;
    if (row >= 0 && row < num_rows) {
      const int pos = start_pos[row] + t;
      if (pos >= 0 && pos / bs < max_blocks) {
        const int b = tables[static_cast<size_t>(row) * max_blocks + pos / bs];
        if (b >= 0 && b < num_blocks) {
          blk = b;
          off = pos % bs;
        }
      }
    }
  }
  auto ld4 = [](const T* p, float (&f)[4]) {
    const raw4 r = *reinterpret_cast<const raw4*>(p);
    if constexpr (BF16) {
      f[0] = __uint_as_float(r[0] << 16);
      f[1] = __uint_as_float(r[0] & 0xffff0000u);
      f[2] = __uint_as_float(r[1] << 16);
      f[3] = __uint_as_float(r[1] & 0xffff0000u);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) f[e] = r[e];
    }
  };
  auto st4 = [](T* p, const float (&f)[4]) {
    if constexpr (BF16) {
      *reinterpret_cast<u32x2*>(p) =
          u32x2{static_cast<uint32_t>(f32_to_bf16(f[0])) | (static_cast<uint32_t>(f32_to_bf16(f[1])) << 16),
                static_cast<uint32_t>(f32_to_bf16(f[2])) | (static_cast<uint32_t>(f32_to_bf16(f[3])) << 16)};
    } else {
      *reinterpret_cast<f32x4*>(p) = f32x4{f[0], f[1], f[2], f[3]};
    }
  };
  // rotated heads: Hq query heads then Hkv key heads
  for (int idx = threadIdx.x; idx < (Hq + Hkv) * TPH; idx += blockDim.x) {
    const int h = idx / TPH, j = (idx % TPH) * 4;
    const T* x = src + h * D;
    float a[4], bb[4], cl[4], ch[4], sl[4], sh[4], lo[4], hi[4];
    ld4(x + j, a);
    ld4(x + j + half, bb);
    ld4(cr + j, cl);
    ld4(cr + j + half, ch);
    ld4(sr + j, sl);
    ld4(sr + j + half, sh);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lo[e] = E::rnd(__fadd_rn(E::rnd(__fmul_rn(a[e], cl[e])), E::rnd(__fmul_rn(-bb[e], sl[e]))));
      hi[e] = E::rnd(__fadd_rn(E::rnd(__fmul_rn(bb[e], ch[e])), E::rnd(__fmul_rn(a[e], sh[e]))));
    }
    T* dst;
    if (h < Hq) {
      dst = static_cast<T*>(q_out) + (static_cast<size_t>(tok) * Hq + h) * D;
    } else if (blk >= 0) {
      dst = static_cast<T*>(k_pool) + ((static_cast<size_t>(blk) * Hkv + (h - Hq)) * bs + off) * D;
    } else {
      continue;
    }
    st4(dst + j, lo);
    st4(dst + j + half, hi);
  }
  if (blk >= 0) {
    // V goes channel-major into the block ([D][bs] per head): scalar stores
    const T* vs = src + (Hq + Hkv) * D;
    for (int idx = threadIdx.x; idx < Hkv * D / 4; idx += blockDim.x) {
      const int h = idx / (D / 4), d = (idx % (D / 4)) * 4;
      const raw4 r = *reinterpret_cast<const raw4*>(vs + h * D + d);
      T* vd = static_cast<T*>(v_pool) + ((static_cast<size_t>(blk) * Hkv + h) * D + d) * bs + off;
      if constexpr (BF16) {
        vd[0] = static_cast<T>(r[0] & 0xffffu);
        vd[bs] = static_cast<T>(r[0] >> 16);
        vd[2 * bs] = static_cast<T>(r[1] & 0xffffu);
        vd[3 * bs] = static_cast<T>(r[1] >> 16);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) vd[e * bs] = r[e];
      }
    }
  }
}

// ---- SiLU * up -----------------------------------------------------------------
// gate_up row: [gate F | up F]; out = cast(silu(gate)) * up, each op rounded to
// the model dtype as torch does (silu computes x / (1 + exp(-x)) in float32).
// Grid (F / (256 * VN) rounded up, rows); one 16-byte vector per thread.
template <bool BF16>
__global__ __launch_bounds__(256) void silu_mul_kernel(const void* gate_up, void* out, int F) {
  using E = Elem<BF16>;
  using V = Vec<BF16>;
  using raw = typename V::raw;
  constexpr int VN = V::N;
  const int m = blockIdx.y;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= F / VN) return;
  const typename E::T* row = static_cast<const typename E::T*>(gate_up) + static_cast<size_t>(m) * 2 * F;
  float g[VN], u[VN], o[VN];
  V::unpack(reinterpret_cast<const raw*>(row)[i], g);
  V::unpack(reinterpret_cast<const raw*>(row + F)[i], u);
#pragma unroll
  for (int e = 0; e < VN; ++e) {
    const float sg = E::rnd(__fdiv_rn(g[e], __fadd_rn(1.0f, expf(-g[e]))));
    o[e] = __fmul_rn(sg, u[e]);
  }
  reinterpret_cast<raw*>(static_cast<typename E::T*>(out) + static_cast<size_t>(m) * F)[i] = V::pack(o);
}

// The per-pass prologue, one launch in place of the embedding lookup, the
// start positions and the RoPE table gathers (Qwen2Model's embed_tokens and
// rotary_emb ahead of the layer loop, kvengine/forward.py:176-184): row
// m = b * T + t gets embed[ids[m]] and cos/sin[min(lens[rows[b]] + t, P - 1)]
// (the table lookup of the same positions the reference computes). An id
// outside the vocabulary gives a zero row. Pure copies: the same bits as the
// torch ops. One workgroup per row, 16-byte vectors.
__global__ __launch_bounds__(128) void pass_prologue_kernel(
    const int64_t* ids, const uint16_t* embed, int64_t V, int H, const int32_t* lens,
    const int32_t* rows, int num_rows, int T, const uint16_t* cos_t, const uint16_t* sin_t, int P,
    int D, uint16_t* hidden, uint16_t* cos, uint16_t* sin) {
  const int m = blockIdx.x;
  const int b = m / T, t = m - b * T;
  const int64_t id = ids[m];
  const bool ok = id >= 0 && id < V;
  const u32x4* src = reinterpret_cast<const u32x4*>(embed + (ok ? id : 0) * static_cast<int64_t>(H));
  u32x4* dst = reinterpret_cast<u32x4*>(hidden + static_cast<size_t>(m) * H);
  for (int i = threadIdx.x; i < H / 8; i += 128) dst[i] = ok ? src[i] : u32x4{0, 0, 0, 0};
  // a table row outside [0, num_rows) is never read: its tokens take position t
  const int row = rows[b];
  int pos = (row >= 0 && row < num_rows ? lens[row] : 0) + t;
  pos = pos < 0 ? 0 : (pos > P - 1 ? P - 1 : pos);
  const u32x4* cs = reinterpret_cast<const u32x4*>(cos_t + static_cast<size_t>(pos) * D);
  const u32x4* ss = reinterpret_cast<const u32x4*>(sin_t + static_cast<size_t>(pos) * D);
  u32x4* cd = reinterpret_cast<u32x4*>(cos + static_cast<size_t>(m) * D);
  u32x4* sd = reinterpret_cast<u32x4*>(sin + static_cast<size_t>(m) * D);
  for (int i = threadIdx.x; i < D / 8; i += 128) {
    cd[i] = cs[i];
    sd[i] = ss[i];
  }
}

}  // namespace kve

using namespace kve;

template <bool BF16>
static void launch_rmsnorm(int NV, dim3 grid, hipStream_t st, const void* x, const void* delta,
                           void* residual_out, const void* weight, void* out, int H, float eps,
                           int ob) {
  if (NV == 1)
    hipLaunchKernelGGL((rmsnorm_kernel<BF16, 1>), grid, dim3(256), 0, st, x, delta, residual_out, weight, out, H, eps, ob);
  else if (NV == 2)
    hipLaunchKernelGGL((rmsnorm_kernel<BF16, 2>), grid, dim3(256), 0, st, x, delta, residual_out, weight, out, H, eps, ob);
  else if (NV <= 4)
    hipLaunchKernelGGL((rmsnorm_kernel<BF16, 4>), grid, dim3(256), 0, st, x, delta, residual_out, weight, out, H, eps, ob);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<BF16, 8>), grid, dim3(256), 0, st, x, delta, residual_out, weight, out, H, eps, ob);
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

extern "C" int kve_rmsnorm(const void* x, const void* delta, void* residual_out,
                           const void* weight, void* out, int rows, int hidden, float eps,
                           int dtype, int layout, void* stream) {
  clear_error();
  if (rows == 0) return KVE_OK;
  KVE_REQUIRE(x && weight && out && rows > 0 && hidden > 0, "kve_rmsnorm: bad arguments");
  KVE_REQUIRE(dtype == KVE_DTYPE_BF16 || dtype == KVE_DTYPE_F32, "kve_rmsnorm: dtype %d", dtype);
  const int vn = dtype == KVE_DTYPE_BF16 ? 8 : 4;
  KVE_REQUIRE(hidden % vn == 0 && hidden <= 256 * 8 * vn,
              "kve_rmsnorm: hidden %d must be a multiple of %d and at most %d", hidden, vn, 256 * 8 * vn);
  KVE_REQUIRE(aligned16(x) && aligned16(weight) && aligned16(out) && (!delta || aligned16(delta)) &&
                  (!residual_out || aligned16(residual_out)),
              "kve_rmsnorm: buffers must be 16-byte aligned");
  KVE_REQUIRE(layout == KVE_LAYOUT_ROWS ||
                  (layout == KVE_LAYOUT_BLOCKED && dtype == KVE_DTYPE_BF16 && hidden % 32 == 0),
              "kve_rmsnorm: layout %d with dtype %d, hidden %d", layout, dtype, hidden);
  const int ob = layout == KVE_LAYOUT_BLOCKED ? 1 : 0;
  const int NV = cdiv(hidden / vn, 256);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == KVE_DTYPE_BF16)
    launch_rmsnorm<true>(NV, dim3(rows), st, x, delta, residual_out, weight, out, hidden, eps, ob);
  else
    launch_rmsnorm<false>(NV, dim3(rows), st, x, delta, residual_out, weight, out, hidden, eps, ob);
  return check_launch("kve_rmsnorm");
}

extern "C" int kve_rope_kv_write(const void* qkv, const void* cos, const void* sin, void* q_out,
                                 void* k_pool, void* v_pool, const int32_t* block_tables,
                                 const int32_t* seq_rows, const int32_t* start_pos,
                                 const int32_t* q_lens, int num_seqs, int q_len, int num_q_heads,
                                 int num_kv_heads, int head_dim, int block_size, int max_blocks,
                                 int num_rows, int num_blocks, int dtype, void* stream) {
  clear_error();
  if (num_seqs == 0) return KVE_OK;
  KVE_REQUIRE(qkv && cos && sin && q_out && k_pool && v_pool && block_tables && start_pos,
              "kve_rope_kv_write: null pointer argument");
  KVE_REQUIRE(num_seqs > 0 && q_len > 0 && num_q_heads > 0 && num_kv_heads > 0 &&
                  head_dim > 0 && head_dim % 2 == 0 && block_size > 0 && max_blocks > 0 &&
                  num_rows > 0 && num_blocks > 0,
              "kve_rope_kv_write: bad sizes");
  KVE_REQUIRE(dtype == KVE_DTYPE_BF16 || dtype == KVE_DTYPE_F32, "kve_rope_kv_write: dtype %d",
              dtype);
  KVE_REQUIRE(head_dim == 64 || head_dim == 128, "kve_rope_kv_write: head_dim %d (64 or 128)",
              head_dim);
  KVE_REQUIRE(aligned16(qkv) && aligned16(cos) && aligned16(sin) && aligned16(q_out) &&
                  aligned16(k_pool),
              "kve_rope_kv_write: buffers must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(num_seqs * q_len);
#define KVE_ROPE(B, DD)                                                                         \
  hipLaunchKernelGGL((rope_kv_write_kernel<B, DD>), grid, dim3(256), 0, st, qkv, cos, sin, q_out, \
                     k_pool, v_pool, block_tables, seq_rows, start_pos, q_lens, q_len,            \
                     num_q_heads, num_kv_heads, block_size, max_blocks, num_rows, num_blocks)
  if (dtype == KVE_DTYPE_BF16) {
    if (head_dim == 64) KVE_ROPE(true, 64);
    else KVE_ROPE(true, 128);
  } else {
    if (head_dim == 64) KVE_ROPE(false, 64);
    else KVE_ROPE(false, 128);
  }
#undef KVE_ROPE
  return check_launch("kve_rope_kv_write");
}

extern "C" int kve_silu_mul(const void* gate_up, void* out, int rows, int ffn, int dtype,
                            void* stream) {
  clear_error();
  if (rows == 0) return KVE_OK;
  KVE_REQUIRE(gate_up && out && rows > 0 && ffn > 0, "kve_silu_mul: bad arguments");
  KVE_REQUIRE(dtype == KVE_DTYPE_BF16 || dtype == KVE_DTYPE_F32, "kve_silu_mul: dtype %d", dtype);
  const int vn = dtype == KVE_DTYPE_BF16 ? 8 : 4;
  KVE_REQUIRE(ffn % vn == 0 && rows <= 65535, "kve_silu_mul: ffn %d must be a multiple of %d", ffn, vn);
  KVE_REQUIRE(aligned16(gate_up) && aligned16(out), "kve_silu_mul: buffers must be 16-byte aligned");
  const dim3 grid(cdiv(ffn / vn, 256), rows);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == KVE_DTYPE_BF16)
    hipLaunchKernelGGL(silu_mul_kernel<true>, grid, dim3(256), 0, st, gate_up, out, ffn);
  else
    hipLaunchKernelGGL(silu_mul_kernel<false>, grid, dim3(256), 0, st, gate_up, out, ffn);
  return check_launch("kve_silu_mul");
}

extern "C" int kve_pass_prologue(const int64_t* ids, const void* embed, int64_t vocab, int hidden,
                                 const int32_t* lens, const int32_t* seq_rows, int num_rows,
                                 int num_seqs, int q_len, const void* cos_table,
                                 const void* sin_table,
                                 int positions, int head_dim, void* hidden_out, void* cos_out,
                                 void* sin_out, void* stream) {
  clear_error();
  if (num_seqs == 0 || q_len == 0) return KVE_OK;
  KVE_REQUIRE(ids && embed && lens && seq_rows && cos_table && sin_table && hidden_out && cos_out &&
                  sin_out,
              "kve_pass_prologue: null pointer argument");
  KVE_REQUIRE(num_seqs > 0 && q_len > 0 && vocab > 0 && positions > 0 && num_rows > 0,
              "kve_pass_prologue: num_seqs %d q_len %d vocab %lld positions %d num_rows %d",
              num_seqs, q_len, static_cast<long long>(vocab), positions, num_rows);
  KVE_REQUIRE(hidden > 0 && hidden % 8 == 0 && head_dim > 0 && head_dim % 8 == 0,
              "kve_pass_prologue: hidden %d and head_dim %d must be multiples of 8", hidden, head_dim);
  const uintptr_t al = reinterpret_cast<uintptr_t>(embed) | reinterpret_cast<uintptr_t>(cos_table) |
                       reinterpret_cast<uintptr_t>(sin_table) |
                       reinterpret_cast<uintptr_t>(hidden_out) | reinterpret_cast<uintptr_t>(cos_out) |
                       reinterpret_cast<uintptr_t>(sin_out);
  KVE_REQUIRE((al & 15) == 0, "kve_pass_prologue: buffers must be 16-byte aligned");
  hipLaunchKernelGGL(pass_prologue_kernel, dim3(num_seqs * q_len), dim3(128), 0,
                     static_cast<hipStream_t>(stream), ids, static_cast<const uint16_t*>(embed),
                     vocab, hidden, lens, seq_rows, num_rows, q_len,
                     static_cast<const uint16_t*>(cos_table),
                     static_cast<const uint16_t*>(sin_table), positions, head_dim,
                     static_cast<uint16_t*>(hidden_out), static_cast<uint16_t*>(cos_out),
                     static_cast<uint16_t*>(sin_out));
  return check_launch("kve_pass_prologue");
}
