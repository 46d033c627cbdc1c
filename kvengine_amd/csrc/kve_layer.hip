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

// ---- RMSNorm (+ residual) ----------------------------------------------------
// One workgroup per row. torch's Qwen2RMSNorm: x.float(); var = x.pow(2).mean();
// x * rsqrt(var + eps); cast to the input dtype; weight * x (in the dtype).
template <bool BF16>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const void* x, const void* delta,
                                                      void* residual_out, const void* weight,
                                                      void* out, int H, float eps) {
  using E = Elem<BF16>;
  using T = typename E::T;
  extern __shared__ float sm_row[];
  __shared__ float sm_part[4];
  const int row = blockIdx.x;
  const T* xr = static_cast<const T*>(x) + static_cast<size_t>(row) * H;
  const T* dr = delta ? static_cast<const T*>(delta) + static_cast<size_t>(row) * H : nullptr;
  T* rr = residual_out ? static_cast<T*>(residual_out) + static_cast<size_t>(row) * H : nullptr;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < H; i += blockDim.x) {
    float v = E::ld(xr, i);
    if (dr) v = E::rnd(__fadd_rn(v, E::ld(dr, i)));  // residual add in the model dtype
    if (rr) rr[i] = E::cvt(v);
    sm_row[i] = v;
    ss = __fadd_rn(ss, __fmul_rn(v, v));
  }
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  if ((threadIdx.x & 63) == 0) sm_part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
  for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) tot += sm_part[w];
  const float inv = rsqrtf(__fadd_rn(__fmul_rn(tot, 1.0f / static_cast<float>(H)), eps));
  const T* wr = static_cast<const T*>(weight);
  T* orow = static_cast<T*>(out) + static_cast<size_t>(row) * H;
  for (int i = threadIdx.x; i < H; i += blockDim.x) {
    const float nv = E::rnd(__fmul_rn(sm_row[i], inv));
    orow[i] = E::cvt(__fmul_rn(E::ld(wr, i), nv));
  }
}

// ---- RoPE + KV write ---------------------------------------------------------
// One workgroup per token. qkv row: [Hq*D | Hkv*D | Hkv*D] (bias already added
// by the projection). cos/sin rows [D] in the model dtype (transformers computes
// them in float32 and casts). rotate_half(x)[d] = -x[d + D/2] (d < D/2), x[d - D/2].
template <bool BF16>
__global__ __launch_bounds__(256) void rope_kv_write_kernel(
    const void* qkv, const void* cos, const void* sin, void* q_out, void* k_pool, void* v_pool,
    const int32_t* tables, const int32_t* seq_rows, const int32_t* start_pos,
    const int32_t* q_lens, int Tq, int Hq, int Hkv, int D, int bs, int max_blocks, int num_rows,
    int num_blocks) {
  using E = Elem<BF16>;
  using T = typename E::T;
  const int tok = blockIdx.x;
  const int i = tok / Tq, t = tok % Tq;
  const int width = (Hq + 2 * Hkv) * D;
  const T* src = static_cast<const T*>(qkv) + static_cast<size_t>(tok) * width;
  const T* cr = static_cast<const T*>(cos) + static_cast<size_t>(tok) * D;
  const T* sr = static_cast<const T*>(sin) + static_cast<size_t>(tok) * D;
  const int half = D / 2;
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
  // rotated heads: Hq query heads then Hkv key heads, pairs (j, j + D/2)
  for (int idx = threadIdx.x; idx < (Hq + Hkv) * half; idx += blockDim.x) {
    const int h = idx / half, j = idx % half;
    const T* x = src + h * D;
    const float a = E::ld(x, j), bb = E::ld(x, j + half);
    const float lo = E::rnd(__fadd_rn(E::rnd(__fmul_rn(a, E::ld(cr, j))),
                                      E::rnd(__fmul_rn(-bb, E::ld(sr, j)))));
    const float hi = E::rnd(__fadd_rn(E::rnd(__fmul_rn(bb, E::ld(cr, j + half))),
                                      E::rnd(__fmul_rn(a, E::ld(sr, j + half)))));
    if (h < Hq) {
      T* qo = static_cast<T*>(q_out) + (static_cast<size_t>(tok) * Hq + h) * D;
      qo[j] = E::cvt(lo);
      qo[j + half] = E::cvt(hi);
    } else if (blk >= 0) {
      const int kh = h - Hq;
      T* kd = static_cast<T*>(k_pool) + ((static_cast<size_t>(blk) * Hkv + kh) * bs + off) * D;
      kd[j] = E::cvt(lo);
      kd[j + half] = E::cvt(hi);
    }
  }
  if (blk >= 0) {
    const T* vs = src + (Hq + Hkv) * D;
    for (int idx = threadIdx.x; idx < Hkv * D; idx += blockDim.x) {
      const int h = idx / D, d = idx % D;
      T* vd = static_cast<T*>(v_pool) + ((static_cast<size_t>(blk) * Hkv + h) * D + d) * bs + off;
      *vd = vs[idx];
    }
  }
}

// ---- SiLU * up -----------------------------------------------------------------
// gate_up row: [gate F | up F]; out = cast(silu(gate)) * up, each op rounded to
// the model dtype as torch does (silu computes x / (1 + exp(-x)) in float32).
template <bool BF16>
__global__ __launch_bounds__(256) void silu_mul_kernel(const void* gate_up, void* out, int M,
                                                       int F) {
  using E = Elem<BF16>;
  using T = typename E::T;
  const size_t n = static_cast<size_t>(M) * F;
  for (size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < n;
       idx += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t m = idx / F, f = idx % F;
    const T* row = static_cast<const T*>(gate_up) + m * 2 * F;
    const float g = E::ld(row, f);
    const float s = E::rnd(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))));
    static_cast<T*>(out)[idx] = E::cvt(__fmul_rn(s, E::ld(row, F + f)));
  }
}

}  // namespace kve

using namespace kve;

extern "C" int kve_rmsnorm(const void* x, const void* delta, void* residual_out,
                           const void* weight, void* out, int rows, int hidden, float eps,
                           int dtype, void* stream) {
  clear_error();
  if (rows == 0) return KVE_OK;
  KVE_REQUIRE(x && weight && out && rows > 0 && hidden > 0, "kve_rmsnorm: bad arguments");
  KVE_REQUIRE(hidden <= 16384, "kve_rmsnorm: hidden %d too large", hidden);
  KVE_REQUIRE(dtype == KVE_DTYPE_BF16 || dtype == KVE_DTYPE_F32, "kve_rmsnorm: dtype %d", dtype);
  const size_t lds = static_cast<size_t>(hidden) * sizeof(float);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == KVE_DTYPE_BF16)
    hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3(rows), dim3(256), lds, st, x, delta,
                       residual_out, weight, out, hidden, eps);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3(rows), dim3(256), lds, st, x, delta,
                       residual_out, weight, out, hidden, eps);
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
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(num_seqs * q_len);
  if (dtype == KVE_DTYPE_BF16)
    hipLaunchKernelGGL(rope_kv_write_kernel<true>, grid, dim3(256), 0, st, qkv, cos, sin, q_out,
                       k_pool, v_pool, block_tables, seq_rows, start_pos, q_lens, q_len,
                       num_q_heads, num_kv_heads, head_dim, block_size, max_blocks, num_rows,
                       num_blocks);
  else
    hipLaunchKernelGGL(rope_kv_write_kernel<false>, grid, dim3(256), 0, st, qkv, cos, sin, q_out,
                       k_pool, v_pool, block_tables, seq_rows, start_pos, q_lens, q_len,
                       num_q_heads, num_kv_heads, head_dim, block_size, max_blocks, num_rows,
                       num_blocks);
  return check_launch("kve_rope_kv_write");
}

extern "C" int kve_silu_mul(const void* gate_up, void* out, int rows, int ffn, int dtype,
                            void* stream) {
  clear_error();
  if (rows == 0) return KVE_OK;
  KVE_REQUIRE(gate_up && out && rows > 0 && ffn > 0, "kve_silu_mul: bad arguments");
  KVE_REQUIRE(dtype == KVE_DTYPE_BF16 || dtype == KVE_DTYPE_F32, "kve_silu_mul: dtype %d", dtype);
  const size_t n = static_cast<size_t>(rows) * ffn;
  const int blocks = static_cast<int>(std::min<size_t>((n + 255) / 256, 65536));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == KVE_DTYPE_BF16)
    hipLaunchKernelGGL(silu_mul_kernel<true>, dim3(blocks), dim3(256), 0, st, gate_up, out, rows,
                       ffn);
  else
    hipLaunchKernelGGL(silu_mul_kernel<false>, dim3(blocks), dim3(256), 0, st, gate_up, out, rows,
                       ffn);
  return check_launch("kve_silu_mul");
}
