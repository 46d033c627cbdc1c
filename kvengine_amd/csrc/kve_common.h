// Shared helpers for the gfx950 verify-path kernels: error reporting for the C
// ABI, bf16 bit handling, MFMA operand types and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/kve.h"

namespace kve {

// ---- error reporting -------------------------------------------------------

void set_error(const char* fmt, ...);
void clear_error();

#define KVE_REQUIRE(cond, ...)            \
  do {                                    \
    if (!(cond)) {                        \
      ::kve::set_error(__VA_ARGS__);      \
      return KVE_EINVAL;                  \
    }                                     \
  } while (0)

// Check the launch that was just issued; returns a negative code on failure.
int check_launch(const char* what);

// ---- types -----------------------------------------------------------------

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// bf16 bits -> float (exact)
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// float -> bf16 bits, round to nearest even; NaN stays NaN (quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// float rounded to bf16 and back to float
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Monotone map of a float to uint32 (larger float -> larger key); every NaN
// maps above +inf so it wins a max, matching torch.argmax.
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float unorder_key(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// ---- MFMA wrappers ----------------------------------------------------------
// All 16x16 MFMAs used here return C with lane l, register i holding
// C[4*(l/16) + i][l % 16]; A rows and B columns are indexed by l % 16, and A
// and B share the same lane -> k-slot assignment, so any consistent mapping of
// the reduction index onto k-slots gives the same product.

// 16x16x32 bf16 -> f32 (gfx950). a, b: 8 bf16 values (as 4 packed u32) per lane.
__device__ __forceinline__ f32x4 mfma16x16x32_bf16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// 16x16x16 bf16 -> f32. a, b: 4 bf16 values (as 2 packed u32) per lane.
__device__ __forceinline__ f32x4 mfma16x16x16_bf16(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                   __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
}

// 16x16x4 f32 -> f32. one value per lane.
__device__ __forceinline__ f32x4 mfma16x16x4_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---- wave reductions across the four 16-lane groups -------------------------
// Lanes l, l^16, l^32, l^48 hold the same row; gfx950's permlane swaps exchange
// the 32-lane halves and the odd/even 16-lane rows of a register inside the
// VALU, so a reduction over the four groups is two swaps and two ops, with no
// LDS round trip. swap32(x, x) gives {x[lower half] twice, x[upper half] twice};
// swap16(x, x) gives {even rows duplicated, odd rows duplicated}. Every lane of
// a row ends with the same value (a + b == b + a).

__device__ __forceinline__ float max_across_groups(float v) {
  const uint32_t u = __float_as_uint(v);
  const auto h = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  v = fmaxf(__uint_as_float(h[0]), __uint_as_float(h[1]));
  const uint32_t w = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane16_swap(w, w, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float sum_across_groups(float v) {
  const uint32_t u = __float_as_uint(v);
  const auto h = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  v = __uint_as_float(h[0]) + __uint_as_float(h[1]);
  const uint32_t w = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane16_swap(w, w, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over the whole wave, every lane gets the total: DPP moves inside each
// 16-lane row (swap neighbours, swap pairs, mirror halves, mirror the row),
// then the permlane swaps across rows. All VALU, no LDS traffic.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  return sum_across_groups(v);
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t max_across_groups_u64(uint64_t v) {
  {
    const uint32_t lo = static_cast<uint32_t>(v), hi = static_cast<uint32_t>(v >> 32);
    const auto l = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto h = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    v = umax64((static_cast<uint64_t>(h[0]) << 32) | l[0], (static_cast<uint64_t>(h[1]) << 32) | l[1]);
  }
  const uint32_t lo = static_cast<uint32_t>(v), hi = static_cast<uint32_t>(v >> 32);
  const auto l = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
  const auto h = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
  return umax64((static_cast<uint64_t>(h[0]) << 32) | l[0], (static_cast<uint64_t>(h[1]) << 32) | l[1]);
}

// ---- top-2 of 64-bit keys -----------------------------------------------------
// (a, b) holds the largest and second largest key seen, a > b (0 = none). Keys
// are distinct (they embed a unique index), so the merged pair of two sets is
// (max(a, a'), max(min(a, a'), max(b, b'))).

__device__ __forceinline__ void top2_insert(uint64_t& a, uint64_t& b, uint64_t k) {
  if (k > a) {
    b = a;
    a = k;
  } else if (k > b) {
    b = k;
  }
}

__device__ __forceinline__ void top2_merge(uint64_t& a, uint64_t& b, uint64_t a2, uint64_t b2) {
  const uint64_t lo = a < a2 ? a : a2;
  a = umax64(a, a2);
  b = umax64(lo, umax64(b, b2));
}

// The 64-bit value v of the lane in the other half (swap32) / other odd-even
// 16-lane row (swap16): permlane swaps of its two 32-bit words.
__device__ __forceinline__ uint64_t swap32_u64(uint64_t v) {
  const uint32_t lo = static_cast<uint32_t>(v), hi = static_cast<uint32_t>(v >> 32);
  const auto l = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
  const auto h = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
  // {own half, other half} in some order: the partner is the entry != own lane's
  const bool upper = (__lane_id() & 32) != 0;
  return upper ? ((static_cast<uint64_t>(h[0]) << 32) | l[0])
               : ((static_cast<uint64_t>(h[1]) << 32) | l[1]);
}

__device__ __forceinline__ uint64_t swap16_u64(uint64_t v) {
  const uint32_t lo = static_cast<uint32_t>(v), hi = static_cast<uint32_t>(v >> 32);
  const auto l = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
  const auto h = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
  const bool odd = (__lane_id() & 16) != 0;
  return odd ? ((static_cast<uint64_t>(h[0]) << 32) | l[0])
             : ((static_cast<uint64_t>(h[1]) << 32) | l[1]);
}

// Top-2 over the four 16-lane groups that hold the same row (lanes l, l^16,
// l^32, l^48); every lane of the row ends with the merged pair.
__device__ __forceinline__ void top2_across_groups(uint64_t& a, uint64_t& b) {
  uint64_t a2 = swap32_u64(a), b2 = swap32_u64(b);
  top2_merge(a, b, a2, b2);
  a2 = swap16_u64(a);
  b2 = swap16_u64(b);
  top2_merge(a, b, a2, b2);
}

// Two floats -> packed bf16 pair (low half = a), round to nearest even, with
// gfx950's conversion instruction.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t x = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, bf16x2_t));
}

// float -> float rounded to bf16 (nearest even), with the conversion instruction
__device__ __forceinline__ float round_bf16_hw(float x) {
  return __uint_as_float(pack_bf16x2(x, 0.0f) << 16);
}

__host__ __device__ constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }

// Blocked layout of a bf16 [R, C] matrix (C a multiple of 32, R padded up to a
// multiple of 16 in the allocation): 16-row x 32-column blocks of 1 KB, row
// tiles outermost; element (r, c) sits at blk_off(r, c, C). A DMA chunk of the
// projections (16-row tiles x 1-4 k-steps of 32) then reads whole 512-byte runs
// instead of one 64-128 byte piece per row.
__host__ __device__ __forceinline__ size_t blk_off(int r, int c, int cols) {
  return (static_cast<size_t>(r >> 4) * (cols >> 5) + (c >> 5)) * 512 + (r & 15) * 32 + (c & 31);
}
// element offset of (r, c) in the row-major (ld = row stride) or blocked layout
__host__ __device__ __forceinline__ size_t mat_off(int r, int c, int cols, int64_t ld, bool blocked) {
  return blocked ? blk_off(r, c, cols) : static_cast<size_t>(r) * ld + c;
}

}  // namespace kve
