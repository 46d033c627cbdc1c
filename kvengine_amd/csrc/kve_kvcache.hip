// KV-cache bookkeeping kernels for the verify loop: scatter new K/V into paged
// slots, advance lengths, roll sequences back, and the greedy accept.
//
// These replace the host-side index arithmetic and index_copy_ of
// kvengine/paged.py (slot_indices 197-205, write 288-311, commit 333-342,
// truncate 344-380) and the Python accept loop of kvengine/speculative.py
// (169-197), so the loop never has to upload a block table or read back a
// token before the whole iteration is queued.

#include "kve_common.h"

#include <type_traits>

namespace kve {

// One workgroup per (sequence, token); threads cover (kv head, 16-byte chunk).
// K rows land token-major ([blk][h][off][:]); V is stored channel-major
// ([blk][h][:][off]) so each channel's 16 tokens are contiguous for the
// attention kernel's transposed operand.
template <bool BF16>
__global__ void kv_write_kernel(const void* k_new, const void* v_new, int64_t stride,
                                void* k_pool, void* v_pool, const int32_t* tables,
                                const int32_t* seq_rows, const int32_t* start_pos,
                                const int32_t* q_lens, int Tq, int Hkv, int D, int bs,
                                int max_blocks, int num_rows, int num_blocks) {
  using elem_t = std::conditional_t<BF16, uint16_t, float>;
  constexpr int VEC = 16 / sizeof(elem_t);
  const int i = blockIdx.x / Tq, t = blockIdx.x % Tq;
  const int T = q_lens ? min(q_lens[i], Tq) : Tq;
  if (t >= T) return;
  const int chunks = D / VEC;
  const int c = threadIdx.x;
  if (c >= Hkv * chunks) return;
  const int h = c / chunks, d0 = (c % chunks) * VEC;
  const int row = seq_rows ? seq_rows[i] : i;
  if (row < 0 || row >= num_rows) return;
  const int pos = start_pos[row] + t;
  if (pos < 0) return;
  const int lb = pos / bs;
  if (lb >= max_blocks) return;
  const int blk = tables[static_cast<size_t>(row) * max_blocks + lb];
  if (blk < 0 || blk >= num_blocks) return;
  const int off = pos % bs;
  const size_t src = (static_cast<size_t>(i) * Tq + t) * stride + h * D + d0;
  const elem_t* ks = static_cast<const elem_t*>(k_new) + src;
  const elem_t* vs = static_cast<const elem_t*>(v_new) + src;
  elem_t* kd = static_cast<elem_t*>(k_pool) + ((static_cast<size_t>(blk) * Hkv + h) * bs + off) * D + d0;
  *reinterpret_cast<u32x4*>(kd) = *reinterpret_cast<const u32x4*>(ks);
  elem_t vv[VEC];
  *reinterpret_cast<u32x4*>(vv) = *reinterpret_cast<const u32x4*>(vs);
  elem_t* vd = static_cast<elem_t*>(v_pool) + ((static_cast<size_t>(blk) * Hkv + h) * D + d0) * bs + off;
#pragma unroll
  for (int e = 0; e < VEC; ++e) vd[static_cast<size_t>(e) * bs] = vv[e];
}

__global__ void commit_kernel(int32_t* lens, int num_rows, const int32_t* seq_rows,
                              const int32_t* q_lens, int n, int q_len) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int row = seq_rows ? seq_rows[i] : i;
  if (row < 0 || row >= num_rows) return;
  lens[row] += q_lens ? q_lens[i] : q_len;
}

// One workgroup per sequence.
__global__ void rollback_kernel(int32_t* tables, int32_t* lens, int num_rows,
                                const int32_t* seq_rows, const int32_t* keep, int max_blocks,
                                int bs) {
  const int i = blockIdx.x;
  const int row = seq_rows ? seq_rows[i] : i;
  if (row < 0 || row >= num_rows) return;
  __shared__ int new_len;
  if (threadIdx.x == 0) new_len = min(lens[row], max(keep[i], 0));
  __syncthreads();
  const int nb = cdiv(new_len, bs);
  int32_t* tab = tables + static_cast<size_t>(row) * max_blocks;
  for (int e = nb + threadIdx.x; e < max_blocks; e += blockDim.x) tab[e] = -1;
  __syncthreads();
  if (threadIdx.x == 0) lens[row] = new_len;
}

__global__ void accept_kernel(const int32_t* drafts, const int32_t* preds, const int32_t* lens,
                              int num_rows, const int32_t* seq_rows, int n, int k, int32_t* n_acc,
                              int32_t* emitted, int32_t* keep) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t* d = drafts + static_cast<size_t>(i) * k;
  const int32_t* p = preds + static_cast<size_t>(i) * (k + 1);
  int a = 0;
  while (a < k && p[a] == d[a]) ++a;
  int32_t* e = emitted + static_cast<size_t>(i) * (k + 1);
  for (int j = 0; j <= k; ++j) e[j] = j < a ? d[j] : (j == a ? p[a] : -1);
  n_acc[i] = a;
  if (keep) {
    const int row = seq_rows ? seq_rows[i] : i;
    keep[i] = (row >= 0 && row < num_rows) ? lens[row] - k + a : 0;
  }
}

}  // namespace kve

using namespace kve;

extern "C" int kve_kv_write(const void* k_new, const void* v_new, int64_t src_token_stride,
                            void* k_pool, void* v_pool, const int32_t* block_tables,
                            const int32_t* seq_rows, const int32_t* start_pos,
                            const int32_t* q_lens, int num_seqs, int q_len, int num_kv_heads,
                            int head_dim, int block_size, int max_blocks, int num_rows,
                            int num_blocks, int dtype, void* stream) {
  clear_error();
  if (num_seqs == 0) return KVE_OK;
  KVE_REQUIRE(k_new && v_new && k_pool && v_pool && block_tables && start_pos,
              "kve_kv_write: null pointer argument");
  KVE_REQUIRE(num_seqs > 0 && q_len > 0 && num_kv_heads > 0 && block_size > 0 && max_blocks > 0 &&
                  num_rows > 0 && num_blocks > 0,
              "kve_kv_write: bad sizes");
  KVE_REQUIRE(dtype == KVE_DTYPE_BF16 || dtype == KVE_DTYPE_F32, "kve_kv_write: dtype %d", dtype);
  const int vec = dtype == KVE_DTYPE_BF16 ? 8 : 4;
  KVE_REQUIRE(head_dim > 0 && head_dim % vec == 0, "kve_kv_write: head_dim %d", head_dim);
  KVE_REQUIRE(src_token_stride >= static_cast<int64_t>(num_kv_heads) * head_dim &&
                  src_token_stride % vec == 0,
              "kve_kv_write: src_token_stride %lld", static_cast<long long>(src_token_stride));
  const int threads = num_kv_heads * head_dim / vec;
  KVE_REQUIRE(threads <= 1024, "kve_kv_write: %d threads per token", threads);
  const dim3 grid(num_seqs * q_len), block((threads + 63) / 64 * 64);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == KVE_DTYPE_BF16)
    hipLaunchKernelGGL(kv_write_kernel<true>, grid, block, 0, st, k_new, v_new, src_token_stride,
                       k_pool, v_pool, block_tables, seq_rows, start_pos, q_lens, q_len,
                       num_kv_heads, head_dim, block_size, max_blocks, num_rows, num_blocks);
  else
    hipLaunchKernelGGL(kv_write_kernel<false>, grid, block, 0, st, k_new, v_new, src_token_stride,
                       k_pool, v_pool, block_tables, seq_rows, start_pos, q_lens, q_len,
                       num_kv_heads, head_dim, block_size, max_blocks, num_rows, num_blocks);
  return check_launch("kve_kv_write");
}

extern "C" int kve_commit(int32_t* lens, int num_rows, const int32_t* seq_rows,
                          const int32_t* q_lens, int num_seqs, int q_len, void* stream) {
  clear_error();
  if (num_seqs == 0) return KVE_OK;
  KVE_REQUIRE(lens && num_seqs > 0 && num_rows > 0 && (q_lens || q_len >= 0),
              "kve_commit: bad arguments");
  hipLaunchKernelGGL(commit_kernel, dim3(cdiv(num_seqs, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), lens, num_rows, seq_rows, q_lens, num_seqs,
                     q_len);
  return check_launch("kve_commit");
}

extern "C" int kve_rollback(int32_t* block_tables, int32_t* lens, int num_rows,
                            const int32_t* seq_rows, const int32_t* keep_lens, int num_seqs,
                            int max_blocks, int block_size, void* stream) {
  clear_error();
  if (num_seqs == 0) return KVE_OK;
  KVE_REQUIRE(block_tables && lens && keep_lens && num_seqs > 0 && max_blocks > 0 &&
                  block_size > 0 && num_rows > 0,
              "kve_rollback: bad arguments");
  hipLaunchKernelGGL(rollback_kernel, dim3(num_seqs), dim3(64), 0,
                     static_cast<hipStream_t>(stream), block_tables, lens, num_rows, seq_rows,
                     keep_lens, max_blocks, block_size);
  return check_launch("kve_rollback");
}

extern "C" int kve_accept(const int32_t* drafts, const int32_t* preds, const int32_t* lens,
                          int num_rows, const int32_t* seq_rows, int num_seqs, int k,
                          int32_t* n_acc, int32_t* emitted, int32_t* keep_lens, void* stream) {
  clear_error();
  if (num_seqs == 0) return KVE_OK;
  KVE_REQUIRE(drafts && preds && n_acc && emitted && num_seqs > 0 && k >= 1,
              "kve_accept: bad arguments");
  KVE_REQUIRE(!keep_lens || (lens && num_rows > 0), "kve_accept: keep_lens needs lens");
  hipLaunchKernelGGL(accept_kernel, dim3(cdiv(num_seqs, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), drafts, preds, lens, num_rows, seq_rows,
                     num_seqs, k, n_acc, emitted, keep_lens);
  return check_launch("kve_accept");
}
