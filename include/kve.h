/*
 * kve.h - C ABI of the MI355X (gfx950) verify-path library libkve (_kve.so).
 *
 * Plain pointers and sizes only. Every pointer is device memory owned by the
 * caller (PyTorch tensors in the Python host); the library never allocates.
 * `stream` is a hipStream_t passed as void* (torch's current stream); every
 * entry point is stream-ordered and never synchronises the host.
 *
 * Return value: 0 on success, a negative KVE_E* code otherwise; the message of
 * the last failure on the calling thread is available from kve_last_error().
 *
 * Paged pool layout for ONE layer (the caller passes a layer's slice):
 *   K: [num_blocks, num_kv_heads, block_size, head_dim]   (token-major per head)
 *   V: [num_blocks, num_kv_heads, head_dim, block_size]   (channel-major per head)
 * so the 16 tokens of one (block, kv head) are one contiguous 2-4 KB tile of K
 * and one of V. The reference keeps [num_blocks, block_size, num_kv_heads,
 * head_dim] for both (kvengine/paged.py:59-61); the logical content addressed
 * through a block table is the same, only the in-block order differs.
 *
 * Sequence indexing: a launch covers `num_seqs` sequences; sequence i uses
 * row seq_rows[i] of `block_tables` ([num_rows, max_blocks] int32) and of the
 * per-row length array (seq_rows == NULL means row i). A length is the number
 * of tokens already committed to the cache for that row (the reference's
 * PagedSequenceCache.length, kvengine/paged.py:149-151).
 *
 * Device-side values are range-checked inside the kernels so that a bad table
 * can never address memory outside the buffers: a sequence whose row is
 * >= num_rows, or whose history exceeds max_ctx, is skipped; a block id outside
 * [0, num_blocks) is never dereferenced (attention reads block 0 instead and
 * the KV write drops the row). Such results are wrong by construction; the
 * host allocator never produces them.
 */
#ifndef KVE_H
#define KVE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVE_DTYPE_F32 0
#define KVE_DTYPE_BF16 1

/*
 * Matrix layouts of the projections' operands (the `layout` argument).
 * KVE_LAYOUT_ROWS: row-major. KVE_LAYOUT_BLOCKED: a bf16 [R, C] matrix (C a
 * multiple of 32) stored as 16-row x 32-column blocks of 1 KB, row tiles
 * outermost: element (r, c) at ((r / 16) * (C / 32) + c / 32) * 512 +
 * (r % 16) * 32 + c % 32; the allocation holds R rounded up to 16 rows. No
 * counterpart in the reference (a storage order only; every sum is the same):
 * the projections' direct-to-LDS loads then read whole 512-byte runs instead
 * of one short piece per row, so a producer (kve_rmsnorm, kve_residual_norm,
 * kve_paged_verify_attn, kve_gate_up_silu) can hand its output blocked to the
 * projection that reads it, with weights copied once into the blocked layout.
 */
#define KVE_LAYOUT_ROWS 0
#define KVE_LAYOUT_BLOCKED 1

#define KVE_OK 0
#define KVE_EINVAL (-1)     /* bad shape, pointer, dtype or size */
#define KVE_EWORKSPACE (-2) /* workspace too small */
#define KVE_ELAUNCH (-3)    /* HIP launch or runtime error */
#define KVE_EUNSUPPORTED (-4)

/* Message of the last failure on this thread ("" if none). */
const char* kve_last_error(void);

/* Library version string and the gfx target it was built for. */
const char* kve_version(void);

/*
 * Paged GQA verify attention for one layer.
 *
 * Replaces, per layer, the reference's gather-then-attend:
 *   PagedSequenceCache._gather        kvengine/paged.py:315-331
 *   repeat_kv                         kvengine/forward.py:72-82
 *   causal_mask                       kvengine/forward.py:85-103
 *   attend (SDPA / eager)             kvengine/forward.py:106-144
 * for a whole batch in one launch (the reference attends one sequence at a time).
 *
 * q:   [num_seqs, q_len, num_q_heads, head_dim] (dtype), contiguous
 * out: same shape as q
 * start_pos[row]: committed length before this pass; query t of sequence i sits
 *      at absolute position start_pos[row]+t and sees keys 0..start_pos[row]+t,
 *      which must already be written (kve_kv_write) for this layer
 * q_lens: per-sequence query count (NULL: all q_len); rows past it are left
 *      untouched in `out`
 * max_ctx: upper bound on start_pos[row]+q_len over the batch (sizes the plan;
 *      sequences longer than this are not read)
 * unit_blocks, key_waves: how a row's keys are summed. A sequence's history is
 *      cut into units of unit_blocks 16-token tiles at fixed offsets, each
 *      unit summed by key_waves waves (bursts at fixed offsets), the waves'
 *      and then the units' partial softmax states folded in order. With both
 *      fixed (> 0), a row's result depends only on its query and its keys: not
 *      on q_len, the rest of the batch, or how many units its history has.
 *      0 chooses each from the launch's shape (fastest, not batch-invariant).
 *      unit_blocks <= 56 tiles; key_waves in {1, 2, 4, 8}.
 * scale: softmax scale (head_dim ** -0.5 for Qwen2)
 * plan: a plan written by kve_attn_plan for the same tables, lengths and shape
 *      parameters (every layer of a forward pass can share one), or NULL: the
 *      plan is then built in the workspace first (one more small launch)
 * workspace: kve_attn_workspace_bytes(...) bytes, 256-byte aligned (the units'
 *      partial states of long histories, and the plan when plan is NULL); no
 *      initialisation needed. When max_ctx allows a history of more than one
 *      unit, a second small kernel merges their states on `stream`.
 * head_dim must be 64 or 128; num_q_heads a multiple of num_kv_heads.
 * layout: `out` as [num_seqs * q_len, num_q_heads * head_dim] row-major
 *      (KVE_LAYOUT_ROWS, the q shape) or blocked (bf16 only).
 */
size_t kve_attn_workspace_bytes(int num_seqs, int q_len, int num_q_heads, int num_kv_heads,
                                int head_dim, int block_size, int max_ctx, int unit_blocks,
                                int key_waves, int dtype);

int kve_paged_verify_attn(const void* q, const void* k_pool, const void* v_pool,
                          const int32_t* block_tables, const int32_t* seq_rows,
                          const int32_t* start_pos, const int32_t* q_lens, int num_seqs,
                          int q_len, int num_q_heads, int num_kv_heads, int head_dim,
                          int block_size, int max_blocks, int num_rows, int num_blocks,
                          int max_ctx, int unit_blocks, int key_waves, float scale, int dtype,
                          const void* plan, void* out, void* workspace, size_t workspace_bytes,
                          int layout, void* stream);

/*
 * Work plan of kve_paged_verify_attn for one forward pass: the units of every
 * (sequence, row group) with their block ids. The per-sequence half of the
 * reference's gather (kvengine/paged.py:315-331: which blocks a sequence's
 * history occupies), resolved once for all layers of a pass instead of per
 * layer. Same shape arguments as kve_paged_verify_attn; plan: a 16-byte
 * aligned buffer of kve_attn_plan_bytes(...) bytes. Tables and lengths must
 * not change between this call and the attention launches that use the plan.
 */
size_t kve_attn_plan_bytes(int num_seqs, int q_len, int num_q_heads, int num_kv_heads,
                           int head_dim, int block_size, int max_ctx, int unit_blocks,
                           int key_waves, int dtype);

int kve_attn_plan(const int32_t* block_tables, const int32_t* seq_rows, const int32_t* start_pos,
                  const int32_t* q_lens, int num_seqs, int q_len, int num_q_heads,
                  int num_kv_heads, int head_dim, int block_size, int max_blocks, int num_rows,
                  int num_blocks, int max_ctx, int unit_blocks, int key_waves, int dtype,
                  void* plan, size_t plan_bytes, void* stream);

/*
 * Scatter the new K/V rows of one layer into their paged slots.
 *
 * Replaces PagedSequenceCache.slot_indices + write's index_copy_
 * (kvengine/paged.py:197-205, 288-311) for a whole batch.
 * k_new/v_new: token (i, t) starts at k_new + (i*q_len + t)*src_token_stride
 *      elements and holds [num_kv_heads, head_dim] contiguous values.
 * Token t of sequence i goes to position start_pos[row]+t, i.e. block
 * block_tables[row][pos/block_size], offset pos%block_size. The table entries
 * must already hold allocated blocks (the host reserve()).
 */
int kve_kv_write(const void* k_new, const void* v_new, int64_t src_token_stride, void* k_pool,
                 void* v_pool, const int32_t* block_tables, const int32_t* seq_rows,
                 const int32_t* start_pos, const int32_t* q_lens, int num_seqs, int q_len,
                 int num_kv_heads, int head_dim, int block_size, int max_blocks, int num_rows,
                 int num_blocks, int dtype, void* stream);

/*
 * Advance committed lengths after a forward pass: lens[row] += q_len (or q_lens[i]).
 * Replaces PagedSequenceCache.commit (kvengine/paged.py:333-342); capacity is
 * checked by the host before the pass.
 */
int kve_commit(int32_t* lens, int num_rows, const int32_t* seq_rows, const int32_t* q_lens,
               int num_seqs, int q_len, void* stream);

/*
 * Roll sequences back: lens[row] = min(lens[row], keep_lens[i]) and every table
 * entry at or past ceil(new_len/block_size) becomes -1.
 * Replaces the table/length half of PagedSequenceCache.truncate
 * (kvengine/paged.py:344-380) as driven by speculative.py:193-197
 * (truncate(min(length, keep))). The host allocator frees the same blocks in
 * table order.
 */
int kve_rollback(int32_t* block_tables, int32_t* lens, int num_rows, const int32_t* seq_rows,
                 const int32_t* keep_lens, int num_seqs, int max_blocks, int block_size,
                 void* stream);

/*
 * LM head with fused row argmax: logits = hidden . weight^T (tied embedding,
 * no bias), rounded to the model dtype exactly as the reference's logits are,
 * then the first index of the row maximum (torch.argmax semantics; a NaN counts
 * as the maximum), and optionally the runner-up for top-2 margin accounting.
 *
 * Replaces model.lm_head(hidden) + torch.argmax (kvengine/forward.py:215,
 * kvengine/speculative.py:155,167) for the rows the loop reads.
 * hidden: [M, H] with row stride hidden_row_stride elements; weight: [V, H]
 * argmax: [M] int32; maxval: [M] float (the rounded row maximum) or NULL
 * second_id, second_val: [M] int32 / float or NULL: the largest rounded logit
 *      at any id other than argmax[m] and its id (lowest id among equal
 *      logits, so a tie at the top gives second_val == maxval); asking for
 *      either adds a second atomic per workgroup and row
 * workspace: kve_lmhead_workspace_bytes(M) bytes, zero-filled once before first
 *      use; every launch leaves it zeroed again
 * H must be a multiple of 32.
 * layout: KVE_LAYOUT_BLOCKED reads hidden [M, H] and weight [V, H] both blocked
 *      (bf16, V a multiple of 16; hidden_row_stride unused).
 */
size_t kve_lmhead_workspace_bytes(int M);

int kve_lmhead_argmax(const void* hidden, int64_t hidden_row_stride, const void* weight, int M,
                      int H, int V, int dtype, int32_t* argmax, float* maxval, int32_t* second_id,
                      float* second_val, void* workspace, size_t workspace_bytes, int layout,
                      void* stream);

/*
 * kve_lmhead_argmax_noalloc: kve_lmhead_argmax (same arguments, results and
 * kernels) without a workspace argument and without any allocation. It has no
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid hipMalloc).
 * The key copies live in a file-scope device array of
 * KVE_LMHEAD_NOALLOC_MAX_ROWS * 64 * 2 keys (256 KiB on each GPU the library
 * runs on, held until the process ends); M above KVE_LMHEAD_NOALLOC_MAX_ROWS is
 * rejected with KVE_EINVAL before anything is launched. Every call on a GPU
 * shares that GPU's array: calls that overlap in time on one GPU (two streams,
 * two host threads) race, and the caller must serialise them. The first call
 * on a device resolves the array's address and clears it on `stream`.
 */
#define KVE_LMHEAD_NOALLOC_MAX_ROWS 256

int kve_lmhead_argmax_noalloc(const void* hidden, int64_t hidden_row_stride, const void* weight,
                              int M, int H, int V, int dtype, int32_t* argmax, float* maxval,
                              int32_t* second_id, float* second_val, void* stream);

/*
 * Greedy accept: n_acc[i] = longest prefix with preds[i][j] == drafts[i][j];
 * emitted[i] = drafts[i][:n_acc] + [preds[i][n_acc]] padded with -1 to k+1;
 * keep_lens[i] = lens[row] - k + n_acc[i] (the target's length after rollback
 * when lens already includes the k drafts).
 * Replaces the accept loop and keep arithmetic of kvengine/speculative.py:169-197.
 * drafts: [num_seqs, k]; preds: [num_seqs, k+1] (argmax of rows u-1..u-1+k)
 */
int kve_accept(const int32_t* drafts, const int32_t* preds, const int32_t* lens, int num_rows,
               const int32_t* seq_rows, int num_seqs, int k, int32_t* n_acc,
               int32_t* emitted, int32_t* keep_lens, void* stream);

/*
 * Fused per-layer elementwise kernels (model dtype bf16 or f32). Each rounds
 * at the same points as the torch ops it replaces in transformers' Qwen2
 * layer as driven by kvengine/forward.py:190-207.
 *
 * kve_rmsnorm: r = x (+ delta, rounded to the dtype); if residual_out, r is
 * stored there; out = weight * cast(r * rsqrt(mean(r*r) + eps)).
 * Replaces Qwen2RMSNorm (modeling_qwen2.py:237-255) and, with delta, the
 * residual add before it (forward.py:204-207). x, delta, residual_out, out:
 * [rows, hidden] contiguous; residual_out may alias x. layout: `out` row-major
 * or blocked (bf16, hidden % 32 == 0); x, delta and residual_out stay row-major.
 */
int kve_rmsnorm(const void* x, const void* delta, void* residual_out, const void* weight,
                void* out, int rows, int hidden, float eps, int dtype, int layout, void* stream);

/*
 * kve_rope_kv_write: from the fused QKV projection rows
 * qkv [num_seqs*q_len, (Hq + 2*Hkv)*D] (bias included) and cos/sin
 * [num_seqs*q_len, D] (model dtype), apply rotary embedding to the q and k heads
 * (x*cos + rotate_half(x)*sin, forward.py:49-69), write the rotated queries to
 * q_out [num_seqs*q_len, Hq, D], and scatter rotated k and plain v into the
 * pool at positions start_pos[row] + t exactly as kve_kv_write does (tokens
 * past q_lens[i] are not written). Replaces apply_rope + cache.write's
 * index_copy_ (forward.py:198-201, paged.py:288-311).
 */
int kve_rope_kv_write(const void* qkv, const void* cos, const void* sin, void* q_out,
                      void* k_pool, void* v_pool, const int32_t* block_tables,
                      const int32_t* seq_rows, const int32_t* start_pos, const int32_t* q_lens,
                      int num_seqs, int q_len, int num_q_heads, int num_kv_heads, int head_dim,
                      int block_size, int max_blocks, int num_rows, int num_blocks, int dtype,
                      void* stream);

/*
 * kve_silu_mul: out[m, f] = cast(silu(gate_up[m, f])) * gate_up[m, F + f] for the
 * fused gate/up projection [rows, 2F]; out [rows, F]. Replaces
 * act_fn(gate_proj(x)) * up_proj(x) (modeling_qwen2.py:35-48).
 */
int kve_silu_mul(const void* gate_up, void* out, int rows, int ffn, int dtype, void* stream);

/*
 * kve_pass_prologue: the inputs of a forward pass's layer loop in one launch
 * (embed_tokens and rotary_emb ahead of it, kvengine/forward.py:176-184):
 * for row m = b * q_len + t, hidden_out[m] = embed[ids[m]] (zero for an id
 * outside [0, vocab)) and cos_out/sin_out[m] = cos/sin_table[min(lens[seq_rows[b]]
 * + t, positions - 1)]; lens holds num_rows entries and a seq_rows entry outside
 * [0, num_rows) is never dereferenced (its tokens take positions t = 0, 1, ...).
 * bf16; ids int64 [num_seqs * q_len]; tables [positions, head_dim]; outputs
 * [num_seqs * q_len, hidden] and [num_seqs * q_len, head_dim].
 */
int kve_pass_prologue(const int64_t* ids, const void* embed, int64_t vocab, int hidden,
                      const int32_t* lens, const int32_t* seq_rows, int num_rows, int num_seqs,
                      int q_len, const void* cos_table, const void* sin_table, int positions,
                      int head_dim, void* hidden_out, void* cos_out, void* sin_out, void* stream);

/*
 * Fused skinny projections for decode-sized batches (bf16 only, rows =
 * num_seqs*q_len <= 64). Weights are nn.Linear layout [out, in], row-major
 * (layout KVE_LAYOUT_ROWS) or blocked (KVE_LAYOUT_BLOCKED: a wave's 16-row x
 * 32-column weight fragment is then one contiguous 1 KB load); the other
 * operands are row-major either way.
 * Each rounds to bf16 where the reference's module sequence does, so the
 * result equals the unfused kernels' up to the float32 summation order of the
 * dot products and of RMSNorm's mean.
 *
 * kve_fused_qkv: x = RMSNorm(residual) (Qwen2RMSNorm, modeling_qwen2.py:237-255),
 * qkv = x W^T + b for the [q|k|v] weight [(Hq + 2*Hkv)*D, hidden]
 * (q_proj/k_proj/v_proj, modeling_qwen2.py:175-234 as driven by
 * forward.py:190-197), then exactly kve_rope_kv_write: rotated q to q_out
 * [rows, Hq, D], rotated k and plain v into the pool at start_pos[row] + t.
 * residual [rows, hidden]; cos/sin [rows, D]. hidden % 32 == 0 and the
 * normalised rows must fit in LDS (rows rounded up to 16 times (hidden + 8)
 * bf16 plus the head tile: up to hidden 896 at 64 rows, 2048 at 32).
 */
int kve_fused_qkv(const void* residual, const void* norm_weight, float eps, const void* weight,
                  const void* bias, const void* cos, const void* sin, void* q_out, void* k_pool,
                  void* v_pool, const int32_t* block_tables, const int32_t* seq_rows,
                  const int32_t* start_pos, const int32_t* q_lens, int num_seqs, int q_len,
                  int hidden, int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                  int max_blocks, int num_rows, int num_blocks, int layout, void* stream);

/*
 * kve_linear_residual: residual[m, n] = residual[m, n] + cast(x[m, :] . weight[n, :])
 * in place, both terms bf16 (o_proj / down_proj plus the residual add,
 * forward.py:202-207). x [rows, in], weight [out, in], residual [rows, out];
 * out % 16 == 0, in % 32 == 0.
 */
int kve_linear_residual(const void* x, const void* weight, void* residual, int rows,
                        int out_features, int in_features, int layout, void* stream);

/*
 * kve_fused_gate_up: x = RMSNorm(residual); g, u = x Wg^T, x Wu^T for the
 * [gate|up] weight [2*ffn, hidden]; act = cast(silu(g)) * u, act [rows, ffn]
 * (post_attention_layernorm + Qwen2MLP up to down_proj, modeling_qwen2.py:35-48).
 * hidden % 32 == 0, ffn % 32 == 0, same LDS limit as kve_fused_qkv. layout is
 * the weight's; act_layout KVE_LAYOUT_BLOCKED writes act as a blocked matrix
 * (rows padded to 16, the padding rows left unwritten) for kve_linear_splitk.
 */
int kve_fused_gate_up(const void* residual, const void* norm_weight, float eps, const void* weight,
                      void* act, int rows, int hidden, int ffn, int layout, int act_layout,
                      void* stream);

/*
 * Split-K layers (bf16): the decode layer (rows <= 64) and the wide layer
 * (rows <= 160, its QKV projection also split, kve_qkv_part_rope). The same
 * Qwen2 layer as the entry points above (modeling_qwen2.py:35-48, 237-255
 * called from kvengine/forward.py:190-207), cut differently: every projection
 * is split into k-slices so that hundreds of workgroups share the weight
 * stream, and the slices are reduced by the kernel that consumes them. Slice
 * counts and bounds depend only on the weight shape and all sums run in a
 * fixed order, so a row's result does not depend on the other rows of the
 * batch.
 */

/* k-slices kve_linear_splitk uses for an [out_features, in_features] weight (1..8). */
int kve_splitk_slices(int out_features, int in_features);

/*
 * kve_linear_splitk: partials[s, m, n] = x[m, slice s] . weight[n, slice s] in
 * float32, s < slices = kve_splitk_slices(out, in) (any other count is an
 * error). x [rows, in] bf16, weight [out, in] bf16, partials [slices, rows, out].
 * out % 64 == 0, in % 32 == 0, rows <= 160. layout: x and weight both
 * row-major or both blocked; partials are row-major either way.
 */
int kve_linear_splitk(const void* x, const void* weight, float* partials, int rows,
                      int out_features, int in_features, int slices, int layout, void* stream);

/*
 * kve_residual_norm: residual = cast(residual + cast(sum_s partials[s])) in
 * place (slices summed in order 0, 1, ...), then xn = RMSNorm(residual) with
 * norm_weight (the residual add after o_proj / down_proj and the following
 * Qwen2RMSNorm, forward.py:202-207). residual, xn [rows, hidden] bf16;
 * hidden % 4 == 0, hidden <= 2048, slices <= 16. layout: xn row-major or
 * blocked (hidden % 32 == 0); the residual stays row-major.
 */
int kve_residual_norm(const float* partials, int slices, void* residual, const void* norm_weight,
                      float eps, void* xn, int rows, int hidden, int layout, void* stream);

/*
 * kve_kv_slots: pool slot (block * block_size + offset) of token t of sequence
 * i at slots[i * q_len + t], -1 where nothing is to be written (t >= q_lens[i],
 * bad row, position outside the table, block id outside the pool). The
 * per-token address computation of PagedSequenceCache.write
 * (kvengine/paged.py:288-331), done once per forward pass.
 */
int kve_kv_slots(const int32_t* block_tables, const int32_t* seq_rows, const int32_t* start_pos,
                 const int32_t* q_lens, int num_seqs, int q_len, int block_size, int max_blocks,
                 int num_rows, int num_blocks, int32_t* slots, void* stream);

/*
 * kve_qkv_rope: [q|k|v] = xn W^T + bias from normalised rows xn [rows, hidden];
 * q and k rotated (apply_rotary_pos_emb, forward.py:55-69), q to q_out
 * [rows, Hq, D], k and v written to the pools at `slots` (kve_kv_slots; -1
 * writes nothing). Same layouts and rounding as kve_fused_qkv. layout: xn and
 * weight both row-major or both blocked.
 */
int kve_qkv_rope(const void* xn, const void* weight, const void* bias, const void* cos,
                 const void* sin, const int32_t* slots, void* q_out, void* k_pool, void* v_pool,
                 int rows, int hidden, int num_q_heads, int num_kv_heads, int head_dim,
                 int block_size, int layout, void* stream);

/*
 * kve_qkv_part_rope: the same outputs as kve_qkv_rope from the k-slice partial
 * products of the [q|k|v] projection (kve_linear_splitk of xn with the
 * [q|k|v] weight; partials [slices, rows, (Hq + 2 Hkv) * head_dim] fp32):
 * each column's slices are summed in slice order, bias added, the result
 * rounded to bf16, then RoPE and the q / K / V writes. For rows <= 160
 * (kve_linear_splitk's limit); a row's result does not depend on `rows`.
 */
int kve_qkv_part_rope(const float* partials, int slices, const void* bias, const void* cos,
                      const void* sin, const int32_t* slots, void* q_out, void* k_pool,
                      void* v_pool, int rows, int num_q_heads, int num_kv_heads, int head_dim,
                      int block_size, void* stream);

/*
 * kve_gate_up_silu: act = cast(silu(xn Wg^T)) * (xn Wu^T) for normalised rows
 * xn [rows <= 160, hidden] and the [gate|up] weight [2*ffn, hidden] (Qwen2MLP
 * up to down_proj, modeling_qwen2.py:35-48). A row's result does not depend
 * on `rows`. layout: xn, weight and act all row-major or all blocked.
 */
int kve_gate_up_silu(const void* xn, const void* weight, void* act, int rows, int hidden, int ffn,
                     int layout, void* stream);

/*
 * kve_linear_rows: the split-K layer's projections for any number of rows (a
 * prefill, the recompute of a preempted request), each row bit-identical to
 * what kve_linear_splitk + its reduction, or kve_gate_up_silu, give that row
 * in a pass of at most 160 rows (the q/k/v/o/gate/up/down Linear calls of
 * forward.py:190-207 over a whole prompt). x [rows, in] bf16, weight [out, in]
 * bf16, in % 64 == 0, out % 128 == 0.
 *   mode 0, 1: out = fp32 partials [S, rows, out], S = kve_linear_rows_slices(...):
 *           S = 1 holds the slices' whole sum in kve_residual_norm's order
 *           (mode 0) or kve_qkv_part_rope's (mode 1); S > 1 holds every
 *           k-slice as kve_linear_splitk does (chosen when the row count is
 *           too small to fill the chip otherwise). Finish with
 *           kve_residual_norm / kve_qkv_part_rope(out, S, ...).
 *   mode 2: weight = [gate|up] [2 ffn, in]; out [rows, ffn] bf16 =
 *           kve_gate_up_silu's act. out_features = 2 ffn.
 * layout: x and weight (and mode 2's out) all row-major or all blocked; the
 *      fp32 partials are row-major either way.
 */
int kve_linear_rows(const void* x, const void* weight, void* out, int rows, int out_features,
                    int in_features, int mode, int layout, void* stream);

/* Slices kve_linear_rows writes for these sizes on the current device (0: bad sizes). */
int kve_linear_rows_slices(int rows, int out_features, int in_features, int mode);

#ifdef __cplusplus
}
#endif

#endif /* KVE_H */
