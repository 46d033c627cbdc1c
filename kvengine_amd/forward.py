"""The Qwen2 forward pass over a paged cache, with HIP attention and KV write.

Same layer loop as kvengine/forward.py:147-215 (and the same module calls, so
embedding, RMSNorm, projections, RoPE and MLP round exactly as there), with the
cache access replaced:

* the reference calls cache.write (index_copy_ + gather of the whole history,
  paged.py:288-331) and then attend (repeat_kv + SDPA, forward.py:106-144);
* here each layer launches the KV-write kernel for the new rows and the paged
  verify-attention kernel, which reads K/V through the device block table.

`forward_hidden` runs a batch of sequences (B rows of T tokens, optionally
ragged through q_lens) and returns the final-normed hidden states, leaving the
LM head to the caller (the spec loop fuses it with argmax).
`forward_with_own_cache` keeps the reference's single-request signature.
"""

from __future__ import annotations

import os

import torch

from . import kernels
from .paged import DeviceKV

USE_SDPA = os.environ.get("KVENGINE_EAGER_ATTN", "0") != "1"


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat([-x[..., half:], x[..., :half]], dim=-1)


def apply_rope(q, k, cos, sin, unsqueeze_dim: int = 1):
    """x*cos + rotate_half(x)*sin (kvengine/forward.py:55-69); cos/sin [B, T, D]
    broadcast over the head axis at `unsqueeze_dim`."""
    cos = cos.unsqueeze(unsqueeze_dim)
    sin = sin.unsqueeze(unsqueeze_dim)
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """[B, Hkv, T, D] -> [B, Hkv*n_rep, T, D]; q head h reads kv head h // n_rep."""
    if n_rep == 1:
        return x
    b, h, t, d = x.shape
    return x[:, :, None].expand(b, h, n_rep, t, d).reshape(b, h * n_rep, t, d)


def causal_mask(q_len: int, kv_len: int, dtype, device):
    """Additive mask; query i sits at kv_len - q_len + i; None for one query."""
    if q_len == 1:
        return None
    q_pos = torch.arange(kv_len - q_len, kv_len, device=device).unsqueeze(1)
    k_pos = torch.arange(kv_len, device=device).unsqueeze(0)
    mask = torch.zeros(q_len, kv_len, dtype=dtype, device=device)
    mask.masked_fill_(k_pos > q_pos, torch.finfo(dtype).min)
    return mask[None, None]


def attend(attn_module, q, k, v, mask, use_sdpa: bool | None = None):
    """Dense attention over gathered K/V (API compatibility; the forward pass uses
    the paged kernel). q [B, Hq, T, D], k/v [B, Hkv, L, D] -> [B, T, Hq, D]."""
    use_sdpa = USE_SDPA if use_sdpa is None else use_sdpa
    k = repeat_kv(k, attn_module.num_key_value_groups)
    v = repeat_kv(v, attn_module.num_key_value_groups)
    if use_sdpa:
        out = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask,
                                                               scale=attn_module.scaling)
        return out.transpose(1, 2).contiguous()
    scores = torch.matmul(q, k.transpose(2, 3)) * attn_module.scaling
    if mask is not None:
        scores = scores + mask
    probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(q.dtype)
    return torch.matmul(probs, v).transpose(1, 2).contiguous()


class LayerAttention:
    """The paged verify-attention launches of one forward pass: one work plan
    (kve_attn_plan) shared by every layer, and the summation order `attn` =
    (unit_blocks, key_waves) of kve_paged_verify_attn ((0, 0): chosen per
    launch; fixed values make a row's result independent of the batch)."""

    def __init__(self, kv: DeviceKV, rows, B: int, T: int, Hq: int, max_ctx: int, q_lens,
                 dtype, attn: tuple[int, int] = (0, 0)):
        self.kv, self.rows, self.q_lens, self.max_ctx = kv, rows, q_lens, max_ctx
        self.unit_blocks, self.key_waves = attn
        _, NB, Hkv, bs, D = kv.k.shape
        self.plan = kernels.attn_plan(kv.tables, kv.lens, B, T, Hq, Hkv, D, bs, NB, max_ctx, dtype,
                                      seq_rows=rows, q_lens=q_lens, unit_blocks=self.unit_blocks,
                                      key_waves=self.key_waves)

    def __call__(self, q, li: int, scale: float, out=None, blocked: bool = False):
        kv = self.kv
        return kernels.paged_verify_attn(q, kv.k[li], kv.v[li], kv.tables, kv.lens, self.max_ctx,
                                         seq_rows=self.rows, q_lens=self.q_lens, scale=scale,
                                         unit_blocks=self.unit_blocks, key_waves=self.key_waves,
                                         plan=self.plan, out=out, blocked=blocked)


def _q_heads(model, kv: DeviceKV) -> int:
    return model.model.layers[0].self_attn.num_key_value_groups * kv.k.shape[2]


def _fusable(model) -> bool:
    layers = model.model.layers
    if not len(layers) or getattr(layers[0].self_attn, "qkv_weight", None) is None:
        return False
    return layers[0].self_attn.qkv_weight.dtype in (torch.bfloat16, torch.float32)


# Decode-sized bf16 batches (<= 64 rows) skip hipBLASLt. "splitk" (default):
# every projection is cut into k-slices over the whole chip, the o_proj and
# down_proj partial sums are reduced by a kernel that also adds the residual and
# applies the next RMSNorm, and the QKV and gate/up projections take the
# normalised rows with bias + RoPE + KV write and SiLU*up in their epilogues
# (seven launches per layer; the row count never changes a row's rounding).
# "fused": RMSNorm inside the QKV and gate/up projections, residual adds inside
# o_proj/down_proj (six launches per layer, whole columns per workgroup).
# "auto" (default): fused up to FUSED_MAX_ROWS rows, split-K above. Measured on
# the 0.5B forward (one token per sequence, HIP graph, blocked weights): split-K
# / fused 917 / 771 us at 4 rows, 937 / 821 at 8, 949 / 879 at 12, 963 / 929 at
# 16, 956 / 1119 at 24, 982 / 1232 at 32; since the fused o/down and q/k/v
# kernels run 4-column workgroups, 976 / 830 at 8 rows, 1000 / 920 at 16,
# 1023 / 1180 at 32 (600-token histories); with every load of a split-K layer
# issued ahead of its waits (six launches: QKV+RoPE, attention, o_proj +
# residual, gate/up with RMSNorm, down_proj k-slices, residual + RMSNorm),
# 741 / 711 at 1 row, 747 / 725 at 2, 759 / 741 at 4, 785 / 790 at 8,
# 829 / 887 at 16, 930 / 1136 at 32, so split-K from 5 rows. A model whose
# layers hold at least
# SPLITK_ALWAYS_LAYER_BYTES of projection weights takes split-K at every row
# count: whole-column workgroups leave most of the chip idle on weights that
# size (the 3B, 154 MB per layer, 36 layers, one sequence: split-K / fused /
# wide layer 2152 / 2311 / 2236 us at 1 row, 2164 / 2443 / 2244 at 5). Each
# path gives a row the same bits at any row count of its range; a model whose
# passes straddle FUSED_MAX_ROWS and must not change with the batch width takes
# the wide layer (invariant_gemm_rows). Set SMALL_BATCH_FUSION = False to force
# the hipBLASLt path.
SMALL_BATCH_FUSION = True
SMALL_BATCH_PATH = "auto"
FUSED_MAX_ROWS = 4
SPLITK_ALWAYS_LAYER_BYTES = 64 << 20


def _layer_proj_bytes(model) -> int:
    layer = model.model.layers[0]
    a, mlp = layer.self_attn, layer.mlp
    ws = (a.qkv_weight, a.o_proj.weight, mlp.gate_up_weight, mlp.down_proj.weight)
    return sum(w.numel() * w.element_size() for w in ws)


def _small_path(model, n: int) -> str:
    if SMALL_BATCH_PATH == "auto":
        if _layer_proj_bytes(model) >= SPLITK_ALWAYS_LAYER_BYTES:
            return "splitk"
        return "fused" if n <= FUSED_MAX_ROWS else "splitk"
    return SMALL_BATCH_PATH


def _decode_variant(model, n: int) -> tuple[str, bool]:
    """The decode layer n rows take (where _small_fusable holds): its path and,
    for split-K, whether o_proj and gate/up run fused (_forward_splitk)."""
    path = _small_path(model, n)
    return path, path == "splitk" and SPLITK_FUSED_O and n <= SPLITK_FUSED_O_ROWS


def _small_fusable(model, rows: int) -> bool:
    if not SMALL_BATCH_FUSION:
        return False
    layers = model.model.layers
    a = layers[0].self_attn
    w = a.qkv_weight
    if w.dtype != torch.bfloat16 or a.qkv_bias is None or a.head_dim not in (64, 128):
        return False
    if a.o_proj.bias is not None or layers[0].mlp.down_proj.bias is not None:
        return False
    if layers[0].mlp.gate_up_weight.shape[0] % 64:
        return False
    return kernels.fused_fits(rows, w.shape[1], a.head_dim)


@torch.no_grad()
def forward_hidden(model, input_ids: torch.Tensor, kv: DeviceKV, rows: torch.Tensor, max_ctx: int,
                   q_lens: torch.Tensor | None = None, attn_order: tuple[int, int] = (0, 0),
                   fused: bool | None = None, gemm_rows: int | None = None,
                   blocked_out: bool = False) -> torch.Tensor:
    """Final-normed hidden states [B, T, H] for `input_ids` [B, T] (device int64).

    Row i of the batch is table/length row rows[i]; its tokens land at positions
    kv.lens[rows[i]] + t, t < q_lens[i] (or T). Lengths are NOT advanced here:
    the caller commits (host and device) once the pass is queued.
    max_ctx must bound kv.lens[rows[i]] + T for every i.

    gemm_rows: the most rows any pass of this model will have (bf16, <= 160), from
    invariant_gemm_rows: the wide split-K layer then runs every pass, however few
    rows it has, so a sequence's results do not depend on how many others share
    the pass (None where the decode layer already takes every such pass).

    With fused projections (model.prepare_fused) each layer is: RMSNorm(+residual)
    kernel, one [q|k|v] GEMM, RoPE + KV write kernel, attention, o_proj GEMM,
    residual + RMSNorm kernel, one [gate|up] GEMM, SiLU*up kernel, down GEMM; the
    residual add of the MLP is folded into the next layer's RMSNorm. Otherwise the
    layer runs transformers-style module calls with the same kernels for the cache.

    blocked_out: return the final hidden states as the [B*T, H] blocked matrix
    (kernels.to_blocked layout, rows padded to 16) for a blocked LM head; only
    where blocked_forward(model, input_ids.numel(), gemm_rows) holds.
    """
    if fused is None:
        fused = _fusable(model)
    n = input_ids.numel()
    if blocked_out:
        if not (fused and blocked_forward(model, n, gemm_rows)):
            raise ValueError("blocked_out needs the blocked split-K layer (blocked_forward)")
    if fused and gemm_rows is not None and n <= gemm_rows and _wide_ok(model, gemm_rows):
        return _forward_splitk(model, input_ids, kv, rows, max_ctx, q_lens, attn_order, wide=True,
                               blocked_out=blocked_out)
    if fused:
        if _small_fusable(model, n):
            if _small_path(model, n) == "splitk":
                return _forward_splitk(model, input_ids, kv, rows, max_ctx, q_lens, attn_order,
                                       blocked_out=blocked_out)
            return _forward_small(model, input_ids, kv, rows, max_ctx, q_lens, attn_order)
        if n <= SPLITK_MAX_ROWS and _wide_ok(model, n):
            return _forward_splitk(model, input_ids, kv, rows, max_ctx, q_lens, attn_order, wide=True,
                                   blocked_out=blocked_out)
        return _forward_fused(model, input_ids, kv, rows, max_ctx, q_lens, attn_order)
    inner = model.model
    B, T = input_ids.shape
    hidden = inner.embed_tokens(input_ids)
    start = kv.lens.index_select(0, rows).to(torch.long)
    positions = start[:, None] + torch.arange(T, device=input_ids.device)[None, :]
    cos, sin = inner.rotary_emb(hidden, positions, max_ctx)
    layer_attn = LayerAttention(kv, rows, B, T, _q_heads(model, kv), max_ctx, q_lens, kv.k.dtype,
                                attn_order)
    for layer in inner.layers:
        attn = layer.self_attn
        if getattr(attn, "sliding_window", None) is not None:
            raise NotImplementedError("sliding-window attention needs a windowed mask; this model uses it")
        li = attn.layer_idx
        D = attn.head_dim
        residual = hidden
        h = layer.input_layernorm(hidden)
        q = attn.q_proj(h).view(B, T, -1, D)
        k = attn.k_proj(h).view(B, T, -1, D)
        v = attn.v_proj(h).view(B, T, -1, D)
        q, k = apply_rope(q, k, cos, sin, unsqueeze_dim=2)
        kernels.kv_write(k, v, kv.k[li], kv.v[li], kv.tables, kv.lens, seq_rows=rows,
                         q_lens=q_lens)
        out = layer_attn(q, li, attn.scaling)
        hidden = residual + attn.o_proj(out.view(B, T, -1))
        residual = hidden
        hidden = residual + layer.mlp(layer.post_attention_layernorm(hidden))
    return inner.norm(hidden)


# bf16 batches up to this many rows run o_proj and down_proj as split-K
# projections whose reduction kernel also adds the residual and applies the next
# RMSNorm (instead of hipBLASLt + a separate residual/RMSNorm kernel).
SPLITK_MAX_ROWS = 160
# The split-K decode layer (not the wide one) runs o_proj as whole columns per
# workgroup adding into the residual in place, and gate/up with the RMSNorm in
# its prologue (kve_linear_residual, kve_fused_gate_up writing a blocked act),
# instead of o_proj k-slices + kve_residual_norm + kve_gate_up_silu: one launch
# fewer per layer (0.5B at 32 rows 5.1 + 9.9 us against 4.2 + 4.7 + 8.2; 3B at
# one row 5.9 + 21.2 against 4.8 + 4.8 + 19.6), up to SPLITK_FUSED_O_ROWS rows
# (whole forwards: 0.5B at 32 rows 1022 -> 1013 us, 3B at one row 2151 -> 2109,
# at 5 rows 2169 -> 2175; at 64 rows the 0.5B took 1146 -> 1292). False: the
# seven-launch layer at every width.
SPLITK_FUSED_O = True
SPLITK_FUSED_O_ROWS = 32


def _splitk_ok(model, rows: int) -> bool:
    if not SMALL_BATCH_FUSION or rows > SPLITK_MAX_ROWS:
        return False
    layer = model.model.layers[0]
    a, mlp = layer.self_attn, layer.mlp
    if a.qkv_weight.dtype != torch.bfloat16 or a.o_proj.bias is not None or mlp.down_proj.bias is not None:
        return False
    H = a.o_proj.weight.shape[0]
    return H % 64 == 0 and H <= 2048 and a.o_proj.weight.shape[1] % 32 == 0 \
        and mlp.down_proj.weight.shape[1] % 32 == 0


def invariant_gemm_rows(model, rows: int, wide: bool = False) -> tuple[bool, int | None]:
    """(ok, gemm_rows): with ok, forward_hidden(..., gemm_rows=gemm_rows) gives
    each sequence the same bits in every pass of at most `rows` rows, whatever
    else shares the pass. gemm_rows is None when the decode layer takes every
    such pass (<= 64 rows), else `rows` (the wide split-K layer). wide: take
    the wide layer whatever the row count (its arithmetic is also what
    forward_packed_wide gives a prefill, so a model whose every pass is wide
    gets the same bits for a token from a prefill, a recompute or a verify
    pass)."""
    if not _fusable(model):
        return False, None
    if wide:
        return (True, rows) if _wide_ok(model, rows) else (False, None)
    if _small_fusable(model, rows) and _decode_variant(model, rows) == _decode_variant(model, 1):
        return True, None  # every pass of at most `rows` rows takes one decode path
    if _wide_ok(model, rows):
        return True, rows
    return False, None


def _wide_ok(model, rows: int) -> bool:
    """The wide split-K layer (QKV as k-slices + a bias/RoPE/KV-write epilogue,
    gate/up + SiLU, o_proj / down_proj k-slices + residual/RMSNorm) fits; above
    SPLITK_MAX_ROWS its projections run as kve_linear_rows, whose tiles need
    128-multiple outputs and 64-multiple inputs."""
    if not _splitk_ok(model, min(rows, SPLITK_MAX_ROWS)):
        return False
    a = model.model.layers[0].self_attn
    mlp = model.model.layers[0].mlp
    if not (a.qkv_bias is not None and a.head_dim in (64, 128)
            and a.qkv_weight.shape[0] % 64 == 0 and a.qkv_weight.shape[1] % 32 == 0
            and mlp.gate_up_weight.shape[0] % 64 == 0):
        return False
    if rows <= SPLITK_MAX_ROWS:
        return True
    outs = (a.qkv_weight.shape[0], a.o_proj.weight.shape[0], mlp.down_proj.weight.shape[0],
            mlp.gate_up_weight.shape[0])
    ins = (a.qkv_weight.shape[1], a.o_proj.weight.shape[1], mlp.down_proj.weight.shape[1])
    return all(n % 128 == 0 for n in outs) and all(k % 64 == 0 for k in ins)


def _forward_fused(model, input_ids, kv: DeviceKV, rows, max_ctx, q_lens, attn_order):
    inner = model.model
    layers = inner.layers
    B, T = input_ids.shape
    splitk = _splitk_ok(model, B * T)
    residual = inner.embed_tokens(input_ids)
    start = kv.lens.index_select(0, rows).to(torch.long)
    positions = start[:, None] + torch.arange(T, device=input_ids.device)[None, :]
    cos, sin = inner.rotary_emb(residual, positions, max_ctx)
    cos, sin = cos.contiguous(), sin.contiguous()
    first = layers[0].input_layernorm
    h = kernels.rmsnorm(residual, first.weight, first.variance_epsilon)
    layer_attn = LayerAttention(kv, rows, B, T, _q_heads(model, kv), max_ctx, q_lens, kv.k.dtype,
                                attn_order)
    for i, layer in enumerate(layers):
        attn = layer.self_attn
        if getattr(attn, "sliding_window", None) is not None:
            raise NotImplementedError("sliding-window attention needs a windowed mask; this model uses it")
        li = attn.layer_idx
        qkv = torch.nn.functional.linear(h, attn.qkv_weight, attn.qkv_bias)
        q = kernels.rope_kv_write(qkv, cos, sin, kv.k[li], kv.v[li], kv.tables, kv.lens,
                                  attn.num_key_value_groups * kv.k.shape[2], seq_rows=rows,
                                  q_lens=q_lens)
        out = layer_attn(q, li, attn.scaling)
        post = layer.post_attention_layernorm
        if splitk:
            part = kernels.linear_splitk(out.view(B * T, -1), attn.o_proj.weight)
            h = kernels.residual_norm(part, part.shape[0], residual, post.weight,
                                      post.variance_epsilon, xn=h)
        else:
            o = attn.o_proj(out.view(B, T, -1))
            h = kernels.rmsnorm(residual, post.weight, post.variance_epsilon, delta=o,
                                residual_out=residual)
        mlp = layer.mlp
        act = kernels.silu_mul(torch.nn.functional.linear(h, mlp.gate_up_weight))
        nxt = layers[i + 1].input_layernorm if i + 1 < len(layers) else inner.norm
        if splitk:
            part = kernels.linear_splitk(act, mlp.down_proj.weight)
            h = kernels.residual_norm(part, part.shape[0], residual, nxt.weight,
                                      nxt.variance_epsilon, xn=h)
        else:
            d = mlp.down_proj(act)
            h = kernels.rmsnorm(residual, nxt.weight, nxt.variance_epsilon, delta=d,
                                residual_out=residual)
    return h


def forward_packed(model, ids: torch.Tensor, dst: torch.Tensor, B: int, T: int, kv: DeviceKV,
                   rows: torch.Tensor, max_ctx: int, q_lens: torch.Tensor,
                   attn_order: tuple[int, int] = (0, 0)) -> torch.Tensor:
    """Prefill forward over N packed tokens (fused model): final-normed hidden
    states [N, H] for ids [N] (device int64), where packed row j is token t of
    sequence b at dst[j] = b * T + t (t < q_lens[b] <= T). Embedding, norms and
    projections run on the N real rows only; RoPE + KV write and attention run
    on the padded [B, T] layout, which packed rows are scattered into and
    gathered back from. Same per-sequence semantics as forward_hidden over the
    padded [B, T] batch; the caller commits lengths afterwards."""
    inner = model.model
    layers = inner.layers
    a0 = layers[0].self_attn
    width = a0.qkv_weight.shape[0]
    residual = inner.embed_tokens(ids)
    start = kv.lens.index_select(0, rows).to(torch.long)
    positions = start[:, None] + torch.arange(T, device=ids.device)[None, :]
    cos, sin = inner.rotary_emb(residual, positions, max_ctx)
    cos, sin = cos.contiguous(), sin.contiguous()
    # padded rows are never read (q_lens masks them); zero them once anyway
    qkv_pad = torch.zeros(B * T, width, dtype=residual.dtype, device=ids.device)
    first = layers[0].input_layernorm
    h = kernels.rmsnorm(residual, first.weight, first.variance_epsilon)
    layer_attn = LayerAttention(kv, rows, B, T, _q_heads(model, kv), max_ctx, q_lens, kv.k.dtype,
                                attn_order)
    for i, layer in enumerate(layers):
        attn = layer.self_attn
        if getattr(attn, "sliding_window", None) is not None:
            raise NotImplementedError("sliding-window attention needs a windowed mask; this model uses it")
        li = attn.layer_idx
        qkv = torch.nn.functional.linear(h, attn.qkv_weight, attn.qkv_bias)
        qkv_pad.index_copy_(0, dst, qkv)
        q = kernels.rope_kv_write(qkv_pad.view(B, T, width), cos, sin, kv.k[li], kv.v[li],
                                  kv.tables, kv.lens, attn.num_key_value_groups * kv.k.shape[2],
                                  seq_rows=rows, q_lens=q_lens)
        out = layer_attn(q, li, attn.scaling)
        o = attn.o_proj(out.view(B * T, -1).index_select(0, dst))
        post = layer.post_attention_layernorm
        h = kernels.rmsnorm(residual, post.weight, post.variance_epsilon, delta=o,
                            residual_out=residual)
        mlp = layer.mlp
        act = kernels.silu_mul(torch.nn.functional.linear(h, mlp.gate_up_weight))
        nxt = layers[i + 1].input_layernorm if i + 1 < len(layers) else inner.norm
        d = mlp.down_proj(act)
        h = kernels.rmsnorm(residual, nxt.weight, nxt.variance_epsilon, delta=d,
                            residual_out=residual)
    return h


def _wide_proj(x: torch.Tensor, weight: torch.Tensor, mode: int, blocked: bool = False,
               rows: int | None = None) -> torch.Tensor:
    """One projection of the wide split-K layer over any number of rows: k-slice
    partials [S, rows, out] (or act for gate/up) from the split-K kernels up to
    SPLITK_MAX_ROWS rows, else the same sums from kve_linear_rows as one slice
    [1, rows, out]. Either way each row gets the same bits. blocked: x, weight
    and the gate/up act are blocked matrices (x holding `rows` rows)."""
    if rows is None:
        rows = x.numel() // x.shape[-1]
    if rows <= SPLITK_MAX_ROWS:
        if mode == kernels.ROWS_GATE_UP:
            return kernels.gate_up_silu(x, weight, blocked=blocked, rows=rows)
        return kernels.linear_splitk(x, weight, blocked=blocked, rows=rows)
    return kernels.linear_rows(x, weight, mode, blocked=blocked, rows=rows)


def forward_packed_wide(model, ids: torch.Tensor, dst: torch.Tensor, B: int, T: int, kv: DeviceKV,
                        rows: torch.Tensor, max_ctx: int, q_lens: torch.Tensor,
                        attn_order: tuple[int, int] = (0, 0)) -> torch.Tensor:
    """forward_packed (same arguments and per-sequence semantics) with the wide
    split-K layer's arithmetic on the N packed rows: every token's K/V, hidden
    state and final norm are bit-identical to what _forward_splitk(wide=True)
    gives it in a pass of any width at the same position and prefix, given the
    same attention order. A prompt prefilled here, or a preempted request's
    tokens recomputed here, therefore continue exactly as if every token had
    come from a verify pass (the reference recomputes the same way,
    kvengine/engine.py:425-440)."""
    inner = model.model
    layers = inner.layers
    N = ids.numel()
    residual = inner.embed_tokens(ids).contiguous()
    start = kv.lens.index_select(0, rows).to(torch.long)
    positions = start[:, None] + torch.arange(T, device=ids.device)[None, :]
    cos, sin = inner.rotary_emb(residual, positions, max_ctx)
    D = cos.shape[-1]
    cos = cos.reshape(B * T, D).index_select(0, dst).contiguous()
    sin = sin.reshape(B * T, D).index_select(0, dst).contiguous()
    slots = kernels.kv_slots(kv.tables, kv.lens, B, T, kv.block_size, kv.k.shape[1], seq_rows=rows,
                             q_lens=q_lens).index_select(0, dst)
    Hq = _q_heads(model, kv)
    # padded rows are never read (q_lens masks them); zero them once anyway
    q_pad = torch.zeros(B * T, Hq * D, dtype=residual.dtype, device=ids.device)
    # blocked weights: the normalised rows and the gate/up activations between the
    # launches are blocked matrices (o_proj reads the gathered attention rows
    # row-major); the final hidden states are row-major
    blk = _has_blocked(model)
    first = layers[0].input_layernorm
    xn = kernels.rmsnorm(residual, first.weight, first.variance_epsilon, blocked=blk)
    layer_attn = LayerAttention(kv, rows, B, T, Hq, max_ctx, q_lens, kv.k.dtype, attn_order)
    for i, layer in enumerate(layers):
        attn = layer.self_attn
        if getattr(attn, "sliding_window", None) is not None:
            raise NotImplementedError("sliding-window attention needs a windowed mask; this model uses it")
        li = attn.layer_idx
        mlp = layer.mlp
        part = _wide_proj(xn, attn.qkv_weight_blk if blk else attn.qkv_weight, kernels.ROWS_QKV,
                          blocked=blk, rows=N)
        q = kernels.qkv_part_rope(part, attn.qkv_bias, cos, sin, slots, kv.k[li], kv.v[li], Hq, N)
        q_pad.index_copy_(0, dst, q.view(N, Hq * D))
        out = layer_attn(q_pad.view(B, T, Hq, D), li, attn.scaling)
        o_in = out.reshape(B * T, Hq * D).index_select(0, dst)
        part = _wide_proj(o_in, attn.o_proj.weight, kernels.ROWS_RESIDUAL)
        post = layer.post_attention_layernorm
        xn = kernels.residual_norm(part, part.shape[0], residual, post.weight, post.variance_epsilon,
                                   xn=xn, blocked=blk)
        act = _wide_proj(xn, mlp.gate_up_weight_blk if blk else mlp.gate_up_weight,
                         kernels.ROWS_GATE_UP, blocked=blk, rows=N)
        part = _wide_proj(act, mlp.down_weight_blk if blk else mlp.down_proj.weight,
                          kernels.ROWS_RESIDUAL, blocked=blk, rows=N)
        last = i + 1 == len(layers)
        nxt = inner.norm if last else layers[i + 1].input_layernorm
        xn = kernels.residual_norm(part, part.shape[0], residual, nxt.weight, nxt.variance_epsilon,
                                   xn=None if (last and blk) else xn, blocked=blk and not last)
    return xn


def _prologue(model, input_ids, kv: DeviceKV, rows, max_ctx):
    """Embedding rows and RoPE cos/sin of a pass's tokens in one launch (the
    same values as embed_tokens and rotary_emb's table lookup)."""
    inner = model.model
    emb = inner.embed_tokens.weight
    cos_t, sin_t = inner.rotary_emb.table(emb, max_ctx)
    return kernels.pass_prologue(input_ids, emb, kv.lens, rows, cos_t, sin_t)


def _forward_small(model, input_ids, kv: DeviceKV, rows, max_ctx, q_lens, attn_order):
    """Five launches per layer: fused QKV (RMSNorm, bias, RoPE, KV write),
    attention (+ its split merge), o_proj + residual, fused gate/up (RMSNorm,
    SiLU*up), down_proj + residual. The residual stream is updated in place."""
    inner = model.model
    B, T = input_ids.shape
    blk = _has_blocked(model)  # weights only: the kernels' other operands stay row-major
    residual, cos, sin = _prologue(model, input_ids, kv, rows, max_ctx)
    layer_attn = LayerAttention(kv, rows, B, T, _q_heads(model, kv), max_ctx, q_lens, kv.k.dtype,
                                attn_order)
    for layer in inner.layers:
        attn = layer.self_attn
        if getattr(attn, "sliding_window", None) is not None:
            raise NotImplementedError("sliding-window attention needs a windowed mask; this model uses it")
        li = attn.layer_idx
        norm = layer.input_layernorm
        mlp = layer.mlp
        q = kernels.fused_qkv(residual, norm.weight, norm.variance_epsilon,
                              attn.qkv_weight_blk if blk else attn.qkv_weight, attn.qkv_bias, cos,
                              sin, kv.k[li], kv.v[li], kv.tables, kv.lens,
                              attn.num_key_value_groups * kv.k.shape[2], seq_rows=rows,
                              q_lens=q_lens, blocked_w=blk)
        out = layer_attn(q, li, attn.scaling)
        kernels.linear_residual(out.view(B * T, -1), attn.o_weight_blk if blk else attn.o_proj.weight,
                                residual, blocked_w=blk)
        post = layer.post_attention_layernorm
        act = kernels.fused_gate_up(residual, post.weight, post.variance_epsilon,
                                    mlp.gate_up_weight_blk if blk else mlp.gate_up_weight,
                                    blocked_w=blk)
        kernels.linear_residual(act, mlp.down_weight_blk if blk else mlp.down_proj.weight, residual,
                                blocked_w=blk)
    return kernels.rmsnorm(residual, inner.norm.weight, inner.norm.variance_epsilon)


# The split-K layer hands its projections blocked activations (16-row x
# 32-column blocks, kernels.to_blocked) and reads the blocked weight copies made
# by model.prepare_fused: a projection's direct-to-LDS loads then read 512-byte
# runs instead of one 64-128 byte piece per row (3B gate/up at 160 rows 52 ->
# 33 us, down 37 -> 19 us; 0.5B gate/up at 32 rows 12 -> 7 us). The sums are
# the same in either layout. False: row-major operands throughout.
BLOCKED_LAYERS = True


def _has_blocked(model) -> bool:
    a = model.model.layers[0].self_attn
    return BLOCKED_LAYERS and getattr(a, "qkv_weight_blk", None) is not None


def blocked_forward(model, n: int, gemm_rows: int | None = None) -> bool:
    """forward_hidden of n rows (with this gemm_rows) runs the split-K layer on
    blocked operands, so it can return its hidden states blocked."""
    if not (_fusable(model) and _has_blocked(model) and n <= SPLITK_MAX_ROWS):
        return False
    if gemm_rows is not None and n <= gemm_rows and _wide_ok(model, gemm_rows):
        return True
    if _small_fusable(model, n):
        return _small_path(model, n) == "splitk"
    return _wide_ok(model, n)


def _forward_splitk(model, input_ids, kv: DeviceKV, rows, max_ctx, q_lens, attn_order,
                    wide: bool = False, blocked_out: bool = False):
    """Six launches per layer: QKV (+bias, RoPE, KV write), attention (+ its
    split merge), o_proj + residual (whole columns per workgroup), gate/up with
    the RMSNorm in its prologue + SiLU*up, down_proj k-slices, residual add +
    the next layer's RMSNorm (the final norm after the last layer). The KV
    slots of the new tokens are resolved once.
    wide (up to 160 rows): o_proj runs as k-slices + residual add + RMSNorm and
    gate/up on the normalised rows, and the QKV projection as k-slices too, with
    its bias / RoPE / KV write in a separate epilogue launch (eight per layer):
    these are the sums kve_linear_rows reproduces for a prefill.
    With blocked weights the normalised rows, the attention output (wide) and
    the gate/up activations between the launches are blocked matrices; the
    final hidden states are row-major [B, T, H] unless blocked_out."""
    inner = model.model
    layers = inner.layers
    B, T = input_ids.shape
    n = B * T
    blk = _has_blocked(model) and n <= SPLITK_MAX_ROWS
    fused_o = not wide and SPLITK_FUSED_O and n <= SPLITK_FUSED_O_ROWS
    residual, cos, sin = _prologue(model, input_ids, kv, rows, max_ctx)
    slots = kernels.kv_slots(kv.tables, kv.lens, B, T, kv.block_size, kv.k.shape[1], seq_rows=rows,
                             q_lens=q_lens)
    first = layers[0].input_layernorm
    xn = kernels.rmsnorm(residual, first.weight, first.variance_epsilon, blocked=blk)
    layer_attn = LayerAttention(kv, rows, B, T, _q_heads(model, kv), max_ctx, q_lens, kv.k.dtype,
                                attn_order)
    for i, layer in enumerate(layers):
        attn = layer.self_attn
        if getattr(attn, "sliding_window", None) is not None:
            raise NotImplementedError("sliding-window attention needs a windowed mask; this model uses it")
        li = attn.layer_idx
        Hq = attn.num_key_value_groups * kv.k.shape[2]
        mlp = layer.mlp
        if blk:
            if wide:
                part = kernels.linear_splitk(xn, attn.qkv_weight_blk, blocked=True, rows=n)
                q = kernels.qkv_part_rope(part, attn.qkv_bias, cos, sin, slots, kv.k[li], kv.v[li],
                                          Hq, n).view(B, T, Hq, -1)
            else:
                q = kernels.qkv_rope(xn, attn.qkv_weight_blk, attn.qkv_bias, cos, sin, slots,
                                     kv.k[li], kv.v[li], Hq, blocked=True, bt=(B, T))
            if fused_o:
                out = layer_attn(q, li, attn.scaling)
                kernels.linear_residual(out.view(n, -1), attn.o_weight_blk, residual, blocked_w=True)
            else:
                out = layer_attn(q, li, attn.scaling, blocked=True)
                part = kernels.linear_splitk(out, attn.o_weight_blk, blocked=True, rows=n)
        else:
            if wide:
                part = _wide_proj(xn, attn.qkv_weight, kernels.ROWS_QKV)
                q = kernels.qkv_part_rope(part, attn.qkv_bias, cos, sin, slots, kv.k[li], kv.v[li],
                                          Hq, n).view(B, T, Hq, -1)
            else:
                q = kernels.qkv_rope(xn, attn.qkv_weight, attn.qkv_bias, cos, sin, slots, kv.k[li],
                                     kv.v[li], Hq)
            out = layer_attn(q, li, attn.scaling)
            if fused_o:
                kernels.linear_residual(out.view(n, -1), attn.o_proj.weight, residual)
            else:
                part = _wide_proj(out.view(n, -1), attn.o_proj.weight, kernels.ROWS_RESIDUAL)
        post = layer.post_attention_layernorm
        if fused_o:
            act = kernels.fused_gate_up(residual, post.weight, post.variance_epsilon,
                                        mlp.gate_up_weight_blk if blk else mlp.gate_up_weight,
                                        blocked_w=blk, blocked_act=blk)
        else:
            xn = kernels.residual_norm(part, part.shape[0], residual, post.weight,
                                       post.variance_epsilon, xn=xn, blocked=blk)
        if blk:
            if not fused_o:
                act = kernels.gate_up_silu(xn, mlp.gate_up_weight_blk, blocked=True, rows=n)
            part = kernels.linear_splitk(act, mlp.down_weight_blk, blocked=True, rows=n)
        else:
            if not fused_o:
                act = _wide_proj(xn, mlp.gate_up_weight, kernels.ROWS_GATE_UP)
            part = _wide_proj(act, mlp.down_proj.weight, kernels.ROWS_RESIDUAL)
        last = i + 1 == len(layers)
        nxt = inner.norm if last else layers[i + 1].input_layernorm
        out_blk = blk and (blocked_out or not last)
        xn = kernels.residual_norm(part, part.shape[0], residual, nxt.weight, nxt.variance_epsilon,
                                   xn=xn if out_blk == blk else None, blocked=out_blk)
    return xn


@torch.no_grad()
def forward_with_own_cache(model, input_ids: torch.Tensor, cache, all_logits: bool = False,
                           return_hidden: bool = False) -> torch.Tensor:
    """One forward pass over input_ids [1, T], appending to `cache`.

    Same contract as kvengine/forward.py:148-215: reserve(T) before any layer
    writes, every layer writes at the same start, commit(T) once after the
    layers; returns logits [1, T, V] if all_logits else [1, 1, V].
    """
    assert input_ids.dim() == 2 and input_ids.shape[0] == 1, "one request at a time"
    T = input_ids.shape[1]
    start = cache.length
    cache.reserve(T)
    ids = input_ids.to(device=cache.device_kv().k.device, dtype=torch.long)
    hidden = forward_hidden(model, ids, cache.device_kv(), cache.row_dev, start + T)
    cache.commit(T)
    if return_hidden:
        return hidden if all_logits else hidden[:, -1:, :]
    if not all_logits:
        hidden = hidden[:, -1:, :]
    return model.lm_head(hidden)
