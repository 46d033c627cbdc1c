"""Qwen2 module tree with the attribute layout kvengine's forward pass reads.

kvengine drives transformers' Qwen2 modules through a duck-type
(kvengine/forward.py:168-215): model.model.{embed_tokens, rotary_emb, norm,
layers[i]}, per layer .self_attn.{q_proj, k_proj, v_proj, o_proj, head_dim,
num_key_value_groups, scaling, layer_idx, sliding_window}, .input_layernorm,
.post_attention_layernorm, .mlp, and model.lm_head / config /
generation_config. This module provides that tree, built straight on the
device from a state dict, with the same torch arithmetic as transformers'
modules (models/qwen2/modeling_qwen2.py: RMSNorm 237-255, rotary 51-102,
MLP 35-48) so the forward pass is interchangeable with a real
Qwen2ForCausalLM. The LM head is tied to the embedding.
"""

from __future__ import annotations

from types import SimpleNamespace

import torch
import torch.nn as nn
import torch.nn.functional as F

from .arch import Qwen2Arch
from .weights import generate_state_dict


class RMSNorm(nn.Module):
    def __init__(self, hidden: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden))
        self.variance_epsilon = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        in_dtype = x.dtype
        x = x.to(torch.float32)
        var = x.pow(2).mean(-1, keepdim=True)
        x = x * torch.rsqrt(var + self.variance_epsilon)
        return self.weight * x.to(in_dtype)


class RotaryEmbedding(nn.Module):
    """cos/sin for absolute positions; inv_freq is computed on the CPU in float32
    exactly as transformers does, so every device sees the same frequencies."""

    def __init__(self, head_dim: int, theta: float):
        super().__init__()
        inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
        self.register_buffer("inv_freq", inv, persistent=False)
        self.attention_scaling = 1.0
        self._table = None  # (cos, sin) [P, D] for positions 0..P-1
        self._outgrown = []

    @torch.no_grad()
    def _compute(self, x: torch.Tensor, position_ids: torch.Tensor):
        inv = self.inv_freq[None, :, None].float().expand(position_ids.shape[0], -1, 1)
        pos = position_ids[:, None, :].float()
        freqs = (inv.float() @ pos.float()).transpose(1, 2)
        emb = torch.cat((freqs, freqs), dim=-1)
        cos = emb.cos() * self.attention_scaling
        sin = emb.sin() * self.attention_scaling
        return cos.to(dtype=x.dtype), sin.to(dtype=x.dtype)

    @torch.no_grad()
    def table(self, x: torch.Tensor, num_positions: int):
        """cos/sin [P, D] for positions 0..P-1 (P >= num_positions), computed by the
        same ops as forward() and kept; each entry depends only on its position."""
        t = self._table
        if t is None or t[0].shape[0] < num_positions or t[0].dtype != x.dtype \
                or t[0].device != x.device:
            P = max(num_positions, 4096, 2 * t[0].shape[0] if t is not None else 0)
            pos = torch.arange(P, device=x.device)[None]
            cos, sin = self._compute(x, pos)
            if t is not None:
                self._outgrown.append(t)  # a captured graph may still read it
            self._table = t = (cos[0].contiguous(), sin[0].contiguous())
        return t

    @torch.no_grad()
    def forward(self, x: torch.Tensor, position_ids: torch.Tensor, max_positions: int | None = None):
        """cos, sin [B, T, D] for position_ids [B, T]. With max_positions (> every
        position id) they are gathered from the kept table: same values, two
        launches instead of the product, concatenation, cos, sin and casts."""
        if max_positions is None:
            return self._compute(x, position_ids)
        cos_t, sin_t = self.table(x, max_positions)
        idx = position_ids.clamp(0, cos_t.shape[0] - 1)
        return cos_t[idx], sin_t[idx]


class Attention(nn.Module):
    def __init__(self, arch: Qwen2Arch, layer_idx: int):
        super().__init__()
        self.layer_idx = layer_idx
        self.head_dim = arch.head_dim
        self.num_heads = arch.num_q_heads
        self.num_key_value_heads = arch.num_kv_heads
        self.num_key_value_groups = arch.group
        self.scaling = arch.head_dim ** -0.5
        self.sliding_window = None
        self.q_proj = nn.Linear(arch.hidden, arch.q_dim, bias=True)
        self.k_proj = nn.Linear(arch.hidden, arch.kv_dim, bias=True)
        self.v_proj = nn.Linear(arch.hidden, arch.kv_dim, bias=True)
        self.o_proj = nn.Linear(arch.q_dim, arch.hidden, bias=False)


class MLP(nn.Module):
    def __init__(self, arch: Qwen2Arch):
        super().__init__()
        self.gate_proj = nn.Linear(arch.hidden, arch.ffn, bias=False)
        self.up_proj = nn.Linear(arch.hidden, arch.ffn, bias=False)
        self.down_proj = nn.Linear(arch.ffn, arch.hidden, bias=False)
        self.act_fn = F.silu

    def forward(self, x):
        return self.down_proj(self.act_fn(self.gate_proj(x)) * self.up_proj(x))


class DecoderLayer(nn.Module):
    def __init__(self, arch: Qwen2Arch, layer_idx: int):
        super().__init__()
        self.self_attn = Attention(arch, layer_idx)
        self.mlp = MLP(arch)
        self.input_layernorm = RMSNorm(arch.hidden, arch.rms_eps)
        self.post_attention_layernorm = RMSNorm(arch.hidden, arch.rms_eps)


class Qwen2Inner(nn.Module):
    def __init__(self, arch: Qwen2Arch):
        super().__init__()
        self.embed_tokens = nn.Embedding(arch.vocab, arch.hidden)
        self.layers = nn.ModuleList(DecoderLayer(arch, i) for i in range(arch.num_layers))
        self.norm = RMSNorm(arch.hidden, arch.rms_eps)
        self.rotary_emb = RotaryEmbedding(arch.head_dim, arch.rope_theta)


class Qwen2ForCausalLM(nn.Module):
    """Tied-embedding Qwen2 causal LM (HF attribute layout)."""

    def __init__(self, arch: Qwen2Arch):
        super().__init__()
        self.arch = arch
        self.model = Qwen2Inner(arch)
        self.lm_head = nn.Linear(arch.hidden, arch.vocab, bias=False)
        self.config = SimpleNamespace(
            num_hidden_layers=arch.num_layers, num_attention_heads=arch.num_q_heads,
            num_key_value_heads=arch.num_kv_heads, head_dim=arch.head_dim,
            hidden_size=arch.hidden, vocab_size=arch.vocab, intermediate_size=arch.ffn,
            rms_norm_eps=arch.rms_eps, tie_word_embeddings=True)
        self.generation_config = SimpleNamespace(eos_token_id=None)


def build_model(arch: Qwen2Arch, state_dict: dict | None = None, seed: int = 0,
                dtype: torch.dtype = torch.bfloat16, device: str | torch.device = "cuda"):
    """Qwen2ForCausalLM on `device` from a state dict (generated from `seed` if None).

    Parameters are created on the meta device and then bound to device copies
    of the state dict, so nothing is initialised twice. The inv_freq buffer is
    computed on the CPU in float32 and copied.
    """
    if state_dict is None:
        state_dict = generate_state_dict(arch, seed, dtype=dtype)
    with torch.device("meta"):
        m = Qwen2ForCausalLM(arch)
    dev = torch.device(device)
    params = {n: t.to(device=dev, dtype=dtype) for n, t in state_dict.items()}
    emb = params["model.embed_tokens.weight"]
    params["lm_head.weight"] = emb
    missing, unexpected = m.load_state_dict(params, strict=False, assign=True)
    assert not unexpected, unexpected
    assert not missing, missing
    m.lm_head.weight = m.model.embed_tokens.weight  # tie (same storage)
    rot = RotaryEmbedding(arch.head_dim, arch.rope_theta)
    m.model.rotary_emb = rot.to(dev)
    prepare_fused(m)
    return m.eval().requires_grad_(False)


@torch.no_grad()
def prepare_fused(model) -> None:
    """Give every layer one [q|k|v] projection and one [gate|up] projection.

    The concatenated weights become the storage: q_proj/k_proj/v_proj and
    gate_proj/up_proj are re-pointed to views of them, so memory does not grow
    and the module path keeps working. Works on any model with transformers'
    Qwen2 attribute layout.
    """
    for layer in model.model.layers:
        a, mlp = layer.self_attn, layer.mlp
        if getattr(a, "qkv_weight", None) is not None:
            continue
        ws = [a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]
        bs = [a.q_proj.bias, a.k_proj.bias, a.v_proj.bias]
        qkv_w = torch.cat([w.data for w in ws], 0).contiguous()
        qkv_b = torch.cat([b.data for b in bs], 0).contiguous()
        o = 0
        for lin, w in zip((a.q_proj, a.k_proj, a.v_proj), ws):
            n = w.shape[0]
            lin.weight = nn.Parameter(qkv_w[o:o + n], requires_grad=False)
            lin.bias = nn.Parameter(qkv_b[o:o + n], requires_grad=False)
            o += n
        a.qkv_weight, a.qkv_bias = qkv_w, qkv_b
        gu = torch.cat([mlp.gate_proj.weight.data, mlp.up_proj.weight.data], 0).contiguous()
        f = mlp.gate_proj.weight.shape[0]
        mlp.gate_proj.weight = nn.Parameter(gu[:f], requires_grad=False)
        mlp.up_proj.weight = nn.Parameter(gu[f:], requires_grad=False)
        mlp.gate_up_weight = gu
        _add_blocked(a, mlp)


def _blockable(*ws) -> bool:
    return all(w.is_cuda and w.dtype == torch.bfloat16 and w.dim() == 2 and w.shape[0] % 16 == 0
               and w.shape[1] % 32 == 0 for w in ws)


@torch.no_grad()
def _add_blocked(a, mlp) -> None:
    """Blocked copies (kernels.to_blocked) of a layer's projection weights for
    the split-K layer's direct-to-LDS loads; the row-major weights stay for
    every other path. bf16 on the GPU only."""
    ws = (a.qkv_weight, a.o_proj.weight, mlp.gate_up_weight, mlp.down_proj.weight)
    if not _blockable(*ws):
        return
    from .kernels import to_blocked
    a.qkv_weight_blk, a.o_weight_blk = to_blocked(ws[0]), to_blocked(ws[1])
    mlp.gate_up_weight_blk, mlp.down_weight_blk = to_blocked(ws[2]), to_blocked(ws[3])


@torch.no_grad()
def lm_head_blocked(model) -> torch.Tensor | None:
    """A blocked copy of the LM-head weight (made once and kept on the model),
    or None where the head or its shape does not allow one."""
    blk = getattr(model, "_lm_head_blk", None)
    if blk is None:
        w = lm_head_weight(model)
        if w is None or not _blockable(w):
            return None
        from .kernels import to_blocked
        blk = to_blocked(w)
        model._lm_head_blk = blk
    return blk


def lm_head_weight(model) -> torch.Tensor | None:
    """The dense [V, H] LM-head weight when the head is a plain bias-free Linear
    (the fused argmax kernel applies); None for any other head."""
    head = getattr(model, "lm_head", None)
    if isinstance(head, nn.Linear) and head.bias is None:
        return head.weight
    return None
