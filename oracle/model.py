"""Oracle Qwen2 forward pass. TEST INFRASTRUCTURE.

Restates kvengine/forward.py:147-215 (`forward_with_own_cache`) together with the
transformers Qwen2 modules it calls, using the same torch calls in the same
order so that on the CPU the results are bit-identical to the reference:

* embedding: F.embedding (forward.py:176)
* rotary: inv_freq = 1/(theta ** (arange(0, D, 2, float32)/D)); freqs =
  (inv_freq[None,:,None] @ pos[:,None,:]).transpose(1,2); emb = cat(freqs,
  freqs); cos/sin in float32 times attention_scaling (1.0), then cast to the
  model dtype (transformers models/qwen2/modeling_qwen2.py:51-102; forward.py:180)
* causal mask: additive finfo(dtype).min where key > L-T+i, None when T == 1
  (forward.py:85-103)
* RMSNorm: float32 variance, x*rsqrt(var+eps), cast back, then weight * x
  (modeling_qwen2.py:237-255)
* q/k/v: F.linear with bias, view [1,T,H,D] then transpose(1,2) (forward.py:193-196)
* RoPE: x*cos + rotate_half(x)*sin with cos/sin unsqueezed on dim 1
  (forward.py:49-69)
* cache.write then attend: repeat_kv, then SDPA with the additive mask and
  scale D**-0.5, or the eager float32-softmax form (forward.py:106-144)
* o_proj without bias, residual add, post-attention RMSNorm, SwiGLU MLP
  down(silu(gate(x)) * up(x)), residual add (forward.py:204-207;
  modeling_qwen2.py:35-48)
* final norm, tied LM head on all rows or the last row (forward.py:212-215)
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

USE_SDPA = True


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat([-x[..., half:], x[..., :half]], dim=-1)


def apply_rope(q, k, cos, sin):
    cos = cos.unsqueeze(1)
    sin = sin.unsqueeze(1)
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    if n_rep == 1:
        return x
    b, h, t, d = x.shape
    return x[:, :, None, :, :].expand(b, h, n_rep, t, d).reshape(b, h * n_rep, t, d)


def causal_mask(q_len: int, kv_len: int, dtype, device="cpu"):
    if q_len == 1:
        return None
    q_pos = torch.arange(kv_len - q_len, kv_len, device=device).unsqueeze(1)
    k_pos = torch.arange(kv_len, device=device).unsqueeze(0)
    mask = torch.zeros(q_len, kv_len, dtype=dtype, device=device)
    mask.masked_fill_(k_pos > q_pos, torch.finfo(dtype).min)
    return mask[None, None, :, :]


def attend(q, k, v, mask, n_rep: int, scaling: float, use_sdpa: bool | None = None):
    """q [B,Hq,T,D], k/v [B,Hkv,L,D] -> [B,T,Hq,D]."""
    if use_sdpa is None:
        use_sdpa = USE_SDPA
    k = repeat_kv(k, n_rep)
    v = repeat_kv(v, n_rep)
    if use_sdpa:
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=scaling)
        return out.transpose(1, 2).contiguous()
    scores = torch.matmul(q, k.transpose(2, 3)) * scaling
    if mask is not None:
        scores = scores + mask
    probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(q.dtype)
    return torch.matmul(probs, v).transpose(1, 2).contiguous()


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    in_dtype = x.dtype
    x = x.to(torch.float32)
    var = x.pow(2).mean(-1, keepdim=True)
    x = x * torch.rsqrt(var + eps)
    return weight * x.to(in_dtype)


class RefQwen2:
    """CPU Qwen2 with tied embeddings, driven like kvengine's forward pass."""

    def __init__(self, arch, state_dict: dict, dtype=torch.float32):
        self.arch = arch
        self.dtype = dtype
        self.w = {n: t.to(dtype) for n, t in state_dict.items()}
        self.scaling = arch.head_dim ** -0.5
        self.n_rep = arch.num_q_heads // arch.num_kv_heads
        d = arch.head_dim
        self.inv_freq = 1.0 / (arch.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float) / d))
        self.lm_head_hook = None  # optional transform of logits (hostile drafts)

    def rotary(self, x: torch.Tensor, position_ids: torch.Tensor):
        inv = self.inv_freq[None, :, None].float().expand(position_ids.shape[0], -1, 1)
        pos = position_ids[:, None, :].float()
        freqs = (inv.float() @ pos.float()).transpose(1, 2)
        emb = torch.cat((freqs, freqs), dim=-1)
        cos = emb.cos() * 1.0
        sin = emb.sin() * 1.0
        return cos.to(dtype=x.dtype), sin.to(dtype=x.dtype)

    def lm_head(self, hidden: torch.Tensor) -> torch.Tensor:
        logits = F.linear(hidden, self.w["model.embed_tokens.weight"])
        if self.lm_head_hook is not None:
            logits = self.lm_head_hook(logits)
        return logits

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor, cache, all_logits: bool = False,
                return_hidden: bool = False):
        assert input_ids.dim() == 2 and input_ids.shape[0] == 1
        a, w = self.arch, self.w
        T = input_ids.shape[1]
        start = cache.length
        cache.reserve(T)
        hidden = F.embedding(input_ids, w["model.embed_tokens.weight"])
        position_ids = torch.arange(start, start + T).unsqueeze(0)
        cos, sin = self.rotary(hidden, position_ids)
        mask = causal_mask(T, start + T, hidden.dtype)
        for i in range(a.num_layers):
            p = f"model.layers.{i}."
            residual = hidden
            h = rms_norm(hidden, w[p + "input_layernorm.weight"], a.rms_eps)
            shape = (1, T, -1, a.head_dim)
            q = F.linear(h, w[p + "self_attn.q_proj.weight"], w[p + "self_attn.q_proj.bias"])
            k = F.linear(h, w[p + "self_attn.k_proj.weight"], w[p + "self_attn.k_proj.bias"])
            v = F.linear(h, w[p + "self_attn.v_proj.weight"], w[p + "self_attn.v_proj.bias"])
            q = q.view(shape).transpose(1, 2)
            k = k.view(shape).transpose(1, 2)
            v = v.view(shape).transpose(1, 2)
            q, k = apply_rope(q, k, cos, sin)
            k_all, v_all = cache.write(i, k, v, start)
            out = attend(q, k_all, v_all, mask, self.n_rep, self.scaling)
            hidden = residual + F.linear(out.reshape(1, T, -1), w[p + "self_attn.o_proj.weight"])
            residual = hidden
            h = rms_norm(hidden, w[p + "post_attention_layernorm.weight"], a.rms_eps)
            gate = F.linear(h, w[p + "mlp.gate_proj.weight"])
            up = F.linear(h, w[p + "mlp.up_proj.weight"])
            hidden = residual + F.linear(F.silu(gate) * up, w[p + "mlp.down_proj.weight"])
        cache.commit(T)
        hidden = rms_norm(hidden, w["model.norm.weight"], a.rms_eps)
        if not all_logits:
            hidden = hidden[:, -1:, :]
        if return_hidden:
            return hidden
        return self.lm_head(hidden)
