"""Seeded random weights for the Qwen2 architectures (synthetic, no checkpoint).

Scheme (the same on every machine with this torch build):

* every Linear weight, q/k/v bias and the embedding are N(0, 0.02);
  RMSNorm gains are 1; o_proj and the MLP have no bias; the LM head is the
  embedding (tied), as in transformers' Qwen2 init (modeling_utils `_init_weights`:
  normal(0, initializer_range=0.02) for Linear/Embedding, ones for RMSNorm).
  Biases are drawn rather than zeroed so the bias path is exercised.
* each tensor is filled in chunks of 2**22 elements; chunk c of tensor `name`
  is `torch.randn(n, generator=Generator().manual_seed(s)) * 0.02` in float32,
  with s = blake2b(f"{seed}:{name}:{c}") truncated to 63 bits. Chunks are
  independent, so generation runs on a thread pool and a 3B model takes seconds.
* the float32 values are then cast (round to nearest even) to the model dtype.

Names follow transformers' Qwen2ForCausalLM state dict, so the same dict loads
into that class with `load_state_dict` (the golden-fixture script does this).
"""

from __future__ import annotations

import hashlib
import os
from concurrent.futures import ThreadPoolExecutor

import torch

from .arch import Qwen2Arch

INIT_STD = 0.02
CHUNK = 1 << 22


def param_specs(arch: Qwen2Arch) -> list[tuple[str, tuple[int, ...], str]]:
    """(name, shape, init) for every stored parameter; init is 'normal' or 'ones'."""
    h, f, qd, kd = arch.hidden, arch.ffn, arch.q_dim, arch.kv_dim
    specs: list[tuple[str, tuple[int, ...], str]] = [
        ("model.embed_tokens.weight", (arch.vocab, h), "normal")
    ]
    for i in range(arch.num_layers):
        p = f"model.layers.{i}."
        specs += [
            (p + "self_attn.q_proj.weight", (qd, h), "normal"),
            (p + "self_attn.q_proj.bias", (qd,), "normal"),
            (p + "self_attn.k_proj.weight", (kd, h), "normal"),
            (p + "self_attn.k_proj.bias", (kd,), "normal"),
            (p + "self_attn.v_proj.weight", (kd, h), "normal"),
            (p + "self_attn.v_proj.bias", (kd,), "normal"),
            (p + "self_attn.o_proj.weight", (h, qd), "normal"),
            (p + "mlp.gate_proj.weight", (f, h), "normal"),
            (p + "mlp.up_proj.weight", (f, h), "normal"),
            (p + "mlp.down_proj.weight", (h, f), "normal"),
            (p + "input_layernorm.weight", (h,), "ones"),
            (p + "post_attention_layernorm.weight", (h,), "ones"),
        ]
    specs.append(("model.norm.weight", (h,), "ones"))
    return specs


def _chunk_seed(seed: int, name: str, chunk: int) -> int:
    digest = hashlib.blake2b(f"{seed}:{name}:{chunk}".encode(), digest_size=8).digest()
    return int.from_bytes(digest, "little") & ((1 << 63) - 1)


def _fill_chunk(flat: torch.Tensor, seed: int, name: str, chunk: int) -> None:
    lo = chunk * CHUNK
    n = min(CHUNK, flat.numel() - lo)
    g = torch.Generator().manual_seed(_chunk_seed(seed, name, chunk))
    vals = torch.randn(n, generator=g, dtype=torch.float32) * INIT_STD
    flat[lo:lo + n].copy_(vals)  # copy_ casts with round-to-nearest-even


def generate_state_dict(arch: Qwen2Arch, seed: int, dtype: torch.dtype = torch.float32,
                        threads: int | None = None) -> dict[str, torch.Tensor]:
    """CPU state dict (HF names, tied LM head omitted) for `arch` at `seed`."""
    threads = threads or min(16, os.cpu_count() or 1)
    out: dict[str, torch.Tensor] = {}
    jobs = []
    for name, shape, init in param_specs(arch):
        t = torch.empty(shape, dtype=dtype)
        out[name] = t
        if init == "ones":
            t.fill_(1.0)
            continue
        flat = t.view(-1)
        for c in range((flat.numel() + CHUNK - 1) // CHUNK):
            jobs.append((flat, name, c))
    # torch releases the GIL inside randn/copy_, so threads scale.
    prev = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        with ThreadPoolExecutor(max_workers=threads) as ex:
            list(ex.map(lambda j: _fill_chunk(j[0], seed, j[1], j[2]), jobs))
    finally:
        torch.set_num_threads(prev)
    return out


def state_dict_checksum(sd: dict[str, torch.Tensor]) -> str:
    """Short content hash, recorded next to fixtures so weight drift is detected."""
    h = hashlib.blake2b(digest_size=8)
    for name in sorted(sd):
        t = sd[name].contiguous()
        h.update(name.encode())
        h.update(t.view(torch.uint8).numpy().tobytes() if t.dtype != torch.bfloat16
                 else t.view(torch.int16).numpy().tobytes())
    return h.hexdigest()
