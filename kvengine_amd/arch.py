"""Qwen2-family architecture descriptions used by the verify path.

The reference reads these numbers off a transformers config
(kvengine/loader.py:55-73 `model_shape_info`); here they are plain frozen
dataclasses so a model can be built from a seed without any download.
Both presets carry q/k/v biases and tie the LM head to the embedding, which is
what reproduces the reference's published parameter counts exactly
(results/spec_decoding_mps_fp16.json:5-6: 3,085,938,688 and 494,032,768).
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Qwen2Arch:
    name: str
    num_layers: int
    hidden: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    ffn: int
    vocab: int = 151936
    rms_eps: float = 1e-6
    rope_theta: float = 1e6

    @property
    def group(self) -> int:
        return self.num_q_heads // self.num_kv_heads

    @property
    def q_dim(self) -> int:
        return self.num_q_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.num_kv_heads * self.head_dim

    def num_params(self) -> int:
        """Parameter count with tied embeddings and q/k/v biases."""
        h, f = self.hidden, self.ffn
        attn = h * self.q_dim + self.q_dim + 2 * (h * self.kv_dim + self.kv_dim) + self.q_dim * h
        mlp = 3 * h * f
        norms = 2 * h
        return self.num_layers * (attn + mlp + norms) + self.vocab * h + h

    def kv_bytes_per_token(self, elem_bytes: int) -> int:
        """K+V bytes one token occupies across every layer."""
        return 2 * self.num_layers * self.kv_dim * elem_bytes

    def shape_info(self) -> dict:
        """Same keys as the reference's model_shape_info (loader.py:55-73)."""
        return {
            "num_layers": self.num_layers,
            "num_attention_heads": self.num_q_heads,
            "num_key_value_heads": self.num_kv_heads,
            "head_dim": self.head_dim,
            "hidden_size": self.hidden,
            "vocab_size": self.vocab,
        }


QWEN25_0_5B = Qwen2Arch("qwen2.5-0.5b", num_layers=24, hidden=896, num_q_heads=14,
                        num_kv_heads=2, head_dim=64, ffn=4864)
QWEN25_3B = Qwen2Arch("qwen2.5-3b", num_layers=36, hidden=2048, num_q_heads=16,
                      num_kv_heads=2, head_dim=128, ffn=11008)

# Small shapes with the same structure, for tests that must finish in seconds on
# a CPU. TINY keeps the 0.5B head geometry (7 q heads per kv head, head_dim 64);
# TINY128 keeps the 3B geometry (8 per kv head, head_dim 128).
TINY = Qwen2Arch("tiny-gqa7-d64", num_layers=2, hidden=128, num_q_heads=14,
                 num_kv_heads=2, head_dim=64, ffn=256, vocab=1000)
TINY128 = Qwen2Arch("tiny-gqa8-d128", num_layers=2, hidden=256, num_q_heads=16,
                    num_kv_heads=2, head_dim=128, ffn=512, vocab=1024)

PRESETS = {a.name: a for a in (QWEN25_0_5B, QWEN25_3B, TINY, TINY128)}


def layer_slice(arch: Qwen2Arch, num_layers: int) -> Qwen2Arch:
    """The same architecture with fewer layers (fixtures and CPU timing samples)."""
    return Qwen2Arch(f"{arch.name}-L{num_layers}", num_layers, arch.hidden, arch.num_q_heads,
                     arch.num_kv_heads, arch.head_dim, arch.ffn, arch.vocab, arch.rms_eps,
                     arch.rope_theta)
