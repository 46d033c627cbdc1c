"""kvengine_amd: kvengine's speculative-decoding verify path on MI355X (gfx950).

Host API mirrors kvengine (BlockManager, PagedKVCache / PagedSequenceCache,
forward_with_own_cache, speculative_greedy); the attention, KV write/rollback,
LM-head argmax and accept steps run as HIP kernels from `_kve.so`.
"""

from .arch import QWEN25_0_5B, QWEN25_3B, Qwen2Arch

__all__ = ["QWEN25_0_5B", "QWEN25_3B", "Qwen2Arch"]
