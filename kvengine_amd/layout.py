"""Conversions between the reference pool layout and the kernel layout.

Reference (kvengine/paged.py:59-61): K and V both [NB, bs, Hkv, D].
Kernel: K [NB, Hkv, bs, D] (each (block, head) a contiguous token-major tile),
        V [NB, Hkv, D, bs] (each (block, head) a contiguous channel-major tile).
The extra layer axis in front (when present) is carried through unchanged.
"""

from __future__ import annotations

import torch


def to_kernel_layout(k_ref: torch.Tensor, v_ref: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """[..., NB, bs, Hkv, D] -> (K [..., NB, Hkv, bs, D], V [..., NB, Hkv, D, bs])."""
    k = k_ref.transpose(-3, -2).contiguous()
    v = v_ref.permute(*range(v_ref.dim() - 3), -2, -1, -3).contiguous()
    return k, v


def to_reference_layout(k: torch.Tensor, v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Inverse of to_kernel_layout."""
    k_ref = k.transpose(-3, -2).contiguous()
    v_ref = v.permute(*range(v.dim() - 3), -1, -3, -2).contiguous()
    return k_ref, v_ref
