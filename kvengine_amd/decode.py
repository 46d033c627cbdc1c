"""Greedy decoding on the HIP path (kvengine/decode.py semantics).

`greedy_paged` is the plain-greedy baseline the speculative sweep is compared
against (kvengine/decode.py:261-332, scripts/phase5_demo.py:93): prefill once,
then one token per forward, argmax over the LM head. Here the LM head and the
argmax are the fused kernel, so each step reads one int32 back instead of a
151936-wide logits row.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch

from . import kernels
from .forward import forward_hidden
from .model import lm_head_weight

AUTO_EOS = "auto"


def _resolve_eos(model, eos_token_id) -> set[int]:
    if eos_token_id == AUTO_EOS:
        eos_token_id = getattr(getattr(model, "generation_config", None), "eos_token_id", None)
    if eos_token_id is None:
        return set()
    if isinstance(eos_token_id, int):
        return {eos_token_id}
    return set(eos_token_id)


def _sync(device: torch.device) -> None:
    if device.type == "cuda":
        torch.cuda.synchronize(device)


def argmax_rows(model, hidden_rows: torch.Tensor) -> torch.Tensor:
    """Greedy ids for hidden rows [M, H] as int32 [M] on the device.

    A plain tied Linear head goes through the fused LM-head argmax kernel; any
    other head (a wrapper that edits logits) is called as given and its logits
    reduced with torch.argmax on the device.
    """
    w = lm_head_weight(model)
    if w is not None:
        return kernels.lmhead_argmax(hidden_rows, w)
    logits = model.lm_head(hidden_rows)
    return torch.argmax(logits, dim=-1).to(torch.int32)


@dataclass
class GenerationResult:
    prompt_token_ids: list[int]
    new_token_ids: list[int]
    elapsed_s: float
    stopped_on_eos: bool
    step_logits: torch.Tensor | None = field(default=None, repr=False)
    cache_utilization: float | None = None
    blocks_held: int | None = None
    sequence: object | None = field(default=None, repr=False)

    @property
    def all_token_ids(self) -> list[int]:
        return self.prompt_token_ids + self.new_token_ids

    @property
    def tokens_per_s(self) -> float:
        return len(self.new_token_ids) / self.elapsed_s if self.elapsed_s else 0.0


def _step(model, cache, ids: torch.Tensor, collect: list | None):
    T = ids.shape[1]
    start = cache.length
    cache.reserve(T)
    hidden = forward_hidden(model, ids, cache.device_kv(), cache.row_dev, start + T)
    cache.commit(T)
    last = hidden[0, -1:, :]
    if collect is not None:
        collect.append(model.lm_head(last)[0].float().cpu())
    return argmax_rows(model, last)


@torch.no_grad()
def greedy_decode(model, input_ids: torch.Tensor, cache, max_new_tokens: int = 32,
                  eos_token_id=AUTO_EOS, collect_logits: bool = False) -> GenerationResult:
    """Greedy decode into any cache with the device_kv/row_dev interface."""
    assert input_ids.dim() == 2 and input_ids.shape[0] == 1, "one request at a time"
    device = cache.device_kv().k.device
    eos_ids = _resolve_eos(model, eos_token_id)
    prompt = input_ids[0].tolist()
    new: list[int] = []
    logs: list | None = [] if collect_logits else None
    stopped = False
    _sync(device)
    t0 = time.perf_counter()
    nxt = _step(model, cache, input_ids.to(device=device, dtype=torch.long), logs)
    for _ in range(max_new_tokens):
        tok = int(nxt.item())
        new.append(tok)
        if tok in eos_ids:
            stopped = True
            break
        # like the reference, the last token is fed too (its K/V lands in the cache)
        nxt = _step(model, cache, nxt.view(1, 1).to(torch.long), logs)
    _sync(device)
    return GenerationResult(prompt, new, time.perf_counter() - t0, stopped,
                            torch.stack(logs) if logs else None)


@torch.no_grad()
def greedy_paged(model, input_ids: torch.Tensor, pool, max_new_tokens: int = 32,
                 eos_token_id=AUTO_EOS, collect_logits: bool = False, request_id: object = "req",
                 free_on_finish: bool = True) -> GenerationResult:
    """Plain greedy on a paged pool; blocks are freed on exit unless asked otherwise."""
    seq = pool.new_sequence(request_id)
    try:
        r = greedy_decode(model, input_ids, seq, max_new_tokens, eos_token_id, collect_logits)
        r.cache_utilization = seq.utilization()
        r.blocks_held = len(seq.blocks)
    finally:
        if free_on_finish:
            seq.free()
    r.sequence = None if free_on_finish else seq
    return r


@torch.no_grad()
def greedy_own_cache(model, input_ids: torch.Tensor, max_new_tokens: int = 32,
                     eos_token_id=AUTO_EOS, collect_logits: bool = False, cache=None,
                     max_seq_len: int | None = None) -> GenerationResult:
    """Greedy decode on a contiguous cache (kvengine/decode.py:193-258)."""
    from .paged import ContiguousKVCache

    if cache is None:
        room = max_seq_len if max_seq_len is not None else input_ids.shape[1] + max_new_tokens
        cache = ContiguousKVCache.for_model(model, max_seq_len=room)
    r = greedy_decode(model, input_ids, cache, max_new_tokens, eos_token_id, collect_logits)
    r.cache_utilization = cache.utilization()
    return r
