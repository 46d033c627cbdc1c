"""Greedy speculative decoding on the HIP path, with kvengine's API and semantics.

`speculative_greedy` follows kvengine/speculative.py:111-215 step for step:
the draft is fed the tokens its cache has not seen, then k-1 single tokens,
proposing argmax(logits[-1]) each time; the target verifies unseen + drafts in
one pass; n_acc is the longest agreeing prefix and the emitted tokens are
drafts[:n_acc] + [target's prediction at n_acc]; both caches roll back to
len(tokens)-1; EOS and the budget trim the output. Cache reserve/commit/
truncate calls happen in the same order, so block tables match the reference
bit for bit.

What changes is where the work runs. Drafts stay on the device: each proposal
is the fused LM-head argmax kernel's int32 output, fed straight into the next
draft forward; the target's k+1 predictions, the accept loop and the keep
length are kernels too. The host reads back one small vector per iteration
(n_acc and the emitted tokens), where the reference synchronises once per
draft token and once per verify (speculative.py:155,167).

`propose` (optional) replaces draft proposals: an object with
`predraw(pos) -> token or -1` is applied on the device without a sync (the
oracle-acceptance drafts); any other callable `propose(pos, natural)` is called
with the draft's own proposal, which costs a read-back per token.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch

from . import kernels
from .decode import AUTO_EOS, _resolve_eos, _sync, argmax_rows
from .forward import forward_hidden


@dataclass
class SpecDecodeResult:
    prompt_token_ids: list[int]
    new_token_ids: list[int]
    elapsed_s: float
    stopped_on_eos: bool
    iterations: int = 0
    tokens_drafted: int = 0
    tokens_accepted: int = 0
    accepted_per_iter: list[int] = field(default_factory=list)
    target_forwards: int = 0
    draft_forwards: int = 0

    @property
    def tokens_per_s(self) -> float:
        return len(self.new_token_ids) / self.elapsed_s if self.elapsed_s else 0.0

    @property
    def acceptance_rate(self) -> float:
        """Accepted prefix tokens / drafted tokens (kvengine/speculative.py:75-81)."""
        return self.tokens_accepted / self.tokens_drafted if self.tokens_drafted else 0.0

    @property
    def tokens_per_target_forward(self) -> float:
        return len(self.new_token_ids) / self.target_forwards if self.target_forwards else 0.0

    def summary(self) -> dict:
        return {
            "new_tokens": len(self.new_token_ids),
            "elapsed_s": round(self.elapsed_s, 3),
            "tokens_per_s": round(self.tokens_per_s, 2),
            "iterations": self.iterations,
            "tokens_drafted": self.tokens_drafted,
            "tokens_accepted": self.tokens_accepted,
            "acceptance_rate": round(self.acceptance_rate, 4),
            "tokens_per_target_forward": round(self.tokens_per_target_forward, 3),
            "target_forwards": self.target_forwards,
            "draft_forwards": self.draft_forwards,
            "stopped_on_eos": self.stopped_on_eos,
        }


def _feed(model, cache, ids: torch.Tensor) -> torch.Tensor:
    """One forward of ids [1, T] into cache; returns hidden [T, H]."""
    T = ids.shape[1]
    start = cache.length
    cache.reserve(T)
    hidden = forward_hidden(model, ids, cache.device_kv(), cache.row_dev, start + T)
    cache.commit(T)
    return hidden[0]


@torch.no_grad()
def speculative_greedy(target_model, draft_model, input_ids: torch.Tensor, target_cache,
                       draft_cache, k: int = 4, max_new_tokens: int = 32,
                       eos_token_id=AUTO_EOS, propose=None) -> SpecDecodeResult:
    """Greedy speculative decoding; output equals greedy decoding of the target."""
    assert input_ids.dim() == 2 and input_ids.shape[0] == 1, "one request at a time"
    assert k >= 1, "k must be at least 1"
    assert target_cache.length == 0 and draft_cache.length == 0, "caches must be empty"
    device = target_cache.device_kv().k.device
    eos_ids = _resolve_eos(target_model, eos_token_id)
    prompt = input_ids[0].tolist()
    tokens = list(prompt)
    res = SpecDecodeResult(prompt_token_ids=prompt, new_token_ids=[], elapsed_s=0.0,
                           stopped_on_eos=False)
    drafts = torch.empty(k, dtype=torch.int32, device=device)
    predraw = getattr(propose, "predraw", None)

    def host_ids(lst):
        return torch.tensor([lst], dtype=torch.long).to(device, non_blocking=True)

    _sync(device)
    t0 = time.perf_counter()
    while len(res.new_token_ids) < max_new_tokens:
        # --- 1. draft proposes k tokens; proposals never leave the device ---
        hidden = _feed(draft_model, draft_cache, host_ids(tokens[draft_cache.length:]))
        res.draft_forwards += 1
        for j in range(k):
            prop = argmax_rows(draft_model, hidden[-1:])
            if predraw is not None:
                forced = predraw(len(tokens) + j)
                if forced >= 0:
                    prop.fill_(forced)
            elif propose is not None:
                prop.fill_(int(propose(len(tokens) + j, int(prop.item()))))
            drafts[j:j + 1].copy_(prop)
            if j < k - 1:
                hidden = _feed(draft_model, draft_cache, drafts[j:j + 1].view(1, 1).to(torch.long))
                res.draft_forwards += 1

        # --- 2. target verifies all k in one pass ---
        unseen = tokens[target_cache.length:]
        u = len(unseen)
        ids = torch.cat([host_ids(unseen)[0], drafts.to(torch.long)]).view(1, -1)
        hidden_t = _feed(target_model, target_cache, ids)
        res.target_forwards += 1
        preds = argmax_rows(target_model, hidden_t[u - 1:])

        # --- 3. accept on the device, one read-back ---
        n_acc_d, emitted_d, _ = kernels.accept(drafts.view(1, k), preds.view(1, k + 1))
        back = torch.cat([n_acc_d, emitted_d[0]]).cpu().tolist()
        n_acc = back[0]
        emitted = back[1:2 + n_acc]
        res.iterations += 1
        res.tokens_drafted += k
        res.tokens_accepted += n_acc
        res.accepted_per_iter.append(n_acc)

        # --- 4. commit and roll both caches back to the accepted sequence ---
        tokens.extend(emitted)
        res.new_token_ids.extend(emitted)
        keep = len(tokens) - 1
        target_cache.truncate(min(target_cache.length, keep))
        draft_cache.truncate(min(draft_cache.length, keep))

        if any(t in eos_ids for t in emitted):
            first = next(i for i, t in enumerate(emitted) if t in eos_ids)
            trim = len(emitted) - (first + 1)
            if trim:
                res.new_token_ids = res.new_token_ids[:-trim]
            res.stopped_on_eos = True
            break

    _sync(device)
    res.elapsed_s = time.perf_counter() - t0
    if len(res.new_token_ids) > max_new_tokens:
        res.new_token_ids = res.new_token_ids[:max_new_tokens]
        res.stopped_on_eos = res.new_token_ids[-1] in eos_ids
    return res
