"""Oracle speculative loop, plain greedy, accept and rollback. TEST INFRASTRUCTURE.

Restates kvengine/speculative.py:111-215 and kvengine/decode.py:261-332:

* each iteration feeds the draft the tokens its cache has not seen
  (speculative.py:149-151), then k-1 single-token feeds, proposing
  argmax(logits[-1]) each time (154-158); `propose` optionally replaces the
  proposal (oracle-acceptance drafts) while the draft forwards still run
* the target is fed unseen + drafts in one pass (160-164); preds =
  argmax(t_logits[u-1:]) (167)
* n_acc = longest agreeing prefix, emitted = drafts[:n_acc] + [preds[n_acc]]
  (169-182)
* keep = len(tokens)-1; both caches truncate to min(length, keep) (193-197)
* EOS cut (199-206) and budget trim (211-214)

`accept_closed_form` and `keep_lengths` state the same arithmetic without loops,
for the exhaustive pinning test.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch


@dataclass
class RefSpecResult:
    prompt_token_ids: list
    new_token_ids: list
    elapsed_s: float = 0.0
    stopped_on_eos: bool = False
    iterations: int = 0
    tokens_drafted: int = 0
    tokens_accepted: int = 0
    accepted_per_iter: list = field(default_factory=list)
    target_forwards: int = 0
    draft_forwards: int = 0
    # per iteration: (target blocks, draft blocks) after rollback, when paged
    block_trace: list = field(default_factory=list)
    # per iteration: target float32 logits rows [k+1, V] (only if asked)
    verify_logits: list = field(default_factory=list)

    @property
    def acceptance_rate(self) -> float:
        return self.tokens_accepted / self.tokens_drafted if self.tokens_drafted else 0.0


def accept(drafts: list[int], preds: list[int]) -> tuple[int, list[int]]:
    """Longest agreeing prefix and the emitted tokens (speculative.py:169-182)."""
    k = len(drafts)
    n = 0
    while n < k and preds[n] == drafts[n]:
        n += 1
    return n, list(drafts[:n]) + [preds[n]]


def accept_closed_form(agree: list[bool]) -> int:
    """n_acc from an agreement mask: index of the first False, else k."""
    return next((i for i, a in enumerate(agree) if not a), len(agree))


def keep_lengths(n_tokens_before: int, target_len_before: int, draft_len_after: int,
                 u: int, k: int, n_acc: int) -> tuple[int, int]:
    """Target/draft lengths after rollback (speculative.py:193-197).

    n_tokens_before: len(tokens) before the iteration's tokens are appended.
    """
    keep = n_tokens_before + n_acc + 1 - 1
    target_after_verify = target_len_before + u + k
    return min(target_after_verify, keep), min(draft_len_after, keep)


@torch.no_grad()
def ref_speculative_greedy(target, draft, input_ids, t_cache, d_cache, k=4, max_new_tokens=32,
                           eos_ids=(), propose=None, record_logits=False, deadline_s=None,
                           forced_preds=None):
    """deadline_s: stop after the iteration that crosses this many seconds
    (bounded CPU-baseline samples); None runs to the budget like the reference.
    forced_preds: a token list by absolute position (prompt + a continuation)
    that replaces the target's argmax wherever it reaches: a timing replay in
    which the target behaves as that continuation while every forward and
    argmax still runs (the reference's own bf16 verify and decode passes
    choose different ids at near ties, so its greedy continuation is not what
    its verify passes pick)."""
    assert input_ids.dim() == 2 and input_ids.shape[0] == 1
    assert k >= 1
    assert t_cache.length == 0 and d_cache.length == 0
    eos_ids = set(eos_ids)
    prompt = input_ids[0].tolist()
    tokens = list(prompt)
    res = RefSpecResult(prompt_token_ids=prompt, new_token_ids=[])

    def feed(model, cache, ids):
        return model.forward(torch.tensor([ids], dtype=torch.long), cache, all_logits=True)[0]

    t0 = time.perf_counter()
    while len(res.new_token_ids) < max_new_tokens:
        logits = feed(draft, d_cache, tokens[d_cache.length:])
        res.draft_forwards += 1
        drafts: list[int] = []
        for j in range(k):
            proposal = int(torch.argmax(logits[-1]))
            if propose is not None:
                proposal = propose(len(tokens) + j, proposal)
            drafts.append(proposal)
            if j < k - 1:
                logits = feed(draft, d_cache, [drafts[-1]])
                res.draft_forwards += 1
        unseen = tokens[t_cache.length:]
        u = len(unseen)
        t_logits = feed(target, t_cache, unseen + drafts)
        res.target_forwards += 1
        rows = t_logits[u - 1:]
        if record_logits:
            res.verify_logits.append(rows.float().clone())
        preds = torch.argmax(rows, dim=-1).tolist()
        if forced_preds is not None:
            base = len(tokens)
            preds = [forced_preds[base + j] if base + j < len(forced_preds) else pr
                     for j, pr in enumerate(preds)]
        n_acc, emitted = accept(drafts, preds)
        res.iterations += 1
        res.tokens_drafted += k
        res.tokens_accepted += n_acc
        res.accepted_per_iter.append(n_acc)
        tokens.extend(emitted)
        res.new_token_ids.extend(emitted)
        keep = len(tokens) - 1
        t_cache.truncate(min(t_cache.length, keep))
        d_cache.truncate(min(d_cache.length, keep))
        if hasattr(t_cache, "blocks"):
            res.block_trace.append((list(t_cache.blocks), list(d_cache.blocks)))
        if any(t in eos_ids for t in emitted):
            first = next(i for i, t in enumerate(emitted) if t in eos_ids)
            trim = len(emitted) - (first + 1)
            if trim:
                res.new_token_ids = res.new_token_ids[:-trim]
            res.stopped_on_eos = True
            break
        if deadline_s is not None and time.perf_counter() - t0 > deadline_s:
            break
    res.elapsed_s = time.perf_counter() - t0
    if len(res.new_token_ids) > max_new_tokens:
        res.new_token_ids = res.new_token_ids[:max_new_tokens]
        res.stopped_on_eos = res.new_token_ids[-1] in eos_ids
    return res


@dataclass
class RefGreedyResult:
    prompt_token_ids: list
    new_token_ids: list
    step_logits: torch.Tensor | None = None
    elapsed_s: float = 0.0


@torch.no_grad()
def ref_greedy(model, input_ids, cache, max_new_tokens=32, eos_ids=(), collect_logits=False):
    """Plain greedy on one cache (decode.py:261-332 without the pool plumbing)."""
    eos_ids = set(eos_ids)
    prompt = input_ids[0].tolist()
    out: list[int] = []
    rows = []
    t0 = time.perf_counter()
    logits = model.forward(input_ids, cache)
    nxt = logits[0, -1, :]
    for _ in range(max_new_tokens):
        if collect_logits:
            rows.append(nxt.detach().float().clone())
        tok = int(torch.argmax(nxt))
        out.append(tok)
        if tok in eos_ids:
            break
        logits = model.forward(torch.tensor([[tok]], dtype=torch.long), cache)
        nxt = logits[0, -1, :]
    return RefGreedyResult(prompt, out, torch.stack(rows) if rows else None,
                           time.perf_counter() - t0)


def top2_margin(logits_row: torch.Tensor) -> float:
    """top-1 minus top-2 logit of one row (ties give 0)."""
    v = torch.topk(logits_row.float(), 2).values
    return float(v[0] - v[1])
