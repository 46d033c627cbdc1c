"""Oracle lockstep replay of batched speculative decoding. TEST INFRASTRUCTURE.

Runs the reference's per-request speculative algorithm
(kvengine/speculative.py:147-206, restated in oracle/spec.py) for several
requests in lockstep over shared reference-layout pools, with the scheduling
policy the batched engine documents:

* admission: FIFO into free slots in ascending order; a request is admitted if
  blocks_needed(len(tokens)-1 + k + 1) fits the free count of both pools, and
  its tokens[:-1] are prefilled into the target, then the draft
  (the reference Engine admits FIFO against free blocks, engine.py:284-324;
  its recompute prefill input is prompt + outputs[:-1], engine.py:137-146)
* per iteration: if the blocks the iteration will allocate do not fit, preempt
  the most recently admitted request (free target then draft, requeue at the
  front) and re-check (engine.py:394-403, 425-440);
  then allocation order: draft feed 1 for every slot (ascending), draft feeds
  2..k each for every slot, the verify for every slot;
  then per slot (ascending): extend tokens, target truncate then draft truncate
  to min(length, len(tokens)-1), EOS/budget trim, retire (free target then
  draft);
* after the iteration, admit again.

Prefix sharing (share_prefixes=True; the reference Engine's, engine.py:314-319,
364-369, 414-419): at admission each cache adopts the published full blocks of
the request's tokens (paged.py:209-245) and only the rest is prefilled; the
full blocks are published after the prefill and again after every iteration
(generated tokens are shareable too), once both caches are truncated.

Abort backstops (the reference Engine's, engine.py:262-267, 297-306, 394-402):
a request that could never be admitted (its first iteration needs more blocks
than a pool holds, or prompt + budget + k + 2 exceeds max_ctx when given) is
retired as aborted_prompt_too_long and admission goes on; a lone running
request whose iteration does not fit is retired as aborted_cache_exhausted;
when nothing runs and nothing can be admitted the head of the queue is retired
as aborted_no_progress. Finished requests carry "eos" or "length".
"""

from __future__ import annotations

import torch

from .spec import accept


class RefLockstepRequest:
    def __init__(self, request_id, prompt, max_new_tokens, propose=None, eos_ids=()):
        self.request_id = request_id
        self.prompt = list(prompt)
        self.max_new_tokens = max_new_tokens
        self.propose = propose
        self.eos_ids = set(eos_ids)
        self.new_token_ids: list[int] = []
        self.accepted_per_iter: list[int] = []
        self.preemptions = 0
        self.finished = False
        self.finish_reason = None
        self.stopped_on_eos = False
        self.prefix_reused = 0

    @property
    def tokens(self):
        return self.prompt + self.new_token_ids


def ref_lockstep_spec(target, draft, requests, k, slots, t_pool, d_pool, trace=None,
                      max_ctx=None, events=None, share_prefixes=False):
    """Decode `requests` to completion; `trace` (a list) receives, after every
    iteration, [(slot, request_id, target blocks, draft blocks), ...];
    `events` (a list) receives ("admit", id, slot), ("preempt", id) and
    ("finish", id, reason) in the order they happen."""
    queue = list(requests)
    done = []

    def event(*e):
        if events is not None:
            events.append(e)
    S = slots
    live: list = [None] * S     # (req, t_seq, d_seq)
    order: list[int] = []

    def feed(model, seq, ids):
        return model.forward(torch.tensor([ids], dtype=torch.long), seq, all_logits=True)[0]

    def release(i):
        req, t, d = live[i]
        t.free()
        d.free()
        live[i] = None
        order.remove(i)

    def finish(req, reason):
        req.finished = True
        req.finish_reason = reason
        done.append(req)
        event("finish", req.request_id, reason)

    def admit():
        i = 0
        while i < S and queue:
            if live[i] is not None:
                i += 1
                continue
            req = queue[0]
            n = len(req.tokens) - 1
            first = n + k + 1
            too_long = max_ctx is not None and (
                len(req.tokens) + req.max_new_tokens - len(req.new_token_ids) + k + 2 > max_ctx)
            if (too_long or t_pool.manager.blocks_needed(first) > t_pool.manager.num_blocks
                    or d_pool.manager.blocks_needed(first) > d_pool.manager.num_blocks):
                finish(queue.pop(0), "aborted_prompt_too_long")
                continue
            if (t_pool.manager.blocks_needed(first) > t_pool.manager.num_free
                    or d_pool.manager.blocks_needed(first) > d_pool.manager.num_free):
                return
            t = t_pool.new_sequence(req.request_id)
            d = d_pool.new_sequence(req.request_id)
            toks = req.tokens
            nt = t.adopt_prefix(toks) if share_prefixes else 0
            nd = d.adopt_prefix(toks) if share_prefixes else 0
            if n > nt:
                feed(target, t, toks[nt:-1])
            if n > nd:
                feed(draft, d, toks[nd:-1])
            if share_prefixes:
                req.prefix_reused += nt + nd
                t.register_prefix_blocks(toks)
                d.register_prefix_blocks(toks)
            queue.pop(0)
            live[i] = (req, t, d)
            order.append(i)
            event("admit", req.request_id, i)
            i += 1

    def demand():
        nt = nd = 0
        for e in live:
            if e is None:
                continue
            req, t, d = e
            u = len(req.tokens) - d.length
            nd += max(0, d_pool.manager.blocks_needed(d.length + u + k - 1) - len(d.blocks))
            nt += max(0, t_pool.manager.blocks_needed(t.length + k + 1) - len(t.blocks))
        return nt, nd

    admit()
    while any(e is not None for e in live) or queue:
        if all(e is None for e in live):
            admit()
            if all(e is None for e in live):
                if queue:
                    finish(queue.pop(0), "aborted_no_progress")
                continue
        while True:
            nt, nd = demand()
            if nt <= t_pool.manager.num_free and nd <= d_pool.manager.num_free:
                break
            if len(order) <= 1:
                req = live[order[0]][0]
                release(order[0])
                finish(req, "aborted_cache_exhausted")
                break
            victim = order[-1]
            req = live[victim][0]
            req.preemptions += 1
            release(victim)
            queue.insert(0, req)
            event("preempt", req.request_id)
        act = [i for i in range(S) if live[i] is not None]
        if not act:
            continue
        drafts = {i: [] for i in act}
        logits = {}
        for i in act:
            req, t, d = live[i]
            logits[i] = feed(draft, d, req.tokens[d.length:])
        for j in range(k):
            for i in act:
                req, t, d = live[i]
                prop = int(torch.argmax(logits[i][-1]))
                if req.propose is not None:
                    prop = req.propose(len(req.tokens) + j, prop)
                drafts[i].append(prop)
            if j < k - 1:
                for i in act:
                    req, t, d = live[i]
                    logits[i] = feed(draft, d, [drafts[i][-1]])
        preds = {}
        for i in act:
            req, t, d = live[i]
            unseen = req.tokens[t.length:]
            tl = feed(target, t, unseen + drafts[i])
            preds[i] = torch.argmax(tl[len(unseen) - 1:], dim=-1).tolist()
        for i in act:
            req, t, d = live[i]
            n, emitted = accept(drafts[i], preds[i])
            req.new_token_ids.extend(emitted)
            req.accepted_per_iter.append(n)
            keep = len(req.tokens) - 1
            t.truncate(min(t.length, keep))
            d.truncate(min(d.length, keep))
            if share_prefixes:
                t.register_prefix_blocks(req.tokens)
                d.register_prefix_blocks(req.tokens)
            if any(x in req.eos_ids for x in emitted):
                first = next(j for j, x in enumerate(emitted) if x in req.eos_ids)
                trim = len(emitted) - (first + 1)
                if trim:
                    del req.new_token_ids[-trim:]
                req.stopped_on_eos = True
            if req.stopped_on_eos or len(req.new_token_ids) >= req.max_new_tokens:
                if len(req.new_token_ids) > req.max_new_tokens:
                    del req.new_token_ids[req.max_new_tokens:]
                    req.stopped_on_eos = req.new_token_ids[-1] in req.eos_ids
                release(i)
                finish(req, "eos" if req.stopped_on_eos else "length")
        if trace is not None:
            trace.append([(i, live[i][0].request_id, list(live[i][1].blocks), list(live[i][2].blocks))
                          for i in range(S) if live[i] is not None])
        if queue:
            admit()
    return requests
