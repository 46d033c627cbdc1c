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

Steady-state iterations (the target has one unseen token, the draft one or
two) of bf16 models with plain tied LM heads on paged caches replay a HIP graph
per draft feed length and context bucket: issued one kernel at a time from
Python, an iteration's ~700 launches cost more host time than the GPU spends
on them. Each iteration's cache blocks are reserved before the replay (in the
reference's order: the draft's u + k - 1 tokens, then the target's k + 1; the
allocator hands out blocks one at a time, so the tables are the same as with
one reserve per pass), the graph commits and rolls back the device lengths and
tables, and the host applies the same commits and truncates to its own
bookkeeping afterwards. The context bucket keeps each pass's attention
summation order (the automatic order depends on the bound only through whether
it passes 896 tokens), so a replayed iteration gives the eager iteration's bits.
"""

from __future__ import annotations

import time
import weakref
from dataclasses import dataclass, field

import torch

from . import kernels
from .decode import AUTO_EOS, _resolve_eos, _sync, argmax_rows
from .forward import forward_hidden
from .model import lm_head_weight
from .paged import PagedSequenceCache


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


# Context bucket of the replayed iterations: the automatic attention order of a
# pass depends on its bound only through whether it exceeds one unit record
# (56 blocks of 16 tokens), so a bucket on the same side of that bound as every
# pass's exact bound (start + tokens) sums every row as the eager pass does.
ONE_UNIT_CTX = 896
CTX_STEP = 256


class _IterationGraphs:
    """Steady-state speculative iterations of one (target, draft, target pool,
    draft pool, k) as replayed HIP graphs, one per draft feed length u (1 or 2)
    and context bucket: the draft's k passes with their picks (oracle overrides
    applied on the device), the verify pass and its argmax rows, the accept,
    the device commits and both caches' rollbacks to the accepted length, then
    one read-back of (n_acc, emitted). The sequences' table rows are inputs of
    the replay, so the graphs serve every later call on the same models and
    pools (`for_call`); the first iteration of a shape runs the same launches
    eagerly as a real iteration and the capture follows it."""

    def __init__(self, t_pool, k: int):
        dev = t_pool.device
        self.k = k
        # feed[2], last token, overrides[k], target row, draft row
        self.inp_host = torch.zeros(5 + k, dtype=torch.long).pin_memory()
        self.inp = torch.zeros(5 + k, dtype=torch.long, device=dev)
        self.drafts = torch.zeros(k, dtype=torch.int32, device=dev)
        self.out = torch.zeros(k + 2, dtype=torch.int32, device=dev)  # n_acc, emitted[k + 1]
        self.stream = torch.cuda.Stream(device=dev)
        self.graphs: dict[tuple[int, int], torch.cuda.CUDAGraph] = {}
        self.t = self.d = self.target = self.draft = None  # bound for one call

    @staticmethod
    def usable(target, draft, t_cache, d_cache, propose) -> bool:
        p, q = next(target.parameters()), next(draft.parameters())
        return (p.is_cuda and p.dtype == torch.bfloat16 and q.dtype == torch.bfloat16
                and lm_head_weight(target) is not None and lm_head_weight(draft) is not None
                and isinstance(t_cache, PagedSequenceCache)
                and isinstance(d_cache, PagedSequenceCache)
                and (propose is None or hasattr(propose, "predraw")))

    @staticmethod
    def for_call(target, draft, t_cache, d_cache, k: int) -> "_IterationGraphs":
        """The graphs of these models and pools (made on first use; dropped
        when any of them is freed), bound to this call's caches."""
        tp, dp = t_cache.pool, d_cache.pool
        # every address a replay reads: a model whose weights or a pool whose
        # tables were replaced since the capture gets new graphs
        key = (id(target), id(draft), id(tp), id(dp), k, _addresses(target), _addresses(draft),
               tuple(t.data_ptr() for p in (tp, dp) for t in (p.tables, p.lens, p.k, p.v)))
        g = _GRAPHS.get(key)
        if g is None:
            g = _GRAPHS[key] = _IterationGraphs(t_cache.pool, k)
            for obj in (target, draft, t_cache.pool, d_cache.pool):
                weakref.finalize(obj, _GRAPHS.pop, key, None)
        g.target, g.draft, g.t, g.d = target, draft, t_cache, d_cache
        return g

    def unbind(self) -> None:
        self.t = self.d = self.target = self.draft = None

    def bucket(self, u: int) -> int | None:
        """The context bound for this iteration's passes, or None (eager)."""
        exact = [self.d.length + u + j for j in range(self.k)] + [self.t.length + 1 + self.k]
        lo, hi = min(exact), max(exact)
        cap = min(c.pool.max_blocks * c.block_size for c in (self.t, self.d))
        if hi > cap:
            return None
        if hi <= ONE_UNIT_CTX:
            return min(ONE_UNIT_CTX, cap)
        if lo > ONE_UNIT_CTX:
            return min(-(-hi // CTX_STEP) * CTX_STEP, cap)
        return None

    def fits(self, u: int) -> bool:
        """Both caches can take the iteration's tokens (else the eager path
        runs and raises where the reference raises)."""
        for c, n in ((self.d, u + self.k - 1), (self.t, self.k + 1)):
            mgr = c.pool.manager
            need = mgr.blocks_needed(c.length + n) - len(c.blocks)
            if need > mgr.num_free or mgr.blocks_needed(c.length + n) > c.pool.max_blocks:
                return False
        if self.d.pool is self.t.pool:
            mgr = self.d.pool.manager
            need = (mgr.blocks_needed(self.d.length + u + self.k - 1) - len(self.d.blocks)
                    + mgr.blocks_needed(self.t.length + self.k + 1) - len(self.t.blocks))
            return need <= mgr.num_free
        return True

    def _pick(self, j: int, hid_row: torch.Tensor, ov: torch.Tensor) -> None:
        a = kernels.lmhead_argmax(hid_row, lm_head_weight(self.draft))
        self.drafts[j:j + 1].copy_(torch.where(ov[j:j + 1] >= 0, ov[j:j + 1], a))

    def _iteration(self, u: int, ctx: int) -> None:
        k = self.k
        dkv, tkv = self.d.pool.device_kv(), self.t.pool.device_kv()
        ov = self.inp[3:3 + k].to(torch.int32)
        rows = self.inp[3 + k:5 + k].to(torch.int32)
        trow, drow = rows[0:1], rows[1:2]
        hid = forward_hidden(self.draft, self.inp[:u].view(1, u), dkv, drow, ctx)
        kernels.commit(dkv.lens, 1, u, seq_rows=drow)
        self._pick(0, hid[0, u - 1:u], ov)
        for j in range(1, k):
            ids = self.drafts[j - 1:j].view(1, 1).to(torch.long)
            hid = forward_hidden(self.draft, ids, dkv, drow, ctx)
            kernels.commit(dkv.lens, 1, 1, seq_rows=drow)
            self._pick(j, hid[0, -1:], ov)
        ids = torch.cat([self.inp[2:3], self.drafts.to(torch.long)]).view(1, k + 1)
        hid = forward_hidden(self.target, ids, tkv, trow, ctx)
        kernels.commit(tkv.lens, 1, k + 1, seq_rows=trow)
        preds = kernels.lmhead_argmax(hid[0], lm_head_weight(self.target))
        n_acc, emitted, keep = kernels.accept(self.drafts.view(1, k), preds.view(1, k + 1),
                                              lens=tkv.lens, seq_rows=trow)
        kernels.rollback(tkv.tables, tkv.lens, keep, self.t.block_size, seq_rows=trow)
        kernels.rollback(dkv.tables, dkv.lens, keep, self.d.block_size, seq_rows=drow)
        self.out[:1].copy_(n_acc)
        self.out[1:].copy_(emitted[0])

    def run(self, u: int, ctx: int, feed: list[int], last: int, overrides: list[int]):
        """Reserve, run the iteration (a replay, or on a shape's first use the
        same launches eagerly, then its capture), read back; returns (n_acc,
        emitted) with the device caches at the accepted length (the host
        commits follow)."""
        k = self.k
        self.d.reserve(u + k - 1)
        self.t.reserve(k + 1)
        vals = self.inp_host.numpy()
        vals[:u] = feed
        vals[u:2] = 0
        vals[2] = last
        vals[3:3 + k] = overrides
        vals[3 + k] = self.t.row
        vals[4 + k] = self.d.row
        self.inp.copy_(self.inp_host, non_blocking=True)
        g = self.graphs.get((u, ctx))
        if g is not None:
            g.replay()
        else:
            # the iteration itself, then the capture (which runs nothing), on
            # this object's stream: the library keys its workspaces by stream
            cur = torch.cuda.current_stream()
            s = self.stream
            s.wait_stream(cur)
            with torch.cuda.stream(s):
                self._iteration(u, ctx)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                self._iteration(u, ctx)
            cur.wait_stream(s)
            self.graphs[(u, ctx)] = g
        back = self.out.cpu().tolist()
        return back[0], back[1:2 + back[0]]


_GRAPHS: dict[tuple, _IterationGraphs] = {}


def _addresses(model) -> int:
    """A digest of the device addresses of every tensor a forward pass of the
    model reads (parameters, buffers, tensor attributes such as the fused and
    blocked weight copies)."""
    ptrs = []
    for m in model.modules():
        for t in (*m._parameters.values(), *m._buffers.values(), *vars(m).values()):
            if isinstance(t, torch.Tensor):
                ptrs.append(t.data_ptr())
    return hash(tuple(ptrs))


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

    graphs = (_IterationGraphs.for_call(target_model, draft_model, target_cache, draft_cache, k)
              if _IterationGraphs.usable(target_model, draft_model, target_cache, draft_cache,
                                         propose) else None)

    try:
        _sync(device)
        t0 = time.perf_counter()
        while len(res.new_token_ids) < max_new_tokens:
            u = len(tokens) - draft_cache.length
            ctx = graphs.bucket(u) if graphs is not None and u in (1, 2) else None
            if (ctx is not None and len(tokens) - target_cache.length == 1 and graphs.fits(u)):
                # --- steady state: steps 1-4 below as one replayed graph ---
                over = [predraw(len(tokens) + j) if predraw is not None else -1 for j in range(k)]
                n_acc, emitted = graphs.run(u, ctx, tokens[draft_cache.length:], tokens[-1], over)
                res.draft_forwards += k
                res.target_forwards += 1
                draft_cache.sync_committed(u + k - 1)
                target_cache.sync_committed(k + 1)
                res.iterations += 1
                res.tokens_drafted += k
                res.tokens_accepted += n_acc
                res.accepted_per_iter.append(n_acc)
                tokens.extend(emitted)
                res.new_token_ids.extend(emitted)
                keep = len(tokens) - 1
                target_cache.truncate(min(target_cache.length, keep), device_done=True)
                draft_cache.truncate(min(draft_cache.length, keep), device_done=True)
                if any(t in eos_ids for t in emitted):
                    first = next(i for i, t in enumerate(emitted) if t in eos_ids)
                    trim = len(emitted) - (first + 1)
                    if trim:
                        res.new_token_ids = res.new_token_ids[:-trim]
                    res.stopped_on_eos = True
                    break
                continue

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
    finally:
        if graphs is not None:
            graphs.unbind()  # the graph cache keeps no model, pool or cache alive

    _sync(device)
    res.elapsed_s = time.perf_counter() - t0
    if len(res.new_token_ids) > max_new_tokens:
        res.new_token_ids = res.new_token_ids[:max_new_tokens]
        res.stopped_on_eos = res.new_token_ids[-1] in eos_ids
    return res
