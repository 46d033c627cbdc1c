"""Batched greedy speculative decoding with the whole iteration on the device.

The reference decodes speculatively one request at a time
(kvengine/speculative.py:111-215, asserting batch 1 at line 127) and batches
only plain decode (kvengine/engine.py, batch.py). This engine runs the same
per-request algorithm for up to `slots` requests at once:

per iteration, for every active request (slot i uses table row i of both pools)
  1. draft feed of the 1-2 tokens the draft cache has not seen, then k-1 feeds
     of its own proposals (argmax of the last row; optionally replaced by an
     oracle-acceptance proposal);
  2. one target pass over [last token, d_1..d_k];
  3. accept: longest agreeing prefix n, emitted = d_1..d_n + target[n];
  4. both caches roll back to len(tokens)-1 (target keep = len - k + n).

Steady state is exactly the reference's: the target holds len(tokens)-1
tokens, so every verify has q_len = k+1. Prefill feeds prompt[:-1] to both
caches (no LM head needed), so the first iteration is already steady state
(the reference merges prefill into the first verify; tokens are the same,
block tables differ on the first iteration only).

Block allocation order (bit-exact against the lockstep replay in the oracle):
before an iteration's device work the host performs, for slots in ascending
order, the draft reserve of feed 1, then for j = 2..k the draft reserve of
feed j for every slot, then the target reserve of the verify for every slot;
after it, per slot in ascending order, target truncate then draft truncate
(same order as the reference: speculative.py:196-197). No block is freed
between those reserves, so doing them up front allocates exactly what
interleaving them with the forwards would.

Device work of one iteration (k draft forwards, the verify forward, LM-head
argmax, accept, rollback) reads only static buffers, so it is captured as a HIP
graph and replayed; the host uploads one packed int32 vector (the slots' table
rows and inputs) and reads back n_acc and the emitted tokens. Slots are addressed
through a row list, so an iteration may also run narrower than `slots`
(`narrow_batches`: one graph per power-of-two width, padded with empty slots,
which every kernel skips).
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch

from . import kernels
from .forward import (SPLITK_MAX_ROWS, _fusable, forward_hidden, forward_packed,
                      forward_packed_wide, invariant_gemm_rows, blocked_forward)
from .model import lm_head_blocked
from .paged import PagedKVCache, PagedSequenceCache

BIG = 1 << 30
# Summation order of the target's verify attention (kve_paged_verify_attn
# unit_blocks, key_waves): fixed, so that a position's result does not depend
# on the batch, the verify window or a recompute after preemption.
TARGET_ATTN = (8, 2)
# Engines whose histories may pass LONG_CTX_AT tokens use 16-block units (the
# order stays fixed for the engine's lifetime): 8-block units give short
# histories more workgroups, 16-block ones give long histories fewer states.
TARGET_ATTN_LONG = (16, 2)
LONG_CTX_AT = 4096


@dataclass
class SpecRequest:
    request_id: object
    prompt: list[int]
    max_new_tokens: int
    propose: object = None            # OracleAcceptance-like: predraw(pos) -> token or -1
    eos_ids: frozenset = frozenset()
    # results
    new_token_ids: list[int] = field(default_factory=list)
    accepted_per_iter: list[int] = field(default_factory=list)
    iterations: int = 0
    finished: bool = False
    stopped_on_eos: bool = False
    preemptions: int = 0
    # "eos" | "length" | "aborted_prompt_too_long" | "aborted_cache_exhausted" |
    # "aborted_no_progress" (the reference Engine's reasons, engine.py:157-161,
    # 262-267, 297-306, 394-402)
    finish_reason: str | None = None

    @property
    def aborted(self) -> bool:
        return bool(self.finish_reason) and self.finish_reason.startswith("aborted")

    @property
    def tokens(self) -> list[int]:
        return self.prompt + self.new_token_ids

    # The per-iteration host path reads a few positions and the length; these
    # do not build the prompt + output list.
    @property
    def n_tokens(self) -> int:
        return len(self.prompt) + len(self.new_token_ids)

    def token(self, i: int) -> int:
        n = len(self.prompt)
        if i < 0:
            i += n + len(self.new_token_ids)
        return self.prompt[i] if i < n else self.new_token_ids[i - n]


@dataclass
class EngineStats:
    iterations: int = 0
    prefill_tokens: int = 0
    output_tokens: int = 0
    drafted: int = 0
    accepted: int = 0
    preemptions: int = 0
    recomputed_tokens: int = 0     # tokens prefilled again when preempted requests resume
    aborted: int = 0
    prefix_reused_tokens: int = 0  # prompt tokens adopted from published blocks (both pools)
    # most blocks held at once during an iteration (after its reserves)
    peak_target_blocks: int = 0
    peak_draft_blocks: int = 0
    elapsed_s: float = 0.0
    prefill_s: float = 0.0

    @property
    def tokens_per_s(self) -> float:
        return self.output_tokens / self.elapsed_s if self.elapsed_s else 0.0

    @property
    def acceptance_rate(self) -> float:
        return self.accepted / self.drafted if self.drafted else 0.0


class _Slot:
    def __init__(self, req: SpecRequest, t_seq: PagedSequenceCache, d_seq: PagedSequenceCache):
        self.req = req
        self.t = t_seq
        self.d = d_seq


def _packed_groups(lens: list[int], max_real: int, max_pad: int) -> list[tuple[int, int]]:
    """Consecutive [a, b) groups of lens (sorted longest first), each within
    max_real real rows and max_pad padded rows ((b - a) * lens[a]); a single
    item may exceed them."""
    out, a, real = [], 0, 0
    for i, n in enumerate(lens):
        if i > a and (real + n > max_real or (i + 1 - a) * lens[a] > max_pad):
            out.append((a, i))
            a, real = i, 0
        real += n
    if lens:
        out.append((a, len(lens)))
    return out


def _partition_by_cost(lens: list[int], fixed: int, max_rows: int) -> list[tuple[int, int]]:
    """Cut lens (sorted longest first) into consecutive [a, b) groups that
    minimise sum(fixed + (b - a) * lens[a]) with (b - a) * lens[a] <= max_rows
    (a single item may exceed it); exact, by dynamic programming."""
    n = len(lens)
    best = [0] + [None] * n
    cut = [0] * (n + 1)
    for i in range(1, n + 1):
        for j in range(i - 1, -1, -1):
            rows = (i - j) * lens[j]
            if rows > max_rows and i - j > 1:
                break
            c = best[j] + fixed + rows
            if best[i] is None or c < best[i]:
                best[i], cut[i] = c, j
    out, i = [], n
    while i > 0:
        out.append((cut[i], i))
        i = cut[i]
    return out[::-1]


def _bind_row(seq: PagedSequenceCache, row: int) -> None:
    """Pin a sequence to a given table row (engine slots own rows 0..S-1)."""
    seq._row = row
    seq._row_dev = torch.tensor([row], dtype=torch.int32, device=seq.pool.device)


class _Batch:
    """Static device buffers of one batch width (read by a captured iteration)
    and the graph captured for it. Host upload, one packed int32 vector:
    [rows(n) | draft feed-1 tokens(2n) | feed-1 lengths(n) | live(n) |
    last token(n) | oracle proposals(n*k)]."""

    def __init__(self, n: int, k: int, dev):
        self.n = n
        self.rows = torch.zeros(n, dtype=torch.int32, device=dev)
        self.in_draft = torch.zeros(n, 2, dtype=torch.long, device=dev)
        self.q1 = torch.zeros(n, dtype=torch.int32, device=dev)
        self.act = torch.zeros(n, dtype=torch.int32, device=dev)
        self.qv = torch.zeros(n, dtype=torch.int32, device=dev)
        self.last = torch.zeros(n, dtype=torch.long, device=dev)
        self.override = torch.full((n, k), -1, dtype=torch.int32, device=dev)
        self.drafts = torch.zeros(n, k, dtype=torch.int32, device=dev)
        self.out = torch.zeros(n, k + 2, dtype=torch.int32, device=dev)
        self.ar = torch.arange(n, device=dev)
        n_pack = 6 * n + n * k
        self.pack_host = torch.zeros(n_pack, dtype=torch.int32, pin_memory=True)
        self.pack_dev = torch.zeros(n_pack, dtype=torch.int32, device=dev)
        self.out_host = torch.zeros(n, k + 2, dtype=torch.int32, pin_memory=True)
        self.graphs: dict = {}  # context bound -> captured iteration


class _PrefillGraph:
    """One captured single-sequence prefill forward of a padded token count:
    static ids (padded with zeros), table row and real token count."""

    def __init__(self, T: int, dev):
        self.T = T
        self.ids = torch.zeros(T, dtype=torch.long, device=dev)
        self.meta = torch.zeros(2, dtype=torch.int32, device=dev)  # table row, real tokens
        self.dst = torch.arange(T, device=dev)
        self.ids_host = torch.zeros(T, dtype=torch.long, pin_memory=True)
        self.meta_host = torch.zeros(2, dtype=torch.int32, pin_memory=True)
        self.graph = None
        self.done = None  # event after the copies out of the pinned buffers


class SpecEngine:
    """Speculative decoding for a batch of requests on fixed device slots."""

    def __init__(self, target, draft, k: int, slots: int, t_blocks: int, d_blocks: int,
                 block_size: int = 16, max_ctx: int = 2048, use_graph: bool = True,
                 target_attn: tuple[int, int] | None = None, trace: list | None = None,
                 prefix_sharing: bool = False, narrow_batches: bool | None = None,
                 events: list | None = None):
        assert k >= 1
        self.target, self.draft = target, draft
        # Admission adopts the published full blocks of a prompt's prefix
        # (refcounted, content-addressed: kvengine/paged.py:209-279) and
        # publishes its own after the prefill, so requests sharing a prompt
        # prefix read the same physical blocks.
        self.prefix_sharing = prefix_sharing
        self.k, self.S = k, slots
        self.max_ctx = max_ctx
        # The target's verify attention sums every row's keys in one fixed order
        # (units of blocks, key waves: TARGET_ATTN, or TARGET_ATTN_LONG when
        # max_ctx passes LONG_CTX_AT), so a position's result is the same
        # whatever else shares its pass and whenever it is computed; the
        # draft's launches choose their own (its numbers only steer proposals).
        if target_attn is None:
            target_attn = TARGET_ATTN_LONG if max_ctx > LONG_CTX_AT else TARGET_ATTN
        self.target_attn = tuple(target_attn)
        self.draft_attn = (0, 0)
        p = next(target.parameters())
        self.device = p.device
        mb = -(-max_ctx // block_size)
        self.t_pool = PagedKVCache.for_model(target, t_blocks, block_size, max_seqs=slots)
        self.d_pool = PagedKVCache.for_model(draft, d_blocks, block_size, max_seqs=slots)
        for pool in (self.t_pool, self.d_pool):
            pool._free_rows = []  # rows are owned by slots
            pool.max_blocks = min(pool.max_blocks, max(mb, 1))
            pool.tables = pool.tables[:, : pool.max_blocks].contiguous()
        # The kernels' context bound: a sequence never holds more tokens than a
        # table row (or a pool smaller than one) can address. max_ctx itself
        # stays the admission bound, so a pool smaller than a row lets a request
        # run until it exhausts the pool, as the reference does.
        self.kernel_ctx = min(max_ctx, self.t_pool.max_blocks * block_size,
                              self.d_pool.max_blocks * block_size)
        self.slots: list[_Slot | None] = [None] * slots
        dev = self.device
        S = slots
        # One set of static buffers (and one captured graph) per batch width.
        # With narrow_batches an iteration runs at the smallest power-of-two
        # width that holds every occupied slot, so the tail of a workload with
        # few live requests does not pay for the full batch. Outputs depend on
        # the target alone, so narrow batches need the target's passes to be
        # width-invariant (bf16: the wide split-K layer at every width, below);
        # the draft takes the fastest path for each width (its proposals may
        # then differ at a draft near tie between widths, which moves
        # acceptance, never the output). None (default) turns narrow batches on
        # exactly when the target is invariant; forced on elsewhere, outputs may
        # differ at near-ties from a full-width run.
        self.use_graph = use_graph
        # the target takes the wide layer at every width and in its prefill:
        # a token's K/V and logits then do not depend on the pass that made them
        t_ok, t_rows = invariant_gemm_rows(target, S * (k + 1), wide=True)
        if narrow_batches is None:
            narrow_batches = t_ok
        if narrow_batches:
            widths = sorted({min(S, 1 << j) for j in range(max(S - 1, 0).bit_length() + 1)})
        else:
            widths = [S]
        self.narrow_batches = narrow_batches
        self.t_gemm_rows = t_rows if narrow_batches and t_ok else None
        self.d_gemm_rows = None
        lm_head_blocked(target)  # made here, outside any graph capture
        self.batches = {n: _Batch(n, k, dev) for n in widths}
        self._pgraphs: dict = {}
        self._side = torch.cuda.Stream(device=dev) if dev.type == "cuda" else None
        # Prefill graphs are captured on a stream of their model's own: the
        # library caches workspaces (attention plans and unit states) per
        # stream, and captures on torch's shared capture stream would record
        # the same buffers for the draft's and the target's graphs, which
        # replay concurrently (the draft's on the side stream).
        self._cap_streams: dict = {}
        self.stats = EngineStats()
        self.queue: list[SpecRequest] = []
        self.done: list[SpecRequest] = []
        self.admit_order: list[int] = []
        # trace: per iteration [(slot, request id, target blocks, draft blocks)];
        # events: ("admit", id, slot), ("preempt", id), ("finish", id, reason)
        self.trace = trace
        self.events = events

    # ------------------------------------------------------------ device step

    def _unpack(self, b: "_Batch") -> None:
        n, k = b.n, self.k
        p = b.pack_dev
        b.rows.copy_(p[:n])
        b.in_draft.copy_(p[n:3 * n].view(n, 2))
        b.q1.copy_(p[3 * n:4 * n])
        b.act.copy_(p[4 * n:5 * n])
        b.qv.copy_(b.act * (k + 1))
        b.last.copy_(p[5 * n:6 * n])
        b.override.copy_(p[6 * n:].view(n, k))

    def _pick(self, b: "_Batch", j: int, hid_rows: torch.Tensor) -> None:
        a = kernels.lmhead_argmax(hid_rows, self.draft.lm_head.weight)
        o = b.override[:, j]
        b.drafts[:, j] = torch.where(o >= 0, o, a)

    # Context bound of the short-context graphs: one attention unit record holds
    # 56 blocks of 16 tokens, so with every live sequence under this bound no
    # draft attention item is split and no merge kernel runs (0.5B forward at 32
    # rows: 1100 -> 1042 us).
    SHORT_CTX = 896

    def _device_iteration(self, b: "_Batch", ctx: int) -> None:
        """Everything between the input upload and the result read-back, for
        the slots (table rows) listed in b.rows; ctx bounds every pass's
        lengths + tokens."""
        n, k = b.n, self.k
        self._unpack(b)
        dkv, tkv = self.d_pool.device_kv(), self.t_pool.device_kv()
        hid = forward_hidden(self.draft, b.in_draft, dkv, b.rows, ctx,
                             q_lens=b.q1, attn_order=self.draft_attn,
                             gemm_rows=self.d_gemm_rows)
        kernels.commit(dkv.lens, n, 2, seq_rows=b.rows, q_lens=b.q1)
        idx = (b.q1.to(torch.long) - 1).clamp(min=0)
        self._pick(b, 0, hid[b.ar, idx])
        for j in range(1, k):
            ids = b.drafts[:, j - 1:j].to(torch.long)
            hid = forward_hidden(self.draft, ids, dkv, b.rows, ctx, q_lens=b.act,
                                 attn_order=self.draft_attn, gemm_rows=self.d_gemm_rows)
            kernels.commit(dkv.lens, n, 1, seq_rows=b.rows, q_lens=b.act)
            self._pick(b, j, hid[:, 0])
        ids_v = torch.cat([b.last[:, None], b.drafts.to(torch.long)], dim=1)
        m = n * (k + 1)
        head_blk = lm_head_blocked(self.target)
        blk = head_blk is not None and blocked_forward(self.target, m, self.t_gemm_rows)
        hid = forward_hidden(self.target, ids_v, tkv, b.rows, ctx, q_lens=b.qv,
                             attn_order=self.target_attn, gemm_rows=self.t_gemm_rows,
                             blocked_out=blk)
        kernels.commit(tkv.lens, n, k + 1, seq_rows=b.rows, q_lens=b.qv)
        if blk:
            preds = kernels.lmhead_argmax(hid, head_blk, blocked=True, rows=m)
        else:
            preds = kernels.lmhead_argmax(hid.view(m, -1), self.target.lm_head.weight)
        n_acc, emitted, keep = kernels.accept(b.drafts, preds.view(n, k + 1), lens=tkv.lens,
                                              seq_rows=b.rows)
        keep = torch.where(b.act > 0, keep, torch.full_like(keep, BIG))
        kernels.rollback(tkv.tables, tkv.lens, keep, self.t_pool.block_size, seq_rows=b.rows)
        kernels.rollback(dkv.tables, dkv.lens, keep, self.d_pool.block_size, seq_rows=b.rows)
        b.out[:, 0] = n_acc
        b.out[:, 1:] = emitted

    def _run_device(self, b: "_Batch", ctx: int) -> None:
        b.pack_dev.copy_(b.pack_host, non_blocking=True)
        if not self.use_graph:
            self._device_iteration(b, ctx)
            return
        g = b.graphs.get(ctx)
        if g is None:
            # warm up (allocates workspaces), then capture on a side stream
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                self._snapshot_state()
                self._device_iteration(b, ctx)
                self._restore_state()
            torch.cuda.current_stream().wait_stream(s)
            g = torch.cuda.CUDAGraph()
            self._snapshot_state()
            with torch.cuda.graph(g):
                self._device_iteration(b, ctx)
            self._restore_state()
            b.graphs[ctx] = g
        g.replay()

    def _snapshot_state(self) -> None:
        self._saved = [t.clone() for t in (self.t_pool.tables, self.t_pool.lens,
                                           self.d_pool.tables, self.d_pool.lens)]

    def _restore_state(self) -> None:
        for dst, src in zip((self.t_pool.tables, self.t_pool.lens, self.d_pool.tables,
                             self.d_pool.lens), self._saved):
            dst.copy_(src)
        self._saved = None

    # ------------------------------------------------------------ host side

    def add_request(self, req: SpecRequest) -> None:
        self.queue.append(req)

    def _admit(self) -> None:
        """FIFO admission into free slots (ascending), prefilling tokens[:-1]
        into both caches; stops at the first request that does not fit with a
        watermark of one iteration's growth (kvengine/engine.py:284-324).

        Blocks are reserved request by request as each is admitted (so the
        admission test and the allocation order are those of one-at-a-time
        prefill); the prefill forwards of everything admitted in one call then
        run batched, requests of similar length together (`_prefill_batch`).
        With prefix sharing a request may adopt blocks a predecessor in the
        same call publishes: blocks are published as soon as they are reserved,
        and the batch of pending prefills is run before any request that adopts
        one of its blocks joins a batch (the forward that reads a block comes
        after the one that writes it, in stream order)."""
        pending = []
        pend_blocks: set[tuple[int, int]] = set()  # (pool id, block) published by `pending`

        def flush():
            if pending:
                # the two models' prefills write separate pools: the draft's runs
                # on a side stream beside the target's
                cur = torch.cuda.current_stream()
                side = self._side if self._side is not None else cur
                side.wait_stream(cur)
                self._prefill_batch(self.target, [(t, tk) for t, _, tk, _ in pending],
                                    reserved=True)
                with torch.cuda.stream(side):
                    self._prefill_batch(self.draft, [(d, dk) for _, d, _, dk in pending],
                                        reserved=True, fixed_rows=self.PREFILL_FIXED_ROWS_DRAFT)
                cur.wait_stream(side)
                pending.clear()
                pend_blocks.clear()

        i = 0
        while i < self.S and self.queue:
            if self.slots[i] is not None:
                i += 1
                continue
            req = self.queue[0]
            toks = req.tokens
            n = len(toks) - 1
            tm, dm = self.t_pool.manager, self.d_pool.manager
            first = n + self.k + 1  # tokens held during the first iteration
            if (len(toks) + (req.max_new_tokens - len(req.new_token_ids)) + self.k + 2 > self.max_ctx
                    or tm.blocks_needed(first) > tm.num_blocks
                    or dm.blocks_needed(first) > dm.num_blocks):
                # Would not fit a device table row (max_ctx) or even an empty
                # pool, so waiting can never help: retire it and go on with the
                # queue (kvengine/engine.py:297-306).
                self.queue.pop(0)
                self._finish(req, "aborted_prompt_too_long")
                continue
            if tm.blocks_needed(first) > tm.num_free or dm.blocks_needed(first) > dm.num_free:
                break
            if req.new_token_ids:
                self.stats.recomputed_tokens += n
            t_seq = self.t_pool.new_sequence(req.request_id)
            d_seq = self.d_pool.new_sequence(req.request_id)
            _bind_row(t_seq, i)
            _bind_row(d_seq, i)
            if self.prefix_sharing:
                nt = t_seq.adopt_prefix(toks)
                nd = d_seq.adopt_prefix(toks)
                bs_t, bs_d = self.t_pool.block_size, self.d_pool.block_size
                adopted = {(0, b) for b in t_seq.blocks[: nt // bs_t]} | \
                    {(1, b) for b in d_seq.blocks[: nd // bs_d]}
                if adopted & pend_blocks:
                    flush()
                self.stats.prefix_reused_tokens += nt + nd
                if n > nt:
                    t_seq.reserve(n - nt)
                if n > nd:
                    d_seq.reserve(n - nd)
                t_seq.register_prefix_blocks(toks, ahead=n - nt)
                d_seq.register_prefix_blocks(toks, ahead=n - nd)
                # the blocks this prefill writes (adopted ones are already written)
                pend_blocks.update((0, b) for b in t_seq.blocks[nt // bs_t:])
                pend_blocks.update((1, b) for b in d_seq.blocks[nd // bs_d:])
                pending.append((t_seq, d_seq, toks[nt:-1], toks[nd:-1]))
            else:
                if n:
                    t_seq.reserve(n)
                    d_seq.reserve(n)
                pending.append((t_seq, d_seq, toks[:-1], toks[:-1]))
            self.queue.pop(0)
            self.slots[i] = _Slot(req, t_seq, d_seq)
            self.admit_order.append(i)
            self._event("admit", req.request_id, i)
            i += 1
        flush()

    # Prefill batches: a padded [count, longest] forward costs about
    # fixed + rows, in units of one row, where `fixed` is what a forward costs
    # whatever its row count (weight streaming and per-layer launches at small
    # row counts). Measured on MI355X for 32 prompts of 43-349 tokens: the 3B
    # prefill took 58.6 ms in five batches of at most 1.25x padding, 54.8 ms in
    # the three batches of fixed = 800 rows and 51.6 ms in the two of
    # fixed >= 1200 (7230 padded rows for 4767 tokens); the 0.5B (about
    # 3.8 ms + 1 us per row) is best with few batches as well.
    # Batches are capped at PREFILL_ROWS rows (activation memory).
    PREFILL_FIXED_ROWS = 1500
    PREFILL_FIXED_ROWS_DRAFT = 4000
    PREFILL_ROWS = 8192
    # Packed prefill (fused models): projections run on the real tokens only,
    # so batches are bounded by PREFILL_ROWS real tokens and PREFILL_PAD_ROWS
    # padded [B, T] rows (the RoPE/KV-write and attention layout).
    PREFILL_PAD_ROWS = 32768

    def _attn_of(self, model) -> tuple[int, int]:
        return self.target_attn if model is self.target else self.draft_attn

    # Single-sequence prefills (the recompute of a preempted request, a lone
    # admission) replay a graph captured per (model, padded token count): their
    # eager launches cost as much host time as the GPU takes. Padding rows past
    # the real token count are masked (no K/V write, no attention row); the
    # target's layer is row-independent, so the real rows keep their bits.
    PREFILL_GRAPH_MAX = 1024

    @staticmethod
    def _prefill_bucket(T: int) -> int:
        step = 32 if T <= 256 else 64 if T <= 512 else 128
        return -(-T // step) * step

    def _prefill_graphed(self, model, seq: PagedSequenceCache, toks: list[int], wide: bool) -> bool:
        T = len(toks)
        Tb = self._prefill_bucket(T)
        if (not self.use_graph or Tb > self.PREFILL_GRAPH_MAX
                or seq.length + Tb > self.kernel_ctx):
            return False
        key = (id(model), Tb)
        ent = self._pgraphs.get(key)
        if ent is None:
            ent = self._pgraphs[key] = _PrefillGraph(Tb, self.device)
        if ent.done is not None:
            ent.done.synchronize()  # the last copies out of these pinned buffers ran
        ent.ids_host.zero_()
        ent.ids_host[:T] = torch.tensor(toks, dtype=torch.long)
        ent.meta_host[0] = seq.row
        ent.meta_host[1] = T
        ent.ids.copy_(ent.ids_host, non_blocking=True)
        ent.meta.copy_(ent.meta_host, non_blocking=True)
        kv = seq.device_kv()

        def run():
            if wide:
                forward_packed_wide(model, ent.ids, ent.dst, 1, Tb, kv, ent.meta[0:1],
                                    self.kernel_ctx, ent.meta[1:2], attn_order=self._attn_of(model))
            else:
                forward_hidden(model, ent.ids.view(1, Tb), kv, ent.meta[0:1], self.kernel_ctx,
                               q_lens=ent.meta[1:2], attn_order=self._attn_of(model))

        ent.done = torch.cuda.Event()
        ent.done.record()
        if ent.graph is None:
            run()  # the prefill itself; the capture below records without running
            cap = self._cap_streams.get(id(model))
            if cap is None:
                cap = self._cap_streams[id(model)] = torch.cuda.Stream(device=self.device)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cap):
                run()
            ent.graph = g
        else:
            ent.graph.replay()
        return True

    def _prefill_batch(self, model, items, reserved: bool = False,
                       fixed_rows: int | None = None) -> None:
        """Feed each (sequence, tokens) pair's tokens at the sequence's current
        length, sequences sorted by token count. Fused models: consecutive
        groups within the packed caps, each one `forward_packed` (projections
        on the real tokens only) unless it is one sequence or at most the
        split-K layer's rows. Otherwise: groups that minimise the summed cost
        fixed_rows + count x longest of one padded [B, T] forward (ragged
        through q_lens) per group."""
        items = [(seq, toks) for seq, toks in items if toks]
        if not items:
            return
        if not reserved:
            for seq, toks in items:
                seq.reserve(len(toks))
        items.sort(key=lambda it: -len(it[1]))
        lens = [len(t) for _, t in items]
        packed = _fusable(model)
        # The target's prefill (and recompute after preemption) takes the wide
        # layer's arithmetic whenever its verify passes do, so a token's K/V do
        # not depend on whether a prefill or a verify pass produced them.
        wide = packed and model is self.target and self.t_gemm_rows is not None
        if packed:
            groups = _packed_groups(lens, self.PREFILL_ROWS, self.PREFILL_PAD_ROWS)
        else:
            groups = _partition_by_cost(lens, self.PREFILL_FIXED_ROWS if fixed_rows is None
                                        else fixed_rows, self.PREFILL_ROWS)
        groups = [items[a:b] for a, b in groups]
        for g in groups:
            B, T = len(g), len(g[0][1])
            n_real = sum(len(t) for _, t in g)
            if B == 1 and packed and (wide or model is not self.target):
                seq, toks = g[0]
                if self._prefill_graphed(model, seq, toks, wide):
                    seq.commit(len(toks))
                    self.stats.prefill_tokens += len(toks)
                    continue
            if wide or (packed and B > 1 and n_real > SPLITK_MAX_ROWS):
                flat, dst = [], []
                for j, (seq, toks) in enumerate(g):
                    flat.extend(toks)
                    dst.extend(range(j * T, j * T + len(toks)))
                meta = torch.tensor([[seq.row for seq, _ in g], [len(t) for _, t in g]],
                                    dtype=torch.int32)
                ids = torch.tensor(flat, dtype=torch.long).to(self.device)
                dsti = torch.tensor(dst, dtype=torch.long).to(self.device)
                meta = meta.to(self.device)
                max_ctx = max(seq.length for seq, _ in g) + T
                fwd = forward_packed_wide if wide else forward_packed
                fwd(model, ids, dsti, B, T, g[0][0].device_kv(), meta[0], max_ctx, meta[1],
                    attn_order=self._attn_of(model))
                for seq, toks in g:
                    seq.commit(len(toks))
                    self.stats.prefill_tokens += len(toks)
                continue
            ids = torch.zeros(B, T, dtype=torch.long)
            meta = torch.empty(2, B, dtype=torch.int32)
            for j, (seq, toks) in enumerate(g):
                ids[j, :len(toks)] = torch.tensor(toks, dtype=torch.long)
                meta[0, j] = seq.row
                meta[1, j] = len(toks)
            ids, meta = ids.to(self.device), meta.to(self.device)
            max_ctx = max(seq.length for seq, _ in g) + T
            forward_hidden(model, ids, g[0][0].device_kv(), meta[0], max_ctx,
                           q_lens=None if B == 1 else meta[1], attn_order=self._attn_of(model))
            for seq, toks in g:
                seq.commit(len(toks))
                self.stats.prefill_tokens += len(toks)

    def _demand(self) -> tuple[int, int]:
        """Blocks the next iteration will allocate in the target and draft pools."""
        k = self.k
        need_t = need_d = 0
        for sl in self.slots:
            if sl is None:
                continue
            u = sl.req.n_tokens - sl.d.length
            need_d += max(0, sl.d.pool.manager.blocks_needed(sl.d.length + u + k - 1) - len(sl.d.blocks))
            need_t += max(0, sl.t.pool.manager.blocks_needed(sl.t.length + k + 1) - len(sl.t.blocks))
        return need_t, need_d

    def _make_room(self) -> None:
        """Preempt the most recently admitted request until the iteration fits
        (recompute on readmission, kvengine/engine.py:394-403, 425-440). A lone
        request that still does not fit cannot be served by pools this small:
        it is retired as aborted_cache_exhausted (engine.py:394-402)."""
        while True:
            need_t, need_d = self._demand()
            if need_t <= self.t_pool.manager.num_free and need_d <= self.d_pool.manager.num_free:
                return
            live = [i for i in self.admit_order if self.slots[i] is not None]
            if len(live) <= 1:
                self._retire(live[0], "aborted_cache_exhausted")
                return
            victim = live[-1]
            req = self.slots[victim].req
            req.preemptions += 1
            self.stats.preemptions += 1
            self._release(victim)
            self.queue.insert(0, req)
            self._event("preempt", req.request_id)

    def _reserve_iteration(self) -> list[int]:
        """Host reserves for one iteration in the documented order; returns the
        draft feed-1 length per slot (0 for empty slots)."""
        k = self.k
        u = [0] * self.S
        for i, sl in enumerate(self.slots):
            if sl is None:
                continue
            u[i] = sl.req.n_tokens - sl.d.length
            assert u[i] in (1, 2), (sl.req.request_id, u[i])
            self._grow(sl.d, u[i])
        for _ in range(1, k):
            for sl in self.slots:
                if sl is not None:
                    self._grow(sl.d, 1)
        for sl in self.slots:
            if sl is not None:
                self._grow(sl.t, k + 1)
        return u

    @staticmethod
    def _grow(seq: PagedSequenceCache, n: int) -> None:
        """reserve(n) counted from the length the sequence will have after the
        reserves already made this iteration (pending tokens)."""
        pend = seq._pending_total if getattr(seq, "_pending_total", None) else 0
        need = seq.pool.manager.blocks_needed(seq.length + pend + n) - len(seq.blocks)
        if need > 0:
            new = seq.pool.manager.allocate(need, owner=seq.request_id)
            seq._set_entries(len(seq.blocks), new)
            seq.blocks.extend(new)
        seq._pending_total = pend + n

    def _pack(self, u: list[int], b: "_Batch", rows: list[int]) -> None:
        n, k = b.n, self.k
        vals = b.pack_host.numpy()
        vals[:] = 0
        vals[:n] = rows
        ov = vals[6 * n:].reshape(n, k)
        ov[:] = -1
        for j, i in enumerate(rows):
            sl = self.slots[i]
            if sl is None:
                continue
            req = sl.req
            d_len = sl.d.length
            vals[n + 2 * j] = req.token(d_len)
            vals[n + 2 * j + 1] = req.token(d_len + 1) if u[i] == 2 else 0
            vals[3 * n + j] = u[i]
            vals[4 * n + j] = 1
            vals[5 * n + j] = req.token(-1)
            if req.propose is not None:
                base = req.n_tokens
                for t in range(k):
                    ov[j, t] = req.propose.predraw(base + t)

    def step(self) -> None:
        """One speculative iteration over every occupied slot."""
        k = self.k
        self._make_room()
        live = [i for i, sl in enumerate(self.slots) if sl is not None]
        if not live:
            return
        for i in live:
            self.slots[i].d._pending_total = 0
            self.slots[i].t._pending_total = 0
        u = self._reserve_iteration()
        st = self.stats
        st.peak_target_blocks = max(st.peak_target_blocks, self.t_pool.manager.num_allocated)
        st.peak_draft_blocks = max(st.peak_draft_blocks, self.d_pool.manager.num_allocated)
        b = self.batches[min(n for n in self.batches if n >= len(live))]
        # rows past the live slots are empty slots (no tokens: every kernel skips them)
        rows = live + [i for i, sl in enumerate(self.slots) if sl is None][:b.n - len(live)]
        self._pack(u, b, rows)
        # every pass's lengths + tokens: draft feeds reach d.length + u + k - 1,
        # the verify t.length + k + 1
        need = max(max(self.slots[i].d.length + u[i] + k - 1, self.slots[i].t.length + k + 1)
                   for i in live)
        ctx = self.SHORT_CTX if need <= self.SHORT_CTX < self.kernel_ctx else self.kernel_ctx
        self._run_device(b, ctx)
        b.out_host.copy_(b.out, non_blocking=True)
        torch.cuda.current_stream().synchronize()
        res = b.out_host.tolist()
        st.iterations += 1
        for j, i in enumerate(live):
            sl = self.slots[i]
            n = res[j][0]
            emitted = res[j][1:2 + n]
            req = sl.req
            sl.t.sync_committed(k + 1)
            sl.d.sync_committed(u[i] + k - 1)
            sl.t._pending_total = 0
            sl.d._pending_total = 0
            req.new_token_ids.extend(emitted)
            req.accepted_per_iter.append(n)
            req.iterations += 1
            st.drafted += k
            st.accepted += n
            keep = req.n_tokens - 1
            sl.t.truncate(min(sl.t.length, keep), device_done=True)
            sl.d.truncate(min(sl.d.length, keep), device_done=True)
            if self.prefix_sharing:
                # generated tokens are shareable too (kvengine/engine.py:414-419)
                toks = req.tokens
                sl.t.register_prefix_blocks(toks)
                sl.d.register_prefix_blocks(toks)
            hit_eos = [t for t in emitted if t in req.eos_ids]
            if hit_eos:
                first = next(j for j, t in enumerate(emitted) if t in req.eos_ids)
                trim = len(emitted) - (first + 1)
                if trim:
                    del req.new_token_ids[-trim:]
                req.stopped_on_eos = True
            if req.stopped_on_eos or len(req.new_token_ids) >= req.max_new_tokens:
                if len(req.new_token_ids) > req.max_new_tokens:
                    # the budget trim can cut an EOS that sat past the budget
                    # (kvengine/speculative.py:211-214)
                    del req.new_token_ids[req.max_new_tokens:]
                    req.stopped_on_eos = req.new_token_ids[-1] in req.eos_ids
                self._retire(i, "eos" if req.stopped_on_eos else "length")
        if self.trace is not None:
            self.trace.append([(i, sl.req.request_id, list(sl.t.blocks), list(sl.d.blocks))
                               for i, sl in enumerate(self.slots) if sl is not None])

    def _release(self, i: int) -> None:
        """Free slot i's blocks in both pools and clear its device rows."""
        sl = self.slots[i]
        for seq in (sl.t, sl.d):
            if seq.blocks:
                seq.pool.manager.free(seq.blocks)
                seq.blocks = []
            seq.pool.tables[i].fill_(-1)
            seq.pool.lens[i].fill_(0)
            seq._length = 0
        self.slots[i] = None
        if i in self.admit_order:
            self.admit_order.remove(i)

    def _retire(self, i: int, reason: str) -> None:
        """Release slot i and finish its request with `reason`."""
        req = self.slots[i].req
        self._release(i)
        self._finish(req, reason)

    def _finish(self, req: SpecRequest, reason: str) -> None:
        req.finished = True
        req.finish_reason = reason
        if req.aborted:
            self.stats.aborted += 1
        self.stats.output_tokens += len(req.new_token_ids)
        self.done.append(req)
        self._event("finish", req.request_id, reason)

    def _event(self, *e) -> None:
        if self.events is not None:
            self.events.append(e)

    def reset_stats(self, clear_prefix_cache: bool = False) -> None:
        """Forget finished requests and counters (pools must be empty); with
        clear_prefix_cache also forget every published prefix block, so the next
        run prefills its prompts exactly as a first run would."""
        assert all(sl is None for sl in self.slots) and not self.queue
        self.stats = EngineStats()
        self.done = []
        if clear_prefix_cache:
            for pool in (self.t_pool, self.d_pool):
                assert pool.manager.num_allocated == 0
                pool.manager.reset()

    def run(self, requests: list[SpecRequest]) -> EngineStats:
        """Decode every request to completion; returns throughput statistics."""
        for r in requests:
            self.add_request(r)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        self._admit()
        torch.cuda.synchronize()
        self.stats.prefill_s += time.perf_counter() - t0
        while any(s is not None for s in self.slots) or self.queue:
            if all(s is None for s in self.slots):
                self._admit()
                if all(s is None for s in self.slots):
                    if self.queue:
                        # Nothing running and nothing admissible: no later step
                        # can differ, so abort the head of the queue rather
                        # than spin (kvengine/engine.py:262-267).
                        self._finish(self.queue.pop(0), "aborted_no_progress")
                    continue
            self.step()
            if self.queue:
                self._admit()
        torch.cuda.synchronize()
        self.stats.elapsed_s += time.perf_counter() - t0
        return self.stats
