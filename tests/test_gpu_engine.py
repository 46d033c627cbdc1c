"""Batched speculative engine against the oracle's lockstep replay.

The engine decodes many requests per iteration (one HIP graph replay per
iteration); the oracle runs the reference's per-request loop for the same
requests in the documented lockstep order on the CPU. Tokens, accept traces,
preemptions and both pools' block tables after every iteration must agree.
"""

import random

import pytest
import torch

from kvengine_amd.arch import TINY
from kvengine_amd.decode import greedy_paged
from kvengine_amd.engine import SpecEngine, SpecRequest, _bind_row
from kvengine_amd.model import build_model
from kvengine_amd.paged import PagedKVCache
from kvengine_amd.weights import generate_state_dict
from kvengine_amd.workloads import OracleAcceptance
from oracle.batch import RefLockstepRequest, ref_lockstep_spec
from oracle.model import RefQwen2
from oracle.paged import RefPagedKVCache

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def models():
    sd_t = generate_state_dict(TINY, seed=3, dtype=torch.float32)
    sd_d = generate_state_dict(TINY, seed=4, dtype=torch.float32)
    return {
        "gpu": (build_model(TINY, sd_t, dtype=torch.float32, device=DEV),
                build_model(TINY, sd_d, dtype=torch.float32, device=DEV)),
        "cpu": (RefQwen2(TINY, sd_t), RefQwen2(TINY, sd_d)),
    }


def ref_pool(blocks, bs=4):
    return RefPagedKVCache(TINY.num_layers, TINY.num_kv_heads, TINY.head_dim, blocks, bs,
                           torch.float32)


def workload(n, seed, budgets=(3, 24)):
    rng = random.Random(seed)
    return [([rng.randrange(TINY.vocab) for _ in range(rng.randint(5, 21))], rng.randint(*budgets))
            for _ in range(n)]


def continuation(model, prompt, n):
    pool = PagedKVCache.for_model(model, 64, 4)
    return greedy_paged(model, torch.tensor([prompt], device=DEV), pool, max_new_tokens=n,
                        eos_token_id=None).new_token_ids


@pytest.mark.parametrize("use_graph,narrow", [(True, False), (False, False), (True, True)])
@pytest.mark.parametrize("k,slots,t_blocks,oracle_p", [(3, 4, 80, None), (4, 3, 26, 0.65),
                                                       (2, 5, 200, 0.9)])
def test_engine_matches_lockstep_oracle(gpu_lib, models, use_graph, narrow, k, slots, t_blocks,
                                        oracle_p):
    """narrow: iterations run at the smallest power-of-two width holding the live
    slots (rows given by a slot list, padded with empty slots)."""
    # the 26-block pool cannot hold three long requests at once: preemption must fire
    work = workload(7, seed=k * 10 + slots, budgets=(30, 40) if t_blocks == 26 else (3, 24))
    tgt, drf = models["gpu"]
    conts = [continuation(tgt, p, m) for p, m in work] if oracle_p else [None] * len(work)

    def propose(i):
        if oracle_p is None:
            return None
        p = work[i][0]
        return OracleAcceptance([0] * len(p) + conts[i], oracle_p, seed=100 + i, vocab=TINY.vocab)

    trace_g, events_g = [], []
    eng = SpecEngine(tgt, drf, k=k, slots=slots, t_blocks=t_blocks, d_blocks=t_blocks,
                     block_size=4, max_ctx=64, use_graph=use_graph, trace=trace_g,
                     narrow_batches=narrow, events=events_g)
    reqs = [SpecRequest(i, p, m, propose=propose(i)) for i, (p, m) in enumerate(work)]
    eng.run(reqs)

    ref_t, ref_d = models["cpu"]
    trace_c, events_c = [], []
    rreqs = [RefLockstepRequest(i, p, m, propose=propose(i)) for i, (p, m) in enumerate(work)]
    ref_lockstep_spec(ref_t, ref_d, rreqs, k, slots, ref_pool(t_blocks), ref_pool(t_blocks),
                      trace=trace_c, events=events_c)
    for a, b in zip(reqs, rreqs):
        assert a.new_token_ids == b.new_token_ids, a.request_id
        assert a.accepted_per_iter == b.accepted_per_iter, a.request_id
        assert a.preemptions == b.preemptions
        assert a.finish_reason == b.finish_reason == "length"
    assert trace_g == trace_c, "block tables differ from the lockstep replay"
    assert events_g == events_c, "admission / preemption order differs from the lockstep replay"
    if oracle_p:
        for i, r in enumerate(reqs):
            assert r.new_token_ids == conts[i][: len(r.new_token_ids)]
    eng.t_pool.manager.check_invariants()
    assert eng.t_pool.manager.num_allocated == 0 and eng.d_pool.manager.num_allocated == 0
    if t_blocks == 26:
        assert eng.stats.preemptions > 0, "pool was meant to force preemption"


def test_engine_output_is_target_greedy(gpu_lib, models):
    """Any draft: every request's output equals its own plain greedy run."""
    tgt, drf = models["gpu"]
    work = workload(5, seed=1)
    eng = SpecEngine(tgt, drf, k=4, slots=8, t_blocks=200, d_blocks=200, block_size=16,
                     max_ctx=128)
    reqs = [SpecRequest(i, p, m) for i, (p, m) in enumerate(work)]
    eng.run(reqs)
    for r, (p, m) in zip(reqs, work):
        assert r.new_token_ids == continuation(tgt, p, m)


@pytest.mark.parametrize("slots,t_blocks", [(8, 200), (3, 60)])
def test_engine_prefix_sharing(gpu_lib, models, slots, t_blocks):
    """Requests sharing a prompt prefix adopt its published blocks (refcounted)
    and still decode exactly their own greedy continuation, with and without
    preemption and slot reuse; the adopted blocks are the first request's."""
    tgt, drf = models["gpu"]
    rng = random.Random(7)
    prefix = [rng.randrange(TINY.vocab) for _ in range(37)]  # 9 full blocks of 4 within len-1
    work = [(prefix + [rng.randrange(TINY.vocab) for _ in range(rng.randint(2, 9))],
             rng.randint(10, 30)) for _ in range(6)]
    seen_tables = []
    orig = SpecEngine._admit

    def admit_and_record(self):
        orig(self)
        for sl in self.slots:
            if sl is not None:
                seen_tables.append(list(sl.t.blocks[:9]))

    SpecEngine._admit = admit_and_record
    try:
        eng = SpecEngine(tgt, drf, k=3, slots=slots, t_blocks=t_blocks, d_blocks=t_blocks,
                         block_size=4, max_ctx=96, prefix_sharing=True)
        reqs = [SpecRequest(i, p, m) for i, (p, m) in enumerate(work)]
        st = eng.run(reqs)
    finally:
        SpecEngine._admit = orig
    for r, (p, m) in zip(reqs, work):
        assert r.new_token_ids == continuation(tgt, p, m)
    # every later admission (both pools) reused the 9 shared blocks = 36 tokens
    assert st.prefix_reused_tokens >= 2 * 36 * (len(work) - 1)
    assert all(t == seen_tables[0] for t in seen_tables), "shared prefix blocks differ"
    # pools empty again: every refcount returned to zero
    for pool in (eng.t_pool, eng.d_pool):
        assert pool.manager.num_free == pool.manager.num_blocks  # free counts reclaimable blocks


@pytest.mark.parametrize("prefix_len", [0, 29])
def test_engine_packed_prefill_output_is_target_greedy(gpu_lib, models, prefix_len):
    """Prompts long enough that admission runs the packed prefill (more than the
    split-K layer's 160 rows of real tokens in one batch), with and without a
    shared prefix (then the first request is prefilled alone and the others,
    which adopt its blocks, together): every output equals its own greedy run."""
    tgt, drf = models["gpu"]
    rng = random.Random(21)
    prefix = [rng.randrange(TINY.vocab) for _ in range(prefix_len)]
    work = [(prefix + [rng.randrange(TINY.vocab) for _ in range(rng.randint(25, 60))],
             rng.randint(4, 12)) for _ in range(8)]
    assert sum(len(p) - 1 for p, _ in work[1:]) - 7 * prefix_len > 160
    eng = SpecEngine(tgt, drf, k=3, slots=8, t_blocks=300, d_blocks=300, block_size=4,
                     max_ctx=128, prefix_sharing=prefix_len > 0)
    reqs = [SpecRequest(i, p, m) for i, (p, m) in enumerate(work)]
    eng.run(reqs)
    for r, (p, m) in zip(reqs, work):
        assert r.new_token_ids == continuation(tgt, p, m)
    if prefix_len:
        assert eng.stats.prefix_reused_tokens >= 2 * 7 * (prefix_len // 4) * 4


def run_both(models, work, k, slots, blocks, max_ctx=64, hold=0):
    """Engine and lockstep oracle on the same requests; `hold` target blocks are
    taken from both target pools before the run (held outside the scheduler)."""
    tgt, drf = models["gpu"]
    ref_t, ref_d = models["cpu"]
    ev_g, ev_c = [], []
    eng = SpecEngine(tgt, drf, k=k, slots=slots, t_blocks=blocks, d_blocks=blocks, block_size=4,
                     max_ctx=max_ctx, events=ev_g)
    rt, rd = ref_pool(blocks), ref_pool(blocks)
    if hold:
        eng.t_pool.manager.allocate(hold, owner="elsewhere")
        rt.manager.allocate(hold, owner="elsewhere")
    reqs = [SpecRequest(i, p, m) for i, (p, m) in enumerate(work)]
    eng.run(reqs)
    rreqs = [RefLockstepRequest(i, p, m) for i, (p, m) in enumerate(work)]
    ref_lockstep_spec(ref_t, ref_d, rreqs, k, slots, rt, rd, max_ctx=max_ctx, events=ev_c)
    for a, b in zip(reqs, rreqs):
        assert a.new_token_ids == b.new_token_ids, a.request_id
        assert a.finish_reason == b.finish_reason, (a.request_id, a.finish_reason, b.finish_reason)
    assert ev_g == ev_c
    assert eng.t_pool.manager.num_allocated == hold and eng.d_pool.manager.num_allocated == 0
    return reqs, eng


def test_engine_aborts_prompt_larger_than_pool(gpu_lib, models):
    """aborted_prompt_too_long at once (kvengine/engine.py:297-306); the
    requests behind it are served."""
    rng = random.Random(2)
    work = [([rng.randrange(TINY.vocab) for _ in range(20)], 10),
            ([rng.randrange(TINY.vocab) for _ in range(3)], 4),
            ([rng.randrange(TINY.vocab) for _ in range(30)], 4)]
    reqs, eng = run_both(models, work, k=3, slots=2, blocks=5)
    assert [r.finish_reason for r in reqs] == ["aborted_prompt_too_long", "length",
                                              "aborted_prompt_too_long"]
    assert reqs[0].new_token_ids == [] and eng.stats.aborted == 2
    assert reqs[1].new_token_ids == continuation(models["gpu"][0], work[1][0], 4)


def test_engine_aborts_what_max_ctx_cannot_hold(gpu_lib, models):
    work = [(list(range(10)), 50), ([5, 6, 7], 6)]
    reqs, _ = run_both(models, work, k=3, slots=2, blocks=64, max_ctx=48)
    assert [r.finish_reason for r in reqs] == ["aborted_prompt_too_long", "length"]


def test_engine_aborts_generation_outgrowing_pool(gpu_lib, models):
    """A lone request that cannot grow: aborted_cache_exhausted with the tokens
    produced so far (kvengine/engine.py:394-402)."""
    work = [(list(range(5, 10)), 60)]
    reqs, _ = run_both(models, work, k=3, slots=1, blocks=4, max_ctx=128)
    assert reqs[0].finish_reason == "aborted_cache_exhausted"
    assert 0 < len(reqs[0].new_token_ids) < 60


def test_engine_no_progress_backstop(gpu_lib, models):
    """Nothing running and the queue head cannot be admitted although an empty
    pool would hold it: aborted_no_progress, then the next request is served."""
    work = [(list(range(30)), 4), ([7, 8, 9], 3)]
    reqs, _ = run_both(models, work, k=3, slots=1, blocks=10, hold=6)
    assert [r.finish_reason for r in reqs] == ["aborted_no_progress", "length"]


def test_engine_eos_past_the_budget(gpu_lib, models):
    """The budget trim cuts an EOS emitted past the budget; the request then
    finished on length, not EOS (kvengine/speculative.py:211-214)."""
    tgt, _ = models["gpu"]
    prompt = list(range(40, 52))
    cont = continuation(tgt, prompt, 12)
    for budget in range(1, 10):
        eos = cont[budget]
        if eos in cont[:budget]:
            continue
        eng = SpecEngine(tgt, tgt, k=4, slots=1, t_blocks=64, d_blocks=64, block_size=4, max_ctx=64)
        req = SpecRequest(0, prompt, budget, eos_ids=frozenset({eos}))
        eng.run([req])
        assert req.new_token_ids == cont[:budget]
        assert not req.stopped_on_eos and req.finish_reason == "length"


# ---- bf16: preemption and recompute do not change any output -------------------

@pytest.fixture(scope="module")
def bf16_models():
    from kvengine_amd.arch import TINY128

    return tuple(build_model(TINY128, generate_state_dict(TINY128, seed=s), dtype=torch.bfloat16,
                             device=DEV) for s in (31, 32))


@pytest.mark.parametrize("k,slots", [(1, 24), (4, 20), (8, 20)])
def test_bf16_preemption_keeps_every_output(gpu_lib, bf16_models, k, slots):
    """bf16 target on the wide layer at every width (k=1: 48-row verify passes;
    k=8: 180 rows, kve_linear_rows) and in its prefill: a run whose pools force
    preemption and recompute gives every request exactly the tokens of a run
    with roomy pools, though the draft's proposals (and so the iterations)
    differ between the runs."""
    from kvengine_amd.arch import TINY128

    tgt, drf = bf16_models
    rng = random.Random(40 + k)
    work = [([rng.randrange(TINY128.vocab) for _ in range(rng.randint(20, 120))],
             rng.randint(10, 40)) for _ in range(slots + 4)]
    outs, stats = [], []
    for blocks in (2000, 260):
        eng = SpecEngine(tgt, drf, k=k, slots=slots, t_blocks=blocks, d_blocks=blocks,
                         block_size=4, max_ctx=256)
        assert eng.t_gemm_rows == slots * (k + 1) and eng.narrow_batches
        reqs = [SpecRequest(i, p, m) for i, (p, m) in enumerate(work)]
        eng.run(reqs)
        assert all(r.finish_reason == "length" for r in reqs)
        assert eng.t_pool.manager.num_allocated == 0 and eng.d_pool.manager.num_allocated == 0
        outs.append([r.new_token_ids for r in reqs])
        stats.append(eng.stats)
    assert stats[0].preemptions == 0 and stats[1].preemptions > 0, stats[1].preemptions
    for i, (a, b) in enumerate(zip(*outs)):
        assert a == b, f"request {i} changed under preemption"


@pytest.mark.parametrize("slots,t_blocks,k", [(8, 200, 3), (3, 26, 3), (4, 80, 8)])
def test_engine_prefix_sharing_matches_lockstep_oracle(gpu_lib, models, slots, t_blocks, k):
    """Prefix sharing against the lockstep oracle with the reference Engine's
    adopt / publish points (engine.py:314-319, 364-369, 414-419): tokens,
    accept traces, admission / preemption / finish events, both pools' block
    tables after every iteration and the adopted-token counts agree, with and
    without preemption. Generated tokens' blocks are published too, so a later
    request whose prompt repeats an earlier one's output adopts them."""
    tgt, drf = models["gpu"]
    ref_t, ref_d = models["cpu"]
    rng = random.Random(11 + slots)
    prefix = [rng.randrange(TINY.vocab) for _ in range(37)]
    work = [(prefix + [rng.randrange(TINY.vocab) for _ in range(rng.randint(2, 9))],
             rng.randint(10, 30)) for _ in range(6)]
    # a follow-up turn: request 0's prompt and greedy output, then a new token
    follow = work[0][0] + continuation(tgt, *work[0]) + [rng.randrange(TINY.vocab)]
    work.append((follow, 12))
    trace_g, events_g = [], []
    eng = SpecEngine(tgt, drf, k=k, slots=slots, t_blocks=t_blocks, d_blocks=t_blocks,
                     block_size=4, max_ctx=128, prefix_sharing=True, trace=trace_g,
                     events=events_g)
    reqs = [SpecRequest(i, p, m) for i, (p, m) in enumerate(work)]
    st = eng.run(reqs)
    trace_c, events_c = [], []
    rt, rd = ref_pool(t_blocks), ref_pool(t_blocks)
    rreqs = [RefLockstepRequest(i, p, m) for i, (p, m) in enumerate(work)]
    ref_lockstep_spec(ref_t, ref_d, rreqs, k, slots, rt, rd, trace=trace_c, max_ctx=128,
                      events=events_c, share_prefixes=True)
    for a, b in zip(reqs, rreqs):
        assert a.new_token_ids == b.new_token_ids, a.request_id
        assert a.accepted_per_iter == b.accepted_per_iter, a.request_id
        assert a.finish_reason == b.finish_reason == "length"
    assert events_g == events_c
    assert trace_g == trace_c, "block tables differ from the lockstep replay"
    assert st.prefix_reused_tokens == sum(r.prefix_reused for r in rreqs)
    assert st.prefix_reused_tokens >= 2 * 36 * (len(work) - 2)
    for pool in (eng.t_pool, eng.d_pool):
        pool.manager.check_invariants()
        assert pool.manager.num_allocated == 0
    if t_blocks == 26:
        assert st.preemptions > 0, "pool was meant to force preemption"


def test_short_context_graphs_keep_outputs(gpu_lib, bf16_models):
    """Iterations whose sequences all fit SpecEngine.SHORT_CTX replay a graph
    captured with that context bound (no draft attention merge); the run
    crosses the bound mid-way and its outputs equal a run that always uses the
    full bound."""
    from kvengine_amd.arch import TINY128

    tgt, drf = bf16_models
    rng = random.Random(77)
    work = [([rng.randrange(TINY128.vocab) for _ in range(rng.randint(820, 880))],
             rng.randint(40, 80)) for _ in range(4)]
    outs, used = [], []
    for short in (SpecEngine.SHORT_CTX, 0):
        eng = SpecEngine(tgt, drf, k=4, slots=4, t_blocks=1200, d_blocks=1200, block_size=16,
                         max_ctx=2048)
        eng.SHORT_CTX = short
        reqs = [SpecRequest(i, p, m) for i, (p, m) in enumerate(work)]
        eng.run(reqs)
        outs.append([r.new_token_ids for r in reqs])
        used.append(sorted({c for b in eng.batches.values() for c in b.graphs}))
    assert outs[0] == outs[1]
    assert used[0] == [SpecEngine.SHORT_CTX, 2048], used
    assert used[1] == [2048], used


def test_graphed_prefill_writes_eager_kv(gpu_lib, bf16_models):
    """A single-sequence prefill (a recompute after preemption, a lone
    admission) replays a graph captured per padded token count. Its capture
    run and its replays (other sequences, other lengths in the bucket, a
    nonzero start) write the K/V bits of the eager forward: the target's those
    of the eager wide prefill, the draft's (on the side stream, beside the
    target's prefill, as admission runs them) those of the same padded forward
    run eagerly."""
    from kvengine_amd.arch import TINY128
    from kvengine_amd.forward import forward_hidden

    tgt, drf = bf16_models
    rng = random.Random(9)
    eng = SpecEngine(tgt, drf, k=4, slots=4, t_blocks=800, d_blocks=800, block_size=16,
                     max_ctx=1024)
    assert eng.use_graph and eng._side is not None

    def toks(n):
        return [rng.randrange(TINY128.vocab) for _ in range(n)]

    def kv_bits(seq):
        return [torch.cat([t.view(torch.int16).flatten() for t in seq._gather(li, seq.length)])
                for li in range(TINY128.num_layers)]

    def draft_eager(seq, part):
        T = len(part)
        Tb = eng._prefill_bucket(T)
        seq.reserve(T)
        ids = torch.zeros(1, Tb, dtype=torch.long)
        ids[0, :T] = torch.tensor(part)
        forward_hidden(drf, ids.to(DEV), seq.device_kv(), seq.row_dev, eng.kernel_ctx,
                       q_lens=torch.tensor([T], dtype=torch.int32, device=DEV),
                       attn_order=eng._attn_of(drf))
        seq.commit(T)

    # (tokens already cached, new tokens): 40, 57 and 33 share the 64-token graph
    cases = [(0, 40), (0, 57), (57, 33), (0, 300), (0, 40)]
    side = eng._side
    for i, (p, n) in enumerate(cases):
        parts = [part for part in (toks(p), toks(n)) if part]
        tg, te = eng.t_pool.new_sequence(("g", i)), eng.t_pool.new_sequence(("e", i))
        dg, de = eng.d_pool.new_sequence(("g", i)), eng.d_pool.new_sequence(("e", i))
        for row, seq in ((0, tg), (1, te), (0, dg), (1, de)):
            _bind_row(seq, row)  # the engine's slots own the table rows
        for part in parts:
            cur = torch.cuda.current_stream()
            side.wait_stream(cur)
            eng.use_graph = True
            eng._prefill_batch(tgt, [(tg, part)])
            with torch.cuda.stream(side):
                eng._prefill_batch(drf, [(dg, part)])
            cur.wait_stream(side)
            eng.use_graph = False
            eng._prefill_batch(tgt, [(te, part)])
            draft_eager(de, part)
        for name, a, b in (("target", tg, te), ("draft", dg, de)):
            assert a.length == b.length == p + n
            for li, (x, y) in enumerate(zip(kv_bits(a), kv_bits(b))):
                assert torch.equal(x, y), f"case {i} {name} layer {li}"
        for seq in (tg, te, dg, de):
            seq.free()
    assert sorted(tb for _, tb in eng._pgraphs) == [64, 64, 320, 320]
    assert all(g.graph is not None for g in eng._pgraphs.values())
