"""Pin the oracle's lockstep replay of batched speculative decoding (CPU).

`oracle/batch.py` is the checker of the batched engine. It composes pinned
pieces (RefQwen2, RefPagedKVCache, accept), but its own scheduling has no
reference counterpart, so it is pinned here by what the reference fixes:

* the spec == greedy invariant (tests/test_phase5.py:62-85) for every request,
  for a self, a hostile and an oracle-acceptance draft, with and without
  preemption;
* with one slot and no preemption it is the reference's speculative_greedy:
  tokens, accepted_per_iter and forward-count-independent traces equal the
  fixtures the reference itself wrote (tiny_fp32.json);
* the reference Engine's preemption known answers (tests/test_phase3.py:161-232,
  kvengine/engine.py:137-146, 425-440): the newest running request is the
  victim, it is requeued at the front, it resumes by recomputing
  prompt + outputs[:-1], and output is preserved exactly;
* the abort backstops (engine.py:262-267, 297-306, 394-402).
"""

import copy
import random

import pytest
import torch

from conftest import load_json
from kvengine_amd.arch import TINY
from kvengine_amd.weights import generate_state_dict
from kvengine_amd.workloads import OracleAcceptance
from oracle.batch import RefLockstepRequest, ref_lockstep_spec
from oracle.model import RefQwen2
from oracle.paged import RefPagedKVCache
from oracle.spec import ref_greedy


@pytest.fixture(scope="module")
def models():
    # thousands of tiny forwards: one intra-op thread (a busy host otherwise
    # makes torch's thread pool 30x slower on them)
    threads = torch.get_num_threads()
    torch.set_num_threads(1)
    sd_t = generate_state_dict(TINY, seed=3, dtype=torch.float32)
    sd_d = generate_state_dict(TINY, seed=4, dtype=torch.float32)
    yield RefQwen2(TINY, sd_t), RefQwen2(TINY, sd_d)
    torch.set_num_threads(threads)


def pool(n, bs=4):
    return RefPagedKVCache(TINY.num_layers, TINY.num_kv_heads, TINY.head_dim, n, bs, torch.float32)


def hostile(model):
    m = copy.copy(model)
    m.lm_head_hook = lambda logits: logits.roll(shifts=1, dims=-1)
    return m


def greedy(model, prompt, n):
    seq = pool(-(-(len(prompt) + n + 1) // 4)).new_sequence("greedy")
    return ref_greedy(model, torch.tensor([prompt]), seq, max_new_tokens=n).new_token_ids


def workload(n, seed, budgets=(3, 24)):
    rng = random.Random(seed)
    return [([rng.randrange(TINY.vocab) for _ in range(rng.randint(5, 21))], rng.randint(*budgets))
            for _ in range(n)]


class Recorder:
    """Delegates to a model and logs (request id, cache length, fed ids) per forward."""

    def __init__(self, model, log):
        self.m = model
        self.log = log

    def forward(self, ids, cache, all_logits=False):
        self.log.append((cache.request_id, cache.length, ids[0].tolist()))
        return self.m.forward(ids, cache, all_logits=all_logits)


@pytest.mark.parametrize("draft_kind", ["self", "other", "hostile", "oracle"])
@pytest.mark.parametrize("k,slots,blocks", [(1, 3, 200), (3, 4, 200), (4, 3, 26)])
def test_every_request_equals_its_greedy(models, draft_kind, k, slots, blocks):
    tgt, other = models
    draft = {"self": tgt, "other": other, "hostile": hostile(tgt), "oracle": other}[draft_kind]
    work = workload(6, seed=k * 7 + slots, budgets=(30, 40) if blocks == 26 else (3, 24))
    conts = [greedy(tgt, p, m) for p, m in work]
    reqs = []
    for i, (p, m) in enumerate(work):
        prop = None
        if draft_kind == "oracle":
            prop = OracleAcceptance([0] * len(p) + conts[i], 0.65, seed=50 + i, vocab=TINY.vocab)
        reqs.append(RefLockstepRequest(i, p, m, propose=prop))
    tp, dp = pool(blocks), pool(blocks)
    ref_lockstep_spec(tgt, draft, reqs, k, slots, tp, dp)
    for r, c in zip(reqs, conts):
        assert r.new_token_ids == c, r.request_id
        assert r.finish_reason == "length"
    for p in (tp, dp):
        p.manager.check_invariants()
        assert p.manager.num_allocated == 0
    if blocks == 26:
        assert sum(r.preemptions for r in reqs) > 0, "pool was meant to force preemption"
    if draft_kind == "self":
        assert all(a == k for r in reqs for a in r.accepted_per_iter[:-1])
    if draft_kind == "hostile":
        assert sum(sum(r.accepted_per_iter) for r in reqs) <= len(reqs)


@pytest.mark.parametrize("k", [1, 2, 4, 8])
def test_one_slot_is_the_reference_loop(models, k):
    """One slot, no preemption: the reference's own traces (self draft)."""
    tgt, _ = models
    fx = load_json("tiny_fp32.json")
    want = fx["spec_self"][[1, 2, 4, 8].index(k)]
    req = RefLockstepRequest(0, fx["prompt"], 20)
    ref_lockstep_spec(tgt, tgt, [req], k, 1, pool(64), pool(64))
    assert req.new_token_ids == want["new_token_ids"]
    assert req.accepted_per_iter == want["accepted_per_iter"]


@pytest.mark.parametrize("k", [1, 3, 8])
def test_one_slot_hostile_is_the_reference_loop(models, k):
    tgt, _ = models
    fx = load_json("tiny_fp32.json")
    want = fx["spec_hostile"][[1, 3, 8].index(k)]
    req = RefLockstepRequest(0, fx["prompt"], 16)
    ref_lockstep_spec(tgt, hostile(tgt), [req], k, 1, pool(64), pool(64))
    assert req.new_token_ids == want["new_token_ids"]
    assert req.accepted_per_iter == want["accepted_per_iter"]


def test_one_slot_oracle_acceptance_is_the_reference_loop(models):
    tgt, _ = models
    fx = load_json("tiny_fp32.json")
    want = fx["spec_oracle"]
    cont = [0] * len(fx["prompt"]) + fx["greedy"]["new_token_ids"]
    prop = OracleAcceptance(cont, want["p_accept"], want["seed"], TINY.vocab)
    req = RefLockstepRequest(0, fx["prompt"], 16, propose=prop)
    ref_lockstep_spec(tgt, tgt, [req], 4, 1, pool(64), pool(64))
    assert req.new_token_ids == want["new_token_ids"]
    assert req.accepted_per_iter == want["accepted_per_iter"]


def check_schedule(events, request_ids):
    """FIFO admission; the victim of a preemption is the most recently admitted
    running request; it goes back to the front of the queue."""
    queue = list(request_ids)
    live: list = []
    for e in events:
        if e[0] == "admit":
            assert e[1] == queue.pop(0), f"admitted out of order: {e}"
            live.append(e[1])
        elif e[0] == "preempt":
            assert e[1] == live[-1], f"victim {e[1]} is not the newest of {live}"
            live.pop()
            queue.insert(0, e[1])
        else:
            if e[1] in live:
                live.remove(e[1])
            elif e[1] in queue:  # aborted before admission
                queue.remove(e[1])
    assert not live and not queue


@pytest.mark.parametrize("slots,blocks,n", [(3, 30, 4), (3, 30, 6), (4, 24, 5)])
def test_preemption_known_answers(models, slots, blocks, n):
    """Newest victim, requeued at the front, resumed by recomputing
    prompt + outputs[:-1] (no token duplicated or dropped at the boundary);
    output preserved exactly."""
    tgt, drf = models
    rng = random.Random(slots * 100 + blocks + n)
    work = [([rng.randrange(TINY.vocab) for _ in range(rng.randint(6, 12))], rng.randint(30, 40))
            for _ in range(n)]
    conts = [greedy(tgt, p, m) for p, m in work]
    log: list = []
    events: list = []
    reqs = [RefLockstepRequest(i, p, m) for i, (p, m) in enumerate(work)]
    k = 3
    tp, dp = pool(blocks), pool(blocks)
    ref_lockstep_spec(Recorder(tgt, log), drf, reqs, k, slots, tp, dp, events=events)
    for r, c in zip(reqs, conts):
        assert r.new_token_ids == c
    assert sum(r.preemptions for r in reqs) > 0, "pool was meant to force preemption"
    assert sum(1 for e in events if e[0] == "preempt") == sum(r.preemptions for r in reqs)
    check_schedule(events, [r.request_id for r in reqs])
    for r in reqs:
        full = r.prompt + r.new_token_ids
        feeds = [(length, ids) for rid, length, ids in log if rid == r.request_id]
        prefills = [(length, ids) for length, ids in feeds if length == 0]
        assert len(prefills) == 1 + r.preemptions
        assert prefills[0][1] == r.prompt[:-1]
        for length, ids in prefills[1:]:
            # prompt + the outputs generated so far, minus the last one
            assert len(ids) >= len(r.prompt) and ids == full[: len(ids)]
        for length, ids in feeds:
            if length == 0:
                continue
            # every verify starts at the token right after what the cache holds
            assert len(ids) == k + 1 and ids[0] == full[length]
    for p in (tp, dp):
        assert p.manager.num_allocated == 0


def test_prompt_larger_than_pool_is_rejected_not_retried(models):
    """tests/test_phase3.py:206-221: aborted at once, no blocks held; the
    requests behind it are still served."""
    tgt, drf = models
    rng = random.Random(2)
    big = ([rng.randrange(TINY.vocab) for _ in range(20)], 10)
    small = ([rng.randrange(TINY.vocab) for _ in range(3)], 4)
    reqs = [RefLockstepRequest(0, *big), RefLockstepRequest(1, *small)]
    tp, dp = pool(5), pool(5)
    ref_lockstep_spec(tgt, drf, reqs, 3, 1, tp, dp)
    assert reqs[0].finish_reason == "aborted_prompt_too_long" and reqs[0].new_token_ids == []
    assert reqs[1].finish_reason == "length"
    assert reqs[1].new_token_ids == greedy(tgt, small[0], small[1])
    assert tp.manager.num_allocated == 0 and dp.manager.num_allocated == 0


def test_max_ctx_rejects_what_a_table_row_cannot_hold(models):
    tgt, drf = models
    req = RefLockstepRequest(0, list(range(10)), 50)
    ref_lockstep_spec(tgt, drf, [req], 3, 1, pool(64), pool(64), max_ctx=48)
    assert req.finish_reason == "aborted_prompt_too_long"


def test_generation_outgrowing_pool_aborts_rather_than_truncating(models):
    """tests/test_phase3.py:224-236: the prompt fits, the output cannot."""
    tgt, drf = models
    req = RefLockstepRequest(0, list(range(5, 10)), 60)
    tp, dp = pool(4), pool(4)
    ref_lockstep_spec(tgt, drf, [req], 3, 1, tp, dp)
    assert req.finish_reason == "aborted_cache_exhausted"
    assert 0 < len(req.new_token_ids) < 60
    assert req.new_token_ids == greedy(tgt, req.prompt, 60)[: len(req.new_token_ids)]
    assert tp.manager.num_allocated == 0 and dp.manager.num_allocated == 0


def test_no_progress_backstop(models):
    """Nothing running and the queue head cannot be admitted although it would
    fit an empty pool (blocks held outside the scheduler): it is aborted
    rather than retried forever; the next request is then served."""
    tgt, drf = models
    tp, dp = pool(10), pool(10)
    held = tp.manager.allocate(6, owner="elsewhere")
    reqs = [RefLockstepRequest(0, list(range(30)), 4), RefLockstepRequest(1, [7, 8, 9], 3)]
    ref_lockstep_spec(tgt, drf, reqs, 3, 1, tp, dp)
    assert reqs[0].finish_reason == "aborted_no_progress" and reqs[0].new_token_ids == []
    assert reqs[1].finish_reason == "length" and len(reqs[1].new_token_ids) == 3
    tp.manager.free(held)
    assert tp.manager.num_allocated == 0


def test_eos_past_the_budget_is_not_reported(models):
    """speculative.py:211-214: the budget trim can cut an EOS that was
    emitted past the budget; stopped_on_eos follows the last kept token."""
    tgt, _ = models
    prompt = list(range(40, 52))
    cont = greedy(tgt, prompt, 12)
    for budget in range(1, 10):
        eos = cont[budget]  # the token right after the budget
        if eos in cont[:budget]:
            continue
        req = RefLockstepRequest(0, prompt, budget, eos_ids=(eos,))
        ref_lockstep_spec(tgt, tgt, [req], 4, 1, pool(64), pool(64))
        assert req.new_token_ids == cont[:budget]
        assert req.stopped_on_eos is False and req.finish_reason == "length"


def test_forced_preds_replay_follows_the_continuation(models):
    """The CPU baseline's timing replay: with the target's argmax replaced by a
    continuation, the loop emits that continuation, accepts exactly the
    oracle's successful draws, and where the continuation is the target's own
    fp32 greedy (self-consistent) nothing changes."""
    from oracle.spec import ref_speculative_greedy

    tgt, drf = models
    prompt, n = [5, 17, 300, 2, 9, 41, 77], 30
    cont = greedy(tgt, prompt, n)

    def run(forced, seed):
        prop = OracleAcceptance([0] * len(prompt) + cont, 0.65, seed=seed, vocab=TINY.vocab)
        return ref_speculative_greedy(tgt, drf, torch.tensor([prompt]), pool(40).new_sequence("t"),
                                      pool(40).new_sequence("d"), k=4, max_new_tokens=n,
                                      propose=prop, forced_preds=forced)

    plain = run(None, 9)
    forced = run(prompt + cont, 9)
    assert plain.new_token_ids == forced.new_token_ids == cont
    assert plain.accepted_per_iter == forced.accepted_per_iter
    # an arbitrary continuation is followed too, whatever the model predicts
    other = [(t * 7 + 3) % TINY.vocab for t in cont]
    r = ref_speculative_greedy(tgt, drf, torch.tensor([prompt]), pool(40).new_sequence("t"),
                               pool(40).new_sequence("d"), k=4, max_new_tokens=n,
                               propose=OracleAcceptance([0] * len(prompt) + other, 0.65, seed=3,
                                                        vocab=TINY.vocab),
                               forced_preds=prompt + other)
    assert r.new_token_ids == other
    assert sum(r.accepted_per_iter) + r.iterations >= n


def test_prefix_sharing_known_answers(models):
    """The oracle's prefix sharing (reference Engine adopt/publish points): every
    request still equals its greedy continuation; the first request's prompt
    blocks are adopted by every later one in both pools; a follow-up whose
    prompt repeats request 0's prompt and output adopts the blocks request 0
    published during decoding (generated tokens are shareable, engine.py:414-419);
    pools end empty with the published blocks reclaimable."""
    tgt, drf = models
    rng = random.Random(5)
    prefix = [rng.randrange(TINY.vocab) for _ in range(37)]  # 9 full blocks of 4 within len - 1
    work = [(prefix + [rng.randrange(TINY.vocab) for _ in range(rng.randint(2, 9))],
             rng.randint(10, 20)) for _ in range(4)]
    cont0 = greedy(tgt, *work[0])
    follow = work[0][0] + cont0 + [7]
    work.append((follow, 6))
    tp, dp = pool(120), pool(120)
    reqs = [RefLockstepRequest(i, p, m) for i, (p, m) in enumerate(work)]
    ev = []
    ref_lockstep_spec(tgt, drf, reqs, 3, 2, tp, dp, events=ev, share_prefixes=True)
    for r, (p, m) in zip(reqs, work):
        assert r.new_token_ids == greedy(tgt, p, m)
    assert reqs[0].prefix_reused == 0
    assert all(r.prefix_reused >= 2 * 36 for r in reqs[1:4])
    # the follow-up (admitted after request 0 finished) reuses at least the blocks
    # request 0 held over its prompt and output, in both pools
    full0 = (len(work[0][0]) + len(cont0) - 1) // 4 * 4
    assert reqs[4].prefix_reused >= 2 * (full0 - 4)
    for p_ in (tp, dp):
        p_.manager.check_invariants()
        assert p_.manager.num_allocated == 0
