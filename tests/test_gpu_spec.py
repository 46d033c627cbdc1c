"""End-to-end parity of the HIP speculative path against the reference's fixtures.

The anchors are the reference's own (tests/test_phase5.py): speculative output
equals plain greedy for any draft (self, hostile, oracle-acceptance) and any k;
here additionally the tokens, accept traces and block tables are compared with
fixtures written by the reference itself (tests/golden/make_golden.py).

GPU and CPU float arithmetic differ in summation order, so a token may differ
from the reference only where the reference's own top-2 logit margin is tiny
(a near tie); every such step is counted and must be a near tie.
"""

import copy

import pytest
import torch

from conftest import load_json
from kvengine_amd.arch import PRESETS, QWEN25_0_5B, TINY
from kvengine_amd.decode import greedy_own_cache, greedy_paged
from kvengine_amd.forward import forward_with_own_cache
from kvengine_amd.model import build_model
from kvengine_amd.paged import ContiguousKVCache, PagedKVCache
from kvengine_amd.speculative import speculative_greedy
from kvengine_amd.weights import generate_state_dict
from kvengine_amd.workloads import OracleAcceptance

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = {"torch.float32": torch.float32, "torch.bfloat16": torch.bfloat16}


class HostileDraft:
    """Rolls the vocabulary axis by one, as the reference's tests/test_phase5.py:35-50."""

    def __init__(self, base):
        self.model = base.model
        self.config = base.config
        self.generation_config = base.generation_config
        self._head = base.lm_head
        self.arch = base.arch

    def lm_head(self, hidden):
        return self._head(hidden).roll(shifts=1, dims=-1)

    def parameters(self):
        return self.model.parameters()


def near_tie_ok(got, want, top2_values, tol):
    """Tokens equal, or the first difference sits at a reference near tie."""
    for i, (a, b) in enumerate(zip(got, want)):
        if a != b:
            margin = top2_values[i][0] - top2_values[i][1]
            assert margin <= tol, f"step {i}: {a} != {b} with reference margin {margin}"
            return i
    assert len(got) == len(want)
    return None


@pytest.fixture(scope="module")
def tiny_models():
    out = {}
    for name in ("tiny_fp32.json", "tiny_bf16.json"):
        fx = load_json(name)
        arch = PRESETS[fx["arch"]]
        dtype = DTYPES[fx["dtype"]]
        sd = generate_state_dict(arch, seed=fx["weight_seed"], dtype=torch.float32)
        out[name] = (fx, build_model(arch, sd, dtype=dtype, device=DEV))
    return out


def pool_for(model, blocks=64, bs=4):
    return PagedKVCache.for_model(model, num_blocks=blocks, block_size=bs)


def test_greedy_matches_reference_fp32(gpu_lib, tiny_models):
    """fp32: the same tokens and logits within 1e-4 of the reference's."""
    fx, model = tiny_models["tiny_fp32.json"]
    ids = torch.tensor([fx["prompt"]], device=DEV)
    g = greedy_paged(model, ids, pool_for(model), max_new_tokens=20, eos_token_id=None,
                     collect_logits=True)
    want = fx["greedy"]
    near_tie_ok(g.new_token_ids, want["new_token_ids"], want["top2_values"], 1e-4)
    ref_logits = torch.tensor(want["step_logits"])
    n = len(g.new_token_ids)
    err = (g.step_logits[:n] - ref_logits[:n]).abs().max().item()
    assert err < 1e-4, f"logits drift {err}"


def test_greedy_matches_reference_bf16_teacher_forced(gpu_lib, tiny_models):
    """bf16: the reference's tokens fed one at a time (decode passes, as
    greedy_paged runs them); at every one of the 20 steps the GPU's argmax is
    the reference's top-1 or a mismatch within kvengine_amd.margins.TOL_ULPS of
    it, and every logit is within that many ulps of the reference's."""
    from kvengine_amd.forward import forward_with_own_cache
    from kvengine_amd.margins import TOL_ULPS, bf16_ulp, compare_steps

    fx, model = tiny_models["tiny_bf16.json"]
    want = fx["greedy"]
    ref = torch.tensor(want["step_logits"], dtype=torch.float32)
    seq = pool_for(model).new_sequence("tf")
    got = [forward_with_own_cache(model, torch.tensor([fx["prompt"]], device=DEV), seq)[0, -1]]
    for t in want["new_token_ids"][:-1]:
        got.append(forward_with_own_cache(model, torch.tensor([[t]], device=DEV), seq)[0, -1])
    got = torch.stack(got).float().cpu()
    assert got.shape == ref.shape == (20, model.arch.vocab)
    top = torch.topk(ref, 8, dim=-1)
    ids, vals = [], []
    for v, j in zip(top.values.tolist(), top.indices.tolist()):
        pairs = sorted(zip(v, j), key=lambda p: (-p[0], p[1]))
        vals.append([p[0] for p in pairs])
        ids.append([p[1] for p in pairs])
    am = got.argmax(-1).tolist()
    r = compare_steps(am, ids, vals, got_values=[got[i, a].item() for i, a in enumerate(am)])
    assert r["steps"] == 20 and not r["outside_tolerance"], r
    for i in range(20):
        ulp = bf16_ulp(vals[i][0])
        assert (got[i] - ref[i]).abs().max().item() <= TOL_ULPS * ulp, f"step {i}"


@pytest.mark.parametrize("k", [1, 2, 4, 8])
def test_self_draft_trace_and_blocks_match_reference(gpu_lib, tiny_models, k):
    fx, model = tiny_models["tiny_fp32.json"]
    want = fx["spec_self"][[1, 2, 4, 8].index(k)]
    ids = torch.tensor([fx["prompt"]], device=DEV)
    tp, dp = pool_for(model), pool_for(model)
    ts, ds = tp.new_sequence("target"), dp.new_sequence("draft")
    trace = []
    orig_t, orig_d = ts.truncate, ds.truncate

    def rec(seq, orig, name):
        def f(n, **kw):
            orig(n, **kw)
            trace.append([name, n, list(seq.blocks)])
        return f

    ts.truncate = rec(ts, orig_t, "target")
    ds.truncate = rec(ds, orig_d, "draft")
    r = speculative_greedy(model, model, ids, ts, ds, k=k, max_new_tokens=20, eos_token_id=None)
    assert r.new_token_ids == want["new_token_ids"]
    assert r.accepted_per_iter == want["accepted_per_iter"]
    assert (r.target_forwards, r.draft_forwards) == (want["target_forwards"], want["draft_forwards"])
    assert trace == [list(t) for t in want["truncate_log"]], "block tables differ from the reference"
    assert ts.blocks == want["final_target_blocks"] and ds.blocks == want["final_draft_blocks"]
    # the device tables hold exactly the host tables
    for seq in (ts, ds):
        row = seq.pool.tables[seq.row].cpu().tolist()
        assert row[: len(seq.blocks)] == seq.blocks and all(x == -1 for x in row[len(seq.blocks):])
        assert seq.pool.lens[seq.row].item() == seq.length


@pytest.mark.parametrize("k", [1, 3, 8])
def test_hostile_draft_still_matches_greedy(gpu_lib, tiny_models, k):
    fx, model = tiny_models["tiny_fp32.json"]
    want = fx["spec_hostile"][[1, 3, 8].index(k)]
    ids = torch.tensor([fx["prompt"]], device=DEV)
    r = speculative_greedy(model, HostileDraft(model), ids, pool_for(model).new_sequence("t"),
                           pool_for(model).new_sequence("d"), k=k, max_new_tokens=16,
                           eos_token_id=None)
    assert r.new_token_ids == want["new_token_ids"] == fx["greedy"]["new_token_ids"][:16]
    assert r.accepted_per_iter == want["accepted_per_iter"]
    assert r.acceptance_rate < 0.1


def test_oracle_acceptance_draft(gpu_lib, tiny_models):
    fx, model = tiny_models["tiny_fp32.json"]
    want = fx["spec_oracle"]
    ids = torch.tensor([fx["prompt"]], device=DEV)
    cont = [0] * ids.shape[1] + fx["greedy"]["new_token_ids"]
    oracle = OracleAcceptance(cont, want["p_accept"], want["seed"], TINY.vocab)
    r = speculative_greedy(model, model, ids, pool_for(model).new_sequence("t"),
                           pool_for(model).new_sequence("d"), k=4, max_new_tokens=16,
                           eos_token_id=None, propose=oracle)
    assert r.new_token_ids == want["new_token_ids"]
    assert r.accepted_per_iter == want["accepted_per_iter"]


@pytest.mark.parametrize("k", [1, 2, 4, 8])
def test_bf16_spec_equals_gpu_greedy(gpu_lib, tiny_models, k):
    """The invariant on the GPU itself: spec output == plain greedy, any k."""
    fx, model = tiny_models["tiny_bf16.json"]
    ids = torch.tensor([fx["prompt"]], device=DEV)
    g = greedy_paged(model, ids, pool_for(model), max_new_tokens=20, eos_token_id=None)
    r = speculative_greedy(model, model, ids, pool_for(model).new_sequence("t"),
                           pool_for(model).new_sequence("d"), k=k, max_new_tokens=20,
                           eos_token_id=None)
    assert r.new_token_ids == g.new_token_ids
    h = speculative_greedy(model, HostileDraft(model), ids, pool_for(model).new_sequence("t"),
                           pool_for(model).new_sequence("d"), k=k, max_new_tokens=20,
                           eos_token_id=None)
    assert h.new_token_ids == g.new_token_ids


@pytest.mark.parametrize("k", [1, 4, 8])
@pytest.mark.parametrize("oracle", [False, True], ids=["self", "oracle"])
def test_replayed_iterations_equal_eager(gpu_lib, tiny_models, k, oracle, monkeypatch):
    """bf16 steady-state iterations replay captured graphs (blocks reserved
    before the replay, device commits and rollbacks inside it); the same run
    with every iteration eager gives the same tokens, accept trace, forward
    counts, blocks after every rollback, and device tables and lengths. A
    second call on the same models and pools, its sequences on other table
    rows, replays the graphs the first one captured and gives the same
    tokens, accept trace and forward counts."""
    from kvengine_amd import speculative as spec_mod

    fx, model = tiny_models["tiny_bf16.json"]
    ids = torch.tensor([fx["prompt"]], device=DEV)
    g = greedy_paged(model, ids, pool_for(model), max_new_tokens=48, eos_token_id=None)
    cont = [0] * ids.shape[1] + g.new_token_ids
    replays = []
    orig_run = spec_mod._IterationGraphs.run

    def counted(self, *a):
        replays.append(a[0])
        return orig_run(self, *a)

    monkeypatch.setattr(spec_mod._IterationGraphs, "run", counted)

    def run(tp, dp):
        ts, ds = tp.new_sequence("t"), dp.new_sequence("d")
        trace = []
        for seq, name in ((ts, "target"), (ds, "draft")):
            orig = seq.truncate

            def rec(n, _orig=orig, _seq=seq, _name=name, **kw):
                _orig(n, **kw)
                trace.append([_name, n, list(_seq.blocks)])

            seq.truncate = rec
        propose = OracleAcceptance(cont, 0.5, 3, PRESETS[fx["arch"]].vocab) if oracle else None
        r = speculative_greedy(model, model, ids, ts, ds, k=k, max_new_tokens=40,
                               eos_token_id=None, propose=propose)
        dev = [(seq.pool.tables[seq.row].cpu().tolist(), int(seq.pool.lens[seq.row])) for seq in (ts, ds)]
        out = (r.new_token_ids, r.accepted_per_iter, r.target_forwards, r.draft_forwards,
               trace, list(ts.blocks), list(ds.blocks), dev)
        rows = (ts.row, ds.row)
        ts.free()
        ds.free()
        return out, rows

    def captured():
        return sum(len(x.graphs) for x in spec_mod._GRAPHS.values())

    tp, dp = pool_for(model), pool_for(model)
    graphed, rows1 = run(tp, dp)
    n_replays, n_graphs = len(replays), captured()
    # the second call's sequences take other table rows
    held = [tp.new_sequence("x"), dp.new_sequence("x")]
    for h in held:
        _ = h.row
    again, rows2 = run(tp, dp)
    assert rows2 != rows1
    assert again[:4] == graphed[:4]
    assert captured() == n_graphs and len(replays) == 2 * n_replays
    monkeypatch.setattr(spec_mod._IterationGraphs, "usable", staticmethod(lambda *a: False))
    eager, _ = run(pool_for(model), pool_for(model))
    assert len(replays) == 2 * n_replays and n_replays >= len(graphed[1]) - 1 > 0
    if oracle and k <= 4:
        # both feed lengths replayed (two-token feeds follow a full accept: 1 in 2**k at p 0.5)
        assert {1, 2} <= set(replays), replays
    assert graphed == eager
    assert graphed[0] == g.new_token_ids[:40]


@pytest.mark.parametrize("k", [2, 4])
def test_replayed_iterations_across_the_one_unit_bound(gpu_lib, tiny_models, k, monkeypatch):
    """A history that grows past 896 tokens: iterations whose passes straddle
    the bound run eagerly, later ones replay graphs of 256-token context
    buckets above it; tokens, accept trace, blocks after every rollback and
    device rows equal the all-eager run. (Plain greedy is not compared here:
    its one-token passes and the verify passes can fall on different sides of
    the bound at the same position, and so sum a row's keys in different
    orders.)"""
    from kvengine_amd import speculative as spec_mod

    fx, model = tiny_models["tiny_bf16.json"]
    vocab = PRESETS[fx["arch"]].vocab
    g0 = torch.Generator().manual_seed(5)
    prompt = torch.randint(0, vocab, (1, 860), generator=g0).to(DEV)
    buckets = []
    orig_run = spec_mod._IterationGraphs.run

    def counted(self, u, ctx, *a):
        buckets.append(ctx)
        return orig_run(self, u, ctx, *a)

    monkeypatch.setattr(spec_mod._IterationGraphs, "run", counted)

    def run():
        ts, ds = pool_for(model, blocks=320).new_sequence("t"), pool_for(model, blocks=320).new_sequence("d")
        trace = []
        for seq, name in ((ts, "target"), (ds, "draft")):
            orig = seq.truncate

            def rec(n, _orig=orig, _seq=seq, _name=name, **kw):
                _orig(n, **kw)
                trace.append([_name, n, list(_seq.blocks)])

            seq.truncate = rec
        r = speculative_greedy(model, model, prompt, ts, ds, k=k, max_new_tokens=80,
                               eos_token_id=None)
        dev = [(seq.pool.tables[seq.row].cpu().tolist(), int(seq.pool.lens[seq.row])) for seq in (ts, ds)]
        return (r.new_token_ids, r.accepted_per_iter, r.target_forwards, r.draft_forwards, trace, dev)

    graphed = run()
    assert 896 in buckets and any(b > 896 for b in buckets), buckets
    monkeypatch.setattr(spec_mod._IterationGraphs, "usable", staticmethod(lambda *a: False))
    eager = run()
    assert graphed == eager


def test_budget_trim_and_contiguous_cache(gpu_lib, tiny_models):
    fx, model = tiny_models["tiny_fp32.json"]
    ids = torch.tensor([fx["prompt"]], device=DEV)
    full = fx["greedy"]["new_token_ids"]
    for budget in (1, 3, 7, 10):
        r = speculative_greedy(model, model, ids, ContiguousKVCache.for_model(model, 64),
                               ContiguousKVCache.for_model(model, 64), k=4, max_new_tokens=budget,
                               eos_token_id=None)
        assert r.new_token_ids == full[:budget]
    g = greedy_own_cache(model, ids, max_new_tokens=12, eos_token_id=None)
    assert g.new_token_ids == full[:12]


def test_eos_stops_without_emitting_past_it(gpu_lib, tiny_models):
    fx, model = tiny_models["tiny_fp32.json"]
    ids = torch.tensor([fx["prompt"]], device=DEV)
    full = fx["greedy"]["new_token_ids"]
    eos = full[6]
    r = speculative_greedy(model, model, ids, pool_for(model).new_sequence("t"),
                           pool_for(model).new_sequence("d"), k=4, max_new_tokens=20,
                           eos_token_id=eos)
    stop = full.index(eos)
    assert r.stopped_on_eos and r.new_token_ids == full[: stop + 1]


def test_rejected_blocks_return_to_the_pool(gpu_lib, tiny_models):
    """Hostile k=8 with block_size 4 (tests/test_phase5.py:178-201)."""
    fx, model = tiny_models["tiny_fp32.json"]
    ids = torch.tensor([fx["prompt"]], device=DEV)
    pool = pool_for(model, blocks=64, bs=4)
    ts, ds = pool.new_sequence("target"), pool.new_sequence("draft")
    r = speculative_greedy(model, HostileDraft(model), ids, ts, ds, k=8, max_new_tokens=16,
                           eos_token_id=None)
    assert len(ts.blocks) == pool.manager.blocks_needed(ts.length)
    assert ts.length <= ids.shape[1] + len(r.new_token_ids)
    pool.manager.check_invariants()
    ts.free()
    ds.free()
    assert pool.manager.num_allocated == 0


def test_truncate_then_continue_matches_uninterrupted(gpu_lib, tiny_models):
    """Speculate junk, roll back, continue: same tokens (tests/test_phase5.py:240-266)."""
    fx, model = tiny_models["tiny_fp32.json"]
    ids = torch.tensor([fx["prompt"]], device=DEV)
    pool = pool_for(model)
    cache = pool.new_sequence("r")
    logits = forward_with_own_cache(model, ids, cache)
    produced = []
    for step in range(12):
        tok = int(torch.argmax(logits[0, -1, :]))
        produced.append(tok)
        if step == 5:
            mark = cache.length
            forward_with_own_cache(model, torch.tensor([[tok, tok, tok]], device=DEV), cache)
            cache.truncate(mark)
        logits = forward_with_own_cache(model, torch.tensor([[tok]], device=DEV), cache)
    assert produced == fx["greedy"]["new_token_ids"][:12]


def test_write_then_gather_roundtrips_known_values(gpu_lib, tiny_models):
    """Token t -> value t, v = 100 t, 10 tokens over bs=4 (tests/test_phase2.py:254-274)."""
    _, model = tiny_models["tiny_fp32.json"]
    pool = PagedKVCache.for_model(model, num_blocks=8, block_size=4)
    seq = pool.new_sequence("rt")
    H, D, n = pool.num_kv_heads, pool.head_dim, 10
    k = torch.arange(1, n + 1, dtype=pool.dtype, device=DEV).view(1, 1, n, 1).expand(1, H, n, D)
    k = k.contiguous()
    v = k * 100
    seq.reserve(n)
    k_all, v_all = seq.write(0, k, v, start=0)
    seq.commit(n)
    assert torch.equal(k_all, k) and torch.equal(v_all, v)
    assert len(seq.blocks) == 3


@pytest.mark.slow
def test_config0_self_speculation(gpu_lib):
    """BASELINE config 0 on the GPU: 0.5B arch fp32, k=4, 64 tokens, paged bs=16."""
    fx = load_json("c0_spec.json")
    sd = generate_state_dict(QWEN25_0_5B, seed=0, dtype=torch.float32)
    model = build_model(QWEN25_0_5B, sd, dtype=torch.float32, device=DEV)
    ids = torch.tensor([fx["prompt"]], device=DEV)
    g = greedy_paged(model, ids, PagedKVCache.for_model(model, 512, 16), max_new_tokens=64,
                     eos_token_id=None)
    want = fx["greedy"]
    first = near_tie_ok(g.new_token_ids, want["new_token_ids"], want["top2_values"], 1e-3)
    r = speculative_greedy(model, model, ids, PagedKVCache.for_model(model, 512, 16).new_sequence("t"),
                           PagedKVCache.for_model(model, 512, 16).new_sequence("d"), k=4,
                           max_new_tokens=64, eos_token_id=None)
    assert r.new_token_ids == g.new_token_ids, "spec != greedy on the GPU"
    assert r.acceptance_rate > 0.9
    if first is None:
        assert r.accepted_per_iter == fx["spec_self"]["accepted_per_iter"]
