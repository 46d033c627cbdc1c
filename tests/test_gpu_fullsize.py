"""Full-depth bf16 parity with the reference at the benchmark configurations.

Models: Qwen2.5-3B-architecture target and 0.5B-architecture draft, bf16,
seed 1 (the single-sequence, batched and prefix-shared configurations). The
fixtures hold the reference's own greedy continuations with the ranked top-8
logits of every step (tests/golden/make_golden.py: c2_full, c3_full, c4_full)
and its verify-shaped passes over the same positions (c2_verify, c3_verify).

bf16 rounding depends on GEMM shapes and summation order, so two correct
implementations may pick different ids where the top-2 margin is tiny; the
reference itself does so between its verify and decode passes. The HIP path is
therefore run teacher-forced (fed the reference's tokens) and compared step by
step: every step must pick the reference's id, or an id within TOL_ULPS bf16
ulps of the reference's top-1 logit (kvengine_amd.margins). Mismatches and
near ties are counted and printed. Free-running runs (speculative_greedy, the
batched engine) must equal the reference's tokens up to a first divergence
that sits at such a near tie, and must equal the GPU's own greedy output
everywhere (spec == greedy, tests/test_phase5.py:62-85).
"""

import os

import pytest
import torch

from conftest import GOLDEN, load_json
from kvengine_amd import kernels
from kvengine_amd.arch import QWEN25_0_5B, QWEN25_3B
from kvengine_amd.engine import SpecEngine, SpecRequest
from kvengine_amd.forward import forward_hidden, invariant_gemm_rows
from kvengine_amd.margins import (TOL_ULPS, bf16_ulp, common_id_diffs, compare_steps,
                                  decision_losses, exact_steps, first_divergence, logit_errors,
                                  merge_reports, spread, value_diffs)
from kvengine_amd.model import build_model
from kvengine_amd.paged import PagedKVCache
from kvengine_amd.speculative import speculative_greedy
from kvengine_amd.weights import generate_state_dict, state_dict_checksum
from kvengine_amd.workloads import OracleAcceptance, batched_spec_workload, prefix_shared_workload

pytestmark = pytest.mark.gpu
DEV = "cuda"


def needs(*names):
    missing = [n for n in names if not os.path.exists(os.path.join(GOLDEN, n))]
    return pytest.mark.skipif(bool(missing), reason=f"fixture not generated: {missing}")


@pytest.fixture(scope="module")
def models():
    fx = load_json("c2_full.json")
    sd_t = generate_state_dict(QWEN25_3B, seed=1, dtype=torch.bfloat16)
    sd_d = generate_state_dict(QWEN25_0_5B, seed=1, dtype=torch.bfloat16)
    assert state_dict_checksum(sd_t) == fx["target_checksum"], "target weights differ from the fixture's"
    assert state_dict_checksum(sd_d) == fx["draft_checksum"], "draft weights differ from the fixture's"
    tgt = build_model(QWEN25_3B, sd_t, dtype=torch.bfloat16, device=DEV)
    drf = build_model(QWEN25_0_5B, sd_d, dtype=torch.bfloat16, device=DEV)
    del sd_t, sd_d
    return tgt, drf


def report(name, r, sp=None):
    msg = (f"[parity] {name}: {r['steps']} steps, {r['mismatches']} mismatches "
           f"(near ties {r['near_ties']}, exact ties {r['exact_ties']}), outside tolerance "
           f"{len(r['outside_tolerance'])}")
    if sp is not None:
        msg += (f"; logits at the reference's top-8 ids differ by median {sp['median']:.2f}, "
                f"p90 {sp['p90']:.2f}, max {sp['max']:.2f} ulp")
    print(msg, flush=True)


# Logit-level bounds (ulps of each step's top-1) for the GPU's logits at the
# reference's top-8 ids. The reference's own verify and decode passes differ by
# median 1, p90 2.5, max 7 on the single-sequence fixture; a dropped term, a
# wrong sign or a swapped operand anywhere in 36 layers moves logits by tens to
# hundreds of ulps. The maximum sits above the reference's self-spread
# because the reference is itself up to 12.4 ulps from the exact logits (the
# exact anchor below): two implementations each within that of the model can
# be farther apart than either is from it.
MEDIAN_ULPS, P90_ULPS, MAX_ULPS = 2.0, 5.0, 12.0


def check_spread(sp):
    assert sp["median"] <= MEDIAN_ULPS and sp["p90"] <= P90_ULPS and sp["max"] <= MAX_ULPS, sp


# The exact anchor (tests/golden/exact_*.json, make_exact.py): float64 logits
# of the same bf16-weight model at the same teacher-forced steps. Both bf16
# implementations are compared with it. The HIP path's logit error (|logit -
# exact| at the reference's top-8 ids, in ulps of the step's top-1) may exceed
# the reference's own on the same steps by at most one ulp at the 90th
# percentile, and its largest error may exceed the reference's largest over
# every exact fixture (C2, C3 and C4: 2754 steps, 22,032 logits) by at most
# one ulp: the maximum of a few hundred values is too noisy to compare set by
# set. A greedy pick's decision loss is the exact top-1 minus the exact logit
# of the id picked; the reference's own picks lose up to REF_MAX_LOSS ulps
# (the reference's bf16 logits order the exact argmax below another id by up
# to 9 ulps, as far as its own verify and decode passes disagree). A
# mismatch with the reference beyond TOL_ULPS is accepted only where the HIP
# path's pick loses no more than the reference's worst pick plus one ulp.
EXACT_SLACK_ULPS = 1.0


def _exact_sets():
    sets = [(load_json("c2_full.json")["target_greedy"], load_json("exact_c2.json"))]
    for cfg in ("c3", "c4"):
        fx, ex = load_json(f"{cfg}_full.json"), load_json(f"exact_{cfg}.json")
        sets += [(r["greedy"], ex["requests"][str(r["index"])]) for r in fx["requests"]]
    return sets


def reference_max_loss() -> float:
    """The reference's largest greedy decision loss over the exact fixtures."""
    worst = 0.0
    for g, e in _exact_sets():
        losses = decision_losses(exact_steps(g["top_ids"], e), g["top_values"],
                                 [x[0] for x in g["top_ids"]])
        worst = max(worst, max(x for x in losses if x is not None))
    return worst


def reference_max_error() -> float:
    """The reference's largest logit error over the exact fixtures."""
    return max(max(logit_errors(exact_steps(g["top_ids"], e), g["top_values"], g["top_values"]))
               for g, e in _exact_sets())


def exact_anchor(name, steps, ref_vals, ref_ids_chosen, gpu_vals_at_ref, gpu_chosen,
                 outside=()):
    """Checks one comparison against the exact logits; returns the summary."""
    ref_err = spread(logit_errors(steps, ref_vals, ref_vals))
    gpu_err = spread(logit_errors(steps, ref_vals, gpu_vals_at_ref))
    rl = decision_losses(steps, ref_vals, ref_ids_chosen)
    gl = decision_losses(steps, ref_vals, gpu_chosen)
    ref_loss = max(x for x in rl if x is not None)
    ref_worst = reference_max_loss()
    ref_max_err = reference_max_error()
    assert all(x is not None for x in gl), (name, "a chosen id is below the exact top-16")
    gpu_loss = max(gl)
    near2 = sum(1 for st, v in zip(steps, ref_vals) if v[0] - v[1] <= 2 * bf16_ulp(v[0]))
    summary = {"ref_err": ref_err, "gpu_err": gpu_err, "ref_max_loss": ref_loss,
               "gpu_max_loss": gpu_loss, "ref_max_loss_all_fixtures": ref_worst,
               "ref_max_err_all_fixtures": ref_max_err,
               "ref_off_exact_argmax": sum(1 for x in rl if x is not None and x > 0),
               "gpu_off_exact_argmax": sum(1 for x in gl if x > 0),
               "near_ties_2ulp": near2}
    print(f"[exact] {name}: logit error vs exact (ulps) reference median {ref_err['median']:.2f} "
          f"p90 {ref_err['p90']:.2f} max {ref_err['max']:.2f} (largest over every fixture "
          f"{ref_max_err:.2f}), HIP median {gpu_err['median']:.2f} "
          f"p90 {gpu_err['p90']:.2f} max {gpu_err['max']:.2f}; picks off the exact argmax: "
          f"reference {summary['ref_off_exact_argmax']}, HIP {summary['gpu_off_exact_argmax']} of "
          f"{len(steps)} (largest loss {ref_loss:.2f} / {gpu_loss:.2f} ulps; the reference's "
          f"largest over every fixture {ref_worst:.2f}); reference near ties within 2 ulps "
          f"{near2}, within {TOL_ULPS:g} ulps {sum(1 for v in ref_vals if v[0] - v[1] <= TOL_ULPS * bf16_ulp(v[0]))}",
          flush=True)
    assert gpu_err["p90"] <= ref_err["p90"] + EXACT_SLACK_ULPS, (name, summary)
    assert gpu_err["max"] <= ref_max_err + EXACT_SLACK_ULPS, (name, summary)
    return summary


def unexplained(steps, ref, outside):
    """compare_steps' outside-tolerance entries whose pick lies further below
    the exact argmax than the reference's own worst greedy pick (+1 ulp)."""
    bound = reference_max_loss() + EXACT_SLACK_ULPS
    left = []
    for o in outside:
        st = steps[o["step"]]
        loss = decision_losses([st], [ref["top_values"][o["step"]]], [o["got"]])[0]
        if loss is None or loss > bound:
            left.append({**o, "exact_loss_ulps": loss, "bound_ulps": bound})
    return left


def heads(model, hidden):
    """argmax, its value, runner-up id of hidden rows [M, H] (fused LM head)."""
    M = hidden.shape[0]
    am = torch.empty(M, dtype=torch.int32, device=DEV)
    mx = torch.empty(M, dtype=torch.float32, device=DEV)
    sid = torch.empty(M, dtype=torch.int32, device=DEV)
    kernels.lmhead_argmax(hidden, model.lm_head.weight, argmax=am, maxval=mx, second_id=sid)
    return am, mx, sid


def values_at(model, hidden, ids):
    """The model's logits (bf16-rounded float32 dot products) of hidden rows
    [N, H] at ids [N][n]."""
    idx = torch.tensor(ids, dtype=torch.long, device=DEV)
    w = model.lm_head.weight[idx].float()                      # [N, n, H]
    v = torch.bmm(w, hidden.float().unsqueeze(-1)).squeeze(-1)  # [N, n]
    return v.to(torch.bfloat16).float().cpu().tolist()


def run_pass(model, seq, ids, gemm_rows=None):
    """One forward of ids (list) into seq; final-normed hidden rows [T, H]."""
    T = len(ids)
    start = seq.length
    seq.reserve(T)
    x = torch.tensor([ids], dtype=torch.long, device=DEV)
    h = forward_hidden(model, x, seq.device_kv(), seq.row_dev, start + T, gemm_rows=gemm_rows)
    seq.commit(T)
    return h[0]


def teacher_forced_greedy(model, prompt, cont):
    """The reference's greedy_paged shapes (prefill the prompt, then one token
    per pass), fed the reference's tokens: (ids chosen for cont[0..], their
    logits, the hidden rows)."""
    pool = PagedKVCache.for_model(model, -(-(len(prompt) + len(cont) + 1) // 16) + 1, 16)
    seq = pool.new_sequence("tf")
    rows = [run_pass(model, seq, prompt)[-1:].clone()]
    for t in cont[:-1]:
        rows.append(run_pass(model, seq, [t]).clone())
    seq.free()
    hid = torch.cat(rows)
    am, mx, _ = heads(model, hid)
    return am.tolist(), mx.tolist(), hid


def teacher_forced_windows(model, prompt, cont, window, gemm_rows):
    """Verify-shaped passes: prompt[:-1] prefilled, then windows of `window`
    tokens of prompt[-1:] + cont (the engine's steady-state verify)."""
    pool = PagedKVCache.for_model(model, -(-(len(prompt) + len(cont) + 1) // 16) + 1, 16)
    seq = pool.new_sequence("tfw")
    run_pass(model, seq, prompt[:-1])
    toks = prompt[-1:] + cont[:-1]
    rows = []
    for w in range(0, len(toks), window):
        rows.append(run_pass(model, seq, toks[w:w + window], gemm_rows=gemm_rows).clone())
    seq.free()
    hid = torch.cat(rows)
    am, mx, _ = heads(model, hid)
    return am.tolist(), mx.tolist(), hid


def logit_spread(model, hid, ref):
    return spread(value_diffs(ref["top_ids"], ref["top_values"],
                              values_at(model, hid, ref["top_ids"])))


def engine_gemm_rows(model, slots=32, k=4):
    ok, rows = invariant_gemm_rows(model, slots * (k + 1))
    assert ok
    return rows


# ------------------------------------------------------------ single sequence

def test_c2_target_greedy_teacher_forced(gpu_lib, models):
    tgt, _ = models
    fx = load_json("c2_full.json")
    g = fx["target_greedy"]
    am, mx, hid = teacher_forced_greedy(tgt, fx["prompt"], g["new_token_ids"])
    r = compare_steps(am, g["top_ids"], g["top_values"], mx)
    sp = logit_spread(tgt, hid, g)
    report("3B greedy (q_len 1) vs reference greedy", r, sp)
    steps = exact_steps(g["top_ids"], load_json("exact_c2.json"))
    assert r["steps"] == 128 and not unexplained(steps, g, r["outside_tolerance"]), \
        r["outside_tolerance"]
    check_spread(sp)
    exact_anchor("C2 3B greedy (q_len 1)", steps, g["top_values"], [x[0] for x in g["top_ids"]],
                 values_at(tgt, hid, g["top_ids"]), am)


def test_c2_draft_greedy_teacher_forced(gpu_lib, models):
    _, drf = models
    fx = load_json("c2_full.json")
    g = fx["draft_greedy"]
    am, mx, hid = teacher_forced_greedy(drf, fx["prompt"], g["new_token_ids"])
    r = compare_steps(am, g["top_ids"], g["top_values"], mx)
    sp = logit_spread(drf, hid, g)
    report("0.5B greedy (q_len 1) vs reference greedy", r, sp)
    assert r["steps"] == 128 and not r["outside_tolerance"], r["outside_tolerance"]
    check_spread(sp)


def test_c2_target_verify_windows_teacher_forced(gpu_lib, models):
    """The engine's verify pass (wide split-K layer, q_len 5) against the
    reference's verify-shaped pass and against its greedy, same positions."""
    tgt, _ = models
    fx = load_json("c2_full.json")
    vw = load_json("c2_verify.json")["target"]
    g = fx["target_greedy"]
    am, mx, hid = teacher_forced_windows(tgt, fx["prompt"], g["new_token_ids"], 5,
                                         engine_gemm_rows(tgt))
    r = compare_steps(am, vw["top_ids"], vw["top_values"], mx)
    sp = logit_spread(tgt, hid, vw)
    report("3B verify windows vs reference verify windows", r, sp)
    assert r["steps"] == 128 and not r["outside_tolerance"], r["outside_tolerance"]
    check_spread(sp)
    r2 = compare_steps(am, g["top_ids"], g["top_values"], mx)
    sp2 = logit_spread(tgt, hid, g)
    report("3B verify windows vs reference greedy", r2, sp2)
    steps = exact_steps(g["top_ids"], load_json("exact_c2.json"))
    assert not unexplained(steps, g, r2["outside_tolerance"]), r2["outside_tolerance"]
    check_spread(sp2)
    exact_anchor("C2 3B verify windows (q_len 5)", steps, g["top_values"],
                 [x[0] for x in g["top_ids"]], values_at(tgt, hid, g["top_ids"]), am)
    # the reference's own two passes, for scale
    r3 = compare_steps([row[0] for row in vw["top_ids"]], g["top_ids"], g["top_values"])
    sp3 = spread(common_id_diffs(g["top_ids"], g["top_values"], vw["top_ids"], vw["top_values"]))
    report("reference verify windows vs reference greedy", r3, sp3)


def check_free_running(name, tokens, accepted, ref_greedy, ref_spec):
    """tokens equal the reference's greedy continuation up to a first
    divergence at a near tie; the accept trace equals the reference's
    speculative trace while both token streams are still that continuation.
    Returns (first divergence, iterations compared)."""
    cont = ref_greedy["new_token_ids"]
    d = first_divergence(tokens, cont)
    if d is not None:
        top = compare_steps([tokens[d]], [ref_greedy["top_ids"][d]], [ref_greedy["top_values"][d]])
        assert not top["outside_tolerance"], (name, d, top)
    ref_d = first_divergence(ref_spec["new_token_ids"], cont)
    lim = min(x for x in (d, ref_d, len(cont)) if x is not None)
    done = n = 0
    for a, b in zip(accepted, ref_spec["accepted_per_iter"]):
        if done + a + 1 > lim:
            break
        assert a == b, (name, n, accepted[:n + 1], ref_spec["accepted_per_iter"][:n + 1])
        done += a + 1
        n += 1
    return d, n


def test_c2_speculative_and_engine(gpu_lib, models):
    """speculative_greedy and a one-slot engine with oracle acceptance p=0.65 on
    the reference's continuation: tokens equal the reference's up to a first
    divergence at a near tie, accept traces equal the reference's while the
    token streams agree."""
    tgt, drf = models
    fx = load_json("c2_full.json")
    prompt, g = fx["prompt"], fx["target_greedy"]
    so = fx["spec_oracle"]
    cont = [0] * len(prompt) + g["new_token_ids"]

    def oracle():
        return OracleAcceptance(cont, 0.65, seed=so["seed"], vocab=QWEN25_3B.vocab)

    ids = torch.tensor([prompt], device=DEV)
    r = speculative_greedy(tgt, drf, ids, PagedKVCache.for_model(tgt, 64, 16).new_sequence("t"),
                           PagedKVCache.for_model(drf, 64, 16).new_sequence("d"), k=4,
                           max_new_tokens=128, eos_token_id=None, propose=oracle())
    eng = SpecEngine(tgt, drf, k=4, slots=1, t_blocks=64, d_blocks=64, block_size=16, max_ctx=256)
    req = SpecRequest(0, prompt, 128, propose=oracle())
    eng.run([req])
    assert len(r.new_token_ids) == len(req.new_token_ids) == 128
    d1, n1 = check_free_running("speculative_greedy", r.new_token_ids, r.accepted_per_iter, g, so)
    d2, n2 = check_free_running("engine", req.new_token_ids, req.accepted_per_iter, g, so)
    print(f"[parity] C2 vs reference: speculative_greedy first divergence {d1} ({n1} accept "
          f"iterations equal), one-slot engine {d2} ({n2}); reference's own spec leaves its "
          f"greedy at {first_divergence(so['new_token_ids'], g['new_token_ids'])}", flush=True)


# ------------------------------------------------------------ batched (32 requests)

@needs("c3_full.json", "c3_verify.json", "exact_c3.json")
def test_c3_teacher_forced_batched_verify(gpu_lib, models):
    """All 32 requests at once in the engine's verify shape (32 x 5 rows, wide
    split-K layer, ragged tails), fed the reference's continuations."""
    tgt, _ = models
    fx = load_json("c3_full.json")
    vw = {r["index"]: r for r in load_json("c3_verify.json")["requests"]}
    work = batched_spec_workload(seed=0, n=32, vocab=QWEN25_3B.vocab)
    reqs = fx["requests"]
    for r in reqs:
        assert work[r["index"]][0][:8] == r["prompt_head"]
    B, W = len(reqs), 5
    gemm_rows = engine_gemm_rows(tgt)
    nb = sum(-(-(len(work[r["index"]][0]) + r["max_new_tokens"] + W) // 16) + 1 for r in reqs)
    pool = PagedKVCache.for_model(tgt, nb, 16, max_seqs=B)
    seqs = [pool.new_sequence(i) for i in range(B)]
    for s, r in zip(seqs, reqs):
        run_pass(tgt, s, work[r["index"]][0][:-1])
    toks = [work[r["index"]][0][-1:] + r["greedy"]["new_token_ids"][:-1] for r in reqs]
    got = [[] for _ in reqs]
    rows = torch.tensor([s.row for s in seqs], dtype=torch.int32, device=DEV)
    longest = max(len(t) for t in toks)
    for w in range(0, longest, W):
        chunk = [t[w:w + W] for t in toks]
        ql = [len(c) for c in chunk]
        ids = torch.zeros(B, W, dtype=torch.long)
        for i, c in enumerate(chunk):
            if c:
                ids[i, :len(c)] = torch.tensor(c, dtype=torch.long)
                seqs[i].reserve(len(c))
        max_ctx = max(s.length for s in seqs) + W
        h = forward_hidden(tgt, ids.to(DEV), pool.device_kv(), rows, max_ctx,
                           q_lens=torch.tensor(ql, dtype=torch.int32, device=DEV),
                           gemm_rows=gemm_rows)
        hb = h.reshape(B, W, -1)
        for i, c in enumerate(chunk):
            if c:
                seqs[i].commit(len(c))
                got[i].append(hb[i, :len(c)].clone())
    vs_greedy, vs_windows, dg, dw = [], [], [], []
    exact = load_json("exact_c3.json")["requests"]
    all_steps, ref_vals, ref_pick, gpu_vals, gpu_pick, left = [], [], [], [], [], []
    for i, r in enumerate(reqs):
        hid = torch.cat(got[i])
        am, mx, _ = heads(tgt, hid)
        a, m = am.tolist(), mx.tolist()
        gr, w = r["greedy"], vw[r["index"]]
        cg = compare_steps(a, gr["top_ids"], gr["top_values"], m)
        cw = compare_steps(a, w["top_ids"], w["top_values"], m)
        vs_greedy.append(cg)
        vs_windows.append(cw)
        vals = values_at(tgt, hid, gr["top_ids"])
        dg.extend(value_diffs(gr["top_ids"], gr["top_values"], vals))
        dw.extend(value_diffs(w["top_ids"], w["top_values"], values_at(tgt, hid, w["top_ids"])))
        steps = exact_steps(gr["top_ids"], exact[str(r["index"])])
        left += [{**o, "request": r["index"]} for o in unexplained(steps, gr, cg["outside_tolerance"])]
        left += [{**o, "request": r["index"], "vs": "windows"}
                 for o in unexplained(steps, gr, cw["outside_tolerance"])]
        all_steps += steps
        ref_vals += gr["top_values"]
        ref_pick += [x[0] for x in gr["top_ids"]]
        gpu_vals += vals
        gpu_pick += a
    rg, rw = merge_reports(vs_greedy), merge_reports(vs_windows)
    report("C3 32x5 verify passes vs reference greedy", rg, spread(dg))
    report("C3 32x5 verify passes vs reference verify windows", rw, spread(dw))
    print(f"[parity] C3: {len(rg['outside_tolerance'])} + {len(rw['outside_tolerance'])} "
          f"mismatches beyond {rg['tolerance_ulps']} reference ulps, all but {len(left)} "
          f"within the reference's own exact decision loss: "
          f"{(rg['outside_tolerance'] + rw['outside_tolerance'])[:4]}", flush=True)
    assert rg["steps"] == sum(r["max_new_tokens"] for r in reqs)
    assert not left, left[:5]
    check_spread(spread(dg))
    check_spread(spread(dw))
    exact_anchor("C3 32x5 verify passes", all_steps, ref_vals, ref_pick, gpu_vals, gpu_pick)


def concurrent_peak(target, draft, work, conts, k):
    """Most target blocks held at once in an unconstrained engine run."""
    eng = SpecEngine(target, draft, k=k, slots=32, t_blocks=2000, d_blocks=2000, block_size=16,
                     max_ctx=1664)
    eng.run([SpecRequest(i, p, o, propose=OracleAcceptance([0] * len(p) + conts[i], 0.65,
                                                           seed=1000 + i, vocab=QWEN25_3B.vocab))
             for i, (p, o) in enumerate(work)])
    return eng.stats.peak_target_blocks, eng.stats.peak_draft_blocks


@needs("c3_full.json")
def test_c3_engine_against_reference(gpu_lib, models):
    """The batched configuration as benchmarked, at every k of its sweep
    (1, 2, 4, 8; scripts/phase5_demo.py:102-141 checks each k the same way):
    32 requests, oracle acceptance p=0.65 (seed 1000 + i) on the reference's
    greedy continuations, pools at 80% of that k's concurrent peak so
    preemption fires. Every request's tokens equal the reference's up to a
    first divergence at a near tie; the reference's continuations do not
    depend on k, and neither may the engine's: every k gives every request
    the same tokens (the GPU's own greedy continuation). The accept traces
    at k=4 equal the reference's speculative traces while both streams are
    the reference continuation."""
    tgt, drf = models
    fx = load_json("c3_full.json")
    work = batched_spec_workload(seed=0, n=32, vocab=QWEN25_3B.vocab)
    reqs_fx = {r["index"]: r for r in fx["requests"]}
    conts = [reqs_fx[i]["greedy"]["new_token_ids"] for i in range(32)]
    outs = {}
    for k in (1, 2, 4, 8):
        pt, pd = concurrent_peak(tgt, drf, work, conts, k)
        pool = int(0.8 * max(pt, pd))
        eng = SpecEngine(tgt, drf, k=k, slots=32, t_blocks=pool, d_blocks=pool, block_size=16,
                         max_ctx=1664)
        reqs = [SpecRequest(i, p, o, propose=OracleAcceptance([0] * len(p) + conts[i], 0.65,
                                                              seed=1000 + i,
                                                              vocab=QWEN25_3B.vocab))
                for i, (p, o) in enumerate(work)]
        st = eng.run(reqs)
        print(f"[parity] C3 engine k={k}: peak blocks {pt}/{pd}, pool {pool}, preemptions "
              f"{st.preemptions}, recomputed tokens {st.recomputed_tokens}, acceptance "
              f"{st.acceptance_rate:.3f}", flush=True)
        assert st.preemptions > 0 and st.aborted == 0
        diverged, same_trace_iters = [], 0
        for i, r in enumerate(reqs):
            f = reqs_fx[i]
            assert len(r.new_token_ids) == f["max_new_tokens"] and r.finish_reason == "length"
            if k == 4:
                d, n = check_free_running(f"request {i}", r.new_token_ids, r.accepted_per_iter,
                                          f["greedy"], f["spec_oracle"])
                same_trace_iters += n
            else:
                d = first_divergence(r.new_token_ids, f["greedy"]["new_token_ids"])
                if d is not None:
                    top = compare_steps([r.new_token_ids[d]], [f["greedy"]["top_ids"][d]],
                                        [f["greedy"]["top_values"][d]])
                    assert not top["outside_tolerance"], (k, i, d, top)
            if d is not None:
                diverged.append((i, d))
        print(f"[parity] C3 engine k={k} vs reference: {len(diverged)} of 32 requests diverge "
              f"at a near tie {diverged}" +
              (f"; {same_trace_iters} accept-trace iterations checked" if k == 4 else ""),
              flush=True)
        for pool_ in (eng.t_pool, eng.d_pool):
            pool_.manager.check_invariants()
            assert pool_.manager.num_allocated == 0
        outs[k] = [r.new_token_ids for r in reqs]
        del eng
    for k in (1, 2, 8):
        assert outs[k] == outs[4], f"k={k} tokens differ from k=4"


# ------------------------------------------------------------ prefix-shared long context

@needs("c4_full.json", "exact_c4.json")
def test_c4_prefix_shared_teacher_forced(gpu_lib, models):
    """Two requests of the prefix-shared configuration: the second adopts the
    first's 128 published prefix blocks (refcount 2) and both are verified in
    k=8 windows (q_len 9) over the reference's continuations."""
    tgt, _ = models
    fx = load_json("c4_full.json")
    work = prefix_shared_workload(seed=0, vocab=QWEN25_3B.vocab)
    pool = PagedKVCache.for_model(tgt, 400, 16, max_seqs=4)
    seqs = []
    for r in fx["requests"]:
        prompt = work[r["index"]][0]
        assert prompt[:8] == r["prompt_head"]
        s = pool.new_sequence(r["index"])
        n = s.adopt_prefix(prompt)
        if seqs:
            assert n == 2048 and s.blocks == seqs[0].blocks[:128]
        run_pass(tgt, s, prompt[n:-1])
        s.register_prefix_blocks(prompt[:-1])
        seqs.append(s)
    assert pool.manager.refcount(seqs[0].blocks[0]) == 2
    reports, diffs, left = [], [], []
    exact = load_json("exact_c4.json")["requests"]
    all_steps, ref_vals, ref_pick, gpu_vals, gpu_pick = [], [], [], [], []
    for sq, r in zip(seqs, fx["requests"]):
        prompt = work[r["index"]][0]
        toks = prompt[-1:] + r["greedy"]["new_token_ids"][:-1]
        rows = [run_pass(tgt, sq, toks[w:w + 9], gemm_rows=engine_gemm_rows(tgt, 16, 8)).clone()
                for w in range(0, len(toks), 9)]
        hid = torch.cat(rows)
        am, mx, _ = heads(tgt, hid)
        gr = r["greedy"]
        c = compare_steps(am.tolist(), gr["top_ids"], gr["top_values"], mx.tolist())
        reports.append(c)
        vals = values_at(tgt, hid, gr["top_ids"])
        diffs.extend(value_diffs(gr["top_ids"], gr["top_values"], vals))
        steps = exact_steps(gr["top_ids"], exact[str(r["index"])])
        left += unexplained(steps, gr, c["outside_tolerance"])
        all_steps += steps
        ref_vals += gr["top_values"]
        ref_pick += [x[0] for x in gr["top_ids"]]
        gpu_vals += vals
        gpu_pick += am.tolist()
    rr = merge_reports(reports)
    report("C4 shared-prefix verify windows (q_len 9) vs reference greedy", rr, spread(diffs))
    assert rr["steps"] == 64 and not left, rr["outside_tolerance"]
    check_spread(spread(diffs))
    exact_anchor("C4 shared-prefix verify windows (q_len 9)", all_steps, ref_vals, ref_pick,
                 gpu_vals, gpu_pick)


@needs("c4_full.json")
def test_c4_engine_to_8192(gpu_lib, models):
    """The prefix-shared configuration through the batched engine until the
    contexts reach 8192 tokens: 16 requests of a 2048-token shared prefix +
    a 256-token suffix, 5888 new tokens each, k=8, oracle acceptance p=0.5,
    prefix sharing on. The target's verify attention runs in the engine's
    long-context order (16-block units past 4096 tokens, up to 32 units
    merged per sequence) over the 128 shared physical blocks. Every request
    adopts the first request's published prefix (refcount 16 while all are
    running, kvengine/blocks.py:232-306, kvengine/engine.py:410-419), every
    request's tokens equal the GPU's own greedy continuation (the engine with
    the target as its own draft), requests 0 and 1 equal the reference's
    first 32 greedy tokens up to a near-tie divergence, and both pools pass
    their invariants and end empty."""
    from kvengine_amd.engine import LONG_CTX_AT, TARGET_ATTN_LONG

    tgt, drf = models
    fx = load_json("c4_full.json")
    k, p, new = 8, 0.5, 5888
    work = prefix_shared_workload(seed=0, vocab=QWEN25_3B.vocab, new_tokens=new)
    max_ctx = -(-(2048 + 256 + new + k + 2) // 64) * 64
    assert max_ctx > LONG_CTX_AT
    blocks = 128 + 16 * (-(-(256 + new + k + 16) // 16) + 1)

    def engine(draft):
        return SpecEngine(tgt, draft, k=k, slots=16, t_blocks=blocks, d_blocks=blocks,
                          block_size=16, max_ctx=max_ctx, prefix_sharing=True)

    ce = engine(tgt)
    base = [SpecRequest(i, pr, o) for i, (pr, o) in enumerate(work)]
    ce.run(base)
    conts = [r.new_token_ids for r in base]
    del ce
    for r in fx["requests"]:
        d = first_divergence(conts[r["index"]][:32], r["greedy"]["new_token_ids"])
        if d is not None:
            top = compare_steps([conts[r["index"]][d]], [r["greedy"]["top_ids"][d]],
                                [r["greedy"]["top_values"][d]])
            assert not top["outside_tolerance"], (r["index"], d, top)
    eng = engine(drf)
    assert eng.target_attn == TARGET_ATTN_LONG
    reqs = [SpecRequest(i, pr, o, propose=OracleAcceptance([0] * len(pr) + conts[i], p,
                                                           seed=1000 + i, vocab=QWEN25_3B.vocab))
            for i, (pr, o) in enumerate(work)]
    for r in reqs:
        eng.add_request(r)
    eng._admit()
    live = [s for s in eng.slots if s is not None]
    assert len(live) == 16
    shared = live[0].t.blocks[:128]
    for s in live[1:]:
        assert s.t.blocks[:128] == shared
    assert all(eng.t_pool.manager.refcount(b) == 16 for b in shared)
    st = eng.run([])
    print(f"[parity] C4 engine to {2048 + 256 + new} tokens: {st.iterations} iterations, "
          f"acceptance {st.acceptance_rate:.3f}, prefix tokens adopted {st.prefix_reused_tokens}",
          flush=True)
    assert st.aborted == 0 and st.prefix_reused_tokens >= 2 * 15 * 2048
    for i, r in enumerate(reqs):
        assert len(r.new_token_ids) == new and r.finish_reason == "length"
        assert r.new_token_ids == conts[i], f"request {i} leaves the greedy continuation"
    for pool_ in (eng.t_pool, eng.d_pool):
        pool_.manager.check_invariants()
        assert pool_.manager.num_allocated == 0
