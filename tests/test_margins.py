"""Margin accounting (kvengine_amd.margins) and the tolerance it uses.

bf16_ulp is checked against torch's own bf16 spacing; compare_steps against
hand-made rankings; TOL_ULPS against what the reference's own fixtures show:
its verify-shaped pass and its decode pass (both written by the reference,
tests/golden/make_golden.py) must agree within the tolerance on every step and
every shared logit, since the tolerance is meant to cover exactly that spread.
"""

import os

import pytest
import torch

from conftest import GOLDEN, load_json
from kvengine_amd.margins import (TOL_ULPS, bf16_ulp, common_id_diffs, compare_steps,
                                  first_divergence, merge_reports, spread)


@pytest.mark.parametrize("x", [1.0, 1.5, 3.609375, 4.0, 0.3, -2.75, 100.0, 1e-3])
def test_bf16_ulp_is_torch_spacing(x):
    b = torch.tensor([x], dtype=torch.bfloat16)
    up = (b.view(torch.int16) + (1 if x > 0 else -1)).view(torch.bfloat16)
    # spacing above |x| for a positive number, below for a negative one
    assert bf16_ulp(float(b)) == abs(float(up) - float(b))


def test_compare_steps_known_cases():
    ids = [[5, 9, 2], [7, 1, 3], [4, 6, 8], [11, 12, 13]]
    vals = [[4.0, 3.875, 3.0], [2.0, 2.0, 1.0], [1.0, 0.5, 0.25], [3.0, 2.0, 1.0]]
    # step 0: other id 1 ulp (2**-5 at 4.0) below: within 9 ulps
    # step 1: exact tie, got the higher id: within tolerance, counted as exact tie
    # step 2: match
    # step 3: id not in the reference's list: outside tolerance
    r = compare_steps([9, 1, 4, 99], ids, vals, got_values=[3.875, 2.0, 1.0, 0.0])
    assert (r["steps"], r["matches"], r["mismatches"]) == (4, 1, 3)
    assert r["exact_ties"] == 1 and r["near_ties"] == 2
    assert [o["step"] for o in r["outside_tolerance"]] == [3]
    assert r["mismatch_steps"] == [0, 1, 3]
    # 2 ulps of tolerance: step 0 (4 ulps below at 4.0: 0.125 / 2**-5) is outside
    r2 = compare_steps([9], ids[:1], vals[:1], ulps=2)
    assert r2["outside_tolerance"] and r2["outside_tolerance"][0]["margin_ulps"] == 4.0
    m = merge_reports([r, r2])
    assert m["steps"] == 5 and len(m["outside_tolerance"]) == 2
    assert first_divergence([1, 2, 3], [1, 2, 4]) == 2 and first_divergence([1, 2], [1, 2, 3]) is None
    assert spread([3, 1, 2])["median"] == 2 and spread([])["n"] == 0


@pytest.mark.skipif(not os.path.exists(os.path.join(GOLDEN, "c2_verify.json")),
                    reason="verify-window fixture not generated")
def test_tolerance_covers_the_references_own_passes():
    """The reference's verify-shaped pass vs its decode pass, same positions
    (3B architecture, seed 1, 128 steps): every id flip and every shared logit
    difference is within TOL_ULPS, and the reference does flip (the tolerance
    is not slack for a path that never disagrees)."""
    g = load_json("c2_full.json")["target_greedy"]
    vw = load_json("c2_verify.json")["target"]
    r = compare_steps([row[0] for row in vw["top_ids"]], g["top_ids"], g["top_values"])
    assert r["mismatches"] > 0 and not r["outside_tolerance"], r
    sp = spread(common_id_diffs(g["top_ids"], g["top_values"], vw["top_ids"], vw["top_values"]))
    assert sp["max"] <= TOL_ULPS, sp
    # and the reference's speculative output leaves its own greedy output
    so = load_json("c2_full.json")["spec_oracle"]
    assert first_divergence(so["new_token_ids"], g["new_token_ids"]) is not None


@pytest.mark.skipif(not all(os.path.exists(os.path.join(GOLDEN, f))
                            for f in ("c3_full.json", "c3_verify.json")),
                    reason="batched-workload fixtures not generated")
def test_tolerance_covers_the_references_own_batched_passes():
    """The same on the 32-request batched workload (3B architecture, 2562
    steps): the reference's verify windows against its decode steps flip
    only within TOL_ULPS and differ by at most TOL_ULPS on shared logits, and
    the largest flip margin needs all of it (the tolerance is no wider than
    the reference's own disagreement)."""
    full, vw = load_json("c3_full.json"), load_json("c3_verify.json")
    reps, diffs, worst = [], [], 0.0
    for r, w in zip(full["requests"], vw["requests"]):
        assert r["index"] == w["index"]
        g = r["greedy"]
        rep = compare_steps([row[0] for row in w["top_ids"]], g["top_ids"], g["top_values"],
                            ulps=1e9)
        reps.append(rep)
        for st in rep["mismatch_steps"]:
            ids, vals = g["top_ids"][st], g["top_values"][st]
            worst = max(worst, (vals[0] - vals[ids.index(w["top_ids"][st][0])]) / bf16_ulp(vals[0]))
        diffs += common_id_diffs(g["top_ids"], g["top_values"], w["top_ids"], w["top_values"])
    m = merge_reports(reps)
    assert m["steps"] == 2562 and m["mismatches"] > 0
    assert worst == TOL_ULPS, worst
    assert spread(diffs)["max"] <= TOL_ULPS


# ---- the exact anchor -------------------------------------------------------

def test_exact_anchor_helpers_known_cases():
    from kvengine_amd.margins import decision_losses, exact_lookup, logit_errors

    st = [{"ref_ids": [5, 9, 2], "at_ref": [4.0, 4.0625, 3.0],
           "top_ids": [9, 5, 7, 2], "top_values": [4.0625, 4.0, 3.5, 3.0]}]
    assert exact_lookup(st[0], 9) == 4.0625 and exact_lookup(st[0], 7) == 3.5
    assert exact_lookup(st[0], 123) is None
    ref_vals = [[4.0, 3.875, 3.0]]
    # errors in ulps of the reference top-1 (2**-5 at 4.0)
    assert logit_errors(st, ref_vals, [[4.0, 3.875, 3.0]]) == [0.0, 6.0, 0.0]
    # the reference picked 5 (exact 4.0): 2 ulps below the exact argmax 9
    assert decision_losses(st, ref_vals, [5]) == [2.0]
    assert decision_losses(st, ref_vals, [9]) == [0.0]
    assert decision_losses(st, ref_vals, [123]) == [None]
    assert decision_losses(st, ref_vals, [7]) == [18.0]


def _exact_sets():
    """(name, reference greedy records, exact records) of every exact fixture."""
    out = []
    if os.path.exists(os.path.join(GOLDEN, "exact_c2.json")):
        out.append(("c2", [load_json("c2_full.json")["target_greedy"]],
                    [load_json("exact_c2.json")]))
    for cfg in ("c3", "c4"):
        if os.path.exists(os.path.join(GOLDEN, f"exact_{cfg}.json")):
            fx, ex = load_json(f"{cfg}_full.json"), load_json(f"exact_{cfg}.json")
            recs = [(r["greedy"], ex["requests"][str(r["index"])]) for r in fx["requests"]
                    if str(r["index"]) in ex["requests"]]
            out.append((cfg, [a for a, _ in recs], [b for _, b in recs]))
    return out


@pytest.mark.parametrize("name,refs,exacts", _exact_sets(), ids=[x[0] for x in _exact_sets()])
def test_exact_fixtures_agree_with_the_reference(name, refs, exacts):
    """The float64 logits (tests/golden/make_exact.py: the oracle's forward pass,
    pinned to the reference in fp32 and bf16, run in float64 on the same bf16
    weights) are the model the reference's bf16 run approximates: every
    reference top-8 logit lies within 16 bf16 ulps of its exact value (a
    dropped term or a misplaced position moves logits by hundreds), the
    reference's greedy pick is among the exact top-16 at every step and is the
    exact argmax at most steps, and both stored views of a logit agree."""
    from kvengine_amd.margins import exact_steps, logit_errors

    n = agree = 0
    errs = []
    for g, e in zip(refs, exacts):
        steps = exact_steps(g["top_ids"], e)
        assert len(steps) == len(g["top_ids"])
        errs += logit_errors(steps, g["top_values"], g["top_values"])
        for st, ids in zip(steps, g["top_ids"]):
            assert ids[0] in st["top_ids"]
            for tok, v in zip(st["ref_ids"], st["at_ref"]):
                if tok in st["top_ids"]:
                    assert st["top_values"][st["top_ids"].index(tok)] == v
                else:
                    assert v <= st["top_values"][-1]
            n += 1
            agree += ids[0] == st["top_ids"][0]
    assert max(errs) <= 16.0, max(errs)
    assert agree >= 0.8 * n, (agree, n)
