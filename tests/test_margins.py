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
