"""Top-2 margin accounting for greedy token streams computed in bf16.

Greedy decoding picks argmax(logits). Two implementations that round the same
bf16 model differently (another GEMM shape, another summation order) agree
on every step whose top-2 logit margin is larger than their rounding
difference, and may pick either id where the margin is smaller: a near tie.
The reference shows this on itself: its bf16 verify pass (q_len = k+1) and
its bf16 decode pass (q_len = 1) pick different ids at near ties of the same
positions (kvengine/speculative.py:160-167 vs kvengine/decode.py:296-310 on
the CPU), so its speculative output leaves its own greedy output there.

A comparison therefore walks the steps of a token stream against the
reference's ranked top entries for the same positions (same prefix, i.e.
teacher-forced, or up to the first divergence when free-running): a step
matches when the chosen id is the reference's top-1; a mismatch is within
tolerance when the chosen id is among the reference's top entries with a
logit no more than `ulps` bf16 ulps (at the top-1 magnitude) below the top-1.
"""

from __future__ import annotations

import math

# Tolerance in bf16 ulps at the top-1 magnitude: as far as the reference's
# own two bf16 passes disagree. Its verify pass (q_len 5) and decode pass
# (q_len 1) give the same positions logit values up to 7 ulps apart on the
# 3B-architecture single sequence (seed 1, 128 steps; flips on 13 steps at
# margins up to 4 ulps) and up to 9 ulps apart on the 32-request batched
# workload (2562 steps; 225 flips, the largest at a 9-ulp margin). Two
# roundings that far apart can flip any step whose margin is below their
# difference, so a mismatch is within tolerance up to a 9-ulp margin.
TOL_ULPS = 9.0


def bf16_ulp(x: float) -> float:
    """Spacing of bf16 numbers at |x| (8 significant bits)."""
    a = abs(float(x))
    if a == 0.0 or not math.isfinite(a):
        return 2.0 ** -133
    return 2.0 ** (math.floor(math.log2(a)) - 7)


def margin_tolerance(top1: float, ulps: float = TOL_ULPS) -> float:
    return ulps * bf16_ulp(top1)


def compare_steps(got_ids, ref_top_ids, ref_top_values, got_values=None,
                  ulps: float = TOL_ULPS) -> dict:
    """Step-by-step comparison of chosen ids with the reference's ranked top
    entries (lists per step, ordered by value then id).

    Returns counts (steps, matches, mismatches, near_ties: steps whose
    reference top-2 margin is within tolerance), the mismatches outside
    tolerance with their reference margins, and, when got_values (the logit
    of each chosen id) is given, the largest difference between a chosen
    id's value and the reference's value for that id, in ulps."""
    steps = min(len(got_ids), len(ref_top_ids))
    out = {"steps": steps, "matches": 0, "mismatches": 0, "near_ties": 0, "exact_ties": 0,
           "mismatch_steps": [], "outside_tolerance": [], "max_value_diff_ulps": 0.0,
           "tolerance_ulps": ulps}
    for i in range(steps):
        ids, vals = list(ref_top_ids[i]), list(ref_top_values[i])
        u = bf16_ulp(vals[0])
        tol = ulps * u
        if vals[0] - vals[1] <= tol:
            out["near_ties"] += 1
        if vals[0] == vals[1]:
            out["exact_ties"] += 1
        g = int(got_ids[i])
        if g == ids[0]:
            out["matches"] += 1
        else:
            out["mismatches"] += 1
            out["mismatch_steps"].append(i)
            if g in ids:
                margin = vals[0] - vals[ids.index(g)]
                if margin > tol:
                    out["outside_tolerance"].append(
                        {"step": i, "got": g, "ref": ids[0], "margin_ulps": margin / u})
            else:
                out["outside_tolerance"].append(
                    {"step": i, "got": g, "ref": ids[0],
                     "margin_ulps_at_least": (vals[0] - vals[-1]) / u})
        if got_values is not None and g in ids:
            d = abs(float(got_values[i]) - vals[ids.index(g)]) / u
            out["max_value_diff_ulps"] = max(out["max_value_diff_ulps"], d)
    return out


def first_divergence(a, b) -> int | None:
    """First index where two token lists differ (None if one is a prefix of the other)."""
    return next((i for i, (x, y) in enumerate(zip(a, b)) if x != y), None)


def merge_reports(reports) -> dict:
    """Sum of compare_steps reports (outside-tolerance lists concatenated)."""
    out = {"steps": 0, "matches": 0, "mismatches": 0, "near_ties": 0, "exact_ties": 0,
           "outside_tolerance": [], "max_value_diff_ulps": 0.0}
    for r in reports:
        for key in ("steps", "matches", "mismatches", "near_ties", "exact_ties"):
            out[key] += r[key]
        out["outside_tolerance"].extend(r["outside_tolerance"])
        out["max_value_diff_ulps"] = max(out["max_value_diff_ulps"], r["max_value_diff_ulps"])
        out["tolerance_ulps"] = r.get("tolerance_ulps")
    return out


def value_diffs(ref_top_ids, ref_top_values, got_values_at_ids) -> list[float]:
    """|got - ref| in ulps (of each step's top-1) for every reference top entry;
    got_values_at_ids[i][j] is the other side's logit at ref_top_ids[i][j]."""
    out = []
    for ids, vals, got in zip(ref_top_ids, ref_top_values, got_values_at_ids):
        u = bf16_ulp(vals[0])
        out.extend(abs(float(g) - v) / u for v, g in zip(vals, got))
    return out


def spread(diffs) -> dict:
    """Median, 90th percentile and maximum of a list of differences."""
    d = sorted(diffs)
    if not d:
        return {"n": 0, "median": 0.0, "p90": 0.0, "max": 0.0}
    return {"n": len(d), "median": d[len(d) // 2], "p90": d[int(0.9 * (len(d) - 1))], "max": d[-1]}


def common_id_diffs(a_ids, a_vals, b_ids, b_vals) -> list[float]:
    """Differences (in ulps of a's top-1) between two rankings' values at the
    ids both list, step by step."""
    out = []
    for ai, av, bi, bv in zip(a_ids, a_vals, b_ids, b_vals):
        u = bf16_ulp(av[0])
        pos = {x: j for j, x in enumerate(bi)}
        out.extend(abs(v - bv[pos[x]]) / u for x, v in zip(ai, av) if x in pos)
    return out


# ---- exact-arithmetic anchor ------------------------------------------------
# Both the reference and the HIP path round a bf16 model; neither is the model.
# The fixtures tests/golden/exact_*.json hold, for the same teacher-forced
# steps, float64 logits of the model itself (the same bf16 weights, every
# operation in float64): at the reference's top-8 ids and the exact top-16.
# Against them each side has a logit error (|value - exact| in ulps of the
# step's top-1) and a decision loss (how far, in exact logits, the id it picks
# falls below the exact argmax).

def exact_lookup(step: dict, tok: int) -> float | None:
    """Exact logit of id tok at one step (None if below the exact top-16 and
    not among the reference's top-8)."""
    if tok in step["ref_ids"]:
        return step["at_ref"][step["ref_ids"].index(tok)]
    if tok in step["top_ids"]:
        return step["top_values"][step["top_ids"].index(tok)]
    return None


def exact_steps(ref_top_ids, exact: dict) -> list[dict]:
    """Per-step lookup records from an exact fixture entry (exact_at_ref_top,
    exact_top_ids, exact_top_values) and the reference ids it was written for."""
    return [{"ref_ids": list(ri), "at_ref": list(ea), "top_ids": list(ti), "top_values": list(tv)}
            for ri, ea, ti, tv in zip(ref_top_ids, exact["exact_at_ref_top"],
                                      exact["exact_top_ids"], exact["exact_top_values"])]


def logit_errors(steps: list[dict], ref_top_values, values_at_ref_ids) -> list[float]:
    """|values - exact| in ulps of each step's reference top-1, at the
    reference's top-8 ids; values_at_ref_ids[i][j] is one side's logit there."""
    out = []
    for st, rv, vals in zip(steps, ref_top_values, values_at_ref_ids):
        u = bf16_ulp(rv[0])
        out.extend(abs(float(v) - e) / u for v, e in zip(vals, st["at_ref"]))
    return out


def decision_losses(steps: list[dict], ref_top_values, chosen) -> list[float | None]:
    """Exact top-1 minus the exact logit of the chosen id, in ulps of the
    step's reference top-1 (None when the chosen id is not in the fixture)."""
    out = []
    for st, rv, tok in zip(steps, ref_top_values, chosen):
        e = exact_lookup(st, int(tok))
        out.append(None if e is None else (st["top_values"][0] - e) / bf16_ulp(rv[0]))
    return out
