"""Write exact-arithmetic logit fixtures for the full-depth bf16 parity tests.

The reference's bf16 runs (c2_full.json, c3_full.json, c4_full.json) round
every activation to bf16, and so does the HIP path, at different points; two
correct implementations therefore disagree by a few bf16 ulps, and pick
different ids at near ties. To tell which side is closer to the model they
both approximate, this script evaluates that model exactly: the same bf16
weights, cast to float64, through the oracle's Qwen2 forward pass (oracle/
model.py, pinned bit-exactly to the reference in fp32 and bf16) run entirely
in float64, teacher-forced on the reference's own greedy tokens. Every step's
row is the logits after prompt + greedy[:step], as in the bf16 fixtures.

Per step it stores the float64 logits at the reference's top-8 ids (from the
bf16 fixture) and the exact top-16 entries (ids and values, ordered by value
then id). Positions come from the fixtures; nothing here imports or runs the
reference, and nothing runs on the GPU box.

  exact_c2.json   the 128 target greedy steps of c2_full.json
  exact_c3.json   every greedy step of the 32 requests of c3_full.json
  exact_c4.json   the 2 x 32 steps of c4_full.json

Usage: python tests/golden/make_exact.py [--only c2,c3,c4] [--requests 0,1,...]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from kvengine_amd.arch import QWEN25_3B  # noqa: E402
from kvengine_amd.weights import generate_state_dict, state_dict_checksum  # noqa: E402
from oracle.model import RefQwen2  # noqa: E402

TOPN = 16


class ContiguousCache:
    """Single-sequence contiguous K/V store with the oracle's cache protocol."""

    def __init__(self, layers: int):
        self.length = 0
        self.k = [None] * layers
        self.v = [None] * layers

    def reserve(self, n: int) -> None:
        pass

    def write(self, layer: int, k, v, start: int):
        if self.k[layer] is None:
            self.k[layer], self.v[layer] = k, v
        else:
            self.k[layer] = torch.cat([self.k[layer][:, :, :start], k], dim=2)
            self.v[layer] = torch.cat([self.v[layer][:, :, :start], v], dim=2)
        return self.k[layer], self.v[layer]

    def commit(self, n: int) -> None:
        self.length += n


def exact_steps(model: RefQwen2, prompt: list[int], greedy: list[int], ref_top_ids):
    """float64 logits for the greedy steps: row s follows prompt + greedy[:s]."""
    ids = torch.tensor([prompt + greedy[:-1]])
    hidden = model.forward(ids, ContiguousCache(model.arch.num_layers), all_logits=True,
                           return_hidden=True)
    rows = hidden[0, len(prompt) - 1:]
    assert rows.shape[0] == len(greedy)
    logits = model.lm_head(rows)
    out = {"exact_at_ref_top": [], "exact_top_ids": [], "exact_top_values": []}
    vals, idx = torch.topk(logits, 2 * TOPN, dim=-1)
    for s in range(len(greedy)):
        out["exact_at_ref_top"].append(logits[s, ref_top_ids[s]].tolist())
        pairs = sorted(zip(vals[s].tolist(), idx[s].tolist()), key=lambda p: (-p[0], p[1]))[:TOPN]
        out["exact_top_values"].append([p[0] for p in pairs])
        out["exact_top_ids"].append([p[1] for p in pairs])
    return out


def load(name):
    with open(os.path.join(HERE, name)) as f:
        return json.load(f)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", default="c2,c3,c4")
    ap.add_argument("--requests", default="", help="c3 request indices (default: all)")
    args = ap.parse_args()
    torch.set_num_threads(os.cpu_count() or 8)
    t0 = time.time()
    sd = generate_state_dict(QWEN25_3B, seed=1, dtype=torch.bfloat16)
    checksum = state_dict_checksum(sd)
    model = RefQwen2(QWEN25_3B, sd, dtype=torch.float64)
    del sd
    meta = {"target_arch": QWEN25_3B.name, "weight_seed": 1, "weights": "bf16 cast to float64",
            "arithmetic": "float64 throughout (oracle/model.py)", "target_checksum": checksum}
    print(f"float64 model built in {time.time() - t0:.1f}s", flush=True)
    only = set(args.only.split(","))
    if "c2" in only:
        fx = load("c2_full.json")
        assert fx["target_checksum"] == checksum
        g = fx["target_greedy"]
        t = time.time()
        res = {**meta, **exact_steps(model, fx["prompt"], g["new_token_ids"], g["top_ids"])}
        with open(os.path.join(HERE, "exact_c2.json"), "w") as f:
            json.dump(res, f, separators=(",", ":"))
        print(f"c2: {len(g['new_token_ids'])} steps in {time.time() - t:.1f}s", flush=True)
    if "c3" in only:
        from kvengine_amd.workloads import batched_spec_workload

        fx = load("c3_full.json")
        assert fx["target_checksum"] == checksum
        work = batched_spec_workload(seed=0, n=32, vocab=QWEN25_3B.vocab)
        pick = [int(x) for x in args.requests.split(",")] if args.requests else range(len(work))
        path = os.path.join(HERE, "exact_c3.json")
        res = load("exact_c3.json") if os.path.exists(path) else {**meta, "requests": {}}
        for i in pick:
            r = fx["requests"][i]
            prompt = work[i][0]
            assert prompt[:8] == r["prompt_head"] and len(prompt) == r["prompt_len"]
            t = time.time()
            res["requests"][str(i)] = exact_steps(model, prompt, r["greedy"]["new_token_ids"],
                                                  r["greedy"]["top_ids"])
            with open(path, "w") as f:
                json.dump(res, f, separators=(",", ":"))
            print(f"c3 request {i}: prompt {len(prompt)}, {r['max_new_tokens']} steps, "
                  f"{time.time() - t:.1f}s", flush=True)
    if "c4" in only:
        from kvengine_amd.workloads import prefix_shared_workload

        fx = load("c4_full.json")
        assert fx["target_checksum"] == checksum
        work = prefix_shared_workload(seed=0, vocab=QWEN25_3B.vocab)
        res = {**meta, "requests": {}}
        for r in fx["requests"]:
            i = r["index"]
            prompt = work[i][0]
            t = time.time()
            res["requests"][str(i)] = exact_steps(model, prompt, r["greedy"]["new_token_ids"],
                                                  r["greedy"]["top_ids"])
            print(f"c4 request {i}: {time.time() - t:.1f}s", flush=True)
        with open(os.path.join(HERE, "exact_c4.json"), "w") as f:
            json.dump(res, f, separators=(",", ":"))


if __name__ == "__main__":
    main()
