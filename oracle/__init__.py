"""CPU oracle for kvengine's speculative-decoding verify path. TEST INFRASTRUCTURE.

This package restates, on the CPU and with the reference's own numerics, the
algorithm of siddharth-diwakar/kvengine's hot path:

* blocks.py     LIFO, refcounted, prefix-registry block allocator (kvengine/blocks.py)
* paged.py      reference-layout paged pool with gather-then-attend reads
                (kvengine/paged.py)
* model.py      the Qwen2 forward pass exactly as kvengine/forward.py drives
                transformers' Qwen2 modules (same torch calls, same order)
* spec.py       greedy speculative loop, plain greedy, accept and rollback
                arithmetic (kvengine/speculative.py, kvengine/decode.py)
* attention.py  gather-then-attend verify attention for one layer, plus a
                float64 brute-force form used to pin it

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import this package, and only as the checker (or, for the CPU
baseline, as the timed reference CPU path). The product package
`kvengine_amd` never imports it: its compute runs in HIP kernels, and it raises
if the HIP library is missing.

How each part is pinned (see tests/test_oracle_*.py):

* blocks.py: the reference's own known-answer and churn tests restated
  (tests/test_blocks.py, tests/test_phase6.py allocator half), plus golden
  block-table traces written by the reference itself.
* paged.py: the reference's known-value round trips (tests/test_phase2.py:254-300)
  and truncate block counts (tests/test_phase5.py:220-237).
* model.py, spec.py: golden token/logit/trace fixtures written by the real
  reference (tests/golden/make_golden.py), compared bit-exactly, and the
  spec == greedy invariant for self, hostile and oracle-acceptance drafts.
* attention.py: golden outputs of the reference's write+gather+attend, and a
  float64 brute force on the same inputs.
* accept/rollback arithmetic: exhaustive enumeration over all
  (draft, prediction) agreement patterns for k <= 8 against a closed form.
"""
