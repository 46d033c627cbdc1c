"""Pin the CPU oracle against fixtures written by the real reference.

The fixtures (tests/golden/make_golden.py) come from kvengine's own
forward_with_own_cache / PagedKVCache / speculative_greedy over transformers'
Qwen2 modules. The oracle restates the same torch calls in the same order, so on
the CPU it must agree bit for bit: tokens, float logits, accept traces, and the
block table after every rollback.
"""

import copy

import pytest
import torch

from conftest import load_json, load_npz_tensors
from kvengine_amd.arch import PRESETS, QWEN25_0_5B, QWEN25_3B, TINY, layer_slice
from kvengine_amd.weights import generate_state_dict, state_dict_checksum
from kvengine_amd.workloads import OracleAcceptance
from oracle.attention import attend_fp64, gather_then_attend, normalized_error
from oracle.model import RefQwen2
from oracle.paged import RefPagedKVCache
from oracle.spec import ref_greedy, ref_speculative_greedy

DTYPES = {"torch.float32": torch.float32, "torch.bfloat16": torch.bfloat16}


def ref_pool(arch, dtype, num_blocks, block_size):
    return RefPagedKVCache(arch.num_layers, arch.num_kv_heads, arch.head_dim, num_blocks,
                           block_size, dtype)


def hostile(model):
    m = copy.copy(model)
    m.lm_head_hook = lambda logits: logits.roll(shifts=1, dims=-1)
    return m


def check_trace(res, t_seq, d_seq, fx):
    assert res.new_token_ids == fx["new_token_ids"]
    assert res.accepted_per_iter == fx["accepted_per_iter"]
    assert res.iterations == fx["iterations"]
    assert res.tokens_drafted == fx["tokens_drafted"]
    assert res.tokens_accepted == fx["tokens_accepted"]
    assert res.target_forwards == fx["target_forwards"]
    assert res.draft_forwards == fx["draft_forwards"]
    assert t_seq.blocks == fx["final_target_blocks"]
    assert d_seq.blocks == fx["final_draft_blocks"]
    assert t_seq.length == fx["target_len"] and d_seq.length == fx["draft_len"]
    # Block tables after every rollback, target then draft, in call order.
    got = []
    for tb, db in res.block_trace:
        got.append(("target", tb))
        got.append(("draft", db))
    want = [(rid, blocks) for rid, _n, blocks in fx["truncate_log"]]
    assert got == [tuple(w) for w in want]


@pytest.mark.parametrize("fixture", ["tiny_fp32.json", "tiny_bf16.json"])
def test_tiny_model_matches_reference_bit_exactly(fixture):
    fx = load_json(fixture)
    arch = PRESETS[fx["arch"]]
    dtype = DTYPES[fx["dtype"]]
    sd = generate_state_dict(arch, seed=fx["weight_seed"], dtype=torch.float32)
    assert state_dict_checksum(sd) == fx["weights_checksum"]
    model = RefQwen2(arch, sd, dtype)
    ids = torch.tensor([fx["prompt"]])

    pool = ref_pool(arch, dtype, 64, 4)
    g = ref_greedy(model, ids, pool.new_sequence("req"), 20, collect_logits=True)
    assert g.new_token_ids == fx["greedy"]["new_token_ids"]
    assert torch.equal(g.step_logits, torch.tensor(fx["greedy"]["step_logits"]))

    for k, want in zip((1, 2, 4, 8), fx["spec_self"]):
        t, d = ref_pool(arch, dtype, 64, 4), ref_pool(arch, dtype, 64, 4)
        ts, ds = t.new_sequence("target"), d.new_sequence("draft")
        res = ref_speculative_greedy(model, model, ids, ts, ds, k=k, max_new_tokens=20)
        check_trace(res, ts, ds, want)
        assert res.new_token_ids == fx["greedy"]["new_token_ids"]

    for k, want in zip((1, 3, 8), fx["spec_hostile"]):
        t, d = ref_pool(arch, dtype, 64, 4), ref_pool(arch, dtype, 64, 4)
        ts, ds = t.new_sequence("target"), d.new_sequence("draft")
        res = ref_speculative_greedy(model, hostile(model), ids, ts, ds, k=k, max_new_tokens=16)
        check_trace(res, ts, ds, want)

    want = fx["spec_oracle"]
    cont = [0] * ids.shape[1] + fx["greedy"]["new_token_ids"]
    oracle = OracleAcceptance(cont, want["p_accept"], want["seed"], arch.vocab)
    t, d = ref_pool(arch, dtype, 64, 4), ref_pool(arch, dtype, 64, 4)
    ts, ds = t.new_sequence("target"), d.new_sequence("draft")
    res = ref_speculative_greedy(model, model, ids, ts, ds, k=4, max_new_tokens=16,
                                 propose=oracle)
    check_trace(res, ts, ds, want)


@pytest.mark.slow
def test_c2_slice_oracle_acceptance_matches_reference():
    fx = load_json("c2_slice.json")
    tgt_arch, dr_arch = layer_slice(QWEN25_3B, 2), layer_slice(QWEN25_0_5B, 2)
    assert fx["target_arch"] == tgt_arch.name and fx["draft_arch"] == dr_arch.name
    sd_t = generate_state_dict(tgt_arch, seed=1, dtype=torch.float32)
    sd_d = generate_state_dict(dr_arch, seed=1, dtype=torch.float32)
    assert state_dict_checksum(sd_t) == fx["target_checksum"]
    target, draft = RefQwen2(tgt_arch, sd_t), RefQwen2(dr_arch, sd_d)
    ids = torch.tensor([fx["prompt"]])
    g = ref_greedy(target, ids, ref_pool(tgt_arch, torch.float32, 64, 16).new_sequence("r"), 24)
    assert g.new_token_ids == fx["greedy"]["new_token_ids"]
    want = fx["spec_oracle"]
    oracle = OracleAcceptance([0] * 64 + g.new_token_ids, 0.65, 7, tgt_arch.vocab)
    ts = ref_pool(tgt_arch, torch.float32, 64, 16).new_sequence("target")
    ds = ref_pool(dr_arch, torch.float32, 64, 16).new_sequence("draft")
    res = ref_speculative_greedy(target, draft, ids, ts, ds, k=4, max_new_tokens=24,
                                 propose=oracle)
    check_trace(res, ts, ds, want)
    assert res.new_token_ids == g.new_token_ids


@pytest.mark.slow
def test_c0_self_speculation_matches_reference():
    """0.5B arch fp32, self-draft k=4, 64 tokens, 100% accept."""
    fx = load_json("c0_spec.json")
    arch = QWEN25_0_5B
    sd = generate_state_dict(arch, seed=0, dtype=torch.float32)
    assert state_dict_checksum(sd) == fx["weights_checksum"]
    model = RefQwen2(arch, sd)
    ids = torch.tensor([fx["prompt"]])
    want = fx["spec_self"]
    ts = ref_pool(arch, torch.float32, 512, 16).new_sequence("target")
    ds = ref_pool(arch, torch.float32, 512, 16).new_sequence("draft")
    res = ref_speculative_greedy(model, model, ids, ts, ds, k=4, max_new_tokens=64)
    check_trace(res, ts, ds, want)
    assert res.new_token_ids == fx["greedy"]["new_token_ids"]
    assert res.acceptance_rate == 1.0


@pytest.mark.parametrize("name", ["attn_fp32.npz", "attn_bf16.npz", "attn_bf16_eager.npz"])
def test_gather_then_attend_matches_reference(name):
    fx = load_npz_tensors(name)
    out = gather_then_attend(fx["q"], fx["k_pool"], fx["v_pool"], fx["tables"], fx["ctx_lens"],
                             use_sdpa=fx["use_sdpa"])
    assert torch.equal(out, fx["out"])
    # and the restatement agrees with the float64 textbook definition
    ref64 = attend_fp64(fx["q"], fx["k_pool"], fx["v_pool"], fx["tables"], fx["ctx_lens"])
    tol = 1e-6 if fx["dtype"] == torch.float32 else 1e-2
    assert normalized_error(out, ref64) < tol


def test_tiny_arch_geometry():
    assert TINY.group == 7 and TINY.head_dim == 64
    assert QWEN25_3B.num_params() == 3_085_938_688
    assert QWEN25_0_5B.num_params() == 494_032_768
