"""Write golden fixtures by running the real reference (this container only).

The reference (siddharth-diwakar/kvengine, mounted read-only at /root/reference)
is pure Python over torch and transformers. Its composed numerics cannot be
pinned from closed forms, so this script imports it and records small
input/output vectors:

  tiny_fp32.json / tiny_bf16.json   2-layer GQA-7 model (TINY arch): greedy_paged
      tokens and per-step last-row logits, speculative_greedy traces (self
      draft, hostile draft, oracle-acceptance draft) with block tables after
      every rollback, both caches paged with block_size 4
  c0_spec.json   BASELINE config 0: Qwen2.5-0.5B architecture, fp32, seed 0,
      32-token random prompt, 64 greedy tokens, self-speculation k=4, paged
      block_size 16; per-step top-2 logit values/ids of the greedy run
  c2_slice.json  3B-architecture target and 0.5B-architecture draft cut to 2
      layers, fp32, seed 1, 64-token prompt, 24 tokens, k=4, oracle acceptance
      p=0.65 (seed 7) on the greedy continuation
  attn_{fp32,bf16}.npz   verify attention through the reference's
      PagedSequenceCache.write + attend: 4 sequences, 5 queries each,
      14 q / 2 kv heads, head_dim 64, block_size 16, fragmented block tables

Full-depth bf16 fixtures (Qwen2.5-3B-architecture target, Qwen2.5-0.5B-
architecture draft, seed 1; every greedy step records the emitted token and
the 8 largest logits with their ids, ordered by value then id):

  c2_full.json   single-sequence config: 64-token prompt (randint, seed 1),
      128 greedy steps of the target and of the draft, and speculative_greedy
      with k=4 and oracle acceptance p=0.65 (seed 1000) on the target's greedy
      continuation: tokens, accepted_per_iter, forward counts, the block
      tables after every rollback (paged, block_size 16)
  c3_full.json   the batched config's 32 requests (workloads.batched_spec_workload
      seed 0): each request's target greedy continuation over its whole output
      budget, and its speculative_greedy trace at k=4 with oracle acceptance
      p=0.65 (seed 1000 + request index)
  c4_full.json   the prefix-shared config: requests 0 and 1 of
      workloads.prefix_shared_workload (a 2048-token shared prefix + a
      256-token suffix each), 32 target greedy steps each
  c2_verify.json / c3_verify.json   teacher-forced verify passes of the
      target at the verify shape: prompt[:-1] prefilled, then windows of k+1 = 5
      tokens of the greedy continuation (prompt[-1], g0, g1, ...) fed with
      all_logits=True; the top entries of every row (row j predicts the token
      after window token j). The same positions as the greedy fixtures, through
      the reference's own verify-shaped pass.

Models are transformers' Qwen2ForCausalLM built from a local config (no
download) with kvengine_amd.weights' seeded state dict loaded into it.
Nothing here runs on the GPU box; the fixtures travel, the reference does not.

Usage: python tests/golden/make_golden.py [--skip-c0] [--only c2full,c3full,c4full,c2verify,c3verify]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
sys.path.insert(0, "/root/reference")

import kvengine as ref  # noqa: E402  (the reference package)
from kvengine import forward as ref_forward  # noqa: E402
from transformers import Qwen2Config, Qwen2ForCausalLM  # noqa: E402

from kvengine_amd.arch import QWEN25_0_5B, QWEN25_3B, TINY, layer_slice  # noqa: E402
from kvengine_amd.weights import generate_state_dict, state_dict_checksum  # noqa: E402
from kvengine_amd.workloads import OracleAcceptance  # noqa: E402


def hf_model(arch, sd, dtype):
    cfg = Qwen2Config(
        vocab_size=arch.vocab, hidden_size=arch.hidden, intermediate_size=arch.ffn,
        num_hidden_layers=arch.num_layers, num_attention_heads=arch.num_q_heads,
        num_key_value_heads=arch.num_kv_heads, rms_norm_eps=arch.rms_eps,
        rope_parameters={"rope_type": "default", "rope_theta": arch.rope_theta},
        tie_word_embeddings=True, use_sliding_window=False, eos_token_id=None,
        max_position_embeddings=32768,
    )
    cfg.head_dim = arch.head_dim
    m = Qwen2ForCausalLM(cfg)
    missing, unexpected = m.load_state_dict({k: v.to(torch.float32) for k, v in sd.items()},
                                            strict=False)
    assert set(missing) <= {"lm_head.weight"}, missing
    assert not unexpected, unexpected
    m.tie_weights()
    assert m.lm_head.weight.data_ptr() == m.model.embed_tokens.weight.data_ptr()
    # Cast parameters only: from_pretrained(dtype=...) also leaves the rotary
    # inv_freq buffer in float32 (it is built with an explicit float32 arange).
    for p in m.parameters():
        p.data = p.data.to(dtype)
    m.eval()
    assert m.model.rotary_emb.inv_freq.dtype == torch.float32
    m.generation_config.eos_token_id = None
    return m


class HostileDraft:
    """Rolls the vocabulary axis by one (tests/test_phase5.py:35-50)."""

    def __init__(self, base):
        self.model = base.model
        self.config = base.config
        self.generation_config = base.generation_config
        self._head = base.lm_head

    def lm_head(self, hidden):
        return self._head(hidden).roll(shifts=1, dims=-1)


class ForcedDraft:
    """Replaces the draft's proposal for the last row through the LM head.

    The reference's loop has no proposal hook, so oracle acceptance is injected
    where the proposal is read: after cache.commit, cache.length is the absolute
    position being predicted by the last row.
    """

    def __init__(self, base, propose, cache_ref):
        self.model = base.model
        self.config = base.config
        self.generation_config = base.generation_config
        self._head = base.lm_head
        self.propose = propose
        self.cache_ref = cache_ref

    def lm_head(self, hidden):
        logits = self._head(hidden)
        pos = self.cache_ref[0].length
        natural = int(torch.argmax(logits[0, -1]))
        tok = self.propose(pos, natural)
        logits = logits.clone()
        logits[0, -1, tok] = logits[0, -1].max() + 1.0
        return logits


def record_truncates():
    """Wrap PagedSequenceCache.truncate to log (request_id, n, blocks after)."""
    log = []
    orig = ref.PagedSequenceCache.truncate

    def wrapped(self, n):
        orig(self, n)
        log.append((str(self.request_id), int(n), list(self.blocks)))

    ref.PagedSequenceCache.truncate = wrapped
    return log, lambda: setattr(ref.PagedSequenceCache, "truncate", orig)


def spec_trace(target, draft, ids, pool_t, pool_d, k, max_new):
    log, undo = record_truncates()
    try:
        t_seq = pool_t.new_sequence("target")
        d_seq = pool_d.new_sequence("draft")
        if isinstance(draft, ForcedDraft):
            draft.cache_ref[0] = d_seq
        r = ref.speculative_greedy(target, draft, ids, t_seq, d_seq, k=k,
                                   max_new_tokens=max_new, eos_token_id=None)
    finally:
        undo()
    return {
        "k": k,
        "new_token_ids": r.new_token_ids,
        "accepted_per_iter": r.accepted_per_iter,
        "iterations": r.iterations,
        "tokens_drafted": r.tokens_drafted,
        "tokens_accepted": r.tokens_accepted,
        "target_forwards": r.target_forwards,
        "draft_forwards": r.draft_forwards,
        "truncate_log": log,
        "final_target_blocks": list(t_seq.blocks),
        "final_draft_blocks": list(d_seq.blocks),
        "target_len": t_seq.length,
        "draft_len": d_seq.length,
    }


def greedy_record(model, ids, pool, max_new, topk_only):
    g = ref.greedy_paged(model, ids, pool, max_new_tokens=max_new, eos_token_id=None,
                         collect_logits=True, free_on_finish=False)
    seq = g.sequence
    out = {"new_token_ids": g.new_token_ids, "blocks": list(seq.blocks)}
    top = torch.topk(g.step_logits, 2, dim=-1)
    out["top2_values"] = top.values.tolist()
    out["top2_ids"] = top.indices.tolist()
    if not topk_only:
        out["step_logits"] = g.step_logits.tolist()
    seq.free()
    return out


def hf_model_direct(arch, sd):
    """Qwen2ForCausalLM holding the given tensors as its parameters (no float32
    copy, no random init): built on the meta device, then assigned. The values
    are those of hf_model(arch, fp32 dict, dtype) when sd is that dict cast to
    dtype (generate_state_dict casts with round-to-nearest-even either way)."""
    cfg = Qwen2Config(
        vocab_size=arch.vocab, hidden_size=arch.hidden, intermediate_size=arch.ffn,
        num_hidden_layers=arch.num_layers, num_attention_heads=arch.num_q_heads,
        num_key_value_heads=arch.num_kv_heads, rms_norm_eps=arch.rms_eps,
        rope_parameters={"rope_type": "default", "rope_theta": arch.rope_theta},
        tie_word_embeddings=True, use_sliding_window=False, eos_token_id=None,
        max_position_embeddings=32768,
    )
    cfg.head_dim = arch.head_dim
    with torch.device("meta"):
        m = Qwen2ForCausalLM(cfg)
    missing, unexpected = m.load_state_dict(sd, strict=False, assign=True)
    assert set(missing) <= {"lm_head.weight"}, missing
    assert not unexpected, unexpected
    m.tie_weights()
    assert m.lm_head.weight.data_ptr() == m.model.embed_tokens.weight.data_ptr()
    # the rotary buffer is computed at construction: rebuild it on the CPU (float32)
    m.model.rotary_emb = type(m.model.rotary_emb)(config=cfg)
    assert m.model.rotary_emb.inv_freq.dtype == torch.float32
    for name, t in list(m.named_parameters()) + list(m.named_buffers()):
        assert t.device.type == "cpu", name
    m.eval()
    m.generation_config.eos_token_id = None
    return m


TOPN = 8


def top_entries(logits: torch.Tensor, n: int = TOPN):
    """The n largest entries of each row as (values, ids), ordered by value
    (descending) then id (ascending), so equal logits list the lowest id first
    (torch.argmax picks it)."""
    vals, ids = torch.topk(logits.float(), 2 * n, dim=-1)
    out_v, out_i = [], []
    for v, i in zip(vals.tolist(), ids.tolist()):
        pairs = sorted(zip(v, i), key=lambda p: (-p[0], p[1]))[:n]
        out_v.append([p[0] for p in pairs])
        out_i.append([p[1] for p in pairs])
    return out_v, out_i


def greedy_top(model, ids, pool, max_new):
    """Reference greedy_paged with the top entries of every step's logits."""
    g = ref.greedy_paged(model, ids, pool, max_new_tokens=max_new, eos_token_id=None,
                         collect_logits=True)
    v, i = top_entries(g.step_logits)
    assert [row[0] for row in i] == g.new_token_ids
    return {"new_token_ids": g.new_token_ids, "top_values": v, "top_ids": i}


def full_models():
    from kvengine_amd.arch import QWEN25_0_5B as D, QWEN25_3B as T
    t = time.time()
    sd_t = generate_state_dict(T, seed=1, dtype=torch.bfloat16)
    sd_d = generate_state_dict(D, seed=1, dtype=torch.bfloat16)
    meta = {"target_arch": T.name, "draft_arch": D.name, "weight_seed": 1,
            "dtype": "torch.bfloat16", "target_checksum": state_dict_checksum(sd_t),
            "draft_checksum": state_dict_checksum(sd_d)}
    target, draft = hf_model_direct(T, sd_t), hf_model_direct(D, sd_d)
    print(f"full-depth models built in {time.time() - t:.1f}s", flush=True)
    return target, draft, meta


def spec_oracle_trace(target, draft, prompt, cont, seed, k, max_new, blocks):
    oracle = OracleAcceptance([0] * len(prompt) + cont, 0.65, seed=seed, vocab=target.config.vocab_size)
    fd = ForcedDraft(draft, oracle, [None])
    mk_t = lambda: ref.PagedKVCache.for_model(target, num_blocks=blocks, block_size=16)  # noqa: E731
    mk_d = lambda: ref.PagedKVCache.for_model(draft, num_blocks=blocks, block_size=16)  # noqa: E731
    tr = spec_trace(target, fd, torch.tensor([prompt]), mk_t(), mk_d(), k, max_new)
    tr.update({"p_accept": 0.65, "seed": seed})
    return tr


def c2_full_fixture(path):
    target, draft, fx = full_models()
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, target.config.vocab_size, (1, 64), generator=g)
    fx["prompt"] = ids[0].tolist()
    mk = lambda m: ref.PagedKVCache.for_model(m, num_blocks=64, block_size=16)  # noqa: E731
    t = time.time()
    fx["target_greedy"] = greedy_top(target, ids, mk(target), 128)
    fx["draft_greedy"] = greedy_top(draft, ids, mk(draft), 128)
    print(f"c2 greedy done in {time.time() - t:.1f}s", flush=True)
    cont = fx["target_greedy"]["new_token_ids"]
    fx["spec_oracle"] = spec_oracle_trace(target, draft, fx["prompt"], cont, 1000, 4, 128, 64)
    fx["spec_oracle"]["equals_greedy"] = fx["spec_oracle"]["new_token_ids"] == cont
    with open(path, "w") as f:
        json.dump(fx, f, separators=(",", ":"))


def c3_full_fixture(path):
    from kvengine_amd.workloads import batched_spec_workload

    target, draft, fx = full_models()
    work = batched_spec_workload(seed=0, n=32, vocab=target.config.vocab_size)
    fx["workload"] = "batched_spec_workload(seed=0, n=32)"
    fx["k"] = 4
    reqs = []
    for i, (prompt, budget) in enumerate(work):
        t = time.time()
        blocks = -(-(len(prompt) + budget + 16) // 16) + 2
        ids = torch.tensor([prompt])
        gr = greedy_top(target, ids, ref.PagedKVCache.for_model(target, num_blocks=blocks,
                                                                 block_size=16), budget)
        tr = spec_oracle_trace(target, draft, prompt, gr["new_token_ids"], 1000 + i, 4, budget, blocks)
        reqs.append({"index": i, "prompt_len": len(prompt), "max_new_tokens": budget,
                     "prompt_head": prompt[:8], "greedy": gr,
                     "spec_oracle": {key: tr[key] for key in (
                         "new_token_ids", "accepted_per_iter", "iterations", "target_forwards",
                         "draft_forwards", "seed", "p_accept")}})
        reqs[-1]["spec_oracle"]["equals_greedy"] = tr["new_token_ids"] == gr["new_token_ids"]
        print(f"c3 request {i}: prompt {len(prompt)}, {budget} tokens, "
              f"{time.time() - t:.1f}s", flush=True)
    fx["requests"] = reqs
    with open(path, "w") as f:
        json.dump(fx, f, separators=(",", ":"))


def c4_full_fixture(path):
    from kvengine_amd.workloads import prefix_shared_workload

    target, _, fx = full_models()
    work = prefix_shared_workload(seed=0, vocab=target.config.vocab_size)
    fx["workload"] = "prefix_shared_workload(seed=0)"
    reqs = []
    for i in (0, 1):
        prompt = work[i][0]
        ids = torch.tensor([prompt])
        gr = greedy_top(target, ids, ref.PagedKVCache.for_model(target, num_blocks=168,
                                                                 block_size=16), 32)
        reqs.append({"index": i, "prompt_len": len(prompt), "prompt_head": prompt[:8],
                     "greedy": gr})
        print(f"c4 request {i} done", flush=True)
    fx["requests"] = reqs
    with open(path, "w") as f:
        json.dump(fx, f, separators=(",", ":"))


def verify_windows(model, prompt, cont, window, blocks):
    """Reference forward over prompt + cont in verify-shaped passes (see the
    module docstring); top entries of the rows predicting cont[0..]."""
    pool = ref.PagedKVCache.for_model(model, num_blocks=blocks, block_size=16)
    seq = pool.new_sequence("windows")
    ref_forward.forward_with_own_cache(model, torch.tensor([prompt[:-1]]), seq)
    toks = prompt[-1:] + cont[:-1]
    vals, ids = [], []
    for w in range(0, len(toks), window):
        logits = ref_forward.forward_with_own_cache(model, torch.tensor([toks[w:w + window]]), seq,
                                                    all_logits=True)[0]
        v, i = top_entries(logits)
        vals.extend(v)
        ids.extend(i)
    seq.free()
    return {"window": window, "top_values": vals, "top_ids": ids}


def c2_verify_fixture(path):
    target, _, fx = full_models()
    c2 = json.load(open(os.path.join(HERE, "c2_full.json")))
    fx["prompt"] = c2["prompt"]
    cont = c2["target_greedy"]["new_token_ids"]
    fx["target"] = verify_windows(target, c2["prompt"], cont, 5, 64)
    with open(path, "w") as f:
        json.dump(fx, f, separators=(",", ":"))


def c3_verify_fixture(path):
    from kvengine_amd.workloads import batched_spec_workload

    target, _, fx = full_models()
    c3 = json.load(open(os.path.join(HERE, "c3_full.json")))
    work = batched_spec_workload(seed=0, n=32, vocab=target.config.vocab_size)
    reqs = []
    for r in c3["requests"]:
        prompt, budget = work[r["index"]]
        cont = r["greedy"]["new_token_ids"]
        blocks = -(-(len(prompt) + budget + 16) // 16) + 2
        w = verify_windows(target, prompt, cont, 5, blocks)
        w["index"] = r["index"]
        reqs.append(w)
        print(f"c3 verify windows {r['index']} done", flush=True)
    fx["requests"] = reqs
    with open(path, "w") as f:
        json.dump(fx, f, separators=(",", ":"))


def tiny_fixture(dtype, path):
    arch = TINY
    sd = generate_state_dict(arch, seed=3, dtype=torch.float32)
    model = hf_model(arch, sd, dtype)
    g = torch.Generator().manual_seed(11)
    ids = torch.randint(0, arch.vocab, (1, 12), generator=g)
    mk = lambda: ref.PagedKVCache.for_model(model, num_blocks=64, block_size=4)  # noqa: E731
    fx = {"arch": arch.name, "weight_seed": 3, "dtype": str(dtype),
          "weights_checksum": state_dict_checksum(sd), "prompt": ids[0].tolist()}
    fx["greedy"] = greedy_record(model, ids, mk(), 20, topk_only=False)
    fx["spec_self"] = [spec_trace(model, model, ids, mk(), mk(), k, 20) for k in (1, 2, 4, 8)]
    fx["spec_hostile"] = [spec_trace(model, HostileDraft(model), ids, mk(), mk(), k, 16)
                          for k in (1, 3, 8)]
    cont = fx["greedy"]["new_token_ids"]
    full = ids[0].tolist() + cont
    oracle = OracleAcceptance([0] * ids.shape[1] + cont, 0.65, seed=7, vocab=arch.vocab)
    assert full[ids.shape[1]:] == cont
    fd = ForcedDraft(model, oracle, [None])
    fx["spec_oracle"] = spec_trace(model, fd, ids, mk(), mk(), 4, 16)
    fx["spec_oracle"]["p_accept"] = 0.65
    fx["spec_oracle"]["seed"] = 7
    with open(path, "w") as f:
        json.dump(fx, f)


def c0_fixture(path):
    arch = QWEN25_0_5B
    t = time.time()
    sd = generate_state_dict(arch, seed=0, dtype=torch.float32)
    model = hf_model(arch, sd, torch.float32)
    print(f"c0 model built in {time.time() - t:.1f}s", flush=True)
    g = torch.Generator().manual_seed(0)
    ids = torch.randint(0, arch.vocab, (1, 32), generator=g)
    mk = lambda: ref.PagedKVCache.for_model(model, num_blocks=512, block_size=16)  # noqa: E731
    fx = {"arch": arch.name, "weight_seed": 0, "dtype": "torch.float32",
          "weights_checksum": state_dict_checksum(sd), "prompt": ids[0].tolist()}
    fx["greedy"] = greedy_record(model, ids, mk(), 64, topk_only=True)
    print("c0 greedy done", flush=True)
    fx["spec_self"] = spec_trace(model, model, ids, mk(), mk(), 4, 64)
    with open(path, "w") as f:
        json.dump(fx, f)


def c2_slice_fixture(path):
    tgt_arch = layer_slice(QWEN25_3B, 2)
    dr_arch = layer_slice(QWEN25_0_5B, 2)
    sd_t = generate_state_dict(tgt_arch, seed=1, dtype=torch.float32)
    sd_d = generate_state_dict(dr_arch, seed=1, dtype=torch.float32)
    target = hf_model(tgt_arch, sd_t, torch.float32)
    draft = hf_model(dr_arch, sd_d, torch.float32)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, tgt_arch.vocab, (1, 64), generator=g)
    mk_t = lambda: ref.PagedKVCache.for_model(target, num_blocks=64, block_size=16)  # noqa: E731
    mk_d = lambda: ref.PagedKVCache.for_model(draft, num_blocks=64, block_size=16)  # noqa: E731
    fx = {"target_arch": tgt_arch.name, "draft_arch": dr_arch.name, "weight_seed": 1,
          "dtype": "torch.float32", "target_checksum": state_dict_checksum(sd_t),
          "draft_checksum": state_dict_checksum(sd_d), "prompt": ids[0].tolist()}
    fx["greedy"] = greedy_record(target, ids, mk_t(), 24, topk_only=True)
    cont = fx["greedy"]["new_token_ids"]
    oracle = OracleAcceptance([0] * ids.shape[1] + cont, 0.65, seed=7, vocab=tgt_arch.vocab)
    fd = ForcedDraft(draft, oracle, [None])
    fx["spec_oracle"] = spec_trace(target, fd, ids, mk_t(), mk_d(), 4, 24)
    fx["spec_oracle"].update({"p_accept": 0.65, "seed": 7})
    with open(path, "w") as f:
        json.dump(fx, f)


class _AttnModule:
    def __init__(self, groups, scaling):
        self.num_key_value_groups = groups
        self.scaling = scaling


def attn_fixture(dtype, path, use_sdpa=True):
    """Reference write+gather+attend for one layer over 4 sequences."""
    Hq, Hkv, D, bs, T = 14, 2, 64, 16, 5
    g = torch.Generator().manual_seed(5)
    ctx = [37, 64, 131, 200]
    nb = 40
    # Fragment the LIFO stack with a seeded permutation so tables are scattered.
    pool = ref.PagedKVCache(1, Hkv, D, nb, bs, dtype, "cpu")
    order = torch.randperm(nb, generator=g).tolist()
    held = pool.manager.allocate(nb, owner="frag")
    pool.manager.free([held[i] for i in order])
    seqs, qs, outs, tables = [], [], [], []
    hist_k, hist_v, new_k, new_v = [], [], [], []
    for L in ctx:
        s = pool.new_sequence(f"s{L}")
        kh = torch.randn(1, Hkv, L - T, D, generator=g).to(dtype)
        vh = torch.randn(1, Hkv, L - T, D, generator=g).to(dtype)
        s.reserve(L - T)
        s.write(0, kh, vh, 0)
        s.commit(L - T)
        kn = torch.randn(1, Hkv, T, D, generator=g).to(dtype)
        vn = torch.randn(1, Hkv, T, D, generator=g).to(dtype)
        q = torch.randn(1, T, Hq, D, generator=g).to(dtype)
        s.reserve(T)
        k_all, v_all = s.write(0, kn, vn, L - T)
        s.commit(T)
        mask = ref_forward.causal_mask(T, L, dtype, torch.device("cpu"))
        out = ref_forward.attend(_AttnModule(Hq // Hkv, D ** -0.5), q.transpose(1, 2),
                                 k_all, v_all, mask, use_sdpa=use_sdpa)
        seqs.append(s)
        qs.append(q[0])
        outs.append(out[0])
        tables.append(list(s.blocks))
        hist_k.append(kh)
        hist_v.append(vh)
        new_k.append(kn)
        new_v.append(vn)

    def arr(t):
        t = t.contiguous()
        return t.view(torch.int16).numpy() if t.dtype == torch.bfloat16 else t.numpy()

    maxb = max(len(t) for t in tables)
    tab = np.full((len(ctx), maxb), -1, dtype=np.int32)
    for i, t in enumerate(tables):
        tab[i, : len(t)] = t
    np.savez_compressed(
        path, dtype=str(dtype), ctx_lens=np.array(ctx, dtype=np.int32), tables=tab,
        q=arr(torch.stack(qs)), out=arr(torch.stack(outs)),
        k_pool=arr(pool.k[0]), v_pool=arr(pool.v[0]), block_size=bs, q_len=T,
        use_sdpa=use_sdpa,
    )


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--skip-c0", action="store_true")
    ap.add_argument("--only", default="")
    a = ap.parse_args()
    torch.set_num_threads(os.cpu_count() or 1)
    jobs = {
        "attn": lambda: (attn_fixture(torch.float32, os.path.join(HERE, "attn_fp32.npz")),
                         attn_fixture(torch.bfloat16, os.path.join(HERE, "attn_bf16.npz")),
                         attn_fixture(torch.bfloat16, os.path.join(HERE, "attn_bf16_eager.npz"),
                                      use_sdpa=False)),
        "tiny": lambda: (tiny_fixture(torch.float32, os.path.join(HERE, "tiny_fp32.json")),
                         tiny_fixture(torch.bfloat16, os.path.join(HERE, "tiny_bf16.json"))),
        "c2": lambda: c2_slice_fixture(os.path.join(HERE, "c2_slice.json")),
        "c0": lambda: c0_fixture(os.path.join(HERE, "c0_spec.json")),
        "c2full": lambda: c2_full_fixture(os.path.join(HERE, "c2_full.json")),
        "c3full": lambda: c3_full_fixture(os.path.join(HERE, "c3_full.json")),
        "c4full": lambda: c4_full_fixture(os.path.join(HERE, "c4_full.json")),
        "c2verify": lambda: c2_verify_fixture(os.path.join(HERE, "c2_verify.json")),
        "c3verify": lambda: c3_verify_fixture(os.path.join(HERE, "c3_verify.json")),
    }
    full = {"c2full", "c3full", "c4full", "c2verify", "c3verify"}
    for name, job in jobs.items():
        if a.only and name not in a.only.split(","):
            continue
        if name == "c0" and a.skip_c0:
            continue
        if name in full and not a.only:
            continue  # full-depth jobs run only when named (--only c2full,...)
        t = time.time()
        job()
        print(f"{name}: {time.time() - t:.1f}s", flush=True)


if __name__ == "__main__":
    main()
