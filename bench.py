#!/usr/bin/env python3
"""Benchmark of the speculative-decoding verify path on one MI355X.

value: whole-job output tokens/s of batched greedy speculative decoding,
    Qwen2.5-3B-architecture target + Qwen2.5-0.5B-architecture draft (bf16,
    seeded random weights), 32 requests arriving at once with lognormal prompt
    (median 128, 16-1024) and output (median 64, 8-512) lengths, k=4, oracle
    acceptance p=0.65 against the target's own greedy continuation, block size
    16, KV pools sized to --pool-frac of the most blocks the workload holds at
    once (measured in an unconstrained run), so the scheduler preempts and
    recomputes. A step is one full run of the workload (prefill included).
roofline: the paged verify-attention kernel on the verify microbench
    (32 sequences, lognormal(512, 0.8) contexts in [64, 4096], 5 queries,
    14/2 heads, head_dim 64, bf16), pools rotated over > 2x the 256 MB
    Infinity Cache; algorithmic bytes / average launch time from HIP events.
    Long-context rows beside it: 32 x 4096 tokens and 16 x 8192 tokens sharing
    a 2048-token prefix.
parity_vs_reference: the GPU's greedy continuations against the reference's
    own (tests/golden/c3_full.json): identical requests, and where one parts,
    the reference's top-2 margin there.
cpu_baseline: the CPU oracle of the reference's loop (per-request
    speculative_greedy, bf16) on the same models, on every CPU this process may
    use, time-bounded; with a teacher-forced parity check of the GPU's tokens.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--k 4]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

METRIC = "spec-decode tok/s (3B target, 0.5B draft, k=4, bs=32); verify-attn HBM GB/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--k", type=int, default=4)
    ap.add_argument("--p-accept", type=float, default=0.65)
    ap.add_argument("--slots", type=int, default=32)
    ap.add_argument("--pool-frac", type=float, default=0.8)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--attn-launches", type=int, default=400)
    ap.add_argument("--attn-units", type=int, default=0,
                    help="verify attention unit size in blocks (0: chosen per launch)")
    ap.add_argument("--attn-waves", type=int, default=0,
                    help="verify attention key waves (0: chosen per launch)")
    ap.add_argument("--skip-spec", action="store_true", help="kernel microbenches only")
    ap.add_argument("--skip-micro", action="store_true", help="no kernel microbenches")
    ap.add_argument("--mode", default="c3", choices=["c3", "c2", "ksweep", "c4", "forward"],
                    help="c3: the batched headline run (default). c2: one request, 64-token "
                         "prompt, 128 tokens. ksweep: the batched run for k in 1,2,4,8. c4: 16 "
                         "requests sharing a 2048-token prefix, k=8, p=0.5, decoding "
                         "--c4-new tokens each (to 8192-token contexts) and verify attention "
                         "at 2-8k shared contexts. forward: one model's forward pass at the "
                         "engine's shapes (--fwd-*), replayed as a HIP graph (for kernel "
                         "traces and counter passes)")
    ap.add_argument("--fwd-model", default="draft", choices=["draft", "target"])
    ap.add_argument("--fwd-seqs", type=int, default=32)
    ap.add_argument("--fwd-q", type=int, default=1, help="tokens per sequence")
    ap.add_argument("--fwd-ctx", type=int, default=600, help="history length of every sequence")
    ap.add_argument("--fwd-reps", type=int, default=20)
    ap.add_argument("--fwd-api", action="store_true",
                    help="forward mode: the layer and attention order speculative_greedy and "
                         "greedy_decode take (no gemm_rows) instead of the batched engine's")
    ap.add_argument("--c4-new", type=int, default=5888)
    ap.add_argument("--attn-only", action="store_true",
                    help="only the verify-attention microbench (for counter passes)")
    ap.add_argument("--attn-large", default="", choices=["", "32x4096", "16x8192"],
                    help="only one long-context verify-attention case (for counter passes): "
                         "32 x 4096 tokens (14/2 heads, D=64, q_len 5) or 16 x 8192 tokens "
                         "sharing 2048 (16/2 heads, D=128, q_len 9)")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MB",
                    help="only copy MB megabytes device-to-device 20 times: the known-size "
                         "transfer that scales FETCH_SIZE / WRITE_SIZE counter readings")
    return ap.parse_args()


def copy_calibration(mb: int) -> dict:
    n = mb * 2**20 // 4
    src = torch.randn(n, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(20):
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"copy_bytes": n * 4, "copies": 20}


# ---------------------------------------------------------------- microbenches

def time_launches(fn, n: int, warm: int = 10):
    """Average per-launch time (us) two ways: an event pair around every launch,
    and one event pair around a HIP graph replaying n launches."""
    for i in range(warm):
        fn(i)
    torch.cuda.synchronize()
    st = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    en = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    for i in range(n):
        st[i].record()
        fn(i)
        en[i].record()
    torch.cuda.synchronize()
    per = [a.elapsed_time(b) * 1e3 for a, b in zip(st, en)]
    per.sort()
    ev_mean = sum(per) / n
    ev_median = per[n // 2]
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(0)
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(g):
        for i in range(n):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 3
    a.record()
    for _ in range(reps):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    graph_us = a.elapsed_time(b) * 1e3 / (reps * n)
    return {"event_mean_us": ev_mean, "event_median_us": ev_median, "graph_us": graph_us}


def attn_timings(q, ks, vs, tab, start, max_ctx, unit_blocks, key_waves, launches, out):
    """Per-launch times of one layer's verify attention over rotated pools:
    with a work plan built once per pass (kve_attn_plan, shared by every layer
    of a forward pass; `graph_us`), the plan kernel alone (`plan_us`), and a
    launch that builds its own plan (`standalone_us`)."""
    from kvengine_amd import kernels

    copies = len(ks)
    B, T, Hq, D = q.shape
    _, Hkv, bs, _ = ks[0].shape
    NB = ks[0].shape[0]

    def plan():
        return kernels.attn_plan(tab, start, B, T, Hq, Hkv, D, bs, NB, max_ctx, q.dtype,
                                 unit_blocks=unit_blocks, key_waves=key_waves)

    p = plan()

    def launch(i):
        c = i % copies
        kernels.paged_verify_attn(q, ks[c], vs[c], tab, start, max_ctx, out=out,
                                  unit_blocks=unit_blocks, key_waves=key_waves, plan=p)

    t = time_launches(launch, launches)
    tp = time_launches(lambda i: plan(), 200, warm=5)
    p = plan()

    def standalone(i):
        c = i % copies
        kernels.paged_verify_attn(q, ks[c], vs[c], tab, start, max_ctx, out=out,
                                  unit_blocks=unit_blocks, key_waves=key_waves)

    ts = time_launches(standalone, launches)
    return {**{k: round(v, 3) for k, v in t.items()}, "plan_us": round(tp["graph_us"], 3),
            "standalone_us": round(ts["graph_us"], 3)}


def verify_attn_microbench(n_launch: int, unit_blocks: int, key_waves: int) -> dict:
    from kvengine_amd.layout import to_kernel_layout
    from kvengine_amd.workloads import verify_attn_case

    case = verify_attn_case(seed=0, dtype=torch.bfloat16)
    k_l, v_l = to_kernel_layout(case.pool[0], case.pool[1])
    copy_bytes = (k_l.numel() + v_l.numel()) * 2
    copies = max(2, math.ceil(2.2 * 256 * 2**20 / copy_bytes))
    ks = [k_l.to("cuda") for _ in range(copies)]
    vs = [v_l.to("cuda") for _ in range(copies)]
    B = len(case.ctx_lens)
    width = max(len(t) for t in case.tables)
    tab = torch.full((B, width), -1, dtype=torch.int32)
    for i, t in enumerate(case.tables):
        tab[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
    tab = tab.cuda()
    T = case.q.shape[1]
    start = torch.tensor([L - T for L in case.ctx_lens], dtype=torch.int32, device="cuda")
    q = case.q.cuda()
    out = torch.empty_like(q)
    t = attn_timings(q, ks, vs, tab, start, max(case.ctx_lens), unit_blocks, key_waves, n_launch,
                     out)
    nbytes = case.algorithmic_bytes()
    res = {
        "workload": "32 seqs, ctx lognormal(median 512, sigma 0.8) in [64,4096], T=5, "
                    "14/2 heads, D=64, bf16, block 16",
        "ctx_tokens": sum(case.ctx_lens),
        "max_ctx": max(case.ctx_lens),
        "algorithmic_bytes": nbytes,
        "pool_copies": copies,
        "rotated_bytes": copies * copy_bytes,
        "unit_blocks": unit_blocks,
        "key_waves": key_waves,
        **t,
    }
    for key in ("event_mean_us", "graph_us", "standalone_us"):
        res[key.replace("_us", "_gbs")] = round(nbytes / (t[key] * 1e-6) / 1e9, 1)
    return res


def attn_case(B: int, L: int, Hq: int, Hkv: int, D: int, T: int, shared: int,
              unit_blocks: int = 0, key_waves: int = 0, launches: int = 100) -> dict:
    """Verify attention over B sequences of L tokens (q_len T, heads Hq/Hkv,
    head_dim D, bf16) whose first `shared` blocks are the same physical blocks;
    block ids scattered by a seeded permutation, pools rotated past the 256 MB
    Infinity Cache. Bytes: K/V read once per sequence (logical) and once per
    distinct block (unique), plus Q and O."""
    nb_seq = -(-L // 16)
    NB = shared + B * (nb_seq - shared)
    g = torch.Generator(device="cuda").manual_seed(5)
    pool_bytes = NB * Hkv * 16 * D * 2 * 2
    copies = max(2, math.ceil(2.2 * 256 * 2**20 / pool_bytes))
    kps = [torch.randn(NB, Hkv, 16, D, device="cuda", generator=g).to(torch.bfloat16)
           for _ in range(copies)]
    vps = [torch.randn(NB, Hkv, D, 16, device="cuda", generator=g).to(torch.bfloat16)
           for _ in range(copies)]
    tab = torch.empty(B, nb_seq, dtype=torch.int32)
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(6))
    for s_ in range(B):
        tab[s_, :shared] = perm[:shared]
        tab[s_, shared:] = perm[shared + s_ * (nb_seq - shared):shared + (s_ + 1) * (nb_seq - shared)]
    tab = tab.cuda()
    q = torch.randn(B, T, Hq, D, device="cuda", generator=g).to(torch.bfloat16)
    start = torch.full((B,), L - T, dtype=torch.int32, device="cuda")
    o = torch.empty_like(q)
    t = attn_timings(q, kps, vps, tab, start, L, unit_blocks, key_waves, launches, o)
    tok_bytes = Hkv * D * 2 * 2
    qo = 2 * B * T * Hq * D * 2
    logical = B * L * tok_bytes + qo
    unique = (shared * 16 + B * (L - shared * 16)) * tok_bytes + qo
    us = t["graph_us"]
    return {"workload": f"{B} x {L} tokens ({shared * 16} shared), q_len {T}, heads {Hq}/{Hkv}, "
                        f"D={D}, bf16",
            "unit_blocks": unit_blocks, "key_waves": key_waves,
            "graph_us": round(us, 2), "event_mean_us": round(t["event_mean_us"], 2),
            "plan_us": t["plan_us"], "standalone_us": t["standalone_us"],
            "logical_bytes": logical, "unique_bytes": unique,
            "logical_gbs": round(logical / (us * 1e-6) / 1e9, 1),
            "unique_gbs": round(unique / (us * 1e-6) / 1e9, 1),
            "unique_frac_of_peak": round(unique / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "pool_copies": copies}


def verify_attn_large(unit_blocks: int, key_waves: int) -> dict:
    """Verify attention at long contexts: 32 sequences of 4096 tokens with the
    verify microbench's heads (14/2, D=64, q_len 5), and the prefix-shared
    configuration's last verify (16 sequences at 8192 tokens sharing a 2048-token
    prefix, 3B heads 16/2, D=128, q_len 9)."""
    return {"32x4096": attn_case(32, 4096, 14, 2, 64, 5, 0, unit_blocks, key_waves),
            "16x8192_shared_2048": attn_case(16, 8192, 16, 2, 128, 9, 128, unit_blocks, key_waves)}


def lmhead_microbench(weight: torch.Tensor, M: int, weight_blk: torch.Tensor | None = None) -> dict:
    """The target's LM head + argmax over M rows: blocked operands (what the
    engine's verify pass runs) when weight_blk is given, row-major beside it."""
    from kvengine_amd import kernels

    V, H = weight.shape
    hs = [torch.randn(M, H, device="cuda", dtype=weight.dtype) for _ in range(4)]
    hbs = [kernels.to_blocked(h) for h in hs]
    am = torch.empty(M, dtype=torch.int32, device="cuda")

    def launch_rows(i):
        kernels.lmhead_argmax(hs[i % 4], weight, argmax=am)

    def launch_blk(i):
        kernels.lmhead_argmax(hbs[i % 4], weight_blk, argmax=am, blocked=True, rows=M)

    nbytes = V * H * 2 + M * H * 2 + M * 4
    flops = 2 * M * H * V
    t_rows = time_launches(launch_rows, 30, warm=3)
    t = time_launches(launch_blk, 30, warm=3) if weight_blk is not None else t_rows
    us = t["event_mean_us"]
    return {
        "workload": f"M={M} rows x H={H} x V={V} bf16 (3B verify rows at B=32, k=4)",
        "layout": "blocked" if weight_blk is not None else "rows",
        "algorithmic_bytes": nbytes,
        "flops": flops,
        **{k: round(v, 2) for k, v in t.items()},
        "hbm_gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
        "tflops": round(flops / (us * 1e-6) / 1e12, 1),
        "row_major_graph_us": round(t_rows["graph_us"], 2),
    }


# ---------------------------------------------------------------- main

def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the verify path is built and measured on a single MI355X)", file=sys.stderr)
        sys.exit(2)
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    from kvengine_amd import _lib
    from kvengine_amd.arch import QWEN25_0_5B, QWEN25_3B
    from kvengine_amd.engine import SpecEngine, SpecRequest
    from kvengine_amd.model import build_model, lm_head_blocked
    from kvengine_amd.weights import generate_state_dict
    from kvengine_amd.workloads import OracleAcceptance, batched_spec_workload

    _lib.lib()
    torch.backends.cuda.matmul.allow_tf32 = False
    k = args.k
    out: dict = {}
    if args.copy_calib:
        print(json.dumps(copy_calibration(args.copy_calib)), flush=True)
        return
    if args.attn_only:
        print(json.dumps(verify_attn_microbench(args.attn_launches, args.attn_units, args.attn_waves)), flush=True)
        return
    if args.attn_large:
        shape = {"32x4096": (32, 4096, 14, 2, 64, 5, 0), "16x8192": (16, 8192, 16, 2, 128, 9, 128)}
        print(json.dumps(attn_case(*shape[args.attn_large], args.attn_units, args.attn_waves,
                                   launches=args.attn_launches)), flush=True)
        return
    if args.mode != "c3":
        print(json.dumps(MODES[args.mode](args)), flush=True)
        return

    attn = {"event_mean_us": float("nan"), "event_mean_gbs": float("nan"),
            "graph_us": float("nan"), "graph_gbs": float("nan")}
    attn_large = {}
    if not args.skip_micro:
        log("verify-attention microbench")
        attn = verify_attn_microbench(args.attn_launches, args.attn_units, args.attn_waves)
        log(f"verify-attn: {attn}")
        attn_large = verify_attn_large(args.attn_units, args.attn_waves)
        log(f"verify-attn, long contexts: {attn_large}")

    t_arch, d_arch = QWEN25_3B, QWEN25_0_5B
    t0 = time.time()
    sd_t = generate_state_dict(t_arch, seed=args.seed, dtype=torch.bfloat16)
    sd_d = generate_state_dict(d_arch, seed=args.seed, dtype=torch.bfloat16)
    target = build_model(t_arch, sd_t, dtype=torch.bfloat16, device="cuda")
    draft = build_model(d_arch, sd_d, dtype=torch.bfloat16, device="cuda")
    log(f"models built in {time.time() - t0:.1f}s")

    lm = {}
    if not args.skip_micro:
        lm = lmhead_microbench(target.lm_head.weight, args.slots * (k + 1), lm_head_blocked(target))
        log(f"lm-head: {lm}")

    work = batched_spec_workload(seed=0, n=args.slots, vocab=t_arch.vocab)
    bs = 16
    max_ctx = -(-(max(len(p) + o for p, o in work) + k + 2) // 64) * 64
    roomy = 2 * sum(-(-(len(p) + o + k + 1) // bs) for p, o in work)

    spec, conts, parity = {}, None, None
    if not args.skip_spec:
        # 1. the target's greedy continuation, through the engine with the real draft
        #    (unconstrained pools), then its parity with the reference's continuation
        eng = SpecEngine(target, draft, k=k, slots=args.slots, t_blocks=roomy, d_blocks=roomy,
                         block_size=bs, max_ctx=max_ctx)
        t0 = time.time()
        base = [SpecRequest(i, p, o) for i, (p, o) in enumerate(work)]
        st0 = eng.run(base)
        conts = [r.new_token_ids for r in base]
        log(f"continuation run (draft model proposals): {st0.output_tokens} tokens, "
            f"{st0.tokens_per_s:.1f} tok/s, acceptance {st0.acceptance_rate:.3f}, "
            f"{time.time() - t0:.1f}s")
        parity = reference_parity(conts)
        log(f"parity with the reference: {parity}")

        def fresh():
            return [SpecRequest(i, p, o, propose=OracleAcceptance(
                [0] * len(p) + conts[i], args.p_accept, seed=1000 + i, vocab=t_arch.vocab))
                for i, (p, o) in enumerate(work)]

        # 2. the most blocks the timed workload holds at once (unconstrained pools)
        eng.reset_stats()
        eng.run(fresh())
        peak = max(eng.stats.peak_target_blocks, eng.stats.peak_draft_blocks)
        pool_blocks = max(math.ceil(args.pool_frac * peak),
                          max(-(-(len(p) + k + 1) // bs) for p, _ in work))
        log(f"concurrent peak {eng.stats.peak_target_blocks} target / "
            f"{eng.stats.peak_draft_blocks} draft blocks; pools of {pool_blocks}")
        del eng
        # 3. timed runs with both pools at pool_frac of that peak (preemption and recompute)
        eng = SpecEngine(target, draft, k=k, slots=args.slots, t_blocks=pool_blocks,
                         d_blocks=pool_blocks, block_size=bs, max_ctx=max_ctx)
        for w in range(args.warmup):
            eng.reset_stats()
            eng.run(fresh())
            log(f"warmup {w}: {eng.stats.tokens_per_s:.1f} tok/s, "
                f"{eng.stats.preemptions} preemptions")
        total_tokens = 0
        iters = drafted = accepted = preempt = recomputed = aborted = 0
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        runs = []
        for s_ in range(args.steps):
            eng.reset_stats()
            reqs = fresh()
            st = eng.run(reqs)
            total_tokens += st.output_tokens
            iters += st.iterations
            drafted += st.drafted
            accepted += st.accepted
            preempt += st.preemptions
            recomputed += st.recomputed_tokens
            aborted += st.aborted
            runs.append(reqs)
            log(f"step {s_}: {st.output_tokens} tok in {st.elapsed_s:.3f}s "
                f"({st.tokens_per_s:.1f} tok/s, {st.iterations} iterations, "
                f"{st.preemptions} preemptions)")
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        diverged = sorted({i for reqs in runs for i, r in enumerate(reqs)
                           if r.new_token_ids != conts[i]})
        n_req = sum(len(r.accepted_per_iter) for reqs in runs for r in reqs)
        spec = {
            "value": total_tokens / elapsed,
            "ms_per_step": elapsed / args.steps * 1e3,
            "output_tokens_per_step": total_tokens // args.steps,
            "iterations_per_step": iters // args.steps,
            "acceptance_rate": accepted / drafted if drafted else 0.0,
            "tokens_per_request_iteration": (total_tokens / n_req) if n_req else 0.0,
            "preemptions_per_step": preempt / args.steps,
            "recomputed_tokens_per_step": recomputed / args.steps,
            "aborted": aborted,
            "token_identical_to_greedy_continuation": not diverged,
            "requests_differing_from_continuation": diverged,
            "pool_blocks": pool_blocks,
            "concurrent_peak_blocks": peak,
            "narrow_batches": eng.narrow_batches,
        }
        if preempt == 0:
            log("WARNING: the timed runs never preempted; the pool is not below the peak")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(work, conts, sd_t, sd_d, t_arch, d_arch, k, args.p_accept,
                           args.cpu_seconds)
        log(f"cpu baseline: {cpu}")

    # Per-launch duration for the roofline: one HIP event pair around replays
    # of a graph of the timed launches, divided by the launch count -- the
    # kernels' own time (it agrees with the rocprof durations of the attention
    # and merge kernels); the per-launch event pairs add the gap each pair puts
    # between launches and are reported beside it.
    us = attn["graph_us"]
    traffic = None
    try:
        with open(os.path.join(HERE, "profiles", "verify_attn_c1_traffic.json")) as f:
            traffic = json.load(f)["hbm_bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        pass
    line = {
        "metric": METRIC,
        "value": round(spec.get("value", 0.0), 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(spec.get("ms_per_step", 0.0), 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,0.02) weights of the Qwen2.5-3B/0.5B architectures, "
                "uniform-random prompt ids",
        "config": {
            "workload": f"batched greedy speculative decode, 3B-arch target / 0.5B-arch draft, "
                        f"{args.slots} requests at once, prompts lognormal(median 128) in [16,1024], "
                        f"outputs lognormal(median 64) in [8,512], k={k}, oracle acceptance "
                        f"p={args.p_accept}, block 16, pools {args.pool_frac:.0%} of the "
                        f"concurrent peak",
            "batch": args.slots,
            "k": k,
            "p_accept": args.p_accept,
        },
        "roofline": {
            "kernel": "kve_paged_verify_attn (verify microbench)",
            "bound": "hbm",
            "achieved": round(attn["graph_gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(attn["graph_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": "profiles/verify_attn_c1_traffic.json (FETCH_SIZE/WRITE_SIZE passes "
                              "scaled by a 256 MiB copy)",
            "launch_us": round(us, 3),
            "timing": "HIP events around graph replays of the timed launches (per-launch "
                      "event pairs: verify_attn.event_mean_us)",
        },
        "verify_attn": attn,
        "verify_attn_large": attn_large,
        "lmhead": lm,
        "spec": spec,
        "parity_vs_reference": parity,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


# ---------------------------------------------------------------- other configs

def _models(seed: int):
    from kvengine_amd.arch import QWEN25_0_5B, QWEN25_3B
    from kvengine_amd.model import build_model
    from kvengine_amd.weights import generate_state_dict

    sd_t = generate_state_dict(QWEN25_3B, seed=seed, dtype=torch.bfloat16)
    sd_d = generate_state_dict(QWEN25_0_5B, seed=seed, dtype=torch.bfloat16)
    return (build_model(QWEN25_3B, sd_t, dtype=torch.bfloat16, device="cuda"),
            build_model(QWEN25_0_5B, sd_d, dtype=torch.bfloat16, device="cuda"), QWEN25_3B)


def _engine_runs(target, draft, work, k, p_accept, slots, pool_blocks, max_ctx, steps,
                 prefix_sharing=False, conts=None, pool_frac=None,
                 cont_draft=None):
    """Continuation (target greedy, via the engine with the real draft, or with
    cont_draft) unless given, then `steps` timed oracle-acceptance runs; with
    pool_frac, the timed runs use pools of pool_frac x the most blocks an
    unconstrained oracle run holds at once (pool_blocks is then the
    unconstrained size). Returns (stats dict, conts)."""
    from kvengine_amd.engine import SpecEngine, SpecRequest
    from kvengine_amd.workloads import OracleAcceptance

    def engine(blocks, drf=draft):
        return SpecEngine(target, drf, k=k, slots=slots, t_blocks=blocks, d_blocks=blocks,
                          block_size=16, max_ctx=max_ctx, prefix_sharing=prefix_sharing)

    vocab = target.config.vocab_size
    if conts is None:
        ce = engine(pool_blocks, cont_draft or draft)
        base = [SpecRequest(i, p, o) for i, (p, o) in enumerate(work)]
        t0 = time.perf_counter()
        ce.run(base)
        log(f"continuation: {sum(len(r.new_token_ids) for r in base)} tokens in "
            f"{time.perf_counter() - t0:.1f}s")
        conts = [r.new_token_ids for r in base]
        del ce

    def fresh():
        return [SpecRequest(i, p, o, propose=OracleAcceptance(
            [0] * len(p) + conts[i], p_accept, seed=1000 + i, vocab=vocab))
            for i, (p, o) in enumerate(work)]

    eng = engine(pool_blocks)
    eng.run(fresh())  # warm-up (graph capture) and the concurrent peak
    peak = max(eng.stats.peak_target_blocks, eng.stats.peak_draft_blocks)
    if pool_frac is not None:
        pool_blocks = max(math.ceil(pool_frac * peak),
                          max(-(-(len(p) + k + 1) // 16) for p, _ in work))
        del eng
        eng = engine(pool_blocks)
        eng.run(fresh())
    tot = iters = drafted = accepted = preempt = 0
    prefill_s = 0.0
    identical = True
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        eng.reset_stats(clear_prefix_cache=prefix_sharing)
        reqs = fresh()
        st = eng.run(reqs)
        tot += st.output_tokens
        iters += st.iterations
        drafted += st.drafted
        accepted += st.accepted
        preempt += st.preemptions
        prefill_s += st.prefill_s
        identical &= all(r.new_token_ids == conts[i] for i, r in enumerate(reqs))
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    return {"tok_s": round(tot / el, 1), "output_tokens": tot // steps,
            "iterations": iters // steps, "ms_per_run": round(el / steps * 1e3, 1),
            "admission_prefill_ms_per_run": round(prefill_s / steps * 1e3, 1),
            "acceptance_rate": round(accepted / max(drafted, 1), 4),
            "preemptions_per_run": preempt / steps, "pool_blocks": pool_blocks,
            "concurrent_peak_blocks": peak,
            "prefix_reused_tokens": st.prefix_reused_tokens,
            "token_identical_to_greedy_continuation": identical}, conts


def mode_c2(args) -> dict:
    """One request: 64-token random prompt, 128 new tokens, k=4, p=0.65, 3B/0.5B bf16 seed 1;
    timed through the batched engine with one slot and through speculative_greedy (the
    reference's B=1 API: one host sync per iteration)."""
    from kvengine_amd.decode import greedy_paged
    from kvengine_amd.paged import PagedKVCache
    from kvengine_amd.speculative import speculative_greedy
    from kvengine_amd.workloads import OracleAcceptance

    target, draft, arch = _models(1)
    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, arch.vocab, (64,), generator=g).tolist()
    ids = torch.tensor([prompt], device="cuda")

    # one pair of pools for every run, as a serving process keeps its pools (the
    # runs' iteration graphs, captured on the first, are replayed by the rest)
    t_pool, d_pool = PagedKVCache.for_model(target, 64, 16), PagedKVCache.for_model(draft, 64, 16)

    def spec(propose=None):
        ts, ds = t_pool.new_sequence("t"), d_pool.new_sequence("d")
        try:
            return speculative_greedy(target, draft, ids, ts, ds, k=args.k, max_new_tokens=128,
                                      eos_token_id=None, propose=propose)
        finally:
            ts.free()
            ds.free()

    # The oracle's continuation is the target's greedy output under the same code
    # path (speculative decoding with the real draft emits exactly it): plain
    # greedy feeds other row counts, whose GEMMs may round differently and part
    # at a near tie on these random-weight models.
    cont = spec().new_token_ids
    runs = [spec(OracleAcceptance([0] * 64 + cont, args.p_accept, seed=1000, vocab=arch.vocab))
            for _ in range(3)]
    best = min(runs[1:], key=lambda r: r.elapsed_s)
    eng, econt = _engine_runs(target, draft, [(prompt, 128)], args.k, args.p_accept, 1, 64, 256, 3)
    greedy = [greedy_paged(target, ids, PagedKVCache.for_model(target, 64, 16), max_new_tokens=128,
                           eos_token_id=None) for _ in range(3)]
    gbest = min(greedy[1:], key=lambda r: r.elapsed_s)

    def first_diff(a, b):
        return next((i for i, (x, y) in enumerate(zip(a, b)) if x != y), None)

    return {"metric": "single-sequence spec decode tok/s (3B target, 0.5B draft, k=4, p=0.65)",
            "speculative_greedy": {"tok_s": round(best.tokens_per_s, 1), "iterations": best.iterations,
                                   "acceptance_rate": round(best.acceptance_rate, 4),
                                   "tokens_equal_continuation": best.new_token_ids == cont},
            "engine_1slot": eng,
            "plain_greedy": {"tok_s": round(gbest.tokens_per_s, 1),
                             "first_token_differing_from_spec": first_diff(gbest.new_token_ids, cont)},
            "roofline_tok_s": 2000}


def mode_ksweep(args) -> dict:
    """The batched workload (32 requests) for k in 1, 2, 4, 8 at p=0.65."""
    from kvengine_amd.workloads import batched_spec_workload

    target, draft, arch = _models(args.seed)
    work = batched_spec_workload(seed=0, n=args.slots, vocab=arch.vocab)
    out = {}
    for k in (1, 2, 4, 8):
        max_ctx = -(-(max(len(p) + o for p, o in work) + k + 2) // 64) * 64
        roomy = 2 * sum(-(-(len(p) + o + k + 1) // 16) for p, o in work)
        # continuation from the same engine configuration (same verify shapes)
        res, _ = _engine_runs(target, draft, work, k, args.p_accept, args.slots, roomy, max_ctx, 1,
                              pool_frac=args.pool_frac)
        out[f"k={k}"] = res
        log(f"k={k}: {res}")
    return {"metric": "batched spec decode tok/s vs k (3B/0.5B bf16, B=32, p=0.65)",
            "results": {key: out[key] for key in ("k=1", "k=2", "k=4", "k=8")}}


def mode_c4(args) -> dict:
    """16 requests sharing a 2048-token prefix (128 refcounted blocks) + a 256-token suffix
    each, k=8, p=0.5, decoding --c4-new tokens each (5888: contexts reach 8192). The greedy
    continuation comes from the engine with the target as its own draft (every verify pass
    is the same as with the real draft, so the tokens are the target's greedy; a self-draft
    accepts nearly everything, so it needs ~9x fewer iterations). Then the verify-attention
    kernel alone at the 3B shapes (16/2 heads, D=128, q_len 9) on 16 sequences sharing the
    128 prefix blocks, at contexts 2304, 4096 and 8192."""
    from kvengine_amd.workloads import prefix_shared_workload

    target, draft, arch = _models(args.seed)
    k, p = 8, 0.5
    work = prefix_shared_workload(seed=0, vocab=arch.vocab, new_tokens=args.c4_new)
    max_ctx = -(-(2048 + 256 + args.c4_new + k + 2) // 64) * 64
    pool = 128 + 16 * (-(-(256 + args.c4_new + k + 16) // 16) + 1)
    eng, _ = _engine_runs(target, draft, work, k, p, 16, pool, max_ctx, 1, prefix_sharing=True,
                          cont_draft=target)
    log(f"c4 engine: {eng}")
    att = {}
    for L in (2304, 4096, 8192):
        att[f"ctx={L}"] = attn_case(16, L, 16, 2, 128, 9, 128, args.attn_units, args.attn_waves)
        log(f"c4 attention {L}: {att[f'ctx={L}']}")
    return {"metric": "prefix-shared verify (3B/0.5B bf16, 16 requests, 2048 shared + 256, k=8, p=0.5)",
            "engine": eng, "new_tokens_per_request": args.c4_new,
            "final_context": 2048 + 256 + args.c4_new, "verify_attention": att}


def mode_forward(args) -> dict:
    """One forward pass of the 0.5B draft or the 3B target (seeded weights) over
    --fwd-seqs sequences of --fwd-ctx history tokens and --fwd-q new tokens, as
    the batched engine runs it (the target on the wide layer with gemm_rows 160
    and the engine's fixed attention order; the draft's automatic order), block
    ids a seeded permutation; a HIP graph of the pass replayed --fwd-reps times
    (the lengths are not advanced, so every replay writes the same slots). With
    --fwd-api the target takes the path of the single-sequence API instead."""
    from kvengine_amd.arch import QWEN25_0_5B, QWEN25_3B
    from kvengine_amd.engine import TARGET_ATTN
    from kvengine_amd.forward import forward_hidden
    from kvengine_amd.model import build_model
    from kvengine_amd.paged import PagedKVCache

    tgt = args.fwd_model == "target"
    arch = QWEN25_3B if tgt else QWEN25_0_5B
    B, T, ctx = args.fwd_seqs, args.fwd_q, args.fwd_ctx
    model = build_model(arch, seed=args.seed, dtype=torch.bfloat16, device="cuda")
    per_seq = -(-(ctx + T) // 16) + 1
    pool = PagedKVCache.for_model(model, num_blocks=B * per_seq + 4, max_seqs=B)
    perm = torch.randperm(B * per_seq, generator=torch.Generator().manual_seed(args.seed))
    pool.tables[:, :per_seq] = perm.to(torch.int32).view(B, per_seq).cuda()
    pool.lens.fill_(ctx)
    rows = torch.arange(B, dtype=torch.int32, device="cuda")
    ids = torch.randint(0, arch.vocab, (B, T), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(args.seed))
    kw = {"gemm_rows": 160, "attn_order": TARGET_ATTN} if tgt and not args.fwd_api else {}

    def run():
        return forward_hidden(model, ids, pool.device_kv(), rows, ctx + T, **kw)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            run()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            run()
        for _ in range(3):
            g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(args.fwd_reps):
            g.replay()
        e1.record(s)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / args.fwd_reps
    wbytes = sum(p.numel() * p.element_size() for n, p in model.named_parameters() if "layers" in n)
    return {"metric": "forward pass us (HIP graph)", "model": arch.name, "seqs": B, "q": T,
            "ctx": ctx, "rows": B * T, "us": round(us, 1),
            "us_per_layer": round(us / arch.num_layers, 2),
            "layer_weight_bytes": wbytes // arch.num_layers,
            "weight_gbs": round(wbytes / (us * 1e-6) / 1e9, 1)}


MODES = {"c2": mode_c2, "ksweep": mode_ksweep, "c4": mode_c4, "forward": mode_forward}


def reference_parity(conts) -> dict | None:
    """The GPU's greedy continuations of the batched workload against the
    reference's own (tests/golden/c3_full.json, written by the reference's
    greedy_paged in bf16 with the ranked top-8 logits of every step): per
    request, the first step where they part and whether the reference's top-2
    margin there is within the stated tolerance (a near tie). After a
    divergence the two streams continue from different prefixes, so nothing
    past it is compared; tests/test_gpu_fullsize.py compares every step
    teacher-forced."""
    from kvengine_amd.margins import TOL_ULPS, bf16_ulp, compare_steps, first_divergence

    path = os.path.join(HERE, "tests", "golden", "c3_full.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        fx = json.load(f)
    identical, near, outside, compared = 0, [], [], 0
    for r in fx["requests"]:
        i, g = r["index"], r["greedy"]
        if i >= len(conts):
            continue
        d = first_divergence(conts[i], g["new_token_ids"])
        if d is None:
            identical += 1
            compared += len(g["new_token_ids"])
            continue
        compared += d + 1
        rep = compare_steps([conts[i][d]], [g["top_ids"][d]], [g["top_values"][d]])
        vals = g["top_values"][d]
        entry = {"request": i, "step": d,
                 "reference_top2_margin_ulps": round((vals[0] - vals[1]) / bf16_ulp(vals[0]), 2)}
        (outside if rep["outside_tolerance"] else near).append(entry)
    return {"reference": "tests/golden/c3_full.json (reference greedy_paged, bf16)",
            "requests": len(fx["requests"]), "identical": identical,
            "diverged_at_near_tie": near, "mismatches_outside_tolerance": len(outside),
            "outside": outside, "steps_compared": compared, "tolerance_ulps": TOL_ULPS}


def cpu_share() -> dict:
    """Host CPUs this process may use: the affinity mask, capped by a cgroup
    CPU quota when one is set (a container's share of a larger host)."""
    n_aff = len(os.sched_getaffinity(0))
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, per = f.read().split()
            if q != "max":
                quota = int(q) / int(per)
    except (OSError, ValueError):
        pass
    threads = n_aff if quota is None else max(1, min(n_aff, int(quota)))
    return {"os_cpu_count": os.cpu_count(), "affinity": n_aff, "cgroup_quota": quota,
            "threads": threads}


def cpu_baseline(work, conts, sd_t, sd_d, t_arch, d_arch, k, p_accept, seconds):
    """The reference's per-request loop (the CPU oracle of speculative_greedy,
    bf16) on two requests of the workload -- the one with the shortest prompt
    and the one with the median prompt length -- on every CPU this process
    may use. Three legs per request:
    * parity: one teacher-forced CPU forward over prompt + the GPU's
      continuation; the GPU's token at every step against the CPU's logits;
    * the CPU's own greedy continuation of the request (its time is reported);
    * timed: speculative_greedy with oracle acceptance p on that continuation,
      the target's argmax replaced by the continuation (the CPU's bf16 verify
      passes leave its own greedy at near ties, as the reference's do, after
      which oracle drafts are rejected: acceptance 0.005 measured), so the
      CPU runs the forwards of the same acceptance process as the GPU run;
      bounded at `seconds` per request.
    value = the two timed legs' output tokens / their time."""
    from kvengine_amd.margins import compare_steps
    from kvengine_amd.workloads import OracleAcceptance
    from oracle.model import RefQwen2
    from oracle.paged import RefPagedKVCache
    from oracle.spec import ref_greedy, ref_speculative_greedy

    share = cpu_share()
    cores = share["threads"]
    torch.set_num_threads(cores)
    by_len = sorted(range(len(work)), key=lambda j: (len(work[j][0]), j))
    picks = [("shortest prompt", by_len[0]), ("median prompt", by_len[len(by_len) // 2])]
    ref_t = RefQwen2(t_arch, sd_t, dtype=torch.bfloat16)
    ref_d = RefQwen2(d_arch, sd_d, dtype=torch.bfloat16)
    legs = []
    for label, i in picks:
        prompt, budget = work[i]
        nb = -(-(len(prompt) + budget + k + 2) // 16) + 2

        def pool(arch):
            return RefPagedKVCache(arch.num_layers, arch.num_kv_heads, arch.head_dim, nb, 16,
                                   torch.bfloat16)

        log(f"cpu baseline on request {i} ({label}: prompt {len(prompt)}, {budget} tokens), "
            f"{cores} threads ({share})")
        parity = None
        if conts is not None:
            t0 = time.perf_counter()
            seq = pool(t_arch).new_sequence("tf")
            full = prompt + conts[i][:-1]
            logits = ref_t.forward(torch.tensor([full]), seq, all_logits=True)[0, len(prompt) - 1:]
            top = torch.topk(logits.float(), 8, dim=-1)
            ids, vals = [], []
            for v, j in zip(top.values.tolist(), top.indices.tolist()):
                pairs = sorted(zip(v, j), key=lambda p: (-p[0], p[1]))
                vals.append([p[0] for p in pairs])
                ids.append([p[1] for p in pairs])
            rep = compare_steps(conts[i], ids, vals)
            parity = {k_: rep[k_] for k_ in ("steps", "matches", "mismatches", "near_ties",
                                              "exact_ties", "tolerance_ulps")}
            parity["mismatches_outside_tolerance"] = len(rep["outside_tolerance"])
            parity["seconds"] = round(time.perf_counter() - t0, 1)
            log(f"cpu teacher-forced parity: {parity}")
        g = ref_greedy(ref_t, torch.tensor([prompt]), pool(t_arch).new_sequence("g"),
                       max_new_tokens=budget)
        cpu_cont = g.new_token_ids
        propose = OracleAcceptance([0] * len(prompt) + cpu_cont, p_accept, seed=1000 + i,
                                   vocab=t_arch.vocab)
        r = ref_speculative_greedy(ref_t, ref_d, torch.tensor([prompt]),
                                   pool(t_arch).new_sequence("t"), pool(d_arch).new_sequence("d"),
                                   k=k, max_new_tokens=budget, propose=propose,
                                   deadline_s=seconds, forced_preds=prompt + cpu_cont)
        legs.append({"request": i, "which": label, "prompt_tokens": len(prompt),
                     "budget": budget, "tokens": len(r.new_token_ids),
                     "iterations": r.iterations, "seconds": round(r.elapsed_s, 2),
                     "tok_s": round(len(r.new_token_ids) / r.elapsed_s, 3),
                     "measured_acceptance": round(r.tokens_accepted / max(r.tokens_drafted, 1), 3),
                     "greedy_tok_s": round(len(cpu_cont) / g.elapsed_s, 3),
                     "teacher_forced_parity": parity})
        log(f"cpu baseline leg: {legs[-1]}")
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            cpu_model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    tok = sum(x["tokens"] for x in legs)
    sec = sum(x["seconds"] for x in legs)
    return {
        "value": round(tok / sec, 3),
        "unit": "tok/s",
        "cores": cores,
        "kind": "port",
        "sample": f"CPU oracle of the reference loop (speculative_greedy, bf16, k={k}, oracle "
                  f"acceptance p={p_accept} on the CPU's own greedy continuation, the target "
                  f"following that continuation) on two requests, one at a time as the reference "
                  f"decodes: " + "; ".join(
                      f"request {x['request']} ({x['which']}, {x['prompt_tokens']} tokens): "
                      f"{x['tokens']} tokens in {x['iterations']} iterations, {x['seconds']:.1f}s, "
                      f"{x['tok_s']:.1f} tok/s" for x in legs) +
                  f" (each bounded at {seconds:.0f}s)",
        "legs": legs,
        "cpu_model": cpu_model,
        "cpu_share": share,
    }


if __name__ == "__main__":
    main()
