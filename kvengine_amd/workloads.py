"""Synthetic workloads for the verify path: context lengths, paged pools, drafts.

Everything is drawn from explicit seeds with torch's CPU generator (or Python's
`random.Random` for per-token draft decisions), so the same inputs are rebuilt
on any machine and handed both to the HIP path and to the CPU reference.
"""

from __future__ import annotations

import math
import random
from dataclasses import dataclass

import torch


def lognormal_lengths(n: int, median: float, sigma: float, lo: int, hi: int,
                      gen: torch.Generator) -> list[int]:
    """clip(round(exp(N(ln median, sigma))), lo, hi).

    The reference's length sampler (kvengine/bench.py:73-81) sets mu = ln(mean),
    so its "mean" is the median; this helper takes the median explicitly.
    """
    z = torch.randn(n, generator=gen, dtype=torch.float64)
    mu = math.log(median)
    return [int(min(hi, max(lo, round(math.exp(mu + sigma * float(x)))))) for x in z]


class OracleAcceptance:
    """Draft proposals with a controlled acceptance probability.

    `continuation[p]` is the target's own greedy token at absolute position p.
    Each call draws u ~ U[0,1) from a seeded stream: the proposal becomes
    continuation[p] when u < p_accept, else a uniform id different from it.
    One draw per drafted token (not per position), so re-drafting a position
    after a rejection is an independent trial. The draft model still runs; its
    own argmax is only replaced. Positions past the continuation keep the
    draft's proposal.
    """

    def __init__(self, continuation: list[int], p_accept: float, seed: int, vocab: int):
        self.cont = list(continuation)
        self.p = p_accept
        self.vocab = vocab
        self.rng = random.Random(seed)
        self.draws = 0

    def predraw(self, pos: int) -> int:
        """The proposal for absolute position `pos`, or -1 to keep the draft's own
        argmax. Consumes exactly the draws one __call__ does, so a loop that
        pre-draws on the host reproduces a loop that asks per token."""
        self.draws += 1
        u = self.rng.random()
        r = self.rng.randrange(self.vocab - 1)
        if pos >= len(self.cont):
            return -1
        want = self.cont[pos]
        if u < self.p:
            return want
        return r if r < want else r + 1

    def __call__(self, pos: int, proposal: int) -> int:
        t = self.predraw(pos)
        return proposal if t < 0 else t


@dataclass
class VerifyAttnCase:
    """One verify-attention launch: paged K/V plus the queries of the draft window."""

    ctx_lens: list[int]          # tokens per sequence, including the q_len new ones
    tables: list[list[int]]      # logical block -> physical block
    q: torch.Tensor              # [B, T, Hq, D]
    pool: torch.Tensor           # [2, NB, bs, Hkv, D]: K and V in the reference layout
    block_size: int

    @property
    def num_blocks(self) -> int:
        return self.pool.shape[1]

    def algorithmic_bytes(self) -> int:
        """K/V read once + Q read + O write + block tables + context lengths."""
        B, T, Hq, D = self.q.shape
        Hkv = self.pool.shape[3]
        e = self.q.element_size()
        kv = sum(2 * L * Hkv * D * e for L in self.ctx_lens)
        qo = 2 * B * T * Hq * D * e
        tbl = sum(4 * (-(-L // self.block_size)) for L in self.ctx_lens) + 4 * B
        return kv + qo + tbl


def verify_attn_case(seed: int, num_seqs: int = 32, q_len: int = 5, num_q_heads: int = 14,
                     num_kv_heads: int = 2, head_dim: int = 64, block_size: int = 16,
                     median: float = 512, sigma: float = 0.8, lo: int = 64, hi: int = 4096,
                     pool_factor: float = 1.25, dtype=torch.bfloat16,
                     ctx_lens: list[int] | None = None) -> VerifyAttnCase:
    """Verify-attention microbench inputs.

    Context lengths are lognormal (median, sigma) clipped to [lo, hi] and include
    the q_len window; the pool holds ceil(pool_factor * needed) blocks; physical
    ids are randperm(NB)[:needed] handed out in sequence order; Q/K/V ~ N(0, 1).
    """
    g = torch.Generator().manual_seed(seed)
    if ctx_lens is None:
        ctx_lens = lognormal_lengths(num_seqs, median, sigma, lo, hi, g)
    need = [-(-L // block_size) for L in ctx_lens]
    nb = max(1, math.ceil(pool_factor * sum(need)))
    perm = torch.randperm(nb, generator=g).tolist()
    tables, at = [], 0
    for n in need:
        tables.append(perm[at:at + n])
        at += n
    q = torch.randn(len(ctx_lens), q_len, num_q_heads, head_dim, generator=g).to(dtype)
    pool = torch.randn(2, nb, block_size, num_kv_heads, head_dim, generator=g).to(dtype)
    return VerifyAttnCase(ctx_lens, tables, q, pool, block_size)


def reference_lognormal(rng: random.Random, mean: float, sigma: float, lo: int, hi: int) -> int:
    """The reference's length sampler (kvengine/bench.py:73-81): mu = ln(mean),
    so `mean` is the median; rounded and clamped to [lo, hi]."""
    mu = math.log(max(mean, 1.0))
    return max(lo, min(hi, int(round(math.exp(rng.gauss(mu, sigma))))))


def batched_spec_workload(seed: int = 0, n: int = 32, vocab: int = 151936,
                          prompt_mean: float = 128, output_mean: float = 64, sigma: float = 0.6,
                          prompt_range=(16, 1024), output_range=(8, 512)):
    """(prompt ids, output budget) per request for the batched speculative
    workload: lognormal lengths with the reference's sampler (default sigma
    0.6, kvengine/bench.py:89,91) and uniform-random prompt ids."""
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        p = reference_lognormal(rng, prompt_mean, sigma, *prompt_range)
        o = reference_lognormal(rng, output_mean, sigma, *output_range)
        out.append(([rng.randrange(vocab) for _ in range(p)], o))
    return out


def prefix_shared_workload(seed: int = 0, n: int = 16, prefix_len: int = 2048,
                           suffix_len: int = 256, vocab: int = 151936, new_tokens: int = 256):
    """Long-context prefix-shared verify: n requests = one shared random prefix
    of prefix_len tokens + a distinct random suffix each; every request decodes
    new_tokens tokens (the full run decodes until the context reaches 8192)."""
    rng = random.Random(seed)
    prefix = [rng.randrange(vocab) for _ in range(prefix_len)]
    return [(prefix + [rng.randrange(vocab) for _ in range(suffix_len)], new_tokens)
            for _ in range(n)]
