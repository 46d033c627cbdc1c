"""Oracle verify attention for one layer. TEST INFRASTRUCTURE.

`gather_then_attend` is the reference's read path for a batch of sequences,
one sequence at a time (the reference has no batched verify):
gather whole blocks in block-table order from the [NB, bs, Hkv, D] pool and trim
to the context (kvengine/paged.py:315-331), expand GQA heads with repeat_kv
(forward.py:72-82, 130-131), then SDPA with the additive finfo.min causal mask
for the last T positions (forward.py:85-103, 133-137), or the eager form with a
float32 softmax whose probabilities are cast back to the input dtype before the
PV product (forward.py:139-144).

`attend_fp64` is the textbook definition evaluated in float64 with explicit
loops over the causal window; it pins the restatement above.
"""

from __future__ import annotations

import torch

from .model import attend, causal_mask


def gather_blocks(pool_layer: torch.Tensor, blocks: list[int], end: int) -> torch.Tensor:
    """[NB, bs, Hkv, D] pool, table -> [1, Hkv, end, D] contiguous."""
    bs = pool_layer.shape[1]
    nb = -(-end // bs)
    ids = torch.tensor(blocks[:nb], dtype=torch.long)
    rows = pool_layer[ids].reshape(nb * bs, pool_layer.shape[2], pool_layer.shape[3])
    return rows[:end].transpose(0, 1).unsqueeze(0).contiguous()


def gather_then_attend(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                       tables: list[list[int]], ctx_lens: list[int], q_lens: list[int] | None = None,
                       scale: float | None = None, use_sdpa: bool = True) -> torch.Tensor:
    """q [B, Tmax, Hq, D]; ctx_lens include the new tokens. Returns [B, Tmax, Hq, D]
    (rows past a sequence's q_len are zero)."""
    B, Tmax, Hq, D = q.shape
    Hkv = k_pool.shape[2]
    scale = D ** -0.5 if scale is None else scale
    out = torch.zeros_like(q)
    for b in range(B):
        T = Tmax if q_lens is None else q_lens[b]
        L = ctx_lens[b]
        kb = gather_blocks(k_pool, tables[b], L)
        vb = gather_blocks(v_pool, tables[b], L)
        qb = q[b:b + 1, :T].transpose(1, 2)
        mask = causal_mask(T, L, q.dtype)
        out[b, :T] = attend(qb, kb, vb, mask, Hq // Hkv, scale, use_sdpa)[0]
    return out


def attend_fp64(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                tables: list[list[int]], ctx_lens: list[int], q_lens: list[int] | None = None,
                scale: float | None = None) -> torch.Tensor:
    """Brute-force float64 verify attention; query t of sequence b sits at
    position ctx_len - q_len + t and sees keys 0..that position."""
    B, Tmax, Hq, D = q.shape
    bs, Hkv = k_pool.shape[1], k_pool.shape[2]
    G = Hq // Hkv
    scale = D ** -0.5 if scale is None else scale
    out = torch.zeros(q.shape, dtype=torch.float64)
    for b in range(B):
        T = Tmax if q_lens is None else q_lens[b]
        L = ctx_lens[b]
        pos = torch.arange(L)
        blk = torch.tensor(tables[b], dtype=torch.long)[pos // bs]
        K = k_pool[blk, pos % bs].double()  # [L, Hkv, D]
        V = v_pool[blk, pos % bs].double()
        for h in range(Hq):
            kv = h // G
            for t in range(T):
                last = L - T + t
                s = (K[: last + 1, kv] @ q[b, t, h].double()) * scale
                p = torch.exp(s - s.max())
                out[b, t, h] = (p[:, None] * V[: last + 1, kv]).sum(0) / p.sum()
    return out


def normalized_error(out: torch.Tensor, ref: torch.Tensor) -> float:
    """max over (seq, head) of max|out-ref| / max|ref| on that (seq, head) slice."""
    o = out.double()
    r = ref.double()
    err = (o - r).abs().amax(dim=(1, 3))
    mag = r.abs().amax(dim=(1, 3)).clamp_min(1e-30)
    return float((err / mag).max())



def relative_rms_error(out: torch.Tensor, ref: torch.Tensor) -> float:
    """max over (seq, head) of ||out-ref||_2 / ||ref||_2 on that (seq, head) slice.

    The bf16 criterion: a bf16 output differs from any other bf16 rounding of
    the same value by up to one unit in the last place (2**-8 relative), so a
    per-element max criterion below that cannot be met; the RMS ratio is
    2e-3-scale for a correct kernel and O(1) for a masking or indexing bug.
    """
    o = out.double()
    r = ref.double()
    num = (o - r).pow(2).sum(dim=(1, 3)).sqrt()
    den = r.pow(2).sum(dim=(1, 3)).sqrt().clamp_min(1e-30)
    return float((num / den).max())
