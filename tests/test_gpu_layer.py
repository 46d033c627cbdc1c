"""Fused layer kernels against the torch op sequences they replace.

Elementwise kernels (RoPE + KV write, SiLU*up) round at exactly the points the
torch ops do, so they must agree bit for bit. RMSNorm's mean is a float32 sum
in a different order, which may move the float32 result by an ulp and,
rarely, the rounded model-dtype output by one ulp; that is bounded here.
"""

import pytest
import torch
import torch.nn.functional as F

from kvengine_amd import _lib, kernels
from kvengine_amd.arch import TINY, TINY128
from kvengine_amd.decode import greedy_paged
from kvengine_amd.forward import apply_rope, forward_hidden
from kvengine_amd.model import RMSNorm, RotaryEmbedding, build_model
from kvengine_amd.paged import PagedKVCache
from kvengine_amd.weights import generate_state_dict

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.bfloat16, torch.float32]


def ulps_apart(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in units of the last place of the model dtype, elementwise."""
    if a.dtype == torch.bfloat16:
        ia, ib = a.view(torch.int16).int(), b.view(torch.int16).int()
    else:
        ia, ib = a.view(torch.int32).long(), b.view(torch.int32).long()
    return (ia - ib).abs()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("H", [128, 896, 2048])
@pytest.mark.parametrize("with_delta", [False, True])
def test_rmsnorm_matches_module(gpu_lib, dtype, H, with_delta):
    g = torch.Generator().manual_seed(H)
    x = torch.randn(37, H, generator=g).to(dtype).to(DEV)
    d = torch.randn(37, H, generator=g).to(dtype).to(DEV) if with_delta else None
    norm = RMSNorm(H, 1e-6).to(DEV)
    norm.weight.data = (1 + 0.1 * torch.randn(H, generator=g)).to(dtype).to(DEV)
    r_ref = x + d if with_delta else x
    ref = norm(r_ref)
    r_out = torch.empty_like(x)
    out = kernels.rmsnorm(x, norm.weight.data, 1e-6, delta=d, residual_out=r_out)
    assert torch.equal(r_out, r_ref)
    dist = ulps_apart(out, ref)
    if dtype == torch.bfloat16:
        assert dist.max().item() <= 1, "more than one ulp from the module"
        assert (dist > 0).float().mean().item() < 0.01
    else:
        # the float32 mean is summed in another order: a few ulps at most
        assert dist.max().item() <= 8


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("arch", [TINY, TINY128], ids=["gqa7-d64", "gqa8-d128"])
def test_rope_kv_write_matches_unfused(gpu_lib, dtype, arch):
    B, T, Hq, Hkv, D = 3, 5, arch.num_q_heads, arch.num_kv_heads, arch.head_dim
    g = torch.Generator().manual_seed(1)
    qkv = torch.randn(B, T, (Hq + 2 * Hkv) * D, generator=g).to(dtype).to(DEV)
    rot = RotaryEmbedding(D, 1e6).to(DEV)
    start = torch.tensor([3, 0, 17], dtype=torch.int32, device=DEV)
    pos = start.long()[:, None] + torch.arange(T, device=DEV)[None]
    cos, sin = rot(qkv, pos)
    nb, bs = 12, 16
    tables = torch.tensor([[4, 9, -1], [0, -1, -1], [7, 2, -1]], dtype=torch.int32, device=DEV)
    q_lens = torch.tensor([5, 2, 4], dtype=torch.int32, device=DEV)
    pools = [(torch.zeros(nb, Hkv, bs, D, dtype=dtype, device=DEV),
              torch.zeros(nb, Hkv, D, bs, dtype=dtype, device=DEV)) for _ in range(2)]
    q_f = kernels.rope_kv_write(qkv, cos.contiguous(), sin.contiguous(), *pools[0], tables, start,
                                Hq, q_lens=q_lens)
    q = qkv[..., : Hq * D].view(B, T, Hq, D)
    k = qkv[..., Hq * D:(Hq + Hkv) * D].view(B, T, Hkv, D)
    v = qkv[..., (Hq + Hkv) * D:].reshape(B, T, Hkv, D).contiguous()
    q_r, k_r = apply_rope(q, k, cos, sin, unsqueeze_dim=2)
    kernels.kv_write(k_r.contiguous(), v, *pools[1], tables, start, q_lens=q_lens)
    assert torch.equal(q_f, q_r)
    assert torch.equal(pools[0][0], pools[1][0]) and torch.equal(pools[0][1], pools[1][1])


@pytest.mark.parametrize("dtype", DTYPES)
def test_silu_mul_matches_torch(gpu_lib, dtype):
    g = torch.Generator().manual_seed(2)
    gu = (3 * torch.randn(19, 2 * 4864, generator=g)).to(dtype).to(DEV)
    F_ = gu.shape[-1] // 2
    ref = F.silu(gu[:, :F_]) * gu[:, F_:]
    out = kernels.silu_mul(gu)
    dist = ulps_apart(out, ref)
    assert dist.max().item() <= 1
    assert (dist > 0).float().mean().item() < 0.001


@pytest.mark.parametrize("dtype", DTYPES)
def test_fused_forward_matches_module_forward(gpu_lib, dtype):
    model = build_model(TINY, generate_state_dict(TINY, seed=3), dtype=dtype, device=DEV)
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, TINY.vocab, (2, 9), generator=g).to(DEV)
    outs = []
    for fused in (True, False):
        pool = PagedKVCache.for_model(model, 16, 4)
        seqs = [pool.new_sequence(i) for i in range(2)]
        for s in seqs:
            s.reserve(9)
        rows = torch.tensor([s.row for s in seqs], dtype=torch.int32, device=DEV)
        outs.append(forward_hidden(model, ids, pool.device_kv(), rows, 9, fused=fused))
    a, b = outs
    if dtype == torch.float32:
        assert (a - b).abs().max().item() < 1e-4
    else:
        assert ulps_apart(a, b).max().item() <= 4


def test_fused_greedy_tokens_equal_module_greedy(gpu_lib):
    from kvengine_amd import forward as fwd

    model = build_model(TINY, generate_state_dict(TINY, seed=3), dtype=torch.float32, device=DEV)
    ids = torch.randint(0, TINY.vocab, (1, 12), generator=torch.Generator().manual_seed(4)).to(DEV)
    fused = greedy_paged(model, ids, PagedKVCache.for_model(model, 64, 4), 24, eos_token_id=None)
    orig = fwd._fusable
    try:
        fwd._fusable = lambda m: False
        plain = greedy_paged(model, ids, PagedKVCache.for_model(model, 64, 4), 24, eos_token_id=None)
    finally:
        fwd._fusable = orig
    assert fused.new_token_ids == plain.new_token_ids


# ---- fused skinny projections (bf16, decode-sized batches) --------------------
# They replace hipBLASLt GEMMs whose float32 dot products are summed in another
# order, so a Linear output may differ by one bf16 ulp and what follows it by a
# little more; everything else is rounded at the reference's points.

def close_bf16(a: torch.Tensor, b: torch.Tensor, rel: float = 2 ** -6, frac: float = 0.05):
    """Elementwise within `rel` of the reference's scale, and most elements equal."""
    a, b = a.float(), b.float()
    scale = b.abs() + b.pow(2).mean().sqrt()
    bad = (a - b).abs() > rel * scale
    assert not bad.any(), f"{int(bad.sum())} elements off by more than {rel} relative"
    diff = (a != b).float().mean().item()
    assert diff < frac, f"{diff:.3f} of elements differ"


@pytest.mark.parametrize("arch", [TINY, TINY128], ids=["d64", "d128"])
@pytest.mark.parametrize("B,T", [(3, 5), (32, 2), (7, 1)])
def test_fused_qkv_matches_unfused(gpu_lib, arch, B, T):
    g = torch.Generator().manual_seed(5)
    H, Hq, Hkv, D = arch.hidden, arch.num_q_heads, arch.num_kv_heads, arch.head_dim
    dt = torch.bfloat16
    res = torch.randn(B, T, H, generator=g).to(dt).to(DEV)
    nw = (1 + 0.1 * torch.randn(H, generator=g)).to(dt).to(DEV)
    W = (0.05 * torch.randn((Hq + 2 * Hkv) * D, H, generator=g)).to(dt).to(DEV)
    bias = (0.1 * torch.randn((Hq + 2 * Hkv) * D, generator=g)).to(dt).to(DEV)
    rot = RotaryEmbedding(D, 1e6).to(DEV)
    start = torch.randint(0, 40, (B,), generator=g, dtype=torch.int32).to(DEV)
    pos = start.long()[:, None] + torch.arange(T, device=DEV)[None]
    cos, sin = rot(res, pos)
    cos, sin = cos.contiguous(), sin.contiguous()
    nb, bs, width = 4 * B + 8, 16, 4
    perm = torch.randperm(nb, generator=g)[: B * width].view(B, width).to(torch.int32).to(DEV)
    q_lens = torch.randint(1, T + 1, (B,), generator=g, dtype=torch.int32).to(DEV)
    pools = [(torch.zeros(nb, Hkv, bs, D, dtype=dt, device=DEV),
              torch.zeros(nb, Hkv, D, bs, dtype=dt, device=DEV)) for _ in range(2)]
    h = kernels.rmsnorm(res, nw, 1e-6)
    qkv = F.linear(h, W, bias)
    q_ref = kernels.rope_kv_write(qkv, cos, sin, *pools[0], perm, start, Hq, q_lens=q_lens)
    q = kernels.fused_qkv(res, nw, 1e-6, W, bias, cos, sin, *pools[1], perm, start, Hq, q_lens=q_lens)
    close_bf16(q, q_ref)
    close_bf16(pools[1][0], pools[0][0])
    close_bf16(pools[1][1], pools[0][1])
    # rows past q_len wrote nothing
    assert torch.equal(pools[1][0] == 0, pools[0][0] == 0)


@pytest.mark.parametrize("M,N,K", [(32, 896, 896), (64, 896, 4864), (5, 128, 256), (17, 2048, 2048)])
def test_linear_residual_matches_linear_then_add(gpu_lib, M, N, K):
    g = torch.Generator().manual_seed(M + N)
    dt = torch.bfloat16
    x = torch.randn(M, K, generator=g).to(dt).to(DEV)
    W = (0.03 * torch.randn(N, K, generator=g)).to(dt).to(DEV)
    res = torch.randn(M, N, generator=g).to(dt).to(DEV)
    want = res + F.linear(x, W)
    got = kernels.linear_residual(x, W, res.clone())
    close_bf16(got, want)


@pytest.mark.parametrize("M,H,Fd", [(32, 896, 4864), (64, 896, 4864), (9, 128, 256)])
def test_fused_gate_up_matches_unfused(gpu_lib, M, H, Fd):
    g = torch.Generator().manual_seed(M + H)
    dt = torch.bfloat16
    res = torch.randn(M, H, generator=g).to(dt).to(DEV)
    nw = (1 + 0.1 * torch.randn(H, generator=g)).to(dt).to(DEV)
    W = (0.05 * torch.randn(2 * Fd, H, generator=g)).to(dt).to(DEV)
    want = kernels.silu_mul(F.linear(kernels.rmsnorm(res, nw, 1e-6), W))
    got = kernels.fused_gate_up(res, nw, 1e-6, W)
    close_bf16(got, want)


def _forward_rows(model, ids, gemm_rows=None):
    B, T = ids.shape
    pool = PagedKVCache.for_model(model, max(16, B * -(-T // 4) + 4), 4, max_seqs=max(B, 8))
    seqs = [pool.new_sequence(i) for i in range(ids.shape[0])]
    for s in seqs:
        s.reserve(ids.shape[1])
    rows = torch.tensor([s.row for s in seqs], dtype=torch.int32, device=DEV)
    return forward_hidden(model, ids, pool.device_kv(), rows, ids.shape[1], fused=True,
                          gemm_rows=gemm_rows)


@pytest.mark.parametrize("path", ["splitk", "fused"])
def test_small_batch_forward_matches_hipblaslt_forward(gpu_lib, path):
    from kvengine_amd import forward as fwd

    model = build_model(TINY, generate_state_dict(TINY, seed=3), dtype=torch.bfloat16, device=DEV)
    ids = torch.randint(0, TINY.vocab, (4, 3), generator=torch.Generator().manual_seed(6)).to(DEV)
    outs = []
    prev = fwd.SMALL_BATCH_PATH
    for small in (True, False):
        fwd.SMALL_BATCH_FUSION = small
        fwd.SMALL_BATCH_PATH = path
        try:
            outs.append(_forward_rows(model, ids))
        finally:
            fwd.SMALL_BATCH_FUSION = True
            fwd.SMALL_BATCH_PATH = prev
    close_bf16(outs[0], outs[1], rel=2 ** -5, frac=0.2)


@pytest.mark.parametrize("arch", [TINY, TINY128], ids=["d64", "d128"])
@pytest.mark.parametrize("B,T", [(32, 5), (13, 9)])
def test_large_batch_splitk_projections_match_hipblaslt(gpu_lib, arch, B, T):
    """65-160 rows: o_proj / down_proj as split-K with the fused residual + RMSNorm
    reduction against hipBLASLt + the separate residual/RMSNorm kernel."""
    from kvengine_amd import forward as fwd

    model = build_model(arch, generate_state_dict(arch, seed=4), dtype=torch.bfloat16, device=DEV)
    ids = torch.randint(0, arch.vocab, (B, T), generator=torch.Generator().manual_seed(3)).to(DEV)
    assert fwd._splitk_ok(model, B * T) and not fwd._small_fusable(model, B * T)
    outs = []
    for on in (True, False):
        fwd.SMALL_BATCH_FUSION = on
        try:
            outs.append(_forward_rows(model, ids))
        finally:
            fwd.SMALL_BATCH_FUSION = True
    close_bf16(outs[0], outs[1], rel=2 ** -5, frac=0.2)


@pytest.mark.parametrize("arch", [TINY, TINY128], ids=["d64", "d128"])
@pytest.mark.parametrize("path,B", [("splitk", 9), ("splitk7", 9), ("fused", 4)])
def test_decode_paths_are_batch_invariant(gpu_lib, arch, path, B):
    """A sequence's hidden states do not depend on which other sequences share
    the pass, on either decode path (split-K: slices and sums depend on weight
    shapes only; fused: whole columns per workgroup, rows independent), with
    the split-K layer's o_proj and gate/up fused (up to 32 rows) or as k-slices
    + kve_residual_norm (splitk7)."""
    from kvengine_amd import forward as fwd

    model = build_model(arch, generate_state_dict(arch, seed=8), dtype=torch.bfloat16, device=DEV)
    ids = torch.randint(0, arch.vocab, (B, 2), generator=torch.Generator().manual_seed(2)).to(DEV)
    prev, prev_o = fwd.SMALL_BATCH_PATH, fwd.SPLITK_FUSED_O
    fwd.SMALL_BATCH_PATH = "splitk" if path == "splitk7" else path
    fwd.SPLITK_FUSED_O = path != "splitk7"
    try:
        full = _forward_rows(model, ids)
        for i in (0, B // 2, B - 1):
            one = _forward_rows(model, ids[i:i + 1])
            assert torch.equal(one[0], full[i]), f"row {i} differs alone"
        assert torch.equal(_forward_rows(model, ids[1:3]), full[1:3])
    finally:
        fwd.SMALL_BATCH_PATH, fwd.SPLITK_FUSED_O = prev, prev_o


@pytest.mark.parametrize("arch", [TINY, TINY128], ids=["d64", "d128"])
def test_splitk_layers_with_and_without_fused_o_agree(gpu_lib, arch):
    """The split-K decode layer with o_proj + residual and RMSNorm + gate/up
    fused (whole-K o_proj sums, the norm in the gate/up prologue) against the
    seven-launch layer (o_proj k-slices, kve_residual_norm, kve_gate_up_silu):
    the same layer up to bf16 rounding, and a blocked activation written by
    kve_fused_gate_up equals the row-major one bit for bit."""
    from kvengine_amd import forward as fwd

    model = build_model(arch, generate_state_dict(arch, seed=9), dtype=torch.bfloat16, device=DEV)
    ids = torch.randint(0, arch.vocab, (6, 3), generator=torch.Generator().manual_seed(3)).to(DEV)
    prev, prev_o = fwd.SMALL_BATCH_PATH, fwd.SPLITK_FUSED_O
    outs = []
    try:
        fwd.SMALL_BATCH_PATH = "splitk"
        for on in (True, False):
            fwd.SPLITK_FUSED_O = on
            outs.append(_forward_rows(model, ids))
    finally:
        fwd.SMALL_BATCH_PATH, fwd.SPLITK_FUSED_O = prev, prev_o
    close_bf16(outs[0], outs[1], rel=2 ** -5, frac=0.2)
    layer = model.model.layers[0]
    H = layer.mlp.gate_up_weight.shape[1]
    x = torch.randn(18, H, generator=torch.Generator().manual_seed(4)).to(DEV, torch.bfloat16)
    nw = layer.post_attention_layernorm.weight
    row = kernels.fused_gate_up(x, nw, 1e-6, layer.mlp.gate_up_weight_blk, blocked_w=True)
    blk = kernels.fused_gate_up(x, nw, 1e-6, layer.mlp.gate_up_weight_blk, blocked_w=True,
                                blocked_act=True)
    assert torch.equal(kernels.from_blocked(blk, 18), row)


def test_invariant_gemm_rows_picks_one_path_for_every_width(gpu_lib):
    """When a model's full-width pass misses the decode layer (the 3B verify pass
    at k=1: 64 rows) but its narrow passes fit it, every width must still take
    the wide layer: one path, so one rounding, for every batch width."""
    from kvengine_amd import forward as fwd

    for arch, rows in ((TINY, 64), (TINY128, 160)):
        m = build_model(arch, generate_state_dict(arch, seed=1), dtype=torch.bfloat16, device=DEV)
        ok, gr = fwd.invariant_gemm_rows(m, rows)
        assert ok
        orig = fwd._small_fusable
        try:
            # a model whose full-width pass misses the decode layer but whose narrow passes fit it
            fwd._small_fusable = lambda mm, n: n <= rows // 2
            ok, gr = fwd.invariant_gemm_rows(m, rows)
            assert ok and gr == rows
            calls = []
            orig_split = fwd._forward_splitk
            fwd._forward_splitk = lambda *a, **k: calls.append(k.get("wide", False)) or orig_split(*a, **k)
            try:
                for w in (1, rows // 5 // 2, rows // 5):
                    ids = torch.randint(0, arch.vocab, (max(w, 1), 5),
                                        generator=torch.Generator().manual_seed(w)).to(DEV)
                    _forward_rows(m, ids, gemm_rows=gr)
            finally:
                fwd._forward_splitk = orig_split
            assert calls and all(calls), calls
        finally:
            fwd._small_fusable = orig


@pytest.mark.parametrize("arch", [TINY, TINY128], ids=["d64", "d128"])
def test_wide_verify_forward_is_width_invariant(gpu_lib, arch):
    """gemm_rows=160 takes the wide split-K layer for every pass, so a verify pass
    over 1, 2, 4 ... of 32 sequences gives each sequence the bits it gets in
    the full 160-row pass."""
    model = build_model(arch, generate_state_dict(arch, seed=9), dtype=torch.bfloat16, device=DEV)
    ids = torch.randint(0, arch.vocab, (32, 5), generator=torch.Generator().manual_seed(5)).to(DEV)
    full = _forward_rows(model, ids, gemm_rows=160)
    assert torch.equal(full, _forward_rows(model, ids))
    for w in (1, 2, 4, 8, 16):
        part = _forward_rows(model, ids[32 - w:], gemm_rows=160)
        assert torch.equal(part, full[32 - w:]), f"width {w} differs"


# ---- split-K decode layer -------------------------------------------------------

@pytest.mark.parametrize("M,N,K", [(32, 896, 896), (64, 896, 4864), (5, 128, 256), (17, 2048, 2048),
                                   (1, 2048, 11008), (160, 2048, 11008), (100, 2048, 2048),
                                   (40, 2560, 2048), (80, 896, 4864), (130, 128, 256)])
def test_linear_splitk_partials_sum_to_the_product(gpu_lib, M, N, K):
    g = torch.Generator().manual_seed(M + N + K)
    dt = torch.bfloat16
    x = torch.randn(M, K, generator=g).to(dt).to(DEV)
    W = (0.03 * torch.randn(N, K, generator=g)).to(dt).to(DEV)
    S = kernels.splitk_slices(N, K)
    assert 1 <= S <= 16
    part = kernels.linear_splitk(x, W)
    assert part.shape == (S, M, N)
    exact = (x.double() @ W.double().T)
    got = part.double().sum(0)
    err = (got - exact).abs().max().item() / exact.abs().max().item()
    assert err < 1e-5, err
    # rows are independent of each other: a sub-batch gives the same bits
    sub = kernels.linear_splitk(x[M // 2:].contiguous(), W)
    assert torch.equal(sub, part[:, M // 2:])


@pytest.mark.parametrize("M,H", [(32, 896), (64, 2048), (3, 128), (160, 2048)])
def test_residual_norm_matches_add_then_rmsnorm(gpu_lib, M, H):
    g = torch.Generator().manual_seed(M * H)
    dt = torch.bfloat16
    S = 5
    part = torch.randn(S, M, H, generator=g).to(DEV)
    res = torch.randn(M, H, generator=g).to(dt).to(DEV)
    nw = (1 + 0.1 * torch.randn(H, generator=g)).to(dt).to(DEV)
    acc = part[0].clone()
    for s in range(1, S):
        acc = acc + part[s]
    want_r = res + acc.to(dt)
    want_x = kernels.rmsnorm(want_r, nw, 1e-6)
    r = res.clone()
    xn = kernels.residual_norm(part, S, r, nw, 1e-6)
    assert torch.equal(r, want_r)
    dist = ulps_apart(xn, want_x)
    assert dist.max().item() <= 1 and (dist > 0).float().mean().item() < 0.01


def test_kv_slots_resolve_block_and_offset(gpu_lib):
    B, T, bs, width = 4, 3, 4, 5
    tables = torch.tensor([[7, 2, 9, -1, -1], [1, 3, -1, -1, -1], [0, 4, 5, 6, 8], [11, 12, 13, 14, 15]],
                          dtype=torch.int32)
    start = torch.tensor([5, 0, 17, 3], dtype=torch.int32)
    q_lens = torch.tensor([3, 2, 3, 0], dtype=torch.int32)
    got = kernels.kv_slots(tables.to(DEV), start.to(DEV), B, T, bs, 14, q_lens=q_lens.to(DEV)).cpu()
    want = []
    for i in range(B):
        for t in range(T):
            pos = int(start[i]) + t
            blk = int(tables[i, pos // bs]) if t < q_lens[i] and pos // bs < width else -1
            want.append(blk * bs + pos % bs if 0 <= blk < 14 else -1)
    assert got.tolist() == want


@pytest.mark.parametrize("arch", [TINY, TINY128], ids=["d64", "d128"])
@pytest.mark.parametrize("B,T", [(3, 5), (32, 2), (7, 1)])
def test_qkv_rope_matches_unfused(gpu_lib, arch, B, T):
    g = torch.Generator().manual_seed(7)
    H, Hq, Hkv, D = arch.hidden, arch.num_q_heads, arch.num_kv_heads, arch.head_dim
    dt = torch.bfloat16
    res = torch.randn(B, T, H, generator=g).to(dt).to(DEV)
    nw = (1 + 0.1 * torch.randn(H, generator=g)).to(dt).to(DEV)
    W = (0.05 * torch.randn((Hq + 2 * Hkv) * D, H, generator=g)).to(dt).to(DEV)
    bias = (0.1 * torch.randn((Hq + 2 * Hkv) * D, generator=g)).to(dt).to(DEV)
    rot = RotaryEmbedding(D, 1e6).to(DEV)
    start = torch.randint(0, 40, (B,), generator=g, dtype=torch.int32).to(DEV)
    pos = start.long()[:, None] + torch.arange(T, device=DEV)[None]
    cos, sin = rot(res, pos)
    cos, sin = cos.contiguous(), sin.contiguous()
    nb, bs, width = 4 * B + 8, 16, 4
    perm = torch.randperm(nb, generator=g)[: B * width].view(B, width).to(torch.int32).to(DEV)
    q_lens = torch.randint(1, T + 1, (B,), generator=g, dtype=torch.int32).to(DEV)
    pools = [(torch.zeros(nb, Hkv, bs, D, dtype=dt, device=DEV),
              torch.zeros(nb, Hkv, D, bs, dtype=dt, device=DEV)) for _ in range(2)]
    h = kernels.rmsnorm(res, nw, 1e-6)
    q_ref = kernels.rope_kv_write(F.linear(h, W, bias), cos, sin, *pools[0], perm, start, Hq,
                                  q_lens=q_lens)
    slots = kernels.kv_slots(perm, start, B, T, bs, nb, q_lens=q_lens)
    q = kernels.qkv_rope(h, W, bias, cos, sin, slots, *pools[1], Hq)
    close_bf16(q, q_ref)
    close_bf16(pools[1][0], pools[0][0])
    close_bf16(pools[1][1], pools[0][1])
    assert torch.equal(pools[1][0] == 0, pools[0][0] == 0)
    # the wide layer's form: k-slice partials, then sum + bias + RoPE + KV write
    pool3 = (torch.zeros_like(pools[0][0]), torch.zeros_like(pools[0][1]))
    part = kernels.linear_splitk(h, W)
    q3 = kernels.qkv_part_rope(part, bias, cos, sin, slots, *pool3, Hq, B * T).view(B, T, Hq, D)
    close_bf16(q3, q_ref)
    close_bf16(pool3[0], pools[0][0])
    close_bf16(pool3[1], pools[0][1])
    assert torch.equal(pool3[0] == 0, pools[0][0] == 0)
    # rows are independent: the first rows alone give the same bits
    n = max(1, (B * T) // 2)
    pool4 = (torch.zeros_like(pools[0][0]), torch.zeros_like(pools[0][1]))
    q4 = kernels.qkv_part_rope(kernels.linear_splitk(h.view(B * T, H)[:n].contiguous(), W), bias,
                               cos.view(B * T, D)[:n].contiguous(), sin.view(B * T, D)[:n].contiguous(),
                               slots[:n].contiguous(), *pool4, Hq, n)
    assert torch.equal(q4, q3.view(B * T, Hq, D)[:n])


@pytest.mark.parametrize("M,H,Fd", [(32, 896, 4864), (64, 896, 4864), (9, 128, 256), (20, 2048, 11008),
                                    (160, 2048, 11008), (97, 896, 4864), (130, 128, 256),
                                    (100, 128, 96), (150, 256, 224), (5, 2048, 11008),
                                    (40, 2048, 11008), (64, 2048, 11008), (100, 2048, 11008),
                                    (12, 1024, 8192)])
def test_gate_up_silu_matches_unfused(gpu_lib, M, H, Fd):
    """Every tile shape: 32-pair tiles (narrow widths, 1-4 row tiles), 48-pair
    tiles on 6 waves (wide widths at 1-4 row tiles) and on 12 waves (6-10 row
    tiles), the last workgroup of a width that 48 does not divide (11008: 16
    pairs, 8192: 32), 64-row tiles (widths not a multiple of 64)."""
    g = torch.Generator().manual_seed(M + H + 1)
    dt = torch.bfloat16
    h = kernels.rmsnorm(torch.randn(M, H, generator=g).to(dt).to(DEV),
                        (1 + 0.1 * torch.randn(H, generator=g)).to(dt).to(DEV), 1e-6)
    W = (0.05 * torch.randn(2 * Fd, H, generator=g)).to(dt).to(DEV)
    want = kernels.silu_mul(F.linear(h, W))
    got = kernels.gate_up_silu(h, W)
    close_bf16(got, want)
    # a row's bits do not depend on how many rows share the launch
    assert torch.equal(kernels.gate_up_silu(h[M // 3:].contiguous(), W), got[M // 3:])


@pytest.mark.parametrize("arch", [TINY, TINY128], ids=["d64", "d128"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_packed_prefill_matches_padded_forward(gpu_lib, arch, dtype):
    """The engine's packed prefill (projections on the real tokens only, RoPE /
    KV write / attention on the padded [B, T] layout) against the padded
    forward over the same ragged batch: same hidden states for every real
    token and the same K/V in the pool, on top of a history of different
    lengths per sequence."""
    from kvengine_amd.forward import forward_packed

    model = build_model(arch, generate_state_dict(arch, seed=12), dtype=dtype, device=DEV)
    g = torch.Generator().manual_seed(12)
    hist = [9, 1, 33, 17, 4]
    new = [37, 5, 120, 64, 1]
    B, T = len(new), max(new)
    out = []
    for packed in (True, False):
        pool = PagedKVCache.for_model(model, 64, 16, max_seqs=8)
        seqs = [pool.new_sequence(i) for i in range(B)]
        rows = torch.tensor([s.row for s in seqs], dtype=torch.int32, device=DEV)
        gh = torch.Generator().manual_seed(5)
        hid = torch.randint(0, arch.vocab, (B, max(hist)), generator=gh).to(DEV)
        for s, n, m in zip(seqs, hist, new):
            s.reserve(n + m)
        qh = torch.tensor(hist, dtype=torch.int32, device=DEV)
        forward_hidden(model, hid, pool.device_kv(), rows, max(hist), q_lens=qh, fused=True)
        for s, n in zip(seqs, hist):
            s.commit(n)
        ids = torch.randint(0, arch.vocab, (B, T), generator=torch.Generator().manual_seed(7))
        ql = torch.tensor(new, dtype=torch.int32, device=DEV)
        max_ctx = max(h + n for h, n in zip(hist, new))
        if packed:
            flat = torch.cat([ids[b, :n] for b, n in enumerate(new)]).to(DEV)
            dst = torch.cat([torch.arange(n) + b * T for b, n in enumerate(new)]).to(DEV)
            h = forward_packed(model, flat, dst, B, T, pool.device_kv(), rows, max_ctx, ql)
        else:
            hp = forward_hidden(model, ids.to(DEV), pool.device_kv(), rows, max_ctx, q_lens=ql,
                                fused=True)
            h = torch.cat([hp[b, :n] for b, n in enumerate(new)])
        torch.cuda.synchronize()
        out.append((h, pool.k.clone(), pool.v.clone()))
    (h1, k1, v1), (h2, k2, v2) = out
    assert h1.shape == h2.shape == (sum(new), arch.hidden)
    if dtype == torch.float32:
        assert (h1 - h2).abs().max().item() < 1e-4
        assert (k1 - k2).abs().max().item() < 1e-4 and (v1 - v2).abs().max().item() < 1e-4
    else:
        close_bf16(h1, h2, rel=2 ** -5, frac=0.2)
        close_bf16(k1, k2, rel=2 ** -5, frac=0.2)
        close_bf16(v1, v2, rel=2 ** -5, frac=0.2)


# ---- many-row projections (prefill) with the split-K layer's sums ---------------

def _splitk_rows_reference(x, W, mode, chunk=160):
    """What the split-K kernels give each row, in passes of at most `chunk` rows:
    slices summed in the reduction kernels' order (mode 0: t0 + t1 + ..., mode
    1: 0 + t0 + t1 + ...), or gate_up_silu's act (mode 2)."""
    outs = []
    for a in range(0, x.shape[0], chunk):
        xs = x[a:a + chunk].contiguous()
        if mode == kernels.ROWS_GATE_UP:
            outs.append(kernels.gate_up_silu(xs, W))
            continue
        part = kernels.linear_splitk(xs, W)
        t = part[0].clone() if mode == kernels.ROWS_RESIDUAL else torch.zeros_like(part[0]) + part[0]
        for s in range(1, part.shape[0]):
            t += part[s]
        outs.append(t)
    return torch.cat(outs)


@pytest.mark.parametrize("M,N,K,mode", [
    (300, 2048, 2048, 0), (1000, 2048, 11008, 0), (4100, 2048, 2048, 0), (161, 896, 4864, 0),
    (1, 896, 896, 0), (700, 2560, 2048, 1), (3500, 2560, 2048, 1), (200, 1152, 896, 1),
    (129, 1152, 128, 1), (500, 22016, 2048, 2), (300, 9728, 896, 2), (37, 512, 128, 2)])
def test_linear_rows_is_the_splitk_layer_bit_for_bit(gpu_lib, M, N, K, mode):
    """kve_linear_rows gives every row the bits the split-K kernels give it in a
    pass of at most 160 rows (3B and 0.5B projection shapes, 1 to 4100 rows; the
    whole sum or every slice, as the row count decides)."""
    g = torch.Generator().manual_seed(M + N + K + mode)
    dt = torch.bfloat16
    x = torch.randn(M, K, generator=g).to(dt).to(DEV)
    W = (0.03 * torch.randn(N, K, generator=g)).to(dt).to(DEV)
    got = kernels.linear_rows(x, W, mode)
    want = _splitk_rows_reference(x, W, mode)
    if mode == kernels.ROWS_GATE_UP:
        assert got.shape == (M, N // 2)
        assert torch.equal(got, want)
        return
    S = got.shape[0]
    assert got.shape[1:] == (M, N) and S in (1, kernels.splitk_slices(N, K))
    if S > 1:
        # every slice as linear_splitk writes it (it is row-independent)
        assert torch.equal(got[:, :160], kernels.linear_splitk(x[:160].contiguous(), W))
    t = got[0].clone() if mode == kernels.ROWS_RESIDUAL else torch.zeros_like(got[0]) + got[0]
    for s in range(1, S):
        t += got[s]
    assert torch.equal(t, want)
    exact = x.double() @ W.double().T
    err = (t.double() - exact).abs().max().item() / exact.abs().max().item()
    assert err < 1e-5, err


def test_linear_rows_takes_both_forms(gpu_lib):
    lib = gpu_lib
    assert lib.kve_linear_rows_slices(300, 2048, 2048, 0) == kernels.splitk_slices(2048, 2048)
    assert lib.kve_linear_rows_slices(5400, 2048, 2048, 0) == 1
    assert lib.kve_linear_rows_slices(10, 22016, 2048, 2) == 1


def test_linear_rows_rejects_what_it_cannot_tile(gpu_lib):
    x = torch.zeros(300, 2048, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_lib.KveError, match="multiple of 128"):
        kernels.linear_rows(x, torch.zeros(2000, 2048, dtype=torch.bfloat16, device=DEV), 0)
    with pytest.raises(_lib.KveError, match="multiple of 64"):
        kernels.linear_rows(x[:, :2016].contiguous(),
                            torch.zeros(2048, 2016, dtype=torch.bfloat16, device=DEV), 0)


def _prefill_wide(model, pool, seqs, toks, attn):
    from kvengine_amd.forward import forward_packed_wide

    B, T = len(seqs), max(len(t) for t in toks)
    flat, dst = [], []
    for j, t in enumerate(toks):
        flat += t
        dst += range(j * T, j * T + len(t))
    for s, t in zip(seqs, toks):
        s.reserve(len(t))
    rows = torch.tensor([s.row for s in seqs], dtype=torch.int32, device=DEV)
    q_lens = torch.tensor([len(t) for t in toks], dtype=torch.int32, device=DEV)
    max_ctx = max(s.length for s in seqs) + T
    h = forward_packed_wide(model, torch.tensor(flat, device=DEV), torch.tensor(dst, device=DEV),
                            B, T, pool.device_kv(), rows, max_ctx, q_lens, attn_order=attn)
    for s, t in zip(seqs, toks):
        s.commit(len(t))
    return h


@pytest.mark.parametrize("order", ["short", "long"])
@pytest.mark.parametrize("arch", [TINY, TINY128], ids=["d64", "d128"])
def test_wide_prefill_equals_verify_passes(gpu_lib, arch, order):
    """A packed prefill through the wide layer (kve_linear_rows above 160 rows)
    writes the same K/V bits and gives the same hidden states as feeding each
    sequence in verify-shaped windows of 5 tokens through the wide split-K
    layer, at a fixed attention order: the recompute of a preempted request
    reproduces what its verify passes wrote. Both of the engine's target
    orders: 8-block units (histories crossing up to two unit boundaries) and
    the 16-block units it takes past 4096 tokens (histories of up to 620
    tokens, crossing two 256-token unit boundaries, so the merge of several
    units is compared too)."""
    model = build_model(arch, generate_state_dict(arch, seed=12), dtype=torch.bfloat16, device=DEV)
    g = torch.Generator().manual_seed(4)
    from kvengine_amd.engine import TARGET_ATTN, TARGET_ATTN_LONG

    lens = [203, 37, 5, 170, 1] if order == "short" else [620, 37, 5, 300, 1]
    toks = [torch.randint(0, arch.vocab, (n,), generator=g).tolist() for n in lens]
    attn = TARGET_ATTN if order == "short" else TARGET_ATTN_LONG
    pa = PagedKVCache.for_model(model, 128, 16, max_seqs=8)
    pb = PagedKVCache.for_model(model, 128, 16, max_seqs=8)
    sa = [pa.new_sequence(i) for i in range(len(lens))]
    sb = [pb.new_sequence(i) for i in range(len(lens))]
    # a first part through the windows in both pools, so the prefill starts mid-sequence too
    head = 7
    hb = [[] for _ in lens]
    for j, (s, t) in enumerate(zip(sb, toks)):
        for a in range(0, len(t), 5):
            w = t[a:a + 5]
            s.reserve(len(w))
            rows = torch.tensor([s.row], dtype=torch.int32, device=DEV)
            h = forward_hidden(model, torch.tensor([w], device=DEV), pb.device_kv(), rows,
                               s.length + len(w), attn_order=attn, fused=True, gemm_rows=160)
            s.commit(len(w))
            hb[j].append(h[0])
    for s, t in zip(sa, toks):
        if len(t) > head:
            _prefill_wide(model, pa, [s], [t[:head]], attn)
    rest = [t[head:] if len(t) > head else t for t in toks]
    ha = _prefill_wide(model, pa, sa, rest, attn)
    off = 0
    for j, t in enumerate(toks):
        want = torch.cat(hb[j])[len(t) - len(rest[j]):]
        assert torch.equal(ha[off:off + len(rest[j])], want), f"sequence {j} hidden states"
        off += len(rest[j])
        for li in range(arch.num_layers):
            ka, va = sa[j]._gather(li, len(t))
            kb, vb = sb[j]._gather(li, len(t))
            assert torch.equal(ka, kb) and torch.equal(va, vb), f"sequence {j} layer {li} K/V"


def test_pass_prologue_is_the_torch_ops(gpu_lib):
    """kve_pass_prologue: the embedding rows and RoPE cos/sin of a pass's
    tokens, bit-identical to embed_tokens + rotary_emb's table lookup; ids
    outside the vocabulary give zero rows; positions past the table clamp; a
    sequence row outside the lengths table (-1, or past its end) is not read
    and its tokens take positions 0, 1, ..."""
    model = build_model(TINY128, generate_state_dict(TINY128, seed=5), dtype=torch.bfloat16,
                        device=DEV)
    inner = model.model
    B, T = 5, 3
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, TINY128.vocab, (B, T), generator=g).to(DEV)
    ids[2, 1] = TINY128.vocab + 5
    ids[4, 0] = -1
    lens = torch.tensor([0, 7, 100, 4093, 30, 0, 0, 0], dtype=torch.int32, device=DEV)
    rows = torch.tensor([1, 0, 2, 3, 4], dtype=torch.int32, device=DEV)
    emb = inner.embed_tokens.weight
    cos_t, sin_t = inner.rotary_emb.table(emb, 4096)
    h, c, s = kernels.pass_prologue(ids, emb, lens, rows, cos_t, sin_t)
    valid = (ids >= 0) & (ids < TINY128.vocab)
    want_h = inner.embed_tokens(ids.clamp(0, TINY128.vocab - 1)) * valid[..., None]
    pos = lens.index_select(0, rows).long()[:, None] + torch.arange(T, device=DEV)[None]
    want_c, want_s = inner.rotary_emb(emb, pos, 4096)
    assert torch.equal(h, want_h)
    assert torch.equal(c, want_c) and torch.equal(s, want_s)
    # rows outside the lengths table: the embedding rows are unchanged, the
    # positions start at 0
    bad = torch.tensor([1, -1, 2, 8, 4], dtype=torch.int32, device=DEV)
    h2, c2, s2 = kernels.pass_prologue(ids, emb, lens, bad, cos_t, sin_t)
    assert torch.equal(h2, want_h)
    lens_b = torch.cat([lens, torch.zeros(1, dtype=torch.int32, device=DEV)])
    pos2 = lens_b.index_select(0, torch.where((bad >= 0) & (bad < 8), bad, 8).long()).long()
    want_c2, want_s2 = inner.rotary_emb(emb, pos2[:, None] + torch.arange(T, device=DEV)[None], 4096)
    assert torch.equal(c2, want_c2) and torch.equal(s2, want_s2)


@pytest.mark.parametrize("path", ["splitk", "fused", "wide"])
def test_decode_paths_match_the_oracle_on_a_3b_slice(gpu_lib, path):
    """Each bf16 layer path (split-K decode layer, fused decode layer, wide
    split-K layer) on the first two layers of the 3B architecture against the
    oracle's CPU forward (oracle/model.py, pinned to the reference's fixtures)
    over the same 40-token prompt: the K/V every layer writes and the final
    logits. Layer 0's K/V differ from the oracle's only by the rounding of
    a differently ordered fp32 sum (at most one bf16 ulp, on few elements);
    the logits at the oracle's top-8 ids stay within the reference's own
    verify/decode spread (TOL_ULPS)."""
    from kvengine_amd import forward as fwd
    from kvengine_amd.arch import QWEN25_3B, layer_slice
    from kvengine_amd.margins import TOL_ULPS, bf16_ulp
    from oracle.model import RefQwen2
    from oracle.paged import RefPagedKVCache

    arch = layer_slice(QWEN25_3B, 2)
    sd = generate_state_dict(arch, seed=1, dtype=torch.bfloat16)
    ids = torch.randint(0, arch.vocab, (1, 40), generator=torch.Generator().manual_seed(9))
    ref = RefQwen2(arch, sd, dtype=torch.bfloat16)
    rc = RefPagedKVCache(arch.num_layers, arch.num_kv_heads, arch.head_dim, 8, 16, torch.bfloat16)
    rseq = rc.new_sequence("r")
    ref_logits = ref.forward(ids, rseq)[0, -1].float()

    model = build_model(arch, sd, dtype=torch.bfloat16, device=DEV)
    pool = PagedKVCache.for_model(model, 8, 16)
    seq = pool.new_sequence("g")
    seq.reserve(40)
    prev = fwd.SMALL_BATCH_PATH
    fwd.SMALL_BATCH_PATH = "fused" if path == "fused" else "splitk"
    try:
        hid = forward_hidden(model, ids.to(DEV), pool.device_kv(), seq.row_dev, 40,
                             gemm_rows=160 if path == "wide" else None)
    finally:
        fwd.SMALL_BATCH_PATH = prev
    seq.commit(40)
    logits = model.lm_head(hid[:, -1:])[0, 0].float().cpu()
    for li in range(arch.num_layers):
        kr, vr = rseq.gather(li, 40)
        kg, vg = seq._gather(li, 40)
        for name, a, b in (("K", kg.cpu(), kr), ("V", vg.cpu(), vr)):
            a, b = a.reshape(-1, arch.head_dim).float(), b.reshape(-1, arch.head_dim).float()
            assert a.shape == b.shape
            if li == 0:
                # elementwise: the same bf16 value or its neighbour
                ulp = torch.tensor([bf16_ulp(x) for x in b.reshape(-1).abs().clamp(min=2 ** -30).tolist()])
                d = (a.reshape(-1) - b.reshape(-1)).abs() / ulp
                assert d.max().item() <= 1.0, f"layer 0 {name}: {d.max().item()} ulps"
                assert (d > 0).float().mean().item() < 0.05, f"layer 0 {name}"
            else:
                # per (token, head) row, in ulps of the row's largest value
                ulp = torch.tensor([bf16_ulp(x) for x in b.abs().amax(-1).tolist()])
                d = (a - b).abs().amax(-1) / ulp
                assert d.max().item() <= TOL_ULPS, f"layer {li} {name}: {d.max().item()} ulps"
    top = torch.topk(ref_logits, 8)
    u = bf16_ulp(top.values[0].item())
    diff = (logits[top.indices] - top.values).abs().max().item() / u
    assert diff <= TOL_ULPS, diff


# ---- blocked operand layout -----------------------------------------------------

@pytest.mark.parametrize("M", [5, 33, 160])
def test_blocked_projections_equal_row_major(gpu_lib, M):
    """The projections, the reductions that feed them and the LM head give the
    same bits with blocked operands (16 x 32 blocks) as with row-major ones."""
    g = torch.Generator().manual_seed(M)
    dt = torch.bfloat16
    H, Fd, N = 896, 4864, 1152
    x = torch.randn(M, H, generator=g).to(dt).to(DEV)
    xb = kernels.to_blocked(x)
    W = (0.03 * torch.randn(N, H, generator=g)).to(dt).to(DEV)
    assert torch.equal(kernels.linear_splitk(xb, kernels.to_blocked(W), blocked=True, rows=M),
                       kernels.linear_splitk(x, W))
    Wgu = (0.03 * torch.randn(2 * Fd, H, generator=g)).to(dt).to(DEV)
    act = kernels.gate_up_silu(xb, kernels.to_blocked(Wgu), blocked=True, rows=M)
    want = kernels.gate_up_silu(x, Wgu)
    assert torch.equal(kernels.from_blocked(act, M), want)
    Wd = (0.03 * torch.randn(H, Fd, generator=g)).to(dt).to(DEV)
    assert torch.equal(kernels.linear_splitk(act, kernels.to_blocked(Wd), blocked=True, rows=M),
                       kernels.linear_splitk(want, Wd))
    part = kernels.linear_splitk(want, Wd)
    nw = (1 + 0.1 * torch.randn(H, generator=g)).to(dt).to(DEV)
    r1, r2 = x.clone(), x.clone()
    xn1 = kernels.residual_norm(part, part.shape[0], r1, nw, 1e-6)
    xn2 = kernels.residual_norm(part, part.shape[0], r2, nw, 1e-6, blocked=True)
    assert torch.equal(r1, r2) and torch.equal(kernels.from_blocked(xn2, M), xn1)
    assert torch.equal(kernels.from_blocked(kernels.rmsnorm(x, nw, 1e-6, blocked=True), M),
                       kernels.rmsnorm(x, nw, 1e-6))
    if M <= 64:
        # the fused kernels' register-loaded weight fragments, blocked or not
        Wo = (0.03 * torch.randn(H, 896, generator=g)).to(dt).to(DEV)
        xo = torch.randn(M, 896, generator=g).to(dt).to(DEV)
        r1, r2 = x.clone(), x.clone()
        kernels.linear_residual(xo, Wo, r1)
        kernels.linear_residual(xo, kernels.to_blocked(Wo), r2, blocked_w=True)
        assert torch.equal(r1, r2)
        assert torch.equal(kernels.fused_gate_up(x, nw, 1e-6, kernels.to_blocked(Wgu), blocked_w=True),
                           kernels.fused_gate_up(x, nw, 1e-6, Wgu))
    V = 151936 // 8
    Wv = (0.05 * torch.randn(V, H, generator=g)).to(dt).to(DEV)
    outs = []
    for blk in (False, True):
        mx = torch.empty(M, dtype=torch.float32, device=DEV)
        sid = torch.empty(M, dtype=torch.int32, device=DEV)
        sv = torch.empty(M, dtype=torch.float32, device=DEV)
        am, mx = kernels.lmhead_argmax(xb if blk else x, kernels.to_blocked(Wv) if blk else Wv,
                                       maxval=mx, second_id=sid, second_val=sv, blocked=blk, rows=M)
        outs.append((am, mx, sid, sv))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("arch", [TINY, TINY128], ids=["d64", "d128"])
def test_blocked_layers_equal_row_major_layers(gpu_lib, arch):
    """A forward pass on blocked operands (the split-K decode layer at 24 x 1
    rows, the wide layer at 32 x 5) gives the hidden states of the row-major
    one bit for bit, and blocked_out hands back the same rows blocked."""
    from kvengine_amd import forward as fwd

    model = build_model(arch, generate_state_dict(arch, seed=4), dtype=torch.bfloat16, device=DEV)
    assert getattr(model.model.layers[0].self_attn, "qkv_weight_blk", None) is not None
    for B, T, gr in ((24, 1, None), (32, 5, 160), (3, 5, 160), (4, 1, None)):
        ids = torch.randint(0, arch.vocab, (B, T), generator=torch.Generator().manual_seed(B)).to(DEV)
        # 4 x 1 rows without gemm_rows take the fused path: blocked weights,
        # row-major activations
        split = gr is not None or B * T > fwd.FUSED_MAX_ROWS
        assert fwd.blocked_forward(model, B * T, gr) == split
        got = _forward_rows(model, ids, gemm_rows=gr)
        prev = fwd.BLOCKED_LAYERS
        fwd.BLOCKED_LAYERS = False
        try:
            want = _forward_rows(model, ids, gemm_rows=gr)
        finally:
            fwd.BLOCKED_LAYERS = prev
        assert torch.equal(got, want), (B, T)
        if not split:
            continue
        pool = PagedKVCache.for_model(model, max(16, B * -(-T // 4) + 4), 4, max_seqs=max(B, 8))
        seqs = [pool.new_sequence(i) for i in range(B)]
        for s in seqs:
            s.reserve(T)
        rows = torch.tensor([s.row for s in seqs], dtype=torch.int32, device=DEV)
        hb = forward_hidden(model, ids, pool.device_kv(), rows, T, fused=True, gemm_rows=gr,
                            blocked_out=True)
        assert torch.equal(kernels.from_blocked(hb, B * T), want.reshape(B * T, -1))


@pytest.mark.parametrize("M,N,K,mode", [(300, 2048, 2048, 0), (161, 896, 4864, 0), (700, 2560, 2048, 1),
                                        (500, 22016, 2048, 2), (37, 512, 128, 2), (1000, 2048, 11008, 0)])
def test_blocked_linear_rows_equals_row_major(gpu_lib, M, N, K, mode):
    """kve_linear_rows on blocked operands gives the row-major launch's bits (the
    prefill's projections), whole sums or slices alike."""
    g = torch.Generator().manual_seed(M + N + mode)
    dt = torch.bfloat16
    x = torch.randn(M, K, generator=g).to(dt).to(DEV)
    W = (0.03 * torch.randn(N, K, generator=g)).to(dt).to(DEV)
    want = kernels.linear_rows(x, W, mode)
    got = kernels.linear_rows(kernels.to_blocked(x), kernels.to_blocked(W), mode, blocked=True, rows=M)
    if mode == kernels.ROWS_GATE_UP:
        got = kernels.from_blocked(got, M)
    assert torch.equal(got, want)
