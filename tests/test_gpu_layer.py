"""Fused layer kernels against the torch op sequences they replace.

Elementwise kernels (RoPE + KV write, SiLU*up) round at exactly the points the
torch ops do, so they must agree bit for bit. RMSNorm's mean is a float32 sum
in a different order, which may move the float32 result by an ulp and,
rarely, the rounded model-dtype output by one ulp; that is bounded here.
"""

import pytest
import torch
import torch.nn.functional as F

from kvengine_amd import kernels
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
