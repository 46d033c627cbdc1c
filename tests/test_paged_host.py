"""Host bookkeeping of the paged cache (no kernels): runs with device tables on the CPU.

Restates the reference's truncate and allocation expectations
(tests/test_phase5.py:220-237, tests/test_phase2.py:157-214) and checks that
the device-side table rows and lengths mirror the host lists after every call.
"""

import pytest
import torch

from kvengine_amd.blocks import OutOfBlocks
from kvengine_amd.paged import ContiguousKVCache, KVCacheFull, PagedKVCache
from oracle.paged import RefPagedKVCache


def pool(num_blocks=32, bs=4, max_seqs=8):
    return PagedKVCache(2, 2, 64, num_blocks, bs, torch.float32, "cpu", max_seqs=max_seqs)


def mirrored(seq):
    row = seq.pool.tables[seq.row].tolist()
    return (row[: len(seq.blocks)] == seq.blocks and all(x == -1 for x in row[len(seq.blocks):])
            and seq.pool.lens[seq.row].item() == seq.length)


def test_truncate_frees_whole_blocks_only():
    p = pool()
    seq = p.new_sequence("t")
    seq.reserve(16)
    seq.commit(16)
    assert len(seq.blocks) == 4 and mirrored(seq)
    seq.truncate(9)
    assert seq.length == 9 and len(seq.blocks) == 3 and p.manager.num_free == 29 and mirrored(seq)
    seq.truncate(8)
    assert len(seq.blocks) == 2 and mirrored(seq)
    seq.truncate(0)
    assert len(seq.blocks) == 0 and mirrored(seq)
    p.manager.check_invariants()
    with pytest.raises(ValueError):
        seq.truncate(1)


def test_reserve_is_lazy_and_atomic():
    p = pool(num_blocks=4, bs=4)
    seq = p.new_sequence("a")
    seq.reserve(3)
    seq.commit(3)
    assert len(seq.blocks) == 1
    seq.reserve(1)
    seq.commit(1)
    assert len(seq.blocks) == 1, "allocated while the block had room"
    seq.reserve(1)
    assert len(seq.blocks) == 2
    other = p.new_sequence("b")
    with pytest.raises(OutOfBlocks):
        other.reserve(9)
    assert p.manager.num_allocated == 2 and not other.blocks
    p.manager.check_invariants()


def test_same_allocation_order_as_reference():
    """Interleaved reserve/commit/truncate/free: identical tables to the oracle's."""
    import random

    rng = random.Random(3)
    mine, ref = pool(num_blocks=48, bs=4, max_seqs=16), RefPagedKVCache(1, 2, 8, 48, 4, torch.float32)
    seqs_m, seqs_r = {}, {}
    for step in range(600):
        op = rng.random()
        name = rng.randrange(6)
        if name not in seqs_m:
            seqs_m[name], seqs_r[name] = mine.new_sequence(name), ref.new_sequence(name)
        a, b = seqs_m[name], seqs_r[name]
        if op < 0.5:
            n = rng.randint(1, 9)
            try:
                a.reserve(n)
            except OutOfBlocks:
                with pytest.raises(Exception):
                    b.reserve(n)
                continue
            b.reserve(n)
            a.commit(n)
            b.commit(n)
        elif op < 0.85:
            n = rng.randint(0, a.length)
            a.truncate(n)
            b.truncate(n)
        else:
            a.free()
            b.free()
            del seqs_m[name], seqs_r[name]
            continue
        assert a.blocks == b.blocks and a.length == b.length, f"step {step}"
        assert mirrored(a)
    mine.manager.check_invariants()


def test_prefix_adopt_and_shared_rollback_refusal():
    p = pool(num_blocks=16, bs=4)
    toks = list(range(100, 113))  # 13 tokens -> 3 full blocks
    a = p.new_sequence("a")
    a.reserve(13)
    a.commit(13)
    assert a.register_prefix_blocks(toks) == 3
    b = p.new_sequence("b")
    assert b.adopt_prefix(toks) == 12
    assert b.blocks == a.blocks[:3] and mirrored(b)
    assert p.manager.refcount(a.blocks[0]) == 2
    with pytest.raises(ValueError):
        a.truncate(5)  # would reach into a block b shares
    b.free()
    a.truncate(5)
    assert mirrored(a)
    p.manager.check_invariants()


def test_rows_are_recycled():
    p = pool(max_seqs=2)
    s1, s2 = p.new_sequence(1), p.new_sequence(2)
    s1.reserve(1)
    s2.reserve(1)
    with pytest.raises(RuntimeError):
        p.new_sequence(3).reserve(1)
    s1.free()
    s3 = p.new_sequence(3)
    s3.reserve(2)
    assert mirrored(s3)


def test_contiguous_cache_contract():
    c = ContiguousKVCache(2, 2, 64, 8, torch.float32, "cpu")
    c.reserve(8)
    c.commit(8)
    with pytest.raises(KVCacheFull):
        c.reserve(1)
    c.truncate(3)
    assert c.length == 3 and c.lens.item() == 3
    with pytest.raises(ValueError):
        c.truncate(4)


# ---------------------------------------------------------------- prefill batching

def _brute_partitions(n):
    """Every way to cut range(n) into consecutive non-empty groups."""
    if n == 0:
        yield []
        return
    for first in range(1, n + 1):
        for rest in _brute_partitions(n - first):
            yield [(0, first)] + [(a + first, b + first) for a, b in rest]


def test_prefill_partition_is_the_cheapest_cut():
    """The engine's prefill grouping minimises sum(fixed + count * longest)
    under the row cap; checked against every cut of small sorted inputs."""
    import random

    from kvengine_amd.engine import _partition_by_cost

    rng = random.Random(5)
    for _ in range(200):
        n = rng.randint(1, 8)
        lens = sorted((rng.randint(1, 400) for _ in range(n)), reverse=True)
        fixed = rng.choice([0, 50, 800, 5000])
        cap = rng.choice([10**9, 900])

        def cost(groups):
            return sum(fixed + (b - a) * lens[a] for a, b in groups)

        def ok(groups):
            return all((b - a) * lens[a] <= cap or b - a == 1 for a, b in groups)

        got = _partition_by_cost(lens, fixed, cap)
        assert [a for a, _ in got] == [0] + [b for _, b in got[:-1]] and got[-1][1] == n
        assert ok(got)
        assert cost(got) == min(cost(g) for g in _brute_partitions(n) if ok(g))


def test_prefill_partition_edge_cases():
    from kvengine_amd.engine import _partition_by_cost

    assert _partition_by_cost([], 100, 8192) == []
    assert _partition_by_cost([7], 100, 8192) == [(0, 1)]
    # an item longer than the cap still gets a batch of its own
    assert _partition_by_cost([9000, 10], 100, 8192) == [(0, 1), (1, 2)]
    # no fixed cost: no padding at all pays, every length alone
    assert _partition_by_cost([5, 4, 3], 0, 8192) == [(0, 1), (1, 2), (2, 3)]
    # a large fixed cost: one batch
    assert _partition_by_cost([5, 4, 3], 10**6, 8192) == [(0, 3)]


def test_packed_prefill_groups_respect_both_caps():
    from kvengine_amd.engine import _packed_groups

    rng = __import__("random").Random(8)
    for _ in range(300):
        lens = sorted((rng.randint(1, 500) for _ in range(rng.randint(0, 40))), reverse=True)
        real_cap, pad_cap = rng.choice([(8192, 32768), (600, 32768), (8192, 900)])
        groups = _packed_groups(lens, real_cap, pad_cap)
        assert not groups or [a for a, _ in groups] == [0] + [b for _, b in groups[:-1]]
        assert (groups[-1][1] if groups else 0) == len(lens)
        for a, b in groups:
            if b - a > 1:
                assert sum(lens[a:b]) <= real_cap and (b - a) * lens[a] <= pad_cap
            # greedy: the next item would not have fitted
            if b < len(lens):
                assert sum(lens[a:b + 1]) > real_cap or (b + 1 - a) * lens[a] > pad_cap
