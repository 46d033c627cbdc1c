"""Block allocator: the reference's known-answer tests, for the product and the oracle.

Restated from the reference's tests/test_blocks.py:15-210 and the allocator half
of tests/test_phase6.py:40-222; both implementations must pass every one, and a
differential churn test checks they hand out identical block ids.
"""

import random

import pytest

from kvengine_amd import blocks as prod
from oracle import blocks as orc

IMPLS = [
    pytest.param((prod.BlockManager, prod.OutOfBlocks, prod.DoubleFree, prod.chain_digest,
                  prod.ROOT_DIGEST), id="product"),
    pytest.param((orc.RefBlockManager, orc.OutOfBlocks, orc.DoubleFree, orc.chain_digest,
                  orc.ROOT_DIGEST), id="oracle"),
]


@pytest.fixture(params=IMPLS)
def impl(request):
    return request.param


def test_starts_fully_free(impl):
    BM = impl[0]
    m = BM(8, 16)
    assert m.num_free == 8 and m.num_allocated == 0
    assert m.num_blocks * m.block_size == 128
    m.check_invariants()


def test_lifo_order_and_first_ids(impl):
    BM = impl[0]
    m = BM(8, 16)
    assert m.allocate(3, owner="a") == [0, 1, 2]
    first = m.allocate(1, owner="b")
    m.free(first)
    assert m.allocate(1, owner="c") == first, "expected the most recently freed block back"


def test_blocks_needed_rounds_up(impl):
    m = impl[0](100, 16)
    assert [m.blocks_needed(n) for n in (0, 1, 16, 17, 32)] == [0, 1, 1, 2, 2]


def test_oom_raises_and_changes_nothing(impl):
    BM, OOB = impl[0], impl[1]
    m = BM(4, 16)
    held = m.allocate(3, owner="a")
    with pytest.raises(OOB) as exc:
        m.allocate(2, owner="b")
    assert exc.value.requested == 2 and exc.value.available == 1
    assert m.num_free == 1 and m.num_allocated == len(held)
    m.check_invariants()
    assert len(m.allocate(1, owner="c")) == 1


def test_zero_allocation_and_exact_fit(impl):
    BM, OOB = impl[0], impl[1]
    m = BM(4, 16)
    assert m.allocate(0, owner="a") == []
    assert len(m.allocate(4, owner="a")) == 4
    with pytest.raises(OOB):
        m.allocate(1)
    with pytest.raises(ValueError):
        m.allocate(-1)


def test_double_free_and_atomic_batch_free(impl):
    BM, DF = impl[0], impl[2]
    m = BM(8, 16)
    blocks = m.allocate(2, owner="a")
    m.free(blocks)
    with pytest.raises(DF):
        m.free(blocks)
    good = m.allocate(3, owner="b")
    with pytest.raises(DF):
        m.free(good + [7])
    assert m.num_allocated == 3, "partial free left the pool inconsistent"
    m.check_invariants()


def test_free_owner_releases_only_that_request(impl):
    m = impl[0](16, 8)
    m.allocate(4, owner="a")
    b = m.allocate(4, owner="b")
    assert len(m.free_owner("a")) == 4
    assert m.num_allocated == 4 and all(m.owner_of(x) == "b" for x in b)
    m.check_invariants()


def test_rejects_nonsense_construction(impl):
    with pytest.raises(ValueError):
        impl[0](0, 16)
    with pytest.raises(ValueError):
        impl[0](16, 0)


def test_churn_preserves_invariants(impl):
    """4000 random ops, seed 1234, invariants after each (tests/test_blocks.py:152-192)."""
    BM, OOB = impl[0], impl[1]
    rng = random.Random(1234)
    m = BM(64, 8)
    live, nid, allocs, rejects = {}, 0, 0, 0
    for _ in range(4000):
        if live and rng.random() < 0.45:
            m.free(live.pop(rng.choice(list(live))))
        else:
            owner = f"r{nid}"
            nid += 1
            try:
                live[owner] = m.allocate(rng.randint(1, 12), owner=owner)
                allocs += 1
            except OOB:
                rejects += 1
        m.check_invariants()
        seen = set()
        for bl in live.values():
            assert not seen & set(bl)
            seen.update(bl)
    assert allocs > 100 and rejects > 0
    for bl in live.values():
        m.free(bl)
    assert m.num_free == 64


# --- refcounts and the prefix registry (tests/test_phase6.py:40-222) ---

def test_refcount_sharing(impl):
    BM, DF = impl[0], impl[2]
    m = BM(8, 4)
    blocks = m.allocate(2, owner="a")
    m.incref(blocks)
    assert m.refcount(blocks[0]) == 2 and m.num_allocated == 2 and m.num_free == 6
    m.free(blocks)
    assert m.num_allocated == 2
    m.free(blocks)
    assert m.num_allocated == 0 and m.num_free == 8
    with pytest.raises(DF):
        m.free(blocks)
    m.check_invariants()


def test_registered_block_becomes_reclaimable(impl):
    BM, _, _, cd, root = impl
    m = BM(8, 4)
    (b,) = m.allocate(1, owner="a")
    d = cd(root, [1, 2, 3, 4])
    assert m.register_prefix(b, d, [1, 2, 3, 4])
    m.free([b])
    assert m.num_allocated == 0 and m.num_reclaimable == 1 and m.num_unused == 7
    assert m.num_free == 8
    assert m.lookup_prefix(d, [1, 2, 3, 4]) == b
    m.incref([b])
    assert m.refcount(b) == 1 and m.num_reclaimable == 0
    m.check_invariants()


def test_unused_blocks_spent_before_cached_ones(impl):
    BM, _, _, cd, root = impl
    m = BM(4, 4)
    (c,) = m.allocate(1, owner="a")
    m.register_prefix(c, cd(root, [9, 9, 9, 9]), [9, 9, 9, 9])
    m.free([c])
    taken = m.allocate(3, owner="b")
    assert c not in taken and m.num_reclaimable == 1 and m.evictions == 0


def test_eviction_is_lru_and_unregisters(impl):
    BM, _, _, cd, root = impl
    m = BM(3, 4)
    ids = m.allocate(3, owner="a")
    digs = []
    for i, b in enumerate(ids):
        toks = [i] * 4
        d = cd(root, toks)
        m.register_prefix(b, d, toks)
        digs.append((d, toks))
    m.free(ids)
    (t,) = m.allocate(1, owner="b")
    assert t == ids[0] and m.evictions == 1
    assert m.lookup_prefix(*digs[0]) is None
    assert m.lookup_prefix(*digs[1]) == ids[1]
    m.check_invariants()


def test_lookup_verifies_tokens_and_partial_refused(impl):
    BM, _, _, cd, root = impl
    m = BM(4, 4)
    (b,) = m.allocate(1, owner="a")
    d = cd(root, [1, 2, 3, 4])
    m.register_prefix(b, d, [1, 2, 3, 4])
    assert m.lookup_prefix(d, [1, 2, 3, 5]) is None
    with pytest.raises(ValueError):
        m.register_prefix(b, cd(root, [1, 2]), [1, 2])


def test_digest_chain_binds_position(impl):
    cd, root = impl[3], impl[4]
    assert cd(root, [7] * 4) != cd(cd(root, [1, 2, 3, 4]), [7] * 4)


def test_unregister_frees_unreferenced_block(impl):
    BM, _, _, cd, root = impl
    m = BM(4, 4)
    (b,) = m.allocate(1, owner="a")
    d = cd(root, [1, 2, 3, 4])
    m.register_prefix(b, d, [1, 2, 3, 4])
    m.free([b])
    assert m.unregister_prefix(b)
    assert m.num_reclaimable == 0 and m.num_unused == 4
    assert m.lookup_prefix(d, [1, 2, 3, 4]) is None


def test_sharing_churn(impl):
    """2000 ops with sharing, seed 99 (tests/test_phase6.py:185-222)."""
    BM, OOB = impl[0], impl[1]
    rng = random.Random(99)
    m = BM(32, 4)
    live, shared, nid = {}, [], 0
    for _ in range(2000):
        roll = rng.random()
        if live and roll < 0.35:
            m.free(live.pop(rng.choice(list(live))))
        elif shared and roll < 0.55:
            owner = f"s{nid}"
            nid += 1
            take = rng.sample(shared, min(len(shared), rng.randint(1, 3)))
            take = [b for b in take if m.refcount(b) > 0]
            if take:
                m.incref(take)
                live[owner] = take
        else:
            owner = f"r{nid}"
            nid += 1
            try:
                bl = m.allocate(rng.randint(1, 5), owner=owner)
                live[owner] = bl
                shared = [b for b in (shared + bl) if m.refcount(b) > 0][-12:]
            except OOB:
                pass
        m.check_invariants()
    for bl in live.values():
        m.free(bl)
    assert m.num_allocated == 0


def test_product_and_oracle_hand_out_identical_ids():
    """Differential churn with registry traffic: every return value must agree."""
    rng = random.Random(7)
    a, b = prod.BlockManager(40, 4), orc.RefBlockManager(40, 4)
    live = {}
    nid = 0
    for step in range(3000):
        r = rng.random()
        if live and r < 0.4:
            owner = rng.choice(sorted(live))
            ids = live.pop(owner)
            a.free(ids)
            b.free(ids)
        elif r < 0.5:
            toks = [rng.randrange(5) for _ in range(4)]
            d = prod.chain_digest(prod.ROOT_DIGEST, toks)
            ra, rb = a.lookup_prefix(d, toks), b.lookup_prefix(d, toks)
            assert ra == rb
            if ra is not None and rng.random() < 0.5:
                a.incref([ra])
                b.incref([rb])
                live[f"x{nid}"] = [ra]
                nid += 1
        else:
            n = rng.randint(1, 6)
            try:
                ia = a.allocate(n, owner=nid)
            except prod.OutOfBlocks as e:
                with pytest.raises(orc.OutOfBlocks):
                    b.allocate(n, owner=nid)
                assert e.available == b.num_free
                continue
            ib = b.allocate(n, owner=nid)
            assert ia == ib, f"step {step}"
            live[f"r{nid}"] = ia
            nid += 1
            if rng.random() < 0.5:
                # publish the fresh block once, as paged.py does for a full block
                toks = [rng.randrange(5) for _ in range(4)]
                da = prod.chain_digest(prod.ROOT_DIGEST, toks)
                assert da == orc.chain_digest(orc.ROOT_DIGEST, toks)
                assert a.register_prefix(ia[0], da, toks) == b.register_prefix(ib[0], da, toks)
        assert (a.num_free, a.num_unused, a.num_reclaimable, a.num_allocated) == \
               (b.num_free, b.num_unused, b.num_reclaimable, b.num_allocated)
        a.check_invariants()
        b.check_invariants()
