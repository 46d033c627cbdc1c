"""Host block allocator with kvengine's BlockManager semantics.

Same contract as the reference (kvengine/blocks.py:70-353), which the paged
cache and the batched scheduler depend on for bit-exact block tables:

* LIFO reuse: the free stack starts as N-1..0 so the first allocations are
  0, 1, 2, ...; freed blocks are pushed and popped again first
  (blocks.py:91-93, 166-174, 211-213)
* all-or-nothing allocate raising OutOfBlocks(requested, available) before any
  state changes; free blocks before reclaimable ones, reclaimable ones evicted
  least recently released first (blocks.py:150-174, 297-306)
* free validates the whole batch (DoubleFree) before decrementing; a block
  reaching zero references becomes reclaimable if it holds a registered
  prefix, else free (blocks.py:194-213)
* content-addressed registry of full blocks with token verification
  (blocks.py:46-50, 232-295)

Implementation: per-block state lives in flat arrays (reference count, owner,
registry slot), so the batched scheduler can query many blocks without dict
churn; the reclaimable set is an insertion-ordered dict used as an LRU queue.
`BlockAllocator` is an alias (the name used for this component elsewhere).
"""

from __future__ import annotations

import hashlib
import struct
from collections import OrderedDict
from collections.abc import Sequence

ROOT_DIGEST = b"\x00" * 16


def chain_digest(parent: bytes, token_ids: Sequence[int]) -> bytes:
    """Content address of a block: blake2b-128 of the parent digest, then the
    block's tokens as little-endian int32 (kvengine/blocks.py:46-50)."""
    h = hashlib.blake2b(parent, digest_size=16)
    h.update(struct.pack(f"<{len(token_ids)}i", *token_ids))
    return h.digest()


class OutOfBlocks(RuntimeError):
    """Not enough allocatable blocks; carries what the scheduler needs."""

    def __init__(self, requested: int, available: int):
        super().__init__(f"requested {requested} blocks, only {available} available")
        self.requested = requested
        self.available = available


class DoubleFree(RuntimeError):
    """A block was released while not referenced by anything."""


class BlockManager:
    """Reference-counted slab pool over `num_blocks` KV blocks.

    A block is free (holds nothing), reclaimable (unreferenced but holding a
    registered prefix; reusable in LRU order) or referenced (refcount > 0).
    """

    def __init__(self, num_blocks: int, block_size: int):
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.reset()
        self.prefix_hits = 0
        self.prefix_misses = 0
        self.evictions = 0

    def reset(self) -> None:
        n = self.num_blocks
        self._free = list(range(n - 1, -1, -1))
        self._ref = [0] * n
        self._owner: list[object] = [None] * n
        self._n_live = 0
        self._reclaim: OrderedDict[int, None] = OrderedDict()
        self._digest: list[bytes | None] = [None] * n
        self._tokens: list[tuple | None] = [None] * n
        self._by_digest: dict[bytes, int] = {}

    # --- state ---

    @property
    def num_free(self) -> int:
        """Allocatable now: free plus reclaimable."""
        return len(self._free) + len(self._reclaim)

    @property
    def num_unused(self) -> int:
        return len(self._free)

    @property
    def num_reclaimable(self) -> int:
        return len(self._reclaim)

    @property
    def num_allocated(self) -> int:
        return self._n_live

    @property
    def total_slots(self) -> int:
        return self.num_blocks * self.block_size

    def pool_utilization(self) -> float:
        return self._n_live / self.num_blocks

    def owner_of(self, block_id: int):
        return self._owner[block_id]

    def refcount(self, block_id: int) -> int:
        return self._ref[block_id]

    def blocks_needed(self, n_tokens: int) -> int:
        return (n_tokens + self.block_size - 1) // self.block_size

    # --- allocate / free ---

    def allocate(self, n_blocks: int, owner: object = None) -> list[int]:
        if n_blocks < 0:
            raise ValueError("n_blocks must be non-negative")
        avail = len(self._free) + len(self._reclaim)
        if n_blocks > avail:
            raise OutOfBlocks(n_blocks, avail)
        out = []
        for _ in range(n_blocks):
            b = self._free.pop() if self._free else self._evict_lru()
            self._ref[b] = 1
            self._owner[b] = owner
            out.append(b)
        self._n_live += n_blocks
        return out

    def incref(self, block_ids: Sequence[int]) -> None:
        ids = list(block_ids)
        for b in ids:
            if self._ref[b] <= 0 and b not in self._reclaim:
                raise DoubleFree(f"block {b} is neither referenced nor reclaimable")
        for b in ids:
            if b in self._reclaim:
                del self._reclaim[b]
                self._ref[b] = 1
                self._n_live += 1
            else:
                self._ref[b] += 1

    def free(self, block_ids) -> None:
        ids = list(block_ids)
        for b in ids:
            if not (0 <= b < self.num_blocks) or self._ref[b] <= 0:
                raise DoubleFree(f"block {b} is not referenced")
        for b in ids:
            self._ref[b] -= 1
            if self._ref[b]:
                continue
            self._n_live -= 1
            if self._digest[b] is not None:
                self._reclaim[b] = None
            else:
                self._owner[b] = None
                self._free.append(b)

    def free_owner(self, owner: object) -> list[int]:
        ids = [b for b in range(self.num_blocks) if self._ref[b] > 0 and self._owner[b] == owner]
        self.free(ids)
        return ids

    # --- prefix registry ---

    def register_prefix(self, block_id: int, digest: bytes, token_ids: Sequence[int]) -> bool:
        if len(token_ids) != self.block_size:
            raise ValueError(f"only full blocks are shareable: got {len(token_ids)} tokens, "
                             f"block_size is {self.block_size}")
        held = self._by_digest.get(digest)
        if held is not None:
            return held == block_id
        if self._ref[block_id] <= 0:
            raise ValueError(f"cannot register unreferenced block {block_id}")
        self._by_digest[digest] = block_id
        self._digest[block_id] = digest
        self._tokens[block_id] = tuple(token_ids)
        return True

    def lookup_prefix(self, digest: bytes, token_ids: Sequence[int]) -> int | None:
        b = self._by_digest.get(digest)
        if b is None or self._tokens[b] != tuple(token_ids):
            self.prefix_misses += 1
            return None
        self.prefix_hits += 1
        if b in self._reclaim:
            self._reclaim.move_to_end(b)
        return b

    def unregister_prefix(self, block_id: int) -> bool:
        d = self._digest[block_id]
        if d is None:
            return False
        self._digest[block_id] = None
        self._tokens[block_id] = None
        if self._by_digest.get(d) == block_id:
            del self._by_digest[d]
        if block_id in self._reclaim:
            del self._reclaim[block_id]
            self._owner[block_id] = None
            self._free.append(block_id)
        return True

    def _evict_lru(self) -> int:
        b, _ = self._reclaim.popitem(last=False)
        d = self._digest[b]
        if d is not None:
            self._by_digest.pop(d, None)
        self._digest[b] = None
        self._tokens[b] = None
        self._owner[b] = None
        self.evictions += 1
        return b

    def prefix_hit_rate(self) -> float:
        total = self.prefix_hits + self.prefix_misses
        return self.prefix_hits / total if total else 0.0

    # --- invariants ---

    def check_invariants(self) -> None:
        free = set(self._free)
        assert len(free) == len(self._free), "duplicate block in free list"
        recl = set(self._reclaim)
        live = {b for b in range(self.num_blocks) if self._ref[b] > 0}
        assert not (free & live), f"blocks both free and referenced: {sorted(free & live)}"
        assert not (free & recl), f"blocks both free and reclaimable: {sorted(free & recl)}"
        assert not (recl & live), f"blocks both reclaimable and referenced: {sorted(recl & live)}"
        assert free | recl | live == set(range(self.num_blocks)), "blocks leaked"
        assert all(r >= 0 for r in self._ref), "negative refcount"
        assert len(live) == self._n_live, "live count out of sync"
        for d, b in self._by_digest.items():
            assert self._digest[b] == d, f"prefix registry disagrees with itself for block {b}"
        for b in recl:
            assert self._digest[b] is not None, f"reclaimable block {b} holds no registered prefix"

    def __repr__(self) -> str:
        return (f"BlockManager(num_blocks={self.num_blocks}, block_size={self.block_size}, "
                f"unused={self.num_unused}, reclaimable={self.num_reclaimable}, "
                f"referenced={self.num_allocated})")


BlockAllocator = BlockManager
