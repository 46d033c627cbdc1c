"""Oracle block allocator: a restatement of kvengine/blocks.py. TEST INFRASTRUCTURE.

Semantics followed, with the reference lines they come from:

* free list is a stack seeded with ids N-1..0 so the first pops are 0,1,2,...
  (blocks.py:91-93); allocation pops, release pushes (LIFO, blocks.py:168, 213)
* allocate is all-or-nothing and raises OutOfBlocks(requested, available)
  before touching state (blocks.py:160-163); free blocks are used before
  reclaimable ones, which are evicted least-recently-released first
  (blocks.py:166-170, 297-306)
* free validates every id first (DoubleFree) and only then decrements; a block
  reaching zero becomes reclaimable if it carries a registered prefix, else it
  is pushed back on the free stack (blocks.py:194-213)
* incref resurrects reclaimable blocks (blocks.py:176-192)
* chain_digest = blake2b(parent, digest_size=16) updated with the tokens packed
  as little-endian int32 (blocks.py:46-50); root is 16 zero bytes (blocks.py:43)
* register/lookup/unregister of full blocks only (blocks.py:232-295)
"""

from __future__ import annotations

import hashlib
import struct
from collections import OrderedDict

ROOT_DIGEST = bytes(16)


def chain_digest(parent: bytes, token_ids) -> bytes:
    h = hashlib.blake2b(parent, digest_size=16)
    h.update(struct.pack(f"<{len(token_ids)}i", *token_ids))
    return h.digest()


class OutOfBlocks(RuntimeError):
    def __init__(self, requested: int, available: int):
        super().__init__(f"requested {requested} blocks, only {available} available")
        self.requested = requested
        self.available = available


class DoubleFree(RuntimeError):
    pass


class RefBlockManager:
    def __init__(self, num_blocks: int, block_size: int):
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.reset()

    def reset(self) -> None:
        self._stack = list(range(self.num_blocks - 1, -1, -1))
        self._refs: dict[int, int] = {}
        self._owner: dict[int, object] = {}
        self._lru: OrderedDict[int, None] = OrderedDict()
        self._by_digest: dict[bytes, int] = {}
        self._digest_of: dict[int, bytes] = {}
        self._tokens_of: dict[int, tuple] = {}
        self.prefix_hits = 0
        self.prefix_misses = 0
        self.evictions = 0

    # counts
    @property
    def num_free(self) -> int:
        return len(self._stack) + len(self._lru)

    @property
    def num_unused(self) -> int:
        return len(self._stack)

    @property
    def num_reclaimable(self) -> int:
        return len(self._lru)

    @property
    def num_allocated(self) -> int:
        return len(self._refs)

    def refcount(self, b: int) -> int:
        return self._refs.get(b, 0)

    def owner_of(self, b: int):
        return self._owner.get(b)

    def blocks_needed(self, n_tokens: int) -> int:
        return -(-n_tokens // self.block_size)

    # allocation
    def allocate(self, n: int, owner=None) -> list[int]:
        if n < 0:
            raise ValueError("n_blocks must be non-negative")
        if n > self.num_free:
            raise OutOfBlocks(n, self.num_free)
        got = []
        for _ in range(n):
            got.append(self._stack.pop() if self._stack else self._evict())
        for b in got:
            self._refs[b] = 1
            self._owner[b] = owner
        return got

    def incref(self, ids) -> None:
        ids = list(ids)
        if any(b not in self._refs and b not in self._lru for b in ids):
            raise DoubleFree("block is neither referenced nor reclaimable")
        for b in ids:
            if b in self._lru:
                del self._lru[b]
                self._refs[b] = 1
            else:
                self._refs[b] += 1

    def free(self, ids) -> None:
        ids = list(ids)
        if any(self._refs.get(b, 0) <= 0 for b in ids):
            raise DoubleFree("block is not referenced")
        for b in ids:
            self._refs[b] -= 1
            if self._refs[b]:
                continue
            del self._refs[b]
            if b in self._digest_of:
                self._lru[b] = None
            else:
                self._owner.pop(b, None)
                self._stack.append(b)

    def free_owner(self, owner) -> list[int]:
        ids = [b for b, o in self._owner.items() if o == owner and b in self._refs]
        self.free(ids)
        return ids

    # prefix registry
    def register_prefix(self, b: int, digest: bytes, tokens) -> bool:
        if len(tokens) != self.block_size:
            raise ValueError("only full blocks are shareable")
        if digest in self._by_digest:
            return self._by_digest[digest] == b
        if self.refcount(b) <= 0:
            raise ValueError(f"cannot register unreferenced block {b}")
        self._by_digest[digest] = b
        self._digest_of[b] = digest
        self._tokens_of[b] = tuple(tokens)
        return True

    def lookup_prefix(self, digest: bytes, tokens):
        b = self._by_digest.get(digest)
        if b is None or self._tokens_of.get(b) != tuple(tokens):
            self.prefix_misses += 1
            return None
        self.prefix_hits += 1
        if b in self._lru:
            self._lru.move_to_end(b)
        return b

    def unregister_prefix(self, b: int) -> bool:
        digest = self._digest_of.pop(b, None)
        if digest is None:
            return False
        if self._by_digest.get(digest) == b:
            del self._by_digest[digest]
        self._tokens_of.pop(b, None)
        if b in self._lru:
            del self._lru[b]
            self._owner.pop(b, None)
            self._stack.append(b)
        return True

    def _evict(self) -> int:
        b, _ = self._lru.popitem(last=False)
        d = self._digest_of.pop(b, None)
        if d is not None:
            self._by_digest.pop(d, None)
        self._tokens_of.pop(b, None)
        self._owner.pop(b, None)
        self.evictions += 1
        return b

    def check_invariants(self) -> None:
        free = set(self._stack)
        assert len(free) == len(self._stack)
        lru, live = set(self._lru), set(self._refs)
        assert not (free & live) and not (free & lru) and not (lru & live)
        assert free | lru | live == set(range(self.num_blocks))
        assert all(c > 0 for c in self._refs.values())
        for d, b in self._by_digest.items():
            assert self._digest_of.get(b) == d
        assert all(b in self._digest_of for b in lru)
