"""Oracle paged KV cache: a restatement of kvengine/paged.py. TEST INFRASTRUCTURE.

Reference layout and behaviour:

* pool tensors k, v of shape [L, NB, bs, Hkv, D], zero-initialised and never
  re-zeroed; flat views [L, NB*bs, Hkv, D] (paged.py:59-67)
* reserve(n): grow the table to blocks_needed(len+n) with one atomic allocate,
  then plan slots (paged.py:179-195); slot = table[pos//bs]*bs + pos%bs
  (paged.py:197-205)
* write: assert start == length and a matching reserve, index_copy_ the
  [T, Hkv, D] rows into the flat pool, then gather (paged.py:288-313)
* gather: whole blocks in block-table order, reshape, trim to `end`,
  transpose to [1, Hkv, end, D], contiguous (paged.py:315-331)
* commit: length += n, OutOfBlocks past capacity (paged.py:333-342)
* truncate(n): ValueError outside [0, len]; published blocks from n//bs on are
  unregistered, or refused with ValueError when shared; then
  free(blocks[ceil(n/bs):]) in table order (paged.py:344-380)
* free(): release every block, idempotent (paged.py:384-398)
* adopt_prefix / register_prefix_blocks: full-block content-addressed sharing,
  at most len-1 tokens adopted (paged.py:209-279)
"""

from __future__ import annotations

import torch

from .blocks import ROOT_DIGEST, OutOfBlocks, RefBlockManager, chain_digest


class RefPagedKVCache:
    def __init__(self, num_layers, num_kv_heads, head_dim, num_blocks, block_size, dtype,
                 device="cpu"):
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.dtype = dtype
        self.device = torch.device(device)
        shape = (num_layers, num_blocks, block_size, num_kv_heads, head_dim)
        self.k = torch.zeros(shape, dtype=dtype, device=self.device)
        self.v = torch.zeros(shape, dtype=dtype, device=self.device)
        flat = (num_layers, num_blocks * block_size, num_kv_heads, head_dim)
        self.k_flat = self.k.view(flat)
        self.v_flat = self.v.view(flat)
        self.manager = RefBlockManager(num_blocks, block_size)

    def new_sequence(self, request_id) -> "RefPagedSequence":
        return RefPagedSequence(self, request_id)


class RefPagedSequence:
    def __init__(self, pool: RefPagedKVCache, request_id):
        self.pool = pool
        self.request_id = request_id
        self.blocks: list[int] = []
        self._length = 0
        self._ids = torch.empty(0, dtype=torch.long)
        self._pending = None
        self._pending_n = 0
        self._chain: list[bytes] = []
        self._registered = 0
        self.tokens_reused = 0

    @property
    def length(self) -> int:
        return self._length

    @property
    def block_size(self) -> int:
        return self.pool.block_size

    @property
    def capacity(self) -> int:
        return len(self.blocks) * self.block_size

    def _upload(self) -> None:
        self._ids = torch.tensor(self.blocks, dtype=torch.long, device=self.pool.device)

    def slot_indices(self, start: int, n: int) -> torch.Tensor:
        pos = torch.arange(start, start + n, device=self.pool.device)
        return self._ids[pos // self.block_size] * self.block_size + pos % self.block_size

    def reserve(self, n: int) -> None:
        need = self.pool.manager.blocks_needed(self._length + n) - len(self.blocks)
        if need > 0:
            self.blocks.extend(self.pool.manager.allocate(need, owner=self.request_id))
            self._upload()
        self._pending = self.slot_indices(self._length, n)
        self._pending_n = n

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor, start: int):
        assert k.shape == v.shape and k.shape[0] == 1
        n = k.shape[2]
        assert start == self._length, "write must start at the sequence length"
        assert self._pending is not None and self._pending_n == n, "reserve() first"
        self.pool.k_flat[layer].index_copy_(0, self._pending, k[0].transpose(0, 1).contiguous())
        self.pool.v_flat[layer].index_copy_(0, self._pending, v[0].transpose(0, 1).contiguous())
        return self.gather(layer, start + n)

    def gather(self, layer: int, end: int):
        nb = self.pool.manager.blocks_needed(end)
        ids = self._ids[:nb]
        shape = (nb * self.block_size, self.pool.num_kv_heads, self.pool.head_dim)
        k_all = self.pool.k[layer][ids].reshape(shape)[:end].transpose(0, 1).unsqueeze(0)
        v_all = self.pool.v[layer][ids].reshape(shape)[:end].transpose(0, 1).unsqueeze(0)
        return k_all.contiguous(), v_all.contiguous()

    def commit(self, n: int) -> None:
        if self._length + n > self.capacity:
            raise OutOfBlocks(self.pool.manager.blocks_needed(self._length + n) - len(self.blocks),
                              self.pool.manager.num_free)
        self._length += n
        self._pending = None
        self._pending_n = 0

    def truncate(self, n: int) -> None:
        if not 0 <= n <= self._length:
            raise ValueError(f"cannot truncate to {n}, length is {self._length}")
        first_invalid = n // self.block_size
        mgr = self.pool.manager
        for i in range(first_invalid, min(self._registered, len(self.blocks))):
            if mgr.refcount(self.blocks[i]) > 1:
                raise ValueError(f"block {self.blocks[i]} is shared by another sequence")
            mgr.unregister_prefix(self.blocks[i])
        keep = mgr.blocks_needed(n)
        if keep < len(self.blocks):
            mgr.free(self.blocks[keep:])
            self.blocks = self.blocks[:keep]
            self._upload()
        self._registered = min(self._registered, first_invalid)
        del self._chain[first_invalid:]
        self._length = n
        self._pending = None
        self._pending_n = 0

    def free(self) -> None:
        if self.blocks:
            self.pool.manager.free(self.blocks)
            self.blocks = []
            self._ids = torch.empty(0, dtype=torch.long)
        self._length = 0
        self._pending = None
        self._pending_n = 0
        self._chain = []
        self._registered = 0
        self.tokens_reused = 0

    def adopt_prefix(self, token_ids) -> int:
        assert self._length == 0 and not self.blocks
        bs = self.block_size
        parent, adopted, chain = ROOT_DIGEST, [], []
        for i in range(max(len(token_ids) - 1, 0) // bs):
            chunk = token_ids[i * bs:(i + 1) * bs]
            d = chain_digest(parent, chunk)
            b = self.pool.manager.lookup_prefix(d, chunk)
            if b is None:
                break
            adopted.append(b)
            chain.append(d)
            parent = d
        if adopted:
            self.pool.manager.incref(adopted)
            self.blocks.extend(adopted)
            self._chain = chain
            self._registered = len(adopted)
            self._length = len(adopted) * bs
            self._upload()
        self.tokens_reused = self._length
        return self._length

    def register_prefix_blocks(self, token_ids) -> int:
        bs = self.block_size
        full = min(self._length // bs, len(token_ids) // bs, len(self.blocks))
        while len(self._chain) < full:
            i = len(self._chain)
            parent = self._chain[-1] if self._chain else ROOT_DIGEST
            self._chain.append(chain_digest(parent, token_ids[i * bs:(i + 1) * bs]))
        published = 0
        for i in range(self._registered, full):
            if self.pool.manager.register_prefix(self.blocks[i], self._chain[i],
                                                 token_ids[i * bs:(i + 1) * bs]):
                published += 1
        self._registered = max(self._registered, full)
        return published
