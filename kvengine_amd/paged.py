"""Paged KV cache with device-resident block tables (kvengine's API, MI355X layout).

Host side keeps the reference's interface and bookkeeping exactly
(kvengine/paged.py:38-404): `BlockManager` allocation with the same call order,
`length / reserve / write / commit / truncate / free`, prefix adopt/publish.
Device side differs by design:

* pool tensors per layer in the kernel layout, K [L, NB, Hkv, bs, D] and
  V [L, NB, Hkv, D, bs] (each (block, head) is one contiguous tile);
* one int32 block table row and one length per live sequence, held on the
  device ([max_seqs, max_blocks] and [max_seqs]) and updated in place, so
  kernels never need a host copy of a table (the reference re-uploads a Python
  list after every growth or shrink, paged.py:281-284);
* `write` scatters with the KV-write kernel; the forward pass never gathers
  (attention reads blocks through the table), and `_gather` exists only for
  API compatibility and tests.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import kernels
from .blocks import ROOT_DIGEST, BlockManager, OutOfBlocks, chain_digest

DEFAULT_BLOCK_SIZE = 16


@dataclass
class DeviceKV:
    """What the kernels need from a cache for one forward pass."""

    k: torch.Tensor          # [L, NB, Hkv, bs, D]
    v: torch.Tensor          # [L, NB, Hkv, D, bs]
    tables: torch.Tensor     # [rows, max_blocks] int32
    lens: torch.Tensor       # [rows] int32, committed length per row
    block_size: int


def _model_info(model) -> dict:
    if hasattr(model, "arch"):
        return model.arch.shape_info()
    cfg = model.config
    return {
        "num_layers": cfg.num_hidden_layers,
        "num_key_value_heads": getattr(cfg, "num_key_value_heads", cfg.num_attention_heads),
        "head_dim": getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads,
    }


class PagedKVCache:
    """The shared pool: block tensors, the allocator, device tables and lengths."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, num_blocks: int,
                 block_size: int, dtype: torch.dtype, device, max_seqs: int = 64,
                 max_blocks_per_seq: int | None = None):
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.dtype = dtype
        self.device = torch.device(device)
        self.k = torch.zeros((num_layers, num_blocks, num_kv_heads, block_size, head_dim),
                             dtype=dtype, device=self.device)
        self.v = torch.zeros((num_layers, num_blocks, num_kv_heads, head_dim, block_size),
                             dtype=dtype, device=self.device)
        self.max_blocks = max_blocks_per_seq or num_blocks
        self.max_seqs = max_seqs
        self.tables = torch.full((max_seqs, self.max_blocks), -1, dtype=torch.int32,
                                 device=self.device)
        self.lens = torch.zeros(max_seqs, dtype=torch.int32, device=self.device)
        self.manager = BlockManager(num_blocks, block_size)
        self._free_rows = list(range(max_seqs - 1, -1, -1))

    @classmethod
    def for_model(cls, model, num_blocks: int, block_size: int = DEFAULT_BLOCK_SIZE,
                  max_seqs: int = 64) -> "PagedKVCache":
        info = _model_info(model)
        p = next(model.parameters())
        return cls(info["num_layers"], info["num_key_value_heads"], info["head_dim"], num_blocks,
                   block_size, p.dtype, p.device, max_seqs=max_seqs)

    # --- rows of the device tables ---

    def acquire_row(self) -> int:
        if not self._free_rows:
            raise RuntimeError(f"all {self.max_seqs} sequence rows of this pool are in use")
        return self._free_rows.pop()

    def release_row(self, row: int) -> None:
        self.tables[row].fill_(-1)
        self.lens[row].fill_(0)
        self._free_rows.append(row)

    def device_kv(self) -> DeviceKV:
        return DeviceKV(self.k, self.v, self.tables, self.lens, self.block_size)

    # --- capacity accounting (kvengine/paged.py:92-113) ---

    def nbytes(self) -> int:
        return self.k.numel() * self.k.element_size() * 2

    def bytes_per_block(self) -> int:
        return self.nbytes() // self.num_blocks

    @property
    def total_slots(self) -> int:
        return self.num_blocks * self.block_size

    def new_sequence(self, request_id: object) -> "PagedSequenceCache":
        return PagedSequenceCache(self, request_id)

    def stats(self) -> dict:
        return {
            "num_blocks": self.num_blocks,
            "block_size": self.block_size,
            "blocks_allocated": self.manager.num_allocated,
            "blocks_free": self.manager.num_free,
            "pool_utilization": self.manager.pool_utilization(),
            "mib": self.nbytes() / 2**20,
        }

    def __repr__(self) -> str:
        return (f"PagedKVCache(blocks={self.num_blocks}x{self.block_size}, "
                f"free={self.manager.num_free}, {self.nbytes() / 2**20:.1f} MiB)")


class PagedSequenceCache:
    """One request's view of the pool: a block table row plus a token count."""

    def __init__(self, pool: PagedKVCache, request_id: object):
        self.pool = pool
        self.request_id = request_id
        self.blocks: list[int] = []
        self._length = 0
        self._row: int | None = None
        self._row_dev: torch.Tensor | None = None
        self._pending_n = 0
        self._pending = False
        self._digest_chain: list[bytes] = []
        self._registered = 0
        self.tokens_reused = 0

    # --- state ---

    @property
    def length(self) -> int:
        return self._length

    @property
    def block_size(self) -> int:
        return self.pool.block_size

    @property
    def capacity(self) -> int:
        return len(self.blocks) * self.block_size

    def free_slots(self) -> int:
        return self.capacity - self._length

    def utilization(self) -> float:
        return self._length / self.capacity if self.blocks else 0.0

    def nbytes(self) -> int:
        return len(self.blocks) * self.pool.bytes_per_block()

    @property
    def row(self) -> int:
        """This sequence's row in the pool's device tables (acquired on demand)."""
        if self._row is None:
            self._row = self.pool.acquire_row()
            self._row_dev = torch.tensor([self._row], dtype=torch.int32, device=self.pool.device)
        return self._row

    @property
    def row_dev(self) -> torch.Tensor:
        _ = self.row
        return self._row_dev

    def device_kv(self) -> DeviceKV:
        return self.pool.device_kv()

    def _set_entries(self, start: int, ids: list[int]) -> None:
        if not ids:
            return
        if len(ids) == 1:
            self.pool.tables[self.row, start].fill_(ids[0])
        else:
            src = torch.tensor(ids, dtype=torch.int32)
            self.pool.tables[self.row, start:start + len(ids)].copy_(src, non_blocking=False)

    # --- allocation (kvengine/paged.py:179-205) ---

    def reserve(self, n_tokens: int) -> None:
        need = self.pool.manager.blocks_needed(self._length + n_tokens)
        extra = need - len(self.blocks)
        if extra > 0:
            if need > self.pool.max_blocks:
                raise OutOfBlocks(extra, self.pool.manager.num_free)
            new = self.pool.manager.allocate(extra, owner=self.request_id)
            self._set_entries(len(self.blocks), new)
            self.blocks.extend(new)
        _ = self.row
        self._pending_n = n_tokens
        self._pending = True

    def slot_indices(self, start: int, n_tokens: int) -> torch.Tensor:
        bs = self.block_size
        ids = torch.tensor(self.blocks, dtype=torch.long)
        pos = torch.arange(start, start + n_tokens)
        return (ids[pos // bs] * bs + pos % bs).to(self.pool.device)

    # --- write / gather (kvengine/paged.py:288-331) ---

    def write(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor, start: int):
        """k, v [1, Hkv, T, D]: scatter into the pool; returns the gathered history
        [1, Hkv, start+T, D] (API compatibility; the forward pass never gathers)."""
        assert k.shape == v.shape, f"k/v shape mismatch: {k.shape} vs {v.shape}"
        assert k.shape[0] == 1, "one request per sequence cache"
        n = k.shape[2]
        assert start == self._length, f"write at {start} but sequence length is {self._length}"
        assert self._pending and self._pending_n == n, (
            "reserve() must be called with this pass's token count before write()")
        self.write_rows(layer_idx, k[0].transpose(0, 1).unsqueeze(0).contiguous(),
                        v[0].transpose(0, 1).unsqueeze(0).contiguous())
        return self._gather(layer_idx, start + n)

    def write_rows(self, layer_idx: int, k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        """k_new/v_new [1, T, Hkv, D] at positions length..length+T-1 (kernel scatter)."""
        kernels.kv_write(k_new, v_new, self.pool.k[layer_idx], self.pool.v[layer_idx],
                         self.pool.tables, self.pool.lens, seq_rows=self.row_dev)

    def _gather(self, layer_idx: int, end: int):
        nb = self.pool.manager.blocks_needed(end)
        ids = torch.tensor(self.blocks[:nb], dtype=torch.long, device=self.pool.device)
        k = self.pool.k[layer_idx][ids]            # [nb, Hkv, bs, D]
        v = self.pool.v[layer_idx][ids]            # [nb, Hkv, D, bs]
        Hkv, D, bs = self.pool.num_kv_heads, self.pool.head_dim, self.block_size
        k_all = k.permute(1, 0, 2, 3).reshape(Hkv, nb * bs, D)[:, :end]
        v_all = v.permute(1, 0, 3, 2).reshape(Hkv, nb * bs, D)[:, :end]
        return k_all.unsqueeze(0).contiguous(), v_all.unsqueeze(0).contiguous()

    def commit(self, n_tokens: int) -> None:
        if self._length + n_tokens > self.capacity:
            raise OutOfBlocks(self.pool.manager.blocks_needed(self._length + n_tokens)
                              - len(self.blocks), self.pool.manager.num_free)
        self._length += n_tokens
        self.pool.lens[self.row].fill_(self._length)
        self._pending = False
        self._pending_n = 0

    def sync_committed(self, n_tokens: int) -> None:
        """Host-side commit after the device length was advanced by a kernel."""
        if self._length + n_tokens > self.capacity:
            raise OutOfBlocks(self.pool.manager.blocks_needed(self._length + n_tokens)
                              - len(self.blocks), self.pool.manager.num_free)
        self._length += n_tokens
        self._pending = False
        self._pending_n = 0

    # --- rollback (kvengine/paged.py:344-380) ---

    def truncate(self, n_tokens: int, device_done: bool = False) -> None:
        """Roll back to n_tokens, returning wholly unused blocks in table order.

        device_done=True means the rollback kernel already updated this row's
        device length and table; only the host bookkeeping is applied then.
        """
        if not 0 <= n_tokens <= self._length:
            raise ValueError(f"cannot truncate to {n_tokens}, length is {self._length}")
        bs = self.block_size
        mgr = self.pool.manager
        first_invalid = n_tokens // bs
        for i in range(first_invalid, min(self._registered, len(self.blocks))):
            b = self.blocks[i]
            if mgr.refcount(b) > 1:
                raise ValueError(f"block {b} is shared by another sequence; cannot roll back into it")
            mgr.unregister_prefix(b)
        keep = mgr.blocks_needed(n_tokens)
        if keep < len(self.blocks):
            mgr.free(self.blocks[keep:])
            self.blocks = self.blocks[:keep]
            if not device_done:
                self.pool.tables[self.row, keep:].fill_(-1)
        self._registered = min(self._registered, first_invalid)
        del self._digest_chain[first_invalid:]
        self._length = n_tokens
        if not device_done and self._row is not None:
            self.pool.lens[self._row].fill_(n_tokens)
        self._pending = False
        self._pending_n = 0

    def free(self) -> None:
        """Return every block to the pool; idempotent (kvengine/paged.py:384-398)."""
        if self.blocks:
            self.pool.manager.free(self.blocks)
            self.blocks = []
        if self._row is not None:
            self.pool.release_row(self._row)
            self._row = None
            self._row_dev = None
        self._length = 0
        self._pending = False
        self._pending_n = 0
        self._digest_chain = []
        self._registered = 0
        self.tokens_reused = 0

    # --- prefix sharing (kvengine/paged.py:209-279) ---

    def adopt_prefix(self, token_ids: list[int]) -> int:
        assert self._length == 0 and not self.blocks, "adopt_prefix needs a fresh sequence"
        bs = self.block_size
        reusable = max(len(token_ids) - 1, 0)
        parent = ROOT_DIGEST
        adopted: list[int] = []
        chain: list[bytes] = []
        for i in range(reusable // bs):
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
            self._set_entries(0, adopted)
            self.blocks.extend(adopted)
            self._digest_chain = chain
            self._registered = len(adopted)
            self._length = len(adopted) * bs
            self.pool.lens[self.row].fill_(self._length)
        self.tokens_reused = self._length
        return self._length

    def register_prefix_blocks(self, token_ids: list[int], ahead: int = 0) -> int:
        """Publish this sequence's full blocks of token_ids (paged.py:263-279).
        ahead: tokens reserved past the length whose K/V a forward already
        queued (or about to be queued before any reader) will write; their full
        blocks are published too (the engine's batched admission)."""
        bs = self.block_size
        full = min((self._length + ahead) // bs, len(token_ids) // bs, len(self.blocks))
        while len(self._digest_chain) < full:
            i = len(self._digest_chain)
            parent = self._digest_chain[-1] if self._digest_chain else ROOT_DIGEST
            self._digest_chain.append(chain_digest(parent, token_ids[i * bs:(i + 1) * bs]))
        published = 0
        for i in range(self._registered, full):
            if self.pool.manager.register_prefix(self.blocks[i], self._digest_chain[i],
                                                 token_ids[i * bs:(i + 1) * bs]):
                published += 1
        self._registered = max(self._registered, full)
        return published

    def __repr__(self) -> str:
        return (f"PagedSequenceCache(req={self.request_id!r}, len={self._length}, "
                f"blocks={len(self.blocks)}, util={self.utilization():.1%})")


class KVCacheFull(RuntimeError):
    """A request needs more positions than its contiguous cache holds."""


class ContiguousKVCache:
    """One request, one worst-case buffer (kvengine/cache.py:26-155).

    Stored as a single block of max_seq_len tokens in the kernel layout, so the
    same attention and KV-write kernels serve it (block table [[0]]).
    `truncate` only moves the length; stale positions are never read.
    """

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, max_seq_len: int,
                 dtype: torch.dtype, device):
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.max_seq_len = max_seq_len
        self.dtype = dtype
        self.device = torch.device(device)
        self.k = torch.zeros((num_layers, 1, num_kv_heads, max_seq_len, head_dim), dtype=dtype,
                             device=self.device)
        self.v = torch.zeros((num_layers, 1, num_kv_heads, head_dim, max_seq_len), dtype=dtype,
                             device=self.device)
        self.tables = torch.zeros((1, 1), dtype=torch.int32, device=self.device)
        self.lens = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.row_dev = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.row = 0
        self._length = 0

    @classmethod
    def for_model(cls, model, max_seq_len: int) -> "ContiguousKVCache":
        info = _model_info(model)
        p = next(model.parameters())
        return cls(info["num_layers"], info["num_key_value_heads"], info["head_dim"], max_seq_len,
                   p.dtype, p.device)

    @property
    def length(self) -> int:
        return self._length

    @property
    def capacity(self) -> int:
        return self.max_seq_len

    @property
    def block_size(self) -> int:
        return self.max_seq_len

    def free_slots(self) -> int:
        return self.max_seq_len - self._length

    def utilization(self) -> float:
        return self._length / self.max_seq_len if self.max_seq_len else 0.0

    def nbytes(self) -> int:
        return self.k.numel() * self.k.element_size() * 2

    def reset(self) -> None:
        self._length = 0
        self.lens.fill_(0)

    def device_kv(self) -> DeviceKV:
        return DeviceKV(self.k, self.v, self.tables, self.lens, self.max_seq_len)

    def reserve(self, n_tokens: int) -> None:
        if self._length + n_tokens > self.max_seq_len:
            raise KVCacheFull(f"need {self._length + n_tokens} positions, capacity {self.max_seq_len}")

    def write(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor, start: int):
        assert k.shape == v.shape and k.shape[0] == 1
        n = k.shape[2]
        end = start + n
        if end > self.max_seq_len:
            raise KVCacheFull(f"need {end} positions but cache holds {self.max_seq_len}")
        self.k[layer_idx, 0, :, start:end, :] = k[0]
        self.v[layer_idx, 0, :, :, start:end] = v[0].transpose(1, 2)
        return (self.k[layer_idx, 0, :, :end, :].unsqueeze(0),
                self.v[layer_idx, 0, :, :, :end].transpose(1, 2).unsqueeze(0))

    def write_rows(self, layer_idx: int, k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        kernels.kv_write(k_new, v_new, self.k[layer_idx], self.v[layer_idx], self.tables,
                         self.lens, seq_rows=self.row_dev)

    def truncate(self, n_tokens: int, device_done: bool = False) -> None:
        if not 0 <= n_tokens <= self._length:
            raise ValueError(f"cannot truncate to {n_tokens}, length is {self._length}")
        self._length = n_tokens
        if not device_done:
            self.lens.fill_(n_tokens)

    def commit(self, n_tokens: int) -> None:
        if self._length + n_tokens > self.max_seq_len:
            raise KVCacheFull(f"committing {n_tokens} would exceed capacity {self.max_seq_len}")
        self._length += n_tokens
        self.lens.fill_(self._length)

    def sync_committed(self, n_tokens: int) -> None:
        if self._length + n_tokens > self.max_seq_len:
            raise KVCacheFull(f"committing {n_tokens} would exceed capacity {self.max_seq_len}")
        self._length += n_tokens
