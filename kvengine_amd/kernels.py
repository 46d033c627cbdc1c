"""Torch-facing wrappers over the C ABI: shape checks, workspaces, streams.

Each wrapper takes device tensors, validates them on the host before anything
is launched, and calls the HIP library on torch's current stream. Workspaces
are cached per (device, stream, kind), zero-filled once, and grown on demand; the
kernels leave them zeroed, so a cached workspace can be reused and captured in
a HIP graph. An outgrown workspace is kept alive (never freed), so a graph
captured with it stays valid after a later launch grows the cache.
"""

from __future__ import annotations

import torch

from . import _lib

_WS: dict[tuple, torch.Tensor] = {}
_RETIRED: list[torch.Tensor] = []  # outgrown workspaces, never freed


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return _lib.DTYPE_BF16
    if t.dtype == torch.float32:
        return _lib.DTYPE_F32
    raise TypeError(f"unsupported dtype {t.dtype} (bfloat16 or float32)")


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    """The current HIP stream of `device` as a handle. torch's raw accessor
    costs well under a microsecond; torch.cuda.current_stream() builds a Stream
    object (2.8 us per call measured), which every launch would pay."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(idx)
    return torch.cuda.current_stream(device).cuda_stream


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _check_i32(t: torch.Tensor | None, name: str, device) -> None:
    if t is None:
        return
    _need(t.dtype == torch.int32, f"{name} must be int32, got {t.dtype}")
    _need(t.device == device, f"{name} on {t.device}, expected {device}")
    _need(t.is_contiguous(), f"{name} must be contiguous")


# Matrix layouts (include/kve.h): row-major, or 16-row x 32-column blocks of 1 KB
LAYOUT_ROWS, LAYOUT_BLOCKED = 0, 1


def _layout(blocked: bool) -> int:
    return LAYOUT_BLOCKED if blocked else LAYOUT_ROWS


def blocked_rows(rows: int) -> int:
    """Rows a blocked matrix of `rows` rows allocates (a multiple of 16)."""
    return -(-rows // 16) * 16


def blocked_matrix(rows: int, cols: int, device, dtype=torch.bfloat16) -> torch.Tensor:
    """An uninitialised [rows rounded up to 16, cols] buffer for a blocked matrix."""
    _need(cols % 32 == 0, f"blocked matrices need a multiple of 32 columns, not {cols}")
    return torch.empty(blocked_rows(rows), cols, dtype=dtype, device=device)


def to_blocked(m: torch.Tensor) -> torch.Tensor:
    """Row-major [R, C] (C % 32 == 0) -> blocked layout, R padded to 16 with zeros:
    element (r, c) lands at ((r // 16) * (C // 32) + c // 32) * 512 + (r % 16) * 32 + c % 32."""
    R, C = m.shape
    _need(C % 32 == 0, f"blocked matrices need a multiple of 32 columns, not {C}")
    Rp = blocked_rows(R)
    if Rp != R:
        m = torch.cat([m, m.new_zeros(Rp - R, C)])
    return m.reshape(Rp // 16, 16, C // 32, 32).permute(0, 2, 1, 3).contiguous().view(Rp, C)


def from_blocked(b: torch.Tensor, rows: int) -> torch.Tensor:
    """Blocked [R16, C] -> row-major [rows, C]."""
    R16, C = b.shape[0], b.shape[-1]
    return b.reshape(R16 // 16, C // 32, 16, 32).permute(0, 2, 1, 3).reshape(R16, C)[:rows]


def workspace(kind: str, nbytes: int, device: torch.device, dtype=torch.uint8) -> torch.Tensor:
    """Zero-filled buffer of at least nbytes, cached per device, stream and kind.

    A kind is used for one purpose only: the kernels rely on counter and key
    buffers being zero on entry and leave them zero, which holds only if no
    other data is ever written into them. Launches on different streams may
    overlap in time, so each stream has its own buffer.
    """
    dev = device.index if device.index is not None else torch.cuda.current_device()
    key = (kind, dev, _stream(torch.device("cuda", dev)))
    ws = _WS.get(key)
    esz = torch.empty(0, dtype=dtype).element_size()
    if ws is None or ws.numel() * esz < nbytes:
        if ws is not None:
            # a captured graph may hold the old buffer's address: keep it alive
            _RETIRED.append(ws)
        ws = torch.zeros(max(-(-nbytes // esz), 64), dtype=dtype, device=device)
        _WS[key] = ws
    return ws



class AttnPlan:
    """A verify-attention work plan (kve_attn_plan) for one forward pass: the
    device buffer plus the shape it was built for. Every layer of the pass
    (same tables, lengths, q_len and attention configuration) can use it."""

    __slots__ = ("buf", "key")

    def __init__(self, buf: torch.Tensor, key: tuple):
        self.buf = buf
        self.key = key


def _attn_key(B, T, Hq, Hkv, D, bs, max_ctx, unit_blocks, key_waves, dtype):
    return (B, T, Hq, Hkv, D, bs, int(max_ctx), int(unit_blocks), int(key_waves), dtype)


def attn_workspace_bytes(num_seqs, q_len, num_q_heads, num_kv_heads, head_dim, block_size,
                         max_ctx, unit_blocks, key_waves, dtype) -> int:
    code = _lib.DTYPE_BF16 if dtype == torch.bfloat16 else _lib.DTYPE_F32
    return int(_lib.lib().kve_attn_workspace_bytes(num_seqs, q_len, num_q_heads, num_kv_heads,
                                                   head_dim, block_size, max_ctx, unit_blocks,
                                                   key_waves, code))


def _attn_checks(block_tables, start_pos, seq_rows, q_lens, B, bs, max_ctx, dev):
    for t, n in ((block_tables, "block_tables"), (start_pos, "start_pos"), (seq_rows, "seq_rows"),
                 (q_lens, "q_lens")):
        _check_i32(t, n, dev)
    _need(block_tables.dim() == 2, "block_tables must be [rows, max_blocks]")
    max_blocks = block_tables.shape[1]
    _need(max_ctx >= 1 and max_blocks * bs >= max_ctx,
          f"max_ctx {max_ctx} exceeds table capacity {max_blocks * bs}")
    num_rows = block_tables.shape[0]
    _need(start_pos.numel() >= num_rows, "start_pos needs one entry per table row")
    if seq_rows is not None:
        _need(seq_rows.numel() == B, "seq_rows must have one entry per sequence")
    else:
        _need(num_rows >= B, "too few table rows")
    if q_lens is not None:
        _need(q_lens.numel() == B, "q_lens must have one entry per sequence")
    return max_blocks, num_rows


def attn_plan(block_tables: torch.Tensor, start_pos: torch.Tensor, num_seqs: int, q_len: int,
              num_q_heads: int, num_kv_heads: int, head_dim: int, block_size: int,
              num_blocks: int, max_ctx: int, dtype, seq_rows: torch.Tensor | None = None,
              q_lens: torch.Tensor | None = None, unit_blocks: int = 0,
              key_waves: int = 0) -> AttnPlan:
    """Work plan of paged_verify_attn for every layer of one forward pass
    (kve_attn_plan). The buffer is cached per device, stream and size, and a
    plan is meant to be used by the launches queued after it on the same
    stream, before the next plan of that size."""
    dev = block_tables.device
    max_blocks, num_rows = _attn_checks(block_tables, start_pos, seq_rows, q_lens, num_seqs,
                                        block_size, max_ctx, dev)
    code = _lib.DTYPE_BF16 if dtype == torch.bfloat16 else _lib.DTYPE_F32
    nbytes = int(_lib.lib().kve_attn_plan_bytes(num_seqs, q_len, num_q_heads, num_kv_heads,
                                                head_dim, block_size, max_ctx, unit_blocks,
                                                key_waves, code))
    buf = workspace("attn_plan", nbytes, dev)
    rc = _lib.lib().kve_attn_plan(block_tables.data_ptr(), _ptr(seq_rows), start_pos.data_ptr(),
                                  _ptr(q_lens), num_seqs, q_len, num_q_heads, num_kv_heads,
                                  head_dim, block_size, max_blocks, num_rows, num_blocks,
                                  int(max_ctx), int(unit_blocks), int(key_waves), code,
                                  buf.data_ptr(), buf.numel() * buf.element_size(), _stream(dev))
    _lib.check(rc, "kve_attn_plan")
    return AttnPlan(buf, _attn_key(num_seqs, q_len, num_q_heads, num_kv_heads, head_dim,
                                   block_size, max_ctx, unit_blocks, key_waves, dtype))


def paged_verify_attn(q: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor,
                      block_tables: torch.Tensor, start_pos: torch.Tensor, max_ctx: int,
                      seq_rows: torch.Tensor | None = None, q_lens: torch.Tensor | None = None,
                      scale: float | None = None, unit_blocks: int = 0, key_waves: int = 0,
                      plan: AttnPlan | None = None, out: torch.Tensor | None = None,
                      ws: torch.Tensor | None = None, blocked: bool = False) -> torch.Tensor:
    """q [B, T, Hq, D]; k_layer [NB, Hkv, bs, D]; v_layer [NB, Hkv, D, bs].

    start_pos[row] is the committed length before this pass (the new tokens'
    K/V must already be written). unit_blocks / key_waves fix the summation
    order (0: chosen per launch). plan: from attn_plan with the same arguments
    (else the launch builds its own). Returns out [B, T, Hq, D]; blocked: out
    is the [B*T, Hq*D] matrix in the blocked layout (blocked_matrix), bf16 only.
    """
    dev = q.device
    _need(q.dim() == 4 and q.is_contiguous(), "q must be contiguous [B, T, Hq, D]")
    B, T, Hq, D = q.shape
    _need(k_layer.dim() == 4 and v_layer.dim() == 4, "k/v layer must be 4-d")
    NB, Hkv, bs, Dk = k_layer.shape
    _need(Dk == D and tuple(v_layer.shape) == (NB, Hkv, D, bs),
          f"pool shapes k{tuple(k_layer.shape)} v{tuple(v_layer.shape)} do not match q D={D}")
    _need(k_layer.is_contiguous() and v_layer.is_contiguous(), "k/v layer must be contiguous")
    _need(k_layer.dtype == q.dtype == v_layer.dtype, "q/k/v dtype mismatch")
    _need(Hq % Hkv == 0, f"{Hq} q heads not a multiple of {Hkv} kv heads")
    max_blocks, num_rows = _attn_checks(block_tables, start_pos, seq_rows, q_lens, B, bs, max_ctx,
                                        dev)
    if plan is not None:
        _need(plan.key == _attn_key(B, T, Hq, Hkv, D, bs, max_ctx, unit_blocks, key_waves, q.dtype),
              "attention plan was built for another shape or configuration")
    if blocked:
        _need(q.dtype == torch.bfloat16 and (Hq * D) % 32 == 0, "blocked out is bf16, Hq*D % 32")
        if out is None:
            out = blocked_matrix(B * T, Hq * D, dev)
        _need(out.dtype == q.dtype and out.is_contiguous()
              and out.numel() >= blocked_rows(B * T) * Hq * D, "bad blocked out")
    elif out is None:
        out = torch.empty_like(q)
    else:
        _need(out.shape == q.shape and out.dtype == q.dtype and out.is_contiguous(), "bad out")
    scale = D ** -0.5 if scale is None else scale
    nbytes = attn_workspace_bytes(B, T, Hq, Hkv, D, bs, max_ctx, unit_blocks, key_waves, q.dtype)
    if ws is None:
        ws = workspace("attn_partials", nbytes, dev)
    _need(ws.numel() * ws.element_size() >= nbytes, "attention workspace too small")
    rc = _lib.lib().kve_paged_verify_attn(
        q.data_ptr(), k_layer.data_ptr(), v_layer.data_ptr(), block_tables.data_ptr(),
        _ptr(seq_rows), start_pos.data_ptr(), _ptr(q_lens), B, T, Hq, Hkv, D, bs, max_blocks,
        num_rows, NB, int(max_ctx), int(unit_blocks), int(key_waves), float(scale),
        _dtype_code(q), None if plan is None else plan.buf.data_ptr(), out.data_ptr(),
        ws.data_ptr(), ws.numel() * ws.element_size(), _layout(blocked), _stream(dev))
    _lib.check(rc, "kve_paged_verify_attn")
    return out


def kv_write(k_new: torch.Tensor, v_new: torch.Tensor, k_layer: torch.Tensor,
             v_layer: torch.Tensor, block_tables: torch.Tensor, start_pos: torch.Tensor,
             seq_rows: torch.Tensor | None = None, q_lens: torch.Tensor | None = None) -> None:
    """k_new/v_new [B, T, Hkv, D] (token rows may be strided, channels contiguous)."""
    dev = k_new.device
    _need(k_new.dim() == 4 and k_new.shape == v_new.shape, "k_new/v_new must be [B, T, Hkv, D]")
    B, T, Hkv, D = k_new.shape
    _need(k_new.stride() == v_new.stride(), "k_new/v_new strides differ")
    st = k_new.stride()
    _need(st[3] == 1 and st[2] == D and st[0] == T * st[1],
          f"k_new layout {tuple(st)} not [B, T, Hkv, D] with contiguous heads")
    NB, Hkv2, bs, D2 = k_layer.shape
    _need(Hkv2 == Hkv and D2 == D and tuple(v_layer.shape) == (NB, Hkv, D, bs), "pool shape")
    _need(k_new.dtype == k_layer.dtype == v_layer.dtype == v_new.dtype, "dtype mismatch")
    for t, n in ((block_tables, "block_tables"), (start_pos, "start_pos"), (seq_rows, "seq_rows"),
                 (q_lens, "q_lens")):
        _check_i32(t, n, dev)
    _need(k_new.data_ptr() % 16 == 0 and v_new.data_ptr() % 16 == 0, "k_new/v_new not 16-byte aligned")
    num_rows = block_tables.shape[0]
    _need(start_pos.numel() >= num_rows, "start_pos needs one entry per table row")
    _need(seq_rows is not None or num_rows >= B, "too few table rows")
    rc = _lib.lib().kve_kv_write(
        k_new.data_ptr(), v_new.data_ptr(), st[1], k_layer.data_ptr(), v_layer.data_ptr(),
        block_tables.data_ptr(), _ptr(seq_rows), start_pos.data_ptr(), _ptr(q_lens), B, T, Hkv,
        D, bs, block_tables.shape[1], num_rows, NB, _dtype_code(k_new), _stream(dev))
    _lib.check(rc, "kve_kv_write")


def commit(lens: torch.Tensor, num_seqs: int, q_len: int, seq_rows: torch.Tensor | None = None,
           q_lens: torch.Tensor | None = None) -> None:
    _check_i32(lens, "lens", lens.device)
    _need(seq_rows is not None or lens.numel() >= num_seqs, "too few length rows")
    rc = _lib.lib().kve_commit(lens.data_ptr(), lens.numel(), _ptr(seq_rows), _ptr(q_lens),
                               num_seqs, q_len, _stream(lens.device))
    _lib.check(rc, "kve_commit")


def rollback(block_tables: torch.Tensor, lens: torch.Tensor, keep_lens: torch.Tensor,
             block_size: int, seq_rows: torch.Tensor | None = None) -> None:
    dev = lens.device
    for t, n in ((block_tables, "block_tables"), (lens, "lens"), (keep_lens, "keep_lens"),
                 (seq_rows, "seq_rows")):
        _check_i32(t, n, dev)
    n = keep_lens.numel()
    _need(block_tables.shape[0] == lens.numel(), "one length per table row")
    _need(seq_rows is not None or lens.numel() >= n, "too few table rows")
    rc = _lib.lib().kve_rollback(block_tables.data_ptr(), lens.data_ptr(), lens.numel(),
                                 _ptr(seq_rows), keep_lens.data_ptr(), n, block_tables.shape[1],
                                 block_size, _stream(dev))
    _lib.check(rc, "kve_rollback")


def lmhead_argmax(hidden: torch.Tensor, weight: torch.Tensor, argmax: torch.Tensor | None = None,
                  maxval: torch.Tensor | None = None, ws: torch.Tensor | None = None,
                  second_id: torch.Tensor | None = None, second_val: torch.Tensor | None = None,
                  blocked: bool = False, rows: int | None = None):
    """hidden [M, H] (row-strided), weight [V, H] -> argmax [M] int32.

    maxval [M] f32 receives the rounded row maximum; second_id [M] int32 and
    second_val [M] f32 (either or both) the runner-up, the largest logit at any
    other id (ties: the lowest such id), which costs a second atomic per
    workgroup and row. Returns argmax alone, or (argmax, maxval) when maxval is
    given; the runner-up buffers are filled in place. blocked: hidden (its first
    `rows` rows are read) and weight are blocked matrices (blocked_matrix,
    to_blocked), bf16 only."""
    dev = hidden.device
    _need(hidden.dim() == 2 and hidden.stride(1) == 1, "hidden must be [M, H] with unit column stride")
    _need(weight.dim() == 2 and weight.is_contiguous(), "weight must be contiguous [V, H]")
    M, H = hidden.shape
    if blocked:
        M = M if rows is None else rows
        _need(hidden.is_contiguous() and hidden.shape[0] >= blocked_rows(M), "blocked hidden")
    V, H2 = weight.shape
    _need(H == H2, f"hidden width {H} != weight width {H2}")
    _need(hidden.dtype == weight.dtype, "hidden/weight dtype mismatch")
    if argmax is None:
        argmax = torch.empty(M, dtype=torch.int32, device=dev)
    _check_i32(argmax, "argmax", dev)
    _need(argmax.numel() >= M, "argmax too small")
    if maxval is not None:
        _need(maxval.dtype == torch.float32 and maxval.numel() >= M, "maxval must be f32 [M]")
    if second_id is not None:
        _check_i32(second_id, "second_id", dev)
        _need(second_id.numel() >= M, "second_id too small")
    if second_val is not None:
        _need(second_val.dtype == torch.float32 and second_val.numel() >= M,
              "second_val must be f32 [M]")
    nbytes = int(_lib.lib().kve_lmhead_workspace_bytes(M))
    if ws is None:
        ws = workspace("lmhead_keys", nbytes, dev)
    _need(ws.numel() * ws.element_size() >= nbytes, "lmhead workspace too small")
    rc = _lib.lib().kve_lmhead_argmax(hidden.data_ptr(), hidden.stride(0), weight.data_ptr(), M, H,
                                      V, _dtype_code(hidden), argmax.data_ptr(), _ptr(maxval),
                                      _ptr(second_id), _ptr(second_val), ws.data_ptr(),
                                      ws.numel() * ws.element_size(), _layout(blocked), _stream(dev))
    _lib.check(rc, "kve_lmhead_argmax")
    return argmax if maxval is None else (argmax, maxval)


def accept(drafts: torch.Tensor, preds: torch.Tensor, lens: torch.Tensor | None = None,
           seq_rows: torch.Tensor | None = None, n_acc=None, emitted=None, keep=None):
    """drafts [B, k], preds [B, k+1] int32 -> (n_acc [B], emitted [B, k+1], keep [B] or None)."""
    dev = drafts.device
    _need(drafts.dim() == 2 and preds.dim() == 2, "drafts [B, k], preds [B, k+1]")
    B, k = drafts.shape
    _need(tuple(preds.shape) == (B, k + 1), f"preds shape {tuple(preds.shape)} != ({B}, {k + 1})")
    for t, nm in ((drafts, "drafts"), (preds, "preds"), (lens, "lens"), (seq_rows, "seq_rows")):
        _check_i32(t, nm, dev)
    if n_acc is None:
        n_acc = torch.empty(B, dtype=torch.int32, device=dev)
    if emitted is None:
        emitted = torch.empty(B, k + 1, dtype=torch.int32, device=dev)
    if keep is None and lens is not None:
        keep = torch.empty(B, dtype=torch.int32, device=dev)
    num_rows = 0 if lens is None else lens.numel()
    _need(lens is None or seq_rows is not None or num_rows >= B, "too few length rows")
    rc = _lib.lib().kve_accept(drafts.data_ptr(), preds.data_ptr(), _ptr(lens), num_rows,
                               _ptr(seq_rows), B, k, n_acc.data_ptr(), emitted.data_ptr(),
                               _ptr(keep), _stream(dev))
    _lib.check(rc, "kve_accept")
    return n_acc, emitted, keep


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, delta: torch.Tensor | None = None,
            residual_out: torch.Tensor | None = None, out: torch.Tensor | None = None,
            blocked: bool = False) -> torch.Tensor:
    """out = weight * cast(r * rsqrt(mean(r^2) + eps)) with r = x (+ delta); r is
    written to residual_out when given (may be x itself). Rows are the last dim.
    blocked: out is the [rows, H] blocked matrix (bf16)."""
    H = x.shape[-1]
    _need(x.is_contiguous() and weight.numel() == H and weight.dtype == x.dtype, "rmsnorm shapes")
    rows = x.numel() // H
    for t in (delta, residual_out):
        if t is not None:
            _need(t.shape == x.shape and t.dtype == x.dtype and t.is_contiguous(), "rmsnorm operand")
    if out is None:
        out = blocked_matrix(rows, H, x.device, x.dtype) if blocked else torch.empty_like(x)
    if blocked:
        _need(out.is_contiguous() and out.numel() >= blocked_rows(rows) * H, "blocked out")
    rc = _lib.lib().kve_rmsnorm(x.data_ptr(), _ptr(delta), _ptr(residual_out), weight.data_ptr(),
                                out.data_ptr(), rows, H, float(eps), _dtype_code(x),
                                _layout(blocked), _stream(x.device))
    _lib.check(rc, "kve_rmsnorm")
    return out


def rope_kv_write(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, k_layer: torch.Tensor,
                  v_layer: torch.Tensor, block_tables: torch.Tensor, start_pos: torch.Tensor,
                  num_q_heads: int, seq_rows: torch.Tensor | None = None,
                  q_lens: torch.Tensor | None = None, q_out: torch.Tensor | None = None) -> torch.Tensor:
    """qkv [B, T, (Hq+2Hkv)*D] -> rotated q [B, T, Hq, D]; rotated k and v go to the pool."""
    dev = qkv.device
    _need(qkv.dim() == 3 and qkv.is_contiguous(), "qkv must be contiguous [B, T, width]")
    B, T, width = qkv.shape
    NB, Hkv, bs, D = k_layer.shape
    _need(width == (num_q_heads + 2 * Hkv) * D, f"qkv width {width} != ({num_q_heads}+2*{Hkv})*{D}")
    _need(tuple(v_layer.shape) == (NB, Hkv, D, bs), "pool shape")
    _need(cos.shape[-1] == D and cos.numel() == B * T * D and sin.shape == cos.shape, "cos/sin shape")
    _need(cos.is_contiguous() and sin.is_contiguous(), "cos/sin must be contiguous")
    _need(qkv.dtype == cos.dtype == sin.dtype == k_layer.dtype == v_layer.dtype, "dtype mismatch")
    for t, n in ((block_tables, "block_tables"), (start_pos, "start_pos"), (seq_rows, "seq_rows"),
                 (q_lens, "q_lens")):
        _check_i32(t, n, dev)
    num_rows = block_tables.shape[0]
    _need(start_pos.numel() >= num_rows, "start_pos needs one entry per table row")
    _need(seq_rows is not None or num_rows >= B, "too few table rows")
    if q_out is None:
        q_out = torch.empty(B, T, num_q_heads, D, dtype=qkv.dtype, device=dev)
    rc = _lib.lib().kve_rope_kv_write(
        qkv.data_ptr(), cos.data_ptr(), sin.data_ptr(), q_out.data_ptr(), k_layer.data_ptr(),
        v_layer.data_ptr(), block_tables.data_ptr(), _ptr(seq_rows), start_pos.data_ptr(),
        _ptr(q_lens), B, T, num_q_heads, Hkv, D, bs, block_tables.shape[1], num_rows, NB,
        _dtype_code(qkv), _stream(dev))
    _lib.check(rc, "kve_rope_kv_write")
    return q_out


def pass_prologue(ids: torch.Tensor, embed: torch.Tensor, lens: torch.Tensor, seq_rows: torch.Tensor,
                  cos_table: torch.Tensor, sin_table: torch.Tensor):
    """ids [B, T] int64 -> (embed[ids] [B, T, H], cos [B, T, D], sin [B, T, D]) at
    positions lens[seq_rows[b]] + t (clamped to the table), one launch. A
    seq_rows entry outside [0, lens.numel()) is not dereferenced on the device
    (its tokens take positions t = 0, 1, ...)."""
    dev = ids.device
    _need(ids.dim() == 2 and ids.dtype == torch.int64, "ids must be int64 [B, T]")
    ids = ids.contiguous()
    B, T = ids.shape
    V, H = embed.shape
    P, D = cos_table.shape
    _need(embed.dtype == cos_table.dtype == sin_table.dtype == torch.bfloat16, "bf16 tables")
    _need(embed.is_contiguous() and cos_table.is_contiguous() and sin_table.is_contiguous()
          and tuple(sin_table.shape) == (P, D), "contiguous embedding and RoPE tables")
    _check_i32(lens, "lens", dev)
    _check_i32(seq_rows, "seq_rows", dev)
    _need(seq_rows.numel() >= B, "one table row per sequence")
    hidden = torch.empty(B, T, H, dtype=embed.dtype, device=dev)
    cos = torch.empty(B, T, D, dtype=embed.dtype, device=dev)
    sin = torch.empty(B, T, D, dtype=embed.dtype, device=dev)
    _need(lens.numel() > 0, "lens must hold at least one table row")
    rc = _lib.lib().kve_pass_prologue(ids.data_ptr(), embed.data_ptr(), V, H, lens.data_ptr(),
                                      seq_rows.data_ptr(), lens.numel(), B, T, cos_table.data_ptr(),
                                      sin_table.data_ptr(), P, D, hidden.data_ptr(), cos.data_ptr(),
                                      sin.data_ptr(), _stream(dev))
    _lib.check(rc, "kve_pass_prologue")
    return hidden, cos, sin


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """gate_up [..., 2F] -> silu(gate) * up [..., F]."""
    _need(gate_up.is_contiguous() and gate_up.shape[-1] % 2 == 0, "gate_up must be contiguous [.., 2F]")
    F2 = gate_up.shape[-1]
    rows = gate_up.numel() // F2
    if out is None:
        out = torch.empty(*gate_up.shape[:-1], F2 // 2, dtype=gate_up.dtype, device=gate_up.device)
    rc = _lib.lib().kve_silu_mul(gate_up.data_ptr(), out.data_ptr(), rows, F2 // 2,
                                 _dtype_code(gate_up), _stream(gate_up.device))
    _lib.check(rc, "kve_silu_mul")
    return out


# ---- fused skinny projections (bf16, decode-sized batches) ---------------------

FUSED_MAX_ROWS = 64
_LDS_BYTES = 159 * 1024


def fused_fits(rows: int, hidden: int, head_dim: int) -> bool:
    """Whether rows x hidden fits the fused projections' LDS staging."""
    if rows <= 0 or rows > FUSED_MAX_ROWS or hidden % 32 or hidden > 2048:
        return False
    mp = -(-rows // 16) * 16
    return mp * (hidden + 8) * 2 + mp * max(head_dim + 1, 64) * 4 <= _LDS_BYTES


def fused_qkv(residual: torch.Tensor, norm_weight: torch.Tensor, eps: float, weight: torch.Tensor,
              bias: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, k_layer: torch.Tensor,
              v_layer: torch.Tensor, block_tables: torch.Tensor, start_pos: torch.Tensor,
              num_q_heads: int, seq_rows: torch.Tensor | None = None,
              q_lens: torch.Tensor | None = None, q_out: torch.Tensor | None = None,
              blocked_w: bool = False) -> torch.Tensor:
    """RMSNorm(residual [B, T, H]) -> [q|k|v] projection + bias -> RoPE; k/v to the pool,
    rotated q [B, T, Hq, D] returned (blocked_w: weight is a blocked matrix)."""
    dev = residual.device
    _need(residual.dim() == 3 and residual.is_contiguous(), "residual must be contiguous [B, T, H]")
    B, T, H = residual.shape
    NB, Hkv, bs, D = k_layer.shape
    _need(residual.dtype == torch.bfloat16, "fused_qkv is bf16 only")
    _need(tuple(weight.shape) == ((num_q_heads + 2 * Hkv) * D, H) and weight.is_contiguous(),
          "qkv weight shape")
    _need(bias.numel() == weight.shape[0] and norm_weight.numel() == H, "bias / norm weight")
    _need(tuple(v_layer.shape) == (NB, Hkv, D, bs), "pool shape")
    _need(cos.numel() == B * T * D and sin.shape == cos.shape and cos.is_contiguous()
          and sin.is_contiguous(), "cos/sin shape")
    for t, n in ((block_tables, "block_tables"), (start_pos, "start_pos"), (seq_rows, "seq_rows"),
                 (q_lens, "q_lens")):
        _check_i32(t, n, dev)
    num_rows = block_tables.shape[0]
    _need(seq_rows is not None or num_rows >= B, "too few table rows")
    if q_out is None:
        q_out = torch.empty(B, T, num_q_heads, D, dtype=residual.dtype, device=dev)
    rc = _lib.lib().kve_fused_qkv(
        residual.data_ptr(), norm_weight.data_ptr(), float(eps), weight.data_ptr(), bias.data_ptr(),
        cos.data_ptr(), sin.data_ptr(), q_out.data_ptr(), k_layer.data_ptr(), v_layer.data_ptr(),
        block_tables.data_ptr(), _ptr(seq_rows), start_pos.data_ptr(), _ptr(q_lens), B, T, H,
        num_q_heads, Hkv, D, bs, block_tables.shape[1], num_rows, NB, _layout(blocked_w), _stream(dev))
    _lib.check(rc, "kve_fused_qkv")
    return q_out


def linear_residual(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor,
                    blocked_w: bool = False) -> torch.Tensor:
    """residual += cast(x @ weight^T) in place (bf16); x [..., in], residual [..., out]
    (blocked_w: weight is a blocked matrix)."""
    _need(x.dtype == weight.dtype == residual.dtype == torch.bfloat16, "linear_residual is bf16 only")
    _need(x.is_contiguous() and weight.is_contiguous() and residual.is_contiguous(), "contiguous")
    N, K = weight.shape
    rows = x.numel() // K
    _need(x.shape[-1] == K and residual.numel() == rows * N, "linear_residual shapes")
    rc = _lib.lib().kve_linear_residual(x.data_ptr(), weight.data_ptr(), residual.data_ptr(), rows,
                                        N, K, _layout(blocked_w), _stream(x.device))
    _lib.check(rc, "kve_linear_residual")
    return residual


def fused_gate_up(residual: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                  weight: torch.Tensor, act: torch.Tensor | None = None,
                  blocked_w: bool = False, blocked_act: bool = False) -> torch.Tensor:
    """RMSNorm(residual [..., H]) -> [gate|up] projection -> silu(gate) * up [..., F]
    (blocked_w: weight is a blocked matrix; blocked_act: act is returned as the
    [rows, F] blocked matrix, for linear_splitk)."""
    _need(residual.dtype == weight.dtype == torch.bfloat16, "fused_gate_up is bf16 only")
    _need(residual.is_contiguous() and weight.is_contiguous(), "contiguous")
    H = residual.shape[-1]
    F2, K = weight.shape
    _need(K == H and F2 % 2 == 0 and norm_weight.numel() == H, "gate_up shapes")
    rows = residual.numel() // H
    F = F2 // 2
    if act is None:
        act = (blocked_matrix(rows, F, residual.device) if blocked_act else
               torch.empty(*residual.shape[:-1], F, dtype=residual.dtype, device=residual.device))
    _need(act.dtype == torch.bfloat16 and act.is_contiguous()
          and act.numel() >= (blocked_rows(rows) if blocked_act else rows) * F, "act buffer")
    rc = _lib.lib().kve_fused_gate_up(residual.data_ptr(), norm_weight.data_ptr(), float(eps),
                                      weight.data_ptr(), act.data_ptr(), rows, H, F,
                                      _layout(blocked_w), _layout(blocked_act),
                                      _stream(residual.device))
    _lib.check(rc, "kve_fused_gate_up")
    return act


# ---- split-K layers (bf16: decode layer up to 64 rows, wide layer up to 160) ----


def splitk_slices(out_features: int, in_features: int) -> int:
    """k-slices the split-K projection uses for a [out, in] weight (shape only)."""
    return int(_lib.lib().kve_splitk_slices(out_features, in_features))


def linear_splitk(x: torch.Tensor, weight: torch.Tensor, partials: torch.Tensor | None = None,
                  blocked: bool = False, rows: int | None = None):
    """fp32 partial products [S, rows, out] of x [..., in] @ weight^T over S k-slices.
    blocked: x (its first `rows` rows) and weight are blocked matrices."""
    _need(x.dtype == weight.dtype == torch.bfloat16, "linear_splitk is bf16 only")
    _need(x.is_contiguous() and weight.is_contiguous(), "contiguous")
    N, K = weight.shape
    if rows is None:
        rows = x.numel() // K
    _need(x.shape[-1] == K and x.numel() >= (blocked_rows(rows) if blocked else rows) * K,
          "linear_splitk shapes")
    S = splitk_slices(N, K)
    if partials is None:
        partials = torch.empty(S, rows, N, dtype=torch.float32, device=x.device)
    _need(partials.dtype == torch.float32 and partials.is_contiguous()
          and partials.numel() >= S * rows * N, "partials buffer")
    rc = _lib.lib().kve_linear_splitk(x.data_ptr(), weight.data_ptr(), partials.data_ptr(), rows, N,
                                      K, S, _layout(blocked), _stream(x.device))
    _lib.check(rc, "kve_linear_splitk")
    return partials


def residual_norm(partials: torch.Tensor, slices: int, residual: torch.Tensor,
                  norm_weight: torch.Tensor, eps: float, xn: torch.Tensor | None = None,
                  blocked: bool = False):
    """residual += cast(sum of the slices) in place; returns xn = RMSNorm(residual)
    (blocked: xn is the [rows, H] blocked matrix)."""
    H = residual.shape[-1]
    rows = residual.numel() // H
    _need(residual.dtype == norm_weight.dtype == torch.bfloat16 and residual.is_contiguous(),
          "residual_norm is bf16, contiguous")
    _need(partials.dtype == torch.float32 and partials.is_contiguous()
          and partials.numel() >= slices * rows * H, "partials buffer")
    if xn is None:
        xn = blocked_matrix(rows, H, residual.device) if blocked else torch.empty_like(residual)
    _need(xn.is_contiguous() and xn.numel() >= (blocked_rows(rows) if blocked else rows) * H,
          "xn buffer")
    rc = _lib.lib().kve_residual_norm(partials.data_ptr(), slices, residual.data_ptr(),
                                      norm_weight.data_ptr(), float(eps), xn.data_ptr(), rows, H,
                                      _layout(blocked), _stream(residual.device))
    _lib.check(rc, "kve_residual_norm")
    return xn


def kv_slots(block_tables: torch.Tensor, start_pos: torch.Tensor, num_seqs: int, q_len: int,
             block_size: int, num_blocks: int, seq_rows: torch.Tensor | None = None,
             q_lens: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Pool slot (block * bs + offset) of each new token [num_seqs * q_len], -1 for none."""
    dev = block_tables.device
    for t, n in ((block_tables, "block_tables"), (start_pos, "start_pos"), (seq_rows, "seq_rows"),
                 (q_lens, "q_lens")):
        _check_i32(t, n, dev)
    num_rows = block_tables.shape[0]
    _need(seq_rows is not None or num_rows >= num_seqs, "too few table rows")
    if out is None:
        out = torch.empty(num_seqs * q_len, dtype=torch.int32, device=dev)
    rc = _lib.lib().kve_kv_slots(block_tables.data_ptr(), _ptr(seq_rows), start_pos.data_ptr(),
                                 _ptr(q_lens), num_seqs, q_len, block_size, block_tables.shape[1],
                                 num_rows, num_blocks, out.data_ptr(), _stream(dev))
    _lib.check(rc, "kve_kv_slots")
    return out


def qkv_rope(xn: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, cos: torch.Tensor,
             sin: torch.Tensor, slots: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor,
             num_q_heads: int, q_out: torch.Tensor | None = None, blocked: bool = False,
             bt: tuple[int, int] | None = None) -> torch.Tensor:
    """Normalised rows xn [B, T, H] -> [q|k|v] + bias -> RoPE; k/v written at `slots`,
    rotated q [B, T, Hq, D] returned. blocked: xn is the [B*T, H] blocked matrix
    (B, T given by bt) and weight is blocked."""
    dev = xn.device
    if blocked:
        B, T = bt
        H = xn.shape[-1]
        _need(xn.is_contiguous() and xn.dtype == torch.bfloat16
              and xn.numel() >= blocked_rows(B * T) * H, "blocked xn")
    else:
        _need(xn.dim() == 3 and xn.is_contiguous() and xn.dtype == torch.bfloat16,
              "xn [B, T, H] bf16")
        B, T, H = xn.shape
    NB, Hkv, bs, D = k_layer.shape
    _need(tuple(weight.shape) == ((num_q_heads + 2 * Hkv) * D, H) and weight.is_contiguous(),
          "qkv weight shape")
    _need(bias.numel() == weight.shape[0] and tuple(v_layer.shape) == (NB, Hkv, D, bs), "bias/pool")
    _need(cos.numel() == B * T * D and sin.shape == cos.shape and cos.is_contiguous()
          and sin.is_contiguous(), "cos/sin shape")
    _check_i32(slots, "slots", dev)
    _need(slots.numel() >= B * T, "one slot per row")
    if q_out is None:
        q_out = torch.empty(B, T, num_q_heads, D, dtype=xn.dtype, device=dev)
    rc = _lib.lib().kve_qkv_rope(xn.data_ptr(), weight.data_ptr(), bias.data_ptr(), cos.data_ptr(),
                                 sin.data_ptr(), slots.data_ptr(), q_out.data_ptr(),
                                 k_layer.data_ptr(), v_layer.data_ptr(), B * T, H, num_q_heads, Hkv,
                                 D, bs, _layout(blocked), _stream(dev))
    _lib.check(rc, "kve_qkv_rope")
    return q_out


def qkv_part_rope(partials: torch.Tensor, bias: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                  slots: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor,
                  num_q_heads: int, rows: int, q_out: torch.Tensor | None = None) -> torch.Tensor:
    """Split-K [q|k|v] partials [S, rows, (Hq + 2 Hkv) D] -> sum + bias -> RoPE; k/v
    written at `slots`, rotated q [rows, Hq, D] returned (as qkv_rope)."""
    dev = partials.device
    NB, Hkv, bs, D = k_layer.shape
    N = (num_q_heads + 2 * Hkv) * D
    _need(partials.dtype == torch.float32 and partials.is_contiguous() and partials.dim() == 3
          and partials.shape[1] == rows and partials.shape[2] == N, "partials [S, rows, N] fp32")
    _need(bias.numel() == N and bias.dtype == torch.bfloat16 and k_layer.dtype == torch.bfloat16
          and tuple(v_layer.shape) == (NB, Hkv, D, bs), "bias/pool")
    _need(cos.numel() == rows * D and sin.shape == cos.shape and cos.is_contiguous()
          and sin.is_contiguous(), "cos/sin shape")
    _check_i32(slots, "slots", dev)
    _need(slots.numel() >= rows, "one slot per row")
    if q_out is None:
        q_out = torch.empty(rows, num_q_heads, D, dtype=torch.bfloat16, device=dev)
    rc = _lib.lib().kve_qkv_part_rope(partials.data_ptr(), partials.shape[0], bias.data_ptr(),
                                      cos.data_ptr(), sin.data_ptr(), slots.data_ptr(),
                                      q_out.data_ptr(), k_layer.data_ptr(), v_layer.data_ptr(), rows,
                                      num_q_heads, Hkv, D, bs, _stream(dev))
    _lib.check(rc, "kve_qkv_part_rope")
    return q_out


def gate_up_silu(xn: torch.Tensor, weight: torch.Tensor, act: torch.Tensor | None = None,
                 blocked: bool = False, rows: int | None = None):
    """Normalised rows xn [..., H] -> [gate|up] projection -> cast(silu(gate)) * up [..., F].
    blocked: xn (first `rows` rows), weight and act are blocked matrices."""
    _need(xn.dtype == weight.dtype == torch.bfloat16 and xn.is_contiguous()
          and weight.is_contiguous(), "gate_up_silu is bf16, contiguous")
    H = xn.shape[-1]
    F2, K = weight.shape
    _need(K == H and F2 % 2 == 0, "gate_up shapes")
    if rows is None:
        rows = xn.numel() // H
    if act is None:
        act = (blocked_matrix(rows, F2 // 2, xn.device) if blocked
               else torch.empty(*xn.shape[:-1], F2 // 2, dtype=xn.dtype, device=xn.device))
    if blocked:
        _need(xn.numel() >= blocked_rows(rows) * H and act.is_contiguous()
              and act.numel() >= blocked_rows(rows) * (F2 // 2), "blocked xn / act")
    rc = _lib.lib().kve_gate_up_silu(xn.data_ptr(), weight.data_ptr(), act.data_ptr(), rows, H,
                                     F2 // 2, _layout(blocked), _stream(xn.device))
    _lib.check(rc, "kve_gate_up_silu")
    return act


# kve_linear_rows modes
ROWS_RESIDUAL, ROWS_QKV, ROWS_GATE_UP = 0, 1, 2


def linear_rows(x: torch.Tensor, weight: torch.Tensor, mode: int, out: torch.Tensor | None = None,
                blocked: bool = False, rows: int | None = None):
    """The split-K layer's projection for any number of rows, each row bit-identical
    to linear_splitk + its reduction (mode ROWS_RESIDUAL: residual_norm's order,
    ROWS_QKV: qkv_part_rope's order; fp32 partials [S, rows, out] with S = 1 (the
    whole sum) or every k-slice, for the reductions to finish) or to gate_up_silu
    (ROWS_GATE_UP: bf16 act [rows, ffn]). blocked: x (its first `rows` rows),
    weight and the mode-2 act are blocked matrices."""
    _need(x.dtype == weight.dtype == torch.bfloat16 and x.is_contiguous()
          and weight.is_contiguous(), "linear_rows is bf16, contiguous")
    N, K = weight.shape
    _need(x.shape[-1] == K, "linear_rows shapes")
    if rows is None:
        rows = x.numel() // K
    _need(x.numel() >= (blocked_rows(rows) if blocked else rows) * K, "linear_rows x rows")
    lib = _lib.lib()
    if mode == ROWS_GATE_UP:
        shape = (blocked_rows(rows) if blocked else rows, N // 2)
        dtype = torch.bfloat16
    else:
        S = lib.kve_linear_rows_slices(rows, N, K, int(mode))
        _need(S >= 1, "linear_rows sizes")
        shape, dtype = (S, rows, N), torch.float32
    if out is None:
        out = torch.empty(*shape, dtype=dtype, device=x.device)
    _need(out.dtype == dtype and out.is_contiguous() and tuple(out.shape) == shape,
          "linear_rows output")
    rc = lib.kve_linear_rows(x.data_ptr(), weight.data_ptr(), out.data_ptr(), rows, N, K,
                             int(mode), _layout(blocked), _stream(x.device))
    _lib.check(rc, "kve_linear_rows")
    return out
