"""The C-ABI library loads without a GPU and exports every function kve.h declares."""

import os
import re

from conftest import REPO


def declared_functions():
    text = open(os.path.join(REPO, "include", "kve.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kve_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_verify_path():
    names = declared_functions()
    for required in ("kve_paged_verify_attn", "kve_kv_write", "kve_rollback",
                     "kve_lmhead_argmax", "kve_accept", "kve_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from kvengine_amd import _lib

    lib = _lib.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared_functions()) == set(_lib.EXPORTS)
    assert lib.kve_version().decode().endswith("gfx950")


def test_error_paths_need_no_gpu():
    """Argument validation happens on the host and reports through kve_last_error."""
    from kvengine_amd import _lib

    lib = _lib.lib()
    rc = lib.kve_paged_verify_attn(None, None, None, None, None, None, None, 1, 5, 14, 2, 64, 16,
                                   8, 1, 8, 128, 0, 0, 0.125, 1, None, None, None, 0, 0, None)
    assert rc == -1
    assert b"null pointer" in lib.kve_last_error()
    assert lib.kve_lmhead_workspace_bytes(160) >= 160 * 8
    # long histories need unit states; a plan buffer holds one 256-byte record per unit
    assert lib.kve_attn_workspace_bytes(32, 5, 14, 2, 64, 16, 4096, 0, 0, 1) > 0
    assert lib.kve_attn_plan_bytes(32, 5, 14, 2, 64, 16, 4096, 16, 2, 1) >= 32 * 16 * 256
    rc = lib.kve_attn_plan(None, None, None, None, 1, 5, 14, 2, 64, 16, 8, 1, 8, 128, 0, 0, 1,
                           None, 0, None)
    assert rc == -1
    rc = lib.kve_paged_verify_attn(16, 16, 16, 16, None, 16, None, 1, 5, 14, 2, 64, 16, 8, 1, 8,
                                   128, 0, 3, 0.125, 1, None, 16, None, 0, 0, None)
    assert rc == -1 and b"key_waves" in lib.kve_last_error()
    rc = lib.kve_accept(None, None, None, 0, None, 4, 0, None, None, None, None)
    assert rc == -1


def test_blocked_layout_is_the_documented_one():
    """kernels.to_blocked puts element (r, c) of an [R, C] matrix at
    ((r // 16) * (C // 32) + c // 32) * 512 + (r % 16) * 32 + c % 32, pads the
    rows to 16, and from_blocked inverts it."""
    import torch
    from kvengine_amd import kernels

    for R, C in ((1, 32), (16, 64), (37, 96), (160, 128)):
        m = torch.arange(R * C, dtype=torch.float32).reshape(R, C)
        b = kernels.to_blocked(m)
        assert b.shape == (-(-R // 16) * 16, C)
        flat = b.flatten()
        r = torch.arange(R)[:, None]
        c = torch.arange(C)[None, :]
        idx = ((r // 16) * (C // 32) + c // 32) * 512 + (r % 16) * 32 + c % 32
        assert torch.equal(flat[idx], m)
        assert torch.equal(kernels.from_blocked(b, R), m)
        assert flat.abs().sum() == m.abs().sum()  # the padding rows are zeros
