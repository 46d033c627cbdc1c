"""kve_lmhead_argmax_noalloc (no workspace, no allocation) against
kve_lmhead_argmax (caller workspace), both called through the C ABI.

The no-allocation entry point takes its key copies from a device array the
library owns; every call on a GPU shares it and each call must leave it clean
for the next. So it is compared bit for bit with the workspace entry point on
calls in a row whose row counts shrink and grow, with and without the
runner-up, and its size limit is checked before any launch.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF16, F32 = 1, 0


def outputs(M):
    return (torch.full((M,), -7, dtype=torch.int32, device=DEV),
            torch.full((M,), float("nan"), dtype=torch.float32, device=DEV),
            torch.full((M,), -7, dtype=torch.int32, device=DEV),
            torch.full((M,), float("nan"), dtype=torch.float32, device=DEV))


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def call(lib, hidden, weight, dtype, top2, noalloc):
    M, H = hidden.shape
    V = weight.shape[0]
    am, mx, sid, sv = outputs(M)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [ptr(hidden), hidden.stride(0), ptr(weight), M, H, V, dtype, ptr(am), ptr(mx),
            ptr(sid) if top2 else None, ptr(sv) if top2 else None]
    if noalloc:
        rc = lib.kve_lmhead_argmax_noalloc(*args, stream)
    else:
        nbytes = lib.kve_lmhead_workspace_bytes(M)
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
        rc = lib.kve_lmhead_argmax(*args, ptr(ws), nbytes, 0, stream)
    assert rc == 0, lib.kve_last_error()
    torch.cuda.synchronize()
    return [t.cpu() for t in (am, mx, sid, sv)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_equals_workspace_entry_point_on_calls_in_a_row(gpu_lib, dtype):
    code = BF16 if dtype == torch.bfloat16 else F32
    g = torch.Generator().manual_seed(17)
    V, H = 151936, 896
    weight = (torch.randn(V, H, generator=g) * 0.02).to(dtype).to(DEV)
    # rows shrink, grow to the limit, shrink again: each call starts from what
    # the previous one left in the shared array
    for M, top2 in ((160, True), (37, True), (256, False), (5, True), (1, False), (96, True)):
        hidden = torch.randn(M, H, generator=g).to(dtype).to(DEV)
        want = call(gpu_lib, hidden, weight, code, top2, noalloc=False)
        got = call(gpu_lib, hidden, weight, code, top2, noalloc=True)
        assert torch.equal(got[0], want[0]), (M, "argmax")
        assert torch.equal(got[1], want[1]), (M, "maxval")
        if top2:
            assert torch.equal(got[2], want[2]), (M, "second id")
            assert torch.equal(got[3], want[3]), (M, "second value")
        else:
            assert bool((got[2] == -7).all()), "runner-up written although not asked for"


def test_noalloc_strided_rows(gpu_lib):
    """Rows read with a stride (the verify pass's hidden rows of a wider buffer)."""
    g = torch.Generator().manual_seed(3)
    V, H = 5000, 256
    weight = (torch.randn(V, H, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wide = torch.randn(40, 2 * H, generator=g).to(torch.bfloat16).to(DEV)
    hidden = wide[:, :H]
    want = call(gpu_lib, hidden, weight, BF16, True, noalloc=False)
    got = call(gpu_lib, hidden, weight, BF16, True, noalloc=True)
    for a, b in zip(got, want):
        assert torch.equal(a, b)


def test_noalloc_rejects_more_rows_than_its_array_holds(gpu_lib):
    H, V = 128, 1000
    hidden = torch.zeros(257, H, dtype=torch.bfloat16, device=DEV)
    weight = torch.zeros(V, H, dtype=torch.bfloat16, device=DEV)
    am = torch.zeros(257, dtype=torch.int32, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = gpu_lib.kve_lmhead_argmax_noalloc(ptr(hidden), H, ptr(weight), 257, H, V, BF16, ptr(am),
                                           None, None, None, stream)
    assert rc == -1
    assert b"256" in gpu_lib.kve_last_error()
    torch.cuda.synchronize()
    assert bool((am.cpu() == 0).all()), "a rejected call must launch nothing"
    # and the next call is unaffected
    hidden = torch.randn(3, H).to(torch.bfloat16).to(DEV)
    w = torch.randn(V, H).to(torch.bfloat16).to(DEV)
    assert torch.equal(call(gpu_lib, hidden, w, BF16, True, noalloc=True)[0],
                       call(gpu_lib, hidden, w, BF16, True, noalloc=False)[0])
