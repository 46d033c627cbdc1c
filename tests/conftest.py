import json
import os
import sys

import numpy as np
import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

GOLDEN = os.path.join(REPO, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")
    config.addinivalue_line("markers", "slow: CPU test that takes more than a few seconds")


def load_json(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def load_npz_tensors(name):
    """Fixture arrays; bf16 tensors are stored as int16 bit patterns."""
    z = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
    dtype = torch.bfloat16 if "bfloat16" in str(z["dtype"]) else torch.float32
    out = {"dtype": dtype}
    for key in ("q", "out", "k_pool", "v_pool"):
        a = torch.from_numpy(z[key].copy())
        out[key] = a.view(torch.bfloat16) if dtype == torch.bfloat16 else a
    out["ctx_lens"] = z["ctx_lens"].tolist()
    out["tables"] = [[int(b) for b in row if b >= 0] for row in z["tables"]]
    out["block_size"] = int(z["block_size"])
    out["q_len"] = int(z["q_len"])
    out["use_sdpa"] = bool(z["use_sdpa"])
    return out


@pytest.fixture(scope="session")
def gpu_lib():
    """The HIP library, loaded; skips when no GPU is visible."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from kvengine_amd import _lib
    return _lib.lib()
