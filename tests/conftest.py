"""Test configuration: the ``gpu`` marker, the repository root on ``sys.path`` and the golden
fixture loader.

``-m "not gpu"`` runs the oracle against the reference's golden vectors, closed forms and known
answers, the host logic, and the C-ABI library's symbol table (no compute without a GPU).
``-m gpu`` runs the HIP library through its C-ABI against the oracle.
"""

from __future__ import annotations

import hashlib
import json
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def load_golden(name: str) -> dict:
    """A golden fixture, verified against its SHA-256 in ``tests/golden/MANIFEST.json``."""
    from safetensors.numpy import load_file
    import torch

    manifest = json.loads((GOLDEN / "MANIFEST.json").read_text())
    path = GOLDEN / name
    digest = hashlib.sha256(path.read_bytes()).hexdigest()
    assert digest == manifest["files"][name]["sha256"], f"{name}: SHA-256 mismatch"
    return {k: torch.from_numpy(v.copy()) for k, v in load_file(str(path)).items()}


@pytest.fixture(scope="session")
def cuda_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda", 0)


@pytest.fixture(autouse=True, scope="session")
def _single_thread_torch():
    """Pin torch to a fixed thread count (the reference's test session does the same), so the
    oracle's reductions take one order."""
    import torch

    torch.set_num_threads(int(os.environ.get("HSN_TEST_THREADS", "4")))
    yield


def nan_state_window(N=16, d=8, K=2, T=6, seed=31):
    """A window whose start state holds a NaN in a cell no slot ever writes (its logits are
    -inf), with a reset at position 3 of row 1: row 0's maxima are NaN throughout, row 1's until
    the reset and finite from there."""
    import torch

    from hsn_amd.workload import CONFIGS, make_window

    cfg = CONFIGS["tiny"].scaled(B=2, T=T, N=N, d=d, K=K, h0_sigma=0.3, reset_at=((1, 3),))
    w = make_window(cfg, seed)
    quiet = N - 2
    w["logits"][:, :, quiet] = float("-inf")
    w["h0"][:, quiet, d // 2] = float("nan")
    w["q0"] = torch.where(torch.isnan(w["h0"]), torch.zeros_like(w["h0"]), w["h0"]).mean(dim=1)
    return cfg, w, quiet
