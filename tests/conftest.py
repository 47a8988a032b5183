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


def sweep_problem(B=2, T=5, K=3, N=7, d=4, H=6, M=3, D=3, n_read=0, n_extra=None,
                  cand_norm=True, cell_norm=True, act="gelu", seed=0, pad_every=4,
                  resets=((1, 2),), alpha_one=False):
    """A random window for the state-gradient sweep in float64: the cell's weights
    (``oracle.state_gradient.CellWeights``), a message graph with padded source slots, distinct
    cells per position (every ``pad_every``-th slot padded), resets, the start state and input
    columns, the forward's outputs and record (``window_outputs``), and random cotangents of the
    outputs (zero on padded slots' ``h_sel``)."""
    import torch

    from oracle import state_gradient as S

    g = torch.Generator().manual_seed(seed)
    f64 = torch.float64

    def rnd(*shape, scale=1.0):
        return torch.randn(*shape, generator=g, dtype=f64) * scale

    n_extra = 2 * d if n_extra is None else n_extra
    n = n_extra + 2 * d
    pad_src = torch.randint(0, N, (N, D), generator=g)
    pad_mask = torch.rand(N, D, generator=g) < 0.75
    pad_mask[:, 0] = True
    edge_weights = torch.where(pad_mask, rnd(N, D, scale=0.5), torch.zeros((), dtype=f64))
    w = S.CellWeights(
        w1=rnd(M, n, H, scale=n ** -0.5), b1=rnd(M, H, scale=0.1),
        w2=rnd(M, H, d, scale=H ** -0.5), b2=rnd(M, d, scale=0.1),
        gate_w=rnd(d, n, scale=n ** -0.5), gate_b=rnd(d, scale=0.1),
        norm_gain=(1.0 + rnd(n, scale=0.2)) if cell_norm else None, norm_eps=1e-6,
        cand_gain=(1.0 + rnd(d, scale=0.2)) if cand_norm else None, cand_eps=1e-6,
        w_out=rnd(d, d, scale=d ** -0.5), v=rnd(d, d, scale=d ** -0.5),
        pad_src=pad_src, pad_mask=pad_mask, edge_weights=edge_weights, activation=act)
    cells = torch.stack([torch.stack([torch.randperm(N, generator=g)[:K] for _ in range(T)])
                         for _ in range(B)])
    valid = torch.ones(B, T, K, dtype=torch.bool)
    flat = valid.view(-1)
    flat[pad_every - 1::pad_every] = False
    cells = torch.where(valid, cells, torch.zeros_like(cells))
    units = torch.randint(0, M, (B, T, K), generator=g)
    units = torch.where(valid, units, torch.zeros_like(units))
    alpha = torch.ones(B, T, K, dtype=f64) if alpha_one else 0.5 + torch.rand(B, T, K, generator=g,
                                                                               dtype=f64)
    reset = torch.zeros(B, T, dtype=torch.bool)
    for row, t in resets:
        if row < B and t < T:
            reset[row, t] = True
    h0 = rnd(B, N, d, scale=0.5)
    extra = rnd(B, T, K, n_extra)
    with torch.no_grad():
        outs, rec = S.window_outputs(h0, extra, cells, units, valid, alpha, reset, w, n_read)
    cot = {
        "d_q_pre": rnd(B, T, d), "d_q_post": rnd(B, T, d),
        "d_h_sel": torch.where(valid[..., None], rnd(B, T, K, d), torch.zeros((), dtype=f64)),
        "d_h_fast": rnd(B, T, n_read, d) if n_read else None,
    }
    record = {"y": rec["y"], "alpha": alpha, "hidden": rec["hidden"],
              "gate_pre": rec["gate_pre"], "m": rec["m"]}
    if cell_norm:
        record["rms"] = rec["rms"]
    return {"w": w, "consts": S.cell_constants(w), "cells": cells, "units": units, "valid": valid,
            "alpha": alpha, "reset": reset, "h0": h0, "extra": extra, "outs": outs,
            "c": rec["c"], "b": rec["b"], "h_old": rec["h_old"], "record": record, "cot": cot,
            "N": N, "n_read": n_read}


def sweep_oracle(p, consts=None, trace=None):
    """``oracle.state_gradient.state_gradient_backward`` on a ``sweep_problem``."""
    from oracle import state_gradient as S

    cot = p["cot"]
    return S.state_gradient_backward(
        p["c"], p["b"], p["h_old"], p["cells"], p["units"], p["valid"], p["reset"], p["N"],
        cot["d_q_pre"], cot["d_q_post"], cot["d_h_sel"], cot["d_h_fast"], p["record"],
        p["consts"] if consts is None else consts, trace=trace)


def round_problem(B=4, N=32, d=64, K=4, M=8, H=512, D=4, cand_norm=True, seed=11, pad=0.0,
                  alpha_one=True, edge_density=0.75):
    """One position of the fused cell round (``hsn::window_cell_round``) in float64, shaped as the
    reference's fused-round tests build it (tests/kernels/test_p2_10_window.py:185-222): weights
    moved away from their initial values, states uniform in [-0.8, 0.8], ``q`` near their mean,
    small ages and positions, distinct cells a row, a fraction ``pad`` of the slots padded (cell
    0, unit 0, as the router pads), a padded message graph (weight 0, source 0 on padding).
    Keys are ``oracle.hsn_oracle.window_cell_round``'s arguments."""
    import torch

    g = torch.Generator().manual_seed(seed)
    f64 = torch.float64

    def rnd(*shape, scale=1.0):
        return torch.randn(*shape, generator=g, dtype=f64) * scale

    n = 4 * d
    cells = torch.stack([torch.randperm(N, generator=g)[:K] for _ in range(B)])
    units = torch.randint(0, M, (B, K), generator=g)
    valid = torch.rand(B, K, generator=g) >= pad
    cells = torch.where(valid, cells, torch.zeros_like(cells))
    units = torch.where(valid, units, torch.zeros_like(units))
    mask = torch.rand(N, D, generator=g) < edge_density
    if D:
        mask[:, 0] = True
    pad_src = torch.where(mask, torch.randint(0, N, (N, D), generator=g), torch.zeros((), dtype=torch.int64))
    edge_w = torch.where(mask, torch.softmax(rnd(N, D), dim=1), torch.zeros((), dtype=f64))
    h = torch.rand(B, N, d, generator=g, dtype=f64) * 1.6 - 0.8
    return dict(
        u=rnd(B, d), eps=rnd(B, d), h=h, q=h.mean(dim=1) + 0.01,
        age=torch.randint(0, 9, (B, N), generator=g), pos=torch.randint(0, 50, (B,), generator=g),
        cells=cells, units=units, valid=valid,
        alpha=(valid.to(f64) if alpha_one else 0.5 + torch.rand(B, K, generator=g, dtype=f64)),
        V=rnd(d, d, scale=d ** -0.5) + 0.2 * rnd(d, d), edge_w=edge_w, pad_src=pad_src,
        norm_w=1.0 + 0.2 * rnd(n), norm_eps=1e-6,
        gate_w=rnd(d, n, scale=n ** -0.5) + 0.2 * rnd(d, n, scale=0.1), gate_b=0.2 * rnd(d),
        W1=rnd(M, n, H, scale=n ** -0.5), b1=0.2 * rnd(M, H),
        W2=rnd(M, H, d, scale=H ** -0.5), b2=0.2 * rnd(M, d),
        W_out=rnd(d, d, scale=d ** -0.5) + 0.2 * rnd(d, d, scale=0.2),
        cand_w=1.0 + 0.2 * rnd(d), cand_norm=cand_norm, cand_eps=1e-6)
