"""The fused cell round on the card (``hsn_amd.kernels.window.cell_round_op``, the HIP entry point
``hsn_win_cell_round`` of ``include/hsn_round.h``) against the CPU oracle
(``oracle.hsn_oracle.window_cell_round``, float64 on the same fp32 inputs). GPU only.

The cases follow the reference's own (tests/kernels/test_p2_10_window.py:226-308): the default
cell at B 32, a budget that pads slots, no candidate norm, odd sizes, one unit and one slot, 256
positions in a row. Bars: h, q and h_sel ``|got - want| <= 1e-5 max(|want|, 1)`` (the
reference holds its fused round to 2e-5 against its native one), ages and positions exact, cells
no slot writes bit for bit.
"""

from __future__ import annotations

import pytest
import torch

from conftest import round_problem
from oracle import hsn_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-5
FLOATS = ("u", "eps", "h", "q", "alpha", "V", "edge_w", "norm_w", "gate_w", "gate_b", "W1", "b1",
          "W2", "b2", "W_out", "cand_w")
OP_ARGS = ("u", "eps", "h", "q", "age", "cells", "units", "valid", "alpha", "V", "edge_w",
           "pad_src", "norm_w", "gate_w", "gate_b", "W1", "b1", "W2", "b2", "W_out", "cand_w")


@pytest.fixture(scope="module")
def dev(cuda_device):
    from hsn_amd import _lib

    _lib.library()
    return cuda_device


def _as_f32(p):
    """The problem rounded to fp32 (kept in float64 for the oracle: the kernels and the oracle
    then start from the same values)."""
    return {k: (v.float().double() if k in FLOATS else v) for k, v in p.items()}


def _run(p, dev):
    from hsn_amd.kernels.window import cell_round_op

    args = [p[k].to(dev, torch.float32) if k in FLOATS else p[k].to(dev) for k in OP_ARGS]
    return cell_round_op(*args, bool(p["cand_norm"]), float(p["norm_eps"]), float(p["cand_eps"]))


def _close(got, want, what, tol=TOL):
    got = got.detach().double().cpu()
    err = (got - want).abs()
    bound = tol * want.abs().clamp(min=1.0)
    bad = ~(err <= bound)
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} of {got.numel()} elements off; worst "
        f"{float((err / want.abs().clamp(min=1.0)).max()):.3e} (bar {tol})")


def _check(p, out, what):
    want = O.window_cell_round(**p)
    h_new, q_new, age_new, h_sel = out
    _close(h_new, want[0], f"{what} h")
    _close(q_new, want[1], f"{what} q")
    assert torch.equal(age_new.cpu(), want[2]), f"{what} age"
    _close(h_sel, want[4], f"{what} h_sel")
    written = O.selection_mask(p["cells"], p["valid"], p["h"].shape[1])
    assert torch.equal(h_new.cpu().double()[~written], p["h"][~written]), f"{what} unwritten"


CASES = {
    "default_b32": dict(B=32),  # the reference's A6 recipe sizes
    "padded_b32": dict(B=32, pad=0.4, seed=3),  # a budget that pads slots
    "no_cand_norm": dict(B=5, cand_norm=False, seed=4),
    "odd": dict(B=7, N=11, d=24, K=5, M=3, H=77, D=3, seed=5, pad=0.2),
    "one": dict(B=1, K=1, M=1, H=33, seed=6),
    "alpha": dict(B=3, alpha_one=False, seed=7),
    "alpha_no_cand_norm": dict(B=3, alpha_one=False, cand_norm=False, seed=8),
    "no_edges": dict(B=2, D=0, seed=9),
    "sweep_model": dict(B=32, N=256, d=64, K=8, M=8, H=512, D=8, seed=10, pad=1 / 16),
    "wide_d": dict(B=4, N=40, d=128, K=6, M=4, H=200, D=5, seed=13),
    "d256_many_slots": dict(B=2, N=70, d=256, K=20, M=3, H=64, D=2, seed=14),  # >64 KiB of LDS
    "one_unit_many_slots": dict(B=64, N=64, d=32, K=16, M=1, H=96, D=4, seed=15),
    "max_slots": dict(B=128, N=96, d=16, K=64, M=4, H=64, D=2, seed=16, pad=0.1),  # B K = 8192
    "wide_row_slots": dict(B=2, N=80, d=128, K=64, M=2, H=64, D=3, seed=17),  # >64 KiB in back
    "smallest": dict(B=3, N=9, d=4, K=2, M=2, H=5, D=1, seed=18),  # one step a lane group
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_round_matches_oracle(dev, name):
    print(f"case {name}", flush=True)
    p = _as_f32(round_problem(**CASES[name]))
    _check(p, _run(p, dev), name)


def test_round_is_reproducible(dev):
    p = _as_f32(round_problem(B=16, seed=21))
    a = _run(p, dev)
    b = _run(p, dev)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_round_reads_out_of_range_cells_as_padded(dev):
    """A valid slot naming a cell outside [0, N) writes nothing (the kernels' bounds rule) and a
    unit outside [0, M) reads as the nearest unit."""
    p = _as_f32(round_problem(B=3, seed=22))
    bad = dict(p, cells=p["cells"].clone(), units=p["units"].clone())
    bad["cells"][0, 1] = p["h"].shape[1] + 5
    bad["units"][1, 0] = 99
    out = _run(bad, dev)
    want = dict(p, valid=p["valid"].clone(), cells=p["cells"].clone(), units=p["units"].clone())
    want["valid"][0, 1] = False
    want["cells"][0, 1] = 0
    want["units"][1, 0] = p["W1"].shape[0] - 1
    want["alpha"] = want["alpha"] * want["valid"]
    _check(want, out, "out of range")


def test_round_over_256_positions_stays_close(dev):
    """256 fused rounds against 256 oracle rounds from the same start, the same decisions each
    position (reference test_fused_cell_round_over_a_window_stays_close: worst |h| error 1e-4)."""
    from hsn_amd.kernels.window import cell_round_op

    base = _as_f32(round_problem(B=8, seed=5))
    g = torch.Generator().manual_seed(9)
    B, N, d = base["h"].shape
    K, M = base["cells"].shape[1], base["W1"].shape[0]
    weights = {k: base[k].to(dev, torch.float32) for k in FLOATS if k not in ("u", "eps", "h",
                                                                                "q", "alpha")}
    state = (base["h"].to(dev, torch.float32), base["q"].to(dev, torch.float32),
             base["age"].to(dev))
    ref = (base["h"], base["q"], base["age"], base["pos"])
    worst = 0.0
    for t in range(256):
        u = torch.randn(B, d, generator=g).double()
        eps = torch.randn(B, d, generator=g).double()
        cells = torch.argsort(torch.rand(B, N, generator=g), dim=-1)[:, :K]
        units = torch.randint(0, M, (B, K), generator=g)
        valid = torch.ones(B, K, dtype=torch.bool)
        alpha = valid.double()
        p = dict(base, u=u, eps=eps, cells=cells, units=units, valid=valid, alpha=alpha,
                 h=ref[0], q=ref[1], age=ref[2], pos=ref[3])
        ref = O.window_cell_round(**p)[:4]
        h, q, age, _ = cell_round_op(
            u.float().to(dev), eps.float().to(dev), state[0], state[1], state[2], cells.to(dev),
            units.to(dev), valid.to(dev), alpha.float().to(dev), weights["V"],
            weights["edge_w"], base["pad_src"].to(dev), weights["norm_w"], weights["gate_w"],
            weights["gate_b"], weights["W1"], weights["b1"], weights["W2"], weights["b2"],
            weights["W_out"], weights["cand_w"], True, 1e-6, 1e-6)
        state = (h, q, age)
        worst = max(worst, float((h.double().cpu() - ref[0]).abs().max()))
    assert worst <= 1e-4, worst
    assert float((state[1].double().cpu() - ref[1]).abs().max()) <= 1e-4
    assert torch.equal(state[2].cpu(), ref[2])


def test_cell_round_wrapper_and_its_declines(dev):
    """``cell_round`` on a cell object (the reference's PDGCell attribute names) equals the op
    on the same tensors and ticks ``pos``; ``cell_round_error`` names what the fused round does
    not implement (reference window.py:202-230)."""
    from types import SimpleNamespace

    from hsn_amd.kernels import window as W
    from hsn_amd.workload import make_round_cell, make_round_positions

    cell, edge_w = make_round_cell(N=32, d=64, M=8, H=512, D=4, seed=3, device=dev)
    pos = make_round_positions(B=4, K=4, N=32, d=64, M=8, T=1, seed=4, device=dev)
    assert W.cell_round_error(cell) is None
    st, h_sel = W.cell_round(cell, pos["u"][0], pos["eps"][0], pos["state"], pos["cells"][0],
                             pos["units"][0], pos["valid"][0], edge_w)
    p = {
        "u": pos["u"][0], "eps": pos["eps"][0], "h": pos["state"].h, "q": pos["state"].q,
        "age": pos["state"].age, "pos": pos["state"].pos, "cells": pos["cells"][0],
        "units": pos["units"][0], "valid": pos["valid"][0],
        "alpha": pos["valid"][0].double(), "V": cell.V.weight, "edge_w": edge_w,
        "pad_src": cell.graph._pad_src, "norm_w": cell.norm.weight, "norm_eps": 1e-6,
        "gate_w": cell.gate.weight, "gate_b": cell.gate.bias, "W1": cell.units.W1,
        "b1": cell.units.b1, "W2": cell.units.W2, "b2": cell.units.b2,
        "W_out": cell.W_out.weight, "cand_w": cell.cand_norm.weight, "cand_norm": True,
        "cand_eps": 1e-6}
    p = {k: (v.detach().cpu().double() if torch.is_tensor(v) and v.is_floating_point()
             else (v.cpu() if torch.is_tensor(v) else v)) for k, v in p.items()}
    want = O.window_cell_round(**p)
    _close(st.h, want[0], "wrapper h")
    _close(st.q, want[1], "wrapper q")
    assert torch.equal(st.age.cpu(), want[2]) and torch.equal(st.pos.cpu(), want[3])
    _close(h_sel, want[4], "wrapper h_sel")
    # the eager wrapper runs the op's body without the custom op's dispatch: the registered op
    # gives the same bits
    with torch.no_grad():
        op = W.cell_round_op(
            pos["u"][0], pos["eps"][0], pos["state"].h, pos["state"].q, pos["state"].age,
            pos["cells"][0], pos["units"][0], pos["valid"][0], pos["valid"][0].float(),
            cell.V.weight, edge_w.float(), cell.graph._pad_src, cell.norm.weight,
            cell.gate.weight, cell.gate.bias, cell.units.W1, cell.units.b1, cell.units.W2,
            cell.units.b2, cell.W_out.weight, cell.cand_norm.weight, True,
            float(getattr(cell.norm, "eps", None) or 0.0),
            float(getattr(cell.cand_norm, "eps", None) or 0.0))
    for got, ref, what in zip((st.h, st.q, st.age, h_sel), op, ("h", "q", "age", "h_sel")):
        assert torch.equal(got, ref), f"wrapper against the registered op: {what}"

    def variant(**kw):
        v = SimpleNamespace(**vars(cell))
        for k, x in kw.items():
            setattr(v, k, x)
        return v

    assert "ablate_shared_u" in W.cell_round_error(variant(ablate_shared_u=True))
    assert "cell_norm" in W.cell_round_error(variant(cell_norm="layer"))
    assert "GELU" in W.cell_round_error(
        variant(units=SimpleNamespace(**dict(vars(cell.units), activation_name="silu"))))
    assert "disabled_cells" in W.cell_round_error(variant(disabled_cells=(3,)))
    assert "fp32" in W.cell_round_error(variant(V=torch.nn.Linear(64, 64).double()))
    odd, _ = make_round_cell(N=8, d=6, M=2, H=8, D=2)
    assert "multiple of 4" in W.cell_round_error(odd)


def test_round_replays_in_a_graph(dev):
    """The three launches captured in a HIP graph (torch's, the scratch from its pool) and
    replayed for new inputs: every replay equals the eager round bit for bit."""
    from hsn_amd.kernels.window import cell_round_op

    p = _as_f32(round_problem(B=8, seed=30))
    static = {k: (p[k].to(dev, torch.float32) if k in FLOATS else p[k].to(dev))
              for k in OP_ARGS}
    extra = (bool(p["cand_norm"]), float(p["norm_eps"]), float(p["cand_eps"]))
    cell_round_op(*[static[k] for k in OP_ARGS], *extra)  # warm up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = cell_round_op(*[static[k] for k in OP_ARGS], *extra)
    for seed in (31, 32, 33):
        q = _as_f32(round_problem(B=8, seed=seed))
        for k in ("u", "eps", "h", "q", "age", "cells", "units", "valid", "alpha"):
            static[k].copy_(q[k].to(dev, static[k].dtype))
        graph.replay()
        torch.cuda.synchronize()
        want = cell_round_op(*[static[k] for k in OP_ARGS], *extra)
        torch.cuda.synchronize()
        for x, y in zip(out, want):
            assert torch.equal(x, y), f"replay {seed}"
