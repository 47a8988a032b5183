"""The state-gradient reverse sweep on the card (``hsn_amd.state_sweep``: the HIP glue steps of
``include/hsn_sweep.h`` between hipBLASLt products) against the CPU oracle
(``oracle/state_gradient.py``, float64, itself pinned by autograd). GPU only.

Bars: fp32 products ``|got - want| <= 1e-5 * max(|want|, 1)`` for ``dL/dc`` and ``dL/db`` over the
whole window; bf16 products (autocast's) ``2e-2 * max(|want|, 1)``; a captured graph's replays
equal the eager sweep bit for bit.
"""

from __future__ import annotations

import pytest
import torch

from conftest import sweep_oracle, sweep_problem

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
BF16_TOL = 2e-2


@pytest.fixture(scope="module")
def dev(cuda_device):
    from hsn_amd import _lib

    _lib.library()
    return cuda_device


def _args(p, dev, product_dtype=torch.float32):
    def f(x):
        return None if x is None else x.to(dev, torch.float32)

    record = {k: (v.to(dev, product_dtype) if k == "hidden" else f(v))
              for k, v in p["record"].items()}
    cot = p["cot"]
    return ((f(p["c"]), f(p["b"]), f(p["h_old"]), p["cells"].to(dev), p["units"].to(dev),
             p["valid"].to(dev), p["reset"].to(dev), p["N"], f(cot["d_q_pre"]),
             f(cot["d_q_post"]), f(cot["d_h_sel"]), f(cot["d_h_fast"]), record, p["consts"]),
            dict(n_read=p["n_read"]))


def _close(got, want, tol, what):
    got = got.detach().double().cpu()
    err = (got - want).abs()
    bound = tol * want.abs().clamp(min=1.0)
    bad = ~(err <= bound)
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} of {got.numel()} elements off; worst error "
        f"{float((err / want.abs().clamp(min=1.0)).max()):.3e} (bar {tol})")


CASES = {
    "norms_gelu": dict(B=3, T=12, K=5, N=40, d=16, H=24, M=3, D=4),
    "no_cand_norm_relu": dict(B=2, T=10, K=4, N=30, d=8, H=20, M=2, cand_norm=False, act="relu"),
    "no_cell_norm_silu": dict(B=2, T=10, K=4, N=30, d=32, H=40, M=4, cell_norm=False, act="silu"),
    "no_norms_tanh": dict(B=2, T=9, K=3, N=20, d=8, H=16, M=2, cand_norm=False, cell_norm=False,
                          act="tanh"),
    "fast_read_resets": dict(B=3, T=12, K=4, N=24, d=16, H=24, M=3, n_read=3,
                             resets=((0, 0), (0, 11), (1, 5), (1, 6), (2, 3))),
    "odd_widths": dict(B=2, T=7, K=6, N=33, d=72, H=70, M=5, D=5, seed=3),
    "wide_d": dict(B=2, T=6, K=3, N=18, d=256, H=64, M=2, seed=5),
    "model_shape": dict(B=4, T=16, K=8, N=256, d=64, H=128, M=8, D=8, seed=7, pad_every=9),
}


def _run(args, kw, fused, graph=False):
    """The runner on one window with the fused step forced on or off; skips where the fused step
    does not take the shape."""
    from hsn_amd.state_sweep import SweepRunner

    try:
        return SweepRunner(graph=graph, fused=fused)(*args, **kw)
    except ValueError as e:
        if fused and "fused step" in str(e):
            pytest.skip(str(e))
        raise


@pytest.fixture(params=[True, False], ids=["fused", "three_steps"])
def fused(request):
    """Every sweep test runs the fused step (hsn_win_back_cell) and the three glue steps around
    the all-units GEMMs."""
    return request.param


@pytest.mark.parametrize("name", sorted(CASES))
def test_sweep_matches_oracle(dev, name, fused):
    print(f"case {name} fused={fused}", flush=True)
    p = sweep_problem(**CASES[name])
    want_dc, want_db = sweep_oracle(p)
    args, kw = _args(p, dev)
    out = _run(args, kw, fused)
    assert out is not None, "the runner declined a shape it takes"
    _close(out[0], want_dc, F32_TOL, f"{name} dL/dc")
    _close(out[1], want_db, F32_TOL, f"{name} dL/db")


@pytest.mark.parametrize("name", ["norms_gelu", "model_shape", "fast_read_resets", "wide_d"])
def test_sweep_with_bf16_products(dev, name, fused):
    """Autocast's sweep: the hidden record, the operands and the products in bf16 (fp32
    accumulation), the state's cotangent in fp32."""
    print(f"case {name} bf16 fused={fused}", flush=True)
    p = sweep_problem(**CASES[name])
    want_dc, want_db = sweep_oracle(p)
    args, kw = _args(p, dev, torch.bfloat16)
    out = _run(args, kw, fused)
    assert out is not None
    _close(out[0], want_dc, BF16_TOL, f"{name} bf16 dL/dc")
    _close(out[1], want_db, BF16_TOL, f"{name} bf16 dL/db")


def test_fixed_unit_slots_take_the_same_sweep(dev, fused):
    """Leading slots with a fixed unit (``n_fast``) are swept like the others: the same values as
    without the distinction."""
    p = sweep_problem(B=2, T=8, K=4, N=20, d=16, H=24, M=4, seed=11)
    args, kw = _args(p, dev)
    plain = _run(args, kw, fused)
    fixed = _run(args, dict(kw, n_fast=2), fused)
    assert plain is not None and fixed is not None
    assert torch.equal(plain[0], fixed[0]) and torch.equal(plain[1], fixed[1])


def test_graph_replays_equal_the_eager_sweep(dev, fused):
    """One runner captures the shape's graph at its first window and replays it for the next
    ones (new values loaded between replays, eager work in between): every window equals an
    eager sweep of the same window bit for bit, and the oracle."""
    from hsn_amd.state_sweep import SweepRunner

    graphed = SweepRunner(graph=True, fused=fused)
    eager = SweepRunner(graph=False, fused=fused)
    cell = None
    for seed in (21, 22, 23):
        p = sweep_problem(B=3, T=10, K=4, N=30, d=16, H=32, M=3, seed=seed, n_read=2)
        cell = p["consts"] if cell is None else cell
        p["consts"] = cell  # one model: its weights and message graph stay between windows
        args, kw = _args(p, dev)
        got = graphed(*args, **kw)
        torch.cuda.synchronize()
        want = eager(*args, **kw)
        assert got is not None and want is not None
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1]), f"window {seed}"
        want_dc, want_db = sweep_oracle(p)
        _close(got[0], want_dc, F32_TOL, f"graph window {seed} dL/dc")
        _close(got[1], want_db, F32_TOL, f"graph window {seed} dL/db")
    assert graphed.captures == 1 and graphed.calls == 3


def test_runner_declines_what_it_does_not_take(dev):
    from hsn_amd.state_sweep import SweepRunner

    runner = SweepRunner(graph=False)
    p = sweep_problem(B=2, T=4, K=3, N=10, d=8, H=8, M=2)
    args, kw = _args(p, dev)
    cpu_args, _ = _args(p, torch.device("cpu"))
    assert runner(*cpu_args, **kw) is None  # another device
    as64 = (args[0].double(),) + args[1:]
    assert runner(*as64, **kw) is None  # a float64 state
    assert runner(*args, limits=(1.0, None, None), **kw) is None  # the row limit
    record = dict(args[12], hidden=args[12]["hidden"].half())
    assert runner(*args[:12], record, args[13], **kw) is None  # fp16 products
    wide = sweep_problem(B=1, T=2, K=2, N=6, d=260, H=8, M=2)
    wargs, wkw = _args(wide, dev)
    assert runner(*wargs, **wkw) is None  # d above 256
    assert runner.calls == 0
