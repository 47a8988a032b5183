"""The per-position mirrors of the reference's window module on the GPU: one position's router
decision (``select``, ``select_tape``, ``select_fold``) and end of round (``cell_update``,
``update_tape``) against the CPU oracle on the same seeded inputs. GPU only.

Bars: decisions, units, valid, refreshed, theta, ages and positions bit-exact; fp32 state within
1e-5 (|got - want| <= 1e-5 * max(|want|, 1)).
"""

from __future__ import annotations

import pytest
import torch

from oracle import hsn_oracle as O

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5


@pytest.fixture(scope="module")
def win(cuda_device):
    from hsn_amd.kernels import window

    assert window.available(), "the HIP library must be built for the GPU tests"
    window.prepare(0)
    return window


def _close(got, want, what, tol=F32_TOL):
    got, want = got.detach().float().cpu(), want.detach().float().cpu()
    err = (got - want).abs()
    bound = tol * want.abs().clamp(min=1.0)
    assert bool((err <= bound).all()), f"{what}: max err {float(err.max()):.3g}"


def _same(got, want, what):
    """Bit-exact, with NaN equal to NaN (a row whose scores hold a NaN has a NaN threshold)."""
    got = got.cpu().to(want.dtype)
    if want.is_floating_point():
        torch.testing.assert_close(got, want, atol=0, rtol=0, equal_nan=True, msg=what)
    else:
        assert torch.equal(got, want), what


SELECT_CASES = [
    dict(B=3, N=40, M=1, k=5),
    dict(B=2, N=300, M=3, k=16, lambda_cost=0.05, cell_overhead=0.01, limit=0.5),
    dict(B=4, N=64, M=2, k=8, probes=True, age_max=2, reserved=2),
    dict(B=2, N=1000, M=1, k=32, bf16=True),
    dict(B=3, N=17, M=1, k=17, ties=True),
]


def _select_inputs(c, seed):
    g = torch.Generator().manual_seed(seed)
    B, N, M = c["B"], c["N"], c["M"]
    logits = torch.randn(B, N, M, generator=g)
    if c.get("ties"):  # half-integer ties, a NaN, +-inf, -0
        logits = (logits * 2).round() / 2
        logits[0, 3, 0] = float("nan")
        logits[1, 5, 0] = float("inf")
        logits[2, 7, 0] = float("-inf")
        logits[0, 9, 0] = -0.0
    if c.get("bf16"):
        logits = logits.to(torch.bfloat16)
    age = torch.randint(0, 5, (B, N), generator=g, dtype=torch.int64)
    cost = torch.rand(M, generator=g) * 0.1 + 0.01 if M > 1 else torch.full((1,), 1.0 / N)
    kw = dict(k=c["k"], age_max=c.get("age_max", 0), probes=c.get("probes", False),
              lambda_cost=c.get("lambda_cost", 0.0), cell_overhead=c.get("cell_overhead", 0.0),
              shared_cost=0.0, limit=c.get("limit", 1.0 + O.BUDGET_SLACK),
              reserved=c.get("reserved", 0), reserved_units=False)
    return logits, age, cost, kw


@pytest.mark.parametrize("case", range(len(SELECT_CASES)))
def test_select_matches_router_oracle(win, cuda_device, case):
    c = SELECT_CASES[case]
    logits, age, cost, kw = _select_inputs(c, 500 + case)
    want = O.router_select(logits.float(), age, cost, **kw)
    got = win.select(logits.to(cuda_device), age.to(cuda_device), cost.to(cuda_device), **kw)
    for name, g_, w_ in zip(("cells", "units", "valid", "theta", "refreshed"), got, want):
        _same(g_, w_, name)


@pytest.mark.parametrize("case", [0, 2, 4])
def test_select_tape_and_fold_write_their_record(win, cuda_device, case):
    """The tape form writes record t of the decision tape from record t of the ages; the folded
    form reads the same logits in place from a wider product."""
    c = SELECT_CASES[case]
    logits, age, cost, kw = _select_inputs(c, 600 + case)
    B, N, M = logits.shape
    k, n, t = kw["k"], 4, 2
    want = O.router_select(logits.float(), age, cost, **kw)
    del kw["k"]  # the tape forms take k from the tape's shape
    dev = cuda_device
    tape_age = torch.zeros(B, n + 1, N, dtype=torch.int64)
    tape_age[:, t] = age
    tape_age = tape_age.to(dev)
    tapes = dict(cells=torch.full((B, n, k), -7, dtype=torch.int64, device=dev),
                 units=torch.full((B, n, k), -7, dtype=torch.int64, device=dev),
                 valid=torch.zeros((B, n, k), dtype=torch.bool, device=dev),
                 theta=torch.full((B, n), -7.0, device=dev),
                 refreshed=torch.zeros((B, n, k), dtype=torch.bool, device=dev))
    win.select_tape(logits.to(dev), tape_age, cost.to(dev), tapes["cells"], tapes["units"],
                    tapes["valid"], tapes["theta"], tapes["refreshed"], t=t, **kw)
    for name, w_ in zip(("cells", "units", "valid", "theta", "refreshed"), want):
        _same(tapes[name][:, t], w_, name)
    assert bool((tapes["cells"][:, t - 1].cpu() == -7).all())  # other records untouched

    W = M + 3  # the scorer's product: the unit logits first, then other columns
    scored = torch.randn(B * N, W)
    scored[:, :M] = logits.float().reshape(B * N, M)
    fold = {name: torch.zeros_like(v) for name, v in tapes.items()}
    win.select_fold(scored.to(dev), tape_age, cost.to(dev), fold["cells"], fold["units"],
                    fold["valid"], fold["theta"], fold["refreshed"], t=t, n_units=M, **kw)
    for name, w_ in zip(("cells", "units", "valid", "theta", "refreshed"), want):
        _same(fold[name][:, t], w_, name)


UPDATE_CASES = [
    dict(B=3, N=32, d=16, K=4),
    dict(B=2, N=256, d=64, K=8, rms=True),
    dict(B=4, N=37, d=5, K=3, padded=True),
    dict(B=2, N=100, d=24, K=20),
]


def _update_inputs(c, seed):
    g = torch.Generator().manual_seed(seed)
    B, N, d, K = c["B"], c["N"], c["d"], c["K"]
    h = torch.randn(B, N, d, generator=g) * 0.3
    q = h.mean(dim=1)
    age = torch.randint(0, 9, (B, N), generator=g, dtype=torch.int64)
    pos = torch.randint(0, 100, (B,), generator=g, dtype=torch.int64)
    cells = torch.stack([torch.randperm(N, generator=g)[:K] for _ in range(B)])
    valid = torch.ones(B, K, dtype=torch.bool)
    if c.get("padded"):
        valid[:, -1] = False
        valid[0, 0] = False
    cells = cells.masked_fill(~valid, 0)
    y = torch.randn(B, K, d, generator=g)
    gate = torch.randn(B, K, d, generator=g) * 0.5 + 2.0
    w = torch.rand(d, generator=g) + 0.5 if c.get("rms") else torch.ones(d)
    return h, q, age, pos, cells, valid, y, gate, w


@pytest.mark.parametrize("case", range(len(UPDATE_CASES)))
def test_cell_update_matches_oracle(win, cuda_device, case):
    c = UPDATE_CASES[case]
    h, q, age, pos, cells, valid, y, gate, w = _update_inputs(c, 700 + case)
    rms = bool(c.get("rms"))
    want = O.cell_update(y, gate, h, q, age, pos, cells, valid, cand_norm=rms,
                         cand_w=w if rms else None, cand_eps=1e-6)
    D = [t.to(cuda_device) for t in (y, gate, h, q, age, pos, cells, valid, w)]
    got = win.cell_update_op(*D, rms, 1e-6)
    _close(got[0], want[0], "h")
    # cells no valid slot names are copied bit for bit (test_p2_10_window.py:272,442)
    untouched = ~O.selection_mask(cells, valid, h.shape[1])
    assert torch.equal(got[0].cpu()[untouched], h[untouched]), "unselected cells"
    _close(got[1], want[1], "q")
    assert torch.equal(got[2].cpu(), want[2]), "age"
    assert torch.equal(got[3].cpu(), want[3]), "pos"
    _close(got[4], want[4], "h_sel")
    _close(got[5], want[5], "h_max")


def test_update_tape_writes_the_next_record(win, cuda_device):
    """Record t+1 of the state tape is the round's result, zeroed where the next position
    resets; qs and h_max are the values after the position, before that reset."""
    c = UPDATE_CASES[1]
    h, q, age, pos, cells, valid, y, gate, w = _update_inputs(c, 800)
    B, N, d = h.shape
    K = cells.shape[1]
    n, t = 3, 1
    want = O.cell_update(y, gate, h, q, age, pos, cells, valid, cand_norm=True, cand_w=w,
                         cand_eps=1e-6)
    dev = cuda_device
    tape_h = torch.zeros(B, n + 1, N, d)
    tape_q = torch.zeros(B, n + 1, d)
    tape_age = torch.zeros(B, n + 1, N, dtype=torch.int64)
    tape_h[:, t], tape_q[:, t], tape_age[:, t] = h, q, age
    dec_cells = torch.zeros(B, n, K, dtype=torch.int64)
    dec_valid = torch.zeros(B, n, K, dtype=torch.bool)
    dec_cells[:, t], dec_valid[:, t] = cells, valid
    reset = torch.zeros(B, n, dtype=torch.bool)
    reset[1, t + 1] = True
    tape_hsel = torch.zeros(B, n, K, d)
    h_max = torch.zeros(B, n)
    qs = torch.zeros(B, n, d)
    T = [x.to(dev) for x in (tape_h, tape_q, tape_age, dec_cells, dec_valid, reset, tape_hsel,
                             h_max, qs)]
    win.update_tape_op(y.to(dev), gate.to(dev), T[0], T[1], T[2], T[3], T[4], w.to(dev), T[5],
                       T[6], T[7], T[8], t, True, 1e-6)
    keep = torch.tensor([True] + [False] + [True] * (B - 2))
    _close(T[0][keep, t + 1], want[0][keep], "h record t+1")
    untouched = ~O.selection_mask(cells, valid, N) & keep[:, None]
    assert torch.equal(T[0][:, t + 1].cpu()[untouched], h[untouched]), "unselected cells"
    assert bool((T[0][1, t + 1] == 0).all()), "the reset row restarts at zero"
    _close(T[1][keep, t + 1], want[1][keep], "q record t+1")
    assert torch.equal(T[2][keep, t + 1].cpu(), want[2][keep]), "age record t+1"
    assert bool((T[2][1, t + 1] == 0).all())
    _close(T[6][:, t], want[4], "h_sel")
    _close(T[7][:, t], want[5], "h_max")
    _close(T[8][:, t], want[1], "qs (before the reset)")
    _close(T[0][:, t], h, "record t unchanged")


@pytest.mark.parametrize("N,d", [(256, 64), (300, 16)])
def test_cell_update_h_max_propagates_a_nan(win, cuda_device, N, d):
    """One position's row maximum is NaN when a cell no slot writes holds a NaN, and the NaN
    stays in its cell (test_p2_10_window.py:540-560)."""
    c = dict(B=2, N=N, d=d, K=4)
    h, q, age, pos, cells, valid, y, gate, w = _update_inputs(c, 900 + N)
    quiet = int(torch.ones(N).index_fill(0, cells[0], 0).nonzero()[0])
    h[0, quiet, d // 2] = float("nan")
    want = O.cell_update(y, gate, h, q, age, pos, cells, valid)
    D = [t.to(cuda_device) for t in (y, gate, h, q, age, pos, cells, valid, w)]
    got = win.cell_update_op(*D, False, 1e-6)
    assert bool(torch.isnan(got[5][0].cpu())) and bool(torch.isnan(want[5][0]))
    _close(got[5][1], want[5][1], "finite row")
    assert torch.equal(torch.isnan(got[0].cpu()), torch.isnan(want[0]))
