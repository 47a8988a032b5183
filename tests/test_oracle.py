"""The CPU oracle pinned against the reference's golden vectors, autograd closed forms, the
router's known answers and brute force. CPU only."""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest
import torch

from conftest import load_golden, nan_state_window
from oracle import hsn_oracle as O

F64 = torch.float64


def _close(got, want, atol=1e-5, rtol=1e-5):
    torch.testing.assert_close(got, want, atol=atol, rtol=rtol)


# --------------------------------------------------------------------------------------------
# the golden vectors of the reference's four-op ABI (gated update, gather)
# --------------------------------------------------------------------------------------------


@pytest.mark.parametrize("size", ["tiny", "ref", "odd"])
def test_gated_update_matches_golden_vectors(size):
    v = load_golden(f"{size}_gated_delta_update.safetensors")
    h_out, q_out, age_out, h_old = O.gated_delta_update_abi(
        v["h"], v["q"], v["age"], v["cell_idx"], v["valid"], v["c"], v["b"])
    _close(h_out, v["h_out"])
    _close(q_out, v["q_out"])
    assert torch.equal(age_out, v["age_out"])
    _close(h_old, v["h_old_saved"])
    gh, gq, gc, gb = O.gated_delta_update_bwd(v["cell_idx"], v["valid"], v["c"], v["b"],
                                              v["h_old_saved"], v["grad_h_out"], v["grad_q_out"])
    _close(gh, v["grad_h"])
    _close(gq, v["grad_q"])
    _close(gc, v["grad_c"])
    _close(gb, v["grad_b"])


@pytest.mark.parametrize("size", ["tiny", "ref", "odd"])
def test_gather_concat_matches_golden_vectors(size):
    v = load_golden(f"{size}_gather_concat.safetensors")
    out = O.gather_concat(v["u"], v["eps"], v["h"], v["m"], v["cell_idx"])
    _close(out, v["v"])
    N = v["h"].shape[1]
    gu, ge, gh, gm = O.gather_concat_bwd(v["grad_v"], v["cell_idx"], N)
    _close(gu, v["grad_u"])
    _close(ge, v["grad_eps"])
    _close(gh, v["grad_h"])
    _close(gm, v["grad_m"])


@pytest.mark.parametrize("size", ["tiny", "ref", "odd"])
def test_grouped_unit_mlp_matches_golden_vectors(size):
    """The reference's f64 Rust oracle's vectors for the grouped unit MLP (inputs on a
    bf16-exact grid, outputs rounded once to f32); the odd vector has a unit without pairs, whose
    gradients are zero."""
    v = load_golden(f"{size}_grouped_unit_mlp.safetensors")
    out, hidden = O.grouped_unit_mlp(v["v"], v["unit_idx"], v["W1"], v["b1"], v["W2"], v["b2"])
    _close(out, v["out"])
    _close(hidden, v["hidden_saved"])
    got = O.grouped_unit_mlp_bwd(v["v"], v["unit_idx"], v["W1"], v["W2"], v["hidden_saved"],
                                 v["grad_out"])
    for g_, name in zip(got, ("grad_v", "grad_W1", "grad_b1", "grad_W2", "grad_b2")):
        _close(g_, v[name])
    if size == "odd":
        absent = sorted(set(range(v["W1"].shape[0])) - set(v["unit_idx"].tolist()))
        assert absent and bool((v["grad_W1"][absent] == 0).all())


@pytest.mark.parametrize("size", ["tiny", "ref", "odd"])
def test_csr_messages_match_golden_vectors(size):
    """The reference's vectors for the CSR messages: repeated slots (tiny: cell 1 twice in row 1)
    and edges whose row no slot selects (their grad_a is zero)."""
    v = load_golden(f"{size}_csr_messages.safetensors")
    m = O.csr_messages(v["h"], v["indptr"], v["indices"], v["a"], v["V"], v["cell_idx"])
    _close(m, v["m"])
    gh, ga, gV = O.csr_messages_bwd(v["h"], v["indptr"], v["indices"], v["a"], v["V"],
                                    v["cell_idx"], v["grad_m"])
    _close(gh, v["grad_h"])
    _close(ga, v["grad_a"])
    _close(gV, v["grad_V"])


def test_unit_and_message_backwards_equal_autograd():
    """Both backwards against float64 autograd of their forwards, on random inputs with a unit
    no pair uses, an empty CSR row and repeated slots."""
    g = torch.Generator().manual_seed(12)
    P, M, d, H = 9, 4, 3, 5
    v = torch.randn(P, 4 * d, generator=g, dtype=F64, requires_grad=True)
    idx = torch.tensor([0, 2, 2, 0, 1, 2, 0, 1, 2])  # unit 3 unused
    W1 = torch.randn(M, 4 * d, H, generator=g, dtype=F64, requires_grad=True)
    b1 = torch.randn(M, H, generator=g, dtype=F64, requires_grad=True)
    W2 = torch.randn(M, H, d, generator=g, dtype=F64, requires_grad=True)
    b2 = torch.randn(M, d, generator=g, dtype=F64, requires_grad=True)
    out, hidden = O.grouped_unit_mlp(v, idx, W1, b1, W2, b2)
    gout = torch.randn(P, d, generator=g, dtype=F64)
    want = torch.autograd.grad((out * gout).sum(), (v, W1, b1, W2, b2))
    got = O.grouped_unit_mlp_bwd(v.detach(), idx, W1.detach(), W2.detach(), hidden.detach(), gout)
    for a, b in zip(got, want):
        torch.testing.assert_close(a, b, atol=1e-12, rtol=1e-12)
    B, N, K = 2, 5, 3
    h = torch.randn(B, N, d, generator=g, dtype=F64, requires_grad=True)
    indptr = torch.tensor([0, 2, 2, 5, 6, 7], dtype=torch.int32)  # row 1 empty
    indices = torch.tensor([1, 3, 0, 2, 4, 4, 1], dtype=torch.int32)
    a = torch.rand(7, generator=g, dtype=F64, requires_grad=True)
    V = torch.randn(d, d, generator=g, dtype=F64, requires_grad=True)
    cell_idx = torch.tensor([[1, 2, 2], [0, 4, 1]], dtype=torch.int32)
    m = O.csr_messages(h, indptr, indices, a, V, cell_idx)
    gm = torch.randn(B, K, d, generator=g, dtype=F64)
    want = torch.autograd.grad((m * gm).sum(), (h, a, V))
    got = O.csr_messages_bwd(h.detach(), indptr, indices, a.detach(), V.detach(), cell_idx, gm)
    for x, y in zip(got, want):
        torch.testing.assert_close(x, y, atol=1e-12, rtol=1e-12)
    assert bool((m[0, 0] == 0).all())  # the empty row's message


def test_golden_tiny_vector_has_padded_repeat():
    """The tiny vector holds the case the dummy row exists for: a padded slot repeating a valid
    slot's cell (``cell_idx=[[0,1],[2,2]]``, ``valid=[[1,1],[1,0]]``)."""
    v = load_golden("tiny_gated_delta_update.safetensors")
    assert v["cell_idx"].tolist() == [[0, 1], [2, 2]]
    assert v["valid"].tolist() == [[1, 1], [1, 0]]


def test_gated_update_bwd_equals_autograd():
    g = torch.Generator().manual_seed(3)
    B, N, d, K = 3, 7, 5, 4
    h = torch.randn(B, N, d, generator=g, dtype=F64, requires_grad=True)
    q = torch.randn(B, d, generator=g, dtype=F64, requires_grad=True)
    c = torch.randn(B, K, d, generator=g, dtype=F64, requires_grad=True)
    b = torch.rand(B, K, d, generator=g, dtype=F64, requires_grad=True)
    cells = torch.stack([torch.randperm(N, generator=g)[:K] for _ in range(B)])
    valid = torch.rand(B, K, generator=g) > 0.3
    cells = torch.where(valid, cells, torch.zeros_like(cells))
    age = torch.zeros(B, N, dtype=torch.int64)
    h2, q2, _, h_old = O.gated_delta_update(h, q, age, cells, c, b, valid)
    G = torch.randn(B, N, d, generator=g, dtype=F64)
    gq = torch.randn(B, d, generator=g, dtype=F64)
    want = torch.autograd.grad((h2 * G).sum() + (q2 * gq).sum(), [h, q, c, b])
    got = O.gated_delta_update_bwd(cells.to(torch.int32), valid.to(torch.int32), c.detach(),
                                   b.detach(), h_old.detach(), G, gq)
    for x, y in zip(got, want):
        _close(x, y, atol=1e-12, rtol=1e-12)


# --------------------------------------------------------------------------------------------
# the backward recurrence and the carried-state gradient against float64 autograd
# --------------------------------------------------------------------------------------------


def _recurrence_case(seed=7, B=3, T=9, N=5, K=3, d=4):
    g = torch.Generator().manual_seed(seed)
    c = torch.rand(B, T, K, d, generator=g, dtype=F64, requires_grad=True)
    b = torch.rand(B, T, K, d, generator=g, dtype=F64, requires_grad=True)
    cells = torch.stack([torch.stack([torch.randperm(N, generator=g)[:K] for _ in range(T)])
                         for _ in range(B)])
    valid = torch.rand(B, T, K, generator=g) > 0.3
    cells = torch.where(valid, cells, torch.zeros_like(cells))
    reset = torch.zeros(B, T, dtype=torch.bool)
    reset[0, 0] = reset[1, 4] = reset[2, 7] = reset[2, 8] = True
    w_pre = torch.randn(B, T, d, generator=g, dtype=F64)
    w_post = torch.randn(B, T, d, generator=g, dtype=F64)
    w_sel = torch.randn(B, T, K, d, generator=g, dtype=F64)
    w_hT = torch.randn(B, N, d, generator=g, dtype=F64)
    w_qT = torch.randn(B, d, generator=g, dtype=F64)
    h0 = torch.rand(B, N, d, generator=g, dtype=F64, requires_grad=True)
    q0 = torch.randn(B, d, generator=g, dtype=F64, requires_grad=True)
    return locals()


@pytest.mark.parametrize("carry_end", [False, True])
def test_recurrence_equals_autograd_of_the_update_chain(carry_end):
    """``split.recurrence_backward`` is the VJP of ``gated_delta_update`` and ``reset`` over the
    window (the reference's own check, ``tests/test_p2_10_split_window.py:31-84``), extended with
    the start-state outputs ``d_h0, d_q0`` and an end-state cotangent."""
    s = _recurrence_case()
    B, T, N, K, d = s["B"], s["T"], s["N"], s["K"], s["d"]
    h, q = s["h0"], s["q0"]
    age = torch.zeros(B, N, dtype=torch.int64)
    pos = torch.zeros(B, dtype=torch.int64)
    total = torch.zeros((), dtype=F64)
    h_old = []
    for t in range(T):
        h, q, age, pos = O.reset_state(h, q, age, pos, s["reset"][:, t])
        total = total + (q * s["w_pre"][:, t]).sum()
        index = s["cells"][:, t, :, None].expand(B, K, d)
        h_old.append(h.gather(1, index).detach())
        h, q, age, _ = O.gated_delta_update(h, q, age, s["cells"][:, t], s["c"][:, t],
                                            s["b"][:, t], s["valid"][:, t])
        total = total + (q * s["w_post"][:, t]).sum()
        chosen = h.gather(1, index)
        total = total + (torch.where(s["valid"][:, t, :, None], chosen, 0.0) * s["w_sel"][:, t]).sum()
    if carry_end:
        total = total + (h * s["w_hT"]).sum() + (q * s["w_qT"]).sum()
    want_c, want_b, want_h0, want_q0 = torch.autograd.grad(total, [s["c"], s["b"], s["h0"], s["q0"]])
    got_c, got_b, got_h0, got_q0 = O.recurrence_backward(
        s["c"].detach(), s["b"].detach(), torch.stack(h_old, dim=1), s["cells"], s["valid"],
        s["reset"], N, s["w_pre"], s["w_post"], torch.where(s["valid"][..., None], s["w_sel"], 0.0),
        s["w_hT"] if carry_end else None, s["w_qT"] if carry_end else None, carried=True)
    for got, want in ((got_c, want_c), (got_b, want_b), (got_h0, want_h0), (got_q0, want_q0)):
        _close(got, want, atol=1e-13, rtol=1e-12)
    assert bool((got_c[~s["valid"]] == 0).all()) and bool((got_b[~s["valid"]] == 0).all())


def test_carried_gradient_is_zero_through_a_reset_at_zero():
    s = _recurrence_case()
    reset = torch.ones(s["B"], s["T"], dtype=torch.bool)
    _, _, d_h0, d_q0 = O.recurrence_backward(
        s["c"].detach(), s["b"].detach(), s["c"].detach(), s["cells"], s["valid"], reset, s["N"],
        s["w_pre"], s["w_post"], None, s["w_hT"], s["w_qT"], carried=True)
    assert bool((d_h0 == 0).all()) and bool((d_q0 == 0).all())


def test_recurrence_keeps_a_padded_nan_out():
    """``tests/test_p2_10_split_window.py:87-100``."""
    B, T, N, K, d = 1, 2, 3, 2, 2
    c = torch.full((B, T, K, d), 0.5, dtype=F64)
    c[0, 0, 1] = float("nan")
    b = torch.full((B, T, K, d), 0.25, dtype=F64)
    cells = torch.tensor([[[1, 0], [2, 0]]])
    valid = torch.tensor([[[True, False], [True, False]]])
    reset = torch.zeros(B, T, dtype=torch.bool)
    ones = torch.ones(B, T, d, dtype=F64)
    dc, db = O.recurrence_backward(c, b, torch.zeros_like(c), cells, valid, reset, N, None, ones,
                                   None)
    assert bool(torch.isfinite(dc).all()) and bool(torch.isfinite(db).all())


def test_dense_recurrence_equals_autograd():
    g = torch.Generator().manual_seed(5)
    Bd, T, N, d = 2, 6, 4, 3
    c = torch.rand(Bd, T, N, d, generator=g, dtype=F64, requires_grad=True)
    b = torch.rand(Bd, T, N, d, generator=g, dtype=F64, requires_grad=True)
    reset = torch.zeros(Bd, T, dtype=torch.bool)
    reset[1, 3] = True
    w_pre = torch.randn(Bd, T, d, generator=g, dtype=F64)
    w_post = torch.randn(Bd, T, d, generator=g, dtype=F64)
    h = torch.rand(Bd, N, d, generator=g, dtype=F64)
    q = h.mean(dim=1)
    total = torch.zeros((), dtype=F64)
    h_old = []
    for t in range(T):
        row = reset[:, t]
        h = h.masked_fill(row[:, None, None], 0)
        q = q.masked_fill(row[:, None], 0)
        total = total + (q * w_pre[:, t]).sum()
        h_old.append(h.detach())
        h = (1 - b[:, t]) * h + b[:, t] * c[:, t]
        q = h.mean(dim=1)
        total = total + (q * w_post[:, t]).sum()
    want = torch.autograd.grad(total, [c, b])
    got = O.dense_recurrence_backward(c.detach(), b.detach(), torch.stack(h_old, dim=1), reset, N,
                                      w_pre, w_post)
    for x, y in zip(got, want):
        _close(x, y, atol=1e-13, rtol=1e-12)


# --------------------------------------------------------------------------------------------
# the router: known answers, brute force, threshold and probes
# --------------------------------------------------------------------------------------------


def test_router_known_answers():
    """``tests/test_p2_1_router.py:443-453``: all-equal logits select cells ``0..K-1`` with unit 0;
    a two-way tie between cells 9 and 2 puts the lower index first; a unit tie picks unit 0."""
    N, M = 16, 4
    cost = torch.full((M,), 1.0 / (N * M))
    cells, units, valid, theta, _ = O.router_select(torch.zeros(2, N, M), None, cost, k=5)
    assert cells.tolist() == [[0, 1, 2, 3, 4]] * 2 and units.tolist() == [[0] * 5] * 2
    assert bool(valid.all())
    tied = torch.zeros(1, N, M)
    tied[0, 9, 3] = 1.0
    tied[0, 2, 0] = 1.0
    tied[0, 2, 1] = 1.0
    cells, units, *_ = O.router_select(tied, None, cost, k=3)
    assert cells[0].tolist() == [2, 9, 0] and units[0].tolist() == [0, 3, 0]


def _f32(x):
    return float(np.float32(x))


def _brute_select(scores_cell, unit_arg, cost, K, limit, shared, overhead, age=None, age_max=0,
                  probes=False, reserved=0, fixed_units=False, M=1):
    """A direct restatement on Python lists: stable order by (-score, index) with NaN first,
    budget by a double running sum rounded to fp32, the threshold from its definition, the
    probes by repeated stalest-first picks."""
    N = len(scores_cell)

    # reserved first (+inf), then NaN (torch sorts NaN above +inf: handled by explicit rank)
    nan_cells = [n for n in range(reserved, N) if math.isnan(scores_cell[n])]
    rest = [n for n in range(reserved, N) if not math.isnan(scores_cell[n])]
    rest.sort(key=lambda n: (-scores_cell[n], n))
    order = nan_cells + list(range(reserved)) + rest if nan_cells else list(range(reserved)) + rest
    top = order[:K]
    units = [(k % M) if (fixed_units and k < reserved) else unit_arg[c] for k, c in enumerate(top)]
    acc = 0.0
    valid = []
    for u in units:
        acc += _f32(_f32(overhead) + cost[u])
        valid.append(_f32(_f32(shared) + _f32(acc)) <= _f32(limit))
    cells = [c if v else 0 for c, v in zip(top, valid)]
    units = [u if v else 0 for u, v in zip(units, valid)]
    sel = {c for c, v in zip(cells, valid) if v}
    lo = [scores_cell[n] for n in sel if n >= reserved]
    hi = [scores_cell[n] for n in range(N) if n not in sel]

    def amin(xs):
        return math.nan if any(math.isnan(x) for x in xs) else (min(xs) if xs else math.inf)

    def amax(xs):
        return math.nan if any(math.isnan(x) for x in xs) else (max(xs) if xs else -math.inf)

    theta = _f32(0.5 * _f32(amin(lo) + amax(hi)))
    refreshed = [False] * K
    if probes:
        n_valid = sum(valid)
        stale = [n for n in range(N) if age[n] > age_max and n not in sel]
        n_force = min(len(stale), max(n_valid - reserved, 0))
        stale.sort(key=lambda n: (-_f32(age[n]), n))
        new_cells, new_units = list(cells), list(units)
        for j in range(n_force):
            kk = n_valid - 1 - j
            new_cells[kk] = stale[j]
            new_units[kk] = unit_arg[stale[j]]
            refreshed[kk] = True
        spent = 0.0
        for u, v in zip(new_units, valid):
            spent = _f32(spent + (_f32(_f32(overhead) + cost[u]) if v else 0.0))
        if _f32(_f32(shared) + spent) > _f32(limit):
            refreshed = [False] * K
        else:
            cells, units = new_cells, new_units
    return cells, units, valid, theta, refreshed


@pytest.mark.parametrize("trial", range(24))
def test_router_matches_brute_force(trial):
    g = torch.Generator().manual_seed(100 + trial)
    B, N, M = 3, 9, 1 + trial % 3
    K = 1 + trial % 6
    logits = torch.randn(B, N, M, generator=g)
    if trial % 2:
        logits = (logits * 2).round() / 2  # exact ties between cells and between units
    if trial % 5 == 0:
        logits[0, 3, 0] = float("nan")
    cost = torch.tensor([0.125, 0.0625, 0.25][:M])  # dyadic: sums are order-independent
    overhead = 0.0625 if trial % 4 == 1 else 0.0
    shared = 0.125 if trial % 3 == 2 else 0.0
    limit = [10.0, 0.3, 0.5][trial % 3]
    reserved = 2 if (trial % 7 == 3 and K > 2) else 0
    fixed_units = reserved > 0 and trial % 2 == 1
    age = torch.randint(0, 6, (B, N), generator=g)
    probes = trial % 3 != 0
    cells, units, valid, theta, refreshed = O.router_select(
        logits, age, cost, k=K, age_max=2, probes=probes, cell_overhead=overhead,
        shared_cost=shared, limit=limit, reserved=reserved, reserved_units=fixed_units)
    for r in range(B):
        sc = logits[r].float().amax(dim=-1).tolist()
        ua = logits[r].float().argmax(dim=-1).tolist()
        want = _brute_select(sc, ua, cost.tolist(), K, limit, shared, overhead, age=age[r].tolist(),
                             age_max=2, probes=probes, reserved=reserved, fixed_units=fixed_units,
                             M=M)
        assert cells[r].tolist() == want[0]
        assert units[r].tolist() == want[1]
        assert valid[r].tolist() == want[2]
        th = float(theta[r])
        assert (math.isnan(th) and math.isnan(want[3])) or th == want[3]
        assert refreshed[r].tolist() == want[4]


def test_router_enumerates_stable_order_exhaustively():
    """Every assignment of scores from {0, 0.5, 1} to 4 cells: the selected cells are the first
    K of the permutation sorted by (descending score, ascending index)."""
    N, K = 4, 2
    cost = torch.tensor([1.0 / N])
    for values in itertools.product([0.0, 0.5, 1.0], repeat=N):
        logits = torch.tensor(values).reshape(1, N, 1)
        cells, *_ = O.router_select(logits, None, cost, k=K)
        want = sorted(range(N), key=lambda n: (-values[n], n))[:K]
        assert cells[0].tolist() == want


def test_router_theta_conventions():
    N = 4
    cost = torch.tensor([1.0 / N])
    logits = torch.tensor([[[1.0], [2.0], [3.0], [4.0]]])
    *_, theta, _ = O.router_select(logits, None, cost, k=2)
    assert float(theta[0]) == 2.5  # midpoint of 3 (lowest in) and 2 (highest out)
    *_, theta, _ = O.router_select(logits, None, cost, k=4)
    assert float(theta[0]) == -math.inf  # everything selected
    *_, theta, _ = O.router_select(logits, None, cost, k=2, limit=0.0)
    assert float(theta[0]) == math.inf  # nothing selected


# --------------------------------------------------------------------------------------------
# the window: composition and invariants, and its backward against float64 autograd
# --------------------------------------------------------------------------------------------


def _tiny_window(seed=1, B=2, T=8, N=16, d=16, K=2, M=1, rms=False):
    from hsn_amd.workload import CONFIGS, make_window

    cfg = CONFIGS["tiny"].scaled(B=B, T=T, N=N, d=d, K=K, M=M, h0_sigma=0.3)
    w = make_window(cfg, seed)
    return cfg, w


def test_window_forward_invariants():
    cfg, w = _tiny_window()
    out = O.window_forward(w["logits"], w["y"], w["gate_pre"], w["reset"], w["h0"], w["q0"],
                           w["age0"], w["pos0"], w["cost"], k=cfg.K)
    B, T, N, d = cfg.B, cfg.T, cfg.N, cfg.d
    # q stays the mean of h (q0 = mean h0 and every update moves q by the mean delta)
    _close(out["q"], out["h"].mean(dim=1), atol=1e-6, rtol=1e-5)
    # ages and positions from a direct count
    for r in range(B):
        resets = [t for t in range(T) if w["reset"][r, t]]
        lr = resets[-1] if resets else -1
        assert int(out["pos"][r]) == (T - lr if lr >= 0 else T)
        for n in range(N):
            sel = [t for t in range(T) if bool(((out["cells"][r, t] == n) & out["valid"][r, t]).any())]
            ls = sel[-1] if sel else -1
            want = T - 1 - ls if (ls >= 0 and ls >= lr) else (T - lr if lr >= 0 else T)
            assert int(out["age"][r, n]) == want
    # h_sel of a valid slot is the updated state; h_old the pre-round one
    assert out["h_sel"].shape == (B, T, cfg.K, d) and out["h_old"].shape == (B, T, cfg.K, d)


@pytest.mark.parametrize("rms", [False, True])
def test_window_backward_equals_autograd_of_the_forward(rms):
    """``window_backward`` (recurrence + activation VJPs + carried state) is the float64 autograd
    gradient of a window objective built from the restated forward chain."""
    cfg, w = _tiny_window(B=2, T=7, N=6, d=5, K=3)
    g = torch.Generator().manual_seed(11)
    B, T, N, d, K = cfg.B, cfg.T, cfg.N, cfg.d, cfg.K
    y = w["y"].to(F64).requires_grad_(True)
    gp = w["gate_pre"].to(F64).requires_grad_(True)
    h0 = w["h0"].to(F64).requires_grad_(True)
    q0 = w["q0"].to(F64).detach().requires_grad_(True)
    cw = (torch.rand(d, generator=g, dtype=F64) + 0.5).requires_grad_(True) if rms else None
    w_pre = torch.randn(B, T, d, generator=g, dtype=F64)
    w_post = torch.randn(B, T, d, generator=g, dtype=F64)
    w_sel = torch.randn(B, T, K, d, generator=g, dtype=F64)
    w_hT = torch.randn(B, N, d, generator=g, dtype=F64)
    w_qT = torch.randn(B, d, generator=g, dtype=F64)
    reset = w["reset"].clone()
    reset[1, 3] = True
    total = O.window_objective_f64(w["logits"], y, gp, reset, h0, q0, w["cost"], K, w_pre, w_post,
                                   w_sel, w_hT, w_qT, cand_norm=rms, cand_w=cw)
    wanted = [y, gp, h0, q0] + ([cw] if rms else [])
    want = torch.autograd.grad(total, wanted)
    fwd = O.window_forward(w["logits"], y.detach(), gp.detach(), reset, h0.detach(), q0.detach(),
                           w["age0"], w["pos0"], w["cost"], k=K, cand_norm=rms,
                           cand_w=None if cw is None else cw.detach())
    # window_backward computes in fp32 on widened inputs; rebuild it in float64 for the pin
    yf = y.detach().requires_grad_(True)
    gf = gp.detach().requires_grad_(True)
    wf = None if cw is None else cw.detach().requires_grad_(True)
    c = O.candidate(yf, rms, wf)
    b = O.gate(gf)
    dc, db, d_h0, d_q0 = O.recurrence_backward(
        c.detach(), b.detach(), fwd["h_old"].to(F64), fwd["cells"], fwd["valid"], reset, N, w_pre,
        w_post, torch.where(fwd["valid"][..., None], w_sel, 0.0), w_hT, w_qT, carried=True)
    inputs = [yf, gf] + ([wf] if rms else [])
    got = list(torch.autograd.grad([c, b], inputs, [dc, db]))
    got = got[:2] + [d_h0, d_q0] + got[2:]
    for x, ref in zip(got, want):
        _close(x, ref, atol=1e-12, rtol=1e-10)
    # and the fp32 entry point agrees with the float64 pin to fp32 rounding
    dy, dg, dh0, dq0, dw = O.window_backward(
        w["y"], w["gate_pre"], fwd["h_old"].float(), fwd["cells"], fwd["valid"], reset, N,
        w_pre.float(), w_post.float(), w_sel.float(), w_hT.float(), w_qT.float(), cand_norm=rms,
        cand_w=None if cw is None else cw.detach().float())
    for x, ref in zip([dy, dg, dh0, dq0] + ([dw] if rms else []), want):
        _close(x.double(), ref, atol=2e-5, rtol=2e-4)


def test_planted_mistake_fails_the_pin():
    """A dropped summary term (``share``) in the sweep is caught by the autograd comparison."""
    s = _recurrence_case()
    N = s["N"]

    def broken(c, b, h_old, cells, valid, reset, n, dpre, dpost, dsel):
        # the sweep without R / N in g: a plausible dropped term
        return O.recurrence_backward(c, b, h_old, cells, valid, reset, n, None, None, dsel)

    B, T, K, d = s["B"], s["T"], s["K"], s["d"]
    h, q = s["h0"], s["q0"]
    age = torch.zeros(B, N, dtype=torch.int64)
    pos = torch.zeros(B, dtype=torch.int64)
    total = torch.zeros((), dtype=F64)
    h_old = []
    for t in range(T):
        h, q, age, pos = O.reset_state(h, q, age, pos, s["reset"][:, t])
        total = total + (q * s["w_pre"][:, t]).sum()
        h_old.append(h.gather(1, s["cells"][:, t, :, None].expand(B, K, d)).detach())
        h, q, age, _ = O.gated_delta_update(h, q, age, s["cells"][:, t], s["c"][:, t],
                                            s["b"][:, t], s["valid"][:, t])
        total = total + (q * s["w_post"][:, t]).sum()
    want_c, _ = torch.autograd.grad(total, [s["c"], s["b"]])
    got_c, _ = broken(s["c"].detach(), s["b"].detach(), torch.stack(h_old, 1), s["cells"],
                      s["valid"], s["reset"], N, s["w_pre"], s["w_post"], None)
    assert not torch.allclose(got_c, want_c)


# --------------------------------------------------------------------------------------------
# the RMS candidate: tanh(RMSNorm(y)) with torch's nn.RMSNorm(d, eps=1e-6) (the reference's
# python/hsn/model/cell.py:206-212,480-484), pinned by its published definition, a closed form,
# an invariant and finite differences; planted mistakes must fail these pins
# --------------------------------------------------------------------------------------------


def _rms_rows(seed=21, d=12):
    """Rows of several magnitudes: unit scale, large, and small enough that eps dominates."""
    g = torch.Generator().manual_seed(seed)
    y = torch.randn(6, d, generator=g, dtype=F64)
    y[2] *= 40.0
    y[3] *= 1e-3  # mean(y^2) ~ 1e-6: eps = 1e-6 matters here
    y[4] *= 3e-4
    w = torch.rand(d, generator=g, dtype=F64) + 0.5
    return y, w


def _rms_pins_hold(cand, eps=1e-6) -> bool:
    """Every pin of the RMS candidate against a candidate function ``cand(y, w, eps)``:

    1. torch's documented RMSNorm, ``y / sqrt(mean(y^2) + eps) * weight`` (eps inside the root,
       the mean over the last dimension, the gain after the normalisation), in float64;
    2. the constant row ``y = c * 1``: ``tanh(c / sqrt(c^2 + eps) * w)``;
    3. with a unit gain and ``eps = 0``, ``atanh(candidate)`` has mean square exactly 1 per row.
    """
    y, w = _rms_rows()
    ok = True
    want = torch.tanh(y / torch.sqrt((y * y).sum(-1, keepdim=True) / y.shape[-1] + eps) * w)
    ok &= bool(torch.allclose(cand(y, w, eps), want, atol=1e-12, rtol=1e-12))
    for c in (0.7, -2.5, 1e-3, -3e-4):
        row = torch.full((1, y.shape[-1]), c, dtype=F64)
        closed = torch.tanh(torch.tensor(c, dtype=F64) / math.sqrt(c * c + eps) * w)
        ok &= bool(torch.allclose(cand(row, w, eps)[0], closed, atol=1e-12, rtol=1e-12))
    pre = torch.atanh(cand(y[:2], torch.ones_like(w), 0.0))
    ok &= bool(torch.allclose((pre * pre).mean(-1), torch.ones(2, dtype=F64), atol=1e-10))
    return ok


def test_rms_candidate_pins():
    assert _rms_pins_hold(lambda y, w, eps: O.candidate(y, True, w, eps))


def test_rms_candidate_planted_mistakes_fail_the_pins():
    """Plausible mistakes in the candidate each fail at least one pin."""
    def norm(y, w, eps, *, inside=True, mean=True, gain=True, gain_first=False):
        x = y * w if gain_first else y
        ms = (x * x).mean(-1, keepdim=True) if mean else (x * x).sum(-1, keepdim=True)
        den = torch.sqrt(ms + eps) if inside else torch.sqrt(ms) + eps
        out = x / den
        return torch.tanh(out * w if (gain and not gain_first) else out)

    mistakes = {
        "eps 1e-5": lambda y, w, eps: norm(y, w, 1e-5),
        "eps outside the root": lambda y, w, eps: norm(y, w, eps, inside=False),
        "sum for mean": lambda y, w, eps: norm(y, w, eps, mean=False),
        "gain dropped": lambda y, w, eps: norm(y, w, eps, gain=False),
        "gain before the norm": lambda y, w, eps: norm(y, w, eps, gain_first=True),
    }
    assert _rms_pins_hold(lambda y, w, eps: norm(y, w, eps))  # the correct form passes
    for name, bad in mistakes.items():
        assert not _rms_pins_hold(bad), f"the pins miss the mistake: {name}"


def test_rms_candidate_gradient_matches_finite_differences():
    """The oracle's d(candidate)/d(y, w) (autograd, which the window backward's d_cand_w uses)
    against central finite differences in float64."""
    y, w = _rms_rows(seed=22, d=5)
    y = y[[0, 2, 3]].clone().requires_grad_(True)
    w = w.clone().requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b: O.candidate(a, True, b, 1e-6), (y, w),
                                    eps=1e-7, atol=1e-6, rtol=1e-5)


# --------------------------------------------------------------------------------------------
# the row maximum h_max: NaN-propagating (the reference's test_p2_10_window.py:540-560)
# --------------------------------------------------------------------------------------------


def test_h_max_propagates_a_nan_in_an_unwritten_cell():
    cfg, w, quiet = nan_state_window()
    out = O.window_forward(w["logits"], w["y"], w["gate_pre"], w["reset"], w["h0"], w["q0"],
                           w["age0"], w["pos0"], w["cost"], k=cfg.K)
    assert not bool((out["cells"] == quiet).any()), "the NaN cell must stay unwritten"
    hm = out["h_max"]
    assert bool(torch.isnan(hm[0]).all())
    assert bool(torch.isnan(hm[1, :3]).all()) and bool(torch.isfinite(hm[1, 3:]).all())
    # the NaN never reaches the summaries or the written slots
    for key in ("q_pre", "q_post", "h_old", "h_sel"):
        assert bool(torch.isfinite(out[key]).all()), key
    # a plain max (NaN-ignoring, as a careless reduction would be) fails this pin
    finite = torch.nan_to_num(out["h"], nan=0.0).abs().flatten(1).amax(1)
    assert not bool(torch.isnan(finite).any())


# ------------------------------------------------------------------------------------------------
# The trainer passes' oracle (fma32 and the tr_* restatements)
# ------------------------------------------------------------------------------------------------

def _round32(x):
    """The float32 nearest (ties to even) to the exact rational x (a Fraction), as numpy float32."""
    import numpy as np
    from fractions import Fraction

    if x == 0:
        return np.float32(0.0)
    sign = -1 if x < 0 else 1
    ax = abs(x)
    e = ax.numerator.bit_length() - ax.denominator.bit_length()
    if Fraction(2) ** e > ax:
        e -= 1
    quantum = Fraction(2) ** (max(e, -126) - 23)  # subnormals below 2^-126
    q = ax / quantum
    n = q.numerator // q.denominator
    rest = q - n
    if rest > Fraction(1, 2) or (rest == Fraction(1, 2) and n % 2 == 1):
        n += 1
    v = n * quantum
    if v >= Fraction(2) ** 128:
        return np.float32(sign * np.inf)
    return np.float32(sign * float(v))


def _bits(x):
    import numpy as np

    return np.asarray(x, np.float32).view(np.int32)


def test_fma32_rounds_once_like_exact_arithmetic():
    """fma32 against the exact rational a * b + c rounded once: random operands over many
    magnitudes, planted float32 midpoints with no tail (ties to even) and with a tail of either
    sign, signed zeros, subnormal results and an overflow."""
    import numpy as np
    from fractions import Fraction

    rng = np.random.default_rng(11)
    n = 3000
    a = (rng.standard_normal(n) * 10.0 ** rng.integers(-20, 20, n)).astype(np.float32)
    b = (rng.standard_normal(n) * 10.0 ** rng.integers(-20, 20, n)).astype(np.float32)
    c = (rng.standard_normal(n) * 10.0 ** rng.integers(-20, 20, n)).astype(np.float32)
    half = np.float32(2.0 ** -12)
    tail = np.float32(2.0 ** -12 * (1 + 2.0 ** -23))
    extra = [
        (half, half, 1.0),        # 1 + 2^-24 exactly: a tie, to the even 1
        (tail, half, 1.0),        # above the midpoint: up to 1 + 2^-23
        (-tail, half, 1.0),       # below 1 - 2^-25 ... down from the midpoint below 1
        (half, half, 1.0 + 2.0 ** -23),  # a tie whose even neighbour is above
        (0.0, 3.0, -0.0), (-0.0, 3.0, -0.0), (0.0, -3.0, 0.0),
        (1e-30, 1e-15, 0.0),      # a subnormal product
        (3e-39, 0.5, 1e-45),      # subnormal operands
        (1e30, 1e10, -1.0),       # overflow
    ]
    a = np.concatenate([a, np.float32([e[0] for e in extra])])
    b = np.concatenate([b, np.float32([e[1] for e in extra])])
    c = np.concatenate([c, np.float32([e[2] for e in extra])])
    got = O.fma32(a, b, c)
    for i in range(a.size):
        exact = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        want = _round32(exact)
        if exact == 0:  # the sign of an exact zero: -0 only from -0 + -0
            want = np.float32(-0.0) if (np.signbit(a[i] * b[i]) and np.signbit(c[i])) else np.float32(0.0)
        assert _bits(got[i]) == _bits(want), (a[i], b[i], c[i], got[i], want)


def test_lerp_oracle_hits_its_end_points_and_rounds_each_branch_once():
    import numpy as np
    from fractions import Fraction

    rng = np.random.default_rng(12)
    s = rng.standard_normal(500).astype(np.float32)
    e = rng.standard_normal(500).astype(np.float32)
    assert np.array_equal(_bits(O.tr_lerp(s, e, 0.0)), _bits(s))
    assert np.array_equal(_bits(O.tr_lerp(s, e, 1.0)), _bits(e))
    for w in (np.float32(0.1), np.float32(0.49), np.float32(0.5), np.float32(0.99)):
        got = O.tr_lerp(s, e, w)
        diff = (e - s).astype(np.float32)
        for i in range(s.size):
            if w < 0.5:
                exact = Fraction(float(s[i])) + Fraction(float(w)) * Fraction(float(diff[i]))
            else:
                one_minus = np.float32(1.0) - w
                exact = Fraction(float(e[i])) - Fraction(float(diff[i])) * Fraction(float(one_minus))
            assert _bits(got[i]) == _bits(_round32(exact)), (w, i)


def test_plain_trainer_passes_equal_torch_cpu_operations():
    """The passes with no fused operation against torch's CPU operations bit for bit: the float64
    clip's scaling, the update caps' squares and projection."""
    import numpy as np

    g = torch.Generator().manual_seed(13)
    p = torch.randn(4000, generator=g)
    old = torch.randn(4000, generator=g)
    p[:4] = torch.tensor([0.0, -0.0, 1e-42, 3e30])
    coef = torch.tensor(0.3713, dtype=torch.float64)
    want = (p.double() * coef).float()
    assert np.array_equal(_bits(O.tr_scale64(p.numpy(), float(coef))), _bits(want.numpy()))
    sq_old, sq_delta = O.tr_limit_squares(p.numpy(), old.numpy())
    assert np.array_equal(_bits(sq_old), _bits(old.square().numpy()))
    assert np.array_equal(_bits(sq_delta), _bits((p - old).square().numpy()))
    for clipped in (True, False):
        scale = torch.tensor(0.625)
        want_p = torch.where(torch.tensor(clipped), old + (p - old) * scale, p)
        got_p, got_sq = O.tr_limit_project(p.numpy(), old.numpy(), 0.625, clipped)
        assert np.array_equal(_bits(got_p), _bits(want_p.numpy()))
        assert np.array_equal(_bits(got_sq), _bits((want_p - old).square().numpy()))


def test_adamw_oracle_first_steps_reduce_to_their_closed_forms():
    """From an all-zero state the first step's moments are single roundings: m = (1 - beta1) g
    (the lerp from 0) and, with beta2 = 0, v = g^2; with beta1 = 0 the lerp's weight is 1 and m is
    g itself. A zero gradient from a zero state leaves the weight at its decayed value."""
    import numpy as np

    rng = np.random.default_rng(14)
    p = rng.standard_normal(800).astype(np.float32)
    g = rng.standard_normal(800).astype(np.float32)
    z = np.zeros_like(p)
    lr, eps, wd = 2.5e-3, 1e-8, 0.01
    for beta1, beta2 in ((0.9, 0.0), (0.0, 0.0)):
        coefs = [1 - lr * wd, 1 - beta1, beta2, 1 - beta2, 1.0 / (1 - beta2) ** 0.5, eps,
                 -lr / (1 - beta1)]
        _, m, v = O.tr_adamw(p, g, z, z, coefs, True)
        assert np.array_equal(_bits(m), _bits(np.float32(1 - beta1) * g))
        assert np.array_equal(_bits(v), _bits(g * g))
    coefs = [1 - lr * wd, 0.1, 0.999, 0.001, 1.0 / 0.001 ** 0.5, eps, -lr / 0.1]
    p1, m, v = O.tr_adamw(p, z, z, z, coefs, True)
    assert np.array_equal(_bits(p1), _bits(p * np.float32(1 - lr * wd)))
    assert not m.any() and not v.any()
    # the unit form with every unit active and equal coefficients is the dense form
    M = 8
    pu = p.reshape(M, -1)
    table = np.float32([[1.0] * M, [coefs[0]] * M, [coefs[1]] * M, [coefs[2]] * M,
                        [0.001 ** 0.5] * M, [lr / 0.1] * M])
    gu = g.reshape(M, -1)
    pd, md, vd = O.tr_adamw(p, g, z, z, [coefs[0], coefs[1], coefs[2], coefs[3],
                                         np.float32(1.0) / np.float32(0.001 ** 0.5), eps, -lr / 0.1], True)
    pu1, mu, vu = O.tr_adamw_units(pu, gu, z.reshape(M, -1), z.reshape(M, -1), table, 0.001, eps, True)
    assert np.array_equal(_bits(mu.reshape(-1)), _bits(md))
    assert np.array_equal(_bits(vu.reshape(-1)), _bits(vd))


# --------------------------------------------------------------------------------------------
# the fused cell round's contract (window_cell_round)
# --------------------------------------------------------------------------------------------


def _round_by_state_gradient(p):
    """The same round from ``oracle.state_gradient.cell_round`` (the cell's equations restated
    separately: the sources gathered and summed by hand, alpha on W_out's output) and the gated
    update written out: ``(h', q', age', pos', h_sel)``."""
    from oracle import state_gradient as S

    B, N, d = p["h"].shape
    K = p["cells"].shape[1]
    D = p["pad_src"].shape[1]
    w = S.CellWeights(
        w1=p["W1"], b1=p["b1"], w2=p["W2"], b2=p["b2"], gate_w=p["gate_w"], gate_b=p["gate_b"],
        norm_gain=p["norm_w"], norm_eps=p["norm_eps"],
        cand_gain=p["cand_w"] if p["cand_norm"] else None, cand_eps=p["cand_eps"],
        w_out=p["W_out"], v=p["V"], pad_src=p["pad_src"],
        pad_mask=torch.ones(N, D, dtype=torch.bool), edge_weights=p["edge_w"], activation="gelu")
    extra = torch.cat([p["u"], p["eps"]], dim=-1)[:, None, :].expand(B, K, 2 * d)
    c, b, _ = S.cell_round(p["h"], extra, p["cells"], p["units"], p["valid"], p["alpha"], w)
    h2 = p["h"].clone()
    age2 = p["age"] + 1
    for r in range(B):
        for k in range(K):
            if bool(p["valid"][r, k]):
                i = int(p["cells"][r, k])
                h2[r, i] = (1 - b[r, k]) * p["h"][r, i] + b[r, k] * c[r, k]
                age2[r, i] = 0
    q2 = p["q"] + (h2 - p["h"]).sum(dim=1) / N
    safe = torch.where(p["valid"], p["cells"], torch.zeros_like(p["cells"]))
    h_sel = torch.stack([h2[r, safe[r]] for r in range(B)])
    return h2, q2, age2, p["pos"] + 1, h_sel


@pytest.mark.parametrize("case", [
    dict(),  # the reference's default cell at B=4
    dict(pad=0.4, seed=3),  # a budget that pads slots
    dict(cand_norm=False, B=5, seed=4),
    dict(B=7, N=11, d=24, K=5, M=3, H=77, D=3, seed=5, pad=0.2),  # its odd sizes
    dict(B=1, N=32, d=64, K=1, M=1, H=33, D=4, seed=6),  # one unit, one slot
    dict(alpha_one=False, seed=7, B=3),  # alpha away from 1: its place relative to the norm
    dict(alpha_one=False, cand_norm=False, seed=8, B=3),
    dict(D=0, seed=9, B=2),  # no edges
])
def test_window_cell_round_matches_the_cell_equations(case):
    """``window_cell_round`` (the P2.9 ops, golden-pinned, composed in the native round's order)
    equals the cell's equations restated separately, to float64 rounding; cells no slot writes
    keep their state bit for bit."""
    from conftest import round_problem

    p = round_problem(**case)
    got = O.window_cell_round(**p)
    want = _round_by_state_gradient(p)
    for name, a, b in zip(("h", "q", "age", "pos", "h_sel"), got, want):
        if a.dtype == torch.int64:
            assert torch.equal(a, b), name
        else:
            _close(a, b, atol=1e-12, rtol=1e-12)
    written = O.selection_mask(p["cells"], p["valid"], p["h"].shape[1])
    assert torch.equal(got[0][~written], p["h"][~written])


@pytest.mark.parametrize("cand_norm", [False, True])
def test_window_cell_round_closed_form(cand_norm):
    """With the first layer and the gate's weights zero, F is the unit's output bias and the gate
    its bias: h' = (1 - sigmoid(gate_b)) h + sigmoid(gate_b) tanh(alpha W_out b2_j) (with the
    candidate norm, W_out b2_j normalised first). W_out is not symmetric, so a transposed W_out
    fails; alpha is not 1, so alpha on the wrong side of the norm fails."""
    from conftest import round_problem

    p = round_problem(B=3, N=9, d=8, K=3, M=2, H=5, D=2, cand_norm=cand_norm, alpha_one=False,
                      seed=12)
    p["W1"] = torch.zeros_like(p["W1"])
    p["b1"] = torch.zeros_like(p["b1"])
    p["gate_w"] = torch.zeros_like(p["gate_w"])
    h2, q2, _, _, _ = O.window_cell_round(**p)
    sg = 1.0 / (1.0 + torch.exp(-p["gate_b"]))
    for r in range(3):
        for k in range(3):
            if not bool(p["valid"][r, k]):
                continue
            i, j, a = int(p["cells"][r, k]), int(p["units"][r, k]), float(p["alpha"][r, k])
            y = p["W_out"] @ p["b2"][j]
            if cand_norm:
                y = y / torch.sqrt((y * y).mean() + p["cand_eps"]) * p["cand_w"]
            c = torch.tanh(a * y)
            _close(h2[r, i], (1 - sg) * p["h"][r, i] + sg * c, atol=1e-13, rtol=1e-13)
    assert not torch.allclose(p["W_out"], p["W_out"].T)


@pytest.mark.parametrize("mistake", [
    ("alpha before the candidate norm",
     "y = torch.nn.functional.rms_norm(F @ W_out.T", "y = torch.nn.functional.rms_norm((a * F) @ W_out.T"),
    ("gate on the raw input", "b = gate(v @ gate_w.T", "b = gate(v_raw @ gate_w.T"),
    ("W_out transposed", "c = torch.tanh((a * F) @ W_out.T)", "c = torch.tanh((a * F) @ W_out)"),
    ("unit MLP on the raw input", "grouped_unit_mlp(v.reshape", "grouped_unit_mlp(v_raw.reshape"),
], ids=lambda m: m[0].replace(" ", "_"))
def test_window_cell_round_planted_mistakes_fail_the_pin(mistake):
    """Each plausible mistake, planted in a copy of ``window_cell_round``'s source, moves the new
    state away from the cell's equations on at least one of the pin's cases."""
    import inspect

    from conftest import round_problem

    name, old, new = mistake
    src = inspect.getsource(O.window_cell_round)
    assert old in src, name
    namespace = dict(vars(O))
    exec(src.replace(old, new), namespace)
    planted = namespace["window_cell_round"]
    caught = 0
    for case in (dict(), dict(alpha_one=False, seed=7, B=3),
                 dict(alpha_one=False, cand_norm=False, seed=8, B=3)):
        p = round_problem(**case)
        got = planted(**p)[0]
        want = _round_by_state_gradient(p)[0]
        caught += not torch.allclose(got, want, atol=1e-12, rtol=1e-12)
    assert caught, f"the planted mistake '{name}' passed the pin"
