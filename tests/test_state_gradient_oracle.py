"""Pins of the state-gradient sweep's oracle (``oracle/state_gradient.py``), on the CPU in
float64: the hand-written backward against autograd of the forward it belongs to."""

from __future__ import annotations

import pytest
import torch

from conftest import sweep_oracle, sweep_problem
from oracle import hsn_oracle as O
from oracle import state_gradient as S

F64 = torch.float64


@pytest.mark.parametrize("name", S.ACTIVATIONS)
def test_activation_grad_is_autograd_of_the_activation(name):
    x = torch.linspace(-4, 4, 801, dtype=F64).requires_grad_(True)
    (grad,) = torch.autograd.grad(S.activation(name, x).sum(), x)
    keep = x.detach().abs() > 1e-9  # relu's kink
    torch.testing.assert_close(S.activation_grad(name, x.detach())[keep], grad[keep],
                               rtol=1e-12, atol=1e-13)


@pytest.mark.parametrize("cand_norm,cell_norm,act", [
    (True, True, "gelu"), (False, True, "relu"), (True, False, "silu"), (False, False, "tanh"),
])
def test_cell_state_vjp_is_autograd_of_the_cell_round(cand_norm, cell_norm, act):
    """The VJP of one position's candidates and gates with respect to the cell's own pre-round
    state and its weighted source sum, against autograd of ``cell_round`` with those as leaves."""
    p = sweep_problem(B=3, T=1, K=4, N=9, d=5, H=7, M=3, cand_norm=cand_norm,
                      cell_norm=cell_norm, act=act, seed=3)
    w = p["w"]
    B, K, d = 3, 4, 5
    cells, units, valid, alpha = p["cells"][:, 0], p["units"][:, 0], p["valid"][:, 0], p["alpha"][:, 0]
    h = p["h0"]
    safe = torch.where(valid, cells, torch.zeros_like(cells))
    own = torch.stack([h[i, safe[i]] for i in range(B)]).requires_grad_(True)
    src = w.pad_src[safe]
    gathered = torch.stack([h[i, src[i]] for i in range(B)])
    src_sum = (w.edge_weights[safe][..., None] * gathered).sum(dim=2).requires_grad_(True)
    c, b, rec = S.cell_round(h, p["extra"][:, 0], cells, units, valid, alpha, w, src_sum=src_sum,
                             own=own)
    g = torch.Generator().manual_seed(5)
    w_c = torch.randn(B, K, d, generator=g, dtype=F64)
    w_b = torch.randn(B, K, d, generator=g, dtype=F64)
    d_own, d_src = torch.autograd.grad((w_c * c).sum() + (w_b * b).sum(), [own, src_sum])
    dh, dvm = S.cell_state_vjp(
        w_c, w_b, c=c.detach(), b=b.detach(), h_old=own.detach(), units=units,
        y=rec["y"].detach(), alpha=alpha, hidden=rec["hidden"].detach(),
        gate_pre=rec["gate_pre"].detach(), m=rec["m"].detach(),
        rms=rec["rms"].detach() if cell_norm else None, consts=p["consts"])
    torch.testing.assert_close(dh, d_own, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(dvm, d_src, rtol=1e-10, atol=1e-12)


def _autograd_sweep(p):
    """dL/dc and dL/db of every position from autograd of the window's forward, through probes
    added where c and b are used, with L the cotangents' inner product with the outputs."""
    B, T, K = p["cells"].shape
    d = p["h0"].shape[-1]
    probe_c = torch.zeros(B, T, K, d, dtype=F64, requires_grad=True)
    probe_b = torch.zeros(B, T, K, d, dtype=F64, requires_grad=True)
    outs, _ = S.window_outputs(p["h0"], p["extra"], p["cells"], p["units"], p["valid"],
                               p["alpha"], p["reset"], p["w"], p["n_read"], probe_c, probe_b)
    cot = p["cot"]
    loss = ((cot["d_q_pre"] * outs["q_pre"]).sum() + (cot["d_q_post"] * outs["q_post"]).sum()
            + (cot["d_h_sel"] * outs["h_sel"]).sum())
    if cot["d_h_fast"] is not None:
        loss = loss + (cot["d_h_fast"] * outs["h_fast"]).sum()
    dc, db = torch.autograd.grad(loss, [probe_c, probe_b])
    return dc, db


CASES = {
    "norms_gelu": dict(),
    "no_cand_norm_relu": dict(cand_norm=False, act="relu"),
    "no_cell_norm_silu": dict(cell_norm=False, act="silu"),
    "no_norms_tanh": dict(cand_norm=False, cell_norm=False, act="tanh"),
    "fast_read": dict(n_read=2, resets=((0, 1), (1, 3))),
    "reset_first_last_and_twice": dict(T=6, resets=((0, 0), (0, 5), (1, 2), (1, 3))),
    "alpha_one_no_padding": dict(alpha_one=True, pad_every=10 ** 6),
    "wide_fan_out": dict(N=5, D=4, K=4, seed=9),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_sweep_is_autograd_of_the_window(name):
    """The reverse sweep's total dL/dc and dL/db against float64 autograd of the window's
    forward with the state read live (every later position's read of every cell and source)."""
    p = sweep_problem(**CASES[name])
    want_dc, want_db = _autograd_sweep(p)
    dc, db = sweep_oracle(p)
    assert not torch.equal(want_dc, torch.zeros_like(want_dc))
    torch.testing.assert_close(dc, want_dc, rtol=1e-9, atol=1e-11)
    torch.testing.assert_close(db, want_db, rtol=1e-9, atol=1e-11)


def test_sweep_without_the_state_read_is_the_window_recurrence():
    """With the cell's read of the state switched off (no first-layer or gate weight on the
    state columns, no messages, no cell norm: the norm's scale reads the state too) the sweep is
    the window path's pinned recurrence backward."""
    p = sweep_problem(seed=4)
    c = p["consts"]
    quiet = c._replace(w1_state=torch.zeros_like(c.w1_state),
                       gate_state=torch.zeros_like(c.gate_state), v=torch.zeros_like(c.v),
                       norm_gain_state=None)
    dc, db = sweep_oracle(p, consts=quiet)
    cot = p["cot"]
    want = O.recurrence_backward(p["c"], p["b"], p["h_old"], p["cells"], p["valid"], p["reset"],
                                 p["N"], cot["d_q_pre"], cot["d_q_post"], cot["d_h_sel"])
    torch.testing.assert_close(dc, want[0], rtol=1e-12, atol=1e-14)
    torch.testing.assert_close(db, want[1], rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("mistake", ["tanh_gelu", "in_dim", "edge_weight", "cand_eps", "v_t"])
def test_planted_mistakes_fail_the_autograd_pin(mistake, monkeypatch):
    """Plausible mistakes in the sweep or its constants each move dL/dc or dL/db away from
    autograd: a tanh-approximated GELU derivative, the cell norm's width off by one, the message
    weights dropped, the candidate norm's eps wrong, V transposed."""
    p = sweep_problem(seed=6, n_read=1)
    c = p["consts"]
    consts = c
    if mistake == "tanh_gelu":
        exact = S.activation_grad

        def approx(name, x):
            if name != "gelu":
                return exact(name, x)
            k = (2.0 / torch.pi) ** 0.5
            u = k * (x + 0.044715 * x ** 3)
            t = torch.tanh(u)
            return 0.5 * (1 + t) + 0.5 * x * (1 - t * t) * k * (1 + 3 * 0.044715 * x * x)

        monkeypatch.setattr(S, "activation_grad", approx)
    elif mistake == "in_dim":
        consts = c._replace(in_dim=c.in_dim + 1)
    elif mistake == "edge_weight":
        consts = c._replace(edge_weights=torch.where(c.pad_mask, 1.0, 0.0).to(F64))
    elif mistake == "cand_eps":
        consts = c._replace(cand_eps=1e-2)
    else:
        consts = c._replace(v=c.v.T.contiguous())
    want_dc, want_db = _autograd_sweep(p)
    dc, db = sweep_oracle(p, consts=consts)
    close = torch.allclose(dc, want_dc, rtol=1e-9, atol=1e-11) and torch.allclose(
        db, want_db, rtol=1e-9, atol=1e-11)
    assert not close, f"the planted mistake {mistake} passed the pin"


def test_out_adjacency_lists_every_edge_by_its_source():
    g = torch.Generator().manual_seed(2)
    pad_src = torch.randint(0, 6, (6, 3), generator=g)
    pad_mask = torch.rand(6, 3, generator=g) < 0.7
    out_tgt, out_edge = S.out_adjacency(pad_src, pad_mask)
    edges = sorted((int(pad_src[t, s]), t, t * 3 + s) for t in range(6) for s in range(3)
                   if bool(pad_mask[t, s]))
    listed = sorted((n, int(out_tgt[n, j]), int(out_edge[n, j])) for n in range(6)
                    for j in range(out_tgt.shape[1]) if int(out_tgt[n, j]) >= 0)
    assert listed == edges
    for n in range(6):  # by target, then slot
        row = [(int(out_tgt[n, j]), int(out_edge[n, j])) for j in range(out_tgt.shape[1])
               if int(out_tgt[n, j]) >= 0]
        assert row == sorted(row)
