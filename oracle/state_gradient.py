"""CPU oracle of the state-gradient reverse sweep (P2.10c): a PyTorch-CPU restatement of the
reference's ``python/hsn/train/state_gradient.py``.

TEST INFRASTRUCTURE ONLY. Only ``tests/`` may import this module, and only as the checker. The
product (``hsn_amd.state_sweep``) never calls it: its sweep runs the HIP library or declines.

Functions and what they restate:

* ``activation_grad``: ``state_gradient.py:174-188`` (the exact, erf GELU).
* ``out_adjacency``: ``python/hsn/train/state_sweep.py:86-109`` (the message graph by source).
* ``cell_state_vjp``: ``state_gradient.py:288-350``: the selected cells' candidate and gate,
  backward into the state they read (their own cell and their messages' weighted source sum).
* ``state_gradient_backward``: ``state_gradient.py:353-474`` without the row limit: the reverse
  sweep, total ``dL/dc`` and ``dL/db`` of every position.
* ``cell_round`` / ``window_outputs``: the forward these are the backward of, restated from the
  equations of ``state_gradient.py:32-59`` (the cell at a selected slot) and the window's gated
  update (``python/hsn/model/state.py``, ``native.gated_delta_update``): the pins' float64
  autograd runs through them.

Pins (``tests/test_state_gradient_oracle.py``): ``activation_grad`` against autograd of torch's
activations; ``cell_state_vjp`` against float64 autograd of ``cell_round`` with respect to the
cell's own pre-round state and its weighted source sum; ``state_gradient_backward`` against
float64 autograd of ``window_outputs`` (the total derivative with respect to every position's
``c`` and ``b``, through every later position's read of the state), with resets, padded slots,
fast-read cells, both norms on and off and every activation; with the state read switched off
it is the window path's pinned ``recurrence_backward``; planted mistakes (the norm's inner
product dropped, the tanh-approximated GELU, the message weight left out) each fail a pin.
"""

from __future__ import annotations

import math
from typing import NamedTuple, Optional

import torch
from torch import Tensor

__all__ = [
    "CellConstants",
    "CellWeights",
    "activation",
    "activation_grad",
    "cell_constants",
    "cell_round",
    "cell_state_vjp",
    "out_adjacency",
    "state_gradient_backward",
    "window_outputs",
]

ACTIVATIONS = ("gelu", "relu", "silu", "tanh")


class CellConstants(NamedTuple):
    """What the sweep reads of the cell's weights (the reference's ``CellConstants``,
    ``state_gradient.py:134-156``): ``w_out [d, d]`` (y = F @ w_out.T), ``cand_gain [d]`` or
    None, ``cand_eps``, ``w2 [M, H, d]``, ``w1_state [M, 2d, H]`` (the first layer's rows at the
    state columns), ``b1 [M, H]``, ``gate_state [d, 2d]``, ``gate_bias [d]``, ``norm_gain_state
    [2d]`` or None, ``in_dim`` (n), ``v [d, d]`` (V h = h @ v.T), ``edge_weights [N, D]``,
    ``pad_src`` int64 ``[N, D]``, ``activation``, ``pad_mask`` bool ``[N, D]``."""

    w_out: Tensor
    cand_gain: Optional[Tensor]
    cand_eps: float
    w2: Tensor
    w1_state: Tensor
    b1: Tensor
    gate_state: Tensor
    gate_bias: Tensor
    norm_gain_state: Optional[Tensor]
    in_dim: int
    v: Tensor
    edge_weights: Tensor
    pad_src: Tensor
    activation: str
    pad_mask: Optional[Tensor] = None


class CellWeights(NamedTuple):
    """The whole cell of the forward (``cell_round``): the first layer over all ``n`` input
    columns ``w1 [M, n, H]``, ``b1 [M, H]``, ``w2 [M, H, d]``, ``b2 [M, d]``, the gate ``gate_w
    [d, n]``, ``gate_b [d]``, the cell norm's gain ``norm_gain [n]`` (None: no cell norm) and eps,
    the candidate norm's gain ``cand_gain [d]`` (None: none) and eps, ``w_out [d, d]``, ``v [d,
    d]``, the message graph ``pad_src [N, D]``, ``pad_mask [N, D]``, ``edge_weights [N, D]`` (0 on
    padding), the activation's name."""

    w1: Tensor
    b1: Tensor
    w2: Tensor
    b2: Tensor
    gate_w: Tensor
    gate_b: Tensor
    norm_gain: Optional[Tensor]
    norm_eps: float
    cand_gain: Optional[Tensor]
    cand_eps: float
    w_out: Tensor
    v: Tensor
    pad_src: Tensor
    pad_mask: Tensor
    edge_weights: Tensor
    activation: str


def activation(name: str, x: Tensor) -> Tensor:
    """``model.activation`` (the reference's encoder ACTIVATIONS): exact GELU, ReLU, SiLU, tanh."""
    if name == "gelu":
        return torch.nn.functional.gelu(x)
    if name == "relu":
        return torch.relu(x)
    if name == "silu":
        return torch.nn.functional.silu(x)
    if name == "tanh":
        return torch.tanh(x)
    raise ValueError(f"unknown activation {name!r}")


def activation_grad(name: str, x: Tensor) -> Tensor:
    """The activation's derivative at ``x`` (state_gradient.py:174-188)."""
    if name == "gelu":
        cdf = 0.5 * (1.0 + torch.erf(x / math.sqrt(2.0)))
        return cdf + x * torch.exp(-0.5 * x * x) / math.sqrt(2.0 * math.pi)
    if name == "relu":
        return (x > 0).to(x.dtype)
    if name == "silu":
        s = torch.sigmoid(x)
        return s * (1.0 + x * (1.0 - s))
    if name == "tanh":
        return 1.0 - torch.tanh(x).square()
    raise ValueError(f"no derivative for model.activation={name!r}")


def cell_constants(w: CellWeights, dtype: torch.dtype = torch.float64) -> CellConstants:
    """The sweep's view of a cell (state_gradient.py:159-171): the state columns are the last
    ``2d`` of the cell input."""
    d = int(w.w_out.shape[0])
    n = int(w.w1.shape[1])
    return CellConstants(
        w_out=w.w_out.to(dtype),
        cand_gain=None if w.cand_gain is None else w.cand_gain.to(dtype),
        cand_eps=float(w.cand_eps),
        w2=w.w2.to(dtype),
        w1_state=w.w1[:, n - 2 * d:, :].to(dtype),
        b1=w.b1.to(dtype),
        gate_state=w.gate_w[:, n - 2 * d:].to(dtype),
        gate_bias=w.gate_b.to(dtype),
        norm_gain_state=None if w.norm_gain is None else w.norm_gain[n - 2 * d:].to(dtype),
        in_dim=n,
        v=w.v.to(dtype),
        edge_weights=w.edge_weights.to(dtype),
        pad_src=w.pad_src,
        activation=w.activation,
        pad_mask=w.pad_mask,
    )


def out_adjacency(pad_src: Tensor, pad_mask: Tensor) -> tuple[Tensor, Tensor]:
    """The message graph by source (state_sweep.py:86-109): ``out_tgt [N, D_out]`` (the targets
    of cell n's out-edges ordered by target then by the target's slot, -1 on padding) and
    ``out_edge [N, D_out]`` (the edge's index ``target * D + slot`` in the padded view)."""
    N, D = (int(n) for n in pad_src.shape)
    lists: list[list[tuple[int, int]]] = [[] for _ in range(N)]
    for target in range(N):
        for slot in range(D):
            if bool(pad_mask[target, slot]):
                lists[int(pad_src[target, slot])].append((target, target * D + slot))
    d_out = max(max((len(x) for x in lists), default=0), 1)
    out_tgt = torch.full((N, d_out), -1, dtype=torch.int64)
    out_edge = torch.zeros((N, d_out), dtype=torch.int64)
    for n, edges in enumerate(lists):
        for j, (target, flat) in enumerate(edges):
            out_tgt[n, j] = target
            out_edge[n, j] = flat
    return out_tgt, out_edge


def _by_unit(x: Tensor, units: Tensor, weight: Tensor) -> Tensor:
    """``out[p] = x[p] @ weight[units[p]]`` (state_gradient.py:191-203), slot by slot."""
    flat = x.reshape(-1, int(x.shape[-1]))
    index = units.reshape(-1)
    out = flat.new_zeros(flat.shape[0], int(weight.shape[-1]))
    for p in range(flat.shape[0]):
        out[p] = flat[p] @ weight[int(index[p])]
    return out.reshape(*x.shape[:-1], int(weight.shape[-1]))


def cell_state_vjp(dc, db, *, c, b, h_old, units, y, alpha, hidden, gate_pre, m, rms,
                   consts: CellConstants) -> tuple[Tensor, Tensor]:
    """``(dh, dvm)`` of the selected cells (state_gradient.py:288-350): the cotangent of the
    slot's own pre-round state through the cell input, and ``V^T dm``, the cotangent of the
    slot's weighted source sum (a source e of the cell receives ``a_e * dvm``)."""
    dtype = c.dtype
    d = int(c.shape[-1])
    dz = dc * (1.0 - c * c)
    weight = alpha.to(dtype)[..., None]
    if consts.cand_gain is not None:  # c = tanh(alpha * RMSNorm(y)), y = W_out F
        scaled = consts.cand_gain * (weight * dz)
        rho = torch.rsqrt(y.square().mean(dim=-1, keepdim=True) + consts.cand_eps)
        dy = rho * scaled - rho.pow(3) * y * (y * scaled).mean(dim=-1, keepdim=True)
        d_unit = dy @ consts.w_out
    else:  # c = tanh(W_out(alpha * F))
        d_unit = weight * (dz @ consts.w_out)
    hid = hidden.to(dtype)
    d_gate = db * b * (1.0 - b)
    d_act = _by_unit(d_unit, units, consts.w2.transpose(1, 2))
    d_hid = d_act * activation_grad(consts.activation, hid)
    dv = _by_unit(d_hid, units, consts.w1_state.transpose(1, 2))
    dv = dv + d_gate @ consts.gate_state
    if consts.norm_gain_state is not None:
        sigma = (d_hid * (hid - consts.b1[units])).sum(dim=-1)
        sigma = sigma + (d_gate * (gate_pre - consts.gate_bias)).sum(dim=-1)
        state = torch.cat([h_old, m], dim=-1)
        r = rms.to(dtype)[..., None]
        ds = r * (consts.norm_gain_state * dv) - (r * r / consts.in_dim) * state * sigma[..., None]
    else:
        ds = dv
    return ds[..., :d], ds[..., d:] @ consts.v


def state_gradient_backward(c, b, h_old, cells, units, valid, reset, n_cells, d_q_pre, d_q_post,
                            d_h_sel, d_h_fast, record: dict, consts: CellConstants,
                            trace: Optional[dict] = None,
                            initial: Optional[tuple[Tensor, Tensor]] = None):
    """The reverse sweep (state_gradient.py:353-474, without the row limit): ``(dc, db)``, each
    ``[B, T, K, d]``. Padded slots get exact zeros and never touch the state cotangent.
    ``trace`` receives ``A [B, T, N, d]`` and ``R [B, T, d]`` (the cotangent of the state position
    t reads, before its reset zeroes it) and ``dh``, ``dvm`` per position."""
    B, T, K, d = (int(n) for n in c.shape)
    N = int(n_cells)
    D = int(consts.pad_src.shape[1])
    n_fast = 0 if d_h_fast is None else int(d_h_fast.shape[2])
    A = c.new_zeros(B, N + 1, d)  # row N: the padded slots' dummy cell
    R = c.new_zeros(B, d)
    if initial is not None:
        A = torch.cat([initial[0].to(c.dtype), A[:, N:]], dim=1)
        R = initial[1].to(c.dtype)
    dc = torch.zeros_like(c)
    db = torch.zeros_like(b)
    zero = c.new_zeros(())
    rms = record.get("rms")
    steps: dict[str, list[Tensor]] = {"A": [], "R": [], "dh": [], "dvm": []}
    for t in range(T - 1, -1, -1):
        ok = valid[:, t, :, None]
        safe = torch.where(valid[:, t], cells[:, t], torch.zeros_like(cells[:, t]))
        index = torch.where(valid[:, t], cells[:, t], torch.full_like(cells[:, t], N))
        index = index[:, :, None].expand(B, K, d)
        if d_q_post is not None:
            R = R + d_q_post[:, t]
        if d_h_fast is not None and n_fast:
            A = torch.cat([A[:, :n_fast] + d_h_fast[:, t], A[:, n_fast:]], dim=1)
        if d_h_sel is not None:
            A = A.scatter_add(1, index, torch.where(ok, d_h_sel[:, t], zero))
        carried = A.gather(1, index)
        share = (R / N)[:, None, :]
        g = carried + share
        b_t, c_t, h_t = b[:, t], c[:, t], h_old[:, t]
        dc_t = torch.where(ok, b_t * g, zero)
        db_t = torch.where(ok, (c_t - h_t) * g, zero)
        dc[:, t] = dc_t
        db[:, t] = db_t
        dh, dvm = cell_state_vjp(
            dc_t, db_t, c=c_t, b=b_t, h_old=h_t, units=units[:, t], y=record["y"][:, t],
            alpha=record["alpha"][:, t], hidden=record["hidden"][:, t],
            gate_pre=record["gate_pre"][:, t], m=record["m"][:, t],
            rms=None if rms is None else rms[:, t], consts=consts)
        dh = torch.where(ok, dh, zero)
        dvm = torch.where(ok, dvm, zero)
        A = A.scatter(1, index, torch.where(ok, (1 - b_t) * carried - b_t * share + dh, zero))
        source = consts.pad_src[safe].reshape(B, K * D, 1).expand(B, K * D, d)
        weighted = consts.edge_weights[safe][..., None] * dvm[:, :, None, :]
        A = A.scatter_add(1, source, weighted.reshape(B, K * D, d))
        if d_q_pre is not None:
            R = R + d_q_pre[:, t]
        if trace is not None:
            steps["A"].append(A[:, :N])
            steps["R"].append(R)
            steps["dh"].append(dh)
            steps["dvm"].append(dvm)
        row = reset[:, t]
        A = A.masked_fill(row[:, None, None], 0)
        R = R.masked_fill(row[:, None], 0)
    if trace is not None:
        for key, values in steps.items():
            trace[key] = torch.stack(values[::-1], dim=1)
    return dc, db


# ---------------------------------------------------------------------------------------------
# The forward these are the backward of (the pins' float64 autograd runs through it)
# ---------------------------------------------------------------------------------------------

def cell_round(h: Tensor, extra: Tensor, cells: Tensor, units: Tensor, valid: Tensor,
               alpha: Tensor, w: CellWeights, *, src_sum: Optional[Tensor] = None,
               own: Optional[Tensor] = None):
    """The selected cells' candidate and gate from the pre-round state (state_gradient.py:
    32-43): ``h [B, N, d]``, ``extra [B, K, n - 2d]`` (the input columns that are not the state:
    u and eps), ``cells``/``units`` int64 ``[B, K]`` (cell 0, unit 0 on padded slots), ``alpha
    [B, K]``. The slot's input is ``x = [extra; h[cell]; m]`` with ``m = V (sum_e a_e h[src_e])``.
    ``src_sum``/``own`` replace the weighted source sum / the cell's own state (the VJP pin's
    leaves). Returns ``(c, b, record)`` with the record's ``y, hidden, gate_pre, m, rms`` (rms:
    the cell norm's ``1 / sqrt(mean(x^2) + eps)``)."""
    B, K = (int(n) for n in cells.shape)
    safe = torch.where(valid, cells, torch.zeros_like(cells))
    if own is None:
        own = torch.stack([h[i, safe[i]] for i in range(B)])  # [B, K, d]
    if src_sum is None:
        src = w.pad_src[safe]  # [B, K, D]
        a = w.edge_weights[safe]  # [B, K, D]
        gathered = torch.stack([h[i, src[i]] for i in range(B)])  # [B, K, D, d]
        src_sum = (a[..., None] * gathered).sum(dim=2)
    m = src_sum @ w.v.T
    x = torch.cat([extra, own, m], dim=-1)
    if w.norm_gain is not None:
        rms = torch.rsqrt(x.square().mean(dim=-1) + w.norm_eps)
        v = w.norm_gain * x * rms[..., None]
    else:
        rms = torch.ones(x.shape[:-1], dtype=x.dtype)
        v = x
    W1 = w.w1[units]  # [B, K, n, H]
    hidden = (v[..., None, :] @ W1).squeeze(-2) + w.b1[units]
    F = (activation(w.activation, hidden)[..., None, :] @ w.w2[units]).squeeze(-2) + w.b2[units]
    gate_pre = v @ w.gate_w.T + w.gate_b
    b = torch.sigmoid(gate_pre)
    y = F @ w.w_out.T
    if w.cand_gain is not None:
        rho = torch.rsqrt(y.square().mean(dim=-1, keepdim=True) + w.cand_eps)
        c = torch.tanh(alpha[..., None] * (w.cand_gain * y * rho))
    else:
        c = torch.tanh(alpha[..., None] * y)
    return c, b, {"y": y, "hidden": hidden, "gate_pre": gate_pre, "m": m, "rms": rms}


def window_outputs(h0: Tensor, extra: Tensor, cells: Tensor, units: Tensor, valid: Tensor,
                   alpha: Tensor, reset: Tensor, w: CellWeights, n_read: int = 0,
                   probe_c: Optional[Tensor] = None, probe_b: Optional[Tensor] = None):
    """A window of rounds (the split window's forward with the state read live): at every
    position the row resets if asked (h = 0), the selected cells read the pre-round state
    (``cell_round``), and the gated update ``h[cell] = (1 - b) h[cell] + b c`` writes them; ``q``
    is the mean of h over the cells. ``probe_c``/``probe_b [B, T, K, d]`` are added to ``c``/``b``
    where they are used, so autograd's derivative with respect to them is the total ``dL/dc``,
    ``dL/db`` of the sweep. Returns the outputs (``q_pre, q_post [B, T, d]``, ``h_sel [B, T, K,
    d]`` (zero on padded slots), ``h_fast [B, T, n_read, d]``) and the record the sweep reads (``c, b, h_old`` and the
    cell's values, ``[B, T, K, ...]``)."""
    B, T, K = (int(n) for n in cells.shape)
    N, d = (int(n) for n in h0.shape[1:])
    h = h0
    outs = {"q_pre": [], "q_post": [], "h_sel": [], "h_fast": []}
    rec = {k: [] for k in ("c", "b", "h_old", "y", "hidden", "gate_pre", "m", "rms")}
    for t in range(T):
        h = torch.where(reset[:, t, None, None], torch.zeros_like(h), h)
        outs["q_pre"].append(h.mean(dim=1))
        c, b, record = cell_round(h, extra[:, t], cells[:, t], units[:, t], valid[:, t],
                                  alpha[:, t], w)
        safe = torch.where(valid[:, t], cells[:, t], torch.zeros_like(cells[:, t]))
        h_old = torch.stack([h[i, safe[i]] for i in range(B)])
        rec["c"].append(c)
        rec["b"].append(b)
        rec["h_old"].append(h_old)
        for key, value in record.items():
            rec[key].append(value)
        if probe_c is not None:
            c = c + probe_c[:, t]
        if probe_b is not None:
            b = b + probe_b[:, t]
        new = (1 - b) * h_old + b * c
        rows = []
        for i in range(B):
            row = h[i]
            for k in range(K):
                if bool(valid[i, t, k]):
                    cell = int(cells[i, t, k])
                    row = torch.cat([row[:cell], new[i, k][None], row[cell + 1:]], dim=0)
            rows.append(row)
        h = torch.stack(rows)
        outs["q_post"].append(h.mean(dim=1))
        sel = torch.stack([h[i, safe[i]] for i in range(B)])
        outs["h_sel"].append(torch.where(valid[:, t, :, None], sel, torch.zeros_like(sel)))
        outs["h_fast"].append(h[:, :n_read])
    return ({k: torch.stack(v, dim=1) for k, v in outs.items()},
            {k: torch.stack(v, dim=1) for k, v in rec.items()})
