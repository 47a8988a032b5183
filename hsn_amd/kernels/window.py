"""The reference's window-kernel module on MI355X: the same names, signatures, custom ops and
decline convention as ``hsn.kernels.window`` (python/hsn/kernels/window.py:56-1143), backed by
``libhsn_amd.so`` (``include/hsn_window.h``) instead of a CUDA fatbin.

Convention, as there: a wrapper returns ``None`` for inputs it does not take (dtype, device,
shape) so the caller keeps its own path; misuse raises; a missing or stale library raises on
:func:`prepare`. Beyond the reference: no 48 KiB shared-memory ceiling (the recurrence and the
update take any ``N`` whose state slice fits the 160 KiB LDS), the carried-state outputs
(:func:`recurrence_backward_carried`), bf16 storage, and N up to 4096 in the router.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch
from torch import Tensor
from torch.utils._python_dispatch import _get_current_dispatch_mode

from .. import _lib
from .._lib import DTYPE_BF16, DTYPE_F32, call, ptr, stream_of
from ..state import CellGraphState
from ..window import check_reserved, rms_scratch_bytes

_prepared: set[int] = set()

def available() -> bool:
    """Library presence and freshness only: never initialises the GPU."""
    return _lib.available()


def prepare(device: int = 0) -> None:
    """Load the library for ``device`` (idempotent); raises when it is missing or stale."""
    _lib.library()
    _prepared.add(int(device))


def prepared(device: torch.device) -> bool:
    return device.type == "cuda" and (device.index or 0) in _prepared


# --------------------------------------------------------------------------------------------
# the backward recurrence (reference window.py:108-192)
# --------------------------------------------------------------------------------------------


def _recurrence(c, b, h_old, cells, valid, reset, n_cells, d_q_pre, d_q_post, d_h_sel, d_h_T,
                d_q_T, carried):
    if not prepared(c.device) or c.dtype != torch.float32 or cells.dtype != torch.int64:
        return None
    for cot in (d_q_pre, d_q_post, d_h_sel, d_h_T, d_q_T):
        if cot is not None and cot.dtype != torch.float32:
            return None
    B, T, K, d = (int(n) for n in c.shape)
    N = int(n_cells)
    if _lib.unsupported(_lib.OP_RECURRENCE, B, T, N, d, K) is not None:
        return None
    dc = torch.empty(B, T, K, d, dtype=torch.float32, device=c.device)
    db = torch.empty_like(dc)
    d_h0 = torch.empty(B, N, d, dtype=torch.float32, device=c.device) if carried else None
    d_q0 = torch.empty(B, d, dtype=torch.float32, device=c.device) if carried else None
    cont = lambda t: None if t is None else t.contiguous()  # noqa: E731
    args = [cont(t) for t in (c, b, h_old, cells, valid, reset, d_q_pre, d_q_post, d_h_sel,
                              d_h_T, d_q_T)]
    call("hsn_win_recurrence", *(ptr(t) for t in args), ptr(dc), ptr(db), ptr(d_h0), ptr(d_q0),
         B, T, K, d, N, stream_of(c.device))
    return (dc, db, d_h0, d_q0) if carried else (dc, db)


def recurrence_backward(c: Tensor, b: Tensor, h_old: Tensor, cells: Tensor, valid: Tensor,
                        reset: Tensor, n_cells: int, d_q_pre: Optional[Tensor],
                        d_q_post: Optional[Tensor], d_h_sel: Optional[Tensor]):
    """``hsn.train.split.recurrence_backward`` (python/hsn/train/split.py:128-174) as one
    launch: ``(dc, db)`` or ``None`` when the inputs are not fp32 / int64 on a prepared device.
    The reference's kernel declines above 48 KiB of shared memory; this one takes any N whose
    ``[N, S]`` cotangent slice fits the LDS."""
    return _recurrence(c, b, h_old, cells, valid, reset, n_cells, d_q_pre, d_q_post, d_h_sel,
                       None, None, False)


def recurrence_backward_carried(c, b, h_old, cells, valid, reset, n_cells, d_q_pre, d_q_post,
                                d_h_sel, d_h_T=None, d_q_T=None):
    """:func:`recurrence_backward` with the carried state: ``d_h_T [B,N,d]`` / ``d_q_T [B,d]``
    seed the cotangents (the next window's start-state gradient) and the result adds
    ``d_h0, d_q0``, the gradient into this window's start state: ``(dc, db, d_h0, d_q0)``."""
    return _recurrence(c, b, h_old, cells, valid, reset, n_cells, d_q_pre, d_q_post, d_h_sel,
                       d_h_T, d_q_T, True)


def dense_recurrence_backward(c: Tensor, b: Tensor, h_old: Tensor, reset: Tensor, n_cells: int,
                              d_q_pre: Optional[Tensor], d_q_post: Optional[Tensor]):
    """``hsn.train.split.dense_recurrence_backward`` (split.py:177-209) as one launch, or
    ``None`` for non-fp32 inputs or an unprepared device."""
    if not prepared(c.device) or c.dtype != torch.float32:
        return None
    Bd, T, N, d = (int(n) for n in c.shape)
    if N != int(n_cells):
        return None
    for cot in (d_q_pre, d_q_post):
        if cot is not None and cot.dtype != torch.float32:
            return None
    dc = torch.empty(Bd, T, N, d, dtype=torch.float32, device=c.device)
    db = torch.empty_like(dc)
    cont = lambda t: None if t is None else t.contiguous()  # noqa: E731
    call("hsn_win_recurrence_dense", ptr(cont(c)), ptr(cont(b)), ptr(cont(h_old)),
         ptr(cont(reset)), ptr(cont(d_q_pre)), ptr(cont(d_q_post)), ptr(dc), ptr(db), Bd, T, N, d,
         stream_of(c.device))
    return dc, db


# --------------------------------------------------------------------------------------------
# the per-position decision (reference window.py:356-602)
# --------------------------------------------------------------------------------------------


def _io(t: Tensor) -> int:
    return DTYPE_BF16 if t.dtype == torch.bfloat16 else DTYPE_F32


def _launch_select(logits, width, n_units, age, cost, cells, units, valid, theta, refreshed, t,
                   n_out, n_age, B, N, k, age_max, probes, lambda_cost, cell_overhead,
                   shared_cost, limit, reserved, reserved_units):
    check_reserved(int(k), reserved, bool(reserved_units))
    call("hsn_win_select", ptr(logits), _io(logits), int(width), ptr(age) if probes else None,
         ptr(cost), ptr(cells), ptr(units), ptr(valid), ptr(theta), ptr(refreshed), B, N,
         int(n_units), int(k), int(t), int(n_out), int(n_age), int(age_max), int(bool(probes)),
         float(lambda_cost), float(cell_overhead), float(shared_cost), float(limit),
         int(reserved), int(bool(reserved_units)), stream_of(logits.device))


@torch.library.custom_op("hsn::window_select", mutates_args=(), device_types="cuda")
def select_op(logits: Tensor, age: Tensor, cost: Tensor, k: int, age_max: int, probes: bool,
              lambda_cost: float, cell_overhead: float, shared_cost: float, limit: float,
              reserved: int = 0, reserved_units: bool = False
              ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """One position's decision ``(cells, units, valid, theta, refreshed)`` from ``logits
    [B,N,M]`` (fp32 or bf16), ``age [B,N]`` int64, ``cost [M]`` fp32 (reference
    window.py:233-283)."""
    B, N, M = (int(n) for n in logits.shape)
    dev = logits.device
    cells = torch.empty((B, k), dtype=torch.int64, device=dev)
    units = torch.empty((B, k), dtype=torch.int64, device=dev)
    valid = torch.empty((B, k), dtype=torch.bool, device=dev)
    theta = torch.empty((B,), dtype=torch.float32, device=dev)
    refreshed = torch.empty((B, k), dtype=torch.bool, device=dev)
    _launch_select(logits, M, M, age, cost, cells, units, valid, theta, refreshed, 0, 1, 1, B, N,
                   k, age_max, probes, lambda_cost, cell_overhead, shared_cost, limit, reserved,
                   reserved_units)
    return cells, units, valid, theta, refreshed


@select_op.register_fake
def _select_fake(logits, age, cost, k, age_max, probes, lambda_cost, cell_overhead, shared_cost,
                 limit, reserved=0, reserved_units=False):
    B = logits.shape[0]
    return (logits.new_empty((B, k), dtype=torch.int64), logits.new_empty((B, k), dtype=torch.int64),
            logits.new_empty((B, k), dtype=torch.bool), logits.new_empty((B,), dtype=torch.float32),
            logits.new_empty((B, k), dtype=torch.bool))


@torch.library.custom_op("hsn::window_select_tape",
                         mutates_args=("cells", "units", "valid", "theta", "refreshed"),
                         device_types="cuda")
def select_tape_op(logits: Tensor, age: Tensor, cost: Tensor, cells: Tensor, units: Tensor,
                   valid: Tensor, theta: Tensor, refreshed: Tensor, t: int, age_max: int,
                   probes: bool, lambda_cost: float, cell_overhead: float, shared_cost: float,
                   limit: float, reserved: int = 0, reserved_units: bool = False) -> None:
    """:func:`select_op` into record ``t`` of the decision tape (``[B, n, K]``, ``theta
    [B, n]``) from the ages ``age[:, t]`` (``[B, n + 1, N]``) (reference window.py:356-420)."""
    B, N, M = (int(n) for n in logits.shape)
    n, k = int(cells.shape[1]), int(cells.shape[2])
    _launch_select(logits, M, M, age, cost, cells, units, valid, theta, refreshed, t, n,
                   int(age.shape[1]), B, N, k, age_max, probes, lambda_cost, cell_overhead,
                   shared_cost, limit, reserved, reserved_units)


@select_tape_op.register_fake
def _select_tape_fake(logits, age, cost, cells, units, valid, theta, refreshed, t, age_max, probes,
                      lambda_cost, cell_overhead, shared_cost, limit, reserved=0,
                      reserved_units=False):
    return None


@torch.library.custom_op("hsn::window_select_fold",
                         mutates_args=("cells", "units", "valid", "theta", "refreshed"),
                         device_types="cuda")
def select_fold_op(scored: Tensor, age: Tensor, cost: Tensor, cells: Tensor, units: Tensor,
                   valid: Tensor, theta: Tensor, refreshed: Tensor, t: int, n_units: int,
                   age_max: int, probes: bool, lambda_cost: float, cell_overhead: float,
                   shared_cost: float, limit: float, reserved: int = 0,
                   reserved_units: bool = False) -> None:
    """:func:`select_tape_op` on the scorer's product as it is: ``scored [B*N, W]`` (fp32 or
    bf16) holds the logits in its first ``n_units`` columns, read in place (reference
    window.py:421-486)."""
    rows, width = int(scored.shape[0]), int(scored.shape[1])
    B = int(cells.shape[0])
    N = rows // B
    n, k = int(cells.shape[1]), int(cells.shape[2])
    _launch_select(scored, width, n_units, age, cost, cells, units, valid, theta, refreshed, t, n,
                   int(age.shape[1]), B, N, k, age_max, probes, lambda_cost, cell_overhead,
                   shared_cost, limit, reserved, reserved_units)


@select_fold_op.register_fake
def _select_fold_fake(scored, age, cost, cells, units, valid, theta, refreshed, t, n_units,
                      age_max, probes, lambda_cost, cell_overhead, shared_cost, limit, reserved=0,
                      reserved_units=False):
    return None


def select_unsupported(n_cells: int, k: int, n_units: int = 1) -> Optional[str]:
    """Why :func:`select` cannot take a model of this shape (``None``: it can), by the
    library's own checks (reference window.py:557-565)."""
    why = _lib.unsupported(_lib.OP_ROUTE, 1, 1, int(n_cells), 1, int(k))
    return None if why is None else f"model.n_cells={n_cells}, k_select={k}: {why}"


def select(logits: Tensor, age: Tensor, cost_table: Tensor, *, k: int, age_max: int, probes: bool,
           lambda_cost: float, cell_overhead: float, shared_cost: float, limit: float,
           reserved: int = 0, reserved_units: bool = False):
    """``Router.select`` for the forward sweep (mode ``topk``, the hard decision, the refresh
    probes when ``probes``): ``(cells, units, valid, theta, refreshed)`` with the router's
    values and tie rules (reference window.py:568-602). ``limit = budget * (1 + slack)``."""
    logits = logits if logits.dtype in (torch.float32, torch.bfloat16) else logits.float()
    return select_op(logits.contiguous(), age.contiguous(), cost_table.to(torch.float32).contiguous(),
                     k, age_max, probes, lambda_cost, cell_overhead, shared_cost, limit, reserved,
                     reserved_units)


def select_tape(logits, tape_age, cost_table, cells, units, valid, theta, refreshed, *, t, age_max,
                probes, lambda_cost, cell_overhead, shared_cost, limit, reserved=0,
                reserved_units=False) -> None:
    """:func:`select` for position ``t``, written into record ``t`` of the decision tape."""
    logits = logits if logits.dtype in (torch.float32, torch.bfloat16) else logits.float()
    select_tape_op(logits.contiguous(), tape_age, cost_table.to(torch.float32).contiguous(), cells,
                   units, valid, theta, refreshed, t, age_max, probes, lambda_cost, cell_overhead,
                   shared_cost, limit, reserved, reserved_units)


def select_fold(scored, tape_age, cost_table, cells, units, valid, theta, refreshed, *, t, n_units,
                age_max, probes, lambda_cost, cell_overhead, shared_cost, limit, reserved=0,
                reserved_units=False) -> None:
    """:func:`select_tape` reading the logits in place from a wider product."""
    select_fold_op(scored, tape_age, cost_table.to(torch.float32).contiguous(), cells, units,
                   valid, theta, refreshed, t, n_units, age_max, probes, lambda_cost,
                   cell_overhead, shared_cost, limit, reserved, reserved_units)


# --------------------------------------------------------------------------------------------
# the per-position end of round (reference window.py:605-1004)
# --------------------------------------------------------------------------------------------


def _launch_update(y, gate, cand_w, cand_norm, cand_eps, h, q, age, pos, cells, valid, h_next,
                   q_next, age_next, pos_next, h_sel, h_max, reset, q_post, B, N, d, K, t, n_state,
                   n_slot, t_out):
    scratch = None
    if cand_norm:
        elem = 4 if y.dtype == torch.float32 else 2
        scratch = torch.empty(rms_scratch_bytes(B * K, d, elem), dtype=torch.uint8,
                              device=y.device)
    call("hsn_win_cell_update", ptr(y), ptr(gate), _io(y), ptr(cand_w) if cand_norm else None,
         int(bool(cand_norm)), float(cand_eps), ptr(scratch), ptr(h), ptr(q), ptr(age), ptr(pos),
         ptr(cells), ptr(valid), ptr(h_next), ptr(q_next), ptr(age_next), ptr(pos_next),
         ptr(h_sel), ptr(h_max), ptr(reset), ptr(q_post), B, N, d, K, t, n_state, n_slot, t_out,
         stream_of(y.device))


@torch.library.custom_op("hsn::window_cell_update", mutates_args=(), device_types="cuda")
def cell_update_op(y: Tensor, gate: Tensor, h: Tensor, q: Tensor, age: Tensor, pos: Tensor,
                   cells: Tensor, valid: Tensor, cand_w: Tensor, cand_norm: bool, cand_eps: float
                   ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """The end of one position's round: ``(h, q, age, pos, h_sel, h_max)`` (reference
    window.py:605-659). ``y, gate [B,K,d]`` fp32 (or bf16); state fp32 / int64; cells int64."""
    B, N, d = (int(n) for n in h.shape)
    K = int(cells.shape[1])
    h_next = torch.empty_like(h)
    q_next = torch.empty_like(q)
    age_next = torch.empty_like(age)
    pos_next = torch.empty_like(pos)
    h_sel = h.new_empty((B, K, d))
    h_max = h.new_empty((B,))
    _launch_update(y, gate, cand_w, cand_norm, cand_eps, h, q, age, pos, cells, valid, h_next,
                   q_next, age_next, pos_next, h_sel, h_max, None, None, B, N, d, K, 0, 1, 1, 0)
    return h_next, q_next, age_next, pos_next, h_sel, h_max


@cell_update_op.register_fake
def _cell_update_fake(y, gate, h, q, age, pos, cells, valid, cand_w, cand_norm, cand_eps):
    return (torch.empty_like(h), torch.empty_like(q), torch.empty_like(age), torch.empty_like(pos),
            h.new_empty((*cells.shape, h.shape[2])), h.new_empty((h.shape[0],)))


@torch.library.custom_op("hsn::window_update_tape",
                         mutates_args=("tape_h", "tape_q", "tape_age", "tape_hsel", "h_max", "qs"),
                         device_types="cuda")
def update_tape_op(y: Tensor, gate: Tensor, tape_h: Tensor, tape_q: Tensor, tape_age: Tensor,
                   cells: Tensor, valid: Tensor, cand_w: Tensor, reset: Tensor, tape_hsel: Tensor,
                   h_max: Tensor, qs: Tensor, t: int, cand_norm: bool, cand_eps: float) -> None:
    """:func:`cell_update_op` on a tape (reference window.py:682-741): reads record ``t`` of
    ``tape_h [B,n+1,N,d]``, ``tape_q [B,n+1,d]``, ``tape_age [B,n+1,N]`` and of the decision
    ``[B,n,K]``; writes record ``t+1`` of the state tape (zeroed on rows whose ``reset[:, t+1]``
    is set, never for the last record) and record ``t`` of ``tape_hsel [B,n,K,d]``,
    ``h_max [B,n]`` and ``qs [B,n,d]`` (the summary after the position, before that reset)."""
    B, n_state, N, d = (int(n) for n in tape_h.shape)
    n, K = int(cells.shape[1]), int(cells.shape[2])
    _launch_update(y, gate, cand_w, cand_norm, cand_eps, tape_h, tape_q, tape_age, None, cells,
                   valid, tape_h, tape_q, tape_age, None, tape_hsel, h_max, reset, qs, B, N, d, K, t,
                   n_state, n, t + 1)


@update_tape_op.register_fake
def _update_tape_fake(y, gate, tape_h, tape_q, tape_age, cells, valid, cand_w, reset, tape_hsel,
                      h_max, qs, t, cand_norm, cand_eps):
    return None


@torch.library.custom_op(
    "hsn::window_update_fold",
    mutates_args=("tape_h", "tape_q", "tape_age", "tape_hsel", "h_max", "qs", "x"),
    device_types="cuda")
def update_fold_op(y: Tensor, gate: Tensor, tape_h: Tensor, tape_q: Tensor, tape_age: Tensor,
                   cells: Tensor, valid: Tensor, cand_w: Tensor, reset: Tensor, tape_hsel: Tensor,
                   h_max: Tensor, qs: Tensor, x: Tensor, z: Tensor, context: Tensor, t: int,
                   cand_norm: bool, cand_eps: float, n_fast: int = 0) -> None:
    """:func:`update_tape_op` on the round's products as they are (reference window.py:765-853):
    ``y [B,K,d]`` and ``gate [B*K,d]`` (a strided view of a wider product allowed) in fp32 or
    bf16, widened to fp32 before the round (exact), then record ``t + 1`` of
    ``x [n,B,d_z+d+d_c(+d)]`` (when ``t + 1 < n``) becomes ``[z; q; context(; f)]`` of position
    ``t + 1`` (``hsn_win_fold_row``): ``q`` after the round and the next reset, ``f`` the mean of
    cells ``0 .. n_fast-1`` of that record's state, each value rounded to ``x``'s dtype."""
    B, n_state, N, d = (int(n) for n in tape_h.shape)
    n, K = int(cells.shape[1]), int(cells.shape[2])
    d_z, d_c = int(z.shape[2]), int(context.shape[2])
    if tuple(x.shape) != (n, B, d_z + d + d_c + (d if n_fast else 0)):
        raise ValueError(f"x must be [n, B, d_z + d + d_c (+ d)], got {tuple(x.shape)}")
    if not 0 <= n_fast <= N:
        raise ValueError(f"n_fast must lie in [0, {N}], got {n_fast}")
    if not x.is_contiguous() or not z.is_contiguous() or not context.is_contiguous():
        raise ValueError("x, z and context must be contiguous")
    y32 = y.float().contiguous()
    gate32 = gate.float().reshape(B, K, d).contiguous()
    _launch_update(y32, gate32, cand_w, cand_norm, cand_eps, tape_h, tape_q, tape_age, None, cells,
                   valid, tape_h, tape_q, tape_age, None, tape_hsel, h_max, reset, qs, B, N, d, K, t,
                   n_state, n, t + 1)
    if t + 1 < n:
        call("hsn_win_fold_row", ptr(x), _io(x), ptr(z), _io(z), d_z, ptr(context), _io(context),
             d_c, ptr(tape_q), ptr(tape_h), int(n_fast), B, N, d, n, n_state, t + 1,
             stream_of(x.device))


@update_fold_op.register_fake
def _update_fold_fake(y, gate, tape_h, tape_q, tape_age, cells, valid, cand_w, reset, tape_hsel,
                      h_max, qs, x, z, context, t, cand_norm, cand_eps, n_fast=0):
    return None


def cell_update_unsupported(n_cells: int, d: int, k: int) -> Optional[str]:
    """Why :func:`cell_update` cannot take a model of this shape (``None``: it can), by the
    library's own geometry (reference window.py:626-640)."""
    why = _lib.unsupported(_lib.OP_CELL_UPDATE, 1, 1, int(n_cells), int(d), int(k))
    return None if why is None else f"model.n_cells={n_cells}, d={d}, k_select={k}: {why}"


def _cand(cell):
    cand_norm = getattr(cell, "cand_norm_kind", "none") != "none"
    if cand_norm:
        w = cell.cand_norm.weight
        eps = float(getattr(cell.cand_norm, "eps", None) or 0.0)
    else:
        w = cell.norm.weight
        eps = 0.0
    return cand_norm, w.detach().to(torch.float32).contiguous(), eps


def cell_update(cell, y: Tensor, gate: Tensor, state: CellGraphState, cells: Tensor,
                valid: Tensor):
    """The round of one position from its products: candidate (norm, tanh), the gate's
    sigmoid, the gated delta update and the tick as one launch. Returns the state after the
    position, the slots' cells after the update ``[B,K,d]`` (cell 0 on padded slots) and each
    row's ``max |h|`` ``[B]`` (reference window.py:900-931)."""
    cand_norm, w, eps = _cand(cell)
    h, q, age, pos, h_sel, h_max = cell_update_op(
        y.contiguous(), gate.contiguous(), state.h.contiguous(), state.q.contiguous(),
        state.age.contiguous(), state.pos.contiguous(), cells.contiguous(), valid.contiguous(), w,
        cand_norm, eps)
    return CellGraphState.make(h=h, q=q, age=age, pos=pos), h_sel, h_max


def update_fold(cell, y, gate, tape_h, tape_q, tape_age, cells, valid, reset, tape_hsel, h_max, qs,
                x, z, context, *, t: int, n_fast: int = 0) -> None:
    """:func:`update_tape` from the round's products as they are, with the next position's
    input of the first product written into ``x`` (:func:`update_fold_op`; reference
    window.py:1099-1143)."""
    cand_norm, w, eps = _cand(cell)
    update_fold_op(y, gate, tape_h, tape_q, tape_age, cells, valid, w, reset, tape_hsel, h_max, qs,
                   x, z, context, t, cand_norm, eps, n_fast)


def update_tape(cell, y, gate, tape_h, tape_q, tape_age, cells, valid, reset, tape_hsel, h_max, qs,
                *, t: int) -> None:
    """:func:`cell_update` for position ``t`` on its tapes, in place (reference
    window.py:967-1004)."""
    cand_norm, w, eps = _cand(cell)
    update_tape_op(y.contiguous(), gate.contiguous(), tape_h, tape_q, tape_age, cells, valid, w,
                   reset, tape_hsel, h_max, qs, t, cand_norm, eps)


# --------------------------------------------------------------------------------------------
# the fused cell round (reference window.py:195-330, 1007-1048; include/hsn_round.h)
# --------------------------------------------------------------------------------------------

_ROUND_POINTERS = ("u", "eps", "h", "q", "age", "cells", "units", "valid", "alpha", "V", "edge_w",
                   "pad_src", "norm_w", "gate_w", "gate_b", "W1", "b1", "W2", "b2", "W_out",
                   "cand_w", "work", "h_new", "q_new", "age_new", "h_sel")


class _Round(ctypes.Structure):
    """``hsn_cell_round`` (include/hsn_round.h), field for field."""

    _fields_ = ([(name, ctypes.c_int32) for name in ("B", "N", "d", "K", "M", "H", "D",
                                                     "cand_norm")]
                + [("norm_eps", ctypes.c_float), ("cand_eps", ctypes.c_float)]
                + [(name, ctypes.c_void_p) for name in _ROUND_POINTERS])


def _round_struct(B, N, d, K, M, H, D, cand_norm, norm_eps, cand_eps, **pointers) -> _Round:
    return _Round(B, N, d, K, M, H, D, int(bool(cand_norm)), float(norm_eps), float(cand_eps),
                  *[pointers.get(name) for name in _ROUND_POINTERS])


_round_work: dict[tuple, int] = {}  # scratch bytes by (B, K, d, H): host arithmetic only
#: The operands' dtypes and shapes by (B, N, d, K, M, H, D), in the struct's pointer order.
_round_specs: dict[tuple, tuple] = {}
#: Byte offset of the struct's first pointer field; the operands' pointers are the next twenty.
_ROUND_FIRST = _Round.u.offset
_ROUND_OPERANDS = _ROUND_POINTERS[:20]


def _round_unsupported(B, N, d, K, M, H, D, cand_norm) -> Optional[str]:
    """The library's own verdict on a shape (``hsn_win_cell_round_check`` on placeholder
    pointers: the check reads no memory)."""
    s = _round_struct(B, N, d, K, M, H, D, cand_norm, 0.0, 0.0,
                      **{name: 256 for name in _ROUND_POINTERS})
    lib = _lib.library()
    if lib.hsn_win_cell_round_check(ctypes.byref(s)) == _lib.HSN_OK:
        return None
    return lib.hsn_win_last_error().decode(errors="replace")


def cell_round_error(cell) -> Optional[str]:
    """Why the fused cell round cannot run this cell, or ``None`` when it can (reference
    window.py:202-230): the same model switches, then the library's geometry (``d`` a multiple
    of 4 up to 256, at most 255 units; the slot count is checked per call)."""
    d = int(cell.d)
    if getattr(cell, "ablate_shared_u", False):
        return ("model.ablate_shared_u: the fused round builds the 4d cell input [u; eps; h; m] "
                "in its kernel")
    if not available():
        return "the HIP library is not built (hsn_amd.build.build())"
    if getattr(cell, "cell_norm", "rms") != "rms":
        return f"model.cell_norm={cell.cell_norm!r}: the fused round implements the RMS norm"
    if cell.units.activation_name != "gelu":
        return (f"model.activation={cell.units.activation_name!r}: the fused round implements "
                "GELU")
    if getattr(cell, "disabled_cells", None):
        return "model.disabled_cells is a test hook of the native round"
    if cell.V.weight.dtype != torch.float32:
        return f"fp32 master weights only, got {cell.V.weight.dtype}"
    pad_src = cell.graph._pad_src
    N, D = int(pad_src.shape[0]), int(pad_src.shape[1])
    M, _, H = (int(n) for n in cell.units.W1.shape)
    why = _round_unsupported(1, N, d, 1, M, H, D, getattr(cell, "cand_norm_kind", "none") != "none")
    return None if why is None else f"model.d={d}, model.hidden={H}, model.n_units={M}: {why}"


def _need(name: str, t: Tensor, dtype: torch.dtype, shape: tuple, index: int) -> None:
    if t.dtype is not dtype or t.shape != shape or t.get_device() != index:
        raise ValueError(f"cell round: {name} must be {dtype} {list(shape)} on cuda:{index}, "
                         f"got {t.dtype} {list(t.shape)} on {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"cell round: {name} must be contiguous")


def _cell_round_run(u: Tensor, eps: Tensor, h: Tensor, q: Tensor, age: Tensor, cells: Tensor,
                    units: Tensor, valid: Tensor, alpha: Tensor, V: Tensor, edge_w: Tensor,
                    pad_src: Tensor, norm_w: Tensor, gate_w: Tensor, gate_b: Tensor, W1: Tensor,
                    b1: Tensor, W2: Tensor, b2: Tensor, W_out: Tensor, cand_w: Tensor,
                    cand_norm: bool, norm_eps: float, cand_eps: float
                    ) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """The op's body: the checks, the outputs and the call of ``hsn_win_cell_round``. Eager
    callers outside a compiled region call it directly (:func:`cell_round`): the custom op's
    dispatch adds its Python autograd and aliasing layers to every position."""
    B, N, d = (int(n) for n in h.shape)
    K = int(cells.shape[1])
    M, n_in, H = (int(n) for n in W1.shape)
    D = int(edge_w.shape[1])
    dev = h.device
    if not h.is_cuda:
        raise ValueError(f"cell round: h on {dev}; the round takes tensors on one ROCm device")
    index = h.get_device()
    f32, i64 = torch.float32, torch.int64
    operands = (u, eps, h, q, age, cells, units, valid, alpha, V, edge_w, pad_src, norm_w, gate_w,
                gate_b, W1, b1, W2, b2, W_out)
    skey = (B, N, d, K, M, H, D)
    specs = _round_specs.get(skey)
    if specs is None:
        shapes = ((B, d), (B, d), (B, N, d), (B, d), (B, N), (B, K), (B, K), (B, K), (B, K), (d, d),
                  (N, D), (N, D), (4 * d,), (d, 4 * d), (d,), (M, 4 * d, H), (M, H), (M, H, d),
                  (M, d), (d, d))
        dtypes = (f32, f32, f32, f32, i64, i64, i64, torch.bool, f32, f32, f32, i64, f32, f32, f32,
                  f32, f32, f32, f32, f32)
        specs = _round_specs[skey] = (dtypes, shapes)
    # the checks and the pointers in one native call where the host helper is built; a mismatch
    # (or no helper) takes the checks one by one, which name it
    native = _lib.host_tables()
    table = native.tensor_table(operands, specs[0], specs[1], index) if native is not None else None
    if not isinstance(table, bytearray):
        for name, t, dtype, shape in zip(_ROUND_OPERANDS, operands, *specs):
            _need(name, t, dtype, shape, index)
        table = bytearray((ctypes.c_int64 * 20)(*[t.data_ptr() for t in operands]))
    if cand_norm:  # otherwise unused (the reference passes the cell norm's gain in its place)
        _need("cand_w", cand_w, f32, (d,), index)
    h_new = torch.empty_like(h)
    q_new = torch.empty_like(q)
    age_new = torch.empty_like(age)
    h_sel = h.new_empty((B, K, d))
    key = (B, K, d, H)
    nbytes = _round_work.get(key)
    if nbytes is None:
        probe = _round_struct(B, N, d, K, M, H, D, cand_norm, norm_eps, cand_eps)
        out = ctypes.c_int64(0)
        call("hsn_win_cell_round_workspace", ctypes.byref(probe), ctypes.byref(out))
        nbytes = _round_work[key] = int(out.value)
    work = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    s = _Round(B, N, d, K, M, H, D, int(bool(cand_norm)), float(norm_eps), float(cand_eps))
    ctypes.memmove(ctypes.addressof(s) + _ROUND_FIRST, bytes(table), 8 * 20)  # u .. W_out
    if not D:  # no edges: no edge weights or sources
        s.edge_w = None
        s.pad_src = None
    s.cand_w = cand_w.data_ptr() if cand_norm else None
    s.work = work.data_ptr()
    s.h_new = h_new.data_ptr()
    s.q_new = q_new.data_ptr()
    s.age_new = age_new.data_ptr()
    s.h_sel = h_sel.data_ptr()
    call("hsn_win_cell_round", ctypes.byref(s), stream_of(dev))
    return h_new, q_new, age_new, h_sel


@torch.library.custom_op("hsn::window_cell_round", mutates_args=(), device_types="cuda")
def cell_round_op(u: Tensor, eps: Tensor, h: Tensor, q: Tensor, age: Tensor, cells: Tensor,
                  units: Tensor, valid: Tensor, alpha: Tensor, V: Tensor, edge_w: Tensor,
                  pad_src: Tensor, norm_w: Tensor, gate_w: Tensor, gate_b: Tensor, W1: Tensor,
                  b1: Tensor, W2: Tensor, b2: Tensor, W_out: Tensor, cand_w: Tensor,
                  cand_norm: bool, norm_eps: float, cand_eps: float
                  ) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """The sparse round and the tick, forward only: ``(h_new, q_new, age_new, h_sel)``
    (reference window.py:233-330; ``hsn_win_cell_round``). Contiguous fp32 / int64 / bool
    tensors on one device, as the reference's op takes them; not differentiable."""
    return _cell_round_run(u, eps, h, q, age, cells, units, valid, alpha, V, edge_w, pad_src,
                           norm_w, gate_w, gate_b, W1, b1, W2, b2, W_out, cand_w, cand_norm,
                           norm_eps, cand_eps)


@cell_round_op.register_fake
def _cell_round_fake(u, eps, h, q, age, cells, units, valid, alpha, V, edge_w, pad_src, norm_w,
                     gate_w, gate_b, W1, b1, W2, b2, W_out, cand_w, cand_norm, norm_eps, cand_eps):
    return (torch.empty_like(h), torch.empty_like(q), torch.empty_like(age),
            h.new_empty((*cells.shape, h.shape[2])))


def cell_round(cell, u: Tensor, eps: Tensor, state: CellGraphState, cells: Tensor, units: Tensor,
               valid: Tensor, edge_weights: Tensor):
    """``PDGCell.step_sparse`` and the tick of one position as the fused op: the state after the
    position and the selected slots' updated states ``[B, K, d]`` (cell 0 on padded slots).
    ``cells`` / ``units`` / ``valid`` are a hard decision (``alpha`` is 1 on its valid slots),
    ``edge_weights`` the window's padded edge weights. fp32 state, no autograd (reference
    window.py:1007-1048)."""
    cand_norm = getattr(cell, "cand_norm_kind", "none") != "none"
    norm_w = cell.norm.weight
    # eagerly the op's body itself; the registered op where anything traces (a compiled region,
    # a dispatch mode, fake or functional tensors)
    traced = (torch.compiler.is_compiling() or _get_current_dispatch_mode() is not None
              or type(state.h) is not Tensor)
    run = cell_round_op if traced else _cell_round_run
    with torch.no_grad():
        h_new, q_new, age_new, h_sel = run(
            u.contiguous(), eps.contiguous(), state.h.contiguous(), state.q.contiguous(),
            state.age.contiguous(), cells.contiguous(), units.contiguous(), valid.contiguous(),
            valid.to(torch.float32).contiguous(), cell.V.weight.detach(),
            edge_weights.to(torch.float32).contiguous(), cell.graph._pad_src,
            norm_w.detach(), cell.gate.weight.detach(), cell.gate.bias.detach(),
            cell.units.W1.detach(), cell.units.b1.detach(), cell.units.W2.detach(),
            cell.units.b2.detach(), cell.W_out.weight.detach(),
            (cell.cand_norm.weight if cand_norm else norm_w).detach(),
            cand_norm, float(getattr(cell.norm, "eps", None) or 0.0),
            float(getattr(cell.cand_norm, "eps", None) or 0.0) if cand_norm else 0.0)
    return CellGraphState.make(h=h_new, q=q_new, age=age_new, pos=state.pos + 1), h_sel
