"""The window hot path on MI355X: route -> forward sweep -> backward recurrence, with the
carried-state gradient.

This is the window-level counterpart of the reference's split/fused window
(python/hsn/train/split.py:372-762, python/hsn/train/compile.py:892-1024): instead of one to
five launches per position and a full-state tape ``[B, T+1, N, d]``, a window is the route and
forward sweep (``hsn_win_route_forward``: one launch where the forward's workgroups decide the
window themselves, else ``hsn_win_route`` then ``hsn_win_forward``) and the backward
(``hsn_win_backward``), and the tape is the slots' pre-round states ``h_old [B, T, K, d]``. Every function requires CUDA (ROCm) tensors and the
built HIP library; there is no CPU path here.

Decisions (``cells``, ``units``) are int32 in the window form (the reference's per-position
ops keep int64, see :mod:`hsn_amd.kernels.window`); ``valid``, ``refreshed`` and ``reset`` are
bool. The state is fp32; inputs and per-slot outputs are fp32 or bf16 (``io`` storage).
"""

from __future__ import annotations

import dataclasses
from typing import Optional

import torch
from torch import Tensor

from . import _lib
from ._lib import DTYPE_BF16, DTYPE_F32, call, ptr, stream_of

#: ``python/hsn/model/router.py:196``: the budget's relative slack.
BUDGET_SLACK = 1e-5

__all__ = [
    "BUDGET_SLACK",
    "RouteConfig",
    "check_reserved",
    "route",
    "forward",
    "route_forward",
    "route_forward_fuses",
    "exchange_timeouts",
    "backward",
    "window_forward",
    "window_backward",
    "WindowRecurrence",
    "pack_slots",
]


@dataclasses.dataclass(frozen=True)
class RouteConfig:
    """The router's hard-decision settings (``Router.select`` with mode ``topk``;
    ``limit = budget * (1 + BUDGET_SLACK)``)."""

    k: int
    age_max: int = 0
    probes: bool = False
    lambda_cost: float = 0.0
    cell_overhead: float = 0.0
    shared_cost: float = 0.0
    limit: float = 1.0 + BUDGET_SLACK
    reserved: int = 0
    reserved_units: bool = False

    def __post_init__(self):
        check_reserved(self.k, self.reserved, self.reserved_units)


def check_reserved(k: int, reserved: int, reserved_units: bool) -> None:
    """The router's checks of the fast cells (``python/hsn/model/router.py:1328-1339``):
    ``reserved`` an int in ``[0, k)``, and ``reserved_units`` only with ``reserved > 0``."""
    if isinstance(reserved, bool) or not isinstance(reserved, int) or reserved < 0:
        raise ValueError(f"reserved must be an int >= 0, got {reserved!r}")
    if reserved and reserved >= k:
        raise ValueError(f"reserved={reserved} must be < k_max={k}")
    if not reserved and reserved_units:
        raise ValueError("reserved_units needs reserved > 0")


def _io_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return DTYPE_F32
    if dtype == torch.bfloat16:
        return DTYPE_BF16
    raise ValueError(f"storage dtype must be float32 or bfloat16, got {dtype}")


def _check(t: Tensor, name: str, shape: tuple, dtype=None, device=None) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def route(logits: Tensor, cost: Tensor, cfg: RouteConfig, *, reset: Optional[Tensor] = None,
          age0: Optional[Tensor] = None, h_max_zero: Optional[Tensor] = None,
          with_slots: bool = False):
    """Every position's decision: ``(cells, units, valid, theta, refreshed)`` with shapes
    ``[B,T,K]`` (int32, int32, bool), ``[B,T]`` fp32 and ``[B,T,K]`` bool; with ``with_slots``
    a sixth ``slots [B,T,K]`` int32, the packed decision the sweeps read (the cell where the slot
    is valid, -1 where it is padded).

    ``logits [B,T,N,M]`` fp32/bf16, ``cost [M]`` fp32. With ``cfg.probes`` the ages evolve
    with the decisions from ``age0 [B,N]`` (int64) and the resets ``reset [B,T]``.
    ``h_max_zero [B,T]`` fp32, if given, is zeroed for :func:`forward`'s row maxima."""
    B, T, N, M = (int(s) for s in logits.shape)
    dev = logits.device
    _check(logits, "logits", (B, T, N, M))
    _check(cost, "cost", (M,), torch.float32, dev)
    if cfg.probes:
        if reset is None or age0 is None:
            raise ValueError("probes need reset and age0")
        _check(reset, "reset", (B, T), torch.bool, dev)
        _check(age0, "age0", (B, N), torch.int64, dev)
    K = cfg.k
    cells = torch.empty(B, T, K, dtype=torch.int32, device=dev)
    units = torch.empty_like(cells)
    valid = torch.empty(B, T, K, dtype=torch.bool, device=dev)
    refreshed = torch.empty_like(valid)
    theta = torch.empty(B, T, dtype=torch.float32, device=dev)
    slots = torch.empty(B, T, K, dtype=torch.int32, device=dev) if with_slots else None
    if h_max_zero is not None:
        _check(h_max_zero, "h_max_zero", (B, T), torch.float32, dev)
    call("hsn_win_route", ptr(logits), _io_code(logits.dtype), M, ptr(cost),
         ptr(age0) if cfg.probes else None, ptr(reset) if cfg.probes else None, ptr(cells),
         ptr(units), 32, ptr(valid), ptr(theta), ptr(refreshed), ptr(slots), ptr(h_max_zero), B, T,
         N, M, K,
         int(cfg.age_max), int(bool(cfg.probes)), float(cfg.lambda_cost),
         float(cfg.cell_overhead), float(cfg.shared_cost), float(cfg.limit), int(cfg.reserved),
         int(bool(cfg.reserved_units)), stream_of(dev))
    if with_slots:
        return cells, units, valid, theta, refreshed, slots
    return cells, units, valid, theta, refreshed


def pack_slots(cells: Tensor, valid: Tensor) -> Tensor:
    """The packed decision ``where(valid, cells, -1)`` as int32 (what :func:`route` emits as
    ``slots``), for decisions that come from elsewhere."""
    return torch.where(valid, cells.to(torch.int32), torch.full_like(cells, -1, dtype=torch.int32))


def rms_scratch_bytes(slots: int, d: int, elem: int) -> int:
    """Bytes of the RMS candidate's workspace: ``[slots, d]`` of the storage type, then
    ``[slots]`` fp32 at the next 16-byte boundary (``include/hsn_window.h``)."""
    return ((slots * d * elem + 15) & ~15) + 4 * slots


def _workspace(op: int, B: int, T: int, N: int, d: int, K: int, io: torch.dtype,
               cand_norm: bool, dev) -> tuple[Optional[Tensor], int]:
    """The workspace of a forward / backward call (``None`` where the call needs none) and its
    size, as the library reports it for the path the call takes."""
    n = _lib.workspace_bytes(op, B, T, N, d, K, _io_code(io), cand_norm)
    return (torch.empty(n, dtype=torch.uint8, device=dev) if n else None), n


def forward(y: Tensor, gate_pre: Tensor, reset: Tensor, slots: Tensor, h0: Tensor, q0: Tensor,
            age0: Tensor, pos0: Tensor, n_cells: int, *, cand_norm: bool = False,
            cand_w: Optional[Tensor] = None, cand_eps: float = 1e-6,
            h_max: Optional[Tensor] = None, h_max_zeroed: bool = False) -> dict:
    """The forward sweep from given decisions (``slots [B,T,K]`` int32, see :func:`route`).
    Returns ``q_pre, q_post [B,T,d]``,
    ``h_sel, h_old [B,T,K,d]`` (storage dtype), the end state ``h [B,N,d], q [B,d]`` (fp32),
    ``age [B,N], pos [B]`` (int64) and, when a buffer ``h_max [B,T]`` is passed, the row maxima
    in it. The sweep max-reduces into that buffer, so it is zeroed here first unless
    ``h_max_zeroed`` says :func:`route` already did (its ``h_max_zero``)."""
    B, T, K, d = (int(s) for s in y.shape)
    N = int(n_cells)
    dev, io = y.device, y.dtype
    _check(y, "y", (B, T, K, d))
    _check(gate_pre, "gate_pre", (B, T, K, d), io, dev)
    _check(reset, "reset", (B, T), torch.bool, dev)
    _check(slots, "slots", (B, T, K), torch.int32, dev)
    _check(h0, "h0", (B, N, d), torch.float32, dev)
    _check(q0, "q0", (B, d), torch.float32, dev)
    _check(age0, "age0", (B, N), torch.int64, dev)
    _check(pos0, "pos0", (B,), torch.int64, dev)
    if cand_norm:
        if cand_w is None:
            raise ValueError("cand_norm needs cand_w")
        _check(cand_w, "cand_w", (d,), torch.float32, dev)
    ws, ws_bytes = _workspace(_lib.OP_FORWARD, B, T, N, d, K, io, cand_norm, dev)
    out = {
        "q_pre": torch.empty(B, T, d, dtype=io, device=dev),
        "q_post": torch.empty(B, T, d, dtype=io, device=dev),
        "h_sel": torch.empty(B, T, K, d, dtype=io, device=dev),
        "h_old": torch.empty(B, T, K, d, dtype=io, device=dev),
        "h": torch.empty(B, N, d, dtype=torch.float32, device=dev),
        "q": torch.empty(B, d, dtype=torch.float32, device=dev),
        "age": torch.empty(B, N, dtype=torch.int64, device=dev),
        "pos": torch.empty(B, dtype=torch.int64, device=dev),
    }
    if h_max is not None:
        _check(h_max, "h_max", (B, T), torch.float32, dev)
        if not h_max_zeroed:
            h_max.zero_()
        out["h_max"] = h_max
    call("hsn_win_forward", ptr(y), ptr(gate_pre), _io_code(io), ptr(cand_w) if cand_norm else None,
         int(bool(cand_norm)), float(cand_eps), ptr(ws), ws_bytes, ptr(reset), ptr(slots),
         ptr(h0), ptr(q0), ptr(age0), ptr(pos0), ptr(out["q_pre"]), ptr(out["q_post"]),
         ptr(out["h_sel"]), ptr(out["h_old"]), ptr(h_max), ptr(out["h"]), ptr(out["q"]),
         ptr(out["age"]), ptr(out["pos"]), B, T, N, d, K, stream_of(dev))
    return out


def backward(y: Tensor, gate_pre: Tensor, h_old: Tensor, slots: Tensor,
             reset: Tensor, n_cells: int, d_q_pre: Optional[Tensor], d_q_post: Optional[Tensor],
             d_h_sel: Optional[Tensor], d_h_T: Optional[Tensor] = None,
             d_q_T: Optional[Tensor] = None, *, cand_norm: bool = False,
             cand_w: Optional[Tensor] = None, cand_eps: float = 1e-6):
    """The window's backward with the activations fused: ``(dy, dgate, d_h0, d_q0, d_cand_w)``.

    ``d_q_pre, d_q_post [B,T,d]`` and ``d_h_sel [B,T,K,d]`` (storage dtype) are the cotangents
    of the forward's outputs, ``None`` when absent; ``d_h_T [B,N,d]``, ``d_q_T [B,d]`` (fp32)
    the cotangent of the end state (the next window's ``d_h0, d_q0`` in a TBPTT segment).
    ``d_cand_w`` is ``None`` without the RMS candidate."""
    B, T, K, d = (int(s) for s in y.shape)
    N = int(n_cells)
    dev, io = y.device, y.dtype
    _check(y, "y", (B, T, K, d))
    for name, t in (("gate_pre", gate_pre), ("h_old", h_old)):
        _check(t, name, (B, T, K, d), io, dev)
    _check(slots, "slots", (B, T, K), torch.int32, dev)
    _check(reset, "reset", (B, T), torch.bool, dev)
    for name, t in (("d_q_pre", d_q_pre), ("d_q_post", d_q_post)):
        if t is not None:
            _check(t, name, (B, T, d), io, dev)
    if d_h_sel is not None:
        _check(d_h_sel, "d_h_sel", (B, T, K, d), io, dev)
    if d_h_T is not None:
        _check(d_h_T, "d_h_T", (B, N, d), torch.float32, dev)
    if d_q_T is not None:
        _check(d_q_T, "d_q_T", (B, d), torch.float32, dev)
    d_w = None
    if cand_norm:
        if cand_w is None:
            raise ValueError("cand_norm needs cand_w")
        _check(cand_w, "cand_w", (d,), torch.float32, dev)
        d_w = torch.empty(d, dtype=torch.float32, device=dev)
    ws, ws_bytes = _workspace(_lib.OP_BACKWARD, B, T, N, d, K, io, cand_norm, dev)
    dy = torch.empty_like(y)
    dgate = torch.empty_like(y)
    d_h0 = torch.empty(B, N, d, dtype=torch.float32, device=dev)
    d_q0 = torch.empty(B, d, dtype=torch.float32, device=dev)
    call("hsn_win_backward", ptr(y), ptr(gate_pre), ptr(h_old), _io_code(io),
         ptr(cand_w) if cand_norm else None, int(bool(cand_norm)), float(cand_eps), ptr(ws),
         ws_bytes, ptr(slots), ptr(reset), ptr(d_q_pre), ptr(d_q_post), ptr(d_h_sel),
         ptr(d_h_T), ptr(d_q_T), ptr(dy), ptr(dgate), ptr(d_h0), ptr(d_q0), ptr(d_w), B, T, N, d, K,
         stream_of(dev))
    return dy, dgate, d_h0, d_q0, d_w


def route_forward(logits: Tensor, y: Tensor, gate_pre: Tensor, reset: Tensor, h0: Tensor,
                  q0: Tensor, age0: Tensor, pos0: Tensor, cost: Tensor, cfg: RouteConfig, *,
                  cand_norm: bool = False, cand_w: Optional[Tensor] = None,
                  cand_eps: float = 1e-6, with_h_max: bool = True) -> dict:
    """:func:`route` (without probes) and :func:`forward` on its slots as one call
    (``hsn_win_route_forward``): the decisions ``cells, units, valid, theta, refreshed, slots``,
    the sweep's outputs and ``h_max [B,T]`` (when ``with_h_max``), bit for bit those of the two
    calls. One launch where :func:`route_forward_fuses` says so, else the two."""
    if cfg.probes:
        raise ValueError("route_forward decides without probes (use route, then forward)")
    B, T, N, M = (int(s) for s in logits.shape)
    K, d = cfg.k, int(y.shape[3])
    dev, io = y.device, y.dtype
    _check(logits, "logits", (B, T, N, M), device=dev)
    _check(cost, "cost", (M,), torch.float32, dev)
    _check(y, "y", (B, T, K, d))
    _check(gate_pre, "gate_pre", (B, T, K, d), io, dev)
    _check(reset, "reset", (B, T), torch.bool, dev)
    _check(h0, "h0", (B, N, d), torch.float32, dev)
    _check(q0, "q0", (B, d), torch.float32, dev)
    _check(age0, "age0", (B, N), torch.int64, dev)
    _check(pos0, "pos0", (B,), torch.int64, dev)
    if cand_norm:
        if cand_w is None:
            raise ValueError("cand_norm needs cand_w")
        _check(cand_w, "cand_w", (d,), torch.float32, dev)
    ws, ws_bytes = _workspace(_lib.OP_FORWARD, B, T, N, d, K, io, cand_norm, dev)
    cells = torch.empty(B, T, K, dtype=torch.int32, device=dev)
    out = {
        "cells": cells,
        "units": torch.empty_like(cells),
        "valid": torch.empty(B, T, K, dtype=torch.bool, device=dev),
        "refreshed": torch.empty(B, T, K, dtype=torch.bool, device=dev),
        "theta": torch.empty(B, T, dtype=torch.float32, device=dev),
        "slots": torch.empty_like(cells),
        "q_pre": torch.empty(B, T, d, dtype=io, device=dev),
        "q_post": torch.empty(B, T, d, dtype=io, device=dev),
        "h_sel": torch.empty(B, T, K, d, dtype=io, device=dev),
        "h_old": torch.empty(B, T, K, d, dtype=io, device=dev),
        "h": torch.empty(B, N, d, dtype=torch.float32, device=dev),
        "q": torch.empty(B, d, dtype=torch.float32, device=dev),
        "age": torch.empty(B, N, dtype=torch.int64, device=dev),
        "pos": torch.empty(B, dtype=torch.int64, device=dev),
    }
    h_max = torch.empty(B, T, dtype=torch.float32, device=dev) if with_h_max else None
    if h_max is not None:
        out["h_max"] = h_max
    call("hsn_win_route_forward", ptr(logits), _io_code(logits.dtype), M, ptr(cost),
         ptr(out["cells"]), ptr(out["units"]), 32, ptr(out["valid"]), ptr(out["theta"]),
         ptr(out["refreshed"]), ptr(out["slots"]), M, float(cfg.lambda_cost),
         float(cfg.cell_overhead), float(cfg.shared_cost), float(cfg.limit), int(cfg.reserved),
         int(bool(cfg.reserved_units)), ptr(y), ptr(gate_pre), _io_code(io),
         ptr(cand_w) if cand_norm else None, int(bool(cand_norm)), float(cand_eps), ptr(ws),
         ws_bytes, ptr(reset), ptr(h0), ptr(q0), ptr(age0), ptr(pos0), ptr(out["q_pre"]),
         ptr(out["q_post"]), ptr(out["h_sel"]), ptr(out["h_old"]), ptr(h_max), ptr(out["h"]),
         ptr(out["q"]), ptr(out["age"]), ptr(out["pos"]), B, T, N, d, K, stream_of(dev))
    return out


def route_forward_fuses(B: int, T: int, N: int, d: int, K: int, *, M: int = 1,
                        logits_dtype: torch.dtype = torch.float32,
                        io: torch.dtype = torch.float32, cand_norm: bool = False,
                        device=None) -> tuple[bool, Optional[str]]:
    """Whether :func:`route_forward` of this shape on the current stream of ``device`` is one
    launch, and the reason when it is two (host arithmetic; claims nothing)."""
    import ctypes

    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    out = ctypes.c_int(0)
    call("hsn_win_route_forward_fuses", int(M), _io_code(logits_dtype), 32, _io_code(io),
         int(bool(cand_norm)), B, T, N, d, K, stream_of(dev), ctypes.byref(out))
    if out.value:
        return True, None
    return False, _lib.library().hsn_win_last_error().decode(errors="replace")


def exchange_timeouts(clear: bool = True) -> int:
    """The one-launch route and forward's exchange waits that hit their limit since the last
    clear (0 unless a grid could not keep a row's workgroups resident; synchronises the
    device)."""
    import ctypes

    out = ctypes.c_uint(0)
    call("hsn_win_exchange_timeouts", ctypes.byref(out), int(bool(clear)))
    return int(out.value)


def window_forward(logits: Tensor, y: Tensor, gate_pre: Tensor, reset: Tensor, h0: Tensor,
                   q0: Tensor, age0: Tensor, pos0: Tensor, cost: Tensor, cfg: RouteConfig, *,
                   cand_norm: bool = False, cand_w: Optional[Tensor] = None,
                   cand_eps: float = 1e-6, with_h_max: bool = True) -> dict:
    """Route and forward sweep of one window: the decisions (``cells, units, valid, theta,
    refreshed``), the sweep's outputs (:func:`forward`) and ``h_max [B,T]``; without probes
    :func:`route_forward`, with them :func:`route` (whose ages evolve with the decisions) and
    then :func:`forward`."""
    if not cfg.probes:
        return route_forward(logits, y, gate_pre, reset, h0, q0, age0, pos0, cost, cfg,
                             cand_norm=cand_norm, cand_w=cand_w, cand_eps=cand_eps,
                             with_h_max=with_h_max)
    B, T, N, M = (int(s) for s in logits.shape)
    h_max = torch.empty(B, T, dtype=torch.float32, device=y.device) if with_h_max else None
    cells, units, valid, theta, refreshed, slots = route(logits, cost, cfg, reset=reset,
                                                         age0=age0, h_max_zero=h_max,
                                                         with_slots=True)
    out = forward(y, gate_pre, reset, slots, h0, q0, age0, pos0, N, cand_norm=cand_norm,
                  cand_w=cand_w, cand_eps=cand_eps, h_max=h_max, h_max_zeroed=True)
    out.update(cells=cells, units=units, valid=valid, theta=theta, refreshed=refreshed,
               slots=slots)
    return out


def window_backward(y, gate_pre, h_old, cells, valid, reset, n_cells, d_q_pre, d_q_post, d_h_sel,
                    d_h_T=None, d_q_T=None, *, cand_norm=False, cand_w=None, cand_eps=1e-6):
    """:func:`backward` with the oracle's argument order (separate cells and valid)."""
    return backward(y, gate_pre, h_old, pack_slots(cells, valid), reset, n_cells, d_q_pre,
                    d_q_post, d_h_sel, d_h_T, d_q_T, cand_norm=cand_norm, cand_w=cand_w,
                    cand_eps=cand_eps)


class WindowRecurrence(torch.autograd.Function):
    """One window as one autograd node, with the gradient into its start state.

    The counterpart of the reference's ``StateRecurrence`` (python/hsn/train/split.py:230-302)
    with the candidate / gate activations fused and the carried state made differentiable:
    ``forward(y, gate_pre, h0, q0, cand_w, logits, reset, age0, pos0, cost, cfg, cand_norm,
    cand_eps)`` returns ``(q_pre, q_post, h_sel, h_T, q_T)``; backward gives ``dL/dy``,
    ``dL/dgate_pre``, ``dL/dh0``, ``dL/dq0`` (and ``dL/dcand_w`` with the norm). A later
    window's loss reaches this one through ``h_T, q_T`` (the reference's ``tbptt_windows``
    semantics, docs/tbptt_windows.md); detach them to cut the segment. The decisions, ages and
    positions are in ``ctx.window`` after the forward."""

    @staticmethod
    def forward(ctx, y, gate_pre, h0, q0, cand_w, logits, reset, age0, pos0, cost, cfg,
                cand_norm=False, cand_eps=1e-6):
        out = window_forward(logits, y, gate_pre, reset, h0.detach().float().contiguous(),
                             q0.detach().float().contiguous(), age0, pos0, cost, cfg,
                             cand_norm=cand_norm, cand_w=cand_w, cand_eps=cand_eps)
        ctx.save_for_backward(y, gate_pre, out["h_old"], out["slots"], reset,
                              cand_w if cand_norm else None)
        ctx.n_cells = int(logits.shape[2])
        ctx.cand_norm = cand_norm
        ctx.cand_eps = cand_eps
        ctx.window = out
        return out["q_pre"], out["q_post"], out["h_sel"], out["h"], out["q"]

    @staticmethod
    def backward(ctx, d_q_pre, d_q_post, d_h_sel, d_h_T, d_q_T):
        y, gate_pre, h_old, slots, reset, cand_w = ctx.saved_tensors
        io = y.dtype

        def cot(t, dtype):
            return None if t is None else t.to(dtype).contiguous()

        dy, dgate, d_h0, d_q0, d_w = backward(
            y, gate_pre, h_old, slots, reset, ctx.n_cells, cot(d_q_pre, io),
            cot(d_q_post, io), cot(d_h_sel, io), cot(d_h_T, torch.float32),
            cot(d_q_T, torch.float32), cand_norm=ctx.cand_norm, cand_w=cand_w,
            cand_eps=ctx.cand_eps)
        return dy, dgate, d_h0, d_q0, d_w, None, None, None, None, None, None, None, None


def available() -> bool:
    return _lib.available()
