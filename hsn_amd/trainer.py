"""The trainer's per-step passes after ``backward()`` as single launches on MI355X
(``include/hsn_trainer.h``; the reference's ``python/hsn/kernels/trainer.py``).

The optimiser step (``hsn.train.lazy_adam``), the float64 clip's scaling (``grad_norm``), the
update caps (``update_limit``) and the weight average (``weight_ema``) each walk a list of tensors
with a few elementwise operations; here each is one pass over the whole list. Same functions,
arguments and return convention as the reference: ``True`` when the pass ran, ``False`` when it did
not, having touched nothing (the tensors are not contiguous fp32 tensors on one ROCm device, the
list is empty, or the passes are switched off by :func:`set_enabled` or ``HSN_TRAINER_KERNELS=0``);
the caller then runs its PyTorch operations, which each pass equals bit for bit. A missing or stale
HIP library raises (there is no other implementation here).
"""

from __future__ import annotations

import ctypes
import os
from collections.abc import Sequence

import torch
from torch import Tensor

from . import _lib

# The pointer tables in one native call (hsn_amd/host/tables.cpp) when that module is built from
# the current source; otherwise the same checks and tables are made here, tensor by tensor.
_native = _lib.host_tables()

__all__ = [
    "MAX_UNITS",
    "adamw",
    "adamw_units",
    "copy",
    "enabled",
    "lerp",
    "limit_project",
    "limit_squares",
    "ready",
    "scale64",
    "set_enabled",
]

#: The most units a stacked unit tensor may have (reference ``HSN_TR_UNITS``).
MAX_UNITS = 64

_enabled = os.environ.get("HSN_TRAINER_KERNELS", "1") != "0"


def set_enabled(flag: bool) -> bool:
    """Switch the passes on or off for this process; returns the previous setting."""
    global _enabled
    previous = _enabled
    _enabled = bool(flag)
    return previous


def enabled() -> bool:
    return _enabled


def ready(device: torch.device) -> bool:
    """Whether the passes run on ``device``: switched on and a ROCm device. The library must be
    built and current (else ``RuntimeError``)."""
    if not _enabled or device.type != "cuda":
        return False
    _lib.library()
    return True


def _fits(rows: Sequence[Sequence[Tensor]]) -> bool:
    """Whether the rows fit a pass, checked tensor by tensor (the native tables' checks)."""
    first = rows[0]
    if not first or any(len(row) != len(first) for row in rows):
        return False
    device = first[0].device
    for row in rows:
        for t in row:
            if t.dtype != torch.float32 or not t.is_contiguous() or t.device != device:
                return False
    for j, t in enumerate(first):
        if any(row[j].numel() != t.numel() for row in rows):
            return False
    return ready(device)


def _pointers(row: Sequence[Tensor]):
    return (ctypes.c_void_p * len(row))(*[t.data_ptr() for t in row])


def _numels(row: Sequence[Tensor]):
    return (ctypes.c_int64 * len(row))(*[t.numel() for t in row])


def _tables(rows: Sequence[Sequence[Tensor]]):
    """``(pointer arrays, element counts)`` of R lists of n tensors as the C entry points take
    them (one ``void*[n]`` a list, the first list's ``int64[n]``), or ``None`` when the lists do
    not fit a pass: an empty list, lists of different lengths, a tensor that is not a contiguous
    fp32 tensor on the first one's device, different counts at one index, or passes that do not
    run on that device (:func:`ready`)."""
    if _native is None:
        if not _fits(rows):
            return None
        return [_pointers(r) for r in rows], _numels(rows[0])
    buf = _native.list_table(rows)
    if buf is None or not ready(rows[0][0].device):
        return None
    n, R = len(rows[0]), len(rows)
    pointers = ctypes.c_void_p * n
    return ([pointers.from_buffer(buf, 8 * n * r) for r in range(R)],
            (ctypes.c_int64 * n).from_buffer(buf, 8 * n * R))


def adamw(
    params: Sequence[Tensor],
    grads: Sequence[Tensor],
    exp_avgs: Sequence[Tensor],
    exp_avg_sqs: Sequence[Tensor],
    *,
    lr: float,
    beta1: float,
    beta2: float,
    eps: float,
    weight_decay: float,
    step: int,
) -> bool:
    """``LazyAdamW._dense_steps`` as one pass: the AdamW step of ordinary tensors at the step
    count ``step`` (already advanced); the coefficients from the same host arithmetic (reference
    ``python/hsn/kernels/trainer.py:111-144``)."""
    tables = _tables((params, grads, exp_avgs, exp_avg_sqs))
    if tables is None:
        return False
    bias_correction1 = 1 - beta1**step
    bias_correction2 = 1 - beta2**step
    step_size = lr / bias_correction1
    bias_correction2_sqrt = bias_correction2**0.5
    coefs = (ctypes.c_float * 7)(
        1 - lr * weight_decay,
        1 - beta1,
        beta2,
        1 - beta2,
        1.0 / bias_correction2_sqrt,  # multiplied by 1/s, matching torch's rounding of list / scalar
        eps,
        -step_size,
    )
    device = params[0].device
    _lib.call("hsn_tr_adamw", *tables[0], tables[1], len(params), int(weight_decay != 0), coefs,
              _lib.stream_of(device))
    return True


def adamw_units(
    params: Sequence[Tensor],
    grads: Sequence[Tensor],
    exp_avgs: Sequence[Tensor],
    exp_avg_sqs: Sequence[Tensor],
    *,
    n_units: int,
    active: Sequence[bool],
    decay: Sequence[float],
    lerp_weight: Sequence[float],
    beta2_factor: Sequence[float],
    bias_correction2_sqrt: Sequence[float],
    step_size: Sequence[float],
    beta2: float,
    eps: float,
    weight_decay: float,
) -> bool:
    """``LazyAdamW._unit_step`` as one pass for stacked unit tensors ``[n_units, ...]`` that
    share their per-unit coefficients (each a sequence of ``n_units`` values: the coefficient
    tensors of ``_unit_step``; reference ``trainer.py:147-191``)."""
    if n_units > MAX_UNITS or n_units < 1 or any(p.dim() == 0 or p.shape[0] != n_units for p in params):
        return False
    tables = _tables((params, grads, exp_avgs, exp_avg_sqs))
    if tables is None:
        return False
    table = [[1.0 if flag else 0.0 for flag in active], decay, lerp_weight, beta2_factor,
             bias_correction2_sqrt, step_size]
    if any(len(row) != n_units for row in table):
        return False
    coefs = (ctypes.c_float * (6 * n_units))(*[float(v) for row in table for v in row])
    device = params[0].device
    _lib.call("hsn_tr_adamw_units", *tables[0], tables[1], len(params), n_units, int(weight_decay != 0), coefs, 1 - beta2, eps, _lib.stream_of(device))
    return True


def lerp(selfs: Sequence[Tensor], ends: Sequence[Tensor], weight: float) -> bool:
    """Move every ``selfs[i]`` toward ``ends[i]`` by ``weight`` in place, one launch for the
    whole list; the same result as ``torch._foreach_lerp_``."""
    tables = _tables((selfs, ends))
    if tables is None:
        return False
    _lib.call("hsn_tr_lerp", *tables[0], tables[1], len(selfs), float(weight),
              _lib.stream_of(selfs[0].device))
    return True


def scale64(grads: Sequence[Tensor], coefficient: Tensor) -> bool:
    """``grad.copy_((grad.double() * coefficient).float())`` for every gradient as one pass;
    ``coefficient`` is a one-element float64 tensor on the gradients' device."""
    tables = _tables((grads,))
    if tables is None:
        return False
    if (coefficient.dtype != torch.float64 or coefficient.numel() != 1
            or coefficient.device != grads[0].device):
        return False
    _lib.call("hsn_tr_scale64", *tables[0], tables[1], len(grads), coefficient.data_ptr(),
              _lib.stream_of(grads[0].device))
    return True


def copy(dsts: Sequence[Tensor], srcs: Sequence[Tensor]) -> bool:
    """Overwrite each fp32 ``dsts[i]`` with ``srcs[i]``, one launch for the whole list (what
    ``torch._foreach_copy_`` does)."""
    tables = _tables((dsts, srcs))
    if tables is None:
        return False
    _lib.call("hsn_tr_copy", *tables[0], tables[1], len(dsts), _lib.stream_of(dsts[0].device))
    return True


def limit_squares(
    params: Sequence[Tensor],
    olds: Sequence[Tensor],
    old_squares: Sequence[Tensor],
    delta_squares: Sequence[Tensor],
) -> bool:
    """Element-wise squares for the limiter's two norms, written into the given buffers:
    ``old_squares[i] = olds[i] ** 2`` (the norm of the previous weights) and
    ``delta_squares[i] = (params[i] - olds[i]) ** 2`` (the norm of the proposed step)."""
    tables = _tables((params, olds, old_squares, delta_squares))
    if tables is None:
        return False
    _lib.call("hsn_tr_limit_squares", *tables[0], tables[1], len(params),
              _lib.stream_of(params[0].device))
    return True


def limit_project(
    params: Sequence[Tensor],
    olds: Sequence[Tensor],
    applied_squares: Sequence[Tensor],
    groups: Sequence[Tensor],
) -> bool:
    """Pull each tensor of a clipped group back toward its previous weights: for tensor ``j``,
    ``groups[j]`` is a two-element fp32 device tensor ``[scale, clipped]``; where ``clipped`` is
    set the step ``params[j] - olds[j]`` is multiplied by ``scale`` in place. Every tensor's
    final step squared goes to ``applied_squares[j]``."""
    if len(groups) != len(params):
        return False
    tables = _tables((params, olds, applied_squares))
    if tables is None:
        return False
    # the groups: contiguous fp32 pairs on the same device
    pairs = _tables((groups,))
    if pairs is None or any(c != 2 for c in pairs[1]) or groups[0].device != params[0].device:
        return False
    _lib.call("hsn_tr_limit_project", *tables[0], pairs[0][0], tables[1], len(params),
              _lib.stream_of(params[0].device))
    return True
