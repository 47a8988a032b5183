"""The four-op numerical ABI of the sparse round on the HIP library: the gather of the selected
cells' state into the cell input and the gated delta update, with their backwards.

Mirrors the reference's custom ops (python/hsn/kernels/ops.py:91-130 for the gather,
:224-300 for the update): the same op names (``hsn::gather_concat``,
``hsn::gather_concat_backward``, ``hsn::gated_delta_update`` in place on ``h, q, age``,
``hsn::gated_delta_update_functional``, ``hsn::gated_delta_update_state``,
``hsn::gated_delta_update_backward``), schemas, mutation sets, fakes and autograd
registrations. Each op is one call of ``include/hsn_ops.h`` on torch's current stream; inputs are
made contiguous and indices int32 as that ABI takes them. There is no other implementation:
without the library every op raises.
"""

from __future__ import annotations

from typing import Any

import torch
from torch import Tensor

from .._lib import call, ptr, stream_of

__all__ = [
    "available",
    "gather_concat",
    "gather_concat_backward",
    "gated_delta_update",
    "gated_delta_update_functional",
    "gated_delta_update_state",
    "gated_delta_update_backward",
]

_DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def available() -> bool:
    from .. import _lib

    return _lib.available()


def _code(t: Tensor) -> int:
    try:
        return _DTYPE[t.dtype]
    except KeyError:
        raise TypeError(f"hsn ops take float32, float16 or bfloat16, not {t.dtype}") from None


def _i32(t: Tensor) -> Tensor:
    return t.to(torch.int32).contiguous()


@torch.library.custom_op("hsn::gather_concat", mutates_args=(), device_types="cuda")
def gather_concat(u: Tensor, eps: Tensor, h: Tensor, m: Tensor, idx: Tensor) -> Tensor:
    """``v[r,k] = [u[r]; eps[r]; h[r, idx[r,k]]; m[r,k]]`` (reference hsn_ops.h:79-87)."""
    B, N, d = h.shape
    K = idx.shape[1]
    u, eps, h, m, idx = u.contiguous(), eps.contiguous(), h.contiguous(), m.contiguous(), _i32(idx)
    v = h.new_empty((B, K, 4 * d))
    call("hsn_gather_concat", ptr(u), ptr(eps), ptr(h), ptr(m), ptr(idx), ptr(v), B, N, d, K,
         _code(h), stream_of(h.device))
    return v


@gather_concat.register_fake
def _gather_fake(u, eps, h, m, idx):
    return h.new_empty((*idx.shape, 4 * h.shape[2]))


@torch.library.custom_op("hsn::gather_concat_backward", mutates_args=(), device_types="cuda")
def gather_concat_backward(dv: Tensor, idx: Tensor, n: int) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """``(grad_u, grad_eps, grad_h, grad_m)`` of the gather (reference hsn_ops.h:88-99)."""
    B, K, width = dv.shape
    d = width // 4
    dv, idx = dv.contiguous(), _i32(idx)
    du, de = dv.new_empty((B, d)), dv.new_empty((B, d))
    dh, dm = dv.new_empty((B, n, d)), dv.new_empty((B, K, d))
    call("hsn_gather_concat_bwd", ptr(dv), ptr(idx), ptr(du), ptr(de), ptr(dh), ptr(dm), B, n, d,
         K, _code(dv), 1, stream_of(dv.device))
    return du, de, dh, dm


@gather_concat_backward.register_fake
def _gather_bwd_fake(dv, idx, n):
    B, K, width = dv.shape
    d = width // 4
    return dv.new_empty((B, d)), dv.new_empty((B, d)), dv.new_empty((B, n, d)), dv.new_empty((B, K, d))


def _gather_setup(ctx: Any, inputs: tuple[Any, ...], output: Tensor) -> None:
    ctx.save_for_backward(inputs[4])
    ctx.n = inputs[2].shape[1]


def _gather_grad(ctx: Any, dv: Tensor) -> tuple[Any, ...]:
    return (*gather_concat_backward(dv.contiguous(), ctx.saved_tensors[0], ctx.n), None)


gather_concat.register_autograd(_gather_grad, setup_context=_gather_setup)


def _update(h: Tensor, q: Tensor, age: Tensor, idx: Tensor, valid: Tensor, c: Tensor,
            b: Tensor) -> Tensor:
    """The in-place update of contiguous ``h, q`` (float) and ``age`` (int32); returns
    ``h_old_saved``."""
    B, N, d = h.shape
    K = idx.shape[1]
    old = torch.empty_like(c, memory_format=torch.contiguous_format)
    call("hsn_gated_delta_update", ptr(h), ptr(q), ptr(age), ptr(_i32(idx)), ptr(_i32(valid)),
         ptr(c.contiguous()), ptr(b.contiguous()), ptr(old), B, N, d, K, _code(h),
         stream_of(h.device))
    return old


def _check_inplace(h: Tensor, q: Tensor, age: Tensor) -> None:
    if not (h.is_contiguous() and q.is_contiguous() and age.is_contiguous()):
        raise ValueError("gated_delta_update updates h, q, age in place: they must be contiguous")
    if age.dtype != torch.int32:
        raise TypeError("gated_delta_update: age must be int32 (the ABI's counters)")


@torch.library.custom_op("hsn::gated_delta_update", mutates_args=("h", "q", "age"),
                         device_types="cuda")
def gated_delta_update(h: Tensor, q: Tensor, age: Tensor, idx: Tensor, valid: Tensor, c: Tensor,
                       b: Tensor) -> Tensor:
    """In place on ``h, q, age`` (reference hsn_ops.h:155-171); returns ``h_old_saved``."""
    if any(t.requires_grad for t in (h, q, c, b)) and torch.is_grad_enabled():
        raise RuntimeError("use the functional update for training")
    _check_inplace(h, q, age)
    return _update(h, q, age, idx, valid, c, b)


@gated_delta_update.register_fake
def _update_inplace_fake(h, q, age, idx, valid, c, b):
    return torch.empty_like(c)


def _functional(h, q, age, idx, valid, c, b):
    hn, qn = h.contiguous().clone(), q.contiguous().clone()
    an = age.to(torch.int32).contiguous().clone()
    old = _update(hn, qn, an, idx, valid, c, b)
    return hn, qn, an.to(age.dtype), old


@torch.library.custom_op("hsn::gated_delta_update_functional", mutates_args=(),
                         device_types="cuda")
def gated_delta_update_functional(h: Tensor, q: Tensor, age: Tensor, idx: Tensor, valid: Tensor,
                                  c: Tensor, b: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """``(h', q', age', h_old_saved)`` without touching the inputs."""
    return _functional(h, q, age, idx, valid, c, b)


@gated_delta_update_functional.register_fake
def _update_fake(h, q, age, idx, valid, c, b):
    return torch.empty_like(h), torch.empty_like(q), torch.empty_like(age), torch.empty_like(c)


@torch.library.custom_op("hsn::gated_delta_update_state", mutates_args=(), device_types="cuda")
def gated_delta_update_state(h: Tensor, q: Tensor, age: Tensor, idx: Tensor, valid: Tensor,
                             c: Tensor, b: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """The state-producing form (the reference's op 8): the same outputs as the functional
    update, written into fresh tensors."""
    return _functional(h, q, age, idx, valid, c, b)


@gated_delta_update_state.register_fake
def _state_update_fake(h, q, age, idx, valid, c, b):
    return torch.empty_like(h), torch.empty_like(q), torch.empty_like(age), torch.empty_like(c)


@torch.library.custom_op("hsn::gated_delta_update_backward", mutates_args=(), device_types="cuda")
def gated_delta_update_backward(idx: Tensor, valid: Tensor, c: Tensor, b: Tensor, old: Tensor,
                                G: Tensor, g: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """``(grad_h, grad_q, grad_c, grad_b)`` from ``grad_h_out = G``, ``grad_q_out = g``
    (reference hsn_ops.h:173-187)."""
    B, N, d = G.shape
    K = idx.shape[1]
    c, b, old, G, g = c.contiguous(), b.contiguous(), old.contiguous(), G.contiguous(), g.contiguous()
    dh, dq = torch.empty_like(G), torch.empty_like(g)
    dc, db = torch.empty_like(c), torch.empty_like(b)
    call("hsn_gated_delta_update_bwd", ptr(_i32(idx)), ptr(_i32(valid)), ptr(c), ptr(b), ptr(old),
         ptr(G), ptr(g), ptr(dh), ptr(dq), ptr(dc), ptr(db), B, N, d, K, _code(G),
         stream_of(G.device))
    return dh, dq, dc, db


@gated_delta_update_backward.register_fake
def _update_bwd_fake(idx, valid, c, b, old, G, g):
    return torch.empty_like(G), torch.empty_like(g), torch.empty_like(c), torch.empty_like(b)


def _update_setup(ctx: Any, inputs: tuple[Any, ...], output: tuple[Tensor, ...]) -> None:
    _, _, _, idx, valid, c, b = inputs
    ctx.save_for_backward(idx, valid, c, b, output[3])
    ctx.mark_non_differentiable(output[2], output[3])


def _update_grad(ctx: Any, G: Tensor, g: Tensor, dage: Tensor, dold: Tensor) -> tuple[Any, ...]:
    dh, dq, dc, db = gated_delta_update_backward(*ctx.saved_tensors, G.contiguous(), g.contiguous())
    return dh, dq, None, None, None, dc, db


gated_delta_update_functional.register_autograd(_update_grad, setup_context=_update_setup)
gated_delta_update_state.register_autograd(_update_grad, setup_context=_update_setup)
