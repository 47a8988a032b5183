"""The numerical ABI of the sparse round on the HIP library: the gather of the selected cells'
state into the cell input, the grouped unit MLP, the CSR neighbour messages and the gated delta
update, with their backwards.

Mirrors the reference's custom ops (python/hsn/kernels/ops.py:91-130 for the gather, :133-180
for the unit MLP, :183-221 for the messages, :224-300 for the update): the same op names
(``hsn::gather_concat``, ``hsn::gather_concat_backward``, ``hsn::grouped_unit_mlp``,
``hsn::grouped_unit_mlp_backward``, ``hsn::csr_messages``, ``hsn::csr_messages_backward``,
``hsn::gated_delta_update`` in place on ``h, q, age``, ``hsn::gated_delta_update_functional``,
``hsn::gated_delta_update_state``, ``hsn::gated_delta_update_backward``), schemas, mutation
sets, fakes and autograd registrations. Each op is one call of ``include/hsn_ops.h`` on torch's current stream; inputs are
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
    "grouped_unit_mlp",
    "grouped_unit_mlp_backward",
    "csr_messages",
    "csr_messages_backward",
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
    hn = h.clone(memory_format=torch.contiguous_format)
    qn = q.clone(memory_format=torch.contiguous_format)
    an = age.to(torch.int32, copy=True, memory_format=torch.contiguous_format)
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


# --------------------------------------------------------------------------------------------
# the grouped unit MLP (reference python/hsn/kernels/ops.py:133-180)
# --------------------------------------------------------------------------------------------


@torch.library.custom_op("hsn::grouped_unit_mlp", mutates_args=(), device_types="cuda")
def grouped_unit_mlp(v: Tensor, idx: Tensor, w1: Tensor, b1: Tensor, w2: Tensor,
                     b2: Tensor) -> tuple[Tensor, Tensor]:
    """``(out [P,d], hidden [P,H])``: unit ``idx[p]`` on pair ``p``, ``hidden`` the saved
    pre-GELU ``z1`` (reference hsn_ops.h:101-112)."""
    P, M, d, H = v.shape[0], w1.shape[0], w2.shape[2], w1.shape[2]
    v, idx, w1, b1, w2, b2 = (v.contiguous(), _i32(idx), w1.contiguous(), b1.contiguous(),
                              w2.contiguous(), b2.contiguous())
    out, hidden = v.new_empty((P, d)), v.new_empty((P, H))
    call("hsn_grouped_unit_mlp_fwd", ptr(v), ptr(idx), ptr(w1), ptr(b1), ptr(w2), ptr(b2),
         ptr(hidden), ptr(out), P, M, d, H, _code(v), stream_of(v.device))
    return out, hidden


@grouped_unit_mlp.register_fake
def _mlp_fake(v, idx, w1, b1, w2, b2):
    return v.new_empty((v.shape[0], w2.shape[2])), v.new_empty((v.shape[0], w1.shape[2]))


@torch.library.custom_op("hsn::grouped_unit_mlp_backward", mutates_args=(), device_types="cuda")
def grouped_unit_mlp_backward(v: Tensor, idx: Tensor, w1: Tensor, w2: Tensor, hidden: Tensor,
                              dout: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """``(dv, dw1, db1, dw2, db2)`` from the saved ``z1`` (reference hsn_ops.h:114-130)."""
    P, M, d, H = v.shape[0], w1.shape[0], w2.shape[2], w1.shape[2]
    v, idx, w1, w2, hidden, dout = (v.contiguous(), _i32(idx), w1.contiguous(), w2.contiguous(),
                                    hidden.contiguous(), dout.contiguous())
    dv, dw1, dw2 = torch.empty_like(v), torch.empty_like(w1), torch.empty_like(w2)
    db1, db2 = w1.new_empty((M, H)), w2.new_empty((M, d))
    call("hsn_grouped_unit_mlp_bwd", ptr(v), ptr(idx), ptr(w1), ptr(w2), ptr(hidden), ptr(dout),
         ptr(dv), ptr(dw1), ptr(db1), ptr(dw2), ptr(db2), P, M, d, H, _code(v), 1,
         stream_of(v.device))
    return dv, dw1, db1, dw2, db2


@grouped_unit_mlp_backward.register_fake
def _mlp_bwd_fake(v, idx, w1, w2, hidden, dout):
    return (torch.empty_like(v), torch.empty_like(w1), w1.new_empty((w1.shape[0], w1.shape[2])),
            torch.empty_like(w2), w2.new_empty((w2.shape[0], w2.shape[2])))


def _mlp_setup(ctx: Any, inputs: tuple[Any, ...], output: tuple[Tensor, Tensor]) -> None:
    v, idx, w1, _, w2, _ = inputs
    ctx.save_for_backward(v, idx, w1, w2, output[1])
    ctx.mark_non_differentiable(output[1])


def _mlp_grad(ctx: Any, dout: Tensor, dhidden: Tensor) -> tuple[Any, ...]:
    dv, dw1, db1, dw2, db2 = grouped_unit_mlp_backward(*ctx.saved_tensors, dout.contiguous())
    return dv, None, dw1, db1, dw2, db2


grouped_unit_mlp.register_autograd(_mlp_grad, setup_context=_mlp_setup)


# --------------------------------------------------------------------------------------------
# the CSR neighbour messages (reference python/hsn/kernels/ops.py:183-221)
# --------------------------------------------------------------------------------------------


@torch.library.custom_op("hsn::csr_messages", mutates_args=(), device_types="cuda")
def csr_messages(h: Tensor, indptr: Tensor, indices: Tensor, a: Tensor, V: Tensor,
                 idx: Tensor) -> Tensor:
    """``m [B,K,d]``: ``m[r,k] = sum_e a[e] (V h[r, indices[e]])`` over the edges of row
    ``idx[r,k]`` (reference hsn_ops.h:132-143)."""
    B, N, d = h.shape
    K, E = idx.shape[1], a.numel()
    h, indptr, indices, a, V, idx = (h.contiguous(), _i32(indptr), _i32(indices), a.contiguous(),
                                     V.contiguous(), _i32(idx))
    m = h.new_empty((B, K, d))
    call("hsn_csr_messages", ptr(h), ptr(indptr), ptr(indices), ptr(a), ptr(V), ptr(idx), ptr(m),
         B, N, d, K, E, _code(h), stream_of(h.device))
    return m


@csr_messages.register_fake
def _messages_fake(h, indptr, indices, a, V, idx):
    return h.new_empty((*idx.shape, h.shape[2]))


@torch.library.custom_op("hsn::csr_messages_backward", mutates_args=(), device_types="cuda")
def csr_messages_backward(h: Tensor, indptr: Tensor, indices: Tensor, a: Tensor, V: Tensor,
                          idx: Tensor, dm: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """``(dh, da, dV)`` of the messages (reference hsn_ops.h:145-153)."""
    B, N, d = h.shape
    K, E = idx.shape[1], a.numel()
    h, indptr, indices, a, V, idx, dm = (h.contiguous(), _i32(indptr), _i32(indices),
                                         a.contiguous(), V.contiguous(), _i32(idx),
                                         dm.contiguous())
    dh, da, dV = torch.empty_like(h), torch.empty_like(a), torch.empty_like(V)
    call("hsn_csr_messages_bwd", ptr(h), ptr(indptr), ptr(indices), ptr(a), ptr(V), ptr(idx),
         ptr(dm), ptr(dh), ptr(da), ptr(dV), B, N, d, K, E, _code(h), 1, stream_of(h.device))
    return dh, da, dV


@csr_messages_backward.register_fake
def _messages_bwd_fake(h, indptr, indices, a, V, idx, dm):
    return torch.empty_like(h), torch.empty_like(a), torch.empty_like(V)


def _messages_setup(ctx: Any, inputs: tuple[Any, ...], output: Tensor) -> None:
    ctx.save_for_backward(*inputs)


def _messages_grad(ctx: Any, dm: Tensor) -> tuple[Any, ...]:
    dh, da, dV = csr_messages_backward(*ctx.saved_tensors, dm.contiguous())
    return dh, None, None, da, dV, None


csr_messages.register_autograd(_messages_grad, setup_context=_messages_setup)
