"""The sparse round's four operators on the HIP library, as a backend of the reference's kernel
layer: the gather of the selected cells' state into the cell input, the grouped unit MLP, the CSR
neighbour messages and the gated delta update, with their backwards.

Two levels, as the reference's ``python/hsn/kernels/ops.py`` has them:

* the raw custom ops under the reference's op names and schemas (:91-300): ``gather_op``
  (``hsn::gather_concat``) and ``gather_backward``, ``mlp_op`` / ``mlp_backward``
  (``hsn::grouped_unit_mlp{,_backward}``), ``messages_op`` / ``messages_backward``
  (``hsn::csr_messages{,_backward}``), ``update_inplace`` (``hsn::gated_delta_update``, in place
  on ``h, q, age``), ``update_op`` (``..._functional``), ``state_update_op`` (``..._state``) and
  ``update_backward``, each with its fake and autograd registration; each is one call of
  ``include/hsn_ops.h`` on torch's current stream;
* the ``KernelOps`` adapters (:320-444) that the reference's ``hsn.kernels.ops()`` returns for a
  selected backend: ``gather_concat``, ``grouped_unit_mlp``, ``csr_messages`` and
  ``gated_delta_update``, with the model's objects as arguments. Where the library's single-dtype
  ABI cannot express a call (``u=None``, autocast, a non-GELU bank, mixed dtypes, a tensor off
  the GPU) the adapter hands it to the fallback backend (:func:`set_fallback`; by default the
  reference's ``hsn.kernels.native``) instead of computing it here.

There is no implementation of the ops in this module besides the library: without it every raw op
raises.
"""

from __future__ import annotations

from typing import Any, Optional

import torch
from torch.utils._python_dispatch import _get_current_dispatch_mode
from torch import Tensor

from .._lib import call, ptr, stream_of

__all__ = [
    "available",
    "prepare_cuda",
    "set_fallback",
    # the KernelOps adapters
    "gather_concat",
    "grouped_unit_mlp",
    "csr_messages",
    "gated_delta_update",
    # the raw custom ops
    "gather_op",
    "gather_backward",
    "mlp_op",
    "mlp_backward",
    "messages_op",
    "messages_backward",
    "update_inplace",
    "update_op",
    "state_update_op",
    "update_backward",
]

_DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def available() -> bool:
    from .. import _lib

    return _lib.available()


def prepare_cuda(device: int = 0) -> None:
    """Make the library ready on ``device`` before warm-up or graph capture (the reference's
    ``prepare_cuda``): load it, then run every raw op and its backward once on tiny inputs there,
    so no kernel is loaded for the first time inside a capture."""
    from .. import _lib

    _lib.library()
    dev = torch.device("cuda", device)
    with torch.cuda.device(dev):
        f = lambda *shape: torch.full(shape, 0.5, device=dev)  # noqa: E731
        idx = torch.zeros(1, 1, dtype=torch.int32, device=dev)
        one = torch.ones(1, 1, dtype=torch.int32, device=dev)
        gather_backward(gather_op(f(1, 4), f(1, 4), f(1, 2, 4), f(1, 1, 4), idx), idx, 2)
        unit = torch.zeros(1, dtype=torch.int32, device=dev)
        out, hidden = mlp_op(f(1, 16), unit, f(1, 16, 4), f(1, 4), f(1, 4, 4), f(1, 4))
        mlp_backward(f(1, 16), unit, f(1, 16, 4), f(1, 4, 4), hidden, out)
        indptr = torch.tensor([0, 1, 1], dtype=torch.int32, device=dev)
        edges = torch.zeros(1, dtype=torch.int32, device=dev)
        m = messages_op(f(1, 2, 4), indptr, edges, f(1), f(4, 4), idx)
        messages_backward(f(1, 2, 4), indptr, edges, f(1), f(4, 4), idx, m)
        age = torch.zeros(1, 2, dtype=torch.int32, device=dev)
        _, _, _, old = update_op(f(1, 2, 4), f(1, 4), age, idx, one, f(1, 1, 4), f(1, 1, 4))
        update_backward(idx, one, f(1, 1, 4), f(1, 1, 4), old, f(1, 2, 4), f(1, 4))
        torch.cuda.synchronize(dev)


def _eager(op: Any, body: Any, *args: Any) -> Any:
    """``op(*args)`` where a gradient can flow or anything traces (a compiled region, a dispatch
    mode such as AOT autograd's, fake or functional tensors); elsewhere (plain tensors, no grad
    mode or no input that requires grad, as in the backward formulas) the op's body itself, with
    the same results: the custom op's dispatch adds its Python autograd and aliasing layers,
    about 10 us, to every call."""
    tensors = [a for a in args if isinstance(a, Tensor)]
    if (torch.compiler.is_compiling() or _get_current_dispatch_mode() is not None
            or any(type(t) not in (Tensor, torch.nn.Parameter) for t in tensors)
            or (torch.is_grad_enabled() and any(t.requires_grad for t in tensors))):
        return op(*args)
    return body(*args)


def _code(t: Tensor) -> int:
    try:
        return _DTYPE[t.dtype]
    except KeyError:
        raise TypeError(f"hsn ops take float32, float16 or bfloat16, not {t.dtype}") from None


def _i32(t: Tensor) -> Tensor:
    """Indices as the ABI takes them: int32, contiguous. An int64 index is clamped into
    [-1, 2^31 - 1] first, so a huge value becomes an out-of-range or padded index instead of
    wrapping into a valid one (the reference's ops.py:307-311)."""
    if t.dtype == torch.int32:
        return t.contiguous()
    if t.dtype != torch.int64:
        raise ValueError(f"indices must be int32 or int64, not {t.dtype}")
    return t.clamp(-1, 2**31 - 1).to(torch.int32).contiguous()


def _flags(t: Tensor) -> Tensor:
    """Per-slot 0/1 flags (bool or integer) as int32."""
    return t.to(torch.int32).contiguous()


def _gather_body(u: Tensor, eps: Tensor, h: Tensor, m: Tensor, idx: Tensor) -> Tensor:
    B, N, d = h.shape
    K = idx.shape[1]
    u, eps, h, m, idx = u.contiguous(), eps.contiguous(), h.contiguous(), m.contiguous(), _i32(idx)
    v = h.new_empty((B, K, 4 * d))
    call("hsn_gather_concat", ptr(u), ptr(eps), ptr(h), ptr(m), ptr(idx), ptr(v), B, N, d, K,
         _code(h), stream_of(h.device))
    return v


@torch.library.custom_op("hsn::gather_concat", mutates_args=(), device_types="cuda")
def gather_op(u: Tensor, eps: Tensor, h: Tensor, m: Tensor, idx: Tensor) -> Tensor:
    """``v[r,k] = [u[r]; eps[r]; h[r, idx[r,k]]; m[r,k]]`` (reference hsn_ops.h:79-87)."""
    return _gather_body(u, eps, h, m, idx)


@gather_op.register_fake
def _gather_fake(u, eps, h, m, idx):
    return h.new_empty((*idx.shape, 4 * h.shape[2]))


def _gather_bwd_body(dv: Tensor, idx: Tensor, n: int) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    B, K, width = dv.shape
    d = width // 4
    dv, idx = dv.contiguous(), _i32(idx)
    du, de = dv.new_empty((B, d)), dv.new_empty((B, d))
    dh, dm = dv.new_empty((B, n, d)), dv.new_empty((B, K, d))
    call("hsn_gather_concat_bwd", ptr(dv), ptr(idx), ptr(du), ptr(de), ptr(dh), ptr(dm), B, n, d,
         K, _code(dv), 1, stream_of(dv.device))
    return du, de, dh, dm


@torch.library.custom_op("hsn::gather_concat_backward", mutates_args=(), device_types="cuda")
def gather_backward(dv: Tensor, idx: Tensor, n: int) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """``(grad_u, grad_eps, grad_h, grad_m)`` of the gather (reference hsn_ops.h:88-99)."""
    return _gather_bwd_body(dv, idx, n)


@gather_backward.register_fake
def _gather_bwd_fake(dv, idx, n):
    B, K, width = dv.shape
    d = width // 4
    return dv.new_empty((B, d)), dv.new_empty((B, d)), dv.new_empty((B, n, d)), dv.new_empty((B, K, d))


def _gather_setup(ctx: Any, inputs: tuple[Any, ...], output: Tensor) -> None:
    ctx.save_for_backward(inputs[4])
    ctx.n = inputs[2].shape[1]


def _gather_grad(ctx: Any, dv: Tensor) -> tuple[Any, ...]:
    return (*_eager(gather_backward, _gather_bwd_body, dv.contiguous(), ctx.saved_tensors[0],
                    ctx.n), None)


gather_op.register_autograd(_gather_grad, setup_context=_gather_setup)


def _update(h: Tensor, q: Tensor, age: Tensor, idx: Tensor, valid: Tensor, c: Tensor,
            b: Tensor) -> Tensor:
    """The in-place update of contiguous ``h, q`` (float) and ``age`` (int32); returns
    ``h_old_saved``."""
    B, N, d = h.shape
    K = idx.shape[1]
    old = torch.empty_like(c, memory_format=torch.contiguous_format)
    call("hsn_gated_delta_update", ptr(h), ptr(q), ptr(age), ptr(_i32(idx)), ptr(_flags(valid)),
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
def update_inplace(h: Tensor, q: Tensor, age: Tensor, idx: Tensor, valid: Tensor, c: Tensor,
                   b: Tensor) -> Tensor:
    """In place on ``h, q, age`` (reference hsn_ops.h:155-171); returns ``h_old_saved``."""
    if any(t.requires_grad for t in (h, q, c, b)) and torch.is_grad_enabled():
        raise RuntimeError("use the functional update for training")
    _check_inplace(h, q, age)
    return _update(h, q, age, idx, valid, c, b)


@update_inplace.register_fake
def _update_inplace_fake(h, q, age, idx, valid, c, b):
    return torch.empty_like(c)


def _functional(h, q, age, idx, valid, c, b):
    hn = h.clone(memory_format=torch.contiguous_format)
    qn = q.clone(memory_format=torch.contiguous_format)
    if age.dtype == torch.int32:
        an = age.clone(memory_format=torch.contiguous_format)
        old = _update(hn, qn, an, idx, valid, c, b)
        return hn, qn, an, old
    # wider ages stay exact: the kernel zeroes the selected cells of an int32 mask of ones, and
    # the same cells' ages are zeroed in the caller's dtype
    keep = torch.ones(age.shape, dtype=torch.int32, device=age.device)
    old = _update(hn, qn, keep, idx, valid, c, b)
    return hn, qn, age.masked_fill(keep == 0, 0), old


@torch.library.custom_op("hsn::gated_delta_update_functional", mutates_args=(),
                         device_types="cuda")
def update_op(h: Tensor, q: Tensor, age: Tensor, idx: Tensor, valid: Tensor, c: Tensor,
              b: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """``(h', q', age', h_old_saved)`` without touching the inputs."""
    return _functional(h, q, age, idx, valid, c, b)


@update_op.register_fake
def _update_fake(h, q, age, idx, valid, c, b):
    return torch.empty_like(h), torch.empty_like(q), torch.empty_like(age), torch.empty_like(c)


@torch.library.custom_op("hsn::gated_delta_update_state", mutates_args=(), device_types="cuda")
def state_update_op(h: Tensor, q: Tensor, age: Tensor, idx: Tensor, valid: Tensor, c: Tensor,
                    b: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """The state-producing form (the reference's op 8): the same outputs as the functional
    update, written into fresh tensors."""
    return _functional(h, q, age, idx, valid, c, b)


@state_update_op.register_fake
def _state_update_fake(h, q, age, idx, valid, c, b):
    return torch.empty_like(h), torch.empty_like(q), torch.empty_like(age), torch.empty_like(c)


def _update_bwd_body(idx: Tensor, valid: Tensor, c: Tensor, b: Tensor, old: Tensor, G: Tensor,
                     g: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    B, N, d = G.shape
    K = idx.shape[1]
    c, b, old, G, g = c.contiguous(), b.contiguous(), old.contiguous(), G.contiguous(), g.contiguous()
    dh, dq = torch.empty_like(G), torch.empty_like(g)
    dc, db = torch.empty_like(c), torch.empty_like(b)
    call("hsn_gated_delta_update_bwd", ptr(_i32(idx)), ptr(_flags(valid)), ptr(c), ptr(b), ptr(old),
         ptr(G), ptr(g), ptr(dh), ptr(dq), ptr(dc), ptr(db), B, N, d, K, _code(G),
         stream_of(G.device))
    return dh, dq, dc, db


@torch.library.custom_op("hsn::gated_delta_update_backward", mutates_args=(), device_types="cuda")
def update_backward(idx: Tensor, valid: Tensor, c: Tensor, b: Tensor, old: Tensor, G: Tensor,
                    g: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """``(grad_h, grad_q, grad_c, grad_b)`` from ``grad_h_out = G``, ``grad_q_out = g``
    (reference hsn_ops.h:173-187)."""
    return _update_bwd_body(idx, valid, c, b, old, G, g)


@update_backward.register_fake
def _update_bwd_fake(idx, valid, c, b, old, G, g):
    return torch.empty_like(G), torch.empty_like(g), torch.empty_like(c), torch.empty_like(b)


def _update_setup(ctx: Any, inputs: tuple[Any, ...], output: tuple[Tensor, ...]) -> None:
    _, _, _, idx, valid, c, b = inputs
    ctx.save_for_backward(idx, valid, c, b, output[3])
    ctx.mark_non_differentiable(output[2], output[3])


def _update_grad(ctx: Any, G: Tensor, g: Tensor, dage: Tensor, dold: Tensor) -> tuple[Any, ...]:
    dh, dq, dc, db = _eager(update_backward, _update_bwd_body, *ctx.saved_tensors,
                            G.contiguous(), g.contiguous())
    return dh, dq, None, None, None, dc, db


update_op.register_autograd(_update_grad, setup_context=_update_setup)
state_update_op.register_autograd(_update_grad, setup_context=_update_setup)


# --------------------------------------------------------------------------------------------
# the grouped unit MLP (reference python/hsn/kernels/ops.py:133-180)
# --------------------------------------------------------------------------------------------


def _mlp_body(v: Tensor, idx: Tensor, w1: Tensor, b1: Tensor, w2: Tensor,
              b2: Tensor) -> tuple[Tensor, Tensor]:
    P, M, d, H = v.shape[0], w1.shape[0], w2.shape[2], w1.shape[2]
    v, idx, w1, b1, w2, b2 = (v.contiguous(), _i32(idx), w1.contiguous(), b1.contiguous(),
                              w2.contiguous(), b2.contiguous())
    out, hidden = v.new_empty((P, d)), v.new_empty((P, H))
    call("hsn_grouped_unit_mlp_fwd", ptr(v), ptr(idx), ptr(w1), ptr(b1), ptr(w2), ptr(b2),
         ptr(hidden), ptr(out), P, M, d, H, _code(v), stream_of(v.device))
    return out, hidden


@torch.library.custom_op("hsn::grouped_unit_mlp", mutates_args=(), device_types="cuda")
def mlp_op(v: Tensor, idx: Tensor, w1: Tensor, b1: Tensor, w2: Tensor,
           b2: Tensor) -> tuple[Tensor, Tensor]:
    """``(out [P,d], hidden [P,H])``: unit ``idx[p]`` on pair ``p``, ``hidden`` the saved
    pre-GELU ``z1`` (reference hsn_ops.h:101-112)."""
    return _mlp_body(v, idx, w1, b1, w2, b2)


@mlp_op.register_fake
def _mlp_fake(v, idx, w1, b1, w2, b2):
    return v.new_empty((v.shape[0], w2.shape[2])), v.new_empty((v.shape[0], w1.shape[2]))


def _mlp_bwd_body(v: Tensor, idx: Tensor, w1: Tensor, w2: Tensor, hidden: Tensor,
                  dout: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    P, M, d, H = v.shape[0], w1.shape[0], w2.shape[2], w1.shape[2]
    v, idx, w1, w2, hidden, dout = (v.contiguous(), _i32(idx), w1.contiguous(), w2.contiguous(),
                                    hidden.contiguous(), dout.contiguous())
    dv, dw1, dw2 = torch.empty_like(v), torch.empty_like(w1), torch.empty_like(w2)
    db1, db2 = w1.new_empty((M, H)), w2.new_empty((M, d))
    call("hsn_grouped_unit_mlp_bwd", ptr(v), ptr(idx), ptr(w1), ptr(w2), ptr(hidden), ptr(dout),
         ptr(dv), ptr(dw1), ptr(db1), ptr(dw2), ptr(db2), P, M, d, H, _code(v), 1,
         stream_of(v.device))
    return dv, dw1, db1, dw2, db2


@torch.library.custom_op("hsn::grouped_unit_mlp_backward", mutates_args=(), device_types="cuda")
def mlp_backward(v: Tensor, idx: Tensor, w1: Tensor, w2: Tensor, hidden: Tensor,
                 dout: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """``(dv, dw1, db1, dw2, db2)`` from the saved ``z1`` (reference hsn_ops.h:114-130)."""
    return _mlp_bwd_body(v, idx, w1, w2, hidden, dout)


@mlp_backward.register_fake
def _mlp_bwd_fake(v, idx, w1, w2, hidden, dout):
    return (torch.empty_like(v), torch.empty_like(w1), w1.new_empty((w1.shape[0], w1.shape[2])),
            torch.empty_like(w2), w2.new_empty((w2.shape[0], w2.shape[2])))


def _mlp_setup(ctx: Any, inputs: tuple[Any, ...], output: tuple[Tensor, Tensor]) -> None:
    v, idx, w1, _, w2, _ = inputs
    ctx.save_for_backward(v, idx, w1, w2, output[1])
    ctx.mark_non_differentiable(output[1])


def _mlp_grad(ctx: Any, dout: Tensor, dhidden: Tensor) -> tuple[Any, ...]:
    dv, dw1, db1, dw2, db2 = _eager(mlp_backward, _mlp_bwd_body, *ctx.saved_tensors,
                                    dout.contiguous())
    return dv, None, dw1, db1, dw2, db2


mlp_op.register_autograd(_mlp_grad, setup_context=_mlp_setup)


# --------------------------------------------------------------------------------------------
# the CSR neighbour messages (reference python/hsn/kernels/ops.py:183-221)
# --------------------------------------------------------------------------------------------


def _messages_body(h: Tensor, indptr: Tensor, indices: Tensor, a: Tensor, V: Tensor,
                   idx: Tensor) -> Tensor:
    B, N, d = h.shape
    K, E = idx.shape[1], a.numel()
    h, indptr, indices, a, V, idx = (h.contiguous(), _i32(indptr), _i32(indices), a.contiguous(),
                                     V.contiguous(), _i32(idx))
    m = h.new_empty((B, K, d))
    call("hsn_csr_messages", ptr(h), ptr(indptr), ptr(indices), ptr(a), ptr(V), ptr(idx), ptr(m),
         B, N, d, K, E, _code(h), stream_of(h.device))
    return m


@torch.library.custom_op("hsn::csr_messages", mutates_args=(), device_types="cuda")
def messages_op(h: Tensor, indptr: Tensor, indices: Tensor, a: Tensor, V: Tensor,
                idx: Tensor) -> Tensor:
    """``m [B,K,d]``: ``m[r,k] = sum_e a[e] (V h[r, indices[e]])`` over the edges of row
    ``idx[r,k]`` (reference hsn_ops.h:132-143)."""
    return _messages_body(h, indptr, indices, a, V, idx)


@messages_op.register_fake
def _messages_fake(h, indptr, indices, a, V, idx):
    return h.new_empty((*idx.shape, h.shape[2]))


def _messages_bwd_body(h: Tensor, indptr: Tensor, indices: Tensor, a: Tensor, V: Tensor,
                       idx: Tensor, dm: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    B, N, d = h.shape
    K, E = idx.shape[1], a.numel()
    h, indptr, indices, a, V, idx, dm = (h.contiguous(), _i32(indptr), _i32(indices),
                                         a.contiguous(), V.contiguous(), _i32(idx),
                                         dm.contiguous())
    dh, da, dV = torch.empty_like(h), torch.empty_like(a), torch.empty_like(V)
    call("hsn_csr_messages_bwd", ptr(h), ptr(indptr), ptr(indices), ptr(a), ptr(V), ptr(idx),
         ptr(dm), ptr(dh), ptr(da), ptr(dV), B, N, d, K, E, _code(h), 1, stream_of(h.device))
    return dh, da, dV


@torch.library.custom_op("hsn::csr_messages_backward", mutates_args=(), device_types="cuda")
def messages_backward(h: Tensor, indptr: Tensor, indices: Tensor, a: Tensor, V: Tensor,
                      idx: Tensor, dm: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """``(dh, da, dV)`` of the messages (reference hsn_ops.h:145-153)."""
    return _messages_bwd_body(h, indptr, indices, a, V, idx, dm)


@messages_backward.register_fake
def _messages_bwd_fake(h, indptr, indices, a, V, idx, dm):
    return torch.empty_like(h), torch.empty_like(a), torch.empty_like(V)


def _messages_setup(ctx: Any, inputs: tuple[Any, ...], output: Tensor) -> None:
    ctx.save_for_backward(*inputs)


def _messages_grad(ctx: Any, dm: Tensor) -> tuple[Any, ...]:
    dh, da, dV = _eager(messages_backward, _messages_bwd_body, *ctx.saved_tensors,
                        dm.contiguous())
    return dh, None, None, da, dV, None


messages_op.register_autograd(_messages_grad, setup_context=_messages_setup)


# --------------------------------------------------------------------------------------------
# the KernelOps adapters (reference python/hsn/kernels/ops.py:320-444, the protocol of
# python/hsn/kernels/__init__.py:56-103)
# --------------------------------------------------------------------------------------------

_fallback: Any = None


def set_fallback(backend: Any) -> None:
    """The backend that takes the calls the adapters decline: a module or object with the four
    ``KernelOps`` functions. ``None`` restores the default, the reference's
    ``hsn.kernels.native``, imported at the first declined call."""
    global _fallback
    _fallback = backend


def _declined(name: str, why: str) -> Any:
    """The fallback's function ``name``, for a call this library does not take (``why``)."""
    global _fallback
    if _fallback is None:
        try:
            import importlib

            _fallback = importlib.import_module("hsn.kernels.native")
        except ImportError:
            raise NotImplementedError(
                f"hsn_amd.kernels.ops.{name}: the library does not take this call ({why}) and no "
                "fallback backend is set (set_fallback, or install the reference's hsn package)"
            ) from None
    return getattr(_fallback, name)


def _on_device(t: Tensor) -> bool:
    """A tensor the library's ABI takes: on the GPU, in one of its three float dtypes."""
    return t.is_cuda and t.dtype in _DTYPE


def _autocast() -> bool:
    return torch.is_autocast_enabled("cuda")


def _dtype_for(t: Tensor) -> torch.dtype:
    """The dtype the ops compute ``t``'s call in: autocast's for fp32 inputs under autocast."""
    return torch.get_autocast_dtype("cuda") if _autocast() and t.dtype == torch.float32 else t.dtype


def gather_concat(u: Optional[Tensor], eps: Tensor, h: Tensor, m: Tensor, cell_idx: Tensor) -> Tensor:
    """``v [B, K, 4d] = [u; eps; h[cell_idx]; m]`` of the selected cells (``m`` cast to ``h``'s
    dtype). ``u=None`` (the three-block input ``[eps; h; m]``) and tensors off the GPU go to the
    fallback: the ABI's input is four blocks wide."""
    if u is None or not _on_device(h):
        why = "a three-block input (u=None)" if u is None else "h off the GPU or of another dtype"
        return _declined("gather_concat", why)(u, eps, h, m, cell_idx)
    if u.dtype != h.dtype or eps.dtype != h.dtype:
        raise ValueError("u, eps and h must have the same state dtype")
    return _eager(gather_op, _gather_body, u.contiguous(), eps.contiguous(), h.contiguous(),
                  m.to(h.dtype).contiguous(), _i32(cell_idx))


def grouped_unit_mlp(v: Tensor, unit_idx: Tensor, bank: Any, *, static: bool = False,
                     w1_flat: Optional[Tensor] = None) -> Tensor:
    """``out [P, d]``: unit ``unit_idx[p]`` of ``bank`` (its ``W1 [M, 4d, H]``, ``b1``,
    ``W2 [M, H, d]``, ``b2``) on pair ``p``, GELU between the layers. ``w1_flat [4d, M H]``, when
    given, replaces ``bank.W1`` (the bank's flat first-layer weight). Unless ``static``, a unit
    outside the bank raises ``IndexError`` (one device synchronisation).

    The fallback takes: autocast (its reduced-precision intermediates are not what the ABI's
    fp32 intermediates give), an activation other than GELU, an input width other than 4d, and
    tensors off the GPU."""
    why = None
    if not _on_device(v):
        why = "v off the GPU or of another dtype"
    elif bank.activation_name != "gelu":
        why = f"the {bank.activation_name} activation"
    elif _autocast():
        why = "autocast"
    elif bank.in_dim != 4 * bank.d:
        why = f"an input width of {bank.in_dim} (the ABI's is 4d = {4 * bank.d})"
    if why is not None:
        return _declined("grouped_unit_mlp", why)(v, unit_idx, bank, static=static, w1_flat=w1_flat)
    if not static:
        lo, hi = (int(x) for x in torch.stack([unit_idx.min(), unit_idx.max()]).tolist())
        if lo < 0 or hi >= bank.n_units:
            raise IndexError(f"unit_idx outside the unit bank: values in [{lo}, {hi}], "
                             f"{bank.n_units} units")
    dtype = _dtype_for(v)
    # the master weights are cast per call and never cached in another dtype: their gradients
    # reach the masters through the cast
    w1 = bank.W1 if w1_flat is None else \
        w1_flat.reshape(bank.in_dim, bank.n_units, bank.hidden).permute(1, 0, 2)
    out, _ = _eager(mlp_op, _mlp_body, v.to(dtype).contiguous(), _i32(unit_idx),
                    w1.to(dtype).contiguous(), bank.b1.to(dtype).contiguous(),
                    bank.W2.to(dtype).contiguous(), bank.b2.to(dtype).contiguous())
    return out


def csr_messages(h: Tensor, graph: Any, V: Any, cell_idx: Tensor, *,
                 weights: Optional[Tensor] = None, validate: bool = True) -> Tensor:
    """``m [B, K, d]``: for each selected cell the edge-weighted sum of ``V h`` over its
    in-neighbours in ``graph`` (a CSR ``indptr`` / ``indices`` by target). The edge weights are
    ``graph.edge_weights()``, or ``weights`` in the padded ``[N, D]`` layout gathered at the
    graph's edge positions; ``V`` is a bias-free linear map. The graph checks ``h`` and
    ``cell_idx`` itself (``validate``: with their values). Autocast and tensors off the GPU go to
    the fallback."""
    if not _on_device(h) or _autocast():
        why = "autocast" if _on_device(h) else "h off the GPU or of another dtype"
        return _declined("csr_messages", why)(h, graph, V, cell_idx, weights=weights,
                                              validate=validate)
    B = graph._check_h(h)[0]
    graph._check_cell_idx(cell_idx, B, check_values=validate)
    if V.bias is not None:
        raise ValueError("CSR messages need a projection without bias")
    a = graph.edge_weights() if weights is None else weights.reshape(-1)[graph._edge_pos]
    dtype = _dtype_for(h)
    return _eager(messages_op, _messages_body, h.to(dtype).contiguous(), _i32(graph.indptr),
                  _i32(graph.indices), a.to(dtype).contiguous(), V.weight.to(dtype).contiguous(),
                  _i32(cell_idx))


def _check_valid(valid: Any, shape: tuple, device: torch.device) -> None:
    if not isinstance(valid, Tensor):
        raise TypeError(f"valid must be a torch.Tensor, not {type(valid).__name__}")
    if valid.dtype != torch.bool:
        raise ValueError(f"valid must have dtype torch.bool, got {valid.dtype}")
    if tuple(valid.shape) != tuple(shape):
        raise ValueError(f"valid must have shape {tuple(shape)}, got {tuple(valid.shape)}")
    if valid.device != device:
        raise ValueError(f"valid must be on {device}, got {valid.device}")


def _check_selection(cell_idx: Tensor, valid: Tensor, n_cells: int) -> None:
    """The valid slots name cells in ``[0, n_cells)``, distinct within each row; one device
    synchronisation. Invalid slots are ignored."""
    B, K = (int(n) for n in cell_idx.shape)
    if B * K == 0:
        return
    ids = cell_idx.to(torch.int64)
    lo = torch.where(valid, ids, torch.full_like(ids, n_cells)).amin()
    hi = torch.where(valid, ids, torch.full_like(ids, -1)).amax()
    # a padded slot takes a key of its own past every cell, so only valid repeats compare equal
    keys = torch.where(valid, ids, n_cells + torch.arange(K, device=ids.device).expand(B, K))
    keys = keys.sort(dim=1).values
    repeats = (keys[:, 1:] == keys[:, :-1]).sum()
    lo, hi, repeats = (int(x) for x in torch.stack([lo, hi, repeats]).tolist())
    if lo < 0 or hi >= n_cells:
        raise IndexError(f"valid cell_idx entries must lie in [0, {n_cells}), got values in "
                         f"[{lo}, {hi}]")
    if repeats:
        raise ValueError(f"valid cell_idx entries must be distinct within each row ({repeats} "
                         "repeated)")


def _with_state(like: Any, h: Tensor, q: Tensor, age: Tensor, pos: Tensor) -> Any:
    """A state of ``like``'s type holding the four tensors: the reference's ``CellGraphState``
    through its unchecked constructor ``_make(h, q, age, pos)``, a named tuple (this package's
    :class:`hsn_amd.state.CellGraphState`) field by field."""
    if isinstance(like, tuple):
        return type(like)(h, q, age, pos)
    return type(like)._make(h, q, age, pos)


def gated_delta_update(state: Any, cell_idx: Tensor, c: Tensor, b: Tensor, valid: Tensor, *,
                       validate: bool = True) -> Any:
    """The next state after every valid slot's gated update ``h[cell] <- (1 - b) h[cell] + b c``
    (``q`` follows by the slots' deltas over N; a selected cell's age restarts at 0; ``pos`` is
    kept). ``valid [B, K]`` is bool on the state's device; ``validate`` checks the valid slots'
    cells for range and repeats. A state off the GPU, or ``c`` / ``b`` in another dtype than the
    state's (the ABI has one dtype), goes to the fallback."""
    h = state.h
    if not _on_device(h) or c.dtype != h.dtype or b.dtype != h.dtype:
        why = "the state off the GPU" if not _on_device(h) else "c or b in another dtype than the state"
        return _declined("gated_delta_update", why)(state, cell_idx, c, b, valid, validate=validate)
    _check_valid(valid, tuple(cell_idx.shape), h.device)
    if validate:
        _check_selection(cell_idx, valid, int(h.shape[1]))
    hn, qn, age, _ = _eager(state_update_op, _functional, h.contiguous(), state.q.contiguous(),
                            state.age.contiguous(), _i32(cell_idx), _flags(valid), c.contiguous(),
                            b.contiguous())
    return _with_state(state, hn, qn, age, state.pos)
