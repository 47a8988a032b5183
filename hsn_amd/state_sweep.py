"""The state-gradient reverse sweep (P2.10c) on MI355X: the reference's
``python/hsn/train/state_sweep.py`` (``ReverseSweep``, ``SweepRunner``, ``out_adjacency``,
``sweep_shape``) on the HIP glue steps of ``include/hsn_sweep.h``.

A window's sweep walks its positions ``T - 1 .. 0``; a position is the head, the first
transposed product, the middle, the second product and the tail. The glue steps are the
library's kernels (``hsn_win_back_head`` / ``_mid`` / ``_tail``); the products are plain GEMMs
(``torch.mm``, hipBLASLt) on the operands the glue writes, with ``W_out`` folded into the second
layer's transposed weights and the cell norm's gain and ``V`` into the first layer's, once per
window (state_sweep.py:226-248). Every buffer is allocated once per shape, so the loop over the
positions is captured once as a HIP graph and replayed for every window (``capture``).

:class:`SweepRunner` is the reference's plug-in: installed with the reference's
``hsn.train.state_gradient.set_fast_sweep``, it is called with ``state_gradient_backward``'s
arguments and returns ``(dL/dc, dL/db)``, or ``None`` for what it does not take (another device,
a state dtype other than fp32, products other than fp32 / bf16, the row limit, a shape the
kernels do not take); the caller then runs its PyTorch sweep. There is no other implementation
here: a missing or stale library raises.
"""

from __future__ import annotations

import ctypes
from typing import Any, NamedTuple, Optional

import torch
from torch import Tensor

from . import _lib

__all__ = [
    "ACTIVATION_CODES",
    "CellConstants",
    "ReverseSweep",
    "SweepRunner",
    "SweepShape",
    "back_unsupported",
    "out_adjacency",
    "sweep_shape",
]

#: ``model.activation`` as the kernels' code (include/hsn_sweep.h HSN_ACT_*).
ACTIVATION_CODES: dict[str, int] = {"gelu": 0, "relu": 1, "silu": 2, "tanh": 3}


class CellConstants(NamedTuple):
    """What the sweep reads of the cell's weights: the fields of the reference's
    ``hsn.train.state_gradient.CellConstants`` (state_gradient.py:134-156), which the runner
    takes as well. ``w_out [d, d]`` (y = F @ w_out.T), ``cand_gain [d]`` or None, ``cand_eps``,
    ``w2 [M, H, d]``, ``w1_state [M, 2d, H]`` (the first layer at the state columns), ``b1 [M,
    H]``, ``gate_state [d, 2d]``, ``gate_bias [d]``, ``norm_gain_state [2d]`` or None,
    ``in_dim``, ``v [d, d]`` (V h = h @ v.T), ``edge_weights [N, D]``, ``pad_src [N, D]``,
    ``activation``, ``pad_mask [N, D]``."""

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


class SweepShape(NamedTuple):
    """The sizes a :class:`ReverseSweep` is built for (the reference's ``SweepShape``,
    state_sweep.py:71-83). ``n_fast`` leading slots have a fixed unit (here they take the
    all-units layout like the others: the same arithmetic); ``n_read`` cells ``0 .. n_read-1`` are
    read after every position; ``d_out`` is the largest number of cells one cell is a message
    source of."""

    B: int
    T: int
    K: int
    N: int
    d: int
    H: int
    M: int
    n_fast: int
    n_read: int
    in_dim: int
    d_out: int


def out_adjacency(pad_src: Tensor, pad_mask: Tensor) -> tuple[Tensor, Tensor]:
    """The message graph by source, for the reverse sweep's scatter to message sources
    (interface and order of the reference's state_sweep.py:89-109): ``out_edge [N, D_out]``
    holds each out-edge of cell ``n`` as its index ``target * D + slot`` into the padded
    ``[N, D]`` view, ascending (by target, then slot), and ``out_tgt [N, D_out]`` its target;
    rows are padded with -1 targets and edge 0, and ``D_out`` is the largest out-degree (1 at
    least).

    The real edges' flat indices come out of the mask already ascending, so one sort of the
    composite key ``source * N * D + flat`` groups them by source in that order; an edge's
    column is its distance from the first edge of its source in the sorted list."""
    N, D = (int(n) for n in pad_src.shape)
    dev = pad_src.device
    flat = pad_mask.reshape(-1).nonzero().reshape(-1)  # real edges, ascending flat index
    source = pad_src.reshape(-1)[flat].to(torch.int64)
    if source.numel() and bool(((source < 0) | (source >= N)).any()):
        raise ValueError("a message source lies outside [0, N)")
    key, perm = torch.sort(source * (N * D) + flat)
    source, flat = key // (N * D), flat[perm]
    column = torch.arange(flat.numel(), device=dev) - torch.searchsorted(source, source)
    d_out = int(column.max()) + 1 if column.numel() else 1
    out_edge = torch.zeros((N, d_out), dtype=torch.int64, device=dev)
    out_edge[source, column] = flat
    out_tgt = torch.full((N, d_out), -1, dtype=torch.int64, device=dev)
    out_tgt[source, column] = flat // D
    return out_tgt, out_edge


def _graph_token(pad_src: Tensor, pad_mask: Tensor) -> tuple:
    """What identifies a message graph between windows: both tensors and their version counters
    (an in-place change of either bumps its counter, so a cached adjacency is rebuilt)."""
    return (pad_src, pad_src._version, pad_mask, pad_mask._version)


def _same_graph(token: Optional[tuple], pad_src: Tensor, pad_mask: Tensor) -> bool:
    return (token is not None and token[0] is pad_src and token[1] == pad_src._version
            and token[2] is pad_mask and token[3] == pad_mask._version)


def sweep_shape(c: Tensor, record: dict[str, Tensor], consts: Any, n_cells: int, n_fast: int,
                n_read: int, d_out: Optional[int] = None) -> SweepShape:
    """The :class:`SweepShape` of a window's sweep arguments (state_sweep.py:531-560); ``d_out``
    the message graph's out-degree when the caller knows it (else computed)."""
    B, T, K, d = (int(n) for n in c.shape)
    if consts.pad_mask is None:
        raise ValueError("the reverse sweep needs the graph's padding mask (pad_mask)")
    if d_out is None:
        d_out = int(out_adjacency(consts.pad_src, consts.pad_mask)[0].shape[1])
    return SweepShape(B=B, T=T, K=K, N=int(n_cells), d=d, H=int(record["hidden"].shape[-1]),
                      M=int(consts.w2.shape[0]), n_fast=int(n_fast), n_read=int(n_read),
                      in_dim=int(consts.in_dim), d_out=d_out)


class _Struct(ctypes.Structure):
    """``hsn_back_sweep`` (include/hsn_sweep.h), field for field."""

    _fields_ = [(name, ctypes.c_int32) for name in (
        "B", "T", "K", "N", "d", "H", "M", "n_read", "in_dim", "d_out", "d_in", "product_dtype",
        "activation", "cand_norm", "cell_norm")] + [("cand_eps", ctypes.c_float)] + [
        (name, ctypes.c_void_p) for name in (
            "A", "R", "sigma", "c", "b", "h_old", "y", "gate_pre", "mv", "alpha", "rms", "hidden",
            "slots", "units", "reset", "d_q_pre", "d_q_post", "d_h_sel", "d_h_fast", "cand_gain",
            "gate_bias", "b1", "out_tgt", "out_w", "in_src", "op1", "op2", "act", "dv", "dc",
            "db", "w2f", "w1f", "carry", "ds")]


def _product_code(dtype: torch.dtype) -> int:
    return {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16}.get(dtype, -1)


def back_unsupported(shape: SweepShape, *, d_in: int = 1, product_dtype: torch.dtype = torch.float32,
                     activation: str = "gelu", cand_norm: bool = True,
                     cell_norm: bool = True) -> Optional[str]:
    """Why the glue kernels cannot take this sweep (``None``: they can), from the library's own
    check (``hsn_win_back_check``; host arithmetic only, no GPU). The reference's
    ``back_unsupported`` (python/hsn/kernels/window.py:1165-1176)."""
    if activation not in ACTIVATION_CODES:
        return f"model.activation={activation!r} has no kernel"
    s = _Struct()
    for name, value in (("B", shape.B), ("T", shape.T), ("K", shape.K), ("N", shape.N),
                        ("d", shape.d), ("H", shape.H), ("M", shape.M), ("n_read", shape.n_read),
                        ("in_dim", shape.in_dim), ("d_out", shape.d_out), ("d_in", d_in),
                        ("product_dtype", _product_code(product_dtype)),
                        ("activation", ACTIVATION_CODES[activation]),
                        ("cand_norm", int(cand_norm)), ("cell_norm", int(cell_norm))):
        setattr(s, name, int(value))
    s.cand_eps = 1e-6
    for name, _ in _Struct._fields_[16:]:  # placeholders: the check reads no memory
        setattr(s, name, 1)
    lib = _lib.library()
    if lib.hsn_win_back_check(ctypes.byref(s)) == _lib.HSN_OK:
        return None
    return lib.hsn_win_last_error().decode(errors="replace")


class ReverseSweep:
    """The reverse sweep of one window shape on static buffers (state_sweep.py:112-528), its glue
    steps on the HIP kernels. ``load`` copies a window's record, cotangents and weights into the
    buffers; ``run`` walks the positions and returns ``(dc, db)`` (the buffers: the next ``load``
    overwrites them). ``product_dtype`` is the products' and their operands' dtype (bf16 under
    autocast, else fp32). Raises ``ValueError`` for what the kernels do not take."""

    def __init__(self, shape: SweepShape, consts: Any, *, device: torch.device,
                 state_dtype: torch.dtype = torch.float32,
                 product_dtype: torch.dtype = torch.float32, limits: Any = None,
                 fused: Optional[bool] = None) -> None:
        B, T, K, N, d, H, M, F, n_read, n, d_out = shape
        if device.type != "cuda":
            raise ValueError("the reverse sweep's kernels run on a ROCm device")
        if state_dtype != torch.float32:
            raise ValueError("the reverse sweep's kernels keep the state's cotangent in fp32")
        if limits is not None:
            raise ValueError("the row limit's step has no kernel")
        if not 0 <= F < K:
            raise ValueError(f"n_fast={F} must leave a routed slot of the {K} slots")
        if consts.pad_mask is None:
            raise ValueError("the reverse sweep needs the graph's padding mask (pad_mask)")
        self.shape = shape
        self.device = device
        self.state_dtype = state_dtype
        self.product_dtype = product_dtype
        self.activation = consts.activation
        self.cand_norm = consts.cand_gain is not None
        self.cand_eps = float(consts.cand_eps)
        self.cell_norm = consts.norm_gain_state is not None
        self.d_in = int(consts.pad_src.shape[1])
        why = back_unsupported(shape, d_in=self.d_in, product_dtype=product_dtype,
                               activation=self.activation, cand_norm=self.cand_norm,
                               cell_norm=self.cell_norm)
        if why is not None:
            raise ValueError(f"the reverse sweep's kernels do not take this sweep: {why}")
        f32 = dict(dtype=torch.float32, device=device)
        prod = dict(dtype=product_dtype, device=device)
        i32 = dict(dtype=torch.int32, device=device)
        rows = B * K
        self.A, self.R, self.sigma = torch.zeros(B, N, d, **f32), torch.zeros(B, d, **f32), \
            torch.zeros(B, K, **f32)
        # the cotangents entering the window (after its last position), kept apart from the
        # running A and R so that every pass, eager or replayed, starts from them
        self.A_in, self.R_in = torch.zeros(B, N, d, **f32), torch.zeros(B, d, **f32)
        self.c, self.b, self.h_old = (torch.zeros(B, T, K, d, **f32) for _ in range(3))
        self.y, self.gate_pre, self.mv = (torch.zeros(B, T, K, d, **f32) for _ in range(3))
        self.alpha, self.rms = torch.ones(B, T, K, **f32), torch.ones(B, T, K, **f32)
        self.hidden = torch.zeros(B, T, K, H, **prod)
        self.slots, self.units = torch.full((B, T, K), -1, **i32), torch.zeros(B, T, K, **i32)
        self.reset = torch.zeros(B, T, dtype=torch.uint8, device=device)
        self.d_q_pre, self.d_q_post = torch.zeros(B, T, d, **f32), torch.zeros(B, T, d, **f32)
        self.d_h_sel = torch.zeros(B, T, K, d, **f32)
        self.d_h_fast = torch.zeros(B, T, max(n_read, 1), d, **f32)
        self.cand_gain, self.gate_bias = torch.ones(d, **f32), torch.zeros(d, **f32)
        self.b1 = torch.zeros(M, H, **f32)
        self.w2_t = torch.zeros(M * d, H, **prod)
        self.w1_state_t = torch.zeros(M * H + d, 2 * d, **prod)
        self.out_tgt = torch.full((N, d_out), -1, **i32)
        self.out_w = torch.zeros(N, d_out, **f32)
        self.in_src = torch.full((N, self.d_in), -1, **i32)
        self._graph_of: Optional[tuple] = None  # the message graph the adjacency was built from
        self.op1, self.op2 = torch.zeros(rows, M * d, **prod), torch.zeros(rows, M * H + d, **prod)
        self.act, self.dv = torch.zeros(rows, H, **prod), torch.zeros(rows, 2 * d, **prod)
        self.dc, self.db = torch.zeros(B, T, K, d, **f32), torch.zeros(B, T, K, d, **f32)
        self.w2f = torch.zeros(M, H, d, **prod)
        self.w1f = torch.zeros(M, 2 * d, H + d, **prod)
        self.carry = torch.zeros(rows, d, **f32)
        self.ds = torch.zeros(rows, 2 * d, **f32)
        self._graph: Optional[torch.cuda.CUDAGraph] = None
        s = _Struct()
        for name, value in (("B", B), ("T", T), ("K", K), ("N", N), ("d", d), ("H", H), ("M", M),
                            ("n_read", n_read), ("in_dim", n), ("d_out", d_out),
                            ("d_in", self.d_in), ("product_dtype", _product_code(product_dtype)),
                            ("activation", ACTIVATION_CODES[self.activation]),
                            ("cand_norm", int(self.cand_norm)), ("cell_norm", int(self.cell_norm))):
            setattr(s, name, int(value))
        s.cand_eps = self.cand_eps
        for name in ("A", "R", "sigma", "c", "b", "h_old", "y", "gate_pre", "mv", "alpha", "rms",
                     "hidden", "slots", "units", "reset", "d_q_pre", "d_q_post", "d_h_sel",
                     "cand_gain", "gate_bias", "b1", "out_tgt", "out_w", "in_src", "op1", "op2",
                     "act", "dv", "dc", "db", "w2f", "w1f", "carry", "ds"):
            setattr(s, name, getattr(self, name).data_ptr())
        s.d_h_fast = self.d_h_fast.data_ptr() if n_read else None
        self._struct = s
        _lib.call("hsn_win_back_check", ctypes.byref(s))
        lib = _lib.library()
        takes_fused = lib.hsn_win_back_cell_check(ctypes.byref(s)) == _lib.HSN_OK
        if fused and not takes_fused:
            raise ValueError("the fused step does not take this sweep: "
                             + lib.hsn_win_last_error().decode(errors="replace"))
        #: One launch for the head, both products and the middle (``hsn_win_back_cell``), with
        #: only each unit's own blocks multiplied; else the reference's three glue steps around
        #: two all-units GEMMs.
        self.fused = takes_fused if fused is None else bool(fused)

    # -- loading a window ------------------------------------------------------------------------

    def load_weights(self, consts: Any) -> None:
        """The cell's weights of this window, folded for the products (state_sweep.py:216-262):
        ``w2_t`` row ``j d + k`` is unit j's ``(W_out W2_j^T)[k]`` (the candidate's ``W_out`` in the
        second layer), ``w1_state_t`` is ``[W1_s; G_s]^T`` times ``blockdiag(diag(g_h), diag(g_m) V)``
        (the cell norm's gain and ``V`` after the first layer)."""
        s = self.shape
        d, M, H = s.d, s.M, s.H
        w_out = consts.w_out.to(self.device, torch.float32)
        w2 = consts.w2.to(self.device, torch.float32)  # [M, H, d]
        w2_t = w2.permute(0, 2, 1).reshape(M, d, H)
        self.w2_t.copy_(torch.matmul(w_out, w2_t).reshape(M * d, H))  # row j d + k
        w1 = consts.w1_state.to(self.device, torch.float32)  # [M, 2d, H]
        w1_t = torch.cat([w1.permute(0, 2, 1).reshape(M * H, 2 * d),
                          consts.gate_state.to(self.device, torch.float32)], dim=0)
        fold = torch.zeros(2 * d, 2 * d, dtype=torch.float32, device=self.device)
        v = consts.v.to(self.device, torch.float32)
        gain = consts.norm_gain_state
        if gain is None:
            fold[:d, :d] = torch.eye(d, dtype=torch.float32, device=self.device)
            fold[d:, d:] = v
        else:
            gain = gain.to(self.device, torch.float32)
            fold[:d, :d] = torch.diag(gain[:d])
            fold[d:, d:] = gain[d:, None] * v
        folded = w1_t @ fold  # [M H + d, 2d]
        self.w1_state_t.copy_(folded)
        second = torch.matmul(w_out, w2_t)  # [M, d, H]: unit j's W_out W2_j^T
        self.w2f.copy_(second.transpose(1, 2))
        gate_rows = folded[M * H:]
        self.w1f.copy_(torch.cat([folded[:M * H].reshape(M, H, 2 * d),
                                  gate_rows.expand(M, d, 2 * d)], dim=1).transpose(1, 2))
        if consts.cand_gain is not None:
            self.cand_gain.copy_(consts.cand_gain)
        self.gate_bias.copy_(consts.gate_bias)
        self.b1.copy_(consts.b1)
        if not _same_graph(self._graph_of, consts.pad_src, consts.pad_mask):
            pad_src = consts.pad_src.to(self.device)
            pad_mask = consts.pad_mask.to(self.device)
            if bool(((pad_src < 0) | (pad_src >= s.N))[pad_mask].any()):
                raise ValueError("a message source lies outside [0, N)")
            out_tgt, out_edge = out_adjacency(pad_src, pad_mask)
            if tuple(out_tgt.shape) != tuple(self.out_tgt.shape):
                raise ValueError(f"the message graph's out-degree {int(out_tgt.shape[1])} is not "
                                 f"the shape's d_out = {s.d_out}")
            self.out_tgt.copy_(out_tgt)
            self._out_edge = out_edge
            self.in_src.copy_(torch.where(pad_mask, pad_src, torch.full_like(pad_src, -1)))
            self._graph_of = _graph_token(consts.pad_src, consts.pad_mask)
        weights = consts.edge_weights.to(self.device, torch.float32).reshape(-1)[self._out_edge]
        self.out_w.copy_(torch.where(self.out_tgt >= 0, weights, torch.zeros_like(weights)))

    def load(self, c: Tensor, b: Tensor, h_old: Tensor, cells: Tensor, units: Tensor,
             valid: Tensor, reset: Tensor, d_q_pre: Optional[Tensor], d_q_post: Optional[Tensor],
             d_h_sel: Optional[Tensor], d_h_fast: Optional[Tensor], record: dict[str, Tensor],
             consts: Any, initial: Optional[tuple[Tensor, Tensor]] = None) -> None:
        """A window into the buffers (state_sweep.py:264-313): ``state_gradient_backward``'s
        arguments; ``None`` for a read that carried no cotangent; ``initial`` the cotangent of the
        state after the last position (``None``: zero). Cells outside ``[0, N)`` or units outside
        ``[0, M)`` on valid slots raise."""
        s = self.shape
        valid = valid.to(self.device, torch.bool)
        cells = cells.to(self.device)
        units = units.to(self.device)
        bad = valid & ((cells < 0) | (cells >= s.N) | (units < 0) | (units >= s.M))
        if bool(bad.any()):
            raise ValueError("a valid slot's cell or unit is out of range")
        self.c.copy_(c)
        self.b.copy_(b)
        self.h_old.copy_(h_old)
        self.slots.copy_(torch.where(valid, cells, torch.full_like(cells, -1)))
        self.units.copy_(torch.where(valid, units, torch.zeros_like(units)))
        self.reset.copy_(reset)
        for buffer, value in ((self.d_q_pre, d_q_pre), (self.d_q_post, d_q_post),
                              (self.d_h_sel, d_h_sel)):
            if value is None:
                buffer.zero_()
            else:
                buffer.copy_(value)
        if s.n_read and d_h_fast is not None:
            self.d_h_fast.copy_(d_h_fast)
        else:
            self.d_h_fast.zero_()
        if self.cand_norm:
            self.y.copy_(record["y"])
        self.gate_pre.copy_(record["gate_pre"])
        alpha = record.get("alpha")
        if alpha is None:
            self.alpha.fill_(1.0)
        else:
            self.alpha.copy_(alpha)
        self.hidden.copy_(record["hidden"])
        if self.cell_norm:
            self.rms.copy_(record["rms"])
            torch.matmul(record["m"].to(self.device, torch.float32),
                         consts.v.to(self.device, torch.float32), out=self.mv)
        self.load_weights(consts)
        for entry, value in zip((self.A_in, self.R_in), initial or (None, None)):
            if value is None:
                entry.zero_()
            else:
                entry.copy_(value)

    # -- the sweep -------------------------------------------------------------------------------

    def _window(self) -> None:
        """One whole pass over the loaded window: the running cotangents start from ``A_in`` /
        ``R_in`` and the products' operand rows from zero (rows of padded slots are never
        written), then the positions ``T - 1 .. 0``. The pass reads nothing a previous pass
        left, so it may run any number of times, and a graph of it needs no restore."""
        self.A.copy_(self.A_in)
        self.R.copy_(self.R_in)
        self.op1.zero_()  # fill kernels (no memset nodes in a captured graph)
        self.op2.zero_()
        for t in reversed(range(self.shape.T)):
            self.step(t)

    def run(self) -> tuple[Tensor, Tensor]:
        """The loaded window's sweep: ``(dc, db)``, the buffers (the graph when captured)."""
        if self._graph is None:
            self._window()
        else:
            self._graph.replay()
        return self.dc, self.db

    def capture(self, warm_up: int = 2) -> None:
        """Record one pass as a HIP graph for later ``run`` calls. ``warm_up`` eager passes go
        first, so the products' library calls have chosen their kernels and workspaces before
        the capture; since every pass restarts itself, nothing is saved or put back."""
        for _ in range(warm_up):
            self._window()
        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self._window()
        self._graph = graph

    def step(self, t: int) -> None:
        """Position ``t``: the fused step and its tail, or the three glue steps and the two
        transposed products between them."""
        stream = _lib.stream_of(self.device)
        ref = ctypes.byref(self._struct)
        if self.fused:
            _lib.call("hsn_win_back_cell", ref, t, stream)
            _lib.call("hsn_win_back_cell_tail", ref, t, stream)
            return
        _lib.call("hsn_win_back_head", ref, t, stream)
        torch.mm(self.op1, self.w2_t, out=self.act)
        _lib.call("hsn_win_back_mid", ref, t, stream)
        torch.mm(self.op2, self.w1_state_t, out=self.dv)
        _lib.call("hsn_win_back_tail", ref, t, stream)


class SweepRunner:
    """The reverse sweep of a training run on the card (state_sweep.py:563-662): one
    :class:`ReverseSweep` per window shape, loaded with every window's values, by default as a
    HIP graph captured at the shape's first window. Called with ``state_gradient_backward``'s
    arguments; returns ``None`` for what it does not take, and the caller keeps its PyTorch sweep."""

    def __init__(self, *, graph: bool = True, fused: Optional[bool] = None) -> None:
        self.graph = graph
        self.fused = fused
        self.sweeps: dict[tuple, ReverseSweep] = {}
        # the out-degree per message graph (its pad_src tensor, kept alive with it): the graph is
        # fixed between windows, and finding the degree takes host synchronisations
        self._d_out: dict[int, tuple[tuple, int]] = {}
        #: Windows swept, and how many of them captured a graph.
        self.calls = 0
        self.captures = 0

    def __call__(self, c: Tensor, b: Tensor, h_old: Tensor, cells: Tensor, units: Tensor,
                 valid: Tensor, reset: Tensor, n_cells: int, d_q_pre: Optional[Tensor],
                 d_q_post: Optional[Tensor], d_h_sel: Optional[Tensor],
                 d_h_fast: Optional[Tensor], record: dict[str, Tensor], consts: Any, *,
                 n_fast: int = 0, n_read: int = 0,
                 limits: Any = None) -> Optional[tuple[Tensor, Tensor]]:
        device = c.device
        if device.type != "cuda" or c.dtype != torch.float32:
            return None
        if limits is not None:  # the limit's step is not a kernel: the PyTorch sweep
            return None
        if consts.activation not in ACTIVATION_CODES or consts.pad_mask is None:
            return None
        product_dtype = record["hidden"].dtype
        if product_dtype not in (torch.float32, torch.bfloat16):
            return None
        known = self._d_out.get(id(consts.pad_src))
        if known is None or not _same_graph(known[0], consts.pad_src, consts.pad_mask):
            degree = int(out_adjacency(consts.pad_src, consts.pad_mask)[0].shape[1])
            known = self._d_out[id(consts.pad_src)] = (_graph_token(consts.pad_src, consts.pad_mask), degree)
        shape = sweep_shape(c, record, consts, n_cells, n_fast, n_read, d_out=known[1])
        cand_norm = consts.cand_gain is not None
        cell_norm = consts.norm_gain_state is not None
        if back_unsupported(shape, d_in=int(consts.pad_src.shape[1]), product_dtype=product_dtype,
                            activation=consts.activation, cand_norm=cand_norm,
                            cell_norm=cell_norm) is not None:
            return None
        if not 0 <= n_fast < shape.K:
            return None
        key = (shape, product_dtype, device, consts.activation, cand_norm, cell_norm,
               int(consts.pad_src.shape[1]))
        sweep = self.sweeps.get(key)
        if sweep is None:
            sweep = ReverseSweep(shape, consts, device=device, state_dtype=c.dtype,
                                 product_dtype=product_dtype, fused=self.fused)
            self.sweeps[key] = sweep
        sweep.load(c, b, h_old, cells, units, valid, reset, d_q_pre, d_q_post, d_h_sel, d_h_fast,
                   record, consts)
        if self.graph and sweep._graph is None:
            sweep.capture()
            self.captures += 1
        dc, db = sweep.run()
        self.calls += 1
        return dc.clone(), db.clone()  # the buffers are the next window's
