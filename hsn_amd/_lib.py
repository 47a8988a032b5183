"""The C ABI of ``libhsn_amd.so`` (``include/hsn_window.h``, ``include/hsn_ops.h``,
``include/hsn_trainer.h``, ``include/hsn_sweep.h``, ``include/hsn_round.h``) via ctypes.

The library is the product: every operator in :mod:`hsn_amd` reaches the GPU through these
entry points, and nothing here falls back to another implementation. :func:`library` raises a
``RuntimeError`` when the library is missing or was built from other sources, and
:func:`call` turns a non-zero status into a ``RuntimeError`` carrying the library's message.
Loading the library initialises no GPU context; the first kernel launch does.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import c_char_p, c_float, c_int, c_int64, c_void_p
from functools import lru_cache

from . import build as _build

HSN_OK = 0
STATUS = {
    1: "HSN_ERR_INVALID_ARGUMENT",
    2: "HSN_ERR_UNSUPPORTED_DTYPE",
    3: "HSN_ERR_INDEX_OUT_OF_RANGE",
    4: "HSN_ERR_DUPLICATE_INDEX",
    5: "HSN_ERR_SIZE_OVERFLOW",
    6: "HSN_ERR_BAD_GRAPH",
    7: "HSN_ERR_BACKEND",
}
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2

P, I, F, L = c_void_p, c_int, c_float, c_int64

#: argument types of every exported entry point, in declaration order of the headers
SIGNATURES: dict[str, list] = {
    "hsn_win_abi_version": [],
    "hsn_win_last_error": [],
    "hsn_win_supports": [I, I, I, I, I, I],
    "hsn_win_set_path": [I],
    "hsn_win_path": [I, I, I, I, I, I, I, P],
    "hsn_win_workspace_bytes": [I, I, I, I, I, I, I, I, P],
    "hsn_win_route": [P, I, L, P, P, P, P, P, I, P, P, P, P, P, I, I, I, I, I, I, I, F, F, F, F, I,
                      I, P],
    "hsn_win_select": [P, I, L, P, P, P, P, P, P, P, I, I, I, I, I, I, I, I, I, F, F, F, F, I, I, P],
    "hsn_win_forward": [P, P, I, P, I, F, P, L, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, I, I, I,
                        I, I, P],
    "hsn_win_forward_noalloc": [P, P, I, P, I, F, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, I,
                                I, I, I, I, P],
    "hsn_win_route_forward": [P, I, L, P, P, P, I, P, P, P, P, I, F, F, F, F, I, I, P, P, I, P, I,
                              F, P, L, P, P, P, P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I,
                              P],
    "hsn_win_set_route_forward": [I],
    "hsn_win_route_forward_fuses": [I, I, I, I, I, I, I, I, I, I, P, P],
    "hsn_win_exchange_timeouts": [P, I],
    "hsn_win_backward": [P, P, P, I, P, I, F, P, L, P, P, P, P, P, P, P, P, P, P, P, P, I, I, I, I,
                         I, P],
    "hsn_win_recurrence": [P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, P],
    "hsn_win_recurrence_dense": [P, P, P, P, P, P, P, P, I, I, I, I, P],
    "hsn_win_cell_update": [P, P, I, P, I, F, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, I, I, I,
                            I, I, I, I, I, P],
    "hsn_win_fold_row": [P, I, P, I, I, P, I, I, P, P, I, I, I, I, I, I, I, P],
    "hsn_gather_concat": [P, P, P, P, P, P, I, I, I, I, I, P],
    "hsn_gather_concat_bwd": [P, P, P, P, P, P, I, I, I, I, I, I, P],
    "hsn_grouped_unit_mlp_fwd": [P, P, P, P, P, P, P, P, I, I, I, I, I, P],
    "hsn_grouped_unit_mlp_bwd": [P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, P],
    "hsn_csr_messages": [P, P, P, P, P, P, P, I, I, I, I, I, I, P],
    "hsn_csr_messages_bwd": [P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, I, P],
    "hsn_gated_delta_update": [P, P, P, P, P, P, P, P, I, I, I, I, I, P],
    "hsn_gated_delta_update_bwd": [P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, P],
    "hsn_tr_adamw": [P, P, P, P, P, I, I, P, P],
    "hsn_tr_adamw_units": [P, P, P, P, P, I, I, I, P, F, F, P],
    "hsn_tr_lerp": [P, P, P, I, F, P],
    "hsn_tr_scale64": [P, P, I, P, P],
    "hsn_tr_copy": [P, P, P, I, P],
    "hsn_tr_limit_squares": [P, P, P, P, P, I, P],
    "hsn_tr_limit_project": [P, P, P, P, P, I, P],
    "hsn_win_back_check": [P],
    "hsn_win_back_head": [P, I, P],
    "hsn_win_back_mid": [P, I, P],
    "hsn_win_back_tail": [P, I, P],
    "hsn_win_back_cell_check": [P],
    "hsn_win_back_cell": [P, I, P],
    "hsn_win_back_cell_tail": [P, I, P],
    "hsn_win_cell_round_check": [P],
    "hsn_win_cell_round_workspace": [P, P],
    "hsn_win_cell_round": [P, P],
}

_lock = threading.Lock()


@lru_cache(maxsize=None)
def host_tables():
    """The host helper module ``hsn_amd._tables`` (the Python mirror's checks and pointer tables
    in one native call) when it is built from the current source, else ``None``: the callers then
    make the same checks and tables in Python."""
    if _build.host_stale() is not None:
        return None
    from . import _tables

    return _tables


@lru_cache(maxsize=1)
def library() -> ctypes.CDLL:
    """The loaded library (built in-tree and matching its sources), else ``RuntimeError``."""
    with _lock:
        why = _build.stale()
        if why is not None:
            raise RuntimeError(f"hsn_amd HIP library unusable: {why}")
        lib = ctypes.CDLL(str(_build.LIBRARY))
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = c_char_p if name == "hsn_win_last_error" else c_int
        return lib


def available() -> bool:
    """Whether the library is built and current (no load, no GPU work)."""
    return _build.stale() is None


def call(name: str, *args) -> None:
    """Call entry point ``name``; a non-zero status raises ``RuntimeError``."""
    lib = library()
    status = getattr(lib, name)(*args)
    if status != HSN_OK:
        message = lib.hsn_win_last_error().decode(errors="replace")
        raise RuntimeError(f"{name}: {STATUS.get(status, status)}: {message}")


OP_FORWARD, OP_BACKWARD, OP_RECURRENCE, OP_CELL_UPDATE, OP_ROUTE = 0, 1, 2, 3, 4


def unsupported(op: int, B: int, T: int, N: int, d: int, K: int) -> str | None:
    """Why entry point ``op`` does not take this shape (``None``: it does), from the library's
    own geometry (``hsn_win_supports``; host arithmetic only, no GPU)."""
    lib = library()
    if lib.hsn_win_supports(op, B, T, N, d, K) == HSN_OK:
        return None
    return lib.hsn_win_last_error().decode(errors="replace")


ROUTE_FORWARD = {"auto": 0, "one": 1, "two": 2}


def set_route_forward(mode: str) -> None:
    """How later route-and-forward calls of this process run: ``"auto"`` (the library's choice,
    the default), ``"one"`` (one launch wherever the routed forward takes the call) or
    ``"two"`` (the router, then the forward)."""
    call("hsn_win_set_route_forward", ROUTE_FORWARD[mode])


PATHS = {"auto": 0, "slice": 1, "chain": 2, "evmap": 3}
PATH_NAMES = {v: k for k, v in PATHS.items()}


def set_path(path: str) -> None:
    """Fix the sweeps' design for later forward / backward calls of this process: ``"auto"``
    (the default), ``"slice"`` (time-chunked slices in LDS), ``"chain"`` (cell chains) or
    ``"evmap"`` (time-chunked slices with event maps)."""
    call("hsn_win_set_path", PATHS[path])


def path_for(op: int, B: int, T: int, N: int, d: int, K: int, io_code: int) -> str:
    """The design a forward / backward call of this shape takes (``"slice"``, ``"chain"`` or
    ``"evmap"``)."""
    out = ctypes.c_int(0)
    call("hsn_win_path", op, B, T, N, d, K, io_code, ctypes.byref(out))
    return PATH_NAMES[out.value]


def workspace_bytes(op: int, B: int, T: int, N: int, d: int, K: int, io_code: int,
                    cand_norm: bool) -> int:
    """Bytes of the workspace a forward / backward call of this shape needs (host arithmetic)."""
    out = ctypes.c_int64(0)
    call("hsn_win_workspace_bytes", op, B, T, N, d, K, io_code, int(bool(cand_norm)),
         ctypes.byref(out))
    return int(out.value)


def ptr(t) -> int | None:
    """Device address of a tensor (``None`` for an absent optional tensor); a tensor in host
    memory raises ``ValueError`` (the kernels would read its address as device memory)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError(f"a {tuple(t.shape)} tensor on {t.device}: the kernels take ROCm device "
                         "tensors")
    return t.data_ptr()


def stream_of(device) -> int:
    """The current torch stream of ``device`` as a hipStream_t handle."""
    import torch

    return torch.cuda.current_stream(device).cuda_stream
