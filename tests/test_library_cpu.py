"""The C-ABI library on the CPU: it is built from the current sources, it loads without a GPU,
and it exports every entry point the headers declare with the status codes of the reference's
ABI. No kernel runs here."""

from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]


def _declared() -> set[str]:
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(hsn_\w+)\s*\(", text))
    return names


def test_headers_declare_the_hot_path_entry_points():
    names = _declared()
    for expected in ("hsn_win_route", "hsn_win_select", "hsn_win_forward", "hsn_win_backward",
                     "hsn_win_recurrence", "hsn_win_recurrence_dense", "hsn_win_cell_update",
                     "hsn_gated_delta_update", "hsn_gated_delta_update_bwd", "hsn_gather_concat",
                     "hsn_gather_concat_bwd", "hsn_grouped_unit_mlp_fwd",
                     "hsn_grouped_unit_mlp_bwd", "hsn_csr_messages", "hsn_csr_messages_bwd",
                     "hsn_win_abi_version", "hsn_win_last_error", "hsn_tr_adamw",
                     "hsn_tr_adamw_units", "hsn_tr_lerp", "hsn_tr_scale64", "hsn_tr_copy",
                     "hsn_tr_limit_squares", "hsn_tr_limit_project", "hsn_win_back_check",
                     "hsn_win_back_head", "hsn_win_back_mid", "hsn_win_back_tail",
                     "hsn_win_back_cell", "hsn_win_back_cell_tail", "hsn_win_cell_round",
                     "hsn_win_cell_round_check", "hsn_win_cell_round_workspace"):
        assert expected in names


def test_library_is_current_and_exports_every_declared_symbol():
    from hsn_amd import _lib, build

    why = build.stale()
    if why is not None:
        pytest.skip(f"library not built here: {why}")
    out = subprocess.run(["nm", "-D", "--defined-only", str(build.LIBRARY)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (hsn_\w+)$", out, flags=re.M))
    assert _declared() <= exported, _declared() - exported
    assert set(_lib.SIGNATURES) == _declared()
    lib = _lib.library()  # loads without a GPU
    assert lib.hsn_win_abi_version() == 2


def test_status_codes_match_the_reference_abi():
    """HSN_OK and HSN_ERR_* 1..7 as kernels/include/hsn_ops.h:69-77 numbers them."""
    text = (ROOT / "include" / "hsn_ops.h").read_text()
    codes = dict(re.findall(r"#define (HSN_(?:OK|ERR_\w+)) (\d+)", text))
    assert codes == {"HSN_OK": "0", "HSN_ERR_INVALID_ARGUMENT": "1",
                     "HSN_ERR_UNSUPPORTED_DTYPE": "2", "HSN_ERR_INDEX_OUT_OF_RANGE": "3",
                     "HSN_ERR_DUPLICATE_INDEX": "4", "HSN_ERR_SIZE_OVERFLOW": "5",
                     "HSN_ERR_BAD_GRAPH": "6", "HSN_ERR_BACKEND": "7"}


def test_argument_errors_return_status_without_a_gpu():
    """Preconditions that need no device are checked before any launch: the call returns the
    status code and a message, and never touches the GPU."""
    from hsn_amd import _lib, build

    if build.stale() is not None:
        pytest.skip("library not built here")
    lib = _lib.library()
    # K > N is rejected up front
    status = lib.hsn_win_route(1, 0, 1, 1, None, None, 1, 1, 32, 1, 1, 1, None, None, 1, 1, 4, 1,
                               8, 0, 0, 0.0, 0.0, 0.0, 1.0, 0, 0, None)
    assert status == 1
    assert b"K <= N" in lib.hsn_win_last_error()
    # f16 is not a window storage type
    status = lib.hsn_win_forward(1, 1, 1, None, 0, 0.0, None, 0, 1, 1, 1, 1, None, None, None, None,
                                 None, None, None, None, None, None, None, 1, 1, 4, 4, 2, None)
    assert status == 2
    # a NULL required pointer
    status = lib.hsn_gated_delta_update(None, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 0, None)
    assert status == 1
    # the router's fast cells (router.py:1328-1339): reserved == K, and reserved_units alone
    status = lib.hsn_win_route(1, 0, 1, 1, None, None, 1, 1, 32, 1, 1, 1, None, None, 1, 1, 8, 1,
                               4, 0, 0, 0.0, 0.0, 0.0, 1.0, 4, 0, None)
    assert status == 1 and b"reserved" in lib.hsn_win_last_error()
    status = lib.hsn_win_select(1, 0, 1, None, 1, 1, 1, 1, 1, 1, 1, 8, 1, 4, 0, 1, 1, 0, 0, 0.0,
                                0.0, 0.0, 1.0, 0, 1, None)
    assert status == 1 and b"reserved_units" in lib.hsn_win_last_error()


def test_reverse_sweep_check_follows_the_kernels_limits():
    """``back_unsupported`` is the library's own check (no GPU): the ref model's sweep is taken;
    d above 256, a row table over 64 KiB of LDS, fp16 products and an unknown activation are
    not, each with its reason."""
    import torch

    from hsn_amd import build
    from hsn_amd.state_sweep import SweepShape, back_unsupported

    if build.stale() is not None:
        pytest.skip("library not built here")
    ref = SweepShape(B=32, T=256, K=8, N=256, d=64, H=512, M=8, n_fast=0, n_read=0, in_dim=256,
                     d_out=8)
    assert back_unsupported(ref) is None
    assert back_unsupported(ref, product_dtype=torch.bfloat16) is None
    assert "256" in back_unsupported(ref._replace(d=300))
    assert "LDS" in back_unsupported(ref._replace(N=8000))
    assert "bf16" in back_unsupported(ref, product_dtype=torch.float16)
    assert "activation" in back_unsupported(ref, activation="softplus")


def test_cell_round_check_and_workspace_follow_the_kernels_limits():
    """The fused cell round's check and scratch size are host arithmetic (no GPU): the
    reference's cells and the sweep's model are taken; d not a multiple of 4, d above 256, more
    than 255 units, more than 8192 slots and a NULL buffer are not, each with its reason."""
    import ctypes

    from hsn_amd import _lib, build
    from hsn_amd.kernels import window as W

    if build.stale() is not None:
        pytest.skip("library not built here")
    assert W._round_unsupported(32, 32, 64, 4, 8, 512, 4, True) is None
    assert W._round_unsupported(32, 256, 64, 8, 8, 512, 8, False) is None
    assert W._round_unsupported(7, 11, 24, 5, 3, 77, 3, True) is None
    assert W._round_unsupported(2, 70, 256, 20, 3, 64, 0, True) is None
    assert "multiple of 4" in W._round_unsupported(1, 8, 6, 1, 2, 8, 2, True)
    assert "256" in W._round_unsupported(1, 8, 260, 1, 2, 8, 2, True)
    assert "255 units" in W._round_unsupported(1, 8, 64, 1, 300, 8, 2, True)
    assert "8192 slots" in W._round_unsupported(2048, 8, 64, 8, 2, 8, 2, True)
    lib = _lib.library()
    s = W._round_struct(32, 256, 64, 8, 8, 512, 8, True, 1e-6, 1e-6,
                        **{name: 256 for name in W._ROUND_POINTERS})
    s.W1 = None
    assert lib.hsn_win_cell_round_check(ctypes.byref(s)) == 1
    assert "NULL" in lib.hsn_win_last_error().decode()
    s.W1 = 256
    n = ctypes.c_int64(0)
    assert lib.hsn_win_cell_round_workspace(ctypes.byref(s), ctypes.byref(n)) == 0
    P, d = 32 * 8, 64
    assert n.value == P * d * 4 + 8 * P * d * 4  # the gate, 8 chunks of F


def test_trainer_pass_arguments_are_checked_before_any_launch():
    """The trainer passes' list checks run on the host: a bad unit count, a tensor that is not a
    whole number of units, a NULL pointer of a non-empty tensor and a negative size return
    HSN_ERR_INVALID_ARGUMENT with a message; a list of empty tensors (whose pointers may be NULL,
    as torch's are) is nothing to do and returns HSN_OK without a launch."""
    import ctypes

    from hsn_amd import _lib, build

    if build.stale() is not None:
        pytest.skip("library not built here")
    lib = _lib.library()

    def ptrs(*values):
        return (ctypes.c_void_p * len(values))(*values)

    def sizes(*values):
        return (ctypes.c_int64 * len(values))(*values)

    fake = 0x10000  # never dereferenced: every case below fails its checks first
    rows = [ptrs(fake) for _ in range(4)]
    coefs = (ctypes.c_float * (6 * 65))()
    assert lib.hsn_tr_adamw_units(*rows, sizes(130), 1, 65, 1, coefs, 0.001, 1e-8, None) == 1
    assert b"n_units" in lib.hsn_win_last_error()
    assert lib.hsn_tr_adamw_units(*rows, sizes(10), 1, 3, 1, coefs, 0.001, 1e-8, None) == 1
    assert b"whole number" in lib.hsn_win_last_error()
    assert lib.hsn_tr_lerp(ptrs(fake), ptrs(None), sizes(5), 1, 0.5, None) == 1
    assert b"NULL" in lib.hsn_win_last_error()
    assert lib.hsn_tr_copy(ptrs(fake), ptrs(fake), sizes(-1), 1, None) == 1
    assert b"negative" in lib.hsn_win_last_error()
    assert lib.hsn_tr_scale64(ptrs(fake), sizes(4), 1, None, None) == 1
    assert b"coefficient" in lib.hsn_win_last_error()
    assert lib.hsn_tr_lerp(ptrs(None, None), ptrs(None, None), sizes(0, 0), 2, 0.5, None) == 0


@pytest.mark.parametrize("reserved,units,ok", [(0, False, True), (3, True, True), (4, False, False),
                                               (5, False, False), (0, True, False),
                                               (-1, False, False), (True, False, False)])
def test_reserved_cells_follow_the_router_rules(reserved, units, ok):
    """``reserved`` must be an int in [0, k) and ``reserved_units`` needs reserved > 0, in the
    window path's settings, the per-position wrappers and the oracle alike (ValueError)."""
    from hsn_amd.window import RouteConfig
    from oracle import hsn_oracle as O

    logits = torch.zeros(1, 8, 2)
    cost = torch.full((2,), 1 / 16)
    if ok:
        RouteConfig(k=4, reserved=reserved, reserved_units=units)
        O.router_select(logits, None, cost, k=4, reserved=reserved, reserved_units=units)
    else:
        with pytest.raises(ValueError):
            RouteConfig(k=4, reserved=reserved, reserved_units=units)
        with pytest.raises(ValueError):
            O.router_select(logits, None, cost, k=4, reserved=reserved, reserved_units=units)


def test_product_path_fails_loudly_without_the_library(monkeypatch):
    """No CPU fallback: a missing library raises on first use."""
    from hsn_amd import _lib, build

    monkeypatch.setattr(build, "stale", lambda: "the HIP library is not built (test)")
    _lib.library.cache_clear()
    try:
        with pytest.raises(RuntimeError, match="not built"):
            _lib.library()
    finally:
        monkeypatch.undo()
        _lib.library.cache_clear()


def test_decline_predicates_follow_the_library_geometry():
    """The Python decline checks ask the library's own launch geometry (``hsn_win_supports``),
    so a shape the kernels cannot take declines (``None`` / a reason) instead of raising at
    launch: K = 65 and N = 20460 in the recurrence, K = 65 in the update, N = 4097 in the router
    (the reference's convention, python/hsn/kernels/window.py:119-128)."""
    from hsn_amd import _lib, build
    from hsn_amd.kernels import window as W

    if build.stale() is not None:
        pytest.skip("library not built here")
    assert _lib.unsupported(_lib.OP_RECURRENCE, 2, 16, 256, 64, 8) is None
    assert _lib.unsupported(_lib.OP_RECURRENCE, 2, 16, 256, 64, 65) is not None
    assert _lib.unsupported(_lib.OP_RECURRENCE, 2, 16, 20460, 64, 8) is not None
    assert _lib.unsupported(_lib.OP_FORWARD, 32, 256, 256, 64, 8) is None
    assert _lib.unsupported(_lib.OP_BACKWARD, 32, 256, 256, 64, 8) is None
    # K = 65 leaves no slice with a slot per lane; the cell chains take it, unless the slices
    # are forced
    for op in (_lib.OP_FORWARD, _lib.OP_BACKWARD):
        assert _lib.unsupported(op, 2, 16, 256, 64, 65) is None
        try:
            _lib.set_path("slice")
            assert "slice path" in _lib.unsupported(op, 2, 16, 256, 64, 65)
            _lib.set_path("chain")
            assert "chain path" in _lib.unsupported(op, 2, 16, 512, 64, 257)
        finally:
            _lib.set_path("auto")
    assert _lib.unsupported(_lib.OP_FORWARD, 2, 16, 14000, 64, 8) is not None  # neither
    assert W.cell_update_unsupported(256, 64, 8) is None
    assert W.cell_update_unsupported(256, 64, 65) is not None
    assert W.cell_update_unsupported(16, 8, 17) is not None
    assert W.select_unsupported(4096, 32) is None
    assert W.select_unsupported(4097, 8) is not None
    assert W.select_unsupported(256, 65) is not None
    # a shape the launcher refuses is exactly one hsn_win_supports refuses
    lib = _lib.library()
    status = lib.hsn_win_recurrence(1, 1, 1, 1, 1, 1, None, None, None, None, None, 1, 1, None,
                                    None, 2, 4, 65, 64, 256, None)
    assert status == 1 and b"LDS" in lib.hsn_win_last_error()


def _align(n: int) -> int:
    return (n + 255) // 256 * 256


@pytest.mark.parametrize("name", ["ref", "bf16", "tbptt", "skewed", "tiny"])
def test_workspace_and_path_follow_the_shape(name):
    """The path a forward / backward call takes and the workspace it needs, host arithmetic
    only: the event maps for an fp32 forward or backward with d a multiple of 8, T <= 256, K <= 8,
    the tables of N cells in LDS and a grid of B d / 8 workgroups within one round of the 256
    CUs (ref, tiny), no workspace; otherwise the slices where a wavefront's piece of a slot row is a full 32-byte sector and the
    state slice N * S is at most 2048 words (ref: 8 fp32 columns of 256 cells), the cell chains
    where the piece would be narrower (bf16: 4 bf16 columns, skewed: 2) or the slice larger
    (tbptt: 8 columns of 512 cells); the chain workspace is the row lists (B(N+1) + BTK int32), the per-position
    sums (BTd fp32) and, in the forward, the per-slot deltas (BTKd fp32) and a row-maximum
    table per workgroup of cells (BTG words, 1 <= G <= N / 16), each 256-aligned, then the RMS
    candidate's input."""
    from hsn_amd import _lib, build
    from hsn_amd.window import rms_scratch_bytes
    from hsn_amd.workload import CONFIGS

    if build.stale() is not None:
        pytest.skip("library not built here")
    c = CONFIGS[name]
    io = _lib.DTYPE_BF16 if c.io == "bf16" else _lib.DTYPE_F32
    elem = 2 if c.io == "bf16" else 4
    want = "chain" if name in ("bf16", "skewed", "tbptt") else "slice"
    B, T, N, d, K = c.B, c.T, c.N, c.d, c.K
    rms = _align(rms_scratch_bytes(B * T * K, d, elem))
    for op in (_lib.OP_FORWARD, _lib.OP_BACKWARD):
        evm = (c.io == "f32" and d % 8 == 0 and T <= 256 and K <= 8 and N <= 512
               and B * (d // 8) <= 256)  # the grid in one round of the 256 CUs
        auto = "evmap" if evm else want
        assert _lib.path_for(op, B, T, N, d, K, io) == auto
        chain, table = 0, (0, 0)
        if auto == "chain":
            chain = _align(B * (N + 1) * 4) + _align(B * T * K * 4) + _align(B * T * d * 4)
            if op == _lib.OP_FORWARD:
                chain += _align(B * T * K * d * 4)
                table = (_align(B * T * 4), _align(B * T * max(1, N // 16) * 4))
        got = _lib.workspace_bytes(op, B, T, N, d, K, io, False)
        assert chain + table[0] <= got <= chain + table[1]
        assert _lib.workspace_bytes(op, B, T, N, d, K, io, True) == got + rms
    try:  # a forced path changes the answer where both paths take the shape
        _lib.set_path("chain")
        assert _lib.path_for(_lib.OP_FORWARD, B, T, N, d, K, io) == "chain"
        _lib.set_path("slice")
        assert _lib.path_for(_lib.OP_FORWARD, B, T, N, d, K, io) == "slice"
    finally:
        _lib.set_path("auto")
    # the event maps, when set: both directions (fp32, d a multiple of 8, T <= 256, K <= 8), no
    # workspace but the RMS input's; a shape they do not take is refused with the reason
    try:
        _lib.set_path("evmap")
        takes = c.io == "f32" and d % 8 == 0 and T <= 256 and K <= 8
        for op in (_lib.OP_FORWARD, _lib.OP_BACKWARD):
            why = None
            try:
                got_path = _lib.path_for(op, B, T, N, d, K, io)
            except RuntimeError as e:
                got_path, why = None, str(e)
            if takes:
                assert got_path == "evmap"
                assert _lib.workspace_bytes(op, B, T, N, d, K, io, False) == 0
                assert _lib.workspace_bytes(op, B, T, N, d, K, io, True) == rms
            else:
                assert "event-map path" in why
    finally:
        _lib.set_path("auto")
    lib = _lib.library()
    assert lib.hsn_win_set_path(4) == 1 and b"path" in lib.hsn_win_last_error()


def test_forward_rejects_a_short_workspace_without_a_gpu():
    """A workspace below what hsn_win_workspace_bytes reports is refused before any launch."""
    from hsn_amd import _lib, build

    if build.stale() is not None:
        pytest.skip("library not built here")
    lib = _lib.library()
    B, T, N, d, K = 2, 8, 64, 64, 16  # bf16: the chain path, a workspace is needed
    need = _lib.workspace_bytes(_lib.OP_FORWARD, B, T, N, d, K, _lib.DTYPE_BF16, False)
    assert need > 0
    status = lib.hsn_win_forward(1, 1, _lib.DTYPE_BF16, None, 0, 0.0, 1, need - 1, 1, 1, 1, 1,
                                 None, None, None, None, None, None, None, None, None, None,
                                 None, B, T, N, d, K, None)
    assert status == 1 and b"workspace must hold" in lib.hsn_win_last_error()


def test_noalloc_forward_rejects_a_workspace_above_its_array_without_a_gpu():
    """The no-allocation forward checks its workspace against its 32 MiB array before any HIP
    call: 1,048,576 slots of d = 64 (the RMS input alone is 260 MiB) return
    HSN_ERR_SIZE_OVERFLOW."""
    from hsn_amd import _lib, build

    if build.stale() is not None:
        pytest.skip("library not built here")
    lib = _lib.library()
    status = lib.hsn_win_forward_noalloc(1, 1, 0, 1, 1, 1e-6, 1, 1, 1, 1, None, None, None, None,
                                         None, None, None, None, None, None, None, 16, 4096, 256,
                                         64, 16, None)
    assert status == 5
    assert b"scratch array" in lib.hsn_win_last_error()


def test_route_forward_declines_follow_the_routed_kernels_limits():
    """Where hsn_win_route_forward is two launches, and why (host arithmetic: every declined
    shape is decided before the call touches a device)."""
    import ctypes

    from hsn_amd import _lib, build

    if build.stale() is not None:
        pytest.skip("library not built here")
    lib = _lib.library()
    F32, BF16 = _lib.DTYPE_F32, _lib.DTYPE_BF16
    out = ctypes.c_int(1)

    def reason(M, logits, bits, io, rms, B, T, N, d, K):
        out.value = 1
        assert lib.hsn_win_route_forward_fuses(M, logits, bits, io, rms, B, T, N, d, K, None,
                                               ctypes.byref(out)) == _lib.HSN_OK
        assert out.value == 0
        return lib.hsn_win_last_error().decode()

    assert "library's choice" in reason(1, F32, 32, F32, 0, 32, 256, 256, 64, 8)
    _lib.set_route_forward("two")
    assert "are set" in reason(1, F32, 32, F32, 0, 32, 256, 256, 64, 8)
    _lib.set_route_forward("one")
    try:
        _route_forward_reasons(reason, F32, BF16)
    finally:
        _lib.set_route_forward("auto")
    with pytest.raises(RuntimeError, match="unknown mode"):
        _lib.call("hsn_win_set_route_forward", 7)


def _route_forward_reasons(reason, F32, BF16):
    from hsn_amd import _lib

    assert "one unit" in reason(2, F32, 32, F32, 0, 2, 64, 64, 16, 4)
    assert "fp32 logits" in reason(1, BF16, 32, F32, 0, 2, 64, 64, 16, 4)
    assert "int32" in reason(1, F32, 64, F32, 0, 2, 64, 64, 16, 4)
    assert "fp32 rows" in reason(1, F32, 32, BF16, 0, 2, 64, 64, 16, 4)
    assert "event maps" in reason(1, F32, 32, F32, 0, 8, 300, 64, 64, 8)  # T > 256
    assert "event maps" in reason(1, F32, 32, F32, 0, 64, 64, 64, 64, 8)  # 512 workgroups
    assert "T <= 32 d / 8" in reason(1, F32, 32, F32, 0, 2, 100, 64, 16, 4)
    assert "N <= 512" in reason(1, F32, 32, F32, 0, 2, 64, 513, 16, 4)
    _lib.set_path("evmap")
    try:
        assert "256 workgroups" in reason(1, F32, 32, F32, 0, 64, 64, 64, 64, 8)
    finally:
        _lib.set_path("auto")


def test_device_pointers_refuse_host_tensors():
    """A host tensor never reaches a kernel as an address (the eager paths that skip the custom
    ops' device dispatch rely on it): ``ptr`` raises for it and passes ``None`` through."""
    from hsn_amd import _lib

    assert _lib.ptr(None) is None
    with pytest.raises(ValueError, match="ROCm device"):
        _lib.ptr(torch.zeros(3))
