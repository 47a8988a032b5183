"""The host helper's pointer tables on the CPU (``hsn_amd/_tables.so``, built from
``hsn_amd/host/tables.cpp``): for the trainer's lists it takes and declines exactly the lists the
per-tensor checks do, and its tables hold each tensor's data pointer and element count; for the
cell round's operands it checks dtype, shape, layout and device and names the first mismatch.
Host code only: no kernel runs."""

from __future__ import annotations

import ctypes

import pytest
import torch

from hsn_amd import build, trainer


@pytest.fixture(scope="module")
def native():
    why = build.host_stale()
    if why is not None:
        pytest.fail(f"the host helper is not current: {why} (run __graft_entry__.build())")
    assert trainer._native is not None, "the trainer did not take the native tables"
    return trainer._native


def _expected(rows):
    """What the per-tensor checks take, without the device check (these tensors are on the
    CPU): the pointers list after list, then the first list's counts; None when declined."""
    first = rows[0]
    if not first or any(len(row) != len(first) for row in rows):
        return None
    device = first[0].device
    for row in rows:
        for t in row:
            if t.dtype != torch.float32 or not t.is_contiguous() or t.device != device:
                return None
    for j, t in enumerate(first):
        if any(row[j].numel() != t.numel() for row in rows):
            return None
    return [t.data_ptr() for row in rows for t in row] + [t.numel() for t in first]


def _table(native, rows):
    buf = native.list_table(rows)
    if buf is None:
        return None
    n = len(buf) // 8
    return list((ctypes.c_int64 * n).from_buffer(buf))


def test_tables_hold_the_pointers_and_counts(native):
    gen = torch.Generator().manual_seed(3)
    sizes = [64 * 64] * 5 + [1] + [256 * 64] * 3 + [0] + [7]
    rows = tuple([torch.randn(n, generator=gen) for n in sizes] for _ in range(4))
    rows[1][2] = torch.randn(2 * 64 * 64, generator=gen)[64 * 64:]  # a view at an offset
    want = _expected(rows)
    assert want is not None
    got = _table(native, rows)
    assert [v & 0xFFFFFFFFFFFFFFFF for v in got] == [v & 0xFFFFFFFFFFFFFFFF for v in want]
    # tuples of tuples and a single list take the same path
    assert _table(native, tuple(tuple(r) for r in rows)) == got
    single = _table(native, (rows[2],))
    assert single == want[2 * len(sizes):3 * len(sizes)] + want[-len(sizes):]


def test_tables_decline_what_the_checks_decline(native):
    a = torch.randn(100)
    b = torch.randn(100)
    cases = {
        "float64": ([a.double()], [b.double()]),
        "strided": ([a[::2]], [b[::2]]),
        "unequal counts": ([a], [b[:50]]),
        "one list shorter": ([a, a], [b]),
        "empty": ([], []),
        "no lists": (),
        "a 2-d transpose": ([a.view(10, 10).t()], [b.view(10, 10)]),
        "bfloat16 in the second list": ([a], [b.bfloat16()]),
        "meta device in the second list": ([a], [torch.empty(100, device="meta")]),
    }
    for name, rows in cases.items():
        assert native.list_table(rows) is None, name
        if rows:
            assert _expected(rows) is None, name
    assert native.list_table(([a.view(10, 10)], [b.view(100)])) is not None  # shapes may differ


def test_tables_reject_what_is_not_a_tensor_list(native):
    with pytest.raises(TypeError):
        native.list_table(([torch.zeros(3)], [None]))
    with pytest.raises(TypeError):
        native.list_table(5)
    with pytest.raises(TypeError):
        native.list_table(([torch.zeros(3)], 7))


def test_pass_tables_match_the_per_tensor_path(native, monkeypatch):
    """``trainer._tables`` gives the C entry points the same arrays with and without the native
    module (the device check forced to pass for these CPU tensors)."""
    monkeypatch.setattr(trainer, "ready", lambda device: True)
    gen = torch.Generator().manual_seed(5)
    rows = tuple([torch.randn(n, generator=gen) for n in (5, 64, 3)] for _ in range(3))
    with_native = trainer._tables(rows)
    monkeypatch.setattr(trainer, "_native", None)
    without = trainer._tables(rows)
    assert with_native is not None and without is not None
    assert [list(t) for t in with_native[0]] == [list(t) for t in without[0]]
    assert list(with_native[1]) == list(without[1])
    assert trainer._tables(([], [])) is None


def test_operand_table_checks_dtype_shape_device_and_layout(native):
    """``tensor_table`` (the cell round's twenty operands): the data pointers when every tensor
    has its dtype and shape, is contiguous and on the device (-1: the CPU); else the index of the
    first that does not."""
    f32, i64 = torch.float32, torch.int64
    ts = [torch.zeros(4, 3), torch.zeros(5, dtype=i64), torch.zeros(2, 0), torch.zeros((), dtype=f32),
          torch.zeros(6, dtype=torch.bool)]
    dtypes = [f32, i64, f32, f32, torch.bool]
    shapes = [(4, 3), (5,), (2, 0), (), (6,)]
    buf = native.tensor_table(ts, dtypes, shapes, -1)
    assert isinstance(buf, bytearray)
    got = list((ctypes.c_int64 * len(ts)).from_buffer(buf))
    assert [v & 0xFFFFFFFFFFFFFFFF for v in got] == [t.data_ptr() & 0xFFFFFFFFFFFFFFFF for t in ts]
    assert native.tensor_table(ts, dtypes, shapes, 0) == 0  # not on device 0
    for i, (t, dt, sh) in enumerate([
            (torch.zeros(5, dtype=torch.int32), i64, (5,)),  # dtype
            (torch.zeros(3, 4), f32, (4, 3)),  # shape
            (torch.zeros(4, 3)[:, :2].contiguous().t(), f32, (2, 4)),  # layout
            (torch.zeros(4, 3), f32, (4, 3, 1))]):  # rank
        bad_ts, bad_dt, bad_sh = list(ts), list(dtypes), list(shapes)
        bad_ts[1], bad_dt[1], bad_sh[1] = t, dt, sh
        assert native.tensor_table(bad_ts, bad_dt, bad_sh, -1) == 1, i
    with pytest.raises(ValueError):
        native.tensor_table(ts, dtypes[:2], shapes, -1)
    with pytest.raises(TypeError):
        native.tensor_table(ts, ["float32"] * 5, shapes, -1)
