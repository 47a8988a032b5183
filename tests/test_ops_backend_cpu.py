"""The ``KernelOps`` adapters of ``hsn_amd.kernels.ops`` on the CPU: which calls they hand to the
fallback backend (the reference's ``python/hsn/kernels/ops.py:320-444`` keeps the native path for
the same ones), the index conversion the ABI takes, and the selection checks of the update. No
library call is made here: every call below is declined or fails a check first."""

from __future__ import annotations

import types

import pytest
import torch
from torch import nn

from hsn_amd.kernels import ops
from hsn_amd.state import CellGraphState


class Recorder:
    """A fallback backend that records each call and returns a marker."""

    def __init__(self):
        self.calls = []

    def __getattr__(self, name):
        if name.startswith("_"):
            raise AttributeError(name)

        def fn(*args, **kwargs):
            self.calls.append((name, args, kwargs))
            return ("fallback", name)

        return fn


@pytest.fixture
def recorder():
    rec = Recorder()
    ops.set_fallback(rec)
    yield rec
    ops.set_fallback(None)


def _bank(d=4, M=3, H=5, activation="gelu", in_dim=None):
    in_dim = 4 * d if in_dim is None else in_dim
    return types.SimpleNamespace(
        activation_name=activation, in_dim=in_dim, d=d, n_units=M, hidden=H,
        W1=torch.zeros(M, in_dim, H), b1=torch.zeros(M, H), W2=torch.zeros(M, H, d),
        b2=torch.zeros(M, d))


def test_gather_declines_a_three_block_input_and_host_tensors(recorder):
    h = torch.zeros(2, 5, 4)
    eps, m, idx = torch.zeros(2, 4), torch.zeros(2, 3, 4), torch.zeros(2, 3, dtype=torch.int64)
    assert ops.gather_concat(None, eps, h, m, idx) == ("fallback", "gather_concat")
    assert ops.gather_concat(eps, eps, h, m, idx) == ("fallback", "gather_concat")
    name, args, _ = recorder.calls[0]
    assert name == "gather_concat" and args[0] is None and args[2] is h


def test_unit_mlp_declines_host_tensors_and_other_activations(recorder):
    v, idx = torch.zeros(6, 16), torch.zeros(6, dtype=torch.int64)
    assert ops.grouped_unit_mlp(v, idx, _bank()) == ("fallback", "grouped_unit_mlp")
    assert ops.grouped_unit_mlp(v, idx, _bank(activation="relu"), static=True) == \
        ("fallback", "grouped_unit_mlp")
    w1 = torch.zeros(12, 15)
    ops.grouped_unit_mlp(torch.zeros(6, 12), idx, _bank(in_dim=12), w1_flat=w1)
    _, _, kwargs = recorder.calls[-1]
    assert kwargs == {"static": False, "w1_flat": w1}  # keywords passed on as given


def test_messages_and_update_decline_host_tensors(recorder):
    h = torch.zeros(2, 5, 4)
    V = nn.Linear(4, 4, bias=False)
    idx = torch.zeros(2, 3, dtype=torch.int64)
    assert ops.csr_messages(h, object(), V, idx, validate=False) == ("fallback", "csr_messages")
    assert recorder.calls[-1][2] == {"weights": None, "validate": False}
    state = CellGraphState.zeros(2, 5, 4)
    c = b = torch.zeros(2, 3, 4)
    valid = torch.ones(2, 3, dtype=torch.bool)
    assert ops.gated_delta_update(state, idx, c, b, valid) == ("fallback", "gated_delta_update")
    assert recorder.calls[-1][2] == {"validate": True}


def test_a_declined_call_without_a_fallback_names_the_reason():
    ops.set_fallback(None)
    import importlib.util

    if importlib.util.find_spec("hsn") is not None:
        pytest.skip("the reference's hsn package is importable here")
    with pytest.raises(NotImplementedError, match="u=None"):
        ops.gather_concat(None, torch.zeros(1, 2), torch.zeros(1, 3, 2), torch.zeros(1, 1, 2),
                          torch.zeros(1, 1, dtype=torch.int64))


def test_indices_are_clamped_before_narrowing():
    got = ops._i32(torch.tensor([2**40, 2**32 + 1, -(2**35), -1, 0, 7]))
    assert got.dtype == torch.int32
    assert got.tolist() == [2**31 - 1, 2**31 - 1, -1, -1, 0, 7]  # nothing wraps into a cell
    same = torch.tensor([3, -1], dtype=torch.int32)
    assert ops._i32(same).tolist() == [3, -1]
    with pytest.raises(ValueError, match="int32 or int64"):
        ops._i32(torch.tensor([1.0]))
    assert ops._flags(torch.tensor([True, False])).tolist() == [1, 0]


def test_selection_checks():
    valid = torch.tensor([[True, True, False], [True, False, False]])
    ops._check_selection(torch.tensor([[0, 4, 4], [2, 2, -9]]), valid, 5)  # padded repeats: fine
    with pytest.raises(IndexError, match=r"\[0, 5\)"):
        ops._check_selection(torch.tensor([[0, 5, 1], [2, 0, 0]]), valid, 5)
    with pytest.raises(IndexError):
        ops._check_selection(torch.tensor([[0, -1, 1], [2, 0, 0]]), valid, 5)
    with pytest.raises(ValueError, match="distinct"):
        ops._check_selection(torch.tensor([[3, 3, 1], [2, 0, 0]]), valid, 5)
    ops._check_selection(torch.zeros(0, 3, dtype=torch.int64), torch.zeros(0, 3, dtype=torch.bool), 5)


def test_valid_flags_are_checked():
    dev = torch.device("cpu")
    ops._check_valid(torch.ones(2, 3, dtype=torch.bool), (2, 3), dev)
    with pytest.raises(ValueError, match="torch.bool"):
        ops._check_valid(torch.ones(2, 3, dtype=torch.int32), (2, 3), dev)
    with pytest.raises(ValueError, match="shape"):
        ops._check_valid(torch.ones(3, 2, dtype=torch.bool), (2, 3), dev)
    with pytest.raises(TypeError):
        ops._check_valid([[True]], (1, 1), dev)


def test_states_are_rebuilt_in_their_own_type():
    t = [torch.zeros(1)] * 4
    assert isinstance(ops._with_state(CellGraphState(*t), *t), CellGraphState)

    class Reference:  # the reference's class: an unchecked classmethod constructor
        @classmethod
        def _make(cls, h, q, age, pos):
            s = object.__new__(cls)
            s.h, s.q, s.age, s.pos = h, q, age, pos
            return s

    made = ops._with_state(Reference._make(*t), *t)
    assert type(made) is Reference and made.pos is t[3]
