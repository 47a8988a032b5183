"""``hsn_amd.kernels.ops`` as the reference's ``KernelOps`` backend on the GPU.

* The four adapters (``gather_concat``, ``grouped_unit_mlp``, ``csr_messages``,
  ``gated_delta_update``) called with the model's objects (a ``CellGraphState``, a unit bank, a
  CSR graph and a bias-free ``nn.Linear``), against the float64 oracle on the golden vectors.
* The raw custom ops under the reference's callable names, as its device tests use them
  (``tests/kernels/test_p2_10_cuda.py``): torch's op checks, an fp32 gradient check by finite
  differences, ``torch.compile(fullgraph=True)`` forward and backward, and a HIP graph of forward
  plus backward replayed after the routing changed.
"""

from __future__ import annotations

import types

import pytest
import torch
from torch import nn

from conftest import load_golden

pytestmark = pytest.mark.gpu

OPS = ("gather_concat", "grouped_unit_mlp", "csr_messages", "gated_delta_update")
INPUTS = {
    "gather_concat": ("u", "eps", "h", "m", "cell_idx"),
    "grouped_unit_mlp": ("v", "unit_idx", "W1", "b1", "W2", "b2"),
    "csr_messages": ("h", "indptr", "indices", "a", "V", "cell_idx"),
    "gated_delta_update": ("h", "q", "age", "cell_idx", "valid", "c", "b"),
}


@pytest.fixture(scope="module")
def ops(cuda_device):
    from hsn_amd.kernels import ops

    assert ops.available(), "the HIP library must be built for the GPU tests"
    return ops


def _vector(op, size, dev, grad=True):
    """The golden vector's tensors on the GPU; its floating inputs require grad."""
    t = {k: v.to(dev) for k, v in load_golden(f"{size}_{op}.safetensors").items()}
    if grad:
        for name in INPUTS[op]:
            if t[name].is_floating_point():
                t[name] = t[name].detach().requires_grad_(True)
    return t


def _forward(ops, op, t):
    args = [t[n] for n in INPUTS[op]]
    if op == "gather_concat":
        return {"v": ops.gather_op(*args)}
    if op == "grouped_unit_mlp":
        out, hidden = ops.mlp_op(*args)
        return {"out": out, "hidden_saved": hidden}
    if op == "csr_messages":
        return {"m": ops.messages_op(*args)}
    h, q, age, old = ops.update_op(*args)
    return {"h_out": h, "q_out": q, "age_out": age, "h_old_saved": old}


def _grads(op, t, out):
    """The floating inputs' gradients for the vector's output cotangents (``grad_<output>``)."""
    inputs = [n for n in INPUTS[op] if t[n].is_floating_point()]
    outputs = [n for n in out if "grad_" + n in t]
    got = torch.autograd.grad([out[n] for n in outputs], [t[n] for n in inputs],
                              [t["grad_" + n] for n in outputs])
    return dict(zip(inputs, got))


# ---- the adapters ---------------------------------------------------------------------------


class _Graph:
    """The CSR graph's face as the adapter reads it: ``indptr`` / ``indices`` by target, the
    edge weights, the edges' positions in the padded ``[N, D]`` layout and the two checks."""

    def __init__(self, indptr, indices, a, D):
        self.indptr, self.indices, self._a = indptr.to(torch.int64), indices.to(torch.int64), a
        N = indptr.numel() - 1
        self.N = N
        deg = indptr[1:] - indptr[:-1]
        tgt = torch.repeat_interleave(torch.arange(N, device=indptr.device), deg.long())
        slot = torch.arange(indices.numel(), device=indptr.device) - indptr[:-1].long()[tgt]
        self._edge_pos = tgt * D + slot

    def edge_weights(self):
        return self._a

    def _check_h(self, h):
        assert h.dim() == 3 and h.shape[1] == self.N
        return tuple(h.shape)

    def _check_cell_idx(self, cell_idx, B, check_values=True):
        assert cell_idx.shape[0] == B
        if check_values:
            assert int(cell_idx.min()) >= 0 and int(cell_idx.max()) < self.N


@pytest.mark.parametrize("size", ["tiny", "odd"])
def test_adapters_match_the_oracle(ops, cuda_device, size):
    from oracle import hsn_oracle as O

    dev = cuda_device
    f64 = lambda x: x.detach().double().cpu()  # noqa: E731
    close = lambda got, want: torch.testing.assert_close(  # noqa: E731
        got.detach().double().cpu(), want, atol=1e-5, rtol=1e-5)

    t = _vector("gather_concat", size, dev, grad=False)
    idx64 = t["cell_idx"].to(torch.int64)
    close(ops.gather_concat(t["u"], t["eps"], t["h"], t["m"].double(), idx64),
          O.gather_concat(f64(t["u"]), f64(t["eps"]), f64(t["h"]), f64(t["m"]), idx64.cpu()))

    t = _vector("grouped_unit_mlp", size, dev, grad=False)
    M, in_dim, H = t["W1"].shape
    d = t["W2"].shape[2]
    bank = types.SimpleNamespace(activation_name="gelu", in_dim=in_dim, d=d, n_units=M, hidden=H,
                                 W1=t["W1"], b1=t["b1"], W2=t["W2"], b2=t["b2"])
    want, _ = O.grouped_unit_mlp(f64(t["v"]), t["unit_idx"].cpu(), f64(t["W1"]), f64(t["b1"]),
                                 f64(t["W2"]), f64(t["b2"]))
    close(ops.grouped_unit_mlp(t["v"], t["unit_idx"].to(torch.int64), bank), want)
    flat = t["W1"].permute(1, 0, 2).reshape(in_dim, M * H)  # the bank's flat first layer
    close(ops.grouped_unit_mlp(t["v"], t["unit_idx"], bank, static=True, w1_flat=flat), want)
    with pytest.raises(IndexError):
        ops.grouped_unit_mlp(t["v"], torch.full_like(t["unit_idx"], M), bank)

    t = _vector("csr_messages", size, dev, grad=False)
    N, d = t["h"].shape[1], t["h"].shape[2]
    D = int((t["indptr"][1:] - t["indptr"][:-1]).max()) or 1
    graph = _Graph(t["indptr"], t["indices"], t["a"], D)
    V = nn.Linear(d, d, bias=False).to(dev)
    with torch.no_grad():
        V.weight.copy_(t["V"])
    want = O.csr_messages(f64(t["h"]), t["indptr"].cpu(), t["indices"].cpu(), f64(t["a"]),
                          f64(t["V"]), t["cell_idx"].cpu())
    close(ops.csr_messages(t["h"], graph, V, t["cell_idx"].to(torch.int64)), want)
    padded = torch.zeros(N * D, device=dev).index_copy_(0, graph._edge_pos, t["a"]).reshape(N, D)
    close(ops.csr_messages(t["h"], graph, V, t["cell_idx"], weights=padded, validate=False), want)
    with pytest.raises(ValueError, match="bias"):
        ops.csr_messages(t["h"], graph, nn.Linear(d, d).to(dev), t["cell_idx"])

    from hsn_amd.state import CellGraphState

    t = _vector("gated_delta_update", size, dev, grad=False)
    age = t["age"].to(torch.int64) + (1 << 33)  # ages past int32 stay exact
    state = CellGraphState(h=t["h"], q=t["q"], age=age, pos=torch.arange(t["h"].shape[0], device=dev))
    valid = t["valid"].bool()
    cells = t["cell_idx"].to(torch.int64)
    nxt = ops.gated_delta_update(state, cells, t["c"], t["b"], valid)
    h2, q2, age2, _ = O.gated_delta_update(f64(t["h"]), f64(t["q"]), age.cpu(), cells.cpu(),
                                           f64(t["c"]), f64(t["b"]), valid.cpu())
    assert isinstance(nxt, CellGraphState) and nxt.pos is state.pos
    close(nxt.h, h2)
    close(nxt.q, q2)
    assert nxt.age.dtype == torch.int64 and torch.equal(nxt.age.cpu(), age2)
    assert torch.equal(state.h, t["h"])  # the state it came from is left as it was


def test_update_adapter_checks_the_selection(ops, cuda_device):
    from hsn_amd.state import CellGraphState

    dev = cuda_device
    state = CellGraphState.zeros(2, 6, 8, device=dev)
    c = b = torch.zeros(2, 3, 8, device=dev)
    valid = torch.tensor([[True, True, False], [True, False, True]], device=dev)
    with pytest.raises(IndexError):
        ops.gated_delta_update(state, torch.tensor([[0, 6, 1], [0, 1, 2]], device=dev), c, b, valid)
    with pytest.raises(ValueError, match="distinct"):
        ops.gated_delta_update(state, torch.tensor([[4, 4, 1], [0, 1, 2]], device=dev), c, b, valid)
    with pytest.raises(ValueError, match="bool"):
        ops.gated_delta_update(state, torch.zeros(2, 3, dtype=torch.int64, device=dev), c, b,
                               valid.to(torch.int32))
    # a padded slot's index, however large, is ignored; int64 indices are clamped, not wrapped
    cells = torch.tensor([[0, 1, 2**40], [3, -(2**40), 5]], device=dev)
    nxt = ops.gated_delta_update(state, cells, c + 1.0, b + 0.5, valid)
    touched = torch.zeros(2, 6, dtype=torch.bool)
    touched[0, [0, 1]] = True
    touched[1, [3, 5]] = True
    assert torch.equal((nxt.h.cpu() != 0).any(-1), touched)


# ---- the raw ops ----------------------------------------------------------------------------


def test_prepare_cuda_runs_every_op_once(ops, cuda_device):
    ops.prepare_cuda(cuda_device.index or 0)


@pytest.mark.parametrize("op", OPS)
def test_opcheck(ops, cuda_device, op):
    fn = {"gather_concat": ops.gather_op, "grouped_unit_mlp": ops.mlp_op,
          "csr_messages": ops.messages_op, "gated_delta_update": ops.update_op}[op]
    t = _vector(op, "tiny", cuda_device)
    torch.library.opcheck(fn, tuple(t[n] for n in INPUTS[op]))


@pytest.mark.parametrize("op", OPS)
def test_gradcheck_fp32(ops, cuda_device, op):
    """Finite differences in fp32 on the tiny vector (the ABI has no float64): the step and the
    tolerances are sized for fp32 rounding; the float64 oracle pins the gradients tightly in the
    parity tests."""
    t = _vector(op, "tiny", cuda_device)
    floating = [n for n in INPUTS[op] if t[n].is_floating_point()]

    def fn(*xs):
        out = _forward(ops, op, {**t, **dict(zip(floating, xs))})
        return tuple(v for k, v in out.items() if "grad_" + k in t)

    assert torch.autograd.gradcheck(fn, tuple(t[n] for n in floating), eps=1e-3, atol=5e-3,
                                    rtol=5e-3, fast_mode=True)


@pytest.mark.parametrize("op", OPS)
def test_compile_fullgraph_forward_and_backward(ops, cuda_device, op):
    t = _vector(op, "tiny", cuda_device)
    names = INPUTS[op]

    def fn(*xs):
        return _forward(ops, op, dict(zip(names, xs)))

    compiled = torch.compile(fn, fullgraph=True)
    out = compiled(*(t[n] for n in names))
    eager = _forward(ops, op, t)
    for k in eager:
        torch.testing.assert_close(out[k], eager[k])
    got, want = _grads(op, t, out), _grads(op, t, eager)
    for k in want:
        torch.testing.assert_close(got[k], want[k], msg=k)


@pytest.mark.parametrize("op", OPS)
def test_graph_replay_follows_changed_routing(ops, cuda_device, op):
    """Forward and backward captured as one HIP graph; the routing input is changed in place
    (the cells' order per row, the pairs' units, or for the update the candidate values) and the
    replay must give what an eager call on the changed inputs gives."""
    t = _vector(op, "tiny", cuda_device)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm the allocator and the libraries off the capture
        for _ in range(3):
            _grads(op, t, _forward(ops, op, t))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = _forward(ops, op, t)
        grads = _grads(op, t, out)
    with torch.no_grad():
        if op == "grouped_unit_mlp":
            t["unit_idx"].copy_((t["unit_idx"] + 1) % t["W1"].shape[0])
        elif op == "gated_delta_update":
            t["c"].add_(0.25)
        else:
            t["cell_idx"].copy_(t["cell_idx"].flip(1))
    for _ in range(2):
        graph.replay()
        torch.cuda.synchronize()
        eager = _forward(ops, op, t)
        want = _grads(op, t, eager)
        for k in eager:
            torch.testing.assert_close(out[k], eager[k], msg=k)
        for k in want:
            torch.testing.assert_close(grads[k], want[k], msg=k)


def test_eager_bodies_equal_the_registered_ops(ops):
    """Outside grad mode (and in the backward formulas) the adapters call each op's body without
    the custom op's dispatch: every forward and backward body gives the registered op's bits."""
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(12)
    B, K, N, d, E, P, M, H = 4, 4, 32, 64, 128, 16, 8, 512

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to(dev)

    idx = torch.stack([torch.randperm(N, generator=g)[:K] for _ in range(B)]).to(dev)
    valid = torch.ones(B, K, dtype=torch.int32, device=dev)
    valid[1, 2] = 0
    h, q = rnd(B, N, d, scale=0.5), rnd(B, d)
    age = torch.randint(0, 9, (B, N), generator=g).to(dev)
    c, b = rnd(B, K, d).tanh(), torch.sigmoid(rnd(B, K, d))
    u, eps, m = rnd(B, d), rnd(B, d), rnd(B, K, d)
    unit = torch.randint(0, M, (P,), generator=g).to(dev)
    v = rnd(P, 4 * d)
    w1, b1 = rnd(M, 4 * d, H, scale=(4 * d) ** -0.5), rnd(M, H, scale=0.1)
    w2, b2 = rnd(M, H, d, scale=H ** -0.5), rnd(M, d, scale=0.1)
    indptr = torch.arange(0, E + 1, E // N, dtype=torch.int64).to(dev)
    indices = torch.randint(0, N, (E,), generator=g).to(dev)
    a = torch.rand(E, generator=g).to(dev)
    V = rnd(d, d, scale=d ** -0.5)
    with torch.no_grad():
        out, hidden = ops.mlp_op(v, unit, w1, b1, w2, b2)
        cases = {
            "gather": (ops.gather_op, ops._gather_body, (u, eps, h, m, idx)),
            "gather backward": (ops.gather_backward, ops._gather_bwd_body,
                                (rnd(B, K, 4 * d), idx, N)),
            "mlp": (ops.mlp_op, ops._mlp_body, (v, unit, w1, b1, w2, b2)),
            "mlp backward": (ops.mlp_backward, ops._mlp_bwd_body, (v, unit, w1, w2, hidden, out)),
            "messages": (ops.messages_op, ops._messages_body, (h, indptr, indices, a, V, idx)),
            "messages backward": (ops.messages_backward, ops._messages_bwd_body,
                                  (h, indptr, indices, a, V, idx, m)),
            "update": (ops.state_update_op, ops._functional, (h, q, age, idx, valid, c, b)),
            "update backward": (ops.update_backward, ops._update_bwd_body,
                                (idx, valid, c, b, c, h, q)),
        }
        for name, (op, body, args) in cases.items():
            want, got = op(*args), body(*args)
            want = want if isinstance(want, tuple) else (want,)
            got = got if isinstance(got, tuple) else (got,)
            assert len(want) == len(got), name
            for i, (x, y) in enumerate(zip(got, want)):
                assert x.dtype == y.dtype and x.shape == y.shape, (name, i)
                assert torch.equal(x, y) or bool(((x == y) | (x.isnan() & y.isnan())).all()), \
                    f"{name}: output {i} differs from the registered op's"
