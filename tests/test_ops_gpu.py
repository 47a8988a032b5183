"""The sparse round's op ABI (gather of the selected cells, grouped unit MLP, CSR messages, gated
delta update, their backwards) on the GPU against the reference's golden vectors and the CPU
oracle, through the custom ops of ``hsn_amd.kernels.ops``. GPU only.

The vectors' inputs lie on an f16/bf16-exact grid and their outputs come from the reference's
f64 oracle rounded once to f32, so one vector serves every dtype: f32 within 1e-5, f16 and bf16
within 1e-2 (atol = rtol, the reference's tolerances, tests/golden/MANIFEST.json).
"""

from __future__ import annotations

import pytest
import torch

from conftest import load_golden

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}
SIZES = ["tiny", "ref", "odd"]
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


@pytest.fixture(scope="module")
def ops(cuda_device):
    from hsn_amd.kernels import ops

    assert ops.available(), "the HIP library must be built for the GPU tests"
    return ops


def _close(got, want, dtype, what, scaled=False):
    """``scaled``: the absolute tolerance relative to the largest expected value, for sums so
    long that fp32 rounding alone passes the fixed tolerance where they cancel (at d = 1024 a
    dot product rounds to about sqrt(d) 2^-24 of its terms' scale, and grad_a sums d-long
    products of d-long sums)."""
    tol = TOL[dtype]
    got, want = got.float().cpu(), want.float()
    atol = tol * max(1.0, float(want.abs().max())) if scaled else tol
    err = float((got - want).abs().max()) if want.numel() else 0.0
    torch.testing.assert_close(got, want, atol=atol, rtol=tol,
                               msg=f"{what}: max |error| {err:.3g}, max |want| "
                                   f"{float(want.abs().max()) if want.numel() else 0.0:.3g}")


def _put(v, dev, dtype):
    return {k: (t.to(dev, dtype) if t.is_floating_point() else t.to(dev)) for k, t in v.items()}


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("size", SIZES)
def test_gated_update_matches_golden(ops, cuda_device, size, dtype):
    v = load_golden(f"{size}_gated_delta_update.safetensors")
    D = _put(v, cuda_device, dtype)
    h, q, age = D["h"].clone(), D["q"].clone(), D["age"].clone()
    old = ops.update_inplace(h, q, age, D["cell_idx"], D["valid"], D["c"], D["b"])
    _close(h, v["h_out"], dtype, "h_out")
    _close(q, v["q_out"], dtype, "q_out")
    assert torch.equal(age.cpu(), v["age_out"])
    _close(old, v["h_old_saved"], dtype, "h_old_saved")
    gh, gq, gc, gb = ops.update_backward(D["cell_idx"], D["valid"], D["c"], D["b"],
                                                     D["h_old_saved"], D["grad_h_out"],
                                                     D["grad_q_out"])
    for name, got in zip(("grad_h", "grad_q", "grad_c", "grad_b"), (gh, gq, gc, gb)):
        _close(got, v[name], dtype, name)


@pytest.mark.parametrize("size", SIZES)
def test_functional_update_autograd_matches_golden(ops, cuda_device, size):
    """The functional op leaves its inputs alone and its autograd gives the golden gradients."""
    v = load_golden(f"{size}_gated_delta_update.safetensors")
    D = _put(v, cuda_device, torch.float32)
    h = D["h"].clone().requires_grad_(True)
    q = D["q"].clone().requires_grad_(True)
    c = D["c"].clone().requires_grad_(True)
    b = D["b"].clone().requires_grad_(True)
    for op in (ops.update_op, ops.state_update_op):
        hn, qn, an, old = op(h, q, D["age"], D["cell_idx"], D["valid"], c, b)
        assert torch.equal(h.detach(), D["h"]) and torch.equal(D["age"].cpu(), v["age"])
        _close(hn.detach(), v["h_out"], torch.float32, "h_out")
        assert torch.equal(an.cpu(), v["age_out"])
        grads = torch.autograd.grad((hn, qn), (h, q, c, b), (D["grad_h_out"], D["grad_q_out"]))
        for name, got in zip(("grad_h", "grad_q", "grad_c", "grad_b"), grads):
            _close(got, v[name], torch.float32, name)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("size", SIZES)
def test_gather_concat_matches_golden(ops, cuda_device, size, dtype):
    v = load_golden(f"{size}_gather_concat.safetensors")
    D = _put(v, cuda_device, dtype)
    out = ops.gather_op(D["u"], D["eps"], D["h"], D["m"], D["cell_idx"])
    _close(out, v["v"], dtype, "v")
    N = v["h"].shape[1]
    gu, ge, gh, gm = ops.gather_backward(D["grad_v"], D["cell_idx"], N)
    for name, got in zip(("grad_u", "grad_eps", "grad_h", "grad_m"), (gu, ge, gh, gm)):
        _close(got, v[name], dtype, name)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gather_backward_slot_batches_match_oracle(ops, cuda_device, dtype):
    """K = 19 slots, three of the kernel's batches of 8, with cells repeated inside a batch,
    across batches and three times in a row: grad_h is the scatter-add of the slots' third
    block, in slot order (the float64 oracle adds them in any order)."""
    from oracle import hsn_oracle as O

    g = torch.Generator().manual_seed(91)
    B, N, K, d = 3, 30, 19, 36
    grad_v = (torch.randn(B, K, 4 * d, generator=g) * 0.5).to(dtype)
    cells = torch.randint(0, N, (B, K), generator=g, dtype=torch.int32)
    cells[0, 5] = cells[0, 2]      # inside the first batch
    cells[1, 17] = cells[1, 3]     # across batches
    cells[2, [4, 9, 18]] = 7       # three batches
    want = O.gather_concat_bwd(grad_v.double(), cells, N)
    dev = cuda_device
    got = ops.gather_backward(grad_v.to(dev), cells.to(dev), N)
    for name, g_, w_ in zip(("grad_u", "grad_eps", "grad_h", "grad_m"), got, want):
        _close(g_, w_, dtype, name)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gather_backward_rounds_a_repeated_cell_once(ops, cuda_device, dtype):
    """A cell taken by many slots of a row in 16-bit storage: its grad_h is the fp32 sum of the
    slots' third blocks in slot order, rounded once to the storage dtype (the ABI's accumulation),
    not a rounding after every repeat. 40 slots, 30 of them on cell 2 (five of the kernel's
    batches of 8), with small values that a per-repeat rounding would lose."""
    g = torch.Generator().manual_seed(93)
    B, N, K, d = 2, 9, 40, 24
    grad_v = torch.randn(B, K, 4 * d, generator=g)
    grad_v[:, :, 2 * d:3 * d] = 1.0 + torch.rand(B, K, d, generator=g) * 2.0 ** -6
    grad_v = grad_v.to(dtype)
    cells = torch.randint(0, N, (B, K), generator=g, dtype=torch.int32)
    cells[:, torch.randperm(K, generator=g)[:30]] = 2
    # the expectation: slot-order fp32 sums per (row, cell), each rounded once
    want = torch.zeros(B, N, d)
    third = grad_v[:, :, 2 * d:3 * d].float()
    for r in range(B):
        acc = {}
        for k in range(K):
            c = int(cells[r, k])
            acc[c] = acc.get(c, torch.zeros(d)) + third[r, k]
        for c, v in acc.items():
            want[r, c] = v
    want = want.to(dtype)
    got = ops.gather_backward(grad_v.to(cuda_device), cells.to(cuda_device), N)[2].cpu()
    assert torch.equal(got, want)


def test_gather_autograd_matches_golden(ops, cuda_device):
    v = load_golden("odd_gather_concat.safetensors")
    D = _put(v, cuda_device, torch.float32)
    leaves = [D[k].clone().requires_grad_(True) for k in ("u", "eps", "h", "m")]
    out = ops.gather_op(*leaves, D["cell_idx"])
    grads = torch.autograd.grad(out, leaves, D["grad_v"])
    for name, got in zip(("grad_u", "grad_eps", "grad_h", "grad_m"), grads):
        _close(got, v[name], torch.float32, name)


def test_inplace_update_rejects_a_strided_state(ops, cuda_device):
    """The ABI updates h, q, age in place through plain pointers: a strided view is refused
    rather than silently copied."""
    v = load_golden("ref_gated_delta_update.safetensors")
    D = _put(v, cuda_device, torch.float32)
    h = D["h"].transpose(1, 2).contiguous().transpose(1, 2)
    with pytest.raises(ValueError, match="contiguous"):
        ops.update_inplace(h, D["q"].clone(), D["age"].clone(), D["cell_idx"], D["valid"],
                               D["c"], D["b"])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("size", SIZES)
def test_grouped_unit_mlp_matches_golden(ops, cuda_device, size, dtype):
    """Forward and backward against the vectors (the odd one has a unit without pairs: zero
    gradients); in f16 / bf16 the saved z1 is the storage dtype's, as the ABI stores it."""
    v = load_golden(f"{size}_grouped_unit_mlp.safetensors")
    D = _put(v, cuda_device, dtype)
    out, hidden = ops.mlp_op(D["v"], D["unit_idx"], D["W1"], D["b1"], D["W2"], D["b2"])
    _close(hidden, v["hidden_saved"], dtype, "hidden_saved")
    _close(out, v["out"], dtype, "out")
    got = ops.mlp_backward(D["v"], D["unit_idx"], D["W1"], D["W2"],
                                        D["hidden_saved"], D["grad_out"])
    for name, g_ in zip(("grad_v", "grad_W1", "grad_b1", "grad_W2", "grad_b2"), got):
        _close(g_, v[name], dtype, name)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("size", SIZES)
def test_csr_messages_match_golden(ops, cuda_device, size, dtype):
    """Forward and backward against the vectors: repeated slots (tiny: cell 1 twice in row 1) and
    edges of rows no slot selects (their grad_a is exactly zero)."""
    v = load_golden(f"{size}_csr_messages.safetensors")
    D = _put(v, cuda_device, dtype)
    m = ops.messages_op(D["h"], D["indptr"], D["indices"], D["a"], D["V"], D["cell_idx"])
    _close(m, v["m"], dtype, "m")
    gh, ga, gV = ops.messages_backward(D["h"], D["indptr"], D["indices"], D["a"], D["V"],
                                           D["cell_idx"], D["grad_m"])
    for name, g_ in zip(("grad_h", "grad_a", "grad_V"), (gh, ga, gV)):
        _close(g_, v[name], dtype, name)
    assert bool((ga.cpu()[v["grad_a"] == 0] == 0).all())


def test_unit_mlp_and_messages_autograd_match_golden(ops, cuda_device):
    """The custom ops' autograd registrations give the vectors' gradients."""
    v = load_golden("odd_grouped_unit_mlp.safetensors")
    D = _put(v, cuda_device, torch.float32)
    leaves = [D[k].clone().requires_grad_(True) for k in ("v", "W1", "b1", "W2", "b2")]
    out, _ = ops.mlp_op(leaves[0], D["unit_idx"], *leaves[1:])
    grads = torch.autograd.grad(out, leaves, D["grad_out"])
    for name, g_ in zip(("grad_v", "grad_W1", "grad_b1", "grad_W2", "grad_b2"), grads):
        _close(g_, v[name], torch.float32, name)
    v = load_golden("odd_csr_messages.safetensors")
    D = _put(v, cuda_device, torch.float32)
    h, a, V = (D[k].clone().requires_grad_(True) for k in ("h", "a", "V"))
    m = ops.messages_op(h, D["indptr"], D["indices"], a, V, D["cell_idx"])
    for name, g_ in zip(("grad_h", "grad_a", "grad_V"),
                        torch.autograd.grad(m, (h, a, V), D["grad_m"])):
        _close(g_, v[name], torch.float32, name)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_unit_mlp_and_messages_match_oracle_on_ragged_shapes(ops, cuda_device, dtype):
    """Shapes the vectors leave open: units with more than 16 pairs (several row chunks), one
    unit without pairs, H and 4d off the 64-column tiles, d past one tile; a CSR with empty rows,
    self loops, repeated slots and d = 100 (two column tiles). Inputs rounded to the storage
    dtype first, the oracle run on them in float64."""
    from oracle import hsn_oracle as O

    g = torch.Generator().manual_seed(41)
    tol = TOL[dtype]
    P, M, d, H = 70, 5, 24, 200
    rnd = lambda *s: (torch.randn(*s, generator=g) * 0.5).to(dtype)  # noqa: E731
    v, W1, b1, W2, b2 = rnd(P, 4 * d), rnd(M, 4 * d, H), rnd(M, H), rnd(M, H, d), rnd(M, d)
    idx = torch.randint(0, M - 1, (P,), generator=g, dtype=torch.int32)  # unit M-1 unused
    dout = rnd(P, d)
    f64 = lambda t: t.double()  # noqa: E731
    want_out, want_h = O.grouped_unit_mlp(f64(v), idx, f64(W1), f64(b1), f64(W2), f64(b2))
    dev = cuda_device
    out, hidden = ops.mlp_op(v.to(dev), idx.to(dev), W1.to(dev), b1.to(dev),
                                       W2.to(dev), b2.to(dev))
    _close(hidden, want_h, dtype, "hidden")
    _close(out, want_out, dtype, "out")
    want = O.grouped_unit_mlp_bwd(f64(v), idx, f64(W1), f64(W2), f64(hidden.cpu()), f64(dout))
    got = ops.mlp_backward(v.to(dev), idx.to(dev), W1.to(dev), W2.to(dev), hidden,
                                        dout.to(dev))
    for name, g_, w_ in zip(("dv", "dW1", "db1", "dW2", "db2"), got, want):
        _close(g_, w_, dtype, name)
    assert bool((got[1][M - 1] == 0).all()) and bool((got[3][M - 1] == 0).all())
    B, N, K, d = 3, 50, 7, 100
    deg = torch.randint(0, 4, (N,), generator=g)
    deg[[3, 17]] = 0  # empty rows
    indptr = torch.cat([torch.zeros(1, dtype=torch.int64), deg.cumsum(0)]).to(torch.int32)
    E = int(indptr[-1])
    indices = torch.randint(0, N, (E,), generator=g, dtype=torch.int32)
    indices[0] = 0  # a self loop where row 0 has an edge
    a = torch.rand(E, generator=g).to(dtype)
    h, V = rnd(B, N, d), rnd(d, d)
    cell_idx = torch.randint(0, N, (B, K), generator=g, dtype=torch.int32)
    cell_idx[0, 1] = cell_idx[0, 0]  # a repeated slot
    cell_idx[1, 2] = 3  # an empty row
    gm = rnd(B, K, d)
    want_m = O.csr_messages(f64(h), indptr, indices, f64(a), f64(V), cell_idx)
    m = ops.messages_op(h.to(dev), indptr.to(dev), indices.to(dev), a.to(dev), V.to(dev),
                         cell_idx.to(dev))
    _close(m, want_m, dtype, "m")
    assert bool((m[1, 2] == 0).all())
    want = O.csr_messages_bwd(f64(h), indptr, indices, f64(a), f64(V), cell_idx, f64(gm))
    got = ops.messages_backward(h.to(dev), indptr.to(dev), indices.to(dev), a.to(dev),
                                    V.to(dev), cell_idx.to(dev), gm.to(dev))
    for name, g_, w_ in zip(("dh", "da", "dV"), got, want):
        _close(g_, w_, dtype, name)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gated_update_slot_groups_match_oracle_and_slot_order(ops, cuda_device, dtype):
    """K = 19 slots (three groups of the kernel's 8) with padded slots. Rows without repeated
    cells: against the float64 oracle. Rows with a cell repeated inside a group and across
    groups: against 19 single-slot calls in slot order, since the ABI's update is in place and
    each slot reads h after the slots before it."""
    from oracle import hsn_oracle as O

    g = torch.Generator().manual_seed(77)
    B, N, K, d = 3, 40, 19, 70
    rnd = lambda *s: (torch.randn(*s, generator=g) * 0.5).to(dtype)  # noqa: E731
    h, q, c, b = rnd(B, N, d), rnd(B, d), rnd(B, K, d), torch.rand(B, K, d, generator=g).to(dtype)
    age = torch.randint(0, 9, (B, N), generator=g, dtype=torch.int32)
    cells = torch.stack([torch.randperm(N, generator=g)[:K] for _ in range(B)]).to(torch.int32)
    valid = (torch.rand(B, K, generator=g) > 0.2).to(torch.int32)
    dev = cuda_device
    f64 = lambda t: t.double()  # noqa: E731
    want = O.gated_delta_update_abi(f64(h), f64(q), age, cells, valid, f64(c), f64(b))
    got = ops.update_op(h.to(dev), q.to(dev), age.to(dev), cells.to(dev),
                                            valid.to(dev), c.to(dev), b.to(dev))
    for name, g_, w_ in zip(("h", "q", "age", "h_old"), got, want):
        _close(g_, w_, dtype, name)
    G, gq = rnd(B, N, d), rnd(B, d)  # the backward over the same three groups of slots
    old = got[3].cpu()
    want = O.gated_delta_update_bwd(cells, valid, f64(c), f64(b), f64(old), f64(G), f64(gq))
    back = ops.update_backward(cells.to(dev), valid.to(dev), c.to(dev), b.to(dev),
                                           old.to(dev), G.to(dev), gq.to(dev))
    for name, g_, w_ in zip(("grad_h", "grad_q", "grad_c", "grad_b"), back, want):
        _close(g_, w_, dtype, name)
    rep = cells.clone()
    rep[0, 3] = rep[0, 1]     # inside the first group
    rep[1, 12] = rep[1, 2]    # across groups
    rep[2, 18] = rep[2, 9]
    rep[2, 10] = rep[2, 9]
    valid[:, [1, 2, 3, 9, 10, 12, 18]] = 1
    got = ops.update_op(h.to(dev), q.to(dev), age.to(dev), rep.to(dev),
                                            valid.to(dev), c.to(dev), b.to(dev))
    hs, qs, ages = h.to(dev), q.to(dev), age.to(dev)
    olds = []
    for k in range(K):
        one = torch.zeros_like(valid)
        one[:, k] = valid[:, k]
        hs, qs, ages, old = ops.update_op(hs, qs, ages, rep.to(dev),
                                                              one.to(dev), c.to(dev), b.to(dev))
        olds.append(old[:, k])
    _close(got[0], hs.cpu(), dtype, "h")
    _close(got[1], qs.cpu(), dtype, "q")
    assert torch.equal(got[2].cpu(), ages.cpu())
    _close(got[3], torch.stack(olds, 1).cpu(), dtype, "h_old")


@pytest.mark.parametrize("B,N,K,d,deg,dtype", [
    (32, 256, 8, 64, 8, torch.float32),    # the model's round: grad_V over 16 groups of slots
    (32, 256, 8, 64, 8, torch.bfloat16),   # the same in bf16 (half the room for the partials)
    (8, 40, 80, 24, 3, torch.float32),     # K above 64: the per-wavefront grad_h kernel
    (4, 300, 64, 40, 60, torch.float32),   # rows of thousands of edges, 3 cell blocks, d off 16
    (2, 24, 4, 1024, 3, torch.float32),    # d at its limit: the forward's [16][d] rows past 64 KiB
    (3, 17, 5, 900, 2, torch.bfloat16),    # d just past the 64 KiB default, bf16
])
def test_csr_messages_backward_paths_match_oracle(ops, cuda_device, B, N, K, d, deg, dtype):
    """The CSR forward's and backward's kernels at the shapes that pick each path, against the float64
    oracle on inputs rounded to the storage dtype; hubs (cells of in-degree up to 4 deg) make
    the rows' edge lists run past one LDS block."""
    from oracle import hsn_oracle as O

    g = torch.Generator().manual_seed(B * 1000 + K)
    rnd = lambda *s: (torch.randn(*s, generator=g) * 0.5).to(dtype)  # noqa: E731
    degs = torch.randint(0, deg + 1, (N,), generator=g)
    degs[: N // 10] *= 4
    indptr = torch.cat([torch.zeros(1, dtype=torch.int64), degs.cumsum(0)]).to(torch.int32)
    E = int(indptr[-1])
    indices = torch.randint(0, N, (E,), generator=g, dtype=torch.int32)
    a = torch.rand(E, generator=g).to(dtype)
    h, V, gm = rnd(B, N, d), rnd(d, d), rnd(B, K, d)
    cell_idx = torch.randint(0, N, (B, K), generator=g, dtype=torch.int32)
    cell_idx[:, 0] = 0  # every row selects a hub
    f64 = lambda t: t.double()  # noqa: E731
    dev = cuda_device
    m = ops.messages_op(h.to(dev), indptr.to(dev), indices.to(dev), a.to(dev), V.to(dev),
                         cell_idx.to(dev))  # hubs: slot lists past the forward's LDS list
    wide = d > 256
    _close(m, O.csr_messages(f64(h), indptr, indices, f64(a), f64(V), cell_idx), dtype, "m",
           scaled=wide)
    want = O.csr_messages_bwd(f64(h), indptr, indices, f64(a), f64(V), cell_idx, f64(gm))
    got = ops.messages_backward(h.to(dev), indptr.to(dev), indices.to(dev), a.to(dev),
                                    V.to(dev), cell_idx.to(dev), gm.to(dev))
    for name, g_, w_ in zip(("dh", "da", "dV"), got, want):
        _close(g_, w_, dtype, name, scaled=wide)
    again = ops.messages_backward(h.to(dev), indptr.to(dev), indices.to(dev), a.to(dev),
                                      V.to(dev), cell_idx.to(dev), gm.to(dev))
    assert all(torch.equal(x, y) for x, y in zip(got, again))


def test_unit_mlp_and_messages_are_reproducible(ops, cuda_device):
    """Every sum has a fixed order: two runs agree bit for bit."""
    v = load_golden("ref_grouped_unit_mlp.safetensors")
    D = _put(v, cuda_device, torch.float32)
    args = (D["v"], D["unit_idx"], D["W1"], D["W2"], D["hidden_saved"], D["grad_out"])
    first = ops.mlp_backward(*args)
    second = ops.mlp_backward(*args)
    assert all(torch.equal(x, y) for x, y in zip(first, second))
    v = load_golden("ref_csr_messages.safetensors")
    D = _put(v, cuda_device, torch.float32)
    args = (D["h"], D["indptr"], D["indices"], D["a"], D["V"], D["cell_idx"], D["grad_m"])
    first, second = ops.messages_backward(*args), ops.messages_backward(*args)
    assert all(torch.equal(x, y) for x, y in zip(first, second))


@pytest.mark.parametrize("P,M,d,H", [
    (40, 3, 6, 50),      # d not a multiple of 4: the scanning kernel
    (64, 4, 16, 77),     # H not a multiple of 4: the row-tile kernel's unaligned loads
    (20000, 2, 4, 8),    # more pairs than the row-tile kernel's slot table: the scanning kernel
    (300, 6, 64, 512),   # the reference model's widths, several tiles a unit
    (2000, 2, 8, 64),    # grad_W2 too small to hold dz1: grad_v in one launch
])
def test_unit_mlp_forward_paths_match_oracle(ops, cuda_device, P, M, d, H):
    """Both forward kernels and both grad_v kernels (by row tiles, and the pair-scanning ones for
    shapes the first do not take) against the oracle in float64 on fp32 inputs."""
    from oracle import hsn_oracle as O

    g = torch.Generator().manual_seed(P + d)
    rnd = lambda *s, scale=1.0: torch.randn(*s, generator=g) * scale  # noqa: E731
    v, b1, b2 = rnd(P, 4 * d), rnd(M, H, scale=0.1), rnd(M, d, scale=0.1)
    W1, W2 = rnd(M, 4 * d, H, scale=(4 * d) ** -0.5), rnd(M, H, d, scale=H ** -0.5)
    idx = torch.randint(0, M, (P,), generator=g, dtype=torch.int32)
    want_out, want_h = O.grouped_unit_mlp(v.double(), idx, W1.double(), b1.double(), W2.double(),
                                          b2.double())
    dev = cuda_device
    out, hidden = ops.mlp_op(v.to(dev), idx.to(dev), W1.to(dev), b1.to(dev),
                                       W2.to(dev), b2.to(dev))
    dout = rnd(P, d)
    grads = ops.mlp_backward(v.to(dev), idx.to(dev), W1.to(dev), W2.to(dev), hidden,
                                          dout.to(dev))
    want_g = O.grouped_unit_mlp_bwd(v.double(), idx, W1.double(), W2.double(),
                                    hidden.double().cpu(), dout.double())
    pairs = [("hidden", hidden, want_h), ("out", out, want_out)]
    pairs += list(zip(("dv", "dW1", "db1", "dW2", "db2"), grads, want_g))
    for name, got, want in pairs:
        # the weight gradients sum over a unit's pairs in fp32: the bar grows with the square
        # root of their count (the random walk of the roundings; 10000 pairs at P = 20000)
        bar = 1e-5 * (max(1.0, (P / M / 64) ** 0.5) if name[1] in "Wb" else 1.0)
        err = (got.double().cpu() - want).abs() / want.abs().clamp(min=1.0)
        assert float(err.max()) <= bar, f"{name}: worst {float(err.max()):.3e} (bar {bar:.1e})"
