"""The drop-in boundary's contract on the GPU, as the reference's kernel tests check it:
``torch.library.opcheck`` of every custom op (schema, fake tensor, autograd registration,
mutation annotations), the first dispatch of every op on a fresh thread
(``tests/kernels/test_p2_10_cuda.py:100-131``), and the tape forms walked over a block of
positions against the plain per-position ops bit for bit, with resets at the block's first,
interior and last positions and two in a row (``tests/kernels/test_p2_10_window.py:453-537``).
GPU only.
"""

from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mods(cuda_device):
    from hsn_amd.kernels import ops, window

    assert window.available(), "the HIP library must be built for the GPU tests"
    window.prepare(0)
    return ops, window


def _cases(dev):
    """Small inputs for every custom op: name -> (op, args, differentiable argument names)."""
    from hsn_amd.kernels import ops, window

    g = torch.Generator().manual_seed(5)
    B, N, d, K, M, n = 3, 12, 8, 3, 2, 4
    f = lambda *s: torch.randn(*s, generator=g).to(dev)  # noqa: E731
    idx = torch.stack([torch.randperm(N, generator=g)[:K] for _ in range(B)]).to(dev)
    valid = torch.ones(B, K, dtype=torch.int32, device=dev)
    valid[1, 2] = 0
    logits = f(B, N, M)
    age = torch.randint(0, 5, (B, N), generator=g).to(dev)
    tape_age = torch.randint(0, 5, (B, n + 1, N), generator=g).to(dev)
    cost = torch.tensor([0.03125, 0.0625], device=dev)
    sel = (2, True, 0.0, 0.0, 0.0, 1.0 + 1e-5, 0, False)  # age_max .. reserved_units

    def tapes():
        return (torch.zeros(B, n, K, dtype=torch.int64, device=dev),
                torch.zeros(B, n, K, dtype=torch.int64, device=dev),
                torch.zeros(B, n, K, dtype=torch.bool, device=dev),
                torch.zeros(B, n, device=dev),
                torch.zeros(B, n, K, dtype=torch.bool, device=dev))

    h = f(B, N, d) * 0.3
    q = h.mean(dim=1)
    cells64 = idx.clone()
    valid_b = valid.bool()
    cells64[~valid_b] = 0
    y, gate = f(B, K, d), f(B, K, d) + 2.0
    w = torch.rand(d, generator=g).to(dev) + 0.5
    pos = torch.randint(0, 9, (B,), generator=g).to(dev)
    th = torch.zeros(B, n + 1, N, d, device=dev)
    th[:, 1] = h
    tq = torch.zeros(B, n + 1, d, device=dev)
    tq[:, 1] = q
    ta = torch.zeros(B, n + 1, N, dtype=torch.int64, device=dev)
    ta[:, 1] = age
    dec_c = torch.zeros(B, n, K, dtype=torch.int64, device=dev)
    dec_v = torch.zeros(B, n, K, dtype=torch.bool, device=dev)
    dec_c[:, 1], dec_v[:, 1] = cells64, valid_b
    reset = torch.zeros(B, n, dtype=torch.bool, device=dev)
    reset[2, 2] = True
    c, b = f(B, K, d).tanh(), torch.sigmoid(f(B, K, d))
    wide = f(B * K, d + 3)  # a wider product: the gate is its last d columns (a strided view)
    deg = torch.tensor([2, 0, 1, 3, 1, 0, 2, 1, 1, 0, 2, 1])
    indptr = torch.cat([torch.zeros(1, dtype=torch.int64), deg.cumsum(0)]).to(torch.int32)
    csr = (indptr.to(dev), torch.randint(0, N, (int(indptr[-1]),), generator=g,
                                         dtype=torch.int32).to(dev),
           torch.rand(int(indptr[-1]), generator=g).to(dev))
    return {
        "gather_concat": (ops.gather_op, (f(B, d), f(B, d), f(B, N, d), f(B, K, d), idx),
                          (0, 1, 2, 3)),
        "gather_concat_backward": (ops.gather_backward, (f(B, K, 4 * d), idx, N), ()),
        "grouped_unit_mlp": (ops.mlp_op,
                             (f(5, 4 * d), torch.tensor([0, 1, 1, 0, 1], device=dev),
                              f(3, 4 * d, 6), f(3, 6), f(3, 6, d), f(3, d)), (0, 2, 3, 4, 5)),
        "grouped_unit_mlp_backward": (ops.mlp_backward,
                                      (f(5, 4 * d), torch.tensor([0, 1, 1, 0, 1], device=dev),
                                       f(3, 4 * d, 6), f(3, 6, d), f(5, 6), f(5, d)), ()),
        "csr_messages": (ops.messages_op,
                         (f(B, N, d), csr[0], csr[1], csr[2], f(d, d), idx), (0, 3, 4)),
        "csr_messages_backward": (ops.messages_backward,
                                  (f(B, N, d), csr[0], csr[1], csr[2], f(d, d), idx, f(B, K, d)),
                                  ()),
        "gated_delta_update": (ops.update_inplace,
                               (h.clone(), q.clone(), age.to(torch.int32), idx, valid, c, b), ()),
        "gated_delta_update_functional": (ops.update_op,
                                          (h.clone(), q.clone(), age, idx, valid, c, b),
                                          (0, 1, 5, 6)),
        "gated_delta_update_state": (ops.state_update_op,
                                     (h.clone(), q.clone(), age, idx, valid, c, b), (0, 1, 5, 6)),
        "gated_delta_update_backward": (ops.update_backward,
                                        (idx, valid, c, b, h[:, :K].contiguous(), f(B, N, d),
                                         f(B, d)), ()),
        "window_select": (window.select_op, (logits, age, cost, K) + sel, ()),
        "window_select_tape": (window.select_tape_op, (logits, tape_age, cost) + tapes() + (1,) + sel,
                               ()),
        "window_select_fold": (window.select_fold_op,
                               (torch.cat([logits.reshape(B * N, M), f(B * N, 3)], 1), tape_age,
                                cost) + tapes() + (1, M) + sel, ()),
        "window_cell_update": (window.cell_update_op,
                               (y, gate, h, q, age, pos, cells64, valid_b, w, True, 1e-6), ()),
        "window_update_fold": (window.update_fold_op,
                               (y.to(torch.bfloat16), wide[:, 3:], th, tq, ta, dec_c, dec_v, w,
                                reset, torch.zeros(B, n, K, d, device=dev),
                                torch.zeros(B, n, device=dev), torch.zeros(B, n, d, device=dev),
                                torch.zeros(n, B, 5 + 2 * d + 3, dtype=torch.bfloat16, device=dev),
                                f(B, n, 5), f(B, n, 3).to(torch.bfloat16), 1, True, 1e-6, 2), ()),
        "window_cell_round": (window.cell_round_op,
                              (f(B, d), f(B, d), h, q, age, cells64,
                               torch.randint(0, M, (B, K), generator=g).to(dev), valid_b,
                               valid_b.float(), f(d, d), torch.rand(N, 2, generator=g).to(dev),
                               torch.randint(0, N, (N, 2), generator=g).to(dev), f(4 * d),
                               f(d, 4 * d), f(d), f(M, 4 * d, 6), f(M, 6), f(M, 6, d), f(M, d),
                               f(d, d), w, True, 1e-6, 1e-6), ()),
        "window_update_tape": (window.update_tape_op,
                               (y, gate, th, tq, ta, dec_c, dec_v, w, reset,
                                torch.zeros(B, n, K, d, device=dev), torch.zeros(B, n, device=dev),
                                torch.zeros(B, n, d, device=dev), 1, True, 1e-6), ()),
    }


OP_NAMES = ["gather_concat", "gather_concat_backward", "grouped_unit_mlp",
            "grouped_unit_mlp_backward", "csr_messages", "csr_messages_backward",
            "gated_delta_update",
            "gated_delta_update_functional", "gated_delta_update_state",
            "gated_delta_update_backward", "window_select", "window_select_tape",
            "window_select_fold", "window_cell_update", "window_update_tape",
            "window_update_fold", "window_cell_round"]


def _clone(args):
    return tuple(a.clone() if isinstance(a, torch.Tensor) else a for a in args)


@pytest.mark.parametrize("name", OP_NAMES)
def test_opcheck_each_op(mods, cuda_device, name):
    op, args, grads = _cases(cuda_device)[name]
    args = list(_clone(args))
    for i in grads:
        args[i] = args[i].detach().requires_grad_(True)
    torch.library.opcheck(op, tuple(args))


def _outputs(res):
    if res is None:
        return ()
    return tuple(res) if isinstance(res, (tuple, list)) else (res,)


@pytest.mark.parametrize("name", OP_NAMES)
def test_first_dispatch_on_a_fresh_thread(mods, cuda_device, name):
    """The library is prepared on the main thread; a thread that never called it gets the same
    results (its own last-error slot, the device's current stream), and the mutated inputs of
    the in-place and tape ops too."""
    op, args, _ = _cases(cuda_device)[name]
    a_main = _clone(args)
    want = _outputs(op(*a_main))
    torch.cuda.synchronize()

    def first_call():
        a = _clone(args)
        out = _outputs(op(*a))
        torch.cuda.synchronize()
        return out, a

    with ThreadPoolExecutor(max_workers=1) as pool:
        got, a_thread = pool.submit(first_call).result(timeout=60)
    for x, y in zip(got, want):
        assert torch.equal(x, y)
    for x, y in zip(a_thread, a_main):  # in-place and tape outputs
        if isinstance(x, torch.Tensor):
            assert torch.equal(x, y)


@pytest.mark.parametrize("cand_norm", ["rms", "none"])
def test_tape_ops_write_what_the_plain_ops_return(mods, cuda_device, cand_norm):
    """``select_tape`` / ``update_tape`` over a block of positions against ``select`` /
    ``cell_update`` and ``CellGraphState.reset`` position by position (the same kernels, so bit
    for bit): record ``t`` of the decision tape; record ``t + 1`` of the state tape with the next
    position's reset applied (resets at the block's first, interior and last positions, and two
    in a row); the summary, slots and maxima before that reset; a last record that is never
    reset; and no record written but the position's own (the tapes start as a sentinel)."""
    from hsn_amd.state import CandidateSpec, CellGraphState
    from hsn_amd.window import BUDGET_SLACK

    _, window = mods
    dev = cuda_device
    g = torch.Generator().manual_seed(23)
    B, n, N, M, d, K = 5, 6, 24, 3, 8, 4
    cost = torch.tensor([0.03125, 0.0234375, 0.0390625], device=dev)
    cell = (CandidateSpec.rms((torch.rand(d, generator=g) + 0.5).to(dev))
            if cand_norm == "rms" else CandidateSpec.plain(d, dev))
    state = CellGraphState.make(h=(torch.rand(B, N, d, generator=g) * 1.6 - 0.8).to(dev),
                                q=torch.zeros(B, d, device=dev),
                                age=torch.zeros(B, N, dtype=torch.int64, device=dev),
                                pos=torch.zeros(B, dtype=torch.int64, device=dev))
    state = state._replace(q=state.h.mean(dim=1))
    for _ in range(4):
        state = state.tick((torch.rand(B, N, generator=g) < 0.5).to(dev))
    reset = torch.zeros(B, n, dtype=torch.bool)
    reset[0, 0] = True
    reset[1, 3] = True
    reset[2, n - 1] = True
    reset[3, 1] = reset[3, 2] = True
    reset = reset.to(dev)
    sentinel = 7.0
    tape_h = torch.full((B, n + 1, N, d), sentinel, device=dev)
    tape_q = torch.full((B, n + 1, d), sentinel, device=dev)
    tape_age = torch.full((B, n + 1, N), 7, dtype=torch.int64, device=dev)
    cells = torch.full((B, n, K), 7, dtype=torch.int64, device=dev)
    units = torch.full((B, n, K), 7, dtype=torch.int64, device=dev)
    valid = torch.zeros((B, n, K), dtype=torch.bool, device=dev)
    refreshed = torch.zeros((B, n, K), dtype=torch.bool, device=dev)
    theta = torch.full((B, n), sentinel, device=dev)
    h_sel = torch.full((B, n, K, d), sentinel, device=dev)
    h_max = torch.full((B, n), sentinel, device=dev)
    qs = torch.full((B, n, d), sentinel, device=dev)
    first = state.reset(reset[:, 0])
    tape_h[:, 0], tape_q[:, 0], tape_age[:, 0] = first.h, first.q, first.age
    keys = dict(age_max=2, probes=True, lambda_cost=0.0, cell_overhead=0.0, shared_cost=0.0,
                limit=0.1 * (1.0 + BUDGET_SLACK))
    fired = padded = 0
    for t in range(n):
        pre = state.reset(reset[:, t])
        assert torch.equal(tape_h[:, t], pre.h) and torch.equal(tape_q[:, t], pre.q)
        assert torch.equal(tape_age[:, t], pre.age)
        logits = torch.randn(B, N, M, generator=g).to(dev)
        want = window.select(logits, pre.age, cost, k=K, **keys)
        window.select_tape(logits, tape_age, cost, cells, units, valid, theta, refreshed, t=t,
                           **keys)
        got = (cells[:, t], units[:, t], valid[:, t], theta[:, t], refreshed[:, t])
        for a, b in zip(got, want):
            assert torch.equal(a, b)
        assert bool((cells[:, t + 1:] == 7).all()) and bool((theta[:, t + 1:] == 7).all())
        fired += int(refreshed[:, t].sum())
        padded += int((~valid[:, t]).sum())
        y = torch.randn(B, K, d, generator=g).to(dev)
        gate = torch.randn(B, K, d, generator=g).to(dev)
        after, slots, top = window.cell_update(cell, y, gate, pre, want[0], want[2])
        window.update_tape(cell, y, gate, tape_h, tape_q, tape_age, cells, valid, reset, h_sel,
                           h_max, qs, t=t)
        nxt = after.reset(reset[:, t + 1]) if t + 1 < n else after
        assert torch.equal(tape_h[:, t + 1], nxt.h) and torch.equal(tape_q[:, t + 1], nxt.q)
        assert torch.equal(tape_age[:, t + 1], nxt.age)
        assert torch.equal(qs[:, t], after.q) and torch.equal(h_sel[:, t], slots)
        assert torch.equal(h_max[:, t], top)
        assert bool((tape_h[:, t + 2:] == sentinel).all())
        assert bool((qs[:, t + 1:] == sentinel).all())
        assert torch.equal(tape_h[:, t], pre.h)  # the record it read is untouched
        state = after
    assert fired > 0 and padded > 0  # probes and padded slots were exercised


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n_fast", [0, 3])
def test_update_fold_is_update_tape_and_the_next_row(mods, cuda_device, x_dtype, n_fast):
    """``update_fold`` on the products as they are (bf16 ``y``, an fp32 gate that is a strided
    view of a wider product) writes exactly what ``update_tape`` writes from their fp32 copies,
    and record ``t + 1`` of ``x`` is ``[z; q; context(; f)]`` of position ``t + 1`` rounded to
    ``x``'s dtype: ``q`` after the next reset (set on row 1), ``f`` the mean of the first
    ``n_fast`` cells summed in cell order; at the last record ``x`` is left alone
    (reference window.py:765-853)."""
    _, window = mods
    dev = cuda_device
    g = torch.Generator().manual_seed(61)
    B, n, N, d, K, d_z, d_c = 3, 4, 20, 16, 4, 6, 5
    f = lambda *s: torch.randn(*s, generator=g).to(dev)  # noqa: E731
    w = (torch.rand(d, generator=g) + 0.5).to(dev)
    th, tq = f(B, n + 1, N, d) * 0.4, f(B, n + 1, d) * 0.1
    ta = torch.randint(0, 5, (B, n + 1, N), generator=g).to(dev)
    dec_c = torch.stack([torch.stack([torch.randperm(N, generator=g)[:K] for _ in range(n)])
                         for _ in range(B)]).to(dev)
    dec_v = torch.ones(B, n, K, dtype=torch.bool, device=dev)
    dec_v[2, :, 1] = False
    reset = torch.zeros(B, n, dtype=torch.bool, device=dev)
    reset[1, 2] = True
    z = f(B, n, d_z).to(torch.bfloat16)
    ctx = f(B, n, d_c)
    width = d_z + d + d_c + (d if n_fast else 0)
    for t in (1, n - 1):
        y = f(B, K, d).to(torch.bfloat16)
        wide = f(B * K, d + 7)
        gate = wide[:, 7:]
        outs = []
        for fold in (False, True):
            tapes = [th.clone(), tq.clone(), ta.clone()]
            rec = [torch.full((B, n, K, d), 7.0, device=dev), torch.full((B, n), 7.0, device=dev),
                   torch.full((B, n, d), 7.0, device=dev)]
            x = torch.full((n, B, width), 7.0, device=dev).to(x_dtype)
            if fold:
                window.update_fold_op(y, gate, *tapes, dec_c, dec_v, w, reset, *rec, x, z, ctx, t,
                                      True, 1e-6, n_fast)
            else:
                window.update_tape_op(y.float(), gate.contiguous().reshape(B, K, d), *tapes, dec_c,
                                      dec_v, w, reset, *rec, t, True, 1e-6)
            outs.append((tapes, rec, x))
        for a, b_ in zip(outs[0][0] + outs[0][1], outs[1][0] + outs[1][1]):
            assert torch.equal(a, b_)
        x = outs[1][2]
        if t + 1 < n:
            h1, q1 = outs[0][0][0][:, t + 1].cpu(), outs[0][0][1][:, t + 1].cpu()
            parts = [z[:, t + 1].float().cpu(), q1, ctx[:, t + 1].cpu()]
            if n_fast:
                s = torch.zeros(B, d)
                for cell in range(n_fast):
                    s = s + h1[:, cell]
                parts.append(s / n_fast)
            want = torch.cat(parts, dim=1).to(x_dtype)
            assert torch.equal(x[t + 1].cpu(), want)
            assert bool((q1[1] == 0).all())  # the reset of row 1 at position t + 1 = 2
            others = [r for r in range(n) if r != t + 1]
            assert bool((x[others].float() == 7.0).all())
        else:
            assert bool((x.float() == 7.0).all())


@pytest.mark.parametrize("x_dtype,cand_norm", [(torch.float32, True), (torch.bfloat16, False)])
def test_folded_sweep_walks_a_block_like_the_oracle(mods, cuda_device, x_dtype, cand_norm):
    """The folded sweep as the reference's model runs it over a block (``select_fold`` ->
    ``update_fold`` position by position, the logits read in place from a wider scorer product,
    a bf16 ``y``, the gate a strided view of a wider fp32 product), against the oracle's
    per-position chain (``reset -> Router.select -> candidate / gate -> gated update -> tick``,
    the state in float64): resets at the block's first, interior and last positions and two in
    a row, two reserved cells with fixed units, probes on the ages, a row budget that pads
    slots, and the fast read of the first three cells into each next row of ``x``. Decisions
    and ages bit for bit; states, summaries, maxima and the folded rows within 1e-5 (fp32
    ``x``) or one bf16 rounding."""
    from oracle import hsn_oracle as O

    from hsn_amd.window import BUDGET_SLACK

    _, window = mods
    dev = cuda_device
    g = torch.Generator().manual_seed(71)
    B, n, N, M, d, K, d_z, d_c, n_fast, pad = 4, 9, 30, 2, 16, 6, 5, 3, 3, 4
    cost = torch.tensor([0.03125, 0.046875])
    keys = dict(age_max=3, probes=True, lambda_cost=0.0, cell_overhead=0.0, shared_cost=0.0,
                limit=0.12 * (1.0 + BUDGET_SLACK), reserved=2, reserved_units=True)
    cand_w = torch.rand(d, generator=g) + 0.5
    eps = 1e-6
    reset = torch.zeros(B, n, dtype=torch.bool)
    reset[0, 0] = True
    reset[1, 4] = True
    reset[2, n - 1] = True
    reset[3, 2] = reset[3, 3] = True
    h0 = torch.rand(B, N, d, generator=g) * 1.6 - 0.8
    q0 = h0.mean(dim=1)
    age0 = torch.randint(0, 6, (B, N), generator=g)
    pos0 = torch.randint(0, 9, (B,), generator=g)
    logits = torch.randn(B, n, N, M, generator=g)
    ys = torch.randn(B, n, K, d, generator=g).to(torch.bfloat16)  # the product as the model has it
    gates = torch.randn(n, B * K, d + pad, generator=g)  # the gate: columns pad.. of a wider product
    z = torch.randn(B, n, d_z, generator=g).to(x_dtype)
    ctx = torch.randn(B, n, d_c, generator=g)

    # the oracle: float64 state, decisions from the fp32 logits and the integer ages
    h, q, age, pos = h0.double(), q0.double(), age0.clone(), pos0.clone()
    rec = {k: [] for k in ("h", "q", "age", "cells", "units", "valid", "theta", "refreshed",
                           "q_post", "h_sel", "h_max")}
    for t in range(n):
        h, q, age, pos = O.reset_state(h, q, age, pos, reset[:, t])
        rec["h"].append(h), rec["q"].append(q), rec["age"].append(age)
        cells, units, valid, theta, refreshed = O.router_select(logits[:, t], age, cost, k=K, **keys)
        gate_t = gates[t, :, pad:].reshape(B, K, d)
        h, q, age, pos, h_sel, h_max, _ = O.cell_update(
            ys[:, t].float(), gate_t, h, q, age, pos, cells, valid, cand_norm=cand_norm,
            cand_w=cand_w.double() if cand_norm else None, cand_eps=eps)
        for k_, v_ in (("cells", cells), ("units", units), ("valid", valid), ("theta", theta),
                       ("refreshed", refreshed), ("q_post", q), ("h_sel", h_sel),
                       ("h_max", h_max)):
            rec[k_].append(v_)
    rec["h"].append(h), rec["q"].append(q), rec["age"].append(age)  # the block's end
    assert any(bool(v.all()) is False for v in rec["valid"])  # the budget padded some slots

    # the GPU: the tapes, record 0 the start state after the first reset
    first = O.reset_state(h0, q0, age0, pos0, reset[:, 0])
    tape_h = torch.full((B, n + 1, N, d), 7.0, device=dev)
    tape_q = torch.full((B, n + 1, d), 7.0, device=dev)
    tape_age = torch.full((B, n + 1, N), 7, dtype=torch.int64, device=dev)
    tape_h[:, 0], tape_q[:, 0], tape_age[:, 0] = first[0].to(dev), first[1].to(dev), first[2].to(dev)
    cells = torch.zeros(B, n, K, dtype=torch.int64, device=dev)
    units = torch.zeros(B, n, K, dtype=torch.int64, device=dev)
    valid = torch.zeros(B, n, K, dtype=torch.bool, device=dev)
    refreshed = torch.zeros(B, n, K, dtype=torch.bool, device=dev)
    theta = torch.zeros(B, n, device=dev)
    h_sel = torch.zeros(B, n, K, d, device=dev)
    h_max = torch.zeros(B, n, device=dev)
    qs = torch.zeros(B, n, d, device=dev)
    x = torch.full((n, B, d_z + d + d_c + d), 7.0, device=dev).to(x_dtype)
    zd, ctxd, cw, rd = z.to(dev), ctx.to(dev), cand_w.to(dev), reset.to(dev)
    gd = gates.to(dev)
    for t in range(n):
        scored = torch.cat([logits[:, t].reshape(B * N, M), torch.randn(B * N, 3, generator=g)],
                           dim=1).to(dev)  # the logits in the product's first M columns
        window.select_fold_op(scored, tape_age, cost.to(dev), cells, units, valid, theta,
                              refreshed, t, M, keys["age_max"], keys["probes"],
                              keys["lambda_cost"], keys["cell_overhead"], keys["shared_cost"],
                              keys["limit"], keys["reserved"], keys["reserved_units"])
        window.update_fold_op(ys[:, t].to(dev), gd[t, :, pad:], tape_h, tape_q, tape_age, cells,
                              valid, cw, rd, h_sel, h_max, qs, x, zd, ctxd, t, cand_norm, eps,
                              n_fast)
    torch.cuda.synchronize()

    for name, got in (("cells", cells), ("units", units), ("valid", valid),
                      ("refreshed", refreshed), ("theta", theta)):
        want = torch.stack(rec[name], dim=1)
        got = got.cpu()
        if name in ("cells", "units"):  # padded slots: the router's placeholders
            got, want = got.masked_fill(~valid.cpu(), 0), want.masked_fill(~valid.cpu(), 0)
        assert torch.equal(got, want), name
    assert torch.equal(tape_age.cpu(), torch.stack(rec["age"], dim=1))
    tol = dict(atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(tape_h.cpu().double(), torch.stack(rec["h"], dim=1), **tol)
    torch.testing.assert_close(tape_q.cpu().double(), torch.stack(rec["q"], dim=1), **tol)
    torch.testing.assert_close(qs.cpu().double(), torch.stack(rec["q_post"], dim=1), **tol)
    torch.testing.assert_close(h_max.cpu().double(), torch.stack(rec["h_max"], dim=1), **tol)
    vm = valid.cpu()[..., None]
    torch.testing.assert_close(torch.where(vm, h_sel.cpu().double(), 0.0),
                               torch.where(vm, torch.stack(rec["h_sel"], dim=1), 0.0), **tol)
    # the folded rows: record t + 1's [z; q; context; mean of cells 0 .. n_fast - 1]
    for t in range(n - 1):
        hr, qr = rec["h"][t + 1], rec["q"][t + 1]
        fast = hr[:, :n_fast].sum(dim=1) / n_fast
        want = torch.cat([z[:, t + 1].double(), qr, ctx[:, t + 1].double(), fast], dim=1)
        xt = x[t + 1].cpu().double()
        if x_dtype == torch.float32:
            torch.testing.assert_close(xt, want, **tol)
        else:  # one rounding to bf16 of values within fp32 error of the oracle's
            torch.testing.assert_close(xt, want, atol=1e-2, rtol=8e-3)
    assert bool((x[0].float() == 7.0).all())  # record 0 is the caller's
