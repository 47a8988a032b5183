"""The trainer's per-step passes (``hsn_amd.trainer``, ``include/hsn_trainer.h``) against the
PyTorch multi-tensor operations they replace, on the same device, bit for bit, and against the CPU
oracle. GPU only.

The operation sequences below are the reference callers' (``python/hsn/train/lazy_adam.py:462-486``
for the dense step, ``:573-626`` for the masked unit step, ``weight_ema``'s ``_foreach_lerp_``,
``grad_norm``'s float64 scaling, ``update_limit``'s squares and projection). Bar: every output
element's bits equal (NaN payloads aside: a NaN matches a NaN).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import hsn_oracle as O

pytestmark = pytest.mark.gpu

# ragged sizes: one element, under a chunk (1024 elements), a whole chunk, one over, several
SIZES = (1, 7, 1023, 1024, 1025, 4096, 70001)


@pytest.fixture(scope="module")
def dev(cuda_device):
    from hsn_amd import trainer

    assert trainer.ready(cuda_device), "the HIP library must be built for the GPU tests"
    return cuda_device


def _same_bits(got: torch.Tensor, want: torch.Tensor, what: str = ""):
    got = got.detach().contiguous()
    want = want.detach().contiguous()
    assert got.shape == want.shape and got.dtype == want.dtype, what
    both_nan = torch.isnan(got) & torch.isnan(want)
    differ = (got.view(torch.int32) != want.view(torch.int32)) & ~both_nan
    if bool(differ.any()):
        i = int(differ.flatten().nonzero()[0])
        raise AssertionError(
            f"{what}: {int(differ.sum())} of {got.numel()} elements differ; first at {i}: "
            f"got {got.flatten()[i].item()!r}, want {want.flatten()[i].item()!r}")


class _Slab:
    """Tensors carved out of one buffer with guard words between them (a pass that writes past a
    tensor's end changes a guard)."""

    GUARD = 64
    SENTINEL = -12345.678

    def __init__(self, sizes, dev, aligned=False):
        """aligned: every view starts on a 16-byte boundary; else the views start wherever the
        sizes put them."""
        total = sum(sizes) + (self.GUARD + 4) * (len(sizes) + 1)
        self.buf = torch.full((total,), self.SENTINEL, device=dev)
        self.views, self.guards = [], []
        at = self.GUARD
        self.guards.append((0, self.GUARD))
        for s in sizes:
            self.views.append(self.buf[at:at + s])
            at += s
            end = at + self.GUARD + ((-(at + self.GUARD)) % 4 if aligned else 0)
            self.guards.append((at, end))
            at = end

    def check_guards(self):
        for a, b in self.guards:
            assert bool((self.buf[a:b] == self.SENTINEL).all()), f"guard [{a}, {b}) overwritten"


def _rows(sizes, dev, n_rows, gen, special=False, aligned=False):
    slabs = [_Slab(sizes, dev, aligned) for _ in range(n_rows)]
    for slab in slabs:
        for v in slab.views:
            v.copy_(torch.randn(v.numel(), generator=gen).to(dev))
            if special and v.numel() >= 8:
                v[:8] = torch.tensor([0.0, -0.0, 1e-40, -3e-39, 1e30, -2e-30, 7.0, 1.0])
    return slabs


def _dense_reference(params, grads, exp_avgs, exp_avg_sqs, step, lr, betas, eps, wd):
    beta1, beta2 = betas
    if wd != 0:
        torch._foreach_mul_(params, 1 - lr * wd)
    torch._foreach_lerp_(exp_avgs, grads, 1 - beta1)
    torch._foreach_mul_(exp_avg_sqs, beta2)
    torch._foreach_addcmul_(exp_avg_sqs, grads, grads, value=1 - beta2)
    bias_correction1 = 1 - beta1**step
    bias_correction2 = 1 - beta2**step
    step_size = lr / bias_correction1
    denoms = torch._foreach_sqrt(exp_avg_sqs)
    torch._foreach_div_(denoms, bias_correction2**0.5)
    torch._foreach_add_(denoms, eps)
    torch._foreach_addcdiv_(params, exp_avgs, denoms, value=-step_size)


@pytest.mark.parametrize("aligned", [True, False])
@pytest.mark.parametrize("betas,wd", [((0.9, 0.999), 0.01), ((0.9, 0.999), 0.0),
                                      ((0.0, 0.95), 0.1), ((0.5, 0.0), 0.01)])
def test_adamw_pass_equals_the_multi_tensor_step(dev, betas, wd, aligned):
    from hsn_amd import trainer

    gen = torch.Generator().manual_seed(101)
    lr, eps = 3e-3, 1e-8
    mine = _rows(SIZES, dev, 4, gen, special=True, aligned=aligned)
    for r in (2, 3):  # moments start at zero, then grow
        for v in mine[r].views:
            v.zero_()
    theirs = [[v.clone() for v in slab.views] for slab in mine]
    for step in range(1, 7):
        grads = [torch.randn(s, generator=gen).to(dev) * (10.0 ** (step - 3)) for s in SIZES]
        if step == 4:
            grads[2].zero_()  # a zero gradient on a moving state
        for slab, g in zip(mine[1].views, grads):
            slab.copy_(g)
        for t, g in zip(theirs[1], grads):
            t.copy_(g)
        assert trainer.adamw(mine[0].views, mine[1].views, mine[2].views, mine[3].views, lr=lr,
                             beta1=betas[0], beta2=betas[1], eps=eps, weight_decay=wd, step=step)
        _dense_reference(theirs[0], theirs[1], theirs[2], theirs[3], step, lr, betas, eps, wd)
        torch.cuda.synchronize()
        for r, name in ((0, "param"), (2, "exp_avg"), (3, "exp_avg_sq")):
            for j, (got, want) in enumerate(zip(mine[r].views, theirs[r])):
                _same_bits(got, want, f"step {step} {name}[{j}] ({SIZES[j]} elements)")
    for slab in mine:
        slab.check_guards()


def _unit_reference(p, grad, exp_avg, exp_avg_sq, step_cpu, active_cpu, lr, betas, eps, wd):
    """lazy_adam._unit_step's operations for one stacked tensor (the step count already
    advanced in step_cpu)."""
    beta1, beta2 = betas
    M = p.shape[0]
    view = (M,) + (1,) * (p.dim() - 1)
    actv = active_cpu.to(p.device).view(view)

    def const(value):
        return torch.tensor(value, dtype=p.dtype, device=p.device)

    def coef(on, off):
        return torch.where(actv, const(on), const(off))

    g = torch.where(actv, grad, const(0.0))
    if wd != 0:
        p.mul_(coef(1 - lr * wd, 1.0))
    exp_avg.lerp_(g, coef(1 - beta1, 0.0))
    exp_avg_sq.mul_(coef(beta2, 1.0)).addcmul_(g, g, value=1 - beta2)
    step_size, bc2s = _unit_bias_terms(step_cpu, active_cpu, lr, betas)
    denom = exp_avg_sq.sqrt().div_(bc2s.to(p.device).view(view)).add_(eps)
    p.addcdiv_(exp_avg.mul(step_size.to(p.device).view(view)), denom, value=-1.0)


def _unit_bias_terms(step_cpu, active_cpu, lr, betas):
    beta1, beta2 = betas
    steps = step_cpu.to(torch.float64)
    bias_correction1 = 1 - torch.pow(beta1, steps)
    bias_correction2 = 1 - torch.pow(beta2, steps)
    zero = torch.zeros((), dtype=torch.float64)
    one = torch.ones((), dtype=torch.float64)
    step_size = torch.where(active_cpu, lr / bias_correction1, zero).to(torch.float32)
    bc2s = torch.where(active_cpu, bias_correction2.pow(0.5), one).to(torch.float32)
    return step_size, bc2s


def _unit_call(trainer, ps, gs, ms, vs, step_cpu, active_cpu, lr, betas, eps, wd):
    """_unit_steps_fused's coefficients (lazy_adam.py:528-571) and the pass."""
    beta1, beta2 = betas
    step_size, bc2s = _unit_bias_terms(step_cpu, active_cpu, lr, betas)
    active = active_cpu.tolist()
    return trainer.adamw_units(
        ps, gs, ms, vs, n_units=len(active), active=active,
        decay=[1 - lr * wd if on else 1.0 for on in active],
        lerp_weight=[1 - beta1 if on else 0.0 for on in active],
        beta2_factor=[beta2 if on else 1.0 for on in active],
        bias_correction2_sqrt=bc2s.tolist(), step_size=step_size.tolist(),
        beta2=beta2, eps=eps, weight_decay=wd)


@pytest.mark.parametrize("M", [1, 5, 64])
@pytest.mark.parametrize("wd", [0.01, 0.0])
def test_unit_pass_equals_the_masked_step(dev, M, wd):
    from hsn_amd import trainer

    gen = torch.Generator().manual_seed(202 + M)
    lr, betas, eps = 1e-3, (0.9, 0.99), 1e-8
    # units shorter and longer than a chunk (1024 elements)
    shapes = [(M,), (M, 3), (M, 7, 33), (M, 1100), (M, 4500)]
    ps = [torch.randn(s, generator=gen).to(dev) for s in shapes]
    ms = [torch.zeros(s, device=dev) for s in shapes]
    vs = [torch.zeros(s, device=dev) for s in shapes]
    theirs = [[t.clone() for t in row] for row in (ps, ms, vs)]
    step_mine = torch.zeros(M, dtype=torch.int64)
    step_theirs = torch.zeros(M, dtype=torch.int64)
    for it in range(6):
        active = torch.rand(M, generator=gen) < 0.6
        if it == 0:
            active[:] = True
        gs = [torch.randn(s, generator=gen).to(dev) * 3.0 for s in shapes]
        advance = active.to(torch.int64)
        assert _unit_call(trainer, ps, gs, ms, vs, step_mine + advance, active, lr, betas, eps, wd)
        step_mine += advance
        step_theirs += advance
        for j in range(len(shapes)):
            _unit_reference(theirs[0][j], gs[j], theirs[1][j], theirs[2][j], step_theirs, active,
                            lr, betas, eps, wd)
        torch.cuda.synchronize()
        for r, (mine_row, name) in enumerate(((ps, "param"), (ms, "exp_avg"), (vs, "exp_avg_sq"))):
            for j in range(len(shapes)):
                _same_bits(mine_row[j], theirs[r][j], f"iteration {it} {name}{shapes[j]}")


def test_adamw_passes_equal_the_oracle(dev):
    """The dense and unit passes against the oracle's restatement on the same inputs (the oracle's
    own pins are CPU tests)."""
    from hsn_amd import trainer

    rng = np.random.default_rng(303)
    lr, beta1, beta2, eps, wd, step = 2e-3, 0.9, 0.999, 1e-8, 0.05, 3
    p, g, m = (rng.standard_normal(3000).astype(np.float32) for _ in range(3))
    v = np.abs(rng.standard_normal(3000)).astype(np.float32)
    dev_rows = [torch.from_numpy(x.copy()).to(dev) for x in (p, g, m, v)]
    assert trainer.adamw([dev_rows[0]], [dev_rows[1]], [dev_rows[2]], [dev_rows[3]], lr=lr,
                         beta1=beta1, beta2=beta2, eps=eps, weight_decay=wd, step=step)
    coefs = [1 - lr * wd, 1 - beta1, beta2, 1 - beta2, 1.0 / (1 - beta2**step) ** 0.5, eps,
             -lr / (1 - beta1**step)]
    want = O.tr_adamw(p, g, m, v, coefs, True)
    for got, w, name in zip((dev_rows[0], dev_rows[2], dev_rows[3]), want, ("p", "m", "v")):
        _same_bits(got.cpu(), torch.from_numpy(np.ascontiguousarray(w)), f"dense {name}")

    M = 6
    shape = (M, 250)
    pu, gu, mu = (rng.standard_normal(shape).astype(np.float32) for _ in range(3))
    vu = np.abs(rng.standard_normal(shape)).astype(np.float32)
    active = [True, False, True, True, False, True]
    steps = [3, 1, 2, 5, 4, 1]
    table = np.float32([
        [1.0 if a else 0.0 for a in active],
        [1 - lr * wd if a else 1.0 for a in active],
        [1 - beta1 if a else 0.0 for a in active],
        [beta2 if a else 1.0 for a in active],
        [(1 - beta2**s) ** 0.5 if a else 1.0 for a, s in zip(active, steps)],
        [lr / (1 - beta1**s) if a else 0.0 for a, s in zip(active, steps)],
    ])
    rows = [torch.from_numpy(x.copy()).to(dev) for x in (pu, gu, mu, vu)]
    assert trainer.adamw_units([rows[0]], [rows[1]], [rows[2]], [rows[3]], n_units=M,
                               active=active, decay=table[1].tolist(),
                               lerp_weight=table[2].tolist(), beta2_factor=table[3].tolist(),
                               bias_correction2_sqrt=table[4].tolist(),
                               step_size=table[5].tolist(), beta2=beta2, eps=eps,
                               weight_decay=wd)
    want = O.tr_adamw_units(pu, gu, mu, vu, table, 1 - beta2, eps, True)
    for got, w, name in zip((rows[0], rows[2], rows[3]), want, ("p", "m", "v")):
        _same_bits(got.cpu(), torch.from_numpy(np.ascontiguousarray(w)), f"units {name}")


@pytest.mark.parametrize("weight", [0.0, 1e-3, 0.3, 0.4999, 0.5, 0.75, 1.0])
def test_lerp_pass_equals_foreach_lerp(dev, weight):
    """103 tensors: more than one launch holds."""
    from hsn_amd import trainer

    gen = torch.Generator().manual_seed(404)
    sizes = [int(s) for s in torch.randint(0, 9000, (103,), generator=gen)]
    sizes[5] = 0
    mine = _rows(sizes, dev, 2, gen, special=True, aligned=weight < 0.5)
    theirs = [t.clone() for t in mine[0].views]
    ends = [t.clone() for t in mine[1].views]
    oracle = [O.tr_lerp(s.cpu().numpy(), e.cpu().numpy(), weight)
              for s, e in zip(theirs[:12], ends)]
    assert trainer.lerp(mine[0].views, mine[1].views, weight)
    torch._foreach_lerp_(theirs, ends, weight)
    torch.cuda.synchronize()
    for j, (got, want) in enumerate(zip(mine[0].views, theirs)):
        _same_bits(got, want, f"lerp w={weight} tensor {j}")
    for j, want in enumerate(oracle):
        _same_bits(mine[0].views[j].cpu(), torch.from_numpy(want), f"lerp tensor {j} vs the oracle")
    mine[0].check_guards()


@pytest.mark.parametrize("aligned", [True, False])
def test_scale64_copy_and_limit_passes(dev, aligned):
    from hsn_amd import trainer

    gen = torch.Generator().manual_seed(505)
    sizes = list(SIZES) + [0, 3]
    grads = _rows(sizes, dev, 1, gen, special=True, aligned=aligned)[0]
    c = 0.123456789012345
    want = [(g.double() * c).float() for g in grads.views]
    oracle = [O.tr_scale64(g.cpu().numpy(), c) for g in grads.views]
    assert trainer.scale64(grads.views, torch.tensor(c, dtype=torch.float64, device=dev))
    torch.cuda.synchronize()
    for j, (got, w, o) in enumerate(zip(grads.views, want, oracle)):
        _same_bits(got, w, f"scale64 tensor {j}")
        _same_bits(got.cpu(), torch.from_numpy(o), f"scale64 tensor {j} vs the oracle")
    grads.check_guards()

    dst = _rows(sizes, dev, 1, gen, aligned=aligned)[0]
    assert trainer.copy(dst.views, grads.views)
    torch.cuda.synchronize()
    for got, w in zip(dst.views, grads.views):
        _same_bits(got, w, "copy")
    dst.check_guards()

    params, olds, old_sq, delta_sq = _rows(sizes, dev, 4, gen, special=True, aligned=aligned)
    assert trainer.limit_squares(params.views, olds.views, old_sq.views, delta_sq.views)
    torch.cuda.synchronize()
    for j in range(len(sizes)):
        _same_bits(old_sq.views[j], olds.views[j].square(), f"old^2 tensor {j}")
        _same_bits(delta_sq.views[j], (params.views[j] - olds.views[j]).square(),
                   f"delta^2 tensor {j}")
        want_o, want_d = O.tr_limit_squares(params.views[j].cpu().numpy(),
                                            olds.views[j].cpu().numpy())
        _same_bits(old_sq.views[j].cpu(), torch.from_numpy(want_o), "old^2 vs the oracle")
        _same_bits(delta_sq.views[j].cpu(), torch.from_numpy(want_d), "delta^2 vs the oracle")
    for slab in (old_sq, delta_sq):
        slab.check_guards()

    applied = _rows(sizes, dev, 1, gen, aligned=aligned)[0]
    groups = [torch.tensor([0.37 + 0.01 * j, float(j % 2)], device=dev) for j in range(len(sizes))]
    before = [p.clone() for p in params.views]
    assert trainer.limit_project(params.views, olds.views, applied.views, groups)
    torch.cuda.synchronize()
    for j, (p0, old, grp) in enumerate(zip(before, olds.views, groups)):
        scale, clipped = grp[0], bool(grp[1] != 0)
        want_p = old + (p0 - old) * scale if clipped else p0
        _same_bits(params.views[j], want_p, f"projected param {j}")
        _same_bits(applied.views[j], (want_p - old).square(), f"applied^2 {j}")
        got_p, got_sq = O.tr_limit_project(p0.cpu().numpy(), old.cpu().numpy(), float(scale),
                                           clipped)
        _same_bits(params.views[j].cpu(), torch.from_numpy(got_p), "projection vs the oracle")
        _same_bits(applied.views[j].cpu(), torch.from_numpy(got_sq), "applied^2 vs the oracle")
    params.check_guards()
    applied.check_guards()


def test_passes_decline_what_they_cannot_take(dev):
    """False and nothing touched for tensors the passes do not take (the caller then runs its
    PyTorch operations)."""
    from hsn_amd import trainer

    a = torch.randn(100, device=dev)
    b = torch.randn(100, device=dev)
    keep = a.clone()
    assert not trainer.lerp([a.double()], [b.double()], 0.5)
    assert not trainer.lerp([a[::2]], [b[::2]], 0.5)  # strided
    assert not trainer.lerp([a], [b[:50]], 0.5)  # unequal sizes
    assert not trainer.lerp([a], [b.cpu()], 0.5)  # another device
    assert not trainer.lerp([], [], 0.5)  # nothing to do
    assert not trainer.adamw_units([a.view(10, 10)], [b.view(10, 10)], [a.view(10, 10)],
                                   [b.view(10, 10)], n_units=65, active=[True] * 65,
                                   decay=[1.0] * 65, lerp_weight=[0.1] * 65,
                                   beta2_factor=[0.9] * 65, bias_correction2_sqrt=[1.0] * 65,
                                   step_size=[0.1] * 65, beta2=0.9, eps=1e-8, weight_decay=0.0)
    assert not trainer.scale64([a], torch.tensor(0.5, device=dev))  # a float32 coefficient
    previous = trainer.set_enabled(False)
    try:
        assert not trainer.lerp([a], [b], 0.5)
    finally:
        trainer.set_enabled(previous)
    torch.cuda.synchronize()
    _same_bits(a, keep, "declined passes leave the tensors alone")
    assert trainer.lerp([a], [b], 0.5)  # and the same call runs once switched back on


def test_adamw_pass_replays_in_a_graph(dev):
    """The pass captured in a HIP graph (its pointer table and coefficients fixed at capture) and
    replayed three times, with eager work and synchronisations between the replays: every replay
    equals the PyTorch sequence at the same step count."""
    from hsn_amd import trainer

    gen = torch.Generator().manual_seed(606)
    sizes = (5, 1024, 3000, 70001)
    lr, betas, eps, wd, step = 1e-3, (0.9, 0.999), 1e-8, 0.02, 4
    rows = [[torch.randn(n, generator=gen).to(dev) for n in sizes] for _ in range(4)]
    for v in rows[3]:
        v.abs_()
    theirs = [[t.clone() for t in row] for row in rows]
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        assert trainer.adamw(*rows, lr=lr, beta1=betas[0], beta2=betas[1], eps=eps,
                             weight_decay=wd, step=step)
    torch.cuda.synchronize()
    # capture records the launch without running it: the state is still the initial one
    for r in (0, 2, 3):
        for got, want in zip(rows[r], theirs[r]):
            _same_bits(got, want, "capture ran nothing")
    for replay in range(3):
        graph.replay()
        _dense_reference(*theirs, step, lr, betas, eps, wd)
        torch.cuda.synchronize()
        for r, name in ((0, "param"), (2, "exp_avg"), (3, "exp_avg_sq")):
            for j, (got, want) in enumerate(zip(rows[r], theirs[r])):
                _same_bits(got, want, f"replay {replay} {name}[{j}]")
        for g in rows[1]:  # eager work between replays: new gradients in place
            g.mul_(-0.5)
        for g in theirs[1]:
            g.mul_(-0.5)
