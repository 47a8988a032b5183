"""The benchmark contract's five configurations on the GPU at their full sizes: tiny (exactly as
stated), bf16 (N=1024, K=16), the TBPTT segment (N=512, d=128, carried over windows) and the
skewed window (N=4096, K=32, Zipf-biased logits). GPU only.

Each test checks size-independent properties on every row: the decisions of spaced positions
equal the oracle's router; q stays the mean of h; the backward is linear in its cotangents
(scaling every cotangent by 2 scales every gradient by exactly 2). One row is also checked
against the oracle's full window. The TBPTT tests check the carried state and its gradient:
two windows with the state carried (forward) and the next window's d_h0, d_q0 fed back as the
end cotangent (backward, the reference's segment semantics) equal one window of twice the
length, and one row of that segment equals the oracle's long window. Config 1 runs exactly as
the contract states it. Bars as in test_window_gpu: decisions bit-exact, fp32 1e-5, bf16 2e-2.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import hsn_oracle as O
from test_window_gpu import BF16_TOL, F32_TOL, _close, _d_q0_exact, _route_cfg

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(cuda_device):
    from hsn_amd import window

    assert window.available(), "the HIP library must be built for the GPU tests"
    return cuda_device


def _put(w, dev):
    return {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in w.items()}


def _forward(w, D, cfg):
    from hsn_amd import window

    return window.window_forward(D["logits"], D["y"], D["gate_pre"], D["reset"], D["h0"],
                                 D["q0"], D["age0"], D["pos0"], D["cost"], cfg)


def _backward(w, got, D, C, n_cells, scale=1.0, d_h_T=None, d_q_T=None):
    from hsn_amd import window

    s = lambda t: None if t is None else t * scale  # noqa: E731
    return window.backward(D["y"], D["gate_pre"], got["h_old"], got["slots"], D["reset"], n_cells,
                           s(C["d_q_pre"]), s(C["d_q_post"]), s(C["d_h_sel"]),
                           s(C["d_h_T"] if d_h_T is None else d_h_T),
                           s(C["d_q_T"] if d_q_T is None else d_q_T))


def _check_config(dev, cfg_w, seed, row, every, tol):
    from hsn_amd.workload import make_cotangents, make_window

    w = make_window(cfg_w, seed)
    cot = make_cotangents(cfg_w, seed)
    cfg = _route_cfg(k=cfg_w.K)
    D, C = _put(w, dev), _put(cot, dev)
    got = _forward(w, D, cfg)
    assert bool(got["valid"].all())  # budget 1.0 and uniform costs: every slot valid
    _close(got["q"], got["h"].mean(dim=1), 1e-5, "q_T vs mean h_T")
    for t in range(0, cfg_w.T, every):
        want = O.router_select(w["logits"][:, t], None, w["cost"], k=cfg_w.K)
        assert torch.equal(got["cells"][:, t].cpu().long(), want[0]), t
        assert torch.equal(got["theta"][:, t].cpu(), want[3]), t
    # one row against the oracle's window (rows are independent)
    sub = {k: (v[[row]] if isinstance(v, torch.Tensor) and v.dim() > 0 and v.shape[0] == cfg_w.B
               else v) for k, v in w.items()}
    want = O.window_forward(sub["logits"], sub["y"], sub["gate_pre"], sub["reset"], sub["h0"],
                            sub["q0"], sub["age0"], sub["pos0"], w["cost"], k=cfg_w.K)
    for name in ("cells", "units"):
        assert torch.equal(got[name][[row]].cpu().long(), want[name]), name
    assert torch.equal(got["theta"][[row]].cpu(), want["theta"])
    for name in ("q_pre", "q_post", "h_old", "h_sel", "h_max"):
        _close(got[name][[row]], want[name], tol, name)
    _close(got["h"][[row]], want["h"], tol, "h_T")
    assert torch.equal(got["age"][[row]].cpu(), want["age"])
    # the backward: linear in its cotangents on every row, and the row against the oracle
    g1 = _backward(w, got, D, C, cfg_w.N)
    g2 = _backward(w, got, D, C, cfg_w.N, scale=2.0)
    for a, b_ in zip(g1[:4], g2[:4]):
        assert torch.equal(2 * a, b_)
    csub = {k: (v[[row]] if v is not None else None) for k, v in cot.items()}
    wb = O.window_backward(sub["y"], sub["gate_pre"], want["h_old"], want["cells"], want["valid"],
                           sub["reset"], cfg_w.N, csub["d_q_pre"], csub["d_q_post"],
                           csub["d_h_sel"], csub["d_h_T"], csub["d_q_T"])
    for name, g_, w_ in zip(("dy", "dgate", "d_h0"), g1[:3], wb[:3]):
        _close(g_[[row]], w_, tol, name)
    _close(g1[3][[row]], _d_q0_exact(sub["reset"], csub["d_q_pre"], csub["d_q_post"],
                                     csub["d_q_T"], cfg_w.N), tol, "d_q0")
    assert math.isfinite(float(got["h_max"].max()))


def test_bf16_config_full_size(dev):
    """Config 3 at its full size: B64 T512 N1024 d64 K16, bf16 storage."""
    from hsn_amd.workload import CONFIGS

    _check_config(dev, CONFIGS["bf16"], seed=31, row=5, every=64, tol=BF16_TOL)


def test_skewed_config_full_size(dev):
    """Config 5 at its full size: B256 T1024 N4096 d64 K32, bf16 storage, Zipf-biased logits
    (65,536 router wavefronts over 2.1 GB of logits); the properties on every row, one row
    against the oracle."""
    from hsn_amd.workload import CONFIGS

    _check_config(dev, CONFIGS["skewed"], seed=51, row=3, every=128, tol=BF16_TOL)


def test_tiny_config_exactly(dev):
    """Config 1 as the benchmark contract states it: B2 T8 N16 d16 K2, fp32, zero start state,
    one reset at row 1, position 4; forward and backward with the carried state against the
    oracle's whole window."""
    from hsn_amd.workload import CONFIGS, make_cotangents, make_window

    cfg_w = CONFIGS["tiny"]
    w = make_window(cfg_w, 1)
    assert not bool(w["h0"].any()) and w["reset"].nonzero().tolist() == [[1, 4]]
    cot = make_cotangents(cfg_w, 1)
    D, C = _put(w, dev), _put(cot, dev)
    got = _forward(w, D, _route_cfg(k=cfg_w.K))
    want = O.window_forward(w["logits"], w["y"], w["gate_pre"], w["reset"], w["h0"], w["q0"],
                            w["age0"], w["pos0"], w["cost"], k=cfg_w.K)
    for name in ("cells", "units"):
        assert torch.equal(got[name].cpu().long(), want[name]), name
    for name in ("valid", "theta", "age", "pos"):
        assert torch.equal(got[name].cpu(), want[name]), name
    for name in ("q_pre", "q_post", "h_old", "h_sel", "h_max", "h", "q"):
        _close(got[name], want[name], F32_TOL, name)
    gb = _backward(w, got, D, C, cfg_w.N)
    wb = O.window_backward(w["y"], w["gate_pre"], want["h_old"], want["cells"], want["valid"],
                           w["reset"], cfg_w.N, cot["d_q_pre"], cot["d_q_post"], cot["d_h_sel"],
                           cot["d_h_T"], cot["d_q_T"])
    for name, g_, w_ in zip(("dy", "dgate", "d_h0"), gb[:3], wb[:3]):
        _close(g_, w_, F32_TOL, name)
    _close(gb[3], _d_q0_exact(w["reset"], cot["d_q_pre"], cot["d_q_post"], cot["d_q_T"],
                              cfg_w.N), F32_TOL, "d_q0")
    # row 1 restarts at position 4: its state before that position is zero
    assert bool((got["q_pre"][1, 4] == 0).all())


def test_tbptt_config_rows_match_oracle(dev):
    """Config 4 (B128 T128 N512 d128 K8, fp32): one window, the properties on every row and one
    row against the oracle's window, forward and backward."""
    from hsn_amd.workload import CONFIGS

    _check_config(dev, CONFIGS["tbptt"], seed=43, row=17, every=16, tol=F32_TOL)


def _cat(a, b, key):
    return torch.cat([a[key], b[key]], dim=1)


def test_tbptt_two_windows_equal_one(dev):
    """Config 4 (B128 T128 N512 d128 K8, fp32): window 1 started from window 0's end state
    (h, q, ages, positions) gives the outputs of one 256-position window over both; the backward
    run window by window, window 1's d_h0, d_q0 fed to window 0 as its end cotangent, gives the
    long window's gradients."""
    from hsn_amd.workload import CONFIGS, make_cotangents, make_window

    cfg_w = CONFIGS["tbptt"]
    cfg = _route_cfg(k=cfg_w.K)
    w0, w1 = make_window(cfg_w, 41, window=0), make_window(cfg_w, 41, window=1)
    c0, c1 = make_cotangents(cfg_w, 41), make_cotangents(cfg_w, 42)
    D0, D1 = _put(w0, dev), _put(w1, dev)
    g0 = _forward(w0, D0, cfg)
    D1 = dict(D1, h0=g0["h"], q0=g0["q"], age0=g0["age"], pos0=g0["pos"])
    g1 = _forward(w1, D1, cfg)
    wl = {k: _cat(w0, w1, k) for k in ("logits", "y", "gate_pre", "reset")}
    wl.update(h0=w0["h0"], q0=w0["q0"], age0=w0["age0"], pos0=w0["pos0"], cost=w0["cost"])
    DL = _put(wl, dev)
    gl = _forward(wl, DL, cfg)
    T = cfg_w.T
    for name in ("cells", "valid", "theta"):
        assert torch.equal(gl[name][:, :T].cpu(), g0[name].cpu()), name
        assert torch.equal(gl[name][:, T:].cpu(), g1[name].cpu()), name
    for name in ("q_pre", "q_post", "h_old", "h_sel", "h_max"):
        _close(gl[name][:, :T], g0[name], F32_TOL, name)
        _close(gl[name][:, T:], g1[name], F32_TOL, name)
    _close(gl["h"], g1["h"], F32_TOL, "h_T")
    _close(gl["q"], g1["q"], F32_TOL, "q_T")
    assert torch.equal(gl["age"].cpu(), g1["age"].cpu())
    assert torch.equal(gl["pos"].cpu(), g1["pos"].cpu())

    C0, C1 = _put(c0, dev), _put(c1, dev)
    b1 = _backward(w1, g1, D1, C1, cfg_w.N)
    b0 = _backward(w0, g0, D0, C0, cfg_w.N, d_h_T=b1[2], d_q_T=b1[3])
    CL = {k: (torch.cat([C0[k], C1[k]], dim=1) if k in ("d_q_pre", "d_q_post", "d_h_sel")
              else C1[k]) for k in C0}
    bl = _backward(wl, gl, DL, CL, cfg_w.N)
    for name, i in (("dy", 0), ("dgate", 1)):
        _close(bl[i][:, :T], b0[i], F32_TOL, name + " window 0")
        _close(bl[i][:, T:], b1[i], F32_TOL, name + " window 1")
    _close(bl[2], b0[2], F32_TOL, "d_h0")
    _close(bl[3], b0[3], F32_TOL, "d_q0")

    # one row of the segment against the oracle's long window, forward and backward
    r = 9
    row = lambda t: t[[r]]  # noqa: E731
    want = O.window_forward(row(wl["logits"]), row(wl["y"]), row(wl["gate_pre"]),
                            row(wl["reset"]), row(wl["h0"]), row(wl["q0"]), row(wl["age0"]),
                            row(wl["pos0"]), wl["cost"], k=cfg_w.K)
    for name in ("cells", "theta"):
        assert torch.equal(torch.cat([g0[name][[r]], g1[name][[r]]], 1).cpu().to(want[name].dtype),
                           want[name]), name
    for name in ("q_pre", "q_post", "h_old", "h_sel", "h_max"):
        _close(torch.cat([g0[name][[r]], g1[name][[r]]], 1), want[name], F32_TOL, name + " row")
    _close(g1["h"][[r]], want["h"], F32_TOL, "h_T row")
    CLc = {k: (None if v is None else row(v.cpu())) for k, v in CL.items()}
    wb = O.window_backward(row(wl["y"]), row(wl["gate_pre"]), want["h_old"], want["cells"],
                           want["valid"], row(wl["reset"]), cfg_w.N, CLc["d_q_pre"],
                           CLc["d_q_post"], CLc["d_h_sel"], CLc["d_h_T"], CLc["d_q_T"])
    _close(torch.cat([b0[0][[r]], b1[0][[r]]], 1), wb[0], F32_TOL, "dy row")
    _close(torch.cat([b0[1][[r]], b1[1][[r]]], 1), wb[1], F32_TOL, "dgate row")
    _close(b0[2][[r]], wb[2], F32_TOL, "d_h0 row")


def test_tbptt_sixteen_window_segment(dev):
    """Config 4's whole segment: 16 windows with the state carried forward and the gradient
    carried back (segment mode). The end state keeps q = mean(h); the segment's gradients are
    finite and linear in the cotangents (all scaled by 2: every window's d_h0 exactly doubles)."""
    from hsn_amd.workload import CONFIGS, make_cotangents, make_window

    cfg_w = CONFIGS["tbptt"]
    cfg = _route_cfg(k=cfg_w.K)
    state = None
    fwd = []
    for k in range(cfg_w.windows):
        D = _put(make_window(cfg_w, 61, window=k), dev)
        if state is not None:
            D.update(h0=state["h"], q0=state["q"], age0=state["age"], pos0=state["pos"])
        got = _forward(None, D, cfg)
        fwd.append((D, got))
        state = got
    _close(state["q"], state["h"].mean(dim=1), 1e-5, "q_T vs mean h_T")
    assert int(state["pos"].max()) <= cfg_w.T * cfg_w.windows

    def segment(scale):
        d_h, d_q = None, None
        out = []
        for k in reversed(range(cfg_w.windows)):
            D, got = fwd[k]
            C = _put(make_cotangents(cfg_w, 70 + k), dev)
            g = _backward(None, got, D, C, cfg_w.N, scale=scale,
                          d_h_T=None if d_h is None else d_h / scale,
                          d_q_T=None if d_q is None else d_q / scale)
            d_h, d_q = g[2], g[3]
            out.append((g[2], g[3]))
        return out

    s1, s2 = segment(1.0), segment(2.0)
    for (h1, q1), (h2, q2) in zip(s1, s2):
        assert bool(torch.isfinite(h1).all()) and bool(torch.isfinite(q1).all())
        assert torch.equal(2 * h1, h2) and torch.equal(2 * q1, q2)
