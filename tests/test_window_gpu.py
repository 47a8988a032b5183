"""The HIP window path (route, forward sweep, backward recurrence with the carried state) against
the CPU oracle on the same seeded inputs. GPU only.

Bars: decisions (cells, units, valid, refreshed, ages, positions) bit-exact; theta bit-exact;
fp32 outputs and gradients within 1e-5 (|got - want| <= 1e-5 * max(|want|, 1)); bf16 storage
within 2e-2 of the oracle run on the same bf16 inputs.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import hsn_oracle as O

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
BF16_TOL = 2e-2


@pytest.fixture(scope="module")
def dev(cuda_device):
    from hsn_amd import window

    assert window.available(), "the HIP library must be built for the GPU tests"
    return cuda_device


@pytest.fixture(params=["evmap", "slice", "chain"])
def path(request, dev):
    """Each forward / backward test runs on every sweep design (the library's path setting)."""
    from hsn_amd import _lib

    _lib.set_path(request.param)
    yield request.param
    _lib.set_path("auto")


def _skip_unless_taken(path, c):
    """Skip where the forced sweep design does not take the case's shape (the event maps: fp32
    rows, d a multiple of 8, T <= 256 and K <= 8)."""
    from hsn_amd import _lib

    code = _lib.DTYPE_BF16 if c.get("io") == "bf16" else _lib.DTYPE_F32
    for op in (_lib.OP_FORWARD, _lib.OP_BACKWARD):
        try:
            _lib.path_for(op, c["B"], c["T"], c["N"], c["d"], c["K"], code)
        except RuntimeError as why:
            pytest.skip(f"the {path} path does not take this shape: {why}")


def _close(got, want, tol, what=""):
    got = got.detach().float().cpu()
    want = want.detach().float().cpu()
    assert got.shape == want.shape, (what, got.shape, want.shape)
    both_nan = torch.isnan(got) & torch.isnan(want)
    err = (got - want).abs().masked_fill(both_nan, 0)
    bound = tol * want.abs().clamp(min=1.0)
    bad = ~((err <= bound) | both_nan)  # (a NaN in want makes its bound NaN)
    if bool(bad.any()):
        i = int(bad.flatten().nonzero()[0])
        raise AssertionError(f"{what}: {int(bad.sum())} elements out of tolerance {tol}; first at "
                             f"{i}: got {got.flatten()[i].item()} want {want.flatten()[i].item()} "
                             f"(max err {float(err.max()):.3g})")


def _d_q0_exact(reset, d_q_pre, d_q_post, d_q_T, n_cells):
    """The summary cotangent after position 0 (``d_q0``) from the oracle's recurrence in float64.

    ``R`` is a running sum of the window's ``2T`` summary cotangents. Summed in fp32 in the
    reference's sequential order it carries about sqrt(2T)/2 ulps of its largest partial (2e-5
    at the ref shape, above the 1e-5 bar), and the HIP sweep sums it chunk by chunk in fp64, so
    ``d_q0`` is checked against the exact sum. ``R`` reads no other input."""
    B, T, d = (d_q_post if d_q_post is not None else d_q_pre).shape
    z = torch.zeros(B, T, 1, d, dtype=torch.float64)
    cells = torch.zeros(B, T, 1, dtype=torch.int64)
    valid = torch.zeros(B, T, 1, dtype=torch.bool)
    f = lambda t: None if t is None else t.detach().cpu().double()  # noqa: E731
    return O.recurrence_backward(z, z, z, cells, valid, reset.cpu(), n_cells, f(d_q_pre),
                                 f(d_q_post), None, None, f(d_q_T), carried=True)[3]


def _route_cfg(**kw):
    from hsn_amd.window import RouteConfig

    return RouteConfig(**kw)


def _oracle_route_kwargs(cfg):
    return dict(k=cfg.k, age_max=cfg.age_max, probes=cfg.probes, lambda_cost=cfg.lambda_cost,
                cell_overhead=cfg.cell_overhead, shared_cost=cfg.shared_cost, limit=cfg.limit,
                reserved=cfg.reserved, reserved_units=cfg.reserved_units)


# --------------------------------------------------------------------------------------------
# routing: bit-exact against the oracle's Router.select restatement
# --------------------------------------------------------------------------------------------

ROUTE_CASES = [
    # B, T, N, M, K, settings, logit dtype, special values
    (3, 5, 9, 1, 4, dict(), torch.float32, "ties"),
    (2, 4, 16, 3, 5, dict(lambda_cost=0.05, limit=0.1), torch.float32, "ties"),
    (2, 3, 70, 2, 7, dict(cell_overhead=0.0625, shared_cost=0.125, limit=0.5), torch.float32, "nan"),
    (4, 6, 256, 1, 8, dict(), torch.float32, "plain"),
    (2, 5, 300, 4, 12, dict(reserved=3, reserved_units=True), torch.float32, "ties"),
    (2, 4, 1024, 1, 16, dict(), torch.bfloat16, "plain"),
    (1, 3, 4096, 1, 32, dict(), torch.bfloat16, "zipf"),
    (2, 3, 33, 2, 33, dict(limit=0.75), torch.float32, "zeros"),
    (2, 2, 64, 1, 64, dict(), torch.float32, "plain"),
    # one unit: N % 4 != 0 at four cells a lane (scalar loads) with a cost term (the product and
    # the difference rounded apart); bf16 runs of two and four cells a lane (vector loads)
    (2, 4, 130, 1, 8, dict(lambda_cost=0.05), torch.float32, "ties"),
    (2, 4, 100, 1, 6, dict(reserved=2), torch.bfloat16, "nan"),
    (2, 3, 200, 1, 8, dict(), torch.bfloat16, "plain"),
    # one unit, two positions a wavefront of 32 lanes (N <= 256, K < 32): every score +-0 (more
    # candidates than the group's lanes: the one-position fallback), the uniform rows (N = 256)
    # with ties and with a cost term, an odd number of positions (a wavefront's second group
    # past the window), reserved cells with NaN / inf, 31 slots
    (2, 3, 200, 1, 8, dict(), torch.float32, "zeros"),
    (3, 3, 256, 1, 8, dict(), torch.float32, "ties"),
    (1, 5, 256, 1, 8, dict(lambda_cost=0.05, limit=0.02), torch.float32, "plain"),
    (2, 4, 48, 1, 5, dict(reserved=2), torch.float32, "nan"),
    (2, 3, 256, 1, 31, dict(), torch.bfloat16, "ties"),
    # one unit, sixteen or more cells a lane (keys recomputed from the logits in each pass): a row
    # not a multiple of the lane block (scalar loads) with half-integer ties; reserved cells with
    # a cost term and NaN / inf; every logit +-0 (more than 64 candidates: the argmax rounds);
    # fp32 at 4096 cells and 64 slots
    (2, 3, 600, 1, 12, dict(), torch.float32, "ties"),
    (2, 3, 1000, 1, 16, dict(reserved=3, lambda_cost=0.05), torch.bfloat16, "nan"),
    (2, 2, 512, 1, 20, dict(limit=0.7), torch.float32, "zeros"),
    (1, 2, 4096, 1, 64, dict(), torch.float32, "ties"),
    # one unit, more than 1024 cells (a workgroup per position): a partial last block with
    # reserved cells, a cost term and NaN / inf; every logit +-0 across the four wavefronts
    (2, 3, 2000, 1, 24, dict(reserved=4, lambda_cost=0.05), torch.bfloat16, "nan"),
    (1, 2, 3000, 1, 16, dict(limit=0.6), torch.float32, "zeros"),
]


def _logits(B, T, N, M, kind, g):
    x = torch.randn(B, T, N, M, generator=g)
    if kind == "ties":
        x = (x * 2).round() / 2
    elif kind == "nan":
        x[0, 1, 3, 0] = float("nan")
        x[1, 2, 5, :] = float("nan")
        x[0, 0, 7, 0] = float("inf")
        x[1, 0, 2, 0] = float("-inf")
    elif kind == "zipf":
        rank = torch.randperm(N, generator=g).float()
        x = x - 1.1 * torch.log1p(rank)[None, None, :, None]
    elif kind == "zeros":
        x = torch.zeros_like(x)
        x[..., 0, :] = -0.0
    return x


@pytest.mark.parametrize("case", range(len(ROUTE_CASES)))
def test_route_matches_oracle_bit_exact(dev, case):
    from hsn_amd import window

    B, T, N, M, K, kw, dtype, kind = ROUTE_CASES[case]
    g = torch.Generator().manual_seed(1000 + case)
    logits = _logits(B, T, N, M, kind, g).to(dtype)
    cost = torch.full((M,), 1.0 / 64) if M == 1 else torch.tensor([0.125, 0.0625, 0.25, 0.03125][:M])
    cfg = _route_cfg(k=K, **kw)
    got = window.route(logits.to(dev), cost.to(dev), cfg)
    for t in range(T):
        want = O.router_select(logits[:, t], None, cost, **_oracle_route_kwargs(cfg))
        for name, gv, wv in zip(("cells", "units", "valid", "theta", "refreshed"), got, want):
            gv = gv[:, t].cpu()
            if name in ("cells", "units"):
                assert torch.equal(gv.long(), wv), (name, t, gv, wv)
            elif name == "theta":
                assert torch.equal(gv.view(torch.int32), wv.view(torch.int32)) or (
                    bool(torch.isnan(gv).eq(torch.isnan(wv)).all()) and
                    bool((gv[~torch.isnan(gv)] == wv[~torch.isnan(wv)]).all())), (t, gv, wv)
            else:
                assert torch.equal(gv, wv), (name, t, gv, wv)


@pytest.mark.parametrize("seed", range(4))
def test_route_with_probes_walks_ages_like_the_oracle(dev, seed):
    """Refresh probes: the decisions depend on the ages, which evolve with the decisions and the
    resets; the window form walks each row in order exactly like the oracle's forward loop."""
    from hsn_amd import window
    from hsn_amd.workload import CONFIGS, make_window

    cfg_w = CONFIGS["tiny"].scaled(B=3, T=24, N=20, d=4, K=5, M=2, h0_sigma=0.3, reset_p=0.1)
    w = make_window(cfg_w, 50 + seed)
    w["logits"] = (w["logits"] * 2).round() / 2
    w["age0"] = torch.randint(0, 4, (cfg_w.B, cfg_w.N), generator=torch.Generator().manual_seed(seed))
    cost = torch.tensor([0.0625, 0.125])
    cfg = _route_cfg(k=5, age_max=2, probes=True, limit=[10.0, 0.5, 0.3, 0.45][seed],
                     reserved=1 if seed == 3 else 0)
    want = O.window_forward(w["logits"], w["y"], w["gate_pre"], w["reset"], w["h0"], w["q0"],
                            w["age0"], w["pos0"], cost, **_oracle_route_kwargs(cfg))
    cells, units, valid, theta, refreshed = window.route(
        w["logits"].to(dev), cost.to(dev), cfg, reset=w["reset"].to(dev), age0=w["age0"].to(dev))
    assert torch.equal(cells.cpu().long(), want["cells"])
    assert torch.equal(units.cpu().long(), want["units"])
    assert torch.equal(valid.cpu(), want["valid"])
    assert torch.equal(refreshed.cpu(), want["refreshed"])
    assert torch.equal(theta.cpu(), want["theta"])
    assert bool(refreshed.any()) or seed == 2  # the case exercises the probes


# --------------------------------------------------------------------------------------------
# forward sweep and backward recurrence against the oracle
# --------------------------------------------------------------------------------------------

WINDOW_CASES = [
    # B, T, N, d, K, M, io, rms, route settings
    dict(B=2, T=8, N=16, d=16, K=2, io="f32"),  # the tiny config's shape
    dict(B=3, T=21, N=13, d=5, K=3, io="f32", limit=0.2),  # odd d, padded slots
    dict(B=4, T=40, N=64, d=16, K=4, io="f32", rms=True),
    dict(B=2, T=33, N=37, d=12, K=9, io="f32", M=2, limit=0.6, reserved=2),
    dict(B=8, T=24, N=256, d=64, K=8, io="f32"),
    dict(B=2, T=20, N=40, d=8, K=20, io="f32"),  # two slots per lane
    dict(B=2, T=17, N=48, d=32, K=32, io="f32", rms=True),  # many slots per lane
    dict(B=4, T=32, N=128, d=64, K=16, io="bf16"),
    dict(B=2, T=16, N=64, d=16, K=8, io="bf16", rms=True, limit=0.1),
    dict(B=8, T=300, N=64, d=64, K=8, io="f32"),  # chunks longer than a register sub-block
    dict(B=256, T=70, N=32, d=64, K=8, io="f32"),  # one chunk per row, several sub-blocks
    dict(B=3, T=5, N=16, d=4, K=4, io="f32"),  # fewer positions than chunks per row
    dict(B=3, T=7, N=20, d=7, K=3, io="bf16", rms=True),  # odd d and odd B*T*K: RMS workspace
    dict(B=2, T=200, N=8, d=100, K=4, io="f32"),  # long chains: several event windows per cell
    # hot cells (Zipf bias) whose events overflow a chain group's staged list; padded slots
    dict(B=2, T=256, N=512, d=16, K=16, io="bf16", bias="zipf", limit=0.02),
]


def _window_case(c, seed):
    from hsn_amd.workload import CONFIGS, make_window, make_cotangents

    M = c.get("M", 1)
    cfg_w = CONFIGS["tiny"].scaled(B=c["B"], T=c["T"], N=c["N"], d=c["d"], K=c["K"], M=M,
                                   h0_sigma=0.3, reset_p=0.08, reset_at=((0, 3),),
                                   io=c["io"], logit_bias=c.get("bias", "none"))
    w = make_window(cfg_w, seed)
    cot = make_cotangents(cfg_w, seed, carried=True)
    cost = torch.full((M,), 1.0 / (c["N"] * M)) if M == 1 else torch.tensor([0.03125, 0.0625])
    cfg = _route_cfg(k=c["K"], limit=c.get("limit", 1.0 + 1e-5), reserved=c.get("reserved", 0))
    cand_w = (torch.rand(c["d"], generator=torch.Generator().manual_seed(seed)) + 0.5) if c.get("rms") else None
    return cfg_w, w, cot, cost, cfg, cand_w


def _valid_mask(t, valid):
    return torch.where(valid[..., None], t, torch.zeros((), dtype=t.dtype))


@pytest.mark.parametrize("case", range(len(WINDOW_CASES)))
def test_window_forward_and_backward_match_oracle(dev, path, case):
    from hsn_amd import window

    c = WINDOW_CASES[case]
    _skip_unless_taken(path, c)
    cfg_w, w, cot, cost, cfg, cand_w = _window_case(c, 300 + case)
    rms = bool(c.get("rms"))
    tol = BF16_TOL if c["io"] == "bf16" else F32_TOL
    want = O.window_forward(w["logits"], w["y"], w["gate_pre"], w["reset"], w["h0"], w["q0"],
                            w["age0"], w["pos0"], cost, cand_norm=rms, cand_w=cand_w,
                            **_oracle_route_kwargs(cfg))
    D = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in w.items()}
    got = window.window_forward(D["logits"], D["y"], D["gate_pre"], D["reset"], D["h0"], D["q0"],
                                D["age0"], D["pos0"], cost.to(dev), cfg, cand_norm=rms,
                                cand_w=None if cand_w is None else cand_w.to(dev))
    for name in ("cells", "units"):
        assert torch.equal(got[name].cpu().long(), want[name]), name
    for name in ("valid", "refreshed", "age", "pos"):
        assert torch.equal(got[name].cpu(), want[name]), name
    assert torch.equal(got["theta"].cpu(), want["theta"])
    for name in ("q_pre", "q_post", "h_old", "h_max"):
        _close(got[name], want[name], tol, name)
    _close(_valid_mask(got["h_sel"].cpu(), want["valid"]), _valid_mask(want["h_sel"], want["valid"]),
           tol, "h_sel")
    _close(got["h"], want["h"], tol, "h_T")
    _close(got["q"], want["q"], tol, "q_T")

    # backward from the same tape (the oracle's h_old), cotangents masked by valid for h_sel; the
    # oracle in float64 for fp32 rows (its inputs are the fp32 values the GPU reads)
    d_h_sel = _valid_mask(cot["d_h_sel"], want["valid"])
    up = (lambda t: None if t is None else t.double()) if c["io"] == "f32" else (lambda t: t)  # noqa: E731
    wb = O.window_backward(up(w["y"]), up(w["gate_pre"]), up(want["h_old"]), want["cells"],
                           want["valid"], w["reset"], cfg_w.N, up(cot["d_q_pre"]),
                           up(cot["d_q_post"]), up(d_h_sel), up(cot["d_h_T"]), up(cot["d_q_T"]),
                           cand_norm=rms, cand_w=up(cand_w))
    gb = window.backward(D["y"], D["gate_pre"], want["h_old"].to(dev), got["slots"],
                         D["reset"], cfg_w.N, cot["d_q_pre"].to(dev),
                         cot["d_q_post"].to(dev), d_h_sel.to(dev), cot["d_h_T"].to(dev),
                         cot["d_q_T"].to(dev), cand_norm=rms,
                         cand_w=None if cand_w is None else cand_w.to(dev))
    for name, g_, w_ in zip(("dy", "dgate", "d_h0"), gb[:3], wb[:3]):
        _close(g_, w_, tol, name)
    _close(gb[3], _d_q0_exact(w["reset"], cot["d_q_pre"], cot["d_q_post"], cot["d_q_T"], cfg_w.N),
           tol, "d_q0")
    if rms:  # a sum over every slot of the window: fp32 against float64 at the same bar
        _close(gb[4], wb[4], tol if c["io"] == "f32" else tol * 10, "d_cand_w")
    zero_pad = ~want["valid"]
    assert bool((gb[0].cpu()[zero_pad] == 0).all()) and bool((gb[1].cpu()[zero_pad] == 0).all())


@pytest.mark.parametrize("N,d", [(256, 64), (300, 16), (16, 8)])
def test_forward_h_max_propagates_a_nan_in_an_unwritten_cell(dev, path, N, d):
    """A NaN in a start-state cell no slot writes makes the row maximum NaN until a reset clears
    the row (the reference's test_p2_10_window.py:540-560), on both of the forward's maxima
    paths: per-cell maxima in LDS (N <= 256) and the tracked maximum with rescans (N > 256)."""
    from conftest import nan_state_window
    from hsn_amd import window

    cfg, w, quiet = nan_state_window(N=N, d=d, K=4, T=12)
    want = O.window_forward(w["logits"], w["y"], w["gate_pre"], w["reset"], w["h0"], w["q0"],
                            w["age0"], w["pos0"], w["cost"], k=cfg.K)
    D = {k: v.to(dev) for k, v in w.items()}
    got = window.window_forward(D["logits"], D["y"], D["gate_pre"], D["reset"], D["h0"], D["q0"],
                                D["age0"], D["pos0"], D["cost"], _route_cfg(k=cfg.K))
    assert torch.equal(got["cells"].cpu().long(), want["cells"])
    hm = got["h_max"].cpu()
    assert torch.equal(torch.isnan(hm), torch.isnan(want["h_max"]))
    assert bool(torch.isnan(hm[0]).all()) and bool(torch.isnan(hm[1, :3]).all())
    _close(hm[1, 3:], want["h_max"][1, 3:], F32_TOL, "h_max after the reset")
    for name in ("q_pre", "q_post", "h_old"):
        _close(got[name], want[name], F32_TOL, name)
    assert torch.equal(torch.isnan(got["h"].cpu()), torch.isnan(want["h"]))


def test_forward_zeroes_a_row_maximum_buffer_it_is_given(dev, path):
    """``forward(h_max=buf)`` max-reduces into ``buf``: it zeroes it first, so a buffer holding
    garbage (here larger than every maximum) gives the same maxima as the routed window."""
    from hsn_amd import window

    c = WINDOW_CASES[4]
    cfg_w, w, cot, cost, cfg, _ = _window_case(c, 404)
    D = {k: v.to(dev) for k, v in w.items()}
    ref = window.window_forward(D["logits"], D["y"], D["gate_pre"], D["reset"], D["h0"], D["q0"],
                                D["age0"], D["pos0"], cost.to(dev), cfg)
    buf = torch.full((c["B"], c["T"]), 1e30, device=dev)
    out = window.forward(D["y"], D["gate_pre"], D["reset"], ref["slots"], D["h0"], D["q0"],
                         D["age0"], D["pos0"], c["N"], h_max=buf)
    assert torch.equal(out["h_max"], ref["h_max"]) and out["h_max"] is buf


def test_backward_without_optional_cotangents(dev, path):
    from hsn_amd import window

    c = dict(B=2, T=12, N=24, d=8, K=4, io="f32", limit=0.2)
    cfg_w, w, cot, cost, cfg, _ = _window_case(c, 77)
    fw = O.window_forward(w["logits"], w["y"], w["gate_pre"], w["reset"], w["h0"], w["q0"],
                          w["age0"], w["pos0"], cost, **_oracle_route_kwargs(cfg))
    args_cpu = (w["y"], w["gate_pre"], fw["h_old"], fw["cells"], fw["valid"], w["reset"], cfg_w.N)
    for present in [(True, False, False), (False, True, False), (False, False, True)]:
        pre, post, sel = (cot[k] if p else None for k, p in zip(("d_q_pre", "d_q_post", "d_h_sel"), present))
        sel = None if sel is None else _valid_mask(sel, fw["valid"])
        wb = O.window_backward(*args_cpu, pre, post, sel)
        gb = window.window_backward(w["y"].to(dev), w["gate_pre"].to(dev), fw["h_old"].to(dev),
                             fw["cells"].int().to(dev), fw["valid"].to(dev), w["reset"].to(dev),
                             cfg_w.N, None if pre is None else pre.to(dev),
                             None if post is None else post.to(dev),
                             None if sel is None else sel.to(dev))
        for name, g_, w_ in zip(("dy", "dgate", "d_h0"), gb[:3], wb[:3]):
            _close(g_, w_, F32_TOL, f"{name} {present}")
        if pre is not None or post is not None:
            _close(gb[3], _d_q0_exact(w["reset"], pre, post, None, cfg_w.N), F32_TOL,
                   f"d_q0 {present}")
        else:
            assert bool((gb[3] == 0).all())


def test_backward_propagates_a_nan_gate(dev, path):
    """A NaN gate input on a selected slot: the backward's NaNs fall where the oracle's do (that
    slot's column, the cell's earlier positions through its cotangent, its later ones through
    h_old) and the rest stays within tolerance; padded slots still write exact zeros."""
    from hsn_amd import window

    c = dict(B=2, T=40, N=24, d=16, K=4, io="f32", limit=0.15)
    _skip_unless_taken(path, c)
    cfg_w, w, cot, cost, cfg, _ = _window_case(c, 91)
    plain = O.window_forward(w["logits"], w["y"], w["gate_pre"], w["reset"], w["h0"], w["q0"],
                             w["age0"], w["pos0"], cost, **_oracle_route_kwargs(cfg))
    t, k = 21, 1
    assert bool(plain["valid"][0, t, k]) and bool((~plain["valid"]).any())
    w["gate_pre"][0, t, k, 3] = float("nan")
    fw = O.window_forward(w["logits"], w["y"], w["gate_pre"], w["reset"], w["h0"], w["q0"],
                          w["age0"], w["pos0"], cost, **_oracle_route_kwargs(cfg))
    sel = _valid_mask(cot["d_h_sel"], fw["valid"])
    wb = O.window_backward(w["y"], w["gate_pre"], fw["h_old"], fw["cells"], fw["valid"],
                           w["reset"], cfg_w.N, cot["d_q_pre"], cot["d_q_post"], sel,
                           cot["d_h_T"], cot["d_q_T"])
    gb = window.window_backward(w["y"].to(dev), w["gate_pre"].to(dev), fw["h_old"].to(dev),
                                fw["cells"].int().to(dev), fw["valid"].to(dev),
                                w["reset"].to(dev), cfg_w.N, cot["d_q_pre"].to(dev),
                                cot["d_q_post"].to(dev), sel.to(dev), cot["d_h_T"].to(dev),
                                cot["d_q_T"].to(dev))
    assert bool(torch.isnan(wb[0][0, t, k, 3])) and bool(torch.isnan(wb[1][0, t, k, 3]))
    for name, g_, w_ in zip(("dy", "dgate", "d_h0"), gb[:3], wb[:3]):
        assert torch.equal(torch.isnan(g_.cpu()), torch.isnan(w_)), name
        _close(g_, w_, F32_TOL, name)
    pad = ~fw["valid"]
    assert bool((gb[0].cpu()[pad] == 0).all()) and bool((gb[1].cpu()[pad] == 0).all())


def test_bf16_storage_rounds_like_torch(dev, path):
    """The bf16 narrowing of the kernels (gfx950's v_cvt_pk_bf16_f32) against torch's
    round-to-nearest-even cast, bit for bit: every cell is written at position 0 (K = N), so
    h_old[:, 0] is the cast of h0's rows, here ties to even in both directions, denormals, the
    largest finite value (rounds to inf), infinities and signed zeros; a NaN stays a NaN."""
    from hsn_amd import window

    B, T, N, d, K = 2, 2, 16, 64, 16
    _skip_unless_taken(path, dict(B=B, T=T, N=N, d=d, K=K, io="bf16"))
    g = torch.Generator().manual_seed(8)
    one = 1.0
    special = torch.tensor([one + 2.0 ** -8, one + 3 * 2.0 ** -8, -(one + 2.0 ** -8),
                            -(one + 3 * 2.0 ** -8), 1e-40, -1e-40, 2.0 ** -133, 3.4028234663852886e38,
                            -3.4028234663852886e38, float("inf"), float("-inf"), 0.0, -0.0,
                            float("nan"), one + 2.0 ** -9, 0.1], dtype=torch.float32)
    h0 = torch.randn(B, N, d, generator=g)
    h0[:, :, :16] = special  # every cell's first 16 columns
    h0[1, :, 16:32] = torch.randn(N, 16, generator=g) * 1e-39  # denormals of every kind
    y = torch.randn(B, T, K, d, generator=g).to(torch.bfloat16)
    gate = torch.randn(B, T, K, d, generator=g).to(torch.bfloat16)
    cells = torch.arange(N).expand(B, T, N).contiguous()
    slots = window.pack_slots(cells, torch.ones(B, T, K, dtype=torch.bool)).to(dev)
    reset = torch.zeros(B, T, dtype=torch.bool, device=dev)
    out = window.forward(y.to(dev), gate.to(dev), reset, slots, h0.to(dev),
                         torch.zeros(B, d, device=dev), torch.zeros(B, N, dtype=torch.int64, device=dev),
                         torch.zeros(B, dtype=torch.int64, device=dev), N)
    got = out["h_old"][:, 0].cpu()
    want = h0.to(torch.bfloat16)
    nan = torch.isnan(want)
    assert torch.equal(torch.isnan(got), nan)
    assert torch.equal(got.view(torch.int16)[~nan], want.view(torch.int16)[~nan])


@pytest.mark.parametrize("io", ["f32", "bf16"])
def test_chain_takes_more_slots_than_a_wavefront(dev, io):
    """K = 80 slots per position, more than a wavefront's lanes: the slices (a slot per lane)
    and the router decline it, the cell chains take up to 255. The oracle's decisions, packed,
    through the forward and the backward against the oracle; a budget of 0.3 leaves 20 padded
    slots per position."""
    from hsn_amd import _lib, window

    c = dict(B=2, T=12, N=200, d=32, K=80, io=io, limit=0.3)
    cfg_w, w, cot, cost, cfg, _ = _window_case(c, 91)
    B, T, N, d, K = c["B"], c["T"], c["N"], c["d"], c["K"]
    code = _lib.DTYPE_F32 if io == "f32" else _lib.DTYPE_BF16
    assert _lib.path_for(_lib.OP_FORWARD, B, T, N, d, K, code) == "chain"
    assert _lib.path_for(_lib.OP_BACKWARD, B, T, N, d, K, code) == "chain"
    tol = BF16_TOL if io == "bf16" else F32_TOL
    want = O.window_forward(w["logits"], w["y"], w["gate_pre"], w["reset"], w["h0"], w["q0"],
                            w["age0"], w["pos0"], cost, **_oracle_route_kwargs(cfg))
    assert 0 < int((~want["valid"]).sum()) < want["valid"].numel()
    D = {k: v.to(dev) for k, v in w.items()}
    slots = window.pack_slots(want["cells"], want["valid"]).to(dev)
    h_max = torch.empty(B, T, device=dev)
    got = window.forward(D["y"], D["gate_pre"], D["reset"], slots, D["h0"], D["q0"], D["age0"],
                         D["pos0"], N, h_max=h_max)
    for name in ("q_pre", "q_post", "h_old", "h_max"):
        _close(got[name], want[name], tol, name)
    _close(got["h_sel"], want["h_sel"], tol, "h_sel")  # padded slots show cell 0 after the update
    _close(got["h"], want["h"], tol, "h_T")
    _close(got["q"], want["q"], tol, "q_T")
    assert torch.equal(got["age"].cpu(), want["age"]) and torch.equal(got["pos"].cpu(), want["pos"])
    d_h_sel = _valid_mask(cot["d_h_sel"], want["valid"])
    wb = O.window_backward(w["y"], w["gate_pre"], want["h_old"], want["cells"], want["valid"],
                           w["reset"], N, cot["d_q_pre"], cot["d_q_post"], d_h_sel, cot["d_h_T"],
                           cot["d_q_T"])
    gb = window.backward(D["y"], D["gate_pre"], want["h_old"].to(dev), slots, D["reset"], N,
                         cot["d_q_pre"].to(dev), cot["d_q_post"].to(dev), d_h_sel.to(dev),
                         cot["d_h_T"].to(dev), cot["d_q_T"].to(dev))
    for name, g_, w_ in zip(("dy", "dgate", "d_h0"), gb[:3], wb[:3]):
        _close(g_, w_, tol, name)
    _close(gb[3], _d_q0_exact(w["reset"], cot["d_q_pre"], cot["d_q_post"], cot["d_q_T"], N), tol,
           "d_q0")
    zero_pad = ~want["valid"]
    assert bool((gb[0].cpu()[zero_pad] == 0).all()) and bool((gb[1].cpu()[zero_pad] == 0).all())


@pytest.mark.parametrize("shape", [(3, 7, 5, 3, 4), (1, 1, 2, 1, 1), (4, 50, 300, 8, 64),
                                   (2, 16, 32, 4, 37)])
def test_recurrence_backward_matches_oracle(dev, shape):
    """The reference-compatible recurrence (c, b given; int64 cells) with the carried state."""
    from hsn_amd.kernels import window as W

    B, T, N, K, d = shape
    g = torch.Generator().manual_seed(sum(shape))
    cells = torch.stack([torch.stack([torch.randperm(N, generator=g)[:K] for _ in range(T)])
                         for _ in range(B)])
    valid = torch.rand(B, T, K, generator=g) > 0.25
    reset = torch.rand(B, T, generator=g) < 0.05
    c = torch.rand(B, T, K, d, generator=g) * 2 - 1
    b = torch.rand(B, T, K, d, generator=g)
    h_old = torch.rand(B, T, K, d, generator=g) * 2 - 1
    pre, post = torch.randn(B, T, d, generator=g), torch.randn(B, T, d, generator=g)
    sel = torch.randn(B, T, K, d, generator=g)
    dhT, dqT = torch.randn(B, N, d, generator=g), torch.randn(B, d, generator=g)
    cells = torch.where(valid, cells, torch.zeros_like(cells))
    want = O.recurrence_backward(c, b, h_old, cells, valid, reset, N, pre, post, sel, dhT, dqT,
                                 carried=True)
    W.prepare(0)
    put = lambda t: t.to(dev)  # noqa: E731
    got = W.recurrence_backward_carried(put(c), put(b), put(h_old), put(cells), put(valid),
                                        put(reset), N, put(pre), put(post), put(sel), put(dhT),
                                        put(dqT))
    for name, g_, w_ in zip(("dc", "db", "d_h0"), got, want):
        _close(g_, w_, F32_TOL, name)
    _close(got[3], _d_q0_exact(reset, pre, post, dqT, N), F32_TOL, "d_q0")
    dc, db = W.recurrence_backward(put(c), put(b), put(h_old), put(cells), put(valid), put(reset),
                                   N, put(pre), put(post), put(sel))
    want2 = O.recurrence_backward(c, b, h_old, cells, valid, reset, N, pre, post, sel)
    _close(dc, want2[0], F32_TOL, "dc")
    _close(db, want2[1], F32_TOL, "db")


def test_recurrence_keeps_a_padded_nan_out(dev):
    """reference tests/test_p2_10_split_window.py:87-100 on the GPU."""
    from hsn_amd.kernels import window as W

    B, T, N, K, d = 1, 2, 3, 2, 2
    c = torch.full((B, T, K, d), 0.5)
    c[0, 0, 1] = float("nan")
    b = torch.full((B, T, K, d), 0.25)
    cells = torch.tensor([[[1, 0], [2, 0]]])
    valid = torch.tensor([[[True, False], [True, False]]])
    reset = torch.zeros(B, T, dtype=torch.bool)
    ones = torch.ones(B, T, d)
    W.prepare(0)
    dc, db = W.recurrence_backward(c.to(dev), b.to(dev), torch.zeros_like(c).to(dev),
                                   cells.to(dev), valid.to(dev), reset.to(dev), N, None,
                                   ones.to(dev), None)
    assert bool(torch.isfinite(dc).all()) and bool(torch.isfinite(db).all())


def test_dense_recurrence_matches_oracle(dev):
    from hsn_amd.kernels import window as W

    g = torch.Generator().manual_seed(5)
    Bd, T, N, d = 3, 9, 7, 6
    c = torch.rand(Bd, T, N, d, generator=g)
    b = torch.rand(Bd, T, N, d, generator=g)
    h_old = torch.rand(Bd, T, N, d, generator=g)
    reset = torch.zeros(Bd, T, dtype=torch.bool)
    reset[1, 3] = True
    pre, post = torch.randn(Bd, T, d, generator=g), torch.randn(Bd, T, d, generator=g)
    W.prepare(0)
    for p_, q_ in ((pre, post), (None, post), (pre, None)):
        want = O.dense_recurrence_backward(c, b, h_old, reset, N, p_, q_)
        got = W.dense_recurrence_backward(c.to(dev), b.to(dev), h_old.to(dev), reset.to(dev), N,
                                          None if p_ is None else p_.to(dev),
                                          None if q_ is None else q_.to(dev))
        _close(got[0], want[0], F32_TOL, "dc")
        _close(got[1], want[1], F32_TOL, "db")


# --------------------------------------------------------------------------------------------
# the autograd node and the carried-state gradient across windows
# --------------------------------------------------------------------------------------------


def test_window_recurrence_autograd_carries_across_windows(dev):
    """Two windows chained through the carried state (a TBPTT segment of two windows): the
    gradient of a loss on the second window reaches the first window's inputs and start state,
    equal to float64 autograd of the restated forward chain."""
    from hsn_amd.window import WindowRecurrence
    from hsn_amd.workload import CONFIGS, make_window

    cfg_w = CONFIGS["tiny"].scaled(B=2, T=6, N=10, d=4, K=3, h0_sigma=0.3, reset_p=0.1)
    w1 = make_window(cfg_w, 1)
    w2 = make_window(cfg_w, 2)
    cost = torch.full((1,), 1.0 / 10)
    cfg = _route_cfg(k=3)
    g = torch.Generator().manual_seed(9)
    wq = torch.randn(2, cfg_w.T, cfg_w.d, generator=g)
    wh = torch.randn(2, cfg_w.T, cfg_w.K, cfg_w.d, generator=g)

    def chain(dev_, wf):
        y1 = w1["y"].to(dev_, wf).requires_grad_(True)
        g1 = w1["gate_pre"].to(dev_, wf).requires_grad_(True)
        h0 = w1["h0"].to(dev_, wf).requires_grad_(True)
        q0 = w1["q0"].to(dev_, wf).requires_grad_(True)
        y2 = w2["y"].to(dev_, wf).requires_grad_(True)
        g2 = w2["gate_pre"].to(dev_, wf).requires_grad_(True)
        return y1, g1, h0, q0, y2, g2

    # GPU: two autograd nodes chained through (h_T, q_T)
    y1, g1, h0, q0, y2, g2 = chain(dev, torch.float32)
    age0 = w1["age0"].to(dev)
    pos0 = w1["pos0"].to(dev)
    out1 = WindowRecurrence.apply(y1, g1, h0, q0, None, w1["logits"].to(dev), w1["reset"].to(dev),
                                  age0, pos0, cost.to(dev), cfg)
    hT, qT = out1[3], out1[4]
    out2 = WindowRecurrence.apply(y2, g2, hT, qT, None, w2["logits"].to(dev), w2["reset"].to(dev),
                                  age0, pos0, cost.to(dev), cfg)
    loss = (out2[1] * wq.to(dev)).sum() + (out2[2] * wh.to(dev)).sum()
    got = torch.autograd.grad(loss, [y1, g1, h0, q0, y2, g2])

    # float64 reference: the oracle's objective over the two windows chained
    y1c, g1c, h0c, q0c, y2c, g2c = chain("cpu", torch.float64)
    # window 1 carries no loss of its own; window 2's start state is window 1's end state
    total = _two_window_objective(w1, w2, y1c, g1c, h0c, q0c, y2c, g2c, cost, wq.double(),
                                  wh.double())
    want = torch.autograd.grad(total, [y1c, g1c, h0c, q0c, y2c, g2c])
    for name, g_, w_ in zip(("dy1", "dg1", "dh0", "dq0", "dy2", "dg2"), got, want):
        _close(g_, w_, 1e-5, name)


def _two_window_objective(w1, w2, y1, g1, h0, q0, y2, g2, cost, wq, wh):
    B, T, N, _ = w1["logits"].shape
    K = y1.shape[2]
    d = y1.shape[3]

    def run(w, y, gp, h, q, loss_on):
        age = torch.zeros(B, N, dtype=torch.int64)
        pos = torch.zeros(B, dtype=torch.int64)
        total = torch.zeros((), dtype=torch.float64)
        for t in range(T):
            h, q, age, pos = O.reset_state(h, q, age, pos, w["reset"][:, t])
            cells, units, valid, theta, _ = O.router_select(w["logits"][:, t], age, cost, k=K)
            c = O.candidate(y[:, t])
            b = O.gate(gp[:, t])
            h, q, age, _ = O.gated_delta_update(h, q, age, cells, c, b, valid)
            age, pos = O.tick(age, pos, O.selection_mask(cells, valid, N))
            if loss_on:
                total = total + (q * wq[:, t]).sum()
                chosen = h.gather(1, cells.masked_fill(~valid, 0)[:, :, None].expand(B, K, d))
                total = total + (torch.where(valid[..., None], chosen, 0.0) * wh[:, t]).sum()
        return h, q, total

    h1, q1, _ = run(w1, y1, g1, h0, q0, False)
    _, _, total = run(w2, y2, g2, h1, q1, True)
    return total


# --------------------------------------------------------------------------------------------
# the ref-shape window: full-size properties and a per-row oracle check
# --------------------------------------------------------------------------------------------


def test_ref_shape_window_rows_match_oracle(dev, path):
    """The metric's configuration (B32 T256 N256 d64 K8 fp32) on the GPU; rows are independent,
    so rows 0 and 17 are checked against the oracle run on those rows alone, and size-independent
    properties on all rows: q stays the mean of h (q0 = mean h0 and every update moves q by the
    mean delta), the decisions of every 16th position equal the oracle's, and the backward is
    linear in its cotangents (scaling them by 2 scales every gradient by exactly 2)."""
    from hsn_amd import window
    from hsn_amd.workload import CONFIGS, make_cotangents, make_window

    cfg_w = CONFIGS["ref"]
    w = make_window(cfg_w, 2)
    cot = make_cotangents(cfg_w, 2)
    cost = w["cost"]
    cfg = _route_cfg(k=cfg_w.K)
    D = {k: v.to(dev) for k, v in w.items()}
    got = window.window_forward(D["logits"], D["y"], D["gate_pre"], D["reset"], D["h0"], D["q0"],
                                D["age0"], D["pos0"], D["cost"], cfg)
    # every slot valid (budget 1.0, uniform costs)
    assert bool(got["valid"].all())
    # q == mean(h) at the end of the window, from the end state of every row
    _close(got["q"], got["h"].mean(dim=1), 1e-5, "q_T vs mean h_T")
    for t in range(0, cfg_w.T, 16):
        want = O.router_select(w["logits"][:, t], None, cost, k=cfg_w.K)
        assert torch.equal(got["cells"][:, t].cpu().long(), want[0])
        assert torch.equal(got["theta"][:, t].cpu(), want[3])
    rows = [0, 17]
    sub = {k: (v[rows] if isinstance(v, torch.Tensor) and v.dim() > 0 and v.shape[0] == cfg_w.B
               else v) for k, v in w.items()}
    want = O.window_forward(sub["logits"], sub["y"], sub["gate_pre"], sub["reset"], sub["h0"],
                            sub["q0"], sub["age0"], sub["pos0"], cost, k=cfg_w.K)
    for name in ("q_pre", "q_post", "h_old", "h_sel", "h_max"):
        _close(got[name][rows], want[name], F32_TOL, name)
    _close(got["h"][rows], want["h"], F32_TOL, "h_T")
    assert torch.equal(got["age"][rows].cpu(), want["age"])
    d_sel = cot["d_h_sel"]
    args = (D["y"], D["gate_pre"], got["h_old"], got["slots"], D["reset"], cfg_w.N)
    g1 = window.backward(*args, cot["d_q_pre"].to(dev), cot["d_q_post"].to(dev), d_sel.to(dev),
                         cot["d_h_T"].to(dev), cot["d_q_T"].to(dev))
    g2 = window.backward(*args, 2 * cot["d_q_pre"].to(dev), 2 * cot["d_q_post"].to(dev),
                         2 * d_sel.to(dev), 2 * cot["d_h_T"].to(dev), 2 * cot["d_q_T"].to(dev))
    for a, b_ in zip(g1[:4], g2[:4]):
        assert torch.equal(2 * a, b_)
    csub = {k: (v[rows] if v is not None else None) for k, v in cot.items()}
    wb = O.window_backward(sub["y"], sub["gate_pre"], want["h_old"], want["cells"], want["valid"],
                           sub["reset"], cfg_w.N, csub["d_q_pre"], csub["d_q_post"],
                           csub["d_h_sel"], csub["d_h_T"], csub["d_q_T"])
    for name, g_, w_ in zip(("dy", "dgate", "d_h0"), g1[:3], wb[:3]):
        _close(g_[rows], w_, F32_TOL, name)
    _close(g1[3][rows], _d_q0_exact(sub["reset"], csub["d_q_pre"], csub["d_q_post"],
                                    csub["d_q_T"], cfg_w.N), F32_TOL, "d_q0")
    assert math.isfinite(float(got["h_max"].max()))


@pytest.mark.parametrize("path", ["evmap", "slice"])
def test_backward_resets_at_chunk_edges_and_padded_nans(dev, path):
    """The backward's chunked maps at their edges, on the ref shape's sizes (T = 256: sixteen
    chunks of 16 positions on the event maps, eight of 32 on the slices) for two rows.
    - Resets at position 0, at the last position of a chunk (15), at the first of the next (16)
      and at the window's last position (255); two in a row (127, 128) on the other row.
    - NaN and inf in the padded slots' y, gate and h_old (the slots write exact zeros and add
      nothing).
    - A NaN summary cotangent at a position the later reset cuts off from everything before it.
    Against the float64 oracle, d_q0 against the exact sum."""
    from hsn_amd import _lib, window

    cfg_w, w, cot, cost, cfg, _ = _window_case(dict(B=2, T=256, N=256, d=64, K=8, io="f32",
                                                    limit=0.02), 4242)  # 5 of 8 slots valid
    reset = torch.zeros(2, 256, dtype=torch.bool)
    reset[0, [0, 15, 16, 255]] = True
    reset[1, [127, 128]] = True
    fw = O.window_forward(w["logits"], w["y"], w["gate_pre"], reset, w["h0"], w["q0"], w["age0"],
                          w["pos0"], cost, **_oracle_route_kwargs(cfg))
    valid = fw["valid"]
    assert bool((~valid).any())  # the budget pads slots
    y, gp, h_old = w["y"].clone(), w["gate_pre"].clone(), fw["h_old"].clone()
    pad = ~valid
    y[pad] = float("nan")
    gp[pad] = float("inf")
    h_old[pad] = float("nan")
    d_q_pre = cot["d_q_pre"].clone()
    d_q_pre[1, 100, :] = float("nan")  # before the reset at 127: cut off from positions < 127
    d_h_sel = _valid_mask(cot["d_h_sel"], valid)
    wb = O.window_backward(w["y"].double(), w["gate_pre"].double(), fw["h_old"].double(),
                           fw["cells"], valid, reset, 256, d_q_pre.double(),
                           cot["d_q_post"].double(), d_h_sel.double(), cot["d_h_T"].double(),
                           cot["d_q_T"].double())
    _lib.set_path(path)
    try:
        if _lib.path_for(_lib.OP_BACKWARD, 2, 256, 256, 64, 8, _lib.DTYPE_F32) != path:
            pytest.skip(f"the {path} path does not take this shape")
        slots = torch.where(valid, fw["cells"], torch.full_like(fw["cells"], -1)).int()
        gb = window.backward(y.to(dev), gp.to(dev), h_old.to(dev), slots.to(dev), reset.to(dev),
                             256, d_q_pre.to(dev), cot["d_q_post"].to(dev), d_h_sel.to(dev),
                             cot["d_h_T"].to(dev), cot["d_q_T"].to(dev))
    finally:
        _lib.set_path("auto")
    dy, dg = gb[0].cpu(), gb[1].cpu()
    assert bool((dy[pad] == 0).all()) and bool((dg[pad] == 0).all())  # exact zeros, no NaN
    # row 1: the NaN at position 100 reaches the shares of positions <= 100 only up to the
    # reset at 127 ... it lies before 127, so it spreads to every position up to 100 (its own
    # q cotangent); positions from 127 on must be clean
    d_h0 = gb[2].cpu()
    for name, g_, w_ in (("dy", dy, wb[0]), ("dgate", dg, wb[1]), ("d_h0", d_h0, wb[2])):
        nan = torch.isnan(w_)
        assert torch.equal(torch.isnan(g_), nan), name  # NaN exactly where the oracle has it
        assert not bool(torch.isnan(g_[0]).any()), name
        _close(g_[~nan], w_[~nan], F32_TOL, name)
    assert not bool(torch.isnan(dy[1, 127:]).any()) and not bool(torch.isnan(dg[1, 127:]).any())
