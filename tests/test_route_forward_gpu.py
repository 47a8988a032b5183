"""The route and forward sweep as one call (``hsn_win_route_forward``) against the two calls it
replaces (``hsn_win_route`` then ``hsn_win_forward``) on the same inputs. GPU only.

Where the call is one launch, the forward's workgroups decide the window themselves and hand the
decisions to each other through device memory; every output must be bit for bit the two calls'
(the same selection code, the same sweep). The exchange is stamped per launch, so calls of other
shapes in between, repeated calls and graph replays must each see their own decisions only.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

OUTPUTS = ("cells", "units", "valid", "refreshed", "theta", "slots", "q_pre", "q_post", "h_sel",
           "h_old", "h", "q", "age", "pos", "h_max")


@pytest.fixture(scope="module")
def dev(cuda_device):
    """The device, with the one launch switched on for this module (the library's default takes
    the two launches, which measure faster at the ref shape)."""
    from hsn_amd import _lib, window

    assert window.available(), "the HIP library must be built for the GPU tests"
    _lib.set_route_forward("one")
    yield cuda_device
    _lib.set_route_forward("auto")


def _bits(t):
    t = t.detach().cpu()
    if t.dtype == torch.float32:
        return t.view(torch.int32)
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16)
    return t


def _inputs(dev, B, T, N, d, K, seed, *, kind="plain", reset_p=0.05):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(B, T, N, 1, generator=g)
    if kind == "ties":  # half-integer logits: many equal scores
        logits = (logits * 2).round() / 2
    elif kind == "nan":
        logits[0, 1, 3, 0] = float("nan")
        logits[-1, 2, 5, 0] = float("nan")
        logits[0, 0, 7, 0] = float("inf")
        logits[-1, 0, 2, 0] = float("-inf")
    elif kind == "zeros":  # every score +-0: more candidates than a wavefront's lanes
        logits = torch.zeros_like(logits)
        logits[..., ::3, :] = -0.0
    w = dict(
        logits=logits,
        y=torch.randn(B, T, K, d, generator=g),
        gate_pre=torch.randn(B, T, K, d, generator=g) * 0.5 + 2.0,
        reset=torch.rand(B, T, generator=g) < reset_p,
        h0=torch.randn(B, N, d, generator=g) * 0.3,
        age0=torch.randint(0, 50, (B, N), generator=g),
        pos0=torch.randint(0, 1000, (B,), generator=g),
        cost=torch.full((1,), 1.0 / N),
    )
    w["q0"] = w["h0"].mean(dim=1)
    w["reset"][0, min(3, T - 1)] = True
    return {k: v.to(dev) for k, v in w.items()}


def _two_calls(w, cfg, *, cand_w=None):
    """hsn_win_route then hsn_win_forward (the sweep's max-reduction into the router's zeros)."""
    from hsn_amd import window

    B, T, N, _ = w["logits"].shape
    h_max = torch.empty(B, T, device=w["y"].device)
    cells, units, valid, theta, refreshed, slots = window.route(
        w["logits"], w["cost"], cfg, h_max_zero=h_max, with_slots=True)
    out = window.forward(w["y"], w["gate_pre"], w["reset"], slots, w["h0"], w["q0"], w["age0"],
                         w["pos0"], N, cand_norm=cand_w is not None, cand_w=cand_w, h_max=h_max,
                         h_max_zeroed=True)
    out.update(cells=cells, units=units, valid=valid, theta=theta, refreshed=refreshed,
               slots=slots)
    return out


def _one_call(w, cfg, *, cand_w=None):
    from hsn_amd import window

    return window.route_forward(w["logits"], w["y"], w["gate_pre"], w["reset"], w["h0"],
                                w["q0"], w["age0"], w["pos0"], w["cost"], cfg,
                                cand_norm=cand_w is not None, cand_w=cand_w)


def _assert_same(got, want, what=""):
    for name in OUTPUTS:
        assert torch.equal(_bits(got[name]), _bits(want[name])), f"{what}: {name}"


CASES = [
    # B, T, N, d, K, route settings, logits kind
    (32, 256, 256, 64, 8, dict(), "plain"),  # the ref shape: one position a wavefront, four each
    (8, 64, 200, 16, 5, dict(), "ties"),  # two slices of 32 positions, N not a power of two
    (4, 40, 64, 32, 3, dict(reserved=1, lambda_cost=0.25, cell_overhead=0.01), "nan"),
    (16, 250, 512, 64, 8, dict(limit=0.01), "plain"),  # eight cells a lane; 5 slots in budget
    (2, 8, 16, 16, 2, dict(), "zeros"),  # the tiny shape, every score +-0
    (4, 32, 130, 16, 4, dict(), "zeros"),  # 130 equal scores: more candidates than lanes
    (3, 21, 40, 8, 4, dict(shared_cost=0.05, limit=0.1), "ties"),  # one slice of 21; 2 in budget
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_one_launch_equals_route_then_forward(dev, case):
    from hsn_amd import window

    B, T, N, d, K, settings, kind = CASES[case]
    fuses, why = window.route_forward_fuses(B, T, N, d, K)
    assert fuses, why
    cfg = window.RouteConfig(k=K, **settings)
    w = _inputs(dev, B, T, N, d, K, 70 + case, kind=kind)
    got = _one_call(w, cfg)
    want = _two_calls(w, cfg)
    _assert_same(got, want, f"case {case}")
    assert bool((~want["valid"]).any()) == ("limit" in settings)  # padded slots where cut
    assert window.exchange_timeouts() == 0


def test_rms_candidate_takes_one_launch_too(dev):
    from hsn_amd import window

    B, T, N, d, K = 4, 64, 128, 32, 6
    assert window.route_forward_fuses(B, T, N, d, K, cand_norm=True)[0]
    cfg = window.RouteConfig(k=K)
    w = _inputs(dev, B, T, N, d, K, 5)
    cand_w = torch.rand(d, generator=torch.Generator().manual_seed(9)).to(dev) + 0.5
    _assert_same(_one_call(w, cfg, cand_w=cand_w), _two_calls(w, cfg, cand_w=cand_w), "rms")


def test_calls_of_other_shapes_in_between_see_their_own_decisions(dev):
    """The exchange words of a row are reused by every launch: a launch of another shape, a
    repeat of the same inputs and new inputs of the first shape each read only their own."""
    from hsn_amd import window

    seq = [(8, 64, 200, 16, 5, 1), (8, 128, 256, 64, 8, 2), (8, 64, 200, 16, 5, 1),
           (8, 64, 200, 16, 5, 3), (32, 256, 256, 64, 8, 4), (8, 64, 200, 16, 5, 5)]
    for i, (B, T, N, d, K, seed) in enumerate(seq):
        cfg = window.RouteConfig(k=K)
        w = _inputs(dev, B, T, N, d, K, seed)
        got = _one_call(w, cfg)
        _assert_same(got, _two_calls(w, cfg), f"call {i}")
    assert window.exchange_timeouts() == 0


def test_without_row_maxima(dev):
    from hsn_amd import window

    B, T, N, d, K = 8, 96, 256, 32, 8
    cfg = window.RouteConfig(k=K)
    w = _inputs(dev, B, T, N, d, K, 11)
    got = window.route_forward(w["logits"], w["y"], w["gate_pre"], w["reset"], w["h0"], w["q0"],
                               w["age0"], w["pos0"], w["cost"], cfg, with_h_max=False)
    want = _two_calls(w, cfg)
    assert "h_max" not in got
    for name in OUTPUTS[:-1]:
        assert torch.equal(_bits(got[name]), _bits(want[name])), name


def test_two_launches_where_the_one_does_not_take_the_call(dev):
    from hsn_amd import window

    cases = [
        (dict(B=8, T=300, N=64, d=64, K=8), "event maps"),  # T above the event maps' 256
        (dict(B=64, T=64, N=64, d=64, K=8), "event maps"),  # 512 workgroups: not one round
        (dict(B=2, T=100, N=64, d=16, K=4), "T <= 32 d / 8"),  # 50 positions a workgroup
        (dict(B=2, T=64, N=513, d=16, K=4), "N <= 512"),
    ]
    for shape, reason in cases:
        fuses, why = window.route_forward_fuses(**shape)
        assert not fuses and reason in why, (shape, why)
    fuses, why = window.route_forward_fuses(2, 64, 64, 16, 4, io=torch.bfloat16)
    assert not fuses and "fp32 rows" in why
    fuses, why = window.route_forward_fuses(2, 64, 64, 16, 4, M=2)
    assert not fuses and "one unit" in why
    # a declined shape still gives the two calls' results
    B, T, N, d, K = 2, 100, 64, 16, 4
    cfg = window.RouteConfig(k=K)
    w = _inputs(dev, B, T, N, d, K, 21)
    _assert_same(_one_call(w, cfg), _two_calls(w, cfg), "declined")


def test_the_default_and_the_setting_take_two_launches(dev):
    from hsn_amd import _lib, window

    B, T, N, d, K = 8, 64, 200, 16, 5
    cfg = window.RouteConfig(k=K)
    w = _inputs(dev, B, T, N, d, K, 51)
    want = _one_call(w, cfg)
    for mode, reason in (("auto", "library's choice"), ("two", "are set")):
        _lib.set_route_forward(mode)
        try:
            fuses, why = window.route_forward_fuses(B, T, N, d, K)
            assert not fuses and reason in why, (mode, why)
            _assert_same(_one_call(w, cfg), want, mode)
        finally:
            _lib.set_route_forward("one")


def test_another_stream_takes_two_launches(dev):
    """The exchange buffers serve the device's first fusing stream; another stream's calls are
    the two launches, ordered on that stream, with the same results."""
    from hsn_amd import window

    B, T, N, d, K = 8, 64, 200, 16, 5
    cfg = window.RouteConfig(k=K)
    w = _inputs(dev, B, T, N, d, K, 31)
    want = _one_call(w, cfg)  # on the current stream, which keeps the buffers
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        fuses, why = window.route_forward_fuses(B, T, N, d, K)
        assert not fuses and "another stream" in why
        got = _one_call(w, cfg)
    torch.cuda.current_stream(dev).wait_stream(side)
    _assert_same(got, want, "side stream")


def test_graph_capture_takes_two_launches_and_replays(dev):
    """A capturing stream never takes the exchange buffers: the captured call is the two
    launches, and each replay (with eager one-launch calls in between) gives the eager result."""
    from hsn_amd import window

    B, T, N, d, K = 8, 64, 200, 16, 5
    cfg = window.RouteConfig(k=K)
    w = _inputs(dev, B, T, N, d, K, 41)
    want = _one_call(w, cfg)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):  # warm-up on the capture stream, as torch advises
        _one_call(w, cfg)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    with torch.cuda.graph(graph):
        static = _one_call(w, cfg)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize(dev)
        _assert_same(static, want, f"replay {i}")
        other = _inputs(dev, B, T, N, d, K, 100 + i)
        _assert_same(_one_call(other, cfg), _two_calls(other, cfg), f"eager after replay {i}")
    assert window.exchange_timeouts() == 0
