"""The entry point that allocates nothing (``hsn_win_forward_noalloc``: its workspace is the
library's own device array) against ``hsn_win_forward`` with a caller workspace, through the C
ABI, on two calls in a row, the second with a smaller window, on each sweep design. The same
kernels run on the same inputs, so every output is bit-identical. GPU only."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _window(dev, B, T, N, d, K, io, seed):
    from hsn_amd.window import RouteConfig, route
    from hsn_amd.workload import CONFIGS, make_window

    cfg = CONFIGS["tiny"].scaled(B=B, T=T, N=N, d=d, K=K, io=io, h0_sigma=0.3, reset_p=0.05)
    w = {k: v.to(dev) for k, v in make_window(cfg, seed).items()}
    slots = route(w["logits"], w["cost"], RouteConfig(k=K), with_slots=True)[5]
    cand_w = (torch.rand(d, generator=torch.Generator().manual_seed(seed)) + 0.5).to(dev)
    return w, slots, cand_w


def _outputs(dev, B, T, N, d, K, io):
    dt = torch.float32 if io == "f32" else torch.bfloat16
    return {"q_pre": torch.full((B, T, d), 3.0, dtype=dt, device=dev),
            "q_post": torch.full((B, T, d), 3.0, dtype=dt, device=dev),
            "h_sel": torch.full((B, T, K, d), 3.0, dtype=dt, device=dev),
            "h_old": torch.full((B, T, K, d), 3.0, dtype=dt, device=dev),
            "h_max": torch.zeros(B, T, device=dev),
            "h": torch.full((B, N, d), 3.0, device=dev),
            "q": torch.full((B, d), 3.0, device=dev),
            "age": torch.zeros(B, N, dtype=torch.int64, device=dev),
            "pos": torch.zeros(B, dtype=torch.int64, device=dev)}


def _call(name, dev, w, slots, cand_w, out, dims, io, workspace=None):
    from hsn_amd import _lib
    from hsn_amd._lib import ptr

    B, T, N, d, K = dims
    code = _lib.DTYPE_F32 if io == "f32" else _lib.DTYPE_BF16
    head = [ptr(w["y"]), ptr(w["gate_pre"]), code, ptr(cand_w), 1, 1e-6]
    if name == "hsn_win_forward":
        head += [ptr(workspace), 0 if workspace is None else workspace.numel()]
    tail = [ptr(w["reset"]), ptr(slots), ptr(w["h0"]), ptr(w["q0"]), ptr(w["age0"]),
            ptr(w["pos0"]), ptr(out["q_pre"]), ptr(out["q_post"]), ptr(out["h_sel"]),
            ptr(out["h_old"]), ptr(out["h_max"]), ptr(out["h"]), ptr(out["q"]), ptr(out["age"]),
            ptr(out["pos"]), B, T, N, d, K, _lib.stream_of(dev)]
    _lib.call(name, *head, *tail)


@pytest.mark.parametrize("path", ["slice", "chain", "evmap"])
@pytest.mark.parametrize("io", ["f32", "bf16"])
def test_noalloc_forward_equals_the_forward_with_a_workspace(cuda_device, io, path):
    from hsn_amd import _lib

    dev = cuda_device
    code = _lib.DTYPE_F32 if io == "f32" else _lib.DTYPE_BF16
    try:
        _lib.set_path(path)
        if path == "evmap" and io != "f32":
            pytest.skip("the event maps take fp32 rows")
        odd_d = 8 if path == "evmap" else 7  # (the event maps take d a multiple of 8)
        for dims, seed in (((6, 40, 64, 32, 8), 3), ((2, 9, 20, odd_d, 3), 4)):  # second smaller
            B, T, N, d, K = dims
            assert _lib.path_for(_lib.OP_FORWARD, B, T, N, d, K, code) == path
            w, slots, cand_w = _window(dev, B, T, N, d, K, io, seed)
            n = _lib.workspace_bytes(_lib.OP_FORWARD, B, T, N, d, K, code, True)
            ws = torch.empty(n, dtype=torch.uint8, device=dev)
            want = _outputs(dev, B, T, N, d, K, io)
            _call("hsn_win_forward", dev, w, slots, cand_w, want, dims, io, ws)
            got = _outputs(dev, B, T, N, d, K, io)
            _call("hsn_win_forward_noalloc", dev, w, slots, cand_w, got, dims, io)
            torch.cuda.synchronize()
            for name in want:
                assert torch.equal(got[name], want[name]), (name, dims, io, path)
    finally:
        _lib.set_path("auto")
