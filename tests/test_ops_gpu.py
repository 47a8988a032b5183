"""The four-op ABI (gather of the selected cells, gated delta update, their backwards) on the GPU
against the reference's golden vectors, through the custom ops of ``hsn_amd.kernels.ops``.
GPU only.

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


def _close(got, want, dtype, what):
    tol = TOL[dtype]
    torch.testing.assert_close(got.float().cpu(), want.float(), atol=tol, rtol=tol, msg=what)


def _put(v, dev, dtype):
    return {k: (t.to(dev, dtype) if t.is_floating_point() else t.to(dev)) for k, t in v.items()}


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("size", SIZES)
def test_gated_update_matches_golden(ops, cuda_device, size, dtype):
    v = load_golden(f"{size}_gated_delta_update.safetensors")
    D = _put(v, cuda_device, dtype)
    h, q, age = D["h"].clone(), D["q"].clone(), D["age"].clone()
    old = ops.gated_delta_update(h, q, age, D["cell_idx"], D["valid"], D["c"], D["b"])
    _close(h, v["h_out"], dtype, "h_out")
    _close(q, v["q_out"], dtype, "q_out")
    assert torch.equal(age.cpu(), v["age_out"])
    _close(old, v["h_old_saved"], dtype, "h_old_saved")
    gh, gq, gc, gb = ops.gated_delta_update_backward(D["cell_idx"], D["valid"], D["c"], D["b"],
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
    for op in (ops.gated_delta_update_functional, ops.gated_delta_update_state):
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
    out = ops.gather_concat(D["u"], D["eps"], D["h"], D["m"], D["cell_idx"])
    _close(out, v["v"], dtype, "v")
    N = v["h"].shape[1]
    gu, ge, gh, gm = ops.gather_concat_backward(D["grad_v"], D["cell_idx"], N)
    for name, got in zip(("grad_u", "grad_eps", "grad_h", "grad_m"), (gu, ge, gh, gm)):
        _close(got, v[name], dtype, name)


def test_gather_autograd_matches_golden(ops, cuda_device):
    v = load_golden("odd_gather_concat.safetensors")
    D = _put(v, cuda_device, torch.float32)
    leaves = [D[k].clone().requires_grad_(True) for k in ("u", "eps", "h", "m")]
    out = ops.gather_concat(*leaves, D["cell_idx"])
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
        ops.gated_delta_update(h, D["q"].clone(), D["age"].clone(), D["cell_idx"], D["valid"],
                               D["c"], D["b"])
