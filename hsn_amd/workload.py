"""Synthetic window workloads: the five configurations of the benchmark contract.

Every tensor is drawn on the CPU from ``torch.Generator().manual_seed(seed)`` in a fixed order,
so a checker on the CPU and the GPU path see identical bits after a copy. The draws follow the
workload definitions (units ``M = 1``, uniform cost table ``1/(N*M)``, zero overhead and shared
cost, budget 1.0 so all ``K`` slots are valid, candidate ``tanh(y)``, write gate
``b = sigmoid(gate_pre)``):

==========  ==========================  ==========================================  =========
config      B, T, N, d, K               distributions                               storage
==========  ==========================  ==========================================  =========
tiny        2, 8, 16, 16, 2             y, logits ~ N(0,1); gate_pre ~ N(2,0.5);     fp32
                                        h0 = q0 = 0; one reset at row 1, pos 4
ref         32, 256, 256, 64, 8         h0 ~ N(0, 0.1^2), q0 = mean_n h0;            fp32
                                        reset ~ Bernoulli(1/256)
bf16        64, 512, 1024, 64, 16       logits += bias_n ~ N(0, 0.5^2);              bf16 I/O
                                        reset ~ Bernoulli(1/128)
tbptt       128, 128 (x16), 512, 128, 8 gate_pre ~ N(3, 0.5); reset ~ Bernoulli(1/256)  fp32
skewed      256, 1024, 4096, 64, 32     logits += -1.1 ln(1 + rank_n) (Zipf bias);   bf16 I/O
                                        reset ~ Bernoulli(1/512)
==========  ==========================  ==========================================  =========

Builder decisions (fixed here, used on both sides): the "decay gate" is the write gate's
pre-activation; ``N(0, 0.1)`` means sigma = 0.1; the cotangents ``d_q_pre, d_q_post [B,T,d]``,
``d_h_sel [B,T,K,d]`` and the end-state cotangents ``d_h_T [B,N,d]``, ``d_q_T [B,d]`` are N(0,1).
"""

from __future__ import annotations

import dataclasses
import math
from typing import Optional

import torch

__all__ = ["Config", "CONFIGS", "make_window", "make_cotangents", "byte_model"]


@dataclasses.dataclass(frozen=True)
class Config:
    name: str
    B: int
    T: int
    N: int
    d: int
    K: int
    M: int = 1
    io: str = "f32"  # storage dtype of inputs/outputs: "f32" or "bf16"
    gate_mu: float = 2.0
    h0_sigma: float = 0.1  # 0 => zero initial state
    reset_p: float = 0.0
    reset_at: Optional[tuple] = None  # explicit (row, pos) resets
    logit_bias: str = "none"  # "none" | "normal" | "zipf"
    windows: int = 1

    @property
    def dtype(self) -> torch.dtype:
        return torch.bfloat16 if self.io == "bf16" else torch.float32

    def scaled(self, **kw) -> "Config":
        return dataclasses.replace(self, **kw)


CONFIGS = {
    "tiny": Config("tiny", 2, 8, 16, 16, 2, h0_sigma=0.0, reset_at=((1, 4),)),
    "ref": Config("ref", 32, 256, 256, 64, 8, reset_p=1 / 256),
    "bf16": Config("bf16", 64, 512, 1024, 64, 16, io="bf16", reset_p=1 / 128,
                   logit_bias="normal"),
    "tbptt": Config("tbptt", 128, 128, 512, 128, 8, gate_mu=3.0, reset_p=1 / 256, windows=16),
    "skewed": Config("skewed", 256, 1024, 4096, 64, 32, io="bf16", reset_p=1 / 512,
                     logit_bias="zipf"),
}


def make_window(cfg: Config, seed: int, *, window: int = 0) -> dict:
    """The inputs of one window of ``cfg`` as CPU tensors (``window`` > 0: the later windows of
    a TBPTT segment draw fresh inputs from the same generator stream but keep the config's
    start state only for window 0)."""
    g = torch.Generator().manual_seed(seed)
    B, T, N, d, K, M = cfg.B, cfg.T, cfg.N, cfg.d, cfg.K, cfg.M
    bias = torch.zeros(N)
    if cfg.logit_bias == "normal":
        bias = torch.randn(N, generator=g) * 0.5
    elif cfg.logit_bias == "zipf":
        rank = torch.randperm(N, generator=g).to(torch.float32)
        bias = -1.1 * torch.log1p(rank)
    for _ in range(window):  # advance the stream deterministically per window
        torch.randn(1, generator=g)
    logits = torch.randn(B, T, N, M, generator=g) + bias[None, None, :, None]
    y = torch.randn(B, T, K, d, generator=g)
    gate_pre = torch.randn(B, T, K, d, generator=g) * 0.5 + cfg.gate_mu
    if cfg.h0_sigma > 0:
        h0 = torch.randn(B, N, d, generator=g) * cfg.h0_sigma
    else:
        h0 = torch.zeros(B, N, d)
    q0 = h0.mean(dim=1)
    reset = torch.zeros(B, T, dtype=torch.bool)
    if cfg.reset_p > 0:
        reset = torch.rand(B, T, generator=g) < cfg.reset_p
    if cfg.reset_at:
        for r, t in cfg.reset_at:
            reset[r, t] = True
    dt = cfg.dtype
    return {
        "logits": logits.to(dt),
        "y": y.to(dt),
        "gate_pre": gate_pre.to(dt),
        "reset": reset,
        "h0": h0,
        "q0": q0,
        "age0": torch.zeros(B, N, dtype=torch.int64),
        "pos0": torch.zeros(B, dtype=torch.int64),
        "cost": torch.full((M,), 1.0 / (N * M), dtype=torch.float32),
    }


def make_cotangents(cfg: Config, seed: int, *, carried: bool = True) -> dict:
    """The backward inputs: cotangents of ``q`` before / after each position, of the selected
    updated states, and (``carried``) of the window's end state."""
    g = torch.Generator().manual_seed(seed + 7919)
    B, T, N, d, K = cfg.B, cfg.T, cfg.N, cfg.d, cfg.K
    dt = cfg.dtype
    out = {
        "d_q_pre": torch.randn(B, T, d, generator=g).to(dt),
        "d_q_post": torch.randn(B, T, d, generator=g).to(dt),
        "d_h_sel": torch.randn(B, T, K, d, generator=g).to(dt),
        "d_h_T": None,
        "d_q_T": None,
    }
    if carried:
        out["d_h_T"] = torch.randn(B, N, d, generator=g)
        out["d_q_T"] = torch.randn(B, d, generator=g)
    return out


def byte_model(cfg: Config) -> dict:
    """Algorithmic HBM bytes per (row, position) of the window's fwd + bwd.

    F = storage bytes (4 fp32, 2 bf16), S = 4 (fp32 state), indices int32, valid/reset u8.

    forward reads  N*M*F (logits) + 2*K*d*F (y, gate_pre) + 1 (reset)
    forward writes 4K + K + 4 (cells, valid, theta) + 2*d*F (q_pre, q_post)
                   + 2*K*d*F (h_sel, h_old)
    forward state  (2*N*d*S + 2*d*S + 2*N*8) / T (h0 in, h_T out, q0/q_T, age0/age_T)
    backward reads 2*K*d*F (y, gate_pre) + K*d*F (h_old) + 5K + 1 (cells, valid, reset)
                   + 2*d*F (d_q_pre, d_q_post) + K*d*F (d_h_sel)
    backward writes 2*K*d*F (dy, dgate)
    backward state (2*N*d*S + 2*d*S) / T (d_h_T, d_q_T in; d_h0, d_q0 out)
    """
    F = 2 if cfg.io == "bf16" else 4
    S = 4
    B, T, N, d, K, M = cfg.B, cfg.T, cfg.N, cfg.d, cfg.K, cfg.M
    route = N * M * F + 1 + 4 * K + K + 4
    fwd_only = 2 * K * d * F + 2 * d * F + 2 * K * d * F + (2 * N * d * S + 2 * d * S + 2 * N * 8) / T
    fwd = route + fwd_only
    bwd = 2 * K * d * F + K * d * F + 5 * K + 1 + 2 * d * F + K * d * F + 2 * K * d * F \
        + (2 * N * d * S + 2 * d * S) / T
    return {"route": route, "forward": fwd, "forward_update": fwd_only, "backward": bwd,
            "total": fwd + bwd, "window_bytes": (fwd + bwd) * B * T}


def describe(cfg: Config) -> str:
    return f"B{cfg.B} T{cfg.T} N{cfg.N} d{cfg.d} K{cfg.K} M{cfg.M} {cfg.io}"


def _check_byte_model() -> None:  # pragma: no cover - used interactively
    for name, cfg in CONFIGS.items():
        bm = byte_model(cfg)
        print(name, round(bm["forward"]), round(bm["backward"]), round(bm["total"]),
              bm["window_bytes"] / 1e6, math.floor(8e12 / bm["total"] / 1e6))


#: The reverse sweep's workloads. "ref" is the reference's model at its ref shape (B 32, K 8,
#: d 64, M 8 units of H 512 over a 256-position window of 256 cells; the cell input is
#: [u; eps; h; m], 4d wide; 8 message sources a cell).
SWEEP_CONFIGS = {
    "ref": dict(B=32, T=256, K=8, N=256, d=64, H=512, M=8, D=8),
    "tiny": dict(B=2, T=8, K=3, N=16, d=8, H=16, M=2, D=3),
}


def make_sweep_window(B: int, T: int, K: int, N: int, d: int, H: int, M: int, D: int, *,
                      seed: int = 0, device="cpu", product_dtype=torch.float32):
    """Synthetic arguments of the state-gradient sweep (``state_gradient_backward``'s, for
    ``hsn_amd.state_sweep.SweepRunner``): seeded values of a window's shape: distinct cells per
    position (one slot in 16 padded), units, a few resets, candidates and gates in their ranges,
    a random cell (both norms, GELU) and message graph. Returns ``(args, kwargs)``."""
    from .state_sweep import CellConstants

    g = torch.Generator().manual_seed(seed)
    f32 = torch.float32

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to(device)

    n = 4 * d
    cells = torch.argsort(torch.rand(B, T, N, generator=g), dim=-1)[..., :K]
    valid = torch.rand(B, T, K, generator=g) >= 1.0 / 16
    units = torch.randint(0, M, (B, T, K), generator=g)
    reset = torch.rand(B, T, generator=g) < 1.0 / 64
    pad_src = torch.randint(0, N, (N, D), generator=g)
    pad_mask = torch.rand(N, D, generator=g) < 0.9
    consts = CellConstants(
        w_out=rnd(d, d, scale=d ** -0.5), cand_gain=1.0 + rnd(d, scale=0.1), cand_eps=1e-6,
        w2=rnd(M, H, d, scale=H ** -0.5), w1_state=rnd(M, 2 * d, H, scale=n ** -0.5),
        b1=rnd(M, H, scale=0.1), gate_state=rnd(d, 2 * d, scale=n ** -0.5),
        gate_bias=rnd(d, scale=0.1), norm_gain_state=1.0 + rnd(2 * d, scale=0.1), in_dim=n,
        v=rnd(d, d, scale=d ** -0.5),
        edge_weights=torch.where(pad_mask.to(device), rnd(N, D, scale=0.3), torch.zeros((), device=device)),
        pad_src=pad_src.to(device), activation="gelu", pad_mask=pad_mask.to(device))
    c = torch.tanh(rnd(B, T, K, d))
    b = torch.sigmoid(rnd(B, T, K, d))
    record = {
        "y": rnd(B, T, K, d), "alpha": torch.ones(B, T, K, dtype=f32, device=device),
        "hidden": rnd(B, T, K, H).to(product_dtype), "gate_pre": rnd(B, T, K, d),
        "m": rnd(B, T, K, d, scale=0.5), "rms": 0.5 + torch.rand(B, T, K, generator=g).to(device),
    }
    args = (c, b, rnd(B, T, K, d, scale=0.5), cells.to(device), units.to(device), valid.to(device),
            reset.to(device), N, rnd(B, T, d), rnd(B, T, d), rnd(B, T, K, d), None, record, consts)
    return args, dict(n_read=0)


# --------------------------------------------------------------------------------------------
# the fused cell round (hsn_amd.kernels.window.cell_round)
# --------------------------------------------------------------------------------------------

#: the round's bench shape: the reverse sweep's model (B 32, K 8 slots of N 256 cells, d 64,
#: H 512 hidden units in each of M 8 units, D 8 padded in-edges)
ROUND_CONFIGS = {
    "ref": dict(B=32, K=8, N=256, d=64, H=512, M=8, D=8),
    "tiny": dict(B=2, K=3, N=16, d=8, H=16, M=2, D=3),
}


def make_round_cell(*, N: int, d: int, M: int, H: int, D: int, cand_norm: bool = True,
                    seed: int = 0, device="cpu"):
    """A cell with what the fused round reads, under the reference PDGCell's attribute names
    (``V``, ``norm``, ``gate``, ``W_out``, ``cand_norm``, ``units.W1 / b1 / W2 / b2``,
    ``graph._pad_src``; python/hsn/model/cell.py), seeded values away from their initial ones,
    and the window's padded edge weights ``[N, D]`` (softmax over each cell's edges, 0 on
    padding). Returns ``(cell, edge_weights)``."""
    from types import SimpleNamespace

    g = torch.Generator().manual_seed(seed)
    n = 4 * d

    def rnd(*shape, scale=1.0):
        return torch.randn(*shape, generator=g) * scale

    def linear(out_f, in_f, bias):
        lin = torch.nn.Linear(in_f, out_f, bias=bias)
        with torch.no_grad():
            lin.weight.copy_(rnd(out_f, in_f, scale=in_f ** -0.5) + 0.2 * rnd(out_f, in_f,
                                                                               scale=0.2))
            if bias:
                lin.bias.copy_(0.2 * rnd(out_f))
        return lin.to(device)

    def rms_norm(width):
        norm = torch.nn.RMSNorm(width, eps=1e-6)
        with torch.no_grad():
            norm.weight.copy_(1.0 + 0.2 * rnd(width))
        return norm.to(device)

    mask = torch.rand(N, D, generator=g) < 0.75
    if D:
        mask[:, 0] = True
    pad_src = torch.where(mask, torch.randint(0, N, (N, D), generator=g), torch.zeros((), dtype=torch.int64))
    weights = torch.where(mask, torch.softmax(rnd(N, D), dim=1), torch.zeros(()))
    units = SimpleNamespace(
        activation_name="gelu", hidden=H,
        W1=(rnd(M, n, H, scale=n ** -0.5)).to(device), b1=(0.2 * rnd(M, H)).to(device),
        W2=(rnd(M, H, d, scale=H ** -0.5)).to(device), b2=(0.2 * rnd(M, d)).to(device))
    cell = SimpleNamespace(
        d=d, ablate_shared_u=False, cell_norm="rms", disabled_cells=(),
        cand_norm_kind="rms" if cand_norm else "none",
        V=linear(d, d, False), norm=rms_norm(n), gate=linear(d, n, True),
        W_out=linear(d, d, False),
        cand_norm=rms_norm(d) if cand_norm else torch.nn.Identity(),
        units=units, graph=SimpleNamespace(_pad_src=pad_src.to(device)))
    return cell, weights.to(device)


def make_round_positions(*, B: int, K: int, N: int, d: int, M: int, T: int, seed: int = 0,
                         pad_every: int = 16, device="cpu"):
    """``T`` positions of inputs and hard decisions for the fused round: ``u, eps [T, B, d]``,
    ``cells, units [T, B, K]`` (distinct cells a row), ``valid [T, B, K]`` (every
    ``pad_every``-th slot padded: cell 0, unit 0), and a start state (states uniform in
    [-0.8, 0.8], ``q`` their mean, small ages)."""
    from .state import CellGraphState

    g = torch.Generator().manual_seed(seed)
    cells = torch.argsort(torch.rand(T, B, N, generator=g), dim=-1)[..., :K]
    units = torch.randint(0, M, (T, B, K), generator=g)
    valid = torch.ones(T, B, K, dtype=torch.bool)
    valid.view(-1)[pad_every - 1::pad_every] = False
    cells = torch.where(valid, cells, torch.zeros_like(cells))
    units = torch.where(valid, units, torch.zeros_like(units))
    h = torch.rand(B, N, d, generator=g) * 1.6 - 0.8
    state = CellGraphState.make(h=h.to(device), q=h.mean(dim=1).to(device),
                                age=torch.randint(0, 9, (B, N), generator=g).to(device),
                                pos=torch.zeros(B, dtype=torch.int64, device=device))
    return dict(u=torch.randn(T, B, d, generator=g).to(device),
                eps=torch.randn(T, B, d, generator=g).to(device), cells=cells.to(device),
                units=units.to(device), valid=valid.to(device), state=state)


def round_bytes(cfg: dict, units_present: int) -> int:
    """Algorithmic HBM bytes of one position's fused round: the state read and written once
    (h, the ages), q, the decision and inputs, the slots' message sources, and the weights the
    position reads once (V, the gate, W_out, the norms' gains, and each present unit's W1, W2,
    biases). The scratch between the launches (v, gate, F's chunk shares) is not counted: it is
    the kernels' own traffic, not the algorithm's."""
    B, K, N, d, H, D = (cfg[k] for k in ("B", "K", "N", "d", "H", "D"))
    n = 4 * d
    state = B * N * d * 4 * 2 + B * N * 8 * 2 + B * d * 4 * 2  # h, age, q: read and written
    slots = B * K * (8 + 8 + 1 + 4) + B * d * 4 * 2 + B * K * d * 4  # decision, u, eps, h_sel
    sources = B * K * (D * (8 + 4) + (D + 1) * d * 4)  # edges, source rows and the own row
    shared = 4 * (d * d + d * n + d + n + d * d + d) + N * D * 12
    unit = 4 * (n * H + H + H * d + d)
    return state + slots + sources + shared + units_present * unit
