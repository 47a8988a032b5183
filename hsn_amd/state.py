"""The window state and its boundary semantics, as the reference's ``CellGraphState``
(python/hsn/model/state.py:197-361): ``h [B,N,d]`` fp32, ``q [B,d]`` fp32 (the incremental
summary), ``age [B,N]`` int64, ``pos [B]`` int64.

A plain container for the per-position operators of :mod:`hsn_amd.kernels.window`; the
whole-window path (:mod:`hsn_amd.window`) keeps the state on chip and takes these tensors as
its start state. ``reset`` zeroes rows with ``masked_fill`` (a NaN in a reset row cannot leak,
state.py:267-283); ``tick`` is ``age += ~selected, pos += 1`` (state.py:316-324).
"""

from __future__ import annotations

import dataclasses
from typing import NamedTuple, Optional

import torch
from torch import Tensor


class CellGraphState(NamedTuple):
    h: Tensor
    q: Tensor
    age: Tensor
    pos: Tensor

    @classmethod
    def make(cls, *, h: Tensor, q: Tensor, age: Tensor, pos: Tensor) -> "CellGraphState":
        """The reference's ``CellGraphState._make(h=, q=, age=, pos=)``."""
        return cls(h=h, q=q, age=age, pos=pos)

    @classmethod
    def zeros(cls, B: int, N: int, d: int, device=None) -> "CellGraphState":
        return cls(
            h=torch.zeros(B, N, d, device=device),
            q=torch.zeros(B, d, device=device),
            age=torch.zeros(B, N, dtype=torch.int64, device=device),
            pos=torch.zeros(B, dtype=torch.int64, device=device),
        )

    def reset(self, mask: Tensor) -> "CellGraphState":
        return CellGraphState(
            h=self.h.masked_fill(mask[:, None, None], 0),
            q=self.q.masked_fill(mask[:, None], 0),
            age=self.age.masked_fill(mask[:, None], 0),
            pos=self.pos.masked_fill(mask, 0),
        )

    def tick(self, selected: Tensor) -> "CellGraphState":
        return self._replace(age=self.age + (~selected).to(torch.int64), pos=self.pos + 1)

    def detach(self) -> "CellGraphState":
        return CellGraphState(*(t.detach() for t in self))


@dataclasses.dataclass
class _Norm:
    weight: Tensor
    eps: Optional[float] = 1e-6


@dataclasses.dataclass
class CandidateSpec:
    """What the per-position update reads off the reference's ``PDGCell``
    (python/hsn/model/cell.py:211,480-484): the candidate's norm kind (``"none"`` or
    ``"rms"``), its gain and eps. Any object with ``cand_norm_kind``, ``cand_norm`` (``weight``,
    ``eps``) and ``norm`` (``weight``) works in its place, a ``PDGCell`` included."""

    cand_norm_kind: str
    cand_norm: Optional[_Norm]
    norm: _Norm

    @classmethod
    def plain(cls, d: int, device=None) -> "CandidateSpec":
        w = torch.ones(d, device=device)
        return cls("none", None, _Norm(w))

    @classmethod
    def rms(cls, weight: Tensor, eps: float = 1e-6) -> "CandidateSpec":
        return cls("rms", _Norm(weight, eps), _Norm(weight))
