"""Soft Needleman-Wunsch (global alignment, linear gap) on the HIP device.

Same API as the reference's ``d2p.nw`` for the linear-gap family
(/root/reference/d2p/nw.py:68-200): ``soft_nw`` returns ``NWResult(score,
alignment)``; ``SoftNW`` is the ``nn.Module`` wrapper with optional learnable gap
and temperature.  The value is alpha[L1, L2] of the global recurrence
(alpha[i,0] = i*gap, alpha[0,j] = j*gap, no restart term); gradients flow through
the value (scores, and gap / temperature when given as tensors) and through the
alignment output (the second-order sweeps: HVP against the alignment cotangent and
its dot products with dP/dgap and dP/dT).  The affine-gap NW family is not part of
this build.
"""
from __future__ import annotations

from typing import NamedTuple, Optional, Union

import torch
import torch.nn as nn

from . import _ops
from .sw import _validate_gap, _validate_temperature

Param = Union[float, torch.Tensor]


class NWResult(NamedTuple):
    """score: the soft global alignment value alpha[L1, L2] [B]; alignment: the
    marginal probability that each cell pair is aligned [B, L1, L2]."""
    score: torch.Tensor
    alignment: torch.Tensor


def _make_lengths(scores: torch.Tensor) -> torch.Tensor:
    B, L1, L2 = scores.shape
    lengths = torch.full((B, 2), L1, dtype=torch.int32, device=scores.device)
    lengths[:, 1].fill_(L2)
    return lengths


def soft_nw(scores: torch.Tensor, gap: Param = -1.0, temperature: Param = 1.0,
            lengths: Optional[torch.Tensor] = None) -> NWResult:
    """Soft Needleman-Wunsch global alignment of scores [B, L1, L2]."""
    _validate_temperature(temperature)
    _validate_gap(gap)
    if lengths is None:
        lengths = _make_lengths(scores)
    gap_t = isinstance(gap, torch.Tensor)
    temp_t = isinstance(temperature, torch.Tensor)
    if gap_t or temp_t:
        if not gap_t:
            gap = torch.tensor([gap], device=scores.device)
        if not temp_t:
            temperature = torch.tensor([temperature], device=scores.device)
        out = _ops.soft_nw(scores, gap, temperature, lengths)
    else:
        out = _ops.soft_nw_float(scores, gap, temperature, lengths)
    return NWResult(out[0], out[1])


class SoftNW(nn.Module):
    """Soft Needleman-Wunsch as a module; ``learnable=True`` makes gap and
    temperature parameters."""

    def __init__(self, gap: float = -1.0, temperature: float = 1.0, learnable: bool = False):
        super().__init__()
        if temperature <= 0:
            raise ValueError(f"temperature must be positive, got {temperature}")
        if learnable:
            self.gap = nn.Parameter(torch.tensor([gap]))
            self.temperature = nn.Parameter(torch.tensor([temperature]))
        else:
            self.register_buffer("gap", torch.tensor([gap]))
            self.register_buffer("temperature", torch.tensor([temperature]))

    def forward(self, scores: torch.Tensor, lengths: Optional[torch.Tensor] = None) -> NWResult:
        if lengths is None:
            lengths = _make_lengths(scores)
        out = _ops.soft_nw(scores, self.gap, self.temperature, lengths)
        return NWResult(out[0], out[1])
