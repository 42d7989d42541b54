"""Soft Needleman-Wunsch (global alignment) on the HIP device, linear and affine gaps.

Same API as the reference's ``d2p.nw`` (/root/reference/d2p/nw.py:68-240):
``soft_nw`` and ``soft_nw_affine`` return ``NWResult(score, alignment)``; ``SoftNW``
and ``SoftNWAffine`` are the ``nn.Module`` wrappers with optional learnable
parameters.  The linear-gap value is alpha[L1, L2] of the global recurrence
(alpha[i,0] = i*gap, alpha[0,j] = j*gap, no restart term); the affine-gap value is
the LSE of the terminal cell's three states (M, I, D), with the boundary chains
I[i,0] = open + (i-1) ext and D[0,j] = open + (j-1) ext.  Gradients flow through the
value (scores, and the parameters when given as tensors) and through the alignment
output (the second-order sweeps: HVP against the alignment cotangent and its dot
products with the parameter Jacobians of the marginals).
"""
from __future__ import annotations

import warnings
from typing import NamedTuple, Optional, Union

import torch
import torch.nn as nn

from . import _ops
from .sw import _validate_temperature

Param = Union[float, torch.Tensor]


class NWResult(NamedTuple):
    """score: the soft global alignment value alpha[L1, L2] [B]; alignment: the
    marginal probability that each cell pair is aligned [B, L1, L2]."""
    score: torch.Tensor
    alignment: torch.Tensor


def _validate_gap(gap: Param, name: str = "gap") -> None:
    """Warns on a positive float gap (the text of /root/reference/d2p/nw.py:54-60)."""
    if isinstance(gap, (int, float)) and gap > 0:
        warnings.warn(f"{name}={gap} is positive. Gap penalties are typically negative.",
                      UserWarning, stacklevel=3)


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


def soft_nw_affine(scores: torch.Tensor, gap_open: Param = -2.0, gap_ext: Param = -0.5,
                   temperature: Param = 1.0,
                   lengths: Optional[torch.Tensor] = None) -> NWResult:
    """Soft Needleman-Wunsch global alignment of scores [B, L1, L2] with affine gaps
    (a gap of length k costs gap_open + (k - 1) * gap_ext)."""
    _validate_temperature(temperature)
    _validate_gap(gap_open, "gap_open")
    _validate_gap(gap_ext, "gap_ext")
    if lengths is None:
        lengths = _make_lengths(scores)
    params = [gap_open, gap_ext, temperature]
    if any(isinstance(p, torch.Tensor) for p in params):
        params = [p if isinstance(p, torch.Tensor) else torch.tensor([p], device=scores.device)
                  for p in params]
        out = _ops.soft_nw_affine(scores, *params, lengths)
    else:
        out = _ops.soft_nw_affine_float(scores, *params, lengths)
    return NWResult(out[0], out[1])


class SoftNWAffine(nn.Module):
    """Affine-gap soft Needleman-Wunsch as a module; ``learnable=True`` makes
    gap_open, gap_ext and temperature parameters."""

    def __init__(self, gap_open: float = -2.0, gap_ext: float = -0.5, temperature: float = 1.0,
                 learnable: bool = False):
        super().__init__()
        if temperature <= 0:
            raise ValueError(f"temperature must be positive, got {temperature}")
        for name, v in (("gap_open", gap_open), ("gap_ext", gap_ext),
                        ("temperature", temperature)):
            t = torch.tensor([v])
            if learnable:
                setattr(self, name, nn.Parameter(t))
            else:
                self.register_buffer(name, t)

    def forward(self, scores: torch.Tensor, lengths: Optional[torch.Tensor] = None) -> NWResult:
        if lengths is None:
            lengths = _make_lengths(scores)
        out = _ops.soft_nw_affine(scores, self.gap_open, self.gap_ext, self.temperature, lengths)
        return NWResult(out[0], out[1])


# low-level re-exports, as in /root/reference/d2p/nw.py:243-256
soft_nw_forward = _ops.soft_nw_float
soft_nw_with_grads = _ops.soft_nw_with_grads
soft_nw_hvp = _ops.soft_nw_hvp
soft_nw_param_jacobian = _ops.soft_nw_param_jacobian
soft_nw_backward_full = _ops.soft_nw_backward_full
soft_nw_affine_forward = _ops.soft_nw_affine_float
soft_nw_affine_with_grads = _ops.soft_nw_affine_with_grads
soft_nw_affine_hvp = _ops.soft_nw_affine_hvp
soft_nw_affine_param_jacobian = _ops.soft_nw_affine_param_jacobian
soft_nw_affine_backward_full = _ops.soft_nw_affine_backward_full
