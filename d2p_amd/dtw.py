"""Soft Dynamic Time Warping: high-level API and module.

Drop-in for the reference's ``d2p/dtw.py`` (``soft_dtw`` ``:57-105``,
``SoftDTW`` ``:108-150``, ``DTWResult`` ``:30-38``).  ``bandwidth <= 0`` means
no Sakoe-Chiba band and is passed to the operators as -1 (``d2p/dtw.py:98``).
"""
from __future__ import annotations

from typing import NamedTuple, Optional, Union

import torch
import torch.nn as nn

from . import _ops
from ._pt2_utils import use_pt2_ops


class DTWResult(NamedTuple):
    """``cost`` [B] (soft-min alignment cost) and ``alignment`` [B, L1, L2]."""
    cost: torch.Tensor
    alignment: torch.Tensor


def _validate_temperature(temperature: Union[float, torch.Tensor]) -> None:
    if isinstance(temperature, (int, float)):
        if temperature <= 0:
            raise ValueError(f"temperature must be positive, got {temperature}")
    elif isinstance(temperature, torch.Tensor):
        if use_pt2_ops(temperature):
            return
        if not temperature.requires_grad and temperature.numel() == 1:
            value = temperature.item()
            if value <= 0:
                raise ValueError(f"temperature must be positive, got {value}")


def _full_lengths(costs: torch.Tensor) -> torch.Tensor:
    B, L1, L2 = costs.shape
    lengths = torch.full((B, 2), L1, dtype=torch.int32, device=costs.device)
    lengths[:, 1].fill_(L2)
    return lengths


def soft_dtw(costs: torch.Tensor, temperature: Union[float, torch.Tensor] = 1.0,
             bandwidth: int = 0, lengths: Optional[torch.Tensor] = None) -> DTWResult:
    """Soft DTW over a cost matrix [B, L1, L2] (lower cost = better match).

    Returns DTWResult(cost [B], alignment [B, L1, L2]).
    """
    _validate_temperature(temperature)
    bw = bandwidth if bandwidth > 0 else -1
    if isinstance(temperature, torch.Tensor):
        if lengths is None:
            lengths = _full_lengths(costs)
        out = _ops.soft_dtw(costs, temperature, lengths, bw)
    else:
        out = _ops.soft_dtw_float(costs, float(temperature), lengths, bw)
    return DTWResult(out[0], out[1])


class SoftDTW(nn.Module):
    """nn.Module wrapper of :func:`soft_dtw` with an optional learnable temperature."""

    def __init__(self, temperature: float = 1.0, bandwidth: int = 0, learnable: bool = False):
        super().__init__()
        if temperature <= 0:
            raise ValueError(f"temperature must be positive, got {temperature}")
        self.bandwidth = bandwidth
        t = torch.tensor([temperature])
        if learnable:
            self.temperature = nn.Parameter(t)
        else:
            self.register_buffer("temperature", t)

    def forward(self, costs: torch.Tensor, lengths: Optional[torch.Tensor] = None) -> DTWResult:
        if lengths is None:
            lengths = _full_lengths(costs)
        bw = self.bandwidth if self.bandwidth > 0 else -1
        out = _ops.soft_dtw(costs, self.temperature, lengths, bw)
        return DTWResult(out[0], out[1])


soft_dtw_forward = _ops.soft_dtw_float
soft_dtw_with_grads = _ops.soft_dtw_with_grads
soft_dtw_hvp = _ops.soft_dtw_hvp
soft_dtw_backward_full = _ops.soft_dtw_backward_full
