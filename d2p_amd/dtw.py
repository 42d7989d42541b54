"""Soft Dynamic Time Warping: high-level API and module.

Drop-in for the reference's ``d2p/dtw.py`` (``soft_dtw`` ``:57-105``,
``SoftDTW`` ``:108-150``, ``DTWResult`` ``:30-38``).  ``bandwidth <= 0`` means
no Sakoe-Chiba band and is passed to the operators as -1 (``d2p/dtw.py:98``).

``soft_dtw_sqeuclidean(x, y)`` has no counterpart in the reference: it is soft DTW
over the squared-Euclidean costs ``sum_d (x_i - y_j)^2`` that callers otherwise build
with ``torch.cdist(x, y) ** 2`` (/root/reference/docs/algorithms/dtw.md:52), with the
costs formed on the matrix cores into the alignment buffer (which the forward sweep
reads and the reverse sweep overwrites), so no [B, L1, L2] memory beyond the outputs.
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


class _SoftDTWSqEuclidean(torch.autograd.Function):
    """Value and alignment of soft DTW over c[b,i,j] = |x[b,i] - y[b,j]|^2.

    Backward: the cost gradient G is grad_value[b] * alignment (value path) plus,
    when the alignment itself receives a gradient, soft_dtw_backward_full over the
    cost matrix (formed by d2p_amd::pairwise_sqdist, bit-identical to the op's own
    costs); then dL/dx_i = 2 (rowsum(G)_i x_i - (G y)_i) and dL/dy_j = 2 (colsum(G)_j y_j
    - (G^T x)_j) in one kernel (d2p_amd::sqeuclid_feature_grad, the products on the
    matrix cores).  On the value path alone G is a per-element multiple of the
    alignment, so the kernel reads the alignment itself with the per-element factor:
    no [B, L1, L2] temporary."""

    @staticmethod
    def forward(ctx, x, y, temperature, lengths, bandwidth, t_tensor):
        ctx.set_materialize_grads(False)   # an unused output's gradient stays None
        value, align, grad_t = torch.ops.d2p_amd.soft_dtw_sqeuclidean(x, y, temperature, lengths,
                                                                     bandwidth)
        ctx.save_for_backward(x, y, align, grad_t, lengths if lengths is not None else x.new_empty(0))
        ctx.temperature, ctx.bandwidth, ctx.has_lengths = temperature, bandwidth, lengths is not None
        ctx.mark_non_differentiable(grad_t)
        return value, align

    @staticmethod
    def backward(ctx, g_value, g_align):
        x, y, align, grad_t, lengths = ctx.saved_tensors
        lengths = lengths if ctx.has_lengths else None
        # G = scale[b] * M: M the alignment (value path alone, scale = grad_value) or
        # the full cost gradient (scale = 1)
        M, scale, gT = None, None, None
        if g_value is not None:
            M, scale = align, g_value
            gT = (g_value * grad_t).sum().reshape(1)
        if g_align is not None:
            costs = torch.ops.d2p_amd.pairwise_sqdist(x, y)
            gs, gt2 = torch.ops.d2p.soft_dtw_backward_full(
                costs, g_align.contiguous().float(), ctx.temperature, lengths, ctx.bandwidth)
            M = gs if M is None else g_value[:, None, None] * align + gs
            scale = None
            gT = gt2 if gT is None else gT + gt2
        gx = gy = None
        if M is not None and (ctx.needs_input_grad[0] or ctx.needs_input_grad[1]):
            # dL/dx = 2 s (x rowsum(M) - M y), dL/dy = 2 s (y colsum(M) - M^T x): one
            # kernel, the products on the matrix cores
            s = scale.float().contiguous() if scale is not None else None
            gx, gy = torch.ops.d2p_amd.sqeuclid_feature_grad(M.contiguous(), x, y, s)
            gx = gx if ctx.needs_input_grad[0] else None
            gy = gy if ctx.needs_input_grad[1] else None
        g_temp = gT if ctx.needs_input_grad[5] else None
        return gx, gy, None, None, None, g_temp


def soft_dtw_sqeuclidean(x: torch.Tensor, y: torch.Tensor,
                         temperature: Union[float, torch.Tensor] = 1.0, bandwidth: int = 0,
                         lengths: Optional[torch.Tensor] = None) -> DTWResult:
    """Soft DTW between feature sequences x [B, L1, D] and y [B, L2, D] (1 <= D <= 128)
    under the squared-Euclidean cost |x_i|^2 + |y_j|^2 - 2 x_i . y_j (clamped at 0),
    with the dot products on the matrix cores.

    Same result as ``soft_dtw(torch.cdist(x, y) ** 2, ...)`` up to the rounding of the
    costs (torch.cdist takes the same expansion at these sizes); gradients flow to x, y
    and a tensor temperature.
    """
    _validate_temperature(temperature)
    bw = bandwidth if bandwidth > 0 else -1
    # the sweeps compute in float32 (as every d2p op under autocast)
    x, y = x.float().contiguous(), y.float().contiguous()
    t_tensor = temperature if isinstance(temperature, torch.Tensor) else None
    T = float(temperature.detach().reshape(-1)[0]) if t_tensor is not None else float(temperature)
    value, align = _SoftDTWSqEuclidean.apply(x, y, T, lengths, bw, t_tensor)
    return DTWResult(value, align)
