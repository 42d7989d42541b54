"""Soft Smith-Waterman (linear and affine gap): high-level API and modules.

Drop-in for the reference's ``d2p/sw.py`` (``soft_sw`` ``:247-331``,
``soft_sw_affine`` ``:334-421``, ``SoftSW`` ``:429-511``, ``SoftSWAffine``
``:514-604``, ``SWResult`` ``:44-72``): same signatures, validation, warnings,
mask handling and result type.  Scalar (Python float) parameters call the
``*_float`` operators; tensor parameters call the tensor operators so their
gradients flow.

Differences that do not change results: when neither ``lengths`` nor masks are
given, the float path lets the operator build the full-length table on the
device instead of copying a host list, and the tensor path fills it on the
device.
"""
from __future__ import annotations

import warnings
from typing import NamedTuple, Optional, Union

import torch
import torch.nn as nn

from . import _ops
from ._pt2_utils import use_pt2_ops

Param = Union[float, torch.Tensor]


class SWResult(NamedTuple):
    """``value`` [B] (log-partition) and ``marginals`` [B, L1, L2].

    ``score``/``alignment``/``posteriors`` are aliases kept for compatibility.
    """
    value: torch.Tensor
    marginals: torch.Tensor

    @property
    def score(self) -> torch.Tensor:
        return self.value

    @property
    def alignment(self) -> torch.Tensor:
        return self.marginals

    @property
    def posteriors(self) -> torch.Tensor:
        return self.marginals


# ---------------------------------------------------------------------------
# validation helpers (behaviour of d2p/sw.py:80-239)
# ---------------------------------------------------------------------------

def _validate_temperature(temperature: Param, name: str = "temperature") -> None:
    if isinstance(temperature, (int, float)):
        if temperature <= 0:
            raise ValueError(f"{name} must be positive, got {temperature}")
        return
    if isinstance(temperature, torch.Tensor):
        if use_pt2_ops(temperature):
            return
        if not temperature.requires_grad and temperature.numel() == 1:
            value = temperature.item()
            if value <= 0:
                raise ValueError(f"{name} must be positive, got {value}")


def _validate_gap(gap: Param, name: str = "gap") -> None:
    if isinstance(gap, (int, float)) and gap > 0:
        warnings.warn(
            f"{name}={gap} is positive. Gap penalties are typically negative. "
            "If this is intentional, pass as tensor to suppress this warning.",
            UserWarning, stacklevel=3)


def _as_param_tensor(p: Param, scores: torch.Tensor) -> torch.Tensor:
    """Scalar parameter as a [1] tensor on the scores' device and dtype."""
    if isinstance(p, torch.Tensor):
        if p.dim() == 0:
            p = p.view(1)
        if p.device != scores.device or p.dtype != scores.dtype:
            p = p.to(device=scores.device, dtype=scores.dtype)
        return p
    return torch.tensor([p], device=scores.device, dtype=scores.dtype)


def _full_lengths(scores: torch.Tensor) -> torch.Tensor:
    B, L1, L2 = scores.shape
    lengths = torch.full((B, 2), L1, dtype=torch.int32, device=scores.device)
    lengths[:, 1].fill_(L2)
    return lengths


def _prefix_mask_lengths(mask: torch.Tensor, name: str) -> torch.Tensor:
    """Lengths of a prefix-only boolean mask [B, L]; raises on holes."""
    m = mask.to(torch.int32)
    if m.shape[1] > 1:
        rises = (m[:, 1:] - m[:, :-1]) > 0      # a False followed by a True
        bad = rises.any(dim=1)
        if bad.any():
            idx = bad.nonzero(as_tuple=True)[0].tolist()
            raise ValueError(
                f"{name} is not prefix-only (has holes) at batch indices: {idx}. "
                "Masks must have all True values at the beginning, followed by all False values.")
    return m.sum(dim=1).to(torch.int32)


def _masks_to_lengths(mask1, mask2, B, L1, L2, device) -> torch.Tensor:
    lengths = torch.empty((B, 2), dtype=torch.int32, device=device)
    lengths[:, 0] = _prefix_mask_lengths(mask1, "mask1") if mask1 is not None else L1
    lengths[:, 1] = _prefix_mask_lengths(mask2, "mask2") if mask2 is not None else L2
    return lengths


def _resolve_lengths(scores, lengths, mask1, mask2):
    if lengths is not None and (mask1 is not None or mask2 is not None):
        raise ValueError("Cannot specify both 'lengths' and 'mask1'/'mask2'")
    if mask1 is not None or mask2 is not None:
        B, L1, L2 = scores.shape
        return _masks_to_lengths(mask1, mask2, B, L1, L2, scores.device)
    return lengths


# ---------------------------------------------------------------------------
# functional API
# ---------------------------------------------------------------------------

def soft_sw(scores: torch.Tensor, gap: Param = -1.0, temperature: Param = 1.0,
            lengths: Optional[torch.Tensor] = None, *,
            mask1: Optional[torch.Tensor] = None,
            mask2: Optional[torch.Tensor] = None) -> SWResult:
    """Soft Smith-Waterman local alignment with a linear gap penalty.

    Args:
        scores: similarity matrix [B, L1, L2] (float32, on the HIP device).
        gap: gap penalty (float or scalar tensor; a tensor with requires_grad
            receives a gradient).
        temperature: soft-max temperature > 0 (float or scalar tensor).
        lengths: optional int32 [B, 2] valid lengths per pair.
        mask1, mask2: optional prefix boolean masks [B, L1] / [B, L2] instead of lengths.

    Returns:
        SWResult(value [B], marginals [B, L1, L2]).
    """
    _validate_temperature(temperature)
    _validate_gap(gap)
    lengths = _resolve_lengths(scores, lengths, mask1, mask2)
    if isinstance(gap, torch.Tensor) or isinstance(temperature, torch.Tensor):
        if lengths is None:
            lengths = _full_lengths(scores)
        out = _ops.soft_sw(scores, _as_param_tensor(gap, scores),
                           _as_param_tensor(temperature, scores), lengths)
    else:
        out = _ops.soft_sw_float(scores, float(gap), float(temperature), lengths)
    return SWResult(out[0], out[1])


def soft_sw_affine(scores: torch.Tensor, gap_open: Param = -2.0, gap_ext: Param = -0.5,
                   temperature: Param = 1.0, lengths: Optional[torch.Tensor] = None, *,
                   mask1: Optional[torch.Tensor] = None,
                   mask2: Optional[torch.Tensor] = None) -> SWResult:
    """Soft Smith-Waterman with affine gaps (3-state M/I/D model).

    A gap of length k costs ``gap_open + (k - 1) * gap_ext`` (the reference's
    recurrence, /root/reference/src/sw_affine/kernels_cpu.cpp:149-161).
    """
    _validate_temperature(temperature)
    _validate_gap(gap_open, "gap_open")
    _validate_gap(gap_ext, "gap_ext")
    lengths = _resolve_lengths(scores, lengths, mask1, mask2)
    if any(isinstance(p, torch.Tensor) for p in (gap_open, gap_ext, temperature)):
        if lengths is None:
            lengths = _full_lengths(scores)
        out = _ops.soft_sw_affine(scores, _as_param_tensor(gap_open, scores),
                                  _as_param_tensor(gap_ext, scores),
                                  _as_param_tensor(temperature, scores), lengths)
    else:
        out = _ops.soft_sw_affine_float(scores, float(gap_open), float(gap_ext),
                                        float(temperature), lengths)
    return SWResult(out[0], out[1])


# ---------------------------------------------------------------------------
# modules
# ---------------------------------------------------------------------------

def _param_or_buffer(module: nn.Module, name: str, value: float, learn: bool) -> None:
    t = torch.tensor([value])
    if learn:
        setattr(module, name, nn.Parameter(t))
    else:
        module.register_buffer(name, t)


def _deprecated_learnable(learnable: Optional[bool], message: str) -> bool:
    if learnable is None:
        return False
    warnings.warn(message, DeprecationWarning, stacklevel=3)
    return bool(learnable)


class SoftSW(nn.Module):
    """nn.Module wrapper of :func:`soft_sw` with optional learnable gap/temperature."""

    def __init__(self, gap: float = -1.0, temperature: float = 1.0,
                 learnable: Optional[bool] = None, learn_gap: bool = False,
                 learn_temperature: bool = False):
        super().__init__()
        if temperature <= 0:
            raise ValueError(f"temperature must be positive, got {temperature}")
        if _deprecated_learnable(
                learnable, "The 'learnable' parameter is deprecated. "
                "Use 'learn_gap' and/or 'learn_temperature' instead."):
            learn_gap = learn_temperature = True
        _param_or_buffer(self, "gap", gap, learn_gap)
        _param_or_buffer(self, "temperature", temperature, learn_temperature)

    def forward(self, scores: torch.Tensor, lengths: Optional[torch.Tensor] = None, *,
                mask1: Optional[torch.Tensor] = None,
                mask2: Optional[torch.Tensor] = None) -> SWResult:
        return soft_sw(scores, gap=self.gap, temperature=self.temperature, lengths=lengths,
                       mask1=mask1, mask2=mask2)


class SoftSWAffine(nn.Module):
    """nn.Module wrapper of :func:`soft_sw_affine`."""

    def __init__(self, gap_open: float = -2.0, gap_ext: float = -0.5,
                 temperature: float = 1.0, learnable: Optional[bool] = None,
                 learn_gap_open: bool = False, learn_gap_ext: bool = False,
                 learn_temperature: bool = False):
        super().__init__()
        if temperature <= 0:
            raise ValueError(f"temperature must be positive, got {temperature}")
        if _deprecated_learnable(
                learnable, "The 'learnable' parameter is deprecated. Use 'learn_gap_open', "
                "'learn_gap_ext', and/or 'learn_temperature' instead."):
            learn_gap_open = learn_gap_ext = learn_temperature = True
        _param_or_buffer(self, "gap_open", gap_open, learn_gap_open)
        _param_or_buffer(self, "gap_ext", gap_ext, learn_gap_ext)
        _param_or_buffer(self, "temperature", temperature, learn_temperature)

    def forward(self, scores: torch.Tensor, lengths: Optional[torch.Tensor] = None, *,
                mask1: Optional[torch.Tensor] = None,
                mask2: Optional[torch.Tensor] = None) -> SWResult:
        return soft_sw_affine(scores, gap_open=self.gap_open, gap_ext=self.gap_ext,
                              temperature=self.temperature, lengths=lengths,
                              mask1=mask1, mask2=mask2)


# low-level re-exports, as in d2p/sw.py:612-620
soft_sw_forward = _ops.soft_sw_float
soft_sw_with_grads = _ops.soft_sw_with_grads
soft_sw_hvp = _ops.soft_sw_hvp
soft_sw_backward_full = _ops.soft_sw_backward_full
soft_sw_affine_forward = _ops.soft_sw_affine_float
soft_sw_affine_with_grads = _ops.soft_sw_affine_with_grads
soft_sw_affine_hvp = _ops.soft_sw_affine_hvp
soft_sw_affine_backward_full = _ops.soft_sw_affine_backward_full
