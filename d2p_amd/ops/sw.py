"""Structured low-level API for linear-gap soft Smith-Waterman.

Same entry points as the reference's ``d2p/ops/sw.py`` (``forward``,
``forward_t``, ``value_grad_params``, ``marginals_backward``,
``marginals_hvp``, ``marginals_grad_gap``, ``marginals_grad_temp``), each a
pass-through to the ``d2p::sw_*`` operator of the same name.
"""
from typing import Optional, Tuple

from torch import Tensor

from .. import _ops


def forward(scores: Tensor, gap: float, temp: float,
            lengths: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
    """value [B], marginals [B, L1, L2] with scalar parameters."""
    return _ops.sw_forward(scores, gap, temp, lengths)


def forward_t(scores: Tensor, gap: Tensor, temp: Tensor,
              lengths: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
    """value, marginals with tensor parameters (gradients flow to gap/temp)."""
    if lengths is None:
        from ..sw import _full_lengths
        lengths = _full_lengths(scores)
    return _ops.sw_forward_t(scores, gap, temp, lengths)


def value_grad_params(scores: Tensor, gap: float, temp: float,
                      lengths: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
    """d value / d gap [B], d value / d temp [B]."""
    return _ops.sw_value_grad_params(scores, gap, temp, lengths)


def marginals_backward(scores: Tensor, grad_marginals: Tensor, gap: float, temp: float,
                       lengths: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor]:
    """Gradients of <grad_marginals, marginals> w.r.t. scores, gap and temp."""
    return _ops.sw_marginals_backward(scores, grad_marginals, gap, temp, lengths)


def marginals_hvp(scores: Tensor, v: Tensor, gap: float, temp: float,
                  lengths: Optional[Tensor] = None) -> Tensor:
    """Hessian-vector product H @ v with H = d^2 value / d scores^2."""
    return _ops.sw_marginals_hvp(scores, v, gap, temp, lengths)


def marginals_grad_gap(scores: Tensor, gap: float, temp: float,
                       lengths: Optional[Tensor] = None) -> Tensor:
    """d marginals / d gap [B, L1, L2]."""
    return _ops.sw_marginals_grad_gap(scores, gap, temp, lengths)


def marginals_grad_temp(scores: Tensor, gap: float, temp: float,
                        lengths: Optional[Tensor] = None) -> Tensor:
    """d marginals / d temp [B, L1, L2]."""
    return _ops.sw_marginals_grad_temp(scores, gap, temp, lengths)
