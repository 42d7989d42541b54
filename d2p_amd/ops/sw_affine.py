"""Structured low-level API for affine-gap soft Smith-Waterman.

Same entry points as the reference's ``d2p/ops/sw_affine.py``, each a
pass-through to the ``d2p::sw_affine_*`` operator of the same name.
"""
from typing import Optional, Tuple

from torch import Tensor

from .. import _ops


def forward(scores: Tensor, gap_open: float, gap_ext: float, temp: float,
            lengths: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
    """value [B], marginals [B, L1, L2] with scalar parameters."""
    return _ops.sw_affine_forward(scores, gap_open, gap_ext, temp, lengths)


def forward_t(scores: Tensor, gap_open: Tensor, gap_ext: Tensor, temp: Tensor,
              lengths: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
    """value, marginals with tensor parameters (gradients flow to the parameters)."""
    if lengths is None:
        from ..sw import _full_lengths
        lengths = _full_lengths(scores)
    return _ops.sw_affine_forward_t(scores, gap_open, gap_ext, temp, lengths)


def value_grad_params(scores: Tensor, gap_open: float, gap_ext: float, temp: float,
                      lengths: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor]:
    """d value / d gap_open, d gap_ext, d temp, each [B]."""
    return _ops.sw_affine_value_grad_params(scores, gap_open, gap_ext, temp, lengths)


def marginals_backward(scores: Tensor, grad_marginals: Tensor, gap_open: float,
                       gap_ext: float, temp: float, lengths: Optional[Tensor] = None):
    """Gradients of <grad_marginals, marginals> w.r.t. scores, gap_open, gap_ext, temp."""
    return _ops.sw_affine_marginals_backward(scores, grad_marginals, gap_open, gap_ext, temp,
                                             lengths)


def marginals_hvp(scores: Tensor, v: Tensor, gap_open: float, gap_ext: float, temp: float,
                  lengths: Optional[Tensor] = None) -> Tensor:
    """Hessian-vector product H @ v with H = d^2 value / d scores^2."""
    return _ops.sw_affine_marginals_hvp(scores, v, gap_open, gap_ext, temp, lengths)


def marginals_grad_gap_open(scores: Tensor, gap_open: float, gap_ext: float, temp: float,
                            lengths: Optional[Tensor] = None) -> Tensor:
    """d marginals / d gap_open [B, L1, L2]."""
    return _ops.sw_affine_marginals_grad_gap_open(scores, gap_open, gap_ext, temp, lengths)


def marginals_grad_gap_ext(scores: Tensor, gap_open: float, gap_ext: float, temp: float,
                           lengths: Optional[Tensor] = None) -> Tensor:
    """d marginals / d gap_ext [B, L1, L2]."""
    return _ops.sw_affine_marginals_grad_gap_ext(scores, gap_open, gap_ext, temp, lengths)


def marginals_grad_temp(scores: Tensor, gap_open: float, gap_ext: float, temp: float,
                        lengths: Optional[Tensor] = None) -> Tensor:
    """d marginals / d temp [B, L1, L2]."""
    return _ops.sw_affine_marginals_grad_temp(scores, gap_open, gap_ext, temp, lengths)
