"""torch.compile / AMP glue: fake (meta) kernels and autocast rules for d2p ops.

Behaviour of the reference's ``d2p/_compile.py`` for the SW, affine, DTW and
NW families (fakes ``:24-415``, autocast ``:857-931``):
* every ``d2p::`` op gets a fake kernel describing its output shapes;
* under ``torch.autocast("cuda")`` every op runs in float32 (inputs are upcast),
  because the DP recurrences accumulate error in 16-bit formats.
The parameter-gradient outputs of ``*_backward_full`` are [1], the shape the
real operators return (the reference's fakes say [B]; the real op wins).
"""
from __future__ import annotations

import torch
from torch.library import register_fake

from . import _ops  # noqa: F401  (registers the d2p namespace)


def _value_marginals(x):
    B, L1, L2 = x.shape
    return [x.new_empty([B]), x.new_empty([B, L1, L2])]


def _per_batch(x, n):
    return tuple(x.new_empty([x.size(0)]) for _ in range(n))


def _full(x, nparams):
    return (x.new_empty(x.shape),) + tuple(x.new_empty([1]) for _ in range(nparams))


_FAKES = {
    # linear SW
    "soft_sw": lambda s, g, t, l: _value_marginals(s),
    "soft_sw_float": lambda s, g, t, l: _value_marginals(s),
    "sw_forward": lambda s, g, t, l: _value_marginals(s),
    "sw_forward_t": lambda s, g, t, l: _value_marginals(s),
    "soft_sw_with_grads": lambda s, g, t, l: tuple(_value_marginals(s)) + _per_batch(s, 2),
    "sw_value_grad_params": lambda s, g, t, l: _per_batch(s, 2),
    "soft_sw_hvp": lambda s, v, g, t, l: s.new_empty(s.shape),
    "sw_marginals_hvp": lambda s, v, g, t, l: s.new_empty(s.shape),
    "soft_sw_param_jacobian": lambda s, p, g, t, l: s.new_empty(s.shape),
    "sw_marginals_grad_gap": lambda s, g, t, l: s.new_empty(s.shape),
    "sw_marginals_grad_temp": lambda s, g, t, l: s.new_empty(s.shape),
    "soft_sw_backward_full": lambda s, ga, g, t, l: _full(s, 2),
    "sw_marginals_backward": lambda s, ga, g, t, l: _full(s, 2),
    # affine SW
    "soft_sw_affine": lambda s, go, ge, t, l: _value_marginals(s),
    "soft_sw_affine_float": lambda s, go, ge, t, l: _value_marginals(s),
    "sw_affine_forward": lambda s, go, ge, t, l: _value_marginals(s),
    "sw_affine_forward_t": lambda s, go, ge, t, l: _value_marginals(s),
    "soft_sw_affine_with_grads":
        lambda s, go, ge, t, l: tuple(_value_marginals(s)) + _per_batch(s, 3),
    "sw_affine_value_grad_params": lambda s, go, ge, t, l: _per_batch(s, 3),
    "soft_sw_affine_hvp": lambda s, v, go, ge, t, l: s.new_empty(s.shape),
    "sw_affine_marginals_hvp": lambda s, v, go, ge, t, l: s.new_empty(s.shape),
    "soft_sw_affine_param_jacobian": lambda s, p, go, ge, t, l: s.new_empty(s.shape),
    "sw_affine_marginals_grad_gap_open": lambda s, go, ge, t, l: s.new_empty(s.shape),
    "sw_affine_marginals_grad_gap_ext": lambda s, go, ge, t, l: s.new_empty(s.shape),
    "sw_affine_marginals_grad_temp": lambda s, go, ge, t, l: s.new_empty(s.shape),
    "soft_sw_affine_backward_full": lambda s, ga, go, ge, t, l: _full(s, 3),
    "sw_affine_marginals_backward": lambda s, ga, go, ge, t, l: _full(s, 3),
    # DTW
    "soft_dtw": lambda c, t, l, bw: _value_marginals(c),
    "soft_dtw_float": lambda c, t, l, bw: _value_marginals(c),
    "soft_dtw_with_grads": lambda c, t, l, bw: tuple(_value_marginals(c)) + _per_batch(c, 1),
    "soft_dtw_hvp": lambda c, v, t, l, bw: c.new_empty(c.shape),
    "soft_dtw_param_jacobian": lambda c, t, l, bw: c.new_empty(c.shape),
    "soft_dtw_backward_full": lambda c, ga, t, l, bw: _full(c, 1),
    # linear NW
    "soft_nw": lambda s, g, t, l: _value_marginals(s),
    "soft_nw_float": lambda s, g, t, l: _value_marginals(s),
    "nw_forward": lambda s, g, t, l: _value_marginals(s),
    "nw_forward_t": lambda s, g, t, l: _value_marginals(s),
    "soft_nw_with_grads": lambda s, g, t, l: tuple(_value_marginals(s)) + _per_batch(s, 2),
    "nw_value_grad_params": lambda s, g, t, l: _per_batch(s, 2),
    "soft_nw_hvp": lambda s, v, g, t, l: s.new_empty(s.shape),
    "nw_marginals_hvp": lambda s, v, g, t, l: s.new_empty(s.shape),
    "soft_nw_param_jacobian": lambda s, p, g, t, l: s.new_empty(s.shape),
    "nw_marginals_grad_gap": lambda s, g, t, l: s.new_empty(s.shape),
    "nw_marginals_grad_temp": lambda s, g, t, l: s.new_empty(s.shape),
    "soft_nw_backward_full": lambda s, ga, g, t, l: _full(s, 2),
    "nw_marginals_backward": lambda s, ga, g, t, l: _full(s, 2),
    # affine NW
    "soft_nw_affine": lambda s, go, ge, t, l: _value_marginals(s),
    "soft_nw_affine_float": lambda s, go, ge, t, l: _value_marginals(s),
    "nw_affine_forward": lambda s, go, ge, t, l: _value_marginals(s),
    "nw_affine_forward_t": lambda s, go, ge, t, l: _value_marginals(s),
    "soft_nw_affine_with_grads":
        lambda s, go, ge, t, l: tuple(_value_marginals(s)) + _per_batch(s, 3),
    "nw_affine_value_grad_params": lambda s, go, ge, t, l: _per_batch(s, 3),
    "soft_nw_affine_hvp": lambda s, v, go, ge, t, l: s.new_empty(s.shape),
    "nw_affine_marginals_hvp": lambda s, v, go, ge, t, l: s.new_empty(s.shape),
    "soft_nw_affine_param_jacobian": lambda s, p, go, ge, t, l: s.new_empty(s.shape),
    "nw_affine_marginals_grad_gap_open": lambda s, go, ge, t, l: s.new_empty(s.shape),
    "nw_affine_marginals_grad_gap_ext": lambda s, go, ge, t, l: s.new_empty(s.shape),
    "nw_affine_marginals_grad_temp": lambda s, go, ge, t, l: s.new_empty(s.shape),
    "soft_nw_affine_backward_full": lambda s, ga, go, ge, t, l: _full(s, 3),
    "nw_affine_marginals_backward": lambda s, ga, go, ge, t, l: _full(s, 3),
}

for _name, _fn in _FAKES.items():
    register_fake(f"d2p::{_name}")(_fn)

# ops of this build without a reference counterpart (namespace d2p_amd)
_AMD_FAKES = {
    "soft_dtw_sqeuclidean": lambda x, y, t, l, bw: (
        x.new_empty([x.size(0)]), x.new_empty([x.size(0), x.size(1), y.size(1)]),
        x.new_empty([x.size(0)])),
    "pairwise_sqdist": lambda x, y: x.new_empty([x.size(0), x.size(1), y.size(1)]),
    "sqeuclid_feature_grad": lambda G, x, y, s: (x.new_empty(x.shape), y.new_empty(y.shape)),
}
for _name, _fn in _AMD_FAKES.items():
    register_fake(f"d2p_amd::{_name}")(_fn)

try:
    from torch.library import register_autocast
except ImportError:  # older torch: autocast rules unavailable
    register_autocast = None

if register_autocast is not None:
    for _name in _FAKES:
        register_autocast(f"d2p::{_name}", "cuda", torch.float32)
    for _name in _AMD_FAKES:
        register_autocast(f"d2p_amd::{_name}", "cuda", torch.float32)

OPS = tuple(_FAKES)
