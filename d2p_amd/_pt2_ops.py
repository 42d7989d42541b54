"""torch.compile-friendly custom ops (``d2p_py::``) over the ``torch.ops.d2p`` kernels.

Behaviour of the reference's ``d2p/_pt2_ops.py`` for the SW, affine, DTW and
linear NW families (``:72-487,914-1083``): every op is an opaque ``torch.library``
custom op with a fake implementation, so dynamo and FakeTensor tracing never
enter the HIP library; the two value ops of each family (tensor and float
parameters) carry a Python autograd formula:

* value path: ``grad_scores = grad_value[b] * marginals``; parameter gradients
  ``sum_b grad_value[b] * dS_b/dtheta`` from ``*_with_grads``;
* marginal path: ``*_backward_full`` (HVP against the marginal cotangent and its
  dot products with dP/dtheta).

``d2p_amd._ops`` routes a call here while dynamo traces or when an argument is a
FakeTensor; eager calls go straight to ``torch.ops.d2p``.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch.library import custom_op

from ._pt2_utils import _is_fake


def _scalar(value, default: float = 0.0) -> float:
    """A float from a Python number or a one-element tensor (fake tensors carry no
    value: the default stands in; a positive one for temperatures)."""
    if isinstance(value, torch.Tensor):
        return default if _is_fake(value) else float(value.item())
    return float(value)


def _add(a: Optional[torch.Tensor], b: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    if a is None:
        return b
    return a if b is None else a + b


def _scale_rows(g: Optional[torch.Tensor], marginals: torch.Tensor) -> Optional[torch.Tensor]:
    if g is None:
        return None
    return g.view([marginals.size(0)] + [1] * (marginals.dim() - 1)) * marginals


def _dot_sum(g: Optional[torch.Tensor], per_batch: torch.Tensor) -> Optional[torch.Tensor]:
    return None if g is None else (g * per_batch).sum().reshape([1])


def _value_marginals_fake(x):
    B, L1, L2 = x.shape
    return x.new_empty([B]), x.new_empty([B, L1, L2])


def _define(name: str, schema: str, fake):
    """A d2p_py custom op forwarding to torch.ops.d2p.<name>, with a fake kernel."""
    target = getattr(torch.ops.d2p, name)

    def impl(*args):
        out = target(*args)
        return tuple(out) if isinstance(out, (list, tuple)) else out

    op = custom_op(f"d2p_py::{name}", impl, mutates_args=(), schema=schema)
    op.register_fake(fake)
    return op


# ------------------------------------------------------------------ linear-gap SW

_SW_FLOAT = "float gap, float temperature, Tensor? lengths"

soft_sw_with_grads = _define(
    "soft_sw_with_grads", f"(Tensor scores, {_SW_FLOAT}) -> (Tensor, Tensor, Tensor, Tensor)",
    lambda s, g, t, l: (*_value_marginals_fake(s), s.new_empty([s.size(0)]),
                        s.new_empty([s.size(0)])))
soft_sw_hvp = _define(
    "soft_sw_hvp", f"(Tensor scores, Tensor tangent, {_SW_FLOAT}) -> Tensor",
    lambda s, v, g, t, l: s.new_empty(s.shape))
soft_sw_param_jacobian = _define(
    "soft_sw_param_jacobian", f"(Tensor scores, int param_type, {_SW_FLOAT}) -> Tensor",
    lambda s, p, g, t, l: s.new_empty(s.shape))
soft_sw_backward_full = _define(
    "soft_sw_backward_full",
    f"(Tensor scores, Tensor grad_alignment, {_SW_FLOAT}) -> (Tensor, Tensor, Tensor)",
    lambda s, ga, g, t, l: (s.new_empty(s.shape), s.new_empty([1]), s.new_empty([1])))
soft_sw = _define(
    "soft_sw", "(Tensor scores, Tensor gap, Tensor temperature, Tensor lengths) -> "
    "(Tensor, Tensor)", lambda s, g, t, l: _value_marginals_fake(s))
soft_sw_float = _define(
    "soft_sw_float", f"(Tensor scores, {_SW_FLOAT}) -> (Tensor, Tensor)",
    lambda s, g, t, l: _value_marginals_fake(s))


def _sw_setup(ctx, inputs, output):
    scores, gap, temperature, lengths = inputs
    ctx.save_for_backward(scores, output[1])
    ctx.params = (_scalar(gap), _scalar(temperature, 1.0))
    ctx.lengths = lengths


def _sw_backward(ctx, grad_value, grad_marginals):
    scores, marginals = ctx.saved_tensors
    want = ctx.needs_input_grad[1:3]
    grad_scores = _scale_rows(grad_value, marginals)
    grads = [None, None]
    if grad_value is not None and any(want):
        per_batch = soft_sw_with_grads(scores, *ctx.params, ctx.lengths)[2:]
        grads = [_dot_sum(grad_value, g) if w else None for g, w in zip(per_batch, want)]
    if grad_marginals is not None:
        gs, *gp = soft_sw_backward_full(scores, grad_marginals.contiguous(), *ctx.params,
                                        ctx.lengths)
        grad_scores = _add(grad_scores, gs)
        grads = [_add(a, b) if w else None for a, b, w in zip(grads, gp, want)]
    return grad_scores, *grads, None


soft_sw.register_autograd(_sw_backward, setup_context=_sw_setup)
soft_sw_float.register_autograd(_sw_backward, setup_context=_sw_setup)

# ------------------------------------------------------------------ affine-gap SW

_SWA_FLOAT = "float gap_open, float gap_ext, float temperature, Tensor? lengths"

soft_sw_affine_with_grads = _define(
    "soft_sw_affine_with_grads",
    f"(Tensor scores, {_SWA_FLOAT}) -> (Tensor, Tensor, Tensor, Tensor, Tensor)",
    lambda s, o, e, t, l: (*_value_marginals_fake(s),
                           *(s.new_empty([s.size(0)]) for _ in range(3))))
soft_sw_affine_hvp = _define(
    "soft_sw_affine_hvp", f"(Tensor scores, Tensor tangent, {_SWA_FLOAT}) -> Tensor",
    lambda s, v, o, e, t, l: s.new_empty(s.shape))
soft_sw_affine_param_jacobian = _define(
    "soft_sw_affine_param_jacobian", f"(Tensor scores, int param_type, {_SWA_FLOAT}) -> Tensor",
    lambda s, p, o, e, t, l: s.new_empty(s.shape))
soft_sw_affine_backward_full = _define(
    "soft_sw_affine_backward_full",
    f"(Tensor scores, Tensor grad_alignment, {_SWA_FLOAT}) -> (Tensor, Tensor, Tensor, Tensor)",
    lambda s, ga, o, e, t, l: (s.new_empty(s.shape), *(s.new_empty([1]) for _ in range(3))))
soft_sw_affine = _define(
    "soft_sw_affine", "(Tensor scores, Tensor gap_open, Tensor gap_ext, Tensor temperature, "
    "Tensor lengths) -> (Tensor, Tensor)", lambda s, o, e, t, l: _value_marginals_fake(s))
soft_sw_affine_float = _define(
    "soft_sw_affine_float", f"(Tensor scores, {_SWA_FLOAT}) -> (Tensor, Tensor)",
    lambda s, o, e, t, l: _value_marginals_fake(s))


def _swa_setup(ctx, inputs, output):
    scores, go, ge, temperature, lengths = inputs
    ctx.save_for_backward(scores, output[1])
    ctx.params = (_scalar(go), _scalar(ge), _scalar(temperature, 1.0))
    ctx.lengths = lengths


def _swa_backward(ctx, grad_value, grad_marginals):
    scores, marginals = ctx.saved_tensors
    want = ctx.needs_input_grad[1:4]
    grad_scores = _scale_rows(grad_value, marginals)
    grads = [None, None, None]
    if grad_value is not None and any(want):
        per_batch = soft_sw_affine_with_grads(scores, *ctx.params, ctx.lengths)[2:]
        grads = [_dot_sum(grad_value, g) if w else None for g, w in zip(per_batch, want)]
    if grad_marginals is not None:
        gs, *gp = soft_sw_affine_backward_full(scores, grad_marginals.contiguous(), *ctx.params,
                                               ctx.lengths)
        grad_scores = _add(grad_scores, gs)
        grads = [_add(a, b) if w else None for a, b, w in zip(grads, gp, want)]
    return grad_scores, *grads, None


soft_sw_affine.register_autograd(_swa_backward, setup_context=_swa_setup)
soft_sw_affine_float.register_autograd(_swa_backward, setup_context=_swa_setup)

# ------------------------------------------------------------------ soft DTW

_DTW_FLOAT = "float temperature, Tensor? lengths, int? bandwidth"

soft_dtw_with_grads = _define(
    "soft_dtw_with_grads", f"(Tensor costs, {_DTW_FLOAT}) -> (Tensor, Tensor, Tensor)",
    lambda c, t, l, bw: (*_value_marginals_fake(c), c.new_empty([c.size(0)])))
soft_dtw_hvp = _define(
    "soft_dtw_hvp", f"(Tensor costs, Tensor tangent, {_DTW_FLOAT}) -> Tensor",
    lambda c, v, t, l, bw: c.new_empty(c.shape))
soft_dtw_param_jacobian = _define(
    "soft_dtw_param_jacobian", f"(Tensor costs, {_DTW_FLOAT}) -> Tensor",
    lambda c, t, l, bw: c.new_empty(c.shape))
soft_dtw_backward_full = _define(
    "soft_dtw_backward_full", f"(Tensor costs, Tensor grad_alignment, {_DTW_FLOAT}) -> "
    "(Tensor, Tensor)", lambda c, ga, t, l, bw: (c.new_empty(c.shape), c.new_empty([1])))
soft_dtw = _define(
    "soft_dtw", "(Tensor costs, Tensor temperature, Tensor lengths, int bandwidth) -> "
    "(Tensor, Tensor)", lambda c, t, l, bw: _value_marginals_fake(c))
soft_dtw_float = _define(
    "soft_dtw_float", f"(Tensor costs, {_DTW_FLOAT}) -> (Tensor, Tensor)",
    lambda c, t, l, bw: _value_marginals_fake(c))


def _dtw_setup(ctx, inputs, output):
    costs, temperature, lengths, bandwidth = inputs
    ctx.save_for_backward(costs, output[1])
    ctx.temperature = _scalar(temperature, 1.0)
    ctx.lengths = lengths
    ctx.bandwidth = bandwidth


def _dtw_backward(ctx, grad_value, grad_marginals):
    costs, marginals = ctx.saved_tensors
    want_T = ctx.needs_input_grad[1]
    grad_costs = _scale_rows(grad_value, marginals)
    grad_T = None
    if grad_value is not None and want_T:
        per_batch = soft_dtw_with_grads(costs, ctx.temperature, ctx.lengths, ctx.bandwidth)[2]
        grad_T = _dot_sum(grad_value, per_batch)
    if grad_marginals is not None:
        gc, gt = soft_dtw_backward_full(costs, grad_marginals.contiguous(), ctx.temperature,
                                        ctx.lengths, ctx.bandwidth)
        grad_costs = _add(grad_costs, gc)
        if want_T:
            grad_T = _add(grad_T, gt)
    return grad_costs, grad_T, None, None


soft_dtw.register_autograd(_dtw_backward, setup_context=_dtw_setup)
soft_dtw_float.register_autograd(_dtw_backward, setup_context=_dtw_setup)

# ------------------------------------------------------------------ linear-gap NW

soft_nw_with_grads = _define(
    "soft_nw_with_grads", f"(Tensor scores, {_SW_FLOAT}) -> (Tensor, Tensor, Tensor, Tensor)",
    lambda s, g, t, l: (*_value_marginals_fake(s), s.new_empty([s.size(0)]),
                        s.new_empty([s.size(0)])))
soft_nw_hvp = _define(
    "soft_nw_hvp", f"(Tensor scores, Tensor tangent, {_SW_FLOAT}) -> Tensor",
    lambda s, v, g, t, l: s.new_empty(s.shape))
soft_nw_param_jacobian = _define(
    "soft_nw_param_jacobian", f"(Tensor scores, int param_type, {_SW_FLOAT}) -> Tensor",
    lambda s, p, g, t, l: s.new_empty(s.shape))
soft_nw_backward_full = _define(
    "soft_nw_backward_full",
    f"(Tensor scores, Tensor grad_alignment, {_SW_FLOAT}) -> (Tensor, Tensor, Tensor)",
    lambda s, ga, g, t, l: (s.new_empty(s.shape), s.new_empty([1]), s.new_empty([1])))
soft_nw = _define(
    "soft_nw", "(Tensor scores, Tensor gap, Tensor temperature, Tensor lengths) -> "
    "(Tensor, Tensor)", lambda s, g, t, l: _value_marginals_fake(s))
soft_nw_float = _define(
    "soft_nw_float", f"(Tensor scores, {_SW_FLOAT}) -> (Tensor, Tensor)",
    lambda s, g, t, l: _value_marginals_fake(s))


def _nw_backward(ctx, grad_value, grad_marginals):
    scores, marginals = ctx.saved_tensors
    want = ctx.needs_input_grad[1:3]
    grad_scores = _scale_rows(grad_value, marginals)
    grads = [None, None]
    if grad_value is not None and any(want):
        per_batch = soft_nw_with_grads(scores, *ctx.params, ctx.lengths)[2:]
        grads = [_dot_sum(grad_value, g) if w else None for g, w in zip(per_batch, want)]
    if grad_marginals is not None:
        gs, *gp = soft_nw_backward_full(scores, grad_marginals.contiguous(), *ctx.params,
                                        ctx.lengths)
        grad_scores = _add(grad_scores, gs)
        grads = [_add(a, b) if w else None for a, b, w in zip(grads, gp, want)]
    return grad_scores, *grads, None


soft_nw.register_autograd(_nw_backward, setup_context=_sw_setup)
soft_nw_float.register_autograd(_nw_backward, setup_context=_sw_setup)
