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

Parameters keep the form the caller gave them.  A tensor parameter (a learnable
gap or temperature) is saved for backward like any other tensor and reaches the
backward kernels through ``d2p_py::*_tp`` ops whose schema takes the parameters
as ``Tensor[]``: their real implementation reads the values, so a compiled
backward always runs with the parameters of its own forward.  (Reading a value
while tracing would see a FakeTensor, which carries none.)

``d2p_amd._ops`` routes a call here while dynamo traces or when an argument is a
FakeTensor; eager calls go straight to ``torch.ops.d2p``.
"""
from __future__ import annotations

from typing import List, Optional, Sequence

import torch
from torch.library import custom_op


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


def _define_tp(name: str, head: str, tail: str, result: str, fake):
    """``d2p_py::<name>_tp``: torch.ops.d2p.<name> with its float parameters passed as
    one-element tensors.  ``head`` are the tensor arguments before the parameters,
    ``tail`` the arguments after them."""
    target = getattr(torch.ops.d2p, name)
    n_head = head.count("Tensor")

    def impl(*args):
        lead, params, rest = args[:n_head], args[n_head], args[n_head + 1:]
        values = [float(p.reshape(-1)[0].item()) for p in params]
        out = target(*lead, *values, *rest)
        return tuple(out) if isinstance(out, (list, tuple)) else out

    schema = f"({head}, Tensor[] params, {tail}) -> {result}"
    op = custom_op(f"d2p_py::{name}_tp", impl, mutates_args=(), schema=schema)
    op.register_fake(fake)
    return op


# ------------------------------------------------------------------ saved parameters

def _save(ctx, main: Sequence[torch.Tensor], params: Sequence, lengths) -> None:
    """Saves the main tensors, the parameters (tensors through save_for_backward,
    numbers as floats) and the lengths."""
    tensors = list(main)
    ctx.param_is_tensor = [isinstance(p, torch.Tensor) for p in params]
    ctx.param_floats = [None if t else float(p) for p, t in zip(params, ctx.param_is_tensor)]
    tensors += [p for p in params if isinstance(p, torch.Tensor)]
    ctx.has_lengths = isinstance(lengths, torch.Tensor)
    if ctx.has_lengths:
        tensors.append(lengths)
    ctx.n_main = len(main)
    ctx.save_for_backward(*tensors)


def _restore(ctx):
    """(main tensors, parameters as saved, lengths or None)."""
    saved = list(ctx.saved_tensors)
    main, rest = saved[:ctx.n_main], saved[ctx.n_main:]
    params = []
    for is_t, f in zip(ctx.param_is_tensor, ctx.param_floats):
        params.append(rest.pop(0) if is_t else f)
    lengths = rest.pop(0) if ctx.has_lengths else None
    return main, params, lengths


def _param_tensors(params: List, like: torch.Tensor) -> List[torch.Tensor]:
    return [p if isinstance(p, torch.Tensor) else like.new_tensor([p]) for p in params]


def _call(float_op, tp_op, lead: Sequence[torch.Tensor], params: List, rest: Sequence):
    """The float-parameter op when every parameter is a number, else the _tp op."""
    if any(isinstance(p, torch.Tensor) for p in params):
        return tp_op(*lead, _param_tensors(params, lead[0]), *rest)
    return float_op(*lead, *params, *rest)


# ------------------------------------------------------------------ linear-gap SW

_SW_FLOAT = "float gap, float temperature, Tensor? lengths"


def _sw_grads_fake(s, *_):
    return (*_value_marginals_fake(s), s.new_empty([s.size(0)]), s.new_empty([s.size(0)]))


def _sw_full_fake(s, ga, *_):
    return s.new_empty(s.shape), s.new_empty([1]), s.new_empty([1])


soft_sw_with_grads = _define(
    "soft_sw_with_grads", f"(Tensor scores, {_SW_FLOAT}) -> (Tensor, Tensor, Tensor, Tensor)",
    _sw_grads_fake)
soft_sw_hvp = _define(
    "soft_sw_hvp", f"(Tensor scores, Tensor tangent, {_SW_FLOAT}) -> Tensor",
    lambda s, v, g, t, l: s.new_empty(s.shape))
soft_sw_param_jacobian = _define(
    "soft_sw_param_jacobian", f"(Tensor scores, int param_type, {_SW_FLOAT}) -> Tensor",
    lambda s, p, g, t, l: s.new_empty(s.shape))
soft_sw_backward_full = _define(
    "soft_sw_backward_full",
    f"(Tensor scores, Tensor grad_alignment, {_SW_FLOAT}) -> (Tensor, Tensor, Tensor)",
    _sw_full_fake)
soft_sw = _define(
    "soft_sw", "(Tensor scores, Tensor gap, Tensor temperature, Tensor lengths) -> "
    "(Tensor, Tensor)", lambda s, g, t, l: _value_marginals_fake(s))
soft_sw_float = _define(
    "soft_sw_float", f"(Tensor scores, {_SW_FLOAT}) -> (Tensor, Tensor)",
    lambda s, g, t, l: _value_marginals_fake(s))
soft_sw_with_grads_tp = _define_tp(
    "soft_sw_with_grads", "Tensor scores", "Tensor? lengths",
    "(Tensor, Tensor, Tensor, Tensor)", _sw_grads_fake)
soft_sw_backward_full_tp = _define_tp(
    "soft_sw_backward_full", "Tensor scores, Tensor grad_alignment", "Tensor? lengths",
    "(Tensor, Tensor, Tensor)", _sw_full_fake)


def _first_order_setup(ctx, inputs, output):
    """Inputs (scores, *params, lengths) of a family's value op."""
    scores, *params, lengths = inputs
    _save(ctx, (scores, output[1]), params, lengths)


def _first_order_backward(with_grads, with_grads_tp, backward_full, backward_full_tp):
    """Autograd formula of a family's value ops (value path and marginal path)."""

    def backward(ctx, grad_value, grad_marginals):
        (scores, marginals), params, lengths = _restore(ctx)
        want = ctx.needs_input_grad[1:1 + len(params)]
        grad_scores = _scale_rows(grad_value, marginals)
        grads = [None] * len(params)
        if grad_value is not None and any(want):
            per_batch = _call(with_grads, with_grads_tp, (scores,), params, (lengths,))[2:]
            grads = [_dot_sum(grad_value, g) if w else None for g, w in zip(per_batch, want)]
        if grad_marginals is not None:
            gs, *gp = _call(backward_full, backward_full_tp,
                            (scores, grad_marginals.contiguous()), params, (lengths,))
            grad_scores = _add(grad_scores, gs)
            grads = [_add(a, b) if w else None for a, b, w in zip(grads, gp, want)]
        return grad_scores, *grads, None

    return backward


_sw_backward = _first_order_backward(soft_sw_with_grads, soft_sw_with_grads_tp,
                                     soft_sw_backward_full, soft_sw_backward_full_tp)
soft_sw.register_autograd(_sw_backward, setup_context=_first_order_setup)
soft_sw_float.register_autograd(_sw_backward, setup_context=_first_order_setup)

# ------------------------------------------------------------------ affine-gap SW

_SWA_FLOAT = "float gap_open, float gap_ext, float temperature, Tensor? lengths"


def _swa_grads_fake(s, *_):
    return (*_value_marginals_fake(s), *(s.new_empty([s.size(0)]) for _ in range(3)))


def _swa_full_fake(s, ga, *_):
    return (s.new_empty(s.shape), *(s.new_empty([1]) for _ in range(3)))


soft_sw_affine_with_grads = _define(
    "soft_sw_affine_with_grads",
    f"(Tensor scores, {_SWA_FLOAT}) -> (Tensor, Tensor, Tensor, Tensor, Tensor)",
    _swa_grads_fake)
soft_sw_affine_hvp = _define(
    "soft_sw_affine_hvp", f"(Tensor scores, Tensor tangent, {_SWA_FLOAT}) -> Tensor",
    lambda s, v, o, e, t, l: s.new_empty(s.shape))
soft_sw_affine_param_jacobian = _define(
    "soft_sw_affine_param_jacobian", f"(Tensor scores, int param_type, {_SWA_FLOAT}) -> Tensor",
    lambda s, p, o, e, t, l: s.new_empty(s.shape))
soft_sw_affine_backward_full = _define(
    "soft_sw_affine_backward_full",
    f"(Tensor scores, Tensor grad_alignment, {_SWA_FLOAT}) -> (Tensor, Tensor, Tensor, Tensor)",
    _swa_full_fake)
soft_sw_affine = _define(
    "soft_sw_affine", "(Tensor scores, Tensor gap_open, Tensor gap_ext, Tensor temperature, "
    "Tensor lengths) -> (Tensor, Tensor)", lambda s, o, e, t, l: _value_marginals_fake(s))
soft_sw_affine_float = _define(
    "soft_sw_affine_float", f"(Tensor scores, {_SWA_FLOAT}) -> (Tensor, Tensor)",
    lambda s, o, e, t, l: _value_marginals_fake(s))
soft_sw_affine_with_grads_tp = _define_tp(
    "soft_sw_affine_with_grads", "Tensor scores", "Tensor? lengths",
    "(Tensor, Tensor, Tensor, Tensor, Tensor)", _swa_grads_fake)
soft_sw_affine_backward_full_tp = _define_tp(
    "soft_sw_affine_backward_full", "Tensor scores, Tensor grad_alignment", "Tensor? lengths",
    "(Tensor, Tensor, Tensor, Tensor)", _swa_full_fake)

_swa_backward = _first_order_backward(soft_sw_affine_with_grads, soft_sw_affine_with_grads_tp,
                                      soft_sw_affine_backward_full,
                                      soft_sw_affine_backward_full_tp)
soft_sw_affine.register_autograd(_swa_backward, setup_context=_first_order_setup)
soft_sw_affine_float.register_autograd(_swa_backward, setup_context=_first_order_setup)

# ------------------------------------------------------------------ soft DTW

_DTW_FLOAT = "float temperature, Tensor? lengths, int? bandwidth"


def _dtw_grads_fake(c, *_):
    return (*_value_marginals_fake(c), c.new_empty([c.size(0)]))


def _dtw_full_fake(c, ga, *_):
    return c.new_empty(c.shape), c.new_empty([1])


soft_dtw_with_grads = _define(
    "soft_dtw_with_grads", f"(Tensor costs, {_DTW_FLOAT}) -> (Tensor, Tensor, Tensor)",
    _dtw_grads_fake)
soft_dtw_hvp = _define(
    "soft_dtw_hvp", f"(Tensor costs, Tensor tangent, {_DTW_FLOAT}) -> Tensor",
    lambda c, v, t, l, bw: c.new_empty(c.shape))
soft_dtw_param_jacobian = _define(
    "soft_dtw_param_jacobian", f"(Tensor costs, {_DTW_FLOAT}) -> Tensor",
    lambda c, t, l, bw: c.new_empty(c.shape))
soft_dtw_backward_full = _define(
    "soft_dtw_backward_full", f"(Tensor costs, Tensor grad_alignment, {_DTW_FLOAT}) -> "
    "(Tensor, Tensor)", _dtw_full_fake)
soft_dtw = _define(
    "soft_dtw", "(Tensor costs, Tensor temperature, Tensor lengths, int bandwidth) -> "
    "(Tensor, Tensor)", lambda c, t, l, bw: _value_marginals_fake(c))
soft_dtw_float = _define(
    "soft_dtw_float", f"(Tensor costs, {_DTW_FLOAT}) -> (Tensor, Tensor)",
    lambda c, t, l, bw: _value_marginals_fake(c))
soft_dtw_with_grads_tp = _define_tp(
    "soft_dtw_with_grads", "Tensor costs", "Tensor? lengths, int? bandwidth",
    "(Tensor, Tensor, Tensor)", _dtw_grads_fake)
soft_dtw_backward_full_tp = _define_tp(
    "soft_dtw_backward_full", "Tensor costs, Tensor grad_alignment",
    "Tensor? lengths, int? bandwidth", "(Tensor, Tensor)", _dtw_full_fake)


def _dtw_setup(ctx, inputs, output):
    costs, temperature, lengths, bandwidth = inputs
    _save(ctx, (costs, output[1]), [temperature], lengths)
    ctx.bandwidth = bandwidth


def _dtw_backward(ctx, grad_value, grad_marginals):
    (costs, marginals), params, lengths = _restore(ctx)
    want_T = ctx.needs_input_grad[1]
    rest = (lengths, ctx.bandwidth)
    grad_costs = _scale_rows(grad_value, marginals)
    grad_T = None
    if grad_value is not None and want_T:
        per_batch = _call(soft_dtw_with_grads, soft_dtw_with_grads_tp, (costs,), params, rest)[2]
        grad_T = _dot_sum(grad_value, per_batch)
    if grad_marginals is not None:
        gc, gt = _call(soft_dtw_backward_full, soft_dtw_backward_full_tp,
                       (costs, grad_marginals.contiguous()), params, rest)
        grad_costs = _add(grad_costs, gc)
        if want_T:
            grad_T = _add(grad_T, gt)
    return grad_costs, grad_T, None, None


soft_dtw.register_autograd(_dtw_backward, setup_context=_dtw_setup)
soft_dtw_float.register_autograd(_dtw_backward, setup_context=_dtw_setup)

# ------------------------------------------------------------------ linear-gap NW

soft_nw_with_grads = _define(
    "soft_nw_with_grads", f"(Tensor scores, {_SW_FLOAT}) -> (Tensor, Tensor, Tensor, Tensor)",
    _sw_grads_fake)
soft_nw_hvp = _define(
    "soft_nw_hvp", f"(Tensor scores, Tensor tangent, {_SW_FLOAT}) -> Tensor",
    lambda s, v, g, t, l: s.new_empty(s.shape))
soft_nw_param_jacobian = _define(
    "soft_nw_param_jacobian", f"(Tensor scores, int param_type, {_SW_FLOAT}) -> Tensor",
    lambda s, p, g, t, l: s.new_empty(s.shape))
soft_nw_backward_full = _define(
    "soft_nw_backward_full",
    f"(Tensor scores, Tensor grad_alignment, {_SW_FLOAT}) -> (Tensor, Tensor, Tensor)",
    _sw_full_fake)
soft_nw = _define(
    "soft_nw", "(Tensor scores, Tensor gap, Tensor temperature, Tensor lengths) -> "
    "(Tensor, Tensor)", lambda s, g, t, l: _value_marginals_fake(s))
soft_nw_float = _define(
    "soft_nw_float", f"(Tensor scores, {_SW_FLOAT}) -> (Tensor, Tensor)",
    lambda s, g, t, l: _value_marginals_fake(s))
soft_nw_with_grads_tp = _define_tp(
    "soft_nw_with_grads", "Tensor scores", "Tensor? lengths",
    "(Tensor, Tensor, Tensor, Tensor)", _sw_grads_fake)
soft_nw_backward_full_tp = _define_tp(
    "soft_nw_backward_full", "Tensor scores, Tensor grad_alignment", "Tensor? lengths",
    "(Tensor, Tensor, Tensor)", _sw_full_fake)

_nw_backward = _first_order_backward(soft_nw_with_grads, soft_nw_with_grads_tp,
                                     soft_nw_backward_full, soft_nw_backward_full_tp)
soft_nw.register_autograd(_nw_backward, setup_context=_first_order_setup)
soft_nw_float.register_autograd(_nw_backward, setup_context=_first_order_setup)

# ------------------------------------------------------------------ affine-gap NW

soft_nw_affine_with_grads = _define(
    "soft_nw_affine_with_grads",
    f"(Tensor scores, {_SWA_FLOAT}) -> (Tensor, Tensor, Tensor, Tensor, Tensor)",
    _swa_grads_fake)
soft_nw_affine_hvp = _define(
    "soft_nw_affine_hvp", f"(Tensor scores, Tensor tangent, {_SWA_FLOAT}) -> Tensor",
    lambda s, v, o, e, t, l: s.new_empty(s.shape))
soft_nw_affine_param_jacobian = _define(
    "soft_nw_affine_param_jacobian", f"(Tensor scores, int param_type, {_SWA_FLOAT}) -> Tensor",
    lambda s, p, o, e, t, l: s.new_empty(s.shape))
soft_nw_affine_backward_full = _define(
    "soft_nw_affine_backward_full",
    f"(Tensor scores, Tensor grad_alignment, {_SWA_FLOAT}) -> (Tensor, Tensor, Tensor, Tensor)",
    _swa_full_fake)
soft_nw_affine = _define(
    "soft_nw_affine", "(Tensor scores, Tensor gap_open, Tensor gap_ext, Tensor temperature, "
    "Tensor lengths) -> (Tensor, Tensor)", lambda s, o, e, t, l: _value_marginals_fake(s))
soft_nw_affine_float = _define(
    "soft_nw_affine_float", f"(Tensor scores, {_SWA_FLOAT}) -> (Tensor, Tensor)",
    lambda s, o, e, t, l: _value_marginals_fake(s))
soft_nw_affine_with_grads_tp = _define_tp(
    "soft_nw_affine_with_grads", "Tensor scores", "Tensor? lengths",
    "(Tensor, Tensor, Tensor, Tensor, Tensor)", _swa_grads_fake)
soft_nw_affine_backward_full_tp = _define_tp(
    "soft_nw_affine_backward_full", "Tensor scores, Tensor grad_alignment", "Tensor? lengths",
    "(Tensor, Tensor, Tensor, Tensor)", _swa_full_fake)

_nwa_backward = _first_order_backward(soft_nw_affine_with_grads, soft_nw_affine_with_grads_tp,
                                      soft_nw_affine_backward_full,
                                      soft_nw_affine_backward_full_tp)
soft_nw_affine.register_autograd(_nwa_backward, setup_context=_first_order_setup)
soft_nw_affine_float.register_autograd(_nwa_backward, setup_context=_first_order_setup)
