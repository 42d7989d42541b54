"""Operator access for d2p_amd: loads the in-tree HIP operator library.

Mirrors the reference's ``d2p/_ops.py`` (loader ``:43-97``, CUDA-dispatch probe
``:36-40``, ``_wrap`` ``:153-167``): the library registers the ``d2p``
dispatcher namespace, and every public op here is a thin wrapper that routes
eager calls to ``torch.ops.d2p.<name>`` and compile-time / fake-tensor calls to
the ``d2p_py::`` custom ops in ``_pt2_ops``.

There is no CPU fallback.  If the native library is missing the import fails,
and CPU tensors are rejected by the operator layer itself.
"""
from __future__ import annotations

import os

import torch

from ._pt2_utils import use_pt2_ops

_HERE = os.path.dirname(os.path.abspath(__file__))
OP_LIBRARY = os.path.join(_HERE, "_C.so")
KERNEL_LIBRARY = os.path.join(_HERE, "libd2p_amd.so")

_extension_loaded = False
_cuda_dispatch_available = False


def _has_cuda_dispatch() -> bool:
    try:
        return torch._C._dispatch_has_kernel_for_dispatch_key("d2p::soft_sw_float", "CUDA")
    except (AttributeError, RuntimeError):
        return False


def _load_extension() -> None:
    global _extension_loaded, _cuda_dispatch_available
    if _extension_loaded:
        return
    if not os.path.exists(OP_LIBRARY):
        raise ImportError(
            f"d2p_amd native library not built ({OP_LIBRARY} missing). Build it in-tree with "
            "`python -m d2p_amd._build` (needs hipcc for gfx950).")
    try:
        torch.ops.load_library(OP_LIBRARY)
    except OSError as exc:
        if "undefined symbol" in str(exc):
            raise ImportError(
                f"d2p_amd's operator library does not match the installed torch "
                f"{torch.__version__}; rebuild it with `python -m d2p_amd._build`.\n"
                f"Original error: {exc}") from exc
        raise
    _extension_loaded = True
    _cuda_dispatch_available = _has_cuda_dispatch()


def loaded_libraries() -> list:
    """Paths of the native libraries this package loaded."""
    return [OP_LIBRARY, KERNEL_LIBRARY] if _extension_loaded else []


_load_extension()

d2p = torch.ops.d2p

_pt2_ops_mod = None


def _get_pt2_ops():
    global _pt2_ops_mod
    if _pt2_ops_mod is None:
        from . import _pt2_ops
        _pt2_ops_mod = _pt2_ops
    return _pt2_ops_mod


def _wrap(name: str):
    raw = getattr(torch.ops.d2p, name)

    def wrapped(*args, **kwargs):
        if use_pt2_ops(*args, *kwargs.values()):
            pt2 = _get_pt2_ops()
            if hasattr(pt2, name):
                return getattr(pt2, name)(*args, **kwargs)
        return raw(*args, **kwargs)

    wrapped.__name__ = name
    wrapped.__qualname__ = name
    wrapped.__doc__ = f"Calls ``torch.ops.d2p.{name}`` ({raw.default._schema})."
    return wrapped


# linear-gap Smith-Waterman
soft_sw = _wrap("soft_sw")
soft_sw_float = _wrap("soft_sw_float")
soft_sw_with_grads = _wrap("soft_sw_with_grads")
soft_sw_hvp = _wrap("soft_sw_hvp")
soft_sw_param_jacobian = _wrap("soft_sw_param_jacobian")
soft_sw_backward_full = _wrap("soft_sw_backward_full")
sw_forward = _wrap("sw_forward")
sw_forward_t = _wrap("sw_forward_t")
sw_value_grad_params = _wrap("sw_value_grad_params")
sw_marginals_backward = _wrap("sw_marginals_backward")
sw_marginals_hvp = _wrap("sw_marginals_hvp")
sw_marginals_grad_gap = _wrap("sw_marginals_grad_gap")
sw_marginals_grad_temp = _wrap("sw_marginals_grad_temp")

# affine-gap Smith-Waterman
soft_sw_affine = _wrap("soft_sw_affine")
soft_sw_affine_float = _wrap("soft_sw_affine_float")
soft_sw_affine_with_grads = _wrap("soft_sw_affine_with_grads")
soft_sw_affine_hvp = _wrap("soft_sw_affine_hvp")
soft_sw_affine_param_jacobian = _wrap("soft_sw_affine_param_jacobian")
soft_sw_affine_backward_full = _wrap("soft_sw_affine_backward_full")
sw_affine_forward = _wrap("sw_affine_forward")
sw_affine_forward_t = _wrap("sw_affine_forward_t")
sw_affine_value_grad_params = _wrap("sw_affine_value_grad_params")
sw_affine_marginals_backward = _wrap("sw_affine_marginals_backward")
sw_affine_marginals_hvp = _wrap("sw_affine_marginals_hvp")
sw_affine_marginals_grad_gap_open = _wrap("sw_affine_marginals_grad_gap_open")
sw_affine_marginals_grad_gap_ext = _wrap("sw_affine_marginals_grad_gap_ext")
sw_affine_marginals_grad_temp = _wrap("sw_affine_marginals_grad_temp")

# linear-gap Needleman-Wunsch (first order)
soft_nw = _wrap("soft_nw")
soft_nw_float = _wrap("soft_nw_float")
soft_nw_with_grads = _wrap("soft_nw_with_grads")
nw_forward = _wrap("nw_forward")
nw_forward_t = _wrap("nw_forward_t")
nw_value_grad_params = _wrap("nw_value_grad_params")
soft_nw_hvp = _wrap("soft_nw_hvp")
soft_nw_param_jacobian = _wrap("soft_nw_param_jacobian")
soft_nw_backward_full = _wrap("soft_nw_backward_full")
nw_marginals_backward = _wrap("nw_marginals_backward")
nw_marginals_hvp = _wrap("nw_marginals_hvp")
nw_marginals_grad_gap = _wrap("nw_marginals_grad_gap")
nw_marginals_grad_temp = _wrap("nw_marginals_grad_temp")

# affine-gap Needleman-Wunsch
soft_nw_affine = _wrap("soft_nw_affine")
soft_nw_affine_float = _wrap("soft_nw_affine_float")
soft_nw_affine_with_grads = _wrap("soft_nw_affine_with_grads")
soft_nw_affine_hvp = _wrap("soft_nw_affine_hvp")
soft_nw_affine_param_jacobian = _wrap("soft_nw_affine_param_jacobian")
soft_nw_affine_backward_full = _wrap("soft_nw_affine_backward_full")
nw_affine_forward = _wrap("nw_affine_forward")
nw_affine_forward_t = _wrap("nw_affine_forward_t")
nw_affine_value_grad_params = _wrap("nw_affine_value_grad_params")
nw_affine_marginals_backward = _wrap("nw_affine_marginals_backward")
nw_affine_marginals_hvp = _wrap("nw_affine_marginals_hvp")
nw_affine_marginals_grad_gap_open = _wrap("nw_affine_marginals_grad_gap_open")
nw_affine_marginals_grad_gap_ext = _wrap("nw_affine_marginals_grad_gap_ext")
nw_affine_marginals_grad_temp = _wrap("nw_affine_marginals_grad_temp")

# soft DTW
soft_dtw = _wrap("soft_dtw")
soft_dtw_float = _wrap("soft_dtw_float")
soft_dtw_with_grads = _wrap("soft_dtw_with_grads")
soft_dtw_hvp = _wrap("soft_dtw_hvp")
soft_dtw_param_jacobian = _wrap("soft_dtw_param_jacobian")
soft_dtw_backward_full = _wrap("soft_dtw_backward_full")
