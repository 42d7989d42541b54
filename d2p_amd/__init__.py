"""d2p_amd -- MI355X (gfx950) soft-alignment dynamic programming for PyTorch-ROCm.

Drop-in for the soft Smith-Waterman (linear and affine gap), soft-DTW and soft
Needleman-Wunsch (linear and affine gap) part of orikata-bio/d2p, first and second
order: the same Python API (``soft_sw``, ``soft_sw_affine``, ``soft_dtw``,
``soft_nw``, ``soft_nw_affine``, the ``nn.Module`` wrappers, ``ops``, the legacy flat
names) and the same ``torch.ops.d2p`` operator schemas, computed by hand-written HIP
kernels for CDNA4.  Tensors must live on the HIP device.
"""
from . import _ops
from . import _compile  # noqa: F401  (fake/meta and autocast registrations)

from .sw import soft_sw, soft_sw_affine, SWResult, SoftSW, SoftSWAffine
from .dtw import soft_dtw, soft_dtw_sqeuclidean, DTWResult, SoftDTW
from .nw import soft_nw, soft_nw_affine, NWResult, SoftNW, SoftNWAffine
from . import ops

# legacy flat names (reference d2p/__init__.py:120-139)
soft_sw_float = _ops.soft_sw_float
soft_sw_with_grads = _ops.soft_sw_with_grads
soft_sw_hvp = _ops.soft_sw_hvp
soft_sw_param_jacobian = _ops.soft_sw_param_jacobian
soft_sw_backward_full = _ops.soft_sw_backward_full
soft_sw_affine_float = _ops.soft_sw_affine_float
soft_sw_affine_with_grads = _ops.soft_sw_affine_with_grads
soft_sw_affine_hvp = _ops.soft_sw_affine_hvp
soft_sw_affine_param_jacobian = _ops.soft_sw_affine_param_jacobian
soft_sw_affine_backward_full = _ops.soft_sw_affine_backward_full
soft_dtw_float = _ops.soft_dtw_float
soft_dtw_with_grads = _ops.soft_dtw_with_grads
soft_dtw_hvp = _ops.soft_dtw_hvp
soft_dtw_param_jacobian = _ops.soft_dtw_param_jacobian
soft_dtw_backward_full = _ops.soft_dtw_backward_full
soft_nw_float = _ops.soft_nw_float
soft_nw_with_grads = _ops.soft_nw_with_grads
soft_nw_forward = _ops.soft_nw_float
soft_nw_hvp = _ops.soft_nw_hvp
soft_nw_param_jacobian = _ops.soft_nw_param_jacobian
soft_nw_backward_full = _ops.soft_nw_backward_full
soft_nw_affine_float = _ops.soft_nw_affine_float
soft_nw_affine_with_grads = _ops.soft_nw_affine_with_grads
soft_nw_affine_hvp = _ops.soft_nw_affine_hvp
soft_nw_affine_param_jacobian = _ops.soft_nw_affine_param_jacobian
soft_nw_affine_backward_full = _ops.soft_nw_affine_backward_full

__all__ = [
    "soft_sw", "soft_sw_affine", "SWResult", "SoftSW", "SoftSWAffine",
    "soft_dtw", "soft_dtw_sqeuclidean", "DTWResult", "SoftDTW", "ops",
    "soft_sw_float", "soft_sw_with_grads", "soft_sw_hvp", "soft_sw_param_jacobian",
    "soft_sw_backward_full",
    "soft_sw_affine_float", "soft_sw_affine_with_grads", "soft_sw_affine_hvp",
    "soft_sw_affine_param_jacobian", "soft_sw_affine_backward_full",
    "soft_dtw_float", "soft_dtw_with_grads", "soft_dtw_hvp", "soft_dtw_param_jacobian",
    "soft_dtw_backward_full",
    "soft_nw", "NWResult", "SoftNW", "soft_nw_float", "soft_nw_with_grads", "soft_nw_forward",
    "soft_nw_hvp", "soft_nw_param_jacobian", "soft_nw_backward_full",
    "soft_nw_affine", "SoftNWAffine", "soft_nw_affine_float", "soft_nw_affine_with_grads",
    "soft_nw_affine_hvp", "soft_nw_affine_param_jacobian", "soft_nw_affine_backward_full",
]
