"""When a call must take the torch.compile-friendly ``d2p_py::`` custom ops.

Two situations hand the operators tensors that carry no data: dynamo tracing a
function, and FakeTensor propagation (``torch._subclasses.FakeTensorMode``, the
meta pass of ``aot_autograd``).  The raw ``torch.ops.d2p`` kernels would read
device memory (and the tensor-parameter ops call ``.item()``), so both are routed
to the custom ops, whose fake kernels only produce shapes.  Same routing rule as
the reference (``d2p/_pt2_utils.py:21-30``).
"""
from __future__ import annotations

import torch
from torch._subclasses.fake_tensor import FakeTensor, is_fake


def _under_dynamo() -> bool:
    """True while dynamo traces the calling frame (torch.compile)."""
    return bool(torch.compiler.is_compiling())


def _carries_no_data(obj: object) -> bool:
    """A FakeTensor, or a wrapper (functional tensor, subclass) around one."""
    return isinstance(obj, torch.Tensor) and (isinstance(obj, FakeTensor) or is_fake(obj))


def use_pt2_ops(*args: object) -> bool:
    """Whether a call with these arguments must go through ``d2p_amd._pt2_ops``."""
    return _under_dynamo() or any(_carries_no_data(a) for a in args)
