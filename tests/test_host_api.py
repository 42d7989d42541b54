"""Host-side behaviour of the drop-in (no GPU needed): the torch.ops.d2p
dispatcher surface, its fake and autocast registrations, the refusal of CPU
tensors, and the Python layer's validation and mask handling, mirroring
/root/reference/d2p/sw.py:80-239,334-421,429-604 and d2p/dtw.py.
"""
import glob
import os
import re
import warnings

import pytest
import torch

import d2p_amd
from d2p_amd import _compile, sw as swmod

REF = "/root/reference"

AUTOGRAD_OPS = {"soft_sw", "soft_sw_float", "sw_forward", "sw_forward_t", "soft_sw_affine",
                "soft_sw_affine_float", "sw_affine_forward", "sw_affine_forward_t", "soft_dtw",
                "soft_dtw_float", "soft_nw", "soft_nw_float", "nw_forward", "nw_forward_t",
                "soft_nw_affine", "soft_nw_affine_float", "nw_affine_forward",
                "nw_affine_forward_t"}


def reference_schemas():
    out = {}
    for path in glob.glob(os.path.join(REF, "src", "*", "registry.cpp")):
        if os.path.basename(os.path.dirname(path)) not in ("sw", "sw_affine", "dtw", "nw",
                                                           "nw_affine"):
            continue
        for s in re.findall(r'm\.def\("([^"]+)"\)', open(path).read()):
            out[s.split("(")[0]] = s
    return out


@pytest.mark.skipif(not os.path.isdir(REF), reason="reference sources absent")
def test_schemas_byte_identical_to_reference():
    ref = reference_schemas()
    assert len(ref) == 60   # 13 linear SW + 14 affine SW + 6 DTW + 13 linear NW + 14 affine NW
    for name, schema in ref.items():
        ours = str(getattr(torch.ops.d2p, name).default._schema)
        assert ours == "d2p::" + schema, (ours, schema)


def test_dispatch_keys():
    for name in _compile.OPS:
        q = f"d2p::{name}"
        assert torch._C._dispatch_has_kernel_for_dispatch_key(q, "CUDA"), name
        assert torch._C._dispatch_has_kernel_for_dispatch_key(q, "AutocastCUDA"), name
        assert (torch._C._dispatch_has_kernel_for_dispatch_key(q, "AutogradCUDA")
                == (name in AUTOGRAD_OPS)), name
    assert d2p_amd._ops._has_cuda_dispatch()


def test_cpu_tensors_fail_loudly():
    x = torch.randn(1, 4, 5)
    for call in (lambda: torch.ops.d2p.soft_sw_float(x, -1.0, 1.0, None),
                 lambda: torch.ops.d2p.soft_sw_affine_hvp(x, x, -2.0, -0.5, 1.0, None),
                 lambda: torch.ops.d2p.soft_dtw_float(x.abs(), 1.0, None, -1),
                 lambda: d2p_amd.soft_sw(x)):
        with pytest.raises(RuntimeError, match="HIP"):
            call()


def _fake_calls(x):
    s, f1, l = x, 1.0, None
    return {
        "soft_sw_float": ((s, -1.0, f1, l), [(2,), (2, 5, 7)]),
        "soft_sw_with_grads": ((s, -1.0, f1, l), [(2,), (2, 5, 7), (2,), (2,)]),
        "soft_sw_hvp": ((s, s, -1.0, f1, l), [(2, 5, 7)]),
        "soft_sw_param_jacobian": ((s, 1, -1.0, f1, l), [(2, 5, 7)]),
        "soft_sw_backward_full": ((s, s, -1.0, f1, l), [(2, 5, 7), (1,), (1,)]),
        "soft_sw_affine_float": ((s, -2.0, -0.5, f1, l), [(2,), (2, 5, 7)]),
        "soft_sw_affine_with_grads": ((s, -2.0, -0.5, f1, l),
                                      [(2,), (2, 5, 7), (2,), (2,), (2,)]),
        "soft_sw_affine_backward_full": ((s, s, -2.0, -0.5, f1, l),
                                         [(2, 5, 7), (1,), (1,), (1,)]),
        "sw_affine_value_grad_params": ((s, -2.0, -0.5, f1, l), [(2,), (2,), (2,)]),
        "soft_nw_affine_float": ((s, -2.0, -0.5, f1, l), [(2,), (2, 5, 7)]),
        "soft_nw_affine_with_grads": ((s, -2.0, -0.5, f1, l),
                                      [(2,), (2, 5, 7), (2,), (2,), (2,)]),
        "soft_nw_affine_backward_full": ((s, s, -2.0, -0.5, f1, l),
                                         [(2, 5, 7), (1,), (1,), (1,)]),
        "nw_affine_value_grad_params": ((s, -2.0, -0.5, f1, l), [(2,), (2,), (2,)]),
        "soft_dtw_float": ((s, f1, l, -1), [(2,), (2, 5, 7)]),
        "soft_dtw_with_grads": ((s, f1, l, -1), [(2,), (2, 5, 7), (2,)]),
        "soft_dtw_backward_full": ((s, s, f1, l, -1), [(2, 5, 7), (1,)]),
    }


def test_fake_kernels_give_output_shapes():
    """FakeTensor calls through the public wrappers reach the d2p_py custom ops (the
    autograd-registered value ops) or the d2p fakes, never the HIP library."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x = torch.empty(2, 5, 7, device="cuda")
        for name, (args, shapes) in _fake_calls(x).items():
            for fn in (getattr(d2p_amd._ops, name),) + (
                    () if name in AUTOGRAD_OPS else (getattr(torch.ops.d2p, name),)):
                out = fn(*args)
                out = [out] if isinstance(out, torch.Tensor) else list(out)
                assert [tuple(o.shape) for o in out] == shapes, name
                assert all(o.device.type == "cuda" and o.dtype == torch.float32 for o in out)


def test_pt2_value_ops_trace_with_autograd():
    """The d2p_py value ops carry an autograd formula that traces under fake tensors:
    value path (scale by marginals) and marginal path (backward_full).  Fake CPU
    tensors: the autograd engine needs a real device context for fake HIP ones."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    from d2p_amd import _pt2_ops as P
    with FakeTensorMode():
        x = torch.empty(2, 5, 7, requires_grad=True)
        lens = torch.empty(2, 2, dtype=torch.int32)
        gap = torch.empty(1, requires_grad=True)
        temp = torch.empty(1, requires_grad=True)
        for value, marg in (P.soft_sw(x, gap, temp, lens), P.soft_sw_float(x, -1.0, 1.0, None),
                            P.soft_sw_affine(x, gap, gap, temp, lens),
                            P.soft_dtw(x, temp, lens, -1), P.soft_dtw_float(x, 1.0, None, -1)):
            gx, = torch.autograd.grad(value.sum() + marg.sum(), x, retain_graph=True)
            assert gx.shape == x.shape


def test_pt2_parameter_gradients_trace_with_tensor_parameters():
    """Tensor gap/temperature reach the backward as saved tensors (the _tp ops), so
    their gradients trace under fake tensors on both paths."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    from d2p_amd import _pt2_ops as P
    with FakeTensorMode():
        x = torch.empty(2, 5, 7, requires_grad=True)
        lens = torch.empty(2, 2, dtype=torch.int32)
        gap = torch.empty(1, requires_grad=True)
        temp = torch.empty(1, requires_grad=True)
        for out, params in ((P.soft_sw(x, gap, temp, lens), (gap, temp)),
                            (P.soft_nw(x, gap, temp, lens), (gap, temp)),
                            (P.soft_sw_affine(x, gap, gap, temp, lens), (gap, temp)),
                            (P.soft_dtw(x, temp, lens, -1), (temp,))):
            value, marg = out
            grads = torch.autograd.grad(value.sum() + marg.sum(), (x, *params))
            assert grads[0].shape == x.shape
            assert all(g.shape == (1,) for g in grads[1:])


def test_pt2_saved_parameters_round_trip():
    """Numbers stay numbers and tensors come back as the saved tensors."""
    from d2p_amd import _pt2_ops as P

    class Ctx:
        def save_for_backward(self, *t):
            self.saved_tensors = t

    ctx = Ctx()
    s, m, g, lens = torch.zeros(1, 2, 2), torch.ones(1, 2, 2), torch.tensor([-3.0]), \
        torch.zeros(1, 2, dtype=torch.int32)
    P._save(ctx, (s, m), [g, 0.25], lens)
    (s2, m2), params, l2 = P._restore(ctx)
    assert s2 is s and m2 is m and params[0] is g and params[1] == 0.25 and l2 is lens
    ctx = Ctx()
    P._save(ctx, (s, m), [-1.0, 2.0], None)
    assert P._restore(ctx)[1:] == ([-1.0, 2.0], None)


def test_use_pt2_ops_predicate():
    from torch._subclasses.fake_tensor import FakeTensorMode
    from d2p_amd._pt2_utils import use_pt2_ops
    real = torch.zeros(2)
    assert not use_pt2_ops(real, 1.0, None)
    with FakeTensorMode():
        fake = torch.zeros(2)
    assert use_pt2_ops(real, fake)

    def f(x):
        return x + (1.0 if use_pt2_ops() else 0.0)

    assert torch.compile(f, backend="eager", fullgraph=True)(real).tolist() == [1.0, 1.0]
    assert f(real).tolist() == [0.0, 0.0]


def test_meta_tensors_route_to_fakes():
    x = torch.empty(3, 4, 6, device="meta")
    v, m = torch.ops.d2p.soft_sw_float(x, -1.0, 1.0, None)
    assert v.shape == (3,) and m.shape == (3, 4, 6)


# ------------------------------------------------------------------ python layer

def test_temperature_validation():
    x = torch.randn(1, 3, 3)
    for bad in (0.0, -1.0, torch.tensor(0.0), torch.tensor([-0.5])):
        with pytest.raises(ValueError, match="temperature must be positive"):
            d2p_amd.soft_sw(x, temperature=bad)
        with pytest.raises(ValueError, match="temperature must be positive"):
            d2p_amd.soft_sw_affine(x, temperature=bad)
        with pytest.raises(ValueError, match="temperature must be positive"):
            d2p_amd.soft_dtw(x.abs(), temperature=bad)
    for cls in (d2p_amd.SoftSW, d2p_amd.SoftSWAffine):
        with pytest.raises(ValueError):
            cls(temperature=0.0)


def test_positive_gap_warns():
    x = torch.randn(1, 3, 3)
    with pytest.warns(UserWarning, match="positive"):
        with pytest.raises(RuntimeError):       # then the CPU tensor is refused
            d2p_amd.soft_sw(x, gap=0.5)
    with warnings.catch_warnings():
        warnings.simplefilter("error", UserWarning)
        with pytest.raises(RuntimeError):
            d2p_amd.soft_sw(x, gap=torch.tensor(0.5))   # tensors do not warn


def test_lengths_and_masks_are_exclusive():
    x = torch.randn(2, 4, 5)
    with pytest.raises(ValueError, match="Cannot specify both"):
        d2p_amd.soft_sw(x, lengths=torch.tensor([[4, 5], [4, 5]], dtype=torch.int32),
                        mask1=torch.ones(2, 4, dtype=torch.bool))


def test_mask_holes_rejected():
    x = torch.randn(2, 4, 5)
    m1 = torch.tensor([[1, 1, 0, 0], [1, 0, 1, 0]], dtype=torch.bool)
    with pytest.raises(ValueError, match=r"mask1 is not prefix-only .* \[1\]"):
        d2p_amd.soft_sw(x, mask1=m1)


def test_masks_to_lengths():
    m1 = torch.tensor([[1, 1, 1, 0], [1, 0, 0, 0], [0, 0, 0, 0]], dtype=torch.bool)
    m2 = torch.tensor([[1, 1, 1, 1, 1], [1, 1, 0, 0, 0], [1, 0, 0, 0, 0]], dtype=torch.bool)
    x = torch.randn(3, 4, 5)
    got = swmod._resolve_lengths(x, None, m1, m2)
    assert got.dtype == torch.int32 and got.tolist() == [[3, 5], [1, 2], [0, 1]]
    got = swmod._resolve_lengths(x, None, m1, None)
    assert got.tolist() == [[3, 5], [1, 5], [0, 5]]


def test_result_aliases_and_modules():
    v, m = torch.randn(2), torch.randn(2, 3, 4)
    r = d2p_amd.SWResult(v, m)
    assert r.score is r.value and r.alignment is r.marginals and r.posteriors is r.marginals
    mod = d2p_amd.SoftSW(gap=-0.5, temperature=0.7, learn_gap=True)
    assert isinstance(mod.gap, torch.nn.Parameter) and not isinstance(mod.temperature,
                                                                       torch.nn.Parameter)
    with pytest.warns(DeprecationWarning):
        mod = d2p_amd.SoftSWAffine(learnable=True)
    assert all(isinstance(getattr(mod, n), torch.nn.Parameter)
               for n in ("gap_open", "gap_ext", "temperature"))


def test_public_names():
    for name in ("soft_sw", "soft_sw_affine", "soft_dtw", "SoftSW", "SoftSWAffine", "SWResult",
                 "soft_sw_hvp", "soft_sw_param_jacobian", "soft_sw_backward_full",
                 "soft_sw_affine_hvp", "soft_sw_affine_param_jacobian",
                 "soft_sw_affine_backward_full", "soft_dtw_hvp", "soft_dtw_param_jacobian",
                 "soft_dtw_backward_full"):
        assert hasattr(d2p_amd, name), name
    from d2p_amd import ops
    for name in ("forward", "forward_t", "value_grad_params", "marginals_backward",
                 "marginals_hvp", "marginals_grad_gap", "marginals_grad_temp"):
        assert hasattr(ops.sw, name)
    for name in ("forward", "forward_t", "value_grad_params", "marginals_backward",
                 "marginals_hvp", "marginals_grad_gap_open", "marginals_grad_gap_ext",
                 "marginals_grad_temp"):
        assert hasattr(ops.sw_affine, name)
