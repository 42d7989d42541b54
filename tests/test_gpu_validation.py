"""Boundary behaviour of the HIP operators against the reference's own tests.

Ported from the reference's single-GPU validation and memory-safety tests (the
two-device tests need a second GPU and are left out):
  /root/reference/tests/test_soft_sw_regular.py:376-451 (lengths range, HVP and
  backward_full shape mismatch), :672-691 (zero-storage oversized shapes rejected
  before any allocation); /root/reference/tests/test_soft_sw_affine.py:546-575;
  /root/reference/tests/test_soft_nw.py:505-525,704-745.  The regexes are the
  reference's.  Also the launch property of
  /root/reference/tests/test_soft_sw_regular.py:632-743: the value path launches
  no second-order kernels, the marginal path does (under this library's kernel
  names, read from its launch profile).
"""
import ctypes

import pytest
import torch

import d2p_amd
from _capi import check, lib

pytestmark = pytest.mark.gpu

INT32_MAX = 2 ** 31 - 1


@pytest.mark.parametrize(("lengths", "match"), [
    ([[-1, 5]], r"lengths\[0,0\] must be between 0 and 4"),
    ([[4, 6]], r"lengths\[0,1\] must be between 0 and 5"),
])
@pytest.mark.parametrize("family", ["sw", "swa", "nw", "nwa", "dtw"])
def test_invalid_lengths_raise(cuda, family, lengths, match):
    scores = torch.randn(1, 4, 5, device=cuda)
    ln = torch.tensor(lengths, dtype=torch.int32, device=cuda)
    call = {"sw": lambda: d2p_amd.soft_sw_float(scores, -1.0, 1.0, ln),
            "swa": lambda: d2p_amd.soft_sw_affine_float(scores, -2.0, -0.5, 1.0, ln),
            "nw": lambda: d2p_amd.soft_nw_float(scores, -1.0, 1.0, ln),
            "nwa": lambda: d2p_amd.soft_nw_affine_float(scores, -2.0, -0.5, 1.0, ln),
            "dtw": lambda: d2p_amd.soft_dtw_float(scores.abs(), 1.0, ln, -1)}[family]
    with pytest.raises(RuntimeError, match=match):
        call()


def test_lengths_checked_again_after_any_change(cuda):
    """A lengths tensor checked on the host by the previous call is not copied again
    while it is unchanged; any change is checked again: an in-place write (to the
    tensor or through a view), other memory under the same tensor, another (L1, L2),
    another tensor with the same values."""
    scores = torch.randn(2, 4, 5, device=cuda)
    ln = torch.tensor([[4, 5], [3, 2]], dtype=torch.int32, device=cuda)
    first = d2p_amd.soft_sw_affine_float(scores, -2.0, -0.5, 1.0, ln)
    again = d2p_amd.soft_sw_affine_float(scores, -2.0, -0.5, 1.0, ln)
    assert torch.equal(first[0], again[0]) and torch.equal(first[1], again[1])
    ln[1, 0] = 9                                     # in place
    with pytest.raises(RuntimeError, match=r"lengths\[1,0\] must be between 0 and 4"):
        d2p_amd.soft_sw_affine_float(scores, -2.0, -0.5, 1.0, ln)
    ln[1, 0] = 3
    d2p_amd.soft_sw_affine_float(scores, -2.0, -0.5, 1.0, ln)
    ln[:, 1].fill_(7)                                # through a view
    with pytest.raises(RuntimeError, match=r"lengths\[0,1\] must be between 0 and 5"):
        d2p_amd.soft_sw_affine_float(scores, -2.0, -0.5, 1.0, ln)
    ln[:, 1].fill_(5)
    d2p_amd.soft_sw_affine_float(scores, -2.0, -0.5, 1.0, ln)
    ln.data = torch.tensor([[4, 5], [-1, 2]], dtype=torch.int32, device=cuda)   # new memory
    with pytest.raises(RuntimeError, match=r"lengths\[1,0\] must be between 0 and 4"):
        d2p_amd.soft_sw_affine_float(scores, -2.0, -0.5, 1.0, ln)
    small = torch.randn(2, 3, 5, device=cuda)        # another L1
    ok = torch.tensor([[3, 5], [3, 2]], dtype=torch.int32, device=cuda)
    d2p_amd.soft_sw_affine_float(scores, -2.0, -0.5, 1.0, ok)
    ok[0, 0] = 4
    d2p_amd.soft_sw_affine_float(scores, -2.0, -0.5, 1.0, ok)
    with pytest.raises(RuntimeError, match=r"lengths\[0,0\] must be between 0 and 3"):
        d2p_amd.soft_sw_affine_float(small, -2.0, -0.5, 1.0, ok)
    with torch.inference_mode():                     # no version counter: always checked
        inf = torch.tensor([[4, 5], [5, 2]], dtype=torch.int32, device=cuda)
        with pytest.raises(RuntimeError, match=r"lengths\[1,0\] must be between 0 and 4"):
            d2p_amd.soft_sw_affine_float(scores, -2.0, -0.5, 1.0, inf)


@pytest.mark.parametrize("family", ["sw", "swa", "nw", "nwa"])
def test_hvp_shape_mismatch_raises(cuda, family):
    scores = torch.randn(1, 4, 5, device=cuda)
    tangent = torch.randn(1, 4, 4, device=cuda)
    call = {"sw": lambda: d2p_amd.soft_sw_hvp(scores, tangent, -1.0, 1.0, None),
            "swa": lambda: d2p_amd.soft_sw_affine_hvp(scores, tangent, -2.0, -0.5, 1.0, None),
            "nw": lambda: d2p_amd.soft_nw_hvp(scores, tangent, -1.0, 1.0, None),
            "nwa": lambda: d2p_amd.soft_nw_affine_hvp(scores, tangent, -2.0, -0.5, 1.0,
                                                      None)}[family]
    with pytest.raises(RuntimeError, match=r"scores and tangent must have same shape"):
        call()


def test_dtw_hvp_shape_mismatch_raises(cuda):
    costs = torch.rand(1, 4, 5, device=cuda)
    with pytest.raises(RuntimeError, match=r"tangent must have same shape as costs"):
        d2p_amd.soft_dtw_hvp(costs, torch.rand(1, 4, 4, device=cuda), 1.0, None, -1)
    with pytest.raises(RuntimeError, match=r"grad_alignment must have same shape as costs"):
        d2p_amd.soft_dtw_backward_full(costs, torch.rand(1, 4, 4, device=cuda), 1.0, None, -1)


@pytest.mark.parametrize("family", ["sw", "swa", "nw", "nwa"])
def test_backward_full_rejects_bad_grad_alignment(cuda, family):
    scores = torch.randn(2, 3, 4, device=cuda)
    fn = {"sw": lambda ga: d2p_amd.soft_sw_backward_full(scores, ga, -1.0, 1.0, None),
          "swa": lambda ga: d2p_amd.soft_sw_affine_backward_full(scores, ga, -2.0, -0.5, 1.0,
                                                                 None),
          "nw": lambda ga: d2p_amd.soft_nw_backward_full(scores, ga, -1.0, 1.0, None),
          "nwa": lambda ga: d2p_amd.soft_nw_affine_backward_full(scores, ga, -2.0, -0.5, 1.0,
                                                                 None)}[family]
    with pytest.raises(RuntimeError, match=r"grad_alignment must have same shape as scores"):
        fn(torch.randn(2, 3, 3, device=cuda))
    with pytest.raises(RuntimeError, match=r"grad_alignment must be a CUDA tensor"):
        fn(torch.randn(2, 3, 4))


def test_nw_rank_and_param_type_checks(cuda):
    scores4 = torch.randn(1, 2, 3, 4, device=cuda)
    with pytest.raises(RuntimeError, match=r"scores must be 3D"):
        d2p_amd.soft_nw_hvp(scores4, torch.randn_like(scores4), -1.0, 1.0, None)
    with pytest.raises(RuntimeError, match=r"scores must be 3D"):
        d2p_amd.soft_sw_hvp(scores4, torch.randn_like(scores4), -1.0, 1.0, None)
    scores = torch.randn(2, 4, 5, device=cuda)
    with pytest.raises(RuntimeError, match=r"param_type must be 0 or 1"):
        d2p_amd.soft_nw_param_jacobian(scores, 2, -1.0, 1.0, None)
    with pytest.raises(RuntimeError, match=r"param_type must be 0 or 1"):
        d2p_amd.soft_sw_param_jacobian(scores, 2, -1.0, 1.0, None)
    with pytest.raises(RuntimeError, match=r"param_type must be 0, 1, or 2"):
        d2p_amd.soft_sw_affine_param_jacobian(scores, 3, -2.0, -0.5, 1.0, None)


def test_sw_oversized_dp_table_rejected_before_allocation(cuda):
    """Zero-storage shapes whose table exceeds int32: every SW entry point raises the
    reference's message before any workspace exists."""
    scores = torch.empty((0, 46341, 46341), device=cuda)
    tangent = torch.empty_like(scores)
    lengths = torch.empty((0, 2), dtype=torch.int32, device=cuda)
    gap = torch.tensor([-1.0], device=cuda)
    temperature = torch.tensor([1.0], device=cuda)
    for call in (lambda: d2p_amd.soft_sw(scores, gap, temperature, lengths),
                 lambda: d2p_amd.soft_sw_float(scores, -1.0, 1.0, None),
                 lambda: d2p_amd.soft_sw_with_grads(scores, -1.0, 1.0, None),
                 lambda: d2p_amd.soft_sw_hvp(scores, tangent, -1.0, 1.0, None),
                 lambda: d2p_amd.soft_sw_param_jacobian(scores, 0, -1.0, 1.0, None),
                 lambda: d2p_amd.soft_sw_backward_full(scores, tangent, -1.0, 1.0, None)):
        with pytest.raises(RuntimeError, match="SW CUDA DP table is too large"):
            call()


def test_affine_and_dtw_oversized_rejected_before_allocation(cuda):
    too_wide = INT32_MAX // 3
    with pytest.raises(RuntimeError, match="sw_affine DP table too large"):
        d2p_amd.soft_sw_affine_with_grads(torch.empty((1, 0, too_wide), device=cuda),
                                          -2.0, -0.5, 1.0, None)
    with pytest.raises(RuntimeError, match="DTW alpha table is too large for CUDA kernels"):
        d2p_amd.soft_dtw_float(torch.empty((0, 65536, 65536), device=cuda), 1.0, None, -1)


def _kernels_launched(fn):
    lib().d2p_profile_reset()
    check(lib().d2p_profile_enable(1))
    try:
        fn()
        torch.cuda.synchronize()
    finally:
        check(lib().d2p_profile_enable(0))
    buf = ctypes.create_string_buffer(1 << 16)
    check(lib().d2p_profile_report(buf, len(buf)))
    return {line.split()[0] for line in buf.value.decode().splitlines()}


SECOND_ORDER = ("sw_tangent", "sw_dual", "nw_tangent", "nw_dual", "swa_tangent", "swa_dual",
                "nwa_tangent", "nwa_dual",
                "dtw_tangent", "dtw_dual")


@pytest.mark.parametrize("family", ["sw", "swa", "dtw", "nw", "nwa"])
def test_value_path_launches_no_second_order_kernels(cuda, family):
    s = torch.randn(2, 70, 90, device=cuda)
    if family == "dtw":
        s = s.abs()
    fn = {"sw": lambda x: d2p_amd.soft_sw(x, gap=-1.0, temperature=1.0),
          "swa": lambda x: d2p_amd.soft_sw_affine(x, gap_open=-2.0, gap_ext=-0.5),
          "dtw": lambda x: d2p_amd.soft_dtw(x, temperature=0.5),
          "nw": lambda x: d2p_amd.soft_nw(x, gap=-1.0, temperature=1.0),
          "nwa": lambda x: d2p_amd.soft_nw_affine(x, gap_open=-2.0, gap_ext=-0.5)}[family]

    def value_path():
        x = s.clone().requires_grad_(True)
        fn(x)[0].sum().backward()

    def marginal_path():
        x = s.clone().requires_grad_(True)
        r = fn(x)
        (r[0].sum() + 0 * r[1].sum()).backward()

    names = _kernels_launched(value_path)
    assert "scale_by_batch" in names
    assert not names & set(SECOND_ORDER), names
    names = _kernels_launched(marginal_path)
    prefix = {"sw": "sw", "swa": "swa", "dtw": "dtw", "nw": "nw", "nwa": "nwa"}[family]
    assert {f"{prefix}_tangent", f"{prefix}_dual"} <= names, names


def test_null_lengths_mean_full_lengths(cuda):
    """A NULL lengths pointer in the C ABI is the full (max_L1, max_L2) of every
    element: bit-identical to passing those lengths."""
    from _capi import ptr, stream, sw_forward_marginals
    g = torch.Generator().manual_seed(71)
    B, L1, L2 = 3, 200, 150
    x = torch.randn((B, L1, L2), generator=g).to(cuda)
    want = sw_forward_marginals(x, None, -1.0, 1.0)
    outs = [torch.empty(B, device=cuda), torch.empty(B, L1, L2, device=cuda),
            torch.empty(B, device=cuda), torch.empty(B, device=cuda)]
    n = lib().d2p_sw_workspace_bytes(B, L1, L2)
    ws = torch.empty(n, dtype=torch.uint8, device=cuda)
    check(lib().d2p_sw_forward_marginals(ptr(x), None, B, L1, L2, -1.0, 1.0,
                                         *[ptr(o) for o in outs], ptr(ws), n, stream()))
    torch.cuda.synchronize()
    for a, b in zip(outs, want):
        assert torch.equal(a, b)
