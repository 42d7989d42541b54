"""Parity at the benchmark configurations' own sizes.

The inputs come from the functions bench.py times (make_c3, make_c4, make_c5), so
these tests check exactly the workloads the throughput figures are quoted on.

- C3 (soft_sw_affine, [64,1024,1024], ragged lengths) and C4 (soft_dtw,
  [512,256,256], T=0.1): the public API's value and marginals against the CPU
  oracle (bit-identical to the reference's CPU kernels) at the north-star contract,
  value 1e-5 relative and marginals 1e-4 absolute; the parameter gradients as in the
  smaller tests (tests/_paramgrad.py).
- C5 HVP ([16,4096,4096]): two full elements against the double-precision oracle,
  under the rule of the long-element tests (tests/_parity.check_vs_exact).
- C5 under bf16 autocast: two full elements rounded to bf16 against the same
  elements in fp32.  The values differ by the input rounding, so the check is what
  that rounding must do.  Each value is held to the contract (1e-5 relative)
  against the double-precision oracle.  The soft-SW value is convex in the scores,
  hence for D = s_bf16 - s_fp32 the exact value change is sandwiched by the two
  runs' marginals,
      <P_fp32, D> <= S_bf16 - S_fp32 <= <P_bf16, D>;
  and the marginal change follows
  the Hessian, P_bf16 - P_fp32 = (H_fp32 D + H_bf16 D) / 2 + O(|D|^3) (trapezoid
  rule on the path between the inputs), held to 2e-3 absolute entry-wise.  The
  stated tolerance against fp32 inputs: the value within the rounding bound
  2^-9 * sum(max(P_bf16, P_fp32) |s|) (plus 1e-5 relative per value), the marginals
  within 3e-2 absolute.  The gradient under autocast is the bf16 run's marginals
  rounded to the input's dtype.
"""
import os
import sys

import numpy as np
import pytest
import torch

import _capi
from _paramgrad import check_param_grad
from _parity import check_vs_exact, close_entrywise
from oracle import oracle as O

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402

pytestmark = pytest.mark.gpu

BF16_MARG_ATOL = 2e-3     # marginal change off the Hessian (trapezoid) prediction
BF16_MARG_SHIFT = 3e-2    # marginal change, bf16-rounded against fp32 input scores


def _threads():
    O.set_threads(min(16, os.cpu_count() or 1))


def test_c3_full_size(cuda):
    import d2p_amd
    _threads()
    cfg = bench.make_c3()
    s, lens = cfg["inputs"]["scores"], cfg["inputs"]["lengths"]
    go, ge, T = -11.0, -1.0, 0.5
    x = s.to(cuda).requires_grad_(True)
    r = d2p_amd.soft_sw_affine(x, gap_open=go, gap_ext=ge, temperature=T, lengths=lens.to(cuda))
    r.value.sum().backward()
    k = O.get("oracle")
    rp, rm, ro, re, rt = k.soft_sw_affine(s.numpy(), go, ge, T, lengths=lens.numpy())
    np.testing.assert_allclose(r.value.detach().cpu().numpy(), rp, rtol=1e-5, atol=1e-6)
    e = close_entrywise(r.marginals, rm, "C3 marginals", atol=0.0, extra=1e-4)
    assert torch.equal(x.grad, r.marginals.detach())
    print(f"C3 max |marginals - oracle| = {e:.2e}")
    part, marg, g_o, g_e, g_t = [t.cpu().numpy() for t in
                                 _capi.swa_forward_marginals(s.to(cuda), lens, go, ge, T)]
    assert np.array_equal(marg, r.marginals.detach().cpu().numpy())
    ln = lens.numpy()
    exact = lambda: k.param_grads64("swa", s.numpy(), ln, go, ge, T)
    check_param_grad(g_o, ro, lambda: exact()[:, 0])
    check_param_grad(g_e, re, lambda: exact()[:, 1])
    check_param_grad(g_t, rt, lambda: exact()[:, 2], rtol=1e-3,
                     atol=2e-5 * (np.abs(rp).max() + 1.0) / T)
    for b, (l1, l2) in enumerate(ln):
        assert not marg[b, l1:, :].any() and not marg[b, :, l2:].any()


def test_c4_full_size(cuda):
    import d2p_amd
    _threads()
    c = bench.make_c4()["inputs"]["costs"]
    T = 0.1
    x = c.to(cuda).requires_grad_(True)
    r = d2p_amd.soft_dtw(x, temperature=T)
    r.cost.sum().backward()
    k = O.get("oracle")
    rv, rm, rt = k.soft_dtw(c.numpy(), T)
    np.testing.assert_allclose(r.cost.detach().cpu().numpy(), rv, rtol=1e-5, atol=1e-6)
    e = close_entrywise(r.alignment, rm, "C4 marginals", atol=0.0, extra=1e-4)
    assert torch.equal(x.grad, r.alignment.detach())
    print(f"C4 max |marginals - oracle| = {e:.2e}")
    _, _, gt = _capi.dtw_forward_marginals(c.to(cuda), None, T)
    check_param_grad(gt.cpu().numpy(), rt, lambda: k.param_grads64("dtw", c.numpy(), None, T)[:, 0],
                     rtol=1e-3, atol=2e-5 * (np.abs(rv).max() + 1.0) / T)


@pytest.fixture(scope="module")
def c5_two():
    """The first two elements of the C5 inputs (scores and the HVP direction)."""
    cfg = bench.make_c5(hvp=True)
    s, V = cfg["inputs"]["scores"][:2].clone(), cfg["inputs"]["V"][:2].clone()
    del cfg
    return s, V


def test_c5_hvp_two_full_elements(cuda, c5_two):
    _threads()
    s, V = c5_two
    k32, k64 = O.get("oracle"), O.get("oracle64")
    s64, v64 = s.numpy().astype(np.float64), V.numpy().astype(np.float64)
    gpu = _capi.sw_hvp(s.to(cuda), V.to(cuda), None, -1.0, 1.0)
    e_gpu, e_ref = check_vs_exact(gpu, k64.soft_sw_hvp(s64, v64, -1.0, 1.0),
                                  k32.soft_sw_hvp(s.numpy(), V.numpy(), -1.0, 1.0),
                                  "C5 hvp 2x4096^2")
    print(f"C5 HVP max |gpu - exact| = {e_gpu:.2e} (fp32 reference {e_ref:.2e})")


def test_c5_bf16_autocast_two_full_elements(cuda, c5_two):
    import d2p_amd
    s, _ = c5_two
    s16 = s.to(cuda).to(torch.bfloat16)
    s32 = s.to(cuda)
    x16 = s16.clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        r16 = d2p_amd.soft_sw(x16, gap=-1.0, temperature=1.0)
        assert r16.value.dtype == torch.float32 and r16.marginals.dtype == torch.float32
        r16.value.sum().backward()
    assert x16.grad.dtype == torch.bfloat16
    assert torch.equal(x16.grad, r16.marginals.detach().to(torch.bfloat16))
    x32 = s32.clone().requires_grad_(True)
    r32 = d2p_amd.soft_sw(x32, gap=-1.0, temperature=1.0)
    r32.value.sum().backward()
    # the bf16 run is the fp32 path on the rounded input, bit for bit
    r16f = d2p_amd.soft_sw(s16.float(), gap=-1.0, temperature=1.0)
    assert torch.equal(r16f.value, r16.value) and torch.equal(r16f.marginals, r16.marginals)
    # each value against the double-precision oracle, at the contract
    _threads()
    k64 = O.get("oracle64")
    x16_64 = s16.float().cpu().numpy().astype(np.float64)
    e16, m16 = [torch.from_numpy(a) for a in k64.soft_sw(x16_64, -1.0, 1.0)[:2]]
    e32, m32 = [torch.from_numpy(a) for a in k64.soft_sw(s.numpy().astype(np.float64), -1.0, 1.0)[:2]]
    for got, want in ((r16.value, e16), (r32.value, e32)):
        err = (got.detach().cpu().double() - want).abs()
        assert torch.all(err <= 1e-5 * want.abs()), (got, want)
    P16, P32 = r16.marginals.detach().double(), r32.marginals.detach().double()
    k32 = O.get("oracle")
    for got, want, x in ((P16, m16, s16.float().cpu().numpy()), (P32, m32, s.numpy())):
        # 4096^2 marginals in fp32 sit up to a few 1e-4 from the exact ones; the
        # fp32 reference's own error on the same input sets the bound
        e_gpu = float((got.cpu() - want).abs().max())
        e_ref = float((torch.from_numpy(k32.soft_sw(x, -1.0, 1.0)[1]).double() - want).abs().max())
        print(f"marginals |gpu - exact| {e_gpu:.2e}, fp32 reference {e_ref:.2e}")
        assert e_gpu <= max(1e-4, 2.0 * e_ref), (e_gpu, e_ref)
    # the exact value change sandwiched by the two runs' marginals; the marginals'
    # own errors move each bound by at most sum |P_gpu - P_exact| |D|
    D = (s16.float() - s32).double()
    dS = e16 - e32
    lo, hi = (P32 * D).sum(dim=(1, 2)).cpu(), (P16 * D).sum(dim=(1, 2)).cpu()
    Dc = D.abs().cpu()
    slack = torch.maximum(((P32.cpu() - m32).abs() * Dc).sum(dim=(1, 2)),
                          ((P16.cpu() - m16).abs() * Dc).sum(dim=(1, 2)))
    # the stated tolerance of bf16 autocast against fp32 inputs: the value moves by
    # at most the rounding of the scores under the marginals (|D| <= 2^-9 |s|,
    # and S16 - S32 lies between <P32, D> and <P16, D>), plus the contract on each
    # value; the marginals move by at most BF16_MARG_SHIFT absolute
    dv = (r16.value - r32.value).detach().double().cpu()
    bound = 2.0 ** -9 * (torch.maximum(P16, P32) * s32.double().abs()).sum(dim=(1, 2)).cpu() \
        + 1e-5 * (e16.abs() + e32.abs())
    assert torch.all(dv.abs() <= bound), (dv, bound)
    rel = float((dv.abs() / e32.abs()).max())
    H = 0.5 * (_capi.sw_hvp(s32, D.float(), None, -1.0, 1.0).double()
               + _capi.sw_hvp(s16.float(), D.float(), None, -1.0, 1.0).double())
    e = float((P16 - P32 - H).abs().max())
    shift = float((P16 - P32).abs().max())
    print(f"bf16 autocast: exact value change {dS.tolist()} in [{lo.tolist()}, {hi.tolist()}] "
          f"(slack {slack.tolist()}); value moves {rel:.2e} relative; max marginal change "
          f"{shift:.2e}, off the Hessian prediction by {e:.2e}", flush=True)
    assert torch.all(dS >= lo - slack) and torch.all(dS <= hi + slack), (dS, lo, hi)
    assert e <= BF16_MARG_ATOL, (e, shift)
    assert shift <= BF16_MARG_SHIFT, shift
