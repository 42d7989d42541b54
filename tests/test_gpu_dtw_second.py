"""GPU parity of the soft-DTW second-order quantities against the CPU oracle:
Hessian-vector products, the Jacobian of the marginals in temperature, and the
marginal-path backward (backward_full and autograd through the marginals).

The oracle restates /root/reference/src/dtw/kernels_cpu.cpp:229-534 and is
bit-identical to a build of those sources.  Tolerance: 1e-4 absolute (the
north-star contract), scaled by max(1, max|expected|) since these are not bounded
by 1.  The temperature Jacobian is ill-conditioned in fp32: it differences
alphas and tangents that grow along the warping path, so half-ulp noise on the
costs alone moves the reference's own Jacobian by up to ~1.3e-4 (600x70, max|J|
0.73).  Its tolerance adds three times that movement, measured on the oracle for
each case (the Jacobian at costs * (1 + 6e-8 N(0,1)) against the unperturbed one).
"""
import numpy as np
import pytest
import torch

import _capi
from _parity import close_entrywise, dot_consistent
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ATOL = 1e-4


def _seeded(seed, shape, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32) * scale


def _close(gpu, ref, what, extra=0.0):
    close_entrywise(gpu, ref, what, extra, ATOL)


CASES = [
    # (seed, B, L1, L2, T, bandwidth)
    (0, 3, 7, 9, 1.0, -1),
    (1, 2, 40, 50, 0.5, -1),
    (2, 2, 100, 120, 1.0, -1),
    (3, 2, 65, 130, 2.0, -1),
    (4, 1, 1, 1, 1.0, -1),
    (5, 2, 120, 100, 1.0, 10),       # Sakoe-Chiba band
    (6, 1, 600, 70, 1.0, -1),        # more stripes than waves in a workgroup
]


@pytest.mark.parametrize("seed,B,L1,L2,T,bw", CASES)
def test_dtw_hvp(cuda, seed, B, L1, L2, T, bw):
    c = _seeded(seed, (B, L1, L2)).abs()
    v = _seeded(seed + 100, (B, L1, L2))
    ref = O.get("oracle").soft_dtw_hvp(c.numpy(), v.numpy(), T, None, bw)
    _close(_capi.dtw_hvp(c.to(cuda), v.to(cuda), None, T, bw), ref, "dtw hvp")


def _jac_allow(k, c, T, lengths=None, bw=-1):
    """3x the reference's own Jacobian movement under half-ulp noise on the costs,
    plus 3x its deviation from two exact zeros: every warping path passes (1,1) and
    (L1,L2), so P = 1 there at every temperature and dP/dT = 0 exactly; what the
    reference's fp32 sweeps leave in those cells measures the rounding they
    accumulate (the temperature tangent (softmin - E[alpha]) / T cancels alphas of
    hundreds down to O(T) in every cell)."""
    rng = np.random.default_rng(0)
    J = k.soft_dtw_param_jacobian(c, T, lengths, bw)
    cp = (c * (1 + 6e-8 * rng.standard_normal(c.shape))).astype(np.float32)
    move = float(np.abs(k.soft_dtw_param_jacobian(cp, T, lengths, bw) - J).max())
    B, L1, L2 = c.shape
    dev = 0.0
    for b in range(B):
        l1, l2 = (L1, L2) if lengths is None else (int(lengths[b][0]), int(lengths[b][1]))
        if l1 > 0 and l2 > 0:
            dev = max(dev, abs(float(J[b, 0, 0])), abs(float(J[b, l1 - 1, l2 - 1])))
    return 3.0 * move + 3.0 * dev


@pytest.mark.parametrize("seed,B,L1,L2,T,bw", CASES)
def test_dtw_param_jacobian(cuda, seed, B, L1, L2, T, bw):
    c = _seeded(seed, (B, L1, L2)).abs()
    k = O.get("oracle")
    ref = k.soft_dtw_param_jacobian(c.numpy(), T, None, bw)
    _close(_capi.dtw_param_jacobian(c.to(cuda), None, T, bw), ref, "dtw dP/dT",
           _jac_allow(k, c.numpy(), T, None, bw))


def test_dtw_second_ragged(cuda):
    B, L1, L2 = 5, 90, 110
    c = _seeded(7, (B, L1, L2)).abs()
    v = _seeded(8, (B, L1, L2))
    lens = np.array([[90, 110], [0, 40], [33, 0], [1, 1], [57, 81]], np.int32)
    lt = torch.from_numpy(lens).to(cuda)
    k = O.get("oracle")
    for bw in (-1, 15):
        _close(_capi.dtw_hvp(c.to(cuda), v.to(cuda), lt, 0.7, bw),
               k.soft_dtw_hvp(c.numpy(), v.numpy(), 0.7, lens, bw), "dtw hvp ragged")
        _close(_capi.dtw_param_jacobian(c.to(cuda), lt, 0.7, bw),
               k.soft_dtw_param_jacobian(c.numpy(), 0.7, lens, bw), "dtw jacobian ragged",
               _jac_allow(k, c.numpy(), 0.7, lens, bw))


def test_dtw_backward_full_and_marginal_autograd(cuda):
    import d2p_amd
    B, L1, L2 = 3, 60, 70
    c = _seeded(9, (B, L1, L2)).abs()
    W = _seeded(10, (B, L1, L2))
    k = O.get("oracle")
    H = k.soft_dtw_hvp(c.numpy(), W.numpy(), 0.8)
    J = k.soft_dtw_param_jacobian(c.numpy(), 0.8)
    dT = (J.astype(np.float64) * W.numpy()).sum()
    gc, gt = d2p_amd.soft_dtw_backward_full(c.to(cuda), W.to(cuda), 0.8, None, None)
    _close(gc, H, "dtw backward_full costs")
    allow = _jac_allow(k, c.numpy(), 0.8)
    tol = (1e-4 * max(1.0, np.abs(J).max()) + allow) * float(np.abs(W.numpy()).sum()) + 1e-4 * abs(dT)
    assert abs(float(gt) - dT) <= tol, (float(gt), dT)
    # autograd through the marginals with a learnable temperature
    x = c.to(cuda).requires_grad_(True)
    T = torch.tensor(0.8, device=cuda, requires_grad=True)
    res = d2p_amd.soft_dtw(x, temperature=T)
    ((res.alignment * W.to(cuda)).sum() + 0.25 * res.cost.sum()).backward()
    _, rm, rgt = k.soft_dtw(c.numpy(), 0.8)
    _close(x.grad, H + 0.25 * rm, "dtw marginal-path grad_costs")
    ref = dT + 0.25 * float(rgt.sum())
    assert abs(float(T.grad) - ref) <= tol + 1e-3 * abs(ref), (float(T.grad), ref)
    # against the GPU's own Jacobian and value-path gradient
    _, _, dt = _capi.dtw_forward_marginals(c.to(cuda), None, 0.8)
    Jg = _capi.dtw_param_jacobian(c.to(cuda), None, 0.8)
    dot_consistent(T.grad, Jg, W, 0.25 * float(dt.double().sum()), "dtw T")
    dot_consistent(gt, Jg, W, 0.0, "dtw backward_full T")
