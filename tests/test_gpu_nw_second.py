"""GPU parity of the soft Needleman-Wunsch second-order quantities against the CPU
oracle: Hessian-vector products, Jacobians of the marginals in gap and temperature,
the marginal-path backward (backward_full) and autograd through the alignment.

The oracle restates /root/reference/src/nw/kernels_cpu.cpp (nw_hvp_cpu,
nw_param_grad_cpu) and is bit-identical to a build of those sources.  The terminal
beta is the constant 1, so, unlike Smith-Waterman, no dS/dtheta enters the sweeps.

Tolerances: 1e-4 absolute scaled by max(1, max|ref|).
The Jacobians are compared with the double-precision oracle (liboracle64.so) and
allowed, beyond that, 3x the fp32 reference's own distance from it: the GPU pivots
its weighted means on the largest candidate and the reference does not, so along
long alignments the two fp32 evaluations drift apart by about the reference's own
rounding error.
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


@pytest.fixture
def parts(monkeypatch):
    def force(n):
        monkeypatch.setenv("D2P_AMD_SPLIT", str(n))
    return force


def _close(gpu, ref, what, extra=0.0):
    close_entrywise(gpu, ref, what, extra, ATOL)


def _jacobian_ref(s, ptype, gap, T, lengths=None):
    """The double-precision Jacobian and 3x the fp32 reference's distance from it."""
    J64 = O.get("oracle64").soft_nw_param_jacobian(s.astype(np.float64), ptype, gap, T, lengths)
    J32 = O.get("oracle").soft_nw_param_jacobian(s, ptype, gap, T, lengths)
    return J64, 3.0 * float(np.abs(J32 - J64).max(initial=0.0))


CASES = [
    # (seed, B, L1, L2, gap, T)
    (0, 3, 7, 9, -1.0, 1.0),
    (1, 1, 1, 1, -1.0, 1.0),
    (2, 2, 40, 50, -1.0, 0.5),
    (3, 2, 100, 120, -0.5, 1.0),
    (4, 2, 65, 130, -1.0, 2.0),
    (5, 2, 1, 130, -0.5, 1.0),
    (6, 2, 130, 1, -0.5, 1.0),
    (7, 1, 600, 70, -1.0, 1.0),      # more stripes than waves in a workgroup
    (8, 2, 64, 64, 0.3, 1.0),        # positive gap
]


@pytest.mark.parametrize("seed,B,L1,L2,gap,T", CASES)
def test_nw_hvp(cuda, seed, B, L1, L2, gap, T):
    s = _seeded(seed, (B, L1, L2))
    v = _seeded(seed + 100, (B, L1, L2))
    ref = O.get("oracle").soft_nw_hvp(s.numpy(), v.numpy(), gap, T)
    gpu = _capi.nw_hvp(s.to(cuda), v.to(cuda), None, gap, T)
    _close(gpu, ref, "hvp")


@pytest.mark.parametrize("seed,B,L1,L2,gap,T", CASES)
@pytest.mark.parametrize("ptype", [0, 1])
def test_nw_param_jacobian(cuda, seed, B, L1, L2, gap, T, ptype):
    s = _seeded(seed, (B, L1, L2))
    ref, allow = _jacobian_ref(s.numpy(), ptype, gap, T)
    gpu = _capi.nw_param_jacobian(s.to(cuda), ptype, None, gap, T)
    _close(gpu, ref, f"dP/d{'gap' if ptype == 0 else 'T'}", allow)


def test_nw_second_ragged(cuda):
    B, L1, L2 = 6, 90, 110
    s = _seeded(17, (B, L1, L2))
    v = _seeded(18, (B, L1, L2))
    lens = np.array([[90, 110], [0, 40], [33, 0], [1, 1], [57, 81], [0, 0]], np.int32)
    lt = torch.from_numpy(lens).to(cuda)
    h = _capi.nw_hvp(s.to(cuda), v.to(cuda), lt, -1.0, 0.7)
    _close(h, O.get("oracle").soft_nw_hvp(s.numpy(), v.numpy(), -1.0, 0.7, lens), "hvp ragged")
    for p in (0, 1):
        ref, allow = _jacobian_ref(s.numpy(), p, -1.0, 0.7, lens)
        J = _capi.nw_param_jacobian(s.to(cuda), p, lt, -1.0, 0.7)
        _close(J, ref, f"jacobian {p} ragged", allow)
        Jn = J.cpu().numpy()
        for b, (l1, l2) in enumerate(lens):
            assert np.all(Jn[b, l1:, :] == 0.0) and np.all(Jn[b, :, l2:] == 0.0)


@pytest.mark.parametrize("n", [2, 3])
def test_nw_second_split_parts(cuda, parts, n):
    parts(n)
    s = _seeded(40 + n, (2, 700, 90))
    v = _seeded(50 + n, (2, 700, 90))
    _close(_capi.nw_hvp(s.to(cuda), v.to(cuda), None, -1.0, 1.0),
           O.get("oracle").soft_nw_hvp(s.numpy(), v.numpy(), -1.0, 1.0), "hvp split")
    for p in (0, 1):
        ref, allow = _jacobian_ref(s.numpy(), p, -1.0, 1.0)
        _close(_capi.nw_param_jacobian(s.to(cuda), p, None, -1.0, 1.0), ref,
               f"jacobian {p} split", allow)


def test_nw_backward_full(cuda):
    """grad_scores = H ga; per-element <ga, dP/dgap>, <ga, dP/dT> (summed by the op)."""
    B, L1, L2 = 3, 80, 96
    s = _seeded(9, (B, L1, L2))
    ga = _seeded(10, (B, L1, L2))
    gs, gg, gt = _capi.nw_backward_full(s.to(cuda), ga.to(cuda), None, -1.0, 1.0)
    _close(gs, O.get("oracle").soft_nw_hvp(s.numpy(), ga.numpy(), -1.0, 1.0),
           "backward_full scores")
    for p, g in ((0, gg), (1, gt)):
        J, allow = _jacobian_ref(s.numpy(), p, -1.0, 1.0)
        ref = (J * ga.numpy()).sum(axis=(1, 2))
        per = ATOL * max(1.0, np.abs(J).max()) + allow
        tol = per * np.abs(ga.numpy()).sum(axis=(1, 2))
        assert np.all(np.abs(g.cpu().numpy() - ref) <= tol), (p, g.cpu().numpy(), ref, tol)


def test_nw_ops_match_oracle(cuda):
    """torch.ops.d2p NW second-order ops route to the same kernels."""
    import d2p_amd
    from d2p_amd import ops
    s = _seeded(21, (2, 50, 60))
    v = _seeded(22, (2, 50, 60))
    ref_h = O.get("oracle").soft_nw_hvp(s.numpy(), v.numpy(), -1.0, 1.0)
    _close(d2p_amd.soft_nw_hvp(s.to(cuda), v.to(cuda), -1.0, 1.0, None), ref_h, "soft_nw_hvp")
    _close(ops.nw_marginals_hvp(s.to(cuda), v.to(cuda), -1.0, 1.0, None), ref_h,
           "nw_marginals_hvp")
    for p, fn in ((0, ops.nw_marginals_grad_gap), (1, ops.nw_marginals_grad_temp)):
        ref, allow = _jacobian_ref(s.numpy(), p, -1.0, 1.0)
        _close(d2p_amd.soft_nw_param_jacobian(s.to(cuda), p, -1.0, 1.0, None), ref,
               "soft_nw_param_jacobian", allow)
        _close(fn(s.to(cuda), -1.0, 1.0, None), ref, "nw_marginals_grad", allow)
    gs, gg, gt = d2p_amd.soft_nw_backward_full(s.to(cuda), v.to(cuda), -1.0, 1.0, None)
    assert gg.shape == (1,) and gt.shape == (1,)
    _close(gs, ref_h, "soft_nw_backward_full")
    gs2, gg2, gt2 = ops.nw_marginals_backward(s.to(cuda), v.to(cuda), -1.0, 1.0, None)
    torch.testing.assert_close(gs2, gs, rtol=0, atol=0)


def test_nw_marginal_path_autograd(cuda):
    """loss = <W, alignment> + 0.5 sum(score): d loss / d scores = H W + 0.5 P,
    d loss / d gap = <W, dP/dgap> + 0.5 dS/dgap (and the same for T)."""
    import d2p_amd
    s = _seeded(31, (2, 40, 45))
    W = _seeded(32, (2, 40, 45))
    x = s.to(cuda).requires_grad_(True)
    gap = torch.tensor([-1.0], device=cuda, requires_grad=True)
    T = torch.tensor([0.8], device=cuda, requires_grad=True)
    res = d2p_amd.soft_nw(x, gap=gap, temperature=T)
    loss = (res.alignment * W.to(cuda)).sum() + 0.5 * res.score.sum()
    loss.backward()
    k = O.get("oracle")
    _, rm, _, _ = k.soft_nw(s.numpy(), -1.0, 0.8)
    _, _, eg, et = O.get("oracle64").soft_nw(s.numpy().astype(np.float64), -1.0, 0.8)
    expect = k.soft_nw_hvp(s.numpy(), W.numpy(), -1.0, 0.8) + 0.5 * rm
    _close(x.grad, expect, "marginal-path grad_scores")
    for p, g, rv in ((0, gap, eg), (1, T, et)):
        J, allow = _jacobian_ref(s.numpy(), p, -1.0, 0.8)
        ref = float((J * W.numpy()).sum() + 0.5 * rv.sum())
        tol = (ATOL * max(1.0, np.abs(J).max()) + allow) * float(np.abs(W.numpy()).sum()) \
            + 1e-3 * abs(ref)
        assert abs(float(g.grad) - ref) <= tol, (p, float(g.grad), ref, tol)
    # the same gradients against the GPU's own Jacobians and value-path gradients
    _, _, dg, dt = _capi.nw_forward_marginals(s.to(cuda), None, -1.0, 0.8)
    for p, g, dv in ((0, gap, dg), (1, T, dt)):
        Jg = _capi.nw_param_jacobian(s.to(cuda), p, None, -1.0, 0.8)
        dot_consistent(g.grad, Jg, W, 0.5 * float(dv.double().sum()), f"nw param {p}")
    # float parameters: the scores gradient alone, equal to the tensor-parameter one
    x2 = s.to(cuda).requires_grad_(True)
    r2 = d2p_amd.soft_nw(x2, gap=-1.0, temperature=0.8)
    ((r2.alignment * W.to(cuda)).sum() + 0.5 * r2.score.sum()).backward()
    torch.testing.assert_close(x2.grad, x.grad, rtol=0, atol=0)
