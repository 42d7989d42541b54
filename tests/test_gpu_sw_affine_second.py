"""GPU parity of the affine-gap second-order quantities against the CPU oracle:
Hessian-vector products, Jacobians of the marginals in gap_open, gap_ext and
temperature, and the marginal-path backward (backward_full).

The oracle restates /root/reference/src/sw_affine/kernels_cpu.cpp:362-921 and is
bit-identical to a build of those sources.  Tolerance: 1e-4 absolute on HVP
entries, scaled by max(1, max|H|) since a Hessian-vector
product against an N(0,1) direction is not bounded by 1; the same for Jacobians.

As for the linear gap, the Jacobian sweep starts its second channel from
beta_init * (U - dS/dtheta) / T with dS/dtheta from the marginal backward, which
the reference sums sequentially in fp32.  The expected Jacobian is therefore the
reference's sweep driven by dS/dtheta summed in double from the reference's own
per-cell terms (oracle.param_grads64), and the tolerance adds the conditioning
allowance 2e-6 * |dS/dtheta| / T * max(P): any two fp32 evaluations of dS/dtheta
differ by ~1e-6 relative and every Jacobian entry moves by that error times P / T;
plus 3x the reference's own movement under half-ulp noise on the scores (the GPU's
alphas and partition round differently).
"""
import numpy as np
import pytest
import torch

import _capi
from _parity import close_entrywise, dot_consistent
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ATOL = 1e-4
NAMES = ("open", "ext", "T")


def _seeded(seed, shape, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32) * scale


def _jacobian_ref(k, s, ptype, go, ge, T, lengths=None):
    """The reference's Jacobian sweep driven by the double-summed dS/dtheta, and the
    conditioning allowance 2e-6 * |dS/dtheta| / T * max(P) per element."""
    alpha, part = k.swa_forward(s, lengths, go, ge, T)
    post, _, _, _ = k.swa_backward(alpha, s, part, lengths, go, ge, T)
    dS = k.param_grads64("swa", s, lengths, go, ge, T)[:, ptype]
    J = k.swa_param_grad(alpha, s, part, dS.astype(np.float32), lengths, go, ge, T, ptype)
    allow = 2e-6 * np.abs(dS) / T * post.reshape(len(dS), -1).max(axis=1, initial=0.0)
    return J, float(allow.max(initial=0.0)) + _noise_move(k, s, ptype, go, ge, T, lengths, J)


def _noise_move(k, s, ptype, go, ge, T, lengths, J):
    """3x the reference's own Jacobian movement under half-ulp noise on the scores:
    any fp32 evaluation (the GPU's alphas and partition round differently) perturbs
    the sweep by about that much."""
    rng = np.random.default_rng(0)
    sp = (s * (1 + 6e-8 * rng.standard_normal(s.shape))).astype(np.float32)
    alpha, part = k.swa_forward(sp, lengths, go, ge, T)
    dS = k.param_grads64("swa", sp, lengths, go, ge, T)[:, ptype]
    Jp = k.swa_param_grad(alpha, sp, part, dS.astype(np.float32), lengths, go, ge, T, ptype)
    return 3.0 * float(np.abs(Jp - J).max(initial=0.0))


def _close(gpu, ref, what, extra=0.0):
    close_entrywise(gpu, ref, what, extra, ATOL)


CASES = [
    # (seed, B, L1, L2, gap_open, gap_ext, T)
    (0, 3, 7, 9, -2.0, -0.5, 1.0),
    (1, 2, 40, 50, -1.5, -0.3, 0.5),
    (2, 2, 100, 120, -2.0, -0.5, 1.0),
    (3, 2, 65, 130, -1.0, -1.0, 2.0),
    (4, 1, 1, 1, -2.0, -0.5, 1.0),
    (5, 2, 200, 90, -3.0, -0.2, 1.0),
    (6, 1, 600, 70, -2.0, -0.5, 1.0),      # more stripes than waves in a workgroup
    (7, 1, 130, 1200, -2.0, -0.5, 1.0),    # long rows: ring length near the LDS budget
]


@pytest.mark.parametrize("seed,B,L1,L2,go,ge,T", CASES)
def test_swa_hvp(cuda, seed, B, L1, L2, go, ge, T):
    s = _seeded(seed, (B, L1, L2))
    v = _seeded(seed + 100, (B, L1, L2))
    ref = O.get("oracle").soft_sw_affine_hvp(s.numpy(), v.numpy(), go, ge, T)
    gpu = _capi.swa_hvp(s.to(cuda), v.to(cuda), None, go, ge, T)
    _close(gpu, ref, "hvp")


@pytest.mark.parametrize("seed,B,L1,L2,go,ge,T", CASES)
@pytest.mark.parametrize("ptype", [0, 1, 2])
def test_swa_param_jacobian(cuda, seed, B, L1, L2, go, ge, T, ptype):
    s = _seeded(seed, (B, L1, L2))
    ref, allow = _jacobian_ref(O.get("oracle"), s.numpy(), ptype, go, ge, T)
    gpu = _capi.swa_param_jacobian(s.to(cuda), ptype, None, go, ge, T)
    _close(gpu, ref, f"dP/d{NAMES[ptype]}", allow)


def test_swa_second_ragged(cuda):
    B, L1, L2 = 5, 90, 110
    s = _seeded(7, (B, L1, L2))
    v = _seeded(8, (B, L1, L2))
    lens = np.array([[90, 110], [0, 40], [33, 0], [1, 1], [57, 81]], np.int32)
    k = O.get("oracle")
    lt = torch.from_numpy(lens).to(cuda)
    _close(_capi.swa_hvp(s.to(cuda), v.to(cuda), lt, -2.0, -0.5, 0.7),
           k.soft_sw_affine_hvp(s.numpy(), v.numpy(), -2.0, -0.5, 0.7, lens), "hvp ragged")
    for p in (0, 1, 2):
        ref, allow = _jacobian_ref(k, s.numpy(), p, -2.0, -0.5, 0.7, lens)
        _close(_capi.swa_param_jacobian(s.to(cuda), p, lt, -2.0, -0.5, 0.7), ref,
               f"jacobian {NAMES[p]} ragged", allow)


def test_swa_backward_full(cuda):
    """grad_scores = H ga; per-element <ga, dP/dopen>, <ga, dP/dext>, <ga, dP/dT>."""
    B, L1, L2 = 3, 80, 96
    go, ge, T = -2.0, -0.5, 1.0
    s = _seeded(9, (B, L1, L2))
    ga = _seeded(10, (B, L1, L2))
    k = O.get("oracle")
    gs, *gp = _capi.swa_backward_full(s.to(cuda), ga.to(cuda), None, go, ge, T)
    _close(gs, k.soft_sw_affine_hvp(s.numpy(), ga.numpy(), go, ge, T), "backward_full scores")
    for p, g in enumerate(gp):
        J, allow = _jacobian_ref(k, s.numpy(), p, go, ge, T)
        ref = (J.astype(np.float64) * ga.numpy()).sum(axis=(1, 2))
        got = g.cpu().numpy()
        # entry errors up to 1e-4 * max|J| + allow, partly cancelling in the dot product
        per = 1e-4 * max(1.0, np.abs(J).max()) + allow
        tol = per * np.abs(ga.numpy()).sum(axis=(1, 2))
        assert np.all(np.abs(got - ref) <= tol), (NAMES[p], got, ref, tol)


def test_swa_ops_match_capi(cuda):
    """torch.ops.d2p affine second-order ops route to the same kernels."""
    import d2p_amd
    from d2p_amd import ops
    go, ge, T = -2.0, -0.5, 1.0
    s = _seeded(21, (2, 50, 60))
    v = _seeded(22, (2, 50, 60))
    k = O.get("oracle")
    href = k.soft_sw_affine_hvp(s.numpy(), v.numpy(), go, ge, T)
    _close(d2p_amd.soft_sw_affine_hvp(s.to(cuda), v.to(cuda), go, ge, T, None), href,
           "soft_sw_affine_hvp op")
    _close(ops.sw_affine.marginals_hvp(s.to(cuda), v.to(cuda), go, ge, T), href,
           "sw_affine_marginals_hvp op")
    fns = (ops.sw_affine.marginals_grad_gap_open, ops.sw_affine.marginals_grad_gap_ext,
           ops.sw_affine.marginals_grad_temp)
    for p, fn in enumerate(fns):
        ref, allow = _jacobian_ref(k, s.numpy(), p, go, ge, T)
        _close(d2p_amd.soft_sw_affine_param_jacobian(s.to(cuda), p, go, ge, T, None), ref,
               "soft_sw_affine_param_jacobian op", allow)
        _close(fn(s.to(cuda), go, ge, T), ref, "sw_affine_marginals_grad op", allow)
    gs, g_o, g_e, g_t = d2p_amd.soft_sw_affine_backward_full(s.to(cuda), v.to(cuda), go, ge, T,
                                                             None)
    assert g_o.shape == (1,) and g_e.shape == (1,) and g_t.shape == (1,)
    _close(gs, href, "backward_full op")
    r = ops.sw_affine.marginals_backward(s.to(cuda), v.to(cuda), go, ge, T)
    _close(r[0], href, "sw_affine_marginals_backward op")


def test_swa_marginal_path_autograd(cuda):
    """loss = <W, marginals> + value / 2: d loss / d scores = H W + P / 2 and the
    parameter gradients <W, dP/dtheta> + sum_b dS_b/dtheta / 2."""
    import d2p_amd
    s = _seeded(31, (2, 40, 45))
    W = _seeded(32, (2, 40, 45))
    k = O.get("oracle")
    x = s.to(cuda).requires_grad_(True)
    go = torch.tensor(-2.0, device=cuda, requires_grad=True)
    ge = torch.tensor(-0.5, device=cuda, requires_grad=True)
    T = torch.tensor(0.8, device=cuda, requires_grad=True)
    res = d2p_amd.soft_sw_affine(x, gap_open=go, gap_ext=ge, temperature=T)
    loss = (res.marginals * W.to(cuda)).sum() + 0.5 * res.value.sum()
    loss.backward()
    rp, rm, rgo, rge, rgt = k.soft_sw_affine(s.numpy(), -2.0, -0.5, 0.8)
    expect = k.soft_sw_affine_hvp(s.numpy(), W.numpy(), -2.0, -0.5, 0.8) + 0.5 * rm
    _close(x.grad, expect, "marginal-path grad_scores")
    for p, g, rv in ((0, go, rgo), (1, ge, rge), (2, T, rgt)):
        J, allow = _jacobian_ref(k, s.numpy(), p, -2.0, -0.5, 0.8)
        ref = float((J.astype(np.float64) * W.numpy()).sum() + 0.5 * rv.sum())
        tol = (1e-4 * max(1.0, np.abs(J).max()) + allow) * float(np.abs(W.numpy()).sum()) \
            + 1e-3 * abs(ref)
        assert abs(float(g.grad) - ref) <= tol, (NAMES[p], float(g.grad), ref, tol)
    # the same gradients against the GPU's own Jacobians and value-path gradients
    _, _, d_o, d_e, d_t = _capi.swa_forward_marginals(s.to(cuda), None, -2.0, -0.5, 0.8)
    for p, g, dv in ((0, go, d_o), (1, ge, d_e), (2, T, d_t)):
        Jg = _capi.swa_param_jacobian(s.to(cuda), p, None, -2.0, -0.5, 0.8)
        dot_consistent(g.grad, Jg, W, 0.5 * float(dv.double().sum()), f"affine {NAMES[p]}")


def test_swa_marginal_path_float_params(cuda):
    """Float parameters: only the scores receive the marginal-path gradient."""
    import d2p_amd
    s = _seeded(41, (2, 33, 47))
    W = _seeded(42, (2, 33, 47))
    x = s.to(cuda).requires_grad_(True)
    res = d2p_amd.soft_sw_affine(x, gap_open=-2.0, gap_ext=-0.5, temperature=1.0)
    (res.marginals * W.to(cuda)).sum().backward()
    ref = O.get("oracle").soft_sw_affine_hvp(s.numpy(), W.numpy(), -2.0, -0.5, 1.0)
    _close(x.grad, ref, "float-parameter marginal path")
