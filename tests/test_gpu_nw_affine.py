"""GPU parity of affine-gap soft Needleman-Wunsch against the CPU oracle.

The global-alignment mode of the affine stripe sweeps (``d2p_nwa_*``) against
oracle/d2p_oracle.c's NW-affine restatement (oracle_nwa_*, bit-exact with the
reference's own nw_affine/kernels_cpu.cpp) and its double-precision build
(liboracle64.so).

Tolerances: marginals 1e-4 absolute; the value 1e-5 relative plus 1e-6 of the terms
it is the difference of (expected path score, open and extend costs); dS/dopen,
dS/dext and dS/dT 1e-3 relative to the exact (double) values plus 2e-5 * (|value| +
scale) / T.  Second order: HVP entries 1e-4 * max(1, |ref|) against the fp32
reference; Jacobian entries against the double-precision oracle with 1e-4 * max(1,
|ref|) plus 3x the fp32 reference's own distance from it.  Cases cover single cells
and rows, stripe boundaries, ragged and empty elements (whose value is the boundary
chain open + (L - 1) ext), low temperature, split elements and long rows.
"""
import numpy as np
import pytest
import torch

import _capi
from _parity import close_entrywise
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


def _check(gpu, s, go, ge, T, lengths=None):
    v, marg, g_o, g_e, g_t = [x.detach().cpu().numpy().astype(np.float64) for x in gpu]
    ln = None if lengths is None else np.asarray(lengths, np.int32)
    rv, rm, _, _, _ = O.get("oracle").soft_nw_affine(s, go, ge, T, ln)
    ev, em, eo, ee, et = O.get("oracle64").soft_nw_affine(s.astype(np.float64), go, ge, T, ln)
    scale = (em * np.abs(s)).sum(axis=(1, 2)) + abs(go) * np.abs(eo) + abs(ge) * np.abs(ee)
    tol = 1e-5 * np.abs(ev) + 1e-6 * scale + 1e-6
    assert np.all(np.abs(v - ev) <= tol), ("value", v, ev, tol)
    err = np.abs(marg - rm).max(initial=0.0)
    assert err <= 1e-4, ("marginals", err)
    atol = 2e-5 * (np.abs(ev) + scale + 1.0) / T
    for name, g, e in (("dS/dopen", g_o, eo), ("dS/dext", g_e, ee), ("dS/dT", g_t, et)):
        assert np.all(np.abs(g - e) <= 1e-3 * np.abs(e) + atol), (name, g, e)
    if lengths is not None:
        for b, (l1, l2) in enumerate(lengths):
            assert np.all(marg[b, l1:, :] == 0.0) and np.all(marg[b, :, l2:] == 0.0)


CASES = [
    # (seed, B, L1, L2, go, ge, T)
    (0, 3, 7, 9, -2.0, -0.5, 1.0),
    (1, 1, 1, 1, -2.0, -0.5, 1.0),
    (2, 2, 1, 130, -1.0, -0.3, 1.0),
    (3, 2, 130, 1, -1.0, -0.3, 1.0),
    (4, 2, 100, 120, -2.0, -0.5, 1.0),
    (5, 3, 65, 130, -3.0, -1.0, 0.5),
    (6, 2, 64, 64, -11.0, -1.0, 0.5),
    (7, 2, 513, 257, -2.0, -0.5, 2.0),
    (8, 2, 90, 70, -2.0, -0.5, 0.1),        # low temperature
    (9, 4, 300, 300, -2.0, -0.5, 1.0),
]


@pytest.mark.parametrize("seed,B,L1,L2,go,ge,T", CASES)
def test_nwa_matches_oracle(cuda, seed, B, L1, L2, go, ge, T):
    s = _seeded(seed, (B, L1, L2))
    gpu = _capi.nwa_forward_marginals(s.to(cuda), None, go, ge, T)
    torch.cuda.synchronize()
    _check(gpu, s.numpy(), go, ge, T)


def test_nwa_ragged_and_empty(cuda):
    B, L1, L2 = 7, 200, 150
    s = _seeded(20, (B, L1, L2))
    lens = [[200, 150], [0, 40], [70, 0], [0, 0], [1, 1], [133, 17], [64, 150]]
    lt = torch.tensor(lens, dtype=torch.int32)
    gpu = _capi.nwa_forward_marginals(s.to(cuda), lt.to(cuda), -2.0, -0.5, 0.8)
    torch.cuda.synchronize()
    _check(gpu, s.numpy(), -2.0, -0.5, 0.8, lens)
    v = gpu[0].cpu().numpy()
    assert v[1] == pytest.approx(-2.0 + 39 * -0.5) and v[2] == pytest.approx(-2.0 + 69 * -0.5)
    assert v[3] == 0.0
    g_o, g_e = gpu[2].cpu().numpy(), gpu[3].cpu().numpy()
    assert (g_o[1], g_e[1], g_o[2], g_e[2], g_o[3], g_e[3]) == (1, 39, 1, 69, 0, 0)


@pytest.mark.parametrize("n", [2, 3, 11])
def test_nwa_split_parts(cuda, parts, n):
    parts(n)
    s = _seeded(30 + n, (2, 700, 90))
    gpu = _capi.nwa_forward_marginals(s.to(cuda), None, -2.0, -0.5, 1.0)
    torch.cuda.synchronize()
    _check(gpu, s.numpy(), -2.0, -0.5, 1.0)


def test_nwa_split_ragged(cuda, parts):
    parts(4)
    s = _seeded(40, (5, 700, 110))
    lens = [[700, 110], [0, 40], [193, 0], [1, 1], [257, 81]]
    gpu = _capi.nwa_forward_marginals(s.to(cuda), torch.tensor(lens, dtype=torch.int32).to(cuda),
                                      -2.0, -0.5, 0.7)
    torch.cuda.synchronize()
    _check(gpu, s.numpy(), -2.0, -0.5, 0.7, lens)


@pytest.mark.parametrize("n", [0, 1])
def test_nwa_long_rows(cuda, parts, n):
    """Rows too long for unsplit stripe rings force parts of at most 8 stripes."""
    parts(n)
    s = _seeded(50, (1, 300, 9000))
    gpu = _capi.nwa_forward_marginals(s.to(cuda), None, -2.0, -0.5, 1.0)
    torch.cuda.synchronize()
    _check(gpu, s.numpy(), -2.0, -0.5, 1.0)


# ------------------------------------------------------------------ second order

def _close(gpu, ref, what, extra=0.0):
    return close_entrywise(gpu, ref, what, extra, ATOL)


def _jacobian_ref(s, ptype, go, ge, T, lengths=None):
    """The double-precision Jacobian and 3x the fp32 reference's distance from it."""
    J64 = O.get("oracle64").soft_nw_affine_param_jacobian(s.astype(np.float64), ptype, go, ge, T,
                                                          lengths)
    J32 = O.get("oracle").soft_nw_affine_param_jacobian(s, ptype, go, ge, T, lengths)
    return J64, 3.0 * float(np.abs(J32 - J64).max(initial=0.0))


SECOND = [
    # (seed, B, L1, L2, go, ge, T)
    (0, 3, 7, 9, -2.0, -0.5, 1.0),
    (1, 1, 1, 1, -2.0, -0.5, 1.0),
    (2, 2, 40, 50, -2.0, -0.5, 0.5),
    (3, 2, 100, 120, -1.0, -0.3, 1.0),
    (4, 2, 65, 130, -3.0, -1.0, 2.0),
    (5, 2, 1, 130, -1.0, -0.3, 1.0),
    (6, 2, 130, 1, -1.0, -0.3, 1.0),
    (7, 1, 600, 70, -2.0, -0.5, 1.0),       # more stripes than waves in a workgroup
]
NAMES = ("open", "ext", "T")


@pytest.mark.parametrize("seed,B,L1,L2,go,ge,T", SECOND)
def test_nwa_hvp(cuda, seed, B, L1, L2, go, ge, T):
    s = _seeded(seed, (B, L1, L2))
    v = _seeded(seed + 100, (B, L1, L2))
    ref = O.get("oracle").soft_nw_affine_hvp(s.numpy(), v.numpy(), go, ge, T)
    e = _close(_capi.nwa_hvp(s.to(cuda), v.to(cuda), None, go, ge, T), ref, "hvp")
    print(f"hvp max err {e:.2e}")


@pytest.mark.parametrize("seed,B,L1,L2,go,ge,T", SECOND)
@pytest.mark.parametrize("ptype", [0, 1, 2])
def test_nwa_param_jacobian(cuda, seed, B, L1, L2, go, ge, T, ptype):
    s = _seeded(seed, (B, L1, L2))
    ref, allow = _jacobian_ref(s.numpy(), ptype, go, ge, T)
    gpu = _capi.nwa_param_jacobian(s.to(cuda), ptype, None, go, ge, T)
    _close(gpu, ref, f"dP/d{NAMES[ptype]}", allow)


def test_nwa_second_ragged(cuda):
    B, L1, L2 = 6, 90, 110
    s = _seeded(17, (B, L1, L2))
    v = _seeded(18, (B, L1, L2))
    lens = np.array([[90, 110], [0, 40], [33, 0], [1, 1], [57, 81], [0, 0]], np.int32)
    lt = torch.from_numpy(lens).to(cuda)
    h = _capi.nwa_hvp(s.to(cuda), v.to(cuda), lt, -2.0, -0.5, 0.7)
    _close(h, O.get("oracle").soft_nw_affine_hvp(s.numpy(), v.numpy(), -2.0, -0.5, 0.7, lens),
           "hvp ragged")
    for p in (0, 1, 2):
        ref, allow = _jacobian_ref(s.numpy(), p, -2.0, -0.5, 0.7, lens)
        J = _capi.nwa_param_jacobian(s.to(cuda), p, lt, -2.0, -0.5, 0.7)
        _close(J, ref, f"jacobian {NAMES[p]} ragged", allow)
        Jn = J.cpu().numpy()
        for b, (l1, l2) in enumerate(lens):
            assert np.all(Jn[b, l1:, :] == 0.0) and np.all(Jn[b, :, l2:] == 0.0)


@pytest.mark.parametrize("n", [2, 3])
def test_nwa_second_split_parts(cuda, parts, n):
    parts(n)
    s = _seeded(40 + n, (2, 700, 90))
    v = _seeded(50 + n, (2, 700, 90))
    _close(_capi.nwa_hvp(s.to(cuda), v.to(cuda), None, -2.0, -0.5, 1.0),
           O.get("oracle").soft_nw_affine_hvp(s.numpy(), v.numpy(), -2.0, -0.5, 1.0), "hvp split")
    for p in (0, 1, 2):
        ref, allow = _jacobian_ref(s.numpy(), p, -2.0, -0.5, 1.0)
        _close(_capi.nwa_param_jacobian(s.to(cuda), p, None, -2.0, -0.5, 1.0), ref,
               f"jacobian {NAMES[p]} split", allow)


def test_nwa_backward_full(cuda):
    """grad_scores = H ga; per element <ga, dP/dX> for X in (open, ext, T), against the
    double dot product of the GPU's own (entry-pinned) Jacobians."""
    B, L1, L2 = 3, 80, 96
    s = _seeded(9, (B, L1, L2))
    ga = _seeded(10, (B, L1, L2))
    gs, *gp = _capi.nwa_backward_full(s.to(cuda), ga.to(cuda), None, -2.0, -0.5, 1.0)
    _close(gs, O.get("oracle").soft_nw_affine_hvp(s.numpy(), ga.numpy(), -2.0, -0.5, 1.0),
           "backward_full scores")
    W = ga.numpy().astype(np.float64)
    for p, g in enumerate(gp):
        J = _capi.nwa_param_jacobian(s.to(cuda), p, None, -2.0, -0.5, 1.0).cpu().numpy()
        ref = (J.astype(np.float64) * W).sum(axis=(1, 2))
        tol = 1e-5 * np.abs(J * W).sum(axis=(1, 2)) + 1e-6
        assert np.all(np.abs(g.cpu().numpy() - ref) <= tol), (NAMES[p], g.cpu().numpy(), ref)


# ------------------------------------------------------------------ torch API

def test_nwa_api_value_path(cuda):
    """soft_nw_affine's value backpropagates through the marginals; tensor gap_open,
    gap_ext and temperature receive the batch sums of dS/dX (against the double
    oracle); float parameters and the module give the same value."""
    import d2p_amd
    s = _seeded(60, (3, 50, 40))
    x = s.to(cuda).requires_grad_(True)
    go = torch.tensor([-1.8], device=cuda, requires_grad=True)
    ge = torch.tensor([-0.4], device=cuda, requires_grad=True)
    T = torch.tensor([0.9], device=cuda, requires_grad=True)
    res = d2p_amd.soft_nw_affine(x, gap_open=go, gap_ext=ge, temperature=T)
    w = torch.tensor([1.0, -2.0, 0.5], device=cuda)
    (res.score * w).sum().backward()
    ev, em, eo, ee, et = O.get("oracle64").soft_nw_affine(s.numpy().astype(np.float64), -1.8,
                                                          -0.4, 0.9)
    np.testing.assert_allclose(res.score.detach().cpu().numpy(), ev, rtol=1e-5, atol=1e-5)
    wn = w.cpu().numpy()
    assert np.abs(x.grad.cpu().numpy() - em * wn[:, None, None]).max() <= 2e-4
    for g, e in ((go, eo), (ge, ee), (T, et)):
        np.testing.assert_allclose(g.grad.cpu().numpy(), [(e * wn).sum()], rtol=1e-3, atol=1e-3)
    r2 = d2p_amd.soft_nw_affine(s.to(cuda), gap_open=-1.8, gap_ext=-0.4, temperature=0.9)
    torch.testing.assert_close(r2.score, res.score.detach(), rtol=0, atol=0)
    m = d2p_amd.SoftNWAffine(gap_open=-1.8, gap_ext=-0.4, temperature=0.9).to(cuda)
    torch.testing.assert_close(m(s.to(cuda)).score, res.score.detach(), rtol=0, atol=0)


def test_nwa_marginal_path_autograd(cuda):
    """loss = <W, alignment> + 0.5 sum(score): d loss / d scores = H W + 0.5 P and the
    parameter gradients <W, dP/dX> + 0.5 sum dS/dX, the latter against the double
    dot product of the GPU's own (entry-pinned) Jacobians."""
    import d2p_amd
    from _parity import dot_consistent
    s = _seeded(31, (2, 40, 45))
    W = _seeded(32, (2, 40, 45))
    x = s.to(cuda).requires_grad_(True)
    ps = [torch.tensor([v], device=cuda, requires_grad=True) for v in (-2.0, -0.5, 0.8)]
    res = d2p_amd.soft_nw_affine(x, gap_open=ps[0], gap_ext=ps[1], temperature=ps[2])
    ((res.alignment * W.to(cuda)).sum() + 0.5 * res.score.sum()).backward()
    k = O.get("oracle")
    _, rm, _, _, _ = k.soft_nw_affine(s.numpy(), -2.0, -0.5, 0.8)
    expect = k.soft_nw_affine_hvp(s.numpy(), W.numpy(), -2.0, -0.5, 0.8) + 0.5 * rm
    _close(x.grad, expect, "marginal-path grad_scores")
    per = _capi.nwa_forward_marginals(s.to(cuda), None, -2.0, -0.5, 0.8)[2:]
    for p, (g, dv) in enumerate(zip(ps, per)):
        J = _capi.nwa_param_jacobian(s.to(cuda), p, None, -2.0, -0.5, 0.8)
        dot_consistent(g.grad, J, W, 0.5 * float(dv.double().sum()), f"nwa {NAMES[p]}")
    # float parameters: the scores gradient alone, equal to the tensor-parameter one
    x2 = s.to(cuda).requires_grad_(True)
    r2 = d2p_amd.soft_nw_affine(x2, gap_open=-2.0, gap_ext=-0.5, temperature=0.8)
    ((r2.alignment * W.to(cuda)).sum() + 0.5 * r2.score.sum()).backward()
    torch.testing.assert_close(x2.grad, x.grad, rtol=0, atol=0)


def test_nwa_ops_match_capi(cuda):
    """torch.ops.d2p NW-affine ops route to the same kernels as the C ABI."""
    import d2p_amd
    from d2p_amd import ops
    s = _seeded(21, (2, 50, 60)).to(cuda)
    v = _seeded(22, (2, 50, 60)).to(cuda)
    h = _capi.nwa_hvp(s, v, None, -2.0, -0.5, 1.0)
    torch.testing.assert_close(d2p_amd.soft_nw_affine_hvp(s, v, -2.0, -0.5, 1.0, None), h,
                               rtol=0, atol=0)
    torch.testing.assert_close(ops.nw_affine_marginals_hvp(s, v, -2.0, -0.5, 1.0, None), h,
                               rtol=0, atol=0)
    for p, fn in enumerate((ops.nw_affine_marginals_grad_gap_open,
                            ops.nw_affine_marginals_grad_gap_ext,
                            ops.nw_affine_marginals_grad_temp)):
        J = _capi.nwa_param_jacobian(s, p, None, -2.0, -0.5, 1.0)
        torch.testing.assert_close(fn(s, -2.0, -0.5, 1.0, None), J, rtol=0, atol=0)
        torch.testing.assert_close(d2p_amd.soft_nw_affine_param_jacobian(s, p, -2.0, -0.5, 1.0,
                                                                         None), J, rtol=0, atol=0)
    ref = _capi.nwa_forward_marginals(s, None, -2.0, -0.5, 1.0)
    got = d2p_amd.soft_nw_affine_with_grads(s, -2.0, -0.5, 1.0, None)
    for a, b in zip(got, ref):
        torch.testing.assert_close(a, b, rtol=0, atol=0)
    vg = ops.nw_affine_value_grad_params(s, -2.0, -0.5, 1.0, None)
    for a, b in zip(vg, (ref[0], ref[2], ref[3])):
        torch.testing.assert_close(a, b, rtol=0, atol=0)
    gs, *gp = _capi.nwa_backward_full(s, v, None, -2.0, -0.5, 1.0)
    for fn in (d2p_amd.soft_nw_affine_backward_full, ops.nw_affine_marginals_backward):
        r = fn(s, v, -2.0, -0.5, 1.0, None)
        torch.testing.assert_close(r[0], gs, rtol=0, atol=0)
        for a, b in zip(r[1:], gp):
            torch.testing.assert_close(a, b.sum().reshape(1), rtol=0, atol=0)
    for fwd in (ops.nw_affine_forward(s, -2.0, -0.5, 1.0, None),
                ops.nw_affine_forward_t(s, *[torch.tensor([v], device=cuda)
                                             for v in (-2.0, -0.5, 1.0)],
                                        torch.tensor([[50, 60]] * 2, dtype=torch.int32,
                                                     device=cuda))):
        torch.testing.assert_close(fwd[0], ref[0], rtol=0, atol=0)
        torch.testing.assert_close(fwd[1], ref[1], rtol=0, atol=0)
