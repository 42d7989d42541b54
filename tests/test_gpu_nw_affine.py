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
