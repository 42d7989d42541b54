"""GPU parity of linear-gap soft Needleman-Wunsch against the CPU oracle.

The global-alignment mode of the linear stripe sweeps (``d2p_nw_forward_marginals``,
``d2p_amd.soft_nw``) against oracle/d2p_oracle.c's NW restatement (bit-exact with
the reference's own nw/kernels_cpu.cpp) and its double-precision build
(liboracle64.so) for the parameter gradients.

Tolerances: marginals 1e-4 absolute; the value 1e-5 relative, plus 1e-6 of the
terms it is the difference of (the expected path score and gap * expected gaps,
which can cancel to a value near zero); dS/dgap and dS/dT 1e-3 relative to the
exact (double) values plus 2e-5 * (|value| + scale) / T.  Cases cover single
cells and rows, stripes boundaries, ragged and empty elements (whose value is the
boundary (L1 + L2) * gap), positive gaps, low temperature, split elements and rows
too long for unsplit stripe rings.
"""
import numpy as np
import pytest
import torch

import _capi
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _seeded(seed, shape, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32) * scale


@pytest.fixture
def parts(monkeypatch):
    def force(n):
        monkeypatch.setenv("D2P_AMD_SPLIT", str(n))
    return force


def _check(gpu, s, gap, T, lengths=None):
    v, marg, gg, gt = [x.detach().cpu().numpy().astype(np.float64) for x in gpu]
    ln = None if lengths is None else np.asarray(lengths, np.int32)
    rv, rm, _, _ = O.get("oracle").soft_nw(s, gap, T, ln)
    ev, em, eg, et = O.get("oracle64").soft_nw(s.astype(np.float64), gap, T, ln)
    scale = (em * np.abs(s)).sum(axis=(1, 2)) + abs(gap) * np.abs(eg)
    tol = 1e-5 * np.abs(ev) + 1e-6 * scale + 1e-6
    assert np.all(np.abs(v - ev) <= tol), ("value", v, ev, tol)
    assert np.abs(marg - rm).max() <= 1e-4, ("marginals", np.abs(marg - rm).max())
    atol = 2e-5 * (np.abs(ev) + scale + 1.0) / T
    assert np.all(np.abs(gg - eg) <= 1e-3 * np.abs(eg) + atol), ("dS/dgap", gg, eg)
    assert np.all(np.abs(gt - et) <= 1e-3 * np.abs(et) + atol), ("dS/dT", gt, et)
    if lengths is not None:
        for b, (l1, l2) in enumerate(lengths):
            assert np.all(marg[b, l1:, :] == 0.0) and np.all(marg[b, :, l2:] == 0.0)


CASES = [
    # (seed, B, L1, L2, gap, T)
    (0, 3, 7, 9, -1.0, 1.0),
    (1, 1, 1, 1, -1.0, 1.0),
    (2, 2, 1, 130, -0.5, 1.0),
    (3, 2, 130, 1, -0.5, 1.0),
    (4, 2, 100, 120, -1.0, 1.0),
    (5, 3, 65, 130, -1.0, 0.5),
    (6, 2, 64, 64, 0.3, 1.0),          # positive gap
    (7, 2, 513, 257, -1.0, 2.0),
    (8, 2, 90, 70, -1.0, 0.1),         # low temperature
    (9, 4, 300, 300, -2.0, 1.0),
]


@pytest.mark.parametrize("seed,B,L1,L2,gap,T", CASES)
def test_nw_matches_oracle(cuda, seed, B, L1, L2, gap, T):
    s = _seeded(seed, (B, L1, L2))
    gpu = _capi.nw_forward_marginals(s.to(cuda), None, gap, T)
    torch.cuda.synchronize()
    _check(gpu, s.numpy(), gap, T)


def test_nw_ragged_and_empty(cuda):
    B, L1, L2 = 7, 200, 150
    s = _seeded(20, (B, L1, L2))
    lens = [[200, 150], [0, 40], [70, 0], [0, 0], [1, 1], [133, 17], [64, 150]]
    lt = torch.tensor(lens, dtype=torch.int32)
    gpu = _capi.nw_forward_marginals(s.to(cuda), lt.to(cuda), -0.7, 0.8)
    torch.cuda.synchronize()
    _check(gpu, s.numpy(), -0.7, 0.8, lens)
    v = gpu[0].cpu().numpy()
    assert v[1] == pytest.approx(40 * -0.7) and v[2] == pytest.approx(70 * -0.7) and v[3] == 0.0


@pytest.mark.parametrize("n", [2, 3, 11])
def test_nw_split_parts(cuda, parts, n):
    parts(n)
    s = _seeded(30 + n, (2, 700, 90))
    gpu = _capi.nw_forward_marginals(s.to(cuda), None, -1.0, 1.0)
    torch.cuda.synchronize()
    _check(gpu, s.numpy(), -1.0, 1.0)


def test_nw_split_ragged(cuda, parts):
    parts(4)
    s = _seeded(40, (5, 700, 110))
    lens = [[700, 110], [0, 40], [193, 0], [1, 1], [257, 81]]
    gpu = _capi.nw_forward_marginals(s.to(cuda), torch.tensor(lens, dtype=torch.int32).to(cuda),
                                     -1.0, 0.7)
    torch.cuda.synchronize()
    _check(gpu, s.numpy(), -1.0, 0.7, lens)


@pytest.mark.parametrize("n", [0, 1])
def test_nw_long_rows(cuda, parts, n):
    """Rows too long for unsplit stripe rings force parts of at most 8 stripes."""
    parts(n)
    s = _seeded(50, (1, 600, 12000))
    gpu = _capi.nw_forward_marginals(s.to(cuda), None, -1.0, 1.0)
    torch.cuda.synchronize()
    _check(gpu, s.numpy(), -1.0, 1.0)


def test_nw_api_autograd(cuda):
    """soft_nw's value backpropagates through the marginals; tensor gap and
    temperature receive the batch sums of dS/dgap and dS/dT."""
    import d2p_amd
    s = _seeded(60, (3, 50, 40))
    x = s.to(cuda).requires_grad_(True)
    gap = torch.tensor([-0.8], device=cuda, requires_grad=True)
    T = torch.tensor([0.9], device=cuda, requires_grad=True)
    res = d2p_amd.soft_nw(x, gap=gap, temperature=T)
    w = torch.tensor([1.0, -2.0, 0.5], device=cuda)
    (res.score * w).sum().backward()
    ev, em, eg, et = O.get("oracle64").soft_nw(s.numpy().astype(np.float64), -0.8, 0.9)
    np.testing.assert_allclose(res.score.detach().cpu().numpy(), ev, rtol=1e-5, atol=1e-5)
    want = em * w.cpu().numpy()[:, None, None]
    assert np.abs(x.grad.cpu().numpy() - want).max() <= 2e-4
    wn = w.cpu().numpy()
    np.testing.assert_allclose(gap.grad.cpu().numpy(), [(eg * wn).sum()], rtol=1e-3, atol=1e-3)
    np.testing.assert_allclose(T.grad.cpu().numpy(), [(et * wn).sum()], rtol=1e-3, atol=1e-3)
    # float parameters and the module wrapper give the same value
    r2 = d2p_amd.soft_nw(s.to(cuda), gap=-0.8, temperature=0.9)
    torch.testing.assert_close(r2.score, res.score.detach(), rtol=0, atol=0)
    m = d2p_amd.SoftNW(gap=-0.8, temperature=0.9).to(cuda)
    torch.testing.assert_close(m(s.to(cuda)).score, res.score.detach(), rtol=0, atol=0)
