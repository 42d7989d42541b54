"""Soft DTW with a Sakoe-Chiba band: banded sweeps and banded tables on the GPU.

With bandwidth >= 0 every stripe sweeps only the steps of its band window and the
skewed alpha (and tangent) tables keep only those steps, so time and workspace
shrink with the band (d2p_dtw_workspace_bytes_banded).  Cells outside the window
are out of the band: the marginals, HVP and Jacobian there must be exactly zero,
and everything else must match the CPU oracle to the tolerances of
test_gpu_dtw / test_gpu_dtw_second.  The cases cover narrow and zero bands, steep
slopes in both directions (L1 >> L2 and L1 << L2, where a stripe's window runs over
many columns), ragged lengths, split elements (D2P_AMD_SPLIT) and long banded
sequences.  A guard region after a workspace of exactly the banded size must come
back untouched, and the banded results must equal, bit for bit, those computed
in a workspace of the unbanded size.
"""
import ctypes

import numpy as np
import pytest
import torch

import _capi
from oracle import oracle as O
from test_gpu_dtw import _check, _sq_dist_costs
from test_gpu_dtw_second import _close, _jac_allow

pytestmark = pytest.mark.gpu

GUARD = 1 << 16


def _seeded(seed, shape, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32) * scale


@pytest.fixture
def parts(monkeypatch):
    def force(n):
        monkeypatch.setenv("D2P_AMD_SPLIT", str(n))
    return force


CASES = [
    # (seed, B, L1, L2, T, bandwidth, parts; 0 = automatic)
    (0, 3, 256, 256, 1.0, 0, 1),        # only the diagonal and its rounding neighbours
    (1, 3, 256, 256, 0.5, 16, 1),
    (2, 4, 700, 170, 0.7, 5, 1),        # L1 > L2: rows share columns
    (3, 3, 170, 700, 0.7, 5, 1),        # L1 < L2: a stripe's window spans ~4 columns a row
    (4, 2, 1000, 64, 1.0, 3, 0),
    (5, 2, 64, 1000, 1.0, 3, 0),
    (6, 2, 900, 900, 1.0, 8, 3),        # split parts, narrow band
    (7, 1, 3000, 3000, 1.0, 32, 0),     # long banded sequence, automatic parts
    (8, 1, 3000, 3000, 1.0, 32, 1),     # the same in one workgroup
    (9, 2, 1300, 1100, 0.5, 200, 2),    # wide band
]


@pytest.mark.parametrize("seed,B,L1,L2,T,bw,n", CASES)
def test_banded_matches_oracle(cuda, parts, seed, B, L1, L2, T, bw, n):
    parts(n)
    c = _seeded(seed, (B, L1, L2)).abs()
    ref = O.get("oracle").soft_dtw(c.numpy(), T, None, bw)
    gpu = _capi.dtw_forward_marginals(c.to(cuda), None, T, bw)
    torch.cuda.synchronize()
    _check(gpu, ref, c.numpy(), T, bw)


def test_banded_c4_style(cuda):
    """Config C4's costs (squared distances, T = 0.1) under a band of 16."""
    c = _sq_dist_costs(3, 16, 256, 256, 64)
    ref = O.get("oracle").soft_dtw(c.numpy(), 0.1, None, 16)
    gpu = _capi.dtw_forward_marginals(c.to(cuda), None, 0.1, 16)
    torch.cuda.synchronize()
    _check(gpu, ref, c.numpy(), 0.1, 16)


@pytest.mark.parametrize("n", [1, 4])
def test_banded_ragged(cuda, parts, n):
    parts(n)
    B, L1, L2 = 7, 700, 300
    c = _seeded(20, (B, L1, L2)).abs()
    lens = torch.tensor([[700, 300], [0, 50], [640, 0], [1, 300], [300, 1], [193, 123],
                         [450, 290]], dtype=torch.int32)
    for bw in (0, 7, 60):
        ref = O.get("oracle").soft_dtw(c.numpy(), 0.7, lens.numpy(), bw)
        gpu = _capi.dtw_forward_marginals(c.to(cuda), lens.to(cuda), 0.7, bw)
        torch.cuda.synchronize()
        _check(gpu, ref, c.numpy(), 0.7, bw, lens.tolist())


def _run_guarded(fn_name, size_name, args, B, L1, L2, bw, dev):
    """Calls a DTW entry point with a workspace of exactly the banded size followed by
    a guard region, and with one of the unbanded size; returns both workspaces."""
    lib = _capi.lib()
    nb = getattr(lib, size_name + "_banded")(B, L1, L2, bw)
    nf = getattr(lib, size_name)(B, L1, L2)
    assert nb <= nf
    out = []
    for n in (nb, nf):
        ws = torch.full((n + GUARD,), 0x5A, dtype=torch.uint8, device=dev)
        _capi.check(getattr(lib, fn_name)(*args(), _capi.ptr(ws), ctypes.c_size_t(n),
                                          _capi.stream()))
        _capi._check_status(ws, B)
        torch.cuda.synchronize()
        assert bool((ws[n:] == 0x5A).all()), f"{fn_name} wrote past its {n}-byte workspace"
        out.append(ws)
    return nb, nf


@pytest.mark.parametrize("n", [1, 3])
def test_banded_workspace_is_enough(cuda, parts, n):
    """Exactly d2p_dtw_workspace_bytes_banded suffices, the guard after it stays intact,
    and the results equal the unbanded-size workspace's bit for bit."""
    parts(n)
    B, L1, L2, bw = 3, 1500, 1200, 20
    c = _seeded(30, (B, L1, L2)).abs().to(cuda)
    lens = torch.tensor([[1500, 1200], [900, 1200], [1500, 333]], dtype=torch.int32,
                        device=cuda)
    res = []

    def args():
        outs = [torch.empty(B, device=cuda), torch.empty(B, L1, L2, device=cuda),
                torch.empty(B, device=cuda)]
        res.append(outs)
        return (_capi.ptr(c), _capi.ptr(lens), B, L1, L2, 1.0, bw, *[_capi.ptr(o) for o in outs])

    nb, nf = _run_guarded("d2p_dtw_forward_marginals", "d2p_dtw_workspace_bytes", args,
                          B, L1, L2, bw, cuda)
    assert nb < nf / 3, (nb, nf)
    for a, b in zip(*res):
        torch.testing.assert_close(a, b, rtol=0, atol=0)
    ref = O.get("oracle").soft_dtw(c.cpu().numpy(), 1.0, lens.cpu().numpy(), bw)
    _check(res[0], ref, c.cpu().numpy(), 1.0, bw, lens.tolist())


# ------------------------------------------------------------ second order

SECOND = [
    # (seed, B, L1, L2, T, bandwidth, parts)
    (40, 2, 300, 300, 1.0, 0, 1),
    (41, 2, 700, 170, 0.7, 6, 1),
    (42, 2, 170, 700, 0.7, 6, 2),
    (43, 2, 900, 900, 1.0, 10, 3),
    (44, 1, 2000, 2000, 1.0, 20, 0),
]


@pytest.mark.parametrize("seed,B,L1,L2,T,bw,n", SECOND)
def test_banded_hvp_and_jacobian(cuda, parts, seed, B, L1, L2, T, bw, n):
    parts(n)
    c = _seeded(seed, (B, L1, L2)).abs()
    v = _seeded(seed + 100, (B, L1, L2))
    k = O.get("oracle")
    _close(_capi.dtw_hvp(c.to(cuda), v.to(cuda), None, T, bw),
           k.soft_dtw_hvp(c.numpy(), v.numpy(), T, None, bw), f"banded hvp bw={bw}")
    _close(_capi.dtw_param_jacobian(c.to(cuda), None, T, bw),
           k.soft_dtw_param_jacobian(c.numpy(), T, None, bw), f"banded dP/dT bw={bw}",
           _jac_allow(k, c.numpy(), T, None, bw))


@pytest.mark.parametrize("n", [1, 4])
def test_banded_second_ragged(cuda, parts, n):
    parts(n)
    B, L1, L2 = 5, 700, 300
    c = _seeded(50, (B, L1, L2)).abs()
    v = _seeded(51, (B, L1, L2))
    lens = np.array([[700, 300], [0, 40], [193, 0], [300, 1], [450, 290]], np.int32)
    lt = torch.from_numpy(lens).to(cuda)
    k = O.get("oracle")
    for bw in (0, 12):
        _close(_capi.dtw_hvp(c.to(cuda), v.to(cuda), lt, 0.7, bw),
               k.soft_dtw_hvp(c.numpy(), v.numpy(), 0.7, lens, bw), f"hvp ragged bw={bw}")
        _close(_capi.dtw_param_jacobian(c.to(cuda), lt, 0.7, bw),
               k.soft_dtw_param_jacobian(c.numpy(), 0.7, lens, bw), f"jacobian ragged bw={bw}",
               _jac_allow(k, c.numpy(), 0.7, lens, bw))


def test_banded_backward_full(cuda, parts):
    parts(3)
    B, L1, L2, bw = 2, 800, 600, 9
    c = _seeded(60, (B, L1, L2)).abs()
    W = _seeded(61, (B, L1, L2))
    k = O.get("oracle")
    gc, gt = _capi.dtw_backward_full(c.to(cuda), W.to(cuda), None, 0.8, bw)
    _close(gc, k.soft_dtw_hvp(c.numpy(), W.numpy(), 0.8, None, bw), "banded backward_full")
    J = k.soft_dtw_param_jacobian(c.numpy(), 0.8, None, bw)
    ref = (J.astype(np.float64) * W.numpy()).sum(axis=(1, 2))
    per = 1e-4 * max(1.0, np.abs(J).max()) + _jac_allow(k, c.numpy(), 0.8, None, bw)
    tol = per * np.abs(W.numpy()).sum(axis=(1, 2))
    assert np.all(np.abs(gt.cpu().numpy() - ref) <= tol), (gt.cpu().numpy(), ref, tol)


@pytest.mark.parametrize("n", [1, 3])
def test_banded_second_workspace_is_enough(cuda, parts, n):
    parts(n)
    B, L1, L2, bw = 2, 1300, 1000, 15
    c = _seeded(70, (B, L1, L2)).abs().to(cuda)
    v = _seeded(71, (B, L1, L2)).to(cuda)
    lens = torch.tensor([[1300, 1000], [800, 990]], dtype=torch.int32, device=cuda)
    res = []

    def args():
        out = torch.empty(B, L1, L2, device=cuda)
        res.append(out)
        return (_capi.ptr(c), _capi.ptr(v), _capi.ptr(lens), B, L1, L2, 1.0, bw, _capi.ptr(out))

    nb, nf = _run_guarded("d2p_dtw_hvp", "d2p_dtw_second_workspace_bytes", args, B, L1, L2, bw,
                          cuda)
    assert nb < nf / 2, (nb, nf)
    torch.testing.assert_close(res[0], res[1], rtol=0, atol=0)
    ref = O.get("oracle").soft_dtw_hvp(c.cpu().numpy(), v.cpu().numpy(), 1.0,
                                       lens.cpu().numpy(), bw)
    _close(res[0], ref, "hvp in an exact banded workspace")
