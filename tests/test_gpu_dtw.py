"""GPU parity of soft DTW against the CPU oracle.

The HIP path is called through the C ABI (tests/_capi.py) and through the
PyTorch API; the oracle (oracle/liboracle.so, bit-identical to the reference's
own CPU kernels, src/dtw/kernels_cpu.cpp) supplies the expected values on the
same seeded inputs.

Tolerances: value within 1e-5 relative, marginals within 1e-4 absolute (the
north-star contract).  A soft-DTW value is the expected path cost minus an entropy
term of the same size (T log of the number of paths), so it can cancel to near
zero while both terms are hundreds; the value check therefore also allows 1e-7 of
the expected path cost sum(P * c), about one fp32 rounding of the cancelling
terms.  grad_T = sum beta * (softmin - E[alpha_pred]) / T is a
sum of cancelling terms of size |alpha| / T: 1e-3 relative plus 1e-5 * |value| / T
of the reference, or of its per-cell terms summed in double where the
reference's sequential fp32 sum has drifted further (tests/_paramgrad.py).
"""
import numpy as np
import pytest
import torch

import _capi
from _paramgrad import check_param_grad
from oracle import oracle as O

pytestmark = pytest.mark.gpu

VALUE_RTOL = 1e-5
MARG_ATOL = 1e-4


def _seeded(seed, shape, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32) * scale


def _sq_dist_costs(seed, B, L1, L2, D):
    """Config C4 style costs: pairwise squared Euclidean distances, built on the CPU."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((B, L1, D), generator=g, dtype=torch.float32)
    y = torch.randn((B, L2, D), generator=g, dtype=torch.float32)
    return torch.cdist(x, y, compute_mode="donot_use_mm_for_euclid_dist") ** 2


def _check(gpu, ref, costs, T, bw=-1, lengths=None):
    v, marg, gt = [x.detach().cpu().numpy() for x in gpu]
    rv, rm, rt = ref
    cancel = (rm.astype(np.float64) * costs).sum(axis=(1, 2))   # expected path cost
    tol = VALUE_RTOL * np.abs(rv) + 1e-7 * np.abs(cancel) + 1e-6
    assert np.all(np.abs(v.astype(np.float64) - rv) <= tol), (v, rv, tol)
    assert np.abs(marg - rm).max() <= MARG_ATOL, np.abs(marg - rm).max()
    k = O.get("oracle")
    ln = None if lengths is None else np.asarray(lengths, np.int32)
    check_param_grad(gt, rt, lambda: k.param_grads64("dtw", costs, ln, T, bandwidth=bw),
                     rtol=1e-3,
                     atol=1e-5 * (np.abs(rv[np.abs(rv) < 1e29]).max(initial=0.0) + 1.0) / T)
    if lengths is not None:
        for b, (l1, l2) in enumerate(lengths):
            assert np.all(marg[b, l1:, :] == 0.0) and np.all(marg[b, :, l2:] == 0.0)


CASES = [
    # (seed, B, L1, L2, T, bandwidth)
    (0, 3, 7, 9, 1.0, -1),
    (1, 4, 16, 16, 0.5, -1),
    (2, 2, 100, 120, 1.0, -1),
    (3, 3, 65, 130, 1.0, -1),      # one row past a 64-row stripe
    (4, 2, 128, 1, 1.0, -1),       # N x 1: value = sum of costs
    (5, 2, 1, 128, 1.0, -1),       # 1 x N
    (6, 1, 1, 1, 1.0, -1),
    (7, 2, 200, 300, 0.3, -1),
    (8, 2, 600, 90, 1.0, -1),      # more stripes than waves in a workgroup
    (9, 3, 120, 100, 1.0, 10),     # Sakoe-Chiba band
    (10, 2, 90, 90, 0.5, 0),       # zero-width band: the diagonal path only
    (11, 1, 600, 2500, 1.0, -1),   # long rows: 8-step backward chunks
]


@pytest.mark.parametrize("seed,B,L1,L2,T,bw", CASES)
def test_dtw_matches_oracle(cuda, seed, B, L1, L2, T, bw):
    c = _seeded(seed, (B, L1, L2)).abs()
    ref = O.get("oracle").soft_dtw(c.numpy(), T, None, bw)
    gpu = _capi.dtw_forward_marginals(c.to(cuda), None, T, bw)
    _check(gpu, ref, c.numpy(), T, bw)


def test_dtw_config_c4_style(cuda):
    """Squared-distance costs of 64-d features at T = 0.1 (config C4, fewer items)."""
    c = _sq_dist_costs(3, 4, 256, 256, 64)
    ref = O.get("oracle").soft_dtw(c.numpy(), 0.1)
    gpu = _capi.dtw_forward_marginals(c.to(cuda), None, 0.1)
    _check(gpu, ref, c.numpy(), 0.1)


@pytest.mark.parametrize("B,L1,L2,n_parts,ragged", [(4, 256, 256, 1, False),
                                                    (3, 700, 110, 4, True),
                                                    (2, 130, 300, 1, True),
                                                    (5, 64, 90, 1, True)])
def test_dtw_helper_waves_bit_identical(cuda, monkeypatch, B, L1, L2, n_parts, ragged):
    """Unbanded parts of at most four stripes run both sweeps with helper waves (the
    forward's load the costs and write the alpha table, the reverse sweep's load the
    alpha rows and write the marginals); the arithmetic is the sweeping wave's either
    way, so every output equals the form without helpers bit for bit (split parts and
    ragged lengths included)."""
    c = _sq_dist_costs(41, B, L1, L2, 16).to(cuda)
    lens = None
    if ragged:
        rows = [[L1, L2], [max(L1 - 37, 1), L2 // 2], [0, 7], [5, 0], [1, 1]][:B]
        lens = torch.tensor(rows, dtype=torch.int32, device=cuda)
    monkeypatch.setenv("D2P_AMD_SPLIT", str(n_parts))
    monkeypatch.setenv("D2P_AMD_DTW_HELPERS", "1")
    with_h = _capi.dtw_forward_marginals(c, lens, 0.3)
    monkeypatch.setenv("D2P_AMD_DTW_HELPERS", "0")
    without = _capi.dtw_forward_marginals(c, lens, 0.3)
    for a, b in zip(with_h, without):
        assert torch.equal(a, b)


def test_dtw_ragged_lengths_and_band(cuda):
    B, L1, L2 = 6, 150, 170
    c = _seeded(4, (B, L1, L2)).abs()
    lens = torch.tensor([[150, 170], [0, 50], [40, 0], [0, 0], [77, 123], [1, 170]],
                        dtype=torch.int32)
    for bw in (-1, 20):
        ref = O.get("oracle").soft_dtw(c.numpy(), 0.7, lens.numpy(), bw)
        gpu = _capi.dtw_forward_marginals(c.to(cuda), lens.to(cuda), 0.7, bw)
        _check(gpu, ref, c.numpy(), 0.7, bw, lens.tolist())


def test_dtw_api_value_backward(cuda):
    import d2p_amd
    c = _seeded(11, (3, 70, 90)).abs()
    x = c.to(cuda).requires_grad_(True)
    res = d2p_amd.soft_dtw(x, temperature=0.5)
    w = torch.tensor([1.0, -2.0, 0.5], device=cuda)
    (res.cost * w).sum().backward()
    rv, rm, _ = O.get("oracle").soft_dtw(c.numpy(), 0.5)
    np.testing.assert_allclose(res.cost.detach().cpu().numpy(), rv, rtol=VALUE_RTOL)
    expect = rm * w.cpu().numpy()[:, None, None]
    assert np.abs(x.grad.cpu().numpy() - expect).max() <= 2 * MARG_ATOL


def test_dtw_tensor_temperature_grad(cuda):
    import d2p_amd
    c = _seeded(12, (2, 40, 50)).abs()
    T = torch.tensor(0.7, device=cuda, requires_grad=True)
    res = d2p_amd.soft_dtw(c.to(cuda), temperature=T)
    res.cost.sum().backward()
    rv, _, rt = O.get("oracle").soft_dtw(c.numpy(), 0.7)
    np.testing.assert_allclose(T.grad.cpu().numpy(), rt.sum(), rtol=2e-3,
                               atol=1e-5 * np.abs(rv).sum() / 0.7)
