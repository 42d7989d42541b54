"""GPU parity of affine-gap soft Smith-Waterman against the CPU oracle.

The HIP path is called through the C ABI (tests/_capi.py) and through the
PyTorch API; the oracle (oracle/liboracle.so, bit-identical to the reference's
own CPU kernels, src/sw_affine/kernels_cpu.cpp) supplies the expected values on
the same seeded inputs.

Tolerances: value within 1e-5 relative, marginals within 1e-4 absolute (the
north-star contract).  grad_open / grad_ext within 3e-4 relative and grad_T
within 1e-3 relative plus 2e-5 * S / T -- of the reference, or, where its
sequential fp32 sums have drifted further, of the reference's per-cell terms
summed in double (tests/_paramgrad.py).
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


def _check(gpu, ref, scores, go, ge, T, lengths=None):
    part, marg, g_o, g_e, gt = [x.detach().cpu().numpy() for x in gpu]
    rp, rm, ro, re, rt = ref
    np.testing.assert_allclose(part, rp, rtol=VALUE_RTOL, atol=1e-6)
    assert np.abs(marg - rm).max() <= MARG_ATOL, np.abs(marg - rm).max()
    k = O.get("oracle")
    ln = None if lengths is None else np.asarray(lengths, np.int32)
    exact = lambda: k.param_grads64("swa", scores, ln, go, ge, T)
    check_param_grad(g_o, ro, lambda: exact()[:, 0])
    check_param_grad(g_e, re, lambda: exact()[:, 1])
    check_param_grad(gt, rt, lambda: exact()[:, 2], rtol=1e-3,
                     atol=2e-5 * (np.abs(rp).max() + 1.0) / T)
    if lengths is not None:
        for b, (l1, l2) in enumerate(lengths):
            assert np.all(marg[b, l1:, :] == 0.0) and np.all(marg[b, :, l2:] == 0.0)


CASES = [
    # (seed, B, L1, L2, gap_open, gap_ext, T)
    (0, 3, 7, 9, -2.0, -0.5, 1.0),
    (1, 4, 16, 16, -11.0, -1.0, 0.5),      # config C3 parameters
    (2, 2, 100, 120, -2.0, -0.5, 1.0),
    (3, 3, 65, 130, -3.0, -1.0, 1.0),      # one row past a 64-row stripe
    (4, 2, 128, 1, -2.0, -0.5, 1.0),
    (5, 2, 1, 128, -2.0, -0.5, 1.0),
    (6, 1, 1, 1, -2.0, -0.5, 1.0),
    (7, 2, 200, 300, -11.0, -1.0, 0.5),
    (8, 2, 600, 90, -2.0, -0.5, 1.0),      # more stripes than waves in a workgroup
]


@pytest.mark.parametrize("seed,B,L1,L2,go,ge,T", CASES)
def test_affine_matches_oracle(cuda, seed, B, L1, L2, go, ge, T):
    s = _seeded(seed, (B, L1, L2), 2.0)
    ref = O.get("oracle").soft_sw_affine(s.numpy(), go, ge, T)
    gpu = _capi.swa_forward_marginals(s.to(cuda), None, go, ge, T)
    _check(gpu, ref, s.numpy(), go, ge, T)


def test_affine_ragged_lengths(cuda):
    """Per-item lengths (config C3 style, scaled down), including empty items."""
    B, L1, L2 = 6, 300, 260
    s = _seeded(2, (B, L1, L2), 2.0)
    g = torch.Generator().manual_seed(5)
    lens = torch.randint(64, L1 + 1, (B, 2), generator=g, dtype=torch.int32)
    lens[:, 1] = torch.clamp(lens[:, 1], max=L2)
    lens[1] = torch.tensor([0, 100])
    lens[2] = torch.tensor([70, 0])
    lens[3] = torch.tensor([L1, L2])
    ref = O.get("oracle").soft_sw_affine(s.numpy(), -11.0, -1.0, 0.5, lens.numpy())
    gpu = _capi.swa_forward_marginals(s.to(cuda), lens.to(cuda), -11.0, -1.0, 0.5)
    _check(gpu, ref, s.numpy(), -11.0, -1.0, 0.5, lens.tolist())


def test_affine_api_value_backward(cuda):
    import d2p_amd
    s = _seeded(11, (3, 70, 90), 2.0)
    x = s.to(cuda).requires_grad_(True)
    res = d2p_amd.soft_sw_affine(x, gap_open=-11.0, gap_ext=-1.0, temperature=0.5)
    w = torch.tensor([1.0, -2.0, 0.5], device=cuda)
    (res.value * w).sum().backward()
    rp, rm, _, _, _ = O.get("oracle").soft_sw_affine(s.numpy(), -11.0, -1.0, 0.5)
    np.testing.assert_allclose(res.value.detach().cpu().numpy(), rp, rtol=VALUE_RTOL, atol=1e-6)
    expect = rm * w.cpu().numpy()[:, None, None]
    assert np.abs(x.grad.cpu().numpy() - expect).max() <= 2 * MARG_ATOL


def test_affine_tensor_params_grads(cuda):
    import d2p_amd
    s = _seeded(12, (2, 40, 50), 2.0)
    go = torch.tensor(-3.0, device=cuda, requires_grad=True)
    ge = torch.tensor(-0.5, device=cuda, requires_grad=True)
    T = torch.tensor(0.7, device=cuda, requires_grad=True)
    res = d2p_amd.soft_sw_affine(s.to(cuda), gap_open=go, gap_ext=ge, temperature=T)
    res.value.sum().backward()
    _, _, ro, re, rt = O.get("oracle").soft_sw_affine(s.numpy(), -3.0, -0.5, 0.7)
    np.testing.assert_allclose(go.grad.cpu().numpy(), ro.sum(), rtol=3e-4, atol=1e-4)
    np.testing.assert_allclose(ge.grad.cpu().numpy(), re.sum(), rtol=3e-4, atol=1e-4)
    np.testing.assert_allclose(T.grad.cpu().numpy(), rt.sum(), rtol=2e-3, atol=1e-3)
