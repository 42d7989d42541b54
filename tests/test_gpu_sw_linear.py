"""GPU parity of linear-gap soft Smith-Waterman against the CPU oracle.

The HIP path is called through the C ABI (tests/_capi.py) and through the
PyTorch API; the oracle (oracle/liboracle.so, bit-identical to the reference's
own CPU kernels) supplies the expected values on the same seeded inputs.

Tolerances: value within 1e-5 relative, marginals within
1e-4 absolute.  grad_gap within 3e-4 relative and grad_T within 1e-3 relative
plus 2e-5 * S / T (a difference of two O(S) numbers divided by T) -- of the
reference, or, where the reference's sequential fp32 sum over millions of cells
has drifted further than that, of the reference's per-cell terms summed in
double (tests/_paramgrad.py).
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


def _check(gpu, ref, lengths=None, gap=-1.0, T=1.0, scores=None):
    part, marg, gg, gt = [x.detach().cpu().numpy() for x in gpu]
    rp, rm, rg, rt = ref
    np.testing.assert_allclose(part, rp, rtol=VALUE_RTOL, atol=1e-6)
    assert np.abs(marg - rm).max() <= MARG_ATOL, np.abs(marg - rm).max()
    k = O.get("oracle")
    exact = lambda: k.param_grads64("sw", scores, lengths, gap, T)
    check_param_grad(gg, rg, lambda: exact()[:, 0])
    check_param_grad(gt, rt, lambda: exact()[:, 1], rtol=1e-3,
                     atol=2e-5 * (np.abs(rp).max() + 1.0) / T)
    if lengths is not None:
        for b, (l1, l2) in enumerate(lengths):
            assert np.all(marg[b, l1:, :] == 0.0) and np.all(marg[b, :, l2:] == 0.0)


CASES = [
    # (seed, B, L1, L2, gap, T)
    (0, 3, 7, 9, -1.0, 1.0),
    (1, 4, 16, 16, -1.0, 0.1),
    (2, 4, 5, 20, -0.5, 2.0),
    (42, 2, 100, 120, -1.0, 1.0),      # README quick-start / config C1 shape
    (3, 3, 65, 130, -1.0, 1.0),        # one row past a 64-row stripe
    (4, 2, 64, 64, -1.0, 1.0),
    (5, 2, 128, 1, -1.0, 1.0),
    (6, 2, 1, 128, -1.0, 1.0),
    (7, 1, 1, 1, -1.0, 1.0),
    (8, 2, 200, 300, -1.0, 0.5),
    (9, 9, 300, 70, -2.0, 1.5),
    (10, 2, 600, 90, -1.0, 1.0),       # more stripes than waves in a workgroup
    (11, 1, 1100, 300, -1.0, 1.0),     # ... more than two rounds of waves
    (12, 1, 600, 2500, -1.0, 1.0),     # long rows: rings too long for 16-step backward chunks
    (13, 1, 4096, 4096, -1.0, 1.0),    # config C5 element (64 stripes, 8 rounds of waves)
]


@pytest.mark.parametrize("seed,B,L1,L2,gap,T", CASES)
def test_sw_capi_matches_oracle(cuda, seed, B, L1, L2, gap, T):
    s = _seeded(seed, (B, L1, L2))
    ref = O.get("oracle").soft_sw(s.numpy(), gap, T)
    out = _capi.sw_forward_marginals(s.to(cuda), None, gap, T)
    torch.cuda.synchronize()
    _check(out, ref, gap=gap, T=T, scores=s.numpy())


def test_sw_capi_ragged_lengths(cuda):
    B, L1, L2 = 7, 150, 170
    s = _seeded(11, (B, L1, L2), 2.0)
    g = np.random.default_rng(11)
    lengths = np.stack([g.integers(0, L1 + 1, B), g.integers(0, L2 + 1, B)], 1).astype(np.int32)
    lengths[0] = [L1, L2]
    lengths[1] = [0, 5]
    lengths[2] = [64, 0]
    lengths[3] = [1, 1]
    ref = O.get("oracle").soft_sw(s.numpy(), -1.0, 0.5, lengths)
    out = _capi.sw_forward_marginals(s.to(cuda), torch.from_numpy(lengths).to(cuda), -1.0, 0.5)
    torch.cuda.synchronize()
    _check(out, ref, lengths=lengths, gap=-1.0, T=0.5, scores=s.numpy())


def test_sw_capi_config_c2_full_size(cuda):
    """North-star config C2: scores [256, 512, 512] ~ N(0,1), seed 1, gap -1, T 1."""
    s = _seeded(1, (256, 512, 512))
    ref = O.get("oracle").soft_sw(s.numpy(), -1.0, 1.0)
    out = _capi.sw_forward_marginals(s.to(cuda), None, -1.0, 1.0)
    torch.cuda.synchronize()
    _check(out, ref, scores=s.numpy())
    marg = out[1]
    assert float(marg.min()) >= 0.0 and float(marg.max()) <= 1.0 + 1e-5


@pytest.mark.parametrize("shape", [(5, 33, 17), (3, 64, 80), (2, 512, 512)])
def test_scale_by_batch(cuda, shape):
    """Scalar rows (33*17 floats), 16-byte rows with a partial last chunk (1280
    float4s), and the C2 row length."""
    src = _seeded(3, shape).to(cuda)
    g = _seeded(4, (shape[0],)).to(cuda)
    out = _capi.scale_by_batch(src, g)
    torch.cuda.synchronize()
    torch.testing.assert_close(out, g.view(-1, 1, 1) * src, rtol=0, atol=0)


@pytest.mark.parametrize("kind", ["expanded", "every_other", "contiguous"])
def test_scale_by_batch_strided(cuda, kind):
    """Factors read in place by stride: one value expanded over the batch (stride 0,
    the gradient of value.sum()), every other element of a longer vector, and a
    contiguous vector; each bit-identical to the broadcast product."""
    src = _seeded(5, (6, 40, 36)).to(cuda)
    base = _seeded(6, (12,)).to(cuda)
    g = {"expanded": base[3:4].expand(6), "every_other": base[::2],
         "contiguous": base[:6]}[kind]
    out = _capi.scale_by_batch_strided(src, g)
    torch.cuda.synchronize()
    torch.testing.assert_close(out, g.reshape(-1, 1, 1) * src, rtol=0, atol=0)


@pytest.mark.parametrize("shape,kind", [((5, 33, 17), "contiguous"), ((6, 64, 80), "expanded"),
                                        ((4, 40, 36), "every_other"), ((3, 7, 5), "contiguous")])
def test_scale_by_batch_lengths(cuda, shape, kind):
    """Tables that are zero outside ragged lengths (empty, partial and full elements):
    bit-identical to the broadcast product, padding included (g * 0 keeps the sign of
    a negative factor), with only the cells inside the lengths read (the padding
    holds NaN in src here, which a read would carry into the output)."""
    B, L1, L2 = shape
    src = _seeded(7, shape).to(cuda)
    lens = torch.tensor([[L1, L2], [0, L2], [L1 - 3, 1], [2, L2 - 1], [L1, 0], [1, 1]][:B],
                        dtype=torch.int32)
    mask = torch.zeros(shape, dtype=torch.bool)
    for b in range(B):
        mask[b, :lens[b, 0], :lens[b, 1]] = True
    mask = mask.to(cuda)
    base = _seeded(8, (2 * B,)).to(cuda)
    g = {"expanded": base[3:4].expand(B), "every_other": base[::2],
         "contiguous": base[:B]}[kind]
    expect = g.reshape(-1, 1, 1) * torch.where(mask, src, torch.zeros_like(src))
    poisoned = torch.where(mask, src, torch.full_like(src, float("nan")))
    out = _capi.scale_by_batch_lengths(poisoned, g, lens.to(cuda))
    torch.cuda.synchronize()
    torch.testing.assert_close(out, expect, rtol=0, atol=0)
    assert torch.equal(torch.signbit(out), torch.signbit(expect))
    # no lengths: the full product
    full = _capi.scale_by_batch_lengths(src, g, None)
    torch.testing.assert_close(full, g.reshape(-1, 1, 1) * src, rtol=0, atol=0)


def test_ragged_value_backward_is_the_scaled_marginals(cuda):
    """soft_sw / soft_sw_affine with ragged lengths, value.sum() and a weighted sum
    backward: the gradient equals grad_value[b] * marginals bit for bit."""
    import d2p_amd
    s = _seeded(9, (3, 70, 90)).to(cuda)
    lens = torch.tensor([[70, 90], [33, 41], [5, 90]], dtype=torch.int32, device=cuda)
    w = torch.tensor([1.5, -2.0, 0.25], device=cuda)
    for fn in (lambda x: d2p_amd.soft_sw(x, gap=-1.0, temperature=1.0, lengths=lens),
               lambda x: d2p_amd.soft_sw_affine(x, gap_open=-2.0, gap_ext=-0.5,
                                                temperature=1.0, lengths=lens)):
        x = s.detach().requires_grad_(True)
        r = fn(x)
        (r.value * w).sum().backward()
        torch.cuda.synchronize()
        torch.testing.assert_close(x.grad, w.view(-1, 1, 1) * r.marginals.detach(),
                                   rtol=0, atol=0)


def test_soft_sw_api_value_backward(cuda):
    """d2p_amd.soft_sw + value.sum().backward(): grad equals the marginals."""
    import d2p_amd
    s = _seeded(42, (2, 100, 120))
    ref = O.get("oracle").soft_sw(s.numpy(), -1.0, 1.0)
    x = s.to(cuda).requires_grad_(True)
    res = d2p_amd.soft_sw(x, gap=-1.0, temperature=1.0)
    res.value.sum().backward()
    torch.cuda.synchronize()
    np.testing.assert_allclose(res.value.detach().cpu().numpy(), ref[0], rtol=VALUE_RTOL)
    assert np.abs(res.marginals.detach().cpu().numpy() - ref[1]).max() <= MARG_ATOL
    assert np.abs(x.grad.cpu().numpy() - ref[1]).max() <= MARG_ATOL
    assert res.score is res.value and res.alignment is res.marginals


def test_soft_sw_api_weighted_backward_and_param_grads(cuda):
    """Upstream weights scale the marginals; tensor gap/T receive sum_b w_b * dS_b/dtheta."""
    import d2p_amd
    s = _seeded(5, (3, 40, 50))
    ref = O.get("oracle").soft_sw(s.numpy(), -1.0, 0.8)
    x = s.to(cuda).requires_grad_(True)
    gap = torch.tensor([-1.0], device=cuda, requires_grad=True)
    temp = torch.tensor([0.8], device=cuda, requires_grad=True)
    w = torch.tensor([1.0, -2.0, 0.5], device=cuda)
    res = d2p_amd.soft_sw(x, gap=gap, temperature=temp)
    (res.value * w).sum().backward()
    torch.cuda.synchronize()
    wn = w.cpu().numpy()
    exp_grad = wn[:, None, None] * ref[1]
    assert np.abs(x.grad.cpu().numpy() - exp_grad).max() <= 2 * MARG_ATOL
    np.testing.assert_allclose(gap.grad.cpu().numpy(), [(wn * ref[2]).sum()], rtol=1e-4, atol=1e-3)
    np.testing.assert_allclose(temp.grad.cpu().numpy(), [(wn * ref[3]).sum()], rtol=1e-3, atol=1e-2)
    assert gap.grad.shape == (1,) and temp.grad.shape == (1,)


def test_soft_sw_api_masks_match_lengths(cuda):
    import d2p_amd
    B, L1, L2 = 3, 30, 40
    s = _seeded(6, (B, L1, L2)).to(cuda)
    lengths = torch.tensor([[30, 40], [12, 33], [1, 7]], dtype=torch.int32, device=cuda)
    m1 = torch.arange(L1, device=cuda)[None, :] < lengths[:, :1]
    m2 = torch.arange(L2, device=cuda)[None, :] < lengths[:, 1:]
    a = d2p_amd.soft_sw(s, lengths=lengths)
    b = d2p_amd.soft_sw(s, mask1=m1, mask2=m2)
    torch.testing.assert_close(a.value, b.value, rtol=0, atol=0)
    torch.testing.assert_close(a.marginals, b.marginals, rtol=0, atol=0)
