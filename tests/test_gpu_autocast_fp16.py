"""float16 autocast (the reference's tests/test_autocast.py:17-140, float16 cases).

Under torch.autocast("cuda", float16) every d2p op upcasts its floating inputs to
float32 (/root/reference/d2p/_compile.py:857-931), so its outputs are float32 and
equal, bit for bit, the float32 run on the upcast input; that run is also held to the
oracle at the north-star tolerances (value 1e-5 relative, marginals 1e-4 absolute).
The gradient flows back to a float16 input in float16 (the marginals rounded), and
float32 inputs are unchanged under autocast.  Covered: soft_sw, soft_sw_affine,
soft_dtw and the low-level d2p.sw.soft_sw_forward / soft_sw_affine_forward ops.
"""
import numpy as np
import pytest
import torch

import d2p_amd
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _half(seed, shape, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dev).half()


def _oracle_close(value, marg, ref):
    np.testing.assert_allclose(value.cpu().numpy(), ref[0], rtol=1e-5, atol=1e-6)
    assert np.abs(marg.cpu().numpy() - ref[1]).max() <= 1e-4


def test_soft_sw_fp16_autocast_promotes_to_fp32(cuda):
    s16 = _half(1, (2, 8, 10), cuda)
    with torch.autocast("cuda", dtype=torch.float16):
        r = d2p_amd.soft_sw(s16, gap=-1.0)
    assert r.value.dtype == torch.float32 and r.marginals.dtype == torch.float32
    ref = d2p_amd.soft_sw(s16.float(), gap=-1.0)
    assert torch.equal(r.value, ref.value) and torch.equal(r.marginals, ref.marginals)
    _oracle_close(r.value, r.marginals, O.get("oracle").soft_sw(s16.float().cpu().numpy(), -1.0))


def test_soft_sw_affine_fp16_autocast(cuda):
    s16 = _half(2, (2, 8, 10), cuda)
    with torch.autocast("cuda", dtype=torch.float16):
        r = d2p_amd.soft_sw_affine(s16, gap_open=-2.0, gap_ext=-0.5)
    assert r.value.dtype == torch.float32 and r.marginals.dtype == torch.float32
    ref = d2p_amd.soft_sw_affine(s16.float(), gap_open=-2.0, gap_ext=-0.5)
    assert torch.equal(r.value, ref.value) and torch.equal(r.marginals, ref.marginals)
    _oracle_close(r.value, r.marginals,
                  O.get("oracle").soft_sw_affine(s16.float().cpu().numpy(), -2.0, -0.5))


def test_soft_dtw_fp16_autocast(cuda):
    c16 = _half(3, (3, 12, 9), cuda).abs()
    with torch.autocast("cuda", dtype=torch.float16):
        r = d2p_amd.soft_dtw(c16, temperature=0.5)
    assert r[0].dtype == torch.float32 and r[1].dtype == torch.float32
    ref = d2p_amd.soft_dtw(c16.float(), temperature=0.5)
    assert torch.equal(r[0], ref[0]) and torch.equal(r[1], ref[1])
    _oracle_close(r[0], r[1], O.get("oracle").soft_dtw(c16.float().cpu().numpy(), 0.5))


def test_fp16_autocast_gradient_flow(cuda):
    s = _half(4, (2, 8, 10), cuda).requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.float16):
        r = d2p_amd.soft_sw(s, gap=-1.0)
        loss = r.value.sum()
    loss.backward()
    assert s.grad is not None and s.grad.dtype == torch.float16
    assert torch.equal(s.grad, r.marginals.detach().half())


def test_fp16_autocast_numerical_stability(cuda):
    """The reference's comparison: float16 inputs under autocast against the same
    values in float32 without it, within 1e-5 (here: identical)."""
    torch.manual_seed(42)
    s16 = torch.randn(4, 16, 20, device=cuda, dtype=torch.float16)
    with torch.autocast("cuda", dtype=torch.float16):
        ra = d2p_amd.soft_sw(s16, gap=-1.0)
    rf = d2p_amd.soft_sw(s16.float(), gap=-1.0)
    torch.testing.assert_close(ra.value, rf.value, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(ra.marginals, rf.marginals, rtol=1e-5, atol=1e-5)


def test_fp32_unchanged_under_fp16_autocast(cuda):
    g = torch.Generator().manual_seed(5)
    s = torch.randn((2, 8, 10), generator=g).to(cuda)
    ref = d2p_amd.soft_sw(s, gap=-1.0)
    with torch.autocast("cuda", dtype=torch.float16):
        r = d2p_amd.soft_sw(s, gap=-1.0)
    assert r.value.dtype == torch.float32 and r.marginals.dtype == torch.float32
    assert torch.equal(r.value, ref.value) and torch.equal(r.marginals, ref.marginals)


def test_low_level_ops_fp16_autocast(cuda):
    s16 = _half(6, (2, 8, 10), cuda)
    with torch.autocast("cuda", dtype=torch.float16):
        v, m = d2p_amd.sw.soft_sw_forward(s16, -1.0, 1.0, None)
        va, ma = d2p_amd.sw.soft_sw_affine_forward(s16, -2.0, -0.5, 1.0, None)
    for t in (v, m, va, ma):
        assert t.dtype == torch.float32
    rv, rm = d2p_amd.sw.soft_sw_forward(s16.float(), -1.0, 1.0, None)
    assert torch.equal(v, rv) and torch.equal(m, rm)
    rva, rma = d2p_amd.sw.soft_sw_affine_forward(s16.float(), -2.0, -0.5, 1.0, None)
    assert torch.equal(va, rva) and torch.equal(ma, rma)
