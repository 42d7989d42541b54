"""Ops run on the caller's current stream (/root/reference/src/common/cuda_utils.h:58-93:
kernels launch on the current stream and the tensors they touch are recorded on it).

The default stream is parked behind a bounded spin kernel (torch.cuda._sleep, about
half a second); soft_sw, soft_sw_affine and soft_dtw then run forward and backward on a
side stream, which is synchronised on its own.  The default stream must still be busy
afterwards (nothing the ops launched or waited for sat behind it: no launch on the
null stream, no device-wide synchronisation), and every result matches the oracle at
the north-star tolerances (value 1e-5 relative, marginals and gradients 1e-4 absolute).
"""
import numpy as np
import pytest
import torch

import d2p_amd
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def test_ops_run_on_the_current_stream(cuda):
    g = torch.Generator().manual_seed(80)
    s_cpu = torch.randn((3, 70, 90), generator=g)
    c_cpu = torch.randn((3, 60, 50), generator=g).abs()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        s = s_cpu.to(cuda).requires_grad_(True)
        sa = s_cpu.to(cuda).requires_grad_(True)
        c = c_cpu.to(cuda).requires_grad_(True)
    side.synchronize()
    torch.cuda.synchronize()

    torch.cuda._sleep(int(1.2e9))     # about 0.5 s on the default stream
    with torch.cuda.stream(side):
        r = d2p_amd.soft_sw(s, gap=-1.0, temperature=1.0)
        r.value.sum().backward()
        ra = d2p_amd.soft_sw_affine(sa, gap_open=-3.0, gap_ext=-0.5, temperature=0.8)
        ra.value.sum().backward()
        rd = d2p_amd.soft_dtw(c, temperature=0.5)
        rd[0].sum().backward()
    side.synchronize()
    busy = not torch.cuda.default_stream().query()
    torch.cuda.synchronize()
    assert busy, "an op launched on, or waited for, the default stream"

    k = O.get("oracle")
    ref = k.soft_sw(s_cpu.numpy(), -1.0, 1.0)
    np.testing.assert_allclose(r.value.detach().cpu().numpy(), ref[0], rtol=1e-5)
    assert np.abs(r.marginals.detach().cpu().numpy() - ref[1]).max() <= 1e-4
    assert np.abs(s.grad.cpu().numpy() - ref[1]).max() <= 1e-4
    ref = k.soft_sw_affine(s_cpu.numpy(), -3.0, -0.5, 0.8)
    np.testing.assert_allclose(ra.value.detach().cpu().numpy(), ref[0], rtol=1e-5)
    assert np.abs(sa.grad.cpu().numpy() - ref[1]).max() <= 1e-4
    ref = k.soft_dtw(c_cpu.numpy(), 0.5)
    np.testing.assert_allclose(rd[0].detach().cpu().numpy(), ref[0], rtol=1e-5)
    assert np.abs(c.grad.cpu().numpy() - ref[1]).max() <= 1e-4
