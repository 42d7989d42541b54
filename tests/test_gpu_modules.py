"""The nn.Module wrappers with learnable parameters, on the GPU, against the oracle.

/root/reference/d2p/sw.py:429-604 and d2p/dtw.py define SoftSW, SoftSWAffine and
SoftDTW: the parameters are 1-element tensors (nn.Parameter when learnable, a
buffer otherwise) handed to the ops as tensor parameters.  Each module runs on
ragged lengths (and a band for DTW):
- value path, loss = sum(value): value 1e-5 relative and marginals 1e-4 absolute
  against the oracle, grad of the scores equal to the marginals, parameter
  gradients against the oracle's per-element gradients summed (tests/_paramgrad.py);
- marginal path, loss = sum(value) + <W, marginals>: parameter gradients against
  the GPU's own per-element gradients and Jacobians (tests/_parity.dot_consistent).
"""
import numpy as np
import pytest
import torch

import _capi
from _paramgrad import check_param_grad
from _parity import dot_consistent
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _seeded(seed, shape):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32)


LENGTHS = [[50, 60], [37, 60], [50, 21]]


def _family(name, cuda):
    import d2p_amd
    k = O.get("oracle")
    lens = np.asarray(LENGTHS, np.int32)
    if name == "sw":
        mod = d2p_amd.SoftSW(gap=-0.7, temperature=0.6, learn_gap=True, learn_temperature=True)
        params = (-0.7, 0.6)
        names = ("gap", "temperature")
        oracle = lambda s: k.soft_sw(s, *params, lengths=lens)
        grads = lambda s, dev: _capi.sw_forward_marginals(s, torch.from_numpy(lens), *params)[2:]
        jac = lambda s, p: _capi.sw_param_jacobian(s, p, torch.from_numpy(lens), *params)
        fam64 = "sw"
    elif name == "swa":
        mod = d2p_amd.SoftSWAffine(gap_open=-1.5, gap_ext=-0.4, temperature=0.6,
                                   learn_gap_open=True, learn_gap_ext=True,
                                   learn_temperature=True)
        params = (-1.5, -0.4, 0.6)
        names = ("gap_open", "gap_ext", "temperature")
        oracle = lambda s: k.soft_sw_affine(s, *params, lengths=lens)
        grads = lambda s, dev: _capi.swa_forward_marginals(s, torch.from_numpy(lens), *params)[2:]
        jac = lambda s, p: _capi.swa_param_jacobian(s, p, torch.from_numpy(lens), *params)
        fam64 = "swa"
    else:
        mod = d2p_amd.SoftDTW(temperature=0.6, bandwidth=20, learnable=True)
        params = (0.6,)
        names = ("temperature",)
        oracle = lambda s: k.soft_dtw(s, 0.6, lengths=lens, bandwidth=20)
        grads = lambda s, dev: _capi.dtw_forward_marginals(s, torch.from_numpy(lens), 0.6, 20)[2:]
        jac = lambda s, p: _capi.dtw_param_jacobian(s, torch.from_numpy(lens), 0.6, 20)
        fam64 = "dtw"
    return mod, params, names, oracle, grads, jac, fam64, lens


@pytest.mark.parametrize("family", ["sw", "swa", "dtw"])
def test_module_learnable_value_path(cuda, family):
    mod, params, names, oracle, _, _, fam64, lens = _family(family, cuda)
    mod = mod.to(cuda)
    s = _seeded(40, (3, 50, 60))
    if family == "dtw":
        s = s.abs()
    x = s.to(cuda).requires_grad_(True)
    r = mod(x, torch.from_numpy(lens).to(cuda))
    r[0].sum().backward()
    ref = oracle(s.numpy())
    rv, rm = ref[0], ref[1]
    np.testing.assert_allclose(r[0].detach().cpu().numpy(), rv, rtol=1e-5, atol=1e-6)
    assert np.abs(r[1].detach().cpu().numpy() - rm).max() <= 1e-4
    assert torch.equal(x.grad, r[1].detach())
    k = O.get("oracle")
    bw = {"bandwidth": 20} if family == "dtw" else {}
    T = params[-1]
    for i, n in enumerate(names):
        g = getattr(mod, n).grad
        assert g is not None and g.shape == (1,), n
        want = np.asarray(ref[2 + i], np.float64)
        exact = lambda i=i: k.param_grads64(fam64, s.numpy(), lens, *params, **bw)[:, i]
        rtol, atol = (1e-3, 2e-5 * (np.abs(rv).max() + 1.0) / T) if n == "temperature" \
            else (3e-4, 1e-4)
        # the module's gradient is the per-element sum; check it against the sum
        check_param_grad(np.array([float(g)]), np.array([want.sum()]),
                         lambda: np.array([exact().sum()]), rtol=rtol, atol=3 * atol)


@pytest.mark.parametrize("family", ["sw", "swa", "dtw"])
def test_module_learnable_marginal_path(cuda, family):
    mod, params, names, _, grads, jac, _, lens = _family(family, cuda)
    mod = mod.to(cuda)
    s = _seeded(41, (3, 50, 60))
    if family == "dtw":
        s = s.abs()
    W = _seeded(42, (3, 50, 60))
    x = s.to(cuda).requires_grad_(True)
    r = mod(x, torch.from_numpy(lens).to(cuda))
    (r[0].sum() + (r[1] * W.to(cuda)).sum()).backward()
    per_elem = grads(s.to(cuda), cuda)
    for i, n in enumerate(names):
        g = getattr(mod, n).grad
        value_term = float(per_elem[i].double().sum())
        dot_consistent(g, jac(s.to(cuda), i), W, value_term, f"{family} {n}")
