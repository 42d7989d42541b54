"""Squared-Euclidean costs + soft DTW from features (d2p_amd.soft_dtw_sqeuclidean).

No counterpart in the reference (its callers build torch.cdist(x, y) ** 2 first,
/root/reference/docs/algorithms/dtw.md:52).  Pinned three ways:
- the costs: d2p_amd::pairwise_sqdist (the op's own costs, |x|^2 + |y|^2 - 2 x.y with
  the dot products on the matrix cores, clamped at 0) within the expansion's bound
  (D + 4) u (|x_i| + |y_j|)^2 (u = 2^-24) of the exact float64 costs, and against
  torch.cdist(x, y, compute_mode="donot_use_mm_for_euclid_dist") ** 2 within that bound
  plus the direct sum's own (D + 2) u c (torch.cdist's default mode takes the same
  expansion at these sizes);
- the sweeps: the fused op against soft_dtw on the kernel's own costs, bit for bit
  (the same costs feed the same forward recurrence, and both run the one reverse
  sweep, which reads only the alpha table); and those results against the CPU oracle
  at the north-star contract (value 1e-5 relative, marginals 1e-4 absolute);
- the gradients dL/dx, dL/dy (value path and marginal path) against the same chain
  rule evaluated in float64 from the double-precision oracle on the exact costs, per
  entry within 2 eps_P sum_j |x_i - y_j| + 1e-4 (x) and the transposed sum (y), where
  eps_P is the marginals' (or the marginal-path cost gradient's) own measured
  distance from the double oracle.
"""
import numpy as np
import pytest
import torch

import _capi
from oracle import oracle as O

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


def _seeded(seed, shape):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32)


@pytest.fixture
def parts(monkeypatch):
    def force(n):
        monkeypatch.setenv("D2P_AMD_SPLIT", str(n))
    return force


def _exact_costs(x, y):
    x64, y64 = x.double().cpu(), y.double().cpu()
    return ((x64[:, :, None, :] - y64[:, None, :, :]) ** 2).sum(-1)


@pytest.mark.parametrize("B,L1,L2,D", [(2, 50, 70, 64), (3, 33, 17, 5), (1, 200, 130, 128),
                                       (2, 64, 64, 32), (1, 1, 1, 1)])
def test_pairwise_sqdist_bounds(cuda, B, L1, L2, D):
    import d2p_amd  # noqa: F401  (loads the operator library)
    x, y = _seeded(1, (B, L1, D)), _seeded(2, (B, L2, D))
    got = torch.ops.d2p_amd.pairwise_sqdist(x.to(cuda), y.to(cuda)).cpu().double()
    assert torch.equal(got.float(), _capi.pairwise_sqdist(x.to(cuda), y.to(cuda)).cpu())
    exact = _exact_costs(x, y)
    nx = x.double().norm(dim=2)[:, :, None]
    ny = y.double().norm(dim=2)[:, None, :]
    bound = (D + 4) * U * (nx + ny) ** 2 + 1e-30
    assert torch.all((got - exact).abs() <= bound), float(((got - exact).abs() / bound).max())
    cd = torch.cdist(x.to(cuda), y.to(cuda), compute_mode="donot_use_mm_for_euclid_dist") ** 2
    err = (got - cd.cpu().double()).abs()
    assert torch.all(err <= bound + (D + 2) * U * exact + 1e-6), float(err.max())
    print(f"costs: max |kernel - exact| / bound = {float(((got - exact).abs() / bound).max()):.2f},"
          f" max |kernel - cdist^2| = {float(err.max()):.2e}")


CASES = [
    # (seed, B, L1, L2, D, T, bandwidth)
    (0, 3, 40, 50, 64, 1.0, 0),
    (1, 2, 130, 70, 16, 0.5, 0),
    (2, 4, 256, 256, 64, 0.1, 0),        # C4's shape and temperature
    (3, 2, 100, 100, 128, 1.0, 0),
    (4, 2, 300, 200, 8, 1.0, 20),        # Sakoe-Chiba band
    (5, 1, 1, 1, 3, 1.0, 0),
]


@pytest.mark.parametrize("seed,B,L1,L2,D,T,bw", CASES)
def test_fused_matches_unfused_and_oracle(cuda, seed, B, L1, L2, D, T, bw):
    import d2p_amd
    x, y = _seeded(seed, (B, L1, D)), _seeded(seed + 50, (B, L2, D))
    xc, yc = x.to(cuda), y.to(cuda)
    costs = torch.ops.d2p_amd.pairwise_sqdist(xc, yc)
    fused = d2p_amd.soft_dtw_sqeuclidean(xc, yc, temperature=T, bandwidth=bw)
    plain = d2p_amd.soft_dtw(costs, temperature=T, bandwidth=bw)
    assert torch.equal(fused.cost, plain.cost)
    assert torch.equal(fused.alignment, plain.alignment)
    bwv = bw if bw > 0 else -1
    v, m, gT = _capi.dtw_sqeuclid_forward_marginals(xc, yc, None, T, bwv)
    _, _, gT_plain = _capi.dtw_forward_marginals(costs, None, T, bwv)
    assert torch.equal(v, fused.cost) and torch.equal(m, fused.alignment)
    assert torch.equal(gT, gT_plain)
    rv, rm, rt = O.get("oracle").soft_dtw(costs.cpu().numpy(), T, bandwidth=bwv)
    np.testing.assert_allclose(v.cpu().numpy(), rv, rtol=1e-5, atol=1e-6)
    assert np.abs(m.cpu().numpy() - rm).max() <= 1e-4


def test_fused_ragged_and_split(cuda, parts):
    import d2p_amd
    x, y = _seeded(7, (5, 700, 24)), _seeded(8, (5, 110, 24))
    lens = torch.tensor([[700, 110], [0, 40], [193, 0], [1, 1], [257, 81]], dtype=torch.int32,
                        device=cuda)
    xc, yc = x.to(cuda), y.to(cuda)
    costs = torch.ops.d2p_amd.pairwise_sqdist(xc, yc)
    for n in (1, 4):
        parts(n)
        f = d2p_amd.soft_dtw_sqeuclidean(xc, yc, temperature=0.7, lengths=lens)
        p = d2p_amd.soft_dtw(costs, temperature=0.7, lengths=lens)
        assert torch.equal(f.cost, p.cost), n
        assert torch.equal(f.alignment, p.alignment), n


@pytest.mark.parametrize("B,L1,L2,D,n_parts", [(4, 256, 256, 64, 1), (2, 700, 110, 24, 4),
                                               (1, 200, 130, 128, 1), (3, 64, 90, 5, 1)])
def test_fused_helper_waves_bit_identical(cuda, parts, monkeypatch, B, L1, L2, D, n_parts):
    """Parts of at most four stripes move their data in helper waves in both sweeps;
    the arithmetic is unchanged, so every output equals the single-wave form bit for
    bit (split parts included)."""
    x, y = _seeded(31, (B, L1, D)).to(cuda), _seeded(32, (B, L2, D)).to(cuda)
    parts(n_parts)
    monkeypatch.setenv("D2P_AMD_DTW_HELPERS", "1")
    with_h = _capi.dtw_sqeuclid_forward_marginals(x, y, None, 0.3)
    monkeypatch.setenv("D2P_AMD_DTW_HELPERS", "0")
    without = _capi.dtw_sqeuclid_forward_marginals(x, y, None, 0.3)
    for a, b in zip(with_h, without):
        assert torch.equal(a, b)


def test_fused_rejects_bad_inputs(cuda):
    import d2p_amd
    x = torch.randn(2, 10, 8, device=cuda)
    with pytest.raises(RuntimeError, match="same feature dimension"):
        d2p_amd.soft_dtw_sqeuclidean(x, torch.randn(2, 10, 9, device=cuda))
    with pytest.raises(RuntimeError, match="same batch size"):
        d2p_amd.soft_dtw_sqeuclidean(x, torch.randn(3, 10, 8, device=cuda))
    with pytest.raises(RuntimeError, match="between 1 and 128"):
        d2p_amd.soft_dtw_sqeuclidean(torch.randn(1, 4, 129, device=cuda),
                                     torch.randn(1, 4, 129, device=cuda))



def test_fused_long_sequences(cuda):
    """No length limit beyond the sweeps' own: the costs are not staged in LDS."""
    import d2p_amd
    x, y = _seeded(41, (2, 300, 64)).to(cuda), _seeded(42, (2, 5000, 64)).to(cuda)
    f = d2p_amd.soft_dtw_sqeuclidean(x, y, temperature=0.5)
    p = d2p_amd.soft_dtw(torch.ops.d2p_amd.pairwise_sqdist(x, y), temperature=0.5)
    assert torch.equal(f.cost, p.cost) and torch.equal(f.alignment, p.alignment)


def _grad_refs(x, y, T, W=None):
    """float64 chain rule from the double oracle on the exact costs: the cost gradient
    G (value path: the marginals; marginal path: H W) and dL/dx, dL/dy."""
    c = _exact_costs(x, y).numpy()
    k64 = O.get("oracle64")
    if W is None:
        _, G, _ = k64.soft_dtw(c, T)
    else:
        G = k64.soft_dtw_hvp(c, W.numpy().astype(np.float64), T)
    G = torch.from_numpy(G)
    x64, y64 = x.double(), y.double()
    gx = 2 * (x64 * G.sum(2, keepdim=True) - torch.bmm(G, y64))
    Gt = G.transpose(1, 2).contiguous()
    gy = 2 * (y64 * Gt.sum(2, keepdim=True) - torch.bmm(Gt, x64))
    return G, gx, gy


def _check_grad(got, ref, eps, absdiff_rows, what):
    bound = 2 * eps * absdiff_rows + 1e-4
    err = (got.cpu().double() - ref).abs()
    assert torch.all(err <= bound), (what, float(err.max()), float((err / bound).max()))
    print(f"{what}: max err {float(err.max()):.2e} (bound ratio {float((err / bound).max()):.2f})")


@pytest.mark.parametrize("path", ["value", "marginal"])
def test_fused_gradients(cuda, path):
    import d2p_amd
    B, L1, L2, D, T = 2, 60, 70, 16, 1.0
    x, y = _seeded(11, (B, L1, D)), _seeded(12, (B, L2, D))
    W = _seeded(13, (B, L1, L2)) if path == "marginal" else None
    xc, yc = x.to(cuda).requires_grad_(True), y.to(cuda).requires_grad_(True)
    r = d2p_amd.soft_dtw_sqeuclidean(xc, yc, temperature=T)
    loss = r.cost.sum() if W is None else (r.alignment * W.to(cuda)).sum()
    loss.backward()
    G, gx, gy = _grad_refs(x, y, T, W)
    # eps: the GPU cost gradient's own distance from the double oracle
    if W is None:
        Gg = r.alignment.detach().cpu().double()
    else:
        costs = torch.ops.d2p_amd.pairwise_sqdist(x.to(cuda), y.to(cuda))
        Gg = d2p_amd.soft_dtw_backward_full(costs, W.to(cuda), T, None, -1)[0].cpu().double()
    eps = float((Gg - G).abs().max())
    assert eps <= 1e-4 * max(1.0, float(G.abs().max())), eps
    ad = (x.double()[:, :, None, :] - y.double()[:, None, :, :]).abs()   # [B, L1, L2, D]
    _check_grad(xc.grad, gx, eps, ad.sum(2), f"{path} dL/dx")
    _check_grad(yc.grad, gy, eps, ad.sum(1), f"{path} dL/dy")


def test_fused_temperature_gradient_and_autocast(cuda):
    import d2p_amd
    x, y = _seeded(21, (3, 40, 48, )), _seeded(22, (3, 44, 48))
    T = torch.tensor([0.8], device=cuda, requires_grad=True)
    r = d2p_amd.soft_dtw_sqeuclidean(x.to(cuda), y.to(cuda), temperature=T)
    r.cost.sum().backward()
    costs = torch.ops.d2p_amd.pairwise_sqdist(x.to(cuda), y.to(cuda))
    _, _, gT = _capi.dtw_forward_marginals(costs, None, 0.8)
    torch.testing.assert_close(T.grad, gT.sum().reshape(1), rtol=0, atol=0)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        rb = d2p_amd.soft_dtw_sqeuclidean(x.to(cuda).bfloat16(), y.to(cuda).bfloat16(), 0.8)
    assert rb.cost.dtype == torch.float32
    ref = d2p_amd.soft_dtw_sqeuclidean(x.to(cuda).bfloat16().float(),
                                       y.to(cuda).bfloat16().float(), 0.8)
    assert torch.equal(rb.cost, ref.cost)


@pytest.mark.parametrize("B,L1,L2,D,scaled", [(2, 256, 256, 64, True), (3, 70, 130, 5, False),
                                              (1, 1, 200, 128, True), (2, 65, 1, 32, False),
                                              (1, 300, 90, 100, True), (2, 64, 64, 1, False),
                                              (2, 300, 260, 36, True), (1, 129, 132, 128, False),
                                              (3, 33, 516, 20, True)])
def test_feature_grad_kernel(cuda, B, L1, L2, D, scaled):
    """d2p_amd::sqeuclid_feature_grad (one kernel, the products on the matrix cores)
    against the chain rule in float64: within the summation bound (K + 4) u |f|
    (|x_i| sum_j |G_ij| + sum_j |G_ij| |y_j|) per entry (K the contraction length),
    and equal to the C ABI entry point bit for bit."""
    import d2p_amd  # noqa: F401
    G, x, y = _seeded(51, (B, L1, L2)), _seeded(52, (B, L1, D)), _seeded(53, (B, L2, D))
    s = _seeded(54, (B,)) if scaled else None
    args = [G.to(cuda), x.to(cuda), y.to(cuda), s.to(cuda) if scaled else None]
    gx, gy = torch.ops.d2p_amd.sqeuclid_feature_grad(*args)
    cx, cy = _capi.sqeuclid_feature_grad(*args)
    assert torch.equal(gx, cx) and torch.equal(gy, cy)
    G64, x64, y64 = G.double(), x.double(), y.double()
    f = 2.0 * (s.double() if scaled else torch.ones(B, dtype=torch.float64))[:, None, None]
    ex = f * (x64 * G64.sum(2, keepdim=True) - torch.bmm(G64, y64))
    ey = f * (y64 * G64.sum(1)[:, :, None] - torch.bmm(G64.transpose(1, 2), x64))
    aG = G64.abs()
    bx = (L2 + 4) * U * f.abs() * (x64.abs() * aG.sum(2, keepdim=True) + torch.bmm(aG, y64.abs()))
    by = (L1 + 4) * U * f.abs() * (y64.abs() * aG.sum(1)[:, :, None] +
                                   torch.bmm(aG.transpose(1, 2), x64.abs()))
    for got, exact, bound, what in ((gx, ex, bx, "dL/dx"), (gy, ey, by, "dL/dy")):
        err = (got.cpu().double() - exact).abs()
        assert torch.all(err <= bound + 1e-30), (what, float((err / (bound + 1e-30)).max()))
        print(f"{what}: max err / bound {float((err / (bound + 1e-30)).max()):.3f}")
