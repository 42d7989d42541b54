"""Split elements: an element's stripes divided among several workgroups ("parts")
that hand the boundary row (forward) and the boundary flows (reverse sweep) to each
other through global memory -- linear-gap and affine-gap Smith-Waterman and
soft-DTW.

D2P_AMD_SPLIT=<n> forces n parts per element (1: never split); unset, the library
splits only long elements of small batches.  Every case is checked against the CPU
oracle to the north-star tolerances (value 1e-5 relative, marginals 1e-4
absolute, parameter gradients as in test_gpu_sw_linear), with the pipeline status
words required to stay 0 (no wait ran into its bound).  The HVP case checks that
the second-order entry points (primal sweeps, tangent sweep and two-channel reverse
sweep all split) stay within 1e-4 * max(1, max|H|), and the Jacobians and the
marginal-path backward within the allowances of test_gpu_sw_second.
"""
import numpy as np
import pytest
import torch

import _capi
from oracle import oracle as O
from test_gpu_sw_linear import _check, _seeded
from test_gpu_sw_second import _close, _jacobian_ref

pytestmark = pytest.mark.gpu


@pytest.fixture
def parts(monkeypatch):
    def force(n):
        monkeypatch.setenv("D2P_AMD_SPLIT", str(n))
    return force


CASES = [
    # (seed, B, L1, L2, parts)
    (20, 2, 600, 90, 1),       # unsplit, more stripes than waves
    (21, 1, 1100, 300, 1),     # unsplit, more than two rounds of waves
    (22, 1, 300, 200, 2),      # 5 stripes in parts of 3 and 2
    (23, 3, 500, 257, 8),      # one stripe per part
    (24, 2, 1300, 150, 2),     # parts of 11 and 10 stripes: several stripes per wave
    (25, 1, 1100, 2500, 2),    # long rows: 8-step backward chunks, parts of 9 stripes
    (26, 9, 200, 70, 4),       # B not a multiple of 8: idle workgroups in the grid
    (27, 2, 1024, 1024, 0),    # automatic choice (4 parts of 4 stripes)
    (28, 1, 129, 64, 3),       # last part of a single short stripe
]


@pytest.mark.parametrize("seed,B,L1,L2,n", CASES)
def test_sw_split_matches_oracle(cuda, parts, seed, B, L1, L2, n):
    parts(n)
    s = _seeded(seed, (B, L1, L2))
    ref = O.get("oracle").soft_sw(s.numpy(), -1.0, 1.0)
    out = _capi.sw_forward_marginals(s.to(cuda), None, -1.0, 1.0)
    torch.cuda.synchronize()
    _check(out, ref, scores=s.numpy())


def test_sw_split_ragged(cuda, parts):
    """Ragged lengths under 4 parts of 3 stripes: elements whose later parts hold no
    stripe, empty elements, and one-row elements."""
    parts(4)
    B, L1, L2 = 7, 700, 170
    s = _seeded(29, (B, L1, L2), 2.0)
    g = np.random.default_rng(29)
    lengths = np.stack([g.integers(0, L1 + 1, B), g.integers(0, L2 + 1, B)], 1).astype(np.int32)
    lengths[0] = [L1, L2]
    lengths[1] = [0, 5]
    lengths[2] = [640, 0]
    lengths[3] = [1, 1]
    lengths[4] = [193, 170]      # the first part only (stripes 0..3 of 11)
    ref = O.get("oracle").soft_sw(s.numpy(), -1.0, 0.5, lengths)
    out = _capi.sw_forward_marginals(s.to(cuda), torch.from_numpy(lengths).to(cuda), -1.0, 0.5)
    torch.cuda.synchronize()
    _check(out, ref, lengths=lengths, gap=-1.0, T=0.5, scores=s.numpy())


@pytest.mark.parametrize("B,L1,L2,n", [(2, 700, 260, 4), (3, 200, 300, 1), (1, 1500, 90, 8),
                                       (4, 64, 64, 1), (3, 512, 300, 1), (2, 330, 200, 1),
                                       (2, 1500, 90, 3), (3, 512, 512, 1), (2, 330, 208, 1),
                                       (3, 400, 64, 1), (2, 1500, 96, 3)])
def test_sw_helper_waves_bit_identical(cuda, parts, monkeypatch, B, L1, L2, n):
    """Parts hand their data movement (tile loads, the alpha table and marginal
    write-outs) to helper waves in the forward and reverse sweeps: the idle waves of the
    workgroup for parts of at most four stripes (also in the second-order reverse
    sweep), a second set of eight waves for parts of five to eight (the last three
    cases; those whose rows start 64-byte aligned, L2 a multiple of 16, also write the
    marginals as whole aligned row segments).  The arithmetic is unchanged, so every
    output equals the single-wave form
    bit for bit: SW and NW first order, the SW and NW HVPs, the SW parameter
    Jacobians, the marginal-path backward and affine SW first order, ragged lengths
    and split parts included."""
    s = _seeded(41, (B, L1, L2)).to(cuda)
    lens = torch.tensor([[max(1, L1 - 37 * i), max(1, L2 - 11 * i)] for i in range(B)],
                        dtype=torch.int32, device=cuda)
    V = _seeded(42, (B, L1, L2)).to(cuda)
    parts(n)
    out = {}
    for flag in ("1", "0"):
        monkeypatch.setenv("D2P_AMD_SW_HELPERS", flag)
        out[flag] = (list(_capi.sw_forward_marginals(s, lens, -1.0, 0.9)) +
                     list(_capi.nw_forward_marginals(s, lens, -1.0, 0.9)) +
                     [_capi.sw_hvp(s, V, lens, -1.0, 0.9), _capi.nw_hvp(s, V, lens, -1.0, 0.9),
                      _capi.sw_param_jacobian(s, 0, lens, -1.0, 0.9),
                      _capi.sw_param_jacobian(s, 1, lens, -1.0, 0.9)] +
                     list(_capi.sw_backward_full(s, V, lens, -1.0, 0.9)) +
                     list(_capi.swa_forward_marginals(s, lens, -3.0, -0.5, 0.9)))
    for i, (a, b) in enumerate(zip(out["1"], out["0"])):
        assert torch.equal(a, b), f"output {i}: max |diff| {float((a - b).abs().max()):.3e}"
    ref = O.get("oracle").soft_sw(s.cpu().numpy(), -1.0, 0.9, lens.cpu().numpy())
    np.testing.assert_allclose(out["1"][0].cpu().numpy(), ref[0], rtol=1e-5, atol=1e-6)


def test_sw_split_repeated_launches(cuda, parts):
    """Consecutive launches on one workspace: the progress words of one launch never
    satisfy the waits of the next (epochs), and the results repeat exactly."""
    parts(3)
    s = _seeded(30, (2, 700, 120)).to(cuda)
    first = _capi.sw_forward_marginals(s, None, -1.0, 1.0)
    for _ in range(3):
        again = _capi.sw_forward_marginals(s, None, -1.0, 1.0)
        for a, b in zip(first, again):
            torch.testing.assert_close(a, b, rtol=0, atol=0)


@pytest.mark.parametrize("n", [2, 3, 11])
def test_sw_split_hvp(cuda, parts, n):
    parts(n)
    s = _seeded(31, (2, 700, 90))
    v = _seeded(32, (2, 700, 90))
    ref = O.get("oracle").soft_sw_hvp(s.numpy(), v.numpy(), -1.0, 1.0)
    _close(_capi.sw_hvp(s.to(cuda), v.to(cuda), None, -1.0, 1.0), ref, f"hvp, {n} parts")


def test_sw_split_hvp_ragged(cuda, parts):
    parts(4)
    B, L1, L2 = 5, 700, 110
    s = _seeded(34, (B, L1, L2))
    v = _seeded(35, (B, L1, L2))
    lens = np.array([[700, 110], [0, 40], [193, 0], [1, 1], [257, 81]], np.int32)
    ref = O.get("oracle").soft_sw_hvp(s.numpy(), v.numpy(), -1.0, 0.7, lens)
    got = _capi.sw_hvp(s.to(cuda), v.to(cuda), torch.from_numpy(lens).to(cuda), -1.0, 0.7)
    _close(got, ref, "hvp ragged, 4 parts")


@pytest.mark.parametrize("n", [2, 4])
def test_sw_split_param_jacobian(cuda, parts, n):
    parts(n)
    s = _seeded(33, (2, 500, 80))
    k = O.get("oracle")
    for p in (0, 1):
        ref, allow = _jacobian_ref(k, s.numpy(), p, -1.0, 1.0)
        _close(_capi.sw_param_jacobian(s.to(cuda), p, None, -1.0, 1.0), ref,
               f"dP/d{('gap', 'T')[p]}, {n} parts", allow)


def test_sw_split_backward_full(cuda, parts):
    """The dot-product reverse sweeps (<ga, dP/dtheta>) sum their parts."""
    parts(3)
    B, L1, L2 = 2, 450, 96
    s = _seeded(36, (B, L1, L2))
    ga = _seeded(37, (B, L1, L2))
    k = O.get("oracle")
    gs, gg, gt = _capi.sw_backward_full(s.to(cuda), ga.to(cuda), None, -1.0, 1.0)
    _close(gs, k.soft_sw_hvp(s.numpy(), ga.numpy(), -1.0, 1.0), "backward_full scores")
    for p, g in ((0, gg), (1, gt)):
        J, allow = _jacobian_ref(k, s.numpy(), p, -1.0, 1.0)
        ref = (J.astype(np.float64) * ga.numpy()).sum(axis=(1, 2))
        per = 1e-4 * max(1.0, np.abs(J).max()) + allow
        tol = per * np.abs(ga.numpy()).sum(axis=(1, 2))
        assert np.all(np.abs(g.cpu().numpy() - ref) <= tol), (p, g.cpu().numpy(), ref, tol)


# ---------------------------------------------------------------- affine gap

AFFINE_CASES = [
    # (seed, B, L1, L2, gap_open, gap_ext, T, parts)
    (40, 2, 600, 90, -2.0, -0.5, 1.0, 1),     # unsplit, more stripes than waves
    (41, 1, 300, 200, -11.0, -1.0, 0.5, 2),   # parts of 3 and 2 stripes
    (42, 3, 500, 130, -2.0, -0.5, 1.0, 8),    # one stripe per part
    (43, 2, 1300, 150, -3.0, -1.0, 1.0, 2),   # several stripes per wave in each part
    (44, 9, 200, 70, -2.0, -0.5, 1.0, 4),     # idle workgroups in the grid
    (45, 2, 1024, 1024, -11.0, -1.0, 0.5, 0), # automatic choice (4 parts of 4 stripes)
]


@pytest.mark.parametrize("seed,B,L1,L2,go,ge,T,n", AFFINE_CASES)
def test_affine_split_matches_oracle(cuda, parts, seed, B, L1, L2, go, ge, T, n):
    from test_gpu_sw_affine import _check as _check_affine
    parts(n)
    s = _seeded(seed, (B, L1, L2), 2.0)
    ref = O.get("oracle").soft_sw_affine(s.numpy(), go, ge, T)
    gpu = _capi.swa_forward_marginals(s.to(cuda), None, go, ge, T)
    torch.cuda.synchronize()
    _check_affine(gpu, ref, s.numpy(), go, ge, T)


def test_affine_split_ragged(cuda, parts):
    """Config C3 style lengths under 4 parts: elements whose later parts are empty."""
    from test_gpu_sw_affine import _check as _check_affine
    parts(4)
    B, L1, L2 = 6, 700, 260
    s = _seeded(46, (B, L1, L2), 2.0)
    g = torch.Generator().manual_seed(47)
    lens = torch.randint(64, L1 + 1, (B, 2), generator=g, dtype=torch.int32)
    lens[:, 1] = torch.clamp(lens[:, 1], max=L2)
    lens[1] = torch.tensor([0, 100])
    lens[2] = torch.tensor([640, 0])
    lens[3] = torch.tensor([L1, L2])
    lens[4] = torch.tensor([150, 260])
    ref = O.get("oracle").soft_sw_affine(s.numpy(), -11.0, -1.0, 0.5, lens.numpy())
    gpu = _capi.swa_forward_marginals(s.to(cuda), lens.to(cuda), -11.0, -1.0, 0.5)
    torch.cuda.synchronize()
    _check_affine(gpu, ref, s.numpy(), -11.0, -1.0, 0.5, lens.tolist())


@pytest.mark.parametrize("n", [2, 3, 11])
def test_affine_split_hvp(cuda, parts, n):
    """Primal, tangent and two-channel reverse sweeps of the affine HVP all split."""
    from test_gpu_sw_affine_second import _close as _close_affine
    parts(n)
    s = _seeded(48, (2, 700, 90))
    v = _seeded(49, (2, 700, 90))
    ref = O.get("oracle").soft_sw_affine_hvp(s.numpy(), v.numpy(), -2.0, -0.5, 1.0)
    _close_affine(_capi.swa_hvp(s.to(cuda), v.to(cuda), None, -2.0, -0.5, 1.0), ref,
                  f"affine hvp, {n} parts")


def test_affine_split_hvp_ragged(cuda, parts):
    from test_gpu_sw_affine_second import _close as _close_affine
    parts(4)
    B, L1, L2 = 5, 700, 110
    s = _seeded(70, (B, L1, L2))
    v = _seeded(71, (B, L1, L2))
    lens = np.array([[700, 110], [0, 40], [193, 0], [1, 1], [257, 81]], np.int32)
    ref = O.get("oracle").soft_sw_affine_hvp(s.numpy(), v.numpy(), -2.0, -0.5, 0.7, lens)
    got = _capi.swa_hvp(s.to(cuda), v.to(cuda), torch.from_numpy(lens).to(cuda), -2.0, -0.5,
                        0.7)
    _close_affine(got, ref, "affine hvp ragged, 4 parts")


@pytest.mark.parametrize("n", [2, 4])
def test_affine_split_param_jacobian(cuda, parts, n):
    from test_gpu_sw_affine_second import _close as _close_affine
    from test_gpu_sw_affine_second import _jacobian_ref as _jacobian_affine
    parts(n)
    s = _seeded(72, (2, 500, 80))
    k = O.get("oracle")
    for p in (0, 1, 2):
        ref, allow = _jacobian_affine(k, s.numpy(), p, -2.0, -0.5, 1.0)
        _close_affine(_capi.swa_param_jacobian(s.to(cuda), p, None, -2.0, -0.5, 1.0), ref,
                      f"affine dP/d{('open', 'ext', 'T')[p]}, {n} parts", allow)


def test_affine_split_backward_full(cuda, parts):
    """The affine dot-product reverse sweeps sum their parts."""
    from test_gpu_sw_affine_second import _close as _close_affine
    from test_gpu_sw_affine_second import _jacobian_ref as _jacobian_affine
    parts(3)
    B, L1, L2 = 2, 450, 96
    go, ge, T = -2.0, -0.5, 1.0
    s = _seeded(73, (B, L1, L2))
    ga = _seeded(74, (B, L1, L2))
    k = O.get("oracle")
    gs, *gp = _capi.swa_backward_full(s.to(cuda), ga.to(cuda), None, go, ge, T)
    _close_affine(gs, k.soft_sw_affine_hvp(s.numpy(), ga.numpy(), go, ge, T),
                  "affine backward_full scores")
    for p, g in enumerate(gp):
        J, allow = _jacobian_affine(k, s.numpy(), p, go, ge, T)
        ref = (J.astype(np.float64) * ga.numpy()).sum(axis=(1, 2))
        per = 1e-4 * max(1.0, np.abs(J).max()) + allow
        tol = per * np.abs(ga.numpy()).sum(axis=(1, 2))
        assert np.all(np.abs(g.cpu().numpy() - ref) <= tol), (p, g.cpu().numpy(), ref, tol)


# ---------------------------------------------------------------- soft-DTW

DTW_CASES = [
    # (seed, B, L1, L2, T, bandwidth, parts)
    (50, 2, 600, 90, 1.0, -1, 1),      # unsplit, more stripes than waves
    (51, 1, 300, 200, 0.5, -1, 2),     # parts of 3 and 2 stripes
    (52, 3, 500, 130, 1.0, -1, 8),     # one stripe per part
    (53, 2, 1300, 150, 1.0, -1, 2),    # several stripes per wave in each part
    (54, 2, 700, 650, 1.0, 40, 3),     # Sakoe-Chiba band across parts
    (55, 1, 1100, 2500, 1.0, -1, 2),   # long rows: 8-step backward chunks
    (56, 2, 1024, 1024, 0.5, -1, 0),   # automatic choice (4 parts of 4 stripes)
]


@pytest.mark.parametrize("seed,B,L1,L2,T,bw,n", DTW_CASES)
def test_dtw_split_matches_oracle(cuda, parts, seed, B, L1, L2, T, bw, n):
    from test_gpu_dtw import _check as _check_dtw
    parts(n)
    c = _seeded(seed, (B, L1, L2)).abs()
    ref = O.get("oracle").soft_dtw(c.numpy(), T, None, bw)
    gpu = _capi.dtw_forward_marginals(c.to(cuda), None, T, bw)
    torch.cuda.synchronize()
    _check_dtw(gpu, ref, c.numpy(), T, bw)


def test_dtw_split_ragged(cuda, parts):
    """Ragged lengths under 4 parts: the terminal cell in any part, empty elements."""
    from test_gpu_dtw import _check as _check_dtw
    parts(4)
    B, L1, L2 = 6, 700, 170
    c = _seeded(57, (B, L1, L2)).abs()
    lens = torch.tensor([[700, 170], [0, 50], [640, 0], [0, 0], [193, 123], [1, 170]],
                        dtype=torch.int32)
    for bw in (-1, 30):
        ref = O.get("oracle").soft_dtw(c.numpy(), 0.7, lens.numpy(), bw)
        gpu = _capi.dtw_forward_marginals(c.to(cuda), lens.to(cuda), 0.7, bw)
        torch.cuda.synchronize()
        _check_dtw(gpu, ref, c.numpy(), 0.7, bw, lens.tolist())


@pytest.mark.parametrize("n,bw", [(2, -1), (3, 40), (11, -1)])
def test_dtw_split_hvp(cuda, parts, n, bw):
    """Primal, tangent and two-channel reverse sweeps of the soft-DTW HVP all split."""
    from test_gpu_dtw_second import _close as _close_dtw
    parts(n)
    c = _seeded(75, (2, 700, 90)).abs()
    v = _seeded(76, (2, 700, 90))
    ref = O.get("oracle").soft_dtw_hvp(c.numpy(), v.numpy(), 0.8, None, bw)
    _close_dtw(_capi.dtw_hvp(c.to(cuda), v.to(cuda), None, 0.8, bw), ref,
               f"dtw hvp, {n} parts, band {bw}")


def test_dtw_split_second_ragged(cuda, parts):
    from test_gpu_dtw_second import _close as _close_dtw, _jac_allow
    parts(4)
    B, L1, L2 = 5, 700, 110
    c = _seeded(77, (B, L1, L2)).abs()
    v = _seeded(78, (B, L1, L2))
    lens = np.array([[700, 110], [0, 40], [193, 0], [1, 1], [257, 81]], np.int32)
    lt = torch.from_numpy(lens).to(cuda)
    k = O.get("oracle")
    for bw in (-1, 30):
        _close_dtw(_capi.dtw_hvp(c.to(cuda), v.to(cuda), lt, 0.7, bw),
                   k.soft_dtw_hvp(c.numpy(), v.numpy(), 0.7, lens, bw),
                   f"dtw hvp ragged, 4 parts, band {bw}")
        _close_dtw(_capi.dtw_param_jacobian(c.to(cuda), lt, 0.7, bw),
                   k.soft_dtw_param_jacobian(c.numpy(), 0.7, lens, bw),
                   f"dtw jacobian ragged, 4 parts, band {bw}",
                   _jac_allow(k, c.numpy(), 0.7, lens, bw))


@pytest.mark.parametrize("n", [2, 4])
def test_dtw_split_param_jacobian(cuda, parts, n):
    from test_gpu_dtw_second import _close as _close_dtw, _jac_allow
    parts(n)
    c = _seeded(79, (2, 500, 80)).abs()
    k = O.get("oracle")
    _close_dtw(_capi.dtw_param_jacobian(c.to(cuda), None, 1.0, -1),
               k.soft_dtw_param_jacobian(c.numpy(), 1.0, None, -1), f"dtw dP/dT, {n} parts",
               _jac_allow(k, c.numpy(), 1.0))


def test_dtw_split_backward_full(cuda, parts):
    """The soft-DTW dot-product reverse sweep (<W, dP/dT>) sums its parts."""
    from test_gpu_dtw_second import _close as _close_dtw, _jac_allow
    parts(3)
    B, L1, L2 = 2, 450, 96
    c = _seeded(80, (B, L1, L2)).abs()
    W = _seeded(81, (B, L1, L2))
    k = O.get("oracle")
    gc, gt = _capi.dtw_backward_full(c.to(cuda), W.to(cuda), None, 0.8)
    _close_dtw(gc, k.soft_dtw_hvp(c.numpy(), W.numpy(), 0.8), "dtw backward_full costs")
    J = k.soft_dtw_param_jacobian(c.numpy(), 0.8)
    ref = (J.astype(np.float64) * W.numpy()).sum(axis=(1, 2))
    per = 1e-4 * max(1.0, np.abs(J).max()) + _jac_allow(k, c.numpy(), 0.8)
    tol = per * np.abs(W.numpy()).sum(axis=(1, 2))
    got = gt.cpu().numpy()
    assert np.all(np.abs(got - ref) <= tol), (got, ref, tol)


# ------------------------------------------------- rows too long for unsplit rings

# An unsplit element with more stripes than waves needs stripe rings about a row
# long; when they do not fit in LDS the launch splits the element into parts of at
# most 8 stripes, whose minimum rings always fit -- also when D2P_AMD_SPLIT=1.
@pytest.mark.parametrize("n", [0, 1])
def test_sw_long_rows_force_parts(cuda, parts, n):
    parts(n)
    s = _seeded(60, (1, 600, 12000))
    ref = O.get("oracle").soft_sw(s.numpy(), -1.0, 1.0)
    out = _capi.sw_forward_marginals(s.to(cuda), None, -1.0, 1.0)
    torch.cuda.synchronize()
    _check(out, ref, scores=s.numpy())


def test_sw_hvp_long_rows_force_parts(cuda, parts):
    parts(1)
    s = _seeded(61, (1, 600, 6000))
    v = _seeded(62, (1, 600, 6000))
    ref = O.get("oracle").soft_sw_hvp(s.numpy(), v.numpy(), -1.0, 1.0)
    _close(_capi.sw_hvp(s.to(cuda), v.to(cuda), None, -1.0, 1.0), ref, "hvp, 600 x 6000")


def test_affine_long_rows_force_parts(cuda, parts):
    from test_gpu_sw_affine import _check as _check_affine
    parts(1)
    s = _seeded(63, (1, 600, 4000), 2.0)
    ref = O.get("oracle").soft_sw_affine(s.numpy(), -11.0, -1.0, 0.5)
    gpu = _capi.swa_forward_marginals(s.to(cuda), None, -11.0, -1.0, 0.5)
    torch.cuda.synchronize()
    _check_affine(gpu, ref, s.numpy(), -11.0, -1.0, 0.5)


def test_dtw_long_rows_force_parts(cuda, parts):
    from test_gpu_dtw import _check as _check_dtw
    parts(1)
    c = _seeded(64, (1, 600, 12000)).abs()
    ref = O.get("oracle").soft_dtw(c.numpy(), 1.0, None, -1)
    gpu = _capi.dtw_forward_marginals(c.to(cuda), None, 1.0, -1)
    torch.cuda.synchronize()
    _check_dtw(gpu, ref, c.numpy(), 1.0, -1)


def test_affine_hvp_long_rows_force_parts(cuda, parts):
    from test_gpu_sw_affine_second import _close as _close_affine
    parts(1)
    s = _seeded(65, (1, 600, 3000))
    v = _seeded(66, (1, 600, 3000))
    ref = O.get("oracle").soft_sw_affine_hvp(s.numpy(), v.numpy(), -2.0, -0.5, 1.0)
    _close_affine(_capi.swa_hvp(s.to(cuda), v.to(cuda), None, -2.0, -0.5, 1.0), ref,
                  "affine hvp, 600 x 3000")


def test_dtw_hvp_long_rows_force_parts(cuda, parts):
    # 6000-column rows: the float32 oracle is itself up to 3e-2 from the exact HVP
    # here (130761 entries beyond 1e-4 max(1, |x|)), so the GPU is held to the
    # double-precision oracle under the long-element rule
    from _parity import check_vs_exact
    parts(1)
    c = _seeded(67, (1, 600, 6000)).abs()
    v = _seeded(68, (1, 600, 6000))
    ref32 = O.get("oracle").soft_dtw_hvp(c.numpy(), v.numpy(), 1.0, None, -1)
    exact = O.get("oracle64").soft_dtw_hvp(c.numpy().astype(np.float64),
                                           v.numpy().astype(np.float64), 1.0, None, -1)
    e_gpu, e_ref = check_vs_exact(_capi.dtw_hvp(c.to(cuda), v.to(cuda), None, 1.0, -1), exact,
                                  ref32, "dtw hvp, 600 x 6000")
    print(f"dtw hvp 600 x 6000: |gpu - exact| {e_gpu:.3e}, |fp32 oracle - exact| {e_ref:.3e}")
