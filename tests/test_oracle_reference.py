"""The CPU oracle against the reference's own CPU kernels, bit for bit.

``oracle/_ref/libd2p_ref.so`` is compiled by ``oracle/Makefile`` from
/root/reference/src/{sw,sw_affine,dtw,nw}/kernels_cpu.cpp where those sources
exist (this container); both libraries are built with -ffp-contract=off, so
every output of every function must be identical, including the regimes only
the reference's own rounding fixes: low temperature, |x / T| beyond the
exp clamp of 88, near-ties at large alpha (C4-style costs scaled by 128),
ragged lengths, empty elements and DTW bands.  Skipped where the reference
build is absent (the GPU box); the committed golden fixtures carry the same
evidence there.
"""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.skipif(not O.reference_available(),
                                reason="reference CPU build (oracle/_ref) absent")


def _rand(seed, shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def _same(a, b, what):
    a = a if isinstance(a, tuple) else (a,)
    b = b if isinstance(b, tuple) else (b,)
    for i, (x, y) in enumerate(zip(a, b)):
        x, y = np.asarray(x), np.asarray(y)
        assert x.shape == y.shape and np.array_equal(x.view(np.uint32), y.view(np.uint32)), \
            f"{what}[{i}]: max |diff| = {np.abs(x.astype(np.float64) - y).max():.3e}"


LENS = np.array([[20, 24], [7, 3], [0, 9], [20, 1], [1, 24]], np.int32)

SW_CASES = [
    # (seed, B, L1, L2, scale, gap, T, lengths)
    (0, 2, 16, 21, 1.0, -1.0, 1.0, None),
    (1, 5, 20, 24, 2.0, -0.5, 0.1, LENS),
    (2, 2, 12, 12, 60.0, -1.0, 0.5, None),     # |x / T| > 88: exp clamp active
    (3, 3, 9, 30, 1.0, 0.5, 2.0, None),        # positive gap
]


@pytest.mark.parametrize("seed,B,L1,L2,scale,gap,T,lens", SW_CASES)
def test_sw_bit_exact(seed, B, L1, L2, scale, gap, T, lens):
    o, r = O.get("oracle"), O.get("reference")
    s = _rand(seed, (B, L1, L2), scale)
    V = _rand(seed + 1, (B, L1, L2))
    _same(o.soft_sw(s, gap, T, lens), r.soft_sw(s, gap, T, lens), "soft_sw")
    _same(o.soft_sw_hvp(s, V, gap, T, lens), r.soft_sw_hvp(s, V, gap, T, lens), "hvp")
    for p in (0, 1):
        _same(o.soft_sw_param_jacobian(s, p, gap, T, lens),
              r.soft_sw_param_jacobian(s, p, gap, T, lens), f"jacobian {p}")


@pytest.mark.parametrize("seed,B,L1,L2,scale,gap,T,lens", SW_CASES)
def test_nw_bit_exact(seed, B, L1, L2, scale, gap, T, lens):
    o, r = O.get("oracle"), O.get("reference")
    s = _rand(seed + 70, (B, L1, L2), scale)
    _same(o.soft_nw(s, gap, T, lens), r.soft_nw(s, gap, T, lens), "soft_nw")
    V = _rand(seed + 71, (B, L1, L2))
    _same(o.soft_nw_hvp(s, V, gap, T, lens), r.soft_nw_hvp(s, V, gap, T, lens), "nw hvp")
    for p in (0, 1):
        _same(o.soft_nw_param_jacobian(s, p, gap, T, lens),
              r.soft_nw_param_jacobian(s, p, gap, T, lens), f"nw jacobian {p}")


@pytest.mark.parametrize("seed,B,L1,L2,scale,gap,T,lens", SW_CASES)
def test_nw_affine_bit_exact(seed, B, L1, L2, scale, gap, T, lens):
    o, r = O.get("oracle"), O.get("reference")
    s = _rand(seed + 80, (B, L1, L2), scale)
    go, ge = -3.0 * abs(gap), -0.5 * abs(gap)
    _same(o.soft_nw_affine(s, go, ge, T, lens), r.soft_nw_affine(s, go, ge, T, lens),
          "soft_nw_affine")
    alpha_o, _ = o.nwa_forward(s, lens, go, ge, T)
    alpha_r, _ = r.nwa_forward(s, lens, go, ge, T)
    _same(alpha_o, alpha_r, "nw_affine alpha")
    V = _rand(seed + 81, (B, L1, L2))
    _same(o.soft_nw_affine_hvp(s, V, go, ge, T, lens), r.soft_nw_affine_hvp(s, V, go, ge, T, lens),
          "nw_affine hvp")
    for p in (0, 1, 2):
        _same(o.soft_nw_affine_param_jacobian(s, p, go, ge, T, lens),
              r.soft_nw_affine_param_jacobian(s, p, go, ge, T, lens), f"nw_affine jacobian {p}")


@pytest.mark.parametrize("seed,B,L1,L2,scale,gap,T,lens", SW_CASES)
def test_affine_bit_exact(seed, B, L1, L2, scale, gap, T, lens):
    o, r = O.get("oracle"), O.get("reference")
    s = _rand(seed + 10, (B, L1, L2), scale)
    V = _rand(seed + 11, (B, L1, L2))
    go, ge = -11.0 * abs(gap), -1.0 * abs(gap)
    _same(o.soft_sw_affine(s, go, ge, T, lens), r.soft_sw_affine(s, go, ge, T, lens), "affine")
    _same(o.soft_sw_affine_hvp(s, V, go, ge, T, lens), r.soft_sw_affine_hvp(s, V, go, ge, T, lens),
          "hvp")
    for p in (0, 1, 2):
        _same(o.soft_sw_affine_param_jacobian(s, p, go, ge, T, lens),
              r.soft_sw_affine_param_jacobian(s, p, go, ge, T, lens), f"jacobian {p}")


DTW_CASES = [
    # (seed, B, L1, L2, scale, T, bandwidth, lengths)
    (0, 2, 16, 21, 1.0, 1.0, -1, None),
    (1, 5, 20, 24, 1.0, 0.1, -1, LENS),
    (2, 2, 18, 18, 128.0, 0.1, -1, None),      # C4-style costs: near-ties at large alpha
    (3, 2, 15, 22, 1.0, 0.5, 3, None),
    (4, 2, 12, 12, 1.0, 0.5, 0, None),
]


@pytest.mark.parametrize("seed,B,L1,L2,scale,T,bw,lens", DTW_CASES)
def test_dtw_bit_exact(seed, B, L1, L2, scale, T, bw, lens):
    o, r = O.get("oracle"), O.get("reference")
    c = np.abs(_rand(seed + 20, (B, L1, L2), scale))
    V = _rand(seed + 21, (B, L1, L2))
    _same(o.soft_dtw(c, T, lens, bw), r.soft_dtw(c, T, lens, bw), "soft_dtw")
    _same(o.soft_dtw_hvp(c, V, T, lens, bw), r.soft_dtw_hvp(c, V, T, lens, bw), "hvp")
    _same(o.soft_dtw_param_jacobian(c, T, lens, bw), r.soft_dtw_param_jacobian(c, T, lens, bw),
          "jacobian")


def test_config_c1_bit_exact():
    """Config C1: soft_sw on [2, 100, 120], gap -1, T 1."""
    o, r = O.get("oracle"), O.get("reference")
    s = _rand(42, (2, 100, 120))
    _same(o.soft_sw(s, -1.0, 1.0), r.soft_sw(s, -1.0, 1.0), "C1")
