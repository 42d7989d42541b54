"""Pins the CPU oracle (oracle/d2p_oracle.c) by mathematics alone, without the
reference's code:

* closed forms: 1x1 SW / affine S = T log(1 + e^{s/T}); DTW 1x1, 1xN and Nx1
  values are cost sums with all-ones posteriors (the known answers of
  /root/reference/tests/test_soft_dtw.py:503-536);
* brute-force path enumeration on grids up to 3x3 (SW, affine, DTW);
* a float64 restatement of the recurrences with autograd derivatives
  (tests/mathref.py) for values, marginals, parameter gradients, Hessian-vector
  products and parameter Jacobians, on full and ragged batches and DTW bands;
* limits and invariants: hard-max limit as T -> 0 (bounded by T log(#paths)),
  marginals in [0, 1], zero padding, lengths equal to slicing, HVP symmetry and
  linearity, bit-identical results for every thread count;
* the worked example of /root/reference/docs/algorithms/sw.md:67-101.
A plausible slip in the oracle (a dropped candidate, a wrong sign, a swapped
operand or index) moves at least one of these by far more than its tolerance.
"""
import math

import numpy as np
import pytest

import mathref as M
from oracle import oracle as O


def _k():
    return O.get("oracle")


def _rand(seed, shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def _close(got, want, atol, rtol=0.0, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    tol = atol + rtol * np.abs(want)
    assert np.all(err <= tol), f"{what}: max err {err.max():.3e} (tol {tol.max():.3e})"


# ------------------------------------------------------------------ closed forms

@pytest.mark.parametrize("s", [-3.0, -0.5, 0.0, 0.7, 4.0])
@pytest.mark.parametrize("T", [0.1, 0.5, 1.0, 3.0])
def test_sw_1x1_closed_form(s, T):
    x = np.full((1, 1, 1), s, np.float32)
    S = T * np.logaddexp(0.0, np.float64(np.float32(s)) / T)
    sig = 1.0 / (1.0 + math.exp(-float(np.float32(s)) / T))
    dT = S / T - float(np.float32(s)) / T * sig
    for part, post, *grads in (_k().soft_sw(x, -1.0, T), _k().soft_sw_affine(x, -2.0, -0.5, T)):
        _close(part, [S], 2e-6, 2e-6, "1x1 value")
        _close(post, [[[sig]]], 2e-6, 0, "1x1 marginal")
        for g in grads[:-1]:                      # gap gradients: no gap can occur
            assert float(g[0]) == 0.0
        # dS/dT = (S - s P) / T cancels: fp32 rounding of S and s P over T
        _close(grads[-1], [dT], 2e-6 + 2e-6 * (abs(S) + abs(s)) / T, 0, "1x1 dS/dT")


@pytest.mark.parametrize("shape", [(1, 1), (1, 3), (3, 1), (1, 7), (5, 1)])
def test_dtw_single_path_closed_form(shape):
    c = np.abs(_rand(3, (1,) + shape)) + 0.1
    for T in (0.1, 1.0, 10.0):
        score, post, gt = _k().soft_dtw(c, T)
        _close(score, [c.astype(np.float64).sum()], 1e-6, 1e-6, "single-path value")
        assert np.all(post == 1.0)
        # one path: dS/dT = 0 up to the fp32 rounding of softmin - E[alpha] over T
        assert abs(float(gt[0])) <= 2e-6 * (1.0 + float(c.sum()) / T)


def test_dtw_reference_known_answers():
    """/root/reference/tests/test_soft_dtw.py:503-536."""
    score, post, _ = _k().soft_dtw(np.array([[[0.5]]], np.float32), 1.0)
    assert float(score[0]) == pytest.approx(0.5) and float(post[0, 0, 0]) == 1.0
    for c in (np.array([[[0.1, 0.2, 0.3]]], np.float32), np.array([[[0.1], [0.2], [0.3]]],
                                                                   np.float32)):
        score, post, _ = _k().soft_dtw(c, 1.0)
        assert float(score[0]) == pytest.approx(0.6, abs=1e-6)
        assert np.allclose(post, 1.0)


# ------------------------------------------------------------------ brute force

SMALL = [(1, 2), (2, 1), (2, 2), (2, 3), (3, 2), (3, 3)]


@pytest.mark.parametrize("shape", SMALL)
@pytest.mark.parametrize("T", [0.3, 1.0])
def test_values_against_path_enumeration(shape, T):
    s = _rand(hash(shape) % 1000, (1,) + shape)
    c = np.abs(s) + 0.05
    S_sw = M.sw_brute(s[0], -0.7, T)
    S_swa = M.swa_brute(s[0], -1.3, -0.4, T)
    S_dtw = M.dtw_brute(c[0], T)
    S_nw = M.nw_brute(s[0], -0.7, T)
    _close(_k().soft_nw(s, -0.7, T)[0], [S_nw], 2e-6, 2e-6, "NW vs paths")
    _close(_k().soft_sw(s, -0.7, T)[0], [S_sw], 2e-6, 2e-6, "SW vs paths")
    _close(_k().soft_sw_affine(s, -1.3, -0.4, T)[0], [S_swa], 2e-6, 2e-6, "affine vs paths")
    _close(_k().soft_dtw(c, T)[0], [S_dtw], 2e-6, 2e-6, "DTW vs paths")
    # the float64 restatement agrees with the enumeration to rounding
    t = lambda a: M.torch.as_tensor(a, dtype=M.D)  # noqa: E731
    assert float(M.sw_value(t(s[0]), t(-0.7), t(T))) == pytest.approx(S_sw, rel=1e-12)
    assert float(M.swa_value(t(s[0]), t(-1.3), t(-0.4), t(T))) == pytest.approx(S_swa, rel=1e-12)
    assert float(M.dtw_value(t(c[0]), t(T))) == pytest.approx(S_dtw, rel=1e-12)
    assert float(M.nw_value(t(s[0]), t(-0.7), t(T))) == pytest.approx(S_nw, rel=1e-12)


@pytest.mark.parametrize("s", [-3.0, 0.0, 2.5])
@pytest.mark.parametrize("gap", [-1.0, 0.5])
@pytest.mark.parametrize("T", [0.2, 1.0])
def test_nw_1x1_closed_form(s, gap, T):
    """1x1 global alignment: the diagonal (s) or a down and a right move in either
    order (2 gap each): S = T log(e^{s/T} + 2 e^{2 gap/T}); P = the diagonal's share;
    dS/dgap = 2 (1 - P)."""
    x = np.full((1, 1, 1), s, np.float32)
    S, P, gg, gt = _k().soft_nw(x, gap, T)
    ed, eg = math.exp(s / T), 2 * math.exp(2 * gap / T)
    _close(S, [T * math.log(ed + eg)], 1e-5, 1e-6, "value")
    _close(P, [[[ed / (ed + eg)]]], 1e-6, 0, "marginal")
    _close(gg, [2 * eg / (ed + eg)], 1e-5, 1e-5, "dS/dgap")


# ------------------------------------------------------------------ float64 restatement

FIRST = [
    # (seed, B, L1, L2, T, lengths)
    (0, 1, 5, 7, 1.0, None),
    (1, 2, 8, 6, 0.5, None),
    (2, 3, 6, 7, 2.0, [[6, 7], [3, 5], [0, 4]]),
    (3, 2, 4, 9, 0.25, [[4, 9], [1, 1]]),
]


@pytest.mark.parametrize("seed,B,L1,L2,T,lens", FIRST)
def test_sw_first_order_against_math(seed, B, L1, L2, T, lens):
    s = _rand(seed, (B, L1, L2))
    ln = None if lens is None else np.array(lens, np.int32)
    part, post, gg, gt = _k().soft_sw(s, -0.8, T, ln)
    v, m, mg, mt = M.sw(s, -0.8, T, ln)
    _close(part, v, 1e-5, 1e-6, "value")
    _close(post, m, 2e-5, 0, "marginals")
    _close(gg, mg, 1e-4, 1e-4, "dS/dgap")
    _close(gt, mt, 1e-4, 1e-4, "dS/dT")


@pytest.mark.parametrize("seed,B,L1,L2,T,lens", FIRST)
def test_swa_first_order_against_math(seed, B, L1, L2, T, lens):
    s = _rand(seed + 10, (B, L1, L2))
    ln = None if lens is None else np.array(lens, np.int32)
    part, post, g_o, g_e, gt = _k().soft_sw_affine(s, -1.5, -0.4, T, ln)
    v, m, mo, me, mt = M.swa(s, -1.5, -0.4, T, ln)
    _close(part, v, 1e-5, 1e-6, "value")
    _close(post, m, 2e-5, 0, "marginals")
    _close(g_o, mo, 1e-4, 1e-4, "dS/dopen")
    _close(g_e, me, 1e-4, 1e-4, "dS/dext")
    _close(gt, mt, 1e-4, 1e-4, "dS/dT")


@pytest.mark.parametrize("seed,B,L1,L2,T,lens", FIRST)
def test_nw_first_order_against_math(seed, B, L1, L2, T, lens):
    s = _rand(seed + 60, (B, L1, L2))
    ln = None if lens is None else np.array(lens, np.int32)
    v, post, gg, gt = _k().soft_nw(s, -0.8, T, ln)
    mv, m, mg, mt = M.nw(s, -0.8, T, ln)
    _close(v, mv, 1e-5, 1e-6, "value")
    _close(post, m, 2e-5, 0, "marginals")
    _close(gg, mg, 1e-4, 1e-4, "dS/dgap")
    _close(gt, mt, 1e-4, 1e-4, "dS/dT")


DTW_FIRST = [
    # (seed, B, L1, L2, T, bandwidth, lengths)
    (0, 1, 5, 7, 1.0, -1, None),
    (1, 2, 8, 6, 0.1, -1, None),
    (2, 2, 7, 7, 0.5, 1, None),
    (3, 2, 6, 9, 1.0, 2, None),
    (4, 3, 6, 7, 0.7, -1, [[6, 7], [3, 5], [2, 1]]),
    (5, 2, 6, 6, 0.5, 0, None),
]


@pytest.mark.parametrize("seed,B,L1,L2,T,bw,lens", DTW_FIRST)
def test_dtw_first_order_against_math(seed, B, L1, L2, T, bw, lens):
    c = np.abs(_rand(seed + 20, (B, L1, L2))) + 0.05
    ln = None if lens is None else np.array(lens, np.int32)
    score, post, gt = _k().soft_dtw(c, T, ln, bw)
    v, m, mt = M.dtw(c, T, bw, ln)
    _close(score, v, 1e-5, 1e-6, "value")
    _close(post, m, 2e-5, 0, "marginals")
    _close(gt, mt, 1e-4, 1e-4, "dS/dT")


SECOND = [(0, 1, 5, 6, 1.0, None), (1, 2, 6, 5, 0.5, None),
          (2, 2, 6, 7, 1.5, [[6, 7], [2, 4]])]


@pytest.mark.parametrize("seed,B,L1,L2,T,lens", SECOND)
def test_hvp_against_math(seed, B, L1, L2, T, lens):
    s = _rand(seed + 30, (B, L1, L2))
    V = _rand(seed + 31, (B, L1, L2))
    c = np.abs(s) + 0.05
    ln = None if lens is None else np.array(lens, np.int32)
    for got, want in (
            (_k().soft_sw_hvp(s, V, -0.8, T, ln), M.hvp("sw", s, V, (-0.8, T), ln)),
            (_k().soft_sw_affine_hvp(s, V, -1.5, -0.4, T, ln),
             M.hvp("swa", s, V, (-1.5, -0.4, T), ln)),
            (_k().soft_dtw_hvp(c, V, T, ln), M.hvp("dtw", c, V, (T,), ln)),
            (_k().soft_nw_hvp(s, V, -0.8, T, ln), M.hvp("nw", s, V, (-0.8, T), ln))):
        _close(got, want, 1e-4 * max(1.0, np.abs(want).max()), 0, "hvp")


@pytest.mark.parametrize("seed,B,L1,L2,T,lens", SECOND)
def test_param_jacobians_against_math(seed, B, L1, L2, T, lens):
    s = _rand(seed + 40, (B, L1, L2))
    c = np.abs(s) + 0.05
    ln = None if lens is None else np.array(lens, np.int32)
    pairs = [(_k().soft_sw_param_jacobian(s, p, -0.8, T, ln),
              M.param_jacobian("sw", s, (-0.8, T), p, ln)) for p in (0, 1)]
    pairs += [(_k().soft_sw_affine_param_jacobian(s, p, -1.5, -0.4, T, ln),
               M.param_jacobian("swa", s, (-1.5, -0.4, T), p, ln)) for p in (0, 1, 2)]
    pairs += [(_k().soft_dtw_param_jacobian(c, T, ln), M.param_jacobian("dtw", c, (T,), 0, ln))]
    pairs += [(_k().soft_nw_param_jacobian(s, p, -0.8, T, ln),
               M.param_jacobian("nw", s, (-0.8, T), p, ln)) for p in (0, 1)]
    for i, (got, want) in enumerate(pairs):
        _close(got, want, 2e-4 * max(1.0, np.abs(want).max()), 0, f"jacobian {i}")


def test_dtw_band_second_order_against_math():
    c = np.abs(_rand(50, (2, 7, 8))) + 0.05
    V = _rand(51, (2, 7, 8))
    _close(_k().soft_dtw_hvp(c, V, 0.5, None, 2), M.hvp("dtw", c, V, (0.5,), None, 2), 1e-4,
           0, "banded hvp")
    _close(_k().soft_dtw_param_jacobian(c, 0.5, None, 2),
           M.param_jacobian("dtw", c, (0.5,), 0, None, 2), 2e-4, 0, "banded jacobian")


# ------------------------------------------------------------------ limits, invariants

def _hard_sw(s, gap):
    L1, L2 = s.shape
    H = np.full((L1 + 1, L2 + 1), -np.inf)
    N = np.zeros((L1 + 1, L2 + 1))             # number of paths ending at each cell
    for i in range(1, L1 + 1):
        for j in range(1, L2 + 1):
            x = float(s[i - 1, j - 1])
            c = [x]
            n = 1.0
            if i > 1 and j > 1:
                c.append(H[i - 1, j - 1] + x)
                n += N[i - 1, j - 1]
            if i > 1:
                c.append(H[i - 1, j] + gap)
                n += N[i - 1, j]
            if j > 1:
                c.append(H[i, j - 1] + gap)
                n += N[i, j - 1]
            H[i, j] = max(c)
            N[i, j] = n
    return max(0.0, H[1:, 1:].max()), N.sum()


def _hard_dtw(c):
    L1, L2 = c.shape
    A = np.full((L1 + 1, L2 + 1), np.inf)
    N = np.zeros((L1 + 1, L2 + 1))
    A[0, 0], N[0, 0] = 0.0, 1.0
    for i in range(1, L1 + 1):
        for j in range(1, L2 + 1):
            A[i, j] = c[i - 1, j - 1] + min(A[i - 1, j - 1], A[i - 1, j], A[i, j - 1])
            N[i, j] = N[i - 1, j - 1] + N[i - 1, j] + N[i, j - 1]
    return A[L1, L2], N[L1, L2]


@pytest.mark.parametrize("T", [0.05, 0.01])
def test_hard_limit(T):
    s = _rand(60, (2, 6, 8), 2.0)
    S = _k().soft_sw(s, -1.0, T)[0]
    for b in range(2):
        hard, npaths = _hard_sw(s[b], -1.0)
        assert hard - 1e-4 <= S[b] <= hard + T * math.log1p(npaths) + 1e-4
    c = np.abs(s) + 0.1
    D = _k().soft_dtw(c, T)[0]
    for b in range(2):
        hard, npaths = _hard_dtw(c[b])
        assert hard - T * math.log(npaths) - 1e-4 <= D[b] <= hard + 1e-4


def test_marginals_range_and_padding():
    s = _rand(70, (3, 20, 24), 2.0)
    ln = np.array([[20, 24], [11, 7], [0, 5]], np.int32)
    for post in (_k().soft_sw(s, -1.0, 0.7, ln)[1], _k().soft_sw_affine(s, -2, -0.5, 0.7, ln)[1],
                 _k().soft_dtw(np.abs(s), 0.7, ln)[1]):
        assert post.min() >= 0.0 and post.max() <= 1.0 + 1e-6
        for b, (l1, l2) in enumerate(ln):
            assert np.all(post[b, l1:, :] == 0.0) and np.all(post[b, :, l2:] == 0.0)


def test_lengths_equal_slicing():
    s = _rand(80, (1, 17, 23))
    ln = np.array([[11, 14]], np.int32)
    sl = np.ascontiguousarray(s[:, :11, :14])
    for full, cut in ((_k().soft_sw(s, -1.0, 0.6, ln), _k().soft_sw(sl, -1.0, 0.6)),
                      (_k().soft_sw_affine(s, -2, -0.5, 0.6, ln),
                       _k().soft_sw_affine(sl, -2, -0.5, 0.6)),
                      (_k().soft_dtw(np.abs(s), 0.6, ln), _k().soft_dtw(np.abs(sl), 0.6))):
        assert np.array_equal(full[0], cut[0])
        assert np.array_equal(full[1][:, :11, :14], cut[1])
        for a, b in zip(full[2:], cut[2:]):
            assert np.array_equal(a, b)


def test_hvp_symmetry_and_linearity():
    s = _rand(90, (1, 12, 14))
    u = _rand(91, (1, 12, 14))
    v = _rand(92, (1, 12, 14))
    for f in (lambda x: _k().soft_sw_hvp(s, x, -1.0, 0.8),
              lambda x: _k().soft_sw_affine_hvp(s, x, -2.0, -0.5, 0.8),
              lambda x: _k().soft_dtw_hvp(np.abs(s) + 0.1, x, 0.8)):
        Hu, Hv = f(u).astype(np.float64), f(v).astype(np.float64)
        a, b = float((u * Hv).sum()), float((v * Hu).sum())
        assert abs(a - b) <= 1e-4 * max(1.0, abs(a))
        lin = f((2.0 * u - 0.5 * v).astype(np.float32)).astype(np.float64)
        _close(lin, 2.0 * Hu - 0.5 * Hv, 1e-4 * max(1.0, np.abs(lin).max()), 0, "linearity")


def test_thread_count_invariance():
    s = _rand(100, (8, 24, 20))
    outs = []
    for n in (1, 2, 4, 8):
        O.set_threads(n)
        k = _k()
        outs.append((k.soft_sw(s, -1.0, 0.9), k.soft_sw_affine(s, -2.0, -0.5, 0.9),
                     k.soft_dtw(np.abs(s), 0.9), k.soft_sw_hvp(s, s, -1.0, 0.9)))
    O.set_threads(8)
    ref = outs[0]
    for o in outs[1:]:
        for a, b in zip(ref, o):
            for x, y in zip(a if isinstance(a, tuple) else (a,), b if isinstance(b, tuple) else (b,)):
                assert np.array_equal(x, y)


def test_worked_example_motif():
    """The SW worked example: motif ACGTA inside different flanks, +1 match, -1
    mismatch, gap -1, T = 0.5; marginals of the motif diagonal are 0.87, 0.97, 0.98,
    0.97, 0.87 and the flanks carry almost no mass (0.01, 0.10, ..., 0.11, 0.01)."""
    seq1, seq2 = "TTACGTAGG", "CACGTATT"
    a = np.array([ord(ch) for ch in seq1])
    b = np.array([ord(ch) for ch in seq2])
    s = (2.0 * (a[:, None] == b[None, :]) - 1.0).astype(np.float32)[None]
    m = _k().soft_sw(s, -1.0, 0.5)[1][0]
    want = [(0, 0, 0.01), (1, 0, 0.10), (2, 1, 0.87), (3, 2, 0.97), (4, 3, 0.98),
            (5, 4, 0.97), (6, 5, 0.87), (7, 6, 0.11), (8, 7, 0.01)]
    for i, j, mass in want:
        assert int(m[i].argmax()) == j
        assert round(float(m[i, j]), 2) == mass


def test_double_summed_parameter_gradients_against_math():
    """oracle param_grads64 (the reference's per-cell terms summed in double, used by
    the GPU parity tests) against the float64 restatement."""
    s = _rand(110, (2, 9, 11))
    c = np.abs(s) + 0.05
    ln = np.array([[9, 11], [5, 7]], np.int32)
    g = _k().param_grads64("sw", s, ln, -0.8, 0.7)
    _, _, mg, mt = M.sw(s, -0.8, 0.7, ln)
    _close(g[:, 0], mg, 2e-5, 2e-5, "sums64 gap")
    _close(g[:, 1], mt, 2e-5, 2e-5, "sums64 T")
    g = _k().param_grads64("swa", s, ln, -1.5, -0.4, 0.7)
    _, _, mo, me, mt = M.swa(s, -1.5, -0.4, 0.7, ln)
    for k, want in enumerate((mo, me, mt)):
        _close(g[:, k], want, 2e-5, 2e-5, f"sums64 affine {k}")
    g = _k().param_grads64("dtw", c, ln, 0.7)
    _close(g, M.dtw(c, 0.7, -1, ln)[2], 2e-5, 2e-5, "sums64 dtw")


# ------------------------------------------------------ the double-precision build

def _k64():
    return O.get("oracle64")


@pytest.mark.parametrize("seed,B,L1,L2,T,lens", SECOND)
def test_oracle64_against_math(seed, B, L1, L2, T, lens):
    """liboracle64.so (the restatement compiled in double) matches the float64
    autograd restatement to near double precision: values, marginals, HVPs and
    every parameter Jacobian.  The GPU tests of long elements use it as the exact
    value against which both the GPU's and the fp32 reference's errors are measured."""
    s = _rand(seed + 40, (B, L1, L2)).astype(np.float64)
    V = _rand(seed + 41, (B, L1, L2)).astype(np.float64)
    c = np.abs(s) + 0.05
    ln = None if lens is None else np.array(lens, np.int32)
    k = _k64()
    pairs = [(k.soft_sw(s, -0.8, T, ln), M.sw(s, -0.8, T, ln)),
             (k.soft_sw_affine(s, -1.5, -0.4, T, ln), M.swa(s, -1.5, -0.4, T, ln)),
             (k.soft_dtw(c, T, ln), M.dtw(c, T, -1, ln)),
             (k.soft_nw(s, -0.8, T, ln), M.nw(s, -0.8, T, ln))]
    for got, want in pairs:
        for g, w in zip(got, want):
            _close(g, w, 1e-9 * max(1.0, np.abs(w).max()), 0, "first order")
    pairs = [(k.soft_sw_hvp(s, V, -0.8, T, ln), M.hvp("sw", s, V, (-0.8, T), ln)),
             (k.soft_sw_affine_hvp(s, V, -1.5, -0.4, T, ln),
              M.hvp("swa", s, V, (-1.5, -0.4, T), ln)),
             (k.soft_dtw_hvp(c, V, T, ln), M.hvp("dtw", c, V, (T,), ln))]
    pairs += [(k.soft_sw_param_jacobian(s, p, -0.8, T, ln),
               M.param_jacobian("sw", s, (-0.8, T), p, ln)) for p in (0, 1)]
    pairs += [(k.soft_sw_affine_param_jacobian(s, p, -1.5, -0.4, T, ln),
               M.param_jacobian("swa", s, (-1.5, -0.4, T), p, ln)) for p in (0, 1, 2)]
    pairs += [(k.soft_dtw_param_jacobian(c, T, ln), M.param_jacobian("dtw", c, (T,), 0, ln))]
    pairs += [(k.soft_nw_hvp(s, V, -0.8, T, ln), M.hvp("nw", s, V, (-0.8, T), ln))]
    pairs += [(k.soft_nw_param_jacobian(s, p, -0.8, T, ln),
               M.param_jacobian("nw", s, (-0.8, T), p, ln)) for p in (0, 1)]
    for i, (got, want) in enumerate(pairs):
        assert got.dtype == np.float64
        _close(got, want, 1e-9 * max(1.0, np.abs(want).max()), 0, f"second order {i}")


@pytest.mark.parametrize("s,go,ge,T", [(0.7, -2.0, -0.5, 1.0), (-1.3, -1.0, -0.2, 0.5),
                                       (2.0, -3.0, -1.0, 2.0)])
def test_nw_affine_small_closed_forms(s, go, ge, T):
    """1x1: paths M (score s) and the two two-gap paths I->D / D->I (2 open each), so
    value = T log(e^{s/T} + 2 e^{2 open/T}), marginal = e^{s/T} / that sum, and the
    open count 4 e^{2 open/T} / sum.  Empty rows/columns: the boundary chain open +
    (n-1) ext, with gradients 1 and n-1."""
    k = O.get("oracle")
    sc = np.array([[[s]]], np.float32)
    v, post, gO, gE, gT = k.soft_nw_affine(sc, go, ge, T)
    Z = np.exp(s / T) + 2 * np.exp(2 * go / T)
    assert v[0] == pytest.approx(T * np.log(Z), rel=1e-6, abs=1e-6)
    assert post[0, 0, 0] == pytest.approx(np.exp(s / T) / Z, rel=1e-5, abs=1e-6)
    assert gO[0] == pytest.approx(4 * np.exp(2 * go / T) / Z, rel=1e-5, abs=1e-6)
    assert gE[0] == pytest.approx(0.0, abs=1e-7)
    x = np.zeros((3, 5, 4), np.float32)
    lens = np.array([[5, 0], [0, 4], [0, 0]], np.int32)
    v, post, gO, gE, gT = k.soft_nw_affine(x, go, ge, T, lens)
    np.testing.assert_allclose(v, [go + 4 * ge, go + 3 * ge, 0.0], rtol=1e-6)
    np.testing.assert_allclose(gO, [1.0, 1.0, 0.0])
    np.testing.assert_allclose(gE, [4.0, 3.0, 0.0])
    assert not post.any()


@pytest.mark.parametrize("seed,L1,L2,T", [(0, 5, 7, 1.0), (1, 9, 6, 0.5), (2, 12, 12, 2.0)])
def test_nw_affine_hvp_is_derivative_of_marginals(seed, L1, L2, T):
    """In double precision the affine NW HVP equals the central difference of the
    marginals along V (the marginals are dvalue/dscores, so H V = d marginals / d eps)."""
    k = O.get("oracle64")
    rng = np.random.default_rng(seed)
    s = rng.standard_normal((2, L1, L2))
    V = rng.standard_normal((2, L1, L2))
    go, ge, eps = -2.0, -0.5, 1e-6
    H = k.soft_nw_affine_hvp(s, V, go, ge, T)
    mp = k.soft_nw_affine(s + eps * V, go, ge, T)[1]
    mm = k.soft_nw_affine(s - eps * V, go, ge, T)[1]
    np.testing.assert_allclose(H, (mp - mm) / (2 * eps), rtol=1e-5, atol=1e-7)
    # and the marginals are the value's gradient
    vp = k.soft_nw_affine(s + eps * V, go, ge, T)[0]
    vm = k.soft_nw_affine(s - eps * V, go, ge, T)[0]
    m = k.soft_nw_affine(s, go, ge, T)[1]
    np.testing.assert_allclose((vp - vm) / (2 * eps), (m * V).sum(axis=(1, 2)), rtol=1e-6,
                               atol=1e-8)


@pytest.mark.parametrize("seed,L1,L2,T", [(3, 6, 8, 1.0), (4, 10, 7, 0.7)])
def test_nw_affine_jacobians_are_derivatives_of_marginals(seed, L1, L2, T):
    """In double precision dP/d(open, ext, T) equal central differences of the
    marginals, and the value's parameter gradients those of the value."""
    k = O.get("oracle64")
    rng = np.random.default_rng(seed)
    s = rng.standard_normal((2, L1, L2))
    p0, eps = np.array([-2.0, -0.5, T]), 1e-6
    v, m, gO, gE, gT = k.soft_nw_affine(s, *p0)
    for q, g in enumerate((gO, gE, gT)):
        dp = np.zeros(3)
        dp[q] = eps
        hi, lo = k.soft_nw_affine(s, *(p0 + dp)), k.soft_nw_affine(s, *(p0 - dp))
        J = k.soft_nw_affine_param_jacobian(s, q, *p0)
        np.testing.assert_allclose(J, (hi[1] - lo[1]) / (2 * eps), rtol=1e-5, atol=1e-7)
        np.testing.assert_allclose(g, (hi[0] - lo[0]) / (2 * eps), rtol=1e-6, atol=1e-8)
