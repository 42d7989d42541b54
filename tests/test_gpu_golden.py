"""The HIP path against the reference's own outputs (tests/golden/*.npz, written
by tests/golden/make_golden.py from the reference's CPU kernels), through the C
ABI.

Tolerances: value 1e-5 relative; marginals 1e-4 absolute;
HVP and Jacobian entries 1e-4 * max(1, max|ref|).  Parameter gradients are sums
of cancelling per-cell terms: 1e-3 relative plus 1e-5 * (|value| + 1) / T.  The
Jacobians also move with the fp32 evaluation of dS/dtheta (each entry by that
error times P / T): 1e-5 * |dS/dtheta| / T * max(P) is added at these sizes.
The temperature Jacobians of SW carry per-cell terms P (alpha - S) / T^2 whose
inputs hold fp32 rounding of |alpha| <= |value|: 4e-7 * (|value| + 1) / T^2 more.
The soft-DTW temperature Jacobian is exactly 0 at (1,1) and (L1,L2) (every path
passes both cells, so P = 1 there at every T); what the reference's fp32 sweeps
leave in those cells measures the rounding they accumulate, and 3x that is added.
"""
import os

import numpy as np
import pytest
import torch

import _capi
from test_golden import GOLDEN, load

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


def _check(name, key, got, want, atol, rtol=0.0):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    finite = np.abs(want) < 1e29
    assert np.array_equal(finite, np.abs(got) < 1e29), f"{name}:{key} reachability differs"
    err = np.abs(got - want)[finite]
    tol = (atol + rtol * np.abs(want))[finite]
    assert np.all(err <= tol), f"{name}:{key} max err {err.max(initial=0):.3e}"


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: os.path.basename(p)[:-4])
def test_hip_matches_golden(cuda, path):
    f = load(path)
    name = os.path.basename(path)[:-4]
    ln = torch.from_numpy(f["lengths"]).to(cuda)
    T = float(f["T"])
    x = torch.from_numpy(f["costs" if name.startswith("dtw") else "scores"]).to(cuda)
    V = torch.from_numpy(f["V"]).to(cuda)
    if name.startswith("swa_"):
        go, ge = float(f["gap_open"]), float(f["gap_ext"])
        value, marg, *pg = _capi.swa_forward_marginals(x, ln, go, ge, T)
        pnames = ("open", "ext", "T")
        hvp = _capi.swa_hvp(x, V, ln, go, ge, T)
        jac = [_capi.swa_param_jacobian(x, p, ln, go, ge, T) for p in range(3)]
    elif name.startswith("sw_"):
        gap = float(f["gap"])
        value, marg, *pg = _capi.sw_forward_marginals(x, ln, gap, T)
        pnames = ("gap", "T")
        hvp = _capi.sw_hvp(x, V, ln, gap, T)
        jac = [_capi.sw_param_jacobian(x, p, ln, gap, T) for p in range(2)]
    else:
        bw = int(f["bandwidth"])
        value, marg, *pg = _capi.dtw_forward_marginals(x, ln, T, bw)
        pnames = ("T",)
        hvp = _capi.dtw_hvp(x, V, ln, T, bw)
        jac = [_capi.dtw_param_jacobian(x, ln, T, bw)]
    rv = f["value"]
    _check(name, "value", _np(value), rv, 1e-6, 1e-5)
    _check(name, "marginals", _np(marg), f["marginals"], 1e-4)
    _check(name, "hvp", _np(hvp), f["hvp"], 1e-4 * np.maximum(1.0, np.abs(f["hvp"])))
    vmax = np.abs(rv[np.abs(rv) < 1e29]).max(initial=0.0)
    pmax = np.abs(f["marginals"]).max()
    for pn, g, J in zip(pnames, pg, jac):
        dS = f[f"grad_{pn}"]
        _check(name, f"grad_{pn}", _np(g), dS, 1e-5 * (vmax + 1.0) / T, 1e-3)
        want = f[f"jac_{pn}"]
        allow = 1e-5 * np.abs(dS).max() / T * pmax
        if pn == "T" and not name.startswith("dtw"):
            allow += 4e-7 * (vmax + 1.0) / T ** 2
        if pn == "T" and name.startswith("dtw"):
            zeros = [abs(float(want[b, 0, 0])) + abs(float(want[b, l1 - 1, l2 - 1]))
                     for b, (l1, l2) in enumerate(f["lengths"]) if l1 > 0 and l2 > 0]
            allow += 3.0 * max(zeros, default=0.0)
        _check(name, f"jac_{pn}", _np(J), want, 1e-4 * max(1.0, np.abs(want).max()) + allow)
