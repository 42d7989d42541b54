"""The CPU oracle against the committed golden fixtures (tests/golden/*.npz,
written by tests/golden/make_golden.py from the reference's own CPU kernels).

Bit-exact: the oracle restates the reference's arithmetic in the same order and
both are compiled without FMA contraction.  Runs wherever the oracle is built,
including hosts without /root/reference.
"""
import glob
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                       "*.npz")))


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def oracle_outputs(k, f, name):
    """Every output the fixture stores, recomputed by the CPU library k."""
    ln = f["lengths"]
    if name.startswith("swa_"):
        s, V = f["scores"], f["V"]
        go, ge, T = float(f["gap_open"]), float(f["gap_ext"]), float(f["T"])
        part, post, g_o, g_e, gt = k.soft_sw_affine(s, go, ge, T, ln)
        return dict(value=part, marginals=post, grad_open=g_o, grad_ext=g_e, grad_T=gt,
                    hvp=k.soft_sw_affine_hvp(s, V, go, ge, T, ln),
                    jac_open=k.soft_sw_affine_param_jacobian(s, 0, go, ge, T, ln),
                    jac_ext=k.soft_sw_affine_param_jacobian(s, 1, go, ge, T, ln),
                    jac_T=k.soft_sw_affine_param_jacobian(s, 2, go, ge, T, ln))
    if name.startswith("sw_"):
        s, V = f["scores"], f["V"]
        gap, T = float(f["gap"]), float(f["T"])
        part, post, gg, gt = k.soft_sw(s, gap, T, ln)
        return dict(value=part, marginals=post, grad_gap=gg, grad_T=gt,
                    hvp=k.soft_sw_hvp(s, V, gap, T, ln),
                    jac_gap=k.soft_sw_param_jacobian(s, 0, gap, T, ln),
                    jac_T=k.soft_sw_param_jacobian(s, 1, gap, T, ln))
    c, V = f["costs"], f["V"]
    T, bw = float(f["T"]), int(f["bandwidth"])
    score, post, gt = k.soft_dtw(c, T, ln, bw)
    return dict(value=score, marginals=post, grad_T=gt, hvp=k.soft_dtw_hvp(c, V, T, ln, bw),
                jac_T=k.soft_dtw_param_jacobian(c, T, ln, bw))


def test_fixtures_present():
    assert len(GOLDEN) >= 10


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: os.path.basename(p)[:-4])
def test_oracle_matches_golden(path):
    f = load(path)
    name = os.path.basename(path)
    got = oracle_outputs(O.get("oracle"), f, name)
    for key, val in got.items():
        want = f[key]
        assert val.shape == want.shape, key
        assert np.array_equal(val.view(np.uint32), want.view(np.uint32)), \
            f"{name}:{key} max |diff| {np.abs(val.astype(np.float64) - want).max():.3e}"
