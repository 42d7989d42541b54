"""Writes the golden fixtures of this directory from the reference's own CPU
kernels (oracle/_ref/libd2p_ref.so, compiled by oracle/Makefile from
/root/reference/src/{sw,sw_affine,dtw}/kernels_cpu.cpp).

Run in a container that has /root/reference:
    make -C oracle all && python tests/golden/make_golden.py

Each fixture ``<family>_<case>.npz`` holds the inputs (seeded numpy draws), the
parameters and every output of the reference's binding-level call sequence:
value, marginals, parameter gradients, the Hessian-vector product against the
stored direction ``V`` and the parameter Jacobians.  The cases cover the regimes
only the reference's exact rounding pins: low temperature, |x / T| beyond the
exp clamp, C4-style large costs with near-ties, ragged and empty lengths, and
DTW bands.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402


def _rand(seed, shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


LENS = np.array([[16, 20], [7, 3], [0, 9], [16, 1]], np.int32)

SW = {
    # name: (seed, B, L1, L2, scale, gap, T, lengths)
    "basic": (0, 2, 12, 17, 1.0, -1.0, 1.0, None),
    "lowT_ragged": (1, 4, 16, 20, 2.0, -0.5, 0.1, LENS),
    "clamp": (2, 2, 10, 10, 60.0, -1.0, 0.5, None),
}
SWA = {
    "basic": (10, 2, 12, 17, 1.0, -2.0, -0.5, 1.0, None),
    "c3_params_ragged": (11, 4, 16, 20, 2.0, -11.0, -1.0, 0.5, LENS),
    "clamp": (12, 2, 10, 10, 60.0, -11.0, -1.0, 0.5, None),
}
DTW = {
    # name: (seed, B, L1, L2, scale, T, bandwidth, lengths)
    "basic": (20, 2, 12, 17, 1.0, 1.0, -1, None),
    "c4_style": (21, 2, 14, 14, 128.0, 0.1, -1, None),
    "band": (22, 2, 13, 18, 1.0, 0.5, 3, None),
    "ragged": (23, 4, 16, 20, 1.0, 0.7, -1, LENS),
}


def main():
    if not O.reference_available():
        raise SystemExit("oracle/_ref/libd2p_ref.so is not built (needs /root/reference)")
    r = O.get("reference")
    written = []
    for name, (seed, B, L1, L2, scale, gap, T, ln) in SW.items():
        s = _rand(seed, (B, L1, L2), scale)
        V = _rand(seed + 1, (B, L1, L2))
        part, post, gg, gt = r.soft_sw(s, gap, T, ln)
        out = dict(scores=s, V=V, gap=np.float32(gap), T=np.float32(T), value=part,
                   marginals=post, grad_gap=gg, grad_T=gt,
                   hvp=r.soft_sw_hvp(s, V, gap, T, ln),
                   jac_gap=r.soft_sw_param_jacobian(s, 0, gap, T, ln),
                   jac_T=r.soft_sw_param_jacobian(s, 1, gap, T, ln))
        written.append(_save(f"sw_{name}", out, ln, B, L1, L2))
    for name, (seed, B, L1, L2, scale, go, ge, T, ln) in SWA.items():
        s = _rand(seed, (B, L1, L2), scale)
        V = _rand(seed + 1, (B, L1, L2))
        part, post, g_o, g_e, gt = r.soft_sw_affine(s, go, ge, T, ln)
        out = dict(scores=s, V=V, gap_open=np.float32(go), gap_ext=np.float32(ge),
                   T=np.float32(T), value=part, marginals=post, grad_open=g_o, grad_ext=g_e,
                   grad_T=gt, hvp=r.soft_sw_affine_hvp(s, V, go, ge, T, ln),
                   jac_open=r.soft_sw_affine_param_jacobian(s, 0, go, ge, T, ln),
                   jac_ext=r.soft_sw_affine_param_jacobian(s, 1, go, ge, T, ln),
                   jac_T=r.soft_sw_affine_param_jacobian(s, 2, go, ge, T, ln))
        written.append(_save(f"swa_{name}", out, ln, B, L1, L2))
    for name, (seed, B, L1, L2, scale, T, bw, ln) in DTW.items():
        c = np.abs(_rand(seed, (B, L1, L2), scale))
        V = _rand(seed + 1, (B, L1, L2))
        score, post, gt = r.soft_dtw(c, T, ln, bw)
        out = dict(costs=c, V=V, T=np.float32(T), bandwidth=np.int64(bw), value=score,
                   marginals=post, grad_T=gt, hvp=r.soft_dtw_hvp(c, V, T, ln, bw),
                   jac_T=r.soft_dtw_param_jacobian(c, T, ln, bw))
        written.append(_save(f"dtw_{name}", out, ln, B, L1, L2))
    print("\n".join(written))


def _save(name, out, ln, B, L1, L2):
    lengths = np.array([[L1, L2]] * B, np.int32) if ln is None else np.asarray(ln, np.int32)
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, lengths=lengths, **out)
    return path


if __name__ == "__main__":
    main()
