"""CPU parity checker for the d2p_amd HIP path (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may import this module.  It wraps two interchangeable CPU libraries behind one
numpy interface:

* ``liboracle.so`` -- this repo's C restatement of the reference CPU kernels
  (``oracle/d2p_oracle.c``; each function cites the reference file:line it
  follows);
* ``_ref/libd2p_ref.so`` -- the reference's own CPU kernels
  (``/root/reference/src/{sw,sw_affine,dtw}/kernels_cpu.cpp``), compiled by
  ``oracle/Makefile`` where those sources exist;
* ``liboracle64.so`` -- the same C restatement compiled with every ``float`` as
  ``double`` (and ``expf``/``logf``/``fabsf`` as their double versions): the
  reference's algorithm in double precision, a near-exact value for quantities
  whose fp32 evaluation is ill-conditioned (second-order Jacobians of long
  elements), against which the fp32 reference's own error can be measured.
  ``get("oracle64")`` takes and returns float64 arrays.

Both expose the reference's CPU signatures (``src/sw/kernels_cpu.h:95-183``,
``src/sw_affine/kernels_cpu.h:80-167``, ``src/dtw/kernels_cpu.h:83-161``), so
the same Python code drives either and their outputs can be compared bit for
bit.  The composite helpers at the bottom restate the reference's binding-level
call sequences (``src/sw/torch_cpu.cpp:114-259``,
``src/sw_affine/torch_cpu.cpp:122-290``, ``src/dtw/torch_cpu.cpp:122-256``).
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "liboracle.so")
ORACLE64_LIB = os.path.join(HERE, "liboracle64.so")
REF_LIB = os.path.join(HERE, "_ref", "libd2p_ref.so")

_F = ctypes.POINTER(ctypes.c_float)
_I = ctypes.POINTER(ctypes.c_int)
_i = ctypes.c_int
_f = ctypes.c_float
_l = ctypes.c_int64

# (oracle symbol, reference symbol, argtypes)
_SIGS = {
    "sw_forward": ("oracle_sw_forward", "sw_regular_forward_cpu",
                   [_F, _F, _F, _I, _i, _i, _i, _f, _f]),
    "sw_backward": ("oracle_sw_backward", "sw_regular_backward_cpu",
                    [_F, _F, _F, _F, _F, _F, _F, _I, _i, _i, _i, _f, _f]),
    "sw_hvp": ("oracle_sw_hvp", "sw_regular_hvp_cpu",
               [_F, _F, _F, _F, _F, _F, _F, _F, _F, _I, _i, _i, _i, _f, _f]),
    "sw_param_grad": ("oracle_sw_param_grad", "sw_regular_param_grad_cpu",
                      [_F, _F, _F, _F, _F, _F, _F, _F, _I, _i, _i, _i, _f, _f, _i]),
    "swa_forward": ("oracle_swa_forward", "sw_affine_forward_cpu",
                    [_F, _F, _F, _I, _i, _i, _i, _f, _f, _f]),
    "swa_backward": ("oracle_swa_backward", "sw_affine_backward_cpu",
                     [_F, _F, _F, _F, _F, _F, _F, _F, _I, _i, _i, _i, _f, _f, _f]),
    "swa_hvp": ("oracle_swa_hvp", "sw_affine_hvp_cpu",
                [_F, _F, _F, _F, _F, _F, _F, _F, _I, _i, _i, _i, _f, _f, _f]),
    "swa_param_grad": ("oracle_swa_param_grad", "sw_affine_param_grad_cpu",
                       [_F, _F, _F, _F, _F, _F, _F, _F, _I, _i, _i, _i, _f, _f, _f, _i]),
    "dtw_forward": ("oracle_dtw_forward", "dtw_forward_cpu",
                    [_F, _F, _F, _I, _i, _i, _i, _f, _l]),
    "dtw_backward": ("oracle_dtw_backward", "dtw_backward_cpu",
                     [_F, _F, _F, _F, _F, _F, _I, _i, _i, _i, _f, _l]),
    "dtw_hvp": ("oracle_dtw_hvp", "dtw_hvp_cpu",
                [_F, _F, _F, _F, _F, _F, _F, _F, _F, _I, _i, _i, _i, _f, _l]),
    "dtw_param_grad": ("oracle_dtw_param_grad", "dtw_param_grad_cpu",
                       [_F, _F, _F, _F, _F, _F, _F, _I, _i, _i, _i, _f, _l]),
    "nw_forward": ("oracle_nw_forward", "nw_forward_cpu",
                   [_F, _F, _F, _I, _i, _i, _i, _f, _f]),
    "nw_backward": ("oracle_nw_backward", "nw_backward_cpu",
                    [_F, _F, _F, _F, _F, _F, _F, _I, _i, _i, _i, _f, _f]),
    "nw_hvp": ("oracle_nw_hvp", "nw_hvp_cpu",
               [_F, _F, _F, _F, _F, _F, _F, _F, _F, _I, _i, _i, _i, _f, _f]),
    "nw_param_grad": ("oracle_nw_param_grad", "nw_param_grad_cpu",
                      [_F, _F, _F, _F, _F, _F, _F, _F, _I, _i, _i, _i, _f, _f, _i]),
    "nwa_forward": ("oracle_nwa_forward", "nw_affine_forward_cpu",
                    [_F, _F, _F, _I, _i, _i, _i, _f, _f, _f]),
    "nwa_backward": ("oracle_nwa_backward", "nw_affine_backward_cpu",
                     [_F, _F, _F, _F, _F, _F, _F, _F, _I, _i, _i, _i, _f, _f, _f]),
    "nwa_hvp": ("oracle_nwa_hvp", "nw_affine_hvp_cpu",
                [_F, _F, _F, _F, _F, _F, _F, _F, _F, _I, _i, _i, _i, _f, _f, _f]),
    "nwa_param_grad": ("oracle_nwa_param_grad", "nw_affine_param_grad_cpu",
                       [_F, _F, _F, _F, _F, _F, _F, _F, _I, _i, _i, _i, _f, _f, _f, _i]),
}


_D = ctypes.POINTER(ctypes.c_double)

# test-only extensions of the oracle (no reference counterpart): backward sweeps
# whose parameter gradients are also summed in double
_SIGS64 = {
    "sw_backward_sums64": ("oracle_sw_backward_sums64",
                           [_F, _F, _F, _F, _F, _D, _I, _i, _i, _i, _f, _f]),
    "swa_backward_sums64": ("oracle_swa_backward_sums64",
                            [_F, _F, _F, _F, _F, _D, _I, _i, _i, _i, _f, _f, _f]),
    "dtw_backward_sums64": ("oracle_dtw_backward_sums64",
                            [_F, _F, _F, _F, _F, _D, _I, _i, _i, _i, _f, _l]),
}


def _p(a: np.ndarray):
    if a.dtype == np.int32:
        return a.ctypes.data_as(_I)
    if a.dtype == np.float64:
        return a.ctypes.data_as(_D)
    return a.ctypes.data_as(_F)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _lengths(lengths, B, L1, L2) -> np.ndarray:
    if lengths is None:
        out = np.empty((B, 2), dtype=np.int32)
        out[:, 0] = L1
        out[:, 1] = L2
        return out
    return np.ascontiguousarray(np.asarray(lengths, dtype=np.int32)).reshape(B, 2)


class CpuKernels:
    """numpy front end over one CPU library (``kind`` = "oracle", "reference" or
    "oracle64")."""

    def __init__(self, kind: str = "oracle"):
        if kind not in ("oracle", "reference", "oracle64"):
            raise ValueError(kind)
        path = {"oracle": ORACLE_LIB, "reference": REF_LIB, "oracle64": ORACLE64_LIB}[kind]
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is not built; run `make -C oracle` (reference build needs "
                "/root/reference)")
        if kind == "reference":
            import torch  # noqa: F401  -- loads libtorch_cpu/libc10 the library links
        self.kind = kind
        self.path = path
        self.ft = np.float64 if kind == "oracle64" else np.float32
        # the double build takes double arrays and scalars where the others take float
        wide = {_F: _D, _f: ctypes.c_double} if kind == "oracle64" else {}
        self.lib = ctypes.CDLL(path)
        self.fn = {}
        for name, (osym, rsym, argt) in _SIGS.items():
            f = getattr(self.lib, rsym if kind == "reference" else osym)
            f.argtypes = [wide.get(t, t) for t in argt]
            f.restype = None
            self.fn[name] = f
        if kind != "reference":
            for name, (osym, argt) in _SIGS64.items():
                f = getattr(self.lib, osym)
                f.argtypes = [wide.get(t, t) for t in argt]
                f.restype = None
                self.fn[name] = f

    def _a(self, a) -> np.ndarray:
        """A contiguous array of the library's float type."""
        return np.ascontiguousarray(np.asarray(a, dtype=self.ft))

    def param_grads64(self, family, inputs, lengths, *params, bandwidth=-1):
        """Per-element parameter gradients with the reference's per-cell terms summed
        in double (oracle only): SW [B,2] (gap, T), affine [B,3] (open, ext, T),
        DTW [B] (T)."""
        if self.kind == "reference":
            raise RuntimeError("double-accumulated sums exist in the oracle only")
        x = self._a(inputs)
        B, L1, L2 = x.shape
        ln = _lengths(lengths, B, L1, L2)
        post = np.zeros_like(x)
        if family == "sw":
            alpha, part = self.sw_forward(x, lengths, *params)
            out = np.zeros((B, 2), np.float64)
            self.fn["sw_backward_sums64"](_p(alpha), _p(x), _p(part), _p(np.zeros_like(alpha)),
                                          _p(post), _p(out), _p(ln), B, L1, L2, *params)
        elif family == "swa":
            alpha, part = self.swa_forward(x, lengths, *params)
            out = np.zeros((B, 3), np.float64)
            self.fn["swa_backward_sums64"](_p(alpha), _p(x), _p(part),
                                           _p(np.zeros_like(alpha)), _p(post), _p(out), _p(ln),
                                           B, L1, L2, *params)
        elif family == "dtw":
            alpha, score = self.dtw_forward(x, lengths, params[0], bandwidth)
            out = np.zeros((B,), np.float64)
            self.fn["dtw_backward_sums64"](_p(alpha), _p(x), _p(score), _p(np.zeros_like(alpha)),
                                           _p(post), _p(out), _p(ln), B, L1, L2, params[0],
                                           bandwidth)
        else:
            raise ValueError(family)
        return out

    # ---------------- linear-gap SW ----------------
    def sw_forward(self, scores, lengths, gap, T):
        s = self._a(scores)
        B, L1, L2 = s.shape
        ln = _lengths(lengths, B, L1, L2)
        alpha = np.zeros((B, (L1 + 1) * (L2 + 1)), self.ft)
        part = np.zeros((B,), self.ft)
        self.fn["sw_forward"](_p(s), _p(alpha), _p(part), _p(ln), B, L1, L2, gap, T)
        return alpha, part

    def sw_backward(self, alpha, scores, part, lengths, gap, T):
        s = self._a(scores)
        B, L1, L2 = s.shape
        ln = _lengths(lengths, B, L1, L2)
        beta = np.zeros_like(alpha)
        post = np.zeros_like(s)
        gg = np.zeros((B,), self.ft)
        gt = np.zeros((B,), self.ft)
        self.fn["sw_backward"](_p(alpha), _p(s), _p(part), _p(beta), _p(post), _p(gg),
                               _p(gt), _p(ln), B, L1, L2, gap, T)
        return post, gg, gt

    def sw_hvp(self, alpha, scores, part, V, lengths, gap, T):
        s = self._a(scores)
        v = self._a(V)
        B, L1, L2 = s.shape
        ln = _lengths(lengths, B, L1, L2)
        da = np.zeros_like(alpha)
        dp = np.zeros((B,), self.ft)
        be = np.zeros_like(alpha)
        dbe = np.zeros_like(alpha)
        H = np.zeros_like(s)
        self.fn["sw_hvp"](_p(alpha), _p(s), _p(part), _p(v), _p(da), _p(dp), _p(be),
                          _p(dbe), _p(H), _p(ln), B, L1, L2, gap, T)
        return H, dp

    def sw_param_grad(self, alpha, scores, part, dS, lengths, gap, T, ptype):
        s = self._a(scores)
        B, L1, L2 = s.shape
        ln = _lengths(lengths, B, L1, L2)
        dS = self._a(dS)
        U = np.zeros_like(alpha)
        be = np.zeros_like(alpha)
        W = np.zeros_like(alpha)
        dP = np.zeros_like(s)
        self.fn["sw_param_grad"](_p(alpha), _p(s), _p(part), _p(dS), _p(U), _p(be), _p(W),
                                 _p(dP), _p(ln), B, L1, L2, gap, T, ptype)
        return dP

    # ---------------- affine SW ----------------
    def swa_forward(self, scores, lengths, go, ge, T):
        s = self._a(scores)
        B, L1, L2 = s.shape
        ln = _lengths(lengths, B, L1, L2)
        alpha = np.zeros((B, 3 * (L1 + 1) * (L2 + 1)), self.ft)
        part = np.zeros((B,), self.ft)
        self.fn["swa_forward"](_p(s), _p(alpha), _p(part), _p(ln), B, L1, L2, go, ge, T)
        return alpha, part

    def swa_backward(self, alpha, scores, part, lengths, go, ge, T):
        s = self._a(scores)
        B, L1, L2 = s.shape
        ln = _lengths(lengths, B, L1, L2)
        beta = np.zeros_like(alpha)
        post = np.zeros_like(s)
        g_o = np.zeros((B,), self.ft)
        g_e = np.zeros((B,), self.ft)
        gt = np.zeros((B,), self.ft)
        self.fn["swa_backward"](_p(alpha), _p(s), _p(part), _p(beta), _p(post), _p(g_o),
                                _p(g_e), _p(gt), _p(ln), B, L1, L2, go, ge, T)
        return post, g_o, g_e, gt

    def swa_hvp(self, alpha, scores, part, V, lengths, go, ge, T):
        s = self._a(scores)
        v = self._a(V)
        B, L1, L2 = s.shape
        ln = _lengths(lengths, B, L1, L2)
        da = np.zeros_like(alpha)
        dp = np.zeros((B,), self.ft)
        dbe = np.zeros_like(alpha)
        H = np.zeros_like(s)
        self.fn["swa_hvp"](_p(alpha), _p(s), _p(part), _p(v), _p(da), _p(dp), _p(dbe),
                           _p(H), _p(ln), B, L1, L2, go, ge, T)
        return H, dp

    def swa_param_grad(self, alpha, scores, part, dS, lengths, go, ge, T, ptype):
        s = self._a(scores)
        B, L1, L2 = s.shape
        ln = _lengths(lengths, B, L1, L2)
        dS = self._a(dS)
        U = np.zeros_like(alpha)
        be = np.zeros_like(alpha)
        W = np.zeros_like(alpha)
        dP = np.zeros_like(s)
        self.fn["swa_param_grad"](_p(alpha), _p(s), _p(part), _p(dS), _p(U), _p(be),
                                  _p(W), _p(dP), _p(ln), B, L1, L2, go, ge, T, ptype)
        return dP

    # ---------------- DTW ----------------
    def dtw_forward(self, costs, lengths, T, bandwidth=-1):
        c = self._a(costs)
        B, L1, L2 = c.shape
        ln = _lengths(lengths, B, L1, L2)
        alpha = np.zeros((B, (L1 + 1) * (L2 + 1)), self.ft)
        score = np.zeros((B,), self.ft)
        self.fn["dtw_forward"](_p(c), _p(alpha), _p(score), _p(ln), B, L1, L2, T, bandwidth)
        return alpha, score

    def dtw_backward(self, alpha, costs, score, lengths, T, bandwidth=-1):
        c = self._a(costs)
        B, L1, L2 = c.shape
        ln = _lengths(lengths, B, L1, L2)
        beta = np.zeros_like(alpha)
        post = np.zeros_like(c)
        gt = np.zeros((B,), self.ft)
        self.fn["dtw_backward"](_p(alpha), _p(c), _p(score), _p(beta), _p(post), _p(gt),
                                _p(ln), B, L1, L2, T, bandwidth)
        return post, gt

    def dtw_hvp(self, alpha, costs, score, V, lengths, T, bandwidth=-1):
        c = self._a(costs)
        v = self._a(V)
        B, L1, L2 = c.shape
        ln = _lengths(lengths, B, L1, L2)
        da = np.zeros_like(alpha)
        ds = np.zeros((B,), self.ft)
        be = np.zeros_like(alpha)
        dbe = np.zeros_like(alpha)
        H = np.zeros_like(c)
        self.fn["dtw_hvp"](_p(alpha), _p(c), _p(score), _p(v), _p(da), _p(ds), _p(be),
                           _p(dbe), _p(H), _p(ln), B, L1, L2, T, bandwidth)
        return H, ds

    def dtw_param_grad(self, alpha, costs, score, lengths, T, bandwidth=-1):
        c = self._a(costs)
        B, L1, L2 = c.shape
        ln = _lengths(lengths, B, L1, L2)
        U = np.zeros_like(alpha)
        be = np.zeros_like(alpha)
        W = np.zeros_like(alpha)
        dP = np.zeros_like(c)
        self.fn["dtw_param_grad"](_p(alpha), _p(c), _p(score), _p(U), _p(be), _p(W),
                                  _p(dP), _p(ln), B, L1, L2, T, bandwidth)
        return dP

    # ---------------- linear-gap NW ----------------
    def nw_forward(self, scores, lengths, gap, T):
        s = self._a(scores)
        B, L1, L2 = s.shape
        ln = _lengths(lengths, B, L1, L2)
        alpha = np.zeros((B, (L1 + 1) * (L2 + 1)), self.ft)
        score = np.zeros((B,), self.ft)
        self.fn["nw_forward"](_p(s), _p(alpha), _p(score), _p(ln), B, L1, L2, gap, T)
        return alpha, score

    def nw_backward(self, alpha, scores, score, lengths, gap, T):
        s = self._a(scores)
        B, L1, L2 = s.shape
        ln = _lengths(lengths, B, L1, L2)
        beta = np.zeros_like(alpha)
        post = np.zeros_like(s)
        gg = np.zeros((B,), self.ft)
        gt = np.zeros((B,), self.ft)
        self.fn["nw_backward"](_p(alpha), _p(s), _p(score), _p(beta), _p(post), _p(gg),
                               _p(gt), _p(ln), B, L1, L2, gap, T)
        return post, gg, gt

    def nw_hvp(self, alpha, scores, score, V, lengths, gap, T):
        s = self._a(scores)
        v = self._a(V)
        B, L1, L2 = s.shape
        ln = _lengths(lengths, B, L1, L2)
        da = np.zeros_like(alpha)
        ds = np.zeros((B,), self.ft)
        be = np.zeros_like(alpha)
        dbe = np.zeros_like(alpha)
        H = np.zeros_like(s)
        self.fn["nw_hvp"](_p(alpha), _p(s), _p(score), _p(v), _p(da), _p(ds), _p(be), _p(dbe),
                          _p(H), _p(ln), B, L1, L2, gap, T)
        return H, ds

    def nw_param_grad(self, alpha, scores, score, lengths, gap, T, ptype):
        s = self._a(scores)
        B, L1, L2 = s.shape
        ln = _lengths(lengths, B, L1, L2)
        dS = np.zeros((B,), self.ft)   # unused: the terminal beta is constant
        U = np.zeros_like(alpha)
        be = np.zeros_like(alpha)
        W = np.zeros_like(alpha)
        dP = np.zeros_like(s)
        self.fn["nw_param_grad"](_p(alpha), _p(s), _p(score), _p(dS), _p(U), _p(be), _p(W),
                                 _p(dP), _p(ln), B, L1, L2, gap, T, ptype)
        return dP

    # ---------------- affine-gap NW ----------------
    def nwa_forward(self, scores, lengths, go, ge, T):
        s = self._a(scores)
        B, L1, L2 = s.shape
        ln = _lengths(lengths, B, L1, L2)
        alpha = np.zeros((B, 3 * (L1 + 1) * (L2 + 1)), self.ft)
        score = np.zeros((B,), self.ft)
        self.fn["nwa_forward"](_p(s), _p(alpha), _p(score), _p(ln), B, L1, L2, go, ge, T)
        return alpha, score

    def nwa_backward(self, alpha, scores, score, lengths, go, ge, T):
        s = self._a(scores)
        B, L1, L2 = s.shape
        ln = _lengths(lengths, B, L1, L2)
        beta = np.zeros_like(alpha)
        post = np.zeros_like(s)
        g = [np.zeros((B,), self.ft) for _ in range(3)]
        self.fn["nwa_backward"](_p(alpha), _p(s), _p(score), _p(beta), _p(post), _p(g[0]),
                                _p(g[1]), _p(g[2]), _p(ln), B, L1, L2, go, ge, T)
        return post, g[0], g[1], g[2]

    def nwa_hvp(self, alpha, scores, score, V, lengths, go, ge, T):
        s = self._a(scores)
        v = self._a(V)
        B, L1, L2 = s.shape
        ln = _lengths(lengths, B, L1, L2)
        da = np.zeros_like(alpha)
        ds = np.zeros((B,), self.ft)
        be = np.zeros_like(alpha)
        dbe = np.zeros_like(alpha)
        H = np.zeros_like(s)
        self.fn["nwa_hvp"](_p(alpha), _p(s), _p(score), _p(v), _p(da), _p(ds), _p(be), _p(dbe),
                           _p(H), _p(ln), B, L1, L2, go, ge, T)
        return H, ds

    def soft_nw_affine_hvp(self, scores, V, go=-2.0, ge=-0.5, T=1.0, lengths=None):
        alpha, score = self.nwa_forward(scores, lengths, go, ge, T)
        return self.nwa_hvp(alpha, scores, score, V, lengths, go, ge, T)[0]

    def soft_nw_affine_param_jacobian(self, scores, ptype, go=-2.0, ge=-0.5, T=1.0,
                                      lengths=None):
        alpha, score = self.nwa_forward(scores, lengths, go, ge, T)
        s = self._a(scores)
        B, L1, L2 = s.shape
        ln = _lengths(lengths, B, L1, L2)
        dS = np.zeros((B,), self.ft)   # unused: the terminal betas carry their tangents
        U, be, W = np.zeros_like(alpha), np.zeros_like(alpha), np.zeros_like(alpha)
        dP = np.zeros_like(s)
        self.fn["nwa_param_grad"](_p(alpha), _p(s), _p(score), _p(dS), _p(U), _p(be), _p(W),
                                  _p(dP), _p(ln), B, L1, L2, go, ge, T, ptype)
        return dP

    def soft_nw_affine(self, scores, go=-2.0, ge=-0.5, T=1.0, lengths=None):
        """value, marginals, grad_open, grad_ext, grad_T (nw_affine forward + backward)."""
        alpha, score = self.nwa_forward(scores, lengths, go, ge, T)
        post, gO, gE, gT = self.nwa_backward(alpha, scores, score, lengths, go, ge, T)
        return score, post, gO, gE, gT

    # ---------------- binding-level composites ----------------
    def soft_nw_hvp(self, scores, V, gap=-1.0, T=1.0, lengths=None):
        alpha, score = self.nw_forward(scores, lengths, gap, T)
        return self.nw_hvp(alpha, scores, score, V, lengths, gap, T)[0]

    def soft_nw_param_jacobian(self, scores, ptype, gap=-1.0, T=1.0, lengths=None):
        alpha, score = self.nw_forward(scores, lengths, gap, T)
        return self.nw_param_grad(alpha, scores, score, lengths, gap, T, ptype)

    def soft_nw(self, scores, gap=-1.0, T=1.0, lengths=None):
        """value, marginals, grad_gap, grad_T (src/nw/torch_cpu.cpp forward + backward)."""
        alpha, score = self.nw_forward(scores, lengths, gap, T)
        post, gg, gt = self.nw_backward(alpha, scores, score, lengths, gap, T)
        return score, post, gg, gt

    def soft_sw(self, scores, gap=-1.0, T=1.0, lengths=None):
        """value, marginals, grad_gap, grad_T (src/sw/torch_cpu.cpp:114-165)."""
        alpha, part = self.sw_forward(scores, lengths, gap, T)
        post, gg, gt = self.sw_backward(alpha, scores, part, lengths, gap, T)
        return part, post, gg, gt

    def soft_sw_hvp(self, scores, V, gap=-1.0, T=1.0, lengths=None):
        alpha, part = self.sw_forward(scores, lengths, gap, T)
        return self.sw_hvp(alpha, scores, part, V, lengths, gap, T)[0]

    def soft_sw_param_jacobian(self, scores, ptype, gap=-1.0, T=1.0, lengths=None):
        alpha, part = self.sw_forward(scores, lengths, gap, T)
        _, gg, gt = self.sw_backward(alpha, scores, part, lengths, gap, T)
        return self.sw_param_grad(alpha, scores, part, gg if ptype == 0 else gt,
                                  lengths, gap, T, ptype)

    def soft_sw_affine(self, scores, go=-2.0, ge=-0.5, T=1.0, lengths=None):
        alpha, part = self.swa_forward(scores, lengths, go, ge, T)
        post, g_o, g_e, gt = self.swa_backward(alpha, scores, part, lengths, go, ge, T)
        return part, post, g_o, g_e, gt

    def soft_sw_affine_hvp(self, scores, V, go=-2.0, ge=-0.5, T=1.0, lengths=None):
        alpha, part = self.swa_forward(scores, lengths, go, ge, T)
        return self.swa_hvp(alpha, scores, part, V, lengths, go, ge, T)[0]

    def soft_sw_affine_param_jacobian(self, scores, ptype, go=-2.0, ge=-0.5, T=1.0,
                                      lengths=None):
        alpha, part = self.swa_forward(scores, lengths, go, ge, T)
        _, g_o, g_e, gt = self.swa_backward(alpha, scores, part, lengths, go, ge, T)
        dS = (g_o, g_e, gt)[ptype]
        return self.swa_param_grad(alpha, scores, part, dS, lengths, go, ge, T, ptype)

    def soft_dtw(self, costs, T=1.0, lengths=None, bandwidth=-1):
        alpha, score = self.dtw_forward(costs, lengths, T, bandwidth)
        post, gt = self.dtw_backward(alpha, costs, score, lengths, T, bandwidth)
        return score, post, gt

    def soft_dtw_hvp(self, costs, V, T=1.0, lengths=None, bandwidth=-1):
        alpha, score = self.dtw_forward(costs, lengths, T, bandwidth)
        return self.dtw_hvp(alpha, costs, score, V, lengths, T, bandwidth)[0]

    def soft_dtw_param_jacobian(self, costs, T=1.0, lengths=None, bandwidth=-1):
        alpha, score = self.dtw_forward(costs, lengths, T, bandwidth)
        return self.dtw_param_grad(alpha, costs, score, lengths, T, bandwidth)


_cache = {}


def get(kind: str = "oracle") -> CpuKernels:
    if kind not in _cache:
        _cache[kind] = CpuKernels(kind)
    return _cache[kind]


def reference_available() -> bool:
    return os.path.exists(REF_LIB)


def set_threads(n: int) -> None:
    """Thread count for both libraries (OpenMP for the oracle, ATen for _ref)."""
    lib = ctypes.CDLL(ORACLE_LIB)
    try:
        gomp = ctypes.CDLL("libgomp.so.1")
        gomp.omp_set_num_threads(int(n))
    except OSError:
        pass
    del lib
    try:
        import torch
        torch.set_num_threads(int(n))
    except Exception:
        pass


def build(quiet: bool = True) -> None:
    """Compile liboracle.so (and _ref when /root/reference exists)."""
    import subprocess
    r = subprocess.run(["make", "-C", HERE, "all"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + r.stdout + r.stderr)
    if not quiet:
        print(r.stdout)
