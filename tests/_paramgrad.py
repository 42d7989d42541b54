"""Checks of per-element parameter gradients (dS/dgap, dS/dT, ...).

These gradients are sums over every cell of a DP table.  The reference adds the
terms sequentially in fp32, which drifts from the exact sum as tables grow (a sum
of millions of small positive terms against a running total hundreds of times
larger): at 512x512 the drift is ~1e-4 relative, at 600x2500 ~2e-3.  The HIP
kernels reduce in a tree and stay closer to the exact value.  So a gradient that
misses the reference's fp32 value is held instead to the same per-cell terms of
the reference summed in double (``oracle.CpuKernels.param_grads64``), which
removes only the summation drift.  (A finite difference of the fp32 partition
function is too noisy for this at these sizes: S itself carries ~1e-6 relative
rounding noise that does not cancel between nearby parameter values.)
"""
import numpy as np


def check_param_grad(gpu, ref, exact_fn, rtol=3e-4, atol=1e-4):
    """gpu, ref: [B] gradients; exact_fn() -> [B] double-accumulated gradients."""
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    if np.all(np.abs(gpu - ref) <= atol + rtol * np.abs(ref)):
        return
    exact = np.asarray(exact_fn(), np.float64)
    bad = np.abs(gpu - exact) > atol + rtol * np.abs(exact)
    assert not np.any(bad), f"gradient {gpu} vs reference {ref} vs double-summed {exact}"
