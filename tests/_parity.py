"""Shared parity checks for the GPU tests."""
import numpy as np


def dot_consistent(got, J_gpu, W, value_term, what):
    """A marginal-path parameter gradient against the double dot product of W with
    the GPU's own Jacobian (itself pinned entry by entry to the oracle by the Jacobian
    tests) plus the value-path term.  The gradient kernel accumulates that dot product
    inside its sweep, the Jacobian kernel writes the entries, so only rounding
    separates the two: the bound is 1e-5 of the terms' absolute sum."""
    J = J_gpu.detach().cpu().numpy().astype(np.float64)
    Wd = W.detach().cpu().numpy().astype(np.float64)
    ref = float((J * Wd).sum() + value_term)
    tol = 1e-5 * (float(np.abs(J * Wd).sum()) + abs(value_term)) + 1e-6
    err = abs(float(got) - ref)
    assert err <= tol, f"{what}: {float(got)!r} vs {ref!r} (|diff| {err:.2e} > {tol:.2e})"
    print(f"{what}: |grad - <W, J> - value term| = {err:.2e} ({err / max(abs(ref), 1e-30):.1e} "
          "relative)")
    return err / max(abs(ref), 1e-30)


def close_entrywise(gpu, ref, what, extra=0.0, atol=1e-4):
    """Entry-wise bound atol * max(1, |ref_ij|) + extra: atol absolute wherever
    |ref| <= 1, atol relative above.  Returns the largest |gpu - ref| for reporting."""
    import torch
    gpu = gpu.detach().cpu().numpy() if torch.is_tensor(gpu) else np.asarray(gpu)
    gpu = gpu.astype(np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(gpu - ref)
    tol = atol * np.maximum(1.0, np.abs(ref)) + extra
    bad = err > tol
    if bad.any():
        i = np.unravel_index(int(np.argmax(err - tol)), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} entries out of bound; worst at {i}: "
                             f"gpu {gpu[i]:.6e} ref {ref[i]:.6e} (tol {tol[i]:.3e}); "
                             f"max |gpu - ref| {err.max():.3e}")
    return float(err.max(initial=0.0))


def check_vs_exact(gpu, exact, ref32, what):
    """Second-order results of long elements against the double-precision oracle:
    the GPU's error stays within 1e-4 * max(1, max|exact|) or within twice the fp32
    reference's own error on the same input, whichever is larger (the fp32
    reference differs from the exact values by more than the 1e-4 contract at
    these sizes)."""
    import torch
    gpu = gpu.detach().cpu().numpy() if torch.is_tensor(gpu) else np.asarray(gpu)
    gpu = gpu.astype(np.float64)
    e_gpu = float(np.abs(gpu - exact).max())
    e_ref = float(np.abs(ref32.astype(np.float64) - exact).max())
    tol = max(1e-4 * max(1.0, float(np.abs(exact).max())), 2.0 * e_ref)
    assert e_gpu <= tol, f"{what}: |gpu - exact| {e_gpu:.3e} > {tol:.3e} (fp32 reference {e_ref:.3e})"
    return e_gpu, e_ref
