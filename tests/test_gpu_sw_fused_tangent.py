"""The HVP's forward tangent fused into the primal forward sweep (linear gap, SW and
NW): one pass computes alpha and its tangent along the direction V from the same
softmax weights, and folds the value's tangent dS = sum p_cell x_cell into the
partition's own online log-sum-exp (no second pass for the cell probabilities).
D2P_AMD_SW_FUSED_TANGENT=0 runs the two sweeps of /root/reference/src/sw/
kernels_cpu.cpp:279-477 (forward, then the tangent sweep over the stored table).

Both forms are held to the oracle: 1e-4 * max(1, |ref|) entry-wise at sizes where
the fp32 reference is itself that close to exact arithmetic, and otherwise the
long-element rule (within 1e-4 * max(1, max|exact|) of the double-precision
oracle, or within twice the fp32 reference's own error).  Cases cover the
half-workgroup helper form (parts of at most four stripes), the plain form (more
stripes per part, and helpers switched off), split parts whose first stripe takes
both the alpha and the tangent row above through global memory, ragged lengths
with empty elements, and backward_full, whose score gradient is the same HVP.
The two forms must also agree with each other to 1e-4 * max(1, max|H|): they differ
in the order of two additions per cell and in how dS is summed (online, at the
partition's running scale, against a second pass with the final partition), which
moves the fp32 tangents by a few ulp.
"""
import numpy as np
import pytest
import torch

import _capi
from _parity import check_vs_exact, close_entrywise
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _seeded(seed, shape):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32)


def _both(monkeypatch, fn):
    out = {}
    for flag in ("1", "0"):
        monkeypatch.setenv("D2P_AMD_SW_FUSED_TANGENT", flag)
        out[flag] = [t.detach().clone() for t in fn()]
        torch.cuda.synchronize()
    monkeypatch.delenv("D2P_AMD_SW_FUSED_TANGENT")
    for a, b in zip(out["1"], out["0"]):
        scale = max(1.0, float(b.abs().max())) if b.numel() else 1.0
        diff = float((a - b).abs().max()) if b.numel() else 0.0
        print(f"fused vs two sweeps: max diff {diff:.3e} (scale {scale:.3e})", flush=True)
        assert diff <= 1e-4 * scale
    return out["1"], out["0"]


CASES = [
    # (seed, fam, B, L1, L2, parts, helpers, ragged)
    (80, "sw", 3, 7, 9, 0, "1", False),
    (81, "sw", 2, 100, 120, 0, "1", False),      # two stripes, helper waves
    (82, "sw", 2, 330, 200, 0, "1", True),       # six stripes: plain form, ragged
    (83, "sw", 2, 256, 300, 0, "0", False),      # helpers off
    (84, "sw", 2, 1024, 256, 4, "1", True),      # four parts of four stripes, ragged
    (85, "sw", 1, 1500, 90, 3, "1", False),      # three parts of eight stripes (plain)
    (86, "sw", 1, 600, 70, 0, "1", False),       # automatic split
    (87, "sw", 4, 1, 64, 0, "1", False),         # one row
    (88, "nw", 2, 100, 120, 0, "1", False),
    (89, "nw", 2, 1024, 256, 4, "1", True),
    (90, "nw", 1, 1500, 90, 3, "1", False),
]


@pytest.mark.parametrize("seed,fam,B,L1,L2,parts,helpers,ragged", CASES)
def test_fused_tangent_hvp(cuda, monkeypatch, seed, fam, B, L1, L2, parts, helpers, ragged):
    print(f"case seed={seed} {fam} B={B} L1={L1} L2={L2} parts={parts} helpers={helpers}",
          flush=True)
    if parts:
        monkeypatch.setenv("D2P_AMD_SPLIT", str(parts))
    monkeypatch.setenv("D2P_AMD_SW_HELPERS", helpers)
    s = _seeded(seed, (B, L1, L2))
    v = _seeded(seed + 1000, (B, L1, L2))
    lengths = None
    if ragged:
        g = np.random.default_rng(seed)
        lengths = np.stack([g.integers(0, L1 + 1, B), g.integers(0, L2 + 1, B)],
                           1).astype(np.int32)
        lengths[0] = [L1, L2]
        lengths[-1] = [0, L2]
    dl = None if lengths is None else torch.from_numpy(lengths).to(cuda)
    sd, vd = s.to(cuda), v.to(cuda)
    hvp = _capi.nw_hvp if fam == "nw" else _capi.sw_hvp
    fused, two = _both(monkeypatch, lambda: [hvp(sd, vd, dl, -1.0, 0.9)])
    k32 = O.get("oracle")
    ref_fn = k32.soft_nw_hvp if fam == "nw" else k32.soft_sw_hvp
    ref = ref_fn(s.numpy(), v.numpy(), -1.0, 0.9, lengths)
    if L1 * L2 <= 300 * 300:
        ef = close_entrywise(fused[0], ref, f"{fam} hvp fused")
        et = close_entrywise(two[0], ref, f"{fam} hvp two sweeps")
        print(f"|fused - ref| {ef:.3e}, |two sweeps - ref| {et:.3e}", flush=True)
    else:
        k64 = O.get("oracle64")
        ex_fn = k64.soft_nw_hvp if fam == "nw" else k64.soft_sw_hvp
        exact = ex_fn(s.numpy().astype(np.float64), v.numpy().astype(np.float64), -1.0, 0.9,
                      lengths)
        ef, er = check_vs_exact(fused[0], exact, ref, f"{fam} hvp fused")
        et, _ = check_vs_exact(two[0], exact, ref, f"{fam} hvp two sweeps")
        print(f"|fused - exact| {ef:.3e}, |two sweeps - exact| {et:.3e}, "
              f"|fp32 reference - exact| {er:.3e}", flush=True)


@pytest.mark.parametrize("parts", [1, 3])
def test_fused_tangent_large_values(cuda, monkeypatch, parts):
    """Scores of about 50 at T = 0.5 (values near 2000, as the reference's clamp
    fixture): the value's tangent must weight the cells by 2^((alpha - S) c) with the
    fp32 partition S, whose rounding moves the weights' sum off 1 by about 1e-4 here,
    as the reverse sweep and the reference do."""
    monkeypatch.setenv("D2P_AMD_SPLIT", str(parts))
    s = _seeded(93, (2, 700, 90)) * 50.0
    v = _seeded(94, (2, 700, 90))
    sd, vd = s.to(cuda), v.to(cuda)
    fused, two = _both(monkeypatch, lambda: [_capi.sw_hvp(sd, vd, None, -1.0, 0.5)])
    ref = O.get("oracle").soft_sw_hvp(s.numpy(), v.numpy(), -1.0, 0.5)
    close_entrywise(fused[0], ref, "hvp fused, large values")
    close_entrywise(two[0], ref, "hvp two sweeps, large values")


@pytest.mark.parametrize("fam", ["sw", "nw"])
def test_fused_tangent_backward_full(cuda, monkeypatch, fam):
    s = _seeded(91, (3, 200, 150))
    ga = _seeded(92, (3, 200, 150))
    sd, gd = s.to(cuda), ga.to(cuda)
    full = _capi.nw_backward_full if fam == "nw" else _capi.sw_backward_full
    fused, _ = _both(monkeypatch, lambda: list(full(sd, gd, None, -1.0, 1.0)))
    k32 = O.get("oracle")
    ref_fn = k32.soft_nw_hvp if fam == "nw" else k32.soft_sw_hvp
    close_entrywise(fused[0], ref_fn(s.numpy(), ga.numpy(), -1.0, 1.0), f"{fam} backward_full")
