"""Store or recompute: first-order linear-gap SW calls whose reverse sweep runs with
helper waves (16-wave workgroups for parts of five to eight stripes, C2's 512-row
elements; half-workgroup helpers for parts of at most four, C5's split parts) can
store only the forward's checkpoint rows (two steps per 16-step chunk and the last two steps)
and rebuild every other alpha row in the reverse sweep's helper waves, from those
rows, the stripe above's last row and the scores.  The rebuilt rows must equal the
stored ones, so every output equals the full-table form
(D2P_AMD_SW_RECOMPUTE=0) bit for bit: full and ragged lengths, empty elements,
rows shorter than a chunk, columns past the element, split parts, the
allocation-free entry point, and the public op.  Each case is also held to the
oracle at the north-star tolerances (value 1e-5 relative, marginals 1e-4 absolute).
"""
import numpy as np
import pytest
import torch

import _capi
from oracle import oracle as O
from test_gpu_sw_linear import _check, _seeded

pytestmark = pytest.mark.gpu


def _both(monkeypatch, fn):
    out = {}
    for flag in ("1", "0"):
        monkeypatch.setenv("D2P_AMD_SW_RECOMPUTE", flag)
        out[flag] = [t.clone() for t in fn()]
        torch.cuda.synchronize()
    for a, b in zip(out["1"], out["0"]):
        assert torch.equal(a, b)
    return out["1"]


CASES = [
    # (seed, B, L1, L2, parts, ragged)
    (60, 4, 512, 512, 1, False),    # the C2 shape, unsplit 16-wave sweeps
    (61, 3, 330, 200, 1, True),     # six stripes, ragged lengths and an empty element
    (62, 2, 512, 70, 1, False),     # rows shorter than the stripe skew
    (63, 5, 300, 1, 1, False),      # one column
    (64, 2, 320, 257, 1, True),     # five stripes, a last stripe of full height
    (65, 1, 1500, 90, 3, False),    # three parts of eight stripes
    (66, 9, 450, 33, 1, True),      # B not a multiple of 8, ragged
    # parts of at most four stripes (half-workgroup helpers)
    (70, 3, 256, 300, 1, False),    # four stripes, unsplit
    (71, 2, 1024, 512, 4, True),    # four parts of four stripes, ragged
    (72, 1, 2048, 640, 0, False),   # automatic split
    (73, 5, 200, 96, 1, True),      # aligned rows, ragged, four stripes
]


@pytest.mark.parametrize("seed,B,L1,L2,n,ragged", CASES)
def test_recompute_bit_identical_and_matches_oracle(cuda, monkeypatch, seed, B, L1, L2, n,
                                                    ragged):
    monkeypatch.setenv("D2P_AMD_SPLIT", str(n))
    s = _seeded(seed, (B, L1, L2), 1.5)
    lengths = None
    if ragged:
        g = np.random.default_rng(seed)
        lengths = np.stack([g.integers(0, L1 + 1, B), g.integers(0, L2 + 1, B)],
                           1).astype(np.int32)
        lengths[0] = [L1, L2]
        lengths[-1] = [0, L2]
    dl = None if lengths is None else torch.from_numpy(lengths).to(cuda)
    sd = s.to(cuda)
    out = _both(monkeypatch, lambda: _capi.sw_forward_marginals(sd, dl, -1.0, 0.8))
    ref = O.get("oracle").soft_sw(s.numpy(), -1.0, 0.8, lengths)
    _check(out, ref, lengths=lengths, gap=-1.0, T=0.8, scores=s.numpy())


def test_recompute_noalloc_entry(cuda, monkeypatch):
    s = _seeded(67, (8, 512, 384)).to(cuda)
    B, L1, L2 = s.shape
    lens = torch.tensor([[L1, L2]] * B, dtype=torch.int32, device=cuda)

    def run():
        outs = [torch.full((B,), 7.0, device=cuda), torch.full((B, L1, L2), 7.0, device=cuda),
                torch.full((B,), 7.0, device=cuda), torch.full((B,), 7.0, device=cuda)]
        _capi.check(_capi.lib().d2p_sw_forward_marginals_noalloc(
            _capi.ptr(s), _capi.ptr(lens), B, L1, L2, -1.0, 1.0,
            *[_capi.ptr(o) for o in outs], _capi.stream()))
        return outs
    _both(monkeypatch, run)


def test_recompute_public_op(cuda, monkeypatch):
    import d2p_amd
    s = _seeded(68, (6, 400, 300)).to(cuda)

    def run():
        x = s.clone().requires_grad_(True)
        r = d2p_amd.soft_sw(x, gap=-1.0, temperature=1.0)
        r.value.sum().backward()
        return [r.value.detach(), r.marginals.detach(), x.grad]
    _both(monkeypatch, run)
