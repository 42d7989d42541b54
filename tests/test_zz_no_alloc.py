"""d2p_sw_forward_marginals_noalloc: the allocation-free entry point against the
workspace entry point it mirrors, through the C ABI.

Both run the same kernels on the same inputs, so the outputs must be bit-identical.
Two calls in a row, the second on a smaller input, check that the static scratch
keeps no state the next call depends on (the array holds the last call's contents).
Shapes beyond the scratch are rejected with an error, and no kernel runs.
"""
import ctypes

import pytest
import torch

from _capi import check, lib, ptr, stream, sw_forward_marginals

pytestmark = pytest.mark.gpu


def _inputs(B, L1, L2, seed, ragged):
    g = torch.Generator().manual_seed(seed)
    s = torch.randn((B, L1, L2), generator=g, dtype=torch.float32)
    if ragged:
        lens = torch.stack([torch.randint(1, L1 + 1, (B,), generator=g),
                            torch.randint(1, L2 + 1, (B,), generator=g)], 1).int()
    else:
        lens = torch.tensor([[L1, L2]] * B, dtype=torch.int32)
    return s, lens


def _noalloc(x, lengths, gap, T):
    B, L1, L2 = x.shape
    dev = x.device
    outs = [torch.full((B,), 7.0, device=dev), torch.full((B, L1, L2), 7.0, device=dev),
            torch.full((B,), 7.0, device=dev), torch.full((B,), 7.0, device=dev)]
    check(lib().d2p_sw_forward_marginals_noalloc(ptr(x), ptr(lengths), B, L1, L2, gap, T,
                                                 *[ptr(o) for o in outs], stream()))
    return outs


def test_noalloc_matches_workspace_entry_point_twice(cuda):
    assert lib().d2p_sw_noalloc_scratch_bytes() == 64 << 20
    # first call: 9 stripes, ragged; second: smaller, full lengths, other parameters
    for (B, L1, L2, seed, ragged, gap, T) in ((5, 530, 300, 61, True, -1.0, 1.0),
                                               (2, 100, 130, 62, False, -0.5, 0.7)):
        assert lib().d2p_sw_workspace_bytes(B, L1, L2) <= 64 << 20
        s, lens = _inputs(B, L1, L2, seed, ragged)
        x, ln = s.to(cuda), lens.to(cuda)
        got = _noalloc(x, ln, gap, T)
        want = sw_forward_marginals(x, ln, gap, T)
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b)
        assert torch.isfinite(got[0]).all()


def test_noalloc_rejects_shapes_beyond_the_scratch(cuda):
    B, L1, L2 = 64, 512, 512    # about 79 MB of workspace
    assert lib().d2p_sw_workspace_bytes(B, L1, L2) > 64 << 20
    x = torch.zeros((1,), device=cuda)
    rc = lib().d2p_sw_forward_marginals_noalloc(ptr(x), ptr(x), B, L1, L2, -1.0, 1.0, ptr(x),
                                                ptr(x), ptr(x), ptr(x), stream())
    assert rc != 0
    assert b"static scratch" in lib().d2p_last_error()
