"""The timeout contract of the pipeline waits, forced from the host.

The sweeps' stripes and parts wait on each other through bounded polls (no
counterpart in the reference, whose kernels never wait on each other).  A wait
that reaches its bound gives up, marks its batch element in the workspace's status
words, and the kernel runs on to its end; every entry point then overwrites all
outputs of a marked element with NaN, and the torch layer raises when
D2P_AMD_CHECK_STATUS=1.  Here d2p_set_spin_limit(1) makes every wait that is not
satisfied at its first poll give up, so elements with more than one stripe are
marked while every kernel still exits normally; the bound is restored afterwards
and a normal call must be clean again.
"""
import ctypes
import os

import numpy as np
import pytest
import torch

import d2p_amd
from _capi import check, lib, ptr, stream
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEFAULT_SPINS = 1 << 22


@pytest.fixture
def low_spin_limit(cuda):
    check(lib().d2p_set_spin_limit(1))
    try:
        yield
    finally:
        check(lib().d2p_set_spin_limit(DEFAULT_SPINS))


def _scores(B, L1, L2, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn((B, L1, L2), generator=g, dtype=torch.float32)


def _status_words(ws, B):
    torch.cuda.synchronize()
    return ws[:4 * B].view(torch.int32).cpu().numpy()


def _sw_call(x, lengths, split=None):
    B, L1, L2 = x.shape
    dev = x.device
    outs = [torch.empty(B, device=dev), torch.empty(B, L1, L2, device=dev),
            torch.empty(B, device=dev), torch.empty(B, device=dev)]
    n = lib().d2p_sw_workspace_bytes(B, L1, L2)
    ws = torch.empty(n, dtype=torch.uint8, device=dev)
    old = os.environ.get("D2P_AMD_SPLIT")
    if split is not None:
        os.environ["D2P_AMD_SPLIT"] = str(split)
    try:
        check(lib().d2p_sw_forward_marginals(ptr(x), ptr(lengths), B, L1, L2, -1.0, 1.0,
                                             *[ptr(o) for o in outs], ptr(ws), n, stream()))
    finally:
        if split is not None:
            if old is None:
                del os.environ["D2P_AMD_SPLIT"]
            else:
                os.environ["D2P_AMD_SPLIT"] = old
    return outs, ws


def _assert_contract(outs, status, reference):
    """Marked elements: every output NaN.  Unmarked: the clean run's results."""
    value, marg, gg, gt = [o.cpu().numpy() for o in outs]
    ref_v, ref_m = reference
    assert status.any(), "no element gave up a wait"
    for b, st in enumerate(status):
        if st:
            assert np.isnan(value[b]) and np.isnan(gg[b]) and np.isnan(gt[b])
            assert np.isnan(marg[b]).all()
        else:
            assert abs(value[b] - ref_v[b]) <= 1e-5 * max(1.0, abs(ref_v[b]))
            assert np.abs(marg[b] - ref_m[b]).max() <= 1e-4


@pytest.mark.parametrize("helpers", ["0", "1"])
@pytest.mark.parametrize("split", [None, 3])
def test_sw_forward_marginals_gives_up_to_nan(cuda, low_spin_limit, monkeypatch, split, helpers):
    # element 0 has one stripe, the others several.  Without helper waves a one-stripe
    # element never waits; with them (parts of at most four stripes: both split
    # settings here) its sweeping wave and its helper wait on each other, so it may be
    # marked too.
    monkeypatch.setenv("D2P_AMD_SW_HELPERS", helpers)
    s = _scores(3, 330, 150, 41)
    lengths = torch.tensor([[50, 150], [330, 150], [260, 120]], dtype=torch.int32)
    part, post, _, _ = O.get("oracle").soft_sw(s.numpy(), -1.0, 1.0, lengths.numpy())
    x, ln = s.to(cuda), lengths.to(cuda)
    outs, ws = _sw_call(x, ln, split)
    status = _status_words(ws, 3)
    assert status[1] != 0 and status[2] != 0
    if helpers == "0":
        assert status[0] == 0
    _assert_contract(outs, status, (part, post))
    st = ctypes.c_int(0)
    check(lib().d2p_sw_status(ptr(ws), 3, ctypes.byref(st), stream()))
    assert st.value != 0


def test_second_order_and_other_families_give_up_to_nan(cuda, low_spin_limit):
    s = _scores(2, 200, 90, 42).to(cuda)
    v = _scores(2, 200, 90, 43).to(cuda)
    # (unsplit soft DTW: its reverse sweep writes the NaN itself, value included)
    dtw = d2p_amd.soft_dtw(s.abs(), temperature=0.5)
    fx, fy = _scores(2, 200, 16, 44).to(cuda), _scores(2, 90, 16, 45).to(cuda)
    dtw_feat = d2p_amd.soft_dtw_sqeuclidean(fx, fy, 0.5)
    outs = {
        "sw_hvp": d2p_amd.soft_sw_hvp(s, v, -1.0, 1.0, None),
        "sw_jac": d2p_amd.soft_sw_param_jacobian(s, 1, -1.0, 1.0, None),
        "sw_full": d2p_amd.soft_sw_backward_full(s, v, -1.0, 1.0, None)[0],
        "nw_hvp": d2p_amd.soft_nw_hvp(s, v, -1.0, 1.0, None),
        "swa": d2p_amd.soft_sw_affine(s, gap_open=-2.0, gap_ext=-0.5).marginals,
        "swa_hvp": d2p_amd.soft_sw_affine_hvp(s, v, -2.0, -0.5, 1.0, None),
        "dtw": dtw.alignment,
        "dtw_cost": dtw.cost,
        "dtw_feat": dtw_feat.alignment,
        "dtw_feat_cost": dtw_feat.cost,
        "dtw_hvp": d2p_amd.soft_dtw_hvp(s.abs(), v, 0.5, None, None),
    }
    torch.cuda.synchronize()
    for name, out in outs.items():
        assert torch.isnan(out).all(), name


def test_torch_layer_raises_when_asked(cuda, low_spin_limit, monkeypatch):
    s = _scores(2, 200, 90, 44).to(cuda)
    r = d2p_amd.soft_sw(s, gap=-1.0, temperature=1.0)
    torch.cuda.synchronize()
    assert torch.isnan(r.value).all() and torch.isnan(r.marginals).all()
    monkeypatch.setenv("D2P_AMD_CHECK_STATUS", "1")
    with pytest.raises(RuntimeError, match="pipeline wait of the DP sweeps gave up"):
        d2p_amd.soft_sw(s, gap=-1.0, temperature=1.0)
    with pytest.raises(RuntimeError, match="gave up"):
        d2p_amd.soft_dtw(s.abs(), temperature=0.5)


def test_default_bound_is_clean_again(cuda, monkeypatch):
    """After the bound is restored the same calls are clean and raise nothing."""
    check(lib().d2p_set_spin_limit(DEFAULT_SPINS))
    monkeypatch.setenv("D2P_AMD_CHECK_STATUS", "1")
    s = _scores(3, 330, 150, 41)
    lengths = torch.tensor([[50, 150], [330, 150], [260, 120]], dtype=torch.int32)
    part, post, _, _ = O.get("oracle").soft_sw(s.numpy(), -1.0, 1.0, lengths.numpy())
    r = d2p_amd.soft_sw(s.to(cuda), gap=-1.0, temperature=1.0, lengths=lengths.to(cuda))
    assert np.abs(r.marginals.cpu().numpy() - post).max() <= 1e-4
    outs, ws = _sw_call(s.to(cuda), lengths.to(cuda), 3)
    assert not _status_words(ws, 3).any()
