"""GPU behaviour of the public API around the kernels: bf16 autocast and
torch.compile tracing.

* Autocast (behaviour of /root/reference/d2p/_compile.py:857-931): under
  torch.autocast("cuda", bfloat16) every d2p op upcasts its floating inputs to
  float32, so outputs are float32, the value equals the float32 run on the
  upcast input (same kernels, same bits), and the gradient flows back to the
  bfloat16 input in its own dtype.
* torch.compile: the public functions route traced calls to the d2p_py custom
  ops; the compiled value and gradient equal the eager ones.
"""
import pytest
import torch

import d2p_amd

pytestmark = pytest.mark.gpu


def _seeded(seed, shape, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32) * scale


@pytest.mark.parametrize("family", ["sw", "swa", "dtw"])
def test_bf16_autocast_upcasts(cuda, family):
    x16 = _seeded(1, (3, 70, 90)).to(cuda).bfloat16()
    if family == "dtw":
        x16 = x16.abs()
    fn = {"sw": lambda s: d2p_amd.soft_sw(s, gap=-1.0, temperature=1.0),
          "swa": lambda s: d2p_amd.soft_sw_affine(s, gap_open=-11.0, gap_ext=-1.0,
                                                  temperature=0.5),
          "dtw": lambda s: d2p_amd.soft_dtw(s, temperature=0.5)}[family]
    x = x16.clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        r = fn(x)
    value, marg = r[0], r[1]
    assert value.dtype == torch.float32 and marg.dtype == torch.float32
    value.sum().backward()
    assert x.grad.dtype == torch.bfloat16
    ref = fn(x16.float().detach())
    assert torch.equal(value, ref[0]) and torch.equal(marg, ref[1])
    assert torch.equal(x.grad, ref[1].bfloat16())


def test_bf16_autocast_second_order_ops(cuda):
    s = _seeded(2, (2, 40, 50)).to(cuda)
    v = _seeded(3, (2, 40, 50)).to(cuda)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        h = d2p_amd.soft_sw_hvp(s.bfloat16(), v.bfloat16(), -1.0, 1.0, None)
    assert h.dtype == torch.float32
    ref = d2p_amd.soft_sw_hvp(s.bfloat16().float(), v.bfloat16().float(), -1.0, 1.0, None)
    assert torch.equal(h, ref)


def test_torch_compile_matches_eager(cuda):
    s = _seeded(4, (2, 60, 64)).to(cuda)
    w = _seeded(5, (2, 60, 64)).to(cuda)

    def loss(x):
        r = d2p_amd.soft_sw(x, gap=-1.0, temperature=0.8)
        return r.value.sum() + (r.marginals * w).sum()

    compiled = torch.compile(loss, backend="aot_eager", fullgraph=True)
    xe = s.clone().requires_grad_(True)
    le = loss(xe)
    le.backward()
    xc = s.clone().requires_grad_(True)
    lc = compiled(xc)
    lc.backward()
    assert torch.allclose(lc, le, rtol=1e-6, atol=1e-5)
    assert torch.allclose(xc.grad, xe.grad, rtol=1e-5, atol=1e-5)


def test_torch_compile_dtw_and_affine(cuda):
    c = _seeded(6, (2, 48, 40)).to(cuda).abs()
    s = _seeded(7, (2, 48, 40)).to(cuda)

    def f(x, y):
        return (d2p_amd.soft_dtw(x, temperature=0.3).cost.sum()
                + d2p_amd.soft_sw_affine(y, gap_open=-2.0, gap_ext=-0.5).value.sum())

    compiled = torch.compile(f, backend="aot_eager")
    xe, ye = c.clone().requires_grad_(True), s.clone().requires_grad_(True)
    f(xe, ye).backward()
    xc, yc = c.clone().requires_grad_(True), s.clone().requires_grad_(True)
    compiled(xc, yc).backward()
    assert torch.allclose(xc.grad, xe.grad, atol=1e-6) and torch.allclose(yc.grad, ye.grad,
                                                                          atol=1e-6)


def test_torch_compile_nw(cuda):
    """soft_nw under torch.compile (fake kernels for shapes), through both outputs."""
    s = _seeded(8, (2, 40, 52)).to(cuda)
    w = _seeded(9, (2, 40, 52)).to(cuda)

    def loss(x):
        r = d2p_amd.soft_nw(x, gap=-1.0, temperature=0.8)
        return r.score.sum() + (r.alignment * w).sum()

    compiled = torch.compile(loss, backend="aot_eager", fullgraph=True)
    xe = s.clone().requires_grad_(True)
    le = loss(xe)
    le.backward()
    xc = s.clone().requires_grad_(True)
    lc = compiled(xc)
    lc.backward()
    assert torch.allclose(lc, le, rtol=1e-6, atol=1e-5)
    assert torch.allclose(xc.grad, xe.grad, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("family", ["sw", "nw", "swa", "nwa", "dtw"])
def test_torch_compile_learnable_parameters(cuda, family):
    """Modules with learnable parameters under torch.compile: the compiled backward
    runs the kernels with the forward's own gap/temperature values (tensors saved for
    backward, not placeholders), on the value path and on the marginal path."""
    torch.manual_seed(0)
    s = _seeded(10, (2, 40, 48)).to(cuda)
    w = _seeded(11, (2, 40, 48)).to(cuda)
    if family == "dtw":
        s = s.abs()
    make = {"sw": lambda: d2p_amd.SoftSW(gap=-0.7, temperature=0.6, learn_gap=True,
                                         learn_temperature=True),
            "nw": lambda: d2p_amd.SoftNW(gap=-0.7, temperature=0.6, learnable=True),
            "swa": lambda: d2p_amd.SoftSWAffine(gap_open=-1.5, gap_ext=-0.4, temperature=0.6,
                                                learn_gap_open=True, learn_gap_ext=True,
                                                learn_temperature=True),
            "nwa": lambda: d2p_amd.SoftNWAffine(gap_open=-1.5, gap_ext=-0.4, temperature=0.6,
                                                learnable=True),
            "dtw": lambda: d2p_amd.SoftDTW(temperature=0.6, learnable=True)}[family]

    def run(mod, x):
        r = mod(x)
        return r[0].sum() + (r[1] * w).sum()

    results = []
    for compiled in (False, True):
        mod = make().to(cuda)
        x = s.clone().requires_grad_(True)
        fn = torch.compile(run, backend="aot_eager") if compiled else run
        loss = fn(mod, x)
        loss.backward()
        results.append((loss.detach(), x.grad, [p.grad.clone() for p in mod.parameters()]))
    (le, ge, pe), (lc, gc, pc) = results
    assert len(pe) == len(pc) > 0
    assert torch.allclose(lc, le, rtol=1e-6, atol=1e-5)
    assert torch.allclose(gc, ge, rtol=1e-5, atol=1e-5)
    for a, b in zip(pc, pe):
        assert torch.allclose(a, b, rtol=1e-5, atol=1e-4), (a, b)
