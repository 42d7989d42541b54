"""An element past the pipeline's former 2^30-cell limit: one [1, 33000, 33000] soft-SW
element (1.089e9 cells, (L1 + 1)(L2 + 1) within the reference's INT32_MAX rule) through
the C ABI, so that every offset of the sweeps (scores, marginals, the skewed table and
its checkpoint rows, last rows, split-part flows) runs at its largest values.

The oracle needs minutes for a table this size, so the input is built to have a known
answer: scores of -100 everywhere except two 256 x 256 blocks of N(0,1) scores, one
near the top-left corner and one in the bottom-right corner, with gap = -50 and T = 1.
Every candidate that crosses from outside into a block (or back) then carries a factor
below 2^-149 in fp32, i.e. exactly 0, so each block's alphas and betas are those of
the block as an element of its own, and the cells outside add nothing representable to
the partition.  With Z_k the partition of block k on its own (its alpha[0,0] = 0 term
included) and the table's one alpha[0,0] term, the expected results are
    S = log(Z_1 + Z_2 - 1),   marginals in block k = P_k * Z_k / e^S,
    marginals elsewhere = 0,  grad_gap = sum_k g_k * Z_k / e^S,
    grad_T = (S - (sum_k Z_k / e^S * <P_k, s_k> + grad_gap * gap)) / T,
from the oracle on each block, held to the north-star tolerances.
"""
import numpy as np
import pytest
import torch

import _capi
from oracle import oracle as O

pytestmark = pytest.mark.gpu

L = 33000
BLK = 256


def test_sw_element_past_2_30_cells(cuda):
    gap, T = -50.0, 1.0
    g = torch.Generator().manual_seed(70)
    blocks = [torch.randn(BLK, BLK, generator=g), torch.randn(BLK, BLK, generator=g)]
    origins = [(100, 200), (L - BLK, L - BLK)]
    print(f"[1, {L}, {L}] soft_sw, two {BLK}^2 blocks", flush=True)
    s = torch.full((1, L, L), -100.0, device=cuda)
    for (r, c), blk in zip(origins, blocks):
        s[0, r:r + BLK, c:c + BLK] = blk.to(cuda)
    part, marg, gg, gt = _capi.sw_forward_marginals(s, None, gap, T)
    torch.cuda.synchronize()
    del s

    k = O.get("oracle")
    refs = [k.soft_sw(blk.numpy()[None], gap, T) for blk in blocks]
    Sk = np.array([float(r[0][0]) for r in refs])
    S = np.log(np.exp(Sk).sum() - 1.0)
    w = np.exp(Sk - S)
    assert abs(float(part[0]) - S) <= 1e-5 * abs(S), (float(part[0]), S)

    for (r, c), ref, wk in zip(origins, refs, w):
        got = marg[0, r:r + BLK, c:c + BLK].cpu().numpy()
        assert np.abs(got - ref[1][0] * wk).max() <= 1e-4
        marg[0, r:r + BLK, c:c + BLK] = 0.0
    assert float(marg.abs().max()) <= 1e-6

    g_exp = float(sum(ref[2][0] * wk for ref, wk in zip(refs, w)))
    np.testing.assert_allclose(float(gg[0]), g_exp, rtol=3e-4)
    e_exp = sum(wk * float((ref[1][0].astype(np.float64) * blk.numpy()).sum())
                for ref, wk, blk in zip(refs, w, blocks))
    t_exp = (S - (e_exp + g_exp * gap)) / T
    assert abs(float(gt[0]) - t_exp) <= 1e-3 * abs(t_exp) + 2e-5 * (abs(S) + 1.0) / T
