"""Sakoe-Chiba band windows of the soft-DTW sweeps (CPU, no GPU needed).

With a band every stripe of 64 rows sweeps only the steps of its window, and the
skewed tables keep only those steps at a per-element stripe stride.  These tests
restate the window and size rules of d2p_amd/csrc/dtw_internal.hip.h in float32
numpy and check, by brute force over the cells, the properties the kernels rely on:

- every in-band cell (the reference's float test |j - i*L2/L1| <= bw,
  /root/reference/src/dtw/kernels_cpu.cpp:24-29) lies inside its stripe's window;
- window starts never move left from one stripe to the next (a stripe never reads
  last-row steps of the stripe above that lie before that stripe's window);
- a stripe's stored steps (APAD + its forward chunks + one trailing chunk) fit the
  stripe stride, the stripes of any element fit the per-element reservation, and the
  reverse sweeps' table reads (first chunk up to its top step, last chunk down to
  P + 1 steps below) stay inside the stored steps for P = 16, 8 and 4.
"""
import numpy as np
import pytest

APAD, PF = 18, 16


def stored_steps(L2max):
    return APAD + ((L2max + 63 + 15) // 16) * 16


def centre(i, L1, L2):
    return np.float32(np.float32(i * L2) / np.float32(L1))


def band_cap(bw):
    return min(bw, 1 << 20)


def margin(bw):
    return 2 * band_cap(bw) + 160


def window(s, L1, L2, bw):
    i0 = 64 * s
    rows = min(64, L1 - i0)
    lo = max(int(np.floor(centre(i0 + 1, L1, L2))) - bw - 2, 0)
    hi = min(int(np.ceil(centre(i0 + rows, L1, L2))) + bw, L2 - 1)
    return lo, hi + rows - 1


def stride(L1, L2, bw, NT):
    r = min(64, L1) - 1
    span = (r * L2 + L1 - 1) // L1
    return min(NT, margin(bw) + span)


def elem_steps(max_L1, max_L2, bw):
    ns = (max_L1 + 63) // 64
    full = ns * stored_steps(max_L2)
    return min(full, ns * (margin(bw) + 1) + 2 * max_L2)


def in_band_cells(L1, L2, bw):
    i = np.arange(1, L1 + 1)
    j = np.arange(1, L2 + 1, dtype=np.float32)
    e = (np.float32(1) * (i * L2).astype(np.float32) / np.float32(L1)).astype(np.float32)
    return np.abs(j[None, :] - e[:, None]) <= np.float32(bw)


SHAPES = [(1, 1), (1, 300), (300, 1), (64, 64), (65, 65), (100, 37), (37, 100),
          (256, 256), (513, 129), (129, 513), (700, 170), (1000, 64), (64, 1000),
          (4096, 4096), (4096, 300), (300, 4096), (1234, 3000)]


@pytest.mark.parametrize("L1,L2", SHAPES)
@pytest.mark.parametrize("bw", [0, 1, 3, 10, 40, 200])
def test_windows_cover_the_band(L1, L2, bw):
    if L1 * L2 > 4_000_000:
        pytest.skip("brute force only on moderate shapes")
    band = in_band_cells(L1, L2, bw)
    NT = stored_steps(L2)
    nsteps, nch = L2 + 63, (L2 + 63 + PF - 1) // PF
    st = stride(L1, L2, bw, NT)
    prev = None
    for s in range((L1 + 63) // 64):
        lo, hi = window(s, L1, L2, bw)
        rows = band[64 * s:64 * s + 64]
        r, c = np.nonzero(rows)
        if len(r):
            t = c + r
            assert lo <= t.min() and t.max() <= hi, (s, lo, hi, t.min(), t.max())
        if prev is not None:
            assert lo >= prev
        prev = lo
        if lo > hi:
            continue
        k_lo, k_hi = lo // PF, hi // PF
        k_top = min(k_hi + 2, nch)            # stored: [k_lo*PF - APAD, k_top*PF)
        assert APAD + (k_top - k_lo) * PF <= st
        for P in (16, 8, 4):
            kb_lo, kb_end = (nsteps - 1 - hi) // P, (nsteps - 1 - lo) // P + 1
            th0 = nsteps - 1 - kb_lo * P
            th_last = nsteps - 1 - (kb_end - 1) * P
            assert th0 <= k_top * PF - 1 and th0 - 1 >= k_lo * PF - APAD
            assert th_last - P - 1 >= k_lo * PF - APAD


@pytest.mark.parametrize("max_L1,max_L2", [(64, 64), (300, 257), (1024, 1024), (4096, 4096),
                                           (5000, 70), (70, 5000)])
@pytest.mark.parametrize("bw", [0, 5, 64, 500, 1 << 30])
def test_elements_fit_their_reservation(max_L1, max_L2, bw):
    NT = stored_steps(max_L2)
    cap = elem_steps(max_L1, max_L2, bw)
    rng = np.random.default_rng(max_L1 * 7 + max_L2)
    L1s = np.unique(np.concatenate([np.arange(1, min(max_L1, 200) + 1),
                                    rng.integers(1, max_L1 + 1, 300), [max_L1]]))
    L2s = np.unique(np.concatenate([np.arange(1, min(max_L2, 200) + 1, 7),
                                    rng.integers(1, max_L2 + 1, 60), [max_L2]]))
    for L1 in L1s:
        ns = (int(L1) + 63) // 64
        for L2 in L2s:
            assert ns * stride(int(L1), int(L2), bw, NT) <= cap, (L1, L2)
    # the banded reservation is far below the full table for narrow bands of
    # sequences of similar lengths
    if bw <= 64 and max_L2 >= 1024 and max_L1 >= max_L2:
        assert cap < (max_L1 + 63) // 64 * NT / 2
