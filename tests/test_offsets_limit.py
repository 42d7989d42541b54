"""32-bit offsets at the largest shapes the C ABI accepts (CPU only, no kernel runs).

The entry points accept any element the reference accepts, (L1 + 1)(L2 + 1) <=
INT32_MAX, with max_L2 <= 262080 and max_L1 <= 2097088 (the stripe pipeline's chunk
and stripe counters).  The kernels keep 64-bit (size_t) bases per element, stripe and
table plane, and 32-bit per-lane offsets from those bases.  This test evaluates the
largest value each 32-bit offset expression takes, with Python's exact integers, at
the limit shapes, and checks it against the type it is held in:

- matrix offsets from a stripe's first row (dma_tile, dma_quads, write_quads and
  write_tile inside chunks, stage_quads, stage_row; wavefront.hip.h): at most 64
  rows plus a chunk, as uint32 bytes;
- the one absolute matrix offset, the boundary form of write_quads
  (row * L2max + col, wavefront.hip.h): int32 floats;
- skewed-table rows (dma_rows, stage_rows, the checkpoint loads): step * 256 bytes
  plus the lane's 16-byte quad, uint32;
- last rows and boundary flows by step (roff, foff and their affine and
  second-order forms): at most four floats plus one per step, uint32 bytes;
- progress words: stripe * 65536 + chunks in an int, with at most 65536 chunks (only
  >= comparisons read them, so a stripe's final word may equal the next stripe
  index's base).

The limit shapes: a square [33000, 33000] (1.09e9 cells, the GPU test's size), the
longest rows [8192, 262080], the most rows [2097088, 1023], and the reference's affine
CUDA limit 3 (L1 + 1)(L2 + 1) <= INT32_MAX, [26753, 26753].  The C ABI must accept
each (only the deliberately short workspace is refused).
"""
import ctypes
import os

import pytest

import _capi

INT32_MAX = 2 ** 31 - 1
UINT32_MAX = 2 ** 32 - 1
APAD, STEP_QUANTUM, MAX_L2, MAX_L1 = 18, 16, (1 << 18) - 64, 32767 * 64
FAKE = ctypes.c_void_p(0x1000)

SHAPES = [(33000, 33000), (8192, 262080), (2097088, 1023), (26753, 26753)]


def stored_steps(L2max):
    return APAD + (L2max + 63 + STEP_QUANTUM - 1) // STEP_QUANTUM * STEP_QUANTUM


def max_offsets(L1max, L2max):
    """Largest value of each 32-bit offset expression (bytes unless stated)."""
    nsteps = L2max + 63
    P_max = 20                      # the widest per-lane window (stage_row of 5 quads)
    stripe_rel = (63 * L2max + (L2max - 1) + P_max) * 4
    absolute = (L1max - 1) * L2max + (L2max - 1)          # floats, int32
    table_row = (stored_steps(L2max) + APAD) * 256 + 16 * 63
    flows = ((nsteps + 63) * 4 + 4 * 16 + 3) * 4
    ns = (L1max + 63) // 64
    nch_min_p = (nsteps + 3) // 4                          # chunks of the shortest P (4)
    progress = (ns - 1) * 65536 + nch_min_p
    return dict(stripe_rel=stripe_rel, absolute=absolute, table_row=table_row, flows=flows,
                progress=progress, chunks=nch_min_p)


@pytest.mark.parametrize("L1,L2", SHAPES)
def test_offsets_fit_their_types(L1, L2):
    assert (L1 + 1) * (L2 + 1) <= INT32_MAX and L2 <= MAX_L2 and L1 <= MAX_L1
    m = max_offsets(L1, L2)
    assert m["stripe_rel"] <= UINT32_MAX
    assert m["absolute"] <= INT32_MAX
    assert m["table_row"] <= UINT32_MAX
    assert m["flows"] <= UINT32_MAX
    assert m["progress"] <= INT32_MAX and m["chunks"] <= 1 << 16


def test_the_limits_are_tight():
    """One more row or column breaks the reference's rule or a pipeline counter."""
    assert (33000 + 1) * (33000 + 1) <= INT32_MAX
    assert (8193 + 1) * (262080 + 1) > INT32_MAX
    assert (2097088 + 1) * (1024 + 1) > INT32_MAX
    assert 3 * (26754 + 1) * (26754 + 1) > INT32_MAX >= 3 * (26753 + 1) * (26753 + 1)
    assert max_offsets(64, MAX_L2 + 64)["chunks"] > 1 << 16


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_capi.LIB_PATH):
        pytest.skip("libd2p_amd.so not built (run __graft_entry__.build())")
    return _capi.lib()


@pytest.mark.parametrize("L1,L2", SHAPES)
def test_c_abi_accepts_the_limit_shapes(lib, L1, L2):
    for fn, extra in ((lib.d2p_sw_forward_marginals, ()),
                      (lib.d2p_dtw_forward_marginals, None)):
        need = (lib.d2p_sw_workspace_bytes if extra is not None
                else lib.d2p_dtw_workspace_bytes)(1, L1, L2)
        assert need >= (L1 + 1) * (L2 + 1) * 4
    z = ctypes.c_size_t(64)
    rc = lib.d2p_sw_forward_marginals(FAKE, FAKE, 1, L1, L2, -1.0, 1.0, FAKE, FAKE, FAKE, FAKE,
                                      FAKE, z, None)
    assert rc == 1 and b"workspace" in lib.d2p_last_error()
    rc = lib.d2p_swa_forward_marginals(FAKE, FAKE, 1, L1, L2, -2.0, -0.5, 1.0, FAKE, FAKE, FAKE,
                                       FAKE, FAKE, FAKE, z, None)
    assert rc == 1 and b"workspace" in lib.d2p_last_error()
    rc = lib.d2p_dtw_forward_marginals(FAKE, FAKE, 1, L1, L2, 1.0, -1, FAKE, FAKE, FAKE, FAKE,
                                       z, None)
    assert rc == 1 and b"workspace" in lib.d2p_last_error()
