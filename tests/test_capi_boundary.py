"""The C ABI boundary on the host (no GPU needed): libd2p_amd.so loads, exports
every function include/d2p_amd.h declares, the test bindings cover all of them,
workspace sizes follow the documented layout, and argument validation rejects
bad calls with a message before any device work is enqueued.

Every call here returns from host-side checks; pointer arguments that must be
non-null are dummies that are never dereferenced.
"""
import ctypes
import os
import re
import subprocess

import pytest

import _capi

D2P_OK, D2P_ERR_ARG = 0, 1
FAKE = ctypes.c_void_p(0x1000)        # non-null, never dereferenced by the host checks


def declared_functions():
    text = open(_capi.HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(d2p_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_capi.LIB_PATH):
        pytest.skip("libd2p_amd.so not built (run __graft_entry__.build())")
    return _capi.lib()


def test_header_declares_entry_points():
    names = declared_functions()
    assert len(names) >= 25
    for fam in ("sw", "swa", "dtw"):
        for suffix in ("workspace_bytes", "forward_marginals", "second_workspace_bytes", "hvp",
                       "param_jacobian", "backward_full"):
            assert f"d2p_{fam}_{suffix}" in names


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", _capi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\s[TW]\s+(d2p_\w+)$", out, flags=re.M))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing
    for n in declared_functions():
        assert getattr(lib, n) is not None


def test_bindings_cover_header():
    assert sorted(_capi.SIGNATURES) == declared_functions()


def test_abi_version_and_error_string(lib):
    assert lib.d2p_abi_version() == 1
    assert isinstance(lib.d2p_last_error(), bytes)


@pytest.mark.parametrize("fn,planes", [("d2p_sw_workspace_bytes", 1),
                                       ("d2p_swa_workspace_bytes", 3),
                                       ("d2p_nwa_workspace_bytes", 3),
                                       ("d2p_dtw_workspace_bytes", 1)])
def test_workspace_sizes(lib, fn, planes):
    f = getattr(lib, fn)
    assert f(0, 10, 10) == 0 and f(-1, 10, 10) == 0 and f(2, -1, 10) == 0
    small, big = f(2, 100, 120), f(2, 100, 1200)
    assert small > 0 and big > small
    assert f(4, 100, 120) > small
    # skewed table: stripes of 64 rows x (18 pad + ceil((L2 + 63) / 16) * 16 steps) x 64
    # floats per plane, plus one last row per stripe and plane
    steps = 18 + (120 + 63 + 15) // 16 * 16
    table = 2 * 2 * planes * steps * (64 + 1) * 4
    if fn in ("d2p_sw_workspace_bytes", "d2p_dtw_workspace_bytes"):
        # split elements: boundary flows, one (up, diagonal) pair per stripe and step
        table += 2 * 2 * steps * 2 * 4
    else:
        # split elements: boundary flows, a float4 and a float2 per stripe and step (the
        # global alignment's second flow entry is a pair)
        table += 2 * 2 * steps * 6 * 4
    assert table <= small <= table + 4096
    # every workspace starts with status words: never zero for B > 0
    assert f(1, 0, 0) > 0


def test_second_workspaces_hold_the_first(lib):
    steps = 18 + (90 + 63 + 15) // 16 * 16
    for first, second, planes in (
            ("d2p_sw_workspace_bytes", "d2p_sw_second_workspace_bytes", 1),
            ("d2p_swa_workspace_bytes", "d2p_swa_second_workspace_bytes", 3),
            ("d2p_nwa_workspace_bytes", "d2p_nwa_second_workspace_bytes", 3),
            ("d2p_dtw_workspace_bytes", "d2p_dtw_second_workspace_bytes", 1)):
        a = getattr(lib, first)(3, 200, 90)
        b = getattr(lib, second)(3, 200, 90)
        tangent = 3 * 4 * planes * steps * (64 + 1) * 4
        assert b >= a + tangent       # primal workspace plus tangent tables


def _err(lib):
    return lib.d2p_last_error().decode()


def test_scale_by_batch_validation(lib):
    """Argument checks that run before any device work (no GPU needed)."""
    rc = lib.d2p_scale_by_batch_strided(FAKE, FAKE, -1, FAKE, 2, 16, None)
    assert rc == D2P_ERR_ARG and "negative factor stride" in _err(lib)
    rc = lib.d2p_scale_by_batch_strided(FAKE, FAKE, 0, FAKE, -1, 16, None)
    assert rc == D2P_ERR_ARG and "negative" in _err(lib)
    rc = lib.d2p_scale_by_batch(FAKE, FAKE, FAKE, 2, -3, None)
    assert rc == D2P_ERR_ARG and "negative" in _err(lib)
    rc = lib.d2p_scale_by_batch_lengths(FAKE, FAKE, -1, FAKE, FAKE, 2, 4, 4, None)
    assert rc == D2P_ERR_ARG and "negative factor stride" in _err(lib)
    rc = lib.d2p_scale_by_batch_lengths(FAKE, FAKE, 0, FAKE, FAKE, 2, -4, 4, None)
    assert rc == D2P_ERR_ARG and "negative" in _err(lib)
    assert lib.d2p_scale_by_batch_lengths(None, None, 0, None, None, 0, 4, 4, None) == 0
    # empty work is a no-op, even with null pointers
    assert lib.d2p_scale_by_batch_strided(None, None, 0, None, 0, 16, None) == 0
    assert lib.d2p_scale_by_batch(None, None, None, 4, 0, None) == 0


def test_forward_validation(lib):
    z = ctypes.c_size_t(1 << 20)
    rc = lib.d2p_sw_forward_marginals(FAKE, FAKE, 2, 10, 10, -1.0, 0.0, FAKE, FAKE, FAKE, FAKE,
                                      FAKE, z, None)
    assert rc == D2P_ERR_ARG and "temperature" in _err(lib)
    rc = lib.d2p_swa_forward_marginals(FAKE, FAKE, -1, 10, 10, -2.0, -0.5, 1.0, FAKE, FAKE, FAKE,
                                       FAKE, FAKE, FAKE, z, None)
    assert rc == D2P_ERR_ARG and "negative" in _err(lib)
    rc = lib.d2p_dtw_forward_marginals(FAKE, FAKE, 2, 10, 10, 1.0, -1, FAKE, FAKE, FAKE, None,
                                       z, None)
    assert rc == D2P_ERR_ARG and "workspace" in _err(lib)
    rc = lib.d2p_sw_forward_marginals(None, FAKE, 2, 10, 10, -1.0, 1.0, FAKE, FAKE, FAKE, FAKE,
                                      FAKE, z, None)
    assert rc == D2P_ERR_ARG and "null" in _err(lib)
    rc = lib.d2p_sw_forward_marginals(FAKE, FAKE, 2, 10, 10, -1.0, 1.0, FAKE, FAKE, FAKE, FAKE,
                                      FAKE, ctypes.c_size_t(64), None)
    assert rc == D2P_ERR_ARG and "workspace" in _err(lib)
    rc = lib.d2p_sw_forward_marginals(FAKE, FAKE, 2, 10, 1 << 20, -1.0, 1.0, FAKE, FAKE, FAKE,
                                      FAKE, FAKE, z, None)
    assert rc == D2P_ERR_ARG and "max_L2 exceeds" in _err(lib)


def test_empty_batch_is_a_no_op(lib):
    assert lib.d2p_sw_forward_marginals(None, None, 0, 10, 10, -1.0, 1.0, None, None, None,
                                        None, None, 0, None) == D2P_OK
    assert lib.d2p_swa_hvp(None, None, None, 0, 5, 5, -2.0, -0.5, 1.0, None, None, 0,
                           None) == D2P_OK
    assert lib.d2p_dtw_backward_full(None, None, None, 0, 5, 5, 1.0, -1, None, None, None, 0,
                                     None) == D2P_OK


def test_second_order_validation(lib):
    z = ctypes.c_size_t(1 << 30)
    rc = lib.d2p_sw_param_jacobian(FAKE, 2, FAKE, 2, 10, 10, -1.0, 1.0, FAKE, FAKE, z, None)
    assert rc == D2P_ERR_ARG and "param_type" in _err(lib)
    rc = lib.d2p_swa_param_jacobian(FAKE, 3, FAKE, 2, 10, 10, -2.0, -0.5, 1.0, FAKE, FAKE, z,
                                    None)
    assert rc == D2P_ERR_ARG and "param_type" in _err(lib)
    rc = lib.d2p_dtw_hvp(FAKE, FAKE, FAKE, 2, 10, 10, 0.0, -1, FAKE, FAKE, z, None)
    assert rc == D2P_ERR_ARG and "temperature" in _err(lib)
    rc = lib.d2p_swa_backward_full(FAKE, FAKE, FAKE, 2, 10, 10, -2.0, -0.5, 1.0, FAKE, FAKE,
                                   FAKE, FAKE, FAKE, ctypes.c_size_t(8), None)
    assert rc == D2P_ERR_ARG and "workspace" in _err(lib)
    # more stripes than waves and rows too long for unsplit stripe rings: every sweep
    # splits such elements into parts instead of refusing them; the workspace check
    # still runs before any device work
    rc = lib.d2p_sw_hvp(FAKE, FAKE, FAKE, 1, 1024, 200000, -1.0, 1.0, FAKE, FAKE, z, None)
    assert rc == D2P_ERR_ARG and "workspace" in _err(lib)
    rc = lib.d2p_swa_hvp(FAKE, FAKE, FAKE, 1, 1024, 200000, -2.0, -0.5, 1.0, FAKE, FAKE, z, None)
    assert rc == D2P_ERR_ARG and "workspace" in _err(lib)
    rc = lib.d2p_dtw_hvp(FAKE, FAKE, FAKE, 1, 1024, 200000, 1.0, -1, FAKE, FAKE, z, None)
    assert rc == D2P_ERR_ARG and "workspace" in _err(lib)


def test_profile_report_buffer(lib):
    buf = ctypes.create_string_buffer(0)
    assert lib.d2p_profile_report(buf, 0) == D2P_ERR_ARG
    lib.d2p_profile_reset()
    buf = ctypes.create_string_buffer(256)
    assert lib.d2p_profile_report(buf, 256) == D2P_OK


def test_c_abi_accepts_the_reference_table_range(lib):
    """The C ABI sizes a workspace for any table the reference accepts, up to
    (L1 + 1) * (L2 + 1) = INT32_MAX (here [1, 40000, 40000], 1.6e9 cells), and
    rejects the next shape up; no kernel runs."""
    assert lib.d2p_sw_workspace_bytes(1, 40000, 40000) > 40000 * 40000 * 4
    rc = lib.d2p_sw_forward_marginals(FAKE, FAKE, 1, 46341, 46341, -1.0, 1.0, FAKE, FAKE, FAKE,
                                      FAKE, FAKE, 1 << 40, None)
    assert rc == D2P_ERR_ARG and b"DP table too large" in lib.d2p_last_error()
    # rows longer than the pipeline's chunk counters allow: its own message
    rc = lib.d2p_swa_forward_marginals(FAKE, FAKE, 1, 2, 262081, -2.0, -0.5, 1.0, FAKE, FAKE,
                                       FAKE, FAKE, FAKE, FAKE, 1 << 40, None)
    assert rc == D2P_ERR_ARG and b"max_L2 exceeds 262080" in lib.d2p_last_error()


def test_pairwise_sqdist_has_no_grid_limits(lib):
    """d2p_pairwise_sqdist strides over batch elements and row tiles, so shapes past
    the grid extents (B > 65535, L1 > 32 * 65535) reach the null-pointer check
    instead of a size limit; D outside [1, 128] is refused.  No kernel runs."""
    rc = lib.d2p_pairwise_sqdist(None, FAKE, 70000, 3_000_000, 8, 16, FAKE, None)
    assert rc == D2P_ERR_ARG and "null pointer" in _err(lib)
    rc = lib.d2p_pairwise_sqdist(FAKE, FAKE, 2, 4, 4, 129, FAKE, None)
    assert rc == D2P_ERR_ARG and "feature dimension" in _err(lib)
    assert lib.d2p_pairwise_sqdist(None, None, 70000, 0, 8, 16, None, None) == D2P_OK
