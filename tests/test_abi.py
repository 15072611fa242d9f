"""CPU-side checks of the C ABI: the library loads, exports exactly what
include/u15h.h declares, and its host-only logic behaves (no GPU calls)."""
import ctypes

import numpy as np
import pytest

import u15h


def test_library_exports_every_declared_symbol():
    lib = u15h.load_library()
    declared = u15h.declared_symbols()
    assert len(declared) >= 18
    missing = [s for s in declared if not hasattr(lib, s)]
    assert missing == []


def test_abi_version_and_status_strings():
    lib = u15h.load_library()
    assert lib.u15h_abi_version() == 1
    for st in range(5):
        assert lib.u15h_status_str(st)
    assert lib.u15h_status_str(99) == b"unknown status"


def test_null_context_is_rejected_without_a_device():
    lib = u15h.load_library()
    assert lib.u15h_linear(None, None, None, None, None, None, 1, 8, 8) == u15h.EINVAL
    assert lib.u15h_enable_i8_gemm(None, 1) == 0
    assert lib.u15h_last_error(None) == b"null context"
    lib.u15h_destroy(None)                 # no-op
    assert lib.u15h_create(0, None) == u15h.EINVAL


def test_create_refuses_without_gfx950():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present; covered by the GPU tests")
    lib = u15h.load_library()
    ctx = ctypes.c_void_p()
    assert lib.u15h_create(0, ctypes.byref(ctx)) == u15h.ENODEV
    assert not ctx.value


def test_route_rows_is_a_stable_partition():
    rng = np.random.default_rng(0)
    e = rng.integers(0, 2, 1000).astype(np.uint8)
    perm, mu, mg = u15h.route_rows(e)
    assert mu == int((e == 0).sum()) and mg == 1000 - mu
    assert np.array_equal(perm[:mu], np.flatnonzero(e == 0))
    assert np.array_equal(perm[mu:], np.flatnonzero(e == 1))
    assert sorted(perm.tolist()) == list(range(1000))


def test_route_rows_edge_cases():
    perm, mu, mg = u15h.route_rows([])
    assert (len(perm), mu, mg) == (0, 0, 0)
    perm, mu, mg = u15h.route_rows([1, 1, 1])
    assert (list(perm), mu, mg) == ([0, 1, 2], 0, 3)
    with pytest.raises(u15h.U15hError):
        u15h.route_rows([0, 2])


def test_build_rope_tables_matches_oracle():
    """u15h_build_rope_tables is host code (no device): bit-equal to the
    oracle's restatement of build_rope_tables, including long positions."""
    import numpy as np
    import oracle
    rng = np.random.default_rng(4)
    T, D = 50, 128
    pt = rng.integers(0, 20000, T)
    ph = rng.integers(0, 64, T)
    pw = rng.integers(0, 64, T)
    c, s = u15h.build_rope_tables(pt, ph, pw, D, 64, 32)
    oc, osn = oracle.rope_tables(pt, ph, pw, D, 64, 32)
    assert np.array_equal(c, oc) and np.array_equal(s, osn)
    with pytest.raises(u15h.U15hError):
        u15h.build_rope_tables(pt, ph, pw, D, 64, 30)   # 64 + 60 != 128
    c0, s0 = u15h.build_rope_tables([], [], [], D, 64, 32)
    assert c0.shape == (0, D)


def test_qweight_geometry_rule():
    """bind_matrix_'s shape rule (src/u15-weights.cc:247-325)."""
    assert u15h.qweight_geometry(4096, 64, 1024) == (8, 64)
    assert u15h.qweight_geometry(4096, 128, 512) == (4, 32)
    assert u15h.qweight_geometry(12288, 192, 3072) == (8, 64)
    for K, sc, cc in ((4096, 100, 1024), (4096, 64, 1000), (4096, 16, 1024),
                      (4096, 64, 2048), (4096, 0, 1024), (0, 64, 1024),
                      (4096, 128, 768)):
        with pytest.raises(u15h.U15hError):
            u15h.qweight_geometry(K, sc, cc)
