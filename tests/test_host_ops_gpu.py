"""The host-pointer element-wise ops through logan-metal's C names
(coli_metal_rmsnorm / coli_metal_add / coli_metal_silu_mul,
logan-metal/src/lib.rs:454-456; backend_metal.mm:2147-2204) against the
oracle: in place on host f32 arrays, 1 on success, 0 on bad arguments."""
import ctypes as C

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def _lib():
    from logan_amd import _lib

    h = _lib.lib()
    h.coli_metal_rmsnorm.restype = C.c_int32
    h.coli_metal_rmsnorm.argtypes = [C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_float]
    h.coli_metal_add.restype = C.c_int32
    h.coli_metal_add.argtypes = [C.c_void_p, C.c_void_p, C.c_int32]
    h.coli_metal_silu_mul.restype = C.c_int32
    h.coli_metal_silu_mul.argtypes = [C.c_void_p, C.c_void_p, C.c_int32]
    return h


@pytest.mark.parametrize("n,nrows", [(4096, 1), (2048, 7), (33, 3), (14336, 2)])
def test_coli_metal_rmsnorm(gpu, n, nrows):
    h = _lib()
    rng = np.random.default_rng(n + nrows)
    x = (rng.standard_normal((nrows, n)) * 2).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    want = oracle.rmsnorm(x, w, 1e-5)
    assert h.coli_metal_rmsnorm(x.ctypes.data, w.ctypes.data, n, nrows, 1e-5) == 1
    assert np.abs(x - want).max() <= 2e-6 * np.abs(want).max()


@pytest.mark.parametrize("n", [1, 7, 4096, 100003])
def test_coli_metal_add_and_silu_mul(gpu, n):
    h = _lib()
    rng = np.random.default_rng(n)
    y = rng.standard_normal(n).astype(np.float32)
    a = rng.standard_normal(n).astype(np.float32)
    want = oracle.add(y, a)
    assert h.coli_metal_add(y.ctypes.data, a.ctypes.data, n) == 1
    np.testing.assert_array_equal(y, want)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    want = oracle.silu_mul(g, u)
    assert h.coli_metal_silu_mul(g.ctypes.data, u.ctypes.data, n) == 1
    assert np.abs(g - want).max() <= 1e-6 * max(1.0, np.abs(want).max())


def test_host_ops_decline_bad_arguments(gpu):
    h = _lib()
    x = np.ones(8, np.float32)
    assert h.coli_metal_rmsnorm(None, x.ctypes.data, 8, 1, 1e-5) == 0
    assert h.coli_metal_rmsnorm(x.ctypes.data, x.ctypes.data, 0, 1, 1e-5) == 0
    assert h.coli_metal_add(x.ctypes.data, None, 8) == 0
    assert h.coli_metal_silu_mul(x.ctypes.data, x.ctypes.data, -1) == 0
    np.testing.assert_array_equal(x, np.ones(8, np.float32))
