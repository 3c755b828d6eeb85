"""shs_matmul_device_noalloc (the entry point that allocates nothing) against
shs_matmul_device: bit-identical outputs on two calls in a row, the second smaller, so
the second reads scratch the first filled; and a size past the scratch is refused
before anything runs."""
import ctypes as C

import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu


def _dev(hip, nbytes):
    p = C.c_void_p()
    assert hip.hipMalloc(C.byref(p), C.c_size_t(nbytes)) == 0
    return p


def test_no_alloc_matmul_equals_the_allocating_entry(shs, oracle):
    hip = C.CDLL("libamdhip64.so.7")
    for qt, rows, cols in ((2, 1000, 3072), (7, 300, 9216)):
        w = H.random_blocks(qt, rows, cols, seed=qt)
        m = shs.WeightMatrix(qt, rows, cols, w)
        for T in (300, 37, 3):
            x = np.random.default_rng(T).standard_normal((T, cols)).astype(np.float32)
            xd, ya, yb = _dev(hip, x.nbytes), _dev(hip, T * rows * 4), _dev(hip, T * rows * 4)
            try:
                assert hip.hipMemcpy(xd, x.ctypes.data_as(C.c_void_p), C.c_size_t(x.nbytes), 1) == 0
                m.forward_device(xd.value, T, ya.value)
                m.forward_device_noalloc(xd.value, T, yb.value)
                a = np.empty((T, rows), np.float32)
                b = np.empty((T, rows), np.float32)
                assert hip.hipMemcpy(a.ctypes.data_as(C.c_void_p), ya, C.c_size_t(a.nbytes), 2) == 0
                assert hip.hipMemcpy(b.ctypes.data_as(C.c_void_p), yb, C.c_size_t(b.nbytes), 2) == 0
            finally:
                for p in (xd, ya, yb):
                    hip.hipFree(p)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (qt, T)
            assert np.array_equal(b, oracle.matmul(qt, w, rows, cols, x, T)), (qt, T)


def test_no_alloc_matmul_refuses_a_size_past_its_scratch(shs):
    w = H.random_blocks(2, 64, 3072, seed=1)
    m = shs.WeightMatrix(2, 64, 3072, w)
    with pytest.raises(shs.ArgumentOutOfRangeError, match="scratch"):
        m.forward_device_noalloc(0x1000, 4096, 0x2000)  # refused before any pointer is touched
