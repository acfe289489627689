"""The engine's atan2f (fd_atan2f in puffysics_amd/csrc/b3d_math.h) against
the host C library's, which the reference's twist calls
(src/puffysics/03_math.inl:305-306).

The engine's copy is the host build of the same header (tests/emu).  Its
single-argument core must agree with libm's atanf on every one of the 2^32
floats; the two-argument form on pairs from the twist's domain (x = |q.s|
in [0, 1], y in [-1, 1]), on arbitrary bit patterns, and on IEEE edge
values.  The device build is held to the same bits in test_gpu_atan2.py.
"""
import ctypes as C
import os

import numpy as np

from b3test import emu

THREADS = min(8, os.cpu_count() or 1)


def _mismatches(mode, lo, hi, seed=1):
    e = emu()
    e.emu_atan_mismatches.restype = C.c_ulonglong
    e.emu_atan_mismatches.argtypes = [C.c_int, C.c_ulonglong, C.c_ulonglong, C.c_ulonglong, C.c_int]
    return e.emu_atan_mismatches(mode, lo, hi, seed, THREADS)


def test_atanf_core_equals_libm_on_every_float():
    assert _mismatches(0, 0, 1 << 32) == 0


def test_atan2f_equals_libm_on_the_twist_domain():
    assert _mismatches(1, 0, 200_000_000, seed=7) == 0


def test_atan2f_equals_libm_on_arbitrary_bit_patterns():
    assert _mismatches(2, 0, 50_000_000, seed=11) == 0


def edge_pairs():
    v = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 1e-38, 3e38, -3e38,
                  0.5, 2.0, 0.4375, 0.6875, 1.1875, 2.4375, 2 ** -29, 2 ** -26, 2 ** 25, 2 ** 26, 2 ** 60,
                  2 ** -60, 2 ** 61, 2 ** -61, np.nextafter(np.float32(1), np.float32(0))], np.float32)
    y, x = np.meshgrid(v, v, indexing="ij")
    return np.ascontiguousarray(y.ravel()), np.ascontiguousarray(x.ravel())


def _call(fn, y, x):
    out = np.empty_like(y)
    fn.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_long]
    fn(y.ctypes.data, x.ctypes.data, out.ctypes.data, len(y))
    return out


def test_atan2f_equals_libm_on_edge_values():
    y, x = edge_pairs()
    want = _call(emu().emu_libm_atan2f, y, x)
    got = _call(emu().emu_fd_atan2f, y, x)
    same = (want.view(np.uint32) == got.view(np.uint32)) | (np.isnan(want) & np.isnan(got))
    assert same.all(), list(zip(y[~same][:5], x[~same][:5]))


def test_atan2f_is_close_to_the_true_angle():
    """Independent of any libm: within 2 ulp of the float64 angle, and with
    the quadrant and the signed zeros IEEE 754 fixes."""
    rng = np.random.default_rng(3)
    y = rng.uniform(-1, 1, 1 << 20).astype(np.float32)
    x = rng.uniform(-1, 1, 1 << 20).astype(np.float32)
    got = _call(emu().emu_fd_atan2f, y, x)
    true = np.arctan2(y.astype(np.float64), x.astype(np.float64))
    ulp = np.spacing(np.abs(true).astype(np.float32)).astype(np.float64)
    assert (np.abs(got - true) <= 2 * ulp).all()
    got = _call(emu().emu_fd_atan2f, np.array([0.0, -0.0, 0.0, -0.0], np.float32),
                np.array([1.0, 1.0, -1.0, -1.0], np.float32))
    assert got[0] == 0 and not np.signbit(got[0]) and got[1] == 0 and np.signbit(got[1])
    assert got[2] == np.float32(np.pi) and got[3] == -np.float32(np.pi)
