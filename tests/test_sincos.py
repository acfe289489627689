"""The engine's sinf and cosf (or_sinf, or_cosf in
puffysics_amd/csrc/b3d_math.h) against the host C library's, which the
reference's b3_q_axis_angle calls (src/puffysics/03_math.inl:321-326) on
the reduced-coordinate integrator's joint angles.

The engine's copy is the host build of the same header (tests/emu); it must
give the library's bits on every one of the 2^32 floats (NaN payloads
aside).  The device build is held to the same bits in test_gpu_sincos.py.
The method cannot be checked here against anything but the library's
outputs: what fixes its bits is the library's own arithmetic.  The
closed-form checks below pin what the mathematics fixes whatever the
library: exact values, symmetries and the Pythagorean identity."""
import ctypes as C
import math
import os

import numpy as np

from b3test import emu

THREADS = min(8, os.cpu_count() or 1)


def _mismatches(lo, hi):
    e = emu()
    e.emu_sincos_mismatches.restype = None
    e.emu_sincos_mismatches.argtypes = [C.c_ulonglong, C.c_ulonglong, C.c_int, C.c_void_p]
    out = np.zeros(2, np.uint64)
    e.emu_sincos_mismatches(lo, hi, THREADS, out.ctypes.data)
    return int(out[0]), int(out[1])


def test_sinf_cosf_equal_libm_on_every_float():
    assert _mismatches(0, 1 << 32) == (0, 0)


def _engine_sincos(x):
    """The engine's or_sinf and or_cosf (host build) over an array."""
    s = np.empty_like(x)
    c = np.empty_like(x)
    fn = emu().emu_or_sincosf
    fn.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_long]
    fn(x.ctypes.data, s.ctypes.data, c.ctypes.data, len(x))
    return s, c


def test_what_the_mathematics_fixes():
    x = np.array([0.0, -0.0, 1e-30, math.pi / 6, 1.0, 2.0, 100.0, 1e6, 3e38], np.float32)
    s, c = _engine_sincos(x)
    assert s[0] == 0.0 and not np.signbit(s[0]) and np.signbit(s[1]) and c[0] == 1.0 and c[1] == 1.0
    assert s[2] == x[2]                                         # sin x = x below 2^-12
    ref = np.array([math.sin(float(v)) for v in x]), np.array([math.cos(float(v)) for v in x])
    ulp = np.spacing(np.abs(ref[0]).astype(np.float32)).astype(np.float64)
    assert (np.abs(s - ref[0]) <= ulp).all()                    # within an ulp of the float64 value
    ulp = np.spacing(np.abs(ref[1]).astype(np.float32)).astype(np.float64)
    assert (np.abs(c - ref[1]) <= ulp).all()
    rng = np.random.default_rng(3)
    y = rng.uniform(-50, 50, 100000).astype(np.float32)
    sp, cp = _engine_sincos(y)
    sn, cn = _engine_sincos(-y)
    assert (sn == -sp).all() and (cn == cp).all()               # odd and even
    assert np.abs(sp.astype(np.float64) ** 2 + cp.astype(np.float64) ** 2 - 1).max() < 3e-7


def test_two_over_pi_table_is_two_over_pi():
    """The Payne-Hanek reduction's table (two_over_pi_window in b3d_math.h)
    against 2/pi computed here from Machin's formula: window i >= 3 holds
    bits 8 (i - 3) .. 8 (i - 3) + 31 of 2/pi's binary fraction, windows 0-2
    its first 8, 16 and 24 bits."""
    import re
    from b3test import ROOT

    def arctan_inv(x, bits):                    # arctan(1/x) * 2^bits
        one = 1 << (bits + 20)
        total, term, k, sign = 0, one // x, 1, 1
        while term:
            total += sign * (term // k)
            term //= x * x
            k += 2
            sign = -sign
        return total >> 20

    bits = 1200
    pi = 4 * (4 * arctan_inv(5, bits) - arctan_inv(239, bits))
    frac = bin((2 << (2 * bits)) // pi)[2:].zfill(bits)
    want = [int(frac[:8], 2), int(frac[:16], 2), int(frac[:24], 2)] + [int(frac[8 * i:8 * i + 32], 2)
                                                                      for i in range(21)]
    src = open(os.path.join(ROOT, "puffysics_amd", "csrc", "b3d_math.h")).read()
    body = src[src.index("two_over_pi_window"):]
    body = body[body.index("{", body.index("w[24]")) + 1:body.index("};")]
    got = [int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", body)]
    assert got == want
    assert float.fromhex("0x1.45f306dc9c883p-1") == 2 / math.pi      # hpi_inv / 2^24
    assert float.fromhex("0x1.921fb54442d18p+0") == math.pi / 2
