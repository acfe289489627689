"""The device build of the engine's sinf and cosf (or_sinf, or_cosf, used by
the reduced-coordinate integrator's b3_q_axis_angle) against the host C
library's, which the reference's CPU path calls
(src/puffysics/03_math.inl:321-326).  The device evaluates them through
tests/emu/libb3devcheck.so, a kernel around the same header the step
kernels include; the host values come from libm on this machine."""
import ctypes as C
import os

import numpy as np
import pytest

from b3test import ROOT, emu

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEVCHECK = os.path.join(ROOT, "tests", "emu", "libb3devcheck.so")


def _device(x):
    lib = C.CDLL(DEVCHECK)
    lib.devcheck_sincosf.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_long, C.c_void_p]
    xd = torch.from_numpy(x).cuda()
    s, c = torch.empty_like(xd), torch.empty_like(xd)
    rc = lib.devcheck_sincosf(xd.data_ptr(), s.data_ptr(), c.data_ptr(), len(x),
                              torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    return s.cpu().numpy(), c.cpu().numpy()


def _host(x):
    s, c = np.empty_like(x), np.empty_like(x)
    fn = emu().emu_libm_sincosf
    fn.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_long]
    fn(x.ctypes.data, s.ctypes.data, c.ctypes.data, len(x))
    return s, c


def _same(a, b):
    return (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))


def test_device_sincosf_equals_host_libm_below_120():
    """2^25 floats of each sign below 120 in magnitude (the direct and
    Cody-Waite paths, which every joint angle takes), uniform in their bit
    patterns, and every float in [0.5, 0.5 + 2^-4) and [3, 3 + 2^-6)."""
    rng = np.random.default_rng(7)
    n = 1 << 25
    bits = rng.integers(0, 0x42f00000, n, dtype=np.uint32) | (rng.integers(0, 2, n, dtype=np.uint32) << 31)
    dense = np.concatenate([np.arange(0x3f000000, 0x3f080000, dtype=np.uint32),
                            np.arange(0x40400000, 0x40402000 + 0x20000, dtype=np.uint32)])
    x = np.concatenate([bits, dense]).view(np.float32)
    ds, dc = _device(x)
    hs, hc = _host(x)
    for d, h, name in ((ds, hs, "sin"), (dc, hc, "cos")):
        ok = _same(d, h)
        assert ok.all(), "%s: %d differ, e.g. x=%r" % (name, (~ok).sum(), x[~ok][:3])


def test_device_sincosf_equals_host_libm_on_large_and_arbitrary_floats():
    """The Payne-Hanek path (|x| >= 120) and arbitrary bit patterns."""
    rng = np.random.default_rng(13)
    big = rng.integers(0x42f00000, 0x7f800000, 1 << 24, dtype=np.uint32)
    big |= rng.integers(0, 2, 1 << 24, dtype=np.uint32) << 31
    anyb = rng.integers(0, 1 << 32, 1 << 24, dtype=np.uint64).astype(np.uint32)
    edge = np.array([0x42f00000, 0x42efffff, 0x3f490fdb, 0x3f490fda, 0x39800000, 0x397fffff, 0x7f7fffff, 0x00000001,
                     0x7f800000, 0xff800000, 0x7fc00000], np.uint32)
    x = np.concatenate([big, anyb, edge, edge | 0x80000000]).view(np.float32)
    ds, dc = _device(x)
    hs, hc = _host(x)
    assert _same(ds, hs).all() and _same(dc, hc).all()
