"""The device build of the engine's atan2f (fd_atan2f, used by the hinge
twist) against the host C library's atan2f, which the reference's CPU path
calls (src/puffysics/03_math.inl:305-306).  The device evaluates it through
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


def _device_atan2f(y, x):
    lib = C.CDLL(DEVCHECK)
    lib.devcheck_atan2f.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_long, C.c_void_p]
    yd = torch.from_numpy(y).cuda()
    xd = torch.from_numpy(x).cuda()
    out = torch.empty_like(yd)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.devcheck_atan2f(yd.data_ptr(), xd.data_ptr(), out.data_ptr(), len(y), stream)
    assert rc == 0
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _host_atan2f(y, x):
    out = np.empty_like(y)
    fn = emu().emu_libm_atan2f
    fn.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_long]
    fn(y.ctypes.data, x.ctypes.data, out.ctypes.data, len(y))
    return out


def _same(a, b):
    return (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))


def test_device_atan2f_equals_host_libm_on_the_twist_domain():
    rng = np.random.default_rng(5)
    n = 1 << 25
    x = rng.integers(0, 0x3f800001, n, dtype=np.uint32).view(np.float32)
    y = (rng.integers(0, 0x3f800001, n, dtype=np.uint32) | (rng.integers(0, 2, n, dtype=np.uint32) << 31))
    y = y.view(np.float32)
    got, want = _device_atan2f(y, x), _host_atan2f(y, x)
    ok = _same(got, want)
    assert ok.all(), "%d differ, e.g. y=%r x=%r" % ((~ok).sum(), y[~ok][:3], x[~ok][:3])


def test_device_atan2f_equals_host_libm_on_unit_quaternions_and_bit_patterns():
    rng = np.random.default_rng(9)
    q = rng.normal(size=(1 << 23, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    qz, qs = q[:, 2].astype(np.float32), q[:, 3].astype(np.float32)
    y = np.where(qs < 0, -qz, qz).astype(np.float32)
    x = np.where(qs < 0, -qs, qs).astype(np.float32)
    bits = rng.integers(0, 1 << 32, (2, 1 << 23), dtype=np.uint64).astype(np.uint32)
    y = np.concatenate([y, bits[0].view(np.float32)])
    x = np.concatenate([x, bits[1].view(np.float32)])
    v = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 1e-45, 3e38, 0.4375, 2.4375, 2 ** 25, 2 ** -29],
                 np.float32)
    ey, ex = (a.ravel() for a in np.meshgrid(v, v, indexing="ij"))
    y = np.ascontiguousarray(np.concatenate([y, ey]))
    x = np.ascontiguousarray(np.concatenate([x, ex]))
    got, want = _device_atan2f(y, x), _host_atan2f(y, x)
    ok = _same(got, want)
    assert ok.all(), "%d differ, e.g. y=%r x=%r" % ((~ok).sum(), y[~ok][:3], x[~ok][:3])
