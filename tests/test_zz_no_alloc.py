"""b3_batch_step_worlds_gpu, the step without allocation, against
b3_batch_step_gpu (the engine's step) on the same worlds.

The new entry point steps caller-owned device B3World structs in place with
its scratch in a fixed device array of the library.  Its results must equal
the engine's word for word; it must leave unselected worlds, corrupt worlds
and the bytes around each world (an Env struct's other fields) untouched,
and refuse a batch beyond its array without launching.  Two calls in a row,
the second on a smaller batch of another signature, share the array.
"""
import numpy as np
import pytest

from b3test import clone, diff_words, oracle_run
from puffysics_amd import _native, scenes
from puffysics_amd.b3types import B3Batch

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

HIP_ERROR_OUT_OF_MEMORY = 2
FILL = 0xA5


def _lib():
    return _native.engine_lib()


def _to_device(worlds, stride, offset):
    """Worlds embedded at `offset` in `stride`-byte records (the rest FILL)."""
    wb = worlds.dtype.itemsize
    host = np.full((len(worlds), stride), FILL, np.uint8)
    host[:, offset:offset + wb] = worlds.view(np.uint8).reshape(len(worlds), wb)
    return torch.from_numpy(host.ravel()).cuda()


def _from_device(dev, dtype, count, stride, offset):
    host = dev.cpu().numpy().reshape(count, stride)
    wb = dtype.itemsize
    worlds = np.ascontiguousarray(host[:, offset:offset + wb]).reshape(-1).view(dtype)
    return worlds, host


def _engine_steps(worlds, sig, dt, substeps, active, steps):
    from puffysics_amd.engine import B3Engine
    eng = B3Engine(worlds, sig)
    act = None if active is None else torch.from_numpy(active).cuda()
    for _ in range(steps):
        eng.step(dt, substeps, act)
    torch.cuda.synchronize()
    out = eng.download()
    eng.close()
    return out


def _warm_worlds(scene, count, steps=10):
    worlds = scenes.build(scene, count)
    oracle_run(scene, worlds, clone(worlds), 0, steps, threads=8)
    return worlds


@pytest.mark.parametrize("order", [0, 1])
def test_no_alloc_step_equals_engine_step(order):
    """Call 1: 300 arm worlds inside 37,336-byte records at offset 32, with
    a step mask, stepped 3 times.  Call 2: 70 box-stack worlds packed, every
    world, twice.  Each equals the engine's step on the same worlds; the
    record padding and the unselected worlds keep their bytes."""
    lib = _lib()
    stream = torch.cuda.current_stream().cuda_stream
    cases = [(5, 300, 64, 32, 3), (2, 70, 0, 0, 2)]
    if order:
        cases = cases[::-1]
    for scene, count, pad, offset, steps in cases:
        sc = scenes.SCENES[scene]
        worlds = _warm_worlds(scene, count)
        wb = worlds.dtype.itemsize
        stride = wb + pad
        active = None
        if scene == 5:
            active = (np.arange(count) % 7 != 3).astype(np.uint8)
        dev = _to_device(worlds, stride, offset)
        act = None if active is None else torch.from_numpy(active).cuda()
        batch = B3Batch(dev.data_ptr(), stride, offset, count)
        for _ in range(steps):
            rc = lib.b3_batch_step_worlds_gpu(batch, sc.sig, sc.dt, sc.substeps,
                                              None if act is None else act.data_ptr(), stream)
            assert rc == 0
        torch.cuda.synchronize()
        got, raw = _from_device(dev, worlds.dtype, count, stride, offset)
        want = _engine_steps(worlds, sc.sig, sc.dt, sc.substeps, active, steps)
        bad = diff_words(got, want, sc.sig)
        assert len(bad) == 0, "scene %d: %d differing words, first %s" % (scene, len(bad), bad[:4].tolist())
        assert (raw[:, :offset] == FILL).all() and (raw[:, offset + wb:] == FILL).all()
        if active is not None:
            # raw words (indexing a structured array does not copy its padding)
            idle = active == 0
            before = worlds.view(np.uint32).reshape(count, -1)
            after = got.view(np.uint32).reshape(count, -1)
            assert (after[idle] == before[idle]).all()
        assert (got["contact_count"] > 0).any()


def test_no_alloc_step_skips_corrupt_worlds():
    """A world whose shape names a body past its body count is left exactly
    as it is; the others step as the engine steps them."""
    lib = _lib()
    scene, count = 4, 100
    sc = scenes.SCENES[scene]
    worlds = _warm_worlds(scene, count, 5)
    bad_worlds = clone(worlds)
    bad_worlds["shapes"]["body"][7, 2] = 99
    dev = _to_device(bad_worlds, worlds.dtype.itemsize, 0)
    rc = lib.b3_batch_step_worlds_gpu(B3Batch(dev.data_ptr(), worlds.dtype.itemsize, 0, count), sc.sig, sc.dt,
                                      sc.substeps, None, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    got, _ = _from_device(dev, worlds.dtype, count, worlds.dtype.itemsize, 0)
    assert (got.view(np.uint32).reshape(count, -1)[7] == bad_worlds.view(np.uint32).reshape(count, -1)[7]).all()
    active = np.ones(count, np.uint8)
    active[7] = 0
    want = _engine_steps(worlds, sc.sig, sc.dt, sc.substeps, active, 1)
    keep = np.arange(count) != 7
    assert len(diff_words(got[keep], want[keep], sc.sig)) == 0


def test_no_alloc_step_refuses_a_batch_beyond_its_array():
    """4,000 arm worlds need more than the 256 MiB array: refused with
    hipErrorOutOfMemory, nothing launched, the worlds untouched.  Invalid
    arguments are refused before any launch as well."""
    lib = _lib()
    sc = scenes.SCENES[5]
    wb = 37272
    dev = torch.full((4000 * wb,), 7, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.b3_batch_step_worlds_gpu(B3Batch(dev.data_ptr(), wb, 0, 4000), sc.sig, sc.dt, sc.substeps, None,
                                      stream)
    assert rc == HIP_ERROR_OUT_OF_MEMORY
    assert lib.b3_batch_step_worlds_gpu(B3Batch(dev.data_ptr(), wb - 4, 0, 10), sc.sig, sc.dt, sc.substeps,
                                        None, stream) != 0
    assert lib.b3_batch_step_worlds_gpu(B3Batch(dev.data_ptr() + 2, wb, 0, 10), sc.sig, sc.dt, sc.substeps,
                                        None, stream) != 0
    assert lib.b3_batch_step_worlds_gpu(B3Batch(dev.data_ptr(), wb, 0, 10), sc.sig, float("nan"), sc.substeps,
                                        None, stream) != 0
    assert lib.b3_batch_step_worlds_gpu(B3Batch(None, wb, 0, 0), sc.sig, sc.dt, sc.substeps, None, stream) == 0
    torch.cuda.synchronize()
    assert int((dev != 7).sum()) == 0
