"""The C ABI: every declared entry point is exported, and argument
validation rejects bad input before touching a device (so these run on a
machine without a GPU)."""
import ctypes as C
import os
import re

import numpy as np

from puffysics_amd import _native, scenes
from puffysics_amd.b3types import B3Batch, batch_of

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIP_ERROR_INVALID_VALUE = 1


def declared(header):
    """Names of the functions a header declares at file scope."""
    text = open(os.path.join(ROOT, "include", header)).read()
    return set(re.findall(r"^(?:hipError_t|int|void) (\w+)\(", text, re.M))


def test_every_declared_symbol_is_exported():
    lib = _native.engine_lib()
    names = declared("b3_engine.h") | declared("b3_workload.h")
    assert len(names) >= 13
    for n in names:
        assert hasattr(lib, n), n
    assert names == {n for n, _, _ in _native.ENGINE_SYMBOLS}


def test_invalid_create_arguments():
    lib = _native.engine_lib()
    h = C.c_void_p()
    sig = scenes.SCENES[1].sig
    worlds = scenes.build(1, 4)
    good = batch_of(worlds)
    cases = [
        B3Batch(None, good.stride, 0, 4),                      # NULL data with count > 0
        B3Batch(good.data, good.stride - 8, 0, 4),             # stride < sizeof(B3World)
        B3Batch(good.data, good.stride + 16, 32, 4),           # offset past the slack
        B3Batch(good.data, good.stride, 0, -1),                # negative count
    ]
    for b in cases:
        assert lib.b3_engine_create(C.byref(h), b, sig) == HIP_ERROR_INVALID_VALUE
        assert not h.value
    assert lib.b3_engine_create(C.byref(h), good, 0) == HIP_ERROR_INVALID_VALUE  # bad signature
    assert lib.b3_engine_create(None, good, sig) == HIP_ERROR_INVALID_VALUE
    # a body index out of range is rejected before any allocation
    bad = worlds.copy()
    bad["shapes"][2]["body"][1] = 7
    assert lib.b3_engine_create(C.byref(h), batch_of(bad), sig) == HIP_ERROR_INVALID_VALUE
    bad = worlds.copy()
    bad["contact_count"][0] = 5  # above the capacity of 4
    assert lib.b3_engine_create(C.byref(h), batch_of(bad), sig) == HIP_ERROR_INVALID_VALUE


def test_null_engine_is_rejected():
    lib = _native.engine_lib()
    assert lib.b3_batch_step_gpu(None, 1.0 / 60, 4, None, None, None) == HIP_ERROR_INVALID_VALUE
    assert lib.b3_batch_restore_gpu(None, None, None) == HIP_ERROR_INVALID_VALUE
    assert lib.b3_batch_apply_gpu(None, None, None, None, None, None) == HIP_ERROR_INVALID_VALUE
    assert lib.b3_engine_count(None) == -1
    assert lib.b3_engine_destroy(None) == 0
    assert lib.b3w_masks_gpu(9, 1, 0, 4, None, None, None) == HIP_ERROR_INVALID_VALUE
    assert lib.b3w_inputs_gpu(None, 1, 1, 0, None, None) == HIP_ERROR_INVALID_VALUE


def test_scene_worlds_have_reference_layout():
    for n, sc in scenes.SCENES.items():
        w = scenes.build(n, 2)
        assert w.dtype.itemsize == {1: 3472, 2: 9880, 3: 21488, 4: 71320, 5: 37272}[n]
        assert (w["body_count"] > 0).all()
        assert np.isfinite(w["bodies"]["position"]["y"]).all()
