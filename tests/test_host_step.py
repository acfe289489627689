"""The library's CPU step: b3_host_step / b3_host_batch_step, exported by
libb3engine.so and wrapped under the reference's names b3_step and
b3_batch_step by include/b3_setup.h (09_step.inl:262-264,
b3_batch.cuh:39-48).  They run the engine's lane code built for the host
with one world per tile, in place on plain B3World structs, and must equal
the oracle (the reference's CPU path restated) bit for bit, prepared contact
fields included.  Everything goes through the C ABI; no GPU is needed.
"""
import os
import subprocess

import numpy as np
import pytest

from b3test import ROOT, clone, diff_words, oracle_run, oracle_step_batch
from puffysics_amd import _native, scenes
from puffysics_amd.b3types import B3Batch, batch_of, world_dtype


def _lib():
    return _native.engine_lib()


def host_run(scene, worlds, initial, t0, nsteps):
    """The scene workload on the host: masks, b3_batch_restore, inputs,
    b3_batch_step over the masked batch."""
    sc = scenes.SCENES[scene]
    for t in range(t0, t0 + nsteps):
        reset, stepm = scenes.masks(scene, len(worlds), t)
        r = reset.astype(bool)
        worlds[r] = initial[r]
        scenes.apply_inputs(scene, worlds, t, stepm)
        assert _lib().b3_host_batch_step(batch_of(worlds), sc.sig, sc.dt, sc.substeps, stepm.ctypes.data) == 1


@pytest.mark.parametrize("scene,count,steps", [(1, 64, 60), (2, 32, 60), (3, 24, 40), (4, 12, 25), (5, 48, 40)])
def test_host_batch_step_matches_oracle(scene, count, steps):
    worlds = scenes.build(scene, count)
    initial = clone(worlds)
    ref = clone(worlds)
    host_run(scene, worlds, initial, 0, steps)
    oracle_run(scene, ref, initial, 0, steps)
    bad = diff_words(worlds, ref, scenes.SCENES[scene].sig)
    assert len(bad) == 0, "%d differing words, first %s" % (len(bad), bad[:4].tolist())
    if scene != 3:
        assert ref["contact_count"].sum() > 0


def test_host_step_feature_worlds():
    """Welds, spring / motor / limit / fixed hinges, kinematic bodies,
    restitution, rolling, locks, filters and contact overflow, with a step
    mask on every third step, through b3_host_batch_step; and one world
    through b3_host_step."""
    from b3test import feature_worlds
    from puffysics_amd.creation import CUSTOM_SIG
    worlds = feature_worlds(40)
    ref = clone(worlds)
    active = (np.arange(40) % 5 != 2).astype(np.uint8)
    for t in range(40):
        act = active if t % 3 == 0 else None
        oracle_step_batch(ref, CUSTOM_SIG, 1.0 / 60.0, 4, act)
        assert _lib().b3_host_batch_step(batch_of(worlds), CUSTOM_SIG, 1.0 / 60.0, 4,
                                         None if act is None else act.ctypes.data) == 1
    bad = diff_words(worlds, ref, CUSTOM_SIG)
    assert len(bad) == 0, bad[:10].tolist()
    one = clone(worlds[3:4])
    want = clone(one)
    _lib().b3_host_step(one.ctypes.data, CUSTOM_SIG, 1.0 / 60.0, 4)
    oracle_step_batch(want, CUSTOM_SIG, 1.0 / 60.0, 4)
    assert len(diff_words(one, want, CUSTOM_SIG)) == 0
    assert (ref["contacts_dropped"] > 0).any() and np.abs(ref["joints"]["motor_impulse"]).max() > 0


def test_host_batch_step_strided_and_invalid_arguments():
    """Worlds embedded in larger records (stride, world_offset) step in place
    with the rest of each record untouched; invalid batches, dt, substeps or
    a corrupt selected world return 0 and change nothing; dt == 0 and empty
    batches return 1."""
    scene, count = 5, 10
    sc = scenes.SCENES[scene]
    worlds = scenes.build(scene, count)
    wb = worlds.dtype.itemsize
    stride, offset = wb + 16, 8
    buf = np.full((count, stride), 0x5A, np.uint8)
    buf[:, offset:offset + wb] = worlds.view(np.uint8).reshape(count, wb)
    lib = _lib()
    batch = B3Batch(buf.ctypes.data, stride, offset, count)
    assert lib.b3_host_batch_step(batch, sc.sig, sc.dt, sc.substeps, None) == 1
    got = np.ascontiguousarray(buf[:, offset:offset + wb]).reshape(-1).view(worlds.dtype)
    ref = clone(worlds)
    oracle_step_batch(ref, sc.sig, sc.dt, sc.substeps)
    assert len(diff_words(got, ref, sc.sig)) == 0
    assert (buf[:, :offset] == 0x5A).all() and (buf[:, offset + wb:] == 0x5A).all()
    before = buf.copy()
    for b, dt, subs in ((B3Batch(buf.ctypes.data, wb - 4, 0, count), sc.dt, sc.substeps),
                        (B3Batch(None, stride, 0, count), sc.dt, sc.substeps),
                        (B3Batch(buf.ctypes.data, stride, offset, -1), sc.dt, sc.substeps),
                        (batch, float("nan"), sc.substeps), (batch, -1.0, sc.substeps), (batch, sc.dt, 0)):
        assert lib.b3_host_batch_step(b, sc.sig, dt, subs, None) == 0
    assert lib.b3_host_batch_step(batch, sc.sig + 1, sc.dt, sc.substeps, None) == 0
    assert lib.b3_host_batch_step(batch, sc.sig, 0.0, sc.substeps, None) == 1
    assert lib.b3_host_batch_step(B3Batch(None, stride, 0, 0), sc.sig, sc.dt, sc.substeps, None) == 1
    # a corrupt world in the batch: nothing steps
    bad = buf.copy()
    bw = bad[:, offset:offset + wb].copy().reshape(-1).view(worlds.dtype)
    bw["shapes"]["body"][6, 3] = 77
    bad[:, offset:offset + wb] = bw.view(np.uint8).reshape(count, wb)
    snap = bad.copy()
    assert lib.b3_host_batch_step(B3Batch(bad.ctypes.data, stride, offset, count), sc.sig, sc.dt, sc.substeps,
                                  None) == 0
    assert (bad == snap).all()
    active = np.ones(count, np.uint8)
    active[6] = 0                                   # ... unless it is not selected
    assert lib.b3_host_batch_step(B3Batch(bad.ctypes.data, stride, offset, count), sc.sig, sc.dt, sc.substeps,
                                  active.ctypes.data) == 1
    assert (buf == before).all()


def test_c99_program_links_and_steps():
    """A C99 program including b3_engine.h and b3_setup.h, built with gcc
    -std=c99 and linked with -lb3engine, builds a hinged scene with the
    creation API and steps it with b3_step and b3_batch_step; its worlds
    equal the oracle's."""
    from puffysics_amd.creation import CUSTOM_SIG
    out_dir = os.path.join(ROOT, "tests", "c99", "_build")
    os.makedirs(out_dir, exist_ok=True)
    exe = os.path.join(out_dir, "b3_c99_step")
    lib_dir = os.path.join(ROOT, "puffysics_amd")
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-O2", "-D__HIP_PLATFORM_AMD__",
                    "-I" + os.path.join(ROOT, "include"), "-isystem", "/opt/rocm/include",
                    os.path.join(ROOT, "tests", "c99", "b3_c99_step.c"), "-o", exe, "-L" + lib_dir, "-lb3engine",
                    "-lm", "-Wl,-rpath," + lib_dir], check=True)
    data = os.path.join(out_dir, "worlds.bin")
    run = subprocess.run([exe, data], check=True, capture_output=True, text=True)
    assert ("signature %x" % CUSTOM_SIG) in run.stdout
    dt = world_dtype(CUSTOM_SIG)
    w = np.fromfile(data, dtype=np.uint8).view(dt)
    assert len(w) == 4
    initial = w[0:1]
    single = clone(initial)
    for t in range(90):
        single["bodies"]["torque"]["z"][0, 1] += np.float32(2.0 if t % 20 < 10 else -2.0)
        oracle_step_batch(single, CUSTOM_SIG, 1.0 / 60.0, 4)
    pair = clone(np.concatenate([initial, initial]))
    active = np.array([1, 0], np.uint8)
    for t in range(45):
        oracle_step_batch(pair, CUSTOM_SIG, 1.0 / 60.0, 4, None if t % 3 else active)
    assert len(diff_words(w[1:2], single, CUSTOM_SIG)) == 0
    assert len(diff_words(w[2:4], pair, CUSTOM_SIG)) == 0
    assert single["contact_count"][0] > 0 and np.abs(single["joints"]["motor_impulse"][0, 0]) > 0
