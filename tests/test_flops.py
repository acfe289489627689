"""The counting build of the oracle (oracle/liboracle_flops.so), which
produces the per-configuration flop counts of tests/golden/flops.json.

Pins that do not restate the counter:
  - the counting build steps worlds to the oracle's bits exactly (the
    counted arithmetic is the reference's arithmetic);
  - counts add over worlds: n copies of a world cost n times one;
  - a world of free-flying bodies (no contacts, no joints) costs a + b k
    for k bodies and c + d s for s substeps, exactly (the step's work is a
    fixed part plus per-body and per-substep parts);
  - the committed fixture matches a fresh count on a prefix of its run.
"""
import ctypes as C
import json
import os

import numpy as np

from b3test import ROOT, clone, diff_words, oracle_step_batch
from puffysics_amd import scenes

LIB = os.path.join(ROOT, "oracle", "liboracle_flops.so")


def _count(worlds, sig, dt, substeps, active=None):
    lib = C.CDLL(LIB)
    fn = lib.ocount_batch_step
    fn.restype = C.c_longlong
    fn.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_int, C.c_ulonglong, C.c_float, C.c_int, C.c_void_p]
    act = None if active is None else np.ascontiguousarray(active, np.uint8)
    return fn(worlds.ctypes.data, worlds.dtype.itemsize, 0, len(worlds), sig, dt, substeps,
              None if act is None else act.ctypes.data)


def test_counting_build_steps_to_the_oracle_bits():
    for scene, count, steps in ((2, 16, 40), (3, 8, 20), (5, 16, 30)):
        sc = scenes.SCENES[scene]
        a = scenes.build(scene, count)
        b = clone(a)
        for _ in range(steps):
            assert _count(a, sc.sig, sc.dt, sc.substeps) > 0
            oracle_step_batch(b, sc.sig, sc.dt, sc.substeps)
        assert len(diff_words(a, b, sc.sig)) == 0


def test_counts_add_over_worlds():
    sc = scenes.SCENES[5]
    w = scenes.build(5, 1)
    for _ in range(12):
        oracle_step_batch(w, sc.sig, sc.dt, sc.substeps)
    one = _count(clone(w), sc.sig, sc.dt, sc.substeps)
    many = _count(np.concatenate([clone(w)] * 7), sc.sig, sc.dt, sc.substeps)
    assert one > 10000 and many == 7 * one
    # an unselected world costs nothing
    assert _count(np.concatenate([clone(w)] * 3), sc.sig, sc.dt, sc.substeps, np.array([1, 0, 1])) == 2 * one


def _free_world(k):
    """k dynamic spheres far apart in the air, nothing else."""
    from puffysics_amd import creation as cr
    w = cr.new_worlds(1)
    for i in range(k):
        b = cr.body(w, 0, 2, (3.0 * i, 10.0, 0.0))
        cr.sphere(w, 0, b, 0.25)
        cr.finalize_mass(w, 0, b)
    return w, cr.CUSTOM_SIG


def test_free_flight_costs_are_affine():
    counts = []
    for k in (1, 2, 3, 5, 8):
        w, sig = _free_world(k)
        counts.append(_count(w, sig, 1.0 / 60.0, 4))
    k = np.array([1, 2, 3, 5, 8])
    slope = (counts[1] - counts[0])
    assert slope > 0
    assert all(counts[i] == counts[0] + slope * (k[i] - 1) for i in range(len(k))), counts
    subs = []
    for s in (1, 2, 3, 6):
        w, sig = _free_world(3)
        subs.append(_count(w, sig, 1.0 / 60.0, s))
    d = subs[1] - subs[0]
    assert d > 0 and subs[2] == subs[0] + 2 * d and subs[3] == subs[0] + 5 * d, subs


def test_fixture_matches_a_fresh_count():
    with open(os.path.join(ROOT, "tests", "golden", "flops.json")) as f:
        fx = json.load(f)
    for scene in (1, 3, 5):
        entry = fx["scenes"][str(scene)]
        sc = scenes.SCENES[scene]
        count = entry["worlds_sampled"]
        worlds = scenes.build(scene, count)
        initial = clone(worlds)
        for t in range(6):
            reset, stepm = scenes.masks(scene, count, t)
            r = reset.astype(bool)
            worlds[r] = initial[r]
            scenes.apply_inputs(scene, worlds, t, stepm)
            flops = _count(worlds, sc.sig, sc.dt, sc.substeps, stepm)
            assert abs(flops / max(int(stepm.sum()), 1) - entry["flops_per_env_step"][t]) < 0.1
