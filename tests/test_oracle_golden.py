"""The oracle and the engine's lane code against the reference's own
outputs.

tests/golden/scene<n>.npz hold B3World bytes written by the reference's CPU
path (compiled from its sources by oracle/Makefile; see make_golden.py):
the initial worlds of each scene and their states after 1, 10 and ~60
vector steps of the scene's workload (masks, restores, inputs).  Every
check here is bit-exact on the words b3_step defines.
"""
import os

import numpy as np
import pytest

from b3test import GOLDEN_DIR, EmuBatch, clone, diff_words, oracle_run, ref_lib
from puffysics_amd import scenes
from puffysics_amd.b3types import world_dtype

SCENE_IDS = [1, 2, 3, 4, 5]


def golden(scene):
    z = np.load(os.path.join(GOLDEN_DIR, "scene%d.npz" % scene))
    sig = int(z["signature"][0])
    assert sig == scenes.SCENES[scene].sig
    dt = world_dtype(sig)
    states = {k: np.frombuffer(z[k].tobytes(), dtype=dt).copy() for k in z.files if k.startswith(("initial", "step"))}
    return states, [int(c) for c in z["checkpoints"]]


@pytest.mark.parametrize("scene", SCENE_IDS)
def test_builders_match_reference_worlds(scene):
    states, _ = golden(scene)
    init = states["initial"]
    mine = scenes.build(scene, len(init))
    assert len(diff_words(mine, init, scenes.SCENES[scene].sig)) == 0


@pytest.mark.parametrize("scene", SCENE_IDS)
def test_oracle_matches_reference_outputs(scene):
    states, checkpoints = golden(scene)
    init = states["initial"]
    worlds = clone(init)
    t = 0
    for cp in checkpoints:
        oracle_run(scene, worlds, clone(init), t, cp - t)
        t = cp
        bad = diff_words(worlds, states["step%d" % cp], scenes.SCENES[scene].sig)
        assert len(bad) == 0, "step %d: %s" % (cp, bad[:8].tolist())


@pytest.mark.parametrize("scene", SCENE_IDS)
def test_lane_code_matches_reference_outputs(scene):
    states, checkpoints = golden(scene)
    init = states["initial"]
    emu = EmuBatch(scene, init)
    t = 0
    for cp in checkpoints:
        emu.run(t, cp - t)
        t = cp
        bad = diff_words(emu.worlds(), states["step%d" % cp], scenes.SCENES[scene].sig)
        assert len(bad) == 0, "step %d: %s" % (cp, bad[:8].tolist())


def test_fixtures_exercise_resets_and_contacts():
    """The fixtures are not trivial: the arm scene resets worlds within
    the recorded window and every contact scene has live contacts."""
    states, cps = golden(5)
    resets = sum(int(scenes.masks(5, len(states["initial"]), t)[0].sum()) for t in range(cps[-1]))
    assert resets > 0
    for scene in (1, 2, 4, 5):
        states, cps = golden(scene)
        total = sum(int(states["step%d" % c]["contact_count"].sum()) for c in cps)
        assert total > 0, scene


@pytest.mark.skipif(ref_lib(1) is None, reason="reference CPU path not built here (no reference tree)")
@pytest.mark.parametrize("scene", SCENE_IDS)
def test_oracle_matches_reference_build_longer(scene):
    """Where the reference itself is built (oracle/_ref), compare the oracle
    with it over a longer run and more worlds than the fixtures hold."""
    ref = ref_lib(scene)
    sc = scenes.SCENES[scene]
    count, steps = (24, 200) if scene != 4 else (8, 120)
    a = scenes.build(scene, count)
    b = clone(a)
    init = clone(a)
    ref.ref_run(scene, a.ctypes.data, init.ctypes.data, count, scenes.SEED, 0, steps, sc.dt, sc.substeps, 4, None)
    oracle_run(scene, b, clone(init), 0, steps, threads=4)
    assert len(diff_words(a, b, sc.sig)) == 0


@pytest.mark.skipif(ref_lib(4) is None, reason="reference CPU path not built here (no reference tree)")
def test_reference_capsule_box_nan_is_reproduced():
    """The reference's own step gives world 745 of the bin scene a contact
    (capsule shape 15 against box shape 31) with a NaN normal at step 22,
    and the oracle does the same: a NaN in the compared state is the
    reference's result, which is why word comparisons treat NaN as equal to
    NaN whatever its sign and payload."""
    sc = scenes.SCENES[4]
    count = 768
    a = scenes.build(4, count)
    init = clone(a)
    b = clone(a)
    ref = ref_lib(4)
    ref.ref_run(4, a.ctypes.data, init.ctypes.data, count, scenes.SEED, 0, 23, sc.dt, sc.substeps, 4, None)
    oracle_run(4, b, clone(init), 0, 23, threads=4)
    for w in (a, b):
        ct = w["contacts"][745, 12]
        assert (int(ct["shape_a"]), int(ct["shape_b"])) == (15, 31)
        assert np.isnan(ct["normal"]["x"]) and np.isnan(ct["normal"]["y"])
    assert len(diff_words(a, b, sc.sig)) == 0


@pytest.mark.parametrize("scene", SCENE_IDS)
def test_fast_reference_builds_match_the_reference(scene):
    """The -O3 x86-64-v3 / v4 builds of the reference's CPU path that time
    the CPU baseline step to the -O2 build's bits (every level this host
    can run), over 40 steps of the scene's workload."""
    from b3test import fast_levels_supported, ref_fast_lib
    base = ref_lib(scene)
    if base is None:
        pytest.skip("reference build absent")
    sc = scenes.SCENES[scene]
    count = 48
    ws = base.ref_world_size()
    want = np.zeros(count * ws, np.uint8)
    base.ref_build_batch(scene, want.ctypes.data, count, scenes.SEED, 0)
    initial = want.copy()
    base.ref_run(scene, want.ctypes.data, initial.ctypes.data, count, scenes.SEED, 0, 40, sc.dt, sc.substeps, 1, None)
    levels = fast_levels_supported()
    assert levels, "this host runs neither x86-64-v3 nor v4"
    for level, _ in levels:
        lib = ref_fast_lib(scene, level)
        assert lib is not None, level
        got = initial.copy()
        lib.ref_run(scene, got.ctypes.data, initial.ctypes.data, count, scenes.SEED, 0, 40, sc.dt, sc.substeps, 2,
                    None)
        dt = world_dtype(sc.sig)
        assert len(diff_words(got.view(dt), want.view(dt), sc.sig)) == 0, level
