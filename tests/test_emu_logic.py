"""The engine's per-lane step code, built for the host, against the oracle.

The lane code (puffysics_amd/csrc/b3d_lane.h, b3d_inputs.h) is what the
gfx950 step kernel runs per world.  Compiled with g++ -ffp-contract=off and
the same libm, it must reproduce the oracle bit for bit: this pins the
word-transposed tile layout, the restore ranges, the merge-pointer warm
start and every index the kernels compute, without a GPU.
"""
import numpy as np
import pytest

from b3test import EmuBatch, clone, diff_words, oracle_run
from puffysics_amd import scenes

CASES = [(1, 70, 40), (2, 70, 65), (3, 70, 25), (4, 66, 12), (5, 130, 40)]


@pytest.mark.parametrize("scene,count,steps", CASES)
def test_lane_code_matches_oracle(scene, count, steps):
    worlds = scenes.build(scene, count)
    initial = clone(worlds)
    emu = EmuBatch(scene, worlds)
    ref = clone(worlds)
    oracle_run(scene, ref, initial, 0, steps)
    emu.run(0, steps)
    got = emu.worlds()
    bad = diff_words(got, ref, scenes.SCENES[scene].sig)
    assert len(bad) == 0, "first differences (world, word): %s" % bad[:10].tolist()
    # the run did something: contacts exist where the scene has any
    if scene != 3:
        assert ref["contact_count"].sum() > 0


def test_lane_code_covers_every_feature():
    """Welds (rigid and soft), spring-only and fixed hinges, kinematic
    bodies, restitution, rolling, locks, damping, filters and contact
    overflow: bit-exact against the oracle over 80 steps."""
    from b3test import EmuSig, feature_worlds, oracle_step_batch
    from puffysics_amd.creation import CUSTOM_SIG
    worlds = feature_worlds(40)
    ref = clone(worlds)
    emu = EmuSig(CUSTOM_SIG, worlds)
    active = (np.arange(40) % 5 != 2).astype(np.uint8)
    for t in range(80):
        act = active if t % 3 == 0 else None
        oracle_step_batch(ref, CUSTOM_SIG, 1.0 / 60.0, 4, act)
        emu.step(1.0 / 60.0, 4, act)
    got = emu.worlds()
    bad = diff_words(got, ref, CUSTOM_SIG)
    assert len(bad) == 0, bad[:10].tolist()
    # the features are really exercised
    assert ref["contact_overflow"][3::4].all() and ref["contacts_dropped"].max() > 0
    assert (ref["contact_count"] > 0).all()
    j = ref["joints"]
    assert (j["fixed_rotation"][:, 2][np.arange(40) % 4 != 3] == 1).all()
    assert np.abs(j["angular_impulse"]["x"][:, 0]).max() > 0           # welds carry load


def test_lane_code_single_joint_worlds():
    """Coverage worlds without hinges hold one weld joint each, so every
    joint sweep solves the same joint twice in a row."""
    from b3test import EmuSig, feature_worlds, oracle_step_batch
    from puffysics_amd.creation import CUSTOM_SIG
    worlds = feature_worlds(24, seed=11, hinges=False)
    assert set(worlds["joint_count"].tolist()) <= {0, 1}
    ref = clone(worlds)
    emu = EmuSig(CUSTOM_SIG, worlds)
    for t in range(40):
        oracle_step_batch(ref, CUSTOM_SIG, 1.0 / 60.0, 4)
        emu.step(1.0 / 60.0, 4)
    bad = diff_words(emu.worlds(), ref, CUSTOM_SIG)
    assert len(bad) == 0, bad[:10].tolist()


@pytest.mark.parametrize("scene,count,steps", [(2, 70, 65), (4, 66, 12), (5, 130, 40)])
def test_lane_code_default_options(scene, count, steps):
    """Default options (prepared solver fields not written back, the warm
    start fused into preparation where no contact has restitution): every
    live word except those solver fields equals the oracle's."""
    from b3test import emu, solver_field_words, live_word_mask, words
    import ctypes as C
    worlds = scenes.build(scene, count)
    initial = clone(worlds)
    lib = emu()
    lib.emu_set_options.argtypes = [C.c_uint]
    lib.emu_set_options(0)
    try:
        e = EmuBatch(scene, worlds)
        e.run(0, steps)
        got = e.worlds()
    finally:
        lib.emu_set_options(1)
    ref = clone(worlds)
    oracle_run(scene, ref, initial, 0, steps)
    sig = scenes.SCENES[scene].sig
    live = live_word_mask(ref, sig) & live_word_mask(got, sig)
    diff = (words(got) != words(ref)) & live
    solver = solver_field_words(ref)
    assert not (diff & ~solver).any(), np.argwhere(diff & ~solver)[:10].tolist()
    assert (diff & solver).any()   # the lean path really ran


def test_lane_code_default_options_feature_worlds():
    """The same on the coverage worlds, where some worlds have restitution
    contacts (separate warm start) and some do not (fused)."""
    import ctypes as C
    from b3test import EmuSig, emu, feature_worlds, live_word_mask, oracle_step_batch, solver_field_words, words
    from puffysics_amd.creation import CUSTOM_SIG
    worlds = feature_worlds(40)
    ref = clone(worlds)
    lib = emu()
    lib.emu_set_options.argtypes = [C.c_uint]
    lib.emu_set_options(0)
    try:
        e = EmuSig(CUSTOM_SIG, worlds)
        for t in range(40):
            oracle_step_batch(ref, CUSTOM_SIG, 1.0 / 60.0, 4)
            e.step(1.0 / 60.0, 4)
        got = e.worlds()
    finally:
        lib.emu_set_options(1)
    live = live_word_mask(ref, CUSTOM_SIG) & live_word_mask(got, CUSTOM_SIG)
    diff = (words(got) != words(ref)) & live
    assert not (diff & ~solver_field_words(ref)).any()
    rest = ref["contacts"]["restitution"] > 0
    has = np.array([rest[i, :ref["contact_count"][i]].any() for i in range(40)])
    assert has.any() and not has.all()


@pytest.mark.parametrize("scene,count,steps", [(1, 70, 80), (2, 70, 65), (3, 70, 40), (4, 66, 12), (5, 130, 40)])
def test_shared_tile_path_on_the_host(scene, count, steps):
    """The shared-tile path of small batches (staged narrowphase, staged
    preparation, contact levels, level-by-level warm start and sweeps), run
    on the host with one wave per tile: a level's contacts are then solved
    in level order instead of contact order, which a correct levelling does
    not change, so the worlds equal the oracle's word for word."""
    worlds = scenes.build(scene, count)
    initial = clone(worlds)
    e = EmuBatch(scene, worlds)
    e.run(0, steps, shared=True)
    ref = clone(worlds)
    oracle_run(scene, ref, initial, 0, steps)
    bad = diff_words(e.worlds(), ref, scenes.SCENES[scene].sig)
    assert len(bad) == 0, "%d differing words, first %s" % (len(bad), bad[:4].tolist())


@pytest.mark.parametrize("scene,count,steps,masks", [(1, 70, 30, -1), (2, 70, 30, 1), (3, 70, 20, -1),
                                                     (4, 66, 8, -1), (5, 130, 25, -1), (5, 130, 25, 0)])
def test_shared_tile_idle_lanes_on_the_host(scene, count, steps, masks):
    """Idle lanes of a shared tile (worlds past the batch's end or outside
    the step mask) run the shared path with their work skipped, as wave 0
    and as a helper wave: they change no word of their worlds (the oracle
    leaves them alone too) and pass the barriers of a lane with no contact
    levels, while each stepping lane passes those of its own levels."""
    worlds = scenes.build(scene, count)
    initial = clone(worlds)
    e = EmuBatch(scene, worlds)
    e.run(0, steps, shared="idle", masks=masks)
    ref = clone(worlds)
    oracle_run(scene, ref, initial, 0, steps)
    bad = diff_words(e.worlds(), ref, scenes.SCENES[scene].sig)
    assert len(bad) == 0, "%d differing words, first %s" % (len(bad), bad[:4].tolist())


@pytest.mark.parametrize("scene,count,steps,masks", [(2, 70, 65, 1), (4, 66, 12, 0), (5, 130, 40, 0)])
def test_shared_candidate_search_variants_on_the_host(scene, count, steps, masks):
    """Both candidate searches of the shared path on the scenes where the
    engine picks the other one: the overlap masks walked in (i, j) order
    with a binary search for the old contacts (masks=1), and wave 0's
    merged list (masks=0), each equal to the oracle word for word."""
    worlds = scenes.build(scene, count)
    initial = clone(worlds)
    e = EmuBatch(scene, worlds)
    e.run(0, steps, shared=True, masks=masks)
    ref = clone(worlds)
    oracle_run(scene, ref, initial, 0, steps)
    bad = diff_words(e.worlds(), ref, scenes.SCENES[scene].sig)
    assert len(bad) == 0, "%d differing words, first %s" % (len(bad), bad[:4].tolist())


@pytest.mark.parametrize("masks,joint_lds", [(-1, -1), (0, -1), (-1, 1), (0, 1)])
def test_shared_tile_path_on_the_host_feature_worlds(masks, joint_lds):
    """The same on the coverage worlds (restitution, rolling, kinematic and
    locked bodies, welds and hinges), also with the joint rows in LDS
    (joint_lds=1: staged once per step, impulses updated there and written
    back at the end; these capacities leave the device no room for them)."""
    import ctypes as C
    from b3test import EmuSig, emu, feature_worlds, oracle_step_batch
    from puffysics_amd.creation import CUSTOM_SIG
    worlds = feature_worlds(40, hinges=True)
    ref = clone(worlds)
    emu_ = EmuSig(CUSTOM_SIG, worlds)
    lib = emu()
    lib.emu_set_joint_lds.argtypes = [C.c_int]
    lib.emu_set_joint_lds(joint_lds)
    try:
        for _ in range(15):
            oracle_step_batch(ref, CUSTOM_SIG, 1.0 / 60.0, 4)
            emu_.step_shared(1.0 / 60.0, 4, masks=masks)
    finally:
        lib.emu_set_joint_lds(-1)
    bad = diff_words(emu_.worlds(), ref, CUSTOM_SIG)
    assert len(bad) == 0, "%d differing words, first %s" % (len(bad), bad[:4].tolist())


def _with_joint_impulses_lds(mode, fn):
    """Run fn with emu_step keeping the joint impulses in LDS (mode -1: as
    the one-wave kernel chooses, 1: always), then restore the default."""
    import ctypes as C
    from b3test import emu
    lib = emu()
    lib.emu_set_joint_impulses_lds.argtypes = [C.c_int]
    lib.emu_set_joint_impulses_lds(mode)
    try:
        return fn()
    finally:
        lib.emu_set_joint_impulses_lds(0)


@pytest.mark.parametrize("scene,count,steps", [(3, 70, 25), (5, 130, 40)])
def test_lane_code_joint_impulses_in_lds(scene, count, steps):
    """The one-wave step with the joints' accumulated impulses in LDS (staged
    by the joint warm start, written back at the end of the step), as the
    device runs the arm and chain scenes: bit-exact against the oracle."""
    worlds = scenes.build(scene, count)
    initial = clone(worlds)
    e = EmuBatch(scene, worlds)
    _with_joint_impulses_lds(-1, lambda: e.run(0, steps))
    ref = clone(worlds)
    oracle_run(scene, ref, initial, 0, steps)
    bad = diff_words(e.worlds(), ref, scenes.SCENES[scene].sig)
    assert len(bad) == 0, "first differences (world, word): %s" % bad[:10].tolist()
    assert np.abs(ref["joints"]["motor_impulse"]).max() > 0


def test_lane_code_joint_impulses_in_lds_every_feature():
    """Welds (rigid and soft), spring-only and fixed hinges with the
    impulses in LDS (forced: these worlds' joints do not fit the device's
    LDS rows): bit-exact against the oracle over 60 steps with a mask."""
    from b3test import EmuSig, feature_worlds, oracle_step_batch
    from puffysics_amd.creation import CUSTOM_SIG
    worlds = feature_worlds(40)
    ref = clone(worlds)
    emu = EmuSig(CUSTOM_SIG, worlds)
    active = (np.arange(40) % 5 != 2).astype(np.uint8)

    def run():
        for t in range(60):
            act = active if t % 3 == 0 else None
            oracle_step_batch(ref, CUSTOM_SIG, 1.0 / 60.0, 4, act)
            emu.step(1.0 / 60.0, 4, act)

    _with_joint_impulses_lds(1, run)
    bad = diff_words(emu.worlds(), ref, CUSTOM_SIG)
    assert len(bad) == 0, bad[:10].tolist()
    assert np.abs(ref["joints"]["angular_impulse"]["x"][:, 0]).max() > 0


def _with_kept_row0(fn):
    """Run fn with emu_step keeping contact 0's row for the
    step (as b3k_step<JI, true> does), then restore the default."""
    import ctypes as C
    from b3test import emu
    lib = emu()
    lib.emu_set_keep_row0.argtypes = [C.c_int]
    lib.emu_set_keep_row0(1)
    try:
        return fn()
    finally:
        lib.emu_set_keep_row0(0)


@pytest.mark.parametrize("scene,count,steps", [(1, 130, 80), (2, 70, 40), (5, 70, 30)])
def test_lane_code_kept_contact_row(scene, count, steps):
    """The one-wave step with contact 0's row kept for the step
    (delta poses reloaded after each position update, impulses updated in
    place): bit-exact against the oracle.  The hover's worlds have at most
    one contact, as the device's worlds of two shapes; the stacks and the
    arm add contacts after the kept one, which the sweep loads as usual."""
    worlds = scenes.build(scene, count)
    initial = clone(worlds)
    e = EmuBatch(scene, worlds)
    _with_kept_row0(lambda: e.run(0, steps))
    ref = clone(worlds)
    oracle_run(scene, ref, initial, 0, steps)
    bad = diff_words(e.worlds(), ref, scenes.SCENES[scene].sig)
    assert len(bad) == 0, "first differences (world, word): %s" % bad[:10].tolist()
    assert (ref["contact_count"] > 0).any()


def test_lane_code_kept_contact_row_every_feature():
    """The kept row on the coverage worlds (restitution, which rewrites the
    kept row's impulses, rolling, friction, welds and hinges) with a step
    mask, in the default options (the fused warm start) and with the solver
    fields kept: every live word but those fields equals the oracle's."""
    import ctypes as C
    from b3test import EmuSig, emu, feature_worlds, live_word_mask, oracle_step_batch, solver_field_words, words
    from puffysics_amd.creation import CUSTOM_SIG
    lib = emu()
    lib.emu_set_options.argtypes = [C.c_uint]
    for opts in (1, 0):
        worlds = feature_worlds(40)
        ref = clone(worlds)
        e = EmuSig(CUSTOM_SIG, worlds)
        active = (np.arange(40) % 5 != 2).astype(np.uint8)

        def run():
            for t in range(50):
                act = active if t % 3 == 0 else None
                oracle_step_batch(ref, CUSTOM_SIG, 1.0 / 60.0, 4, act)
                e.step(1.0 / 60.0, 4, act)

        lib.emu_set_options(opts)
        try:
            _with_kept_row0(run)
        finally:
            lib.emu_set_options(1)
        got = e.worlds()
        live = live_word_mask(ref, CUSTOM_SIG) & live_word_mask(got, CUSTOM_SIG)
        diff = (words(got) != words(ref)) & live
        if opts:
            assert not diff.any(), np.argwhere(diff)[:10].tolist()
        else:
            assert not (diff & ~solver_field_words(ref)).any()
    rest = ref["contacts"]["restitution"] > 0
    assert any(rest[i, :ref["contact_count"][i]].any() for i in range(40))


def test_lane_code_kept_contact_row_two_shape_worlds():
    """The kept row on varied worlds of two shapes (the worlds the device
    steps with it): restitution bounces, rolling, friction and four-point box
    contacts, bit-exact against the oracle over 120 steps."""
    from b3test import EmuSig, oracle_step_batch, two_shape_worlds
    sig = scenes.SCENES[1].sig
    worlds = two_shape_worlds(120)
    ref = clone(worlds)
    e = EmuSig(sig, worlds)
    rest_hits = 0

    def run():
        nonlocal rest_hits
        for t in range(120):
            oracle_step_batch(ref, sig, 1.0 / 60.0, 4)
            e.step(1.0 / 60.0, 4)
            rest_hits += int(((ref["contacts"]["restitution"][:, 0] > 0) & (ref["contact_count"] > 0)).sum())

    _with_kept_row0(run)
    bad = diff_words(e.worlds(), ref, sig)
    assert len(bad) == 0, bad[:10].tolist()
    assert rest_hits > 0 and (ref["contacts"]["point_count"][:, 0] == 4).any()
