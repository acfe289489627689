"""Parity at the benchmark's full sizes.

The other GPU tests compare against the oracle at sizes it finishes in
seconds.  These run the engine on whole benchmark batches and check
properties that do not depend on the batch size:
  - one step from the same state, at 65,536 arm worlds, against the oracle
    stepping the same 65,536 downloaded worlds: every world word for word;
  - every scene at its benchmark size (4,096 worlds; 65,536 for the arm)
    over many vector steps (masks, resets, inputs), bit-identical to the
    oracle on every world.
"""
import numpy as np
import pytest

from b3test import clone, diff_words, oracle_run
from puffysics_amd import scenes

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _engine(worlds, scene):
    from puffysics_amd.engine import B3_ENGINE_KEEP_SOLVER_FIELDS, B3Engine
    eng = B3Engine(worlds, scenes.SCENES[scene].sig)
    eng.set_options(B3_ENGINE_KEEP_SOLVER_FIELDS)
    return eng


def _gpu_run(eng, scene, t0, nsteps):
    sc = scenes.SCENES[scene]
    reset = torch.zeros(eng.count, dtype=torch.uint8, device="cuda")
    stepm = torch.zeros(eng.count, dtype=torch.uint8, device="cuda")
    for t in range(t0, t0 + nsteps):
        eng.scene_masks(scene, scenes.SEED, t, reset, stepm)
        eng.restore(reset)
        eng.scene_inputs(scene, scenes.SEED, t, stepm)
        eng.step(sc.dt, sc.substeps, stepm)
    torch.cuda.synchronize()


def _assert_same_contacts(got, ref):
    """Contact count, shape pair, point count and feature ids of every live
    contact, vectorised over the batch."""
    assert (got["contact_count"] == ref["contact_count"]).all()
    cg, cr = got["contacts"], ref["contacts"]
    live = np.arange(cg.shape[1])[None, :] < ref["contact_count"][:, None]
    for f in ("shape_a", "shape_b", "body_a", "body_b", "point_count"):
        bad = (cg[f] != cr[f]) & live
        assert not bad.any(), "%s differs at %s" % (f, np.argwhere(bad)[:5].tolist())
    pc = np.where(live, cr["point_count"], 0)
    for p in range(cg["points"].shape[2]):
        on = pc > p
        bad = (cg["points"]["feature"][:, :, p] != cr["points"]["feature"][:, :, p]) & on
        assert not bad.any(), "feature %d differs at %s" % (p, np.argwhere(bad)[:5].tolist())


def test_arm_65536_one_step_from_the_same_state():
    """The 65,536-world arm batch after 40 vector steps on the device, then
    one more step on the device and on the oracle from that same state:
    identical contacts and identical worlds, word for word, in every world
    (the hinge twist's atan2f has the host library's bits on the device)."""
    scene, count, warm = 5, 65536, 40
    sig = scenes.SCENES[scene].sig
    worlds = scenes.build(scene, count)
    eng = _engine(worlds, scene)
    _gpu_run(eng, scene, 0, warm)
    state = eng.download()
    ref = clone(state)
    oracle_run(scene, ref, worlds, warm, 1, threads=16)
    _gpu_run(eng, scene, warm, 1)
    got = eng.download()
    eng.close()
    assert ref["contact_count"].mean() > 8          # a contact-rich state
    _assert_same_contacts(got, ref)
    bad = diff_words(got, ref, sig)
    assert len(bad) == 0, "%d differing words in worlds %s" % (len(bad), np.unique(bad[:, 0])[:10].tolist())


@pytest.mark.parametrize("scene,steps", [(1, 200), (2, 120), (3, 100), (4, 30), (5, 40)])
def test_scene_at_benchmark_size_bit_exact(scene, steps):
    """Hover, stacks, chains and bin at 4,096 worlds and the arm at 65,536,
    with the scenes' masks, resets and inputs."""
    count = scenes.SCENES[scene].worlds
    worlds = scenes.build(scene, count)
    eng = _engine(worlds, scene)
    ref = clone(worlds)
    oracle_run(scene, ref, clone(worlds), 0, steps, threads=16)
    _gpu_run(eng, scene, 0, steps)
    got = eng.download()
    eng.close()
    if scene in (3, 5):                             # the hinges' spring / motor / limit rows ran
        j = ref["joints"]
        assert np.abs(j["spring_impulse"]).max() + np.abs(j["motor_impulse"]).max() > 0
    bad = diff_words(got, ref, scenes.SCENES[scene].sig)
    assert len(bad) == 0, "%d differing words, first %s" % (len(bad), bad[:4].tolist())
