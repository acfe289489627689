"""Parity at the benchmark's full sizes.

The other GPU tests compare against the oracle at sizes it finishes in
seconds.  These run the engine on whole benchmark batches and check
properties that do not depend on the batch size:
  - one step from the same state, at 65,536 arm worlds, against the oracle
    stepping the same 65,536 downloaded worlds: contact pairs, point counts
    and features identical everywhere, body state within the single-step
    tolerance;
  - hinge-free scenes at 4,096 worlds over many vector steps (masks, resets,
    inputs) bit-identical to the oracle on every world.
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


def _body_state(worlds):
    b = worlds["bodies"]
    cols = []
    for f in ("position", "center", "lin_vel", "ang_vel"):
        cols += [b[f][a] for a in "xyz"]
    cols += [b["rotation"]["v"][a] for a in "xyz"] + [b["rotation"]["s"]]
    return np.stack(cols, axis=-1)


def _pre_step(scene, state, initial, t, idx):
    """World idx as step t's b3_step sees it: restored if the reset mask
    selects it, then with step t's scene inputs; and whether it steps."""
    reset, stepm = scenes.masks(scene, 1, t, first=int(idx))
    w = clone(initial[idx:idx + 1] if reset[0] else state[idx:idx + 1])
    scenes.apply_inputs(scene, w, t, stepm, first=int(idx))
    return w, bool(stepm[0])


def test_arm_65536_one_step_from_the_same_state():
    """The 65,536-world arm batch after 40 vector steps on the device, then
    one more step on the device and on the oracle from that same state.

    Contact pairs, point counts and features are identical in every world.
    Body state is within the single-step tolerance in all but a handful of
    worlds (6 of 65,536 when measured): there a contact or joint row sits at
    a clamp or branch threshold, and the 1-ulp difference between the
    device's and glibc's atan2f (the hinge twist) lands on the other side.
    For each such world the test shows that this is the only cause: the same
    lane code built for the host with glibc's atan2f (tests/emu) reproduces
    the oracle bit for bit from the world's pre-step state, and the device,
    stepping that world alone, reproduces its own result in the full batch
    bit for bit (no dependence on the other worlds of its tile)."""
    from b3test import EmuSig
    from puffysics_amd.engine import B3_ENGINE_KEEP_SOLVER_FIELDS, B3Engine
    scene, count, warm = 5, 65536, 40
    sig = scenes.SCENES[scene].sig
    sc = scenes.SCENES[scene]
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
    g, r = _body_state(got), _body_state(ref)
    err = np.abs(g - r)
    ok = err <= 1e-5 + 1e-4 * np.abs(r)
    outliers = np.unique(np.argwhere(~ok)[:, 0])
    assert len(outliers) <= count // 2000, "%d worlds outside the tolerance" % len(outliers)
    assert (err <= 1e-2 + 1e-2 * np.abs(r)).all(), "max err %g" % err.max()
    for i in outliers:
        pre, stepped = _pre_step(scene, state, worlds, warm, i)
        assert stepped
        emu = EmuSig(sig, pre)
        emu.step(sc.dt, sc.substeps)
        assert len(diff_words(emu.worlds(), ref[i:i + 1], sig)) == 0, "lane code on the host differs in world %d" % i
        alone = B3Engine(pre, sig)
        alone.set_options(B3_ENGINE_KEEP_SOLVER_FIELDS)
        alone.step(sc.dt, sc.substeps)
        torch.cuda.synchronize()
        same = len(diff_words(alone.download(), got[i:i + 1], sig)) == 0
        alone.close()
        assert same, "world %d alone differs from the batch" % i


@pytest.mark.parametrize("scene,steps", [(1, 200), (2, 120), (4, 30)])
def test_hinge_free_scene_4096_bit_exact(scene, steps):
    count = scenes.SCENES[scene].worlds
    worlds = scenes.build(scene, count)
    eng = _engine(worlds, scene)
    ref = clone(worlds)
    oracle_run(scene, ref, clone(worlds), 0, steps, threads=16)
    _gpu_run(eng, scene, 0, steps)
    got = eng.download()
    eng.close()
    bad = diff_words(got, ref, scenes.SCENES[scene].sig)
    assert len(bad) == 0, "%d differing words, first %s" % (len(bad), bad[:4].tolist())
