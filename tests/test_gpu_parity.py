"""GPU engine against the oracle (the reference's b3_step restated on the CPU).

Everything runs through the C ABI of libb3engine.so.  Tolerances are the
parity contract of the engine:
  - contact pairs, point counts and feature ids bit-exact;
  - single-step body state within 1e-4 relative / 1e-5 absolute;
  - over long runs, per-world mean height and mean energy within 1%
    (tests/test_gpu_fullsize.py, at the benchmarks' full sizes and
    lengths).
The hinge twist's atan2f runs the host C library's method on the device
(fd_atan2f in puffysics_amd/csrc/b3d_math.h, pinned bit for bit against
glibc in tests/test_atan2.py and tests/test_gpu_atan2.py), so every scene,
hinged or not, must be bit-identical to the oracle.
"""
import numpy as np
import pytest

from b3test import clone, diff_words, oracle_run, solver_field_words, words
from puffysics_amd import scenes

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _engine(worlds, scene, keep=True):
    """An engine on `worlds`; `keep` also maintains the contacts' prepared
    solver fields, so that whole worlds compare word for word."""
    from puffysics_amd.engine import B3_ENGINE_KEEP_SOLVER_FIELDS, B3Engine
    eng = B3Engine(worlds, scenes.SCENES[scene].sig)
    if keep:
        eng.set_options(B3_ENGINE_KEEP_SOLVER_FIELDS)
    return eng


def gpu_run(eng, scene, t0, nsteps, seed=scenes.SEED):
    """The workload loop on the device: masks, restore, inputs, step."""
    sc = scenes.SCENES[scene]
    reset = torch.zeros(eng.count, dtype=torch.uint8, device="cuda")
    stepm = torch.zeros(eng.count, dtype=torch.uint8, device="cuda")
    for t in range(t0, t0 + nsteps):
        eng.scene_masks(scene, seed, t, reset, stepm)
        eng.restore(reset)
        eng.scene_inputs(scene, seed, t, stepm)
        eng.step(sc.dt, sc.substeps, stepm)
    torch.cuda.synchronize()


def describe(bad, got, ref, initial):
    """First differing words with the device, oracle and initial values."""
    wg, wr, wi = words(got), words(ref), words(initial)
    rows = ["world %d word %d: device %08x oracle %08x initial %08x" % (i, k, wg[i, k], wr[i, k], wi[i, k])
            for i, k in bad[:8]]
    return "%d differing words in worlds %s\n%s" % (len(bad), np.unique(bad[:, 0])[:20].tolist(), "\n".join(rows))


def contact_keys(worlds):
    """(world, contact, shape_a, shape_b, point_count, features...) rows."""
    rows = []
    for i, w in enumerate(worlds):
        for c in range(int(w["contact_count"])):
            ct = w["contacts"][c]
            pc = int(ct["point_count"])
            feats = tuple(int(ct["points"][p]["feature"]) for p in range(pc))
            rows.append((i, c, int(ct["shape_a"]), int(ct["shape_b"]), pc) + feats)
    return rows


def body_state(worlds):
    b = worlds["bodies"]
    cols = []
    for f in ("position", "center", "lin_vel", "ang_vel"):
        cols += [b[f][a] for a in "xyz"]
    cols += [b["rotation"]["v"][a] for a in "xyz"] + [b["rotation"]["s"]]
    return np.stack(cols, axis=-1)


def assert_close_state(got, ref, rel=1e-4, abs_=1e-5):
    g, r = body_state(got), body_state(ref)
    err = np.abs(g - r)
    ok = err <= abs_ + rel * np.abs(r)
    assert ok.all(), "max err %g at %s" % (err.max(), np.argwhere(~ok)[:5].tolist())


@pytest.mark.parametrize("scene,count,steps", [(1, 200, 120), (2, 200, 130), (3, 200, 120), (4, 130, 60),
                                               (5, 200, 80)])
def test_scenes_bit_exact(scene, count, steps):
    worlds = scenes.build(scene, count)
    eng = _engine(worlds, scene)
    ref = clone(worlds)
    oracle_run(scene, ref, clone(worlds), 0, steps, threads=8)
    gpu_run(eng, scene, 0, steps)
    got = eng.download()
    bad = diff_words(got, ref, scenes.SCENES[scene].sig)
    assert len(bad) == 0, describe(bad, got, ref, worlds)


@pytest.mark.parametrize("scene,count", [(1, 130), (2, 130), (3, 130), (4, 70), (5, 200)])
def test_single_step_parity(scene, count):
    worlds = scenes.build(scene, count)
    # advance a little on the oracle so contacts and warm starts exist
    warm = 30 if scene != 4 else 20
    oracle_run(scene, worlds, clone(worlds), 0, warm, threads=8)
    fresh = scenes.build(scene, count)
    eng = _engine(worlds, scene)
    eng.set_snapshots(fresh)
    ref = clone(worlds)
    oracle_run(scene, ref, fresh, warm, 1)
    gpu_run(eng, scene, warm, 1)
    got = eng.download()
    assert contact_keys(got) == contact_keys(ref)
    assert_close_state(got, ref)


def test_fused_reset_equals_restore_then_step():
    scene = 5
    sc = scenes.SCENES[scene]
    worlds = scenes.build(scene, 192)
    a = _engine(worlds, scene)
    b = _engine(worlds, scene)
    gpu_run(a, scene, 0, 5)
    gpu_run(b, scene, 0, 5)
    reset = torch.zeros(192, dtype=torch.uint8, device="cuda")
    reset[::7] = 1
    stepm = torch.ones(192, dtype=torch.uint8, device="cuda")
    stepm[::3] = 0
    a.step(sc.dt, sc.substeps, stepm, reset)
    b.restore(reset)
    b.step(sc.dt, sc.substeps, stepm)
    torch.cuda.synchronize()
    assert len(diff_words(a.download(), b.download(), sc.sig)) == 0


def test_apply_matches_host_apply():
    scene = 2
    sc = scenes.SCENES[scene]
    worlds = scenes.build(scene, 96)
    eng = _engine(worlds, scene)
    nb = sc.caps[0]
    g = torch.Generator().manual_seed(3)
    f = torch.randn(96, nb, 3, generator=g)
    tq = torch.randn(96, nb, 3, generator=g)
    imp = torch.randn(96, nb, 3, generator=g)
    mask = (torch.arange(96) % 4 != 1).to(torch.uint8)
    eng.apply(f.cuda(), tq.cuda(), imp.cuda(), mask.cuda())
    torch.cuda.synchronize()
    got = eng.download()
    ref = clone(worlds)
    fn, tn, pn = f.numpy(), tq.numpy(), imp.numpy()
    live = np.arange(nb)[None, :] < ref["body_count"][:, None]
    sel = mask.numpy().astype(bool)[:, None] & live
    dyn = sel & (ref["bodies"]["type"] == 2)
    for k, a in enumerate("xyz"):
        F = ref["bodies"]["force"][a]
        F[sel] = (F + fn[:, :, k])[sel]
        T = ref["bodies"]["torque"][a]
        T[sel] = (T + tn[:, :, k])[sel]
        V = ref["bodies"]["lin_vel"][a]
        V[dyn] = (V + ref["bodies"]["inv_mass"] * pn[:, :, k])[dyn]
    assert len(diff_words(got, ref, sc.sig)) == 0


def test_stats_match_worlds():
    scene = 4
    worlds = scenes.build(scene, 70)
    eng = _engine(worlds, scene)
    gpu_run(eng, scene, 0, 30)
    st = eng.stats()
    got = eng.download()
    assert (st["contact_count"] == got["contact_count"]).all()
    assert (st["body_count"] == got["body_count"]).all()
    assert (st["contacts_dropped"] == got["contacts_dropped"]).all()


def test_invalid_arguments_do_not_launch():
    from puffysics_amd.engine import b3_batch_step_gpu, HIP_ERROR_INVALID_VALUE
    scene = 1
    worlds = scenes.build(scene, 64)
    eng = _engine(worlds, scene)
    before = eng.download()
    for dt, subs in ((float("nan"), 4), (-1.0, 4), (float("inf"), 4), (1.0 / 60, 0)):
        assert b3_batch_step_gpu(eng.handle, dt, subs) == HIP_ERROR_INVALID_VALUE
    assert b3_batch_step_gpu(eng.handle, 0.0, 4) == 0
    torch.cuda.synchronize()
    assert (eng.download().view(np.uint8) == before.view(np.uint8)).all()


@pytest.mark.parametrize("scene", [1, 2, 3, 4, 5])
def test_against_reference_fixtures(scene):
    """The device against the reference's own outputs (tests/golden), bit
    for bit at every checkpoint, hinged scenes included (the hinge twist's
    atan2f has the host library's bits on the device)."""
    from test_oracle_golden import golden
    states, checkpoints = golden(scene)
    init = states["initial"]
    eng = _engine(init, scene)
    t = 0
    for cp in checkpoints:
        gpu_run(eng, scene, t, cp - t)
        t = cp
        got, ref = eng.download(), states["step%d" % cp]
        assert contact_keys(got) == contact_keys(ref)
        bad = diff_words(got, ref, scenes.SCENES[scene].sig)
        assert len(bad) == 0, describe(bad, got, ref, init)


def test_feature_worlds_without_hinges_bit_exact():
    """Welds, kinematic bodies, restitution, rolling, locks, damping,
    filters and contact overflow on the device: bit-identical to the oracle
    over 80 steps with a step mask on every third step."""
    from b3test import feature_worlds, oracle_step_batch
    from puffysics_amd.creation import CUSTOM_SIG
    from puffysics_amd.engine import B3_ENGINE_KEEP_SOLVER_FIELDS, B3Engine
    worlds = feature_worlds(100, hinges=False)
    ref = clone(worlds)
    eng = B3Engine(worlds, CUSTOM_SIG)
    eng.set_options(B3_ENGINE_KEEP_SOLVER_FIELDS)
    active = (np.arange(100) % 5 != 2).astype(np.uint8)
    d_active = torch.from_numpy(active).cuda()
    for t in range(80):
        act = t % 3 == 0
        oracle_step_batch(ref, CUSTOM_SIG, 1.0 / 60.0, 4, active if act else None)
        eng.step(1.0 / 60.0, 4, d_active if act else None)
    torch.cuda.synchronize()
    got = eng.download()
    bad = diff_words(got, ref, CUSTOM_SIG)
    assert len(bad) == 0, describe(bad, got, ref, worlds)
    assert ref["contacts_dropped"].max() > 0


def test_feature_worlds_with_hinges_bit_exact():
    """The coverage worlds with hinges too (springs, motors, limits and
    fixed hinges, whose rows use the twist's atan2f): bit-identical to the
    oracle over 60 steps with a step mask on every third step."""
    from b3test import feature_worlds, oracle_step_batch
    from puffysics_amd.creation import CUSTOM_SIG
    from puffysics_amd.engine import B3_ENGINE_KEEP_SOLVER_FIELDS, B3Engine
    worlds = feature_worlds(100)
    ref = clone(worlds)
    eng = B3Engine(worlds, CUSTOM_SIG)
    eng.set_options(B3_ENGINE_KEEP_SOLVER_FIELDS)
    active = (np.arange(100) % 5 != 2).astype(np.uint8)
    d_active = torch.from_numpy(active).cuda()
    for t in range(60):
        act = t % 3 == 0
        oracle_step_batch(ref, CUSTOM_SIG, 1.0 / 60.0, 4, active if act else None)
        eng.step(1.0 / 60.0, 4, d_active if act else None)
    torch.cuda.synchronize()
    got = eng.download()
    bad = diff_words(got, ref, CUSTOM_SIG)
    assert len(bad) == 0, describe(bad, got, ref, worlds)
    assert np.abs(ref["joints"]["motor_impulse"]).max() > 0


def test_default_options_differ_only_in_solver_fields():
    """Without B3_ENGINE_KEEP_SOLVER_FIELDS the worlds evolve identically;
    only the prepared solver fields of the live contacts are not written."""
    worlds = scenes.build(4, 130)
    keep = _engine(worlds, 4)
    lean = _engine(worlds, 4, keep=False)
    gpu_run(keep, 4, 0, 40)
    gpu_run(lean, 4, 0, 40)
    a, b = keep.download(), lean.download()
    bad = diff_words(a, b, scenes.SCENES[4].sig)
    allowed = solver_field_words(a)
    assert len(bad) > 0   # the lean rows do hold stale values
    assert allowed[bad[:, 0], bad[:, 1]].all(), bad[~allowed[bad[:, 0], bad[:, 1]]][:10].tolist()


@pytest.mark.parametrize("scene,count,steps", [(2, 256, 40), (4, 192, 10), (5, 256, 30)])
def test_shared_narrowphase_matches_one_wave_per_tile(scene, count, steps):
    """Batches of at most one tile per CU split the step over eight waves
    per tile (the narrowphase over four of them); the worlds equal those of
    the one-wave launch word for word, through masks, resets (restored by
    eight waves) and the fused reset."""
    from puffysics_amd.engine import B3_ENGINE_KEEP_SOLVER_FIELDS, B3_ENGINE_ONE_WAVE_PER_TILE
    worlds = scenes.build(scene, count)
    shared = _engine(worlds, scene)
    one = _engine(worlds, scene, keep=False)
    one.set_options(B3_ENGINE_KEEP_SOLVER_FIELDS | B3_ENGINE_ONE_WAVE_PER_TILE)
    gpu_run(shared, scene, 0, steps)
    gpu_run(one, scene, 0, steps)
    sc = scenes.SCENES[scene]
    reset = torch.from_numpy((np.arange(count) % 7 == 3).astype(np.uint8)).cuda()
    for eng in (shared, one):
        eng.step(sc.dt, sc.substeps, None, reset)
    torch.cuda.synchronize()
    a, b = shared.download(), one.download()
    shared.close()
    one.close()
    bad = diff_words(a, b, sc.sig)
    assert len(bad) == 0, "%d differing words, first %s" % (len(bad), bad[:4].tolist())
    assert a["contact_count"].sum() > 0


@pytest.mark.parametrize("one_wave", [False, True], ids=["shared", "one_wave"])
def test_default_options_mixed_waves(one_wave):
    """Default options on the coverage worlds, where worlds with and without
    restitution share waves: in the one-wave kernel (the kernel of large
    batches, forced here) those without it warm-start inside preparation,
    the others in the separate pass, and every wave computes the packed
    records' slots over all of its lanes; the shared-tile kernel (200 worlds
    are 4 tiles) warm-starts level by level.  Every live word except the
    prepared solver fields equals the oracle's, bit for bit, on the
    hinge-free worlds."""
    from b3test import feature_worlds, live_word_mask, oracle_step_batch
    from puffysics_amd.creation import CUSTOM_SIG
    from puffysics_amd.engine import B3_ENGINE_ONE_WAVE_PER_TILE, B3Engine
    worlds = feature_worlds(200, seed=3, hinges=False)
    ref = clone(worlds)
    eng = B3Engine(worlds, CUSTOM_SIG)
    if one_wave:
        eng.set_options(B3_ENGINE_ONE_WAVE_PER_TILE)
    active = (np.arange(200) % 7 != 4).astype(np.uint8)
    d_active = torch.from_numpy(active).cuda()
    for t in range(40):
        act = t % 2 == 1
        oracle_step_batch(ref, CUSTOM_SIG, 1.0 / 60.0, 4, active if act else None)
        eng.step(1.0 / 60.0, 4, d_active if act else None)
    torch.cuda.synchronize()
    got = eng.download()
    eng.close()
    live = live_word_mask(ref, CUSTOM_SIG) & live_word_mask(got, CUSTOM_SIG)
    diff = (words(got) != words(ref)) & live & ~solver_field_words(ref)
    assert not diff.any(), describe(np.argwhere(diff), got, ref, worlds)
    rest = np.array([(ref["contacts"]["restitution"][i, :ref["contact_count"][i]] > 0).any() for i in range(200)])
    assert rest.any() and not rest.all()


@pytest.mark.parametrize("scene,count,steps", [(5, 300, 60), (4, 130, 40), (2, 200, 60)])
def test_default_options_one_wave_scenes(scene, count, steps):
    """The one-wave kernel with the default options (the kernel and options
    of the 65,536-world arm benchmark) on the scenes' own workloads: every
    live word except the prepared solver fields equals the oracle's."""
    from b3test import live_word_mask
    from puffysics_amd.engine import B3_ENGINE_ONE_WAVE_PER_TILE
    worlds = scenes.build(scene, count)
    eng = _engine(worlds, scene, keep=False)
    eng.set_options(B3_ENGINE_ONE_WAVE_PER_TILE)
    ref = clone(worlds)
    oracle_run(scene, ref, clone(worlds), 0, steps, threads=8)
    gpu_run(eng, scene, 0, steps)
    got = eng.download()
    eng.close()
    sig = scenes.SCENES[scene].sig
    live = live_word_mask(ref, sig) & live_word_mask(got, sig)
    wg, wr = words(got), words(ref)
    both_nan = np.isnan(wg.view(np.float32)) & np.isnan(wr.view(np.float32))
    diff = (wg != wr) & live & ~solver_field_words(ref) & ~both_nan
    assert not diff.any(), describe(np.argwhere(diff), got, ref, worlds)
    assert ref["contact_count"].sum() > 0


@pytest.mark.parametrize("keep", [True, False], ids=["keep", "default"])
def test_two_shape_worlds_kept_row(keep):
    """Worlds of two shapes step on the one-wave kernel with their contact's
    row kept for the step (b3k_step<JI, true>) at any batch size: varied
    hover worlds (restitution bounces, rolling, friction, four-point box
    contacts) with a step mask on every other step, against the oracle over
    120 steps; with the solver fields kept every word matches, in the
    default options every live word but those fields."""
    from b3test import live_word_mask, oracle_step_batch, solver_field_words, two_shape_worlds, words
    from puffysics_amd.engine import B3_ENGINE_KEEP_SOLVER_FIELDS, B3Engine
    sig = scenes.SCENES[1].sig
    worlds = two_shape_worlds(300)
    ref = clone(worlds)
    eng = B3Engine(worlds, sig)
    eng.set_options(B3_ENGINE_KEEP_SOLVER_FIELDS if keep else 0)
    active = (np.arange(300) % 7 != 3).astype(np.uint8)
    d_active = torch.from_numpy(active).cuda()
    for t in range(120):
        act = t % 2 == 0
        oracle_step_batch(ref, sig, 1.0 / 60.0, 4, active if act else None)
        eng.step(1.0 / 60.0, 4, d_active if act else None)
    torch.cuda.synchronize()
    got = eng.download()
    if keep:
        bad = diff_words(got, ref, sig)
        assert len(bad) == 0, describe(bad, got, ref, worlds)
    else:
        live = live_word_mask(ref, sig) & live_word_mask(got, sig)
        diff = (words(got) != words(ref)) & live
        assert not (diff & ~solver_field_words(ref)).any(), np.argwhere(diff & ~solver_field_words(ref))[:10].tolist()
    assert (ref["contacts"]["point_count"][:, 0] == 4).any()
