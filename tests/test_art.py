"""Articulation-aware contacts: the step of the reference built with
B3_ART_CONTACTS=1 (01_config.inl:176-187; b3_art.cuh; 08_contacts.inl:
194-232, 422-437), behind B3_ENGINE_ART_CONTACTS; and that build's
reduced-coordinate integrator b3_art_step (09_step.inl:266-323) behind
b3_batch_art_step_gpu.

The oracle's articulated path (oracle/art.inc) is pinned against the
reference's own build of it (oracle/_ref/libb3ref_art_*.so) bit for bit,
and against closed forms of the Delassus operator: a link on one hinge
responds at a point p along n with ((p - anchor) x n . u)^2 / I_axis, and a
floating body with its independent-body mass.  The host build of the lane
code and the device must then match the oracle: bit for bit on worlds whose
hinges are passive (no atan2f on the path), within the single-step
tolerance on the arm scene (motors and limits).

The reduced integrator's restatement is pinned the same way against the
reference's b3_art_step, by a closed form (a hinged box released at rest:
one substep gives the angular acceleration m g d / I_axis, the joint angle
h^2 alpha, and the pose forward kinematics places), and by invariants the
method fixes exactly (tree joints stay joined, loop cuts stay closed).  Its
joint angles go through sinf, cosf and atan2f, so the device matches within
the single-step tolerance, and bit for bit on worlds it sends to the
ordinary step.
"""
import numpy as np
import pytest

import b3test as T
from b3test import clone, diff_words
from puffysics_amd import creation as cr
from puffysics_amd import scenes
from puffysics_amd.b3types import B3_DYNAMIC, B3_STATIC

CUSTOM_SIG = cr.CUSTOM_SIG
DT = 1.0 / 60.0


def _arm_inputs(worlds, t):
    scenes.apply_inputs(5, worlds, t)


CASES = [("passive", 0, 40, None), ("features", 0, 20, None), ("arm", 5, 10, _arm_inputs), ("chain", 3, 10, None)]


def _case_worlds(name, count):
    if name == "passive":
        return T.passive_hinge_worlds(count), CUSTOM_SIG
    if name == "features":
        return T.feature_worlds(count, hinges=True), CUSTOM_SIG
    scene = {"arm": 5, "chain": 3}[name]
    return scenes.build(scene, count), scenes.SCENES[scene].sig


@pytest.mark.parametrize("name,caps,steps,inputs", CASES, ids=[c[0] for c in CASES])
def test_oracle_matches_reference_art_build(name, caps, steps, inputs):
    lib = T.ref_art_lib(caps)
    if lib is None:
        pytest.skip("reference not built (oracle/_ref)")
    worlds, sig = _case_worlds(name, 8)
    assert lib.refa_sig() == sig
    a, b, plain = clone(worlds), clone(worlds), clone(worlds)
    for t in range(steps):
        if inputs:
            for w in (a, b, plain):
                inputs(w, t)
        T.oracle_step_art(a, sig, DT, 4)
        for k in range(len(b)):
            lib.refa_step(b[k:k + 1].ctypes.data, DT, 4)
        T.oracle_step_batch(plain, sig, DT, 4)
    assert len(diff_words(a, b, sig)) == 0
    changed = len(diff_words(a, plain, sig)) > 0
    # the chain scene has no contacts, so the articulated path never runs
    assert changed == (name != "chain")


def test_worlds_without_joints_step_as_usual():
    worlds = scenes.build(2, 6)
    a, b = clone(worlds), clone(worlds)
    for _ in range(20):
        T.oracle_step_art(a, scenes.SCENES[2].sig, DT, 4)
        T.oracle_step_batch(b, scenes.SCENES[2].sig, DT, 4)
    assert len(diff_words(a, b, scenes.SCENES[2].sig)) == 0


def _hinged_box_world():
    """No gravity.  A box of half extent 0.1 (8 kg) hangs on a hinge about z
    at the static post's origin (0, 0.2, 0), centred at (0.3, 0.1, 0), its
    bottom face resting exactly on the ground; a free box rests on the
    ground elsewhere."""
    w = cr.new_worlds(1, gravity=(0.0, 0.0, 0.0))
    g = cr.body(w, 0, B3_STATIC, (0.0, -0.5, 0.0))
    cr.box(w, 0, g, (5.0, 0.5, 5.0))
    post = cr.body(w, 0, B3_STATIC, (0.0, 0.2, 0.0))
    link = cr.body(w, 0, B3_DYNAMIC, (0.3, 0.1, 0.0))
    cr.box(w, 0, link, (0.1, 0.1, 0.1))
    cr.finalize_mass(w, 0, link)
    cr.revolute(w, 0, post, link, (0.0, 0.0, 0.0), (-0.3, 0.1, 0.0), (0.0, 0.0, 1.0))
    free = cr.body(w, 0, B3_DYNAMIC, (-2.0, 0.1, 1.0))
    cr.box(w, 0, free, (0.1, 0.1, 0.1))
    cr.finalize_mass(w, 0, free)
    return w, link, free


def test_delassus_closed_forms():
    """Normal masses written by the articulated sweep: for the hinged box,
    1 / w with w = ((p - anchor) x n . z)^2 / (I_com,z + m d^2) = p_x^2 / I_axis;
    for the free box, the independent-body mass 1 / (1/m + (r x n) . I^-1 (r x n))."""
    w, link, free = _hinged_box_world()
    T.oracle_step_art(w, CUSTOM_SIG, DT, 4)
    m = 8.0
    i_axis = m / 3.0 * (0.01 + 0.01) + m * (0.3 ** 2 + 0.1 ** 2)
    i_com = m / 3.0 * 0.02
    seen = {link: 0, free: 0}
    for c in range(int(w["contact_count"][0])):
        ct = w["contacts"][0, c]
        b = int(ct["body_b"])
        n = np.array([ct["normal"][a] for a in "xyz"], np.float64)
        np.testing.assert_allclose(n, [0.0, 1.0, 0.0], atol=1e-6)
        center = np.array([w["bodies"]["center"][0, b][a] for a in "xyz"], np.float64)
        for p in range(int(ct["point_count"])):
            rb = np.array([ct["points"][p]["r_b"][a] for a in "xyz"], np.float64)
            got = float(ct["points"][p]["normal_mass"])
            if b == link:
                pw = center + rb - np.array([0.0, 0.2, 0.0])
                wgt = np.cross(pw, n)[2] ** 2 / i_axis
            else:
                rn = np.cross(rb, n)
                wgt = 1.0 / m + rn @ rn / i_com
            np.testing.assert_allclose(got, 1.0 / wgt, rtol=1e-5)
            seen[b] += 1
    assert seen[link] >= 2 and seen[free] >= 2


def test_lane_code_matches_oracle():
    for name, steps in (("passive", 30), ("features", 15)):
        worlds, sig = _case_worlds(name, 70)
        ref = clone(worlds)
        emu = T.EmuSig(sig, worlds)
        active = (np.arange(70) % 4 != 1).astype(np.uint8)
        for t in range(steps):
            act = active if t % 2 else None
            T.oracle_step_art(ref, sig, DT, 4, act)
            emu.step_art(DT, 4, act)
        assert len(diff_words(emu.worlds(), ref, sig)) == 0, name


def test_art_option_is_validated_without_a_device():
    from puffysics_amd import _native
    lib = _native.engine_lib()
    assert lib.b3_engine_set_options(None, 2) == 1
    assert lib.b3_engine_set_options(None, 8) == 1


# ---- the reduced-coordinate integrator (b3_art_step) ----

REDUCED_CASES = [("reduced", 0, 40), ("passive", 0, 20), ("arm", 5, 10), ("plain", 2, 10)]


def _reduced_case(name, count):
    if name == "reduced":
        return T.reduced_tree_worlds(count), CUSTOM_SIG
    if name == "passive":
        return T.passive_hinge_worlds(count), CUSTOM_SIG
    scene = {"arm": 5, "plain": 2}[name]
    return scenes.build(scene, count), scenes.SCENES[scene].sig


@pytest.mark.parametrize("name,caps,steps", REDUCED_CASES, ids=[c[0] for c in REDUCED_CASES])
def test_oracle_art_step_matches_reference(name, caps, steps):
    """Bit for bit against the reference's b3_art_step: trees with loop cuts
    and floating roots, the passive-hinge worlds, and worlds it hands to the
    ordinary step (the arm's motors and limits; no joints at all)."""
    lib = T.ref_art_lib(caps)
    if lib is None:
        pytest.skip("reference not built (oracle/_ref)")
    worlds, sig = _reduced_case(name, 8)
    a, b, plain = clone(worlds), clone(worlds), clone(worlds)
    for t in range(steps):
        if name == "arm":
            for w in (a, b, plain):
                _arm_inputs(w, t)
        T.oracle_art_step(a, sig, DT, 4)
        for k in range(len(b)):
            lib.refa_art_step(b[k:k + 1].ctypes.data, DT, 4)
        T.oracle_step_art(plain, sig, DT, 4)
    assert len(diff_words(a, b, sig)) == 0
    reduced = [len(diff_words(a[k:k + 1], plain[k:k + 1], sig)) > 0 for k in range(len(a))]
    if name == "reduced":
        # every fourth world has a motor and takes the ordinary step
        assert reduced == [k % 4 != 3 for k in range(len(a))]
    elif name in ("arm", "plain"):
        assert not any(reduced)


def _qrot(q, v):
    """Rotate vectors v (..., 3) by unit quaternions q (..., 4) = (x, y, z, s)."""
    u, s = q[..., :3], q[..., 3:4]
    t = 2.0 * np.cross(u, v)
    return v + s * t + np.cross(u, t)


def _v(a):
    return np.stack([a[c] for c in "xyz"], axis=-1).astype(np.float64)


def _q(a):
    return np.concatenate([_v(a["v"]), a["s"][..., None].astype(np.float64)], axis=-1)


def test_reduced_hinge_closed_form():
    """A box (half extents 0.2, 0.05, 0.05, density 1) hangs level from a
    static post on a hinge about z at its end, at rest, with no contacts.
    One step of one substep: alpha = -m g hx / (m (hx^2 + hy^2) / 3 + m hx^2);
    the angular velocity is h alpha, the centre's velocity h alpha hx along
    y, the joint angle h^2 alpha (the rate is updated before the angle), and
    the pose is the rotation by that angle about the pivot."""
    w = cr.new_worlds(1, gravity=(0.0, -9.81, 0.0))
    post = cr.body(w, 0, B3_STATIC, (0.0, 2.0, 0.0))
    hx, hy = 0.2, 0.05
    link = cr.body(w, 0, B3_DYNAMIC, (hx, 2.0, 0.0))
    cr.box(w, 0, link, (hx, hy, 0.05))
    cr.finalize_mass(w, 0, link)
    cr.revolute(w, 0, post, link, (0.0, 0.0, 0.0), (-hx, 0.0, 0.0), (0.0, 0.0, 1.0))
    h = DT
    T.oracle_art_step(w, CUSTOM_SIG, h, 1)
    m = 1.0 / float(w["bodies"]["inv_mass"][0, link])
    alpha = -m * 9.81 * hx / (m * (hx * hx + hy * hy) / 3.0 + m * hx * hx)
    b = w["bodies"][0, link]
    np.testing.assert_allclose(_v(b["ang_vel"]), [0.0, 0.0, h * alpha], rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(_v(b["lin_vel"]), [0.0, h * alpha * hx, 0.0], rtol=1e-5, atol=1e-7)
    q = h * h * alpha
    np.testing.assert_allclose(_q(b["rotation"]), [0.0, 0.0, np.sin(q / 2), np.cos(q / 2)], rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(_v(b["center"]), [hx * np.cos(q), 2.0 + hx * np.sin(q), 0.0], rtol=1e-6, atol=1e-7)
    assert int(w["contact_count"][0]) == 0


def _joint_gaps(worlds):
    """World-space distance between the two anchors of every joint."""
    bodies, joints = worlds["bodies"], worlds["joints"]
    pos, rot = _v(bodies["position"]), _q(bodies["rotation"])
    rows = np.arange(worlds.shape[0])[:, None]
    ends = []
    for side in "ab":
        b = joints["body_" + side].astype(np.int64)
        ends.append(pos[rows, b] + _qrot(rot[rows, b], _v(joints["local_anchor_" + side])))
    return np.linalg.norm(ends[1] - ends[0], axis=-1)


def test_reduced_trees_stay_joined_and_loops_closed():
    """Forward kinematics places every child exactly at its hinge, so the
    tree joints' anchors coincide to rounding after any number of steps;
    the cut of each four-bar loop is held by the 5x5 block solve."""
    worlds = T.reduced_tree_worlds(12)
    for _ in range(30):
        T.oracle_art_step(worlds, CUSTOM_SIG, DT, 4)
    gaps = _joint_gaps(worlds)
    for k in range(len(worlds)):
        nj = int(worlds["joint_count"][k])
        g = np.sort(gaps[k, :nj])
        if k % 4 == 3:
            continue            # the ordinary step: soft joints
        assert g[-2] < 1e-4, (k, g)
        assert g[-1] < 2e-2, (k, g)


def test_reduced_lane_code_matches_oracle():
    worlds = T.reduced_tree_worlds(70)
    ref = clone(worlds)
    emu = T.EmuSig(CUSTOM_SIG, worlds)
    active = (np.arange(70) % 4 != 1).astype(np.uint8)
    for t in range(30):
        act = active if t % 2 else None
        T.oracle_art_step(ref, CUSTOM_SIG, DT, 4, act)
        emu.art_step(DT, 4, act)
    assert len(diff_words(emu.worlds(), ref, CUSTOM_SIG)) == 0
    assert ref["contact_count"].sum() > 0


def test_ulp_envelope():
    """The perturbed-libm oracle is the oracle where no sinf, cosf or atan2f
    is on the path (hinge-free worlds: zero spread), and spreads where the
    joint angles are."""
    worlds = scenes.build(2, 6)
    for _ in range(5):
        T.oracle_art_step(worlds, scenes.SCENES[2].sig, DT, 4)
    assert T.ulp_spread(worlds, scenes.SCENES[2].sig, DT, 4, runs=4).max() == 0.0
    trees = T.reduced_tree_worlds(6)
    assert T.ulp_spread(trees, CUSTOM_SIG, DT, 4, runs=4).max() > 0.0


def test_art_step_is_validated_without_a_device():
    from puffysics_amd import _native
    lib = _native.engine_lib()
    assert lib.b3_batch_art_step_gpu(None, DT, 4, None, None, None) == 1


# ---- device ----

torch = pytest.importorskip("torch")


def _dev(a):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.gpu
def test_device_art_bit_exact_on_passive_hinges():
    from puffysics_amd.engine import B3_ENGINE_ART_CONTACTS, B3Engine
    worlds = T.passive_hinge_worlds(130)
    ref = clone(worlds)
    eng = B3Engine(worlds, CUSTOM_SIG)
    eng.set_options(B3_ENGINE_ART_CONTACTS)
    active = (np.arange(130) % 6 != 3).astype(np.uint8)
    d_active = _dev(active)
    for t in range(40):
        act = t % 3 == 1
        T.oracle_step_art(ref, CUSTOM_SIG, DT, 4, active if act else None)
        eng.step(DT, 4, d_active if act else None)
    torch.cuda.synchronize()
    got = eng.download()
    eng.close()
    bad = diff_words(got, ref, CUSTOM_SIG)
    assert len(bad) == 0, "%d differing words, first %s" % (len(bad), bad[:4].tolist())
    assert ref["contact_count"].sum() > 0


@pytest.mark.gpu
def test_device_art_steps_on_the_arm_scene_bit_exact():
    """The arm scene (motors, limits, contacts on the links) with
    articulated contacts over 20 steps with its inputs: every live word
    equals the oracle's (the hinge twist's atan2f has the host library's
    bits on the device)."""
    from puffysics_amd.engine import B3_ENGINE_ART_CONTACTS, B3Engine
    from test_gpu_parity import contact_keys
    sig = scenes.SCENES[5].sig
    worlds = scenes.build(5, 128)
    for t in range(3):
        _arm_inputs(worlds, t)
        T.oracle_step_art(worlds, sig, DT, 4)
    ref = clone(worlds)
    eng = B3Engine(worlds, sig)
    eng.set_options(B3_ENGINE_ART_CONTACTS)
    for t in range(3, 23):
        _arm_inputs(ref, t)
        T.oracle_step_art(ref, sig, DT, 4)
        eng.scene_inputs(5, scenes.SEED, t)              # the same inputs on the device
        eng.step(DT, 4)
    torch.cuda.synchronize()
    got = eng.download()
    eng.close()
    assert contact_keys(got) == contact_keys(ref)
    bad = diff_words(got, ref, sig)
    assert len(bad) == 0, "%d differing words in worlds %s" % (len(bad), np.unique(bad[:, 0])[:10].tolist())


@pytest.mark.gpu
def test_device_art_rejects_force_laws_and_resets():
    """The force-law entry point is not available with the option on; the
    fused reset works as in the ordinary step."""
    from puffysics_amd.engine import B3_ENGINE_ART_CONTACTS, B3Engine, b3_batch_step_gravity_gpu
    worlds = T.passive_hinge_worlds(64)
    eng = B3Engine(worlds, CUSTOM_SIG)
    eng.set_options(B3_ENGINE_ART_CONTACTS)
    assert b3_batch_step_gravity_gpu(eng.handle, DT, 4, 1.0, 0.1) == 801   # hipErrorNotSupported
    for _ in range(5):
        eng.step(DT, 4)
    reset = np.zeros(64, np.uint8)
    reset[::4] = 1
    eng.step(DT, 4, _dev(1 - reset), _dev(reset))
    torch.cuda.synchronize()
    got = eng.download()
    eng.close()
    assert len(diff_words(got[::4], worlds[::4], CUSTOM_SIG)) == 0


@pytest.mark.gpu
def test_device_art_step_one_step_on_reduced_trees():
    """One b3_art_step from the same state as the oracle, bit for bit: the
    joint angles go through sinf, cosf and atan2f, which the device
    evaluates with the host library's bits (or_sinf, or_cosf and fd_atan2f
    in b3d_math.h)."""
    from puffysics_amd.engine import B3_ENGINE_ART_CONTACTS, B3Engine
    from test_gpu_parity import contact_keys
    worlds = T.reduced_tree_worlds(130)
    for _ in range(15):
        T.oracle_art_step(worlds, CUSTOM_SIG, DT, 4)
    ref = clone(worlds)
    eng = B3Engine(worlds, CUSTOM_SIG)
    eng.set_options(B3_ENGINE_ART_CONTACTS)
    T.oracle_art_step(ref, CUSTOM_SIG, DT, 4)
    eng.art_step(DT, 4)
    torch.cuda.synchronize()
    got = eng.download()
    eng.close()
    assert ref["contact_count"].sum() > 100
    assert contact_keys(got) == contact_keys(ref)
    bad = diff_words(got, ref, CUSTOM_SIG)
    assert len(bad) == 0, "%d differing words in worlds %s" % (len(bad), np.unique(bad[:, 0])[:10].tolist())


@pytest.mark.gpu
def test_device_art_step_bit_exact_on_reduced_trees_with_masks():
    """b3_art_step over 30 steps with a step mask on every other step, from
    the worlds' initial state: every live word equals the oracle's."""
    from puffysics_amd.engine import B3_ENGINE_ART_CONTACTS, B3Engine
    worlds = T.reduced_tree_worlds(256)
    ref = clone(worlds)
    eng = B3Engine(worlds, CUSTOM_SIG)
    eng.set_options(B3_ENGINE_ART_CONTACTS)
    active = (np.arange(256) % 7 != 5).astype(np.uint8)
    d_active = _dev(active)
    for t in range(30):
        act = t % 2 == 1
        T.oracle_art_step(ref, CUSTOM_SIG, DT, 4, active if act else None)
        eng.art_step(DT, 4, d_active if act else None)
    torch.cuda.synchronize()
    got = eng.download()
    eng.close()
    bad = diff_words(got, ref, CUSTOM_SIG)
    assert len(bad) == 0, "%d differing words in worlds %s" % (len(bad), np.unique(bad[:, 0])[:10].tolist())
    assert ref["contact_count"].sum() > 0


@pytest.mark.gpu
def test_device_art_step_bit_exact_where_it_falls_back():
    """Worlds without joints take the ordinary step inside b3_art_step:
    bit for bit with the oracle through masks and a fused reset.  Without
    B3_ENGINE_ART_CONTACTS the entry point is refused."""
    from puffysics_amd.engine import B3_ENGINE_ART_CONTACTS, B3Engine, b3_batch_art_step_gpu
    sig = scenes.SCENES[2].sig
    worlds = scenes.build(2, 200)
    ref = clone(worlds)
    eng = B3Engine(worlds, sig)
    assert b3_batch_art_step_gpu(eng.handle, DT, 4) == 801      # hipErrorNotSupported
    eng.set_options(B3_ENGINE_ART_CONTACTS)
    active = (np.arange(200) % 5 != 2).astype(np.uint8)
    d_active = _dev(active)
    for t in range(30):
        act = t % 2 == 1
        T.oracle_art_step(ref, sig, DT, 4, active if act else None)
        eng.art_step(DT, 4, d_active if act else None)
    reset = (np.arange(200) % 4 == 0).astype(np.uint8)
    eng.art_step(DT, 4, _dev(1 - reset), _dev(reset))
    T.oracle_art_step(ref, sig, DT, 4, 1 - reset)
    ref[reset == 1] = worlds[reset == 1]
    torch.cuda.synchronize()
    got = eng.download()
    eng.close()
    bad = diff_words(got, ref, sig)
    assert len(bad) == 0, "%d differing words, first %s" % (len(bad), bad[:4].tolist())
    assert ref["contact_count"].sum() > 0


@pytest.mark.gpu
def test_device_art_step_invariants_at_4096_worlds():
    """4,096 reduced-tree worlds over 25 steps on the device: tree joints
    joined to rounding and loop cuts closed in every world the integrator
    takes, as on the oracle."""
    from puffysics_amd.engine import B3_ENGINE_ART_CONTACTS, B3Engine
    worlds = T.reduced_tree_worlds(4096)
    eng = B3Engine(worlds, CUSTOM_SIG)
    eng.set_options(B3_ENGINE_ART_CONTACTS)
    for _ in range(25):
        eng.art_step(DT, 4)
    torch.cuda.synchronize()
    got = eng.download()
    eng.close()
    reduced = np.arange(4096) % 4 != 3
    finite = np.isfinite(_v(got["bodies"]["center"])).all(axis=(1, 2))
    assert finite[reduced].mean() > 0.99
    gaps = np.sort(_joint_gaps(got), axis=1)
    sel = reduced & finite
    assert (gaps[sel, -2] < 1e-4).all(), gaps[sel, -2].max()
    assert (gaps[sel, -1] < 2e-2).all(), gaps[sel, -1].max()
    assert got["contact_count"].sum() > 4096
