"""The per-substep force hook (B3_USER_FORCES, 01_config.inl:189-198 and
09_step.inl:20-53) with the built-in law: pairwise gravity
(nbody_rigid.cuh:15-66).

The oracle's hook and law are pinned three ways on the CPU: against the
reference's own b3_step compiled with its hook running the reference's own
b3_nbody_apply_forces (oracle/_ref/libb3ref_gravity_*.so), against closed
forms and a float64 integration of two bodies, and against invariants
(momentum of an isolated pair, a massless body, a static source).  The lane
code (host build) and the device (b3_batch_step_gravity_gpu) must then match
the oracle bit for bit on scenes without hinges.
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


def _ref_run(lib, worlds, steps, dt, subs, G, soft, masses=None, inputs=None):
    for t in range(steps):
        if inputs:
            inputs(worlds, t)
        for k in range(len(worlds)):
            mp = None if masses is None else masses[k].ctypes.data
            lib.refg_step(worlds[k:k + 1].ctypes.data, dt, subs, G, soft, mp)


def _oracle_run(worlds, sig, steps, dt, subs, G, soft, masses=None, inputs=None):
    for t in range(steps):
        if inputs:
            inputs(worlds, t)
        T.oracle_step_gravity(worlds, sig, dt, subs, G, soft, masses)


def _arm_inputs(worlds, t):
    scenes.apply_inputs(5, worlds, t)


CASES = [
    # (capacity set, worlds, steps, G, softening, masses?, inputs)
    ("features", 0, 30, 20.0, 0.05, False, None),
    ("stack", 2, 20, 3.0, 0.2, True, None),
    ("bin", 4, 20, 5.0, 0.1, False, None),
    ("arm", 5, 10, 2.0, 0.1, False, _arm_inputs),
]


def _case_worlds(caps, count):
    if caps == 0:
        return T.feature_worlds(count, hinges=True), CUSTOM_SIG
    return scenes.build(caps, count), scenes.SCENES[caps].sig


@pytest.mark.parametrize("name,caps,steps,G,soft,use_masses,inputs", CASES, ids=[c[0] for c in CASES])
def test_oracle_matches_reference_hook(name, caps, steps, G, soft, use_masses, inputs):
    """The oracle's hook and law against the reference's own step, hook
    and b3_nbody_apply_forces, bit for bit on every live word (hinges
    included: both sides use glibc's atan2f)."""
    lib = T.ref_gravity_lib(caps)
    if lib is None:
        pytest.skip("reference not built (oracle/_ref)")
    worlds, sig = _case_worlds(caps, 6)
    assert lib.refg_sig() == sig
    masses = None
    if use_masses:
        masses = np.random.default_rng(3).uniform(0.0, 50.0, (6, sig & 0xFFFF)).astype(np.float32)
        masses[:, 2] = 0.0
    a, b = clone(worlds), clone(worlds)
    _oracle_run(a, sig, steps, DT, 4, G, soft, masses, inputs)
    _ref_run(lib, b, steps, DT, 4, G, soft, masses, inputs)
    assert len(diff_words(a, b, sig)) == 0
    plain = clone(worlds)
    for t in range(steps):
        if inputs:
            inputs(plain, t)
        T.oracle_step_batch(plain, sig, DT, 4)
    assert len(diff_words(a, plain, sig)) > 0   # the law acted


def _pair(m_scale=1.0, d=1.0, static_b=False, vel=(0.0, 0.0, 0.0)):
    """One world, no gravity, two spheres of radius 0.1 a distance d apart
    on x (too far apart to touch)."""
    w = cr.new_worlds(1, gravity=(0.0, 0.0, 0.0))
    a = cr.body(w, 0, B3_DYNAMIC, (0.0, 0.0, 0.0), lin_vel=vel)
    cr.sphere(w, 0, a, 0.1, density=1000.0 * m_scale)
    cr.finalize_mass(w, 0, a)
    b = cr.body(w, 0, B3_STATIC if static_b else B3_DYNAMIC, (d, 0.0, 0.0))
    cr.sphere(w, 0, b, 0.1, density=2000.0)
    if not static_b:
        cr.finalize_mass(w, 0, b)
    return w


def _mass(w, b):
    return 1.0 / float(w["bodies"]["inv_mass"][0, b])


def _v3(a):
    """float64 [..., 3] from a (structured) B3Vec3 array."""
    return np.stack([a["x"], a["y"], a["z"]], -1).astype(np.float64)


def test_gravity_two_bodies_closed_form():
    """One substep: dv_a = G m_b d / (d^2 + eps^2)^1.5 dt toward b, and
    the opposite impulse on b (momentum of the pair stays zero)."""
    G, eps, d, dt = 2.0, 0.1, 1.0, 0.01
    w = _pair(d=d)
    ma, mb = _mass(w, 0), _mass(w, 1)
    T.oracle_step_gravity(w, CUSTOM_SIG, dt, 1, G, eps)
    s = G * d / (d * d + eps * eps) ** 1.5 * dt
    va, vb = _v3(w["bodies"]["lin_vel"][0, 0]), _v3(w["bodies"]["lin_vel"][0, 1])
    np.testing.assert_allclose(va, [s * mb, 0.0, 0.0], rtol=1e-5, atol=0)
    np.testing.assert_allclose(vb, [-s * ma, 0.0, 0.0], rtol=1e-5, atol=0)
    assert abs(ma * va[0] + mb * vb[0]) <= 1e-5 * ma * abs(va[0])
    # the applied forces are zero again after the step (restored, then cleared)
    assert not _v3(w["bodies"]["force"][0, :2]).any()


def test_gravity_reads_current_centers():
    """Strong attraction over 4 substeps against a float64 integration of
    the same semi-implicit scheme (v += a(x) h, then x += v h) with the
    force evaluated at the positions of each substep.  A law that read the
    start-of-step centers would miss by several percent."""
    G, eps, d, dt, subs = 1000.0, 0.1, 1.0, 0.01, 4
    w = _pair(d=d)
    ma, mb = _mass(w, 0), _mass(w, 1)
    T.oracle_step_gravity(w, CUSTOM_SIG, dt, subs, G, eps)
    h = dt / subs
    x = np.array([0.0, d])
    v = np.zeros(2)
    m = np.array([ma, mb])
    for _ in range(subs):
        r = x[1] - x[0]
        f = G * ma * mb * r / (r * r + eps * eps) ** 1.5
        v = v + np.array([f, -f]) / m * h
        x = x + v * h
    np.testing.assert_allclose(_v3(w["bodies"]["lin_vel"][0, :2])[:, 0], v, rtol=1e-4)
    np.testing.assert_allclose(_v3(w["bodies"]["center"][0, :2])[:, 0], x, rtol=1e-4, atol=1e-6)
    # start-of-step centers: distinguishable at this tolerance
    f0 = G * ma * mb * d / (d * d + eps * eps) ** 1.5
    assert abs(f0 / ma * dt - v[0]) > 0.02 * abs(v[0])


def test_gravity_masses_static_source_and_massless_body():
    """Caller masses: a static body with mass sources gravity but does not
    move; a dynamic body of mass 0 neither feels nor sources it."""
    G, eps, d, dt = 1.0, 0.05, 1.0, 0.01
    w = _pair(d=d, static_b=True)
    masses = np.array([[3.0, 5.0] + [0.0] * 14], np.float32)
    T.oracle_step_gravity(w, CUSTOM_SIG, dt, 1, G, eps, masses)
    a = 1.0 * 3.0 * 5.0 * d / (d * d + eps * eps) ** 1.5
    np.testing.assert_allclose(_v3(w["bodies"]["lin_vel"][0, 0]), [a / _mass(w, 0) * dt, 0, 0], rtol=1e-5)
    assert not _v3(w["bodies"]["lin_vel"][0, 1]).any()
    w = _pair(d=d)
    masses = np.array([[0.0, 5.0] + [0.0] * 14], np.float32)
    T.oracle_step_gravity(w, CUSTOM_SIG, dt, 1, G, eps, masses)
    assert not _v3(w["bodies"]["lin_vel"][0, :2]).any()


def test_zero_strength_equals_plain_step():
    """gravity = 0 adds +0 to every force: the step is b3_step's."""
    worlds = T.feature_worlds(6, hinges=True)
    a, b = clone(worlds), clone(worlds)
    for _ in range(10):
        T.oracle_step_gravity(a, CUSTOM_SIG, DT, 4, 0.0, 0.1)
        T.oracle_step_batch(b, CUSTOM_SIG, DT, 4)
    assert len(diff_words(a, b, CUSTOM_SIG)) == 0


@pytest.mark.parametrize("caps", [0, 2, 4, 5])
def test_lane_code_matches_oracle(caps):
    """The host build of the lane code with the law in its hook."""
    worlds, sig = _case_worlds(caps, 70)
    masses = None
    if caps == 2:
        masses = np.random.default_rng(4).uniform(0.0, 20.0, (70, 6)).astype(np.float32)
    ref = clone(worlds)
    emu = T.EmuSig(sig, worlds)
    active = (np.arange(70) % 4 != 1).astype(np.uint8)
    for t in range(8):
        act = active if t % 2 else None
        T.oracle_step_gravity(ref, sig, DT, 4, 4.0, 0.1, masses, act)
        emu.step_gravity(DT, 4, 4.0, 0.1, masses, act)
    assert len(diff_words(emu.worlds(), ref, sig)) == 0


def test_invalid_law_is_rejected_without_a_device():
    from puffysics_amd import _native
    from puffysics_amd.b3types import B3GravityLaw
    lib = _native.engine_lib()
    for G, soft in [(-1.0, 0.1), (1.0, 0.0), (1.0, -0.1), (float("nan"), 0.1), (1.0, float("nan"))]:
        assert lib.b3_batch_step_gravity_gpu(None, DT, 4, None, None, B3GravityLaw(G, soft), None, None) == 1


# ---- device ----

torch = pytest.importorskip("torch")


def _dev(a):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.gpu
@pytest.mark.parametrize("caps", [0, 2, 4])
def test_device_gravity_bit_exact(caps):
    """b3_batch_step_gravity_gpu against the oracle on hinge-free worlds,
    with step masks and caller masses: bit-identical."""
    from puffysics_amd.engine import B3_ENGINE_KEEP_SOLVER_FIELDS, B3Engine
    if caps == 0:
        worlds, sig = T.feature_worlds(100, hinges=False), CUSTOM_SIG
    else:
        worlds, sig = scenes.build(caps, 100), scenes.SCENES[caps].sig
    masses = None
    if caps == 2:
        masses = np.random.default_rng(5).uniform(0.0, 20.0, (100, 6)).astype(np.float32)
    ref = clone(worlds)
    eng = B3Engine(worlds, sig)
    eng.set_options(B3_ENGINE_KEEP_SOLVER_FIELDS)
    active = (np.arange(100) % 5 != 2).astype(np.uint8)
    d_active, d_masses = _dev(active), _dev(masses)
    for t in range(30):
        act = t % 3 == 0
        T.oracle_step_gravity(ref, sig, DT, 4, 4.0, 0.1, masses, active if act else None)
        eng.step_gravity(DT, 4, 4.0, 0.1, d_masses, d_active if act else None)
    torch.cuda.synchronize()
    got = eng.download()
    bad = diff_words(got, ref, sig)
    assert len(bad) == 0, "%d differing words, first %s" % (len(bad), bad[:4].tolist())
    eng.close()


@pytest.mark.gpu
def test_device_gravity_with_resets_and_hinges():
    """The arm scene (motors, limits, contacts): ten gravity steps with the
    scene's inputs from a warmed state, bit for bit with the oracle (the
    hinge twist's atan2f has the host library's bits on the device), and a
    fused reset restores the snapshot."""
    from puffysics_amd.engine import B3_ENGINE_KEEP_SOLVER_FIELDS, B3Engine
    sig = scenes.SCENES[5].sig
    worlds = scenes.build(5, 128)
    for t in range(3):
        scenes.apply_inputs(5, worlds, t)
        T.oracle_step_gravity(worlds, sig, DT, 4, 2.0, 0.1)
    ref = clone(worlds)
    eng = B3Engine(worlds, sig)
    eng.set_options(B3_ENGINE_KEEP_SOLVER_FIELDS)
    for t in range(3, 13):
        scenes.apply_inputs(5, ref, t)
        T.oracle_step_gravity(ref, sig, DT, 4, 2.0, 0.1)
        eng.scene_inputs(5, scenes.SEED, t)
        eng.step_gravity(DT, 4, 2.0, 0.1)
    torch.cuda.synchronize()
    bad = diff_words(eng.download(), ref, sig)
    assert len(bad) == 0, "%d differing words, first %s" % (len(bad), bad[:4].tolist())
    eng.set_snapshots(worlds)
    reset = np.zeros(128, np.uint8)
    reset[::3] = 1
    stepm = 1 - reset
    eng.step_gravity(DT, 4, 2.0, 0.1, None, _dev(stepm), _dev(reset))
    torch.cuda.synchronize()
    got = eng.download()
    assert len(diff_words(got[::3], worlds[::3], scenes.SCENES[5].sig)) == 0
    eng.close()


@pytest.mark.gpu
def test_device_gravity_bad_arguments():
    from puffysics_amd.engine import B3Engine, b3_batch_step_gravity_gpu
    worlds = scenes.build(2, 64)
    eng = B3Engine(worlds, scenes.SCENES[2].sig)
    for G, soft, dt, subs in [(-1.0, 0.1, DT, 4), (1.0, 0.0, DT, 4), (1.0, 0.1, -DT, 4), (1.0, 0.1, DT, 0),
                              (1.0, 0.1, float("inf"), 4)]:
        assert b3_batch_step_gravity_gpu(eng.handle, dt, subs, G, soft) == 1
    before = eng.download()
    assert b3_batch_step_gravity_gpu(eng.handle, 0.0, 4, 1.0, 0.1) == 0
    torch.cuda.synchronize()
    assert len(diff_words(eng.download(), before, scenes.SCENES[2].sig)) == 0
    eng.close()
