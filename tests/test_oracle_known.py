"""Known answers for the oracle: closed forms, textbook geometry, special
cases and invariants that hold whatever the reference's arithmetic order,
so that a dropped term, a wrong sign or a swapped operand in the oracle
fails here even where the golden fixtures do not reach.  Worlds are built
with the creation API (puffysics_amd.creation) and stepped by the oracle.
"""
import math

import numpy as np
import pytest

from b3test import oracle, oracle_run
from puffysics_amd import creation as cr
from puffysics_amd import scenes
from puffysics_amd.b3types import B3_BOX, B3_DYNAMIC, B3_STATIC

SIG = cr.CUSTOM_SIG


def step(worlds, k, dt=1.0 / 60.0, substeps=4):
    oracle().ocpu_step(worlds.ctypes.data + k * worlds.dtype.itemsize, SIG, dt, substeps)


def find_contacts(worlds, k):
    oracle().ocpu_find_contacts(worlds.ctypes.data + k * worlds.dtype.itemsize, SIG)


def apply_force(worlds, k, b, f):
    oracle().ocpu_apply_force(worlds.ctypes.data + k * worlds.dtype.itemsize, SIG, b, *f)


def soft64(hertz, zeta, h):
    omega = 2.0 * math.pi * hertz
    a1 = 2.0 * zeta + h * omega
    a2 = h * omega * a1
    return omega / a1, a2 / (1.0 + a2), 1.0 / (1.0 + a2)


def vec(v):
    return np.array([v["x"], v["y"], v["z"]], np.float64)


def ground_world(n=1):
    w = cr.new_worlds(n, gravity=(0.0, -9.81, 0.0))
    for k in range(n):
        g = cr.body(w, k, B3_STATIC, (0.0, -0.5, 0.0))
        cr.box(w, k, g, (5.0, 0.5, 5.0))
    return w


def test_soft_constraint_coefficients_closed_form():
    """Contact softness of a static contact (2x the 30 Hz contact rate,
    half the damping) and the 90 Hz / zeta 2 joint softness."""
    import ctypes as C
    from b3test import oracle as _o
    _o().ocpu_apply_force.argtypes = [C.c_void_p, C.c_ulonglong, C.c_int, C.c_float, C.c_float, C.c_float]
    w = ground_world()
    b = cr.body(w, 0, B3_DYNAMIC, (0.0, 0.5, 0.0))
    cr.box(w, 0, b, (0.5, 0.5, 0.5))
    cr.finalize_mass(w, 0, b)
    step(w, 0)
    c = w[0]["contacts"][0]
    h = (1.0 / 60.0) / 4
    hertz = min(30.0, 0.25 * 4 * 60.0)
    want = soft64(2.0 * hertz, 0.5 * 10.0, h)
    got = (c["softness"]["bias_rate"], c["softness"]["mass_scale"], c["softness"]["impulse_scale"])
    assert int(c["static_contact"]) == 1
    np.testing.assert_allclose(got, want, rtol=2e-6)
    # hinge chain joints: constraint_hertz 90, constraint_damping 2
    ch = scenes.build(3, 1)
    oracle_run(3, ch, ch.copy(), 0, 1)
    j = ch[0]["joints"][0]
    want = soft64(90.0, 2.0, (1.0 / 120.0) / 8)
    got = (j["softness"]["bias_rate"], j["softness"]["mass_scale"], j["softness"]["impulse_scale"])
    np.testing.assert_allclose(got, want, rtol=2e-6)


def test_free_flight_is_semi_implicit_euler():
    import ctypes as C
    oracle().ocpu_apply_force.argtypes = [C.c_void_p, C.c_ulonglong, C.c_int, C.c_float, C.c_float, C.c_float]
    w = cr.new_worlds(1, gravity=(0.0, -9.81, 0.0))
    b = cr.body(w, 0, B3_DYNAMIC, (0.0, 10.0, 0.0), lin_vel=(1.0, 2.0, 3.0))
    cr.sphere(w, 0, b, 0.25)
    cr.set_inertial(w, 0, b, 2.0, (0.1, 0.1, 0.1))
    apply_force(w, 0, b, (0.0, 5.0, 0.0))
    dt, n = 1.0 / 60.0, 4
    h = dt / n
    a = np.array([0.0, 5.0 / 2.0 - 9.81, 0.0])
    v0 = np.array([1.0, 2.0, 3.0])
    p0 = np.array([0.0, 10.0, 0.0])
    step(w, 0, dt, n)
    body = w[0]["bodies"][b]
    np.testing.assert_allclose(vec(body["lin_vel"]), v0 + n * h * a, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(vec(body["position"]), p0 + h * (n * v0 + h * a * n * (n + 1) / 2), rtol=1e-6, atol=1e-6)
    assert (vec(body["force"]) == 0).all() and (vec(body["torque"]) == 0).all()


@pytest.mark.parametrize("gap,expect", [(0.0, 1), (-0.01, 1), (0.002, 0)])
def test_sphere_on_box_contact(gap, expect):
    """Sphere-box manifolds exist only for touching or penetrating spheres
    (05_collision.inl:131-150 has no speculative margin), with the normal
    from the box (shape A) to the sphere and separation = -penetration."""
    w = ground_world()
    b = cr.body(w, 0, B3_DYNAMIC, (0.3, 0.5 + gap, -0.2))
    cr.sphere(w, 0, b, 0.5)
    cr.finalize_mass(w, 0, b)
    find_contacts(w, 0)
    assert int(w[0]["contact_count"]) == expect
    if not expect:
        return
    c = w[0]["contacts"][0]
    assert (int(c["shape_a"]), int(c["shape_b"]), int(c["point_count"])) == (0, 1, 1)
    assert int(c["points"][0]["feature"]) == 3            # sphere-box
    np.testing.assert_allclose(vec(c["normal"]), [0.0, 1.0, 0.0], atol=1e-7)   # A (box) -> B (sphere)
    p = c["points"][0]
    sep = p["base_sep"] + np.dot(vec(p["r_b"]) - vec(p["r_a"]), vec(c["normal"]))
    assert abs(sep - gap) < 1e-6


def test_resting_cube_gets_four_face_points():
    w = ground_world()
    b = cr.body(w, 0, B3_DYNAMIC, (0.0, 0.5, 0.0))
    cr.box(w, 0, b, (0.5, 0.5, 0.5))
    cr.finalize_mass(w, 0, b)
    find_contacts(w, 0)
    assert int(w[0]["contact_count"]) == 1
    c = w[0]["contacts"][0]
    assert int(c["point_count"]) == 4
    feats = sorted(int(c["points"][p]["feature"]) for p in range(4))
    assert feats in ([16, 17, 18, 19], [20, 21, 22, 23])
    center_b = vec(w[0]["bodies"][b]["center"])
    corners = set()
    for p in range(4):
        pt = c["points"][p]
        sep = pt["base_sep"] + np.dot(vec(pt["r_b"]) - vec(pt["r_a"]), vec(c["normal"]))
        assert abs(sep) < 1e-6
        world_b = vec(pt["r_b"]) + center_b
        corners.add((round(world_b[0], 5), round(world_b[1], 5), round(world_b[2], 5)))
    assert corners == {(sx, 0.0, sz) for sx in (-0.5, 0.5) for sz in (-0.5, 0.5)}


def test_crossed_capsules_closest_segments():
    """Capsule A along y, capsule B along x (rotated 90 deg about z) just
    overlapping its top: the closest points are the segment end of A and
    B's midpoint, the normal is +y and the separation the overlap."""
    w = cr.new_worlds(1, gravity=(0.0, 0.0, 0.0))
    a = cr.body(w, 0, B3_DYNAMIC, (0.0, 0.0, 0.0))
    cr.capsule(w, 0, a, 0.3, 0.1)
    s = math.sin(math.pi / 4)
    b = cr.body(w, 0, B3_DYNAMIC, (0.0, 0.3 + 0.1 + 0.1 - 0.005, 0.0), rot=(0.0, 0.0, s, s))
    cr.capsule(w, 0, b, 0.4, 0.1)
    for k in (a, b):
        cr.finalize_mass(w, 0, k)
    find_contacts(w, 0)
    c = w[0]["contacts"][0]
    assert int(c["point_count"]) == 1 and int(c["points"][0]["feature"]) == 2
    np.testing.assert_allclose(vec(c["normal"]), [0.0, 1.0, 0.0], atol=1e-6)
    p = c["points"][0]
    sep = p["base_sep"] + np.dot(vec(p["r_b"]) - vec(p["r_a"]), vec(c["normal"]))
    assert abs(sep + 0.005) < 1e-6


def test_head_on_collision_conserves_linear_momentum():
    w = cr.new_worlds(1, gravity=(0.0, 0.0, 0.0))
    a = cr.body(w, 0, B3_DYNAMIC, (-0.26, 0.0, 0.0), lin_vel=(2.0, 0.3, 0.0))
    cr.sphere(w, 0, a, 0.25)
    b = cr.body(w, 0, B3_DYNAMIC, (0.26, 0.05, 0.0), lin_vel=(-1.0, 0.0, 0.1))
    cr.sphere(w, 0, b, 0.25, density=3000.0)
    for k in (a, b):
        cr.finalize_mass(w, 0, k)

    def momentum():
        bs = w[0]["bodies"]
        return sum(vec(bs[k]["lin_vel"]) / bs[k]["inv_mass"] for k in (a, b))

    p0 = momentum()
    touched = 0
    for _ in range(20):
        step(w, 0)
        touched += int(w[0]["contact_count"])
    assert touched > 0
    np.testing.assert_allclose(momentum(), p0, rtol=1e-5, atol=1e-4)


def test_bin_invariants():
    count = 6
    worlds = scenes.build(4, count)
    oracle_run(4, worlds, worlds.copy(), 0, 150, threads=4)
    b = worlds["bodies"]
    live = np.arange(b.shape[1])[None, :] < worlds["body_count"][:, None]
    qn = sum(b["rotation"]["v"][a].astype(np.float64) ** 2 for a in "xyz") + b["rotation"]["s"].astype(np.float64) ** 2
    assert np.abs(qn[live] - 1.0).max() < 1e-5
    for key in ("force", "torque"):
        assert all((b[key][a][live] == 0).all() for a in "xyz")
    for w in worlds:
        n = int(w["contact_count"])
        assert 0 < n <= 128 and int(w["contacts_dropped"]) == 0
        pairs = [(int(c["shape_a"]), int(c["shape_b"])) for c in w["contacts"][:n]]
        assert all(x < y for x, y in pairs)
        assert pairs == sorted(set(pairs))
        for c in w["contacts"][:n]:
            ni = np.array([c["points"][p]["normal_impulse"] for p in range(int(c["point_count"]))])
            assert (ni >= 0).all()
            fi = math.hypot(float(c["friction_impulse"]["x"]), float(c["friction_impulse"]["y"]))
            assert fi <= float(c["friction"]) * ni.sum() * (1 + 1e-5) + 1e-7


def test_hinge_limit_acts_only_beyond_the_limit():
    """A hinge about z with limits +-0.5 rad and no gravity: a child
    twisted to 0.7 rad is pulled back toward the limit (the angle, read as
    2 atan2(q.z, q.s) for a pure z rotation, decreases but stays above the
    limit after one soft step); a child at 0.2 rad is left exactly alone."""
    for angle in (0.7, 0.2):
        w = cr.new_worlds(1, gravity=(0.0, 0.0, 0.0))
        base = cr.body(w, 0, B3_STATIC, (0.0, 0.0, 0.0))
        child = cr.body(w, 0, B3_DYNAMIC, (0.0, 0.0, 0.0))
        cr.box(w, 0, child, (0.2, 0.2, 0.2))
        cr.finalize_mass(w, 0, child)
        j = cr.revolute(w, 0, base, child, (0.0, 0.0, 0.0), (0.0, 0.0, 0.0), (0.0, 0.0, 1.0))
        cr.joint_limits(w, 0, j, -0.5, 0.5)
        w["bodies"]["rotation"]["v"]["z"][0, child] = math.sin(angle / 2)
        w["bodies"]["rotation"]["s"][0, child] = math.cos(angle / 2)
        step(w, 0)
        q = w[0]["bodies"][child]["rotation"]
        after = 2.0 * math.atan2(float(q["v"]["z"]), float(q["s"]))
        assert abs(float(q["v"]["x"])) < 1e-6 and abs(float(q["v"]["y"])) < 1e-6
        if angle > 0.5:
            assert 0.5 < after < angle - 1e-3
        else:
            assert abs(after - angle) < 1e-6
            jt = w[0]["joints"][j]
            assert float(jt["upper_impulse"]) == 0.0 and float(jt["lower_impulse"]) == 0.0
