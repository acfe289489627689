"""Shared helpers of the test suite: the oracle (CPU restatement of the
reference b3_step), the host build of the engine's lane code, and world
comparisons.  The oracle and the emulation library are test
infrastructure; the engine never loads them."""
import ctypes as C
import os

import numpy as np

from puffysics_amd import scenes
from puffysics_amd.b3types import B3Contact, B3Point, world_ctype, world_dtype

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_PATH = os.path.join(ROOT, "oracle", "liboracle.so")
REF_DIR = os.path.join(ROOT, "oracle", "_ref")
EMU_PATH = os.path.join(ROOT, "tests", "emu", "libb3emu.so")
GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")

_vp, _i, _ull, _f = C.c_void_p, C.c_int, C.c_ulonglong, C.c_float
_oracle = None
_emu = None
_refs = {}


def oracle():
    global _oracle
    if _oracle is None:
        lib = C.CDLL(ORACLE_PATH)
        lib.ocpu_world_size.restype = C.c_size_t
        lib.ocpu_world_size.argtypes = [_ull]
        lib.ocpu_step.argtypes = [_vp, _ull, _f, _i]
        lib.ocpu_find_contacts.argtypes = [_vp, _ull]
        for n in range(1, 6):
            fn = getattr(lib, "ocpu_run_%d" % n)
            fn.restype = C.c_longlong
            fn.argtypes = [_vp, _vp, _i, _ull, _i, _i, _f, _i, _i, _vp]
        _oracle = lib
    return _oracle


def ref_lib(scene):
    """The reference's own CPU path compiled from its sources, or None."""
    path = os.path.join(REF_DIR, "libb3ref_%d.so" % scene)
    if not os.path.exists(path):
        return None
    if scene not in _refs:
        lib = C.CDLL(path)
        lib.ref_sig.restype = C.c_ulonglong
        lib.ref_world_size.restype = C.c_size_t
        lib.ref_build.argtypes = [_i, _vp, _ull, _i]
        lib.ref_build_batch.argtypes = [_i, _vp, _i, _ull, _i]
        lib.ref_step.argtypes = [_vp, _f, _i]
        lib.ref_run.restype = C.c_longlong
        lib.ref_run.argtypes = [_i, _vp, _vp, _i, _ull, _i, _i, _f, _i, _i, _vp]
        _refs[scene] = lib
    return _refs[scene]


# The -O3 builds of the reference's CPU path (oracle/Makefile FAST_CFLAGS),
# by the x86-64 level they need: the flags each level adds over the last.
FAST_LEVELS = (
    ("v4", "-O3 -march=x86-64-v4 -ffp-contract=off -fno-fast-math",
     {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"}),
    ("v3", "-O3 -march=x86-64-v3 -ffp-contract=off -fno-fast-math",
     {"avx", "avx2", "bmi1", "bmi2", "f16c", "fma", "abm", "movbe", "xsave"}),
)


def host_cpu_flags():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    return set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return set()


def fast_levels_supported():
    """The -O3 build levels this host can run, best first."""
    flags = host_cpu_flags()
    out = []
    need = set()
    for name, cflags, req in reversed(FAST_LEVELS):
        need |= req
        if need <= flags:
            out.append((name, cflags))
    return out[::-1]


def ref_fast_lib(scene, level):
    """The reference's CPU path built -O3 for x86-64 `level`, or None."""
    path = os.path.join(REF_DIR, "libb3ref_%s_%d.so" % (level, scene))
    if not os.path.exists(path):
        return None
    key = (level, scene)
    if key not in _refs:
        lib = C.CDLL(path)
        lib.ref_world_size.restype = C.c_size_t
        lib.ref_build_batch.argtypes = [_i, _vp, _i, _ull, _i]
        lib.ref_run.restype = C.c_longlong
        lib.ref_run.argtypes = [_i, _vp, _vp, _i, _ull, _i, _i, _f, _i, _i, _vp]
        _refs[key] = lib
    return _refs[key]


def emu():
    global _emu
    if _emu is None:
        lib = C.CDLL(EMU_PATH)
        lib.emu_upload.argtypes = [_vp, _i, _ull, _vp]
        lib.emu_download.argtypes = [_vp, _i, _ull, _vp]
        lib.emu_restore.argtypes = [_vp, _vp, _i, _ull, _vp]
        lib.emu_step.argtypes = [_vp, _i, _ull, _f, _i, _vp]
        lib.emu_inputs.argtypes = [_vp, _i, _ull, _i, _ull, _i, _vp]
        lib.emu_world_words.argtypes = [_ull]
        _emu = lib
    return _emu


def oracle_run(scene, worlds, initial, t0, nsteps, seed=scenes.SEED, threads=1):
    """Steps [t0, t0+nsteps) of a scene's workload on the oracle, in place:
    masks, restore, inputs, step (puffysics_amd/scenes/b3_workload.h)."""
    sc = scenes.SCENES[scene]
    fn = getattr(oracle(), "ocpu_run_%d" % scene)
    return fn(worlds.ctypes.data, initial.ctypes.data, len(worlds), seed, t0, nsteps, sc.dt, sc.substeps,
              threads, None)


class EmuBatch:
    """Word-transposed tiles stepped by the host build of the lane code."""

    def __init__(self, scene, worlds):
        self.scene = scene
        self.sc = scenes.SCENES[scene]
        self.count = len(worlds)
        self.dtype = worlds.dtype
        words = emu().emu_world_words(self.sc.sig)
        ntiles = (self.count + 63) // 64
        self.tiles = np.zeros(ntiles * words * 64, np.uint32)
        w = np.ascontiguousarray(worlds)
        self.snap = w.view(np.uint32).copy()   # snapshots stay plain B3World structs
        emu().emu_upload(w.ctypes.data, self.count, self.sc.sig, self.tiles.ctypes.data)

    def run(self, t0, nsteps, seed=scenes.SEED, shared=False, masks=-1):
        """`shared`: the shared-tile path with one wave per tile ("idle":
        with the idle lanes run too, checking every lane's barrier count);
        `masks` -1 picks its candidate search by shape capacity as the
        engine does, 0 / 1 force wave 0's list / the overlap masks."""
        e = emu()
        if shared == "idle":
            e.emu_step_shared_idle.argtypes = [_vp, _i, _ull, _f, _i, _vp, _i]

            def step(*a):
                rc = e.emu_step_shared_idle(*a, masks)
                assert rc == 0, "world %d passed other barriers than a lane of its levels" % (-1 - rc)
        elif shared:
            e.emu_step_shared.argtypes = [_vp, _i, _ull, _f, _i, _vp, _i]
            step = lambda *a: e.emu_step_shared(*a, masks)
        else:
            step = e.emu_step
            step.argtypes = [_vp, _i, _ull, _f, _i, _vp]
        for t in range(t0, t0 + nsteps):
            reset, stepm = scenes.masks(self.scene, self.count, t, seed)
            if reset.any():
                e.emu_restore(self.tiles.ctypes.data, self.snap.ctypes.data, self.count, self.sc.sig,
                              reset.ctypes.data)
            e.emu_inputs(self.tiles.ctypes.data, self.count, self.sc.sig, self.scene, seed, t, stepm.ctypes.data)
            step(self.tiles.ctypes.data, self.count, self.sc.sig, self.sc.dt, self.sc.substeps, stepm.ctypes.data)

    def worlds(self):
        out = np.zeros(self.count, dtype=self.dtype)
        emu().emu_download(self.tiles.ctypes.data, self.count, self.sc.sig, out.ctypes.data)
        return out


# B3Shape has 4 bytes of padding before its 8-aligned category field.
SHAPE_PAD_WORD = 17


def clone(worlds):
    """Byte-exact copy.  numpy copies structured arrays field by field and
    leaves padding bytes of the copy as the allocator returned them."""
    out = np.empty_like(worlds)
    out.view(np.uint8)[:] = np.ascontiguousarray(worlds).view(np.uint8)
    return out


def live_word_mask(worlds, sig):
    """Boolean [count, words] mask of the words b3_step defines: header,
    live bodies / shapes / joints, live contacts without their unused
    point slots.  Struct padding is left out."""
    W = world_ctype(sig)
    nwords = C.sizeof(W) // 4
    n = len(worlds)
    mask = np.zeros((n, nwords), bool)
    bo, so, co, jo = (W.bodies.offset // 4, W.shapes.offset // 4, W.contacts.offset // 4, W.joints.offset // 4)
    bw, sw, cw, jw = 50, 22, C.sizeof(B3Contact) // 4, 115
    pts = B3Contact.points.offset // 4
    pw = C.sizeof(B3Point) // 4
    mask[:, :17] = True
    counts = {f: np.asarray(worlds[f]).astype(np.int64) for f in
              ("body_count", "shape_count", "joint_count", "contact_count")}

    def slots(base, width, cap, count):
        for k in range(cap):
            mask[:, base + k * width:base + (k + 1) * width] = (k < count)[:, None]

    slots(bo, bw, worlds.dtype["bodies"].shape[0], counts["body_count"])
    slots(so, sw, worlds.dtype["shapes"].shape[0], counts["shape_count"])
    mask[:, so + SHAPE_PAD_WORD:so + sw * worlds.dtype["shapes"].shape[0]:sw] = False
    slots(jo, jw, worlds.dtype["joints"].shape[0], counts["joint_count"])
    max_c = worlds.dtype["contacts"].shape[0]
    pc = np.asarray(worlds["contacts"]["point_count"]).astype(np.int64)
    for c in range(max_c):
        live = c < counts["contact_count"]
        base = co + c * cw
        mask[:, base:base + pts] = live[:, None]
        for p in range(4):
            mask[:, base + pts + pw * p:base + pts + pw * (p + 1)] = (live & (p < pc[:, c]))[:, None]
        mask[:, base + pts + pw * 4:base + cw] = live[:, None]
    return mask


def words(worlds):
    return np.ascontiguousarray(worlds).view(np.uint32).reshape(len(worlds), -1)


def diff_words(a, b, sig):
    """Indices (world, word) where two batches differ on live words.  A word
    that reads as a NaN float on both sides counts as equal: the sign and
    payload of a NaN depend on operand order (the reference's capsule-box
    manifold can produce a NaN normal, e.g. the bin scene's world 745 at
    step 22, and the reference, the oracle and the engine then carry NaNs
    with different bits)."""
    m = live_word_mask(a, sig) & live_word_mask(b, sig)
    wa, wb = words(a), words(b)
    both_nan = np.isnan(wa.view(np.float32)) & np.isnan(wb.view(np.float32))
    d = (wa != wb) & m & ~both_nan
    return np.argwhere(d)


# ---- the contacts' prepared solver fields (written only with B3_ENGINE_KEEP_SOLVER_FIELDS) ----

SOLVER_FIELDS = ("inv_mass_a", "inv_mass_b", "inv_i_a", "inv_i_b", "softness", "center_a", "center_b",
                 "tangent_mass", "twist_mass", "rolling_mass")
POINT_SOLVER_FIELDS = ("normal_mass", "rel_vel", "lever")


def solver_field_words(worlds):
    """Mask (world, word) of the prepared solver fields of live contacts."""
    dt = worlds.dtype
    nwords = dt.itemsize // 4
    mask = np.zeros((len(worlds), nwords), bool)
    c_dt = dt.fields["contacts"][0].base
    c_off = dt.fields["contacts"][1]
    p_dt = c_dt.fields["points"][0].base
    p_off = c_dt.fields["points"][1]
    ncount = np.asarray(worlds["contact_count"]).astype(np.int64)
    pc = np.asarray(worlds["contacts"]["point_count"]).astype(np.int64)

    def span(off, sub):
        return off // 4, (off + sub.itemsize) // 4

    for c in range(dt.fields["contacts"][0].shape[0]):
        live = c < ncount
        base = c_off + c * c_dt.itemsize
        for f in SOLVER_FIELDS:
            a, b = span(base + c_dt.fields[f][1], c_dt.fields[f][0])
            mask[:, a:b] |= live[:, None]
        for p in range(c_dt.fields["points"][0].shape[0]):
            on = live & (p < pc[:, c])
            pb = base + p_off + p * p_dt.itemsize
            for f in POINT_SOLVER_FIELDS:
                a, b = span(pb + p_dt.fields[f][1], p_dt.fields[f][0])
                mask[:, a:b] |= on[:, None]
    return mask


# ---- coverage worlds: features the five benchmark scenes do not reach ----

def feature_worlds(count, seed=7, hinges=True):
    """Worlds of capacity set 16/16/32/8 (puffysics_amd.creation) mixing
    weld joints (rigid and soft), spring-only and fixed-rotation hinges,
    kinematic movers, restitution, rolling resistance, axis locks, damping,
    gravity scale, collide_connected, category/mask filtering, and (every
    fourth world) a pile dense enough to overflow the contact capacity.
    `hinges=False` leaves out revolute joints (no atan2f on the path)."""
    from puffysics_amd import creation as cr
    from puffysics_amd.b3types import B3_DYNAMIC, B3_KINEMATIC, B3_STATIC
    rng = np.random.default_rng(seed)
    w = cr.new_worlds(count, gravity=(0.0, -9.81, 0.0))
    for k in range(count):
        g = cr.body(w, k, B3_STATIC, (0.0, -0.5, 0.0))
        cr.box(w, k, g, (5.0, 0.5, 5.0), restitution=float(rng.choice([0.0, 0.3])))
        if k % 4 == 3:
            # overflow pile: 14 small spheres packed in a 3 x 3 x 2 block
            for i in range(14):
                p = (0.1 * (i % 3), 0.12 + 0.1 * (i // 9), 0.1 * ((i // 3) % 3))
                b = cr.body(w, k, B3_DYNAMIC, p)
                cr.sphere(w, k, b, 0.1)
                cr.finalize_mass(w, k, b)
            continue
        kin = cr.body(w, k, B3_KINEMATIC, (-1.0, 0.35, 0.0), lin_vel=(0.4, 0.0, 0.0), ang_vel=(0.0, 0.5, 0.0))
        cr.box(w, k, kin, (0.3, 0.3, 0.3))
        bodies = []
        for i in range(7):
            p = (rng.uniform(-0.8, 0.8), rng.uniform(0.15, 1.5), rng.uniform(-0.8, 0.8))
            ang = rng.uniform(-1, 1, 3)
            q = np.concatenate([np.sin(0.5) * ang / np.linalg.norm(ang), [np.cos(0.5)]])
            b = cr.body(w, k, B3_DYNAMIC, p, rot=tuple(q), lin_vel=tuple(rng.uniform(-1, 1, 3)))
            kind = i % 3
            if kind == 0:
                cr.sphere(w, k, b, rng.uniform(0.1, 0.25), restitution=float(rng.choice([0.0, 0.5])))
            elif kind == 1:
                cr.box(w, k, b, tuple(rng.uniform(0.1, 0.25, 3)))
            else:
                cr.capsule(w, k, b, rng.uniform(0.1, 0.2), rng.uniform(0.05, 0.12))
            cr.finalize_mass(w, k, b)
            bodies.append(b)
        bd = w["bodies"]
        sh = w["shapes"]
        bd["linear_damping"][k, bodies[0]] = 0.3
        bd["angular_damping"][k, bodies[1]] = 0.5
        bd["gravity_scale"][k, bodies[2]] = 0.5
        bd["flags"][k, bodies[3]] |= 0x08 | 0x10 | 0x20          # angular locks
        bd["flags"][k, bodies[4]] |= 0x04                        # linear z lock
        sh["rolling"][k, 3] = 0.05                               # rolling resistance on one shape
        sh["mask"][k, 4] = 0xfffffffffffffffe                    # ignores category bit 0 ...
        sh["category"][k, 0] = 1                                 # ... which the ground box holds
        j = cr.weld(w, k, bodies[5], bodies[6], (0.2, 0.0, 0.0), (-0.2, 0.0, 0.0))
        if k % 2:
            w["joints"]["linear_hertz"][k, j] = 5.0
            w["joints"]["linear_damping"][k, j] = 0.7
            w["joints"]["angular_hertz"][k, j] = 3.0
            w["joints"]["angular_damping"][k, j] = 0.5
        if hinges:
            j = cr.revolute(w, k, bodies[1], bodies[2], (0.0, 0.2, 0.0), (0.0, -0.2, 0.0), (1.0, 0.0, 0.0))
            cr.joint_spring(w, k, j, 0.4, 4.0, 0.7)
            w["joints"]["collide_connected"][k, j] = 1
            j = cr.revolute(w, k, g, kin, (1.0, 0.5, 0.0), (0.0, 0.0, 0.0), (0.0, 1.0, 0.0))  # fixed rotation
            cr.joint_limits(w, k, j, -0.3, 0.3)
            j = cr.revolute(w, k, g, bodies[0], (0.5, 1.0, 0.5), (0.0, 0.1, 0.0), (0.0, 0.0, 1.0))
            cr.joint_limits(w, k, j, -0.4, 0.6)
            cr.joint_motor(w, k, j, 0.5, 2.0)
            cr.joint_spring(w, k, j, -0.2, 2.0, 1.0)
    return w


def passive_hinge_worlds(count, seed=5):
    """Worlds of capacity set 16/16/32/8 for the articulated-contact path:
    a ground box, a static post with a chain of three links on passive
    hinges (no spring, motor or limit, so no atan2f on the path) swinging
    into the ground and into each other, a second two-link chain hinged
    between two dynamic bodies (a floating tree), and three free spheres or
    boxes; every fifth world has no joints (the ordinary contact path)."""
    from puffysics_amd import creation as cr
    from puffysics_amd.b3types import B3_DYNAMIC, B3_STATIC
    rng = np.random.default_rng(seed)
    w = cr.new_worlds(count, gravity=(0.0, -9.81, 0.0))
    for k in range(count):
        g = cr.body(w, k, B3_STATIC, (0.0, -0.5, 0.0))
        cr.box(w, k, g, (5.0, 0.5, 5.0), friction=float(rng.uniform(0.3, 0.9)))
        if k % 5 != 4:
            post = cr.body(w, k, B3_STATIC, (0.0, 1.2, 0.0))
            prev, anchor = post, (0.0, 0.0, 0.0)
            axis = tuple(rng.normal(size=3) * 0.2 + np.array([0.0, 0.0, 1.0]))
            for i in range(3):
                half = tuple(rng.uniform(0.06, 0.12, 3))
                pos = (0.25 * (i + 1) + rng.uniform(-0.05, 0.05), 1.2 - 0.15 * i, rng.uniform(-0.1, 0.1))
                b = cr.body(w, k, B3_DYNAMIC, pos, lin_vel=tuple(rng.uniform(-1, 1, 3)))
                if i == 1:
                    cr.capsule(w, k, b, 0.08, 0.06)
                else:
                    cr.box(w, k, b, half)
                cr.finalize_mass(w, k, b)
                local = (-0.125, 0.075, 0.0)
                cr.revolute(w, k, prev, b, anchor, local, axis)
                prev, anchor = b, (0.125, -0.075, 0.0)
            a = cr.body(w, k, B3_DYNAMIC, (-0.6, 0.4, 0.2))
            cr.box(w, k, a, (0.1, 0.1, 0.1))
            cr.finalize_mass(w, k, a)
            b = cr.body(w, k, B3_DYNAMIC, (-0.6, 0.7, 0.2), ang_vel=tuple(rng.uniform(-2, 2, 3)))
            cr.sphere(w, k, b, 0.09)
            cr.finalize_mass(w, k, b)
            cr.revolute(w, k, a, b, (0.0, 0.15, 0.0), (0.0, -0.15, 0.0), (1.0, 0.0, 0.0))
        for i in range(3):
            p = (rng.uniform(-0.8, 0.8), rng.uniform(0.2, 1.0), rng.uniform(-0.8, 0.8))
            b = cr.body(w, k, B3_DYNAMIC, p, lin_vel=tuple(rng.uniform(-1, 1, 3)))
            if i % 2:
                cr.sphere(w, k, b, rng.uniform(0.08, 0.15), restitution=float(rng.choice([0.0, 0.4])))
            else:
                cr.box(w, k, b, tuple(rng.uniform(0.06, 0.12, 3)))
            cr.finalize_mass(w, k, b)
    return w


def reduced_tree_worlds(count, seed=11):
    """Worlds of capacity set 16/16/32/8 for the reduced-coordinate
    integrator, every joint passive and revolute with coincident anchors:
    a ground box; a static post carrying a hanging chain of three links
    whose hinge axes lean off z and whose tip swings into a free box on the
    ground, and a four-bar loop (three links and four hinges, so one hinge
    is a loop cut); a floating two-link tree dropped on the ground; a free
    sphere.  Every fourth world puts a motor on its last joint, which sends
    it to the articulated-contact step instead.

    The reference's reduced integrator gains energy on fast swings (a chain
    released horizontally diverges within a second), so the scene starts
    near rest: the oracle follows the reference either way, but the tests
    want finite states to compare."""
    from puffysics_amd import creation as cr
    from puffysics_amd.b3types import B3_DYNAMIC, B3_STATIC
    rng = np.random.default_rng(seed)
    w = cr.new_worlds(count, gravity=(0.0, -9.81, 0.0))
    for k in range(count):
        g = cr.body(w, k, B3_STATIC, (0.0, -0.5, 0.0))
        cr.box(w, k, g, (5.0, 0.5, 5.0), friction=float(rng.uniform(0.3, 0.9)))
        post = cr.body(w, k, B3_STATIC, (0.0, 1.0, 0.0))
        prev = post
        for i in range(3):
            b = cr.body(w, k, B3_DYNAMIC, (0.0, 0.85 - 0.3 * i, 0.0),
                        ang_vel=(0.0, 0.0, float(rng.uniform(-0.8, 0.8))))
            if i == 1:
                cr.capsule(w, k, b, 0.1, 0.04)
            else:
                cr.box(w, k, b, (0.04, 0.15, 0.04))
            cr.finalize_mass(w, k, b)
            axis = tuple(rng.normal(size=3) * 0.15 + np.array([0.0, 0.0, 1.0]))
            anchor = (0.0, 0.0, 0.0) if prev == post else (0.0, -0.15, 0.0)
            cr.revolute(w, k, prev, b, anchor, (0.0, 0.15, 0.0), axis)
            prev = b
        tip = cr.body(w, k, B3_DYNAMIC, (float(rng.uniform(0.1, 0.16)), 0.06, 0.0))
        cr.box(w, k, tip, (0.06, 0.06, 0.06))
        cr.finalize_mass(w, k, tip)
        x0 = float(rng.uniform(-1.2, -0.8))
        la = cr.body(w, k, B3_DYNAMIC, (x0, 0.8, 0.5))
        cr.box(w, k, la, (0.03, 0.2, 0.03))
        cr.finalize_mass(w, k, la)
        lb = cr.body(w, k, B3_DYNAMIC, (x0 + 0.2, 0.6, 0.5))
        cr.box(w, k, lb, (0.2, 0.03, 0.03))
        cr.finalize_mass(w, k, lb)
        lc = cr.body(w, k, B3_DYNAMIC, (x0 + 0.4, 0.8, 0.5), ang_vel=(0.0, 0.0, float(rng.uniform(-1, 1))))
        cr.box(w, k, lc, (0.03, 0.2, 0.03))
        cr.finalize_mass(w, k, lc)
        z = (0.0, 0.0, 1.0)
        cr.revolute(w, k, post, la, (x0, 0.0, 0.5), (0.0, 0.2, 0.0), z)
        cr.revolute(w, k, la, lb, (0.0, -0.2, 0.0), (-0.2, 0.0, 0.0), z)
        cr.revolute(w, k, lb, lc, (0.2, 0.0, 0.0), (0.0, -0.2, 0.0), z)
        cr.revolute(w, k, lc, post, (0.0, 0.2, 0.0), (x0 + 0.4, 0.0, 0.5), z)
        fa = cr.body(w, k, B3_DYNAMIC, (0.8, 0.3, -0.8), lin_vel=tuple(rng.uniform(-0.5, 0.5, 3)))
        cr.box(w, k, fa, (0.08, 0.08, 0.08))
        cr.finalize_mass(w, k, fa)
        fb = cr.body(w, k, B3_DYNAMIC, (0.8, 0.6, -0.8), ang_vel=tuple(rng.uniform(-1, 1, 3)))
        cr.sphere(w, k, fb, 0.07)
        cr.finalize_mass(w, k, fb)
        cr.revolute(w, k, fa, fb, (0.0, 0.15, 0.0), (0.0, -0.15, 0.0), (1.0, 0.0, 0.0))
        s = cr.body(w, k, B3_DYNAMIC, (float(rng.uniform(-0.4, 0.4)), 0.3, float(rng.uniform(-0.5, -0.2))),
                    lin_vel=tuple(rng.uniform(-1, 1, 3)))
        cr.sphere(w, k, s, float(rng.uniform(0.06, 0.1)), restitution=float(rng.choice([0.0, 0.4])))
        cr.finalize_mass(w, k, s)
        if k % 4 == 3:
            cr.joint_motor(w, k, 7, 1.0, 5.0)
    return w


def oracle_step_art(worlds, sig, dt, substeps, active=None):
    """b3_step built with articulated contacts, world by world on the oracle."""
    lib = oracle()
    lib.ocpu_step_art.argtypes = [_vp, _ull, _f, _i]
    for k in range(len(worlds)):
        if active is None or active[k]:
            lib.ocpu_step_art(worlds[k:k + 1].ctypes.data, sig, dt, substeps)


def oracle_art_step(worlds, sig, dt, substeps, active=None):
    """b3_art_step, the reduced-coordinate integrator, world by world on the oracle."""
    lib = oracle()
    lib.ocpu_art_step.argtypes = [_vp, _ull, _f, _i]
    for k in range(len(worlds)):
        if active is None or active[k]:
            lib.ocpu_art_step(worlds[k:k + 1].ctypes.data, sig, dt, substeps)


ORACLE_ULP_PATH = os.path.join(ROOT, "oracle", "liboracle_ulp.so")
_oracle_ulp = None


def ulp_spread(worlds, sig, dt, substeps, runs=24, entry="ocpu_art_step"):
    """Largest deviation, per body-state entry (body_state layout), of the
    oracle with its sinf, cosf and atan2f results moved by one ulp at random
    (oracle/ulp_envelope.c) from the plain oracle, over `runs` seeds, for one
    step of `worlds` through `entry`: the envelope of a faithful
    implementation whose libm differs from glibc's in the last place."""
    global _oracle_ulp
    if _oracle_ulp is None:
        lib = C.CDLL(ORACLE_ULP_PATH)
        lib.oulp_seed.argtypes = [_ull]
        _oracle_ulp = lib
    lib = _oracle_ulp
    fn = getattr(lib, entry)
    fn.argtypes = [_vp, _ull, _f, _i]
    exact = clone(worlds)
    ofn = getattr(oracle(), entry)
    ofn.argtypes = [_vp, _ull, _f, _i]
    for k in range(len(exact)):
        ofn(exact[k:k + 1].ctypes.data, sig, dt, substeps)
    ref = body_state(exact)
    spread = np.zeros_like(ref)
    for seed in range(runs):
        lib.oulp_seed(seed + 1)
        w = clone(worlds)
        for k in range(len(w)):
            fn(w[k:k + 1].ctypes.data, sig, dt, substeps)
        spread = np.maximum(spread, np.abs(body_state(w) - ref))
    return spread


def body_state(worlds):
    """Per body: position, center, linear and angular velocity, rotation
    (x, y, z, s), as float64 [world, body, 16]."""
    b = worlds["bodies"]
    cols = []
    for f in ("position", "center", "lin_vel", "ang_vel"):
        cols += [b[f][a] for a in "xyz"]
    cols += [b["rotation"]["v"][a] for a in "xyz"] + [b["rotation"]["s"]]
    return np.stack(cols, axis=-1).astype(np.float64)


def ref_art_lib(caps):
    """The reference's b3_step built with B3_ART_CONTACTS=1 for capacity set
    `caps` (0, 2, 3 or 5), or None where the reference was not built."""
    path = os.path.join(REF_DIR, "libb3ref_art_%d.so" % caps)
    if not os.path.exists(path):
        return None
    key = "art_%d" % caps
    if key not in _refs:
        lib = C.CDLL(path)
        lib.refa_sig.restype = C.c_ulonglong
        lib.refa_step.argtypes = [_vp, _f, _i]
        lib.refa_art_step.argtypes = [_vp, _f, _i]
        _refs[key] = lib
    return _refs[key]


def two_shape_worlds(count):
    """Worlds of the hover's capacities (2 bodies, 2 shapes, 4 contacts, 2
    joints: at most one candidate pair, so at most one contact) varied for
    the kept-row step: restitution on every third dynamic shape (with a
    fast fall, so that bounces happen), rolling resistance on every fourth,
    friction from 0.2 to 1.0, and every sixth sphere made a box (contacts of
    up to four points)."""
    w = clone(scenes.build(1, count))
    sh, bo = w["shapes"], w["bodies"]
    k = np.arange(count)
    sh["restitution"][:, 1] = np.where(k % 3 == 1, np.float32(0.6), np.float32(0.0))
    sh["rolling"][:, 1] = np.where(k % 4 == 2, np.float32(0.05), np.float32(0.0))
    sh["friction"][:, 1] = (np.float32(0.2) + np.float32(0.2) * (k % 5)).astype(np.float32)
    bo["lin_vel"]["y"][:, 1] = np.where(k % 2 == 0, np.float32(-4.0), bo["lin_vel"]["y"][:, 1])
    box = k % 6 == 5
    sh["type"][box, 1] = sh["type"][0, 0]                 # the ground's type: box
    sh["half"]["x"][box, 1] = np.float32(0.3)
    sh["half"]["y"][box, 1] = np.float32(0.2)
    sh["half"]["z"][box, 1] = np.float32(0.25)
    return w


def oracle_step_batch(worlds, sig, dt, substeps, active=None):
    """b3_batch_step over a contiguous batch on the oracle."""
    lib = oracle()
    lib.ocpu_batch_step.argtypes = [_vp, C.c_size_t, C.c_size_t, _i, _ull, _f, _i, _vp]
    act = None if active is None else np.ascontiguousarray(active, np.uint8)
    return lib.ocpu_batch_step(worlds.ctypes.data, worlds.dtype.itemsize, 0, len(worlds), sig, dt, substeps,
                               None if act is None else act.ctypes.data)


def oracle_step_gravity(worlds, sig, dt, substeps, gravity, softening, masses=None, active=None):
    """b3_step with pairwise gravity in the force hook, world by world on
    the oracle; `masses` is None or [count, max_bodies] float32."""
    lib = oracle()
    lib.ocpu_step_gravity.argtypes = [_vp, _ull, _f, _i, _f, _f, _vp]
    m = None if masses is None else np.ascontiguousarray(masses, np.float32)
    for k in range(len(worlds)):
        if active is not None and not active[k]:
            continue
        lib.ocpu_step_gravity(worlds[k:k + 1].ctypes.data, sig, dt, substeps, gravity, softening,
                              None if m is None else m[k].ctypes.data)


def ref_gravity_lib(caps):
    """The reference's b3_step with its B3_USER_FORCES hook running the
    reference's pairwise gravity, for capacity set `caps` (0, 2, 4 or 5), or
    None where the reference was not built."""
    path = os.path.join(REF_DIR, "libb3ref_gravity_%d.so" % caps)
    if not os.path.exists(path):
        return None
    key = "gravity_%d" % caps
    if key not in _refs:
        lib = C.CDLL(path)
        lib.refg_sig.restype = C.c_ulonglong
        lib.refg_step.argtypes = [_vp, _f, _i, _f, _f, _vp]
        _refs[key] = lib
    return _refs[key]


class EmuSig:
    """Word-transposed tiles of any signature stepped by the host build of
    the lane code, without scene inputs."""

    def __init__(self, sig, worlds):
        self.sig = sig
        self.count = len(worlds)
        self.dtype = worlds.dtype
        words_ = emu().emu_world_words(sig)
        self.tiles = np.zeros(((self.count + 63) // 64) * words_ * 64, np.uint32)
        w = np.ascontiguousarray(worlds)
        emu().emu_upload(w.ctypes.data, self.count, sig, self.tiles.ctypes.data)

    def step(self, dt, substeps, active=None):
        act = None if active is None else np.ascontiguousarray(active, np.uint8)
        emu().emu_step(self.tiles.ctypes.data, self.count, self.sig, dt, substeps,
                       None if act is None else act.ctypes.data)

    def step_shared(self, dt, substeps, active=None, masks=-1):
        lib = emu()
        lib.emu_step_shared.argtypes = [_vp, _i, _ull, _f, _i, _vp, _i]
        act = None if active is None else np.ascontiguousarray(active, np.uint8)
        lib.emu_step_shared(self.tiles.ctypes.data, self.count, self.sig, dt, substeps,
                            None if act is None else act.ctypes.data, masks)

    def step_gravity(self, dt, substeps, gravity, softening, masses=None, active=None):
        lib = emu()
        lib.emu_step_gravity.argtypes = [_vp, _i, _ull, _f, _i, _vp, _f, _f, _vp]
        act = None if active is None else np.ascontiguousarray(active, np.uint8)
        m = None if masses is None else np.ascontiguousarray(masses, np.float32)
        lib.emu_step_gravity(self.tiles.ctypes.data, self.count, self.sig, dt, substeps,
                             None if act is None else act.ctypes.data, gravity, softening,
                             None if m is None else m.ctypes.data)

    def step_art(self, dt, substeps, active=None):
        lib = emu()
        lib.emu_step_art.argtypes = [_vp, _i, _ull, _f, _i, _vp]
        act = None if active is None else np.ascontiguousarray(active, np.uint8)
        lib.emu_step_art(self.tiles.ctypes.data, self.count, self.sig, dt, substeps,
                         None if act is None else act.ctypes.data)

    def art_step(self, dt, substeps, active=None):
        lib = emu()
        lib.emu_art_step.argtypes = [_vp, _i, _ull, _f, _i, _vp]
        act = None if active is None else np.ascontiguousarray(active, np.uint8)
        lib.emu_art_step(self.tiles.ctypes.data, self.count, self.sig, dt, substeps,
                         None if act is None else act.ctypes.data)

    def worlds(self):
        out = np.zeros(self.count, dtype=self.dtype)
        emu().emu_download(self.tiles.ctypes.data, self.count, self.sig, out.ctypes.data)
        return out


# ---- the hover environment (oracle and, where built, the reference task) ----

HOVER_OBS = 3


def hover_actions(n, steps, seed=5):
    """Actions of a hover run: the three levels and the values at and just
    below the level thresholds (hover_task.h:69)."""
    rng = np.random.default_rng(seed)
    vals = np.array([0.0, 1.0, 2.0, 0.49, 0.5, 1.49, 1.5, -1.0, 3.0], np.float32)
    return rng.choice(vals, size=(steps, n)).astype(np.float32)


def _hover_bind(lib, p):
    getattr(lib, p + "_env_bytes").restype = C.c_size_t
    getattr(lib, p + "_signature").restype = C.c_ulonglong
    getattr(lib, p + "_init").argtypes = [_vp, _i, _f, _f, _f, _i, _i, C.c_uint32]
    getattr(lib, p + "_reset").argtypes = [_vp, _i, _vp, _vp, _vp]
    getattr(lib, p + "_step").argtypes = [_vp, _i, _vp, _vp, _vp, _vp]
    getattr(lib, p + "_log").argtypes = [_vp, _i, _vp]
    getattr(lib, p + "_world").argtypes = [_vp, _i, _vp]


def hover_cpu_run(lib, prefix, n, actions, seed=1, config=(2.0, 10.0, 1.0 / 60.0, 4, 256)):
    """Run the CPU hover envs of `lib` (`ohover` oracle or `rhover`
    reference): init, reset, then one step per row of `actions`.  Returns
    observations (steps+1, n, 3), rewards and terminals (steps+1, n), the
    summed log and the final worlds' bytes."""
    _hover_bind(lib, prefix)
    f = lambda s: getattr(lib, prefix + s)
    steps = len(actions)
    envs = np.zeros(f("_env_bytes")() * n, np.uint8)
    f("_init")(envs.ctypes.data, n, *config, seed)
    obs = np.zeros((steps + 1, n, HOVER_OBS), np.float32)
    rew = np.zeros((steps + 1, n), np.float32)
    term = np.zeros((steps + 1, n), np.float32)
    f("_reset")(envs.ctypes.data, n, obs[0].ctypes.data, rew[0].ctypes.data, term[0].ctypes.data)
    for t in range(steps):
        a = np.ascontiguousarray(actions[t], np.float32)
        f("_step")(envs.ctypes.data, n, a.ctypes.data, obs[t + 1].ctypes.data, rew[t + 1].ctypes.data,
                   term[t + 1].ctypes.data)
    log = np.zeros(5, np.float32)
    f("_log")(envs.ctypes.data, n, log.ctypes.data)
    sig = f("_signature")()
    from puffysics_amd.b3types import world_dtype
    dt = world_dtype(sig)
    worlds = np.zeros(n, dt)
    for i in range(n):
        f("_world")(envs.ctypes.data, i, worlds[i:i + 1].ctypes.data)
    return obs, rew, term, log, worlds


def hover_ref_lib():
    """oracle/_ref/libhover_ref.so (the reference's hover task), or None."""
    path = os.path.join(ROOT, "oracle", "_ref", "libhover_ref.so")
    return C.CDLL(path) if os.path.exists(path) else None


def gpu_run(eng, scene, t0, nsteps, seed=scenes.SEED):
    """The workload loop on the device: masks, restore, inputs, step."""
    import torch
    sc = scenes.SCENES[scene]
    reset = torch.zeros(eng.count, dtype=torch.uint8, device="cuda")
    stepm = torch.zeros(eng.count, dtype=torch.uint8, device="cuda")
    for t in range(t0, t0 + nsteps):
        eng.scene_masks(scene, seed, t, reset, stepm)
        eng.restore(reset)
        eng.scene_inputs(scene, seed, t, stepm)
        eng.step(sc.dt, sc.substeps, stepm)
    torch.cuda.synchronize()


# ---- per-world aggregates and body checksums from the body block ----
# A batch's bodies as a [count, max_bodies, 50] block of 32-bit words (the
# B3Body layout of include/b3_types.h), read from host worlds or from the
# engine's device tiles, so that the same statistics can be taken every
# vector step on both sides without downloading whole worlds.

BODY_WORDS = 50
BW_ROT, BW_CENTER, BW_LIN_VEL, BW_ANG_VEL, BW_INV_MASS, BW_INV_INERTIA, BW_TYPE = 3, 7, 13, 16, 32, 33, 48
CANON_NAN = 0x7FC00000
GRAVITY = 9.81


def body_block(worlds):
    """uint32 [count, max_bodies, 50] view of the host worlds' bodies."""
    bo = worlds.dtype.fields["bodies"][1] // 4
    nb = worlds.dtype["bodies"].shape[0]
    return words(worlds)[:, bo:bo + nb * BODY_WORDS].reshape(len(worlds), nb, BODY_WORDS)


def device_body_block(tiles, worlds_dtype, count):
    """int32 [count, max_bodies, 50] copy of the bodies in the engine's
    device tiles ([tiles, world_words, 64], word k of world w at
    tiles[w // 64, k, w % 64])."""
    bo = worlds_dtype.fields["bodies"][1] // 4
    nb = worlds_dtype["bodies"].shape[0]
    blk = tiles[:, bo:bo + nb * BODY_WORDS, :].permute(0, 2, 1)
    return blk.reshape(-1, nb, BODY_WORDS)[:count]


def _cross(ax, ay, az, bx, by, bz):
    return ay * bz - az * by, az * bx - ax * bz, ax * by - ay * bx


def stats_of_block(blk):
    """Per-world mean height and mean energy of the dynamic bodies (numpy,
    float64): linear and rotational kinetic energy (0.5 w.I w with
    I = R diag(1/inv_i) R^T, evaluated in the body frame) plus gravitational
    potential energy."""
    need = [BW_ROT, BW_ROT + 1, BW_ROT + 2, BW_ROT + 3, BW_CENTER + 1, BW_LIN_VEL, BW_LIN_VEL + 1, BW_LIN_VEL + 2,
            BW_ANG_VEL, BW_ANG_VEL + 1, BW_ANG_VEL + 2, BW_INV_MASS, BW_INV_INERTIA, BW_INV_INERTIA + 1,
            BW_INV_INERTIA + 2, BW_TYPE]
    sel = np.ascontiguousarray(blk[..., need])        # one gather of the words used
    f = sel.view(np.float32).astype(np.float64)
    at = {k: i for i, k in enumerate(need)}

    def col(k):
        return f[..., at[k]]

    dyn = sel[..., at[BW_TYPE]].view(np.int32) == 2
    inv_m = col(BW_INV_MASS)
    m = np.where(inv_m > 0, 1.0 / np.where(inv_m > 0, inv_m, 1.0), 0.0)
    vx, vy, vz = col(BW_LIN_VEL), col(BW_LIN_VEL + 1), col(BW_LIN_VEL + 2)
    v2 = vx * vx + vy * vy + vz * vz
    nx, ny, nz = -col(BW_ROT), -col(BW_ROT + 1), -col(BW_ROT + 2)
    qs = col(BW_ROT + 3)
    wx, wy, wz = col(BW_ANG_VEL), col(BW_ANG_VEL + 1), col(BW_ANG_VEL + 2)
    tx, ty, tz = (2.0 * c for c in _cross(nx, ny, nz, wx, wy, wz))     # body-frame w: R^T w
    cx, cy, cz = _cross(nx, ny, nz, tx, ty, tz)
    lx, ly, lz = wx + qs * tx + cx, wy + qs * ty + cy, wz + qs * tz + cz
    rot = 0.0
    for k, wl in enumerate((lx, ly, lz)):
        ii = col(BW_INV_INERTIA + k)
        inertia = np.where(ii > 0, 1.0 / np.where(ii > 0, ii, 1.0), 0.0)
        rot = rot + inertia * wl * wl
    rot = 0.5 * rot
    y = col(BW_CENTER + 1)
    e = 0.5 * m * v2 + rot + m * GRAVITY * y
    n = np.maximum(dyn.sum(axis=1), 1)
    return np.where(dyn, y, 0).sum(axis=1) / n, np.where(dyn, e, 0).sum(axis=1) / n


def stats_of_device_block(blk):
    """stats_of_block for a torch int32 block on the device, same operations
    in float64; returns a [2, count] tensor (mean height, mean energy)."""
    import torch
    f = blk.view(torch.float32).double()
    dyn = blk[..., BW_TYPE] == 2
    inv_m = f[..., BW_INV_MASS]
    pos = inv_m > 0
    m = torch.where(pos, 1.0 / torch.where(pos, inv_m, torch.ones_like(inv_m)), torch.zeros_like(inv_m))
    v2 = (f[..., BW_LIN_VEL:BW_LIN_VEL + 3] ** 2).sum(-1)
    qv = f[..., BW_ROT:BW_ROT + 3]
    qs = f[..., BW_ROT + 3:BW_ROT + 4]
    w = f[..., BW_ANG_VEL:BW_ANG_VEL + 3]
    t = 2.0 * torch.linalg.cross(-qv, w)
    wl = w + qs * t + torch.linalg.cross(-qv, t)
    ii = f[..., BW_INV_INERTIA:BW_INV_INERTIA + 3]
    ipos = ii > 0
    inertia = torch.where(ipos, 1.0 / torch.where(ipos, ii, torch.ones_like(ii)), torch.zeros_like(ii))
    rot = 0.5 * (inertia * wl * wl).sum(-1)
    y = f[..., BW_CENTER + 1]
    e = 0.5 * m * v2 + rot + m * GRAVITY * y
    n = dyn.sum(dim=1).clamp(min=1).double()
    zero = torch.zeros_like(y)
    return torch.stack([torch.where(dyn, y, zero).sum(dim=1) / n, torch.where(dyn, e, zero).sum(dim=1) / n])


def _hash_weights(nwords):
    """Fixed weights in [1, 1024): a word times its weight stays below 2^42
    and a sum of up to 2^11 such products below 2^53, so the float64 sums
    below are exact whatever their order, and any single differing word
    changes the sum."""
    k = np.arange(nwords, dtype=np.int64)
    return ((k * 2654435761 + 12345) % 1023 + 1).astype(np.float64)


def body_hash(blk):
    """Per-world exact checksum of a uint32 body block (NaN floats
    canonicalised: their bits depend on operand order)."""
    x = blk.reshape(len(blk), -1)
    x = np.where(np.isnan(x.view(np.float32)), np.uint32(CANON_NAN), x)
    return x.astype(np.float64) @ _hash_weights(x.shape[1])


def device_body_hash(blk):
    """body_hash of a torch int32 body block on the device."""
    import torch
    x = blk.reshape(blk.shape[0], -1)
    x = torch.where(torch.isnan(x.view(torch.float32)), torch.full_like(x, CANON_NAN), x)
    u = x.long() & 0xFFFFFFFF
    wts = torch.from_numpy(_hash_weights(x.shape[1])).to(x.device)
    return u.double() @ wts


def oracle_stats(worlds, checksum=True):
    """[3, count]: mean height, mean energy and body checksum (zero unless
    `checksum`) per world, from the oracle library's C restatement of
    stats_of_block and body_hash."""
    lib = oracle()
    fn = lib.ostat_bodies
    fn.restype = None
    fn.argtypes = [_vp, _i, C.c_size_t, _i, _i, _vp, _vp, _vp]
    w = np.ascontiguousarray(worlds)
    n = len(w)
    out = np.zeros((3, n), np.float64)
    fn(w.ctypes.data, n, w.dtype.itemsize, w.dtype.fields["bodies"][1] // 4, w.dtype["bodies"].shape[0],
       out[0].ctypes.data, out[1].ctypes.data, out[2].ctypes.data if checksum else None)
    return out
